// gguf.cpp - GGUF v2/v3 reader and v3 writer (host code; include/rlq.h rlq_gguf_*).
//
// Behaviour follows the reference's frozen reader and writer (paths relative
// to the rust-llama repository):
//   header parse   crates/gguf/src/raw.rs:85-300 (RawGguf::read_with_payload_validation)
//   value parse    crates/gguf/src/lib.rs:513-633 (Parser), limits lib.rs:172-193
//   payload reads  crates/gguf/src/lib.rs:322-360
//   writer         crates/gguf/src/writer.rs:133-460 (layout_inner, Encoder), the
//                  native header of raw.rs:346-390 (gguf_get_meta_data) and the
//                  raw v3 writer of writer.rs:476-486
// Errors map to RLQ_GGUF_IO / _INVALID / _LIMIT / _UNSUPPORTED with a = the
// header byte position where the check failed (0 when not positional).
#include <errno.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <memory>
#include <new>
#include <set>
#include <string>
#include <vector>

#include "rlq.h"
#include "rlq_dtype.hpp"

namespace rlq {
namespace gguf {

struct Fail {
    int32_t code;
    uint64_t a, b;
};
[[noreturn]] inline void fail(int32_t code, uint64_t a = 0, uint64_t b = 0) { throw Fail{code, a, b}; }

// Limits::default() (lib.rs:182-193)
struct Limits {
    uint64_t max_metadata_bytes = 256ull << 20;
    uint64_t max_string_bytes = 16ull << 20;
    uint64_t max_array_values = 1000000;
    uint64_t max_total_values = 4000000;
    uint64_t max_tensors = 100000;
    uint64_t max_metadata_entries = 100000;
    uint64_t max_tensor_read_bytes = 2ull << 30;
};

constexpr uint32_t kArray = 9, kString = 8, kBool = 7;

struct Value {
    uint32_t type = 0;
    uint64_t bits = 0;                 // scalars: the value's bits, zero-extended (bool: 0 / 1)
    std::string str;                   // type 8
    uint32_t elem = 0;                 // type 9: element type
    std::vector<uint64_t> abits;       // arrays of scalars
    std::vector<std::string> astr;     // arrays of strings
    uint64_t count() const {
        return type == kArray ? (elem == kString ? astr.size() : abits.size()) : (type == kString ? str.size() : 1);
    }
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint32_t dtype = 0;
    uint64_t offset = 0, bytes = 0;
};

// Random-access byte source: a file (with a read-ahead window) or a copy of
// a memory image.
struct Source {
    virtual ~Source() = default;
    virtual void read_at(uint64_t off, void* dst, uint64_t n) = 0;
    uint64_t len = 0;
};

struct FileSource : Source {
    FILE* f = nullptr;
    std::vector<uint8_t> win;
    uint64_t win_off = 0, win_len = 0;
    ~FileSource() override {
        if (f) fclose(f);
    }
    void read_at(uint64_t off, void* dst, uint64_t n) override {
        uint8_t* d = (uint8_t*)dst;
        if (n > win.size() / 2) {  // large payloads bypass the window
            if (fseeko(f, (off_t)off, SEEK_SET) != 0 || fread(d, 1, n, f) != n) fail(RLQ_GGUF_IO, (uint64_t)errno, off);
            return;
        }
        if (off < win_off || off + n > win_off + win_len) {
            if (fseeko(f, (off_t)off, SEEK_SET) != 0) fail(RLQ_GGUF_IO, (uint64_t)errno, off);
            win_off = off;
            win_len = fread(win.data(), 1, win.size(), f);
            if (win_len < n) fail(RLQ_GGUF_IO, (uint64_t)EIO, off);
        }
        memcpy(d, win.data() + (off - win_off), n);
    }
};

struct MemSource : Source {
    std::vector<uint8_t> bytes;
    void read_at(uint64_t off, void* dst, uint64_t n) override {
        if (off > bytes.size() || n > bytes.size() - off) fail(RLQ_GGUF_IO, (uint64_t)EIO, off);
        memcpy(dst, bytes.data() + off, n);
    }
};

struct File {
    std::unique_ptr<Source> src;
    uint32_t version = 0, alignment = 32;
    bool big = false;
    uint64_t data_offset = 0, file_len = 0;
    std::vector<std::string> keys;     // file order
    std::vector<Value> values;
    std::vector<Tensor> tensors;
    Limits limits;
};

inline std::string c_string(const std::string& s) {
    const size_t z = s.find('\0');
    return z == std::string::npos ? s : s.substr(0, z);
}

inline uint64_t align_up(uint64_t n, uint64_t a) {
    if (n > UINT64_MAX - (a - 1)) fail(RLQ_GGUF_INVALID, n);  // "alignment overflow"
    return (n + a - 1) & ~(a - 1);
}

inline bool pow2(uint64_t v) { return v && !(v & (v - 1)); }

// dimension_elements (lib.rs:284-299): every dimension and the running product
// within the signed GGML range.
inline uint64_t elements(const uint64_t* dims, uint32_t nd, uint64_t pos) {
    uint64_t count = 1;
    for (uint32_t i = 0; i < nd; ++i) {
        if (dims[i] > (uint64_t)INT64_MAX) fail(RLQ_GGUF_INVALID, pos);
        if (dims[i] && count > UINT64_MAX / dims[i]) fail(RLQ_GGUF_INVALID, pos);
        count *= dims[i];
        if (count > (uint64_t)INT64_MAX) fail(RLQ_GGUF_INVALID, pos);
    }
    return count;
}

// Stored bytes of a tensor: DType::row_bytes of dimension 0, times the rest.
inline uint64_t tensor_bytes(uint32_t dtype, const uint64_t* dims, uint32_t nd, uint64_t pos) {
    if (nd > 4) fail(RLQ_GGUF_INVALID, pos);
    elements(dims, nd, pos);
    const uint64_t row = nd ? dims[0] : 1, bs = block_size(dtype), ts = type_size(dtype);
    if (!dtype_known(dtype) || row % bs != 0) fail(RLQ_GGUF_INVALID, pos);
    uint64_t bytes;
    if (__builtin_mul_overflow(row / bs, ts, &bytes)) fail(RLQ_GGUF_INVALID, pos);
    for (uint32_t i = 1; i < nd; ++i)
        if (__builtin_mul_overflow(bytes, dims[i], &bytes)) fail(RLQ_GGUF_INVALID, pos);
    return bytes;
}

// ---- reader ---------------------------------------------------------------------

struct Parser {
    Source& src;
    bool big;
    uint64_t pos, file_len;
    const Limits& L;
    uint64_t total_values = 0;

    void charge(uint64_t n) {
        if (n > UINT64_MAX - pos) fail(RLQ_GGUF_INVALID, pos);
        pos += n;
        if (pos > file_len) fail(RLQ_GGUF_INVALID, pos);           // truncated metadata
        if (pos > L.max_metadata_bytes) fail(RLQ_GGUF_LIMIT, pos);  // metadata byte budget
    }
    uint64_t uint(int n) {
        charge((uint64_t)n);
        uint8_t b[8];
        src.read_at(pos - n, b, (uint64_t)n);
        uint64_t v = 0;
        for (int i = 0; i < n; ++i) v |= (uint64_t)b[big ? n - 1 - i : i] << (8 * i);
        return v;
    }
    uint64_t count(uint64_t max) {
        const uint64_t at = pos, n = uint(8);
        if (n > max) fail(RLQ_GGUF_LIMIT, at);
        return n;
    }
    void minimum_encoded(uint64_t count, uint64_t each) {
        uint64_t minimum;
        if (__builtin_mul_overflow(count, each, &minimum)) fail(RLQ_GGUF_LIMIT, pos);
        if (minimum > (file_len > pos ? file_len - pos : 0)) fail(RLQ_GGUF_INVALID, pos);
        if (minimum > (L.max_metadata_bytes > pos ? L.max_metadata_bytes - pos : 0)) fail(RLQ_GGUF_LIMIT, pos);
    }
    std::string string() {
        const uint64_t n = count(L.max_string_bytes);
        charge(n);
        std::string s(n, '\0');
        if (n) src.read_at(pos - n, &s[0], n);
        return s;
    }
    Value value(uint32_t ty, bool in_array) {
        if (++total_values > L.max_total_values) fail(RLQ_GGUF_LIMIT, pos);
        Value v;
        v.type = ty;
        switch (ty) {
            case 0: case 1: v.bits = uint(1); break;
            case 2: case 3: v.bits = uint(2); break;
            case 4: case 5: case 6: v.bits = uint(4); break;
            case kBool: v.bits = uint(1) != 0 ? 1 : 0; break;
            case kString: v.str = string(); break;
            case 10: case 11: case 12: v.bits = uint(8); break;
            case kArray: {
                if (in_array) fail(RLQ_GGUF_INVALID, pos);  // nested arrays
                const uint64_t at = pos;
                v.elem = (uint32_t)uint(4);
                if (v.elem > 12 || v.elem == kArray) fail(RLQ_GGUF_INVALID, at);
                const uint64_t n = count(L.max_array_values);
                if (n > (L.max_total_values > total_values ? L.max_total_values - total_values : 0))
                    fail(RLQ_GGUF_LIMIT, pos);
                const uint64_t min = v.elem == 0 || v.elem == 1 || v.elem == kBool ? 1
                                     : v.elem == 2 || v.elem == 3               ? 2
                                     : v.elem >= 4 && v.elem <= 6               ? 4
                                                                                 : 8;
                minimum_encoded(n, min);
                if (v.elem == kString) v.astr.reserve(n);
                else v.abits.reserve(n);
                for (uint64_t i = 0; i < n; ++i) {
                    Value e = value(v.elem, true);
                    if (v.elem == kString) v.astr.push_back(std::move(e.str));
                    else v.abits.push_back(e.bits);
                }
                break;
            }
            default: fail(RLQ_GGUF_INVALID, pos);  // unknown metadata type
        }
        return v;
    }
};

void parse(File& g, bool validate_payload) {
    Source& src = *g.src;
    g.file_len = src.len;
    if (g.file_len < 8) fail(RLQ_GGUF_IO, (uint64_t)EIO, 0);  // read_exact of magic / version
    uint8_t head[8];
    src.read_at(0, head, 8);
    if (memcmp(head, "GGUF", 4) != 0) fail(RLQ_GGUF_INVALID, 0);
    const uint32_t le = (uint32_t)head[4] | (uint32_t)head[5] << 8 | (uint32_t)head[6] << 16 | (uint32_t)head[7] << 24;
    const uint32_t be = (uint32_t)head[7] | (uint32_t)head[6] << 8 | (uint32_t)head[5] << 16 | (uint32_t)head[4] << 24;
    if (le == 2 || le == 3) g.version = le, g.big = false;
    else if (be == 2 || be == 3) g.version = be, g.big = true;
    else fail(RLQ_GGUF_UNSUPPORTED, 4);
    Parser p{src, g.big, 8, g.file_len, g.limits};
    const uint64_t nt = p.count(g.limits.max_tensors);
    const uint64_t nk = p.count(g.limits.max_metadata_entries);
    p.minimum_encoded(nk, 14);
    std::set<std::string> seen;
    for (uint64_t i = 0; i < nk; ++i) {
        const uint64_t at = p.pos;
        std::string key = p.string();
        if (key.empty()) fail(RLQ_GGUF_INVALID, at);
        const uint32_t ty = (uint32_t)p.uint(4);
        Value v = p.value(ty, false);
        if (!seen.insert(key).second) fail(RLQ_GGUF_INVALID, at);  // duplicate key
        g.keys.push_back(std::move(key));
        g.values.push_back(std::move(v));
    }
    g.alignment = 32;
    for (size_t i = 0; i < g.keys.size(); ++i)
        if (c_string(g.keys[i]) == "general.alignment") {
            if (g.values[i].type != 4) fail(RLQ_GGUF_INVALID, p.pos);
            g.alignment = (uint32_t)g.values[i].bits;
            break;
        }
    if (!pow2(g.alignment) || g.alignment > (1u << 20)) fail(RLQ_GGUF_INVALID, p.pos);
    p.minimum_encoded(nt, 24);
    std::set<std::string> names;
    uint64_t expected = 0;
    g.tensors.reserve(nt);
    for (uint64_t i = 0; i < nt; ++i) {
        const uint64_t at = p.pos;
        Tensor t;
        t.name = p.string();
        if (t.name.size() >= 64 || !names.insert(t.name).second) fail(RLQ_GGUF_INVALID, at);
        t.n_dims = (uint32_t)p.uint(4);
        if (t.n_dims > 4) fail(RLQ_GGUF_INVALID, at);
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            t.dims[d] = p.uint(8);
            if (t.dims[d] > (uint64_t)INT64_MAX) fail(RLQ_GGUF_INVALID, at);
        }
        t.dtype = (uint32_t)p.uint(4);
        if (!dtype_known(t.dtype)) fail(RLQ_GGUF_INVALID, at);
        t.bytes = tensor_bytes(t.dtype, t.dims, t.n_dims, at);
        t.offset = p.uint(8);
        // descriptor-order contiguous padded payloads (raw.rs:209-217)
        if (t.offset != expected) fail(RLQ_GGUF_INVALID, at, t.offset);
        const uint64_t padded = align_up(t.bytes, g.alignment);
        if (padded > UINT64_MAX - expected) fail(RLQ_GGUF_INVALID, at);
        expected += padded;
        g.tensors.push_back(std::move(t));
    }
    g.data_offset = nt == 0 ? p.pos : align_up(p.pos, g.alignment);
    if (g.data_offset > g.limits.max_metadata_bytes) fail(RLQ_GGUF_LIMIT, p.pos);
    for (const Tensor& t : g.tensors) {
        uint64_t start, end;
        if (__builtin_add_overflow(g.data_offset, t.offset, &start) || __builtin_add_overflow(start, t.bytes, &end))
            fail(RLQ_GGUF_INVALID, t.offset);
        if (validate_payload && end > g.file_len) fail(RLQ_GGUF_INVALID, t.offset);
    }
}

// ---- writer -----------------------------------------------------------------------

struct Policy {
    bool native = false;    // gguf_get_meta_data: C-string tensor names, collapsed rank
    uint32_t version = 3;
    uint32_t alignment = 0;  // physical alignment; 0 = general.alignment (or 32)
};

struct Kv {
    const std::string* key;
    const Value* value;
};

uint32_t native_rank(const Tensor& t) {
    for (int i = (int)t.n_dims - 1; i > 0; --i)
        if (t.dims[i] > 1) return (uint32_t)i + 1;
    return 1;
}

struct Layout {
    uint64_t header = 0, data_offset = 0, file_bytes = 0;
    uint32_t alignment = 32;
    std::vector<uint64_t> offsets;
};

void add(uint64_t& total, uint64_t n, const Limits& L) {
    if (n > UINT64_MAX - total) fail(RLQ_GGUF_LIMIT, total);
    total += n;
    if (total > L.max_metadata_bytes) fail(RLQ_GGUF_LIMIT, total);
}

uint64_t string_size(const std::string& s, const Limits& L) {
    if (s.size() > L.max_string_bytes) fail(RLQ_GGUF_LIMIT, s.size());
    return (uint64_t)s.size() + 8;
}

uint64_t value_size(const Value& v, const Limits& L, uint64_t& total_values) {
    if (++total_values > L.max_total_values) fail(RLQ_GGUF_LIMIT, total_values);
    switch (v.type) {
        case 0: case 1: case kBool: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        case kString: return string_size(v.str, L);
        case kArray: {
            if (v.elem > 12 || v.elem == kArray) fail(RLQ_GGUF_INVALID, v.elem);
            const uint64_t n = v.count();
            if (n > L.max_array_values || n > (L.max_total_values > total_values ? L.max_total_values - total_values : 0))
                fail(RLQ_GGUF_LIMIT, n);
            uint64_t bytes = 12;
            for (uint64_t i = 0; i < n; ++i) {
                Value e;
                e.type = v.elem;
                if (v.elem == kString) e.str = v.astr[i];
                add(bytes, value_size(e, L, total_values), L);
            }
            return bytes;
        }
        default: fail(RLQ_GGUF_INVALID, v.type);
    }
}

Layout layout(const std::vector<Kv>& kv, const std::vector<Tensor>& tensors, const Limits& L, const Policy& pol) {
    if (kv.size() > L.max_metadata_entries || tensors.size() > L.max_tensors) fail(RLQ_GGUF_LIMIT, kv.size());
    uint32_t meta_alignment = 32;
    for (const Kv& e : kv)
        if (c_string(*e.key) == "general.alignment") {
            if (e.value->type != 4) fail(RLQ_GGUF_INVALID, 0);
            meta_alignment = (uint32_t)e.value->bits;
            break;
        }
    if (!pow2(meta_alignment) || meta_alignment > (1u << 20)) fail(RLQ_GGUF_INVALID, meta_alignment);
    Layout out;
    out.alignment = pol.alignment ? pol.alignment : meta_alignment;
    if (!pow2(out.alignment) || out.alignment > (1u << 20)) fail(RLQ_GGUF_INVALID, out.alignment);
    if (pol.version != 2 && pol.version != 3) fail(RLQ_GGUF_UNSUPPORTED, pol.version);
    uint64_t header = 0, values = 0;
    add(header, 24, L);
    std::set<std::string> keys;
    for (const Kv& e : kv) {
        if (e.key->empty() || !keys.insert(*e.key).second) fail(RLQ_GGUF_INVALID, header);
        add(header, string_size(*e.key, L), L);
        add(header, 4, L);
        add(header, value_size(*e.value, L, values), L);
    }
    uint64_t minimum;
    if (__builtin_mul_overflow((uint64_t)tensors.size(), (uint64_t)24, &minimum) ||
        minimum > (L.max_metadata_bytes > header ? L.max_metadata_bytes - header : 0))
        fail(RLQ_GGUF_LIMIT, header);
    std::set<std::string> names;
    uint64_t offset = 0;
    for (const Tensor& t : tensors) {
        if (t.name.size() >= 64 || !names.insert(t.name).second) fail(RLQ_GGUF_INVALID, header);
        const uint64_t bytes = tensor_bytes(t.dtype, t.dims, t.n_dims, header);
        const uint32_t rank = pol.native ? native_rank(t) : t.n_dims;
        add(header, string_size(pol.native ? c_string(t.name) : t.name, L), L);
        add(header, 16 + (uint64_t)rank * 8, L);
        out.offsets.push_back(offset);
        const uint64_t padded = align_up(bytes, out.alignment);
        if (padded > UINT64_MAX - offset) fail(RLQ_GGUF_INVALID, offset);
        offset += padded;
    }
    out.header = header;
    out.data_offset = align_up(header, out.alignment);
    if (out.data_offset > L.max_metadata_bytes) fail(RLQ_GGUF_LIMIT, out.data_offset);
    if (offset > UINT64_MAX - out.data_offset) fail(RLQ_GGUF_INVALID, offset);
    out.file_bytes = out.data_offset + offset;
    return out;
}

struct Encoder {
    std::vector<uint8_t>& out;
    void raw(const void* p, size_t n) { out.insert(out.end(), (const uint8_t*)p, (const uint8_t*)p + n); }
    void u(uint64_t v, int n) {
        for (int i = 0; i < n; ++i) out.push_back((uint8_t)(v >> (8 * i)));
    }
    void string(const std::string& s) {
        u(s.size(), 8);
        raw(s.data(), s.size());
    }
    void scalar(uint32_t type, uint64_t bits) {
        const int n = type <= 1 || type == kBool ? 1 : type <= 3 ? 2 : type <= 6 ? 4 : 8;
        u(type == kBool ? (bits != 0) : bits, n);
    }
    void value(const Value& v) {
        if (v.type == kString) {
            string(v.str);
        } else if (v.type == kArray) {
            u(v.elem, 4);
            u(v.count(), 8);
            for (uint64_t i = 0; i < v.count(); ++i) {
                if (v.elem == kString) string(v.astr[i]);
                else scalar(v.elem, v.abits[i]);
            }
        } else {
            scalar(v.type, v.bits);
        }
    }
};

// The header bytes (with padding up to the data offset).
std::vector<uint8_t> encode_header(const std::vector<Kv>& kv, const std::vector<Tensor>& tensors, const Limits& L,
                                   const Policy& pol, Layout* lay_out) {
    const Layout lay = layout(kv, tensors, L, pol);
    std::vector<uint8_t> out;
    out.reserve(lay.data_offset);
    Encoder e{out};
    e.raw("GGUF", 4);
    e.u(pol.version, 4);
    e.u(tensors.size(), 8);
    e.u(kv.size(), 8);
    for (const Kv& k : kv) {
        e.string(*k.key);
        e.u(k.value->type, 4);
        e.value(*k.value);
    }
    for (size_t i = 0; i < tensors.size(); ++i) {
        const Tensor& t = tensors[i];
        e.string(pol.native ? c_string(t.name) : t.name);
        const uint32_t rank = pol.native ? native_rank(t) : t.n_dims;
        e.u(rank, 4);
        for (uint32_t d = 0; d < rank; ++d) e.u(d < t.n_dims ? t.dims[d] : 1, 8);
        e.u(t.dtype, 4);
        e.u(lay.offsets[i], 8);
    }
    if (out.size() > lay.data_offset) fail(RLQ_GGUF_INVALID, out.size());  // preflight and encoding disagree
    out.resize(lay.data_offset, 0);
    if (lay_out) *lay_out = lay;
    return out;
}

// Values and descriptors from the C structs (validated by the layout).
Value from_c(const rlq_gguf_kv& k) {
    Value v;
    v.type = k.type;
    auto scalar_bits = [](uint32_t type, const uint8_t* p) {
        const int n = type <= 1 || type == kBool ? 1 : type <= 3 ? 2 : type <= 6 ? 4 : 8;
        uint64_t b = 0;
        for (int i = 0; i < n; ++i) b |= (uint64_t)p[i] << (8 * i);
        return b;
    };
    if (k.type == kString) {
        if (k.count && !k.data) fail(RLQ_INVALID_ARGUMENT);
        v.str.assign((const char*)k.data, k.count);
    } else if (k.type == kArray) {
        v.elem = k.element_type;
        if (k.count && !k.data) fail(RLQ_INVALID_ARGUMENT);
        const uint8_t* p = (const uint8_t*)k.data;
        if (v.elem == kString) {
            if (k.count && !k.lengths) fail(RLQ_INVALID_ARGUMENT);
            for (uint64_t i = 0; i < k.count; ++i) {
                v.astr.emplace_back((const char*)p, k.lengths[i]);
                p += k.lengths[i];
            }
        } else if (v.elem <= 12 && v.elem != kArray) {
            const int n = v.elem <= 1 || v.elem == kBool ? 1 : v.elem <= 3 ? 2 : v.elem <= 6 ? 4 : 8;
            for (uint64_t i = 0; i < k.count; ++i) v.abits.push_back(scalar_bits(v.elem, p + i * n));
        }
    } else if (k.type <= 12) {
        if (!k.data) fail(RLQ_INVALID_ARGUMENT);
        v.bits = scalar_bits(k.type, (const uint8_t*)k.data);
        if (k.type == kBool) v.bits = v.bits != 0;
    }
    return v;
}

Tensor from_c(const rlq_gguf_tensor& t) {
    Tensor o;
    if (t.name_len && !t.name) fail(RLQ_INVALID_ARGUMENT);
    o.name.assign((const char*)t.name, t.name_len);
    o.n_dims = t.n_dims;
    if (t.n_dims > 4) fail(RLQ_GGUF_INVALID, t.n_dims);
    for (uint32_t d = 0; d < t.n_dims; ++d) o.dims[d] = t.dims[d];
    o.dtype = t.dtype;
    return o;
}

}  // namespace gguf
}  // namespace rlq

struct rlq_gguf {
    rlq::gguf::File f;
};

using namespace rlq::gguf;

namespace {

int32_t set_err(rlq_error* err, int32_t code, uint64_t a = 0, uint64_t b = 0) {
    if (err) *err = rlq_error{code, 0, a, b};
    return code;
}

template <typename F>
int32_t guarded(rlq_error* err, F&& body) {
    try {
        body();
        return set_err(err, RLQ_OK);
    } catch (const Fail& e) {
        return set_err(err, e.code, e.a, e.b);
    } catch (const std::bad_alloc&) {
        return set_err(err, RLQ_GGUF_LIMIT);
    }
}

}  // namespace

extern "C" {

int32_t rlq_gguf_open(const char* path, rlq_gguf** out, rlq_error* err) {
    if (!path || !out) return set_err(err, RLQ_INVALID_ARGUMENT);
    *out = nullptr;
    std::unique_ptr<rlq_gguf> g(new (std::nothrow) rlq_gguf);
    if (!g) return set_err(err, RLQ_ALLOCATION_FAILED);
    const int32_t rc = guarded(err, [&] {
        auto src = std::make_unique<FileSource>();
        src->f = fopen(path, "rb");
        if (!src->f) fail(RLQ_GGUF_IO, (uint64_t)errno);
        if (fseeko(src->f, 0, SEEK_END) != 0) fail(RLQ_GGUF_IO, (uint64_t)errno);
        const off_t end = ftello(src->f);
        if (end < 0) fail(RLQ_GGUF_IO, (uint64_t)errno);
        src->len = (uint64_t)end;
        src->win.resize(1u << 20);
        g->f.src = std::move(src);
        parse(g->f, true);
    });
    if (rc == RLQ_OK) *out = g.release();
    return rc;
}

int32_t rlq_gguf_read_header_memory(const uint8_t* bytes, uint64_t len, rlq_gguf** out, rlq_error* err) {
    if ((!bytes && len) || !out) return set_err(err, RLQ_INVALID_ARGUMENT);
    *out = nullptr;
    std::unique_ptr<rlq_gguf> g(new (std::nothrow) rlq_gguf);
    if (!g) return set_err(err, RLQ_ALLOCATION_FAILED);
    const int32_t rc = guarded(err, [&] {
        auto src = std::make_unique<MemSource>();
        src->bytes.assign(bytes, bytes + len);
        src->len = len;
        g->f.src = std::move(src);
        parse(g->f, false);
    });
    if (rc == RLQ_OK) *out = g.release();
    return rc;
}

void rlq_gguf_close(rlq_gguf* g) { delete g; }

void rlq_gguf_header(const rlq_gguf* g, uint32_t* version, uint32_t* alignment, uint64_t* data_offset,
                     uint64_t* n_kv, uint64_t* n_tensors, int32_t* big_endian) {
    if (!g) return;
    if (version) *version = g->f.version;
    if (alignment) *alignment = g->f.alignment;
    if (data_offset) *data_offset = g->f.data_offset;
    if (n_kv) *n_kv = g->f.keys.size();
    if (n_tensors) *n_tensors = g->f.tensors.size();
    if (big_endian) *big_endian = g->f.big ? 1 : 0;
}

int32_t rlq_gguf_kv_at(const rlq_gguf* g, uint64_t i, const uint8_t** key, uint64_t* key_len, uint32_t* type,
                       uint32_t* element_type, uint64_t* count, rlq_error* err) {
    if (!g || i >= g->f.keys.size()) return set_err(err, RLQ_INVALID_ARGUMENT, i);
    const Value& v = g->f.values[i];
    if (key) *key = (const uint8_t*)g->f.keys[i].data();
    if (key_len) *key_len = g->f.keys[i].size();
    if (type) *type = v.type;
    if (element_type) *element_type = v.elem;
    if (count) *count = v.count();
    return set_err(err, RLQ_OK);
}

int32_t rlq_gguf_kv_scalar(const rlq_gguf* g, uint64_t i, uint64_t j, uint64_t* bits, rlq_error* err) {
    if (!g || !bits || i >= g->f.keys.size()) return set_err(err, RLQ_INVALID_ARGUMENT, i);
    const Value& v = g->f.values[i];
    if (v.type == kArray && v.elem != kString && j < v.abits.size()) *bits = v.abits[j];
    else if (v.type != kArray && v.type != kString && j == 0) *bits = v.bits;
    else return set_err(err, RLQ_INVALID_ARGUMENT, i, j);
    return set_err(err, RLQ_OK);
}

int32_t rlq_gguf_kv_string(const rlq_gguf* g, uint64_t i, uint64_t j, const uint8_t** s, uint64_t* len,
                           rlq_error* err) {
    if (!g || !s || !len || i >= g->f.keys.size()) return set_err(err, RLQ_INVALID_ARGUMENT, i);
    const Value& v = g->f.values[i];
    const std::string* str = nullptr;
    if (v.type == kString && j == 0) str = &v.str;
    else if (v.type == kArray && v.elem == kString && j < v.astr.size()) str = &v.astr[j];
    if (!str) return set_err(err, RLQ_INVALID_ARGUMENT, i, j);
    *s = (const uint8_t*)str->data();
    *len = str->size();
    return set_err(err, RLQ_OK);
}

int64_t rlq_gguf_find_kv(const rlq_gguf* g, const uint8_t* key, uint64_t len) {
    if (!g || (!key && len)) return -1;
    const std::string want = c_string(std::string((const char*)key, len));
    for (size_t i = 0; i < g->f.keys.size(); ++i)
        if (c_string(g->f.keys[i]) == want) return (int64_t)i;
    return -1;
}

int32_t rlq_gguf_tensor_at(const rlq_gguf* g, uint64_t i, const uint8_t** name, uint64_t* name_len, uint32_t* n_dims,
                           uint64_t* dims, uint32_t* dtype, uint64_t* offset, uint64_t* bytes, rlq_error* err) {
    if (!g || i >= g->f.tensors.size()) return set_err(err, RLQ_INVALID_ARGUMENT, i);
    const Tensor& t = g->f.tensors[i];
    if (name) *name = (const uint8_t*)t.name.data();
    if (name_len) *name_len = t.name.size();
    if (n_dims) *n_dims = t.n_dims;
    if (dims)
        for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (dtype) *dtype = t.dtype;
    if (offset) *offset = t.offset;
    if (bytes) *bytes = t.bytes;
    return set_err(err, RLQ_OK);
}

int64_t rlq_gguf_find_tensor(const rlq_gguf* g, const uint8_t* name, uint64_t len) {
    if (!g || (!name && len)) return -1;
    const std::string want = c_string(std::string((const char*)name, len));
    for (size_t i = 0; i < g->f.tensors.size(); ++i)
        if (c_string(g->f.tensors[i].name) == want) return (int64_t)i;
    return -1;
}

int32_t rlq_gguf_read_tensor(rlq_gguf* g, uint64_t i, void* out, uint64_t out_len, rlq_error* err) {
    if (!g || i >= g->f.tensors.size()) return set_err(err, RLQ_INVALID_ARGUMENT, i);
    const Tensor& t = g->f.tensors[i];
    if (out_len != t.bytes) return set_err(err, RLQ_INVALID_LENGTH, t.bytes, out_len);
    if (!out && t.bytes) return set_err(err, RLQ_INVALID_ARGUMENT, i);
    return guarded(err, [&] {
        if (t.bytes > g->f.limits.max_tensor_read_bytes) fail(RLQ_GGUF_LIMIT, t.bytes);
        uint64_t start, end;
        if (__builtin_add_overflow(g->f.data_offset, t.offset, &start) || __builtin_add_overflow(start, t.bytes, &end) ||
            end > g->f.file_len)
            fail(RLQ_GGUF_INVALID, t.offset);  // tensor read exceeds file length
        if (t.bytes) g->f.src->read_at(start, out, t.bytes);
    });
}

int32_t rlq_gguf_native_header(const rlq_gguf* g, uint8_t* out, uint64_t cap, uint64_t* len, rlq_error* err) {
    if (!g || !len) return set_err(err, RLQ_INVALID_ARGUMENT);
    return guarded(err, [&] {
        std::vector<Kv> kv;
        for (size_t i = 0; i < g->f.keys.size(); ++i) kv.push_back(Kv{&g->f.keys[i], &g->f.values[i]});
        Policy pol;
        pol.native = true;
        pol.version = g->f.version;
        pol.alignment = g->f.alignment;
        const std::vector<uint8_t> bytes = encode_header(kv, g->f.tensors, g->f.limits, pol, nullptr);
        *len = bytes.size();
        if (out && cap >= bytes.size()) memcpy(out, bytes.data(), bytes.size());
        else if (out) fail(RLQ_INVALID_LENGTH, bytes.size(), cap);
    });
}

int32_t rlq_gguf_write_header(const rlq_gguf_kv* kv, uint64_t n_kv, const rlq_gguf_tensor* tensors, uint64_t n_tensors,
                              uint8_t* out, uint64_t cap, uint64_t* len, uint64_t* file_bytes, rlq_error* err) {
    if ((!kv && n_kv) || (!tensors && n_tensors) || !len) return set_err(err, RLQ_INVALID_ARGUMENT);
    return guarded(err, [&] {
        std::vector<std::string> keys;
        std::vector<Value> values;
        std::vector<Tensor> ts;
        keys.reserve(n_kv), values.reserve(n_kv), ts.reserve(n_tensors);
        for (uint64_t i = 0; i < n_kv; ++i) {
            if (!kv[i].key && kv[i].key_len) fail(RLQ_INVALID_ARGUMENT, i);
            keys.emplace_back((const char*)kv[i].key, kv[i].key_len);
            values.push_back(from_c(kv[i]));
        }
        std::vector<Kv> refs;
        for (uint64_t i = 0; i < n_kv; ++i) refs.push_back(Kv{&keys[i], &values[i]});
        for (uint64_t i = 0; i < n_tensors; ++i) ts.push_back(from_c(tensors[i]));
        Layout lay;
        const std::vector<uint8_t> bytes = encode_header(refs, ts, Limits{}, Policy{}, &lay);
        *len = bytes.size();
        if (file_bytes) *file_bytes = lay.file_bytes;
        if (out && cap >= bytes.size()) memcpy(out, bytes.data(), bytes.size());
        else if (out) fail(RLQ_INVALID_LENGTH, bytes.size(), cap);
    });
}

int32_t rlq_gguf_write(const char* path, const rlq_gguf_kv* kv, uint64_t n_kv, const rlq_gguf_tensor* tensors,
                       uint64_t n_tensors, rlq_error* err) {
    if (!path || (!kv && n_kv) || (!tensors && n_tensors)) return set_err(err, RLQ_INVALID_ARGUMENT);
    return guarded(err, [&] {
        std::vector<std::string> keys;
        std::vector<Value> values;
        std::vector<Tensor> ts;
        for (uint64_t i = 0; i < n_kv; ++i) {
            if (!kv[i].key && kv[i].key_len) fail(RLQ_INVALID_ARGUMENT, i);
            keys.emplace_back((const char*)kv[i].key, kv[i].key_len);
            values.push_back(from_c(kv[i]));
        }
        std::vector<Kv> refs;
        for (uint64_t i = 0; i < n_kv; ++i) refs.push_back(Kv{&keys[i], &values[i]});
        for (uint64_t i = 0; i < n_tensors; ++i) ts.push_back(from_c(tensors[i]));
        Layout lay;
        const std::vector<uint8_t> header = encode_header(refs, ts, Limits{}, Policy{}, &lay);
        for (uint64_t i = 0; i < n_tensors; ++i)
            if (!tensors[i].data && tensor_bytes(ts[i].dtype, ts[i].dims, ts[i].n_dims, 0)) fail(RLQ_INVALID_ARGUMENT, i);
        // validation is complete: write the header, then each payload and its padding
        FILE* f = fopen(path, "wb");
        if (!f) fail(RLQ_GGUF_IO, (uint64_t)errno);
        std::unique_ptr<FILE, int (*)(FILE*)> closer(f, fclose);
        if (fwrite(header.data(), 1, header.size(), f) != header.size()) fail(RLQ_GGUF_IO, (uint64_t)errno);
        static const uint8_t zeros[4096] = {0};
        for (uint64_t i = 0; i < n_tensors; ++i) {
            const uint64_t bytes = tensor_bytes(ts[i].dtype, ts[i].dims, ts[i].n_dims, 0);
            if (bytes && fwrite(tensors[i].data, 1, bytes, f) != bytes) fail(RLQ_GGUF_IO, (uint64_t)errno);
            uint64_t pad = align_up(bytes, lay.alignment) - bytes;
            while (pad) {
                const size_t n = pad < sizeof(zeros) ? (size_t)pad : sizeof(zeros);
                if (fwrite(zeros, 1, n, f) != n) fail(RLQ_GGUF_IO, (uint64_t)errno);
                pad -= n;
            }
        }
        if (fflush(f) != 0) fail(RLQ_GGUF_IO, (uint64_t)errno);
    });
}

}  // extern "C"
