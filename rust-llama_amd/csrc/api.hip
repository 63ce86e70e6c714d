// api.hip - the C ABI (include/rlq.h) over the gfx950 kernels.
//
// Validation order follows the reference function each entry point replaces
// (cited per function).  Data checks that need the input values (finite scan,
// scale preflight) run on the GPU inside the quantizer kernels and land in a
// device error word; nothing is copied to the caller when it is set.
#include "rlq.h"

#include <math.h>
#include <string.h>

#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "rlq_device.hpp"
#include "rlq_internal.hpp"
#include "rlq_dtype.hpp"
#include "rlq_layout.hpp"

using namespace rlq;

namespace {

int32_t fail(rlq_error* err, int32_t code, uint32_t dtype = 0, uint64_t a = 0, uint64_t b = 0) {
    if (err) *err = rlq_error{code, dtype, a, b};
    return code;
}
int32_t ok(rlq_error* err) { return fail(err, RLQ_OK); }

int32_t hip_fail(rlq_error* err, hipError_t e) { return fail(err, RLQ_DEVICE_ERROR, 0, (uint64_t)e); }

#define HIP_TRY(expr)                                  \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) return hip_fail(err, e_); \
    } while (0)

// DType::row_bytes
int32_t row_bytes(uint32_t t, uint64_t elements, uint64_t* out, rlq_error* err) {
    if (!dtype_known(t)) return fail(err, RLQ_INVALID_TYPE, t);
    const uint64_t bs = block_size(t);
    if (elements % bs != 0) return fail(err, RLQ_NON_MULTIPLE, t, elements, bs);
    uint64_t r;
    if (__builtin_mul_overflow(elements / bs, type_size(t), &r)) return fail(err, RLQ_SIZE_OVERFLOW, t);
    *out = r;
    return ok(err);
}

// lib.rs:310-319
int32_t validate(uint32_t t, uint64_t bytes, uint64_t elements, rlq_error* err) {
    uint64_t expected;
    const int32_t rc = row_bytes(t, elements, &expected, err);
    if (rc) return rc;
    if (bytes != expected) return fail(err, RLQ_INVALID_LENGTH, t, expected, bytes);
    return ok(err);
}

// matvec.rs:7-18
int32_t activation_dtype(uint32_t w, uint32_t* out, rlq_error* err) {
    if (!dtype_known(w)) return fail(err, RLQ_INVALID_TYPE, w);
    switch (w) {
        case 41: case 42: case 2: case 6: case 8: case 39: case 40: case 20: *out = 8; break;
        case 3: case 7: *out = 9; break;
        case 10: case 11: case 12: case 13: case 14: case 16: case 17: case 22: case 18: case 21: case 19: case 29:
        case 23: case 34: case 35:
            *out = 15;
            break;
        case 0: case 1: case 43: *out = 0; break;
        case 30: *out = 30; break;
        default: return fail(err, RLQ_UNSUPPORTED_MATVEC, w);
    }
    return ok(err);
}

bool path_weight(uint32_t t) {
    return t == kQ8_0 || t == kQ2_K || t == kQ3_K || t == kQ4_K || t == kQ5_K || t == kQ6_K;
}

// Batches up to this size run the decode kernels (one pass over the weights
// per 8 columns); larger Q4_K batches run the prefill GEMM.
constexpr uint64_t kDecodeMaxBatch = 8;

// ---- device buffers ---------------------------------------------------------

struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
};

}  // namespace

struct rlq_context {
    int device = 0;
    uint8_t* scratch = nullptr;  // this device's copy of the static `scratch` array (rlq_matmul_noalloc)
    hipStream_t stream = nullptr;
    unsigned long long* err_words = nullptr;  // [0] device API (sticky), [1] host API (per call)
    unsigned long long* host_err = nullptr;   // pinned readback
    // keys: the decode launches' argmax state (kArgmaxStateBytes; its counter
    // set to 0 when the buffer is made, and left at 0 by every launch), then
    // the prefill path's per-column keys
    DevBuf planes, keys, stage_in, stage_w, stage_out, gate;
};

struct rlq_weights {
    int device;  // the creating context's device; the handle may outlive that context
    uint32_t dtype;
    uint64_t rows, cols;
    uint8_t* dev;
    uint64_t bytes;                  // GGUF bytes of all matrices
    uint64_t n2 = 1, n3 = 1;         // stacked matrices (GGML ne[2], ne[3])
    uint64_t mat_bytes = 0;          // device bytes of one tiled matrix
};

namespace {

// Grow-only scratch.  Growing waits for the whole device first (callers may
// pass their own streams), so no kernel still reads the old buffer when it is
// freed.  *grown (may be null) tells whether the buffer was replaced: its
// contents are then undefined, even when the allocator hands back the old
// address.
hipError_t ensure(rlq_context* ctx, DevBuf& b, size_t need, bool* grown = nullptr) {
    (void)ctx;
    if (grown) *grown = false;
    if (b.n >= need) return hipSuccess;
    if (grown) *grown = true;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.n = 0;
    size_t n = need < 4096 ? 4096 : need;
    e = hipMalloc(&b.p, n);
    if (e != hipSuccess) return e;
    b.n = n;
    return hipSuccess;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) (void)hipSetDevice(dev);
        else prev = -1;
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// Device calls run on the caller's stream; NULL is HIP's null stream.
hipStream_t pick(rlq_context* ctx, void* stream) {
    (void)ctx;
    return (hipStream_t)stream;
}

// A model stage (rlq_device.hpp ModelStage) as the reference reports it: the
// QuantError of an activation quantizer (0), or the NonFinite check (rlq.h
// rlq_nonfinite_check).
uint32_t stage_check(uint32_t stage) {
    switch (stage) {
        case kStAttnNormScale: case kStFfnNormScale: return RLQ_CHECK_RMS_SCALE;
        case kStAttnNormOut: case kStFfnNormOut: return RLQ_CHECK_RMS_OUTPUT;
        case kStOIn: case kStDownIn: return RLQ_CHECK_MATRIX_INPUT;
        case kStQkvOut: case kStOOut: case kStGuOut: case kStDownOut: return RLQ_CHECK_MATRIX_OUTPUT;
        case kStScore: return RLQ_CHECK_ATTENTION_SCORE;
        case kStAttnOut: return RLQ_CHECK_ATTENTION_OUTPUT;
        case kStLayerOut: return RLQ_CHECK_LAYER_OUTPUT;
        default: return 0;  // kStQkvQuant, kStOQuant, kStGuQuant, kStDownQuant
    }
}

// Decode an error key (see rlq_device.hpp) into an rlq_error.
int32_t key_to_error(unsigned long long key, uint32_t dtype, rlq_error* err) {
    if (key == ~0ull) return ok(err);
    const uint64_t field = key >> 41, kind = (key >> 40) & 1, index = key & ((1ull << 40) - 1);
    if (field == kModelField) {  // model-runtime checks: layer, stage, index
        const uint64_t layer = (key >> 25) & 0xffff, stage = (key >> 20) & 31, idx = key & 0xfffff;
        const uint32_t check = stage_check((uint32_t)stage);
        if (check == 0) return fail(err, RLQ_UNREPRESENTABLE_SCALE, dtype, idx, layer);
        return fail(err, RLQ_NON_FINITE, dtype, check, layer);
    }
    if (field == 0) return fail(err, RLQ_TENSOR_BOUNDS, dtype, index);
    return fail(err, kind == (uint64_t)kKindNonFinite ? RLQ_NON_FINITE_INPUT : RLQ_UNREPRESENTABLE_SCALE, dtype,
                index, field - 1);
}

// Read and clear error word `slot` after the stream drains.
int32_t take_error(rlq_context* ctx, int slot, hipStream_t s, uint32_t dtype, rlq_error* err) {
    HIP_TRY(hipMemcpyAsync(ctx->host_err, ctx->err_words + slot, 8, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    const unsigned long long key = *ctx->host_err;
    if (key != ~0ull) {
        HIP_TRY(launch_fill_u64(ctx->err_words + slot, 1, ~0ull, s));
        HIP_TRY(hipStreamSynchronize(s));
    }
    return key_to_error(key, dtype, err);
}

// The context of the entry points that take none (rlq_quantize_into and the
// like), created on first use under g_default_mu.  It is never handed to a
// caller and never destroyed: it lives until the process ends, and no static
// destructor or exit handler of this library calls HIP.
std::mutex g_default_mu;
rlq_context* g_default = nullptr;

}  // namespace

// ---- static scratch of rlq_matmul_noalloc ----------------------------------
// Device memory that rlq_matmul_noalloc uses instead of allocating: with an
// argmax, the decode launches' argmax state (kArgmaxStateBytes) and, on the
// prefill path, 8 bytes of keys per column (padded to 256); then the prefill
// GEMM's activation image (gemm_planes_bytes).  Each device holds its own
// copy for the life of the process.  Host code never passes the array's name
// to a kernel (on the host it is only a handle): every use goes through the
// device address hipGetSymbolAddress returns, taken once per device at
// context creation with that device current.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kScratchDevices = 256;
std::mutex g_scratch_mu;
uint8_t* g_scratch_addr[kScratchDevices];

// The calling thread's current device must be `device`.
hipError_t scratch_address(int device, uint8_t** out) {
    if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_addr[device] = (uint8_t*)p;
    }
    *out = g_scratch_addr[device];
    return hipSuccess;
}

int32_t default_context(rlq_context** out, rlq_error* err) {
    if (!g_default) {
        const int32_t rc = rlq_context_create(-1, &g_default, err);
        if (rc) return rc;
    }
    *out = g_default;
    return ok(err);
}

// Upload GGUF weights (host or device bytes) into a fresh device buffer in
// the tiled layout (rlq_layout.hpp).  Host bytes go through a temporary
// device copy that is freed before returning.
hipError_t upload_weights(uint32_t t, const void* bytes, uint64_t len, uint64_t rows, uint64_t cols, bool on_device,
                          uint8_t** dev, hipStream_t s, uint64_t mats = 1) {
    *dev = nullptr;
    const uint64_t mb = layout_bytes(t, rows, cols);
    hipError_t e = hipMalloc((void**)dev, mb * mats);
    if (e != hipSuccess) return e;
    const uint8_t* src = (const uint8_t*)bytes;
    void* tmp = nullptr;
    if (on_device) {
        e = hipDeviceSynchronize();  // the bytes may still be in flight on another stream
    } else {
        e = hipMalloc(&tmp, len);
        if (e == hipSuccess) e = hipMemcpyAsync(tmp, src, len, hipMemcpyHostToDevice, s);
        src = (const uint8_t*)tmp;
    }
    for (uint64_t m = 0; m < mats && e == hipSuccess; ++m)
        e = launch_repack(t, src + m * (len / mats), rows, cols, *dev + m * mb, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (tmp) (void)hipFree(tmp);
    if (e != hipSuccess) {
        (void)hipFree(*dev);
        *dev = nullptr;
    }
    return e;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" {

const char* rlq_status_string(int32_t code) {
    switch (code) {
        case RLQ_OK: return "ok";
        case RLQ_INVALID_TYPE: return "GGML type is unknown or reserved";
        case RLQ_UNSUPPORTED_MATVEC: return "no matrix-vector weight dot for this type";
        case RLQ_INVALID_VECTOR_LENGTH: return "wrong vector length";
        case RLQ_INVALID_MATRIX_SHAPE: return "matrix dimensions must be positive";
        case RLQ_NON_MULTIPLE: return "row length is not a multiple of the block size";
        case RLQ_SIZE_OVERFLOW: return "tensor byte length exceeds addressable memory";
        case RLQ_INVALID_LENGTH: return "wrong byte length";
        case RLQ_ALLOCATION_FAILED: return "unable to allocate tensor output";
        case RLQ_UNSUPPORTED_QUANTIZATION: return "encoder not available for this type";
        case RLQ_UNSUPPORTED_WEIGHTED_QUANTIZATION: return "importance-weighted encoder not available";
        case RLQ_IMPORTANCE_WEIGHTS_REQUIRED: return "the type requires importance weights";
        case RLQ_INVALID_IMPORTANCE_LENGTH: return "wrong importance weight count";
        case RLQ_INVALID_IMPORTANCE_WEIGHT: return "importance weight must be finite and nonnegative";
        case RLQ_UNSUPPORTED_INTEGER_CONVERSION: return "integer assignment not defined for this type";
        case RLQ_INTEGER_OUT_OF_RANGE: return "element outside the integer range";
        case RLQ_NON_FINITE_INPUT: return "non-finite quantizer input";
        case RLQ_UNREPRESENTABLE_SCALE: return "quantizer scale is not representable";
        case RLQ_DEVICE_ERROR: return "HIP runtime error";
        case RLQ_UNIMPLEMENTED: return "type or operation is outside the Q8_0/Q2_K..Q6_K path";
        case RLQ_INVALID_ARGUMENT: return "null pointer or handle";
        case RLQ_INVALID_CONFIG: return "invalid model configuration";
        case RLQ_INVALID_TOKEN: return "token outside the vocabulary";
        case RLQ_INVALID_STATE: return "KV cache is full";
        case RLQ_TENSOR_SHAPE: return "MUL_MAT / MUL_MAT_ID dimensions are incompatible";
        case RLQ_TENSOR_BOUNDS: return "expert id outside the expert tensor";
        case RLQ_TENSOR_UNSUPPORTED: return "right-hand side must be F32 or the activation type";
        case RLQ_GGUF_IO: return "GGUF file could not be read or written";
        case RLQ_GGUF_INVALID: return "GGUF file is malformed";
        case RLQ_GGUF_LIMIT: return "GGUF file exceeds a reader limit";
        case RLQ_GGUF_UNSUPPORTED: return "GGUF content is not supported";
        case RLQ_NON_FINITE: return "non-finite value";
        case RLQ_SCRATCH_LIMIT: return "workspace exceeds the library's static scratch";
        default: return "unknown status";
    }
}

int32_t rlq_row_bytes(uint32_t dtype, uint64_t elements, uint64_t* out, rlq_error* err) {
    uint64_t r = 0;
    const int32_t rc = row_bytes(dtype, elements, &r, err);
    if (rc == RLQ_OK && out) *out = r;
    return rc;
}

int32_t rlq_matvec_activation_dtype(uint32_t w, uint32_t* out, rlq_error* err) {
    uint32_t a = 0;
    const int32_t rc = activation_dtype(w, &a, err);
    if (rc == RLQ_OK && out) *out = a;
    return rc;
}

// ---- context ----------------------------------------------------------------

int32_t rlq_context_create(int32_t device, rlq_context** out, rlq_error* err) {
    if (!out) return fail(err, RLQ_INVALID_ARGUMENT);
    if (device < 0) HIP_TRY(hipGetDevice(&device));
    DeviceGuard g(device);
    rlq_context* ctx = new (std::nothrow) rlq_context;
    if (!ctx) return fail(err, RLQ_ALLOCATION_FAILED);
    ctx->device = device;
    hipError_t e = scratch_address(device, &ctx->scratch);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc((void**)&ctx->err_words, 2 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipHostMalloc((void**)&ctx->host_err, sizeof(unsigned long long), hipHostMallocDefault);
    if (e == hipSuccess) e = launch_fill_u64(ctx->err_words, 2, ~0ull, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        rlq_context_destroy(ctx);
        return hip_fail(err, e);
    }
    *out = ctx;
    return ok(err);
}

void rlq_context_destroy(rlq_context* ctx) {
    if (!ctx) return;
    DeviceGuard g(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (DevBuf* b : {&ctx->planes, &ctx->keys, &ctx->stage_in, &ctx->stage_w, &ctx->stage_out, &ctx->gate})
        if (b->p) (void)hipFree(b->p);
    if (ctx->err_words) (void)hipFree(ctx->err_words);
    if (ctx->host_err) (void)hipHostFree(ctx->host_err);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

void* rlq_context_stream(rlq_context* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

// ---- weights ------------------------------------------------------------------

// Matrix::from_quantized (crates/model-runtime/src/math.rs:35-70), for a
// stack of n2 x n3 matrices
int32_t rlq_weights_create_stacked(rlq_context* ctx, uint32_t dtype, const void* bytes, uint64_t len, uint64_t rows,
                                   uint64_t cols, uint64_t n2, uint64_t n3, int32_t bytes_on_device,
                                   rlq_weights** out, rlq_error* err) {
    if (!ctx || !out) return fail(err, RLQ_INVALID_ARGUMENT);
    uint32_t at;
    int32_t rc = activation_dtype(dtype, &at, err);
    if (rc) return rc;
    if (!path_weight(dtype)) return fail(err, RLQ_UNIMPLEMENTED, dtype);
    if (rows == 0 || cols == 0) return fail(err, RLQ_INVALID_MATRIX_SHAPE, dtype, rows, cols);
    if (n2 == 0 || n3 == 0) return fail(err, RLQ_TENSOR_SHAPE, dtype, n2, n3);
    uint64_t rb, expected, mats;
    rc = row_bytes(dtype, cols, &rb, err);
    if (rc) return rc;
    if (__builtin_mul_overflow(rb, rows, &expected) || __builtin_mul_overflow(n2, n3, &mats) ||
        __builtin_mul_overflow(expected, mats, &expected))
        return fail(err, RLQ_SIZE_OVERFLOW, dtype);
    if (len != expected) return fail(err, RLQ_INVALID_LENGTH, dtype, expected, len);
    if (!bytes) return fail(err, RLQ_INVALID_ARGUMENT, dtype);
    DeviceGuard g(ctx->device);
    rlq_weights* w = new (std::nothrow) rlq_weights{ctx->device, dtype, rows, cols, nullptr, len};
    if (!w) return fail(err, RLQ_ALLOCATION_FAILED);
    w->n2 = n2, w->n3 = n3, w->mat_bytes = layout_bytes(dtype, rows, cols);
    const hipError_t e =
        upload_weights(dtype, bytes, len, rows, cols, bytes_on_device != 0, &w->dev, ctx->stream, mats);
    if (e != hipSuccess) {
        delete w;
        return e == hipErrorOutOfMemory ? fail(err, RLQ_ALLOCATION_FAILED, dtype) : hip_fail(err, e);
    }
    *out = w;
    return ok(err);
}

int32_t rlq_weights_create(rlq_context* ctx, uint32_t dtype, const void* bytes, uint64_t len, uint64_t rows,
                           uint64_t cols, int32_t bytes_on_device, rlq_weights** out, rlq_error* err) {
    return rlq_weights_create_stacked(ctx, dtype, bytes, len, rows, cols, 1, 1, bytes_on_device, out, err);
}

void rlq_weights_destroy(rlq_weights* w) {
    if (!w) return;
    DeviceGuard g(w->device);
    // hipFree waits for every queued use of the buffer on the device.
    if (w->dev) (void)hipFree(w->dev);
    delete w;
}

void rlq_weights_shape(const rlq_weights* w, uint64_t* rows, uint64_t* cols, uint32_t* dtype) {
    if (!w) return;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (dtype) *dtype = w->dtype;
}

void rlq_weights_stack(const rlq_weights* w, uint64_t* n2, uint64_t* n3) {
    if (!w) return;
    if (n2) *n2 = w->n2;
    if (n3) *n3 = w->n3;
}

// ---- GGML MUL_MAT with broadcast, MUL_MAT_ID ---------------------------------------

namespace {

// Every right-hand column quantized once (F32) or taken as given (packed
// activation bytes) into the context's planes; then the gate kernel.
int32_t mm_stage(rlq_context* ctx, const rlq_weights* w, uint32_t at, uint32_t x_dtype, const void* x,
                 uint64_t columns, const int32_t* ids, uint64_t pairs, float* y, hipStream_t s, ActPlanes* planes,
                 uint32_t** gate, rlq_error* err) {
    const uint64_t K = w->cols, nb = K / block_size(at);
    HIP_TRY(ensure(ctx, ctx->planes, act_planes_bytes(at, K, columns)));
    HIP_TRY(ensure(ctx, ctx->gate, sizeof(uint32_t)));
    *planes = act_planes_carve(ctx->planes.p, at, K, columns);
    *gate = (uint32_t*)ctx->gate.p;
    if (x_dtype == 0) {
        if (at == kQ8_K) HIP_TRY(launch_quantize_q8k((const float*)x, K, columns, planes, nullptr, ctx->err_words, s));
        else HIP_TRY(launch_quantize_q8_0((const float*)x, K, columns, planes, nullptr, ctx->err_words, s));
    } else {
        HIP_TRY(launch_act_from_gguf(at, (const uint8_t*)x, K, columns, planes, s));
    }
    HIP_TRY(launch_mm_prepare(ids, pairs, (uint32_t)w->n2, planes->bad, columns * nb, y, w->rows, *gate,
                              ctx->err_words, s));
    return ok(err);
}

// Common argument checks: (x_dtype, x alignment, column count).
int32_t mm_check_rhs(const rlq_weights* w, uint32_t at, uint32_t x_dtype, const void* x, const float* y,
                     uint64_t columns, rlq_error* err) {
    if (x_dtype != 0 && x_dtype != at) return fail(err, RLQ_TENSOR_UNSUPPORTED, x_dtype);
    if (!x || !y) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    if ((x_dtype == 0 && ((uintptr_t)x & 15)) || ((uintptr_t)y & 3)) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    // one quantizer launch covers every column (grid rows), and error keys
    // carry the column
    if (columns > 65535) return fail(err, RLQ_UNIMPLEMENTED, w->dtype, columns, 65535);
    return ok(err);
}

}  // namespace

// MUL_MAT (crates/tensor/src/cpu_extra.rs:756-873)
int32_t rlq_mul_mat(rlq_context* ctx, const rlq_weights* w, uint32_t x_dtype, const void* x, uint64_t ncols,
                    uint64_t n2, uint64_t n3, float* y, void* stream, rlq_error* err) {
    if (!ctx || !w) return fail(err, RLQ_INVALID_ARGUMENT);
    uint32_t at;
    int32_t rc = activation_dtype(w->dtype, &at, err);
    if (rc) return rc;
    if (n2 % w->n2 != 0 || n3 % w->n3 != 0) return fail(err, RLQ_TENSOR_SHAPE, w->dtype, n2, n3);  // :759-769
    uint64_t columns;
    if (__builtin_mul_overflow(ncols, n2, &columns) || __builtin_mul_overflow(columns, n3, &columns))
        return fail(err, RLQ_SIZE_OVERFLOW, w->dtype);
    if (x_dtype != 0 && x_dtype != at) return fail(err, RLQ_TENSOR_UNSUPPORTED, x_dtype);  // :779-784
    if (columns == 0) return ok(err);
    rc = mm_check_rhs(w, at, x_dtype, x, y, columns, err);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    const hipStream_t s = pick(ctx, stream);
    if (columns == 1 && x_dtype == 0) {  // one f32 column: one launch that quantizes it in every workgroup
        HIP_TRY(launch_matvec_ex(w->dtype, w->dev, w->rows, w->cols, (const float*)x, nullptr, 1, y, w->rows,
                                 nullptr, ctx->err_words, nullptr, nullptr, MvExtra{}, s));
        return ok(err);
    }
    ActPlanes planes;
    uint32_t* gate;
    rc = mm_stage(ctx, w, at, x_dtype, x, columns, nullptr, 0, y, s, &planes, &gate, err);
    if (rc) return rc;
    const uint64_t K = w->cols, nb = K / block_size(at), r2 = n2 / w->n2, r3 = n3 / w->n3;
    for (uint64_t i3 = 0; i3 < n3; ++i3)
        for (uint64_t i2 = 0; i2 < n2; ++i2) {
            const uint64_t slice = i3 * n2 + i2, c0 = slice * ncols;
            const uint64_t m = (i3 / r3) * w->n2 + i2 / r2;  // the broadcast source matrix
            ActPlanes p = planes;
            p.q += c0 * K;
            p.d += c0 * nb;
            p.bad += c0 * nb;
            if (p.bsum) p.bsum += c0 * (K / 16);
            MvExtra ex;
            ex.gate = gate;
            ex.column_base = c0;
            HIP_TRY(launch_matvec_ex(w->dtype, w->dev + m * w->mat_bytes, w->rows, K, nullptr, &p, ncols,
                                     y + c0 * w->rows, w->rows, nullptr, ctx->err_words, nullptr, nullptr, ex, s));
        }
    return ok(err);
}

// MUL_MAT_ID (crates/tensor/src/cpu_index.rs:169-236)
int32_t rlq_mul_mat_id(rlq_context* ctx, const rlq_weights* w, uint32_t x_dtype, const void* x, uint64_t ncols,
                       uint64_t tokens, const int32_t* ids, uint64_t slots, float* y, void* stream,
                       rlq_error* err) {
    if (!ctx || !w) return fail(err, RLQ_INVALID_ARGUMENT);
    uint32_t at;
    int32_t rc = activation_dtype(w->dtype, &at, err);
    if (rc) return rc;
    if (w->n3 != 1 || ncols == 0 || slots % ncols != 0)  // :179-194
        return fail(err, RLQ_TENSOR_SHAPE, w->dtype, slots, ncols);
    if (x_dtype != 0 && x_dtype != at) return fail(err, RLQ_TENSOR_UNSUPPORTED, x_dtype);  // :195-199
    uint64_t pairs, columns;
    if (__builtin_mul_overflow(tokens, slots, &pairs) || __builtin_mul_overflow(tokens, ncols, &columns))
        return fail(err, RLQ_SIZE_OVERFLOW, w->dtype);
    if (pairs == 0) return ok(err);  // :205-208: an empty output
    if (!ids) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    if (w->n2 > 0x7fffffffull) return fail(err, RLQ_UNIMPLEMENTED, w->dtype, w->n2);
    rc = mm_check_rhs(w, at, x_dtype, x, y, columns, err);
    if (rc) return rc;
    if (pairs > 0xffffffffull) return fail(err, RLQ_UNIMPLEMENTED, w->dtype, pairs);
    DeviceGuard g(ctx->device);
    const hipStream_t s = pick(ctx, stream);
    MvExtra ex;
    ex.ids = ids;
    ex.id_pairs = pairs;
    ex.id_slots = (uint32_t)slots;
    ex.id_cols = (uint32_t)ncols;
    ex.id_experts = (uint32_t)w->n2;
    ex.expert_bytes = w->mat_bytes;
    // one token with one f32 column (MoE decode): a single launch checks the
    // ids and quantizes the column in every workgroup; otherwise the column
    // planes, the gate and the product
    if (tokens == 1 && ncols == 1 && x_dtype == 0 && ((uintptr_t)x & 15) == 0) {
        ex.id_inline = true;
        HIP_TRY(launch_matvec_ex(w->dtype, w->dev, w->rows, w->cols, (const float*)x, nullptr, 1, y, w->rows,
                                 nullptr, ctx->err_words, nullptr, nullptr, ex, s));
        return ok(err);
    }
    ActPlanes planes;
    uint32_t* gate;
    rc = mm_stage(ctx, w, at, x_dtype, x, columns, ids, pairs, y, s, &planes, &gate, err);
    if (rc) return rc;
    ex.gate = gate;
    HIP_TRY(launch_matvec_ex(w->dtype, w->dev, w->rows, w->cols, nullptr, &planes, 1, y, w->rows, nullptr,
                             ctx->err_words, nullptr, nullptr, ex, s));
    return ok(err);
}

// ---- device matmul --------------------------------------------------------------

// Q4_K / Q5_K columns from this many per launch on are quantized once by the
// planes kernel instead of in every workgroup's prologue (with one workgroup
// per CU; 14336x4096 batch 8: 12.6 us for both launches against 12.9 us
// fused, batch 6: 12.5 against 11.8; 6144x4096 batch 8: 9.8 against 10.9).
constexpr uint64_t kPlanesMinBatch = 7;

// The decode launch of `batch` (<= 8) f32 columns: the fused kernels, or the
// Q8_K planes kernel and then the matvec over the planes.
static hipError_t decode_launch(rlq_context* ctx, const rlq_weights* w, const float* x, uint64_t batch, float* y,
                                const MvArgmax* am, int32_t* isum, int32_t* imin, const MvExtra& ex, hipStream_t s) {
    if ((w->dtype == kQ4_K || w->dtype == kQ5_K) && batch >= kPlanesMinBatch && ex.epilogue == 0) {
        hipError_t e = ensure(ctx, ctx->planes, act_planes_bytes(kQ8_K, w->cols, batch));
        if (e != hipSuccess) return e;
        const ActPlanes pl = act_planes_carve(ctx->planes.p, kQ8_K, w->cols, batch);
        e = launch_quantize_q8k(x, w->cols, batch, &pl, nullptr, ctx->err_words, s);
        if (e != hipSuccess) return e;
        return launch_matvec_ex(w->dtype, w->dev, w->rows, w->cols, nullptr, &pl, batch, y, w->rows, am,
                                ctx->err_words, isum, imin, ex, s);
    }
    return launch_matvec_ex(w->dtype, w->dev, w->rows, w->cols, x, nullptr, batch, y, w->rows, am, ctx->err_words,
                            isum, imin, ex, s);
}

// Columns per call: an error key holds column + 1 in 23 bits below the
// model runtime's field 0x7fffff (rlq_device.hpp).
constexpr uint64_t kMaxKeyColumns = (1ull << 23) - 2;

static int32_t matmul_impl(rlq_context* ctx, const rlq_weights* w, const float* x, uint64_t batch, float* y,
                           uint32_t* argmax, void* stream, rlq_error* err) {
    if (!ctx || !w || !x || !y) return fail(err, RLQ_INVALID_ARGUMENT);
    if (((uintptr_t)x & 15) || ((uintptr_t)y & 3)) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    if (batch == 0) return ok(err);
    if (batch > kMaxKeyColumns) return fail(err, RLQ_UNIMPLEMENTED, w->dtype, batch, kMaxKeyColumns);
    DeviceGuard g(ctx->device);
    const hipStream_t s = pick(ctx, stream);
    const bool gemm = w->dtype == kQ4_K && batch > kDecodeMaxBatch;
    if (argmax) {
        bool grown = false;
        HIP_TRY(ensure(ctx, ctx->keys, kArgmaxStateBytes + (gemm ? batch * sizeof(unsigned long long) : 0), &grown));
        if (grown) HIP_TRY(launch_fill_u64((unsigned long long*)ctx->keys.p, 1, 0ull, s));  // the arrival counter
    }
    if (gemm) {  // prefill: the MFMA GEMM, then the argmax over the stored rows
        HIP_TRY(ensure(ctx, ctx->planes, gemm_planes_bytes(batch, w->cols)));
        HIP_TRY(launch_gemm_q4k(w->dev, w->rows, w->cols, x, batch, y, w->rows, ctx->planes.p, ctx->err_words, nullptr,
                                nullptr, s));
        if (argmax) {
            unsigned long long* keys = (unsigned long long*)((uint8_t*)ctx->keys.p + kArgmaxStateBytes);
            HIP_TRY(launch_fill_u64(keys, batch, 0ull, s));
            HIP_TRY(launch_argmax_rows(y, batch, w->rows, keys, s));
            HIP_TRY(launch_argmax_finish(keys, batch, y, w->rows, argmax, s));
        }
    } else {  // decode: the argmax is finished inside each launch
        const MvArgmax am = argmax_state(ctx->keys.p, argmax);
        HIP_TRY(decode_launch(ctx, w, x, batch, y, argmax ? &am : nullptr, nullptr, nullptr, MvExtra{}, s));
    }
    return ok(err);
}

int32_t rlq_matmul(rlq_context* ctx, const rlq_weights* w, const float* x, uint64_t batch, float* y, void* stream,
                   rlq_error* err) {
    return matmul_impl(ctx, w, x, batch, y, nullptr, stream, err);
}

// Matrix::multiply (crates/model-runtime/src/math.rs:144-169): the input's
// finite scan is the quantizer's own (the first non-finite value refuses the
// call), then the product, then the finite scan of the outputs.
int32_t rlq_multiply(rlq_context* ctx, const rlq_weights* w, const float* x, float* y, void* stream, rlq_error* err) {
    if (!ctx || !w || !x || !y) return fail(err, RLQ_INVALID_ARGUMENT);
    if (((uintptr_t)x & 15) || ((uintptr_t)y & 3)) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    DeviceGuard g(ctx->device);
    MvExtra ex;
    ex.chk = mv_chk(0, kStOIn, kStOQuant, kStOOut, 0);  // matrix input, the quantizer, matrix output
    HIP_TRY(launch_matvec_ex(w->dtype, w->dev, w->rows, w->cols, x, nullptr, 1, y, w->rows, nullptr, ctx->err_words,
                             nullptr, nullptr, ex, pick(ctx, stream)));
    return ok(err);
}

int32_t rlq_matmul_argmax(rlq_context* ctx, const rlq_weights* w, const float* x, uint64_t batch, float* y,
                          uint32_t* argmax, void* stream, rlq_error* err) {
    if (!argmax) return fail(err, RLQ_INVALID_ARGUMENT);
    return matmul_impl(ctx, w, x, batch, y, argmax, stream, err);
}

// rlq_matmul / rlq_matmul_argmax on the same kernels, with every buffer
// beyond the inputs and outputs taken from this device's static scratch:
// nothing is allocated or freed.  The keys are cleared by a fill kernel
// (never a memset, so the call may be captured in a graph).
int32_t rlq_matmul_noalloc(rlq_context* ctx, const rlq_weights* w, const float* x, uint64_t batch, float* y,
                           uint32_t* argmax, void* stream, rlq_error* err) {
    if (!ctx || !w || !x || !y) return fail(err, RLQ_INVALID_ARGUMENT);
    if (((uintptr_t)x & 15) || ((uintptr_t)y & 3)) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    if (batch == 0) return ok(err);
    if (batch > kMaxKeyColumns) return fail(err, RLQ_UNIMPLEMENTED, w->dtype, batch, kMaxKeyColumns);
    const bool gemm = w->dtype == kQ4_K && batch > kDecodeMaxBatch;
    const uint64_t state_bytes = argmax ? kArgmaxStateBytes : 0;
    const uint64_t keys_bytes = argmax && gemm ? (batch * 8 + 255) / 256 * 256 : 0;
    const uint64_t need = state_bytes + keys_bytes + (gemm ? gemm_planes_bytes(batch, w->cols) : 0);
    if (need > kScratchBytes) return fail(err, RLQ_SCRATCH_LIMIT, w->dtype, need, kScratchBytes);
    if (!ctx->scratch) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    DeviceGuard g(ctx->device);
    const hipStream_t s = pick(ctx, stream);
    // the scratch keeps the last call's contents: what must start at 0 is cleared
    if (argmax) HIP_TRY(launch_fill_u64((unsigned long long*)ctx->scratch, 1, 0ull, s));  // the arrival counter
    if (gemm) {
        HIP_TRY(launch_gemm_q4k(w->dev, w->rows, w->cols, x, batch, y, w->rows, ctx->scratch + state_bytes + keys_bytes,
                                ctx->err_words, nullptr, nullptr, s));
        if (argmax) {
            unsigned long long* keys = (unsigned long long*)(ctx->scratch + state_bytes);
            HIP_TRY(launch_fill_u64(keys, batch, 0ull, s));
            HIP_TRY(launch_argmax_rows(y, batch, w->rows, keys, s));
            HIP_TRY(launch_argmax_finish(keys, batch, y, w->rows, argmax, s));
        }
    } else {
        const MvArgmax am = argmax_state(ctx->scratch, argmax);
        HIP_TRY(launch_matvec(w->dtype, w->dev, w->rows, w->cols, x, nullptr, batch, y, w->rows,
                              argmax ? &am : nullptr, ctx->err_words, nullptr, nullptr, s));
    }
    return ok(err);
}

int32_t rlq_quantize_device(rlq_context* ctx, uint32_t dtype, const float* x, uint64_t cols, uint64_t batch,
                            uint8_t* out, void* stream, rlq_error* err) {
    if (!ctx) return fail(err, RLQ_INVALID_ARGUMENT);
    if (!dtype_known(dtype)) return fail(err, RLQ_INVALID_TYPE, dtype);
    if (dtype != kQ8_K && !path_weight(dtype)) return fail(err, RLQ_UNIMPLEMENTED, dtype);
    uint64_t rb, n;
    int32_t rc = row_bytes(dtype, cols, &rb, err);
    if (rc) return rc;
    if (__builtin_mul_overflow(cols, batch, &n)) return fail(err, RLQ_SIZE_OVERFLOW, dtype);
    if (n == 0) return ok(err);
    if (!x || !out || ((uintptr_t)x & 15)) return fail(err, RLQ_INVALID_ARGUMENT, dtype);
    if (batch > kMaxKeyColumns) return fail(err, RLQ_UNIMPLEMENTED, dtype, batch, kMaxKeyColumns);
    DeviceGuard g(ctx->device);
    const hipStream_t s = pick(ctx, stream);
    unsigned long long* ew = ctx->err_words;
    if (dtype == kQ8_K) HIP_TRY(launch_quantize_q8k(x, cols, batch, nullptr, out, ew, s));
    else if (dtype == kQ8_0) HIP_TRY(launch_quantize_q8_0(x, cols, batch, nullptr, out, ew, s));
    else {
        // the K encoders see the rows as one run of blocks (rows are whole blocks)
        HIP_TRY(launch_finite_scan(x, n, ew, s));
        HIP_TRY(launch_encode_k(dtype, x, n, out, ew, s));
    }
    return ok(err);
}

int32_t rlq_sync(rlq_context* ctx, void* stream, rlq_error* err) {
    if (!ctx) return fail(err, RLQ_INVALID_ARGUMENT);
    DeviceGuard g(ctx->device);
    const hipStream_t s = pick(ctx, stream);
    HIP_TRY(hipStreamSynchronize(s));
    return take_error(ctx, 0, s, 0, err);
}

// ---- dense Llama decode step ---------------------------------------------------

}  // extern "C"

struct rlq_llama {
    rlq_context* ctx;
    rlq::LlamaModel m;
};

namespace {

// LlamaConfig::validate (crates/model-runtime/src/llama.rs:19-56) in its
// order, then this library's limits.
int32_t check_llama_config(const rlq_llama_config& c, rlq_error* err) {
    for (uint64_t v : {c.vocabulary, c.width, c.feed_forward, c.heads, c.kv_heads, c.max_context})
        if (v == 0 || v > 0xffffffffull) return fail(err, RLQ_INVALID_CONFIG, 0, 1);  // lib.rs:197-206
    if (!(c.rms_epsilon > 0.0f) || !(c.rms_epsilon <= 3.402823466e38f))
        return fail(err, RLQ_INVALID_CONFIG, 0, 2);  // lib.rs:207-215
    if (c.width % c.heads != 0 || c.heads % c.kv_heads != 0) return fail(err, RLQ_INVALID_CONFIG, 0, 3);
    const uint64_t hd = c.width / c.heads, kvw = c.kv_heads * hd;
    if (hd % 2 != 0) return fail(err, RLQ_INVALID_CONFIG, 0, 4);
    if (!(c.rope_base > 0.0f) || !(c.rope_base <= 3.402823466e38f)) return fail(err, RLQ_INVALID_CONFIG, 0, 5);
    if (c.attention_scale != 0.0f && !(fabsf(c.attention_scale) <= 3.402823466e38f))
        return fail(err, RLQ_INVALID_CONFIG, 0, 6);
    uint64_t cache;
    if (__builtin_mul_overflow(kvw, c.max_context, &cache)) return fail(err, RLQ_INVALID_CONFIG, 0, 7);
    // the device error keys carry the layer in 16 bits
    if (c.n_layers > 0xffff) return fail(err, RLQ_UNIMPLEMENTED, 0, c.n_layers, 0xffff);
    for (uint32_t t : {c.weight_type, c.output_type, c.embedding_type}) {
        if (!dtype_known(t)) return fail(err, RLQ_INVALID_TYPE, t);
        if (!path_weight(t)) return fail(err, RLQ_UNIMPLEMENTED, t);
    }
    // whole K-quant blocks along every row; whole 16-row tiles for the fused
    // Q/K/V and gate/up matrices
    if (c.width % 256 != 0 || c.feed_forward % 256 != 0 || kvw % 16 != 0)
        return fail(err, RLQ_UNIMPLEMENTED, c.weight_type, c.width, c.feed_forward);
    if (hd % 16 != 0 || hd > 256) return fail(err, RLQ_UNIMPLEMENTED, 0, hd);  // dots in quarters of whole float4s
    // LDS of the attention workgroups (the G query heads of a KV head; it
    // does not grow with the context)
    if (llama_attn_lds_bytes(c.heads, c.kv_heads, hd) > 159 * 1024)
        return fail(err, RLQ_UNIMPLEMENTED, 0, c.heads / c.kv_heads, hd);
    return ok(err);
}

}  // namespace

extern "C" {

int32_t rlq_llama_create(rlq_context* ctx, const rlq_llama_config* cfg, const rlq_llama_tensors* t, rlq_llama** out,
                         rlq_error* err) {
    if (!ctx || !cfg || !t || !out) return fail(err, RLQ_INVALID_ARGUMENT);
    int32_t rc = check_llama_config(*cfg, err);
    if (rc) return rc;
    if (!t->embedding || !t->output_norm || !t->output || (cfg->n_layers && !t->layers))
        return fail(err, RLQ_INVALID_ARGUMENT);
    for (uint64_t l = 0; l < cfg->n_layers; ++l) {
        const rlq_llama_layer& L = t->layers[l];
        if (!L.attention_norm || !L.query || !L.key || !L.value || !L.attention_output || !L.feed_forward_norm ||
            !L.gate || !L.up || !L.down)
            return fail(err, RLQ_INVALID_ARGUMENT, 0, l);
        for (int k = 0; k < 7; ++k) {  // per-matrix types: on the path
            const uint32_t ty = L.types[k] ? L.types[k] : cfg->weight_type;
            if (!dtype_known(ty)) return fail(err, RLQ_INVALID_TYPE, ty, l, k);
            if (!path_weight(ty)) return fail(err, RLQ_UNIMPLEMENTED, ty, l, k);
        }
    }
    DeviceGuard g(ctx->device);
    rlq_llama* m = new (std::nothrow) rlq_llama;
    if (!m) return fail(err, RLQ_ALLOCATION_FAILED);
    m->ctx = ctx;
    m->m.device = ctx->device;
    std::vector<LlamaHostLayer> layers;
    try {
        layers.resize(cfg->n_layers);
    } catch (const std::exception&) {  // bad_alloc, length_error: no abort across the C ABI
        delete m;
        return fail(err, RLQ_ALLOCATION_FAILED);
    }
    for (uint64_t l = 0; l < cfg->n_layers; ++l) {
        const rlq_llama_layer& L = t->layers[l];
        layers[l] = LlamaHostLayer{L.attention_norm, L.query, L.key, L.value, L.attention_output,
                                   L.feed_forward_norm, L.gate, L.up, L.down, {}};
        for (int k = 0; k < 7; ++k) layers[l].types[k] = L.types[k] ? L.types[k] : cfg->weight_type;
    }
    const LlamaDims d{cfg->vocabulary, cfg->width, cfg->feed_forward, cfg->heads, cfg->kv_heads, cfg->max_context,
                      cfg->n_layers, cfg->rms_epsilon, cfg->rope_base, cfg->attention_scale, cfg->weight_type,
                      cfg->output_type, cfg->embedding_type};
    const LlamaHostTensors ht{t->embedding, t->output_norm, t->output, layers.data(), t->on_device != 0};
    hipError_t e = t->on_device ? hipDeviceSynchronize() : hipSuccess;  // device bytes may be in flight
    if (e == hipSuccess) e = m->m.create(d, ht, ctx->stream);
    if (e != hipSuccess) {
        delete m;
        return e == hipErrorOutOfMemory ? fail(err, RLQ_ALLOCATION_FAILED) : hip_fail(err, e);
    }
    *out = m;
    return ok(err);
}

// ---- LlamaModel from a GGUF file (crates/inference/src/loader.rs:242-410) ----------

namespace {

struct GgufReader {
    rlq_gguf* g = nullptr;
    ~GgufReader() { rlq_gguf_close(g); }
    int64_t find(const char* key) const { return rlq_gguf_find_kv(g, (const uint8_t*)key, strlen(key)); }
    uint32_t type(int64_t i) const {
        uint32_t t = 0;
        rlq_gguf_kv_at(g, (uint64_t)i, nullptr, nullptr, &t, nullptr, nullptr, nullptr);
        return t;
    }
    uint64_t bits(int64_t i) const {
        uint64_t b = 0;
        rlq_gguf_kv_scalar(g, (uint64_t)i, 0, &b, nullptr);
        return b;
    }
    std::string str(int64_t i) const {
        const uint8_t* p = nullptr;
        uint64_t n = 0;
        if (rlq_gguf_kv_string(g, (uint64_t)i, 0, &p, &n, nullptr) != RLQ_OK) return std::string();
        return std::string((const char*)p, n);
    }
};

// Loader check failures: a = the check number of rlq_llama_create_from_gguf.
constexpr int32_t kInvalid = RLQ_GGUF_INVALID, kUnsupported = RLQ_GGUF_UNSUPPORTED;

}  // namespace

int32_t rlq_llama_create_from_gguf(rlq_context* ctx, const char* path, uint64_t context_length, rlq_llama** out,
                                   rlq_error* err) {
    if (!ctx || !path || !out) return fail(err, RLQ_INVALID_ARGUMENT);
    if (context_length == 0) return fail(err, kInvalid, 0, 1);  // validate_options
    GgufReader r;
    int32_t rc = rlq_gguf_open(path, &r.g, err);
    if (rc) return rc;
    // loader.rs:12-30: hparams are exact UINT32 / finite FLOAT32 values
    auto uint = [&](const char* key, int64_t dflt, uint64_t check, uint64_t* v) -> int32_t {
        const int64_t i = r.find(key);
        if (i < 0) {
            if (dflt < 0) return fail(err, kInvalid, 0, check);
            *v = (uint64_t)dflt;
            return RLQ_OK;
        }
        if (r.type(i) != 4) return fail(err, kInvalid, 0, check);
        *v = r.bits(i);
        return RLQ_OK;
    };
    auto real = [&](const char* key, float dflt, uint64_t check, float* v) -> int32_t {
        const int64_t i = r.find(key);
        if (i < 0) {
            *v = dflt;
            return RLQ_OK;
        }
        if (r.type(i) != 6) return fail(err, kInvalid, 0, check);
        const uint32_t b = (uint32_t)r.bits(i);
        memcpy(v, &b, 4);
        if (!(fabsf(*v) <= 3.402823466e38f)) return fail(err, kInvalid, 0, check);
        return RLQ_OK;
    };
#define RLQ_TRY(x)                 \
    do {                           \
        const int32_t rc_ = (x);   \
        if (rc_) return rc_;       \
    } while (0)
    // architecture and shared metadata (loader.rs:75-89, 244-280)
    const int64_t ia = r.find("general.architecture");
    if (ia < 0 || r.type(ia) != 8) return fail(err, kInvalid, 0, 2);
    if (r.str(ia) != "llama") return fail(err, kUnsupported, 0, 2);
    const int64_t it = r.find("general.type");
    if (it >= 0 && r.type(it) != 8) return fail(err, kInvalid, 0, 3);
    if (it >= 0 && r.str(it) != "model") return fail(err, kUnsupported, 0, 3);
    uint64_t nextn = 0;
    RLQ_TRY(uint("llama.nextn_predict_layers", 0, 4, &nextn));
    if (nextn != 0) return fail(err, kUnsupported, 0, 4);
    if (r.find("prism.hadamard.version") >= 0) return fail(err, kUnsupported, 0, 5);
    // the vocabulary: the tokenizer's token list
    const int64_t itok = r.find("tokenizer.ggml.tokens");
    uint32_t tok_type = 0, tok_elem = 0;
    uint64_t vocab = 0;
    if (itok >= 0) rlq_gguf_kv_at(r.g, (uint64_t)itok, nullptr, nullptr, &tok_type, &tok_elem, &vocab, nullptr);
    if (itok < 0 || tok_type != 9 || tok_elem != 8 || vocab == 0) return fail(err, kInvalid, 0, 6);
    // hparams (loader.rs:282-331)
    uint64_t width, heads, kv_heads, layers, ff, train_context, v;
    RLQ_TRY(uint("llama.embedding_length", -1, 7, &width));
    RLQ_TRY(uint("llama.attention.head_count", -1, 8, &heads));
    if (width == 0 || heads == 0 || width % heads != 0) return fail(err, kInvalid, 0, 9);
    const uint64_t hd = width / heads;
    RLQ_TRY(uint("llama.attention.head_count_kv", (int64_t)heads, 10, &kv_heads));
    RLQ_TRY(uint("llama.block_count", -1, 11, &layers));
    if (layers == 0 || layers > 512) return fail(err, kInvalid, 0, 11);
    RLQ_TRY(uint("llama.feed_forward_length", -1, 12, &ff));
    RLQ_TRY(uint("llama.context_length", -1, 13, &train_context));
    RLQ_TRY(uint("llama.rope.dimension_count", (int64_t)hd, 14, &v));
    if (v != hd) return fail(err, kUnsupported, 0, 14);
    for (const char* key : {"llama.attention.key_length", "llama.attention.value_length"}) {
        RLQ_TRY(uint(key, (int64_t)hd, 15, &v));
        if (v != hd) return fail(err, kUnsupported, 0, 15);
    }
    for (const char* key : {"llama.attention.sliding_window", "llama.expert_count", "llama.expert_used_count"}) {
        RLQ_TRY(uint(key, 0, 16, &v));
        if (v != 0) return fail(err, kUnsupported, 0, 16);
    }
    const int64_t ic = r.find("llama.attention.causal");  // require_causal (loader.rs:31-45)
    if (ic >= 0 && r.type(ic) != 7) return fail(err, kInvalid, 0, 17);
    if (ic >= 0 && r.bits(ic) != 1) return fail(err, kUnsupported, 0, 17);
    // require_unscaled_rope (loader.rs:46-74)
    const int64_t is = r.find("llama.rope.scaling.type");
    if (is >= 0 && r.type(is) != 8) return fail(err, kInvalid, 0, 18);
    const std::string kind = is >= 0 ? r.str(is) : std::string("linear");
    if (kind != "none" && kind != "linear") return fail(err, kUnsupported, 0, 18);
    float factor = 0.0f, gain = 1.0f;
    RLQ_TRY(real(r.find("llama.rope.scaling.factor") >= 0 ? "llama.rope.scaling.factor" : "llama.rope.scale_linear",
                 0.0f, 19, &factor));
    if (kind != "none" && factor != 0.0f && factor != 1.0f) return fail(err, kUnsupported, 0, 19);
    RLQ_TRY(real("llama.rope.scaling.attn_factor", 1.0f, 20, &gain));
    if (gain != 1.0f) return fail(err, kUnsupported, 0, 20);
    for (const char* key : {"llama.attention.qk_norm", "llama.attention.qk_norm_rms"}) {
        const int64_t i = r.find(key);
        if (i >= 0 && !(r.type(i) == 7 && r.bits(i) == 0)) return fail(err, kUnsupported, 0, 21);
    }
    float eps, rope_base, scale;
    RLQ_TRY(real("llama.attention.layer_norm_rms_epsilon", 1e-5f, 22, &eps));
    RLQ_TRY(real("llama.rope.freq_base", 10000.0f, 23, &rope_base));
    RLQ_TRY(real("llama.attention.scale", 0.0f, 24, &scale));
    const uint64_t kvw = kv_heads * hd;  // kv_heads == 0 and heads % kv_heads: check_llama_config
    // tensors (loader.rs:96-160, 338-409): GGML shapes, trailing axes of one
    uint64_t n_tensors = 0;
    rlq_gguf_header(r.g, nullptr, nullptr, nullptr, nullptr, &n_tensors, nullptr);
    std::vector<uint8_t> used(n_tensors, 0);
    struct Got {
        int64_t i;
        uint32_t dtype;
        uint64_t bytes;
    };
    auto tensor = [&](const std::string& name, uint64_t d0, uint64_t d1, bool optional, bool vector, uint64_t check,
                      Got* got) -> int32_t {
        got->i = rlq_gguf_find_tensor(r.g, (const uint8_t*)name.data(), name.size());
        if (got->i < 0) return optional ? RLQ_OK : fail(err, kInvalid, 0, check);
        uint32_t nd;
        uint64_t dims[4], off;
        rlq_gguf_tensor_at(r.g, (uint64_t)got->i, nullptr, nullptr, &nd, dims, &got->dtype, &off, &got->bytes, nullptr);
        const uint64_t want[4] = {d0, vector ? 1 : d1, 1, 1};
        for (int k = 0; k < 4; ++k)
            if (dims[k] != want[k]) return fail(err, kInvalid, 0, check);
        if (vector ? got->dtype != 0 : !path_weight(got->dtype)) return fail(err, RLQ_UNIMPLEMENTED, got->dtype, check);
        used[(size_t)got->i] = 1;
        return RLQ_OK;
    };
    Got emb, onorm, outw;
    RLQ_TRY(tensor("token_embd.weight", width, vocab, false, false, 30, &emb));
    RLQ_TRY(tensor("output_norm.weight", width, 0, false, true, 31, &onorm));
    RLQ_TRY(tensor("output.weight", width, vocab, true, false, 32, &outw));
    static const char* const kNames[7] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                                          "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
    std::vector<Got> mats(layers * 7), norms(layers * 2);
    for (uint64_t l = 0; l < layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        const uint64_t shapes[7][2] = {{width, width}, {width, kvw}, {width, kvw}, {width, width},
                                       {width, ff},    {width, ff},  {ff, width}};
        for (int k = 0; k < 7; ++k)
            RLQ_TRY(tensor(b + kNames[k], shapes[k][0], shapes[k][1], false, false, 40 + k, &mats[l * 7 + k]));
        RLQ_TRY(tensor(b + "attn_norm.weight", width, 0, false, true, 47, &norms[l * 2]));
        RLQ_TRY(tensor(b + "ffn_norm.weight", width, 0, false, true, 48, &norms[l * 2 + 1]));
        // biases: the reference adds them (loader.rs:364-388); this step has none
        for (const char* bias : {"attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias", "ffn_gate.bias",
                                 "ffn_up.bias", "ffn_down.bias"}) {
            const std::string nm = b + bias;
            if (rlq_gguf_find_tensor(r.g, (const uint8_t*)nm.data(), nm.size()) >= 0)
                return fail(err, RLQ_UNIMPLEMENTED, 0, 49);
        }
    }
    std::vector<uint8_t> host;  // every payload this model reads
    std::vector<uint64_t> at(n_tensors, 0);
    uint64_t total = 0;
    for (uint64_t i = 0; i < n_tensors; ++i)
        if (used[i]) {
            uint64_t nb;
            rlq_gguf_tensor_at(r.g, i, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &nb, nullptr);
            at[i] = total;
            total += (nb + 255) & ~255ull;
        }
    const int64_t irf = rlq_gguf_find_tensor(r.g, (const uint8_t*)"rope_freqs.weight", 17);
    if (irf >= 0) {  // loader.rs:395-402: all-one frequency factors only
        uint32_t nd, dt;
        uint64_t dims[4], off, nb;
        rlq_gguf_tensor_at(r.g, (uint64_t)irf, nullptr, nullptr, &nd, dims, &dt, &off, &nb, nullptr);
        if (dt != 0) return fail(err, RLQ_UNIMPLEMENTED, dt, 50);
        std::vector<float> f(nb / 4);
        rc = rlq_gguf_read_tensor(r.g, (uint64_t)irf, f.data(), nb, err);
        if (rc) return rc;
        if (dims[0] * dims[1] * dims[2] * dims[3] != hd / 2) return fail(err, kUnsupported, 0, 50);
        for (float x : f)
            if (x != 1.0f) return fail(err, kUnsupported, 0, 50);
        used[(size_t)irf] = 1;
    }
    for (uint64_t i = 0; i < n_tensors; ++i)
        if (!used[i]) return fail(err, kUnsupported, 0, 51, i);  // unimplemented tensors
    try {
        host.resize(total);
    } catch (const std::bad_alloc&) {
        return fail(err, RLQ_ALLOCATION_FAILED);
    }
    for (uint64_t i = 0; i < n_tensors; ++i)
        if (used[i] && (int64_t)i != irf) {
            uint64_t nb;
            rlq_gguf_tensor_at(r.g, i, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &nb, nullptr);
            rc = rlq_gguf_read_tensor(r.g, i, host.data() + at[i], nb, err);
            if (rc) return rc;
        }
    auto ptr = [&](const Got& g) -> const void* { return host.data() + at[(size_t)g.i]; };
    std::vector<rlq_llama_layer> ls(layers);
    for (uint64_t l = 0; l < layers; ++l) {
        const Got* m = &mats[l * 7];
        ls[l] = rlq_llama_layer{(const float*)ptr(norms[l * 2]), ptr(m[0]), ptr(m[1]), ptr(m[2]), ptr(m[3]),
                                (const float*)ptr(norms[l * 2 + 1]), ptr(m[4]), ptr(m[5]), ptr(m[6]), {}};
        for (int k = 0; k < 7; ++k) ls[l].types[k] = m[k].dtype;
    }
    const bool tied = outw.i < 0;  // no output.weight: the embedding matrix projects (loader.rs:345-355)
    rlq_llama_config cfg{vocab,
                         width,
                         ff,
                         heads,
                         kv_heads,
                         train_context < context_length ? train_context : context_length,
                         layers,
                         eps,
                         rope_base,
                         scale,
                         mats[0].dtype,
                         tied ? emb.dtype : outw.dtype,
                         emb.dtype};
    rlq_llama_tensors tensors{ptr(emb), (const float*)ptr(onorm), tied ? ptr(emb) : ptr(outw), ls.data(), 0};
#undef RLQ_TRY
    return rlq_llama_create(ctx, &cfg, &tensors, out, err);
}

void rlq_llama_config_of(const rlq_llama* m, rlq_llama_config* out) {
    if (!m || !out) return;
    const LlamaDims& d = m->m.d;
    *out = rlq_llama_config{d.vocab,        d.width,     d.feed_forward,    d.heads,       d.kv_heads,
                            d.max_context,  d.n_layers,  d.rms_epsilon,     d.rope_base,   d.attention_scale,
                            d.weight_type,  d.output_type, d.embedding_type};
}

void rlq_llama_destroy(rlq_llama* m) {
    if (!m) return;
    DeviceGuard g(m->m.device);
    delete m;
}

int32_t rlq_llama_truncate(rlq_llama* m, uint64_t rows, rlq_error* err) {
    if (!m) return fail(err, RLQ_INVALID_ARGUMENT);
    if (rows < m->m.n_cached) m->m.n_cached = rows;
    return ok(err);
}

uint64_t rlq_llama_cached(const rlq_llama* m) { return m ? m->m.n_cached : 0; }

int32_t rlq_llama_embedding(rlq_llama* m, uint32_t token, float* hidden, void* stream, rlq_error* err) {
    if (!m || !hidden) return fail(err, RLQ_INVALID_ARGUMENT);
    if (token >= m->m.d.vocab) return fail(err, RLQ_INVALID_TOKEN, 0, token, m->m.d.vocab);  // llama.rs:214-219
    DeviceGuard g(m->m.device);
    HIP_TRY(m->m.embedding(token, hidden, (hipStream_t)stream));
    return ok(err);
}

int32_t rlq_llama_step(rlq_llama* m, float* hidden, uint64_t position, float* embedding, float* logits,
                       uint32_t* argmax, void* stream, rlq_error* err) {
    if (!m || !hidden) return fail(err, RLQ_INVALID_ARGUMENT);
    if (m->m.n_cached >= m->m.d.max_context) return fail(err, RLQ_INVALID_STATE, 0, m->m.n_cached, m->m.d.max_context);
    if (position >= m->m.d.max_context) return fail(err, RLQ_INVALID_STATE, 0, position, m->m.d.max_context);
    DeviceGuard g(m->m.device);
    HIP_TRY(m->m.step(hidden, position, embedding, logits, argmax, m->ctx->err_words, (hipStream_t)stream));
    return ok(err);
}

int32_t rlq_llama_intermediates(const rlq_llama* m, float* qkv, float* attention, float* ffn_input, float* ffn,
                                void* stream, rlq_error* err) {
    if (!m) return fail(err, RLQ_INVALID_ARGUMENT);
    DeviceGuard g(m->m.device);
    const LlamaDims& d = m->m.d;
    const uint64_t kvw = d.kv_heads * (d.width / d.heads);
    const hipStream_t s = (hipStream_t)stream;
    if (qkv) HIP_TRY(hipMemcpyAsync(qkv, m->m.qkv, (d.width + 2 * kvw) * 4, hipMemcpyDeviceToDevice, s));
    if (attention) HIP_TRY(hipMemcpyAsync(attention, m->m.att, d.width * 4, hipMemcpyDeviceToDevice, s));
    if (ffn_input) HIP_TRY(hipMemcpyAsync(ffn_input, m->m.mid, d.width * 4, hipMemcpyDeviceToDevice, s));
    if (ffn) HIP_TRY(m->m.ffn_activation(ffn, s));
    return ok(err);
}

int32_t rlq_llama_trace(rlq_llama* m, float* layer_outputs, rlq_error* err) {
    if (!m) return fail(err, RLQ_INVALID_ARGUMENT);
    m->m.trace = layer_outputs;
    return ok(err);
}

int32_t rlq_block_sums_ex(rlq_context* ctx, const rlq_weights* w, const float* x, uint64_t batch, uint32_t flags,
                          int32_t* isum, int32_t* imin, float* y, void* stream, rlq_error* err) {
    if (!ctx || !w || !x || !isum || !imin) return fail(err, RLQ_INVALID_ARGUMENT);
    if (((uintptr_t)x & 15) || ((uintptr_t)y & 3)) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    if (batch == 0 || (flags & ~RLQ_SUMS_SILU_PAIR)) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
    const bool pair = (flags & RLQ_SUMS_SILU_PAIR) != 0;
    // the SiLU-pair epilogue: one column of Q4_K / Q5_K rows in whole gate/up tile pairs
    if (pair && (batch != 1 || (w->dtype != kQ4_K && w->dtype != kQ5_K) || w->rows % (2 * kTileRows) != 0))
        return fail(err, RLQ_INVALID_ARGUMENT, w->dtype, batch, w->rows);
    DeviceGuard g(ctx->device);
    const hipStream_t s = pick(ctx, stream);
    if (!y) {
        HIP_TRY(ensure(ctx, ctx->stage_out, batch * w->rows * sizeof(float)));
        y = (float*)ctx->stage_out.p;
    }
    if (w->dtype == kQ4_K && batch > kDecodeMaxBatch) {
        HIP_TRY(ensure(ctx, ctx->planes, gemm_planes_bytes(batch, w->cols)));
        HIP_TRY(launch_gemm_q4k(w->dev, w->rows, w->cols, x, batch, y, w->rows, ctx->planes.p, ctx->err_words, isum,
                                imin, s));
    } else {
        if (batch > kDecodeMaxBatch) return fail(err, RLQ_INVALID_ARGUMENT, w->dtype);
        MvExtra ex;
        ex.epilogue = pair ? 1u : 0u;
        HIP_TRY(decode_launch(ctx, w, x, batch, y, nullptr, isum, imin, ex, s));
    }
    return ok(err);
}

int32_t rlq_block_sums(rlq_context* ctx, const rlq_weights* w, const float* x, uint64_t batch, int32_t* isum,
                       int32_t* imin, void* stream, rlq_error* err) {
    return rlq_block_sums_ex(ctx, w, x, batch, 0, isum, imin, nullptr, stream, err);
}

// ---- host drop-ins ----------------------------------------------------------------

// quantize_into (crates/quant/src/encode.rs:37-100; encode_k.rs:11-33)
int32_t rlq_quantize_into(uint32_t dtype, const float* values, uint64_t n, uint8_t* out, uint64_t out_len,
                          rlq_error* err) {
    int32_t rc = validate(dtype, out_len, n, err);
    if (rc) return rc;
    // supported() (encode.rs:102-113)
    if (dtype == 16 || dtype == 17 || dtype == 19) return fail(err, RLQ_IMPORTANCE_WEIGHTS_REQUIRED, dtype);
    if (dtype == 24 || dtype == 25 || dtype == 26 || dtype == 27) return fail(err, RLQ_UNSUPPORTED_QUANTIZATION, dtype);
    if (dtype != kQ8_K && !path_weight(dtype)) return fail(err, RLQ_UNIMPLEMENTED, dtype);
    if (n == 0) return ok(err);
    if (!values || !out) return fail(err, RLQ_INVALID_ARGUMENT, dtype);
    std::lock_guard<std::mutex> lock(g_default_mu);
    rlq_context* ctx;
    rc = default_context(&ctx, err);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    const hipStream_t s = ctx->stream;
    HIP_TRY(ensure(ctx, ctx->stage_in, n * sizeof(float)));
    HIP_TRY(ensure(ctx, ctx->stage_out, out_len));
    float* xd = (float*)ctx->stage_in.p;
    uint8_t* od = (uint8_t*)ctx->stage_out.p;
    unsigned long long* ew = ctx->err_words + 1;
    HIP_TRY(hipMemcpyAsync(xd, values, n * sizeof(float), hipMemcpyHostToDevice, s));
    if (dtype == kQ8_K) HIP_TRY(launch_quantize_q8k(xd, n, 1, nullptr, od, ew, s));
    else if (dtype == kQ8_0) HIP_TRY(launch_quantize_q8_0(xd, n, 1, nullptr, od, ew, s));
    else {
        HIP_TRY(launch_finite_scan(xd, n, ew, s));
        HIP_TRY(launch_encode_k(dtype, xd, n, od, ew, s));
    }
    rc = take_error(ctx, 1, s, dtype, err);
    if (rc) {
        if (err) err->b = 0;
        return rc;
    }
    HIP_TRY(hipMemcpyAsync(out, od, out_len, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return ok(err);
}

// dequantize_into (crates/quant/src/lib.rs:299-308)
int32_t rlq_dequantize_into(uint32_t dtype, const uint8_t* bytes, uint64_t len, float* out, uint64_t n,
                            rlq_error* err) {
    int32_t rc = validate(dtype, len, n, err);
    if (rc) return rc;
    if (dtype != kQ8_K && !path_weight(dtype)) return fail(err, RLQ_UNIMPLEMENTED, dtype);
    if (n == 0) return ok(err);
    if (!bytes || !out) return fail(err, RLQ_INVALID_ARGUMENT, dtype);
    std::lock_guard<std::mutex> lock(g_default_mu);
    rlq_context* ctx;
    rc = default_context(&ctx, err);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    const hipStream_t s = ctx->stream;
    HIP_TRY(ensure(ctx, ctx->stage_w, len));
    HIP_TRY(ensure(ctx, ctx->stage_out, n * sizeof(float)));
    HIP_TRY(hipMemcpyAsync(ctx->stage_w.p, bytes, len, hipMemcpyHostToDevice, s));
    HIP_TRY(launch_dequantize(dtype, (const uint8_t*)ctx->stage_w.p, n, (float*)ctx->stage_out.p, s));
    HIP_TRY(hipMemcpyAsync(out, ctx->stage_out.p, n * sizeof(float), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return ok(err);
}

// dot_packed (crates/quant/src/matvec.rs:90-103)
int32_t rlq_dot_packed(uint32_t wtype, const uint8_t* weights, uint64_t weights_len, const uint8_t* activation,
                       uint64_t activation_len, uint64_t elements, float* out, rlq_error* err) {
    uint32_t at;
    int32_t rc = activation_dtype(wtype, &at, err);
    if (rc) return rc;
    if (block_size(wtype) == 1) return fail(err, RLQ_UNSUPPORTED_MATVEC, wtype);
    if (!path_weight(wtype)) return fail(err, RLQ_UNIMPLEMENTED, wtype);
    rc = validate(wtype, weights_len, elements, err);
    if (rc) return rc;
    rc = validate(at, activation_len, elements, err);
    if (rc) return rc;
    if (!out) return fail(err, RLQ_INVALID_ARGUMENT, wtype);
    if (elements == 0) {  // no blocks: the reference's sums stay 0.0
        *out = 0.0f;
        return ok(err);
    }
    if (!weights || !activation) return fail(err, RLQ_INVALID_ARGUMENT, wtype);
    std::lock_guard<std::mutex> lock(g_default_mu);
    rlq_context* ctx;
    rc = default_context(&ctx, err);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    const hipStream_t s = ctx->stream;
    uint8_t* wd = nullptr;
    hipError_t e = upload_weights(wtype, weights, weights_len, 1, elements, false, &wd, s);
    if (e != hipSuccess) return hip_fail(err, e);
    e = ensure(ctx, ctx->stage_in, activation_len);
    if (e == hipSuccess) e = ensure(ctx, ctx->planes, act_planes_bytes(at, elements, 1));
    if (e == hipSuccess) e = ensure(ctx, ctx->stage_out, sizeof(float));
    ActPlanes planes{};
    if (e == hipSuccess) {
        planes = act_planes_carve(ctx->planes.p, at, elements, 1);
        e = hipMemcpyAsync(ctx->stage_in.p, activation, activation_len, hipMemcpyHostToDevice, s);
    }
    if (e == hipSuccess) e = launch_act_from_gguf(at, (const uint8_t*)ctx->stage_in.p, elements, 1, &planes, s);
    if (e == hipSuccess)
        e = launch_matvec(wtype, wd, 1, elements, nullptr, &planes, 1, (float*)ctx->stage_out.p, 1, nullptr,
                          ctx->err_words + 1, nullptr, nullptr, s);
    if (e == hipSuccess) e = hipMemcpyAsync(out, ctx->stage_out.p, sizeof(float), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(wd);
    return e == hipSuccess ? ok(err) : hip_fail(err, e);
}

// matvec (crates/quant/src/matvec.rs:24-87)
int32_t rlq_matvec(uint32_t wtype, const uint8_t* weights, uint64_t weights_len, uint64_t rows, uint64_t cols,
                   const float* input, uint64_t input_len, float* output, rlq_error* err) {
    uint32_t at;
    int32_t rc = activation_dtype(wtype, &at, err);
    if (rc) return rc;
    if (!path_weight(wtype)) return fail(err, RLQ_UNIMPLEMENTED, wtype);
    if (rows == 0 || cols == 0) return fail(err, RLQ_INVALID_MATRIX_SHAPE, wtype, rows, cols);
    if (input_len != cols) return fail(err, RLQ_INVALID_VECTOR_LENGTH, wtype, cols, input_len);
    uint64_t rb, expected;
    rc = row_bytes(wtype, cols, &rb, err);
    if (rc) return rc;
    if (__builtin_mul_overflow(rb, rows, &expected)) return fail(err, RLQ_SIZE_OVERFLOW, wtype);
    if (weights_len != expected) return fail(err, RLQ_INVALID_LENGTH, wtype, expected, weights_len);
    if (!weights || !input || !output) return fail(err, RLQ_INVALID_ARGUMENT, wtype);
    std::lock_guard<std::mutex> lock(g_default_mu);
    rlq_context* ctx;
    rc = default_context(&ctx, err);
    if (rc) return rc;
    DeviceGuard g(ctx->device);
    const hipStream_t s = ctx->stream;
    uint8_t* wd = nullptr;
    hipError_t e = upload_weights(wtype, weights, weights_len, rows, cols, false, &wd, s);
    if (e != hipSuccess) return e == hipErrorOutOfMemory ? fail(err, RLQ_ALLOCATION_FAILED, wtype) : hip_fail(err, e);
    e = ensure(ctx, ctx->stage_in, cols * sizeof(float));
    if (e == hipSuccess) e = ensure(ctx, ctx->stage_out, rows * sizeof(float));
    if (e == hipSuccess) e = hipMemcpyAsync(ctx->stage_in.p, input, cols * sizeof(float), hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = launch_matvec(wtype, wd, rows, cols, (const float*)ctx->stage_in.p, nullptr, 1, (float*)ctx->stage_out.p,
                          rows, nullptr, ctx->err_words + 1, nullptr, nullptr, s);
    if (e != hipSuccess) {
        (void)hipFree(wd);
        return hip_fail(err, e);
    }
    rc = take_error(ctx, 1, s, at, err);
    (void)hipFree(wd);
    if (rc) {
        if (err) err->b = 0;
        return rc;
    }
    HIP_TRY(hipMemcpyAsync(output, ctx->stage_out.p, rows * sizeof(float), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return ok(err);
}

}  // extern "C"
