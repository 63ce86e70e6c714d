"""GGUF reader and writer: the library's C++ code (rlq_gguf_*, host only) and
the oracle's restatement (oracle/gguf.py), both against the reference's
frozen reader corpus (tests/golden/gguf-*-reference.tsv, copied from
fixtures/gguf-bytes: the original C getters' observations of 1093 + 512
headers, crates/gguf/tests/raw_native.rs:54-300) and a real vocabulary-only
Llama file.  Per case: admission, version, alignment, data offset, every
metadata getter (type, C-string key, first native lookup, scalar bits,
strings, arrays), every tensor descriptor, the exact gguf_get_meta_data
bytes, and for v3 files without booleans the raw writer reproducing the
input header byte for byte.  Byte work: every comparison is exact.
"""
import os

import numpy as np
import pytest

from oracle import gguf as G
from rlq_loader import load

rlq = load()
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _scalar_bytes(ty, bits):
    return int(bits).to_bytes(G._SCALAR[ty], "little")


class OracleView:
    def __init__(self, data):
        self.h = G.read_header(data)
        self.version, self.alignment, self.data_offset = self.h.version, self.h.alignment, self.h.data_offset

    def kvs(self):
        return [(k, v.type, v.data if v.type == 8 else (v.elem, v.items) if v.type == 9 else v.bits)
                for k, v in zip(self.h.keys, self.h.values)]

    def tensors(self):
        return [(t.name, t.dims, t.dtype, t.offset, t.nbytes) for t in self.h.tensors]

    def find_kv(self, key):
        return self.h.find_kv(key)

    def find_tensor(self, name):
        return self.h.find_tensor(name)

    def native_header(self):
        return G.native_header(self.h)

    def raw_header(self):
        return G.write_header(self.h.keys, self.h.values, self.h.tensors)


class LibraryView:
    def __init__(self, data):
        self.g = rlq.GgufFile.from_bytes(data)
        self.version, self.alignment, self.data_offset = self.g.version, self.g.alignment, self.g.data_offset

    def kvs(self):
        return [self.g.kv(i) for i in range(self.g.n_kv)]

    def tensors(self):
        return [self.g.tensor(i) for i in range(self.g.n_tensors)]

    def find_kv(self, key):
        return self.g.find_kv(key)

    def find_tensor(self, name):
        return self.g.find_tensor(name)

    def native_header(self):
        return self.g.native_header()

    def raw_header(self):
        kvs = self.kvs()
        tensors = [(n, d, t, None) for n, d, t, _, _ in self.tensors()]
        return rlq.gguf_header(kvs, tensors)


def admit(view_cls, data):
    try:
        return view_cls(data)
    except (G.GgufError, rlq.QuantError):
        return None


def run_corpus(view_cls, tsv, blob, want_cases, want_admitted, want_raw):
    rows = [r for r in open(os.path.join(HERE, tsv)).read().splitlines() if not r.startswith("#")]
    data = open(os.path.join(HERE, blob), "rb").read()
    cases = admitted = raw = 0
    cur, kvs, ts, ms, tn, name = None, None, None, 0, 0, ""
    for row in rows:
        c = row.split("\t")
        if c[0] == "C":
            name, start, n = c[1], int(c[3]), int(c[4])
            cases += 1
            ms = tn = 0
            cur = admit(view_cls, data[start:start + n])
            assert (cur is not None) == (c[2] == "1"), f"{name}: admission"
            if cur is None:
                continue
            admitted += 1
            assert (cur.version, cur.alignment, cur.data_offset) == (int(c[7]), int(c[8]), int(c[9])), name
            off, nb = int(c[5]), int(c[6])
            assert cur.native_header() == data[off:off + nb], f"{name}: gguf_get_meta_data bytes"
            kvs, ts = cur.kvs(), cur.tensors()
            has_bool = any(t == 7 or (t == 9 and v[0] == 7) for _, t, v in kvs)
            if cur.version == 3 and not has_bool:
                wire, file_bytes = cur.raw_header()
                assert wire == data[start:start + len(wire)] and file_bytes == n, f"{name}: raw writer"
                raw += 1
        elif c[0] == "M":
            i = int(c[1])
            assert i == ms
            ms += 1
            key, ty, val = kvs[i]
            assert G.c_string(key) == bytes.fromhex(c[2]) and ty == int(c[3]), f"{name}: key {i}"
            assert cur.find_kv(bytes.fromhex(c[2])) == int(c[4]), f"{name}: lookup {i}"
            if c[5] == "n":
                assert _scalar_bytes(ty, val) == bytes.fromhex(c[6]), f"{name}: scalar {i}"
            elif c[5] == "s":
                assert G.c_string(val) == bytes.fromhex(c[6]), f"{name}: string {i}"
            else:
                el, items = val
                assert (el, len(items)) == (int(c[6]), int(c[7])), f"{name}: array {i}"
                if el == 8:
                    want = [bytes.fromhex(x) for x in c[8].split(",")] if items else []
                    assert [G.c_string(x) for x in items] == want, f"{name}: string array {i}"
                else:
                    assert b"".join(_scalar_bytes(el, x) for x in items) == bytes.fromhex(c[8]), f"{name}: array {i}"
        elif c[0] == "T":
            i = int(c[1])
            assert i == tn
            tn += 1
            tname, dims, dtype, offset, nbytes = ts[i]
            assert G.c_string(tname) == bytes.fromhex(c[2]), f"{name}: tensor name {i}"
            assert cur.find_tensor(bytes.fromhex(c[2])) == int(c[3]), f"{name}: tensor lookup {i}"
            assert (list(dims) + [1, 1, 1, 1])[:4] == [int(x) for x in c[4].split(",")], f"{name}: dims {i}"
            assert (dtype, offset, nbytes) == (int(c[5]), int(c[6]), int(c[7])), f"{name}: tensor {i}"
        elif c[0] == "E":
            if cur is not None:
                assert (len(kvs), len(ts)) == (ms, tn), f"{name}: every getter observed"
            cur = None
    assert (cases, admitted, raw) == (want_cases, want_admitted, want_raw)


@pytest.mark.parametrize("view", [OracleView, LibraryView], ids=["oracle", "library"])
def test_reader_corpus(view):
    run_corpus(view, "gguf-reader-reference.tsv", "gguf-reader-data.bin", 1093, 1080, 1073)


@pytest.mark.parametrize("view", [OracleView, LibraryView], ids=["oracle", "library"])
def test_boolean_corpus(view):
    run_corpus(view, "gguf-booleans-reference.tsv", "gguf-booleans-data.bin", 512, 512, 0)


def test_planted_reader_mistakes_fail():
    """An alignment that ignores general.alignment, or an offset check that
    accepts gaps, disagrees with the corpus."""
    data = open(os.path.join(HERE, "gguf-reader-data.bin"), "rb").read()
    rows = [r.split("\t") for r in open(os.path.join(HERE, "gguf-reader-reference.tsv")).read().splitlines()
            if r.startswith("C\t")]
    aligned = [r for r in rows if r[2] == "1" and int(r[8]) != 32]
    rejected = [r for r in rows if r[2] == "0"]
    assert aligned and rejected
    assert all(G.read_header(data[int(r[3]):int(r[3]) + int(r[4])]).alignment != 32 for r in aligned)
    for r in rejected:
        with pytest.raises(G.GgufError):
            G.read_header(data[int(r[3]):int(r[3]) + int(r[4])])


def test_real_vocab_file():
    path = os.path.join(HERE, "ggml-vocab-llama-spm.gguf")
    raw = open(path, "rb").read()
    g = rlq.GgufFile.open(path)
    o = OracleView(raw)
    assert (g.version, g.alignment, g.data_offset) == (o.version, o.alignment, o.data_offset) == (3, 32, len(raw))
    assert [g.kv(i) for i in range(g.n_kv)] == o.kvs()
    # written by the original converter, which ends a file without tensors at
    # the encoded header (writer.rs:55-57); gguf_get_meta_data pads it to the
    # alignment
    nh = g.native_header()
    assert nh == o.native_header() and nh[:len(raw)] == raw
    assert len(nh) == (len(raw) + 31) // 32 * 32 and nh[len(raw):] == bytes(len(nh) - len(raw))
    k, t, (el, tokens) = g.kv(g.find_kv(b"tokenizer.ggml.tokens"))
    assert (t, el, len(tokens)) == (9, 8, 32000)
    assert g.kv(g.find_kv(b"llama.embedding_length"))[2] == 4096


def test_write_read_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    kvs = [(b"general.architecture", 8, b"llama"), (b"a.u8", 0, 200), (b"a.i16", 3, 0xfffe),
           (b"a.f32", 6, int(np.float32(1.5).view(np.uint32))), (b"a.bool", 7, 1), (b"a.u64", 10, 1 << 40),
           (b"a.f64", 12, int(np.float64(-2.25).view(np.uint64))), (b"a.strs", 9, (8, [b"x", b"", b"\x00y"])),
           (b"a.i32s", 9, (5, [1, 0xffffffff, 7])), (b"general.alignment", 4, 64)]
    w1 = rng.integers(0, 256, 3 * 144, dtype=np.uint8)
    w2 = rng.standard_normal(10).astype(np.float32).view(np.uint8)
    tensors = [(b"blk.0.w", [256, 3], 12, w1), (b"v", [10], 0, w2)]
    path = str(tmp_path / "t.gguf")
    rlq.gguf_write(path, kvs, tensors)
    raw = open(path, "rb").read()
    g = rlq.GgufFile.open(path)
    assert (g.version, g.alignment) == (3, 64)
    assert [g.kv(i) for i in range(g.n_kv)] == kvs
    assert g.tensor(0)[:4] == (b"blk.0.w", [256, 3], 12, 0) and g.tensor(1)[3] == 448
    assert np.array_equal(g.read_tensor(0), w1) and np.array_equal(g.read_tensor(1), w2)
    assert len(raw) == g.data_offset + 448 + 64 and raw[g.data_offset + 432:g.data_offset + 448] == bytes(16)
    o = OracleView(raw)
    assert o.kvs() == kvs and o.native_header() == g.native_header()
    header, file_bytes = rlq.gguf_header(kvs, [(n, d, t, None) for n, d, t, _ in tensors])
    assert header == raw[:g.data_offset] and file_bytes == len(raw)


def test_writer_rejects_before_writing(tmp_path):
    path = str(tmp_path / "bad.gguf")
    cases = [
        ([(b"k", 8, b"v"), (b"k", 8, b"w")], []),                  # duplicate key
        ([(b"general.alignment", 4, 48)], []),                     # not a power of two
        ([(b"general.alignment", 5, 32)], []),                     # not UINT32
        ([], [(b"t", [100], 12, np.zeros(0, np.uint8))]),          # not whole Q4_K blocks
        ([], [(b"x" * 64, [4], 0, np.zeros(16, np.uint8))]),       # name of 64 bytes
    ]
    for kvs, tensors in cases:
        with pytest.raises(rlq.QuantError) as e:
            rlq.gguf_write(path, kvs, tensors)
        assert e.value.name == "GgufInvalid"
        assert not os.path.exists(path)


def test_reader_errors(tmp_path):
    """Every truncation of a file (header, padding or payload) is refused by
    the payload-checking open (crates/gguf/src/lib.rs:689-699 tests the same)."""
    path = str(tmp_path / "g.gguf")
    rlq.gguf_write(path, [(b"k", 4, 1)], [(b"t", [8], 0, np.arange(8, dtype=np.float32).view(np.uint8))])
    good = open(path, "rb").read()
    g = rlq.GgufFile.open(path)
    assert len(good) == g.data_offset + 32
    for n in range(len(good)):
        cut = str(tmp_path / f"c{n}.gguf")
        with open(cut, "wb") as f:
            f.write(good[:n])
        with pytest.raises(rlq.QuantError):
            rlq.GgufFile.open(cut)
    with pytest.raises(rlq.QuantError) as e:
        rlq.GgufFile.from_bytes(b"GGUF" + (4).to_bytes(4, "little") + bytes(16))
    assert e.value.name == "GgufUnsupported"
    with pytest.raises(rlq.QuantError) as e:
        rlq.GgufFile.from_bytes(b"GGUX" + good[4:])
    assert e.value.name == "GgufInvalid"
