"""Readers for the golden records in this directory.

The files keep the record layouts of the reference's fixtures
(crates/quant/tests/fixtures/*.bin, read by crates/quant/tests/{matvec,
matvec_extended,reference,encoders_extended}.rs); extract_reference_fixtures.py
copied the Q8_0 / Q4_K / Q6_K / Q8_K records.
"""
import os
import struct
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


class _Reader:
    def __init__(self, name, magic):
        self.data = open(os.path.join(HERE, name), "rb").read()
        self.pos = 0
        got = self.take(8)
        assert got == magic, (name, got)
        self.count = self.word()

    def take(self, n):
        out = self.data[self.pos:self.pos + n]
        assert len(out) == n
        self.pos += n
        return out

    def word(self):
        return struct.unpack("<I", self.take(4))[0]

    def floats(self, n):
        return np.frombuffer(self.take(4 * n), dtype="<f4").astype(np.float32)

    def bytes_(self, n):
        return np.frombuffer(self.take(n), dtype=np.uint8).copy()

    def done(self):
        assert self.pos == len(self.data)


@dataclass
class MatvecRecord:
    dtype: int
    rows: int
    cols: int
    weights: np.ndarray
    x: np.ndarray
    activation: np.ndarray  # packed activation bytes (None for GGQM records)
    generic: np.ndarray     # original generic C output
    native: np.ndarray      # original GGML graph output


def matvec_extended(name="matvec-extended-q4k-q6k.bin"):
    """GGQX: 24 Q4_K + 24 Q6_K records (matvec_extended.rs:50-103), or with
    name="matvec-extended-q2k-q3k-q5k.bin" 24 each of Q2_K, Q3_K, Q5_K."""
    r = _Reader(name, b"GGQX0001")
    out = []
    for _ in range(r.count):
        dtype, rows, cols, wsize, asize = (r.word() for _ in range(5))
        w = r.bytes_(wsize)
        x = r.floats(cols)
        act = r.bytes_(asize)
        out.append(MatvecRecord(dtype, rows, cols, w, x, act, r.floats(rows), r.floats(rows)))
    r.done()
    return out


def matvec_q8_0():
    """GGQM: 18 Q8_0 records (matvec.rs:26-63)."""
    r = _Reader("matvec-q8_0.bin", b"GGQM0001")
    out = []
    for _ in range(r.count):
        dtype, rows, cols, size = (r.word() for _ in range(4))
        w = r.bytes_(size)
        x = r.floats(cols)
        out.append(MatvecRecord(dtype, rows, cols, w, x, None, r.floats(rows), r.floats(rows)))
    r.done()
    return out


def q8k():
    """GGQ8: 30 Q8_K encodings (matvec_extended.rs:105-141): (x, expected bytes)."""
    r = _Reader("q8k.bin", b"GGQ80001")
    out = []
    for _ in range(r.count):
        n, size = r.word(), r.word()
        out.append((r.floats(n), r.bytes_(size)))
    r.done()
    return out


def encoders(names=("quant-q8_0-q4k-q6k-q8k.bin", "encoder-extended-q8_0-q4k-q6k.bin")):
    """GGQE records: (dtype, x, expected bytes) from quant-reference (Q8_0) and
    encoder-extended-reference (Q4_K, Q6_K) (reference.rs:56-81,
    encoders_extended.rs:27-63); names=("encoder-extended-q2k-q3k-q5k.bin",)
    gives the Q2_K, Q3_K and Q5_K records."""
    out = []
    for name in names:
        r = _Reader(name, b"GGQE0001")
        for _ in range(r.count):
            dtype, n, size = r.word(), r.word(), r.word()
            out.append((dtype, r.floats(n), r.bytes_(size)))
        r.done()
    return out


def dequant(name="dequant-q8_0-q4k-q6k-q8k.bin"):
    """GGQD records: (dtype, n, packed bytes, expected f32) (reference.rs:20-55);
    name="dequant-q2k-q3k-q5k.bin" for Q2_K, Q3_K, Q5_K."""
    r = _Reader(name, b"GGQD0001")
    out = []
    for _ in range(r.count):
        dtype, n, size = r.word(), r.word(), r.word()
        b = r.bytes_(size)
        out.append((dtype, n, b, r.floats(n)))
    r.done()
    return out


# ---- GGML graph records (crates/tensor/tests/{extended,indexing}.rs) ------------

# bytes per element / block and elements per block of the types in these records
_GG_TYPES = {0: (4, 1), 26: (4, 1), 8: (34, 32), 10: (84, 256), 11: (110, 256), 12: (144, 256), 13: (176, 256),
             14: (210, 256), 15: (292, 256)}


@dataclass
class GgTensor:
    dtype: int
    shape: tuple      # ne[0..3]
    strides: tuple    # nb[0..3] in bytes (contiguous for expected outputs)
    data: bytes

    def contiguous(self):
        """Rows of ne[0] elements, row (i1, i2, i3) at offset i1 nb1 + i2 nb2 +
        i3 nb3 of the record, packed one after another (the reference's
        Tensor::contiguous)."""
        ts, bs = _GG_TYPES[self.dtype]
        rb = self.shape[0] // bs * ts
        out = bytearray()
        for i3 in range(self.shape[3]):
            for i2 in range(self.shape[2]):
                for i1 in range(self.shape[1]):
                    o = i1 * self.strides[1] + i2 * self.strides[2] + i3 * self.strides[3]
                    out += self.data[o:o + rb]
        return np.frombuffer(bytes(out), np.uint8).copy()


@dataclass
class GgCase:
    name: str
    tag: str
    inputs: list
    expected: GgTensor


def ggml_cases(name):
    """GGTR0002 records: mul-mat-broadcast.bin (MUL_MAT: weights, rhs) and
    mul-mat-id.bin (MUL_MAT_ID: experts, rhs, ids), expected f32 output."""
    r = _Reader(name, b"GGTR0002")

    def u64():
        return struct.unpack("<Q", r.take(8))[0]

    def string():
        return r.take(r.word()).decode()

    def tensor(strided):
        dtype = r.word()
        shape = tuple(u64() for _ in range(4))
        strides = tuple(u64() for _ in range(4)) if strided else None
        data = r.take(u64())
        if strides is None:
            ts, bs = _GG_TYPES[dtype]
            rb = shape[0] // bs * ts
            strides = (ts, rb, rb * shape[1], rb * shape[1] * shape[2])
        return GgTensor(dtype, shape, strides, data)

    out = []
    for _ in range(r.count):
        nm, tag = string(), string()
        r.word()
        r.take(8 * r.word())
        r.take(4 * r.word())
        nt = r.word()
        inputs = [tensor(True) for _ in range(nt)]
        out.append(GgCase(nm, tag, inputs, tensor(False)))
    r.done()
    return out
