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
