#!/usr/bin/env python3
"""Copy the reference's golden records for Q8_0 / Q4_K / Q6_K / Q8_K (and the
other K formats Q2_K / Q3_K / Q5_K) into tests/golden/.

Run once, in a container where the reference checkout is mounted:

    python tests/golden/extract_reference_fixtures.py [/root/reference]

The reference's quant crate pins its scalar path with little-endian binary
fixtures produced from the original ggml C code (crates/quant/README.md:45-57).
This script reads those DATA files only (never code) and keeps the records whose
dtype is on the quantized-matvec path: 8 (Q8_0), 12 (Q4_K), 14 (Q6_K) and
15 (Q8_K), then, in files of their own, 10 (Q2_K), 11 (Q3_K) and 13 (Q5_K).  Each output file keeps the source's record layout and magic, with
the record count rewritten, so a reader of the original format reads it too.
`manifest.json` records, per output, the source file, its SHA-256, the source
record indices kept and the SHA-256 of the output.

Record layouts (all integers u32 LE, floats f32 LE), as read by the reference's
tests:
  GGQX  crates/quant/tests/matvec_extended.rs:50-86
        dtype rows cols wsize asize | w[wsize] x[cols] act[asize] generic[rows] native[rows]
  GGQM  crates/quant/tests/matvec.rs:26-47
        dtype rows cols size | w[size] x[cols] generic[rows] native[rows]
  GGQ8  crates/quant/tests/matvec_extended.rs:109-123
        elements bytes | x[elements] q8k[bytes]
  GGQE  crates/quant/tests/reference.rs:56-75, encoders_extended.rs:27-44
        dtype n size | x[n] expected[size]
  GGQD  crates/quant/tests/reference.rs:20-38
        dtype n size | bytes[size] expected[n]
  GGTR0002  crates/tensor/tests/extended.rs:30-42, 185-204 and indexing.rs:28-41, 90-110
        name tag flag | ni ints[i64] | nf floats | nt tensors | expected tensor
        with tensor = dtype shape[4 x u64] (strides[4 x u64], inputs only) nbytes[u64] bytes
        (strings are u32 length + UTF-8).  Kept: the GGML MUL_MAT and MUL_MAT_ID
        graphs whose weight (first input) type is on the path.
Copied whole (GGUF reader corpus and a real file; crates/gguf/tests/raw_native.rs:286-300):
  fixtures/gguf-bytes/{reader,booleans}-data.bin and -reference.tsv (1093 + 512
  header cases with the original C getters' observations) and
  fixtures/inference/ggml-vocab-llama-spm.gguf (a vocabulary-only Llama GGUF).
"""
import hashlib
import json
import os
import struct
import sys

KEEP = {8, 12, 14, 15}
KEEP_K = {10, 11, 13}
KEEP_MM = {8, 10, 11, 12, 13, 14}
SRC_DIR = "crates/quant/tests/fixtures"
TENSOR_DIR = "crates/tensor/tests/fixtures"


class Reader:
    def __init__(self, data):
        self.data = data
        self.pos = 0

    def take(self, n):
        out = self.data[self.pos:self.pos + n]
        if len(out) != n:
            raise ValueError("truncated fixture")
        self.pos += n
        return out

    def word(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def string(self):
        return self.take(self.word()).decode()

    def ggtr_tensor(self, strided):
        dtype = self.word()
        self.take(32)  # shape
        if strided:
            self.take(32)
        self.take(self.u64())
        return dtype


def split_records(kind, data):
    """Yield (dtype, raw_record_bytes) for every record of a fixture file."""
    r = Reader(data)
    magic = r.take(8)
    count = r.word()
    records = []
    for _ in range(count):
        start = r.pos
        if kind == "GGQX":
            dtype, rows, cols, wsize, asize = (r.word() for _ in range(5))
            r.take(wsize + cols * 4 + asize + rows * 8)
        elif kind == "GGQM":
            dtype, rows, cols, size = (r.word() for _ in range(4))
            r.take(size + cols * 4 + rows * 8)
        elif kind == "GGQ8":
            dtype = 15
            elements, size = r.word(), r.word()
            r.take(elements * 4 + size)
        elif kind == "GGQE":
            dtype, n, size = (r.word() for _ in range(3))
            r.take(n * 4 + size)
        elif kind == "GGQD":
            dtype, n, size = (r.word() for _ in range(3))
            r.take(size + n * 4)
        elif kind == "GGTR0002":
            r.string()
            tag = r.string()
            r.word()
            r.take(8 * r.word())
            r.take(4 * r.word())
            nt = r.word()
            types = [r.ggtr_tensor(True) for _ in range(nt)]
            r.ggtr_tensor(False)
            dtype = types[0] if tag in ("mul_mat", "mul_mat_id") else -1
        else:
            raise ValueError(kind)
        records.append((dtype, data[start:r.pos]))
    if r.pos != len(data):
        raise ValueError("trailing bytes in fixture")
    return magic, records


FILES = [
    ("matvec-extended-reference.bin", "GGQX", "matvec-extended-q4k-q6k.bin", KEEP),
    ("matvec-reference.bin", "GGQM", "matvec-q8_0.bin", KEEP),
    ("q8k-reference.bin", "GGQ8", "q8k.bin", KEEP),
    ("quant-reference.bin", "GGQE", "quant-q8_0-q4k-q6k-q8k.bin", KEEP),
    ("encoder-extended-reference.bin", "GGQE", "encoder-extended-q8_0-q4k-q6k.bin", KEEP),
    ("dequant-reference.bin", "GGQD", "dequant-q8_0-q4k-q6k-q8k.bin", KEEP),
    # the other K formats on the same dot: Q2_K (10), Q3_K (11), Q5_K (13)
    ("matvec-extended-reference.bin", "GGQX", "matvec-extended-q2k-q3k-q5k.bin", KEEP_K),
    ("encoder-extended-reference.bin", "GGQE", "encoder-extended-q2k-q3k-q5k.bin", KEEP_K),
    ("dequant-reference.bin", "GGQD", "dequant-q2k-q3k-q5k.bin", KEEP_K),
    # GGML MUL_MAT with ne2/ne3 broadcast and MUL_MAT_ID with expert ids
    (TENSOR_DIR + "/cpu-extended-reference.bin", "GGTR0002", "mul-mat-broadcast.bin", KEEP_MM),
    (TENSOR_DIR + "/cpu-indexing-gnu-reference.bin", "GGTR0002", "mul-mat-id.bin", KEEP_MM),
]


COPIES = [
    ("fixtures/gguf-bytes/reader-data.bin", "gguf-reader-data.bin"),
    ("fixtures/gguf-bytes/reader-reference.tsv", "gguf-reader-reference.tsv"),
    ("fixtures/gguf-bytes/booleans-data.bin", "gguf-booleans-data.bin"),
    ("fixtures/gguf-bytes/booleans-reference.tsv", "gguf-booleans-reference.tsv"),
    ("fixtures/inference/ggml-vocab-llama-spm.gguf", "ggml-vocab-llama-spm.gguf"),
]


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    here = os.path.dirname(os.path.abspath(__file__))
    manifest = {"source_root": "rust-llama " + SRC_DIR, "kept_dtypes": sorted(KEEP | KEEP_K), "files": {}}
    for src, kind, dst, keep in FILES:
        if "/" not in src:
            src = f"{SRC_DIR}/{src}"
        data = open(os.path.join(root, src), "rb").read()
        magic, records = split_records(kind, data)
        kept = [(i, d, raw) for i, (d, raw) in enumerate(records) if d in keep]
        out = magic + struct.pack("<I", len(kept)) + b"".join(raw for _, _, raw in kept)
        with open(os.path.join(here, dst), "wb") as f:
            f.write(out)
        per_type = {}
        for _, d, _ in kept:
            per_type[str(d)] = per_type.get(str(d), 0) + 1
        manifest["files"][dst] = {
            "source": src,
            "source_sha256": hashlib.sha256(data).hexdigest(),
            "source_records": len(records),
            "kept_source_indices": [i for i, _, _ in kept],
            "kept_per_dtype": per_type,
            "sha256": hashlib.sha256(out).hexdigest(),
            "bytes": len(out),
        }
        print(f"{dst}: {len(kept)} of {len(records)} records, {len(out)} bytes, {per_type}")
    for src, dst in COPIES:
        data = open(os.path.join(root, src), "rb").read()
        with open(os.path.join(here, dst), "wb") as f:
            f.write(data)
        manifest["files"][dst] = {"source": src, "source_sha256": hashlib.sha256(data).hexdigest(),
                                  "sha256": hashlib.sha256(data).hexdigest(), "bytes": len(data), "copied": True}
        print(f"{dst}: copied, {len(data)} bytes")
    with open(os.path.join(here, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
