"""GPU parity over a seeded sweep of shapes: every weight type at row counts
around the kernels' dispatch boundaries (the 16-row tile, partial last tiles,
the balanced deal's 6144..16384 rows and just outside it), block counts from
1 to 72 per row (the K splits of 4 and 16 and the shared-quantization kernel
beyond 64 blocks), and batches 1..8 (one pass of the decode kernels) and 9 or
12 (the prefill GEMM for Q4_K, passes of at most 8 columns otherwise).

Bars, as in test_gpu_parity: column 0's per-block integers bitwise (every
batch for Q4_K, up to 8 columns otherwise), every column's f32 outputs within
relative L2 1e-5 of the oracle, and bitwise where the kernels keep the
reference's f32 order (Q8_0 and Q2_K at every batch, Q3_K, Q4_K, Q5_K and
Q6_K with one column).  A second draw of 48 cases takes most row counts at random and
batches of 13 to 33.  Weights: the library's encoder on N(0, 0.02)
values for Q4_K, Q6_K and Q8_0; random GGUF blocks (random quants and scales,
finite positive f16 super-scales) for Q2_K, Q3_K and Q5_K, as in
test_gpu_kformats.  Every case prints itself before touching the GPU.
"""
import numpy as np
import pytest

import oracle as O
from rlq_loader import load

rlq = load()
torch = rlq.torch
DT = rlq.DType

REL_L2 = 1e-5
DECODE_MAX_BATCH = 8
EXACT_ALWAYS = (DT.Q8_0, DT.Q2_K)
EXACT_ONE_COLUMN = (DT.Q3_K, DT.Q4_K, DT.Q5_K, DT.Q6_K)
# byte offsets of the f16 super-block scales of the random-block formats
HALVES = {DT.Q2_K: (80, 82), DT.Q3_K: (108,), DT.Q5_K: (0, 2)}

TYPES = (DT.Q4_K, DT.Q6_K, DT.Q8_0, DT.Q5_K, DT.Q2_K, DT.Q3_K)
ROW_POOL = (1, 15, 16, 17, 255, 257, 4095, 4097, 6128, 6144, 6150, 8176, 8192, 8200, 10224, 10240, 10250,
            12288, 12290, 14320, 14330, 14336, 16368, 16384, 16400)
NB_POOL = (1, 2, 3, 5, 8, 12, 16, 17, 24, 56, 64, 72)  # 256-value blocks per row
NB_POOL_Q8_0 = (1, 3, 7, 28, 29, 64, 128, 224, 448)  # 32-value blocks per row
BATCHES = (1, 1, 1, 2, 3, 4, 5, 6, 7, 8, 9, 12)
MAX_BLOCKS = {"k": 16384 * 16, "q8_0": 16384 * 128}  # bounds the oracle's work per case


def _cases(n=96, seed=0x5EED, batches=BATCHES, pooled=0.7):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        t = TYPES[i % len(TYPES)]
        rows = int(rng.choice(ROW_POOL)) if rng.random() < pooled else int(rng.integers(1, 17000))
        if t == DT.Q8_0:
            nb, bs, cap = int(rng.choice(NB_POOL_Q8_0)), 32, MAX_BLOCKS["q8_0"]
        else:
            nb, bs, cap = int(rng.choice(NB_POOL)), 256, MAX_BLOCKS["k"]
        while rows * nb > cap and nb > 1:
            nb //= 2
        out.append((t, rows, nb * bs, int(rng.choice(batches))))
    return out


CASES = _cases()
# a second draw: row counts mostly at random, batches of 13 to 33 (two to
# five passes of the decode kernels; Q4_K's GEMM with one ragged token tile)
CASES_WIDE = _cases(48, seed=0xC0FFEE, batches=(1, 2, 5, 8, 13, 16, 17, 24, 31, 33), pooled=0.3)


def say(*a):
    print("[case]", *a, flush=True)


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return np.linalg.norm(got - want) / (den if den > 0 else 1.0)


def _weights(t, rows, cols, seed):
    rng = np.random.default_rng(seed)
    if t not in HALVES:
        return rlq.quantize(t, (rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    nblk = rows * (cols // 256)
    b = rng.integers(0, 256, (nblk, O.TYPE_SIZE[int(t)]), dtype=np.uint8)
    for off in HALVES[t]:
        b[:, off:off + 2] = rng.uniform(2.0 ** -14, 2.0 ** -6, nblk).astype(np.float16).view(np.uint8).reshape(nblk, 2)
    return b.reshape(-1)


def test_sweep_covers_the_dispatch_boundaries():
    """The sweep reaches every weight type, both sides of the balanced deal's
    row band, block counts on both sides of 16 and 64, and batches on both
    sides of 8 (a regression guard for the case generator itself)."""
    types = {c[0] for c in CASES}
    assert types == set(TYPES)
    rows = [c[1] for c in CASES]
    assert any(r < 6144 for r in rows) and any(6144 <= r <= 16384 for r in rows) and any(r > 16384 for r in rows)
    nbs = [c[2] // 256 for c in CASES if c[0] != DT.Q8_0]
    assert any(n <= 16 for n in nbs) and any(16 < n <= 64 for n in nbs)
    batches = [c[3] for c in CASES]
    assert any(b == 1 for b in batches) and any(1 < b <= 8 for b in batches) and any(b > 8 for b in batches)


@pytest.mark.gpu
@pytest.mark.parametrize("t,rows,cols,batch", CASES + CASES_WIDE,
                         ids=[f"{DT(c[0]).name}-{c[1]}x{c[2]}-b{c[3]}" for c in CASES + CASES_WIDE])
def test_sweep(t, rows, cols, batch):
    say("sweep", DT(t).name, rows, cols, "batch", batch)
    seed = rows * 131 + cols * 7 + batch + int(t)
    w = _weights(t, rows, cols, seed)
    x = np.random.default_rng(seed + 1).standard_normal(batch * cols).astype(np.float32).reshape(batch, cols)
    ctx = rlq.Context(0)
    try:
        W = rlq.Weights(ctx, t, w, rows, cols)
        xd = torch.from_numpy(x).cuda()
        sums = t == DT.Q4_K or batch <= DECODE_MAX_BATCH
        if sums:
            isum, imin, y = ctx.block_sums_ex(W, xd)
        else:
            y = ctx.matmul(W, xd)
        ctx.sync()
        got = y.cpu().numpy().reshape(batch, rows)
        if sums:
            nb = cols // O.BLOCK[int(t)]
            act = O.quantize(O.matvec_activation_dtype(int(t)), x[0])
            stride = w.size // rows
            want_i = np.zeros((rows, nb), np.int32)
            want_m = np.zeros((rows, nb), np.int32)
            for r in range(rows):
                want_i[r], want_m[r] = O.block_sums(int(t), w[r * stride:(r + 1) * stride], act, nb)
            assert np.array_equal(isum.cpu().numpy(), want_i)
            assert np.array_equal(imin.cpu().numpy(), want_m)
        want = O.matmul(int(t), w, rows, cols, x, threads=16)
        for b in range(batch):
            assert rel_l2(got[b], want[b]) <= REL_L2, b
        if t in EXACT_ALWAYS or (batch == 1 and t in EXACT_ONE_COLUMN):  # the reference's f32 order
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        W.close()
    finally:
        ctx.close()
