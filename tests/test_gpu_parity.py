"""GPU parity: the HIP path (librlq.so through its C ABI) against the golden
records and the CPU oracle.

Bars:
  - bytes the reference pins bit-exactly (quantizer and encoder outputs,
    decoders) are compared bit-exactly;
  - per-block integer dot sums are compared bit-exactly (rlq_block_sums);
  - f32 outputs: relative L2 error <= 1e-5 against the oracle / golden C
    output, plus a per-element bound of 2e-5 * (1 + |e|) where the reference's
    own tests use that bound (matvec.rs:55);
  - f32 outputs bit-exact where the kernels follow the reference's f32 order:
    Q8_0 at every batch size, Q4_K / Q5_K / Q6_K with one column (the
    reference's eight lane accumulators, matvec_extra.rs:223-294).
Every test prints its case before touching the GPU.
"""
import numpy as np
import pytest

import oracle as O
from golden import fixtures as F
from rlq_loader import load

pytestmark = pytest.mark.gpu

rlq = load()
torch = rlq.torch
DT = rlq.DType

REL_L2 = 1e-5


def say(*a):
    print("[case]", *a, flush=True)


def bits(y):
    return np.asarray(y, np.float32).view(np.uint32)


def exact(t, batch):
    """Whether a launch of `batch` columns gives the reference's f32 bits."""
    return t == DT.Q8_0 or (batch == 1 and t in (DT.Q4_K, DT.Q5_K, DT.Q6_K))


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return np.linalg.norm(got - want) / (den if den > 0 else 1.0)


def elem_tol(t, w, rows, act, cols, want):
    """Per-element bound: the reference tests' 2e-5 * (1 + |e|) (matvec.rs:55)
    widened by the f32 summation-order bound of each row (the GPU adds the
    same exact integer block sums in another order; records built for
    cancellation need the latter)."""
    nb = cols // O.BLOCK[int(t)]
    return 2e-5 * (1 + np.abs(np.asarray(want, np.float64))) + O.order_tolerance(int(t), w, rows, act, nb)


@pytest.fixture(scope="module")
def ctx():
    c = rlq.Context(0)
    yield c
    c.close()


def randn(seed, n, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


# ------------------------------------------------------------ golden records

def test_q8k_quantizer_golden_bitwise():
    for i, (x, expected) in enumerate(F.q8k()):
        say("q8k record", i, x.size)
        assert np.array_equal(rlq.quantize(DT.Q8_K, x), expected), i
    for i, r in enumerate(F.matvec_extended()):
        say("GGQX activation", i)
        assert np.array_equal(rlq.quantize(DT.Q8_K, r.x), r.activation), i


def test_encoders_golden_bitwise():
    for i, (t, x, expected) in enumerate(F.encoders()):
        say("encoder record", i, t, x.size)
        got = rlq.quantize(t, x)
        assert np.array_equal(got, expected), (i, t, np.nonzero(got != expected)[0][:8])


def test_decoders_golden_bitwise():
    for t, n, b, expected in F.dequant():
        say("decoder", t, n)
        y = rlq.dequantize(t, b, n)
        same = (y.view(np.uint32) == expected.view(np.uint32)) | (np.isnan(y) & np.isnan(expected))
        assert same.all(), t


def test_matvec_golden_q4k_q6k():
    for i, r in enumerate(F.matvec_extended()):
        say("GGQX matvec", i, r.dtype, r.rows, r.cols)
        y = rlq.matvec(r.dtype, r.weights, r.rows, r.cols, r.x)
        assert rel_l2(y, r.generic) <= REL_L2, i
        tol = elem_tol(r.dtype, r.weights, r.rows, r.activation, r.cols, r.generic)
        assert np.all(np.abs(y - r.generic) <= tol), (i, np.abs(y - r.generic) - tol)
        if exact(r.dtype, 1):
            assert np.array_equal(bits(y), bits(r.generic)), i
        stride = r.weights.size // r.rows
        for row in range(r.rows):
            d = rlq.dot_packed(r.dtype, r.weights[row * stride:(row + 1) * stride], r.activation, r.cols)
            assert abs(d - r.generic[row]) <= tol[row], (i, row)
            if exact(r.dtype, 1):
                assert bits(d) == bits(r.generic[row]), (i, row)


def test_matvec_golden_q8_0():
    for i, r in enumerate(F.matvec_q8_0()):
        say("GGQM matvec", i, r.rows, r.cols)
        y = rlq.matvec(r.dtype, r.weights, r.rows, r.cols, r.x)
        assert rel_l2(y, r.generic) <= REL_L2, i
        tol = elem_tol(r.dtype, r.weights, r.rows, O.quantize(O.Q8_0, r.x), r.cols, r.native)
        assert np.all(np.abs(y - r.native) <= tol), i
        # Q8_0 adds the block terms in the reference's order: bit-exact
        assert np.array_equal(y.view(np.uint32), r.generic.view(np.uint32)), i


# ------------------------------------------------------------ exact integer parts

def _weights(t, rows, cols, seed):
    return rlq.quantize(t, randn(seed, rows * cols, 0.02))


@pytest.mark.parametrize("t,rows,cols,batch", [
    (DT.Q4_K, 300, 4096, 1), (DT.Q4_K, 300, 4096, 2), (DT.Q4_K, 300, 4096, 3), (DT.Q4_K, 300, 4096, 8),
    (DT.Q6_K, 300, 4096, 1), (DT.Q6_K, 300, 4096, 5), (DT.Q8_0, 300, 896, 1), (DT.Q8_0, 300, 896, 8),
    (DT.Q8_0, 21, 96, 3), (DT.Q4_K, 7, 768, 1), (DT.Q4_K, 7, 768, 4), (DT.Q6_K, 5, 2304, 1)])
def test_block_sums_bit_exact(ctx, t, rows, cols, batch):
    """Exact per-block integers of column 0 inside every kernel variant (the
    batch size picks the kernel: Q4_K 1-2 VALU dot4, 3-8 MFMA; Q6_K 5-8 two
    column groups; Q8_0 with an odd block count)."""
    say("block sums", t, rows, cols, batch)
    w = _weights(t, rows, cols, 100 + rows)
    x = randn(200 + rows, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    isum, imin = ctx.block_sums(W, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    at = O.matvec_activation_dtype(int(t))
    act = O.quantize(at, x[0])
    nb = cols // O.BLOCK[int(t)]
    stride = w.size // rows
    want_i = np.zeros((rows, nb), np.int32)
    want_m = np.zeros((rows, nb), np.int32)
    for r in range(rows):
        want_i[r], want_m[r] = O.block_sums(int(t), w[r * stride:(r + 1) * stride], act, nb)
    assert np.array_equal(isum.cpu().numpy(), want_i)
    assert np.array_equal(imin.cpu().numpy(), want_m)


def _q5k_blocks(rows, cols, seed):
    """GGUF Q5_K bytes of rows x cols: random quants and scales, f16 d and
    dmin drawn from [2^-14, 2^-6] (they reach the high bits and sub-block
    scales that encoded Gaussian rows rarely set)."""
    rng = np.random.default_rng(seed)
    nblk = rows * (cols // 256)
    b = rng.integers(0, 256, (nblk, 176), dtype=np.uint8)
    for off in (0, 2):
        b[:, off:off + 2] = rng.uniform(2.0 ** -14, 2.0 ** -6, nblk).astype(np.float16).view(np.uint8).reshape(nblk, 2)
    return b.reshape(-1)


def _packed(t, rows, cols, seed):
    return _q5k_blocks(rows, cols, seed) if t == DT.Q5_K else _weights(t, rows, cols, seed)


def _oracle_sums(t, w, rows, act, nb):
    stride = w.size // rows
    want_i = np.zeros((rows, nb), np.int32)
    want_m = np.zeros((rows, nb), np.int32)
    for r in range(rows):
        want_i[r], want_m[r] = O.block_sums(int(t), w[r * stride:(r + 1) * stride], act, nb)
    return want_i, want_m


@pytest.mark.parametrize("t,rows,cols,variant", [
    (DT.Q4_K, 4096, 4096, "batch-1 kernel, one tile slot, K split 4 (< 384 tiles)"),
    (DT.Q4_K, 6144, 4096, "batch-1 kernel, balanced deal, u = 3: one workgroup of two slots per CU, a full and a half tile"),
    (DT.Q4_K, 8192, 4096, "batch-1 kernel, balanced deal, u = 4: two slots per CU, two full tiles"),
    (DT.Q4_K, 10240, 4096, "batch-1 kernel, balanced deal, u = 5: four slots per CU, two full tiles, a half, one idle"),
    (DT.Q4_K, 6400, 4096, "batch-1 kernel, two tile slots, K split 4, grid-strided (400 tiles)"),
    (DT.Q4_K, 12288, 4096, "batch-1 kernel, balanced deal, u = 6: four slots per CU, one idle"),
    (DT.Q4_K, 14336, 4096, "batch-1 kernel, balanced deal, u = 7: four slots per CU, the last a half tile: the headline"),
    (DT.Q4_K, 14330, 4096, "balanced deal, u = 7, the last tile partial and dealt out in halves"),
    (DT.Q4_K, 16384, 4096, "batch-1 kernel, balanced deal, u = 8: four full tiles per CU"),
    (DT.Q4_K, 14336, 512, "balanced deal, two blocks per row: two of each slot's four K parts idle"),
    (DT.Q5_K, 14336, 768, "Q5_K, balanced deal, three blocks per row"),
    (DT.Q5_K, 14336, 4096, "Q5_K, batch-1 kernel, balanced deal, u = 7"),
    (DT.Q4_K, 4096, 14336, "batch-1 kernel, 16 waves, K split 16 (> 16 blocks)"),
    (DT.Q4_K, 333, 16384, "batch-1 kernel, K split 16 at 64 blocks: 4 blocks per wave, the most it takes"),
    (DT.Q4_K, 333, 18432, "72 blocks: the shared-quantization kernel, 16 waves, K split 16"),
    (DT.Q4_K, 333, 28672, "112 blocks (a Llama-70B down projection): the compact activation image"),
    (DT.Q5_K, 40, 32768, "Q5_K, 128 blocks: the compact activation image"),
    (DT.Q5_K, 4096, 4096, "Q5_K, batch-1 kernel, K split 4"),
    (DT.Q5_K, 4096, 14336, "Q5_K, batch-1 kernel, K split 16")])
def test_block_sums_every_decode_variant(ctx, t, rows, cols, variant):
    """rlq_block_sums runs the very kernel variant rlq_matmul picks for a
    shape (the batch-1 variants are chosen by tile and block counts): the
    integers of every (row, block) bitwise, and the same launch's f32
    outputs against the oracle."""
    say("block sums, batch 1,", t, rows, cols, variant)
    w = _packed(t, rows, cols, 300 + rows + cols)
    x = randn(400 + rows, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    isum, imin, y = ctx.block_sums_ex(W, torch.from_numpy(x).cuda())
    ctx.sync()
    nb = cols // 256
    want_i, want_m = _oracle_sums(t, w, rows, O.quantize(O.Q8_K, x), nb)
    assert np.array_equal(isum.cpu().numpy(), want_i)
    assert np.array_equal(imin.cpu().numpy(), want_m)
    want = O.matvec(int(t), w, rows, cols, x, threads=16)
    assert rel_l2(y.cpu().numpy(), want) <= REL_L2
    assert np.array_equal(bits(y.cpu().numpy()), bits(want))


def test_one_column_beyond_the_one_column_kernels(ctx):
    """One Q4_K column of 65536 values (256 blocks per row): the one-column
    kernels' compact image and one tile's parked terms exceed the LDS, so the
    batched kernel runs it: integers bitwise, outputs within the f32 bar."""
    t, rows, cols = DT.Q4_K, 40, 65536
    say("one column beyond the one-column kernels", t, rows, cols)
    w = _packed(t, rows, cols, 77)
    x = randn(78, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    isum, imin, y = ctx.block_sums_ex(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want_i, want_m = _oracle_sums(t, w, rows, O.quantize(O.Q8_K, x), cols // 256)
    assert np.array_equal(isum.cpu().numpy(), want_i)
    assert np.array_equal(imin.cpu().numpy(), want_m)
    assert rel_l2(y.cpu().numpy(), O.matvec(int(t), w, rows, cols, x, threads=16)) <= REL_L2


@pytest.mark.parametrize("t,rows,cols,batch", [
    (DT.Q4_K, 14336, 4096, 2), (DT.Q4_K, 14336, 4096, 5), (DT.Q4_K, 14336, 4096, 8), (DT.Q4_K, 14330, 4096, 3),
    (DT.Q4_K, 6144, 4096, 4), (DT.Q5_K, 14336, 4096, 6), (DT.Q4_K, 14336, 512, 3), (DT.Q4_K, 12288, 8192, 2),
    (DT.Q4_K, 14336, 768, 7)])
def test_block_sums_balanced_columns(ctx, t, rows, cols, batch):
    """Two to eight columns in the balanced deal (one workgroup per CU: four
    tile slots at 12288..16384 rows, the last a half tile at 14336, two slots
    at 6144; fused quantization below seven columns, the planes from
    seven): column 0's integers bitwise, every column's outputs against the
    oracle."""
    say("block sums, balanced deal,", t, rows, cols, "batch", batch)
    w = _packed(t, rows, cols, 900 + rows + batch)
    x = randn(950 + batch, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    isum, imin, y = ctx.block_sums_ex(W, torch.from_numpy(x).cuda())
    ctx.sync()
    nb = cols // 256
    want_i, want_m = _oracle_sums(t, w, rows, O.quantize(O.Q8_K, x[0]), nb)
    assert np.array_equal(isum.cpu().numpy(), want_i)
    assert np.array_equal(imin.cpu().numpy(), want_m)
    got = y.cpu().numpy().reshape(batch, rows)
    for b in range(batch):
        assert rel_l2(got[b], O.matvec(int(t), w, rows, cols, x[b], threads=16)) <= REL_L2, b


def _interleave_tiles(g, u, rows, row_bytes):
    """[gate tile 0, up tile 0, gate tile 1, ...] of two GGUF matrices of
    `rows` rows (a multiple of 16): the decode step's gate/up layout."""
    gt = g.reshape(rows // 16, 16 * row_bytes)
    ut = u.reshape(rows // 16, 16 * row_bytes)
    return np.stack([gt, ut], axis=1).reshape(-1)


@pytest.mark.parametrize("t,ff,cols", [(DT.Q4_K, 14336, 4096), (DT.Q4_K, 512, 4096), (DT.Q5_K, 14336, 4096),
                                       (DT.Q4_K, 1024, 2048)])
def test_silu_pair_kernel_integers_and_outputs(ctx, t, ff, cols):
    """The decode step's gate/up kernel (two gate/up tile pairs per
    workgroup, K split over two waves per tile, silu(gate) * up in the
    epilogue): integers of every gate and up row bitwise, and silu(gate) * up
    within 1e-5 of the oracle's (llama.rs:367-371)."""
    say("SiLU-pair gate/up kernel", t, ff, cols)
    rb = rlq.row_bytes(t, cols)
    g = _packed(t, ff, cols, 500 + ff)
    u = _packed(t, ff, cols, 600 + ff)
    W = rlq.Weights(ctx, t, _interleave_tiles(g, u, ff, rb), 2 * ff, cols)
    x = randn(700 + ff, cols)
    isum, imin, y = ctx.block_sums_ex(W, torch.from_numpy(x).cuda(), flags=ctx.SUMS_SILU_PAIR)
    ctx.sync()
    nb = cols // 256
    act = O.quantize(O.Q8_K, x)
    gi, gm = _oracle_sums(t, g, ff, act, nb)
    ui, um = _oracle_sums(t, u, ff, act, nb)
    wi = np.stack([gi.reshape(ff // 16, 16, nb), ui.reshape(ff // 16, 16, nb)], axis=1).reshape(2 * ff, nb)
    wm = np.stack([gm.reshape(ff // 16, 16, nb), um.reshape(ff // 16, 16, nb)], axis=1).reshape(2 * ff, nb)
    assert np.array_equal(isum.cpu().numpy(), wi)
    assert np.array_equal(imin.cpu().numpy(), wm)
    want = O.silu(O.matvec(int(t), g, ff, cols, x, threads=16)) * O.matvec(int(t), u, ff, cols, x, threads=16)
    assert rel_l2(y.cpu().numpy(), want) <= REL_L2
    assert np.array_equal(bits(y.cpu().numpy()), bits(want))


def test_block_sums_golden_records(ctx):
    for i, r in enumerate(F.matvec_extended()):
        say("GGQX block sums", i)
        W = rlq.Weights(ctx, r.dtype, r.weights, r.rows, r.cols)
        isum, imin = ctx.block_sums(W, torch.from_numpy(r.x).cuda())
        nb = r.cols // 256
        stride = r.weights.size // r.rows
        for row in range(r.rows):
            wi, wm = O.block_sums(r.dtype, r.weights[row * stride:(row + 1) * stride], r.activation, nb)
            assert np.array_equal(isum[row].cpu().numpy(), wi), (i, row)
            assert np.array_equal(imin[row].cpu().numpy(), wm), (i, row)


# ------------------------------------------------------------ batched device API

@pytest.mark.parametrize("t,rows,cols", [(DT.Q4_K, 2000, 4096), (DT.Q6_K, 1500, 4096), (DT.Q8_0, 2000, 896),
                                         (DT.Q4_K, 333, 14336)])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 8, 11])
def test_matmul_batches_against_oracle(ctx, t, rows, cols, batch):
    say("matmul", t, rows, cols, batch)
    w = _weights(t, rows, cols, 7 + rows)
    x = randn(11 + batch, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    y = ctx.matmul(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matmul(int(t), w, rows, cols, x, threads=8)
    got = y.cpu().numpy()
    for b in range(batch):
        assert rel_l2(got[b], want[b]) <= REL_L2, b
    if exact(t, batch):  # the reference's f32 order: bit-exact
        assert np.array_equal(bits(got), bits(want))


# ------------------------------------------------------------ the benchmark shapes

def test_q4k_14336x4096_encoder_and_matvec(ctx):
    rows, cols = 14336, 4096
    say("Q4_K full shape", rows, cols)
    xw = randn(0x51A7E002, rows * cols, 0.02)
    w = rlq.quantize(DT.Q4_K, xw)
    stride = w.size // rows
    for r in (0, 1, 5000, rows - 1):  # GPU encoder == oracle encoder, bit for bit
        assert np.array_equal(w[r * stride:(r + 1) * stride], O.quantize(O.Q4_K, xw[r * cols:(r + 1) * cols])), r
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    for batch in (1, 4, 8):
        x = randn(batch, batch * cols).reshape(batch, cols)
        y = ctx.matmul(W, torch.from_numpy(x).cuda())
        ctx.sync()
        want = O.matmul(O.Q4_K, w, rows, cols, x, threads=16)
        for b in range(batch):
            assert rel_l2(y[b].cpu().numpy(), want[b]) <= REL_L2, (batch, b)
        if exact(DT.Q4_K, batch):
            assert np.array_equal(bits(y.cpu().numpy()), bits(want)), batch


def test_q6k_lm_head_128256x4096_argmax(ctx):
    rows, cols = 128256, 4096
    say("Q6_K lm_head", rows, cols)
    xw = randn(0x51A7E004, rows * cols, 0.02)
    w = rlq.quantize(DT.Q6_K, xw)
    stride = w.size // rows
    for r in (0, 77777, rows - 1):
        assert np.array_equal(w[r * stride:(r + 1) * stride], O.quantize(O.Q6_K, xw[r * cols:(r + 1) * cols])), r
    del xw
    W = rlq.Weights(ctx, DT.Q6_K, w, rows, cols)
    # 256 workgroups of 512 threads: batches 1 and 2 leave the last workgroup
    # one slot key per thread, 4 and 8 several (loaded eight at a time)
    for batch in (1, 2, 4, 8):
        x = randn(40 + batch, batch * cols).reshape(batch, cols)
        y, am = ctx.matmul_argmax(W, torch.from_numpy(x).cuda())
        ctx.sync()
        got = y.cpu().numpy()
        want = O.matmul(O.Q6_K, w, rows, cols, x, threads=16)
        for b in range(batch):
            assert rel_l2(got[b], want[b]) <= REL_L2, (batch, b)
            i = int(am[b])
            assert i == O.argmax(got[b]), b  # fused argmax == greedy choice on the same logits
            assert want[b][i] >= want[b].max() - 1e-5 * abs(want[b].max()), b
        if exact(DT.Q6_K, batch):
            assert np.array_equal(bits(got), bits(want)), batch
            assert int(am[0]) == O.argmax(want[0])


def test_q8_0_qwen_ffn_up_4864x896(ctx):
    """The Qwen2.5-0.5B FFN-up shape at batch 1 (the benchmark's Q8_0
    configuration, 304 tiles): the library's encoder equals the oracle's on
    sampled rows, and the outputs are bitwise the oracle's (the reference's
    block-order f32 sum), for N(0, 1) input and a few edge columns."""
    rows, cols = 4864, 896
    say("Q8_0 FFN up", rows, cols)
    xw = randn(0x51A7E001, rows * cols, 0.02)
    w = rlq.quantize(DT.Q8_0, xw)
    stride = w.size // rows
    for r in (0, 1, 2431, rows - 1):
        assert np.array_equal(w[r * stride:(r + 1) * stride], O.quantize(O.Q8_0, xw[r * cols:(r + 1) * cols])), r
    W = rlq.Weights(ctx, DT.Q8_0, w, rows, cols)
    cases = [randn(0x51A7E101, cols), np.zeros(cols, np.float32), np.full(cols, 1e-6, np.float32),
             (randn(0x51A7E102, cols) * np.float32(1e4)).astype(np.float32)]
    for k, x in enumerate(cases):
        y = ctx.matmul(W, torch.from_numpy(x.reshape(1, cols)).cuda())
        ctx.sync()
        want = O.matvec(O.Q8_0, w, rows, cols, x, threads=16)
        assert np.array_equal(bits(y.cpu().numpy()[0]), bits(want)), k


@pytest.mark.parametrize("rows,cols,batch", [(4096, 14336, 1), (33, 14336, 2), (70, 16384, 1)])
def test_q8_0_long_rows_compact_parking(ctx, rows, cols, batch):
    """Q8_0 rows of 448-512 blocks, too long for the K-split kernels' eight
    parked columns: 16 waves of a 16-way split park only the batch's
    columns.  Every output bitwise the oracle's (block order), and the fused
    argmax of column 0 the oracle's."""
    say("Q8_0 long rows", rows, cols, "batch", batch)
    w = rlq.quantize(DT.Q8_0, randn(0x51A7E201 + rows, rows * cols, 0.02))
    W = rlq.Weights(ctx, DT.Q8_0, w, rows, cols)
    x = randn(0x51A7E301 + batch, batch * cols).reshape(batch, cols)
    y, am = ctx.matmul_argmax(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matmul(O.Q8_0, w, rows, cols, x, threads=16)
    assert np.array_equal(bits(y.cpu().numpy().reshape(batch, rows)), bits(want))
    for b in range(batch):
        assert int(am[b]) == O.argmax(want[b]), b


def test_q8_0_qwen_lm_head_151936x896(ctx):
    rows, cols = 151936, 896
    say("Q8_0 lm_head", rows, cols)
    xw = randn(0x51A7E005, rows * cols, 0.02)
    w = rlq.quantize(DT.Q8_0, xw)
    assert np.array_equal(w[:952 * 3], O.quantize(O.Q8_0, xw[:896 * 3]))
    W = rlq.Weights(ctx, DT.Q8_0, w, rows, cols)
    # three workgroups per CU: several slot keys per thread of the last one
    for batch in (1, 2):
        x = randn(5 + batch, batch * cols).reshape(batch, cols)
        y, am = ctx.matmul_argmax(W, torch.from_numpy(x).cuda())
        ctx.sync()
        want = O.matmul(O.Q8_0, w, rows, cols, x, threads=16)
        for b in range(batch):
            assert rel_l2(y[b].cpu().numpy(), want[b]) <= REL_L2, (batch, b)
            assert int(am[b]) == O.argmax(y[b].cpu().numpy()), (batch, b)


def test_argmax_keys_across_calls(ctx):
    """The greedy-token kernel sets the argmax keys back to 0, and a call
    clears only keys past those: batches 3, 1, 5, 2, 12 (the prefill GEMM)
    and 1 in a row, each argmax the first maximum of its own logits."""
    rows, cols = 1000, 2048
    w = _weights(DT.Q4_K, rows, cols, 77)
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    for i, batch in enumerate((3, 1, 5, 2, 12, 1)):
        say("argmax keys across calls, batch", batch)
        x = randn(300 + i, batch * cols).reshape(batch, cols)
        y, am = ctx.matmul_argmax(W, torch.from_numpy(x).cuda())
        ctx.sync()
        got = y.cpu().numpy()
        for b in range(batch):
            assert int(am[b]) == O.argmax(got[b]), (batch, b)


@pytest.mark.parametrize("t,rows,cols", [(DT.Q8_0, 9000, 896), (DT.Q6_K, 3000, 2048), (DT.Q4_K, 5000, 4096),
                                         (DT.Q4_K, 9000, 2048), (DT.Q4_K, 14336, 4096)])
def test_argmax_nan_rows(ctx, t, rows, cols):
    """The greedy scan (sampling.rs:607-618) starts from row 0 and keeps the
    first strict maximum: a NaN at row 0 is the answer (nothing compares
    greater), a NaN anywhere else never wins.  NaN logits come from a NaN f16
    scale in one row's first block.  Batches 1 and 3, over the in-launch
    argmax of the decode kernels (at 14336 rows also a NaN in a tile that the
    batch-1 kernel deals out in halves)."""
    say("argmax with NaN logits", t, rows, cols)
    w = _weights(t, rows, cols, 88)
    rb = w.size // rows
    dpos = {DT.Q8_0: 0, DT.Q6_K: 208, DT.Q4_K: 0}[t]  # the f16 d of block 0
    for nan_row in (0, 1234) + ((rows - 300,) if rows > 12288 else ()):
        wn = w.copy()
        wn[nan_row * rb + dpos:nan_row * rb + dpos + 2] = np.array([0x7E00], np.uint16).view(np.uint8)
        W = rlq.Weights(ctx, t, wn, rows, cols)
        for batch in (1, 3):
            x = torch.from_numpy(randn(90 + batch, batch * cols).reshape(batch, cols)).cuda()
            y, am = ctx.matmul_argmax(W, x)
            ctx.sync()
            got = y.cpu().numpy()
            for b in range(batch):
                assert np.isnan(got[b][nan_row]), (nan_row, b)
                assert int(am[b]) == O.argmax(got[b]), (nan_row, b)
                if nan_row == 0:
                    assert int(am[b]) == 0
        W.close()


# ------------------------------------------------------------ errors and edges

def test_host_errors_leave_output_untouched():
    say("host errors")
    w = _weights(DT.Q4_K, 4, 512, 3)
    x = np.ones(512, np.float32)
    x[300] = np.inf
    with pytest.raises(rlq.QuantError) as e:
        rlq.matvec(DT.Q4_K, w, 4, 512, x)
    assert (e.value.name, e.value.index) == ("NonFiniteInput", 300)
    x = np.ones(512, np.float32)
    x[256:] = np.frombuffer(np.uint32(1).tobytes(), np.float32)[0]
    with pytest.raises(rlq.QuantError) as e:
        rlq.matvec(DT.Q4_K, w, 4, 512, x)
    assert (e.value.name, e.value.block) == ("UnrepresentableScale", 1)
    out = np.full(584, 0xA5, np.uint8)
    with pytest.raises(rlq.QuantError):
        rlq.quantize_into(DT.Q8_K, x, out)
    assert (out == 0xA5).all()
    rlq.quantize_into(DT.Q8_K, np.full(512, -0.0, np.float32), out)
    assert (out == 0).all()
    x = np.ones(64, np.float32)
    x[40] = np.nan
    with pytest.raises(rlq.QuantError) as e:
        rlq.quantize(DT.Q8_0, x)
    assert (e.value.name, e.value.index) == ("NonFiniteInput", 40)
    with pytest.raises(rlq.QuantError) as e:
        rlq.quantize(DT.Q8_0, np.full(64, 3e38, np.float32))
    assert (e.value.name, e.value.block) == ("UnrepresentableScale", 0)
    xk = randn(9, 512)
    xk[17] = np.nan
    for t in (DT.Q4_K, DT.Q6_K):
        with pytest.raises(rlq.QuantError) as e:
            rlq.quantize(t, xk)
        assert (e.value.name, e.value.index) == ("NonFiniteInput", 17)


def test_device_errors_suppress_outputs_and_report_first_column(ctx):
    say("device errors")
    rows, cols = 64, 512
    W = rlq.Weights(ctx, DT.Q4_K, _weights(DT.Q4_K, rows, cols, 4), rows, cols)
    x = torch.ones((3, cols), dtype=torch.float32, device="cuda")
    x[2, 7] = float("nan")
    x[1, 256:] = 1e-45  # unrepresentable scale in column 1, block 1
    y = torch.full((3, rows), 123.0, device="cuda")
    ctx.matmul(W, x, y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.block, e.value.b) == ("UnrepresentableScale", 1, 1)
    assert bool((y == 123.0).all())
    ctx.sync()  # the error word was cleared
    x = torch.zeros((2, cols), dtype=torch.float32, device="cuda")
    ctx.matmul(W, x, y[:2])
    ctx.sync()
    assert bool((y[:2] == 0).all())


def test_device_errors_of_six_to_eight_columns(ctx):
    """Six to eight Q4_K / Q5_K columns are quantized once by the planes
    kernel, then multiplied: the first error (by column, then the
    reference's order inside it) is reported, no output is written, and a
    clean call is exact against the oracle."""
    for t in (DT.Q4_K, DT.Q5_K):
        rows, cols, batch = 1000, 1024, 7
        say("device errors, planes path", t, rows, cols, batch)
        w = _weights(t, rows, cols, 7) if t == DT.Q4_K else _q5k_blocks(rows, cols, 7)
        W = rlq.Weights(ctx, t, w, rows, cols)
        x = torch.from_numpy(randn(8, batch * cols).reshape(batch, cols)).cuda()
        y = torch.full((batch, rows), 123.0, device="cuda")
        bad = x.clone()
        bad[5, 600] = float("inf")
        bad[3, 256:512] = 1e-45
        ctx.matmul(W, bad, y)
        with pytest.raises(rlq.QuantError) as e:
            ctx.sync()
        assert (e.value.name, e.value.block, e.value.b) == ("UnrepresentableScale", 1, 3)
        assert bool((y == 123.0).all())
        ctx.matmul(W, x, y)
        ctx.sync()
        got, xs = y.cpu().numpy(), x.cpu().numpy()
        for b in range(batch):
            assert rel_l2(got[b], O.matvec(int(t), w, rows, cols, xs[b], threads=16)) <= REL_L2, (t, b)


def test_device_errors_of_the_batch1_plain_kernel(ctx):
    """One f32 column over 513 tiles (the batch-1 kernel whose workgroups
    each quantize their own blocks): the first error is reported and no
    output is written; a clean call afterwards is exact."""
    rows, cols = 8208, 1024
    say("device errors, batch-1 kernel", rows, cols)
    w = _weights(DT.Q4_K, rows, cols, 5)
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    y = torch.full((1, rows), 123.0, device="cuda")
    x = torch.from_numpy(randn(6, cols)).cuda()
    bad = x.clone()
    bad[900] = float("nan")
    bad[300] = float("inf")
    ctx.matmul(W, bad.view(1, cols), y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index) == ("NonFiniteInput", 300)
    assert bool((y == 123.0).all())
    tiny = x.clone()
    tiny[768:] = 1e-45
    ctx.matmul(W, tiny.view(1, cols), y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.block) == ("UnrepresentableScale", 3)
    assert bool((y == 123.0).all())
    ctx.matmul(W, x.view(1, cols), y)
    ctx.sync()
    assert rel_l2(y.cpu().numpy()[0], O.matvec(O.Q4_K, w, rows, cols, x.cpu().numpy(), threads=16)) <= REL_L2


from test_oracle_llama import huge_q4k  # noqa: E402


@pytest.mark.parametrize("rows", [64, 8208])
def test_multiply_finite_checks(ctx, rows):
    """Matrix::multiply (math.rs:144-169): finite(input) as NonFinite
    "matrix input" before anything is written, the quantizer's
    UnrepresentableScale, and finite(output) as NonFinite "matrix output"
    (an f32 overflow forced by extreme weights and input; the oracle's own
    product overflows the same way); a finite product equals rlq_matmul's
    bitwise.  8208 rows (513 tiles) run the batch-1 plain-column kernel."""
    cols = 1024
    say("Matrix::multiply finite checks", rows, cols)
    W = rlq.Weights(ctx, DT.Q4_K, _weights(DT.Q4_K, rows, cols, 12), rows, cols)
    x = torch.from_numpy(randn(13, cols)).cuda()
    y = ctx.multiply(W, x)
    ctx.sync()
    assert torch.equal(y.view(torch.int32), ctx.matmul(W, x)[0].view(torch.int32))
    bad = x.clone()
    bad[700] = float("inf")
    y.fill_(7.0)
    ctx.multiply(W, bad, y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.a, e.value.b) == ("NonFinite", 3, 0)
    assert bool((y == 7.0).all())
    tiny = x.clone()
    tiny[512:768] = 1e-45
    ctx.multiply(W, tiny, y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.block) == ("UnrepresentableScale", 2)
    assert bool((y == 7.0).all())
    Wh = rlq.Weights(ctx, DT.Q4_K, huge_q4k(rows, cols), rows, cols)
    big = np.full(cols, 1e36, np.float32)
    want = O.matvec(O.Q4_K, huge_q4k(rows, cols), rows, cols, big)
    assert not np.all(np.isfinite(want))  # the reference's multiply fails its output check here
    y = ctx.multiply(Wh, torch.from_numpy(big).cuda())
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.a, e.value.b) == ("NonFinite", 4, 0)
    assert not bool(torch.isfinite(y).all())
    ctx.matmul(Wh, torch.from_numpy(big).cuda())  # llama_quant::matvec has no output check
    ctx.sync()


def test_bound_matmul_is_matmul(ctx):
    """Context.bind_matmul: the prepared call writes what matmul writes, the
    argmax form what matmul_argmax writes, every time it runs; a data error
    raises from the call's sync like matmul's."""
    rows, cols = 9000, 2048
    say("prepared matmul calls", rows, cols)
    W = rlq.Weights(ctx, DT.Q4_K, _weights(DT.Q4_K, rows, cols, 21), rows, cols)
    x = torch.from_numpy(randn(22, cols)).cuda().view(1, cols)
    want = ctx.matmul(W, x)
    want_y, want_am = ctx.matmul_argmax(W, x)
    y = torch.empty((1, rows), device="cuda")
    y2, am = torch.empty((1, rows), device="cuda"), torch.empty(1, dtype=torch.int32, device="cuda")
    call, call_am = ctx.bind_matmul(W, x, y), ctx.bind_matmul(W, x, y2, am)
    for _ in range(3):
        y.fill_(0.0)
        call()
        call_am()
        ctx.sync()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32))
        assert torch.equal(y2.view(torch.int32), want_y.view(torch.int32)) and int(am[0]) == int(want_am[0])
    x[0, 5] = float("nan")
    call()
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index) == ("NonFiniteInput", 5)


def test_zero_weights_give_zero(ctx):
    say("zero weights")
    for t, cols in ((DT.Q4_K, 1024), (DT.Q6_K, 1024), (DT.Q8_0, 96)):
        W = rlq.Weights(ctx, t, np.zeros(rlq.row_bytes(t, cols) * 9, np.uint8), 9, cols)
        y = ctx.matmul(W, torch.from_numpy(randn(1, 2 * cols).reshape(2, cols)).cuda())
        ctx.sync()
        assert bool((y == 0).all())


# ------------------------------------------------------------ streams and lifetimes

@pytest.mark.parametrize("t", [DT.Q4_K, DT.Q6_K, DT.Q8_0, DT.Q8_K])
def test_device_quantize_is_ordered_after_torch_producer(ctx, t):
    """Calls with stream=None run on torch's current stream, so a quantize
    queued right after the kernel that writes its input sees the final
    values (no host synchronisation in between)."""
    rows, cols = 2048, 4096
    say("ordered quantize", t, rows, cols)
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    xw = torch.randn((rows, cols), generator=g, device="cuda", dtype=torch.float32) * 0.02
    packed = ctx.quantize(t, xw)
    ctx.sync()
    host_x = xw.cpu().numpy().reshape(-1)
    want = O.quantize(int(t), host_x)
    assert np.array_equal(packed.cpu().numpy(), want)


def test_weights_outlive_their_context():
    say("weights after context")
    c = rlq.Context(0)
    W = rlq.Weights(c, DT.Q4_K, _weights(DT.Q4_K, 8, 256, 5), 8, 256)
    c.close()
    W.close()


@pytest.mark.parametrize("t,batch", [(DT.Q4_K, 1), (DT.Q4_K, 3), (DT.Q6_K, 1)])
def test_fused_quantizer_on_golden_q8k_inputs(ctx, t, batch):
    """The matvec kernels quantize x to Q8_K themselves.  Fed the golden Q8_K
    inputs (zeros, signed zeros, +/- ties, F32 max, tiny scales), the exact
    block integers must equal those of the golden activation bytes, and the
    f32 outputs those of the oracle for every row whose sum of absolute terms
    stays below F32 max / 2.  (Rows built from x near F32 max can overflow in
    some summation orders and not in others: the reference's eight lane sums
    and separate mins sum, or the GPU's per-block terms.)"""
    for i, (x, expected) in enumerate(F.q8k()):
        cols, rows = x.size, 32
        say("fused q8k golden", t, batch, i, cols)
        w = _weights(t, rows, cols, 500 + i)
        W = rlq.Weights(ctx, t, w, rows, cols)
        xb = np.tile(x, (batch, 1))
        isum, imin = ctx.block_sums(W, torch.from_numpy(xb).cuda())
        torch.cuda.synchronize()
        stride = w.size // rows
        nb = cols // 256
        for r in range(rows):
            wi, wm = O.block_sums(int(t), w[r * stride:(r + 1) * stride], expected, nb)
            assert np.array_equal(isum[r].cpu().numpy(), wi), (i, r)
            assert np.array_equal(imin[r].cpu().numpy(), wm), (i, r)
        y = ctx.matmul(W, torch.from_numpy(xb).cuda())
        ctx.sync()
        want = O.matvec(int(t), w, rows, cols, x)
        got = y[0].cpu().numpy()
        in_range = np.array([O.abs_terms(int(t), w[r * stride:(r + 1) * stride], expected, nb)
                             < float(np.finfo(np.float32).max) / 2 for r in range(rows)])  # compared in f64
        assert np.isfinite(want[in_range]).all() and np.isfinite(got[in_range]).all(), i
        if in_range.any():
            tol = elem_tol(t, w, rows, expected, cols, want)[in_range]
            assert np.all(np.abs(got[in_range].astype(np.float64) - want[in_range]) <= tol), i


# ------------------------------------------------------------ prefill GEMM (Q4_K, batch > 8)

@pytest.mark.parametrize("rows,cols,batch", [(300, 4096, 16), (300, 4096, 200), (70, 768, 129), (64, 256, 9)])
def test_gemm_block_sums_bit_exact(ctx, rows, cols, batch):
    """Token 0's exact per-block integers inside the prefill GEMM (two-plane
    MFMA sums and base-128 mins digits), on partial row and token tiles."""
    say("gemm block sums", rows, cols, batch)
    w = _weights(DT.Q4_K, rows, cols, 900 + rows)
    x = randn(901 + batch, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    isum, imin = ctx.block_sums(W, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    act = O.quantize(O.Q8_K, x[0])
    nb = cols // 256
    stride = w.size // rows
    for r in range(rows):
        wi, wm = O.block_sums(O.Q4_K, w[r * stride:(r + 1) * stride], act, nb)
        assert np.array_equal(isum[r].cpu().numpy(), wi), r
        assert np.array_equal(imin[r].cpu().numpy(), wm), r


@pytest.mark.parametrize("level,split", [(69 / 127, False), (70 / 127, True), (1.0, True)])
def test_gemm_exact_at_the_f32_bound(ctx, level, split):
    """The GEMM sums sc*q*q8 in f32 chains, exact while every partial sum
    stays below 2^24.  Weights of all +1 encode to sc = 63, q = 15 (sc*q =
    945, the largest); token 0's blocks hold one 1.0 and 255 values `level`,
    all of one sign (no cancellation): sum |q8| = 127 + 255 round(127 level).
    69/127 gives 17722 <= 17753, one chain per block with |sum| = 945 * 17722
    = 16747290 < 2^24; 70/127 and 1.0 exceed 17753, the token's tile folds
    half blocks (1.0: a full-block chain would pass odd partial sums above
    2^24).  The other tokens are random, so the flag decides for a mixed tile."""
    rows, cols, batch = 48, 512, 16
    say("gemm exact at the f32 bound", level, split)
    w = O.quantize(O.Q4_K, np.ones(rows * cols, np.float32))
    x = randn(903, batch * cols).reshape(batch, cols)
    x[0] = np.float32(level)
    x[0, ::256] = 1.0
    act = O.quantize(O.Q8_K, x[0])
    q8 = np.concatenate([act[b * 292 + 4:b * 292 + 260].view(np.int8) for b in range(cols // 256)])
    assert (int(np.abs(q8.astype(np.int64)).reshape(-1, 256).sum(axis=1).max()) > 17753) == split
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    isum, imin = ctx.block_sums(W, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    stride = w.size // rows
    for r in range(rows):
        wi, wm = O.block_sums(O.Q4_K, w[r * stride:(r + 1) * stride], act, cols // 256)
        assert np.array_equal(isum[r].cpu().numpy(), wi), r
        assert np.array_equal(imin[r].cpu().numpy(), wm), r
    assert abs(int(isum[0, 0])) > 16_000_000  # the construction reaches the bound
    y = ctx.matmul(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matmul(O.Q4_K, w, rows, cols, x, threads=16)
    got = y.cpu().numpy()
    for b in range(batch):
        assert rel_l2(got[b], want[b]) <= REL_L2, b


@pytest.mark.parametrize("rows,cols,batch", [(333, 4096, 64), (1000, 2048, 129), (96, 14336, 17)])
def test_gemm_against_oracle(ctx, rows, cols, batch):
    say("gemm", rows, cols, batch)
    w = _weights(DT.Q4_K, rows, cols, 77 + rows)
    x = randn(78 + batch, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    y = ctx.matmul(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matmul(O.Q4_K, w, rows, cols, x, threads=16)
    got = y.cpu().numpy()
    for b in range(batch):
        assert rel_l2(got[b], want[b]) <= REL_L2, b


def test_gemm_prefill_shape_512x14336x4096(ctx):
    """The prefill benchmark shape: every token against the oracle on a
    sample of rows, and the full output's per-token relative L2 on 64
    tokens."""
    rows, cols, batch = 14336, 4096, 512
    say("gemm prefill shape", rows, cols, batch)
    xw = randn(0x51A7E003, rows * cols, 0.02)
    w = rlq.quantize(DT.Q4_K, xw)
    del xw
    x = randn(0x51A7E003 + 7, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    y = ctx.matmul(W, torch.from_numpy(x).cuda())
    ctx.sync()
    got = y.cpu().numpy()
    stride = w.size // rows
    sample = np.arange(0, rows, 97)
    ws = np.concatenate([w[r * stride:(r + 1) * stride] for r in sample])
    want = O.matmul(O.Q4_K, ws, sample.size, cols, x, threads=16)
    for b in range(batch):
        assert rel_l2(got[b, sample], want[b]) <= REL_L2, b
    want_full = O.matmul(O.Q4_K, w, rows, cols, x[:64:9], threads=16)
    for k, b in enumerate(range(0, 64, 9)):
        assert rel_l2(got[b], want_full[k]) <= REL_L2, b


def test_gemm_argmax_and_errors(ctx):
    rows, cols, batch = 1000, 1024, 24
    say("gemm argmax and errors", rows, cols, batch)
    w = _weights(DT.Q4_K, rows, cols, 41)
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    x = randn(42, batch * cols).reshape(batch, cols)
    y, am = ctx.matmul_argmax(W, torch.from_numpy(x).cuda())
    ctx.sync()
    got = y.cpu().numpy()
    for b in range(batch):
        assert int(am[b]) == O.argmax(got[b]), b
    xt = torch.from_numpy(x).cuda()
    xt[13, 500] = float("inf")
    y2 = torch.full((batch, rows), 7.0, device="cuda")
    ctx.matmul(W, xt, y2)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index, e.value.b) == ("NonFiniteInput", 500, 13)
    assert bool((y2 == 7.0).all())


def test_gemm_many_token_tiles(ctx):
    """Seventeen and thirty-three token tiles: every token against the oracle
    at 2100 tokens (a partial last tile), then a non-finite value in the last
    of 4100 tokens, which every workgroup's scan of the records' flags must
    reach: the call reports its column and element and writes nothing."""
    rows, cols = 64, 4096
    w = _weights(DT.Q4_K, rows, cols, 91)
    W = rlq.Weights(ctx, DT.Q4_K, w, rows, cols)
    batch = 2100
    say("gemm many token tiles", rows, cols, batch)
    x = randn(92, batch * cols).reshape(batch, cols)
    y = ctx.matmul(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matmul(O.Q4_K, w, rows, cols, x, threads=16)
    got = y.cpu().numpy()
    for b in range(batch):
        assert rel_l2(got[b], want[b]) <= REL_L2, b
    batch = 4100
    say("gemm many token tiles, error in the last token", rows, cols, batch)
    xt = torch.from_numpy(randn(93, batch * cols).reshape(batch, cols)).cuda()
    xt[batch - 1, 4095] = float("nan")
    y2 = torch.full((batch, rows), 7.0, device="cuda")
    ctx.matmul(W, xt, y2)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index, e.value.b) == ("NonFiniteInput", 4095, batch - 1)
    assert bool((y2 == 7.0).all())
