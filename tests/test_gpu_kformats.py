"""GPU parity of the Q2_K, Q3_K and Q5_K weight formats (matvec.hip kernels,
quantize.hip decoders) against the golden records and the CPU oracle, and of
the one-column split kernels Q3_K and Q6_K share, on every launch shape.

Bars, as for Q4_K / Q6_K:
  - decoders and per-block integer dot sums: bit-exact;
  - f32 outputs: relative L2 <= 1e-5 and the per-element bound of the
    reference's tests (2e-5 * (1 + |e|), matvec.rs:55) widened by the
    summation-order bound of each row;
  - Q2_K: bit-exact.  The reference adds `d * isum - mn * mins` per block into
    one f32 sum (matvec_extra.rs:193-195) and the kernel's lane does the same
    in block order.
  - Q3_K and Q5_K with one column: bit-exact.  The one-column kernels keep
    the reference's eight lane accumulators (matvec_extra.rs:223-294).
Weights are the oracle's encoder outputs for small cases and random GGUF
blocks (every bit of the quants and scales random, finite f16 super-scales)
for the rest, which reaches sub-block scales and high bits that encoded
Gaussian data rarely sets.
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
K_OTHER = (DT.Q2_K, DT.Q3_K, DT.Q5_K)
# byte offsets of the f16 super-block scales (d, and dmin where present)
HALVES = {DT.Q2_K: (80, 82), DT.Q3_K: (108,), DT.Q5_K: (0, 2), DT.Q6_K: (208,)}


def say(*a):
    print("[case]", *a, flush=True)


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return np.linalg.norm(got - want) / (den if den > 0 else 1.0)


def elem_tol(t, w, rows, act, cols, want):
    nb = cols // 256
    return 2e-5 * (1 + np.abs(np.asarray(want, np.float64))) + O.order_tolerance(int(t), w, rows, act, nb)


def bits(y):
    return np.asarray(y, np.float32).view(np.uint32)


def exact(t, batch):
    """Whether a launch of `batch` columns gives the reference's f32 bits."""
    return t == DT.Q2_K or (batch == 1 and t in (DT.Q3_K, DT.Q5_K))


def random_blocks(t, rows, cols, seed):
    """GGUF bytes of rows x cols: random quants and scales, f16 super-scales
    drawn from [2^-14, 2^-6] (normal, finite, positive)."""
    rng = np.random.default_rng(seed)
    ts = O.TYPE_SIZE[int(t)]
    nblk = rows * (cols // 256)
    b = rng.integers(0, 256, (nblk, ts), dtype=np.uint8)
    for off in HALVES[t]:
        h = rng.uniform(2.0 ** -14, 2.0 ** -6, nblk).astype(np.float16)
        b[:, off:off + 2] = h.view(np.uint8).reshape(nblk, 2)
    return b.reshape(-1)


def encoded(t, rows, cols, seed):
    x = np.random.default_rng(seed).standard_normal(rows * cols).astype(np.float32) * np.float32(0.02)
    return O.quantize(int(t), x)


def randn(seed, n):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


@pytest.fixture(scope="module")
def ctx():
    c = rlq.Context(0)
    yield c
    c.close()


# ------------------------------------------------------------ golden records

def test_decoders_golden_bitwise():
    for t, n, b, expected in F.dequant("dequant-q2k-q3k-q5k.bin"):
        say("decoder", t, n)
        y = rlq.dequantize(t, b, n)
        same = (bits(y) == bits(expected)) | (np.isnan(y) & np.isnan(expected))
        assert same.all(), t


def test_encoders_golden_bitwise():
    """The device Q2_K / Q3_K / Q5_K encoders (quantize.hip) reproduce the
    reference's encoder records (encoders_extended.rs:27-63) byte for byte."""
    for i, (t, x, expected) in enumerate(F.encoders(("encoder-extended-q2k-q3k-q5k.bin",))):
        say("encoder record", i, t, x.size)
        got = rlq.quantize(t, x)
        assert np.array_equal(got, expected), (i, t, np.nonzero(got != expected)[0][:8])


def edge_blocks(seed):
    """Blocks of 256 values that reach each branch of the encoders: zeros,
    constants of both signs, one spike, all-negative and all-positive
    ramps, scales that round to a zero or subnormal f16, tiny and large
    magnitudes, alternating signs, and Gaussian rows at 0.02 and 1."""
    rng = np.random.default_rng(seed)
    g = lambda s: rng.standard_normal(256).astype(np.float32) * np.float32(s)
    spike = np.zeros(256, np.float32)
    spike[7] = 1.0
    half = g(1.0)
    half[:128] = 0.0
    alt = np.where(np.arange(256) % 2 == 0, 1e-3, -1e-3).astype(np.float32)
    blocks = [np.zeros(256, np.float32), np.full(256, 0.5, np.float32), np.full(256, -0.5, np.float32), spike,
              -np.linspace(0.01, 1.0, 256, dtype=np.float32), np.linspace(0.01, 1.0, 256, dtype=np.float32),
              g(1e-8), g(1e-6), g(1e-30), np.abs(g(1.0)), -np.abs(g(1.0)), g(1e3), g(3e3), half, alt,
              g(0.02), g(1.0)]
    return np.concatenate(blocks + [g(0.02) for _ in range(15)])


@pytest.mark.parametrize("t", K_OTHER)
def test_encoders_against_oracle(ctx, t):
    """Host and device encoders against the oracle's encoder (encode_k.rs),
    bit for bit, on edge blocks and 64 Gaussian rows of 4096; then the
    first UnrepresentableScale block and the first non-finite index."""
    say("encoder vs oracle", t)
    x = edge_blocks(70 + int(t))
    want = O.quantize(int(t), x)
    assert np.array_equal(rlq.quantize(t, x), want)
    xr = np.random.default_rng(71).standard_normal(64 * 4096).astype(np.float32) * np.float32(0.02)
    want_r = O.quantize(int(t), xr)
    got_r = ctx.quantize(t, torch.from_numpy(xr.reshape(64, 4096)).cuda())
    ctx.sync()
    assert np.array_equal(got_r.cpu().numpy(), want_r)
    # a block whose super-scale overflows f16, after two good blocks and
    # before another overflowing one: block 2 is reported
    bad = np.concatenate([x[:512], np.full(256, 1e9, np.float32) * np.sign(x[:256] + 0.5), x[:256] * 1e9])
    with pytest.raises(O.OracleError) as oe:
        O.quantize(int(t), bad)
    with pytest.raises(rlq.QuantError) as e:
        rlq.quantize(t, bad)
    assert (e.value.name, e.value.block) == (oe.value.name, 2) == ("UnrepresentableScale", 2)
    with pytest.raises(rlq.QuantError) as e:
        ctx.quantize(t, torch.from_numpy(bad.reshape(2, 512)).cuda())
        ctx.sync()
    assert (e.value.name, e.value.block) == ("UnrepresentableScale", 2)
    bad[700] = np.nan  # non-finite values are reported before any scale
    with pytest.raises(rlq.QuantError) as e:
        rlq.quantize(t, bad)
    assert (e.value.name, e.value.index) == ("NonFiniteInput", 700)


def test_matvec_golden_records():
    for i, r in enumerate(F.matvec_extended("matvec-extended-q2k-q3k-q5k.bin")):
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


def test_block_sums_golden_records(ctx):
    for i, r in enumerate(F.matvec_extended("matvec-extended-q2k-q3k-q5k.bin")):
        say("GGQX block sums", i, r.dtype)
        W = rlq.Weights(ctx, r.dtype, r.weights, r.rows, r.cols)
        isum, imin = ctx.block_sums(W, torch.from_numpy(r.x).cuda())
        nb = r.cols // 256
        stride = r.weights.size // r.rows
        for row in range(r.rows):
            wi, wm = O.block_sums(r.dtype, r.weights[row * stride:(row + 1) * stride], r.activation, nb)
            assert np.array_equal(isum[row].cpu().numpy(), wi), (i, row)
            assert np.array_equal(imin[row].cpu().numpy(), wm), (i, row)


# ------------------------------------------------------------ exact integer parts

@pytest.mark.parametrize("t", K_OTHER)
@pytest.mark.parametrize("rows,cols,batch", [(300, 4096, 1), (300, 4096, 2), (300, 4096, 3), (300, 4096, 5),
                                             (300, 4096, 8), (7, 768, 1), (37, 2304, 4)])
def test_block_sums_bit_exact(ctx, t, rows, cols, batch):
    """Exact per-block integers of column 0 inside every kernel variant (Q5_K:
    the one-column kernel, then the K-split MFMA kernel from 2 columns; Q2_K /
    Q3_K: the one-column Q3_K kernels, then one or two column groups), rows
    that leave a partial last tile."""
    say("block sums", t, rows, cols, batch)
    w = random_blocks(t, rows, cols, 100 + rows + int(t))
    x = randn(200 + rows, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    isum, imin = ctx.block_sums(W, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    act = O.quantize(O.Q8_K, x[0])
    nb = cols // 256
    stride = w.size // rows
    want_i = np.zeros((rows, nb), np.int32)
    want_m = np.zeros((rows, nb), np.int32)
    for r in range(rows):
        want_i[r], want_m[r] = O.block_sums(int(t), w[r * stride:(r + 1) * stride], act, nb)
    assert np.array_equal(isum.cpu().numpy(), want_i)
    assert np.array_equal(imin.cpu().numpy(), want_m)


@pytest.mark.parametrize("t", (DT.Q2_K, DT.Q3_K))
@pytest.mark.parametrize("rows,batch", [(14336, 1), (14336, 3), (14330, 2), (12288, 4), (10240, 1), (14336, 5),
                                        (14336, 8), (16384, 7)])
def test_block_sums_balanced_deal(ctx, t, rows, batch):
    """Q2_K / Q3_K at 10240..16384 rows run the K-split kernel in the
    balanced deal (one workgroup per CU, four tile slots, the
    last a half tile at 14336 rows; Q3_K with one column the one-column
    kernel): column 0's integers bitwise, every column's outputs against the
    oracle (Q2_K, and Q3_K with one column, bitwise)."""
    cols = 4096
    say("block sums, balanced deal", t, rows, cols, batch)
    w = random_blocks(t, rows, cols, 300 + rows + int(t))
    x = randn(400 + rows + batch, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    isum, imin, y = ctx.block_sums_ex(W, torch.from_numpy(x).cuda())
    ctx.sync()
    act = O.quantize(O.Q8_K, x[0])
    nb = cols // 256
    stride = w.size // rows
    want_i = np.zeros((rows, nb), np.int32)
    want_m = np.zeros((rows, nb), np.int32)
    for r in range(rows):
        want_i[r], want_m[r] = O.block_sums(int(t), w[r * stride:(r + 1) * stride], act, nb)
    assert np.array_equal(isum.cpu().numpy(), want_i)
    assert np.array_equal(imin.cpu().numpy(), want_m)
    got = y.cpu().numpy().reshape(batch, rows)
    want = O.matmul(int(t), w, rows, cols, x, threads=16)
    for b in range(batch):
        assert rel_l2(got[b], want[b]) <= REL_L2, b
    if exact(t, batch):
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("t", [DT.Q3_K, DT.Q6_K])
@pytest.mark.parametrize("rows,cols", [(300, 4096), (7, 768), (6144, 4096), (8200, 2048), (14336, 4096),
                                       (33, 49152), (20, 65536), (16384, 1024), (16400, 1024)])
def test_one_column_split_every_launch_bitwise(ctx, t, rows, cols):
    """Q3_K and Q6_K with one column, each launch shape of the split kernels:
    one 16-wave tile slot of a K split of 16 (no more tiles than CUs; 3
    blocks a row leave most waves without a block, 192 blocks a row fill
    most of LDS), two 8-wave slots of a split of 4 (more tiles, not the
    balanced deal), the balanced deal, and one wave per tile where the parked
    terms of one tile no longer fit LDS (256 blocks a row); Q6_K above 1024
    tiles (16400 rows) walks whole tiles as for the output head.  Column 0's
    integers and every output against the oracle bitwise, and the fused
    argmax against the oracle's."""
    say(t.name, "one column", rows, cols)
    w = random_blocks(t, rows, cols, 500 + rows)
    x = randn(600 + rows, cols).reshape(1, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    isum, imin, y = ctx.block_sums_ex(W, torch.from_numpy(x).cuda())
    ctx.sync()
    act = O.quantize(O.Q8_K, x[0])
    nb = cols // 256
    stride = w.size // rows
    want_i = np.zeros((rows, nb), np.int32)
    for r in range(rows):
        want_i[r] = O.block_sums(int(t), w[r * stride:(r + 1) * stride], act, nb)[0]
    assert np.array_equal(isum.cpu().numpy(), want_i)
    assert not imin.cpu().numpy().any()
    want = O.matmul(int(t), w, rows, cols, x, threads=16)
    assert np.array_equal(bits(y.cpu().numpy().reshape(1, rows)), bits(want))
    y2, am = ctx.matmul_argmax(W, torch.from_numpy(x).cuda())
    ctx.sync()
    assert np.array_equal(bits(y2.cpu().numpy().reshape(1, rows)), bits(want))
    assert int(am[0]) == O.argmax(want[0])


@pytest.mark.parametrize("rows,cols", [(6144, 4096), (8192, 2048)])
@pytest.mark.parametrize("batch", [1, 4])
def test_q2k_balanced_deal_two_slots(ctx, rows, cols, batch):
    """Q2_K at 1.5 and 2 tiles per CU (6144 and 8192 rows on 256 CUs): the
    balanced deal in 8-wave workgroups of two tile slots.  Every output
    bitwise the oracle's (Q2_K keeps the reference's block order at every
    batch)."""
    t = DT.Q2_K
    say("Q2_K balanced deal, two slots", rows, cols, "batch", batch)
    w = random_blocks(t, rows, cols, 900 + rows + batch)
    x = randn(910 + rows + batch, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    y = ctx.matmul(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matmul(int(t), w, rows, cols, x, threads=16)
    assert np.array_equal(bits(y.cpu().numpy().reshape(batch, rows)), bits(want))


# ------------------------------------------------------------ batched device API

@pytest.mark.parametrize("t", K_OTHER)
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 8, 11])
def test_matmul_batches_against_oracle(ctx, t, batch):
    rows, cols = 1000, 4096
    say("matmul", t, rows, cols, batch)
    w = random_blocks(t, rows, cols, 7 + int(t))
    x = randn(11 + batch, batch * cols).reshape(batch, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    y = ctx.matmul(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matmul(int(t), w, rows, cols, x, threads=8)
    got = y.cpu().numpy()
    for b in range(batch):
        assert rel_l2(got[b], want[b]) <= REL_L2, b
    if exact(t, batch):
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("t", K_OTHER)
@pytest.mark.parametrize("batch", [2, 1])
def test_encoded_weights_against_oracle(ctx, t, batch):
    """Weights from the oracle's encoders (the reference's encode_k.rs), a
    shape with 17 blocks per row and a partial last tile (batch 1: the
    16-wave K split that rows of more than 16 blocks take)."""
    rows, cols = 77, 17 * 256
    say("encoded weights matvec", t, rows, cols, "batch", batch)
    w = encoded(t, rows, cols, 31)
    x = randn(32, 2 * cols).reshape(2, cols)[:batch]
    W = rlq.Weights(ctx, t, w, rows, cols)
    y = ctx.matmul(W, torch.from_numpy(np.ascontiguousarray(x)).cuda())
    ctx.sync()
    want = O.matmul(int(t), w, rows, cols, x, threads=8)
    got = y.cpu().numpy()
    for b in range(batch):
        act = O.quantize(O.Q8_K, x[b])
        assert rel_l2(got[b], want[b]) <= REL_L2
        assert np.all(np.abs(got[b] - want[b]) <= elem_tol(t, w, rows, act, cols, want[b]))
    if exact(t, batch):
        assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("t", K_OTHER)
def test_decode_shape_14336x4096_and_argmax(ctx, t):
    rows, cols = 14336, 4096
    say("decode shape + argmax", t, rows, cols)
    w = random_blocks(t, rows, cols, 41 + int(t))
    x = randn(42, cols).reshape(1, cols)
    W = rlq.Weights(ctx, t, w, rows, cols)
    y, am = ctx.matmul_argmax(W, torch.from_numpy(x).cuda())
    ctx.sync()
    want = O.matvec(int(t), w, rows, cols, x[0], threads=16)
    got = y[0].cpu().numpy()
    assert rel_l2(got, want) <= REL_L2
    assert int(am[0]) == O.argmax(got)
    if exact(t, 1):
        assert np.array_equal(bits(got), bits(want))


def test_zero_weights_give_zero(ctx):
    say("zero weights, other K formats")
    for t in K_OTHER:
        W = rlq.Weights(ctx, t, np.zeros(rlq.row_bytes(t, 1024) * 9, np.uint8), 9, 1024)
        y = ctx.matmul(W, torch.from_numpy(randn(1, 2 * 1024).reshape(2, 1024)).cuda())
        ctx.sync()
        assert bool((y == 0).all())


def test_random_block_decoders_bitwise():
    say("decoders on random blocks")
    for t in K_OTHER:
        b = random_blocks(t, 3, 2048, 51 + int(t))
        y = rlq.dequantize(t, b, 3 * 2048)
        want = O.dequantize(int(t), b, 3 * 2048)
        assert np.array_equal(bits(y), bits(want)), t
