"""GPU parity of GGML MUL_MAT with broadcast (rlq_mul_mat) and MUL_MAT_ID
(rlq_mul_mat_id) against the reference's graph fixtures and the oracle.

Bars: Q8_0 and Q2_K outputs bitwise (each adds its block terms in the
reference's order); the other K formats relative L2 <= 1e-5 per output row
and per element 2e-5 * (1 + |e|) plus the summation-order bound of the row
(the exact block integers are the reference's; only the f32 order differs).
Errors: the reference's order (Shape, Unsupported at the call; Bounds before
any quantizer error at rlq_sync) and no output written by a refused call.
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
EXACT = (O.Q8_0, O.Q2_K)


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = rlq.Context(0)
    yield c
    c.close()


def bits(y):
    return np.asarray(y, np.float32).view(np.uint32)


def check_rows(t, mats, rows, cols, acts, got, want, where):
    """got/want [..., rows] rows of outputs; mats[i] the GGUF bytes of the
    matrix and acts[i] the activation bytes of output row i."""
    got = np.asarray(got, np.float32).reshape(-1, rows)
    want = np.asarray(want, np.float32).reshape(-1, rows)
    if t in EXACT:
        assert np.array_equal(bits(got), bits(want)), where
        return
    nb = cols // O.BLOCK[t]
    for i in range(got.shape[0]):
        if mats[i] is None:  # an expert slot with id -1
            assert np.all(got[i] == 0.0), (where, i)
            continue
        g, e = got[i].astype(np.float64), want[i].astype(np.float64)
        den = np.linalg.norm(e)
        assert np.linalg.norm(g - e) <= 1e-5 * (den if den > 0 else 1.0), (where, i)
        tol = 2e-5 * (1 + np.abs(e)) + O.order_tolerance(t, mats[i], rows, acts[i], nb)
        assert np.all(np.abs(g - e) <= tol), (where, i)


def rhs_device(b, xd, x):
    if xd == O.F32:
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    return torch.from_numpy(np.ascontiguousarray(x, np.uint8)).cuda()


def act_rows(at, xd, x, cols, n):
    if xd == at:
        return np.ascontiguousarray(x, np.uint8).reshape(n, -1)
    xs = np.ascontiguousarray(x, np.float32).reshape(n, cols)
    return np.stack([O.quantize(at, xs[i]) for i in range(n)])


# ------------------------------------------------------------ golden graph records

def test_mul_mat_broadcast_golden(ctx):
    for c in F.ggml_cases("mul-mat-broadcast.bin"):
        say("MUL_MAT broadcast record", c.name)
        a, b = c.inputs[0], c.inputs[1]
        K, rows, wn2, wn3 = a.shape
        _, ncols, n2, n3 = b.shape
        t, xd = a.dtype, b.dtype
        xb = b.contiguous()
        x = xb.view(np.float32) if xd == O.F32 else xb
        wb = a.contiguous()
        W = rlq.Weights(ctx, t, wb, rows, K, wn2, wn3)
        xdev = rhs_device(b, xd, x).reshape(n3, n2, ncols, -1)
        y = ctx.mul_mat(W, xdev, x_dtype=xd)
        ctx.sync()
        want = np.frombuffer(c.expected.data, np.float32)
        at = O.matvec_activation_dtype(t)
        acts = act_rows(at, xd, x, K, ncols * n2 * n3)
        mb = rows * O.row_bytes(t, K)
        mats = []
        for i3 in range(n3):
            for i2 in range(n2):
                m = (i3 // (n3 // wn3)) * wn2 + i2 // (n2 // wn2)
                mats += [wb[m * mb:(m + 1) * mb]] * ncols
        check_rows(t, mats, rows, K, acts, y.cpu().numpy(), want, c.name)


def test_mul_mat_id_golden(ctx):
    for c in F.ggml_cases("mul-mat-id.bin"):
        say("MUL_MAT_ID record", c.name)
        a, b, it = c.inputs
        K, rows, experts, _ = a.shape
        _, ncols, tokens, _ = b.shape
        t, xd = a.dtype, b.dtype
        ids = np.frombuffer(it.contiguous().tobytes(), np.int32).reshape(it.shape[1], it.shape[0]).copy()
        xb = b.contiguous()
        x = xb.view(np.float32) if xd == O.F32 else xb
        wb = a.contiguous()
        W = rlq.Weights(ctx, t, wb, rows, K, experts)
        y = ctx.mul_mat_id(W, rhs_device(b, xd, x).reshape(tokens, ncols, -1), torch.from_numpy(ids).cuda(),
                           x_dtype=xd)
        ctx.sync()
        want = np.frombuffer(c.expected.data, np.float32)
        at = O.matvec_activation_dtype(t)
        acts_c = act_rows(at, xd, x, K, tokens * ncols)
        mb = rows * O.row_bytes(t, K)
        mats, acts = [], []
        for tk in range(tokens):
            for s in range(ids.shape[1]):
                e = ids[tk, s]
                mats.append(None if e < 0 else wb[e * mb:(e + 1) * mb])
                acts.append(acts_c[tk * ncols + s % ncols])
        check_rows(t, mats, rows, K, acts, y.cpu().numpy(), want, c.name)


# ------------------------------------------------------------ larger shapes vs oracle

def random_w(t, rows, cols, mats, seed):
    x = np.random.default_rng(seed).standard_normal(rows * cols * mats).astype(np.float32) * np.float32(0.02)
    return O.quantize(t, x)


@pytest.mark.parametrize("t", [O.Q4_K, O.Q6_K, O.Q2_K, O.Q8_0, O.Q5_K])
def test_mul_mat_id_decode_shape(ctx, t):
    """8 experts of 512 x 2048, 3 tokens x 4 slots over one shared column
    (the gate/up shape) and over one column per slot (the down shape)."""
    rows, cols, experts, tokens, slots = 512, 2048, 8, 3, 4
    w = random_w(t, rows, cols, experts, 60 + t)
    W = rlq.Weights(ctx, t, w, rows, cols, experts)
    rng = np.random.default_rng(61)
    ids = np.stack([rng.permutation(experts)[:slots] for _ in range(tokens)]).astype(np.int32)
    ids[1, 2] = -1
    for ncols in (1, slots):
        say("MUL_MAT_ID", t, rows, cols, experts, tokens, slots, ncols)
        x = rng.standard_normal((tokens, ncols, cols)).astype(np.float32)
        y = ctx.mul_mat_id(W, torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda())
        ctx.sync()
        want = O.mul_mat_id(t, w, rows, cols, experts, O.F32, x, ncols, tokens, ids)
        at = O.matvec_activation_dtype(t)
        acts_c = act_rows(at, O.F32, x, cols, tokens * ncols)
        mb = rows * O.row_bytes(t, cols)
        mats = [None if ids[k, s] < 0 else w[ids[k, s] * mb:(ids[k, s] + 1) * mb]
                for k in range(tokens) for s in range(slots)]
        acts = [acts_c[k * ncols + s % ncols] for k in range(tokens) for s in range(slots)]
        check_rows(t, mats, rows, cols, acts, y.cpu().numpy(), want, (t, ncols))


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q3_K, O.Q2_K, O.Q8_0])
@pytest.mark.parametrize("rows,cols", [(300, 2048), (40, 4352)])
def test_mul_mat_id_one_token_single_launch(ctx, t, rows, cols):
    """One token with one f32 column shared by its slots (MoE decode): one
    launch checks the ids and quantizes the column in every workgroup.  Its
    outputs equal the planes path's bit for bit (the same column given as
    activation bytes), meet the oracle's bars, and refusals write nothing."""
    experts, slots = 6, 3
    say("MUL_MAT_ID one token", t, rows, cols, experts, slots)
    w = random_w(t, rows, cols, experts, 70 + t)
    W = rlq.Weights(ctx, t, w, rows, cols, experts)
    rng = np.random.default_rng(71)
    x = rng.standard_normal((1, 1, cols)).astype(np.float32)
    at = O.matvec_activation_dtype(t)
    xq = O.quantize(at, x.reshape(-1))
    mb = rows * O.row_bytes(t, cols)
    for ids in ([[4, 0, -1]], [[2, 2, 5]], [[-1, -1, -1]]):
        ids = np.array(ids, np.int32)
        y = ctx.mul_mat_id(W, torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda())
        yq = ctx.mul_mat_id(W, torch.from_numpy(xq).cuda().reshape(1, 1, -1), torch.from_numpy(ids).cuda(),
                            x_dtype=DT(at))
        ctx.sync()
        got = y.cpu().numpy()
        assert np.array_equal(bits(got), bits(yq.cpu().numpy())), ids
        want = O.mul_mat_id(t, w, rows, cols, experts, O.F32, x, 1, 1, ids)
        mats = [None if i < 0 else w[i * mb:(i + 1) * mb] for i in ids[0]]
        check_rows(t, mats, rows, cols, [xq] * slots, got, want, (t, ids.tolist()))
    # an id out of range: Bounds at its flat index, before the bad column
    xb = x.copy()
    xb[0, 0, 100] = np.nan
    y = torch.full((1, slots, rows), 7.0, device="cuda")
    ctx.mul_mat_id(W, torch.from_numpy(xb).cuda(), torch.tensor([[0, 6, -1]], dtype=torch.int32, device="cuda"), y=y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.a) == ("Bounds", 1)
    assert bool((y == 7.0).all())
    # valid ids and a non-finite value: refused, nothing written (the -1 slot included)
    ctx.mul_mat_id(W, torch.from_numpy(xb).cuda(), torch.tensor([[0, 5, -1]], dtype=torch.int32, device="cuda"), y=y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index, e.value.b) == ("NonFiniteInput", 100, 0)
    assert bool((y == 7.0).all())


def test_mul_mat_id_many_pairs_packed_rhs(ctx):
    """64 tokens x 2 slots of 16 Q4_K experts with Q8_K activation bytes as
    the right-hand side (used as given)."""
    t, rows, cols, experts, tokens, slots = O.Q4_K, 96, 1024, 16, 64, 2
    say("MUL_MAT_ID packed", rows, cols, experts, tokens, slots)
    w = random_w(t, rows, cols, experts, 70)
    W = rlq.Weights(ctx, t, w, rows, cols, experts)
    rng = np.random.default_rng(71)
    ids = rng.integers(-1, experts, (tokens, slots)).astype(np.int32)
    xf = rng.standard_normal((tokens * slots, cols)).astype(np.float32)
    packed = np.concatenate([O.quantize(O.Q8_K, r) for r in xf])
    y = ctx.mul_mat_id(W, torch.from_numpy(packed).cuda().reshape(tokens, slots, -1), torch.from_numpy(ids).cuda(),
                       x_dtype=DT.Q8_K)
    ctx.sync()
    want = O.mul_mat_id(t, w, rows, cols, experts, O.Q8_K, packed, slots, tokens, ids)
    mb = rows * O.row_bytes(t, cols)
    arb = O.row_bytes(O.Q8_K, cols)
    mats = [None if ids[k, s] < 0 else w[ids[k, s] * mb:(ids[k, s] + 1) * mb]
            for k in range(tokens) for s in range(slots)]
    acts = [packed[(k * slots + s) * arb:(k * slots + s + 1) * arb] for k in range(tokens) for s in range(slots)]
    check_rows(t, mats, rows, cols, acts, y.cpu().numpy(), want, "packed")


@pytest.mark.parametrize("t,xd", [(O.Q4_K, O.F32), (O.Q3_K, O.Q8_K), (O.Q8_0, O.Q8_0)])
def test_mul_mat_broadcast_shapes(ctx, t, xd):
    rows, cols, wn2, wn3, n2, n3, ncols = 100, 1024, 2, 3, 4, 3, 5
    say("MUL_MAT broadcast", t, xd, rows, cols, (wn2, wn3), (n2, n3), ncols)
    w = random_w(t, rows, cols, wn2 * wn3, 80 + t)
    W = rlq.Weights(ctx, t, w, rows, cols, wn2, wn3)
    xf = np.random.default_rng(81).standard_normal((n3, n2, ncols, cols)).astype(np.float32)
    if xd == O.F32:
        x, xdev = xf, torch.from_numpy(xf).cuda()
    else:
        x = np.concatenate([O.quantize(xd, r) for r in xf.reshape(-1, cols)])
        xdev = torch.from_numpy(x).cuda().reshape(n3, n2, ncols, -1)
    y = ctx.mul_mat(W, xdev, x_dtype=xd)
    ctx.sync()
    want = O.mul_mat(t, w, rows, cols, wn2, wn3, xd, x, ncols, n2, n3)
    at = O.matvec_activation_dtype(t)
    acts = act_rows(at, xd, x, cols, n3 * n2 * ncols)
    mb = rows * O.row_bytes(t, cols)
    mats = []
    for i3 in range(n3):
        for i2 in range(n2):
            m = (i3 // (n3 // wn3)) * wn2 + i2 // (n2 // wn2)
            mats += [w[m * mb:(m + 1) * mb]] * ncols
    check_rows(t, mats, rows, cols, acts, y.cpu().numpy(), want, (t, xd))


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q3_K, O.Q2_K, O.Q8_0])
def test_mul_mat_one_column_single_launch(ctx, t):
    """MUL_MAT of one f32 column (a decode step's GGML graph): one launch
    that quantizes the column in every workgroup.  Bitwise equal to the
    planes path (the column given as activation bytes), the oracle's bars,
    and a non-finite value refuses the call."""
    rows, cols = 300, 2304 if t == O.Q8_0 else 2048
    say("MUL_MAT one column", t, rows, cols)
    w = random_w(t, rows, cols, 1, 90 + t)
    W = rlq.Weights(ctx, t, w, rows, cols)
    x = np.random.default_rng(91).standard_normal((1, 1, 1, cols)).astype(np.float32)
    at = O.matvec_activation_dtype(t)
    xq = O.quantize(at, x.reshape(-1))
    y = ctx.mul_mat(W, torch.from_numpy(x).cuda())
    yq = ctx.mul_mat(W, torch.from_numpy(xq).cuda().reshape(1, 1, 1, -1), x_dtype=DT(at))
    ctx.sync()
    got = y.cpu().numpy()
    assert np.array_equal(bits(got), bits(yq.cpu().numpy()))
    want = O.mul_mat(t, w, rows, cols, 1, 1, O.F32, x, 1, 1, 1)
    check_rows(t, [w], rows, cols, [xq], got, want, t)
    x[0, 0, 0, 33] = np.inf
    y = torch.full((1, 1, 1, rows), 7.0, device="cuda")
    ctx.mul_mat(W, torch.from_numpy(x).cuda(), y=y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index, e.value.b) == ("NonFiniteInput", 33, 0)
    assert bool((y == 7.0).all())


# ------------------------------------------------------------ errors

def test_errors_refuse_the_whole_call(ctx):
    t, rows, cols, experts = O.Q4_K, 32, 512, 3
    say("MUL_MAT_ID errors")
    w = random_w(t, rows, cols, experts, 90)
    W = rlq.Weights(ctx, t, w, rows, cols, experts)
    x = torch.ones((2, 2, cols), dtype=torch.float32, device="cuda")
    y = torch.full((2, 2, rows), 7.0, device="cuda")
    with pytest.raises(rlq.QuantError) as e:  # 3 slots over 2 columns
        ctx.mul_mat_id(W, x, torch.zeros((2, 3), dtype=torch.int32, device="cuda"), y=torch.empty((2, 3, rows),
                                                                                                  device="cuda"))
    assert e.value.name == "Shape"
    with pytest.raises(rlq.QuantError) as e:
        ctx.mul_mat_id(W, x, torch.zeros((2, 2), dtype=torch.int32, device="cuda"), x_dtype=DT.Q8_0)
    assert e.value.name == "Unsupported"
    # an id out of range: Bounds at sync (index = flat position), before the
    # non-finite column, and nothing written
    x[0, 1, 5] = float("nan")
    ids = torch.tensor([[0, 1], [3, -1]], dtype=torch.int32, device="cuda")
    ctx.mul_mat_id(W, x, ids, y=y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.a) == ("Bounds", 2)
    assert bool((y == 7.0).all())
    # valid ids: the non-finite value of column 1, nothing written
    ids = torch.tensor([[0, 1], [2, -1]], dtype=torch.int32, device="cuda")
    ctx.mul_mat_id(W, x, ids, y=y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index, e.value.b) == ("NonFiniteInput", 5, 1)
    assert bool((y == 7.0).all())
    # clean: every slot written, -1 as zero
    x[0, 1, 5] = 1.0
    ctx.mul_mat_id(W, x, ids, y=y)
    ctx.sync()
    assert bool((y[1, 1] == 0).all()) and not bool((y == 7.0).any())
    # MUL_MAT: a broadcast that does not divide, a data error in a later slice
    W2 = rlq.Weights(ctx, t, w[:2 * rows * O.row_bytes(t, cols)], rows, cols, 2, 1)
    with pytest.raises(rlq.QuantError) as e:
        ctx.mul_mat(W2, torch.ones((1, 3, 1, cols), device="cuda"))
    assert e.value.name == "Shape"
    xm = torch.ones((1, 4, 2, cols), device="cuda")
    xm[0, 3, 1, 9] = float("inf")
    ym = torch.full((1, 4, 2, rows), 7.0, device="cuda")
    ctx.mul_mat(W2, xm, y=ym)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index, e.value.b) == ("NonFiniteInput", 9, 7)
    assert bool((ym == 7.0).all())
