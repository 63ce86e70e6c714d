"""rlq_matmul_noalloc (the entry point that allocates nothing; its argmax
keys and the prefill GEMM's activation image live in the library's static
device scratch) against rlq_matmul / rlq_matmul_argmax, which allocate their
scratch in the context: the same kernels, so the outputs must be bitwise
equal.  Two calls in a row, the second with a smaller input, so stale
scratch contents of the first call cannot leak into the second."""
import numpy as np
import pytest

from rlq_loader import load

pytestmark = pytest.mark.gpu

rlq = load()
torch = rlq.torch
DT = rlq.DType


def say(*a):
    print("[case]", *a, flush=True)


def bits(t):
    return t.view(torch.int32)


@pytest.fixture(scope="module")
def ctx():
    c = rlq.Context(0)
    yield c
    c.close()


def weights(ctx, t, rows, cols, seed):
    x = (np.random.default_rng(seed).standard_normal(rows * cols) * 0.02).astype(np.float32)
    return rlq.Weights(ctx, t, rlq.quantize(t, x), rows, cols)


def inputs(seed, batch, cols):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn((batch, cols), generator=g, device="cuda", dtype=torch.float32)


@pytest.mark.parametrize("t,rows,cols,batches,with_argmax", [
    (DT.Q4_K, 1000, 4096, (300, 40), True),     # prefill GEMM: activation image in the scratch
    (DT.Q4_K, 1000, 4096, (300, 40), False),
    (DT.Q4_K, 2000, 2048, (7, 3), True),        # decode kernels: only the argmax keys in the scratch
    (DT.Q5_K, 1500, 4096, (8, 7), True),        # 7-8 columns: fused quantizer here, planes kernel in rlq_matmul
    (DT.Q5_K, 1500, 4096, (8, 7), False),
    (DT.Q6_K, 3000, 4096, (8, 1), True),
    (DT.Q8_0, 2000, 896, (5, 2), True),
    (DT.Q3_K, 2048, 4096, (2, 1), True),        # Q3_K one column: the class-ordered split kernel
    (DT.Q2_K, 1500, 2048, (1, 3), True)])
def test_noalloc_equals_allocating_entry_point(ctx, t, rows, cols, batches, with_argmax):
    W = weights(ctx, t, rows, cols, 31 + rows)
    for i, batch in enumerate(batches):
        say("matmul_noalloc", t, rows, cols, "batch", batch, "argmax" if with_argmax else "")
        x = inputs(100 * i + batch, batch, cols)
        y = torch.full((batch, rows), 5.0, device="cuda")
        am = torch.full((batch,), -1, dtype=torch.int32, device="cuda") if with_argmax else None
        ctx.matmul_noalloc(W, x, y, am)
        ctx.sync()
        if with_argmax:
            y_ref, am_ref = ctx.matmul_argmax(W, x)
        else:
            y_ref, am_ref = ctx.matmul(W, x), None
        ctx.sync()
        assert torch.equal(bits(y), bits(y_ref)), (batch, i)
        if with_argmax:
            assert torch.equal(am, am_ref), (batch, i)


def test_noalloc_refuses_workspace_beyond_the_scratch(ctx):
    say("matmul_noalloc, workspace beyond the static scratch")
    W = weights(ctx, DT.Q4_K, 64, 4096, 5)
    x = torch.zeros((8192, 4096), device="cuda")
    y = torch.full((8192, 64), 5.0, device="cuda")
    with pytest.raises(rlq.QuantError) as e:
        ctx.matmul_noalloc(W, x, y)
    assert e.value.name == "ScratchLimit" and e.value.b == 32 << 20 and e.value.a > e.value.b
    assert bool((y == 5.0).all())


def test_noalloc_data_errors_and_refusal(ctx):
    """A non-finite input refuses the call as rlq_matmul does (no output,
    the error at sync), and the next call works."""
    say("matmul_noalloc, data error then a clean call")
    W = weights(ctx, DT.Q4_K, 512, 2048, 6)
    x = inputs(9, 20, 2048)
    x[3, 100] = float("nan")
    y = torch.full((20, 512), 5.0, device="cuda")
    ctx.matmul_noalloc(W, x, y)
    with pytest.raises(rlq.QuantError) as e:
        ctx.sync()
    assert (e.value.name, e.value.index, e.value.b) == ("NonFiniteInput", 100, 3)
    assert bool((y == 5.0).all())
    x[3, 100] = 0.0
    ctx.matmul_noalloc(W, x, y)
    ctx.sync()
    assert torch.equal(bits(y), bits(ctx.matmul(W, x)))


@pytest.mark.parametrize("t", [DT.Q4_K, DT.Q5_K])
@pytest.mark.parametrize("batch", [7, 8])
def test_noalloc_errors_of_seven_and_eight_columns(ctx, t, batch):
    """At 7-8 Q4_K / Q5_K columns rlq_matmul quantizes every column in the
    planes kernel first, while rlq_matmul_noalloc quantizes in each decode
    workgroup's prologue: both must report the same first error (by column,
    then the reference's order inside it) and leave every output untouched."""
    W = weights(ctx, t, 768, 4096, 7)
    for case in ("nan", "scale"):
        say("matmul_noalloc errors", t, "batch", batch, case)
        x = inputs(11, batch, 4096)
        if case == "nan":
            x[5, 1000] = float("nan")
            x[6, 10] = float("inf")
        else:
            x[4, 512:768] = 1e-45  # column 4, block 2: an unrepresentable scale
            x[5, 3] = float("nan")
        got = []
        for call in (ctx.matmul_noalloc, ctx.matmul):
            y = torch.full((batch, 768), 5.0, device="cuda")
            call(W, x, y)
            with pytest.raises(rlq.QuantError) as e:
                ctx.sync()
            got.append((e.value.name, e.value.a, e.value.b))
            assert bool((y == 5.0).all()), call
        assert got[0] == got[1]
        assert got[0] == (("NonFiniteInput", 1000, 5) if case == "nan" else ("UnrepresentableScale", 2, 4))
