"""Pins for the oracle's GGML MUL_MAT (broadcast) and MUL_MAT_ID restatements
(oracle/__init__.py mul_mat, mul_mat_id; crates/tensor/src/cpu_extra.rs:756-873,
crates/tensor/src/cpu_index.rs:169-236).

The reference's graph fixtures (tests/golden/mul-mat-broadcast.bin,
mul-mat-id.bin, copied from crates/tensor/tests/fixtures) hold exact native
output bytes for every weight type on the path, with F32 and packed
activation right-hand sides, strided inputs and -1 expert ids.  The error
order and payloads follow the reference's checks.
"""
import numpy as np
import pytest

import oracle as O
from golden import fixtures as F


def case_inputs(c):
    a, b = c.inputs[0], c.inputs[1]
    xd = b.dtype
    xb = b.contiguous()
    x = xb.view(np.float32) if xd == O.F32 else xb
    return a, b, xd, x


def ids_of(c):
    t = c.inputs[2]
    return np.frombuffer(t.contiguous().tobytes(), np.int32).reshape(t.shape[1], t.shape[0])


def test_mul_mat_broadcast_golden_bitwise():
    cases = F.ggml_cases("mul-mat-broadcast.bin")
    assert sorted({c.inputs[0].dtype for c in cases}) == [8, 10, 11, 12, 13, 14]
    for c in cases:
        a, b, xd, x = case_inputs(c)
        K, rows, wn2, wn3 = a.shape
        assert (b.shape[2] // wn2, b.shape[3] // wn3) == (2, 2)  # both batch dimensions broadcast
        y = O.mul_mat(a.dtype, a.contiguous(), rows, K, wn2, wn3, xd, x, b.shape[1], b.shape[2], b.shape[3])
        want = np.frombuffer(c.expected.data, np.float32)
        assert np.array_equal(y.reshape(-1).view(np.uint32), want.view(np.uint32)), c.name


def test_mul_mat_id_golden_bitwise():
    cases = F.ggml_cases("mul-mat-id.bin")
    assert sorted({c.inputs[0].dtype for c in cases}) == [8, 10, 11, 12, 13, 14]
    for c in cases:
        a, b, xd, x = case_inputs(c)
        ids = ids_of(c)
        assert (ids == -1).any() and ids.shape[1] % b.shape[1] == 0 and ids.shape[1] > b.shape[1]
        y = O.mul_mat_id(a.dtype, a.contiguous(), a.shape[1], a.shape[0], a.shape[2], xd, x, b.shape[1],
                         b.shape[2], ids)
        want = np.frombuffer(c.expected.data, np.float32)
        assert np.array_equal(y.reshape(-1).view(np.uint32), want.view(np.uint32)), c.name


def test_mul_mat_id_planted_mistakes_fail():
    """Selecting the right-hand column by expert instead of by slot, or
    leaving -1 slots to expert 0, changes the golden outputs."""
    c = next(c for c in F.ggml_cases("mul-mat-id.bin") if c.inputs[0].dtype == 12 and c.inputs[1].dtype == 0)
    a, b, xd, x = case_inputs(c)
    ids = ids_of(c)
    want = np.frombuffer(c.expected.data, np.float32).reshape(ids.shape[0], ids.shape[1], a.shape[1])
    w, K, rows = a.contiguous(), a.shape[0], a.shape[1]
    rb = O.row_bytes(12, K)
    xs = x.reshape(ids.shape[0], b.shape[1], K)
    wrong_col = np.zeros_like(want)
    for t in range(ids.shape[0]):
        for s in range(ids.shape[1]):
            e = ids[t, s]
            if e >= 0:
                wrong_col[t, s] = O.matvec(12, w[e * rows * rb:(e + 1) * rows * rb], rows, K, xs[t, e % b.shape[1]])
    assert not np.array_equal(wrong_col, want)
    zero_to_0 = O.mul_mat_id(12, w, rows, K, a.shape[2], xd, x, b.shape[1], b.shape[2], np.maximum(ids, 0))
    assert not np.array_equal(zero_to_0, want)


def _w(t, rows, cols, mats, seed):
    x = np.random.default_rng(seed).standard_normal(rows * cols * mats).astype(np.float32) * np.float32(0.02)
    return O.quantize(t, x)


def test_error_order_and_payloads():
    w = _w(O.Q4_K, 4, 256, 3, 1)
    x = np.ones((2, 2, 256), np.float32)
    ids = np.array([[0, 1], [2, -1]], np.int32)
    # Shape: 3 slots over 2 right-hand columns; a batch dimension that does
    # not repeat the weights' (4 % 3)
    with pytest.raises(O.OracleError) as e:
        O.mul_mat_id(O.Q4_K, w, 4, 256, 3, O.F32, x, 2, 2, np.zeros((2, 3), np.int32))
    assert e.value.name == "Shape"
    with pytest.raises(O.OracleError) as e:
        O.mul_mat(O.Q4_K, w, 4, 256, 3, 1, O.F32, np.ones((1, 4, 1, 256), np.float32), 1, 4, 1)
    assert e.value.name == "Shape"
    # Unsupported right-hand type (F16 is not the Q8_K activation type)
    with pytest.raises(O.OracleError) as e:
        O.mul_mat_id(O.Q4_K, w, 4, 256, 3, 1, x, 2, 2, ids)
    assert e.value.name == "Unsupported"
    # Bounds before any quantization error; its index is the flat position
    xn = x.copy()
    xn[0, 1, 5] = np.nan
    with pytest.raises(O.OracleError) as e:
        O.mul_mat_id(O.Q4_K, w, 4, 256, 3, O.F32, xn, 2, 2, np.array([[0, 1], [3, -2]], np.int32))
    assert (e.value.name, e.value.a) == ("Bounds", 2)
    # then the first non-finite value of the first bad column (b = column)
    with pytest.raises(O.OracleError) as e:
        O.mul_mat_id(O.Q4_K, w, 4, 256, 3, O.F32, xn, 2, 2, ids)
    assert (e.value.name, e.value.a, e.value.b) == ("NonFiniteInput", 5, 1)
    # a column no expert reads is still quantized, and rejected
    with pytest.raises(O.OracleError) as e:
        O.mul_mat_id(O.Q4_K, w, 4, 256, 3, O.F32, xn, 2, 2, np.array([[-1, -1], [0, 0]], np.int32))
    assert (e.value.name, e.value.b) == ("NonFiniteInput", 1)
    # an empty output returns before any quantization
    assert O.mul_mat_id(O.Q4_K, w, 4, 256, 3, O.F32, xn, 2, 0, np.zeros((0, 2), np.int32)).size == 0


def test_broadcast_equals_matvec_per_slice():
    """Closed form: every output slice is the plain matvec of its source
    matrix (i2 / r2, i3 / r3) on its columns."""
    rows, cols, wn2, wn3, n2, n3, ncols = 5, 512, 2, 1, 4, 3, 3
    w = _w(O.Q6_K, rows, cols, wn2 * wn3, 2)
    x = np.random.default_rng(3).standard_normal((n3, n2, ncols, cols)).astype(np.float32)
    y = O.mul_mat(O.Q6_K, w, rows, cols, wn2, wn3, O.F32, x, ncols, n2, n3)
    mb = rows * O.row_bytes(O.Q6_K, cols)
    for i3 in range(n3):
        for i2 in range(n2):
            m = (i3 // (n3 // wn3)) * wn2 + i2 // (n2 // wn2)
            want = O.matmul(O.Q6_K, w[m * mb:(m + 1) * mb], rows, cols, x[i3, i2])
            assert np.array_equal(y[i3, i2], want)
