"""Pin the CPU oracle (oracle/rlq_oracle.c) before trusting it.

1. Every golden record the reference holds for Q8_0 / Q4_K / Q6_K / Q8_K
   (tests/golden/*.bin, copied from crates/quant/tests/fixtures) must be
   reproduced BIT-EXACTLY, as the reference's own tests demand
   (matvec_extended.rs:50-103, matvec.rs:26-63, reference.rs:20-81,
   encoders_extended.rs:27-63).
2. The reference's error-path tests, restated.
3. Checks fixed by the mathematics: closed forms, invariants, brute force in
   f64 on tiny inputs.
4. Sensitivity: plausible mistakes (swapped nibbles, dropped mins term, wrong
   Q6_K offset, wrong Q8_K rounding) made in an independent numpy dot are
   caught by the golden records, so the records do pin these parts.
"""
import numpy as np
import pytest

import oracle as O
from golden import fixtures as F


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- golden records

def test_matvec_extended_q4k_q6k_bitwise():
    recs = F.matvec_extended()
    assert len(recs) == 48
    assert sorted({r.dtype for r in recs}) == [O.Q4_K, O.Q6_K]
    for i, r in enumerate(recs):
        act = O.quantize(O.Q8_K, r.x)
        assert np.array_equal(act, r.activation), f"record {i}: activation bytes"
        y = O.matvec(r.dtype, r.weights, r.rows, r.cols, r.x)
        assert np.array_equal(bits(y), bits(r.generic)), f"record {i}: generic C"
        assert np.array_equal(bits(y), bits(r.native)), f"record {i}: GGML graph"
        stride = O.row_bytes(r.dtype, r.cols)
        for row in range(r.rows):
            d = O.dot_packed(r.dtype, r.weights[row * stride:(row + 1) * stride], r.activation, r.cols)
            assert bits(d) == bits(y[row])


def test_matvec_q8_0_bitwise_generic_and_within_native_tolerance():
    recs = F.matvec_q8_0()
    assert len(recs) == 18
    for i, r in enumerate(recs):
        y = O.matvec(r.dtype, r.weights, r.rows, r.cols, r.x)
        assert np.array_equal(bits(y), bits(r.generic)), f"record {i}"
        tol = 2e-5 * (1.0 + np.abs(r.native))  # matvec.rs:55
        assert np.all(np.abs(y - r.native) <= tol)


def test_q8k_encoder_bitwise_and_bsum_invariant():
    recs = F.q8k()
    assert len(recs) == 30
    for i, (x, expected) in enumerate(recs):
        got = O.quantize(O.Q8_K, x)
        assert np.array_equal(got, expected), f"record {i}"
        for blk in got.reshape(-1, 292):
            qs = blk[4:260].view(np.int8).astype(np.int32)
            bs = blk[260:292].view("<i2").astype(np.int32)
            assert np.array_equal(bs, qs.reshape(16, 16).sum(1))


def test_encoders_bitwise():
    recs = F.encoders()
    counts = {}
    for i, (t, x, expected) in enumerate(recs):
        got = O.quantize(t, x)
        assert np.array_equal(got, expected), f"record {i} dtype {t}"
        dest = np.full(expected.size, 0xA5, np.uint8)
        O.quantize_into(t, x, dest)
        assert np.array_equal(dest, got)
        counts[t] = counts.get(t, 0) + 1
    assert counts == {O.Q8_0: 10, O.Q4_K: 52, O.Q6_K: 52}


def test_decoders_bitwise():
    recs = F.dequant()
    assert sorted(r[0] for r in recs) == [O.Q8_0, O.Q4_K, O.Q6_K, O.Q8_K]
    for t, n, b, expected in recs:
        y = O.dequantize(t, b, n)
        same = (bits(y) == bits(expected)) | (np.isnan(y) & np.isnan(expected))
        assert same.all(), t


K_OTHER = "matvec-extended-q2k-q3k-q5k.bin"


def test_matvec_extended_q2k_q3k_q5k_bitwise():
    recs = F.matvec_extended(K_OTHER)
    assert len(recs) == 72
    assert sorted({r.dtype for r in recs}) == [O.Q2_K, O.Q3_K, O.Q5_K]
    for i, r in enumerate(recs):
        act = O.quantize(O.Q8_K, r.x)
        assert np.array_equal(act, r.activation), f"record {i}: activation bytes"
        y = O.matvec(r.dtype, r.weights, r.rows, r.cols, r.x)
        assert np.array_equal(bits(y), bits(r.generic)), f"record {i} dtype {r.dtype}: generic C"
        assert np.array_equal(bits(y), bits(r.native)), f"record {i} dtype {r.dtype}: GGML graph"


def test_encoders_q2k_q3k_q5k_bitwise():
    recs = F.encoders(("encoder-extended-q2k-q3k-q5k.bin",))
    counts = {}
    for i, (t, x, expected) in enumerate(recs):
        got = O.quantize(t, x)
        assert np.array_equal(got, expected), f"record {i} dtype {t}"
        counts[t] = counts.get(t, 0) + 1
    assert counts == {O.Q2_K: 52, O.Q3_K: 52, O.Q5_K: 52}


def test_decoders_q2k_q3k_q5k_bitwise():
    recs = F.dequant("dequant-q2k-q3k-q5k.bin")
    assert sorted(r[0] for r in recs) == [O.Q2_K, O.Q3_K, O.Q5_K]
    for t, n, b, expected in recs:
        y = O.dequantize(t, b, n)
        same = (bits(y) == bits(expected)) | (np.isnan(y) & np.isnan(expected))
        assert same.all(), t


@pytest.mark.parametrize("t", [O.Q2_K, O.Q3_K, O.Q5_K])
def test_other_k_dot_equals_f64_of_decoded_operands_and_block_sums(t):
    """The dot of encoded random rows against quantized activations equals
    the f64 dot of the decoded operands up to f32 rounding, and the block
    integers rebuild it (Q2_K, Q5_K: d*isum - dmin*imin; Q3_K: d*isum)."""
    rng = np.random.default_rng(17)
    nb = 3
    n = 256 * nb
    w = O.quantize(t, rng.standard_normal(n).astype(np.float32) * 0.05)
    x = rng.standard_normal(n).astype(np.float32)
    act = O.quantize(O.Q8_K, x)
    got = float(O.dot_packed(t, w, act, n))
    wf = O.dequantize(t, w, n).astype(np.float64)
    af = O.dequantize(O.Q8_K, act, n).astype(np.float64)
    assert abs(got - float(np.dot(wf, af))) <= 1e-5 * float(np.dot(np.abs(wf), np.abs(af)))
    isum, imin = O.block_sums(t, w, act, nb)
    ws, as_ = w.reshape(nb, -1), act.reshape(nb, -1)
    tot = 0.0
    for k in range(nb):
        da = np.float64(as_[k, :4].view(np.float32)[0])
        if t == O.Q2_K:
            d, dm = (np.float64(v) for v in ws[k, 80:84].view(np.float16))
        elif t == O.Q3_K:
            d, dm = np.float64(ws[k, 108:110].view(np.float16)[0]), 0.0
        else:
            d, dm = (np.float64(v) for v in ws[k, 0:4].view(np.float16))
        tot += d * da * isum[k] - dm * da * imin[k]
    assert abs(got - tot) <= 1e-5 * float(np.dot(np.abs(wf), np.abs(af)))


# ---------------------------------------------------------------- error paths

def test_q8k_preflight_and_canonical_zero_blocks():
    """matvec_extended.rs:143-170"""
    out = np.full(584, 0xA5, np.uint8)
    x = np.ones(512, np.float32)
    x[256:] = np.frombuffer(np.uint32(1).tobytes(), np.float32)[0]
    with pytest.raises(O.OracleError) as e:
        O.quantize_into(O.Q8_K, x, out)
    assert (e.value.name, e.value.a) == ("UnrepresentableScale", 1)
    assert (out == 0xA5).all()
    x[300] = np.inf
    with pytest.raises(O.OracleError) as e:
        O.quantize_into(O.Q8_K, x, out)
    assert (e.value.name, e.value.a) == ("NonFiniteInput", 300)
    assert (out == 0xA5).all()
    O.quantize_into(O.Q8_K, np.full(512, -0.0, np.float32), out)
    assert (out == 0).all()
    with pytest.raises(O.OracleError) as e:
        O.quantize(O.Q8_K, np.ones(255, np.float32))
    assert e.value.name == "NonMultiple"
    with pytest.raises(O.OracleError) as e:
        O.quantize_into(O.Q8_K, np.ones(256, np.float32), np.zeros(291, np.uint8))
    assert e.value.name == "InvalidLength"


@pytest.mark.parametrize("t", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_matvec_rejects_malformed_dimensions(t):
    """matvec_extended.rs:172-230 for the path's weight types."""
    n = O.BLOCK[t]
    x = np.ones(n, np.float32)
    w = np.zeros(O.TYPE_SIZE[t], np.uint8)
    act = O.quantize(O.matvec_activation_dtype(t), x)
    for args, name in [((t, w[:-1], 1, n, x), "InvalidLength"),
                       ((t, w, 1, n, x[:-1]), "InvalidVectorLength"),
                       ((t, w, 0, n, x), "InvalidMatrixShape"),
                       ((t, w, 1, n - 1, x[:-1]), "NonMultiple"),
                       ((t, w, 2 ** 64 - 1, n, x), "SizeOverflow")]:
        with pytest.raises(O.OracleError) as e:
            O.matvec(*args)
        assert e.value.name == name
    with pytest.raises(O.OracleError):
        O.dot_packed(t, w, act[:-1], n)
    with pytest.raises(O.OracleError):
        O.dot_packed(t, w, act, n - 1)
    bad = x.copy()
    bad[n - 1] = np.nan
    with pytest.raises(O.OracleError) as e:
        O.matvec(t, w, 1, n, bad)
    assert (e.value.name, e.value.a) == ("NonFiniteInput", n - 1)


def test_activation_dtype_capabilities():
    """matvec_extended.rs:232-246 and matvec.rs:91-94"""
    excluded = {9, 15, 24, 25, 26, 27, 28}
    for t in [0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26,
              27, 28, 29, 30, 34, 35, 39, 40, 41, 42, 43]:
        try:
            O.matvec_activation_dtype(t)
            ok = True
        except O.OracleError as e:
            assert e.name == "UnsupportedMatVec"
            ok = False
        assert ok == (t not in excluded), t
    assert O.matvec_activation_dtype(O.Q4_K) == O.Q8_K
    assert O.matvec_activation_dtype(O.Q6_K) == O.Q8_K
    assert O.matvec_activation_dtype(O.Q8_0) == O.Q8_0
    for bad in [4, 5, 31, 44, 2 ** 32 - 1]:
        with pytest.raises(O.OracleError) as e:
            O.matvec_activation_dtype(bad)
        assert e.value.name == "InvalidType"


def test_row_bytes():
    assert O.row_bytes(O.Q4_K, 4096) == 2304
    assert O.row_bytes(O.Q6_K, 4096) == 3360
    assert O.row_bytes(O.Q8_0, 896) == 952
    assert O.row_bytes(O.Q8_K, 4096) == 4672
    with pytest.raises(O.OracleError) as e:
        O.row_bytes(O.Q6_K, 896)  # the Qwen vocab width has no Q6_K encoding
    assert (e.value.name, e.value.a, e.value.b) == ("NonMultiple", 896, 256)


@pytest.mark.filterwarnings("ignore:overflow encountered in cast")
def test_half_conversions_ieee():
    """reference.rs:119-140"""
    assert O.f16_to_f32(1) == 2.0 ** -24
    assert O.f16_to_f32(0x3FF) == 1023 * 2.0 ** -24
    assert O.f16_to_f32(0x400) == 2.0 ** -14
    assert O.f32_to_f16(65504.0) == 0x7BFF
    assert O.f32_to_f16(65520.0) == 0x7C00
    assert O.f32_to_f16(1.0 + 2.0 ** -11) == 0x3C00
    assert O.f32_to_f16(1.0 + 3 * 2.0 ** -11) == 0x3C02
    assert O.f32_to_f16(2.0 ** -25) == 0
    # numpy's float16 is IEEE binary16 with ties-to-even: an independent check
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 2000),
                           np.float32([0.0, -0.0, 6.1e-5, 5.96e-8, 2.98e-8, 65519.0, 1e6])])
    for v in vals.astype(np.float32):
        assert O.f32_to_f16(v) == np.float32(v).astype(np.float16).view(np.uint16), v
    for h in range(0, 65536, 7):
        f = np.uint16(h).view(np.float16)
        if not np.isnan(f):
            assert O.f16_to_f32(h) == np.float32(f)


def test_argmax_first_strict_maximum():
    assert O.argmax(np.float32([1, 3, 3, 2])) == 1
    assert O.argmax(np.float32([-np.inf, -np.inf])) == 0
    assert O.argmax(np.float32([0.0, -0.0, 0.0])) == 0
    assert O.argmax(np.float32([np.nan, 5.0])) == 0
    assert O.argmax(np.float32([1.0, np.nan, 5.0])) == 2


# ---------------------------------------------------------------- mathematics

def _rand_q4k_row(rng, nb):
    """Random but valid Q4_K bytes: finite f16 scales, arbitrary nibbles."""
    b = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    d = (rng.random(nb) * 0.01).astype(np.float16).view(np.uint8).reshape(nb, 2)
    m = (rng.random(nb) * 0.01).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 0:2], b[:, 2:4] = d, m
    return b.reshape(-1)


def _rand_q6k_row(rng, nb):
    b = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    b[:, 208:210] = (rng.random(nb) * 0.01).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


@pytest.mark.parametrize("t", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_dot_equals_f64_brute_force_of_decoded_operands(t):
    """The dot is the exact sum of decoded weights times decoded activation
    up to f32 rounding of the scales: compare to f64 on tiny inputs."""
    rng = np.random.default_rng(7)
    for nb in (1, 2, 3):
        n = nb * O.BLOCK[t]
        if t == O.Q4_K:
            w = _rand_q4k_row(rng, nb)
        elif t == O.Q6_K:
            w = _rand_q6k_row(rng, nb)
        else:
            w = O.quantize(O.Q8_0, rng.standard_normal(n).astype(np.float32))
        x = rng.standard_normal(n).astype(np.float32)
        at = O.matvec_activation_dtype(t)
        act = O.quantize(at, x)
        got = float(O.dot_packed(t, w, act, n))
        wf = O.dequantize(t, w, n).astype(np.float64)
        af = O.dequantize(at, act, n).astype(np.float64)
        ref = float(np.dot(wf, af))
        scale = float(np.dot(np.abs(wf), np.abs(af)))
        assert abs(got - ref) <= 1e-5 * scale + 1e-30, (t, nb, got, ref)


def test_zero_weights_and_zero_activation():
    rng = np.random.default_rng(3)
    for t in (O.Q4_K, O.Q6_K):
        x = rng.standard_normal(512).astype(np.float32)
        assert np.all(O.matvec(t, np.zeros(2 * O.row_bytes(t, 512), np.uint8), 2, 512, x) == 0)
        w = _rand_q4k_row(rng, 2) if t == O.Q4_K else _rand_q6k_row(rng, 2)
        y = O.matvec(t, w, 1, 512, np.zeros(512, np.float32))
        assert np.all(y == 0)
    assert np.all(O.quantize(O.Q8_K, np.zeros(512, np.float32)) == 0)


def test_q8k_quantizer_properties():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32) * 3
    a = O.quantize(O.Q8_K, x).reshape(-1, 292)
    for k, blk in enumerate(a):
        qs = blk[4:260].view(np.int8).astype(np.int32)
        d = blk[0:4].view(np.float32)[0]
        xb = x[k * 256:(k + 1) * 256]
        i = int(np.argmax(np.abs(xb)))  # first index of largest |x|
        assert qs[i] == -127  # inverse = -127 / max sends the max to -127
        assert np.all(np.abs(qs) <= 127)
        # reconstruction within half a step
        assert np.all(np.abs(d * qs - xb) <= abs(d) * 0.5 * (1 + 1e-6))


def test_q8k_linearity_in_activation_scale():
    """Scaling x by a power of two scales d exactly and leaves q unchanged."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal(1024).astype(np.float32)
    a1 = O.quantize(O.Q8_K, x).reshape(-1, 292)
    a2 = O.quantize(O.Q8_K, x * np.float32(8)).reshape(-1, 292)
    assert np.array_equal(a1[:, 4:], a2[:, 4:])
    assert np.array_equal(a1[:, :4].view(np.float32) * 8, a2[:, :4].view(np.float32))
    w = _rand_q4k_row(rng, 4)
    y1 = O.matvec(O.Q4_K, w, 1, 1024, x)[0]
    y2 = O.matvec(O.Q4_K, w, 1, 1024, x * np.float32(8))[0]
    assert y2 == y1 * 8


def test_block_sums_add_up_to_the_dot():
    """isum/imin are the dot's integer parts: d*isum - dmin*imin summed over
    blocks (in f64) reproduces the dot up to f32 rounding."""
    rng = np.random.default_rng(9)
    for t in (O.Q4_K, O.Q6_K, O.Q8_0):
        nb = 6
        n = nb * O.BLOCK[t]
        w = _rand_q4k_row(rng, nb) if t == O.Q4_K else (
            _rand_q6k_row(rng, nb) if t == O.Q6_K else O.quantize(O.Q8_0, rng.standard_normal(n)))
        x = rng.standard_normal(n).astype(np.float32)
        at = O.matvec_activation_dtype(t)
        act = O.quantize(at, x)
        isum, imin = O.block_sums(t, w, act, nb)
        ws, as_ = w.reshape(nb, -1), act.reshape(nb, -1)
        tot = 0.0
        for k in range(nb):
            if t == O.Q8_0:
                d = np.float64(ws[k, :2].view(np.float16)[0]) * np.float64(as_[k, :2].view(np.float16)[0])
                tot += d * isum[k]
            else:
                ya = np.float64(as_[k, :4].view(np.float32)[0])
                off = 0 if t == O.Q4_K else 208
                d = np.float64(ws[k, off:off + 2].view(np.float16)[0]) * ya
                dm = np.float64(ws[k, 2:4].view(np.float16)[0]) * ya if t == O.Q4_K else 0.0
                tot += d * isum[k] - dm * imin[k]
        got = float(O.dot_packed(t, w, act, n))
        assert abs(got - tot) <= 1e-5 * max(1.0, abs(tot)), t


# ---------------------------------------------------------------- sensitivity

def _np_q4k_dot(w, act, nb, swap_nibbles=False, drop_mins=False):
    """Independent numpy dot (f64 accumulation) with optional planted mistakes."""
    w, act = w.reshape(nb, 144), act.reshape(nb, 292)
    tot = 0.0
    for k in range(nb):
        p = w[k, 4:16].astype(np.int32)
        sc = np.zeros(8, np.int32)
        mn = np.zeros(8, np.int32)
        for j in range(8):
            if j < 4:
                sc[j], mn[j] = p[j] & 63, p[j + 4] & 63
            else:
                sc[j] = (p[j + 4] & 15) | ((p[j - 4] >> 6) << 4)
                mn[j] = (p[j + 4] >> 4) | ((p[j] >> 6) << 4)
        qs = w[k, 16:144].reshape(4, 32).astype(np.int32)
        lo, hi = qs & 15, qs >> 4
        if swap_nibbles:
            lo, hi = hi, lo
        q = np.stack([lo, hi], 1).reshape(8, 32)
        a = act[k, 4:260].view(np.int8).astype(np.int32).reshape(8, 32)
        bs = act[k, 260:292].view("<i2").astype(np.int32).reshape(8, 2).sum(1)
        ya = float(act[k, :4].view(np.float32)[0])
        d = float(w[k, 0:2].view(np.float16)[0]) * ya
        dm = float(w[k, 2:4].view(np.float16)[0]) * ya
        tot += d * float((sc[:, None] * q * a).sum()) - (0.0 if drop_mins else dm * float((mn * bs).sum()))
    return tot


def _np_q6k_dot(w, act, nb, offset=32):
    w, act = w.reshape(nb, 210), act.reshape(nb, 292)
    tot = 0.0
    for k in range(nb):
        b = w[k].astype(np.int32)
        j = np.arange(256)
        g, s, p = j // 128, (j % 128) // 32, j % 32
        low = (b[g * 64 + (s % 2) * 32 + p] >> (4 * (s // 2))) & 15
        high = (b[128 + g * 32 + p] >> (2 * s)) & 3
        q = (low | (high << 4)) - offset
        sc = w[k, 192:208].view(np.int8).astype(np.int32)[j // 16]
        a = act[k, 4:260].view(np.int8).astype(np.int32)
        d = float(w[k, 208:210].view(np.float16)[0]) * float(act[k, :4].view(np.float32)[0])
        tot += d * float((sc * q * a).sum())
    return tot


def test_golden_records_catch_planted_mistakes():
    recs = F.matvec_extended()
    caught = {"swap": 0, "mins": 0, "offset": 0}
    clean_ok = 0
    for r in recs:
        stride = r.weights.size // r.rows
        nb = r.cols // 256
        for row in range(r.rows):
            w = r.weights[row * stride:(row + 1) * stride]
            e = float(r.generic[row])
            tol = 1e-5 * max(1.0, abs(e))
            if r.dtype == O.Q4_K:
                clean_ok += abs(_np_q4k_dot(w, r.activation, nb) - e) <= tol
                caught["swap"] += abs(_np_q4k_dot(w, r.activation, nb, swap_nibbles=True) - e) > tol
                caught["mins"] += abs(_np_q4k_dot(w, r.activation, nb, drop_mins=True) - e) > tol
            else:
                clean_ok += abs(_np_q6k_dot(w, r.activation, nb) - e) <= tol
                caught["offset"] += abs(_np_q6k_dot(w, r.activation, nb, offset=31) - e) > tol
    # the independent numpy dot agrees wherever the record is not degenerate
    assert clean_ok >= 0.9 * sum(r.rows for r in recs)
    assert all(v > 0 for v in caught.values()), caught


def test_q8k_records_catch_wrong_rounding_and_tie_break():
    """Rounding half away from zero instead of ties-to-even, or taking the
    last (not first) largest |x|, changes some golden Q8_K bytes."""
    recs = F.q8k()
    diff_round = diff_tie = 0
    for x, expected in recs:
        for k, xb in enumerate(x.reshape(-1, 256)):
            e = expected[k * 292:(k + 1) * 292]
            amax = np.abs(xb).max()
            if amax == 0:
                continue
            first = xb[int(np.argmax(np.abs(xb)))]
            last = xb[255 - int(np.argmax(np.abs(xb[::-1])))]
            inv = np.float32(-127.0) / np.float32(first)
            v = (inv * xb).astype(np.float32)
            away = np.minimum(np.sign(v) * np.floor(np.abs(v) + 0.5), 127).astype(np.int8)
            diff_round += not np.array_equal(away.view(np.uint8), e[4:260])
            inv2 = np.float32(-127.0) / np.float32(last)
            q2 = np.minimum(np.rint((inv2 * xb).astype(np.float32)), 127).astype(np.int8)
            diff_tie += not np.array_equal(q2.view(np.uint8), e[4:260])
    assert diff_round > 0 and diff_tie > 0


# ---------------------------------------------------------------- order tolerance

def _exact_f64(t, w_row, act, nb):
    """The dot with exact integer block sums and f32 block scales, summed in
    f64 (no f32 rounding after the scales)."""
    isum, imin = O.block_sums(t, w_row, act, nb)
    ws, as_ = w_row.reshape(nb, -1), act.reshape(nb, -1)
    tot = 0.0
    for k in range(nb):
        if t == O.Q8_0:
            d = np.float32(np.float32(ws[k, :2].view(np.float16)[0]) * np.float32(as_[k, :2].view(np.float16)[0]))
            tot += float(d) * int(isum[k])
        else:
            ya = np.float32(as_[k, :4].view(np.float32)[0])
            off = 0 if t == O.Q4_K else 208
            d = np.float32(np.float32(ws[k, off:off + 2].view(np.float16)[0]) * ya)
            dm = np.float32(np.float32(ws[k, 2:4].view(np.float16)[0]) * ya) if t == O.Q4_K else np.float32(0)
            tot += float(d) * int(isum[k]) - float(dm) * int(imin[k])
    return tot


def test_order_tolerance_bounds_the_reference_rounding():
    """The reference's own f32 result (golden generic C output) lies within
    half of order_tolerance of the exact value, for every golden row,
    including the records built for cancellation; and the bound is never
    below the exact magnitude's rounding."""
    for r in F.matvec_extended():
        nb = r.cols // 256
        tol = O.order_tolerance(r.dtype, r.weights, r.rows, r.activation, nb)
        stride = r.weights.size // r.rows
        for row in range(r.rows):
            exact = _exact_f64(r.dtype, r.weights[row * stride:(row + 1) * stride], r.activation, nb)
            assert abs(float(r.generic[row]) - exact) <= tol[row] / 2, (r.dtype, r.cols, row)
            assert tol[row] >= 2 * 2.0 ** -24 * abs(exact)
    for r in F.matvec_q8_0():
        nb = r.cols // 32
        act = O.quantize(O.Q8_0, r.x)
        tol = O.order_tolerance(r.dtype, r.weights, r.rows, act, nb)
        stride = r.weights.size // r.rows
        for row in range(r.rows):
            exact = _exact_f64(r.dtype, r.weights[row * stride:(row + 1) * stride], act, nb)
            assert abs(float(r.generic[row]) - exact) <= tol[row] / 2, (r.cols, row)


def test_order_tolerance_rejects_a_dropped_block():
    """Dropping one block's term moves a random row's dot far outside the
    order tolerance: the bound is tight enough to catch a lost block."""
    rng = np.random.default_rng(31)
    for t in (O.Q4_K, O.Q6_K, O.Q8_0):
        nb = 16 if t != O.Q8_0 else 28
        n = nb * O.BLOCK[t]
        w = O.quantize(t, (rng.standard_normal(n) * 0.02).astype(np.float32))
        act = O.quantize(O.matvec_activation_dtype(t), rng.standard_normal(n).astype(np.float32))
        full = _exact_f64(t, w, act, nb)
        bs = O.row_bytes(t, O.BLOCK[t])
        dropped = _exact_f64(t, w[:-bs], act[:-O.row_bytes(O.matvec_activation_dtype(t), O.BLOCK[t])], nb - 1)
        tol = O.order_tolerance(t, w, 1, act, nb)[0]
        assert abs(full - dropped) > 20 * tol, t
