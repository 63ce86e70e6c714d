"""Pins for the CPU restatement of the Llama decode step (oracle/rlq_oracle_llama.c).

The reference holds no fixtures for the model-level path, so each function is
pinned by what the mathematics fixes: closed forms, invariants and special
cases chosen so that a plausible slip (a dropped term, a wrong sign or index,
a transposed operand, a missing residual) fails one of them.
"""
import math

import numpy as np
import pytest

import oracle as O


# ---- SSE2 exponential (crates/quant/src/cpu_math.rs:94-123) -------------------

def test_sse2_exp_special_values():
    assert O.sse2_exp(0.0) == np.float32(1.0)
    assert O.sse2_exp(-np.inf) == 0.0
    assert O.sse2_exp(-200.0) == 0.0  # |n| > 192: high * high underflows
    assert np.isinf(O.sse2_exp(200.0))


def test_sse2_exp_relative_error_and_monotonicity():
    xs = np.linspace(-87.0, 88.0, 20001, dtype=np.float32)
    got = np.array([O.sse2_exp(x) for x in xs], dtype=np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got / want - 1.0)) < 4e-7
    assert np.all(np.diff(got) >= 0)


def test_sse2_exp_subnormal_branch():
    # 126 < |n| <= 192: the result is scaled through the subnormal range
    for x in (-88.0, -90.0, -95.5, -100.0, -103.0):
        want = math.exp(x)
        got = float(O.sse2_exp(x))
        assert abs(got - want) <= 2.0 ** -149 + 4e-7 * want, x


# ---- SiLU, softmax ------------------------------------------------------------

def test_silu_closed_form():
    v = np.array([0.0, 1.0, -1.0, 5.0, -20.0, 0.125, 30.0, -3.5], np.float32)
    got = O.silu(v).astype(np.float64)
    want = v / (1.0 + np.exp(-v.astype(np.float64)))
    assert got[0] == 0.0
    assert np.allclose(got, want, rtol=1e-6, atol=1e-30)


def test_silu_tail_uses_scalar_exp():
    # 6 values: the last two (the tail past the four-value prefix) take libm expf
    v = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5], np.float32)
    got = O.silu(v)
    tail = v[4:] / (np.float32(1.0) + np.exp(-v[4:]).astype(np.float32))
    assert np.allclose(got[4:], tail, rtol=2e-7)


def test_softmax_sums_to_one_and_masks_padding():
    rng = np.random.default_rng(1)
    v = rng.normal(0, 3, 300).astype(np.float32)
    padded = np.concatenate([v, np.full(212, -np.inf, np.float32)])
    p = O.softmax(padded)
    assert np.all(p[300:] == 0.0)
    assert abs(float(np.sum(p.astype(np.float64))) - 1.0) < 1e-6
    want = np.exp(v.astype(np.float64) - v.max())
    want /= want.sum()
    assert np.allclose(p[:300], want, rtol=2e-6, atol=1e-12)


def test_softmax_single_and_uniform():
    assert O.softmax(np.array([3.0], np.float32))[0] == 1.0
    p = O.softmax(np.full(8, 0.7, np.float32))
    assert np.all(p == np.float32(0.125))


def test_softmax_rejects_nan_and_all_masked():
    with pytest.raises(O.OracleError):
        O.softmax(np.array([1.0, np.nan], np.float32))
    with pytest.raises(O.OracleError):
        O.softmax(np.full(4, -np.inf, np.float32))


# ---- RMSNorm (math.rs:214-228) ------------------------------------------------

def test_rms_norm_closed_form():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, 512).astype(np.float32)
    w = rng.normal(1, 0.1, 512).astype(np.float32)
    got = O.rms_norm(x, w, 1e-5).astype(np.float64)
    ms = np.mean(x.astype(np.float64) ** 2)
    want = x / np.sqrt(ms + 1e-5) * w
    assert np.allclose(got, want, rtol=1e-6)


def test_rms_norm_constant_row():
    # x = c everywhere: mean square c^2, so out = c / sqrt(c^2 + eps) * w
    x = np.full(256, 2.0, np.float32)
    got = O.rms_norm(x, np.ones(256, np.float32), 1e-5)
    assert np.allclose(got, 2.0 / math.sqrt(4.0 + 1e-5), rtol=1e-7)


# ---- RoPE (math.rs:322-334) ---------------------------------------------------

def test_rope_position_zero_is_identity():
    v = np.random.default_rng(3).normal(0, 1, 256).astype(np.float32)
    assert np.array_equal(O.rope(v, 64, 0, 10000.0), v)


def test_rope_rotates_pairs():
    rng = np.random.default_rng(4)
    v = rng.normal(0, 1, 128).astype(np.float32)
    pos, base, hd = 37, 10000.0, 64
    got = O.rope(v, hd, pos, base).astype(np.float64).reshape(2, hd // 2, 2)
    x = v.astype(np.float64).reshape(2, hd // 2, 2)
    theta = pos * base ** (-2.0 * np.arange(hd // 2) / hd)
    c, s = np.cos(theta), np.sin(theta)
    want = np.stack([x[..., 0] * c - x[..., 1] * s, x[..., 0] * s + x[..., 1] * c], axis=-1)
    assert np.allclose(got, want, atol=2e-5)
    # norms of the pairs are kept
    assert np.allclose(np.hypot(got[..., 0], got[..., 1]), np.hypot(x[..., 0], x[..., 1]), rtol=1e-6)


def test_rope_table_matches_rope():
    hd, pos, base = 64, 123, 500000.0
    t = O.rope_table(hd, pos, base)
    v = np.random.default_rng(5).normal(0, 1, hd).astype(np.float32)
    x, y = v[0::2], v[1::2]
    s, c = t[0::2], t[1::2]
    manual = np.empty_like(v)
    manual[0::2] = x * c - y * s
    manual[1::2] = x * s + y * c
    assert np.array_equal(manual, O.rope(v, hd, pos, base))


# ---- attention (math.rs:427-497) ----------------------------------------------

def test_attention_single_row_returns_value():
    rng = np.random.default_rng(6)
    heads, kvh, hd = 4, 2, 32
    q = rng.normal(0, 1, heads * hd).astype(np.float32)
    k = rng.normal(0, 1, kvh * hd).astype(np.float32)
    v = rng.normal(0, 1, kvh * hd).astype(np.float32)
    out = O.attention(q, k, v, 1, heads, kvh, hd, 0.125).reshape(heads, hd)
    for h in range(heads):  # grouped heads share kv head h // 2
        assert np.array_equal(out[h], v.reshape(kvh, hd)[h // 2])


def test_attention_zero_query_averages_values():
    rng = np.random.default_rng(7)
    heads, kvh, hd, n = 2, 1, 16, 9
    q = np.zeros(heads * hd, np.float32)
    k = rng.normal(0, 1, (n, kvh * hd)).astype(np.float32)
    v = rng.normal(0, 1, (n, kvh * hd)).astype(np.float32)
    out = O.attention(q, k, v, n, heads, kvh, hd, 0.25).reshape(heads, hd)
    assert np.allclose(out[0], v.astype(np.float64).mean(axis=0), rtol=1e-6, atol=1e-7)
    assert np.array_equal(out[0], out[1])


def test_attention_against_dense_softmax():
    rng = np.random.default_rng(8)
    heads, kvh, hd, n = 8, 2, 64, 270  # crosses the 256-column padding
    q = rng.normal(0, 1, heads * hd).astype(np.float32)
    k = rng.normal(0, 1, (n, kvh * hd)).astype(np.float32)
    v = rng.normal(0, 1, (n, kvh * hd)).astype(np.float32)
    scale = np.float32(1.0 / math.sqrt(hd))
    out = O.attention(q, k, v, n, heads, kvh, hd, scale).reshape(heads, hd).astype(np.float64)
    for h in range(heads):
        g = h // (heads // kvh)
        kk = k[:, g * hd:(g + 1) * hd].astype(np.float64)
        vv = v[:, g * hd:(g + 1) * hd].astype(np.float64)
        s = kk @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(out[h], p @ vv, rtol=1e-5, atol=1e-6)


# ---- the decode step (llama.rs:222-392) ----------------------------------------

from llama_fixture import make_config, make_tensors  # noqa: E402


def test_step_without_layers_is_norm_then_output():
    cfg = make_config(n_layers=0)
    t = make_tensors(cfg, seed=11)
    m = O.LlamaOracle(cfg, t)
    h0 = m.embedding(5)
    h, logits = m.step(h0, 0)
    assert np.array_equal(h, h0)
    norm = O.rms_norm(h0, t["output_norm"], cfg.rms_epsilon)
    assert np.array_equal(logits, O.matvec(cfg.output_type, t["output"], cfg.vocabulary, cfg.width, norm))


def test_zero_matrices_leave_the_residual_stream_unchanged():
    # zero Q/K/V/O and zero down: attention and FFN add exactly 0 to hidden
    cfg = make_config(n_layers=2)
    t = make_tensors(cfg, seed=12, zero_layers=True)
    m = O.LlamaOracle(cfg, t)
    h0 = m.embedding(9)
    h, _ = m.step(h0, 0)
    assert np.array_equal(h, h0)
    h, _ = m.step(h0, 1)
    assert np.array_equal(h, h0)


def test_step_appends_roped_keys_and_values():
    cfg = make_config(n_layers=1)
    t = make_tensors(cfg, seed=13)
    m = O.LlamaOracle(cfg, t)
    h0 = m.embedding(3)
    m.step(h0, 4)
    L = t["layers"][0]
    norm = O.rms_norm(h0, L["attention_norm"], cfg.rms_epsilon)
    k = O.matvec(cfg.weight_type, L["key"], cfg.kv_width, cfg.width, norm)
    v = O.matvec(cfg.weight_type, L["value"], cfg.kv_width, cfg.width, norm)
    assert np.array_equal(m.k_cache[0, 0], O.rope(k, cfg.head_dim, 4, cfg.rope_base))
    assert np.array_equal(m.v_cache[0, 0], v)
    assert m.cached == 1


def test_one_layer_step_by_parts():
    """The whole layer rebuilt from the pinned parts above must equal the step."""
    cfg = make_config(n_layers=1)
    t = make_tensors(cfg, seed=14)
    m = O.LlamaOracle(cfg, t)
    L = t["layers"][0]
    W, kvw, hd, F, wt = cfg.width, cfg.kv_width, cfg.head_dim, cfg.feed_forward, cfg.weight_type
    h0 = m.embedding(7)
    m.step(m.embedding(2), 0)  # one cached row first
    h, logits = m.step(h0, 1)
    norm = O.rms_norm(h0, L["attention_norm"], cfg.rms_epsilon)
    q = O.rope(O.matvec(wt, L["query"], W, W, norm), hd, 1, cfg.rope_base)
    att = O.attention(q, m.k_cache[0, :2], m.v_cache[0, :2], 2, cfg.heads, cfg.kv_heads, hd,
                      np.float32(1.0) / np.sqrt(np.float32(hd)))
    hm = h0 + O.matvec(wt, L["attention_output"], W, W, att)
    n2 = O.rms_norm(hm, L["feed_forward_norm"], cfg.rms_epsilon)
    g = O.silu(O.matvec(wt, L["gate"], F, W, n2)) * O.matvec(wt, L["up"], F, W, n2)
    want = hm + O.matvec(wt, L["down"], W, F, g)
    assert np.array_equal(h, want)
    n3 = O.rms_norm(want, t["output_norm"], cfg.rms_epsilon)
    assert np.array_equal(logits, O.matvec(cfg.output_type, t["output"], cfg.vocabulary, W, n3))


def huge_q4k(rows, cols):
    """Q4_K bytes whose dots overflow f32 against a large input: f16 d =
    65504, every sub-block scale 63 and min 0 (matvec_extra.rs:212-221),
    every quant 15."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0x7BFF], np.uint16).view(np.uint8)
    blk[4:8], blk[8:12], blk[12:16] = 0xFF, 0x00, 0x0F
    blk[16:] = 0xFF
    return np.tile(blk, rows * cols // 256)


def nonfinite_cases():
    """(model config, tensors, input hidden or None for the embedding of
    token 3, expected (check, layer)) of the decode step's NonFinite checks:
    logits that overflow ("matrix output" in finish_hidden, layer =
    n_layers = 0); FFN-norm weights of 1e36, whose gate and up stay finite
    but silu(gate) * up overflows ("matrix input" of the down projection,
    layer 0); a NaN hidden state (the first RMSNorm's "scale", layer 0)."""
    cfg0 = make_config(n_layers=0, output_type=O.Q4_K)
    t0 = dict(make_tensors(cfg0, 29))
    t0["output"] = huge_q4k(cfg0.vocabulary, cfg0.width)
    t0["output_norm"] = np.full(cfg0.width, 1e30, np.float32)
    cfg1 = make_config(n_layers=1)
    t1 = make_tensors(cfg1, 30)
    L = dict(t1["layers"][0])
    L["feed_forward_norm"] = np.full(cfg1.width, 1e36, np.float32)
    t1 = dict(t1, layers=[L])
    return [(cfg0, t0, None, (4, 0)), (cfg1, t1, None, (3, 0)),
            (cfg1, t1, np.full(cfg1.width, np.nan, np.float32), (1, 0))]


@pytest.mark.parametrize("case", range(3))
def test_step_nonfinite_checks(case):
    """The reference's first failing check and its layer (llama.rs:250-392,
    math.rs:144-228): the overflow and NaN constructions fail where f32
    arithmetic says they must (the product, the f32 square, checked here
    with numpy), and the step reports that check."""
    cfg, t, h, (check, layer) = nonfinite_cases()[case]
    o = O.LlamaOracle(cfg, t)
    x = o.embedding(3) if h is None else h
    if case == 0:  # the final norm is finite, the logits are not
        n = O.rms_norm(x, t["output_norm"], cfg.rms_epsilon)
        assert np.all(np.isfinite(n))
        assert not np.all(np.isfinite(O.matvec(O.Q4_K, t["output"], cfg.vocabulary, cfg.width, n)))
    with pytest.raises(O.OracleError) as e:
        o.step(x, 0)
    assert (e.value.name, e.value.a, e.value.b) == ("NonFinite", check, layer)


def test_layer_by_layer_equals_the_step():
    """The checker's per-layer entry points restate the same step: every
    layer run on its own, then finish_hidden, give the step's last-layer
    output and logits bit for bit over several positions (KV rows shared)."""
    cfg = make_config(n_layers=3)
    t = make_tensors(cfg, 41)
    a, b = O.LlamaOracle(cfg, t), O.LlamaOracle(cfg, t)
    for pos, tok in enumerate((5, 17, 999, 0)):
        h_step, lg_step = a.step(a.embedding(tok), pos)
        h = b.embedding(tok)
        for li in range(cfg.n_layers):
            h = b.layer(li, h, pos)
        b.advance()
        emb, lg = b.finish(h)
        assert np.array_equal(h.view(np.uint32), h_step.view(np.uint32)), pos
        assert np.array_equal(lg.view(np.uint32), lg_step.view(np.uint32)), pos
        assert np.array_equal(emb, O.rms_norm(h, t["output_norm"], cfg.rms_epsilon)), pos
