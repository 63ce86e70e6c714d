"""GPU parity of the dense Llama decode step (rlq_llama_*, llama.hip) against
the CPU oracle (oracle/rlq_oracle_llama.c).

Bars, per part of the step (tests/llama_fixture.py models):
  - embedding rows and the final RMSNorm: bit-exact;
  - Q/K/V projections (RMSNorm fused into the quantizer) against the oracle's
    matvec of its own RMSNorm: bit-exact (every weight type's one-column
    kernel keeps the reference's f32 order);
  - attention, given the GPU's own q/k/v: bit-exact (the same RoPE table; the
    QK dots, softmax totals and P.V sums certified equal to the reference's
    f64 order, or repeated in it);
  - the layer output, given the GPU's own residual stream after attention
    and silu(gate) * up, and the residual stream after attention and
    silu(gate) * up, each given the GPU's own input: bit-exact;
  - free-running multi-layer steps: logits bit-exact and the same greedy
    token every step.
Every test prints its case before touching the GPU.
"""
import numpy as np
import pytest

import oracle as O
from llama_fixture import LLAMA3_8B, gguf_contents, gpu_tensors, make_config, make_tensors, matrix_type
from rlq_loader import load

pytestmark = pytest.mark.gpu

rlq = load()
torch = rlq.torch


def say(*a):
    print("[case]", *a, flush=True)


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return np.linalg.norm(got - want) / (den if den > 0 else 1.0)


@pytest.fixture(scope="module")
def ctx():
    c = rlq.Context(0)
    yield c
    c.close()


def gpu_config(cfg):
    return rlq.LlamaConfig(cfg.vocabulary, cfg.width, cfg.feed_forward, cfg.heads, cfg.kv_heads, cfg.max_context,
                           cfg.n_layers, float(cfg.rms_epsilon), float(cfg.rope_base), float(cfg.attention_scale),
                           cfg.weight_type, cfg.output_type, cfg.embedding_type)


def models(ctx, n_layers, seed, mixed=False, **kw):
    cfg = make_config(n_layers=n_layers, **kw)
    t = make_tensors(cfg, seed, mixed=mixed)
    return cfg, t, rlq.LlamaModel(ctx, gpu_config(cfg), t), O.LlamaOracle(cfg, t)


def host(x):
    return x.detach().cpu().numpy()


def bits(y):
    return np.asarray(y, np.float32).view(np.uint32)


# weight types whose one-column kernels give the reference's f32 bits
EXACT_TYPES = (O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0)


def part_bar(exact, got, want, what):
    """Bit-exact when the kernels keep the reference's f32 order, else
    relative L2 <= 1e-5; returns the relative L2."""
    e = rel_l2(got, want)
    if exact:
        assert np.array_equal(bits(got), bits(want)), (what, e)
    assert e <= 1e-5, (what, e)
    return e


@pytest.mark.parametrize("et", [O.Q4_K, O.Q8_0, O.Q2_K, O.Q3_K, O.Q5_K, O.Q6_K])
def test_embedding_rows_exact(ctx, et):
    say("llama embedding rows, 0 layers, embedding type", et)
    cfg, t, g, o = models(ctx, 0, 21, embedding_type=et)
    for tok in (0, 1, 499, 999):
        assert np.array_equal(host(g.embedding(tok)), o.embedding(tok)), tok
    with pytest.raises(rlq.QuantError) as e:
        g.embedding(cfg.vocabulary)
    assert e.value.name == "InvalidToken"


@pytest.mark.parametrize("ot", [O.Q6_K, O.Q8_0, O.Q4_K, O.Q5_K])
def test_output_head_without_layers(ctx, ot):
    """RMSNorm fused into the output matvec's quantizer (Q8_K, or Q8_0 for
    Q8_0 weights); the fused greedy argmax."""
    say("llama step, 0 layers: final norm + output matvec + argmax, output type", ot)
    cfg, t, g, o = models(ctx, 0, 22, output_type=ot)
    for tok, pos in ((3, 0), (77, 1), (998, 2)):
        h = g.embedding(tok)
        emb, logits, am = g.step(h, pos, embedding=True, logits=True, argmax=True)
        ctx.sync()
        h_o, logits_o = o.step(o.embedding(tok), pos)
        assert np.array_equal(host(emb), O.rms_norm(h_o, t["output_norm"], cfg.rms_epsilon))
        assert rel_l2(host(logits), logits_o) <= 1e-5
        lg = host(logits)
        assert int(host(am)[0]) == int(np.argmax(lg))


@pytest.mark.parametrize("wt,mixed", [(O.Q4_K, False), (O.Q5_K, False), (O.Q6_K, False), (O.Q8_0, False),
                                      (O.Q3_K, False), (O.Q2_K, False), (O.Q4_K, True)])
def test_one_layer_parts(ctx, wt, mixed):
    """Each part of one layer against the oracle fed with the GPU's own
    intermediates, over several steps (the cache grows past 64 rows: two
    attention chunks).  Q4_K / Q5_K layers run silu(gate) * up in the gate/up
    epilogue, the other types in the down projection's quantizer; Q8_0
    layers quantize their activations to Q8_0.  mixed: V and down in Q6_K
    (a Q4_K_M layer), so Q/K/V run as three launches."""
    say("llama 1 layer, parts, 70 steps, layer type", wt, "mixed" if mixed else "")
    cfg, t, g, o = models(ctx, 1, 23, mixed=mixed, weight_type=wt)
    L = t["layers"][0]
    W, kvw, hd, F = cfg.width, cfg.kv_width, cfg.head_dim, cfg.feed_forward
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kc = np.zeros((cfg.max_context, kvw), np.float32)
    vc = np.zeros_like(kc)
    rng = np.random.default_rng(5)
    worst = {}
    mt = lambda name: matrix_type(cfg, L, name)  # noqa: E731
    ex = lambda *names: all(mt(n) in EXACT_TYPES for n in names)  # noqa: E731
    for step in range(70):
        tok = int(rng.integers(cfg.vocabulary))
        h0 = o.embedding(tok)
        h = torch.from_numpy(h0).cuda()
        g.step(h, step, embedding=False, logits=False)
        qkv, att, gu, mid = (host(x) for x in g.intermediates())
        ctx.sync()
        # Q/K/V from the exact RMSNorm
        norm = O.rms_norm(h0, L["attention_norm"], cfg.rms_epsilon)
        for name, lo, hi, rows in (("query", 0, W, W), ("key", W, W + kvw, kvw), ("value", W + kvw, W + 2 * kvw, kvw)):
            e = part_bar(ex(name), qkv[lo:hi], O.matvec(mt(name), L[name], rows, W, norm), (step, name))
            worst[name] = max(worst.get(name, 0), e)
        # attention from the GPU's q/k/v: bit-exact
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        want_att = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        assert np.array_equal(bits(att), bits(want_att)), step
        # the rest of the layer, each part from the GPU's own inputs: the
        # residual after attention from its attention output, silu(gate) * up
        # from its residual stream (the FFN norm's input), the layer output
        # from its residual stream and silu(gate) * up
        hm = h0 + O.matvec(mt("attention_output"), L["attention_output"], W, W, att)
        e = part_bar(ex("attention_output"), mid, hm, (step, "ffn_input"))
        worst["ffn_input"] = max(worst.get("ffn_input", 0), e)
        n2 = O.rms_norm(mid, L["feed_forward_norm"], cfg.rms_epsilon)
        want_ffn = O.silu(O.matvec(mt("gate"), L["gate"], F, W, n2)) * O.matvec(mt("up"), L["up"], F, W, n2)
        e = part_bar(ex("gate", "up"), gu, want_ffn, (step, "silu_gate_up"))
        worst["silu_gate_up"] = max(worst.get("silu_gate_up", 0), e)
        want_h = mid + O.matvec(mt("down"), L["down"], W, F, gu)
        e = part_bar(ex("down"), host(h), want_h, (step, "hidden"))
        worst["hidden"] = max(worst.get("hidden", 0), e)
    print("worst relative L2 per part:", worst)


@pytest.mark.parametrize("heads,kv_heads,width", [(4, 4, 256), (8, 1, 256), (16, 4, 256), (1, 1, 256),
                                                  (32, 1, 512), (12, 4, 768), (32, 8, 4096), (8, 2, 1024)])
def test_attention_head_shapes(ctx, heads, kv_heads, width):
    """The attention kernels over head layouts the 8B shape does not use:
    MHA (one query head per KV head), 8 and 32 query heads per KV head (more
    heads than P.V waves), 3 per KV head (waves left idle), head dimensions
    16 (the smallest: quarters of one float4) and 256 (the largest), and
    the Llama-3-8B heads (32 query / 8 KV heads of 128).  70 steps cross five 16-token score chunks and the 64-column
    P.V boundary; the attention output is checked bitwise against the oracle
    fed with the GPU's own q/k/v."""
    say("llama attention heads", heads, "kv heads", kv_heads, "width", width, "70 steps")
    cfg, t, g, o = models(ctx, 1, 31, width=width, heads=heads, kv_heads=kv_heads, max_context=80)
    W, kvw, hd = cfg.width, cfg.kv_width, cfg.head_dim
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kc = np.zeros((cfg.max_context, kvw), np.float32)
    vc = np.zeros_like(kc)
    rng = np.random.default_rng(9)
    for step in range(70):
        h = torch.from_numpy(o.embedding(int(rng.integers(cfg.vocabulary)))).cuda()
        g.step(h, step, embedding=False, logits=False)
        qkv, att, _, _ = (host(x) for x in g.intermediates())
        ctx.sync()
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        want = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        assert np.array_equal(bits(att), bits(want)), step


def test_attention_repeats_equal_certified_sums(ctx, monkeypatch):
    """The repeats in the reference's order, which run when a certificate
    fails (rare), forced for every QK dot, softmax total and P.V sum with
    RLQ_ATTN_REPEAT_ALL=1: the attention output is bitwise the certified
    kernels' (both are the reference's f32 values) and the oracle's."""
    say("llama attention, every sum repeated in the reference's order, 70 steps")
    cfg, t, g, o = models(ctx, 1, 35, heads=8, kv_heads=2, max_context=80)
    monkeypatch.setenv("RLQ_ATTN_REPEAT_ALL", "1")
    g2 = rlq.LlamaModel(ctx, gpu_config(cfg), t)
    monkeypatch.delenv("RLQ_ATTN_REPEAT_ALL")
    W, kvw, hd = cfg.width, cfg.kv_width, cfg.head_dim
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kc = np.zeros((cfg.max_context, kvw), np.float32)
    vc = np.zeros_like(kc)
    rng = np.random.default_rng(17)
    for step in range(70):
        h0 = o.embedding(int(rng.integers(cfg.vocabulary)))
        g.step(torch.from_numpy(h0).cuda(), step, embedding=False, logits=False)
        qkv, att, _, _ = (host(x) for x in g.intermediates())
        g2.step(torch.from_numpy(h0).cuda(), step, embedding=False, logits=False)
        qkv2, att2, _, _ = (host(x) for x in g2.intermediates())
        ctx.sync()
        assert np.array_equal(qkv.view(np.uint32), qkv2.view(np.uint32)), step
        assert np.array_equal(att.view(np.uint32), att2.view(np.uint32)), step
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        want = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        assert np.array_equal(bits(att2), bits(want)), step
    g2.close()


def test_attention_scores_below_the_plain_exponential(ctx):
    """Scores spread over hundreds (the attention RMSNorm weights times 20,
    so q and k grow 20-fold): softmax arguments below -87.3 take the
    exponential's other branch (subnormal results; zero below about -133.5).
    The attention output is bitwise the oracle's at every step, and the run
    is checked to reach both ranges."""
    say("llama attention, attention norm x20 (scores below exp's plain range), 70 steps")
    cfg = make_config(n_layers=1, heads=8, kv_heads=2, max_context=80)
    t0 = make_tensors(cfg, 37)
    L = dict(t0["layers"][0])
    L["attention_norm"] = (L["attention_norm"] * np.float32(20.0)).astype(np.float32)
    t = dict(t0, layers=[L])  # (a copy: the fixture's tensors are shared)
    g, o = rlq.LlamaModel(ctx, gpu_config(cfg), t), O.LlamaOracle(cfg, t)
    W, kvw, hd = cfg.width, cfg.kv_width, cfg.head_dim
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kc = np.zeros((cfg.max_context, kvw), np.float32)
    vc = np.zeros_like(kc)
    rng = np.random.default_rng(19)
    plain = subnormal = zero = 0
    for step in range(70):
        h = torch.from_numpy(o.embedding(int(rng.integers(cfg.vocabulary)))).cuda()
        g.step(h, step, embedding=False, logits=False)
        qkv, att, _, _ = (host(x) for x in g.intermediates())
        ctx.sync()
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        want = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        assert np.array_equal(bits(att), bits(want)), step
        G = cfg.heads // cfg.kv_heads
        for hh in range(cfg.heads):
            kv = hh // G
            s = kc[:step + 1, kv * hd:(kv + 1) * hd].astype(np.float64) @ q[hh * hd:(hh + 1) * hd] * float(scale)
            x = s - s.max()
            plain += int((x > -86.0).sum())
            subnormal += int(((x < -89.0) & (x > -132.0)).sum())
            zero += int((x < -135.0).sum())
    g.close()
    assert plain > 0 and subnormal > 0 and zero > 0, (plain, subnormal, zero)


def test_attention_long_context(ctx):
    """2,600 rows of cache with four query heads per KV head: each P.V lane
    keeps its first 2 column groups (1,024 columns over the workgroup) in
    registers and reloads the rest, and the workgroup's LDS does not grow
    with the context.  Checked against the oracle around the register
    boundary, past 2,048 rows and at the end."""
    say("llama attention, context 2600, 4 heads / 1 kv head")
    cfg, t, g, o = models(ctx, 1, 33, heads=4, kv_heads=1, max_context=2600)
    W, kvw, hd = cfg.width, cfg.kv_width, cfg.head_dim
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kc = np.zeros((cfg.max_context, kvw), np.float32)
    vc = np.zeros_like(kc)
    rng = np.random.default_rng(13)
    toks = rng.integers(cfg.vocabulary, size=cfg.max_context)
    checked = 0
    for step in range(cfg.max_context):
        h = torch.from_numpy(o.embedding(int(toks[step]))).cuda()
        g.step(h, step, embedding=False, logits=False)
        qkv, att, _, _ = (host(x) for x in g.intermediates())
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        if step in (1022, 1023, 1024, 1025, 1026, 2048, 2599):
            ctx.sync()
            q = O.rope(qkv[:W], hd, step, cfg.rope_base)
            want = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
            assert np.array_equal(bits(att), bits(want)), step
            checked += 1
    ctx.sync()
    assert checked == 7


@pytest.mark.parametrize("wt,ot", [(O.Q4_K, O.Q6_K), (O.Q6_K, O.Q8_0), (O.Q3_K, O.Q6_K)])
def test_free_running_steps(ctx, wt, ot):
    """Two layers, 24 steps, each step's token the previous step's greedy
    token (the first random): the logits bitwise the oracle's and the same
    token every step (the oracle's token is fed to both)."""
    say("llama 2 layers, 24 free-running steps, logits vs oracle, types", wt, ot)
    cfg, t, g, o = models(ctx, 2, 24, weight_type=wt, output_type=ot)
    exact = wt in EXACT_TYPES and ot in EXACT_TYPES
    tok = int(np.random.default_rng(6).integers(cfg.vocabulary))
    worst = 0.0
    for step in range(24):
        h = g.embedding(tok)
        _, logits, am = g.step(h, step, embedding=False, logits=True, argmax=True)
        ctx.sync()
        _, logits_o = o.step(o.embedding(tok), step)
        lg = host(logits)
        e = rel_l2(lg, logits_o)
        worst = max(worst, e)
        assert e <= 2e-3, (step, e)
        if exact:
            assert np.array_equal(bits(lg), bits(logits_o)), (step, e)
            assert int(host(am)[0]) == O.argmax(logits_o), step
        else:
            top = np.sort(logits_o.astype(np.float64))[::-1]
            if top[0] - top[1] > 4 * np.max(np.abs(lg.astype(np.float64) - logits_o)):
                assert int(host(am)[0]) == O.argmax(logits_o), step
        tok = O.argmax(logits_o)
    print("worst logits relative L2:", worst)


@pytest.mark.parametrize("case", range(3))
def test_nonfinite_checks_of_the_step(ctx, case):
    """The step's NonFinite checks report what the oracle's sequential step
    reports first (the check in rlq_error.a, the layer in b): overflowing
    logits ("matrix output" of finish_hidden), an overflowing silu(gate) *
    up ("matrix input" of the down projection), a NaN hidden state (the
    first RMSNorm's scale); see test_oracle_llama.nonfinite_cases."""
    from test_oracle_llama import nonfinite_cases
    cfg, t, h, (check, layer) = nonfinite_cases()[case]
    say("llama NonFinite check", check, "layer", layer)
    o = O.LlamaOracle(cfg, t)
    x = o.embedding(3) if h is None else h
    with pytest.raises(O.OracleError) as want:
        o.step(x, 0)
    g = rlq.LlamaModel(ctx, gpu_config(cfg), t)
    g.step(torch.from_numpy(np.array(x)).cuda(), 0, embedding=True, logits=True, argmax=True)
    with pytest.raises(rlq.QuantError) as got:
        ctx.sync()
    assert (got.value.name, got.value.a, got.value.b) == (want.value.name, want.value.a, want.value.b) == \
        ("NonFinite", check, layer)
    ctx.sync()  # the error word was cleared
    g.close()


def test_cache_limit_and_truncate(ctx):
    say("llama 1 layer, context 8: cache full, truncate")
    cfg, t, g, o = models(ctx, 1, 25, max_context=8)
    h = g.embedding(1)
    for step in range(8):
        g.step(h, step, embedding=False, logits=False)
    assert g.cached == 8
    with pytest.raises(rlq.QuantError) as e:
        g.step(h, 8, embedding=False, logits=False)
    assert e.value.name == "InvalidState"
    g.truncate(3)
    assert g.cached == 3
    g.step(h, 3, embedding=False, logits=False)
    ctx.sync()
    assert g.cached == 4


@pytest.mark.parametrize("field,value,check", [
    ("heads", 3, 3), ("kv_heads", 3, 3), ("rms_epsilon", 0.0, 2), ("rope_base", -1.0, 5), ("vocabulary", 0, 1)])
def test_config_checks(ctx, field, value, check):
    say("llama config check", field, value)
    cfg = make_config(n_layers=1)
    t = make_tensors(cfg, 26)
    c = gpu_config(cfg)
    setattr(c, field, value)
    with pytest.raises(rlq.QuantError) as e:
        rlq.LlamaModel(ctx, c, t)
    assert e.value.name == "InvalidConfig" and e.value.a == check


# ------------------------------------------------------------ models from GGUF files

@pytest.mark.parametrize("tied", [False, True])
def test_gguf_model_equals_direct_creation(ctx, tmp_path, tied):
    """A model written with the library's GGUF writer and loaded by
    rlq_llama_create_from_gguf (mixed per-matrix types; tied: no
    output.weight, the embedding projects) runs the same kernels on the same
    bytes as the model created from the tensors: identical logits, and the
    oracle's within the free-running bar."""
    say("llama GGUF round trip, 2 layers, mixed types, tied output" if tied else "llama GGUF round trip, 2 layers")
    cfg = make_config(n_layers=2, output_type=O.Q4_K if tied else O.Q6_K)
    t = make_tensors(cfg, 27, mixed=True)
    if tied:
        t = dict(t, output=t["embedding"])
    kvs, tensors = gguf_contents(cfg, t, tied=tied)
    path = str(tmp_path / "model.gguf")
    rlq.gguf_write(path, kvs, tensors)
    g = rlq.LlamaModel.from_gguf(ctx, path, 4096)
    c = g.config
    assert (c.vocabulary, c.width, c.feed_forward, c.heads, c.kv_heads, c.max_context, c.n_layers) == \
        (cfg.vocabulary, cfg.width, cfg.feed_forward, cfg.heads, cfg.kv_heads, cfg.max_context, cfg.n_layers)
    assert (c.weight_type, c.output_type, c.embedding_type) == (cfg.weight_type, cfg.output_type, cfg.embedding_type)
    assert (c.rms_epsilon, c.rope_base, c.attention_scale) == (cfg.rms_epsilon, cfg.rope_base, 0.0)
    d = rlq.LlamaModel(ctx, gpu_config(cfg), t)
    o = O.LlamaOracle(cfg, t)
    rng = np.random.default_rng(9)
    for step in range(8):
        tok = int(rng.integers(cfg.vocabulary))
        assert np.array_equal(host(g.embedding(tok)), host(d.embedding(tok)))
        _, lg, ag = g.step(g.embedding(tok), step, embedding=False, logits=True, argmax=True)
        _, ld, ad = d.step(d.embedding(tok), step, embedding=False, logits=True, argmax=True)
        ctx.sync()
        assert np.array_equal(host(lg), host(ld)) and int(host(ag)[0]) == int(host(ad)[0]), step
        _, lo = o.step(o.embedding(tok), step)
        assert rel_l2(host(lg), lo) <= 2e-3, step


def test_gguf_loader_checks(ctx, tmp_path):
    """The reference loader's checks (loader.rs:242-410), with the check
    number in the error payload."""
    cfg = make_config(n_layers=1)
    t = make_tensors(cfg, 28)
    path = str(tmp_path / "bad.gguf")
    W = cfg.width
    cases = [
        (dict(drop=[b"llama.embedding_length"]), "GgufInvalid", 7),
        (dict(extra_kv=[(b"llama.expert_count", 4, 8)]), "GgufUnsupported", 16),
        (dict(drop=[b"general.architecture"], extra_kv=[(b"general.architecture", 8, b"gpt2")]), "GgufUnsupported", 2),
        (dict(extra_kv=[(b"llama.rope.scaling.type", 8, b"yarn")]), "GgufUnsupported", 18),
        (dict(drop=[b"llama.context_length"], extra_kv=[(b"llama.context_length", 10, 300)]), "GgufInvalid", 13),
        (dict(extra_tensors=[(b"blk.0.attn_q.bias", [W], 0, np.zeros(4 * W, np.uint8))]), "Unimplemented", 49),
        (dict(extra_tensors=[(b"vision.weight", [4], 0, np.zeros(16, np.uint8))]), "GgufUnsupported", 51),
        (dict(drop=[b"blk.0.ffn_down.weight"]), "GgufInvalid", 46),
    ]
    for kw, name, check in cases:
        say("GGUF loader check", name, check)
        kvs, tensors = gguf_contents(cfg, t, **kw)
        rlq.gguf_write(path, kvs, tensors)
        with pytest.raises(rlq.QuantError) as e:
            rlq.LlamaModel.from_gguf(ctx, path, 4096)
        assert (e.value.name, e.value.a) == (name, check), (kw, e.value)
    kvs, tensors = gguf_contents(cfg, t)
    rlq.gguf_write(path, kvs, tensors)
    with pytest.raises(rlq.QuantError) as e:
        rlq.LlamaModel.from_gguf(ctx, path, 0)
    assert (e.value.name, e.value.a) == ("GgufInvalid", 1)
    m = rlq.LlamaModel.from_gguf(ctx, path, 100)  # min(context_length, the file's)
    assert m.config.max_context == 100


# ------------------------------------------------------------ the Llama-3-8B decode-step shape

def config_8b(n_layers, max_context):
    L = LLAMA3_8B
    return make_config(n_layers=n_layers, vocabulary=L["vocabulary"], width=L["width"],
                       feed_forward=L["feed_forward"], heads=L["heads"], kv_heads=L["kv_heads"],
                       max_context=max_context, rope_base=L["rope_base"])


def test_8b_shape_one_layer_parts(ctx):
    """One layer at the Llama-3-8B shape (d 4096, 32 query / 8 KV heads of
    128, FFN 14336, vocabulary 128256), so every kernel the decode step
    launches runs at its production shape: the fused Q/K/V matvec (6144 rows,
    RMSNorm in the quantizer), attention at head_dim 128 with 4 query heads
    per KV head, the O projection with its residual, the 28672-row gate/up
    kernel with the SiLU-pair epilogue, the 16-wave down projection (56
    blocks per row) and the 128256-row Q6_K output matvec with the final
    RMSNorm and the fused argmax.  70 steps (five 16-token score chunks,
    past the 64-column P.V boundary); each part against the oracle fed the
    GPU's own inputs, at the bars of test_one_layer_parts (bit-exact), at
    selected steps; the logits bitwise the oracle's from the GPU's own last
    hidden state."""
    say("llama 1 layer at the 8B shape, parts, 70 steps")
    cfg = config_8b(1, 128)
    dev, t = gpu_tensors(rlq, ctx, cfg, 0x8B01)
    g = rlq.LlamaModel(ctx, gpu_config(cfg), dev)
    del dev
    o = O.LlamaOracle(cfg, t, threads=16)
    L = t["layers"][0]
    W, kvw, hd, F, V = cfg.width, cfg.kv_width, cfg.head_dim, cfg.feed_forward, cfg.vocabulary
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kc = np.zeros((cfg.max_context, kvw), np.float32)
    vc = np.zeros_like(kc)
    rng = np.random.default_rng(8)
    worst = {}

    def bar(name, got, want):  # Q4_K / Q6_K matvecs: the reference's f32 bits
        worst[name] = max(worst.get(name, 0.0), part_bar(True, got, want, (step, name)))

    for step in range(70):
        tok = int(rng.integers(V))
        h0 = o.embedding(tok)
        assert np.array_equal(host(g.embedding(tok)), h0), step
        h = torch.from_numpy(h0).cuda()
        emb, logits, am = g.step(h, step, embedding=True, logits=True, argmax=True)
        qkv, att, gu, mid = (host(x) for x in g.intermediates())
        ctx.sync()
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        if step not in (0, 1, 2, 15, 16, 17, 63, 64, 65, 69):
            continue
        norm = O.rms_norm(h0, L["attention_norm"], cfg.rms_epsilon)
        bar("query", qkv[:W], O.matvec(O.Q4_K, L["query"], W, W, norm, threads=16))
        bar("key", qkv[W:W + kvw], O.matvec(O.Q4_K, L["key"], kvw, W, norm, threads=16))
        bar("value", qkv[W + kvw:], O.matvec(O.Q4_K, L["value"], kvw, W, norm, threads=16))
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        want_att = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        assert np.array_equal(bits(att), bits(want_att)), step
        bar("ffn_input", mid, h0 + O.matvec(O.Q4_K, L["attention_output"], W, W, att, threads=16))
        n2 = O.rms_norm(mid, L["feed_forward_norm"], cfg.rms_epsilon)
        want_ffn = O.silu(O.matvec(O.Q4_K, L["gate"], F, W, n2, threads=16)) * \
            O.matvec(O.Q4_K, L["up"], F, W, n2, threads=16)
        bar("silu_gate_up", gu, want_ffn)
        hh = host(h)
        bar("hidden", hh, mid + O.matvec(O.Q4_K, L["down"], W, F, gu, threads=16))
        e0 = O.rms_norm(hh, t["output_norm"], cfg.rms_epsilon)
        assert np.array_equal(host(emb), e0), step
        lg = host(logits)
        bar("logits", lg, O.matvec(O.Q6_K, t["output"], V, W, e0, threads=16))
        assert int(host(am)[0]) == O.argmax(lg), step
    print("worst relative L2 per part:", worst)
    g.close()


def test_8b_shape_full_model(ctx):
    """The decode step of the whole Llama-3-8B-shape model (32 layers; the
    config the benchmark times).  Three steps with every part of every layer
    checked bitwise against the oracle fed that part's GPU input
    (rlq_llama_trace): Q/K/V, the attention (K/V history from the GPU's own
    rows), the residual after attention, silu(gate) * up, the layer output,
    the final norm and the logits, with the same greedy token.  The logits of
    those steps are also bitwise the oracle's own step's; then 29 more steps
    run free, each step's token the previous step's greedy token, with the
    GPU's logits bitwise the oracle's and the same token every step.  Then
    the cache filled to 1,000 rows with every step's logits finite and its
    argmax the first maximum of its own logits, and a second pass over the
    same tokens after truncate(0) bitwise equal to the first."""
    say("llama 32 layers at the 8B shape: 3 steps part by part, 32 free-running steps vs the oracle, "
        "then 1000 rows twice")
    cfg = config_8b(32, 1024)
    dev, t = gpu_tensors(rlq, ctx, cfg, 0x8B20)
    g = rlq.LlamaModel(ctx, gpu_config(cfg), dev)
    del dev
    torch.cuda.empty_cache()
    o = O.LlamaOracle(cfg, t, threads=16)
    rng = np.random.default_rng(20)
    toks = rng.integers(cfg.vocabulary, size=1000).tolist()
    W, kvw, hd, F, V = cfg.width, cfg.kv_width, cfg.head_dim, cfg.feed_forward, cfg.vocabulary
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    trace = torch.empty((cfg.n_layers, g.trace_stride), dtype=torch.float32, device="cuda")
    g.trace(trace)
    kc = np.zeros((cfg.n_layers, 3, kvw), np.float32)
    vc = np.zeros_like(kc)
    worst = {}

    def bar(name, got, want):  # Q4_K / Q6_K matvecs: the reference's f32 bits
        worst[name] = max(worst.get(name, 0.0), part_bar(True, got, want, (step, li, name)))

    for step in range(3):
        h0 = o.embedding(toks[step])
        emb, logits, am = g.step(torch.from_numpy(h0).cuda(), step, embedding=True, logits=True, argmax=True)
        rows = host(trace)
        ctx.sync()
        for li in range(cfg.n_layers):
            L = t["layers"][li]
            qkv, att, mid, gu, out = g.split_trace(rows[li])
            x = h0 if li == 0 else g.split_trace(rows[li - 1])[4]
            norm = O.rms_norm(x, L["attention_norm"], cfg.rms_epsilon)
            bar("query", qkv[:W], O.matvec(O.Q4_K, L["query"], W, W, norm, threads=16))
            bar("key", qkv[W:W + kvw], O.matvec(O.Q4_K, L["key"], kvw, W, norm, threads=16))
            bar("value", qkv[W + kvw:], O.matvec(O.Q4_K, L["value"], kvw, W, norm, threads=16))
            kc[li, step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
            vc[li, step] = qkv[W + kvw:]
            q = O.rope(qkv[:W], hd, step, cfg.rope_base)
            want = O.attention(q, kc[li, :step + 1], vc[li, :step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
            assert np.array_equal(bits(att), bits(want)), (step, li)
            bar("ffn_input", mid, x + O.matvec(O.Q4_K, L["attention_output"], W, W, att, threads=16))
            n2 = O.rms_norm(mid, L["feed_forward_norm"], cfg.rms_epsilon)
            bar("silu_gate_up", gu, O.silu(O.matvec(O.Q4_K, L["gate"], F, W, n2, threads=16)) *
                                       O.matvec(O.Q4_K, L["up"], F, W, n2, threads=16))
            bar("output", out, mid + O.matvec(O.Q4_K, L["down"], W, F, gu, threads=16))
        last = g.split_trace(rows[-1])[4]
        assert np.array_equal(host(emb), O.rms_norm(last, t["output_norm"], cfg.rms_epsilon)), step
        lg = host(logits)
        li = "logits"
        bar("logits", lg, O.matvec(O.Q6_K, t["output"], V, W, host(emb), threads=16))
        assert int(host(am)[0]) == O.argmax(lg), step
        assert np.array_equal(bits(lg), bits(o.step(h0, step)[1])), step
    g.trace(None)
    print("worst relative L2 per part over 32 layers x 3 steps:", worst)
    # free-running: the previous step's greedy token, on both sides
    tok = O.argmax(lg)
    for step in range(3, 32):
        say("free-running step", step, "token", tok)
        _, logits, am = g.step(g.embedding(tok), step, embedding=False, logits=True, argmax=True)
        ctx.sync()
        _, want = o.step(o.embedding(tok), step)
        lg = host(logits)
        assert np.array_equal(bits(lg), bits(want)), (step, rel_l2(lg, want))
        assert int(host(am)[0]) == O.argmax(want), step
        tok = O.argmax(want)
    del o, t
    g.truncate(3)
    marks = (3, 255, 256, 511, 767, 998, 999)

    def run(start):
        kept = {}
        for step in range(start, 1000):
            _, logits, am = g.step(g.embedding(toks[step]), step, embedding=False, logits=True, argmax=True)
            if step in marks:
                ctx.sync()
                lg = host(logits)
                assert np.all(np.isfinite(lg)), step
                assert int(host(am)[0]) == O.argmax(lg), step
                kept[step] = lg
        ctx.sync()
        return kept

    first = run(3)
    assert g.cached == 1000
    g.truncate(0)
    for step in range(3):
        g.step(g.embedding(toks[step]), step, embedding=False, logits=False)
    second = run(3)
    for step in marks:
        assert np.array_equal(first[step].view(np.uint32), second[step].view(np.uint32)), step
    g.close()
