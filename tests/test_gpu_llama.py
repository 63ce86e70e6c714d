"""GPU parity of the dense Llama decode step (rlq_llama_*, llama.hip) against
the CPU oracle (oracle/rlq_oracle_llama.c).

Bars, per part of the step (tests/llama_fixture.py models):
  - embedding rows and the final RMSNorm: bit-exact;
  - Q/K/V projections (RMSNorm fused into the quantizer): relative L2 <= 1e-5
    against the oracle's matvec of its own RMSNorm (the quantized activation
    is the same bytes; only the f32 combine order of the exact integer block
    sums differs);
  - attention, given the GPU's own q/k/v: within one f32 ulp per output (the
    same RoPE table; QK dots and softmax totals certified equal to the
    reference's f64 order; the P.V f64 sums in another order);
  - the layer output, given the GPU's own attention output and silu(gate) *
    up: relative L2 <= 1e-5 (the O and down inputs quantize to the same
    bytes);
  - silu(gate) * up: relative L2 <= 1e-3.  The input of gate/up is the RMSNorm of a residual
    stream that already differs from the oracle's in the last f32 bits (the O
    projection's combine order), so one Q8_K rounding of its values may land
    on the other side; one such flip moves the product by about 4e-4;
  - free-running multi-layer steps: relative L2 <= 2e-3 on the logits for
    the same reason, and the same greedy token where the oracle's top-two
    margin exceeds the observed error.
Every test prints its case before touching the GPU.
"""
import numpy as np
import pytest

import oracle as O
from llama_fixture import gguf_contents, make_config, make_tensors, matrix_type
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
    for step in range(70):
        tok = int(rng.integers(cfg.vocabulary))
        h0 = o.embedding(tok)
        h = torch.from_numpy(h0).cuda()
        g.step(h, step, embedding=False, logits=False)
        qkv, att, gu = (host(x) for x in g.intermediates())
        ctx.sync()
        # Q/K/V from the exact RMSNorm
        norm = O.rms_norm(h0, L["attention_norm"], cfg.rms_epsilon)
        for name, lo, hi, rows in (("query", 0, W, W), ("key", W, W + kvw, kvw), ("value", W + kvw, W + 2 * kvw, kvw)):
            e = rel_l2(qkv[lo:hi], O.matvec(matrix_type(cfg, L, name), L[name], rows, W, norm))
            worst[name] = max(worst.get(name, 0), e)
            assert e <= 1e-5, (step, name, e)
        # attention from the GPU's q/k/v: bit-exact
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        want_att = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        # P.V adds the reference's f64 terms in another order: at most the
        # last f32 bit of an output may differ
        assert np.all(np.abs(att - want_att) <= np.spacing(np.abs(want_att))), step
        off = int(np.sum(att != want_att))
        worst["attention_last_bit"] = worst.get("attention_last_bit", 0) + off
        # the rest of the layer from the GPU's attention output and silu(gate) * up
        mt = lambda name: matrix_type(cfg, L, name)  # noqa: E731
        hm = h0 + O.matvec(mt("attention_output"), L["attention_output"], W, W, att)
        n2 = O.rms_norm(hm, L["feed_forward_norm"], cfg.rms_epsilon)
        want_ffn = O.silu(O.matvec(mt("gate"), L["gate"], F, W, n2)) * O.matvec(mt("up"), L["up"], F, W, n2)
        e = rel_l2(gu, want_ffn)
        worst["silu_gate_up"] = max(worst.get("silu_gate_up", 0), e)
        assert e <= 1e-3, (step, e)
        want_h = hm + O.matvec(mt("down"), L["down"], W, F, gu)
        e = rel_l2(host(h), want_h)
        worst["hidden"] = max(worst.get("hidden", 0), e)
        assert e <= 1e-5, (step, e)
    print("worst relative L2 per part:", worst)


@pytest.mark.parametrize("heads,kv_heads,width", [(4, 4, 256), (8, 1, 256), (16, 4, 256), (1, 1, 256),
                                                  (32, 1, 512), (12, 4, 768)])
def test_attention_head_shapes(ctx, heads, kv_heads, width):
    """The attention kernels over head layouts the 8B shape does not use:
    MHA (one query head per KV head), 8 and 32 query heads per KV head (more
    heads than P.V waves), 3 per KV head (waves left idle), and head
    dimensions 16 (the smallest: quarters of one float4) and 256 (the
    largest).  70 steps cross five 16-token score chunks and the 64-column
    P.V boundary; the attention output is checked against the oracle fed
    with the GPU's own q/k/v."""
    say("llama attention heads", heads, "kv heads", kv_heads, "width", width, "70 steps")
    cfg, t, g, o = models(ctx, 1, 31, width=width, heads=heads, kv_heads=kv_heads, max_context=80)
    W, kvw, hd = cfg.width, cfg.kv_width, cfg.head_dim
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    kc = np.zeros((cfg.max_context, kvw), np.float32)
    vc = np.zeros_like(kc)
    rng = np.random.default_rng(9)
    last_bit = 0
    for step in range(70):
        h = torch.from_numpy(o.embedding(int(rng.integers(cfg.vocabulary)))).cuda()
        g.step(h, step, embedding=False, logits=False)
        qkv, att, _ = (host(x) for x in g.intermediates())
        ctx.sync()
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        want = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        assert np.all(np.abs(att - want) <= np.spacing(np.abs(want))), step
        last_bit += int(np.sum(att != want))
    print("outputs differing in the last bit:", last_bit, "of", 70 * W)


def test_attention_repeats_equal_certified_sums(ctx, monkeypatch):
    """The repeats in the reference's order, which run when a certificate
    fails (rare), forced for every QK dot and softmax total with
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
        qkv, att, _ = (host(x) for x in g.intermediates())
        g2.step(torch.from_numpy(h0).cuda(), step, embedding=False, logits=False)
        qkv2, att2, _ = (host(x) for x in g2.intermediates())
        ctx.sync()
        assert np.array_equal(qkv.view(np.uint32), qkv2.view(np.uint32)), step
        assert np.array_equal(att.view(np.uint32), att2.view(np.uint32)), step
        q = O.rope(qkv[:W], hd, step, cfg.rope_base)
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        want = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
        assert np.all(np.abs(att2 - want) <= np.spacing(np.abs(want))), step
    g2.close()


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
        qkv, att, _ = (host(x) for x in g.intermediates())
        kc[step] = O.rope(qkv[W:W + kvw], hd, step, cfg.rope_base)
        vc[step] = qkv[W + kvw:]
        if step in (1022, 1023, 1024, 1025, 1026, 2048, 2599):
            ctx.sync()
            q = O.rope(qkv[:W], hd, step, cfg.rope_base)
            want = O.attention(q, kc[:step + 1], vc[:step + 1], step + 1, cfg.heads, cfg.kv_heads, hd, scale)
            assert np.all(np.abs(att - want) <= np.spacing(np.abs(want))), step
            checked += 1
    ctx.sync()
    assert checked == 7


@pytest.mark.parametrize("wt,ot", [(O.Q4_K, O.Q6_K), (O.Q6_K, O.Q8_0)])
def test_free_running_steps(ctx, wt, ot):
    say("llama 2 layers, 12 free-running steps, logits vs oracle, types", wt, ot)
    cfg, t, g, o = models(ctx, 2, 24, weight_type=wt, output_type=ot)
    rng = np.random.default_rng(6)
    worst = 0.0
    for step in range(12):
        tok = int(rng.integers(cfg.vocabulary))
        h = g.embedding(tok)
        _, logits, am = g.step(h, step, embedding=False, logits=True, argmax=True)
        ctx.sync()
        _, logits_o = o.step(o.embedding(tok), step)
        lg = host(logits)
        e = rel_l2(lg, logits_o)
        worst = max(worst, e)
        assert e <= 2e-3, (step, e)
        top = np.sort(logits_o.astype(np.float64))[::-1]
        margin = top[0] - top[1]
        if margin > 4 * np.max(np.abs(lg.astype(np.float64) - logits_o)):
            assert int(host(am)[0]) == O.argmax(logits_o), step
    print("worst logits relative L2:", worst)


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
