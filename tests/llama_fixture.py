"""Small random-init Llama models for the decode-step tests.

Weights are N(0, 0.02) f32 quantized with the oracle's encoders (Q4_K layer
matrices and embedding, Q6_K output, as a Q4_K_M-style file), norm weights
N(1, 0.05); one seed per model.  The shapes are the smallest that keep every
path of the GPU kernels live: two query heads per KV head, a head dimension of
64, a context that crosses the 256-column softmax padding.
"""
import functools
import types

import numpy as np

import oracle as O


def make_config(n_layers=2, vocabulary=1000, width=256, feed_forward=512, heads=4, kv_heads=2, max_context=300,
                rms_epsilon=1e-5, rope_base=10000.0, weight_type=O.Q4_K, output_type=O.Q6_K,
                embedding_type=O.Q4_K):
    c = types.SimpleNamespace(vocabulary=vocabulary, width=width, feed_forward=feed_forward, heads=heads,
                              kv_heads=kv_heads, max_context=max_context, n_layers=n_layers,
                              rms_epsilon=np.float32(rms_epsilon), rope_base=np.float32(rope_base),
                              attention_scale=np.float32(0.0), weight_type=weight_type, output_type=output_type,
                              embedding_type=embedding_type)
    c.head_dim = width // heads
    c.kv_width = kv_heads * c.head_dim
    return c


def _matrix(rng, dtype, rows, cols, zero=False):
    if zero:
        x = np.zeros(rows * cols, np.float32)
    else:
        x = rng.normal(0.0, 0.02, rows * cols).astype(np.float32)
    return O.quantize(dtype, x)


# A Q4_K_M-like mix (llama.cpp keeps some attn_v / ffn_down in Q6_K): per
# layer, the matrices whose type differs from weight_type.  Layer 1 also
# gives gate and up different types, which splits their launch.
MIXED_TYPES = ({"value": O.Q6_K, "down": O.Q6_K}, {"gate": O.Q5_K, "key": O.Q8_0})


@functools.lru_cache(maxsize=8)
def _tensors(key):
    (n_layers, vocabulary, width, feed_forward, kv_width, wt, ot, et), seed, zero_layers, mixed = key
    rng = np.random.default_rng(seed)
    layers = []
    for i in range(n_layers):
        types = dict(MIXED_TYPES[i % len(MIXED_TYPES)]) if mixed else {}
        t = lambda name: types.get(name, wt)  # noqa: E731
        layers.append({
            "attention_norm": rng.normal(1.0, 0.05, width).astype(np.float32),
            "query": _matrix(rng, t("query"), width, width, zero_layers),
            "key": _matrix(rng, t("key"), kv_width, width, zero_layers),
            "value": _matrix(rng, t("value"), kv_width, width, zero_layers),
            "attention_output": _matrix(rng, t("attention_output"), width, width, zero_layers),
            "feed_forward_norm": rng.normal(1.0, 0.05, width).astype(np.float32),
            "gate": _matrix(rng, t("gate"), feed_forward, width),
            "up": _matrix(rng, t("up"), feed_forward, width),
            "down": _matrix(rng, t("down"), width, feed_forward, zero_layers),
            "types": types,
        })
    # token embeddings of unit scale, as a trained model's
    emb = O.quantize(et, rng.normal(0.0, 1.0, vocabulary * width).astype(np.float32))
    return {"embedding": emb, "output_norm": rng.normal(1.0, 0.05, width).astype(np.float32),
            "output": _matrix(rng, ot, vocabulary, width), "layers": layers}


def make_tensors(cfg, seed, zero_layers=False, mixed=False):
    shape = (cfg.n_layers, cfg.vocabulary, cfg.width, cfg.feed_forward, cfg.kv_width, cfg.weight_type,
             cfg.output_type, cfg.embedding_type)
    return _tensors((shape, seed, zero_layers, mixed))


def matrix_type(cfg, layer, name):
    return layer.get("types", {}).get(name, cfg.weight_type)


def gguf_contents(cfg, t, tied=False, extra_kv=(), extra_tensors=(), drop=()):
    """The metadata and tensors of a llama GGUF file holding this model (the
    library's llama_gguf_contents), with keys or tensors dropped or added."""
    from rlq_loader import load

    kvs, tensors = load().llama_gguf_contents(cfg, t, tied=tied)
    kvs = [kv for kv in kvs if kv[0] not in drop] + list(extra_kv)
    tensors = [x for x in tensors if x[0] not in drop] + list(extra_tensors)
    return kvs, tensors


# Llama-3-8B decode-step shape: 32 layers, d_model 4096, 32 query / 8 KV heads of 128, FFN 14336,
# vocabulary 128256; Q4_K layer matrices and embedding, Q6_K output.
LLAMA3_8B = dict(vocabulary=128256, width=4096, feed_forward=14336, heads=32, kv_heads=8, rope_base=500000.0)


def gpu_tensors(rlq, ctx, cfg, seed):
    """Random-init tensors of `cfg` made on the GPU: matrices N(0, 0.02) and
    the embedding N(0, 1) in f32, encoded by the library's Q4_K / Q6_K
    encoders (bit-exact with the oracle's); norm weights N(1, 0.05).  The
    8B-shape weights (4.7 GB) are too many for the oracle's CPU encoders.
    Returns (device tensors, host copies)."""
    torch = rlq.torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)

    def mat(dtype, rows, cols, std=0.02):
        parts, step = [], max(1, (1 << 26) // cols)
        for r0 in range(0, rows, step):
            x = torch.randn((min(step, rows - r0), cols), generator=g, device="cuda", dtype=torch.float32) * std
            parts.append(ctx.quantize(dtype, x))
        return torch.cat(parts) if len(parts) > 1 else parts[0]

    def norm(n):
        return torch.randn(n, generator=g, device="cuda", dtype=torch.float32) * 0.05 + 1.0

    W, F, kvw = cfg.width, cfg.feed_forward, cfg.kv_width
    wt, ot, et = cfg.weight_type, cfg.output_type, cfg.embedding_type
    layers = [{"attention_norm": norm(W), "query": mat(wt, W, W), "key": mat(wt, kvw, W), "value": mat(wt, kvw, W),
               "attention_output": mat(wt, W, W), "feed_forward_norm": norm(W), "gate": mat(wt, F, W),
               "up": mat(wt, F, W), "down": mat(wt, W, F)} for _ in range(cfg.n_layers)]
    dev = {"embedding": mat(et, cfg.vocabulary, W, 1.0), "output_norm": norm(W), "output": mat(ot, cfg.vocabulary, W),
           "layers": layers}
    ctx.sync()
    host = {k: v.cpu().numpy() for k, v in dev.items() if k != "layers"}
    host["layers"] = [{k: v.cpu().numpy() for k, v in L.items()} for L in layers]
    return dev, host
