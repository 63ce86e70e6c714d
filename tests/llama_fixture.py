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


GGUF_NAMES = {"query": "attn_q", "key": "attn_k", "value": "attn_v", "attention_output": "attn_output",
              "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down", "attention_norm": "attn_norm",
              "feed_forward_norm": "ffn_norm"}


def gguf_contents(cfg, t, tied=False, extra_kv=(), extra_tensors=(), drop=()):
    """The metadata and tensors of a llama GGUF file holding this model, in
    the names and GGML shapes of the reference's loader
    (crates/inference/src/loader.rs:282-394): (kvs, tensors) for the
    library's GGUF writer.  tied: no output.weight (the embedding projects;
    the model's output matrix must then be the embedding)."""
    f32 = lambda x: int(np.float32(x).view(np.uint32))  # noqa: E731
    kvs = [(b"general.architecture", 8, b"llama"), (b"general.name", 8, b"random-init"),
           (b"llama.block_count", 4, cfg.n_layers), (b"llama.context_length", 4, cfg.max_context),
           (b"llama.embedding_length", 4, cfg.width), (b"llama.feed_forward_length", 4, cfg.feed_forward),
           (b"llama.attention.head_count", 4, cfg.heads), (b"llama.attention.head_count_kv", 4, cfg.kv_heads),
           (b"llama.attention.layer_norm_rms_epsilon", 6, f32(cfg.rms_epsilon)),
           (b"llama.rope.freq_base", 6, f32(cfg.rope_base)), (b"llama.rope.dimension_count", 4, cfg.head_dim),
           (b"tokenizer.ggml.model", 8, b"llama"),
           (b"tokenizer.ggml.tokens", 9, (8, [b"t%d" % i for i in range(cfg.vocabulary)]))]
    kvs = [kv for kv in kvs if kv[0] not in drop] + list(extra_kv)
    W, F, kvw = cfg.width, cfg.feed_forward, cfg.kv_width
    tensors = [(b"token_embd.weight", [W, cfg.vocabulary], cfg.embedding_type, t["embedding"]),
               (b"output_norm.weight", [W], 0, t["output_norm"].view(np.uint8))]
    if not tied:
        tensors.append((b"output.weight", [W, cfg.vocabulary], cfg.output_type, t["output"]))
    shapes = {"query": [W, W], "key": [W, kvw], "value": [W, kvw], "attention_output": [W, W], "gate": [W, F],
              "up": [W, F], "down": [F, W]}
    for i, L in enumerate(t["layers"]):
        for name, g in GGUF_NAMES.items():
            nm = b"blk.%d.%s.weight" % (i, g.encode())
            if name.endswith("norm"):
                tensors.append((nm, [W], 0, L[name].view(np.uint8)))
            else:
                tensors.append((nm, shapes[name], matrix_type(cfg, L, name), L[name]))
    tensors = [x for x in tensors if x[0] not in drop] + list(extra_tensors)
    return kvs, tensors
