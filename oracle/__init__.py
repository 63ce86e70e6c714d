"""ctypes binding of the CPU oracle (librlq_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP path.  Only the tests, the
smoke check and the CPU-baseline leg of bench.py import this module; the
product package never does.

The library restates rust-llama's scalar `llama-quant` path in C
(crates/quant/src/{lib,matvec,matvec_extra,activation,encode,encode_k,decode}.rs);
see rlq_oracle.h for the per-function citations.  `make -C oracle` builds it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("RLQ_ORACLE_LIB") or os.path.join(HERE, "librlq_oracle.so")

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 8, 10, 11, 12, 13, 14, 15
BLOCK = {Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256}
TYPE_SIZE = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292}

# Status codes in the order of the reference's QuantError (lib.rs:45-63).
ERROR_NAMES = {
    0: "Ok", 1: "InvalidType", 2: "UnsupportedMatVec", 3: "InvalidVectorLength",
    4: "InvalidMatrixShape", 5: "NonMultiple", 6: "SizeOverflow", 7: "InvalidLength",
    8: "AllocationFailed", 9: "UnsupportedQuantization", 10: "UnsupportedWeightedQuantization",
    11: "ImportanceWeightsRequired", 12: "InvalidImportanceLength", 13: "InvalidImportanceWeight",
    14: "UnsupportedIntegerConversion", 15: "IntegerOutOfRange", 16: "NonFiniteInput",
    17: "UnrepresentableScale", 18: "DeviceError", 19: "Unimplemented", 20: "InvalidArgument",
    21: "InvalidConfig", 22: "InvalidToken", 23: "InvalidState",
    24: "Shape", 25: "Bounds", 26: "Unsupported",
    27: "GgufIo", 28: "GgufInvalid", 29: "GgufLimit", 30: "GgufUnsupported",
    31: "NonFinite", 32: "ScratchLimit",
}
F32 = 0
SHAPE, BOUNDS, UNSUPPORTED = 24, 25, 26


class OracleError(Exception):
    def __init__(self, code, dtype, a, b):
        self.code, self.dtype, self.a, self.b = code, dtype, a, b
        super().__init__(f"{ERROR_NAMES.get(code, code)}(dtype={dtype}, a={a}, b={b})")

    @property
    def name(self):
        return ERROR_NAMES.get(self.code, str(self.code))


class _Err(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("dtype", ctypes.c_uint32),
                ("a", ctypes.c_uint64), ("b", ctypes.c_uint64)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `make -C oracle`")
    lib = ctypes.CDLL(LIB_PATH)
    P, U64, U32, I = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
    E = ctypes.POINTER(_Err)
    lib.oracle_f16_to_f32.argtypes, lib.oracle_f16_to_f32.restype = [ctypes.c_uint16], ctypes.c_float
    lib.oracle_f32_to_f16.argtypes, lib.oracle_f32_to_f16.restype = [ctypes.c_float], ctypes.c_uint16
    lib.oracle_row_bytes.argtypes = [U32, U64, ctypes.POINTER(U64), E]
    lib.oracle_matvec_activation_dtype.argtypes = [U32, ctypes.POINTER(U32), E]
    lib.oracle_quantize_into.argtypes = [U32, P, U64, P, U64, E]
    lib.oracle_dequantize_into.argtypes = [U32, P, U64, P, U64, E]
    lib.oracle_dot_packed.argtypes = [U32, P, U64, P, U64, U64, ctypes.POINTER(ctypes.c_float), E]
    lib.oracle_matvec.argtypes = [U32, P, U64, U64, U64, P, U64, P, I, E]
    lib.oracle_matmul.argtypes = [U32, P, U64, U64, U64, P, U64, P, I, E]
    lib.oracle_block_sums.argtypes = [U32, P, P, U64, P, P]
    lib.oracle_block_sums.restype = None
    lib.oracle_argmax.argtypes, lib.oracle_argmax.restype = [P, U64], U64
    lib.oracle_abs_terms.argtypes, lib.oracle_abs_terms.restype = [U32, P, P, U64], ctypes.c_double
    F = ctypes.c_float
    lib.oracle_sse2_exp.argtypes, lib.oracle_sse2_exp.restype = [F], F
    lib.oracle_silu.argtypes, lib.oracle_silu.restype = [P, U64], None
    lib.oracle_softmax.argtypes, lib.oracle_softmax.restype = [P, U64], ctypes.c_int
    lib.oracle_rms_norm.argtypes, lib.oracle_rms_norm.restype = [P, P, U64, F, P], ctypes.c_int
    lib.oracle_rope.argtypes, lib.oracle_rope.restype = [P, U64, U64, U64, F], None
    lib.oracle_rope_table.argtypes, lib.oracle_rope_table.restype = [U64, U64, F, P], None
    lib.oracle_attention.argtypes = [P, P, P, U64, U64, U64, U64, F, P]
    lib.oracle_attention.restype = ctypes.c_int
    lib.oracle_llama_embedding.argtypes, lib.oracle_llama_embedding.restype = [P, U32, P], ctypes.c_int
    lib.oracle_llama_step.argtypes = [P, P, U64, U64, P, P, P, I, E]
    lib.oracle_llama_step.restype = ctypes.c_int
    lib.oracle_llama_run_layer.argtypes = [P, U64, P, U64, U64, P, P, I, E]
    lib.oracle_llama_run_layer.restype = ctypes.c_int
    lib.oracle_llama_finish.argtypes = [P, P, P, P, I, E]
    lib.oracle_llama_finish.restype = ctypes.c_int
    for f in ("oracle_row_bytes", "oracle_matvec_activation_dtype", "oracle_quantize_into",
              "oracle_dequantize_into", "oracle_dot_packed", "oracle_matvec", "oracle_matmul"):
        getattr(lib, f).restype = ctypes.c_int
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None and a.size else None


def _check(rc, err):
    if rc != 0:
        raise OracleError(err.code, err.dtype, err.a, err.b)


def f16_to_f32(bits):
    return lib().oracle_f16_to_f32(int(bits))


def f32_to_f16(value):
    return lib().oracle_f32_to_f16(float(value))


def row_bytes(dtype, elements):
    out, err = ctypes.c_uint64(), _Err()
    _check(lib().oracle_row_bytes(dtype, elements, ctypes.byref(out), ctypes.byref(err)), err)
    return out.value


def matvec_activation_dtype(dtype):
    out, err = ctypes.c_uint32(), _Err()
    _check(lib().oracle_matvec_activation_dtype(dtype, ctypes.byref(out), ctypes.byref(err)), err)
    return out.value


def quantize_into(dtype, x, out):
    x = np.ascontiguousarray(x, dtype=np.float32)
    err = _Err()
    _check(lib().oracle_quantize_into(dtype, _ptr(x), x.size, _ptr(out), out.size, ctypes.byref(err)), err)
    return out


def quantize(dtype, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(row_bytes(dtype, x.size), dtype=np.uint8)
    return quantize_into(dtype, x, out)


def dequantize(dtype, b, n):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.zeros(n, dtype=np.float32)
    err = _Err()
    _check(lib().oracle_dequantize_into(dtype, _ptr(b), b.size, _ptr(out), n, ctypes.byref(err)), err)
    return out


def dot_packed(dtype, w, act, elements):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    act = np.ascontiguousarray(act, dtype=np.uint8)
    out, err = ctypes.c_float(), _Err()
    _check(lib().oracle_dot_packed(dtype, _ptr(w), w.size, _ptr(act), act.size, elements,
                                   ctypes.byref(out), ctypes.byref(err)), err)
    return np.float32(out.value)


def matvec(dtype, w, rows, cols, x, threads=1):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(rows, dtype=np.float32) if rows < (1 << 40) else None
    err = _Err()
    rc = lib().oracle_matvec(dtype, _ptr(w), w.size, rows, cols, _ptr(x), x.size,
                             _ptr(y) if y is not None else ctypes.c_void_p(1), threads,
                             ctypes.byref(err))
    _check(rc, err)
    return y


def matmul(dtype, w, rows, cols, x, threads=1):
    """x is [batch, cols] f32; returns [batch, rows] f32 (GGML MUL_MAT order)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    y = np.zeros((x.shape[0], rows), dtype=np.float32)
    err = _Err()
    _check(lib().oracle_matmul(dtype, _ptr(w), w.size, rows, cols, _ptr(x), x.shape[0], _ptr(y),
                               threads, ctypes.byref(err)), err)
    return y


# ---- GGML MUL_MAT with broadcast and MUL_MAT_ID over quantized weights ------------
# Loops over the C dot above; the error payloads add the failing column
# (b) to the reference's QuantError, as the device API reports it.

def _rhs_rows(at, x_dtype, x, cols, n):
    """The n right-hand rows as activation bytes: packed rows as given, or
    each f32 row quantized in order (cpu_extra.rs:815-822, cpu_index.rs:209-214)."""
    arb = row_bytes(at, cols)
    if x_dtype == at:
        return np.ascontiguousarray(x, dtype=np.uint8).reshape(n, arb)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(n, cols)
    out = np.zeros((n, arb), np.uint8)
    for c in range(n):
        try:
            out[c] = quantize(at, x[c])
        except OracleError as e:
            raise OracleError(e.code, e.dtype, e.a, c) from None
    return out


def mul_mat(wtype, w, rows, cols, wn2, wn3, x_dtype, x, ncols, n2, n3):
    """crates/tensor/src/cpu_extra.rs:756-873 for quantized weights: w holds
    wn3 x wn2 matrices of rows x cols (GGUF rows, contiguous), x the right-hand
    side [n3][n2][ncols][cols] (f32, or rows of the activation type).
    Returns y [n3][n2][ncols][rows] f32: y[i3,i2,c,r] = dot_packed(row r of
    matrix (i2 / (n2/wn2), i3 / (n3/wn3)), column (i3, i2, c))."""
    at = matvec_activation_dtype(wtype)                                    # :758
    if cols == 0 or wn2 == 0 or wn3 == 0 or n2 % wn2 or n3 % wn3:          # :759-769
        raise OracleError(SHAPE, wtype, n2, n3)
    if x_dtype not in (F32, at):                                           # :779-784
        raise OracleError(UNSUPPORTED, x_dtype, 0, 0)
    n = ncols * n2 * n3
    y = np.zeros((n3, n2, ncols, rows), np.float32)
    if n == 0:
        return y
    right = _rhs_rows(at, x_dtype, x, cols, n)
    rb = row_bytes(wtype, cols)
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(wn3, wn2, rows, rb)
    r2, r3 = n2 // wn2, n3 // wn3
    for i3 in range(n3):                                                   # :811-869
        for i2 in range(n2):
            mat = w[i3 // r3, i2 // r2]
            for c in range(ncols):
                col = right[(i3 * n2 + i2) * ncols + c]
                for r in range(rows):
                    y[i3, i2, c, r] = dot_packed(wtype, mat[r], col, cols)
    return y


def mul_mat_id(wtype, w, rows, cols, experts, x_dtype, x, ncols, tokens, ids):
    """crates/tensor/src/cpu_index.rs:169-236 for quantized experts: w holds
    `experts` matrices of rows x cols, x [tokens][ncols][cols], ids
    [tokens][slots] int32.  Returns y [tokens][slots][rows] f32 with
    y[t,s] = expert ids[t,s] . column (t, s % ncols), zero for id -1."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(tokens, -1) if tokens else np.zeros((0, 0), np.int32)
    slots = ids.shape[1]
    at = matvec_activation_dtype(wtype)                                    # :173
    if cols == 0 or experts == 0 or ncols == 0 or slots % ncols:           # :179-194
        raise OracleError(SHAPE, wtype, slots, ncols)
    if x_dtype not in (F32, at):                                           # :195-199
        raise OracleError(UNSUPPORTED, x_dtype, 0, 0)
    flat = ids.reshape(-1)
    bad = np.nonzero((flat < -1) | (flat >= experts))[0]                   # :200-205
    if bad.size:
        raise OracleError(BOUNDS, wtype, int(bad[0]), 0)
    y = np.zeros((tokens, slots, rows), np.float32)                       # :206-209
    if y.size == 0:
        return y
    right = _rhs_rows(at, x_dtype, x, cols, tokens * ncols)               # :210-216
    rb = row_bytes(wtype, cols)
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(experts, rows, rb)
    for t in range(tokens):                                                # :219-233
        for s_ in range(slots):
            e = int(ids[t, s_])
            if e == -1:
                continue
            col = right[t * ncols + s_ % ncols]
            for r in range(rows):
                y[t, s_, r] = dot_packed(wtype, w[e, r], col, cols)
    return y


def block_sums(dtype, w_row, act_row, nblocks):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    act_row = np.ascontiguousarray(act_row, dtype=np.uint8)
    isum = np.zeros(nblocks, dtype=np.int32)
    imin = np.zeros(nblocks, dtype=np.int32)
    lib().oracle_block_sums(dtype, _ptr(w_row), _ptr(act_row), nblocks, _ptr(isum), _ptr(imin))
    return isum, imin


def abs_terms(dtype, w_row, act_row, nblocks):
    """Sum of |term| over every f32 term of one row's dot (tolerance helper)."""
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    act_row = np.ascontiguousarray(act_row, dtype=np.uint8)
    return float(lib().oracle_abs_terms(dtype, _ptr(w_row), _ptr(act_row), nblocks))


def order_tolerance(dtype, w, rows, act, nblocks):
    """Per-row bound on the difference between two f32 summation orders of
    the same dot: 2 * (n + 8) * 2^-24 * abs_terms, where n = nblocks * 2 + 16
    bounds the additions any one term passes through in either order (the
    reference's eight serial lanes, a blocked GPU partial sum and its
    reduction tree) and 8 covers the rounding of each term itself."""
    stride = w.size // rows
    n = 2 * nblocks + 16
    return np.array([2.0 * (n + 8) * 2.0 ** -24 * abs_terms(dtype, w[r * stride:(r + 1) * stride], act, nblocks)
                     for r in range(rows)])


def argmax(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().oracle_argmax(_ptr(x), x.size))


# ---- dense Llama decode step (rlq_oracle_llama.c) ---------------------------

def _f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _rc(rc):
    if rc != 0:
        raise OracleError(rc, 0, 0, 0)


def sse2_exp(x):
    """cpu_math.rs:94-123, one lane."""
    return np.float32(lib().oracle_sse2_exp(float(x)))


def silu(v):
    """cpu_math.rs:28-53 (SSE2 policy) on a copy."""
    v = _f32c(v).copy()
    lib().oracle_silu(_ptr(v), v.size)
    return v


def softmax(v):
    """math.rs:293-318 on a copy."""
    v = _f32c(v).copy()
    _rc(lib().oracle_softmax(_ptr(v), v.size))
    return v


def rms_norm(x, w, eps):
    """math.rs:214-228."""
    x, w = _f32c(x), _f32c(w)
    out = np.zeros_like(x)
    _rc(lib().oracle_rms_norm(_ptr(x), _ptr(w), x.size, float(eps), _ptr(out)))
    return out


def rope(v, head_dim, position, base):
    """math.rs:322-334 on a copy."""
    v = _f32c(v).copy()
    lib().oracle_rope(_ptr(v), v.size, int(head_dim), int(position), float(base))
    return v


def rope_table(head_dim, position, base):
    t = np.zeros(int(head_dim), dtype=np.float32)
    lib().oracle_rope_table(int(head_dim), int(position), float(base), _ptr(t))
    return t


def attention(q, keys, values, count, heads, kv_heads, head_dim, scale):
    """math.rs:427-497 with the contiguous padded layout."""
    q, keys, values = _f32c(q), _f32c(keys), _f32c(values)
    out = np.zeros(int(heads) * int(head_dim), dtype=np.float32)
    _rc(lib().oracle_attention(_ptr(q), _ptr(keys), _ptr(values), int(count), int(heads), int(kv_heads),
                               int(head_dim), float(scale), _ptr(out)))
    return out


LAYER_FIELDS = ("attention_norm", "query", "key", "value", "attention_output", "feed_forward_norm", "gate", "up",
                "down")


# the seven matrices in the order of a layer's per-matrix type array
MATRIX_FIELDS = ("query", "key", "value", "attention_output", "gate", "up", "down")


class _Layer(ctypes.Structure):
    _fields_ = [(f, ctypes.c_void_p) for f in LAYER_FIELDS] + [("types", ctypes.c_uint32 * 7)]


def layer_types(L):
    """A layer dict's optional per-matrix types ({name: type}), 0 = the
    model's weight_type."""
    t = L.get("types", {})
    return [int(t.get(f, 0)) for f in MATRIX_FIELDS]


class _Model(ctypes.Structure):
    _fields_ = [("vocab", ctypes.c_uint64), ("width", ctypes.c_uint64), ("feed_forward", ctypes.c_uint64),
                ("heads", ctypes.c_uint64), ("kv_heads", ctypes.c_uint64), ("max_context", ctypes.c_uint64),
                ("n_layers", ctypes.c_uint64), ("rms_epsilon", ctypes.c_float), ("rope_base", ctypes.c_float),
                ("attention_scale", ctypes.c_float), ("weight_type", ctypes.c_uint32),
                ("output_type", ctypes.c_uint32), ("embedding_type", ctypes.c_uint32),
                ("embedding", ctypes.c_void_p), ("output_norm", ctypes.c_void_p), ("output", ctypes.c_void_p),
                ("layers", ctypes.POINTER(_Layer))]


class LlamaOracle:
    """LlamaModel (crates/model-runtime/src/llama.rs) restated on the CPU with
    its own f32 KV cache.  `cfg` has the LlamaConfig fields and the tensor
    types; `tensors` is the dict of numpy arrays the GPU model takes."""

    def __init__(self, cfg, tensors, threads=8):
        self.cfg, self.threads = cfg, threads
        keep = self._keep = []

        def p(a, f32):
            a = np.ascontiguousarray(a, dtype=np.float32 if f32 else np.uint8)
            keep.append(a)
            return a.ctypes.data_as(ctypes.c_void_p)

        n = len(tensors["layers"])
        self._layers = (_Layer * max(1, n))()
        for i, L in enumerate(tensors["layers"]):
            for f in LAYER_FIELDS:
                setattr(self._layers[i], f, p(L[f], f.endswith("norm")))
            for k, ty in enumerate(layer_types(L)):
                self._layers[i].types[k] = ty
        self._m = _Model(cfg.vocabulary, cfg.width, cfg.feed_forward, cfg.heads, cfg.kv_heads, cfg.max_context, n,
                         cfg.rms_epsilon, cfg.rope_base, cfg.attention_scale, cfg.weight_type, cfg.output_type,
                         cfg.embedding_type, p(tensors["embedding"], False), p(tensors["output_norm"], True),
                         p(tensors["output"], False), self._layers)
        hd = cfg.width // cfg.heads
        kvw = cfg.kv_heads * hd
        self.k_cache = np.zeros((max(1, n), cfg.max_context, kvw), dtype=np.float32)
        self.v_cache = np.zeros_like(self.k_cache)
        self.cached = 0

    def embedding(self, token):
        out = np.zeros(self.cfg.width, dtype=np.float32)
        _rc(lib().oracle_llama_embedding(ctypes.byref(self._m), int(token), _ptr(out)))
        return out

    def step(self, hidden, position):
        """Returns (last layer output, logits); appends one KV row."""
        h = _f32c(hidden).copy()
        logits = np.zeros(self.cfg.vocabulary, dtype=np.float32)
        err = _Err()
        rc = lib().oracle_llama_step(ctypes.byref(self._m), _ptr(h), int(position), self.cached,
                                     _ptr(self.k_cache), _ptr(self.v_cache), _ptr(logits), self.threads,
                                     ctypes.byref(err))
        self.cached += 1
        if rc != 0:  # NonFinite: a = the check, b = the layer; a quantizer's QuantError: b = the layer
            raise OracleError(rc, err.dtype, err.a, err.b)
        return h, logits

    def layer(self, index, hidden, position):
        """Layer `index` alone over a copy of hidden at `position`, writing
        that layer's KV row `cached` (advance() moves to the next row once
        every layer of a step has run)."""
        h = _f32c(hidden).copy()
        err = _Err()
        rc = lib().oracle_llama_run_layer(ctypes.byref(self._m), int(index), _ptr(h), int(position), self.cached,
                                      _ptr(self.k_cache), _ptr(self.v_cache), self.threads, ctypes.byref(err))
        if rc != 0:
            raise OracleError(rc, err.dtype, err.a, err.b)
        return h

    def advance(self):
        self.cached += 1

    def finish(self, hidden):
        """finish_hidden of a last-layer output: (embedding, logits)."""
        h = _f32c(hidden)
        emb = np.zeros(self.cfg.width, dtype=np.float32)
        logits = np.zeros(self.cfg.vocabulary, dtype=np.float32)
        err = _Err()
        rc = lib().oracle_llama_finish(ctypes.byref(self._m), _ptr(h), _ptr(emb), _ptr(logits), self.threads,
                                       ctypes.byref(err))
        if rc != 0:
            raise OracleError(rc, err.dtype, err.a, err.b)
        return emb, logits
