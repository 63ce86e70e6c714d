"""rust-llama_amd: MI355X (gfx950) drop-in for rust-llama's quantized matvec path.

Python mirror of the reference crate `llama-quant` (crates/quant/src/lib.rs:36-41)
over the C ABI in include/rlq.h (librlq.so).  Names, argument meaning and error
behaviour follow the Rust API:

    matvec(DType, weights, rows, cols, input) -> f32[rows]      matvec.rs:24-87
    dot_packed(DType, weights, activation, elements) -> f32     matvec.rs:90-103
    matvec_activation_dtype(DType) -> DType                      matvec.rs:7-18
    quantize(DType, values) / quantize_into(DType, values, out)  encode.rs:10-100
    dequantize(DType, bytes, elements) / dequantize_into         lib.rs:288-308
    DType, QuantError                                            lib.rs:45-169

Errors raise QuantError with the reference variant's name and payload.
Every computation runs on the GPU through librlq.so; there is no CPU path, and
importing this package fails if the library has not been built
(`python rust-llama_amd/build.py`).

The device API (Context, Weights) keeps weights resident in HBM and takes
torch tensors on the GPU; torch supplies device memory and streams only.
LlamaModel mirrors model-runtime's LlamaModel (crates/model-runtime/src/
llama.rs): embedding(token) and step(hidden, position) -> (embedding, logits)
over quantized matrices and a resident f32 KV cache.
"""
import atexit
import ctypes
import enum
import os

import numpy as np

try:  # load torch's HIP runtime first so librlq.so binds to the same one
    import torch
except ImportError:  # pragma: no cover - the host API still works without torch
    torch = None

HERE = os.path.dirname(os.path.abspath(__file__))
# RLQ_LIB_PATH selects another build of the library (the host-sanitizer build
# of `build.py --sanitize`, for CPU test runs)
LIB_PATH = os.environ.get("RLQ_LIB_PATH") or os.path.join(HERE, "librlq.so")


class DType(enum.IntEnum):
    """GGML numeric type ids (crates/quant/src/lib.rs:132-169)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    IQ1_M = 29
    BF16 = 30
    TQ1_0 = 34
    TQ2_0 = 35
    MXFP4 = 39
    NVFP4 = 40
    Q1_0 = 41
    Q2_0 = 42
    F8_E4M3 = 43


# Status codes: QuantError variants in declaration order (lib.rs:45-63), then
# this library's own.
ERROR_NAMES = {
    1: "InvalidType", 2: "UnsupportedMatVec", 3: "InvalidVectorLength", 4: "InvalidMatrixShape",
    5: "NonMultiple", 6: "SizeOverflow", 7: "InvalidLength", 8: "AllocationFailed",
    9: "UnsupportedQuantization", 10: "UnsupportedWeightedQuantization",
    11: "ImportanceWeightsRequired", 12: "InvalidImportanceLength", 13: "InvalidImportanceWeight",
    14: "UnsupportedIntegerConversion", 15: "IntegerOutOfRange", 16: "NonFiniteInput",
    17: "UnrepresentableScale", 18: "DeviceError", 19: "Unimplemented", 20: "InvalidArgument",
    21: "InvalidConfig", 22: "InvalidToken", 23: "InvalidState",
    24: "Shape", 25: "Bounds", 26: "Unsupported",
    27: "GgufIo", 28: "GgufInvalid", 29: "GgufLimit", 30: "GgufUnsupported",
    31: "NonFinite", 32: "ScratchLimit",
}

# NonFinite checks (QuantError.a of a NonFinite error): the names the
# reference's model-runtime reports
NONFINITE_CHECKS = {1: "RMS normalization scale", 2: "RMS normalization output", 3: "matrix input",
                    4: "matrix output", 5: "attention score", 6: "attention output", 7: "Llama layer output"}


class QuantError(Exception):
    """A QuantError variant: `name`, numeric `code`, `dtype` and the payload
    fields of the variant (index, block, expected/actual, rows/cols...)."""

    def __init__(self, code, dtype, a, b, message):
        self.code, self.dtype, self.a, self.b = code, dtype, a, b
        self.name = ERROR_NAMES.get(code, str(code))
        super().__init__(f"{self.name}: {message} (dtype={dtype}, a={a}, b={b})")

    @property
    def index(self):  # NonFiniteInput{index}
        return self.a

    @property
    def block(self):  # UnrepresentableScale{block}
        return self.a

    @property
    def expected(self):  # InvalidVectorLength / InvalidLength
        return self.a

    @property
    def actual(self):
        return self.b


class _Err(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int32), ("dtype", ctypes.c_uint32), ("a", ctypes.c_uint64),
                ("b", ctypes.c_uint64)]


# Every entry point of include/rlq.h with its ctypes signature.
_P, _U64, _U32, _I32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int32
_E = ctypes.POINTER(_Err)
SIGNATURES = {
    "rlq_status_string": ([_I32], ctypes.c_char_p),
    "rlq_row_bytes": ([_U32, _U64, ctypes.POINTER(_U64), _E], _I32),
    "rlq_matvec_activation_dtype": ([_U32, ctypes.POINTER(_U32), _E], _I32),
    "rlq_quantize_into": ([_U32, _P, _U64, _P, _U64, _E], _I32),
    "rlq_dequantize_into": ([_U32, _P, _U64, _P, _U64, _E], _I32),
    "rlq_dot_packed": ([_U32, _P, _U64, _P, _U64, _U64, ctypes.POINTER(ctypes.c_float), _E], _I32),
    "rlq_matvec": ([_U32, _P, _U64, _U64, _U64, _P, _U64, _P, _E], _I32),
    "rlq_context_create": ([_I32, ctypes.POINTER(_P), _E], _I32),
    "rlq_context_destroy": ([_P], None),
    "rlq_context_stream": ([_P], _P),
    "rlq_weights_create": ([_P, _U32, _P, _U64, _U64, _U64, _I32, ctypes.POINTER(_P), _E], _I32),
    "rlq_weights_create_stacked": ([_P, _U32, _P, _U64, _U64, _U64, _U64, _U64, _I32, ctypes.POINTER(_P), _E],
                                   _I32),
    "rlq_weights_destroy": ([_P], None),
    "rlq_weights_shape": ([_P, ctypes.POINTER(_U64), ctypes.POINTER(_U64), ctypes.POINTER(_U32)], None),
    "rlq_weights_stack": ([_P, ctypes.POINTER(_U64), ctypes.POINTER(_U64)], None),
    "rlq_mul_mat": ([_P, _P, _U32, _P, _U64, _U64, _U64, _P, _P, _E], _I32),
    "rlq_mul_mat_id": ([_P, _P, _U32, _P, _U64, _U64, _P, _U64, _P, _P, _E], _I32),
    "rlq_matmul": ([_P, _P, _P, _U64, _P, _P, _E], _I32),
    "rlq_multiply": ([_P, _P, _P, _P, _P, _E], _I32),
    "rlq_matmul_noalloc": ([_P, _P, _P, _U64, _P, _P, _P, _E], _I32),
    "rlq_matmul_argmax": ([_P, _P, _P, _U64, _P, _P, _P, _E], _I32),
    "rlq_quantize_device": ([_P, _U32, _P, _U64, _U64, _P, _P, _E], _I32),
    "rlq_sync": ([_P, _P, _E], _I32),
    "rlq_block_sums": ([_P, _P, _P, _U64, _P, _P, _P, _E], _I32),
    "rlq_block_sums_ex": ([_P, _P, _P, _U64, _U32, _P, _P, _P, _P, _E], _I32),
    "rlq_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(_P), _E], _I32),
    "rlq_gguf_read_header_memory": ([_P, _U64, ctypes.POINTER(_P), _E], _I32),
    "rlq_gguf_close": ([_P], None),
    "rlq_gguf_header": ([_P, ctypes.POINTER(_U32), ctypes.POINTER(_U32), ctypes.POINTER(_U64), ctypes.POINTER(_U64),
                         ctypes.POINTER(_U64), ctypes.POINTER(_I32)], None),
    "rlq_gguf_kv_at": ([_P, _U64, ctypes.POINTER(_P), ctypes.POINTER(_U64), ctypes.POINTER(_U32),
                        ctypes.POINTER(_U32), ctypes.POINTER(_U64), _E], _I32),
    "rlq_gguf_kv_scalar": ([_P, _U64, _U64, ctypes.POINTER(_U64), _E], _I32),
    "rlq_gguf_kv_string": ([_P, _U64, _U64, ctypes.POINTER(_P), ctypes.POINTER(_U64), _E], _I32),
    "rlq_gguf_find_kv": ([_P, _P, _U64], ctypes.c_int64),
    "rlq_gguf_tensor_at": ([_P, _U64, ctypes.POINTER(_P), ctypes.POINTER(_U64), ctypes.POINTER(_U32), _P,
                            ctypes.POINTER(_U32), ctypes.POINTER(_U64), ctypes.POINTER(_U64), _E], _I32),
    "rlq_gguf_find_tensor": ([_P, _P, _U64], ctypes.c_int64),
    "rlq_gguf_read_tensor": ([_P, _U64, _P, _U64, _E], _I32),
    "rlq_gguf_native_header": ([_P, _P, _U64, ctypes.POINTER(_U64), _E], _I32),
    "rlq_gguf_write_header": ([_P, _U64, _P, _U64, _P, _U64, ctypes.POINTER(_U64), ctypes.POINTER(_U64), _E], _I32),
    "rlq_gguf_write": ([ctypes.c_char_p, _P, _U64, _P, _U64, _E], _I32),
    "rlq_llama_create": ([_P, _P, _P, ctypes.POINTER(_P), _E], _I32),
    "rlq_llama_create_from_gguf": ([_P, ctypes.c_char_p, _U64, ctypes.POINTER(_P), _E], _I32),
    "rlq_llama_config_of": ([_P, _P], None),
    "rlq_llama_destroy": ([_P], None),
    "rlq_llama_truncate": ([_P, _U64, _E], _I32),
    "rlq_llama_cached": ([_P], _U64),
    "rlq_llama_embedding": ([_P, _U32, _P, _P, _E], _I32),
    "rlq_llama_step": ([_P, _P, _U64, _P, _P, _P, _P, _E], _I32),
    "rlq_llama_intermediates": ([_P, _P, _P, _P, _P, _P, _E], _I32),
    "rlq_llama_trace": ([_P, _P, _E], _I32),
    "rlq_probe_mfma": ([_U32, _U32, _U32, _P, _P], _I32),
    "rlq_probe_stream": ([_P, _U64, _U32, _P, _P], _I32),
    "rlq_probe_stream_shape": ([_P, _U64, _U32, _U32, _U32, _U32, _P, _P], _I32),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python rust-llama_amd/build.py`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        f = getattr(lib, name)
        f.argtypes, f.restype = args, res
    return lib


_lib = _load()

# Handles still alive when the interpreter exits are left to the process
# teardown: HIP calls from finalizers after torch has shut its runtime down are
# not safe.
_exiting = False


def _at_exit():
    global _exiting
    _exiting = True


atexit.register(_at_exit)


def lib():
    return _lib


def _check(rc, err):
    if rc != 0:
        msg = _lib.rlq_status_string(err.code).decode()
        raise QuantError(err.code, err.dtype, err.a, err.b, msg)


def _u8(a):
    a = np.ascontiguousarray(a)
    if a.dtype != np.uint8:
        a = a.view(np.uint8).reshape(-1) if a.dtype.itemsize == 1 else np.frombuffer(a.tobytes(), np.uint8)
    return a.reshape(-1)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a.size else None


# ---- metadata --------------------------------------------------------------

def row_bytes(dtype, elements):
    """DType::row_bytes (lib.rs:274-285)."""
    out, err = ctypes.c_uint64(), _Err()
    _check(_lib.rlq_row_bytes(int(dtype), int(elements), ctypes.byref(out), ctypes.byref(err)), err)
    return out.value


def matvec_activation_dtype(weights_type):
    out, err = ctypes.c_uint32(), _Err()
    _check(_lib.rlq_matvec_activation_dtype(int(weights_type), ctypes.byref(out), ctypes.byref(err)), err)
    return DType(out.value)


# ---- host drop-ins (synchronous) -----------------------------------------------

def quantize_into(dtype, values, out):
    values = _f32(values)
    if not (isinstance(out, np.ndarray) and out.dtype == np.uint8 and out.flags.c_contiguous):
        raise TypeError("out must be a contiguous uint8 numpy array")
    err = _Err()
    _check(_lib.rlq_quantize_into(int(dtype), _ptr(values), values.size, _ptr(out), out.size,
                                  ctypes.byref(err)), err)
    return out


def quantize(dtype, values):
    values = _f32(values)
    out = np.zeros(row_bytes(dtype, values.size), dtype=np.uint8)
    return quantize_into(dtype, values, out)


def dequantize_into(dtype, data, out):
    data = _u8(data)
    if not (isinstance(out, np.ndarray) and out.dtype == np.float32 and out.flags.c_contiguous):
        raise TypeError("out must be a contiguous float32 numpy array")
    err = _Err()
    _check(_lib.rlq_dequantize_into(int(dtype), _ptr(data), data.size, _ptr(out), out.size,
                                    ctypes.byref(err)), err)
    return out


def dequantize(dtype, data, elements):
    return dequantize_into(dtype, data, np.zeros(int(elements), dtype=np.float32))


def dot_packed(weights_type, weights, activation, elements):
    weights, activation = _u8(weights), _u8(activation)
    out, err = ctypes.c_float(), _Err()
    _check(_lib.rlq_dot_packed(int(weights_type), _ptr(weights), weights.size, _ptr(activation),
                               activation.size, int(elements), ctypes.byref(out), ctypes.byref(err)), err)
    return np.float32(out.value)


def matvec(weights_type, weights, rows, cols, input):
    weights, input = _u8(weights), _f32(input)
    out = np.zeros(int(rows) if int(rows) < (1 << 34) else 0, dtype=np.float32)
    err = _Err()
    outp = _ptr(out) if out.size else ctypes.c_void_p(16)  # never written unless shapes validate
    _check(_lib.rlq_matvec(int(weights_type), _ptr(weights), weights.size, int(rows), int(cols),
                           _ptr(input), input.size, outp, ctypes.byref(err)), err)
    return out


# ---- device API -------------------------------------------------------------

def _dev_ptr(t, dtype):
    if torch is None or not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError("expected a torch tensor on the GPU")
    if t.dtype != dtype or not t.is_contiguous():
        raise TypeError(f"expected a contiguous {dtype} tensor")
    return ctypes.c_void_p(t.data_ptr())


def _stream_ptr(stream):
    if stream is None:
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(stream if isinstance(stream, int) else stream.cuda_stream)


class Context:
    """rlq_context: device scratch, the context's own stream and the device
    error word.  Kernels run on torch's current stream unless one is given."""

    def __init__(self, device=-1):
        if device >= 0 and torch is not None:
            torch.cuda.set_device(device)
        h, err = ctypes.c_void_p(), _Err()
        _check(_lib.rlq_context_create(int(device), ctypes.byref(h), ctypes.byref(err)), err)
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            if _exiting is False:  # None once module teardown has cleared the globals
                _lib.rlq_context_destroy(self._h)
            self._h = None

    __del__ = close

    def matmul(self, w, x, y=None, stream=None):
        """MUL_MAT / Matrix::multiply: x [batch, cols] f32 -> y [batch, rows] f32."""
        x2 = x.reshape(-1, w.cols)
        if y is None:
            y = torch.empty((x2.shape[0], w.rows), dtype=torch.float32, device=x.device)
        err = _Err()
        _check(_lib.rlq_matmul(self._h, w._h, _dev_ptr(x2, torch.float32), x2.shape[0],
                               _dev_ptr(y, torch.float32), _stream_ptr(stream), ctypes.byref(err)), err)
        return y

    def multiply(self, w, x, y=None, stream=None):
        """Matrix::multiply (math.rs:144-169): one input vector x [cols] ->
        y [rows], with the reference's finite checks of the input and the
        output (NonFinite errors at sync)."""
        if y is None:
            y = torch.empty(w.rows, dtype=torch.float32, device=x.device)
        err = _Err()
        _check(_lib.rlq_multiply(self._h, w._h, _dev_ptr(x, torch.float32), _dev_ptr(y, torch.float32),
                                 _stream_ptr(stream), ctypes.byref(err)), err)
        return y

    def matmul_argmax(self, w, x, y=None, argmax=None, stream=None):
        """matmul followed by the greedy sampler's index per column."""
        x2 = x.reshape(-1, w.cols)
        batch = x2.shape[0]
        if y is None:
            y = torch.empty((batch, w.rows), dtype=torch.float32, device=x.device)
        if argmax is None:
            argmax = torch.empty(batch, dtype=torch.int32, device=x.device)
        err = _Err()
        _check(_lib.rlq_matmul_argmax(self._h, w._h, _dev_ptr(x2, torch.float32), batch,
                                      _dev_ptr(y, torch.float32), _dev_ptr(argmax, torch.int32),
                                      _stream_ptr(stream), ctypes.byref(err)), err)
        return y, argmax

    def bind_matmul(self, w, x, y, argmax=None, stream=None):
        """A prepared matmul (or matmul_argmax when argmax is given): the
        tensors, the stream (torch's current one when None, taken now) and
        the error record are resolved once, and the returned function of no
        arguments launches the same call again with only the C call's own
        cost (for serving loops; it raises like matmul).  The tensors stay
        referenced by the function."""
        x2 = x.reshape(-1, w.cols)
        batch = x2.shape[0]
        if y.numel() != batch * w.rows:
            raise ValueError("y must hold batch * rows f32 values")
        err = _Err()
        ref = ctypes.byref(err)
        h, wh = self._h, w._h
        xp, yp, sp = _dev_ptr(x2, torch.float32), _dev_ptr(y, torch.float32), _stream_ptr(stream)
        keep = (w, x2, y, argmax)
        if argmax is None:
            fn = _lib.rlq_matmul

            def call():
                rc = fn(h, wh, xp, batch, yp, sp, ref)
                if rc:
                    _check(rc, err)
        else:
            fn, ap = _lib.rlq_matmul_argmax, _dev_ptr(argmax, torch.int32)

            def call():
                rc = fn(h, wh, xp, batch, yp, ap, sp, ref)
                if rc:
                    _check(rc, err)
        call.tensors = keep
        return call

    def matmul_noalloc(self, w, x, y, argmax=None, stream=None):
        """rlq_matmul_noalloc: matmul (argmax None) or matmul_argmax into the
        caller's y [batch, rows] (and argmax [batch] int32), with the
        library's static device scratch instead of any allocation."""
        x2 = x.reshape(-1, w.cols)
        err = _Err()
        _check(_lib.rlq_matmul_noalloc(self._h, w._h, _dev_ptr(x2, torch.float32), x2.shape[0],
                                       _dev_ptr(y, torch.float32),
                                       _dev_ptr(argmax, torch.int32) if argmax is not None else None,
                                       _stream_ptr(stream), ctypes.byref(err)), err)
        return y, argmax

    def quantize(self, dtype, x, stream=None):
        """GPU quantize_into for Q8_0 / Q8_K: x [batch, cols] -> GGUF bytes."""
        x2 = x.reshape(x.shape[0] if x.dim() > 1 else 1, -1)
        cols = x2.shape[1]
        out = torch.empty(x2.shape[0] * row_bytes(dtype, cols), dtype=torch.uint8, device=x.device)
        err = _Err()
        _check(_lib.rlq_quantize_device(self._h, int(dtype), _dev_ptr(x2, torch.float32), cols, x2.shape[0],
                                        _dev_ptr(out, torch.uint8), _stream_ptr(stream), ctypes.byref(err)), err)
        return out

    def mul_mat(self, w, x, x_dtype=DType.F32, y=None, stream=None):
        """GGML MUL_MAT with broadcast (cpu_extra.rs:756-873): w stacked
        [w.n3][w.n2] matrices; x [n3, n2, ncols, cols] f32, or uint8 rows of the
        activation type when x_dtype is it -> y [n3, n2, ncols, rows] f32."""
        x_dtype = DType(x_dtype)
        if x.dim() != 4:
            raise ValueError("x must be [n3, n2, ncols, cols] (f32) or [n3, n2, ncols, row bytes] (uint8)")
        n3, n2, ncols = x.shape[:3]
        if y is None:
            y = torch.empty((n3, n2, ncols, w.rows), dtype=torch.float32, device=x.device)
        xp = _dev_ptr(x, x.dtype)  # the library checks x_dtype against the weights
        err = _Err()
        _check(_lib.rlq_mul_mat(self._h, w._h, int(x_dtype), xp, ncols, n2, n3, _dev_ptr(y, torch.float32),
                                _stream_ptr(stream), ctypes.byref(err)), err)
        return y

    def mul_mat_id(self, w, x, ids, x_dtype=DType.F32, y=None, stream=None):
        """GGML MUL_MAT_ID (cpu_index.rs:169-236): experts w [w.n2 matrices],
        x [tokens, ncols, cols] f32 (or activation bytes), ids [tokens, slots]
        int32 on the GPU -> y [tokens, slots, rows] f32 (0 where ids is -1)."""
        x_dtype = DType(x_dtype)
        tokens, ncols = x.shape[:2]
        slots = ids.shape[1]
        if y is None:
            y = torch.empty((tokens, slots, w.rows), dtype=torch.float32, device=x.device)
        xp = _dev_ptr(x, x.dtype)
        err = _Err()
        _check(_lib.rlq_mul_mat_id(self._h, w._h, int(x_dtype), xp, ncols, tokens, _dev_ptr(ids, torch.int32),
                                   slots, _dev_ptr(y, torch.float32), _stream_ptr(stream), ctypes.byref(err)), err)
        return y

    def sync(self, stream=None):
        """Wait for the stream; raise the first data error recorded on the GPU."""
        err = _Err()
        _check(_lib.rlq_sync(self._h, _stream_ptr(stream), ctypes.byref(err)), err)

    def block_sums(self, w, x, stream=None):
        """Exact per-(row, block) integer sums of w against column 0 of x
        ([batch, cols] or [cols], batch <= 8), from the kernel that matmul
        uses for that batch size."""
        x2 = x.reshape(-1, w.cols)
        nb = w.cols // (32 if w.dtype == DType.Q8_0 else 256)
        isum = torch.empty((w.rows, nb), dtype=torch.int32, device=x.device)
        imin = torch.empty((w.rows, nb), dtype=torch.int32, device=x.device)
        err = _Err()
        _check(_lib.rlq_block_sums(self._h, w._h, _dev_ptr(x2, torch.float32), x2.shape[0],
                                   _dev_ptr(isum, torch.int32), _dev_ptr(imin, torch.int32),
                                   _stream_ptr(stream), ctypes.byref(err)), err)
        return isum, imin

    SUMS_SILU_PAIR = 1

    def block_sums_ex(self, w, x, flags=0, stream=None):
        """block_sums plus the same launch's outputs: (isum, imin, y).  With
        flags=SUMS_SILU_PAIR the decode step's gate/up kernel runs over w (Q4_K
        / Q5_K rows whose 16-row tiles alternate gate and up) and y holds
        silu(gate) * up, rows / 2 values; otherwise y is [batch, rows]."""
        x2 = x.reshape(-1, w.cols)
        nb = w.cols // (32 if w.dtype == DType.Q8_0 else 256)
        isum = torch.empty((w.rows, nb), dtype=torch.int32, device=x.device)
        imin = torch.empty((w.rows, nb), dtype=torch.int32, device=x.device)
        n = w.rows // 2 if flags & self.SUMS_SILU_PAIR else x2.shape[0] * w.rows
        y = torch.empty(n, dtype=torch.float32, device=x.device)
        err = _Err()
        _check(_lib.rlq_block_sums_ex(self._h, w._h, _dev_ptr(x2, torch.float32), x2.shape[0], int(flags),
                                      _dev_ptr(isum, torch.int32), _dev_ptr(imin, torch.int32),
                                      _dev_ptr(y, torch.float32), _stream_ptr(stream), ctypes.byref(err)), err)
        return isum, imin, y


class Weights:
    """rlq_weights (Matrix::from_quantized, math.rs:35-70): GGUF bytes kept in
    HBM in the kernels' layout.  `data` is a numpy uint8 array (host) or a
    torch uint8 tensor on the GPU."""

    def __init__(self, ctx, dtype, data, rows, cols, n2=1, n3=1):
        err, h = _Err(), ctypes.c_void_p()
        if torch is not None and isinstance(data, torch.Tensor):
            ptr, n, on_dev = _dev_ptr(data.reshape(-1), torch.uint8), data.numel(), 1
        else:
            arr = _u8(data)
            ptr, n, on_dev, self._keep = _ptr(arr), arr.size, 0, arr
        _check(_lib.rlq_weights_create_stacked(ctx._h, int(dtype), ptr, n, int(rows), int(cols), int(n2), int(n3),
                                               on_dev, ctypes.byref(h), ctypes.byref(err)), err)
        self._h, self.ctx, self.dtype, self.rows, self.cols = h, ctx, DType(dtype), int(rows), int(cols)
        self.n2, self.n3 = int(n2), int(n3)
        self._keep = None

    def close(self):
        if getattr(self, "_h", None):
            if _exiting is False:  # None once module teardown has cleared the globals
                _lib.rlq_weights_destroy(self._h)
            self._h = None

    __del__ = close


# ---- dense Llama decode step ----------------------------------------------------

class LlamaConfig(ctypes.Structure):
    """LlamaConfig (crates/model-runtime/src/llama.rs:6-17) plus the tensor
    types; attention_scale 0 means 1/sqrt(head_dim)."""
    _fields_ = [("vocabulary", _U64), ("width", _U64), ("feed_forward", _U64), ("heads", _U64),
                ("kv_heads", _U64), ("max_context", _U64), ("n_layers", _U64), ("rms_epsilon", ctypes.c_float),
                ("rope_base", ctypes.c_float), ("attention_scale", ctypes.c_float), ("weight_type", _U32),
                ("output_type", _U32), ("embedding_type", _U32)]

    @property
    def head_dim(self):
        return self.width // self.heads

    @property
    def kv_width(self):
        return self.kv_heads * self.head_dim


class _LayerT(ctypes.Structure):
    _fields_ = [("attention_norm", _P), ("query", _P), ("key", _P), ("value", _P), ("attention_output", _P),
                ("feed_forward_norm", _P), ("gate", _P), ("up", _P), ("down", _P), ("types", _U32 * 7)]


# the seven matrices in the order of rlq_llama_layer.types
MATRIX_FIELDS = ("query", "key", "value", "attention_output", "gate", "up", "down")


class _TensorsT(ctypes.Structure):
    _fields_ = [("embedding", _P), ("output_norm", _P), ("output", _P), ("layers", ctypes.POINTER(_LayerT)),
                ("on_device", _I32)]


LAYER_FIELDS = ("attention_norm", "query", "key", "value", "attention_output", "feed_forward_norm", "gate", "up",
                "down")


class LlamaModel:
    """LlamaModel (llama.rs) on the GPU.  `tensors` is a dict with
    `embedding`, `output_norm`, `output` and `layers` (a list of dicts with
    LAYER_FIELDS and optionally `types`, {matrix name: dtype} for matrices
    not of config.weight_type): GGUF bytes of the matrices (rows contiguous)
    and f32 norm weights, either all numpy arrays or all torch tensors on the
    GPU.  The model keeps its own tiled copy; the tensors may be dropped
    afterwards.  LlamaModel.from_gguf loads a GGUF file instead."""

    @classmethod
    def from_gguf(cls, ctx, path, context_length):
        """rlq_llama_create_from_gguf: the inference crate's llama loader."""
        self = cls.__new__(cls)
        h, err = ctypes.c_void_p(), _Err()
        _check(_lib.rlq_llama_create_from_gguf(ctx._h, os.fsencode(path), int(context_length), ctypes.byref(h),
                                               ctypes.byref(err)), err)
        self._h, self.ctx, self.config = h, ctx, LlamaConfig()
        _lib.rlq_llama_config_of(h, ctypes.byref(self.config))
        return self

    def __init__(self, ctx, config, tensors):
        on_dev = torch is not None and isinstance(tensors["embedding"], torch.Tensor)
        keep = []

        def ptr(a, f32):
            if on_dev:
                return _dev_ptr(a.reshape(-1), torch.float32 if f32 else torch.uint8)
            arr = _f32(a) if f32 else _u8(a)
            keep.append(arr)
            return _ptr(arr)

        layers = (_LayerT * max(1, len(tensors["layers"])))()
        for i, L in enumerate(tensors["layers"]):
            for f in LAYER_FIELDS:
                setattr(layers[i], f, ptr(L[f], f.endswith("norm")))
            types = L.get("types", {})
            for k, f in enumerate(MATRIX_FIELDS):
                layers[i].types[k] = int(types.get(f, 0))
        t = _TensorsT(ptr(tensors["embedding"], False), ptr(tensors["output_norm"], True),
                      ptr(tensors["output"], False), layers, 1 if on_dev else 0)
        h, err = ctypes.c_void_p(), _Err()
        _check(_lib.rlq_llama_create(ctx._h, ctypes.byref(config), ctypes.byref(t), ctypes.byref(h),
                                     ctypes.byref(err)), err)
        self._h, self.ctx, self.config = h, ctx, config

    def close(self):
        if getattr(self, "_h", None):
            if _exiting is False:  # None once module teardown has cleared the globals
                _lib.rlq_llama_destroy(self._h)
            self._h = None

    __del__ = close

    @property
    def cached(self):
        """KV rows held: the insertion index of the next step."""
        return int(_lib.rlq_llama_cached(self._h))

    def truncate(self, rows=0):
        err = _Err()
        _check(_lib.rlq_llama_truncate(self._h, int(rows), ctypes.byref(err)), err)

    def embedding(self, token, out=None, stream=None):
        """LlamaModel::embedding (llama.rs:213-221) -> f32 [width] on the GPU."""
        if out is None:
            out = torch.empty(self.config.width, dtype=torch.float32, device="cuda")
        err = _Err()
        _check(_lib.rlq_llama_embedding(self._h, int(token), _dev_ptr(out, torch.float32), _stream_ptr(stream),
                                        ctypes.byref(err)), err)
        return out

    def step(self, hidden, position, embedding=True, logits=True, argmax=False, stream=None):
        """LlamaModel::step (llama.rs:222-248): hidden (f32 [width] on the GPU)
        is updated in place to the last layer's output; returns
        (embedding, logits, argmax), each None unless asked for."""
        c = self.config
        emb = torch.empty(c.width, dtype=torch.float32, device=hidden.device) if embedding else None
        lg = torch.empty(c.vocabulary, dtype=torch.float32, device=hidden.device) if logits else None
        am = torch.empty(1, dtype=torch.int32, device=hidden.device) if argmax else None
        err = _Err()
        _check(_lib.rlq_llama_step(self._h, _dev_ptr(hidden, torch.float32), int(position),
                                   _dev_ptr(emb, torch.float32) if emb is not None else None,
                                   _dev_ptr(lg, torch.float32) if lg is not None else None,
                                   _dev_ptr(am, torch.int32) if am is not None else None,
                                   _stream_ptr(stream), ctypes.byref(err)), err)
        return emb, lg, am

    @property
    def trace_stride(self):
        c = self.config
        return 4 * c.width + 2 * c.kv_width + c.feed_forward

    def trace(self, parts):
        """rlq_llama_trace: with a GPU tensor [n_layers, trace_stride] f32,
        every later step also copies each layer's intermediates there
        (split_trace() names them); None stops it."""
        self._trace = parts  # kept alive while the library writes to it
        err = _Err()
        _check(_lib.rlq_llama_trace(self._h, _dev_ptr(parts, torch.float32) if parts is not None else None,
                                    ctypes.byref(err)), err)

    def split_trace(self, row):
        """One layer's row of the trace as (qkv, attention, ffn_input, ffn, output)."""
        c = self.config
        a = c.width + 2 * c.kv_width
        cuts = (a, a + c.width, a + 2 * c.width, a + 2 * c.width + c.feed_forward)
        return row[:cuts[0]], row[cuts[0]:cuts[1]], row[cuts[1]:cuts[2]], row[cuts[2]:cuts[3]], row[cuts[3]:]

    def intermediates(self, stream=None):
        """The last layer's [q | k | v] (k before RoPE), attention output,
        silu(gate) * up and the residual stream after attention (the FFN
        norm's input) of the latest step, as fresh GPU tensors:
        (qkv, attention, ffn, ffn_input)."""
        c = self.config
        qkv = torch.empty(c.width + 2 * c.kv_width, dtype=torch.float32, device="cuda")
        att = torch.empty(c.width, dtype=torch.float32, device="cuda")
        mid = torch.empty(c.width, dtype=torch.float32, device="cuda")
        gu = torch.empty(c.feed_forward, dtype=torch.float32, device="cuda")
        err = _Err()
        _check(_lib.rlq_llama_intermediates(self._h, _dev_ptr(qkv, torch.float32), _dev_ptr(att, torch.float32),
                                            _dev_ptr(mid, torch.float32), _dev_ptr(gu, torch.float32),
                                            _stream_ptr(stream), ctypes.byref(err)), err)
        return qkv, att, gu, mid


# ---- GGUF files (host only) -------------------------------------------------------

GGUF_SCALAR_BYTES = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


class GgufFile:
    """rlq_gguf: RawGguf (crates/gguf/src/raw.rs) over a file (open) or a
    memory image (from_bytes, header only).  Keys, strings and names are bytes."""

    def __init__(self, handle):
        self._h = handle
        v, a, nk, nt = _U32(), _U32(), _U64(), _U64()
        d, big = _U64(), _I32()
        _lib.rlq_gguf_header(self._h, ctypes.byref(v), ctypes.byref(a), ctypes.byref(d), ctypes.byref(nk),
                             ctypes.byref(nt), ctypes.byref(big))
        self.version, self.alignment, self.data_offset = v.value, a.value, d.value
        self.n_kv, self.n_tensors, self.big_endian = nk.value, nt.value, bool(big.value)

    @classmethod
    def open(cls, path):
        h, err = ctypes.c_void_p(), _Err()
        _check(_lib.rlq_gguf_open(os.fsencode(path), ctypes.byref(h), ctypes.byref(err)), err)
        return cls(h)

    @classmethod
    def from_bytes(cls, data):
        buf = _u8(np.frombuffer(bytes(data), np.uint8))
        h, err = ctypes.c_void_p(), _Err()
        _check(_lib.rlq_gguf_read_header_memory(_ptr(buf), buf.size, ctypes.byref(h), ctypes.byref(err)), err)
        return cls(h)

    def close(self):
        if getattr(self, "_h", None):
            if _exiting is False:  # None once module teardown has cleared the globals
                _lib.rlq_gguf_close(self._h)
            self._h = None

    __del__ = close

    def kv(self, i):
        """(key, type, value): value is an int (scalar bits), bytes (string),
        or (element_type, [int | bytes]) for arrays."""
        k, kl, ty, el, n, err = ctypes.c_void_p(), _U64(), _U32(), _U32(), _U64(), _Err()
        _check(_lib.rlq_gguf_kv_at(self._h, i, ctypes.byref(k), ctypes.byref(kl), ctypes.byref(ty), ctypes.byref(el),
                                   ctypes.byref(n), ctypes.byref(err)), err)
        key = ctypes.string_at(k.value, kl.value) if kl.value else b""
        if ty.value == 8:
            return key, 8, self._string(i, 0)
        if ty.value == 9:
            items = [self._string(i, j) if el.value == 8 else self._scalar(i, j) for j in range(n.value)]
            return key, 9, (el.value, items)
        return key, ty.value, self._scalar(i, 0)

    def _scalar(self, i, j):
        b, err = _U64(), _Err()
        _check(_lib.rlq_gguf_kv_scalar(self._h, i, j, ctypes.byref(b), ctypes.byref(err)), err)
        return b.value

    def _string(self, i, j):
        p, n, err = ctypes.c_void_p(), _U64(), _Err()
        _check(_lib.rlq_gguf_kv_string(self._h, i, j, ctypes.byref(p), ctypes.byref(n), ctypes.byref(err)), err)
        return ctypes.string_at(p.value, n.value) if n.value else b""

    def find_kv(self, key):
        key = bytes(key)
        r = _lib.rlq_gguf_find_kv(self._h, ctypes.c_char_p(key), len(key))
        return None if r < 0 else r

    def tensor(self, i):
        """(name, dims (stored rank), dtype, offset, bytes)."""
        nm, nl, nd, dt, off, nb, err = ctypes.c_void_p(), _U64(), _U32(), _U32(), _U64(), _U64(), _Err()
        dims = (_U64 * 4)()
        _check(_lib.rlq_gguf_tensor_at(self._h, i, ctypes.byref(nm), ctypes.byref(nl), ctypes.byref(nd), dims,
                                       ctypes.byref(dt), ctypes.byref(off), ctypes.byref(nb), ctypes.byref(err)), err)
        name = ctypes.string_at(nm.value, nl.value) if nl.value else b""
        return name, list(dims)[:nd.value], dt.value, off.value, nb.value

    def find_tensor(self, name):
        name = bytes(name)
        r = _lib.rlq_gguf_find_tensor(self._h, ctypes.c_char_p(name), len(name))
        return None if r < 0 else r

    def read_tensor(self, i):
        nb = self.tensor(i)[4]
        out = np.zeros(nb, np.uint8)
        err = _Err()
        _check(_lib.rlq_gguf_read_tensor(self._h, i, _ptr(out) if nb else None, nb, ctypes.byref(err)), err)
        return out

    def native_header(self):
        n, err = _U64(), _Err()
        _check(_lib.rlq_gguf_native_header(self._h, None, 0, ctypes.byref(n), ctypes.byref(err)), err)
        out = np.zeros(n.value, np.uint8)
        _check(_lib.rlq_gguf_native_header(self._h, _ptr(out), n.value, ctypes.byref(n), ctypes.byref(err)), err)
        return out.tobytes()


class _GgufKv(ctypes.Structure):
    _fields_ = [("key", _P), ("key_len", _U64), ("type", _U32), ("element_type", _U32), ("count", _U64),
                ("data", _P), ("lengths", _P)]


class _GgufTensor(ctypes.Structure):
    _fields_ = [("name", _P), ("name_len", _U64), ("n_dims", _U32), ("dims", _U64 * 4), ("dtype", _U32),
                ("data", _P)]


def _gguf_structs(kvs, tensors):
    """kvs: [(key bytes, type, value)] with value as for GgufFile.kv;
    tensors: [(name bytes, dims, dtype, payload uint8 array or None)]."""
    keep = []
    ks = (_GgufKv * max(1, len(kvs)))()
    for i, (key, ty, val) in enumerate(kvs):
        key = bytes(key)
        keep.append(key)
        k = ks[i]
        k.key, k.key_len, k.type = ctypes.cast(ctypes.c_char_p(key), _P), len(key), ty
        if ty == 8:
            buf = bytes(val)
            keep.append(buf)
            k.count, k.data = len(buf), ctypes.cast(ctypes.c_char_p(buf), _P)
        elif ty == 9:
            el, items = val
            k.element_type, k.count = el, len(items)
            if el == 8:
                buf = b"".join(bytes(x) for x in items)
                lens = (_U64 * max(1, len(items)))(*[len(x) for x in items])
                keep += [buf, lens]
                k.data, k.lengths = ctypes.cast(ctypes.c_char_p(buf), _P), ctypes.cast(lens, _P)
            else:
                w = GGUF_SCALAR_BYTES.get(el, 1)
                buf = b"".join(int(x).to_bytes(w, "little") for x in items)
                keep.append(buf)
                k.data = ctypes.cast(ctypes.c_char_p(buf), _P)
        else:
            buf = int(val).to_bytes(GGUF_SCALAR_BYTES.get(ty, 8), "little")
            keep.append(buf)
            k.count, k.data = 1, ctypes.cast(ctypes.c_char_p(buf), _P)
    ts = (_GgufTensor * max(1, len(tensors)))()
    for i, (name, dims, dtype, data) in enumerate(tensors):
        name = bytes(name)
        keep.append(name)
        t = ts[i]
        t.name, t.name_len, t.n_dims, t.dtype = ctypes.cast(ctypes.c_char_p(name), _P), len(name), len(dims), dtype
        for d, v in enumerate(dims):
            t.dims[d] = v
        if data is not None:
            arr = _u8(data)
            keep.append(arr)
            t.data = _ptr(arr)
    return ks, ts, keep


def gguf_header(kvs, tensors):
    """write_raw_header: (header bytes padded to the data offset, file bytes)."""
    ks, ts, keep = _gguf_structs(kvs, tensors)
    n, fb, err = _U64(), _U64(), _Err()
    _check(_lib.rlq_gguf_write_header(ks, len(kvs), ts, len(tensors), None, 0, ctypes.byref(n), ctypes.byref(fb),
                                      ctypes.byref(err)), err)
    out = np.zeros(n.value, np.uint8)
    _check(_lib.rlq_gguf_write_header(ks, len(kvs), ts, len(tensors), _ptr(out), n.value, ctypes.byref(n),
                                      ctypes.byref(fb), ctypes.byref(err)), err)
    del keep
    return out.tobytes(), fb.value


def gguf_write(path, kvs, tensors):
    """write_ordered: a GGUF v3 file of the given metadata and tensors."""
    ks, ts, keep = _gguf_structs(kvs, tensors)
    err = _Err()
    _check(_lib.rlq_gguf_write(os.fsencode(path), ks, len(kvs), ts, len(tensors), ctypes.byref(err)), err)
    del keep


# GGUF tensor names of a llama layer's tensors (crates/inference/src/loader.rs:356-394)
LLAMA_GGUF_NAMES = {"query": "attn_q", "key": "attn_k", "value": "attn_v", "attention_output": "attn_output",
                    "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down", "attention_norm": "attn_norm",
                    "feed_forward_norm": "ffn_norm"}


def llama_gguf_contents(config, tensors, tied=False, tokens=None):
    """The metadata and tensors of a llama GGUF file holding a model, in the
    keys, names and GGML shapes the reference's loader reads
    (crates/inference/src/loader.rs:282-394), for gguf_write.  `config` has
    the LlamaConfig fields, `tensors` the LlamaModel dict (numpy arrays; a
    layer's optional `types` maps matrix names to their types).  tied: no
    output.weight (the embedding projects).  tokens: the vocabulary strings
    (default <t0>, <t1>, ...)."""
    f32 = lambda x: int(np.float32(x).view(np.uint32))  # noqa: E731
    V, W, F = int(config.vocabulary), int(config.width), int(config.feed_forward)
    hd = W // int(config.heads)
    kvw = int(config.kv_heads) * hd
    toks = tokens if tokens is not None else [b"<t%d>" % i for i in range(V)]
    kvs = [(b"general.architecture", 8, b"llama"), (b"general.name", 8, b"random-init"),
           (b"llama.block_count", 4, len(tensors["layers"])), (b"llama.context_length", 4, int(config.max_context)),
           (b"llama.embedding_length", 4, W), (b"llama.feed_forward_length", 4, F),
           (b"llama.attention.head_count", 4, int(config.heads)),
           (b"llama.attention.head_count_kv", 4, int(config.kv_heads)),
           (b"llama.attention.layer_norm_rms_epsilon", 6, f32(config.rms_epsilon)),
           (b"llama.rope.freq_base", 6, f32(config.rope_base)), (b"llama.rope.dimension_count", 4, hd),
           (b"tokenizer.ggml.model", 8, b"llama"), (b"tokenizer.ggml.tokens", 9, (8, toks))]
    if float(config.attention_scale) != 0.0:
        kvs.append((b"llama.attention.scale", 6, f32(config.attention_scale)))
    as_u8 = lambda a: np.ascontiguousarray(a).reshape(-1).view(np.uint8)  # noqa: E731
    out = [(b"token_embd.weight", [W, V], int(config.embedding_type), as_u8(tensors["embedding"])),
           (b"output_norm.weight", [W], 0, as_u8(np.asarray(tensors["output_norm"], np.float32)))]
    if not tied:
        out.append((b"output.weight", [W, V], int(config.output_type), as_u8(tensors["output"])))
    shapes = {"query": [W, W], "key": [W, kvw], "value": [W, kvw], "attention_output": [W, W], "gate": [W, F],
              "up": [W, F], "down": [F, W]}
    for i, L in enumerate(tensors["layers"]):
        types = L.get("types", {})
        for name, g in LLAMA_GGUF_NAMES.items():
            nm = b"blk.%d.%s.weight" % (i, g.encode())
            if name.endswith("norm"):
                out.append((nm, [W], 0, as_u8(np.asarray(L[name], np.float32))))
            else:
                out.append((nm, shapes[name], int(types.get(name, config.weight_type)), as_u8(L[name])))
    return kvs, out


def write_llama_gguf(path, config, tensors, tied=False, tokens=None):
    """A llama GGUF v3 file of the model (gguf_write of llama_gguf_contents)."""
    kvs, ts = llama_gguf_contents(config, tensors, tied, tokens)
    gguf_write(path, kvs, ts)
