"""C ABI checks that need no GPU: the library loads, exports every entry point
include/rlq.h declares, and the metadata / shape validation (which runs
before any device work, matvec.rs:31-50) agrees with the reference order."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle as O
from rlq_loader import ROOT, load

rlq = load()


def declared_functions():
    text = open(os.path.join(ROOT, "include", "rlq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rlq_[a-z_0-9]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 18
    lib = ctypes.CDLL(rlq.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(rlq.SIGNATURES) == names


def test_status_codes_match_quanterror_order():
    for code, name in rlq.ERROR_NAMES.items():
        assert O.ERROR_NAMES[code] == name
    assert rlq.lib().rlq_status_string(16).decode().startswith("non-finite")


ALL_IDS = [0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26,
           27, 28, 29, 30, 34, 35, 39, 40, 41, 42, 43]


@pytest.mark.parametrize("t", ALL_IDS + [4, 31, 44])
def test_activation_dtype_matches_oracle(t):
    try:
        want = O.matvec_activation_dtype(t)
    except O.OracleError as e:
        with pytest.raises(rlq.QuantError) as g:
            rlq.matvec_activation_dtype(t)
        assert g.value.code == e.code and g.value.dtype == e.dtype
        return
    assert rlq.matvec_activation_dtype(t) == want


@pytest.mark.parametrize("t", ALL_IDS)
def test_row_bytes_matches_oracle(t):
    for n in (0, 1, 32, 96, 256, 896, 4096, 4097, 2 ** 64 - 256):
        try:
            want = O.row_bytes(t, n)
        except O.OracleError as e:
            with pytest.raises(rlq.QuantError) as g:
                rlq.row_bytes(t, n)
            assert (g.value.code, g.value.a, g.value.b) == (e.code, e.a, e.b)
            continue
        assert rlq.row_bytes(t, n) == want


@pytest.mark.parametrize("t", [rlq.DType.Q4_K, rlq.DType.Q6_K, rlq.DType.Q8_0])
def test_matvec_shape_errors_before_any_device_work(t):
    n = 256 if t != rlq.DType.Q8_0 else 32
    x = np.ones(n, np.float32)
    w = np.zeros(rlq.row_bytes(t, n), np.uint8)
    cases = [((t, w[:-1], 1, n, x), "InvalidLength"),
             ((t, w, 1, n, x[:-1]), "InvalidVectorLength"),
             ((t, w, 0, n, x), "InvalidMatrixShape"),
             ((t, w, 1, n - 1, x[:-1]), "NonMultiple"),
             ((t, w, 2 ** 64 - 1, n, x), "SizeOverflow")]
    for args, name in cases:
        with pytest.raises(rlq.QuantError) as g:
            rlq.matvec(*args)
        with pytest.raises(O.OracleError) as e:
            O.matvec(*args)
        assert g.value.name == name == e.value.name
        assert (g.value.a, g.value.b) == (e.value.a, e.value.b)


def test_non_path_types_are_unimplemented_not_silently_wrong():
    with pytest.raises(rlq.QuantError) as g:
        rlq.matvec(rlq.DType.Q4_0, np.zeros(18, np.uint8), 1, 32, np.ones(32, np.float32))
    assert g.value.name == "Unimplemented"
    with pytest.raises(rlq.QuantError) as g:
        rlq.matvec(rlq.DType.Q8_K, np.zeros(292, np.uint8), 1, 256, np.ones(256, np.float32))
    assert g.value.name == "UnsupportedMatVec"
    with pytest.raises(rlq.QuantError) as g:
        rlq.quantize(rlq.DType.I64, np.zeros(256, np.float32))
    assert g.value.name == "UnsupportedQuantization"


def test_probe_arguments_refused_before_any_launch():
    """The measurement probes check their arguments before any device call:
    unknown kinds, shapes and runs, a misaligned or ragged buffer, no output
    (the pointers are never dereferenced on these paths)."""
    lib = rlq.lib()
    invalid = 20  # RLQ_INVALID_ARGUMENT
    assert rlq.ERROR_NAMES[invalid] == "InvalidArgument"
    fake = ctypes.c_void_p(4096)
    assert lib.rlq_probe_mfma(9, 1, 1, fake, None) == invalid
    assert lib.rlq_probe_mfma(0, 0, 1, fake, None) == invalid
    assert lib.rlq_probe_mfma(0, 1, 1, None, None) == invalid
    for waves, runs, length, ptr in ((3, 2, 1024, fake), (32, 2, 1024, fake), (2 ** 31 + 4, 2, 1024, fake),
                                     (16, 3, 1024, fake), (16, 0, 1024, fake), (16, 2, 1000, fake),
                                     (16, 2, 1024, ctypes.c_void_p(4100))):
        assert lib.rlq_probe_stream_shape(ptr, length, 1, waves, runs, 1, fake, None) == invalid, (waves, runs)
    assert lib.rlq_probe_stream(fake, 1000, 1, fake, None) == invalid
