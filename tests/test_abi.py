"""CPU-side checks of the C ABI: the library loads, exports every symbol the
public headers declare, and rejects bad arguments before touching a GPU."""
import ctypes as C
import os

import pytest

import g4


def test_library_loads_and_exports_header():
    lib = g4.Lib.get()
    missing = [s for s in g4.header_symbols(g4.HEADER) if not hasattr(lib.L, s)]
    assert not missing, missing


def test_engine_exports_header():
    if not os.path.exists(g4.ENGINE_HEADER):
        pytest.skip("engine not present")
    eng = C.CDLL(g4.ENGINE_PATH)
    missing = [s for s in g4.header_symbols(g4.ENGINE_HEADER) if not hasattr(eng, s)]
    assert not missing, missing


def test_argument_errors_without_gpu():
    L = g4.Lib.get().L
    assert L.g4_mm(None, None, None, 256, 1, 99, None, 0) == g4.G4_ERR_TYPE
    assert b"Unsupported tensor type 99" in L.g4_last_error()
    assert L.g4_mm(None, None, None, 300, 1, g4.Q4_K, None, 0) == g4.G4_ERR_ARG
    assert b"not multiple of QK_K" in L.g4_last_error()
    assert L.g4_quantize_row_q8_K(None, None, 256) == g4.G4_ERR_ARG
    assert L.g4_upload_quant(None, None, 7, 256, 1) == g4.G4_ERR_TYPE
    assert L.g4_tensor_bytes(g4.Q4_K, 2560, 10240) == 14745600
    assert L.g4_tensor_bytes(g4.Q6_K, 2560, 262144) == 550502400
    assert L.g4_tensor_bytes(g4.Q5_K, 2560, 10240) == 18022400
    assert L.g4_q8K_bytes(2560) == 2920


def test_header_cites_reference():
    txt = open(g4.HEADER).read()
    for fn in ("quantize_row_q8_K", "vec_dot_q4_K_q8_K", "mm_quant_dot_rows", "mm_quant_rows", "main.c:1669"):
        assert fn in txt
