"""ctypes binding of libg4hip.so (include/g4hip.h) and libg4engine.so.

Loading fails loudly when the HIP library has not been built: there is no
CPU fallback anywhere on this path.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libg4hip.so")
ENGINE_PATH = os.path.join(PKG, "libg4engine.so")
HEADER = os.path.join(ROOT, "include", "g4hip.h")
ENGINE_HEADER = os.path.join(PKG, "host", "engine.h")

G4_OK, G4_ERR_ARG, G4_ERR_TYPE, G4_ERR_HIP, G4_ERR_NOMEM, G4_ERR_STATE, G4_ERR_NODEV, G4_ERR_FORMAT = range(8)
F32, F16, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 12, 13, 14, 30

VP, I, SZ, F = C.c_void_p, C.c_int, C.c_size_t, C.c_float

_SIGS = {
    "g4_init": (I, [I]),
    "g4_device_info": (I, [VP, C.c_char_p, I]),
    "g4_set_stream": (I, [VP]),
    "g4_get_stream": (VP, []),
    "g4_sync": (I, []),
    "g4_last_error": (C.c_char_p, []),
    "g4_malloc": (I, [C.POINTER(VP), SZ]),
    "g4_free": (I, [VP]),
    "g4_memcpy_h2d": (I, [VP, VP, SZ]),
    "g4_memcpy_d2h": (I, [VP, VP, SZ]),
    "g4_event_create": (I, [C.POINTER(VP)]),
    "g4_event_destroy": (I, [VP]),
    "g4_event_record": (I, [VP]),
    "g4_event_elapsed_ms": (I, [VP, VP, C.POINTER(F)]),
    "g4_tensor_bytes": (SZ, [I, I, I]),
    "g4_upload_quant": (I, [VP, VP, I, I, I]),
    "g4_download_quant": (I, [VP, VP, I, I, I]),
    "g4_relayout_quant": (I, [VP, VP, I, I, I]),
    "g4_q8K_bytes": (SZ, [I]),
    "g4_quantize_row_q8_K": (I, [VP, VP, I]),
    "g4_download_q8K": (I, [VP, VP, I]),
    "g4_upload_q8K": (I, [VP, VP, I]),
    "g4_vec_dot_q4_K_q8_K": (I, [I, VP, VP, VP]),
    "g4_vec_dot_q5_K_q8_K": (I, [I, VP, VP, VP]),
    "g4_vec_dot_q6_K_q8_K": (I, [I, VP, VP, VP]),
    "g4_mm_quant_dot_rows": (I, [VP, VP, I, I, I, VP]),
    "g4_mm_quant_rows": (I, [VP, VP, VP, I, I, I]),
    "g4_mm_quant_rows_softcap": (I, [VP, VP, VP, I, I, I, F]),
    "g4_mm_bf16": (I, [VP, VP, VP, I, I]),
    "g4_mm": (I, [VP, VP, VP, I, I, I, VP, I]),
    "g4_mm_gate_up_gelu": (I, [VP, VP, VP, I, I, I, VP]),
    "g4_debug_block_sums": (I, [VP, I, I, I, VP, VP, VP]),
    "g4_set_gemv_occupancy": (I, [I]),
}


class G4Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"g4 status {code}: {msg}")
        self.code = code


def header_symbols(path: str = HEADER) -> list[str]:
    """Function names declared in a C header (for the export check)."""
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(g4e?_[a-zA-Z0-9_]+)\s*\(", txt)))


class Lib:
    _inst = None

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
        self.path = path
        self.L = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            f = getattr(self.L, name)
            f.restype = res
            f.argtypes = args
        self.initialized = False

    @classmethod
    def get(cls) -> "Lib":
        if cls._inst is None:
            cls._inst = Lib()
        return cls._inst

    def check(self, rc: int) -> None:
        if rc != G4_OK:
            raise G4Error(rc, self.L.g4_last_error().decode())

    def init(self, device: int = 0) -> None:
        if not self.initialized:
            self.check(self.L.g4_init(device))
            self.initialized = True

    def __getattr__(self, name):
        f = getattr(self.L, name)

        def call(*args):
            rc = f(*args)
            if f.restype is I:
                self.check(rc)
            return rc
        return call


class DBuf:
    """A device allocation owned by the library (g4_malloc / g4_free)."""

    def __init__(self, lib: Lib, nbytes: int):
        self.lib = lib
        self.nbytes = int(nbytes)
        p = VP()
        lib.check(lib.L.g4_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, lib: Lib, a: np.ndarray) -> "DBuf":
        a = np.ascontiguousarray(a)
        b = cls(lib, a.nbytes)
        if a.nbytes:
            lib.check(lib.L.g4_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    def to_array(self, dtype, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dt)
        if out.nbytes:
            self.lib.check(self.lib.L.g4_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def write(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        self.lib.check(self.lib.L.g4_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes))

    def free(self) -> None:
        if self.ptr:
            self.lib.L.g4_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def upload_quant(lib: Lib, raw: np.ndarray, qtype: int, n: int, d: int) -> DBuf:
    nbytes = lib.L.g4_tensor_bytes(qtype, n, d)
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    assert raw.size == nbytes, (raw.size, nbytes)
    b = DBuf(lib, nbytes)
    lib.check(lib.L.g4_upload_quant(b.ptr, raw.ctypes.data, qtype, n, d))
    return b


def download_quant(lib: Lib, buf: DBuf, qtype: int, n: int, d: int) -> np.ndarray:
    out = np.empty(lib.L.g4_tensor_bytes(qtype, n, d), np.uint8)
    lib.check(lib.L.g4_download_quant(out.ctypes.data, buf.ptr, qtype, n, d))
    return out
