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
# engine trace: quantization points per layer (engine.h G4E_Q8_SLOT_*) and
# elements per traced Q8_K vector
Q8_SLOTS, Q8_SLOT_ELEMS = 5, 4096
# layer-0 fingerprint tags (engine.h G4E_FP_*), as dump_kv_fingerprint names them
FP_TAGS = ("attn_norm", "K_pre_norm", "K_pre_rope", "K_store", "K_read0", "K_readN", "q_out")
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
    "g4_mm_quant_dot_rows_gelu_mul": (I, [VP, VP, I, I, I, VP, VP]),
    "g4_debug_block_sums": (I, [VP, I, I, I, VP, VP, VP]),
    "g4_set_gemv_occupancy": (I, [I]),
    "g4_mm_residual_q8": (I, [VP, VP, VP, I, I, I, VP, VP, VP, VP, VP, VP, VP, VP, VP, I, F]),
    "g4_mm_residual_q8_pair": (I, [VP, VP, I, VP, VP, I, I, I, VP, VP, VP, VP, VP, VP, VP, VP, I, F]),
    "g4_mm_residual_q8_qkv": (I, [VP, VP, I, VP, VP, I, VP, VP, I, I, I, I, VP, VP, VP, VP, VP, VP, VP, VP, F]),
    "g4_q8K_row_stride": (SZ, [I]),
    "g4_quantize_rows_q8_K": (I, [VP, VP, I, I]),
    "g4_mm_batch_q8": (I, [VP, VP, VP, I, I, I, I]),
    "g4_mm_batch_q8_blocks": (I, [VP, VP, VP, I, I, I, I]),
    "g4_fold_gelu_mul_q8": (I, [VP, VP, I, VP, I, VP, VP, I, I]),
    "g4_mm_batch_q8_multi": (I, [VP, VP, VP, I, VP, I, I, I]),
    "g4_kq_image_bytes": (SZ, [I, I]),
    "g4_kq_image": (I, [VP, VP, I, I, I]),
    "g4_mm_batch_img": (I, [VP, VP, VP, I, I, I, I]),
    "g4_mm_batch_img_multi": (I, [VP, VP, VP, I, VP, I, I, I]),
    "g4_mm_batch_img_tile": (I, [VP, VP, VP, I, I, I, I, I, I]),
    "g4_debug_batch_block_sums": (I, [VP, I, I, I, I, I, VP, VP, VP]),
    "g4_mm_batch": (I, [VP, VP, VP, I, I, I, I, VP]),
    "g4_split_rows_bytes": (SZ, [I, I]),
    "g4_split_rows_f16": (I, [VP, VP, I, I]),
    "g4_gelu_mul_split_rows": (I, [VP, VP, I, VP, I, I]),
    "g4_mm_batch_split": (I, [VP, VP, VP, I, I, I, I]),
    "g4_mm_f16": (I, [VP, VP, VP, I, I]),
    "g4_mm_f32": (I, [VP, VP, VP, I, I]),
    "g4_softcap": (I, [VP, I, F]),
    "g4_hidden_stats": (I, [VP, I, VP]),
    "g4_sample_part_bytes": (SZ, [I]),
    "g4_sample": (I, [VP, I, F, F, I, F, I, VP, VP, I, VP, VP, VP, VP, VP]),
    "g4_emb_lookup_rows": (I, [VP, VP, I, I, VP, I, I, F]),
    "g4_ple_finish_rows": (I, [VP, VP, VP, I, I, VP, VP, I, I, I, F, F, F, F]),
    "g4_gelu_mul_rows": (I, [VP, VP, VP, I, I, I]),
    "g4_residual_norm_rows": (I, [VP, VP, VP, VP, VP, VP, VP, I, I, F, I, I]),
    "g4_rope_table_rows": (I, [VP, I, I, I, F, F, VP]),
    "g4_qkv_post_rows": (I, [VP, VP, VP, VP, VP, VP, VP, I, VP, I, I, I, I, I, F]),
    "g4_kv_store_rows": (I, [VP, VP, VP, VP, I, I, I, I, I]),
    "g4_attn_decode_rows": (I, [VP, VP, VP, VP, VP, I, I, I, I, I, I, I, I, F, I, VP, VP, VP]),
    "g4_rmsnorm": (I, [VP, VP, VP, I, F]),
    "g4_rmsnorm_head_inplace": (I, [VP, VP, I, I, F]),
    "g4_rmsnorm_head_noweight_inplace": (I, [VP, I, I, F]),
    "g4_apply_rope_neox": (I, [VP, I, I, I, I, F, F, VP]),
    "g4_kv_append_rope": (I, [VP, VP, VP, VP, VP, I, I, I, I, I, I, F, F, VP, F]),
    "g4_attn_decode": (I, [VP, VP, VP, I, I, I, I, I, I, F, VP]),
    "g4_attn_decode_ring": (I, [VP, VP, VP, I, I, I, I, I, I, I, F, VP]),
    "g4_attn_decode_noalloc": (I, [VP, VP, VP, I, I, I, I, I, I, F, VP]),
    "g4_softmax": (I, [VP, I]),
    "g4_emb_lookup": (I, [VP, VP, I, I, I, I]),
    "g4_argmax_part_bytes": (SZ, [I]),
    "g4_argmax": (I, [VP, I, VP, VP, VP, VP]),
    "g4_mm_argmax_part_bytes": (SZ, [I]),
    "g4_mm_attn_merge": (I, [VP, VP, I, I, I, VP, I, I, I, VP, VP]),
    "g4_probe_empty": (I, [I]),
    "g4_probe_read": (I, [VP, SZ, VP, I]),
    "g4_probe_handoff": (I, [VP, VP, VP, I, I]),
    "g4_mm_argmax_row": (I, [VP, VP, I, I, I, VP, F, VP, VP, VP, VP, VP]),
    "g4_residual_norm": (I, [VP, VP, VP, VP, VP, VP, VP, I, I, F]),
    "g4_qkv_post": (I, [VP, VP, VP, VP, VP, VP, VP, I, I, VP, I, I, I, I, I, F, F, VP, F, VP]),
    "g4_rope_table": (I, [VP, VP, I, I, F, F, VP]),
    "g4_attn_part_bytes": (SZ, [I, I, I]),
    "g4_attn_decode_dev": (I, [VP, VP, VP, I, I, VP, I, I, I, I, F, I, VP, VP, VP]),
    "g4_attn_decode_fused": (I, [VP, VP, VP, VP, VP, VP, VP, VP, VP, I, I, VP, I, I, I, I, I, VP, F, F, I, VP, VP, VP]),
    "g4_emb_lookup_dev": (I, [VP, VP, I, I, VP, I, F]),
    "g4_emb_lookup_rope": (I, [VP, VP, I, I, VP, I, F, VP, VP, I, F, VP, VP, I, F, VP, F]),
    "g4_emb_lookup_rope_ple": (I, [VP, VP, I, I, VP, I, F, VP, VP, I, F, VP, VP, I, F, VP, F, VP, VP, I, VP]),
    "g4_ple_pairs_bytes": (SZ, [I]),
    "g4_mm_ple_gate_proj": (I, [VP, VP, I, I, VP, I, I, I, VP, VP, VP, VP, VP, F, VP, VP]),
    "g4_ple_finish": (I, [VP, VP, VP, I, I, VP, VP, I, I, I, F, F, F, F]),
    "g4_gelu_mul_quant": (I, [VP, VP, I, VP]),
    "g4_store_i32x2": (I, [VP, I, I]),
    "g4_memset": (I, [VP, I, SZ]),
    "g4_memcpy_h2d_async": (I, [VP, VP, SZ]),
    "g4_memcpy_d2h_async": (I, [VP, VP, SZ]),
    "g4_memcpy_d2d_async": (I, [VP, VP, SZ]),
    "g4_host_alloc": (I, [C.POINTER(VP), SZ]),
    "g4_host_free": (I, [VP]),
    "g4_stream_create": (I, [C.POINTER(VP)]),
    "g4_stream_destroy": (I, [VP]),
    "g4_graph_begin": (I, []),
    "g4_graph_end": (I, [C.POINTER(VP)]),
    "g4_graph_launch": (I, [VP]),
    "g4_graph_destroy": (I, [VP]),
}

_ENGINE_SIGS = {
    "g4e_open_image": (I, [VP, SZ, I, I, C.POINTER(VP)]),
    "g4e_check_image": (I, [VP, SZ, I, VP]),
    "g4e_open_file": (I, [C.c_char_p, I, I, C.POINTER(VP)]),
    "g4e_close": (None, [VP]),
    "g4e_last_error": (C.c_char_p, []),
    "g4e_config": (None, [VP, VP]),
    "g4e_forward": (I, [VP, I, I, I]),
    "g4e_read_logits": (I, [VP, VP]),
    "g4e_read_x": (I, [VP, VP]),
    "g4e_argmax": (I, [VP, C.POINTER(I)]),
    "g4e_set_trace": (I, [VP, I]),
    "g4e_layer_x": (C.POINTER(F), [VP]),
    "g4e_layer_q8": (VP, [VP]),
    "g4e_kv_fingerprint": (I, [VP, VP, VP]),
    "g4e_generate_greedy": (I, [VP, VP, I, I, VP, C.POINTER(C.c_double), C.POINTER(C.c_double), I]),
    "g4e_decode_steps": (I, [VP, I, I, I, I, VP, C.POINTER(C.c_double)]),
    "g4e_generate": (I, [VP, VP, I, I, F, F, I, F, I, C.c_uint64, VP, C.POINTER(C.c_double),
                         C.POINTER(C.c_double), I]),
    "g4e_decode_steps_sampled": (I, [VP, I, I, I, F, F, I, F, I, C.c_uint64, I, VP, C.POINTER(C.c_double)]),
    "g4e_prefill": (I, [VP, VP, I, I]),
    "g4e_prefill_trace_q8": (I, [VP, VP, I, I, VP, VP]),
    "g4e_prefill_trace": (I, [VP, VP, I, I, VP]),
    "g4e_set_prefill_chunk": (I, [VP, I]),
    "g4e_set_f32_matmul": (I, [VP, I]),
    "g4e_sha256_file": (I, [C.c_char_p, C.c_char_p]),
    "g4e_check_sha256sum": (I, [C.c_char_p, C.c_char_p]),
    "g4e_set_dump_hidden_at": (I, [VP, I]),
    "g4e_hidden_stats": (I, [VP, VP]),
    "g4e_read_kv": (I, [VP, I, I, I, VP, VP]),
    "g4e_kv_info": (I, [VP, I, VP]),
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


class EngineLib:
    """libg4engine.so (host/engine.h)."""
    _inst = None

    def __init__(self, path: str = ENGINE_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
        Lib.get()   # load libg4hip.so first (the engine links to it)
        self.L = C.CDLL(path)
        for name, (res, args) in _ENGINE_SIGS.items():
            f = getattr(self.L, name)
            f.restype = res
            f.argtypes = args

    @classmethod
    def get(cls) -> "EngineLib":
        if cls._inst is None:
            cls._inst = EngineLib()
        return cls._inst

    def check(self, rc: int) -> None:
        if rc != G4_OK:
            raise G4Error(rc, self.L.g4e_last_error().decode())

    def sha256_file(self, path: str) -> str:
        out = C.create_string_buffer(65)
        self.check(self.L.g4e_sha256_file(path.encode(), out))
        return out.value.decode()

    def check_sha256sum(self, path: str, sumfile: str) -> None:
        """`sha256sum --check` of one file against a checksum file's line"""
        self.check(self.L.g4e_check_sha256sum(path.encode(), sumfile.encode()))

    def check_image(self, data, max_seq: int = 0) -> list[int]:
        buf = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data
        out = np.zeros(9, np.int32)
        self.check(self.L.g4e_check_image(buf.ctypes.data, buf.size, max_seq, out.ctypes.data))
        return [int(v) for v in out]


class Engine:
    """A model opened by the C engine; forward/generate run on the GPU."""

    def __init__(self, path_or_image, max_seq: int = 0, device: int = 0):
        self.E = EngineLib.get()
        h = VP()
        if isinstance(path_or_image, (str, bytes, os.PathLike)):
            self.E.check(self.E.L.g4e_open_file(os.fsencode(path_or_image), max_seq, device, C.byref(h)))
        else:
            a = np.ascontiguousarray(path_or_image).view(np.uint8).reshape(-1)
            self.E.check(self.E.L.g4e_open_image(a.ctypes.data, a.size, max_seq, device, C.byref(h)))
        self.h = h.value
        cfg = np.zeros(9, np.int32)
        self.E.L.g4e_config(self.h, cfg.ctypes.data)
        (self.dim, self.hidden, self.n_layers, self.n_heads, self.n_kv, self.vocab,
         self.max_seq, self.ple_dim, self.window) = [int(v) for v in cfg]

    def forward(self, token: int, pos: int, lm_mode: int = 1) -> None:
        self.E.check(self.E.L.g4e_forward(self.h, token, pos, lm_mode))

    def logits(self) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        self.E.check(self.E.L.g4e_read_logits(self.h, out.ctypes.data))
        return out

    def x(self) -> np.ndarray:
        out = np.empty(self.dim, np.float32)
        self.E.check(self.E.L.g4e_read_x(self.h, out.ctypes.data))
        return out

    def argmax(self) -> int:
        t = C.c_int()
        self.E.check(self.E.L.g4e_argmax(self.h, C.byref(t)))
        return t.value

    def set_trace(self, on: bool) -> None:
        self.E.check(self.E.L.g4e_set_trace(self.h, int(on)))

    def layer_x(self) -> np.ndarray:
        p = self.E.L.g4e_layer_x(self.h)
        return np.ctypeslib.as_array(p, (self.n_layers + 1, self.dim)).copy()

    def layer_q8(self) -> np.ndarray:
        """Q8_K activations of the last traced step as raw BlockQ8_K bytes,
        (n_layers, Q8_SLOTS, Q8_SLOT_ELEMS // 256, 292): per layer the
        attention input, O input, FFN input, PLE inp_gate and proj inputs."""
        p = self.E.L.g4e_layer_q8(self.h)
        nb = Q8_SLOT_ELEMS // 256
        n = self.n_layers * Q8_SLOTS * nb * 292
        raw = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), (n,)).copy()
        return raw.reshape(self.n_layers, Q8_SLOTS, nb, 292)

    def generate_greedy(self, prompt, max_new: int, use_graph: bool = True):
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max_new + 1, np.int32)
        ps, ds = C.c_double(), C.c_double()
        n = self.E.L.g4e_generate_greedy(self.h, pr.ctypes.data, pr.size, max_new, out.ctypes.data,
                                         C.byref(ps), C.byref(ds), int(use_graph))
        if n < 0:
            self.E.check(-n)
        return out[:n].copy(), ps.value, ds.value

    def generate(self, prompt, max_new: int, temp: float = 0.6, topp: float = 0.9, topk: int = 40,
                 penalty: float = 1.0, penalty_last_n: int = 64, seed: int = 1, use_graph: bool = True):
        """generate() with the device sampler (defaults: the reference's
        temp 0.6, top-p 0.9, top-k 40, penalty 1.0 over 64 tokens); returns
        (tokens, prefill seconds, decode seconds)."""
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max_new + 1, np.int32)
        ps, ds = C.c_double(), C.c_double()
        n = self.E.L.g4e_generate(self.h, pr.ctypes.data, pr.size, max_new, temp, topp, topk, penalty,
                                  penalty_last_n, seed, out.ctypes.data, C.byref(ps), C.byref(ds), int(use_graph))
        if n < 0:
            self.E.check(-n)
        return out[:n].copy(), ps.value, ds.value

    def decode_steps(self, token: int, pos0: int, steps: int, use_graph: bool = True, record: bool = False):
        out = np.zeros(max(steps, 1), np.int32)
        sec = C.c_double()
        self.E.check(self.E.L.g4e_decode_steps(self.h, token, pos0, steps, int(use_graph),
                                               out.ctypes.data if record else None, C.byref(sec)))
        return (out[:steps].copy() if record else None), sec.value

    def decode_steps_sampled(self, token: int, pos0: int, steps: int, temp: float = 0.6, topp: float = 0.9,
                             topk: int = 40, penalty: float = 1.0, penalty_last_n: int = 64, seed: int = 1,
                             use_graph: bool = True, record: bool = False):
        """decode_steps() with the device sampler after each step."""
        out = np.zeros(max(steps, 1), np.int32)
        sec = C.c_double()
        self.E.check(self.E.L.g4e_decode_steps_sampled(self.h, token, pos0, steps, temp, topp, topk, penalty,
                                                       penalty_last_n, seed, int(use_graph),
                                                       out.ctypes.data if record else None, C.byref(sec)))
        return (out[:steps].copy() if record else None), sec.value

    def prefill(self, tokens, pos0: int = 0) -> None:
        """forward() with lm_mode 0 of tokens at positions pos0.., in prompt chunks."""
        t = np.ascontiguousarray(tokens, np.int32)
        self.E.check(self.E.L.g4e_prefill(self.h, t.ctypes.data, t.size, pos0))

    def prefill_trace(self, tokens, pos0: int = 0, q8: bool = False):
        """prefill() that returns each layer's input rows, (n_layers + 1, n, dim):
        [l, t] is layer l's input for token t, [n_layers, t] the last output.
        With q8, also the Q8_K rows of every quantization point as raw
        BlockQ8_K bytes, (n_layers, n, Q8_SLOTS, Q8_SLOT_ELEMS // 256, 292)."""
        t = np.ascontiguousarray(tokens, np.int32)
        tr = np.zeros((self.n_layers + 1, t.size, self.dim), np.float32)
        if not q8:
            self.E.check(self.E.L.g4e_prefill_trace(self.h, t.ctypes.data, t.size, pos0, tr.ctypes.data))
            return tr
        qt = np.empty((self.n_layers, t.size, Q8_SLOTS, Q8_SLOT_ELEMS // 256, 292), np.uint8)
        self.E.check(self.E.L.g4e_prefill_trace_q8(self.h, t.ctypes.data, t.size, pos0, tr.ctypes.data,
                                                   qt.ctypes.data))
        return tr, qt

    def kv_info(self, layer: int):
        """(floats per slot, slots) of a storing layer's KV cache."""
        out = np.zeros(2, np.int32)
        self.E.check(self.E.L.g4e_kv_info(self.h, layer, out.ctypes.data))
        return int(out[0]), int(out[1])

    def set_dump_hidden_at(self, pos: int) -> None:
        """record the --dump-hidden-at fingerprints of position pos (-1: off)"""
        self.E.check(self.E.L.g4e_set_dump_hidden_at(self.h, pos))

    def hidden_stats(self) -> np.ndarray:
        """(2 n_layers + 1, 3) (sum, l2, max): after the embedding, then per
        layer after the attention residual and at the layer's end"""
        out = np.zeros((2 * self.n_layers + 1, 3), np.float32)
        self.E.check(self.E.L.g4e_hidden_stats(self.h, out.ctypes.data))
        return out

    def kv_fingerprint(self):
        """layer-0 dump_kv_fingerprint records of the last dump: ((7, 7)
        floats: per tag sum, l2, max, v0..v3; have[7])"""
        out = np.zeros((7, 7), np.float32)
        have = np.zeros(7, np.int32)
        self.E.check(self.E.L.g4e_kv_fingerprint(self.h, out.ctypes.data, have.ctypes.data))
        return out, have.astype(bool)

    def set_f32_matmul(self, on: bool) -> None:
        """Q4_K/Q5_K through dequantized fp32 weights (the reference's
        --f32-matmul) instead of Q8_K integer dots."""
        self.E.check(self.E.L.g4e_set_f32_matmul(self.h, int(on)))

    def set_prefill_chunk(self, tokens: int) -> None:
        """Tokens per prompt chunk of prefill(); 0: generate_greedy prefills
        token by token."""
        self.E.check(self.E.L.g4e_set_prefill_chunk(self.h, tokens))

    def kv(self, layer: int, slot0: int, nslots: int):
        """(K, V) cache rows slot0..slot0+nslots-1 of a storing layer, each
        n_kv * head_dim floats."""
        kvd, _ = self.kv_info(layer)
        k = np.zeros((nslots, kvd), np.float32)
        v = np.zeros_like(k)
        self.E.check(self.E.L.g4e_read_kv(self.h, layer, slot0, nslots, k.ctypes.data, v.ctypes.data))
        return k, v

    def close(self) -> None:
        if self.h:
            self.E.L.g4e_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Vocab:
    """The engine's text path (host/text.h) over a GGUF's tokenizer metadata."""

    def __init__(self, path: str):
        self.E = EngineLib.get()
        L = self.E.L
        for name, (res, args) in _TEXT_SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        h = VP()
        rc = L.g4t_open_file(os.fsencode(path), C.byref(h))
        if rc:
            raise G4Error(rc, L.g4t_last_error().decode())
        self.L, self.h = L, h.value
        self.size = L.g4t_size(self.h)

    def _check(self, rc: int) -> int:
        if rc < 0:
            raise G4Error(rc, self.L.g4t_last_error().decode())
        return rc

    def specials(self) -> list[int]:
        out = np.zeros(13, np.int32)
        self.L.g4t_specials(self.h, out.ctypes.data)
        return [int(v) for v in out]

    def score(self, i: int) -> float:
        return float(self.L.g4t_score(self.h, i))

    def lookup(self, piece: bytes) -> int:
        return int(self.L.g4t_lookup(self.h, piece, len(piece)))

    def encode_raw(self, data: bytes, cap: int = 1 << 16) -> list[int]:
        out = np.zeros(cap, np.int32)
        n = self._check(self.L.g4t_encode_raw(self.h, data, len(data), out.ctypes.data, cap))
        return [int(v) for v in out[:n]]

    def encode_text(self, text: bytes, cap: int = 1 << 16) -> list[int]:
        out = np.zeros(cap, np.int32)
        n = self._check(self.L.g4t_encode_text(self.h, text, out.ctypes.data, cap))
        return [int(v) for v in out[:n]]

    def chat_encode(self, msgs: list[tuple[int, bytes]], thinking: bool, cap: int = 8192) -> list[int]:
        texts = (C.c_char_p * max(len(msgs), 1))(*[t for _, t in msgs])
        roles = np.array([r for r, _ in msgs] or [0], np.int32)
        out = np.zeros(max(cap, 1), np.int32)
        n = self._check(self.L.g4t_chat_encode(self.h, texts, roles.ctypes.data, len(msgs), int(thinking),
                                               out.ctypes.data, cap))
        return [int(v) for v in out[:n]]

    def decode(self, toks, start: int = 0, end: int | None = None, cap: int = 1 << 20) -> bytes:
        t = np.ascontiguousarray(toks, np.int32)
        end = t.size if end is None else end
        buf = C.create_string_buffer(cap)
        n = self._check(self.L.g4t_decode(self.h, t.ctypes.data, start, end, buf, cap))
        return buf.raw[:n]

    def split_response(self, toks) -> tuple[int, int, int]:
        t = np.ascontiguousarray(toks, np.int32)
        a, b, c = C.c_int(), C.c_int(), C.c_int()
        self.L.g4t_split_response(self.h, t.ctypes.data, t.size, C.byref(a), C.byref(b), C.byref(c))
        return a.value, b.value, c.value

    def is_special(self, i: int) -> bool:
        return bool(self.L.g4t_is_special(self.h, i))

    def close(self) -> None:
        if self.h:
            self.L.g4t_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TextStream:
    """g4t_stream: the thinking/answer state machine of generation."""

    class _S(C.Structure):
        _fields_ = [("v", VP)] + [(n, C.c_int) for n in ("thinking", "show", "budget", "mode", "saw_thought",
                                                         "saw_answer", "skipping_label", "thinking_tokens",
                                                         "budget_hit")]

    def __init__(self, vocab: Vocab, thinking: bool, show: bool, budget: int):
        self.v = vocab
        self.s = TextStream._S()
        vocab.L.g4t_stream_init(C.byref(self.s), vocab.h, int(thinking), int(show), budget)

    def force(self) -> int:
        return int(self.v.L.g4t_stream_force(C.byref(self.s)))

    def push(self, tok: int) -> bytes:
        buf = C.create_string_buffer(4096)
        n = self.v.L.g4t_stream_push(C.byref(self.s), tok, buf, 4096)
        return buf.raw[:n]


_TEXT_SIGS = {
    "g4t_last_error": (C.c_char_p, []),
    "g4t_open_file": (I, [C.c_char_p, C.POINTER(VP)]),
    "g4t_close": (None, [VP]),
    "g4t_size": (I, [VP]),
    "g4t_specials": (None, [VP, VP]),
    "g4t_score": (F, [VP, I]),
    "g4t_lookup": (I, [VP, C.c_char_p, I]),
    "g4t_encode_raw": (I, [VP, C.c_char_p, I, VP, I]),
    "g4t_encode_text": (I, [VP, C.c_char_p, VP, I]),
    "g4t_chat_encode": (I, [VP, VP, VP, I, I, VP, I]),
    "g4t_is_special": (I, [VP, I]),
    "g4t_decode": (I, [VP, VP, I, I, C.c_char_p, SZ]),
    "g4t_split_response": (None, [VP, VP, I, VP, VP, VP]),
    "g4t_stream_init": (None, [VP, VP, I, I, I]),
    "g4t_stream_force": (I, [VP]),
    "g4t_stream_push": (I, [VP, I, C.c_char_p, SZ]),
}
