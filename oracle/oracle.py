"""ctypes bindings for the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker.  ``Oracle`` wraps liboracle.so (the C
restatement of gemma4-4b/cpu-blas/main.c); ``Ref`` wraps _ref/libg4ref.so,
the reference's own BLAS-free functions compiled from main.c (present only
where the reference tree was available when the library was built).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libg4ref.so")

Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert Q8K_DTYPE.itemsize == 292
# quantization points of a layer (g4_oracle.h OR_Q8_SLOT_*): attention input,
# O input, FFN input, PLE inp_gate input, PLE proj input
Q8_SLOTS, Q8_SLOT_BLOCKS = 5, 16
Q8_SLOT_NAMES = ("attn", "o", "ffn", "inp_gate", "proj")

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
VP = C.c_void_p


def build(force: bool = False) -> None:
    if force or not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-s", "-C", HERE], check=True)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        self.L = L
        sig = {
            "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "or_f32_to_f16": (C.c_uint16, [C.c_float]),
            "or_scale_min_k4": (None, [C.c_int, VP, VP, VP]),
            "or_unpack_scales_words": (None, [VP, VP, VP]),
            "or_dequant_block": (None, [VP, C.c_int, VP]),
            "or_quantize_q8K": (None, [VP, VP, C.c_int]),
            "or_q4K_lane_sums": (None, [VP, VP, VP, VP]),
            "or_q5K_lane_sums": (None, [VP, VP, VP, VP]),
            "or_q4K_block_SM": (None, [VP, VP, VP, VP]),
            "or_q5K_block_SM": (None, [VP, VP, VP, VP]),
            "or_q6K_block_S": (C.c_int32, [VP, VP]),
            "or_vec_dot_q4K_q8K": (C.c_float, [C.c_int, VP, VP]),
            "or_vec_dot_q5K_q8K": (C.c_float, [C.c_int, VP, VP]),
            "or_vec_dot_q4K_q8K_generic": (C.c_float, [C.c_int, VP, VP]),
            "or_vec_dot_q5K_q8K_generic": (C.c_float, [C.c_int, VP, VP]),
            "or_vec_dot_q6K_q8K": (C.c_float, [C.c_int, VP, VP]),
            "or_mm_quant_rows": (None, [VP, VP, VP, C.c_int, C.c_int, C.c_int]),
            "or_mm_quant_dot_rows": (None, [VP, VP, C.c_int, C.c_int, C.c_int, VP]),
            "or_mm_bf16": (None, [VP, VP, VP, C.c_int, C.c_int]),
            "or_mm_f16": (None, [VP, VP, VP, C.c_int, C.c_int]),
            "or_mm_f32": (None, [VP, VP, VP, C.c_int, C.c_int]),
            "or_set_f32_matmul": (None, [C.c_int]),
            "or_mm": (C.c_int, [VP, VP, VP, C.c_int, C.c_int, C.c_int, VP, C.c_int]),
            "or_rmsnorm": (None, [VP, VP, VP, C.c_int, C.c_float]),
            "or_rmsnorm_head_inplace": (None, [VP, VP, C.c_int, C.c_int, C.c_float]),
            "or_rmsnorm_head_noweight_inplace": (None, [VP, C.c_int, C.c_int, C.c_float]),
            "or_softmax": (None, [VP, C.c_int]),
            "or_gelu": (C.c_float, [C.c_float]),
            "or_apply_rope_neox": (None, [VP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, VP]),
            "or_emb_lookup": (C.c_int, [VP, VP, C.c_int, C.c_int, C.c_int]),
            "or_attn_decode": (None, [VP, VP, VP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_float, VP, VP]),
            "or_rng_f32": (C.c_float, [VP]),
            "or_sample_token": (C.c_int, [VP, C.c_int, C.c_float, C.c_float, C.c_int, VP]),
            "or_apply_repetition_penalty": (None, [VP, VP, C.c_int, C.c_float, C.c_int]),
            "or_argmax_first": (C.c_int, [VP, C.c_int]),
            "or_hidden_stats": (None, [VP, C.c_int, VP, VP, VP]),
            "or_model_open": (VP, [VP, C.c_size_t, C.c_int, C.c_char_p, C.c_size_t]),
            "or_model_close": (None, [VP]),
            "or_model_config": (None, [VP, VP]),
            "or_forward": (C.c_int, [VP, C.c_int, C.c_int, C.c_int]),
            "or_forward_inject": (C.c_int, [VP, C.c_int, C.c_int, C.c_int, VP, VP]),
            "or_model_logits": (VP, [VP]),
            "or_model_x": (VP, [VP]),
            "or_model_layer_stats": (VP, [VP]),
            "or_model_attn_stats": (VP, [VP]),
            "or_model_layer_x": (VP, [VP]),
            "or_generate_greedy": (C.c_int, [VP, VP, C.c_int, C.c_int, VP, VP, VP]),
            "or_forward_inject_q8": (C.c_int, [VP, C.c_int, C.c_int, C.c_int, VP, VP, VP]),
            "or_forward_inject_kv": (C.c_int, [VP, C.c_int, C.c_int, VP, VP]),
            "or_model_q8_rec": (VP, [VP]),
            "or_model_kv_source": (C.c_int, [VP, C.c_int]),
            "or_model_fingerprint": (C.POINTER(C.c_float), [VP, VP]),
            "or_embed": (C.c_int, [VP, C.c_int, C.c_int]),
            "or_layer_inject": (C.c_int, [VP, C.c_int, C.c_int, C.c_int, VP, VP]),
            "or_lm_head_inject": (C.c_int, [VP, VP]),
            "or_model_state": (C.POINTER(C.c_float), [VP, C.c_char_p]),
            "or_model_kv": (C.POINTER(C.c_float), [VP, C.c_int, C.c_int]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args

    # ---- thin numpy helpers -------------------------------------------------
    def quantize_q8K(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(x.size // 256, Q8K_DTYPE)
        self.L.or_quantize_q8K(_ptr(x), _ptr(y), x.size)
        return y

    def dequant(self, blocks: np.ndarray, qtype: int, n: int) -> np.ndarray:
        from_bytes = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
        bs = {12: 144, 13: 176, 14: 210}[qtype]
        nb = from_bytes.size // bs
        out = np.empty(nb * 256, np.float32)
        for b in range(nb):
            self.L.or_dequant_block(_ptr(from_bytes) + b * bs, qtype, _ptr(out) + b * 1024)
        return out

    def mm_quant_rows(self, x, w, n, d, qtype) -> np.ndarray:
        o = np.empty(d, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w)
        self.L.or_mm_quant_rows(_ptr(o), _ptr(x), _ptr(w), n, d, qtype)
        return o

    def mm_quant_dot_rows(self, w, n, d, qtype, q8) -> np.ndarray:
        o = np.empty(d, np.float32)
        w = np.ascontiguousarray(w)
        self.L.or_mm_quant_dot_rows(_ptr(o), _ptr(w), n, d, qtype, _ptr(q8))
        return o

    def mm_bf16(self, x, w, n, d) -> np.ndarray:
        o = np.empty(d, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.uint16)
        self.L.or_mm_bf16(_ptr(o), _ptr(x), _ptr(w), n, d)
        return o

    def rmsnorm(self, x, w, eps=1e-6) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        o = np.empty_like(x)
        self.L.or_rmsnorm(_ptr(o), _ptr(x), _ptr(w), x.size, eps)
        return o

    def rope(self, v, n_heads, hd, n_rot, pos, base, ff=None) -> np.ndarray:
        v = np.array(v, np.float32, copy=True)
        ffp = None if ff is None else np.ascontiguousarray(ff, np.float32)
        self.L.or_apply_rope_neox(_ptr(v), n_heads, hd, n_rot, pos, base, 1.0,
                                  None if ffp is None else _ptr(ffp))
        return v

    def attn(self, q, kc, vc, kv_stride, t_start, nwin, n_heads, n_kv, hd, scale) -> np.ndarray:
        q = np.ascontiguousarray(q, np.float32)
        kc = np.ascontiguousarray(kc, np.float32)
        vc = np.ascontiguousarray(vc, np.float32)
        att = np.zeros(n_heads * (t_start + nwin) + 1, np.float32)
        out = np.zeros(n_heads * hd, np.float32)
        self.L.or_attn_decode(_ptr(q), _ptr(kc), _ptr(vc), kv_stride, t_start, nwin, n_heads, n_kv, hd,
                              scale, _ptr(att), _ptr(out))
        return out


class OracleModel:
    """forward() of the oracle over a GGUF image (file path, memory-mapped)."""

    def __init__(self, orc: Oracle, path: str, max_seq: int = 0):
        self.o = orc
        self.mm = np.memmap(path, np.uint8, mode="r")
        err = C.create_string_buffer(256)
        h = orc.L.or_model_open(_ptr(self.mm), self.mm.size, max_seq, err, 256)
        if not h:
            raise RuntimeError(err.value.decode())
        self.h = h
        cfg = np.zeros(9, np.int32)
        orc.L.or_model_config(h, _ptr(cfg))
        (self.dim, self.hidden, self.n_layers, self.n_heads, self.n_kv, self.vocab,
         self.max_seq, self.ple_dim, self.window) = [int(v) for v in cfg]

    def forward(self, token: int, pos: int, lm_mode: int = 1) -> None:
        if self.o.L.or_forward(self.h, token, pos, lm_mode) != 0:
            raise RuntimeError("or_forward failed")

    def forward_inject(self, token: int, pos: int, lm_mode: int, x_in: np.ndarray) -> np.ndarray:
        """Each layer run from the given input rows; returns the layer outputs."""
        x_in = np.ascontiguousarray(x_in, np.float32)
        assert x_in.shape == (self.n_layers + 1, self.dim)
        out = np.empty((self.n_layers, self.dim), np.float32)
        if self.o.L.or_forward_inject(self.h, token, pos, lm_mode, _ptr(x_in), _ptr(out)) != 0:
            raise RuntimeError("or_forward_inject failed")
        return out

    def forward_inject_q8(self, token: int, pos: int, lm_mode: int, x_in: np.ndarray,
                          q8_in: np.ndarray) -> np.ndarray:
        """forward_inject with every Q8_K activation taken from q8_in
        ((n_layers, Q8_SLOTS, Q8_SLOT_BLOCKS) of Q8K_DTYPE, as q8_rec())."""
        x_in = np.ascontiguousarray(x_in, np.float32)
        assert x_in.shape == (self.n_layers + 1, self.dim)
        q8_in = np.ascontiguousarray(q8_in)
        assert q8_in.dtype == Q8K_DTYPE and q8_in.shape == (self.n_layers, Q8_SLOTS, Q8_SLOT_BLOCKS)
        out = np.empty((self.n_layers, self.dim), np.float32)
        if self.o.L.or_forward_inject_q8(self.h, token, pos, lm_mode, _ptr(x_in), _ptr(q8_in), _ptr(out)) != 0:
            raise RuntimeError("or_forward_inject_q8 failed")
        return out

    def forward_inject_kv(self, token: int, pos: int, x_in: np.ndarray, q8_in: np.ndarray | None = None) -> None:
        """K/V of every storing layer at pos from the injected layer inputs
        (and, if given, the injected Q8_K as forward_inject_q8)."""
        x_in = np.ascontiguousarray(x_in, np.float32)
        assert x_in.shape == (self.n_layers + 1, self.dim)
        qp = None
        if q8_in is not None:
            q8_in = np.ascontiguousarray(q8_in)
            assert q8_in.dtype == Q8K_DTYPE and q8_in.shape == (self.n_layers, Q8_SLOTS, Q8_SLOT_BLOCKS)
            qp = _ptr(q8_in)
        if self.o.L.or_forward_inject_kv(self.h, token, pos, _ptr(x_in), qp) != 0:
            raise RuntimeError("or_forward_inject_kv failed")

    def q8_rec(self) -> np.ndarray:
        """The oracle's own Q8_K of every quantization point in the last
        forward: (n_layers, Q8_SLOTS, Q8_SLOT_BLOCKS) of Q8K_DTYPE."""
        p = self.o.L.or_model_q8_rec(self.h)
        n = self.n_layers * Q8_SLOTS * Q8_SLOT_BLOCKS
        raw = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), (n * Q8K_DTYPE.itemsize,))
        return raw.copy().view(Q8K_DTYPE).reshape(self.n_layers, Q8_SLOTS, Q8_SLOT_BLOCKS)

    def embed(self, token: int, pos: int) -> None:
        """embedding and build_ple of a token (state x and ple)"""
        if self.o.L.or_embed(self.h, token, pos) != 0:
            raise RuntimeError("or_embed failed")

    def layer_inject(self, token: int, pos: int, layer: int, x_in: np.ndarray) -> np.ndarray:
        """one layer from an injected input; its intermediates stay in state()"""
        x_in = np.ascontiguousarray(x_in, np.float32)
        out = np.empty(self.dim, np.float32)
        if self.o.L.or_layer_inject(self.h, token, pos, layer, _ptr(x_in), _ptr(out)) != 0:
            raise RuntimeError("or_layer_inject failed")
        return out

    def lm_head_inject(self, x_in: np.ndarray) -> np.ndarray:
        x_in = np.ascontiguousarray(x_in, np.float32)
        if self.o.L.or_lm_head_inject(self.h, _ptr(x_in)) != 0:
            raise RuntimeError("or_lm_head_inject failed")
        return self.logits()

    def state(self, name: str, n: int) -> np.ndarray:
        """copy of the first n floats of a state buffer"""
        p = self.o.L.or_model_state(self.h, name.encode())
        if not p:
            raise ValueError(name)
        return np.ctypeslib.as_array(p, (n,)).copy()

    def kv_fingerprint(self):
        """layer-0 fingerprints of the last forward: ((7 tags, 7) floats, have[7])"""
        have = np.zeros(7, np.int32)
        p = self.o.L.or_model_fingerprint(self.h, _ptr(have))
        return np.ctypeslib.as_array(p, (7, 7)).copy(), have.astype(bool)

    def kv_source(self, layer: int) -> int:
        """the layer whose KV cache `layer` reads (main.c:739-746)"""
        return int(self.o.L.or_model_kv_source(self.h, layer))

    def kv(self, layer: int):
        """(K, V) cache views of a storing layer: (max_seq, 1024) float32,
        writable (main.c:1798-1809 layout)."""
        out = []
        for which in (0, 1):
            p = self.o.L.or_model_kv(self.h, layer, which)
            if not p:
                raise ValueError(f"layer {layer} stores no KV")
            out.append(np.ctypeslib.as_array(p, (self.max_seq, 1024)))
        return out[0], out[1]

    def logits(self) -> np.ndarray:
        p = self.o.L.or_model_logits(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (self.vocab,)).copy()

    def x(self) -> np.ndarray:
        p = self.o.L.or_model_x(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (self.dim,)).copy()

    def layer_stats(self) -> np.ndarray:
        p = self.o.L.or_model_layer_stats(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (self.n_layers * 3 + 8,)).copy()

    def attn_stats(self) -> np.ndarray:
        """(n_layers, 3): hidden_stats after each layer's attention residual"""
        p = self.o.L.or_model_attn_stats(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (self.n_layers * 3,)).copy().reshape(-1, 3)

    def layer_x(self) -> np.ndarray:
        p = self.o.L.or_model_layer_x(self.h)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (self.n_layers, self.dim)).copy()

    def generate_greedy(self, prompt, max_new):
        pr = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max_new + 1, np.int32)
        ps, ds = C.c_double(), C.c_double()
        n = self.o.L.or_generate_greedy(self.h, _ptr(pr), pr.size, max_new, _ptr(out), C.byref(ps), C.byref(ds))
        if n < 0:
            raise RuntimeError("or_generate_greedy failed")
        return out[:n].copy(), ps.value, ds.value

    def close(self):
        if self.h:
            self.o.L.or_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Ref:
    """The reference's own functions (oracle/_ref/libg4ref.so)."""

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_SO)

    def __init__(self, path: str = REF_SO):
        L = C.CDLL(path)
        self.L = L
        sig = {
            "ref_quantize_row_q8_K": (None, [VP, VP, C.c_int]),
            "ref_quantize_row_q8_K_ref": (None, [VP, VP, C.c_int]),
            "ref_vec_dot_q4_K_q8_K": (C.c_float, [C.c_int, VP, VP]),
            "ref_vec_dot_q5_K_q8_K": (C.c_float, [C.c_int, VP, VP]),
            "ref_vec_dot_q4_K_q8_K_generic": (C.c_float, [C.c_int, VP, VP]),
            "ref_vec_dot_q5_K_q8_K_generic": (C.c_float, [C.c_int, VP, VP]),
            "ref_host_f16f32": (C.c_float, [C.c_ushort]),
            "ref_host_bf16f32": (C.c_float, [C.c_ushort]),
            "ref_get_scale_min_k4": (None, [C.c_int, VP, VP, VP]),
            "ref_dequant_block": (None, [VP, C.c_int, VP]),
            "ref_mm_quant_rows": (None, [VP, VP, VP, C.c_int, C.c_int, C.c_int]),
            "ref_mm_quant_dot_rows": (None, [VP, VP, C.c_int, C.c_int, C.c_int, VP]),
            "ref_mm_bf16": (None, [VP, VP, VP, C.c_int, C.c_int]),
            "ref_mm_f16": (None, [VP, VP, VP, C.c_int, C.c_int]),
            "ref_rmsnorm": (None, [VP, VP, VP, C.c_int, C.c_float]),
            "ref_rmsnorm_head_inplace": (None, [VP, VP, C.c_int, C.c_int, C.c_float]),
            "ref_rmsnorm_head_noweight_inplace": (None, [VP, C.c_int, C.c_int, C.c_float]),
            "ref_softmax": (None, [VP, C.c_int]),
            "ref_gelu": (C.c_float, [C.c_float]),
            "ref_apply_rope_neox": (None, [VP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, VP]),
            "ref_emb_lookup": (None, [VP, VP, C.c_int, C.c_int, C.c_int]),
            "ref_rng_f32": (C.c_float, [VP]),
            "ref_sample_token": (C.c_int, [VP, C.c_int, C.c_float, C.c_float, C.c_int, VP]),
            "ref_apply_repetition_penalty": (None, [VP, VP, C.c_int, C.c_float, C.c_int]),
            "ref_is_swa_layer": (C.c_int, [C.c_int, C.c_int, C.c_int]),
            "ref_kv_source_for_layer": (C.c_int, [C.c_int, C.c_int, C.c_int]),
            "ref_layer_head_dim": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
            "ref_model_open": (VP, [VP, C.c_size_t]),
            "ref_model_config": (None, [VP, VP, VP, VP]),
            "ref_model_is_swa": (C.c_int, [VP, C.c_int]),
            "ref_model_kv_source": (C.c_int, [VP, C.c_int]),
            "ref_model_tensor": (VP, [VP, C.c_char_p, VP]),
            "ref_tok_specials": (None, [VP, VP]),
            "ref_tok_score": (C.c_float, [VP, C.c_int]),
            "ref_tok_lookup": (C.c_int, [VP, C.c_char_p, C.c_int]),
            "ref_bpe_encode": (C.c_int, [VP, C.c_char_p, C.c_int, VP]),
            "ref_gemma_text": (C.c_int, [VP, C.c_char_p, VP]),
            "ref_chat_encode": (C.c_int, [VP, C.c_char_p, C.c_int, VP]),
            "ref_hidden_stats": (None, [VP, C.c_int, VP, VP, VP]),
            "ref_kv_cache_offset": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
            "ref_tok_open": (VP, [VP, C.c_size_t]),
            "ref_chat_encode_history": (C.c_int, [VP, VP, VP, C.c_int, C.c_int, VP, C.c_int]),
            "ref_tokens_to_text": (C.c_int, [VP, VP, C.c_int, C.c_int, VP, C.c_int]),
            "ref_parse_response": (None, [VP, VP, C.c_int, VP, VP, VP, VP, C.c_int]),
            "ref_is_special": (C.c_int, [VP, C.c_int]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
