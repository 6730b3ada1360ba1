"""Synthetic K-quant workloads and GGUF images for the Gemma 4 E4B decode path.

Block generators follow the synthetic-input recipe of the measured
workloads: fp16 ``d``/``dmin`` = RNE(|N(0,1)| * 1e-3), 12 packed scale bytes
uniform, quant bytes uniform; Q6_K int8 sub-block scales uniform in
[-32, 31].  Block byte layouts are those of gemma4-4b/cpu-blas/main.c:94-116.

The GGUF writer emits exactly what the reference's loader reads
(main.c:841-966 metadata keys and tensor table, main.c:1328-1400 tensor
names), so one image feeds both the CPU oracle and the HIP engine.
"""
from __future__ import annotations

import dataclasses
import fnmatch
import os
import struct
from typing import Iterable

import numpy as np

QK_K = 256
F32, F16, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 12, 13, 14, 30
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210}
ELEM_BYTES = {F32: 4, F16: 2, BF16: 2}


def _f16_bits(a: np.ndarray) -> np.ndarray:
    # numpy's float32 -> float16 cast rounds to nearest even, subnormals included
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def _rand_bytes(rng: np.random.Generator, shape) -> np.ndarray:
    n = int(np.prod(shape))
    return np.frombuffer(rng.bytes(n), np.uint8).reshape(shape)


def rand_q4K(rng: np.random.Generator, rows: int, n: int) -> np.ndarray:
    """rows x (n/256) Q4_K blocks as a uint8 array [rows, nb*144]."""
    nb = n // QK_K
    blk = _rand_bytes(rng, (rows, nb, 144)).copy()
    blk[..., 0:2] = _f16_bits(np.abs(rng.standard_normal((rows, nb))) * 1e-3).view(np.uint8).reshape(rows, nb, 2)
    blk[..., 2:4] = _f16_bits(np.abs(rng.standard_normal((rows, nb))) * 1e-3).view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(rows, nb * 144)


def rand_q5K(rng: np.random.Generator, rows: int, n: int) -> np.ndarray:
    nb = n // QK_K
    blk = _rand_bytes(rng, (rows, nb, 176)).copy()
    blk[..., 0:2] = _f16_bits(np.abs(rng.standard_normal((rows, nb))) * 1e-3).view(np.uint8).reshape(rows, nb, 2)
    blk[..., 2:4] = _f16_bits(np.abs(rng.standard_normal((rows, nb))) * 1e-3).view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(rows, nb * 176)


def rand_q6K(rng: np.random.Generator, rows: int, n: int) -> np.ndarray:
    nb = n // QK_K
    blk = _rand_bytes(rng, (rows, nb, 210)).copy()
    blk[..., 192:208] = rng.integers(-32, 32, (rows, nb, 16), dtype=np.int8).view(np.uint8)
    blk[..., 208:210] = _f16_bits(np.abs(rng.standard_normal((rows, nb))) * 1e-3).view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(rows, nb * 210)


def rand_kquant(rng: np.random.Generator, qtype: int, rows: int, n: int) -> np.ndarray:
    return {Q4_K: rand_q4K, Q5_K: rand_q5K, Q6_K: rand_q6K}[qtype](rng, rows, n)


def rand_bf16(rng: np.random.Generator, rows: int, n: int, scale: float = 0.02) -> np.ndarray:
    a = (rng.standard_normal((rows, n), dtype=np.float32) * scale).view(np.uint32)
    # round to nearest even on the top 16 bits
    a = (a + 0x7FFF + ((a >> 16) & 1)) >> 16
    return a.astype(np.uint16)


# ---------------------------------------------------------------------------
# GGUF writer
# ---------------------------------------------------------------------------
GV_U8, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 = range(13)


def _gstr(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _gval(vt: int, v) -> bytes:
    if vt == GV_U32:
        return struct.pack("<I", v)
    if vt == GV_I32:
        return struct.pack("<i", v)
    if vt == GV_F32:
        return struct.pack("<f", v)
    if vt == GV_BOOL or vt == GV_U8:
        return struct.pack("<B", v)
    if vt == GV_U64:
        return struct.pack("<Q", v)
    if vt == GV_STR:
        return _gstr(v)
    raise ValueError(vt)


def _kv(key: str, vt: int, v) -> bytes:
    out = _gstr(key) + struct.pack("<I", vt)
    if vt == GV_ARR:
        et, items = v
        out += struct.pack("<IQ", et, len(items))
        if et == GV_STR:
            out += b"".join(_gstr(s) for s in items)
        else:
            out += b"".join(_gval(et, x) for x in items)
        return out
    return out + _gval(vt, v)


def tensor_nbytes(qtype: int, ne: tuple[int, ...]) -> int:
    n = int(np.prod(ne))
    if qtype in BLOCK_BYTES:
        return n // QK_K * BLOCK_BYTES[qtype]
    return n * ELEM_BYTES[qtype]


@dataclasses.dataclass
class TensorSpec:
    name: str
    qtype: int
    ne: tuple[int, ...]          # ne[0] = row length (GGUF order)
    make: object                 # callable(rng) -> np.ndarray of raw bytes / elements


def write_gguf(path: str, kvs: list[bytes], tensors: list[TensorSpec], seed: int, alignment: int = 32) -> int:
    """Write a GGUF v3 file; tensor data is generated one tensor at a time."""
    header = bytearray()
    header += struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kvs) + 1)
    header += _kv("general.alignment", GV_U32, alignment)
    for k in kvs:
        header += k
    off = 0
    offsets = []
    for t in tensors:
        offsets.append(off)
        nbytes = tensor_nbytes(t.qtype, t.ne)
        off += (nbytes + alignment - 1) // alignment * alignment
    for t, o in zip(tensors, offsets):
        header += _gstr(t.name) + struct.pack("<I", len(t.ne)) + struct.pack(f"<{len(t.ne)}Q", *t.ne)
        header += struct.pack("<IQ", t.qtype, o)
    pad = (-len(header)) % alignment
    header += b"\0" * pad
    rng = np.random.default_rng(seed)
    with open(path, "wb") as f:
        f.write(header)
        for t, o in zip(tensors, offsets):
            arr = np.ascontiguousarray(t.make(rng))
            raw = arr.view(np.uint8).reshape(-1)
            nbytes = tensor_nbytes(t.qtype, t.ne)
            if raw.size != nbytes:
                raise ValueError(f"{t.name}: {raw.size} bytes, expected {nbytes}")
            f.write(raw.tobytes())
            f.write(b"\0" * ((-nbytes) % alignment))
            del arr, raw
    return os.path.getsize(path)


# ---------------------------------------------------------------------------
# Gemma 4 model shapes
# ---------------------------------------------------------------------------
@dataclasses.dataclass
class ModelShape:
    dim: int = 2560
    hidden: int = 10240
    n_layers: int = 42
    n_heads: int = 8
    n_kv: int = 2
    hd_swa: int = 256
    hd_full: int = 512
    ple_dim: int = 256
    vocab: int = 262144
    window: int = 512
    swa_pattern: int = 6
    n_layer_kv: int = 24          # layers >= this read donors 22/23 (main.c:77, 739-746)
    rope_base: float = 1e6
    rope_base_swa: float = 1e4
    softcap: float = 30.0
    eps: float = 1e-6
    context: int = 8192
    q_type: int = Q4_K            # Q/K/O/gate/up/inp_gate/proj
    v_type: int = Q6_K            # V, down, token embeddings
    ffn_type: int = Q4_K          # gate/up (Q5_K variant possible)
    rope_freqs: bool = False      # include a rope_freqs.weight tensor
    types: tuple = ()             # (glob over tensor names, type) overrides, first match wins
    zeros: tuple = ()             # globs over tensor names whose bytes are all zero
    pieces: tuple = ()            # tokenizer pieces (default: <t0>.. placeholders) ...
    merges: tuple = ()            # ... and merges ("a b") for a model that can tokenize text

    def is_swa(self, l: int) -> bool:
        return (l % self.swa_pattern) < (self.swa_pattern - 1)

    def head_dim(self, l: int) -> int:
        return self.hd_swa if self.is_swa(l) else self.hd_full


E4B = ModelShape()


def tiny_shape(**kw) -> ModelShape:
    """30 layers (so shared-KV readers of both donors exist) at small width."""
    base = dict(dim=256, hidden=512, n_layers=30, n_heads=2, n_kv=1, hd_swa=256, hd_full=512,
                ple_dim=256, vocab=512, window=8, context=64)
    base.update(kw)
    return ModelShape(**base)


def model_tensors(s: ModelShape) -> list[TensorSpec]:
    L = s.n_layers
    ts: list[TensorSpec] = []

    def norm(name, n, lo=0.8, hi=1.2):
        ts.append(TensorSpec(name, F32, (n,), lambda r, n=n: r.uniform(lo, hi, n).astype(np.float32)))

    def mat(name, qtype, n, d):
        for pat, t in s.types:
            if fnmatch.fnmatchcase(name, pat):
                qtype = t
                break
        if any(fnmatch.fnmatchcase(name, pat) for pat in s.zeros):
            ts.append(TensorSpec(name, qtype, (n, d), lambda r, q=qtype, n=n, d=d:
                                 np.zeros(tensor_nbytes(q, (n, d)), np.uint8)))
            return
        if qtype in (F16, F32):
            dt = np.float16 if qtype == F16 else np.float32
            ts.append(TensorSpec(name, qtype, (n, d), lambda r, n=n, d=d, dt=dt:
                                 (r.standard_normal((d, n), dtype=np.float32) * 0.02).astype(dt)))
        elif qtype == BF16:
            ts.append(TensorSpec(name, qtype, (n, d), lambda r, n=n, d=d: rand_bf16(r, d, n)))
        else:
            ts.append(TensorSpec(name, qtype, (n, d), lambda r, q=qtype, n=n, d=d: rand_kquant(r, q, d, n)))

    mat("token_embd.weight", s.v_type, s.dim, s.vocab)
    mat("per_layer_token_embd.weight", s.v_type, s.ple_dim * L, s.vocab)
    mat("per_layer_model_proj.weight", BF16, s.dim, s.ple_dim * L)
    norm("per_layer_proj_norm.weight", s.ple_dim)
    norm("output_norm.weight", s.dim)
    if s.rope_freqs:
        ts.append(TensorSpec("rope_freqs.weight", F32, (s.hd_full // 2,),
                             lambda r, n=s.hd_full // 2: r.uniform(1.0, 4.0, n).astype(np.float32)))
    for l in range(L):
        hd = s.head_dim(l)
        qd, kvd = s.n_heads * hd, s.n_kv * hd
        p = f"blk.{l}."
        norm(p + "attn_norm.weight", s.dim)
        norm(p + "post_attention_norm.weight", s.dim)
        norm(p + "attn_q_norm.weight", hd)
        norm(p + "attn_k_norm.weight", hd)
        mat(p + "attn_q.weight", s.q_type, s.dim, qd)
        if l < s.n_layer_kv:
            mat(p + "attn_k.weight", s.q_type, s.dim, kvd)
            mat(p + "attn_v.weight", s.v_type, s.dim, kvd)
        mat(p + "attn_output.weight", s.q_type, qd, s.dim)
        norm(p + "ffn_norm.weight", s.dim)
        norm(p + "post_ffw_norm.weight", s.dim)
        mat(p + "ffn_gate.weight", s.ffn_type, s.dim, s.hidden)
        mat(p + "ffn_up.weight", s.ffn_type, s.dim, s.hidden)
        mat(p + "ffn_down.weight", s.v_type, s.hidden, s.dim)
        mat(p + "inp_gate.weight", s.q_type, s.dim, s.ple_dim)
        mat(p + "proj.weight", s.q_type, s.ple_dim, s.dim)
        norm(p + "post_norm.weight", s.dim)
        norm(p + "layer_output_scale.weight", 1, 0.85, 0.95)
    return ts


def model_kvs(s: ModelShape) -> list[bytes]:
    a = "gemma4."
    kv = [
        _kv(a + "embedding_length", GV_U32, s.dim),
        _kv(a + "feed_forward_length", GV_U32, s.hidden),
        _kv(a + "block_count", GV_U32, s.n_layers),
        _kv(a + "attention.head_count", GV_U32, s.n_heads),
        _kv(a + "attention.head_count_kv", GV_U32, s.n_kv),
        _kv(a + "attention.key_length_swa", GV_U32, s.hd_swa),
        _kv(a + "attention.key_length", GV_U32, s.hd_full),
        _kv(a + "rope.dimension_count_swa", GV_U32, s.hd_swa),
        _kv(a + "rope.dimension_count", GV_U32, s.hd_full),
        _kv(a + "attention.layer_norm_rms_epsilon", GV_F32, s.eps),
        _kv(a + "rope.freq_base", GV_F32, s.rope_base),
        _kv(a + "rope.freq_base_swa", GV_F32, s.rope_base_swa),
        _kv(a + "attention.sliding_window", GV_U32, s.window),
        _kv(a + "attention.shared_kv_layers", GV_U32, s.n_layers - s.n_layer_kv),
        _kv(a + "embedding_length_per_layer_input", GV_U32, s.ple_dim),
        _kv(a + "final_logit_softcapping", GV_F32, s.softcap),
        _kv(a + "context_length", GV_U32, s.context),
        _kv(a + "attention.sliding_window_pattern", GV_ARR,
            (GV_BOOL, [1 if s.is_swa(l) else 0 for l in range(s.n_layers)])),
        _kv("tokenizer.ggml.eos_token_id", GV_U32, 106 if s.vocab > 106 else s.vocab - 1),
        _kv("tokenizer.ggml.tokens", GV_ARR, (GV_STR, list(s.pieces) + [f"<t{i}>" for i in range(len(s.pieces),
                                                                                                 s.vocab)])),
    ]
    if s.merges:
        kv.append(_kv("tokenizer.ggml.merges", GV_ARR, (GV_STR, list(s.merges))))
    return kv


def write_model_gguf(path: str, s: ModelShape, seed: int, alignment: int = 32) -> int:
    return write_gguf(path, model_kvs(s), model_tensors(s), seed, alignment)


def decode_weight_bytes(s: ModelShape) -> int:
    """Weight bytes streamed by one decode step (everything but the per-layer
    token embedding table, of which one row is read)."""
    total = 0
    for t in model_tensors(s):
        if t.name == "per_layer_token_embd.weight" or t.qtype == F32:
            continue
        total += tensor_nbytes(t.qtype, t.ne)
    return total


def prefill_matmuls(s: ModelShape) -> list[tuple[str, int, int, int]]:
    """(name, type, n, d) of the matrices a prompt token runs through in the
    batched prefill: every 2-D tensor but the two embedding tables (looked
    up, not multiplied; the LM head runs only for the last token)."""
    return [(t.name, t.qtype, t.ne[0], t.ne[1]) for t in model_tensors(s)
            if len(t.ne) == 2 and t.name not in ("token_embd.weight", "per_layer_token_embd.weight")]


def e4b_gguf(seed: int = 4) -> str:
    """Path of the synthetic E4B-shape GGUF of `seed` (about 5.4 GB), written
    once per machine into /dev/shm (or /tmp)."""
    d = "/dev/shm" if os.path.isdir("/dev/shm") else "/tmp"
    path = os.path.join(d, f"g4_e4b_seed{seed}.gguf")
    if not os.path.exists(path):
        tmp = path + f".{os.getpid()}.part"
        write_model_gguf(tmp, E4B, seed)
        os.replace(tmp, path)
    return path


# ---------------------------------------------------------------------------
# Synthetic tokenizer vocabularies (tokenizer.ggml.* metadata only)
# ---------------------------------------------------------------------------
SP = "▁"   # the escaped space of Gemma pieces


def escape_line(line: str, prefix: bool) -> str:
    """a text line as the tokenizer sees it: spaces as U+2581, and one
    leading when the vocabulary asks for a space prefix"""
    s = line.replace(" ", SP)
    return (SP + s) if (prefix and line) else s


def bpe_train(lines: list[str], n_merges: int, prefix: bool) -> list[tuple[str, str]]:
    """Merges learned greedily from the escaped lines: the most frequent
    adjacent pair first (ties: the smallest pair)."""
    seqs = [list(escape_line(l, prefix)) for l in lines if l]
    merges = []
    for _ in range(n_merges):
        counts: dict[tuple[str, str], int] = {}
        for s in seqs:
            for a, b in zip(s, s[1:]):
                counts[(a, b)] = counts.get((a, b), 0) + 1
        if not counts:
            break
        best = min(counts, key=lambda p: (-counts[p], p))
        merges.append(best)
        for i, s in enumerate(seqs):
            out, j = [], 0
            while j < len(s):
                if j + 1 < len(s) and (s[j], s[j + 1]) == best:
                    out.append(s[j] + s[j + 1])
                    j += 2
                else:
                    out.append(s[j])
                    j += 1
            seqs[i] = out
    return merges


def write_vocab_gguf(path: str, pieces: list[str | bytes], merges: list[str] | None = None,
                     scores: list[float] | None = None, bos: int = 2, eos: int = 106,
                     add_space_prefix: bool | None = None) -> int:
    """A GGUF that holds only tokenizer metadata (no tensors)."""
    kvs = [_kv("tokenizer.ggml.model", GV_STR, "gemma4"),
           _kv("tokenizer.ggml.tokens", GV_ARR, (GV_STR, pieces)),
           _kv("tokenizer.ggml.bos_token_id", GV_U32, bos),
           _kv("tokenizer.ggml.eos_token_id", GV_U32, eos)]
    if scores is not None:
        kvs.append(_kv("tokenizer.ggml.scores", GV_ARR, (GV_F32, list(scores))))
    if merges is not None:
        kvs.append(_kv("tokenizer.ggml.merges", GV_ARR, (GV_STR, merges)))
    if add_space_prefix is not None:
        kvs.append(_kv("tokenizer.ggml.add_space_prefix", GV_BOOL, int(add_space_prefix)))
    return write_gguf(path, kvs, [], seed=0)
