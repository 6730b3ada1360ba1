"""Pins of the oracle's model-level functions (or_model_open, build_ple, the
layer step, the final norm and logits_tied, or_hidden_stats, or_mm_f32)
against the reference itself.

The reference's forward() (gemma4-4b/cpu-blas/main.c:1838-2029) cannot be
compiled here: its attention and mm_f32 call OpenBLAS, which this image
lacks.  Everything it calls besides those is compiled from main.c into
oracle/_ref: the GGUF reader and load_weights (main.c:778-966, 1318-1400),
the norms, Q8_K quantizer, K-quant and bf16 GEMVs, RoPE, GELU, emb_lookup
and hidden_stats.  So each piece of forward() is composed here, in
forward()'s statement order, from those functions and the weight pointers
of the reference's own load_weights, and the oracle must match it bit for
bit.  The attention block (main.c:1909-1950) is taken in float64 by brute
force; the composition then continues from the oracle's attention output,
so the layer's remaining statements are still compared bit for bit.

Invariants a plausible slip would break: with zero attention-output, FFN
down and PLE projection weights a layer is out_scale times its input,
exactly; shared-KV layers read donor 22 (sliding) or 23 (full) and nothing
else; the GGUF data offset follows general.alignment; the vocabulary size
is the token list's length.
"""
import ctypes as C

import numpy as np
import pytest

import synth
from oracle import Q8K_DTYPE, OracleModel

F32P = C.POINTER(C.c_float)
LIBM = C.CDLL("libm.so.6")
LIBM.tanhf.restype = C.c_float
LIBM.tanhf.argtypes = [C.c_float]


def _p(a):
    return a.ctypes.data


class RefModel:
    """The reference's own parse_gguf + load_weights over a GGUF file."""

    def __init__(self, ref, path):
        self.ref = ref
        self.buf = np.fromfile(path, np.uint8)
        self.h = ref.L.ref_model_open(_p(self.buf), self.buf.size)
        i = np.zeros(15, np.int32)
        f = np.zeros(4, np.float32)
        doff = C.c_ulonglong()
        ref.L.ref_model_config(self.h, _p(i), _p(f), C.byref(doff))
        (self.dim, self.hidden, self.L, self.nh, self.nkv, self.vocab, self.max_seq, self.pd, self.window,
         self.shared_kv, self.swa_pattern, self.hd_swa, self.hd_full, self.rot_swa, self.rot_full) = [int(v) for v in i]
        self.theta, self.theta_swa, self.eps, self.softcap = [np.float32(v) for v in f]
        self.doff = doff.value
        self.ints, self.floats = i, f

    def t(self, name):
        """(pointer, type) of a tensor, from the reference's find_tensor"""
        ty = C.c_int()
        p = self.ref.L.ref_model_tensor(self.h, name.encode(), C.byref(ty))
        return p, ty.value

    def vec(self, name, n):
        p, _ = self.t(name)
        return None if not p else np.ctypeslib.as_array(C.cast(p, F32P), (n,)).copy()

    def swa(self, l):
        return bool(self.ref.L.ref_model_is_swa(self.h, l))

    def src(self, l):
        return int(self.ref.L.ref_model_kv_source(self.h, l))

    def hd(self, l):
        return self.hd_swa if self.swa(l) else self.hd_full


class Compose:
    """forward()'s statements over the reference's primitives (ref_*)."""

    def __init__(self, ref, rm: RefModel):
        self.r, self.m = ref.L, rm

    def rmsnorm(self, x, w):
        o = np.empty_like(x)
        self.r.ref_rmsnorm(_p(o), _p(np.ascontiguousarray(x)), _p(w), x.size, C.c_float(self.m.eps))
        return o

    def quantize(self, x):
        q8 = np.zeros(x.size // 256, Q8K_DTYPE)
        self.r.ref_quantize_row_q8_K(_p(np.ascontiguousarray(x)), _p(q8), x.size)
        return q8

    def mm(self, x, name, n, d, q8=None):
        """mm(o, x, w, n, d, type, q8, q8_ready), main.c:1669-1694; returns (o, q8 used)"""
        p, ty = self.m.t(name)
        o = np.empty(d, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        if ty in (12, 13):
            if q8 is None:
                q8 = self.quantize(x)
            self.r.ref_mm_quant_dot_rows(_p(o), p, n, d, ty, _p(q8))
        elif ty == 14:
            self.r.ref_mm_quant_rows(_p(o), _p(x), p, n, d, ty)
        elif ty == 30:
            self.r.ref_mm_bf16(_p(o), _p(x), p, n, d)
        elif ty == 1:
            self.r.ref_mm_f16(_p(o), _p(x), p, n, d)
        else:
            raise NotImplementedError(ty)
        return o, q8

    def head_norm(self, v, w, nh, hd):
        v = v.copy()
        if w is None:
            self.r.ref_rmsnorm_head_noweight_inplace(_p(v), nh, hd, C.c_float(self.m.eps))
        else:
            self.r.ref_rmsnorm_head_inplace(_p(v), _p(w), nh, hd, C.c_float(self.m.eps))
        return v

    def rope(self, v, nh, hd, n_rot, pos, base, ff):
        v = v.copy()
        self.r.ref_apply_rope_neox(_p(v), nh, hd, n_rot, pos, C.c_float(base), C.c_float(1.0),
                                   _p(ff) if ff is not None else None)
        return v

    def gelu(self, v):
        return np.array([self.r.ref_gelu(C.c_float(float(a))) for a in v], np.float32)

    # ---- main.c:1849-1854, build_ple 1747-1778 -----------------------------
    def embed(self, token):
        m = self.m
        x = np.empty(m.dim, np.float32)
        p, ty = m.t("token_embd.weight")
        self.r.ref_emb_lookup(_p(x), p, ty, token, m.dim)
        x = x * np.float32(np.sqrt(np.float32(m.dim), dtype=np.float32))
        rd = m.pd * m.L
        row = np.empty(rd, np.float32)
        p, ty = m.t("per_layer_token_embd.weight")
        self.r.ref_emb_lookup(_p(row), p, ty, token, rd)
        row = row * np.sqrt(np.float32(m.pd), dtype=np.float32)
        ctx, _ = self.mm(x, "per_layer_model_proj.weight", m.dim, rd)
        ctx = ctx * (np.float32(1.0) / np.sqrt(np.float32(m.dim), dtype=np.float32))
        pn = m.vec("per_layer_proj_norm.weight", m.pd)
        ctx = np.concatenate([self.rmsnorm(ctx[l * m.pd:(l + 1) * m.pd], pn) for l in range(m.L)])
        mix = np.float32(1.0) / np.sqrt(np.float32(2.0), dtype=np.float32)
        return x, (row + ctx) * mix

    # ---- one layer, main.c:1865-2011 ---------------------------------------
    def pre_attention(self, l, pos, x):
        """attn_norm, Q8_K, Q (+ q_norm, RoPE), K/V (+ norms, RoPE of K)"""
        m = self.m
        hd, swa = m.hd(l), m.swa(l)
        n_rot = m.rot_swa if swa else m.rot_full
        base = m.theta_swa if swa else m.theta
        ff = None if swa else m.vec("rope_freqs.weight", m.hd_full // 2)
        b = f"blk.{l}."
        xb2 = self.rmsnorm(x, m.vec(b + "attn_norm.weight", m.dim))
        q8 = self.quantize(xb2) if m.t(b + "attn_q.weight")[1] in (12, 13) else None
        q, _ = self.mm(xb2, b + "attn_q.weight", m.dim, m.nh * hd, q8)
        q = self.rope(self.head_norm(q, m.vec(b + "attn_q_norm.weight", hd), m.nh, hd), m.nh, hd, n_rot, pos, base, ff)
        if l >= 24:
            return q, None, None
        kq8 = q8 if m.t(b + "attn_k.weight")[1] in (12, 13) else None
        k, _ = self.mm(xb2, b + "attn_k.weight", m.dim, m.nkv * hd, kq8)
        vq8 = q8 if m.t(b + "attn_v.weight")[1] in (12, 13) else None
        v, _ = self.mm(xb2, b + "attn_v.weight", m.dim, m.nkv * hd, vq8)
        k = self.head_norm(k, m.vec(b + "attn_k_norm.weight", hd), m.nkv, hd)
        v = self.head_norm(v, None, m.nkv, hd)
        k = self.rope(k, m.nkv, hd, n_rot, pos, base, ff)
        return q, k, v

    def post_attention(self, l, x, q_out, ple):
        """O, post-attention norm + residual, FFN, PLE gate + projection,
        post_norm + residual, out_scale"""
        m = self.m
        hd, b = m.hd(l), f"blk.{l}."
        o, _ = self.mm(q_out, b + "attn_output.weight", m.nh * hd, m.dim)
        x = x + self.rmsnorm(o, m.vec(b + "post_attention_norm.weight", m.dim))
        xb2 = self.rmsnorm(x, m.vec(b + "ffn_norm.weight", m.dim))
        q8 = self.quantize(xb2) if m.t(b + "ffn_gate.weight")[1] in (12, 13) else None
        g, _ = self.mm(xb2, b + "ffn_gate.weight", m.dim, m.hidden, q8)
        u, _ = self.mm(xb2, b + "ffn_up.weight", m.dim, m.hidden, q8 if m.t(b + "ffn_up.weight")[1] in (12, 13) else None)
        hb = self.gelu(g) * u
        dn, _ = self.mm(hb, b + "ffn_down.weight", m.hidden, m.dim)
        x = x + self.rmsnorm(dn, m.vec(b + "post_ffw_norm.weight", m.dim))
        pg, _ = self.mm(x, b + "inp_gate.weight", m.dim, m.pd)
        pg = self.gelu(pg) * ple[l * m.pd:(l + 1) * m.pd]
        y, _ = self.mm(pg, b + "proj.weight", m.pd, m.dim)
        x = x + self.rmsnorm(y, m.vec(b + "post_norm.weight", m.dim))
        sc = m.vec(b + "layer_output_scale.weight", 1)
        return x * sc[0] if sc is not None else x

    # ---- main.c:2021-2028, logits_tied 1780-1796 ---------------------------
    def lm_head(self, x):
        m = self.m
        xn = self.rmsnorm(x, m.vec("output_norm.weight", m.dim))
        lg, _ = self.mm(xn, "token_embd.weight", m.dim, m.vocab)
        if m.softcap > 0:
            inv = np.float32(1.0) / m.softcap
            lg = np.array([np.float32(m.softcap) * np.float32(LIBM.tanhf(float(np.float32(v) * inv))) for v in lg],
                          np.float32)
        return lg


def attention_f64(q, kc, vc, t_start, pos, nh, nkv, hd, src_hd):
    """main.c:1909-1950 in float64: rows t_start..pos, row stride 1024, kv
    head h / (nh/nkv) at offset kvh * src_hd, attn_scale 1"""
    out = np.empty(nh * hd)
    for h in range(nh):
        kvh = h // (nh // nkv)
        K = kc[t_start:pos + 1, kvh * src_hd:kvh * src_hd + hd].astype(np.float64)
        V = vc[t_start:pos + 1, kvh * src_hd:kvh * src_hd + hd].astype(np.float64)
        s = K @ q[h * hd:(h + 1) * hd].astype(np.float64)
        p = np.exp(s - s.max())
        out[h * hd:(h + 1) * hd] = (p / p.sum()) @ V
    return out


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    s = synth.tiny_shape(rope_freqs=True)
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    synth.write_model_gguf(p, s, seed=4)
    return p


def test_model_open_matches_reference_loader(ref, orc, tmp_path):
    """or_model_open's configuration equals the reference's parse_gguf, for
    GGUFs aligned to 32 and 64 bytes; the data offset follows the alignment
    and the vocabulary is the token list's length."""
    s = synth.tiny_shape(rope_freqs=True, vocab=777)
    for align in (32, 64):
        p = str(tmp_path / f"a{align}.gguf")
        synth.write_model_gguf(p, s, seed=9, alignment=align)
        rm = RefModel(ref, p)
        om = OracleModel(orc, p, max_seq=0)
        try:
            assert rm.doff % align == 0
            assert (om.dim, om.hidden, om.n_layers, om.n_heads, om.n_kv, om.vocab, om.max_seq, om.ple_dim,
                    om.window) == (rm.dim, rm.hidden, rm.L, rm.nh, rm.nkv, rm.vocab, rm.max_seq, rm.pd, rm.window)
            assert rm.vocab == 777 and rm.max_seq == s.context
            assert [om.kv_source(l) for l in range(rm.L)] == [rm.src(l) for l in range(rm.L)]
        finally:
            om.close()
    # the same weights at either alignment give the same logits
    logits = []
    for align in (32, 64):
        om = OracleModel(orc, str(tmp_path / f"a{align}.gguf"), max_seq=16)
        try:
            om.forward(5, 0, 1)
            logits.append(om.logits())
        finally:
            om.close()
    assert _bits_equal(logits[0], logits[1])


def test_layers_composed_from_reference(ref, orc, tiny):
    """build_ple, every layer at two positions (inside and past the 8-slot
    window, so sliding layers start at t_start > 0) and the LM head: the
    oracle equals the composition of the reference's functions bit for bit,
    its attention equals the float64 block to 5e-5 of max |o| (fp32 scores of
    normed q, k with attn_scale 1 enter exp() with absolute errors of ~1e-5)."""
    rm = RefModel(ref, tiny)
    cp = Compose(ref, rm)
    om = OracleModel(orc, tiny, max_seq=32)
    try:
        toks = [7, 300, 12, 99, 5, 410, 33, 2, 250, 17, 64, 128, 3]
        worst_attn = 0.0
        for pos, tok in enumerate(toks):
            om.forward(tok, pos, 0)          # fills the oracle's KV cache for pos
            if pos not in (4, 12):
                continue
            # embedding and PLE
            om.embed(tok, pos)
            x0, ple = cp.embed(tok)
            assert _bits_equal(om.state("x", rm.dim), x0)
            assert _bits_equal(om.state("ple", rm.pd * rm.L), ple)
            rng = np.random.default_rng(pos)
            for l in range(rm.L):
                hd = rm.hd(l)
                x_in = rng.standard_normal(rm.dim).astype(np.float32)
                x_out = om.layer_inject(tok, pos, l, x_in)
                q, k, v = cp.pre_attention(l, pos, x_in)
                assert _bits_equal(om.state("q", rm.nh * hd), q), l
                src = rm.src(l)
                kc, vc = om.kv(src)
                if k is not None:
                    assert _bits_equal(om.state("k", rm.nkv * hd), k), l
                    assert _bits_equal(om.state("v", rm.nkv * hd), v), l
                    assert _bits_equal(kc[pos, :rm.nkv * hd], k) and _bits_equal(vc[pos, :rm.nkv * hd], v), l
                t_start = max(0, pos + 1 - rm.window) if rm.swa(l) else 0
                want = attention_f64(q, kc, vc, t_start, pos, rm.nh, rm.nkv, hd, rm.hd(src))
                q_out = om.state("q_out", rm.nh * hd)
                err = np.max(np.abs(q_out - want)) / np.max(np.abs(want))
                worst_attn = max(worst_attn, err)
                assert err < 5e-5, (l, err)
                assert _bits_equal(x_out, cp.post_attention(l, x_in, q_out, ple)), l
            om.forward(tok, pos, 0)          # restore the cache rows the injections rewrote
        print(f"attention vs float64: worst {worst_attn:.1e}")
        x = np.random.default_rng(1).standard_normal(rm.dim).astype(np.float32)
        assert _bits_equal(om.lm_head_inject(x), cp.lm_head(x))
    finally:
        om.close()


def test_zero_projections_leave_scaled_residual(orc, tmp_path):
    """With zero O, FFN down and PLE projection weights every residual branch
    adds rmsnorm(0) = 0, so each layer outputs out_scale * input exactly (the
    scale multiplies the whole residual stream, last)."""
    s = synth.tiny_shape(rope_freqs=True, zeros=("blk.*.attn_output.weight", "blk.*.ffn_down.weight",
                                                 "blk.*.proj.weight"))
    p = str(tmp_path / "zero.gguf")
    synth.write_model_gguf(p, s, seed=6)
    om = OracleModel(orc, p, max_seq=16)
    try:
        X = np.random.default_rng(2).standard_normal((s.n_layers + 1, s.dim)).astype(np.float32)
        out = om.forward_inject(11, 3, 0, X)
        buf = np.fromfile(p, np.uint8)
        for l in range(s.n_layers):
            sc = _tensor_f32(buf, f"blk.{l}.layer_output_scale.weight")[0]
            assert _bits_equal(out[l], X[l] * sc), l
    finally:
        om.close()


def _tensor_f32(buf, name):
    """an F32 tensor's values, located through the oracle-independent
    GGUF header walk of the reference loader (via RefModel is not needed
    here: the zero model test runs without the reference tree)"""
    import struct
    p = 4 + 4
    n_t, n_kv = struct.unpack_from("<QQ", buf, p)
    p += 16
    align = 32

    def rstr(p):
        n = struct.unpack_from("<Q", buf, p)[0]
        return bytes(buf[p + 8:p + 8 + n]).decode(), p + 8 + n

    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}

    def skip(p, t):
        if t == 8:
            return rstr(p)[1]
        if t == 9:
            et, n = struct.unpack_from("<IQ", buf, p)
            p += 12
            for _ in range(n):
                p = skip(p, et)
            return p
        return p + sizes[t]

    for _ in range(n_kv):
        k, p = rstr(p)
        t = struct.unpack_from("<I", buf, p)[0]
        p += 4
        if k == "general.alignment":
            align = struct.unpack_from("<I", buf, p)[0]
        p = skip(p, t)
    infos = {}
    for _ in range(n_t):
        nm, p = rstr(p)
        nd = struct.unpack_from("<I", buf, p)[0]
        ne = struct.unpack_from(f"<{nd}Q", buf, p + 4)
        p += 4 + 8 * nd
        ty, off = struct.unpack_from("<IQ", buf, p)
        p += 12
        infos[nm] = (ne, ty, off)
    doff = (p + align - 1) // align * align
    ne, ty, off = infos[name]
    assert ty == 0
    return np.frombuffer(buf, np.float32, int(np.prod(ne)), doff + off)


def test_shared_layers_read_their_donors(orc, tiny):
    """Layers 24.. read the KV of donor 22 (sliding) or 23 (full): changing
    one donor's cached rows changes exactly the layers that read it."""
    om = OracleModel(orc, tiny, max_seq=16)
    try:
        for pos, tok in enumerate([4, 8, 15, 16, 23]):
            om.forward(tok, pos, 0)
        pos, tok = 4, 23
        X = np.random.default_rng(3).standard_normal((om.n_layers, om.dim)).astype(np.float32)
        base = [om.layer_inject(tok, pos, l, X[l]) for l in range(om.n_layers)]
        for donor in (22, 23):
            kc, vc = om.kv(donor)
            saved = vc[:pos + 1].copy()
            # readers store nothing, so every row they read may change (not by a
            # pure scale: the norms after the attention would undo it)
            vc[:pos + 1] = np.random.default_rng(donor).standard_normal(saved.shape).astype(np.float32)
            changed = [l for l in range(24, om.n_layers)
                       if not _bits_equal(om.layer_inject(tok, pos, l, X[l]), base[l])]
            vc[:pos + 1] = saved
            assert changed == [l for l in range(24, om.n_layers) if om.kv_source(l) == donor], (donor, changed)
            assert all(om.kv_source(l) in (22, 23) for l in range(24, om.n_layers))
    finally:
        om.close()


def test_hidden_stats_is_the_reference(ref, orc):
    """or_hidden_stats (main.c:1811-1827): double sums, float max |x|, bit
    for bit with the reference's own function."""
    rng = np.random.default_rng(5)
    for n in (1, 7, 256, 2560, 10240):
        v = (rng.standard_normal(n) * 10 ** rng.uniform(-3, 3)).astype(np.float32)
        v[0] = -0.0
        a = [np.zeros(1, np.float32) for _ in range(3)]
        b = [np.zeros(1, np.float32) for _ in range(3)]
        orc.L.or_hidden_stats(_p(v), n, *[_p(x) for x in a])
        ref.L.ref_hidden_stats(_p(v), n, *[_p(x) for x in b])
        assert all(_bits_equal(x, y) for x, y in zip(a, b)), n
        # and the closed form, in float64
        assert abs(float(a[0][0]) - float(np.float32(v.astype(np.float64).sum()))) <= abs(np.spacing(a[0][0]))
        assert float(a[2][0]) == float(np.max(np.abs(v)))


def test_mm_f32_bruteforce(orc):
    """or_mm_f32 (the plain-loop sgemv standing for mm_f32's cblas_sgemv,
    main.c:1494-1517): float64 brute force to 1e-6 of sum |w x| per row."""
    rng = np.random.default_rng(8)
    for n, d in ((256, 40), (2560, 300), (8, 3)):
        W = rng.standard_normal((d, n)).astype(np.float32)
        x = rng.standard_normal(n).astype(np.float32)
        o = np.empty(d, np.float32)
        orc.L.or_mm_f32(_p(o), _p(x), _p(W), n, d)
        want = W.astype(np.float64) @ x.astype(np.float64)
        mag = np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64))
        assert np.max(np.abs(o - want) / mag) < 1e-6


def test_fingerprints_are_reference_stats(ref, orc, tiny):
    """The oracle's layer-0 dump_kv_fingerprint records (main.c:1829-1836,
    1880-1951) are the reference's hidden_stats and first four values of
    the vectors the composition gives at those statements."""
    rm = RefModel(ref, tiny)
    cp = Compose(ref, rm)
    om = OracleModel(orc, tiny, max_seq=16)
    try:
        toks = [7, 300, 12]
        for pos, tok in enumerate(toks):
            om.forward(tok, pos, 0)
        pos, tok = 2, toks[2]
        x = np.random.default_rng(11).standard_normal(rm.dim).astype(np.float32)
        om.layer_inject(tok, pos, 0, x)
        fp, have = om.kv_fingerprint()
        hd = rm.hd(0)
        m = rm
        b = "blk.0."
        xb2 = cp.rmsnorm(x, m.vec(b + "attn_norm.weight", m.dim))
        q8 = cp.quantize(xb2)
        k, _ = cp.mm(xb2, b + "attn_k.weight", m.dim, m.nkv * hd, q8)
        kn = cp.head_norm(k, m.vec(b + "attn_k_norm.weight", hd), m.nkv, hd)
        _, k_store, _ = cp.pre_attention(0, pos, x)
        kc, _ = om.kv(0)
        vecs = {0: xb2, 1: k, 2: kn, 3: k_store, 4: kc[0, :m.nkv * hd], 5: kc[pos, :m.nkv * hd],
                6: om.state("q_out", m.nh * hd)}
        assert have.all()
        for t, v in vecs.items():
            st = [np.zeros(1, np.float32) for _ in range(3)]
            v = np.ascontiguousarray(v, np.float32)
            ref.L.ref_hidden_stats(_p(v), v.size, *[_p(s) for s in st])
            assert _bits_equal(fp[t, :3], np.concatenate(st)), t
            assert _bits_equal(fp[t, 3:], v[:4]), t
        om.forward(toks[0], 0, 0)
        assert not om.kv_fingerprint()[1][5]       # K_readN is printed only at pos > 0
    finally:
        om.close()
