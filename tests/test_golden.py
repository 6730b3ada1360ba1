"""Pins the CPU oracle bit for bit against fixtures written by the
reference's own functions (tests/golden/make_golden.py runs
gemma4-4b/cpu-blas/main.c's hot-path functions, compiled unchanged into
oracle/_ref).  Runs anywhere: the fixtures are data, the reference tree is
not needed."""
import os

import numpy as np
import pytest

from oracle import Q8K_DTYPE

P = lambda a: a.ctypes.data  # noqa: E731
GOLD = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLD)   # plain arrays, no pickle


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_quantize_q8K(orc, g):
    x, offs = g["q8_x"], g["q8_offs"]
    ours = orc.quantize_q8K(x).view(np.uint8)
    assert ours.tobytes() == g["q8_avx"].tobytes()
    assert g["q8_avx"].tobytes() == g["q8_ref"].tobytes()    # the reference's two variants agree
    # per-input slices (quantize_row_q8_K is blockwise)
    for a, b in zip(offs[:-1], offs[1:]):
        part = orc.quantize_q8K(x[a:b]).view(np.uint8)
        assert part.tobytes() == g["q8_avx"][a // 256 * 292:b // 256 * 292].tobytes()


@pytest.mark.parametrize("name,qt", [("q4K", 12), ("q5K", 13)])
def test_kquant_dots(orc, g, name, qt):
    q8 = np.frombuffer(g["dot_q8"].tobytes(), Q8K_DTYPE)
    assert orc.quantize_q8K(np.zeros(0, np.float32)).size == 0
    w = np.ascontiguousarray(g[f"dot_{name}_w"])
    bs = 144 if qt == 12 else 176
    f_avx = orc.L.or_vec_dot_q4K_q8K if qt == 12 else orc.L.or_vec_dot_q5K_q8K
    f_gen = orc.L.or_vec_dot_q4K_q8K_generic if qt == 12 else orc.L.or_vec_dot_q5K_q8K_generic
    avx = np.array([f_avx(2560, P(w) + r * 10 * bs, P(q8)) for r in range(12)], np.float32)
    gen = np.array([f_gen(2560, P(w) + r * 10 * bs, P(q8)) for r in range(12)], np.float32)
    assert np.array_equal(bits(avx), bits(g[f"dot_{name}_avx"]))
    assert np.array_equal(bits(gen), bits(g[f"dot_{name}_generic"]))
    assert np.array_equal(bits(orc.mm_quant_dot_rows(w, 2560, 12, qt, q8)), bits(g[f"mmdot_{name}"]))


def test_mm_quant_rows_q6K(orc, g):
    o = orc.mm_quant_rows(g["mmq6_x"], g["mmq6_w"], 2560, 8, 14)
    assert np.array_equal(bits(o), bits(g["mmq6_o"]))


def test_mm_bf16(orc, g):
    o = orc.mm_bf16(g["bf16_x"], g["bf16_w"], 512, 8)
    assert np.array_equal(bits(o), bits(g["bf16_o"]))


@pytest.mark.parametrize("name,qt", [("q4K", 12), ("q5K", 13), ("q6K", 14)])
def test_dequant(orc, g, name, qt):
    o = orc.dequant(g[f"deq_{name}_w"], qt, 1024)
    assert np.array_equal(bits(o), bits(g[f"deq_{name}_o"]))


def test_norms_softmax_gelu(orc, g):
    assert np.array_equal(bits(orc.rmsnorm(g["norm_x"], g["norm_w"])), bits(g["norm_o"]))
    v = g["head_v"].copy()
    hw = np.ascontiguousarray(g["head_w"])      # keep the array alive across the call
    orc.L.or_rmsnorm_head_inplace(P(v), P(hw), 8, 256, 1e-6)
    assert np.array_equal(bits(v), bits(g["head_o"]))
    v = g["head_v"].copy()
    orc.L.or_rmsnorm_head_noweight_inplace(P(v), 8, 256, 1e-6)
    assert np.array_equal(bits(v), bits(g["headnw_o"]))
    s = g["softmax_x"].copy()
    orc.L.or_softmax(P(s), s.size)
    assert np.array_equal(bits(s), bits(g["softmax_o"]))
    ge = np.array([orc.L.or_gelu(float(v)) for v in g["gelu_x"]], np.float32)
    assert np.array_equal(bits(ge), bits(g["gelu_o"]))


@pytest.mark.parametrize("tag,hd,base", [("swa", 256, 1e4), ("full", 512, 1e6)])
def test_rope(orc, g, tag, hd, base):
    ff = g[f"rope_{tag}_ff"]
    for pos in (0, 1, 511, 4095, 32767):
        o = orc.rope(g[f"rope_{tag}_{pos}_x"], 8, hd, hd, pos, base, ff if ff.size else None)
        assert np.array_equal(bits(o), bits(g[f"rope_{tag}_{pos}_o"])), pos


def test_emb_lookup(orc, g):
    w = np.ascontiguousarray(g["emb_w"])
    for t in range(4):
        o = np.empty(2560, np.float32)
        assert orc.L.or_emb_lookup(P(o), P(w), 14, t, 2560) == 0
        assert np.array_equal(bits(o), bits(g["emb_o"][t]))


def test_sampler(orc, g):
    lg = g["sample_logits"]
    for row in g["sample_draws"]:
        temp, topp, topk, seed = float(row[0]), float(row[1]), int(row[2]), int(row[3])
        st = np.array([seed], np.uint64)
        toks = []
        for _ in range(8):
            work = lg.copy()
            toks.append(orc.L.or_sample_token(P(work), 512, temp, topp, topk, P(st)))
        assert toks == [int(v) for v in row[4:]], (temp, topp, topk, seed)
    assert int(g["sample_draws"][0][4]) == 7          # greedy: first index of the tied maximum


def test_repetition_penalty(orc, g):
    """apply_repetition_penalty (main.c:2114-2126): windows of 64, all, longer
    than the history and 5 tokens; a token repeated four times is penalised
    four times in turn; penalty 1.0 changes nothing."""
    hist = np.ascontiguousarray(g["penalty_hist"], np.int32)
    for (penalty, last_n), want in zip(g["penalty_cases"], g["penalty_out"]):
        work = g["sample_logits"].copy()
        orc.L.or_apply_repetition_penalty(P(work), P(hist), hist.size, float(penalty), int(last_n))
        assert np.array_equal(bits(work), bits(want)), (penalty, last_n)
