"""g4_attn_decode_noalloc: the attention block of main.c:1909-1950 with its
chunk partials in the per-GPU scratch array instead of an allocation.  It
runs the kernels of g4_attn_decode with the same chunk count, so its output
must equal g4_attn_decode's bit for bit, on consecutive calls whose second
one is smaller (the array keeps the first call's partials), and sizes past
the array are refused before anything is launched."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    import g4
    L = g4.Lib.get()
    L.init(0)
    L.L.g4_set_stream(None)
    return L


def _case(lib, orc, hd, n_heads, n_kv, T, t_start, seed):
    from g4 import DBuf
    rng = np.random.default_rng(seed)
    kv_dim = n_kv * hd
    kc = rng.standard_normal((T, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((T, kv_dim)).astype(np.float32)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    qd, kd, vd = (DBuf.from_array(lib, a) for a in (q, kc, vc))
    outs = []
    for fn in (lib.g4_attn_decode, lib.g4_attn_decode_noalloc):
        od = DBuf(lib, 4 * n_heads * hd)
        fn(qd.ptr, kd.ptr, vd.ptr, kv_dim, t_start, T - t_start, n_heads, n_kv, hd, C.c_float(1.0 / 16), od.ptr)
        outs.append(od.to_array(np.float32))
    want = orc.attn(q, kc, vc, kv_dim, t_start, T - t_start, n_heads, n_kv, hd, 1.0 / 16)
    return outs[0], outs[1], want


def test_noalloc_equals_workspace_entry(lib, orc):
    # a 4096-position global layer at head_dim 512, then a smaller call
    # (window 100 at head_dim 256): 128 then 4 chunks of partials
    for hd, n_heads, n_kv, T, t_start in ((512, 8, 2, 4096, 0), (256, 8, 2, 300, 200)):
        a, b, want = _case(lib, orc, hd, n_heads, n_kv, T, t_start, seed=T + hd)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (hd, T)
        assert np.max(np.abs(b - want)) / np.max(np.abs(want)) < 1e-4


def test_noalloc_refuses_past_scratch(lib):
    import g4
    from g4 import DBuf
    # 32 q heads x 293 chunks (300000 positions) x (256 + 2) floats = 9.7 MB >
    # the 8 MiB array: refused by the host check before any launch
    assert lib.L.g4_attn_part_bytes(32, 256, 293) > 8 << 20
    d = DBuf(lib, 256)
    with pytest.raises(g4.G4Error, match="scratch"):
        lib.g4_attn_decode_noalloc(d.ptr, d.ptr, d.ptr, 8 * 256, 0, 300000, 32, 8, 256, C.c_float(1.0), d.ptr)
