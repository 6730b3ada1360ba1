"""The measurement probes behind the floors workload (csrc/probe.hip): they
compute nothing of the model, but their results must be right for their
timings to mean anything -- the last-workgroup hand-off sees every value in
both of its forms, over repeated launches, and the counter is reset."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from g4 import Lib
    L = Lib.get()
    L.init(0)
    L.L.g4_set_stream(None)
    return L


@pytest.mark.parametrize("wg", [1, 13, 160, 640])
@pytest.mark.parametrize("mode", [1, 2])
def test_probe_handoff_sums_every_value(lib, wg, mode):
    from g4 import DBuf
    vals, cnt, out = DBuf(lib, 4 * 16 * 640), DBuf(lib, 256), DBuf(lib, 256)
    lib.check(lib.L.g4_memset(cnt.ptr, 0, 256))
    want = float(np.sum(np.arange(16 * wg, dtype=np.float64)))
    for _ in range(3):
        lib.check(lib.L.g4_memset(out.ptr, 0, 256))
        lib.g4_probe_handoff(vals.ptr, cnt.ptr, out.ptr, wg, mode)
        got = out.to_array(np.float32)[0]
        assert abs(float(got) - want) <= 1e-6 * want
    assert cnt.to_array(np.uint32)[0] == 0


def test_probe_handoff_rejects(lib):
    from g4 import DBuf, G4Error
    b = DBuf(lib, 4 * 16 * 640)
    for wg, mode in [(641, 1), (0, 1), (13, 3)]:
        with pytest.raises(G4Error):
            lib.g4_probe_handoff(b.ptr, b.ptr, b.ptr, wg, mode)


def test_probe_read_sums(lib):
    from g4 import DBuf
    n = 1 << 20
    x = np.arange(n, dtype=np.float32) % 7
    xd = DBuf.from_array(lib, x)
    sink = DBuf(lib, 4 * 64)
    lib.g4_probe_read(xd.ptr, 4 * n, sink.ptr, 64)
    assert float(np.sum(sink.to_array(np.float32)[:64], dtype=np.float64)) == float(np.sum(x, dtype=np.float64))
