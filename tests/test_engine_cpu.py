"""CPU-side checks of the C engine's GGUF path (no GPU): parse_gguf's metadata
defaults and the tensor checks of load_weights turn every malformed input the
reference would exit(1) on (main.c:843, 1396-1399, 1690-1692) into a status
code, before any device work."""
import dataclasses

import numpy as np
import pytest

import synth


@pytest.fixture(scope="module")
def eng():
    import g4
    return g4.EngineLib.get()


def _image(tmp_path, shape, tensors=None, kvs=None, name="m.gguf"):
    p = str(tmp_path / name)
    synth.write_gguf(p, kvs if kvs is not None else synth.model_kvs(shape),
                     tensors if tensors is not None else synth.model_tensors(shape), seed=3)
    return np.fromfile(p, np.uint8)


def test_check_image_ok(tmp_path, eng):
    s = synth.tiny_shape()
    img = _image(tmp_path, s)
    cfg = eng.check_image(img)
    assert cfg == [s.dim, s.hidden, s.n_layers, s.n_heads, s.n_kv, s.vocab, s.context, s.ple_dim, s.window]
    assert eng.check_image(img, max_seq=32)[6] == 32


def _expect(eng, img, code, text):
    import g4
    with pytest.raises(g4.G4Error) as e:
        eng.check_image(img)
    assert e.value.code == code
    assert text in str(e.value)


def test_bad_magic_and_truncation(tmp_path, eng):
    import g4
    img = _image(tmp_path, synth.tiny_shape())
    bad = img.copy()
    bad[0] ^= 0xFF
    _expect(eng, bad, g4.G4_ERR_FORMAT, "invalid GGUF magic")
    _expect(eng, img[:100].copy(), g4.G4_ERR_FORMAT, "truncated")
    _expect(eng, img[: img.size // 2].copy(), g4.G4_ERR_FORMAT, "past the end")
    _expect(eng, img[:10].copy(), g4.G4_ERR_FORMAT, "invalid GGUF magic")


def _tensors_with(shape, name, **change):
    ts = synth.model_tensors(shape)
    out = []
    for t in ts:
        if t.name == name:
            if change.get("drop"):
                continue
            t = dataclasses.replace(t, **{k: v for k, v in change.items() if k != "drop"})
        out.append(t)
    return out


def test_unsupported_type(tmp_path, eng):
    import g4
    s = synth.tiny_shape()
    ts = _tensors_with(s, "blk.3.attn_norm.weight", qtype=synth.F16,
                       make=lambda r: np.ones(s.dim, np.float16))
    _expect(eng, _image(tmp_path, s, ts), g4.G4_ERR_TYPE, "Unsupported tensor type 1 for blk.3.attn_norm.weight")


def test_wrong_shape_and_missing(tmp_path, eng):
    import g4
    s = synth.tiny_shape()
    ts = _tensors_with(s, "blk.2.attn_q.weight", ne=(s.dim, s.n_heads * s.hd_swa + 256),
                       make=lambda r: synth.rand_q4K(r, s.n_heads * s.hd_swa + 256, s.dim))
    _expect(eng, _image(tmp_path, s, ts), g4.G4_ERR_FORMAT, "blk.2.attn_q.weight: shape")
    ts = _tensors_with(s, "blk.7.ffn_down.weight", drop=True)
    _expect(eng, _image(tmp_path, s, ts, name="m2.gguf"), g4.G4_ERR_FORMAT, "missing tensor blk.7.ffn_down.weight")
    ts = _tensors_with(s, "output_norm.weight", drop=True)
    _expect(eng, _image(tmp_path, s, ts, name="m3.gguf"), g4.G4_ERR_FORMAT, "missing tensor output_norm.weight")


def test_token_embd_types(tmp_path, eng):
    """The token table goes through emb_lookup (main.c:1696-1723: F32, F16,
    Q4_K, Q5_K, Q6_K) and mm() for the tied LM head: F32 is accepted, BF16
    (no emb_lookup case: "Unsupported emb type") is not."""
    import g4
    s = synth.tiny_shape()
    ts = _tensors_with(s, "token_embd.weight", qtype=synth.F32, ne=(s.dim, s.vocab),
                       make=lambda r: np.zeros((s.vocab, s.dim), np.float32))
    assert eng.check_image(_image(tmp_path, s, ts, name="f32.gguf"))[5] == s.vocab
    ts = _tensors_with(s, "token_embd.weight", qtype=synth.BF16, ne=(s.dim, s.vocab),
                       make=lambda r: np.zeros((s.vocab, s.dim), np.uint16))
    _expect(eng, _image(tmp_path, s, ts, name="bf16.gguf"), g4.G4_ERR_TYPE, "token_embd.weight")


def test_matrix_types_as_found(tmp_path, eng):
    """Every matrix goes through mm() (main.c:1669-1694), so each may be F32,
    F16, BF16, Q4_K, Q5_K or Q6_K, gate and up of different types; a dense
    row length the GEMV cannot stream is a format error."""
    import g4
    s = dataclasses.replace(synth.tiny_shape(), types=(
        ("blk.2.attn_output.weight", synth.F16), ("blk.4.ffn_gate.weight", synth.Q6_K),
        ("blk.4.ffn_up.weight", synth.F32), ("per_layer_model_proj.weight", synth.F16),
        ("token_embd.weight", synth.Q4_K), ("blk.*.proj.weight", synth.Q5_K)))
    assert eng.check_image(_image(tmp_path, s, name="mixed.gguf"))[0] == s.dim
    bad = _tensors_with(s, "blk.2.attn_output.weight", ne=(s.n_heads * s.hd_swa - 4, s.dim),
                        make=lambda r: np.zeros((s.dim, s.n_heads * s.hd_swa - 4), np.float16))
    _expect(eng, _image(tmp_path, s, bad, name="bad.gguf"), g4.G4_ERR_FORMAT, "blk.2.attn_output.weight")


def test_open_without_gpu_fails_cleanly(tmp_path, eng):
    """No HIP device here: opening reports G4_ERR_NODEV instead of crashing."""
    import g4
    if g4.Lib.get().L.g4_init(0) == g4.G4_OK:
        pytest.skip("a GPU is present")
    img = _image(tmp_path, synth.tiny_shape())
    with pytest.raises(g4.G4Error) as e:
        g4.Engine(img)
    assert e.value.code == g4.G4_ERR_NODEV


@pytest.mark.parametrize("size", [0, 1, 55, 56, 63, 64, 119, 120, 1000, (1 << 20) + 77, 3 << 20])
def test_sha256_file(tmp_path, eng, size):
    """SHA-256 of the model file (the download check of gemma4-4b/Makefile,
    design.md:107-117) against Python's hashlib, across the padding edges
    (55/56, 119/120 bytes) and the 1 MiB read chunks."""
    import hashlib
    data = np.random.default_rng(size).integers(0, 256, size, dtype=np.uint8).tobytes()
    p = tmp_path / f"f{size}.bin"
    p.write_bytes(data)
    assert eng.sha256_file(str(p)) == hashlib.sha256(data).hexdigest()


def test_check_sha256sum(tmp_path, eng):
    """sha256sum --check semantics for one named file: text and binary marks,
    upper-case digests; a mismatch or a missing line is an error."""
    import hashlib
    import g4
    data = b"gguf model bytes" * 1000
    p = tmp_path / "model.gguf"
    p.write_bytes(data)
    h = hashlib.sha256(data).hexdigest()
    ok = tmp_path / "ok.sha256sum"
    ok.write_text(f"{'0' * 64}  other.gguf\n{h.upper()} *model.gguf\n")
    eng.check_sha256sum(str(p), str(ok))
    bad = tmp_path / "bad.sha256sum"
    bad.write_text(f"{'1' * 64}  model.gguf\n")
    with pytest.raises(g4.G4Error) as e:
        eng.check_sha256sum(str(p), str(bad))
    assert "FAILED" in str(e.value)
    none = tmp_path / "none.sha256sum"
    none.write_text(f"{h}  another.gguf\n")
    with pytest.raises(g4.G4Error) as e:
        eng.check_sha256sum(str(p), str(none))
    assert "no checksum line" in str(e.value)
