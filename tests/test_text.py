"""The engine's host text path (gemma4.c_amd/host/text.c) against the
reference's own tokenizer, chat template, detokenizer and response parser,
compiled from gemma4-4b/cpu-blas/main.c (968-1312, 2127-2226) into
oracle/_ref: token ids, scores, special ids and texts must be identical.

Vocabularies are synthetic GGUFs (the real model file is not available):
pieces for every character of a test corpus, merges learned from it, the
Gemma 4 special tokens, and variants for each branch of the template
(combined turn tokens, a separate turn opener, no turn tokens at all), a
score array instead of merges, duplicate pieces.  One vocabulary places the
pieces at the ids of the reference's published --think prompt for
"あなたは何者?" (doc/design.md:1266), which must come out as that id list.
"""
import ctypes as C

import numpy as np
import pytest

import synth

CORPUS = [
    "the quick brown fox jumps over the lazy dog",
    "Hello, how are you? I am fine, thank you.",
    "naïve café über straße",
    "日本語のテキスト、あなたは何者?",
    "emoji 😀 and symbols <|>",
    "  leading spaces and trailing  ",
    "tabs\tand\tmore",
]
TEXTS = [
    "the quick brown fox", "Hello, how are you?", "", "\n", "\n\n", "a\nb", "line one\n\nline three\n",
    "  two leading", "trailing  ", "naïve café", "日本語", "😀😀 x", "unknown ⊕ char", "tabs\tand\tmore",
    "the lazy dog jumps over the quick brown fox the end",
]
RAW = [b"the quick", b"\xe2\x96\x81the\xe2\x96\x81dog", b"\xff\xfe broken", b"caf\xc3", b"\xf0\x9f\x98", b""]

SPECIALS = ["<pad>", "<eos>", "<bos>", "<unk>", "<|turn>", "<turn|>", "<|think|>", "<|channel>", "<channel|>",
            "<|channel>thought\n", "<|turn>user\n", "<|turn>model\n", "<|turn>system\n"]


def _vocab(kind: str):
    """(pieces, merges or None, scores or None, add_space_prefix)"""
    prefix = kind != "scores"
    chars = sorted({c for line in CORPUS for c in synth.escape_line(line, prefix)} |
                   set("usermodelsystemthought<|>\n\t") | {synth.SP})
    merges = synth.bpe_train(CORPUS + ["user", "model", "system"], 300, prefix)
    specials = list(SPECIALS)
    if kind == "no_combined":
        specials = [s for s in specials if not s.endswith("\n") or s == "<|channel>thought\n"]
    if kind == "no_turn":
        specials = [s for s in specials if "turn" not in s]
    pieces = specials + chars + ["\n\n"] + [a + b for a, b in merges]
    if kind == "dups":
        pieces += ["th", "<|turn>", "the"]          # repeated pieces: lookups take the lowest id, specials the highest
    seen, uniq = set(), []
    for p in pieces:                               # merged pieces may repeat a character or an earlier merge
        if kind != "dups" and p in seen:
            continue
        seen.add(p)
        uniq.append(p)
    if kind == "scores":
        # a score array (as SentencePiece models carry) instead of merges:
        # later merges score lower, characters lowest
        rank = {a + b: -float(i) for i, (a, b) in enumerate(merges)}
        return uniq, None, [rank.get(p, -1e4) for p in uniq], False
    return uniq, [f"{a} {b}" for a, b in merges], None, True


@pytest.fixture(scope="module", params=["full", "no_combined", "no_turn", "scores", "dups"])
def pair(request, ref, tmp_path_factory):
    import g4
    pieces, merges, scores, prefix = _vocab(request.param)
    p = str(tmp_path_factory.mktemp("vocab") / f"{request.param}.gguf")
    synth.write_vocab_gguf(p, pieces, merges, scores, bos=2, eos=1, add_space_prefix=prefix)
    buf = np.fromfile(p, np.uint8)
    h = ref.L.ref_tok_open(buf.ctypes.data, buf.size)
    v = g4.Vocab(p)
    yield request.param, v, ref, h, buf, pieces
    v.close()


def _ids(a, n):
    return [int(x) for x in a[:n]]


def test_specials_scores_lookup(pair):
    kind, v, ref, h, _, pieces = pair
    want = np.zeros(13, np.int32)
    ref.L.ref_tok_specials(h, want.ctypes.data)
    assert v.specials() == [int(x) for x in want]
    assert v.size == len(pieces)
    for i, p in enumerate(pieces):
        b = p.encode()
        assert v.score(i) == ref.L.ref_tok_score(h, i), (kind, i, p)
        assert v.lookup(b) == ref.L.ref_tok_lookup(h, b, len(b)), (kind, p)
        assert v.is_special(i) == bool(ref.L.ref_is_special(h, i))
    assert v.lookup(b"\x00 not a piece") == -1


def test_encode_raw_and_text(pair):
    kind, v, ref, h, _, _ = pair
    out = np.zeros(1 << 16, np.int32)
    for raw in RAW + [t.encode() for t in TEXTS]:
        n = ref.L.ref_bpe_encode(h, raw, len(raw), out.ctypes.data)
        assert v.encode_raw(raw) == _ids(out, n), (kind, raw)
    for t in TEXTS:
        b = t.encode()
        n = ref.L.ref_gemma_text(h, b, out.ctypes.data)
        assert v.encode_text(b) == _ids(out, n), (kind, t)


def test_chat_template(pair):
    kind, v, ref, h, _, _ = pair
    out = np.zeros(8192, np.int32)
    histories = [
        [(0, "Hello, how are you?")],
        [(0, "the quick brown fox"), (1, "jumps over\nthe lazy dog"), (0, "日本語?")],
        [(0, "")],
        [],
    ]
    for hist in histories:
        for thinking in (0, 1):
            texts = (C.c_char_p * max(len(hist), 1))(*[t.encode() for _, t in hist])
            roles = np.array([r for r, _ in hist] or [0], np.int32)
            n = ref.L.ref_chat_encode_history(h, texts, roles.ctypes.data, len(hist), thinking, out.ctypes.data, 8192)
            got = v.chat_encode([(r, t.encode()) for r, t in hist], bool(thinking))
            assert got == _ids(out, n), (kind, hist, thinking)
            if hist:
                n1 = ref.L.ref_chat_encode(h, hist[0][1].encode(), thinking, out.ctypes.data) if len(hist) == 1 else n
                if len(hist) == 1:
                    assert got == _ids(out, n1)


def test_chat_template_cap(pair):
    """A conversation that reaches the cap is refused, as chat_encode_history
    returns -1 when the count reaches max_toks."""
    import g4
    kind, v, ref, h, _, _ = pair
    out = np.zeros(64, np.int32)
    msg = ("the quick brown fox " * 6).encode()
    texts = (C.c_char_p * 1)(msg)
    roles = np.zeros(1, np.int32)
    for cap in (8, 20, 40, 64):
        n = ref.L.ref_chat_encode_history(h, texts, roles.ctypes.data, 1, 0, out.ctypes.data, cap)
        if n < 0:
            with pytest.raises(g4.G4Error):
                v.chat_encode([(0, msg)], False, cap=cap)
        else:
            assert v.chat_encode([(0, msg)], False, cap=cap) == _ids(out, n)


def test_decode_and_split(pair):
    kind, v, ref, h, _, pieces = pair
    sp = v.specials()
    buf = C.create_string_buffer(1 << 16)
    rng = np.random.default_rng(3)
    chan, thought, cend = sp[10], sp[11], sp[12]
    nl = v.lookup(b"\n")
    for trial in range(40):
        toks = list(rng.integers(0, len(pieces), 30))
        if trial % 4 == 1 and chan >= 0 and cend >= 0:
            toks[3:3] = [chan] + toks[:2] + [nl]
            toks[15:15] = [cend]
        if trial % 4 == 2 and thought >= 0 and cend >= 0:
            toks[0:0] = [thought]
            toks[20:20] = [cend]
        toks = np.array(toks + [-5, len(pieces) + 3], np.int32)      # ids out of range are dropped too
        n = ref.L.ref_tokens_to_text(h, toks.ctypes.data, 0, toks.size, buf, 1 << 16)
        assert v.decode(toks) == buf.raw[:n], (kind, trial)
        t, a = C.create_string_buffer(1 << 16), C.create_string_buffer(1 << 16)
        tl, al = C.c_int(), C.c_int()
        ref.L.ref_parse_response(h, toks.ctypes.data, toks.size, t, C.byref(tl), a, C.byref(al), 1 << 16)
        ts, te, as_ = v.split_response(toks)
        if tl.value < 0:
            assert (ts, te) == (-1, -1) and v.decode(toks, as_) == a.raw[:al.value]
        else:
            assert v.decode(toks, ts, te) == t.raw[:tl.value] and v.decode(toks, as_) == a.raw[:al.value]


def test_think_prompt_golden(ref, tmp_path):
    """doc/design.md:1266: with --think, "あなたは何者?" is the 20 tokens
    2 105 9731 107 98 107 106 107 105 2364 107 51953 169845 237457 236881 106
    107 105 4368 107.  The vocabulary places each piece at the id the real
    model gives it (no combined turn tokens, no space prefix, merges that
    segment the text the same way); the rest of the 262144 ids are filler."""
    import g4
    golden = [2, 105, 9731, 107, 98, 107, 106, 107, 105, 2364, 107, 51953, 169845, 237457, 236881, 106, 107, 105,
              4368, 107]
    at = {2: "<bos>", 98: "<|think|>", 100: "<|channel>", 101: "<channel|>", 105: "<|turn>", 106: "<turn|>",
          107: "\n", 2364: "user", 4368: "model", 9731: "system", 51953: "あなた", 169845: "は", 237457: "何者",
          236881: "?", 3000: "あ", 3001: "な", 3002: "た", 3003: "何", 3004: "者", 3005: "あな"}
    pieces = [at.get(i, f"<unused{i}>") for i in range(262144)]
    merges = ["あ な", "あな た", "何 者"]
    p = str(tmp_path / "golden.gguf")
    synth.write_vocab_gguf(p, pieces, merges, None, bos=2, eos=106, add_space_prefix=False)
    v = g4.Vocab(p)
    assert v.chat_encode([(0, "あなたは何者?".encode())], True) == golden
    buf = np.fromfile(p, np.uint8)
    h = ref.L.ref_tok_open(buf.ctypes.data, buf.size)
    out = np.zeros(64, np.int32)
    n = ref.L.ref_chat_encode(h, "あなたは何者?".encode(), 1, out.ctypes.data)
    assert _ids(out, n) == golden
    sp = v.specials()
    assert (sp[10], sp[12]) == (100, 101)          # <|channel> and <channel|> as the design notes give them
    v.close()


def test_thinking_stream(pair):
    """The state machine of generate() (main.c:2406-2470) on generated
    token sequences: the printed answer equals parse_response's answer, the
    thinking trace is printed only with show_thinking after a channel label
    line, and the budget forces <channel|>."""
    import g4
    kind, v, ref, h, _, pieces = pair
    sp = v.specials()
    chan, thought, cend = sp[10], sp[11], sp[12]
    if chan < 0 or cend < 0:
        pytest.skip("vocabulary without channel tokens")
    nl = v.lookup(b"\n")
    words = [v.lookup(w.encode()) for w in ("th", "e", "fox", "dog", "a", "b") if v.lookup(w.encode()) >= 0]
    label = v.lookup("thought".encode())
    seq = [chan] + ([label] if label >= 0 else []) + [nl] + words[:3] + [cend] + words[1:]
    # thinking off: everything is answer text
    s = g4.TextStream(v, False, False, -1)
    assert b"".join(s.push(t) for t in seq) == v.decode(seq)
    # thinking on, trace hidden: only the answer after <channel|> prints
    s = g4.TextStream(v, True, False, -1)
    printed = b"".join(s.push(t) for t in seq)
    ts, te, as_ = v.split_response(seq)
    assert printed == v.decode(seq, as_)
    # shown: the label line's newline (the mode switches on that token, which
    # then prints), the trace, then the answer
    s = g4.TextStream(v, True, True, -1)
    printed = b"".join(s.push(t) for t in seq)
    assert printed == v.decode([nl]) + v.decode(seq, ts, te) + v.decode(seq, as_)
    # budget 2: after two thinking tokens <channel|> is forced
    s = g4.TextStream(v, True, False, 2)
    forced = None
    for t in seq:
        if s.force() >= 0:
            forced = s.force()
            break
        s.push(t)
    assert forced == cend


@pytest.mark.parametrize("count", [(1 << 62) + 3, (1 << 64) - 1, 1 << 40])
def test_scores_count_bounded(tmp_path, count):
    """A tokenizer.ggml.scores array whose 64-bit element count overruns the
    file (including counts where count * 4 wraps around 2^64 to a small
    number) is rejected as malformed, never read past the mapping."""
    import struct

    import g4
    pieces = ["a", "b", "ab", "<eos>"]
    p = str(tmp_path / "v.gguf")
    synth.write_vocab_gguf(p, pieces, None, [0.0, -1.0, -2.0, -3.0], bos=0, eos=3)
    g4.Vocab(p).close()                                 # the well-formed file opens
    buf = bytearray(open(p, "rb").read())
    key = b"tokenizer.ggml.scores"
    at = buf.index(key) + len(key)
    assert struct.unpack_from("<II", buf, at) == (9, 6)   # array of f32
    assert struct.unpack_from("<Q", buf, at + 8)[0] == 4
    struct.pack_into("<Q", buf, at + 8, count)
    open(p, "wb").write(bytes(buf))
    with pytest.raises(g4.G4Error):
        g4.Vocab(p)
