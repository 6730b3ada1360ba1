"""g4run end to end on the GPU (host/cli.c over the engine and the text
path), on the small synthetic model with a tokenizer vocabulary
(cli_vocab.py): the prompt token ids are the chat template's, the greedy
generation equals the engine's generate(), --force-gen and the thinking
budget replace tokens as generate() of gemma4-4b/cpu-blas/main.c does
(2406-2470), only the answer is printed in thinking mode, and interactive
mode runs turns until /quit."""
import os
import re
import subprocess

import numpy as np
import pytest

import synth
from cli_vocab import pieces_and_merges

pytestmark = pytest.mark.gpu

G4RUN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gemma4.c_amd", "g4run")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    pieces, merges = pieces_and_merges(512)
    s = synth.tiny_shape(rope_freqs=True, pieces=pieces, merges=merges)
    p = str(tmp_path_factory.mktemp("gguf") / "tiny_vocab.gguf")
    synth.write_model_gguf(p, s, seed=4)
    return p


def _run(model, *args, stdin=None):
    print("g4run", *args, flush=True)
    r = subprocess.run([G4RUN, model, "-l", "64", *args], capture_output=True, text=True, timeout=120, input=stdin)
    assert r.returncode == 0, r.stderr[-2000:]
    return r


def _ids(stderr, label):
    m = re.search(label + r":((?: -?\d+)*)", stderr)
    return [int(x) for x in m.group(1).split()] if m else []


def test_single_shot_greedy(model):
    import g4
    r = _run(model, "-p", "the quick brown fox", "-n", "12", "-t", "0", "--dump-prompt", "--dump-gen")
    prompt = _ids(r.stderr, "Prompt token IDs")
    gen = _ids(r.stderr, "Generated token IDs")
    v = g4.Vocab(model)
    assert prompt == v.chat_encode([(0, b"the quick brown fox")], False)
    em = g4.Engine(model, max_seq=64)
    try:
        want, _, _ = em.generate_greedy(prompt, 12)
    finally:
        em.close()
    assert gen == [int(t) for t in want]
    assert v.decode(gen).decode(errors="replace") in r.stdout
    assert "--- throughput ---" in r.stderr


def test_force_gen_and_thinking_budget(model):
    """--think with a 2-token budget: the forced opener <|channel>thought\\n
    (no label line), two thinking tokens, then <channel|> is forced in place
    of the next forced id; the remaining ids follow; stdout shows only the
    answer."""
    import g4
    v = g4.Vocab(model)
    sp = v.specials()
    thought, cend = sp[11], sp[12]
    a, b, c, d = (v.lookup(x.encode()) for x in ("t", "h", "e", "q"))
    forced = [thought, a, b, c, d]
    r = _run(model, "-p", "hello", "-n", "6", "-t", "0.8", "-s", "7", "--think", "--thinking-budget", "2",
             "--force-gen", ",".join(map(str, forced)), "--dump-gen", "--dump-prompt")
    gen = _ids(r.stderr, "Generated token IDs")
    assert gen[:5] == [thought, a, b, cend, d], gen
    assert "[thinking budget 2 tokens reached; forcing <channel|>]" in r.stderr
    prompt = _ids(r.stderr, "Prompt token IDs")
    assert prompt == v.chat_encode([(0, b"hello")], True)
    ts, te, as_ = v.split_response(np.array(gen, np.int32))
    answer = v.decode(np.array(gen, np.int32), as_).decode(errors="replace")
    body = r.stdout.split("[thinking]\n\n", 1)[1]
    assert body.startswith(answer), (body[:200], answer)


def test_sampled_matches_engine(model):
    """Sampling settings go to the device sampler unchanged: the same seed
    gives generate()'s tokens."""
    import g4
    r = _run(model, "-p", "how are you?", "-n", "10", "-t", "0.7", "-k", "0.9", "-s", "42", "-r", "1.2", "-N", "8",
             "--dump-prompt", "--dump-gen")
    prompt, gen = _ids(r.stderr, "Prompt token IDs"), _ids(r.stderr, "Generated token IDs")
    em = g4.Engine(model, max_seq=64)
    try:
        want, _, _ = em.generate(prompt, 10, 0.7, 0.9, 40, 1.2, 8, 42)
    finally:
        em.close()
    assert gen == [int(t) for t in want]


def test_interactive(model):
    r = _run(model, "-i", "-p", "", "-n", "4", "-t", "0", stdin="hello\nthe lazy dog\n/quit\n")
    turns = [ln for ln in r.stdout.splitlines() if ln.startswith("Model: ") and not ln.startswith("Model: dim=")]
    assert len(turns) == 2 and r.stderr.count("You: ") == 3 and "Bye." in r.stderr


def test_dump_hidden_fingerprints(model):
    """--dump-hidden-at inside the prompt prints the layer-0 kv fingerprint
    lines and the per-layer hidden lines in the reference's format."""
    r = _run(model, "-p", "the quick brown fox", "-n", "2", "-t", "0", "--dump-hidden-at", "1")
    for tag in ("attn_norm", "K_pre_norm", "K_pre_rope", "K_store", "K_read0", "K_readN"):
        assert re.search(r"\[kv L0 P[01]\] " + tag + r" sum=-?\d+\.\d{4} l2=\d+\.\d{4} max=\d+\.\d{4} v0=", r.stderr), tag
    assert "[hidden pos 1] layer  0 q_out sum=" in r.stderr and "[hidden pos 1] after_emb" in r.stderr
