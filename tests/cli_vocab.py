"""A small Gemma-like vocabulary for synthetic models that the CLI can
tokenize: the special pieces at the ids the real model uses (bos 2,
<|think|> 98, <|channel> 100, <channel|> 101, <|turn> 105, <turn|> 106, the
newline 107), the characters of a corpus and merges learned from it."""
import synth

CORPUS = ["the quick brown fox jumps over the lazy dog", "hello, how are you? i am fine", "user model system thought"]
AT = {0: "<pad>", 1: "<eos>", 2: "<bos>", 3: "<unk>", 98: "<|think|>", 100: "<|channel>", 101: "<channel|>",
      105: "<|turn>", 106: "<turn|>", 107: "\n", 108: "<|channel>thought\n"}


def pieces_and_merges(size: int):
    chars = sorted({c for line in CORPUS for c in synth.escape_line(line, True)} | set("<|>?,."))
    merges = synth.bpe_train(CORPUS, 200, True)
    free = [i for i in range(size) if i not in AT]
    pieces = dict(AT)
    seen = set(AT.values())
    items = chars + [a + b for a, b in merges]
    for p in items:
        if p in seen or not free:
            continue
        seen.add(p)
        pieces[free.pop(0)] = p
    out = [pieces.get(i, f"<t{i}>") for i in range(size)]
    return tuple(out), tuple(f"{a} {b}" for a, b in merges)
