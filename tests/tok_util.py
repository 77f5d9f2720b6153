"""Synthetic tokenizer.mmtok files for the tokenizer tests.

write_mmtok follows the file layout the reference's packer writes (tools/provision.py:
201-215). make_tokenizer learns a small BPE vocabulary from a seeded synthetic corpus, in
the SentencePiece style of the real files: <unk>, <s>, </s>, the 256 <0xNN> byte pieces,
single characters, then one piece per learned merge; a few extra merges whose result is
not a vocabulary piece exercise the byte fallback.
"""
import collections
import random
import struct

SP = "▁"


def write_mmtok(path, pieces, merges, bos=1, eos=2, unk=0):
    with open(path, "wb") as f:
        f.write(b"MMTOK1\n\x00")
        f.write(struct.pack("<II", len(pieces), len(merges)))
        f.write(struct.pack("<iii", bos, eos, unk))
        for p in pieces:
            b = p.encode("utf-8")
            f.write(struct.pack("<I", len(b)))
            f.write(b)
        for m in merges:
            b = m.encode("utf-8")
            f.write(struct.pack("<I", len(b)))
            f.write(b)
    return path


WORDS = ["the", "quick", "brown", "fox", "jumps", "over", "lazy", "dog", "once", "upon", "a", "time",
         "capital", "of", "france", "is", "paris", "matmul", "free", "ternary", "weights", "recurrent",
         "state", "hello", "world", "tokens", "über", "naïve", "café", "日本語", "テスト", "emoji😀"]


def corpus(rng, n=400):
    lines = []
    for _ in range(n):
        k = rng.randint(1, 9)
        lines.append(" ".join(rng.choice(WORDS) for _ in range(k)))
    return lines


def make_tokenizer(path, seed=0, n_merges=300, junk_merges=12):
    rng = random.Random(seed)
    seqs = [list(SP + line.replace(" ", SP)) for line in corpus(rng)]
    pieces = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    seen = set(pieces)
    for s in seqs:
        for ch in s:
            if ch not in seen:
                seen.add(ch)
                pieces.append(ch)
    merges = []
    for _ in range(n_merges):
        counts = collections.Counter()
        for s in seqs:
            for a, b in zip(s, s[1:]):
                counts[(a, b)] += 1
        if not counts:
            break
        (a, b), c = max(counts.items(), key=lambda kv: (kv[1], kv[0]))
        if c < 2:
            break
        merges.append(f"{a} {b}")
        if a + b not in seen:
            seen.add(a + b)
            pieces.append(a + b)
        new = []
        for s in seqs:
            out, i = [], 0
            while i < len(s):
                if i + 1 < len(s) and s[i] == a and s[i + 1] == b:
                    out.append(a + b)
                    i += 2
                else:
                    out.append(s[i])
                    i += 1
            new.append(out)
        seqs = new
    # merges whose result is not a piece (byte fallback), and one merge listed twice
    chars = [p for p in pieces[259:] if len(p) == 1]
    for _ in range(junk_merges):
        a, b = rng.choice(chars), rng.choice(chars)
        merges.insert(rng.randrange(len(merges) + 1), f"{a} {b}")
    if merges:
        merges.append(merges[0])
    write_mmtok(path, pieces, merges)
    return pieces, merges


def random_texts(seed=1, n=200):
    rng = random.Random(seed)
    alphabet = list("abcdefghijklmnopqrstuvwxyz  ,.!?'0123456789") + ["é", "ü", "ï", "日", "本", "語", "😀", "\t", "\n"]
    out = ["", " ", "  ", "a", " a", "a ", "the quick brown fox", "café naïve über", "日本語テスト", "emoji😀 x"]
    for _ in range(n):
        k = rng.randint(1, 40)
        if rng.random() < 0.5:
            out.append(" ".join(rng.choice(WORDS) for _ in range(rng.randint(1, 8))))
        else:
            out.append("".join(rng.choice(alphabet) for _ in range(k)))
    raw = [s.encode("utf-8") for s in out]
    # invalid / truncated UTF-8 byte strings
    raw += [b"\xff\xfe abc", b"abc\xe2\x96", b"\xf0\x9f\x98", b"\xc3", b"x\x80y", bytes(range(1, 40)),
            b"\xe6\x97\xa5\xe6\x9c", b"tail \xf4"]
    return raw
