"""Writes the synthetic tokenizer fixture tests/golden/tok/ and the encode
vectors tests/golden/tok_cases.json.

The tokenizer is a byte-level BPE trained with the HuggingFace `tokenizers`
library on seeded synthetic text (the model's own tokenizer files need a
download), exported in the reference's TSV format (vocab.tsv "<id>\\t<token>",
merges.tsv "<rank>\\t<A>\\t<B>", special.tsv "<id>\\t<content>";
tools/export_tokenizer.py:1-9).  The expected ids of each case come from the
same library, configured as the reference's encoder behaves: special tokens
matched literally (earliest, then longest), the GPT-2 split pattern below,
byte-level mapping, BPE with a whole-piece vocabulary lookup before merging
(`ignore_merges`).  The cases keep to text on which the reference's
hand-coded pattern and this regex agree (no tab, vertical tab or form feed
before a letter; non-ASCII code points only letters).

    python tests/golden/make_tok.py
"""
import json
import os
import random

from tokenizers import AddedToken, Regex, Tokenizer, decoders, models, pre_tokenizers, trainers

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "tok")
PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}"
           r"| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")
# (one a prefix of another: the longer wins where both match)
SPECIALS = ["<|startoftext|>", "<|im_start|>", "<|im_end|>", "<think>", "<think></think>", "<|pad|>"]


def corpus(seed=5, n=6000):
    rng = random.Random(seed)
    syl = ["ka", "to", "ri", "en", "the", "and", "ing", "st", "qu", "ion", "ré", "ß", "über",
           "на", "ми", "中", "文", "ño", "ll", "ve", "ai", "ou"]
    words = ["".join(rng.choice(syl) for _ in range(rng.randint(1, 4))) for _ in range(400)]
    words += ["Paris", "France", "capital", "The", "model", "don't", "I'm", "we'll", "they're"]
    punct = [".", ",", "!", "?", ";", ":", "...", "(", ")", "\"", "-", "'", "--", "[]"]
    lines = []
    for _ in range(n):
        toks = []
        for _ in range(rng.randint(3, 14)):
            r = rng.random()
            if r < 0.75:
                w = rng.choice(words)
                toks.append(w.capitalize() if rng.random() < 0.15 else w)
            elif r < 0.87:
                toks.append(str(rng.randint(0, 99999)))
            else:
                toks.append(rng.choice(punct))
        sep = rng.choice([" ", " ", " ", "  ", "\n", " \n", "\n\n"])
        lines.append(" ".join(toks) + sep)
    return lines


def pre_tokenizer():
    return pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])


def train():
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizer()
    tr = trainers.BpeTrainer(vocab_size=1500, min_frequency=2, special_tokens=SPECIALS,
                             initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                             show_progress=False)
    tok.train_from_iterator(corpus(), trainer=tr)
    return json.loads(tok.to_str())


def export(tj):
    os.makedirs(OUT, exist_ok=True)
    vocab, merges = tj["model"]["vocab"], tj["model"]["merges"]
    with open(os.path.join(OUT, "vocab.tsv"), "w", encoding="utf-8", newline="\n") as f:
        for s, i in sorted(vocab.items(), key=lambda kv: kv[1]):
            f.write(f"{i}\t{s}\n")
    with open(os.path.join(OUT, "merges.tsv"), "w", encoding="utf-8", newline="\n") as f:
        for rank, m in enumerate(merges):
            a, b = m.split(" ", 1) if isinstance(m, str) else m
            f.write(f"{rank}\t{a}\t{b}\n")
    with open(os.path.join(OUT, "special.tsv"), "w", encoding="utf-8", newline="\n") as f:
        for a in tj["added_tokens"]:
            f.write(f"{a['id']}\t{a['content']}\n")
    return vocab, [tuple(m.split(" ", 1)) if isinstance(m, str) else tuple(m) for m in merges]


def reference_like(vocab, merges, added):
    """The library configured as the reference encodes."""
    tok = Tokenizer(models.BPE(vocab=vocab, merges=merges, ignore_merges=True))
    tok.pre_tokenizer = pre_tokenizer()
    tok.decoder = decoders.ByteLevel()
    tok.add_special_tokens([AddedToken(a["content"], special=True, normalized=False,
                                       lstrip=False, rstrip=False, single_word=False)
                            for a in added])
    return tok


CASES = [
    "The capital of France is Paris.",
    "<|startoftext|><|im_start|>user\nWhat is the capital of France?<|im_end|>\n"
    "<|im_start|>assistant\n",
    "I'm sure they're right; we'll see, don't you THINK so? 'Tis 'LL 'Re",
    "12345678 3.14159 -42 1,000,000 year2024 x1y22z333",
    "a  b   c    d\n\n\ne \r\n f  \n",
    "trailing spaces   ",
    "   leading spaces",
    "über straße niño на ми 中文 résumé",
    "!!!??? ... --- ((()))\n\n[]{}<>",
    "<|im_end|><|im_end|>\n<|pad|>x<|pad|>",
    "<think></think><think>x</think><think></think",
    "kato rien the ing stion quai",
    "",
    " ",
    "\n",
    "'",
    "'s",
    "a'b",
]


def random_cases(seed=11, n=60):
    rng = random.Random(seed)
    alpha = ("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789"
             "     \n\r.,;:!?'\"()-_/+*=#@&%$<>|[]{}~^`") + "éßñ中文ми"
    out = []
    for _ in range(n):
        s = "".join(rng.choice(alpha) for _ in range(rng.randint(1, 80)))
        if rng.random() < 0.3:
            k = rng.randint(0, len(s))
            s = s[:k] + rng.choice(SPECIALS) + s[k:]
        out.append(s)
    return out


def main():
    tj = train()
    vocab, merges = export(tj)
    tok = reference_like(vocab, merges, tj["added_tokens"])
    cases = []
    for text in CASES + random_cases():
        ids = tok.encode(text, add_special_tokens=False).ids
        cases.append({"text": text, "ids": ids})
    with open(os.path.join(HERE, "tok_cases.json"), "w", encoding="utf-8") as f:
        json.dump({"pattern": PATTERN, "cases": cases}, f, ensure_ascii=False, indent=0)
    print(f"vocab {len(vocab)} merges {len(merges)} special {len(tj['added_tokens'])} "
          f"cases {len(cases)} -> {OUT}")


if __name__ == "__main__":
    main()
