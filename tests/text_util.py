"""A small byte-level BPE vocabulary trained with the `tokenizers` library on a seeded
synthetic corpus, and random texts over code points whose classes (letter, number, mark,
white space) the `regex` module and Unicode 13.0 agree on."""
import json
import random
import unicodedata

import regex

CANDIDATES = (
    [chr(c) for c in range(0x20, 0x7F)] + ["\n", "\r", "\t", "\n\n"]
    + list("éèñüößçÅøÆœ") + list("αβγδεζηθΑΒΓΔ") + list("домикПРИВЕТ")
    + list("一二三中文字漢語") + list("٣٤٥") + ["́", "̈", "ः"]
    + ["😀", "🚀", "€", "©", " ", "　", " "]
)


def _agree(ch):
    if len(ch) != 1:
        return True
    cat = unicodedata.category(ch)
    checks = [(r"\p{L}", cat.startswith("L")), (r"\p{N}", cat.startswith("N")),
              (r"\p{M}", cat.startswith("M"))]
    return all(bool(regex.fullmatch(p, ch)) == want for p, want in checks)


POOL = [c for c in CANDIDATES if _agree(c)]
WORDS = ["hello", "world", "it's", "don't", "we're", "THE", "café", "naïve", "αβγ", "дом",
         "中文", "123456", "42", "x", "ab", "aaaa", "--", "!!", "...", "😀😀"]


def text(rng, n):
    parts = []
    while len(parts) < n:
        r = rng.random()
        if r < 0.5:
            parts.append(rng.choice(WORDS))
        elif r < 0.8:
            parts.append(rng.choice([" ", " ", "  ", "\n", " \n ", "\t"]))
        else:
            parts.append("".join(rng.choice(POOL) for _ in range(rng.randint(1, 4))))
    return "".join(parts)


def corpus(seed=7, lines=400):
    rng = random.Random(seed)
    return [text(rng, 30) for _ in range(lines)]


def trained(vocab_size=800):
    """(tokens in id order, merges as "left right", the tokenizers.Tokenizer)."""
    from tokenizers import Tokenizer, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    tr = trainers.BpeTrainer(vocab_size=vocab_size, show_progress=False,
                             initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(corpus(), tr)
    model = json.loads(tok.to_str())["model"]
    vocab = model["vocab"]
    tokens = [None] * len(vocab)
    for s, i in vocab.items():
        tokens[i] = s
    merges = [m if isinstance(m, str) else f"{m[0]} {m[1]}" for m in model["merges"]]
    return tokens, merges, tok


def hf_with(pattern, tokens, merges, whole):
    """A tokenizers.Tokenizer over the same vocabulary that splits with `pattern` and,
    with `whole`, keeps a pre-token that is a token whole (ignore_merges)."""
    from tokenizers import Regex, Tokenizer, models, pre_tokenizers
    vocab = {t: i for i, t in enumerate(tokens)}
    pairs = [tuple(m.split(" ", 1)) for m in merges]
    tok = Tokenizer(models.BPE(vocab=vocab, merges=pairs, ignore_merges=whole))
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(pattern), "isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    return tok
