"""The tokenizer's oracle (oracle/text.py) pinned against an independent BPE
implementation (the `tokenizers` library) on a vocabulary it trained, and the family
table of the library (no GPU)."""
import random

import pytest

from oracle.text import FAMILY, PATTERNS_17, Vocab, pretokens
from tests.text_util import hf_with, text, trained


@pytest.fixture(scope="module")
def bpe():
    return trained()


@pytest.mark.parametrize("family", ["gpt-2", "llama3", "qwen2", "qwen35"])
def test_oracle_matches_tokenizers_library(bpe, family):
    tokens, merges, _ = bpe
    pattern, whole = FAMILY[family]
    v = Vocab(tokens, merges, family=family)
    hf = hf_with(PATTERNS_17[pattern], tokens, merges, whole)
    rng = random.Random(11)
    for _ in range(300):
        s = text(rng, rng.randint(1, 40))
        assert v.encode(s.encode()) == hf.encode(s).ids, repr(s)


def test_gpt2_split_is_the_byte_level_pretokenizer(bpe):
    """The gpt2 pattern here equals the library's own ByteLevel split."""
    tokens, merges, hf = bpe
    v = Vocab(tokens, merges, family="gpt-2")
    rng = random.Random(12)
    for _ in range(200):
        s = text(rng, rng.randint(1, 40))
        assert v.encode(s.encode()) == hf.encode(s).ids, repr(s)


def test_pretokens_cover_text_and_known_splits():
    rng = random.Random(13)
    for pattern in PATTERNS_17:
        for _ in range(100):
            s = text(rng, 20)
            assert "".join(pretokens(s, pattern)) == s
    # numbers: llama3 groups of three from the left, qwen2 one by one, gpt2 one run
    assert pretokens("x 1234567", "llama3") == ["x", " ", "123", "456", "7"]
    assert pretokens("x 1234567", "qwen2") == ["x", " ", "1", "2", "3", "4", "5", "6", "7"]
    assert pretokens("x 1234567", "gpt2") == ["x", " 1234567"]
    # contractions: any case for llama3, small letters only for gpt2
    assert pretokens("IT'S", "llama3") == ["IT", "'S"]
    assert pretokens("IT'S", "gpt2") == ["IT", "'", "S"]
    # a space run gives back its last space to a following word; newlines end a run
    assert pretokens("a   b", "gpt2") == ["a", "  ", " b"]
    assert pretokens("a \n\n b", "llama3") == ["a", " \n\n", " b"]


def test_decode_round_trip_and_control(bpe):
    tokens, merges, _ = bpe
    types = [1] * len(tokens)
    v = Vocab(tokens, merges, types, family="llama3")
    rng = random.Random(14)
    for _ in range(100):
        b = text(rng, 30).encode()
        assert v.decode(v.encode(b)) == b
    ids = v.encode(b"hello world")
    types[ids[0]] = 3
    v2 = Vocab(tokens, merges, types, family="llama3")
    assert v2.decode(ids) == v.decode(ids[1:])


def test_family_table(lib):
    import ctypes
    row = ctypes.c_uint32()
    names = ["qwen2", "deepseek-r1-qwen", "kormo", "f2llmv2", "llama3", "llama-v3", "llama-bpe",
             "falcon3", "falcon-h1", "pixtral", "midm-2.0", "lfm2", "jina-v5-nano", "gpt-2", "mpt",
             "olmo", "jais", "trillion", "granite-docling", "qwen35"]
    for i, n in enumerate(names):
        assert lib.aotx_text_family_find(n.encode(), len(n), ctypes.byref(row)) == 0 and row.value == i
    assert lib.aotx_text_family_find(b"nope", 4, ctypes.byref(row)) == 1


SPECIALS = ["<|eot|>", "<|start|>", "<|s"]


def with_specials(tokens, merges):
    """The trained vocabulary plus three special tokens (two control, one user type, one a
    prefix of another so that the longest match decides)."""
    toks = list(tokens) + SPECIALS
    types = [1] * len(tokens) + [3, 3, 4]
    return toks, types


@pytest.mark.parametrize("family", ["gpt-2", "llama3"])
def test_special_tokens_match_tokenizers_library(bpe, family):
    from tokenizers import AddedToken
    tokens, merges, _ = bpe
    toks, types = with_specials(tokens, merges)
    pattern, whole = FAMILY[family]
    hf = hf_with(PATTERNS_17[pattern], tokens, merges, whole)
    hf.add_special_tokens([AddedToken(t, special=True, normalized=False) for t in SPECIALS])
    assert [hf.token_to_id(t) for t in SPECIALS] == [len(tokens), len(tokens) + 1, len(tokens) + 2]
    v = Vocab(toks, merges, types, family=family)
    rng = random.Random(15)
    for _ in range(200):
        parts = [text(rng, rng.randint(0, 8)) for _ in range(3)]
        s = rng.choice(SPECIALS).join(parts) + rng.choice(["", "<|start|>x", "<|sx", "<|"])
        assert v.encode(s.encode()) == hf.encode(s).ids, repr(s)


def test_clean_by_hand():
    """Each byte that starts no character becomes U+FFFD (cuda/text/text.cuh:367-374)."""
    from oracle.text import clean
    R = "\ufffd".encode()
    assert clean(b"a\xffb") == b"a" + R + b"b"
    assert clean("中".encode()[:2]) == R + R                     # cut off by the end
    assert clean(b"\xe4\xb8x") == R + R + b"x"                   # cut by a non-continuation
    assert clean(b"\xc0\xaf") == R + R                          # overlong
    assert clean(b"\xed\xa0\x80") == R + R + R                  # surrogate
    assert clean(b"\xf4\x90\x80\x80") == R * 4                  # past U+10FFFF
    assert clean("😀é\ufffd".encode()) == "😀é\ufffd".encode()   # valid text unchanged
    assert clean(b"\x80") == R and clean(b"") == b""
