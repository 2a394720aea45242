"""The tokenizer's character classes at Unicode 15.0 (cuda/text/unicode_tables.cu:7):
the generated device tables (aotx_amd/csrc/unicode_classes.h) and the oracle's patterns.

- Every code point assigned in Unicode 13.0 has its unicodedata 13.0 class.
- Code points that Unicode 14.0 and 15.0 added have the class of their published general
  category; code points first assigned in 15.1, 16.0 or 17.0 are in no class (they were
  unassigned in 15.0)."""
import bisect
import os
import unicodedata

import pytest

from oracle.text import pretokens

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "aotx_amd", "csrc", "unicode_classes.h")

# (code point, class at Unicode 15.0 or None): a sample of 14.0 and 15.0 additions and of
# the later versions' additions
SAMPLES = [
    (0x0870, "letter"),     # 14.0 Arabic Extended-B ARABIC LETTER ALEF WITH ATTACHED FATHA
    (0x10570, "letter"),    # 14.0 Vithkuqi capital letter A
    (0x1E290, "letter"),    # 14.0 Toto letter PA
    (0x1DF00, "letter"),    # 14.0 Latin Extended-G small letter FENG DIGRAPH WITH TRILL
    (0x0C3C, "mark"),       # 14.0 Telugu sign nukta
    (0x1AC1, "mark"),       # 14.0 combining left parenthesis above left
    (0x1E4D0, "letter"),    # 15.0 Nag Mundari letter O
    (0x1E4F0, "number"),    # 15.0 Nag Mundari digit zero
    (0x11F00, "mark"),      # 15.0 Kawi sign candrabindu
    (0x11F04, "letter"),    # 15.0 Kawi letter A
    (0x1D2C0, "number"),    # 15.0 Kaktovik numeral zero
    (0x1E030, "letter"),    # 15.0 modifier letter Cyrillic small A
    (0x31350, "letter"),    # 15.0 CJK Unified Ideographs Extension H, first
    (0x2B739, "letter"),    # 15.0 CJK Extension C addition
    (0x0CF3, "mark"),       # 15.0 Kannada sign combining anusvara above right
    (0x2EBF0, None),        # 15.1 CJK Extension I
    (0x16D40, None),        # 16.0 Kirat Rai
    (0x10D40, None),        # 16.0 Garay digit
    (0x1CCF0, None),        # 16.0 outlined digit zero
    (0x0897, None),         # 16.0 Arabic pepet
    (0xA7CB, None),         # 16.0 Latin capital letter ram's horn
    (0x11F5A, None),        # 16.0 Kawi sign nukta
    (0x323B0, None),        # 17.0 CJK Extension J
    (0x10940, None),        # 17.0 Sidetic
    (0x1ACF, None),         # 17.0 combining mark
]


def _tables():
    src = open(HEADER).read()
    out = {}
    for name in ("letter", "number", "mark", "space"):
        body = src[src.index(f"aotx_uc_{name}["):]
        body = body[body.index("{") + 1:body.index("}")]
        vals = [int(v.strip().rstrip("u"), 16) for v in body.split(",") if v.strip()]
        ranges = list(zip(vals[0::2], vals[1::2]))
        assert all(a <= b for a, b in ranges)
        assert all(ranges[i][1] < ranges[i + 1][0] for i in range(len(ranges) - 1))
        out[name] = ranges
    return out


@pytest.fixture(scope="module")
def member():
    tabs = _tables()
    starts = {n: [a for a, _ in r] for n, r in tabs.items()}

    def f(name, cp):
        i = bisect.bisect_right(starts[name], cp) - 1
        return i >= 0 and tabs[name][i][0] <= cp <= tabs[name][i][1]
    return f


def test_header_states_unicode_15(member):
    assert "Unicode 15.0" in open(HEADER).read()


def test_assigned_in_13_keep_their_13_class(member):
    for cp in range(0x110000):
        cat = unicodedata.category(chr(cp))
        if cat in ("Cn", "Cs"):
            continue
        assert member("letter", cp) == cat.startswith("L"), hex(cp)
        assert member("number", cp) == cat.startswith("N"), hex(cp)
        assert member("mark", cp) == cat.startswith("M"), hex(cp)
        space = cat in ("Zs", "Zl", "Zp") or 0x09 <= cp <= 0x0D or cp == 0x85
        assert member("space", cp) == space, hex(cp)


@pytest.mark.parametrize("cp,cls", SAMPLES)
def test_versions_14_to_17(member, cp, cls):
    for name in ("letter", "number", "mark", "space"):
        assert member(name, cp) == (name == cls), (hex(cp), name)


def test_oracle_patterns_use_15():
    # a 15.0 letter run joins its word, a 15.1 ideograph does not
    assert pretokens("a\U0001E4D0b \U0002EBF0", "llama3") == ["a\U0001E4D0b", " \U0002EBF0"]
    # Kaktovik numerals are numbers: qwen2 takes them one by one
    assert pretokens("x\U0001D2C0\U0001D2C1", "qwen2") == ["x", "\U0001D2C0", "\U0001D2C1"]
    # a 15.0 mark joins the qwen35 letter run; a 16.0 one does not
    assert pretokens("a\U00011F00b", "qwen35") == ["a\U00011F00b"]
    assert pretokens("a\U00011F5Ab", "qwen35") == ["a", "\U00011F5Ab"]
