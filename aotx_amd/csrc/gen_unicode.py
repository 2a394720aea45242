"""Write unicode_classes.h: the code point ranges of the tokenizer's character classes
(letters L*, numbers N*, marks M*, white space) at Unicode 15.0, the version of the
reference's tables (cuda/text/unicode_tables.cu:7).

No Unicode 15.0 database is on this machine: Python's unicodedata is 13.0, and the
`regex` module (which the tokenizer patterns of the `tokenizers` library follow) is 17.0.
The 15.0 classes are therefore the 17.0 classes of `regex` minus every code point that
Unicode 15.1, 16.0 and 17.0 assigned (POST15 below), found three ways:
  - blocks that did not exist in 15.0, taken whole (their names and ranges from the
    block list of fontTools, a 17.0 list);
  - code points that are wide or zero-width in the 16.0/17.0 width tables of `rich` (from
    the wcwidth project) but not in its 15.0 table, inside blocks that already existed;
  - the few narrow letters and marks those versions added to existing blocks, listed by
    hand (NARROW_ADDED).
Every code point assigned in 13.0 keeps its unicodedata 13.0 class (tests check that
the table agrees with unicodedata there, and classify sample code points of 14.0, 15.0
and of the later versions).

Run from the repository root: python3 aotx_amd/csrc/gen_unicode.py"""
import bisect
import importlib.util
import os
import sys
import unicodedata

import regex

SPACE_EXTRA = {0x85}       # NEXT LINE: white space by the Unicode property, category Cc

# blocks first allocated in Unicode 15.1, 16.0 and 17.0
POST15_BLOCKS = [
    "CJK Unified Ideographs Extension I",                                       # 15.1
    "Todhri", "Garay", "Tulu-Tigalari", "Myanmar Extended-C", "Sunuwar",         # 16.0
    "Egyptian Hieroglyphs Extended-A", "Gurung Khema", "Kirat Rai",
    "Symbols for Legacy Computing Supplement", "Ol Onal",
    "Sidetic", "Sharada Supplement", "Tolong Siki", "Beria Erfe",                # 17.0
    "Tangut Components Supplement", "Miscellaneous Symbols Supplement", "Tai Yo",
    "CJK Unified Ideographs Extension J",
]

# narrow letters and marks that 16.0 and 17.0 added to blocks of 15.0 (inclusive ranges)
NARROW_ADDED = [
    (0x088F, 0x088F),      # Arabic Extended-B
    (0x0C5C, 0x0C5C),      # Telugu
    (0x0CDC, 0x0CDC),      # Kannada
    (0x1C89, 0x1C8A),      # Cyrillic Extended-C (TJE)
    (0xA7CB, 0xA7CF), (0xA7D2, 0xA7D2), (0xA7D4, 0xA7D4), (0xA7DA, 0xA7DC),
    (0xA7F1, 0xA7F1),      # Latin Extended-D
    (0x10EC2, 0x10EC7),    # Arabic Extended-C
    (0x2B73A, 0x2B73F),    # CJK Extension C (15.0 ends at U+2B739)
    (0x2CEA2, 0x2CEAD),    # CJK Extension E
]


def _rich_widths(version):
    import rich
    path = os.path.join(os.path.dirname(rich.__file__), "_unicode_data", f"unicode{version}.py")
    spec = importlib.util.spec_from_file_location("w" + version.replace("-", "_"), path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    starts = [a for a, _, _ in mod.cell_table.widths]
    return mod.cell_table.widths, starts


def _width(table, cp):
    widths, starts = table
    i = bisect.bisect_right(starts, cp) - 1
    if i >= 0:
        a, b, w = widths[i]
        if a <= cp <= b:
            return w
    return 1


def post15():
    """Code points assigned after Unicode 15.0."""
    from fontTools.unicodedata import Blocks
    out = set()
    for i, name in enumerate(Blocks.VALUES):
        if name in POST15_BLOCKS:
            end = Blocks.RANGES[i + 1] - 1 if i + 1 < len(Blocks.RANGES) else 0x10FFFF
            out.update(range(Blocks.RANGES[i], end + 1))
    found = {n for n in Blocks.VALUES if n in POST15_BLOCKS}
    assert found == set(POST15_BLOCKS), set(POST15_BLOCKS) - found
    w15 = _rich_widths("15-0-0")
    later = [_rich_widths("16-0-0"), _rich_widths("17-0-0")]
    assigned = regex.compile(r"\p{Assigned}")
    for cp in range(0x110000):
        if 0xD800 <= cp <= 0xDFFF or unicodedata.category(chr(cp)) != "Cn":
            continue                               # assigned in 13.0 (or a surrogate)
        if not assigned.match(chr(cp)):
            continue
        if _width(w15, cp) == 1 and any(_width(t, cp) in (0, 2) for t in later):
            out.add(cp)
    for lo, hi in NARROW_ADDED:
        out.update(range(lo, hi + 1))
    return out


def ranges(pred):
    out, lo = [], None
    for cp in range(0x110000):
        hit = pred(cp)
        if hit and lo is None:
            lo = cp
        elif not hit and lo is not None:
            out.append((lo, cp - 1))
            lo = None
    if lo is not None:
        out.append((lo, 0x10FFFF))
    return out


def classes():
    """(name, predicate) of the four classes at Unicode 15.0."""
    later = post15()
    letter, number, mark = (regex.compile(p) for p in (r"\p{L}", r"\p{N}", r"\p{M}"))
    white = regex.compile(r"\p{White_Space}")

    def of(pat):
        def pred(cp):
            if cp in later or 0xD800 <= cp <= 0xDFFF:
                return False
            return pat.match(chr(cp)) is not None
        return pred

    def space(cp):
        if 0xD800 <= cp <= 0xDFFF:
            return False
        return white.match(chr(cp)) is not None or cp in SPACE_EXTRA

    return [("letter", of(letter)), ("number", of(number)), ("mark", of(mark)), ("space", space)]


def main():
    lines = ["/* Generated by gen_unicode.py: the inclusive code point ranges of the tokenizer's",
             " * character classes at Unicode 15.0, sorted. Do not edit. */",
             "#ifndef AOTX_UNICODE_CLASSES_H", "#define AOTX_UNICODE_CLASSES_H", ""]
    for name, pred in classes():
        rs = ranges(pred)
        lines.append(f"#define AOTX_UC_{name.upper()}_RANGES {len(rs)}u")
        lines.append(f"static __device__ const unsigned int aotx_uc_{name}[{2 * len(rs)}] = {{")
        flat = [f"0x{v:x}u" for r in rs for v in r]
        for i in range(0, len(flat), 10):
            lines.append("    " + ", ".join(flat[i:i + 10]) + ",")
        lines.append("};")
        lines.append("")
    lines.append("#endif")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "unicode_classes.h")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(path, file=sys.stderr)


if __name__ == "__main__":
    main()
