"""Byte-level BPE tokenizer restated in Python — TEST INFRASTRUCTURE ONLY.

Follows the reference's cuda/text/: the byte map of cuda/text/text.cuh:256-290 (the GPT-2
byte-to-code-point map), the split patterns whose alternatives cuda/text/pretok.cu:6-45
states (written here as the published regular expressions of those families, run by the
`regex` module), the merge step of cuda/text/bpe.cu (the pair of lowest merge rank first,
the leftmost of equal ranks; with the family's whole rule a pre-token that is a token
stays whole, cuda/text/families.h:18-23), and the detokenizer of cuda/text/detok.cu
(byte-level code points give their byte, control tokens give nothing).
"""
import os
import sys

import regex

PATTERNS_17 = {
    "qwen2": r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+",
    "llama3": r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+",
    "gpt2": r"'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+",
    "qwen35": r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}\p{M}]?[\p{L}\p{M}]+|\p{N}| ?[^\s\p{L}\p{N}\p{M}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+",
}


def _unicode15():
    """The letter/number/mark class bodies at Unicode 15.0, the reference's table version
    (cuda/text/unicode_tables.cu:7), from the generator of the device tables
    (aotx_amd/csrc/gen_unicode.py: the `regex` module's 17.0 classes minus the code
    points of 15.1-17.0); tests/test_unicode.py pins those tables."""
    here = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "aotx_amd", "csrc")
    sys.path.insert(0, here)
    try:
        import gen_unicode
    finally:
        sys.path.remove(here)
    body = {}
    for name, pred in gen_unicode.classes():
        if name == "space":
            continue
        body[name] = "".join(f"\\U{a:08x}-\\U{b:08x}" for a, b in gen_unicode.ranges(pred))
    return body


def _at15(pattern, body):
    """A pattern with \\p{L}, \\p{N}, \\p{M} replaced by the 15.0 class bodies (inside a
    bracket expression the body alone, outside it a bracket expression of its own)."""
    key = {"L": body["letter"], "N": body["number"], "M": body["mark"]}
    out, i, depth = [], 0, 0
    while i < len(pattern):
        if pattern.startswith("\\p{", i) and pattern[i + 3] in key and pattern[i + 4] == "}":
            b = key[pattern[i + 3]]
            out.append(b if depth else "[" + b + "]")
            i += 5
            continue
        ch = pattern[i]
        if ch == "\\":
            out.append(pattern[i:i + 2])
            i += 2
            continue
        if ch == "[":
            depth += 1
        elif ch == "]" and depth:
            depth -= 1
        out.append(ch)
        i += 1
    return "".join(out)


class _Patterns(dict):
    """The family patterns at Unicode 15.0, built on first use."""

    def __missing__(self, name):
        if not hasattr(self, "_body"):
            self._body = _unicode15()
        self[name] = regex.compile(_at15(PATTERNS_17[name], self._body))
        return self[name]


PATTERNS = _Patterns()

# pattern row and whole rule of each family (cuda/text/families.h:10-43)
FAMILY = {"qwen2": ("qwen2", False), "llama3": ("llama3", True), "llama-bpe": ("llama3", True),
          "gpt-2": ("gpt2", False), "qwen35": ("qwen35", False)}


def byte_point(b):
    if 0x21 <= b <= 0x7E or 0xA1 <= b <= 0xAC or 0xAE <= b <= 0xFF:
        return b
    if b <= 0x20:
        return 0x100 + b
    if b <= 0xA0:
        return 0x100 + 33 + (b - 0x7F)
    return 0x100 + 67


POINT_BYTE = {byte_point(b): b for b in range(256)}


def byte_string(bs):
    """The byte-level string of raw bytes."""
    return "".join(chr(byte_point(b)) for b in bs)


def clean(data):
    """Bytes with every byte that starts no UTF-8 character written as U+FFFD (EF BF BD),
    one per byte (cuda/text/text.cuh:367-374): a lead byte needs its continuation bytes,
    no overlong form, no surrogate, nothing past U+10FFFF."""
    out, pos, n = bytearray(), 0, len(data)
    while pos < n:
        c = data[pos]
        if c < 0x80:
            out.append(c); pos += 1; continue
        if c & 0xE0 == 0xC0:
            need, cp, lo = 1, c & 0x1F, 0x80
        elif c & 0xF0 == 0xE0:
            need, cp, lo = 2, c & 0x0F, 0x800
        elif c & 0xF8 == 0xF0:
            need, cp, lo = 3, c & 0x07, 0x10000
        else:
            need = None
        ok = need is not None and pos + need < n
        if ok:
            for i in range(1, need + 1):
                d = data[pos + i]
                if d & 0xC0 != 0x80:
                    ok = False
                    break
                cp = (cp << 6) | (d & 0x3F)
        if ok and (cp < lo or cp > 0x10FFFF or 0xD800 <= cp <= 0xDFFF):
            ok = False
        if ok:
            out += data[pos:pos + need + 1]; pos += need + 1
        else:
            out += b"\xef\xbf\xbd"; pos += 1
    return bytes(out)


def pretokens(text, pattern):
    """Pre-tokens of a str (consecutive, covering it)."""
    return [m.group(0) for m in PATTERNS[pattern].finditer(text)]


class Vocab:
    def __init__(self, tokens, merges, types=None, family="gpt-2"):
        self.tokens = list(tokens)
        self.id = {}
        for i, t in enumerate(self.tokens):
            self.id.setdefault(t, i)
        self.rank = {}
        for r, m in enumerate(merges):
            sp = m.find(" ", 1)
            if sp < 0:
                continue
            left, right = m[:sp], m[sp + 1:]
            if left in self.id and right in self.id and left + right in self.id:
                self.rank.setdefault((self.id[left], self.id[right]), (r, self.id[left + right]))
        self.types = list(types) if types is not None else [1] * len(self.tokens)
        self.pattern, self.whole = FAMILY[family]
        # tokens of the control (3) and user (4) types: whole matches found first
        self.specials = [(t.encode("utf-8"), i) for i, t in enumerate(self.tokens)
                         if self.types[i] in (3, 4) and t]

    def merge(self, piece_bytes):
        s = byte_string(piece_bytes)
        if self.whole and s in self.id:
            return [self.id[s]]
        sym = [self.id[ch] for ch in s]
        while len(sym) > 1:
            best = None
            for i in range(len(sym) - 1):
                got = self.rank.get((sym[i], sym[i + 1]))
                if got is not None and (best is None or got[0] < best[0]):
                    best = (got[0], i, got[1])
            if best is None:
                break
            _, i, res = best
            sym[i:i + 2] = [res]
        return sym

    def special_at(self, data, at):
        """The longest special token starting at `at` (pretok.cu:339-372): (length, id)."""
        best = (0, None)
        for s, i in self.specials:
            if len(s) > best[0] and data.startswith(s, at):
                best = (len(s), i)
        return best

    def encode(self, data):
        """Token ids of UTF-8 bytes: the leftmost special token splits the text, the
        pattern and the merges run on the text between (pretok.cu:404-431)."""
        out, pos = [], 0
        data = clean(data)
        while pos < len(data):
            stop, (n, sid) = pos, (0, None)
            while stop < len(data) and self.specials:
                n, sid = self.special_at(data, stop)
                if n:
                    break
                stop += 1
            if not self.specials:
                stop = len(data)
            for piece in pretokens(data[pos:stop].decode("utf-8"), self.pattern):
                out += self.merge(piece.encode("utf-8"))
            pos = stop
            if n:
                out.append(sid)
                pos = stop + n
        return out

    def decode(self, ids):
        out = bytearray()
        for i in ids:
            if i >= len(self.tokens) or self.types[i] == 3:
                continue
            for ch in self.tokens[i]:
                p = ord(ch)
                if p in POINT_BYTE:
                    out.append(POINT_BYTE[p])
                else:
                    out += ch.encode("utf-8")
        return bytes(out)
