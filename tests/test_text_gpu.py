"""The tokenizer on the GPU (aotx_text_encode / aotx_text_detok) against its oracle, on a
vocabulary trained by the `tokenizers` library, for four split families."""
import ctypes
import random

import numpy as np
import pytest

import aotx_amd
from aotx_amd import TextSource, TextStore
from oracle.text import Vocab
from tests.text_util import text, trained

pytestmark = pytest.mark.gpu

ROWS = {"qwen2": 0, "llama3": 4, "gpt-2": 13, "qwen35": 19}


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


@pytest.fixture(scope="module")
def bpe():
    return trained()


def _runs(strings):
    data = [s if isinstance(s, bytes) else s.encode("utf-8") for s in strings]
    at = np.zeros(len(data) + 1, dtype=np.uint64)
    at[1:] = np.cumsum([len(d) for d in data])
    return np.frombuffer(b"".join(data), dtype=np.uint8).copy(), at


class Built:
    """The library's vocabulary built from tokens/merges/types for a family."""

    def __init__(self, lib, tokens, merges, types, family):
        self.lib = lib
        self.keep = []
        tb, ta = _runs(tokens)
        mb, ma = _runs(merges)
        ty = np.asarray(types, dtype=np.int32)
        self.keep += [tb, ta, mb, ma, ty]
        src = TextSource()
        src.token_bytes, src.token_at, src.tokens = tb.ctypes.data, ta.ctypes.data, len(tokens)
        src.merge_bytes, src.merge_at, src.merges = mb.ctypes.data, ma.ctypes.data, len(merges)
        src.token_type = ty.ctypes.data
        src.family = ROWS[family]
        self.store = TextStore()
        assert lib.aotx_text_vocab_build(ctypes.byref(src), ctypes.byref(self.store)) == 0

    def close(self):
        self.lib.aotx_text_vocab_release(ctypes.byref(self.store))


def _encode(torch, lib, strings):
    data, at = _runs(strings)
    d = torch.from_numpy(data if len(data) else np.zeros(1, np.uint8)).cuda()
    a = torch.from_numpy(at.view(np.int64)).cuda()
    ids = torch.zeros(max(3 * int(at[-1]), 1), dtype=torch.int32, device="cuda")
    cnt = torch.zeros(len(strings), dtype=torch.int32, device="cuda")
    assert lib.aotx_text_encode(d.data_ptr(), a.data_ptr(), len(strings), ids.data_ptr(),
                                cnt.data_ptr(), None) == 0
    ids, cnt = ids.cpu().numpy(), cnt.cpu().numpy()
    return [list(ids[3 * int(at[i]):3 * int(at[i]) + int(cnt[i])]) for i in range(len(strings))]


def _detok(torch, lib, seqs, limit=4096):
    at = np.zeros(len(seqs) + 1, dtype=np.uint64)
    at[1:] = np.cumsum([len(s) for s in seqs])
    flat = np.asarray([x for s in seqs for x in s] or [0], dtype=np.int32)
    ids = torch.from_numpy(flat).cuda()
    a = torch.from_numpy(at.view(np.int64)).cuda()
    out = torch.zeros(len(seqs) * limit, dtype=torch.uint8, device="cuda")
    ln = torch.zeros(len(seqs), dtype=torch.int32, device="cuda")
    assert lib.aotx_text_detok(ids.data_ptr(), a.data_ptr(), len(seqs), out.data_ptr(), limit,
                               ln.data_ptr(), None) == 0
    torch.cuda.synchronize()
    o, ln = out.cpu().numpy(), ln.cpu().numpy()
    return [bytes(o[i * limit:i * limit + int(ln[i])]) for i in range(len(seqs))]


@pytest.mark.parametrize("family", ["gpt-2", "llama3", "qwen2", "qwen35"])
def test_encode_detok_vs_oracle(torch, lib, bpe, family):
    tokens, merges, _ = bpe
    types = [1] * len(tokens)
    v = Vocab(tokens, merges, types, family=family)
    built = Built(lib, tokens, merges, types, family)
    try:
        rep = (ctypes.c_uint32 * 4)()
        assert lib.aotx_text_vocab_report(rep) == 0
        assert rep[0] == len(tokens) and rep[1] == len(merges) and rep[2] == 0
        rng = random.Random(21 + ROWS[family])
        strings = [text(rng, rng.randint(1, 60)) for _ in range(200)] + ["", "a", " ", "\n\n\n"]
        got = _encode(torch, lib, strings)
        for s, g in zip(strings, got):
            assert g == v.encode(s.encode()), (family, repr(s))
        back = _detok(torch, lib, got)
        assert back == [s.encode() for s in strings]
    finally:
        built.close()


def test_long_piece_and_control(torch, lib, bpe):
    """A letter run longer than the chunk bound is cut and still decodes to itself; a
    control token gives no bytes."""
    tokens, merges, _ = bpe
    types = [1] * len(tokens)
    v = Vocab(tokens, merges, types, family="gpt-2")
    ids = v.encode(b"hello world")
    types[ids[0]] = aotx_amd.AOTX_SEQ_STATE_DONE   # 3: the control type
    built = Built(lib, tokens, merges, types, "gpt-2")
    try:
        long = "ab" * 3000 + " tail"
        got = _encode(torch, lib, [long])[0]
        assert 0 < len(got) < len(long)
        assert _detok(torch, lib, [got], limit=8192)[0] == long.encode()
        assert _detok(torch, lib, [got], limit=100)[0] == long.encode()[:100]   # cut at limit
        assert _detok(torch, lib, [ids])[0] == Vocab(tokens, merges, family="gpt-2").decode(ids[1:])
    finally:
        built.close()


@pytest.mark.parametrize("family", ["gpt-2", "llama3"])
def test_special_tokens_vs_oracle(torch, lib, bpe, family):
    """Control and user tokens are whole matches (longest at the leftmost place); control
    tokens give no bytes back, user tokens give their text."""
    from tests.test_text import SPECIALS, with_specials
    tokens, merges, _ = bpe
    toks, types = with_specials(tokens, merges)
    v = Vocab(toks, merges, types, family=family)
    built = Built(lib, toks, merges, types, family)
    try:
        rng = random.Random(31)
        strings = []
        for _ in range(150):
            parts = [text(rng, rng.randint(0, 8)) for _ in range(3)]
            strings.append(rng.choice(SPECIALS).join(parts) + rng.choice(["", "<|start|>x", "<|sx", "<|"]))
        got = _encode(torch, lib, strings)
        for s, g in zip(strings, got):
            assert g == v.encode(s.encode()), (family, repr(s))
        back = _detok(torch, lib, got)
        assert back == [v.decode(g) for g in got]
        assert _detok(torch, lib, [[len(tokens) + 2]])[0] == b"<|s"      # user type: its text
        assert _detok(torch, lib, [[len(tokens)]])[0] == b""             # control type: nothing
    finally:
        built.close()


def test_text_end_to_end_from_gguf(torch, orc, bpe, tmp_path):
    """Text in, text out: a GGUF file carrying the tiny model and a tokenizer; the prompt
    encoded on the GPU (as the oracle does), a prompt pass and greedy steps through the
    model, the reply decoded on the GPU (as the oracle does)."""
    from aotx_amd import gguf
    from aotx_amd.model import TINY, Runtime, build_host
    from aotx_amd.text import Tokenizer
    from tests.gpu_util import rel_rms
    tokens, merges, _ = bpe
    pad = TINY.vocab - len(tokens)
    toks = list(tokens) + [f"<unused_{i}>" for i in range(pad)]
    types = [1] * len(tokens) + [3] * pad
    region, lay = build_host(TINY, seed=1)
    path = tmp_path / "tiny_text.gguf"
    gguf.export(TINY, region, lay, path, tokenizer=(toks, merges, types, "llama-bpe"))
    region_f, desc = gguf.load(path)
    v = Vocab(toks, merges, types, family="llama3")
    tk = Tokenizer(path=path)
    rt = Runtime(region_f, desc, max_tokens=64, pool_pages=64)
    try:
        prompt = "hello world, it's the café 12345 <unused_3> дом"
        ids = tk.encode([prompt])[0]
        assert ids == v.encode(prompt.encode()) and 0 < len(ids) < 64
        ref = orc.Model(lay.desc, region, slots=8, max_context=128)
        tok, _, logits = rt.step(ids, [0, len(ids)], [2])
        want = ref.step(ids, [0, len(ids)], [2])
        assert rel_rms(logits, want) < 1e-2
        reply = [int(np.argmax(want[0]))]
        for _ in range(7):
            tok, _, logits = rt.step([reply[-1]], [0, 1], [2])
            want = ref.step([reply[-1]], [0, 1], [2])
            assert rel_rms(logits, want) < 1e-2
            reply.append(int(np.argmax(want[0])))
        assert tk.decode([reply])[0] == v.decode(reply)
        assert tk.decode([ids])[0] == v.decode(ids)
        assert rt.faulted() == 0
    finally:
        rt.close()
        tk.close()


def test_invalid_utf8_vs_oracle(torch, lib, bpe):
    """Bytes that start no character are encoded as U+FFFD, as the oracle's clean does."""
    tokens, merges, _ = bpe
    v = Vocab(tokens, merges, family="llama3")
    built = Built(lib, tokens, merges, [1] * len(tokens), "llama3")
    try:
        rng = random.Random(41)
        bad = [b"\xff", b"\x80", b"\xe4\xb8", b"\xc0\xaf", b"\xed\xa0\x80", b"\xf4\x90\x80\x80"]
        strings = []
        for _ in range(100):
            parts = [text(rng, rng.randint(0, 6)).encode() for _ in range(3)]
            strings.append(rng.choice(bad).join(parts) + rng.choice([b"", b"\xe4", b"\xf0\x9f"]))
        got = _encode(torch, lib, strings)
        for s_, g in zip(strings, got):
            assert g == v.encode(s_), repr(s_)
    finally:
        built.close()


NEW_POINTS = ["\u0870", "\U00010570", "\U0001E290", "\u0C3C", "\U0001E4D0", "\U0001E4F0",
              "\U00011F00", "\U00011F04", "\U0001D2C0", "\U0001E030", "\U00031350", "\u0CF3",
              "\U0002EBF0", "\U00016D40", "\U00010D40", "\U0001CCF0", "\u0897", "\uA7CB",
              "\U00011F5A", "\U000323B0"]


@pytest.mark.parametrize("family", ["gpt-2", "llama3", "qwen2", "qwen35"])
def test_unicode_15_classes_vs_oracle(torch, lib, bpe, family):
    """Code points added in Unicode 14.0 and 15.0 split as letters, numbers and marks; those
    added in 15.1-17.0 as unassigned code points (the reference's tables are 15.0)."""
    tokens, merges, _ = bpe
    types = [1] * len(tokens)
    v = Vocab(tokens, merges, types, family=family)
    built = Built(lib, tokens, merges, types, family)
    try:
        rng = random.Random(77 + ROWS[family])
        strings = []
        for _ in range(120):
            parts = []
            for _ in range(rng.randint(1, 12)):
                r = rng.random()
                parts.append(rng.choice(NEW_POINTS) * rng.randint(1, 3) if r < 0.5
                             else rng.choice(["a", "xy", " ", "12", "\n", "!", "é", "中"]))
            strings.append("".join(parts))
        got = _encode(torch, lib, strings)
        for s, g in zip(strings, got):
            assert g == v.encode(s.encode()), (family, repr(s))
        assert _detok(torch, lib, got) == [s.encode() for s in strings]
    finally:
        built.close()
