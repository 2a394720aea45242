"""The tokenizer from Python: a vocabulary from a GGUF file or from arrays, and encode /
decode of strings on the GPU through include/aotx_text.h."""
import ctypes

import numpy as np

from . import TextSource, TextStore, check, lib


def _runs(items):
    data = [x if isinstance(x, bytes) else x.encode("utf-8") for x in items]
    at = np.zeros(len(data) + 1, dtype=np.uint64)
    at[1:] = np.cumsum([len(d) for d in data])
    return np.frombuffer(b"".join(data) or b"\0", dtype=np.uint8).copy(), at


class Tokenizer:
    """The library's current vocabulary (one at a time per process)."""

    def __init__(self, path=None, tokens=None, merges=None, types=None, family="gpt-2"):
        self.L = lib()
        self.store = TextStore()
        if path is not None:
            from .gguf import ModelFile
            with ModelFile(path) as mf:
                check(self.L.aotx_text_vocab_file(mf.h, ctypes.byref(self.store)), "aotx_text_vocab_file")
            return
        tb, ta = _runs(tokens)
        mb, ma = _runs(merges or [])
        ty = np.asarray(types if types is not None else [1] * len(tokens), dtype=np.int32)
        row = ctypes.c_uint32()
        check(self.L.aotx_text_family_find(family.encode(), len(family), ctypes.byref(row)), "family")
        src = TextSource(tb.ctypes.data, ta.ctypes.data, len(tokens), mb.ctypes.data,
                         ma.ctypes.data, len(merges or []), ty.ctypes.data, row.value)
        check(self.L.aotx_text_vocab_build(ctypes.byref(src), ctypes.byref(self.store)), "aotx_text_vocab_build")

    def close(self):
        self.L.aotx_text_vocab_release(ctypes.byref(self.store))

    def encode(self, texts):
        """Token id lists of a list of strings (or bytes)."""
        import torch
        data, at = _runs(texts)
        d = torch.from_numpy(data).cuda()
        a = torch.from_numpy(at.view(np.int64)).cuda()
        ids = torch.zeros(max(3 * int(at[-1]), 1), dtype=torch.int32, device="cuda")
        cnt = torch.zeros(len(texts), dtype=torch.int32, device="cuda")
        check(self.L.aotx_text_encode(d.data_ptr(), a.data_ptr(), len(texts), ids.data_ptr(),
                                      cnt.data_ptr(), None), "aotx_text_encode")
        ids, cnt = ids.cpu().numpy(), cnt.cpu().numpy()
        return [[int(x) for x in ids[3 * int(at[i]):3 * int(at[i]) + int(cnt[i])]] for i in range(len(texts))]

    def decode(self, seqs, limit=1 << 16):
        """Bytes of a list of token id lists."""
        import torch
        at = np.zeros(len(seqs) + 1, dtype=np.uint64)
        at[1:] = np.cumsum([len(s) for s in seqs])
        flat = torch.tensor([x for s in seqs for x in s] or [0], dtype=torch.int32, device="cuda")
        a = torch.from_numpy(at.view(np.int64)).cuda()
        out = torch.zeros(len(seqs) * limit, dtype=torch.uint8, device="cuda")
        ln = torch.zeros(len(seqs), dtype=torch.int32, device="cuda")
        check(self.L.aotx_text_detok(flat.data_ptr(), a.data_ptr(), len(seqs), out.data_ptr(), limit,
                                     ln.data_ptr(), None), "aotx_text_detok")
        o, ln = out.cpu().numpy(), ln.cpu().numpy()
        return [bytes(o[i * limit:i * limit + int(ln[i])]) for i in range(len(seqs))]
