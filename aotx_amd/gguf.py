"""GGUF model files on the host side: a writer, the export of a synthetic model, and the
load of a file into a weights region through the native reader.

The reading, the descriptor and the placement are the library's (include/aotx_modelfile.h:
aotx_modelfile_*, aotx_model_desc_file, aotx_model_place), as the reference's loader reads
its files in C (disk/modelfile/gguf.c, cuda/model/desc_file_host.cu). This module writes
files (the reference ships no writer; its tests build files byte by byte,
tests/gguf_test.c:50-90, :273-317) and drives the C calls.
"""
import ctypes
import struct

import numpy as np

from . import (AOTX_DESC_MAX_BINDINGS, AOTX_MODEL_LANGUAGE, ModelBinding, ModelDesc, check,
               lib)

MAGIC = b"GGUF"
VERSION = 3
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
T_F32, T_F16, T_Q8_0 = 0, 1, 8
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}


def _text(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STRING:
        return _text(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        if etype == STRING:
            return out + b"".join(_text(x) for x in items)
        return out + b"".join(struct.pack(_SCALAR[etype], x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def write(path, metadata, tensors, alignment=32):
    """Write a GGUF v3 file. metadata: [(key, type, value)] (ARRAY value = (element type,
    items)); tensors: [(name, type, dims (fastest first), bytes)]. Tensor bytes are laid
    out in order, each at a multiple of the alignment."""
    head = bytearray(MAGIC + struct.pack("<IQQ", VERSION, len(tensors), len(metadata)))
    for key, vtype, v in metadata:
        head += _text(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, at = [], 0
    for _, _, _, data in tensors:
        at = (at + alignment - 1) // alignment * alignment
        offsets.append(at)
        at += len(data)
    for (name, ttype, dims, _), off in zip(tensors, offsets):
        head += _text(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, off)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        pos = 0
        for data, off in zip((t[3] for t in tensors), offsets):
            f.write(b"\0" * (off - pos))
            f.write(data)
            pos = off + len(data)


def export(shape, region, lay, path, arch=None, tokenizer=None):
    """Write the synthetic model of `lay` (aotx_amd.model.layout / build_host: the same
    bytes) as a GGUF file with the reference's tensor names (cuda/model/names.h,
    kinds_data.h): llama (adjacent rotary pairs) or qwen3 (split pairs, Q/K norm)."""
    from . import SLOT
    d = lay.desc
    if arch is None:
        arch = "qwen3" if shape.qk_norm else "llama"
    h, hd = shape.hidden, shape.head_dim
    wide, narrow, f = shape.heads * hd, shape.kv_heads * hd, shape.ffn
    e = shape.experts

    def q8(rows, k):
        return rows * (k // 32) * 34

    def grab(off, nbytes):
        return bytes(np.asarray(region[off:off + nbytes], dtype=np.uint8))

    tensors = [("token_embd.weight", T_Q8_0, [h, shape.vocab], grab(d.token_embd, q8(shape.vocab, h))),
               ("output_norm.weight", T_F32, [h], grab(d.output_norm, 4 * h))]
    if not shape.tied:
        tensors.append(("output.weight", T_Q8_0, [h, shape.vocab], grab(d.output, q8(shape.vocab, h))))
    for l in range(shape.layers):
        L = d.layer[l].offset
        b = f"blk.{l}."
        tensors += [(b + "attn_norm.weight", T_F32, [h], grab(L[SLOT["attn_norm"]], 4 * h)),
                    (b + "attn_q.weight", T_Q8_0, [h, wide], grab(L[SLOT["attn_q"]], q8(wide, h))),
                    (b + "attn_k.weight", T_Q8_0, [h, narrow], grab(L[SLOT["attn_k"]], q8(narrow, h))),
                    (b + "attn_v.weight", T_Q8_0, [h, narrow], grab(L[SLOT["attn_v"]], q8(narrow, h))),
                    (b + "attn_output.weight", T_Q8_0, [wide, h], grab(L[SLOT["attn_o"]], q8(h, wide)))]
        if shape.qk_norm:
            tensors += [(b + "attn_q_norm.weight", T_F32, [hd], grab(L[SLOT["q_norm"]], 4 * hd)),
                        (b + "attn_k_norm.weight", T_F32, [hd], grab(L[SLOT["k_norm"]], 4 * hd))]
        tensors.append((b + "ffn_norm.weight", T_F32, [h], grab(L[SLOT["ffn_norm"]], 4 * h)))
        if e:
            tensors += [(b + "ffn_gate_exps.weight", T_Q8_0, [h, f, e], grab(L[SLOT["ffn_gate"]], e * q8(f, h))),
                        (b + "ffn_up_exps.weight", T_Q8_0, [h, f, e], grab(L[SLOT["ffn_up"]], e * q8(f, h))),
                        (b + "ffn_down_exps.weight", T_Q8_0, [f, h, e], grab(L[SLOT["ffn_down"]], e * q8(h, f))),
                        (b + "ffn_gate_inp.weight", T_F32, [h, e], grab(L[SLOT["router"]], 4 * h * e))]
        else:
            tensors += [(b + "ffn_gate.weight", T_Q8_0, [h, f], grab(L[SLOT["ffn_gate"]], q8(f, h))),
                        (b + "ffn_up.weight", T_Q8_0, [h, f], grab(L[SLOT["ffn_up"]], q8(f, h))),
                        (b + "ffn_down.weight", T_Q8_0, [f, h], grab(L[SLOT["ffn_down"]], q8(h, f)))]
    meta = [("general.architecture", STRING, arch),
            ("general.alignment", U32, 32),
            (f"{arch}.block_count", U32, shape.layers),
            (f"{arch}.embedding_length", U32, h),
            (f"{arch}.context_length", U32, d.context),
            (f"{arch}.feed_forward_length", U32, f),
            (f"{arch}.attention.head_count", U32, shape.heads),
            (f"{arch}.attention.head_count_kv", U32, shape.kv_heads),
            (f"{arch}.attention.key_length", U32, hd),
            (f"{arch}.rope.freq_base", F32, shape.theta),
            (f"{arch}.attention.layer_norm_rms_epsilon", F32, shape.eps)]
    if e:
        meta += [(f"{arch}.expert_count", U32, e), (f"{arch}.expert_used_count", U32, shape.used)]
    if tokenizer is not None:
        # (tokens, merges "left right", token types, tokenizer.ggml.pre value)
        toks, merges, types, pre = tokenizer
        meta += [("tokenizer.ggml.model", STRING, "gpt2"), ("tokenizer.ggml.pre", STRING, pre),
                 ("tokenizer.ggml.tokens", ARRAY, (STRING, list(toks))),
                 ("tokenizer.ggml.token_type", ARRAY, (I32, [int(t) for t in types])),
                 ("tokenizer.ggml.merges", ARRAY, (STRING, list(merges)))]
    write(path, meta, tensors)


class ModelFile:
    """An open GGUF file (aotx_modelfile_open); close() or use as a context manager."""

    def __init__(self, path):
        self.L = lib()
        self.h = ctypes.c_void_p()
        self.rc = self.L.aotx_modelfile_open(str(path).encode(), ctypes.byref(self.h))
        if self.rc != 0:
            raise OSError(f"aotx_modelfile_open({path}) gave {self.rc}")

    def close(self):
        if self.h:
            self.L.aotx_modelfile_close(self.h)
            self.h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def describe(self, role=AOTX_MODEL_LANGUAGE):
        """(descriptor, bindings) of the file (aotx_model_desc_file); raises with the
        library's reason when the file cannot make a runnable descriptor."""
        desc = ModelDesc()
        binding = (ModelBinding * AOTX_DESC_MAX_BINDINGS)()
        count = ctypes.c_uint32(0)
        reason = ctypes.create_string_buffer(256)
        rc = self.L.aotx_model_desc_file(self.h, role, ctypes.byref(desc), binding,
                                         AOTX_DESC_MAX_BINDINGS, ctypes.byref(count), reason, 256)
        if rc != 0:
            raise ValueError(reason.value.decode())
        return desc, binding, count.value


def load(path, role=AOTX_MODEL_LANGUAGE, device="cuda"):
    """Read a GGUF file into a new weights region on the device: (region tensor, desc).
    The region then goes to aotx_amd.model.Runtime(region, desc)."""
    import torch
    with ModelFile(path) as mf:
        desc, binding, count = mf.describe(role)
        need = mf.L.aotx_model_place_bytes(mf.h, binding, count)
        region = torch.empty(int(need), dtype=torch.uint8, device=device)
        check(mf.L.aotx_mem_weights_set(region.data_ptr(), region.numel()), "weights")
        reason = ctypes.create_string_buffer(256)
        if mf.L.aotx_model_place(mf.h, ctypes.byref(desc), binding, count, reason, 256) != 0:
            raise ValueError(reason.value.decode())
    return region, desc
