"""The GGUF reader and the descriptor built from a file, through the C ABI, without a GPU.

The reader's behaviour follows the reference's own test of its reader (tests/gguf_test.c):
  - round trips of every metadata type, string and number arrays, and tensors of every
    streamed type, each tensor with its own shape and bytes (:92-175, :333-448);
  - each of 18 defects gives the code 2 and no open file (:20-33, :464-489);
  - 64 seeded corruptions of the head give 0, 1 or 2 and never end the process; at
    least 8 are refused, and every file that opens can be walked (:492-574);
  - a head longer than the bound is refused before it is read (:577-612, a sparse file).
The files are built here with a byte builder of this test's own.
The descriptor (aotx_model_desc_file) of an exported synthetic model must equal the one the
runtime builds for it (aotx_amd.model.layout); the rules it follows are pinned by cases that
must be refused: an absent tensor, an unknown architecture, a tensor outside its layer's
kind, and a tensor of the wrong shape or type.
"""
import ctypes
import os
import struct

import numpy as np
import pytest

import aotx_amd
from aotx_amd import TensorInfo, StringArray
from aotx_amd import gguf

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q5_0, T_Q5_1, T_Q8_0, T_Q2_K, T_Q3_K = 0, 1, 2, 3, 6, 7, 8, 10, 11
BLOCK = {T_F32: (1, 4), T_F16: (1, 2), T_Q4_0: (32, 18), T_Q4_1: (32, 20), T_Q5_0: (32, 22),
         T_Q5_1: (32, 24), T_Q8_0: (32, 34), T_Q2_K: (256, 84), T_Q3_K: (256, 110)}
TYPES = [T_F32, T_F16, T_Q4_0, T_Q8_0, T_Q4_1, T_Q5_0, T_Q5_1, T_Q2_K, T_Q3_K]

DEFECTS = ["magic", "version", "meta_count", "tensor_count", "key_long", "string_past",
           "meta_type", "bool", "array_in_array", "array_big", "align", "align_type",
           "dim_count", "row_blocks", "name_long", "offset_align", "tensor_past", "truncate"]


@pytest.fixture(scope="module")
def L():
    return aotx_amd.lib()


def num(v, w):
    return int(v).to_bytes(w, "little", signed=False)


def text(s):
    b = s.encode() if isinstance(s, str) else s
    return num(len(b), 8) + b


def plan(count, defect=None):
    """Tensor plan: every tensor has its own type, shape, bytes and offset."""
    out, at = [], 0
    for i in range(count):
        t = TYPES[i % len(TYPES)]
        nd = 1 + i % 3
        bw, bb = BLOCK[t]
        dims = [(256 if bw == 256 else 32) * (i + 1)] + [((i + d) % 3) + 1 for d in range(1, nd)]
        if defect == "row_blocks" and t == T_Q8_0:
            dims[0] += 1
        weights = int(np.prod(dims))
        nbytes = weights // bw * bb
        out.append(dict(name=f"tensor.{i}.weight", type=t, dims=dims, offset=at, bytes=nbytes))
        at += (nbytes + 31) // 32 * 32
    if defect == "offset_align" and count > 1:
        out[1]["offset"] += 1
        at += 32
    if defect == "tensor_past" and count > 0:
        out[-1]["offset"] += at
    return out, at


def tensor_bytes(i, n):
    k = np.arange(n, dtype=np.uint64)
    return (((i + 1) * 131 + k * 17 + (k >> 8)) & 0xFF).astype(np.uint8)


def pairs(defect, elements):
    b = bytearray()
    b += text("general.architecture") + num(STRING, 4)
    b += (num(1 << 40, 8) + b"aotx.test") if defect == "string_past" else text("aotx.test")
    b += text("general.alignment")
    if defect == "align_type":
        b += num(STRING, 4) + text("32")
    else:
        b += num(U32, 4) + num(33 if defect == "align" else 32, 4)
    b += text("tokenizer.ggml.pre") + num(STRING, 4) + text("qwen2")
    b += text("k" * 511 if defect == "key_long" else "test.u8")
    b += num(99 if defect == "meta_type" else U8, 4) + num(200, 1)
    b += text("test.i8") + num(I8, 4) + num(256 - 100, 1)
    b += text("test.u16") + num(U16, 4) + num(60000, 2)
    b += text("test.i16") + num(I16, 4) + num(65536 - 30000, 2)
    b += text("test.u32") + num(U32, 4) + num(4000000000, 4)
    b += text("test.i32") + num(I32, 4) + num(2 ** 32 - 2000000000, 4)
    b += text("test.f32") + num(F32, 4) + struct.pack("<f", 1.5)
    b += text("test.bool") + num(BOOL, 4) + num(7 if defect == "bool" else 1, 1)
    b += text("test.u64") + num(U64, 4) + num(18000000000000000000, 8)
    b += text("test.i64") + num(I64, 4) + num(2 ** 64 - 9000000000000000000, 8)
    b += text("test.f64") + num(F64, 4) + struct.pack("<d", 2.25)
    b += text("test.strings") + num(ARRAY, 4) + num(ARRAY if defect == "array_in_array" else STRING, 4)
    b += num(elements, 8) + b"".join(text(f"token.{i}") for i in range(elements))
    b += text("test.i32s") + num(ARRAY, 4) + num(I32, 4)
    b += num(100000000 if defect == "array_big" else elements, 8)
    b += b"".join(struct.pack("<i", i - elements // 2) for i in range(elements))
    b += text("test.f32s") + num(ARRAY, 4) + num(F32, 4) + num(elements, 8)
    b += b"".join(struct.pack("<f", i * 0.5 + 0.25) for i in range(elements))
    b += text("test.u8s") + num(ARRAY, 4) + num(U8, 4) + num(elements, 8)
    b += bytes(i & 0xFF for i in range(elements))
    return bytes(b), 18


def build(defect=None, tensors=8, elements=8):
    p, data_bytes = plan(tensors, defect)
    meta, npairs = pairs(defect, elements)
    b = bytearray(b"GGUX" if defect == "magic" else b"GGUF")
    b += num(2 if defect == "version" else 3, 4)
    b += num(1 << 40 if defect == "tensor_count" else tensors, 8)
    b += num(1 << 40 if defect == "meta_count" else npairs, 8)
    b += meta
    for i, t in enumerate(p):
        b += text("n" * 199 if (defect == "name_long" and i == 0) else t["name"])
        b += num(0 if (defect == "dim_count" and i == 0) else len(t["dims"]), 4)
        b += b"".join(num(d, 8) for d in t["dims"])
        b += num(t["type"], 4) + num(t["offset"], 8)
    head_end = (len(b) + 31) // 32 * 32
    b += b"\0" * (head_end - len(b))
    body = np.zeros(data_bytes, dtype=np.uint8)
    for i, t in enumerate(p):
        lo = t["offset"]
        hi = min(lo + t["bytes"], data_bytes)
        if lo < hi:
            body[lo:hi] = tensor_bytes(i, hi - lo)
    return bytes(b) + body.tobytes(), head_end, p


def open_file(L, path):
    h = ctypes.c_void_p()
    rc = L.aotx_modelfile_open(str(path).encode(), ctypes.byref(h))
    return rc, h


def check_file(L, path, tensors, elements, p):
    rc, h = open_file(L, path)
    assert rc == 0 and h
    try:
        s, n = ctypes.c_void_p(), ctypes.c_size_t()
        assert L.aotx_modelfile_string(h, b"general.architecture", ctypes.byref(s), ctypes.byref(n)) == 0
        assert ctypes.string_at(s, n.value) == b"aotx.test"
        assert L.aotx_modelfile_string(h, b"tokenizer.ggml.pre", ctypes.byref(s), ctypes.byref(n)) == 0
        assert ctypes.string_at(s, n.value) == b"qwen2"
        u = ctypes.c_uint32()
        for key, want in ((b"test.u8", 200), (b"test.u16", 60000), (b"test.u32", 4000000000),
                          (b"test.bool", 1)):
            assert L.aotx_modelfile_u32(h, key, ctypes.byref(u)) == 0 and u.value == want, key
        u64 = ctypes.c_uint64()
        assert L.aotx_modelfile_u64(h, b"test.u64", ctypes.byref(u64)) == 0
        assert u64.value == 18000000000000000000
        f = ctypes.c_float()
        assert L.aotx_modelfile_f32(h, b"test.f32", ctypes.byref(f)) == 0 and f.value == 1.5
        assert L.aotx_modelfile_f32(h, b"test.f64", ctypes.byref(f)) == 0 and f.value == 2.25
        assert L.aotx_modelfile_u32(h, b"test.i8", ctypes.byref(u)) == 2      # negative
        assert L.aotx_modelfile_u64(h, b"test.i64", ctypes.byref(u64)) == 2
        assert L.aotx_modelfile_u32(h, b"test.u64", ctypes.byref(u)) == 2     # does not fit
        assert L.aotx_modelfile_u32(h, b"test.absent", ctypes.byref(u)) == 1
        assert L.aotx_modelfile_string(h, b"test.u8", ctypes.byref(s), ctypes.byref(n)) == 2
        arr = StringArray()
        assert L.aotx_modelfile_strings(h, b"test.strings", ctypes.byref(arr)) == 0
        assert arr.count == elements
        for i in range(elements):
            lo, hi = arr.offsets[i], arr.offsets[i + 1]
            assert bytes(arr.bytes[lo:hi]) == f"token.{i}".encode()
        vp, cnt = ctypes.c_void_p(), ctypes.c_uint64()
        assert L.aotx_modelfile_i32s(h, b"test.i32s", ctypes.byref(vp), ctypes.byref(cnt)) == 0
        assert cnt.value == elements
        got = np.ctypeslib.as_array(ctypes.cast(vp, ctypes.POINTER(ctypes.c_int32)), (elements,))
        assert np.array_equal(got, np.arange(elements) - elements // 2)
        assert L.aotx_modelfile_f32s(h, b"test.f32s", ctypes.byref(vp), ctypes.byref(cnt)) == 0
        got = np.ctypeslib.as_array(ctypes.cast(vp, ctypes.POINTER(ctypes.c_float)), (elements,))
        assert np.array_equal(got, np.arange(elements, dtype=np.float32) * 0.5 + 0.25)
        assert L.aotx_modelfile_i32s(h, b"test.u8s", ctypes.byref(vp), ctypes.byref(cnt)) == 2
        assert L.aotx_modelfile_tensor_count(h) == tensors
        info = TensorInfo()
        for i, t in enumerate(p):
            assert L.aotx_modelfile_tensor(h, i, ctypes.byref(info)) == 0
            assert info.name.decode() == t["name"]
            assert info.type == t["type"] and info.dim_count == len(t["dims"])
            assert list(info.dims[:info.dim_count]) == t["dims"]
            assert info.bytes == t["bytes"] and info.offset == t["offset"]
            assert L.aotx_modelfile_find(h, t["name"].encode(), ctypes.byref(info)) == 0
            buf = np.zeros(info.bytes, dtype=np.uint8)
            assert L.aotx_modelfile_read(h, info.offset, info.bytes, buf.ctypes.data) == 0
            assert np.array_equal(buf, tensor_bytes(i, info.bytes))
            if info.bytes > 1:
                half = info.bytes // 2
                a = np.zeros(half, dtype=np.uint8)
                c = np.zeros(info.bytes - half, dtype=np.uint8)
                assert L.aotx_modelfile_read(h, info.offset, half, a.ctypes.data) == 0
                assert L.aotx_modelfile_read(h, info.offset + half, info.bytes - half, c.ctypes.data) == 0
                assert np.array_equal(np.concatenate([a, c]), buf)
        assert L.aotx_modelfile_find(h, b"tensor.absent", ctypes.byref(info)) == 1
        assert L.aotx_modelfile_tensor(h, tensors, ctypes.byref(info)) == 1
        one = np.zeros(8, dtype=np.uint8)
        data = L.aotx_modelfile_data_bytes(h)
        assert L.aotx_modelfile_read(h, data, 1, one.ctypes.data) == 2
        big = np.zeros(data + 1, dtype=np.uint8)
        assert L.aotx_modelfile_read(h, 0, data + 1, big.ctypes.data) == 2
        assert L.aotx_modelfile_file_bytes(h) == os.path.getsize(path)
        assert L.aotx_modelfile_header_bytes(h) % 32 == 0
    finally:
        L.aotx_modelfile_close(h)


@pytest.mark.parametrize("tensors,elements", [(1, 1), (64, 64)])
def test_round_trip(L, tmp_path, tensors, elements):
    data, _, p = build(None, tensors, elements)
    path = tmp_path / f"good-{tensors}.gguf"
    path.write_bytes(data)
    check_file(L, path, tensors, elements, p)


@pytest.mark.parametrize("defect", DEFECTS)
def test_defect_refused(L, tmp_path, defect):
    data, head_end, _ = build(defect, tensors=1 if defect == "align" else 8)
    if defect == "truncate":
        data = data[:head_end // 2]
    path = tmp_path / f"defect-{defect}.gguf"
    path.write_bytes(data)
    rc, h = open_file(L, path)
    assert rc == 2, defect
    assert not h


def test_head_limit(L, tmp_path):
    """A string that claims 280 MB in a 320 MB sparse file: the head bound is 256 MiB."""
    head = b"GGUF" + num(3, 4) + num(0, 8) + num(1, 8) + text("big") + num(STRING, 4) + num(280000000, 8)
    path = tmp_path / "head.gguf"
    with open(path, "wb") as f:
        f.write(head)
        f.truncate(320 * 1024 * 1024)
    rc, h = open_file(L, path)
    assert rc == 2 and not h


def test_missing_file(L, tmp_path):
    rc, h = open_file(L, tmp_path / "absent.gguf")
    assert rc == 1 and not h


def test_fuzz(L, tmp_path):
    data, head_end, _ = build(None, 8, 8)
    seed = 20260827
    refused = opened = 0
    path = tmp_path / "fuzz.gguf"
    for i in range(64):
        copy = bytearray(data)
        seed = (seed * 1103515245 + 12345) & 0xFFFFFFFF
        hits = 1 + (seed >> 16) % 4
        for _ in range(hits):
            seed = (seed * 1103515245 + 12345) & 0xFFFFFFFF
            place = (seed >> 8) % head_end
            seed = (seed * 1103515245 + 12345) & 0xFFFFFFFF
            copy[place] = (seed >> 16) & 0xFF
        if i % 8 == 7:
            seed = (seed * 1103515245 + 12345) & 0xFFFFFFFF
            copy = copy[:(seed >> 8) % len(data)]
        path.write_bytes(bytes(copy))
        rc, h = open_file(L, path)
        assert rc in (0, 1, 2), (i, rc)
        if rc != 0:
            assert not h
            refused += rc == 2
            continue
        opened += 1
        s, n = ctypes.c_void_p(), ctypes.c_size_t()
        L.aotx_modelfile_string(h, b"general.architecture", ctypes.byref(s), ctypes.byref(n))
        arr = StringArray()
        if L.aotx_modelfile_strings(h, b"test.strings", ctypes.byref(arr)) == 0:
            total = arr.offsets[arr.count]
            assert total == sum(arr.offsets[j + 1] - arr.offsets[j] for j in range(arr.count))
        info = TensorInfo()
        small = np.zeros(4096, dtype=np.uint8)
        for t in range(L.aotx_modelfile_tensor_count(h)):
            if L.aotx_modelfile_tensor(h, t, ctypes.byref(info)) == 0:
                L.aotx_modelfile_read(h, info.offset, min(info.bytes, 4096), small.ctypes.data)
        L.aotx_modelfile_close(h)
    assert refused >= 8, refused


# ---- the descriptor of a file ---------------------------------------------------------

@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    from aotx_amd.model import TINY, build_host
    region, lay = build_host(TINY, seed=1)
    path = tmp_path_factory.mktemp("tiny") / "tiny.gguf"
    gguf.export(TINY, region, lay, path)
    return path, region, lay


def _describe(path):
    with gguf.ModelFile(path) as mf:
        return mf.describe()


def test_descriptor_of_exported_model(tiny_file):
    path, region, lay = tiny_file
    d, binding, count = _describe(path)
    w = lay.desc
    for f in ("layers", "hidden", "ffn", "heads", "kv_heads", "head_dim", "vocab", "context",
              "rope_pairs", "expert_count", "expert_used_count", "weight_type"):
        assert getattr(d, f) == getattr(w, f), f
    assert d.rope_theta == np.float32(w.rope_theta) and d.rms_eps == np.float32(w.rms_eps)
    assert list(d.kind[:d.layers]) == list(w.kind[:w.layers])
    assert count == 5 + 9 * d.layers
    names = [binding[i].name.decode() for i in range(count)]
    assert names[:5] == ["token_embd.weight", "output_norm.weight", "output.weight",
                         "cls.output.weight", "rope_freqs.weight"]
    assert names[5] == "blk.0.attn_norm.weight" and names[-1] == f"blk.{d.layers - 1}.ffn_down.weight"
    assert [binding[i].needed for i in range(5)] == [1, 1, 0, 0, 0]
    # the slot of each layer tensor: 5 + layer * 14 + slot
    assert binding[5 + 9 * 3 + 1].slot == 5 + 3 * 14 + aotx_amd.SLOT["attn_q"]


def test_descriptor_qk_norm_and_experts(tmp_path):
    from aotx_amd.model import Shape, build_host
    for name, shape, kind in (
            ("qwen3", Shape(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64,
                            vocab=512, qk_norm=True, pairs=0), aotx_amd.AOTX_LAYER_KIND_ATTENTION),
            ("moe", Shape(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64,
                          vocab=512, experts=4, used=2), aotx_amd.AOTX_LAYER_KIND_FFN_EXPERTS)):
        region, lay = build_host(shape, seed=2)
        path = tmp_path / f"{name}.gguf"
        gguf.export(shape, region, lay, path)
        d, _, _ = _describe(path)
        assert list(d.kind[:2]) == [kind, kind], name
        assert d.rope_pairs == shape.pairs and d.expert_count == shape.experts


def _rewrite(src, dst, drop=(), add=(), meta_change=None):
    """Copy a GGUF file through the reader, dropping or adding tensors or changing keys."""
    import aotx_amd as A
    L = A.lib()
    with gguf.ModelFile(src) as mf:
        tensors = []
        info = TensorInfo()
        for t in range(L.aotx_modelfile_tensor_count(mf.h)):
            L.aotx_modelfile_tensor(mf.h, t, ctypes.byref(info))
            name = info.name.decode()
            if name in drop:
                continue
            buf = np.zeros(info.bytes, dtype=np.uint8)
            assert L.aotx_modelfile_read(mf.h, info.offset, info.bytes, buf.ctypes.data) == 0
            tensors.append((name, info.type, list(info.dims[:info.dim_count]), buf.tobytes()))
    from aotx_amd.model import TINY
    arch = "llama"
    meta = [("general.architecture", gguf.STRING, arch), ("llama.block_count", gguf.U32, TINY.layers),
            ("llama.embedding_length", gguf.U32, TINY.hidden), ("llama.context_length", gguf.U32, 8192),
            ("llama.feed_forward_length", gguf.U32, TINY.ffn),
            ("llama.attention.head_count", gguf.U32, TINY.heads),
            ("llama.attention.head_count_kv", gguf.U32, TINY.kv_heads),
            ("llama.rope.freq_base", gguf.F32, TINY.theta),
            ("llama.attention.layer_norm_rms_epsilon", gguf.F32, TINY.eps)]
    if meta_change:
        meta = meta_change(meta)
    gguf.write(dst, meta, tensors + list(add))


def test_descriptor_refusals(tiny_file, tmp_path):
    path, _, _ = tiny_file
    p = tmp_path / "x.gguf"
    # the head width comes from hidden / heads when the key is absent
    _rewrite(path, p)
    d, _, _ = _describe(p)
    assert d.head_dim == 64
    cases = [
        (dict(drop=("blk.2.attn_k.weight",)), "has no tensor blk.2.attn_k.weight"),
        (dict(drop=("output_norm.weight",)), "has no tensor output_norm.weight"),
        (dict(meta_change=lambda m: [(k.replace("llama.", "gpt9."), t,
                                      "gpt9" if k == "general.architecture" else v)
                                     for k, t, v in m]), "no rotary pair rule"),
        (dict(meta_change=lambda m: [x for x in m if x[0] != "llama.rope.freq_base"]),
         "llama.rope.freq_base"),
        (dict(add=[("blk.1.attn_q.bias", gguf.T_F32, [256], bytes(1024))]), "outside its layer"),
        (dict(add=[("blk.9.attn_q.weight", gguf.T_F32, [256], bytes(1024))]), "past the layer count"),
        (dict(drop=("blk.0.ffn_norm.weight",),
              add=[("blk.0.ffn_norm.weight", gguf.T_F16, [256], bytes(512))]), "type or shape"),
        (dict(drop=("blk.1.attn_v.weight",),
              add=[("blk.1.attn_v.weight", gguf.T_Q8_0, [256, 128], bytes(128 * 8 * 34))]),
         "type or shape"),
        (dict(meta_change=lambda m: [(k, t, 3 if k == "llama.attention.head_count_kv" else v)
                                     for k, t, v in m]), "head count"),
    ]
    for kw, want in cases:
        _rewrite(path, p, **kw)
        with pytest.raises(ValueError) as e:
            _describe(p)
        assert want in str(e.value), (kw, str(e.value))
