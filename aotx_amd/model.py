"""Synthetic Llama/MoE-shaped models for the C ABI, and a thin runtime over it.

The reference loads GGUF files into a runtime-owned weights region and fills a
descriptor of byte offsets (cuda/model/model.cuh:50-86). This module builds the same
two things for the synthetic configurations the benchmarks name: a weights region laid
out tensor by tensor (256-byte aligned) and an `aotx_model_desc` that points into it.
Linear weights are Q8_0 blocks of N(0, sigma) values from the build's deterministic
integer normal generator (identical to `aotx_synth_q8` / `aotx_synth_q8_host`); norm
weights are 1.

`Runtime` drives the model-step operator surface exactly as the reference's tests do
(tests/model_test.cu:281-296): aotx_model_pages -> aotx_kv_serve -> aotx_model_sample.
"""
import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import (AOTX_LAYER_KIND_ATTENTION, AOTX_LAYER_KIND_ATTENTION_NO_QK_NORM,
               AOTX_LAYER_KIND_FFN_EXPERTS, AOTX_MODEL_ABSENT, AOTX_MODEL_LANGUAGE,
               AOTX_ROPE_PAIRS_ADJACENT, AOTX_WEIGHT_F32, AOTX_WEIGHT_Q8_0, SLOT, KvMap,
               ModelDesc, ModelRun, check, lib, neutral_how,
               AOTX_MODEL_ROWS_LAST)

GOLD = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
ALIGN = 256


def splitmix(seed, n):
    """splitmix64 output n of `seed` (vectorised over n)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (n.astype(np.uint64) + np.uint64(1)) * GOLD
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def normal(seed, start, count):
    """Values start..start+count of the integer normal generator (synth.h)."""
    i = np.arange(start, start + count, dtype=np.uint64)
    total = np.zeros(count, dtype=np.int64)
    mask = np.uint64(0xFFFF)
    for j in range(3):
        r = splitmix(seed, np.uint64(3) * i + np.uint64(j))
        for sh in (0, 16, 32, 48):
            total += ((r >> np.uint64(sh)) & mask).astype(np.int64)
    return (total - 393210).astype(np.float32) * np.float32(1.0 / 65536.0)


def quantize_q8(w):
    """float32 [rows][k] -> Q8_0 bytes [rows][k/32*34] (d = max|w|/127, q = rint(w/d))."""
    rows, k = w.shape
    blocks = w.reshape(rows, k // 32, 32).astype(np.float32)
    amax = np.abs(blocks).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    safe = np.where(d == 0, np.float32(1.0), d)
    q = np.where(d[..., None] == 0, np.float32(0.0), np.rint(blocks / safe[..., None]))
    q = np.clip(q, -127, 127).astype(np.int8)
    out = np.empty((rows, k // 32, 34), dtype=np.uint8)
    out[:, :, :2] = d.astype(np.float16).view(np.uint8).reshape(rows, k // 32, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(rows, (k // 32) * 34)


def synth_q8(rows, k, sigma, seed, valid_rows=None, valid_cols=None):
    """Q8_0 tensor of N(0, sigma) values; entries outside valid_rows x valid_cols are 0."""
    w = normal(seed, 0, rows * k).reshape(rows, k) * np.float32(sigma)
    if valid_rows is not None and valid_rows < rows:
        w[valid_rows:, :] = 0
    if valid_cols is not None and valid_cols < k:
        w[:, valid_cols:] = 0
    return quantize_q8(w)


def dequant_q8(q, k):
    """Q8_0 bytes [rows][k/32*34] -> half(q*scale) as float32 [rows][k]."""
    rows = q.shape[0]
    blk = q.reshape(rows, k // 32, 34)
    sc = blk[:, :, :2].copy().view(np.float16).astype(np.float32)
    qq = blk[:, :, 2:].copy().view(np.int8).astype(np.float32)
    return (qq * sc).astype(np.float16).astype(np.float32).reshape(rows, k)


@dataclass
class Shape:
    layers: int
    hidden: int
    ffn: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-5
    theta: float = 10000.0
    ffn_valid: int = 0          # logical FFN width before zero padding (0 = ffn)
    experts: int = 0
    used: int = 0
    tied: bool = False
    qk_norm: bool = False
    pairs: int = AOTX_ROPE_PAIRS_ADJACENT
    sigma: float = 0.02
    cls: bool = False           # a two-row class head (cls_output) for the rank role

    def q8_bytes(self, rows, k):
        return rows * (k // 32) * 34


TINY = Shape(layers=4, hidden=256, ffn=704, ffn_valid=688, heads=4, kv_heads=4, head_dim=64,
             vocab=4096)
LLAMA_8B = Shape(layers=32, hidden=4096, ffn=14336, heads=32, kv_heads=8, head_dim=128,
                 vocab=128256)
MIXTRAL = Shape(layers=32, hidden=4096, ffn=14336, heads=32, kv_heads=8, head_dim=128,
                vocab=32000, experts=8, used=2, theta=1e6)


def layout_pages(context, layers, kv_heads, head_dim, page_bytes=2 * 1024 * 1024, header=256,
                 block=16):
    """Pages one slot needs for `context` positions (cuda/model/kv_layout.cuh:94-103)."""
    block_bytes = 2 * kv_heads * block * head_dim * 2
    per_page = (page_bytes - header) // block_bytes
    if per_page == 0:
        return 0
    blocks = ((context + block - 1) // block) * layers
    return (blocks + per_page - 1) // per_page


def _align(n):
    return (n + ALIGN - 1) // ALIGN * ALIGN


@dataclass
class Layout:
    desc: ModelDesc
    total: int
    tensors: list = field(default_factory=list)   # (offset, kind, rows, k, seed, extra)


def layout(shape: Shape, seed=0x5EED):
    """Place every tensor of the model; return the descriptor and the tensor list."""
    d = ModelDesc()
    d.role = AOTX_MODEL_LANGUAGE
    d.layers = shape.layers
    d.hidden = shape.hidden
    d.ffn = shape.ffn
    d.heads = shape.heads
    d.kv_heads = shape.kv_heads
    d.head_dim = shape.head_dim
    d.vocab = shape.vocab
    d.context = 8192
    d.weight_type = AOTX_WEIGHT_Q8_0
    d.embd_type = AOTX_WEIGHT_Q8_0
    d.tied_output = 1 if shape.tied else 0
    d.rope_theta = shape.theta
    d.rms_eps = shape.eps
    d.rope_pairs = shape.pairs
    d.expert_count = shape.experts
    d.expert_used_count = shape.used
    d.cls_output = AOTX_MODEL_ABSENT
    d.rope_freqs = AOTX_MODEL_ABSENT
    d.output = AOTX_MODEL_ABSENT
    for l in range(64):
        for s in range(14):
            d.layer[l].offset[s] = AOTX_MODEL_ABSENT
            d.layer_type[l][s] = AOTX_WEIGHT_F32
    tensors = []
    cursor = 0
    counter = [0]

    def place(kind, rows, k, extra=None):
        nonlocal cursor
        at = _align(cursor)
        if kind == "q8":
            size = shape.q8_bytes(rows, k)
        else:
            size = rows * k * 4
        counter[0] += 1
        tensors.append((at, kind, rows, k, (seed * 1000003 + counter[0]) & (2 ** 64 - 1), extra))
        cursor = at + size
        return at

    h, f = shape.hidden, shape.ffn
    wide, narrow = shape.heads * shape.head_dim, shape.kv_heads * shape.head_dim
    fv = shape.ffn_valid or f
    d.token_embd = place("q8", shape.vocab, h)
    d.output_norm = place("ones", 1, h)
    if not shape.tied:
        d.output = place("q8", shape.vocab, h)
    for l in range(shape.layers):
        L = d.layer[l]
        expert = shape.experts > 0
        d.kind[l] = (AOTX_LAYER_KIND_FFN_EXPERTS if expert else
                     AOTX_LAYER_KIND_ATTENTION if shape.qk_norm else
                     AOTX_LAYER_KIND_ATTENTION_NO_QK_NORM)
        L.offset[SLOT["attn_norm"]] = place("ones", 1, h)
        L.offset[SLOT["attn_q"]] = place("q8", wide, h)
        L.offset[SLOT["attn_k"]] = place("q8", narrow, h)
        L.offset[SLOT["attn_v"]] = place("q8", narrow, h)
        L.offset[SLOT["attn_o"]] = place("q8", h, wide)
        if shape.qk_norm:
            L.offset[SLOT["q_norm"]] = place("ones", 1, shape.head_dim)
            L.offset[SLOT["k_norm"]] = place("ones", 1, shape.head_dim)
        L.offset[SLOT["ffn_norm"]] = place("ones", 1, h)
        e = max(1, shape.experts)
        L.offset[SLOT["ffn_gate"]] = place("q8", e * f, h, ("rows", fv, f))
        L.offset[SLOT["ffn_up"]] = place("q8", e * f, h, ("rows", fv, f))
        L.offset[SLOT["ffn_down"]] = place("q8", e * h, f, ("cols", fv))
        if expert:
            L.offset[SLOT["router"]] = place("router", shape.experts, h)
        for s in ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_gate", "ffn_up", "ffn_down"):
            d.layer_type[l][SLOT[s]] = AOTX_WEIGHT_Q8_0
    if shape.cls:
        d.cls_output = place("q8", 2, h)
    return Layout(desc=d, total=_align(cursor), tensors=tensors)


def _host_tensor(shape, kind, rows, k, tseed, extra):
    if kind == "ones":
        return np.ones(rows * k, dtype=np.float32).view(np.uint8)
    if kind == "router":
        return (normal(tseed, 0, rows * k) * np.float32(shape.sigma)).astype(np.float32).view(np.uint8)
    if extra is not None and extra[0] == "rows":
        fv, f = extra[1], extra[2]
        w = normal(tseed, 0, rows * k).reshape(rows, k) * np.float32(shape.sigma)
        if fv < f:
            w.reshape(-1, f, k)[:, fv:, :] = 0
        return quantize_q8(w).reshape(-1)
    if extra is not None and extra[0] == "cols":
        fv = extra[1]
        w = normal(tseed, 0, rows * k).reshape(rows, k) * np.float32(shape.sigma)
        if fv < k:
            w[:, fv:] = 0
        return quantize_q8(w).reshape(-1)
    return quantize_q8(normal(tseed, 0, rows * k).reshape(rows, k) * np.float32(shape.sigma)).reshape(-1)


def build_host(shape, seed=0x5EED):
    """The whole weights region on the host (numpy uint8) + layout. Small shapes only."""
    lay = layout(shape, seed)
    region = np.zeros(lay.total, dtype=np.uint8)
    for at, kind, rows, k, tseed, extra in lay.tensors:
        data = _host_tensor(shape, kind, rows, k, tseed, extra)
        region[at:at + data.size] = data
    return region, lay


def build_device(shape, seed=0x5EED, device="cuda"):
    """The weights region built directly in device memory (any shape), + layout.

    Q8 tensors without padding come from aotx_synth_q8 on the GPU (the same bytes
    build_host would write for them); padded and fp32 tensors are made on the host."""
    import torch
    lay = layout(shape, seed)
    region = torch.zeros(lay.total, dtype=torch.uint8, device=device)
    L = lib()
    base = region.data_ptr()
    for at, kind, rows, k, tseed, extra in lay.tensors:
        padded = extra is not None and ((extra[0] == "rows" and extra[1] < extra[2]) or
                                        (extra[0] == "cols" and extra[1] < k))
        if kind == "q8" and not padded:
            check(L.aotx_synth_q8(ctypes.c_void_p(base + at), rows, k, shape.sigma, tseed, None),
                  "aotx_synth_q8")
        else:
            data = _host_tensor(shape, kind, rows, k, tseed, extra)
            region[at:at + data.size].copy_(torch.from_numpy(data))
    torch.cuda.synchronize()
    return region, lay


class Runtime:
    """The model-step surface over one role, as the reference's callers drive it."""

    def __init__(self, region, desc, max_tokens=32, pool_pages=1024, role=AOTX_MODEL_LANGUAGE):
        import torch
        self.torch = torch
        self.L = lib()
        self.role = role
        self.region = region
        self.desc = desc
        check(self.L.aotx_mem_weights_set(region.data_ptr(), region.numel()), "weights")
        check(self.L.aotx_model_set_desc(role, ctypes.byref(desc)), "aotx_model_set_desc")
        check(self.L.aotx_model_open(role, max_tokens), "aotx_model_open")
        self.map = KvMap()
        self.map.limit = pool_pages
        check(self.L.aotx_kv_open(ctypes.byref(self.map)), "aotx_kv_open")
        self.L.aotx_model_forget()
        self.L.aotx_model_restream()
        self.dev = region.device

    def close(self):
        self.L.aotx_model_shut(self.role)
        self.L.aotx_kv_close(ctypes.byref(self.map))

    def _batch(self, ids, offset, agent):
        t = self.torch
        return (t.tensor(np.asarray(ids, dtype=np.int32), device=self.dev),
                t.tensor(np.asarray(offset, dtype=np.uint32).view(np.int32), device=self.dev),
                t.tensor(np.asarray(agent, dtype=np.uint32).view(np.int32), device=self.dev))

    def pages(self, offset_d, agent_d, seqs):
        check(self.L.aotx_model_pages(self.role, offset_d.data_ptr(), seqs, agent_d.data_ptr()),
              "aotx_model_pages")
        self.L.aotx_kv_serve(ctypes.byref(self.map), None)

    def sample(self, ids, offset, agent, how=None):
        """One pass; returns (tokens, draws) as numpy arrays."""
        t = self.torch
        ids_d, off_d, ag_d = self._batch(ids, offset, agent)
        seqs = len(agent)
        self.pages(off_d, ag_d, seqs)
        tok = t.zeros(seqs, dtype=t.int32, device=self.dev)
        draw = t.zeros(seqs, dtype=t.int32, device=self.dev)
        how = how or neutral_how()
        seed = ctypes.c_uint64()
        check(self.L.aotx_model_sample(self.role, ids_d.data_ptr(), off_d.data_ptr(), seqs,
                                       ag_d.data_ptr(), ctypes.byref(how), tok.data_ptr(),
                                       draw.data_ptr(), ctypes.byref(seed)), "aotx_model_sample")
        return tok.cpu().numpy(), draw.cpu().numpy().view(np.uint32)

    def step(self, ids, offset, agent, how=None):
        """One pass through aotx_model_launch with the call block aotx_model_sample builds
        (call_host.cu:71-93), plus the logits of each sequence's last row.
        Returns (tokens, draws, logits [seqs][vocab])."""
        t = self.torch
        ids_d, off_d, ag_d = self._batch(ids, offset, agent)
        seqs = len(agent)
        self.pages(off_d, ag_d, seqs)
        tok = t.zeros(seqs, dtype=t.int32, device=self.dev)
        draw = t.zeros(seqs, dtype=t.int32, device=self.dev)
        logits = t.zeros((seqs, self.desc.vocab), dtype=t.float32, device=self.dev)
        how = how or neutral_how()
        run = ModelRun()
        run.ids = ids_d.data_ptr()
        run.offset = off_d.data_ptr()
        run.agent = ag_d.data_ptr()
        run.logits = logits.data_ptr()
        run.token = tok.data_ptr()
        run.draw = draw.data_ptr()
        run.seed = how.seed
        run.seqs = seqs
        run.tokens = int(offset[-1])
        run.rows = seqs
        run.select = AOTX_MODEL_ROWS_LAST
        run.top_k = how.top_k
        run.top_p = how.top_p
        run.temperature = how.temperature
        check(self.L.aotx_model_launch(self.role, ctypes.byref(run)), "aotx_model_launch")
        return tok.cpu().numpy(), draw.cpu().numpy().view(np.uint32), logits.cpu().numpy()

    def prefill_logits(self, ids, offset, agent):
        """Prefill that returns the logits of every token (aotx_model_prefill)."""
        t = self.torch
        ids_d, off_d, ag_d = self._batch(ids, offset, agent)
        seqs = len(agent)
        self.pages(off_d, ag_d, seqs)
        n = len(ids)
        logits = t.zeros((n, self.desc.vocab), dtype=t.float32, device=self.dev)
        check(self.L.aotx_model_prefill(self.role, ids_d.data_ptr(), off_d.data_ptr(), seqs,
                                        ag_d.data_ptr(), logits.data_ptr(), None),
              "aotx_model_prefill")
        return logits.cpu().numpy()

    def probe(self, ids, offset, agent, layers, how=None):
        """aotx_model_probe with the logits of each sequence's last row and the residual
        capture of `layers`. Returns (logits [seqs][vocab], capture [len(layers)][seqs][hidden])."""
        t = self.torch
        ids_d, off_d, ag_d = self._batch(ids, offset, agent)
        seqs = len(agent)
        self.pages(off_d, ag_d, seqs)
        logits = t.zeros((seqs, self.desc.vocab), dtype=t.float32, device=self.dev)
        cap = t.full((max(1, len(layers)), seqs, self.desc.hidden), float("nan"),
                     dtype=t.float32, device=self.dev)
        lay_d = t.tensor(np.asarray(layers if layers else [0], dtype=np.uint32).view(np.int32),
                         device=self.dev)
        hows = how or [neutral_how() for _ in range(seqs)]
        how_d = t.tensor(np.frombuffer(b"".join(bytes(h) for h in hows), dtype=np.uint8),
                         device=self.dev)
        check(self.L.aotx_model_probe(self.role, ids_d.data_ptr(), off_d.data_ptr(), seqs,
                                      ag_d.data_ptr(), how_d.data_ptr(), logits.data_ptr(),
                                      AOTX_MODEL_ROWS_LAST, cap.data_ptr(), lay_d.data_ptr(),
                                      len(layers)), "aotx_model_probe")
        return logits.cpu().numpy(), cap.cpu().numpy()[:len(layers)]

    def pooled(self, ids, offset, agent):
        """aotx_model_prefill with a pooled buffer and no logits: [seqs][hidden]."""
        t = self.torch
        ids_d, off_d, ag_d = self._batch(ids, offset, agent)
        seqs = len(agent)
        self.pages(off_d, ag_d, seqs)
        out = t.full((seqs, self.desc.hidden), float("nan"), dtype=t.float32, device=self.dev)
        check(self.L.aotx_model_prefill(self.role, ids_d.data_ptr(), off_d.data_ptr(), seqs,
                                        ag_d.data_ptr(), None, out.data_ptr()),
              "aotx_model_prefill")
        return out.cpu().numpy()

    def rerank(self, ids, offset, agent):
        """aotx_model_rerank (the rank role): one score per sequence."""
        t = self.torch
        ids_d, off_d, ag_d = self._batch(ids, offset, agent)
        seqs = len(agent)
        self.pages(off_d, ag_d, seqs)
        out = t.full((seqs,), float("nan"), dtype=t.float32, device=self.dev)
        check(self.L.aotx_model_rerank(ids_d.data_ptr(), off_d.data_ptr(), seqs, ag_d.data_ptr(),
                                       out.data_ptr()), "aotx_model_rerank")
        return out.cpu().numpy()

    def faulted(self):
        return self.L.aotx_model_faulted()
