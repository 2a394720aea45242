#!/usr/bin/env python3
"""Benchmark of the MI355X token loop (BASELINE.json metric: decode tokens/s at batch 1
and 32 on the 8B-shape Q8 decoder; Q8 GEMV achieved HBM GB/s).

Workload: 32 layers, d_model 4096, 32/8 heads x 128, FFN 14336
SwiGLU, vocab 128256, untied head, every linear Q8_0 from N(0, 0.02) (synthetic weights
generated on the GPU). 32 agent slots each seated on a 2048-token paged KV cache (the
pages are requested through the pool, written with random fp16 keys/values, and the
slots' cache positions set), then greedy decode steps through the drop-in operator
surface: aotx_model_pages -> aotx_kv_serve -> aotx_model_sample, one step = one token for
every slot. `value` is the batch-32 whole-step throughput in tokens/s; the batch-1 rate,
the sampled (top-k 40 / top-p 0.9 / T 0.8) rate and the Q8 GEMV table ride along.

`roofline` is measured on the dominant kernel of the batch step, paged decode attention
(aotx_attend_paged) over the seated 32 x 2048-position KV of the timed workload: a HIP graph
of 20 launches replayed on its own stream, timed with HIP events recorded on that stream.
Its algorithmic bytes are the keys and values of every attended position plus q and out.
The Q8 products of the step are reported the same way under `kernels`. `cpu_baseline` times
the repository's C oracle (oracle/) on the host cores over a bounded sample of the same
decode step.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 matrix-core peak
CONFIG4_STEPS = 128           # 128 decode steps from a 2048-token cache
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "attention_b32_ctx2048_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the roofline kernel from the committed counter passes
    (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None when absent."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def step_bytes(lay, shape, batch, ctx_mean):
    """Algorithmic HBM bytes of one decode step: every weight the step reads once (all layer
    matrices, the head, the norm vectors, the routers; every expert of a routed layer, which
    a batch of 64 tokens touches with probability 1 - 1e-8), the B embedding rows (not the
    table), the keys and values of every attended position and the new position of every
    layer, and the logits written and read once."""
    d = lay.desc
    weights = 0
    for at, kind, rows, k, _, _ in lay.tensors:
        if at == d.token_embd:
            continue
        weights += rows * (k // 32) * 34 if kind == "q8" else rows * k * 4
    emb = batch * (shape.hidden // 32) * 34
    kv_tok = 2 * shape.kv_heads * shape.head_dim * 2 * shape.layers
    return weights + emb + batch * (ctx_mean * kv_tok + kv_tok + shape.vocab * 8)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_table(torch, L, shapes, ms, iters=20):
    """Per-launch device time (graph-timed) and achieved GB/s of the Q8_0 product (fp16 out,
    config 2), for the file-layout entry point (aotx_q8_gemv_f16) and for the repacked form
    the decode step streams (aotx_q8r_gemv_f16)."""
    import aotx_amd as A
    out = []
    for n, k in shapes:
        w = torch.empty(n * (k // 32) * 34, dtype=torch.uint8, device="cuda")
        A.check(L.aotx_synth_q8(A.ptr(w), n, k, 0.02, 7, None), "synth")
        # enough copies that consecutive launches stream from HBM, not from the 256 MB
        # last-level cache (each copy read once per pass through them)
        rsize = L.aotx_q8r_size(n, k)
        copies = max(1, min(iters, (640 << 20) // rsize + 1))
        wrs = []
        for _ in range(copies):
            wr = torch.empty(rsize, dtype=torch.uint8, device="cuda")
            A.check(L.aotx_q8_repack(A.ptr(w), n, k, A.ptr(wr), None), "repack")
            wrs.append(wr)
        fsize = w.numel()
        fcopies = max(1, min(iters, (640 << 20) // fsize + 1))
        ws = [w] + [w.clone() for _ in range(fcopies - 1)]
        for m in ms:
            x = torch.randn(m, k, device="cuda").half()
            y = torch.empty(m, n, device="cuda", dtype=torch.float16)
            row = {"n": n, "k": k, "m": m}
            for name, fn, tens in (("file", L.aotx_q8_gemv_f16, ws), ("repacked", L.aotx_q8r_gemv_f16, wrs)):
                turn = [0]

                def launch(st, fn=fn, tens=tens):
                    wt = tens[turn[0] % len(tens)]
                    turn[0] += 1
                    A.check(fn(A.ptr(wt), n, k, A.ptr(x), m, A.ptr(y),
                               ctypes.c_void_p(st.cuda_stream)), "q8 product")
                us = graph_time(torch, launch, reps=iters)
                algo = n * k * 34 // 32 + m * k * 2 + m * n * 2
                row[name + "_us"] = round(us, 2)
                row[name + "_gbs"] = round(algo / us / 1e3, 1)
                row["bytes"] = algo
            out.append(row)
        del w, ws, wrs
    return out


def graph_time(torch, launch, reps=20, replays=5):
    """Average device time (us) of one `launch(stream)`: `reps` launches captured in a HIP
    graph on a side stream, replayed `replays` times between HIP events on that stream."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for _ in range(3):
            launch(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(reps):
            launch(s)
    with torch.cuda.stream(s):
        g.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(replays):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / (reps * replays)


def attention_rate(torch, L, slots, context, heads, kvh, hd, layers):
    """The step's attention over the seated pages (every slot at its last seated position,
    the layers in turn): (us per launch, algorithmic bytes per launch)."""
    import aotx_amd as A
    B = len(slots)
    q = torch.randn(B, heads, hd, device="cuda").half()
    out = torch.empty_like(q)
    pos = torch.full((B,), context - 1, dtype=torch.int32, device="cuda")
    ag = torch.tensor(slots, dtype=torch.int32, device="cuda")

    turn = [0]

    def launch(s):
        # a different layer each launch: 32 x 268 MB of keys and values, so no launch finds
        # the previous one's in the 256 MB last-level cache
        layer = turn[0] % layers
        turn[0] += 1
        A.check(L.aotx_attend_paged(A.ptr(q), A.ptr(pos), A.ptr(ag), B, heads, kvh, hd, layer,
                                    layers, A.ptr(out), ctypes.c_void_p(s.cuda_stream)),
                "aotx_attend_paged")

    us = graph_time(torch, launch)
    algo = B * context * kvh * hd * 2 * 2 + 2 * q.numel() * 2
    return us, algo


def attention_ragged(torch, L, batch=32, lo=512, hi=8192, heads=32, kvh=8, hd=128, layers=4,
                     seed=3):
    """paged decode attention over `batch` sequences with context lengths
    uniform in [lo, hi] (seeded), fp16 N(0, 1) keys/values, one query token per sequence at
    its last position. Pages are handed out one at a time to the sequences in a seeded random
    order, so a sequence's pages are a random selection of the pool's physical pages. The KV
    layout holds `layers` layers (the launches rotate over them, so no launch finds the
    previous one's bytes in the last-level cache). Returns (us per launch, algorithmic bytes
    per launch, the context lengths)."""
    import numpy as np
    import aotx_amd as A
    from aotx_amd.model import layout_pages
    rng = np.random.default_rng(seed)
    ctx = rng.integers(lo, hi + 1, batch)
    need = [layout_pages(int(c) + 1, layers, kvh, hd) for c in ctx]
    kvm = A.KvMap()
    kvm.limit = int(sum(need)) + 8
    A.check(L.aotx_kv_open(ctypes.byref(kvm)), "aotx_kv_open")
    try:
        order = np.repeat(np.arange(batch), need)
        rng.shuffle(order)
        for i, sl in enumerate(order):
            if L.aotx_kv_request(int(sl), 1) != 1:
                raise RuntimeError("page request refused")
            if i % 64 == 63:
                L.aotx_kv_serve(ctypes.byref(kvm), None)
        L.aotx_kv_serve(ctypes.byref(kvm), None)
        n = int(ctx.sum())
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        pos = torch.cat([torch.arange(int(c), dtype=torch.int32) for c in ctx]).cuda()
        ag = torch.cat([torch.full((int(c),), i, dtype=torch.int32)
                        for i, c in enumerate(ctx)]).cuda()
        for layer in range(layers):
            k = torch.randn(n, kvh * hd, device="cuda", generator=g).half()
            v = torch.randn(n, kvh * hd, device="cuda", generator=g).half()
            A.check(L.aotx_kv_write(A.ptr(k), A.ptr(v), A.ptr(pos), A.ptr(ag), n, kvh, hd, layer,
                                    layers, None), "aotx_kv_write")
            del k, v
        torch.cuda.synchronize()
        q = torch.randn(batch, heads, hd, device="cuda", generator=g).half()
        out = torch.empty_like(q)
        qpos = torch.tensor([int(c) - 1 for c in ctx], dtype=torch.int32, device="cuda")
        qag = torch.arange(batch, dtype=torch.int32, device="cuda")
        turn = [0]

        def launch(st):
            layer = turn[0] % layers
            turn[0] += 1
            A.check(L.aotx_attend_paged(A.ptr(q), A.ptr(qpos), A.ptr(qag), batch, heads, kvh, hd,
                                        layer, layers, A.ptr(out), ctypes.c_void_p(st.cuda_stream)),
                    "aotx_attend_paged")

        us = graph_time(torch, launch)
        algo = n * kvh * hd * 2 * 2 + 2 * q.numel() * 2
    finally:
        L.aotx_kv_close(ctypes.byref(kvm))
    return us, algo, ctx


def seat_context(torch, rt, slots, context, reserve, layers, kvh, hd):
    """Request pages for `context + reserve` positions per slot, write random fp16 K/V for
    positions [0, context) of every layer, and seat each slot at `context`."""
    import aotx_amd as A
    from aotx_amd.model import layout_pages
    L = rt.L
    for s in slots:
        need = layout_pages(context + reserve, layers, kvh, hd)
        if L.aotx_kv_request(s, need) != 1:
            raise RuntimeError("page request refused")
    L.aotx_kv_serve(ctypes.byref(rt.map), None)
    n = len(slots) * context
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    k = torch.randn(n, kvh * hd, device="cuda", generator=g).half()
    v = torch.randn(n, kvh * hd, device="cuda", generator=g).half()
    pos = torch.arange(context, device="cuda", dtype=torch.int32).repeat(len(slots))
    ag = torch.tensor(slots, device="cuda", dtype=torch.int32).repeat_interleave(context)
    for layer in range(layers):
        A.check(L.aotx_kv_write(A.ptr(k), A.ptr(v), A.ptr(pos), A.ptr(ag), n, kvh, hd, layer,
                                layers, None), "aotx_kv_write")
    torch.cuda.synchronize()
    for s in slots:
        A.check(L.aotx_model_seat(s, context), "aotx_model_seat")
    del k, v


def decode(torch, rt, slots, steps, warmup, how):
    """Timed decode steps through the operator surface; returns (tokens/s, ms/step)."""
    import aotx_amd as A
    L = rt.L
    B = len(slots)
    off = torch.arange(B + 1, device="cuda", dtype=torch.int32)
    ag = torch.tensor(slots, device="cuda", dtype=torch.int32)
    ids = torch.randint(0, rt.desc.vocab, (B,), device="cuda", dtype=torch.int32)
    tok = torch.zeros(B, device="cuda", dtype=torch.int32)
    draw = torch.zeros(B, device="cuda", dtype=torch.int32)
    seed = ctypes.c_uint64()

    def one():
        nonlocal ids, tok
        A.check(L.aotx_model_pages(rt.role, A.ptr(off), B, A.ptr(ag)), "pages")
        L.aotx_kv_serve(ctypes.byref(rt.map), None)
        A.check(L.aotx_model_sample(rt.role, A.ptr(ids), A.ptr(off), B, A.ptr(ag),
                                    ctypes.byref(how), A.ptr(tok), A.ptr(draw),
                                    ctypes.byref(seed)), "aotx_model_sample")
        ids, tok = tok, ids

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    if L.aotx_model_faulted() != 0:
        raise RuntimeError("page faults during the timed decode")
    return B * steps / dt, dt * 1000.0 / steps


def cpu_baseline(region_dev, lay, torch, batch, context, threads):
    """The C oracle's decode step on the host cores (a bounded sample: one step of the
    batch on a seated context)."""
    from oracle import oracle as orc
    host = region_dev.cpu().numpy()
    m = orc.Model(lay.desc, host, slots=batch, max_context=context + 2, threads=threads)
    m.seat(list(range(batch)), context, seed=7)
    ids = np.random.default_rng(0).integers(0, lay.desc.vocab, batch).astype(np.int32)
    offset = np.arange(batch + 1, dtype=np.uint32)
    agent = np.arange(batch, dtype=np.uint32)
    t0 = time.perf_counter()
    m.step(ids, offset, agent)
    dt = time.perf_counter() - t0
    return batch / dt, dt


def traffic_run(args):
    """Counter pass workload (`--traffic`): the roofline kernel alone on the same seated
    KV (32 slots x 2048 positions, 32 layers' layout, layer 0 attended), five launches, then
    five plain device copies of 256 MiB (the calibration of FETCH_SIZE / WRITE_SIZE per
    dispatch). No model weights are built."""
    import torch
    import aotx_amd as A
    from aotx_amd.model import LLAMA_8B, layout_pages
    L = A.lib()
    shape = LLAMA_8B
    slots = list(range(args.batch))
    kvm = A.KvMap()
    per = layout_pages(args.context + 8, shape.layers, shape.kv_heads, shape.head_dim)
    kvm.limit = per * len(slots) + 8
    A.check(L.aotx_kv_open(ctypes.byref(kvm)), "aotx_kv_open")
    for sl in slots:
        if L.aotx_kv_request(sl, per) != 1:
            raise RuntimeError("page request refused")
    L.aotx_kv_serve(ctypes.byref(kvm), None)
    n = len(slots) * args.context
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    k = torch.randn(n, shape.kv_heads * shape.head_dim, device="cuda", generator=g).half()
    v = torch.randn(n, shape.kv_heads * shape.head_dim, device="cuda", generator=g).half()
    pos = torch.arange(args.context, device="cuda", dtype=torch.int32).repeat(len(slots))
    ag = torch.tensor(slots, device="cuda", dtype=torch.int32).repeat_interleave(args.context)
    A.check(L.aotx_kv_write(A.ptr(k), A.ptr(v), A.ptr(pos), A.ptr(ag), n, shape.kv_heads,
                            shape.head_dim, 0, shape.layers, None), "aotx_kv_write")
    del k, v, pos, ag
    B = len(slots)
    q = torch.randn(B, shape.heads, shape.head_dim, device="cuda").half()
    out = torch.empty_like(q)
    qpos = torch.full((B,), args.context - 1, dtype=torch.int32, device="cuda")
    qag = torch.tensor(slots, dtype=torch.int32, device="cuda")
    for _ in range(5):
        A.check(L.aotx_attend_paged(A.ptr(q), A.ptr(qpos), A.ptr(qag), B, shape.heads,
                                    shape.kv_heads, shape.head_dim, 0, shape.layers,
                                    A.ptr(out), None), "aotx_attend_paged")
    torch.cuda.synchronize()
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    L.aotx_kv_close(ctypes.byref(kvm))
    algo = B * args.context * shape.kv_heads * shape.head_dim * 4 + 2 * q.numel() * 2
    print(json.dumps({"traffic_workload": "attention", "algorithmic_bytes": algo,
                      "copy_bytes": src.numel()}))


def moe_measure(torch, steps, warmup):
    """Mixtral-shape routed-expert decoder (32 layers, d_model 4096, 8
    experts of FFN 14336, top-2, vocab 32000), 64 slots at 4096-token paged KV, one token
    per slot per step, greedy. Returns tokens/s and the step's fraction of the HBM roofline
    (every expert is touched at 128 routed rows per layer)."""
    import aotx_amd as A
    from aotx_amd.model import MIXTRAL, Runtime, build_device, layout_pages
    shape, batch, context = MIXTRAL, 64, 4096
    t0 = time.perf_counter()
    region, lay = build_device(shape, seed=0x5EED)
    log(f"moe: weights {region.numel() / 1e9:.2f} GB built in {time.perf_counter() - t0:.1f}s")
    reserve = warmup * 3 + steps * 3 + 8
    per_slot = layout_pages(context + reserve, shape.layers, shape.kv_heads, shape.head_dim)
    slots = list(range(batch))
    rt = Runtime(region, lay.desc, max_tokens=batch, pool_pages=per_slot * batch + 8)
    seat_context(torch, rt, slots, context, reserve, shape.layers, shape.kv_heads, shape.head_dim)
    log(f"moe: seated {batch} x {context} in {time.perf_counter() - t0:.1f}s")
    tps, ms = decode(torch, rt, slots, steps, warmup, A.neutral_how())
    rt.close()
    del region
    torch.cuda.empty_cache()
    # attended positions per token, averaged over the timed steps (pos + 1)
    ctx_mean = context + warmup + (steps + 1) / 2.0
    sb = step_bytes(lay, shape, batch, ctx_mean)
    return {"metric": "Mixtral-shape MoE decode tokens/s (BASELINE config 5)",
            "value": round(tps, 2), "unit": "tokens/s", "ms_per_step": round(ms, 4),
            "steps": steps, "warmup": warmup, "batch": batch, "context": context,
            "step_gb": round(sb / 1e9, 3),
            "step_roofline_frac": round(sb / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
            "data": "synthetic (seeded N(0,0.02) Q8_0 weights; random fp16 KV; greedy ids)"}


def moe_run(args):
    """`--moe`: BASELINE config 5 alone; prints one JSON line."""
    import torch
    torch.cuda.init()
    print(json.dumps(moe_measure(torch, args.steps, args.warmup)))


def prefill_flops(shape, t):
    """Matrix-core work of one t-token prompt chunk: every dense product over t rows (the
    head over the chunk's last row) plus the causal attention's two products."""
    h, f = shape.hidden, shape.ffn
    wide, narrow = shape.heads * shape.head_dim, shape.kv_heads * shape.head_dim
    per_layer = h * (wide + 2 * narrow) + wide * h + 3 * f * h
    dense = 2.0 * t * per_layer * shape.layers + 2.0 * shape.vocab * h
    attn = 2.0 * 2.0 * shape.head_dim * shape.heads * shape.layers * t * (t + 1) / 2.0
    return dense + attn


def prefill_measure(torch, region, lay, shape, sizes, reps=6):
    """One prompt chunk of each size in `sizes` (a fresh slot each time) through
    aotx_model_launch, the whole step; best of reps - 1 after a warm-up."""
    from aotx_amd.model import Runtime, layout_pages
    per = layout_pages(max(sizes) + 16, shape.layers, shape.kv_heads, shape.head_dim)
    rt = Runtime(region, lay.desc, max_tokens=max(sizes), pool_pages=per * (reps * len(sizes) + 2) + 8)
    rng = np.random.default_rng(0)
    out, slot = {}, 0
    for t in sizes:
        times = []
        for _ in range(reps):
            ids = rng.integers(0, shape.vocab, t).tolist()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            rt.step(ids, [0, t], [slot])
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
            slot += 1
        best = min(times[1:])
        fl = prefill_flops(shape, t)
        out[str(t)] = {"ms": round(best * 1e3, 3), "tokens_per_s": round(t / best, 1),
                       "tflops": round(fl / best / 1e12, 1),
                       "mfma_frac_fp16": round(fl / best / (MFMA_PEAK_FP16_TFLOPS * 1e12), 4)}
    rt.close()
    return out


def prefill_run(args):
    """`--prefill`: one prompt chunk of 128, 256 and 512 tokens of the 8B shape. Prints one
    JSON line."""
    import torch
    from aotx_amd.model import LLAMA_8B, build_device
    torch.cuda.init()
    region, lay = build_device(LLAMA_8B, seed=7)
    out = prefill_measure(torch, region, lay, LLAMA_8B, (128, 256, 512))
    print(json.dumps({"metric": "prefill tokens/s (8B shape, one prompt chunk)", "chunks": out}))


def _text_corpus(seed, lines, words=60):
    """Seeded synthetic text: words from a few scripts, numbers, punctuation, spaces."""
    rng = np.random.default_rng(seed)
    vocab = ["hello", "world", "it's", "the", "café", "naïve", "данные", "中文", "αβγ", "12345",
             "don't", "code", "x", "::", "...", "(", ")", "\n", "  ", "😀"]
    out = []
    for _ in range(lines):
        picks = rng.integers(0, len(vocab), words)
        out.append(" ".join(vocab[i] for i in picks))
    return out


def text_run(args):
    """`--text`: the tokenizer (llama3 split, whole rule) on a vocabulary the `tokenizers`
    library trains on a seeded synthetic corpus: GPU encode and decode throughput over 4096
    texts (~1.2 MB; synchronous calls, best of 5), the CPU oracle's encode on a bounded
    sample beside it. Prints one JSON line."""
    import ctypes
    import torch
    from tokenizers import Tokenizer as HF, models, pre_tokenizers, trainers
    from aotx_amd.text import Tokenizer
    torch.cuda.init()
    hf = HF(models.BPE())
    hf.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    hf.train_from_iterator(_text_corpus(1, 300), trainers.BpeTrainer(
        vocab_size=2000, show_progress=False, initial_alphabet=pre_tokenizers.ByteLevel.alphabet()))
    model = json.loads(hf.to_str())["model"]
    tokens = [None] * len(model["vocab"])
    for tok, i in model["vocab"].items():
        tokens[i] = tok
    merges = [m if isinstance(m, str) else f"{m[0]} {m[1]}" for m in model["merges"]]
    tk = Tokenizer(tokens=tokens, merges=merges, family="llama3")
    texts = _text_corpus(2, 4096)
    raw = [t.encode() for t in texts]
    nbytes = sum(len(r) for r in raw)
    at = np.zeros(len(raw) + 1, dtype=np.uint64)
    at[1:] = np.cumsum([len(r) for r in raw])
    bytes_d = torch.from_numpy(np.frombuffer(b"".join(raw), dtype=np.uint8).copy()).cuda()
    at_d = torch.from_numpy(at.view(np.int64)).cuda()
    ids_d = torch.zeros(3 * nbytes, dtype=torch.int32, device="cuda")
    cnt_d = torch.zeros(len(raw), dtype=torch.int32, device="cuda")
    L = tk.L
    enc = []
    for _ in range(6):           # the library call alone (synchronous), inputs in HBM
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        assert L.aotx_text_encode(bytes_d.data_ptr(), at_d.data_ptr(), len(raw), ids_d.data_ptr(),
                                  cnt_d.data_ptr(), None) == 0
        enc.append(time.perf_counter() - t0)
    cnt = cnt_d.cpu().numpy()
    ids_h = ids_d.cpu().numpy()
    seqs = [ids_h[3 * int(at[i]):3 * int(at[i]) + int(cnt[i])] for i in range(len(raw))]
    flat = torch.from_numpy(np.concatenate(seqs).astype(np.int32)).cuda()
    tat = np.zeros(len(raw) + 1, dtype=np.uint64)
    tat[1:] = np.cumsum(cnt.astype(np.uint64))
    tat_d = torch.from_numpy(tat.view(np.int64)).cuda()
    limit = 2048
    out_d = torch.zeros(len(raw) * limit, dtype=torch.uint8, device="cuda")
    len_d = torch.zeros(len(raw), dtype=torch.int32, device="cuda")
    dec = []
    for _ in range(6):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        assert L.aotx_text_detok(flat.data_ptr(), tat_d.data_ptr(), len(raw), out_d.data_ptr(), limit,
                                 len_d.data_ptr(), None) == 0
        torch.cuda.synchronize()
        dec.append(time.perf_counter() - t0)
    o = out_d[:limit].cpu().numpy()
    assert bytes(o[:int(len_d[0])]) == raw[0]
    ntok = int(cnt.sum())
    e, d = min(enc[1:]), min(dec[1:])
    cpu = None
    if not args.no_cpu:
        from oracle.text import Vocab
        v = Vocab(tokens, merges, family="llama3")
        t0, done = time.perf_counter(), 0
        for r in raw:                  # bounded: at most ~20 s of the same texts
            v.encode(r)
            done += len(r)
            if time.perf_counter() - t0 > 20.0:
                break
        el = time.perf_counter() - t0
        cpu = {"value": round(done / el / 1e6, 4), "unit": "MB/s", "cores": 1, "kind": "port",
               "sample": f"{done} bytes of the same texts through oracle/text.py encode ({el:.1f} s)"}
    tk.close()
    print(json.dumps({"metric": "tokenizer encode MB/s (llama3 split, BPE merge on the GPU)",
                      "value": round(nbytes / e / 1e6, 2), "unit": "MB/s", "texts": len(texts),
                      "bytes": nbytes, "tokens": ntok, "encode_ms": round(e * 1e3, 3),
                      "decode_ms": round(d * 1e3, 3),
                      "decode_mb_s": round(nbytes / d / 1e6, 2),
                      "note": "wall clock of the synchronous library calls on inputs in HBM (encode includes its scratch allocations and one 4-byte read-back)",
                      "cpu_baseline": cpu}))


def tick_run(args):
    """`--tick`: the tick plan and commit kernels (one wave each) for 64 prefill slots of the
    tiny model and a full 512-row batch, timed with HIP events over 200 ticks on one stream.
    Prints one JSON line."""
    import ctypes
    import torch
    import aotx_amd as A
    from aotx_amd.model import TINY, Runtime, build_host
    torch.cuda.init()
    region, lay = build_host(TINY, seed=1)
    rt = Runtime(torch.from_numpy(region).cuda(), lay.desc, max_tokens=512, pool_pages=256)
    L = rt.L
    table = (A.PlanSlot * A.AOTX_SLOTS)()
    for i in range(A.AOTX_SLOTS):
        t = table[i]
        # prefill slots of long prompts: with no model step between ticks nothing enters the
        # pages, so every tick packs the same full batch (512 rows) and records 512 tokens
        t.state, t.role, t.prompt, t.sampled, t.limit = A.AOTX_SEQ_STATE_PREFILL, 2, 4000, 0, 64
        t.seed, t.stop, t.sample = 1000 + i, 0xFFFFFFFF, A.neutral_how()
    slots = torch.from_numpy(np.frombuffer(bytes(table), dtype=np.uint8).copy()).cuda()
    lists = torch.zeros((A.AOTX_SLOTS, 4096), dtype=torch.int32, device="cuda")
    plan = torch.zeros(ctypes.sizeof(A.PlanState), dtype=torch.uint8, device="cuda")
    recs = torch.zeros(1024 * ctypes.sizeof(A.TokenRecord), dtype=torch.uint8, device="cuda")
    tok = torch.zeros(A.AOTX_SLOTS, dtype=torch.int32, device="cuda")
    drw = torch.zeros(A.AOTX_SLOTS, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream()

    def tick():
        assert L.aotx_decode_plan(2, slots.data_ptr(), lists.data_ptr(), 4096, 512, rt.map.limit,
                                  plan.data_ptr(), ctypes.c_void_p(s.cuda_stream)) == 0
        assert L.aotx_decode_commit(2, slots.data_ptr(), lists.data_ptr(), 4096, tok.data_ptr(),
                                    drw.data_ptr(), plan.data_ptr(), recs.data_ptr(), 1024,
                                    ctypes.c_void_p(s.cuda_stream)) == 0
    tick()                                  # asks for the pages
    torch.cuda.synchronize()
    L.aotx_kv_serve(ctypes.byref(rt.map), None)
    for _ in range(5):
        tick()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(200):
        tick()
    e1.record(s)
    torch.cuda.synchronize()
    st = A.PlanState.from_buffer_copy(plan.cpu().numpy().tobytes())
    us = e0.elapsed_time(e1) * 1e3 / 200
    rt.close()
    print(json.dumps({"metric": "tick plan + commit us per tick (64 slots, 512-row batch)",
                      "value": round(us, 2), "unit": "us", "seqs": st.seqs, "rows": st.tokens,
                      "records": st.records,
                      "note": "two one-wave launches per tick, back to back on one stream"}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--context", type=int, default=2048)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the prefill chunk and the Mixtral-shape (config 5) lines")
    ap.add_argument("--moe", action="store_true",
                    help="BASELINE config 5 only: the Mixtral-shape routed-expert decoder")
    ap.add_argument("--prefill", action="store_true",
                    help="time one prompt chunk of 128/256/512 tokens (8B shape) and exit")
    ap.add_argument("--tick", action="store_true",
                    help="time the tick plan + commit kernels and exit")
    ap.add_argument("--text", action="store_true",
                    help="time the tokenizer (encode/decode on the GPU) and exit")
    ap.add_argument("--step-only", action="store_true",
                    help="only the decode steps at batch 32 and 1 (no GEMV table, attention "
                         "timing, ragged case or CPU baseline): the kernel-trace workload")
    ap.add_argument("--traffic", action="store_true",
                    help="run only the roofline kernel and a calibration copy (counter passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the token loop's slots are independent; see the sharding note in DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)

    if args.traffic:
        traffic_run(args)
        return
    if args.moe:
        moe_run(args)
        return
    if args.prefill:
        prefill_run(args)
        return
    if args.text:
        text_run(args)
        return
    if args.tick:
        tick_run(args)
        return

    import torch
    import aotx_amd as A
    from aotx_amd.model import LLAMA_8B, Runtime, build_device
    L = A.lib()
    torch.cuda.init()
    log("bench: device", torch.cuda.get_device_name(0))

    # Q8 GEMV table (config 2) and the roofline of the dominant kernel.
    shapes = [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]
    table = [] if args.step_only else gemv_table(torch, L, shapes, [1, 4, 8, 32])
    for row in table:
        log(f"gemv n={row['n']} k={row['k']} m={row['m']}: file {row['file_us']} us "
            f"{row['file_gbs']} GB/s | repacked {row['repacked_us']} us {row['repacked_gbs']} GB/s")
    dom = next((r for r in table if r["n"] == 14336 and r["k"] == 4096 and r["m"] == args.batch),
               None)

    # 8B-shape decoder, synthetic weights on the GPU.
    shape = LLAMA_8B
    t0 = time.perf_counter()
    region, lay = build_device(shape, seed=0x5EED)
    log(f"bench: weights {region.numel() / 1e9:.2f} GB built in {time.perf_counter() - t0:.1f}s")
    reserve = args.warmup * 3 + args.steps * 3 + 8 + 2 * CONFIG4_STEPS
    from aotx_amd.model import layout_pages
    per_slot = layout_pages(args.context + reserve, shape.layers, shape.kv_heads, shape.head_dim)
    batch_slots = list(range(args.batch))
    one_slot = [63]
    rt = Runtime(region, lay.desc, max_tokens=max(32, args.batch),
                 pool_pages=per_slot * (len(batch_slots) + 1) + 8)
    seat_context(torch, rt, batch_slots + one_slot, args.context, reserve, shape.layers,
                 shape.kv_heads, shape.head_dim)
    if args.step_only:
        tps, ms = decode(torch, rt, batch_slots, args.steps, args.warmup, A.neutral_how())
        tps1, ms1 = decode(torch, rt, one_slot, args.steps, args.warmup, A.neutral_how())
        rt.close()
        print(json.dumps({"step_only": True, "batch": args.batch, "tokens_per_s": round(tps, 2),
                          "ms_per_step": round(ms, 4), "batch1_ms_per_step": round(ms1, 4)}))
        return
    att_us, att_bytes = attention_rate(torch, L, batch_slots, args.context, shape.heads,
                                       shape.kv_heads, shape.head_dim, shape.layers)
    log(f"bench: attention batch {args.batch} ctx {args.context}: {att_us:.2f} us, "
        f"{att_bytes / att_us / 1e3:.1f} GB/s")
    greedy = A.neutral_how()
    tps, ms = decode(torch, rt, batch_slots, args.steps, args.warmup, greedy)
    log(f"bench: batch {args.batch} greedy: {tps:.1f} tokens/s, {ms:.3f} ms/step")
    tps1, ms1 = decode(torch, rt, one_slot, args.steps, args.warmup, greedy)
    log(f"bench: batch 1 greedy: {tps1:.1f} tokens/s, {ms1:.3f} ms/step")
    sampled = A.neutral_how(temperature=0.8, top_k=40, top_p=0.9, seed=0x5EED)
    tpss, mss = decode(torch, rt, batch_slots, max(4, args.steps // 2), 1, sampled)
    log(f"bench: batch {args.batch} top-k 40/top-p 0.9/T 0.8: {tpss:.1f} tokens/s")

    # BASELINE config 4 exactly: 128 greedy steps of the 32 slots from context 2048
    for sl in batch_slots:
        A.check(L.aotx_model_seat(sl, args.context), "aotx_model_seat")
    tps4, ms4 = decode(torch, rt, batch_slots, CONFIG4_STEPS, 0, greedy)
    log(f"bench: config 4 ({CONFIG4_STEPS} steps from {args.context}): {tps4:.1f} tokens/s")

    # algorithmic bytes of one decode step (positions attended averaged over the timed steps)
    ctx_mean = args.context + args.warmup + (args.steps + 1) / 2.0
    step_bytes_b = step_bytes(lay, shape, args.batch, ctx_mean)
    step_bytes1 = step_bytes(lay, shape, 1, ctx_mean)
    step_bytes4 = step_bytes(lay, shape, args.batch, args.context + (CONFIG4_STEPS + 1) / 2.0)

    result = {
        "metric": "decode tokens/s at batch 1 & 32 (8B-shape Q8); Q8 GEMV achieved HBM GB/s",
        "value": round(tps, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights (int8 x fp16 scale), fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) Q8_0 weights; random fp16 KV; greedy ids)",
        "config": {"workload": "8B-shape Q8 decoder decode step, 32 slots x 2048-token paged KV",
                   "layers": 32, "d_model": 4096, "heads": "32/8x128", "ffn": 14336,
                   "vocab": 128256, "batch": args.batch, "context": args.context,
                   "parallelism": "single GPU"},
        "batch1_tokens_per_s": round(tps1, 2),
        "batch1_ms_per_step": round(ms1, 4),
        "sampled_tokens_per_s": round(tpss, 2),
        "step_gb": round(step_bytes_b / 1e9, 4),
        "step_roofline_frac": round(step_bytes_b / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        "step_gb_batch1": round(step_bytes1 / 1e9, 4),
        "step_roofline_frac_batch1": round(step_bytes1 / (ms1 * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        "config4_128_steps": {"tokens_per_s": round(tps4, 2), "ms_per_step": round(ms4, 4),
                              "steps": CONFIG4_STEPS, "context_from": args.context,
                              "step_gb": round(step_bytes4 / 1e9, 4),
                              "step_roofline_frac": round(step_bytes4 / (ms4 * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)},
        "gemv": table,
    }
    result["roofline"] = {
        "bound": "hbm",
        "kernel": f"aotx_attend_mma<128,4,8> (paged decode attention, batch {args.batch}, "
                  f"context {args.context}, 32/8 heads x 128)",
        "achieved": round(att_bytes / att_us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(att_bytes / att_us / 1e3 / HBM_PEAK_GBS, 4),
        "traffic": measured_traffic() if args.batch == 32 and args.context == 2048 else None,
        "bytes_per_launch": att_bytes, "us_per_launch": round(att_us, 2)}
    if dom is not None:
        result["q8_product_roofline"] = {
            "kernel": f"aotx_rgemv (repacked Q8_0 product) n={dom['n']} k={dom['k']} m={dom['m']}",
            "achieved": dom["repacked_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dom["repacked_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_launch": dom["bytes"], "us_per_launch": dom["repacked_us"]}
    rt.close()

    # ragged contexts over permuted pages
    r_us, r_bytes, r_ctx = attention_ragged(torch, L)
    log(f"bench: attention 32 x U[512, 8192] (mean {r_ctx.mean():.0f}): {r_us:.2f} us, "
        f"{r_bytes / r_us / 1e3:.1f} GB/s")
    result["paged_attention_ragged"] = {
        "kernel": "aotx_attend_mma<128,4,8>", "batch": 32, "context": "U[512, 8192] seeded",
        "context_sum": int(r_ctx.sum()), "us_per_launch": round(r_us, 2),
        "bytes_per_launch": int(r_bytes), "achieved": round(r_bytes / r_us / 1e3, 1),
        "unit": "GB/s", "frac": round(r_bytes / r_us / 1e3 / HBM_PEAK_GBS, 4)}

    if not args.no_cpu:
        threads = args.cpu_threads or min(16, len(os.sched_getaffinity(0)))
        cbatch = args.batch
        cps, cdt = cpu_baseline(region, lay, torch, cbatch, args.context, threads)
        result["cpu_baseline"] = {
            "value": round(cps, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "host_cores": os.cpu_count(), "host_cores_available": len(os.sched_getaffinity(0)),
            "sample": f"one oracle decode step, batch {cbatch}, context {args.context} "
                      f"({cdt:.1f} s on {threads} threads)"}

    if not args.no_extra:
        # the prefill path (one 512-token prompt chunk of the same 8B weights) and
        # BASELINE config 5 (Mixtral shape), both timed in this run
        pf = prefill_measure(torch, region, lay, shape, (512,))["512"]
        log(f"bench: prefill 512 tokens: {pf['ms']} ms, {pf['tflops']} TFLOP/s")
        result["prefill_512"] = dict(pf, workload="8B shape, one 512-token prompt chunk, whole step",
                                     peak_tflops=MFMA_PEAK_FP16_TFLOPS)
        del region
        torch.cuda.empty_cache()
        moe = moe_measure(torch, 16, 2)
        log(f"bench: moe config 5: {moe['value']} tokens/s, {moe['ms_per_step']} ms/step")
        result["moe_config5"] = {k: moe[k] for k in ("value", "unit", "ms_per_step", "steps",
                                                     "warmup", "batch", "context", "step_gb",
                                                     "step_roofline_frac")}
    print(json.dumps(result))


if __name__ == "__main__":
    main()
