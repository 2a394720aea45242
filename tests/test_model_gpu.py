"""The model-step operator surface on the GPU vs the oracle's whole-model forward.

BASELINE config 1 (tiny Llama: 4 layers, d_model 256, 4 heads x 64, FFN 688 zero-padded to
704, vocab 4096, eps 1e-5, theta 1e4, Q8 N(0, 0.02)): a 16-token prompt of uniform ids,
then 32 greedy steps through aotx_model_sample. Logits within 1e-2 of max(|want|, rms),
greedy ids equal wherever the oracle's top-2 gap exceeds twice the logit error bound
(docs/17-accuracy.md:41), page-table decisions equal to the reference policy."""
import ctypes

import numpy as np
import pytest

import aotx_amd
from aotx_amd.model import TINY, Shape, Runtime, build_host
from oracle.kvpolicy import KvPolicy, layout_pages
from tests.gpu_util import read_device, rel_rms

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


@pytest.fixture(scope="module")
def tiny(torch):
    region, lay = build_host(TINY, seed=1)
    return region, lay


def _runtime(torch, region, lay, max_tokens=32, pages=64):
    dev_region = torch.from_numpy(region).cuda()
    return Runtime(dev_region, lay.desc, max_tokens=max_tokens, pool_pages=pages)


def _gap_ok(want_row, err):
    s = np.sort(want_row)
    return s[-1] - s[-2] > 2 * err


def test_tiny_prompt_then_greedy(torch, orc, tiny):
    region, lay = tiny
    rt = _runtime(torch, region, lay)
    try:
        ref = orc.Model(lay.desc, region, slots=64, max_context=64)
        rng = np.random.default_rng(1)
        prompt = rng.integers(0, TINY.vocab, 16).tolist()
        tok, draw, logits = rt.step(prompt, [0, 16], [0])
        want = ref.step(prompt, [0, 16], [0])
        assert rel_rms(logits, want) < 1e-2
        flips = 0
        cur = int(tok[0])
        assert cur == int(np.argmax(want[0])) or not _gap_ok(want[0], np.abs(logits - want).max())
        for step in range(32):
            tok, draw, logits = rt.step([cur], [0, 1], [0])
            want = ref.step([cur], [0, 1], [0])
            err = np.abs(logits - want).max()
            assert rel_rms(logits, want) < 1e-2, step
            if int(tok[0]) != int(np.argmax(want[0])):
                assert not _gap_ok(want[0], err), (step, tok[0], np.argmax(want[0]))
                flips += 1
            assert draw[0] == step + 1
            cur = int(np.argmax(want[0]))  # follow the oracle so a flip cannot cascade
        assert flips <= 1
        assert rt.faulted() == 0
    finally:
        rt.close()


def test_tiny_sample_surface_and_pages(torch, orc, tiny):
    """aotx_model_sample (the drop-in operator) on ragged slots; page decisions vs policy."""
    region, lay = tiny
    rt = _runtime(torch, region, lay, pages=32)
    try:
        ref = orc.Model(lay.desc, region, slots=64, max_context=256)
        policy = KvPolicy(32)
        seen = {}
        rng = np.random.default_rng(5)
        slots = [7, 2, 40]
        lens = [20, 3, 9]
        ids = rng.integers(0, TINY.vocab, sum(lens)).tolist()
        offset = np.concatenate([[0], np.cumsum(lens)]).tolist()
        for s, n in zip(slots, lens):
            need = layout_pages(n, TINY.layers, TINY.kv_heads, TINY.head_dim)
            if need:
                policy.request(s, need)
            seen[s] = n
        policy.serve()
        tok, draw = rt.sample(ids, offset, slots)
        want = ref.step(ids, offset, slots)
        for i in range(3):
            assert tok[i] == np.argmax(want[i]) or not _gap_ok(want[i], 1e-2 * np.abs(want[i]).max())
        t = aotx_amd.KvTable()
        rt.L.aotx_kv_table_read(ctypes.byref(t))
        for s in slots:
            got = [(t.page[s][i] - rt.map.range) // aotx_amd.AOTX_KV_PAGE_BYTES for i in range(t.count[s])]
            assert got == policy.page.get(s, [])
        # decode one step for every slot; a slot that crosses into a new page gets it
        nxt = [int(x) for x in tok]
        tok2, draw2 = rt.sample(nxt, [0, 1, 2, 3], slots)
        want2 = ref.step(nxt, [0, 1, 2, 3], slots)
        for i in range(3):
            assert tok2[i] == np.argmax(want2[i]) or not _gap_ok(want2[i], 1e-2 * np.abs(want2[i]).max())
        assert list(draw2) == [1, 1, 1]
        assert rt.faulted() == 0
    finally:
        rt.close()


def test_tiny_sampling_seeded(torch, tiny):
    """Temperature 0 equals argmax; top-k 1 equals greedy; the same seed and draw position
    give the same token; restream replays (tests/model_test.cu:406-518)."""
    region, lay = tiny
    rt = _runtime(torch, region, lay)
    try:
        prompt = list(range(100, 116))
        g, _, lg = rt.step(prompt, [0, 16], [0])
        assert g[0] == np.argmax(lg[0])
        rt.L.aotx_model_forget()
        rt.L.aotx_model_restream()
        k1, _, _ = rt.step(prompt, [0, 16], [0], how=aotx_amd.neutral_how(temperature=0.8, top_k=1, seed=3))
        assert k1[0] == g[0]
        outs = []
        for rep in range(2):
            rt.L.aotx_model_forget()
            rt.L.aotx_model_restream()
            how = aotx_amd.neutral_how(temperature=0.8, top_k=40, top_p=0.9, seed=0x5EED)
            seq = []
            cur = prompt
            for step in range(6):
                t, d, _ = rt.step(cur, [0, len(cur)], [0], how=how)
                seq.append(int(t[0]))
                cur = [int(t[0])]
            outs.append(seq)
        assert outs[0] == outs[1]
    finally:
        rt.close()


def test_graph_replay_equals_eager(torch, tiny):
    """The recorded graph of a bucket gives on every replay, with other work and
    synchronisation between replays, the logits of a graph recorded afresh for the call
    (aotx_model_graphs(0))."""
    region, lay = tiny
    rt = _runtime(torch, region, lay)
    L = rt.L
    try:
        outs = []
        for keep in (1, 0):
            L.aotx_model_graphs(keep)
            rows = []
            for rep in range(4):
                L.aotx_model_forget()
                _, _, lg = rt.step(list(range(50, 60)), [0, 10], [3])
                x = torch.randn(1000, 1000, device="cuda") @ torch.randn(1000, 1000, device="cuda")
                torch.cuda.synchronize()
                rows.append(lg[0].copy())
            outs.append(rows)
        graph, fresh = outs
        for i in range(4):
            assert np.array_equal(graph[i], fresh[0])
            assert np.array_equal(fresh[i], fresh[0])
    finally:
        L.aotx_model_graphs(1)
        rt.close()


def test_qknorm_split_layer_kind(torch, orc):
    """The head-norm layer kind with split rotary pairs (the reference's Qwen3 kind) runs
    the general turn kernel; logits vs the oracle."""
    shape = Shape(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1024,
                  qk_norm=True, pairs=0)
    region, lay = build_host(shape, seed=3)
    rt = _runtime(torch, region, lay)
    try:
        ref = orc.Model(lay.desc, region, slots=8, max_context=64)
        ids = list(range(10, 30))
        _, _, lg = rt.step(ids, [0, 12, 20], [1, 4])
        want = ref.step(ids, [0, 12, 20], [1, 4])
        assert rel_rms(lg, want) < 1e-2
        _, _, lg = rt.step([3, 4], [0, 1, 2], [1, 4])
        want = ref.step([3, 4], [0, 1, 2], [1, 4])
        assert rel_rms(lg, want) < 1e-2
    finally:
        rt.close()


def test_moe_model_vs_oracle(torch, orc):
    """A small routed-expert model (8 experts, top-2, reference routing rule) end to end."""
    shape = Shape(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1024,
                  experts=8, used=2)
    region, lay = build_host(shape, seed=4)
    rt = _runtime(torch, region, lay, max_tokens=64)
    try:
        ref = orc.Model(lay.desc, region, slots=8, max_context=64)
        ids = list(range(200, 240))
        _, _, lg = rt.step(ids, [0, 25, 40], [0, 6])
        want = ref.step(ids, [0, 25, 40], [0, 6])
        assert rel_rms(lg, want) < 1e-2
        _, _, lg = rt.step([9, 8], [0, 1, 2], [0, 6])
        want = ref.step([9, 8], [0, 1, 2], [0, 6])
        assert rel_rms(lg, want) < 1e-2
    finally:
        rt.close()


def test_prefill_all_rows(torch, orc, tiny):
    """aotx_model_prefill with a logits buffer gives every token's row."""
    region, lay = tiny
    rt = _runtime(torch, region, lay)
    try:
        ids = list(range(7, 27))
        lg = rt.prefill_logits(ids, [0, 20], [0])
        ref = orc.Model(lay.desc, region, slots=2, max_context=64)
        for n in (1, 7, 20):
            r2 = orc.Model(lay.desc, region, slots=2, max_context=64)
            want = r2.step(ids[:n], [0, n], [0])
            assert rel_rms(lg[n - 1:n], want) < 1e-2
    finally:
        rt.close()


def _device_model(torch, shape, seed):
    """Weights synthesised on the device (the bytes build_host writes), copied back for the
    oracle: host synthesis of 4096-wide tensors takes minutes."""
    from aotx_amd.model import build_device
    region_dev, lay = build_device(shape, seed=seed)
    return region_dev, region_dev.cpu().numpy(), lay


@pytest.mark.parametrize("rows", [32, 20, 12, 6, 40, 48])
def test_8b_width_wide_batch_vs_oracle(torch, orc, rows):
    """8B-width layer (d_model 4096, FFN 14336, 32/8 heads x 128) at 5..32 batch rows (token
    buckets 8, 16 and 32): QKV (rotary + page write) and O (residual add + sums of squares)
    take the fragment-layout product, with x written in that layout by the norm, the down
    epilogue and the attention; gate/up and down take the wide kernel. A prompt pass of 4
    tokens per slot, then a decode step of one token per slot, logits vs the oracle.
    40 and 48 rows fall in the 64-token bucket: two 32-row passes in one launch, the second
    one partly filled (8 and 16 rows)."""
    shape = Shape(layers=1, hidden=4096, ffn=14336, heads=32, kv_heads=8, head_dim=128,
                  vocab=1024)
    region_dev, region, lay = _device_model(torch, shape, 5)
    rt = Runtime(region_dev, lay.desc, max_tokens=256, pool_pages=256)
    try:
        ref = orc.Model(lay.desc, region, slots=rows, max_context=64, threads=8)
        rng = np.random.default_rng(7)
        ids = rng.integers(0, shape.vocab, 4 * rows).tolist()
        offs = [4 * i for i in range(rows + 1)]
        agents = list(range(rows))
        _, _, lg = rt.step(ids, offs, agents)
        want = ref.step(ids, offs, agents)
        assert rel_rms(lg, want) < 1e-2
        ids = rng.integers(0, shape.vocab, rows).tolist()
        offs = list(range(rows + 1))
        _, _, lg = rt.step(ids, offs, agents)
        want = ref.step(ids, offs, agents)
        assert rel_rms(lg, want) < 1e-2
        assert rt.faulted() == 0
    finally:
        rt.close()


@pytest.mark.parametrize("rows", [32, 8])
def test_wide_qkv_fragment_four_tiles_vs_oracle(torch, orc, rows):
    """64 query heads x 128 over d_model 1024: a QKV product of 10240 rows (640 tiles), which
    the fragment-layout product takes at 4 tiles per workgroup (at the 8B shape only up to
    512 tiles occur), and an O product with k = 8192. A prompt pass of 4 tokens per slot,
    then a decode step, logits vs the oracle."""
    shape = Shape(layers=1, hidden=1024, ffn=1024, heads=64, kv_heads=8, head_dim=128,
                  vocab=1024)
    region_dev, region, lay = _device_model(torch, shape, 9)
    rt = Runtime(region_dev, lay.desc, max_tokens=128, pool_pages=128)
    try:
        ref = orc.Model(lay.desc, region, slots=rows, max_context=64, threads=8)
        rng = np.random.default_rng(11)
        ids = rng.integers(0, shape.vocab, 4 * rows).tolist()
        offs = [4 * i for i in range(rows + 1)]
        agents = list(range(rows))
        _, _, lg = rt.step(ids, offs, agents)
        want = ref.step(ids, offs, agents)
        assert rel_rms(lg, want) < 1e-2
        ids = rng.integers(0, shape.vocab, rows).tolist()
        offs = list(range(rows + 1))
        _, _, lg = rt.step(ids, offs, agents)
        want = ref.step(ids, offs, agents)
        assert rel_rms(lg, want) < 1e-2
        assert rt.faulted() == 0
    finally:
        rt.close()


@pytest.mark.parametrize("rows", [24, 40])
def test_8b_width_experts_wide_batch_vs_oracle(torch, orc, rows):
    """Routed experts at d_model 4096 with 24 and 40 rows: the expert down product (k = 4096)
    takes the wide kernel through the expert row lists; at 40 rows the dense products run
    two 32-row passes in one launch, the second with 8 rows. At 40 rows the first step's 80
    tokens give some expert more than 32 rows, so the routed products' second 32-row pass
    computes rows too."""
    shape = Shape(layers=1, hidden=4096, ffn=4096, heads=32, kv_heads=8, head_dim=128,
                  vocab=1024, experts=4, used=2)
    region_dev, region, lay = _device_model(torch, shape, 6)
    rt = Runtime(region_dev, lay.desc, max_tokens=128, pool_pages=128)
    try:
        ref = orc.Model(lay.desc, region, slots=rows, max_context=64, threads=8)
        rng = np.random.default_rng(8)
        ids = rng.integers(0, shape.vocab, 2 * rows).tolist()
        offs = [2 * i for i in range(rows + 1)]
        agents = list(range(rows))
        _, _, lg = rt.step(ids, offs, agents)
        want = ref.step(ids, offs, agents)
        assert rel_rms(lg, want) < 1e-2
        per_expert = read_device(rt.L.aotx_model_buffer(rt.role, 4), np.uint32, shape.experts)
        assert per_expert.sum() == 2 * rows * shape.used
        assert rows < 40 or per_expert.max() > 32
        ids = rng.integers(0, shape.vocab, rows).tolist()
        offs = list(range(rows + 1))
        _, _, lg = rt.step(ids, offs, agents)
        want = ref.step(ids, offs, agents)
        assert rel_rms(lg, want) < 1e-2
        assert rt.faulted() == 0
    finally:
        rt.close()


@pytest.mark.parametrize("prompt", [100, 300, 512])
def test_8b_width_long_prompt_logits_vs_oracle(torch, orc, prompt):
    """A prompt of 100, 300 and 512 tokens in one pass through aotx_model_prefill on an
    8B-width model (2 layers: d_model 4096, FFN 14336, 32/8 heads x 128): the GEMM of 128
    rows or more (k split for the products of few workgroups) with its QKV rotary/page-write,
    residual and SwiGLU epilogues, and the
    prompt-piece attention; the logits of tokens 1, 17, 130 and 257 and of the last vs the
    oracle
    (cuda/model/gemm.cuh:55-189, cuda/model/attention.cu:22-154)."""
    shape = Shape(layers=2, hidden=4096, ffn=14336, heads=32, kv_heads=8, head_dim=128,
                  vocab=1024)
    region_dev, region, lay = _device_model(torch, shape, 13)
    rt = Runtime(region_dev, lay.desc, max_tokens=512, pool_pages=64)
    try:
        rng = np.random.default_rng(prompt)
        ids = rng.integers(0, shape.vocab, prompt).tolist()
        lg = rt.prefill_logits(ids, [0, prompt], [3])
        ref = orc.Model(lay.desc, region, slots=4, max_context=prompt + 2, threads=8)
        # the oracle in one pass too (its products then read half weights, as the
        # reference's tensor-core tile does for 17 rows or more)
        want = ref.step(ids, [0, prompt], [3])
        assert rel_rms(lg[prompt - 1:prompt], want) < 1e-2
        for n in (1, 17, 130, 257):
            if n >= prompt:
                continue
            r2 = orc.Model(lay.desc, region, slots=4, max_context=prompt + 2, threads=8)
            w = r2.step(ids[:n], [0, n], [3])
            assert rel_rms(lg[n - 1:n], w) < 1e-2, n
        assert rt.faulted() == 0
    finally:
        rt.close()


def test_gguf_file_through_place_and_step(torch, orc, tiny, tmp_path):
    """The tiny model written as a GGUF file, read back by the library's reader, placed into
    a new weights region (aotx_model_place) and run: the same logits, bit for bit, as the
    region built directly (the same bytes through the same kernels), and within 1e-2 of the
    oracle; a second slot decodes after it."""
    from aotx_amd import gguf
    region, lay = tiny
    path = tmp_path / "tiny.gguf"
    gguf.export(TINY, region, lay, path)
    ids = list(range(30, 44))
    direct = _runtime(torch, region, lay)
    try:
        _, _, want_dev = direct.step(ids, [0, 14], [5])
        _, _, want_dev2 = direct.step([7], [0, 1], [5])
    finally:
        direct.close()
    region_f, desc = gguf.load(path)
    assert desc.token_embd != aotx_amd.AOTX_MODEL_ABSENT and desc.tied_output == 0
    rt = Runtime(region_f, desc, max_tokens=32, pool_pages=64)
    try:
        _, _, got = rt.step(ids, [0, 14], [5])
        _, _, got2 = rt.step([7], [0, 1], [5])
        assert np.array_equal(got, want_dev) and np.array_equal(got2, want_dev2)
        ref = orc.Model(lay.desc, region, slots=8, max_context=64)
        assert rel_rms(got, ref.step(ids, [0, 14], [5])) < 1e-2
        assert rel_rms(got2, ref.step([7], [0, 1], [5])) < 1e-2
        assert rt.faulted() == 0
    finally:
        rt.close()
