"""Paged decode attention on the GPU vs the oracle's online-softmax attention
(cuda/model/attention.cu:22-154), over pages the pool hands out by the reference's policy,
with ragged contexts, grouped-query heads and a missing page."""
import ctypes

import numpy as np
import pytest

import aotx_amd
from oracle.kvpolicy import KvPolicy, layout_pages
from tests.gpu_util import dev, p

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def _open_pool(lib, pages):
    m = aotx_amd.KvMap()
    m.limit = pages
    assert lib.aotx_kv_open(ctypes.byref(m)) == 0
    return m


def _fill(torch, lib, slots, contexts, layers, layer, kvh, d, rng):
    """K/V rows for every position of every slot (fp16), written through aotx_kv_write."""
    keys, vals = {}, {}
    for s, n in zip(slots, contexts):
        k = rng.normal(0, 1, (n, kvh, d)).astype(np.float16)
        v = rng.normal(0, 1, (n, kvh, d)).astype(np.float16)
        keys[s], vals[s] = k, v
        pos = np.arange(n, dtype=np.uint32)
        ag = np.full(n, s, dtype=np.uint32)
        assert lib.aotx_kv_write(p(dev(k, torch)), p(dev(v, torch)), p(dev(pos, torch)),
                                 p(dev(ag, torch)), n, kvh, d, layer, layers, None) == 0
    torch.cuda.synchronize()
    return keys, vals


@pytest.mark.parametrize("heads,kvh,d,layers,layer", [(32, 8, 128, 2, 1), (4, 4, 64, 4, 3),
                                                      (8, 4, 128, 1, 0), (16, 2, 64, 3, 0)])
def test_attend_vs_oracle(torch, lib, orc, heads, kvh, d, layers, layer):
    rng = np.random.default_rng(heads * 7 + d)
    slots = [3, 0, 17, 9]
    contexts = [1, 17, 300, 1200]
    pool = 256
    m = _open_pool(lib, pool)
    try:
        policy = KvPolicy(pool)
        for s, n in zip(slots, contexts):
            need = layout_pages(n, layers, kvh, d)
            assert lib.aotx_kv_request(s, need) == 1
            policy.request(s, need)
        assert lib.aotx_kv_serve(ctypes.byref(m), None) == len(slots)
        policy.serve()
        table = aotx_amd.KvTable()
        lib.aotx_kv_table_read(ctypes.byref(table))
        for s in slots:   # page-table decisions bit-exact vs the reference policy
            got = [(table.page[s][i] - m.range) // aotx_amd.AOTX_KV_PAGE_BYTES for i in range(table.count[s])]
            assert got == policy.page[s]
        keys, vals = _fill(torch, lib, slots, contexts, layers, layer, kvh, d, rng)
        # queries: the last position of each slot, plus a middle position of the longest
        qs = [(s, n - 1) for s, n in zip(slots, contexts)] + [(9, 555)]
        q = rng.normal(0, 1, (len(qs), heads, d)).astype(np.float16)
        pos = np.array([x[1] for x in qs], dtype=np.uint32)
        ag = np.array([x[0] for x in qs], dtype=np.uint32)
        out = torch.zeros(len(qs) * heads * d, dtype=torch.float16, device="cuda")
        assert lib.aotx_attend_paged(p(dev(q, torch)), p(dev(pos, torch)), p(dev(ag, torch)), len(qs),
                                     heads, kvh, d, layer, layers, p(out), None) == 0
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(len(qs), heads, d).astype(np.float32)
        g = heads // kvh
        for i, (s, last) in enumerate(qs):
            for hh in range(heads):
                kk = keys[s][:, hh // g, :].astype(np.float32)
                vv = vals[s][:, hh // g, :].astype(np.float32)
                want = orc.attend_one(q[i, hh].astype(np.float32), kk, vv, last)
                err = np.abs(got[i, hh] - want).max()
                assert err < 4e-3, (i, hh, err)
        assert lib.aotx_model_faulted() == 0
    finally:
        lib.aotx_kv_close(ctypes.byref(m))


def test_attend_config3_ragged_permuted(torch, lib, orc):
    """BASELINE config 3 shape: 32 sequences, contexts uniform in [512, 8192], 32/8 heads x
    128, pages handed out one at a time in a seeded random slot order (each sequence gets a
    random selection of the pool's physical pages). One workgroup takes a whole sequence
    here (up to 8192 positions); page decisions bit-exact, outputs vs the oracle."""
    heads, kvh, d, layers, layer = 32, 8, 128, 2, 1
    rng = np.random.default_rng(33)
    slots = list(range(32))
    contexts = [int(c) for c in rng.integers(512, 8193, len(slots))]
    need = {s: layout_pages(n, layers, kvh, d) for s, n in zip(slots, contexts)}
    pool = sum(need.values()) + 4
    m = _open_pool(lib, pool)
    try:
        policy = KvPolicy(pool)
        order = np.repeat(np.array(slots), [need[s] for s in slots])
        rng.shuffle(order)
        for i, s in enumerate(order):
            assert lib.aotx_kv_request(int(s), 1) == 1
            policy.request(int(s), 1)
            if i % 64 == 63:
                lib.aotx_kv_serve(ctypes.byref(m), None)
                policy.serve()
        lib.aotx_kv_serve(ctypes.byref(m), None)
        policy.serve()
        table = aotx_amd.KvTable()
        lib.aotx_kv_table_read(ctypes.byref(table))
        for s in slots:
            got = [(table.page[s][i] - m.range) // aotx_amd.AOTX_KV_PAGE_BYTES for i in range(table.count[s])]
            assert got == policy.page[s]
        keys, vals = _fill(torch, lib, slots, contexts, layers, layer, kvh, d, rng)
        q = rng.normal(0, 1, (len(slots), heads, d)).astype(np.float16)
        pos = np.array([n - 1 for n in contexts], dtype=np.uint32)
        ag = np.array(slots, dtype=np.uint32)
        out = torch.zeros(len(slots) * heads * d, dtype=torch.float16, device="cuda")
        lib.aotx_model_forget()
        assert lib.aotx_attend_paged(p(dev(q, torch)), p(dev(pos, torch)), p(dev(ag, torch)),
                                     len(slots), heads, kvh, d, layer, layers, p(out), None) == 0
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(len(slots), heads, d).astype(np.float32)
        g = heads // kvh
        for i, s in enumerate(slots):
            for hh in range(0, heads, 3):
                kk = keys[s][:, hh // g, :].astype(np.float32)
                vv = vals[s][:, hh // g, :].astype(np.float32)
                want = orc.attend_one(q[i, hh].astype(np.float32), kk, vv, contexts[i] - 1)
                err = np.abs(got[i, hh] - want).max()
                assert err < 4e-3, (i, hh, contexts[i], err)
        assert lib.aotx_model_faulted() == 0
    finally:
        lib.aotx_kv_close(ctypes.byref(m))


def test_attend_missing_page_counts_fault(torch, lib):
    m = _open_pool(lib, 8)
    try:
        lib.aotx_model_forget()
        q = np.zeros((1, 4, 64), dtype=np.float16)
        pos = np.array([40], dtype=np.uint32)
        ag = np.array([5], dtype=np.uint32)          # slot 5 holds no page
        out = torch.zeros(4 * 64, dtype=torch.float16, device="cuda")
        assert lib.aotx_attend_paged(p(dev(q, torch)), p(dev(pos, torch)), p(dev(ag, torch)), 1, 4, 4,
                                     64, 0, 1, p(out), None) == 0
        torch.cuda.synchronize()
        assert lib.aotx_model_faulted() > 0
        lib.aotx_model_forget()
        assert lib.aotx_model_faulted() == 0
    finally:
        lib.aotx_kv_close(ctypes.byref(m))


def test_kv_release_and_reuse(torch, lib):
    """Release gives every page back; the next request takes them LIFO (kv_host.cu:60-74)."""
    m = _open_pool(lib, 16)
    try:
        policy = KvPolicy(16)
        for s, n in ((1, 3), (2, 2)):
            lib.aotx_kv_request(s, n)
            policy.request(s, n)
        lib.aotx_kv_serve(ctypes.byref(m), None)
        policy.serve()
        lib.aotx_kv_release(1)
        policy.release(1)
        lib.aotx_kv_request(4, 4)
        policy.request(4, 4)
        lib.aotx_kv_serve(ctypes.byref(m), None)
        policy.serve()
        t = aotx_amd.KvTable()
        lib.aotx_kv_table_read(ctypes.byref(t))
        for s in (1, 2, 4):
            got = [(t.page[s][i] - m.range) // aotx_amd.AOTX_KV_PAGE_BYTES for i in range(t.count[s])]
            assert got == policy.page.get(s, [])
        assert t.mapped_pages == 6
        # every mapped page carries the fp16 header
        hdr = torch.zeros(16, dtype=torch.uint8, device="cuda")
        import ctypes as C
        assert t.page[4][0] != 0
    finally:
        lib.aotx_kv_close(ctypes.byref(m))


# (slot, cached positions before the piece, piece length)
_PIECES = [(3, 0, 57), (9, 13, 30), (21, 0, 1), (40, 301, 49), (5, 7, 3), (63, 1000, 1)]
# 20 decode rows side by side (a 16-token range of the launch leads 16 pieces, so each
# wave takes several), then a prompt
_SINGLES = [(10 + i, 5 * i + 2, 1) for i in range(20)] + [(50, 3, 117)]


@pytest.mark.parametrize("layout", ["pieces", "singles"])
@pytest.mark.parametrize("heads,kvh,d", [(32, 8, 128), (16, 2, 64), (8, 8, 64)])
def test_attend_prompt_pieces_vs_oracle(torch, lib, orc, heads, kvh, d, layout):
    """A launch of 128 tokens or more (prompt pieces: more tokens than sequence slots) runs
    the piece kernel, where one wave takes up to 16 / G consecutive queries of one sequence
    on a single pass over their keys: pieces that start mid-cache at positions that are
    not multiples of 16 / G, a run cut by the next sequence, single decode rows (many in
    one workgroup's range), causal limits per query; every (token, head) vs the oracle's
    online softmax at its own position."""
    layers, layer = 2, 0
    rng = np.random.default_rng(heads + kvh + d)
    pieces = _PIECES if layout == "pieces" else _SINGLES
    contexts = [c + n for _, c, n in pieces]
    slots = [s for s, _, _ in pieces]
    m = _open_pool(lib, 256)
    try:
        for s, n in zip(slots, contexts):
            assert lib.aotx_kv_request(s, layout_pages(n, layers, kvh, d)) == 1
        lib.aotx_kv_serve(ctypes.byref(m), None)
        keys, vals = _fill(torch, lib, slots, contexts, layers, layer, kvh, d, rng)
        pos = np.concatenate([np.arange(c, c + n) for _, c, n in pieces]).astype(np.uint32)
        ag = np.concatenate([np.full(n, s) for s, _, n in pieces]).astype(np.uint32)
        tokens = len(pos)
        assert tokens >= 128
        q = rng.normal(0, 1, (tokens, heads, d)).astype(np.float16)
        out = torch.zeros(tokens * heads * d, dtype=torch.float16, device="cuda")
        lib.aotx_model_forget()
        assert lib.aotx_attend_paged(p(dev(q, torch)), p(dev(pos, torch)), p(dev(ag, torch)),
                                     tokens, heads, kvh, d, layer, layers, p(out), None) == 0
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(tokens, heads, d).astype(np.float32)
        g = heads // kvh
        for i in range(tokens):
            s, last = int(ag[i]), int(pos[i])
            for hh in range(heads):
                kk = keys[s][:, hh // g, :].astype(np.float32)
                vv = vals[s][:, hh // g, :].astype(np.float32)
                want = orc.attend_one(q[i, hh].astype(np.float32), kk, vv, last)
                err = np.abs(got[i, hh] - want).max()
                assert err < 4e-3, (i, s, last, hh, err)
        assert lib.aotx_model_faulted() == 0
    finally:
        lib.aotx_kv_close(ctypes.byref(m))
