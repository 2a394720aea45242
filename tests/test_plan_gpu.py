"""The tick plan on the GPU (aotx_decode_plan) against its oracle, tick by tick, with the
plan's batch driving the model step: plan -> aotx_model_sample on the plan's device arrays
-> pool serve -> the host's commit of the sampled tokens."""
import ctypes

import numpy as np
import pytest

import aotx_amd
from aotx_amd import (AOTX_MODEL_LANGUAGE, AOTX_SEQ_STATE_DECODE, AOTX_SEQ_STATE_DONE,
                      AOTX_SEQ_STATE_PREFILL, AOTX_SLOTS, PlanSlot, PlanState, neutral_how)
from aotx_amd.model import TINY, Runtime, build_host
from oracle.plan import Plan

pytestmark = pytest.mark.gpu
ROLE = AOTX_MODEL_LANGUAGE
STRIDE = 128


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def _upload(torch, slots, toks):
    table = (PlanSlot * AOTX_SLOTS)()
    for i, s in enumerate(slots):
        t = table[i]
        t.state, t.role, t.prompt, t.sampled = s["state"], s["role"], s["prompt"], s["sampled"]
        t.limit, t.page_limit, t.seed = s["limit"], s["page_limit"], s["seed"]
        t.sample = neutral_how(seed=0)
    raw = np.frombuffer(bytes(table), dtype=np.uint8).copy()
    lists = np.zeros((AOTX_SLOTS, STRIDE), dtype=np.int32)
    for i, l in enumerate(toks):
        lists[i, :len(l)] = l
    return torch.from_numpy(raw).cuda(), torch.from_numpy(lists).cuda()


def _kv(lib):
    table = aotx_amd.KvTable()
    assert lib.aotx_kv_table_read(ctypes.byref(table)) == 0
    return table


@pytest.mark.parametrize("budget,seed", [(24, 1), (7, 2), (512, 3)])
def test_plan_ticks_vs_oracle_driving_the_step(torch, budget, seed):
    rng = np.random.default_rng(seed)
    region, lay = build_host(TINY, seed=1)
    rt = Runtime(torch.from_numpy(region).cuda(), lay.desc, max_tokens=512, pool_pages=256)
    lib = rt.L
    try:
        slots = [dict(state=0, role=ROLE, prompt=0, sampled=0, limit=0, page_limit=0, seed=0)
                 for _ in range(AOTX_SLOTS)]
        toks = [[] for _ in range(AOTX_SLOTS)]
        live = rng.choice(AOTX_SLOTS, size=12, replace=False)
        for j, s in enumerate(live):
            prompt = int(rng.integers(5, 40))
            slots[s].update(state=AOTX_SEQ_STATE_PREFILL, prompt=prompt,
                            limit=int(rng.integers(4, 12)), seed=900 + int(s),
                            page_limit=1 if j == 0 else 0)   # one slot can never hold its pages
            toks[s] = [int(x) for x in rng.integers(0, TINY.vocab, prompt)]
        slots[int(live[1])]["role"] = ROLE + 1                # another role's slot
        pages_of = lambda c: lib.aotx_model_kv_pages(ROLE, c)
        assert pages_of(100) > 0
        plan_d = torch.zeros(ctypes.sizeof(PlanState), dtype=torch.uint8, device="cuda")
        base = plan_d.data_ptr()
        oracle = Plan()
        seen = [0] * AOTX_SLOTS
        token_d = torch.zeros(AOTX_SLOTS, dtype=torch.int32, device="cuda")
        draw_d = torch.zeros(AOTX_SLOTS, dtype=torch.int32, device="cuda")
        steps = 0
        for tick in range(80):
            before = _kv(lib)
            kv = dict(count=list(before.count), made=before.made, served=before.served,
                      mapped_pages=before.mapped_pages, requests=[])
            want = oracle.tick(ROLE, slots, toks, seen, budget, kv, pages_of, rt.map.limit)
            slots_d, lists_d = _upload(torch, slots, toks)
            assert lib.aotx_decode_plan(ROLE, slots_d.data_ptr(), lists_d.data_ptr(), STRIDE,
                                        budget, rt.map.limit, base, None) == 0
            torch.cuda.synchronize()
            got = PlanState.from_buffer_copy(plan_d.cpu().numpy().tobytes())
            after = _kv(lib)
            case = f"budget {budget} seed {seed} tick {tick}"
            assert got.seqs == want["seqs"] and got.tokens == want["tokens"], case
            n, t = got.seqs, got.tokens
            assert list(got.ids[:t]) == want["ids"], case
            assert list(got.offset[:n + 1]) == want["offset"], case
            assert list(got.agent[:n]) == want["agent"], case
            assert [got.how[i].seed for i in range(n)] == want["seed"], case
            assert list(got.rows) == want["rows"] and list(got.place) == want["place"], case
            assert list(got.first) == want["first"], case
            assert list(got.asked) == oracle.asked and list(got.cursor) == oracle.cursor, case
            assert (got.waited, got.short_of, got.steps) == (oracle.waited, oracle.short_of,
                                                             oracle.steps), case
            queued = sorted((after.queue[i % aotx_amd.AOTX_KV_QUEUE_MAX].agent,
                             after.queue[i % aotx_amd.AOTX_KV_QUEUE_MAX].pages)
                            for i in range(before.made, after.made))
            assert queued == sorted(kv["requests"]), case
            if t > 0:
                # the plan's batch, straight from its device arrays, through the model step
                how = neutral_how()
                out_seed = ctypes.c_uint64()
                assert lib.aotx_model_sample(ROLE, base + PlanState.ids.offset,
                                             base + PlanState.offset.offset, n,
                                             base + PlanState.agent.offset, ctypes.byref(how),
                                             token_d.data_ptr(), draw_d.data_ptr(),
                                             ctypes.byref(out_seed)) == 0
                sampled = token_d[:n].cpu().numpy()
                steps += 1
                for j in range(n):          # the host's commit
                    s = got.agent[j]
                    seen[s] += got.offset[j + 1] - got.offset[j]
                    sl = slots[s]
                    if seen[s] >= sl["prompt"] + sl["sampled"]:
                        toks[s].append(int(sampled[j]))
                        sl["sampled"] += 1
                        sl["state"] = (AOTX_SEQ_STATE_DONE if sl["sampled"] >= sl["limit"]
                                       else AOTX_SEQ_STATE_DECODE)
            lib.aotx_kv_serve(ctypes.byref(rt.map), None)
        assert steps > 5 and lib.aotx_model_faulted() == 0
        done = sum(1 for s in slots if s["state"] == AOTX_SEQ_STATE_DONE)
        assert done >= 8, done       # the slots that can run all finished their replies
    finally:
        rt.close()
