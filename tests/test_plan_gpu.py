"""The tick on the GPU against its oracle, tick by tick: aotx_decode_plan packs the batch,
aotx_model_sample runs the step on the plan's device arrays, aotx_decode_commit moves the
slots and writes the token records, and the pool serves the page requests."""
import ctypes

import numpy as np
import pytest

import aotx_amd
from aotx_amd import (AOTX_MODEL_LANGUAGE, AOTX_SEQ_STATE_DONE, AOTX_SEQ_STATE_PREFILL,
                      AOTX_SLOTS, PlanSlot, PlanState, TokenRecord, neutral_how)
from aotx_amd.model import TINY, Runtime, build_host
from oracle.plan import MARK_STOP, Plan, commit

pytestmark = pytest.mark.gpu
ROLE = AOTX_MODEL_LANGUAGE
STRIDE = 128
NO_STOP = 0xFFFFFFFF
FIELDS = ("state", "role", "prompt", "sampled", "limit", "page_limit", "seed", "stop", "flags",
          "last", "draw")


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def _slots_bytes(slots):
    table = (PlanSlot * AOTX_SLOTS)()
    for i, s in enumerate(slots):
        for f in FIELDS:
            setattr(table[i], f, s[f])
        table[i].sample = neutral_how(seed=0)
    return np.frombuffer(bytes(table), dtype=np.uint8).copy()


def _kv(lib):
    table = aotx_amd.KvTable()
    assert lib.aotx_kv_table_read(ctypes.byref(table)) == 0
    return table


def _queued(before, after):
    q = aotx_amd.AOTX_KV_QUEUE_MAX
    return sorted((after.queue[i % q].agent, after.queue[i % q].pages)
                  for i in range(before.made, after.made))


@pytest.mark.parametrize("budget,seed", [(24, 1), (7, 2), (512, 3)])
def test_tick_vs_oracle_plan_step_commit(torch, budget, seed):
    rng = np.random.default_rng(seed)
    region, lay = build_host(TINY, seed=1)
    rt = Runtime(torch.from_numpy(region).cuda(), lay.desc, max_tokens=512, pool_pages=256)
    lib = rt.L
    try:
        slots = [dict(state=0, role=ROLE, prompt=0, sampled=0, limit=0, page_limit=0, seed=0,
                      stop=NO_STOP, flags=0, last=0, draw=0) for _ in range(AOTX_SLOTS)]
        toks = [[] for _ in range(AOTX_SLOTS)]
        live = rng.choice(AOTX_SLOTS, size=12, replace=False)
        for j, s in enumerate(live):
            prompt = int(rng.integers(5, 40))
            slots[s].update(state=AOTX_SEQ_STATE_PREFILL, prompt=prompt,
                            limit=int(rng.integers(4, 12)), seed=900 + int(s),
                            page_limit=1 if j == 0 else 0)   # one slot can never hold its pages
            toks[s] = [int(x) for x in rng.integers(0, TINY.vocab, prompt)]
        slots[int(live[1])]["role"] = ROLE + 1                # another role's slot
        slots[int(live[2])]["flags"] = MARK_STOP              # stopped by its caller
        pages_of = lambda c: lib.aotx_model_kv_pages(ROLE, c)
        slots_d = torch.from_numpy(_slots_bytes(slots)).cuda()
        lists = np.zeros((AOTX_SLOTS, STRIDE), dtype=np.int32)
        for i, l in enumerate(toks):
            lists[i, :len(l)] = l
        lists_d = torch.from_numpy(lists).cuda()
        plan_d = torch.zeros(ctypes.sizeof(PlanState), dtype=torch.uint8, device="cuda")
        rec_cap = 1024
        rec_d = torch.zeros(rec_cap * ctypes.sizeof(TokenRecord), dtype=torch.uint8, device="cuda")
        base = plan_d.data_ptr()
        oracle = Plan()
        seen = [0] * AOTX_SLOTS
        token_d = torch.zeros(AOTX_SLOTS, dtype=torch.int32, device="cuda")
        draw_d = torch.zeros(AOTX_SLOTS, dtype=torch.int32, device="cuda")
        steps = records = 0
        for tick in range(80):
            case = f"budget {budget} seed {seed} tick {tick}"
            before = _kv(lib)
            kv = dict(count=list(before.count), made=before.made, served=before.served,
                      mapped_pages=before.mapped_pages, requests=[])
            want = oracle.tick(ROLE, slots, toks, seen, budget, kv, pages_of, rt.map.limit)
            assert lib.aotx_decode_plan(ROLE, slots_d.data_ptr(), lists_d.data_ptr(), STRIDE,
                                        budget, rt.map.limit, base, None) == 0
            torch.cuda.synchronize()
            got = PlanState.from_buffer_copy(plan_d.cpu().numpy().tobytes())
            after = _kv(lib)
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
            assert _queued(before, after) == sorted(kv["requests"]), case
            sampled = np.zeros(AOTX_SLOTS, dtype=np.int64)
            drawn = np.zeros(AOTX_SLOTS, dtype=np.int64)
            if t > 0:
                how = neutral_how()
                out_seed = ctypes.c_uint64()
                assert lib.aotx_model_sample(ROLE, base + PlanState.ids.offset,
                                             base + PlanState.offset.offset, n,
                                             base + PlanState.agent.offset, ctypes.byref(how),
                                             token_d.data_ptr(), draw_d.data_ptr(),
                                             ctypes.byref(out_seed)) == 0
                sampled[:n] = token_d[:n].cpu().numpy()
                drawn[:n] = draw_d[:n].cpu().numpy().view(np.uint32)
                steps += 1
                for j in range(n):
                    seen[got.agent[j]] += got.offset[j + 1] - got.offset[j]
            # the commit on the device and in the oracle, from the same step outputs
            kv2 = dict(count=list(after.count), releases=[])
            want_rec = commit(oracle, ROLE, slots, toks, want, sampled, drawn, kv2)
            assert lib.aotx_decode_commit(ROLE, slots_d.data_ptr(), lists_d.data_ptr(), STRIDE,
                                          token_d.data_ptr(), draw_d.data_ptr(), base,
                                          rec_d.data_ptr(), rec_cap, None) == 0
            torch.cuda.synchronize()
            got = PlanState.from_buffer_copy(plan_d.cpu().numpy().tobytes())
            table = (PlanSlot * AOTX_SLOTS).from_buffer_copy(slots_d.cpu().numpy().tobytes())
            for i in range(AOTX_SLOTS):
                assert {f: getattr(table[i], f) for f in FIELDS} == slots[i], (case, i)
            assert list(got.kept) == oracle.kept, case
            dev_lists = lists_d.cpu().numpy()
            for i in range(AOTX_SLOTS):
                assert list(dev_lists[i, :len(toks[i])]) == toks[i], (case, i)
            recs = (TokenRecord * rec_cap).from_buffer_copy(rec_d.cpu().numpy().tobytes())
            assert got.records == len(want_rec), case
            assert [(r.slot, r.token, r.position, r.flags, r.seed, r.draw)
                    for r in recs[:got.records]] == want_rec, case
            assert all(r.role == ROLE for r in recs[:got.records])
            records += got.records
            released = _queued(after, _kv(lib))
            assert released == sorted((s, 0) for s in kv2["releases"]), case
            lib.aotx_kv_serve(ctypes.byref(rt.map), None)
        assert steps > 5 and records > 100 and lib.aotx_model_faulted() == 0
        freed = sum(1 for s in slots if s["state"] == 0 and s["prompt"] > 0)
        assert freed >= 8, freed      # ran to their limit (or were stopped) and gave pages back
    finally:
        rt.close()
