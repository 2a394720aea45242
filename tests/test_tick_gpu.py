"""The decode tick as one graph (aotx_decode_tick: plan -> step -> commit, the tick graph of
cuda/model/decode_host.cu:136-157) against the oracle, tick by tick, with per-slot samples
and penalties; and the restore of slots from their token records (aotx_seq_apply,
cuda/model/decode.cu:230-305) continuing the same tokens.

Each sequence's token is the one the oracle's sampler (orc_pick, cuda/model/sample.cu:
456-765) picks from the GPU's own logits of that row after the oracle's penalty adjustment
(orc_pick_adjust, sample.cu:277-319, pinned by a worked case in tests/test_oracle.py) at
the slot's own settings, seed and draw; the oracle's commit (oracle/plan.py) from those
tokens must then give the GPU's slot table, lists and token records exactly."""
import ctypes

import numpy as np
import pytest

import aotx_amd
from aotx_amd import (AOTX_MODEL_LANGUAGE, AOTX_SEQ_STATE_PREFILL, AOTX_SLOTS, PlanSlot,
                      PlanState, TokenRecord, neutral_how)
from aotx_amd.model import TINY, Runtime, build_host
from oracle.plan import Plan, commit

pytestmark = pytest.mark.gpu
ROLE = AOTX_MODEL_LANGUAGE
NO_STOP = 0xFFFFFFFF
FIELDS = ("state", "role", "prompt", "sampled", "limit", "page_limit", "seed", "stop", "flags",
          "last", "draw")
HOW = ("temperature", "top_k", "top_p", "min_p", "repeat_penalty", "repeat_window",
       "presence_penalty", "frequency_penalty")
SAMPLES = [
    dict(temperature=0.0),                                                    # greedy
    dict(temperature=0.8, top_k=40, top_p=0.9),
    dict(temperature=1.0, top_k=10, presence_penalty=0.7, frequency_penalty=0.3),
    dict(temperature=0.7, top_p=0.5, repeat_penalty=1.8, repeat_window=16),
    dict(temperature=1.3, top_k=0, min_p=0.05, presence_penalty=1.5),
    dict(temperature=0.0, repeat_penalty=3.0, repeat_window=64, frequency_penalty=2.0),
]


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def _how(spec):
    h = neutral_how(seed=0)
    for k, v in spec.items():
        setattr(h, k, v)
    return h


def _table(slots, samples):
    table = (PlanSlot * AOTX_SLOTS)()
    for i, s in enumerate(slots):
        for f in FIELDS:
            setattr(table[i], f, s[f])
        table[i].sample = _how(samples[i])
    return np.frombuffer(bytes(table), dtype=np.uint8).copy()


class Tick:
    """Device buffers of the tick and the oracle's mirror of them."""

    def __init__(self, torch, rt, slots, toks, samples, stride, cap=2048):
        self.torch, self.rt, self.lib = torch, rt, rt.L
        self.slots, self.toks, self.samples, self.stride = slots, toks, samples, stride
        self.slots_d = torch.from_numpy(_table(slots, samples)).cuda()
        lists = np.zeros((AOTX_SLOTS, stride), dtype=np.int32)
        for i, l in enumerate(toks):
            lists[i, :min(len(l), stride)] = l[:stride]
        self.lists_d = torch.from_numpy(lists).cuda()
        self.plan_d = torch.zeros(ctypes.sizeof(PlanState), dtype=torch.uint8, device="cuda")
        self.cap = cap
        self.rec_d = torch.zeros(cap * ctypes.sizeof(TokenRecord), dtype=torch.uint8, device="cuda")
        self.logits = torch.zeros((AOTX_SLOTS, TINY.vocab), dtype=torch.float32, device="cuda")
        self.oracle = Plan()
        self.seen = [0] * AOTX_SLOTS
        self.draws = [0] * AOTX_SLOTS

    def kv(self):
        t = aotx_amd.KvTable()
        assert self.lib.aotx_kv_table_read(ctypes.byref(t)) == 0
        return t

    def run(self, budget, orc, case):
        """One tick on the GPU and in the oracle; returns (records, expected tokens by slot)."""
        lib, torch = self.lib, self.torch
        before = self.kv()
        kv = dict(count=list(before.count), made=before.made, served=before.served,
                  mapped_pages=before.mapped_pages, requests=[])
        pages_of = lambda c: lib.aotx_model_kv_pages(ROLE, c)
        want = self.oracle.tick(ROLE, self.slots, self.toks, self.seen, budget, kv, pages_of,
                                self.rt.map.limit, stride=self.stride)
        assert lib.aotx_decode_tick(ROLE, self.slots_d.data_ptr(), self.lists_d.data_ptr(),
                                    self.stride, budget, self.rt.map.limit,
                                    self.plan_d.data_ptr(), self.rec_d.data_ptr(), self.cap,
                                    self.logits.data_ptr()) == 0
        got = PlanState.from_buffer_copy(self.plan_d.cpu().numpy().tobytes())
        n, t = want["seqs"], want["tokens"]
        assert (got.seqs, got.tokens) == (n, t), case
        assert list(got.agent[:n]) == want["agent"] and list(got.offset[:n + 1]) == want["offset"], case
        assert got.refused == self.oracle.refused, case
        logits = self.logits[:max(n, 1)].cpu().numpy()
        token = np.zeros(AOTX_SLOTS, dtype=np.int64)
        drawn = np.zeros(AOTX_SLOTS, dtype=np.int64)
        expect = {}
        for j in range(n):
            slot = want["agent"][j]
            h = _how(self.samples[slot])
            lst = self.toks[slot][:self.slots[slot]["prompt"] + self.slots[slot]["sampled"]]
            row = orc.pick_adjust(logits[j], lst, h.presence_penalty, h.frequency_penalty,
                                  h.repeat_penalty, h.repeat_window)
            tok, _, _ = orc.pick(row, h.top_k, h.top_p, h.min_p, h.temperature,
                                 self.slots[slot]["seed"], slot, self.draws[slot])
            token[j], drawn[j] = tok, self.draws[slot]
            expect[slot] = tok
            self.draws[slot] += 1
            self.seen[slot] += want["offset"][j + 1] - want["offset"][j]
        after = self.kv()
        kv2 = dict(count=list(after.count), releases=[])
        want_rec = commit(self.oracle, ROLE, self.slots, self.toks, want, token, drawn, kv2,
                          stride=self.stride)
        got = PlanState.from_buffer_copy(self.plan_d.cpu().numpy().tobytes())
        table = (PlanSlot * AOTX_SLOTS).from_buffer_copy(self.slots_d.cpu().numpy().tobytes())
        for i in range(AOTX_SLOTS):
            assert {f: getattr(table[i], f) for f in FIELDS} == self.slots[i], (case, i)
        lists = self.lists_d.cpu().numpy()
        for i in range(AOTX_SLOTS):
            k = min(len(self.toks[i]), self.stride)
            assert list(lists[i, :k]) == self.toks[i][:k], (case, i)
        recs = (TokenRecord * self.cap).from_buffer_copy(self.rec_d.cpu().numpy().tobytes())
        got_rec = [(r.slot, r.token, r.position, r.flags, r.seed, r.draw) for r in recs[:got.records]]
        assert got.records + got.dropped == len(want_rec), case
        assert got_rec == want_rec[:got.records], case
        lib.aotx_kv_serve(ctypes.byref(self.rt.map), None)
        return list(recs[:got.records]), expect


def _slots(rng, live, stride, prompts, limits):
    slots = [dict(state=0, role=ROLE, prompt=0, sampled=0, limit=0, page_limit=0, seed=0,
                  stop=NO_STOP, flags=0, last=0, draw=0) for _ in range(AOTX_SLOTS)]
    toks = [[] for _ in range(AOTX_SLOTS)]
    for s, p, l in zip(live, prompts, limits):
        slots[s].update(state=AOTX_SEQ_STATE_PREFILL, prompt=p, limit=l, seed=5000 + 7 * s)
        toks[s] = [int(x) for x in rng.integers(0, TINY.vocab, p)]
    return slots, toks


@pytest.mark.parametrize("budget", [24, 64])
def test_tick_graph_per_slot_samples_and_penalties(torch, orc, budget):
    rng = np.random.default_rng(budget)
    region, lay = build_host(TINY, seed=1)
    rt = Runtime(torch.from_numpy(region).cuda(), lay.desc, max_tokens=64, pool_pages=256)
    try:
        stride = 48
        live = [int(x) for x in rng.choice(AOTX_SLOTS, size=10, replace=False)]
        prompts = [int(x) for x in rng.integers(3, 30, 10)]
        limits = [int(x) for x in rng.integers(6, 30, 10)]
        prompts[0] = 60                    # longer than the list stride: refused every tick
        prompts[1], limits[1] = 40, 20     # the list fills its stride: ends at 48 tokens
        slots, toks = _slots(rng, live, stride, prompts, limits)
        samples = [SAMPLES[i % len(SAMPLES)] for i in range(AOTX_SLOTS)]
        cap = 2048 if budget == 24 else 16      # 16: records past the capacity are counted
        tk = Tick(torch, rt, slots, toks, samples, stride, cap=cap)
        sampled = dropped = 0
        for tick in range(80):
            recs, expect = tk.run(budget, orc, f"budget {budget} tick {tick}")
            sampled += len(expect)
            dropped += PlanState.from_buffer_copy(tk.plan_d.cpu().numpy().tobytes()).dropped
        assert sampled > 60
        assert (dropped > 0) == (cap == 16)
        assert slots[live[1]]["state"] == 0 and len(toks[live[1]]) == stride
        assert tk.oracle.refused >= 80
        # an idle tick (no slot has work) runs the graph on an empty batch
        recs, expect = tk.run(budget, orc, "idle")
        assert recs == [] and expect == {}
        assert rt.faulted() == 0
    finally:
        rt.close()


def test_tick_restore_continues_the_same_tokens(torch, orc):
    """Ticks run to the end; then every slot is opened again from its records up to the
    first `cut` of its sampled tokens (aotx_seq_apply), the lists are prefilled again by
    the following ticks, and the tokens sampled after the cut are the ones of the first run
    (the draw counter continues after the last applied draw)."""
    rng = np.random.default_rng(12)
    region, lay = build_host(TINY, seed=1)
    rt = Runtime(torch.from_numpy(region).cuda(), lay.desc, max_tokens=64, pool_pages=256)
    try:
        stride, budget, cut = 64, 64, 4
        live = [3, 17, 40, 62]
        slots, toks = _slots(rng, live, stride, [9, 14, 5, 11], [12, 10, 14, 9])
        samples = [SAMPLES[1 + i % (len(SAMPLES) - 1)] for i in range(AOTX_SLOTS)]
        tk = Tick(torch, rt, slots, toks, samples, stride)
        history = []
        for tick in range(40):
            recs, _ = tk.run(budget, orc, f"first run tick {tick}")
            history += recs
        first = {s: [r.token for r in history if r.slot == s and r.flags & 2] for s in live}
        assert all(len(first[s]) == slots[s]["limit"] for s in live)
        # records to apply: each slot's prompt and its first `cut` sampled tokens
        keep = []
        for s in live:
            mine = [r for r in history if r.slot == s]
            n_prompt = slots[s]["prompt"]
            keep += [r for r in mine if r.position < n_prompt + cut]
        arr = (TokenRecord * len(keep))(*keep)
        rec_d = torch.from_numpy(np.frombuffer(bytes(arr), dtype=np.uint8).copy()).cuda()
        # the slots are FREE by now (they ended and gave their pages back); open them again
        assert rt.L.aotx_seq_apply(ROLE, tk.slots_d.data_ptr(), tk.lists_d.data_ptr(), stride,
                                   tk.plan_d.data_ptr(), rec_d.data_ptr(), len(keep), None) == 0
        torch.cuda.synchronize()
        table = (PlanSlot * AOTX_SLOTS).from_buffer_copy(tk.slots_d.cpu().numpy().tobytes())
        state = PlanState.from_buffer_copy(tk.plan_d.cpu().numpy().tobytes())
        assert state.refused == 0
        for s in live:
            assert table[s].state == AOTX_SEQ_STATE_PREFILL and table[s].sampled == cut
            assert table[s].draw == [r.draw for r in keep if r.slot == s][-1]
            # the oracle mirror of the restored slot
            slots[s].update({f: getattr(table[s], f) for f in FIELDS})
            toks[s] = toks[s][:slots[s]["prompt"] + cut]
            tk.seen[s] = 0
            tk.draws[s] = int(table[s].draw) + 1
            tk.oracle.kept[s] = slots[s]["prompt"] + cut
            tk.oracle.asked[s] = 0
        again = {s: [] for s in live}
        for tick in range(30):
            recs, _ = tk.run(budget, orc, f"after restore tick {tick}")
            for r in recs:
                if r.flags & 2:
                    again[r.slot].append(r.token)
        for s in live:
            assert again[s] == first[s][cut:], s
        assert rt.faulted() == 0
    finally:
        rt.close()


def test_apply_confirms_the_prompt_of_an_open_slot(torch, orc):
    """Records replayed onto a slot that was opened with its prompt (kept 0): prompt records
    below the slot's prompt confirm the token standing there and change nothing else, a
    wrong token is refused, a sampled record continues the list; a position-0 record on a
    slot that has kept records shuts it and opens it again (cuda/model/decode.cu:240-272)."""
    rng = np.random.default_rng(5)
    region, lay = build_host(TINY, seed=1)
    rt = Runtime(torch.from_numpy(region).cuda(), lay.desc, max_tokens=64, pool_pages=256)
    try:
        stride, s = 32, 9
        slots, toks = _slots(rng, [s], stride, [6], [10])
        samples = [SAMPLES[0]] * AOTX_SLOTS
        tk = Tick(torch, rt, slots, toks, samples, stride)

        def apply(recs):
            arr = (TokenRecord * len(recs))(*recs)
            rec_d = torch.from_numpy(np.frombuffer(bytes(arr), dtype=np.uint8).copy()).cuda()
            assert rt.L.aotx_seq_apply(ROLE, tk.slots_d.data_ptr(), tk.lists_d.data_ptr(),
                                       stride, tk.plan_d.data_ptr(), rec_d.data_ptr(),
                                       len(recs), None) == 0
            torch.cuda.synchronize()
            table = (PlanSlot * AOTX_SLOTS).from_buffer_copy(tk.slots_d.cpu().numpy().tobytes())
            state = PlanState.from_buffer_copy(tk.plan_d.cpu().numpy().tobytes())
            return table[s], state, tk.lists_d.cpu().numpy()[s]

        def rec(token, position, flags, seed=77, draw=0):
            return TokenRecord(slot=s, token=token, position=position, flags=flags, seed=seed,
                               draw=draw, role=ROLE)

        prompt = toks[s]
        seq, state, lst = apply([rec(prompt[i], i, 1) for i in range(6)])
        assert state.refused == 0 and state.kept[s] == 6
        assert (seq.state, seq.prompt, seq.sampled, seq.seed) == (AOTX_SEQ_STATE_PREFILL, 6, 0,
                                                                 slots[s]["seed"])
        assert list(lst[:6]) == prompt
        seq, state, lst = apply([rec((prompt[2] + 1) % TINY.vocab, 2, 1)])
        assert state.refused == 1 and list(lst[:6]) == prompt
        seq, state, lst = apply([rec(123, 6, 2, seed=99, draw=4)])
        assert state.refused == 1 and (seq.prompt, seq.sampled, seq.seed, seq.draw) == (6, 1, 99, 4)
        assert lst[6] == 123 and state.kept[s] == 7
        # a new sequence in the slot: shut and opened again by its position-0 record
        seq, state, lst = apply([rec(555, 0, 1, seed=1234)])
        assert state.refused == 1
        assert (seq.state, seq.prompt, seq.sampled, seq.seed, seq.last) == (
            AOTX_SEQ_STATE_PREFILL, 1, 0, 1234, 555)
        assert lst[0] == 555 and state.kept[s] == 1
        assert rt.faulted() == 0
    finally:
        rt.close()
