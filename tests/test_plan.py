"""The tick plan's oracle (oracle/plan.py) pinned by hand-worked batches and by the
invariants the reference checks on its plan (tests/decode_roles_test.cu:43-57)."""
from oracle.plan import DECODE, DONE, FREE, PREFILL, SLOTS, Plan, kv_pages

BIG = 10 ** 6


def slot(state=FREE, role=2, prompt=0, sampled=0, limit=64, page_limit=0, seed=0):
    return dict(state=state, role=role, prompt=prompt, sampled=sampled, limit=limit,
                page_limit=page_limit, seed=seed)


def kv(count=BIG):
    return dict(count=[count] * SLOTS, made=0, served=0, mapped_pages=0, requests=[])


def lists():
    return [[1000 * s + k for k in range(256)] for s in range(SLOTS)]


def test_worked_batch():
    """Budget 10: decode slots 0 and 2 give one row each, first; prefill slot 1 takes 6,
    slot 3 is cut to the 2 rows left, slot 4 waits (plan.cu:101-124)."""
    slots = [slot() for _ in range(SLOTS)]
    seen = [0] * SLOTS
    slots[0] = slot(DECODE, prompt=5, sampled=3, seed=70); seen[0] = 7
    slots[1] = slot(PREFILL, prompt=6, seed=71)
    slots[2] = slot(DECODE, prompt=4, sampled=2, seed=72); seen[2] = 5
    slots[3] = slot(PREFILL, prompt=6, seed=73)
    slots[4] = slot(PREFILL, prompt=3, seed=74)
    p = Plan()
    out = p.tick(2, slots, lists(), seen, 10, kv(), lambda c: 1, 100)
    assert out["seqs"] == 4 and out["tokens"] == 10
    assert out["agent"] == [0, 2, 1, 3]
    assert out["offset"] == [0, 1, 2, 8, 10]
    assert out["ids"] == [7, 2005, 1000, 1001, 1002, 1003, 1004, 1005, 3000, 3001]
    assert out["rows"][:5] == [1, 6, 1, 2, 0] and out["place"][:5] == [0, 2, 1, 3, SLOTS]
    assert out["seed"] == [70, 72, 71, 73]
    assert p.waited == 1 and p.short_of == 0 and p.steps == 1 and p.cursor[2] == 1


def test_rotation_and_decode_budget():
    """The cursor rotates the slot order; decode rows beyond the budget wait without
    counting as waited (plan.cu:104-106)."""
    slots = [slot() for _ in range(SLOTS)]
    for s in (1, 5, 9, 13, 60):
        slots[s] = slot(DECODE, prompt=2, sampled=1)
    seen = [2] * SLOTS
    p = Plan()
    p.cursor[2] = 9
    out = p.tick(2, slots, lists(), seen, 3, kv(), lambda c: 1, 100)
    assert out["agent"] == [9, 13, 60] and out["tokens"] == 3 and p.waited == 0
    assert out["ids"] == [9002, 13002, 60002] and p.cursor[2] == 10
    # another role's slots and FREE/DONE slots give nothing, and a tick with no rows
    # leaves the cursor
    out = p.tick(3, slots, lists(), seen, 3, kv(), lambda c: 1, 100)
    assert out["tokens"] == 0 and out["offset"] == [0] and p.cursor[3] == 0 and p.steps == 1


def test_page_check():
    """decode_state.cuh:88-107: over the page limit no request; short of pages one request
    of the missing pages, not repeated while queued; asked again once the queue is served
    and the pool has free pages."""
    slots = [slot() for _ in range(SLOTS)]
    slots[0] = slot(PREFILL, prompt=40, limit=24, page_limit=3)   # needs 4 > 3
    slots[1] = slot(PREFILL, prompt=40, limit=24)                  # needs 4, holds 1
    slots[2] = slot(PREFILL, prompt=8, limit=8)                    # needs 1, holds 1
    seen = [0] * SLOTS
    k = kv(count=1)
    p = Plan()
    pages_of = lambda c: (c + 15) // 16                            # one block per page
    out = p.tick(2, slots, lists(), seen, 64, k, pages_of, 100)
    assert k["requests"] == [(1, 3)] and p.asked[1] == 4 and p.asked[2] == 1
    assert out["agent"] == [2] and out["tokens"] == 8 and p.short_of == 2
    p.tick(2, slots, lists(), seen, 64, k, pages_of, 100)
    assert k["requests"] == [(1, 3)]                               # still queued: no new ask
    k["served"] = k["made"]; k["count"][1] = 2; k["mapped_pages"] = 10   # partly served
    p.tick(2, slots, lists(), seen, 64, k, pages_of, 100)
    assert k["requests"] == [(1, 3), (1, 2)]
    k["served"] = k["made"]; k["mapped_pages"] = 100               # pool full: no re-ask
    p.asked[1] = 4
    p.tick(2, slots, lists(), seen, 64, k, pages_of, 100)
    assert len(k["requests"]) == 2
    assert kv_pages(2048, 32, 31) == 2048 // 16 * 32 // 31 + 1


def test_reference_invariants():
    """tests/decode_roles_test.cu:43-57 over 128 ticks: bounded rows and sequences, one
    owner per row, each row the owner's token at its position, every ready slot served."""
    for mode in (PREFILL, DECODE):
        for budget in (1, 17, 256):
            n = 64
            slots = [slot(mode, prompt=32 + i, sampled=1, limit=128, seed=710 + i)
                     for i in range(n)]
            seen = [i if mode == PREFILL else 32 + i for i in range(n)]
            toks = [[1000 + i * 128 + k for k in range(256)] for i in range(n)]
            p = Plan()
            served = [0] * n
            for _ in range(128):
                out = p.tick(2, slots, toks, seen, budget, kv(), lambda c: 1, 10)
                assert 0 < out["tokens"] <= budget and out["seqs"] <= n
                rows = 0
                for i in range(n):
                    if out["rows"][i]:
                        place = out["place"][i]
                        assert place < out["seqs"] and out["agent"][place] == i
                        at = out["offset"][place]
                        for k in range(out["rows"][i]):
                            assert out["ids"][at + k] == 1000 + i * 128 + out["first"][i] + k
                        served[i] += 1
                        rows += out["rows"][i]
                assert rows == out["tokens"]
                offs = out["offset"]
                assert all(a < b for a, b in zip(offs, offs[1:]))
            assert all(served), (mode, budget)


def test_worked_commit():
    """cuda/model/commit.cu:112-176 by hand: a prefill slot that got its whole list moves
    to DECODE and takes the sampled token (its prompt tokens recorded first); a slot cut
    short stays PREFILL with only the rows it gave recorded; a slot at its limit ends with
    the LAST flag; a DONE slot gives its pages back; a stop mark ends a slot."""
    from oracle.plan import LAST, MARK_STOP, PROMPT, SAMPLED, commit
    slots = [slot() for _ in range(SLOTS)]
    slots[0] = slot(PREFILL, prompt=3, limit=4, seed=5)
    slots[1] = slot(PREFILL, prompt=6, limit=4, seed=6)
    slots[2] = slot(DECODE, prompt=2, sampled=1, limit=2, seed=7)
    slots[3] = slot(DONE)
    slots[4] = slot(PREFILL, prompt=2, limit=9)
    for s in slots:
        s.update(stop=0xFFFFFFFF, flags=0, last=0, draw=0)
    slots[4]["flags"] = MARK_STOP
    toks = [[10 * i + k for k in range(8)] for i in range(SLOTS)]
    toks[2] = [20, 21, 22]
    seen = [0] * SLOTS
    seen[2] = 2
    p = Plan()
    p.kept[2] = 3
    out = p.tick(2, slots, toks, seen, 6, kv(), lambda c: 1, 100)
    # decode slot 2 first (1 row), then slot 0 (3 rows), slot 1 cut to 2, slot 4 waits
    assert out["agent"] == [2, 0, 1] and out["offset"] == [0, 1, 4, 6]
    k = dict(count=[1] * SLOTS, releases=[])
    toks[0], toks[1] = toks[0][:3], toks[1][:6]
    rec = commit(p, 2, slots, toks, out, [77, 55, 66], [9, 8, 7], k)
    assert rec == [(0, 0, 0, PROMPT, 5, 0), (0, 1, 1, PROMPT, 5, 0), (0, 2, 2, PROMPT, 5, 0),
                   (0, 55, 3, SAMPLED, 5, 8),
                   (1, 10, 0, PROMPT, 6, 0), (1, 11, 1, PROMPT, 6, 0),
                   (2, 77, 3, SAMPLED | LAST, 7, 9)]
    assert [slots[i]["state"] for i in range(5)] == [DECODE, PREFILL, 3, FREE, 3]
    assert toks[0] == [0, 1, 2, 55] and slots[0]["sampled"] == 1 and slots[2]["flags"] == LAST
    assert k["releases"] == [3] and p.kept[:3] == [4, 2, 4]
