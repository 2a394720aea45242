"""Row packing of one decode tick, restated in Python — TEST INFRASTRUCTURE ONLY.

Follows cuda/model/plan.cu:54-199 (aotx_decode_plan) and the page check
cuda/model/decode_state.cuh:75-107 (aotx_seq_pending, aotx_seq_pages):
  - slot order: lane i takes slot (i + cursor[role]) % SLOTS (plan.cu:70);
  - want = min(prompt + sampled - held, budget) for a slot of the role in PREFILL or DECODE
    whose pages cover prompt + limit; a slot short of pages asks for them and counts in
    short_of (plan.cu:86-99);
  - decode rows first, one per DECODE slot while the inclusive count is within the budget
    (plan.cu:101-108);
  - prefill pieces in the room left; the piece that crosses its end is cut to the room,
    every later piece waits and counts in waited (plan.cu:110-124);
  - sequence places: decode slots in scan order, then the slots given a piece
    (plan.cu:127-146); the last offset is the row count; a tick with rows advances the
    cursor and the step count (plan.cu:163-172).
The gates the reference reads from device globals (ready, scheduler hold, replay, role
rotation) are the caller's here: the plan is called for ticks that run.
"""
SLOTS = 64
TICK_BUDGET = 512
FREE, PREFILL, DECODE, DONE = 0, 1, 2, 3


def kv_pages(context, layers, blocks_page, block=16):
    """cuda/model/kv_layout.cuh: pages of a context (blocks of 16 positions per layer)."""
    if blocks_page == 0:
        return 0
    blocks = (context + block - 1) // block * layers
    return (blocks + blocks_page - 1) // blocks_page


class Plan:
    """Plan state across ticks: cursor per role, asked pages per slot and counters."""

    def __init__(self, roles=5):
        self.cursor = [0] * roles
        self.asked = [0] * SLOTS
        self.kept = [0] * SLOTS
        self.waited = 0
        self.short_of = 0
        self.refused = 0
        self.steps = 0

    def pages(self, kv, slot, need, page_limit, pool_pages, made0):
        """decode_state.cuh:88-107. kv: dict with count [SLOTS], made, served, mapped_pages,
        and requests (list of (slot, pages)) that this appends to. The slots of a tick are
        checked at once (one lane each), so every slot sees the queue as the tick found it
        (made0)."""
        have = kv["count"][slot]
        if page_limit and need > page_limit:
            return False
        if need <= have:
            self.asked[slot] = have
            return True
        asked = max(self.asked[slot], have)
        if asked > have and kv["served"] == made0 and kv["mapped_pages"] < pool_pages:
            asked = have
        if need > asked:
            kv["requests"].append((slot, need - asked))
            kv["made"] += 1
            self.asked[slot] = need
        return False

    def tick(self, role, slots, tokens, seen, budget, kv, pages_of, pool_pages, stride=8192):
        """One tick. slots: list of dicts (state, role, prompt, sampled, limit, page_limit,
        seed); tokens[slot] = the slot's list; seen[slot] = tokens its pages hold;
        pages_of(context) = pages a slot needs; stride = the list capacity (a slot whose
        prompt exceeds it is refused). Returns the batch as a dict."""
        budget = min(budget, TICK_BUDGET)
        order = [(i + self.cursor[role]) % SLOTS for i in range(SLOTS)]
        want = {}
        made0 = kv["made"]
        for slot in order:
            s = slots[slot]
            w = 0
            if s["role"] == role and s["state"] in (PREFILL, DECODE) and s["prompt"] > stride:
                self.refused += 1
            elif s["role"] == role and s["state"] in (PREFILL, DECODE):
                lst = s["prompt"] + s["sampled"]
                pending = min(max(lst - seen[slot], 0), budget)
                if pending:
                    if self.pages(kv, slot, pages_of(s["prompt"] + s["limit"]), s["page_limit"],
                                  pool_pages, made0):
                        w = pending
                    else:
                        self.short_of += 1
            want[slot] = w
        # decode rows first
        decode = [slot for slot in order if slots[slot]["state"] == DECODE and want[slot]]
        made = min(len(decode), budget)
        decode = decode[:made]
        # prefill pieces in the room left
        room = max(budget - made, 0)
        before = 0
        pieces = []
        for slot in order:
            piece = want[slot] if slots[slot]["state"] == PREFILL else 0
            if piece:
                if before < room:
                    pieces.append((slot, min(piece, room - before), made + before))
                else:
                    self.waited += 1
            before += piece
        out = {"rows": [0] * SLOTS, "first": list(seen), "place": [SLOTS] * SLOTS,
               "ids": [], "offset": [], "agent": [], "seed": []}
        seqs = [(slot, 1, i) for i, slot in enumerate(decode)] + pieces
        for place, (slot, rows, start) in enumerate(seqs):
            out["rows"][slot] = rows
            out["place"][slot] = place
            out["agent"].append(slot)
            out["offset"].append(start)
            out["seed"].append(slots[slot]["seed"])
            lst = tokens[slot]
            out["ids"] += [lst[seen[slot] + i] if seen[slot] + i < len(lst) else 0
                           for i in range(rows)]
        total = made + min(before, room)
        out["offset"].append(total)
        out["seqs"] = len(seqs)
        out["tokens"] = total
        assert len(out["ids"]) == total
        if total:
            self.steps += 1
            self.cursor[role] = (self.cursor[role] + 1) % SLOTS
        return out

PROMPT, SAMPLED, LAST, MARK_STOP = 0x1, 0x2, 0x4, 0x100
SEQ_MAX = 8192


def commit(plan, role, slots, tokens, out, token, draw, kv, stride=8192):
    """cuda/model/commit.cu:102-201 without the journal ring, hash and reply wraps: move
    each slot of the role and return the tick's token records (slot, token, position,
    flags, seed, draw), slots in order. plan: the Plan (asked, kept); out: the tick's batch;
    token/draw: the step's outputs by sequence place; kv: dict with count and releases;
    stride: the list capacity (a sequence whose list fills it ends)."""
    records = []
    for slot in range(SLOTS):
        s = slots[slot]
        if s["role"] != role:
            continue
        if s["state"] == DONE:
            kv["releases"].append(slot)
            kv["count"][slot] = 0
            s["state"] = FREE
            plan.asked[slot] = 0
            continue
        if s["state"] not in (PREFILL, DECODE):
            continue
        rows = out["rows"][slot]
        lst = s["prompt"] + s["sampled"]
        end = out["first"][slot] + rows
        kept = plan.kept[slot]
        journal = max(end - kept, 0)
        extra = rows > 0 and end == lst and lst < SEQ_MAX
        if rows:
            s["state"] = DECODE if end == lst else PREFILL
        for i in range(journal):
            records.append((slot, tokens[slot][kept + i], kept + i, PROMPT, s["seed"], 0))
        if extra:
            place = out["place"][slot]
            tok, drawn = int(token[place]), int(draw[place])
            mark = SAMPLED
            tokens[slot].append(tok)
            s["sampled"] += 1
            s["last"], s["draw"] = tok, drawn
            if (tok == s["stop"] or s["sampled"] >= s["limit"] or s["flags"] & MARK_STOP
                    or lst + 1 >= SEQ_MAX or lst + 1 >= stride):
                mark |= LAST
                s["flags"] |= LAST
                s["state"] = DONE
            records.append((slot, tok, lst, mark, s["seed"], drawn))
        plan.kept[slot] = kept + journal + int(bool(extra))
        if s["flags"] & MARK_STOP:
            s["state"] = DONE
    return records
