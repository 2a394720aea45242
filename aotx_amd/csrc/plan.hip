/* The tick plan: row packing of one decode step (cuda/model/plan.cu:54-199).
 *
 * One wave, one lane per sequence slot (AOTX_SLOTS = 64), lane i taking slot
 * (i + cursor) mod 64 so that every slot is first in turn. The three prefix sums of the
 * packing (decode rows, prefill pieces, sequences given a piece) are wave scans over
 * those lanes, in that rotated order, which is the order of the reference's block scans.
 */
#include "aotx_internal.h"
#include "kvcache_dev.h"
#include "../../include/aotx_plan.h"
#include "tick.h"

static_assert(AOTX_SLOTS == 64u, "one lane per slot in one wave");

/* Inclusive sum over the lanes of the wave, in lane order. */
static __device__ __forceinline__ unsigned int plan_scan(unsigned int v)
{
    const unsigned int lane = threadIdx.x;
#pragma unroll
    for (unsigned int d = 1u; d < 64u; d <<= 1) {
        const unsigned int o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    return v;
}

/* Whether the slot holds the pages of a context of `context` positions; otherwise the
 * missing pages are asked for once (a request still queued counts as asked; a partly
 * served one is asked again when the queue is empty and the pool has free pages).
 * cuda/model/decode_state.cuh:88-107. */
static __device__ int plan_pages(aotx_state *st, aotx_plan_state *p, unsigned int slot,
                                 const aotx_kvl_shape &shape, unsigned int context,
                                 unsigned int page_limit, unsigned int pool_pages)
{
    const unsigned int need = aotx_kvl_pages(shape, context);
    const unsigned int have = st->kv.count[slot];
    if (page_limit != 0u && need > page_limit) return 0;
    if (need <= have) {
        p->asked[slot] = have;
        return 1;
    }
    unsigned int asked = p->asked[slot] > have ? p->asked[slot] : have;
    const unsigned int made = atomicAdd(&st->kv.made, 0u), served = atomicAdd(&st->kv.served, 0u);
    if (asked > have && served == made && st->kv.mapped_pages < pool_pages) asked = have;
    if (need > asked) p->asked[slot] = aotx_kv_put(&st->kv, slot, need - asked) ? need : have;
    return 0;
}

__global__ __launch_bounds__(64) void aotx_plan_kernel(unsigned int role, const aotx_plan_slot *slots,
                                                       const int *tokens, unsigned int stride,
                                                       unsigned int budget, unsigned int pool_pages,
                                                       aotx_kvl_shape shape, aotx_state *st,
                                                       aotx_plan_state *p)
{
    const unsigned int lane = threadIdx.x;
    const unsigned int slot = (lane + p->cursor[role]) % AOTX_SLOTS;
    const aotx_plan_slot &seq = slots[slot];
    const unsigned int state = seq.state;
    const unsigned int held = st->seen[slot];

    /* tokens of the list no page holds yet, if the slot's pages are there */
    unsigned int want = 0u;
    if (seq.role == role && (state == AOTX_SEQ_STATE_PREFILL || state == AOTX_SEQ_STATE_DECODE)
        && seq.prompt > stride) {
        atomicAdd(&p->refused, 1u);              /* the list cannot hold the prompt */
    } else if (seq.role == role && (state == AOTX_SEQ_STATE_PREFILL || state == AOTX_SEQ_STATE_DECODE)) {
        const unsigned int list = seq.prompt + seq.sampled;
        unsigned int pending = list > held ? list - held : 0u;
        if (pending > budget) pending = budget;
        if (pending > 0u) {
            if (plan_pages(st, p, slot, shape, seq.prompt + seq.limit, seq.page_limit, pool_pages))
                want = pending;
            else
                atomicAdd(&p->short_of, 1u);
        }
    }

    /* decode rows first: one per decode slot, while they fit the budget */
    unsigned int step = (state == AOTX_SEQ_STATE_DECODE && want > 0u) ? 1u : 0u;
    const unsigned int step_scan = plan_scan(step);
    const unsigned int step_all = __shfl(step_scan, 63, 64);
    const unsigned int made = step_all < budget ? step_all : budget;
    if (step_scan > budget) step = 0u;

    /* prefill pieces in the room left; the piece that crosses its end is cut, later ones wait */
    const unsigned int piece = state == AOTX_SEQ_STATE_PREFILL ? want : 0u;
    const unsigned int piece_scan = plan_scan(piece);
    const unsigned int before = piece_scan - piece;
    const unsigned int room = budget > made ? budget - made : 0u;
    unsigned int give = 0u;
    if (piece > 0u) {
        if (before < room) give = piece < room - before ? piece : room - before;
        else atomicAdd(&p->waited, 1u);
    }
    const unsigned int mark = give > 0u ? 1u : 0u;
    const unsigned int mark_scan = plan_scan(mark);
    const unsigned int piece_all = __shfl(piece_scan, 63, 64);
    const unsigned int total_rows = made + (piece_all < room ? piece_all : room);
    const unsigned int total_seqs = made + __shfl(mark_scan, 63, 64);

    unsigned int rows = 0u, start = 0u, place = AOTX_SLOTS;
    if (step > 0u) {
        rows = 1u;
        start = step_scan - 1u;
        place = start;
    } else if (give > 0u) {
        rows = give;
        start = made + (before < room ? before : room);
        place = made + mark_scan - 1u;
    }
    p->rows[slot] = rows;
    p->first[slot] = held;
    p->place[slot] = place;
    if (rows > 0u) {
        p->agent[place] = slot;
        p->offset[place] = start;
        aotx_model_how how = seq.sample;
        how.seed = seq.seed;
        p->how[place] = how;
    }
    /* the rows' token ids, copied by the whole wave one sequence at a time (a prompt piece
     * can be the whole budget) */
    for (unsigned int j = 0u; j < 64u; ++j) {
        const unsigned int n = __shfl(rows, (int)j, 64);
        if (n == 0u) continue;
        const unsigned int at0 = __shfl(held, (int)j, 64), dst = __shfl(start, (int)j, 64);
        const unsigned int src = __shfl(slot, (int)j, 64);
        for (unsigned int i = lane; i < n; i += 64u) {
            const unsigned int at = at0 + i;
            p->ids[dst + i] = at < stride ? tokens[(unsigned long long)src * stride + at] : 0;
        }
    }
    if (lane == 0u) {
        p->offset[total_seqs] = total_rows;
        p->seqs = total_seqs;
        p->tokens = total_rows;
        if (total_rows > 0u) {
            p->steps += 1ull;
            p->cursor[role] = (p->cursor[role] + 1u) % AOTX_SLOTS;
        }
    }
}

int aotx_plan_launch(unsigned int role, const aotx_plan_slot *slots, const int *tokens,
                     unsigned int stride, unsigned int budget, unsigned int pool_pages,
                     aotx_plan_state *plan, hipStream_t s)
{
    if (role >= AOTX_MODEL_ROLES || slots == nullptr || tokens == nullptr || plan == nullptr
        || stride == 0u)
        return 1;
    aotx_kvl_shape shape;
    if (aotx_role_kv_shape(role, &shape) != 0) return 1;
    if (budget > AOTX_SEQ_TICK_BUDGET) budget = AOTX_SEQ_TICK_BUDGET;
    hipLaunchKernelGGL(aotx_plan_kernel, dim3(1), dim3(64), 0, s, role, slots, tokens, stride,
                       budget, pool_pages, shape, aotx_state_device(), plan);
    AOTX_LAUNCH_CHECK();
    return 0;
}

extern "C" int aotx_decode_plan(unsigned int role, const aotx_plan_slot *slots, const int *tokens,
                                unsigned int stride, unsigned int budget, unsigned int pool_pages,
                                aotx_plan_state *plan, void *stream)
{
    return aotx_plan_launch(role, slots, tokens, stride, budget, pool_pages, plan,
                            aotx_stream(stream));
}

/* ---- commit (cuda/model/commit.cu:102-201) ------------------------------------------------ */

__global__ __launch_bounds__(64) void aotx_commit_kernel(unsigned int role, aotx_plan_slot *slots,
                                                         int *tokens, unsigned int stride,
                                                         const int *token, const unsigned int *draw,
                                                         aotx_state *st, aotx_plan_state *p,
                                                         aotx_token_record *rec, unsigned int cap)
{
    const unsigned int slot = threadIdx.x, lane = threadIdx.x;
    aotx_plan_slot &seq = slots[slot];
    unsigned int journal = 0u, from = 0u, extra = 0u, tok = 0u, mark = 0u;
    unsigned long long drawn = 0ull;
    if (seq.role == role) {
        if (seq.state == AOTX_SEQ_STATE_DONE) {
            if (aotx_kv_put(&st->kv, slot, 0u)) st->kv.count[slot] = 0u;   /* pages back */
            seq.state = AOTX_SEQ_STATE_FREE;
            p->asked[slot] = 0u;
        } else if (seq.state == AOTX_SEQ_STATE_PREFILL || seq.state == AOTX_SEQ_STATE_DECODE) {
            const unsigned int rows = p->rows[slot];
            const unsigned int list = seq.prompt + seq.sampled;
            const unsigned int end = p->first[slot] + rows;
            const unsigned int kept = p->kept[slot];
            journal = end > kept ? end - kept : 0u;
            from = kept;
            /* the draw of a sequence's last row follows the list once all of it is in pages */
            if (rows > 0u && end == list && list < AOTX_SEQ_MAX_TOKENS_PLAN) {
                const unsigned int place = p->place[slot];
                tok = (unsigned int)token[place];
                drawn = draw[place];
                extra = 1u;
            }
            if (rows > 0u) seq.state = end == list ? AOTX_SEQ_STATE_DECODE : AOTX_SEQ_STATE_PREFILL;
            if (extra != 0u) {
                mark = AOTX_TOKEN_SAMPLED;
                if (list < stride) tokens[(unsigned long long)slot * stride + list] = (int)tok;
                seq.sampled += 1u;
                seq.last = tok;
                seq.draw = drawn;
                if (tok == seq.stop || seq.sampled >= seq.limit || (seq.flags & AOTX_DECODE_MARK_STOP) != 0u
                    || list + 1u >= AOTX_SEQ_MAX_TOKENS_PLAN || list + 1u >= stride) {
                    mark |= AOTX_TOKEN_LAST;
                    seq.flags |= AOTX_TOKEN_LAST;
                    seq.state = AOTX_SEQ_STATE_DONE;
                }
            }
            p->kept[slot] = kept + journal + extra;
            if ((seq.flags & AOTX_DECODE_MARK_STOP) != 0u) seq.state = AOTX_SEQ_STATE_DONE;
        }
    }
    /* the tick's records: slots in order, each its list tokens then its sampled token */
    const unsigned int mine = journal + extra;
    const unsigned int scan = plan_scan(mine);
    const unsigned int first = scan - mine;
    /* the list tokens' records, written by the whole wave one slot at a time */
    const unsigned long long seed = seq.seed;
    for (unsigned int j = 0u; j < 64u; ++j) {
        const unsigned int n = __shfl(journal, (int)j, 64);
        if (n == 0u) continue;
        const unsigned int f0 = __shfl(first, (int)j, 64), at0 = __shfl(from, (int)j, 64);
        const unsigned long long sd = __shfl(seed, (int)j, 64);
        for (unsigned int i = lane; i < n; i += 64u) {
            const unsigned int r = f0 + i, at = at0 + i;
            if (r >= cap) break;
            aotx_token_record x;
            x.slot = j;
            x.token = at < stride ? (unsigned int)tokens[(unsigned long long)j * stride + at] : 0u;
            x.position = at;
            x.flags = AOTX_TOKEN_PROMPT;
            x.seed = sd;
            x.draw = 0ull;
            x.role = role;
            x.reserved = 0u;
            rec[r] = x;
        }
    }
    if (extra != 0u && first + journal < cap) {
        aotx_token_record x;
        x.slot = slot;
        x.token = tok;
        x.position = seq.prompt + seq.sampled - 1u;
        x.flags = mark;
        x.seed = seq.seed;
        x.draw = drawn;
        x.role = role;
        x.reserved = 0u;
        rec[first + journal] = x;
    }
    const unsigned int total = __shfl(scan, 63, 64);
    if (slot == 0u) {
        p->records = total < cap ? total : cap;
        p->dropped = total > cap ? total - cap : 0u;
    }
}

int aotx_commit_launch(unsigned int role, aotx_plan_slot *slots, int *tokens, unsigned int stride,
                       const int *token, const unsigned int *draw, aotx_plan_state *plan,
                       aotx_token_record *records, unsigned int capacity, hipStream_t s)
{
    if (role >= AOTX_MODEL_ROLES || slots == nullptr || tokens == nullptr || token == nullptr
        || draw == nullptr || plan == nullptr || stride == 0u || (records == nullptr && capacity != 0u))
        return 1;
    hipLaunchKernelGGL(aotx_commit_kernel, dim3(1), dim3(64), 0, s, role, slots, tokens, stride,
                       token, draw, aotx_state_device(), plan, records, capacity);
    AOTX_LAUNCH_CHECK();
    return 0;
}

extern "C" int aotx_decode_commit(unsigned int role, aotx_plan_slot *slots, int *tokens,
                                  unsigned int stride, const int *token, const unsigned int *draw,
                                  aotx_plan_state *plan, aotx_token_record *records,
                                  unsigned int capacity, void *stream)
{
    return aotx_commit_launch(role, slots, tokens, stride, token, draw, plan, records, capacity,
                              aotx_stream(stream));
}
