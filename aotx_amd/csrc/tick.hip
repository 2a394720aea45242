/* The device side of a decode tick: the call block built from the tick plan, the per-row
 * logit adjustments of the sampler, and the restore of a slot from its token records.
 *
 * Reference: the tick graph of cuda/model/decode_host.cu:136-157 (plan -> forward ->
 * commit), the per-token value of the pick (cuda/model/sample.cu:277-319) and the apply of
 * a journal record (cuda/model/decode.cu:230-305).
 */
#include "tick.h"
#include "kvcache_dev.h"

/* The call block of the tick's step from the plan's batch (one thread): the rows read the
 * plan's ids, offset, agent and per-sequence sample in place. */
__global__ void aotx_tick_begin_kernel(aotx_step *step, const aotx_plan_state *p, int *token,
                                       unsigned int *draw)
{
    aotx_model_run run;
    __builtin_memset(&run, 0, sizeof run);
    run.ids = p->ids;
    run.offset = p->offset;
    run.agent = p->agent;
    run.token = token;
    run.draw = draw;
    run.seqs = p->seqs;
    run.tokens = p->tokens;
    run.rows = p->seqs;
    run.select = AOTX_MODEL_ROWS_LAST;
    run.top_p = 1.0f;
    run.how = p->how;
    step->run = run;
}

void aotx_launch_tick_begin(aotx_step *step, const aotx_plan_state *plan, int *token,
                            unsigned int *draw, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_tick_begin_kernel, dim3(1), dim3(1), 0, s, step, plan, token, draw);
    AOTX_LAUNCH_CHECK();
}

/* Whether a sample adjusts any logit: presence or frequency penalty, or a repeat penalty
 * over a window (the neutral values leave the model logit, sample.cu:283-285, :298-318). */
static __device__ __forceinline__ bool aotx_pen_on(const aotx_model_how &how)
{
    return how.presence_penalty != 0.0f || how.frequency_penalty != 0.0f
        || (how.repeat_window != 0u && how.repeat_penalty != 1.0f);
}

/* One workgroup per row of the step's batch. Every token of the sequence's list adds to
 * the token's count and raises its last position; then one of the list positions of each
 * distinct token (the first to set the claim bit) keeps the model logit in `raw` and
 * writes the adjusted value in its place, as the pick's value function gives it:
 *   value -= presence + frequency * count        (count > 0)
 *   value  = value > 0 ? value / repeat : value * repeat   (a position in the window)
 * The reference's compiler contracts `presence + frequency * count` into one fused
 * multiply-add; it is written as one here. */
__global__ __launch_bounds__(1024) void aotx_pen_adjust_kernel(aotx_pen_args a)
{
    const aotx_model_run *run = &a.step->run;
    const unsigned int r = blockIdx.x;
    if (r >= run->rows || run->how == nullptr) return;
    const unsigned int agent = run->agent[r];
    if (agent >= AOTX_SLOTS) return;
    const aotx_model_how how = run->how[r];
    if (!aotx_pen_on(how)) return;
    const aotx_plan_slot &seq = a.slots[agent];
    unsigned int list = seq.prompt + seq.sampled;
    if (list > a.stride) list = a.stride;
    const int *tok = a.tokens + (unsigned long long)agent * a.stride;
    unsigned int *count = a.count + (unsigned long long)r * a.vocab;
    unsigned int *last = a.last + (unsigned long long)r * a.vocab;
    float *raw = a.raw + (unsigned long long)r * a.vocab;
    float *row = a.logits + (unsigned long long)r * a.ld;
    for (unsigned int i = threadIdx.x; i < list; i += blockDim.x) {
        const unsigned int t = (unsigned int)tok[i];
        if (t >= a.vocab) continue;
        atomicAdd(&count[t], 1u);
        atomicMax(&last[t], i + 1u);
    }
    __syncthreads();
    const unsigned int first = list > how.repeat_window ? list - how.repeat_window : 0u;
    for (unsigned int i = threadIdx.x; i < list; i += blockDim.x) {
        const unsigned int t = (unsigned int)tok[i];
        if (t >= a.vocab) continue;
        const unsigned int was = atomicOr(&count[t], 0x80000000u);
        if ((was & 0x80000000u) != 0u) continue;
        const unsigned int c = was & 0x7FFFFFFFu;
        float value = row[t];
        raw[t] = value;
        if ((how.presence_penalty != 0.0f || how.frequency_penalty != 0.0f) && c != 0u)
            value -= __builtin_fmaf(how.frequency_penalty, (float)c, how.presence_penalty);
        const unsigned int at = __hip_atomic_load(&last[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (how.repeat_window != 0u && how.repeat_penalty != 1.0f && at - 1u >= first)
            value = value > 0.0f ? value / how.repeat_penalty : value * how.repeat_penalty;
        row[t] = value;
    }
}

/* After the pick: the model logits back in place and the counts back to zero. */
__global__ __launch_bounds__(1024) void aotx_pen_restore_kernel(aotx_pen_args a)
{
    const aotx_model_run *run = &a.step->run;
    const unsigned int r = blockIdx.x;
    if (r >= run->rows || run->how == nullptr) return;
    const unsigned int agent = run->agent[r];
    if (agent >= AOTX_SLOTS) return;
    if (!aotx_pen_on(run->how[r])) return;
    const aotx_plan_slot &seq = a.slots[agent];
    unsigned int list = seq.prompt + seq.sampled;
    if (list > a.stride) list = a.stride;
    const int *tok = a.tokens + (unsigned long long)agent * a.stride;
    unsigned int *count = a.count + (unsigned long long)r * a.vocab;
    unsigned int *last = a.last + (unsigned long long)r * a.vocab;
    const float *raw = a.raw + (unsigned long long)r * a.vocab;
    float *row = a.logits + (unsigned long long)r * a.ld;
    for (unsigned int i = threadIdx.x; i < list; i += blockDim.x) {
        const unsigned int t = (unsigned int)tok[i];
        if (t >= a.vocab) continue;
        if (atomicExch(&count[t], 0u) != 0u) {
            row[t] = raw[t];
            last[t] = 0u;
        }
    }
}

void aotx_launch_pen(const aotx_pen_args &a, unsigned int rows_cap, int restore, hipStream_t s)
{
    if (restore)
        hipLaunchKernelGGL(aotx_pen_restore_kernel, dim3(rows_cap), dim3(1024), 0, s, a);
    else
        hipLaunchKernelGGL(aotx_pen_adjust_kernel, dim3(rows_cap), dim3(1024), 0, s, a);
    AOTX_LAUNCH_CHECK();
}

/* Apply token records in order (cuda/model/decode.cu:230-305), one thread:
 *   - a record at position 0 on a slot that already kept records of a sequence shuts it
 *     (its pages go back, the slot is free);
 *   - a free slot opens on a record at position 0 (any other is refused), with the slot's
 *     own limit, stop and sample and the record's seed;
 *   - a prompt record below the slot's prompt (a slot whose open already put the prompt in
 *     its list) must name the token standing there: it confirms it and adds nothing;
 *   - otherwise a record must continue the slot's list: a prompt record puts its token in
 *     the list and extends the prompt; a sampled record appends its token with its seed and
 *     draw, and the slot's draw counter continues after that draw; the last record ends
 *     the slot.
 * The pages of an opened slot are empty, so the next plans prefill the whole list again
 * (the plan's page check asks for the pages). A refused record is counted. */
__global__ void aotx_seq_apply_kernel(unsigned int role, aotx_plan_slot *slots, int *tokens,
                                      unsigned int stride, aotx_plan_state *p,
                                      const aotx_token_record *rec, unsigned int n,
                                      aotx_state *st)
{
    for (unsigned int k = 0u; k < n; ++k) {
        const aotx_token_record b = rec[k];
        const unsigned int slot = b.slot;
        if (slot >= AOTX_SLOTS || b.role != role || b.position >= AOTX_SEQ_MAX_TOKENS_PLAN
            || b.position >= stride) {
            p->refused += 1u;
            continue;
        }
        aotx_plan_slot &seq = slots[slot];
        if (b.position == 0u && seq.state != AOTX_SEQ_STATE_FREE && p->kept[slot] != 0u) {
            if (st->kv.count[slot] != 0u && aotx_kv_put(&st->kv, slot, 0u)) st->kv.count[slot] = 0u;
            seq.state = AOTX_SEQ_STATE_FREE;
            p->asked[slot] = 0u;
        }
        if (seq.state == AOTX_SEQ_STATE_FREE) {
            if (b.position != 0u) {
                p->refused += 1u;
                continue;
            }
            seq.state = AOTX_SEQ_STATE_PREFILL;
            seq.role = role;
            seq.prompt = 0u;
            seq.sampled = 0u;
            seq.seed = b.seed;
            seq.flags = 0u;
            seq.last = 0u;
            seq.draw = 0ull;
            st->seen[slot] = 0u;
            st->draw[slot] = 0u;
            p->asked[slot] = 0u;
            p->kept[slot] = 0u;
        }
        int *list = tokens + (unsigned long long)slot * stride;
        if ((b.flags & AOTX_TOKEN_PROMPT) != 0u && b.position < seq.prompt) {
            if (list[b.position] != (int)b.token) {
                p->refused += 1u;
                continue;
            }
            p->kept[slot] = b.position + 1u;
            continue;
        }
        if (b.position != seq.prompt + seq.sampled) {
            p->refused += 1u;
            continue;
        }
        list[b.position] = (int)b.token;
        seq.last = b.token;
        if ((b.flags & AOTX_TOKEN_SAMPLED) != 0u) {
            seq.sampled = b.position + 1u - seq.prompt;
            seq.seed = b.seed;
            seq.draw = b.draw;
            st->draw[slot] = (unsigned int)b.draw + 1u;
        } else {
            seq.prompt = b.position + 1u;
        }
        p->kept[slot] = b.position + 1u;
        if ((b.flags & AOTX_TOKEN_LAST) != 0u) {
            seq.flags |= AOTX_TOKEN_LAST;
            seq.state = AOTX_SEQ_STATE_DONE;
        }
    }
}

extern "C" int aotx_seq_apply(unsigned int role, aotx_plan_slot *slots, int *tokens,
                              unsigned int stride, aotx_plan_state *plan,
                              const aotx_token_record *records, unsigned int count, void *stream)
{
    if (role >= AOTX_MODEL_ROLES || slots == nullptr || tokens == nullptr || plan == nullptr
        || stride == 0u || (records == nullptr && count != 0u))
        return 1;
    if (count == 0u) return 0;
    hipLaunchKernelGGL(aotx_seq_apply_kernel, dim3(1), dim3(1), 0, aotx_stream(stream), role,
                       slots, tokens, stride, plan, records, count, aotx_state_device());
    AOTX_LAUNCH_CHECK();
    return 0;
}
