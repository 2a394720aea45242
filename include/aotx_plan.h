/* The tick plan: the row packing that builds the batch of one decode step from the
 * sequence slots (the reference's aotx_decode_plan, cuda/model/plan.cu:54-199, with the
 * page check of cuda/model/decode_state.cuh:75-107).
 *
 * The reference's plan reads its slots from the device sequence store and its gates
 * (ready, scheduler hold, journal replay, role rotation) from device globals. Here the
 * caller hands the slot fields the packing reads as a device table and calls the plan
 * only on ticks that run; the batch it writes (ids, offset, agent, how) is what
 * aotx_model_sample / aotx_model_launch take, in device memory, with no host copy. */
#ifndef AOTX_PLAN_H
#define AOTX_PLAN_H

#include "aotx_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define AOTX_SEQ_TICK_BUDGET   512u   /* rows of one tick at most: cuda/model/decode.cuh:15 */

/* Slot states: cuda/model/decode.cuh:19-22. */
#define AOTX_SEQ_STATE_FREE    0u
#define AOTX_SEQ_STATE_PREFILL 1u
#define AOTX_SEQ_STATE_DECODE  2u
#define AOTX_SEQ_STATE_DONE    3u

/* The fields of a sequence slot the plan reads (the reference's aotx_seq: state, role,
 * prompt, sampled, limit, page_limit, seed, sample; read at plan.cu:74-156). */
typedef struct aotx_plan_slot {
    unsigned int state;
    unsigned int role;
    unsigned int prompt;       /* prompt tokens of the list */
    unsigned int sampled;      /* tokens sampled so far (the list holds prompt + sampled) */
    unsigned int limit;        /* reply tokens at most: pages cover prompt + limit */
    unsigned int page_limit;   /* pages the slot may hold (0: no limit) */
    unsigned long long seed;
    aotx_model_how sample;
    unsigned int stop;         /* the token that ends the reply (AOTX_PLAN_NO_STOP: none) */
    unsigned int flags;        /* AOTX_TOKEN_LAST once ended; AOTX_DECODE_MARK_STOP: stop now */
    unsigned int last;         /* the last sampled token */
    unsigned int reserved;
    unsigned long long draw;   /* the draw count of that token */
} aotx_plan_slot;

#define AOTX_PLAN_NO_STOP      0xFFFFFFFFu
#define AOTX_SEQ_MAX_TOKENS_PLAN 8192u     /* a list's tokens at most (AOTX_SEQ_MAX_TOKENS) */
#define AOTX_DECODE_MARK_STOP  0x0100u    /* cuda/model/decode_state.cuh:22 */
/* Token record flags: cuda/seam/wire.h:186-188. */
#define AOTX_TOKEN_PROMPT      0x0001u
#define AOTX_TOKEN_SAMPLED     0x0002u
#define AOTX_TOKEN_LAST        0x0004u

/* One token record of a tick (the reference's aotx_token_body, cuda/seam/wire.h:190-200,
 * without the detokenized text): what a journal replay needs to rebuild the list. */
typedef struct aotx_token_record {
    unsigned int slot;
    unsigned int token;
    unsigned int position;     /* in the slot's list, from 0 */
    unsigned int flags;        /* AOTX_TOKEN_* */
    unsigned long long seed;
    unsigned long long draw;   /* 0 for a prompt token */
    unsigned int role;
    unsigned int reserved;
} aotx_token_record;

/* The batch of one tick and the plan's marks (cuda/model/decode_state.cuh:35-55 without
 * the multimodal input rows and the role/replay gates; asked is aotx_seq_asked,
 * decode_state.cuh:67-70). Device memory, zeroed by the caller before the first tick. */
typedef struct aotx_plan_state {
    int ids[AOTX_SEQ_TICK_BUDGET];          /* the token of every row of the batch */
    unsigned int offset[AOTX_SLOTS + 1u];   /* the first row of each sequence */
    unsigned int agent[AOTX_SLOTS];         /* the slot of each sequence */
    aotx_model_how how[AOTX_SLOTS];         /* the sample of each sequence (seed = slot seed) */
    unsigned int rows[AOTX_SLOTS];          /* rows each slot gave this tick */
    unsigned int first[AOTX_SLOTS];         /* the list position of the first of them */
    unsigned int place[AOTX_SLOTS];         /* the slot's sequence, or AOTX_SLOTS */
    unsigned int asked[AOTX_SLOTS];         /* pages each slot has asked the pool for */
    unsigned int kept[AOTX_SLOTS];          /* tokens of each list already recorded */
    unsigned int cursor[AOTX_MODEL_ROLES];  /* the rotating first slot of each role */
    unsigned int seqs;                      /* sequences of this tick's batch */
    unsigned int tokens;                    /* rows of this tick's batch */
    unsigned int waited;                    /* prefill pieces that got no room, summed */
    unsigned int short_of;                  /* slots that waited for pages, summed */
    unsigned long long steps;               /* ticks that gave a batch of one row or more */
    unsigned int records;                   /* token records of the last commit (at most the
                                               capacity given to it) */
    unsigned int dropped;                   /* records of the last commit past the capacity */
    unsigned int refused;                   /* slots and records refused, summed: a prompt
                                               longer than the list stride, a record that
                                               does not continue its slot */
    unsigned int reserved;
} aotx_plan_state;

/* Plan one tick of `role` (cuda/model/plan.cu:54-199): every slot of the role in state
 * PREFILL or DECODE whose list (prompt + sampled) has tokens no page holds yet (the
 * device's seen count) and whose pages cover prompt + limit takes part; a slot short of
 * pages asks the pool (the device request queue, aotx_kv_serve answers it) and waits.
 * Decode slots give one row each, first, in slot order from the role's cursor; prefill
 * slots then take the rest of `budget` (at most AOTX_SEQ_TICK_BUDGET) in the same order,
 * and the piece that crosses its end is cut. slots [AOTX_SLOTS], tokens [AOTX_SLOTS][stride]
 * (each slot's list) and plan are device pointers; pool_pages is the pool's page count
 * (the map's limit; a partly served request is asked again while pages are free).
 * Returns 1 for a role with no model described or a bad argument. Asynchronous on the
 * stream. */
int aotx_decode_plan(unsigned int role, const aotx_plan_slot *slots, const int *tokens,
                     unsigned int stride, unsigned int budget, unsigned int pool_pages,
                     aotx_plan_state *plan, void *stream);

/* Close the tick of `role` (cuda/model/commit.cu:102-201) after the step ran on the plan's
 * batch: token[place] and draw[place] (device) are the step's outputs. Per slot of the
 * role, in slot order: a DONE slot gives its pages back (a release request) and becomes
 * FREE; a slot that gave rows moves to DECODE when its whole list is in the pages (else
 * stays PREFILL), and then takes the sampled token into its list (slots, tokens [stride]
 * are updated in place), ending (DONE, AOTX_TOKEN_LAST) on its stop token, its limit, the
 * list bound or a stop mark. The records of the tick (the list tokens not yet recorded,
 * then the sampled token) go to records[0 .. plan->records), slots in order, at most
 * capacity. One wave; asynchronous on the stream. Returns 1 for a bad argument. */
int aotx_decode_commit(unsigned int role, aotx_plan_slot *slots, int *tokens,
                       unsigned int stride, const int *token, const unsigned int *draw,
                       aotx_plan_state *plan, aotx_token_record *records,
                       unsigned int capacity, void *stream);

/* One decode tick of `role` as one captured HIP graph (the tick graph of
 * cuda/model/decode_host.cu:136-157): aotx_decode_plan, then the model step over the plan's
 * batch in device memory (no host copy of the batch), each sequence sampled with its own
 * sample (plan->how: temperature, top-k, top-p, min-p, seed) and with the presence,
 * frequency and repeat penalties of that sample over the slot's list (the pick's value
 * function, cuda/model/sample.cu:277-319), then aotx_decode_commit. The arguments are those
 * of the plan and the commit; budget is at most the role's open token capacity. logits
 * (device, may be null) receives the model logits of each sequence's last row,
 * [64][vocab] room. The graph of budget's token bucket is captured on first use and again
 * when an operand changes. Synchronous. The caller serves the pool's page requests
 * (aotx_kv_serve) between ticks. Returns 1 for a bad argument or a role not open. Not
 * built: the reply-wrap thinking mask of the value function (the descriptor carries no
 * wrap tokens). */
int aotx_decode_tick(unsigned int role, aotx_plan_slot *slots, int *tokens, unsigned int stride,
                     unsigned int budget, unsigned int pool_pages, aotx_plan_state *plan,
                     aotx_token_record *records, unsigned int capacity, float *logits);

/* Restore slots of `role` from token records, in order (the reference's aotx_seq_apply,
 * cuda/model/decode.cu:230-305): a record at position 0 opens its slot (a slot that held a
 * sequence gives its pages back first) keeping the slot's limit, stop and sample and taking
 * the record's seed; prompt records rebuild the prompt, sampled records append their token
 * and set the slot's draw counter to the record's draw + 1, so the next sample continues
 * the same Philox stream; a LAST record ends the slot. The slot's pages are empty after an
 * open, so the following ticks prefill the whole list again. A record that does not
 * continue its slot is refused and counted in plan->refused. Device pointers; one thread,
 * asynchronous on the stream. Returns 1 for a bad argument. */
int aotx_seq_apply(unsigned int role, aotx_plan_slot *slots, int *tokens, unsigned int stride,
                   aotx_plan_state *plan, const aotx_token_record *records, unsigned int count,
                   void *stream);

/* Pages a slot of `role` needs for a context of `context` positions (the reference's
 * aotx_kvl_pages over the role's KV shape, cuda/model/kv_layout.cuh); 0 when the role has
 * no model described. */
unsigned int aotx_model_kv_pages(unsigned int role, unsigned int context);

#ifdef __cplusplus
}
#endif

#endif
