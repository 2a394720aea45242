/* Device side of a decode tick (tick.hip): the call block from the tick plan, the
 * sampler's per-row logit adjustments and the restore of slots from token records. */
#ifndef AOTX_TICK_H
#define AOTX_TICK_H

#include "aotx_internal.h"
#include "norm.h"
#include "../../include/aotx_plan.h"

/* Operands of the logit adjustment around the pick: the step's call block (rows, agent,
 * per-row sample), the slot table and lists, the logits [rows][ld], and three scratch
 * arrays [rows][vocab] (counts and last positions zero between calls). */
struct aotx_pen_args {
    const aotx_step *step;
    const aotx_plan_slot *slots;
    const int *tokens;
    unsigned int stride;
    float *logits;
    unsigned int ld;
    unsigned int vocab;
    unsigned int *count;
    unsigned int *last;
    float *raw;
};

void aotx_launch_tick_begin(aotx_step *step, const aotx_plan_state *plan, int *token,
                            unsigned int *draw, hipStream_t s);
/* restore = 0: the adjusted values in place; 1: the model values back. */
void aotx_launch_pen(const aotx_pen_args &a, unsigned int rows_cap, int restore, hipStream_t s);

/* The plan and commit kernels of plan.hip, for the tick graph. */
int aotx_plan_launch(unsigned int role, const aotx_plan_slot *slots, const int *tokens,
                     unsigned int stride, unsigned int budget, unsigned int pool_pages,
                     aotx_plan_state *plan, hipStream_t s);
int aotx_commit_launch(unsigned int role, aotx_plan_slot *slots, int *tokens, unsigned int stride,
                       const int *token, const unsigned int *draw, aotx_plan_state *plan,
                       aotx_token_record *records, unsigned int capacity, hipStream_t s);

#endif
