/* Routed experts (experts.hip): plan and launchers. */
#ifndef AOTX_EXPERTS_H
#define AOTX_EXPERTS_H

#include "aotx_internal.h"

struct aotx_expert_plan {
    const void *gate;             /* [experts][ffn][hidden/32] Q8_0 */
    const void *up;
    const void *down;             /* [experts][hidden][ffn/32] Q8_0 */
    unsigned int experts, used, hidden, ffn;
    unsigned int *list;           /* [experts][cap] routed slots */
    unsigned int *count;          /* [experts] */
    unsigned int cap;             /* tokens of the largest batch */
};

void aotx_launch_route(const float *router, const unsigned short *x, const unsigned int *m_dev,
                       unsigned int tokens, unsigned int hidden, unsigned int experts,
                       unsigned int used, float *prob, unsigned int *ids, hipStream_t s);

/* Slots (token * used + rank) of each expert in slot order: list[e * cap + i], count[e]. */
void aotx_launch_group(const unsigned int *ids, const unsigned int *m_dev, unsigned int tokens,
                       unsigned int used, unsigned int experts, unsigned int *list,
                       unsigned int *count, unsigned int cap, hipStream_t s);

/* Group the routed slots, then gate/up (+SwiGLU) into act [slots][ffn] and down into
 * y [slots][hidden] fp32. tokens = the capacity of the batch (passes of 32 rows). */
int aotx_launch_expert_ffn(const aotx_expert_plan &p, const unsigned short *x,
                           const unsigned int *m_dev, unsigned int tokens,
                           const unsigned int *ids, unsigned short *act, float *y,
                           hipStream_t s);

#endif
