/* Device side of the page pool's request queue, shared by the pool (kvcache.hip) and the
 * tick plan (plan.hip). */
#ifndef AOTX_KVCACHE_DEV_H
#define AOTX_KVCACHE_DEV_H

#include "aotx_internal.h"

/* One request into the queue (cuda/kvcache/pages.cu:13-57). */
static __device__ __forceinline__ int aotx_kv_put(aotx_kv_table *kv, unsigned int agent, unsigned int pages)
{
    if (agent >= AOTX_SLOTS || pages > AOTX_KV_PAGES_EACH) {
        atomicAdd(&kv->refused, 1u);
        return 0;
    }
    unsigned int at = atomicAdd(&kv->made, 0u);
    for (;;) {
        if (at - atomicAdd(&kv->served, 0u) >= AOTX_KV_QUEUE_MAX) {
            atomicAdd(&kv->refused, 1u);
            return 0;
        }
        unsigned int was = atomicCAS(&kv->made, at, at + 1u);
        if (was == at) break;
        at = was;
    }
    kv->queue[at & (AOTX_KV_QUEUE_MAX - 1u)].agent = agent;
    kv->queue[at & (AOTX_KV_QUEUE_MAX - 1u)].pages = pages;
    __threadfence();                 /* the entry is visible before later work that reads it */
    return 1;
}

#endif
