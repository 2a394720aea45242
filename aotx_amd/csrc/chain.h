/* The layer chain (chain.hip): every stage of a narrow decode step's layers in one launch.
 *
 * A stage is one product or the attention of one layer; its items are the workgroups the
 * standalone kernel would launch. Each workgroup of the chain takes items w, w + grid, ...
 * of every stage in order. Before computing an item it waits until the stage it depends
 * on has counted all of its items done; the weight loads of the item (which depend on no
 * earlier stage) are issued before that wait, so the weight stream of a stage overlaps
 * the tail of the one before, and no launch boundary separates them.
 */
#ifndef AOTX_CHAIN_H
#define AOTX_CHAIN_H

#include "attention_dev.h"
#include "rgemv.h"

enum {
    AOTX_CHAIN_TILE = 0,       /* product, one 16-row tile per item, 2 quads per load */
    AOTX_CHAIN_TILE_LONG = 1,  /* the same, 7 quads per load (long k: 14 quads per wave) */
    AOTX_CHAIN_PAIR = 2,       /* gate/up product with SwiGLU, one tile pair per item */
    AOTX_CHAIN_ATTEND = 3      /* attention, d = 128 and 4 query heads per KV head */
};

struct aotx_chain_stage {
    unsigned int kind;
    unsigned int items;
    unsigned int wait;         /* 1 + the stage this one waits for, or 0 */
    unsigned int wait_items;   /* that stage's item count */
    aotx_rgemv_args g;
    aotx_attn_args t;
};

/* Largest dynamic LDS a chain stage may plan for. */
#define AOTX_CHAIN_LDS (64u * 1024u)
/* Words of the arrival counters of a chain of n stages (zero between launches). */
static inline unsigned int aotx_chain_words(unsigned int n) { return n + 2u; }

/* Workgroups of a chain launch with `lds` dynamic bytes: all of them resident at once
 * (0 when the device cannot hold one per CU). */
unsigned int aotx_chain_grid(size_t lds);
/* Launch a chain of n stages from the device table; `done` = aotx_chain_words(n) zeroed
 * words; `stall` (host-visible) is set to 1 if a wait ran out of time. */
void aotx_chain_launch(const aotx_chain_stage *table, unsigned int n, unsigned int *done,
                       unsigned int *stall, size_t lds, hipStream_t stream);

#endif
