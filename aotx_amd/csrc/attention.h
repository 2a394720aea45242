/* Paged decode attention (attention.hip): launch interface for the model runtime. */
#ifndef AOTX_ATTENTION_H
#define AOTX_ATTENTION_H

#include "aotx_internal.h"

/* Chunks per (token, KV head) for a launch of `tokens` rows. */
unsigned int aotx_attn_splits(unsigned int tokens, unsigned int kv_heads,
                              unsigned int max_context);
/* Bytes of the chunk partials of such a launch. */
size_t aotx_attn_scratch(unsigned int tokens, unsigned int kv_heads, unsigned int splits,
                         unsigned int group, unsigned int head_dim);
struct aotx_attn_args;
/* Launches of at least this many tokens (more than the sequence slots, so with prompt
 * pieces) run the piece kernel: the queries of a sequence share their key reads. */
#define AOTX_ATTN_PIECE_TOKENS 128u
/* The arguments of a launch over these operands; 1 when the shape is refused. */
int aotx_attend_plan(aotx_attn_args *args, const unsigned short *q, unsigned short *out,
                     const unsigned int *pos, const unsigned int *agent,
                     const unsigned int *m_dev, unsigned int tokens, unsigned int heads,
                     unsigned int kv_heads, unsigned int head_dim, unsigned int layer,
                     unsigned int layers, unsigned int max_context, float *partial,
                     unsigned int *count);
/* q/out fp16 [tokens][heads][d] (out_frag: out in the fragment layout of aotx_xfrag_at,
 * for at most 32 tokens of decode rows); m_dev = device token count (or null); partial = the
 * caller's chunk buffer and count its [tokens * kv_heads] arrival counters, zeroed once
 * at allocation and left at zero by every launch (either null for the library scratch). */
int aotx_attend_launch(const unsigned short *q, unsigned short *out, const unsigned int *pos,
                       const unsigned int *agent, const unsigned int *m_dev,
                       unsigned int tokens, unsigned int heads, unsigned int kv_heads,
                       unsigned int head_dim, unsigned int layer, unsigned int layers,
                       unsigned int max_context, float *partial, unsigned int *count,
                       hipStream_t stream, unsigned int out_frag = 0u);

#endif
