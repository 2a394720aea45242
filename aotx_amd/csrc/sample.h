/* Sampler (sample.hip): launch interface for the model runtime. */
#ifndef AOTX_SAMPLE_H
#define AOTX_SAMPLE_H

#include "aotx_internal.h"

void aotx_launch_pick(const float *logits, unsigned int ld, unsigned int vocab,
                      const unsigned int *rows_dev, unsigned int rows,
                      const unsigned int *agent, const aotx_model_how *how,
                      unsigned int top_k, float top_p, float temperature,
                      unsigned long long seed, int *token, unsigned int *draw,
                      const aotx_model_run *run, unsigned int *best, hipStream_t s);
/* Bytes of the sampler's buffer (`best`) for `rows` rows of `vocab` logits: the slices'
 * largest logits, the first-pass bucket counts (zeroed once at allocation, left at zero by
 * every call) and the rows' exponentials. */
size_t aotx_pick_scratch(unsigned int rows, unsigned int vocab);

#endif
