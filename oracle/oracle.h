/* CPU oracle of the AOTX-1 token loop — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's algorithms on this path, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker. Nothing in
 * the product (aotx_amd/, include/) links, loads or calls it.
 *
 * Each function cites the reference file:line it restates. Pinning (what checks each
 * function against something other than itself) is listed in the test files:
 *   orc_f32_to_f16 / orc_f16_to_f32  — exhaustive fp16 round trip + numpy float16 casts
 *   orc_q8_*                          — numpy double product; transposed-operand control
 *   orc_philox                        — Random123 known answers (tests/rng_test.cu:61-75)
 *   orc_pick                          — allowed-set restatement (tests/sample_test.cu:177-224),
 *                                       chi-square, argmax by numpy, brute force top-k
 *   orc_route                         — double softmax + rank (tests/expert_test.cu:118-152)
 *   orc_attend_*                      — two-pass textbook softmax attention in numpy
 *   orc_model_*                       — composed from the pinned pieces above; its
 *                                       forward is compared to a numpy float64 forward
 */
#ifndef AOTX_ORACLE_H
#define AOTX_ORACLE_H

#include <stdint.h>

#include "../include/aotx_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
float orc_round_half(float f);

/* half(q * scale) of element j of one Q8_0 row (tests/matrix_test.cu:84-96). */
float orc_q8_value(const uint8_t *row, unsigned int j);

/* y[m][n] in double from half(q*scale) and fp16 x (tests/matrix_test.cu:224-239).
 * swap != 0 gives the transposed-operand control (needs n == k). */
void orc_q8_gemv_f64(const uint8_t *w, unsigned int n, unsigned int k, const uint16_t *x,
                     unsigned int m, double *y, int swap);

/* y[m][n] in fp32 the way the reference's memory-bound product sums: w = fp32(scale) * q
 * (cuda/model/matrix.cuh:499-512), acc += w * x per k in order (cuda/model/gemv.cuh:68-98),
 * one sum per output here. threads > 1 splits rows over threads (CPU baseline). */
void orc_q8_gemv_f32(const uint8_t *w, unsigned int n, unsigned int k, const uint16_t *x,
                     unsigned int m, float *y, unsigned int threads);

/* Philox4x32-10 (cuda/rng/rng.cuh:29-85; tests/rng_test.cu:33-57). */
void orc_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* (seed, stream, lane, position) -> word .x, then (word >> 8) * 2^-24
 * (cuda/rng/rng.cuh:72-94). */
float orc_rng_unit(uint64_t seed, uint32_t stream, uint32_t lane, uint64_t position);

/* One row of the sampler (cuda/model/sample.cu:456-765 with how == null): greedy when
 * temperature <= 0, else the 42-span bucket search, the candidate sort, top-k, min-p,
 * top-p on T=1 probabilities, temperature, and the Philox inverse CDF at
 * (seed, agent, lane 0, position). Writes the token; *count_out (may be null) gets the
 * candidate count and *taken_out the size of the allowed set. */
int orc_pick(const float *row, unsigned int vocab, unsigned int top_k, float top_p,
             float min_p, float temperature, uint64_t seed, unsigned int agent,
             uint64_t position, unsigned int *count_out, unsigned int *taken_out,
             unsigned int *allowed_out);

/* Router (cuda/model/experts.cu:10-75): prob[t][e] = softmax over every expert of the
 * fp32 router row . half x (double arithmetic, as tests/expert_test.cu:118-152 checks);
 * ids[t][r] = rank r, ties to the lower index. */
void orc_route(const float *router, const uint16_t *x, unsigned int tokens,
               unsigned int hidden, unsigned int experts, unsigned int used, float *prob,
               unsigned int *ids);

/* Online-softmax attention of one query head over keys/values 0..last (inclusive):
 * fp16-valued q, k, v given as floats; scale 1/sqrt(d); out = half(sum / mass)
 * (cuda/model/attention.cu:66-129; tests/model_ref.h:356-390). */
void orc_attend_one(const float *q, const float *keys, const float *values,
                    unsigned int stride, unsigned int last, unsigned int d, float *out);

/* ---- whole model on the CPU (tests/model_ref.h:301-427, generalised) ----
 * desc: the same descriptor the library takes; weights: a host copy of the weights
 * region. The oracle keeps each slot's keys and values in plain arrays. */
typedef struct orc_model orc_model;
orc_model *orc_model_new(const aotx_model_desc *desc, const uint8_t *weights,
                         unsigned int slots, unsigned int max_context, unsigned int threads);
void orc_model_free(orc_model *m);
void orc_model_forget(orc_model *m);
/* One pass over a batch (ids/offset/agent as in aotx_model_run). logits receives one row
 * per sequence (its last token) [seqs][vocab]. Returns 0, or 1 when a slot overflows. */
int orc_model_step(orc_model *m, const int *ids, const unsigned int *offset,
                   unsigned int seqs, const unsigned int *agent, float *logits);
/* Seat a slot at `position` with random fp16 keys/values in every layer (the CPU
 * baseline's stand-in for a prefilled context; not a parity function). */
int orc_model_seat(orc_model *m, unsigned int slot, unsigned int position, uint64_t seed);
/* The xnorm (half values as float) of the last row of each sequence of the last step. */
const float *orc_model_last_xnorm(const orc_model *m);
/* The residual row of each sequence's last token after every layer of the last step,
 * [layers][seqs][hidden]. */
const float *orc_model_last_resid(const orc_model *m);
const float *orc_model_last_route(const orc_model *m, const unsigned int **ids,
                                  unsigned int *tokens);
const uint16_t *orc_model_cache(const orc_model *m, unsigned int which);
void orc_pick_adjust(float *row, unsigned int vocab, const int *list, unsigned int n,
                     float presence, float frequency, float repeat_penalty,
                     unsigned int repeat_window);

#ifdef __cplusplus
}
#endif

#endif
