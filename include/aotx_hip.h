/* aotx_hip.h — C ABI of the MI355X (gfx950) language-model token loop.
 *
 * This header is the drop-in boundary. Every entry point takes plain pointers and sizes;
 * no C++ or framework type appears in a signature. The model-step surface keeps the names,
 * argument order, argument meaning and return codes of the reference's operator surface
 * (cuda/model/forward.cuh:325-372, cuda/kvcache/kvcache.cuh:100-111). The kernel-level
 * entry points below it replace the reference's `__global__` matrix, attention, sampler and
 * expert kernels for callers that drive them one at a time (tests, tools, benchmarks).
 *
 * Return codes: 0 = ran, 1 = refused (bounds, empty sequence, over capacity), as in the
 * reference (cuda/model/model_host.cu:97-99, :158-166; cuda/model/call_host.cu:19-30).
 * A failing HIP runtime call prints its site and exits the process, as the reference's
 * check does (cuda/boot/check.h:13-33).
 *
 * Threading: one host thread per runtime; not re-entrant per role.
 * Pointers: "device" = device memory of the current HIP device; "host" = host memory.
 */
#ifndef AOTX_HIP_H
#define AOTX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------
 * Capacities of the MI355X profile. The reference takes them from a compile-time profile
 * (cuda/profile/12g.cuh:17-57). 288 GB of HBM3E per GPU lets the pool be far larger than
 * the reference's 2 GiB range, so the page pool size is chosen at aotx_kv_open time.
 * ------------------------------------------------------------------------------------- */
#define AOTX_SLOTS             64u
#define AOTX_SEQ_MAX_TOKENS    8192u
#define AOTX_KV_PAGES_EACH     640u
#define AOTX_KV_PAGES_MAX      65536u          /* largest pool: 128 GiB of 2 MiB pages */
#define AOTX_KV_PAGE_BYTES     (2ull * 1024ull * 1024ull)
#define AOTX_KV_QUEUE_MAX      256u
#define AOTX_KV_HEADER_BYTES   16u
#define AOTX_KV_TYPE_FP16      1u

/* Layout block of the paged KV cache (cuda/model/kv_layout.cuh:17-23): 16 positions of
 * one layer, [K heads][16][d] then [V heads][16][d] in fp16, packed into 2 MiB pages
 * after a 256-byte header. */
#define AOTX_KVL_BLOCK         16u
#define AOTX_KVL_HEADER        256u

#define AOTX_MODEL_MAX_TOKENS  512u            /* cuda/model/forward.cuh:19 */
#define AOTX_MODEL_MAX_LAYERS  64u             /* cuda/model/names.h:15 */
#define AOTX_LAYER_TENSOR_SLOTS 14u            /* cuda/model/kinds_data.h:209 (widest span) */
#define AOTX_LAYER_EXPERTS_MAX 256u            /* cuda/model/kinds_data.h:34 */
#define AOTX_MODEL_PICK_MAX    256u            /* cuda/model/forward.cuh:68 */
#define AOTX_MODEL_PICK_SPAN   42.0f           /* cuda/model/forward.cuh:72 */
#define AOTX_MODEL_STEERS      2u              /* cuda/model/forward.cuh:80 (affect off) */
#define AOTX_MODEL_CONDUCT_NONE 0xFFFFFFFFu

/* Roles (cuda/model/model.cuh:16-21). The language roles end in the vocabulary head and
 * the sampler; the embedding role in the pooled unit row, the rank role in the score. */
#define AOTX_MODEL_EMBEDDING      0u
#define AOTX_MODEL_RERANKER       1u
#define AOTX_MODEL_LANGUAGE       2u
#define AOTX_MODEL_LANGUAGE_Q4    3u
#define AOTX_MODEL_LANGUAGE_AUDIO 4u
#define AOTX_MODEL_ROLES          5u

/* Weight block types (cuda/model/model.cuh:25-36). */
#define AOTX_WEIGHT_F32        0u
#define AOTX_WEIGHT_F16        1u
#define AOTX_WEIGHT_Q4_0       2u
#define AOTX_WEIGHT_Q8_0       8u

/* Layer kinds (cuda/model/kinds_data.h:11-18). */
#define AOTX_LAYER_KIND_ATTENTION            0u
#define AOTX_LAYER_KIND_ATTENTION_NO_QK_NORM 1u
#define AOTX_LAYER_KIND_FFN_EXPERTS          2u

/* Tensor slots of one layer (cuda/model/kinds_data.h:79-93). */
#define AOTX_SLOT_ATTN_NORM    0u
#define AOTX_SLOT_ATTN_Q       1u
#define AOTX_SLOT_ATTN_K       2u
#define AOTX_SLOT_ATTN_V       3u
#define AOTX_SLOT_ATTN_O       4u
#define AOTX_ATTENTION_Q_NORM  5u
#define AOTX_ATTENTION_K_NORM  6u
#define AOTX_SLOT_FFN_NORM     7u
#define AOTX_SLOT_FFN_GATE     8u
#define AOTX_SLOT_FFN_UP       9u
#define AOTX_SLOT_FFN_DOWN     10u
#define AOTX_EXPERT_ROUTER     11u

#define AOTX_ROPE_PAIRS_SPLIT    0u            /* cuda/model/rope_families.h:11-12 */
#define AOTX_ROPE_PAIRS_ADJACENT 1u

#define AOTX_MODEL_ABSENT      (~0ull)
#define AOTX_MODEL_ROWS_ALL    0u
#define AOTX_MODEL_ROWS_LAST   1u

/* ---------------------------------------------------------------------------------------
 * Data structures, layout-compatible with the reference's affect-off build.
 * ------------------------------------------------------------------------------------- */

/* cuda/model/model.cuh:42-44 */
typedef struct aotx_model_layer {
    unsigned long long offset[AOTX_LAYER_TENSOR_SLOTS];
} aotx_model_layer;

/* cuda/model/model.cuh:50-86. Offsets are bytes from the start of the weights region. */
typedef struct aotx_model_desc {
    unsigned int role;
    unsigned int layers;
    unsigned int probe_layer;
    unsigned int hidden;
    unsigned int ffn;
    unsigned int heads;
    unsigned int kv_heads;
    unsigned int head_dim;
    unsigned int vocab;
    unsigned int context;
    unsigned int weight_type;
    unsigned int embd_type;
    unsigned int tied_output;
    unsigned int pooling;
    float rope_theta;
    unsigned char kind[AOTX_MODEL_MAX_LAYERS];
    float rms_eps;
    unsigned int rope_pairs;
    unsigned int expert_count;
    unsigned int expert_used_count;
    unsigned int delta_dim;
    unsigned int delta_heads;
    unsigned int delta_key_heads;
    unsigned int delta_conv;
    unsigned int delta_inner;
    unsigned int rope_dim;
    unsigned long long token_embd;
    unsigned long long output_norm;
    unsigned long long output;
    unsigned long long cls_output;
    unsigned long long rope_freqs;
    aotx_model_layer layer[AOTX_MODEL_MAX_LAYERS];
    unsigned char layer_type[AOTX_MODEL_MAX_LAYERS][AOTX_LAYER_TENSOR_SLOTS];
} aotx_model_desc;

/* cuda/model/forward.cuh:88-108 (affect off). */
typedef struct aotx_model_how {
    float temperature;
    unsigned int top_k;
    float top_p;
    float min_p;
    float repeat_penalty;
    unsigned int repeat_window;
    float presence_penalty;
    float frequency_penalty;
    unsigned long long seed;
    int think_limit;
    unsigned int steer[AOTX_MODEL_STEERS];
    float steer_strength[AOTX_MODEL_STEERS];
    unsigned int steer_from;
    unsigned int voice;
    unsigned int affect;
    float voice_scale;
} aotx_model_how;

/* cuda/model/forward.cuh:112-117 */
typedef struct aotx_model_input {
    const float *feature;
    unsigned int width;
    unsigned int position[3];
    unsigned long long generation;
} aotx_model_input;

/* cuda/model/forward.cuh:122-145. Every pointer names device memory. */
typedef struct aotx_model_run {
    const int *ids;
    const aotx_model_input *input;
    const unsigned int *offset;
    const unsigned int *agent;
    float *logits;
    float *pooled;
    float *score;
    int *token;
    unsigned int *draw;
    unsigned long long seed;
    unsigned int seqs;
    unsigned int tokens;
    unsigned int rows;
    unsigned int select;
    unsigned int top_k;
    float top_p;
    float temperature;
    const aotx_model_how *how;
    unsigned int telemetry;
    float *capture;
    const unsigned int *capture_layer;
    unsigned int capture_count;
} aotx_model_run;

typedef struct aotx_kv_entry {
    unsigned int agent;
    unsigned int pages;
} aotx_kv_entry;

/* The host-side record of the page pool (cuda/kvcache/kvcache.cuh:88-96). `limit` is
 * read by aotx_kv_open: the pages of the pool (0 = 1024 pages, 2 GiB). The pool is one
 * device allocation; page position i lives at range + i * 2 MiB, as the reference's
 * reserved range places it (cuda/kvcache/kv_host.cu:36-37). */
typedef struct aotx_kv_map {
    unsigned long long range;
    unsigned long long range_bytes;
    unsigned int limit;
    unsigned int held[AOTX_KV_PAGES_MAX];
    unsigned int free_at[AOTX_KV_PAGES_MAX];
    unsigned int free_count;
    unsigned int created;
} aotx_kv_map;

/* The device page table and request queue (cuda/kvcache/kvcache.cuh:55-64). */
typedef struct aotx_kv_table {
    unsigned long long page[AOTX_SLOTS][AOTX_KV_PAGES_EACH];
    unsigned int count[AOTX_SLOTS];
    unsigned int mapped_pages;
    unsigned int short_of;
    unsigned int made;
    unsigned int served;
    unsigned int refused;
    aotx_kv_entry queue[AOTX_KV_QUEUE_MAX];
} aotx_kv_table;

/* ---------------------------------------------------------------------------------------
 * Weights region and descriptors.
 * ------------------------------------------------------------------------------------- */

/* Name the weights region: a device allocation owned by the caller. Replaces the
 * reference's runtime-owned region (aotx_mem_weights_map/base, cuda/mem/mem.cuh:132-138). */
int aotx_mem_weights_set(unsigned long long base, unsigned long long bytes);
unsigned long long aotx_mem_weights_base(void);

/* Give a role its descriptor. Replaces the GGUF-reading aotx_model_describe
 * (cuda/model/forward.cuh:302) and the device symbol aotx_model[role] it fills
 * (cuda/model/model.cuh:88). Returns 1 for a shape this build does not run. */
int aotx_model_set_desc(unsigned int role, const aotx_model_desc *desc);

/* ---------------------------------------------------------------------------------------
 * Model-step operator surface (cuda/model/forward.cuh:325-372).
 * ------------------------------------------------------------------------------------- */

/* Buffers + graph plans for up to max_tokens rows (model_host.cu:95-153). */
int aotx_model_open(unsigned int role, unsigned int max_tokens);
/* Give back buffers, graphs and the stream (model_host.cu:260-286). */
void aotx_model_shut(unsigned int role);
/* Zero every slot's cache position and the fault count (model_host.cu:222-231). */
void aotx_model_forget(void);
/* Zero every slot's draw counter (model_host.cu:233-240). */
void aotx_model_restream(void);
/* Rows that found no cache page (model_host.cu:252-258). */
unsigned int aotx_model_faulted(void);
/* Kernel nodes of the largest captured step graph of a role (model_host.cu:243-250). */
unsigned int aotx_model_nodes(unsigned int role);
/* Ask the page cache for the pages of the next pass (model_host.cu:202-220). offset and
 * agent are device pointers. The caller answers with aotx_kv_serve before launching. */
int aotx_model_pages(unsigned int role, const unsigned int *offset, unsigned int seqs,
                     const unsigned int *agent);
/* One synchronous pass (model_host.cu:155-200). set is a host pointer whose members are
 * device pointers. */
int aotx_model_launch(unsigned int role, const aotx_model_run *set);
/* One pass that samples one token per sequence from its last row (call_host.cu:71-93).
 * ids, offset[seqs+1], agent[seqs], token[seqs], draw[seqs] are device pointers; how and
 * seed are host pointers. */
int aotx_model_sample(unsigned int role, const int *ids, const unsigned int *offset,
                      unsigned int seqs, const unsigned int *agent,
                      const aotx_model_how *how, int *token, unsigned int *draw,
                      unsigned long long *seed);
/* Prefill (call_host.cu:40-56; model.cuh:120-128). logits, when given, receives the row of
 * every token. pooled, when given, receives [seqs][hidden]: each sequence's last residual
 * row under the last RMSNorm, scaled to unit length (cuda/embed/embed.cu:8-65). As in the
 * reference, only the embedding role's pass writes pooled; the other roles leave it as it
 * was. */
int aotx_model_prefill(unsigned int role, const int *ids, const unsigned int *offset,
                       unsigned int seqs, const unsigned int *agent, float *logits,
                       float *pooled);
/* The rank role's score of each sequence (call_host.cu:58-69; model.cuh:130-133):
 * softmax(yes, no)[0] of the two cls_output rows against the last row under the last
 * RMSNorm (cuda/rerank/rerank.cu:8-81). The rank role opens only with a class head of
 * Q8_0, F16 or F32 (the descriptor's weight type). */
int aotx_model_rerank(const int *ids, const unsigned int *offset, unsigned int seqs,
                      const unsigned int *agent, float *score);
/* Language prefill with per-sequence samples, logits and residual capture
 * (call_host.cu:95-117; forward.cuh:361-368). capture, when given with layer_count > 0,
 * receives [layer_count][seqs][hidden]: slot c holds, for each sequence, the residual row
 * of its last token after layer layers[c] (layers: device memory). The reference adds
 * registered steer vectors (how->steer) in the same place; this build has no steer
 * registry, so none is ever registered and none is added, which is what the reference
 * does while its registry is empty. The probe sets `telemetry` as the reference's does; the
 * reference's pick returns before any figure when the call has no token buffer
 * (cuda/model/sample.cu:481-483), and the probe passes none, so neither build computes the
 * per-token logprob and entropy for a probe (the decode tick's figures go to the reference's
 * record stream, which is not part of this path). */
int aotx_model_probe(unsigned int role, const int *ids, const unsigned int *offset,
                     unsigned int seqs, const unsigned int *agent,
                     const aotx_model_how *how, float *logits, unsigned int select,
                     float *capture, const unsigned int *layers, unsigned int layer_count);
/* Keep each token bucket's recorded graph for the calls after (keep = 1, the default), or
 * record and drop a fresh graph on every call (keep = 0), for tests that compare replays
 * with first runs. No counterpart in the reference, which captures once at open. */
void aotx_model_graphs(unsigned int keep);
/* Set one slot's cache position. No counterpart in the reference, which restores a slot
 * by prefilling its tokens again (cuda/model/decode.cu:230-305); this is for callers that
 * write a slot's KV pages out of band (restore from a copy, benchmarks that seat a
 * prefilled context) and then continue decoding at `position`. Returns 1 for a bad slot. */
int aotx_model_seat(unsigned int agent, unsigned int position);
/* Device address of one of a role's step buffers, for checks; no counterpart in the
 * reference. which: 0 the rows after the last norm (half [max_tokens][hidden]; a 5..32-row
 * pass in the fragment layout), 1 the residual stream (float), 2 the head's rows (float
 * [rows][vocab]), 3 the head's input rows (half), 4 the routed rows per expert of the last
 * layer run (u32 [experts]), 5 the experts each token chose there (u32 [tokens][used]), 6 the
 * router's probabilities there (f32 [tokens][experts]).
 * 0 for an unknown buffer or one the role does not have. */
unsigned long long aotx_model_buffer(unsigned int role, unsigned int which);

/* ---------------------------------------------------------------------------------------
 * KV page pool (cuda/kvcache/kvcache.cuh:100-111).
 * ------------------------------------------------------------------------------------- */
int aotx_kv_open(aotx_kv_map *map);
int aotx_kv_reserve(aotx_kv_map *map);
/* Answer every queued request in order; returns the requests answered
 * (kv_host.cu:128-193). stream is a hipStream_t or null. */
int aotx_kv_serve(aotx_kv_map *map, void *stream);
void aotx_kv_close(aotx_kv_map *map);
/* Queue a request for `pages` more pages for a slot, or (release) for every page of the
 * slot to go back, as device code does (cuda/kvcache/pages.cu:38-57); the next
 * aotx_kv_serve answers it. Returns 1 when queued, 0 when refused (full queue, bad slot). */
int aotx_kv_request(unsigned int agent, unsigned int pages);
int aotx_kv_release(unsigned int agent);
/* Copy the device page table out (for checks). */
int aotx_kv_table_read(aotx_kv_table *out);
/* Device address of the page table (aotx_kv.page), for kernel-level attention calls. */
unsigned long long aotx_kv_table_device(void);

/* ---------------------------------------------------------------------------------------
 * Kernel-level entry points. All pointers are device pointers; stream is a hipStream_t
 * (null = the default stream). They return 1 for a shape they refuse.
 * ------------------------------------------------------------------------------------- */

/* Q8_0 product y[m][n] = sum_k x[m][k] * w[n][k]; w row-major [n][k/32] blocks of 34 B,
 * x fp16 [m][k], y fp32 [m][n]. Replaces aotx_model_gemv / aotx_model_gemm for Q8_0
 * (cuda/model/model.cuh:105-116; gemv.cuh:33-195; gemm.cuh:55-189). k % 32 == 0. */
int aotx_q8_gemv(const void *w, unsigned int n, unsigned int k, const void *x,
                 unsigned int m, float *y, void *stream);
/* The same product with fp16 output (the microbenchmark form). */
int aotx_q8_gemv_f16(const void *w, unsigned int n, unsigned int k, const void *x,
                     unsigned int m, void *y, void *stream);

/* The repacked form the model path streams (no counterpart in the reference, whose weights
 * stay in the file's layout). Same bytes per weight (int8 + one fp16 scale per 32),
 * reordered so one wave reads its matrix-core operands with coalesced 16-byte loads:
 * [n/16 tiles][k/128 quads][64 lanes][32 quants] then [tiles][quads][64 lanes] scales
 * (lane = row % 16 + 16 * block-in-quad; the last tile and quad are zero padded).
 * aotx_q8r_size gives the bytes; aotx_q8_repack converts; aotx_q8r_gemv(_f16) is the
 * product over the repacked tensor with the arguments of aotx_q8_gemv. */
unsigned long long aotx_q8r_size(unsigned int n, unsigned int k);
int aotx_q8_repack(const void *w, unsigned int n, unsigned int k, void *dst, void *stream);
int aotx_q8r_gemv(const void *wr, unsigned int n, unsigned int k, const void *x,
                  unsigned int m, float *y, void *stream);
int aotx_q8r_gemv_f16(const void *wr, unsigned int n, unsigned int k, const void *x,
                      unsigned int m, void *y, void *stream);

/* Dequantize rows of a Q8_0 tensor to fp16 (cuda/model/dequant.cu:9-70). */
int aotx_q8_dequant(const void *w, unsigned int k, unsigned int first_row,
                    unsigned int rows, void *out, void *stream);

/* Paged decode attention over the page table of aotx_kv_open (cuda/model/attention.cu).
 * q fp16 [tokens][heads][d]; pos[tokens] = cache position of each token (attends to
 * positions 0..pos); agent[tokens] = slot; out fp16 [tokens][heads][d]. layer and
 * layers give the layout-block index of cuda/model/kv_layout.cuh:121-136.
 * Returns 1 on a refused shape. Missing pages add to the fault counter. */
int aotx_attend_paged(const void *q, const unsigned int *pos, const unsigned int *agent,
                      unsigned int tokens, unsigned int heads, unsigned int kv_heads,
                      unsigned int head_dim, unsigned int layer, unsigned int layers,
                      void *out, void *stream);

/* aotx_attend_paged without any allocation: no counterpart in the reference. For callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The chunk partials and arrival counters live in a fixed
 * device array of the library (2 MiB of partials, 4096 counters, held by each GPU the
 * library runs on until the process ends) instead of the grow-on-demand scratch. Same
 * arguments, kernels and results as aotx_attend_paged. Returns 1 (and prints why) when
 * the launch's partials or counters exceed the array (at most 4096 tokens x KV heads;
 * split launches of few tokens need partials), or when no page pool has been opened.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU race. */
int aotx_attend_paged_static(const void *q, const unsigned int *pos, const unsigned int *agent,
                             unsigned int tokens, unsigned int heads, unsigned int kv_heads,
                             unsigned int head_dim, unsigned int layer, unsigned int layers,
                             void *out, void *stream);

/* Write K (rotated) and V rows of tokens into the pages (the KV half of
 * cuda/model/rope.cu:200-234); k, v fp16 [tokens][kv_heads][d] already rotated. */
int aotx_kv_write(const void *k, const void *v, const unsigned int *pos,
                  const unsigned int *agent, unsigned int tokens, unsigned int kv_heads,
                  unsigned int head_dim, unsigned int layer, unsigned int layers,
                  void *stream);

/* Sampler (cuda/model/sample.cu:456-765): one token per row of fp32 logits [rows][vocab].
 * agent[rows] selects each row's Philox stream and draw counter; how (device, may be
 * null) gives per-row settings, else top_k/top_p/temperature/seed apply to every row.
 * token[rows] and draw[rows] (may be null) are written. The draw counters are the
 * library's per-slot counters (aotx_model_restream zeroes them). */
int aotx_pick(const float *logits, unsigned int rows, unsigned int vocab,
              const unsigned int *agent, const aotx_model_how *how, unsigned int top_k,
              float top_p, float temperature, unsigned long long seed, int *token,
              unsigned int *draw, void *stream);

/* Philox4x32-10 words for n (counter, key) pairs (cuda/rng/rng.cuh:54-85): ctr[4*n],
 * key[2*n], out[4*n] unsigned int, device pointers. */
int aotx_philox(const unsigned int *ctr, const unsigned int *key, unsigned int n,
                unsigned int *out, void *stream);

/* Router (cuda/model/experts.cu:10-75): router fp32 [experts][hidden] . x fp16
 * [tokens][hidden]; softmax over every expert; top `used` ids with lower-index ties. */
int aotx_expert_route(const float *router, const void *x, unsigned int tokens,
                      unsigned int hidden, unsigned int experts, unsigned int used,
                      float *prob, unsigned int *ids, void *stream);

/* Routed expert FFN for one layer with tokens grouped per expert: every expert's weights
 * are read once per call (replaces cuda/model/expert_matrix.cu:8-63, experts.cu:77-98 and
 * the per-rank loop of experts_host.cu:99-111). gate/up: [experts][ffn][hidden/32] Q8_0;
 * down: [experts][hidden][ffn/32] Q8_0; x fp16 [tokens][hidden]; prob/ids from the
 * router; out fp32 [tokens][hidden] = sum over rank of prob * expert(x), in rank order. */
int aotx_expert_ffn(const void *gate, const void *up, const void *down,
                    unsigned int experts, unsigned int used, unsigned int hidden,
                    unsigned int ffn, const void *x, unsigned int tokens,
                    const float *prob, const unsigned int *ids, float *out, void *stream);

/* Deterministic synthetic Q8_0 tensor: rows x k weights drawn from N(0, sigma) by
 * the build's integer normal generator (12 summed 16-bit uniforms of splitmix64 from
 * `seed`), quantized per 32-block with d = max|w|/127, q = rint(w/d). The device and
 * host versions write identical bytes. */
int aotx_synth_q8(void *dst, unsigned long long rows, unsigned int k, float sigma,
                  unsigned long long seed, void *stream);
int aotx_synth_q8_host(void *dst, unsigned long long rows, unsigned int k, float sigma,
                       unsigned long long seed, unsigned int threads);
/* fp16 values from N(0, sigma) by the same generator (count values). */
int aotx_synth_f16(void *dst, unsigned long long count, float sigma,
                   unsigned long long seed, void *stream);
int aotx_synth_f16_host(void *dst, unsigned long long count, float sigma,
                        unsigned long long seed, unsigned int threads);

/* Library version string. */
const char *aotx_version(void);

#ifdef __cplusplus
}
#endif

#endif
