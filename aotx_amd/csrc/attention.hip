/* Paged decode attention on gfx950.
 *
 * Reference: aotx_model_attend (cuda/model/attention.cu:22-154): one warp per (token,
 * query head), a single pass of online softmax over every position <= pos, scale
 * 1/sqrt(d), fp32 sums, out = half(sum / mass); keys and values come from the 16-position
 * layout blocks of cuda/model/kv_layout.cuh. Each query head re-reads its KV head there.
 *
 * Here one workgroup of 8 waves takes (token, KV head, context chunk):
 *   - all G = heads / kv_heads query heads of the KV head share one read of its keys and
 *     values (grouped-query sharing: the KV bytes are read once per token, not G times);
 *   - a wave step is one whole 16-position layout block (4 KB of keys and 4 KB of values
 *     at d = 128), loaded with 16-byte buffer loads from the block's scalar base address,
 *     the next block's loads issued before the current block is computed;
 *   - scores and the probability-weighted sum of values run on the matrix cores
 *     (v_mfma_f32_16x16x32_f16 for K . q^T, v_mfma_f32_16x16x16_f16 for P . V), online
 *     softmax per block in base 2 (scores carry log2(e) / sqrt(d)), fp32 accumulation;
 *   - the waves' (max, mass, sum) are merged in wave order through LDS. At small batches
 *     the context is split over workgroups (flash-decoding) so that the launch still
 *     covers the GPU; the last chunk of a (token, KV head) to finish adds all of its
 *     chunks in chunk order, so the result does not depend on timing and no second
 *     launch is needed.
 */
#include "attention.h"
#include "attention_dev.h"

#include <algorithm>
#include <stdlib.h>

template <int D, int G, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void aotx_attend_mma(aotx_attn_args a)
{
    aotx_args_touch(a);
    aotx_attend_body<D, G, W, 1>(a, blockIdx.x);
}

/* Prompt pieces one wave each (aotx_attend_runs). */
template <int D, int G, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void aotx_attend_run(aotx_attn_args a)
{
    aotx_args_touch(a);
    aotx_attend_runs<D, G, W>(a, blockIdx.x);
}

/* ---------------------------------------------------------------------------------------
 * Host side
 * ------------------------------------------------------------------------------------- */

unsigned int aotx_attn_splits(unsigned int tokens, unsigned int kv_heads,
                              unsigned int max_context)
{
    /* about ATTN_TARGET_GROUPS workgroups over the launch, chunks of at least 64 positions */
    const unsigned int target = ATTN_TARGET_GROUPS;
    unsigned int units = tokens * kv_heads;
    unsigned int s = (target + units - 1u) / units;
    unsigned int cap = (max_context + ATTN_CHUNK_ALIGN - 1u) / ATTN_CHUNK_ALIGN;
    if (s > cap) s = cap;
    if (s > ATTN_MAX_SPLITS) s = ATTN_MAX_SPLITS;
    if (s < 1u) s = 1u;
    return s;
}

size_t aotx_attn_scratch(unsigned int tokens, unsigned int kv_heads, unsigned int splits,
                         unsigned int group, unsigned int head_dim)
{
    return (size_t)tokens * kv_heads * splits * group * (head_dim + 2u) * sizeof(float);
}

/* The arguments of one launch; 1 when the shape is refused. */
int aotx_attend_plan(aotx_attn_args *out_args, const unsigned short *q, unsigned short *out,
                     const unsigned int *pos, const unsigned int *agent,
                     const unsigned int *m_dev, unsigned int tokens, unsigned int heads,
                     unsigned int kv_heads, unsigned int head_dim, unsigned int layer,
                     unsigned int layers, unsigned int max_context, float *partial,
                     unsigned int *count)
{
    if (tokens == 0u || kv_heads == 0u || heads % kv_heads != 0u) return 1;
    if (head_dim != 64u && head_dim != 128u) return 1;
    unsigned int g = heads / kv_heads;
    if (g != 1u && g != 2u && g != 4u && g != 8u) return 1;
    if (layer >= layers || max_context == 0u || max_context > AOTX_SEQ_MAX_TOKENS * 8u) return 1;
    aotx_attn_args a;
    a.q = q;
    a.out = out;
    a.pos = pos;
    a.agent = agent;
    a.m_dev = m_dev;
    a.tokens = tokens;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.layer = layer;
    a.splits = aotx_attn_splits(tokens, kv_heads, max_context);
    a.chunk_max = max_context;
    a.out_frag = 0u;
    a.shape = aotx_kvl_make(layers, kv_heads, head_dim);
    a.state = aotx_state_device();
    a.partial = partial != nullptr
        ? partial
        : (float *)aotx_scratch(AOTX_SCRATCH_ATTN_PARTIAL,
                                aotx_attn_scratch(tokens, kv_heads, a.splits, g, head_dim));
    a.count = count != nullptr
        ? count
        : (unsigned int *)aotx_scratch(AOTX_SCRATCH_ATTN_COUNT,
                                       (size_t)tokens * kv_heads * sizeof(unsigned int));
    *out_args = a;
    return 0;
}

/* Launch attention. q/out fp16; pos/agent device arrays; m_dev optional device count. */
int aotx_attend_launch(const unsigned short *q, unsigned short *out, const unsigned int *pos,
                       const unsigned int *agent, const unsigned int *m_dev,
                       unsigned int tokens, unsigned int heads, unsigned int kv_heads,
                       unsigned int head_dim, unsigned int layer, unsigned int layers,
                       unsigned int max_context, float *partial, unsigned int *count,
                       hipStream_t stream, unsigned int out_frag)
{
    aotx_attn_args a;
    if (aotx_attend_plan(&a, q, out, pos, agent, m_dev, tokens, heads, kv_heads, head_dim,
                         layer, layers, max_context, partial, count) != 0)
        return 1;
    if (out_frag != 0u && (tokens > AOTX_XFRAG_ROWS || (heads * head_dim) % 128u != 0u)) return 1;
    a.out_frag = out_frag;
    const unsigned int g = heads / kv_heads;
    if (tokens >= AOTX_ATTN_PIECE_TOKENS) {
        /* more tokens than sequence slots: a batch with prompt pieces, two waves per piece
         * of consecutive queries of a sequence (each half of its blocks), 8 waves per
         * 16-token range and KV head */
        a.splits = 1u;
        const dim3 rgrid((tokens + AOTX_RUN_RANGE - 1u) / AOTX_RUN_RANGE * kv_heads);
#define AOTX_PIECE_GO(DD, GG)                                                              \
        do {                                                                               \
            hipLaunchKernelGGL((aotx_attend_run<DD, GG, 8>), rgrid, dim3(512), 0, stream, a); \
            AOTX_LAUNCH_CHECK();                                                           \
        } while (0)
        if (head_dim == 128u) {
            if (g == 1u) AOTX_PIECE_GO(128, 1);
            else if (g == 2u) AOTX_PIECE_GO(128, 2);
            else if (g == 4u) AOTX_PIECE_GO(128, 4);
            else AOTX_PIECE_GO(128, 8);
        } else {
            if (g == 1u) AOTX_PIECE_GO(64, 1);
            else if (g == 2u) AOTX_PIECE_GO(64, 2);
            else if (g == 4u) AOTX_PIECE_GO(64, 4);
            else AOTX_PIECE_GO(64, 8);
        }
#undef AOTX_PIECE_GO
        return 0;
    }
    dim3 grid(tokens * kv_heads * a.splits);
#define AOTX_ATTN_GO(DD, GG)                                                               \
    do {                                                                                   \
        hipLaunchKernelGGL((aotx_attend_mma<DD, GG, 8>), grid, dim3(512), 0, stream, a);   \
        AOTX_LAUNCH_CHECK();                                                               \
    } while (0)
    if (head_dim == 128u) {
        if (g == 1u) AOTX_ATTN_GO(128, 1);
        else if (g == 2u) AOTX_ATTN_GO(128, 2);
        else if (g == 4u) AOTX_ATTN_GO(128, 4);
        else AOTX_ATTN_GO(128, 8);
    } else {
        if (g == 1u) AOTX_ATTN_GO(64, 1);
        else if (g == 2u) AOTX_ATTN_GO(64, 2);
        else if (g == 4u) AOTX_ATTN_GO(64, 4);
        else AOTX_ATTN_GO(64, 8);
    }
#undef AOTX_ATTN_GO
    AOTX_LAUNCH_CHECK();
    return 0;
}

extern "C" int aotx_attend_paged(const void *q, const unsigned int *pos,
                                 const unsigned int *agent, unsigned int tokens,
                                 unsigned int heads, unsigned int kv_heads,
                                 unsigned int head_dim, unsigned int layer,
                                 unsigned int layers, void *out, void *stream)
{
    if (q == nullptr || pos == nullptr || agent == nullptr || out == nullptr) return 1;
    return aotx_attend_launch((const unsigned short *)q, (unsigned short *)out, pos, agent,
                              nullptr, tokens, heads, kv_heads, head_dim, layer, layers,
                              AOTX_SEQ_MAX_TOKENS, nullptr, nullptr, aotx_stream(stream));
}

/* ---------------------------------------------------------------------------------------
 * The allocation-free form of aotx_attend_paged.
 *
 * Its chunk partials and arrival counters live in `scratch`, a fixed array in device
 * memory that each GPU holds from library load to process end, instead of the library's
 * grow-on-demand scratch (which calls hipMalloc). Host code never uses the array's name as
 * an address: the device address comes from hipGetSymbolAddress, once per device, and is
 * kept per device. Every call on a GPU shares that GPU's array, so calls that overlap on
 * one GPU race.
 * ------------------------------------------------------------------------------------- */

#define AOTX_ATTN_STATIC_PARTIAL (2u * 1024u * 1024u)   /* chunk partials, bytes */
#define AOTX_ATTN_STATIC_COUNTS  4096u                    /* arrival counters, words */
#define AOTX_MAX_DEVICES         64

static __device__ __align__(256) unsigned char scratch[AOTX_ATTN_STATIC_PARTIAL + AOTX_ATTN_STATIC_COUNTS * 4u];

static unsigned char *aotx_attn_static[AOTX_MAX_DEVICES];

/* The device address of this device's `scratch` (0 when it cannot be resolved). */
static unsigned char *aotx_attn_static_ptr(void)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= AOTX_MAX_DEVICES) return nullptr;
    if (aotx_attn_static[dev] == nullptr) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            fprintf(stderr, "aotx: the attention scratch array has no device address\n");
            return nullptr;
        }
        aotx_attn_static[dev] = (unsigned char *)ptr;
    }
    return aotx_attn_static[dev];
}

__global__ void aotx_attn_clear_kernel(unsigned int *count, unsigned int n)
{
    for (unsigned int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        count[i] = 0u;
}

extern "C" int aotx_attend_paged_static(const void *q, const unsigned int *pos,
                                        const unsigned int *agent, unsigned int tokens,
                                        unsigned int heads, unsigned int kv_heads,
                                        unsigned int head_dim, unsigned int layer,
                                        unsigned int layers, void *out, void *stream)
{
    if (q == nullptr || pos == nullptr || agent == nullptr || out == nullptr) return 1;
    if (tokens == 0u || kv_heads == 0u || heads % kv_heads != 0u) return 1;
    aotx_state *state = aotx_state_existing();
    if (state == nullptr) {
        fprintf(stderr, "aotx_attend_paged_static: no page pool is open on this process\n");
        return 1;
    }
    unsigned char *base = aotx_attn_static_ptr();
    if (base == nullptr) return 1;
    float *partial = (float *)base;
    unsigned int *count = (unsigned int *)(base + AOTX_ATTN_STATIC_PARTIAL);
    /* the shape is checked before anything is enqueued */
    aotx_attn_args plan;
    if (aotx_attend_plan(&plan, (const unsigned short *)q, (unsigned short *)out, pos, agent,
                         nullptr, tokens, heads, kv_heads, head_dim, layer, layers,
                         AOTX_SEQ_MAX_TOKENS, partial, count) != 0)
        return 1;
    /* the scratch this launch needs must fit the fixed array */
    const unsigned int splits = aotx_attn_splits(tokens, kv_heads, AOTX_SEQ_MAX_TOKENS);
    const size_t units = (size_t)tokens * kv_heads;
    const size_t need = aotx_attn_scratch(tokens, kv_heads, splits, heads / kv_heads, head_dim);
    if (units > AOTX_ATTN_STATIC_COUNTS || need > AOTX_ATTN_STATIC_PARTIAL) {
        fprintf(stderr, "aotx_attend_paged_static: %u tokens x %u KV heads need %zu bytes of "
                "partials and %zu counters; the fixed scratch holds %u and %u\n", tokens,
                kv_heads, need, units, AOTX_ATTN_STATIC_PARTIAL, AOTX_ATTN_STATIC_COUNTS);
        return 1;
    }
    hipStream_t s = aotx_stream(stream);
    /* counters start at zero (a fill kernel, which a graph capture may hold) */
    hipLaunchKernelGGL(aotx_attn_clear_kernel, dim3(((unsigned int)units + 255u) / 256u), dim3(256),
                       0, s, count, (unsigned int)units);
    AOTX_LAUNCH_CHECK();
    return aotx_attend_launch((const unsigned short *)q, (unsigned short *)out, pos, agent,
                              nullptr, tokens, heads, kv_heads, head_dim, layer, layers,
                              AOTX_SEQ_MAX_TOKENS, partial, count, s);
}

/* K/V rows into the pages (the page-write half of cuda/model/rope.cu:128-196). */
__global__ void aotx_kv_write_kernel(const unsigned short *k, const unsigned short *v,
                                     const unsigned int *pos, const unsigned int *agent,
                                     unsigned int tokens, unsigned int kv_heads,
                                     unsigned int head_dim, unsigned int layer,
                                     aotx_kvl_shape shape, aotx_state *state)
{
    unsigned int t = blockIdx.x;
    if (t >= tokens) return;
    unsigned int position = pos[t];
    unsigned char *blk = aotx_kvl_block(shape, &state->kv, agent[t], layer, position);
    if (blk == nullptr) {
        if (threadIdx.x == 0u) atomicAdd(&state->faults, 1u);
        return;
    }
    unsigned int narrow = kv_heads * head_dim;
    for (unsigned int i = threadIdx.x; i < narrow; i += blockDim.x) {
        unsigned int h = i / head_dim, d = i % head_dim;
        unsigned short *kr = (unsigned short *)blk
            + (unsigned long long)(h * AOTX_KVL_BLOCK + position % AOTX_KVL_BLOCK) * head_dim;
        unsigned short *vr = (unsigned short *)blk
            + (unsigned long long)((kv_heads + h) * AOTX_KVL_BLOCK + position % AOTX_KVL_BLOCK) * head_dim;
        kr[d] = k[(unsigned long long)t * narrow + i];
        vr[d] = v[(unsigned long long)t * narrow + i];
    }
}

extern "C" int aotx_kv_write(const void *k, const void *v, const unsigned int *pos,
                             const unsigned int *agent, unsigned int tokens,
                             unsigned int kv_heads, unsigned int head_dim, unsigned int layer,
                             unsigned int layers, void *stream)
{
    if (k == nullptr || v == nullptr || pos == nullptr || agent == nullptr) return 1;
    if (tokens == 0u) return 0;
    if (layer >= layers || head_dim == 0u || kv_heads == 0u) return 1;
    hipLaunchKernelGGL(aotx_kv_write_kernel, dim3(tokens), dim3(256), 0, aotx_stream(stream),
                       (const unsigned short *)k, (const unsigned short *)v, pos, agent, tokens,
                       kv_heads, head_dim, layer, aotx_kvl_make(layers, kv_heads, head_dim),
                       aotx_state_device());
    AOTX_LAUNCH_CHECK();
    return 0;
}
