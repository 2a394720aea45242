/* Paged decode attention on gfx950.
 *
 * Reference: aotx_model_attend (cuda/model/attention.cu:22-154): one warp per (token,
 * query head), a single pass of online softmax over every position <= pos, scale
 * 1/sqrt(d), fp32 sums, out = half(sum / mass); keys and values come from the 16-position
 * layout blocks of cuda/model/kv_layout.cuh. Each query head re-reads its KV head there.
 *
 * Here one wave takes (token, KV head, context chunk):
 *   - all G = heads / kv_heads query heads of the KV head share one read of its keys and
 *     values (grouped-query sharing: the KV bytes are read once per token, not G times);
 *   - 8 lanes hold one position: lane (grp = lane / 8, sub = lane % 8) reads the 16-byte
 *     pieces 8*sub and 64 + 8*sub of a 128-element row, so 8 positions of one layout block
 *     are read per instruction pair and every byte of the block is consumed;
 *   - pass 1 writes the scaled scores of the chunk to LDS; the chunk maximum and the
 *     exponentials follow; pass 2 reads the value rows once and accumulates;
 *   - the context is split over several waves (flash-decoding) so that a batch of one
 *     still covers the GPU; each chunk leaves (max, mass, unnormalised sum) and a merge
 *     kernel adds the chunks of a (token, KV head) in chunk order, so the result does not
 *     depend on timing.
 */
#include "aotx_internal.h"

#include <algorithm>

typedef unsigned int aotx_u4a __attribute__((ext_vector_type(4)));

struct aotx_attn_args {
    const unsigned short *q;      /* fp16 [tokens][heads][d] */
    unsigned short *out;          /* fp16 [tokens][heads][d] */
    const unsigned int *pos;      /* [tokens] */
    const unsigned int *agent;    /* [tokens] */
    const unsigned int *m_dev;    /* device token count, or null */
    unsigned int tokens;
    unsigned int heads;
    unsigned int kv_heads;
    unsigned int layer;
    unsigned int splits;          /* chunks per (token, KV head) at most */
    unsigned int chunk_max;       /* LDS capacity in positions */
    aotx_kvl_shape shape;
    aotx_state *state;
    float *partial;               /* [tokens*kv_heads][splits][G*(d+2)] */
};

#define ATTN_UNROLL 4
#define ATTN_MIN_CHUNK 64u

static __device__ __forceinline__ float aotx_attn_h(unsigned int word, int hi)
{
    return aotx_h2f((unsigned short)(hi ? (word >> 16) : (word & 0xFFFFu)));
}

template <int D, int G>
__global__ __launch_bounds__(64) void aotx_attend_kernel(aotx_attn_args a)
{
    constexpr int NP = D / 64;          /* 16-byte pieces per lane per row */
    constexpr int E = 8 * NP;           /* elements per lane */
    extern __shared__ float sc[];       /* [chunk][G] scores, then exponentials */

    const unsigned int lane = threadIdx.x;
    const unsigned int grp = lane >> 3;
    const unsigned int sub = lane & 7u;
    unsigned int tokens = a.m_dev ? *a.m_dev : a.tokens;
    if (tokens > a.tokens) tokens = a.tokens;
    const unsigned int S = a.splits;
    const unsigned int c = blockIdx.x % S;
    const unsigned int rest = blockIdx.x / S;
    const unsigned int kh = rest % a.kv_heads;
    const unsigned int t = rest / a.kv_heads;
    if (t >= tokens) return;
    const unsigned int n = a.pos[t] + 1u;
    unsigned int chunk = (n + S - 1u) / S;
    chunk = (chunk + 15u) & ~15u;
    if (chunk < ATTN_MIN_CHUNK) chunk = ATTN_MIN_CHUNK;
    if (chunk > a.chunk_max) {               /* a position past the planned context */
        if (threadIdx.x == 0u && blockIdx.x % S == 0u) atomicAdd(&a.state->faults, 1u);
        return;
    }
    const unsigned int st = (n + chunk - 1u) / chunk;   /* chunks of this token */
    if (c >= st) return;
    const unsigned int p0 = c * chunk;
    const unsigned int p1 = (p0 + chunk < n) ? p0 + chunk : n;
    const unsigned int cnt = p1 - p0;
    const unsigned int agent = a.agent[t];
    const aotx_kv_table *kv = &a.state->kv;
    const float scale = 1.0f / sqrtf((float)D);

    /* the G query heads of this KV head, as fp32 */
    float qv[G][E];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const unsigned short *qrow = a.q + ((unsigned long long)t * a.heads + kh * G + j) * D;
#pragma unroll
        for (int pc = 0; pc < NP; ++pc) {
            aotx_u4a w = *(const aotx_u4a *)(qrow + 64 * pc + 8 * sub);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qv[j][8 * pc + 2 * e] = aotx_attn_h(w[e], 0);
                qv[j][8 * pc + 2 * e + 1] = aotx_attn_h(w[e], 1);
            }
        }
    }

    int missing = 0;
    const unsigned int kbase = kh * AOTX_KVL_BLOCK;
    const unsigned int vbase = (a.kv_heads + kh) * AOTX_KVL_BLOCK;

    /* pass 1: scores */
    for (unsigned int base = p0; base < p1; base += 8u * ATTN_UNROLL) {
        aotx_u4a kr[ATTN_UNROLL][NP];
        bool valid[ATTN_UNROLL];
#pragma unroll
        for (int u = 0; u < ATTN_UNROLL; ++u) {
            unsigned int p = base + 8u * u + grp;
            valid[u] = p < p1;
            unsigned int pp = valid[u] ? p : p0;
            const unsigned char *blk = aotx_kvl_block(a.shape, kv, agent, a.layer, pp);
            if (blk == nullptr) {
                missing = 1;
                blk = (const unsigned char *)a.q;   /* any readable address */
                valid[u] = false;
            }
            const unsigned short *row = (const unsigned short *)blk
                + (unsigned long long)(kbase + pp % AOTX_KVL_BLOCK) * D;
#pragma unroll
            for (int pc = 0; pc < NP; ++pc) {
                kr[u][pc] = blk == (const unsigned char *)a.q ? (aotx_u4a){0u, 0u, 0u, 0u}
                                                              : *(const aotx_u4a *)(row + 64 * pc + 8 * sub);
            }
        }
#pragma unroll
        for (int u = 0; u < ATTN_UNROLL; ++u) {
            float dot[G];
#pragma unroll
            for (int j = 0; j < G; ++j) dot[j] = 0.0f;
#pragma unroll
            for (int pc = 0; pc < NP; ++pc) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float k0 = aotx_attn_h(kr[u][pc][e], 0);
                    float k1 = aotx_attn_h(kr[u][pc][e], 1);
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        dot[j] += qv[j][8 * pc + 2 * e] * k0;
                        dot[j] += qv[j][8 * pc + 2 * e + 1] * k1;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < G; ++j) {
                dot[j] += __shfl_xor(dot[j], 1, 64);
                dot[j] += __shfl_xor(dot[j], 2, 64);
                dot[j] += __shfl_xor(dot[j], 4, 64);
            }
            unsigned int p = base + 8u * u + grp;
            if (valid[u] && sub == 0u) {
#pragma unroll
                for (int j = 0; j < G; ++j) sc[(p - p0) * G + j] = dot[j] * scale;
            }
        }
    }
    missing = __any(missing);
    if (missing && lane == 0u) atomicAdd(&a.state->faults, 1u);
    __syncthreads();

    /* chunk maximum and mass of each query head */
    float mx[G], mass[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float m = -INFINITY;
        for (unsigned int p = lane; p < cnt; p += 64u) m = fmaxf(m, sc[p * G + j]);
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        mx[j] = missing ? -INFINITY : m;
    }
    __syncthreads();
    float part = 0.0f;
    {
        const unsigned int jj = lane % G;
        float mj = mx[0];
#pragma unroll
        for (int j = 1; j < G; ++j) if ((unsigned int)j == jj) mj = mx[j];
        for (unsigned int idx = lane; idx < cnt * G; idx += 64u) {
            float e = missing ? 0.0f : expf(sc[idx] - mj);
            sc[idx] = e;
            part += e;
        }
    }
    /* lanes with the same lane % G hold one head's partial sums */
    for (int off = 32; off >= G; off >>= 1) part += __shfl_xor(part, off, 64);
#pragma unroll
    for (int j = 0; j < G; ++j) mass[j] = __shfl(part, j, 64);
    __syncthreads();

    /* pass 2: values */
    float o[G][E];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) o[j][e] = 0.0f;
    if (!missing) {
        for (unsigned int base = p0; base < p1; base += 8u * ATTN_UNROLL) {
            aotx_u4a vr[ATTN_UNROLL][NP];
            bool valid[ATTN_UNROLL];
#pragma unroll
            for (int u = 0; u < ATTN_UNROLL; ++u) {
                unsigned int p = base + 8u * u + grp;
                valid[u] = p < p1;
                unsigned int pp = valid[u] ? p : p0;
                const unsigned char *blk = aotx_kvl_block(a.shape, kv, agent, a.layer, pp);
                const unsigned short *row = (const unsigned short *)blk
                    + (unsigned long long)(vbase + pp % AOTX_KVL_BLOCK) * D;
#pragma unroll
                for (int pc = 0; pc < NP; ++pc) vr[u][pc] = *(const aotx_u4a *)(row + 64 * pc + 8 * sub);
            }
#pragma unroll
            for (int u = 0; u < ATTN_UNROLL; ++u) {
                unsigned int p = base + 8u * u + grp;
                float w[G];
#pragma unroll
                for (int j = 0; j < G; ++j) w[j] = valid[u] ? sc[(p - p0) * G + j] : 0.0f;
#pragma unroll
                for (int pc = 0; pc < NP; ++pc) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float v0 = aotx_attn_h(vr[u][pc][e], 0);
                        float v1 = aotx_attn_h(vr[u][pc][e], 1);
#pragma unroll
                        for (int j = 0; j < G; ++j) {
                            o[j][8 * pc + 2 * e] += w[j] * v0;
                            o[j][8 * pc + 2 * e + 1] += w[j] * v1;
                        }
                    }
                }
            }
        }
    }
    /* sum the 8 position groups: lanes with the same sub */
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float v = o[j][e];
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            o[j][e] = v;
        }

    if (st == 1u) {
        if (grp == 0u) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                float back = mass[j] > 0.0f ? 1.0f / mass[j] : 0.0f;
                unsigned short *orow = a.out + ((unsigned long long)t * a.heads + kh * G + j) * D;
#pragma unroll
                for (int pc = 0; pc < NP; ++pc)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        orow[64 * pc + 8 * sub + e] = aotx_f2h(o[j][8 * pc + e] * back);
            }
        }
        return;
    }

    /* split context: leave this chunk's (max, mass, sum) for the merge kernel */
    const unsigned int unit = t * a.kv_heads + kh;
    const unsigned int stride = G * (D + 2);
    float *mine = a.partial + ((unsigned long long)unit * S + c) * stride;
    if (grp == 0u) {
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int pc = 0; pc < NP; ++pc)
#pragma unroll
                for (int e = 0; e < 8; ++e) mine[j * (D + 2) + 2 + 64 * pc + 8 * sub + e] = o[j][8 * pc + e];
    }
    if (lane == 0u) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            mine[j * (D + 2)] = mx[j];
            mine[j * (D + 2) + 1] = mass[j];
        }
    }
}

/* Merge the chunks of every (token, KV head) that was split, in chunk order:
 * M = max m_c, out = half(sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M)). */
template <int D, int G>
__global__ __launch_bounds__(256) void aotx_attend_merge(aotx_attn_args a)
{
    unsigned int tokens = a.m_dev ? *a.m_dev : a.tokens;
    if (tokens > a.tokens) tokens = a.tokens;
    const unsigned int unit = blockIdx.x;
    const unsigned int kh = unit % a.kv_heads;
    const unsigned int t = unit / a.kv_heads;
    if (t >= tokens) return;
    const unsigned int S = a.splits;
    const unsigned int n = a.pos[t] + 1u;
    unsigned int chunk = (n + S - 1u) / S;
    chunk = (chunk + 15u) & ~15u;
    if (chunk < ATTN_MIN_CHUNK) chunk = ATTN_MIN_CHUNK;
    if (chunk > a.chunk_max) return;
    const unsigned int st = (n + chunk - 1u) / chunk;
    if (st <= 1u) return;
    const unsigned int stride = G * (D + 2);
    const float *all = a.partial + (unsigned long long)unit * S * stride;
    for (unsigned int idx = threadIdx.x; idx < (unsigned int)(G * D); idx += blockDim.x) {
        unsigned int j = idx / D;
        unsigned int e = idx - j * D;
        float top = -INFINITY;
        for (unsigned int cc = 0; cc < st; ++cc) top = fmaxf(top, all[cc * stride + j * (D + 2)]);
        float msum = 0.0f, osum = 0.0f;
        for (unsigned int cc = 0; cc < st; ++cc) {
            const float *pc = all + cc * stride + j * (D + 2);
            float mc = pc[0];
            float f = (mc == -INFINITY) ? 0.0f : expf(mc - top);
            msum += pc[1] * f;
            osum += pc[2 + e] * f;
        }
        float back = msum > 0.0f ? 1.0f / msum : 0.0f;
        a.out[((unsigned long long)t * a.heads + kh * G + j) * D + e] = aotx_f2h(osum * back);
    }
}

/* ---------------------------------------------------------------------------------------
 * Host side
 * ------------------------------------------------------------------------------------- */

struct aotx_attn_plan {
    aotx_attn_args a;
    unsigned int group;
};

unsigned int aotx_attn_splits(unsigned int tokens, unsigned int kv_heads,
                              unsigned int max_context)
{
    unsigned int units = tokens * kv_heads;
    unsigned int s = (2048u + units - 1u) / units;
    unsigned int need = (max_context + 1023u) / 1024u;  /* chunk <= 1024 positions */
    if (s < need) s = need;
    if (s > 256u) s = 256u;
    if (s < 1u) s = 1u;
    return s;
}

size_t aotx_attn_scratch(unsigned int tokens, unsigned int kv_heads, unsigned int splits,
                         unsigned int group, unsigned int head_dim)
{
    return (size_t)tokens * kv_heads * splits * group * (head_dim + 2u) * sizeof(float);
}

/* Launch attention. q/out fp16; pos/agent device arrays; m_dev optional device count. */
int aotx_attend_launch(const unsigned short *q, unsigned short *out, const unsigned int *pos,
                       const unsigned int *agent, const unsigned int *m_dev,
                       unsigned int tokens, unsigned int heads, unsigned int kv_heads,
                       unsigned int head_dim, unsigned int layer, unsigned int layers,
                       unsigned int max_context, float *partial, hipStream_t stream)
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
    unsigned int chunk = (max_context + a.splits - 1u) / a.splits;
    chunk = (chunk + 15u) & ~15u;
    if (chunk < ATTN_MIN_CHUNK) chunk = ATTN_MIN_CHUNK;
    a.chunk_max = chunk;
    a.shape = aotx_kvl_make(layers, kv_heads, head_dim);
    a.state = aotx_state_device();
    a.partial = partial != nullptr
        ? partial
        : (float *)aotx_scratch(AOTX_SCRATCH_ATTN_PARTIAL,
                                aotx_attn_scratch(tokens, kv_heads, a.splits, g, head_dim));
    size_t lds = (size_t)chunk * g * sizeof(float);
    dim3 grid(tokens * kv_heads * a.splits);
#define AOTX_ATTN_GO(DD, GG)                                                               \
    do {                                                                                   \
        hipLaunchKernelGGL((aotx_attend_kernel<DD, GG>), grid, dim3(64), lds, stream, a);  \
        AOTX_LAUNCH_CHECK();                                                               \
        if (a.splits > 1u) {                                                               \
            hipLaunchKernelGGL((aotx_attend_merge<DD, GG>), dim3(tokens * kv_heads),       \
                               dim3(256), 0, stream, a);                                   \
        }                                                                                  \
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
                              AOTX_SEQ_MAX_TOKENS, nullptr, aotx_stream(stream));
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
