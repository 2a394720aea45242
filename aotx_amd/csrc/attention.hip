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
    unsigned int chunk_max;       /* the largest context planned for */
    aotx_kvl_shape shape;
    aotx_state *state;
    float *partial;               /* [tokens*kv_heads][splits][G*(d+2)] */
};

#define ATTN_UNROLL 4          /* positions per lane group per block: 32 per wave */
#define ATTN_CHUNK_ALIGN 128u  /* a chunk is a whole number of 4-wave blocks */
#define ATTN_MAX_SPLITS 64u

static __device__ __forceinline__ float aotx_attn_h(unsigned int word, int hi)
{
    return aotx_h2f((unsigned short)(hi ? (word >> 16) : (word & 0xFFFFu)));
}

/* One workgroup = 4 waves = one (token, KV head, context chunk). Each wave takes a
 * quarter of the chunk in blocks of 32 positions (8 lane groups x 4), loads the key and
 * value rows of a block together, and keeps a running maximum and mass (online softmax,
 * as cuda/model/attention.cu:90-104, per block instead of per position). The 4 waves'
 * (max, mass, sum) are merged in wave order through LDS; a chunk that is not the whole
 * context leaves its merged triple for the merge kernel. */
template <int D, int G>
__global__ __launch_bounds__(256) void aotx_attend_kernel(aotx_attn_args a)
{
    constexpr int NP = D / 64;          /* 16-byte pieces per lane per row */
    constexpr int E = 8 * NP;           /* elements per lane */
    constexpr int U = ATTN_UNROLL;      /* positions per lane group per block */
    __shared__ float wm[4][G], wl[4][G];
    __shared__ float wo[4][G][D];

    const unsigned int lane = threadIdx.x & 63u;
    const unsigned int wave = threadIdx.x >> 6;
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
    chunk = (chunk + ATTN_CHUNK_ALIGN - 1u) / ATTN_CHUNK_ALIGN * ATTN_CHUNK_ALIGN;
    const unsigned int st = (n + chunk - 1u) / chunk;   /* chunks of this token */
    if (c >= st) return;
    const unsigned int p0 = c * chunk;
    const unsigned int p1 = (p0 + chunk < n) ? p0 + chunk : n;
    /* this wave's quarter, in whole blocks of 8 * U positions */
    const unsigned int blk = 8u * U;
    const unsigned int nblk = (p1 - p0 + blk - 1u) / blk;
    const unsigned int per = (nblk + 3u) / 4u;
    const unsigned int w0 = p0 + wave * per * blk;
    const unsigned int w1 = (w0 + per * blk < p1) ? w0 + per * blk : p1;
    const unsigned int agent = a.agent[t];
    const aotx_kv_table *kv = &a.state->kv;
    const float scale = 1.0f / sqrtf((float)D);

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
    float o[G][E];
    float mrun[G], lrun[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        mrun[j] = -INFINITY;
        lrun[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) o[j][e] = 0.0f;
    }
    int missing = 0;
    const unsigned int kbase = kh * AOTX_KVL_BLOCK;
    const unsigned int vbase = (a.kv_heads + kh) * AOTX_KVL_BLOCK;

    for (unsigned int base = w0; base < w1; base += blk) {
        aotx_u4a kr[U][NP], vr[U][NP];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            unsigned int p = base + 8u * u + grp;
            valid[u] = p < w1;
            unsigned int pp = valid[u] ? p : w0;
            const unsigned char *bk = aotx_kvl_block(a.shape, kv, agent, a.layer, pp);
            const bool absent = bk == nullptr;
            if (absent) {
                missing = 1;
                valid[u] = false;
                bk = (const unsigned char *)a.q;    /* readable; replaced by zeros below */
            }
            const unsigned short *krow = (const unsigned short *)bk
                + (absent ? 0ull : (unsigned long long)(kbase + pp % AOTX_KVL_BLOCK) * D);
            const unsigned short *vrow = (const unsigned short *)bk
                + (absent ? 0ull : (unsigned long long)(vbase + pp % AOTX_KVL_BLOCK) * D);
            const aotx_u4a zero = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int pc = 0; pc < NP; ++pc) {
                aotx_u4a kk = *(const aotx_u4a *)(krow + (absent ? 0 : 64 * pc + 8 * sub));
                aotx_u4a vv = *(const aotx_u4a *)(vrow + (absent ? 0 : 64 * pc + 8 * sub));
                kr[u][pc] = absent ? zero : kk;
                vr[u][pc] = absent ? zero : vv;
            }
        }
        float sc[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int j = 0; j < G; ++j) sc[u][j] = 0.0f;
#pragma unroll
            for (int pc = 0; pc < NP; ++pc) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float k0 = aotx_attn_h(kr[u][pc][e], 0);
                    float k1 = aotx_attn_h(kr[u][pc][e], 1);
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        sc[u][j] += qv[j][8 * pc + 2 * e] * k0;
                        sc[u][j] += qv[j][8 * pc + 2 * e + 1] * k1;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < G; ++j) {
                float v = sc[u][j];
                v += __shfl_xor(v, 1, 64);
                v += __shfl_xor(v, 2, 64);
                v += __shfl_xor(v, 4, 64);
                sc[u][j] = valid[u] ? v * scale : -INFINITY;
            }
        }
        /* block maximum over the wave's 8 * U positions */
#pragma unroll
        for (int j = 0; j < G; ++j) {
            float mb = sc[0][j];
#pragma unroll
            for (int u = 1; u < U; ++u) mb = fmaxf(mb, sc[u][j]);
            mb = fmaxf(mb, __shfl_xor(mb, 8, 64));
            mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
            mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
            float mnew = fmaxf(mrun[j], mb);
            float shift = (mrun[j] == -INFINITY) ? 0.0f : expf(mrun[j] - mnew);
            if (mnew == -INFINITY) shift = 1.0f;
            lrun[j] *= shift;
#pragma unroll
            for (int e = 0; e < E; ++e) o[j][e] *= shift;
            mrun[j] = mnew;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float pw[G];
#pragma unroll
            for (int j = 0; j < G; ++j) {
                pw[j] = (sc[u][j] == -INFINITY) ? 0.0f : expf(sc[u][j] - mrun[j]);
                lrun[j] += pw[j];
            }
#pragma unroll
            for (int pc = 0; pc < NP; ++pc) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v0 = aotx_attn_h(vr[u][pc][e], 0);
                    float v1 = aotx_attn_h(vr[u][pc][e], 1);
#pragma unroll
                    for (int j = 0; j < G; ++j) {
                        o[j][8 * pc + 2 * e] += pw[j] * v0;
                        o[j][8 * pc + 2 * e + 1] += pw[j] * v1;
                    }
                }
            }
        }
    }
    /* the lane groups' sums of one wave (mass counted once per group: lanes of a group
     * hold the same weights) */
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float l = lrun[j];
        l += __shfl_xor(l, 8, 64);
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        lrun[j] = l;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float v = o[j][e];
            v += __shfl_xor(v, 8, 64);
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            o[j][e] = v;
        }
    }
    missing = __any(missing);
    if (missing && lane == 0u) atomicAdd(&a.state->faults, 1u);
    if (lane == 0u) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            wm[wave][j] = missing ? -INFINITY : mrun[j];
            wl[wave][j] = missing ? 0.0f : lrun[j];
        }
    }
    if (grp == 0u) {
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int pc = 0; pc < NP; ++pc)
#pragma unroll
                for (int e = 0; e < 8; ++e) wo[wave][j][64 * pc + 8 * sub + e] = missing ? 0.0f : o[j][8 * pc + e];
    }
    __syncthreads();
    /* merge the 4 waves in wave order */
    const unsigned int unit = t * a.kv_heads + kh;
    const unsigned int stride = G * (D + 2);
    float *mine = a.partial + ((unsigned long long)unit * S + c) * stride;
    for (unsigned int idx = threadIdx.x; idx < (unsigned int)(G * D); idx += 256u) {
        unsigned int j = idx / D, e = idx - j * D;
        float top = fmaxf(fmaxf(wm[0][j], wm[1][j]), fmaxf(wm[2][j], wm[3][j]));
        float msum = 0.0f, osum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            float f = (wm[w][j] == -INFINITY) ? 0.0f : expf(wm[w][j] - top);
            msum += wl[w][j] * f;
            osum += wo[w][j][e] * f;
        }
        if (st == 1u) {
            float back = msum > 0.0f ? 1.0f / msum : 0.0f;
            a.out[((unsigned long long)t * a.heads + kh * G + j) * D + e] = aotx_f2h(osum * back);
        } else {
            mine[j * (D + 2) + 2 + e] = osum;
            if (e == 0u) {
                mine[j * (D + 2)] = top;
                mine[j * (D + 2) + 1] = msum;
            }
        }
    }
}

/* Merge the chunks of every (token, KV head) that was split, in chunk order:
 * M = max m_c, out = half(sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M)). The chunk
 * weights are computed once into LDS; every load of the sums is independent. */
template <int D, int G>
__global__ __launch_bounds__(256) void aotx_attend_merge(aotx_attn_args a)
{
    __shared__ float fw[ATTN_MAX_SPLITS][G];
    __shared__ float inv[G];
    unsigned int tokens = a.m_dev ? *a.m_dev : a.tokens;
    if (tokens > a.tokens) tokens = a.tokens;
    const unsigned int unit = blockIdx.x;
    const unsigned int kh = unit % a.kv_heads;
    const unsigned int t = unit / a.kv_heads;
    if (t >= tokens) return;
    const unsigned int S = a.splits;
    const unsigned int n = a.pos[t] + 1u;
    unsigned int chunk = (n + S - 1u) / S;
    chunk = (chunk + ATTN_CHUNK_ALIGN - 1u) / ATTN_CHUNK_ALIGN * ATTN_CHUNK_ALIGN;
    const unsigned int st = (n + chunk - 1u) / chunk;
    if (st <= 1u) return;
    const unsigned int stride = G * (D + 2);
    const float *all = a.partial + (unsigned long long)unit * S * stride;
    if (threadIdx.x < (unsigned int)G) {
        const unsigned int j = threadIdx.x;
        float top = -INFINITY;
        for (unsigned int cc = 0; cc < st; ++cc) top = fmaxf(top, all[cc * stride + j * (D + 2)]);
        float msum = 0.0f;
        for (unsigned int cc = 0; cc < st; ++cc) {
            float mc = all[cc * stride + j * (D + 2)];
            float f = (mc == -INFINITY) ? 0.0f : expf(mc - top);
            fw[cc][j] = f;
            msum += all[cc * stride + j * (D + 2) + 1] * f;
        }
        inv[j] = msum > 0.0f ? 1.0f / msum : 0.0f;
    }
    __syncthreads();
    for (unsigned int idx = threadIdx.x; idx < (unsigned int)(G * D); idx += blockDim.x) {
        unsigned int j = idx / D;
        unsigned int e = idx - j * D;
        float osum = 0.0f;
#pragma unroll 8
        for (unsigned int cc = 0; cc < st; ++cc) osum += all[cc * stride + j * (D + 2) + 2 + e] * fw[cc][j];
        a.out[((unsigned long long)t * a.heads + kh * G + j) * D + e] = aotx_f2h(osum * inv[j]);
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
    /* about 1024 workgroups over the launch, chunks of at least 128 positions */
    unsigned int units = tokens * kv_heads;
    unsigned int s = (1024u + units - 1u) / units;
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
    a.chunk_max = max_context;
    a.shape = aotx_kvl_make(layers, kv_heads, head_dim);
    a.state = aotx_state_device();
    a.partial = partial != nullptr
        ? partial
        : (float *)aotx_scratch(AOTX_SCRATCH_ATTN_PARTIAL,
                                aotx_attn_scratch(tokens, kv_heads, a.splits, g, head_dim));
    dim3 grid(tokens * kv_heads * a.splits);
#define AOTX_ATTN_GO(DD, GG)                                                               \
    do {                                                                                   \
        hipLaunchKernelGGL((aotx_attend_kernel<DD, GG>), grid, dim3(256), 0, stream, a);   \
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
