/* Paged decode attention on gfx950.
 *
 * Reference: aotx_model_attend (cuda/model/attention.cu:22-154): one warp per (token,
 * query head), a single pass of online softmax over every position <= pos, scale
 * 1/sqrt(d), fp32 sums, out = half(sum / mass); keys and values come from the 16-position
 * layout blocks of cuda/model/kv_layout.cuh. Each query head re-reads its KV head there.
 *
 * Here one workgroup of 4 waves takes (token, KV head, context chunk):
 *   - all G = heads / kv_heads query heads of the KV head share one read of its keys and
 *     values (grouped-query sharing: the KV bytes are read once per token, not G times);
 *   - d/8 lanes hold one position, one 16-byte piece of the row each, so a wave step
 *     covers one whole 16-position layout block (4 KB of keys and 4 KB of values at
 *     d = 128) with fully used 16-byte loads, and the next block's loads are issued before
 *     the current block is computed;
 *   - scores are fp16 x fp16 products summed in fp32 (v_dot2_f32_f16), reduced over the
 *     row's lanes with lane shuffles; online softmax per block in base 2 (scores carry
 *     log2(e) / sqrt(d)), values accumulated in fp32;
 *   - the 4 waves' (max, mass, sum) are merged in wave order through LDS; the context is
 *     split over workgroups (flash-decoding) so that a batch of one still covers the GPU,
 *     and a merge kernel adds the chunks of a (token, KV head) in chunk order, so the
 *     result does not depend on timing.
 */
#include "aotx_internal.h"

#include <algorithm>
#include <stdlib.h>

typedef unsigned int aotx_u4a __attribute__((ext_vector_type(4)));
typedef _Float16 aotx_h2a __attribute__((ext_vector_type(2)));

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

#define ATTN_CHUNK_ALIGN 64u   /* a chunk is a whole number of 16-position blocks per wave */
#define ATTN_MAX_SPLITS 32u
#define ATTN_TARGET_GROUPS 256u

static __device__ __forceinline__ float aotx_attn_h(unsigned int word, int hi)
{
    return aotx_h2f((unsigned short)(hi ? (word >> 16) : (word & 0xFFFFu)));
}

/* A kernel-constant word (the device token count) read through the scalar cache. */
static __device__ __forceinline__ unsigned int aotx_attn_scalar(const unsigned int *p)
{
    return *(const __attribute__((address_space(4))) unsigned int *)p;
}

/* fp16 pair from one 32-bit word. The word arrives by value: a __builtin_bit_cast of a
 * vector element (v[e]) directly is miscompiled by this hipcc (it reads element 0). */
static __device__ __forceinline__ aotx_h2a aotx_as_h2(unsigned int word)
{
    return __builtin_bit_cast(aotx_h2a, word);
}

/* 2^x with the hardware v_exp_f32: exp2(-inf) = 0, results below 2^-126 flush to 0 (weights
 * that small do not change an fp32 sum of weights of order one). */
static __device__ __forceinline__ float aotx_exp2(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

template <int CTRL>
static __device__ __forceinline__ float aotx_dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, 0xF, false));
}

/* Sum over aligned groups of LPP (8 or 16) lanes, every lane of a group left with the
 * same total: quad swaps, then the mirrors within 8 and within 16. */
template <int LPP>
static __device__ __forceinline__ float aotx_row_sum(float v)
{
    v += aotx_dpp<0xB1>(v);     /* quad_perm [1,0,3,2] */
    v += aotx_dpp<0x4E>(v);     /* quad_perm [2,3,0,1] */
    v += aotx_dpp<0x141>(v);    /* row_half_mirror */
    if (LPP == 16) v += aotx_dpp<0x140>(v);    /* row_mirror */
    return v;
}

/* Max and sum over the lane groups of LPP lanes (every lane ends with the result). */
template <int LPP>
static __device__ __forceinline__ float aotx_groups_max(float v)
{
#pragma unroll
    for (int off = LPP; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

template <int LPP>
static __device__ __forceinline__ float aotx_groups_sum(float v)
{
#pragma unroll
    for (int off = LPP; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

/* Chunk length of a token with n positions under S splits (whole 64-position units). */
static __device__ __forceinline__ unsigned int aotx_attn_chunk(unsigned int n, unsigned int S)
{
    unsigned int chunk = (n + S - 1u) / S;
    return (chunk + ATTN_CHUNK_ALIGN - 1u) / ATTN_CHUNK_ALIGN * ATTN_CHUNK_ALIGN;
}

template <int D>
struct aotx_attn_geom {
    static constexpr int LPP = D / 8;          /* lanes per position */
    static constexpr int NG = 64 / LPP;        /* positions per wave instruction */
    static constexpr int U = 16 / NG;          /* instructions per 16-position block */
};

/* One workgroup = W waves = one (token, KV head, context chunk). */
template <int D, int G, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(G == 1 ? 3 : (G <= 4 ? 2 : 1)))) void aotx_attend_kernel(aotx_attn_args a)
{
    constexpr int LPP = aotx_attn_geom<D>::LPP;
    constexpr int NG = aotx_attn_geom<D>::NG;
    constexpr int U = aotx_attn_geom<D>::U;
    __shared__ float wm[W][G], wl[W][G];
    __shared__ float wo[W][G][D];

    const unsigned int lane = threadIdx.x & 63u;
    const unsigned int wave = threadIdx.x >> 6;
    const unsigned int grp = lane / LPP;
    const unsigned int sub = lane % LPP;
    unsigned int tokens = a.m_dev ? aotx_attn_scalar(a.m_dev) : a.tokens;
    if (tokens > a.tokens) tokens = a.tokens;
    const unsigned int S = a.splits;
    const unsigned int c = blockIdx.x % S;
    const unsigned int rest = blockIdx.x / S;
    const unsigned int kh = rest % a.kv_heads;
    const unsigned int t = rest / a.kv_heads;
    if (t >= tokens) return;
    const unsigned int n = a.pos[t] + 1u;
    const unsigned int chunk = aotx_attn_chunk(n, S);
    const unsigned int st = (n + chunk - 1u) / chunk;   /* chunks of this token */
    if (c >= st) return;
    const unsigned int p0 = c * chunk;
    const unsigned int p1 = (p0 + chunk < n) ? p0 + chunk : n;
    /* this wave's quarter, in whole 16-position blocks */
    const unsigned int nblk = (p1 - p0 + 15u) / 16u;
    const unsigned int per = (nblk + W - 1u) / W;
    const unsigned int b0 = p0 / 16u + wave * per;
    unsigned int b1 = b0 + per;
    if (b1 > (p1 + 15u) / 16u) b1 = (p1 + 15u) / 16u;
    const unsigned int agent = a.agent[t];
    const aotx_kv_table *kv = &a.state->kv;
    /* base-2 scores: s * log2(e) / sqrt(d) */
    const float scale = 1.4426950408889634f / sqrtf((float)D);

    aotx_h2a qv[G][4];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const unsigned short *qrow = a.q + ((unsigned long long)t * a.heads + kh * G + j) * D;
        aotx_u4a w = *(const aotx_u4a *)(qrow + 8 * sub);
#pragma unroll
        for (int e = 0; e < 4; ++e) qv[j][e] = aotx_as_h2(w[e]);
    }
    float o[G][8];
    float mrun[G], lrun[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        mrun[j] = -INFINITY;
        lrun[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[j][e] = 0.0f;
    }
    int missing = 0;
    /* byte offsets of this lane's piece of row grp of the key and value heads */
    const unsigned int kbyte = ((kh * AOTX_KVL_BLOCK + grp) * D + 8u * sub) * 2u;
    const unsigned int vbyte = (((a.kv_heads + kh) * AOTX_KVL_BLOCK + grp) * D + 8u * sub) * 2u;

    aotx_u4a kr[3][U], vr[3][U];     /* a ring of three blocks: two in flight */
    bool absent[3];
    /* layout-block pointers of the wave's blocks, 64 at a time, lane i holding block
     * wbase + i; a block is fetched from the lane that holds it */
    unsigned long long pages = 0ull;
    unsigned int wbase = b0;
#define ATTN_WINDOW(B0)                                                                     \
    do {                                                                                    \
        wbase = (B0);                                                                       \
        unsigned int bl = wbase + lane;                                                     \
        pages = bl < b1 ? (unsigned long long)aotx_kvl_block(a.shape, kv, agent, a.layer, bl * 16u) \
                        : 0ull;                                                             \
    } while (0)
#define ATTN_LOAD(BUF, B)                                                                   \
    do {                                                                                    \
        if ((B) - wbase >= 64u) ATTN_WINDOW(B);                                             \
        unsigned long long pb = __shfl(pages, (int)((B) - wbase), 64);                     \
        /* the block is the same for the whole wave: its address goes to scalar registers, \
         * as a buffer resource whose range is empty for a missing page (loads give 0) */   \
        pb = ((unsigned long long)(unsigned int)__builtin_amdgcn_readfirstlane((unsigned int)(pb >> 32)) << 32) \
           | (unsigned long long)(unsigned int)__builtin_amdgcn_readfirstlane((unsigned int)pb); \
        absent[BUF] = pb == 0ull;                                                           \
        __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(                      \
            (void *)pb, (short)0, absent[BUF] ? 0 : (int)a.shape.block_bytes, 0x00020000);  \
        _Pragma("unroll") for (int u = 0; u < U; ++u) {                                     \
            kr[BUF][u] = __builtin_amdgcn_raw_buffer_load_b128(rs, kbyte + u * NG * D * 2, 0, 0); \
            vr[BUF][u] = __builtin_amdgcn_raw_buffer_load_b128(rs, vbyte + u * NG * D * 2, 0, 0); \
        }                                                                                   \
    } while (0)

#define ATTN_COMPUTE(BUF, B)                                                                \
    do {                                                                                    \
        if (absent[BUF]) missing = 1;                                                       \
        float sc[U][G];                                                                     \
        _Pragma("unroll") for (int u = 0; u < U; ++u) {                                     \
            unsigned int p = (B) * 16u + (unsigned int)u * NG + grp;                        \
            bool ok = p >= p0 && p < p1 && !absent[BUF];                                    \
            aotx_u4a kk = kr[BUF][u];                                                       \
            _Pragma("unroll") for (int j = 0; j < G; ++j) {                                 \
                float v = 0.0f;                                                             \
                _Pragma("unroll") for (int e = 0; e < 4; ++e)                               \
                    v = __builtin_amdgcn_fdot2(qv[j][e], aotx_as_h2(kk[e]), v, false);       \
                v = aotx_row_sum<LPP>(v);                                                   \
                sc[u][j] = ok ? v * scale : -INFINITY;                                      \
            }                                                                               \
        }                                                                                   \
        _Pragma("unroll") for (int j = 0; j < G; ++j) {                                     \
            float mb = sc[0][j];                                                            \
            _Pragma("unroll") for (int u = 1; u < U; ++u) mb = fmaxf(mb, sc[u][j]);         \
            mb = aotx_groups_max<LPP>(mb);                                                  \
            float mnew = fmaxf(mrun[j], mb);                                                \
            if (mnew != mrun[j]) {                                                          \
                float shift = aotx_exp2(mrun[j] - mnew);    /* 0 from -inf */               \
                lrun[j] *= shift;                                                           \
                _Pragma("unroll") for (int e = 0; e < 8; ++e) o[j][e] *= shift;             \
                mrun[j] = mnew;                                                             \
            }                                                                               \
        }                                                                                   \
        _Pragma("unroll") for (int u = 0; u < U; ++u) {                                     \
            aotx_u4a vv = vr[BUF][u];                                                       \
            float vf[8];                                                                    \
            _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                 \
                vf[2 * e] = aotx_attn_h(vv[e], 0);                                          \
                vf[2 * e + 1] = aotx_attn_h(vv[e], 1);                                      \
            }                                                                               \
            _Pragma("unroll") for (int j = 0; j < G; ++j) {                                 \
                float pw = aotx_exp2(sc[u][j] - mrun[j]);   /* 0 for a masked position */   \
                lrun[j] += pw;                                                              \
                _Pragma("unroll") for (int e = 0; e < 8; ++e) o[j][e] += pw * vf[e];        \
            }                                                                               \
        }                                                                                   \
    } while (0)

    if (b0 < b1) {
        unsigned int b = b0;
        ATTN_WINDOW(b0);
        ATTN_LOAD(0, b);
        if (b + 1u < b1) ATTN_LOAD(1, b + 1u);
        for (;;) {
            if (b + 2u < b1) ATTN_LOAD(2, b + 2u);
            ATTN_COMPUTE(0, b);
            b += 1u;
            if (b >= b1) break;
            if (b + 2u < b1) ATTN_LOAD(0, b + 2u);
            ATTN_COMPUTE(1, b);
            b += 1u;
            if (b >= b1) break;
            if (b + 2u < b1) ATTN_LOAD(1, b + 2u);
            ATTN_COMPUTE(2, b);
            b += 1u;
            if (b >= b1) break;
        }
    }
#undef ATTN_WINDOW
#undef ATTN_LOAD
#undef ATTN_COMPUTE

    /* the lane groups' sums of one wave (mass counted once per group: lanes of a group
     * hold the same weights) */
#pragma unroll
    for (int j = 0; j < G; ++j) {
        lrun[j] = aotx_groups_sum<LPP>(lrun[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[j][e] = aotx_groups_sum<LPP>(o[j][e]);
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
            for (int e = 0; e < 8; ++e) wo[wave][j][8 * sub + e] = missing ? 0.0f : o[j][e];
    }
    __syncthreads();
    /* merge the 4 waves in wave order; the chunk's triple keeps the base-2 maximum */
    const unsigned int unit = t * a.kv_heads + kh;
    const unsigned int stride = G * (D + 2);
    float *mine = a.partial + ((unsigned long long)unit * S + c) * stride;
    for (unsigned int idx = threadIdx.x; idx < (unsigned int)(G * D); idx += 64u * W) {
        unsigned int j = idx / D, e = idx - j * D;
        float top = wm[0][j];
#pragma unroll
        for (int w = 1; w < W; ++w) top = fmaxf(top, wm[w][j]);
        float msum = 0.0f, osum = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            float f = (wm[w][j] == -INFINITY) ? 0.0f : exp2f(wm[w][j] - top);
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
 * M = max m_c, out = half(sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M)). One workgroup
 * per (token, KV head, query head), one thread per output column; every thread issues all
 * of its loads (each chunk's maximum, mass and sum) at once and forms the chunk weights
 * itself, so the merge is one round trip to memory with no LDS and no barrier. */
template <int D, int G>
__global__ __launch_bounds__(D) void aotx_attend_merge(aotx_attn_args a)
{
    unsigned int tokens = a.m_dev ? aotx_attn_scalar(a.m_dev) : a.tokens;
    if (tokens > a.tokens) tokens = a.tokens;
    const unsigned int unit = blockIdx.x;
    const unsigned int j = blockIdx.y;
    const unsigned int e = threadIdx.x;
    const unsigned int kh = unit % a.kv_heads;
    const unsigned int t = unit / a.kv_heads;
    if (t >= tokens) return;
    const unsigned int S = a.splits;
    const unsigned int n = a.pos[t] + 1u;
    const unsigned int chunk = aotx_attn_chunk(n, S);
    const unsigned int st = (n + chunk - 1u) / chunk;
    if (st <= 1u) return;
    const unsigned int stride = G * (D + 2);
    const float *all = a.partial + (unsigned long long)unit * S * stride + j * (D + 2);
    float mc[ATTN_MAX_SPLITS], lc[ATTN_MAX_SPLITS], oc[ATTN_MAX_SPLITS];
#pragma unroll
    for (unsigned int c = 0; c < ATTN_MAX_SPLITS; ++c) {
        const bool live = c < st;
        mc[c] = live ? all[c * stride] : -INFINITY;
        lc[c] = live ? all[c * stride + 1u] : 0.0f;
        oc[c] = live ? all[c * stride + 2u + e] : 0.0f;
    }
    float top = -INFINITY;
#pragma unroll
    for (unsigned int c = 0; c < ATTN_MAX_SPLITS; ++c) top = fmaxf(top, mc[c]);
    float msum = 0.0f, osum = 0.0f;
#pragma unroll
    for (unsigned int c = 0; c < ATTN_MAX_SPLITS; ++c) {
        if (c < st) {
            const float f = mc[c] == -INFINITY ? 0.0f : aotx_exp2(mc[c] - top);
            msum += lc[c] * f;
            osum += oc[c] * f;
        }
    }
    const float back = msum > 0.0f ? 1.0f / msum : 0.0f;
    a.out[((unsigned long long)t * a.heads + kh * G + j) * D + e] = aotx_f2h(osum * back);
}

/* ---------------------------------------------------------------------------------------
 * Host side
 * ------------------------------------------------------------------------------------- */

unsigned int aotx_attn_splits(unsigned int tokens, unsigned int kv_heads,
                              unsigned int max_context)
{
    /* about ATTN_TARGET_GROUPS workgroups over the launch (AOTX_ATTN_GROUPS overrides it
     * for measurement sweeps), chunks of at least 64 positions */
    static const unsigned int target = [] {
        const char *e = getenv("AOTX_ATTN_GROUPS");
        unsigned int v = e != nullptr ? (unsigned int)strtoul(e, nullptr, 10) : 0u;
        return v != 0u ? v : ATTN_TARGET_GROUPS;
    }();
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
    /* 8 waves per workgroup (4 for 8 query heads per KV head, whose registers allow no
     * more); AOTX_ATTN_WAVES=4 selects 4 for measurement sweeps */
    static const unsigned int waves = [] {
        const char *e = getenv("AOTX_ATTN_WAVES");
        return e != nullptr && strtoul(e, nullptr, 10) == 4u ? 4u : 8u;
    }();
#define AOTX_ATTN_GO(DD, GG)                                                               \
    do {                                                                                   \
        if (waves == 8u && GG <= 4)                                                        \
            hipLaunchKernelGGL((aotx_attend_kernel<DD, GG, 8>), grid, dim3(512), 0, stream, a); \
        else                                                                               \
            hipLaunchKernelGGL((aotx_attend_kernel<DD, GG, 4>), grid, dim3(256), 0, stream, a); \
        AOTX_LAUNCH_CHECK();                                                               \
        if (a.splits > 1u) {                                                               \
            hipLaunchKernelGGL((aotx_attend_merge<DD, GG>), dim3(tokens * kv_heads, GG),   \
                               dim3(DD), 0, stream, a);                                    \
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
