/* Device code of paged decode attention (attention.hip): the per-workgroup body.
 */
#ifndef AOTX_ATTENTION_DEV_H
#define AOTX_ATTENTION_DEV_H

#include "aotx_internal.h"
#include "coherent.h"

typedef unsigned int aotx_u4a __attribute__((ext_vector_type(4)));
typedef _Float16 aotx_h4a __attribute__((ext_vector_type(4)));
typedef short aotx_s4a __attribute__((ext_vector_type(4)));
typedef _Float16 aotx_h8a __attribute__((ext_vector_type(8)));
typedef float aotx_f4a __attribute__((ext_vector_type(4)));

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
    unsigned int *count;          /* [tokens*kv_heads] chunk arrivals, zero between launches */
    unsigned int out_frag;        /* out in the fragment layout (aotx_xfrag_at) */
};

/* Half index of out for query row t, head h, dimension e. */
static __device__ __forceinline__ unsigned long long aotx_attn_out_at(const aotx_attn_args &a,
                                                                    unsigned int t, unsigned int h,
                                                                    unsigned int e, unsigned int d)
{
    return a.out_frag ? aotx_xfrag_at(t, h * d + e) : ((unsigned long long)t * a.heads + h) * d + e;
}

#define ATTN_CHUNK_ALIGN 64u   /* a chunk is a whole number of 16-position blocks per wave */
#define ATTN_MAX_SPLITS 32u
#define ATTN_TARGET_GROUPS 192u
/* Cache policy bits of the decode key/value block loads: 2 is the non-temporal (nt) bit.
 * Each block is read once per step, so it is streamed past the caches instead of being
 * kept there (batch 32 at context 2048: 50.2 -> 46.0 us per launch; sc1, 16, no change).
 * Prompt pieces keep the default policy: their runs re-read a sequence's prefix. */
#ifndef AOTX_ATTN_CPOL
#define AOTX_ATTN_CPOL 2
#endif
#ifndef AOTX_ATTN_NT_BLOCKS
#define AOTX_ATTN_NT_BLOCKS 32u
#endif

/* A kernel-constant word (the device token count) read through the scalar cache. */
static __device__ __forceinline__ unsigned int aotx_attn_scalar(const unsigned int *p)
{
    return *(const __attribute__((address_space(4))) unsigned int *)p;
}

/* 2^x with the hardware v_exp_f32: exp2(-inf) = 0, results below 2^-126 flush to 0 (weights
 * that small do not change an fp32 sum of weights of order one). */
static __device__ __forceinline__ float aotx_exp2(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

/* Chunk partials cross workgroups on different XCDs: device-scope stores and loads. */
static __device__ __forceinline__ void aotx_attn_put(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ float aotx_attn_get(const float *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Chunk length of a token with n positions under S splits (whole 64-position units). */
static __device__ __forceinline__ unsigned int aotx_attn_chunk(unsigned int n, unsigned int S)
{
    unsigned int chunk = (n + S - 1u) / S;
    return (chunk + ATTN_CHUNK_ALIGN - 1u) / ATTN_CHUNK_ALIGN * ATTN_CHUNK_ALIGN;
}

/* The block loop shared by the attention bodies. They expect, in scope: a, kv, agent, b1,
 * lane, r, g, kbyte, vbyte, wbase, pages, kr, vr, absent, CPOL, KK, VP, NS, VS, D, qb, o,
 * mrun, lrun, missing, scale, p0, plim, vw (this wave's LDS value slot) and vtr.
 * MMA_WINDOW(B0): the page addresses of blocks B0 .. B0 + 63 (one per lane).
 * MMA_LOAD(BUF, B): block B's keys and values into register buffer BUF.
 * MMA_COMPUTE(BUF, B): block B's scores, online softmax and P . V. */
#define MMA_WINDOW(B0)                                                                      \
    do {                                                                                    \
        wbase = (B0);                                                                       \
        unsigned int bl = wbase + lane;                                                     \
        pages = bl < b1 ? (unsigned long long)aotx_kvl_block(a.shape, kv, agent, a.layer, bl * 16u) \
                        : 0ull;                                                             \
    } while (0)
#define MMA_LOAD(BUF, B)                                                                    \
    do {                                                                                    \
        if ((B) - wbase >= 64u) MMA_WINDOW(B);                                              \
        unsigned long long pb = __shfl(pages, (int)((B) - wbase), 64);                     \
        pb = ((unsigned long long)(unsigned int)__builtin_amdgcn_readfirstlane((unsigned int)(pb >> 32)) << 32) \
           | (unsigned long long)(unsigned int)__builtin_amdgcn_readfirstlane((unsigned int)pb); \
        absent[BUF] = pb == 0ull;                                                           \
        __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(                      \
            (void *)pb, (short)0, absent[BUF] ? 0 : (int)a.shape.block_bytes, 0x00020000);  \
        _Pragma("unroll") for (int kk = 0; kk < KK; ++kk)                                   \
            kr[BUF][kk] = __builtin_amdgcn_raw_buffer_load_b128(rs, kbyte + kk * 64, 0, CPOL); \
        _Pragma("unroll") for (int u = 0; u < VP; ++u)                                      \
            vr[BUF][u] = __builtin_amdgcn_raw_buffer_load_b128(rs, vbyte + u * 1024, 0, CPOL); \
    } while (0)

#define MMA_COMPUTE(BUF, B)                                                                 \
    do {                                                                                    \
        if (absent[BUF]) missing = 1;                                                       \
        aotx_f4a sc = {0.0f, 0.0f, 0.0f, 0.0f};                                             \
        _Pragma("unroll") for (int kk = 0; kk < KK; ++kk)                                   \
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(                                    \
                __builtin_bit_cast(aotx_h8a, kr[BUF][kk]), qb[kk], sc, 0, 0, 0);             \
        /* the block's values into this wave's LDS slot (row-major, padded rows) */         \
        _Pragma("unroll") for (int u = 0; u < VP; ++u) {                                    \
            const unsigned int piece = (unsigned int)u * 64u + lane;                        \
            *(aotx_u4a *)(vw + (piece / (D / 8)) * VS + (piece % (D / 8)) * 8u) = vr[BUF][u]; \
        }                                                                                   \
        float pr[4];                                                                        \
        float mb = -INFINITY;                                                               \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                     \
            const unsigned int p = (B) * 16u + 4u * g + (unsigned int)i;                    \
            const bool ok = p >= p0 && p < plim && !absent[BUF];                            \
            pr[i] = ok ? sc[i] * scale : -INFINITY;                                         \
            mb = fmaxf(mb, pr[i]);                                                          \
        }                                                                                   \
        mb = fmaxf(mb, __shfl_xor(mb, 16, 64));                                             \
        mb = fmaxf(mb, __shfl_xor(mb, 32, 64));                                             \
        const float mnew = fmaxf(mrun, mb);                                                 \
        /* 0 from -inf; a column with no position yet keeps its (empty) sums */           \
        const float shift = mnew == -INFINITY ? 1.0f : aotx_exp2(mrun - mnew);              \
        mrun = mnew;                                                                        \
        aotx_h4a pa;                                                                        \
        float mass = 0.0f;                                                                  \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                     \
            const _Float16 ph = mnew == -INFINITY ? (_Float16)0.0f                          \
                              : (_Float16)aotx_exp2(pr[i] - mnew);   /* 0 when masked */    \
            pa[i] = ph;                                                                     \
            mass += (float)ph;                                                              \
        }                                                                                   \
        lrun = lrun * shift + mass;                                                         \
        /* the accumulators of heads 4g + i take those heads' shifts */                     \
        if (__any(shift != 1.0f)) {                                                         \
            float sh[4];                                                                    \
            _Pragma("unroll") for (int i = 0; i < 4; ++i) sh[i] = __shfl(shift, (int)(4u * g) + i, 64); \
            _Pragma("unroll") for (int cc = 0; cc < NS; ++cc)                               \
                _Pragma("unroll") for (int i = 0; i < 4; ++i) o[cc][i] *= sh[i];            \
        }                                                                                   \
        _Pragma("unroll") for (int cc = 0; cc < NS; ++cc) {                                 \
            /* B[k = 4g + i][n = r] = V[row 4g + i][16 cc + r]: one transposing read, each \
             * lane addressing 4 halves of a row (aotx_vtr) */                               \
            const aotx_s4a t4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(                    \
                (__attribute__((address_space(3))) aotx_s4a *)(vw + vtr + 16u * (unsigned int)cc)); \
            o[cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(aotx_h4a, t4), \
                                                          o[cc], 0, 0, 0);                  \
        }                                                                                   \
    } while (0)

/* MMA_COMPUTE_SH(KL, VL, B, LIVE, ABS): MMA_COMPUTE over a block its workgroup staged in
 * LDS (keys at KL, values at VL, rows of VS halves); LIVE: the block is in this wave's
 * range; ABS: its page is missing. */
#define MMA_COMPUTE_SH(KL, VL, B, LIVE, ABS)                                                \
    do {                                                                                    \
        aotx_f4a sc = {0.0f, 0.0f, 0.0f, 0.0f};                                             \
        _Pragma("unroll") for (int kk = 0; kk < KK; ++kk)                                   \
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(                                    \
                *(const aotx_h8a *)((KL) + r * VS + 32u * (unsigned int)kk + 8u * g), qb[kk], sc, 0, 0, 0); \
        float pr[4];                                                                        \
        float mb = -INFINITY;                                                               \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                     \
            const unsigned int p = (B) * 16u + 4u * g + (unsigned int)i;                    \
            const bool ok = (LIVE) && p >= p0 && p < plim && !(ABS);                        \
            pr[i] = ok ? sc[i] * scale : -INFINITY;                                         \
            mb = fmaxf(mb, pr[i]);                                                          \
        }                                                                                   \
        mb = fmaxf(mb, __shfl_xor(mb, 16, 64));                                             \
        mb = fmaxf(mb, __shfl_xor(mb, 32, 64));                                             \
        const float mnew = fmaxf(mrun, mb);                                                 \
        const float shift = mnew == -INFINITY ? 1.0f : aotx_exp2(mrun - mnew);              \
        mrun = mnew;                                                                        \
        aotx_h4a pa;                                                                        \
        float mass = 0.0f;                                                                  \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                     \
            const _Float16 ph = mnew == -INFINITY ? (_Float16)0.0f                          \
                              : (_Float16)aotx_exp2(pr[i] - mnew);                          \
            pa[i] = ph;                                                                     \
            mass += (float)ph;                                                              \
        }                                                                                   \
        lrun = lrun * shift + mass;                                                         \
        if (__any(shift != 1.0f)) {                                                         \
            float sh[4];                                                                    \
            _Pragma("unroll") for (int i = 0; i < 4; ++i) sh[i] = __shfl(shift, (int)(4u * g) + i, 64); \
            _Pragma("unroll") for (int cc = 0; cc < NS; ++cc)                               \
                _Pragma("unroll") for (int i = 0; i < 4; ++i) o[cc][i] *= sh[i];            \
        }                                                                                   \
        _Pragma("unroll") for (int cc = 0; cc < NS; ++cc) {                                 \
            const aotx_s4a t4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(                    \
                (__attribute__((address_space(3))) aotx_s4a *)((VL) + vtr + 16u * (unsigned int)cc)); \
            o[cc] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(aotx_h4a, t4), \
                                                          o[cc], 0, 0, 0);                  \
        }                                                                                   \
    } while (0)

/* One workgroup = W waves = one (token, KV head, context chunk); each wave takes a
 * contiguous run of 16-position layout blocks. Per wave and block, on the matrix cores:
 *   - scores S[pos][head] = K . q^T: one v_mfma_f32_16x16x32_f16 per 32 of d, keys as the A
 *     operand straight from memory (lane (r, g) holds row r, d 32kk + 8g..+7), the query
 *     heads of the KV head as the B columns (heads past G are zero);
 *   - the score layout (lane (r, g): head r, positions 4g..4g+3) is the A-operand layout of
 *     v_mfma_f32_16x16x16_f16, so the probabilities feed P . V as fp16 (the mass adds the
 *     same rounded probabilities, so numerator and denominator agree);
 *   - the values need positions along k: the wave writes its block (row-major, rows padded
 *     against bank conflicts) to a private LDS slot and reads 16-bit columns back;
 *   - online softmax in base 2 per head with a max over the 4 lane groups of the head.
 * The output accumulators hold heads 4g..4g+3 x 16 d columns per lane and PV step. */
template <int D, int G, int W, int QT>
static __device__ __forceinline__ void aotx_attend_body(const aotx_attn_args &a, unsigned int bx)
{
    static_assert(QT == 1, "one query per workgroup: prompt pieces take aotx_attend_runs");
    constexpr int C = G * QT;           /* score columns: G heads */
    static_assert(C <= 16, "one MFMA tile of query columns");
    constexpr int KK = D / 32;          /* score MFMA steps */
    constexpr int VP = D / 32;          /* 16-byte value pieces per lane per block */
    constexpr int NS = D / 16;          /* P.V MFMAs (16 d columns each) */
    constexpr int VS = D + 8;           /* LDS row stride of a value block (halves) */
    __shared__ float wm[W][C], wl[W][C];
    __shared__ float wo[W][C][D];
    __shared__ __attribute__((aligned(16))) unsigned short vl[W][16 * VS];

    const unsigned int lane = threadIdx.x & 63u;
    const unsigned int wave = threadIdx.x >> 6;
    const unsigned int r = lane & 15u, g = lane >> 4;
    /* one unconditional scalar load (of the device count, or of a word of the positions
     * when there is none, then not used): a load under a condition would be waited for
     * where the paths join. (Not the address of an argument: that would point at a private
     * copy of the arguments, which a scalar load cannot read.) */
    const unsigned int counted = aotx_attn_scalar(a.m_dev != nullptr ? a.m_dev : a.pos);
    unsigned int tokens = a.m_dev != nullptr ? counted : a.tokens;
    unsigned int S, c, kh, t, n, st, p0, p1, nq = 1u, plim;
    unsigned int agent;
    S = a.splits;
    /* chunk-major: the workgroups of one chunk index are consecutive, so they spread
     * over every XCD whichever chunks are empty (dispatch goes round the XCDs) */
    const unsigned int units = a.tokens * a.kv_heads;
    c = bx / units;
    const unsigned int rest = bx - c * units;
    kh = rest % a.kv_heads;
    t = rest / a.kv_heads;
    /* the token's position and slot are read before its row count is known (t is below
     * the launch's token capacity, so both words exist): one memory round trip for all
     * three, where a load after the count's test would wait for the count first */
    const unsigned int pos_t = a.pos[t];
    agent = a.agent[t];
    __builtin_amdgcn_sched_barrier(0);
    if (tokens > a.tokens) tokens = a.tokens;
    /* the test reads both words, so neither load is sunk past it (a position of all
     * ones, which no sequence reaches, would end the workgroup as a token past the
     * count does) */
    if (t >= tokens || (pos_t & agent) == 0xFFFFFFFFu) return;
    n = pos_t + 1u;
    const unsigned int chunk = aotx_attn_chunk(n, S);
    st = (n + chunk - 1u) / chunk;
    if (c >= st) return;
    p0 = c * chunk;
    p1 = (p0 + chunk < n) ? p0 + chunk : n;
    plim = p1;
    const unsigned int nblk = (p1 - p0 + 15u) / 16u;
    const unsigned int per = (nblk + W - 1u) / W;
    const unsigned int b0 = p0 / 16u + wave * per;
    unsigned int b1 = b0 + per;
    if (b1 > (p1 + 15u) / 16u) b1 = (p1 + 15u) / 16u;
    const aotx_kv_table *kv = &a.state->kv;
    const float scale = 1.4426950408889634f / sqrtf((float)D);

    aotx_h8a qb[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
        aotx_u4a w = {0u, 0u, 0u, 0u};
        const unsigned int qi = r / (unsigned int)G, hh = r % (unsigned int)G;
        if (r < (unsigned int)C && qi < nq)
            w = co_load4(a.q + ((unsigned long long)(t + qi) * a.heads + kh * G + hh) * D
                             + 32 * kk + 8 * g);
        qb[kk] = __builtin_bit_cast(aotx_h8a, w);
    }
    float mrun = -INFINITY, lrun = 0.0f;     /* head r of this lane */
    aotx_f4a o[NS];
#pragma unroll
    for (int cc = 0; cc < NS; ++cc) o[cc] = (aotx_f4a){0.0f, 0.0f, 0.0f, 0.0f};
    int missing = 0;
    const unsigned int kbyte = ((kh * AOTX_KVL_BLOCK + r) * D + 8u * g) * 2u;
    const unsigned int vbyte = ((a.kv_heads + kh) * AOTX_KVL_BLOCK * D + lane * 8u) * 2u;
    unsigned short *vw = vl[wave];
    /* ds_read_tr16_b64: lane j of a 16-lane group gets halves j % 4 of the chunks that
     * lanes 4e + j / 4 address, e = 0..3; lane (r, g) = 16 g + 4 i + q addresses row 4g + i,
     * halves 4q..4q+3 of a 16-column slice, so that it gets column r of rows 4g..4g+3 */
    const unsigned int vtr = (4u * g + (lane & 15u) / 4u) * VS + 4u * (lane & 3u);

    aotx_u4a kr[2][KK], vr[2][VP];
    bool absent[2];
    unsigned long long pages = 0ull;
    unsigned int wbase = b0;
    /* The next block's loads are issued on every step: past the wave's last block the page
     * address is zero and the loads go through a zero-size resource (they return zeros
     * and touch no memory; that buffer is never computed). With a load on one path only,
     * the compiler's wait before a block's MFMAs would also cover part of the next block's
     * loads. */
#define MMA_RUN()                                                                           \
    do {                                                                                    \
        if (b0 < b1) {                                                                      \
            unsigned int b = b0;                                                            \
            MMA_WINDOW(b0);                                                                 \
            MMA_LOAD(0, b);                                                                 \
            for (;;) {                                                                      \
                MMA_LOAD(1, b + 1u);                                                        \
                MMA_COMPUTE(0, b);                                                          \
                b += 1u;                                                                    \
                if (b >= b1) break;                                                         \
                MMA_LOAD(0, b + 1u);                                                        \
                MMA_COMPUTE(1, b);                                                          \
                b += 1u;                                                                    \
                if (b >= b1) break;                                                         \
            }                                                                               \
        }                                                                                   \
    } while (0)
    /* runs of up to AOTX_ATTN_NT_BLOCKS blocks per wave stream with the policy above; longer
     * runs (one wave's run sets a long sequence's time) keep the default policy */
    if (QT == 1 && b1 - b0 <= AOTX_ATTN_NT_BLOCKS) {
        constexpr int CPOL = AOTX_ATTN_CPOL;
        MMA_RUN();
    } else {
        constexpr int CPOL = 0;
        MMA_RUN();
    }
#undef MMA_RUN
    /* a head's mass over its 4 lane groups */
    lrun += __shfl_xor(lrun, 16, 64);
    lrun += __shfl_xor(lrun, 32, 64);
    missing = __any(missing);
    if (missing && lane == 0u) atomicAdd(&a.state->faults, 1u);
    if (g == 0u && r < (unsigned int)C) {
        wm[wave][r] = missing ? -INFINITY : mrun;
        wl[wave][r] = missing ? 0.0f : lrun;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned int head = 4u * g + (unsigned int)i;
        if (head < (unsigned int)C) {
#pragma unroll
            for (int cc = 0; cc < NS; ++cc) wo[wave][head][16 * cc + r] = missing ? 0.0f : o[cc][i];
        }
    }
    __syncthreads();
    /* merge the W waves in wave order */
    const unsigned int unit = t * a.kv_heads + kh;
    const unsigned int stride = G * (D + 2);
    float *mine = a.partial + ((unsigned long long)unit * S + c) * stride;
    for (unsigned int idx = threadIdx.x; idx < (unsigned int)(C * D / 2); idx += 64u * W) {
        const unsigned int j = idx / (D / 2), e = 2u * (idx - j * (D / 2));
        /* column j: query j / G (of the prompt piece; 0 in decode), head j % G */
        const unsigned int qj = j / (unsigned int)G, hj = j % (unsigned int)G;
        if (qj >= nq) continue;
        float top = wm[0][j];
#pragma unroll
        for (int w = 1; w < W; ++w) top = fmaxf(top, wm[w][j]);
        float msum = 0.0f, osum[2] = {0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < W; ++w) {
            float f = (wm[w][j] == -INFINITY) ? 0.0f : exp2f(wm[w][j] - top);
            msum += wl[w][j] * f;
            osum[0] += wo[w][j][e] * f;
            osum[1] += wo[w][j][e + 1u] * f;
        }
        if (st == 1u) {
            float back = msum > 0.0f ? 1.0f / msum : 0.0f;
            co_store2h(a.out + aotx_attn_out_at(a, t + qj, kh * G + hj, e, D),
                           aotx_f2h(osum[0] * back), aotx_f2h(osum[1] * back));
        } else {
            aotx_attn_put(mine + j * (D + 2) + 2 + e, osum[0]);
            aotx_attn_put(mine + j * (D + 2) + 3 + e, osum[1]);
            if (e == 0u) {
                aotx_attn_put(mine + j * (D + 2), top);
                aotx_attn_put(mine + j * (D + 2) + 1, msum);
            }
        }
    }
    if (st == 1u) return;
    /* The last chunk of the (token, KV head) to finish merges all of them, in chunk order:
     * M = max m_c, out = half(sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M)). Partials
     * are written and read as device-scope accesses (through to the point where all XCDs
     * meet, past the per-XCD L2), and every one of this workgroup's writes has completed
     * before its arrival is counted, so no cache write-back or invalidation is needed. The
     * last arrival puts the counter back to zero for the next launch. */
    __shared__ unsigned int last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0u) {
        last = atomicAdd(a.count + unit, 1u) == st - 1u ? 1u : 0u;
        if (last != 0u) atomicExch(a.count + unit, 0u);
    }
    __syncthreads();
    if (last == 0u) return;
    const float *all = a.partial + (unsigned long long)unit * S * stride;
    /* One output value per lane: a wave's 64 lanes lie in one head (D is 64 or 128). Lane
     * c < st reads chunk c's max and mass and the wave shares them (uniform-index
     * shuffles), so a lane issues st + 2 loads, all in flight together, and the sums run
     * in chunk order as before. */
    for (unsigned int idx = threadIdx.x; idx < (unsigned int)(G * D); idx += 64u * W) {
        const unsigned int j = idx / D, e = idx % D;
        const float *col = all + j * (D + 2);
        const unsigned int cl = lane < st ? lane : 0u;
        const float m_l = aotx_attn_get(col + cl * stride);
        const float l_l = aotx_attn_get(col + cl * stride + 1u);
        float oc[ATTN_MAX_SPLITS];
#pragma unroll
        for (unsigned int cc = 0; cc < ATTN_MAX_SPLITS; ++cc)
            oc[cc] = cc < st ? aotx_attn_get(col + cc * stride + 2u + e) : 0.0f;
        float top = lane < st ? m_l : -INFINITY;
#pragma unroll
        for (int sh = 1; sh < 64; sh <<= 1) top = fmaxf(top, __shfl_xor(top, sh, 64));
        const float f_l = lane < st && m_l != -INFINITY ? aotx_exp2(m_l - top) : 0.0f;
        float msum = 0.0f, osum = 0.0f;
#pragma unroll
        for (unsigned int cc = 0; cc < ATTN_MAX_SPLITS; ++cc) {
            if (cc < st) {
                const float f = __shfl(f_l, (int)cc, 64);
                msum += __shfl(l_l, (int)cc, 64) * f;
                osum += oc[cc] * f;
            }
        }
        const float back = msum > 0.0f ? 1.0f / msum : 0.0f;
        const float v = osum * back;
        const float v1 = __shfl_down(v, 1, 64);
        if ((e & 1u) == 0u)
            co_store2h(a.out + aotx_attn_out_at(a, t, kh * G + j, e, D), aotx_f2h(v), aotx_f2h(v1));
    }
}

/* Prompt pieces two waves each: a workgroup of W = 8 waves takes the pieces led inside its
 * range of AOTX_RUN_RANGE tokens (a piece: up to QT = 16 / G consecutive queries of one
 * sequence, led by a token that starts its sequence's run in the batch or sits at a
 * multiple of QT, as in the decode body's prompt pieces), in rounds of 4 in rank order.
 * Wave k < 4 runs one ordered pass of online softmax (the reference's pass per query,
 * cuda/model/attention.cu:22-154) over the first half of the blocks its round's piece sees,
 * wave k + 4 over the second half; the second half's maxima, masses and accumulators pass
 * through LDS and the first wave adds them in block order and writes the outputs. When
 * a round's pieces are all of one sequence, the halves split the blocks of its longest
 * piece instead, and each half's four waves load every block once, into LDS (double
 * buffered, one barrier per block), where all four read their keys and values; otherwise
 * each wave loads its own blocks (the same blocks as its neighbours, from the caches). */
#define AOTX_RUN_RANGE 16u
template <int D, int G, int W>
static __device__ __forceinline__ void aotx_attend_runs(const aotx_attn_args &a, unsigned int bx)
{
    constexpr int QT = 16 / G;
    constexpr int KK = D / 32;
    constexpr int VP = D / 32;
    constexpr int NS = D / 16;
    constexpr int VS = D + 8;
    constexpr unsigned int RANGE = AOTX_RUN_RANGE;
    constexpr unsigned int WP = 4u;                 /* waves of a round, a piece each */
    static_assert(W == 2 * (int)WP, "two waves per piece: the halves of its blocks");
    static_assert(RANGE + QT <= 64u, "one lane per token word");
    __shared__ __attribute__((aligned(16))) unsigned short vl[W][16 * VS];
    /* the second half's column maxima, masses, page-fault flag and accumulators (by lane) */
    __shared__ float hm[WP][16], hl[WP][16];
    __shared__ int hmiss[WP];
    __shared__ float ho[WP][NS][4][64];
    __shared__ unsigned int rag[WP], rn[WP];

    const unsigned int lane = threadIdx.x & 63u;
    const unsigned int wave = threadIdx.x >> 6;
    const unsigned int wp = wave % WP, half = wave / WP;
    const unsigned int r = lane & 15u, g = lane >> 4;
    const unsigned int counted = aotx_attn_scalar(a.m_dev != nullptr ? a.m_dev : a.pos);
    unsigned int tokens = a.m_dev != nullptr ? counted : a.tokens;
    if (tokens > a.tokens) tokens = a.tokens;
    const unsigned int kh = bx % a.kv_heads;
    const unsigned int r0 = (bx / a.kv_heads) * RANGE;
    if (r0 >= tokens) return;
    /* one round trip: lane i holds the slot and position of token r0 - 1 + i (a token
     * before the batch or past it holds no slot: all ones) */
    const unsigned int ti = r0 + lane - 1u;
    unsigned int ag = 0xFFFFFFFFu, ps = 0u;
    if (lane < RANGE + (unsigned int)QT && (lane != 0u || r0 != 0u) && ti < tokens) {
        ag = a.agent[ti];
        ps = a.pos[ti];
    }
    const unsigned int ag_prev = (unsigned int)__shfl((int)ag, (int)((lane - 1u) & 63u), 64);
    const bool lead = lane >= 1u && lane <= RANGE && ti < tokens
                   && (ag != ag_prev || ps % (unsigned int)QT == 0u);
    const unsigned long long leaders = (unsigned long long)__ballot(lead) >> 1;   /* bit j: token r0 + j */
    /* the same in every wave (one ballot over the same words), so every wave runs the same
     * rounds and meets the same barriers */
    const unsigned int npieces = (unsigned int)__builtin_popcountll(leaders);

    const aotx_kv_table *kv = &a.state->kv;
    const float scale = 1.4426950408889634f / sqrtf((float)D);
    const unsigned int kbyte = ((kh * AOTX_KVL_BLOCK + r) * D + 8u * g) * 2u;
    const unsigned int vbyte = ((a.kv_heads + kh) * AOTX_KVL_BLOCK * D + lane * 8u) * 2u;
    unsigned short *vw = vl[wave];
    /* ds_read_tr16_b64: lane j of a 16-lane group gets halves j % 4 of the chunks that
     * lanes 4e + j / 4 address, e = 0..3; lane (r, g) = 16 g + 4 i + q addresses row 4g + i,
     * halves 4q..4q+3 of a 16-column slice, so that it gets column r of rows 4g..4g+3 */
    const unsigned int vtr = (4u * g + (lane & 15u) / 4u) * VS + 4u * (lane & 3u);
    constexpr int CPOL = 0;

    for (unsigned int round = 0; round * WP < npieces; ++round) {
        /* piece rank (in token order) round * WP + wp, its blocks split in two halves */
        const unsigned int rank = round * WP + wp;
        const bool have = rank < npieces;
        unsigned long long lb = leaders;
        for (unsigned int k = 0; k < rank && lb != 0ull; ++k) lb &= lb - 1ull;
        const unsigned int j = have ? (unsigned int)__builtin_ctzll(lb) : 0u;
        /* the piece led by token t = r0 + j (lane j + 1): the next tokens of its slot off a
         * multiple of QT, up to QT in all */
        const unsigned int lead_lane = j + 1u;
        const unsigned int t = r0 + j;
        const unsigned int agent = (unsigned int)__shfl((int)ag, (int)lead_lane, 64);
        const bool cont = lane > lead_lane && lane < lead_lane + (unsigned int)QT && ag == agent
                       && ps % (unsigned int)QT != 0u;
        const unsigned long long cm = (unsigned long long)__ballot(cont) >> (lead_lane + 1u);
        unsigned int nq = 1u + (unsigned int)__builtin_ctzll(~cm);
        if (nq > (unsigned int)QT) nq = QT;
        const unsigned int n = (unsigned int)__shfl((int)ps, (int)(lead_lane + nq - 1u), 64) + 1u;
        /* this lane's column: query r / G; a column with no query sees position 0 only */
        const unsigned int qpos = (unsigned int)__shfl((int)ps, (int)(lead_lane + r / (unsigned int)G), 64);
        const unsigned int plim = r / (unsigned int)G < nq ? qpos + 1u : 1u;
        const unsigned int p0 = 0u;
        const unsigned int nb = (n + 15u) / 16u;
        const unsigned int mid = (nb + 1u) / 2u;
        const unsigned int b0 = half == 0u ? 0u : mid;
        const unsigned int b1 = !have ? b0 : (half == 0u ? mid : nb);

        float mrun = -INFINITY, lrun = 0.0f;
        aotx_f4a o[NS];
#pragma unroll
        for (int cc = 0; cc < NS; ++cc) o[cc] = (aotx_f4a){0.0f, 0.0f, 0.0f, 0.0f};
        int missing = 0;
        /* the round's sequences and lengths: when its pieces are of one sequence (every
         * range of a prompt but those holding a sequence boundary), each half's four waves
         * stage every block once in LDS and all read it there */
        if (half == 0u && lane == 0u) {
            rag[wp] = have ? agent : 0xFFFFFFFFu;
            rn[wp] = have ? n : 0u;
        }
        __syncthreads();
        unsigned int sag = 0xFFFFFFFFu, nmax = 0u;
        bool one = true;
#pragma unroll
        for (unsigned int i = 0; i < WP; ++i) {
            const unsigned int ai = rag[i];
            if (ai == 0xFFFFFFFFu) continue;
            one = one && (sag == 0xFFFFFFFFu || sag == ai);
            sag = ai;
            nmax = rn[i] > nmax ? rn[i] : nmax;
        }
        if (one && sag != 0xFFFFFFFFu) {
            aotx_h8a qb[KK];
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                aotx_u4a w = {0u, 0u, 0u, 0u};
                const unsigned int qi = r / (unsigned int)G, hh = r % (unsigned int)G;
                if (have && qi < nq)
                    w = co_load4(a.q + ((unsigned long long)(t + qi) * a.heads + kh * G + hh) * D
                                     + 32 * kk + 8 * g);
                qb[kk] = __builtin_bit_cast(aotx_h8a, w);
            }
            /* blocks [0, smid) to the first half, [smid, nbm) to the second; both halves
             * run smid steps (the second's last one, when nbm is odd, adds nothing) */
            const unsigned int nbm = (nmax + 15u) / 16u;
            const unsigned int smid = (nbm + 1u) / 2u;
            const unsigned int sb0 = half == 0u ? 0u : smid;
            const unsigned int sb1 = half == 0u ? smid : nbm;
            const unsigned int hid = wp * 64u + lane;          /* loader lane of the half */
            constexpr unsigned int LP = (unsigned int)D / 64u;  /* 16-byte pieces per lane */
            const unsigned int kbase = kh * AOTX_KVL_BLOCK * D * 2u;
            const unsigned int vbase = (a.kv_heads + kh) * AOTX_KVL_BLOCK * D * 2u;
            unsigned short *const sl = &vl[half * 4u][0];       /* [buf][K, V][16][VS] */
            unsigned long long spages = 0ull;
            unsigned int swbase = 0xFFFFFFFFu;
            aotx_u4a ld[LP];
            bool sabs[2] = {false, false};
            bool labs = false;
            /* block SB's keys and values into the registers ld (a block past the
             * sequence's last reads the last one) */
#define SH_LOAD(SB)                                                                         \
            do {                                                                            \
                const unsigned int bb_ = (SB) < nbm ? (SB) : nbm - 1u;                      \
                if (swbase == 0xFFFFFFFFu || bb_ - swbase >= 64u) {                         \
                    swbase = bb_;                                                           \
                    const unsigned int bl_ = swbase + lane;                                 \
                    spages = bl_ < nbm ? (unsigned long long)aotx_kvl_block(a.shape, kv, sag, a.layer, bl_ * 16u) \
                                       : 0ull;                                              \
                }                                                                           \
                unsigned long long pb_ = __shfl(spages, (int)(bb_ - swbase), 64);           \
                pb_ = ((unsigned long long)(unsigned int)__builtin_amdgcn_readfirstlane((unsigned int)(pb_ >> 32)) << 32) \
                    | (unsigned long long)(unsigned int)__builtin_amdgcn_readfirstlane((unsigned int)pb_); \
                labs = pb_ == 0ull;                                                         \
                const __amdgpu_buffer_rsrc_t rs_ = __builtin_amdgcn_make_buffer_rsrc(       \
                    (void *)pb_, (short)0, labs ? 0 : (int)a.shape.block_bytes, 0x00020000); \
                _Pragma("unroll") for (unsigned int u = 0; u < LP; ++u) {                   \
                    const unsigned int pc = hid + u * 256u;                                 \
                    const unsigned int off = pc < 2u * D ? kbase + pc * 16u : vbase + (pc - 2u * D) * 16u; \
                    ld[u] = __builtin_amdgcn_raw_buffer_load_b128(rs_, (int)off, 0, CPOL);  \
                }                                                                           \
            } while (0)
            /* the registers into LDS buffer BUF (rows padded to VS halves) */
#define SH_STORE(BUF)                                                                       \
            do {                                                                            \
                _Pragma("unroll") for (unsigned int u = 0; u < LP; ++u) {                   \
                    const unsigned int pc = hid + u * 256u;                                 \
                    const unsigned int isv = pc < 2u * D ? 0u : 1u;                         \
                    const unsigned int e = pc - isv * 2u * D;                               \
                    *(aotx_u4a *)(sl + ((BUF) * 2u + isv) * (16u * VS) + (e / (D / 8u)) * VS \
                                  + (e % (D / 8u)) * 8u) = ld[u];                           \
                }                                                                           \
                sabs[BUF] = labs;                                                           \
            } while (0)
            SH_LOAD(sb0);
            SH_STORE(0u);
            __syncthreads();
            for (unsigned int i = 0; i < smid; ++i) {
                const unsigned int bcur = sb0 + i;
                SH_LOAD(bcur + 1u);
                const unsigned int cb = i & 1u;
                const bool live = bcur < sb1;
                if (have && live && sabs[cb] && bcur * 16u < n) missing = 1;
                MMA_COMPUTE_SH(sl + (cb * 2u) * (16u * VS), sl + (cb * 2u + 1u) * (16u * VS), bcur,
                               live, sabs[cb]);
                if ((i & 1u) == 0u) SH_STORE(1u); else SH_STORE(0u);
                __syncthreads();
            }
#undef SH_LOAD
#undef SH_STORE
        } else if (b0 < b1) {
            aotx_h8a qb[KK];
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                aotx_u4a w = {0u, 0u, 0u, 0u};
                const unsigned int qi = r / (unsigned int)G, hh = r % (unsigned int)G;
                if (qi < nq)
                    w = co_load4(a.q + ((unsigned long long)(t + qi) * a.heads + kh * G + hh) * D
                                     + 32 * kk + 8 * g);
                qb[kk] = __builtin_bit_cast(aotx_h8a, w);
            }
            aotx_u4a kr[2][KK], vr[2][VP];
            bool absent[2];
            unsigned long long pages = 0ull;
            unsigned int wbase = b0;
            unsigned int b = b0;
            MMA_WINDOW(b0);
            MMA_LOAD(0, b);
            for (;;) {
                MMA_LOAD(1, b + 1u);
                MMA_COMPUTE(0, b);
                b += 1u;
                if (b >= b1) break;
                MMA_LOAD(0, b + 1u);
                MMA_COMPUTE(1, b);
                b += 1u;
                if (b >= b1) break;
            }
        }
        /* a head's mass over its 4 lane groups; column c's max and mass sit in lane c */
        lrun += __shfl_xor(lrun, 16, 64);
        lrun += __shfl_xor(lrun, 32, 64);
        missing = __any(missing);
        if (missing && lane == 0u) atomicAdd(&a.state->faults, 1u);
        if (half == 1u) {
            if (lane < 16u) {
                hm[wp][lane] = mrun;
                hl[wp][lane] = lrun;
            }
            if (lane == 0u) hmiss[wp] = missing;
#pragma unroll
            for (int cc = 0; cc < NS; ++cc)
#pragma unroll
                for (int i = 0; i < 4; ++i) ho[wp][cc][i][lane] = o[cc][i];
        }
        __syncthreads();
        if (have && half == 0u) {
            /* the halves in block order: M = max(m0, m1), o = o0 2^(m0 - M) + o1 2^(m1 - M),
             * the masses likewise (a half with no position yet has m = -inf: factor 0) */
            const float m1 = hm[wp][r], l1 = hl[wp][r];
            const float top = fmaxf(mrun, m1);
            const float f0 = mrun == -INFINITY ? 0.0f : aotx_exp2(mrun - top);
            const float f1 = m1 == -INFINITY ? 0.0f : aotx_exp2(m1 - top);
            lrun = lrun * f0 + l1 * f1;
            missing = missing || hmiss[wp] != 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned int col = 4u * g + (unsigned int)i;
                const float c0 = __shfl(f0, (int)col, 64), c1 = __shfl(f1, (int)col, 64);
#pragma unroll
                for (int cc = 0; cc < NS; ++cc) o[cc][i] = o[cc][i] * c0 + ho[wp][cc][i][lane] * c1;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned int col = 4u * g + (unsigned int)i;
                const float l = __shfl(lrun, (int)col, 64);
                const float back = !missing && l > 0.0f ? 1.0f / l : 0.0f;
                const unsigned int qc = col / (unsigned int)G, hc = col % (unsigned int)G;
#pragma unroll
                for (int cc = 0; cc < NS; ++cc) {
                    const float v = o[cc][i] * back;
                    const float v1 = __shfl_down(v, 1, 64);
                    if (qc < nq && (r & 1u) == 0u)
                        co_store2h(a.out + aotx_attn_out_at(a, t + qc, kh * G + hc, 16u * cc + r, D),
                                   aotx_f2h(v), aotx_f2h(v1));
                }
            }
        }
        __syncthreads();        /* the second halves' slots are free for the next round */
    }
}

#undef MMA_WINDOW
#undef MMA_LOAD
#undef MMA_COMPUTE
#undef MMA_COMPUTE_SH

#endif
