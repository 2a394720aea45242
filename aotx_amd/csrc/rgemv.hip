/* Streaming Q8 product over repacked (Q8R) weights, for the decode step.
 *
 * Same product and operand values as gemv.hip (A = half(q * scale), B = fp16 activations,
 * fp32 accumulation in v_mfma_f32_16x16x32_f16; reference: cuda/model/gemv.cuh:33-195,
 * cuda/model/gemm.cuh:55-189), arranged so that the weight stream never touches LDS and no
 * wave waits on another inside the k loop:
 *   - a workgroup owns rt 16-row tiles and a k range; its 4 (or 8) waves take contiguous
 *     shares of the k range, each for all rt tiles, and stream their weights with two 16-byte
 *     loads per lane per tile per 128 k (the repacked layout puts a lane's 32 quants of one
 *     block next to each other), `pd` quads ahead of the MFMAs;
 *   - the batch rows of x for the workgroup's k range sit in LDS, staged once at the start
 *     (from fp16 x, or computed there from the residual stream: x = half(rsqrt(ss/h + eps)
 *     * resid * w), the reference's RMSNorm rounding of cuda/model/norm.cu:49-77, so the
 *     norm costs no kernel of its own);
 *   - the waves' accumulators are added in wave order through LDS at the end; with k split
 *     over workgroups the partial tiles go to memory and the last split of the group to
 *     finish (an arrival counter) adds them in split order and applies the epilogue, so
 *     there is no second launch. Results do not depend on timing.
 *   - epilogues as gemv.hip, plus the residual add that also leaves the sums of squares of
 *     every 16 rows for the next norm.
 */
#include "rgemv_dev.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- repack ------------------------------------------------------------------------- */

__global__ void aotx_q8r_repack_kernel(const unsigned char *src, unsigned int n, unsigned int k,
                                       unsigned char *dst)
{
    const unsigned long long qn = aotx_q8r_quads(k);
    const unsigned long long tiles = aotx_q8r_tiles(n);
    const unsigned long long items = tiles * qn * 64ull;
    const unsigned long long quant_bytes = items * 32ull;
    const unsigned int blocks = k / 32u;
    const unsigned long long row_bytes = (unsigned long long)blocks * 34ull;
    for (unsigned long long it = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x;
         it < items; it += (unsigned long long)gridDim.x * blockDim.x) {
        unsigned int lane = (unsigned int)(it % 64ull);
        unsigned long long tq = it / 64ull;
        unsigned long long q = tq % qn;
        unsigned long long t = tq / qn;
        unsigned int r = lane & 15u, g = lane >> 4;
        unsigned long long row = t * 16ull + r;
        unsigned long long blk = q * 4ull + g;
        /* the lane's first 16 quants, then (1 KB on) its second 16 */
        unsigned char *qd = dst + tq * 2048ull + lane * 16u;
        unsigned short *sd = (unsigned short *)(dst + quant_bytes) + it;
        if (row < n && blk < blocks) {
            const unsigned char *b = src + row * row_bytes + blk * 34ull;
            *sd = (unsigned short)(b[0] | (b[1] << 8));
            for (int j = 0; j < 32; ++j) qd[(j >> 4) * 1024 + (j & 15)] = b[2 + j] ^ 0x80u;
        } else {
            *sd = 0u;
            for (int j = 0; j < 32; ++j) qd[(j >> 4) * 1024 + (j & 15)] = 0x80u;   /* q = 0 */
        }
    }
}

void aotx_q8r_repack(const void *src, unsigned int n, unsigned int k, void *dst, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_q8r_repack_kernel, dim3(8192), dim3(256), 0, s,
                       (const unsigned char *)src, n, k, (unsigned char *)dst);
    AOTX_LAUNCH_CHECK();
}

/* ---- narrow batches ------------------------------------------------------------- */

template <int MT, int RT, int PD, int NW, bool NORM, bool DIRECT>
__global__ __launch_bounds__(64 * NW) void aotx_rgemv(aotx_rgemv_args a)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    aotx_args_touch(a);
    rg_narrow<MT, RT, PD, NW, NORM, DIRECT>(a, blockIdx.x, blockIdx.y, lds);
}

/* Wide batches (17..32 rows of fp16 x): a workgroup owns T 16-row tiles; its W = T * P
 * waves are T tile owners times P phases. x passes through LDS in chunks of KC quads,
 * double-buffered (the next chunk is loaded into registers while the current one feeds
 * the MFMAs); the P waves of a tile take its quads of each chunk in turn (phase p: chunk
 * quads p, p + P, ...), so every wave streams its weights one quad ahead of the MFMAs
 * and all waves read the same x chunk. At the end the P phase sums of a tile are added in
 * phase order through LDS and the workgroup applies the epilogue (with k split over
 * workgroups, the last split to finish adds the splits first). More phases put more waves
 * on the same tiles (more loads in flight per CU) at the price of more x staging. */
template <int T, int P, int KC, int PDQ>
__global__ __launch_bounds__(64 * T * P, 4) void aotx_rgemv_wide(aotx_rgemv_args a0)
{
    /* direct rows: grid.y is the 32-row pass (routed experts: the expert) */
    aotx_rgemv_args a = a0;
    if (a0.expert_stride == 0ull) a.m0 = a0.m0 + 32u * blockIdx.y;
    constexpr int MT = 32;
    constexpr int W = T * P;
    constexpr int NT = 64 * W;
    constexpr int NQ = KC / P;                               /* a wave's quads per chunk */
    constexpr int NS = NQ / PDQ;                             /* its load steps per chunk */
    static_assert(KC % P == 0 && NQ % PDQ == 0 && NS % 2 == 0, "whole load pairs per chunk");
    constexpr int XS = KC * 128 + 8;                         /* LDS x row stride (halves) */
    constexpr int PIECES = KC * 16;                          /* 16-byte pieces per row */
    constexpr int PPT = (MT * PIECES + NT - 1) / NT;          /* pieces per thread */
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    aotx_args_touch(a);
    const unsigned int tid = threadIdx.x;
    const unsigned int lane = tid & 63u;
    const unsigned int wave = tid >> 6;
    const unsigned int expert = blockIdx.y;
    const unsigned int *list = nullptr;
    unsigned int mrows = a.m;
    const unsigned int cap = a.m < (unsigned int)MT ? a.m : (unsigned int)MT;
    if (a.expert_stride != 0ull) {
        /* an expert no row chose streams nothing: its row count comes first */
        unsigned int total = rg_scalar(a.list_count + expert);
        mrows = total > a.m0 ? total - a.m0 : 0u;
        list = a.list + (unsigned long long)expert * a.list_cap + a.m0;
        if (mrows > cap) mrows = cap;
        if (mrows == 0u) return;
    }

    const unsigned int group = blockIdx.x / a.splits;
    const unsigned int split = blockIdx.x % a.splits;
    const unsigned int q0 = split * a.qps;
    const unsigned int q1 = q0 + a.qps < a.qn ? q0 + a.qps : a.qn;
    const unsigned int nch = (q1 - q0 + KC - 1u) / KC;
    unsigned short *xl = (unsigned short *)lds;               /* [2][MT][XS] */
    const unsigned int r = lane & 15u, g = lane >> 4;
    const unsigned int tj = wave / P, ph = wave % P;

    unsigned int dummy = 0u;
    const unsigned char *qb = rg_tile(a, group, tj, T, expert, dummy) + lane * 16u;
    const unsigned short *sb = rg_scales(a, group, tj, T, expert) + lane;
    rg_f4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    rg_u4 wa[2][PDQ][2];             /* two buffers of PDQ quads */
    unsigned int ws[2][PDQ];         /* one 32-bit register per scale: no packing waits */

/* the wave's n-th quad: chunk n / NQ, its phase's (n % NQ)-th quad of that chunk */
#define RGW_QUAD(N) (q0 + ((N) / NQ) * KC + ph + P * ((N) % NQ))
#define RGW_LOAD(BUF, N)                                                                 \
    do {                                                                                 \
        _Pragma("unroll") for (int qi = 0; qi < PDQ; ++qi) {                             \
            unsigned int qq = RGW_QUAD((N) + (unsigned int)qi);                          \
            if (qq >= q1) qq = q1 - 1u;         /* past the range: a cache hit, unused */ \
            const rg_u4 *src = (const rg_u4 *)(qb + (unsigned long long)qq * 2048ull);   \
            wa[BUF][qi][0] = __builtin_nontemporal_load(src);                            \
            wa[BUF][qi][1] = __builtin_nontemporal_load(src + 64);                       \
            ws[BUF][qi] = __builtin_nontemporal_load(&sb[(unsigned long long)qq * 64ull]); \
        }                                                                                \
    } while (0)
    /* branch-free: a quad past the range reads a valid x quad and has its scale zeroed */
#define RGW_COMPUTE(BUF, N, XB)                                                          \
    do {                                                                                 \
        _Pragma("unroll") for (int qi = 0; qi < PDQ; ++qi) {                             \
            const unsigned int qq = RGW_QUAD((N) + (unsigned int)qi);                    \
            const unsigned int qx = qq < q1 ? qq : q1 - 1u;                              \
            const unsigned short *xq = (XB) + ((qx - q0) % KC) * 128u + 32u * g;         \
            rg_h8 B[2][4];                                                               \
            _Pragma("unroll") for (int t = 0; t < 2; ++t)                                \
                _Pragma("unroll") for (int s = 0; s < 4; ++s)                            \
                    B[t][s] = *(const rg_h8 *)(xq + ((unsigned int)t * 16u + r) * XS + 8u * s); \
            const unsigned int sbits = qq < q1 ? ws[BUF][qi] : 0u;                       \
            rg_h2 s2 = __builtin_bit_cast(rg_h2, sbits | (sbits << 16));                 \
            const rg_u4 q0v = wa[BUF][qi][0], q1v = wa[BUF][qi][1];                      \
            unsigned int qd[8] = {q0v[0], q0v[1], q0v[2], q0v[3], q1v[0], q1v[1], q1v[2], q1v[3]}; \
            _Pragma("unroll") for (int s = 0; s < 4; ++s) {                              \
                unsigned int d0, d1, d2, d3;                                             \
                rg_dequant4(qd[2 * s], s2, d0, d1);                                      \
                rg_dequant4(qd[2 * s + 1], s2, d2, d3);                                  \
                rg_u4 av = {d0, d1, d2, d3};                                             \
                rg_h8 A = __builtin_bit_cast(rg_h8, av);                                 \
                acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[0][s], acc[0], 0, 0, 0); \
                acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[1][s], acc[1], 0, 0, 0); \
            }                                                                            \
        }                                                                                \
    } while (0)

    /* x chunk c: rows past mrows and k past a.k are zeros. A thread's pieces keep their
     * batch row from chunk to chunk, so the source rows are looked up once, here, before
     * any weight load (a lookup after them would wait for all of them). */
    /* Batch rows of x are loaded for the pass capacity (rows past the count are stale rows
     * of the x buffer: a batch column only feeds its own output column, which is never
     * written), so no load waits for the device row count. Every x load is unconditional,
     * from an address clamped into x, and k past a.k is zeroed where it is stored (the
     * weights there are zero, and zero times a stale infinity would not be): a load under
     * a condition would be waited for where its branch joins, before the weight stream. */
    rg_u4 xr[PPT];
    unsigned int xsrcv[PPT];
    if (list == nullptr && a.xrow == nullptr) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const unsigned int mm = (tid + (unsigned int)i * NT) / PIECES;
            xsrcv[i] = a.m0 + (mm < cap ? mm : 0u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const unsigned int mm = (tid + (unsigned int)i * NT) / PIECES;
            const unsigned int mc = mm < mrows ? mm : 0u;
            xsrcv[i] = list != nullptr ? list[mc] / a.xrow_div : a.xrow[a.m0 + mc];
        }
    }
#define RGW_XLOAD(C)                                                                     \
    do {                                                                                 \
        _Pragma("unroll") for (int i = 0; i < PPT; ++i) {                                \
            unsigned int idx = tid + (unsigned int)i * NT;                               \
            unsigned int p = idx % PIECES;                                               \
            unsigned int kk = (q0 + (C) * KC) * 128u + p * 8u;                           \
            if (!(kk < q1 * 128u && kk < a.k)) kk = 0u;                                  \
            xr[i] = *(const rg_u4 *)(a.x + (unsigned long long)xsrcv[i] * a.ldx + kk);   \
        }                                                                                \
    } while (0)
#define RGW_XSTORE(C)                                                                    \
    do {                                                                                 \
        unsigned short *xb = xl + ((C) & 1u) * (unsigned int)(MT * XS);                  \
        _Pragma("unroll") for (int i = 0; i < PPT; ++i) {                                \
            unsigned int idx = tid + (unsigned int)i * NT;                               \
            unsigned int mm = idx / PIECES, p = idx % PIECES;                            \
            unsigned int kk = (q0 + (C) * KC) * 128u + p * 8u;                           \
            const rg_u4 v = kk < q1 * 128u && kk < a.k ? xr[i] : (rg_u4){0u, 0u, 0u, 0u}; \
            if (idx < (unsigned int)(MT * PIECES))                                       \
                *(rg_u4 *)(xb + mm * XS + p * 8u) = v;                                   \
        }                                                                                \
    } while (0)

    /* x chunk 0 and the first two weight quads go out before the first wait; each buffer
     * is refilled right after its quad is computed, two quads ahead. x chunk c + 1 is
     * requested before chunk c's later weight loads, so storing it waits for nothing
     * issued after it. */
    rg_ss_pre<MT, NT> ssp;
    const bool ss_pre = list == nullptr && rg_row_ss_load<MT, NT>(a, cap, ssp);
    RGW_XLOAD(0u);
    /* the residual epilogue's residual values and next norm weights of few-tile products
     * (down), for direct rows: read with the first loads, unconditionally (from clamped
     * addresses; masked where used), instead of in dependent rounds after the split merge */
    constexpr bool RP = T <= 2;
    constexpr unsigned int RPT = (T * 16u * MT + NT - 1u) / NT;
    __shared__ float rres[RP ? T * 16 * rg_os<MT>() : 1];
    __shared__ float rgw[RP ? T * 16 : 1];
    const bool resid_pre = RP && list == nullptr && a.xrow == nullptr && a.epi == AOTX_EPI_RESID
                        && a.sumsq_out != nullptr;
    float rold[RPT];
    float gwv = 0.0f;
    if (resid_pre) {
#pragma unroll
        for (int it = 0; it < (int)RPT; ++it) {
            const unsigned int idx = tid + (unsigned int)it * NT;
            const unsigned int rr = idx & 15u, rest = idx >> 4;
            const unsigned int j = rest % T, mm = rest / T;
            const unsigned int v0 = rg_vrow(a, group, j, 0u, T);
            const bool ok = idx < T * 16u * MT && mm < cap && v0 + rr < a.n;
            rold[it] = co_loadf((const float *)a.y + (ok ? (unsigned long long)(a.m0 + mm) * a.ldy + v0 + rr
                                                         : (unsigned long long)a.m0 * a.ldy));
        }
        gwv = rg_gw_load(a, group, T, tid);
    }
    RGW_LOAD(0, 0u);
    RGW_LOAD(1, (unsigned int)PDQ);
    __builtin_amdgcn_sched_barrier(0);
    if (list == nullptr && a.m_dev != nullptr) {
        /* the device row count, after the weight stream went out */
        unsigned int total = rg_scalar(a.m_dev);
        mrows = total > a.m0 ? total - a.m0 : 0u;
    }
    if (mrows > cap) mrows = cap;
    __shared__ float rs[MT];
    if (ss_pre) rg_row_ss_sum<MT, NT>(a, mrows, rs, ssp);
    RGW_XSTORE(0u);
    if (resid_pre) {
#pragma unroll
        for (int it = 0; it < (int)RPT; ++it) {
            const unsigned int idx = tid + (unsigned int)it * NT;
            const unsigned int rr = idx & 15u, rest = idx >> 4;
            if (idx < T * 16u * MT) {
                const unsigned int j = rest % T, mm = rest / T;
                const bool ok = mm < cap && rg_vrow(a, group, j, 0u, T) + rr < a.n;
                rres[rg_o<MT>(j * 16u + rr, mm)] = ok ? rold[it] : 0.0f;
            }
        }
        if (tid < T * 16u) rgw[tid] = gwv;
    }
    rg_sync_lds();
    for (unsigned int c = 0; c < nch; ++c) {
        const unsigned short *xb = xl + (c & 1u) * (unsigned int)(MT * XS);
        if (c + 1u < nch) RGW_XLOAD(c + 1u);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            const unsigned int n = c * NQ + (unsigned int)(i * PDQ);
            RGW_COMPUTE(i & 1, n, xb);
            RGW_LOAD(i & 1, n + 2u * PDQ);
        }
        if (c + 1u < nch) RGW_XSTORE(c + 1u);
        rg_sync_lds();
    }
#undef RGW_QUAD
#undef RGW_LOAD
#undef RGW_COMPUTE
#undef RGW_XLOAD
#undef RGW_XSTORE

    /* the waves' tiles into LDS ([W][16][MT], the x buffers are free after the last
     * barrier), then each tile's P phases added in phase order into out [T*16][MT] */
    float *part = (float *)lds;
    const unsigned int gr = T * 16u;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            part[P == 1 ? rg_o<MT>(wave * 16u + 4u * g + (unsigned int)i, (unsigned int)t * 16u + r)
                        : (wave * 16u + 4u * g + (unsigned int)i) * MT + (unsigned int)t * 16u + r] = acc[t][i];
    __syncthreads();
    float *out = part + W * 16 * MT;
    if (P == 1) {
        out = part;
    } else {
        for (unsigned int idx = tid; idx < gr * MT; idx += NT) {
            const unsigned int j = idx / (16u * MT), rest = idx % (16u * MT);
            float sum = part[(j * P) * 16u * MT + rest];
#pragma unroll
            for (int p = 1; p < P; ++p) sum += part[((j * P) + (unsigned int)p) * 16u * MT + rest];
            out[rg_of<MT>(idx)] = sum;
        }
        __syncthreads();
    }
    if (a.splits > 1u) {
        __shared__ unsigned int last;
        if (!rg_split_merge<NT>(a, out, gr * rg_os<MT>(), expert, group, split, &last)) return;
    }
    if (ss_pre) {
        /* rs was written before the loop; the barriers since have published it */
        for (unsigned int idx = tid; idx < gr * MT; idx += NT) out[rg_of<MT>(idx)] *= rs[idx % MT];
        __syncthreads();
    } else if (a.row_ss != nullptr) {
        rg_row_scale<MT, NT>(a, out, gr, mrows, rs);
    }
    rg_epilogue<MT, NT>(a, out, group, T, mrows, list, resid_pre ? rres : nullptr, nullptr,
                        resid_pre ? rgw : nullptr);
}

/* Wide batches (5..32 rows) of a dense model with x in the fragment layout (aotx_xfrag_at):
 * a workgroup owns RT 16-row tiles of one k split, and its NW waves take consecutive runs
 * of that split's quads. Every wave loads, per quad, the tiles' weights (two 1 KB loads per
 * tile) and the quad's 32 x rows as eight B operands (eight 1 KB loads, shared by the RT
 * tiles), PD quads per buffer, two buffers ahead of the MFMAs: no LDS for x and no barrier
 * until the waves' sums are added in wave order. Split partials, the RMSNorm row scale and
 * the epilogues are those of the other products; SS loads the row scale's partial sums
 * with the first loads. */
template <int RT, int NW, int PD, bool SS>
__global__ __launch_bounds__(64 * NW) void aotx_rgemv_frag(aotx_rgemv_args a)
{
    constexpr int MT = 32;
    constexpr unsigned int NT = 64u * NW;
    __shared__ float part[NW * RT * 16 * MT];           /* the waves' sums, then out */
    __shared__ float rres[RT * 16 * rg_os<MT>()];       /* the epilogue's residual values */
    aotx_args_touch(a);
    const unsigned int tid = threadIdx.x;
    const unsigned int lane = tid & 63u;
    const unsigned int wave = tid >> 6;
    const unsigned int r = lane & 15u, g = lane >> 4;
    const unsigned int group = blockIdx.x / a.splits;
    const unsigned int split = blockIdx.x % a.splits;
    const unsigned int q0 = split * a.qps;
    const unsigned int q1 = q0 + a.qps < a.qn ? q0 + a.qps : a.qn;
    const unsigned int nq = q1 - q0;
    const unsigned int per = (nq + NW - 1u) / NW;
    const unsigned int wq0 = q0 + wave * per < q1 ? q0 + wave * per : q1;
    const unsigned int wq1 = wq0 + per < q1 ? wq0 + per : q1;
    const unsigned int qlast = wq0 < wq1 ? wq1 - 1u : q0;
    const unsigned int cap = a.m < (unsigned int)MT ? a.m : (unsigned int)MT;

    const unsigned char *qb[RT];
    const unsigned short *sb[RT];
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        unsigned int dummy = 0u;
        qb[j] = rg_tile(a, group, (unsigned int)j, RT, 0u, dummy) + lane * 16u;
        sb[j] = rg_scales(a, group, (unsigned int)j, RT, 0u) + lane;
    }
    const rg_u4 *xf = (const rg_u4 *)a.x + lane;

    /* ---- loads that do not depend on the weights go out first, unconditionally (from
     * clamped addresses; masked where used): the QKV epilogue's batch words and rope
     * factor, and the residual values the residual epilogue adds to ---- */
    constexpr unsigned int QU = RT * 8u * MT;
    const bool qkv_pre = a.epi == AOTX_EPI_QKV && QU <= NT;
    unsigned int q_pos = 0u, q_agent = 0u;
    float q_fac = 1.0f;
    if (qkv_pre && tid < QU) {
        const unsigned int mm = tid / (RT * 8u);
        const unsigned int mc = mm < cap ? mm : 0u;
        q_pos = a.qkv.pos[mc];
        q_agent = a.qkv.agent[mc];
        q_fac = rg_qkv_factor(a, group, RT, tid % (RT * 8u));
    }
    const bool resid_pre = a.epi == AOTX_EPI_RESID && a.sumsq_out != nullptr && a.splits == 1u;
    constexpr unsigned int RPT = (RT * 16u * MT + NT - 1u) / NT;
    float rold[RPT];
    if (resid_pre) {
#pragma unroll
        for (int it = 0; it < (int)RPT; ++it) {
            const unsigned int idx = tid + (unsigned int)it * NT;
            const unsigned int rr = idx & 15u, rest = idx >> 4;
            const unsigned int j = rest % RT, mm = rest / RT;
            const unsigned int v0 = rg_vrow(a, group, j, 0u, RT);
            const bool ok = idx < RT * 16u * MT && mm < cap && v0 + rr < a.n;
            rold[it] = co_loadf((const float *)a.y + (ok ? (unsigned long long)mm * a.ldy + v0 + rr : 0ull));
        }
    }
    __shared__ float rgw[RT * 16];
    const float gwv = resid_pre ? rg_gw_load(a, group, RT, tid) : 0.0f;
    rg_ss_pre<MT, NT> ssp;
    const bool ss_pre = SS && rg_row_ss_load<MT, NT>(a, cap, ssp);
    __builtin_amdgcn_sched_barrier(0);

    rg_f4 acc[RT][2];
#pragma unroll
    for (int j = 0; j < RT; ++j) acc[j][0] = acc[j][1] = (rg_f4){0.0f, 0.0f, 0.0f, 0.0f};
    rg_u4 wa[2][PD][RT][2];
    unsigned int ws[2][PD][RT];
    rg_u4 xb[2][PD][2][4];
    /* quads past the wave's range reload its last quad (a cache hit) and are not added */
#define RGF_LOAD(BUF, QS)                                                                 \
    do {                                                                                  \
        _Pragma("unroll") for (int qi = 0; qi < PD; ++qi) {                               \
            unsigned int qq = (QS) + (unsigned int)qi;                                    \
            if (qq > qlast) qq = qlast;                                                   \
            _Pragma("unroll") for (int j = 0; j < RT; ++j) {                              \
                const rg_u4 *src = (const rg_u4 *)(qb[j] + (unsigned long long)qq * 2048ull); \
                wa[BUF][qi][j][0] = __builtin_nontemporal_load(src);                      \
                wa[BUF][qi][j][1] = __builtin_nontemporal_load(src + 64);                 \
                ws[BUF][qi][j] = __builtin_nontemporal_load(&sb[j][(unsigned long long)qq * 64ull]); \
            }                                                                             \
            _Pragma("unroll") for (int t = 0; t < 2; ++t)                                 \
                _Pragma("unroll") for (int st = 0; st < 4; ++st)                          \
                    xb[BUF][qi][t][st] = xf[(((unsigned long long)qq * 2u + t) * 4u + st) * 64u]; \
        }                                                                                 \
    } while (0)
#define RGF_COMPUTE(BUF, QS)                                                              \
    do {                                                                                  \
        _Pragma("unroll") for (int qi = 0; qi < PD; ++qi) {                               \
            const unsigned int qq = (QS) + (unsigned int)qi;                              \
            _Pragma("unroll") for (int j = 0; j < RT; ++j) {                              \
                const unsigned int sbits = qq < wq1 ? ws[BUF][qi][j] : 0u;                \
                rg_h2 s2 = __builtin_bit_cast(rg_h2, sbits | (sbits << 16));              \
                const rg_u4 q0v = wa[BUF][qi][j][0], q1v = wa[BUF][qi][j][1];             \
                unsigned int qd[8] = {q0v[0], q0v[1], q0v[2], q0v[3],                     \
                                      q1v[0], q1v[1], q1v[2], q1v[3]};                    \
                _Pragma("unroll") for (int st = 0; st < 4; ++st) {                        \
                    unsigned int d0, d1, d2, d3;                                          \
                    rg_dequant4(qd[2 * st], s2, d0, d1);                                  \
                    rg_dequant4(qd[2 * st + 1], s2, d2, d3);                              \
                    rg_u4 av = {d0, d1, d2, d3};                                          \
                    rg_h8 A = __builtin_bit_cast(rg_h8, av);                              \
                    _Pragma("unroll") for (int t = 0; t < 2; ++t)                         \
                        acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(                \
                            A, __builtin_bit_cast(rg_h8, xb[BUF][qi][t][st]), acc[j][t], 0, 0, 0); \
                }                                                                         \
            }                                                                             \
        }                                                                                 \
    } while (0)

    RGF_LOAD(0, wq0);
    RGF_LOAD(1, wq0 + PD);
    __builtin_amdgcn_sched_barrier(0);
    unsigned int mrows = cap;
    if (a.m_dev != nullptr) {
        /* the device row count, after the weight stream went out */
        const unsigned int total = rg_scalar(a.m_dev);
        mrows = total < cap ? total : cap;
    }
    rg_qkv_pre qpre = {0ull, 0ull, 1.0f, 0.0f, 0u, 0u};
    if (qkv_pre && tid < QU)
        qpre = rg_qkv_prep(a, group, RT, tid % (RT * 8u), tid / (RT * 8u), q_pos, q_agent, q_fac,
                           tid / (RT * 8u) < mrows);
    __shared__ float rs[MT];
    if (ss_pre) rg_row_ss_sum<MT, NT>(a, mrows, rs, ssp);
    if (wq0 < wq1) {
        unsigned int q = wq0;
        for (;;) {
            RGF_COMPUTE(0, q);
            q += PD;
            if (q >= wq1) break;
            RGF_LOAD(0, q + PD);
            RGF_COMPUTE(1, q);
            q += PD;
            if (q >= wq1) break;
            RGF_LOAD(1, q + PD);
        }
    }
#undef RGF_LOAD
#undef RGF_COMPUTE

    /* ---- the waves' sums in wave order ---- */
    constexpr unsigned int GR = RT * 16u;
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                part[(wave * GR + (unsigned int)j * 16u + 4u * g + (unsigned int)i) * MT
                     + (unsigned int)t * 16u + r] = acc[j][t][i];
    if (resid_pre) {
#pragma unroll
        for (int it = 0; it < (int)RPT; ++it) {
            const unsigned int idx = tid + (unsigned int)it * NT;
            const unsigned int rr = idx & 15u, rest = idx >> 4;
            if (idx < RT * 16u * MT) {
                const unsigned int j = rest % RT, mm = rest / RT;
                const bool ok = mm < cap && rg_vrow(a, group, j, 0u, RT) + rr < a.n;
                rres[rg_o<MT>(j * 16u + rr, mm)] = ok ? rold[it] : 0.0f;
            }
        }
        if (tid < GR) rgw[tid] = gwv;
    }
    __syncthreads();
    float sums[(GR * MT + NT - 1u) / NT];
#pragma unroll
    for (unsigned int i = 0; i < (GR * MT + NT - 1u) / NT; ++i) {
        const unsigned int idx = tid + i * NT;
        float sum = 0.0f;
        if (idx < GR * MT) {
            sum = part[idx];
#pragma unroll
            for (int w = 1; w < NW; ++w) sum += part[(unsigned int)w * GR * MT + idx];
        }
        sums[i] = sum;
    }
    __syncthreads();
    float *out = part;
#pragma unroll
    for (unsigned int i = 0; i < (GR * MT + NT - 1u) / NT; ++i)
        if (tid + i * NT < GR * MT) out[rg_of<MT>(tid + i * NT)] = sums[i];
    __syncthreads();
    if (a.splits > 1u) {
        __shared__ unsigned int last;
        if (!rg_split_merge<NT>(a, out, GR * rg_os<MT>(), 0u, group, split, &last)) return;
    }
    if (ss_pre) {
        /* rs was written before the loop; the barriers since have published it */
        for (unsigned int idx = tid; idx < GR * MT; idx += NT) out[rg_of<MT>(idx)] *= rs[idx % MT];
        __syncthreads();
    } else if (a.row_ss != nullptr) {
        rg_row_scale<MT, NT>(a, out, GR, mrows, rs);
    }
    rg_epilogue<MT, NT>(a, out, group, RT, mrows, nullptr, resid_pre ? rres : nullptr,
                        qkv_pre ? &qpre : nullptr, resid_pre ? rgw : nullptr);
}

/* Many batch rows (prefill): a GEMM. A workgroup takes 256 weight rows (16 tiles; for
 * SwiGLU 8 gate/up pairs) by MB batch rows. Each of its 8 waves owns 2 tiles over all MB
 * rows (MB/16 column blocks of accumulators), so every weight is dequantised once per
 * workgroup, each A fragment feeds MB/16 MFMAs, and each B fragment read from LDS feeds 2.
 * Per 128-k quad: the next quad's x rows go to LDS through registers (requested before
 * this quad's MFMAs, stored after them), and the weights are requested two quads ahead
 * and dequantised in registers into the A operand, as in the streaming product. The
 * results pass through LDS to the same epilogues. */
#define RGM_MB 64
#define RGM_RT 16
/* The grid is one-dimensional, ordered so that the row blocks of a weight group run
 * together on one XCD (dispatch goes round the 8 XCDs by workgroup index): they read each
 * weight quad at about the same time, and the XCD's L2 serves all but the first read, so
 * the weights take plain loads. An LDS x buffer holds two quads: one barrier per pair.
 * WIDE_REGS: one workgroup per CU (2 waves per SIMD, up to 256 registers each), for grids
 * of at most one workgroup per CU; larger grids run two per CU at 128 registers, where
 * the second workgroup hides the first one's waits (gate/up at 512 rows: 163 against
 * 181 us), and the MFMA loop reads one x fragment at a time. */
template <int MB, bool WIDE_REGS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WIDE_REGS ? 2 : 4))) void aotx_rgemm(aotx_rgemv_args a0, unsigned int ny)
{
    aotx_args_touch(a0);
    constexpr int RT = RGM_RT;                    /* weight tiles per workgroup */
    constexpr int CB = MB / 16;                   /* column blocks per wave */
    constexpr int NT = 512;
    constexpr int XS = 256 + 8;                   /* LDS x row stride (halves): two quads */
    constexpr int PIECES = 16;                    /* 16-byte pieces of a row per quad */
    constexpr int PPT = MB * PIECES / NT;         /* pieces per thread */
    static_assert(MB * PIECES % NT == 0 && MB % 16 == 0, "whole pieces and blocks");
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const unsigned int tid = threadIdx.x;
    const unsigned int lane = tid & 63u;
    const unsigned int wave = tid >> 6;
    const unsigned int r = lane & 15u, g = lane >> 4;
    /* on an XCD the row block runs fastest, then the k split, then the weight group */
    const unsigned int seq = blockIdx.x >> 3;               /* index on its XCD */
    const unsigned int yb = seq % ny;
    const unsigned int rest = seq / ny;
    const unsigned int split = rest % a0.splits;
    const unsigned int group = (rest / a0.splits) * 8u + (blockIdx.x & 7u);
    if (group >= a0.groups) return;

    aotx_rgemv_args a = a0;
    a.m0 = a0.m0 + yb * (unsigned int)MB;
    unsigned int total = a0.m;
    if (a0.m_dev != nullptr) {
        const unsigned int live = rg_scalar(a0.m_dev);
        total = live < total ? live : total;
    }
    if (a.m0 >= total) return;
    const unsigned int mrows = total - a.m0 < (unsigned int)MB ? total - a.m0 : (unsigned int)MB;

    unsigned short *xl = (unsigned short *)lds;         /* [2][MB][XS] */
    const unsigned char *qb[2];
    const unsigned short *sb[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        unsigned int dummy = 0u;
        qb[t] = rg_tile(a, group, wave * 2u + (unsigned int)t, RT, 0u, dummy) + lane * 16u;
        sb[t] = rg_scales(a, group, wave * 2u + (unsigned int)t, RT, 0u) + lane;
    }
    rg_f4 acc[2][CB];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[t][c] = (rg_f4){0.0f, 0.0f, 0.0f, 0.0f};

    /* piece i of a thread is row tid / 16 + 32 i, place tid % 16 (rows past mrows read a
     * valid row and are stored as zeros) */
    constexpr unsigned int RSTEP = NT / PIECES;
    const unsigned int xrow0 = tid / PIECES, xpc = tid % PIECES;
    unsigned int xoff[PPT];                       /* element offsets from a.x */
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const unsigned int mm = xrow0 + (unsigned int)i * RSTEP;
        xoff[i] = (a.m0 + (mm < mrows ? mm : 0u)) * a.ldx + xpc * 8u;
    }

    rg_u4 wa[2][2][2];
    unsigned int ws[2][2];
    /* this split's quads [qb0, qn) */
    const unsigned int qb0 = split * a.qps;
    const unsigned int qn = qb0 + a.qps < a.qn ? qb0 + a.qps : a.qn;
    /* every call issues the same loads (a quad past k repeats the last: never computed) */
#define RGM_WLOAD(BUF, Q)                                                                \
    do {                                                                                 \
        const unsigned int qq_ = (Q) < qn ? (Q) : qn - 1u;                               \
        _Pragma("unroll") for (int t = 0; t < 2; ++t) {                                  \
            const rg_u4 *src = (const rg_u4 *)(qb[t] + (unsigned long long)qq_ * 2048ull); \
            wa[BUF][t][0] = src[0];                                                      \
            wa[BUF][t][1] = src[64];                                                     \
            ws[BUF][t] = __builtin_nontemporal_load(&sb[t][(unsigned long long)qq_ * 64ull]); \
        }                                                                                \
    } while (0)
    /* x pieces of quad Q (k is a whole number of quads: a quad past k repeats the last) */
    rg_u4 xr[2][PPT];                             /* register buffer XB = Q & 1 holds quad Q */
#define RGM_XLOAD(XB, Q)                                                                 \
    do {                                                                                 \
        const unsigned int qx_ = ((Q) < qn ? (Q) : qn - 1u) * 128u;                      \
        _Pragma("unroll") for (int i = 0; i < PPT; ++i)                                  \
            xr[XB][i] = *(const rg_u4 *)(a.x + xoff[i] + qx_);                           \
    } while (0)
/* the LDS place of quad Q: buffer and offset within a row */
#define RGM_XBUF(Q) ((((Q) - qb0) >> 1) & 1u)
#define RGM_XPOS(Q) ((((Q) - qb0) & 1u) * 128u)
#define RGM_XSTORE(XB, Q)                                                                \
    do {                                                                                 \
        unsigned short *xb_ = xl + RGM_XBUF(Q) * (unsigned int)(MB * XS) + RGM_XPOS(Q)   \
                            + xrow0 * XS + xpc * 8u;                                     \
        _Pragma("unroll") for (int i = 0; i < PPT; ++i)                                  \
            *(rg_u4 *)(xb_ + (unsigned int)i * RSTEP * XS) =                             \
                xrow0 + (unsigned int)i * RSTEP < mrows ? xr[XB][i] : (rg_u4){0u, 0u, 0u, 0u}; \
    } while (0)

    /* Quad q is computed from LDS x buffer q & 1 and weight buffer q & 1. Its step first
     * requests quad q + 2's x (into the registers quad q's x left) and, after the MFMAs,
     * quad q + 2's weights, then stores quad q + 1's x, requested a whole step earlier. */
    RGM_XLOAD(0, qb0);
    RGM_XLOAD(1, qb0 + 1u);
    RGM_WLOAD(0, qb0);
    RGM_WLOAD(1, qb0 + 1u);
    RGM_XSTORE(0, qb0);
    RGM_XSTORE(1, qb0 + 1u);
    rg_sync_lds();
    for (unsigned int q = qb0; q < qn; q += 2u) {
/* quad QQ's MFMAs from weight buffer BUF, then quad QQ + 2's weights into it */
#define RGM_COMPUTE(BUF, QQ)                                                             \
    do {                                                                                 \
        const unsigned int qc_ = (QQ);                                                   \
        const unsigned short *xb = xl + RGM_XBUF(qc_) * (unsigned int)(MB * XS) + RGM_XPOS(qc_); \
        const unsigned int sq_ = qc_ < qn ? 0xffffffffu : 0u;                            \
        rg_h8 A[2][4];                                                                   \
        _Pragma("unroll") for (int t = 0; t < 2; ++t) {                                  \
            const unsigned int sbits = ws[BUF][t] & sq_;                                 \
            rg_h2 s2 = __builtin_bit_cast(rg_h2, sbits | (sbits << 16));                 \
            const rg_u4 q0v = wa[BUF][t][0], q1v = wa[BUF][t][1];                        \
            unsigned int qd[8] = {q0v[0], q0v[1], q0v[2], q0v[3],                        \
                                  q1v[0], q1v[1], q1v[2], q1v[3]};                       \
            _Pragma("unroll") for (int s = 0; s < 4; ++s) {                              \
                unsigned int d0, d1, d2, d3;                                             \
                rg_dequant4(qd[2 * s], s2, d0, d1);                                      \
                rg_dequant4(qd[2 * s + 1], s2, d2, d3);                                  \
                rg_u4 av = {d0, d1, d2, d3};                                             \
                A[t][s] = __builtin_bit_cast(rg_h8, av);                                 \
            }                                                                            \
        }                                                                                \
        if constexpr (WIDE_REGS) {                                                       \
            /* k step outermost: the step's x fragments are read together and its 8 */  \
            /* MFMAs write 8 different accumulators, none waiting for the one before */  \
            _Pragma("unroll") for (int s = 0; s < 4; ++s) {                              \
                rg_h8 B[CB];                                                             \
                _Pragma("unroll") for (int c = 0; c < CB; ++c)                           \
                    B[c] = *(const rg_h8 *)(xb + ((unsigned int)c * 16u + r) * XS        \
                                            + 32u * g + 8u * (unsigned int)s);           \
                _Pragma("unroll") for (int c = 0; c < CB; ++c) {                         \
                    acc[0][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0][s], B[c], acc[0][c], 0, 0, 0); \
                    acc[1][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1][s], B[c], acc[1][c], 0, 0, 0); \
                }                                                                        \
            }                                                                            \
        } else {                                                                         \
            /* one x fragment at a time (fits 128 registers) */                          \
            _Pragma("unroll") for (int c = 0; c < CB; ++c)                               \
                _Pragma("unroll") for (int s = 0; s < 4; ++s) {                          \
                    const rg_h8 B = *(const rg_h8 *)(xb + ((unsigned int)c * 16u + r) * XS \
                                                     + 32u * g + 8u * (unsigned int)s);  \
                    acc[0][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0][s], B, acc[0][c], 0, 0, 0); \
                    acc[1][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1][s], B, acc[1][c], 0, 0, 0); \
                }                                                                        \
        }                                                                                \
        __builtin_amdgcn_sched_barrier(0);     /* the MFMAs before the new loads */      \
        RGM_WLOAD(BUF, qc_ + 2u);                                                        \
        __builtin_amdgcn_sched_barrier(0);                                               \
    } while (0)
        /* the next pair's x first, then both quads, then its store and one barrier */
        RGM_XLOAD(0, q + 2u);
        RGM_XLOAD(1, q + 3u);
        __builtin_amdgcn_sched_barrier(0);
        RGM_COMPUTE(0, q);
        RGM_COMPUTE(1, q + 1u);
        RGM_XSTORE(0, q + 2u);
        RGM_XSTORE(1, q + 3u);
        rg_sync_lds();
#undef RGM_COMPUTE
    }
#undef RGM_XBUF
#undef RGM_XPOS
#undef RGM_WLOAD
#undef RGM_XLOAD
#undef RGM_XSTORE

    /* the residual epilogue's loads or the row scale's partial sums go out first (their
     * round trip overlaps the split merge), then the tile results into LDS as
     * out[rg_o(tile * 16 + row, batch row)] (the x buffers are free after the last
     * barrier), the split merge and the epilogue */
    const bool gresid = a.epi == AOTX_EPI_RESID && a.sumsq_out != nullptr;
    /* one register block holds either (the residual products have no row scale) */
    rg_ss_pre<MB, NT> sspre;
    static_assert(sizeof(sspre.v) == rg_gres<MB, NT, RT>::ITER * sizeof(float), "one block");
    float *gres = &sspre.v[0][0];
    float gw = 0.0f;
    bool ss_early = false;
    if (gresid) rg_gres_load<MB, NT, RT>(a, group, mrows, gres, gw);
    else ss_early = rg_row_ss_load<MB, NT>(a, mrows, sspre);
    float *out = (float *)lds;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                out[rg_o<MB>((wave * 2u + (unsigned int)t) * 16u + 4u * g + (unsigned int)i,
                             (unsigned int)c * 16u + r)] = acc[t][c][i];
    __syncthreads();
    if (a.splits > 1u) {
        /* the last split of (row block, group) to finish adds the splits in order */
        __shared__ unsigned int last;
        if (!rg_split_merge<NT, RT * 4 * MB>(a, out, RT * 16u * MB, yb, group, split, &last)) return;
    }
    __shared__ float rs[MB];
    if (ss_early) {
        rg_row_ss_sum<MB, NT>(a, mrows, rs, sspre);
        __syncthreads();
        for (unsigned int idx = tid; idx < RT * 16u * MB; idx += NT)
            out[rg_of<MB>(idx)] *= rs[idx % MB];
        __syncthreads();
    } else if (a.row_ss != nullptr) {
        rg_row_scale<MB, NT>(a, out, RT * 16u, mrows, rs);
    }
    if (gresid) rg_gres_store<MB, NT, RT>(a, out, group, mrows, gres, gw);
    else rg_epilogue<MB, NT, RT>(a, out, group, RT, mrows, nullptr);
}

/* ---- host ---------------------------------------------------------------------------- */

static size_t aotx_rgemv_lds(const aotx_rgemv_args &a, unsigned int mt)
{
    size_t x = (size_t)a.m * (a.qps * 128u + 8u) * 2u;
    size_t red = (size_t)(a.nw + 1u) * a.rt * 16u * (mt + 1u) * 4u;   /* out rows padded (rg_os) */
    return x > red ? x : red;
}

/* narrow_max: the most batch rows that take the streaming (narrow) kernel. */
static int aotx_rgemv_plan_n(aotx_rgemv_args *a, const void *const *w, const unsigned int *rows,
                             unsigned int nseg, unsigned int k, int epi, unsigned int mt,
                             unsigned int narrow_max, bool routed = false)
{
    memset(a, 0, sizeof *a);
    if (k == 0u || k % 32u != 0u || nseg == 0u || nseg > 3u || mt == 0u || mt > AOTX_RGEMM_ROWS)
        return 1;
    a->m = mt;
    a->k = k;
    a->qn = (unsigned int)aotx_q8r_quads(k);
    a->nseg = nseg;
    a->epi = epi;
    unsigned int total = 0u;
    for (unsigned int s = 0; s < nseg; ++s) {
        if (rows[s] == 0u || w[s] == nullptr) return 1;
        a->w[s] = (const unsigned char *)w[s];
        total += rows[s];
        a->seg_end[s] = total;
        if (s + 1u < nseg && rows[s] % 16u != 0u) return 1;
    }
    unsigned int tiles;
    if (epi == AOTX_EPI_SWIGLU) {
        if (nseg != 2u || rows[0] != rows[1]) return 1;
        a->n = rows[0];
        tiles = 2u * (unsigned int)aotx_q8r_tiles(rows[0]);
    } else {
        a->n = total;
        tiles = (total + 15u) / 16u;
    }
    if (mt > 32u) {
        /* 256 weight rows (16 tiles; SWIGLU: 8 gate/up pairs) by 64 batch rows per workgroup */
        a->gemm = 1u;
        a->rt = 16u;
        a->nw = 8u;
        a->groups = epi == AOTX_EPI_SWIGLU ? ((unsigned int)aotx_q8r_tiles(rows[0]) + 7u) / 8u
                                           : (tiles + 15u) / 16u;
        /* k split while the launch stays within one workgroup per CU and a split keeps 8
         * quads: a workgroup's time is its k length, and a second workgroup on a CU shares
         * its VALU and matrix cores */
        const unsigned int ny = (mt + RGM_MB - 1u) / RGM_MB;
        unsigned int sp = 1u;
        while (a->groups * ny * sp * 2u <= 256u && a->qn / (sp * 2u) >= 8u)
            sp *= 2u;
        a->qps = (a->qn + sp - 1u) / sp;
        a->splits = (a->qn + a->qps - 1u) / a->qps;
        return 0;
    }
    /* 5 to 32 rows: the wide kernel. With 32 batch columns per MFMA it wastes matrix-core
     * work below 32 rows, but the matrix cores are not what bounds these products: at 8
     * rows it streams the config-2 shapes 1.0-1.5x faster than the streaming kernel, whose
     * per-workgroup x staging grows with the rows; at 2 rows the streaming kernel wins. */
    if (mt > narrow_max) {
        /* T tiles x P phases of 8 waves per workgroup (aotx_rgemv_wide): 8 x 1 for many
         * tiles (gate/up pair, head), 4 x 2 for a 14336-row matrix, 2 x 4 for few (QKV, O,
         * down), measured best at the 8B shapes. Products run unsplit (no partials,
         * no second launch) unless they have fewer than 192 workgroups and k of 32 quads or more (down, a 4096-row O):
         * those split k towards 256 workgroups while a split keeps a whole chunk, and the
         * last split of a group to finish adds the partials. */
        a->wide = 1u;
        a->rt = tiles >= 1536u ? 8u : (tiles >= 768u ? 4u : 2u);
        /* routed experts' single products (down): the launch has a workgroup row per
         * expert, so fewer, larger tile groups fill the chip and each reads the expert's x
         * half as often (Mixtral shape, 64 tokens: 73.7 -> 58.3 us per pass with 4 tiles,
         * 65.0 with 8); the gated unit and dense products keep the rule above */
        if (routed && epi != AOTX_EPI_SWIGLU && a->rt == 2u) a->rt = 4u;
        a->pd = 8u / a->rt;                            /* phases */
        const unsigned int kc = a->pd == 4u ? 8u : 4u;
        if (epi == AOTX_EPI_SWIGLU)
            a->groups = ((unsigned int)aotx_q8r_tiles(rows[0]) + a->rt / 2u - 1u) / (a->rt / 2u);
        else a->groups = (tiles + a->rt - 1u) / a->rt;
        /* routed products are not split: their launch has a workgroup row per expert, which
         * fills the chip with whole-k workgroups (Mixtral shape at 64 tokens: the down
         * products of 8 experts as 512 workgroups in one round instead of 2048 in four, the
         * step 16.75 -> 16.15 ms) */
        unsigned int s = 1u;
        if (!routed && a->groups < 192u && a->qn >= 32u)
            while (a->groups * s < 256u && a->qn / (s + 1u) >= kc) s += 1u;
        a->qps = (a->qn + s - 1u) / s;
        a->splits = (a->qn + a->qps - 1u) / a->qps;
        return 0;
    }
    /* rows per workgroup: one tile (measured best at every 8B shape), the gated unit two
     * gate/up pairs. */
    /* the gated unit takes two gate/up pairs per workgroup: its 448 workgroups are resident
     * at once (896 single pairs ran in two rounds) */
    const unsigned int rt = epi == AOTX_EPI_SWIGLU ? 4u : 1u;
    a->rt = rt;
    a->pd = rt == 1u ? 4u : 1u;
    if (epi == AOTX_EPI_SWIGLU) {
        unsigned int half_tiles = (unsigned int)aotx_q8r_tiles(rows[0]);
        a->groups = (half_tiles + rt / 2u - 1u) / (rt / 2u);
    } else {
        a->groups = (tiles + rt - 1u) / rt;
    }
    /* k split: the staged x rows of a workgroup's k range fit 96 KB of LDS; split further
     * while there are fewer than `target` workgroups and a split keeps >= `minq` quads */
    const unsigned int target = 256u, minq = 8u;
    unsigned int kmax = 98304u / (mt * 256u);
    if (kmax < 1u) kmax = 1u;
    unsigned int s = (a->qn + kmax - 1u) / kmax;
    while (a->groups * s < target && (a->qn + s) / (s + 1u) >= minq) s += 1u;
    a->qps = (a->qn + s - 1u) / s;
    a->splits = (a->qn + a->qps - 1u) / a->qps;
    /* 8 waves per workgroup while the launch has few workgroups (each wave then has half
     * the quads to dequantise after its data arrives), 4 otherwise */
    a->nw = a->groups * a->splits <= 256u ? 8u : 4u;
    return 0;
}

/* Up to AOTX_NARROW_ROWS batch rows take the streaming kernel. */
int aotx_rgemv_plan(aotx_rgemv_args *a, const void *const *w, const unsigned int *rows,
                    unsigned int nseg, unsigned int k, int epi, unsigned int mt)
{
    return aotx_rgemv_plan_n(a, w, rows, nseg, k, epi, mt, AOTX_NARROW_ROWS);
}

int aotx_rgemv_plan_routed(aotx_rgemv_args *a, const void *const *w, const unsigned int *rows,
                           unsigned int nseg, unsigned int k, int epi, unsigned int mt)
{
    return aotx_rgemv_plan_n(a, w, rows, nseg, k, epi, mt, AOTX_NARROW_ROWS, true);
}

/* Fragment-layout products: RT tiles x NW waves x PD quads per buffer, measured at the 8B
 * shapes with 32 rows: one tile per workgroup up to 256 tiles (O, down), two up to 512
 * (QKV), four beyond (gate/up pairs, the head); 8 waves up to 256 workgroups (O: 10.1
 * against 10.7 us with 4); two quads per buffer for long k. */
int aotx_rgemv_plan_frag(aotx_rgemv_args *a, const void *const *w, const unsigned int *rows,
                         unsigned int nseg, unsigned int k, int epi, unsigned int mt)
{
    if (k % 128u != 0u || mt == 0u || mt > AOTX_XFRAG_ROWS) return 1;
    if (aotx_rgemv_plan(a, w, rows, nseg, k, epi, mt) != 0) return 1;
    const unsigned int tiles = epi == AOTX_EPI_SWIGLU ? 2u * (unsigned int)aotx_q8r_tiles(a->n)
                                                      : (a->n + 15u) / 16u;
    unsigned int rt = epi == AOTX_EPI_SWIGLU ? 4u : (tiles <= 256u ? 1u : (tiles <= 512u ? 2u : 4u));
    if (epi == AOTX_EPI_SWIGLU && rt == 1u) rt = 2u;
    a->wide = 0u;
    a->gemm = 0u;
    a->frag = 1u;
    a->rt = rt;
    a->groups = epi == AOTX_EPI_SWIGLU ? ((unsigned int)aotx_q8r_tiles(a->n) + rt / 2u - 1u) / (rt / 2u)
                                       : (tiles + rt - 1u) / rt;
    unsigned int s = 1u;
    while (a->groups * s < 192u && a->qn / (s + 1u) >= 8u) s += 1u;
    a->qps = (a->qn + s - 1u) / s;
    a->splits = (a->qn + a->qps - 1u) / a->qps;
    a->nw = a->groups * a->splits <= 256u ? 8u : 4u;
    a->pd = a->qps >= 64u ? 2u : 1u;
    if (rt > 1u) a->pd = 1u;
    return 0;
}

/* grid.y of a product: its experts, or the passes of a wide product of direct rows */
static unsigned int aotx_rgemv_rows_y(const aotx_rgemv_args &a)
{
    if (a.expert_stride != 0ull) return a.experts;
    return a.wide && a.passes > 1u ? a.passes : 1u;
}

size_t aotx_rgemv_partial_bytes(const aotx_rgemv_args &a)
{
    if (a.splits <= 1u) return 0u;
    if (a.gemm) return (size_t)aotx_rgemv_count_words(a) * a.splits * RGM_RT * 16u * RGM_MB * sizeof(float);
    size_t e = aotx_rgemv_rows_y(a);
    return e * a.groups * a.splits * a.rt * 16u * 33u * sizeof(float);   /* rows of 33 (rg_os) */
}

unsigned int aotx_rgemv_count_words(const aotx_rgemv_args &a)
{
    if (a.gemm) return a.groups * ((a.m + RGM_MB - 1u) / RGM_MB);
    return aotx_rgemv_rows_y(a) * a.groups;
}

template <int MT, int RT, int PD>
static void aotx_rgemv_go(const aotx_rgemv_args &a, hipStream_t s)
{
    unsigned int ey = a.expert_stride != 0ull ? a.experts : 1u;
    size_t lds = aotx_rgemv_lds(a, MT);
    const dim3 grid(a.groups * a.splits, ey);
    const bool norm = a.xmode == AOTX_X_NORM;
    const bool direct = a.expert_stride == 0ull && a.list == nullptr && a.xrow == nullptr;
#define RGN_GO(NW, NORM)                                                                   \
    do {                                                                                   \
        if (direct) hipLaunchKernelGGL((aotx_rgemv<MT, RT, PD, NW, NORM, true>), grid, dim3(64 * NW), lds, s, a); \
        else hipLaunchKernelGGL((aotx_rgemv<MT, RT, PD, NW, NORM, false>), grid, dim3(64 * NW), lds, s, a); \
    } while (0)
    if (a.nw == 8u) {
        if (norm) RGN_GO(8, true); else RGN_GO(8, false);
    } else {
        if (norm) RGN_GO(4, true); else RGN_GO(4, false);
    }
#undef RGN_GO
    AOTX_LAUNCH_CHECK();
}

int aotx_rgemv_launch(const aotx_rgemv_args &a0, hipStream_t s)
{
    aotx_rgemv_args a = a0;
    if (a.splits > 1u && a.partial == nullptr) {
        a.partial = (float *)aotx_scratch(AOTX_SCRATCH_GEMV_PARTIAL, aotx_rgemv_partial_bytes(a));
    }
    if (a.splits > 1u && a.count == nullptr) {
        a.count = (unsigned int *)aotx_scratch(AOTX_SCRATCH_GEMV_COUNT,
                                               (size_t)aotx_rgemv_count_words(a) * sizeof(unsigned int));
    }
    if (a.gemm) {
        if (a.xmode != AOTX_X_F16 || a.expert_stride != 0ull || a.list != nullptr
            || a.xrow != nullptr || (a.splits > 1u && (a.partial == nullptr || a.count == nullptr))) {
            fprintf(stderr, "aotx: the GEMM takes fp16 x of direct rows only\n");
            return 1;
        }
        const unsigned int ny = (a.m + RGM_MB - 1u) / RGM_MB;
        const dim3 g1(((a.groups + 7u) / 8u) * 8u * ny * a.splits);
        const size_t x2 = 2u * RGM_MB * (256u + 8u) * 2u, res = RGM_RT * 16u * RGM_MB * 4u;
        if (g1.x <= 256u)
            hipLaunchKernelGGL((aotx_rgemm<RGM_MB, true>), g1, dim3(512), x2 > res ? x2 : res, s, a, ny);
        else
            hipLaunchKernelGGL((aotx_rgemm<RGM_MB, false>), g1, dim3(512), x2 > res ? x2 : res, s, a, ny);
        AOTX_LAUNCH_CHECK();
        return 0;
    }
    if (a.frag) {
        if (a.xmode != AOTX_X_FRAG || a.expert_stride != 0ull || a.list != nullptr
            || a.xrow != nullptr || a.m0 != 0u || a.m > AOTX_XFRAG_ROWS) {
            fprintf(stderr, "aotx: the fragment product takes fragment-layout x of one pass\n");
            return 1;
        }
        const dim3 grid(a.groups * a.splits);
        const bool ss = a.row_ss != nullptr && a.k <= 4096u;
#define RGF_GO(RT, NW, PD)                                                                 \
        do {                                                                               \
            if (ss) hipLaunchKernelGGL((aotx_rgemv_frag<RT, NW, PD, true>), grid, dim3(64 * NW), 0, s, a); \
            else hipLaunchKernelGGL((aotx_rgemv_frag<RT, NW, PD, false>), grid, dim3(64 * NW), 0, s, a); \
        } while (0)
        if (a.rt == 1u) {
            if (a.nw == 8u) { if (a.pd == 2u) RGF_GO(1, 8, 2); else RGF_GO(1, 8, 1); }
            else { if (a.pd == 2u) RGF_GO(1, 4, 2); else RGF_GO(1, 4, 1); }
        } else if (a.rt == 2u) {          /* one quad per buffer (two would spill) */
            if (a.nw == 8u) RGF_GO(2, 8, 1); else RGF_GO(2, 4, 1);
        } else {
            if (a.nw == 8u) RGF_GO(4, 8, 1); else RGF_GO(4, 4, 1);
        }
#undef RGF_GO
        AOTX_LAUNCH_CHECK();
        return 0;
    }
    if (a.xmode == AOTX_X_FRAG) {
        fprintf(stderr, "aotx: fragment-layout x needs the fragment product's plan\n");
        return 1;
    }
    if (a.row_ss != nullptr && (!a.wide || a.list != nullptr || a.xrow != nullptr)) {
        fprintf(stderr, "aotx: the row-scaled product takes wide batches of direct rows only\n");
        return 1;
    }
    if (a.wide) {
        const unsigned int ey = aotx_rgemv_rows_y(a);
        const dim3 grid(a.groups * a.splits, ey);
        if (a.xmode != AOTX_X_F16) {
            fprintf(stderr, "aotx: the wide-batch product takes fp16 x only\n");
            return 1;
        }
        if (a.rt == 2u) {
            const size_t xb = 2u * 32u * (8u * 128u + 8u) * 2u;
            hipLaunchKernelGGL((aotx_rgemv_wide<2, 4, 8, 1>), grid, dim3(512), xb, s, a);
        } else if (a.rt == 4u) {
            const size_t xb = 2u * 32u * (4u * 128u + 8u) * 2u;
            hipLaunchKernelGGL((aotx_rgemv_wide<4, 2, 4, 1>), grid, dim3(512), xb, s, a);
        } else {
            const size_t xb = 2u * 32u * (4u * 128u + 8u) * 2u;
            hipLaunchKernelGGL((aotx_rgemv_wide<8, 1, 4, 2>), grid, dim3(512), xb, s, a);
        }
        AOTX_LAUNCH_CHECK();
        return 0;
    }
    if (a.rt == 1u) {
        if (a.pd >= 8u) aotx_rgemv_go<16, 1, 8>(a, s);
        else aotx_rgemv_go<16, 1, 4>(a, s);
    } else if (a.rt == 2u) {
        if (a.pd >= 4u) aotx_rgemv_go<16, 2, 4>(a, s);
        else aotx_rgemv_go<16, 2, 2>(a, s);
    } else {
        if (a.pd >= 2u) aotx_rgemv_go<16, 4, 2>(a, s);
        else aotx_rgemv_go<16, 4, 1>(a, s);
    }
    return 0;
}

/* ---- kernel-level C ABI ---------------------------------------------------------------- */

extern "C" unsigned long long aotx_q8r_size(unsigned int n, unsigned int k)
{
    if (n == 0u || k == 0u || k % 32u != 0u) return 0ull;
    return aotx_q8r_bytes(n, k);
}

extern "C" int aotx_q8_repack(const void *w, unsigned int n, unsigned int k, void *dst,
                              void *stream)
{
    if (w == nullptr || dst == nullptr || n == 0u || k == 0u || k % 32u != 0u) return 1;
    aotx_q8r_repack(w, n, k, dst, aotx_stream(stream));
    return 0;
}

static int aotx_q8r_gemv_any(const void *wr, unsigned int n, unsigned int k, const void *x,
                             unsigned int m, void *y, int epi, void *stream)
{
    if (wr == nullptr || x == nullptr || y == nullptr || n == 0u || m == 0u) return 1;
    if (k == 0u || k % 32u != 0u || k % 8u != 0u) return 1;
    const void *ws[1] = {wr};
    unsigned int rows[1] = {n};
    for (unsigned int m0 = 0, mt = 0; m0 < m; m0 += mt) {
        /* more than 32 rows: GEMM passes of up to AOTX_RGEMM_ROWS */
        mt = m - m0 > 32u ? (m - m0 < AOTX_RGEMM_ROWS ? m - m0 : AOTX_RGEMM_ROWS) : m - m0;
        aotx_rgemv_args a;
        /* up to 8 rows of a product of at most 256 tiles and k <= 4096 (4096 square) stream
         * faster through the narrow kernel: 9.0 against 9.8 us at 8 rows, where the wide
         * kernel splits k to fill the chip; larger products keep the wide kernel from 5 rows
         * (measured on the four 8B shapes) */
        const unsigned int narrow_max = (n + 15u) / 16u <= 256u && k <= 4096u ? 8u : AOTX_NARROW_ROWS;
        if (aotx_rgemv_plan_n(&a, ws, rows, 1u, k, epi, mt, narrow_max) != 0) return 1;
        a.xmode = AOTX_X_F16;
        a.x = (const unsigned short *)x;
        a.ldx = k;
        a.m0 = m0;
        a.y = y;
        a.ldy = n;
        if (aotx_rgemv_launch(a, aotx_stream(stream)) != 0) return 1;
    }
    return 0;
}

extern "C" int aotx_q8r_gemv(const void *wr, unsigned int n, unsigned int k, const void *x,
                             unsigned int m, float *y, void *stream)
{
    return aotx_q8r_gemv_any(wr, n, k, x, m, y, AOTX_EPI_F32, stream);
}

extern "C" int aotx_q8r_gemv_f16(const void *wr, unsigned int n, unsigned int k, const void *x,
                                 unsigned int m, void *y, void *stream)
{
    return aotx_q8r_gemv_any(wr, n, k, x, m, y, AOTX_EPI_F16, stream);
}
