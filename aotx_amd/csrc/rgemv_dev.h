/* Device code of the streaming Q8 product (rgemv.hip): operand helpers, epilogues and
 * the narrow-batch body.
 */
#ifndef AOTX_RGEMV_DEV_H
#define AOTX_RGEMV_DEV_H

#include "coherent.h"
#include "rgemv.h"

typedef _Float16 rg_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 rg_h2 __attribute__((ext_vector_type(2)));
typedef float rg_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int rg_u4 __attribute__((ext_vector_type(4)));


/* A kernel-constant word read through the scalar cache (counted by lgkmcnt, so waiting for
 * it does not wait for the vector loads issued before it). Only for memory no kernel of
 * the same launch writes. */
static __device__ __forceinline__ unsigned int rg_scalar(const unsigned int *p)
{
    return *(const __attribute__((address_space(4))) unsigned int *)p;
}

/* Workgroup barrier that waits for this wave's LDS operations only: global loads already
 * in flight (the weight stream) stay in flight across it. */
static __device__ __forceinline__ void rg_sync_lds()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

/* The sum over the 16 lanes of a DPP row (every lane gets it): a butterfly over lane
 * distances 1, 2, 4 and 8 with DPP moves inside the row (quad permutations, then the
 * half-row and row mirrors, which pair the same quads and halves), no LDS round trip. Each
 * step adds the same two values a cross-lane shuffle by XOR would, so the sum is the same
 * as long as the summed value is itself rounded (see rg_sq). */
static __device__ __forceinline__ float rg_sum16(float v)
{
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    return v;
}

/* v * v rounded to fp32 before any sum uses it: never fused into the first add of
 * rg_sum16, whose partner lane adds the rounded square */
static __device__ __forceinline__ float rg_sq(float v)
{
#pragma clang fp contract(off)
    return v * v;
}

/* ---- product ------------------------------------------------------------------------ */

/* Four Q8R quants (stored as q + 128, one byte each) to half(q * scale): the byte under
 * exponent bits 0x64 is the half 1024 + byte = 1152 + q, exact; minus 1152 is q, exact; the
 * product with the scale rounds once. */
static __device__ __forceinline__ void rg_dequant4(unsigned int u, rg_h2 s2, unsigned int &lo,
                                                   unsigned int &hi)
{
    unsigned int a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    unsigned int b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const rg_h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(unsigned int, (__builtin_bit_cast(rg_h2, a) - bias) * s2);
    hi = __builtin_bit_cast(unsigned int, (__builtin_bit_cast(rg_h2, b) - bias) * s2);
}

/* The segment holding output row v, and the first row of that segment. Written as sums
 * of one-sided selects, never a select between two fields: the compiler turns the latter
 * into one load from a computed offset, which can keep a copy of the arguments in
 * scratch memory instead of registers. */
static __device__ __forceinline__ unsigned int rg_seg(const aotx_rgemv_args &a, unsigned int v,
                                                      unsigned int &begin)
{
    const bool past0 = a.nseg > 1u && v >= a.seg_end[0];
    const bool past1 = a.nseg > 2u && v >= a.seg_end[1];     /* implies past0 */
    begin = (past0 ? a.seg_end[0] : 0u) + (past1 ? a.seg_end[1] - a.seg_end[0] : 0u);
    return (past0 ? 1u : 0u) + (past1 ? 1u : 0u);
}
static __device__ __forceinline__ unsigned int rg_seg_end(const aotx_rgemv_args &a, unsigned int seg)
{
    return a.seg_end[0] + (seg >= 1u ? a.seg_end[1] - a.seg_end[0] : 0u)
         + (seg >= 2u ? a.seg_end[2] - a.seg_end[1] : 0u);
}
static __device__ __forceinline__ const unsigned char *rg_seg_w(const aotx_rgemv_args &a, unsigned int seg)
{
    const unsigned long long w0 = (unsigned long long)a.w[0], w1 = (unsigned long long)a.w[1],
                             w2 = (unsigned long long)a.w[2];
    const unsigned long long p = w0 + (seg >= 1u ? w1 - w0 : 0ull) + (seg >= 2u ? w2 - w1 : 0ull);
    /* weights are global memory: global (not flat) loads */
    return (const unsigned char *)(const __attribute__((address_space(1))) unsigned char *)p;
}

/* Weight tile j of a workgroup: Q8R base of its 16 rows, and whether it exists. */
static __device__ __forceinline__ const unsigned char *rg_tile(const aotx_rgemv_args &a,
                                                               unsigned int group, unsigned int j,
                                                               unsigned int rt, unsigned int expert,
                                                               unsigned int &quant_off_unused)
{
    (void)quant_off_unused;
    unsigned int seg, tile;  /* tile index inside its segment's tensor */
    if (a.epi == AOTX_EPI_SWIGLU) {
        unsigned int half = rt / 2u;
        seg = j < half ? 0u : 1u;
        tile = group * half + (j < half ? j : j - half);
    } else {
        unsigned int v0 = (group * rt + j) * 16u;
        unsigned int begin;
        seg = rg_seg(a, v0, begin);
        tile = (v0 - begin) / 16u;
        unsigned int seg_tiles = (rg_seg_end(a, seg) - begin + 15u) / 16u;
        if (tile >= seg_tiles) tile = seg_tiles - 1u;   /* past the last row: discarded */
    }
    if (a.epi == AOTX_EPI_SWIGLU) {
        unsigned int seg_tiles = (a.n + 15u) / 16u;
        if (tile >= seg_tiles) tile = seg_tiles - 1u;
    }
    return rg_seg_w(a, seg) + (unsigned long long)expert * a.expert_stride
         + (unsigned long long)tile * a.qn * 2048ull;
}

/* Scale plane of the same tile: the quant plane of the whole tensor comes first. */
static __device__ __forceinline__ const unsigned short *rg_scales(const aotx_rgemv_args &a,
                                                                  unsigned int group, unsigned int j,
                                                                  unsigned int rt, unsigned int expert)
{
    unsigned int seg, tile, seg_rows;
    if (a.epi == AOTX_EPI_SWIGLU) {
        unsigned int half = rt / 2u;
        seg = j < half ? 0u : 1u;
        tile = group * half + (j < half ? j : j - half);
        seg_rows = a.n;
    } else {
        unsigned int v0 = (group * rt + j) * 16u;
        unsigned int begin;
        seg = rg_seg(a, v0, begin);
        tile = (v0 - begin) / 16u;
        seg_rows = rg_seg_end(a, seg) - begin;
    }
    unsigned long long tiles = (seg_rows + 15u) / 16u;
    if (tile >= tiles) tile = (unsigned int)tiles - 1u;
    const unsigned char *base = rg_seg_w(a, seg) + (unsigned long long)expert * a.expert_stride;
    return (const unsigned short *)(base + tiles * a.qn * 2048ull)
         + (unsigned long long)tile * a.qn * 64ull;
}

/* The virtual output row of row rr of tile j (SWIGLU: the gate/up row index). */
static __device__ __forceinline__ unsigned int rg_vrow(const aotx_rgemv_args &a, unsigned int group,
                                                       unsigned int j, unsigned int rr, unsigned int rt)
{
    if (a.epi == AOTX_EPI_SWIGLU) {
        unsigned int half = rt / 2u;
        return (group * half + (j < half ? j : j - half)) * 16u + rr;
    }
    return (group * rt + j) * 16u + rr;
}

/* ---- QKV epilogue (rope of queries and keys, keys and values into the paged cache) ---- */

/* One output pair (rows 2pr, 2pr+1 of a tile) of one batch row, resolved before the
 * product's sums exist: the destination (the query rows, or the cache page and the byte
 * offset in it; the page's load stays in flight until the store uses it) and the rope
 * rotation. mode 0: nothing to write; 1 query, 2 key, 3 value. */
struct rg_qkv_pre {
    unsigned long long base;        /* query rows, or the page (0: absent) */
    unsigned long long off;         /* bytes from base */
    float cs, sn;
    unsigned int mode;
    unsigned int count_fault;       /* a key's dimension 0 counts an absent page */
};

/* The rope frequency factor of the pair (1 without factors): a load that does not depend on
 * the batch, so it can go out with the first loads of the kernel. */
static __device__ __forceinline__ float rg_qkv_factor(const aotx_rgemv_args &a, unsigned int group,
                                                      unsigned int rt, unsigned int pr)
{
    const aotx_qkv_epi &e = a.qkv;
    if (e.factor == nullptr) return 1.0f;
    const unsigned int row = 2u * pr;
    const unsigned int v = rg_vrow(a, group, row / 16u, row % 16u, rt);
    unsigned int begin;
    rg_seg(a, v, begin);
    /* unconditional (a value row, or a row past n, reads a factor it does not use) */
    const unsigned int dim = (v - begin) % e.head_dim;
    return e.factor[dim >> 1];
}

static __device__ __forceinline__ rg_qkv_pre rg_qkv_prep(const aotx_rgemv_args &a, unsigned int group,
                                                         unsigned int rt, unsigned int pr,
                                                         unsigned int mm, unsigned int position,
                                                         unsigned int agent, float fac, bool live)
{
    rg_qkv_pre p = {0ull, 0ull, 1.0f, 0.0f, 0u, 0u};
    const aotx_qkv_epi &e = a.qkv;
    const unsigned int row = 2u * pr;
    const unsigned int v = rg_vrow(a, group, row / 16u, row % 16u, rt);
    if (!live || v >= a.n) return p;
    unsigned int begin;
    const unsigned int sg = rg_seg(a, v, begin);
    const unsigned int d = e.head_dim;
    const unsigned int local = v - begin;
    const unsigned int head = local / d;
    const unsigned int dim = local - head * d;
    if (sg <= 1u) {
        const float step = powf(e.theta, -2.0f / (float)d);
        float angle = (float)position * powf(step, (float)(dim >> 1));
        if (e.factor != nullptr) angle = angle / fac;
        sincosf(angle, &p.sn, &p.cs);
    }
    if (sg == 0u) {
        p.mode = 1u;
        p.base = (unsigned long long)e.qh;
        p.off = 2ull * ((unsigned long long)(a.m0 + mm) * e.heads * d + local);
        return p;
    }
    /* the block of aotx_kvl_block, with the page word kept apart from the offset */
    p.mode = sg == 1u ? 2u : 3u;
    p.count_fault = sg == 1u && dim == 0u ? 1u : 0u;
    const aotx_kvl_shape &s = e.shape;
    if (s.blocks_page == 0u || agent >= AOTX_SLOTS) return p;
    const unsigned int block = (position / AOTX_KVL_BLOCK) * s.layers + e.layer;
    const unsigned int index = block / s.blocks_page;
    if (index >= AOTX_KV_PAGES_EACH) return p;
    p.base = e.state->kv.page[agent][index];
    const unsigned int krow = (sg == 1u ? head : e.kv_heads + head) * AOTX_KVL_BLOCK
                            + position % AOTX_KVL_BLOCK;
    p.off = AOTX_KVL_HEADER + (unsigned long long)(block % s.blocks_page) * s.block_bytes
          + 2ull * ((unsigned long long)krow * d + dim);
    return p;
}

/* rg_qkv_prep without branches around its loads: every field from selects, the page word
 * read unconditionally from a clamped index, so that the preparations of several units
 * have their page-table loads in flight together. Same result as rg_qkv_prep. */
static __device__ __forceinline__ rg_qkv_pre rg_qkv_prep_flat(const aotx_rgemv_args &a, unsigned int group,
                                                              unsigned int rt, unsigned int pr,
                                                              unsigned int mm, unsigned int position,
                                                              unsigned int agent, float fac, bool live)
{
    rg_qkv_pre p;
    const aotx_qkv_epi &e = a.qkv;
    const unsigned int row = 2u * pr;
    const unsigned int v = rg_vrow(a, group, row / 16u, row % 16u, rt);
    const bool ok = live && v < a.n;
    unsigned int begin;
    const unsigned int sg = rg_seg(a, v, begin);
    const unsigned int d = e.head_dim;
    const unsigned int local = v - begin;
    const unsigned int head = local / d;
    const unsigned int dim = local - head * d;
    const aotx_kvl_shape &s = e.shape;
    const unsigned int block = (position / AOTX_KVL_BLOCK) * s.layers + e.layer;
    const unsigned int index = s.blocks_page != 0u ? block / s.blocks_page : 0u;
    const bool page_ok = s.blocks_page != 0u && agent < AOTX_SLOTS && index < AOTX_KV_PAGES_EACH;
    const unsigned long long word = e.state->kv.page[page_ok ? agent : 0u][page_ok ? index : 0u];
    p.cs = 1.0f;
    p.sn = 0.0f;
    if (ok && sg <= 1u) {
        const float step = powf(e.theta, -2.0f / (float)d);
        float angle = (float)position * powf(step, (float)(dim >> 1));
        if (e.factor != nullptr) angle = angle / fac;
        sincosf(angle, &p.sn, &p.cs);
    }
    const unsigned int krow = (sg == 1u ? head : e.kv_heads + head) * AOTX_KVL_BLOCK
                            + position % AOTX_KVL_BLOCK;
    p.mode = !ok ? 0u : (sg == 0u ? 1u : (sg == 1u ? 2u : 3u));
    p.count_fault = ok && sg == 1u && dim == 0u ? 1u : 0u;
    p.base = sg == 0u ? (unsigned long long)e.qh : (page_ok ? word : 0ull);
    p.off = sg == 0u ? 2ull * ((unsigned long long)(a.m0 + mm) * e.heads * d + local)
                     : AOTX_KVL_HEADER + (unsigned long long)(s.blocks_page != 0u ? block % s.blocks_page : 0u)
                                       * s.block_bytes
                       + 2ull * ((unsigned long long)krow * d + dim);
    return p;
}

/* The place of output row `row`, batch row mm in a workgroup's result block out[]. The
 * epilogues read one batch row of consecutive output rows with consecutive lanes; with a
 * plain row stride of 32 or 64 floats those fall in one or two LDS banks. Blocks of 64
 * batch rows (the GEMM's) XOR mm with the row's low bits; blocks of 32 pad each row to 33
 * floats (a constant offset per row, so the accumulators' stores keep immediate offsets);
 * blocks of 16 keep the plain layout. rg_os is the row stride, the block is rows * rg_os. */
template <int MT>
static __device__ __forceinline__ constexpr unsigned int rg_os()
{
    return MT == 32 || MT == 16 ? (unsigned int)MT + 1u : (unsigned int)MT;
}
template <int MT>
static __device__ __forceinline__ unsigned int rg_o(unsigned int row, unsigned int mm)
{
    if constexpr (MT >= 64) return row * (unsigned int)MT + (mm ^ (row & (unsigned int)(MT - 1)));
    else return row * rg_os<MT>() + mm;
}
/* the same for the element idx of the block in row-major order */
template <int MT>
static __device__ __forceinline__ unsigned int rg_of(unsigned int idx)
{
    return rg_o<MT>(idx / (unsigned int)MT, idx % (unsigned int)MT);
}

template <int MT>
static __device__ __forceinline__ void rg_qkv_store(const aotx_rgemv_args &a, const float *out,
                                                    const rg_qkv_pre &p, unsigned int row,
                                                    unsigned int mm)
{
    if (p.mode == 0u) return;
    if (p.base == 0ull) {
        if (p.count_fault != 0u) atomicAdd(&a.qkv.state->faults, 1u);
        return;
    }
    const float a0 = out[rg_o<MT>(row, mm)];
    const float a1 = out[rg_o<MT>(row + 1u, mm)];
    unsigned short *dst = (unsigned short *)(p.base + p.off);
    if (p.mode == 3u) co_store2h(dst, aotx_f2h(a0), aotx_f2h(a1));
    else co_store2h(dst, aotx_f2h(a0 * p.cs - a1 * p.sn), aotx_f2h(a0 * p.sn + a1 * p.cs));
}

/* The next norm's weight of the workgroup's output row tid (tid < rt * 16; the residual
 * epilogue's xg_w), for a load issued before the weight stream: unconditional, from an
 * address clamped into xg_w (or into y when there is no next norm), masked where used. */
static __device__ __forceinline__ float rg_gw_load(const aotx_rgemv_args &a, unsigned int group,
                                                   unsigned int rt, unsigned int tid)
{
    const unsigned int j = tid / 16u;
    const unsigned int v = rg_vrow(a, group, j < rt ? j : 0u, tid % 16u, rt);
    const bool ok = a.xg_w != nullptr && j < rt && v < a.n;
    const float *src = a.xg_w != nullptr ? a.xg_w : (const float *)a.y;
    return src[ok ? v : 0u];
}

/* The GEMM's residual epilogue (rt == RTC, a tile of MT batch rows, the sums of squares
 * wanted): every residual value the thread adds to, and the next norm's weight of its output
 * row, requested together before the accumulators go to LDS, so that their round trip
 * overlaps the split merge and the row scale. With NT a multiple of 16 * RTC a thread keeps
 * one output row (tile j = (tid / 16) % RTC, row rr = tid % 16) for batch rows
 * tid / (16 * RTC) + i * NT / (16 * RTC); rv holds ITER values. */
template <int MT, int NT, int RTC>
struct rg_gres {
    static_assert(NT % (16 * RTC) == 0 && (RTC * 16 * MT) % NT == 0, "whole passes");
    static constexpr unsigned int ITER = (unsigned int)RTC * 16u * MT / NT;
    static constexpr unsigned int MSTEP = NT / (16u * RTC);
};

template <int MT, int NT, int RTC>
static __device__ __forceinline__ void rg_gres_load(const aotx_rgemv_args &a, unsigned int group,
                                                    unsigned int mrows, float *rv, float &gw)
{
    typedef rg_gres<MT, NT, RTC> G;
    const unsigned int tid = threadIdx.x;
    const unsigned int rr = tid & 15u, j = (tid >> 4) % RTC, mm0 = (tid >> 4) / RTC;
    const unsigned int v0 = rg_vrow(a, group, j, 0u, RTC);
    const bool v_ok = v0 + rr < a.n;
    gw = a.xg_out != nullptr ? a.xg_w[v_ok ? v0 + rr : 0u] : 0.0f;
#pragma unroll
    for (unsigned int i = 0; i < G::ITER; ++i) {
        const unsigned int mm = mm0 + i * G::MSTEP;
        /* unconditional, from an address clamped into the operand */
        const unsigned long long at = v_ok && mm < mrows ? (unsigned long long)(a.m0 + mm) * a.ldy + v0 + rr
                                                         : (unsigned long long)a.m0 * a.ldy;
        rv[i] = co_loadf((const float *)a.y + at);
    }
}

template <int MT, int NT, int RTC>
static __device__ __forceinline__ void rg_gres_store(const aotx_rgemv_args &a, const float *out,
                                                     unsigned int group, unsigned int mrows,
                                                     const float *rv, float gw)
{
    typedef rg_gres<MT, NT, RTC> G;
    const unsigned int tid = threadIdx.x;
    const unsigned int rr = tid & 15u, j = (tid >> 4) % RTC, mm0 = (tid >> 4) / RTC;
    const unsigned int v0 = rg_vrow(a, group, j, 0u, RTC);
    float sq[G::ITER];
#pragma unroll
    for (unsigned int i = 0; i < G::ITER; ++i) {
        const unsigned int mm = mm0 + i * G::MSTEP;
        const bool col_ok = mm < mrows && v0 + rr < a.n;
        float v = 0.0f;
        if (col_ok) {
            v = rv[i] + out[rg_o<MT>(j * 16u + rr, mm)];
            co_storef((float *)a.y + (unsigned long long)(a.m0 + mm) * a.ldy + v0 + rr, v);
            if (a.xg_out != nullptr)
                a.xg_out[a.out_frag ? aotx_xfrag_at(a.m0 + mm, v0 + rr)
                                    : (unsigned long long)(a.m0 + mm) * a.n + v0 + rr] = aotx_f2h(v * gw);
        }
        sq[i] = rg_sq(v);
    }
    /* the tiles' sums of squares */
#pragma unroll
    for (unsigned int i = 0; i < G::ITER; ++i) sq[i] = rg_sum16(sq[i]);
#pragma unroll
    for (unsigned int i = 0; i < G::ITER; ++i) {
        const unsigned int mm = mm0 + i * G::MSTEP;
        if (mm < mrows && v0 < a.n && rr == 0u)
            co_storef(a.sumsq_out + (unsigned long long)(a.m0 + mm) * ((a.n + 15u) / 16u) + v0 / 16u, sq[i]);
    }
}

/* Epilogue over the workgroup's result out[rg_o(row, m)], row = tile j * 16 + rr. rpre and
 * gpre, when given, hold the residual values out[] adds to and the next norm's weights of
 * the rows (gpre[row]), read while the weights streamed. */
template <int MT, int NT, int RTC = 0>
static __device__ __forceinline__ void rg_epilogue(const aotx_rgemv_args &a, const float *out,
                                                   unsigned int group, unsigned int rt,
                                                   unsigned int mrows, const unsigned int *list,
                                                   const float *rpre = nullptr,
                                                   const rg_qkv_pre *qp = nullptr,
                                                   const float *gpre = nullptr)
{
    const unsigned int tid = threadIdx.x;
    const unsigned int gr = rt * 16u;
#define RG_YROW(mm) (list != nullptr ? list[(mm)] : a.m0 + (mm))
    if constexpr (RTC > 0) {
        /* rt == RTC, known when compiled (the GEMM's tile; its residual epilogue is
         * rg_gres_store) */
        if (a.epi == AOTX_EPI_QKV && qp == nullptr && list == nullptr) {
            constexpr unsigned int PAIRS = (unsigned int)RTC * 8u;     /* output pairs per batch row */
            constexpr unsigned int ITER = PAIRS * MT / NT;
            constexpr unsigned int CH = ITER < 8u ? ITER : 8u;
            static_assert((PAIRS * MT) % NT == 0u && ITER % CH == 0u, "whole chunks");
            for (unsigned int c0 = 0; c0 < ITER; c0 += CH) {
                unsigned int posv[CH], agv[CH];
                float facv[CH];
#pragma unroll
                for (unsigned int i = 0; i < CH; ++i) {
                    const unsigned int idx = (c0 + i) * NT + tid;
                    const unsigned int pr = idx % PAIRS, mm = idx / PAIRS;
                    const unsigned int tc = a.m0 + (mm < mrows ? mm : 0u);   /* clamped */
                    posv[i] = a.qkv.pos[tc];
                    agv[i] = a.qkv.agent[tc];
                    facv[i] = rg_qkv_factor(a, group, RTC, pr);
                }
                rg_qkv_pre pv[CH];
#pragma unroll
                for (unsigned int i = 0; i < CH; ++i) {
                    const unsigned int idx = (c0 + i) * NT + tid;
                    const unsigned int pr = idx % PAIRS, mm = idx / PAIRS;
                    pv[i] = rg_qkv_prep_flat(a, group, RTC, pr, mm, posv[i], agv[i], facv[i], mm < mrows);
                }
#pragma unroll
                for (unsigned int i = 0; i < CH; ++i) {
                    const unsigned int idx = (c0 + i) * NT + tid;
                    const unsigned int pr = idx % PAIRS, mm = idx / PAIRS;
                    rg_qkv_store<MT>(a, out, pv[i], 2u * pr, mm);
                }
            }
            return;
        }
    }
    if (a.epi == AOTX_EPI_RESID && a.sumsq_out != nullptr) {
        /* one thread per output: 16 consecutive threads hold the 16 rows of one tile for
         * one row of x, add them into the residual stream, and leave the tile's sum of
         * squares for the next norm with a 16-lane shuffle sum */
        const unsigned int total = rt * 16u * MT;          /* a multiple of 16 */
        for (unsigned int base = 0; base < total; base += NT) {
            const unsigned int idx = base + tid;
            const unsigned int rr = idx & 15u, rest = idx >> 4;
            const unsigned int j = rest % rt, mm = rest / rt;
            const unsigned int v0 = rg_vrow(a, group, j, 0u, rt);
            const bool row_ok = idx < total && mm < mrows && v0 < a.n;
            const bool col_ok = row_ok && v0 + rr < a.n;
            /* the next norm's weight is read alongside the residual, not after it */
            const float gw = a.xg_out != nullptr && col_ok
                           ? (gpre != nullptr ? gpre[j * 16u + rr] : a.xg_w[v0 + rr]) : 0.0f;
            float v = 0.0f;
            if (col_ok) {
                float *p = (float *)a.y + (unsigned long long)RG_YROW(mm) * a.ldy + v0 + rr;
                v = (rpre != nullptr ? rpre[rg_o<MT>(j * 16u + rr, mm)] : co_loadf(p))
                  + out[rg_o<MT>(j * 16u + rr, mm)];
                co_storef(p, v);
            }
            if (a.xg_out != nullptr && col_ok)
                a.xg_out[a.out_frag ? aotx_xfrag_at(RG_YROW(mm), v0 + rr)
                                    : (unsigned long long)RG_YROW(mm) * a.n + v0 + rr] = aotx_f2h(v * gw);
            float sq = rg_sq(v);
            sq = rg_sum16(sq);
            if (row_ok && rr == 0u)
                co_storef(a.sumsq_out + (unsigned long long)RG_YROW(mm) * ((a.n + 15u) / 16u) + v0 / 16u, sq);
        }
    } else if (a.epi == AOTX_EPI_F32 || a.epi == AOTX_EPI_F16 || a.epi == AOTX_EPI_RESID) {
        for (unsigned int idx = tid; idx < gr * MT; idx += NT) {
            unsigned int row = idx % gr, mm = idx / gr;
            unsigned int v = rg_vrow(a, group, row / 16u, row % 16u, rt);
            if (mm >= mrows || v >= a.n) continue;
            float val = out[rg_o<MT>(row, mm)];
            unsigned long long at = (unsigned long long)RG_YROW(mm) * a.ldy + v;
            if (a.epi == AOTX_EPI_F32) co_storef((float *)a.y + at, val);
            else if (a.epi == AOTX_EPI_F16) ((unsigned short *)a.y)[at] = aotx_f2h(val);
            else ((float *)a.y)[at] += val;
        }
    } else if (a.epi == AOTX_EPI_SWIGLU) {
        /* a thread takes two adjacent units (one 32-bit store; n and ldy are even) */
        const unsigned int half = rt / 2u;
        for (unsigned int idx = tid; idx < half * 8u * MT; idx += NT) {
            unsigned int row = 2u * (idx % (half * 8u)), mm = idx / (half * 8u);
            unsigned int v = rg_vrow(a, group, row / 16u, row % 16u, rt);
            if (mm >= mrows || v >= a.n) continue;
            unsigned int h[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                float gate = out[rg_o<MT>(row + e, mm)];
                float up = out[rg_o<MT>(row + e + half * 16u, mm)];
                float unit = gate / (1.0f + expf(-gate));
                h[e] = aotx_f2h(unit * up);
            }
            unsigned short *dst = (unsigned short *)a.y
                                + (a.out_frag ? aotx_xfrag_at(RG_YROW(mm), v)
                                              : (unsigned long long)RG_YROW(mm) * a.ldy + v);
            if (v + 1u < a.n) co_store2h(dst, h[0], h[1]);
            else dst[0] = (unsigned short)h[0];            /* odd n */
        }
    } else if (a.epi == AOTX_EPI_QKV) {
        if (qp != nullptr) {
            /* prepared before the weight stream: one unit per thread */
            if (tid < (gr / 2u) * MT) rg_qkv_store<MT>(a, out, *qp, 2u * (tid % (gr / 2u)), tid / (gr / 2u));
        } else {
            for (unsigned int idx = tid; idx < (gr / 2u) * MT; idx += NT) {
                const unsigned int pr = idx % (gr / 2u), mm = idx / (gr / 2u);
                const bool live = mm < mrows;
                const unsigned int t = a.m0 + mm;
                const unsigned int position = live ? a.qkv.pos[t] : 0u;
                const unsigned int agent = live ? a.qkv.agent[t] : 0u;
                const float fac = rg_qkv_factor(a, group, rt, pr);
                const rg_qkv_pre p = rg_qkv_prep(a, group, rt, pr, mm, position, agent, fac, live);
                rg_qkv_store<MT>(a, out, p, 2u * pr, mm);
            }
        }
    }
#undef RG_YROW
}

/* The RMSNorm scale of batch rows given as unscaled x (a.row_ss): out[row][mm] *= rsqrt(
 * sum_i row_ss[m0 + mm][i] / k + eps), 16 threads per batch row adding its k/16 partial
 * sums in a fixed order. rs is MT floats of LDS; ends with a barrier. */
template <int MT, int NT>
static __device__ __forceinline__ void rg_row_scale(const aotx_rgemv_args &a, float *out,
                                                    unsigned int gr, unsigned int mrows, float *rs)
{
    const unsigned int tid = threadIdx.x;
    const unsigned int nss = (a.k + 15u) / 16u;
    for (unsigned int base = 0; base < (unsigned int)MT * 16u; base += NT) {
        const unsigned int mm = (base + tid) >> 4, l = tid & 15u;
        float sum = 0.0f;
        if (mm < mrows) {
            /* 16 loads in flight at a time, added in index order */
            const float *ss = a.row_ss + (unsigned long long)(a.m0 + mm) * nss;
            for (unsigned int i0 = l; i0 < nss; i0 += 256u) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const unsigned int i = i0 + 16u * (unsigned int)u;
                    v[u] = i < nss ? ss[i] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) sum += v[u];
            }
        }
        sum = rg_sum16(sum);
        if (l == 0u && mm < (unsigned int)MT) rs[mm] = rsqrtf(sum / (float)a.k + a.row_eps);
    }
    __syncthreads();
    for (unsigned int idx = tid; idx < gr * MT; idx += NT) out[rg_of<MT>(idx)] *= rs[idx % MT];
    __syncthreads();
}

/* The row scale of rg_row_scale with the partial sums loaded early, before the weight
 * stream, and added as soon as they arrive, before the product's loop (rows of at most 256
 * partials, k <= 4096): the same 16 threads per batch row and the same order of adds, so the
 * scale is bit-identical, and no register holds them through the loop. The loads are
 * unconditional (rows past cap read row 0, partials past the row read its first), masked
 * where they are added. */
template <int MT, int NT>
struct rg_ss_pre {
    float v[(MT * 16 + NT - 1) / NT][16];
};

template <int MT, int NT>
static __device__ __forceinline__ bool rg_row_ss_load(const aotx_rgemv_args &a, unsigned int cap,
                                                      rg_ss_pre<MT, NT> &p)
{
    const unsigned int nss = (a.k + 15u) / 16u;
    if (a.row_ss == nullptr || nss > 256u) return false;
    const unsigned int tid = threadIdx.x, l = tid & 15u;
#pragma unroll
    for (int sl = 0; sl < (MT * 16 + NT - 1) / NT; ++sl) {
        const unsigned int mm = ((unsigned int)sl * NT + tid) >> 4;
        const unsigned int mc = mm < cap ? mm : 0u;
        const float *ss = a.row_ss + (unsigned long long)(a.m0 + mc) * nss;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const unsigned int i = l + 16u * (unsigned int)u;
            p.v[sl][u] = ss[i < nss ? i : 0u];
        }
    }
    return true;
}

/* The row scales from the early partial sums into rs[MT] (LDS); the caller's later
 * barrier publishes them. */
template <int MT, int NT>
static __device__ __forceinline__ void rg_row_ss_sum(const aotx_rgemv_args &a, unsigned int mrows,
                                                     float *rs, const rg_ss_pre<MT, NT> &p)
{
    const unsigned int tid = threadIdx.x, l = tid & 15u;
    const unsigned int nss = (a.k + 15u) / 16u;
#pragma unroll
    for (int sl = 0; sl < (MT * 16 + NT - 1) / NT; ++sl) {
        const unsigned int mm = ((unsigned int)sl * NT + tid) >> 4;
        float sum = 0.0f;
        if (mm < mrows) {
#pragma unroll
            for (int u = 0; u < 16; ++u) sum += l + 16u * (unsigned int)u < nss ? p.v[sl][u] : 0.0f;
        }
        sum = rg_sum16(sum);
        if (l == 0u && mm < (unsigned int)MT) rs[mm] = rsqrtf(sum / (float)a.k + a.row_eps);
    }
}

/* Eight fp16 values x = half(scale * r * w) of the fused norm (cuda/model/norm.cu:49-77),
 * from the residual and norm-weight words already loaded. */
static __device__ __forceinline__ rg_u4 rg_norm_piece(rg_u4 r0, rg_u4 r1, rg_u4 w0, rg_u4 w1,
                                                      float scale)
{
    unsigned int rw[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
    unsigned int ww[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
    unsigned int h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        h[e] = aotx_f2h(scale * __builtin_bit_cast(float, rw[e]) * __builtin_bit_cast(float, ww[e]));
    return (rg_u4){h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

/* Eight values of row `src` of x from k = kk (fp16 x, or the fused norm of the residual
 * stream when scale != 0 is given for AOTX_X_NORM); k past a.k gives zeros. */
static __device__ __forceinline__ rg_u4 rg_x_piece(const aotx_rgemv_args &a, unsigned int src,
                                                   unsigned int kk, float scale)
{
    if (a.xmode == AOTX_X_NORM) {
        const float *rrow = a.resid + (unsigned long long)src * a.k;
        if (kk + 8u <= a.k)
            return rg_norm_piece(co_load4(rrow + kk), co_load4(rrow + kk + 4u),
                                 *(const rg_u4 *)(a.norm_w + kk), *(const rg_u4 *)(a.norm_w + kk + 4u),
                                 scale);
        unsigned int h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            unsigned int kc = kk + (unsigned int)e;
            h[e] = kc < a.k ? aotx_f2h(scale * co_loadf(rrow + kc) * a.norm_w[kc]) : 0u;
        }
        return (rg_u4){h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
    if (kk + 8u <= a.k) return co_load4(a.x + (unsigned long long)src * a.ldx + kk);
    unsigned int h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        h[e] = kk + (unsigned int)e < a.k ? a.x[(unsigned long long)src * a.ldx + kk + e] : 0u;
    return (rg_u4){h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

/* Split partials cross workgroups on different XCDs: device-scope stores and loads (past
 * the per-XCD L2, so no cache write-back or invalidation is needed). */
static __device__ __forceinline__ void rg_put(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ float rg_get(const float *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* k split over workgroups: publish this split's sums out[0, n); the last split of the
 * product group to arrive adds all splits in split order (its own from LDS) into out and
 * returns true; the others return false. The partials move as 16-byte device-coherent
 * (sc1) accesses, the form a relaxed agent-scope atomic word takes, four words at a time
 * (n is a multiple of 16 and the partial blocks are 16-byte aligned). All of this
 * workgroup's stores have completed before its arrival is counted; the last arrival puts
 * the counter back to zero. `last` is one word of LDS. */
#define RG_SC1 16    /* cache-policy bit of device-coherent accesses */
template <int NT, int N4 = 0>
static __device__ __forceinline__ bool rg_split_merge(const aotx_rgemv_args &a, float *out,
                                                      unsigned int n, unsigned int expert,
                                                      unsigned int group, unsigned int split,
                                                      unsigned int *last)
{
    const unsigned int tid = threadIdx.x;
    const unsigned long long tile = (unsigned long long)expert * a.groups + group;
    float *base = a.partial + tile * a.splits * n;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)base, (short)0, (int)(a.splits * n * 4u), 0x00020000);
    const unsigned int n4 = n / 4u;
    const rg_f4 *o4 = (const rg_f4 *)out;
    for (unsigned int i = tid; i < n4; i += NT)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(rg_u4, o4[i]), rs,
                                               (int)((split * n + 4u * i) * 4u), 0, RG_SC1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0u) {
        const unsigned int arrived = atomicAdd(a.count + tile, 1u);
        *last = arrived == a.splits - 1u ? 1u : 0u;
        if (*last != 0u) atomicExch(a.count + tile, 0u);
    }
    __syncthreads();
    if (*last == 0u) return false;
    rg_f4 *w4 = (rg_f4 *)out;
    if constexpr (N4 > 0) {
        /* n4 == N4, known when compiled: every element's loads of SC splits in flight
         * together (one round trip per SC splits instead of one per element and split),
         * added in split order as below */
        constexpr unsigned int IT = ((unsigned int)N4 + NT - 1u) / NT;
        constexpr unsigned int SC = IT >= 8u ? 1u : 4u;
        rg_f4 sum[IT];
#pragma unroll
        for (unsigned int j = 0; j < IT; ++j) sum[j] = (rg_f4){0.0f, 0.0f, 0.0f, 0.0f};
        for (unsigned int sp0 = 0; sp0 < a.splits; sp0 += SC) {
            rg_f4 v[SC][IT];
#pragma unroll
            for (unsigned int c = 0; c < SC; ++c)
#pragma unroll
                for (unsigned int j = 0; j < IT; ++j) {
                    const unsigned int sp = sp0 + c < a.splits ? sp0 + c : split;
                    const unsigned int i = tid + j * NT < (unsigned int)N4 ? tid + j * NT : tid;
                    v[c][j] = sp == split ? w4[i]
                        : __builtin_bit_cast(rg_f4, __builtin_amdgcn_raw_buffer_load_b128(
                              rs, (int)((sp * n + 4u * i) * 4u), 0, RG_SC1));
                }
#pragma unroll
            for (unsigned int c = 0; c < SC; ++c)
#pragma unroll
                for (unsigned int j = 0; j < IT; ++j)
                    if (sp0 + c < a.splits) sum[j] += v[c][j];
        }
        __syncthreads();      /* every read of this split's own values before the sums */
#pragma unroll
        for (unsigned int j = 0; j < IT; ++j)
            if (tid + j * NT < (unsigned int)N4) w4[tid + j * NT] = sum[j];
        __syncthreads();
        return true;
    }
    for (unsigned int i = tid; i < n4; i += NT) {
        rg_f4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
        const rg_f4 mine = w4[i];
#pragma unroll 8
        for (unsigned int sp = 0; sp < a.splits; ++sp) {
            const rg_f4 v = sp == split ? mine
                : __builtin_bit_cast(rg_f4, __builtin_amdgcn_raw_buffer_load_b128(
                      rs, (int)((sp * n + 4u * i) * 4u), 0, RG_SC1));
            sum += v;
        }
        w4[i] = sum;
    }
    __syncthreads();
    return true;
}

/* MT: batch columns of the MFMA (16 or 32); RT: 16-row tiles per workgroup; PD: quads
 * loaded ahead per wave; NW: waves per workgroup, splitting the k range (8 for products of
 * few tiles, so that each wave's share of the dequantisation is short). */
template <int MT, int RT, int PD, int NW, bool NORM, bool DIRECT>
static __device__ __forceinline__ void rg_narrow(const aotx_rgemv_args &a, unsigned int bx,
                                                 unsigned int expert_in, unsigned char *lds)
{
    /* DIRECT: batch row i is row m0 + i (no expert list, no row map), known when compiled */
    const unsigned int expert = DIRECT ? 0u : expert_in;
    constexpr unsigned int NT = 64u * NW;
    const unsigned int tid = threadIdx.x;
    const unsigned int lane = tid & 63u;
    const unsigned int wave = tid >> 6;
    const unsigned int *list = nullptr;
    unsigned int mrows = a.m;
    if (!DIRECT && a.expert_stride != 0ull) {
        /* an expert no row chose streams nothing */
        unsigned int total = rg_scalar(a.list_count + expert);
        mrows = total > a.m0 ? total - a.m0 : 0u;
        list = a.list + (unsigned long long)expert * a.list_cap + a.m0;
        if (mrows == 0u) return;
    }

    const unsigned int group = bx / a.splits;
    const unsigned int split = bx % a.splits;
    const unsigned int q0 = split * a.qps;
    const unsigned int q1 = q0 + a.qps < a.qn ? q0 + a.qps : a.qn;
    const unsigned int kr = a.qps * 128u;          /* LDS k capacity */
    const unsigned int xs = kr + 8u;               /* LDS x row stride (halves) */
    unsigned short *xl = (unsigned short *)lds;
    __shared__ unsigned int xsrc[MT];              /* source row of each batch row */
    __shared__ float xscale[MT];                   /* its RMSNorm scale (AOTX_X_NORM) */

    /* ---- per-wave share of the k range ---- */
    const unsigned int nq = q1 - q0;
    const unsigned int per = (nq + NW - 1u) / NW;
    const unsigned int wq0 = q0 + wave * per < q1 ? q0 + wave * per : q1;
    const unsigned int wq1 = wq0 + per < q1 ? wq0 + per : q1;
    const unsigned int r = lane & 15u, g = lane >> 4;

    const unsigned char *qb[RT];
    const unsigned short *sb[RT];
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        unsigned int dummy = 0u;
        qb[j] = rg_tile(a, group, (unsigned int)j, RT, expert, dummy) + lane * 16u;
        sb[j] = rg_scales(a, group, (unsigned int)j, RT, expert) + lane;
    }

    rg_f4 acc[RT][MT / 16];
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int t = 0; t < MT / 16; ++t) acc[j][t] = (rg_f4){0.0f, 0.0f, 0.0f, 0.0f};

    rg_u4 wa[2][PD][RT][2];
    unsigned int ws[2][PD][RT];    /* one 32-bit register per scale: no packing waits */

    /* loads past the wave's range repeat its last quad (a cache hit), so every load can be
     * issued unconditionally: no register copies that would wait for them */
    const unsigned int qlast = wq0 < wq1 ? wq1 - 1u : q0;
#define RG_LOAD(BUF, QS)                                                                 \
    do {                                                                                 \
        _Pragma("unroll") for (int qi = 0; qi < PD; ++qi) {                              \
            unsigned int qq = (QS) + (unsigned int)qi;                                   \
            if (qq > qlast) qq = qlast;                                                  \
            _Pragma("unroll") for (int j = 0; j < RT; ++j) {                             \
                const rg_u4 *src = (const rg_u4 *)(qb[j] + (unsigned long long)qq * 2048ull); \
                wa[BUF][qi][j][0] = __builtin_nontemporal_load(src);                    \
                wa[BUF][qi][j][1] = __builtin_nontemporal_load(src + 64);                \
                ws[BUF][qi][j] = __builtin_nontemporal_load(&sb[j][(unsigned long long)qq * 64ull]); \
            }                                                                            \
        }                                                                                \
    } while (0)

    /* Branch-free: a quad past the wave's range reads the last quad's x and has its scale
     * forced to zero (it adds nothing); a batch column past mrows reads row 0 of x (its
     * results are never written). */
#define RG_COMPUTE(BUF, QS)                                                              \
    do {                                                                                 \
        _Pragma("unroll") for (int qi = 0; qi < PD; ++qi) {                              \
            const unsigned int qq = (QS) + (unsigned int)qi;                             \
            const unsigned int qx = qq > qlast ? qlast : qq;                             \
            const unsigned short *xq = xl + (qx - q0) * 128u + 32u * g;                  \
            rg_h8 B[MT / 16][4];                                                         \
            _Pragma("unroll") for (int t = 0; t < MT / 16; ++t) {                        \
                const unsigned int mm = (unsigned int)t * 16u + r;                       \
                const unsigned int mr = mm < mrows ? mm : 0u;                            \
                _Pragma("unroll") for (int s = 0; s < 4; ++s)                            \
                    B[t][s] = *(const rg_h8 *)(xq + mr * xs + 8u * s);                   \
            }                                                                            \
            _Pragma("unroll") for (int j = 0; j < RT; ++j) {                             \
                const unsigned int sbits = qq < wq1 ? ws[BUF][qi][j] : 0u;               \
                rg_h2 s2 = __builtin_bit_cast(rg_h2, sbits | (sbits << 16));             \
                const rg_u4 q0v = wa[BUF][qi][j][0], q1v = wa[BUF][qi][j][1];            \
                unsigned int qd[8] = {q0v[0], q0v[1], q0v[2], q0v[3],                    \
                                      q1v[0], q1v[1], q1v[2], q1v[3]};                   \
                _Pragma("unroll") for (int s = 0; s < 4; ++s) {                          \
                    unsigned int d0, d1, d2, d3;                                         \
                    rg_dequant4(qd[2 * s], s2, d0, d1);                                  \
                    rg_dequant4(qd[2 * s + 1], s2, d2, d3);                              \
                    rg_u4 av = {d0, d1, d2, d3};                                         \
                    rg_h8 A = __builtin_bit_cast(rg_h8, av);                             \
                    _Pragma("unroll") for (int t = 0; t < MT / 16; ++t)                  \
                        acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(               \
                            A, B[t][s], acc[j][t], 0, 0, 0);                             \
                }                                                                        \
            }                                                                            \
        }                                                                                \
    } while (0)

    /* ---- loads that do not depend on the weights go out first. With direct rows (batch
     * row i is row m0 + i: no expert list, no row map) that is the first RG_PRE staging
     * rounds of x (or of the residual and norm weights, plus the sums of squares, for the
     * fused norm) and the residual values the epilogue adds to, for every row the pass
     * may hold. vmcnt counts in issue order, so these must precede the weight stream to
     * be waited for without it. ---- */
    constexpr int RG_PRE = 2;
    const bool direct = DIRECT || (list == nullptr && a.xrow == nullptr);
    const bool early = direct;
    const bool norm = NORM;
    const bool resid_pre = early && a.epi == AOTX_EPI_RESID && a.sumsq_out != nullptr;
    const unsigned int cap = a.m < (unsigned int)MT ? a.m : (unsigned int)MT;
    const unsigned int kbeg = q0 * 128u;
    const unsigned int pieces = (q1 - q0) * 16u;       /* 16-byte pieces (8 values) per row */
    const unsigned int nss = (a.k + 15u) / 16u;
    __shared__ float rres[RT * 16 * rg_os<MT>()];      /* the epilogue's residual values */
    __shared__ float rgw[RT * 16];                     /* and the next norm's weights */
    rg_u4 pre[RG_PRE][4];
    float ssp[16];
    float rold[(RT * 16 * MT + 64 * NW - 1) / (64 * NW)];
    /* Every early load is issued unconditionally, from an address clamped into the
     * operand (a piece out of range reads the row m0 at kbeg; kbeg + 8 <= k as k is a
     * multiple of 32), and masked where it is used: a load under a condition would be
     * waited for where its branch joins, before the weight stream goes out. */
    if (early) {
#pragma unroll
        for (int i = 0; i < RG_PRE; ++i) {
            const unsigned int idx = tid + (unsigned int)i * NT;
            unsigned int mm = idx / pieces, p = idx - mm * pieces;
            unsigned int kk = kbeg + p * 8u;
            if (!(mm < cap && kk + 8u <= a.k)) { mm = 0u; kk = kbeg; }
            if (NORM) {
                const float *rrow = a.resid + (unsigned long long)(a.m0 + mm) * a.k + kk;
                pre[i][0] = co_load4(rrow);
                pre[i][1] = co_load4(rrow + 4);
                pre[i][2] = *(const rg_u4 *)(a.norm_w + kk);
                pre[i][3] = *(const rg_u4 *)(a.norm_w + kk + 4u);
            } else {
                pre[i][0] = co_load4(a.x + (unsigned long long)(a.m0 + mm) * a.ldx + kk);
            }
        }
        if (NORM) {
            const unsigned int mm = tid >> 4, l = tid & 15u;
            const unsigned int mc = mm < cap ? mm : 0u;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const unsigned int at = l + 16u * (unsigned int)i;
                ssp[i] = co_loadf(a.sumsq + (unsigned long long)(a.m0 + mc) * nss + (at < nss ? at : 0u));
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    /* the QKV epilogue's batch words (position, slot) and rope factor go out with them: its
     * destinations and rotations are resolved while the weights stream */
    constexpr unsigned int QU = RT * 8u * MT;          /* output pairs of the workgroup */
    const bool qkv_pre = a.epi == AOTX_EPI_QKV && QU <= NT;
    unsigned int q_pos = 0u, q_agent = 0u;
    float q_fac = 1.0f;
    if (qkv_pre && tid < QU) {
        const unsigned int mm = tid / (RT * 8u);
        const unsigned int mc = mm < cap ? mm : 0u;      /* unconditional, as above */
        q_pos = a.qkv.pos[a.m0 + mc];
        q_agent = a.qkv.agent[a.m0 + mc];
        q_fac = rg_qkv_factor(a, group, RT, tid % (RT * 8u));
    }
    constexpr unsigned int RPT = (RT * 16u * MT + NT - 1u) / NT;   /* residual values per thread */
    if (resid_pre) {
#pragma unroll
        for (int it = 0; it < (int)RPT; ++it) {
            const unsigned int idx = tid + (unsigned int)it * NT;
            const unsigned int rr = idx & 15u, rest = idx >> 4;
            const unsigned int j = rest % RT, mm = rest / RT;
            const unsigned int v0 = rg_vrow(a, group, j, 0u, RT);
            const bool ok = idx < RT * 16u * MT && mm < cap && v0 + rr < a.n;
            rold[it] = co_loadf((const float *)a.y + (ok ? (unsigned long long)(a.m0 + mm) * a.ldy + v0 + rr
                                                         : (unsigned long long)a.m0 * a.ldy));
        }
    }
    const float gwv = resid_pre ? rg_gw_load(a, group, RT, tid) : 0.0f;

    __builtin_amdgcn_sched_barrier(0);
    /* with one tile per workgroup only the first buffer goes out before the staging, so
     * every workgroup's x requests queue behind less of the grid's weight stream (measured
     * faster for every one-tile shape; a gate/up pair keeps both buffers ahead) */
    const bool both_first = RT > 1;
    RG_LOAD(0, wq0);
    if (both_first) RG_LOAD(1, wq0 + PD);
    /* nothing that uses an early load may be scheduled above the weight stream's issue: the
     * sums start from a zero the compiler cannot see through, made after it */
    __builtin_amdgcn_sched_barrier(0);
    float zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    if ((DIRECT || a.expert_stride == 0ull) && a.m_dev != nullptr) {
        unsigned int total = rg_scalar(a.m_dev);
        mrows = total > a.m0 ? total - a.m0 : 0u;
    }
    if (mrows > a.m) mrows = a.m;
    if (mrows > (unsigned int)MT) mrows = MT;
    if (mrows == 0u) return;

    /* ---- stage the batch rows of x for [q0, q1) ---- */
    {
        /* sources, and norm scales (16 threads per row add its partial sums of squares) */
        {
            const unsigned int mm = tid >> 4, l = tid & 15u;
            unsigned int src = a.m0 + mm;
            if (!direct && mm < mrows)
                src = list != nullptr ? list[mm] / a.xrow_div : a.xrow[a.m0 + mm];
            if (l == 0u && mm < mrows) xsrc[mm] = src;
            if (norm) {
                float sum = zero;
                if (early) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) sum += l + 16u * (unsigned int)i < nss ? ssp[i] : 0.0f;
                    if (mm < mrows)
                        for (unsigned int i = l + 256u; i < nss; i += 16u)
                            sum += co_loadf(a.sumsq + (unsigned long long)src * nss + i);
                } else if (mm < mrows) {
                    const float *ss = a.sumsq + (unsigned long long)src * nss;
#pragma unroll 4
                    for (unsigned int i = l; i < nss; i += 16u) sum += co_loadf(ss + i);
                }
                sum = rg_sum16(sum);
                if (l == 0u && mm < mrows) xscale[mm] = rsqrtf(sum / (float)a.k + a.eps);
            }
        }
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
            if (tid < RT * 16u) rgw[tid] = gwv;
        }
        rg_sync_lds();
        const unsigned int total = mrows * pieces;
#pragma unroll
        for (int i = 0; i < RG_PRE; ++i) {
            const unsigned int idx = tid + (unsigned int)i * NT;
            if (idx < total) {
                const unsigned int mm = idx / pieces, p = idx - mm * pieces;
                const unsigned int kk = kbeg + p * 8u;
                rg_u4 v;
                if (early && kk + 8u <= a.k)
                    v = norm ? rg_norm_piece(pre[i][0], pre[i][1], pre[i][2], pre[i][3], xscale[mm])
                             : pre[i][0];
                else
                    v = rg_x_piece(a, xsrc[mm], kk, norm ? xscale[mm] : 0.0f);
                *(rg_u4 *)(xl + mm * xs + p * 8u) = v;
            }
        }
        for (unsigned int idx = tid + RG_PRE * NT; idx < total; idx += NT) {
            const unsigned int mm = idx / pieces, p = idx - mm * pieces;
            *(rg_u4 *)(xl + mm * xs + p * 8u) = rg_x_piece(a, xsrc[mm], kbeg + p * 8u,
                                                              norm ? xscale[mm] : 0.0f);
        }
        rg_sync_lds();
    }

    /* each buffer is refilled right after its quads are computed, two steps ahead */
    if (!both_first) RG_LOAD(1, wq0 + PD);
    rg_qkv_pre qpre = {0ull, 0ull, 1.0f, 0.0f, 0u, 0u};
    if (qkv_pre && tid < QU)
        qpre = rg_qkv_prep(a, group, RT, tid % (RT * 8u), tid / (RT * 8u), q_pos, q_agent, q_fac,
                           tid / (RT * 8u) < mrows);
    if (wq0 < wq1) {
        unsigned int q = wq0;
        for (;;) {
            RG_COMPUTE(0, q);
            q += PD;
            if (q >= wq1) break;
            RG_LOAD(0, q + PD);
            RG_COMPUTE(1, q);
            q += PD;
            if (q >= wq1) break;
            RG_LOAD(1, q + PD);
        }
    }
#undef RG_LOAD
#undef RG_COMPUTE

    /* ---- add the NW waves' accumulators in wave order ---- */
    __syncthreads();
    float *part = (float *)lds;                      /* [NW][RT*16][MT] */
    const unsigned int gr = RT * 16u;
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int t = 0; t < MT / 16; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                unsigned int row = (unsigned int)j * 16u + 4u * g + (unsigned int)i;
                part[(wave * gr + row) * MT + (unsigned int)t * 16u + r] = acc[j][t][i];
            }
    __syncthreads();
    float *out = part + NW * gr * MT;
    for (unsigned int idx = tid; idx < gr * MT; idx += NT) {
        float sum = part[idx];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += part[(unsigned int)w * gr * MT + idx];
        out[rg_of<MT>(idx)] = sum;
    }
    __syncthreads();
    if (a.splits > 1u) {
        __shared__ unsigned int last;
        if (!rg_split_merge<NT>(a, out, gr * rg_os<MT>(), expert, group, split, &last)) return;
    }
    rg_epilogue<MT, NT>(a, out, group, RT, mrows, list, resid_pre ? rres : nullptr,
                        qkv_pre ? &qpre : nullptr, resid_pre ? rgw : nullptr);
}


#endif
