/* Q8_0 matrix product for small batches on gfx950 matrix cores.
 *
 * Reference: the memory-bound product aotx_gemv_pass (cuda/model/gemv.cuh:33-125), the
 * hand-written m == 1 module (ptx/gemv_q8.ptx:18-223) and the tensor-core tile
 * aotx_gemm_tile (cuda/model/gemm.cuh:55-189), which dequantizes each weight to
 * half(q * scale) and sums in fp32. This kernel computes the same product with the same
 * operand values: A = half(q * scale) (exact int8 -> fp16, one correctly rounded fp16
 * multiply), B = the fp16 activations, fp32 accumulation in v_mfma_f32_16x16x32_f16.
 *
 * Work layout (one workgroup = 4 waves = 64 weight rows; the batch is the MFMA n side):
 *   - The k range is cut into chunks of cb blocks of 32 (cb = 32 for the production
 *     shapes: 16 rows x 32 blocks x 34 B = 17,408 B = 17 x 16 B per lane of a wave).
 *   - Each wave streams its 16 rows x cb blocks with fully coalesced 16-byte loads (the
 *     34-byte blocks are read as a flat byte run) into LDS, one padded LDS row per weight
 *     row; the next chunk's loads are issued before the current chunk is computed.
 *   - The chunk of the activations x [mt rows][cb*32] is staged once per workgroup in LDS
 *     and shared by the 4 waves.
 *   - A lane (r = lane % 16, g = lane / 16) reads one whole 34-byte block (row r, block
 *     4q + g) from LDS with aligned dword reads and feeds its 32 quants to 4 MFMAs, 8 per
 *     MFMA; the B operand takes the same k positions, so the k order inside each MFMA is a
 *     permutation shared by A and B and the sum is the plain dot product.
 *   - Split-K: when the rows alone give too few workgroups, the chunks are split over
 *     several workgroups; each writes its 64 x mt partial tile, and a second kernel (or
 *     the consumer of the result) adds the partials in split order, so the result does
 *     not depend on timing. Stream order makes the partials visible to it, so no
 *     workgroup waits on another and no device-wide cache write-back is issued.
 */
#include "gemv.h"

#include <algorithm>
#include <string.h>

typedef _Float16 aotx_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 aotx_h2 __attribute__((ext_vector_type(2)));
typedef float aotx_f4 __attribute__((ext_vector_type(4)));

#define GEMV_THREADS 256

typedef unsigned int aotx_u4 __attribute__((ext_vector_type(4)));

/* Four signed bytes -> two packed half2 of half(q * scale), exactly as the reference's
 * value reader rounds (cuda/model/matrix.cuh:413-422). The bytes are biased to unsigned,
 * placed under the fp16 exponent of 1024 (0x64xx = 1024 + byte), and 1152 is taken off:
 * q is exact; one fp16 multiply by the scale rounds once. */
static __device__ __forceinline__ void aotx_dequant4(unsigned int w, aotx_h2 s2,
                                                     unsigned int &lo, unsigned int &hi)
{
    unsigned int u = w ^ 0x80808080u;
    unsigned int a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    unsigned int b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const aotx_h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    aotx_h2 ha = (__builtin_bit_cast(aotx_h2, a) - bias) * s2;
    aotx_h2 hb = (__builtin_bit_cast(aotx_h2, b) - bias) * s2;
    lo = __builtin_bit_cast(unsigned int, ha);
    hi = __builtin_bit_cast(unsigned int, hb);
}

/* The weight rows of one wave's 16-row tile. */
static __device__ __forceinline__ void aotx_gemv_tile(const aotx_gemv_args &a,
                                                      unsigned int group, unsigned int wave,
                                                      const unsigned char *&base,
                                                      unsigned int &row0,
                                                      unsigned int &seg_rows,
                                                      unsigned int &seg)
{
    if (a.epi == AOTX_EPI_SWIGLU) {
        seg = wave >> 1;
        row0 = group * 32u + (wave & 1u) * 16u;
        seg_rows = a.n;
    } else {
        unsigned int v0 = group * 64u + wave * 16u;
        unsigned int begin = 0u;
        seg = 0u;
        while (seg + 1u < a.nseg && v0 >= a.seg_end[seg]) {
            begin = a.seg_end[seg];
            seg += 1u;
        }
        row0 = v0 - begin;
        seg_rows = a.seg_end[seg] - begin;
    }
    base = a.w[seg];
}

/* The epilogues, from the 64 x MT result tile of one row group in LDS (out[row*MT+m]). */
template <int MT>
static __device__ __forceinline__ void aotx_gemv_epilogue(const aotx_gemv_args &a,
                                                          const float *out,
                                                          unsigned int group,
                                                          unsigned int mrows,
                                                          const unsigned int *list)
{
    const unsigned int tid = threadIdx.x;
    /* result row of batch row mm: m0 + mm, or the routed slot */
#define AOTX_YROW(mm) (list != nullptr ? list[(mm)] : a.m0 + (mm))
    const unsigned int m0 = a.m0;
    if (a.epi == AOTX_EPI_F32 || a.epi == AOTX_EPI_F16 || a.epi == AOTX_EPI_RESID) {
        for (unsigned int idx = tid; idx < 64u * MT; idx += GEMV_THREADS) {
            unsigned int row = idx & 63u;
            unsigned int mm = idx >> 6;
            unsigned int vrow = group * 64u + row;
            if (mm >= mrows || vrow >= a.n) continue;
            float v = out[row * MT + mm];
            unsigned long long at = (unsigned long long)AOTX_YROW(mm) * a.ldy + vrow;
            if (a.epi == AOTX_EPI_F32) {
                ((float *)a.y)[at] = v;
            } else if (a.epi == AOTX_EPI_F16) {
                ((unsigned short *)a.y)[at] = aotx_f2h(v);
            } else {
                ((float *)a.y)[at] += v;
            }
        }
    } else if (a.epi == AOTX_EPI_SWIGLU) {
        /* act = half(silu(gate) * up), as cuda/model/norm.cu:92-105 rounds it. */
        for (unsigned int idx = tid; idx < 32u * MT; idx += GEMV_THREADS) {
            unsigned int i = idx & 31u;
            unsigned int mm = idx >> 5;
            unsigned int nrow = group * 32u + i;
            if (mm >= mrows || nrow >= a.n) continue;
            float gate = out[i * MT + mm];
            float up = out[(32u + i) * MT + mm];
            float unit = gate / (1.0f + expf(-gate));
            ((unsigned short *)a.y)[(unsigned long long)AOTX_YROW(mm) * a.ldy + nrow] =
                aotx_f2h(unit * up);
        }
    } else if (a.epi == AOTX_EPI_QKV) {
        /* Adjacent rotary pairs (2i, 2i+1) of a head (cuda/model/rope.cu:88-99, :200-234,
         * llama rule of cuda/model/rope_families.h:18): q -> half(rot(q)) into qh,
         * k -> half(rot(k)) and v -> half(v) into the slot's pages. */
        const aotx_qkv_epi &e = a.qkv;
        const unsigned int d = e.head_dim;
        const float step = powf(e.theta, -2.0f / (float)d);
        unsigned int v0 = group * 64u;
        unsigned int sg = 0u, begin = 0u;
        while (sg + 1u < a.nseg && v0 >= a.seg_end[sg]) {
            begin = a.seg_end[sg];
            sg += 1u;
        }
        for (unsigned int idx = tid; idx < 32u * MT; idx += GEMV_THREADS) {
            unsigned int p = idx & 31u;
            unsigned int mm = idx >> 5;
            unsigned int local = v0 - begin + 2u * p;
            if (mm >= mrows || v0 + 2u * p >= a.n) continue;
            unsigned int t = m0 + mm;
            float a0 = out[(2u * p) * MT + mm];
            float a1 = out[(2u * p + 1u) * MT + mm];
            unsigned int head = local / d;
            unsigned int dim = local - head * d;
            unsigned int position = e.pos[t];
            if (sg == 0u) {
                float angle = (float)position * powf(step, (float)(dim >> 1));
                if (e.factor != nullptr) angle = angle / e.factor[dim >> 1];
                float sn, cs;
                sincosf(angle, &sn, &cs);
                unsigned short *dst = e.qh + (unsigned long long)t * e.heads * d + local;
                dst[0] = aotx_f2h(a0 * cs - a1 * sn);
                dst[1] = aotx_f2h(a0 * sn + a1 * cs);
                continue;
            }
            unsigned char *blk = aotx_kvl_block(e.shape, &e.state->kv, e.agent[t], e.layer,
                                                position);
            if (blk == nullptr) {
                if (dim == 0u && sg == 1u) atomicAdd(&e.state->faults, 1u);
                continue;
            }
            unsigned int row = (sg == 1u ? head : e.kv_heads + head) * AOTX_KVL_BLOCK
                             + position % AOTX_KVL_BLOCK;
            unsigned short *dst = (unsigned short *)blk + (unsigned long long)row * d + dim;
            if (sg == 1u) {
                float angle = (float)position * powf(step, (float)(dim >> 1));
                if (e.factor != nullptr) angle = angle / e.factor[dim >> 1];
                float sn, cs;
                sincosf(angle, &sn, &cs);
                dst[0] = aotx_f2h(a0 * cs - a1 * sn);
                dst[1] = aotx_f2h(a0 * sn + a1 * cs);
            } else {
                dst[0] = aotx_f2h(a0);
                dst[1] = aotx_f2h(a1);
            }
        }
    }
#undef AOTX_YROW
}


/* CB = blocks per chunk known at compile time (32, 16 or 8: the coalesced path), or 0
 * for any other chunk (a plain 2-byte staging path, used by small shapes only). */
template <int MT, int CB>
__global__ __launch_bounds__(GEMV_THREADS) void aotx_gemv_q8(aotx_gemv_args a)
{
    constexpr bool FAST = CB != 0;
    constexpr int NL = FAST ? (34 * CB + 63) / 64 : 1;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

    const unsigned int tid = threadIdx.x;
    const unsigned int lane = tid & 63u;
    const unsigned int wave = tid >> 6;
    const unsigned int expert = blockIdx.y;
    const unsigned int *list = nullptr;
    unsigned int mrows = a.m;
    if (a.expert_stride != 0ull) {
        unsigned int total = a.list_count[expert];
        mrows = total > a.m0 ? total - a.m0 : 0u;
        list = a.list + (unsigned long long)expert * a.list_cap + a.m0;
    } else if (a.m_dev != nullptr) {
        unsigned int total = *a.m_dev;
        mrows = total > a.m0 ? total - a.m0 : 0u;
    }
    if (mrows > (unsigned int)MT) mrows = MT;
    if (mrows == 0u) return;

    const unsigned int group = blockIdx.x / a.splits;
    const unsigned int split = blockIdx.x % a.splits;
    const unsigned int cb = FAST ? (unsigned int)CB : a.cb;
    const unsigned int rb = 34u * cb;                     /* bytes of one row chunk */
    const unsigned int rs = ((rb + 15u) & ~15u) + 16u;    /* padded LDS row stride */
    const unsigned int xs = cb * 32u + 8u;                /* LDS x row stride, halves */
    unsigned char *wl = lds + wave * 16u * rs;
    unsigned short *xl = (unsigned short *)(lds + 64u * rs);

    const unsigned char *wbase;
    unsigned int row0, seg_rows, seg;
    aotx_gemv_tile(a, group, wave, wbase, row0, seg_rows, seg);
    wbase += (unsigned long long)expert * a.expert_stride;

    const unsigned int c_begin = split * a.cps;
    unsigned int c_end = c_begin + a.cps;
    if (c_end > a.chunks) c_end = a.chunks;

    /* Per-lane load plan (FAST path): the i-th 16-byte piece of the tile, as a 32-bit
     * offset from the tile's first row. Every load is issued unconditionally; a piece
     * past the tile re-reads piece 0 and is not stored, so no load waits on a branch. */
    const unsigned int per_row = rb / 16u;
    const unsigned int pieces = 16u * per_row;
    const unsigned int row_first = row0 < seg_rows ? row0 : seg_rows - 1u;
    const unsigned char *tile = wbase + (unsigned long long)row_first * a.row_bytes;
    unsigned int goff[NL];
    unsigned int loff[NL];
    aotx_u4 reg[NL];
    if (FAST) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            unsigned int f = lane + 64u * (unsigned int)i;
            bool in = f < pieces;
            unsigned int ff = in ? f : 0u;
            unsigned int j = ff / per_row;
            unsigned int p = ff - j * per_row;
            unsigned int rr = row0 + j;
            if (rr >= seg_rows) rr = seg_rows - 1u;
            goff[i] = (rr - row_first) * (unsigned int)a.row_bytes + p * 16u;
            loff[i] = in ? j * rs + p * 16u : 0xFFFFFFFFu;
        }
    }

    aotx_f4 acc[MT / 16];
#pragma unroll
    for (int t = 0; t < MT / 16; ++t) acc[t] = (aotx_f4){0.0f, 0.0f, 0.0f, 0.0f};

    const unsigned int r = lane & 15u;
    const unsigned int g = lane >> 4;
    const unsigned int quads = (cb + 3u) / 4u;

    if (FAST && c_begin < c_end) {
        const unsigned char *at = tile + (unsigned long long)c_begin * rb;
#pragma unroll
        for (int i = 0; i < NL; ++i) reg[i] = *(const aotx_u4 *)(at + goff[i]);
    }

    for (unsigned int c = c_begin; c < c_end; ++c) {
        __syncthreads();                       /* the previous chunk is consumed */
        if (FAST) {
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                if (loff[i] != 0xFFFFFFFFu) *(aotx_u4 *)(wl + loff[i]) = reg[i];
            }
        } else {
            const unsigned char *at = wbase + (unsigned long long)c * rb;
            const unsigned int halves = rb / 2u;
            for (unsigned int u = lane; u < 16u * halves; u += 64u) {
                unsigned int j = u / halves;
                unsigned int p = u - j * halves;
                unsigned int rr = row0 + j;
                if (rr >= seg_rows) rr = seg_rows - 1u;
                unsigned short v =
                    *(const unsigned short *)(at + (unsigned long long)rr * a.row_bytes + 2u * p);
                *(unsigned short *)(wl + j * rs + 2u * p) = v;
            }
        }
        /* Stage this chunk of the activations for the whole workgroup. */
        {
            const unsigned int per_m = cb * 4u;   /* 16-byte pieces per x row */
            const unsigned short *xsrc = a.x + (unsigned long long)a.m0 * a.ldx + c * cb * 32u;
            for (unsigned int idx = tid; idx < mrows * per_m; idx += GEMV_THREADS) {
                unsigned int mm = idx / per_m;
                unsigned int p = idx - mm * per_m;
                unsigned long long xr = list != nullptr
                    ? (unsigned long long)(list[mm] / a.xrow_div) * a.ldx - (unsigned long long)a.m0 * a.ldx
                    : (unsigned long long)mm * a.ldx;
                aotx_u4 v = *(const aotx_u4 *)(xsrc + xr + p * 8u);
                *(aotx_u4 *)(xl + mm * xs + p * 8u) = v;
            }
        }
        if (FAST && c + 1u < c_end) {
            const unsigned char *at = tile + (unsigned long long)(c + 1u) * rb;
#pragma unroll
            for (int i = 0; i < NL; ++i) reg[i] = *(const aotx_u4 *)(at + goff[i]);
        }
        __syncthreads();

        for (unsigned int q = 0; q < quads; ++q) {
            unsigned int b = 4u * q + g;
            bool ok = b < cb;
            unsigned int bb = ok ? b : 0u;
            unsigned int o = r * rs + 34u * bb;
            const unsigned int *dp = (const unsigned int *)(wl + (o & ~3u));
            unsigned int dw[9];
#pragma unroll
            for (int t = 0; t < 9; ++t) dw[t] = dp[t];
            bool aligned = (o & 3u) != 0u;   /* scale in the high half: quants aligned */
            unsigned int sbits = aligned ? (dw[0] >> 16) : (dw[0] & 0xFFFFu);
            unsigned int s2bits = sbits | (sbits << 16);
            aotx_h2 s2 = __builtin_bit_cast(aotx_h2, s2bits);
            unsigned int qd[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                qd[t] = aligned ? dw[t + 1] : __builtin_amdgcn_alignbyte(dw[t + 1], dw[t], 2u);
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                unsigned int a0, a1, a2, a3;
                aotx_dequant4(qd[2 * s], s2, a0, a1);
                aotx_dequant4(qd[2 * s + 1], s2, a2, a3);
                aotx_u4 av = {a0, a1, a2, a3};
                aotx_h8 A = __builtin_bit_cast(aotx_h8, av);
                if (!ok) A = (aotx_h8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < MT / 16; ++t) {
                    unsigned int mm = (unsigned int)t * 16u + r;
                    aotx_h8 B = (aotx_h8){0, 0, 0, 0, 0, 0, 0, 0};
                    if (ok && mm < mrows) {
                        B = *(const aotx_h8 *)(xl + mm * xs + 32u * b + 8u * (unsigned int)s);
                    }
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc[t], 0, 0, 0);
                }
            }
        }
    }

    /* Gather the 64 x MT tile of the workgroup in LDS: lane holds rows 4g..4g+3 of its
     * wave's tile at column r of each 16-column MFMA tile. */
    __syncthreads();
    float *out = (float *)lds;
#pragma unroll
    for (int t = 0; t < MT / 16; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            unsigned int row = wave * 16u + 4u * g + (unsigned int)i;
            out[row * MT + (unsigned int)t * 16u + r] = acc[t][i];
        }
    }
    __syncthreads();

    if (a.splits > 1u) {
        /* Split-K: this workgroup's partial tile; a following kernel adds the splits in
         * split order (stream order makes them visible; no cross-workgroup fence). */
        float *mine = a.partial + ((unsigned long long)group * a.splits + split) * 64u * MT;
        for (unsigned int idx = tid; idx < 64u * MT; idx += GEMV_THREADS) mine[idx] = out[idx];
        return;
    }
    aotx_gemv_epilogue<MT>(a, out, group, mrows, list);
}

/* Add the split partials of one 64-row group in split order, then apply the epilogue. */
template <int MT>
__global__ __launch_bounds__(GEMV_THREADS) void aotx_gemv_reduce(aotx_gemv_args a)
{
    __shared__ float out[64 * MT];
    unsigned int mrows = a.m;
    if (a.m_dev != nullptr) {
        unsigned int total = *a.m_dev;
        mrows = total > a.m0 ? total - a.m0 : 0u;
    }
    if (mrows > (unsigned int)MT) mrows = MT;
    if (mrows == 0u) return;
    const unsigned int group = blockIdx.x;
    const float *all = a.partial + (unsigned long long)group * a.splits * 64u * MT;
    for (unsigned int idx = threadIdx.x; idx < 64u * MT; idx += GEMV_THREADS) {
        float sum = 0.0f;
        for (unsigned int sp = 0; sp < a.splits; ++sp) sum += all[(unsigned long long)sp * 64u * MT + idx];
        out[idx] = sum;
    }
    __syncthreads();
    aotx_gemv_epilogue<MT>(a, out, group, mrows, nullptr);
}

/* ---------------------------------------------------------------------------------------
 * Host side
 * ------------------------------------------------------------------------------------- */

static unsigned int aotx_gemv_pick_cb(unsigned int nb)
{
    if (nb % 32u == 0u) return 32u;
    if (nb % 16u == 0u) return 16u;
    if (nb % 8u == 0u) return 8u;
    for (unsigned int c = (nb < 32u ? nb : 32u); c > 0u; --c) {
        if (nb % c == 0u) return c;
    }
    return 1u;
}

int aotx_gemv_plan(aotx_gemv_args *a, const void *const *w, const unsigned int *rows,
                   unsigned int nseg, unsigned int k, int epi)
{
    memset(a, 0, sizeof *a);
    if (k == 0u || k % 32u != 0u || nseg == 0u || nseg > 3u) return 1;
    unsigned int nb = k / 32u;
    a->k = k;
    a->row_bytes = (unsigned long long)nb * 34ull;
    a->cb = aotx_gemv_pick_cb(nb);
    a->chunks = nb / a->cb;
    a->nseg = nseg;
    a->epi = epi;
    unsigned int total = 0u;
    for (unsigned int s = 0; s < nseg; ++s) {
        if (rows[s] == 0u || w[s] == nullptr) return 1;
        a->w[s] = (const unsigned char *)w[s];
        total += rows[s];
        a->seg_end[s] = total;
        if (epi != AOTX_EPI_SWIGLU && s + 1u < nseg && rows[s] % 64u != 0u) return 1;
        if (epi == AOTX_EPI_QKV && rows[s] % 64u != 0u) return 1;
    }
    if (epi == AOTX_EPI_SWIGLU) {
        if (nseg != 2u || rows[0] != rows[1]) return 1;
        a->n = rows[0];
        a->groups = (a->n + 31u) / 32u;
    } else {
        a->n = total;
        a->groups = (total + 63u) / 64u;
    }
    /* Split the chunks until the launch holds about two workgroups per CU. */
    const unsigned int target = 512u;
    unsigned int want = (target + a->groups - 1u) / a->groups;
    if (want > a->chunks) want = a->chunks;
    if (want < 1u) want = 1u;
    a->cps = (a->chunks + want - 1u) / want;
    a->splits = (a->chunks + a->cps - 1u) / a->cps;
    return 0;
}

static size_t aotx_gemv_lds(const aotx_gemv_args &a, int mt)
{
    unsigned int rb = 34u * a.cb;
    unsigned int rs = ((rb + 15u) & ~15u) + 16u;
    size_t w = 64u * (size_t)rs;
    size_t x = (size_t)mt * (a.cb * 32u + 8u) * 2u;
    size_t out = 64u * (size_t)mt * 4u;
    size_t need = w + x;
    return need > out ? need : out;
}

static size_t aotx_gemv_lds_limit = 0;

void aotx_gemv_init(void)
{
    if (aotx_gemv_lds_limit != 0) return;
    int dev = 0, bytes = 0;
    AOTX_CHECK(hipGetDevice(&dev));
    AOTX_CHECK(hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    aotx_gemv_lds_limit = (size_t)bytes;
}

template <int MT, int CB>
static int aotx_gemv_go(const aotx_gemv_args &a, hipStream_t stream)
{
    size_t lds = aotx_gemv_lds(a, MT);
    aotx_gemv_init();
    if (lds + 64u > aotx_gemv_lds_limit) {
        fprintf(stderr, "aotx: the product needs %zu bytes of LDS, the device gives %zu\n",
                lds, aotx_gemv_lds_limit);
        return 1;
    }
    unsigned int ey = a.expert_stride != 0ull ? a.experts : 1u;
    hipLaunchKernelGGL((aotx_gemv_q8<MT, CB>), dim3(a.groups * a.splits, ey), dim3(GEMV_THREADS),
                       lds, stream, a);
    AOTX_LAUNCH_CHECK();
    if (a.splits > 1u && !a.defer) {
        hipLaunchKernelGGL((aotx_gemv_reduce<MT>), dim3(a.groups), dim3(GEMV_THREADS), 0, stream, a);
        AOTX_LAUNCH_CHECK();
    }
    return 0;
}

template <int MT>
static int aotx_gemv_cb(const aotx_gemv_args &a, hipStream_t stream)
{
    bool aligned = (a.row_bytes % 16ull) == 0ull;
    if (aligned && a.cb == 32u) return aotx_gemv_go<MT, 32>(a, stream);
    if (aligned && a.cb == 16u) return aotx_gemv_go<MT, 16>(a, stream);
    if (aligned && a.cb == 8u) return aotx_gemv_go<MT, 8>(a, stream);
    return aotx_gemv_go<MT, 0>(a, stream);
}

int aotx_gemv_launch(aotx_gemv_args a, hipStream_t stream)
{
    /* With a device row count, a.m is the capacity of the pass (16 or 32). */
    unsigned int mt_need = a.m;
    if (a.splits > 1u && a.partial == nullptr) {
        a.partial = (float *)aotx_scratch(AOTX_SCRATCH_GEMV_PARTIAL,
                                          (size_t)a.groups * a.splits * 64u * 32u * sizeof(float));
    }
    if (mt_need <= 16u) return aotx_gemv_cb<16>(a, stream);
    return aotx_gemv_cb<32>(a, stream);
}

int aotx_gemv_run(aotx_gemv_args a, unsigned int m, hipStream_t stream)
{
    for (unsigned int m0 = 0; m0 < m; m0 += 32u) {
        aotx_gemv_args p = a;
        p.m0 = m0;
        p.m = (m - m0 < 32u) ? (m - m0) : 32u;
        p.m_dev = nullptr;
        if (aotx_gemv_launch(p, stream) != 0) return 1;
    }
    return 0;
}

/* ---------------------------------------------------------------------------------------
 * Kernel-level C ABI
 * ------------------------------------------------------------------------------------- */

static int aotx_q8_gemv_any(const void *w, unsigned int n, unsigned int k, const void *x,
                            unsigned int m, void *y, int epi, void *stream)
{
    if (w == nullptr || x == nullptr || y == nullptr || n == 0u || m == 0u) return 1;
    if (k % 32u != 0u || k % 8u != 0u) return 1;
    aotx_gemv_args a;
    const void *ws[1] = {w};
    unsigned int rows[1] = {n};
    if (aotx_gemv_plan(&a, ws, rows, 1u, k, epi) != 0) return 1;
    a.x = (const unsigned short *)x;
    a.ldx = k;
    a.y = y;
    a.ldy = n;
    return aotx_gemv_run(a, m, aotx_stream(stream));
}

extern "C" int aotx_q8_gemv(const void *w, unsigned int n, unsigned int k, const void *x,
                            unsigned int m, float *y, void *stream)
{
    return aotx_q8_gemv_any(w, n, k, x, m, y, AOTX_EPI_F32, stream);
}

extern "C" int aotx_q8_gemv_f16(const void *w, unsigned int n, unsigned int k,
                                const void *x, unsigned int m, void *y, void *stream)
{
    return aotx_q8_gemv_any(w, n, k, x, m, y, AOTX_EPI_F16, stream);
}

/* Dequantize rows to fp16 (cuda/model/dequant.cu:9-70): half(q * scale). */
__global__ void aotx_q8_dequant_kernel(const unsigned char *w, unsigned int k,
                                       unsigned int first, unsigned int rows,
                                       unsigned short *out)
{
    unsigned long long total = (unsigned long long)rows * k;
    unsigned long long row_bytes = (unsigned long long)(k / 32u) * 34ull;
    for (unsigned long long i = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x;
         i < total; i += (unsigned long long)gridDim.x * blockDim.x) {
        unsigned long long r = i / k;
        unsigned int c = (unsigned int)(i - r * k);
        const unsigned char *blk = w + (first + r) * row_bytes + (c / 32u) * 34ull;
        unsigned short sb = (unsigned short)(blk[0] | (blk[1] << 8));
        float scale = aotx_h2f(sb);
        int q = (int)(signed char)blk[2u + c % 32u];
        out[i] = aotx_f2h((float)q * scale);
    }
}

extern "C" int aotx_q8_dequant(const void *w, unsigned int k, unsigned int first_row,
                               unsigned int rows, void *out, void *stream)
{
    if (w == nullptr || out == nullptr || k % 32u != 0u || rows == 0u) return 1;
    unsigned long long total = (unsigned long long)rows * k;
    unsigned int blocks = (unsigned int)std::min<unsigned long long>((total + 255u) / 256u, 65535ull);
    hipLaunchKernelGGL(aotx_q8_dequant_kernel, dim3(blocks), dim3(256), 0, aotx_stream(stream),
                       (const unsigned char *)w, k, first_row, rows, (unsigned short *)out);
    AOTX_LAUNCH_CHECK();
    return 0;
}

size_t aotx_gemv_scratch_partial(const aotx_gemv_args &a)
{
    return a.splits > 1u ? (size_t)a.groups * a.splits * 64u * 32u * sizeof(float) : 0u;
}
