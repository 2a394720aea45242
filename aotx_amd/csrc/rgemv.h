/* The streaming Q8 product over repacked weights (rgemv.hip).
 *
 * Repacked layout ("Q8R") of a Q8_0 tensor [n][k]: the same bytes per weight (one int8
 * per weight, one fp16 scale per 32), reordered at model open so that one wave reads its
 * MFMA operands with fully coalesced 16-byte loads and no LDS:
 *   tiles  T  = ceil(n / 16)         (16 weight rows; rows past n are zero)
 *   quads  Qn = ceil(k / 128)        (4 blocks of 32; blocks past k are zero)
 *   quants: [T][Qn][2 halves][64 lanes][16 B]  lane l = r + 16 g holds row 16t + r,
 *           block 4Q + g: quants 0..15 in the first half, 16..31 in the second, so each of a
 *           wave's two 16-byte loads reads 1 KB of contiguous bytes; each quant is stored
 *           as the byte q + 128 (q XOR 0x80), which the dequantisation uses as it is
 *   scales: [T][Qn][64 lanes] fp16   the scale of that block
 * A tensor is 34/32 bytes per weight plus the padding of the last tile and quad (q = 0,
 * scale 0).
 */
#ifndef AOTX_RGEMV_H
#define AOTX_RGEMV_H

#include "aotx_internal.h"
#include "gemv.h"

static inline __host__ __device__ unsigned long long aotx_q8r_quads(unsigned int k) { return (k + 127u) / 128u; }
static inline __host__ __device__ unsigned long long aotx_q8r_tiles(unsigned int n) { return (n + 15u) / 16u; }
static inline unsigned long long aotx_q8r_quant_bytes(unsigned int n, unsigned int k)
{
    return aotx_q8r_tiles(n) * aotx_q8r_quads(k) * 64ull * 32ull;
}
static inline unsigned long long aotx_q8r_bytes(unsigned int n, unsigned int k)
{
    return aotx_q8r_tiles(n) * aotx_q8r_quads(k) * 64ull * 34ull;
}

/* Repack a Q8_0 tensor (row-major [rows][k/32] blocks) into Q8R on the stream. */
void aotx_q8r_repack(const void *src, unsigned int n, unsigned int k, void *dst, hipStream_t s);

/* How the batch rows of x reach the product. */
enum {
    AOTX_X_F16 = 0,       /* x fp16 [rows][ldx] in device memory */
    AOTX_X_NORM = 1,      /* x = half(rsqrt(ss/h + eps) * resid * w) computed per workgroup */
    AOTX_X_FRAG = 2       /* x fp16 in the fragment layout (aotx_xfrag_at), 32 rows, m0 = 0 */
};

struct aotx_rgemv_args {
    const unsigned char *w[3];    /* Q8R tensors stacked along n */
    unsigned int seg_end[3];      /* cumulative row ends (multiples of 16 except the last) */
    unsigned int nseg;
    unsigned int n;               /* rows (SWIGLU: rows of one of the pair) */
    unsigned int k;
    unsigned int qn;              /* quads of k */
    unsigned int rt;              /* 16-row tiles per workgroup */
    unsigned int wide;            /* 1: the tile-split wide-batch kernel (fp16 x only) */
    unsigned int gemm;            /* 1: the GEMM of 33..512 rows (fp16 x, direct rows) */
    unsigned int frag;            /* 1: the fragment-layout product (AOTX_X_FRAG, 5..32 rows) */
    unsigned int pd;              /* quads loaded ahead per wave (narrow kernel) */
    unsigned int nw;              /* waves per workgroup (narrow kernel: 4 or 8) */
    unsigned int groups;          /* workgroups along n */
    unsigned int splits;          /* workgroups along k */
    unsigned int qps;             /* quads per split */
    /* batch rows */
    int xmode;
    const unsigned short *x;      /* AOTX_X_F16 */
    unsigned int ldx;
    const float *resid;           /* AOTX_X_NORM: [rows][k] */
    const float *norm_w;          /* [k] */
    const float *sumsq;           /* [rows][k/64] partial sums of squares */
    float eps;
    const unsigned int *xrow;     /* optional: batch row i reads row xrow[i] */
    unsigned int m;               /* rows when m_dev is null (also the pass capacity) */
    const unsigned int *m_dev;
    unsigned int m0;
    /* result */
    int epi;
    void *y;
    unsigned int ldy;
    float *partial;               /* splits > 1: [groups][splits][rt*16][MT] */
    unsigned int *count;          /* splits > 1: [experts][groups] arrivals, zero between launches */
    float *sumsq_out;             /* AOTX_EPI_RESID: [rows][n/16] sums of squares */
    unsigned short *xg_out;       /* AOTX_EPI_RESID, optional: fp16 resid * xg_w, [rows][n] */
    unsigned int out_frag;        /* xg_out, and SWIGLU's y, in the fragment layout */
    const float *xg_w;            /* the next norm's weights [n] */
    const float *row_ss;          /* optional (wide batches, direct rows): the rows' partial
                                     sums of squares [rows][k/16]; outputs are multiplied by
                                     rsqrt(sum / k + eps) (the RMSNorm scale of x) */
    float row_eps;
    aotx_qkv_epi qkv;
    /* routed experts (grid.y): as aotx_gemv_args */
    unsigned long long expert_stride;
    const unsigned int *list;
    const unsigned int *list_count;
    unsigned int list_cap;
    unsigned int xrow_div;
    unsigned int experts;
    /* wide products of direct rows: consecutive 32-row passes in one launch (grid.y is the
     * pass, rows m0 + 32 * pass on); 0 or 1 is one pass */
    unsigned int passes;
};

/* Plan a product over Q8R tensors; rows per segment; returns 1 when refused. mt is the
 * pass capacity: up to AOTX_NARROW_ROWS rows take the streaming kernel (which can stage x
 * as the RMSNorm of the residual stream), up to 32 the wide kernel, and up to
 * AOTX_RGEMM_ROWS the GEMM. */
#define AOTX_NARROW_ROWS 4u
#define AOTX_RGEMM_ROWS 512u
int aotx_rgemv_plan(aotx_rgemv_args *a, const void *const *w, const unsigned int *rows,
                    unsigned int nseg, unsigned int k, int epi, unsigned int mt);
/* The same for a routed-expert product (one workgroup row per expert, x rows through the
 * expert's row list): its wide passes may take larger tile groups. */
int aotx_rgemv_plan_routed(aotx_rgemv_args *a, const void *const *w, const unsigned int *rows,
                           unsigned int nseg, unsigned int k, int epi, unsigned int mt);
/* Plan a product whose x is in the fragment layout (AOTX_X_FRAG): a dense product of at
 * most 32 rows (one pass, m0 = 0) over tensors whose k is a multiple of 128; 1 when
 * refused. */
int aotx_rgemv_plan_frag(aotx_rgemv_args *a, const void *const *w, const unsigned int *rows,
                         unsigned int nseg, unsigned int k, int epi, unsigned int mt);
/* Launch one pass (<= 32 rows) and, with splits > 1, the kernel that adds the partials
 * and applies the epilogue. */
int aotx_rgemv_launch(const aotx_rgemv_args &a, hipStream_t stream);   /* 1 when refused */
size_t aotx_rgemv_partial_bytes(const aotx_rgemv_args &a);
/* The split arrival counters a plan needs (one per tile group and expert or row block). */
unsigned int aotx_rgemv_count_words(const aotx_rgemv_args &a);

#endif
