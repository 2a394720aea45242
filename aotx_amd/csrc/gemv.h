/* Q8_0 matrix product for a small batch of activation rows: host-side plan and launch.
 *
 * The kernel (gemv.hip) computes y[m][n] = sum_k x[m][k] * w[n][k] for up to three
 * weight tensors stacked along n, with one of several epilogues fused in: fp32 store,
 * fp16 store, residual add, gated unit (SwiGLU), and the rotary turn with the key/value
 * page write. When the k range is split over workgroups, the partial tiles are added in
 * split order by a second kernel (or by the consumer when `defer` is set). Replaces the reference's aotx_gemv_pass / aotx_gemm_tile and the kernels
 * that follow them in the captured graph (cuda/model/gemv.cuh:33-195,
 * cuda/model/gemm.cuh:55-189, cuda/model/norm.cu:79-105, cuda/model/rope.cu:200-234). */
#ifndef AOTX_GEMV_H
#define AOTX_GEMV_H

#include "aotx_internal.h"

enum {
    AOTX_EPI_F32 = 0,     /* y fp32 [m][ldy] */
    AOTX_EPI_F16 = 1,     /* y fp16 [m][ldy] */
    AOTX_EPI_RESID = 2,   /* y fp32 [m][ldy] += result */
    AOTX_EPI_SWIGLU = 3,  /* segments 0/1 = gate/up; y fp16 act [m][ldy] */
    AOTX_EPI_QKV = 4      /* segments q/k/v; adjacent rotary pairs; qh + pages */
};

/* Rotary + page-write parameters of AOTX_EPI_QKV. */
struct aotx_qkv_epi {
    unsigned short *qh;          /* fp16 [tokens][heads*d] */
    const unsigned int *pos;     /* cache position of each token */
    const unsigned int *agent;   /* slot of each token */
    aotx_state *state;           /* page table + fault count */
    aotx_kvl_shape shape;
    unsigned int layer;
    unsigned int heads;
    unsigned int kv_heads;
    unsigned int head_dim;
    float theta;
    const float *factor;         /* optional rope frequency factors [d/2] */
};

struct aotx_gemv_args {
    const unsigned char *w[3];   /* Q8_0 tensors, row-major [rows][k/32 blocks] */
    unsigned int seg_end[3];     /* cumulative virtual row ends */
    unsigned int nseg;
    unsigned int n;              /* virtual rows (SWIGLU: rows of one of the pair) */
    unsigned int k;
    unsigned long long row_bytes;
    unsigned int cb;             /* blocks of 32 per chunk */
    unsigned int chunks;         /* k / 32 / cb */
    unsigned int cps;            /* chunks per split */
    unsigned int splits;
    unsigned int groups;         /* 64-row groups */
    const unsigned short *x;     /* fp16 [rows][ldx] */
    unsigned int ldx;
    unsigned int m;              /* rows of x when m_dev is null */
    const unsigned int *m_dev;   /* device row count (call block); rows = *m_dev - m0 */
    unsigned int m0;             /* first row of x and y of this pass */
    int epi;
    void *y;
    unsigned int ldy;
    float *partial;              /* [groups][splits][64][MT]; null = library scratch */
    int defer;                   /* 1: a later kernel adds the split partials */
    aotx_qkv_epi qkv;
    /* Routed experts (grid.y = expert): the weights of expert e start e * expert_stride
     * bytes after w[seg]; the batch rows of expert e are list[e * list_cap + i] for
     * i < list_count[e] (slot = token * used + rank); x row = slot / xrow_div; the
     * result row is the slot. Zero expert_stride = a plain product. */
    unsigned long long expert_stride;
    const unsigned int *list;
    const unsigned int *list_count;
    unsigned int list_cap;
    unsigned int xrow_div;
    unsigned int experts;
};

/* Fill the plan of one product. Returns 1 when the shape is refused. */
int aotx_gemv_plan(aotx_gemv_args *a, const void *const *w, const unsigned int *rows,
                   unsigned int nseg, unsigned int k, int epi);

/* Launch the product on rows [m0, m0 + mt) of x, mt <= 32; m is the host row count or
 * the device count at m_dev. Scratch comes from the library. */
int aotx_gemv_launch(aotx_gemv_args a, hipStream_t stream);    /* 1 when refused */

/* Raise the LDS limit of the kernels (once; outside any stream capture). */
void aotx_gemv_init(void);

/* Scratch bytes a planned product needs (partials, counters). */
size_t aotx_gemv_scratch_partial(const aotx_gemv_args &a);

/* The product for any row count: passes of 32 rows. */
int aotx_gemv_run(aotx_gemv_args a, unsigned int m, hipStream_t stream);

#endif
