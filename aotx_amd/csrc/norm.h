/* Row kernels of the step (norm.hip): shared argument blocks and launchers. */
#ifndef AOTX_NORM_H
#define AOTX_NORM_H

#include "aotx_internal.h"

/* The device copy of one pass's call block (cuda/model/forward.cuh:122-147, :159). The
 * graph copies the host block in before its first kernel, so every kernel of a replayed
 * graph reads the batch of the current call. */
struct aotx_step {
    aotx_model_run run;
};

struct aotx_norm_args {
    const unsigned int *m_dev;    /* token count */
    const float *resid;           /* [tokens][hidden] */
    const float *sumsq;           /* [tokens][hidden/16] */
    const float *norm_w;
    float eps;
    unsigned int hidden;
    unsigned short *x;            /* out [tokens][hidden], or null */
    unsigned short *sel;          /* head rows, or null */
    const unsigned int *last;     /* last token row of each sequence */
    const aotx_step *step;        /* seqs and row selection of the call */
    unsigned int x_frag;          /* x in the fragment layout (aotx_xfrag_at) */
};

struct aotx_expert_resid_args {
    const unsigned int *m_dev;
    float *resid;
    float *sumsq;
    const float *y;               /* [tokens*used][hidden] */
    const float *prob;            /* [tokens][experts] */
    const unsigned int *ids;      /* [tokens][used] */
    unsigned int experts, used, hidden;
};

struct aotx_rope_args {
    const unsigned int *m_dev;
    const float *q, *k, *v;       /* fp32 rows: q[t*ld + h*d], k/v[t*ld + kh*d] */
    unsigned int ld;
    unsigned short *qh;
    const unsigned int *pos, *agent;
    const float *q_norm, *k_norm; /* per-head norm weights, or null */
    const float *factor;          /* rope frequency factors or null */
    float eps, theta;
    unsigned int heads, kv_heads, head_dim, pairs, layer;
    aotx_kvl_shape shape;
    aotx_state *state;
};

void aotx_launch_rows(const aotx_step *step, unsigned int max_tokens, unsigned int *pos,
                      unsigned int *tagent, unsigned int *last, hipStream_t s);
void aotx_launch_shut_rows(const aotx_step *step, hipStream_t s);
void aotx_launch_request(const unsigned int *offset, const unsigned int *agent,
                         unsigned int seqs, aotx_kvl_shape shape, hipStream_t s);
void aotx_launch_gather(const aotx_step *step, unsigned int max_tokens,
                        const unsigned char *table, unsigned int embd_type,
                        unsigned int hidden, unsigned int vocab, float *resid, float *sumsq,
                        hipStream_t s);
void aotx_launch_norm(const aotx_norm_args &a, unsigned int max_tokens, hipStream_t s);
void aotx_launch_expert_resid(const aotx_expert_resid_args &a, unsigned int max_tokens,
                              hipStream_t s);
void aotx_launch_rope(const aotx_rope_args &a, unsigned int max_tokens, hipStream_t s);
/* the probe's residual capture after one layer; the embedding and rank heads */
void aotx_launch_capture(const aotx_step *step, const float *resid, unsigned int hidden,
                         unsigned int layer, hipStream_t s);
void aotx_launch_pool(const aotx_step *step, const float *resid, const float *norm_w,
                      unsigned int hidden, float eps, hipStream_t s);
void aotx_launch_score(const aotx_step *step, const float *resid, const float *norm_w,
                       const unsigned char *cls, unsigned int type, unsigned int hidden,
                       float eps, hipStream_t s);

#endif
