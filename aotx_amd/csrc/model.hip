/* The model-step operator surface: buffers, the per-layer kernel sequence, graph capture
 * and the synchronous launch.
 *
 * Reference: cuda/model/model_host.cu (open :95-153, launch :155-200, pages :202-220,
 * forget :222-231, restream :233-240, faulted :252-258, shut :260-286),
 * cuda/model/call_host.cu (sample :71-93, prefill :40-56, probe :95-117) and the per-layer
 * capture of cuda/model/graph_host.cu:52-153 and experts_host.cu:65-114.
 *
 * Per step (decode or prefill chunk) the stream runs:
 *   call block H2D -> rows -> gather + first norm ->
 *   per layer: QKV product (+ rotary turn + page write fused for the adjacent-pair
 *     layer kind, else fp32 QKV + turn kernel) -> attention (+ chunk merge) ->
 *     O product (+ residual, or split partials added by the next kernel) ->
 *     residual + FFN norm -> gate/up product with SwiGLU (or router + grouped experts) ->
 *     down product -> residual + next norm (the last one also selects the head rows) ->
 *   head product -> sampler -> cache positions advance.
 * The reference launches ~14 kernels per layer; this sequence launches 6-7.
 *
 * Every kernel reads the batch from the device copy of the call block, so one captured
 * graph serves every call whose token count fits its bucket (1, 2, 4, ..., max_tokens);
 * graphs are captured on first use of a bucket and replayed after (aotx_model_graphs(0)
 * records a fresh graph for every call instead).
 */
#include "aotx_internal.h"
#include "../../include/aotx_plan.h"
#include "attention.h"
#include "experts.h"
#include "gemv.h"
#include "norm.h"
#include "rgemv.h"
#include "sample.h"
#include "tick.h"

#include <stdlib.h>
#include <string.h>

unsigned long long aotx_mem_weights_bytes(void);

#define AOTX_BUCKETS 10u   /* 1, 2, 4, ..., 512 */
#define AOTX_WIDE_PASSES 4u        /* 32-row passes of a wide product in one launch */
#define AOTX_GEMV_COUNTS 65536u   /* split arrival counters: experts x product groups */
#define AOTX_PIECES 48u            /* device buffers of one role */

/* The operands of a decode tick; a tick graph is captured for one set of them. */
struct aotx_tick_setup {
    const aotx_plan_slot *slots;
    int *tokens;
    unsigned int stride;
    unsigned int budget;
    unsigned int pool_pages;
    aotx_plan_state *plan;
    aotx_token_record *records;
    unsigned int capacity;
    float *logits;
};

/* Repacked (Q8R) copies of one layer's matrices; the library owns them. */
struct aotx_rlayer {
    const unsigned char *q, *k, *v, *o, *gate, *up, *down;
};

struct aotx_hold {
    int ready;
    int record_failed;      /* a launch of the step being recorded was refused */
    int take_failed;        /* open ran out of buffer places */
    int described;
    aotx_model_desc desc;
    unsigned int role;
    unsigned int max_tokens;
    unsigned int max_rows;
    hipStream_t stream;
    aotx_step *pinned;
    aotx_step *step;              /* device copy */
    /* repacked weights */
    unsigned char *rw;
    aotx_rlayer rl[AOTX_MODEL_MAX_LAYERS];
    const unsigned char *rhead;
    /* buffers */
    float *resid;
    float *sumsq;                 /* [tokens][hidden/16] */
    unsigned short *x;
    unsigned short *qh;
    unsigned short *att;
    unsigned short *act;
    unsigned short *sel;
    float *qkv;                   /* fp32 QKV rows of the general path */
    float *logits;                /* [max_rows][vocab] */
    unsigned int *pick_best;      /* the sampler's buffer (aotx_pick_scratch) */
    unsigned int *pos, *tagent, *last;
    float *gemv_partial;
    size_t gemv_partial_bytes;
    unsigned int *gemv_count;     /* split arrivals per product group, zero between launches */
    float *attn_partial;
    unsigned int *attn_count;     /* chunk arrivals per (token, KV head), zero between launches */
    float *prob;
    unsigned int *ids;
    float *ey;
    unsigned short *eact;
    unsigned int *elist, *ecount;
    void *piece[AOTX_PIECES];
    unsigned int pieces;
    /* the decode tick (aotx_decode_tick): the step's outputs, the sampler's adjustment
     * scratch, and one graph per token bucket with the operands it was captured for */
    int *tick_token;
    unsigned int *tick_draw;
    unsigned int *pen_count, *pen_last;
    float *pen_raw;
    aotx_tick_setup tick_setup[AOTX_BUCKETS];
    hipGraphExec_t tick_exec[AOTX_BUCKETS];
    /* graphs per residual capture (probe calls that ask for it), row selection, token
     * bucket and head-row bucket */
    hipGraphExec_t exec[2][2][AOTX_BUCKETS][AOTX_BUCKETS];
    unsigned int nodes;
};

static aotx_hold aotx_holds[AOTX_MODEL_ROLES];

static int aotx_is_language(unsigned int role)
{
    return role == AOTX_MODEL_LANGUAGE || role == AOTX_MODEL_LANGUAGE_Q4
        || role == AOTX_MODEL_LANGUAGE_AUDIO;
}

/* The roles whose passes end in a head of their own instead of the vocabulary head. */
static int aotx_is_head_role(unsigned int role)
{
    return role == AOTX_MODEL_EMBEDDING || role == AOTX_MODEL_RERANKER;
}

static const unsigned char *aotx_tensor(unsigned long long off)
{
    if (off == AOTX_MODEL_ABSENT) return nullptr;
    return (const unsigned char *)(aotx_mem_weights_base() + off);
}

static unsigned int aotx_bucket_of(unsigned int n)
{
    unsigned int b = 0u;
    while ((1u << b) < n) ++b;
    return b;
}

static void *aotx_take(aotx_hold *h, size_t bytes)
{
    void *p = nullptr;
    if (bytes == 0u) bytes = 256u;
    if (h->pieces >= AOTX_PIECES) {
        /* open checks the flag and refuses */
        fprintf(stderr, "aotx: a role holds at most %u buffers\n", AOTX_PIECES);
        h->take_failed = 1;
        return nullptr;
    }
    AOTX_CHECK(hipMalloc(&p, bytes));
    AOTX_CHECK(hipMemset(p, 0, bytes));
    h->piece[h->pieces++] = p;
    return p;
}

/* A layer may take the fused rotary/page-write epilogue: no head norm, adjacent pairs. */
static int aotx_fused_qkv(const aotx_model_desc *d, unsigned int l)
{
    if (d->rope_pairs != AOTX_ROPE_PAIRS_ADJACENT) return 0;
    if (d->kind[l] == AOTX_LAYER_KIND_ATTENTION) return 0;
    if ((d->heads * d->head_dim) % 64u != 0u || (d->kv_heads * d->head_dim) % 64u != 0u) return 0;
    return 1;
}

static int aotx_desc_ok(const aotx_model_desc *d)
{
    if (d->layers == 0u || d->layers > AOTX_MODEL_MAX_LAYERS || d->hidden == 0u) return 0;
    if (d->hidden % 64u != 0u || d->ffn % 32u != 0u || d->ffn == 0u) return 0;
    if (d->head_dim != 64u && d->head_dim != 128u) return 0;
    if (d->kv_heads == 0u || d->heads % d->kv_heads != 0u) return 0;
    unsigned int g = d->heads / d->kv_heads;
    if (g != 1u && g != 2u && g != 4u && g != 8u) return 0;
    if ((d->heads * d->head_dim) % 32u != 0u) return 0;
    if (d->embd_type != AOTX_WEIGHT_Q8_0 && d->embd_type != AOTX_WEIGHT_F16
        && d->embd_type != AOTX_WEIGHT_F32)
        return 0;
    if (d->tied_output && d->embd_type != AOTX_WEIGHT_Q8_0) return 0;
    if (d->token_embd == AOTX_MODEL_ABSENT || d->output_norm == AOTX_MODEL_ABSENT) return 0;
    if (!d->tied_output && d->output == AOTX_MODEL_ABSENT) return 0;
    aotx_kvl_shape shape = aotx_kvl_make(d->layers, d->kv_heads, d->head_dim);
    if (shape.blocks_page == 0u) return 0;
    for (unsigned int l = 0; l < d->layers; ++l) {
        unsigned int kind = d->kind[l];
        if (kind != AOTX_LAYER_KIND_ATTENTION && kind != AOTX_LAYER_KIND_ATTENTION_NO_QK_NORM
            && kind != AOTX_LAYER_KIND_FFN_EXPERTS)
            return 0;
        const aotx_model_layer *L = &d->layer[l];
        const unsigned int mats[] = {AOTX_SLOT_ATTN_Q, AOTX_SLOT_ATTN_K, AOTX_SLOT_ATTN_V,
                                     AOTX_SLOT_ATTN_O, AOTX_SLOT_FFN_GATE, AOTX_SLOT_FFN_UP,
                                     AOTX_SLOT_FFN_DOWN};
        for (unsigned int i = 0; i < 7u; ++i) {
            if (L->offset[mats[i]] == AOTX_MODEL_ABSENT) return 0;
            if (d->layer_type[l][mats[i]] != AOTX_WEIGHT_Q8_0) return 0;
        }
        if (L->offset[AOTX_SLOT_ATTN_NORM] == AOTX_MODEL_ABSENT
            || L->offset[AOTX_SLOT_FFN_NORM] == AOTX_MODEL_ABSENT)
            return 0;
        if (kind == AOTX_LAYER_KIND_ATTENTION
            && (L->offset[AOTX_ATTENTION_Q_NORM] == AOTX_MODEL_ABSENT
                || L->offset[AOTX_ATTENTION_K_NORM] == AOTX_MODEL_ABSENT))
            return 0;
        if (kind == AOTX_LAYER_KIND_FFN_EXPERTS) {
            if (d->expert_count == 0u || d->expert_count > AOTX_LAYER_EXPERTS_MAX
                || d->expert_used_count == 0u || d->expert_used_count > d->expert_count
                || L->offset[AOTX_EXPERT_ROUTER] == AOTX_MODEL_ABSENT)
                return 0;
        }
    }
    return 1;
}

int aotx_role_kv_shape(unsigned int role, aotx_kvl_shape *out)
{
    if (role >= AOTX_MODEL_ROLES || !aotx_holds[role].described) return 1;
    const aotx_model_desc *d = &aotx_holds[role].desc;
    *out = aotx_kvl_make(d->layers, d->kv_heads, d->head_dim);
    return 0;
}

extern "C" unsigned int aotx_model_kv_pages(unsigned int role, unsigned int context)
{
    aotx_kvl_shape shape;
    if (aotx_role_kv_shape(role, &shape) != 0) return 0u;
    return aotx_kvl_pages(shape, context);
}

extern "C" int aotx_model_set_desc(unsigned int role, const aotx_model_desc *desc)
{
    if (role >= AOTX_MODEL_ROLES || desc == nullptr
        || (!aotx_is_language(role) && !aotx_is_head_role(role)))
        return 1;
    if (!aotx_desc_ok(desc)) return 1;
    aotx_hold *h = &aotx_holds[role];
    if (h->ready) return 1;
    h->desc = *desc;
    h->desc.role = role;
    h->described = 1;
    return 0;
}

/* ---- planning helpers -------------------------------------------------------------- */

static void aotx_roperands(aotx_rgemv_args *p, const aotx_rgemv_args &tmpl);

/* One product of a step over repacked weights, in passes of at most 32 batch rows; a
 * batch of at most 16 rows may stage x from the residual stream (norm fused). */
static void aotx_rproduct(aotx_hold *h, const void *const *w, const unsigned int *rows,
                          unsigned int nseg, unsigned int k, int epi, unsigned int cap,
                          const unsigned int *m_dev, const aotx_rgemv_args &tmpl)
{
    /* 128 rows or more of a dense product: one GEMM pass (up to 512 rows; 128-token prompt
     * 10.15 -> 8.49 ms against passes of 32 rows, while at 64 rows its few workgroups are
     * slower than re-reading the weights per 32 rows: the Mixtral-shape step 17.2 -> 19.3
     * ms); routed experts keep passes of 32 rows through their row lists */
    const bool gemm = cap >= 128u && tmpl.expert_stride == 0ull && tmpl.list == nullptr
                   && tmpl.xrow == nullptr && tmpl.xmode == AOTX_X_F16;
    for (unsigned int m0 = 0, mt = 0; m0 < cap; m0 += mt) {
        mt = gemm ? (cap - m0 < AOTX_RGEMM_ROWS ? cap - m0 : AOTX_RGEMM_ROWS)
                  : (cap - m0 < 32u ? cap - m0 : 32u);
        aotx_rgemv_args a;
        const int refused = tmpl.xmode == AOTX_X_FRAG
            ? aotx_rgemv_plan_frag(&a, w, rows, nseg, k, epi, mt)
            : tmpl.expert_stride != 0ull ? aotx_rgemv_plan_routed(&a, w, rows, nseg, k, epi, mt)
                                         : aotx_rgemv_plan(&a, w, rows, nseg, k, epi, mt);
        if (refused != 0) {
            fprintf(stderr, "aotx: a product of the model was refused (k=%u)\n", k);
            h->record_failed = 1;
            return;
        }
        aotx_roperands(&a, tmpl);
        a.m_dev = m_dev;
        a.m0 = m0;
        /* whole 32-row passes of a wide product over direct rows run as one launch (grid.y
         * is the pass): one launch's ramp and tail instead of one per pass */
        if (!gemm && a.wide && mt == 32u && cap - m0 >= 64u && tmpl.expert_stride == 0ull
            && tmpl.list == nullptr && tmpl.xrow == nullptr) {
            a.passes = (cap - m0) / 32u;
            if (a.passes > AOTX_WIDE_PASSES) a.passes = AOTX_WIDE_PASSES;
            mt = 32u * a.passes;
        }
        if (a.splits > 1u) {
            size_t need = aotx_rgemv_partial_bytes(a);
            if (need > h->gemv_partial_bytes) {
                fprintf(stderr, "aotx: split partials exceed the planned buffer\n");
                h->record_failed = 1;
                return;
            }
            a.partial = h->gemv_partial;
            if (aotx_rgemv_count_words(a) > AOTX_GEMV_COUNTS) {
                fprintf(stderr, "aotx: split counters exceed the planned buffer\n");
                h->record_failed = 1;
                return;
            }
            a.count = h->gemv_count;
        }
        if (aotx_rgemv_launch(a, h->stream) != 0) {
            h->record_failed = 1;
            return;
        }
    }
}

/* The call's operands over a plan. */
static void aotx_roperands(aotx_rgemv_args *p, const aotx_rgemv_args &tmpl)
{
    aotx_rgemv_args &a = *p;
    {
        a.xmode = tmpl.xmode;
        a.x = tmpl.x;
        a.ldx = tmpl.ldx;
        a.resid = tmpl.resid;
        a.norm_w = tmpl.norm_w;
        a.sumsq = tmpl.sumsq;
        a.eps = tmpl.eps;
        a.xrow = tmpl.xrow;
        a.y = tmpl.y;
        a.ldy = tmpl.ldy;
        a.sumsq_out = tmpl.sumsq_out;
        a.xg_out = tmpl.xg_out;
        a.xg_w = tmpl.xg_w;
        a.out_frag = tmpl.out_frag;
        a.row_ss = tmpl.row_ss;
        a.row_eps = tmpl.row_eps;
        a.qkv = tmpl.qkv;
        a.expert_stride = tmpl.expert_stride;
        a.list = tmpl.list;
        a.list_count = tmpl.list_count;
        a.list_cap = tmpl.list_cap;
        a.xrow_div = tmpl.xrow_div;
        a.experts = tmpl.experts;
    }
}

/* ---- the step ---------------------------------------------------------------------- */

/* Records one step on h->stream. A refused launch sets h->record_failed and ends the
 * recording at once; the callers record under stream capture and then drop the graph, so
 * nothing of a refused step runs. capture: the probe's residual rows after every layer. */
static void aotx_record_step(aotx_hold *h, unsigned int sel_all, unsigned int bt, unsigned int br,
                             const aotx_tick_setup *tk, bool capture)
{
    (void)sel_all;    /* the head's rows are selected on the device from the call block */
    const aotx_model_desc *d = &h->desc;
    hipStream_t s = h->stream;
    const unsigned int T = 1u << bt;                 /* token capacity of this bucket */
    const unsigned int R = 1u << br;                 /* head rows capacity */
    const unsigned int *m_tokens = &h->step->run.tokens;
    const unsigned int *m_rows = &h->step->run.rows;
    const unsigned int hd = d->head_dim;
    const unsigned int wide = d->heads * hd, narrow = d->kv_heads * hd;
    const aotx_kvl_shape shape = aotx_kvl_make(d->layers, d->kv_heads, hd);
    const unsigned int max_context = AOTX_SEQ_MAX_TOKENS;
    const bool fused_norm = T <= AOTX_NARROW_ROWS;   /* x staged from the residual stream */
    const bool experts = d->expert_count != 0u;
    /* wide batches of a dense model: the residual epilogue that ends each half also writes
     * x = half(resid * w) for the next norm's weights w, and the next product multiplies its
     * outputs by the rows' RMSNorm scale, so no norm kernel runs between them */
    const bool scaled_x = !fused_norm && !experts;
    /* and up to 32 rows, when every width is a multiple of 128: the x of QKV (the first
     * norm's and the down products' output) and of O (the attention's) are written in the
     * fragment layout and read by the fragment product, whose waves load their MFMA
     * operands straight from it; gate/up and down keep the wide kernel, measured faster
     * there */
    const bool frag_dims = d->hidden % 128u == 0u && wide % 128u == 0u && d->ffn % 128u == 0u;
    const bool frag = scaled_x && T <= AOTX_XFRAG_ROWS && frag_dims;
    const int xmode_in = frag ? AOTX_X_FRAG : AOTX_X_F16;

    if (tk != nullptr) {
        /* the tick: the plan packs the batch on the device and the call block points at it */
        if (aotx_plan_launch(h->role, tk->slots, tk->tokens, tk->stride, tk->budget,
                             tk->pool_pages, tk->plan, s) != 0) {
            fprintf(stderr, "aotx: the tick plan was refused\n");
            h->record_failed = 1;
            return;
        }
        aotx_launch_tick_begin(h->step, tk->plan, h->tick_token, h->tick_draw, s);
    } else {
        AOTX_CHECK(hipMemcpyAsync(h->step, h->pinned, sizeof(aotx_step), hipMemcpyHostToDevice, s));
    }
    aotx_launch_rows(h->step, T, h->pos, h->tagent, h->last, s);
    aotx_launch_gather(h->step, T, aotx_tensor(d->token_embd), d->embd_type, d->hidden, d->vocab,
                       h->resid, h->sumsq, s);

    aotx_norm_args nrm;
    memset(&nrm, 0, sizeof nrm);
    nrm.m_dev = m_tokens;
    nrm.resid = h->resid;
    nrm.sumsq = h->sumsq;
    nrm.eps = d->rms_eps;
    nrm.hidden = d->hidden;
    nrm.x = h->x;
    nrm.x_frag = frag ? 1u : 0u;

    for (unsigned int l = 0; l < d->layers; ++l) {
        const aotx_model_layer *L = &d->layer[l];
        const aotx_rlayer *RL = &h->rl[l];
        const float *attn_w = (const float *)aotx_tensor(L->offset[AOTX_SLOT_ATTN_NORM]);
        const float *ffn_w = (const float *)aotx_tensor(L->offset[AOTX_SLOT_FFN_NORM]);

        /* ---- attention half ---- */
        aotx_rgemv_args x_in;
        memset(&x_in, 0, sizeof x_in);
        if (fused_norm) {
            x_in.xmode = AOTX_X_NORM;
            x_in.resid = h->resid;
            x_in.norm_w = attn_w;
            x_in.sumsq = h->sumsq;
            x_in.eps = d->rms_eps;
        } else {
            if (!scaled_x || l == 0u) {
                nrm.norm_w = attn_w;
                aotx_launch_norm(nrm, T, s);
            } else {
                x_in.row_ss = h->sumsq;          /* x = half(resid * attn_w) from the down product */
                x_in.row_eps = d->rms_eps;
            }
            x_in.xmode = xmode_in;
            x_in.x = h->x;
            x_in.ldx = d->hidden;
        }
        const void *qkv_w[3] = {RL->q, RL->k, RL->v};
        unsigned int qkv_rows[3] = {wide, narrow, narrow};
        if (aotx_fused_qkv(d, l)) {
            aotx_rgemv_args t = x_in;
            t.qkv.qh = h->qh;
            t.qkv.pos = h->pos;
            t.qkv.agent = h->tagent;
            t.qkv.state = aotx_state_device();
            t.qkv.shape = shape;
            t.qkv.layer = l;
            t.qkv.heads = d->heads;
            t.qkv.kv_heads = d->kv_heads;
            t.qkv.head_dim = hd;
            t.qkv.theta = d->rope_theta;
            t.qkv.factor = (const float *)aotx_tensor(d->rope_freqs);
            aotx_rproduct(h, qkv_w, qkv_rows, 3u, d->hidden, AOTX_EPI_QKV, T, m_tokens, t);
            if (h->record_failed) return;
        } else {
            aotx_rgemv_args t = x_in;
            t.y = h->qkv;
            t.ldy = wide + 2u * narrow;
            aotx_rproduct(h, qkv_w, qkv_rows, 3u, d->hidden, AOTX_EPI_F32, T, m_tokens, t);
            if (h->record_failed) return;
            aotx_rope_args r;
            memset(&r, 0, sizeof r);
            r.m_dev = m_tokens;
            r.q = h->qkv;
            r.k = h->qkv + wide;
            r.v = h->qkv + wide + narrow;
            r.ld = wide + 2u * narrow;
            r.qh = h->qh;
            r.pos = h->pos;
            r.agent = h->tagent;
            if (d->kind[l] == AOTX_LAYER_KIND_ATTENTION) {
                r.q_norm = (const float *)aotx_tensor(L->offset[AOTX_ATTENTION_Q_NORM]);
                r.k_norm = (const float *)aotx_tensor(L->offset[AOTX_ATTENTION_K_NORM]);
            }
            r.factor = (const float *)aotx_tensor(d->rope_freqs);
            r.eps = d->rms_eps;
            r.theta = d->rope_theta;
            r.heads = d->heads;
            r.kv_heads = d->kv_heads;
            r.head_dim = hd;
            r.pairs = d->rope_pairs;
            r.layer = l;
            r.shape = shape;
            r.state = aotx_state_device();
            aotx_launch_rope(r, T, s);
        }
        if (aotx_attend_launch(h->qh, h->att, h->pos, h->tagent, m_tokens, T, d->heads,
                               d->kv_heads, hd, l, d->layers, max_context, h->attn_partial,
                               h->attn_count, s, frag ? 1u : 0u) != 0) {
            fprintf(stderr, "aotx: attention refused the shape\n");
            h->record_failed = 1;
            return;
        }
        {
            aotx_rgemv_args t;
            memset(&t, 0, sizeof t);
            t.xmode = xmode_in;              /* the attention's output */
            t.x = h->att;
            t.ldx = wide;
            t.y = h->resid;
            t.ldy = d->hidden;
            t.sumsq_out = h->sumsq;
            if (scaled_x) {
                t.xg_out = h->x;                 /* gate/up's x: row layout */
                t.xg_w = ffn_w;
            }
            const void *o_w[1] = {RL->o};
            unsigned int o_rows[1] = {d->hidden};
            aotx_rproduct(h, o_w, o_rows, 1u, wide, AOTX_EPI_RESID, T, m_tokens, t);
            if (h->record_failed) return;
        }

        /* ---- feed-forward half ---- */
        if (experts) {
            nrm.norm_w = ffn_w;
            aotx_launch_norm(nrm, T, s);
            aotx_launch_route((const float *)aotx_tensor(L->offset[AOTX_EXPERT_ROUTER]), h->x, m_tokens,
                              T, d->hidden, d->expert_count, d->expert_used_count, h->prob, h->ids, s);
            const unsigned int used = d->expert_used_count;
            const unsigned int cap = h->max_tokens * used;
            aotx_launch_group(h->ids, m_tokens, T, used, d->expert_count, h->elist, h->ecount, cap, s);
            aotx_rgemv_args t;
            memset(&t, 0, sizeof t);
            t.xmode = AOTX_X_F16;
            t.x = h->x;
            t.ldx = d->hidden;
            t.y = h->eact;
            t.ldy = d->ffn;
            t.expert_stride = aotx_q8r_bytes(d->ffn, d->hidden);
            t.list = h->elist;
            t.list_count = h->ecount;
            t.list_cap = cap;
            t.xrow_div = used;
            t.experts = d->expert_count;
            const void *gu_w[2] = {RL->gate, RL->up};
            unsigned int gu_rows[2] = {d->ffn, d->ffn};
            /* an expert takes at most every token once */
            aotx_rproduct(h, gu_w, gu_rows, 2u, d->hidden, AOTX_EPI_SWIGLU, T, nullptr, t);
            if (h->record_failed) return;
            aotx_rgemv_args u = t;
            u.x = h->eact;
            u.ldx = d->ffn;
            u.y = h->ey;
            u.ldy = d->hidden;
            u.expert_stride = aotx_q8r_bytes(d->hidden, d->ffn);
            u.xrow_div = 1u;
            const void *dn_w[1] = {RL->down};
            unsigned int dn_rows[1] = {d->hidden};
            aotx_rproduct(h, dn_w, dn_rows, 1u, d->ffn, AOTX_EPI_F32, T, nullptr, u);
            if (h->record_failed) return;
            aotx_expert_resid_args er;
            er.m_dev = m_tokens;
            er.resid = h->resid;
            er.sumsq = h->sumsq;
            er.y = h->ey;
            er.prob = h->prob;
            er.ids = h->ids;
            er.experts = d->expert_count;
            er.used = used;
            er.hidden = d->hidden;
            aotx_launch_expert_resid(er, T, s);
        } else {
            aotx_rgemv_args t;
            memset(&t, 0, sizeof t);
            if (fused_norm) {
                t.xmode = AOTX_X_NORM;
                t.resid = h->resid;
                t.norm_w = ffn_w;
                t.sumsq = h->sumsq;
                t.eps = d->rms_eps;
            } else {
                t.xmode = AOTX_X_F16;
                t.x = h->x;                      /* half(resid * ffn_w) from the O product */
                t.ldx = d->hidden;
                t.row_ss = h->sumsq;
                t.row_eps = d->rms_eps;
            }
            t.y = h->act;
            t.ldy = d->ffn;
            const void *gu_w[2] = {RL->gate, RL->up};
            unsigned int gu_rows[2] = {d->ffn, d->ffn};
            aotx_rproduct(h, gu_w, gu_rows, 2u, d->hidden, AOTX_EPI_SWIGLU, T, m_tokens, t);
            if (h->record_failed) return;
            aotx_rgemv_args u;
            memset(&u, 0, sizeof u);
            u.xmode = AOTX_X_F16;
            u.x = h->act;
            u.ldx = d->ffn;
            u.y = h->resid;
            u.ldy = d->hidden;
            u.sumsq_out = h->sumsq;
            if (scaled_x && l + 1u < d->layers) {
                u.xg_out = h->x;
                u.xg_w = (const float *)aotx_tensor(d->layer[l + 1u].offset[AOTX_SLOT_ATTN_NORM]);
                u.out_frag = frag ? 1u : 0u;
            }
            const void *dn_w[1] = {RL->down};
            unsigned int dn_rows[1] = {d->hidden};
            aotx_rproduct(h, dn_w, dn_rows, 1u, d->ffn, AOTX_EPI_RESID, T, m_tokens, u);
            if (h->record_failed) return;
        }
        if (capture) aotx_launch_capture(h->step, h->resid, d->hidden, l, s);
    }
    /* the embedding and rank roles end in their own heads over each sequence's last row
     * (cuda/model/graph_host.cu:115-126) */
    if (aotx_is_head_role(h->role)) {
        const float *out_w = (const float *)aotx_tensor(d->output_norm);
        if (h->role == AOTX_MODEL_EMBEDDING)
            aotx_launch_pool(h->step, h->resid, out_w, d->hidden, d->rms_eps, s);
        else
            aotx_launch_score(h->step, h->resid, out_w, aotx_tensor(d->cls_output), d->weight_type,
                              d->hidden, d->rms_eps, s);
        aotx_launch_shut_rows(h->step, s);
        return;
    }
    /* output head on the selected rows (each sequence's last token, or every token) */
    {
        aotx_rgemv_args t;
        memset(&t, 0, sizeof t);
        /* the selected rows normalised once by a norm kernel: the head has thousands of
         * workgroups, and staging the norm in each costs more than the launch */
        const float *out_w = (const float *)aotx_tensor(d->output_norm);
        {
            aotx_norm_args on = nrm;
            on.norm_w = out_w;
            on.x = nullptr;
            on.x_frag = 0u;
            on.sel = h->sel;
            on.last = h->last;
            on.step = h->step;
            aotx_launch_norm(on, T, s);
            /* the head's rows as plain fp16 for the wide kernel (5-32 rows: 1002 workgroups
             * of 8 tiles with x through LDS measured 15 us faster per batch-32 step than the
             * fragment product's 2004 of 4 tiles) */
            t.xmode = AOTX_X_F16;
            t.x = h->sel;
            t.ldx = d->hidden;
        }
        t.y = h->logits;
        t.ldy = d->vocab;
        const void *hw[1] = {h->rhead};
        unsigned int hrows[1] = {d->vocab};
        aotx_rproduct(h, hw, hrows, 1u, d->hidden, AOTX_EPI_F32, R, m_rows, t);
        if (h->record_failed) return;
    }
    aotx_pen_args pen;
    if (tk != nullptr) {
        /* the sample's penalties over each sequence's list, around the pick */
        pen.step = h->step;
        pen.slots = tk->slots;
        pen.tokens = tk->tokens;
        pen.stride = tk->stride;
        pen.logits = h->logits;
        pen.ld = d->vocab;
        pen.vocab = d->vocab;
        pen.count = h->pen_count;
        pen.last = h->pen_last;
        pen.raw = h->pen_raw;
        aotx_launch_pen(pen, R, 0, s);
    }
    aotx_launch_pick(h->logits, d->vocab, d->vocab, m_rows, R, nullptr, nullptr, 0u, 1.0f, 0.0f,
                     0ull, nullptr, nullptr, &h->step->run, h->pick_best, s);
    if (tk != nullptr) {
        aotx_launch_pen(pen, R, 1, s);
        if (tk->logits != nullptr)
            AOTX_CHECK(hipMemcpyAsync(tk->logits, h->logits, (size_t)R * d->vocab * sizeof(float),
                                      hipMemcpyDeviceToDevice, s));
    }
    aotx_launch_shut_rows(h->step, s);
    if (tk != nullptr
        && aotx_commit_launch(h->role, (aotx_plan_slot *)tk->slots, tk->tokens, tk->stride,
                              h->tick_token, h->tick_draw, tk->plan, tk->records, tk->capacity,
                              s) != 0) {
        fprintf(stderr, "aotx: the tick commit was refused\n");
        h->record_failed = 1;
        return;
    }
}

/* ---- lifecycle ----------------------------------------------------------------------- */

/* Keep each bucket's recorded graph for the calls after (1, the default), or record a
 * fresh graph for every call (0, aotx_model_graphs). */
static int aotx_graph_cache = 1;

extern "C" void aotx_model_graphs(unsigned int keep)
{
    aotx_graph_cache = keep != 0u ? 1 : 0;
}

extern "C" int aotx_model_open(unsigned int role, unsigned int max_tokens)
{
    if (role >= AOTX_MODEL_ROLES || max_tokens == 0u || max_tokens > AOTX_MODEL_MAX_TOKENS) return 1;
    aotx_hold *h = &aotx_holds[role];
    if (!h->described || h->ready) return 1;
    if (aotx_mem_weights_base() == 0ull) {
        fprintf(stderr, "aotx: no weights region\n");
        return 1;
    }
    const aotx_model_desc *d = &h->desc;
    if (role == AOTX_MODEL_RERANKER
        && (d->cls_output == AOTX_MODEL_ABSENT
            || (d->weight_type != AOTX_WEIGHT_Q8_0 && d->weight_type != AOTX_WEIGHT_F16
                && d->weight_type != AOTX_WEIGHT_F32))) {
        fprintf(stderr, "aotx: the rank role needs a class head of Q8_0, F16 or F32\n");
        return 1;
    }
    aotx_gemv_init();
    aotx_state_device();
    /* the token capacity is a power of two, so every bucket of a call fits */
    unsigned int cap = 1u;
    while (cap < max_tokens) cap <<= 1;
    h->max_tokens = cap;
    h->max_rows = cap > AOTX_SLOTS ? cap : AOTX_SLOTS;
    h->role = role;
    const size_t T = cap, R = h->max_rows;
    const unsigned int hd = d->head_dim;
    const size_t wide = (size_t)d->heads * hd, narrow = (size_t)d->kv_heads * hd;
    h->resid = (float *)aotx_take(h, T * d->hidden * 4u);
    h->sumsq = (float *)aotx_take(h, T * ((d->hidden + 15u) / 16u) * 4u);
    /* x, att and act hold 32 rows at least: the fragment layout of 5..32-row buckets */
    const size_t TF = T > AOTX_XFRAG_ROWS ? T : AOTX_XFRAG_ROWS;
    h->x = (unsigned short *)aotx_take(h, TF * d->hidden * 2u);
    h->qh = (unsigned short *)aotx_take(h, T * wide * 2u);
    h->att = (unsigned short *)aotx_take(h, TF * wide * 2u);
    h->act = (unsigned short *)aotx_take(h, TF * d->ffn * 2u);
    h->sel = (unsigned short *)aotx_take(h, R * d->hidden * 2u);
    h->qkv = (float *)aotx_take(h, T * (wide + 2u * narrow) * 4u);
    h->logits = (float *)aotx_take(h, R * d->vocab * 4u);
    h->pick_best = (unsigned int *)aotx_take(h, aotx_pick_scratch(R, d->vocab));
    h->pos = (unsigned int *)aotx_take(h, T * 4u);
    h->tagent = (unsigned int *)aotx_take(h, T * 4u);
    h->last = (unsigned int *)aotx_take(h, AOTX_SLOTS * 4u);

    /* repacked copies of every matrix (the same bytes per weight, MFMA operand order) */
    const unsigned int E = d->expert_count != 0u ? d->expert_count : 1u;
    const unsigned long long bq = aotx_q8r_bytes((unsigned int)wide, d->hidden);
    const unsigned long long bk = aotx_q8r_bytes((unsigned int)narrow, d->hidden);
    const unsigned long long bo = aotx_q8r_bytes(d->hidden, (unsigned int)wide);
    const unsigned long long bg = aotx_q8r_bytes(d->ffn, d->hidden);
    const unsigned long long bd = aotx_q8r_bytes(d->hidden, d->ffn);
    const unsigned long long per_layer = bq + 2ull * bk + bo + E * (2ull * bg + bd);
    const unsigned long long bh = aotx_q8r_bytes(d->vocab, d->hidden);
    const unsigned long long total = per_layer * d->layers + bh;
    h->rw = (unsigned char *)aotx_take(h, (size_t)total);
    {
        unsigned char *at = h->rw;
        const unsigned long long src_g = (unsigned long long)d->ffn * (d->hidden / 32u) * 34ull;
        const unsigned long long src_d = (unsigned long long)d->hidden * (d->ffn / 32u) * 34ull;
        for (unsigned int l = 0; l < d->layers; ++l) {
            const aotx_model_layer *L = &d->layer[l];
            aotx_rlayer *RL = &h->rl[l];
            aotx_q8r_repack(aotx_tensor(L->offset[AOTX_SLOT_ATTN_Q]), (unsigned int)wide, d->hidden, at, nullptr);
            RL->q = at; at += bq;
            aotx_q8r_repack(aotx_tensor(L->offset[AOTX_SLOT_ATTN_K]), (unsigned int)narrow, d->hidden, at, nullptr);
            RL->k = at; at += bk;
            aotx_q8r_repack(aotx_tensor(L->offset[AOTX_SLOT_ATTN_V]), (unsigned int)narrow, d->hidden, at, nullptr);
            RL->v = at; at += bk;
            aotx_q8r_repack(aotx_tensor(L->offset[AOTX_SLOT_ATTN_O]), d->hidden, (unsigned int)wide, at, nullptr);
            RL->o = at; at += bo;
            RL->gate = at;
            for (unsigned int e = 0; e < E; ++e, at += bg)
                aotx_q8r_repack(aotx_tensor(L->offset[AOTX_SLOT_FFN_GATE]) + e * src_g, d->ffn, d->hidden, at, nullptr);
            RL->up = at;
            for (unsigned int e = 0; e < E; ++e, at += bg)
                aotx_q8r_repack(aotx_tensor(L->offset[AOTX_SLOT_FFN_UP]) + e * src_g, d->ffn, d->hidden, at, nullptr);
            RL->down = at;
            for (unsigned int e = 0; e < E; ++e, at += bd)
                aotx_q8r_repack(aotx_tensor(L->offset[AOTX_SLOT_FFN_DOWN]) + e * src_d, d->hidden, d->ffn, at, nullptr);
        }
        const unsigned long long head_off = d->tied_output ? d->token_embd : d->output;
        aotx_q8r_repack(aotx_tensor(head_off), d->vocab, d->hidden, at, nullptr);
        h->rhead = at;
        AOTX_CHECK(hipDeviceSynchronize());
    }

    /* split partials: the largest plan over every product and batch capacity */
    size_t gp = 0u;
    {
        const void *w1[1] = {(const void *)1};
        const void *w2[2] = {(const void *)1, (const void *)1};
        const void *w3[3] = {(const void *)1, (const void *)1, (const void *)1};
        for (unsigned int mt = 1u; mt <= 32u; ++mt) {
            aotx_rgemv_args a;
            unsigned int r3[3] = {(unsigned int)wide, (unsigned int)narrow, (unsigned int)narrow};
            if (aotx_rgemv_plan(&a, w3, r3, 3u, d->hidden, AOTX_EPI_F32, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            unsigned int r1[1] = {d->hidden};
            if (aotx_rgemv_plan(&a, w1, r1, 1u, (unsigned int)wide, AOTX_EPI_RESID, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if ((d->expert_count != 0u ? aotx_rgemv_plan_routed(&a, w1, r1, 1u, d->ffn, AOTX_EPI_RESID, mt)
                                       : aotx_rgemv_plan(&a, w1, r1, 1u, d->ffn, AOTX_EPI_RESID, mt)) == 0) {
                a.expert_stride = d->expert_count != 0u ? 1ull : 0ull;
                a.experts = E;
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            }
            unsigned int r2[2] = {d->ffn, d->ffn};
            if ((d->expert_count != 0u ? aotx_rgemv_plan_routed(&a, w2, r2, 2u, d->hidden, AOTX_EPI_SWIGLU, mt)
                                       : aotx_rgemv_plan(&a, w2, r2, 2u, d->hidden, AOTX_EPI_SWIGLU, mt)) == 0) {
                a.expert_stride = d->expert_count != 0u ? 1ull : 0ull;
                a.experts = E;
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            }
            unsigned int rv[1] = {d->vocab};
            if (aotx_rgemv_plan(&a, w1, rv, 1u, d->hidden, AOTX_EPI_F32, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            /* the fragment products of the same shapes */
            if (aotx_rgemv_plan_frag(&a, w3, r3, 3u, d->hidden, AOTX_EPI_F32, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if (aotx_rgemv_plan_frag(&a, w1, r1, 1u, (unsigned int)wide, AOTX_EPI_RESID, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if (aotx_rgemv_plan_frag(&a, w1, r1, 1u, d->ffn, AOTX_EPI_RESID, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if (aotx_rgemv_plan_frag(&a, w2, r2, 2u, d->hidden, AOTX_EPI_SWIGLU, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if (aotx_rgemv_plan_frag(&a, w1, rv, 1u, d->hidden, AOTX_EPI_F32, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
        }
        /* the GEMM passes (256 rows and more) of the dense products */
        for (unsigned int mt = 64u; mt <= AOTX_RGEMM_ROWS && mt <= cap; mt += 64u) {
            aotx_rgemv_args a;
            unsigned int r3[3] = {(unsigned int)wide, (unsigned int)narrow, (unsigned int)narrow};
            unsigned int r1[1] = {d->hidden};
            unsigned int r2[2] = {d->ffn, d->ffn};
            if (aotx_rgemv_plan(&a, w3, r3, 3u, d->hidden, AOTX_EPI_F32, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if (aotx_rgemv_plan(&a, w1, r1, 1u, (unsigned int)wide, AOTX_EPI_RESID, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if (aotx_rgemv_plan(&a, w1, r1, 1u, d->ffn, AOTX_EPI_RESID, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
            if (aotx_rgemv_plan(&a, w2, r2, 2u, d->hidden, AOTX_EPI_SWIGLU, mt) == 0)
                gp = gp > aotx_rgemv_partial_bytes(a) ? gp : aotx_rgemv_partial_bytes(a);
        }
    }
    h->gemv_partial_bytes = gp * AOTX_WIDE_PASSES + 4096u;   /* passes in one launch */
    h->gemv_partial = (float *)aotx_take(h, h->gemv_partial_bytes);
    h->gemv_count = (unsigned int *)aotx_take(h, AOTX_GEMV_COUNTS * sizeof(unsigned int));
    size_t ap = 0u;
    for (unsigned int t = 1u; t <= cap; t <<= 1) {
        unsigned int sp = aotx_attn_splits(t, d->kv_heads, AOTX_SEQ_MAX_TOKENS);
        size_t need = aotx_attn_scratch(t, d->kv_heads, sp, d->heads / d->kv_heads, hd);
        if (need > ap) ap = need;
    }
    h->attn_partial = (float *)aotx_take(h, ap);
    h->attn_count = (unsigned int *)aotx_take(h, (size_t)T * d->kv_heads * 4u);
    if (d->expert_count != 0u) {
        size_t slots = T * d->expert_used_count;
        h->prob = (float *)aotx_take(h, T * d->expert_count * 4u);
        h->ids = (unsigned int *)aotx_take(h, slots * 4u);
        h->ey = (float *)aotx_take(h, slots * d->hidden * 4u);
        h->eact = (unsigned short *)aotx_take(h, slots * d->ffn * 2u);
        h->elist = (unsigned int *)aotx_take(h, (size_t)d->expert_count * slots * 4u);
        h->ecount = (unsigned int *)aotx_take(h, (size_t)d->expert_count * 4u);
    }
    h->step = (aotx_step *)aotx_take(h, sizeof(aotx_step));
    if (h->take_failed) {
        for (unsigned int i = 0; i < h->pieces; ++i) AOTX_CHECK(hipFree(h->piece[i]));
        aotx_model_desc keep = h->desc;
        memset(h, 0, sizeof *h);
        h->desc = keep;
        h->described = 1;
        return 1;
    }
    AOTX_CHECK(hipHostMalloc((void **)&h->pinned, sizeof(aotx_step), hipHostMallocDefault));
    memset(h->pinned, 0, sizeof(aotx_step));
    AOTX_CHECK(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking));
    AOTX_CHECK(hipDeviceSynchronize());
    h->ready = 1;
    return 0;
}

extern "C" void aotx_model_shut(unsigned int role)
{
    if (role >= AOTX_MODEL_ROLES) return;
    aotx_hold *h = &aotx_holds[role];
    if (!h->ready) return;
    AOTX_CHECK(hipStreamSynchronize(h->stream));
    for (unsigned int c = 0; c < 2u; ++c)
        for (unsigned int a = 0; a < 2u; ++a)
            for (unsigned int i = 0; i < AOTX_BUCKETS; ++i)
                for (unsigned int j = 0; j < AOTX_BUCKETS; ++j)
                    if (h->exec[c][a][i][j] != nullptr)
                        AOTX_CHECK(hipGraphExecDestroy(h->exec[c][a][i][j]));
    for (unsigned int i = 0; i < AOTX_BUCKETS; ++i)
        if (h->tick_exec[i] != nullptr) AOTX_CHECK(hipGraphExecDestroy(h->tick_exec[i]));
    AOTX_CHECK(hipStreamDestroy(h->stream));
    AOTX_CHECK(hipHostFree(h->pinned));
    for (unsigned int i = 0; i < h->pieces; ++i) AOTX_CHECK(hipFree(h->piece[i]));
    aotx_model_desc keep = h->desc;
    int described = h->described;
    memset(h, 0, sizeof *h);
    h->desc = keep;
    h->described = described;
}

extern "C" void aotx_model_forget(void)
{
    aotx_state *st = aotx_state_device();
    AOTX_CHECK(hipDeviceSynchronize());
    AOTX_CHECK(hipMemset(st->seen, 0, sizeof st->seen));
    AOTX_CHECK(hipMemset(&st->faults, 0, sizeof st->faults));
    AOTX_CHECK(hipDeviceSynchronize());
}

extern "C" void aotx_model_restream(void)
{
    aotx_state *st = aotx_state_device();
    AOTX_CHECK(hipDeviceSynchronize());
    AOTX_CHECK(hipMemset(st->draw, 0, sizeof st->draw));
    AOTX_CHECK(hipDeviceSynchronize());
}

extern "C" int aotx_model_seat(unsigned int agent, unsigned int position)
{
    if (agent >= AOTX_SLOTS || position > AOTX_SEQ_MAX_TOKENS) return 1;
    aotx_state *st = aotx_state_device();
    AOTX_CHECK(hipDeviceSynchronize());
    AOTX_CHECK(hipMemcpy(&st->seen[agent], &position, sizeof position, hipMemcpyHostToDevice));
    return 0;
}

extern "C" unsigned int aotx_model_faulted(void)
{
    unsigned int count = 0u;
    AOTX_CHECK(hipDeviceSynchronize());
    AOTX_CHECK(hipMemcpy(&count, &aotx_state_device()->faults, sizeof count, hipMemcpyDeviceToHost));
    return count;
}

extern "C" unsigned int aotx_model_nodes(unsigned int role)
{
    if (role >= AOTX_MODEL_ROLES) return 0u;
    return aotx_holds[role].nodes;
}

extern "C" int aotx_model_pages(unsigned int role, const unsigned int *offset, unsigned int seqs,
                                const unsigned int *agent)
{
    if (role >= AOTX_MODEL_ROLES) return 1;
    aotx_hold *h = &aotx_holds[role];
    if (!h->ready || seqs > AOTX_SLOTS || offset == nullptr || agent == nullptr) return 1;
    if (seqs == 0u) return 0;
    const aotx_model_desc *d = &h->desc;
    aotx_launch_request(offset, agent, seqs, aotx_kvl_make(d->layers, d->kv_heads, d->head_dim),
                        h->stream);
    aotx_wait(h->stream);
    return 0;
}

extern "C" int aotx_model_launch(unsigned int role, const aotx_model_run *set)
{
    if (role >= AOTX_MODEL_ROLES || set == nullptr) return 1;
    aotx_hold *h = &aotx_holds[role];
    if (!h->ready || set->tokens > h->max_tokens || set->rows > h->max_rows || set->seqs > AOTX_SLOTS)
        return 1;
    if (set->tokens == 0u || set->seqs == 0u || set->rows == 0u) return 1;
    /* residual capture: up to one slot per layer, the layer list in device memory; pooled
     * and score are written by the embedding and rank roles' heads (other roles leave them
     * untouched, as the reference's graphs do) */
    if (set->capture != nullptr && set->capture_count != 0u
        && (set->capture_count > AOTX_MODEL_MAX_LAYERS || set->capture_layer == nullptr))
        return 1;
    if (set->token != nullptr && set->select != AOTX_MODEL_ROWS_LAST) return 1;
    if (set->token != nullptr && aotx_is_head_role(role)) return 1;   /* no sampler there */
    if (set->select == AOTX_MODEL_ROWS_LAST && set->rows != set->seqs) return 1;
    if (set->select == AOTX_MODEL_ROWS_ALL && set->rows != set->tokens) return 1;
    h->pinned->run = *set;
    const unsigned int cap = set->capture != nullptr && set->capture_count != 0u ? 1u : 0u;
    unsigned int bt = aotx_bucket_of(set->tokens);
    unsigned int br = aotx_bucket_of(set->rows);
    unsigned int all = set->select == AOTX_MODEL_ROWS_ALL ? 1u : 0u;
    hipGraphExec_t &exec = h->exec[cap][all][bt][br];
    if (exec == nullptr) {
        /* recorded under stream capture: a refused launch leaves a graph that is dropped,
         * so nothing of the step runs */
        hipGraph_t graph = nullptr;
        AOTX_CHECK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
        h->record_failed = 0;
        aotx_record_step(h, all, bt, br, nullptr, cap != 0u);
        AOTX_CHECK(hipStreamEndCapture(h->stream, &graph));
        if (h->record_failed) {
            AOTX_CHECK(hipGraphDestroy(graph));
            return 1;
        }
        size_t count = 0;
        AOTX_CHECK(hipGraphGetNodes(graph, nullptr, &count));
        if ((unsigned int)count > h->nodes) h->nodes = (unsigned int)count;
        AOTX_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        AOTX_CHECK(hipGraphDestroy(graph));
    }
    AOTX_CHECK(hipGraphLaunch(exec, h->stream));
    hipGraphExec_t drop = nullptr;        /* dropped once the call has waited for it */
    if (!aotx_graph_cache) {
        drop = exec;
        exec = nullptr;
    }
    if (set->logits != nullptr && !aotx_is_head_role(role)) {
        AOTX_CHECK(hipMemcpyAsync(set->logits, h->logits,
                                  (size_t)set->rows * h->desc.vocab * sizeof(float),
                                  hipMemcpyDeviceToDevice, h->stream));
    }
    aotx_wait(h->stream);
    if (drop != nullptr) AOTX_CHECK(hipGraphExecDestroy(drop));
    return 0;
}

/* One decode tick as one graph (cuda/model/decode_host.cu:136-157): plan -> the step over
 * the plan's batch, each row sampled with its sequence's own sample and penalties -> commit.
 * The graph of a token bucket (the bucket of `budget`) is captured on first use and again
 * when the operands change. */
extern "C" int aotx_decode_tick(unsigned int role, aotx_plan_slot *slots, int *tokens,
                                unsigned int stride, unsigned int budget, unsigned int pool_pages,
                                aotx_plan_state *plan, aotx_token_record *records,
                                unsigned int capacity, float *logits)
{
    if (role >= AOTX_MODEL_ROLES || slots == nullptr || tokens == nullptr || plan == nullptr
        || stride == 0u || (records == nullptr && capacity != 0u)
        || aotx_is_head_role(role))
        return 1;
    aotx_hold *h = &aotx_holds[role];
    if (!h->ready) return 1;
    if (budget > AOTX_SEQ_TICK_BUDGET) budget = AOTX_SEQ_TICK_BUDGET;
    if (budget == 0u || budget > h->max_tokens) return 1;
    const aotx_model_desc *d = &h->desc;
    if (h->tick_token == nullptr) {
        h->tick_token = (int *)aotx_take(h, AOTX_SLOTS * sizeof(int));
        h->tick_draw = (unsigned int *)aotx_take(h, AOTX_SLOTS * sizeof(unsigned int));
        const size_t cells = (size_t)AOTX_SLOTS * d->vocab;
        h->pen_count = (unsigned int *)aotx_take(h, cells * sizeof(unsigned int));
        h->pen_last = (unsigned int *)aotx_take(h, cells * sizeof(unsigned int));
        h->pen_raw = (float *)aotx_take(h, cells * sizeof(float));
    }
    const unsigned int bt = aotx_bucket_of(budget);
    const unsigned int T = 1u << bt;
    const unsigned int br = aotx_bucket_of(T < AOTX_SLOTS ? T : AOTX_SLOTS);
    aotx_tick_setup tk;
    memset(&tk, 0, sizeof tk);
    tk.slots = slots;
    tk.tokens = tokens;
    tk.stride = stride;
    tk.budget = budget;
    tk.pool_pages = pool_pages;
    tk.plan = plan;
    tk.records = records;
    tk.capacity = capacity;
    tk.logits = logits;
    hipGraphExec_t &exec = h->tick_exec[bt];
    if (exec != nullptr && memcmp(&h->tick_setup[bt], &tk, sizeof tk) != 0) {
        AOTX_CHECK(hipGraphExecDestroy(exec));
        exec = nullptr;
    }
    if (exec == nullptr) {
        hipGraph_t graph = nullptr;
        AOTX_CHECK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
        h->record_failed = 0;
        aotx_record_step(h, 0u, bt, br, &tk, false);
        AOTX_CHECK(hipStreamEndCapture(h->stream, &graph));
        if (h->record_failed) {
            AOTX_CHECK(hipGraphDestroy(graph));
            return 1;
        }
        AOTX_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        AOTX_CHECK(hipGraphDestroy(graph));
        h->tick_setup[bt] = tk;
    }
    AOTX_CHECK(hipGraphLaunch(exec, h->stream));
    aotx_wait(h->stream);
    return 0;
}

/* The call block of one pass (call_host.cu:14-38): the offsets come back from the device
 * and every sequence must hold a token. */
static int aotx_call_set(aotx_model_run *set, const int *ids, const unsigned int *offset,
                         unsigned int seqs, const unsigned int *agent)
{
    unsigned int *rows = (unsigned int *)aotx_pinned();
    memset(set, 0, sizeof *set);
    if (seqs == 0u || seqs > AOTX_SLOTS || ids == nullptr || offset == nullptr || agent == nullptr) {
        fprintf(stderr, "a pass of %u sequences is outside the bounds\n", seqs);
        return 1;
    }
    AOTX_CHECK(hipMemcpyAsync(rows, offset, (seqs + 1u) * sizeof *rows, hipMemcpyDeviceToHost,
                              nullptr));
    aotx_wait(nullptr);
    for (unsigned int s = 0u; s < seqs; ++s) {
        if (rows[s + 1u] <= rows[s]) {
            fprintf(stderr, "the sequence %u of the pass holds no token\n", s);
            return 1;
        }
    }
    if (rows[0] != 0u) return 1;
    set->ids = ids;
    set->offset = offset;
    set->agent = agent;
    set->seqs = seqs;
    set->tokens = rows[seqs];
    set->top_p = 1.0f;
    return 0;
}

extern "C" int aotx_model_sample(unsigned int role, const int *ids, const unsigned int *offset,
                                 unsigned int seqs, const unsigned int *agent,
                                 const aotx_model_how *how, int *token, unsigned int *draw,
                                 unsigned long long *seed)
{
    aotx_model_run set;
    if (how == nullptr || aotx_call_set(&set, ids, offset, seqs, agent) != 0) return 1;
    set.token = token;
    set.draw = draw;
    set.select = AOTX_MODEL_ROWS_LAST;
    set.rows = seqs;
    set.seed = how->seed;
    set.top_k = how->top_k;
    set.top_p = how->top_p;
    set.temperature = how->temperature;
    int state = aotx_model_launch(role, &set);
    if (state == 0 && seed != nullptr) *seed = how->seed;
    return state;
}

/* The rank role's pass (call_host.cu:58-69): the score of each sequence from its last
 * row. */
extern "C" int aotx_model_rerank(const int *ids, const unsigned int *offset, unsigned int seqs,
                                 const unsigned int *agent, float *score)
{
    aotx_model_run set;
    if (aotx_call_set(&set, ids, offset, seqs, agent) != 0) return 1;
    set.score = score;
    set.select = AOTX_MODEL_ROWS_LAST;
    set.rows = seqs;
    return aotx_model_launch(AOTX_MODEL_RERANKER, &set);
}

extern "C" int aotx_model_prefill(unsigned int role, const int *ids, const unsigned int *offset,
                                  unsigned int seqs, const unsigned int *agent, float *logits,
                                  float *pooled)
{
    aotx_model_run set;
    if (aotx_call_set(&set, ids, offset, seqs, agent) != 0) return 1;
    set.logits = logits;
    set.pooled = pooled;
    set.select = logits != nullptr ? AOTX_MODEL_ROWS_ALL : AOTX_MODEL_ROWS_LAST;
    set.rows = set.select == AOTX_MODEL_ROWS_ALL ? set.tokens : seqs;
    return aotx_model_launch(role, &set);
}

extern "C" int aotx_model_probe(unsigned int role, const int *ids, const unsigned int *offset,
                                unsigned int seqs, const unsigned int *agent,
                                const aotx_model_how *how, float *logits, unsigned int select,
                                float *capture, const unsigned int *layers,
                                unsigned int layer_count)
{
    aotx_model_run set;
    if (aotx_call_set(&set, ids, offset, seqs, agent) != 0 || layer_count > AOTX_MODEL_MAX_LAYERS)
        return 1;
    set.logits = logits;
    set.select = (logits != nullptr && select == AOTX_MODEL_ROWS_ALL) ? AOTX_MODEL_ROWS_ALL
                                                                     : AOTX_MODEL_ROWS_LAST;
    set.rows = set.select == AOTX_MODEL_ROWS_ALL ? set.tokens : seqs;
    set.how = how;
    set.capture = capture;
    set.capture_layer = layers;
    set.capture_count = layer_count;
    set.telemetry = 1u;
    return aotx_model_launch(role, &set);
}

extern "C" unsigned long long aotx_model_buffer(unsigned int role, unsigned int which)
{
    if (role >= AOTX_MODEL_ROLES || !aotx_holds[role].ready) return 0ull;
    const aotx_hold *h = &aotx_holds[role];
    switch (which) {
    /* x and sel of a 5..32-row bucket are in the fragment layout (aotx_xfrag_at) */
    case 0: return (unsigned long long)h->x;        /* last norm output, fp16 */
    case 1: return (unsigned long long)h->resid;    /* residual stream, fp32 */
    case 2: return (unsigned long long)h->logits;   /* head rows, fp32 */
    case 3: return (unsigned long long)h->sel;      /* head input rows, fp16 */
    /* routed experts, the last layer of the last pass (null without experts) */
    case 4: return (unsigned long long)h->ecount;   /* rows per expert, u32 [experts] */
    case 5: return (unsigned long long)h->ids;      /* experts of each token, u32 [T][used] */
    case 6: return (unsigned long long)h->prob;     /* router probabilities, f32 [T][experts] */
    default: return 0ull;
    }
}
