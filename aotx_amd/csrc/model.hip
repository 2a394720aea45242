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
 * graphs are captured on first use of a bucket and replayed after (AOTX_GRAPHS=0 launches
 * the same kernels eagerly).
 */
#include "aotx_internal.h"
#include "attention.h"
#include "experts.h"
#include "gemv.h"
#include "norm.h"
#include "sample.h"

#include <stdlib.h>
#include <string.h>

unsigned long long aotx_mem_weights_bytes(void);

#define AOTX_BUCKETS 10u   /* 1, 2, 4, ..., 512 */

struct aotx_hold {
    int ready;
    int described;
    aotx_model_desc desc;
    unsigned int role;
    unsigned int max_tokens;
    unsigned int max_rows;
    hipStream_t stream;
    aotx_step *pinned;
    aotx_step *step;              /* device copy */
    /* buffers */
    float *resid;
    unsigned short *x;
    unsigned short *qh;
    unsigned short *att;
    unsigned short *act;
    unsigned short *sel;
    float *qkv;                   /* fp32 QKV rows of the general path */
    float *logits;                /* [max_rows][vocab] */
    unsigned int *pos, *tagent, *last;
    float *gemv_partial;
    float *attn_partial;
    float *prob;
    unsigned int *ids;
    float *ey;
    unsigned short *eact;
    unsigned int *elist, *ecount;
    void *piece[32];
    unsigned int pieces;
    /* graphs per token bucket and head-row bucket */
    hipGraphExec_t exec[AOTX_BUCKETS][AOTX_BUCKETS];
    unsigned int nodes;
};

static aotx_hold aotx_holds[AOTX_MODEL_ROLES];

static int aotx_is_language(unsigned int role)
{
    return role == AOTX_MODEL_LANGUAGE || role == AOTX_MODEL_LANGUAGE_Q4
        || role == AOTX_MODEL_LANGUAGE_AUDIO;
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
    AOTX_CHECK(hipMalloc(&p, bytes));
    AOTX_CHECK(hipMemset(p, 0, bytes));
    if (h->pieces >= 32u) {
        fprintf(stderr, "aotx: too many buffers\n");
        exit(1);
    }
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

extern "C" int aotx_model_set_desc(unsigned int role, const aotx_model_desc *desc)
{
    if (role >= AOTX_MODEL_ROLES || desc == nullptr || !aotx_is_language(role)) return 1;
    if (!aotx_desc_ok(desc)) return 1;
    aotx_hold *h = &aotx_holds[role];
    if (h->ready) return 1;
    h->desc = *desc;
    h->desc.role = role;
    h->described = 1;
    return 0;
}

/* ---- planning helpers -------------------------------------------------------------- */

static aotx_gemv_args aotx_plan_or_die(const void *const *w, const unsigned int *rows,
                                       unsigned int nseg, unsigned int k, int epi)
{
    aotx_gemv_args a;
    if (aotx_gemv_plan(&a, w, rows, nseg, k, epi) != 0) {
        fprintf(stderr, "aotx: a product of the model was refused (k=%u)\n", k);
        exit(1);
    }
    return a;
}

/* One product of a step: row passes of 32 over the bucket; with one pass and a split k,
 * the partials may be left for the next kernel (defer). */
static void aotx_product(aotx_hold *h, aotx_gemv_args a, unsigned int bucket_rows,
                         const unsigned int *m_dev, int allow_defer, int *deferred)
{
    a.partial = h->gemv_partial;
    a.m_dev = m_dev;
    unsigned int passes = (bucket_rows + 31u) / 32u;
    *deferred = 0;
    for (unsigned int i = 0; i < passes; ++i) {
        aotx_gemv_args p = a;
        p.m0 = 32u * i;
        p.m = bucket_rows <= 16u ? 16u : 32u;
        p.defer = (allow_defer && passes == 1u && a.splits > 1u) ? 1 : 0;
        if (p.defer) *deferred = 1;
        aotx_gemv_launch(p, h->stream);
    }
}

/* ---- the step ---------------------------------------------------------------------- */

static void aotx_record_step(aotx_hold *h, unsigned int bt, unsigned int br)
{
    const aotx_model_desc *d = &h->desc;
    hipStream_t s = h->stream;
    const unsigned int T = 1u << bt;                 /* token capacity of this bucket */
    const unsigned int R = 1u << br;                 /* head rows capacity */
    const unsigned int *m_tokens = &h->step->run.tokens;
    const unsigned int *m_rows = &h->step->run.rows;
    const unsigned int hd = d->head_dim;
    const unsigned int wide = d->heads * hd, narrow = d->kv_heads * hd;
    const unsigned int mt = T <= 16u ? 16u : 32u;
    const aotx_kvl_shape shape = aotx_kvl_make(d->layers, d->kv_heads, hd);
    const unsigned int max_context = AOTX_SEQ_MAX_TOKENS;

    AOTX_CHECK(hipMemcpyAsync(h->step, h->pinned, sizeof(aotx_step), hipMemcpyHostToDevice, s));
    aotx_launch_rows(h->step, T, h->pos, h->tagent, h->last, s);
    aotx_launch_gather(h->step, T, aotx_tensor(d->token_embd), d->embd_type, d->hidden, d->vocab,
                       h->resid, h->x, (const float *)aotx_tensor(d->layer[0].offset[AOTX_SLOT_ATTN_NORM]),
                       d->rms_eps, s);
    for (unsigned int l = 0; l < d->layers; ++l) {
        const aotx_model_layer *L = &d->layer[l];
        int deferred = 0;
        /* attention half */
        const void *qkv_w[3] = {aotx_tensor(L->offset[AOTX_SLOT_ATTN_Q]),
                                aotx_tensor(L->offset[AOTX_SLOT_ATTN_K]),
                                aotx_tensor(L->offset[AOTX_SLOT_ATTN_V])};
        unsigned int qkv_rows[3] = {wide, narrow, narrow};
        if (aotx_fused_qkv(d, l)) {
            aotx_gemv_args a = aotx_plan_or_die(qkv_w, qkv_rows, 3u, d->hidden, AOTX_EPI_QKV);
            a.x = h->x;
            a.ldx = d->hidden;
            a.qkv.qh = h->qh;
            a.qkv.pos = h->pos;
            a.qkv.agent = h->tagent;
            a.qkv.state = aotx_state_device();
            a.qkv.shape = shape;
            a.qkv.layer = l;
            a.qkv.heads = d->heads;
            a.qkv.kv_heads = d->kv_heads;
            a.qkv.head_dim = hd;
            a.qkv.theta = d->rope_theta;
            a.qkv.factor = (const float *)aotx_tensor(d->rope_freqs);
            aotx_product(h, a, T, m_tokens, 0, &deferred);
        } else {
            aotx_gemv_args a = aotx_plan_or_die(qkv_w, qkv_rows, 3u, d->hidden, AOTX_EPI_F32);
            a.x = h->x;
            a.ldx = d->hidden;
            a.y = h->qkv;
            a.ldy = wide + 2u * narrow;
            aotx_product(h, a, T, m_tokens, 0, &deferred);
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
                               d->kv_heads, hd, l, d->layers, max_context, h->attn_partial, s) != 0) {
            fprintf(stderr, "aotx: attention refused the shape\n");
            exit(1);
        }
        const void *o_w[1] = {aotx_tensor(L->offset[AOTX_SLOT_ATTN_O])};
        unsigned int o_rows[1] = {d->hidden};
        aotx_gemv_args o = aotx_plan_or_die(o_w, o_rows, 1u, wide, AOTX_EPI_RESID);
        o.x = h->att;
        o.ldx = wide;
        o.y = h->resid;
        o.ldy = d->hidden;
        aotx_product(h, o, T, m_tokens, 1, &deferred);
        aotx_resid_norm_args rn;
        memset(&rn, 0, sizeof rn);
        rn.m_dev = m_tokens;
        rn.resid = h->resid;
        rn.x = h->x;
        rn.norm_w = (const float *)aotx_tensor(L->offset[AOTX_SLOT_FFN_NORM]);
        rn.eps = d->rms_eps;
        rn.hidden = d->hidden;
        if (deferred) {
            rn.partial = h->gemv_partial;
            rn.splits = o.splits;
            rn.mt = mt;
        }
        aotx_launch_resid_norm(rn, T, s);

        /* feed-forward half */
        aotx_resid_norm_args nx;
        memset(&nx, 0, sizeof nx);
        nx.m_dev = m_tokens;
        nx.resid = h->resid;
        nx.x = h->x;
        nx.eps = d->rms_eps;
        nx.hidden = d->hidden;
        if (d->kind[l] == AOTX_LAYER_KIND_FFN_EXPERTS) {
            aotx_launch_route((const float *)aotx_tensor(L->offset[AOTX_EXPERT_ROUTER]), h->x, m_tokens,
                              T, d->hidden, d->expert_count, d->expert_used_count, h->prob, h->ids, s);
            aotx_expert_plan p;
            p.gate = aotx_tensor(L->offset[AOTX_SLOT_FFN_GATE]);
            p.up = aotx_tensor(L->offset[AOTX_SLOT_FFN_UP]);
            p.down = aotx_tensor(L->offset[AOTX_SLOT_FFN_DOWN]);
            p.experts = d->expert_count;
            p.used = d->expert_used_count;
            p.hidden = d->hidden;
            p.ffn = d->ffn;
            p.list = h->elist;
            p.count = h->ecount;
            p.cap = h->max_tokens * d->expert_used_count;
            if (aotx_launch_expert_ffn(p, h->x, m_tokens, T, h->ids, h->eact, h->ey, s) != 0) {
                fprintf(stderr, "aotx: the expert products were refused\n");
                exit(1);
            }
            nx.expert_y = h->ey;
            nx.expert_prob = h->prob;
            nx.expert_ids = h->ids;
            nx.experts = d->expert_count;
            nx.used = d->expert_used_count;
        } else {
            const void *gu_w[2] = {aotx_tensor(L->offset[AOTX_SLOT_FFN_GATE]),
                                   aotx_tensor(L->offset[AOTX_SLOT_FFN_UP])};
            unsigned int gu_rows[2] = {d->ffn, d->ffn};
            aotx_gemv_args gu = aotx_plan_or_die(gu_w, gu_rows, 2u, d->hidden, AOTX_EPI_SWIGLU);
            gu.x = h->x;
            gu.ldx = d->hidden;
            gu.y = h->act;
            gu.ldy = d->ffn;
            aotx_product(h, gu, T, m_tokens, 0, &deferred);
            const void *dn_w[1] = {aotx_tensor(L->offset[AOTX_SLOT_FFN_DOWN])};
            unsigned int dn_rows[1] = {d->hidden};
            aotx_gemv_args dn = aotx_plan_or_die(dn_w, dn_rows, 1u, d->ffn, AOTX_EPI_RESID);
            dn.x = h->act;
            dn.ldx = d->ffn;
            dn.y = h->resid;
            dn.ldy = d->hidden;
            aotx_product(h, dn, T, m_tokens, 1, &deferred);
            if (deferred) {
                nx.partial = h->gemv_partial;
                nx.splits = dn.splits;
                nx.mt = mt;
            }
        }
        if (l + 1u < d->layers) {
            nx.norm_w = (const float *)aotx_tensor(d->layer[l + 1u].offset[AOTX_SLOT_ATTN_NORM]);
        } else {
            nx.norm_w = (const float *)aotx_tensor(d->output_norm);
            nx.sel = h->sel;
            nx.last = h->last;
            nx.step = h->step;
        }
        aotx_launch_resid_norm(nx, T, s);
    }
    /* output head on the selected rows, then the sampler */
    const unsigned long long head_off = d->tied_output ? d->token_embd : d->output;
    const void *hw[1] = {aotx_tensor(head_off)};
    unsigned int hrows[1] = {d->vocab};
    aotx_gemv_args hp = aotx_plan_or_die(hw, hrows, 1u, d->hidden, AOTX_EPI_F32);
    hp.x = h->sel;
    hp.ldx = d->hidden;
    hp.y = h->logits;
    hp.ldy = d->vocab;
    int deferred = 0;
    aotx_product(h, hp, R, m_rows, 0, &deferred);
    aotx_launch_pick(h->logits, d->vocab, d->vocab, m_rows, R, nullptr, nullptr, 0u, 1.0f, 0.0f,
                     0ull, nullptr, nullptr, &h->step->run, s);
    aotx_launch_shut_rows(h->step, s);
}

/* ---- lifecycle ----------------------------------------------------------------------- */

static int aotx_use_graphs(void)
{
    const char *v = getenv("AOTX_GRAPHS");
    return !(v != nullptr && v[0] == '0');
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
    h->x = (unsigned short *)aotx_take(h, T * (d->hidden > d->ffn ? d->hidden : d->ffn) * 2u);
    h->qh = (unsigned short *)aotx_take(h, T * wide * 2u);
    h->att = (unsigned short *)aotx_take(h, T * wide * 2u);
    h->act = (unsigned short *)aotx_take(h, T * d->ffn * 2u);
    h->sel = (unsigned short *)aotx_take(h, R * d->hidden * 2u);
    h->qkv = (float *)aotx_take(h, T * (wide + 2u * narrow) * 4u);
    h->logits = (float *)aotx_take(h, R * d->vocab * 4u);
    h->pos = (unsigned int *)aotx_take(h, T * 4u);
    h->tagent = (unsigned int *)aotx_take(h, T * 4u);
    h->last = (unsigned int *)aotx_take(h, AOTX_SLOTS * 4u);
    /* split partials: the largest product plan over every bucket */
    size_t gp = 0u;
    {
        const unsigned int ks[3] = {d->hidden, (unsigned int)wide, d->ffn};
        const unsigned int ns[4] = {(unsigned int)(wide + 2u * narrow), d->hidden, 2u * d->ffn, d->vocab};
        for (unsigned int i = 0; i < 3u; ++i) {
            for (unsigned int j = 0; j < 4u; ++j) {
                aotx_gemv_args a;
                const void *w[1] = {(const void *)1};
                unsigned int rows[1] = {ns[j]};
                if (aotx_gemv_plan(&a, w, rows, 1u, ks[i], AOTX_EPI_F32) == 0) {
                    size_t need = aotx_gemv_scratch_partial(a);
                    if (need > gp) gp = need;
                }
            }
        }
    }
    h->gemv_partial = (float *)aotx_take(h, gp + 4096u);
    size_t ap = 0u;
    for (unsigned int t = 1u; t <= cap; t <<= 1) {
        unsigned int sp = aotx_attn_splits(t, d->kv_heads, AOTX_SEQ_MAX_TOKENS);
        size_t need = aotx_attn_scratch(t, d->kv_heads, sp, d->heads / d->kv_heads, hd);
        if (need > ap) ap = need;
    }
    h->attn_partial = (float *)aotx_take(h, ap);
    if (d->expert_count != 0u) {
        size_t slots = T * d->expert_used_count;
        h->prob = (float *)aotx_take(h, T * d->expert_count * 4u);
        h->ids = (unsigned int *)aotx_take(h, slots * 4u);
        h->ey = (float *)aotx_take(h, slots * d->hidden * 4u);
        h->eact = (unsigned short *)aotx_take(h, slots * d->ffn * 2u);
        h->elist = (unsigned int *)aotx_take(h, (size_t)d->expert_count * slots * 4u);
        h->ecount = (unsigned int *)aotx_take(h, (size_t)d->expert_count * 4u);
    }
    AOTX_CHECK(hipHostMalloc((void **)&h->pinned, sizeof(aotx_step), hipHostMallocDefault));
    memset(h->pinned, 0, sizeof(aotx_step));
    h->step = (aotx_step *)aotx_take(h, sizeof(aotx_step));
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
    for (unsigned int i = 0; i < AOTX_BUCKETS; ++i)
        for (unsigned int j = 0; j < AOTX_BUCKETS; ++j)
            if (h->exec[i][j] != nullptr) AOTX_CHECK(hipGraphExecDestroy(h->exec[i][j]));
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
    AOTX_CHECK(hipStreamSynchronize(h->stream));
    return 0;
}

extern "C" int aotx_model_launch(unsigned int role, const aotx_model_run *set)
{
    if (role >= AOTX_MODEL_ROLES || set == nullptr) return 1;
    aotx_hold *h = &aotx_holds[role];
    if (!h->ready || set->tokens > h->max_tokens || set->rows > h->max_rows || set->seqs > AOTX_SLOTS)
        return 1;
    if (set->tokens == 0u || set->seqs == 0u || set->rows == 0u) return 1;
    if (set->pooled != nullptr || set->score != nullptr || set->capture != nullptr) return 1;
    if (set->token != nullptr && set->select != AOTX_MODEL_ROWS_LAST) return 1;
    if (set->select == AOTX_MODEL_ROWS_LAST && set->rows != set->seqs) return 1;
    if (set->select == AOTX_MODEL_ROWS_ALL && set->rows != set->tokens) return 1;
    h->pinned->run = *set;
    unsigned int bt = aotx_bucket_of(set->tokens);
    unsigned int br = aotx_bucket_of(set->rows);
    if (aotx_use_graphs()) {
        hipGraphExec_t &exec = h->exec[bt][br];
        if (exec == nullptr) {
            hipGraph_t graph = nullptr;
            AOTX_CHECK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
            aotx_record_step(h, bt, br);
            AOTX_CHECK(hipStreamEndCapture(h->stream, &graph));
            size_t count = 0;
            AOTX_CHECK(hipGraphGetNodes(graph, nullptr, &count));
            if ((unsigned int)count > h->nodes) h->nodes = (unsigned int)count;
            AOTX_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
            AOTX_CHECK(hipGraphDestroy(graph));
        }
        AOTX_CHECK(hipGraphLaunch(exec, h->stream));
    } else {
        aotx_record_step(h, bt, br);
    }
    if (set->logits != nullptr) {
        AOTX_CHECK(hipMemcpyAsync(set->logits, h->logits,
                                  (size_t)set->rows * h->desc.vocab * sizeof(float),
                                  hipMemcpyDeviceToDevice, h->stream));
    }
    AOTX_CHECK(hipStreamSynchronize(h->stream));
    return 0;
}

/* The call block of one pass (call_host.cu:14-38): the offsets come back from the device
 * and every sequence must hold a token. */
static int aotx_call_set(aotx_model_run *set, const int *ids, const unsigned int *offset,
                         unsigned int seqs, const unsigned int *agent)
{
    unsigned int rows[AOTX_SLOTS + 1u];
    memset(set, 0, sizeof *set);
    if (seqs == 0u || seqs > AOTX_SLOTS || ids == nullptr || offset == nullptr || agent == nullptr) {
        fprintf(stderr, "a pass of %u sequences is outside the bounds\n", seqs);
        return 1;
    }
    AOTX_CHECK(hipMemcpy(rows, offset, (seqs + 1u) * sizeof *rows, hipMemcpyDeviceToHost));
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
    case 0: return (unsigned long long)h->x;        /* last norm output, fp16 */
    case 1: return (unsigned long long)h->resid;    /* residual stream, fp32 */
    case 2: return (unsigned long long)h->logits;   /* head rows, fp32 */
    case 3: return (unsigned long long)h->sel;      /* head input rows, fp16 */
    default: return 0ull;
    }
}
