/* CPU oracle of the AOTX-1 token loop — TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Built with -ffp-contract=off so that every float expression rounds as written. */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------
 * fp16, round to nearest even (the conversion __float2half performs).
 * ---------------------------------------------------------------------------------- */
uint16_t orc_f32_to_f16(float f)
{
    union { float f; uint32_t u; } v = { f };
    uint32_t sign = (v.u >> 16) & 0x8000u;
    uint32_t mag = v.u & 0x7FFFFFFFu;
    if (mag >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (mag > 0x7F800000u ? 0x200u : 0u));
    if (mag >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (mag < 0x38800000u) {
        /* subnormal result: round mag * 2^24 to an integer count of 2^-24 */
        double scaled = (double)v.f * 16777216.0;
        if (scaled < 0) scaled = -scaled;
        double r = nearbyint(scaled);   /* ties to even under the default mode */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t h = (mag >> 13) - (112u << 10);
    uint32_t rem = mag & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    float v;
    if (e == 0u) v = (float)m * (1.0f / 16777216.0f);
    else if (e == 31u) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400u), (int)e - 25);
    return (h & 0x8000u) ? -v : v;
}

float orc_round_half(float f) { return orc_f16_to_f32(orc_f32_to_f16(f)); }

static float orc_lut[65536];
static int orc_lut_ready = 0;

static void orc_lut_init(void)
{
    if (orc_lut_ready) return;
    for (unsigned int i = 0; i < 65536u; ++i) orc_lut[i] = orc_f16_to_f32((uint16_t)i);
    orc_lut_ready = 1;
}

/* ------------------------------------------------------------------------------------
 * Q8_0 (cuda/model/matrix.cuh:6-9: fp16 scale + 32 int8 in 34 bytes)
 * ---------------------------------------------------------------------------------- */
static float orc_q8_scale(const uint8_t *blk)
{
    return orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
}

float orc_q8_value(const uint8_t *row, unsigned int j)
{
    const uint8_t *blk = row + (size_t)(j / 32u) * 34u;
    int q = (int)(int8_t)blk[2u + j % 32u];
    return orc_round_half((float)q * orc_q8_scale(blk));
}

void orc_q8_gemv_f64(const uint8_t *w, unsigned int n, unsigned int k, const uint16_t *x,
                     unsigned int m, double *y, int swap)
{
    size_t stride = (size_t)(k / 32u) * 34u;
    for (unsigned int i = 0; i < m; ++i) {
        for (unsigned int j = 0; j < n; ++j) {
            double sum = 0.0;
            for (unsigned int c = 0; c < k; ++c) {
                const uint8_t *row = w + stride * (swap ? c : j);
                sum += (double)orc_f16_to_f32(x[(size_t)i * k + c])
                     * (double)orc_q8_value(row, swap ? j : c);
            }
            y[(size_t)i * n + j] = sum;
        }
    }
}

struct orc_gemv_job {
    const uint8_t *w; unsigned int n, k; const uint16_t *x; unsigned int m; float *y;
    unsigned int lo, hi;
    const float *xf;
};

/* half(f) for the weight reader: the normal half range by integer rounding to nearest
 * even (identical to orc_round_half there), everything else through orc_round_half. */
static float orc_round_half_w(float f)
{
    union { float f; uint32_t u; } v = { f };
    uint32_t mag = v.u & 0x7FFFFFFFu;
    if (mag < 0x38800000u || mag >= 0x477FE000u) return orc_round_half(f);
    v.u = (v.u + 0xFFFu + ((v.u >> 13) & 1u)) & 0xFFFFE000u;
    return v.f;
}

/* Rows of a product. The reference reads a Q8_0 weight two ways: passes of up to 16 rows
 * (gemv.cuh:68-98 through the group reader, matrix.cuh:499-512, and the one-row PTX
 * module, gemv_q8.ptx:135-147) keep the fp32 product scale * q; passes of 17 rows or more
 * run the tensor-core tile, which stages the weights as half (gemm.cuh:108-113), the
 * value reader's half(scale * q) (matrix.cuh:413-422). The sum over k is serial fp32. */
static void *orc_gemv_worker(void *arg)
{
    struct orc_gemv_job *jb = (struct orc_gemv_job *)arg;
    size_t stride = (size_t)(jb->k / 32u) * 34u;
    unsigned int blocks = jb->k / 32u;
    const int half_w = jb->m >= 17u;
    float *wrow = (float *)malloc((size_t)jb->k * sizeof(float));
    for (unsigned int j = jb->lo; j < jb->hi; ++j) {
        const uint8_t *row = jb->w + stride * j;
        for (unsigned int b = 0; b < blocks; ++b) {
            const uint8_t *blk = row + (size_t)b * 34u;
            float scale = orc_q8_scale(blk);
            for (unsigned int e = 0; e < 32u; ++e) {
                float wv = (float)(int)(int8_t)blk[2u + e] * scale;
                wrow[b * 32u + e] = half_w ? orc_round_half_w(wv) : wv;
            }
        }
        for (unsigned int i = 0; i < jb->m; ++i) {
            const float *xr = jb->xf + (size_t)i * jb->k;
            float acc = 0.0f;
            for (unsigned int c = 0; c < jb->k; ++c) acc += wrow[c] * xr[c];
            jb->y[(size_t)i * jb->n + j] = acc;
        }
    }
    free(wrow);
    return NULL;
}

void orc_q8_gemv_f32(const uint8_t *w, unsigned int n, unsigned int k, const uint16_t *x,
                     unsigned int m, float *y, unsigned int threads)
{
    float *xf = (float *)malloc((size_t)m * k * sizeof(float));
    for (size_t i = 0; i < (size_t)m * k; ++i) xf[i] = orc_f16_to_f32(x[i]);
    if (threads < 1u) threads = 1u;
    if (threads > 256u) threads = 256u;
    if (threads > n) threads = n;
    pthread_t th[256];
    struct orc_gemv_job jobs[256];
    unsigned int per = (n + threads - 1u) / threads;
    for (unsigned int t = 0; t < threads; ++t) {
        jobs[t] = (struct orc_gemv_job){ w, n, k, x, m, y, per * t,
                                         per * (t + 1u) < n ? per * (t + 1u) : n, xf };
        if (threads == 1u) orc_gemv_worker(&jobs[t]);
        else pthread_create(&th[t], NULL, orc_gemv_worker, &jobs[t]);
    }
    if (threads > 1u) for (unsigned int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
    free(xf);
}

/* ------------------------------------------------------------------------------------
 * Philox4x32-10 (tests/rng_test.cu:33-57)
 * ---------------------------------------------------------------------------------- */
void orc_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (unsigned int r = 0; r < 10u; ++r) {
        if (r != 0u) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float orc_rng_unit(uint64_t seed, uint32_t stream, uint32_t lane, uint64_t position)
{
    uint32_t key[2] = { (uint32_t)seed, (uint32_t)(seed >> 32) };
    uint32_t ctr[4] = { (uint32_t)position, (uint32_t)(position >> 32), lane, stream };
    uint32_t out[4];
    orc_philox(ctr, key, out);
    return (float)(out[0] >> 8) * (1.0f / 16777216.0f);
}

/* ------------------------------------------------------------------------------------
 * Sampler (cuda/model/sample.cu:456-765). The reference block has 256 threads: a thread
 * t visits tokens t, t+256, ... and thread 0 then combines the 256 partials in thread
 * order; every sum and comparison below follows that order.
 * ---------------------------------------------------------------------------------- */
#define ORC_THREADS 256u
#define ORC_BUCKETS 256u

typedef struct { float value; unsigned int index; } orc_cand;

static int orc_cand_order(const void *a, const void *b)
{
    const orc_cand *x = (const orc_cand *)a, *y = (const orc_cand *)b;
    if (x->value > y->value) return -1;
    if (x->value < y->value) return 1;
    return (x->index < y->index) ? -1 : (x->index > y->index);
}

int orc_pick(const float *row, unsigned int vocab, unsigned int top_k, float top_p,
             float min_p, float temperature, uint64_t seed, unsigned int agent,
             uint64_t position, unsigned int *count_out, unsigned int *taken_out,
             unsigned int *allowed_out)
{
    /* largest logit and its place (sample.cu:524-549) */
    float part[ORC_THREADS];
    unsigned int mark[ORC_THREADS];
    for (unsigned int t = 0; t < ORC_THREADS; ++t) {
        float best = -INFINITY;
        unsigned int at = 0;
        for (unsigned int i = t; i < vocab; i += ORC_THREADS) {
            if (row[i] > best) { best = row[i]; at = i; }
        }
        part[t] = best;
        mark[t] = at;
    }
    for (unsigned int i = 1; i < ORC_THREADS; ++i) {
        if (part[i] > part[0]) { part[0] = part[i]; mark[0] = mark[i]; }
    }
    float top = part[0];
    if (count_out) *count_out = 0;
    if (taken_out) *taken_out = 1;
    if (temperature <= 0.0f) {
        if (allowed_out) allowed_out[0] = mark[0];
        return (int)mark[0];
    }

    /* bucket search (sample.cu:615-668) */
    float lo = -AOTX_MODEL_PICK_SPAN, hi = 0.0f, shared_sum = 0.0f, cut = lo;
    unsigned int bucket[ORC_BUCKETS];
    for (unsigned int pass = 0; pass < 2u; ++pass) {
        memset(bucket, 0, sizeof bucket);
        float band = hi - lo;
        for (unsigned int t = 0; t < ORC_THREADS; ++t) {
            float row_total = 0.0f;
            for (unsigned int i = t; i < vocab; i += ORC_THREADS) {
                float scaled = row[i] - top;
                if (pass == 0u) row_total += expf(scaled);
                if (scaled >= lo && scaled <= hi) {
                    unsigned int b = (unsigned int)((scaled - lo) * (float)ORC_BUCKETS / band);
                    if (b >= ORC_BUCKETS) b = ORC_BUCKETS - 1u;
                    bucket[b] += 1u;
                }
            }
            part[t] = row_total;
        }
        if (pass == 0u) {
            float sum = 0.0f;
            for (unsigned int i = 0; i < ORC_THREADS; ++i) sum += part[i];
            shared_sum = sum;
        }
        unsigned int held = 0, more = 0;
        float next_lo = lo, next_hi = hi;
        cut = lo;
        for (unsigned int b = ORC_BUCKETS; b != 0u; --b) {
            if (held + bucket[b - 1u] > AOTX_MODEL_PICK_MAX) {
                cut = lo + band * (float)b / (float)ORC_BUCKETS;
                if (held == 0u) {
                    more = 1u;
                    next_lo = lo + band * (float)(b - 1u) / (float)ORC_BUCKETS;
                    next_hi = cut;
                }
                break;
            }
            held += bucket[b - 1u];
        }
        if (!more) break;
        lo = next_lo;
        hi = next_hi;
    }

    /* candidates at or above the cut in token order, at most 256 (the lowest ids when more
     * pass: the reference keeps an arbitrary 256 of them), then largest first with ties to
     * the lower id */
    orc_cand *all = (orc_cand *)malloc((size_t)vocab * sizeof *all);
    unsigned int count = 0;
    for (unsigned int i = 0; i < vocab && count < AOTX_MODEL_PICK_MAX; ++i) {
        float scaled = row[i] - top;
        if (scaled >= cut) { all[count].value = scaled; all[count].index = i; ++count; }
    }
    qsort(all, count, sizeof *all, orc_cand_order);

    /* count cut, min-p, mass cut on T=1, temperature, inverse CDF (sample.cu:715-759) */
    unsigned int keep = (top_k == 0u || top_k > count) ? count : top_k;
    if (min_p > 0.0f && min_p <= 1.0f) {
        unsigned int min_keep = 1u;
        for (unsigned int i = 1; i < keep; ++i) {
            if (expf(all[i].value - all[0].value) < min_p) break;
            min_keep = i + 1u;
        }
        keep = min_keep;
    }
    float limit = (top_p <= 0.0f || top_p > 1.0f) ? 1.0f : top_p;
    float mass = 0.0f;
    unsigned int taken = 0;
    for (unsigned int i = 0; i < keep; ++i) {
        mass += expf(all[i].value) / shared_sum;
        taken = i + 1u;
        if (mass >= limit) break;
    }
    float heat_total = 0.0f;
    for (unsigned int i = 0; i < taken; ++i) heat_total += expf((all[i].value - all[0].value) / temperature);
    float pick = orc_rng_unit(seed, agent, 0u, position) * heat_total;
    float walk = 0.0f;
    unsigned int chosen = all[0].index;
    for (unsigned int i = 0; i < taken; ++i) {
        walk += expf((all[i].value - all[0].value) / temperature);
        chosen = all[i].index;
        if (walk >= pick) break;
    }
    if (count_out) *count_out = count;
    if (taken_out) *taken_out = taken;
    if (allowed_out) for (unsigned int i = 0; i < taken; ++i) allowed_out[i] = all[i].index;
    free(all);
    return (int)chosen;
}

/* ------------------------------------------------------------------------------------
 * The pick's adjusted logit (cuda/model/sample.cu:277-319) with the penalties of a
 * sample over a sequence's token list: presence and frequency penalties on every token the
 * list holds, then the repeat penalty on a token inside the last `repeat_window` tokens.
 * The reference's compiler contracts presence + frequency * count into one fused
 * multiply-add, written here as fmaf. The row is adjusted in place.
 * ---------------------------------------------------------------------------------- */
void orc_pick_adjust(float *row, unsigned int vocab, const int *list, unsigned int n,
                     float presence, float frequency, float repeat_penalty,
                     unsigned int repeat_window)
{
    const int pf = presence != 0.0f || frequency != 0.0f;
    const int rp = repeat_window != 0u && repeat_penalty != 1.0f;
    if (!pf && !rp) return;
    unsigned int first = n > repeat_window ? n - repeat_window : 0u;
    for (unsigned int t = 0; t < vocab; ++t) {
        float value = row[t];
        unsigned int count = 0u, inside = 0u;
        for (unsigned int i = 0; i < n; ++i) {
            if ((unsigned int)list[i] == t) {
                count += 1u;
                if (i >= first) inside = 1u;
            }
        }
        if (pf && count != 0u) value -= fmaf(frequency, (float)count, presence);
        if (rp && inside) value = value > 0.0f ? value / repeat_penalty : value * repeat_penalty;
        row[t] = value;
    }
}

/* ------------------------------------------------------------------------------------
 * Router (cuda/model/experts.cu:10-75), in double as tests/expert_test.cu:118-152 checks.
 * ---------------------------------------------------------------------------------- */
void orc_route(const float *router, const uint16_t *x, unsigned int tokens,
               unsigned int hidden, unsigned int experts, unsigned int used, float *prob,
               unsigned int *ids)
{
    double *logit = (double *)malloc(experts * sizeof(double));
    double *p = (double *)malloc(experts * sizeof(double));
    unsigned int *order = (unsigned int *)malloc(experts * sizeof(unsigned int));
    for (unsigned int t = 0; t < tokens; ++t) {
        double top = -INFINITY, total = 0.0;
        for (unsigned int e = 0; e < experts; ++e) {
            double dot = 0.0;
            for (unsigned int d = 0; d < hidden; ++d) {
                dot += (double)router[(size_t)e * hidden + d]
                     * (double)orc_f16_to_f32(x[(size_t)t * hidden + d]);
            }
            logit[e] = dot;
            if (dot > top) top = dot;
            order[e] = e;
        }
        for (unsigned int e = 0; e < experts; ++e) { p[e] = exp(logit[e] - top); total += p[e]; }
        for (unsigned int e = 0; e < experts; ++e) {
            p[e] /= total;
            prob[(size_t)t * experts + e] = (float)p[e];
        }
        for (unsigned int r = 0; r < experts; ++r) {
            unsigned int best = r;
            for (unsigned int j = r + 1u; j < experts; ++j) {
                if (p[order[j]] > p[order[best]]
                    || (p[order[j]] == p[order[best]] && order[j] < order[best])) best = j;
            }
            unsigned int keep = order[r]; order[r] = order[best]; order[best] = keep;
        }
        for (unsigned int r = 0; r < used; ++r) ids[(size_t)t * used + r] = order[r];
    }
    free(logit); free(p); free(order);
}

/* ------------------------------------------------------------------------------------
 * Attention of one head (cuda/model/attention.cu:66-129)
 * ---------------------------------------------------------------------------------- */
void orc_attend_one(const float *q, const float *keys, const float *values,
                    unsigned int stride, unsigned int last, unsigned int d, float *out)
{
    float scale = 1.0f / sqrtf((float)d);
    float top = -INFINITY, mass = 0.0f;
    float sum[512];
    for (unsigned int i = 0; i < d; ++i) sum[i] = 0.0f;
    for (unsigned int j = 0; j <= last; ++j) {
        const float *key = keys + (size_t)j * stride;
        float dot = 0.0f;
        for (unsigned int i = 0; i < d; ++i) dot += q[i] * key[i];
        dot = dot * scale;
        float raised = fmaxf(top, dot);
        float shift = expf(top - raised);
        float weight = expf(dot - raised);
        const float *value = values + (size_t)j * stride;
        for (unsigned int i = 0; i < d; ++i) sum[i] = sum[i] * shift + weight * value[i];
        mass = mass * shift + weight;
        top = raised;
    }
    float back = mass > 0.0f ? 1.0f / mass : 0.0f;
    for (unsigned int i = 0; i < d; ++i) out[i] = orc_round_half(sum[i] * back);
}

/* The same attention over fp16 rows as the pages hold them. */
static void orc_attend_half(const float *q, const uint16_t *keys, const uint16_t *values,
                            unsigned int stride, unsigned int last, unsigned int d, float *out)
{
    float scale = 1.0f / sqrtf((float)d);
    float top = -INFINITY, mass = 0.0f;
    float sum[512];
    for (unsigned int i = 0; i < d; ++i) sum[i] = 0.0f;
    for (unsigned int j = 0; j <= last; ++j) {
        const uint16_t *key = keys + (size_t)j * stride;
        float dot = 0.0f;
        for (unsigned int i = 0; i < d; ++i) dot += q[i] * orc_lut[key[i]];
        dot = dot * scale;
        float raised = fmaxf(top, dot);
        float shift = expf(top - raised);
        float weight = expf(dot - raised);
        const uint16_t *value = values + (size_t)j * stride;
        for (unsigned int i = 0; i < d; ++i) sum[i] = sum[i] * shift + weight * orc_lut[value[i]];
        mass = mass * shift + weight;
        top = raised;
    }
    float back = mass > 0.0f ? 1.0f / mass : 0.0f;
    for (unsigned int i = 0; i < d; ++i) out[i] = orc_round_half(sum[i] * back);
}

/* ------------------------------------------------------------------------------------
 * Whole model (tests/model_ref.h:301-427, generalised to the layer kinds of the path)
 * ---------------------------------------------------------------------------------- */
struct orc_model {
    aotx_model_desc d;
    const uint8_t *w;
    unsigned int slots, max_context, threads;
    unsigned int *seen;
    uint16_t *keys;  /* [slots][layers][max_context][kv_heads*d], fp16 as the pages hold */
    uint16_t *values;
    float *last_xnorm;
    /* the residual row of each sequence's last token after every layer of the last step,
     * [layers][seqs][hidden] (the probe's capture, cuda/model/conduct.cu:165-173) */
    float *last_resid;
    /* routing of the last experts layer of the last step: [tokens][experts], [tokens][used] */
    float *last_prob;
    unsigned int *last_ids;
    unsigned int last_route_tokens;
};



static const void *orc_tensor(const orc_model *m, unsigned long long off)
{
    return off == AOTX_MODEL_ABSENT ? NULL : (const void *)(m->w + off);
}

orc_model *orc_model_new(const aotx_model_desc *desc, const uint8_t *weights,
                         unsigned int slots, unsigned int max_context, unsigned int threads)
{
    orc_model *m = (orc_model *)calloc(1, sizeof *m);
    m->d = *desc;
    m->w = weights;
    m->slots = slots;
    m->max_context = max_context;
    m->threads = threads ? threads : 1u;
    m->seen = (unsigned int *)calloc(slots, sizeof(unsigned int));
    size_t narrow = (size_t)desc->kv_heads * desc->head_dim;
    size_t cells = (size_t)slots * desc->layers * max_context * narrow;
    orc_lut_init();
    m->keys = (uint16_t *)calloc(cells, sizeof(uint16_t));
    m->values = (uint16_t *)calloc(cells, sizeof(uint16_t));
    m->last_xnorm = (float *)calloc((size_t)slots * desc->hidden, sizeof(float));
    m->last_resid = (float *)calloc((size_t)desc->layers * slots * desc->hidden, sizeof(float));
    return m;
}

void orc_model_free(orc_model *m)
{
    if (!m) return;
    free(m->seen); free(m->keys); free(m->values); free(m->last_xnorm); free(m->last_resid);
    free(m->last_prob); free(m->last_ids); free(m);
}

void orc_model_forget(orc_model *m)
{
    memset(m->seen, 0, m->slots * sizeof(unsigned int));
}

const float *orc_model_last_xnorm(const orc_model *m) { return m->last_xnorm; }
const float *orc_model_last_resid(const orc_model *m) { return m->last_resid; }

/* The router's probabilities and chosen experts of the last experts layer the last step
 * ran; *tokens is the step's row count (0 when no experts layer ran). */
const float *orc_model_last_route(const orc_model *m, const unsigned int **ids,
                                  unsigned int *tokens)
{
    *ids = m->last_ids;
    *tokens = m->last_route_tokens;
    return m->last_prob;
}

/* The model's cache as fp16 words [slots][layers][max_context][kv_heads * head_dim]:
 * which = 0 keys, 1 values. For tests that write the same cache into the device pages. */
const uint16_t *orc_model_cache(const orc_model *m, unsigned int which)
{
    return which == 0u ? m->keys : m->values;
}

/* rows of half values in, fp32 products out: y[t][n] = W x[t] (reference GEMV sums) */
static void orc_matmul(const orc_model *m, const uint8_t *w, unsigned int n, unsigned int k,
                       const float *xh, unsigned int rows, float *y)
{
    uint16_t *x16 = (uint16_t *)malloc((size_t)rows * k * sizeof(uint16_t));
    for (size_t i = 0; i < (size_t)rows * k; ++i) x16[i] = orc_f32_to_f16(xh[i]);
    orc_q8_gemv_f32(w, n, k, x16, rows, y, m->threads);
    free(x16);
}

/* RMSNorm to half (cuda/model/norm.cu:49-77): half(scale * x * w). */
static void orc_rms(const float *in, const float *weight, float *out, unsigned int width,
                    float eps)
{
    float sum = 0.0f;
    for (unsigned int i = 0; i < width; ++i) sum += in[i] * in[i];
    float scale = 1.0f / sqrtf(sum / (float)width + eps);
    for (unsigned int i = 0; i < width; ++i) out[i] = orc_round_half(scale * in[i] * weight[i]);
}

/* Turn one head (cuda/model/rope.cu:88-115, :200-234): angle = pos * step^i,
 * step = theta^(-2/d); pairs split (i, i+d/2) or adjacent (2i, 2i+1). */
static void orc_rope(float *head, unsigned int dim, unsigned int position, float theta,
                     unsigned int pairs, const float *factor)
{
    float step = powf(theta, -2.0f / (float)dim);
    for (unsigned int i = 0; i < dim / 2u; ++i) {
        unsigned int lo = pairs == AOTX_ROPE_PAIRS_ADJACENT ? 2u * i : i;
        unsigned int hi = pairs == AOTX_ROPE_PAIRS_ADJACENT ? 2u * i + 1u : i + dim / 2u;
        float angle = (float)position * powf(step, (float)i);
        if (factor) angle = angle / factor[i];
        float c = cosf(angle), s = sinf(angle);
        float a = head[lo], b = head[hi];
        head[lo] = orc_round_half(a * c - b * s);
        head[hi] = orc_round_half(a * s + b * c);
    }
}

struct orc_attn_job {
    const orc_model *m;
    unsigned int l, tokens;
    const float *q;
    float *att;
    const unsigned int *pos, *slot;
    size_t slot_stride, narrow, wide;
    unsigned int lo, hi;   /* (token, head) items of one worker */
};

static void *orc_attn_worker(void *arg)
{
    struct orc_attn_job *j = (struct orc_attn_job *)arg;
    const aotx_model_desc *d = &j->m->d;
    unsigned int hd = d->head_dim;
    for (unsigned int it = j->lo; it < j->hi; ++it) {
        unsigned int t = it / d->heads, hh = it % d->heads;
        unsigned int kvh = hh / (d->heads / d->kv_heads);
        const uint16_t *kb = j->m->keys + j->slot[t] * j->slot_stride + (size_t)j->l * j->m->max_context * j->narrow;
        const uint16_t *vb = j->m->values + j->slot[t] * j->slot_stride + (size_t)j->l * j->m->max_context * j->narrow;
        orc_attend_half(j->q + (size_t)t * j->wide + (size_t)hh * hd, kb + kvh * hd, vb + kvh * hd,
                        (unsigned int)j->narrow, j->pos[t], hd, j->att + (size_t)t * j->wide + (size_t)hh * hd);
    }
    return NULL;
}

/* Attention of every (token, head) of one layer, over the model's threads. */
static void orc_attn_run(struct orc_attn_job *base)
{
    unsigned int items = base->tokens * base->m->d.heads;
    unsigned int threads = base->m->threads;
    if (threads > items) threads = items;
    if (threads <= 1u) {
        base->lo = 0;
        base->hi = items;
        orc_attn_worker(base);
        return;
    }
    pthread_t th[256];
    struct orc_attn_job jobs[256];
    if (threads > 256u) threads = 256u;
    unsigned int per = (items + threads - 1u) / threads;
    for (unsigned int t = 0; t < threads; ++t) {
        jobs[t] = *base;
        jobs[t].lo = per * t;
        jobs[t].hi = per * (t + 1u) < items ? per * (t + 1u) : items;
        pthread_create(&th[t], NULL, orc_attn_worker, &jobs[t]);
    }
    for (unsigned int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
}

struct orc_seat_job { orc_model *m; unsigned int slot, position, layer; uint64_t seed; };

static void *orc_seat_worker(void *arg)
{
    struct orc_seat_job *j = (struct orc_seat_job *)arg;
    orc_model *m = j->m;
    size_t narrow = (size_t)m->d.kv_heads * m->d.head_dim;
    size_t slot_stride = (size_t)m->d.layers * m->max_context * narrow;
    uint16_t *kb = m->keys + j->slot * slot_stride + (size_t)j->layer * m->max_context * narrow;
    uint16_t *vb = m->values + j->slot * slot_stride + (size_t)j->layer * m->max_context * narrow;
    uint64_t x = j->seed * 0x9E3779B97F4A7C15ull + (uint64_t)j->slot * 1000003ull + j->layer + 1ull;
    for (size_t i = 0; i < (size_t)j->position * narrow; ++i) {
        x ^= x << 13; x ^= x >> 7; x ^= x << 17;
        float u = (float)(x >> 40) * (1.0f / 16777216.0f) * 4.0f - 2.0f;
        kb[i] = orc_f32_to_f16(u);
        x ^= x << 13; x ^= x >> 7; x ^= x << 17;
        u = (float)(x >> 40) * (1.0f / 16777216.0f) * 4.0f - 2.0f;
        vb[i] = orc_f32_to_f16(u);
    }
    return NULL;
}

int orc_model_seat(orc_model *m, unsigned int slot, unsigned int position, uint64_t seed)
{
    if (slot >= m->slots || position > m->max_context) return 1;
    unsigned int layers = m->d.layers;
    pthread_t th[AOTX_MODEL_MAX_LAYERS];
    struct orc_seat_job jobs[AOTX_MODEL_MAX_LAYERS];
    for (unsigned int l = 0; l < layers; ++l) {
        jobs[l] = (struct orc_seat_job){ m, slot, position, l, seed };
        pthread_create(&th[l], NULL, orc_seat_worker, &jobs[l]);
    }
    for (unsigned int l = 0; l < layers; ++l) pthread_join(th[l], NULL);
    m->seen[slot] = position;
    return 0;
}

int orc_model_step(orc_model *m, const int *ids, const unsigned int *offset,
                   unsigned int seqs, const unsigned int *agent, float *logits)
{
    const aotx_model_desc *d = &m->d;
    unsigned int tokens = offset[seqs];
    unsigned int h = d->hidden, f = d->ffn, hd = d->head_dim;
    unsigned int wide = d->heads * hd, narrow = d->kv_heads * hd;
    unsigned int big = h > f ? h : f;
    if (wide > big) big = wide;
    for (unsigned int s = 0; s < seqs; ++s) {
        if (agent[s] >= m->slots || m->seen[agent[s]] + (offset[s + 1] - offset[s]) > m->max_context) return 1;
    }
    m->last_route_tokens = 0;
    float *resid = (float *)calloc((size_t)tokens * h, sizeof(float));
    float *x = (float *)calloc((size_t)tokens * big, sizeof(float));
    float *q = (float *)calloc((size_t)tokens * wide, sizeof(float));
    float *k = (float *)calloc((size_t)tokens * narrow, sizeof(float));
    float *v = (float *)calloc((size_t)tokens * narrow, sizeof(float));
    float *att = (float *)calloc((size_t)tokens * wide, sizeof(float));
    float *proj = (float *)calloc((size_t)tokens * h, sizeof(float));
    float *gate = (float *)calloc((size_t)tokens * f, sizeof(float));
    float *up = (float *)calloc((size_t)tokens * f, sizeof(float));
    float *act = (float *)calloc((size_t)tokens * f, sizeof(float));
    float *esum = (float *)calloc((size_t)tokens * h, sizeof(float));
    unsigned int *pos = (unsigned int *)calloc(tokens, sizeof(unsigned int));
    unsigned int *slot = (unsigned int *)calloc(tokens, sizeof(unsigned int));
    for (unsigned int s = 0; s < seqs; ++s) {
        for (unsigned int t = offset[s]; t < offset[s + 1]; ++t) {
            pos[t] = m->seen[agent[s]] + (t - offset[s]);
            slot[t] = agent[s];
        }
    }

    /* gather (cuda/model/gather.cu:53-80): resid = fp32(scale) * q */
    const uint8_t *emb = (const uint8_t *)orc_tensor(m, d->token_embd);
    size_t erow = (size_t)(h / 32u) * 34u;
    for (unsigned int t = 0; t < tokens; ++t) {
        unsigned int id = (ids[t] < 0 || (unsigned int)ids[t] >= d->vocab) ? 0u : (unsigned int)ids[t];
        const uint8_t *row = emb + erow * id;
        for (unsigned int c = 0; c < h; ++c) {
            const uint8_t *blk = row + (size_t)(c / 32u) * 34u;
            resid[(size_t)t * h + c] = orc_q8_scale(blk) * (float)(int)(int8_t)blk[2u + c % 32u];
        }
    }
    float scale_att = 1.0f / sqrtf((float)hd);
    (void)scale_att;
    const float *factor = (const float *)orc_tensor(m, d->rope_freqs);
    size_t slot_stride = (size_t)d->layers * m->max_context * narrow;
    for (unsigned int l = 0; l < d->layers; ++l) {
        const aotx_model_layer *L = &d->layer[l];
        const float *wn = (const float *)orc_tensor(m, L->offset[AOTX_SLOT_ATTN_NORM]);
        for (unsigned int t = 0; t < tokens; ++t) orc_rms(resid + (size_t)t * h, wn, x + (size_t)t * h, h, d->rms_eps);
        orc_matmul(m, (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_ATTN_Q]), wide, h, x, tokens, q);
        orc_matmul(m, (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_ATTN_K]), narrow, h, x, tokens, k);
        orc_matmul(m, (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_ATTN_V]), narrow, h, x, tokens, v);
        const float *qn = NULL, *kn = NULL;
        if (d->kind[l] == AOTX_LAYER_KIND_ATTENTION) {
            qn = (const float *)orc_tensor(m, L->offset[AOTX_ATTENTION_Q_NORM]);
            kn = (const float *)orc_tensor(m, L->offset[AOTX_ATTENTION_K_NORM]);
        }
        for (unsigned int t = 0; t < tokens; ++t) {
            for (unsigned int hh = 0; hh < d->heads; ++hh) {
                float *head = q + (size_t)t * wide + (size_t)hh * hd;
                if (qn) {
                    float tmp[512];
                    float sum = 0.0f;
                    for (unsigned int i = 0; i < hd; ++i) sum += head[i] * head[i];
                    float sc = 1.0f / sqrtf(sum / (float)hd + d->rms_eps);
                    for (unsigned int i = 0; i < hd; ++i) tmp[i] = sc * head[i] * qn[i];
                    memcpy(head, tmp, hd * sizeof(float));
                }
                orc_rope(head, hd, pos[t], d->rope_theta, d->rope_pairs, factor);
            }
            uint16_t *kc = m->keys + slot[t] * slot_stride + ((size_t)l * m->max_context + pos[t]) * narrow;
            uint16_t *vc = m->values + slot[t] * slot_stride + ((size_t)l * m->max_context + pos[t]) * narrow;
            for (unsigned int hh = 0; hh < d->kv_heads; ++hh) {
                float *head = k + (size_t)t * narrow + (size_t)hh * hd;
                if (kn) {
                    float tmp[512];
                    float sum = 0.0f;
                    for (unsigned int i = 0; i < hd; ++i) sum += head[i] * head[i];
                    float sc = 1.0f / sqrtf(sum / (float)hd + d->rms_eps);
                    for (unsigned int i = 0; i < hd; ++i) tmp[i] = sc * head[i] * kn[i];
                    memcpy(head, tmp, hd * sizeof(float));
                }
                orc_rope(head, hd, pos[t], d->rope_theta, d->rope_pairs, factor);
                for (unsigned int i = 0; i < hd; ++i) {
                    kc[hh * hd + i] = orc_f32_to_f16(head[i]);
                    vc[hh * hd + i] = orc_f32_to_f16(v[(size_t)t * narrow + hh * hd + i]);
                }
            }
        }
        {
            struct orc_attn_job job = { m, l, tokens, q, att, pos, slot, slot_stride, narrow, wide, 0, 0 };
            orc_attn_run(&job);
        }
        orc_matmul(m, (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_ATTN_O]), h, wide, att, tokens, proj);
        for (size_t i = 0; i < (size_t)tokens * h; ++i) resid[i] += proj[i];
        const float *fn = (const float *)orc_tensor(m, L->offset[AOTX_SLOT_FFN_NORM]);
        for (unsigned int t = 0; t < tokens; ++t) orc_rms(resid + (size_t)t * h, fn, x + (size_t)t * h, h, d->rms_eps);
        if (d->kind[l] == AOTX_LAYER_KIND_FFN_EXPERTS) {
            /* route, then each rank's expert in rank order with the products rounded
             * before the sums (cuda/model/experts.cu:77-98) */
            unsigned int E = d->expert_count, used = d->expert_used_count;
            float *prob = (float *)malloc((size_t)tokens * E * sizeof(float));
            unsigned int *sel = (unsigned int *)malloc((size_t)tokens * used * sizeof(unsigned int));
            uint16_t *x16 = (uint16_t *)malloc((size_t)tokens * h * sizeof(uint16_t));
            for (size_t i = 0; i < (size_t)tokens * h; ++i) x16[i] = orc_f32_to_f16(x[i]);
            orc_route((const float *)orc_tensor(m, L->offset[AOTX_EXPERT_ROUTER]), x16, tokens, h, E, used, prob, sel);
            size_t gslice = (size_t)f * (h / 32u) * 34u, dslice = (size_t)h * (f / 32u) * 34u;
            const uint8_t *G = (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_FFN_GATE]);
            const uint8_t *U = (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_FFN_UP]);
            const uint8_t *D = (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_FFN_DOWN]);
            for (unsigned int t = 0; t < tokens; ++t) {
                for (unsigned int r = 0; r < used; ++r) {
                    unsigned int e = sel[(size_t)t * used + r];
                    float p = prob[(size_t)t * E + e];
                    orc_matmul(m, G + e * gslice, f, h, x + (size_t)t * h, 1, gate);
                    orc_matmul(m, U + e * gslice, f, h, x + (size_t)t * h, 1, up);
                    for (unsigned int i = 0; i < f; ++i) {
                        float g = gate[i];
                        act[i] = orc_round_half(g / (1.0f + expf(-g)) * up[i]);
                    }
                    orc_matmul(m, D + e * dslice, h, f, act, 1, proj);
                    for (unsigned int i = 0; i < h; ++i) {
                        float val = proj[i] * p;
                        if (r != 0u) val = esum[(size_t)t * h + i] + val;
                        esum[(size_t)t * h + i] = val;
                    }
                }
            }
            for (size_t i = 0; i < (size_t)tokens * h; ++i) resid[i] += esum[i];
            free(m->last_prob); free(m->last_ids);
            m->last_prob = prob;
            m->last_ids = sel;
            m->last_route_tokens = tokens;
            free(x16);
        } else {
            orc_matmul(m, (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_FFN_GATE]), f, h, x, tokens, gate);
            orc_matmul(m, (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_FFN_UP]), f, h, x, tokens, up);
            for (size_t i = 0; i < (size_t)tokens * f; ++i) {
                float g = gate[i];
                act[i] = orc_round_half(g / (1.0f + expf(-g)) * up[i]);
            }
            orc_matmul(m, (const uint8_t *)orc_tensor(m, L->offset[AOTX_SLOT_FFN_DOWN]), h, f, act, tokens, proj);
            for (size_t i = 0; i < (size_t)tokens * h; ++i) resid[i] += proj[i];
        }
        for (unsigned int s = 0; s < seqs; ++s)
            memcpy(m->last_resid + ((size_t)l * seqs + s) * h,
                   resid + (size_t)(offset[s + 1] - 1u) * h, (size_t)h * sizeof(float));
    }
    /* head: last norm, last row of each sequence, output matrix (graph_host.cu:115-153) */
    const float *on = (const float *)orc_tensor(m, d->output_norm);
    const uint8_t *head = (const uint8_t *)orc_tensor(m, d->tied_output ? d->token_embd : d->output);
    for (unsigned int s = 0; s < seqs; ++s) {
        unsigned int t = offset[s + 1] - 1u;
        orc_rms(resid + (size_t)t * h, on, m->last_xnorm + (size_t)s * h, h, d->rms_eps);
    }
    orc_matmul(m, head, d->vocab, h, m->last_xnorm, seqs, logits);
    for (unsigned int s = 0; s < seqs; ++s) m->seen[agent[s]] += offset[s + 1] - offset[s];
    free(resid); free(x); free(q); free(k); free(v); free(att); free(proj); free(gate);
    free(up); free(act); free(esum); free(pos); free(slot);
    return 0;
}
