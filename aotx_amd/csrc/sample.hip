/* Sampler and Philox stream.
 *
 * Reference: aotx_model_pick (cuda/model/sample.cu:456-765) and the Philox4x32-10 stream
 * (cuda/rng/rng.cuh:29-94). One block of 256 threads takes one row of logits. The steps,
 * their order and every float expression follow the reference so that the same logits
 * give the same token: the largest logit (ties to the lowest thread = token mod 256, then
 * the lowest token), a temperature of zero returns it; otherwise the row sum of
 * exp(v - top), a two-pass 256-bucket search over the 42 below the top for a cut that
 * keeps at most 256 candidates, the candidates sorted largest first, then top-k, min-p,
 * top-p on the T = 1 probabilities, the temperature, and the inverse CDF at the Philox
 * uniform of (seed, slot, lane 0, draw position). Every sum runs in the reference's
 * order: thread t adds tokens t, t + 256, ..., then thread 0 adds the 256 partials in
 * thread order. One deliberate difference: where the reference leaves a choice to timing
 * (which candidates fill the 256 places when more pass the cut; the order of equal values
 * after its bitonic network), this kernel takes the lowest token ids, so the result is a
 * function of the logits alone.
 *
 * The penalties, voice bias and thinking masks of aotx_pick_value (sample.cu:277-319)
 * read the decode runtime's sequence table, which is outside this path; with a null
 * per-row `how` (the aotx_model_sample case) the reference leaves the logit unchanged
 * and so does this kernel.
 */
#include "aotx_internal.h"

#include <hip/hip_runtime.h>

#define PICK_THREADS 256u
#define PICK_BUCKETS 256u
#define PICK_PASSES 2u
#define PICK_CHUNKS 64u   /* workgroups per row of the largest-logit search */
#define PICK_EXP_WGS 32u  /* workgroups per row of the exponentials and first histogram */

#pragma clang fp contract(off)

struct aotx_u32x4 {
    unsigned int x, y, z, w;
};

static __device__ __forceinline__ aotx_u32x4 aotx_philox_dev(unsigned int c0, unsigned int c1,
                                                             unsigned int c2, unsigned int c3,
                                                             unsigned int k0, unsigned int k1)
{
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r != 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        unsigned int lo0 = 0xD2511F53u * c0;
        unsigned int hi0 = __umulhi(0xD2511F53u, c0);
        unsigned int lo1 = 0xCD9E8D57u * c2;
        unsigned int hi1 = __umulhi(0xCD9E8D57u, c2);
        unsigned int n0 = hi1 ^ c1 ^ k0;
        unsigned int n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    aotx_u32x4 out = {c0, c1, c2, c3};
    return out;
}

__global__ void aotx_philox_kernel(const unsigned int *ctr, const unsigned int *key,
                                   unsigned int n, unsigned int *out)
{
    unsigned int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    aotx_u32x4 w = aotx_philox_dev(ctr[4 * i], ctr[4 * i + 1], ctr[4 * i + 2], ctr[4 * i + 3],
                                   key[2 * i], key[2 * i + 1]);
    out[4 * i] = w.x;
    out[4 * i + 1] = w.y;
    out[4 * i + 2] = w.z;
    out[4 * i + 3] = w.w;
}

struct aotx_pick_args {
    const float *logits;          /* [rows][ld] */
    unsigned int ld;
    unsigned int vocab;
    const unsigned int *rows_dev; /* device row count, or null */
    unsigned int rows;
    const unsigned int *agent;    /* [rows] */
    const aotx_model_how *how;    /* per-row settings, or null */
    unsigned int top_k;
    float top_p;
    float temperature;
    unsigned long long seed;
    int *token;
    unsigned int *draw;
    aotx_state *state;
    const aotx_model_run *run;    /* when set, every per-call value comes from here */
    unsigned int *best;           /* [rows][PICK_CHUNKS][2]: each chunk's (value bits, token) */
    unsigned int *hist;           /* [rows][PICK_BUCKETS] first-pass counts, zero between calls */
    float *ex;                    /* [rows][vocab] exp(v - top) */
};

/* (v, i) ranks ahead of (bv, bi) in the reference's largest-logit search: a larger value;
 * among equal values the lower token mod 256 (the reference's lower thread), then the
 * lower token (that thread's earlier stride). NaN ranks nowhere. */
static __device__ __forceinline__ bool aotx_pick_ahead(float v, unsigned int i, float bv,
                                                       unsigned int bi)
{
    return v > bv || (v == bv && ((i & 255u) < (bi & 255u) || ((i & 255u) == (bi & 255u) && i < bi)));
}

/* The row's largest logit from the slices of aotx_argmax_kernel (reference order): one
 * slice per lane, merged across the wave; every lane of a full wave gets the winner. */
static_assert(PICK_CHUNKS <= 64u, "one slice per lane");
static __device__ __forceinline__ void aotx_pick_top(const aotx_pick_args &a, unsigned int r,
                                                     float &best, unsigned int &at)
{
    const unsigned int *cand = a.best + (unsigned long long)r * PICK_CHUNKS * 2u;
    const unsigned int lane = threadIdx.x & 63u;
    best = -INFINITY;
    at = 0u;
    if (lane < PICK_CHUNKS) {
        best = __uint_as_float(cand[2u * lane]);
        at = cand[2u * lane + 1u];
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const unsigned int oi = __shfl_xor(at, off, 64);
        if (aotx_pick_ahead(ov, oi, best, at)) {
            best = ov;
            at = oi;
        }
    }
}

/* The row's sampling settings (a per-row `how` overrides the call's). */
static __device__ __forceinline__ float aotx_pick_warmth(const aotx_pick_args &a, unsigned int r)
{
    const aotx_model_how *how = a.run ? a.run->how : a.how;
    if (how != nullptr) return how[r].temperature;
    return a.run ? a.run->temperature : a.temperature;
}

/* The largest logit of each of PICK_CHUNKS slices of a row (grid: chunks x rows). The
 * winner over the slices under aotx_pick_ahead is the reference's (thread-strided scan,
 * then the thread-order merge), so the slices can be searched in parallel. A slice whose
 * values are all -inf (or NaN) leaves (-inf, 0), as a reference thread does. */
__global__ __launch_bounds__(PICK_THREADS) void aotx_argmax_kernel(aotx_pick_args a)
{
    __shared__ float wv[PICK_THREADS / 64];
    __shared__ unsigned int wi[PICK_THREADS / 64];
    const unsigned int tid = threadIdx.x;
    const unsigned int r = blockIdx.y;
    const unsigned int c = blockIdx.x;
    const aotx_model_run *run = a.run;
    unsigned int rows = run ? run->rows : (a.rows_dev ? *a.rows_dev : a.rows);
    int *token_out = run ? run->token : a.token;
    if (r >= rows || token_out == nullptr) return;
    if (run && run->select != AOTX_MODEL_ROWS_LAST) return;
    /* the row's histogram starts at zero for the exponential pass that follows (its place
     * in the sampler's buffer depends on the call's row count, so an earlier call with
     * another count may have left other words there) */
    if (c == 0u)
        for (unsigned int i = tid; i < PICK_BUCKETS; i += PICK_THREADS)
            a.hist[(unsigned long long)r * PICK_BUCKETS + i] = 0u;
    const float *row = a.logits + (unsigned long long)r * a.ld;
    const unsigned int span = (a.vocab + PICK_CHUNKS - 1u) / PICK_CHUNKS;
    const unsigned int lo = c * span;
    const unsigned int hi = lo + span < a.vocab ? lo + span : a.vocab;
    float best = -INFINITY;
    unsigned int at = 0u;
#pragma unroll 8
    for (unsigned int i = lo + tid; i < hi; i += PICK_THREADS) {
        float one = row[i];
        if (aotx_pick_ahead(one, i, best, at)) {
            best = one;
            at = i;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        float ov = __shfl_xor(best, off, 64);
        unsigned int oi = __shfl_xor(at, off, 64);
        if (aotx_pick_ahead(ov, oi, best, at)) {
            best = ov;
            at = oi;
        }
    }
    if ((tid & 63u) == 0u) {
        wv[tid >> 6] = best;
        wi[tid >> 6] = at;
    }
    __syncthreads();
    if (tid == 0u) {
        for (unsigned int w = 1u; w < PICK_THREADS / 64u; ++w) {
            if (aotx_pick_ahead(wv[w], wi[w], best, at)) {
                best = wv[w];
                at = wi[w];
            }
        }
        unsigned int *out = a.best + ((unsigned long long)r * PICK_CHUNKS + c) * 2u;
        out[0] = __float_as_uint(best);
        out[1] = at;
    }
}

/* exp(v - top) of every logit of a sampled row (stored for the pick's ordered sums) and
 * the first pass of the cut search: the 256-bucket histogram over [top - 42, top], added
 * into the row's counts (integer counts: their order does not matter). Grid: PICK_EXP_WGS
 * x rows; rows at temperature 0 do nothing. */
__global__ __launch_bounds__(PICK_THREADS) void aotx_pick_exp_kernel(aotx_pick_args a)
{
    __shared__ unsigned int bucket[PICK_BUCKETS];
    const unsigned int tid = threadIdx.x;
    const unsigned int r = blockIdx.y;
    const aotx_model_run *run = a.run;
    unsigned int rows = run ? run->rows : (a.rows_dev ? *a.rows_dev : a.rows);
    int *token_out = run ? run->token : a.token;
    if (r >= rows || token_out == nullptr) return;
    if (run && run->select != AOTX_MODEL_ROWS_LAST) return;
    if (aotx_pick_warmth(a, r) <= 0.0f) return;
    float top;
    unsigned int at;
    aotx_pick_top(a, r, top, at);
    for (unsigned int i = tid; i < PICK_BUCKETS; i += PICK_THREADS) bucket[i] = 0u;
    __syncthreads();
    const float *row = a.logits + (unsigned long long)r * a.ld;
    float *ex = a.ex + (unsigned long long)r * a.vocab;
    const float lo = -AOTX_MODEL_PICK_SPAN, hi = 0.0f, band = hi - lo;
    const unsigned int span = (a.vocab + PICK_EXP_WGS - 1u) / PICK_EXP_WGS;
    const unsigned int b0 = blockIdx.x * span;
    const unsigned int b1 = b0 + span < a.vocab ? b0 + span : a.vocab;
#pragma unroll 8
    for (unsigned int i = b0 + tid; i < b1; i += PICK_THREADS) {
        const float scaled = row[i] - top;
        ex[i] = expf(scaled);
        if (scaled >= lo && scaled <= hi) {
            unsigned int b = (unsigned int)((scaled - lo) * (float)PICK_BUCKETS / band);
            if (b >= PICK_BUCKETS) b = PICK_BUCKETS - 1u;
            atomicAdd(&bucket[b], 1u);
        }
    }
    __syncthreads();
    unsigned int *h = a.hist + (unsigned long long)r * PICK_BUCKETS;
    for (unsigned int i = tid; i < PICK_BUCKETS; i += PICK_THREADS)
        if (bucket[i] != 0u) atomicAdd(h + i, bucket[i]);
}

__global__ __launch_bounds__(PICK_THREADS) void aotx_pick_kernel(aotx_pick_args a)
{
    __shared__ float part[PICK_THREADS];
    __shared__ unsigned int mark[PICK_THREADS];
    __shared__ unsigned int bucket[PICK_BUCKETS];
    __shared__ float value[AOTX_MODEL_PICK_MAX];
    __shared__ unsigned int index[AOTX_MODEL_PICK_MAX];
    __shared__ float t_min[AOTX_MODEL_PICK_MAX], t_mass[AOTX_MODEL_PICK_MAX], t_heat[AOTX_MODEL_PICK_MAX];
    __shared__ float s_top, s_sum, s_cut, s_lo, s_hi;
    __shared__ unsigned int s_more, s_position, s_slot;

    const unsigned int tid = threadIdx.x;
    const unsigned int r = blockIdx.x;
    const aotx_model_run *run = a.run;
    unsigned int rows = run ? run->rows : (a.rows_dev ? *a.rows_dev : a.rows);
    int *token_out = run ? run->token : a.token;
    unsigned int *draw_out = run ? run->draw : a.draw;
    if (r >= rows || token_out == nullptr) return;
    if (run && run->select != AOTX_MODEL_ROWS_LAST) return;
    const float *row = a.logits + (unsigned long long)r * a.ld;
    const unsigned int vocab = a.vocab;
    unsigned int agent = run ? run->agent[r] : a.agent[r];
    if (agent >= AOTX_SLOTS) agent = 0u;

    const aotx_model_how *how = run ? run->how : a.how;
    unsigned int want_k = run ? run->top_k : a.top_k;
    float want_p = run ? run->top_p : a.top_p;
    float warmth = run ? run->temperature : a.temperature;
    unsigned long long stream = run ? run->seed : a.seed;
    float min_p = 0.0f;
    if (how != nullptr) {
        want_k = how[r].top_k;
        want_p = how[r].top_p;
        warmth = how[r].temperature;
        stream = how[r].seed;
        min_p = how[r].min_p;
    }

    /* largest logit and its place, from the slices of aotx_argmax_kernel */
    if (tid < 64u) {
        float best;
        unsigned int at;
        aotx_pick_top(a, r, best, at);
        if (tid == 0u) {
            s_top = best;
            mark[0] = at;
            s_position = atomicAdd(&a.state->draw[agent], 1u);
            if (draw_out != nullptr) draw_out[r] = s_position;
        }
    }
    __syncthreads();
    const float top = s_top;
    const unsigned int position = s_position;
    if (warmth <= 0.0f) {
        if (tid == 0u) token_out[r] = (int)mark[0];
        return;
    }

    /* the row sum of exp(v - top) in the reference's order (thread t: tokens t, t + 256,
     * ...; then thread 0 over the threads), from the stored exponentials */
    const float *ex = a.ex + (unsigned long long)r * vocab;
    float row_total = 0.0f;
#pragma unroll 64
    for (unsigned int i = tid; i < vocab; i += PICK_THREADS) row_total += ex[i];
    part[tid] = row_total;
    /* the first pass's counts, handed back to zero for the next call */
    unsigned int *h = a.hist + (unsigned long long)r * PICK_BUCKETS;
    for (unsigned int i = tid; i < PICK_BUCKETS; i += PICK_THREADS) {
        bucket[i] = h[i];
        h[i] = 0u;
    }
    __syncthreads();

    /* bucket search for the cut: pass 0 counted by aotx_pick_exp_kernel, later passes
     * here over the narrowed band */
    float lo = -AOTX_MODEL_PICK_SPAN;
    float hi = 0.0f;
    for (unsigned int pass = 0u; pass < PICK_PASSES; ++pass) {
        float band = hi - lo;
        if (pass != 0u) {
            for (unsigned int i = tid; i < PICK_BUCKETS; i += PICK_THREADS) bucket[i] = 0u;
            __syncthreads();
            /* counts: any order, so 16-byte loads where the row allows */
            const bool aligned = ((unsigned long long)row & 15ull) == 0ull;
            const unsigned int body = aligned ? vocab / 4u * 4u : 0u;
            if (aligned) {
                const float4 *row4 = (const float4 *)row;
#pragma unroll 16
                for (unsigned int i4 = tid; i4 < vocab / 4u; i4 += PICK_THREADS) {
                    const float4 f = row4[i4];
                    const float fs[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float scaled = fs[e] - top;
                        if (scaled >= lo && scaled <= hi) {
                            unsigned int b = (unsigned int)((scaled - lo) * (float)PICK_BUCKETS / band);
                            if (b >= PICK_BUCKETS) b = PICK_BUCKETS - 1u;
                            atomicAdd(&bucket[b], 1u);
                        }
                    }
                }
            }
            for (unsigned int i = body + tid; i < vocab; i += PICK_THREADS) {
                float scaled = row[i] - top;
                if (scaled >= lo && scaled <= hi) {
                    unsigned int b = (unsigned int)((scaled - lo) * (float)PICK_BUCKETS / band);
                    if (b >= PICK_BUCKETS) b = PICK_BUCKETS - 1u;
                    atomicAdd(&bucket[b], 1u);
                }
            }
            __syncthreads();
        }
        if (tid == 0u) {
            if (pass == 0u) {
                float sum = 0.0f;
#pragma unroll 16
                for (unsigned int i = 0u; i < PICK_THREADS; ++i) sum += part[i];
                s_sum = sum;
            }
            unsigned int held = 0u;
            s_more = 0u;
            s_cut = lo;
#pragma unroll 8
            for (unsigned int b = PICK_BUCKETS; b != 0u; --b) {
                if (held + bucket[b - 1u] > AOTX_MODEL_PICK_MAX) {
                    s_cut = lo + band * (float)b / (float)PICK_BUCKETS;
                    if (held == 0u) {
                        s_more = 1u;
                        s_lo = lo + band * (float)(b - 1u) / (float)PICK_BUCKETS;
                        s_hi = s_cut;
                    }
                    break;
                }
                held += bucket[b - 1u];
            }
        }
        __syncthreads();
        if (s_more == 0u) break;
        lo = s_lo;
        hi = s_hi;
        __syncthreads();
    }

    /* candidates at or above the cut. The sort below orders them by (value, id), a total
     * order, so while they fit the 256 places their order of placement does not matter:
     * one coalesced pass gives each the next free place (an LDS counter). Only when more
     * pass the cut (logits equal to within the finest band, where the reference keeps
     * whichever arrive first) are the 256 lowest token ids kept instead: each thread takes
     * a contiguous run of tokens and a prefix over the threads places them in token order. */
    const float cut = s_cut;
    if (tid == 0u) s_slot = 0u;
    __syncthreads();
    {
        /* one coalesced pass: every candidate takes the next place while places remain */
        const unsigned int v4 = vocab / 4u;
        const float4 *row4 = (const float4 *)row;
        const bool aligned = ((unsigned long long)row & 15ull) == 0ull;
        const unsigned int body = aligned ? v4 * 4u : 0u;
        if (aligned) {
#pragma unroll 16
            for (unsigned int i4 = tid; i4 < v4; i4 += PICK_THREADS) {
                const float4 f = row4[i4];
                const float fs[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float scaled = fs[e] - top;
                    if (scaled >= cut) {
                        const unsigned int slot = atomicAdd(&s_slot, 1u);
                        if (slot < AOTX_MODEL_PICK_MAX) {
                            value[slot] = scaled;
                            index[slot] = i4 * 4u + (unsigned int)e;
                        }
                    }
                }
            }
        }
        for (unsigned int i = body + tid; i < vocab; i += PICK_THREADS) {
            const float scaled = row[i] - top;
            if (scaled >= cut) {
                const unsigned int slot = atomicAdd(&s_slot, 1u);
                if (slot < AOTX_MODEL_PICK_MAX) {
                    value[slot] = scaled;
                    index[slot] = i;
                }
            }
        }
    }
    __syncthreads();
    unsigned int count = s_slot;
    if (count <= AOTX_MODEL_PICK_MAX) {
        /* all placed */
    } else {
        const unsigned int per = (vocab + PICK_THREADS - 1u) / PICK_THREADS;
        const unsigned int first = tid * per;
        const unsigned int after = first + per < vocab ? first + per : vocab;
        unsigned int run_mine = 0u;
        for (unsigned int i = first; i < after; ++i) {
            if (row[i] - top >= cut) run_mine += 1u;
        }
        __syncthreads();
        mark[tid] = run_mine;
        __syncthreads();
        if (tid == 0u) {
            unsigned int run = 0u;
            for (unsigned int i = 0u; i < PICK_THREADS; ++i) {
                unsigned int c = mark[i];
                mark[i] = run;
                run += c;
            }
        }
        __syncthreads();
        unsigned int slot = mark[tid];
        for (unsigned int i = first; i < after; ++i) {
            float scaled = row[i] - top;
            if (scaled >= cut) {
                if (slot < AOTX_MODEL_PICK_MAX) {
                    value[slot] = scaled;
                    index[slot] = i;
                }
                slot += 1u;
            }
        }
        count = AOTX_MODEL_PICK_MAX;
    }
    for (unsigned int i = tid; i < AOTX_MODEL_PICK_MAX; i += PICK_THREADS) {
        if (i >= count) {
            value[i] = -INFINITY;
            index[i] = 0xFFFFFFFFu;
        }
    }
    __syncthreads();

    /* bitonic sort, largest first, ties to the lower id */
    for (unsigned int span = 2u; span <= AOTX_MODEL_PICK_MAX; span <<= 1) {
        for (unsigned int step = span >> 1; step != 0u; step >>= 1) {
            unsigned int i = tid;
            unsigned int other = i ^ step;
            if (other > i && i < AOTX_MODEL_PICK_MAX) {
                bool down = (i & span) == 0u;
                float vi = value[i], vo = value[other];
                unsigned int ii = index[i], io = index[other];
                bool o_first = vo > vi || (vo == vi && io < ii);  /* other ranks ahead */
                bool i_first = vi > vo || (vi == vo && ii < io);
                bool swap = down ? o_first : i_first;
                if (swap) {
                    value[i] = vo;
                    index[i] = io;
                    value[other] = vi;
                    index[other] = ii;
                }
            }
            __syncthreads();
        }
    }
    /* the per-candidate terms of the serial loops below, each the same expression as
     * there, computed by all threads; thread 0 then adds them in candidate order */
    const float heat = warmth;
    {
        const float v0 = value[0];
        const float total = s_sum;
        for (unsigned int i = tid; i < AOTX_MODEL_PICK_MAX; i += PICK_THREADS) {
            t_min[i] = expf(value[i] - v0);
            t_mass[i] = expf(value[i]) / total;
            t_heat[i] = expf((value[i] - v0) / heat);
        }
    }
    __syncthreads();
    if (tid != 0u) return;

    unsigned int keep = (want_k == 0u || want_k > count) ? count : want_k;
    if (min_p > 0.0f && min_p <= 1.0f) {
        unsigned int min_keep = 1u;
        for (unsigned int i = 1u; i < keep; ++i) {
            if (t_min[i] < min_p) break;
            min_keep = i + 1u;
        }
        keep = min_keep;
    }
    float limit = (want_p <= 0.0f || want_p > 1.0f) ? 1.0f : want_p;
    float mass = 0.0f;
    unsigned int taken = 0u;
#pragma unroll 8
    for (unsigned int i = 0u; i < keep; ++i) {
        mass += t_mass[i];
        taken = i + 1u;
        if (mass >= limit) break;
    }
    float heat_total = 0.0f;
#pragma unroll 8
    for (unsigned int i = 0u; i < taken; ++i) heat_total += t_heat[i];
    aotx_u32x4 word = aotx_philox_dev(position, 0u, 0u, agent, (unsigned int)stream,
                                      (unsigned int)(stream >> 32));
    float pick = (float)(word.x >> 8) * (1.0f / 16777216.0f) * heat_total;
    float walk = 0.0f;
    unsigned int chosen = index[0];
    for (unsigned int i = 0u; i < taken; ++i) {
        walk += t_heat[i];
        chosen = index[i];
        if (walk >= pick) break;
    }
    token_out[r] = (int)chosen;
}

size_t aotx_pick_scratch(unsigned int rows, unsigned int vocab)
{
    return (size_t)rows * (PICK_CHUNKS * 2u + PICK_BUCKETS) * sizeof(unsigned int)
         + (size_t)rows * vocab * sizeof(float);
}

void aotx_launch_pick(const float *logits, unsigned int ld, unsigned int vocab,
                      const unsigned int *rows_dev, unsigned int rows,
                      const unsigned int *agent, const aotx_model_how *how,
                      unsigned int top_k, float top_p, float temperature,
                      unsigned long long seed, int *token, unsigned int *draw,
                      const aotx_model_run *run, unsigned int *best, hipStream_t s)
{
    aotx_pick_args a;
    a.logits = logits;
    a.ld = ld;
    a.vocab = vocab;
    a.rows_dev = rows_dev;
    a.rows = rows;
    a.agent = agent;
    a.how = how;
    a.top_k = top_k;
    a.top_p = top_p;
    a.temperature = temperature;
    a.seed = seed;
    a.token = token;
    a.draw = draw;
    a.state = aotx_state_device();
    a.run = run;
    a.best = best;
    a.hist = best + (size_t)rows * PICK_CHUNKS * 2u;
    a.ex = (float *)(a.hist + (size_t)rows * PICK_BUCKETS);
    hipLaunchKernelGGL(aotx_argmax_kernel, dim3(PICK_CHUNKS, rows), dim3(PICK_THREADS), 0, s, a);
    AOTX_LAUNCH_CHECK();
    hipLaunchKernelGGL(aotx_pick_exp_kernel, dim3(PICK_EXP_WGS, rows), dim3(PICK_THREADS), 0, s, a);
    AOTX_LAUNCH_CHECK();
    hipLaunchKernelGGL(aotx_pick_kernel, dim3(rows), dim3(PICK_THREADS), 0, s, a);
    AOTX_LAUNCH_CHECK();
}

extern "C" int aotx_pick(const float *logits, unsigned int rows, unsigned int vocab,
                         const unsigned int *agent, const aotx_model_how *how,
                         unsigned int top_k, float top_p, float temperature,
                         unsigned long long seed, int *token, unsigned int *draw, void *stream)
{
    if (logits == nullptr || agent == nullptr || token == nullptr || rows == 0u || vocab == 0u)
        return 1;
    unsigned int *best = (unsigned int *)aotx_scratch(AOTX_SCRATCH_PICK, aotx_pick_scratch(rows, vocab));
    aotx_launch_pick(logits, vocab, vocab, nullptr, rows, agent, how, top_k, top_p,
                     temperature, seed, token, draw, nullptr, best, aotx_stream(stream));
    return 0;
}

extern "C" int aotx_philox(const unsigned int *ctr, const unsigned int *key, unsigned int n,
                           unsigned int *out, void *stream)
{
    if (ctr == nullptr || key == nullptr || out == nullptr) return 1;
    if (n == 0u) return 0;
    hipLaunchKernelGGL(aotx_philox_kernel, dim3((n + 255u) / 256u), dim3(256), 0,
                       aotx_stream(stream), ctr, key, n, out);
    AOTX_LAUNCH_CHECK();
    return 0;
}
