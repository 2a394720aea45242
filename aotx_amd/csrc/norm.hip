/* Row kernels of the step: cache positions, embedding gather, residual + RMSNorm, the
 * rotary turn with the page write (general path), and the weighted expert sum.
 *
 * Reference: cuda/model/gather.cu:8-105 (request, open/shut rows, gather, select),
 * cuda/model/norm.cu:49-105 (norm, residual, SwiGLU), cuda/model/rope.cu:128-234 (turn +
 * page write), cuda/model/experts.cu:77-98 (ordered weighted sum). Every kernel that writes
 * the residual stream also leaves the sum of squares of each 16 columns, so a norm needs
 * no pass of its own over the row: the next product stages x = half(scale * resid * w)
 * itself (small batches), or the norm kernel here writes x (larger batches).
 */
#include "aotx_internal.h"
#include "norm.h"

/* Sum over a 256-thread block: per-wave butterfly, then the 4 wave sums in order. */
static __device__ __forceinline__ float aotx_block_sum(float v, float *share)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const unsigned int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63u) == 0u) share[wave] = v;
    __syncthreads();
    float total = 0.0f;
    const unsigned int waves = (blockDim.x + 63u) >> 6;
    for (unsigned int w = 0; w < waves; ++w) total += share[w];
    return total;
}

static __device__ __forceinline__ unsigned int aotx_which(const unsigned int *offset,
                                                          unsigned int seqs, unsigned int row)
{
    unsigned int low = 0u, high = seqs;
    while (low + 1u < high) {
        unsigned int mid = (low + high) / 2u;
        if (offset[mid] <= row) low = mid; else high = mid;
    }
    return low;
}

/* Cache position and slot of every token (cuda/model/gather.cu:29-40 with the bisection
 * of cuda/model/forward.cuh:200-214); also the row each sequence's last token selects. */
__global__ void aotx_rows_kernel(const aotx_step *step, aotx_state *state, unsigned int *pos,
                                 unsigned int *tagent, unsigned int *last)
{
    const aotx_model_run *run = &step->run;
    unsigned int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < run->seqs) {
        last[t] = run->offset[t + 1u] - 1u;
    }
    if (t >= run->tokens) return;
    unsigned int s = aotx_which(run->offset, run->seqs, t);
    unsigned int agent = run->agent[s];
    unsigned int base = agent < AOTX_SLOTS ? state->seen[agent] : 0u;
    pos[t] = base + (t - run->offset[s]);
    tagent[t] = agent;
}

/* Move every slot's cache position on by its tokens (cuda/model/gather.cu:42-51). */
__global__ void aotx_shut_rows_kernel(const aotx_step *step, aotx_state *state)
{
    const aotx_model_run *run = &step->run;
    unsigned int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= run->seqs) return;
    unsigned int agent = run->agent[s];
    if (agent < AOTX_SLOTS) state->seen[agent] += run->offset[s + 1u] - run->offset[s];
}

/* Ask the page cache for the pages of the next pass (cuda/model/gather.cu:8-26) and
 * queue the request as cuda/kvcache/pages.cu:13-36 does: a full queue or a bad slot is
 * refused and counted. One thread per sequence. */
__global__ void aotx_request_kernel(const unsigned int *offset, const unsigned int *agent,
                                    unsigned int seqs, aotx_kvl_shape shape, aotx_state *state)
{
    unsigned int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= seqs) return;
    unsigned int a = agent[s];
    aotx_kv_table *kv = &state->kv;
    if (a >= AOTX_SLOTS) return;
    unsigned int end = state->seen[a] + (offset[s + 1u] - offset[s]);
    unsigned int need = aotx_kvl_pages(shape, end);
    unsigned int held = kv->count[a];
    if (need <= held) return;
    unsigned int pages = need - held;
    if (pages > AOTX_KV_PAGES_EACH) {
        atomicAdd(&kv->refused, 1u);
        return;
    }
    unsigned int at = atomicAdd(&kv->made, 0u);
    for (;;) {
        if (at - atomicAdd(&kv->served, 0u) >= AOTX_KV_QUEUE_MAX) {
            atomicAdd(&kv->refused, 1u);
            return;
        }
        unsigned int was = atomicCAS(&kv->made, at, at + 1u);
        if (was == at) break;
        at = was;
    }
    kv->queue[at & (AOTX_KV_QUEUE_MAX - 1u)].agent = a;
    kv->queue[at & (AOTX_KV_QUEUE_MAX - 1u)].pages = pages;
}

/* Embedding rows into the residual stream (fp32(scale) * q: cuda/model/gather.cu:53-80 with
 * the Q8_0 reader of cuda/model/blocks.cuh:99-105), and the sum of squares of every 16
 * columns for the first layer's norm. One thread per 16 columns. */
__global__ __launch_bounds__(256) void aotx_gather_kernel(const aotx_step *step,
                                                         const unsigned char *table,
                                                         unsigned int embd_type,
                                                         unsigned int hidden, unsigned int vocab,
                                                         float *resid, float *sumsq)
{
    const aotx_model_run *run = &step->run;
    unsigned int t = blockIdx.x;
    if (t >= run->tokens) return;
    int id = run->ids[t];
    unsigned int row = (id < 0 || (unsigned int)id >= vocab) ? 0u : (unsigned int)id;
    float *r = resid + (unsigned long long)t * hidden;
    const unsigned int tiles = (hidden + 15u) / 16u;
    for (unsigned int tile = threadIdx.x; tile < tiles; tile += blockDim.x) {
        /* the tile's 16 values are loaded together (unrolled), then added in column order */
        float v[16];
#pragma unroll
        for (unsigned int e = 0; e < 16u; ++e) {
            const unsigned int d = tile * 16u + e;
            const unsigned int dc = d < hidden ? d : hidden - 1u;
            if (embd_type == AOTX_WEIGHT_Q8_0) {
                const unsigned char *blk = table + ((unsigned long long)row * (hidden / 32u) + dc / 32u) * 34ull;
                const float scale = aotx_h2f((unsigned short)(blk[0] | (blk[1] << 8)));
                v[e] = scale * (float)(int)(signed char)blk[2u + dc % 32u];
            } else if (embd_type == AOTX_WEIGHT_F16) {
                v[e] = aotx_h2f(((const unsigned short *)table)[(unsigned long long)row * hidden + dc]);
            } else {
                v[e] = ((const float *)table)[(unsigned long long)row * hidden + dc];
            }
        }
        float sum = 0.0f;
#pragma unroll
        for (unsigned int e = 0; e < 16u; ++e) {
            const unsigned int d = tile * 16u + e;
            if (d < hidden) {
                r[d] = v[e];
                sum += v[e] * v[e];
            }
        }
        sumsq[(unsigned long long)t * tiles + tile] = sum;
    }
}

/* x = half(rsqrt(sum/h + eps) * resid * w) (cuda/model/norm.cu:49-77), with the row sum
 * taken from the 16-column partial sums left by the kernel that last wrote the residual.
 * Grid (tokens, column blocks of 1024). The selected head rows also go to sel. */
__global__ __launch_bounds__(256) void aotx_norm_kernel(aotx_norm_args a)
{
    __shared__ float share[4];
    unsigned int tokens = *a.m_dev;
    unsigned int t = blockIdx.x;
    if (t >= tokens) return;
    const unsigned int h = a.hidden;
    const unsigned int tiles = (h + 15u) / 16u;
    const float *ss = a.sumsq + (unsigned long long)t * tiles;
    float sum = 0.0f;
    for (unsigned int i = threadIdx.x; i < tiles; i += blockDim.x) sum += ss[i];
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    if ((threadIdx.x & 63u) == 0u) share[threadIdx.x >> 6] = sum;
    __syncthreads();
    sum = share[0] + share[1] + share[2] + share[3];
    const float scale = rsqrtf(sum / (float)h + a.eps);
    int selected = -1;
    if (a.sel != nullptr && a.last != nullptr && a.step != nullptr) {
        if (a.step->run.select == AOTX_MODEL_ROWS_ALL) {
            selected = (int)t;
        } else {
            const unsigned int seqs = a.step->run.seqs;
            for (unsigned int s = 0; s < seqs; ++s) if (a.last[s] == t) { selected = (int)s; break; }
        }
    }
    const float *r = a.resid + (unsigned long long)t * h;
    const unsigned int d0 = blockIdx.y * 1024u;
    for (unsigned int d = d0 + threadIdx.x; d < h && d < d0 + 1024u; d += blockDim.x) {
        unsigned short hv = aotx_f2h(scale * r[d] * a.norm_w[d]);
        if (a.x != nullptr)
            a.x[a.x_frag ? aotx_xfrag_at(t, d) : (unsigned long long)t * h + d] = hv;
        if (selected >= 0) a.sel[(unsigned long long)selected * h + d] = hv;
    }
}

/* resid += the routed experts' weighted sum, rank by rank with each product rounded before
 * it adds (cuda/model/experts.cu:77-98), then the 16-column sums of squares. Grid (tokens,
 * column blocks of 256); 16 consecutive threads own one 16-column tile. */
__global__ __launch_bounds__(256) void aotx_expert_resid_kernel(aotx_expert_resid_args a)
{
    unsigned int tokens = *a.m_dev;
    unsigned int t = blockIdx.x;
    if (t >= tokens) return;
    const unsigned int h = a.hidden;
    const unsigned int d = blockIdx.y * 256u + threadIdx.x;
    float v2 = 0.0f;
    if (d < h) {
        float acc = 0.0f;
        for (unsigned int rk = 0; rk < a.used; ++rk) {
            unsigned int e = a.ids[t * a.used + rk];
            float p = a.prob[t * a.experts + e];
            float one = __fmul_rn(a.y[((unsigned long long)t * a.used + rk) * h + d], p);
            acc = rk == 0u ? one : __fadd_rn(acc, one);
        }
        float v = a.resid[(unsigned long long)t * h + d] + acc;
        a.resid[(unsigned long long)t * h + d] = v;
        v2 = v * v;
    }
    /* 16 lanes in order: a fixed butterfly */
    v2 += __shfl_xor(v2, 1, 64);
    v2 += __shfl_xor(v2, 2, 64);
    v2 += __shfl_xor(v2, 4, 64);
    v2 += __shfl_xor(v2, 8, 64);
    if ((threadIdx.x & 15u) == 0u && d < h) a.sumsq[(unsigned long long)t * ((h + 15u) / 16u) + d / 16u] = v2;
}

/* Head norm (optional), rotary turn and page write of one (token, head) from fp32 q/k/v
 * rows (cuda/model/rope.cu:128-196, :200-234); the general path for the split pair rule
 * and the head-norm layer kind. Block = d/2 threads (at least 32). */
__global__ void aotx_rope_kernel(aotx_rope_args a)
{
    __shared__ float share[4];
    unsigned int tokens = *a.m_dev;
    unsigned int t = blockIdx.x;
    unsigned int head = blockIdx.y;
    if (t >= tokens || head >= a.heads + a.kv_heads) return;
    const unsigned int d = a.head_dim;
    const unsigned int half_dim = d / 2u;
    const bool is_q = head < a.heads;
    const unsigned int kh = is_q ? 0u : head - a.heads;
    const float *src = is_q ? a.q + (unsigned long long)t * a.ld + (unsigned long long)head * d
                            : a.k + (unsigned long long)t * a.ld + (unsigned long long)kh * d;
    const float *nw = is_q ? a.q_norm : a.k_norm;
    const unsigned int position = a.pos[t];
    float scale = 1.0f;
    if (nw != nullptr) {
        float sum = 0.0f;
        for (unsigned int i = threadIdx.x; i < d; i += blockDim.x) sum += src[i] * src[i];
        sum = aotx_block_sum(sum, share);
        scale = rsqrtf(sum / (float)d + a.eps);
    }
    unsigned short *dst;
    if (is_q) {
        dst = a.qh + ((unsigned long long)t * a.heads + head) * d;
    } else {
        unsigned char *blk = aotx_kvl_block(a.shape, &a.state->kv, a.agent[t], a.layer, position);
        if (blk == nullptr) {
            if (threadIdx.x == 0u) atomicAdd(&a.state->faults, 1u);
            return;
        }
        unsigned short *vrow = (unsigned short *)blk
            + (unsigned long long)((a.kv_heads + kh) * AOTX_KVL_BLOCK + position % AOTX_KVL_BLOCK) * d;
        const float *vsrc = a.v + (unsigned long long)t * a.ld + (unsigned long long)kh * d;
        for (unsigned int i = threadIdx.x; i < d; i += blockDim.x) vrow[i] = aotx_f2h(vsrc[i]);
        dst = (unsigned short *)blk
            + (unsigned long long)(kh * AOTX_KVL_BLOCK + position % AOTX_KVL_BLOCK) * d;
    }
    const float step = powf(a.theta, -2.0f / (float)d);
    for (unsigned int i = threadIdx.x; i < half_dim; i += blockDim.x) {
        unsigned int lo = a.pairs == AOTX_ROPE_PAIRS_ADJACENT ? 2u * i : i;
        unsigned int hi = a.pairs == AOTX_ROPE_PAIRS_ADJACENT ? 2u * i + 1u : i + half_dim;
        float x0 = src[lo], x1 = src[hi];
        if (nw != nullptr) {
            x0 = scale * x0 * nw[lo];
            x1 = scale * x1 * nw[hi];
        }
        float angle = (float)position * powf(step, (float)i);
        if (a.factor != nullptr) angle = angle / a.factor[i];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        dst[lo] = aotx_f2h(x0 * cs - x1 * sn);
        dst[hi] = aotx_f2h(x0 * sn + x1 * cs);
    }
}

/* ---------------------------------------------------------------------------------------
 * Host launchers
 * ------------------------------------------------------------------------------------- */
/* Residual capture of the probe (cuda/model/conduct.cu:99-178, the capture at :165-173):
 * after layer `layer`, the residual row of each sequence's last token goes to capture
 * slot c for every c whose named layer is this one, laid out [c][seq][hidden]. One block
 * per sequence. (The reference adds registered steer vectors in the same kernel; this
 * build has no steer registry, so there is nothing to add, as in the reference with no
 * vector registered.) */
__global__ __launch_bounds__(256) void aotx_capture_kernel(const aotx_step *step,
                                                           const float *resid,
                                                           unsigned int hidden,
                                                           unsigned int layer)
{
    const aotx_model_run *run = &step->run;
    const unsigned int s = blockIdx.x;
    if (run->capture == nullptr || s >= run->seqs) return;
    const unsigned int row = run->offset[s + 1u] - 1u;
    if (row >= run->tokens) return;
    const float *src = resid + (unsigned long long)row * hidden;
    for (unsigned int c = 0; c < run->capture_count; ++c) {
        if (run->capture_layer[c] != layer) continue;
        float *dst = run->capture + ((unsigned long long)c * run->seqs + s) * hidden;
        for (unsigned int d = threadIdx.x; d < hidden; d += blockDim.x) dst[d] = src[d];
    }
}

/* The embedding head (cuda/embed/embed.cu:8-65): for each sequence, its last residual row
 * under the last RMSNorm in fp32, scaled to unit length, into pooled[seq][hidden]. One
 * block per sequence. */
__global__ __launch_bounds__(256) void aotx_pool_kernel(const aotx_step *step, const float *resid,
                                                        const float *norm_w, unsigned int hidden,
                                                        float eps)
{
    __shared__ float share[4];
    const aotx_model_run *run = &step->run;
    const unsigned int s = blockIdx.x;
    if (run->pooled == nullptr || s >= run->seqs) return;
    const unsigned int row = run->offset[s + 1u] - 1u;
    if (row >= run->tokens) return;
    const float *r = resid + (unsigned long long)row * hidden;
    float sq = 0.0f;
    for (unsigned int d = threadIdx.x; d < hidden; d += blockDim.x) sq += r[d] * r[d];
    const float scale = rsqrtf(aotx_block_sum(sq, share) / (float)hidden + eps);
    float len = 0.0f;
    for (unsigned int d = threadIdx.x; d < hidden; d += blockDim.x) {
        const float v = scale * r[d] * norm_w[d];
        len += v * v;
    }
    len = aotx_block_sum(len, share);
    const float unit = len > 0.0f ? rsqrtf(len) : 0.0f;
    float *out = run->pooled + (unsigned long long)s * hidden;
    for (unsigned int d = threadIdx.x; d < hidden; d += blockDim.x)
        out[d] = scale * r[d] * norm_w[d] * unit;
}

/* One weight of a row of the class head: Q8_0 blocks (fp32 scale times the quant, as the
 * reference's reader cuda/model/blocks.cuh:96-105), fp16 or fp32. */
static __device__ __forceinline__ float aotx_cls_at(const unsigned char *w, unsigned int type,
                                                    unsigned long long i)
{
    if (type == AOTX_WEIGHT_Q8_0) {
        const unsigned char *b = w + (i / 32ull) * 34ull;
        const float scale = aotx_h2f((unsigned short)(b[0] | (b[1] << 8)));
        return scale * (float)(int)(signed char)b[2u + (unsigned int)(i % 32ull)];
    }
    if (type == AOTX_WEIGHT_F16) return aotx_h2f(((const unsigned short *)w)[i]);
    return ((const float *)w)[i];
}

/* The rank head (cuda/rerank/rerank.cu:8-81): the last residual row of each sequence
 * under the last RMSNorm in fp32, against the two class rows (yes, no), and the score
 * softmax(yes, no)[0] into score[seq]. One block per sequence. */
__global__ __launch_bounds__(256) void aotx_score_kernel(const aotx_step *step, const float *resid,
                                                         const float *norm_w,
                                                         const unsigned char *cls,
                                                         unsigned int type, unsigned int hidden,
                                                         float eps)
{
    __shared__ float share[4];
    const aotx_model_run *run = &step->run;
    const unsigned int s = blockIdx.x;
    if (run->score == nullptr || s >= run->seqs) return;
    const unsigned int row = run->offset[s + 1u] - 1u;
    if (row >= run->tokens) return;
    const float *r = resid + (unsigned long long)row * hidden;
    float sq = 0.0f;
    for (unsigned int d = threadIdx.x; d < hidden; d += blockDim.x) sq += r[d] * r[d];
    const float scale = rsqrtf(aotx_block_sum(sq, share) / (float)hidden + eps);
    float yes = 0.0f, no = 0.0f;
    for (unsigned int d = threadIdx.x; d < hidden; d += blockDim.x) {
        const float v = scale * r[d] * norm_w[d];
        yes += v * aotx_cls_at(cls, type, d);
        no += v * aotx_cls_at(cls, type, (unsigned long long)hidden + d);
    }
    yes = aotx_block_sum(yes, share);
    no = aotx_block_sum(no, share);
    if (threadIdx.x != 0u) return;
    const float top = fmaxf(yes, no);
    const float ey = expf(yes - top), en = expf(no - top);
    run->score[s] = ey / (ey + en);
}

void aotx_launch_rows(const aotx_step *step, unsigned int max_tokens, unsigned int *pos,
                      unsigned int *tagent, unsigned int *last, hipStream_t s)
{
    unsigned int n = max_tokens > AOTX_SLOTS ? max_tokens : AOTX_SLOTS;
    hipLaunchKernelGGL(aotx_rows_kernel, dim3((n + 255u) / 256u), dim3(256), 0, s, step,
                       aotx_state_device(), pos, tagent, last);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_shut_rows(const aotx_step *step, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_shut_rows_kernel, dim3(1), dim3(AOTX_SLOTS), 0, s, step,
                       aotx_state_device());
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_request(const unsigned int *offset, const unsigned int *agent,
                         unsigned int seqs, aotx_kvl_shape shape, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_request_kernel, dim3(1), dim3(AOTX_SLOTS), 0, s, offset, agent, seqs,
                       shape, aotx_state_device());
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_gather(const aotx_step *step, unsigned int max_tokens,
                        const unsigned char *table, unsigned int embd_type,
                        unsigned int hidden, unsigned int vocab, float *resid, float *sumsq,
                        hipStream_t s)
{
    hipLaunchKernelGGL(aotx_gather_kernel, dim3(max_tokens), dim3(256), 0, s, step, table,
                       embd_type, hidden, vocab, resid, sumsq);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_norm(const aotx_norm_args &a, unsigned int max_tokens, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_norm_kernel, dim3(max_tokens, (a.hidden + 1023u) / 1024u), dim3(256), 0,
                       s, a);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_expert_resid(const aotx_expert_resid_args &a, unsigned int max_tokens,
                              hipStream_t s)
{
    hipLaunchKernelGGL(aotx_expert_resid_kernel, dim3(max_tokens, (a.hidden + 255u) / 256u),
                       dim3(256), 0, s, a);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_rope(const aotx_rope_args &a, unsigned int max_tokens, hipStream_t s)
{
    unsigned int threads = a.head_dim / 2u;
    if (threads < 64u) threads = 64u;
    hipLaunchKernelGGL(aotx_rope_kernel, dim3(max_tokens, a.heads + a.kv_heads), dim3(threads), 0,
                       s, a);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_capture(const aotx_step *step, const float *resid, unsigned int hidden,
                         unsigned int layer, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_capture_kernel, dim3(AOTX_SLOTS), dim3(256), 0, s, step, resid, hidden,
                       layer);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_pool(const aotx_step *step, const float *resid, const float *norm_w,
                      unsigned int hidden, float eps, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_pool_kernel, dim3(AOTX_SLOTS), dim3(256), 0, s, step, resid, norm_w,
                       hidden, eps);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_score(const aotx_step *step, const float *resid, const float *norm_w,
                       const unsigned char *cls, unsigned int type, unsigned int hidden,
                       float eps, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_score_kernel, dim3(AOTX_SLOTS), dim3(256), 0, s, step, resid, norm_w,
                       cls, type, hidden, eps);
    AOTX_LAUNCH_CHECK();
}
