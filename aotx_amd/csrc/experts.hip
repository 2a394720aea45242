/* Routed experts: router, token grouping per expert, grouped expert products.
 *
 * Reference: aotx_model_expert_route (cuda/model/experts.cu:10-75): logits = fp32 router
 * rows . half x, a softmax over every expert, rank with ties to the lower index, the top
 * `used` ids kept and the full-softmax probability as the weight (no renormalisation);
 * aotx_model_expert_matrix (cuda/model/expert_matrix.cu:8-63) runs one batch-1 product
 * per token per rank, so an expert's weights are read once per token that chose it;
 * aotx_model_expert_add (experts.cu:77-98) adds prob * proj rank by rank with the product
 * rounded before the sum.
 *
 * Here the routed (token, rank) slots are grouped per expert (in slot order), and one
 * launch runs every expert's gate/up product with the SwiGLU epilogue, then one launch
 * every expert's down product: each expert's weights are read once per step, whatever the
 * number of tokens that chose it. The ordered weighted sum is fused into the kernel that
 * adds the residual and norms the next layer's input (norm.hip), or done by
 * aotx_expert_sum_kernel for the kernel-level entry point.
 */
#include "aotx_internal.h"
#include "experts.h"
#include "coherent.h"
#include "gemv.h"

#define ROUTE_THREADS 512u
#define ROUTE_VEC 16u            /* 16-byte router loads in flight per lane per step */
#define ROUTE_HIDDEN_LDS 16384u  /* largest hidden staged in LDS (64 KB of floats) */

/* The router of one token (one workgroup). VEC: x staged once in LDS as floats (16-byte
 * loads), then wave w takes experts w, w + 8, ...: a lane adds the products of its 4-value
 * pieces (piece p = lane + 64 i, in i order), with ROUTE_VEC 16-byte router loads issued
 * before their adds, so a row costs one memory round trip, and the wave adds the lanes'
 * sums; for rows or x not 16-byte aligned, or a hidden past ROUTE_HIDDEN_LDS, lanes take
 * single values straight from memory. Then the softmax over every expert and the rank. */
template <bool VEC>
__global__ __launch_bounds__(ROUTE_THREADS) void aotx_route_kernel(
    const float *router, const unsigned short *x, const unsigned int *m_dev, unsigned int tokens,
    unsigned int hidden, unsigned int experts, unsigned int used, float *prob, unsigned int *ids)
{
    extern __shared__ float xs[];
    __shared__ float logit[AOTX_LAYER_EXPERTS_MAX];
    __shared__ float red[ROUTE_THREADS];
    unsigned int count = m_dev ? *m_dev : tokens;
    unsigned int t = blockIdx.x;
    if (t >= count) return;
    const unsigned int lane = threadIdx.x & 63u;
    const unsigned int wave = threadIdx.x >> 6;
    const unsigned short *xr = x + (unsigned long long)t * hidden;
    if constexpr (VEC) {
        const unsigned int pieces8 = hidden / 8u;
#pragma unroll 4
        for (unsigned int p = threadIdx.x; p < pieces8; p += ROUTE_THREADS) {
            const aotx_u4 v = *(const aotx_u4 *)(xr + 8u * p);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xs[8u * p + 2u * (unsigned int)i] = aotx_h2f((unsigned short)(v[i] & 0xffffu));
                xs[8u * p + 2u * (unsigned int)i + 1u] = aotx_h2f((unsigned short)(v[i] >> 16));
            }
        }
        __syncthreads();
    }
    for (unsigned int e = wave; e < experts; e += ROUTE_THREADS / 64u) {
        const float *row = router + (unsigned long long)e * hidden;
        float dot = 0.0f;
        if constexpr (VEC) {
            const unsigned int pieces = hidden / 4u;
            const aotx_u4 *r4 = (const aotx_u4 *)row;
            for (unsigned int base = 0; base < pieces; base += 64u * ROUTE_VEC) {
                aotx_u4 rv[ROUTE_VEC];
#pragma unroll
                for (unsigned int i = 0; i < ROUTE_VEC; ++i) {
                    const unsigned int pc = base + lane + 64u * i;
                    rv[i] = r4[pc < pieces ? pc : 0u];      /* unconditional; masked below */
                }
#pragma unroll
                for (unsigned int i = 0; i < ROUTE_VEC; ++i) {
                    const unsigned int pc = base + lane + 64u * i;
                    if (pc < pieces) {
                        const float *xv = xs + 4u * pc;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const unsigned int w = rv[i][j];   /* a bit cast of the element
                                                                * itself reads element 0 */
                            dot += __uint_as_float(w) * xv[j];
                        }
                    }
                }
            }
        } else {
            for (unsigned int d = lane; d < hidden; d += 64u) dot += row[d] * aotx_h2f(xr[d]);
        }
        for (int off = 32; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
        if (lane == 0u) logit[e] = dot;
    }
    __syncthreads();
    unsigned int e = threadIdx.x;
    red[e] = e < experts ? logit[e] : -INFINITY;
    __syncthreads();
    for (unsigned int step = ROUTE_THREADS / 2u; step != 0u; step >>= 1) {
        if (e < step) red[e] = fmaxf(red[e], red[e + step]);
        __syncthreads();
    }
    float top = red[0];
    __syncthreads();
    float value = e < experts ? expf(logit[e] - top) : 0.0f;
    red[e] = value;
    __syncthreads();
    for (unsigned int step = ROUTE_THREADS / 2u; step != 0u; step >>= 1) {
        if (e < step) red[e] += red[e + step];
        __syncthreads();
    }
    float total = red[0];
    __syncthreads();
    if (e < experts) {
        value /= total;
        logit[e] = value;
        prob[(unsigned long long)t * experts + e] = value;
    }
    __syncthreads();
    if (e < experts) {
        unsigned int rank = 0u;
        for (unsigned int other = 0u; other < experts; ++other) {
            float c = logit[other];
            rank += (c > value || (c == value && other < e)) ? 1u : 0u;
        }
        if (rank < used) ids[(unsigned long long)t * used + rank] = e;
    }
}

#define GROUP_THREADS 256u
#define GROUP_CHUNK 4096u

/* Routed (token, rank) slots grouped per expert, in slot order, the first `cap` of each
 * expert kept and counted (one workgroup): the slots' expert ids come into LDS a chunk at a
 * time with one round of loads, then wave w takes experts w, w + 4, ... and places 64 slots
 * per step with a ballot and a prefix count. */
__global__ __launch_bounds__(GROUP_THREADS) void aotx_group_kernel(
    const unsigned int *ids, const unsigned int *m_dev, unsigned int tokens, unsigned int used,
    unsigned int experts, unsigned int *list, unsigned int *count, unsigned int cap)
{
    __shared__ unsigned int sid[GROUP_CHUNK];
    __shared__ unsigned int cnt[AOTX_LAYER_EXPERTS_MAX];
    const unsigned int n = (m_dev ? *m_dev : tokens) * used;
    const unsigned int lane = threadIdx.x & 63u;
    const unsigned int wave = threadIdx.x >> 6;
    for (unsigned int e = threadIdx.x; e < experts; e += GROUP_THREADS) cnt[e] = 0u;
    for (unsigned int base = 0u; base < n; base += GROUP_CHUNK) {
        const unsigned int len = n - base < GROUP_CHUNK ? n - base : GROUP_CHUNK;
        __syncthreads();
#pragma unroll 4
        for (unsigned int i = threadIdx.x; i < len; i += GROUP_THREADS) sid[i] = ids[base + i];
        __syncthreads();
        for (unsigned int e = wave; e < experts; e += GROUP_THREADS / 64u) {
            unsigned int c = cnt[e];
            for (unsigned int off = 0u; off < len; off += 64u) {
                const unsigned int s = off + lane;
                const bool match = s < len && sid[s] == e;
                const unsigned long long mask = __ballot(match);
                const unsigned int pos = c + (unsigned int)__popcll(mask & ((1ull << lane) - 1ull));
                if (match && pos < cap) list[(unsigned long long)e * cap + pos] = base + s;
                c += (unsigned int)__popcll(mask);
            }
            if (lane == 0u) cnt[e] = c;
        }
    }
    __syncthreads();
    for (unsigned int e = threadIdx.x; e < experts; e += GROUP_THREADS)
        count[e] = cnt[e] < cap ? cnt[e] : cap;
}

/* out[t][d] = sum over rank of prob * y, rank by rank, each product rounded first. */
__global__ void aotx_expert_sum_kernel(const float *y, const float *prob, const unsigned int *ids,
                                       unsigned int tokens, unsigned int used,
                                       unsigned int experts, unsigned int hidden, float *out)
{
    unsigned int t = blockIdx.x;
    if (t >= tokens) return;
    for (unsigned int d = threadIdx.x; d < hidden; d += blockDim.x) {
        float acc = 0.0f;
        for (unsigned int r = 0; r < used; ++r) {
            unsigned int e = ids[t * used + r];
            float one = __fmul_rn(y[((unsigned long long)t * used + r) * hidden + d],
                                  prob[t * experts + e]);
            acc = r == 0u ? one : __fadd_rn(acc, one);
        }
        out[(unsigned long long)t * hidden + d] = acc;
    }
}

void aotx_launch_group(const unsigned int *ids, const unsigned int *m_dev, unsigned int tokens,
                       unsigned int used, unsigned int experts, unsigned int *list,
                       unsigned int *count, unsigned int cap, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_group_kernel, dim3(1), dim3(GROUP_THREADS), 0, s, ids, m_dev,
                       tokens, used, experts, list, count, cap);
    AOTX_LAUNCH_CHECK();
}

void aotx_launch_route(const float *router, const unsigned short *x, const unsigned int *m_dev,
                       unsigned int tokens, unsigned int hidden, unsigned int experts,
                       unsigned int used, float *prob, unsigned int *ids, hipStream_t s)
{
    const bool vec = ((unsigned long long)router & 15ull) == 0ull && ((unsigned long long)x & 15ull) == 0ull
                  && hidden % 8u == 0u && hidden <= ROUTE_HIDDEN_LDS;
    if (vec)
        hipLaunchKernelGGL(aotx_route_kernel<true>, dim3(tokens), dim3(ROUTE_THREADS),
                           (size_t)hidden * sizeof(float), s, router, x, m_dev, tokens, hidden,
                           experts, used, prob, ids);
    else
        hipLaunchKernelGGL(aotx_route_kernel<false>, dim3(tokens), dim3(ROUTE_THREADS), 0, s, router,
                           x, m_dev, tokens, hidden, experts, used, prob, ids);
    AOTX_LAUNCH_CHECK();
}

int aotx_launch_expert_ffn(const aotx_expert_plan &p, const unsigned short *x,
                           const unsigned int *m_dev, unsigned int tokens,
                           const unsigned int *ids, unsigned short *act, float *y, hipStream_t s)
{
    hipLaunchKernelGGL(aotx_group_kernel, dim3(1), dim3(GROUP_THREADS), 0, s, ids,
                       m_dev, tokens, p.used, p.experts, p.list, p.count, p.cap);
    AOTX_LAUNCH_CHECK();
    /* gate + up with the gated unit, per expert; passes of 32 routed rows */
    const void *gu[2] = {p.gate, p.up};
    unsigned int rows2[2] = {p.ffn, p.ffn};
    aotx_gemv_args a;
    if (aotx_gemv_plan(&a, gu, rows2, 2u, p.hidden, AOTX_EPI_SWIGLU) != 0) return 1;
    a.splits = 1u;
    a.cps = a.chunks;
    a.x = x;
    a.ldx = p.hidden;
    a.y = act;
    a.ldy = p.ffn;
    a.expert_stride = (unsigned long long)p.ffn * (p.hidden / 32u) * 34ull;
    a.list = p.list;
    a.list_count = p.count;
    a.list_cap = p.cap;
    a.xrow_div = p.used;
    a.experts = p.experts;
    unsigned int passes = (tokens + 31u) / 32u;
    for (unsigned int i = 0; i < passes; ++i) {
        aotx_gemv_args q = a;
        q.m0 = 32u * i;
        q.m = 32u;
        if (aotx_gemv_launch(q, s) != 0) return 1;
    }
    /* down, per expert, into the routed slot rows */
    const void *dw[1] = {p.down};
    unsigned int rows1[1] = {p.hidden};
    aotx_gemv_args b;
    if (aotx_gemv_plan(&b, dw, rows1, 1u, p.ffn, AOTX_EPI_F32) != 0) return 1;
    b.splits = 1u;
    b.cps = b.chunks;
    b.x = act;
    b.ldx = p.ffn;
    b.y = y;
    b.ldy = p.hidden;
    b.expert_stride = (unsigned long long)p.hidden * (p.ffn / 32u) * 34ull;
    b.list = p.list;
    b.list_count = p.count;
    b.list_cap = p.cap;
    b.xrow_div = 1u;
    b.experts = p.experts;
    for (unsigned int i = 0; i < passes; ++i) {
        aotx_gemv_args q = b;
        q.m0 = 32u * i;
        q.m = 32u;
        if (aotx_gemv_launch(q, s) != 0) return 1;
    }
    return 0;
}

extern "C" int aotx_expert_route(const float *router, const void *x, unsigned int tokens,
                                 unsigned int hidden, unsigned int experts, unsigned int used,
                                 float *prob, unsigned int *ids, void *stream)
{
    if (router == nullptr || x == nullptr || prob == nullptr || ids == nullptr) return 1;
    if (tokens == 0u || experts == 0u || experts > AOTX_LAYER_EXPERTS_MAX || used == 0u || used > experts)
        return 1;
    aotx_launch_route(router, (const unsigned short *)x, nullptr, tokens, hidden, experts, used,
                      prob, ids, aotx_stream(stream));
    return 0;
}

extern "C" int aotx_expert_ffn(const void *gate, const void *up, const void *down,
                               unsigned int experts, unsigned int used, unsigned int hidden,
                               unsigned int ffn, const void *x, unsigned int tokens,
                               const float *prob, const unsigned int *ids, float *out,
                               void *stream)
{
    if (gate == nullptr || up == nullptr || down == nullptr || x == nullptr || prob == nullptr
        || ids == nullptr || out == nullptr)
        return 1;
    if (tokens == 0u || tokens > AOTX_MODEL_MAX_TOKENS || experts == 0u
        || experts > AOTX_LAYER_EXPERTS_MAX || used == 0u || used > experts)
        return 1;
    if (hidden % 256u != 0u && hidden % 32u != 0u) return 1;
    if (ffn % 32u != 0u || hidden % 32u != 0u) return 1;
    hipStream_t s = aotx_stream(stream);
    size_t slots = (size_t)tokens * used;
    unsigned char *buf = (unsigned char *)aotx_scratch(
        AOTX_SCRATCH_EXPERT, slots * ffn * 2u + slots * hidden * 4u
                             + (size_t)experts * tokens * 4u + experts * 4u + 1024u);
    aotx_expert_plan p;
    p.gate = gate;
    p.up = up;
    p.down = down;
    p.experts = experts;
    p.used = used;
    p.hidden = hidden;
    p.ffn = ffn;
    p.cap = tokens;
    unsigned short *act = (unsigned short *)buf;
    float *y = (float *)(buf + ((slots * ffn * 2u + 255u) & ~(size_t)255u));
    unsigned char *tail = (unsigned char *)y + ((slots * hidden * 4u + 255u) & ~(size_t)255u);
    p.list = (unsigned int *)tail;
    p.count = p.list + (size_t)experts * tokens;
    if (aotx_launch_expert_ffn(p, (const unsigned short *)x, nullptr, tokens, ids, act, y, s) != 0)
        return 1;
    hipLaunchKernelGGL(aotx_expert_sum_kernel, dim3(tokens), dim3(256), 0, s, y, prob, ids, tokens,
                       used, experts, hidden, out);
    AOTX_LAUNCH_CHECK();
    return 0;
}
