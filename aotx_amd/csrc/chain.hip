/* The layer chain: one launch for every layer of a narrow decode step.
 *
 * Reference: the per-layer kernel sequence of cuda/model/graph_host.cu:52-153, which
 * launches each product and the attention as kernels of its own. Here the same bodies
 * (rgemv_dev.h, attention_dev.h) run as stages of one persistent launch:
 *   - the grid is exactly the workgroups the device holds at once (one per CU), so every
 *     workgroup a wait depends on is running;
 *   - a workgroup issues an item's weight loads, then waits for the stage the item reads
 *     (an arrival count of that stage's items), then stages its x and computes;
 *   - results that later stages read are written and read with device-scope accesses
 *     (coherent.h), and each item's stores complete before its arrival is counted;
 *   - every wait is bounded in time: past it the chain sets the stall word and stops
 *     waiting (the results are then wrong and the step reports an error), so every wave
 *     of the grid always reaches the end;
 *   - the last workgroup to leave puts the counters back to zero for the next launch.
 */
#include "chain.h"
#include "rgemv_dev.h"

/* A wait gives up after this many ticks of the 100 MHz real-time counter (20 ms). */
#define CHAIN_SPIN_TICKS 2000000ull

struct aotx_chain_wait {
    const unsigned int *count;   /* null: no wait */
    unsigned int target;
    unsigned int *stall_dev;     /* device word: a wait has given up */
    unsigned int *stall;         /* host-visible copy */
    bool seen;                   /* this workgroup has already seen the stage complete */
    __device__ __forceinline__ void operator()()
    {
        if (seen) return;
        seen = true;
        if (count == nullptr) return;
        if (threadIdx.x == 0u) {
            const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
            while (__hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                if (__hip_atomic_load(stall_dev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
                    break;
                if (__builtin_amdgcn_s_memrealtime() - t0 > CHAIN_SPIN_TICKS) {
                    __hip_atomic_store(stall_dev, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(stall, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
    }
};

/* A stage field read through the scalar cache (the table is constant for the launch). */
template <class T>
static __device__ __forceinline__ T chain_const(const T *p)
{
    T v;
    __builtin_memcpy(&v, (const __attribute__((address_space(4))) T *)p, sizeof v);
    return v;
}

/* A pointer of the stage table marked as global memory: the loads through it are then
 * global (vector memory) loads, as in the standalone kernels, not flat loads that would
 * also count against the LDS wait counter. */
template <class T>
static __device__ __forceinline__ T *chain_g(T *p)
{
    return (T *)(__attribute__((address_space(1))) T *)p;
}

static __device__ __forceinline__ aotx_rgemv_args chain_gemv(const aotx_chain_stage *st)
{
    aotx_rgemv_args g = chain_const(&st->g);
    for (int i = 0; i < 3; ++i) g.w[i] = chain_g(g.w[i]);
    g.x = chain_g(g.x);
    g.resid = chain_g(g.resid);
    g.norm_w = chain_g(g.norm_w);
    g.sumsq = chain_g(g.sumsq);
    g.y = chain_g(g.y);
    g.partial = chain_g(g.partial);
    g.count = chain_g(g.count);
    g.sumsq_out = chain_g(g.sumsq_out);
    g.qkv.qh = chain_g(g.qkv.qh);
    g.qkv.pos = chain_g(g.qkv.pos);
    g.qkv.agent = chain_g(g.qkv.agent);
    g.qkv.state = chain_g(g.qkv.state);
    g.qkv.factor = chain_g(g.qkv.factor);
    return g;
}

static __device__ __forceinline__ aotx_attn_args chain_attn(const aotx_chain_stage *st)
{
    aotx_attn_args t = chain_const(&st->t);
    t.q = chain_g(t.q);
    t.out = chain_g(t.out);
    t.pos = chain_g(t.pos);
    t.agent = chain_g(t.agent);
    t.state = chain_g(t.state);
    t.partial = chain_g(t.partial);
    t.count = chain_g(t.count);
    return t;
}

/* One attention item; returns whether the workgroup has now seen the stage it depends on
 * complete. */

static __device__ __forceinline__ bool chain_attend(const aotx_chain_stage *st, unsigned int it,
                                                    aotx_chain_wait w)
{
    const aotx_attn_args t = chain_attn(st);
    aotx_attend_body<128, 4, 8, true>(t, it, w);
    return w.seen;
}

__global__ __launch_bounds__(512) void aotx_chain_kernel(const aotx_chain_stage *table,
                                                         unsigned int n, unsigned int *done,
                                                         unsigned int *stall)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    __shared__ unsigned int leaving;
    unsigned int *const stall_dev = done + n + 1u;
    for (unsigned int s = 0; s < n; ++s) {
        const aotx_chain_stage *st = table + s;
        const unsigned int kind = chain_const(&st->kind);
        const unsigned int items = chain_const(&st->items);
        const unsigned int wait_on = chain_const(&st->wait);
        aotx_chain_wait w;
        w.count = wait_on != 0u ? chain_g(done + (wait_on - 1u)) : nullptr;
        w.target = chain_const(&st->wait_items);
        w.stall_dev = chain_g(stall_dev);
        w.stall = stall;
        w.seen = false;
        unsigned int mine = 0u;
        if (kind == AOTX_CHAIN_TILE) {
            const aotx_rgemv_args g = chain_gemv(st);
            mine = rg_chain_stage<16, 1, 2, 8>(g, blockIdx.x, gridDim.x, items, lds, w);
        } else if (kind == AOTX_CHAIN_TILE_LONG) {
            const aotx_rgemv_args g = chain_gemv(st);
            mine = rg_chain_stage<16, 1, 7, 8>(g, blockIdx.x, gridDim.x, items, lds, w);
        } else if (kind == AOTX_CHAIN_PAIR) {
            const aotx_rgemv_args g = chain_gemv(st);
            mine = rg_chain_stage<16, 2, 2, 8>(g, blockIdx.x, gridDim.x, items, lds, w);
        } else {
            for (unsigned int it = blockIdx.x; it < items; it += gridDim.x, ++mine)
                w.seen = chain_attend(st, it, w);
        }
        /* this workgroup's stores of the stage have completed before its items are counted */
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0u && mine != 0u) atomicAdd(done + s, mine);
    }
    /* the last workgroup to leave clears the counters (every wait is over by then) */
    __syncthreads();
    if (threadIdx.x == 0u) leaving = atomicAdd(done + n, 1u) == gridDim.x - 1u ? 1u : 0u;
    __syncthreads();
    if (leaving != 0u)
        for (unsigned int i = threadIdx.x; i < n + 2u; i += blockDim.x)
            __hip_atomic_store(done + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

unsigned int aotx_chain_grid(size_t lds)
{
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, aotx_chain_kernel, 512, lds) != hipSuccess)
        return 0u;
    int dev = 0;
    AOTX_CHECK(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    AOTX_CHECK(hipGetDeviceProperties(&prop, dev));
    if (per_cu < 1) return 0u;
    return (unsigned int)prop.multiProcessorCount;     /* one per CU */
}

void aotx_chain_launch(const aotx_chain_stage *table, unsigned int n, unsigned int *done,
                       unsigned int *stall, size_t lds, hipStream_t stream)
{
    const unsigned int grid = aotx_chain_grid(lds);
    if (grid == 0u) {
        fprintf(stderr, "aotx: the layer chain does not fit the device\n");
        exit(1);
    }
    hipLaunchKernelGGL(aotx_chain_kernel, dim3(grid), dim3(512), lds, stream, table, n, done, stall);
    AOTX_LAUNCH_CHECK();
}
