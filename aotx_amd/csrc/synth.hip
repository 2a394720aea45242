/* Synthetic weights and activations: the same bytes on the device and on the host. */
#include "aotx_internal.h"
#include "synth.h"

#include <thread>
#include <vector>

__global__ void aotx_synth_q8_kernel(unsigned char *dst, unsigned long long blocks,
                                     float sigma, unsigned long long seed)
{
    for (unsigned long long b = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x;
         b < blocks; b += (unsigned long long)gridDim.x * blockDim.x) {
        unsigned char out[34];
        aotx_synth_block(out, seed, b * 32ull, sigma);
        for (int i = 0; i < 34; ++i) dst[b * 34ull + i] = out[i];
    }
}

__global__ void aotx_synth_f16_kernel(unsigned short *dst, unsigned long long count,
                                      float sigma, unsigned long long seed)
{
    for (unsigned long long i = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x;
         i < count; i += (unsigned long long)gridDim.x * blockDim.x) {
        dst[i] = aotx_f32_to_f16(aotx_synth_normal(seed, i) * sigma);
    }
}

extern "C" int aotx_synth_q8(void *dst, unsigned long long rows, unsigned int k, float sigma,
                             unsigned long long seed, void *stream)
{
    if (dst == nullptr || k % 32u != 0u) return 1;
    unsigned long long blocks = rows * (k / 32u);
    if (blocks == 0ull) return 0;
    hipLaunchKernelGGL(aotx_synth_q8_kernel, dim3(4096), dim3(256), 0, aotx_stream(stream),
                       (unsigned char *)dst, blocks, sigma, seed);
    AOTX_LAUNCH_CHECK();
    return 0;
}

extern "C" int aotx_synth_f16(void *dst, unsigned long long count, float sigma,
                              unsigned long long seed, void *stream)
{
    if (dst == nullptr) return 1;
    if (count == 0ull) return 0;
    hipLaunchKernelGGL(aotx_synth_f16_kernel, dim3(4096), dim3(256), 0, aotx_stream(stream),
                       (unsigned short *)dst, count, sigma, seed);
    AOTX_LAUNCH_CHECK();
    return 0;
}

template <typename F>
static void aotx_parallel(unsigned long long count, unsigned int threads, F fn)
{
    if (threads == 0u) threads = std::thread::hardware_concurrency();
    if (threads == 0u) threads = 1u;
    if (count < 4096ull) threads = 1u;
    std::vector<std::thread> pool;
    unsigned long long per = (count + threads - 1u) / threads;
    for (unsigned int t = 0; t < threads; ++t) {
        unsigned long long lo = per * t;
        unsigned long long hi = lo + per < count ? lo + per : count;
        if (lo >= hi) break;
        pool.emplace_back([=]() { fn(lo, hi); });
    }
    for (auto &th : pool) th.join();
}

extern "C" int aotx_synth_q8_host(void *dst, unsigned long long rows, unsigned int k,
                                  float sigma, unsigned long long seed, unsigned int threads)
{
    if (dst == nullptr || k % 32u != 0u) return 1;
    unsigned long long blocks = rows * (k / 32u);
    unsigned char *out = (unsigned char *)dst;
    aotx_parallel(blocks, threads, [=](unsigned long long lo, unsigned long long hi) {
        for (unsigned long long b = lo; b < hi; ++b) {
            aotx_synth_block(out + b * 34ull, seed, b * 32ull, sigma);
        }
    });
    return 0;
}

extern "C" int aotx_synth_f16_host(void *dst, unsigned long long count, float sigma,
                                   unsigned long long seed, unsigned int threads)
{
    if (dst == nullptr) return 1;
    unsigned short *out = (unsigned short *)dst;
    aotx_parallel(count, threads, [=](unsigned long long lo, unsigned long long hi) {
        for (unsigned long long i = lo; i < hi; ++i) {
            out[i] = aotx_f32_to_f16(aotx_synth_normal(seed, i) * sigma);
        }
    });
    return 0;
}
