/* Word-level accesses shared by the product and attention bodies: 16-byte loads, fp32
 * loads and stores, and a pair of fp16 values written as one 32-bit store. Their
 * producers and consumers are earlier or later launches (a launch boundary makes a result
 * visible to every XCD), so these are ordinary accesses.
 */
#ifndef AOTX_COHERENT_H
#define AOTX_COHERENT_H

#include <hip/hip_runtime.h>

typedef unsigned int aotx_u4 __attribute__((ext_vector_type(4)));

static __device__ __forceinline__ aotx_u4 co_load4(const void *p)
{
    return *(const aotx_u4 *)p;
}

static __device__ __forceinline__ float co_loadf(const float *p)
{
    return *p;
}

static __device__ __forceinline__ void co_storef(float *p, float v)
{
    *p = v;
}

/* Two fp16 values (lo at p[0], hi at p[1]); p is 4-byte aligned. */
static __device__ __forceinline__ void co_store2h(unsigned short *p, unsigned int lo, unsigned int hi)
{
    *(unsigned int *)p = (lo & 0xffffu) | (hi << 16);
}

/* Load one word of every 64-byte line of a kernel's by-value argument block at entry and
 * wait for them once. The compiler spreads the scalar loads of the fields over the
 * prologue, separated by waits for the values it needs first; without this each of those
 * rounds misses the scalar cache and waits for memory again. */
template <typename T>
static __device__ __forceinline__ void aotx_args_touch(const T &a)
{
    typedef const __attribute__((address_space(4))) unsigned int cword;
    cword *p = (cword *)(const void *)&a;
    unsigned int x = 0u;
#pragma unroll
    for (unsigned int i = 0; i < (sizeof(T) + 63u) / 64u; ++i) x ^= p[i * 16u];
    asm volatile("" ::"s"(x));
}

#endif
