/* Accesses to data that another workgroup of the same launch writes or reads.
 *
 * gfx950 has one L2 per XCD and they are not kept coherent with each other for ordinary
 * accesses: a store can sit in the writer's L2 and a load can hit a stale line in the
 * reader's. Device-scope accesses (the sc1 bit) go to the point where all XCDs meet, so
 * a consumer that has seen its producer's arrival count (an atomic) reads the new values
 * with no cache write-back or invalidation. With CH = false these are the ordinary
 * accesses, for kernels whose producers are earlier launches (the launch boundary makes
 * their results visible).
 */
#ifndef AOTX_COHERENT_H
#define AOTX_COHERENT_H

#include <hip/hip_runtime.h>

typedef unsigned int aotx_u4 __attribute__((ext_vector_type(4)));

template <bool CH>
static __device__ __forceinline__ aotx_u4 co_load4(const void *p)
{
    if constexpr (CH) {
        const unsigned long long *q = (const unsigned long long *)p;
        const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return (aotx_u4){(unsigned int)lo, (unsigned int)(lo >> 32), (unsigned int)hi,
                         (unsigned int)(hi >> 32)};
    } else {
        return *(const aotx_u4 *)p;
    }
}

template <bool CH>
static __device__ __forceinline__ float co_loadf(const float *p)
{
    if constexpr (CH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}

template <bool CH>
static __device__ __forceinline__ void co_storef(float *p, float v)
{
    if constexpr (CH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

/* Two fp16 values (lo at p[0], hi at p[1]); p is 4-byte aligned. */
template <bool CH>
static __device__ __forceinline__ void co_store2h(unsigned short *p, unsigned int lo, unsigned int hi)
{
    const unsigned int w = (lo & 0xffffu) | (hi << 16);
    if constexpr (CH) __hip_atomic_store((unsigned int *)p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *(unsigned int *)p = w;
}

/* No wait: the producers of a standalone kernel are earlier launches. */
struct aotx_no_wait {
    bool seen = true;
    __device__ __forceinline__ void operator()() {}
};

#endif
