/* Deterministic synthetic weights: one definition for host and device, so both write the
 * same bytes. Only integer arithmetic and correctly rounded IEEE operations are used
 * (add, multiply, divide, rint), and the fp16 rounding is done here in integers, so no
 * library math function decides a bit.
 *
 * Normal values: value i takes splitmix64 outputs 3i, 3i+1, 3i+2 of `seed`; their twelve
 * 16-bit fields u_j give z = (sum u_j - 393210) / 65536, the Irwin-Hall approximation of
 * N(0, 1) (mean 0, variance 1, support [-6, 6]); w = z * sigma.
 *
 * Q8_0 blocks (the 34-byte layout of cuda/model/matrix.cuh:6-9): d = max|w| / 127 over the
 * 32 weights, q = rint(w / d) clamped to [-127, 127], scale = fp16(d). The reference ships
 * no quantizer; this one is the build's own definition. */
#ifndef AOTX_SYNTH_H
#define AOTX_SYNTH_H

#include <stdint.h>

#ifdef __HIPCC__
#define AOTX_HD __host__ __device__ inline
#else
#define AOTX_HD static inline
#endif

AOTX_HD uint64_t aotx_splitmix(uint64_t seed, uint64_t n)
{
    uint64_t z = seed + (n + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

AOTX_HD float aotx_synth_normal(uint64_t seed, uint64_t i)
{
    int32_t sum = 0;
    for (uint64_t j = 0; j < 3ull; ++j) {
        uint64_t r = aotx_splitmix(seed, 3ull * i + j);
        sum += (int32_t)(r & 0xFFFFu) + (int32_t)((r >> 16) & 0xFFFFu)
             + (int32_t)((r >> 32) & 0xFFFFu) + (int32_t)(r >> 48);
    }
    return (float)(sum - 393210) * (1.0f / 65536.0f);
}

/* fp32 -> fp16 bits, round to nearest even, with subnormals, infinities and NaN. */
AOTX_HD uint16_t aotx_f32_to_f16(float f)
{
    union { float f; uint32_t u; } v;
    v.f = f;
    uint32_t x = v.u;
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mag = x & 0x7FFFFFFFu;
    if (mag >= 0x7F800000u) {                 /* inf or nan */
        return (uint16_t)(sign | 0x7C00u | (mag > 0x7F800000u ? 0x200u : 0u));
    }
    if (mag >= 0x477FF000u) {                 /* rounds to >= 65520: overflow */
        return (uint16_t)(sign | 0x7C00u);
    }
    if (mag < 0x38800000u) {                  /* result is subnormal or zero */
        if (mag < 0x33000000u) {              /* below half the smallest subnormal */
            return (uint16_t)sign;
        }
        uint32_t e = mag >> 23;
        uint32_t m = (mag & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;            /* 14..24: puts the value in units of 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) {
            q += 1u;
        }
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((mag >> 13) - (112u << 10));  /* rebias exponent 127 -> 15 */
    uint32_t rem = mag & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h += 1u;
    }
    return (uint16_t)(sign | h);
}

AOTX_HD float aotx_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (e == 0u) {
        if (m == 0u) {
            bits = sign;
        } else {
            /* subnormal: value = m * 2^-24 */
            union { float f; uint32_t u; } t;
            t.f = (float)m * (1.0f / 16777216.0f);
            bits = sign | t.u;
        }
    } else if (e == 31u) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    union { float f; uint32_t u; } v;
    v.u = bits;
    return v.f;
}

/* One Q8_0 block of 32 weights starting at value index i0 into 34 bytes. */
AOTX_HD void aotx_synth_block(uint8_t *out, uint64_t seed, uint64_t i0, float sigma)
{
    float w[32];
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        w[j] = aotx_synth_normal(seed, i0 + (uint64_t)j) * sigma;
        float a = w[j] < 0.0f ? -w[j] : w[j];
        amax = a > amax ? a : amax;
    }
    float d = amax / 127.0f;
    uint16_t hs = aotx_f32_to_f16(d);
    out[0] = (uint8_t)(hs & 0xFFu);
    out[1] = (uint8_t)(hs >> 8);
    for (int j = 0; j < 32; ++j) {
        float r = (d != 0.0f) ? __builtin_rintf(w[j] / d) : 0.0f;
        int q = (int)r;
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        out[2 + j] = (uint8_t)(int8_t)q;
    }
}

#endif
