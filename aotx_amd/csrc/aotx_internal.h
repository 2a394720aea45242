/* Internal definitions shared by the HIP sources of libaotx_hip.so. */
#ifndef AOTX_INTERNAL_H
#define AOTX_INTERNAL_H

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdio.h>
#include <stdlib.h>
#include <stdint.h>

#include "../../include/aotx_hip.h"

/* A failing runtime call ends the process with its site, as the reference's check does
 * (cuda/boot/check.h:13-33). */
#define AOTX_CHECK(call)                                                                  \
    do {                                                                                  \
        hipError_t aotx_err_ = (call);                                                    \
        if (aotx_err_ != hipSuccess) {                                                    \
            fprintf(stderr, "aotx: %s failed at %s:%d: %s\n", #call, __FILE__, __LINE__,  \
                    hipGetErrorString(aotx_err_));                                        \
            exit(1);                                                                      \
        }                                                                                 \
    } while (0)

#define AOTX_LAUNCH_CHECK() AOTX_CHECK(hipGetLastError())

/* Device-resident state of the runtime: the page table and request queue, every slot's
 * cache position and draw counter, and the fault count. The reference keeps these as
 * device symbols (aotx_kv, aotx_model_seen, aotx_model_draw, aotx_model_faults:
 * cuda/kvcache/kvcache.cuh:66, cuda/model/forward.cuh:180-191); here they are one
 * allocation whose address every kernel takes as an argument. */
struct aotx_state {
    aotx_kv_table kv;
    unsigned int seen[AOTX_SLOTS];
    unsigned int draw[AOTX_SLOTS];
    unsigned int faults;
};

/* The device state of the current device, allocated and zeroed on first use. */
aotx_state *aotx_state_device(void);
aotx_state *aotx_state_existing(void);

/* Per-call scratch of the library (partial sums, arrival counters). One growable buffer
 * per use; counters are zeroed once at allocation and every kernel that uses one puts
 * it back to zero before it exits. */
enum aotx_scratch_kind : int {
    AOTX_SCRATCH_GEMV_PARTIAL = 0,
    AOTX_SCRATCH_GEMV_COUNT,
    AOTX_SCRATCH_ATTN_PARTIAL,
    AOTX_SCRATCH_ATTN_COUNT,
    AOTX_SCRATCH_EXPERT,
    AOTX_SCRATCH_PICK,
    AOTX_SCRATCH_KINDS
};
void *aotx_scratch(aotx_scratch_kind which, size_t bytes);
/* 4 KB of pinned host memory for step read-backs (one host thread per runtime). */
void *aotx_pinned(void);

static inline hipStream_t aotx_stream(void *s) { return (hipStream_t)s; }

/* Wait for a stream's work by polling it. The calls a decode loop makes every step (page
 * requests, serve, the offsets read-back, the step) each wait for the device; a blocking
 * wait is woken tens of microseconds after the work ends, a poll within about one. */
static inline void aotx_wait(hipStream_t s)
{
    for (;;) {
        const hipError_t e = hipStreamQuery(s);
        if (e == hipSuccess) return;
        if (e != hipErrorNotReady) AOTX_CHECK(e);
    }
}

/* ---- paged layout (cuda/model/kv_layout.cuh:37-163), one layer kind: every layer owns
 * KV pages. ---- */
struct aotx_kvl_shape {
    unsigned int layers;
    unsigned int kv_heads;
    unsigned int head_dim;
    unsigned int head_bytes;    /* 16 positions of one head */
    unsigned int block_bytes;   /* K heads then V heads */
    unsigned int blocks_page;
};

static inline __host__ __device__ aotx_kvl_shape aotx_kvl_make(unsigned int layers,
                                                               unsigned int kv_heads,
                                                               unsigned int head_dim)
{
    aotx_kvl_shape s;
    s.layers = layers;
    s.kv_heads = kv_heads;
    s.head_dim = head_dim;
    s.head_bytes = AOTX_KVL_BLOCK * head_dim * 2u;
    s.block_bytes = 2u * kv_heads * s.head_bytes;
    s.blocks_page = s.block_bytes == 0u ? 0u
        : (unsigned int)((AOTX_KV_PAGE_BYTES - AOTX_KVL_HEADER) / s.block_bytes);
    return s;
}

static inline __host__ __device__ unsigned int aotx_kvl_pages(const aotx_kvl_shape &s,
                                                              unsigned int context)
{
    if (s.blocks_page == 0u) return 0u;
    unsigned int blocks = ((context + AOTX_KVL_BLOCK - 1u) / AOTX_KVL_BLOCK) * s.layers;
    return (blocks + s.blocks_page - 1u) / s.blocks_page;
}

/* The KV shape of a role with a model described (model.hip); 1 when it has none. */
int aotx_role_kv_shape(unsigned int role, aotx_kvl_shape *out);

/* First byte of the layout block holding (layer, position) of one slot, or null. */
static inline __device__ unsigned char *aotx_kvl_block(const aotx_kvl_shape &s,
                                                       const aotx_kv_table *kv,
                                                       unsigned int agent,
                                                       unsigned int layer,
                                                       unsigned int position)
{
    if (s.blocks_page == 0u || agent >= AOTX_SLOTS) return nullptr;
    unsigned int block = (position / AOTX_KVL_BLOCK) * s.layers + layer;
    unsigned int index = block / s.blocks_page;
    if (index >= AOTX_KV_PAGES_EACH) return nullptr;
    unsigned long long page = kv->page[agent][index];
    if (page == 0ull) return nullptr;
    return (unsigned char *)(page + AOTX_KVL_HEADER
                             + (unsigned long long)(block % s.blocks_page) * s.block_bytes);
}

/* ---- the fragment layout of a product's x (5..32 batch rows of a dense model) ----
 * The B operand of v_mfma_f32_16x16x32_f16 in the order a product's wave loads it, so every
 * 16-byte load of a wave reads one contiguous kilobyte. Batch row m (< 32) and column k of
 * a row whose width is a multiple of 128 sit at
 *   [quad k/128][row block m/16][step (k%32)/8][lane (m%16) + 16 ((k%128)/32)][k%8]
 * (halves): 32 rows per quad whatever the batch, 8 KB per quad. Lane (r, g) of step s then
 * holds rows 16t + r, columns 128q + 32g + 8s .. +7, the k order of the repacked weights'
 * A operand (lane (r, g) dequantises block 4q + g, values 8s .. 8s + 7 at step s). */
static inline __host__ __device__ unsigned long long aotx_xfrag_at(unsigned int m, unsigned int k)
{
    const unsigned int q = k >> 7, g = (k >> 5) & 3u, st = (k >> 3) & 3u;
    const unsigned int lane = (m & 15u) + 16u * g;
    return ((((unsigned long long)q * 2u + (m >> 4)) * 4u + st) * 64u + lane) * 8u + (k & 7u);
}
#define AOTX_XFRAG_ROWS 32u

/* fp16 <-> fp32 on raw bits */
static inline __device__ float aotx_h2f(unsigned short h)
{
    return __half2float(__ushort_as_half(h));
}
static inline __device__ unsigned short aotx_f2h(float f)
{
    return __half_as_ushort(__float2half(f));
}

#endif
