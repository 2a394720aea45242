/* Library state: the device state block, the scratch pool and the weights region. */
#include "aotx_internal.h"

#include <string.h>

static aotx_state *aotx_state_ptr = nullptr;
static void *aotx_scratch_ptr[AOTX_SCRATCH_KINDS];
static size_t aotx_scratch_size[AOTX_SCRATCH_KINDS];
static unsigned long long aotx_weights_base = 0ull;
static unsigned long long aotx_weights_bytes = 0ull;

aotx_state *aotx_state_device(void)
{
    if (aotx_state_ptr == nullptr) {
        void *p = nullptr;
        AOTX_CHECK(hipMalloc(&p, sizeof(aotx_state)));
        AOTX_CHECK(hipMemset(p, 0, sizeof(aotx_state)));
        AOTX_CHECK(hipDeviceSynchronize());
        aotx_state_ptr = (aotx_state *)p;
    }
    return aotx_state_ptr;
}

/* The state block if some call has created it, else null (allocates nothing). */
aotx_state *aotx_state_existing(void)
{
    return aotx_state_ptr;
}

/* A small pinned host buffer for the few words the host reads back each step (the queue
 * marks of the page pool, a pass's offsets): copies into it skip the pageable staging. */
void *aotx_pinned(void)
{
    static void *p = nullptr;
    if (p == nullptr) AOTX_CHECK(hipHostMalloc(&p, 4096, hipHostMallocDefault));
    return p;
}

/* Grow-only scratch. A larger request waits for the device, frees the old buffer and
 * allocates a zeroed new one. Counters stay zero because every kernel that counts
 * arrivals resets its counter before it exits. Growth inside a stream capture is an
 * error: the model sizes every buffer before it captures. */
void *aotx_scratch(aotx_scratch_kind which, size_t bytes)
{
    if (bytes == 0u) bytes = 256u;
    if (bytes > aotx_scratch_size[which]) {
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        AOTX_CHECK(hipStreamIsCapturing(nullptr, &status));
        size_t grow = bytes + bytes / 4u;
        AOTX_CHECK(hipDeviceSynchronize());
        if (aotx_scratch_ptr[which] != nullptr) AOTX_CHECK(hipFree(aotx_scratch_ptr[which]));
        void *p = nullptr;
        AOTX_CHECK(hipMalloc(&p, grow));
        AOTX_CHECK(hipMemset(p, 0, grow));
        AOTX_CHECK(hipDeviceSynchronize());
        aotx_scratch_ptr[which] = p;
        aotx_scratch_size[which] = grow;
    }
    return aotx_scratch_ptr[which];
}

extern "C" int aotx_mem_weights_set(unsigned long long base, unsigned long long bytes)
{
    if (base == 0ull || bytes == 0ull) return 1;
    aotx_weights_base = base;
    aotx_weights_bytes = bytes;
    return 0;
}

extern "C" unsigned long long aotx_mem_weights_base(void)
{
    return aotx_weights_base;
}

unsigned long long aotx_mem_weights_bytes(void)
{
    return aotx_weights_bytes;
}

extern "C" const char *aotx_version(void)
{
    return "aotx-mi355x 0.1.0 (gfx950)";
}
