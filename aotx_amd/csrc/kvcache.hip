/* KV page pool: the host side of the page table and its request queue.
 *
 * Reference: cuda/kvcache/kv_host.cu (open :76-111, reserve :113-126, serve :128-193,
 * take/give :28-74, close :195-216) and the device queue of cuda/kvcache/pages.cu:13-76.
 * The reference reserves a virtual range and maps 2 MiB physical pages on demand. With
 * 288 GB of HBM per MI355X the pool here is one device allocation made at open, sized by
 * map->limit pages; page position i lives at range + i * 2 MiB exactly as in the
 * reference's range, and the free stack, the queue order and the refusals are the
 * reference's, so every page-table decision is the same.
 */
#include "aotx_internal.h"
#include "kvcache_dev.h"

#include <stddef.h>
#include <string.h>

#define AOTX_KV_DEFAULT_PAGES 1024u

/* Header of every mapped page (cuda/kvcache/pages.cu:60-76): byte 0 = type, 1..15 = 0. */
__global__ void aotx_kv_stamp_kernel(aotx_state *state)
{
    unsigned int agent = blockIdx.x;
    unsigned int index = blockIdx.y * blockDim.x + threadIdx.x;
    if (agent >= AOTX_SLOTS || index >= AOTX_KV_PAGES_EACH) return;
    unsigned long long at = state->kv.page[agent][index];
    if (at == 0ull) return;
    unsigned char *header = (unsigned char *)at;
    header[0] = (unsigned char)AOTX_KV_TYPE_FP16;
    for (unsigned int b = 1u; b < AOTX_KV_HEADER_BYTES; ++b) header[b] = 0u;
}

extern "C" int aotx_kv_open(aotx_kv_map *map)
{
    if (map == nullptr) return 1;
    unsigned int limit = map->limit == 0u ? AOTX_KV_DEFAULT_PAGES : map->limit;
    if (limit > AOTX_KV_PAGES_MAX) return 1;
    memset(map, 0, sizeof *map);
    map->limit = limit;
    size_t free_bytes = 0, total = 0;
    AOTX_CHECK(hipMemGetInfo(&free_bytes, &total));
    unsigned long long bytes = (unsigned long long)limit * AOTX_KV_PAGE_BYTES;
    if (bytes + (256ull << 20) > free_bytes) {
        fprintf(stderr, "cache: the pool needs %llu bytes; %zu bytes free\n", bytes, free_bytes);
        return 1;
    }
    void *range = nullptr;
    AOTX_CHECK(hipMalloc(&range, (size_t)bytes));
    map->range = (unsigned long long)range;
    map->range_bytes = bytes;
    for (unsigned int i = 0u; i < limit; ++i) map->free_at[i] = limit - 1u - i;
    map->free_count = limit;
    map->created = limit;
    aotx_state *state = aotx_state_device();
    AOTX_CHECK(hipMemset(&state->kv, 0, sizeof(aotx_kv_table)));
    AOTX_CHECK(hipDeviceSynchronize());
    return 0;
}

extern "C" int aotx_kv_reserve(aotx_kv_map *map)
{
    /* The pool is backed at open. */
    return (map == nullptr || map->range == 0ull) ? 1 : 0;
}

static int aotx_kv_take(aotx_kv_map *map, unsigned long long *address)
{
    if (map->free_count == 0u) return 1;
    unsigned int at = map->free_at[--map->free_count];
    map->held[at] = 1u;
    *address = map->range + (unsigned long long)at * AOTX_KV_PAGE_BYTES;
    return 0;
}

static void aotx_kv_give(aotx_kv_map *map, unsigned long long address)
{
    if (address < map->range) return;
    unsigned long long at = (address - map->range) / AOTX_KV_PAGE_BYTES;
    if (at >= (unsigned long long)map->limit || map->held[at] == 0u) return;
    map->held[at] = 0u;
    map->free_at[map->free_count++] = (unsigned int)at;
}

extern "C" int aotx_kv_serve(aotx_kv_map *map, void *stream)
{
    if (map == nullptr || map->range == 0ull) return 0;
    hipStream_t s = aotx_stream(stream);
    aotx_state *state = aotx_state_device();
    unsigned int *marks = (unsigned int *)aotx_pinned();
    AOTX_CHECK(hipMemcpyAsync(marks, (unsigned char *)&state->kv + offsetof(aotx_kv_table, made),
                              2u * sizeof *marks, hipMemcpyDeviceToHost, s));
    aotx_wait(s);
    if (marks[0] == marks[1]) return 0;
    static aotx_kv_table table;
    AOTX_CHECK(hipMemcpy(&table, &state->kv, sizeof table, hipMemcpyDeviceToHost));
    if (table.served == table.made) return 0;
    unsigned int done = 0u;
    for (unsigned int at = table.served; at != table.made; ++at) {
        aotx_kv_entry entry = table.queue[at & (AOTX_KV_QUEUE_MAX - 1u)];
        done += 1u;
        if (entry.agent >= AOTX_SLOTS) continue;
        if (entry.pages == 0u) {
            for (unsigned int i = 0u; i < AOTX_KV_PAGES_EACH; ++i) {
                aotx_kv_give(map, table.page[entry.agent][i]);
                table.page[entry.agent][i] = 0ull;
            }
            table.count[entry.agent] = 0u;
            continue;
        }
        unsigned int want = table.count[entry.agent] + entry.pages;
        if (want > AOTX_KV_PAGES_EACH) want = AOTX_KV_PAGES_EACH;
        if (want - table.count[entry.agent] > map->free_count) {
            table.short_of += 1u;
            continue;
        }
        for (unsigned int i = table.count[entry.agent]; i < want; ++i) {
            unsigned long long address = 0ull;
            if (aotx_kv_take(map, &address) != 0) {
                table.short_of += 1u;
                break;
            }
            table.page[entry.agent][i] = address;
            table.count[entry.agent] = i + 1u;
        }
    }
    table.mapped_pages = map->limit - map->free_count;
    table.served = table.made;
    /* The host owns everything before `made`, and `served`; `made` and `refused` belong to
     * device code and are not written over. */
    AOTX_CHECK(hipMemcpy(&state->kv, &table, offsetof(aotx_kv_table, made), hipMemcpyHostToDevice));
    AOTX_CHECK(hipMemcpy((unsigned char *)&state->kv + offsetof(aotx_kv_table, served),
                         &table.served, sizeof table.served, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(aotx_kv_stamp_kernel, dim3(AOTX_SLOTS, (AOTX_KV_PAGES_EACH + 255u) / 256u),
                       dim3(256), 0, s, state);
    AOTX_LAUNCH_CHECK();
    aotx_wait(s);
    return (int)done;
}

extern "C" void aotx_kv_close(aotx_kv_map *map)
{
    if (map == nullptr || map->range == 0ull) return;
    AOTX_CHECK(hipDeviceSynchronize());
    aotx_state *state = aotx_state_device();
    AOTX_CHECK(hipMemset(&state->kv, 0, sizeof(aotx_kv_table)));
    AOTX_CHECK(hipFree((void *)map->range));
    AOTX_CHECK(hipDeviceSynchronize());
    map->range = 0ull;
    map->free_count = 0u;
}

__global__ void aotx_kv_put_kernel(aotx_state *state, unsigned int agent, unsigned int pages,
                                   int release, int *made)
{
    int ok = aotx_kv_put(&state->kv, agent, pages);
    if (release && ok && agent < AOTX_SLOTS) state->kv.count[agent] = 0u;
    *made = ok;
}

static int aotx_kv_put_host(unsigned int agent, unsigned int pages, int release)
{
    static int *made = nullptr;
    if (made == nullptr) AOTX_CHECK(hipMalloc(&made, sizeof(int)));
    hipLaunchKernelGGL(aotx_kv_put_kernel, dim3(1), dim3(1), 0, nullptr, aotx_state_device(), agent,
                       pages, release, made);
    AOTX_LAUNCH_CHECK();
    int out = 0;
    AOTX_CHECK(hipMemcpy(&out, made, sizeof out, hipMemcpyDeviceToHost));
    return out;
}

extern "C" int aotx_kv_request(unsigned int agent, unsigned int pages)
{
    if (pages == 0u) return 0;  /* a request for no page is a release, which has its own call */
    return aotx_kv_put_host(agent, pages, 0);
}

extern "C" int aotx_kv_release(unsigned int agent)
{
    return aotx_kv_put_host(agent, 0u, 1);
}

extern "C" int aotx_kv_table_read(aotx_kv_table *out)
{
    if (out == nullptr) return 1;
    AOTX_CHECK(hipDeviceSynchronize());
    AOTX_CHECK(hipMemcpy(out, &aotx_state_device()->kv, sizeof *out, hipMemcpyDeviceToHost));
    return 0;
}

extern "C" unsigned long long aotx_kv_table_device(void)
{
    return (unsigned long long)&aotx_state_device()->kv;
}
