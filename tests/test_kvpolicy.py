"""Page-table policy (oracle/kvpolicy.py): invariants of cuda/kvcache/kv_host.cu."""
from oracle.kvpolicy import KvPolicy, layout_pages


def test_lifo_order_and_release():
    p = KvPolicy(pool_pages=8, pages_each=4)
    p.request(0, 2)
    p.request(3, 1)
    p.serve()
    assert p.page[0] == [0, 1] and p.page[3] == [2]     # position 0 first (kv_host.cu:97-100)
    p.release(0)
    p.request(5, 3)
    p.serve()
    assert p.page[0] == [] and p.page[5] == [1, 0, 3]   # released pages come back LIFO
    all_pages = [x for v in p.page.values() for x in v]
    assert len(all_pages) == len(set(all_pages))


def test_short_of_and_cap():
    p = KvPolicy(pool_pages=3, pages_each=2)
    p.request(0, 5)          # capped at pages_each
    p.serve()
    assert p.page[0] == [0, 1]
    p.request(1, 2)          # only 1 free: refused whole
    p.serve()
    assert p.short_of == 1 and p.page.get(1, []) == []


def test_layout_pages_8b():
    # 8 KV heads x 128 x 16 positions x 2 (K, V) x 2 B = 64 KiB blocks, 31 per page
    assert layout_pages(16, 32, 8, 128) == 2        # 32 blocks
    assert layout_pages(2048, 32, 8, 128) == (128 * 32 + 30) // 31
    assert layout_pages(0, 32, 8, 128) == 0
