"""Page-table decisions of the reference's KV pool, restated in Python — TEST
INFRASTRUCTURE ONLY.

cuda/kvcache/kv_host.cu:97-100 fills the free stack descending, so position 0 is taken
first; kv_host.cu:28-57 (take) pops it, :60-74 (give) pushes a released position back;
kv_host.cu:128-193 (serve) answers the queue in order, refuses a request that the free
stack cannot fill (short_of), caps a slot at PAGES_EACH; cuda/model/gather.cu:8-26
(request) asks for need - held pages with need = pages(seen + tokens).
"""


class KvPolicy:
    def __init__(self, pool_pages, pages_each=640):
        self.pages_each = pages_each
        self.free = [pool_pages - 1 - i for i in range(pool_pages)]
        self.page = {}          # slot -> list of page positions
        self.short_of = 0
        self.queue = []

    def count(self, slot):
        return len(self.page.get(slot, []))

    def request(self, slot, pages):
        if pages:
            self.queue.append((slot, pages))

    def release(self, slot):
        self.queue.append((slot, 0))

    def serve(self):
        done = len(self.queue)
        for slot, pages in self.queue:
            if pages == 0:
                for p in self.page.get(slot, []):
                    self.free.append(p)
                self.page[slot] = []
                continue
            have = self.count(slot)
            want = min(have + pages, self.pages_each)
            if want - have > len(self.free):
                self.short_of += 1
                continue
            for _ in range(have, want):
                self.page.setdefault(slot, []).append(self.free.pop())
        self.queue = []
        return done


def layout_pages(context, layers, kv_heads, head_dim, page_bytes=2 * 1024 * 1024,
                 header=256, block=16):
    """Pages a context needs (cuda/model/kv_layout.cuh:37-103)."""
    block_bytes = 2 * kv_heads * block * head_dim * 2
    per_page = (page_bytes - header) // block_bytes
    if per_page == 0:
        return 0
    blocks = ((context + block - 1) // block) * layers
    return (blocks + per_page - 1) // per_page
