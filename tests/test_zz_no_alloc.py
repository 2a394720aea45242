"""aotx_attend_paged_static (the allocation-free attention entry point) against
aotx_attend_paged on the same inputs: equal outputs, bit for bit (the same kernels over the
same split), on two calls in a row, the second with fewer tokens; and the refusal of a
launch whose scratch exceeds the fixed array."""
import ctypes

import numpy as np
import pytest

import aotx_amd
from oracle.kvpolicy import layout_pages
from tests.gpu_util import dev, p

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def test_static_attention_equals_allocating(torch, lib):
    heads, kvh, d, layers, layer = 32, 8, 128, 2, 1
    rng = np.random.default_rng(31)
    slots = [4, 11, 2, 60, 7, 33]
    contexts = [900, 37, 2500, 1, 640, 1800]
    lib.aotx_model_forget()
    m = aotx_amd.KvMap()
    m.limit = 512
    assert lib.aotx_kv_open(ctypes.byref(m)) == 0
    try:
        for s, n in zip(slots, contexts):
            assert lib.aotx_kv_request(s, layout_pages(n, layers, kvh, d)) == 1
        assert lib.aotx_kv_serve(ctypes.byref(m), None) == len(slots)
        for s, n in zip(slots, contexts):
            k = rng.normal(0, 1, (n, kvh, d)).astype(np.float16)
            v = rng.normal(0, 1, (n, kvh, d)).astype(np.float16)
            assert lib.aotx_kv_write(p(dev(k, torch)), p(dev(v, torch)),
                                     p(dev(np.arange(n, dtype=np.uint32), torch)),
                                     p(dev(np.full(n, s, dtype=np.uint32), torch)), n, kvh, d,
                                     layer, layers, None) == 0
        torch.cuda.synchronize()
        for count in (6, 2):            # the second call is smaller (more chunks per token)
            q = rng.normal(0, 1, (count, heads, d)).astype(np.float16)
            pos = np.array([n - 1 for n in contexts[:count]], dtype=np.uint32)
            ag = np.array(slots[:count], dtype=np.uint32)
            qd, pd, ad = dev(q, torch), dev(pos, torch), dev(ag, torch)
            want = torch.zeros(count * heads * d, dtype=torch.float16, device="cuda")
            got = torch.full((count * heads * d,), 7.0, dtype=torch.float16, device="cuda")
            assert lib.aotx_attend_paged(p(qd), p(pd), p(ad), count, heads, kvh, d, layer, layers,
                                         p(want), None) == 0
            assert lib.aotx_attend_paged_static(p(qd), p(pd), p(ad), count, heads, kvh, d, layer,
                                                layers, p(got), None) == 0
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), count
        # scratch beyond the fixed array is refused before anything is launched
        big = 4097
        assert lib.aotx_attend_paged_static(p(qd), p(pd), p(ad), big, 8, 1, d, layer, layers,
                                            p(got), None) == 1
        # so are shapes the kernels do not take (head width 96; 3 query heads per KV head):
        # the output keeps what it held, so nothing ran
        before = got.clone()
        assert lib.aotx_attend_paged_static(p(qd), p(pd), p(ad), 2, heads, kvh, 96, layer,
                                            layers, p(got), None) == 1
        assert lib.aotx_attend_paged_static(p(qd), p(pd), p(ad), 2, 24, kvh, d, layer,
                                            layers, p(got), None) == 1
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), before.view(torch.int16))
        assert lib.aotx_model_faulted() == 0
    finally:
        lib.aotx_kv_close(ctypes.byref(m))
