"""The probe's residual capture, the embedding role's pooled rows and the rank role's score
on the GPU against the oracle (cuda/model/call_host.cu:40-117, cuda/model/conduct.cu:165-173,
cuda/embed/embed.cu:8-65, cuda/rerank/rerank.cu:8-81)."""
import numpy as np
import pytest

from aotx_amd import AOTX_MODEL_EMBEDDING, AOTX_MODEL_RERANKER
from aotx_amd.model import Shape, Runtime, build_host, dequant_q8
from tests.gpu_util import rel_rms

pytestmark = pytest.mark.gpu

SHAPE = Shape(layers=3, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1024)


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def _region(shape, seed, norm_scale=True):
    region, lay = build_host(shape, seed=seed)
    if norm_scale:
        # the last norm's weights away from ones, so a head that skips them is caught
        h = shape.hidden
        w = np.random.default_rng(seed).uniform(0.5, 1.5, h).astype(np.float32)
        region[lay.desc.output_norm:lay.desc.output_norm + 4 * h] = w.view(np.uint8)
    return region, lay


def _runtime(torch, region, lay, role=None, max_tokens=32):
    kw = {} if role is None else {"role": role}
    return Runtime(torch.from_numpy(region).cuda(), lay.desc, max_tokens=max_tokens,
                   pool_pages=64, **kw)


def test_probe_capture_vs_oracle(torch, orc):
    """Capture slots in any order (one layer twice) hold each sequence's last residual row
    after the named layer; the logits come out as from a plain pass; a capture of no layer
    and a plain step after it run as before."""
    region, lay = _region(SHAPE, 31)
    rt = _runtime(torch, region, lay)
    try:
        ref = orc.Model(lay.desc, region, slots=8, max_context=64)
        ids = list(range(40, 53))
        offset, agent = [0, 9, 13], [2, 5]
        layers = [2, 0, 1, 2]
        logits, cap = rt.probe(ids, offset, agent, layers)
        want = ref.step(ids, offset, agent)
        want_res = ref.last_resid(len(agent))
        assert rel_rms(logits, want) < 1e-2
        for c, l in enumerate(layers):
            for s in range(len(agent)):
                w = want_res[l, s]
                err = np.abs(cap[c, s] - w).max() / np.abs(w).max()
                assert err < 1e-2, (c, l, s, err)
                if l > 0:   # the layer before is far off: the slot's layer is the named one
                    assert np.abs(cap[c, s] - want_res[l - 1, s]).max() / np.abs(w).max() > 5e-2
        # a probe that names no layer, then a plain decode step
        logits, cap = rt.probe([7, 8], [0, 1, 2], agent, [])
        want = ref.step([7, 8], [0, 1, 2], agent)
        assert rel_rms(logits, want) < 1e-2
        tok, _, logits = rt.step([3, 4], [0, 1, 2], agent)
        want = ref.step([3, 4], [0, 1, 2], agent)
        assert rel_rms(logits, want) < 1e-2
        assert rt.faulted() == 0
    finally:
        rt.close()


def test_embedding_role_pooled_rows(torch, orc):
    """The embedding role's pass writes one unit row per sequence along the last norm of its
    last residual row (the oracle's last-norm row, which rounds to fp16, agrees in direction
    to its rounding); logits and sampled tokens are not asked of that role."""
    region, lay = _region(SHAPE, 32)
    rt = _runtime(torch, region, lay, role=AOTX_MODEL_EMBEDDING)
    try:
        ref = orc.Model(lay.desc, region, slots=8, max_context=64)
        ids = list(range(100, 121))
        offset, agent = [0, 4, 15, 21], [0, 1, 3]
        got = rt.pooled(ids, offset, agent)
        ref.step(ids, offset, agent)
        xn = ref.last_xnorm(len(agent)).astype(np.float64)
        for s in range(len(agent)):
            g = got[s].astype(np.float64)
            assert abs(np.linalg.norm(g) - 1.0) < 1e-5
            cos = float(g @ xn[s] / np.linalg.norm(xn[s]))
            assert cos > 1 - 1e-5, (s, cos)
            # the same unit row from the oracle's fp32 residual, with the norm weights
            r = ref.last_resid(len(agent))[-1, s].astype(np.float64)
            w = region[lay.desc.output_norm:lay.desc.output_norm + 4 * SHAPE.hidden].view(np.float32)
            v = r / np.sqrt((r * r).mean() + SHAPE.eps) * w
            assert np.abs(g - v / np.linalg.norm(v)).max() < 2e-3
        assert rt.faulted() == 0
    finally:
        rt.close()


def test_rank_role_score(torch, orc):
    """The rank role's score of each sequence: softmax over the two class rows (yes, no)
    against its last row under the last norm, from the oracle's residual in float64."""
    shape = Shape(layers=2, hidden=256, ffn=512, heads=4, kv_heads=2, head_dim=64, vocab=1024,
                  cls=True, sigma=0.2)
    region, lay = _region(shape, 33)
    rt = _runtime(torch, region, lay, role=AOTX_MODEL_RERANKER)
    try:
        ref = orc.Model(lay.desc, region, slots=8, max_context=64)
        ids = list(range(200, 230))
        offset, agent = [0, 10, 12, 30], [4, 6, 7]
        got = rt.rerank(ids, offset, agent)
        ref.step(ids, offset, agent)
        h = shape.hidden
        cls = dequant_q8(region[lay.desc.cls_output:lay.desc.cls_output + 2 * (h // 32) * 34]
                         .reshape(2, -1), h).astype(np.float64)
        w = region[lay.desc.output_norm:lay.desc.output_norm + 4 * h].view(np.float32)
        res = ref.last_resid(len(agent))[-1].astype(np.float64)
        spread = []
        for s in range(len(agent)):
            r = res[s]
            v = r / np.sqrt((r * r).mean() + shape.eps) * w
            yes, no = cls @ v
            want = 1.0 / (1.0 + np.exp(no - yes))
            spread.append(want)
            assert abs(float(got[s]) - want) < 2e-3, (s, float(got[s]), want)
        assert max(spread) - min(spread) > 1e-2       # the scores tell the sequences apart
        assert rt.faulted() == 0
    finally:
        rt.close()
