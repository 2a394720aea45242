"""Pin the oracle's whole-model forward against an independent float64 numpy forward of
the same weights (tests/model_ref.h:301-427 generalised to the Llama layer kind: no head
norm, adjacent rotary pairs; and the head-norm kind with split pairs)."""
import math

import numpy as np
import pytest

from aotx_amd import SLOT, AOTX_ROPE_PAIRS_ADJACENT, AOTX_MODEL_ABSENT
from aotx_amd.model import Shape, build_host, dequant_q8


def h(x):
    return np.asarray(x, dtype=np.float64).astype(np.float16).astype(np.float64)


def numpy_forward(region, lay, shape, ids_per_step, renorm=False, layer_resid=None):
    """ids_per_step: list of token lists for one sequence (each list = one pass). renorm
    (a negative control): routed weights renormalised over the chosen experts. layer_resid,
    when a list, receives per pass the residual after every layer of its last token."""
    d = lay.desc
    def t(off, rows, k):
        return dequant_q8(region[off:off + rows * (k // 32) * 34].reshape(rows, -1), k).astype(np.float64)
    def f(off, n):
        return region[off:off + 4 * n].view(np.float32).astype(np.float64)
    H, F = shape.hidden, shape.ffn
    hd = shape.head_dim
    wide, narrow = shape.heads * hd, shape.kv_heads * hd
    emb_blk = region[d.token_embd:d.token_embd + shape.vocab * (H // 32) * 34].reshape(shape.vocab, H // 32, 34)
    keys = [[] for _ in range(shape.layers)]
    vals = [[] for _ in range(shape.layers)]
    pos = 0
    outs = []
    def rms(v, w):
        return h(v / math.sqrt((v * v).sum() / v.size + shape.eps) * w)
    def rope(v, p):
        v = v.copy()
        step = shape.theta ** (-2.0 / hd)
        for i in range(hd // 2):
            lo, hi = (2 * i, 2 * i + 1) if shape.pairs == AOTX_ROPE_PAIRS_ADJACENT else (i, i + hd // 2)
            ang = p * step ** i
            a, b = v[lo], v[hi]
            v[lo] = a * math.cos(ang) - b * math.sin(ang)
            v[hi] = a * math.sin(ang) + b * math.cos(ang)
        return h(v)
    for ids in ids_per_step:
        for ti, tok in enumerate(ids):
            sc = emb_blk[tok, :, :2].copy().view(np.float16).astype(np.float64)
            q8 = emb_blk[tok, :, 2:].copy().view(np.int8).astype(np.float64)
            resid = (q8 * sc).reshape(H)
            for l in range(shape.layers):
                L = d.layer[l]
                x = rms(resid, f(L.offset[SLOT["attn_norm"]], H))
                q = t(L.offset[SLOT["attn_q"]], wide, H) @ x
                k = t(L.offset[SLOT["attn_k"]], narrow, H) @ x
                v = t(L.offset[SLOT["attn_v"]], narrow, H) @ x
                qn = kn = None
                if shape.qk_norm:
                    qn = f(L.offset[SLOT["q_norm"]], hd)
                    kn = f(L.offset[SLOT["k_norm"]], hd)
                qh = []
                for hh in range(shape.heads):
                    head = q[hh * hd:(hh + 1) * hd]
                    if qn is not None:
                        head = head / math.sqrt((head * head).sum() / hd + shape.eps) * qn
                    qh.append(rope(head, pos))
                kr, vr = [], []
                for hh in range(shape.kv_heads):
                    head = k[hh * hd:(hh + 1) * hd]
                    if kn is not None:
                        head = head / math.sqrt((head * head).sum() / hd + shape.eps) * kn
                    kr.append(rope(head, pos))
                    vr.append(h(v[hh * hd:(hh + 1) * hd]))
                keys[l].append(kr)
                vals[l].append(vr)
                att = np.zeros(wide)
                g = shape.heads // shape.kv_heads
                for hh in range(shape.heads):
                    K = np.array([kk[hh // g] for kk in keys[l]])
                    V = np.array([vv[hh // g] for vv in vals[l]])
                    s = K @ qh[hh] / math.sqrt(hd)
                    p = np.exp(s - s.max())
                    att[hh * hd:(hh + 1) * hd] = h((p / p.sum()) @ V)
                resid = resid + t(L.offset[SLOT["attn_o"]], H, wide) @ att
                x = rms(resid, f(L.offset[SLOT["ffn_norm"]], H))
                if shape.experts:
                    # routed experts (cuda/model/experts.cu:10-98): softmax over every
                    # expert of router . half(x), the `used` largest (lower index first
                    # on ties), their outputs weighted by those probabilities as they are
                    # (no renormalisation over the chosen ones)
                    E = shape.experts
                    logit = f(L.offset[SLOT["router"]], E * H).reshape(E, H) @ x
                    prob = np.exp(logit - logit.max())
                    prob /= prob.sum()
                    order = sorted(range(E), key=lambda e: (-prob[e], e))[:shape.used]
                    if renorm:
                        prob = prob / prob[order].sum()
                    gate_all = t(L.offset[SLOT["ffn_gate"]], E * F, H).reshape(E, F, H)
                    up_all = t(L.offset[SLOT["ffn_up"]], E * F, H).reshape(E, F, H)
                    down_all = t(L.offset[SLOT["ffn_down"]], E * H, F).reshape(E, H, F)
                    for e in order:
                        gate, up = gate_all[e] @ x, up_all[e] @ x
                        act = h(gate / (1 + np.exp(-gate)) * up)
                        resid = resid + prob[e] * (down_all[e] @ act)
                else:
                    gate = t(L.offset[SLOT["ffn_gate"]], F, H) @ x
                    up = t(L.offset[SLOT["ffn_up"]], F, H) @ x
                    act = h(gate / (1 + np.exp(-gate)) * up)
                    resid = resid + t(L.offset[SLOT["ffn_down"]], H, F) @ act
                if layer_resid is not None and ti == len(ids) - 1:
                    if l == 0:
                        layer_resid.append([])
                    layer_resid[-1].append(resid.copy())
            pos += 1
        xn = rms(resid, f(d.output_norm, H))
        head_off = d.token_embd if shape.tied else d.output
        outs.append(t(head_off, shape.vocab, H) @ xn)
    return outs


@pytest.mark.parametrize("variant", ["llama", "qknorm_split", "experts"])
def test_oracle_model_vs_numpy(orc, variant):
    shape = Shape(layers=2, hidden=128, ffn=192, heads=4, kv_heads=2, head_dim=64, vocab=512)
    if variant == "qknorm_split":
        shape.qk_norm = True
        shape.pairs = 0
    if variant == "experts":
        shape.experts, shape.used = 8, 2
        shape.sigma = 0.2            # router logits far enough apart that the choice is clear
    region, lay = build_host(shape, seed=21)
    steps = [[5, 77, 300, 12, 9], [400], [13]]
    want = numpy_forward(region, lay, shape, steps)
    m = orc.Model(lay.desc, region, slots=2, max_context=64)
    pos = 0
    for i, ids in enumerate(steps):
        got = m.step(ids, [0, len(ids)], [1])[0]
        err = np.abs(got - want[i]).max() / np.abs(want[i]).max()
        assert err < 5e-3, (i, err)
        assert int(np.argmax(got)) == int(np.argmax(want[i])) or \
            np.sort(want[i])[-1] - np.sort(want[i])[-2] < 2 * np.abs(got - want[i]).max()
    if variant == "experts":
        # the control: renormalising the routed weights is caught by the same figure
        wrong = numpy_forward(region, lay, shape, steps[:1], renorm=True)[0]
        m2 = orc.Model(lay.desc, region, slots=2, max_context=64)
        got = m2.step(steps[0], [0, len(steps[0])], [1])[0]
        assert np.abs(got - wrong).max() / np.abs(wrong).max() > 2e-2


def test_oracle_model_batch_equals_serial(orc):
    """Two sequences in one pass give the rows that each gives alone."""
    shape = Shape(layers=2, hidden=128, ffn=192, heads=4, kv_heads=2, head_dim=64, vocab=512)
    region, lay = build_host(shape, seed=22)
    a = orc.Model(lay.desc, region, slots=4, max_context=64)
    both = a.step([1, 2, 3, 7, 8], [0, 3, 5], [0, 2])
    b = orc.Model(lay.desc, region, slots=4, max_context=64)
    s0 = b.step([1, 2, 3], [0, 3], [0])
    s1 = b.step([7, 8], [0, 2], [2])
    assert np.array_equal(both[0], s0[0]) and np.array_equal(both[1], s1[0])


def test_oracle_layer_residuals_vs_numpy(orc):
    """The residual rows after every layer (the probe's capture) against the numpy forward;
    a wrong layer index (the rows of the layer before) is caught by the same figure."""
    shape = Shape(layers=3, hidden=128, ffn=192, heads=4, kv_heads=2, head_dim=64, vocab=512)
    region, lay = build_host(shape, seed=23)
    steps = [[5, 77, 300, 12], [9]]
    want = []
    numpy_forward(region, lay, shape, steps, layer_resid=want)
    m = orc.Model(lay.desc, region, slots=2, max_context=64)
    for i, ids in enumerate(steps):
        m.step(ids, [0, len(ids)], [1])
        got = m.last_resid(1)[:, 0, :]
        for l in range(shape.layers):
            ref = want[i][l]
            err = np.abs(got[l] - ref).max() / np.abs(ref).max()
            assert err < 5e-3, (i, l, err)
            if l > 0:
                assert np.abs(got[l - 1] - ref).max() / np.abs(ref).max() > 5e-2
