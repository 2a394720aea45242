"""Pin the CPU oracle against the reference's golden vectors and against what the
mathematics fixes (independent numpy restatements, closed forms, brute force)."""
import json
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_philox_known_answers(orc):
    """Random123 known answers quoted in tests/rng_test.cu:61-75."""
    with open(os.path.join(GOLDEN, "philox_kat.json")) as f:
        kat = json.load(f)
    for case in kat["cases"]:
        out = orc.philox(np.array(case["ctr"], dtype=np.uint32), np.array(case["key"], dtype=np.uint32))
        assert [int(v) for v in out] == case["out"]


def _philox_numpy(ctr, key):
    c = [int(v) for v in ctr]
    k = [int(v) for v in key]
    for r in range(10):
        if r:
            k[0] = (k[0] + 0x9E3779B9) & 0xFFFFFFFF
            k[1] = (k[1] + 0xBB67AE85) & 0xFFFFFFFF
        p0 = 0xD2511F53 * c[0]
        p1 = 0xCD9E8D57 * c[2]
        c = [((p1 >> 32) ^ c[1] ^ k[0]) & 0xFFFFFFFF, p1 & 0xFFFFFFFF,
             ((p0 >> 32) ^ c[3] ^ k[1]) & 0xFFFFFFFF, p0 & 0xFFFFFFFF]
    return c


def test_philox_random_vs_python(orc):
    rng = np.random.default_rng(3)
    for _ in range(200):
        ctr = rng.integers(0, 2 ** 32, 4, dtype=np.uint64).astype(np.uint32)
        key = rng.integers(0, 2 ** 32, 2, dtype=np.uint64).astype(np.uint32)
        assert [int(v) for v in orc.philox(ctr, key)] == _philox_numpy(ctr, key)


def test_f16_conversions_exhaustive(orc):
    """Every fp16 bit pattern round-trips; fp32 -> fp16 matches numpy's RNE cast."""
    L = orc.lib()
    for h in range(0, 65536, 1):
        e = (h >> 10) & 0x1F
        v = L.orc_f16_to_f32(h)
        want = np.array([h], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
        if e == 31 and (h & 0x3FF):
            assert math.isnan(v)
            continue
        assert v == want, hex(h)
        assert L.orc_f32_to_f16(v) == h or (v == 0 and h in (0, 0x8000))
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 20000),
                         rng.normal(0, 3e4, 2000)]).astype(np.float32)
    for x in xs[np.abs(xs) < 65504]:
        assert L.orc_f32_to_f16(float(x)) == int(np.array([x]).astype(np.float16).view(np.uint16)[0])


def _q8_random(rng, n, k):
    from aotx_amd.model import quantize_q8
    return quantize_q8(rng.normal(0, 0.02, (n, k)).astype(np.float32))


def test_q8_gemv_f64_vs_numpy(orc):
    from aotx_amd.model import dequant_q8
    rng = np.random.default_rng(5)
    n, k, m = 48, 256, 3
    w = _q8_random(rng, n, k)
    x = rng.normal(0, 1, (m, k)).astype(np.float16)
    got = orc.q8_gemv_f64(w, n, k, x.view(np.uint16))
    want = x.astype(np.float64) @ dequant_q8(w, k).astype(np.float64).T
    assert np.allclose(got, want, rtol=0, atol=1e-9)


def test_q8_gemv_transposed_control(orc):
    """The transposed operand (tests/matrix_test.cu:432-470) must differ: a swapped index
    would pass a symmetric check."""
    rng = np.random.default_rng(6)
    n = k = 64
    w = _q8_random(rng, n, k)
    x = rng.normal(0, 1, (2, k)).astype(np.float16).view(np.uint16)
    right = orc.q8_gemv_f64(w, n, k, x)
    swapped = orc.q8_gemv_f64(w, n, k, x, swap=True)
    assert np.abs(right - swapped).max() > 0.1 * np.abs(right).max()


def test_q8_gemv_f32_close_to_f64(orc):
    """The fp32 reader keeps fp32(scale) * q unrounded (cuda/model/matrix.cuh:499-512): it
    equals a double product of those weights to fp32 rounding, and differs from the
    half-rounded product by about 5e-4 (inside the reference's 1e-2 gate)."""
    rng = np.random.default_rng(7)
    n, k = 64, 4096
    w = _q8_random(rng, n, k)
    x16 = rng.normal(0, 1, (4, k)).astype(np.float16)
    a = orc.q8_gemv_f32(w, n, k, x16.view(np.uint16), threads=4)
    blk = w.reshape(n, k // 32, 34)
    sc = blk[:, :, :2].copy().view(np.float16).astype(np.float32)
    q = blk[:, :, 2:].copy().view(np.int8).astype(np.float32)
    wf = (q * sc).reshape(n, k).astype(np.float64)
    exact = x16.astype(np.float64) @ wf.T
    rms = np.sqrt((exact ** 2).mean())
    assert (np.abs(a - exact) / np.maximum(np.abs(exact), rms)).max() < 2e-5
    b = orc.q8_gemv_f64(w, n, k, x16.view(np.uint16))
    assert (np.abs(a - b) / np.maximum(np.abs(b), rms)).max() < 1e-2


def test_q8_gemv_f32_reader_by_rows(orc):
    """Passes of 17 rows or more read half(scale * q) (the tensor-core tile stages half
    weights, cuda/model/gemm.cuh:108-113); 16 rows or fewer keep fp32(scale) * q. Each form
    equals the double product of its own weights to fp32 sum rounding and not the other's;
    a batch-16 row equals the same row inside a batch of 17 only to the half rounding."""
    from aotx_amd.model import dequant_q8
    rng = np.random.default_rng(8)
    n, k = 96, 2048
    w = _q8_random(rng, n, k)
    x16 = rng.normal(0, 1, (17, k)).astype(np.float16)
    blk = w.reshape(n, k // 32, 34)
    sc = blk[:, :, :2].copy().view(np.float16).astype(np.float32)
    q = blk[:, :, 2:].copy().view(np.int8).astype(np.float32)
    w_f32 = (q * sc).reshape(n, k).astype(np.float64)
    w_half = dequant_q8(w, k).astype(np.float64)
    assert np.abs(w_f32 - w_half).max() > 0          # the two readers differ on these weights
    xf = x16.astype(np.float64)
    want_f32, want_half = xf @ w_f32.T, xf @ w_half.T
    rms = np.sqrt((want_f32 ** 2).mean())

    def err(a, b):
        return (np.abs(a - b) / np.maximum(np.abs(b), rms)).max()
    wide = orc.q8_gemv_f32(w, n, k, x16.view(np.uint16), threads=3)
    narrow = orc.q8_gemv_f32(w, n, k, x16[:16].view(np.uint16), threads=3)
    assert err(wide, want_half) < 2e-5 and err(wide, want_f32) > 5e-5
    assert err(narrow, want_f32[:16]) < 2e-5 and err(narrow, want_half[:16]) > 5e-5
    assert err(narrow, wide[:16]) < 1e-2


def _allowed_numpy(row, top_k, top_p, min_p, temperature):
    """The allowed set restated in double precision (tests/sample_test.cu:177-224)."""
    row = np.asarray(row, dtype=np.float32)
    top = float(row.max())
    vals = (row.astype(np.float64) - top).astype(np.float32)
    order = sorted(range(row.size), key=lambda i: (-vals[i], i))
    s = float(np.exp(vals.astype(np.float64)).sum())
    keep = len(order) if top_k == 0 or top_k > len(order) else top_k
    if 0 < min_p <= 1:
        mk = 1
        for i in range(1, keep):
            if math.exp(float(vals[order[i]]) - float(vals[order[0]])) < min_p:
                break
            mk = i + 1
        keep = mk
    limit = 1.0 if (top_p <= 0 or top_p > 1) else top_p
    mass, taken = 0.0, 0
    for i in range(keep):
        mass += math.exp(float(vals[order[i]])) / s
        taken = i + 1
        if mass >= limit:
            break
    ids = order[:taken]
    w = np.array([math.exp((float(vals[i]) - float(vals[ids[0]])) / temperature) for i in ids])
    return ids, w / w.sum()


@pytest.mark.parametrize("top_k,top_p,min_p,temp", [
    (1, 1.0, 0.0, 0.8), (10, 1.0, 0.0, 1.0), (40, 0.9, 0.0, 0.8), (0, 0.5, 0.0, 1.0),
    (0, 0.9, 0.0, 2.0), (0, 1.0, 0.8, 1.0)])
def test_pick_allowed_set_and_chi_square(orc, top_k, top_p, min_p, temp):
    """orc_pick's allowed set equals the double-precision restatement, and its draws over
    many positions follow the restated probabilities (chi-square, sample_test.cu:231-259)."""
    rng = np.random.default_rng(11)
    vocab = 1000
    row = (rng.normal(0, 2.0, vocab)).astype(np.float32)
    ids, chance = _allowed_numpy(row, top_k, top_p, min_p, temp)
    tok, count, allowed = orc.pick(row, top_k, top_p, min_p, temp, seed=7, agent=3, position=0)
    assert list(allowed) == ids[:len(allowed)] and len(allowed) == len(ids)
    draws = 4000
    counts = {}
    for pos in range(draws):
        t, _, _ = orc.pick(row, top_k, top_p, min_p, temp, seed=7, agent=3, position=pos)
        assert t in ids
        counts[t] = counts.get(t, 0) + 1
    chi, used = 0.0, 0
    rest_seen = rest_want = 0.0
    for i, c in zip(ids, chance):
        want = c * draws
        if want >= 5:
            chi += (counts.get(i, 0) - want) ** 2 / want
            used += 1
        else:
            rest_seen += counts.get(i, 0)
            rest_want += want
    if rest_want >= 5:
        chi += (rest_seen - rest_want) ** 2 / rest_want
        used += 1
    dof = max(used - 1, 1)
    assert chi <= dof + 4 * math.sqrt(2 * dof) + 10


def test_pick_greedy_tie_rule(orc):
    """Greedy = largest logit; equal maxima go to the lowest token mod 256, then the lowest
    token (cuda/model/sample.cu:524-549)."""
    row = np.zeros(1000, dtype=np.float32)
    row[[300, 44, 556]] = 5.0          # 300 % 256 = 44 ties 44 (lower id wins); 556 % 256 = 44
    assert orc.pick(row)[0] == 44
    row = np.zeros(1000, dtype=np.float32)
    row[[513, 260]] = 5.0              # 513 % 256 = 1 beats 260 % 256 = 4
    assert orc.pick(row)[0] == 513
    rng = np.random.default_rng(2)
    for _ in range(50):
        r = rng.normal(0, 1, 5000).astype(np.float32)
        assert orc.pick(r)[0] == int(np.argmax(r))


def test_pick_top_k_is_exact_top_k(orc):
    rng = np.random.default_rng(4)
    r = rng.normal(0, 3, 2048).astype(np.float32)
    _, _, allowed = orc.pick(r, top_k=40, top_p=1.0, temperature=1.0)
    assert set(allowed.tolist()) == set(np.argsort(-r, kind="stable")[:40].tolist())


def test_route_vs_numpy(orc):
    """Full softmax over every expert, no renormalisation, ranks with lower-index ties
    (tests/expert_test.cu:118-152)."""
    rng = np.random.default_rng(8)
    for experts, used in ((8, 2), (3, 1), (7, 7), (1, 1), (64, 8)):
        router = rng.normal(0, 0.05, (experts, 128)).astype(np.float32)
        x = rng.normal(0, 1, (5, 128)).astype(np.float16)
        prob, ids = orc.route(router, x.view(np.uint16), experts, used)
        logits = x.astype(np.float64) @ router.astype(np.float64).T
        p = np.exp(logits - logits.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        assert np.abs(prob - p).max() < 2e-6
        for t in range(5):
            order = sorted(range(experts), key=lambda e: (-p[t, e], e))
            assert ids[t].tolist() == order[:used]
    # ties go to the lower index
    router = np.zeros((4, 32), dtype=np.float32)
    x = np.ones((1, 32), dtype=np.float16)
    _, ids = orc.route(router, x.view(np.uint16), 4, 2)
    assert ids[0].tolist() == [0, 1]


def test_attend_one_vs_two_pass_softmax(orc):
    rng = np.random.default_rng(9)
    for d, n in ((64, 1), (64, 37), (128, 300)):
        q = rng.normal(0, 1, d).astype(np.float16).astype(np.float32)
        k = rng.normal(0, 1, (n, d)).astype(np.float16).astype(np.float32)
        v = rng.normal(0, 1, (n, d)).astype(np.float16).astype(np.float32)
        got = orc.attend_one(q, k, v, n - 1)
        s = (k.astype(np.float64) @ q.astype(np.float64)) / math.sqrt(d)
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ v.astype(np.float64)
        assert np.abs(got - want).max() < 2e-3 * max(1.0, np.abs(want).max())
    # one position: the output is that value row (rounded to half)
    q = np.ones(64, np.float32)
    k = np.ones((1, 64), np.float32)
    v = np.arange(64, dtype=np.float32)[None, :] / 7
    assert np.array_equal(orc.attend_one(q, k, v, 0), v[0].astype(np.float16).astype(np.float32))


def test_pick_adjust_hand_worked(orc):
    """The penalties of the pick's value function (cuda/model/sample.cu:277-319) on a worked
    case: list [3, 3, 5, 1, 3], presence 0.5, frequency 0.25, repeat penalty 2 over the last
    2 tokens (positions 3 and 4: tokens 1 and 3).
      token 1: -1 - (0.5 + 0.25 * 1) = -1.75, in the window and negative: * 2 = -3.5
      token 3:  3 - (0.5 + 0.25 * 3) =  1.75, in the window and positive: / 2 = 0.875
      token 5:  1 - (0.5 + 0.25 * 1) =  0.25, outside the window
      tokens 0, 2, 4 are not in the list and keep their logit."""
    row = np.array([2.0, -1.0, 0.5, 3.0, -2.0, 1.0], np.float32)
    got = orc.pick_adjust(row, [3, 3, 5, 1, 3], presence=0.5, frequency=0.25,
                          repeat_penalty=2.0, repeat_window=2)
    assert got.tolist() == [2.0, -3.5, 0.5, 0.875, -2.0, 0.25]
    # neutral values leave the row; a window of 0 turns the repeat penalty off
    assert orc.pick_adjust(row, [3, 3]).tolist() == row.tolist()
    assert orc.pick_adjust(row, [3], repeat_penalty=2.0, repeat_window=0).tolist() == row.tolist()
