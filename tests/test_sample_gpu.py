"""Sampler and Philox stream on the GPU vs the oracle: identical logits give the same
token (greedy, top-k, top-p, min-p, temperature), the Random123 known answers, and the
draw counter semantics of aotx_model_draw (cuda/model/sample.cu:594-608)."""
import json
import os

import numpy as np
import pytest

import aotx_amd
from tests.gpu_util import dev, p

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def test_philox_device_kat(torch, lib):
    kat = json.load(open(os.path.join(GOLDEN, "philox_kat.json")))["cases"]
    ctr = np.array([c["ctr"] for c in kat], dtype=np.uint32)
    key = np.array([c["key"] for c in kat], dtype=np.uint32)
    out = torch.zeros(4 * len(kat), dtype=torch.int32, device="cuda")
    assert lib.aotx_philox(p(dev(ctr, torch)), p(dev(key, torch)), len(kat), p(out), None) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(len(kat), 4)
    assert got.tolist() == [c["out"] for c in kat]


def test_philox_device_vs_oracle(torch, lib, orc):
    rng = np.random.default_rng(1)
    n = 512
    ctr = rng.integers(0, 2 ** 32, (n, 4), dtype=np.uint64).astype(np.uint32)
    key = rng.integers(0, 2 ** 32, (n, 2), dtype=np.uint64).astype(np.uint32)
    out = torch.zeros(4 * n, dtype=torch.int32, device="cuda")
    lib.aotx_philox(p(dev(ctr, torch)), p(dev(key, torch)), n, p(out), None)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(n, 4)
    for i in range(n):
        assert got[i].tolist() == orc.philox(ctr[i], key[i]).tolist()


CASES = [(0, 1.0, 0.0), (1, 1.0, 0.8), (40, 0.9, 0.8), (10, 1.0, 1.0), (0, 0.5, 1.0),
         (0, 0.9, 2.0), (0, 1.0, 0.7)]


@pytest.mark.parametrize("vocab", [4096, 128256, 1000])
@pytest.mark.parametrize("top_k,top_p,temp", CASES)
def test_pick_matches_oracle(torch, lib, orc, vocab, top_k, top_p, temp):
    rng = np.random.default_rng(vocab + top_k)
    rows = 24
    logits = (rng.normal(0, 2.5, (rows, vocab))).astype(np.float32)
    logits[3, :] = 1.0                       # all equal: candidates overflow the 256 places
    logits[5, 17] = logits[5, 4113 % vocab] = logits[5].max() + 1   # tied maximum
    agent = (np.arange(rows) * 5 % 64).astype(np.uint32)
    lib.aotx_model_restream()
    tok = torch.zeros(rows, dtype=torch.int32, device="cuda")
    draw = torch.zeros(rows, dtype=torch.int32, device="cuda")
    seed = 0x5EED
    for rep in range(2):
        assert lib.aotx_pick(p(dev(logits, torch)), rows, vocab, p(dev(agent, torch)), None, top_k,
                             top_p, temp, seed, p(tok), p(draw), None) == 0
        torch.cuda.synchronize()
        got = tok.cpu().numpy()
        draws = draw.cpu().numpy()
        for r in range(rows):
            assert draws[r] == rep                      # one draw per row per call
            want, _, allowed = orc.pick(logits[r], top_k, top_p, 0.0, temp, seed, int(agent[r]), rep)
            assert got[r] == want, (r, got[r], want)
            assert got[r] in allowed


def test_pick_per_row_how(torch, lib, orc):
    """A per-row sample (aotx_model_how in device memory) overrides the call's four values,
    including min-p."""
    rng = np.random.default_rng(3)
    rows, vocab = 4, 2048
    logits = rng.normal(0, 2, (rows, vocab)).astype(np.float32)
    hows = (aotx_amd.ModelHow * rows)()
    spec = [(0.0, 0, 1.0, 0.0, 1), (0.8, 40, 0.9, 0.0, 2), (1.0, 0, 1.0, 0.5, 3), (1.5, 5, 1.0, 0.0, 4)]
    for i, (t, k, tp, mp, sd) in enumerate(spec):
        hows[i] = aotx_amd.neutral_how(temperature=t, top_k=k, top_p=tp, min_p=mp, seed=sd)
    hbuf = torch.from_numpy(np.frombuffer(bytes(hows), dtype=np.uint8).copy()).cuda()
    agent = np.array([1, 2, 3, 4], dtype=np.uint32)
    lib.aotx_model_restream()
    tok = torch.zeros(rows, dtype=torch.int32, device="cuda")
    assert lib.aotx_pick(p(dev(logits, torch)), rows, vocab, p(dev(agent, torch)), p(hbuf), 0, 1.0,
                         0.0, 0, p(tok), None, None) == 0
    torch.cuda.synchronize()
    for i, (t, k, tp, mp, sd) in enumerate(spec):
        want = orc.pick(logits[i], k, tp, mp, t, sd, int(agent[i]), 0)[0]
        assert tok.cpu().numpy()[i] == want


def test_pick_distribution_chi_square(torch, lib, orc):
    """12,800 draws over positions of one row follow the allowed-set probabilities
    (tests/sample_test.cu:231-259)."""
    rng = np.random.default_rng(9)
    vocab = 4096
    row = rng.normal(0, 2, vocab).astype(np.float32)
    n = 12800
    logits = np.tile(row, (64, 1))
    agent = np.zeros(64, dtype=np.uint32)
    counts = {}
    lib.aotx_model_restream()
    tok = torch.zeros(64, dtype=torch.int32, device="cuda")
    ld, ad = dev(logits, torch), dev(agent, torch)
    for _ in range(n // 64):
        lib.aotx_pick(p(ld), 64, vocab, p(ad), None, 40, 0.9, 0.8, 99, p(tok), None, None)
        torch.cuda.synchronize()
        for t in tok.cpu().numpy():
            counts[int(t)] = counts.get(int(t), 0) + 1
    _, _, allowed = orc.pick(row, 40, 0.9, 0.0, 0.8, 99, 0, 0)
    vals = row[allowed].astype(np.float64)
    w = np.exp((vals - vals[0]) / 0.8)
    chance = w / w.sum()
    assert set(counts) <= set(allowed.tolist())
    chi, used = 0.0, 0
    for i, c in zip(allowed, chance):
        want = c * n
        if want >= 5:
            chi += (counts.get(int(i), 0) - want) ** 2 / want
            used += 1
    dof = max(used - 1, 1)
    assert chi <= dof + 4 * np.sqrt(2 * dof) + 10


def test_pick_alternating_row_counts(torch, lib, orc):
    """Sampled picks whose calls alternate between row counts (the sampler's buffer is carved
    by the call's row count, so each row's histogram must start at zero whatever an earlier
    call left there): every token matches the oracle's on the same logits and draw."""
    rng = np.random.default_rng(17)
    lib.aotx_model_restream()
    draws = {}
    for rows, vocab in ((8, 4096), (3, 2048), (8, 4096), (5, 3000), (3, 2048)):
        logits = rng.normal(0, 2, (rows, vocab)).astype(np.float32)
        agent = np.arange(rows, dtype=np.uint32) + 10
        tok = torch.zeros(rows, dtype=torch.int32, device="cuda")
        assert lib.aotx_pick(p(dev(logits, torch)), rows, vocab, p(dev(agent, torch)), None, 40, 0.9,
                             0.8, 77, p(tok), None, None) == 0
        torch.cuda.synchronize()
        got = tok.cpu().numpy()
        for i in range(rows):
            a = int(agent[i])
            want = orc.pick(logits[i], 40, 0.9, 0.0, 0.8, 77, a, draws.get(a, 0))[0]
            draws[a] = draws.get(a, 0) + 1
            assert got[i] == want, (rows, vocab, i)
