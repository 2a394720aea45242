"""Q8_0 product on the GPU vs the oracle (tests/matrix_test.cu strategy): tolerance
1e-2 of max(|want|, rms) at small shapes in full, spot checks at the benchmark shapes,
the transposed-operand control, fp16 output, and bit-exact dequantisation."""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import dev, p, rel_rms

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def make(torch, lib, n, k, seed):
    w = torch.empty(n * (k // 32) * 34, dtype=torch.uint8, device="cuda")
    assert lib.aotx_synth_q8(p(w), n, k, 0.02, seed, None) == 0
    return w


@pytest.mark.parametrize("n,k", [(64, 256), (128, 704), (80, 128), (1000, 4096), (256, 14336)])
@pytest.mark.parametrize("m", [1, 3, 8, 17, 32, 40])
def test_gemv_small_full(torch, lib, orc, n, k, m):
    w = make(torch, lib, n, k, 7 + n + k)
    rng = np.random.default_rng(n * 131 + m)
    x = rng.normal(0, 1, (m, k)).astype(np.float16)
    xd = dev(x, torch)
    y = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    assert lib.aotx_q8_gemv(p(w), n, k, p(xd), m, p(y), None) == 0
    torch.cuda.synchronize()
    want = orc.q8_gemv_f64(w.cpu().numpy(), n, k, x.view(np.uint16))
    assert rel_rms(y.cpu().numpy().reshape(m, n), want) < TOL


@pytest.mark.parametrize("n,k", [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)])
@pytest.mark.parametrize("m", [1, 4, 8, 32])
def test_gemv_benchmark_shapes_spot(torch, lib, orc, n, k, m):
    """64 spot checks against a double dot product of the same bytes
    (tests/matrix_test.cu:279-312) plus an fp16-output run."""
    w = make(torch, lib, n, k, 1234)
    rng = np.random.default_rng(m)
    x = rng.normal(0, 1, (m, k)).astype(np.float16)
    xd = dev(x, torch)
    y = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    y16 = torch.zeros(m * n, dtype=torch.float16, device="cuda")
    assert lib.aotx_q8_gemv(p(w), n, k, p(xd), m, p(y), None) == 0
    assert lib.aotx_q8_gemv_f16(p(w), n, k, p(xd), m, p(y16), None) == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(m, n)
    got16 = y16.cpu().numpy().reshape(m, n)
    wn = w.cpu().numpy().reshape(n, -1)
    rows = rng.integers(0, n, 64)
    want = orc.q8_gemv_f64(np.ascontiguousarray(wn[rows]), 64, k, x.view(np.uint16))
    rms = np.sqrt((want ** 2).mean())
    err = np.abs(got[:, rows] - want) / np.maximum(np.abs(want), rms)
    assert err.max() < TOL
    assert np.array_equal(got16, got.astype(np.float16))


def test_gemv_transposed_control(torch, lib, orc):
    n = k = 256
    w = make(torch, lib, n, k, 77)
    x = np.random.default_rng(1).normal(0, 1, (2, k)).astype(np.float16)
    y = torch.zeros(2 * n, dtype=torch.float32, device="cuda")
    assert lib.aotx_q8_gemv(p(w), n, k, p(dev(x, torch)), 2, p(y), None) == 0
    torch.cuda.synchronize()
    wn = w.cpu().numpy()
    right = orc.q8_gemv_f64(wn, n, k, x.view(np.uint16))
    swapped = orc.q8_gemv_f64(wn, n, k, x.view(np.uint16), swap=True)
    got = y.cpu().numpy().reshape(2, n)
    assert rel_rms(got, right) < TOL
    assert rel_rms(got, swapped) > 0.1


def test_dequant_bit_exact(torch, lib, orc):
    """Dequantised rows equal half(q * scale) of the host reading bit for bit
    (tests/matrix_test.cu:331-345)."""
    n, k = 40, 512
    w = make(torch, lib, n, k, 5)
    out = torch.zeros(10 * k, dtype=torch.float16, device="cuda")
    assert lib.aotx_q8_dequant(p(w), k, 7, 10, p(out), None) == 0
    torch.cuda.synchronize()
    from aotx_amd.model import dequant_q8
    want = dequant_q8(w.cpu().numpy().reshape(n, -1)[7:17], k).astype(np.float16)
    assert np.array_equal(out.cpu().numpy().reshape(10, k).view(np.uint16), want.view(np.uint16))


def test_device_synth_equals_host(torch, lib):
    n, k = 333, 4096
    w = make(torch, lib, n, k, 0xABCDEF)
    host = np.empty(n * (k // 32) * 34, dtype=np.uint8)
    lib.aotx_synth_q8_host(host.ctypes.data_as(ctypes.c_void_p), n, k, 0.02, 0xABCDEF, 4)
    assert np.array_equal(w.cpu().numpy(), host)


def repack(torch, lib, w, n, k):
    size = lib.aotx_q8r_size(n, k)
    assert size > 0
    wr = torch.empty(size, dtype=torch.uint8, device="cuda")
    assert lib.aotx_q8_repack(p(w), n, k, p(wr), None) == 0
    return wr


@pytest.mark.parametrize("n,k", [(64, 256), (128, 704), (80, 128), (1000, 4096), (256, 14336),
                                 (17, 96)])
@pytest.mark.parametrize("m", [1, 3, 6, 8, 16, 17, 32, 40, 33, 128, 300])
def test_repacked_gemv_small_full(torch, lib, orc, n, k, m):
    """The streaming product over repacked weights (the model path) vs the oracle."""
    w = make(torch, lib, n, k, 11 + n + k)
    wr = repack(torch, lib, w, n, k)
    rng = np.random.default_rng(n * 7 + m)
    x = rng.normal(0, 1, (m, k)).astype(np.float16)
    y = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    assert lib.aotx_q8r_gemv(p(wr), n, k, p(dev(x, torch)), m, p(y), None) == 0
    torch.cuda.synchronize()
    want = orc.q8_gemv_f64(w.cpu().numpy(), n, k, x.view(np.uint16))
    assert rel_rms(y.cpu().numpy().reshape(m, n), want) < TOL


@pytest.mark.parametrize("n,k", [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)])
@pytest.mark.parametrize("m", [1, 4, 8, 32, 128, 512])
def test_repacked_gemv_benchmark_shapes(torch, lib, orc, n, k, m):
    w = make(torch, lib, n, k, 4321)
    wr = repack(torch, lib, w, n, k)
    rng = np.random.default_rng(m + 100)
    x = rng.normal(0, 1, (m, k)).astype(np.float16)
    xd = dev(x, torch)
    y = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    y2 = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    assert lib.aotx_q8r_gemv(p(wr), n, k, p(xd), m, p(y), None) == 0
    assert lib.aotx_q8_gemv(p(w), n, k, p(xd), m, p(y2), None) == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(m, n)
    wn = w.cpu().numpy().reshape(n, -1)
    rows = rng.integers(0, n, 64)
    want = orc.q8_gemv_f64(np.ascontiguousarray(wn[rows]), 64, k, x.view(np.uint16))
    rms = np.sqrt((want ** 2).mean())
    assert (np.abs(got[:, rows] - want) / np.maximum(np.abs(want), rms)).max() < TOL
    # both kernels sum the same fp16 products in fp32: they agree far inside the tolerance
    assert rel_rms(got, y2.cpu().numpy().reshape(m, n)) < 1e-4


def test_repack_layout(torch, lib):
    """Repacked bytes: lane l = r + 16 g of (tile t, quad q) holds row 16t + r, block 4q + g;
    its quants 0..15 sit in the first 1 KB half of the (t, q) record, 16..31 in the second,
    each stored as q + 128 (the byte XOR 0x80); padding is q = 0 with scale 0."""
    n, k = 40, 384
    w = make(torch, lib, n, k, 3)
    wr = repack(torch, lib, w, n, k).cpu().numpy()
    src = w.cpu().numpy().reshape(n, k // 32, 34)
    tiles, quads = (n + 15) // 16, (k + 127) // 128
    quant = wr[:tiles * quads * 64 * 32].reshape(tiles, quads, 2, 64, 16).transpose(0, 1, 3, 2, 4)
    quant = quant.reshape(tiles, quads, 64, 32)
    scale = wr[tiles * quads * 64 * 32:].view(np.uint16).reshape(tiles, quads, 64)
    for t in range(tiles):
        for q in range(quads):
            for lane in range(64):
                r, g = lane % 16, lane // 16
                row, blk = 16 * t + r, 4 * q + g
                if row < n and blk < k // 32:
                    assert np.array_equal(quant[t, q, lane], src[row, blk, 2:] ^ 0x80)
                    assert scale[t, q, lane] == src[row, blk, :2].view(np.uint16)[0]
                else:
                    assert (quant[t, q, lane] == 0x80).all() and scale[t, q, lane] == 0
