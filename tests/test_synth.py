"""The synthetic-weight generator: the numpy statement, the library's host function and
(on the GPU) the device kernel write the same bytes."""
import ctypes

import numpy as np
import pytest

from aotx_amd.model import normal, quantize_q8, synth_q8


def test_numpy_equals_library_host(lib):
    for rows, k, seed in ((3, 64, 1), (17, 256, 99), (5, 4096, 0x5EED)):
        want = synth_q8(rows, k, 0.02, seed).reshape(-1)
        got = np.empty(want.size, dtype=np.uint8)
        assert lib.aotx_synth_q8_host(got.ctypes.data_as(ctypes.c_void_p), rows, k, 0.02, seed, 2) == 0
        assert np.array_equal(got, want)
    vals = normal(7, 0, 1000) * np.float32(0.5)
    got = np.empty(1000, dtype=np.uint16)
    assert lib.aotx_synth_f16_host(got.ctypes.data_as(ctypes.c_void_p), 1000, 0.5, 7, 1) == 0
    assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))


def test_normal_moments():
    z = normal(3, 0, 200000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert z.min() >= -6 and z.max() <= 6


def test_quantizer_round_trip():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (8, 64)).astype(np.float32)
    q = quantize_q8(w).reshape(8, 2, 34)
    d = q[:, :, :2].copy().view(np.float16).astype(np.float32)
    qq = q[:, :, 2:].copy().view(np.int8).astype(np.float32)
    back = (qq * d).reshape(8, 64)
    assert np.abs(back - w).max() <= np.abs(w).max() / 127 * 0.51 + 1e-6
    assert np.abs(qq).max() == 127
