"""Helpers of the GPU tests: device buffers and the reference's comparison rule."""
import ctypes

import numpy as np


KEEP = []   # device copies stay alive until the test ends (see the fixture in conftest)


def dev(a, torch):
    """numpy array -> device tensor holding the same bytes. The tensor is kept alive until
    the end of the test, so a raw pointer taken from it stays valid for the kernel."""
    a = np.ascontiguousarray(a)
    t = torch.from_numpy(a.view(np.uint8).reshape(-1).copy()).cuda()
    KEEP.append(t)
    return t


def p(t):
    return ctypes.c_void_p(t.data_ptr())


def rel_rms(got, want):
    """|got - want| / max(|want|, rms(want)) (tests/matrix_test.cu:246-277)."""
    want = np.asarray(want, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    rms = np.sqrt((want ** 2).mean())
    err = np.abs(got - want) / np.maximum(np.abs(want), rms)
    err[~np.isfinite(got)] = np.inf
    return float(err.max())


def read_device(addr, dtype, count):
    """Copy `count` elements of `dtype` from a device address the library handed out (for
    example aotx_model_buffer) into a numpy array, through the HIP runtime the library
    itself is linked against."""
    import aotx_amd
    import torch
    torch.cuda.synchronize()
    out = np.empty(count, dtype=dtype)
    L = aotx_amd.lib()
    L.hipMemcpy.restype = ctypes.c_int
    L.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rc = L.hipMemcpy(out.ctypes.data, ctypes.c_void_p(addr), out.nbytes, 2)  # device to host
    assert rc == 0, f"hipMemcpy returned {rc}"
    return out
