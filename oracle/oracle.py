"""ctypes wrapper of the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only as the checker / the CPU baseline; the product never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, u32, u64, f32, i32 = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64,
                                  ctypes.c_float, ctypes.c_int)
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [f32]
        L.orc_f16_to_f32.restype = f32
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_q8_gemv_f64.argtypes = [vp, u32, u32, vp, u32, vp, i32]
        L.orc_q8_gemv_f32.argtypes = [vp, u32, u32, vp, u32, vp, u32]
        L.orc_philox.argtypes = [vp, vp, vp]
        L.orc_rng_unit.restype = f32
        L.orc_rng_unit.argtypes = [u64, u32, u32, u64]
        L.orc_pick.restype = i32
        L.orc_pick.argtypes = [vp, u32, u32, f32, f32, f32, u64, u32, u64, vp, vp, vp]
        L.orc_pick_adjust.argtypes = [vp, u32, vp, u32, f32, f32, f32, u32]
        L.orc_route.argtypes = [vp, vp, u32, u32, u32, u32, vp, vp]
        L.orc_attend_one.argtypes = [vp, vp, vp, u32, u32, u32, vp]
        L.orc_model_new.restype = vp
        L.orc_model_new.argtypes = [vp, vp, u32, u32, u32]
        L.orc_model_free.argtypes = [vp]
        L.orc_model_forget.argtypes = [vp]
        L.orc_model_step.restype = i32
        L.orc_model_step.argtypes = [vp, vp, vp, u32, vp, vp]
        L.orc_model_seat.restype = i32
        L.orc_model_seat.argtypes = [vp, u32, u32, u64]
        L.orc_model_last_xnorm.restype = ctypes.POINTER(f32)
        L.orc_model_last_xnorm.argtypes = [vp]
        L.orc_model_last_resid.restype = ctypes.POINTER(f32)
        L.orc_model_last_resid.argtypes = [vp]
        L.orc_model_last_route.restype = ctypes.POINTER(f32)
        L.orc_model_last_route.argtypes = [vp, ctypes.POINTER(ctypes.POINTER(u32)), ctypes.POINTER(u32)]
        L.orc_model_cache.restype = ctypes.POINTER(ctypes.c_uint16)
        L.orc_model_cache.argtypes = [vp, u32]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def q8_gemv_f64(w, n, k, x16, swap=False):
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    m = x16.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    lib().orc_q8_gemv_f64(_p(w), n, k, _p(x16), m, _p(y), 1 if swap else 0)
    return y


def q8_gemv_f32(w, n, k, x16, threads=1):
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    m = x16.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    lib().orc_q8_gemv_f32(_p(w), n, k, _p(x16), m, _p(y), threads)
    return y


def philox(ctr, key):
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, dtype=np.uint32)
    lib().orc_philox(_p(c), _p(k), _p(out))
    return out


def pick(row, top_k=0, top_p=1.0, min_p=0.0, temperature=0.0, seed=0, agent=0, position=0):
    row = np.ascontiguousarray(row, dtype=np.float32)
    count = ctypes.c_uint32()
    taken = ctypes.c_uint32()
    allowed = np.zeros(256, dtype=np.uint32)
    tok = lib().orc_pick(_p(row), row.size, top_k, top_p, min_p, temperature, seed, agent,
                         position, ctypes.byref(count), ctypes.byref(taken), _p(allowed))
    return tok, count.value, allowed[:taken.value].copy()


def pick_adjust(row, tokens, presence=0.0, frequency=0.0, repeat_penalty=1.0, repeat_window=0):
    """The row with the sample's penalties over a token list applied (sample.cu:277-319)."""
    out = np.array(row, dtype=np.float32, copy=True)
    lst = np.ascontiguousarray(tokens, dtype=np.int32)
    lib().orc_pick_adjust(_p(out), out.size, _p(lst), lst.size, presence, frequency,
                          repeat_penalty, repeat_window)
    return out


def route(router, x16, experts, used):
    router = np.ascontiguousarray(router, dtype=np.float32)
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    tokens, hidden = x16.shape
    prob = np.empty((tokens, experts), dtype=np.float32)
    ids = np.empty((tokens, used), dtype=np.uint32)
    lib().orc_route(_p(router), _p(x16), tokens, hidden, experts, used, _p(prob), _p(ids))
    return prob, ids


def attend_one(q, keys, values, last):
    q = np.ascontiguousarray(q, dtype=np.float32)
    keys = np.ascontiguousarray(keys, dtype=np.float32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    d = q.size
    out = np.empty(d, dtype=np.float32)
    lib().orc_attend_one(_p(q), _p(keys), _p(values), keys.shape[1], last, d, _p(out))
    return out


class Model:
    """The oracle's whole-model forward over the same descriptor and weight bytes."""

    def __init__(self, desc, weights, slots, max_context, threads=1):
        self.desc = desc
        self.weights = np.ascontiguousarray(weights, dtype=np.uint8)
        self.vocab = desc.vocab
        self.hidden = desc.hidden
        self.max_context = max_context
        self.slots = slots
        self.h = lib().orc_model_new(ctypes.byref(desc), _p(self.weights), slots,
                                     max_context, threads)

    def step(self, ids, offset, agent):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        offset = np.ascontiguousarray(offset, dtype=np.uint32)
        agent = np.ascontiguousarray(agent, dtype=np.uint32)
        seqs = agent.size
        logits = np.empty((seqs, self.vocab), dtype=np.float32)
        rc = lib().orc_model_step(self.h, _p(ids), _p(offset), seqs, _p(agent), _p(logits))
        if rc != 0:
            raise RuntimeError("oracle step refused (slot or context overflow)")
        return logits

    def last_xnorm(self, seqs):
        p = lib().orc_model_last_xnorm(self.h)
        return np.ctypeslib.as_array(p, shape=(seqs * self.hidden,)).reshape(seqs, self.hidden).copy()

    def last_resid(self, seqs):
        """The residual row of each sequence's last token after every layer of the last
        step, [layers][seqs][hidden]."""
        p = lib().orc_model_last_resid(self.h)
        n = self.desc.layers * seqs * self.hidden
        return np.ctypeslib.as_array(p, shape=(n,)).reshape(self.desc.layers, seqs,
                                                            self.hidden).copy()

    def last_route(self):
        """(probabilities [tokens][experts], ids [tokens][used]) of the last experts layer of
        the last step, or None when that step ran no experts layer."""
        ids = ctypes.POINTER(ctypes.c_uint32)()
        tokens = ctypes.c_uint32(0)
        p = lib().orc_model_last_route(self.h, ctypes.byref(ids), ctypes.byref(tokens))
        t = tokens.value
        if t == 0:
            return None
        d = self.desc
        prob = np.ctypeslib.as_array(p, shape=(t * d.expert_count,)).reshape(t, d.expert_count).copy()
        sel = np.ctypeslib.as_array(ids, shape=(t * d.expert_used_count,)).reshape(
            t, d.expert_used_count).copy()
        return prob, sel

    def cache(self):
        """Views of the cache, (keys, values) fp16 words [slots][layers][max_context][kv_heads *
        head_dim], shared with the oracle (valid while the model lives)."""
        d = self.desc
        shp = (self.slots, d.layers, self.max_context, d.kv_heads * d.head_dim)
        out = []
        for which in (0, 1):
            p = lib().orc_model_cache(self.h, which)
            out.append(np.ctypeslib.as_array(p, shape=(int(np.prod(shp)),)).reshape(shp))
        return out

    def seat(self, slots, position, seed=7):
        for s in slots:
            if lib().orc_model_seat(self.h, s, position, seed) != 0:
                raise RuntimeError("oracle seat refused")

    def forget(self):
        lib().orc_model_forget(self.h)

    def __del__(self):
        try:
            lib().orc_model_free(self.h)
        except Exception:
            pass
