"""aotx_amd — MI355X (gfx950) token loop of AOTX-1 behind the reference's C ABI.

The product is the native library ``libaotx_hip.so`` (HIP kernels + C++ host runtime),
whose entry points are declared in ``include/aotx_hip.h``. This module only loads that
library with ctypes and declares the prototypes, so Python callers (tests, bench) call
exactly what a C caller would. There is no fallback: a missing library raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("AOTX_HIP_LIB") or os.path.join(HERE, "libaotx_hip.so")

AOTX_SLOTS = 64
AOTX_SEQ_MAX_TOKENS = 8192
AOTX_KV_PAGES_EACH = 640
AOTX_KV_PAGES_MAX = 65536
AOTX_KV_PAGE_BYTES = 2 * 1024 * 1024
AOTX_KV_QUEUE_MAX = 256
AOTX_KVL_BLOCK = 16
AOTX_KVL_HEADER = 256
AOTX_MODEL_MAX_TOKENS = 512
AOTX_MODEL_MAX_LAYERS = 64
AOTX_LAYER_TENSOR_SLOTS = 14
AOTX_MODEL_STEERS = 2
AOTX_MODEL_EMBEDDING = 0
AOTX_MODEL_RERANKER = 1
AOTX_MODEL_LANGUAGE = 2
AOTX_WEIGHT_F32 = 0
AOTX_WEIGHT_F16 = 1
AOTX_WEIGHT_Q8_0 = 8
AOTX_LAYER_KIND_ATTENTION = 0
AOTX_LAYER_KIND_ATTENTION_NO_QK_NORM = 1
AOTX_LAYER_KIND_FFN_EXPERTS = 2
AOTX_ROPE_PAIRS_SPLIT = 0
AOTX_ROPE_PAIRS_ADJACENT = 1
AOTX_MODEL_ABSENT = (1 << 64) - 1
AOTX_MODEL_ROWS_ALL = 0
AOTX_MODEL_ROWS_LAST = 1
AOTX_MODEL_CONDUCT_NONE = 0xFFFFFFFF

SLOT = dict(attn_norm=0, attn_q=1, attn_k=2, attn_v=3, attn_o=4, q_norm=5, k_norm=6,
            ffn_norm=7, ffn_gate=8, ffn_up=9, ffn_down=10, router=11)

u32, u64, f32, i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_int32
vp = ctypes.c_void_p


class ModelLayer(ctypes.Structure):
    _fields_ = [("offset", u64 * AOTX_LAYER_TENSOR_SLOTS)]


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("role", u32), ("layers", u32), ("probe_layer", u32), ("hidden", u32), ("ffn", u32),
        ("heads", u32), ("kv_heads", u32), ("head_dim", u32), ("vocab", u32),
        ("context", u32), ("weight_type", u32), ("embd_type", u32), ("tied_output", u32),
        ("pooling", u32), ("rope_theta", f32), ("kind", ctypes.c_uint8 * AOTX_MODEL_MAX_LAYERS),
        ("rms_eps", f32), ("rope_pairs", u32), ("expert_count", u32),
        ("expert_used_count", u32), ("delta_dim", u32), ("delta_heads", u32),
        ("delta_key_heads", u32), ("delta_conv", u32), ("delta_inner", u32), ("rope_dim", u32),
        ("token_embd", u64), ("output_norm", u64), ("output", u64), ("cls_output", u64),
        ("rope_freqs", u64), ("layer", ModelLayer * AOTX_MODEL_MAX_LAYERS),
        ("layer_type", (ctypes.c_uint8 * AOTX_LAYER_TENSOR_SLOTS) * AOTX_MODEL_MAX_LAYERS),
    ]


class ModelHow(ctypes.Structure):
    _fields_ = [
        ("temperature", f32), ("top_k", u32), ("top_p", f32), ("min_p", f32),
        ("repeat_penalty", f32), ("repeat_window", u32), ("presence_penalty", f32),
        ("frequency_penalty", f32), ("seed", u64), ("think_limit", i32),
        ("steer", u32 * AOTX_MODEL_STEERS), ("steer_strength", f32 * AOTX_MODEL_STEERS),
        ("steer_from", u32), ("voice", u32), ("affect", u32), ("voice_scale", f32),
    ]


def neutral_how(**kw):
    """A how row with the neutral values of the reference (greedy, no cut)."""
    h = ModelHow()
    h.temperature = 0.0
    h.top_k = 0
    h.top_p = 1.0
    h.min_p = 0.0
    h.repeat_penalty = 1.0
    h.think_limit = -1
    for i in range(AOTX_MODEL_STEERS):
        h.steer[i] = AOTX_MODEL_CONDUCT_NONE
    h.voice = AOTX_MODEL_CONDUCT_NONE
    h.voice_scale = 1.0
    for k, v in kw.items():
        setattr(h, k, v)
    return h


class ModelRun(ctypes.Structure):
    _fields_ = [
        ("ids", vp), ("input", vp), ("offset", vp), ("agent", vp), ("logits", vp),
        ("pooled", vp), ("score", vp), ("token", vp), ("draw", vp), ("seed", u64),
        ("seqs", u32), ("tokens", u32), ("rows", u32), ("select", u32), ("top_k", u32),
        ("top_p", f32), ("temperature", f32), ("how", vp), ("telemetry", u32),
        ("capture", vp), ("capture_layer", vp), ("capture_count", u32),
    ]


AOTX_MODEL_ROLES = 5
AOTX_SEQ_TICK_BUDGET = 512
AOTX_SEQ_STATE_FREE, AOTX_SEQ_STATE_PREFILL, AOTX_SEQ_STATE_DECODE, AOTX_SEQ_STATE_DONE = 0, 1, 2, 3


class PlanSlot(ctypes.Structure):
    """include/aotx_plan.h aotx_plan_slot (the reference's aotx_seq fields the plan reads)."""
    _fields_ = [("state", u32), ("role", u32), ("prompt", u32), ("sampled", u32),
                ("limit", u32), ("page_limit", u32), ("seed", u64), ("sample", ModelHow),
                ("stop", u32), ("flags", u32), ("last", u32), ("reserved", u32), ("draw", u64)]


class TokenRecord(ctypes.Structure):
    """include/aotx_plan.h aotx_token_record (cuda/seam/wire.h:190-200 without the text)."""
    _fields_ = [("slot", u32), ("token", u32), ("position", u32), ("flags", u32), ("seed", u64),
                ("draw", u64), ("role", u32), ("reserved", u32)]


class PlanState(ctypes.Structure):
    """include/aotx_plan.h aotx_plan_state (cuda/model/decode_state.cuh:35-55)."""
    _fields_ = [
        ("ids", i32 * AOTX_SEQ_TICK_BUDGET), ("offset", u32 * (AOTX_SLOTS + 1)),
        ("agent", u32 * AOTX_SLOTS), ("how", ModelHow * AOTX_SLOTS), ("rows", u32 * AOTX_SLOTS),
        ("first", u32 * AOTX_SLOTS), ("place", u32 * AOTX_SLOTS), ("asked", u32 * AOTX_SLOTS),
        ("kept", u32 * AOTX_SLOTS), ("cursor", u32 * AOTX_MODEL_ROLES), ("seqs", u32),
        ("tokens", u32), ("waited", u32), ("short_of", u32), ("steps", u64), ("records", u32),
        ("dropped", u32), ("refused", u32), ("reserved", u32),
    ]


class TextSource(ctypes.Structure):
    """include/aotx_text.h aotx_text_source (cuda/text/text.cuh:128-137); host arrays."""
    _fields_ = [("token_bytes", vp), ("token_at", vp), ("tokens", u64), ("merge_bytes", vp),
                ("merge_at", vp), ("merges", u64), ("token_type", vp), ("family", u32)]


class TextStore(ctypes.Structure):
    """include/aotx_text.h aotx_text_store (cuda/text/text.cuh:146-150)."""
    _fields_ = [("block", vp * 8), ("blocks", u32), ("bytes", u64)]


class KvEntry(ctypes.Structure):
    _fields_ = [("agent", u32), ("pages", u32)]


class KvMap(ctypes.Structure):
    _fields_ = [
        ("range", u64), ("range_bytes", u64), ("limit", u32),
        ("held", u32 * AOTX_KV_PAGES_MAX), ("free_at", u32 * AOTX_KV_PAGES_MAX),
        ("free_count", u32), ("created", u32),
    ]


class KvTable(ctypes.Structure):
    _fields_ = [
        ("page", (u64 * AOTX_KV_PAGES_EACH) * AOTX_SLOTS), ("count", u32 * AOTX_SLOTS),
        ("mapped_pages", u32), ("short_of", u32), ("made", u32), ("served", u32),
        ("refused", u32), ("queue", KvEntry * AOTX_KV_QUEUE_MAX),
    ]


# name -> (restype, argtypes). Every symbol declared in include/aotx_hip.h.
AOTX_TENSOR_NAME_BYTES = 128
AOTX_TENSOR_DIMS = 4
AOTX_DESC_WHOLE = 5
AOTX_DESC_BUFFER = 48
AOTX_DESC_MAX_BINDINGS = AOTX_DESC_WHOLE + AOTX_MODEL_MAX_LAYERS * AOTX_LAYER_TENSOR_SLOTS


class TensorInfo(ctypes.Structure):
    """include/aotx_modelfile.h aotx_tensor_info (modelfile.h:97-104)."""
    _fields_ = [("name", ctypes.c_char * AOTX_TENSOR_NAME_BYTES), ("dim_count", u32),
                ("type", u32), ("dims", u64 * AOTX_TENSOR_DIMS), ("offset", u64),
                ("bytes", u64)]


class StringArray(ctypes.Structure):
    _fields_ = [("count", u64), ("bytes", ctypes.POINTER(ctypes.c_uint8)),
                ("offsets", ctypes.POINTER(u64))]


class ModelBinding(ctypes.Structure):
    """include/aotx_modelfile.h aotx_model_binding (forward.cuh:290-294)."""
    _fields_ = [("name", ctypes.c_char * AOTX_DESC_BUFFER), ("slot", u32), ("needed", u32)]


PROTOTYPES = {
    "aotx_mem_weights_set": (i32, [u64, u64]),
    "aotx_mem_weights_base": (u64, []),
    "aotx_model_set_desc": (i32, [u32, ctypes.POINTER(ModelDesc)]),
    "aotx_model_open": (i32, [u32, u32]),
    "aotx_model_shut": (None, [u32]),
    "aotx_model_forget": (None, []),
    "aotx_model_restream": (None, []),
    "aotx_model_faulted": (u32, []),
    "aotx_model_nodes": (u32, [u32]),
    "aotx_model_pages": (i32, [u32, vp, u32, vp]),
    "aotx_model_launch": (i32, [u32, ctypes.POINTER(ModelRun)]),
    "aotx_model_sample": (i32, [u32, vp, vp, u32, vp, ctypes.POINTER(ModelHow), vp, vp,
                                ctypes.POINTER(u64)]),
    "aotx_model_prefill": (i32, [u32, vp, vp, u32, vp, vp, vp]),
    "aotx_model_probe": (i32, [u32, vp, vp, u32, vp, vp, vp, u32, vp, vp, u32]),
    "aotx_model_buffer": (u64, [u32, u32]),
    "aotx_model_rerank": (i32, [vp, vp, u32, vp, vp]),
    "aotx_model_graphs": (None, [u32]),
    "aotx_model_seat": (i32, [u32, u32]),
    # the tick plan (include/aotx_plan.h)
    "aotx_decode_plan": (i32, [u32, vp, vp, u32, u32, u32, vp, vp]),
    "aotx_model_kv_pages": (u32, [u32, u32]),
    "aotx_decode_commit": (i32, [u32, vp, vp, u32, vp, vp, vp, vp, u32, vp]),
    "aotx_decode_tick": (i32, [u32, vp, vp, u32, u32, u32, vp, vp, u32, vp]),
    "aotx_seq_apply": (i32, [u32, vp, vp, u32, vp, vp, u32, vp]),
    # the tokenizer (include/aotx_text.h)
    "aotx_text_family_find": (i32, [ctypes.c_char_p, u64, ctypes.POINTER(u32)]),
    "aotx_text_vocab_build": (i32, [ctypes.POINTER(TextSource), ctypes.POINTER(TextStore)]),
    "aotx_text_vocab_release": (None, [ctypes.POINTER(TextStore)]),
    "aotx_text_vocab_report": (i32, [ctypes.POINTER(u32)]),
    "aotx_text_vocab_file": (i32, [vp, ctypes.POINTER(TextStore)]),
    "aotx_text_encode": (i32, [vp, vp, u32, vp, vp, vp]),
    "aotx_text_detok": (i32, [vp, vp, u32, vp, u32, vp, vp]),
    "aotx_kv_open": (i32, [ctypes.POINTER(KvMap)]),
    "aotx_kv_reserve": (i32, [ctypes.POINTER(KvMap)]),
    "aotx_kv_serve": (i32, [ctypes.POINTER(KvMap), vp]),
    "aotx_kv_close": (None, [ctypes.POINTER(KvMap)]),
    "aotx_kv_request": (i32, [u32, u32]),
    "aotx_kv_release": (i32, [u32]),
    "aotx_kv_table_read": (i32, [ctypes.POINTER(KvTable)]),
    "aotx_kv_table_device": (u64, []),
    "aotx_q8_gemv": (i32, [vp, u32, u32, vp, u32, vp, vp]),
    "aotx_q8_gemv_f16": (i32, [vp, u32, u32, vp, u32, vp, vp]),
    "aotx_q8_dequant": (i32, [vp, u32, u32, u32, vp, vp]),
    "aotx_q8r_size": (u64, [u32, u32]),
    "aotx_q8_repack": (i32, [vp, u32, u32, vp, vp]),
    "aotx_q8r_gemv": (i32, [vp, u32, u32, vp, u32, vp, vp]),
    "aotx_q8r_gemv_f16": (i32, [vp, u32, u32, vp, u32, vp, vp]),
    "aotx_attend_paged": (i32, [vp, vp, vp, u32, u32, u32, u32, u32, u32, vp, vp]),
    "aotx_attend_paged_static": (i32, [vp, vp, vp, u32, u32, u32, u32, u32, u32, vp, vp]),
    "aotx_kv_write": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "aotx_pick": (i32, [vp, u32, u32, vp, vp, u32, f32, f32, u64, vp, vp, vp]),
    "aotx_philox": (i32, [vp, vp, u32, vp, vp]),
    "aotx_expert_route": (i32, [vp, vp, u32, u32, u32, u32, vp, vp, vp]),
    "aotx_expert_ffn": (i32, [vp, vp, vp, u32, u32, u32, u32, vp, u32, vp, vp, vp, vp]),
    "aotx_synth_q8": (i32, [vp, u64, u32, f32, u64, vp]),
    "aotx_synth_q8_host": (i32, [vp, u64, u32, f32, u64, u32]),
    "aotx_synth_f16": (i32, [vp, u64, f32, u64, vp]),
    "aotx_synth_f16_host": (i32, [vp, u64, f32, u64, u32]),
    "aotx_version": (ctypes.c_char_p, []),
    # GGUF model files (include/aotx_modelfile.h)
    "aotx_modelfile_open": (i32, [ctypes.c_char_p, ctypes.POINTER(vp)]),
    "aotx_modelfile_close": (None, [vp]),
    "aotx_modelfile_file_bytes": (u64, [vp]),
    "aotx_modelfile_header_bytes": (u64, [vp]),
    "aotx_modelfile_u32": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(u32)]),
    "aotx_modelfile_u64": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(u64)]),
    "aotx_modelfile_f32": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(f32)]),
    "aotx_modelfile_string": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                    ctypes.POINTER(ctypes.c_size_t)]),
    "aotx_modelfile_strings": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(StringArray)]),
    "aotx_modelfile_i32s": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                  ctypes.POINTER(u64)]),
    "aotx_modelfile_f32s": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                  ctypes.POINTER(u64)]),
    "aotx_modelfile_bools": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                   ctypes.POINTER(u64)]),
    "aotx_modelfile_tensor_count": (u64, [vp]),
    "aotx_modelfile_tensor": (i32, [vp, u64, ctypes.POINTER(TensorInfo)]),
    "aotx_modelfile_find": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(TensorInfo)]),
    "aotx_modelfile_data_bytes": (u64, [vp]),
    "aotx_modelfile_read": (i32, [vp, u64, u64, vp]),
    "aotx_model_desc_file": (i32, [vp, u32, ctypes.POINTER(ModelDesc), ctypes.POINTER(ModelBinding),
                                   u32, ctypes.POINTER(u32), ctypes.c_char_p, ctypes.c_size_t]),
    "aotx_model_place_bytes": (u64, [vp, ctypes.POINTER(ModelBinding), u32]),
    "aotx_model_place": (i32, [vp, ctypes.POINTER(ModelDesc), ctypes.POINTER(ModelBinding), u32,
                               ctypes.c_char_p, ctypes.c_size_t]),
}

_lib = None
MISSING = []  # declared symbols the loaded library does not export


def lib():
    """The loaded native library. Raises if it was not built: there is no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m aotx_amd.build` "
                "(the HIP path has no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in PROTOTYPES.items():
            try:
                fn = getattr(handle, name)
            except AttributeError:
                MISSING.append(name)
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def ptr(t):
    """Device (or host) address of a torch tensor, or None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(torch_stream=None):
    import torch
    s = torch_stream or torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} refused (returned {rc})")
    return rc
