"""The C-ABI library loads without a GPU, exports every entry point include/*.h
declares, and the ctypes mirror of its structs has the C layout."""
import ctypes
import os
import re
import subprocess

import pytest

import aotx_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aotx_hip.h")
PLAN_HEADER = os.path.join(ROOT, "include", "aotx_plan.h")
TEXT_HEADER = os.path.join(ROOT, "include", "aotx_text.h")
HEADERS = sorted(os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))
                 if f.endswith(".h"))


def declared_functions():
    names = set()
    for path in HEADERS:
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^[A-Za-z_][\w \*]*?\b(aotx_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(aotx_amd.PROTOTYPES), set(names) ^ set(aotx_amd.PROTOTYPES)
    assert not aotx_amd.MISSING


def test_version_without_gpu(lib):
    assert lib.aotx_version().startswith(b"aotx-mi355x")


def test_refusals_without_gpu(lib):
    """Argument checks that refuse before any device work (return 1, as the reference)."""
    assert lib.aotx_model_open(9, 16) == 1
    assert lib.aotx_model_open(2, 0) == 1
    assert lib.aotx_model_open(2, 513) == 1
    assert lib.aotx_model_set_desc(0, None) == 1
    assert lib.aotx_mem_weights_set(0, 0) == 1
    assert lib.aotx_q8_gemv(None, 1, 32, None, 1, None, None) == 1
    assert lib.aotx_q8_gemv(ctypes.c_void_p(8), 1, 33, ctypes.c_void_p(8), 1, ctypes.c_void_p(8), None) == 1
    assert lib.aotx_pick(None, 1, 1, None, None, 0, 1.0, 0.0, 0, None, None, None) == 1


STRUCTS = {
    "aotx_model_desc": aotx_amd.ModelDesc,
    "aotx_model_how": aotx_amd.ModelHow,
    "aotx_model_run": aotx_amd.ModelRun,
    "aotx_kv_map": aotx_amd.KvMap,
    "aotx_kv_table": aotx_amd.KvTable,
    "aotx_plan_slot": aotx_amd.PlanSlot,
    "aotx_plan_state": aotx_amd.PlanState,
    "aotx_token_record": aotx_amd.TokenRecord,
    "aotx_text_source": aotx_amd.TextSource,
    "aotx_text_store": aotx_amd.TextStore,
}


def test_struct_layouts_match_c(tmp_path):
    fields = {
        "aotx_model_desc": ["layers", "rope_theta", "kind", "rms_eps", "token_embd", "layer", "layer_type"],
        "aotx_model_how": ["top_k", "seed", "think_limit", "voice_scale"],
        "aotx_model_run": ["ids", "seed", "seqs", "select", "temperature", "how", "capture_count"],
        "aotx_kv_map": ["limit", "held", "free_count", "created"],
        "aotx_kv_table": ["count", "made", "served", "queue"],
        "aotx_plan_slot": ["state", "page_limit", "seed", "sample", "stop", "draw"],
        "aotx_plan_state": ["offset", "how", "place", "asked", "kept", "cursor", "seqs", "short_of", "steps", "records"],
        "aotx_token_record": ["position", "seed", "draw", "role"],
        "aotx_text_source": ["tokens", "merge_bytes", "merges", "token_type", "family"],
        "aotx_text_store": ["blocks", "bytes"],
    }
    src = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', f'#include "{PLAN_HEADER}"', f'#include "{TEXT_HEADER}"', 'int main(void){']
    for name, fl in fields.items():
        src.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for f in fl:
            src.append(f'printf("{name}.{f} %zu\\n", offsetof({name}, {f}));')
    src.append("return 0;}")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(c)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    for line in out.split("\n"):
        if not line:
            continue
        key, val = line.split()
        if "." in key:
            s, f = key.split(".")
            assert getattr(STRUCTS[s], f).offset == int(val), key
        else:
            assert ctypes.sizeof(STRUCTS[key]) == int(val), key
