"""The C-ABI library loads and exports every function include/maplemoe.h declares (no GPU needed)."""
import ctypes as C
import os
import re

import maplemoe as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    with open(os.path.join(ROOT, "include", "maplemoe.h")) as f:
        src = f.read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(\w+)\s*\([^;]*\)\s*;", src, flags=re.M)))


def test_exports_every_declared_symbol():
    names = declared()
    assert len(names) > 50 and "gpre_moe" in names and "gfull_moe" in names and "gpux_begin_multi" in names
    lib = C.CDLL(M.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_synth_library_exports_its_header():
    with open(os.path.join(ROOT, "include", "maplesynth.h")) as f:
        src = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    names = sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(\w+)\s*\([^;]*\)\s*;", src, flags=re.M)))
    assert len(names) == 6
    slib = C.CDLL(M.SYNTH_PATH)
    assert all(hasattr(slib, n) for n in names)
    prod = C.CDLL(M.LIB_PATH)   # the product library carries no bench tooling
    assert not any(hasattr(prod, n) for n in names)


def test_reference_entry_points_present():
    # every prototype maple.c declares for its GPU path (maple.c:247-272)
    want = ["gpu_head_init", "gpu_head_init_i8", "gpu_head_run", "gpu_head_run_multi", "gpux_init", "gpux_upload",
            "gpux_begin", "gpux_end", "gpux_begin_multi", "gpux_end_multi", "gpre_init", "gpre_region", "gpre_moe",
            "gpre_stage", "gpre_dense_add", "gpre_dense_done", "gpre_dense", "gpre_blit_seconds", "gfull_init",
            "gfull_begin", "gfull_attn", "gfull_moe", "gfull_read", "gfull_write_x", "gfull_maxtok", "gfull_report"]
    assert set(want) <= set(declared())


def test_fails_loudly_without_gpu():
    if os.path.exists("/dev/kfd"):
        return
    lib = M.lib()
    assert lib.mmoe_init(8) == -1 and b"device" in lib.mmoe_last_error()
    assert lib.gpre_init(8, 8) == -1
