"""The drop-in boundary at build level: maple.c's own prototypes of its GPU entry points (maple.c:246-272,
compiled with -DGPU_HEAD) agree with include/maplemoe.h in one translation unit, and the unchanged maple.c
links against libmaplemoe.so with every GPU symbol resolved by it. Both read maple.c from /root/reference
and are skipped where it is absent (the GPU box); nothing of maple.c is kept in the repository."""
import os
import re
import subprocess

import pytest

import maplemoe as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MAPLE_C = "/root/reference/maple.c"
needs_ref = pytest.mark.skipif(not os.path.exists(MAPLE_C), reason="reference sources absent")


def maple_gpu_block():
    """the text of maple.c's first `#ifdef GPU_HEAD` block: its prototypes of the GPU entry points"""
    src = open(MAPLE_C).read()
    m = re.search(r"^#ifdef GPU_HEAD\n(.*?)^#endif", src, flags=re.S | re.M)
    assert m, "maple.c has no GPU_HEAD prototype block"
    return m.group(1)


@needs_ref
def test_maple_prototypes_match_header(tmp_path):
    block = maple_gpu_block()
    names = re.findall(r"\b(\w+)\s*\(", block)
    assert len(set(names)) == 26 and "gpre_moe" in names and "gpux_begin_multi" in names
    # maple.c's declarations and the header's in one translation unit: any difference in a return or
    # parameter type is a "conflicting types" error
    tu = tmp_path / "proto.c"
    tu.write_text('#include <stdint.h>\n#include <stddef.h>\n#include "maplemoe.h"\n' + block +
                  "\nint proto_probe(void) { return 0; }\n")
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-c", str(tu), "-I", os.path.join(ROOT, "include"),
                        "-o", str(tmp_path / "proto.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # and a deliberately wrong prototype is caught the same way (the check is not vacuous)
    bad = block.replace("int gpre_init(int maxtok, int topk);", "int gpre_init(int maxtok, long topk);")
    assert bad != block
    tu.write_text('#include <stdint.h>\n#include <stddef.h>\n#include "maplemoe.h"\n' + bad)
    r = subprocess.run(["gcc", "-std=c11", "-c", str(tu), "-I", os.path.join(ROOT, "include"), "-o",
                        str(tmp_path / "bad.o")], capture_output=True, text=True)
    assert r.returncode != 0 and "conflicting types" in r.stderr


@needs_ref
def test_unchanged_maple_links_against_library(tmp_path):
    exe = tmp_path / "maple_gpu"
    r = subprocess.run(["gcc", "-O1", "-mavx2", "-mfma", "-mf16c", "-DGPU_HEAD", "-w", "-o", str(exe), MAPLE_C,
                        "-L", os.path.dirname(M.LIB_PATH), "-lmaplemoe", "-Wl,-rpath-link,/opt/rocm/lib",
                        "-Wl,--no-undefined", "-lpthread", "-lm"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    undef = subprocess.run(["nm", "-D", "--undefined-only", str(exe)], capture_output=True, text=True).stdout
    gpu = sorted(set(re.findall(r"\b((?:gpre|gfull|gpux|gpu_head)_\w+)", undef)))
    declared = set(re.findall(r"\b(\w+)\s*\(", maple_gpu_block()))
    assert len(gpu) >= 24 and set(gpu) <= declared, gpu   # the prototypes maple.c's code calls
    exported = subprocess.run(["nm", "-D", "--defined-only", M.LIB_PATH], capture_output=True, text=True).stdout
    assert all(re.search(rf"\bT {n}$", exported, flags=re.M) for n in gpu)
