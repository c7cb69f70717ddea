"""The library's host C code (csrc/ckpt.c, csrc/synth.c) and the oracle (oracle/moe_oracle.c) under
AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU. ckpt.c parses offsets and sizes from layout.bin into
mmapped shards, so besides a valid checkpoint the driver gets corrupted ones (short table, wrong kinds, spans past
a shard, offset overflow, bad shard index, misalignment, missing or empty shard) that must be refused cleanly."""
import os
import shutil
import subprocess

import pytest

from ckpt_synth import REC, write_checkpoint
from helpers import SEED

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "maple-runtime_amd", "csrc")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not shutil.which("gcc"):
        pytest.skip("gcc absent")
    exe = str(tmp_path_factory.mktemp("san") / "san_driver")
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-fno-sanitize-recover=all", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle"),
           os.path.join(ROOT, "tests", "sanitize", "san_driver.c"), os.path.join(CSRC, "ckpt.c"),
           os.path.join(CSRC, "synth.c"), os.path.join(ROOT, "oracle", "moe_oracle.c"), "-lpthread", "-lm", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def run(exe, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, *args], capture_output=True, text=True, env=env, timeout=300)
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr[-3000:])
    return r.stdout


def test_synth_clean(driver):
    assert "expert 255 matches the block: 1" in run(driver, "synth")


def test_oracle_clean(driver):
    assert "pack round trip 1" in run(driver, "oracle")


@pytest.fixture(scope="module")
def good_ckpt(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("good"))
    write_checkpoint(d, SEED)
    return d


def test_valid_checkpoint_clean(driver, good_ckpt):
    out = run(driver, "ckpt", good_ckpt)
    assert "open rc 0" in out and "load rc 0 regions 63" in out   # 3 regions x 21 layers
    assert "load past the region table rc -1" in out


def corrupt(src, dst, fn):
    shutil.copytree(src, dst)
    fn(dst)
    return dst


def rewrite_record(d, i, **kw):
    path = os.path.join(d, "layout.bin")
    raw = bytearray(open(path, "rb").read())
    kind, f, off, soff, rows, cols = REC.unpack_from(raw, i * REC.size)
    v = dict(kind=kind, f=f, off=off, soff=soff, rows=rows, cols=cols)
    v.update(kw)
    REC.pack_into(raw, i * REC.size, v["kind"], v["f"], v["off"], v["soff"], v["rows"], v["cols"])
    open(path, "wb").write(raw)


def shift_record(d, i, by):
    off = REC.unpack_from(open(os.path.join(d, "layout.bin"), "rb").read(), i * REC.size)[2]
    rewrite_record(d, i, off=off + by)


GATE_L0_E0 = 3 + 9          # record of layer 0, expert 0, gate
CASES = {
    "short_table": (lambda d: open(os.path.join(d, "layout.bin"), "r+b").truncate(REC.size * 1000), "too short"),
    "wrong_kind": (lambda d: rewrite_record(d, GATE_L0_E0, kind=ord("b")), "expected"),
    "codes_past_shard": (lambda d: rewrite_record(d, GATE_L0_E0, off=1 << 30), "outside shard"),
    "offset_overflow": (lambda d: rewrite_record(d, GATE_L0_E0, off=(1 << 64) - 64), "outside shard"),
    "scales_past_shard": (lambda d: rewrite_record(d, GATE_L0_E0 + 2, soff=(1 << 64) - 16), "outside shard"),
    "bad_shard_index": (lambda d: rewrite_record(d, GATE_L0_E0 + 1, f=200), "shard 200"),
    "bad_shape": (lambda d: rewrite_record(d, GATE_L0_E0, rows=0xFFFFFFFF, cols=0xFFFFFFFF), "expected 512 x 2048"),
    "misaligned": (lambda d: shift_record(d, GATE_L0_E0 + 3 * 5, 4), "aligned"),
    "router_past_shard": (lambda d: rewrite_record(d, 3 + 4, off=(1 << 40)), "router"),
    "missing_shard": (lambda d: os.remove(os.path.join(d, "shard-00007.bin")), "cannot open"),
    "empty_shard": (lambda d: open(os.path.join(d, "shard-00008.bin"), "wb").close(), "cannot map"),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_corrupt_checkpoint_refused(driver, good_ckpt, tmp_path, case):
    fn, msg = CASES[case]
    d = corrupt(good_ckpt, str(tmp_path / case), fn)
    out = run(driver, "ckpt", d)
    assert "open rc -1" in out and msg in out, out
