"""bench.py pieces that run without a GPU: the one-GPU guard and the lookup of a kernel's measured HBM bytes in the
committed rocprofv3 summary (instantiations with further template arguments included)."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_pmc_traffic_lookup():
    import bench
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    rows = {}
    for line in open(path):
        cols = [c.strip() for c in line.split("|")]
        if len(cols) > 6 and cols[1].startswith("k_") and cols[6].isdigit():
            rows.setdefault(cols[1], int(cols[6]))   # a kernel listed at two grid sizes: its first row
    assert rows, "no kernel rows in the traffic summary"
    for name, v in rows.items():
        assert bench.pmc_traffic(name) == v
    # the bench names the gate/up kernel without its tuning arguments
    gu = [n for n in rows if n.startswith("k_gateup_pk<true")]
    assert gu and bench.pmc_traffic("k_gateup_pk<true>") == rows[gu[0]]
    assert bench.pmc_traffic("k_no_such_kernel") is None
