"""maple.c's CPU-fallback contract (maple.c:1103-1105, 1149-1158): when gpux_init / gpre_init return -1 the
reference prints "unavailable" and keeps that work on its CPU. Here the unchanged maple.c, built as its GPU build
against libmaplemoe.so (oracle/_ref/maple_gpu), runs in a container without a GPU: the library's init calls must
refuse cleanly (no crash, no hang), maple.c must take its fallback, exit 0, and generate exactly the tokens (and
logits) of its own all-CPU run. CPU only: on a machine with a GPU the card would be used instead."""
import os
import subprocess

import numpy as np
import pytest

from ckpt_synth import VOCAB, write_model_checkpoint

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "oracle", "_ref", "maple_gpu")


@pytest.mark.skipif(not os.path.exists(EXE), reason="oracle/_ref/maple_gpu not built (make -C oracle ref)")
@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present: the fallback only shows without one")
def test_maple_c_falls_back_to_cpu_without_a_card(tmp_path):
    d = str(tmp_path / "model")
    os.makedirs(d)
    nv = write_model_checkpoint(d, 20261202)
    ids = ",".join(str((i * 977 + 13) % nv) for i in range(40))

    def run(tag, args):
        dump = str(tmp_path / f"{tag}.bin")
        r = subprocess.run([EXE, d, "--ids", ids, "--n", "4", "--threads", "4", "--nowarm", "--dump", dump] + args,
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-3000:]
        return r.stdout.split(), r.stderr, np.fromfile(dump, np.float32).reshape(-1, VOCAB)

    toks_cpu, err_cpu, lg_cpu = run("cpu", [])
    assert "unavailable" not in err_cpu
    toks, err, lg = run("fallback", ["--gpupre", "64", "--gpux", "16"])
    print("\n" + err)
    assert "gpu expert cache unavailable" in err          # maple.c:1103-1105 after gpux_init returned -1
    assert "prompt on the card unavailable, using cpu" in err   # maple.c:1106 after gpre_init returned -1
    assert "no HIP device" in err                        # the library's own reason, on stderr
    assert toks == toks_cpu and len(toks) == 4
    assert np.array_equal(lg, lg_cpu)
