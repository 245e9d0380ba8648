"""The CPU oracle under the sanitizers: tests/c/oracle_san.c drives every
function family (quantizers, dequant, block sums, both dot forms, the x4
matmul through the pthread pool, windowed ring attention, the sampling chain)
built with AddressSanitizer + UndefinedBehaviorSanitizer and, separately,
ThreadSanitizer for the pool.  Any report aborts the run (-fno-sanitize-recover)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORA = os.path.join(ROOT, "oracle")
SRCS = [os.path.join(ROOT, "tests", "c", "oracle_san.c")] + [os.path.join(ORA, f) for f in
                                                            ("g4o_quants.c", "g4o_model.c", "g4o_sampler.c", "g4o_gemma.c")]


@pytest.mark.parametrize("san", ["address,undefined", "thread"])
def test_oracle_is_clean_under_sanitizers(tmp_path, san):
    exe = str(tmp_path / "oracle_san")
    cmd = ["gcc", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=" + san, "-fno-sanitize-recover=all",
           "-march=x86-64-v3", "-ffp-contract=off", "-I" + ORA] + SRCS + ["-lm", "-lpthread", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.stdout + r.stderr)[-3000:]
