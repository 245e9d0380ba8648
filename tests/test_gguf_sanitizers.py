"""The GGUF reader (g4run_amd/csrc/gguf.cpp, gguf.c:124-404 on a Linux mmap)
built on the host under AddressSanitizer and UBSan and run over a valid
gemma4 file the test writes, truncations of it and copies with bytes of the
header (metadata and tensor table) overwritten: every file must either parse
with all tensor data inside the mapping or be refused, with no sanitizer
report.  Host code only; runs on the CPU."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import gemma_util as GM

HERE = os.path.dirname(__file__)
CSRC = os.path.join(HERE, "..", "g4run_amd", "csrc")


def _build(tmp):
    exe = os.path.join(tmp, "gguf_parse")
    cmd = ["g++", "-O1", "-g", "-std=c++17", "-fno-omit-frame-pointer", "-fsanitize=address,undefined,float-cast-overflow",
           "-fno-sanitize-recover=all", os.path.join(HERE, "c", "gguf_parse.cpp"), os.path.join(CSRC, "gguf.cpp"),
           os.path.join(CSRC, "types.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_gguf_reader_under_sanitizers(oracle, tmp_path):
    exe = _build(str(tmp_path))
    spec = dict(GM.SMALL, n_layer=2, n_kv_shared=0, n_ff=[256, 256], is_swa=[1, 0], n_vocab=64)
    hp, T = GM.make_gemma(oracle, 3, spec=spec)
    good = str(tmp_path / "good.gguf")
    GM.write_gemma(good, hp, T)
    raw = open(good, "rb").read()
    # where the tensor data starts: the header is everything before it
    names = [good]
    rs = np.random.default_rng(4)
    head = raw.find(b"tokenizer.ggml.tokens") + 4096
    head = min(max(head, 1024), len(raw))
    for k, cut in enumerate(sorted(set([0, 3, 4, 8, 16, 24, 40, len(raw) - 1, len(raw) // 2] +
                                       [int(c) for c in rs.integers(0, head, 40)]))):
        p = str(tmp_path / f"cut{k}.gguf")
        open(p, "wb").write(raw[:cut])
        names.append(p)
    buf = bytearray(raw)
    for k in range(400):
        b = bytearray(buf)
        for _ in range(int(rs.integers(1, 4))):
            i = int(rs.integers(0, head))
            b[i] = int(rs.integers(0, 256)) if k % 3 else 0xFF
        p = str(tmp_path / f"mut{k}.gguf")
        open(p, "wb").write(bytes(b))
        names.append(p)
    r = subprocess.run([exe] + names, capture_output=True, encoding="utf-8", errors="replace", timeout=300,
                       env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0"))
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    lines = r.stdout.split()
    assert len(lines) == len(names), r.stdout[-2000:]
    assert lines[0] == "1"                                             # the valid file parses
    assert "bounds" not in r.stdout, r.stdout
    assert all(x in ("0", "1") for x in lines)
    cut_results = lines[1:1 + sum(1 for n in names if "cut" in n)]
    assert all(x == "0" for x in cut_results)                          # every truncation is refused
