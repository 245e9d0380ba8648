"""The g4run.h-compatible C entry points (include/g4run_abi.h) from a real C
caller: tests/c/abi_driver.c and the INTEGRATION.md backend tests/c/g4gpu.c,
compiled with gcc and linked with -lg4hip (and the oracle, as the checker).
CPU: the program compiles and links, and the library exports every symbol the
header declares.  GPU: the program runs every check against the oracle."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "g4run_amd")
ORADIR = os.path.join(ROOT, "oracle")


def declared_g4_symbols():
    text = open(os.path.join(ROOT, "include", "g4run_abi.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    funcs = set(re.findall(r"\b(g4_[A-Za-z0-9_]+)\s*\(", text))
    data = set(re.findall(r"extern\s+[A-Za-z0-9_]+\s+(g4_[A-Za-z0-9_]+)", text))
    return sorted(funcs | data)


def build_driver(tmp_path):
    from oracle import g4o
    g4o.lib()                                    # builds oracle/liboracle.so if missing
    exe = str(tmp_path / "abi_driver")
    cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Werror",
           "-I" + os.path.join(ROOT, "include"), "-I" + ORADIR, "-I" + os.path.join(ROOT, "tests", "c"),
           os.path.join(ROOT, "tests", "c", "abi_driver.c"), os.path.join(ROOT, "tests", "c", "g4gpu.c"),
           "-L" + LIBDIR, "-lg4hip", "-L" + ORADIR, "-l:liboracle.so",
           "-Wl,-rpath," + LIBDIR + ":" + ORADIR, "-lm", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_library_exports_every_g4run_symbol():
    import ctypes as C
    import g4run_amd as G
    L = G.lib()
    names = declared_g4_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the type table needs no device
    L.g4_row_size.restype = C.c_size_t
    L.g4_row_size.argtypes = [C.c_int, C.c_int64]
    assert L.g4_row_size(2, 2560) == 1440 and L.g4_row_size(12, 11008) == 6192 and L.g4_row_size(2, 33) == 0


def test_c_caller_compiles_and_links(tmp_path):
    exe = build_driver(tmp_path)
    assert os.path.exists(exe)


@pytest.mark.gpu
def test_c_caller_against_oracle(tmp_path):
    exe = build_driver(tmp_path)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0 and "PASS" in r.stdout, r.stdout + r.stderr
