"""The C ABI library loads, exports every entry point include/g4hip.h declares,
and its host-side logic (sizes, classes, argument checks, failure paths)
behaves like the reference interfaces it replaces -- all without a GPU."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "g4hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g4h_[A-Za-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import g4run_amd as G
    L = G.lib()
    names = declared_symbols()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the Python front end binds exactly that set
    assert sorted(G.exported_names()) == names


def test_row_size_matches_type_table():
    # gguf.c:11-46: (n/blck)*size, 0 when the block size does not divide n
    import g4run_amd as G
    assert G.row_size(G.Q8_0, 4096) == 4352
    assert G.row_size(G.Q4_0, 2560) == 1440
    assert G.row_size(G.Q4_0, 10240) == 5760
    assert G.row_size(G.Q4_K, 11008) == 6192
    assert G.row_size(G.Q3_K, 11008) == 4730
    assert G.row_size(G.Q2_K, 11008) == 3612
    assert G.row_size(G.Q5_K, 11008) == 43 * 176
    assert G.row_size(G.Q6_K, 11008) == 43 * 210
    assert G.row_size(G.TQ2_0, 11008) == 43 * 66
    assert G.row_size(G.Q8_K, 11008) == 43 * 292
    assert G.row_size(G.Q8_0, 33) == 0
    assert G.row_size(G.Q4_K, 1000) == 0
    assert G.row_size(99, 256) == 0


def test_act_class_and_stride():
    # model.c:132-141 activation classes; model.c:148-149 64-B padded stride
    import g4run_amd as G
    assert G.act_type(G.Q4_0) == G.Q8_0 and G.act_type(G.Q8_0) == G.Q8_0
    for t in (G.Q2_K, G.Q3_K, G.Q4_K, G.Q5_K, G.Q6_K):
        assert G.act_type(t) == G.Q8_K
    assert G.act_type(G.F32) == -1
    assert G.act_stride(G.Q8_0, 4096) == 4352
    assert G.act_stride(G.Q4_0, 2560) == 2752          # 2720 -> 64-B multiple
    assert G.act_stride(G.Q4_K, 11008) == (43 * 292 + 63) // 64 * 64


def test_calls_before_init_fail_with_status_not_exit():
    # the reference exits on bad input (quants.c:529); the ABI returns codes
    import g4run_amd as G
    L = G.lib()
    p = C.c_void_p()
    if not G._inited:
        assert L.g4h_tensor_create(G.Q8_0, 64, 4, C.byref(p)) == G.ERR_DEVICE
        assert b"g4h_init" in L.g4h_last_error()
        assert L.g4h_malloc(C.byref(p), 16) == G.ERR_DEVICE
    assert L.g4h_status_str(G.ERR_SHAPE) == b"invalid shape"


def test_init_without_gfx950_reports_device_error():
    import g4run_amd as G
    L = G.lib()
    rc = L.g4h_init(0)
    if rc == G.OK:
        pytest.skip("a gfx950 device is present")
    assert rc == G.ERR_DEVICE
    assert L.g4h_init(-1) == G.ERR_DEVICE
