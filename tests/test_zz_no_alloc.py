"""g4h_matmul_noalloc: g4h_matmul_ex with the per-device fixed scratch array
instead of the per-stream pool (no device allocation).  Called through the C
ABI and compared bit for bit with g4h_matmul_ex on the same inputs, on two
calls in a row, the second with fewer tokens (the array keeps the first call's
contents, which must not leak into the second)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _mm(G, fn, W, x, pre, stride, Y, nb, path):
    rc = fn(W.ptr, x.ptr if x is not None else None, pre.ptr if pre is not None else None, stride, Y.ptr, nb, path, None)
    G.check(rc)
    G.synchronize()


@pytest.mark.parametrize("qt,rows,cols,nbs,path,use_pre", [
    (12, 1024, 2816, (8, 3), 0, False),       # q4_K: x quantized to q8_K in the scratch, GEMV family
    (8, 512, 4096, (64, 40), 2, False),       # q8_0 matrix cores: planar activation copy in the scratch
    (8, 512, 4096, (64, 33), 2, True),        # the same from pre-quantized rows
    (2, 1024, 2560, (4, 1), 1, False),        # q4_0 GEMV, x quantized in-kernel
    (1, 512, 1024, (8, 2), 0, False),         # f16 rows: x converted to f16 in the scratch
], ids=["q4_K-gemv", "q8_0-mfma", "q8_0-mfma-pre", "q4_0-gemv", "f16"])
def test_noalloc_equals_matmul(gpu, qt, rows, cols, nbs, path, use_pre):
    G = gpu
    from g4run_amd import synth
    L = G.lib()
    w = synth.weights(qt, rows, cols, seed=3)
    W = G.Tensor.from_rows(qt, w, cols)
    for call, nb in enumerate(nbs):
        x = G.Buffer.from_array(synth.activations(nb, cols, seed=10 + call))
        pre, stride = None, 0
        if use_pre:
            stride = G.act_stride(qt, cols)
            pre = G.Buffer(stride * nb)
            G.quantize(G.act_type(qt), x, cols, nb, pre, y_stride=stride)
            x = None
        Y0, Y1 = G.Buffer(nb * rows * 4), G.Buffer(nb * rows * 4)
        _mm(G, L.g4h_matmul_ex, W, x, pre, stride, Y0, nb, path)
        _mm(G, L.g4h_matmul_noalloc, W, x, pre, stride, Y1, nb, path)
        y0 = Y0.download(np.uint32, (nb, rows))
        y1 = Y1.download(np.uint32, (nb, rows))
        assert np.array_equal(y0, y1), f"call {call} (nb={nb}): {int((y0 != y1).sum())} outputs differ"
    W.free()


def test_noalloc_rejects_oversized_calls(gpu):
    G = gpu
    from g4run_amd import synth
    L = G.lib()
    cap = L.g4h_matmul_noalloc_max_bytes()
    assert cap == 4 << 20
    cols, rows = 11008, 256
    nb = cap // G.act_stride(G.Q4_K, cols) + 1                 # its q8_K activations exceed the array
    W = G.Tensor.from_rows(G.Q4_K, synth.weights(G.Q4_K, rows, cols, seed=4), cols)
    x = G.Buffer.from_array(synth.activations(nb, cols, seed=5))
    Y = G.Buffer(nb * rows * 4)
    rc = L.g4h_matmul_noalloc(W.ptr, x.ptr, None, 0, Y.ptr, nb, 1, None)
    assert rc == G.ERR_ARG
    assert b"scratch" in L.g4h_last_error()
    W.free()
