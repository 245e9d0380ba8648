"""GPU parity of the f16 / bf16 weight GEMV (matmul_b's G4_F16 / G4_BF16 rows,
model.c:238-239, over g4_dot_f16 / g4_dot_bf16, quants.c:1319-1347) against the
CPU oracle, whose dots reproduce the reference build's bit for bit
(tests/test_oracle.py).

Float weights have no integer block sums: fp32 results must be within
|gpu - cpu| <= 1e-5 + 1e-3*|cpu| (the GPU sums lanes in another order than the
8-lane AVX2 loop).  The activation conversions of prep_act (model.c:163-180),
dequant, the resident layout round trip and batch invariance are bit-exact.
"""
import os

import numpy as np
import pytest

from test_gpu_gemv import assert_close, bits, gpu_matmul, oracle_matmul

pytestmark = pytest.mark.gpu

FLOAT = [("f16", 1), ("bf16", 30)]
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _weights(wt, rows, cols, seed):
    """N(0, 0.02) weights as f16 (round to nearest) or bf16 (truncated) rows."""
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w = wf.astype(np.float16).view(np.uint16) if wt == 1 else (wf.view(np.uint32) >> 16).astype(np.uint16)
    return np.ascontiguousarray(w).view(np.uint8).reshape(rows, 2 * cols)


@pytest.mark.parametrize("name,wt", FLOAT)
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (2560, 10240), (37, 264)])
def test_gemv_vs_oracle_and_batch_invariance(gpu, oracle, name, wt, rows, cols):
    from g4run_amd import synth
    w = _weights(wt, rows, cols, seed=rows + wt)
    x = synth.activations(5, cols, seed=cols)
    t = gpu.Tensor.from_rows(wt, w, cols)
    try:
        y = gpu_matmul(gpu, t, x=x, nb=5)                         # chunks of 4 + 1 tokens
        assert_close(y, oracle_matmul(oracle, wt, w, x), f"{name} {rows}x{cols}")
        for b in range(5):
            y1 = gpu_matmul(gpu, t, x=x[b:b + 1].copy(), nb=1)
            assert np.array_equal(bits(y1[0]), bits(y[b])), f"token {b}"
    finally:
        t.free()


@pytest.mark.parametrize("name,wt", FLOAT)
def test_in_call_conversion_equals_prep_act_and_round_trip(gpu, oracle, name, wt):
    from g4run_amd import synth
    w = _weights(wt, 64, 1024, seed=3)
    x = synth.activations(3, 1024, seed=4)
    x[0, :8] = [0.0, -0.0, 1e-30, -3e-8, 65504.0, 70000.0, 1.00048828125, -2.5e-5]   # zero, subnormal, overflow, ties
    t = gpu.Tensor.from_rows(wt, w, 1024)
    try:
        a = gpu_matmul(gpu, t, x=x, nb=3)
        b = gpu_matmul(gpu, t, act=oracle.prep_act(wt, x), nb=3)
        assert np.array_equal(bits(a), bits(b))
        for nb in (1, 2):                                   # converted inside the GEMV (one launch)
            a = gpu_matmul(gpu, t, x=x[:nb].copy(), nb=nb)
            assert np.array_equal(bits(a), bits(b[:nb])), f"nb={nb}"
        assert np.array_equal(t.to_rows(), w)
    finally:
        t.free()


@pytest.mark.parametrize("name,wt", FLOAT)
def test_dequant_bit_exact_vs_reference_fixture(gpu, name, wt):
    g = np.load(os.path.join(GOLD, f"dot_{name}.npz"), allow_pickle=False)
    w, n = g["w"], int(g["n"])
    rows = w.shape[0]
    wb = gpu.Buffer.from_array(np.ascontiguousarray(w))
    yb = gpu.Buffer(rows * n * 4)
    gpu.dequant_rows(wt, wb, n, rows, yb)
    assert np.array_equal(bits(yb.download(np.float32, (rows, n))), bits(g["deq"]))


@pytest.mark.parametrize("name,wt", FLOAT)
def test_vec_dot_raw_rows_equal_matmul(gpu, oracle, name, wt):
    from g4run_amd import synth
    w = _weights(wt, 24, 2048, seed=7)
    x = synth.activations(1, 2048, seed=8)
    act = oracle.prep_act(wt, x)
    t = gpu.Tensor.from_rows(wt, w, 2048)
    try:
        y = gpu_matmul(gpu, t, act=act, nb=1)
    finally:
        t.free()
    wb, ab, ob = gpu.Buffer.from_array(w), gpu.Buffer.from_array(act), gpu.Buffer(24 * 4)
    gpu.vec_dot(wt, wb, ab, 2048, 24, ob)
    assert np.array_equal(bits(ob.download(np.float32, (24,))), bits(y[0]))


def test_float_weight_errors(gpu):
    G = gpu
    with pytest.raises(G.G4HError) as e:
        G.Tensor(1, 12, 4)                                          # rows must be a multiple of 8 values
    assert e.value.status == G.ERR_SHAPE
    t = G.Tensor.from_rows(30, _weights(30, 8, 72, seed=1), 72)     # 72 columns: not whole 16-column steps
    t64 = G.Tensor.from_rows(30, _weights(30, 8, 64, seed=1), 64)
    try:
        Y = G.Buffer(8 * 4 * 4)
        x = G.Buffer.from_array(np.ones((4, 72), np.float32))
        with pytest.raises(G.G4HError) as e:
            G.matmul(t, Y, nb=4, x=x, path=2)
        assert e.value.status == G.ERR_TYPE
        with pytest.raises(G.G4HError) as e:
            G.block_sums(t, x, G.Buffer(64))
        assert e.value.status == G.ERR_TYPE
        assert G.matmul_path(t, 512) == 1
        assert [G.matmul_path(t64, n) for n in (1, 8, 9, 512)] == [1, 1, 2, 2]
    finally:
        t.free()
        t64.free()


@pytest.mark.parametrize("name,wt", FLOAT)
@pytest.mark.parametrize("rows,cols,M", [(256, 2048, 64), (2048, 256, 64), (4096, 4096, 40), (100, 80, 33), (33, 1040, 9),
                                         (1, 16, 1)])
def test_matrix_cores_vs_oracle(gpu, oracle, name, wt, rows, cols, M):
    """Prompt batches on the matrix cores (path 2, k_mm_float): 32 x 32 tiles
    of exact f16 x f16 / bf16 x bf16 products summed in fp32, 8 waves splitting
    the 16-column steps and added in wave order; within the fp32 tolerance of
    the oracle's dots.  The fp32 x rounded on load gives the bits of prep_act's
    prepared rows.  Ragged rows and tokens, 5 steps (three waves idle), one
    step, and step counts that take each chunk size."""
    from g4run_amd import synth
    w = _weights(wt, rows, cols, seed=rows * 3 + cols + wt)
    x = synth.activations(M, cols, seed=cols + M)
    t = gpu.Tensor.from_rows(wt, w, cols)
    try:
        assert gpu.matmul_describe(t, M, 2).startswith("k_mm_float")
        y = gpu_matmul(gpu, t, x=x, nb=M, path=2)
        assert_close(y, oracle_matmul(oracle, wt, w, x), f"{name} {rows}x{cols} M={M}")
        b = gpu_matmul(gpu, t, act=oracle.prep_act(wt, x), nb=M, path=2)
        assert np.array_equal(bits(y), bits(b)), f"{name} {rows}x{cols} M={M}: x rounded on load != prepared rows"
    finally:
        t.free()


@pytest.mark.parametrize("name,wt", FLOAT)
def test_matrix_cores_token_results_independent_of_batch(gpu, oracle, name, wt):
    """A token's row from k_mm_float has the same bits in any batch (its
    tile's sums do not depend on the other tokens), and auto path selection
    takes the matrix cores from 9 tokens."""
    from g4run_amd import synth
    w = _weights(wt, 96, 1056, seed=5)
    x = synth.activations(70, 1056, seed=6)
    t = gpu.Tensor.from_rows(wt, w, 1056)
    try:
        full = gpu_matmul(gpu, t, x=x, nb=70, path=2)
        assert_close(full, oracle_matmul(oracle, wt, w, x), f"{name} M=70")
        for m in (1, 9, 31, 32, 33, 64):
            part = gpu_matmul(gpu, t, x=x[:m].copy(), nb=m, path=2)
            assert np.array_equal(bits(part), bits(full[:m])), f"{name} M={m}"
        auto = gpu_matmul(gpu, t, x=x[:9].copy(), nb=9)
        assert np.array_equal(bits(auto), bits(full[:9]))
    finally:
        t.free()
