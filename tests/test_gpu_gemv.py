"""GPU parity of the quantized weight x activation path against the CPU oracle
(itself pinned to the reference build, tests/test_oracle.py).

Bars (north star): integer work bit-exact -- activation quantizers, dequant,
repacking and every per-block int32 sum; fp32 outputs within
|gpu - cpu| <= 1e-5 + 1e-3*|cpu| of the oracle's shipped-order dot.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")
FMTS = [("q8_0", 8), ("q4_0", 2), ("q2_K", 10), ("q3_K", 11), ("q4_K", 12), ("q5_K", 13), ("q6_K", 14), ("tq2_0", 35)]
RTOL, ATOL = 1e-3, 1e-5


def gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_close(gpu, cpu, what=""):
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    err = np.abs(gpu - cpu)
    bad = err > ATOL + RTOL * np.abs(cpu)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside tolerance; worst {err.max():.3g}"


def dev_quantize(G, qt, x):
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    xb = G.Buffer.from_array(x)
    rs = G.row_size(qt, n)
    yb = G.Buffer(rs * rows)
    yb.zero()
    G.quantize(qt, xb, n, rows, yb)
    return yb.download(np.uint8, (rows, rs))


# ------------------------------------------------------------ conversions
def test_fp16_decode_exhaustive(gpu):
    G = gpu
    codes = np.arange(65536, dtype=np.uint16)
    xb = G.Buffer.from_array(codes)
    yb = G.Buffer(65536 * 4)
    G.dequant_rows(G.F16, xb, 65536, 1, yb)
    got = yb.download(np.float32, 65536)
    ref = gold("tables.npz")["fp16_to_fp32"].view(np.float32)
    fin = ~np.isnan(ref)
    assert np.array_equal(bits(got[fin]), bits(ref[fin]))          # incl. all 2046 subnormals
    assert np.isnan(got[~fin]).all()


@pytest.mark.parametrize("qname,qt", [("q8_0", 8), ("q8_K", 15), ("q4_0", 2)])
def test_quantizer_fixtures_bit_exact(gpu, qname, qt):
    g = gold(f"quant_{qname}.npz")
    assert np.array_equal(dev_quantize(gpu, qt, g["x"]), g["y"])


@pytest.mark.parametrize("qt", [8, 15, 2])
def test_quantizers_random_bit_exact(gpu, oracle, qt):
    rng = np.random.default_rng(11)
    for scale in (1.0, 3e-5, 1e-3, 250.0):
        x = (rng.standard_normal((32, 4096)) * scale).astype(np.float32)
        x[3, :256] = 0.0
        assert np.array_equal(dev_quantize(gpu, qt, x), oracle.quantize(qt, x)), f"scale {scale}"


def _q8_K_special_rows(cols, seed):
    """fp32 rows whose superblocks hold the q8_K quantizer's corner cases:
    equal magnitudes of both signs (first one wins), NaN elements, a superblock
    of NaNs, +-inf, subnormals, a lone non-zero, signed zeros."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((8, cols)).astype(np.float32)
    x[0, 10], x[0, 200] = -4.0, 4.0                                   # tie, first is negative
    x[0, 256 + 3], x[0, 256 + 2] = 5.0, -5.0                          # tie inside one lane
    x[1, rng.integers(0, cols, 9)] = np.nan
    x[2, :256] = np.nan
    x[3, 17], x[3, 300] = np.inf, -np.inf
    x[4] *= np.float32(1e-41)                                         # subnormal inputs
    x[5] = 0.0
    x[5, 123] = -0.75
    x[6] = -0.0
    return x


def test_q8_K_quantizer_special_values(gpu, oracle):
    x = _q8_K_special_rows(1024, 21)
    assert np.array_equal(dev_quantize(gpu, 15, x), oracle.quantize(15, x))


# ------------------------------------------------------- dequant / layout
@pytest.mark.parametrize("name,qt", FMTS)
def test_dequant_bit_exact(gpu, name, qt):
    G = gpu
    g = gold(f"dot_{name}.npz")
    w, n = g["w"], int(g["n"])
    wb = G.Buffer.from_array(w)
    yb = G.Buffer(w.shape[0] * n * 4)
    G.dequant_rows(qt, wb, n, w.shape[0], yb)
    assert np.array_equal(bits(yb.download(np.float32, (w.shape[0], n))), bits(g["deq"]))


@pytest.mark.parametrize("name,qt", FMTS)
def test_resident_layout_round_trip(gpu, name, qt):
    from g4run_amd import synth
    w = synth.weights(qt, 37, 1024 if qt in (8, 2) else 2048, seed=3)
    t = gpu.Tensor.from_rows(qt, w, 1024 if qt in (8, 2) else 2048)
    assert np.array_equal(t.to_rows(), w)


# ------------------------------------------------------------ block sums
def gpu_block_sums(G, qt, w, a, n):
    t = G.Tensor.from_rows(qt, w, n)
    st = G.act_stride(qt, n)
    a = np.ascontiguousarray(a, np.uint8).reshape(-1, a.shape[-1])
    ap = np.zeros((a.shape[0], st), np.uint8)
    ap[:, :a.shape[1]] = a
    ab = G.Buffer.from_array(ap)
    cnt = G.n_block_sums(t)
    ob = G.Buffer(t.nrows * cnt * 4)
    G.block_sums(t, ab, ob)
    return ob.download(np.int32, (t.nrows, cnt))


@pytest.mark.parametrize("name,qt", FMTS)
def test_block_sums_vs_reference_fixture(gpu, name, qt):
    g = gold(f"dot_{name}.npz")
    s = gpu_block_sums(gpu, qt, g["w"], g["a"][:1], int(g["n"]))
    assert np.array_equal(s.astype(np.int64), g["sums"])


CONFIG_SHAPES = {8: [(4096, 4096)], 2: [(10240, 2560), (2560, 10240)], 12: [(4096, 11008)], 11: [(4096, 11008)],
                 10: [(4096, 11008)], 13: [(4096, 11008)], 14: [(4096, 11008)], 35: [(4096, 11008)]}


@pytest.mark.parametrize("name,qt", FMTS)
def test_block_sums_full_config_bit_exact(gpu, oracle, name, qt):
    from g4run_amd import synth
    for rows, cols in CONFIG_SHAPES[qt]:
        w = synth.weights(qt, rows, cols, seed=synth.SEEDS["weights"])
        x = synth.activations(1, cols, seed=synth.SEEDS["x"])
        a = oracle.quantize(oracle.ACT[qt], x)
        s = gpu_block_sums(gpu, qt, w, a, cols)
        ref = oracle.block_sums(qt, w, a[0], cols)
        assert np.array_equal(s, ref), f"{name} {rows}x{cols}"


# ------------------------------------------------------------------ GEMV
def oracle_matmul(oracle, qt, w, x):
    act = oracle.prep_act(qt, x)
    oracle.pool_start(8)
    try:
        return oracle.matmul(qt, w, act, x.shape[1], nthreads=8)
    finally:
        oracle.pool_stop()


def gpu_matmul(G, t, x=None, act=None, nb=1, path=0):
    Yb = G.Buffer(nb * t.nrows * 4)
    if x is not None:
        xb = G.Buffer.from_array(np.ascontiguousarray(x, np.float32))
        G.matmul(t, Yb, nb=nb, x=xb, path=path)
    else:
        ab = G.Buffer.from_array(act)
        G.matmul(t, Yb, nb=nb, pre=ab, pre_stride=act.shape[1], path=path)
    return Yb.download(np.float32, (nb, t.nrows))


@pytest.mark.parametrize("name,qt", FMTS)
def test_gemv_full_config_vs_oracle(gpu, oracle, name, qt):
    from g4run_amd import synth
    for rows, cols in CONFIG_SHAPES[qt]:
        w = synth.weights(qt, rows, cols, seed=synth.SEEDS["weights"])
        x = synth.activations(1, cols, seed=synth.SEEDS["x"])
        t = gpu.Tensor.from_rows(qt, w, cols)
        y = gpu_matmul(gpu, t, x=x)
        assert_close(y, oracle_matmul(oracle, qt, w, x), f"{name} {rows}x{cols}")


@pytest.mark.parametrize("name,qt", FMTS)
def test_gemv_vs_reference_fixture(gpu, name, qt):
    g = gold(f"dot_{name}.npz")
    n = int(g["n"])
    t = gpu.Tensor.from_rows(qt, g["w"], n)
    y = gpu_matmul(gpu, t, x=g["x"], nb=g["x"].shape[0])
    assert_close(y, g["dot"], name)


@pytest.mark.parametrize("name,qt", FMTS)
def test_batch_bit_identical_to_single_token(gpu, oracle, name, qt):
    """g4run.h:148-157: token b of a batch equals the 1-token result bit for bit."""
    from g4run_amd import synth
    cols = 2560 if qt in (8, 2) else 2816
    w = synth.weights(qt, 300, cols, seed=21)
    x = synth.activations(8, cols, seed=22)
    act = oracle.prep_act(qt, x)
    t = gpu.Tensor.from_rows(qt, w, cols)
    singles = np.stack([gpu_matmul(gpu, t, act=act[i:i + 1])[0] for i in range(8)])
    for nb in (2, 3, 4, 5, 8):
        y = gpu_matmul(gpu, t, act=act[:nb].copy(), nb=nb)
        assert np.array_equal(bits(y), bits(singles[:nb])), f"nb={nb}"
    assert_close(singles, oracle.matmul(qt, w, act, cols), name)


@pytest.mark.parametrize("qt,rows,cols", [(2, 2560, 10240), (8, 2560, 10240), (2, 700, 14336), (8, 300, 12800)])
def test_eight_tokens_with_large_staging(gpu, oracle, qt, rows, cols):
    """Eight tokens whose q8_0 activations take more than 64 KB of LDS (rows
    of 10240 and more) run as one launch of up to 16 waves per workgroup, one
    workgroup per CU; token b still has the 1-token bits (g4run.h:148-157),
    and 9 tokens (8 + 1) as well."""
    from g4run_amd import synth
    w = synth.weights(qt, rows, cols, seed=rows + 5)
    x = synth.activations(9, cols, seed=cols + 6)
    act = oracle.prep_act(qt, x)
    t = gpu.Tensor.from_rows(qt, w, cols)
    d = gpu.matmul_describe(t, 8, 1)
    assert "nb=8" in d and "(x1 launches)" in d, d
    if (rows, cols) == (2560, 10240):
        assert "grid=256 block=640" in d, d                          # 10 waves, one round
    singles = np.stack([gpu_matmul(gpu, t, act=act[i:i + 1])[0] for i in range(9)])
    for nb in (8, 9):
        y = gpu_matmul(gpu, t, act=act[:nb].copy(), nb=nb, path=1)
        assert np.array_equal(bits(y), bits(singles[:nb])), f"nb={nb}"
    assert_close(singles[:2], oracle.matmul(qt, w, act[:2], cols), f"{qt} {rows}x{cols}")


@pytest.mark.parametrize("name,qt", FMTS)
def test_fused_quantizer_equals_prequantized(gpu, oracle, name, qt):
    from g4run_amd import synth
    cols = 4096
    w = synth.weights(qt, 128, cols, seed=31)
    x = synth.activations(3, cols, seed=32)
    t = gpu.Tensor.from_rows(qt, w, cols)
    a = gpu_matmul(gpu, t, x=x, nb=3)
    b = gpu_matmul(gpu, t, act=oracle.prep_act(qt, x), nb=3)
    assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("qt,rows,cols,nb", [
    (2, 10240, 2560, 1), (2, 2560, 10240, 1), (8, 4096, 4096, 1), (2, 2048, 11008, 1), (8, 1000, 6400, 1),
    (8, 4096, 2048, 2), (2, 4096, 256, 8),
    (12, 4096, 11008, 1), (11, 4096, 11008, 1), (10, 4096, 11008, 1), (13, 1000, 2560, 1), (14, 333, 11008, 1),
    (35, 4096, 4096, 1), (12, 64, 256, 1),
])
def test_in_kernel_quantizer_equals_prequantized(gpu, oracle, qt, rows, cols, nb):
    """The shapes whose fp32 input is quantized inside the GEMV (two groups of
    four inputs per thread, or four for one token in larger workgroups; q8_0
    for q8_0 / q4_0 weights, q8_K with a superblock per 16 or 32 threads for
    K-quants: both lane widths are among these shapes)
    give the bits of the GEMV on the separately quantized input."""
    from g4run_amd import synth
    w = synth.weights(qt, rows, cols, seed=rows + cols)
    x = synth.activations(nb, cols, seed=nb)
    t = gpu.Tensor.from_rows(qt, w, cols)
    assert "quantized in-kernel" in gpu.matmul_describe(t, nb, 1)
    a = gpu_matmul(gpu, t, x=x, nb=nb)
    b = gpu_matmul(gpu, t, act=oracle.prep_act(qt, x), nb=nb)
    assert np.array_equal(bits(a), bits(b))
    if nb == 1:
        assert_close(a, oracle_matmul(oracle, qt, w, x), f"{qt} {rows}x{cols}")


@pytest.mark.parametrize("qt", [12, 14])
def test_in_kernel_q8_K_special_values(gpu, oracle, qt):
    """Ties, NaN elements, a NaN superblock, subnormals and zeros quantized
    inside the GEMV give the bits of the GEMV on the standalone quantizer's
    output, row by row."""
    from g4run_amd import synth
    cols = 11008 if qt == 12 else 2560
    x = _q8_K_special_rows(cols, 5)
    w = synth.weights(qt, 4096, cols, seed=qt)
    t = gpu.Tensor.from_rows(qt, w, cols)
    assert "quantized in-kernel" in gpu.matmul_describe(t, 1, 1)
    for r in range(x.shape[0]):
        if r == 3:
            continue                                                  # inf scales: NaN outputs
        a = gpu_matmul(gpu, t, x=x[r:r + 1].copy(), nb=1)
        b = gpu_matmul(gpu, t, act=dev_quantize(gpu, 15, x[r:r + 1]), nb=1)
        assert np.array_equal(bits(a), bits(b)), f"row {r}"


@pytest.mark.parametrize("name,qt", FMTS)
def test_ragged_shapes(gpu, oracle, name, qt):
    """Row counts that do not fill a workgroup, odd block counts, one row."""
    from g4run_amd import synth
    for rows, cols in ((1, 256), (3, 768), (67, 1280), (129, 6400), (5, 800), (2, 96), (33, 2080)):
        if cols % oracle.BLCK[qt]:
            continue
        w = synth.weights(qt, rows, cols, seed=rows)
        x = synth.activations(2, cols, seed=cols)
        t = gpu.Tensor.from_rows(qt, w, cols)
        assert_close(gpu_matmul(gpu, t, x=x, nb=2), oracle_matmul(oracle, qt, w, x), f"{name} {rows}x{cols}")


@pytest.mark.parametrize("name,qt", FMTS)
def test_vec_dot_raw_rows(gpu, oracle, name, qt):
    G = gpu
    g = gold(f"dot_{name}.npz")
    w, a, n = g["w"], g["a"], int(g["n"])
    wb, ab = G.Buffer.from_array(w), G.Buffer.from_array(a[0].copy())
    ob = G.Buffer(w.shape[0] * 4)
    G.vec_dot(qt, wb, ab, n, w.shape[0], ob)
    assert_close(ob.download(np.float32, w.shape[0]), g["dot"][0], name)


# ---------------------------------------------------------- error paths
def test_error_paths(gpu):
    import ctypes as C
    G = gpu
    L = G.lib()
    p = C.c_void_p()
    assert L.g4h_tensor_create(G.Q4_K, 1000, 4, C.byref(p)) == G.ERR_SHAPE
    assert L.g4h_tensor_create(G.F32, 256, 4, C.byref(p)) == G.ERR_TYPE
    G.lib().g4h_debug_fail_alloc(1)
    assert L.g4h_tensor_create(G.Q8_0, 256, 4, C.byref(p)) == G.ERR_NOMEM
    assert L.g4h_tensor_create(G.Q8_0, 256, 4, C.byref(p)) == G.OK
    t = p.value
    yb = G.Buffer(16)
    # both or neither activation source
    assert L.g4h_matmul(t, None, None, 0, yb.ptr, 1, None) == G.ERR_ARG
    assert L.g4h_quantize_q8_0(yb.ptr, 33, yb.ptr, 34, 33, 1, None) == G.ERR_SHAPE
    assert L.g4h_tensor_free(t) == G.OK
