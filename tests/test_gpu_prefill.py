"""GPU parity of the batched-prefill matmul on the int8 matrix cores (path 2)
against the CPU oracle's shipped-order dots (q8_0 4096x4096 x M tokens, q4_0
FFN shapes, q4_K / q6_K 4096x11008), plus its batch-size invariance and error
paths.

The per-block integer sums come out of one int8 MFMA per block and are exact
by construction; the fp32 results must be within |gpu - cpu| <= 1e-5 +
1e-3*|cpu| of the oracle (the fp32 order differs from the CPU's 8-lane one).
"""
import numpy as np
import pytest

from test_gpu_gemv import assert_close, bits, gpu_matmul, oracle_matmul

pytestmark = pytest.mark.gpu


def _setup(G, qt, rows, cols, M, seed):
    from g4run_amd import synth
    w = synth.weights(qt, rows, cols, seed=seed)
    x = synth.activations(M, cols, seed=seed + 1)
    return w, x, G.Tensor.from_rows(qt, w, cols)


@pytest.mark.parametrize("M", [1, 8, 16, 64, 512])
def test_config3_q8_0_vs_oracle(gpu, oracle, M):
    w, x, t = _setup(gpu, 8, 4096, 4096, M, seed=1234)
    y = gpu_matmul(gpu, t, x=x, nb=M, path=2)
    assert_close(y, oracle_matmul(oracle, 8, w, x), f"q8_0 4096x4096 M={M}")


@pytest.mark.parametrize("rows,cols,M", [(10240, 2560, 128), (2560, 10240, 64)])
def test_q4_0_ffn_shapes_vs_oracle(gpu, oracle, rows, cols, M):
    w, x, t = _setup(gpu, 2, rows, cols, M, seed=rows)
    assert_close(gpu_matmul(gpu, t, x=x, nb=M, path=2), oracle_matmul(oracle, 2, w, x), f"q4_0 {rows}x{cols} M={M}")


@pytest.mark.parametrize("qt", [8, 2])
def test_ragged_shapes(gpu, oracle, qt):
    """Token and row counts that do not fill a tile, odd block counts."""
    for rows, cols, M in ((1, 32, 16), (31, 96, 17), (100, 2080, 33), (65, 800, 65), (257, 1024, 100), (33, 4096, 129)):
        w, x, t = _setup(gpu, qt, rows, cols, M, seed=rows + cols)
        assert_close(gpu_matmul(gpu, t, x=x, nb=M, path=2), oracle_matmul(oracle, qt, w, x), f"{rows}x{cols} M={M}")


@pytest.mark.parametrize("qt", [8, 2])
@pytest.mark.parametrize("rows,cols,M", [(384, 2048, 512), (4096, 512, 256)])
def test_token_results_independent_of_batch(gpu, oracle, qt, rows, cols, M):
    """Within the matrix-core family a token's outputs are bit-identical for any
    batch size (small-M and large-M tile variants keep the same fp32 order).
    4096 rows from 65 tokens run the LDS-staged tiles, 384 rows the one-tile
    kernel, up to 64 tokens the few-token kernel."""
    w, x, t = _setup(gpu, qt, rows, cols, M, seed=5)
    full = gpu_matmul(gpu, t, x=x, nb=M, path=2)
    if rows == 4096:
        assert gpu.matmul_describe(t, M, 2).startswith("k_mm_lds")
        assert gpu.matmul_describe(t, 16, 2).startswith("k_mm_few")
        assert_close(full, oracle_matmul(oracle, qt, w, x), f"{rows}x{cols} M={M}")
    for m in (16, 40, 64, 65, 200):
        part = gpu_matmul(gpu, t, x=x[:m].copy(), nb=m, path=2)
        assert np.array_equal(bits(part), bits(full[:m])), f"M={m}"


@pytest.mark.parametrize("qt", [8, 2])
@pytest.mark.parametrize("rows,cols,M", [(4096, 4096, 128), (2560, 2048, 96), (640, 1024, 300)])
def test_one_tile_kernel_equals_staged_tiles(gpu, oracle, monkeypatch, qt, rows, cols, M):
    """The one-tile kernel and the LDS-staged tiles give the same bits on the
    same call: the selection between them (by tile count, G4H_MM_SMALL_TILES
    overriding it) moves no output."""
    w, x, t = _setup(gpu, qt, rows, cols, M, seed=rows + M)
    out = {}
    for most, name in (("1000000", "k_mm_mfma"), ("0", "k_mm_lds")):
        monkeypatch.setenv("G4H_MM_SMALL_TILES", most)
        assert gpu.matmul_describe(t, M, 2).startswith(name)
        out[name] = gpu_matmul(gpu, t, x=x, nb=M, path=2)
    monkeypatch.delenv("G4H_MM_SMALL_TILES")
    assert np.array_equal(bits(out["k_mm_mfma"]), bits(out["k_mm_lds"]))
    assert_close(out["k_mm_lds"], oracle_matmul(oracle, qt, w, x), f"{rows}x{cols} M={M}")


@pytest.mark.parametrize("qt", [8, 2])
def test_fused_quantizer_equals_prequantized(gpu, oracle, qt):
    w, x, t = _setup(gpu, qt, 256, 4096, 48, seed=9)
    a = gpu_matmul(gpu, t, x=x, nb=48, path=2)
    b = gpu_matmul(gpu, t, act=oracle.prep_act(qt, x), nb=48, path=2)
    assert np.array_equal(bits(a), bits(b))


def test_matrix_core_path_agrees_with_gemv_path(gpu, oracle):
    w, x, t = _setup(gpu, 8, 512, 4096, 32, seed=3)
    ref = oracle_matmul(oracle, 8, w, x)
    assert_close(gpu_matmul(gpu, t, x=x, nb=32, path=1), ref, "gemv")
    assert_close(gpu_matmul(gpu, t, x=x, nb=32, path=2), ref, "mfma")


def test_path_selection_and_errors(gpu):
    from g4run_amd import synth
    G = gpu
    t8 = G.Tensor.from_rows(8, synth.weights(8, 64, 256, seed=1), 256)
    assert [G.matmul_path(t8, n) for n in (1, 8, 9, 16, 512)] == [1, 1, 2, 2, 2]
    for qt in (12, 14):
        t = G.Tensor.from_rows(qt, synth.weights(qt, 64, 256, seed=1), 256)
        assert [G.matmul_path(t, n) for n in (1, 8, 9, 512)] == [1, 1, 2, 2]
        assert G.matmul_describe(t, 64, 2).startswith("k_mmk")
    tk = G.Tensor.from_rows(13, synth.weights(13, 64, 256, seed=1), 256)
    assert G.matmul_path(tk, 512) == 1
    Y = G.Buffer(64 * 16 * 4)
    x = G.Buffer.from_array(synth.activations(16, 256, seed=2))
    with pytest.raises(G.G4HError) as e:
        G.matmul(tk, Y, nb=16, x=x, path=2)
    assert e.value.status == G.ERR_TYPE


@pytest.mark.parametrize("qt", [8, 2])
@pytest.mark.parametrize("rows,cols,Ms", [(4096, 4096, (1, 8, 16, 32, 48, 64)), (100, 2080, (1, 5, 17, 33, 64)),
                                          (33, 1056, (2, 31, 32, 49)), (17, 10240, (3, 16, 19, 63)), (8200, 512, (1, 16, 64)),
                                          (48, 64, (1, 64)), (16, 32, (7,)), (40, 1408, (5, 64))])
def test_few_kernel_equals_tile_kernel(gpu, oracle, monkeypatch, qt, rows, cols, Ms):
    """The few-token kernel (up to 64 tokens; each weight byte read once,
    operands of a block pair swapped across lane halves) gives the tile
    kernel's bits (G4H_MM_FEW=0): the same exact block sums, exact scale
    products and residue-pair partial sums.  Ragged rows, token counts off the
    16-token tile, odd block counts (a lone last block) and block counts off
    the 8-block stage, one and two blocks per row, several workgroups per CU
    (8200 rows).  A wave's pair steps run as 16-step chunks and then one chunk
    each of 8, 4, 2 and 1 for the rest: 10240 columns take 16 + 16 + 8, 2080
    columns 8 + 1 (and 8), 1408 columns 4 + 2 (and 4 + 1), 64 columns one step
    in one wave and none in the other three."""
    w, x, t = _setup(gpu, qt, rows, cols, max(Ms), seed=rows * 7 + cols)
    for M in Ms:
        assert gpu.matmul_describe(t, M, 2).startswith("k_mm_few")
        few = gpu_matmul(gpu, t, x=x[:M].copy(), nb=M, path=2)
        monkeypatch.setenv("G4H_MM_FEW", "0")
        tile = gpu_matmul(gpu, t, x=x[:M].copy(), nb=M, path=2)
        monkeypatch.delenv("G4H_MM_FEW")
        assert np.array_equal(bits(few), bits(tile)), f"{rows}x{cols} M={M}"
        assert_close(few, oracle_matmul(oracle, qt, w, x[:M]), f"{rows}x{cols} M={M}")


@pytest.mark.parametrize("qt", [8, 2])
def test_few_kernel_prequantized_rows(gpu, oracle, qt):
    """GGUF q8_0 activation rows (the act path) re-laid for the few-token
    kernel give the bits of the fused quantizer's layout."""
    w, x, t = _setup(gpu, qt, 200, 2080, 37, seed=11)
    a = gpu_matmul(gpu, t, x=x, nb=37, path=2)
    b = gpu_matmul(gpu, t, act=oracle.prep_act(qt, x), nb=37, path=2)
    assert gpu.matmul_describe(t, 37, 2).startswith("k_mm_few")
    assert np.array_equal(bits(a), bits(b))


# ------------------------------------------------- K-quant weights (k_mmk)
KQ = [("q4_K", 12), ("q6_K", 14)]


@pytest.mark.parametrize("name,qt", KQ)
@pytest.mark.parametrize("M", [64, 512])
def test_kquant_config_vs_oracle(gpu, oracle, name, qt, M):
    w, x, t = _setup(gpu, qt, 4096, 11008, M, seed=77 + qt)
    assert gpu.matmul_describe(t, M, 2).startswith("k_mmk")
    assert gpu.matmul_path(t, M) == 2
    assert_close(gpu_matmul(gpu, t, x=x, nb=M), oracle_matmul(oracle, qt, w, x), f"{name} 4096x11008 M={M}")


def _unit_scales(qt, w, cols, which):
    """Copies of GGUF rows with every superblock's fp16 scales set so that the
    row's output is an integer: q4_K d = 1, dmin = 0 ('isum') or d = 0,
    dmin = 1 ('msum'); q6_K d = 1."""
    w = np.array(w, dtype=np.uint8).reshape(w.shape[0], cols // 256, -1)
    one, zero = np.uint16(0x3C00), np.uint16(0)
    if qt == 12:
        hdr = w[:, :, 0:4].copy().view(np.uint16)
        hdr[..., 0] = one if which == "isum" else zero
        hdr[..., 1] = zero if which == "isum" else one
        w[:, :, 0:4] = hdr.view(np.uint8)
    else:
        w[:, :, 208:210] = np.frombuffer(one.tobytes(), np.uint8)
    return w.reshape(w.shape[0], -1)


@pytest.mark.parametrize("name,qt,which", [("q4_K", 12, "isum"), ("q4_K", 12, "msum"), ("q6_K", 14, "isum")])
@pytest.mark.parametrize("rows,cols,M", [(96, 2048, 40), (33, 256, 9)])
def test_kquant_superblock_sums_exact(gpu, oracle, name, qt, which, rows, cols, M):
    """With unit scales (weight d or dmin 1, activation d 1) every output is
    the sum of the row's exact per-superblock integers: q4_K's sum_j sc_j q.a
    (or minus sum_j m_j bsum), q6_K's sum_s sc_s (q - 32).a.  The GPU's must
    equal the oracle's block sums to the bit (each partial sum stays below
    2^24, where fp32 holds integers exactly)."""
    from g4run_amd import synth
    w = _unit_scales(qt, synth.weights(qt, rows, cols, seed=rows + M), cols, which)
    act = oracle.prep_act(qt, synth.activations(M, cols, seed=cols + M))
    for b in range(cols // 256):
        act[:, 292 * b:292 * b + 4] = np.frombuffer(np.float32(1.0).tobytes(), np.uint8)
    t = gpu.Tensor.from_rows(qt, w, cols)
    y = gpu_matmul(gpu, t, act=act, nb=M, path=2)
    k = 0 if which == "isum" else 1          # q4_K sums come in (isum, msum) pairs per superblock
    exp = np.zeros((M, rows), np.int64)
    for m in range(M):
        s = oracle.block_sums(qt, w, act[m], cols).astype(np.int64)
        s = s[:, k::2] if qt == 12 else s
        assert np.abs(np.cumsum(s, axis=1)).max() < 1 << 24
        exp[m] = s.sum(axis=1) if which == "isum" else -s.sum(axis=1)
    assert np.array_equal(y.astype(np.int64), exp), f"{name} {which} {rows}x{cols} M={M}"
    assert np.array_equal(y, exp.astype(np.float32))


@pytest.mark.parametrize("name,qt", KQ)
def test_kquant_ragged_shapes(gpu, oracle, name, qt):
    """Row counts off the 32-row tile, token counts off the 32-token tile and
    the 128-token workgroup, one superblock per row."""
    for rows, cols, M in ((1, 256, 1), (31, 512, 17), (100, 2304, 33), (65, 768, 65), (257, 1024, 100), (33, 4096, 129)):
        w, x, t = _setup(gpu, qt, rows, cols, M, seed=rows + cols)
        assert_close(gpu_matmul(gpu, t, x=x, nb=M, path=2), oracle_matmul(oracle, qt, w, x), f"{name} {rows}x{cols} M={M}")


@pytest.mark.parametrize("name,qt", KQ)
def test_kquant_token_results_independent_of_batch(gpu, oracle, name, qt):
    w, x, t = _setup(gpu, qt, 320, 2560, 300, seed=13)
    full = gpu_matmul(gpu, t, x=x, nb=300, path=2)
    assert_close(full, oracle_matmul(oracle, qt, w, x), f"{name} M=300")
    for m in (9, 32, 33, 100, 128, 129, 257):
        part = gpu_matmul(gpu, t, x=x[:m].copy(), nb=m, path=2)
        assert np.array_equal(bits(part), bits(full[:m])), f"{name} M={m}"


@pytest.mark.parametrize("name,qt", KQ)
def test_kquant_fused_quantizer_equals_prequantized(gpu, oracle, name, qt):
    w, x, t = _setup(gpu, qt, 130, 2816, 45, seed=21)
    a = gpu_matmul(gpu, t, x=x, nb=45, path=2)
    b = gpu_matmul(gpu, t, act=oracle.prep_act(qt, x), nb=45, path=2)
    assert np.array_equal(bits(a), bits(b))
