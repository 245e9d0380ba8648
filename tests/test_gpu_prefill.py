"""GPU parity of the batched-prefill matmul on the int8 matrix cores (path 2)
against the CPU oracle's shipped-order dots (q8_0 4096x4096
x M tokens), plus its batch-size invariance and error paths.

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
    4096 rows x 256 tokens run the LDS-staged tiles, the smaller batches the
    one-tile kernel."""
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
    tk = G.Tensor.from_rows(12, synth.weights(12, 64, 256, seed=1), 256)
    assert [G.matmul_path(t8, n) for n in (1, 8, 9, 16, 512)] == [1, 1, 2, 2, 2]
    assert G.matmul_path(tk, 512) == 1
    Y = G.Buffer(64 * 16 * 4)
    x = G.Buffer.from_array(synth.activations(16, 256, seed=2))
    with pytest.raises(G.G4HError) as e:
        G.matmul(tk, Y, nb=16, x=x, path=2)
    assert e.value.status == G.ERR_TYPE


@pytest.mark.parametrize("qt", [8, 2])
@pytest.mark.parametrize("rows,cols,Ms", [(4096, 4096, (1, 8, 16, 32, 48, 64)), (100, 2080, (1, 5, 17, 33, 64)),
                                          (33, 1056, (2, 31, 32, 49)), (17, 10240, (3, 16, 19, 63)),
                                          (48, 64, (1, 64)), (16, 32, (7,))])
def test_few_kernel_equals_tile_kernel(gpu, oracle, monkeypatch, qt, rows, cols, Ms):
    """The few-token kernel (up to 64 tokens; each weight byte read once,
    operands of a block pair swapped across lane halves) gives the tile
    kernel's bits (G4H_MM_FEW=0): the same exact block sums, exact scale
    products and residue-pair partial sums.  Ragged rows, token counts off the
    16-token tile, odd block counts (a lone last block) and block counts off
    the 8-block stage, one and two blocks per row."""
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
