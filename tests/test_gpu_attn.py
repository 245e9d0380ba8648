"""Decode attention (attn_kernel, model.c:509-580) and kv_store on the GPU
against the CPU oracle.  KV stores are bit-exact; the attention output is
within |gpu-cpu| <= 1e-5 + 1e-3|cpu| (only the fp32 order of the final
V accumulation differs from the CPU's loop)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-5


def make_cache(G, oracle, kv_type, n_slot, n_kv, hd, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_slot * n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((n_slot * n_kv, hd)).astype(np.float32)
    rb = hd * 2 if kv_type == G.F16 else G.row_size(kv_type, hd)
    kb, vb = G.Buffer(n_slot * n_kv * rb), G.Buffer(n_slot * n_kv * rb)
    G.kv_store(kv_type, G.Buffer.from_array(k), kb, hd, rows=n_slot * n_kv, dst_stride=rb)
    G.kv_store(kv_type, G.Buffer.from_array(v), vb, hd, rows=n_slot * n_kv, dst_stride=rb)
    kh = kb.download(np.uint8, (n_slot * n_kv, rb))
    vh = vb.download(np.uint8, (n_slot * n_kv, rb))
    # kv_store parity (model.c:583-589): bit-exact
    if kv_type == G.F16:
        assert np.array_equal(kh.view(np.uint16), oracle.fp32_to_fp16(k))
    else:
        assert np.array_equal(kh, oracle.quantize(kv_type, k))
    return kb, vb, kh, vh


@pytest.mark.parametrize("kv_type", [1, 8], ids=["f16", "q8_0"])
@pytest.mark.parametrize("n_head,n_kv,hd,n_pos,qscale", [
    (8, 4, 256, 1, 1.0), (8, 4, 256, 65, 1.0), (8, 4, 256, 1000, 1.0), (8, 4, 256, 8192, 1.0),
    (8, 4, 256, 3000, 0.02), (4, 4, 128, 300, 0.1), (8, 1, 64, 777, 0.3), (16, 2, 192, 129, 1.0),
])
def test_attention_vs_oracle(gpu, oracle, kv_type, n_head, n_kv, hd, n_pos, qscale):
    G = gpu
    kb, vb, kh, vh = make_cache(G, oracle, kv_type, n_pos, n_kv, hd, seed=n_pos + hd)
    q = (np.random.default_rng(5).standard_normal((n_head, hd)) * qscale).astype(np.float32)
    out = G.Buffer(n_head * hd * 4)
    G.attn_decode(G.Buffer.from_array(q), kb, vb, kv_type, n_head, n_kv, hd, n_pos, out)
    got = out.download(np.float32, (n_head, hd))
    ref = oracle.attn_decode(q, kh, vh, kv_type, n_head, n_kv, hd, n_pos - 1)
    err = np.abs(got.astype(np.float64) - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} outside tolerance, worst {err.max():.3g}"


def test_attention_identical_keys_average_values(gpu, oracle):
    """All keys equal -> uniform weights fp16(1/n): the output is the mean of V
    up to that rounding (softmax invariant; closed form)."""
    G = gpu
    n_head, n_kv, hd, n_pos = 2, 1, 128, 100
    k = np.tile(np.random.default_rng(1).standard_normal(hd).astype(np.float32), (n_pos, 1))
    v = np.random.default_rng(2).standard_normal((n_pos, hd)).astype(np.float32)
    kb, vb = G.Buffer(n_pos * hd * 2), G.Buffer(n_pos * hd * 2)
    G.kv_store(G.F16, G.Buffer.from_array(k), kb, hd, rows=n_pos)
    G.kv_store(G.F16, G.Buffer.from_array(v), vb, hd, rows=n_pos)
    q = np.random.default_rng(3).standard_normal((n_head, hd)).astype(np.float32)
    out = G.Buffer(n_head * hd * 4)
    G.attn_decode(G.Buffer.from_array(q), kb, vb, G.F16, n_head, n_kv, hd, n_pos, out)
    got = out.download(np.float32, (n_head, hd))
    w = np.float32(np.float16(np.float32(1.0) * np.float32(1.0 / n_pos)))
    vf = oracle.fp16_to_fp32(oracle.fp32_to_fp16(v)).astype(np.float64)
    expect = (w * vf).sum(0)
    assert np.allclose(got, expect[None, :], rtol=1e-5, atol=1e-6)


def test_attention_bad_shapes(gpu):
    import ctypes as C
    G = gpu
    L = G.lib()
    b = G.Buffer(1 << 16)
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.Q4_K, 8, 4, 256, 10, b.ptr, b.ptr, b.nbytes, None) == G.ERR_TYPE
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.F16, 8, 3, 256, 10, b.ptr, b.ptr, b.nbytes, None) == G.ERR_SHAPE
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.F16, 8, 4, 96, 10, b.ptr, b.ptr, b.nbytes, None) == G.ERR_SHAPE
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.F16, 8, 4, 256, 10, b.ptr, b.ptr, 16, None) == G.ERR_ARG
