"""Pins for the oracle's model-level functions (CPU only).

The reference's model.c does not compile in this container (it includes
windows.h), so rms_norm, RoPE, attention, argmax and the decode graph of the
oracle cannot be compared with a reference build.  They are pinned here by
checks that a plausible mistake would fail: float64 recomputations, closed
forms and invariants (scale invariance, rotations, one-hot and identical-key
softmax, the GQA head mapping), and a float64 numpy decode of a tiny model
built only from the oracle's already-pinned primitives (quantizers, dequant).
"""
import numpy as np
import pytest

F16, Q8_0, Q4_0 = 1, 8, 2


# ---------------------------------------------------------------- rms_norm
def test_rms_norm_float64_recomputation(oracle):
    rng = np.random.default_rng(1)
    for n in (64, 256, 2560):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = (1 + 0.05 * rng.standard_normal(n)).astype(np.float32)
        y = oracle.rms_norm(x, w, 1e-6)
        ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
        np.testing.assert_allclose(y, ref, rtol=2e-6, atol=0)      # n-1, a missing eps or a float sum would exceed this


def test_rms_norm_scale_invariance_and_unit_rms(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(2560).astype(np.float32)
    y0 = oracle.rms_norm(x, None, 0.0)
    for k in (-20, -3, 5, 30):                                       # power-of-two scaling is exact
        assert np.array_equal(oracle.rms_norm(np.ldexp(x, k), None, 0.0), y0)
    assert abs(np.mean(y0.astype(np.float64) ** 2) - 1.0) < 1e-6


# -------------------------------------------------------------------- rope
def _rope64(x, pos, base):
    """NeoX rotation of (i, i+n/2) with theta accumulated in fp32 as the
    reference does (theta *= base^(-2/n)), cos/sin in float64."""
    n = x.size
    h = n // 2
    scale = np.float32(np.power(np.float32(base), np.float32(-2.0) / np.float32(n)))
    th = np.empty(h, np.float32)
    t = np.float32(pos)
    for i in range(h):
        th[i] = t
        t = np.float32(t * scale)
    c, s = np.cos(th.astype(np.float64)), np.sin(th.astype(np.float64))
    a, b = x[:h].astype(np.float64), x[h:].astype(np.float64)
    return np.concatenate([a * c - b * s, a * s + b * c])


@pytest.mark.parametrize("n", [64, 128, 256])
def test_rope_against_float64_rotation(oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    for pos in (0, 1, 7, 1000, 8191):
        y = oracle.rope(x, pos, 1e6)
        np.testing.assert_allclose(y, _rope64(x, pos, 1e6), rtol=0, atol=2e-6 * (1 + np.abs(x).max()))
    assert np.array_equal(oracle.rope(x, 0, 1e6), x)                  # position 0 is the identity


def test_rope_is_a_rotation_by_position(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(128).astype(np.float32)
    h = 64
    y = oracle.rope(x, 37, 1e4)
    np.testing.assert_allclose(y[:h] ** 2 + y[h:] ** 2, x[:h] ** 2 + x[h:] ** 2, rtol=1e-5)
    # rotating by a then b equals rotating by a+b (pairs are (i, i+n/2), not (2i, 2i+1))
    np.testing.assert_allclose(oracle.rope(oracle.rope(x, 5, 1e4), 9, 1e4), oracle.rope(x, 14, 1e4), atol=1e-5)


# --------------------------------------------------------------- attention
def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def test_attention_identical_keys_average_values(oracle):
    hd, n_head, n_kv, npos = 64, 2, 1, 300
    rng = np.random.default_rng(4)
    k = np.tile(_f16(rng.standard_normal(hd)), (npos, 1))
    v = _f16(rng.standard_normal((npos, hd)))
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    out = oracle.attn_decode(q, k.view(np.uint16), v.view(np.uint16), F16, n_head, n_kv, hd, npos - 1)
    w = np.float64(np.float16(1.0 / npos))                           # every weight is fp16(1/n)
    ref = w * v.astype(np.float64).sum(0)
    for h in range(n_head):
        np.testing.assert_allclose(out[h], ref, rtol=1e-5, atol=1e-6)


def test_attention_one_hot_and_float64(oracle):
    hd, n_head, n_kv, npos = 128, 8, 4, 257
    rng = np.random.default_rng(5)
    k = _f16(rng.standard_normal((npos, n_kv, hd)) * 0.1)
    v = _f16(rng.standard_normal((npos, n_kv, hd)))
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    k[123, :, :] = _f16(q[::2] * 40)                                  # one dominant key per KV head
    out = oracle.attn_decode(q, k.view(np.uint16), v.view(np.uint16), F16, n_head, n_kv, hd, npos - 1)
    # float64 attention with the reference's roundings of q (fp16) and of the weights (fp16)
    for h in range(n_head):
        g = h // (n_head // n_kv)
        s = k[:, g].astype(np.float64) @ np.float16(q[h]).astype(np.float64)
        e = np.exp(s - s.max())
        w = (e / e.sum()).astype(np.float32).astype(np.float16).astype(np.float64)
        np.testing.assert_allclose(out[h], w @ v[:, g].astype(np.float64), rtol=1e-4, atol=1e-4)
        if h % 2 == 0:
            np.testing.assert_allclose(out[h], v[123, g].astype(np.float64), atol=1e-3)


def test_attention_gqa_head_mapping(oracle):
    """Query head h reads KV head h / (n_head / n_kv) (model.c:1099)."""
    hd, n_head, n_kv, npos = 64, 8, 2, 40
    rng = np.random.default_rng(6)
    k = _f16(rng.standard_normal((npos, n_kv, hd)))
    v = np.zeros((npos, n_kv, hd), np.float16)
    for g in range(n_kv):
        v[:, g, :] = g + 1                                            # a constant per KV head
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    out = oracle.attn_decode(q, k.view(np.uint16), v.view(np.uint16), F16, n_head, n_kv, hd, npos - 1)
    for h in range(n_head):
        np.testing.assert_allclose(out[h], h // (n_head // n_kv) + 1, rtol=2e-3)


# ------------------------------------------------------------------ argmax
def test_argmax_first_maximum_and_nan(oracle):
    L = oracle.lib()

    def am(v):
        v = np.ascontiguousarray(v, np.float32)
        return L.g4o_argmax(v.ctypes.data_as(oracle._vp), v.size)

    assert am([1, 5, 5, 2]) == 1                                     # ties keep the first index
    assert am([np.nan, 5, 7]) == 0                                   # sampler.c:139-144: nothing beats a NaN at 0
    assert am([1, np.nan, 7, np.nan]) == 2                           # later NaNs never win
    assert am([-np.inf, -np.inf]) == 0


# ------------------------------------------------------------ decode graph
def test_decode_graph_float64_recomputation(oracle):
    """A tiny model decoded by the oracle equals a float64 numpy decode built
    from the pinned primitives (dequantized q4_0 weights, q8_0 activations)."""
    from g4run_amd import synth
    rng = np.random.default_rng(7)
    L_, E, H, KV, hd, F, V, ctx = 2, 64, 2, 1, 64, 128, 96, 16
    eps, base = 1e-6, 1e6
    qk = lambda rows, cols, s: oracle.quantize(Q4_0, (rng.standard_normal((rows, cols)) * 0.2).astype(np.float32))
    w = {"wqkv": [qk((H + 2 * KV) * hd, E, 0) for _ in range(L_)], "wo": [qk(E, H * hd, 0) for _ in range(L_)],
         "wgu": [qk(2 * F, E, 0) for _ in range(L_)], "wdown": [qk(E, F, 0) for _ in range(L_)]}
    for nm, n in (("attn_norm", E), ("q_norm", hd), ("k_norm", hd), ("post_attn_norm", E), ("ffn_norm", E),
                  ("post_ffw_norm", E)):
        w[nm] = [(1 + 0.05 * rng.standard_normal(n)).astype(np.float32) for _ in range(L_)]
    w["output_norm"] = (1 + 0.05 * rng.standard_normal(E)).astype(np.float32)
    w["head"] = oracle.quantize(Q8_0, (rng.standard_normal((V, E)) * 0.5).astype(np.float32))
    kc = [_f16(rng.standard_normal(ctx * KV * hd)).view(np.uint8).copy() for _ in range(L_)]
    vc = [_f16(rng.standard_normal(ctx * KV * hd)).view(np.uint8).copy() for _ in range(L_)]
    cfg = {"n_layer": L_, "n_embd": E, "n_head": H, "n_kv": KV, "hd": hd, "n_ff": F, "n_vocab": V, "n_ctx": ctx,
           "rope_base": base, "eps": eps, "kv_type": F16, "wtype": Q4_0, "head_type": Q8_0}
    kc64 = [np.frombuffer(c.tobytes(), np.float16).astype(np.float64).reshape(ctx, KV, hd) for c in kc]
    vc64 = [np.frombuffer(c.tobytes(), np.float16).astype(np.float64).reshape(ctx, KV, hd) for c in vc]
    m = oracle.Model(cfg, w, kc, vc)
    token, pos = 5, 9
    tok, logits = m.decode(token, pos)

    deq = lambda t, a, n: oracle.dequant(t, a, n).astype(np.float64).reshape(-1, n)

    def mm(t, W, x):                          # matmul_b: x quantized to q8_0, then an exact-ish float64 dot
        xq = deq(Q8_0, oracle.quantize(Q8_0, x.astype(np.float32)[None]), x.size)[0]
        return deq(t, W, x.size) @ xq

    def rms(x, wt):
        return x / np.sqrt(np.mean(x * x) + eps) * (1 if wt is None else wt)

    def rope(x):
        return _rope64(x.astype(np.float32), pos, base)

    gelu = lambda x: 0.5 * x * (1 + np.tanh(0.7978845608028654 * x * (1 + 0.044715 * x * x)))
    x = deq(Q8_0, w["head"][token:token + 1], E)[0] * np.float32(np.sqrt(np.float32(E)))
    for l in range(L_):
        qkv = mm(Q4_0, w["wqkv"][l], rms(x, w["attn_norm"][l]))
        q = [rope(rms(qkv[h * hd:(h + 1) * hd], w["q_norm"][l])) for h in range(H)]
        kn = rope(rms(qkv[H * hd:(H + 1) * hd], w["k_norm"][l]))
        vn = rms(qkv[(H + 1) * hd:], None)
        kc64[l][pos, 0] = np.float16(kn)
        vc64[l][pos, 0] = np.float16(vn)
        att = []
        for h in range(H):
            s = kc64[l][:pos + 1, 0] @ np.float16(q[h]).astype(np.float64)
            e = np.exp(s - s.max())
            att.append((e / e.sum()) @ vc64[l][:pos + 1, 0])
        x = x + rms(mm(Q4_0, w["wo"][l], np.concatenate(att)), w["post_attn_norm"][l])
        gu = mm(Q4_0, w["wgu"][l], rms(x, w["ffn_norm"][l]))
        x = x + rms(mm(Q4_0, w["wdown"][l], gelu(gu[:F]) * gu[F:]), w["post_ffw_norm"][l])
    ref = mm(Q8_0, w["head"], rms(x, w["output_norm"]))
    scale = np.abs(ref).max()
    # measured 3.6e-4 of the largest logit (fp16 GELU table, fp16 weights, fp32 dots);
    # a gate/up swap gives 0.15 and a dropped post-attention norm 0.10
    np.testing.assert_allclose(logits, ref, rtol=0, atol=3e-3 * scale)
    assert tok == int(np.argmax(logits))


# ------------------------------------------------- attention, quantized KV
# model.c:530-577 over a q8_0 / q4_0 cache: the query is quantized to q8_0
# (model.c:533), each score is the K row's q8_0 / q4_0 dot with it (model.c:538),
# and the V rows are dequantized and weighted by the fp32 probability e*inv
# with no fp16 rounding (model.c:571-577), unlike the f16 cache (model.c:555).
def _qkv_cache(oracle, kv_type, x):
    """Rows of x [..., hd] stored as kv_type blocks, and their dequantized values."""
    hd = x.shape[-1]
    rows = oracle.quantize(kv_type, x.reshape(-1, hd).astype(np.float32))
    return rows, oracle.dequant(kv_type, rows, hd).astype(np.float64).reshape(x.shape)


@pytest.mark.parametrize("kv_type", [Q8_0, Q4_0], ids=["q8_0", "q4_0"])
@pytest.mark.parametrize("npos", [3, 300])
def test_attention_quantized_identical_keys_fp32_weights(oracle, kv_type, npos):
    """Identical keys give equal scores, so every weight is exactly the fp32
    inv = (float)(1/n).  With n = 3, fp16(1/3) differs from it by 2.4e-4
    relative, so a weight rounded to fp16 (the f16-cache rule) fails the bar."""
    hd, n_head, n_kv = 64, 2, 1
    rng = np.random.default_rng(40 + npos)
    krow, _ = _qkv_cache(oracle, kv_type, rng.standard_normal(hd))
    k = np.tile(krow, (npos, 1))
    v, v64 = _qkv_cache(oracle, kv_type, rng.standard_normal((npos, hd)))
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    out = oracle.attn_decode(q, k, v, kv_type, n_head, n_kv, hd, npos - 1)
    w = np.float64(np.float32(1.0 / npos))
    ref = w * v64.sum(0)
    scale = np.abs(v64).max()
    for h in range(n_head):
        np.testing.assert_allclose(out[h], ref, rtol=1e-6, atol=1e-6 * scale * np.sqrt(npos))
    if npos == 3:
        wrong = np.float64(np.float16(1.0 / npos)) * v64.sum(0)
        assert np.abs(out[0] - wrong).max() > 50 * 1e-6 * scale      # the check can tell the two rules apart


@pytest.mark.parametrize("kv_type", [Q8_0, Q4_0], ids=["q8_0", "q4_0"])
def test_attention_quantized_one_hot_key(oracle, kv_type):
    hd, n_head, n_kv, npos = 128, 4, 2, 130
    rng = np.random.default_rng(41)
    kx = rng.standard_normal((npos, n_kv, hd)) * 0.05
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    kx[77, 0] = q[0] * 30                                               # dominant for heads 0 and 1 of KV head 0
    kx[12, 1] = q[2] * 30                                               # and for heads 2, 3 of KV head 1
    k, _ = _qkv_cache(oracle, kv_type, kx)
    v, v64 = _qkv_cache(oracle, kv_type, rng.standard_normal((npos, n_kv, hd)))
    out = oracle.attn_decode(q, k, v, kv_type, n_head, n_kv, hd, npos - 1)
    np.testing.assert_allclose(out[0], v64[77, 0], atol=1e-4 * np.abs(v64).max())
    np.testing.assert_allclose(out[2], v64[12, 1], atol=1e-4 * np.abs(v64).max())


@pytest.mark.parametrize("kv_type", [Q8_0, Q4_0], ids=["q8_0", "q4_0"])
def test_attention_quantized_float64_recomputation(oracle, kv_type):
    """float64 attention from the dequantized K/V rows and the q8_0-quantized
    query, fp32 weights, within 5e-6 of the largest output (measured: 5.4e-7).
    An fp16 query (the f16-cache rule) moves the outputs by >= 1.4e-3 and fp16
    weights by >= 5e-5 of the largest output on every head here, so the same
    bar rejects both rules by 10x or more."""
    hd, n_head, n_kv, npos = 256, 8, 4, 65
    rng = np.random.default_rng(42)
    k, k64 = _qkv_cache(oracle, kv_type, rng.standard_normal((npos, n_kv, hd)) * 0.15)
    v, v64 = _qkv_cache(oracle, kv_type, rng.standard_normal((npos, n_kv, hd)))
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    out = oracle.attn_decode(q, k, v, kv_type, n_head, n_kv, hd, npos - 1)
    qd = oracle.dequant(Q8_0, oracle.quantize(Q8_0, q), hd).astype(np.float64)
    for h in range(n_head):
        g = h // (n_head // n_kv)
        s = k64[:, g] @ qd[h]
        e = np.exp(s - s.max())
        w = (e / e.sum()).astype(np.float32).astype(np.float64)
        ref = w @ v64[:, g]
        bar = 5e-6 * np.abs(ref).max()
        np.testing.assert_allclose(out[h], ref, rtol=0, atol=bar)
        # the same bar with the other rounding rules fails (so it pins them)
        s16 = k64[:, g] @ np.float16(q[h]).astype(np.float64)
        e16 = np.exp(s16 - s16.max())
        assert np.abs(out[h] - (e16 / e16.sum()) @ v64[:, g]).max() > 10 * bar
        wh = (e / e.sum()).astype(np.float32).astype(np.float16).astype(np.float64)
        assert np.abs(out[h] - wh @ v64[:, g]).max() > 10 * bar
