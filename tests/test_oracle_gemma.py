"""Pins of the oracle's gemma4 forward (oracle/g4o_gemma.c, a restatement of
model.c:592-799, which does not compile here).

- the window / ring attention equals the plain attention over the same
  positions held linearly (bit for bit), also across the ring's wrap;
- RoPE with frequency factors against the float64 angle pos*base^(-2i/n)/ff_i;
- the soft-cap against cap*tanh(l/cap) in float64;
- a batch of tokens equals the same tokens one at a time (bit for bit);
- the whole forward against an independent float64 numpy model of the same
  architecture (dequantized weights, no activation quantization, exact softmax),
  with planted structural mistakes in that float64 model (a missing soft-cap,
  per-layer embedding, output scale, sliding window, V = K fallback, or the
  wrong shared cache) each moving the logits by many times the bar.
"""
import numpy as np
import pytest

import gemma_util as GM

F16 = 1


def test_window_and_ring_equal_linear_attention(oracle):
    rs = np.random.default_rng(1)
    H, hd, slots = 4, 64, 40
    for kv_type in (1, 8, 2):
        rb = hd * 2 if kv_type == F16 else oracle.row_size(kv_type, hd)
        n = 100                                           # positions 0..99, ring of 40 wraps twice
        kv = rs.standard_normal((2, n, hd)).astype(np.float32)

        def store(rows):
            out = np.zeros((len(rows), rb), np.uint8)
            for i, r in enumerate(rows):
                oracle.lib().g4o_kv_store(kv_type, out[i].ctypes.data, np.ascontiguousarray(r).ctypes.data, hd)
            return out

        lin_k, lin_v = store(kv[0]), store(kv[1])
        q = rs.standard_normal(H * hd).astype(np.float32)
        for pos, j0 in ((99, 70), (99, 99), (80, 41)):
            # the ring as the decode leaves it after position pos
            ring_k, ring_v = np.zeros((slots, rb), np.uint8), np.zeros((slots, rb), np.uint8)
            for p in range(pos + 1):
                ring_k[p % slots], ring_v[p % slots] = lin_k[p], lin_v[p]
            a = np.zeros(H * hd, np.float32)
            b = np.zeros(H * hd, np.float32)
            L = oracle.lib()
            L.g4o_attn_window.argtypes = [oracle._vp] * 3 + [oracle.C.c_int] * 7 + [oracle._vp, oracle.C.c_int]
            L.g4o_attn_window(q.ctypes.data, ring_k.ctypes.data, ring_v.ctypes.data, kv_type, H, 1, hd, pos, j0, slots,
                              a.ctypes.data, 1)
            # the same positions as a fresh linear cache starting at j0
            sk, sv = np.ascontiguousarray(lin_k[j0:pos + 1]), np.ascontiguousarray(lin_v[j0:pos + 1])
            L.g4o_attn_decode(q.ctypes.data, sk.ctypes.data, sv.ctypes.data, kv_type, H, 1, hd, pos - j0, b.ctypes.data, 1)
            assert a.tobytes() == b.tobytes(), (kv_type, pos, j0)


def test_rope_frequency_factors(oracle):
    rs = np.random.default_rng(2)
    n, base = 128, 1e6
    ff = (1 + rs.random(n // 2) * 3).astype(np.float32)
    L = oracle.lib()
    L.g4o_rope_cache_ff.argtypes = [oracle._vp, oracle.C.c_int, oracle.C.c_int, oracle.C.c_float, oracle._vp]
    for pos in (0, 1, 37, 900):
        cs = np.zeros(n, np.float32)
        L.g4o_rope_cache_ff(cs.ctypes.data, n, pos, base, ff.ctypes.data)
        ang = pos * np.power(np.float64(base), -2.0 * np.arange(n // 2) / n) / ff.astype(np.float64)
        # theta accumulates in fp32 (model.c:352-356): a relative error of ~i ulps
        tol = 1e-6 * (1 + pos) * (1 + np.arange(n // 2))
        assert np.all(np.abs(cs[0::2] - np.cos(ang)) <= tol + 1e-6)
        assert np.all(np.abs(cs[1::2] - np.sin(ang)) <= tol + 1e-6)


def prefill(og, tokens, nb=16):
    out = []
    for i in range(0, len(tokens), nb):
        lg, hn = og.forward(tokens[i:i + nb], i)
        out.append(lg)
    return np.concatenate(out)


def test_softcap_closed_form(oracle):
    hp, T = GM.make_gemma(oracle, 3)
    toks = np.random.default_rng(3).integers(0, hp["n_vocab"], 12)
    capped = prefill(oracle.Gemma(hp, T, F16, 64), toks)
    raw = prefill(oracle.Gemma(dict(hp, final_softcap=0.0), T, F16, 64), toks)
    cap = np.float64(hp["final_softcap"])
    want = cap * np.tanh(raw.astype(np.float64) / cap)
    assert np.abs(capped - want).max() <= 4e-6 * cap
    assert np.abs(raw).max() > cap                      # the cap bites


def test_batch_equals_one_token_at_a_time(oracle):
    hp, T = GM.make_gemma(oracle, 4)
    toks = np.random.default_rng(4).integers(0, hp["n_vocab"], 20)
    a = prefill(oracle.Gemma(hp, T, F16, 64), toks, nb=20)
    b = prefill(oracle.Gemma(hp, T, F16, 64), toks, nb=1)
    assert a.tobytes() == b.tobytes()


# ------------------------------------------------ independent float64 model
def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def _rms(x, w=None, eps=1e-6):
    y = x / np.sqrt(np.mean(x * x) + eps)
    return y * w if w is not None else y


def _rope(x, pos, base, ff=None):
    n = x.shape[-1]
    ang = pos * np.power(base, -2.0 * np.arange(n // 2) / n)
    if ff is not None:
        ang = ang / ff
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :n // 2], x[..., n // 2:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


def f64_model(oracle, hp, T, tokens, mistake=None):
    """Logits of every position, decoding tokens from position 0."""
    def W(name):
        t, ne, raw = T[name]
        if t == 0:
            return np.asarray(raw, np.float64)
        return oracle.dequant(t, np.ascontiguousarray(raw).reshape(ne[1], -1), ne[0]).astype(np.float64)

    def vec(name):
        return np.asarray(T[name][2], np.float64)

    E, H, PE, NL, nkv = hp["n_embd"], hp["n_head"], hp["n_embd_per_layer"], hp["n_layer"], hp["n_layer_kv"]
    eps = hp["rms_eps"]
    emb, pemb, pproj = W("token_embd.weight"), W("per_layer_token_embd.weight"), W("per_layer_model_proj.weight")
    K, V = {}, {}
    out = []
    for pos, tok in enumerate(tokens):
        x = emb[tok] * np.sqrt(E)
        pt = (pemb[tok] * np.sqrt(PE)).reshape(NL, PE)
        pp = (pproj @ x / np.sqrt(E)).reshape(NL, PE)
        pl = np.stack([(_rms(pp[l], vec("per_layer_proj_norm.weight"), eps) + pt[l]) / np.sqrt(2) for l in range(NL)])
        for il in range(NL):
            p = f"blk.{il}."
            swa = hp["is_swa"][il] and mistake != "no_window"
            hd = hp["head_dim_swa"] if hp["is_swa"][il] else hp["head_dim_full"]
            base = hp["rope_base_swa"] if hp["is_swa"][il] else hp["rope_base_full"]
            ff = None if hp["is_swa"][il] else vec("rope_freqs.weight")
            xb = _rms(x, vec(p + "attn_norm.weight"), eps)
            q = (W(p + "attn_q.weight") @ xb).reshape(H, hd)
            q = _rope(np.stack([_rms(qh, vec(p + "attn_q_norm.weight"), eps) for qh in q]), pos, base, ff)
            if il < nkv:
                k = W(p + "attn_k.weight") @ xb
                if p + "attn_v.weight" in T:
                    v = W(p + "attn_v.weight") @ xb
                else:
                    v = k.copy() if mistake != "no_v_fallback" else np.zeros_like(k)
                K.setdefault(il, []).append(_rope(_rms(k, vec(p + "attn_k_norm.weight"), eps), pos, base, ff))
                V.setdefault(il, []).append(_rms(v, None, eps))
            if il < nkv:
                cil = il
            elif mistake == "wrong_share":
                cil = nkv - 1 if hp["is_swa"][il] else nkv - 2
            else:
                cil = nkv - 2 if hp["is_swa"][il] else nkv - 1
            j0 = max(0, pos - hp["n_swa"] + 1) if swa else 0
            keys, vals = np.array(K[cil][j0:pos + 1]), np.array(V[cil][j0:pos + 1])
            if keys.shape[1] != hd:
                keys, vals = np.zeros((pos + 1 - j0, hd)), np.zeros((pos + 1 - j0, hd))
            s = q @ keys.T
            w = np.exp(s - s.max(axis=1, keepdims=True))
            w /= w.sum(axis=1, keepdims=True)
            o = (w @ vals).reshape(-1)
            x = x + _rms(W(p + "attn_output.weight") @ o, vec(p + "post_attention_norm.weight"), eps)
            xb = _rms(x, vec(p + "ffn_norm.weight"), eps)
            h = _gelu(W(p + "ffn_gate.weight") @ xb) * (W(p + "ffn_up.weight") @ xb)
            x = x + _rms(W(p + "ffn_down.weight") @ h, vec(p + "post_ffw_norm.weight"), eps)
            if mistake != "no_ple":
                g = _gelu(W(p + "inp_gate.weight") @ x) * pl[il]
                x = x + _rms(W(p + "proj.weight") @ g, vec(p + "post_norm.weight"), eps)
            sc = p + "layer_output_scale.weight"
            if sc in T and mistake != "no_out_scale":
                x = x * np.float64(T[sc][2][0])
        lg = emb @ _rms(x, vec("output_norm.weight"), eps)
        if mistake != "no_softcap":
            lg = hp["final_softcap"] * np.tanh(lg / hp["final_softcap"])
        out.append(lg)
    return np.array(out)


def test_forward_matches_float64_model(oracle):
    hp, T = GM.make_gemma(oracle, 5)
    toks = np.random.default_rng(5).integers(0, hp["n_vocab"], 24)       # past the window of 8
    got = prefill(oracle.Gemma(hp, T, F16, 64), toks, nb=8)
    ref = f64_model(oracle, hp, T, toks)
    rng = ref.max(axis=1, keepdims=True) - ref.min(axis=1, keepdims=True)
    err = np.abs(got - ref) / rng
    bar = 2e-2
    print(f"oracle vs float64 model: worst {err.max():.3g} of the logit range (bar {bar})")
    assert err.max() <= bar
    for mistake in ("no_softcap", "no_ple", "no_out_scale", "no_window", "no_v_fallback", "wrong_share"):
        bad = f64_model(oracle, hp, T, toks, mistake)
        moved = (np.abs(bad - ref) / rng).max()
        print(f"  planted {mistake}: moves the float64 model by {moved:.3g}")
        assert moved > 5 * bar, mistake
