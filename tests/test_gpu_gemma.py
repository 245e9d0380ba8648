"""A gemma4 model loaded from a GGUF file the test writes (g4h_gemma_open: the
GPU form of g4_gguf_open + g4_ctx_init + forward_layers/heads) against the
oracle's gemma4 forward on the same tensors (tests/test_oracle_gemma.py pins
that forward).

Bar: part by part.  With the per-token trace (g4h_gemma_trace) every part of
every layer of every token is recomputed by the oracle from the GPU's own
inputs to that part -- the per-layer inputs, each projection, the q/k/v
preparation and the K/V rows stored (bit for bit against the GPU's caches),
the attention over the cache as the GPU holds it, each residual, the GELU
products, the per-layer embedding injection, and the head with its soft-cap --
and held to |gpu - cpu| <= 1e-5 + 1e-3 |cpu| per element (the attention with
the fp16-weight slack of test_gpu_model).  The whole stack is chaotic at the
ulp level (an fp16 query or softmax weight, a q8_0 activation code landing on
the other side of a rounding edge), so only such part-by-part checks hold a
per-element tolerance; the whole-model runs are also held to the oracle's
greedy token where its top-two gap is clear, and a batch to one token at a
time bit for bit."""
import os

import numpy as np
import pytest

import gemma_util as GM

pytestmark = pytest.mark.gpu


BAR = 5e-2
ATOL, RTOL = 1e-5, 1e-3


def _close(got, ref, what, slack=0.0):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref) + slack
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside 1e-3/1e-5, worst {err.max():.3g}"
    return float(err.max())


def _rope_ff(o, x, pos, base, ff):
    """NeoX RoPE with frequency factors (model.c:349-367) through the oracle."""
    import ctypes as C
    L = o.lib()
    L.g4o_rope_cache_ff.argtypes = [o._vp, C.c_int, C.c_int, C.c_float, o._vp]
    L.g4o_rope_apply.argtypes = [o._vp, o._vp, C.c_int]
    x = np.ascontiguousarray(x, np.float32).copy()
    cs = np.zeros(x.size, np.float32)
    ffa = np.ascontiguousarray(ff, np.float32) if ff is not None else None
    L.g4o_rope_cache_ff(cs.ctypes.data, x.size, pos, base, ffa.ctypes.data if ffa is not None else None)
    L.g4o_rope_apply(x.ctypes.data, cs.ctypes.data, x.size)
    return x


def _attn_window(o, q, kc, vc, kv_type, H, hd, pos, j0, slots):
    import ctypes as C
    L = o.lib()
    L.g4o_attn_window.argtypes = [o._vp] * 3 + [C.c_int] * 7 + [o._vp, C.c_int]
    out = np.zeros(H * hd, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    L.g4o_attn_window(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, kv_type, H, 1, hd, pos, j0, slots, out.ctypes.data, 1)
    return out


def _weight_slack(o, q, kc, vc, H, hd, pos, j0, slots):
    """f16 V: where a softmax weight lies within 1e-4 of an fp16 rounding
    midpoint, the GPU's weight (its scores differ by the fp32 order of the dot)
    may take the neighbouring code; per output element the most that can move
    it (test_gpu_model._attn_slack, over a window of a ring)."""
    js = [(j0 + i) % slots for i in range(pos - j0 + 1)]
    K = np.frombuffer(kc.tobytes(), np.float16).reshape(slots, hd)[js].astype(np.float64)
    V = np.frombuffer(vc.tobytes(), np.float16).reshape(slots, hd)[js].astype(np.float64)
    slack = np.zeros((H, hd))
    for h in range(H):
        q16 = q[h * hd:(h + 1) * hd].astype(np.float16).astype(np.float64)
        sc = K @ q16
        w = np.exp(sc - sc.max())
        w /= w.sum()
        w16 = w.astype(np.float32).astype(np.float16)
        a = w16.astype(np.float64)
        up = np.nextafter(w16, np.float16(np.inf)).astype(np.float64)
        dn = np.nextafter(w16, np.float16(-np.inf)).astype(np.float64)
        ulp = np.where(np.abs(w - (a + up) / 2) <= 1e-4 * w, up - a, 0.0) + \
            np.where(np.abs(w - (a + dn) / 2) <= 1e-4 * w, a - dn, 0.0)
        slack[h] = ulp @ np.abs(V)
    return slack.ravel()


RING = 576


def traced_forward(G, o, hp, T, m, kv_type, toks, pos0, n_ctx, prefill=False):
    """m.forward(toks, pos0) (or, with `prefill`, m.prefill: the last
    position's logits only) with the per-token trace; then every part of every
    layer of every token against the oracle on the GPU's own inputs.  Returns
    (logits, hnext) -- ([1][n_vocab], None) for a prefill -- and the worst
    error per part."""
    toks = np.atleast_1d(np.asarray(toks, np.int64))
    nb = toks.size
    E, H, PE, NL, NKV = hp["n_embd"], hp["n_head"], hp["n_embd_per_layer"], hp["n_layer"], hp["n_layer_kv"]
    hdf, hds, eps = hp["head_dim_full"], hp["head_dim_swa"], hp["rms_eps"]
    hdm, Fm, NPL = max(hdf, hds), max(hp["n_ff"][:NL]), NL * PE
    # the caches as the GPU holds them before the call, in the oracle's layout
    ora = {}
    for il in range(NKV):
        swa = hp["is_swa"][il]
        k, v = m.kv(il)
        n = RING if swa else n_ctx
        ora[il] = [k[:k.size * n // (2 * RING if swa else n_ctx)].copy(), v[:v.size * n // (2 * RING if swa else n_ctx)].copy()]
    tb = G.Buffer(nb * m.trace(None) * 4)
    tf = m.trace(tb)
    try:
        if prefill:
            lg, hn = m.prefill(toks, pos0)[None], None
        else:
            lg, hn = m.forward(toks, pos0)
    finally:
        m.trace(None)
    tr = tb.download(np.float32, (nb, tf))
    off, o_ = {}, 0
    for name, n in (("x", E), ("q", H * hdm), ("k", hdm), ("v", hdm), ("att", H * hdm), ("wo", E), ("xmid", E), ("g", Fm),
                    ("u", Fm), ("h", Fm), ("down", E), ("xffn", E), ("plg", PE), ("plh", PE), ("proj", E)):
        off[name] = o_
        o_ += n
    rec = o_
    assert tf == NPL + NL * rec + E
    gpu_kv = {il: m.kv(il) for il in range(NKV)}

    def W(name):
        t, ne, raw = T[name]
        return t, ne[0], np.ascontiguousarray(raw)

    def vec(name):
        return np.frombuffer(np.ascontiguousarray(T[name][2]).tobytes(), np.float32) if name in T else None

    def mm(name, x):
        t, ncols, raw = W(name)
        return o.matmul(t, raw, o.prep_act(t, np.asarray(x, np.float32)[None]), ncols, nthreads=8)[0]

    def row_bytes(hd):
        return hd * 2 if kv_type == 1 else o.row_size(kv_type, hd)

    def store(x, hd):
        x = np.asarray(x, np.float32)[None]
        return (o.fp32_to_fp16(x).view(np.uint8) if kv_type == 1 else o.quantize(kv_type, x)).reshape(row_bytes(hd))

    worst = {}

    def note(k, e):
        worst[k] = max(worst.get(k, 0.0), e)

    # the per-layer inputs (model.c:602-635) from the GPU's scaled embedding
    tt, _, traw = W("per_layer_token_embd.weight")
    for b in range(nb):
        x0 = tr[b, NPL:NPL + E]
        temb = W("token_embd.weight")
        xe = o.dequant(temb[0], temb[2][int(toks[b])], E)[0] * np.float32(np.sqrt(np.float32(E)))
        note("embed", _close(x0, xe, f"token {b} embedding"))
        plp = mm("per_layer_model_proj.weight", x0) * np.float32(1.0 / np.sqrt(np.float32(E)))
        pt = o.dequant(tt, traw[int(toks[b])], NPL)[0] * np.float32(np.sqrt(np.float32(PE)))
        ref = np.concatenate([(o.rms_norm(plp[l * PE:(l + 1) * PE], vec("per_layer_proj_norm.weight"), eps) + pt[l * PE:(l + 1) * PE])
                              * np.float32(1.0 / np.sqrt(np.float32(2.0))) for l in range(NL)])
        note("pl", _close(tr[b, :NPL], ref, f"token {b} per-layer inputs"))
    ff = vec("rope_freqs.weight")
    for il in range(NL):
        p = f"blk.{il}."
        swa = hp["is_swa"][il]
        hd = hds if swa else hdf
        base = hp["rope_base_swa"] if swa else hp["rope_base_full"]
        slots = RING if swa else n_ctx
        own = il < NKV
        cil = il if own else (NKV - 2 if swa else NKV - 1)
        for b in range(nb):
            pos = pos0 + b
            r = tr[b, NPL + il * rec:NPL + (il + 1) * rec]
            g = lambda k, n: r[off[k]:off[k] + n]
            tag = f"layer {il} token {b}"
            x = g("x", E)
            xb = o.rms_norm(x, vec(p + "attn_norm.weight"), eps)
            q = g("q", H * hd)
            note("q", _close(q, mm(p + "attn_q.weight", xb), f"{tag} q"))
            qp = np.concatenate([_rope_ff(o, o.rms_norm(q[h * hd:(h + 1) * hd], vec(p + "attn_q_norm.weight"), eps), pos, base,
                                          None if swa else ff) for h in range(H)])
            if own:
                k = g("k", hd)
                note("k", _close(k, mm(p + "attn_k.weight", xb), f"{tag} k"))
                if p + "attn_v.weight" in T:
                    v = g("v", hd)
                    note("v", _close(v, mm(p + "attn_v.weight", xb), f"{tag} v"))
                else:
                    v = k                                           # V = K (model.c:678)
                kp = _rope_ff(o, o.rms_norm(k, vec(p + "attn_k_norm.weight"), eps), pos, base, None if swa else ff)
                vp = o.rms_norm(v, None, eps)
                rb = row_bytes(hd)
                for c, row in ((0, store(kp, hd)), (1, store(vp, hd))):
                    sl = pos % slots
                    ora[il][c][sl * rb:(sl + 1) * rb] = row
                    assert np.array_equal(gpu_kv[il][c][sl * rb:(sl + 1) * rb], row), f"{tag}: {'KV'[c]} row differs"
                    if swa:                                         # the ring's second copy
                        assert np.array_equal(gpu_kv[il][c][(sl + RING) * rb:(sl + RING + 1) * rb], row), f"{tag}: 2nd copy"
            j0 = max(0, pos - (hp["n_swa"] - 1)) if swa else 0
            kc, vc = ora[cil]
            att_ref = _attn_window(o, qp, kc, vc, kv_type, H, hd, pos, j0, slots)
            sl = _weight_slack(o, qp, kc, vc, H, hd, pos, j0, slots) if kv_type == 1 else 0.0
            att = g("att", H * hd)
            note("att", _close(att, att_ref, f"{tag} attention", sl))
            wo = g("wo", E)
            note("wo", _close(wo, mm(p + "attn_output.weight", att), f"{tag} Wo"))
            xmid = g("xmid", E)
            note("xmid", _close(xmid, x + o.rms_norm(wo, vec(p + "post_attention_norm.weight"), eps), f"{tag} residual"))
            F = hp["n_ff"][il]
            xf = o.rms_norm(xmid, vec(p + "ffn_norm.weight"), eps)
            gg, uu, hh = g("g", F), g("u", F), g("h", F)
            note("gate", _close(gg, mm(p + "ffn_gate.weight", xf), f"{tag} gate"))
            note("up", _close(uu, mm(p + "ffn_up.weight", xf), f"{tag} up"))
            note("h", _close(hh, o.gelu(gg) * uu, f"{tag} gelu(gate)*up"))
            down = g("down", E)
            note("down", _close(down, mm(p + "ffn_down.weight", hh), f"{tag} down"))
            xffn = g("xffn", E)
            note("xffn", _close(xffn, xmid + o.rms_norm(down, vec(p + "post_ffw_norm.weight"), eps), f"{tag} FFN residual"))
            plg, plh = g("plg", PE), g("plh", PE)
            note("plg", _close(plg, mm(p + "inp_gate.weight", xffn), f"{tag} inp_gate"))
            note("plh", _close(plh, o.gelu(plg) * tr[b, il * PE:(il + 1) * PE], f"{tag} per-layer injection"))
            proj = g("proj", E)
            note("proj", _close(proj, mm(p + "proj.weight", plh), f"{tag} proj"))
            sc = vec(p + "layer_output_scale.weight")
            xo = (xffn + o.rms_norm(proj, vec(p + "post_norm.weight"), eps)) * np.float32(sc[0] if sc is not None else 1.0)
            xn = tr[b, NPL + (il + 1) * rec:NPL + (il + 1) * rec + E] if il + 1 < NL else tr[b, NPL + NL * rec:]
            note("x'", _close(xn, xo, f"{tag} layer output"))
    # every position's head with the soft-cap (model.c:790-798), or the last
    # one's (model.c:766-775)
    for i, b in enumerate([nb - 1] if prefill else range(nb)):
        hnr = o.rms_norm(tr[b, NPL + NL * rec:], vec("output_norm.weight"), eps)
        if not prefill:
            note("hnext", _close(hn[b], hnr, f"token {b} head input"))
        lr = mm("token_embd.weight", hnr if prefill else hn[b])
        cap = hp.get("final_softcap", 0.0)
        if cap > 0:
            lr = (cap * np.tanh(lr.astype(np.float64) / cap)).astype(np.float32)
        note("logits", _close(lg[i], lr, f"token {b} logits"))
    return lg, hn, worst


def compare(tag, lg, olg, hn, ohn, bar=BAR):
    worst = 0.0
    for b in range(lg.shape[0]):
        rng = float(olg[b].max() - olg[b].min())
        err = float(np.abs(lg[b].astype(np.float64) - olg[b]).max())
        herr = float(np.abs(hn[b].astype(np.float64) - ohn[b]).max() / np.abs(ohn[b]).max())
        assert err <= bar * rng, f"{tag} row {b}: logits off by {err:.3g} (range {rng:.3g})"
        assert herr <= bar, f"{tag} row {b}: head input off by {herr:.3g}"
        top2 = np.sort(olg[b])[-2:]
        if top2[1] - top2[0] > 2 * err:
            assert int(np.argmax(lg[b])) == int(np.argmax(olg[b])), f"{tag} row {b}: greedy token differs"
        worst = max(worst, err / rng)
    return worst


def run_model(G, oracle, hp, T, path, kv_type, n_ctx, batches, steps, seed):
    """Prefill batches then greedy decode steps: every call traced and held part
    by part (traced_forward), and the whole stack against the oracle's own
    forward at the range-relative bar."""
    m = G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type)
    assert (m.n_vocab, m.n_embd, m.n_layer) == (hp["n_vocab"], hp["n_embd"], hp["n_layer"])
    om = oracle.Gemma(hp, T, kv_type, n_ctx)
    toks = np.random.default_rng(seed).integers(0, hp["n_vocab"], sum(batches))
    pos, worst = 0, {}
    oracle.pool_start(8)
    try:
        for nb in batches:
            lg, hn, w = traced_forward(G, oracle, hp, T, m, kv_type, toks[pos:pos + nb], pos, n_ctx)
            olg, ohn = om.forward(toks[pos:pos + nb], pos, nthreads=8)
            compare(f"prefill@{pos}", lg, olg, hn, ohn)
            worst.update({k: max(v, worst.get(k, 0.0)) for k, v in w.items()})
            pos += nb
        tok = int(np.argmax(olg[-1]))
        for step in range(steps):
            lg, hn, w = traced_forward(G, oracle, hp, T, m, kv_type, [tok], pos, n_ctx)
            olg, ohn = om.forward([tok], pos, nthreads=8)
            compare(f"decode@{pos}", lg, olg, hn, ohn)
            worst.update({k: max(v, worst.get(k, 0.0)) for k, v in w.items()})
            tok, pos = int(np.argmax(olg[0])), pos + 1
    finally:
        oracle.pool_stop()
        m.free()
    print(f"kv {kv_type}: worst per part " + ", ".join(f"{k} {v:.3g}" for k, v in worst.items()), flush=True)


@pytest.mark.parametrize("kv_type", [1, 8, 2], ids=["f16", "q8_0", "q4_0"])
def test_gguf_model_matches_oracle(gpu, oracle, tmp_path, kv_type):
    hp, T = GM.make_gemma(oracle, 11)
    path = tmp_path / "gemma.gguf"
    GM.write_gemma(path, hp, T)
    run_model(gpu, oracle, hp, T, path, kv_type, 64, (7, 13), 6, kv_type)      # prefill past the window of 8


@pytest.mark.parametrize("kv_type", [1, 8, 2], ids=["f16", "q8_0", "q4_0"])
def test_wide_heads_model_matches_oracle(gpu, oracle, tmp_path, kv_type):
    """The reference's head widths: full-attention layers of 8 heads x 512 over
    one KV head, sliding layers of 256 (g4run.h:283-292)."""
    hp, T = GM.make_gemma(oracle, 21, spec=GM.WIDE)
    path = tmp_path / "wide.gguf"
    GM.write_gemma(path, hp, T)
    run_model(gpu, oracle, hp, T, path, kv_type, 48, (13, 9), 4, kv_type + 40)   # prefill past the window of 16


@pytest.mark.parametrize("kv_type", [8, 1], ids=["q8_0", "f16"])
def test_ring_wrap_and_batch_equals_single_tokens(gpu, oracle, tmp_path, kv_type):
    """Positions past the 576-slot ring: prefill 600 tokens in batches of 64,
    then decode; the same run one token at a time gives the same bits."""
    G = gpu
    hp, T = GM.make_gemma(oracle, 12, spec=dict(GM.SMALL, n_swa=40))
    path = tmp_path / "gemma.gguf"
    GM.write_gemma(path, hp, T)
    n_ctx = 640
    a = G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type)
    om = oracle.Gemma(hp, T, kv_type, n_ctx)
    toks = np.random.default_rng(5).integers(0, hp["n_vocab"], 610)
    rows = []
    oracle.pool_start(8)
    try:
        for i in range(0, 600, 64):
            nb = min(64, 600 - i)
            if i == 576:                                 # past the ring's end: held part by part
                lg, hn, _ = traced_forward(G, oracle, hp, T, a, kv_type, toks[i:i + nb], i, n_ctx)
            else:
                lg, hn = a.forward(toks[i:i + nb], i)
            olg, ohn = om.forward(toks[i:i + nb], i, nthreads=8)
            compare(f"prefill@{i}", lg, olg, hn, ohn)
            rows.append(lg)
        for p in range(600, 610):
            lg, hn, _ = traced_forward(G, oracle, hp, T, a, kv_type, [toks[p]], p, n_ctx)
            olg, ohn = om.forward([toks[p]], p, nthreads=8)
            compare(f"decode@{p}", lg, olg, hn, ohn)
            rows.append(lg)
    finally:
        oracle.pool_stop()
    a.free()
    # the same 610 tokens one at a time on a fresh model: identical bits
    b = G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type)
    single = [b.forward([toks[p]], p)[0] for p in range(610)]
    b.free()
    assert np.concatenate(rows).tobytes() == np.concatenate(single).tobytes()


@pytest.mark.parametrize("kv_type", [8, 1], ids=["q8_0", "f16"])
@pytest.mark.parametrize("spec", ["SMALL", "WIDE"])
def test_prefill_on_matrix_cores_part_by_part(gpu, oracle, tmp_path, spec, kv_type):
    """g4h_gemma_prefill (g4_forward_batch, model.c:757-776): batches of 9 or
    more tokens run the q8_0 / q4_0 / q4_K / q6_K projections on the int8
    matrix cores.  Every part of every token is held against the oracle on the
    GPU's own inputs (the K/V rows stored bit for bit), the last logits
    against the oracle's forward, and decode steps then run on the caches the
    prefill wrote."""
    G = gpu
    hp, T = GM.make_gemma(oracle, 31, spec=getattr(GM, spec))
    path = tmp_path / "g.gguf"
    GM.write_gemma(path, hp, T)
    n_ctx = 96
    m = G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type)
    om = oracle.Gemma(hp, T, kv_type, n_ctx)
    toks = np.random.default_rng(17).integers(0, hp["n_vocab"], 64)
    pos = 0
    oracle.pool_start(8)
    try:
        for nb in (33, 9, 16):
            lg, _, _ = traced_forward(G, oracle, hp, T, m, kv_type, toks[pos:pos + nb], pos, n_ctx, prefill=True)
            olg, ohn = om.forward(toks[pos:pos + nb], pos, nthreads=8)
            compare(f"prefill@{pos}", lg, olg[-1:], ohn[-1:], ohn[-1:])
            pos += nb
        assert m.prefill(toks[pos:pos + 3], pos, want_logits=False) is None
        om.forward(toks[pos:pos + 3], pos, nthreads=8)
        pos += 3
        tok = int(toks[pos])
        for _ in range(3):
            lg, hn, _ = traced_forward(G, oracle, hp, T, m, kv_type, [tok], pos, n_ctx)
            olg, ohn = om.forward([tok], pos, nthreads=8)
            compare(f"decode@{pos}", lg, olg, hn, ohn)
            tok, pos = int(np.argmax(olg[0])), pos + 1
    finally:
        oracle.pool_stop()
        m.free()


@pytest.mark.parametrize("spec", ["SMALL", "WIDE"])
def test_prefill_shared_quantizer_same_bits(gpu, oracle, tmp_path, spec):
    """The q / k / v and gate / up projections of a prompt chunk that run
    k_mm_few share one quantizer launch of their xb rows; G4H_FEW_DIRECT=0
    quantizes in every call.  Both give the same logits bit for bit, at token
    counts of one, two (padded) and four tiles."""
    G = gpu
    hp, T = GM.make_gemma(oracle, 37, spec=getattr(GM, spec))
    path = tmp_path / "g.gguf"
    GM.write_gemma(path, hp, T)
    m = G.Gemma(path, n_ctx=160, kv_type=1)
    toks = np.random.default_rng(23).integers(0, hp["n_vocab"], 160)
    try:
        pos = 0
        for nb in (9, 40, 64):
            res = []
            for direct in ("1", "0"):
                print(f"{spec}: prefill of {nb} at {pos}, G4H_FEW_DIRECT={direct}", flush=True)
                os.environ["G4H_FEW_DIRECT"] = direct
                try:
                    res.append(m.prefill(toks[pos:pos + nb], pos).tobytes())
                finally:
                    del os.environ["G4H_FEW_DIRECT"]
            assert res[0] == res[1], f"prefill of {nb}: the shared quantizer changed the bits"
            pos += nb
    finally:
        m.free()


def test_model_file_errors(gpu, oracle, tmp_path):
    G = gpu
    hp, T = GM.make_gemma(oracle, 13)
    bad = dict(T)
    del bad["blk.2.ffn_up.weight"]
    p = tmp_path / "missing.gguf"
    GM.write_gemma(p, hp, bad)
    with pytest.raises(G.G4HError, match="missing tensor blk.2.ffn_up.weight"):
        G.Gemma(p, n_ctx=64)
    hp2, T2 = GM.make_gemma(oracle, 13, spec=dict(GM.SMALL, n_swa=600))
    p2 = tmp_path / "window.gguf"
    GM.write_gemma(p2, hp2, T2)
    with pytest.raises(G.G4HError, match="sliding window"):
        G.Gemma(p2, n_ctx=64)
    with pytest.raises(G.G4HError, match="cannot read"):
        G.Gemma(tmp_path / "nope.gguf", n_ctx=64)
    # the shared-KV layer 3 (sliding) would read layer 1's cache, a full layer's
    hp4, T4 = GM.make_gemma(oracle, 13, spec=dict(GM.SMALL, is_swa=[1, 0, 0, 1]))
    p4 = tmp_path / "shared.gguf"
    GM.write_gemma(p4, hp4, T4)
    with pytest.raises(G.G4HError, match="shared-KV layer 3"):
        G.Gemma(p4, n_ctx=64)
    m = G.Gemma(_ok(oracle, tmp_path), n_ctx=16)
    with pytest.raises(G.G4HError, match="positions outside"):
        m.forward([1, 2], 15)
    with pytest.raises(G.G4HError, match="out of range"):
        m.forward([hp["n_vocab"]], 0)


def test_attention_has_no_bounded_waits(gpu, oracle, tmp_path):
    """The gemma4 forward attends on the matrix cores (f16 cache, heads up to
    256) or with the three-pass kernels (512-wide heads, quantized caches):
    no launch waits on other workgroups, so the test hook that makes the
    one-launch kernels' waits give up changes nothing -- the forward returns
    G4H_OK and is held part by part against the oracle."""
    G = gpu
    for spec in ("SMALL", "WIDE"):
        hp, T = GM.make_gemma(oracle, 15, spec=getattr(GM, spec))
        path = tmp_path / f"t{spec}.gguf"
        GM.write_gemma(path, hp, T)
        m = G.Gemma(path, n_ctx=32, kv_type=G.F16)
        m.forward(np.arange(5), 0)
        oracle.pool_start(8)
        try:
            G.debug_attn_timeout(True)
            lg, _, _ = traced_forward(G, oracle, hp, T, m, G.F16, [7], 5, 32)
        finally:
            G.debug_attn_timeout(False)
            oracle.pool_stop()
        assert np.isfinite(lg).all()
        flags = m.status()
        assert not flags & G.STATUS_ATTN_TIMEOUT
        m.free()


@pytest.mark.parametrize("spec,kv_type", [("SMALL", 1), ("WIDE", 8), ("WIDE", 1)],
                         ids=["small-f16", "wide-q8_0", "wide-f16"])
def test_device_step_graph_equals_forward(gpu, oracle, tmp_path, spec, kv_type):
    """g4h_gemma_step (device token and position) captured once and replayed
    per token: every step's logits equal g4h_gemma_forward's on a second model
    fed the same tokens, bit for bit, the state advances to the greedy token,
    and the last position of the context is reported, not passed."""
    G = gpu
    hp, T = GM.make_gemma(oracle, 31, spec=getattr(GM, spec))
    path = tmp_path / "g.gguf"
    GM.write_gemma(path, hp, T)
    n_ctx = 40
    a, b = G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type), G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type)
    toks = np.random.default_rng(3).integers(0, hp["n_vocab"], 20)
    a.forward(toks, 0)
    b.forward(toks, 0)
    st = G.Stream()
    a.set_state(5, 20, st.ptr)
    a.step(st.ptr)                                      # outside the capture: workspaces set up
    st.synchronize()
    tok0 = int(toks[-1])
    a.set_state(tok0, 20, st.ptr)
    g = G.Graph(st.ptr, lambda: a.step(st.ptr))
    tok = tok0
    for pos in range(20, n_ctx):
        g.launch(st.ptr)
        st.synchronize()
        lg = a.logits()
        ref, _ = b.forward([tok], pos)
        assert lg.tobytes() == ref[0].tobytes(), f"pos {pos}: step logits differ from the forward"
        tok = int(np.argmax(ref[0]))
        t, p = a.get_state(st.ptr)
        assert t == tok and p == min(pos + 1, n_ctx - 1)
    assert a.status(st.ptr) == G.STATUS_CTX_FULL
    a.free()
    b.free()


def _ok(oracle, tmp_path):
    hp, T = GM.make_gemma(oracle, 14)
    p = tmp_path / "ok.gguf"
    GM.write_gemma(p, hp, T)
    return p
