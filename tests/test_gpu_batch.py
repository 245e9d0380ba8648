"""The batched forward (g4h_forward_batch, g4h_forward_batch_heads: the GPU
form of forward_layers for nb tokens, model.c:592-799) and the verify step of
speculative decoding built on it (main.c:383-404).

Bar, verify batch (g4h_forward_batch_heads): bit-exact.  Row b uses the
decode step's arithmetic, so its logits must equal those of decoding
tokens[0..b] one at a time; the verify step must accept exactly the drafted
prefix the greedy decode agrees with and return the greedy token after it.
The decode step itself is checked against the CPU oracle in
test_gpu_model.py; here the batch's head input feature is also checked
against the oracle's rms_norm of the decode step's final x.

Bar, prompt chunk (g4h_forward_batch) from 9 tokens, whose projections run on
the int8 matrix cores: every part of every layer of every row against the
oracle on the GPU's own inputs, per element 1e-3 relative / 1e-5 absolute (the
part-by-part method of test_gpu_model.check_layers), the K/V rows stored bit
for bit, and the last token's logits against the oracle's head.
"""
import os
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL = dict(n_layer=2, n_embd=256, n_head=4, n_kv=2, head_dim=64, n_ff=512, n_vocab=512, n_ctx=64,
             rope_base=1e6, rms_eps=1e-6)
MID = dict(n_layer=2, n_embd=2560, n_head=8, n_kv=4, head_dim=256, n_ff=10240, n_vocab=4096, n_ctx=1024,
           rope_base=1e6, rms_eps=1e-6)


def make_model(G, cfg, kv_type, wtype, seed=7):
    m = G.Model(seed=seed, kv_type=kv_type, wtype=wtype, **cfg)
    m.fill_kv(seed + 1)
    return m


@pytest.mark.parametrize("cfg,kv_type,wtype,nb,pos0", [
    (SMALL, 1, 2, 1, 20), (SMALL, 1, 2, 5, 20), (SMALL, 8, 2, 13, 40), (SMALL, 2, 8, 8, 3),
    (MID, 1, 2, 4, 900), (MID, 8, 2, 9, 1000), (MID, 1, 8, 24, 600)],
    ids=["small-f16-nb1", "small-f16-nb5", "small-q8kv-nb13", "small-q4kv-q8w-nb8", "mid-f16-nb4", "mid-q8kv-nb9",
         "mid-f16-q8w-nb24"])
def test_batch_rows_equal_decode_steps(gpu, oracle, cfg, kv_type, wtype, nb, pos0):
    G = gpu
    m = make_model(G, cfg, kv_type, wtype)
    V, E = cfg["n_vocab"], cfg["n_embd"]
    rs = np.random.default_rng(nb * 31 + pos0)
    tokens = rs.integers(0, V, nb).astype(np.int32)
    print(f"batch of {nb} at pos {pos0} ({cfg['n_embd']}d, kv {kv_type}, w {wtype})", flush=True)
    L, H = m.forward_batch_heads(tokens, pos0)
    G.synchronize()
    bl = L.download(np.float32, (nb, V))
    hn = H.download(np.float32, (nb, E))
    am = G.Buffer(4 * nb)
    G.argmax_rows(L, V, nb, am)
    G.synchronize()
    assert list(am.download(np.int32, nb)) == [int(np.argmax(r)) for r in bl]
    # the same tokens decoded one by one (the batch's K/V rows are rewritten
    # with the same values); the trace gives each step's final x
    trace = G.Buffer(m.trace_floats() * 4)
    m.trace(trace)
    out_norm = m.norm(0, "output_norm")
    fields, rec = m.trace_fields()
    try:
        for b in range(nb):
            m.forward(int(tokens[b]), pos0 + b)
            lg = m.logits()
            assert lg.tobytes() == bl[b].tobytes(), f"row {b}: batch logits differ from the decode step"
            xf = trace.download(np.float32, E, offset=cfg["n_layer"] * rec * 4)
            ref = oracle.rms_norm(xf, out_norm, cfg["rms_eps"])
            np.testing.assert_allclose(hn[b], ref, rtol=1e-6, atol=1e-6)
    finally:
        m.trace(None)
    # g4_forward_batch: the last token's logits; from 9 tokens its projections
    # and its attention run on the matrix cores (other fp32 orders, and fp16
    # softmax weights that may take the neighbouring code, a relative 5e-4 of
    # a weight): the stack agrees to 1e-2 of the logit range, each part of it
    # to 1e-3 / 1e-5 (test_prefill_rows_match_oracle_per_part)
    lg = m.forward_batch(tokens, pos0)
    if nb < 9:
        assert lg.tobytes() == bl[-1].tobytes()
    else:
        rng = float(bl[-1].max() - bl[-1].min())
        assert float(np.abs(lg.astype(np.float64) - bl[-1]).max()) <= 1e-2 * rng


@pytest.mark.parametrize("cfg,kv_type,wtype,nb,pos0", [
    (SMALL, 1, 2, 13, 30), (MID, 1, 2, 24, 600), (MID, 8, 8, 16, 900)],
    ids=["small-f16-q4w-nb13", "mid-f16-q4w-nb24", "mid-q8kv-q8w-nb16"])
def test_prefill_rows_match_oracle_per_part(gpu, oracle, cfg, kv_type, wtype, nb, pos0):
    """g4_forward_batch of a prompt chunk (projections on the int8 matrix
    cores; with an f16 cache the attention too): with the per-token trace,
    each part of each layer of every row is recomputed by the oracle from the
    GPU's own inputs to that part."""
    from test_gpu_model import _attn_slack, _cache_rows, _check_gelu, _close, oracle_model
    from oracle import g4o as o
    G = gpu
    m = make_model(G, cfg, kv_type, wtype)
    om = oracle_model(oracle, G, m)
    E, L, F, eps = cfg["n_embd"], cfg["n_layer"], cfg["n_ff"], cfg["rms_eps"]
    Q = cfg["n_head"] * cfg["head_dim"]
    rs = np.random.default_rng(nb * 7 + pos0)
    tokens = rs.integers(0, cfg["n_vocab"], nb).astype(np.int32)
    tf = m.trace_floats()
    fields, rec = m.trace_fields()
    off = {nm: (a, n) for nm, a, n in fields}
    tb = G.Buffer(nb * tf * 4)
    m.trace(tb)
    try:
        print(f"prefill chunk of {nb} at pos {pos0} ({E}d, kv {kv_type}, w {wtype})", flush=True)
        lg = m.forward_batch(tokens, pos0)
    finally:
        m.trace(None)
    tr = tb.download(np.float32, (nb, tf))
    nth = max(1, min(16, os.cpu_count() or 1))
    oracle.pool_start(nth)
    try:
        w = om.w
        mm = lambda W, x, ncols: o.matmul(wtype, W, o.prep_act(wtype, x[None]), ncols, nthreads=nth)[0]
        for b in range(nb):
            assert np.array_equal(tr[b, :E].view(np.uint32), om.embed(int(tokens[b])).view(np.uint32)), f"row {b}: embedding"
        for l in range(L):
            worst = {}
            for b in range(nb):
                pos = pos0 + b
                r = tr[b, l * rec:(l + 1) * rec]
                v = {nm: r[a:a + n] for nm, (a, n) in off.items()}
                what = f"layer {l} row {b}"
                e = {"qkv": _close(v["qkv"], om.qkv(l, v["x"], nthreads=nth), f"{what} projection")}
                att_ref, qprep = om.attn(l, pos, v["qkv"], nthreads=nth, prepared=True)
                slack = _attn_slack(o, om, l, pos, qprep) if kv_type == G.F16 else 0.0
                e["att"] = _close(v["att"], att_ref, f"{what} attention", slack)
                k_gpu, v_gpu = _cache_rows(G, m, l, pos)
                rb = k_gpu.size
                assert np.array_equal(k_gpu, om.kc[l][pos * rb:(pos + 1) * rb]), f"{what}: K row differs"
                assert np.array_equal(v_gpu, om.vc[l][pos * rb:(pos + 1) * rb]), f"{what}: V row differs"
                e["wo"] = _close(v["wo"], mm(w["wo"][l], v["att"], Q), f"{what} Wo")
                e["xmid"] = _close(v["xmid"], v["x"] + o.rms_norm(v["wo"], w["post_attn_norm"][l], eps), f"{what} residual")
                gu = mm(w["wgu"][l], o.rms_norm(v["xmid"], w["ffn_norm"][l], eps), E)
                e["h"], _ = _check_gelu(o, v["h"], gu[:F], gu[F:], f"{what} FFN")
                e["down"] = _close(v["down"], mm(w["wdown"][l], v["h"], F), f"{what} Wdown")
                if l + 1 < L or b == nb - 1:              # the chunk's final x: its last token's
                    xn = tr[b, (l + 1) * rec:(l + 1) * rec + E]
                    e["x'"] = _close(xn, v["xmid"] + o.rms_norm(v["down"], w["post_ffw_norm"][l], eps), f"{what} FFN residual")
                for k_, x_ in e.items():
                    worst[k_] = max(worst.get(k_, 0.0), x_)
            print(f"layer {l}: max err over {nb} rows " + ", ".join(f"{k_} {x_:.3g}" for k_, x_ in worst.items()), flush=True)
        otok, olg = om.head(tr[nb - 1, L * rec:L * rec + E], nthreads=nth)
        err = _close(lg, olg, "head")
        assert otok == int(np.argmax(lg))
        print(f"head: max err {err:.3g}, token {otok}", flush=True)
    finally:
        oracle.pool_stop()
        m.free()


@pytest.mark.parametrize("cfg,K", [(SMALL, 4), (MID, 6)], ids=["small-K4", "mid-K6"])
def test_verify_accepts_the_greedy_prefix(gpu, cfg, K):
    """main.c:383-404: the target runs [next_tok, drafts] at pos..pos+K; the
    accepted prefix is where its greedy choice equals the draft, and the bonus
    is its choice at the first mismatch."""
    G = gpu
    m = make_model(G, cfg, 1, 2, seed=3)
    V = cfg["n_vocab"]
    pos = cfg["n_ctx"] - K - 8
    tok0 = 17
    greedy, t = [], tok0
    for i in range(K + 1):                     # the plain greedy continuation
        t = m.forward(t, pos + i)
        greedy.append(t)
    am = G.Buffer(4 * (K + 1))
    for j in range(K + 1):                     # drafts correct up to j
        draft = [greedy[i] if i < j else (greedy[i] + 1) % V for i in range(K)]
        L, _ = m.forward_batch_heads([tok0] + draft, pos)
        G.argmax_rows(L, V, K + 1, am)
        G.synchronize()
        a = list(am.download(np.int32, K + 1))
        n_acc = 0
        while n_acc < K and a[n_acc] == draft[n_acc]:
            n_acc += 1
        assert n_acc == min(j, K), f"j={j}: accepted {n_acc}"
        assert a[n_acc] == greedy[n_acc], f"j={j}: bonus {a[n_acc]} vs greedy {greedy[n_acc]}"


def test_prompt_chunk_activation_layout_same_bits(gpu):
    """A prompt chunk's producers write k_mm_few's operand layout themselves
    (the norm, attention and GELU kernels); G4H_FEW_DIRECT=0 keeps GGUF rows
    re-laid per projection.  Both must give every traced part of every row
    and the logits bit for bit, across token counts that change the tile
    count and its padding (40 tokens: three tiles, 8 padding tokens; 64: four
    full tiles; 13: one padded tile) in one model, so each count's padding is
    cleared after the last."""
    G = gpu
    for cfg, wtype, counts in ((SMALL, 2, (13, 40, 13)), (MID, 8, (40, 64, 40)), (MID, 2, (64, 24))):
        m = make_model(G, cfg, 1, wtype)
        tb = G.Buffer(64 * m.trace_floats() * 4)
        m.trace(tb)
        try:
            for i, nb in enumerate(counts):
                tokens = np.random.default_rng(100 + i).integers(0, cfg["n_vocab"], nb).astype(np.int32)
                pos0 = min(cfg["n_ctx"] // 2, cfg["n_ctx"] - nb)
                res = []
                for direct in ("1", "0", "1"):
                    print(f"{cfg['n_embd']}d w {wtype}: chunk of {nb}, G4H_FEW_DIRECT={direct}", flush=True)
                    os.environ["G4H_FEW_DIRECT"] = direct
                    try:
                        lg = m.forward_batch(tokens, pos0)
                    finally:
                        del os.environ["G4H_FEW_DIRECT"]
                    res.append((lg.tobytes(), tb.download(np.float32, nb * m.trace_floats()).tobytes()))
                assert res[0] == res[1] == res[2], f"chunk of {nb}: the producer-written layout changed the bits"
        finally:
            m.trace(None)
            m.free()


def test_batch_argument_errors(gpu):
    G = gpu
    m = make_model(G, SMALL, 1, 2)
    with pytest.raises(G.G4HError):
        m.forward_batch(list(range(65)), 0)                 # more than G4_BATCH_MAX
    with pytest.raises(G.G4HError):
        m.forward_batch([1, 2, 3], SMALL["n_ctx"] - 2)       # runs past the context
    with pytest.raises(G.G4HError):
        m.forward_batch([1, SMALL["n_vocab"]], 0)            # token out of range
