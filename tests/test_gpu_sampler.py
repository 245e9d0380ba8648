"""The device sampler (g4h_sample, the GPU form of sampler.c:74-210) against
the CPU oracle's restated chain (itself pinned bit for bit to the reference's
sampler.c build, tests/test_oracle_sampler.py).

Bar: bit-exact -- the drawn id, every logit the call rewrites (bans, n-gram
hits, penalties), the RNG words and the ring of accepted ids, at every step of
seeded runs.  Covers the config vocabulary (32768), a gemma-size vocabulary
(262144, beyond the register-free 4096-candidate gather), tiny vocabularies
(k >= n_vocab), ties and NaNs (the exact heap replay), -inf-dominated rows,
ring wrap-around, graph replay and the decode step drawing with a sampler.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def run_pair(G, oracle, nv, params, rs, kind, steps, bans=(), hist=(), stream=None):
    """Draw `steps` times on the GPU and with the oracle from identical
    settings, history and logits; compare everything after each draw."""
    gs = G.Sampler(nv, **params)
    os_ = oracle.Sampler(nv, **params)
    for b in bans:
        gs.ban(int(b))
        os_.ban(int(b))
    if len(hist):
        gs.accept(np.asarray(hist, np.int32))
        for t in hist:
            os_.accept(int(t))
    buf = G.Buffer(nv * 4)
    out = G.Buffer(4)
    slow0 = gs.state()[2]
    for step in range(steps):
        lg = make_logits(rs, nv, kind)
        buf.upload(lg)
        gs.sample(buf, out, accept=True)
        G.synchronize()
        gid = int(out.download(np.int32, 1)[0])
        glg = buf.download(np.float32, nv)
        ol = lg.copy()
        oid = os_.sample(ol)
        os_.accept(oid)
        rng, ring, slow = gs.state()
        ctx = f"nv {nv} kind {kind} step {step} params {params}"
        assert gid == oid, f"{ctx}: gpu {gid} oracle {oid}"
        assert glg.tobytes() == ol.tobytes(), f"{ctx}: rewritten logits differ"
        assert rng == os_.rng, ctx
        assert ring == os_.recent(), ctx
    return gs.state()[2] - slow0


def make_logits(rs, nv, kind):
    lg = (rs.standard_normal(nv) * 3).astype(np.float32)
    if kind == "ties":
        lg = (np.round(lg * 2) / 2).astype(np.float32)
    elif kind == "nan":
        lg[rs.integers(0, nv, 2)] = np.nan
    elif kind == "inf":
        lg[rs.random(nv) < 0.95] = -np.inf
    elif kind == "flat":                      # > 4096 values within one boundary key
        lg = np.full(nv, 1.0, np.float32)
        lg[rs.integers(0, nv, 30)] = 2.0 + rs.random(30).astype(np.float32)
    return lg


BASE = dict(temp=0.8, top_k=40, top_p=0.95, repeat_penalty=1.1, repeat_last_n=64, freq_penalty=0.05,
            presence_penalty=0.1, no_repeat_ngram=3, seed=1234)


@pytest.mark.parametrize("nv", [32768, 262144])
def test_default_chain_matches_oracle(gpu, oracle, nv):
    rs = np.random.default_rng(nv)
    hist = rs.integers(0, 50, 200)
    slow = run_pair(gpu, oracle, nv, BASE, rs, "plain", 12, bans=[3, 7, nv - 1], hist=hist)
    assert slow == 0                          # distinct values: the sort-based path


@pytest.mark.parametrize("kind", ["ties", "nan", "inf", "flat"])
def test_exact_heap_replay_matches_oracle(gpu, oracle, kind):
    rs = np.random.default_rng(5)
    nv = 32768
    p = dict(BASE, top_k=64)
    slow = run_pair(gpu, oracle, nv, p, rs, kind, 4, hist=rs.integers(0, nv, 40))
    if kind in ("ties", "nan", "flat"):
        assert slow > 0


@pytest.mark.parametrize("top_k,top_p,temp", [(0, 0.95, 1.0), (1, 0.5, 2.0), (511, 1.0, 0.7), (512, 0.3, 1.3),
                                              (2000, 0.0, 1.0), (64, 0.95, 0.0)])
def test_settings_match_oracle(gpu, oracle, top_k, top_p, temp):
    rs = np.random.default_rng(top_k + 7)
    p = dict(BASE, top_k=top_k, top_p=top_p, temp=temp)
    run_pair(gpu, oracle, 32768, p, rs, "plain", 6, hist=rs.integers(0, 32768, 100))


@pytest.mark.parametrize("nv", [1, 5, 100, 4096, 5000])
def test_small_vocabularies(gpu, oracle, nv):
    rs = np.random.default_rng(nv)
    p = dict(BASE, top_k=512, top_p=1.0, no_repeat_ngram=2)
    run_pair(gpu, oracle, nv, p, rs, "plain", 8, hist=rs.integers(0, nv, 30))


def test_ring_wraps_and_penalty_window(gpu, oracle):
    rs = np.random.default_rng(9)
    nv = 1000
    p = dict(BASE, repeat_last_n=5000, repeat_penalty=1.3, freq_penalty=0.2, no_repeat_ngram=4)
    hist = rs.integers(0, 20, 4500)           # wraps the 4096-id ring
    run_pair(gpu, oracle, nv, p, rs, "plain", 6, hist=hist)


def test_reset_keeps_bans_and_rng(gpu, oracle):
    G = gpu
    nv = 300
    rs = np.random.default_rng(1)
    gs, os_ = G.Sampler(nv, **BASE), oracle.Sampler(nv, **BASE)
    for t in (5, 6):
        gs.ban(t)
        os_.ban(t)
    buf, out = G.Buffer(nv * 4), G.Buffer(4)
    for step in range(6):
        if step == 3:
            gs.reset()
            os_.reset()
        lg = make_logits(rs, nv, "plain")
        buf.upload(lg)
        gs.sample(buf, out, accept=True)
        G.synchronize()
        oid = os_.sample(lg)
        os_.accept(oid)
        assert int(out.download(np.int32, 1)[0]) == oid
        rng, ring, _ = gs.state()
        assert rng == os_.rng and ring == os_.recent()


def test_graph_replays_draw_like_the_oracle(gpu, oracle):
    """A captured g4h_sample replays with the device state (RNG, ring) moving on."""
    G = gpu
    nv = 32768
    rs = np.random.default_rng(2)
    gs, os_ = G.Sampler(nv, **BASE), oracle.Sampler(nv, **BASE)
    buf, out = G.Buffer(nv * 4), G.Buffer(4)
    st = G.Stream()
    graph = G.Graph(st.ptr, lambda: gs.sample(buf, out, accept=True, stream=st.ptr))
    for rep in range(5):
        lg = make_logits(rs, nv, "plain")
        buf.upload(lg)
        graph.launch(st.ptr)
        st.synchronize()
        oid = os_.sample(lg)
        os_.accept(oid)
        assert int(out.download(np.int32, 1)[0]) == oid, f"replay {rep}"
        rng, ring, _ = gs.state()
        assert rng == os_.rng and ring == os_.recent(), f"replay {rep}"


def test_decode_step_draws_with_the_sampler(gpu, oracle):
    """The model's step with a sampler: its token and rewritten logits equal the
    oracle's draw from the logits the same step produces greedily."""
    G = gpu
    cfg = dict(n_layer=2, n_embd=256, n_head=4, n_kv=2, head_dim=64, n_ff=512, n_vocab=512, n_ctx=64,
               rope_base=1e6, rms_eps=1e-6)
    m = G.Model(seed=3, **cfg)
    m.fill_kv(4)
    p = dict(BASE, top_k=20, temp=1.2)
    gs, os_ = G.Sampler(cfg["n_vocab"], **p), oracle.Sampler(cfg["n_vocab"], **p)
    tok, pos = 11, 30
    for step in range(4):
        m.set_sampler(None)
        m.set_state(tok, pos)
        m.forward_state()
        G.synchronize()
        lg = m.logits()                           # the step's logits, untouched by a greedy step
        m.set_sampler(gs)
        m.set_state(tok, pos)
        m.forward_state()
        G.synchronize()
        t_gpu, p_gpu = m.get_state()
        oid = os_.sample(lg)
        os_.accept(oid)
        assert t_gpu == oid and p_gpu == pos + 1, f"step {step}"
        assert m.logits().tobytes() == lg.tobytes()
        assert gs.state()[1] == os_.recent()
        tok, pos = oid, pos + 1
    m.set_sampler(None)


def test_sampler_argument_errors(gpu):
    G = gpu
    s = G.Sampler(100)
    with pytest.raises(G.G4HError):
        s.accept([100])                         # id out of range
    m = G.Model(seed=1, n_layer=1, n_embd=256, n_head=4, n_kv=2, head_dim=64, n_ff=512, n_vocab=512, n_ctx=64,
                rope_base=1e6, rms_eps=1e-6)
    with pytest.raises(G.G4HError):
        m.set_sampler(s)                        # vocabulary differs
