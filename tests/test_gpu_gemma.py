"""A gemma4 model loaded from a GGUF file the test writes (g4h_gemma_open: the
GPU form of g4_gguf_open + g4_ctx_init + forward_layers/heads) against the
oracle's gemma4 forward on the same tensors (tests/test_oracle_gemma.py pins
that forward).

Bars.  The oracle and the GPU compute the same arithmetic up to the fp32
order of the attention's score (f16 cache) and value sums, so runs agree to
~1e-7 of the logit range -- asserted (1e-5) for the first prefill batch --
until, now and then, a last-bit difference lands on a rounding edge (an fp16
query or softmax weight, a q8_0 activation code) and makes a visible step,
which later positions keep through the cache.  That is the whole-stack chaos
of test_gpu_model.py; the attention itself is held per element to 1e-3/1e-5
in test_gpu_attn.py, windows and ring included.  So every position is held
to 5e-2 of the range (measured: up to ~1e-2 after such a step), its greedy
token to the oracle's wherever the top-two gap exceeds twice the row's
difference, and a batch to one token at a time bit for bit."""
import numpy as np
import pytest

import gemma_util as GM

pytestmark = pytest.mark.gpu


BAR = 5e-2


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


@pytest.mark.parametrize("kv_type", [1, 8, 2], ids=["f16", "q8_0", "q4_0"])
def test_gguf_model_matches_oracle(gpu, oracle, tmp_path, kv_type):
    G = gpu
    hp, T = GM.make_gemma(oracle, 11)
    path = tmp_path / "gemma.gguf"
    GM.write_gemma(path, hp, T)
    n_ctx = 64
    m = G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type)
    assert (m.n_vocab, m.n_embd, m.n_layer) == (hp["n_vocab"], hp["n_embd"], hp["n_layer"])
    om = oracle.Gemma(hp, T, kv_type, n_ctx)
    rs = np.random.default_rng(kv_type)
    toks = rs.integers(0, hp["n_vocab"], 20)
    pos = 0
    for nb in (7, 13):                                   # prefill past the window of 8
        lg, hn = m.forward(toks[pos:pos + nb], pos)
        olg, ohn = om.forward(toks[pos:pos + nb], pos, nthreads=8)
        compare(f"prefill@{pos}", lg, olg, hn, ohn, 1e-5 if pos == 0 else BAR)
        pos += nb
    tok = int(np.argmax(olg[-1]))
    for step in range(6):                                # decode steps
        lg, hn = m.forward([tok], pos)
        olg, ohn = om.forward([tok], pos, nthreads=8)
        e = compare(f"decode@{pos}", lg, olg, hn, ohn)
        print(f"kv {kv_type} pos {pos}: max logit diff {e:.3g}", flush=True)
        tok, pos = int(np.argmax(olg[0])), pos + 1
    m.free()


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
    for i in range(0, 600, 64):
        nb = min(64, 600 - i)
        lg, hn = a.forward(toks[i:i + nb], i)
        olg, ohn = om.forward(toks[i:i + nb], i, nthreads=8)
        compare(f"prefill@{i}", lg, olg, hn, ohn)
        rows.append(lg)
    for p in range(600, 610):
        lg, hn = a.forward([toks[p]], p)
        olg, ohn = om.forward([toks[p]], p, nthreads=8)
        compare(f"decode@{p}", lg, olg, hn, ohn)
        rows.append(lg)
    a.free()
    # the same 610 tokens one at a time on a fresh model: identical bits
    b = G.Gemma(path, n_ctx=n_ctx, kv_type=kv_type)
    single = [b.forward([toks[p]], p)[0] for p in range(610)]
    b.free()
    assert np.concatenate(rows).tobytes() == np.concatenate(single).tobytes()


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
    m = G.Gemma(_ok(oracle, tmp_path), n_ctx=16)
    with pytest.raises(G.G4HError, match="positions outside"):
        m.forward([1, 2], 15)
    with pytest.raises(G.G4HError, match="out of range"):
        m.forward([hp["n_vocab"]], 0)


def _ok(oracle, tmp_path):
    hp, T = GM.make_gemma(oracle, 14)
    p = tmp_path / "ok.gguf"
    GM.write_gemma(p, hp, T)
    return p
