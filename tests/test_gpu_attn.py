"""Decode attention (attn_kernel, model.c:509-580) and kv_store on the GPU
against the CPU oracle.  KV stores are bit-exact; the attention output is
within |gpu-cpu| <= 1e-5 + 1e-3|cpu|.  The fp32 order of the f16 score sums,
the grouping of the double softmax normaliser and the fp32 order of the final
V accumulation differ from the CPU's loops; the fp16 rounding of q and of the
weights is the reference's."""
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


@pytest.mark.parametrize("kv_type", [1, 8, 2], ids=["f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("n_head,n_kv,hd,n_pos,qscale", [
    (8, 4, 256, 1, 1.0), (8, 4, 256, 65, 1.0), (8, 4, 256, 1000, 1.0), (8, 4, 256, 8192, 1.0),
    (8, 4, 256, 3000, 0.02), (4, 4, 128, 300, 0.1), (8, 1, 64, 777, 0.3), (16, 2, 192, 129, 1.0),
    # gemma4's full-attention heads: 8 query heads of 512 over one KV head (g4run.h:283-292)
    (8, 1, 512, 1, 1.0), (8, 1, 512, 777, 0.3), (8, 1, 512, 4096, 0.2), (2, 1, 512, 130, 1.0),
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


@pytest.mark.parametrize("kv_type", [1, 8], ids=["f16", "q8_0"])
def test_wide_heads_identical_keys_and_halves(gpu, oracle, kv_type):
    """512-wide heads run as two halves whose partial scores are joined: with
    all keys equal every weight is fp16(1/n) (f16 V) or 1/n, so the output is
    the mean of V (closed form); and keys whose second half is zero give the
    scores of the first half alone, i.e. the 256-wide attention of the first
    halves, element for element in the first half of the output."""
    G = gpu
    n_head, n_kv, hd, n_pos = 4, 1, 512, 300
    rng = np.random.default_rng(17)
    k = np.tile(rng.standard_normal(hd).astype(np.float32), (n_pos, 1))
    v = rng.standard_normal((n_pos, hd)).astype(np.float32)
    rb = hd * 2 if kv_type == G.F16 else G.row_size(kv_type, hd)
    kb, vb = G.Buffer(n_pos * rb), G.Buffer(n_pos * rb)
    G.kv_store(kv_type, G.Buffer.from_array(k), kb, hd, rows=n_pos, dst_stride=rb)
    G.kv_store(kv_type, G.Buffer.from_array(v), vb, hd, rows=n_pos, dst_stride=rb)
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    out = G.Buffer(n_head * hd * 4)
    G.attn_decode(G.Buffer.from_array(q), kb, vb, kv_type, n_head, n_kv, hd, n_pos, out)
    got = out.download(np.float32, (n_head, hd))
    vh = vb.download(np.uint8, (n_pos, rb))
    if kv_type == G.F16:
        w = np.float64(np.float16(np.float32(1.0 / n_pos)))
        vf = oracle.fp16_to_fp32(vh.view(np.uint16).reshape(n_pos, hd)).astype(np.float64)
    else:
        w = np.float64(np.float32(1.0 / n_pos))
        vf = oracle.dequant(kv_type, vh, hd).astype(np.float64)
    assert np.allclose(got, (w * vf).sum(0)[None, :], rtol=1e-5, atol=1e-6)
    # second halves of K zero: the first output half equals the 256-wide attention of the first halves
    k2 = rng.standard_normal((n_pos, hd)).astype(np.float32)
    k2[:, 256:] = 0.0
    kb2 = G.Buffer(n_pos * rb)
    G.kv_store(kv_type, G.Buffer.from_array(k2), kb2, hd, rows=n_pos, dst_stride=rb)
    G.attn_decode(G.Buffer.from_array(q), kb2, vb, kv_type, n_head, n_kv, hd, n_pos, out)
    wide = out.download(np.float32, (n_head, hd))
    half_k, half_v = G.Buffer(n_pos * rb // 2), G.Buffer(n_pos * rb // 2)
    G.kv_store(kv_type, G.Buffer.from_array(np.ascontiguousarray(k2[:, :256])), half_k, 256, rows=n_pos, dst_stride=rb // 2)
    G.kv_store(kv_type, G.Buffer.from_array(np.ascontiguousarray(v[:, :256])), half_v, 256, rows=n_pos, dst_stride=rb // 2)
    o256 = G.Buffer(n_head * 256 * 4)
    G.attn_decode(G.Buffer.from_array(np.ascontiguousarray(q[:, :256])), half_k, half_v, kv_type, n_head, n_kv, 256, n_pos, o256)
    narrow = o256.download(np.float32, (n_head, 256))
    assert np.array_equal(wide[:, :256].view(np.uint32), narrow.view(np.uint32))


def test_attention_bad_shapes(gpu):
    import ctypes as C
    G = gpu
    L = G.lib()
    b = G.Buffer(1 << 16)
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.Q4_K, 8, 4, 256, 10, b.ptr, b.ptr, b.nbytes, None) == G.ERR_TYPE
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.F16, 8, 3, 256, 10, b.ptr, b.ptr, b.nbytes, None) == G.ERR_SHAPE
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.F16, 8, 4, 96, 10, b.ptr, b.ptr, b.nbytes, None) == G.ERR_SHAPE
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.F16, 8, 2, 512, 10, b.ptr, b.ptr, b.nbytes, None) == G.ERR_SHAPE   # one KV head
    assert L.g4h_attn_decode(b.ptr, b.ptr, b.ptr, G.F16, 8, 4, 256, 10, b.ptr, b.ptr, 16, None) == G.ERR_ARG


def _attn(G, q, kb, vb, kv_type, n_head, n_kv, hd, n_pos, ws):
    out = G.Buffer(n_head * hd * 4)
    G.attn_decode(G.Buffer.from_array(q), kb, vb, kv_type, n_head, n_kv, hd, n_pos, out, ws=ws)
    G.synchronize()
    return out.download(np.float32, (n_head, hd))


@pytest.mark.parametrize("n_head,n_kv,hd,n_pos", [
    (8, 4, 256, 1), (8, 4, 256, 127), (8, 4, 256, 128), (8, 4, 256, 129), (8, 4, 256, 8192),
    (4, 4, 64, 700), (8, 1, 128, 5000), (16, 2, 192, 333), (32, 4, 256, 2049), (8, 4, 256, 12000),
    (4, 4, 64, 16384),
])
def test_attention_fused_equals_three_passes(gpu, oracle, monkeypatch, n_head, n_kv, hd, n_pos):
    """The one-launch form (tagged hand-off words between workgroups) gives the
    bits of the three-pass form; run twice on one workspace, then on a shorter
    context, so stale words of an earlier launch are seen to be ignored."""
    G = gpu
    assert G.attn_passes(G.F16, n_head, n_kv, hd, n_pos) == 1
    kb, vb, kh, vh = make_cache(G, oracle, G.F16, n_pos, n_kv, hd, seed=3 * n_pos + hd)
    q = (np.random.default_rng(n_pos).standard_normal((n_head, hd)) * 0.5).astype(np.float32)
    ws = G.Buffer(G.attn_workspace_bytes(n_head, hd, n_pos))
    fused = [_attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n, ws) for n in (n_pos, n_pos, max(1, n_pos // 3))]
    monkeypatch.setenv("G4H_ATTN_PASSES", "3")
    assert G.attn_passes(G.F16, n_head, n_kv, hd, n_pos) == 3
    three = [_attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n, ws) for n in (n_pos, max(1, n_pos // 3))]
    assert np.isfinite(fused[0]).all()
    assert np.array_equal(fused[0].view(np.uint32), three[0].view(np.uint32))
    assert np.array_equal(fused[1].view(np.uint32), three[0].view(np.uint32))
    assert np.array_equal(fused[2].view(np.uint32), three[1].view(np.uint32))
    ref = oracle.attn_decode(q, kh, vh, G.F16, n_head, n_kv, hd, n_pos - 1)
    assert (np.abs(fused[0] - ref) <= ATOL + RTOL * np.abs(ref)).all()


def test_attention_epoch_advances_on_device(gpu, oracle, monkeypatch):
    """The one-launch form tags its hand-off words with a workspace epoch word
    that every launch advances on the device, so a workspace is cleared on its
    first use only: back-to-back calls on a workspace that starts as garbage,
    graph replays with new queries between them and eager calls between the
    replays all give the three-pass bits."""
    G = gpu
    n_head, n_kv, hd, n_pos = 8, 4, 256, 4100
    assert G.attn_passes(G.F16, n_head, n_kv, hd, n_pos) == 1
    kb, vb, kh, vh = make_cache(G, oracle, G.F16, n_pos, n_kv, hd, seed=91)
    rng = np.random.default_rng(92)
    qs = [(rng.standard_normal((n_head, hd)) * 0.5).astype(np.float32) for _ in range(9)]
    monkeypatch.setenv("G4H_ATTN_PASSES", "3")
    ref = [_attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n_pos, None) for q in qs]
    monkeypatch.delenv("G4H_ATTN_PASSES")
    ws = G.Buffer(G.attn_workspace_bytes(n_head, hd, n_pos))
    ws.upload(np.full(ws.nbytes, 0xA5, np.uint8))                  # not a cleared workspace
    for i in range(4):
        got = _attn(G, qs[i], kb, vb, G.F16, n_head, n_kv, hd, n_pos, ws)
        assert np.array_equal(got.view(np.uint32), ref[i].view(np.uint32)), f"call {i}"
    st = G.Stream()
    qb = [G.Buffer(n_head * hd * 4) for _ in range(3)]
    outs = [G.Buffer(n_head * hd * 4) for _ in range(3)]
    for j in range(3):
        qb[j].upload(qs[j])
    g = G.Graph(st.ptr, lambda: [G.attn_decode(qb[j], kb, vb, G.F16, n_head, n_kv, hd, n_pos, outs[j], ws=ws,
                                               stream=st.ptr) for j in range(3)])
    for r in range(3):
        sel = [(3 * r + j + 1) % 9 for j in range(3)]
        for j in range(3):
            qb[j].upload(qs[sel[j]])
        g.launch(st.ptr)
        st.synchronize()
        for j in range(3):
            got = outs[j].download(np.float32, (n_head, hd))
            assert np.array_equal(got.view(np.uint32), ref[sel[j]].view(np.uint32)), f"replay {r} call {j}"
        got = _attn(G, qs[8 - r], kb, vb, G.F16, n_head, n_kv, hd, n_pos, ws)   # an eager call between replays
        assert np.array_equal(got.view(np.uint32), ref[8 - r].view(np.uint32)), f"eager after replay {r}"
    assert not G.attn_status(ws)
    o = oracle.attn_decode(qs[0], kh, vh, G.F16, n_head, n_kv, hd, n_pos - 1)
    assert (np.abs(ref[0] - o) <= ATOL + RTOL * np.abs(o)).all()
    # a decode loop's growing position count changes the workspace layout
    # every call (stale words of other layouts lie everywhere), and a
    # three-pass call writes untagged data into the same workspace
    for n in (n_pos - 300, n_pos - 299, n_pos - 171, 129, 128, 1, n_pos):
        q = qs[n % 9]
        monkeypatch.setenv("G4H_ATTN_PASSES", "3")
        three = _attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n, ws if n == 129 else None)
        monkeypatch.delenv("G4H_ATTN_PASSES")
        got = _attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n, ws)
        assert np.array_equal(got.view(np.uint32), three.view(np.uint32)), f"n_pos {n}"
    assert not G.attn_status(ws)


def test_attention_workspace_reuse_after_free_and_batch(gpu, oracle, monkeypatch):
    """A workspace freed with g4h_free and memory handed out again at the same
    address starts over (cleared on its next use), and a batch call that
    writes its untagged blocks into a workspace makes the next one-launch call
    clear it: both give the three-pass bits."""
    G = gpu
    n_head, n_kv, hd, n_pos = 8, 4, 256, 2000
    kb, vb, kh, vh = make_cache(G, oracle, G.F16, n_pos + 8, n_kv, hd, seed=93)
    q = (np.random.default_rng(94).standard_normal((n_head, hd)) * 0.5).astype(np.float32)
    monkeypatch.setenv("G4H_ATTN_PASSES", "3")
    ref = _attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n_pos, None)
    monkeypatch.delenv("G4H_ATTN_PASSES")
    nbytes = max(G.attn_workspace_bytes(n_head, hd, n_pos + 8), G.attn_prefill_workspace_bytes(n_head, hd, n_pos, 8))
    ws = G.Buffer(nbytes)
    for _ in range(2):
        assert np.array_equal(_attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n_pos, ws).view(np.uint32), ref.view(np.uint32))
    addr = ws.ptr
    ws.free()
    ws2 = G.Buffer(nbytes)
    ws2.upload(np.full(nbytes, 0xFF, np.uint8))                     # garbage, maybe at the same address
    got = _attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n_pos, ws2)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"reused at the same address: {ws2.ptr == addr}"
    qb = G.Buffer.from_array(np.tile(q, (8, 1, 1)))
    out = G.Buffer(8 * n_head * hd * 4)
    G.attn_prefill(qb, kb, vb, G.F16, n_head, n_kv, hd, n_pos - 1, 8, out, ws=ws2)     # untagged blocks
    got = _attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n_pos, ws2)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert not G.attn_status(ws2)


def test_attention_long_context_falls_back_to_three_passes(gpu, oracle):
    """A grid larger than the device holds at once runs the three passes."""
    G = gpu
    n_head, n_kv, hd, n_pos = 8, 8, 64, 40000                       # 8 x 313 workgroups
    assert G.attn_passes(G.F16, n_head, n_kv, hd, n_pos) == 3
    assert G.attn_passes(G.Q8_0, 8, 4, 256, 256) == 3                    # q8_0 caches always do
    kb, vb, kh, vh = make_cache(G, oracle, G.F16, n_pos, n_kv, hd, seed=11)
    q = np.random.default_rng(12).standard_normal((n_head, hd)).astype(np.float32)
    got = _attn(G, q, kb, vb, G.F16, n_head, n_kv, hd, n_pos, None)
    ref = oracle.attn_decode(q, kh, vh, G.F16, n_head, n_kv, hd, n_pos - 1)
    assert (np.abs(got - ref) <= ATOL + RTOL * np.abs(ref)).all()


@pytest.mark.parametrize("kv_type", [1, 8, 2], ids=["f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("pos0,nb", [(0, 9), (300, 7), (4090, 6)])
def test_batched_prefill_attention_is_causal(gpu, oracle, kv_type, pos0, nb):
    """attn_kernel with nb > 1 (model.c:509-545): token b at pos0 + b attends
    exactly the positions up to its own, the batch's rows already cached."""
    G = gpu
    n_head, n_kv, hd = 8, 4, 256
    n_slot = pos0 + nb
    kb, vb, kh, vh = make_cache(G, oracle, kv_type, n_slot, n_kv, hd, seed=n_slot)
    q = (np.random.default_rng(nb).standard_normal((nb, n_head, hd)) * 0.5).astype(np.float32)
    out = G.Buffer(nb * n_head * hd * 4)
    G.attn_prefill(G.Buffer.from_array(q), kb, vb, kv_type, n_head, n_kv, hd, pos0, nb, out)
    got = out.download(np.float32, (nb, n_head, hd))
    for b in range(nb):
        ref = oracle.attn_decode(q[b], kh, vh, kv_type, n_head, n_kv, hd, pos0 + b)
        err = np.abs(got[b].astype(np.float64) - ref)
        assert not (err > ATOL + RTOL * np.abs(ref)).any(), f"token {b}: worst {err.max():.3g}"
    # the first token sees only its own position when pos0 = 0: output = its V row
    if pos0 == 0 and kv_type == 1:
        v0 = oracle.fp16_to_fp32(vh[:n_kv].view(np.uint16).reshape(n_kv, hd))
        assert np.allclose(got[0], np.repeat(v0, n_head // n_kv, axis=0), rtol=0, atol=0)


@pytest.mark.parametrize("kv_type,n_head,n_kv,hd,pos0,nb", [
    (1, 8, 4, 256, 120, 20), (8, 8, 4, 256, 250, 11), (2, 8, 4, 256, 0, 5),
    (1, 4, 4, 64, 1000, 33), (8, 8, 1, 128, 127, 2), (2, 16, 2, 192, 383, 3), (1, 2, 2, 64, 0, 1),
    (1, 8, 1, 512, 120, 20), (8, 8, 1, 512, 255, 4), (2, 4, 1, 512, 0, 9)])
def test_batched_prefill_equals_per_token_calls(gpu, oracle, kv_type, n_head, n_kv, hd, pos0, nb):
    """The one-set batch (three launches, a token grid dimension, a workspace
    block per token) gives every token the bits of a decode call at its
    position -- the per-token launches of the smaller-workspace form and a
    direct g4h_attn_decode -- across chunk boundaries (positions 127/128,
    255/256, 383/384), group sizes 1 to 8 and head sizes 64 to 256."""
    G = gpu
    n_slot = pos0 + nb
    kb, vb, kh, vh = make_cache(G, oracle, kv_type, n_slot, n_kv, hd, seed=n_slot + hd)
    q = (np.random.default_rng(nb + hd).standard_normal((nb, n_head, hd)) * 0.5).astype(np.float32)
    qb = G.Buffer.from_array(q)
    one, loop = G.Buffer(nb * n_head * hd * 4), G.Buffer(nb * n_head * hd * 4)
    G.attn_prefill(qb, kb, vb, kv_type, n_head, n_kv, hd, pos0, nb, one)
    G.attn_prefill(qb, kb, vb, kv_type, n_head, n_kv, hd, pos0, nb, loop, batched=False)
    a = one.download(np.float32, (nb, n_head, hd))
    assert a.tobytes() == loop.download(np.float32, (nb, n_head, hd)).tobytes()
    for b in (0, nb - 1):
        d = G.Buffer(n_head * hd * 4)
        G.attn_decode(G.Buffer.from_array(q[b]), kb, vb, kv_type, n_head, n_kv, hd, pos0 + b + 1, d)
        assert d.download(np.float32, (n_head, hd)).tobytes() == a[b].tobytes(), f"token {b}"
        ref = oracle.attn_decode(q[b], kh, vh, kv_type, n_head, n_kv, hd, pos0 + b)
        assert (np.abs(a[b].astype(np.float64) - ref) <= ATOL + RTOL * np.abs(ref)).all(), f"token {b}"


def test_attention_timeout_reported_by_status(gpu, oracle):
    """The one-launch attention's bounded waits: forced to give up (the test
    hook makes them wait for a tag no store carries, 64 retries), every kernel
    still ends and g4h_attn_status reports it once; in normal operation the
    same call gives the oracle's result and a clear status."""
    G = gpu
    n_head, n_kv, hd, n_pos = 8, 4, 256, 8192
    assert G.attn_passes(G.F16, n_head, n_kv, hd, n_pos) == 1
    kb, vb, kh, vh = make_cache(G, oracle, G.F16, n_pos, n_kv, hd, seed=77)
    q = np.random.default_rng(6).standard_normal((n_head, hd)).astype(np.float32)
    qb, out = G.Buffer.from_array(q), G.Buffer(n_head * hd * 4)
    ws = G.Buffer(G.attn_workspace_bytes(n_head, hd, n_pos))
    ws.zero()
    try:
        G.debug_attn_timeout(True)
        G.attn_decode(qb, kb, vb, G.F16, n_head, n_kv, hd, n_pos, out, ws=ws)
        assert G.attn_status(ws)
        assert not G.attn_status(ws)                       # reported once
    finally:
        G.debug_attn_timeout(False)
    G.attn_decode(qb, kb, vb, G.F16, n_head, n_kv, hd, n_pos, out, ws=ws)
    assert not G.attn_status(ws)
    got = out.download(np.float32, (n_head, hd))
    ref = oracle.attn_decode(q, kh, vh, G.F16, n_head, n_kv, hd, n_pos - 1)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= ATOL + RTOL * np.abs(ref))


def test_attention_after_unread_timeout_is_nan_until_status(gpu, oracle):
    """A give-up that no status call has read yet: the next calls on that
    workspace (waits no longer forced) write NaN, since a workgroup of the
    failed launch that started after its epoch advance may have left words
    under the next launch's tag; the status call then reports the failure
    once, the workspace is cleared before its next use, and results are the
    oracle's again."""
    G = gpu
    n_head, n_kv, hd, n_pos = 8, 4, 256, 1000
    assert G.attn_passes(G.F16, n_head, n_kv, hd, n_pos) == 1
    kb, vb, kh, vh = make_cache(G, oracle, G.F16, n_pos, n_kv, hd, seed=78)
    q = np.random.default_rng(7).standard_normal((n_head, hd)).astype(np.float32)
    qb, out = G.Buffer.from_array(q), G.Buffer(n_head * hd * 4)
    ws = G.Buffer(G.attn_workspace_bytes(n_head, hd, n_pos))
    ws.zero()
    try:
        G.debug_attn_timeout(True)
        G.attn_decode(qb, kb, vb, G.F16, n_head, n_kv, hd, n_pos, out, ws=ws)
    finally:
        G.debug_attn_timeout(False)
    for _ in range(2):
        G.attn_decode(qb, kb, vb, G.F16, n_head, n_kv, hd, n_pos, out, ws=ws)
        assert np.isnan(out.download(np.float32, (n_head, hd))).all()
    assert G.attn_status(ws)
    assert not G.attn_status(ws)
    ref = oracle.attn_decode(q, kh, vh, G.F16, n_head, n_kv, hd, n_pos - 1)
    for _ in range(2):
        G.attn_decode(qb, kb, vb, G.F16, n_head, n_kv, hd, n_pos, out, ws=ws)
        got = out.download(np.float32, (n_head, hd))
        assert np.all(np.abs(got.astype(np.float64) - ref) <= ATOL + RTOL * np.abs(ref))
    assert not G.attn_status(ws)


@pytest.mark.parametrize("kv_type", [1, 8, 2], ids=["f16", "q8_0", "q4_0"])
@pytest.mark.parametrize("n_head,hd,n_pos,window,ring", [
    (4, 64, 9, 8, 40), (4, 64, 100, 8, 40), (8, 256, 1000, 512, 576), (8, 256, 700, 512, 576), (2, 128, 300, 300, 0),
    (4, 64, 50, 1, 40), (8, 128, 5, 512, 576), (8, 256, 1300, 129, 576), (8, 512, 700, 512, 576), (8, 512, 300, 0, 0)])
def test_window_ring_attention_vs_oracle(gpu, oracle, kv_type, n_head, hd, n_pos, window, ring):
    """model.c:517-537: a sliding window over a KV ring (GPU: rows stored at
    slot j % ring and j % ring + ring; oracle: one copy in `ring` slots) and,
    with ring 0, a window over a linear cache."""
    G = gpu
    n_kv = 1
    slots = 2 * ring if ring else n_pos
    rows = np.random.default_rng(n_pos + window).standard_normal((2, n_pos, hd)).astype(np.float32)
    rb = hd * 2 if kv_type == G.F16 else G.row_size(kv_type, hd)

    def stored(x):
        b = G.Buffer(n_pos * rb)
        G.kv_store(kv_type, G.Buffer.from_array(x), b, hd, rows=n_pos, dst_stride=rb)
        return b.download(np.uint8, (n_pos, rb))

    lin = [stored(rows[0]), stored(rows[1])]
    gpu_c = [np.zeros((slots, rb), np.uint8) for _ in range(2)]
    ora_c = [np.zeros((ring if ring else n_pos, rb), np.uint8) for _ in range(2)]
    for j in range(n_pos):                       # the caches as n_pos decode steps leave them
        for c in range(2):
            if ring:
                gpu_c[c][j % ring] = lin[c][j]
                gpu_c[c][j % ring + ring] = lin[c][j]
                ora_c[c][j % ring] = lin[c][j]
            else:
                gpu_c[c][j] = lin[c][j]
                ora_c[c][j] = lin[c][j]
    q = np.random.default_rng(7).standard_normal((n_head, hd)).astype(np.float32)
    out = G.Buffer(n_head * hd * 4)
    G.attn_decode_window(G.Buffer.from_array(q), G.Buffer.from_array(gpu_c[0]), G.Buffer.from_array(gpu_c[1]), kv_type,
                         n_head, n_kv, hd, n_pos, window, ring, out)
    got = out.download(np.float32, (n_head, hd))
    pos = n_pos - 1
    j0 = max(0, pos - window + 1) if window else 0
    ref = np.zeros((n_head, hd), np.float32)
    L = oracle.lib()
    L.g4o_attn_window.argtypes = [oracle._vp] * 3 + [oracle.C.c_int] * 7 + [oracle._vp, oracle.C.c_int]
    L.g4o_attn_window(q.ctypes.data, ora_c[0].ctypes.data, ora_c[1].ctypes.data, kv_type, n_head, n_kv, hd, pos, j0,
                      ring if ring else n_pos, ref.ctypes.data, 1)
    err = np.abs(got.astype(np.float64) - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} outside tolerance, worst {err.max():.3g}"


# ------------------------------------------ prompt batch on the matrix cores
def _mm_slack(q, kc, vc, n_head, n_kv, hd, rows):
    """f16 V: where a softmax weight lies within 1e-4 of an fp16 rounding
    midpoint, the GPU's weight (its scores differ from the CPU's by the fp32
    order of the dot) may take the neighbouring code; per output element the
    most that can move it.  rows: the cache rows the token attends."""
    K = np.frombuffer(kc.tobytes(), np.float16).reshape(-1, n_kv, hd)[rows].astype(np.float64)
    V = np.frombuffer(vc.tobytes(), np.float16).reshape(-1, n_kv, hd)[rows].astype(np.float64)
    grp = n_head // n_kv
    slack = np.zeros((n_head, hd))
    for h in range(n_head):
        sc = K[:, h // grp] @ q[h].astype(np.float16).astype(np.float64)
        w = np.exp(sc - sc.max())
        w /= w.sum()
        w16 = w.astype(np.float32).astype(np.float16)
        a = w16.astype(np.float64)
        up = np.nextafter(w16, np.float16(np.inf)).astype(np.float64)
        dn = np.nextafter(w16, np.float16(-np.inf)).astype(np.float64)
        ulp = np.where(np.abs(w - (a + up) / 2) <= 1e-4 * w, up - a, 0.0) + \
            np.where(np.abs(w - (a + dn) / 2) <= 1e-4 * w, a - dn, 0.0)
        slack[h] = ulp @ np.abs(V[:, h // grp])
    return slack


@pytest.mark.parametrize("n_head,n_kv,hd,pos0,nb", [
    (8, 4, 256, 4096, 64), (8, 4, 256, 0, 9), (8, 4, 256, 300, 33), (8, 1, 256, 1000, 17), (4, 4, 128, 200, 40),
    (8, 2, 64, 77, 20), (16, 8, 128, 513, 100), (8, 4, 256, 127, 1),
    # gemma4's full-attention heads: 8 query heads of 512 over one KV head
    (8, 1, 512, 700, 33), (8, 1, 512, 0, 12), (2, 1, 512, 130, 1)])
def test_prefill_matrix_cores_vs_oracle(gpu, oracle, n_head, n_kv, hd, pos0, nb):
    """g4h_attn_prefill_mm (model.c:509-545 for a prompt batch): every token's
    row against the oracle's attention at its position (with the fp16-weight
    slack of _mm_slack); tiles of 1 / 2 / 4 / 8 query heads per KV head,
    batches off the tile size, chunks and spans ragged, the first token at
    position 0."""
    G = gpu
    n_slot = pos0 + nb
    kb, vb, kh, vh = make_cache(G, oracle, G.F16, n_slot, n_kv, hd, seed=n_slot + hd)
    q = (np.random.default_rng(nb + hd).standard_normal((nb, n_head, hd)) * 0.5).astype(np.float32)
    out = G.Buffer(nb * n_head * hd * 4)
    G.attn_prefill_mm(G.Buffer.from_array(q), kb, vb, G.F16, n_head, n_kv, hd, pos0, nb, out)
    got = out.download(np.float32, (nb, n_head, hd))
    oracle.pool_start(8)
    try:
        for b in range(nb):
            ref = oracle.attn_decode(q[b], kh, vh, G.F16, n_head, n_kv, hd, pos0 + b, nthreads=8)
            err = np.abs(got[b].astype(np.float64) - ref)
            bad = err > ATOL + RTOL * np.abs(ref)
            if bad.any():
                bad &= err > ATOL + RTOL * np.abs(ref) + _mm_slack(q[b], kh, vh, n_head, n_kv, hd, np.arange(pos0 + b + 1))
            assert not bad.any(), f"token {b}: {bad.sum()} outside tolerance, worst {err.max():.3g}"
    finally:
        oracle.pool_stop()


@pytest.mark.parametrize("hd,pos0,nb,window,ring", [(256, 700, 64, 512, 576), (256, 100, 30, 512, 576), (64, 50, 25, 16, 40),
                                                    (128, 0, 12, 8, 20), (256, 300, 40, 300, 0), (512, 600, 20, 300, 0)])
def test_prefill_matrix_cores_window_ring(gpu, oracle, hd, pos0, nb, window, ring):
    """The sliding window over a KV ring (model.c:517-537): token b attends
    max(0, p + 1 - window) .. p; on a ring each position's row sits at slot
    p % ring and again at p % ring + ring, written as the decode steps and
    the batch's own row preparation leave them."""
    G = gpu
    n_head, n_kv = 8, 1
    n_pos = pos0 + nb
    slots = 2 * ring if ring else n_pos
    rows = np.random.default_rng(n_pos + window).standard_normal((2, n_pos, hd)).astype(np.float32)
    rb = hd * 2

    def stored(x):
        b = G.Buffer(n_pos * rb)
        G.kv_store(G.F16, G.Buffer.from_array(x), b, hd, rows=n_pos, dst_stride=rb)
        return b.download(np.uint8, (n_pos, rb))

    lin = [stored(rows[0]), stored(rows[1])]
    gpu_c = [np.zeros((slots, rb), np.uint8) for _ in range(2)]
    for j in range(n_pos):
        for c in range(2):
            if ring:
                gpu_c[c][j % ring] = lin[c][j]
                gpu_c[c][j % ring + ring] = lin[c][j]
            else:
                gpu_c[c][j] = lin[c][j]
    q = (np.random.default_rng(7).standard_normal((nb, n_head, hd)) * 0.5).astype(np.float32)
    out = G.Buffer(nb * n_head * hd * 4)
    G.attn_prefill_mm(G.Buffer.from_array(q), G.Buffer.from_array(gpu_c[0]), G.Buffer.from_array(gpu_c[1]), G.F16,
                      n_head, n_kv, hd, pos0, nb, out, window=window, ring=ring)
    got = out.download(np.float32, (nb, n_head, hd))
    L = oracle.lib()
    L.g4o_attn_window.argtypes = [oracle._vp] * 3 + [oracle.C.c_int] * 7 + [oracle._vp, oracle.C.c_int]
    for b in range(nb):
        pos = pos0 + b
        j0 = max(0, pos - window + 1) if window else 0
        ref = np.zeros((n_head, hd), np.float32)
        qb = np.ascontiguousarray(q[b])
        L.g4o_attn_window(qb.ctypes.data, lin[0].ctypes.data, lin[1].ctypes.data, G.F16, n_head, n_kv, hd, pos, j0, n_pos,
                          ref.ctypes.data, 1)
        err = np.abs(got[b].astype(np.float64) - ref)
        bad = err > ATOL + RTOL * np.abs(ref)
        if bad.any():
            bad &= err > ATOL + RTOL * np.abs(ref) + _mm_slack(qb, lin[0], lin[1], n_head, n_kv, hd, np.arange(j0, pos + 1))
        assert not bad.any(), f"token {b}: {bad.sum()} outside tolerance, worst {err.max():.3g}"


@pytest.mark.parametrize("hd,grp,pos0,nb,window,ring", [(256, 8, 300, 40, 0, 0), (128, 2, 700, 24, 16, 40),
                                                         (256, 8, 700, 40, 512, 576), (64, 4, 5, 30, 0, 0),
                                                         (512, 8, 1000, 33, 0, 0)])
def test_prefill_matrix_cores_rows_independent_of_batch(gpu, oracle, hd, grp, pos0, nb, window, ring):
    """A token's row has the same bits in any batch, alone included: positions
    are cut at multiples of 128 / 256 counted from 0, and each row's sums take
    its own operands in its own order (what lets decode steps, verify batches
    and prompt batches of the gemma4 model share these kernels)."""
    G = gpu
    n_kv = 1 if grp == 8 else 2
    n_head = grp * n_kv
    n_pos = pos0 + nb
    slots = 2 * ring if ring else n_pos
    rng = np.random.default_rng(hd + nb)
    rb = hd * 2
    caches = []
    for c in range(2):
        lin = G.Buffer(n_pos * n_kv * rb)
        G.kv_store(G.F16, G.Buffer.from_array(rng.standard_normal((n_pos * n_kv, hd)).astype(np.float32)), lin, hd,
                   rows=n_pos * n_kv, dst_stride=rb)
        h = lin.download(np.uint8, (n_pos, n_kv * rb))
        g = np.zeros((slots, n_kv * rb), np.uint8)
        for j in range(n_pos):
            g[j % ring if ring else j] = h[j]
            if ring:
                g[j % ring + ring] = h[j]
        caches.append(G.Buffer.from_array(g))
    q = (rng.standard_normal((nb, n_head, hd)) * 0.5).astype(np.float32)

    def run(b0, cnt):
        out = G.Buffer(cnt * n_head * hd * 4)
        G.attn_prefill_mm(G.Buffer.from_array(np.ascontiguousarray(q[b0:b0 + cnt])), caches[0], caches[1], G.F16, n_head,
                          n_kv, hd, pos0 + b0, cnt, out, window=window, ring=ring)
        return out.download(np.float32, (cnt, n_head, hd))

    full = run(0, nb)
    for b0, cnt in ((0, 1), (5, 1), (nb - 1, 1), (3, 9), (10, nb - 10)):
        part = run(b0, cnt)
        assert part.tobytes() == full[b0:b0 + cnt].tobytes(), f"tokens {b0}..{b0 + cnt - 1}"


def test_prefill_matrix_cores_errors(gpu):
    G = gpu
    b = G.Buffer(1 << 20)
    with pytest.raises(G.G4HError) as e:                              # q8_0 caches stay on the per-token form
        G.attn_prefill_mm(b, b, b, G.Q8_0, 8, 4, 256, 10, 16, b)
    assert e.value.status == G.ERR_TYPE
    with pytest.raises(G.G4HError) as e:                              # head dims are 64 / 128 / 256 / 512
        G.attn_prefill_mm(b, b, b, G.F16, 8, 4, 192, 10, 16, b)
    assert e.value.status == G.ERR_TYPE
    with pytest.raises(G.G4HError) as e:                              # a batch longer than the ring allows
        G.attn_prefill_mm(b, b, b, G.F16, 8, 1, 256, 10, 70, b, window=512, ring=576)
    assert e.value.status == G.ERR_ARG
