"""Pins the CPU oracle (oracle/) against the reference's own kernels.

Three independent anchors:
  * the committed golden fixtures made from the reference build
    (tests/golden/gen_golden.py) -- available everywhere;
  * the reference build itself (oracle/_ref/libg4ref.so) on fresh random
    inputs -- when it has been built;
  * mathematics: exhaustive fp16 round trip, numpy's float16 rounding,
    exact-integer brute force of the block sums, dequant consistency.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ------------------------------------------------------------------ fp16
def test_fp16_to_fp32_matches_reference_table(oracle):
    t = gold("tables.npz")["fp16_to_fp32"]
    mine = oracle.fp16_to_fp32(np.arange(65536, dtype=np.uint16))
    assert np.array_equal(bits(mine), t)


def test_fp16_exhaustive_round_trip(oracle):
    # quants.c:1719-1731: every finite code survives fp16 -> fp32 -> fp16
    codes = np.arange(65536, dtype=np.uint16)
    f = oracle.fp16_to_fp32(codes)
    fin = np.isfinite(f)
    back = oracle.fp32_to_fp16(f[fin])
    assert np.array_equal(back, codes[fin])


def test_fp32_to_fp16_is_numpy_rne(oracle):
    # numpy's float32->float16 cast is IEEE round-to-nearest-even with
    # gradual underflow; compare on values straddling ties and subnormals
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 3000),
        (np.arange(-2048, 2048, dtype=np.float32) + 0.5) * 2.0 ** -24,   # exact subnormal ties
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) * 2.0 ** -10,    # exact normal ties
        np.array([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0], dtype=np.float32),
    ]).astype(np.float32)
    assert np.array_equal(oracle.fp32_to_fp16(v), v.astype(np.float16).view(np.uint16))


# ------------------------------------------------------------ quantizers
@pytest.mark.parametrize("qname,qt", [("q8_0", 8), ("q8_K", 15), ("q4_0", 2)])
def test_quantizers_match_reference_fixtures(oracle, qname, qt):
    g = gold(f"quant_{qname}.npz")
    assert np.array_equal(oracle.quantize(qt, g["x"]), g["y"])


def test_quantize_q8_0_closed_form(oracle):
    # amax=127 -> d=1, id=1: quantization is the identity on integers, and
    # 0.5 ties go to even; an all-zero block gives d=0, q=0 (quants.c:91-98)
    x = np.zeros(64, np.float32)
    x[:32] = np.array([127, -127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5] + list(range(24)), np.float32)
    y = oracle.quantize(8, x)[0]
    assert y[0:2].view(np.uint16)[0] == np.float16(1.0).view(np.uint16)
    assert list(y[2:10].view(np.int8)) == [127, -127, 0, 2, 2, 0, -2, -2]
    assert list(y[10:34].view(np.int8)) == list(range(24))
    assert not y[34:].any()


def test_quantize_q8_K_closed_form(oracle):
    # the signed max maps to -127 (iscale = -127/max); q clipped at +127;
    # bsums are the 16-element group sums (quants.c:150-172)
    x = np.linspace(-1, 1, 256).astype(np.float32)
    x[5] = -2.0
    y = oracle.quantize(15, x)[0]
    q = y[4:260].view(np.int8).astype(int)
    assert q[5] == -127
    assert q.max() <= 127
    bs = y[260:292].view(np.int16)
    assert np.array_equal(bs, q.reshape(16, 16).sum(1))
    d = y[0:4].view(np.float32)[0]
    assert d == np.float32(-2.0) * np.float32(-1.0 / 127.0)


def test_quantize_q8_K_ties_nan_and_empty(oracle):
    # the first element of largest |x| sets the scale (quants.c:150-154
    # compares strictly): +127 at 7 beats -127 at 9, so iscale = -1, x[7] ->
    # -127, x[9] -> +127 and 2.5 -> -2.5 -> -2 (half to even); NaN elements
    # fail `ax > amax` and, quantized, give 0 (their bits under the 1.5*2^23
    # trick); a superblock of NaNs has amax 0 and stores zeros (quants.c:155-160)
    x = np.zeros((1, 3 * 256), np.float32)
    x[0, 7], x[0, 9], x[0, 20] = 127.0, -127.0, 2.5
    x[0, 256], x[0, 300], x[0, 306] = np.nan, 2.0, np.nan
    x[0, 512:] = np.nan
    y = oracle.quantize(15, x)[0].reshape(3, 292)
    q = y[:, 4:260].view(np.int8).astype(int)
    d = y[:, 0:4].view(np.float32)[:, 0]
    assert (q[0, 7], q[0, 9], q[0, 20]) == (-127, 127, -2) and not np.delete(q[0], [7, 9, 20]).any()
    assert d[0] == np.float32(127.0) * np.float32(-1.0 / 127.0)
    assert q[1, 44] == -127 and q[1, 0] == 0 and q[1, 50] == 0 and d[1] == np.float32(2.0) * np.float32(-1.0 / 127.0)
    assert not y[2].any()


# ---------------------------------------------------- dots / dequant / sums
FMTS = [("q8_0", 8), ("q4_0", 2), ("q2_K", 10), ("q3_K", 11), ("q4_K", 12), ("q5_K", 13), ("q6_K", 14), ("tq2_0", 35)]


@pytest.mark.parametrize("name,qt", FMTS)
def test_dots_match_reference_fixtures(oracle, name, qt):
    g = gold(f"dot_{name}.npz")
    w, a, n = g["w"], g["a"], int(g["n"])
    at = oracle.ACT[qt]
    # the reference's activation quantization of the stored x
    assert np.array_equal(oracle.quantize(at, g["x"]), a)
    avx = np.array([[oracle.dot(qt, w[r], a[t], n) for r in range(w.shape[0])] for t in range(a.shape[0])], np.float32)
    assert np.array_equal(bits(avx), bits(g["dot"])), "shipped AVX2 dot order not reproduced bit for bit"
    # x4 == x1 in the reference build (g4run.h:148-157)
    assert np.array_equal(bits(g["dot_x4"]), bits(g["dot"]))
    # scalar _ref dots: the README build vectorises them (-Ofast), so only the
    # selftest's tolerance holds (quants.c:1583)
    ref = np.array([[oracle.dot(qt, w[r], a[t], n, "ref") for r in range(w.shape[0])] for t in range(a.shape[0])])
    assert np.all(np.abs(ref - g["dot_ref"]) <= 1e-3 * (1 + np.abs(g["dot_ref"])))


@pytest.mark.parametrize("name,qt", FMTS)
def test_dequant_matches_reference_fixtures(oracle, name, qt):
    g = gold(f"dot_{name}.npz")
    assert np.array_equal(bits(oracle.dequant(qt, g["w"], int(g["n"]))), bits(g["deq"]))


@pytest.mark.parametrize("name,qt", FMTS)
def test_block_sums_match_reference_unit_scale_dots(oracle, name, qt):
    g = gold(f"dot_{name}.npz")
    s = oracle.block_sums(qt, g["w"], g["a"][0], int(g["n"]))
    assert np.array_equal(s.astype(np.int64), g["sums"])


@pytest.mark.parametrize("name,qt", FMTS)
def test_block_sums_brute_force(oracle, name, qt):
    """Integer identity: with every scale set to 1 (and mins to 0), the exact
    dot of dequantized weights and activation quants equals the block sum.
    Computed in int64 from the dequant of a unit-scale copy."""
    g = gold(f"dot_{name}.npz")
    n = int(g["n"])
    w = g["w"][:4].copy()
    a = g["a"][0]
    bs = oracle.SIZE[qt]
    nb = n // oracle.BLCK[qt]
    wv = w.reshape(4, nb, bs)
    one = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    zero = np.zeros(2, np.uint8)
    if qt in (8, 2):
        wv[:, :, 0:2] = one
    elif qt == 11:
        wv[:, :, 108:110] = one
    elif qt == 14:
        wv[:, :, 208:210] = one
    elif qt == 35:
        wv[:, :, 64:66] = one
    elif qt == 10:
        wv[:, :, 80:82] = one; wv[:, :, 82:84] = zero
    else:
        wv[:, :, 0:2] = one; wv[:, :, 2:4] = zero
    deq = oracle.dequant(qt, w, n).astype(np.int64)          # exact small integers
    if oracle.ACT[qt] == 8:
        qa = a.reshape(nb, 34)[:, 2:].view(np.int8).astype(np.int64).reshape(-1)
    else:
        qa = a.reshape(nb, 292)[:, 4:260].view(np.int8).astype(np.int64).reshape(-1)
    per = deq * qa
    blk = oracle.BLCK[qt]
    expect = per.reshape(4, nb, blk).sum(-1)
    s = oracle.block_sums(qt, w, a, n)
    got = s[:, 0::2] if qt in (10, 12, 13) else s
    assert np.array_equal(got.astype(np.int64), expect)


@pytest.mark.parametrize("name,qt", FMTS)
def test_dequant_consistency(oracle, name, qt):
    # quants.c:1604-1663: sum dequant(w) * (d_a*q_a) in double ~= the dot
    g = gold(f"dot_{name}.npz")
    n = int(g["n"])
    w, a = g["w"], g["a"][0]
    deq = oracle.dequant(qt, w, n).astype(np.float64)
    nb = n // oracle.BLCK[qt]
    if oracle.ACT[qt] == 8:
        blocks = a.reshape(nb, 34)
        da = oracle.fp16_to_fp32(blocks[:, 0:2].copy().view(np.uint16).ravel()).astype(np.float64)
        qa = blocks[:, 2:].view(np.int8).astype(np.float64)
        av = (qa * da[:, None]).reshape(-1)
    else:
        blocks = a.reshape(nb, 292)
        da = blocks[:, 0:4].copy().view(np.float32).ravel().astype(np.float64)
        av = (blocks[:, 4:260].view(np.int8).astype(np.float64) * da[:, None]).reshape(-1)
    s = deq @ av
    d = np.array([oracle.dot(qt, w[r], a, n) for r in range(w.shape[0])])
    assert np.all(np.abs(s - d) <= 1e-2 * (1 + np.abs(s)))


# ------------------------------------------------- against the live build
ref_built = pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(os.path.dirname(__file__)), "oracle", "_ref", "libg4ref.so")),
                               reason="oracle/_ref not built (make -C oracle ref)")


@ref_built
def test_reference_selftest_passes(oracle):
    assert oracle.ref().g4_selftest_quants() == 0


@ref_built
@pytest.mark.parametrize("name,qt", FMTS)
def test_random_dots_bit_exact_vs_reference_build(oracle, name, qt):
    from g4run_amd import synth
    n = 4096 if oracle.BLCK[qt] == 32 else 4096
    w = synth.weights(qt, 24, n, seed=5 + qt)
    x = synth.activations(3, n, seed=6 + qt)
    at = oracle.ACT[qt]
    a = oracle.quantize(at, x)
    assert np.array_equal(a, oracle.quantize(at, x, use_ref=True))
    for t in range(3):
        for r in range(24):
            mine = oracle.dot(qt, w[r], a[t], n)
            theirs = oracle.dot(qt, w[r], a[t], n, "refbuild")
            assert np.float32(mine).view(np.uint32) == np.float32(theirs).view(np.uint32)


@ref_built
@pytest.mark.parametrize("qt", [8, 15, 2])
def test_random_quantizers_bit_exact_vs_reference_build(oracle, qt):
    rng = np.random.default_rng(3)
    for scale in (1.0, 1e-4, 300.0):
        x = (rng.standard_normal((64, 1024)) * scale).astype(np.float32)
        assert np.array_equal(oracle.quantize(qt, x), oracle.quantize(qt, x, use_ref=True))


def test_gelu_table_matches_reference(oracle):
    g = gold("tables.npz")["gelu"]
    mine = oracle.gelu_table()
    diff = np.nonzero(mine != g)[0]
    assert diff.size == 0, f"{diff.size} GELU codes differ, first {diff[:8]}"


# ------------------------------------------------------ f16 / bf16 weights
FLOAT_FMTS = [("f16", 1), ("bf16", 30)]


@pytest.mark.parametrize("name,wt", FLOAT_FMTS)
def test_float_dots_match_reference_fixtures(oracle, name, wt):
    """g4_dot_f16 / g4_dot_bf16 of the reference build (8 fused lanes, the
    hsum tree, a scalar tail: n = 2053) reproduced bit for bit."""
    g = gold(f"dot_{name}.npz")
    n = int(g["n"])
    w = g["w"]
    assert np.array_equal(np.stack([oracle.prep_act(wt, g["x"][t:t + 1])[0][: g["a"].shape[1]] for t in range(g["x"].shape[0])]), g["a"])
    d = np.array([[oracle.dot(wt, w[r], g["a"][t], n) for r in range(w.shape[0])] for t in range(g["a"].shape[0])], np.float32)
    assert np.array_equal(bits(d), bits(g["dot"]))
    assert np.array_equal(bits(oracle.dequant(wt, w, n)), bits(g["deq"]))
    # the scalar fallback order only to the selftest's tolerance
    ref = np.array([[oracle.dot(wt, w[r], g["a"][t], n, "ref") for r in range(w.shape[0])] for t in range(g["a"].shape[0])])
    assert np.all(np.abs(ref - g["dot"]) <= 1e-3 * (1 + np.abs(g["dot"])))


def test_bf16_rounding_is_nearest_even(oracle):
    """g4_fp32_to_bf16 (g4run.h:64-68), through prep_act's AC_BF16 rows
    (model.c:172-180), against a selection made in float64: the nearer of the
    two bf16 neighbours (2^128 standing in past the largest finite value),
    ties to the even mantissa, NaN kept quiet with its high half.  The values
    go in as an array: a subnormal passed as a C float argument would be
    flushed by the -Ofast reference library's FTZ mode in this process."""
    rng = np.random.default_rng(11)
    u = rng.integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7f7fffff, 0x00008000, 0x00018000,
                        0x3f808000, 0x3f818000, 0x7fc00001, 0xffa00000, 0x7f800001, 0x00203f76, 0xff7f8d0d], np.uint32)
    xs = np.concatenate([u, special])
    got = oracle.prep_act(30, xs.view(np.float32)[None, :])[0][: 4 * xs.size].view(np.uint32) >> 16
    import math

    def val(b):                                           # exact value of fp32 bits, no FPU subnormal path
        sg = -1.0 if b >> 31 else 1.0
        e, m = (b >> 23) & 0xFF, b & 0x7FFFFF
        return sg * (math.ldexp(m, -149) if e == 0 else math.ldexp(m | 0x800000, e - 150))

    for x, g in zip(xs.tolist(), got.tolist()):
        if (x & 0x7FFFFFFF) > 0x7F800000:
            assert g == ((x >> 16) | 64)
            continue
        lo, hi = x >> 16, (x >> 16) + 1
        f, flo = val(x), val(lo << 16)
        if (hi & 0x7FFF) == 0x7F80:                       # overflow: IEEE measures against 2^128
            fhi = (-1.0 if x >> 31 else 1.0) * 2.0 ** 128
        else:
            fhi = val((hi & 0xFFFF) << 16)
        if (x & 0x7FFFFFFF) == 0x7F800000:
            assert g == lo
            continue
        dl, dh = abs(f - flo), abs(fhi - f)
        want = lo if (dl < dh or (dl == dh and lo % 2 == 0)) else hi
        assert g == (want & 0xFFFF), hex(x)
