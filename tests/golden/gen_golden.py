"""Writes the golden fixtures under tests/golden/ from the reference's own
kernels: oracle/_ref/libg4ref.so, which `make -C oracle ref` compiles in place
from /root/reference/src/quants.c with the reference README's portable-build
flags (-Ofast -march=x86-64-v3 -funroll-loops -ffp-contract=fast).

Run in the build container (where /root/reference exists):
    make -C oracle ref && python tests/golden/gen_golden.py

Each fixture holds inputs and the reference build's outputs, nothing else:
  quant_<q>.npz     activation quantizer cases (random rows + edge cases)
  dot_<fmt>.npz     weight rows, fp32 activations, the reference's quantized
                    activations, AVX2 dots, scalar _ref dots, x4 dots,
                    dequantized rows and per-block integer sums obtained from
                    the reference's scalar dots with unit scales
  dot_f16.npz / dot_bf16.npz  f16 / bf16 weight rows, fp32 activations, the
                    activations as prep_act converts them (model.c:163-180,
                    with the header's inline conversions restated by the
                    oracle), the reference build's g4_dot_f16 / g4_dot_bf16
                    and its dequantized rows
  tables.npz        fp16->fp32 table and GELU fp16 table of g4_init_tables
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.path.join(ROOT, "oracle", "_ref", "libg4ref.so")

Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, TQ2_0 = 2, 8, 10, 11, 12, 13, 14, 15, 35
BLCK = {Q4_0: 32, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256, TQ2_0: 256}
SIZE = {Q4_0: 18, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292, TQ2_0: 66}
ACT = {Q4_0: Q8_0, Q8_0: Q8_0, Q2_K: Q8_K, Q3_K: Q8_K, Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K, TQ2_0: Q8_K}
NAME = {Q4_0: "q4_0", Q8_0: "q8_0", Q2_K: "q2_K", Q3_K: "q3_K", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K",
        TQ2_0: "tq2_0"}
DOT = {Q4_0: "q4_0_q8_0", Q8_0: "q8_0_q8_0", Q2_K: "q2_K_q8_K", Q3_K: "q3_K_q8_K", Q4_K: "q4_K_q8_K", Q5_K: "q5_K_q8_K",
       Q6_K: "q6_K_q8_K", TQ2_0: "tq2_0_q8_K"}
# fp16 scale fields (d, dmin) inside a weight block and the f32 d of q8_K
SCALES = {Q8_0: (0,), Q4_0: (0,), Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,), TQ2_0: (64,)}

vp = C.c_void_p


def load_ref():
    R = C.CDLL(REF)
    R.g4_init_tables()
    for q in ("q8_0", "q8_K", "q4_0"):
        getattr(R, "g4_quantize_" + q).argtypes = [vp, vp, C.c_int64]
    R.g4_dequant_row.argtypes = [C.c_int, vp, vp, C.c_int64]
    for nm in DOT.values():
        for suf in ("", "_ref"):
            f = getattr(R, "g4_dot_" + nm + suf)
            f.restype = C.c_float
            f.argtypes = [vp, vp, C.c_int64]
        f = getattr(R, "g4_dot_" + nm + "_x4")
        f.argtypes = [vp, C.POINTER(vp), C.c_int64, vp]
    return R


def ptr(a):
    return a.ctypes.data_as(vp)


def rsize(t, n):
    return n // BLCK[t] * SIZE[t]


def quant(R, qt, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros((x.shape[0], rsize(qt, x.shape[1])), np.uint8)
    for i in range(x.shape[0]):
        getattr(R, "g4_quantize_" + NAME[qt])(ptr(x[i]), ptr(out[i]), x.shape[1])
    return out


def quant_cases(n):
    rng = np.random.default_rng(7)
    rows = [rng.standard_normal(n) * s for s in (1.0, 1e-3, 50.0, 1e-6)]
    z = np.zeros(n); rows.append(z)                                         # all-zero blocks
    t = np.tile(np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 127.0, -127.0]), n // 8); rows.append(t)  # ties
    m = rng.standard_normal(n); m[::37] = -m[::37] * 40; rows.append(m)      # negative maxima
    e = rng.standard_normal(n); e[1::2] = e[0::2]; rows.append(e)            # repeated magnitudes
    s = rng.standard_normal(n) * 1e-5; rows.append(s)                        # subnormal fp16 scales
    h = np.full(n, 3.0); h[::2] = -3.0; rows.append(h)                       # |max| ties of opposite sign
    # blocks whose scale amax*fp32(1/127) is an exact fp16 rounding tie (the
    # fp32 product must be rounded before the fp16 conversion, quants.c:91-92)
    c = np.float32(1.0 / 127.0)
    cand = (rng.random(4000000) * 8 + 0.5).astype(np.float32)
    ties = cand[((cand * c).view(np.uint32) & 0x1FFF) == 0x1000][: 2 * n // 32]
    t2 = (rng.standard_normal((ties.size, 32)) * 0.2).astype(np.float32)
    t2[:, 5] = ties * np.where(np.arange(ties.size) % 2, 1, -1)
    t2 = t2.reshape(-1)
    rows.append(t2[:n]); rows.append(t2[n:2 * n])
    return np.array(rows, dtype=np.float32)


def weights(qt, rows, n, rng):
    nb = n // BLCK[qt]
    w = rng.integers(0, 256, size=(rows, nb, SIZE[qt]), dtype=np.uint8)
    if qt == Q8_0:
        w[:, :, 2:] = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8).view(np.uint8)
    for off in SCALES[qt]:
        h = (np.abs(rng.standard_normal((rows, nb))) * (0.02 / 127 if qt == Q8_0 else 0.02 / 8 if qt == Q4_0 else 1e-3)
             ).astype(np.float32).astype(np.float16).view(np.uint16)
        w[:, :, off] = h & 0xFF
        w[:, :, off + 1] = h >> 8
    return np.ascontiguousarray(w.reshape(rows, nb * SIZE[qt]))


def unit_sums(R, qt, w_row, a_row, n):
    """Per-block integers through the reference's scalar dots with unit scales."""
    at = ACT[qt]
    nb = n // BLCK[qt]
    per = 2 if qt in (Q2_K, Q4_K, Q5_K) else 1
    out = np.zeros(nb * per, np.int64)
    f = getattr(R, "g4_dot_" + DOT[qt] + "_ref")
    for b in range(nb):
        wb = w_row[b * SIZE[qt]:(b + 1) * SIZE[qt]].copy()
        ab = a_row[b * SIZE[at]:(b + 1) * SIZE[at]].copy()
        if at == Q8_0:
            ab[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        else:
            ab[0:4] = np.frombuffer(np.float32(1.0).tobytes(), np.uint8)
        one = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        zero = np.zeros(2, np.uint8)
        if qt in (Q8_0, Q4_0, Q3_K, Q6_K, TQ2_0):
            wb[SCALES[qt][0]:SCALES[qt][0] + 2] = one
            out[b] = int(f(ptr(wb), ptr(ab), BLCK[qt]))
        else:
            d_off, m_off = SCALES[qt]
            wb[d_off:d_off + 2] = one; wb[m_off:m_off + 2] = zero
            out[2 * b] = int(f(ptr(wb), ptr(ab), 256))
            wb[d_off:d_off + 2] = zero; wb[m_off:m_off + 2] = one
            out[2 * b + 1] = -int(f(ptr(wb), ptr(ab), 256))
    return out


def main(only=None):
    """Writes every fixture, or with format names as arguments (e.g. `q6_K`)
    only those formats' dot fixtures."""
    if not os.path.exists(REF):
        sys.exit(f"{REF} missing: run `make -C oracle ref` first")
    R = load_ref()
    flags = "-Ofast -march=x86-64-v3 -funroll-loops -ffp-contract=fast"

    # activation quantizers
    for qt in (Q8_0, Q8_K, Q4_0):
        if only:
            break
        x = quant_cases(1024)
        np.savez_compressed(os.path.join(HERE, f"quant_{NAME[qt]}.npz"), x=x, y=quant(R, qt, x), flags=flags)

    # dots, x4, dequant, per-block sums
    for qt in (Q8_0, Q4_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, TQ2_0):
        if only and NAME[qt] not in only:
            continue
        rng = np.random.default_rng(100 + qt)
        n = 2048 if BLCK[qt] == 256 else 1024
        rows, nb_tok = 16, 4
        w = weights(qt, rows, n, rng)
        x = rng.standard_normal((nb_tok, n)).astype(np.float32)
        a = quant(R, ACT[qt], x)
        dot = np.zeros((nb_tok, rows), np.float32)
        dot_ref = np.zeros((nb_tok, rows), np.float32)
        dot_x4 = np.zeros((nb_tok, rows), np.float32)
        f, fr, f4 = (getattr(R, "g4_dot_" + DOT[qt] + s) for s in ("", "_ref", "_x4"))
        aps = (vp * 4)(*[a[t].ctypes.data for t in range(4)])
        for r in range(rows):
            for t in range(nb_tok):
                dot[t, r] = f(ptr(w[r]), ptr(a[t]), n)
                dot_ref[t, r] = fr(ptr(w[r]), ptr(a[t]), n)
            o4 = np.zeros(4, np.float32)
            f4(ptr(w[r]), aps, n, ptr(o4))
            dot_x4[:, r] = o4
        deq = np.zeros((rows, n), np.float32)
        for r in range(rows):
            R.g4_dequant_row(qt, ptr(w[r]), ptr(deq[r]), n)
        sums = np.array([unit_sums(R, qt, w[r], a[0], n) for r in range(rows)])
        np.savez_compressed(os.path.join(HERE, f"dot_{NAME[qt]}.npz"), w=w, x=x, a=a, dot=dot, dot_ref=dot_ref,
                            dot_x4=dot_x4, deq=deq, sums=sums, n=n, flags=flags)

    # f16 / bf16 weights (quants.c:1319-1347); n has a tail past the 8-lane loop
    for name, wt in (("f16", 1), ("bf16", 30)):
        if only and name not in only:
            continue
        sys.path.insert(0, ROOT)
        from oracle import g4o
        rng = np.random.default_rng(200 + wt)
        rows, nb_tok, n = 16, 4, 2053
        wf = (rng.standard_normal((rows, n)) * 0.02).astype(np.float32)
        w = g4o.fp32_to_fp16(wf).reshape(rows, n) if wt == 1 else (wf.view(np.uint32) >> 16).astype(np.uint16)
        x = rng.standard_normal((nb_tok, n)).astype(np.float32)
        a = np.stack([g4o.prep_act(wt, x[t:t + 1])[0][: n * (2 if wt == 1 else 4)] for t in range(nb_tok)])
        fn = getattr(R, "g4_dot_" + name)
        fn.restype = C.c_float
        fn.argtypes = [vp, vp, C.c_int64]
        dot = np.array([[fn(ptr(w[r]), ptr(a[t]), n) for r in range(rows)] for t in range(nb_tok)], np.float32)
        deq = np.zeros((rows, n), np.float32)
        for r in range(rows):
            R.g4_dequant_row(wt, ptr(w[r]), ptr(deq[r]), n)
        np.savez_compressed(os.path.join(HERE, f"dot_{name}.npz"), w=w.view(np.uint8).reshape(rows, 2 * n), x=x, a=a,
                            dot=dot, deq=deq, n=n, flags=flags)

    if only:
        print("fixtures written to", HERE)
        return
    f16 = np.ctypeslib.as_array((C.c_float * 65536).in_dll(R, "g4_fp16_to_fp32_table")).copy()
    gelu = np.ctypeslib.as_array((C.c_uint16 * 65536).in_dll(R, "g4_gelu_fp16_table")).copy()
    np.savez_compressed(os.path.join(HERE, "tables.npz"), fp16_to_fp32=f16.view(np.uint32), gelu=gelu, flags=flags)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main(sys.argv[1:] or None)
