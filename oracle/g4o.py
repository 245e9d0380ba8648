"""ctypes front end of the CPU oracle (oracle/liboracle.so) and of the
reference build (oracle/_ref/libg4ref.so, the reference's src/quants.c
compiled in place by `make -C oracle ref`).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py -- never by the g4run_amd package.

Quantized tensors are numpy uint8 arrays of raw GGUF bytes, shape
[rows, row_bytes]; activations likewise, one row per token.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libg4ref.so")

F32, F16, Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, BF16, TQ2_0 = 0, 1, 2, 8, 10, 11, 12, 13, 14, 15, 30, 35
BLCK = {F32: 1, F16: 1, BF16: 1, Q4_0: 32, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256,
        TQ2_0: 256}
SIZE = {F32: 4, F16: 2, BF16: 2, Q4_0: 18, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292, TQ2_0: 66}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q2_K: "q2_K", Q3_K: "q3_K", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", TQ2_0: "tq2_0",
         F16: "f16", BF16: "bf16"}
# activation class (model.c:132-141); bf16 weights take bf16-rounded fp32 rows
ACT = {Q4_0: Q8_0, Q8_0: Q8_0, Q2_K: Q8_K, Q3_K: Q8_K, Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K, TQ2_0: Q8_K, F16: F16, BF16: F32}

_lib = None
_ref = None

_vp = C.c_void_p
_i64 = C.c_int64


def row_size(t: int, n: int) -> int:
    b = BLCK[t]
    return 0 if n % b else (n // b) * SIZE[t]


def act_stride(wtype: int, ncols: int) -> int:
    return (row_size(ACT[wtype], ncols) + 63) & ~63


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_vp)


def lib():
    """Load (building if needed) the oracle restatement."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            import subprocess
            subprocess.run(["make", "-C", HERE, "liboracle.so"], check=True,
                           stdout=subprocess.DEVNULL)
        L = C.CDLL(LIB_PATH)
        L.g4o_fp16_to_fp32.restype = C.c_float
        L.g4o_fp16_to_fp32.argtypes = [C.c_uint16]
        L.g4o_fp32_to_fp16.restype = C.c_uint16
        L.g4o_fp32_to_fp16.argtypes = [C.c_float]
        L.g4o_fp16_to_fp32_n.argtypes = [_vp, _vp, _i64]
        L.g4o_fp32_to_fp16_n.argtypes = [_vp, _vp, _i64]
        L.g4o_nearest_int.restype = C.c_int
        L.g4o_nearest_int.argtypes = [C.c_float]
        for q in ("q8_0", "q8_K", "q4_0"):
            f = getattr(L, "g4o_quantize_" + q)
            f.restype = None
            f.argtypes = [_vp, _vp, _i64]
        L.g4o_dequant_row.restype = C.c_int
        L.g4o_dequant_row.argtypes = [C.c_int, _vp, _vp, _i64]
        L.g4o_block_sums.restype = None
        L.g4o_block_sums.argtypes = [C.c_int, _vp, _vp, _i64, _vp]
        for f in (L.g4o_dot_ref, L.g4o_dot):
            f.restype = C.c_float
            f.argtypes = [C.c_int, _vp, _vp, _i64]
        L.g4o_dot_f16.restype = C.c_float
        L.g4o_dot_f16.argtypes = [_vp, _vp, _i64]
        L.g4o_dot_bf16.restype = C.c_float
        L.g4o_dot_bf16.argtypes = [_vp, _vp, _i64]
        L.g4o_fp32_to_bf16.restype = C.c_uint16
        L.g4o_fp32_to_bf16.argtypes = [C.c_float]
        L.g4o_matmul.restype = None
        L.g4o_matmul.argtypes = [C.c_int, _vp, _vp, C.c_size_t, _vp, _i64, _i64, C.c_int, C.c_int]
        L.g4o_prep_act.restype = None
        L.g4o_prep_act.argtypes = [C.c_int, _vp, _i64, C.c_int, _vp]
        L.g4o_pool_start.argtypes = [C.c_int]
        L.g4o_pool_stop.argtypes = []
        L.g4o_set_dot_fn.argtypes = [C.c_int, _vp]
        L.g4o_set_dot_f16_fn.argtypes = [_vp]
        L.g4o_rms_norm.argtypes = [_vp, _vp, _vp, C.c_int, C.c_float]
        L.g4o_rope_cache.argtypes = [_vp, C.c_int, C.c_int, C.c_float]
        L.g4o_rope_apply.argtypes = [_vp, _vp, C.c_int]
        L.g4o_gelu_table_entry.restype = C.c_uint16
        L.g4o_gelu_table_entry.argtypes = [C.c_uint16]
        L.g4o_gelu.restype = C.c_float
        L.g4o_gelu.argtypes = [C.c_float]
        L.g4o_argmax.restype = C.c_int
        L.g4o_argmax.argtypes = [_vp, C.c_int]
        L.g4o_attn_decode.argtypes = [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, C.c_int]
        L.g4o_kv_store.argtypes = [C.c_int, _vp, _vp, C.c_int]
        L.g4o_model_scratch_bytes.restype = C.c_size_t
        L.g4o_model_scratch_bytes.argtypes = [_vp]
        L.g4o_model_decode.restype = C.c_int
        L.g4o_model_decode.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, C.c_int]
        L.g4o_model_embed.argtypes = [_vp, C.c_int, _vp]
        L.g4o_model_layer.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, C.c_int]
        L.g4o_model_qkv.argtypes = [_vp, C.c_int, _vp, _vp, _vp, C.c_int]
        L.g4o_model_attn.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp, C.c_int]
        L.g4o_model_post.argtypes = [_vp, C.c_int, _vp, _vp, _vp, C.c_int]
        L.g4o_model_head.restype = C.c_int
        L.g4o_model_head.argtypes = [_vp, _vp, _vp, _vp, C.c_int]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own compiled kernels (oracle/_ref/libg4ref.so)."""
    global _ref
    if _ref is None:
        R = C.CDLL(REF_PATH)
        R.g4_init_tables()
        for q in ("q8_0", "q8_K", "q4_0"):
            f = getattr(R, "g4_quantize_" + q)
            f.restype = None
            f.argtypes = [_vp, _vp, _i64]
        R.g4_dequant_row.restype = None
        R.g4_dequant_row.argtypes = [C.c_int, _vp, _vp, _i64]
        for nm in ("q4_0_q8_0", "q8_0_q8_0", "q2_K_q8_K", "q3_K_q8_K", "q4_K_q8_K", "q5_K_q8_K", "q6_K_q8_K", "tq2_0_q8_K"):
            for suf in ("", "_ref"):
                f = getattr(R, "g4_dot_" + nm + suf)
                f.restype = C.c_float
                f.argtypes = [_vp, _vp, _i64]
            f = getattr(R, "g4_dot_" + nm + "_x4")
            f.restype = None
            f.argtypes = [_vp, C.POINTER(_vp), _i64, _vp]
        for nm in ("f16", "bf16"):
            f = getattr(R, "g4_dot_" + nm)
            f.restype = C.c_float
            f.argtypes = [_vp, _vp, _i64]
        R.g4_selftest_quants.restype = C.c_int
        _ref = R
    return _ref


DOT_NAME = {Q4_0: "q4_0_q8_0", Q8_0: "q8_0_q8_0", Q2_K: "q2_K_q8_K", Q3_K: "q3_K_q8_K", Q4_K: "q4_K_q8_K",
            Q5_K: "q5_K_q8_K", Q6_K: "q6_K_q8_K", TQ2_0: "tq2_0_q8_K", F16: "f16", BF16: "bf16"}


# ------------------------------------------------------------------ wrappers
def fp32_to_fp16(x: np.ndarray) -> np.ndarray:
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(flat.size, dtype=np.uint16)
    lib().g4o_fp32_to_fp16_n(_ptr(flat), _ptr(out), flat.size)
    return out.reshape(np.shape(x))


def fp16_to_fp32(h: np.ndarray) -> np.ndarray:
    flat = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(flat.size, dtype=np.float32)
    lib().g4o_fp16_to_fp32_n(_ptr(flat), _ptr(out), flat.size)
    return out.reshape(np.shape(h))


def quantize(qtype: int, x: np.ndarray, use_ref: bool = False) -> np.ndarray:
    """Quantize rows of x (shape [..., n]) to qtype; returns uint8 [rows, row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.reshape(-1, n)
    out = np.zeros((rows.shape[0], row_size(qtype, n)), dtype=np.uint8)
    name = {Q8_0: "q8_0", Q8_K: "q8_K", Q4_0: "q4_0"}[qtype]
    f = getattr(ref(), "g4_quantize_" + name) if use_ref else getattr(lib(), "g4o_quantize_" + name)
    for i in range(rows.shape[0]):
        f(rows[i].ctypes.data_as(_vp), out[i].ctypes.data_as(_vp), n)
    return out


def dequant(qtype: int, w: np.ndarray, n: int, use_ref: bool = False) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_size(qtype, n))
    out = np.zeros((w.shape[0], n), dtype=np.float32)
    for i in range(w.shape[0]):
        if use_ref:
            ref().g4_dequant_row(qtype, w[i].ctypes.data_as(_vp), out[i].ctypes.data_as(_vp), n)
        else:
            rc = lib().g4o_dequant_row(qtype, w[i].ctypes.data_as(_vp), out[i].ctypes.data_as(_vp), n)
            assert rc == 0
    return out


def n_sums_per_row(wtype: int, n: int) -> int:
    if wtype in (Q8_0, Q4_0):
        return n // 32
    if wtype in (Q2_K, Q4_K, Q5_K):
        return 2 * (n // 256)
    return n // 256


def block_sums(wtype: int, w: np.ndarray, a: np.ndarray, n: int) -> np.ndarray:
    """Per-block integer sums of every weight row against one activation row."""
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_size(wtype, n))
    a = np.ascontiguousarray(a, dtype=np.uint8).ravel()
    out = np.zeros((w.shape[0], n_sums_per_row(wtype, n)), dtype=np.int32)
    for i in range(w.shape[0]):
        lib().g4o_block_sums(wtype, w[i].ctypes.data_as(_vp), a.ctypes.data_as(_vp), n, out[i].ctypes.data_as(_vp))
    return out


def dot(wtype: int, w_row: np.ndarray, a_row: np.ndarray, n: int, kind: str = "avx2") -> float:
    """kind: 'avx2' (restated shipped order), 'ref' (restated scalar order),
    'refbuild' / 'refbuild_scalar' (the reference's own compiled kernels)."""
    wp, ap = _ptr(np.ascontiguousarray(w_row)), _ptr(np.ascontiguousarray(a_row))
    if kind == "avx2":
        return lib().g4o_dot(wtype, wp, ap, n)
    if kind == "ref":
        return lib().g4o_dot_ref(wtype, wp, ap, n)
    fn = getattr(ref(), "g4_dot_" + DOT_NAME[wtype] + ("" if kind == "refbuild" else "_ref"))
    return fn(wp, ap, n)


def matmul(wtype: int, W: np.ndarray, act: np.ndarray, ncols: int, nthreads: int = 1) -> np.ndarray:
    """Y[b][r] = dot(W[r], act[b]) with act rows at the 64-B padded stride."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    nrows = W.shape[0]
    st = act_stride(wtype, ncols)
    act = np.ascontiguousarray(act, dtype=np.uint8)
    nb = act.size // st
    Y = np.zeros((nb, nrows), dtype=np.float32)
    lib().g4o_matmul(wtype, _ptr(W), _ptr(act), st, _ptr(Y), ncols, nrows, nb, nthreads)
    return Y


def prep_act(wtype: int, x: np.ndarray) -> np.ndarray:
    """Quantize token rows x[nb][ncols] to the activation format at the padded stride."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb, ncols = x.reshape(-1, x.shape[-1]).shape
    st = act_stride(wtype, ncols)
    out = np.zeros((nb, st), dtype=np.uint8)
    lib().g4o_prep_act(wtype, _ptr(x), ncols, nb, _ptr(out))
    return out


def use_reference_dots(enable: bool) -> None:
    """Route the matmul driver through the reference build's AVX2 dots."""
    L = lib()
    for t, nm in DOT_NAME.items():
        fn = C.cast(getattr(ref(), "g4_dot_" + nm), _vp) if enable else None
        L.g4o_set_dot_fn(t, fn)
    L.g4o_set_dot_f16_fn(C.cast(ref().g4_dot_f16, _vp) if enable else None)


def pool_start(n: int) -> None:
    lib().g4o_pool_start(n)


def pool_stop() -> None:
    lib().g4o_pool_stop()


def rms_norm(x: np.ndarray, w, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    wp = _ptr(np.ascontiguousarray(w, dtype=np.float32)) if w is not None else None
    lib().g4o_rms_norm(_ptr(x), wp, _ptr(y), x.size, eps)
    return y


def rope(x: np.ndarray, pos: int, base: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    n = x.size
    cs = np.zeros(n, dtype=np.float32)
    lib().g4o_rope_cache(_ptr(cs), n, pos, base)
    lib().g4o_rope_apply(_ptr(x), _ptr(cs), n)
    return x


def gelu_table() -> np.ndarray:
    L = lib()
    return np.array([L.g4o_gelu_table_entry(i) for i in range(65536)], dtype=np.uint16)


_gelu_tab = None


def gelu(x: np.ndarray) -> np.ndarray:
    """g4o_gelu over an array: 0 for x <= -10, x for x >= 10, else the fp16
    table entry of fp16(x) (g4run.h:73-77, quants.c:49-58)."""
    global _gelu_tab
    if _gelu_tab is None:
        _gelu_tab = gelu_table()
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = fp16_to_fp32(_gelu_tab[fp32_to_fp16(x)])
    return np.where(x <= -10.0, np.float32(0.0), np.where(x >= 10.0, x, y)).astype(np.float32)


def attn_decode(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, kv_type: int, n_head: int,
                n_kv: int, hd: int, pos: int, nthreads: int = 1) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros((n_head, hd), dtype=np.float32)
    lib().g4o_attn_decode(_ptr(q), _ptr(np.ascontiguousarray(kc)), _ptr(np.ascontiguousarray(vc)),
                          kv_type, n_head, n_kv, hd, pos, _ptr(out), nthreads)
    return out


class _Model(C.Structure):
    _fields_ = [
        ("n_layer", C.c_int), ("n_embd", C.c_int), ("n_head", C.c_int), ("n_kv", C.c_int),
        ("hd", C.c_int), ("n_ff", C.c_int), ("n_vocab", C.c_int), ("n_ctx", C.c_int),
        ("rope_base", C.c_float), ("eps", C.c_float), ("kv_type", C.c_int), ("wtype", C.c_int),
        ("wqkv", C.POINTER(_vp)), ("wo", C.POINTER(_vp)), ("wgu", C.POINTER(_vp)), ("wdown", C.POINTER(_vp)),
        ("attn_norm", C.POINTER(_vp)), ("q_norm", C.POINTER(_vp)), ("k_norm", C.POINTER(_vp)),
        ("post_attn_norm", C.POINTER(_vp)), ("ffn_norm", C.POINTER(_vp)), ("post_ffw_norm", C.POINTER(_vp)),
        ("output_norm", _vp), ("head_type", C.c_int), ("head", _vp),
        ("kc", C.POINTER(_vp)), ("vc", C.POINTER(_vp)),
    ]


class Model:
    """CPU restatement of the synthetic gemma-style decoder.

    `w` is a dict of numpy arrays as produced by g4run_amd.model_weights():
    per-layer lists 'wqkv', 'wo', 'wgu', 'wdown' (uint8 rows) and the norm
    vectors, plus 'head' and 'output_norm'.  KV caches are numpy arrays owned
    here ([n_layer][n_ctx*n_kv*row_bytes]).
    """

    def __init__(self, cfg: dict, w: dict, kc: list, vc: list):
        self.cfg, self.w, self.kc, self.vc = cfg, w, kc, vc
        L = cfg["n_layer"]

        def arr(lst):
            a = (_vp * L)(*[x.ctypes.data_as(_vp) for x in lst])
            return a

        self._keep = []
        m = _Model()
        for k in ("n_layer", "n_embd", "n_head", "n_kv", "hd", "n_ff", "n_vocab", "n_ctx"):
            setattr(m, k, cfg[k])
        m.rope_base, m.eps, m.kv_type, m.wtype = cfg["rope_base"], cfg["eps"], cfg["kv_type"], cfg["wtype"]
        for k in ("wqkv", "wo", "wgu", "wdown", "attn_norm", "q_norm", "k_norm",
                  "post_attn_norm", "ffn_norm", "post_ffw_norm"):
            a = arr(w[k])
            self._keep.append(a)
            setattr(m, k, C.cast(a, C.POINTER(_vp)))
        m.output_norm = w["output_norm"].ctypes.data_as(_vp)
        m.head_type = cfg["head_type"]
        m.head = w["head"].ctypes.data_as(_vp)
        for k, lst in (("kc", kc), ("vc", vc)):
            a = arr(lst)
            self._keep.append(a)
            setattr(m, k, C.cast(a, C.POINTER(_vp)))
        self._m = m
        self._scratch = np.zeros(lib().g4o_model_scratch_bytes(C.byref(m)), dtype=np.uint8)

    def embed(self, token: int) -> np.ndarray:
        x = np.zeros(self.cfg["n_embd"], dtype=np.float32)
        lib().g4o_model_embed(C.byref(self._m), token, _ptr(x))
        return x

    def layer(self, il: int, pos: int, x: np.ndarray, nthreads: int = 1) -> np.ndarray:
        """Layer il at pos applied to a copy of x (stores its K/V rows)."""
        y = np.ascontiguousarray(x, dtype=np.float32).copy()
        lib().g4o_model_layer(C.byref(self._m), il, pos, _ptr(y), _ptr(self._scratch), nthreads)
        return y

    def qkv(self, il: int, x: np.ndarray, nthreads: int = 1) -> np.ndarray:
        c = self.cfg
        out = np.zeros((c["n_head"] + 2 * c["n_kv"]) * c["hd"], dtype=np.float32)
        lib().g4o_model_qkv(C.byref(self._m), il, _ptr(np.ascontiguousarray(x, dtype=np.float32)), _ptr(out),
                            _ptr(self._scratch), nthreads)
        return out

    def attn(self, il: int, pos: int, qkv: np.ndarray, nthreads: int = 1, prepared: bool = False):
        """Prepare q/k/v from the projection output (a copy), store K/V at pos,
        attend; returns the attention output [n_head * hd] (and, with
        prepared=True, the prepared q|k|v rows as well)."""
        c = self.cfg
        q = np.ascontiguousarray(qkv, dtype=np.float32).copy()
        out = np.zeros(c["n_head"] * c["hd"], dtype=np.float32)
        lib().g4o_model_attn(C.byref(self._m), il, pos, _ptr(q), _ptr(out), _ptr(self._scratch), nthreads)
        return (out, q) if prepared else out

    def post(self, il: int, x: np.ndarray, att: np.ndarray, nthreads: int = 1) -> np.ndarray:
        y = np.ascontiguousarray(x, dtype=np.float32).copy()
        lib().g4o_model_post(C.byref(self._m), il, _ptr(y), _ptr(np.ascontiguousarray(att, dtype=np.float32)),
                             _ptr(self._scratch), nthreads)
        return y

    def head(self, x: np.ndarray, nthreads: int = 1):
        logits = np.zeros(self.cfg["n_vocab"], dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        tok = lib().g4o_model_head(C.byref(self._m), _ptr(x), _ptr(logits), _ptr(self._scratch), nthreads)
        return tok, logits

    def decode(self, token: int, pos: int, nthreads: int = 1):
        logits = np.zeros(self.cfg["n_vocab"], dtype=np.float32)
        tok = lib().g4o_model_decode(C.byref(self._m), token, pos, _ptr(logits), _ptr(self._scratch), nthreads)
        return tok, logits


# ------------------------------------------------------------------ sampler
REF_SAMPLER_PATH = os.path.join(HERE, "_ref", "libg4refsampler.so")


class SamplerStruct(C.Structure):
    """g4_sampler as laid out by g4run.h:464-482 (and g4o_sampler)."""
    _fields_ = [("temp", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("repeat_last_n", C.c_int), ("freq_penalty", C.c_float), ("presence_penalty", C.c_float),
                ("no_repeat_ngram", C.c_int), ("seed", C.c_uint64), ("rng", C.c_uint64 * 4),
                ("recent", C.POINTER(C.c_int)), ("recent_cap", C.c_int), ("recent_n", C.c_int),
                ("recent_head", C.c_int), ("cnt", C.POINTER(C.c_int)), ("ban_ids", C.POINTER(C.c_int)),
                ("n_ban", C.c_int), ("ban_cap", C.c_int), ("n_vocab", C.c_int)]


_ref_sampler = None


def ref_sampler_available() -> bool:
    return os.path.exists(REF_SAMPLER_PATH)


def _sampler_lib(use_ref: bool):
    global _ref_sampler
    if not use_ref:
        L = lib()
        names = {"init": L.g4o_sampler_init, "reset": L.g4o_sampler_reset, "free": L.g4o_sampler_free,
                 "ban": L.g4o_sampler_ban, "accept": L.g4o_sampler_accept, "sample": L.g4o_sample}
    else:
        if _ref_sampler is None:
            _ref_sampler = C.CDLL(REF_SAMPLER_PATH)
        R = _ref_sampler
        names = {"init": R.g4_sampler_init, "reset": R.g4_sampler_reset, "free": R.g4_sampler_free,
                 "ban": R.g4_sampler_ban, "accept": R.g4_sampler_accept, "sample": R.g4_sample}
    P = C.POINTER(SamplerStruct)
    names["init"].argtypes = [P, C.c_int]
    names["reset"].argtypes = [P]
    names["free"].argtypes = [P]
    names["ban"].argtypes = [P, C.c_int]
    names["accept"].argtypes = [P, C.c_int]
    names["sample"].argtypes = [P, _vp]
    names["sample"].restype = C.c_int
    for f in ("init", "reset", "free", "ban", "accept"):
        names[f].restype = None
    return names


class Sampler:
    """The sampling chain of sampler.c: the restatement (default) or, with
    use_ref=True, the reference's sampler.c built in oracle/_ref."""
    PARAMS = ("temp", "top_k", "top_p", "repeat_penalty", "repeat_last_n", "freq_penalty", "presence_penalty",
              "no_repeat_ngram", "seed")

    def __init__(self, n_vocab: int, use_ref: bool = False, **params):
        self._f = _sampler_lib(use_ref)
        self.s = SamplerStruct()
        self._f["init"](C.byref(self.s), n_vocab)
        for k, v in params.items():
            if k not in self.PARAMS:
                raise KeyError(k)
            setattr(self.s, k, v)

    def __del__(self):
        try:
            self._f["free"](C.byref(self.s))
        except Exception:
            pass

    def ban(self, tok: int) -> None:
        self._f["ban"](C.byref(self.s), int(tok))

    def accept(self, tok: int) -> None:
        self._f["accept"](C.byref(self.s), int(tok))

    def reset(self) -> None:
        self._f["reset"](C.byref(self.s))

    def sample(self, logits: np.ndarray) -> int:
        """Draw from logits (float32, rewritten in place as the reference does)."""
        assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"] and logits.size == self.s.n_vocab
        return int(self._f["sample"](C.byref(self.s), _ptr(logits)))

    @property
    def rng(self):
        return [int(self.s.rng[i]) for i in range(4)]

    def recent(self):
        """The accepted ids in the ring, oldest first."""
        s = self.s
        return [s.recent[(s.recent_head + i) % s.recent_cap] for i in range(s.recent_n)]


# ------------------------------------------------------------------- gemma4
class _Mat(C.Structure):
    _fields_ = [("data", _vp), ("type", C.c_int), ("ncols", _i64), ("nrows", _i64)]


class _GemmaLayer(C.Structure):
    _fields_ = [(n, _Mat) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down", "inp_gate", "proj")] + \
               [(n, _vp) for n in ("attn_norm", "q_norm", "k_norm", "post_attn_norm", "ffn_norm", "post_ffw_norm",
                                   "post_norm")] + [("out_scale", C.c_float)]


class _Gemma(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_layer_kv", "n_embd", "n_head", "n_vocab", "n_embd_per_layer",
                                       "hd_full", "hd_swa", "n_swa", "n_ctx")] + \
               [(n, C.c_float) for n in ("rope_base_full", "rope_base_swa", "eps", "softcap")] + \
               [("is_swa", _vp), ("n_ff", _vp), ("kv_type", C.c_int),
                ("tok_embd", _Mat), ("per_layer_tok_embd", _Mat), ("per_layer_model_proj", _Mat),
                ("per_layer_proj_norm", _vp), ("output_norm", _vp), ("rope_freqs", _vp),
                ("layers", _vp), ("kc", _vp), ("vc", _vp)]


class Gemma:
    """The gemma4 forward of model.c:592-799 (oracle/g4o_gemma.c) over GGUF
    tensors given by name: {name: (ggml_type, ne list, raw bytes as uint8 or
    float32 array)}; hp uses g4_model_file's field names."""

    def __init__(self, hp: dict, tensors: dict, kv_type: int, n_ctx: int):
        L = lib()
        L.g4o_gemma_forward.argtypes = [_vp, _vp, C.c_int, C.c_int, _vp, _vp, C.c_int]
        L.g4o_gemma_forward.restype = None
        L.g4o_gemma_cache_bytes.argtypes = [_vp, C.c_int]
        L.g4o_gemma_cache_bytes.restype = C.c_size_t
        self.hp, self._keep = hp, []

        def arr(a, dt):
            a = np.ascontiguousarray(a, dtype=dt)
            self._keep.append(a)
            return a

        def mat(name):
            m = _Mat()
            if name not in tensors:
                return m
            t, ne, raw = tensors[name]
            a = arr(np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.uint8), np.uint8)
            m.data, m.type, m.ncols, m.nrows = a.ctypes.data, t, ne[0], ne[1] if len(ne) > 1 else 1
            return m

        def vec(name):
            if name not in tensors:
                return None
            return arr(np.frombuffer(np.ascontiguousarray(tensors[name][2]).tobytes(), np.float32), np.float32).ctypes.data

        nl = hp["n_layer"]
        layers = (_GemmaLayer * nl)()
        for il in range(nl):
            p = f"blk.{il}."
            ly = layers[il]
            for f, n in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"), ("gate", "ffn_gate"),
                         ("up", "ffn_up"), ("down", "ffn_down"), ("inp_gate", "inp_gate"), ("proj", "proj")):
                setattr(ly, f, mat(p + n + ".weight"))
            for f, n in (("attn_norm", "attn_norm"), ("q_norm", "attn_q_norm"), ("k_norm", "attn_k_norm"),
                         ("post_attn_norm", "post_attention_norm"), ("ffn_norm", "ffn_norm"),
                         ("post_ffw_norm", "post_ffw_norm"), ("post_norm", "post_norm")):
                setattr(ly, f, vec(p + n + ".weight"))
            sc = p + "layer_output_scale.weight"
            ly.out_scale = float(np.frombuffer(np.ascontiguousarray(tensors[sc][2]).tobytes(), np.float32)[0]) \
                if sc in tensors else 1.0
        self._layers = layers
        g = _Gemma()
        for f in ("n_layer", "n_layer_kv", "n_embd", "n_head", "n_vocab", "n_embd_per_layer", "n_swa"):
            setattr(g, f, hp[f])
        g.hd_full, g.hd_swa, g.n_ctx = hp["head_dim_full"], hp["head_dim_swa"], n_ctx
        g.rope_base_full, g.rope_base_swa = hp["rope_base_full"], hp["rope_base_swa"]
        g.eps, g.softcap = hp["rms_eps"], hp.get("final_softcap", 0.0)
        g.is_swa = arr(hp["is_swa"][:nl], np.uint8).ctypes.data
        g.n_ff = arr(hp["n_ff"][:nl], np.int32).ctypes.data
        g.kv_type = kv_type
        g.tok_embd, g.per_layer_tok_embd = mat("token_embd.weight"), mat("per_layer_token_embd.weight")
        g.per_layer_model_proj = mat("per_layer_model_proj.weight")
        g.per_layer_proj_norm, g.output_norm = vec("per_layer_proj_norm.weight"), vec("output_norm.weight")
        g.rope_freqs = vec("rope_freqs.weight")
        g.layers = C.cast(layers, _vp)
        self._g = g
        nkv = hp["n_layer_kv"]
        self.kc = [np.zeros(L.g4o_gemma_cache_bytes(C.byref(g), il), np.uint8) for il in range(nkv)]
        self.vc = [np.zeros(L.g4o_gemma_cache_bytes(C.byref(g), il), np.uint8) for il in range(nkv)]
        self._kp = (_vp * max(nkv, 1))(*[a.ctypes.data for a in self.kc])
        self._vp_ = (_vp * max(nkv, 1))(*[a.ctypes.data for a in self.vc])
        g.kc, g.vc = C.cast(self._kp, _vp), C.cast(self._vp_, _vp)

    def forward(self, tokens, pos0: int, nthreads: int = 1):
        """(logits [nb][n_vocab], hnext [nb][n_embd]) of every position."""
        t = np.ascontiguousarray(tokens, np.int32)
        nb = t.size
        logits = np.zeros((nb, self.hp["n_vocab"]), np.float32)
        hn = np.zeros((nb, self.hp["n_embd"]), np.float32)
        lib().g4o_gemma_forward(C.byref(self._g), _ptr(t), nb, pos0, _ptr(logits), _ptr(hn), nthreads)
        return logits, hn
