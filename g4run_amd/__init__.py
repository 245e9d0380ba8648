"""g4run_amd -- MI355X (gfx950) implementation of g4run's quantized
weight x activation hot path, reached through the C ABI of include/g4hip.h.

This module is a thin ctypes front end over g4run_amd/libg4hip.so (built by
g4run_amd/build.py).  It has no CPU fallback: importing it without the built
library, or calling it without a gfx950 device, raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# G4H_LIB names another build of the same library (e.g. one compiled with
# different flags for a side-by-side measurement)
LIB_PATH = os.environ.get("G4H_LIB") or os.path.join(HERE, "libg4hip.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include", "g4hip.h")

# type ids (g4run.h:80-94)
F32, F16, Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, BF16, TQ2_0 = 0, 1, 2, 8, 10, 11, 12, 13, 14, 15, 30, 35
BLCK = {F32: 1, F16: 1, BF16: 1, Q4_0: 32, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256,
        TQ2_0: 256}
SIZE = {F32: 4, F16: 2, BF16: 2, Q4_0: 18, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292, TQ2_0: 66}
TYPE_NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q2_K: "q2_K", Q3_K: "q3_K", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K",
              TQ2_0: "tq2_0", F16: "f16", BF16: "bf16", F32: "f32"}

OK, ERR_ARG, ERR_TYPE, ERR_SHAPE, ERR_NOMEM, ERR_DEVICE, ERR_HIP, ERR_TIMEOUT = range(8)
# g4h_model_status flags
STATUS_CTX_FULL, STATUS_ATTN_TIMEOUT = 1, 2

_vp, _i64, _sz, _int = C.c_void_p, C.c_int64, C.c_size_t, C.c_int


class G4HError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


# (name, restype, argtypes) for every entry point of include/g4hip.h
_SIGS = [
    ("g4h_init", _int, [_int]),
    ("g4h_last_error", C.c_char_p, []),
    ("g4h_status_str", C.c_char_p, [_int]),
    ("g4h_debug_fail_alloc", None, [_int]),
    ("g4h_debug_attn_timeout", None, [_int]),
    ("g4h_malloc", _int, [C.POINTER(_vp), _sz]),
    ("g4h_free", _int, [_vp]),
    ("g4h_memcpy_h2d", _int, [_vp, _vp, _sz, _vp]),
    ("g4h_memcpy_d2h", _int, [_vp, _vp, _sz, _vp]),
    ("g4h_memcpy_d2d", _int, [_vp, _vp, _sz, _vp]),
    ("g4h_memset", _int, [_vp, _int, _sz, _vp]),
    ("g4h_stream_create", _int, [C.POINTER(_vp)]),
    ("g4h_stream_destroy", _int, [_vp]),
    ("g4h_stream_synchronize", _int, [_vp]),
    ("g4h_event_create", _int, [C.POINTER(_vp)]),
    ("g4h_event_destroy", _int, [_vp]),
    ("g4h_event_record", _int, [_vp, _vp]),
    ("g4h_event_elapsed_ms", _int, [C.POINTER(C.c_float), _vp, _vp]),
    ("g4h_graph_begin", _int, [_vp]),
    ("g4h_graph_end", _int, [_vp, C.POINTER(_vp)]),
    ("g4h_graph_launch", _int, [_vp, _vp]),
    ("g4h_graph_destroy", _int, [_vp]),
    ("g4h_row_size", _sz, [_int, _i64]),
    ("g4h_act_type", _int, [_int]),
    ("g4h_act_stride", _sz, [_int, _i64]),
    ("g4h_quantize_q8_0", _int, [_vp, _sz, _vp, _sz, _i64, _int, _vp]),
    ("g4h_quantize_q8_K", _int, [_vp, _sz, _vp, _sz, _i64, _int, _vp]),
    ("g4h_quantize_q4_0", _int, [_vp, _sz, _vp, _sz, _i64, _int, _vp]),
    ("g4h_dequant_rows", _int, [_int, _vp, _sz, _vp, _sz, _i64, _int, _vp]),
    ("g4h_vec_dot", _int, [_int, _vp, _sz, _vp, _i64, _int, _vp, _vp]),
    ("g4h_tensor_create", _int, [_int, _i64, _i64, C.POINTER(_vp)]),
    ("g4h_tensor_load", _int, [_vp, _vp, _int, _vp]),
    ("g4h_tensor_store", _int, [_vp, _vp, _vp]),
    ("g4h_tensor_free", _int, [_vp]),
    ("g4h_tensor_bytes", _sz, [_vp]),
    ("g4h_tensor_info", _int, [_vp, C.POINTER(_int), C.POINTER(_i64), C.POINTER(_i64)]),
    ("g4h_matmul", _int, [_vp, _vp, _vp, _sz, _vp, _int, _vp]),
    ("g4h_matmul_ex", _int, [_vp, _vp, _vp, _sz, _vp, _int, _int, _vp]),
    ("g4h_matmul_path", _int, [_vp, _int]),
    ("g4h_matmul_noalloc", _int, [_vp, _vp, _vp, _sz, _vp, _int, _int, _vp]),
    ("g4h_matmul_noalloc_max_bytes", _sz, []),
    ("g4h_matmul_describe", _int, [_vp, _int, _int, C.c_char_p, C.c_size_t]),
    ("g4h_block_sums", _int, [_vp, _vp, _sz, _int, _vp, _vp]),
    ("g4h_attn_workspace_bytes", _sz, [_int, _int, _int]),
    ("g4h_attn_passes", _int, [_int, _int, _int, _int, _int, C.POINTER(_int)]),
    ("g4h_attn_decode", _int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _vp, _vp, _sz, _vp]),
    ("g4h_attn_status", _int, [_vp, C.POINTER(_int), _vp]),
    ("g4h_attn_decode_window", _int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int, _int, _vp, _vp, _sz, _vp]),
    ("g4h_attn_prefill", _int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int, _vp, _vp, _sz, _vp]),
    ("g4h_attn_prefill_workspace_bytes", _sz, [_int, _int, _int, _int]),
    ("g4h_kv_store", _int, [_int, _vp, _vp, _int, _int, _sz, _vp]),
    ("g4h_model_create", _int, [_vp, C.c_uint64, C.POINTER(_vp)]),
    ("g4h_model_free", _int, [_vp]),
    ("g4h_model_fill_kv", _int, [_vp, C.c_uint64, _vp]),
    ("g4h_forward", _int, [_vp, _int, _int, C.POINTER(_int), _vp]),
    ("g4h_forward_state", _int, [_vp, _vp]),
    ("g4h_model_set_state", _int, [_vp, _int, _int, _vp]),
    ("g4h_model_get_state", _int, [_vp, C.POINTER(_int), C.POINTER(_int), _vp]),
    ("g4h_model_status", _int, [_vp, C.POINTER(_int), _vp]),
    ("g4h_model_gelu_table", _vp, [_vp]),
    ("g4h_model_trace", _int, [_vp, _vp]),
    ("g4h_model_logits", _vp, [_vp]),
    ("g4h_model_matrix", _vp, [_vp, _int, _int]),
    ("g4h_model_norm", _vp, [_vp, _int, _int]),
    ("g4h_model_kv", _int, [_vp, _int, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_sz)]),
    ("g4h_model_weight_bytes", _sz, [_vp]),
    ("g4h_sampler_default_params", None, [_vp]),
    ("g4h_sampler_create", _int, [_int, _vp, C.POINTER(_vp)]),
    ("g4h_sampler_free", _int, [_vp]),
    ("g4h_sampler_set_params", _int, [_vp, _vp, _vp]),
    ("g4h_sampler_set_rng", _int, [_vp, C.POINTER(C.c_uint64), _vp]),
    ("g4h_sampler_reset", _int, [_vp, _vp]),
    ("g4h_sampler_ban", _int, [_vp, _int, _vp]),
    ("g4h_sampler_accept", _int, [_vp, C.POINTER(_int), _int, _vp]),
    ("g4h_sample", _int, [_vp, _vp, _vp, _int, _vp]),
    ("g4h_sampler_get_state", _int, [_vp, C.POINTER(C.c_uint64), C.POINTER(_int), C.POINTER(_int), C.POINTER(_int),
                                     _vp]),
    ("g4h_model_set_sampler", _int, [_vp, _vp]),
    ("g4h_forward_batch", _int, [_vp, C.POINTER(_int), _int, _int, _int, _vp]),
    ("g4h_forward_batch_heads", _int, [_vp, C.POINTER(_int), _int, _int, _vp, _vp, _vp]),
    ("g4h_argmax_rows", _int, [_vp, _int, _int, _vp, _vp]),
    ("g4h_gemma_create", _int, [_vp, _int, _int, C.POINTER(_vp)]),
    ("g4h_gemma_open", _int, [C.c_char_p, _int, _int, C.POINTER(_vp)]),
    ("g4h_gemma_free", _int, [_vp]),
    ("g4h_gemma_info", _int, [_vp, C.POINTER(_int), C.POINTER(_int), C.POINTER(_int), C.POINTER(_int)]),
    ("g4h_gemma_forward", _int, [_vp, C.POINTER(_int), _int, _int, _vp, _vp, _vp]),
    ("g4h_attn_prefill_mm", _int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int, _int, _int, _vp, _vp, _sz, _vp]),
    ("g4h_gemma_prefill", _int, [_vp, C.POINTER(_int), _int, _int, _vp, _vp]),
    ("g4h_read_floor", _int, [_vp, _sz, _vp, C.c_int64, _int, _int, _vp]),
    ("g4h_gemma_trace", _int, [_vp, _vp, C.POINTER(_sz)]),
    ("g4h_gemma_set_state", _int, [_vp, _int, _int, _vp]),
    ("g4h_gemma_step", _int, [_vp, _vp]),
    ("g4h_gemma_get_state", _int, [_vp, C.POINTER(_int), C.POINTER(_int), _vp]),
    ("g4h_gemma_status", _int, [_vp, C.POINTER(_int), _vp]),
    ("g4h_gemma_logits", _vp, [_vp]),
    ("g4h_gemma_kv", _int, [_vp, _int, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_sz)]),
]

_lib = None


def exported_names():
    return [s[0] for s in _SIGS]


def lib():
    """Load libg4hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python -c 'import __graft_entry__ as g; g.build()'` "
                              "(the HIP library has no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise G4HError(rc, lib().g4h_last_error().decode())


_inited = False


def init(device: int = 0) -> None:
    global _inited
    if not _inited:
        check(lib().g4h_init(device))
        _inited = True


def row_size(t: int, n: int) -> int:
    return lib().g4h_row_size(t, n)


def act_type(wtype: int) -> int:
    return lib().g4h_act_type(wtype)


def act_stride(wtype: int, ncols: int) -> int:
    return lib().g4h_act_stride(wtype, ncols)


# --------------------------------------------------------------- plumbing
class Buffer:
    """A device allocation owned by Python."""

    def __init__(self, nbytes: int):
        init()
        p = _vp()
        check(lib().g4h_malloc(C.byref(p), int(nbytes)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray, stream=None) -> "Buffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a, stream)
        return b

    def upload(self, a: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().g4h_memcpy_h2d(self.ptr, a.ctypes.data_as(_vp), a.nbytes, stream))
        check(lib().g4h_stream_synchronize(stream))

    def download(self, dtype, shape, offset: int = 0, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().g4h_memcpy_d2h(out.ctypes.data_as(_vp), self.ptr + offset, out.nbytes, stream))
        return out

    def zero(self, stream=None) -> None:
        check(lib().g4h_memset(self.ptr, 0, self.nbytes, stream))

    def free(self) -> None:
        if self.ptr:
            check(lib().g4h_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize(stream=None) -> None:
    check(lib().g4h_stream_synchronize(stream))


class Stream:
    def __init__(self):
        init()
        p = _vp()
        check(lib().g4h_stream_create(C.byref(p)))
        self.ptr = p.value

    def synchronize(self):
        check(lib().g4h_stream_synchronize(self.ptr))


class Event:
    def __init__(self):
        p = _vp()
        check(lib().g4h_event_create(C.byref(p)))
        self.ptr = p.value

    def record(self, stream=None):
        check(lib().g4h_event_record(self.ptr, stream))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().g4h_event_elapsed_ms(C.byref(ms), self.ptr, end.ptr))
        return ms.value


class Graph:
    """Stream capture of a sequence of library calls, replayed with launch()."""

    def __init__(self, stream, fn):
        check(lib().g4h_graph_begin(stream))
        try:
            fn()
        finally:
            p = _vp()
            check(lib().g4h_graph_end(stream, C.byref(p)))
        self.ptr = p.value

    def launch(self, stream):
        check(lib().g4h_graph_launch(self.ptr, stream))

    def __del__(self):
        try:
            if self.ptr:
                lib().g4h_graph_destroy(self.ptr)
        except Exception:
            pass


# ------------------------------------------------------------------ ops
def quantize(qtype: int, x: Buffer, n: int, rows: int, y: Buffer, x_stride: int = 0, y_stride: int = 0, stream=None) -> None:
    """g4_quantize_q8_0 / q8_K / q4_0 on device rows."""
    fn = {Q8_0: lib().g4h_quantize_q8_0, Q8_K: lib().g4h_quantize_q8_K, Q4_0: lib().g4h_quantize_q4_0}[qtype]
    check(fn(x.ptr if isinstance(x, Buffer) else x, x_stride or n,
             y.ptr if isinstance(y, Buffer) else y, y_stride or row_size(qtype, n), n, rows, stream))


def dequant_rows(qtype: int, x, n: int, rows: int, y, x_stride: int = 0, y_stride: int = 0, stream=None) -> None:
    check(lib().g4h_dequant_rows(qtype, _p(x), x_stride or row_size(qtype, n), _p(y), y_stride or n, n, rows, stream))


def vec_dot(wtype: int, w, a, n: int, rows: int, out, w_stride: int = 0, stream=None) -> None:
    check(lib().g4h_vec_dot(wtype, _p(w), w_stride or row_size(wtype, n), _p(a), n, rows, _p(out), stream))


def _p(x):
    return x.ptr if isinstance(x, (Buffer, Tensor)) else x


class Tensor:
    """Weight matrix resident in HBM (g4h_tensor)."""

    def __init__(self, qtype: int, ncols: int, nrows: int):
        init()
        p = _vp()
        check(lib().g4h_tensor_create(qtype, ncols, nrows, C.byref(p)))
        self.ptr = p.value
        self.type, self.ncols, self.nrows = qtype, ncols, nrows

    @classmethod
    def from_rows(cls, qtype: int, rows: np.ndarray, ncols: int, stream=None) -> "Tensor":
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        rs = row_size(qtype, ncols)
        assert rows.size % rs == 0
        t = cls(qtype, ncols, rows.size // rs)
        check(lib().g4h_tensor_load(t.ptr, rows.ctypes.data_as(_vp), 0, stream))
        return t

    def load_device(self, rows_dev, stream=None) -> None:
        check(lib().g4h_tensor_load(self.ptr, _p(rows_dev), 1, stream))

    def to_rows(self) -> np.ndarray:
        rs = row_size(self.type, self.ncols)
        b = Buffer(rs * self.nrows)
        check(lib().g4h_tensor_store(self.ptr, b.ptr, None))
        return b.download(np.uint8, (self.nrows, rs))

    @property
    def nbytes(self) -> int:
        return lib().g4h_tensor_bytes(self.ptr)

    def free(self):
        if self.ptr:
            check(lib().g4h_tensor_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def matmul(W: Tensor, Y, nb: int = 1, x=None, pre=None, pre_stride: int = 0, path: int = 0, stream=None) -> None:
    """matmul_b: Y[nb][nrows] = W @ act, act from x (fp32, quantized here) or pre."""
    check(lib().g4h_matmul_ex(W.ptr, _p(x) if x is not None else None, _p(pre) if pre is not None else None,
                              pre_stride or (act_stride(W.type, W.ncols) if pre is not None else 0),
                              _p(Y), nb, path, stream))


def matmul_path(W: Tensor, nb: int) -> int:
    """Kernel family g4h_matmul picks for nb tokens: 1 GEMV, 2 int8 matrix cores."""
    return lib().g4h_matmul_path(W.ptr, nb)


def matmul_describe(W: Tensor, nb: int = 1, path: int = 0) -> str:
    """Kernel instantiation and launch shape of g4h_matmul_ex for nb tokens."""
    buf = C.create_string_buffer(256)
    check(lib().g4h_matmul_describe(W.ptr, nb, path, buf, 256))
    return buf.value.decode()


def read_floor(src, nbytes: int, y=None, ny: int = 0, threads: int = 256, loads: int = 1, stream=None) -> None:
    """One launch that only reads nbytes of src (128-bit non-temporal loads)
    and writes ny floats of y: the yardstick a GEMV launch is timed against."""
    check(lib().g4h_read_floor(_p(src), nbytes, _p(y) if y is not None else None, ny, threads, loads, stream))


def block_sums(W: Tensor, pre, out, tok: int = 0, pre_stride: int = 0, stream=None) -> None:
    check(lib().g4h_block_sums(W.ptr, _p(pre), pre_stride or act_stride(W.type, W.ncols), tok, _p(out), stream))


def n_block_sums(W: Tensor) -> int:
    nb = W.ncols // BLCK[W.type]
    return nb * (2 if W.type in (Q2_K, Q4_K, Q5_K) else 1)


# ----------------------------------------------------------------- attention
def attn_workspace_bytes(n_head: int, hd: int, n_pos: int) -> int:
    return lib().g4h_attn_workspace_bytes(n_head, hd, n_pos)


def attn_passes(kv_type: int, n_head: int, n_kv: int, hd: int, n_pos: int) -> int:
    """1 when this shape runs as one fused launch, 3 for the three-pass form."""
    n = _int()
    check(lib().g4h_attn_passes(kv_type, n_head, n_kv, hd, n_pos, C.byref(n)))
    return n.value


def attn_decode(q, kc, vc, kv_type: int, n_head: int, n_kv: int, hd: int, n_pos: int, out, ws=None, stream=None) -> None:
    """attn_kernel for one decode token over cached positions [0, n_pos)."""
    need = attn_workspace_bytes(n_head, hd, n_pos)
    if ws is None:
        ws = Buffer(need)
    check(lib().g4h_attn_decode(_p(q), _p(kc), _p(vc), kv_type, n_head, n_kv, hd, n_pos, _p(out), _p(ws),
                                ws.nbytes if isinstance(ws, Buffer) else need, stream))


def attn_decode_window(q, kc, vc, kv_type: int, n_head: int, n_kv: int, hd: int, n_pos: int, window: int, ring: int, out,
                       ws=None, stream=None) -> None:
    """attn_kernel with a sliding window over a (doubled) KV ring."""
    rows = window if 0 < window < n_pos else n_pos
    need = attn_workspace_bytes(n_head, hd, rows)
    if ws is None:
        ws = Buffer(need)
    check(lib().g4h_attn_decode_window(_p(q), _p(kc), _p(vc), kv_type, n_head, n_kv, hd, n_pos, window, ring, _p(out),
                                       _p(ws), ws.nbytes if isinstance(ws, Buffer) else need, stream))


def attn_status(ws, stream=None) -> bool:
    """True if an attention call on ws had a hand-off wait give up since the
    last query (its outputs are NaN); clears the flag."""
    f = _int()
    check(lib().g4h_attn_status(_p(ws), C.byref(f), stream))
    return bool(f.value)


def debug_attn_timeout(on: bool) -> None:
    """Test hook: every attention hand-off wait gives up (bounded), or normal operation."""
    lib().g4h_debug_attn_timeout(1 if on else 0)


def attn_prefill_workspace_bytes(n_head: int, hd: int, pos0: int, nb: int) -> int:
    return lib().g4h_attn_prefill_workspace_bytes(n_head, hd, pos0, nb)


def attn_prefill_mm(q, kc, vc, kv_type: int, n_head: int, n_kv: int, hd: int, pos0: int, nb: int, out, window: int = 0,
                    ring: int = 0, ws=None, stream=None) -> None:
    """g4h_attn_prefill_mm: the prompt batch's attention on the matrix cores."""
    need = attn_prefill_workspace_bytes(n_head, hd, pos0, nb)
    if ws is None:
        ws = Buffer(need)
    check(lib().g4h_attn_prefill_mm(_p(q), _p(kc), _p(vc), kv_type, n_head, n_kv, hd, pos0, nb, window, ring, _p(out),
                                    _p(ws), ws.nbytes if isinstance(ws, Buffer) else need, stream))


def attn_prefill(q, kc, vc, kv_type: int, n_head: int, n_kv: int, hd: int, pos0: int, nb: int, out, ws=None,
                 stream=None, batched: bool = True) -> None:
    """attn_kernel for nb new tokens at positions pos0.. (causal): one set of
    launches for the whole batch, or (batched=False, a smaller workspace) one
    decode launch per token."""
    need = attn_prefill_workspace_bytes(n_head, hd, pos0, nb) if batched else attn_workspace_bytes(n_head, hd, pos0 + nb)
    if ws is None:
        ws = Buffer(need)
    check(lib().g4h_attn_prefill(_p(q), _p(kc), _p(vc), kv_type, n_head, n_kv, hd, pos0, nb, _p(out), _p(ws),
                                 ws.nbytes if isinstance(ws, Buffer) else need, stream))


def kv_store(kv_type: int, src, dst, hd: int, rows: int = 1, dst_stride: int = 0, stream=None) -> None:
    check(lib().g4h_kv_store(kv_type, _p(src), _p(dst), hd, rows, dst_stride, stream))


# ---------------------------------------------------------------- decode step
class ModelConfig(C.Structure):
    _fields_ = [("n_layer", _int), ("n_embd", _int), ("n_head", _int), ("n_kv", _int), ("head_dim", _int),
                ("n_ff", _int), ("n_vocab", _int), ("n_ctx", _int), ("rope_base", C.c_float), ("rms_eps", C.c_float),
                ("wtype", _int), ("head_type", _int), ("kv_type", _int)]


# 26 layers, d_model 2560, 8 q heads / 4 KV heads of
# 256, gated-GELU FFN 10240, RoPE theta 1e6, q4_0 weights, q8_0 vocab-32768
# head, f16 KV cache of 8192 positions
GEMMA_STYLE = dict(n_layer=26, n_embd=2560, n_head=8, n_kv=4, head_dim=256, n_ff=10240, n_vocab=32768, n_ctx=8192,
                   rope_base=1e6, rms_eps=1e-6, wtype=Q4_0, head_type=Q8_0, kv_type=F16)

_MATS = {"wqkv": 0, "wo": 1, "wgu": 2, "wdown": 3}
_NORMS = {"attn_norm": 0, "q_norm": 1, "k_norm": 2, "post_attn_norm": 3, "ffn_norm": 4, "post_ffw_norm": 5}


class _View:
    """A borrowed device tensor (owned by the model)."""

    def __init__(self, ptr):
        self.ptr = ptr
        t, nc, nr = _int(), _i64(), _i64()
        check(lib().g4h_tensor_info(ptr, C.byref(t), C.byref(nc), C.byref(nr)))
        self.type, self.ncols, self.nrows = t.value, nc.value, nr.value

    def to_rows(self) -> np.ndarray:
        rs = row_size(self.type, self.ncols)
        b = Buffer(rs * self.nrows)
        check(lib().g4h_tensor_store(self.ptr, b.ptr, None))
        return b.download(np.uint8, (self.nrows, rs))


class Gemma:
    """A gemma4 GGUF model resident on the device (g4h_gemma)."""

    def __init__(self, path: str, n_ctx: int = 8192, kv_type: int = F16):
        init()
        p = _vp()
        check(lib().g4h_gemma_open(str(path).encode(), n_ctx, kv_type, C.byref(p)))
        self.ptr = p.value
        v, e, nl, nc = _int(), _int(), _int(), _int()
        check(lib().g4h_gemma_info(self.ptr, C.byref(v), C.byref(e), C.byref(nl), C.byref(nc)))
        self.n_vocab, self.n_embd, self.n_layer, self.n_ctx = v.value, e.value, nl.value, nc.value

    def forward(self, tokens, pos0: int, stream=None):
        """Every position's (logits [nb][n_vocab], hnext [nb][n_embd]) as numpy."""
        t = np.ascontiguousarray(np.atleast_1d(tokens), dtype=np.int32)
        nb = t.size
        L, Hn = Buffer(nb * self.n_vocab * 4), Buffer(nb * self.n_embd * 4)
        check(lib().g4h_gemma_forward(self.ptr, t.ctypes.data_as(C.POINTER(_int)), nb, pos0, L.ptr, Hn.ptr, stream))
        return L.download(np.float32, (nb, self.n_vocab)), Hn.download(np.float32, (nb, self.n_embd))

    def prefill(self, tokens, pos0: int, want_logits: bool = True, stream=None):
        """g4h_gemma_prefill: the last position's logits (or None)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32).ravel()
        L = Buffer(self.n_vocab * 4) if want_logits else None
        check(lib().g4h_gemma_prefill(self.ptr, t.ctypes.data_as(C.POINTER(_int)), t.size, pos0, L.ptr if L else None,
                                      stream))
        return L.download(np.float32, (self.n_vocab,)) if L else None

    def set_state(self, token: int, pos: int, stream=None) -> None:
        check(lib().g4h_gemma_set_state(self.ptr, token, pos, stream))

    def step(self, stream=None) -> None:
        """One decode step from the device state (graph-capturable)."""
        check(lib().g4h_gemma_step(self.ptr, stream))

    def get_state(self, stream=None):
        t, p = _int(), _int()
        check(lib().g4h_gemma_get_state(self.ptr, C.byref(t), C.byref(p), stream))
        return t.value, p.value

    def status(self, stream=None) -> int:
        f = _int()
        check(lib().g4h_gemma_status(self.ptr, C.byref(f), stream))
        return f.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.n_vocab, np.float32)
        check(lib().g4h_memcpy_d2h(out.ctypes.data_as(_vp), lib().g4h_gemma_logits(self.ptr), out.nbytes, None))
        return out

    def trace(self, buf) -> int:
        """Per-token intermediate vectors of later forwards into buf (None: off);
        returns the floats per token (g4h_gemma_trace)."""
        n = _sz()
        check(lib().g4h_gemma_trace(self.ptr, _p(buf) if buf is not None else None, C.byref(n)))
        return n.value

    def kv(self, layer: int):
        """(K bytes, V bytes) of a layer's cache as numpy uint8 (host copies)."""
        k, v, n = _vp(), _vp(), _sz()
        check(lib().g4h_gemma_kv(self.ptr, layer, C.byref(k), C.byref(v), C.byref(n)))
        out = []
        for p in (k, v):
            a = np.empty(n.value, np.uint8)
            check(lib().g4h_memcpy_d2h(a.ctypes.data_as(_vp), p.value, a.nbytes, None))
            out.append(a)
        return out

    def free(self) -> None:
        if getattr(self, "ptr", None):
            lib().g4h_gemma_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def argmax_rows(logits, n: int, nb: int, out, stream=None) -> None:
    """out[b] = first index of the maximum of device row b of logits [nb][n]."""
    check(lib().g4h_argmax_rows(_p(logits), n, nb, _p(out), stream))


class SamplerParams(C.Structure):
    """g4h_sampler_params: the settings of g4_sampler (g4run.h:465-473)."""
    _fields_ = [("temp", C.c_float), ("top_k", _int), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("repeat_last_n", _int), ("freq_penalty", C.c_float), ("presence_penalty", C.c_float),
                ("no_repeat_ngram", _int), ("seed", C.c_uint64)]


SAMPLER_RING = 4096


class Sampler:
    """Device-resident sampling chain (g4h_sampler, the GPU form of sampler.c).
    Keyword settings override g4_sampler_init's defaults."""

    def __init__(self, n_vocab: int, **params):
        init()
        self.n_vocab = n_vocab
        self._p = SamplerParams()
        lib().g4h_sampler_default_params(C.byref(self._p))
        for k, v in params.items():
            setattr(self._p, k, v)
        p = _vp()
        check(lib().g4h_sampler_create(n_vocab, C.byref(self._p), C.byref(p)))
        self.ptr = p.value

    def set(self, stream=None, **params) -> None:
        for k, v in params.items():
            setattr(self._p, k, v)
        check(lib().g4h_sampler_set_params(self.ptr, C.byref(self._p), stream))

    def set_rng(self, words, stream=None) -> None:
        w = (C.c_uint64 * 4)(*[int(x) for x in words])
        check(lib().g4h_sampler_set_rng(self.ptr, w, stream))

    def reset(self, stream=None) -> None:
        check(lib().g4h_sampler_reset(self.ptr, stream))

    def ban(self, tok: int, stream=None) -> None:
        check(lib().g4h_sampler_ban(self.ptr, int(tok), stream))

    def accept(self, ids, stream=None) -> None:
        a = np.ascontiguousarray(np.atleast_1d(ids), dtype=np.int32)
        check(lib().g4h_sampler_accept(self.ptr, a.ctypes.data_as(C.POINTER(_int)), a.size, stream))

    def sample(self, logits, out=None, accept: bool = False, stream=None) -> None:
        """Draw from device logits (rewritten in place); the id goes to device out."""
        check(lib().g4h_sample(self.ptr, _p(logits), _p(out) if out is not None else None, int(accept), stream))

    def state(self, stream=None):
        """(rng words, ring oldest first, slow-path draw count)."""
        rng = (C.c_uint64 * 4)()
        rec = (_int * SAMPLER_RING)()
        n, slow = _int(), _int()
        check(lib().g4h_sampler_get_state(self.ptr, rng, rec, C.byref(n), C.byref(slow), stream))
        return [int(x) for x in rng], [int(rec[i]) for i in range(n.value)], slow.value

    def free(self) -> None:
        if getattr(self, "ptr", None):
            lib().g4h_sampler_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Model:
    """Device-resident decoder (g4h_model) and its decode step."""

    def __init__(self, seed: int = 1, **cfg):
        init()
        c = dict(GEMMA_STYLE)
        c.update(cfg)
        self.cfg = c
        self._c = ModelConfig(**c)
        p = _vp()
        check(lib().g4h_model_create(C.byref(self._c), seed, C.byref(p)))
        self.ptr = p.value

    def fill_kv(self, seed: int = 2, stream=None) -> None:
        check(lib().g4h_model_fill_kv(self.ptr, seed, stream))

    def forward(self, token: int, pos: int, stream=None) -> int:
        nxt = _int()
        check(lib().g4h_forward(self.ptr, token, pos, C.byref(nxt), stream))
        return nxt.value

    def forward_state(self, stream=None) -> None:
        check(lib().g4h_forward_state(self.ptr, stream))

    def set_state(self, token: int, pos: int, stream=None) -> None:
        check(lib().g4h_model_set_state(self.ptr, token, pos, stream))

    def get_state(self, stream=None):
        t, p = _int(), _int()
        check(lib().g4h_model_get_state(self.ptr, C.byref(t), C.byref(p), stream))
        return t.value, p.value

    def forward_batch(self, tokens, pos0: int, want_logits: bool = True, stream=None):
        """g4_forward_batch: layers for the tokens at pos0.., the last token's
        logits (host copy) if want_logits."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        check(lib().g4h_forward_batch(self.ptr, t.ctypes.data_as(C.POINTER(_int)), t.size, pos0, int(want_logits), stream))
        return self.logits() if want_logits else None

    def forward_batch_heads(self, tokens, pos0: int, logits=None, hnext=None, stream=None):
        """g4_forward_batch_heads into device buffers (allocated if not given);
        returns (logits Buffer [nb][n_vocab], hnext Buffer [nb][n_embd])."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        nb = t.size
        logits = logits if logits is not None else Buffer(nb * self.cfg["n_vocab"] * 4)
        hnext = hnext if hnext is not None else Buffer(nb * self.cfg["n_embd"] * 4)
        check(lib().g4h_forward_batch_heads(self.ptr, t.ctypes.data_as(C.POINTER(_int)), nb, pos0, _p(logits), _p(hnext),
                                            stream))
        return logits, hnext

    def set_sampler(self, sampler) -> None:
        """Draw each step's token with a Sampler (accepting it), or greedily with None."""
        check(lib().g4h_model_set_sampler(self.ptr, sampler.ptr if sampler is not None else None))
        self._sampler = sampler

    def status(self, stream=None) -> int:
        """STATUS_* flags of the device-side steps since the last set_state."""
        f = _int()
        check(lib().g4h_model_status(self.ptr, C.byref(f), stream))
        return f.value

    def trace(self, buf) -> None:
        """Copy each layer's input x, q|k|v projection and attention output (and
        the final x) into buf every step (trace_floats() floats; a batched
        forward of nb tokens writes nb such traces), or stop with None."""
        check(lib().g4h_model_trace(self.ptr, _p(buf) if buf is not None else None))

    def trace_fields(self):
        """(name, offset, length) of the per-layer trace record, and its size."""
        c = self.cfg
        E, R, Q, F = c["n_embd"], (c["n_head"] + 2 * c["n_kv"]) * c["head_dim"], c["n_head"] * c["head_dim"], c["n_ff"]
        fields, off = [], 0
        for name, n in (("x", E), ("qkv", R), ("att", Q), ("wo", E), ("xmid", E), ("h", F), ("down", E)):
            fields.append((name, off, n))
            off += n
        return fields, off

    def trace_floats(self) -> int:
        _, rec = self.trace_fields()
        return self.cfg["n_layer"] * rec + self.cfg["n_embd"]

    def gelu_table(self) -> np.ndarray:
        out = np.empty(65536, np.uint16)
        check(lib().g4h_memcpy_d2h(out.ctypes.data_as(_vp), lib().g4h_model_gelu_table(self.ptr), out.nbytes, None))
        return out

    def logits(self) -> np.ndarray:
        n = self.cfg["n_vocab"]
        out = np.empty(n, np.float32)
        check(lib().g4h_memcpy_d2h(out.ctypes.data_as(_vp), lib().g4h_model_logits(self.ptr), n * 4, None))
        return out

    @property
    def weight_bytes(self) -> int:
        return lib().g4h_model_weight_bytes(self.ptr)

    def matrix(self, layer: int, name: str) -> _View:
        return _View(lib().g4h_model_matrix(self.ptr, layer, 4 if name == "head" else _MATS[name]))

    def norm(self, layer: int, name: str) -> np.ndarray:
        c = self.cfg
        n = c["head_dim"] if name in ("q_norm", "k_norm") else c["n_embd"]
        p = lib().g4h_model_norm(self.ptr, layer, 6 if name == "output_norm" else _NORMS[name])
        out = np.empty(n, np.float32)
        check(lib().g4h_memcpy_d2h(out.ctypes.data_as(_vp), p, n * 4, None))
        return out

    def kv(self, layer: int):
        k, v, nb = _vp(), _vp(), _sz()
        check(lib().g4h_model_kv(self.ptr, layer, C.byref(k), C.byref(v), C.byref(nb)))
        out = []
        for p in (k, v):
            a = np.empty(nb.value, np.uint8)
            check(lib().g4h_memcpy_d2h(a.ctypes.data_as(_vp), p.value, nb.value, None))
            out.append(a)
        return out

    def host_copy(self):
        """Every parameter and the KV cache as host arrays (for a CPU check).

        The resident gate/up matrix stores its rows interleaved (gate_i, up_i);
        it is returned as [gate | up] rows, the order of the reference's fused
        w_gate_up (model.c:721-729)."""
        c = self.cfg
        w = {k: [] for k in list(_MATS) + list(_NORMS)}
        kc, vc = [], []
        for l in range(c["n_layer"]):
            for k in _MATS:
                rows = self.matrix(l, k).to_rows()
                if k == "wgu":
                    rows = np.concatenate([rows[0::2], rows[1::2]])
                w[k].append(rows)
            for k in _NORMS:
                w[k].append(self.norm(l, k))
            a, b = self.kv(l)
            kc.append(a)
            vc.append(b)
        w["head"] = self.matrix(0, "head").to_rows()
        w["output_norm"] = self.norm(0, "output_norm")
        return w, kc, vc

    def free(self):
        if getattr(self, "ptr", None):
            check(lib().g4h_model_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
