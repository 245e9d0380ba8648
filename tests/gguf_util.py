"""GGUF files for the tests: a writer (GGUF v2/v3: header, metadata, tensor
table, aligned data) and a ctypes mirror of g4_model_file (g4run.h:172-246,
include/g4run_abi.h) for reading back what the library's g4_gguf_open parsed.

Test infrastructure: the files it writes are small synthetic models in the
gemma4 layout (the tensor names of model.c:377-418, the hparam keys of
gguf.c:190-300)."""
import ctypes as C
import struct

import numpy as np

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def _str(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def _value(vt, v) -> bytes:
    if vt == STR:
        return _str(v.encode() if isinstance(v, str) else v)
    if vt == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for x in items:
            out += _value(et, x)
        return out
    return struct.pack(_FMT[vt], v)


def write_gguf(path, meta, tensors, alignment=32, version=3):
    """meta: [(key, vtype, value)], ARR values are (elem_type, [items]);
    tensors: [(name, ggml_type, ne (list, ne[0] = row length), raw bytes)]."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(meta))
    for key, vt, v in meta:
        head += _str(key.encode()) + struct.pack("<I", vt) + _value(vt, v)
    offs, off = [], 0
    for name, t, ne, raw in tensors:
        offs.append(off)
        off += len(raw)
        off = (off + alignment - 1) // alignment * alignment
    for (name, t, ne, raw), o in zip(tensors, offs):
        head += _str(name.encode()) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", t, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        pos = 0
        for (name, t, ne, raw), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            f.write(bytes(raw))
            pos = o + len(raw)


MAX_LAYERS = 64


class GStr(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("len", C.c_uint32)]

    def bytes(self) -> bytes:
        return C.string_at(self.ptr, self.len) if self.ptr else b""


class GTensor(C.Structure):
    _fields_ = [("name", C.c_char * 80), ("type", C.c_int), ("ndim", C.c_int), ("ne", C.c_int64 * 4),
                ("offset", C.c_uint64), ("data", C.c_void_p)]


class ModelFile(C.Structure):
    """g4_model_file, field for field."""
    _fields_ = [
        ("map_base", C.c_void_p), ("map_size", C.c_uint64), ("h_file", C.c_void_p), ("h_map", C.c_void_p),
        ("version", C.c_uint32), ("n_tensors", C.c_uint64), ("n_kv", C.c_uint64), ("data_start", C.c_uint64),
        ("kv_end", C.c_uint64), ("ff_len_off", C.c_uint64), ("ff_len_vt", C.c_int), ("alignment", C.c_uint32),
        ("tensors", C.POINTER(GTensor)),
        ("arch", C.c_char * 32),
        ("n_layer", C.c_int), ("n_embd", C.c_int), ("n_vocab", C.c_int), ("n_head", C.c_int), ("n_head_kv", C.c_int),
        ("n_embd_per_layer", C.c_int), ("n_ff", C.c_int * MAX_LAYERS),
        ("head_dim_full", C.c_int), ("head_dim_swa", C.c_int), ("n_rot_full", C.c_int), ("n_rot_swa", C.c_int),
        ("rope_base_full", C.c_float), ("rope_base_swa", C.c_float), ("rms_eps", C.c_float),
        ("final_softcap", C.c_float), ("n_swa", C.c_int), ("n_kv_shared", C.c_int), ("n_layer_kv", C.c_int),
        ("is_swa", C.c_uint8 * MAX_LAYERS), ("n_ctx_train", C.c_int),
        ("is_assistant", C.c_bool), ("n_embd_out", C.c_int), ("n_nextn", C.c_int),
        ("is_qwen35", C.c_bool), ("n_embd_head_k", C.c_int), ("n_embd_head_v", C.c_int),
        ("ssm_d_conv", C.c_int), ("ssm_d_inner", C.c_int), ("ssm_d_state", C.c_int), ("ssm_dt_rank", C.c_int),
        ("ssm_n_group", C.c_int), ("full_attn_interval", C.c_int), ("rope_sections", C.c_int * 4),
        ("is_recr", C.c_uint8 * MAX_LAYERS), ("tok_pre", C.c_int),
        ("tok_n", C.c_int), ("tok_text", C.POINTER(GStr)), ("tok_type", C.POINTER(C.c_int32)),
        ("merges_n", C.c_int), ("merges", C.POINTER(GStr)),
        ("bos_id", C.c_int), ("eos_id", C.c_int), ("eot_id", C.c_int), ("unk_id", C.c_int), ("pad_id", C.c_int),
        ("add_bos", C.c_bool), ("meta_temp", C.c_float), ("meta_top_p", C.c_float), ("meta_top_k", C.c_int),
        ("chat_template", GStr),
    ]


def bind(L):
    L.g4_gguf_open.restype = C.c_int
    L.g4_gguf_open.argtypes = [C.POINTER(ModelFile), C.c_char_p, C.c_bool]
    L.g4_gguf_close.restype = None
    L.g4_gguf_close.argtypes = [C.POINTER(ModelFile)]
    L.g4_find_tensor.restype = C.POINTER(GTensor)
    L.g4_find_tensor.argtypes = [C.POINTER(ModelFile), C.c_char_p]


def open_gguf(L, path):
    """(rc, ModelFile) from the library's parser."""
    bind(L)
    mf = ModelFile()
    rc = L.g4_gguf_open(C.byref(mf), str(path).encode(), False)
    return rc, mf


def tensor_bytes(t: GTensor, nbytes: int) -> bytes:
    return C.string_at(t.data, nbytes)
