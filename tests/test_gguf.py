"""The GGUF reader (g4_gguf_open / g4_find_tensor / g4_gguf_close, the Linux
form of gguf.c:124-420) on files the tests write: hparams, tokenizer arrays,
the tensor table with its aligned data offsets, and every error path of the
reference parser.  Host code only -- no GPU."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import gguf_util as GU

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def L():
    import g4run_amd as G
    lib = G.lib()
    GU.bind(lib)
    return lib


def gemma_meta(n_layer=4, vocab=10, extra=()):
    toks = [f"t{i}" for i in range(vocab)]
    return [
        ("general.architecture", GU.STR, "gemma4"),
        ("gemma4.block_count", GU.U32, n_layer),
        ("gemma4.context_length", GU.U32, 4096),
        ("gemma4.embedding_length", GU.U32, 64),
        ("gemma4.feed_forward_length", GU.ARR, (GU.I32, [128, 256, 128, 256][:n_layer])),
        ("gemma4.attention.head_count", GU.U32, 4),
        ("gemma4.attention.head_count_kv", GU.U32, 1),
        ("gemma4.rope.freq_base", GU.F32, 1e6),
        ("gemma4.rope.freq_base_swa", GU.F32, 1e4),
        ("gemma4.attention.layer_norm_rms_epsilon", GU.F32, 1e-6),
        ("gemma4.attention.key_length", GU.U32, 64),
        ("gemma4.attention.key_length_swa", GU.U32, 32),
        ("gemma4.final_logit_softcapping", GU.F32, 30.0),
        ("gemma4.attention.sliding_window", GU.U32, 16),
        ("gemma4.attention.shared_kv_layers", GU.U32, 2),
        ("gemma4.embedding_length_per_layer_input", GU.U32, 8),
        ("gemma4.rope.dimension_count", GU.U32, 64),
        ("gemma4.rope.dimension_count_swa", GU.U32, 32),
        ("gemma4.attention.sliding_window_pattern", GU.ARR, (GU.BOOL, [1, 1, 0, 1][:n_layer])),
        ("tokenizer.ggml.model", GU.STR, "gemma4"),
        ("tokenizer.ggml.tokens", GU.ARR, (GU.STR, toks)),
        ("tokenizer.ggml.token_type", GU.ARR, (GU.I32, [1] * vocab)),
        ("tokenizer.ggml.bos_token_id", GU.U32, 2),
        ("tokenizer.ggml.eos_token_id", GU.I32, 1),
        ("tokenizer.ggml.add_bos_token", GU.BOOL, 0),
        ("general.sampling.temp", GU.F64, 0.7),
        ("general.sampling.top_k", GU.I64, 40),
        ("some.unused.array", GU.ARR, (GU.U16, [1, 2, 3])),
    ] + list(extra)


def some_tensors(rs):
    t = []
    t.append(("output_norm.weight", 0, [64], rs.standard_normal(64).astype(np.float32).tobytes()))
    t.append(("token_embd.weight", 8, [64, 10], rs.integers(0, 256, 10 * 2 * 34, dtype=np.uint8).tobytes()))
    t.append(("blk.0.attn_q.weight", 2, [64, 256], rs.integers(0, 256, 256 * 2 * 18, dtype=np.uint8).tobytes()))
    t.append(("blk.0.ffn_down.weight", 1, [128, 64], rs.standard_normal(128 * 64).astype(np.float16).tobytes()))
    t.append(("blk.0.x.weight", 12, [256, 3], rs.integers(0, 256, 3 * 144, dtype=np.uint8).tobytes()))
    return t


def test_model_file_mirror_matches_the_c_layout(tmp_path):
    """The ctypes mirror used by these tests has g4_model_file's offsets."""
    fields = [f for f, _ in GU.ModelFile._fields_]
    src = tmp_path / "off.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "g4run_abi.h"\nint main(void){\n'
                   + "".join(f'printf("%zu\\n", offsetof(g4_model_file, {f}));\n' for f in fields)
                   + 'printf("%zu\\n", sizeof(g4_model_file));\nreturn 0;}\n')
    exe = tmp_path / "off"
    r = subprocess.run(["gcc", "-std=c11", "-I" + os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()]
    want = [getattr(GU.ModelFile, f).offset for f in fields] + [C.sizeof(GU.ModelFile)]
    assert got == want


@pytest.mark.parametrize("version,alignment", [(3, 32), (2, 32), (3, 64)])
def test_reads_hparams_tokens_and_tensors(L, tmp_path, version, alignment):
    rs = np.random.default_rng(version + alignment)
    tens = some_tensors(rs)
    extra = [("general.alignment", GU.U32, alignment)] if alignment != 32 else []
    p = tmp_path / "m.gguf"
    GU.write_gguf(p, gemma_meta(extra=extra), tens, alignment=alignment, version=version)
    rc, mf = GU.open_gguf(L, p)
    try:
        assert rc == 0
        assert mf.version == version and mf.n_tensors == len(tens) and mf.alignment == alignment
        assert mf.arch == b"gemma4"
        assert (mf.n_layer, mf.n_embd, mf.n_head, mf.n_head_kv, mf.n_vocab, mf.tok_n) == (4, 64, 4, 1, 10, 10)
        assert list(mf.n_ff[:4]) == [128, 256, 128, 256]
        assert list(mf.is_swa[:4]) == [1, 1, 0, 1]
        assert (mf.head_dim_full, mf.head_dim_swa, mf.n_rot_full, mf.n_rot_swa) == (64, 32, 64, 32)
        assert mf.rope_base_full == np.float32(1e6) and mf.rope_base_swa == np.float32(1e4)
        assert mf.rms_eps == np.float32(1e-6) and mf.final_softcap == np.float32(30.0)
        assert (mf.n_swa, mf.n_kv_shared, mf.n_layer_kv, mf.n_embd_per_layer) == (16, 2, 2, 8)
        assert mf.n_ctx_train == 4096 and mf.bos_id == 2 and mf.eos_id == 1 and mf.eot_id == -1
        assert mf.add_bos is True                       # forced on for gemma4 (gguf.c:383-385)
        assert abs(mf.meta_temp - 0.7) < 1e-6 and mf.meta_top_k == 40 and mf.meta_top_p == -1
        assert [mf.tok_text[i].bytes() for i in range(10)] == [f"t{i}".encode() for i in range(10)]
        assert mf.data_start % alignment == 0
        for name, t, ne, raw in tens:
            g = L.g4_find_tensor(C.byref(mf), name.encode())
            assert g, name
            g = g.contents
            assert g.type == t and g.ndim == len(ne) and list(g.ne[:len(ne)]) == ne
            assert g.offset % alignment == 0
            assert GU.tensor_bytes(g, len(raw)) == raw
        assert not L.g4_find_tensor(C.byref(mf), b"missing.weight")
    finally:
        L.g4_gguf_close(C.byref(mf))
    assert mf.map_base is None and mf.n_tensors == 0


def test_qwen35_layer_pattern(L, tmp_path):
    meta = [("general.architecture", GU.STR, "qwen35"), ("qwen35.block_count", GU.U32, 8),
            ("qwen35.embedding_length", GU.U32, 32), ("qwen35.feed_forward_length", GU.U32, 96),
            ("tokenizer.ggml.pre", GU.STR, "qwen35"), ("tokenizer.ggml.tokens", GU.ARR, (GU.STR, ["a", "b"]))]
    p = tmp_path / "q.gguf"
    GU.write_gguf(p, meta, [])
    rc, mf = GU.open_gguf(L, p)
    try:
        assert rc == 0 and mf.is_qwen35 and mf.tok_pre == 1 and mf.full_attn_interval == 4
        assert list(mf.is_recr[:8]) == [1, 1, 1, 0, 1, 1, 1, 0]
        assert list(mf.n_ff[:3]) == [96, 96, 96] and mf.ff_len_off > 0 and mf.ff_len_vt == GU.U32
    finally:
        L.g4_gguf_close(C.byref(mf))


@pytest.mark.parametrize("case", ["magic", "version1", "version4", "truncated", "oob", "badtype", "arch", "layers",
                                  "missing"])
def test_rejects_what_the_reference_rejects(L, tmp_path, case):
    rs = np.random.default_rng(0)
    tens = some_tensors(rs)
    meta = gemma_meta()
    version = 3
    if case == "version1":
        version = 1
    elif case == "version4":
        version = 4
    elif case == "oob":
        tens[-1] = (tens[-1][0], tens[-1][1], [256, 300], tens[-1][3])      # claims more rows than stored
    elif case == "badtype":
        tens[0] = (tens[0][0], 99, tens[0][2], tens[0][3])
    elif case == "arch":
        meta[0] = ("general.architecture", GU.STR, "llama")
    elif case == "layers":
        meta = [m for m in meta if m[0] != "gemma4.attention.shared_kv_layers"]
        meta.append(("gemma4.attention.shared_kv_layers", GU.U32, 3))        # n_layer_kv = 1 < 2
    p = tmp_path / "bad.gguf"
    if case == "missing":
        p = tmp_path / "does-not-exist.gguf"
    else:
        GU.write_gguf(p, meta, tens, version=version)
    if case == "magic":
        b = bytearray(p.read_bytes())
        b[0] = ord("X")
        p.write_bytes(bytes(b))
    elif case == "truncated":
        b = p.read_bytes()
        p.write_bytes(b[:200])
    rc, mf = GU.open_gguf(L, p)
    assert rc == -1
    assert mf.map_base is None and mf.tensors is None or not bool(mf.tensors)
