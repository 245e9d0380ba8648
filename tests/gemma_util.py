"""Synthetic gemma4 models for the tests: random tensors in the GGUF layout of
the reference's model (tensor names of model.c:377-418, hparam keys of
gguf.c:190-300), written to a GGUF file and handed to the oracle.

Weights mix the formats the path supports (q8_0, q4_0, q4_K, q6_K, f16,
bf16); norms and RoPE frequency factors are f32."""
import numpy as np

import gguf_util as GU

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30

SMALL = dict(n_layer=4, n_kv_shared=1, n_embd=256, n_head=4, head_dim_full=128, head_dim_swa=64,
             n_ff=[512, 768, 512, 512], n_embd_per_layer=32, n_vocab=512, n_swa=8, is_swa=[1, 1, 0, 1],
             rope_base_full=1e6, rope_base_swa=1e4, rms_eps=1e-6, final_softcap=15.0)
# the reference's gemma4 head widths (g4run.h:283-292: 8 query heads of 512 on
# the full-attention layers, 256 on the sliding ones), at small model width
WIDE = dict(n_layer=4, n_kv_shared=1, n_embd=512, n_head=8, head_dim_full=512, head_dim_swa=256,
            n_ff=[1024, 768, 1024, 1024], n_embd_per_layer=64, n_vocab=512, n_swa=16, is_swa=[1, 1, 0, 1],
            rope_base_full=1e6, rope_base_swa=1e4, rms_eps=1e-6, final_softcap=15.0)
# the model bench.py times: 8 layers of width 2048, the reference's heads (8 x
# 512 on full layers, 8 x 256 on sliding ones), two shared-KV layers (a sliding
# one reading layer 4, a full one reading layer 5), FFN 6144, 32768 tokens
BENCH = dict(n_layer=8, n_kv_shared=2, n_embd=2048, n_head=8, head_dim_full=512, head_dim_swa=256,
             n_ff=[6144] * 8, n_embd_per_layer=256, n_vocab=32768, n_swa=512, is_swa=[1, 1, 1, 0, 1, 0, 1, 0],
             rope_base_full=1e6, rope_base_swa=1e4, rms_eps=1e-6, final_softcap=30.0)


def _bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def random_rows(oracle, rs, t, nrows, ncols, sigma):
    """nrows GGUF rows of type t with values of roughly N(0, sigma)."""
    if t in (Q8_0, Q4_0):
        return oracle.quantize(t, (rs.standard_normal((nrows, ncols)) * sigma).astype(np.float32))
    if t == F16:
        return (rs.standard_normal((nrows, ncols)) * sigma).astype(np.float16).view(np.uint8).reshape(nrows, -1)
    if t == BF16:
        return _bf16(rs.standard_normal((nrows, ncols)) * sigma).view(np.uint8).reshape(nrows, -1)
    nb = ncols // 256
    if t == Q4_K:      # d, dmin fp16 | 12 scale bytes | 128 nibble bytes
        b = rs.integers(0, 256, (nrows, nb, 144), dtype=np.uint8)
        b[..., 0:2] = np.frombuffer(np.float16(sigma / 300).tobytes(), np.uint8)
        b[..., 2:4] = np.frombuffer(np.float16(sigma / 150).tobytes(), np.uint8)
        return b.reshape(nrows, -1)
    if t == Q6_K:      # 128 ql | 64 qh | 16 int8 scales | d fp16
        b = rs.integers(0, 256, (nrows, nb, 210), dtype=np.uint8)
        b[..., 192:208] = rs.integers(-40, 40, (nrows, nb, 16)).astype(np.int8).view(np.uint8)
        b[..., 208:210] = np.frombuffer(np.float16(sigma / 700).tobytes(), np.uint8)
        return b.reshape(nrows, -1)
    raise ValueError(t)


def make_gemma(oracle, seed, spec=SMALL, types=None):
    """(hp, tensors): hp with g4_model_file's field names, tensors
    {name: (type, ne, raw rows)} in the gemma4 GGUF layout."""
    rs = np.random.default_rng(seed)
    sp = dict(spec)
    E, H, PE, V, NL = sp["n_embd"], sp["n_head"], sp["n_embd_per_layer"], sp["n_vocab"], sp["n_layer"]
    ty = dict(wq=Q8_0, wk=Q4_0, wv=Q8_0, wo=Q4_K, gate=Q4_0, up=Q8_0, down=Q6_K, inp_gate=F16, proj=BF16,
              tok_embd=Q8_0, ple=Q4_0, ple_proj=Q8_0)
    ty.update(types or {})
    T = {}

    def put(name, t, ncols, nrows, sigma):
        T[name] = (t, [ncols, nrows], random_rows(oracle, rs, t, nrows, ncols, sigma))

    def norm(name, n, mean=1.0, sd=0.1):
        T[name] = (F32, [n], (mean + sd * rs.standard_normal(n)).astype(np.float32))

    put("token_embd.weight", ty["tok_embd"], E, V, 0.5)
    put("per_layer_token_embd.weight", ty["ple"], NL * PE, V, 0.5)
    put("per_layer_model_proj.weight", ty["ple_proj"], E, NL * PE, 0.05)
    norm("per_layer_proj_norm.weight", PE)
    norm("output_norm.weight", E)
    T["rope_freqs.weight"] = (F32, [sp["head_dim_full"] // 2],
                              (1.0 + rs.random(sp["head_dim_full"] // 2) * 3).astype(np.float32))
    n_layer_kv = NL - sp["n_kv_shared"]
    for il in range(NL):
        p = f"blk.{il}."
        hd = sp["head_dim_swa"] if sp["is_swa"][il] else sp["head_dim_full"]
        F = sp["n_ff"][il]
        for n in ("attn_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm", "post_norm"):
            norm(p + n + ".weight", E)
        norm(p + "attn_q_norm.weight", hd)
        put(p + "attn_q.weight", ty["wq"], E, H * hd, 0.05)
        if il < n_layer_kv:
            norm(p + "attn_k_norm.weight", hd)
            put(p + "attn_k.weight", ty["wk"], E, hd, 0.05)
            if il != 1:                                   # layer 1: V = K
                put(p + "attn_v.weight", ty["wv"], E, hd, 0.05)
        put(p + "attn_output.weight", ty["wo"], H * hd, E, 0.05)
        put(p + "ffn_gate.weight", ty["gate"], E, F, 0.05)
        put(p + "ffn_up.weight", ty["up"], E, F, 0.05)
        put(p + "ffn_down.weight", ty["down"], F, E, 0.05)
        put(p + "inp_gate.weight", ty["inp_gate"], E, PE, 0.05)
        put(p + "proj.weight", ty["proj"], PE, E, 0.05)
        if il % 2 == 0:
            T[p + "layer_output_scale.weight"] = (F32, [1], np.array([0.75 + 0.1 * il], np.float32))
    hp = dict(sp, n_layer_kv=n_layer_kv, n_rot_full=sp["head_dim_full"], n_rot_swa=sp["head_dim_swa"],
              n_head_kv=1)
    return hp, T


def gguf_meta(hp):
    swa_pat = [int(x) for x in hp["is_swa"]]
    toks = [f"<t{i}>" for i in range(hp["n_vocab"])]
    return [
        ("general.architecture", GU.STR, "gemma4"),
        ("gemma4.block_count", GU.U32, hp["n_layer"]),
        ("gemma4.context_length", GU.U32, 131072),
        ("gemma4.embedding_length", GU.U32, hp["n_embd"]),
        ("gemma4.feed_forward_length", GU.ARR, (GU.I32, list(hp["n_ff"]))),
        ("gemma4.attention.head_count", GU.U32, hp["n_head"]),
        ("gemma4.attention.head_count_kv", GU.U32, 1),
        ("gemma4.rope.freq_base", GU.F32, hp["rope_base_full"]),
        ("gemma4.rope.freq_base_swa", GU.F32, hp["rope_base_swa"]),
        ("gemma4.attention.layer_norm_rms_epsilon", GU.F32, hp["rms_eps"]),
        ("gemma4.attention.key_length", GU.U32, hp["head_dim_full"]),
        ("gemma4.attention.key_length_swa", GU.U32, hp["head_dim_swa"]),
        ("gemma4.final_logit_softcapping", GU.F32, hp["final_softcap"]),
        ("gemma4.attention.sliding_window", GU.U32, hp["n_swa"]),
        ("gemma4.attention.shared_kv_layers", GU.U32, hp["n_kv_shared"]),
        ("gemma4.embedding_length_per_layer_input", GU.U32, hp["n_embd_per_layer"]),
        ("gemma4.rope.dimension_count", GU.U32, hp["head_dim_full"]),
        ("gemma4.rope.dimension_count_swa", GU.U32, hp["head_dim_swa"]),
        ("gemma4.attention.sliding_window_pattern", GU.ARR, (GU.BOOL, swa_pat)),
        ("tokenizer.ggml.tokens", GU.ARR, (GU.STR, toks)),
    ]


def write_gemma(path, hp, T):
    tensors = [(name, t, ne, np.ascontiguousarray(raw).view(np.uint8).tobytes()) for name, (t, ne, raw) in T.items()]
    GU.write_gguf(path, gguf_meta(hp), tensors)
