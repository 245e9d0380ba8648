// gguf.cpp -- GGUF v2/v3 model files on Linux (include/g4run_abi.h): the
// file is mapped read-only and private (mmap), the header is parsed in place
// and every tensor's data pointer resolved into the mapping, with the
// metadata keys, defaults and checks of the reference's parser
// (gguf.c:124-404).  The mapped tensors are what g4h_gemma_create uploads to
// the device.
#include "../../include/g4run_abi.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>

namespace {

// GGUF metadata value types (the file format's ids)
enum : uint32_t { V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 };
constexpr int kScalarBytes[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

// bounds-checked little-endian reads over the mapping; the first overrun
// sets `bad` and every later read returns zero
struct Reader {
    const uint8_t *p, *end;
    bool bad = false;
    bool take(void *dst, size_t n) {
        if (bad || (size_t)(end - p) < n) {
            bad = true;
            return false;
        }
        std::memcpy(dst, p, n);
        p += n;
        return true;
    }
    // whether n items of at least `unit` bytes each can still follow (a
    // count from the file is checked so before anything is sized by it)
    bool fits(uint64_t n, uint64_t unit) {
        if (bad || n > (uint64_t)(end - p) / unit) {
            bad = true;
            return false;
        }
        return true;
    }
    bool skip(uint64_t n) {
        if (bad || (uint64_t)(end - p) < n) {
            bad = true;
            return false;
        }
        p += n;
        return true;
    }
    template <class T>
    T get() {
        T v{};
        take(&v, sizeof v);
        return v;
    }
    g4_str str() {
        g4_str s{nullptr, 0};
        const uint64_t n = get<uint64_t>();
        if (bad || (uint64_t)(end - p) < n) {
            bad = true;
            return s;
        }
        s.ptr = (const char *)p;
        s.len = (uint32_t)n;
        p += n;
        return s;
    }
    // a scalar of any numeric / bool type as double (gguf.c:112-128)
    double scalar(uint32_t vt) {
        switch (vt) {
        case V_U8: return get<uint8_t>();
        case V_I8: return get<int8_t>();
        case V_U16: return get<uint16_t>();
        case V_I16: return get<int16_t>();
        case V_U32: return get<uint32_t>();
        case V_I32: return get<int32_t>();
        case V_F32: return get<float>();
        case V_BOOL: return get<uint8_t>() != 0;
        case V_U64: return (double)get<uint64_t>();
        case V_I64: return (double)get<int64_t>();
        case V_F64: return get<double>();
        default: bad = true; return 0.0;
        }
    }
};

bool is(g4_str k, const char *s) {
    const size_t n = std::strlen(s);
    return k.len == n && std::memcmp(k.ptr, s, n) == 0;
}
// "<arch>.<suffix>" for the gemma4 and gemma4-assistant prefixes (gguf.c:96-102)
bool hkey(g4_str k, const char *suffix) {
    for (const char *arch : {"gemma4.", "gemma4-assistant."}) {
        const size_t a = std::strlen(arch), n = std::strlen(suffix);
        if (k.len == a + n && std::memcmp(k.ptr, arch, a) == 0 && std::memcmp(k.ptr + a, suffix, n) == 0) return true;
    }
    return false;
}

int fail(g4_model_file *mf, const char *fmt, const char *arg = "") {
    std::fprintf(stderr, "g4: ");
    std::fprintf(stderr, fmt, arg);
    std::fprintf(stderr, "\n");
    g4_gguf_close(mf);
    return -1;
}

// per-layer array values copied into a fixed table (at most G4_MAX_LAYERS)
template <class T, class D>
void layer_array(Reader &r, uint64_t n, D *dst) {
    for (uint64_t j = 0; j < n && !r.bad; j++) {
        const T v = r.get<T>();
        if (j < G4_MAX_LAYERS) dst[j] = (D)v;
    }
}

}  // namespace

extern "C" void g4_gguf_close(g4_model_file *mf) {
    if (!mf) return;
    std::free(mf->tensors);
    std::free(mf->tok_text);
    std::free(mf->merges);
    if (mf->map_base) munmap(mf->map_base, (size_t)mf->map_size);
    std::memset(mf, 0, sizeof *mf);
}

extern "C" const g4_tensor *g4_find_tensor(const g4_model_file *mf, const char *name) {
    for (uint64_t i = 0; i < mf->n_tensors; i++)
        if (std::strcmp(mf->tensors[i].name, name) == 0) return &mf->tensors[i];
    return nullptr;
}

extern "C" int g4_gguf_open(g4_model_file *mf, const char *path, bool verbose) {
    // defaults (gguf.c:125-130)
    std::memset(mf, 0, sizeof *mf);
    mf->alignment = 32;
    mf->bos_id = mf->eos_id = mf->eot_id = mf->unk_id = mf->pad_id = -1;
    mf->meta_temp = -1;
    mf->meta_top_p = -1;
    mf->meta_top_k = -1;
    mf->add_bos = true;
    mf->n_ctx_train = 131072;

    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(mf, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return fail(mf, "cannot stat %s", path);
    }
    void *base = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);                                       // the mapping keeps the file
    if (base == MAP_FAILED) return fail(mf, "cannot map %s", path);
    mf->map_base = base;
    mf->map_size = (uint64_t)st.st_size;
    Reader r{(const uint8_t *)base, (const uint8_t *)base + mf->map_size};

    if (r.get<uint32_t>() != 0x46554747u) return fail(mf, "not a GGUF file");   // "GGUF"
    mf->version = r.get<uint32_t>();
    mf->n_tensors = r.get<uint64_t>();
    mf->n_kv = r.get<uint64_t>();
    if (mf->version < 2 || mf->version > 3) return fail(mf, "unsupported GGUF version");

    // ---- metadata (gguf.c:184-300) ----
    for (uint64_t i = 0; i < mf->n_kv && !r.bad; i++) {
        const g4_str key = r.str();
        const uint32_t vt = r.get<uint32_t>();
        if (r.bad) break;
        if (vt == V_STR) {
            const g4_str v = r.str();
            if (r.bad) break;
            if (is(key, "general.architecture")) {
                const size_t n = v.len < sizeof mf->arch - 1 ? v.len : sizeof mf->arch - 1;
                std::memcpy(mf->arch, v.ptr, n);
                mf->arch[n] = 0;
            } else if (is(key, "tokenizer.chat_template")) {
                mf->chat_template = v;
            } else if (is(key, "tokenizer.ggml.pre")) {
                if (v.len == 6 && std::memcmp(v.ptr, "qwen35", 6) == 0) mf->tok_pre = 1;
            } else if (is(key, "tokenizer.ggml.model")) {
                if (v.len == 4 && std::memcmp(v.ptr, "gpt2", 4) == 0) mf->tok_pre = 1;
            }
            continue;
        }
        if (vt == V_ARR) {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (r.bad || et > V_F64 || et == V_ARR) {
                r.bad = true;
                break;
            }
            if (et == V_STR ? !r.fits(n, 8) : !r.fits(n, (uint64_t)kScalarBytes[et])) break;   // 8: a string's length
            if (n > 0x7fffffff) {
                r.bad = true;
                break;
            }
            if (is(key, "tokenizer.ggml.tokens") && et == V_STR) {
                mf->tok_n = (int)n;
                mf->tok_text = (g4_str *)std::malloc((n ? n : 1) * sizeof(g4_str));
                for (uint64_t j = 0; j < n && !r.bad; j++) mf->tok_text[j] = r.str();
            } else if (is(key, "tokenizer.ggml.merges") && et == V_STR) {
                mf->merges_n = (int)n;
                mf->merges = (g4_str *)std::malloc((n ? n : 1) * sizeof(g4_str));
                for (uint64_t j = 0; j < n && !r.bad; j++) mf->merges[j] = r.str();
            } else if (is(key, "tokenizer.ggml.token_type") && et == V_I32) {
                mf->tok_type = (const int32_t *)r.p;
                r.skip(4 * n);
            } else if (hkey(key, "feed_forward_length") && (et == V_U32 || et == V_I32)) {
                if (et == V_U32) layer_array<uint32_t>(r, n, mf->n_ff);
                else layer_array<int32_t>(r, n, mf->n_ff);
            } else if (hkey(key, "attention.sliding_window_pattern") && et == V_BOOL) {
                layer_array<uint8_t>(r, n, mf->is_swa);
            } else if (is(key, "qwen35.rope.dimension_sections") && (et == V_U32 || et == V_I32)) {
                for (uint64_t j = 0; j < n && !r.bad; j++) {
                    const int32_t v = r.get<int32_t>();
                    if (j < 4) mf->rope_sections[j] = v;
                }
            } else if (is(key, "qwen35.attention.recurrent_layers") && et == V_BOOL) {
                layer_array<uint8_t>(r, n, mf->is_recr);
                mf->full_attn_interval = -1;                    // an explicit per-layer list
            } else if (et == V_STR) {
                for (uint64_t j = 0; j < n && !r.bad; j++) r.str();
            } else {
                r.skip((uint64_t)kScalarBytes[et] * n);
            }
            continue;
        }
        const uint64_t off = (uint64_t)(r.p - (const uint8_t *)base);
        const double v = r.scalar(vt);
        // conversions of any file value stay defined: out of range (or NaN)
        // becomes a value the checks below refuse
        const int iv = v > -2147483648.0 && v < 2147483648.0 ? (int)v : v > 0 ? INT_MAX : INT_MIN;
        if (is(key, "general.alignment")) mf->alignment = v >= 0.0 && v < 4294967296.0 ? (uint32_t)v : 0u;
        else if (hkey(key, "block_count")) mf->n_layer = iv;
        else if (hkey(key, "context_length")) mf->n_ctx_train = iv;
        else if (hkey(key, "embedding_length")) mf->n_embd = iv;
        else if (hkey(key, "embedding_length_out")) mf->n_embd_out = iv;
        else if (hkey(key, "nextn_predict_layers")) mf->n_nextn = iv;
        else if (hkey(key, "feed_forward_length")) for (int j = 0; j < G4_MAX_LAYERS; j++) mf->n_ff[j] = iv;
        else if (hkey(key, "attention.head_count")) mf->n_head = iv;
        else if (hkey(key, "attention.head_count_kv")) mf->n_head_kv = iv;
        else if (hkey(key, "rope.freq_base")) mf->rope_base_full = (float)v;
        else if (hkey(key, "rope.freq_base_swa")) mf->rope_base_swa = (float)v;
        else if (hkey(key, "attention.layer_norm_rms_epsilon")) mf->rms_eps = (float)v;
        else if (hkey(key, "attention.key_length")) mf->head_dim_full = iv;
        else if (hkey(key, "attention.key_length_swa")) mf->head_dim_swa = iv;
        else if (hkey(key, "final_logit_softcapping")) mf->final_softcap = (float)v;
        else if (hkey(key, "attention.sliding_window")) mf->n_swa = iv;
        else if (hkey(key, "attention.shared_kv_layers")) mf->n_kv_shared = iv;
        else if (hkey(key, "embedding_length_per_layer_input")) mf->n_embd_per_layer = iv;
        else if (hkey(key, "rope.dimension_count")) mf->n_rot_full = iv;
        else if (hkey(key, "rope.dimension_count_swa")) mf->n_rot_swa = iv;
        else if (is(key, "qwen35.block_count")) mf->n_layer = iv;
        else if (is(key, "qwen35.context_length")) mf->n_ctx_train = iv;
        else if (is(key, "qwen35.embedding_length")) mf->n_embd = iv;
        else if (is(key, "qwen35.feed_forward_length")) {
            for (int j = 0; j < G4_MAX_LAYERS; j++) mf->n_ff[j] = iv;
            mf->ff_len_off = off;
            mf->ff_len_vt = (int)vt;
        }
        else if (is(key, "qwen35.attention.head_count")) mf->n_head = iv;
        else if (is(key, "qwen35.attention.head_count_kv")) mf->n_head_kv = iv;
        else if (is(key, "qwen35.attention.key_length")) mf->n_embd_head_k = iv;
        else if (is(key, "qwen35.attention.value_length")) mf->n_embd_head_v = iv;
        else if (is(key, "qwen35.attention.layer_norm_rms_epsilon")) mf->rms_eps = (float)v;
        else if (is(key, "qwen35.rope.freq_base")) mf->rope_base_full = (float)v;
        else if (is(key, "qwen35.rope.dimension_count")) mf->n_rot_full = iv;
        else if (is(key, "qwen35.full_attention_interval")) mf->full_attn_interval = iv;
        else if (is(key, "qwen35.ssm.conv_kernel")) mf->ssm_d_conv = iv;
        else if (is(key, "qwen35.ssm.inner_size")) mf->ssm_d_inner = iv;
        else if (is(key, "qwen35.ssm.state_size")) mf->ssm_d_state = iv;
        else if (is(key, "qwen35.ssm.time_step_rank")) mf->ssm_dt_rank = iv;
        else if (is(key, "qwen35.ssm.group_count")) mf->ssm_n_group = iv;
        else if (is(key, "tokenizer.ggml.bos_token_id")) mf->bos_id = iv;
        else if (is(key, "tokenizer.ggml.eos_token_id")) mf->eos_id = iv;
        else if (is(key, "tokenizer.ggml.eot_token_id")) mf->eot_id = iv;
        else if (is(key, "tokenizer.ggml.unknown_token_id")) mf->unk_id = iv;
        else if (is(key, "tokenizer.ggml.padding_token_id")) mf->pad_id = iv;
        else if (is(key, "tokenizer.ggml.add_bos_token")) mf->add_bos = v != 0;
        else if (is(key, "general.sampling.temp")) mf->meta_temp = (float)v;
        else if (is(key, "general.sampling.top_p")) mf->meta_top_p = (float)v;
        else if (is(key, "general.sampling.top_k")) mf->meta_top_k = iv;
    }
    if (r.bad) return fail(mf, "header parse error");
    mf->kv_end = (uint64_t)(r.p - (const uint8_t *)base);

    // ---- tensor table (gguf.c:303-333) ----
    if (!r.fits(mf->n_tensors, 24)) return fail(mf, "tensor info parse error");   // name length, ndim, type, offset
    mf->tensors = (g4_tensor *)std::calloc(mf->n_tensors ? mf->n_tensors : 1, sizeof(g4_tensor));
    if (!mf->tensors) return fail(mf, "out of memory for the tensor table");
    for (uint64_t i = 0; i < mf->n_tensors && !r.bad; i++) {
        g4_tensor *t = &mf->tensors[i];
        const g4_str name = r.str();
        const size_t n = name.len < sizeof t->name - 1 ? name.len : sizeof t->name - 1;
        if (name.ptr) std::memcpy(t->name, name.ptr, n);
        t->name[n] = 0;
        t->ndim = (int)r.get<uint32_t>();
        if (t->ndim > 4 || t->ndim < 0) {
            r.bad = true;
            break;
        }
        t->ne[0] = t->ne[1] = t->ne[2] = t->ne[3] = 1;
        for (int d = 0; d < t->ndim; d++) t->ne[d] = (int64_t)r.get<uint64_t>();
        t->type = (int)r.get<uint32_t>();
        t->offset = r.get<uint64_t>();
    }
    if (r.bad) return fail(mf, "tensor info parse error");
    if (mf->alignment == 0) return fail(mf, "bad alignment");
    const uint64_t header_end = (uint64_t)(r.p - (const uint8_t *)base);
    mf->data_start = (header_end + mf->alignment - 1) / mf->alignment * mf->alignment;
    if (mf->data_start > mf->map_size) return fail(mf, "tensor data past the end of the file");
    for (uint64_t i = 0; i < mf->n_tensors; i++) {
        g4_tensor *t = &mf->tensors[i];
        // every dimension at least 1, a row no longer than the file could hold
        // (at most 4 elements per byte in any type), and the byte count
        // computed without overflow, so a corrupt table cannot wrap the
        // bounds check below
        bool shape_ok = t->ne[0] >= 1 && (uint64_t)t->ne[0] <= 4 * mf->map_size;
        uint64_t rows = 1;
        for (int d = 1; d < 4 && shape_ok; d++)
            shape_ok = t->ne[d] >= 1 && !__builtin_mul_overflow(rows, (uint64_t)t->ne[d], &rows);
        if (!shape_ok) return fail(mf, "tensor %s has a bad shape", t->name);
        const size_t rs = g4_row_size(t->type, t->ne[0]);
        if (!rs) return fail(mf, "tensor %s has an unsupported type or row length", t->name);
        uint64_t bytes = 0;
        if (__builtin_mul_overflow((uint64_t)rs, rows, &bytes) || t->offset > mf->map_size || bytes > mf->map_size ||
            mf->data_start + t->offset + bytes > mf->map_size)
            return fail(mf, "tensor %s out of bounds", t->name);
        t->data = (const uint8_t *)base + mf->data_start + t->offset;
    }

    // ---- architecture (gguf.c:336-403) ----
    mf->is_assistant = std::strcmp(mf->arch, "gemma4-assistant") == 0;
    mf->is_qwen35 = std::strcmp(mf->arch, "qwen35") == 0;
    if (mf->is_qwen35) {
        if (mf->n_layer > G4_MAX_LAYERS) return fail(mf, "too many layers");
        if (mf->full_attn_interval == 0) mf->full_attn_interval = 4;
        if (mf->full_attn_interval > 0)
            for (int i = 0; i < mf->n_layer; i++) mf->is_recr[i] = (i + 1) % mf->full_attn_interval != 0;
        mf->n_vocab = mf->tok_n;
        return 0;
    }
    if (std::strcmp(mf->arch, "gemma4") != 0 && !mf->is_assistant)
        return fail(mf, "unsupported architecture '%s' (need gemma4, gemma4-assistant, or qwen35)", mf->arch);
    mf->add_bos = true;                               // gemma4 always adds BOS (gguf.c:383-385)
    if (mf->n_layer > G4_MAX_LAYERS || mf->n_layer < 0 || mf->n_kv_shared < 0 || mf->n_kv_shared > mf->n_layer)
        return fail(mf, "bad layer config");
    mf->n_layer_kv = mf->n_layer - mf->n_kv_shared;
    if (!mf->is_assistant && mf->n_layer_kv < 2) return fail(mf, "bad layer config");
    if (verbose)
        std::fprintf(stderr, "g4: %s: %llu tensors, %llu kv, data @ %llu; arch=%s n_layer=%d n_embd=%d n_vocab=%d\n", path,
                     (unsigned long long)mf->n_tensors, (unsigned long long)mf->n_kv, (unsigned long long)mf->data_start,
                     mf->arch, mf->n_layer, mf->n_embd, mf->tok_n);
    mf->n_vocab = mf->tok_n;
    return 0;
}
