// gguf-model.h drop-in: GGUF v2/v3 reader over a read-only mapping, plus a view of synthetic models.
//
// Behaviour follows the reference (src/gguf-model.cpp): the file is mapped read-only (55-87), every
// tensor's byte range is validated against the file size at open (110-162, 164-200), views point
// into the mapping with GGML ne order, and lookups by name report "missing GGUF tensor: <name>"
// (230-245).  GGML's gguf parser is not available, so the container format (magic "GGUF", version,
// counts, typed key/value pairs, tensor infos, aligned data section) is read here directly.
#include "gguf-model.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <limits>
#include <map>
#include <string>
#include <vector>

#include "qwenasr_amd.h"

struct gguf_context {
    struct Tensor {
        std::string name;
        ggml_type type = GGML_TYPE_COUNT;
        std::vector<int64_t> ne;
        size_t offset = 0;     // relative to the data section
        size_t nbytes = 0;
        const void * data = nullptr;
    };
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> by_name;
    std::map<std::string, uint64_t> u64s;
    std::map<std::string, double> f64s;
    std::map<std::string, std::string> strs;
    std::map<std::string, uint64_t> array_lens;
};

namespace {

void set_error(std::string * error, const std::string & message) {
    if (error) *error = message;
}

struct Reader {
    const uint8_t * p;
    size_t size;
    size_t pos = 0;
    bool ok = true;

    bool need(size_t n) {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1ull << 32) || !need(static_cast<size_t>(n))) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p + pos), static_cast<size_t>(n));
        pos += static_cast<size_t>(n);
        return s;
    }
};

// GGUF value types (the GGUF specification): 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
// 8 string, 9 array, 10 u64, 11 i64, 12 f64.
size_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

bool read_value(Reader & r, uint32_t type, const std::string & key, gguf_context * ctx) {
    if (type == 8) {
        ctx->strs[key] = r.str();
        return r.ok;
    }
    if (type == 9) {
        const uint32_t et = r.get<uint32_t>();
        const uint64_t n = r.get<uint64_t>();
        if (!r.ok) return false;
        ctx->array_lens[key] = n;
        if (et == 8) {
            for (uint64_t i = 0; i < n && r.ok; ++i) (void)r.str();
            return r.ok;
        }
        const size_t es = scalar_size(et);
        if (es == 0 || n > (std::numeric_limits<size_t>::max() / es)) return false;
        if (!r.need(static_cast<size_t>(n) * es)) return false;
        r.pos += static_cast<size_t>(n) * es;
        return true;
    }
    const size_t es = scalar_size(type);
    if (es == 0 || !r.need(es)) return false;
    uint8_t raw[8] = {0};
    std::memcpy(raw, r.p + r.pos, es);
    r.pos += es;
    switch (type) {
        case 0: ctx->u64s[key] = raw[0]; break;
        case 2: { uint16_t v; std::memcpy(&v, raw, 2); ctx->u64s[key] = v; break; }
        case 4: { uint32_t v; std::memcpy(&v, raw, 4); ctx->u64s[key] = v; break; }
        case 10: { uint64_t v; std::memcpy(&v, raw, 8); ctx->u64s[key] = v; break; }
        case 5: { int32_t v; std::memcpy(&v, raw, 4); if (v >= 0) ctx->u64s[key] = static_cast<uint64_t>(v); break; }
        case 6: { float v; std::memcpy(&v, raw, 4); ctx->f64s[key] = v; break; }
        case 12: { double v; std::memcpy(&v, raw, 8); ctx->f64s[key] = v; break; }
        default: break;
    }
    return true;
}

bool type_bytes(ggml_type t, uint64_t n_elems, size_t * out) {
    size_t es = 0;
    if (t == GGML_TYPE_F32) es = 4;
    else if (t == GGML_TYPE_F16 || t == GGML_TYPE_BF16) es = 2;
    else return false;
    if (n_elems > std::numeric_limits<size_t>::max() / es) return false;
    *out = static_cast<size_t>(n_elems) * es;
    return true;
}

bool parse(const uint8_t * data, size_t size, gguf_context * ctx, size_t * data_offset, std::string * error) {
    Reader r{data, size};
    if (!r.need(4) || std::memcmp(data, "GGUF", 4) != 0) {
        set_error(error, "not a GGUF file (bad magic)");
        return false;
    }
    r.pos = 4;
    const uint32_t version = r.get<uint32_t>();
    if (version != 2 && version != 3) {
        set_error(error, "unsupported GGUF version " + std::to_string(version));
        return false;
    }
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    if (!r.ok || n_tensors > (1ull << 24) || n_kv > (1ull << 24)) {
        set_error(error, "corrupt GGUF header");
        return false;
    }
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = r.str();
        const uint32_t type = r.get<uint32_t>();
        if (!r.ok || !read_value(r, type, key, ctx)) {
            set_error(error, "corrupt GGUF key/value section");
            return false;
        }
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        gguf_context::Tensor t;
        t.name = r.str();
        const uint32_t n_dims = r.get<uint32_t>();
        if (!r.ok || n_dims == 0 || n_dims > 4) {
            set_error(error, "corrupt GGUF tensor info");
            return false;
        }
        uint64_t n_elems = 1;
        for (uint32_t d = 0; d < n_dims; ++d) {
            const uint64_t ne = r.get<uint64_t>();
            if (ne == 0 || ne > (1ull << 40) || n_elems > (1ull << 62) / ne) {
                set_error(error, "corrupt GGUF tensor shape: " + t.name);
                return false;
            }
            n_elems *= ne;
            t.ne.push_back(static_cast<int64_t>(ne));
        }
        t.type = static_cast<ggml_type>(r.get<uint32_t>());
        t.offset = static_cast<size_t>(r.get<uint64_t>());
        if (!r.ok) {
            set_error(error, "corrupt GGUF tensor info");
            return false;
        }
        if (!type_bytes(t.type, n_elems, &t.nbytes)) t.nbytes = 0;   // other types are listed, not viewable
        ctx->by_name[t.name] = ctx->tensors.size();
        ctx->tensors.push_back(std::move(t));
    }
    uint64_t alignment = 32;
    auto it = ctx->u64s.find("general.alignment");
    if (it != ctx->u64s.end() && it->second > 0 && (it->second & (it->second - 1)) == 0) alignment = it->second;
    const size_t off = (r.pos + alignment - 1) / alignment * alignment;
    *data_offset = off;
    for (auto & t : ctx->tensors) {
        if (off > size || t.offset > size - off || t.nbytes > size - off - t.offset) {
            set_error(error, "tensor data extends beyond GGUF file: " + t.name);
            return false;
        }
        t.data = data + off + t.offset;
    }
    return true;
}

bool view_of(const gguf_context::Tensor & t, QwenAsrGgufTensorView * out, std::string * error) {
    if (t.nbytes == 0 || !t.data) {
        set_error(error, "unsupported GGUF tensor type: " + t.name);
        return false;
    }
    if (out) {
        out->name = t.name;
        out->type = t.type;
        out->ne = t.ne;
        out->nbytes = t.nbytes;
        out->offset = t.offset;
        out->data = t.data;
    }
    return true;
}

}  // namespace

bool qwenasr_gguf_model_open(const char * path, QwenAsrGgufModel * model, std::string * error) {
    if (!path || !model) {
        set_error(error, "qwenasr_gguf_model_open: path or model is null");
        return false;
    }
    qwenasr_gguf_model_close(model);
    model->fd = open(path, O_RDONLY);
    if (model->fd < 0) {
        set_error(error, std::string("failed to open GGUF file: ") + path + ": " + std::strerror(errno));
        return false;
    }
    struct stat st {};
    if (fstat(model->fd, &st) != 0 || st.st_size <= 0) {
        set_error(error, std::string("GGUF file is empty or unreadable: ") + path);
        qwenasr_gguf_model_close(model);
        return false;
    }
    model->file_size = static_cast<size_t>(st.st_size);
    void * ptr = mmap(nullptr, model->file_size, PROT_READ, MAP_PRIVATE, model->fd, 0);
    if (ptr == MAP_FAILED) {
        set_error(error, std::string("failed to mmap GGUF file: ") + path + ": " + std::strerror(errno));
        model->file_size = 0;
        qwenasr_gguf_model_close(model);
        return false;
    }
    model->mapping = static_cast<const uint8_t *>(ptr);
    model->gguf = new gguf_context();
    if (!parse(model->mapping, model->file_size, model->gguf, &model->data_offset, error)) {
        qwenasr_gguf_model_close(model);
        return false;
    }
    return true;
}

bool qwenasr_gguf_model_from_synthetic(const qa_model * synthetic, QwenAsrGgufModel * model, std::string * error) {
    if (!synthetic || !model) {
        set_error(error, "qwenasr_gguf_model_from_synthetic: null argument");
        return false;
    }
    qwenasr_gguf_model_close(model);
    qa_text_config c{};
    qa_model_config(synthetic, &c);
    gguf_context * ctx = new gguf_context();
    const int64_t H = c.hidden, QD = static_cast<int64_t>(c.n_heads) * c.head_dim,
                  KD = static_cast<int64_t>(c.n_kv_heads) * c.head_dim, I = c.intermediate;
    auto add = [&](const std::string & name, std::vector<int64_t> ne) {
        int64_t n = 0;
        const float * p = qa_model_tensor(synthetic, name.c_str(), &n);
        if (!p) return;
        gguf_context::Tensor t;
        t.name = name;
        t.type = GGML_TYPE_F32;
        t.ne = std::move(ne);
        t.nbytes = static_cast<size_t>(n) * sizeof(float);
        t.data = p;
        ctx->by_name[name] = ctx->tensors.size();
        ctx->tensors.push_back(std::move(t));
    };
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "text.blk." + std::to_string(l) + ".";
        add(p + "attn_norm.weight", {H});
        add(p + "ffn_norm.weight", {H});
        add(p + "attn_q.weight", {H, QD});
        add(p + "attn_k.weight", {H, KD});
        add(p + "attn_v.weight", {H, KD});
        add(p + "attn_output.weight", {QD, H});
        add(p + "attn_q_norm.weight", {c.head_dim});
        add(p + "attn_k_norm.weight", {c.head_dim});
        add(p + "ffn_gate.weight", {H, I});
        add(p + "ffn_up.weight", {H, I});
        add(p + "ffn_down.weight", {I, H});
    }
    add("text.token_embd.weight", {H, c.vocab});
    add("text.output_norm.weight", {H});
    add("text.output.weight", {H, c.vocab});
    ctx->u64s["qwen3-asr.text.vocab_size"] = static_cast<uint64_t>(c.vocab);
    ctx->u64s["qwen3-asr.text.hidden_size"] = static_cast<uint64_t>(c.hidden);
    ctx->u64s["qwen3-asr.text.intermediate_size"] = static_cast<uint64_t>(c.intermediate);
    ctx->u64s["qwen3-asr.text.num_hidden_layers"] = static_cast<uint64_t>(c.n_layers);
    ctx->u64s["qwen3-asr.text.num_attention_heads"] = static_cast<uint64_t>(c.n_heads);
    ctx->u64s["qwen3-asr.text.num_key_value_heads"] = static_cast<uint64_t>(c.n_kv_heads);
    ctx->u64s["qwen3-asr.text.head_dim"] = static_cast<uint64_t>(c.head_dim);
    ctx->f64s["qwen3-asr.text.rope_theta"] = c.rope_theta;
    ctx->f64s["qwen3-asr.text.rms_norm_eps"] = c.rms_norm_eps;
    ctx->u64s["qwen3-asr.token.endoftext_token_id"] = 151643;
    ctx->u64s["qwen3-asr.token.im_end_token_id"] = 151645;
    ctx->u64s["tokenizer.ggml.eos_token_id"] = 151645;
    model->gguf = ctx;
    return true;
}

void qwenasr_gguf_model_close(QwenAsrGgufModel * model) {
    if (!model) return;
    delete model->gguf;
    model->gguf = nullptr;
    if (model->mapping && model->fd >= 0) munmap(const_cast<uint8_t *>(model->mapping), model->file_size);
    if (model->fd >= 0) close(model->fd);
    model->mapping = nullptr;
    model->file_size = 0;
    model->data_offset = 0;
    model->fd = -1;
    model->meta = nullptr;
}

int64_t qwenasr_gguf_model_tensor_count(const QwenAsrGgufModel & model) {
    return model.gguf ? static_cast<int64_t>(model.gguf->tensors.size()) : 0;
}

bool qwenasr_gguf_model_tensor_by_index(const QwenAsrGgufModel & model, int64_t index, QwenAsrGgufTensorView * out,
                                        std::string * error) {
    if (!model.gguf) {
        set_error(error, "GGUF model is not open");
        return false;
    }
    if (index < 0 || index >= static_cast<int64_t>(model.gguf->tensors.size())) {
        set_error(error, "GGUF tensor index is out of range");
        return false;
    }
    return view_of(model.gguf->tensors[static_cast<size_t>(index)], out, error);
}

bool qwenasr_gguf_model_tensor_by_name(const QwenAsrGgufModel & model, const char * name, QwenAsrGgufTensorView * out,
                                       std::string * error) {
    if (!model.gguf || !name) {
        set_error(error, "GGUF model is not open or tensor name is null");
        return false;
    }
    auto it = model.gguf->by_name.find(name);
    if (it == model.gguf->by_name.end()) {
        set_error(error, std::string("missing GGUF tensor: ") + name);
        return false;
    }
    return view_of(model.gguf->tensors[it->second], out, error);
}

bool qwenasr_gguf_model_get_u32(const QwenAsrGgufModel & model, const char * key, uint32_t * out) {
    if (!model.gguf || !key || !out) return false;
    auto it = model.gguf->u64s.find(key);
    if (it == model.gguf->u64s.end() || it->second > 0xffffffffull) return false;
    *out = static_cast<uint32_t>(it->second);
    return true;
}

bool qwenasr_gguf_model_get_f32(const QwenAsrGgufModel & model, const char * key, float * out) {
    if (!model.gguf || !key || !out) return false;
    auto it = model.gguf->f64s.find(key);
    if (it == model.gguf->f64s.end()) return false;
    *out = static_cast<float>(it->second);
    return true;
}

bool qwenasr_gguf_model_get_str(const QwenAsrGgufModel & model, const char * key, std::string * out) {
    if (!model.gguf || !key || !out) return false;
    auto it = model.gguf->strs.find(key);
    if (it == model.gguf->strs.end()) return false;
    *out = it->second;
    return true;
}

bool qwenasr_gguf_model_get_array_len(const QwenAsrGgufModel & model, const char * key, uint64_t * out) {
    if (!model.gguf || !key || !out) return false;
    auto it = model.gguf->array_lens.find(key);
    if (it == model.gguf->array_lens.end()) return false;
    *out = it->second;
    return true;
}
