// Host model layer: a synthetic Qwen3-ASR text model addressed by GGUF tensor names.
//
// Tensor names and shapes follow the reference's loader (src/text-decoder.cpp:191-228, 527-535):
// text.blk.{l}.{attn_norm,ffn_norm,attn_q,attn_k,attn_v,attn_output,attn_q_norm,attn_k_norm,
// ffn_gate,ffn_up,ffn_down}.weight, text.token_embd.weight, text.output_norm.weight,
// text.output.weight; linear weights are row-major [out][in] (GGML ne = [in, out]).
// Qwen3-ASR ties the LM head to the token embedding, so text.output.weight shares the embedding's
// host buffer (one N(0, 0.02) draw keyed "text.token_embd.weight").
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "common.hpp"

struct qa_model {
    qa_text_config cfg{};
    std::map<std::string, std::shared_ptr<std::vector<float>>> tensors;
};

namespace {

using Buf = std::shared_ptr<std::vector<float>>;

Buf normal(uint64_t seed, const std::string & name, size_t n, double stddev) {
    auto b = std::make_shared<std::vector<float>>(n);
    qa_synth_fill_normal(b->data(), n, seed, name.c_str(), stddev);
    return b;
}

Buf ones(size_t n) {
    return std::make_shared<std::vector<float>>(n, 1.0f);
}

}  // namespace

extern "C" int qa_model_synthetic(const qa_text_config * cfg, uint64_t seed, qa_model ** out) {
    using namespace qa;
    if (!out) return fail(QA_ERR_INVALID, "qa_model_synthetic: null output");
    *out = nullptr;
    if (!cfg || cfg->n_layers <= 0 || cfg->hidden <= 0 || cfg->n_heads <= 0 || cfg->n_kv_heads <= 0 ||
        cfg->head_dim <= 0 || cfg->intermediate <= 0 || cfg->vocab <= 0 || cfg->n_heads % cfg->n_kv_heads != 0) {
        return fail(QA_ERR_INVALID, "invalid text decoder configuration");
    }
    std::unique_ptr<qa_model> m(new qa_model());
    m->cfg = *cfg;
    const size_t H = static_cast<size_t>(cfg->hidden);
    const size_t QD = static_cast<size_t>(cfg->n_heads) * cfg->head_dim;
    const size_t KD = static_cast<size_t>(cfg->n_kv_heads) * cfg->head_dim;
    const size_t I = static_cast<size_t>(cfg->intermediate);
    const double sd = 0.02;
    try {
        for (int l = 0; l < cfg->n_layers; ++l) {
            const std::string p = "text.blk." + std::to_string(l) + ".";
            m->tensors[p + "attn_norm.weight"] = ones(H);
            m->tensors[p + "ffn_norm.weight"] = ones(H);
            m->tensors[p + "attn_q_norm.weight"] = ones(static_cast<size_t>(cfg->head_dim));
            m->tensors[p + "attn_k_norm.weight"] = ones(static_cast<size_t>(cfg->head_dim));
            m->tensors[p + "attn_q.weight"] = normal(seed, p + "attn_q.weight", QD * H, sd);
            m->tensors[p + "attn_k.weight"] = normal(seed, p + "attn_k.weight", KD * H, sd);
            m->tensors[p + "attn_v.weight"] = normal(seed, p + "attn_v.weight", KD * H, sd);
            m->tensors[p + "attn_output.weight"] = normal(seed, p + "attn_output.weight", H * QD, sd);
            m->tensors[p + "ffn_gate.weight"] = normal(seed, p + "ffn_gate.weight", I * H, sd);
            m->tensors[p + "ffn_up.weight"] = normal(seed, p + "ffn_up.weight", I * H, sd);
            m->tensors[p + "ffn_down.weight"] = normal(seed, p + "ffn_down.weight", H * I, sd);
        }
        Buf embd = normal(seed, "text.token_embd.weight", static_cast<size_t>(cfg->vocab) * H, sd);
        m->tensors["text.token_embd.weight"] = embd;
        m->tensors["text.output.weight"] = embd;
        m->tensors["text.output_norm.weight"] = ones(H);
    } catch (const std::bad_alloc &) {
        return fail(QA_ERR_ALLOC, "qa_model_synthetic: out of host memory");
    }
    *out = m.release();
    return QA_OK;
}

extern "C" int qa_model_round_bf16(qa_model * model) {
    if (!model) return qa::fail(QA_ERR_INVALID, "qa_model_round_bf16: null model");
    std::set<const std::vector<float> *> done;   // tied tensors share one buffer: round it once
    for (auto & kv : model->tensors) {
        if (!done.insert(kv.second.get()).second) continue;
        for (float & v : *kv.second) {
            uint32_t b;
            std::memcpy(&b, &v, 4);
            if ((b & 0x7f800000u) != 0x7f800000u) b += 0x7fffu + ((b >> 16) & 1u);   // nearest, ties to even
            b &= 0xffff0000u;
            std::memcpy(&v, &b, 4);
        }
    }
    return QA_OK;
}

extern "C" void qa_model_free(qa_model * model) { delete model; }

extern "C" const float * qa_model_tensor(const qa_model * model, const char * name, int64_t * n_elems) {
    if (n_elems) *n_elems = 0;
    if (!model || !name) return nullptr;
    auto it = model->tensors.find(name);
    if (it == model->tensors.end()) return nullptr;
    if (n_elems) *n_elems = static_cast<int64_t>(it->second->size());
    return it->second->data();
}

extern "C" int qa_model_config(const qa_model * model, qa_text_config * cfg) {
    if (!model || !cfg) return qa::fail(QA_ERR_INVALID, "qa_model_config: null argument");
    *cfg = model->cfg;
    return QA_OK;
}

extern "C" int qa_model_weights_view(const qa_model * model, qa_layer_weights * layers, int32_t n_layers,
                                     qa_model_weights * weights) {
    if (!model || !layers || !weights || n_layers != model->cfg.n_layers) {
        return qa::fail(QA_ERR_INVALID, "qa_model_weights_view: invalid arguments");
    }
    auto t = [&](const std::string & n) { return qa_model_tensor(model, n.c_str(), nullptr); };
    for (int l = 0; l < n_layers; ++l) {
        const std::string p = "text.blk." + std::to_string(l) + ".";
        qa_layer_weights & w = layers[l];
        w.attn_norm = t(p + "attn_norm.weight");
        w.ffn_norm = t(p + "ffn_norm.weight");
        w.q = t(p + "attn_q.weight");
        w.k = t(p + "attn_k.weight");
        w.v = t(p + "attn_v.weight");
        w.o = t(p + "attn_output.weight");
        w.q_norm = t(p + "attn_q_norm.weight");
        w.k_norm = t(p + "attn_k_norm.weight");
        w.gate = t(p + "ffn_gate.weight");
        w.up = t(p + "ffn_up.weight");
        w.down = t(p + "ffn_down.weight");
    }
    weights->layers = layers;
    weights->token_embd = t("text.token_embd.weight");
    weights->output_norm = t("text.output_norm.weight");
    weights->output = t("text.output.weight");
    return QA_OK;
}
