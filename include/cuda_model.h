// Drop-in for the reference's cuda_model.h (/root/reference/src/
// cuda_model.h:24-89): class CudaTransformer with the same constructor,
// forward(), prefill() and config(), over the C ABI in llm_engine_amd.h.
//
// It takes the caller's Checkpoint, Config and WeightType from the CPU
// model's header, model.h (model.h:11-63), which this build does not
// replace: include this header after the caller's include path has model.h.
//
// Weights, the KV cache and every activation stay in GPU memory; a call
// uploads its position and tokens and downloads the last row's logits. The
// first one-token forward() is captured into a HIP graph that later ones
// replay. Errors: std::runtime_error from the constructor (a HIP error, or a
// shape the attention kernels cannot run), std::out_of_range for a token
// outside the vocabulary or a bad position, std::invalid_argument for an
// empty prefill (model.h:87-103). Not safe from several host threads at once.
#pragma once

#include <cstddef>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "cuda_matmul.h"  // as the reference's header: callers use cuda_available() from it
#include "llm_engine_amd.h"
#include "model.h"

class CudaTransformer {
public:
    explicit CudaTransformer(const Checkpoint& ckpt, WeightType type = WeightType::f32)
        : cfg_(ckpt.config), logits_(ckpt.config.vocab_size) {
        const em_model_config c{cfg_.dim,        cfg_.hidden_dim, cfg_.n_layers, cfg_.n_heads,
                                cfg_.n_kv_heads, cfg_.vocab_size, cfg_.seq_len};
        const Weights& w = ckpt.weights;
        std::vector<em_layer_weights> layers;
        layers.reserve(w.layers.size());
        for (const LayerWeights& l : w.layers)
            layers.push_back({l.rms_att.data(), l.wqkv.data.data(), l.wo.data.data(),
                              l.rms_ffn.data(), l.w13.data.data(), l.w2.data.data()});
        if (layers.size() != cfg_.n_layers)
            throw std::runtime_error("CudaTransformer: checkpoint has " +
                                     std::to_string(layers.size()) + " layers, config " +
                                     std::to_string(cfg_.n_layers));
        const int rc = em_model_create(
            &c, w.token_embedding.data.data(), layers.data(), w.rms_final.data(),
            w.wcls.data.data(), type == WeightType::q8 ? EM_WEIGHTS_Q8 : EM_WEIGHTS_F32, &m_);
        if (rc != EM_OK) throw std::runtime_error(em_last_error());
    }
    ~CudaTransformer() { em_model_destroy(m_); }

    // load_checkpoint(path) and the constructor in one step, on the GPU
    // (em_model_load): no CPU-side Checkpoint. std::runtime_error for a file
    // the reference's loader rejects, with its message. Not in the
    // reference's class.
    static CudaTransformer load(const std::string& path, WeightType type = WeightType::f32) {
        em_model* raw = nullptr;
        const int rc = em_model_load(path.c_str(),
                                     type == WeightType::q8 ? EM_WEIGHTS_Q8 : EM_WEIGHTS_F32, &raw);
        if (rc == EM_EINVAL) throw std::invalid_argument(em_last_error());
        if (rc != EM_OK) throw std::runtime_error(em_last_error());
        // Owned here until the CudaTransformer holds it, so a throwing
        // constructor (the logits' allocation) does not leak the model.
        std::unique_ptr<em_model, int (*)(em_model*)> m(raw, em_model_destroy);
        em_model_config c{};
        em_model_config_get(m.get(), &c);
        Config cfg{};
        cfg.dim = c.dim;
        cfg.hidden_dim = c.hidden_dim;
        cfg.n_layers = c.n_layers;
        cfg.n_heads = c.n_heads;
        cfg.n_kv_heads = c.n_kv_heads;
        cfg.vocab_size = c.vocab_size;
        cfg.seq_len = c.seq_len;
        CudaTransformer t(m.get(), cfg);
        m.release();
        return t;
    }
    CudaTransformer(CudaTransformer&& o) noexcept
        : cfg_(o.cfg_), m_(o.m_), logits_(std::move(o.logits_)) {
        o.m_ = nullptr;
    }

    CudaTransformer(const CudaTransformer&) = delete;
    CudaTransformer& operator=(const CudaTransformer&) = delete;

    // As Transformer::forward() and Transformer::prefill() (model.h:87-103).
    const std::vector<float>& forward(int token, std::size_t pos) { return run(&token, 1, pos); }
    const std::vector<float>& prefill(const std::vector<int>& tokens, std::size_t pos) {
        if (tokens.empty()) throw std::invalid_argument("prefill: no tokens");
        return run(tokens.data(), tokens.size(), pos);
    }

    const Config& config() const { return cfg_; }

private:
    CudaTransformer(em_model* m, const Config& cfg) : cfg_(cfg), m_(m), logits_(cfg.vocab_size) {}

    const std::vector<float>& run(const int* tokens, std::size_t n, std::size_t pos) {
        const int rc = em_model_forward(m_, tokens, n, pos, logits_.data());
        if (rc == EM_ERANGE) throw std::out_of_range(em_last_error());
        if (rc == EM_EINVAL) throw std::invalid_argument(em_last_error());
        if (rc != EM_OK) throw std::runtime_error(em_last_error());
        return logits_;
    }

    Config cfg_;
    em_model* m_ = nullptr;
    std::vector<float> logits_;
};
