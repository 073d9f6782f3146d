// C entry points over the reference's CPU model, compiled from the source
// files under /root/reference/src by oracle/Makefile into
// oracle/_ref/libref_model.so. TEST INFRASTRUCTURE ONLY: the forward-pass
// tests compare this build's GPU model with it, logits per position, and
// read the reference loader's arrays to pin their own. Nothing in the
// product links it.
//
// Bindings (reference file:line):
//   ref_ckpt_load / ref_ckpt_config / ref_ckpt_array
//                         load_checkpoint, Checkpoint, Weights, LayerWeights
//                         (model.h:11-63, model.cpp:59-163)
//   ref_ckpt_new          a Checkpoint from arrays already in the CPU model's
//                         layout (no file), for models too large to write out
//   ref_model_new / ref_model_run / ref_model_free
//                         Transformer(ckpt, WeightType), forward / prefill
//                         (model.h:79-108, model.cpp:194-322)
//   ref_rope_tables       rope_tables (model.h:65-67, model.cpp:177-192)
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

#include "model.h"

namespace {

thread_local std::string g_error;

// 0 ok, 1 std::out_of_range, 2 std::invalid_argument, 3 anything else.
template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::out_of_range& e) {
        g_error = e.what();
        return 1;
    } catch (const std::invalid_argument& e) {
        g_error = e.what();
        return 2;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 3;
    }
}

std::size_t put(const std::vector<float>& v, float* out, std::size_t cap) {
    if (out && cap >= v.size()) std::memcpy(out, v.data(), v.size() * sizeof(float));
    return v.size();
}

}  // namespace

extern "C" {

const char* ref_model_error(void) { return g_error.c_str(); }

void* ref_ckpt_load(const char* path) {
    Checkpoint* c = nullptr;
    if (guarded([&] { c = new Checkpoint(load_checkpoint(path)); })) return nullptr;
    return c;
}

void ref_ckpt_free(void* h) { delete static_cast<Checkpoint*>(h); }

// cfg7: dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len.
// layers: 6 pointers per layer (rms_att, wqkv, wo, rms_ffn, w13, w2), each
// array in the layout of struct LayerWeights (model.h:29-36).
void* ref_ckpt_new(const std::size_t* cfg7, const float* emb, const float* const* layers,
                   const float* rms_final, const float* wcls) {
    Checkpoint* c = nullptr;
    if (guarded([&] {
            Config cfg{cfg7[0], cfg7[1], cfg7[2], cfg7[3], cfg7[4], cfg7[5], cfg7[6]};
            const std::size_t D = cfg.dim, H = cfg.hidden_dim, KV = cfg.kv_dim(), V = cfg.vocab_size;
            auto tensor = [](std::size_t r, std::size_t cols, const float* src) {
                Tensor t(r, cols);
                std::memcpy(t.data.data(), src, r * cols * sizeof(float));
                return t;
            };
            auto vec = [](std::size_t n, const float* src) { return std::vector<float>(src, src + n); };
            c = new Checkpoint{cfg, {}};
            Weights& w = c->weights;
            w.token_embedding = tensor(V, D, emb);
            for (std::size_t l = 0; l < cfg.n_layers; ++l) {
                const float* const* p = layers + 6 * l;
                w.layers.push_back({vec(D, p[0]), tensor(D, D + 2 * KV, p[1]), tensor(D, D, p[2]),
                                    vec(D, p[3]), tensor(D, 2 * H, p[4]), tensor(H, D, p[5])});
            }
            w.rms_final = vec(D, rms_final);
            w.wcls = tensor(D, V, wcls);
        }))
        return nullptr;
    return c;
}

// dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len.
void ref_ckpt_config(void* h, std::size_t* out7) {
    const Config& c = static_cast<Checkpoint*>(h)->config;
    const std::size_t v[7] = {c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads,
                              c.vocab_size, c.seq_len};
    std::memcpy(out7, v, sizeof v);
}

// Copies the named array (Transformer layout: projections in x out) into out
// when it holds `cap` floats or more; returns its size in floats, 0 if the
// name is unknown.
std::size_t ref_ckpt_array(void* h, const char* name, std::size_t layer, float* out,
                           std::size_t cap) {
    const Weights& w = static_cast<Checkpoint*>(h)->weights;
    const std::string n = name;
    if (n == "token_embedding") return put(w.token_embedding.data, out, cap);
    if (n == "rms_final") return put(w.rms_final, out, cap);
    if (n == "wcls") return put(w.wcls.data, out, cap);
    if (layer >= w.layers.size()) return 0;
    const LayerWeights& l = w.layers[layer];
    if (n == "rms_att") return put(l.rms_att, out, cap);
    if (n == "wqkv") return put(l.wqkv.data, out, cap);
    if (n == "wo") return put(l.wo.data, out, cap);
    if (n == "rms_ffn") return put(l.rms_ffn, out, cap);
    if (n == "w13") return put(l.w13.data, out, cap);
    if (n == "w2") return put(l.w2.data, out, cap);
    return 0;
}

void* ref_model_new(void* ckpt, int q8) {
    Transformer* t = nullptr;
    if (guarded([&] {
            t = new Transformer(*static_cast<Checkpoint*>(ckpt), q8 ? WeightType::q8 : WeightType::f32);
        }))
        return nullptr;
    return t;
}

void ref_model_free(void* h) { delete static_cast<Transformer*>(h); }

// prefill(tokens[0:n], pos), or forward(tokens[0], pos) when n == 1 and
// `single` is set; logits receives vocab_size floats on success.
int ref_model_run(void* h, const int* tokens, std::size_t n, std::size_t pos, int single,
                  float* logits) {
    Transformer* t = static_cast<Transformer*>(h);
    return guarded([&] {
        const std::vector<float>& out =
            (single && n == 1) ? t->forward(tokens[0], pos)
                               : t->prefill(std::vector<int>(tokens, tokens + n), pos);
        std::memcpy(logits, out.data(), out.size() * sizeof(float));
    });
}

void ref_rope_tables(void* ckpt, float* cos_out, float* sin_out) {
    std::vector<float> c, s;
    rope_tables(static_cast<Checkpoint*>(ckpt)->config, c, s);
    std::memcpy(cos_out, c.data(), c.size() * sizeof(float));
    std::memcpy(sin_out, s.data(), s.size() * sizeof(float));
}

}  // extern "C"
