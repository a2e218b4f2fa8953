// ref_harness.cpp -- C entry points around the unmodified Qwen3.5-CPU-cpp engine.
//
// TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile together with the reference's own
// sources (read in place from the reference tree, never copied) into oracle/_ref/. It is
// used to pin the oracle and to write the golden fixtures, and as the "reference" CPU
// baseline. The shipped library never links it.
//
// The reference keeps the per-layer state, the decoder's buffers and the two mixers
// private (include/qwen_model.h:52-80); the harness opens them by compiling the header
// with `private` read as `public`. Standard headers are included first so that only the
// reference's classes are affected.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iostream>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#define private public
#include "qwen_model.h"
#include "qwen_forward.h"
#include "forward_pass.h"
#include "memory_budget.h"
#include "model_config.h"
#include "safetensors_loader.h"
#undef private

namespace {
struct RefHandle {
    ModelConfig cfg;
    SafeTensors st;
    std::unique_ptr<QwenModel> model;
};
}  // namespace

extern "C" {

// Opens <dir>; n_layers > 0 truncates the stack to its first n_layers layers (the residual
// stream after step() is then the hidden state after layer n_layers - 1).
void *ref_open(const char *dir, int max_context, int n_layers) {
    auto *h = new RefHandle();
    load_model_config(std::string(dir) + "/config.json", h->cfg);
    if (!h->st.load_model(dir)) {
        delete h;
        return nullptr;
    }
    if (n_layers > 0 && n_layers < h->cfg.n_layers_total) {
        h->cfg.n_layers_total = n_layers;
        h->cfg.n_layers_attn = n_layers / h->cfg.attn_interval;
        h->cfg.n_layers_gdn = n_layers - h->cfg.n_layers_attn;
    }
    h->model.reset(new QwenModel(h->st, h->cfg, max_context));
    if (!h->model->ok()) {
        delete h;
        return nullptr;
    }
    return h;
}

void ref_close(void *p) { delete static_cast<RefHandle *>(p); }
void ref_reset(void *p) { static_cast<RefHandle *>(p)->model->reset(); }
int ref_position(void *p) { return static_cast<RefHandle *>(p)->model->position(); }
void ref_set_position(void *p, int pos) { static_cast<RefHandle *>(p)->model->pos_ = pos; }
int ref_vocab(void *p) { return static_cast<RefHandle *>(p)->cfg.vocab_size; }
int ref_hidden_size(void *p) { return static_cast<RefHandle *>(p)->cfg.hidden_size; }

int ref_step(void *p, int token, float *logits) {
    auto *h = static_cast<RefHandle *>(p);
    const std::vector<float> &lg = h->model->step(token);
    if (logits) std::memcpy(logits, lg.data(), lg.size() * sizeof(float));
    return 0;
}

int ref_generate_greedy(void *p, const int *prompt, int n_prompt, int n_new, int *out) {
    auto *h = static_cast<RefHandle *>(p);
    std::vector<int> pr(prompt, prompt + n_prompt);
    std::vector<int> g = h->model->generate_greedy(pr, n_new);
    for (size_t i = 0; i < g.size(); ++i) out[i] = g[i];
    return (int)g.size();
}

float *ref_hidden(void *p) { return static_cast<RefHandle *>(p)->model->hidden_.data(); }
float *ref_normed(void *p) { return static_cast<RefHandle *>(p)->model->normed_.data(); }
float *ref_gdn_state(void *p, int i) { return static_cast<RefHandle *>(p)->model->gdn_state_[i].data(); }
float *ref_conv_state(void *p, int i) { return static_cast<RefHandle *>(p)->model->conv_state_[i].data(); }
float *ref_kcache(void *p, int i) { return static_cast<RefHandle *>(p)->model->kcache_[i].data(); }
float *ref_vcache(void *p, int i) { return static_cast<RefHandle *>(p)->model->vcache_[i].data(); }

// One mixer of layer `layer` on the current normed_ buffer (set it through ref_normed),
// at the current position; writes the mixer output [hidden_size].
int ref_mixer(void *p, int layer, float *out) {
    auto *h = static_cast<RefHandle *>(p);
    QwenModel &m = *h->model;
    if (layer < 0 || layer >= (int)m.lw_.size()) return -1;
    m.sbreset();
    if (m.lw_[layer].is_attn) m.attn_step(m.lw_[layer], out);
    else m.gdn_step(m.lw_[layer], out);
    return 0;
}

// QwenForward::prefill over ids; logits gets n * vocab floats (vocab = embed rows).
int ref_prefill(void *p, const int *ids, int n, float *logits) {
    auto *h = static_cast<RefHandle *>(p);
    QwenForward fw(h->st, h->cfg);
    std::vector<int> v(ids, ids + n);
    std::vector<float> lg;
    if (!fw.prefill(v, lg)) return -1;
    if (logits) std::memcpy(logits, lg.data(), lg.size() * sizeof(float));
    return 0;
}

// Reference primitives (src/forward_pass.cpp).
void ref_rmsnorm(const float *x, const float *w, float *y, int n, float eps) { rmsnorm(x, w, y, n, eps); }
void ref_rmsnorm_gated(const float *x, const float *w, const float *g, float *y, int n, float eps) {
    rmsnorm_gated(x, w, g, y, n, eps);
}
void ref_l2norm(float *x, int n, float eps) { l2norm(x, n, eps); }
void ref_apply_rope(float *v, int rot, int pos, double theta) { apply_rope(v, rot, pos, theta); }
void ref_matmul_bf16(const uint16_t *W, const float *x, float *y, int out_dim, int in_dim) {
    WeightView wv;
    wv.bf16 = W;
    wv.numel = (int64_t)out_dim * in_dim;
    matmul(wv, x, y, out_dim, in_dim);
}

// Reference planner (src/memory_budget.cpp), on a config file.
int ref_budget(const char *config_path, int bytes_per_weight, int max_context, int kv_bytes,
               uint64_t *out6) {
    ModelConfig cfg;
    load_model_config(config_path, cfg);
    MemoryBudget b = compute_budget(cfg, bytes_per_weight, max_context, kv_bytes);
    out6[0] = b.weight_bytes;
    out6[1] = b.gdn_state_bytes;
    out6[2] = b.gdn_conv_bytes;
    out6[3] = b.kv_cache_bytes;
    out6[4] = b.activation_bytes;
    out6[5] = b.vision_scratch_bytes;
    return 0;
}
int64_t ref_solve_max_context(const char *config_path, uint64_t ram, uint64_t weight,
                              uint64_t gdn, uint64_t act, uint64_t vision, uint64_t margin,
                              int kv_bytes) {
    ModelConfig cfg;
    load_model_config(config_path, cfg);
    return solve_max_context(cfg, ram, weight, gdn, act, vision, margin, kv_bytes);
}
// ModelConfig as read by load_model_config: 16 ints/longs in a fixed order.
int ref_config(const char *config_path, int64_t *out16, double *theta, float *eps,
               float *partial) {
    ModelConfig cfg;
    bool ok = load_model_config(config_path, cfg);
    int64_t v[16] = {cfg.hidden_size, cfg.n_layers_total, cfg.n_layers_gdn, cfg.n_layers_attn,
                     cfg.gdn_k_heads, cfg.gdn_v_heads, cfg.gdn_k_head_dim, cfg.gdn_v_head_dim,
                     cfg.gdn_conv_kernel, cfg.attn_q_heads, cfg.attn_kv_heads, cfg.attn_head_dim,
                     cfg.ffn_intermediate, cfg.vocab_size, cfg.native_max_context, cfg.n_params};
    std::memcpy(out16, v, sizeof v);
    *theta = cfg.rope_theta;
    *eps = cfg.rms_norm_eps;
    *partial = cfg.partial_rotary_factor;
    return ok ? 0 : -1;
}

}  // extern "C"
