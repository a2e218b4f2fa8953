#pragma once
// Architecture constants of a hybrid Gated-DeltaNet + gated-attention Qwen3.5 model.
//
// Drop-in for the reference's include/model_config.h:11-76: same struct name, fields,
// defaults (the Qwen3.5-0.8B text config) and loader signature, so engine code written
// against the reference compiles unchanged.
#include <cstdint>
#include <string>

struct ModelConfig {
    std::string name = "qwen3.5-0.8b";
    int64_t n_params = 800'000'000;  // rough, recomputed by load_model_config

    int hidden_size = 1024;

    int n_layers_total = 24;
    int n_layers_gdn = 18;
    int n_layers_attn = 6;

    // Gated DeltaNet: k-heads carry q and k, v-heads carry v; v_heads is a multiple of
    // k_heads and each k-head serves v_heads / k_heads consecutive v-heads.
    int gdn_k_heads = 16;
    int gdn_v_heads = 16;
    int gdn_k_head_dim = 128;
    int gdn_v_head_dim = 128;
    int gdn_conv_kernel = 4;
    int gdn_n_heads = 16;    // alias of gdn_v_heads
    int gdn_head_dim = 128;  // alias of gdn_v_head_dim

    // Gated attention (GQA, q-projection emits q and an output gate per head).
    int attn_q_heads = 8;
    int attn_kv_heads = 2;
    int attn_head_dim = 256;
    bool attn_output_gate = true;
    bool attn_qk_norm = true;

    int ffn_intermediate = 3584;
    int vocab_size = 248320;
    int native_max_context = 262144;

    float rms_norm_eps = 1e-6f;
    bool tie_word_embeddings = true;

    double rope_theta = 10'000'000.0;
    float partial_rotary_factor = 0.25f;

    int attn_interval = 4;

    // Layer `layer` (0-based) is full attention when (layer + 1) is a multiple of
    // attn_interval: layers 3, 7, 11, ... for the 3:1 pattern.
    bool is_attention_layer(int layer) const { return ((layer + 1) % attn_interval) == 0; }
};

// Reads a Hugging Face config.json (its "text_config" object when present, else the top
// level). Keys that are absent keep their current value. False when the file cannot be
// opened (the config then keeps its defaults).
bool load_model_config(const std::string& config_json_path, ModelConfig& cfg);

enum class Precision { FP32 = 4, FP16 = 2, INT8 = 1, INT4_PACKED = 0 };
