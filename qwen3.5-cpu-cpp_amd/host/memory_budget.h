#pragma once
// The memory equation that plans the device arenas.
//
// Drop-in for the reference's include/memory_budget.h:6-62 (same struct, functions and
// arithmetic, including the reference's choices that solve_max_context leaves the conv
// window out of its fixed costs and that weight_bytes uses the rough n_params). The
// device runtime sizes its weight arena from the actual tensor bytes instead, and keeps
// the conv window in its state arena (see qwen_model.h).
#include <cstddef>
#include <cstdint>

#include "model_config.h"

struct MemoryBudget {
    size_t weight_bytes = 0;
    size_t gdn_state_bytes = 0;
    size_t gdn_conv_bytes = 0;
    size_t kv_cache_bytes = 0;
    size_t activation_bytes = 0;
    size_t vision_scratch_bytes = 0;

    size_t total() const {
        return weight_bytes + gdn_state_bytes + gdn_conv_bytes + kv_cache_bytes +
               activation_bytes + vision_scratch_bytes;
    }
};

// (kernel - 1) fp32 inputs per conv channel per GDN layer, conv channels = 2*KD + VD.
inline size_t gdn_conv_state_bytes(const ModelConfig& cfg) {
    const size_t kd = static_cast<size_t>(cfg.gdn_k_heads) * cfg.gdn_k_head_dim;
    const size_t vd = static_cast<size_t>(cfg.gdn_v_heads) * cfg.gdn_v_head_dim;
    return static_cast<size_t>(cfg.n_layers_gdn) * (2 * kd + vd) * (cfg.gdn_conv_kernel - 1) *
           sizeof(float);
}

// weights = n_params * bytes_per_weight; gdn = L_gdn * VH * DK * DV * 4;
// kv = L_attn * max_context * 2 * NKV * HD * kv_bytes_per_elem.
MemoryBudget compute_budget(const ModelConfig& cfg, int bytes_per_weight, int max_context,
                            int kv_bytes_per_elem, int max_vision_tiles = 4, int vit_dim = 1024);

// Largest context whose KV cache fits next to the fixed costs, capped at
// native_max_context; -1 when the fixed costs alone exceed the budget.
int64_t solve_max_context(const ModelConfig& cfg, size_t ram_budget_bytes, size_t weight_bytes,
                          size_t gdn_state_bytes, size_t activation_bytes,
                          size_t vision_scratch_bytes, size_t safety_margin_bytes,
                          int kv_bytes_per_elem);

size_t estimate_activation_scratch(const ModelConfig& cfg);
size_t estimate_vision_scratch(int max_tiles, int vit_dim, int patches_per_tile = 256);
