// Memory equation (src/memory_budget.cpp:4-81 of the reference): the same byte counts, so
// a plan printed by either engine is comparable line by line.
#include "memory_budget.h"

#include <algorithm>

size_t estimate_activation_scratch(const ModelConfig& cfg) {
    const size_t ffn = static_cast<size_t>(cfg.ffn_intermediate) * sizeof(float) * 2;
    const size_t attn = static_cast<size_t>(cfg.attn_q_heads * cfg.attn_head_dim +
                                            2 * cfg.attn_kv_heads * cfg.attn_head_dim) *
                        sizeof(float);
    const size_t gdn = static_cast<size_t>(3 * cfg.gdn_n_heads * cfg.gdn_head_dim) * sizeof(float);
    return std::max({ffn, attn, gdn});
}

size_t estimate_vision_scratch(int max_tiles, int vit_dim, int patches_per_tile) {
    const size_t patches = static_cast<size_t>(max_tiles) * patches_per_tile * vit_dim * sizeof(float);
    const size_t working = static_cast<size_t>(patches_per_tile) * vit_dim * sizeof(float) * 2;
    return patches + working;
}

MemoryBudget compute_budget(const ModelConfig& cfg, int bytes_per_weight, int max_context,
                            int kv_bytes_per_elem, int max_vision_tiles, int vit_dim) {
    MemoryBudget b;
    b.weight_bytes = static_cast<size_t>(cfg.n_params) * static_cast<size_t>(bytes_per_weight);
    b.gdn_state_bytes = static_cast<size_t>(cfg.n_layers_gdn) * cfg.gdn_v_heads *
                        cfg.gdn_k_head_dim * cfg.gdn_v_head_dim * sizeof(float);
    b.gdn_conv_bytes = gdn_conv_state_bytes(cfg);
    b.kv_cache_bytes = static_cast<size_t>(cfg.n_layers_attn) * static_cast<size_t>(max_context) *
                       2 * cfg.attn_kv_heads * cfg.attn_head_dim * kv_bytes_per_elem;
    b.activation_bytes = estimate_activation_scratch(cfg);
    b.vision_scratch_bytes = estimate_vision_scratch(max_vision_tiles, vit_dim);
    return b;
}

int64_t solve_max_context(const ModelConfig& cfg, size_t ram_budget_bytes, size_t weight_bytes,
                          size_t gdn_state_bytes, size_t activation_bytes,
                          size_t vision_scratch_bytes, size_t safety_margin_bytes,
                          int kv_bytes_per_elem) {
    const size_t fixed = weight_bytes + gdn_state_bytes + activation_bytes +
                         vision_scratch_bytes + safety_margin_bytes;
    if (fixed >= ram_budget_bytes) return -1;
    const size_t per_token = static_cast<size_t>(cfg.n_layers_attn) * 2 * cfg.attn_kv_heads *
                             cfg.attn_head_dim * kv_bytes_per_elem;
    const int64_t ctx = static_cast<int64_t>((ram_budget_bytes - fixed) / per_token);
    return std::min<int64_t>(ctx, cfg.native_max_context);
}
