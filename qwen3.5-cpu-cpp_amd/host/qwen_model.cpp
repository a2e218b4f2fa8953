// QwenModel over the device runtime: the constructor hands the SafeTensors tensor table to
// q35_model_create (one upload into the weight arena), step() is q35_model_step with the
// logits copied back, generate_greedy() keeps the whole loop on the device.
#include "qwen_model.h"

#include <iostream>

#include "q35_internal.h"

QwenModel::QwenModel(SafeTensors& weights, const ModelConfig& cfg, int max_context) : cfg_(cfg) {
    std::vector<q35_tensor> table;
    weights.device_table(&table);
    q35_dims d;
    q35::dims_from_config(cfg_, &d);
    const q35_status st = q35_model_create(&d, table.data(), static_cast<int32_t>(table.size()), max_context, &m_);
    if (st != Q35_OK) {
        std::cerr << "[qwen] " << q35_last_error() << "\n";
        m_ = nullptr;
        return;
    }
    ok_ = true;
    logits_.assign(static_cast<size_t>(cfg_.vocab_size), 0.0f);
    q35_budget b{};
    q35_model_budget(m_, &b);
    budget_.weight_bytes = b.weight_bytes;
    budget_.gdn_state_bytes = b.gdn_state_bytes;
    budget_.gdn_conv_bytes = b.gdn_conv_bytes;
    budget_.kv_cache_bytes = b.kv_cache_bytes;
    budget_.activation_bytes = b.activation_bytes;
    budget_.vision_scratch_bytes = 0;
    std::cerr << "[qwen] device arenas planned (max_context=" << max_context << "): weights "
              << budget_.weight_bytes / (1024 * 1024) << " MB, gdn_state " << budget_.gdn_state_bytes / 1024
              << " KB, gdn_conv_state " << budget_.gdn_conv_bytes / 1024 << " KB, kv_cache "
              << budget_.kv_cache_bytes / 1024 << " KB, scratch " << budget_.activation_bytes / 1024 << " KB\n";
}

QwenModel::~QwenModel() { q35_model_destroy(m_); }

void QwenModel::reset() {
    if (m_) q35_model_reset(m_);
}

int QwenModel::position() const { return m_ ? static_cast<int>(q35_model_position(m_)) : 0; }

const std::vector<float>& QwenModel::step(int token_id) {
    if (m_ && q35_model_step(m_, token_id, logits_.data(), nullptr) != Q35_OK)
        std::cerr << "[qwen] step: " << q35_last_error() << "\n";
    return logits_;
}

std::vector<int> QwenModel::generate_greedy(const std::vector<int>& prompt, int n_new) {
    std::vector<int> out(static_cast<size_t>(n_new > 0 ? n_new : 0));
    if (!m_ || prompt.empty() || n_new <= 0) return {};
    std::vector<int32_t> pr(prompt.begin(), prompt.end());
    if (q35_model_generate_greedy(m_, pr.data(), static_cast<int32_t>(pr.size()), n_new, out.data()) != Q35_OK) {
        std::cerr << "[qwen] generate_greedy: " << q35_last_error() << "\n";
        return {};
    }
    return out;
}
