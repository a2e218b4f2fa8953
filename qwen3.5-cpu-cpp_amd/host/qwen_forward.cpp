// QwenForward over the device runtime: one device model, made by the first prefill and kept,
// runs every prompt through the chunked path (q35_model_prefill) with the reference
// prefill's output head: the embedding over all its rows (src/qwen_forward.cpp:193-199).
// A longer prompt grows the model's context (q35_model_reserve_context); the weights are
// uploaded once.
#include "qwen_forward.h"

#include <algorithm>
#include <iostream>

#include "q35_internal.h"

QwenForward::~QwenForward() { q35_model_destroy(m_); }

bool QwenForward::prefill(const std::vector<int>& ids, std::vector<float>& logits_out) {
    const int seq = static_cast<int>(ids.size());
    if (seq == 0) return false;
    if (!m_) {
        std::vector<q35_tensor> table;
        w_.device_table(&table);
        q35_dims d;
        q35::dims_from_config(cfg_, &d);
        if (q35_model_create(&d, table.data(), static_cast<int32_t>(table.size()), std::max(seq, kMinContext), &m_) !=
                Q35_OK ||
            q35_model_set_prefill_head(m_, Q35_HEAD_EMBEDDING) != Q35_OK) {
            std::cerr << "[qwen] " << q35_last_error() << "\n";
            q35_model_destroy(m_);
            m_ = nullptr;
            return false;
        }
    }
    if (seq > q35_model_max_context(m_)) {
        // room for prompts up to twice as long first; if that does not fit, exactly this one
        const int64_t want = std::max<int64_t>(seq, 2 * q35_model_max_context(m_));
        if (q35_model_reserve_context(m_, want) != Q35_OK &&
            (want == seq || q35_model_reserve_context(m_, seq) != Q35_OK)) {
            std::cerr << "[qwen] prefill: " << q35_last_error() << "\n";
            return false;
        }
    }
    logits_out.assign(static_cast<size_t>(seq) * static_cast<size_t>(q35_model_prefill_logits_width(m_)), 0.0f);
    std::vector<int32_t> v(ids.begin(), ids.end());
    if (q35_model_prefill(m_, v.data(), seq, logits_out.data()) != Q35_OK) {
        std::cerr << "[qwen] prefill: " << q35_last_error() << "\n";
        return false;
    }
    return true;
}
