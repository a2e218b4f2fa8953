// QwenForward over the device runtime: (re)plans a device model sized for the prompt and
// calls q35_model_prefill. Logits rows cover the embedding rows, as in the reference
// (src/qwen_forward.cpp:196-199).
#include "qwen_forward.h"

#include <iostream>

#include "q35_internal.h"

QwenForward::~QwenForward() { q35_model_destroy(m_); }

bool QwenForward::prefill(const std::vector<int>& ids, std::vector<float>& logits_out) {
    const int seq = static_cast<int>(ids.size());
    if (seq == 0) return false;
    if (!m_ || planned_ < seq) {
        q35_model_destroy(m_);
        m_ = nullptr;
        std::vector<std::string> names;
        for (const auto& kv : w_.entries()) names.push_back(kv.first);
        std::vector<q35_tensor> table;
        for (const std::string& nm : names) {
            const SafeTensors::Entry* e = w_.find(nm);
            q35_tensor t{};
            t.name = nm.c_str();
            t.dtype = e->dtype == "BF16" ? 0 : e->dtype == "F32" ? 1 : 2;
            t.ndim = static_cast<int32_t>(e->shape.size() < 4 ? e->shape.size() : 4);
            for (int i = 0; i < t.ndim; ++i) t.shape[i] = e->shape[static_cast<size_t>(i)];
            t.data = w_.data(nm);
            table.push_back(t);
        }
        q35_dims d;
        q35::dims_from_config(cfg_, &d);
        if (q35_model_create(&d, table.data(), static_cast<int32_t>(table.size()), seq, &m_) != Q35_OK) {
            std::cerr << "[qwen] " << q35_last_error() << "\n";
            m_ = nullptr;
            return false;
        }
        planned_ = seq;
    }
    logits_out.assign(static_cast<size_t>(seq) * cfg_.vocab_size, 0.0f);
    std::vector<int32_t> v(ids.begin(), ids.end());
    if (q35_model_prefill(m_, v.data(), seq, logits_out.data()) != Q35_OK) {
        std::cerr << "[qwen] prefill: " << q35_last_error() << "\n";
        return false;
    }
    return true;
}
