#pragma once
// Whole-prompt forward pass on one MI355X.
//
// Drop-in for the reference's include/qwen_forward.h:18-25: prefill(ids, logits) runs the
// prompt from a zero state and writes [seq * embedding rows] logits from the embedding, as
// the reference's prefill does (its output head is embed_tokens even when the checkpoint has
// an lm_head). One device model serves every call: the weights are uploaded at the first
// prefill, and a longer prompt grows only the KV and scratch arenas.
#include <vector>

#include "../../include/q35.h"
#include "model_config.h"
#include "safetensors_loader.h"

class QwenForward {
public:
    QwenForward(SafeTensors& weights, const ModelConfig& cfg) : w_(weights), cfg_(cfg) {}
    ~QwenForward();
    QwenForward(const QwenForward&) = delete;
    QwenForward& operator=(const QwenForward&) = delete;

    // False when a weight is missing, an id is out of range, or the device fails.
    bool prefill(const std::vector<int>& ids, std::vector<float>& logits_out);

private:
    SafeTensors& w_;
    ModelConfig cfg_;
    q35_model* m_ = nullptr;
    static constexpr int kMinContext = 4096;  // KV capacity of the first device model at least
};
