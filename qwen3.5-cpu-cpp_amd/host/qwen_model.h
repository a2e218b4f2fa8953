#pragma once
// Stateful single-sequence decoder on one MI355X.
//
// Drop-in for the reference's include/qwen_model.h:21-32: same class name, constructor,
// and public methods. The per-layer arenas, the step loop and both mixers run on the GPU
// through libq35.so (include/q35.h); step() returns the logits in a host vector like the
// reference. Device memory is planned once in the constructor (four arenas: weights,
// recurrent state, KV cache, scratch) and step() allocates nothing.
#include <string>
#include <vector>

#include "../../include/q35.h"
#include "memory_budget.h"
#include "model_config.h"
#include "safetensors_loader.h"

class QwenModel {
public:
    QwenModel(SafeTensors& weights, const ModelConfig& cfg, int max_context);
    ~QwenModel();
    QwenModel(const QwenModel&) = delete;
    QwenModel& operator=(const QwenModel&) = delete;

    void reset();                                  // clear all state, position -> 0
    const std::vector<float>& step(int token_id);  // returns logits [vocab]
    int position() const;

    std::vector<int> generate_greedy(const std::vector<int>& prompt, int n_new);

    const MemoryBudget& budget() const { return budget_; }
    bool ok() const { return ok_; }

    // Access to the device model for callers that use the C ABI directly.
    q35_model* device() const { return m_; }

private:
    ModelConfig cfg_;
    q35_model* m_ = nullptr;
    bool ok_ = false;
    std::vector<float> logits_;
    MemoryBudget budget_;
};
