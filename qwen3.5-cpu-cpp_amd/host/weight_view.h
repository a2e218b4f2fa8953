#pragma once
// Non-owning view of one weight tensor in a loaded checkpoint, bf16 or fp32.
// Same type as the reference's include/weight_view.h:7-12.
#include <cstdint>

struct WeightView {
    const uint16_t* bf16 = nullptr;
    const float* f32 = nullptr;
    int64_t numel = 0;
    bool ok() const { return bf16 != nullptr || f32 != nullptr; }
};
