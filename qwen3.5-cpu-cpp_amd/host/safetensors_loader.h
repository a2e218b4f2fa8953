#pragma once
// Safetensors checkpoint reader (8-byte little-endian header length, a JSON tensor table,
// then raw little-endian tensor data).
//
// Drop-in for the reference's include/safetensors_loader.h:24-74 (same class and methods,
// plus device_table). Shards are memory-mapped read-only instead of read into heap buffers,
// so a 3.5 GB checkpoint costs no resident copy until the weights are uploaded to the
// device; each tensor's byte range and size are checked against its shard when it loads.
#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/q35.h"
#include "weight_view.h"

class SafeTensors {
public:
    struct Entry {
        std::string dtype;  // "BF16", "F32", ...
        std::vector<int64_t> shape;
        int shard = 0;
        size_t abs_offset = 0;  // byte offset of the data inside its shard file
        size_t nbytes = 0;
        int64_t numel() const;
    };

    SafeTensors() = default;
    SafeTensors(const SafeTensors&) = delete;
    SafeTensors& operator=(const SafeTensors&) = delete;
    ~SafeTensors();

    // Every *.safetensors file of model_dir, in sorted file-name order.
    bool load_model(const std::string& model_dir);
    bool load(const std::string& path);

    const Entry* find(const std::string& name) const;
    bool has(const std::string& name) const { return find(name) != nullptr; }

    // fp32 copy of a tensor (bf16 widened exactly), converted once and cached.
    const float* get_f32(const std::string& name, int64_t* out_numel = nullptr);
    // In-place view of the mapped data.
    WeightView view(const std::string& name) const;
    // Row `row` of a 2-D tensor as fp32 (embedding lookup); false when out of range.
    bool get_row_f32(const std::string& name, int64_t row, float* dst) const;
    // Raw pointer to a tensor's bytes (nullptr when absent).
    const void* data(const std::string& name) const;

    const std::unordered_map<std::string, Entry>& entries() const { return entries_; }

    // The tensor table of q35_model_create: one q35_tensor per entry, pointing at the mapped
    // bytes (valid while this object lives and is not reloaded).
    void device_table(std::vector<q35_tensor>* out) const;

private:
    struct Shard {
        void* map = nullptr;
        size_t size = 0;
    };
    bool parse_shard(const std::string& path);
    void release();
    std::vector<Shard> shards_;
    std::unordered_map<std::string, Entry> entries_;
    std::unordered_map<std::string, std::vector<float>> f32_cache_;
};

// bf16 is the upper half of an fp32: widening is exact.
inline float bf16_to_f32(uint16_t h) {
    const uint32_t bits = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}
