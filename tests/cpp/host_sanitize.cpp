// Host-side readers and planner under AddressSanitizer / UndefinedBehaviorSanitizer: the
// config.json reader, the safetensors reader (every accessor on every tensor) and the memory
// equation, built with g++ from the library's own host sources (no GPU code involved).
// Test infrastructure, driven by tests/test_host_sanitizers.py:
//   host_sanitize cfg:<config.json> | st:<model dir or .safetensors> | budget:<config.json> ...
// prints one line per argument; any sanitizer report aborts the run with a non-zero status.
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "memory_budget.h"
#include "model_config.h"
#include "safetensors_loader.h"

namespace {

void check_config(const std::string& path) {
    ModelConfig cfg;
    const bool ok = load_model_config(path, cfg);
    std::printf("cfg %d hidden=%d layers=%d gdn=%d attn=%d vocab=%d ffn=%d theta=%g eps=%g n_params=%lld\n",
                ok ? 1 : 0, cfg.hidden_size, cfg.n_layers_total, cfg.n_layers_gdn, cfg.n_layers_attn,
                cfg.vocab_size, cfg.ffn_intermediate, cfg.rope_theta,
                static_cast<double>(cfg.rms_norm_eps), static_cast<long long>(cfg.n_params));
}

void check_tensors(const std::string& path) {
    SafeTensors st;
    const bool is_file = path.size() > 12 && path.compare(path.size() - 12, 12, ".safetensors") == 0;
    const bool ok = is_file ? st.load(path) : st.load_model(path);
    double sum = 0.0;
    int64_t rows_read = 0;
    for (const auto& kv : st.entries()) {
        const std::string& name = kv.first;
        const SafeTensors::Entry& e = kv.second;
        if (!st.has(name) || st.find(name) != &e || !st.data(name)) std::printf("st lookup mismatch %s\n", name.c_str());
        const WeightView w = st.view(name);
        (void)w;
        int64_t n = 0;
        if (const float* f = st.get_f32(name, &n)) {
            for (int64_t i = 0; i < n; ++i) sum += f[i];
        }
        if (e.shape.size() == 2 && e.shape[0] > 0 && e.shape[1] > 0) {
            std::vector<float> row(static_cast<size_t>(e.shape[1]));
            for (int64_t r : {int64_t{0}, e.shape[0] - 1})
                if (st.get_row_f32(name, r, row.data())) ++rows_read;
            // out-of-range rows are refused, not read
            if (st.get_row_f32(name, e.shape[0], row.data()) || st.get_row_f32(name, -1, row.data()))
                std::printf("st row past the end accepted: %s\n", name.c_str());
        }
    }
    std::vector<q35_tensor> table;
    st.device_table(&table);
    std::printf("st %d tensors=%zu table=%zu rows=%lld sum=%.6g\n", ok ? 1 : 0, st.entries().size(),
                table.size(), static_cast<long long>(rows_read), sum);
}

void check_budget(const std::string& path) {
    ModelConfig cfg;
    load_model_config(path, cfg);
    for (int ctx : {0, 1, 4096, 131072}) {
        for (int kvb : {2, 4}) {
            const MemoryBudget b = compute_budget(cfg, 2, ctx, kvb);
            const int64_t m = solve_max_context(cfg, size_t{288} << 30, b.weight_bytes, b.gdn_state_bytes,
                                                b.activation_bytes, b.vision_scratch_bytes, size_t{1} << 30, kvb);
            std::printf("budget ctx=%d kvb=%d total=%zu kv=%zu max_ctx=%lld\n", ctx, kvb, b.total(),
                        b.kv_cache_bytes, static_cast<long long>(m));
        }
    }
}

}  // namespace

int main(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        const size_t c = a.find(':');
        const std::string kind = a.substr(0, c), path = c == std::string::npos ? "" : a.substr(c + 1);
        if (kind == "cfg") check_config(path);
        else if (kind == "st") check_tensors(path);
        else if (kind == "budget") check_budget(path);
        else {
            std::fprintf(stderr, "unknown argument %s\n", a.c_str());
            return 2;
        }
        std::fflush(stdout);
    }
    return 0;
}
