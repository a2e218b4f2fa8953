// Host-only part of the C ABI: errors, config reading, the memory equation and the
// synthetic checkpoint writer. Nothing here touches the GPU.
#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <string>
#include <thread>
#include <vector>

#include "memory_budget.h"
#include "model_config.h"
#include "q35_internal.h"
#include "synth.h"

namespace q35 {

namespace {
thread_local std::string g_last_error;
}

q35_status fail(q35_status code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

void dims_from_config(const ModelConfig& c, q35_dims* d) {
    std::memset(d, 0, sizeof *d);
    d->hidden_size = c.hidden_size;
    d->n_layers_total = c.n_layers_total;
    d->n_layers_gdn = c.n_layers_gdn;
    d->n_layers_attn = c.n_layers_attn;
    d->gdn_k_heads = c.gdn_k_heads;
    d->gdn_v_heads = c.gdn_v_heads;
    d->gdn_k_head_dim = c.gdn_k_head_dim;
    d->gdn_v_head_dim = c.gdn_v_head_dim;
    d->gdn_conv_kernel = c.gdn_conv_kernel;
    d->attn_q_heads = c.attn_q_heads;
    d->attn_kv_heads = c.attn_kv_heads;
    d->attn_head_dim = c.attn_head_dim;
    d->ffn_intermediate = c.ffn_intermediate;
    d->vocab_size = c.vocab_size;
    d->native_max_context = c.native_max_context;
    d->n_params = c.n_params;
    d->rope_theta = c.rope_theta;
    d->rms_norm_eps = c.rms_norm_eps;
    d->partial_rotary_factor = c.partial_rotary_factor;
    d->attn_interval = c.attn_interval;
    d->tie_word_embeddings = c.tie_word_embeddings ? 1 : 0;
}

ModelConfig config_from_dims(const q35_dims& d) {
    ModelConfig c;
    c.hidden_size = d.hidden_size;
    c.n_layers_total = d.n_layers_total;
    c.n_layers_gdn = d.n_layers_gdn;
    c.n_layers_attn = d.n_layers_attn;
    c.gdn_k_heads = d.gdn_k_heads;
    c.gdn_v_heads = d.gdn_v_heads;
    c.gdn_k_head_dim = d.gdn_k_head_dim;
    c.gdn_v_head_dim = d.gdn_v_head_dim;
    c.gdn_conv_kernel = d.gdn_conv_kernel;
    c.gdn_n_heads = d.gdn_v_heads;
    c.gdn_head_dim = d.gdn_v_head_dim;
    c.attn_q_heads = d.attn_q_heads;
    c.attn_kv_heads = d.attn_kv_heads;
    c.attn_head_dim = d.attn_head_dim;
    c.ffn_intermediate = d.ffn_intermediate;
    c.vocab_size = d.vocab_size;
    c.native_max_context = static_cast<int>(d.native_max_context);
    c.n_params = d.n_params;
    c.rope_theta = d.rope_theta;
    c.rms_norm_eps = d.rms_norm_eps;
    c.partial_rotary_factor = d.partial_rotary_factor;
    c.attn_interval = d.attn_interval;
    c.tie_word_embeddings = d.tie_word_embeddings != 0;
    return c;
}

const char* last_error_cstr() { return g_last_error.c_str(); }

}  // namespace q35

namespace {

template <class F>
void parallel_for(int64_t n, int threads, F&& body) {
    if (threads <= 0) threads = static_cast<int>(std::max(1u, std::thread::hardware_concurrency()));
    threads = static_cast<int>(std::min<int64_t>(threads, std::max<int64_t>(1, n / 4096)));
    if (threads <= 1) {
        body(0, n);
        return;
    }
    std::vector<std::thread> pool;
    const int64_t per = (n + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        const int64_t b = t * per, e = std::min(n, b + per);
        if (b >= e) break;
        pool.emplace_back([&body, b, e] { body(b, e); });
    }
    for (auto& th : pool) th.join();
}

struct TensorSpec {
    std::string name;
    std::vector<int64_t> shape;
    int fill;  // 0: N(0, std), 1: zeros, 2: ones
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

std::vector<TensorSpec> checkpoint_layout(const q35_dims& d) {
    const int64_t H = d.hidden_size, I = d.ffn_intermediate, V = d.vocab_size;
    const int64_t NQ = d.attn_q_heads, NKV = d.attn_kv_heads, HD = d.attn_head_dim;
    const int64_t KD = static_cast<int64_t>(d.gdn_k_heads) * d.gdn_k_head_dim;
    const int64_t VD = static_cast<int64_t>(d.gdn_v_heads) * d.gdn_v_head_dim;
    const int64_t VH = d.gdn_v_heads, DV = d.gdn_v_head_dim, KER = d.gdn_conv_kernel;
    const std::string lm = "model.language_model.";
    std::vector<TensorSpec> t;
    t.push_back({lm + "embed_tokens.weight", {V, H}, 0});
    for (int l = 0; l < d.n_layers_total; ++l) {
        const std::string p = lm + "layers." + std::to_string(l) + ".";
        t.push_back({p + "input_layernorm.weight", {H}, 1});
        t.push_back({p + "post_attention_layernorm.weight", {H}, 1});
        t.push_back({p + "mlp.gate_proj.weight", {I, H}, 0});
        t.push_back({p + "mlp.up_proj.weight", {I, H}, 0});
        t.push_back({p + "mlp.down_proj.weight", {H, I}, 0});
        if ((l + 1) % d.attn_interval == 0) {
            const std::string a = p + "self_attn.";
            t.push_back({a + "q_proj.weight", {NQ * HD * 2, H}, 0});
            t.push_back({a + "k_proj.weight", {NKV * HD, H}, 0});
            t.push_back({a + "v_proj.weight", {NKV * HD, H}, 0});
            t.push_back({a + "o_proj.weight", {H, NQ * HD}, 0});
            t.push_back({a + "q_norm.weight", {HD}, 1});
            t.push_back({a + "k_norm.weight", {HD}, 1});
        } else {
            const std::string g = p + "linear_attn.";
            t.push_back({g + "in_proj_qkv.weight", {2 * KD + VD, H}, 0});
            t.push_back({g + "in_proj_z.weight", {VD, H}, 0});
            t.push_back({g + "in_proj_b.weight", {VH, H}, 0});
            t.push_back({g + "in_proj_a.weight", {VH, H}, 0});
            t.push_back({g + "conv1d.weight", {2 * KD + VD, 1, KER}, 0});
            t.push_back({g + "dt_bias", {VH}, 0});
            t.push_back({g + "A_log", {VH}, 0});
            t.push_back({g + "norm.weight", {DV}, 2});
            t.push_back({g + "out_proj.weight", {H, VD}, 0});
        }
    }
    t.push_back({lm + "norm.weight", {H}, 1});
    if (!d.tie_word_embeddings) t.push_back({"lm_head.weight", {V, H}, 0});
    return t;
}

std::string config_json(const q35_dims& d) {
    char buf[2048];
    std::snprintf(buf, sizeof buf,
                  "{\n  \"architectures\": [\"Qwen3_5ForCausalLM\"],\n  \"model_type\": \"qwen3_5\",\n"
                  "  \"text_config\": {\n"
                  "    \"hidden_size\": %d,\n    \"num_hidden_layers\": %d,\n"
                  "    \"full_attention_interval\": %d,\n    \"num_attention_heads\": %d,\n"
                  "    \"num_key_value_heads\": %d,\n    \"head_dim\": %d,\n"
                  "    \"linear_num_key_heads\": %d,\n    \"linear_num_value_heads\": %d,\n"
                  "    \"linear_key_head_dim\": %d,\n    \"linear_value_head_dim\": %d,\n"
                  "    \"linear_conv_kernel_dim\": %d,\n    \"intermediate_size\": %d,\n"
                  "    \"vocab_size\": %d,\n    \"max_position_embeddings\": %lld,\n"
                  "    \"rms_norm_eps\": %.9g,\n    \"rope_theta\": %.17g,\n"
                  "    \"partial_rotary_factor\": %.9g,\n    \"tie_word_embeddings\": %s\n"
                  "  }\n}\n",
                  d.hidden_size, d.n_layers_total, d.attn_interval, d.attn_q_heads,
                  d.attn_kv_heads, d.attn_head_dim, d.gdn_k_heads, d.gdn_v_heads,
                  d.gdn_k_head_dim, d.gdn_v_head_dim, d.gdn_conv_kernel, d.ffn_intermediate,
                  d.vocab_size, static_cast<long long>(d.native_max_context),
                  static_cast<double>(d.rms_norm_eps), d.rope_theta,
                  static_cast<double>(d.partial_rotary_factor),
                  d.tie_word_embeddings ? "true" : "false");
    return buf;
}

}  // namespace

extern "C" {

const char* q35_last_error(void) { return q35::last_error_cstr(); }
const char* q35_version(void) { return "q35-mi355x 0.1 (gfx950)"; }

void q35_dims_default(q35_dims* d) {
    if (d) q35::dims_from_config(ModelConfig{}, d);
}

q35_status q35_load_config(const char* path, q35_dims* d) {
    if (!path || !d) return q35::fail(Q35_ERR_ARG, "q35_load_config: null argument");
    ModelConfig c = q35::config_from_dims(*d);
    if (!load_model_config(path, c)) return q35::fail(Q35_ERR_IO, "cannot open %s", path);
    q35::dims_from_config(c, d);
    return Q35_OK;
}

int32_t q35_is_attention_layer(const q35_dims* d, int32_t layer) {
    return d && d->attn_interval > 0 && ((layer + 1) % d->attn_interval) == 0;
}

uint64_t q35_gdn_conv_state_bytes(const q35_dims* d) {
    return d ? gdn_conv_state_bytes(q35::config_from_dims(*d)) : 0;
}

q35_status q35_compute_budget(const q35_dims* d, int32_t bytes_per_weight, int64_t max_context,
                              int32_t kv_bytes_per_elem, int32_t max_vision_tiles,
                              int32_t vit_dim, q35_budget* out) {
    if (!d || !out) return q35::fail(Q35_ERR_ARG, "q35_compute_budget: null argument");
    if (max_context < 0 || max_context > INT32_MAX)
        return q35::fail(Q35_ERR_RANGE, "max_context %lld out of range", (long long)max_context);
    const MemoryBudget b = compute_budget(q35::config_from_dims(*d), bytes_per_weight,
                                          static_cast<int>(max_context), kv_bytes_per_elem,
                                          max_vision_tiles, vit_dim);
    out->weight_bytes = b.weight_bytes;
    out->gdn_state_bytes = b.gdn_state_bytes;
    out->gdn_conv_bytes = b.gdn_conv_bytes;
    out->kv_cache_bytes = b.kv_cache_bytes;
    out->activation_bytes = b.activation_bytes;
    out->vision_scratch_bytes = b.vision_scratch_bytes;
    out->prompt_arena_bytes = 0;  // no counterpart in the reference's equation
    return Q35_OK;
}

int64_t q35_solve_max_context(const q35_dims* d, uint64_t ram, uint64_t weight, uint64_t gdn,
                              uint64_t activation, uint64_t vision, uint64_t margin,
                              int32_t kv_bytes) {
    if (!d) return -1;
    return solve_max_context(q35::config_from_dims(*d), ram, weight, gdn, activation, vision,
                             margin, kv_bytes);
}

q35_status q35_synth_normal(float* dst, int64_t n, uint64_t seed, uint64_t stream, float std,
                            int32_t threads) {
    if (!dst || n < 0) return q35::fail(Q35_ERR_ARG, "q35_synth_normal: bad argument");
    const uint64_t key = q35synth::stream_key(seed, stream);
    parallel_for(n, threads, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; ++i)
            dst[i] = static_cast<float>(std * q35synth::normal_at(key, static_cast<uint64_t>(i)));
    });
    return Q35_OK;
}

q35_status q35_synth_token_ids(uint64_t seed, int32_t vocab, int32_t n, int32_t* ids) {
    if (!ids || vocab <= 0 || n < 0) return q35::fail(Q35_ERR_ARG, "q35_synth_token_ids: bad argument");
    const uint64_t key = q35synth::stream_key(seed, 0x70726f6d7074ULL /* "prompt" */);
    for (int32_t i = 0; i < n; ++i)
        ids[i] = static_cast<int32_t>((q35synth::mix64(key + static_cast<uint64_t>(i)) >> 11) %
                                      static_cast<uint64_t>(vocab));
    return Q35_OK;
}

q35_status q35_synth_write_model(const char* dir, const q35_dims* d, uint64_t seed, float std,
                                 int32_t threads) {
    if (!dir || !d) return q35::fail(Q35_ERR_ARG, "q35_synth_write_model: null argument");
    std::error_code ec;
    std::filesystem::create_directories(dir, ec);
    const std::vector<TensorSpec> specs = checkpoint_layout(*d);

    std::string header = "{";
    uint64_t off = 0;
    for (size_t i = 0; i < specs.size(); ++i) {
        const TensorSpec& s = specs[i];
        const uint64_t nb = static_cast<uint64_t>(s.numel()) * 2;
        header += (i ? "," : "");
        header += "\"" + s.name + "\":{\"dtype\":\"BF16\",\"shape\":[";
        for (size_t k = 0; k < s.shape.size(); ++k)
            header += (k ? "," : "") + std::to_string(s.shape[k]);
        header += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + nb) + "]}";
        off += nb;
    }
    header += ",\"__metadata__\":{\"format\":\"pt\"}}";
    while (header.size() % 8) header.push_back(' ');

    const std::string st_path = std::string(dir) + "/model.safetensors";
    const std::string tmp_path = st_path + ".tmp";
    FILE* f = std::fopen(tmp_path.c_str(), "wb");
    if (!f) return q35::fail(Q35_ERR_IO, "cannot write %s: %s", tmp_path.c_str(), std::strerror(errno));
    const uint64_t hl = header.size();
    bool ok = std::fwrite(&hl, 8, 1, f) == 1 && std::fwrite(header.data(), 1, hl, f) == hl;
    std::vector<uint16_t> buf;
    for (const TensorSpec& s : specs) {
        if (!ok) break;
        const int64_t n = s.numel();
        buf.resize(static_cast<size_t>(n));
        if (s.fill == 0) {
            const uint64_t key = q35synth::stream_key(seed, q35synth::name_stream(s.name.c_str()));
            uint16_t* p = buf.data();
            parallel_for(n, threads, [&](int64_t b, int64_t e) {
                for (int64_t i = b; i < e; ++i)
                    p[i] = q35synth::f32_to_bf16(static_cast<float>(
                        std * q35synth::normal_at(key, static_cast<uint64_t>(i))));
            });
        } else {
            std::fill(buf.begin(), buf.end(), static_cast<uint16_t>(s.fill == 2 ? 0x3f80 : 0));
        }
        ok = std::fwrite(buf.data(), 2, buf.size(), f) == buf.size();
    }
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) return q35::fail(Q35_ERR_IO, "write failed for %s", tmp_path.c_str());
    if (std::rename(tmp_path.c_str(), st_path.c_str()) != 0)
        return q35::fail(Q35_ERR_IO, "rename to %s failed", st_path.c_str());

    const std::string cfg_path = std::string(dir) + "/config.json";
    FILE* c = std::fopen(cfg_path.c_str(), "wb");
    if (!c) return q35::fail(Q35_ERR_IO, "cannot write %s", cfg_path.c_str());
    const std::string js = config_json(*d);
    ok = std::fwrite(js.data(), 1, js.size(), c) == js.size();
    ok = (std::fclose(c) == 0) && ok;
    return ok ? Q35_OK : q35::fail(Q35_ERR_IO, "write failed for %s", cfg_path.c_str());
}

}  // extern "C"
