// config.json reader. Same keys and derivations as the reference loader
// (src/config_loader.cpp:59-108): scalar values are looked up by their quoted key inside
// the "text_config" object (or the whole file when that object is absent).
#include <cctype>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <iterator>
#include <string>

#include "model_config.h"

namespace {

std::string object_after(const std::string& s, const std::string& key) {
    const size_t at = s.find('"' + key + '"');
    if (at == std::string::npos) return {};
    const size_t open = s.find('{', at);
    if (open == std::string::npos) return {};
    int depth = 0;
    for (size_t i = open; i < s.size(); ++i) {
        if (s[i] == '{') {
            ++depth;
        } else if (s[i] == '}') {
            if (--depth == 0) return s.substr(open, i - open + 1);
        }
    }
    return {};
}

bool number_after(const std::string& s, const std::string& key, double& out) {
    const size_t at = s.find('"' + key + '"');
    if (at == std::string::npos) return false;
    const size_t colon = s.find(':', at);
    if (colon == std::string::npos) return false;
    size_t i = colon + 1;
    while (i < s.size() && std::isspace(static_cast<unsigned char>(s[i]))) ++i;
    const size_t first = i;
    while (i < s.size()) {
        const char c = s[i];
        if (!(std::isdigit(static_cast<unsigned char>(c)) || c == '-' || c == '+' || c == '.' ||
              c == 'e' || c == 'E'))
            break;
        ++i;
    }
    if (i == first) return false;
    const std::string tok = s.substr(first, i - first);
    char* end = nullptr;
    out = std::strtod(tok.c_str(), &end);
    return end != tok.c_str();
}

bool bool_after(const std::string& s, const std::string& key, bool& out) {
    const size_t at = s.find('"' + key + '"');
    if (at == std::string::npos) return false;
    const size_t colon = s.find(':', at);
    if (colon == std::string::npos) return false;
    size_t comma = s.find(',', colon);
    if (comma == std::string::npos) comma = s.size();
    out = s.find("true", colon) < comma;
    return true;
}

int int_after(const std::string& s, const std::string& key, int fallback) {
    double v = 0.0;
    return number_after(s, key, v) ? static_cast<int>(v + 0.5) : fallback;
}

}  // namespace

bool load_model_config(const std::string& path, ModelConfig& cfg) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) {
        std::cerr << "[config] cannot open " << path << " - using built-in defaults\n";
        return false;
    }
    const std::string all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    std::string tc = object_after(all, "text_config");
    if (tc.empty()) tc = all;

    cfg.hidden_size = int_after(tc, "hidden_size", cfg.hidden_size);
    cfg.n_layers_total = int_after(tc, "num_hidden_layers", cfg.n_layers_total);
    cfg.attn_interval = int_after(tc, "full_attention_interval", cfg.attn_interval);
    cfg.attn_q_heads = int_after(tc, "num_attention_heads", cfg.attn_q_heads);
    cfg.attn_kv_heads = int_after(tc, "num_key_value_heads", cfg.attn_kv_heads);
    cfg.attn_head_dim = int_after(tc, "head_dim", cfg.attn_head_dim);
    cfg.gdn_k_heads = int_after(tc, "linear_num_key_heads", cfg.gdn_k_heads);
    cfg.gdn_v_heads = int_after(tc, "linear_num_value_heads", cfg.gdn_v_heads);
    cfg.gdn_k_head_dim = int_after(tc, "linear_key_head_dim", cfg.gdn_k_head_dim);
    cfg.gdn_v_head_dim = int_after(tc, "linear_value_head_dim", cfg.gdn_v_head_dim);
    cfg.gdn_conv_kernel = int_after(tc, "linear_conv_kernel_dim", cfg.gdn_conv_kernel);
    cfg.ffn_intermediate = int_after(tc, "intermediate_size", cfg.ffn_intermediate);
    cfg.vocab_size = int_after(tc, "vocab_size", cfg.vocab_size);
    cfg.native_max_context = int_after(tc, "max_position_embeddings", cfg.native_max_context);
    cfg.gdn_n_heads = cfg.gdn_v_heads;
    cfg.gdn_head_dim = cfg.gdn_v_head_dim;
    cfg.n_layers_attn = cfg.n_layers_total / cfg.attn_interval;
    cfg.n_layers_gdn = cfg.n_layers_total - cfg.n_layers_attn;

    double d = 0.0;
    if (number_after(tc, "rms_norm_eps", d)) cfg.rms_norm_eps = static_cast<float>(d);
    if (number_after(tc, "rope_theta", d)) cfg.rope_theta = d;
    if (number_after(tc, "partial_rotary_factor", d)) cfg.partial_rotary_factor = static_cast<float>(d);
    bool b = false;
    if (bool_after(tc, "tie_word_embeddings", b)) cfg.tie_word_embeddings = b;

    cfg.n_params = static_cast<int64_t>(cfg.vocab_size) * cfg.hidden_size +
                   static_cast<int64_t>(cfg.n_layers_total) * 12 * cfg.hidden_size * cfg.hidden_size;

    std::cerr << "[config] " << path << ": hidden=" << cfg.hidden_size
              << " layers=" << cfg.n_layers_total << " (" << cfg.n_layers_gdn << " gdn / "
              << cfg.n_layers_attn << " attn) ffn=" << cfg.ffn_intermediate
              << " vocab=" << cfg.vocab_size << " tie=" << cfg.tie_word_embeddings << "\n";
    return true;
}
