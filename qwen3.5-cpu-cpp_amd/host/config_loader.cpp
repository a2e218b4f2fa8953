// config.json reader: the keys and derivations of the reference loader
// (src/config_loader.cpp:59-108), table-driven. A lookup is textual, as the reference's is:
// the value of a key is read after the first ':' that follows the first occurrence of the
// quoted key inside the "text_config" object (the whole file when that object is absent);
// a number is the run of [0-9+-.eE] after blanks (absent when out of range; integers round
// as (int)(v + 0.5)), a flag is true when "true" occurs before the next comma. Those rules
// decide what a malformed or unusual file yields, so they are kept; everything else here is
// this library's own.
#include <cctype>
#include <cerrno>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <iterator>
#include <optional>
#include <string>

#include "model_config.h"

namespace {

class ConfigScope {
public:
    // The scope of the lookups: the brace-matched object after "text_config", else `all`.
    explicit ConfigScope(const std::string& all) : text_(all) {
        const size_t key = all.find("\"text_config\"");
        const size_t open = key == std::string::npos ? key : all.find('{', key);
        if (open == std::string::npos) return;
        int depth = 0;
        for (size_t i = open; i < all.size(); ++i) {
            depth += all[i] == '{' ? 1 : all[i] == '}' ? -1 : 0;
            if (all[i] == '}' && depth == 0) {
                text_ = all.substr(open, i - open + 1);
                return;
            }
        }
    }

    std::optional<double> number(const std::string& key) const {
        size_t i = value_start(key);
        if (i == std::string::npos) return std::nullopt;
        while (i < text_.size() && std::string(" \t\n\r").find(text_[i]) != std::string::npos) ++i;
        size_t j = i;
        while (j < text_.size() && (std::isdigit(static_cast<unsigned char>(text_[j])) ||
                                    std::string("+-.eE").find(text_[j]) != std::string::npos))
            ++j;
        if (j == i) return std::nullopt;
        const std::string tok = text_.substr(i, j - i);
        char* end = nullptr;
        errno = 0;
        const double v = std::strtod(tok.c_str(), &end);
        if (end == tok.c_str() || errno == ERANGE) return std::nullopt;  // no number, or out of range
        return v;
    }

    std::optional<bool> flag(const std::string& key) const {
        const size_t i = value_start(key);
        if (i == std::string::npos) return std::nullopt;
        const size_t comma = text_.find(',', i);
        return text_.find("true", i) < (comma == std::string::npos ? text_.size() : comma);
    }

private:
    // just past the ':' after the first occurrence of "key", or npos
    size_t value_start(const std::string& key) const {
        const size_t at = text_.find('"' + key + '"');
        if (at == std::string::npos) return at;
        const size_t colon = text_.find(':', at);
        return colon == std::string::npos ? colon : colon + 1;
    }

    std::string text_;
};

struct IntKey {
    const char* key;
    int ModelConfig::*field;
};

// the integer keys, in the reference's order
constexpr IntKey kIntKeys[] = {
    {"hidden_size", &ModelConfig::hidden_size},
    {"num_hidden_layers", &ModelConfig::n_layers_total},
    {"full_attention_interval", &ModelConfig::attn_interval},
    {"num_attention_heads", &ModelConfig::attn_q_heads},
    {"num_key_value_heads", &ModelConfig::attn_kv_heads},
    {"head_dim", &ModelConfig::attn_head_dim},
    {"linear_num_key_heads", &ModelConfig::gdn_k_heads},
    {"linear_num_value_heads", &ModelConfig::gdn_v_heads},
    {"linear_key_head_dim", &ModelConfig::gdn_k_head_dim},
    {"linear_value_head_dim", &ModelConfig::gdn_v_head_dim},
    {"linear_conv_kernel_dim", &ModelConfig::gdn_conv_kernel},
    {"intermediate_size", &ModelConfig::ffn_intermediate},
    {"vocab_size", &ModelConfig::vocab_size},
    {"max_position_embeddings", &ModelConfig::native_max_context},
};

}  // namespace

bool load_model_config(const std::string& path, ModelConfig& cfg) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) {
        std::cerr << "[config] cannot open " << path << " - using built-in defaults\n";
        return false;
    }
    const ConfigScope scope(std::string((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>()));

    for (const IntKey& k : kIntKeys)
        if (const auto v = scope.number(k.key)) cfg.*k.field = static_cast<int>(*v + 0.5);
    if (const auto v = scope.number("rms_norm_eps")) cfg.rms_norm_eps = static_cast<float>(*v);
    if (const auto v = scope.number("rope_theta")) cfg.rope_theta = *v;
    if (const auto v = scope.number("partial_rotary_factor")) cfg.partial_rotary_factor = static_cast<float>(*v);
    if (const auto v = scope.flag("tie_word_embeddings")) cfg.tie_word_embeddings = *v;

    // derived: the GDN aliases, the layer split (every attn_interval-th layer is attention),
    // the rough parameter count the memory plan uses for weights
    cfg.gdn_n_heads = cfg.gdn_v_heads;
    cfg.gdn_head_dim = cfg.gdn_v_head_dim;
    cfg.n_layers_attn = cfg.n_layers_total / cfg.attn_interval;
    cfg.n_layers_gdn = cfg.n_layers_total - cfg.n_layers_attn;
    cfg.n_params = static_cast<int64_t>(cfg.vocab_size) * cfg.hidden_size +
                   static_cast<int64_t>(cfg.n_layers_total) * 12 * cfg.hidden_size * cfg.hidden_size;

    std::cerr << "[config] " << path << ": hidden=" << cfg.hidden_size << " layers=" << cfg.n_layers_total << " ("
              << cfg.n_layers_gdn << " gdn / " << cfg.n_layers_attn << " attn) ffn=" << cfg.ffn_intermediate
              << " vocab=" << cfg.vocab_size << " tie=" << cfg.tie_word_embeddings << "\n";
    return true;
}
