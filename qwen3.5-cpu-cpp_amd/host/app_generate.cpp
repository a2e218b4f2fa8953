// q35_generate: the reference CLI's flow (src/main.cpp:15-47) on the GPU engine, with
// token ids in and token ids out (text I/O is outside this library):
//
//   q35_generate <model_dir> <n_new> <id,id,...>       greedy continuation of a prompt
//   q35_generate <model_dir> <n_new> --synthetic N S   prompt of N ids drawn with seed S
//
// Prints the generated ids, comma separated, on stdout.
#include <cstdlib>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/q35.h"
#include "model_config.h"
#include "qwen_model.h"
#include "safetensors_loader.h"

int main(int argc, char** argv) {
    if (argc < 4) {
        std::cerr << "usage: q35_generate <model_dir> <n_new> <id,id,...> | --synthetic N SEED\n";
        return 2;
    }
    const std::string dir = argv[1];
    const int n_new = std::atoi(argv[2]);
    ModelConfig cfg;
    load_model_config(dir + "/config.json", cfg);
    SafeTensors weights;
    if (!weights.load_model(dir)) {
        std::cerr << "Could not load weights from '" << dir << "'.\n";
        return 1;
    }
    std::vector<int> prompt;
    if (std::string(argv[3]) == "--synthetic" && argc >= 6) {
        const int n = std::atoi(argv[4]);
        std::vector<int32_t> ids(static_cast<size_t>(n));
        q35_synth_token_ids(std::strtoull(argv[5], nullptr, 10), cfg.vocab_size, n, ids.data());
        prompt.assign(ids.begin(), ids.end());
    } else {
        std::stringstream ss(argv[3]);
        std::string tok;
        while (std::getline(ss, tok, ',')) prompt.push_back(std::atoi(tok.c_str()));
    }
    QwenModel model(weights, cfg, static_cast<int>(prompt.size()) + n_new + 2);
    if (!model.ok()) return 1;
    const std::vector<int> gen = model.generate_greedy(prompt, n_new);
    if (static_cast<int>(gen.size()) != n_new) return 1;
    for (size_t i = 0; i < gen.size(); ++i) std::cout << (i ? "," : "") << gen[i];
    std::cout << "\n";
    return 0;
}
