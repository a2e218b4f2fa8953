// Engine-side caller of the QwenForward drop-in (the reference's include/qwen_forward.h:18-25):
// loads a checkpoint with the reference's loader interface and runs prefill() on each prompt
// given, in order, with one QwenForward object.
//
//   qwen_forward_caller <model_dir> <logits.f32> <id,id,...> [<id,id,...> ...]
//
// The logits of every prompt are appended to <logits.f32> (raw fp32, row-major); one line per
// prompt reports its rows, the row width and the library's device allocation count after it.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "model_config.h"
#include "qwen_forward.h"
#include "safetensors_loader.h"

int main(int argc, char** argv) {
    if (argc < 4) {
        std::fprintf(stderr, "usage: %s <model_dir> <logits.f32> <id,id,...> [...]\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    ModelConfig cfg;
    load_model_config(dir + "/config.json", cfg);
    SafeTensors w;
    if (!w.load_model(dir)) return 1;
    QwenForward fwd(w, cfg);
    FILE* out = std::fopen(argv[2], "wb");
    if (!out) return 1;
    for (int a = 3; a < argc; ++a) {
        std::vector<int> ids;
        for (const char* p = argv[a]; *p;) {
            char* end = nullptr;
            ids.push_back(static_cast<int>(std::strtol(p, &end, 10)));
            p = *end == ',' ? end + 1 : end;
        }
        std::vector<float> logits;
        if (!fwd.prefill(ids, logits)) {
            std::fclose(out);
            return 1;
        }
        std::fwrite(logits.data(), sizeof(float), logits.size(), out);
        std::printf("prompt %d: %zu rows of %zu, device allocations %lld\n", a - 2, ids.size(),
                    logits.size() / ids.size(), static_cast<long long>(q35_device_alloc_count()));
    }
    std::fclose(out);
    return 0;
}
