// Engine-side caller of the forward_pass.h drop-in: written against the reference's
// interface (include/forward_pass.h:21-54) only, compiled with the plain host compiler and
// linked against libq35.so. Each function is called on seeded inputs and compared with the
// oracle's restatement of the same function (liboracle, test infrastructure).
//
//   forward_pass_caller --host-only   the inline activations (no device needed)
//   forward_pass_caller               every function (needs the GPU)
//
// One line per check; the exit status is 0 when every check is within its bar.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "forward_pass.h"
extern "C" {
#include "oracle.h"
}

namespace {

int g_failed = 0;

double rel_l2(const std::vector<float>& a, const std::vector<float>& b) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < a.size(); ++i) {
        const double d = static_cast<double>(a[i]) - b[i];
        num += d * d;
        den += static_cast<double>(b[i]) * b[i];
    }
    return den > 0 ? std::sqrt(num / den) : std::sqrt(num);
}

void report(const std::string& name, double err, double bar) {
    const bool ok = err <= bar;
    if (!ok) ++g_failed;
    std::printf("%-44s rel_l2 %.3g (bar %.0e) %s\n", name.c_str(), err, bar, ok ? "ok" : "FAIL");
}

std::vector<float> normal(std::mt19937_64& g, size_t n, float std = 1.0f) {
    std::normal_distribution<float> d(0.0f, std);
    std::vector<float> v(n);
    for (float& x : v) x = d(g);
    return v;
}

// bf16 patterns of normal values (round to nearest even)
std::vector<uint16_t> normal_bf16(std::mt19937_64& g, size_t n, float std) {
    std::vector<float> f = normal(g, n, std);
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        std::memcpy(&u, &f[i], 4);
        u += 0x7fffu + ((u >> 16) & 1u);
        h[i] = static_cast<uint16_t>(u >> 16);
    }
    return h;
}

void check_activations() {
    int bad = 0;
    for (int i = -4000; i <= 4000; ++i) {
        const float x = 0.0125f * static_cast<float>(i);  // -50 .. 50, through the > 20 branch
        if (silu(x) != orc_silu(x) || sigmoidf(x) != orc_sigmoid(x) || softplusf(x) != orc_softplus(x)) ++bad;
    }
    std::printf("%-44s %d of 8001 differ %s\n", "silu / sigmoidf / softplusf", bad, bad ? "FAIL" : "ok");
    if (bad) ++g_failed;
}

void check_norms(std::mt19937_64& g) {
    for (int n : {128, 1000, 2048, 4099}) {
        std::vector<float> x = normal(g, n, 3.0f), ref = x;
        l2norm(x.data(), n, 1e-6f);
        orc_l2norm(ref.data(), n, 1e-6f);
        report("l2norm n=" + std::to_string(n), rel_l2(x, ref), 1e-6);
    }
    for (int n : {256, 1000, 2048}) {
        std::vector<float> x = normal(g, n), w = normal(g, n, 0.1f), y(n), ref(n);
        rmsnorm(x.data(), w.data(), y.data(), n, 1e-6f);
        orc_rmsnorm(x.data(), w.data(), ref.data(), n, 1e-6f);
        report("rmsnorm n=" + std::to_string(n), rel_l2(y, ref), 1e-6);
        std::vector<float> z = normal(g, n);
        rmsnorm_gated(x.data(), w.data(), z.data(), y.data(), n, 1e-6f);
        orc_rmsnorm_gated(x.data(), w.data(), z.data(), ref.data(), n, 1e-6f);
        report("rmsnorm_gated n=" + std::to_string(n), rel_l2(y, ref), 1e-6);
    }
}

void check_rope(std::mt19937_64& g) {
    const int cases[][2] = {{64, 0}, {64, 12345}, {64, 131071}, {18, 777}, {7, 4096}, {256, 99}, {1, 5}};
    for (const auto& c : cases) {
        const int rot = c[0], pos = c[1];
        const std::vector<float> orig = normal(g, 256);
        std::vector<float> v = orig, ref = orig;
        apply_rope(v.data(), rot, pos, 1e7);
        orc_apply_rope(ref.data(), rot, pos, 1e7);
        report("apply_rope rot=" + std::to_string(rot) + " pos=" + std::to_string(pos), rel_l2(v, ref), 1e-6);
        // dims from the rotary width on are untouched (and the last one of an odd width)
        bool same = true;
        for (int i = 2 * (rot / 2); i < 256; ++i) same = same && v[i] == orig[i];
        if (!same) {
            ++g_failed;
            std::printf("apply_rope rot=%d: dims past the rotary width changed FAIL\n", rot);
        }
    }
}

void check_matmul(std::mt19937_64& g) {
    // (out, in): the matvec, blocks of rows through the staging buffer (> 64 MiB of
    // weights), rows wider than the matvec stages (the GEMM path), rows not a multiple of 8
    const int bf16_cases[][2] = {{257, 2048}, {9000, 4096}, {40, 20000}, {33, 1001}};
    for (const auto& c : bf16_cases) {
        const int out = c[0], in = c[1];
        std::vector<uint16_t> W = normal_bf16(g, static_cast<size_t>(out) * in, 0.02f);
        std::vector<float> x = normal(g, in), y(out), ref(out);
        WeightView v;
        v.bf16 = W.data();
        v.numel = static_cast<int64_t>(W.size());
        matmul(v, x.data(), y.data(), out, in);
        orc_matmul_bf16(W.data(), x.data(), ref.data(), out, in);
        report("matmul(WeightView bf16) " + std::to_string(out) + "x" + std::to_string(in), rel_l2(y, ref), 2e-6);
    }
    const int f32_cases[][2] = {{300, 1000}, {5000, 4096}, {17, 3}};
    for (const auto& c : f32_cases) {
        const int out = c[0], in = c[1];
        std::vector<float> W = normal(g, static_cast<size_t>(out) * in, 0.02f), x = normal(g, in), y(out), ref(out);
        matmul(W.data(), x.data(), y.data(), out, in);
        orc_matmul_f32(W.data(), x.data(), ref.data(), out, in);
        report("matmul(float*) " + std::to_string(out) + "x" + std::to_string(in), rel_l2(y, ref), 2e-6);
        WeightView v;
        v.f32 = W.data();
        v.numel = static_cast<int64_t>(W.size());
        std::fill(y.begin(), y.end(), 0.0f);
        matmul(v, x.data(), y.data(), out, in);
        report("matmul(WeightView f32) " + std::to_string(out) + "x" + std::to_string(in), rel_l2(y, ref), 2e-6);
    }
}

}  // namespace

int main(int argc, char** argv) {
    const bool host_only = argc > 1 && std::strcmp(argv[1], "--host-only") == 0;
    std::mt19937_64 g(20261202);
    check_activations();
    if (!host_only) {
        check_norms(g);
        check_rope(g);
        check_matmul(g);
    }
    std::printf("%s: %d check(s) failed\n", host_only ? "host-only" : "all", g_failed);
    return g_failed ? 1 : 0;
}
