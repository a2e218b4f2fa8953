// The forward_pass.h primitives on host pointers (the reference's include/forward_pass.h:21-54,
// src/forward_pass.cpp:29-112), run by the library's gfx950 kernels through one device
// staging buffer. Host code only: the kernels are those of the C ABI (q35_l2norm,
// q35_matmul_f32 / q35_matmul_bf16 / q35_gemm_bf16, q35_rmsnorm, q35_rmsnorm_gated,
// q35_apply_rope).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../host/forward_pass.h"
#include "../host/q35_internal.h"
#include "launch.hpp"

namespace {

constexpr size_t kStageBytes = size_t{64} << 20;

struct Staging {
    std::mutex mu;
    hipStream_t s = nullptr;
    uint8_t* dev = nullptr;
};

Staging& staging() {
    static Staging st;
    return st;
}

[[noreturn]] void die(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void die(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::fprintf(stderr, "[q35] forward_pass: ");
    std::vfprintf(stderr, fmt, ap);
    std::fprintf(stderr, "\n");
    va_end(ap);
    std::abort();
}

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) die("%s: %s", what, hipGetErrorString(e));
}

void q35_ok(q35_status st, const char* what) {
    if (st != Q35_OK) die("%s: %s", what, q35_last_error());
}

size_t align256(size_t x) { return (x + 255) & ~size_t{255}; }

// One call's hold on the staging buffer (made, with its stream, at the first call).
class Lease {
public:
    Lease() : st_(staging()), lock_(st_.mu) {
        if (!st_.dev) {
            hip_ok(hipStreamCreateWithFlags(&st_.s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
            void* p = nullptr;
            hip_ok(hipMalloc(&p, kStageBytes), "hipMalloc of the staging buffer");
            q35::count_device_alloc();
            st_.dev = static_cast<uint8_t*>(p);
        }
    }
    template <class T = float>
    T* at(size_t byte_off) const { return reinterpret_cast<T*>(st_.dev + byte_off); }
    hipStream_t stream() const { return st_.s; }
    void up(void* d, const void* h, size_t bytes) const {
        hip_ok(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, st_.s), "copy to the device");
    }
    void down(void* h, const void* d, size_t bytes) const {
        hip_ok(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, st_.s), "copy to the host");
    }
    void sync() const { hip_ok(hipStreamSynchronize(st_.s), "hipStreamSynchronize"); }

private:
    Staging& st_;
    std::lock_guard<std::mutex> lock_;
};

// Rows per block of a matmul whose weight rows take row_bytes each, after the input (x_bytes)
// and with 4 bytes of output per row.
int rows_per_block(int out_dim, size_t row_bytes, size_t x_bytes, const char* who) {
    if (align256(x_bytes) + 512 >= kStageBytes)
        die("%s: an input of %zu bytes does not fit the %zu-byte staging buffer", who, x_bytes, kStageBytes);
    const size_t room = kStageBytes - align256(x_bytes) - 512;
    const size_t r = room / (row_bytes + 4);
    if (r == 0) die("%s: a row of %zu bytes does not fit the %zu-byte staging buffer", who, row_bytes, kStageBytes);
    return static_cast<int>(std::min<size_t>(r, static_cast<size_t>(out_dim)));
}

// fp32 weights: y = W x through q35_matmul_f32, in blocks of rows
void matmul_f32_rows(const float* W, const float* x, float* y, int out_dim, int in_dim) {
    const size_t xb = static_cast<size_t>(in_dim) * 4, rb = xb;
    const int blk = rows_per_block(out_dim, rb, xb, "matmul");
    Lease L;
    float* dx = L.at(0);
    L.up(dx, x, xb);
    for (int r0 = 0; r0 < out_dim; r0 += blk) {
        const int n = std::min(blk, out_dim - r0);
        float* dy = L.at(align256(xb));
        float* dw = L.at(align256(xb) + align256(static_cast<size_t>(n) * 4));
        L.up(dw, W + static_cast<size_t>(r0) * in_dim, static_cast<size_t>(n) * rb);
        q35_ok(q35_matmul_f32(dw, dx, dy, n, in_dim, L.stream()), "matmul");
        L.down(y + r0, dy, static_cast<size_t>(n) * 4);
        L.sync();  // the next block reuses the weight and output space
    }
}

}  // namespace

void l2norm(float* x, int n, float eps) {
    if (n <= 0) return;
    const size_t b = static_cast<size_t>(n) * 4;
    if (b > kStageBytes) die("l2norm of %d elements exceeds the staging buffer", n);
    Lease L;
    float* d = L.at(0);
    L.up(d, x, b);
    q35_ok(q35_l2norm(d, 1, n, eps, L.stream()), "l2norm");
    L.down(x, d, b);
    L.sync();
}

void matmul(const float* W, const float* x, float* y, int out_dim, int in_dim) {
    if (out_dim <= 0) return;
    if (in_dim <= 0) {  // empty dot products
        std::fill(y, y + out_dim, 0.0f);
        return;
    }
    matmul_f32_rows(W, x, y, out_dim, in_dim);
}

void matmul(const WeightView& W, const float* x, float* y, int out_dim, int in_dim) {
    if (!W.ok()) die("matmul: the weight view holds neither bf16 nor fp32 data");
    if (!W.bf16) return matmul(W.f32, x, y, out_dim, in_dim);
    if (out_dim <= 0) return;
    if (in_dim <= 0) {
        std::fill(y, y + out_dim, 0.0f);
        return;
    }
    if (in_dim % 8 != 0) {
        // rows the bf16 kernels cannot read 16 bytes at a time: widen them exactly (<< 16) on
        // the host and take the fp32 kernel, block by block
        const int blk = std::max(1, static_cast<int>((size_t{16} << 20) / (static_cast<size_t>(in_dim) * 4)));
        std::vector<float> wide;
        for (int r0 = 0; r0 < out_dim; r0 += blk) {
            const int n = std::min(blk, out_dim - r0);
            wide.resize(static_cast<size_t>(n) * in_dim);
            const uint16_t* src = W.bf16 + static_cast<size_t>(r0) * in_dim;
            for (size_t i = 0; i < wide.size(); ++i) {
                const uint32_t u = static_cast<uint32_t>(src[i]) << 16;
                std::memcpy(&wide[i], &u, 4);
            }
            matmul_f32_rows(wide.data(), x, y + r0, n, in_dim);
        }
        return;
    }
    const size_t xb = static_cast<size_t>(in_dim) * 4, rb = static_cast<size_t>(in_dim) * 2;
    const int blk = rows_per_block(out_dim, rb, xb, "matmul");
    Lease L;
    float* dx = L.at(0);
    L.up(dx, x, xb);
    for (int r0 = 0; r0 < out_dim; r0 += blk) {
        const int n = std::min(blk, out_dim - r0);
        float* dy = L.at(align256(xb));
        uint16_t* dw = L.at<uint16_t>(align256(xb) + align256(static_cast<size_t>(n) * 4));
        L.up(dw, W.bf16 + static_cast<size_t>(r0) * in_dim, static_cast<size_t>(n) * rb);
        if (in_dim <= q35k::kGemvMaxIn)
            q35_ok(q35_matmul_bf16(dw, dx, dy, n, in_dim, L.stream()), "matmul");
        else  // wider than the matvec stages: the token-batched GEMM with one row of x
            q35_ok(q35_gemm_bf16(dx, in_dim, dw, 1, n, in_dim, nullptr, n, dy, n, L.stream()), "matmul");
        L.down(y + r0, dy, static_cast<size_t>(n) * 4);
        L.sync();
    }
}

void rmsnorm(const float* x, const float* weight, float* y, int n, float eps) {
    if (n <= 0) return;
    const size_t b = align256(static_cast<size_t>(n) * 4);
    if (3 * b > kStageBytes) die("rmsnorm of %d elements exceeds the staging buffer", n);
    Lease L;
    float *dx = L.at(0), *dw = L.at(b), *dy = L.at(2 * b);
    L.up(dx, x, static_cast<size_t>(n) * 4);
    L.up(dw, weight, static_cast<size_t>(n) * 4);
    q35_ok(q35_rmsnorm(dx, dw, dy, 1, n, eps, L.stream()), "rmsnorm");
    L.down(y, dy, static_cast<size_t>(n) * 4);
    L.sync();
}

void rmsnorm_gated(const float* x, const float* weight, const float* gate, float* y, int n, float eps) {
    if (n <= 0) return;
    const size_t b = align256(static_cast<size_t>(n) * 4);
    if (4 * b > kStageBytes) die("rmsnorm_gated of %d elements exceeds the staging buffer", n);
    Lease L;
    float *dx = L.at(0), *dw = L.at(b), *dg = L.at(2 * b), *dy = L.at(3 * b);
    L.up(dx, x, static_cast<size_t>(n) * 4);
    L.up(dw, weight, static_cast<size_t>(n) * 4);
    L.up(dg, gate, static_cast<size_t>(n) * 4);
    q35_ok(q35_rmsnorm_gated(dx, dw, dg, dy, 1, n, eps, L.stream()), "rmsnorm_gated");
    L.down(y, dy, static_cast<size_t>(n) * 4);
    L.sync();
}

void apply_rope(float* vec, int rotary_dim, int pos, double theta) {
    if (rotary_dim < 2) return;  // no pair to rotate
    const size_t b = static_cast<size_t>(rotary_dim) * 4;
    if (b > kStageBytes) die("apply_rope of %d dims exceeds the staging buffer", rotary_dim);
    Lease L;
    float* d = L.at(0);
    L.up(d, vec, b);
    q35_ok(q35_apply_rope(d, 1, rotary_dim, rotary_dim, nullptr, pos, theta, L.stream()), "apply_rope");
    L.down(vec, d, b);
    L.sync();
}
