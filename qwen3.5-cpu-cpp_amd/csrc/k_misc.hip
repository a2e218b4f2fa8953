// Small kernels of the decode step and of the primitive entry points: row-wise norms and
// RoPE (src/forward_pass.cpp:77-112), embedding gather
// (SafeTensors::get_row_f32, src/safetensors_loader.cpp:280-298), greedy argmax
// (src/qwen_model.cpp:249-250: first index of the maximum), counters and fills.
#include <math.h>

#include <climits>

#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

// One block per row: y = x * rsqrt(mean(x^2) + eps) * (1 + w), or for the gated form
// y = w * (x * rsqrt(mean(x^2) + eps)) * silu(gate).
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* x, const float* w,
                                                           float* y, int n, float eps,
                                                           int gated, const float* gate, float* ymax,
                                                           int y_tiled) {
    __shared__ double red[4];
    __shared__ float mred[4];
    const int64_t off = static_cast<int64_t>(blockIdx.x) * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const double v = x[off + i];
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(static_cast<float>(ss / n) + eps);
    float mx = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = x[off + i];
        const float o = gated ? w[i] * (v * inv) * silu_f(gate[off + i]) : v * inv * (1.0f + w[i]);
        y[y_tiled ? xt_off(blockIdx.x, i, n) : off + i] = o;
        mx = fmaxf(mx, fabsf(o));
    }
    if (ymax) {  // uniform
        mx = wave_max(mx);
        if ((threadIdx.x & 63) == 0) mred[threadIdx.x >> 6] = mx;
        __syncthreads();
        if (threadIdx.x == 0) ymax[blockIdx.x] = fmaxf(fmaxf(mred[0], mred[1]), fmaxf(mred[2], mred[3]));
    }
}

// The same for rows of n = 256 NV4 floats, one row per wave: the row stays in registers
// between the sum of squares (double, reduced across the wave) and the scaling, so it is
// read once, and no block barrier is needed. y_tiled == 2: the scaled row also stays in
// registers until its maximum is known, then goes out split for the two-part GEMM (scale
// 2^split_row_exp(max), fp16 high and low parts in the layout of xp_off) -- the split the
// GEMM would otherwise redo for every 128-column tile of its output.
template <int NV4>
__global__ __launch_bounds__(256) void rmsnorm_rows_wave_kernel(const float* x, const float* w, float* y,
                                                                int rows, float eps, int gated,
                                                                const float* gate, float* ymax, int y_tiled) {
    constexpr int n = NV4 * 256;
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole waves
    const int64_t off = static_cast<int64_t>(row) * n;
    float4 v[NV4];
#pragma unroll
    for (int i = 0; i < NV4; ++i) v[i] = *reinterpret_cast<const float4*>(x + off + (64 * i + lane) * 4);
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < NV4; ++i)
        ss += static_cast<double>(v[i].x) * v[i].x + static_cast<double>(v[i].y) * v[i].y +
              static_cast<double>(v[i].z) * v[i].z + static_cast<double>(v[i].w) * v[i].w;
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(static_cast<float>(ss / n) + eps);
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < NV4; ++i) {
        const int c = (64 * i + lane) * 4;
        const float4 w4 = *reinterpret_cast<const float4*>(w + c);
        float4 o;
        if (gated) {
            const float4 g4 = *reinterpret_cast<const float4*>(gate + off + c);
            o = make_float4(w4.x * (v[i].x * inv) * silu_f(g4.x), w4.y * (v[i].y * inv) * silu_f(g4.y),
                            w4.z * (v[i].z * inv) * silu_f(g4.z), w4.w * (v[i].w * inv) * silu_f(g4.w));
        } else {
            o = make_float4(v[i].x * inv * (1.0f + w4.x), v[i].y * inv * (1.0f + w4.y), v[i].z * inv * (1.0f + w4.z),
                            v[i].w * inv * (1.0f + w4.w));
        }
        if (y_tiled != 2) *reinterpret_cast<float4*>(y + (y_tiled ? xt_off(row, c, n) : off + c)) = o;
        v[i] = o;
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
    }
    if (ymax || y_tiled == 2) mx = wave_max(mx);  // uniform
    if (y_tiled == 2) {
        const float sc = ldexpf(1.0f, split_row_exp(mx));
        uint16_t* yh = reinterpret_cast<uint16_t*>(y);
        const bool odd = lane & 1;
#pragma unroll
        for (int i = 0; i < NV4; ++i) {
            // 4 consecutive k: lanes 2m and 2m + 1 hold one 8-k group, which the even lane
            // stores as its 16 bytes of high parts and the odd lane as its 16 bytes of low
            // parts, after trading the halves they do not store
            const int c = (64 * i + lane) * 4;
            uint32_t h0, l0, h1, l1;
            split2h_pair(v[i].x * sc, v[i].y * sc, h0, l0);
            split2h_pair(v[i].z * sc, v[i].w * sc, h1, l1);
            const uint32_t r0 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(odd ? h0 : l0), 1));
            const uint32_t r1 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(odd ? h1 : l1), 1));
            const uint4 q = odd ? make_uint4(r0, r1, l0, l1) : make_uint4(h0, h1, r0, r1);
            *reinterpret_cast<uint4*>(yh + xp_off(row, c & ~7, n, odd ? 1 : 0)) = q;
        }
    }
    if (ymax && lane == 0) ymax[row] = mx;
}

// x *= 1 / sqrt(sum(x^2) + eps), in place, one block per row.
__global__ __launch_bounds__(256) void l2norm_rows_kernel(float* x, int n, float eps) {
    __shared__ double red[4];
    const int64_t off = static_cast<int64_t>(blockIdx.x) * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) {
        const double v = x[off + i];
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(static_cast<float>(ss) + eps);
    for (int i = threadIdx.x; i < n; i += 256) x[off + i] *= inv;
}

// Rotate-half on dims [0, rot) of each row; angle pos * theta^(-2i/rot) in double.
__global__ __launch_bounds__(64) void rope_rows_kernel(float* x, int hd, int rot, const int* pos,
                                                       int pos0, double theta) {
    const int half = rot / 2;
    const int p = pos ? pos[blockIdx.x] : pos0;
    float* v = x + static_cast<int64_t>(blockIdx.x) * hd;
    for (int i = threadIdx.x; i < half; i += 64) {
        const double inv_freq = pow(theta, -static_cast<double>(2 * i) / rot);
        const double ang = static_cast<double>(p) * inv_freq;
        const float c = static_cast<float>(cos(ang)), s = static_cast<float>(sin(ang));
        const float x1 = v[i], x2 = v[i + half];
        v[i] = x1 * c - x2 * s;
        v[i + half] = x2 * c + x1 * s;
    }
}

// y = W x with fp32 weights, W row-major [rows][n] (the fp32 overload of the reference's
// matmul, src/forward_pass.cpp:29-33), any n: one row per wave, lanes striding the row
// (coalesced), four independent partial sums per lane, then a wave reduction.
__global__ __launch_bounds__(256) void matvec_f32_kernel(const float* W, const float* x, float* y, int rows, int n) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* w = W + static_cast<int64_t>(row) * n;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int i = lane;
    for (; i + 192 < n; i += 256) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] = fmaf(w[i + 64 * u], x[i + 64 * u], acc[u]);
    }
    for (; i < n; i += 64) acc[0] = fmaf(w[i], x[i], acc[0]);
    const float t = wave_sum((acc[0] + acc[1]) + (acc[2] + acc[3]));
    if (lane == 0) y[row] = t;
}

__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* embed, const int* token,
                                                    float* hidden, int H) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < H) hidden[i] = bf16_to_f32(embed[static_cast<int64_t>(*token) * H + i]);
}

// (value, index) order for the argmax: larger value first, then smaller index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void block_best(float& bv, int& bi) {
    __shared__ float sv[4];
    __shared__ int si[4];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int w = 1; w < 4; ++w)
        if (better(sv[w], si[w], bv, bi)) {
            bv = sv[w];
            bi = si[w];
        }
}

__global__ __launch_bounds__(256) void argmax_pass1(const float* logits, int n, float* pv, int* pi) {
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += 256 * kArgmaxBlocks) {
        const float v = logits[i];
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(256) void argmax_pass2(const float* pv, const int* pi, int n_parts, int* token_out,
                                                    int* ids, int* pos) {
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int b = threadIdx.x; b < n_parts; b += 256)
        if (better(pv[b], pi[b], bv, bi)) {
            bv = pv[b];
            bi = pi[b];
        }
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        const int am = bi == INT_MAX ? 0 : bi;
        *token_out = am;
        if (pos) {
            if (ids) ids[*pos] = am;
            *pos += 1;
        }
    }
}

__global__ void add_int_kernel(int* p, int v) { *p += v; }
__global__ void set_int_kernel(int* p, int v) { *p = v; }

__global__ __launch_bounds__(256) void copy_kernel(float* dst, const float* src, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        dst[i] = src[i];
}

__global__ __launch_bounds__(256) void fill_kernel(float* dst, int64_t n, float v) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        dst[i] = v;
}

__global__ __launch_bounds__(256) void fill_normal_kernel(float* dst, int64_t n, uint64_t key, float std) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        dst[i] = static_cast<float>(std * normal_at(key, static_cast<uint64_t>(i)));
}

__global__ __launch_bounds__(256) void fill_normal_bf16_kernel(uint16_t* dst, int64_t n, uint64_t key, float std) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        dst[i] = f32_to_bf16(static_cast<float>(std * normal_at(key, static_cast<uint64_t>(i))));
}

__global__ __launch_bounds__(256) void rope_table_kernel(float* t, int64_t n_pos, int rot, double theta) {
    const int half = rot / 2;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n_pos * half;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t p = i / half;
        const int k = static_cast<int>(i - p * half);
        const double inv_freq = pow(theta, -static_cast<double>(2 * k) / rot);
        const double ang = static_cast<double>(p) * inv_freq;
        t[p * rot + k] = static_cast<float>(cos(ang));
        t[p * rot + half + k] = static_cast<float>(sin(ang));
    }
}

int grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return static_cast<int>(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace

hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* y, int rows, int n,
                               float eps, int gated, const float* gate, hipStream_t s, float* ymax, int y_tiled) {
    if (y_tiled && n % 32 != 0) return hipErrorInvalidValue;
    // the split form comes from the one-row-per-wave kernels only
    if (y_tiled == 2 && (!ymax || !rmsnorm_rows_splits(n) || ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                                                               reinterpret_cast<uintptr_t>(y)) & 15) != 0 || gated))
        return hipErrorInvalidValue;
    const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                         reinterpret_cast<uintptr_t>(y) | (gated ? reinterpret_cast<uintptr_t>(gate) : 0);
    const int wb = (rows + 3) / 4;
    if ((al & 15) == 0 && n == 1024)
        klaunch(rmsnorm_rows_wave_kernel<4>, wb, 256, 0, s, x, w, y, rows, eps, gated, gate, ymax, y_tiled);
    else if ((al & 15) == 0 && n == 2048)
        klaunch(rmsnorm_rows_wave_kernel<8>, wb, 256, 0, s, x, w, y, rows, eps, gated, gate, ymax, y_tiled);
    else if ((al & 15) == 0 && n == 4096)
        klaunch(rmsnorm_rows_wave_kernel<16>, wb, 256, 0, s, x, w, y, rows, eps, gated, gate, ymax, y_tiled);
    else klaunch(rmsnorm_rows_kernel, rows, 256, 0, s, x, w, y, n, eps, gated, gate, ymax, y_tiled);
    return hipGetLastError();
}

namespace {
// max |w| of n bf16 values as the bits of the largest |bf16| (|bf16| bits compare as unsigned
// in magnitude order for finite values); VEC: 16-byte loads (w 16-byte aligned, n % 8 == 0)
template <bool VEC>
__global__ __launch_bounds__(256) void bf16_absmax_kernel(const uint16_t* w, int64_t n, unsigned* out) {
    unsigned m = 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    if constexpr (VEC) {
        const uint4* w8 = reinterpret_cast<const uint4*>(w);
        auto m2 = [](unsigned x) { return max(x & 0x7fffu, (x >> 16) & 0x7fffu); };
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n / 8; i += stride) {
            const uint4 v = w8[i];
            m = max(m, max(max(m2(v.x), m2(v.y)), max(m2(v.z), m2(v.w))));
        }
    } else {
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
            m = max(m, static_cast<unsigned>(w[i] & 0x7fffu));
    }
    __shared__ unsigned red[4];
    for (int o = 32; o > 0; o >>= 1) m = max(m, static_cast<unsigned>(__shfl_xor(static_cast<int>(m), o)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) atomicMax(out, max(max(red[0], red[1]), max(red[2], red[3])));
}

// wh = fp16(w * scale); VEC: eight values per thread with 16-byte loads and stores
template <bool VEC>
__global__ __launch_bounds__(256) void bf16_to_f16_kernel(const uint16_t* w, uint16_t* wh, int64_t n, float scale) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    if constexpr (VEC) {
        auto cv = [&](unsigned x) {
            const _Float16 lo = static_cast<_Float16>(__uint_as_float(x << 16) * scale);
            const _Float16 hi = static_cast<_Float16>(__uint_as_float(x & 0xffff0000u) * scale);
            return static_cast<unsigned>(__builtin_bit_cast(uint16_t, lo)) |
                   (static_cast<unsigned>(__builtin_bit_cast(uint16_t, hi)) << 16);
        };
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n / 8; i += stride) {
            const uint4 v = reinterpret_cast<const uint4*>(w)[i];
            reinterpret_cast<uint4*>(wh)[i] = make_uint4(cv(v.x), cv(v.y), cv(v.z), cv(v.w));
        }
    } else {
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
            const _Float16 h = static_cast<_Float16>(bf16_to_f32(w[i]) * scale);
            wh[i] = __builtin_bit_cast(uint16_t, h);
        }
    }
}

// Row-major X [M][ldx] -> the tiled layout of the two-part GEMM (rows padded to a multiple
// of 128 with zeros), and each row's max |x|. One workgroup per (padded) row.
__global__ __launch_bounds__(256) void rows_to_tiled_kernel(const float* X, int64_t ldx, int M, int K, float* Xt,
                                                            float* xmax) {
    const int row = blockIdx.x, tid = threadIdx.x;
    float m = 0.0f;
    for (int k = tid; k < K; k += 256) {
        const float v = row < M ? X[static_cast<int64_t>(row) * ldx + k] : 0.0f;
        Xt[xt_off(row, k, K)] = v;
        m = fmaxf(m, fabsf(v));
    }
    __shared__ float red[4];
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    if (tid == 0 && row < M) xmax[row] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
}  // namespace

hipError_t launch_rows_to_tiled(const float* X, int64_t ldx, int M, int K, float* Xt, float* xmax, hipStream_t s) {
    klaunch(rows_to_tiled_kernel, static_cast<int>(rows_tiled(M)), 256, 0, s, X, ldx, M, K, Xt, xmax);
    return hipGetLastError();
}

hipError_t launch_bf16_absmax(const uint16_t* w, int64_t n, unsigned* out, hipStream_t s) {
    // at most 1024 workgroups: each ends with one atomic on the same word
    if ((reinterpret_cast<uintptr_t>(w) & 15) == 0 && n % 8 == 0)
        klaunch(bf16_absmax_kernel<true>, std::min(grid_for(n / 8), 1024), 256, 0, s, w, n, out);
    else klaunch(bf16_absmax_kernel<false>, std::min(grid_for(n), 1024), 256, 0, s, w, n, out);
    return hipGetLastError();
}

hipError_t launch_bf16_to_f16(const uint16_t* w, uint16_t* wh, int64_t n, int e, hipStream_t s) {
    if (((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(wh)) & 15) == 0 && n % 8 == 0)
        klaunch(bf16_to_f16_kernel<true>, grid_for(n / 8), 256, 0, s, w, wh, n, ldexpf(1.0f, e));
    else klaunch(bf16_to_f16_kernel<false>, grid_for(n), 256, 0, s, w, wh, n, ldexpf(1.0f, e));
    return hipGetLastError();
}

hipError_t launch_l2norm_rows(float* x, int rows, int n, float eps, hipStream_t s) {
    klaunch(l2norm_rows_kernel, rows, 256, 0, s, x, n, eps);
    return hipGetLastError();
}

hipError_t launch_rope_rows(float* x, int rows, int hd, int rot, const int* pos, int pos0,
                            double theta, hipStream_t s) {
    klaunch(rope_rows_kernel, rows, 64, 0, s, x, hd, rot, pos, pos0, theta);
    return hipGetLastError();
}

hipError_t launch_matvec_f32(const float* W, const float* x, float* y, int rows, int n, hipStream_t s) {
    klaunch(matvec_f32_kernel, (rows + 3) / 4, 256, 0, s, W, x, y, rows, n);
    return hipGetLastError();
}

hipError_t launch_embed(const uint16_t* embed, const int* token_dev, float* hidden, int H,
                        hipStream_t s) {
    klaunch(embed_kernel, (H + 255) / 256, 256, 0, s, embed, token_dev, hidden, H);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int n, void* part, int* token_out, int* ids,
                         int* pos, hipStream_t s) {
    float* pv = static_cast<float*>(part);
    int* pi = reinterpret_cast<int*>(pv + kArgmaxBlocks);
    klaunch(argmax_pass1, kArgmaxBlocks, 256, 0, s, logits, n, pv, pi);
    klaunch(argmax_pass2, 1, 256, 0, s, pv, pi, kArgmaxBlocks, token_out, ids, pos);
    return hipGetLastError();
}

hipError_t launch_argmax_parts(const void* part, int n_parts, int* token_out, int* ids, int* pos,
                               hipStream_t s) {
    const float* pv = static_cast<const float*>(part);
    klaunch(argmax_pass2, 1, 256, 0, s, pv, reinterpret_cast<const int*>(pv + n_parts), n_parts, token_out, ids, pos);
    return hipGetLastError();
}

hipError_t launch_add_int(int* p, int v, hipStream_t s) {
    klaunch(add_int_kernel, 1, 1, 0, s, p, v);
    return hipGetLastError();
}

hipError_t launch_set_int(int* p, int v, hipStream_t s) {
    klaunch(set_int_kernel, 1, 1, 0, s, p, v);
    return hipGetLastError();
}

hipError_t launch_copy_f32(float* dst, const float* src, int64_t n, hipStream_t s) {
    klaunch(copy_kernel, grid_for(n), 256, 0, s, dst, src, n);
    return hipGetLastError();
}

hipError_t launch_fill_f32(float* dst, int64_t n, float v, hipStream_t s) {
    klaunch(fill_kernel, grid_for(n), 256, 0, s, dst, n, v);
    return hipGetLastError();
}

hipError_t launch_fill_normal(float* dst, int64_t n, uint64_t key, float std, hipStream_t s, bool bf16) {
    if (bf16) klaunch(fill_normal_bf16_kernel, grid_for(n), 256, 0, s, reinterpret_cast<uint16_t*>(dst), n, key, std);
    else klaunch(fill_normal_kernel, grid_for(n), 256, 0, s, dst, n, key, std);
    return hipGetLastError();
}

LaunchTimer*& launch_timer() {
    static thread_local LaunchTimer* t = nullptr;
    return t;
}

hipError_t launch_rope_table(float* t, int64_t n_pos, int rot, double theta, hipStream_t s) {
    if (rot <= 0) return hipSuccess;
    klaunch(rope_table_kernel, grid_for(n_pos * (rot / 2)), 256, 0, s, t, n_pos, rot, theta);
    return hipGetLastError();
}

}  // namespace q35k
