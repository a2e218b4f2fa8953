// bf16-weight x fp32-activation matvec for every projection of the decode step
// (the reference's matmul(WeightView), src/forward_pass.cpp:44-75), with the elementwise
// work that feeds or follows each projection fused in:
//   prologue  rmsnorm (1+w)       input_layernorm / post_attention_layernorm / final norm
//             silu(g) * u         SwiGLU before mlp.down_proj
//             gated rmsnorm        GDN rmsnorm_gated before linear_attn.out_proj
//   epilogue  y = resid + W x     residual add of the mixer / FFN output
//
// HBM-bound: every weight byte is read exactly once per step. A 256-thread workgroup
// stages the transformed input vector in LDS once, then each 64-lane wave streams RPW
// weight rows at a time with 16-byte loads (8 bf16 per lane, 1 KiB per wave per row and
// chunk), issuing up to 4 chunks of loads before consuming them. bf16 is widened exactly
// (shift into the upper half of an fp32) and accumulated in fp32 FMA; the 64 lane partials
// are summed with a butterfly.
#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 load_w(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ float dot8(const u32x4 w, const float4 x0, const float4 x1, float acc) {
    acc = fmaf(bf16_lo(w.x), x0.x, acc);
    acc = fmaf(bf16_hi(w.x), x0.y, acc);
    acc = fmaf(bf16_lo(w.y), x0.z, acc);
    acc = fmaf(bf16_hi(w.y), x0.w, acc);
    acc = fmaf(bf16_lo(w.z), x1.x, acc);
    acc = fmaf(bf16_hi(w.z), x1.y, acc);
    acc = fmaf(bf16_lo(w.w), x1.z, acc);
    acc = fmaf(bf16_hi(w.w), x1.w, acc);
    return acc;
}

template <int PRO>
__device__ __forceinline__ void stage_input(const GemvArgs& a, float* xs) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = a.in_dim;
    __shared__ double red[4];
    __shared__ float head_inv[64];
    if (PRO == kProSwiGlu) {
        for (int i = tid * 4; i < n; i += 1024) {
            const float4 g = *reinterpret_cast<const float4*>(a.x + i);
            const float4 u = *reinterpret_cast<const float4*>(a.x + n + i);
            float4 h;
            h.x = silu_f(g.x) * u.x;
            h.y = silu_f(g.y) * u.y;
            h.z = silu_f(g.z) * u.z;
            h.w = silu_f(g.w) * u.w;
            *reinterpret_cast<float4*>(xs + i) = h;
        }
    } else {
        for (int i = tid * 4; i < n; i += 1024)
            *reinterpret_cast<float4*>(xs + i) = *reinterpret_cast<const float4*>(a.x + i);
    }
    if (PRO == kProRmsNorm) {
        double ss = 0.0;
        for (int i = tid; i < n; i += 256) {
            const double v = a.x[i];
            ss += v * v;
        }
        ss = block_sum(ss, red);
        const float inv = 1.0f / sqrtf(static_cast<float>(ss / n) + a.eps);
        __syncthreads();
        for (int i = tid; i < n; i += 256) xs[i] = xs[i] * inv * (1.0f + a.norm_w[i]);
    }
    if (PRO == kProGatedNorm) {
        const int hd = a.head_dim, nh = n / hd;
        for (int h = wave; h < nh; h += 4) {
            double ss = 0.0;
            for (int i = lane; i < hd; i += 64) {
                const double v = a.x[h * hd + i];
                ss += v * v;
            }
            ss = wave_sum(ss);
            if (lane == 0) head_inv[h] = 1.0f / sqrtf(static_cast<float>(ss / hd) + a.eps);
        }
        __syncthreads();
        for (int i = tid; i < n; i += 256) {
            const int h = i / hd;
            xs[i] = a.norm_w[i - h * hd] * (xs[i] * head_inv[h]) * silu_f(a.gate[i]);
        }
    }
    __syncthreads();
}

template <int PRO, bool RESID, int RPW>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    extern __shared__ float xs[];
    stage_input<PRO>(a, xs);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = a.in_dim;
    const int nfull = n >> 9;              // 512-element chunks: 64 lanes x 8
    const int tail = n - (nfull << 9);     // multiple of 8
    const int row_step = gridDim.x * 4 * RPW;
    for (int r0 = (blockIdx.x * 4 + wave) * RPW; r0 < a.rows; r0 += row_step) {
        const uint16_t* wr[RPW];
        float acc[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = min(r0 + r, a.rows - 1);
            wr[r] = a.W + static_cast<size_t>(row) * n + lane * 8;
            acc[r] = 0.0f;
        }
        int k = 0;
        for (; k + 4 <= nfull; k += 4) {
            u32x4 w[4][RPW];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < RPW; ++r)
                    w[u][r] = load_w(wr[r] + ((k + u) << 9));
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = ((k + u) << 9) + lane * 8;
                const float4 x0 = *reinterpret_cast<const float4*>(xs + c);
                const float4 x1 = *reinterpret_cast<const float4*>(xs + c + 4);
#pragma unroll
                for (int r = 0; r < RPW; ++r) acc[r] = dot8(w[u][r], x0, x1, acc[r]);
            }
        }
        for (; k < nfull; ++k) {
            u32x4 w[RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) w[r] = load_w(wr[r] + (k << 9));
            const int c = (k << 9) + lane * 8;
            const float4 x0 = *reinterpret_cast<const float4*>(xs + c);
            const float4 x1 = *reinterpret_cast<const float4*>(xs + c + 4);
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[r] = dot8(w[r], x0, x1, acc[r]);
        }
        if (lane * 8 < tail) {
            const int c = (nfull << 9) + lane * 8;
            const float4 x0 = *reinterpret_cast<const float4*>(xs + c);
            const float4 x1 = *reinterpret_cast<const float4*>(xs + c + 4);
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const u32x4 w = load_w(wr[r] + (nfull << 9));
                acc[r] = dot8(w, x0, x1, acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == 0 && r0 + r < a.rows) a.y[r0 + r] = RESID ? a.resid[r0 + r] + s : s;
        }
    }
}

template <int PRO, bool RESID>
hipError_t launch_rpw(const GemvArgs& a, hipStream_t s) {
    const size_t lds = static_cast<size_t>(a.in_dim) * sizeof(float);
    constexpr int kMaxBlocks = 2048;
    if (a.rows >= 8192) {
        const int blocks = min(kMaxBlocks, (a.rows + 7) / 8);
        gemv_kernel<PRO, RESID, 2><<<blocks, 256, lds, s>>>(a);
    } else {
        const int blocks = min(kMaxBlocks, (a.rows + 3) / 4);
        gemv_kernel<PRO, RESID, 1><<<blocks, 256, lds, s>>>(a);
    }
    return hipGetLastError();
}

template <int PRO>
hipError_t launch_pro(const GemvArgs& a, hipStream_t s) {
    return a.resid ? launch_rpw<PRO, true>(a, s) : launch_rpw<PRO, false>(a, s);
}

}  // namespace

hipError_t launch_gemv(const GemvArgs& a, int prologue, hipStream_t s) {
    switch (prologue) {
        case kProPlain: return launch_pro<kProPlain>(a, s);
        case kProRmsNorm: return launch_pro<kProRmsNorm>(a, s);
        case kProSwiGlu: return launch_pro<kProSwiGlu>(a, s);
        case kProGatedNorm: return launch_pro<kProGatedNorm>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace q35k
