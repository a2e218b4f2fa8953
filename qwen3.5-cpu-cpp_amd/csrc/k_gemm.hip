// Token-batched projection GEMM for the prefill: Y[M][N] = (R ?) + X[M][K] . W[N][K]^T (K % 8 == 0) with
// fp32 activations X, bf16 weights W (nn.Linear row-major layout, widened exactly) and fp32
// accumulation on the matrix cores (v_mfma_f32_32x32x2_f32). This is the reference's
// per-token matmul (src/forward_pass.cpp:44-75) for all prompt tokens at once.
//
// Tiling: 128 x 128 output tile per 256-thread workgroup, 4 waves in a 2 x 2 arrangement of
// 64 x 64 quadrants, each quadrant 2 x 2 MFMA blocks of 32 x 32 (64 accumulator registers
// per lane). K advances in stages of 32: the X and W tiles of the next stage are loaded
// into registers while the current stage runs from LDS. LDS keeps both tiles k-major
// ([k][m], [k][n]) so every operand read is 32 consecutive floats across lanes.
//
// MFMA operand layout (32x32x2, one block): lane l supplies A[l % 32][l / 32] and
// B[l / 32][l % 32]; the result register v of lane l is D[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
// The two k slots of each instruction take k = 16 (l / 32) + s at step s, a fixed
// permutation of the stage's 32 k values applied to both operands.
#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 32;

template <bool RESID>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
    __shared__ float As[kBK][kBM + 4];
    __shared__ float Bs[kBK][kBN + 4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

    // global -> register mapping: thread t loads row t / 2, k half (t % 2) * 16 of the stage
    const int lr = tid >> 1, lk = (tid & 1) * 16;
    const bool a_ok = m0 + lr < a.M, b_ok = n0 + lr < a.N;
    const float* xrow = a.X + static_cast<int64_t>(a_ok ? m0 + lr : 0) * a.ldx + lk;
    const uint16_t* wrow = a.W + static_cast<int64_t>(b_ok ? n0 + lr : 0) * a.K + lk;
    float4 ra[4];
    uint4 rb[2];
    // K % 8 == 0: a 4-float or 8-bf16 chunk is wholly inside K or wholly past it (zeros)
    auto load_stage = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ra[i] = a_ok && k0 + lk + 4 * i < a.K ? *reinterpret_cast<const float4*>(xrow + k0 + 4 * i)
                                                  : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            rb[i] = b_ok && k0 + lk + 8 * i < a.K ? *reinterpret_cast<const uint4*>(wrow + k0 + 8 * i)
                                                  : make_uint4(0u, 0u, 0u, 0u);
    };
    auto store_stage = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            As[lk + 4 * i + 0][lr] = ra[i].x;
            As[lk + 4 * i + 1][lr] = ra[i].y;
            As[lk + 4 * i + 2][lr] = ra[i].z;
            As[lk + 4 * i + 3][lr] = ra[i].w;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t w4[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                Bs[lk + 8 * i + 2 * j][lr] = bf16_lo(w4[j]);
                Bs[lk + 8 * i + 2 * j + 1][lr] = bf16_hi(w4[j]);
            }
        }
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int am = wm * 64 + (lane & 31), bn = wn * 64 + (lane & 31), kg = (lane >> 5) * 16;
    load_stage(0);
    for (int k0 = 0; k0 < a.K; k0 += kBK) {
        __syncthreads();
        store_stage();
        __syncthreads();
        if (k0 + kBK < a.K) load_stage(k0 + kBK);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float a0 = As[kg + s][am], a1 = As[kg + s][am + 32];
            const float b0 = Bs[kg + s][bn], b1 = Bs[kg + s][bn + 32];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + (lane & 31);
            if (col >= a.N) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (row < a.M) {
                    float* y = a.Y + static_cast<int64_t>(row) * a.ldy + col;
                    *y = RESID ? a.R[static_cast<int64_t>(row) * a.ldr + col] + acc[i][j][v] : acc[i][j][v];
                }
            }
        }
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    dim3 grid((a.N + kBN - 1) / kBN, (a.M + kBM - 1) / kBM);
    if (a.R) gemm_kernel<true><<<grid, 256, 0, s>>>(a);
    else gemm_kernel<false><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace q35k
