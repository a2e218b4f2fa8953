// Token-batched projection GEMM for the prefill: Y[M][N] = (R ?) + X[M][K] . W[N][K]^T (K % 8 == 0)
// with fp32 activations X, bf16 weights W (nn.Linear row-major layout) and fp32 results: the
// reference's per-token matmul (src/forward_pass.cpp:44-75) for all prompt tokens at once.
//
// Exact three-way bf16 split on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16). Every fp32
// x is the exact sum of three bf16 values: hi = x with its low 16 bits cleared, r = x - hi
// (exact, at most 16 significant bits), mid = r with its low 16 bits cleared, lo = r - mid
// (exact, at most 8 significant bits, so a bf16). A bf16 x bf16 product has at most 16
// significant bits and is exact in fp32, so W.x = W.hi + W.mid + W.lo is the fp32 matmul with
// fp32 accumulation -- three bf16 MFMAs at 16x the fp32-MFMA rate instead of one fp32 MFMA.
//
// Tiling: 128 x 128 output tile per 256-thread workgroup, 4 waves in a 2 x 2 arrangement of
// 64 x 64 quadrants, each quadrant 2 x 2 MFMA blocks of 32 x 32 (64 accumulator registers
// per lane). K advances in stages of 32: the X and W tiles of the next stage are loaded into
// registers while the current stage runs from LDS (branch-free loads, LDS-only barriers, so
// the loads stay in flight until the next stage's LDS store needs them). LDS holds the three bf16 parts of the X
// tile and the W tile k-contiguous ([row][k], rows padded to 40 elements), so each MFMA
// operand is one 16-byte read of 8 consecutive k.
//
// MFMA operand layout (32x32x16 bf16, one block): lane l supplies row / column l % 32 and the 8
// k values 8 (l / 32) .. 8 (l / 32) + 7 of the 16-k step; both operands use the same k
// assignment, so the sum covers all 16. The result register v of lane l is
// D[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kLd = kBK + 8;  // padded row (bf16 elements): 80 B, rows start on distinct banks

// EPI: 0 store, 1 add the residual, 2 SwiGLU of interleaved (gate, up) column pairs
template <int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
    __shared__ __align__(16) uint16_t Xs[3][kBM][kLd];
    __shared__ __align__(16) uint16_t Ws[kBN][kLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

    // global -> register mapping: thread t loads row t / 2, k half (t % 2) of the stage
    constexpr int NXQ = kBK / 8, NWQ = kBK / 16;  // 16-byte X / W chunks per thread and stage
    const int lr = tid >> 1, lk = (tid & 1) * (kBK / 2);
    const bool a_ok = m0 + lr < a.M, b_ok = n0 + lr < a.N;
    const float* xrow = a.X + static_cast<int64_t>(a_ok ? m0 + lr : 0) * a.ldx;
    const uint16_t* wrow = a.W + static_cast<int64_t>(b_ok ? n0 + lr : 0) * a.K;
    // The next stage's X / W tiles are requested into registers right after the current
    // stage is in LDS and stay in flight while it is multiplied. Loads are unconditional
    // (clamped to element K - 8 of a valid row); chunks past K or past the last row are
    // zeroed by a bit mask when the stage is stored. A load or a use under a branch would
    // make the wait-count pass wait for every outstanding load at the join.
    // K % 8 == 0: a 4-float or 8-bf16 chunk is wholly inside K or wholly past it (zeros)
    uint4 raA[NXQ];  // fp32 bit patterns
    uint4 rbA[NWQ];
    auto load_stage = [&](uint4 (&ra)[NXQ], uint4 (&rb)[NWQ], int k0) {
#pragma unroll
        for (int i = 0; i < NXQ; ++i)
            ra[i] = *reinterpret_cast<const uint4*>(xrow + min(k0 + lk + 4 * i, a.K - 4));
#pragma unroll
        for (int i = 0; i < NWQ; ++i) rb[i] = *reinterpret_cast<const uint4*>(wrow + min(k0 + lk + 8 * i, a.K - 8));
    };
    auto masked = [](uint4 v, bool live) {
        const uint32_t m = 0u - static_cast<uint32_t>(live);
        return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
    };
    auto store_stage = [&](const uint4 (&rx)[NXQ], const uint4 (&rw)[NWQ], int k0) {
        uint4 ra[NXQ], rb[NWQ];
#pragma unroll
        for (int i = 0; i < NXQ; ++i) ra[i] = masked(rx[i], a_ok && k0 + lk + 4 * i < a.K);
#pragma unroll
        for (int i = 0; i < NWQ; ++i) rb[i] = masked(rw[i], b_ok && k0 + lk + 8 * i < a.K);
        uint32_t hp[2 * NXQ], mp[2 * NXQ], lp[2 * NXQ];  // pairs of bf16 packed in a word
#pragma unroll
        for (int i = 0; i < NXQ; ++i) {
            const float v[4] = {__uint_as_float(ra[i].x), __uint_as_float(ra[i].y), __uint_as_float(ra[i].z),
                                 __uint_as_float(ra[i].w)};
#pragma unroll
            for (int j = 0; j < 4; j += 2) {
                uint32_t h0, m0_, l0, h1, m1, l1;
                split3(v[j], h0, m0_, l0);
                split3(v[j + 1], h1, m1, l1);
                hp[2 * i + j / 2] = h0 | (h1 << 16);
                mp[2 * i + j / 2] = m0_ | (m1 << 16);
                lp[2 * i + j / 2] = l0 | (l1 << 16);
            }
        }
#pragma unroll
        for (int q = 0; q < NWQ; ++q) {
            *reinterpret_cast<uint4*>(&Xs[0][lr][lk + 8 * q]) = make_uint4(hp[4 * q], hp[4 * q + 1], hp[4 * q + 2], hp[4 * q + 3]);
            *reinterpret_cast<uint4*>(&Xs[1][lr][lk + 8 * q]) = make_uint4(mp[4 * q], mp[4 * q + 1], mp[4 * q + 2], mp[4 * q + 3]);
            *reinterpret_cast<uint4*>(&Xs[2][lr][lk + 8 * q]) = make_uint4(lp[4 * q], lp[4 * q + 1], lp[4 * q + 2], lp[4 * q + 3]);
            *reinterpret_cast<uint4*>(&Ws[lr][lk + 8 * q]) = rb[q];
        }
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int ar = wm * 64 + (lane & 31), br = wn * 64 + (lane & 31), kh = (lane >> 5) * 8;
    auto mma = [&]() {
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            const int kk = s * 16 + kh;
            bf16x8 bop[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) bop[j] = *reinterpret_cast<const bf16x8*>(&Ws[br + 32 * j][kk]);
#pragma unroll
            for (int p = 2; p >= 0; --p) {  // lo, mid, hi
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const bf16x8 aop = *reinterpret_cast<const bf16x8*>(&Xs[p][ar + 32 * i][kk]);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop, bop[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    };
    // LDS-only barriers: the next stages' global loads stay in flight through them
    load_stage(raA, rbA, 0);
    for (int k0 = 0; k0 < a.K; k0 += kBK) {
        lds_barrier();  // the previous stage's operands have been read
        store_stage(raA, rbA, k0);
        lds_barrier();
        load_stage(raA, rbA, k0 + kBK);
        mma();
    }
    if constexpr (EPI == 2) {
        // the pair (gate, up) of one output sits in adjacent lanes (even, odd column)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float up = __shfl_xor(acc[i][j][v], 1);
                    const int row = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    if (!(lane & 1) && col + 1 < a.N && row < a.M)
                        a.Y[static_cast<int64_t>(row) * a.ldy + (col >> 1)] = silu_f(acc[i][j][v]) * up;
                }
            }
        return;
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
                    *y = EPI == 1 ? a.R[static_cast<int64_t>(row) * a.ldr + col] + acc[i][j][v] : acc[i][j][v];
                }
            }
        }
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    dim3 grid((a.N + kBN - 1) / kBN, (a.M + kBM - 1) / kBM);
    if (a.swiglu) klaunch(gemm_kernel<2>, grid, 256, 0, s, a);
    else if (a.R) klaunch(gemm_kernel<1>, grid, 256, 0, s, a);
    else klaunch(gemm_kernel<0>, grid, 256, 0, s, a);
    return hipGetLastError();
}

}  // namespace q35k
