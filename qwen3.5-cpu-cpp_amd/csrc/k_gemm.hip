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
// Tiling: 128 x BN output tile per 256-thread workgroup (BN = 128, or 256 for the widest
// projection), each of the 4 waves a 32-row slab of it: 1 x BN / 32 MFMA blocks of 32 x 32
// (64 or 128 accumulator registers per lane). K advances in
// stages of 32: the X and W tiles of the next stage are loaded into registers while the
// current stage runs from LDS (branch-free loads, LDS-only barriers, so the loads stay in
// flight until the next stage's LDS store needs them). LDS holds the X tile as fp32
// ([row][k], rows padded to 36 floats) and the W tile as bf16 ([row][k], rows padded to 40
// elements); a wave reads its 8 fp32 k values of an X row (two 16-byte reads) and splits them
// into the three bf16 A operands in registers, and each W operand is one 16-byte read. Per
// 12 MFMAs a wave reads 32 B of X and 64 B of W per lane from LDS (a quarter less LDS traffic
// than three pre-split bf16 X tiles), and the split of a value happens once, in the one wave
// that uses it.
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
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBK = 32;
constexpr int kLdX = kBK + 4;  // padded X row (floats): 144 B, 16-byte reads of 8 rows hit distinct banks
constexpr int kLd = kBK + 8;   // padded W row (bf16 elements): 80 B

// the three bf16 parts of two floats a, b, each part's pair packed (a low, b high)
__device__ __forceinline__ void split3_pair(float a, float b, uint32_t& h, uint32_t& m, uint32_t& l) {
    const uint32_t ha = __float_as_uint(a) & 0xffff0000u, hb = __float_as_uint(b) & 0xffff0000u;
    const float ra = a - __uint_as_float(ha), rb = b - __uint_as_float(hb);
    const uint32_t ma = __float_as_uint(ra) & 0xffff0000u, mb = __float_as_uint(rb) & 0xffff0000u;
    const float la = ra - __uint_as_float(ma), lb = rb - __uint_as_float(mb);
    h = (ha >> 16) | hb;
    m = (ma >> 16) | mb;
    l = (__float_as_uint(la) >> 16) | (__float_as_uint(lb) & 0xffff0000u);
}

// EPI: 0 store, 1 add the residual, 2 SwiGLU of interleaved (gate, up) column pairs.
// BN: tile width, 128 (4 MFMA blocks per wave) or 256 (8 blocks, two waves per SIMD).
template <int EPI, int BN>
__global__ __launch_bounds__(256, BN == 256 ? 2 : 1) void gemm_kernel(GemmArgs a) {
    constexpr int kBN = BN, kNB = BN / 32;  // 32-column MFMA blocks per wave
    __shared__ __align__(16) float Xs[kBM][kLdX];
    __shared__ __align__(16) uint16_t Ws[kBN][kLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

    // global -> register mapping: thread t loads X row t / 2, k half (t % 2), and W row
    // t * BN / 256 .. of the stage: k half (t % 2) for BN = 128, all of it for BN = 256
    constexpr int NXQ = kBK / 8, NWQ = kBK * BN / (8 * 256);  // 16-byte X / W chunks per thread and stage
    const int lr = tid >> 1, lk = (tid & 1) * (kBK / 2);
    const int wr = BN == 256 ? tid : lr, wk = BN == 256 ? 0 : lk;
    const bool a_ok = m0 + lr < a.M, b_ok = n0 + wr < a.N;
    const float* xrow = a.X + static_cast<int64_t>(a_ok ? m0 + lr : 0) * a.ldx;
    const uint16_t* wrow = a.W + static_cast<int64_t>(b_ok ? n0 + wr : 0) * a.K;
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
        for (int i = 0; i < NWQ; ++i) rb[i] = *reinterpret_cast<const uint4*>(wrow + min(k0 + wk + 8 * i, a.K - 8));
    };
    auto masked = [](uint4 v, bool live) {
        const uint32_t m = 0u - static_cast<uint32_t>(live);
        return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
    };
    auto store_stage = [&](const uint4 (&rx)[NXQ], const uint4 (&rw)[NWQ], int k0) {
#pragma unroll
        for (int i = 0; i < NXQ; ++i)
            *reinterpret_cast<uint4*>(&Xs[lr][lk + 4 * i]) = masked(rx[i], a_ok && k0 + lk + 4 * i < a.K);
#pragma unroll
        for (int q = 0; q < NWQ; ++q)
            *reinterpret_cast<uint4*>(&Ws[wr][wk + 8 * q]) = masked(rw[q], b_ok && k0 + wk + 8 * q < a.K);
    };

    floatx16 acc[kNB];
#pragma unroll
    for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;

    const int ar = wave * 32 + (lane & 31), br = lane & 31, kh = (lane >> 5) * 8;
    auto mma = [&]() {
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            const int kk = s * 16 + kh;
            const float4 x0 = *reinterpret_cast<const float4*>(&Xs[ar][kk]);
            const float4 x1 = *reinterpret_cast<const float4*>(&Xs[ar][kk + 4]);
            bf16x8 bop[kNB];
#pragma unroll
            for (int j = 0; j < kNB; ++j) bop[j] = *reinterpret_cast<const bf16x8*>(&Ws[br + 32 * j][kk]);
            uint32_t h[4], m[4], l[4];
            split3_pair(x0.x, x0.y, h[0], m[0], l[0]);
            split3_pair(x0.z, x0.w, h[1], m[1], l[1]);
            split3_pair(x1.x, x1.y, h[2], m[2], l[2]);
            split3_pair(x1.z, x1.w, h[3], m[3], l[3]);
            const bf16x8 aop[3] = {__builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]}),
                                   __builtin_bit_cast(bf16x8, u32x4{m[0], m[1], m[2], m[3]}),
                                   __builtin_bit_cast(bf16x8, u32x4{l[0], l[1], l[2], l[3]})};
#pragma unroll
            for (int p = 2; p >= 0; --p)  // lo, mid, hi
#pragma unroll
                for (int j = 0; j < kNB; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop[p], bop[j], acc[j], 0, 0, 0);
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
    const int rbase = m0 + wave * 32 + 4 * (lane >> 5);
    if constexpr (EPI == 2) {
        // the pair (gate, up) of one output sits in adjacent lanes (even, odd column)
#pragma unroll
        for (int j = 0; j < kNB; ++j) {
            const int col = n0 + j * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float up = __shfl_xor(acc[j][v], 1);
                const int row = rbase + 8 * (v >> 2) + (v & 3);
                if (!(lane & 1) && col + 1 < a.N && row < a.M)
                    a.Y[static_cast<int64_t>(row) * a.ldy + (col >> 1)] = silu_f(acc[j][v]) * up;
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
        const int col = n0 + j * 32 + (lane & 31);
        if (col >= a.N) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = rbase + 8 * (v >> 2) + (v & 3);
            if (row < a.M) {
                float* y = a.Y + static_cast<int64_t>(row) * a.ldy + col;
                *y = EPI == 1 ? a.R[static_cast<int64_t>(row) * a.ldr + col] + acc[j][v] : acc[j][v];
            }
        }
    }
}

template <int BN>
void launch_bn(const GemmArgs& a, hipStream_t s) {
    dim3 grid((a.N + BN - 1) / BN, (a.M + kBM - 1) / kBM);
    if (a.swiglu) klaunch(gemm_kernel<2, BN>, grid, 256, 0, s, a);
    else if (a.R) klaunch(gemm_kernel<1, BN>, grid, 256, 0, s, a);
    else klaunch(gemm_kernel<0, BN>, grid, 256, 0, s, a);
}

}  // namespace

// 256-wide tiles for the widest projections (the interleaved gate/up: 7% faster at 4096 x
// 12288 x 2048), 128-wide for the rest, where 256-wide tiles leave too few workgroups.
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.N >= 12288) launch_bn<256>(a, s);
    else launch_bn<128>(a, s);
    return hipGetLastError();
}

}  // namespace q35k
