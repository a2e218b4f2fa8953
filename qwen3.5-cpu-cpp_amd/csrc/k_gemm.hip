// Token-batched projection GEMM for the prefill: Y[M][N] = (R ?) + X[M][K] . W[N][K]^T (K % 8 == 0)
// with fp32 activations X, bf16 weights W (nn.Linear row-major layout) and fp32 results: the
// reference's per-token matmul (src/forward_pass.cpp:44-75) for all prompt tokens at once.
//
// Exact three-way bf16 split on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16). Every fp32
// x is the exact sum of three bf16 values: hi = x with its low 16 bits cleared, r = x - hi
// (exact, at most 16 significant bits), mid = r with its low 16 bits cleared, lo = r - mid
// (exact, at most 8 significant bits, so a bf16). A bf16 x bf16 product has at most 16
// significant bits and is exact in fp32, so W.x = W.hi + W.mid + W.lo is the fp32 matmul with
// fp32 accumulation -- three bf16 MFMAs at 16x the fp32-MFMA rate instead of one fp32 MFMA.
//
// Tiling: 128 x 128 output tile per 256-thread workgroup, each of the 4 waves a 32-row slab
// of it: 2 x 8 MFMA blocks of 16 x 16 (64 accumulator registers per lane). K advances in
// stages of 32 (one 16x16x32 MFMA deep): the X and W tiles of the next stage are loaded into
// registers while the current stage runs from LDS (branch-free loads, LDS-only barriers, so
// the loads stay in flight until the next stage's LDS store needs them). LDS holds the X
// tile as fp32 ([row][k], rows padded to 36 floats) and the W tile as bf16 ([row][k], rows
// padded to 40 elements); a wave reads its 8 fp32 k values of an X row (two 16-byte reads)
// and splits them into the three bf16 A operands in registers, and each W operand is one
// 16-byte read (16 consecutive rows at either padding hit distinct banks). The split of a
// value happens once, in the one wave that uses it.
//
// Accumulation: an MFMA adds its exact products into the accumulator with rounding, 3 K / 16
// rounded additions per output over K in one fp32 accumulator (384 at K = 2048): four times
// the error of the matvec's per-lane chains and tree (measured against float64 at K = 2048:
// 4.9e-7 against 1.2e-7), enough to move a 24-layer prefill's state past 1e-5 of the
// sequential reference. Each block of kFlush stages is therefore accumulated from zero and
// then added to the running total: 2.4e-7 at K = 2048 and 6144, for 6% more GEMM time (the
// additions wait for the block's last products; flushing every 8 stages halves the error
// gain per cost, and a second accumulator set costs the second wave per SIMD).
//
// MFMA operand layout (16x16x32 bf16, one block): lane l supplies row / column l % 16 and the
// 8 k values 8 (l / 16) .. 8 (l / 16) + 7 of the 32-k step; both operands use the same k
// assignment, so the sum covers all 32. The result register v of lane l is
// D[4 (l / 16) + v][l % 16].
#include <type_traits>

#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBK = 32;
constexpr int kFlush = 16;    // stages per partial sum (K = 512)
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
template <int EPI>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
    constexpr int kBN = 128;
    __shared__ __align__(16) float Xs[kBM][kLdX];
    __shared__ __align__(16) uint16_t Ws[kBN][kLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

    // global -> register mapping: thread t loads X row t / 2 and W row t / 2, k half (t % 2)
    constexpr int NXQ = kBK / 8, NWQ = kBK / 16;  // 16-byte X / W chunks per thread and stage
    const int lr = tid >> 1, lk = (tid & 1) * (kBK / 2);
    const int wr = lr, wk = lk;
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

    constexpr int kCB = kBN / 16;  // 16-column MFMA blocks per wave (two 16-row blocks)
    floatx4 acc[2][kCB], part[2][kCB];  // running total, partial sum of the current block
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int j = 0; j < kCB; ++j) acc[r][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int l16 = lane & 15, kq = (lane >> 4) * 8;
    auto mma = [&](auto fresh) {
        bf16x8 aop[2][3];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int ar = wave * 32 + 16 * r + l16;
            const float4 x0 = *reinterpret_cast<const float4*>(&Xs[ar][kq]);
            const float4 x1 = *reinterpret_cast<const float4*>(&Xs[ar][kq + 4]);
            uint32_t h[4], m[4], l[4];
            split3_pair(x0.x, x0.y, h[0], m[0], l[0]);
            split3_pair(x0.z, x0.w, h[1], m[1], l[1]);
            split3_pair(x1.x, x1.y, h[2], m[2], l[2]);
            split3_pair(x1.z, x1.w, h[3], m[3], l[3]);
            aop[r][0] = __builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]});
            aop[r][1] = __builtin_bit_cast(bf16x8, u32x4{m[0], m[1], m[2], m[3]});
            aop[r][2] = __builtin_bit_cast(bf16x8, u32x4{l[0], l[1], l[2], l[3]});
        }
#pragma unroll
        for (int j = 0; j < kCB; ++j) {
            const bf16x8 bop = *reinterpret_cast<const bf16x8*>(&Ws[16 * j + l16][kq]);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int p = 2; p >= 0; --p) {  // lo, mid, hi
                    if constexpr (decltype(fresh)::value) {
                        part[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            aop[r][p], bop, p == 2 ? floatx4{0.f, 0.f, 0.f, 0.f} : part[r][j], 0, 0, 0);
                    } else {
                        part[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[r][p], bop, part[r][j], 0, 0, 0);
                    }
                }
        }
    };
    // LDS-only barriers: the next stages' global loads stay in flight through them
    load_stage(raA, rbA, 0);
    for (int kb = 0; kb < a.K; kb += kFlush * kBK) {
#pragma unroll
        for (int f = 0; f < kFlush; ++f) {
            const int k0 = kb + f * kBK;  // stages past K hold zeros (masked when stored)
            lds_barrier();  // the previous stage's operands have been read
            store_stage(raA, rbA, k0);
            lds_barrier();
            load_stage(raA, rbA, k0 + kBK);
            if (f == 0) mma(std::true_type{});
            else mma(std::false_type{});
        }
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < kCB; ++j) acc[r][j] += part[r][j];
    }
    const int rbase = m0 + wave * 32 + 4 * (lane >> 4);
    if constexpr (EPI == 2) {
        // the pair (gate, up) of one output sits in adjacent lanes (even, odd column)
#pragma unroll
        for (int j = 0; j < kCB; ++j) {
            const int col = n0 + 16 * j + l16;
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float up = __shfl_xor(acc[r][j][v], 1);
                    const int row = rbase + 16 * r + v;
                    if (!(lane & 1) && col + 1 < a.N && row < a.M)
                        a.Y[static_cast<int64_t>(row) * a.ldy + (col >> 1)] = silu_f(acc[r][j][v]) * up;
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < kCB; ++j) {
        const int col = n0 + 16 * j + l16;
        if (col >= a.N) continue;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = rbase + 16 * r + v;
                if (row < a.M) {
                    float* y = a.Y + static_cast<int64_t>(row) * a.ldy + col;
                    *y = EPI == 1 ? a.R[static_cast<int64_t>(row) * a.ldr + col] + acc[r][j][v] : acc[r][j][v];
                }
            }
    }
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    dim3 grid((a.N + 127) / 128, (a.M + kBM - 1) / kBM);
    if (a.swiglu) klaunch(gemm_kernel<2>, grid, 256, 0, s, a);
    else if (a.R) klaunch(gemm_kernel<1>, grid, 256, 0, s, a);
    else klaunch(gemm_kernel<0>, grid, 256, 0, s, a);
    return hipGetLastError();
}

}  // namespace q35k
