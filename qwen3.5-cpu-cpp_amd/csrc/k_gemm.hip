// Token-batched projection GEMM for the prefill: Y[M][N] = (R ?) + X[M][K] . W[N][K]^T (K % 8 == 0)
// with fp32 activations X, bf16 weights W (nn.Linear row-major layout) and fp32 results: the
// reference's per-token matmul (src/forward_pass.cpp:44-75) for all prompt tokens at once.
//
// Two paths on the 16-bit matrix cores:
//   bf16 (any caller): exact three-way bf16 split (v_mfma_f32_16x16x32_bf16). Every fp32 x
//   is the exact sum of three bf16 values: hi = x with its low 16 bits cleared, r = x - hi
//   (exact, at most 16 significant bits), mid = r with its low 16 bits cleared, lo = r - mid
//   (exact, at most 8 significant bits, so a bf16). A bf16 x bf16 product has at most 16
//   significant bits and is exact in fp32, so W.x = W.hi + W.mid + W.lo is the fp32 matmul
//   with fp32 accumulation -- three bf16 MFMAs at 16x the fp32-MFMA rate instead of one.
//   fp16 (the model's prefill: Wh, xmax set, X in the tiled layout of xt_off so that each
//   wave-wide 16-byte load reads one contiguous KB): two fp16 parts against an fp16 copy of the
//   weights (Wh = W 2^w_exp, exact for every bf16 weight down to 2^-24 of the largest, which
//   lies in [2^14, 2^15)). Each X row is first scaled by a power of two from its maximum (the
//   producing kernel writes per-row partial maxima) so that it lies in (-2^15, 2^15) with
//   its maximum at or above 2^14; then h = fp16(x), l = fp16(x - h). x - h - l is at most
//   2^-22 |x| (2^-25 absolute below the fp16 normal range, i.e. 2^-39 of the row maximum):
//   four times fp32's unit roundoff 2^-24, so h + l carries about 22 significant bits of x
//   where the three bf16 parts carry all 24. Each fp16 x fp16 product is exact in fp32; the
//   epilogue multiplies by 2^-(row exponent + w_exp), exactly. Two MFMAs per product instead
//   of three: 5-8% faster; against float64 the outputs stay within the fp32 accumulation
//   error (the dropped 2^-22 |x| averages out over K like the accumulator's own roundings).
//   x_planes: the producer (the prefill's input norm) already wrote each row scaled and split
//   the same way (xp_off), and the parts are loaded as the operands themselves -- the split
//   is not repeated for every 128-column tile of the output.
//
// Tiling: 128 x 128 output tile per 256-thread workgroup, each of the 4 waves a 32-row slab
// of it: 2 x 8 MFMA blocks of 16 x 16 (64 accumulator registers per lane). K advances in
// stages of 32 (one 16x16x32 MFMA deep).
//   X (A operand): every X element of the tile is used by one wave only, so each wave loads
//   its own rows straight from global memory into registers (8 consecutive k per lane, two
//   16-byte loads per 16-row block), two stages ahead, and splits them in registers.
//   W (B operand): shared by the four waves, staged through LDS in two buffers: stage f + 1
//   is stored into one buffer while stage f is multiplied from the other, one LDS-only
//   barrier per stage, and its global loads are issued a stage ahead. Rows are padded to
//   96 bytes for the full rate of the 16-byte operand reads on gfx950, where one clock
//   serves lanes 0-7 with 16-23 (then 8-15 with 24-31, and the same in the upper half-wave)
//   and those 16 lanes must cover all 64 banks: lanes 0-7 and 16-23 read rows 0-7 at k
//   offsets 0 and 16 bytes, 16 distinct 16-byte bank slots at a 96-byte pitch (6 slots per
//   row; the 80-byte pitch paired them up, two clocks per read). Measured: a third of the
//   bank-conflict cycles left (the staging stores), 1.4% less GEMM time. Pairing the stores
//   too needs a staging map whose adjacent lanes load different rows, which cost 8%.
// LDS traffic is the W reads alone (the X tile no longer passes through LDS): measured 13-18%
// faster than staging both operands in LDS, with bit-identical results.
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
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kFlush = 16;   // stages per partial sum (K = 512)
constexpr int kLd = kBK + 16;  // padded W row in LDS (bf16 elements): 96 B
constexpr int kCB = kBN / 16;  // 16-column MFMA blocks per wave (two 16-row blocks)

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

// the two fp16 parts of two (scaled) floats a, b: h = rn(x), l = rn(x - h), each pair packed
// One 128 x 128 tile. MASK: some W rows of the tile lie past N or K is not a whole number of
// flush blocks, so W and X chunks past N or K are zeroed (X rows past M are clamped to row 0
// and their outputs dropped).
// EPI: 0 store, 1 add the residual, 2 SwiGLU of interleaved (gate, up) column pairs.
// F16: two fp16 parts per activation against the fp16 weight copy (see launch_gemm).
// XP (with F16): X already split by its producer (x_planes, the layout of xp_off): the two
// parts are loaded as the operands themselves, nothing is split here.
template <int EPI, bool MASK, bool F16, bool XP>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, int tx, int ty, uint16_t (*Ws)[kLd]) {
    using OpT = typename std::conditional<F16, halfx8, bf16x8>::type;
    constexpr int NP = F16 ? 2 : 3;  // parts per activation
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = ty * kBM, n0 = tx * kBN;
    const int l16 = lane & 15, kq = (lane >> 4) * 8;
    const float* arow[2];  // this lane's X row in each of the wave's two 16-row blocks
    int arow_i[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int row = m0 + wave * 32 + 16 * r + l16;
        arow_i[r] = row < a.M ? row : 0;
        // F16 (tiled X): the lane's 16 bytes in the first k block of its row block (XP: of the
        // high part; the low part's are 1 KB further, where the tiled fp32 layout has the
        // second 16 bytes)
        arow[r] = F16 ? a.X + static_cast<int64_t>((m0 >> 4) + 2 * wave + r) * (a.K >> 5) * 512 +
                            (XP ? lane << 2 : (l16 << 4) + ((lane >> 4) << 2))
                      : a.X + static_cast<int64_t>(arow_i[r]) * a.ldx;
    }
    // F16: each row's scale 2^xe, xe = 15 - (exponent of its maximum |x| as in frexp), so
    // the row lies in (-2^15, 2^15) with its maximum at or above 2^14; exact in fp32
    int xe[2] = {0, 0};
    float xs[2] = {1.0f, 1.0f};
    if constexpr (F16) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            float mx = 0.0f;
            for (int j = lane >> 4; j < a.xmax_n; j += 4) mx = fmaxf(mx, a.xmax[static_cast<int64_t>(arow_i[r]) * a.xmax_n + j]);
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            xe[r] = split_row_exp(mx);
            xs[r] = ldexpf(1.0f, xe[r]);
        }
    }
    // W staging: thread t loads 16 k of row t / 2 (half t % 2) of the tile, two 16-byte chunks
    const int wr = tid >> 1, wk = (tid & 1) * 16;
    const bool b_ok = n0 + wr < a.N;
    const uint16_t* wrow = (F16 ? a.Wh : a.W) + static_cast<int64_t>(b_ok ? n0 + wr : 0) * a.K;
    // Loads are unconditional (addresses clamped into the row) so that no load sits under a
    // branch: the wait-count pass would then wait for every outstanding load at the join.
    auto load_a = [&](uint4 (&xa)[2][2], int k0) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                if constexpr (F16)  // one 1 KB contiguous block per wave-wide load
                    xa[r][i] = *reinterpret_cast<const uint4*>(arow[r] + (min(k0, a.K - 32) >> 5) * 512 + 256 * i);
                else
                    xa[r][i] = *reinterpret_cast<const uint4*>(arow[r] + min(k0 + kq + 4 * i, a.K - 4));
            }
    };
    auto load_w = [&](uint4 (&wb)[2], int k0) {
#pragma unroll
        for (int q = 0; q < 2; ++q) wb[q] = *reinterpret_cast<const uint4*>(wrow + min(k0 + wk + 8 * q, a.K - 8));
    };
    auto store_w = [&](const uint4 (&wb)[2], int k0, int buf) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            uint4 v = wb[q];
            if constexpr (MASK) {  // K % 8 == 0: a chunk is wholly inside K or wholly past it
                const uint32_t m = 0u - static_cast<uint32_t>(b_ok && k0 + wk + 8 * q < a.K);
                v = make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
            }
            *reinterpret_cast<uint4*>(&Ws[buf * kBN + wr][wk + 8 * q]) = v;
        }
    };

    floatx4 acc[2][kCB], part[2][kCB];  // running total, partial sum of the current block
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int j = 0; j < kCB; ++j) acc[r][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto split_a = [&](const uint4 (&xa)[2][2], OpT (&aop)[2][NP], int k0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            float4 x0 = __builtin_bit_cast(float4, xa[r][0]), x1 = __builtin_bit_cast(float4, xa[r][1]);
            if constexpr (MASK) {  // k past K: zeros (the clamped values could be infinite)
                if (k0 + kq >= a.K) x0 = make_float4(0.f, 0.f, 0.f, 0.f);
                if (k0 + kq + 4 >= a.K) x1 = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            if constexpr (XP) {  // the parts as stored (k past K: zeros, as below)
                const bool live = !MASK || k0 < a.K;
                aop[r][0] = __builtin_bit_cast(OpT, live ? xa[r][0] : make_uint4(0u, 0u, 0u, 0u));
                aop[r][1] = __builtin_bit_cast(OpT, live ? xa[r][1] : make_uint4(0u, 0u, 0u, 0u));
                continue;
            }
            if constexpr (F16) {
                const float sc = xs[r];
                uint32_t h[4], l[4];
                split2h_pair(x0.x * sc, x0.y * sc, h[0], l[0]);
                split2h_pair(x0.z * sc, x0.w * sc, h[1], l[1]);
                split2h_pair(x1.x * sc, x1.y * sc, h[2], l[2]);
                split2h_pair(x1.z * sc, x1.w * sc, h[3], l[3]);
                aop[r][0] = __builtin_bit_cast(OpT, u32x4{h[0], h[1], h[2], h[3]});
                aop[r][1] = __builtin_bit_cast(OpT, u32x4{l[0], l[1], l[2], l[3]});
                continue;
            }
            uint32_t h[4], m[4], l[4];
            split3_pair(x0.x, x0.y, h[0], m[0], l[0]);
            split3_pair(x0.z, x0.w, h[1], m[1], l[1]);
            split3_pair(x1.x, x1.y, h[2], m[2], l[2]);
            split3_pair(x1.z, x1.w, h[3], m[3], l[3]);
            aop[r][0] = __builtin_bit_cast(OpT, u32x4{h[0], h[1], h[2], h[3]});
            aop[r][1] = __builtin_bit_cast(OpT, u32x4{m[0], m[1], m[2], m[3]});
            aop[r][NP - 1] = __builtin_bit_cast(OpT, u32x4{l[0], l[1], l[2], l[3]});
        }
    };
    // MASK: 16-column blocks wholly past N are skipped (a ragged last column tile, e.g. the
    // 32-column tail of an 8224-row projection, costs its live blocks only)
    const int jlive = MASK ? min(kCB, (a.N - n0 + 15) / 16) : kCB;
    auto mfma = [](const OpT& x, const OpT& w, const floatx4& c) {
        if constexpr (F16) return __builtin_amdgcn_mfma_f32_16x16x32_f16(x, w, c, 0, 0, 0);
        else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, w, c, 0, 0, 0);
    };
    auto products = [&](const OpT (&aop)[2][NP], int buf, auto fresh) {
#pragma unroll
        for (int j = 0; j < kCB; ++j) {
            if (MASK && j >= jlive) {
                if constexpr (decltype(fresh)::value) part[0][j] = part[1][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                continue;
            }
            const OpT bop = *reinterpret_cast<const OpT*>(&Ws[buf * kBN + 16 * j + l16][kq]);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int p = NP - 1; p >= 0; --p) {  // smallest part first
                    if constexpr (decltype(fresh)::value) {
                        part[r][j] = mfma(aop[r][p], bop, p == NP - 1 ? floatx4{0.f, 0.f, 0.f, 0.f} : part[r][j]);
                    } else {
                        part[r][j] = mfma(aop[r][p], bop, part[r][j]);
                    }
                }
        }
    };

    // Stage f: W of stage f is in LDS buffer f % 2, W of stage f + 1 and X of stages f, f + 1
    // are in registers (in flight). Stages past K hold zero W (MASK) or are never reached
    // (K a whole number of flush blocks).
    uint4 xa[2][2][2], wb[2];
    load_w(wb, 0);
    load_a(xa[0], 0);
    load_a(xa[1], kBK);
    store_w(wb, 0, 0);
    load_w(wb, kBK);
    lds_barrier();
    for (int kb = 0; kb < a.K; kb += kFlush * kBK) {
#pragma unroll
        for (int f = 0; f < kFlush; ++f) {  // kFlush is even: buffer and register set = f % 2
            const int k0 = kb + f * kBK;
            store_w(wb, k0 + kBK, (f + 1) & 1);  // its last readers passed the previous barrier
            load_w(wb, k0 + 2 * kBK);
            OpT aop[2][NP];
            split_a(xa[f & 1], aop, k0);
            load_a(xa[f & 1], k0 + 2 * kBK);
            // keep the loads ahead of the products (the scheduler would sink them)
            __builtin_amdgcn_sched_barrier(0);
            // the products at raised wave priority: the issue arbiter then prefers the wave
            // that feeds the matrix core over its SIMD partner's loads and splits
            __builtin_amdgcn_s_setprio(1);
            if (f == 0) products(aop, f & 1, std::true_type{});
            else products(aop, f & 1, std::false_type{});
            __builtin_amdgcn_s_setprio(0);
            lds_barrier();  // LDS only: the loads stay in flight
        }
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < kCB; ++j) acc[r][j] += part[r][j];
    }
    const int rbase = m0 + wave * 32 + 4 * (lane >> 4);
    if constexpr (F16) {
        // undo the scales: output row rbase + 16 r + v is the A row of lane 4 (lane / 16) + v
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float f = ldexpf(1.0f, -(__shfl(xe[r], 4 * (lane >> 4) + v) + a.w_exp));
#pragma unroll
                for (int j = 0; j < kCB; ++j) acc[r][j][v] *= f;
            }
    }
    if constexpr (EPI == 2) {
        // the pair (gate, up) of one output sits in adjacent lanes (even, odd column)
        float ym[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int j = 0; j < kCB; ++j) {
            const int col = n0 + 16 * j + l16;
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float up = __shfl_xor(acc[r][j][v], 1);
                    const int row = rbase + 16 * r + v;
                    const float h = silu_f(acc[r][j][v]) * up;
                    if (!(lane & 1) && col + 1 < a.N) {
                        ym[r][v] = fmaxf(ym[r][v], fabsf(h));
                        if (row < a.M)
                            a.Y[a.y_tiled ? xt_off(row, col >> 1, a.N >> 1)
                                          : static_cast<int64_t>(row) * a.ldy + (col >> 1)] = h;
                    }
                }
        }
        if (a.ymax) {  // uniform: each row's maximum over this tile's outputs
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float m = ym[r][v];
                    m = fmaxf(m, __shfl_xor(m, 1));
                    m = fmaxf(m, __shfl_xor(m, 2));
                    m = fmaxf(m, __shfl_xor(m, 4));
                    m = fmaxf(m, __shfl_xor(m, 8));
                    const int row = rbase + 16 * r + v;
                    if (l16 == 0 && row < a.M) a.ymax[static_cast<int64_t>(row) * gridDim.x + tx] = m;
                }
        }
        return;
    }
    // EPI 1: every residual value is requested before the first store. R may be Y itself, so
    // a load placed after a store waits for that store's round trip (one per element, 64 in a
    // row per lane); reading them all first keeps each element's read before its own write.
    // (Rows and columns past the matrix read a clamped element and store nothing.)
    float rv[kCB][2][4];
    if constexpr (EPI == 1) {
#pragma unroll
        for (int j = 0; j < kCB; ++j) {
            const int col = min(n0 + 16 * j + l16, a.N - 1);
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = min(rbase + 16 * r + v, a.M - 1);
                    rv[j][r][v] = a.R[static_cast<int64_t>(row) * a.ldr + col];
                }
        }
    }
    // a tile inside the matrix stores without per-element bounds checks (a store under a
    // branch would also wait there for the stores before it)
    auto store = [&](auto checked) {
        constexpr bool CK = decltype(checked)::value;
#pragma unroll
        for (int j = 0; j < kCB; ++j) {
            const int col = n0 + 16 * j + l16;
            if (CK && col >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = rbase + 16 * r + v;
                    if (!CK || row < a.M) {
                        float* y = a.Y + static_cast<int64_t>(row) * a.ldy + col;
                        *y = EPI == 1 ? rv[j][r][v] + acc[r][j][v] : acc[r][j][v];
                    }
                }
        }
    };
    if (m0 + kBM <= a.M && n0 + kBN <= a.N) store(std::false_type{});  // uniform
    else store(std::true_type{});
}

template <int EPI, bool F16, bool XP = false>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
    __shared__ __align__(16) uint16_t Ws[2 * kBN][kLd];
    // tile (tx, ty) of workgroup L = x + X y (dispatch order): with a ragged last column
    // tile, its row tiles come first (they are cheaper, so the full tiles fill the rounds
    // behind them instead of a tail of ragged tiles running on a few CUs)
    int tx = blockIdx.x, ty = blockIdx.y;
    if (a.N % kBN != 0) {
        const int nt = gridDim.x, mt = gridDim.y, L = blockIdx.x + nt * blockIdx.y;
        if (L < mt) {
            tx = nt - 1;
            ty = L;
        } else {
            tx = (L - mt) % (nt - 1);
            ty = (L - mt) / (nt - 1);
        }
    }
    // tiles whose W rows all lie inside N (with whole flush blocks of K) store W unmasked
    const bool full = (tx + 1) * kBN <= a.N && a.K % (kFlush * kBK) == 0;
    if (full) gemm_tile<EPI, false, F16, XP>(a, tx, ty, Ws);
    else gemm_tile<EPI, true, F16, XP>(a, tx, ty, Ws);
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    dim3 grid(gemm_col_tiles(a.N), (a.M + kBM - 1) / kBM);
    const bool f16 = a.Wh && a.xmax && a.xmax_n > 0 && a.x_tiled && a.K % 32 == 0;
    // the tiled layouts exist on the two-part path only (Y: its SwiGLU output)
    if ((a.x_tiled && !f16) || (a.y_tiled && !(f16 && a.swiglu && (a.N / 2) % 32 == 0))) return hipErrorInvalidValue;
    if (a.x_planes && !(f16 && a.xmax_n == 1)) return hipErrorInvalidValue;  // the producer's one row maximum
    if (f16 && a.x_planes) {
        if (a.swiglu) klaunch(gemm_kernel<2, true, true>, grid, 256, 0, s, a);
        else if (a.R) klaunch(gemm_kernel<1, true, true>, grid, 256, 0, s, a);
        else klaunch(gemm_kernel<0, true, true>, grid, 256, 0, s, a);
    } else if (f16) {
        if (a.swiglu) klaunch(gemm_kernel<2, true>, grid, 256, 0, s, a);
        else if (a.R) klaunch(gemm_kernel<1, true>, grid, 256, 0, s, a);
        else klaunch(gemm_kernel<0, true>, grid, 256, 0, s, a);
    } else {
        if (a.swiglu) klaunch(gemm_kernel<2, false>, grid, 256, 0, s, a);
        else if (a.R) klaunch(gemm_kernel<1, false>, grid, 256, 0, s, a);
        else klaunch(gemm_kernel<0, false>, grid, 256, 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace q35k
