#pragma once
// Device helpers shared by the gfx950 kernels: 64-lane wavefront reductions, bf16
// widening, the scalar activations of the reference (include/forward_pass.h:21-24).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace q35k {

constexpr int kWave = 64;

// bf16 pair packed in one 32-bit word: element 0 in the low half.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// fp32 -> bf16, round to nearest even (finite inputs)
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }
// x = hi + mid + lo exactly, each a bf16 (returned as its 16-bit pattern): hi = x with its
// low 16 bits cleared, mid the same of the remainder, lo the rest (at most 8 significant
// bits). A product of two bf16 values is exact in fp32, so x * w = hi w + mid w + lo w.
__device__ __forceinline__ void split3(float x, uint32_t& h, uint32_t& m, uint32_t& l) {
    const uint32_t hb = __float_as_uint(x) & 0xffff0000u;
    const float r1 = x - __uint_as_float(hb);
    const uint32_t mb = __float_as_uint(r1) & 0xffff0000u;
    const float r2 = r1 - __uint_as_float(mb);
    h = hb >> 16;
    m = mb >> 16;
    l = __float_as_uint(r2) >> 16;
}

// Wave-wide reductions. Within each row of 16 lanes the partner values move by DPP (quad
// xor 1, quad xor 2, half-row mirror, row mirror: after the four steps every lane holds its
// row's total), the two rows of each half-wave meet through a swizzle (xor 16 within 32
// lanes), and the totals of lanes 0-31 and 32-63 are read as scalars. Partners combine the
// same two values in the same order on both sides, so every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(dpp_i<CTRL>(static_cast<int>(u))),
                   hi = static_cast<uint32_t>(dpp_i<CTRL>(static_cast<int>(u >> 32)));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ float swz16_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ double swz16_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(u), 0x401F)),
                   hi = static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(u >> 32), 0x401F));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double lane_d(double v, int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), l)),
                   hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), l));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad xor 1
    v += dpp_f<0x4E>(v);   // quad xor 2
    v += dpp_f<0x141>(v);  // half-row mirror
    v += dpp_f<0x140>(v);  // row mirror
    v += swz16_f(v);
    return lane_f(v, 0) + lane_f(v, 32);
}
// Sum over each half-wave (lanes 0-31, lanes 32-63), held by every lane of the half.
__device__ __forceinline__ double half_wave_sum(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    return v + swz16_d(v);
}
__device__ __forceinline__ double wave_sum(double v) {
    v = half_wave_sum(v);
    return lane_d(v, 0) + lane_d(v, 32);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, swz16_f(v));
    return fmaxf(lane_f(v, 0), lane_f(v, 32));
}

// silu(x) = x / (1 + e^-x), sigmoid, softplus with the > 20 pass-through.
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// Two-part fp16 form of the prefill GEMM's activations, shared by the GEMM and the kernels
// that write its input already split: the power-of-two exponent that brings a row whose
// largest |x| is mx into [2^14, 2^15) (0 for a zero or non-finite maximum), and for two
// values (already scaled) h = fp16(x), l = fp16(x - h), each pair packed low value first.
__device__ __forceinline__ int split_row_exp(float mx) {
    int ex = 0;
    (void)frexpf(mx, &ex);
    return mx > 0.0f && mx < INFINITY ? min(max(15 - ex, -100), 100) : 0;
}
typedef _Float16 split_h2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split2h_pair(float a, float b, uint32_t& h, uint32_t& l) {
    const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
    const _Float16 la = static_cast<_Float16>(a - static_cast<float>(ha));
    const _Float16 lb = static_cast<_Float16>(b - static_cast<float>(hb));
    h = __builtin_bit_cast(uint32_t, split_h2_t{ha, hb});
    l = __builtin_bit_cast(uint32_t, split_h2_t{la, lb});
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Sum of a double over the whole block (blockDim.x a multiple of 64, <= 1024).
// `red` needs blockDim.x / 64 doubles of LDS. Every thread gets the total.
__device__ __forceinline__ double block_sum(double v, double* red) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// cos / sin (from the double-precision angle pos * theta^(-2i/rot), as the reference's
// apply_rope) of the rotation indices i = (4 lane) mod rot/2 .. + 3 that a lane holding dims
// 4 lane .. 4 lane + 3 of a head needs. Wave-wide (uses lane shuffles): call from all lanes.
__device__ __forceinline__ void rope_cs4(double theta, int rot, int pos, int lane, float4& c4, float4& s4) {
    const int half = rot / 2;
    const int ci = (lane * 4) % (half > 4 ? half : 4);
    auto angle = [&](int i, float& c, float& s) {
        const double inv_freq = pow(theta, -static_cast<double>(2 * i) / rot);
        const double ang = static_cast<double>(pos) * inv_freq;
        c = static_cast<float>(cos(ang));
        s = static_cast<float>(sin(ang));
    };
    if (half <= 64) {  // one angle per lane, then shared
        float cv = 1.0f, sv = 0.0f;
        if (lane < half) angle(lane, cv, sv);
        c4 = make_float4(__shfl(cv, ci), __shfl(cv, ci + 1), __shfl(cv, ci + 2), __shfl(cv, ci + 3));
        s4 = make_float4(__shfl(sv, ci), __shfl(sv, ci + 1), __shfl(sv, ci + 2), __shfl(sv, ci + 3));
    } else {  // wider than 128 rotated dims: each lane its own four
        float cv[4], sv[4];
#pragma unroll 1
        for (int i = 0; i < 4; ++i) angle(ci + i, cv[i], sv[i]);
        c4 = make_float4(cv[0], cv[1], cv[2], cv[3]);
        s4 = make_float4(sv[0], sv[1], sv[2], sv[3]);
    }
}

// Workgroup barrier that orders LDS only: unlike __syncthreads it does not wait for the
// wave's outstanding global loads (a weight stream in flight stays in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// block_sum with LDS-only barriers (for callers that exchange nothing else through memory).
__device__ __forceinline__ double block_sum_lds(double v, double* red) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
    v = wave_sum(v);
    lds_barrier();
    if (lane == 0) red[wave] = v;
    lds_barrier();
    double t = 0.0;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}
// Sum over a 256-thread workgroup, for a single use of `red` per kernel (no barrier before
// the write: nothing read `red` earlier). Every thread gets the total.
__device__ __forceinline__ double block_sum_once_256(double v, double* red) {
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
    lds_barrier();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Counter-based normal draw (splitmix64 finaliser + Box-Muller in double); the same
// formula as the host generator of synthetic checkpoints.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}
__device__ __forceinline__ double normal_at(uint64_t key, uint64_t i) {
    const uint64_t a = mix64(key + 2 * i), b = mix64(key + 2 * i + 1);
    const double u1 = (static_cast<double>(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = static_cast<double>(b >> 11) * (1.0 / 9007199254740992.0);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

}  // namespace q35k
