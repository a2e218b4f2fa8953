// bf16-weight x fp32-activation matvec for every projection of the decode step
// (the reference's matmul(WeightView), src/forward_pass.cpp:44-75), with the elementwise
// work that feeds or follows each projection fused in:
//   prologue  rmsnorm (1+w)       input_layernorm / post_attention_layernorm / final norm;
//                                 the first layer's input can be the token's bf16 embedding
//                                 row (SafeTensors::get_row_f32, src/safetensors_loader.cpp:
//                                 280-298), which workgroup 0 also stores as the residual
//             silu(g) * u         SwiGLU of a [gate | up] input vector
//             gated rmsnorm        GDN rmsnorm_gated before linear_attn.out_proj
//   epilogue  y = resid + W x     residual add of the mixer / FFN output
//             silu(y_2i) y_2i+1   SwiGLU of the interleaved gate / up projection (the
//                                 down_proj matvec then reads silu(gate) * up directly)
//             conv + SiLU          GDN in-projection: each conv channel's causal window
//                                 (QwenModel::gdn_step's conv, src/qwen_model.cpp:173-186)
//                                 runs once, in the wave that produced the channel, instead
//                                 of in every mixer workgroup that reads it
//             argmax partials      output head: each workgroup's largest logit and its row
//                                 (first of equal values), the greedy pick's first pass
//
// HBM-bound: every weight byte is read exactly once per step. A 256-thread workgroup
// stages the transformed input vector in LDS once, then each 64-lane wave streams RPW
// weight rows at a time with 16-byte loads (8 bf16 per lane, 1 KiB per wave per row and
// chunk), issuing up to 4 chunks of loads before consuming them. The first row group's
// loads are issued before the prologue, which they do not depend on, so the HBM latency
// overlaps the input staging (its barriers order LDS only, so they do not wait for the
// weights in flight). bf16 is widened exactly (shift into the upper half of an
// fp32) and accumulated in fp32 FMA; the 64 lane partials are summed with a butterfly.
#include <climits>
#include <cmath>
#include <cstdlib>

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

// 4 consecutive bf16 embedding elements, widened exactly
__device__ __forceinline__ float4 embed4(const uint16_t* row, int i) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + i);
    return make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
}

template <int PRO>
__device__ __forceinline__ void stage_input(const GemvArgs& a, const uint16_t* erow, float* xs) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = a.in_dim;
    __shared__ double red[4];
    __shared__ float head_inv[64];
    if (PRO == kProRmsNorm && erow) {
        for (int i = tid * 4; i < n; i += 1024) {
            const float4 v = embed4(erow, i);
            *reinterpret_cast<float4*>(xs + i) = v;
            if (a.x_out && blockIdx.x == 0) *reinterpret_cast<float4*>(a.x_out + i) = v;
        }
        lds_barrier();  // the sum of squares below reads the staged row
    } else if (PRO == kProSwiGlu) {
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
            const double v = erow ? xs[i] : a.x[i];
            ss += v * v;
        }
        ss = block_sum_lds(ss, red);
        const float inv = 1.0f / sqrtf(static_cast<float>(ss / n) + a.eps);
        lds_barrier();
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
        lds_barrier();
        for (int i = tid; i < n; i += 256) {
            const int h = i / hd;
            xs[i] = a.norm_w[i - h * hd] * (xs[i] * head_inv[h]) * silu_f(a.gate[i]);
        }
    }
    lds_barrier();
}

// Number of 512-element chunks prefetched for the first row group: all KC of them when the
// width is known at compile time (KC > 0), else the first 4.
constexpr int pf_chunks(int KC) { return KC > 0 ? KC : 4; }

// Loads the first row group's chunks (the part that can be in flight before the input).
template <int RPW, int KC>
__device__ __forceinline__ void load_rows(const GemvArgs& a, int r0, u32x4 (&w)[pf_chunks(KC)][RPW]) {
    const int lane = threadIdx.x & 63, n = a.in_dim, nfull = n >> 9;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint16_t* p = a.W + static_cast<size_t>(min(r0 + r, a.rows - 1)) * n + lane * 8;
#pragma unroll
        for (int u = 0; u < pf_chunks(KC); ++u)
            if (KC > 0 || u < nfull) w[u][r] = load_w(p + (u << 9));
    }
}

// Epilogue inputs of a wave's rows, requested with the rows' weights so that the epilogue
// does not wait for them: the conv window (kEpiConvSilu: the four taps and the raw inputs of
// the three previous positions, ring slots (pos - 3..pos - 1) % 4) or the residual
// (kEpiResidual; y may be the residual itself, and each row is read here before its own
// write).
template <int RPW>
struct ConvIn {
    float4 w[RPW];
    float r3[RPW], r2[RPW], r1[RPW];
    float res[RPW];
};

template <int RPW>
__device__ __forceinline__ void load_resid(const GemvArgs& a, int r0, ConvIn<RPW>& cv) {
#pragma unroll
    for (int r = 0; r < RPW; ++r) cv.res[r] = a.resid[min(r0 + r, a.rows - 1)];
}

template <int RPW>
__device__ __forceinline__ void load_conv(const GemvArgs& a, int r0, int pos, ConvIn<RPW>& cv) {
    const int n = a.conv_rows;
    const int64_t s3 = (pos + 1) & 3, s2 = (pos + 2) & 3, s1 = (pos + 3) & 3;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t ch = min(r0 + r, n - 1);  // rows past the conv channels: unused
        cv.w[r] = *reinterpret_cast<const float4*>(a.conv_w + ch * 4);
        cv.r3[r] = a.conv_ring[s3 * n + ch];
        cv.r2[r] = a.conv_ring[s2 * n + ch];
        cv.r1[r] = a.conv_ring[s1 * n + ch];
    }
}

// (value, row) order of the argmax partials: larger value first, then the smaller row
__device__ __forceinline__ bool amax_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

template <int EPI, int RPW>
__device__ __forceinline__ void store_rows(const GemvArgs& a, int r0, const float (&acc)[RPW],
                                           const ConvIn<RPW>& cv, int pos, float& bv, int& bi) {
    const int lane = threadIdx.x & 63;
    float sum[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) sum[r] = wave_sum(acc[r]);
    if (EPI == kEpiStore && a.amax_part) {  // the sums are uniform: every lane tracks them
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (r0 + r < a.rows && amax_better(sum[r], r0 + r, bv, bi)) {
                bv = sum[r];
                bi = r0 + r;
            }
    }
    if (lane != 0) return;
    if (EPI == kEpiConvSilu) {
        // taps oldest first, the raw projection as the newest input; the raw value goes to
        // the ring slot of this position (read by the next three steps)
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = r0 + r;
            if (row >= a.rows) continue;
            if (row < a.conv_rows) {
                float c = 0.0f;
                c += cv.w[r].x * cv.r3[r];
                c += cv.w[r].y * cv.r2[r];
                c += cv.w[r].z * cv.r1[r];
                c += cv.w[r].w * sum[r];
                a.y[row] = silu_f(c);
                a.conv_ring[static_cast<int64_t>(pos & 3) * a.conv_rows + row] = sum[r];
            } else {
                a.y[row] = sum[r];
            }
        }
        return;
    }
    if (EPI == kEpiSwiGluPair) {
        // rows (2i, 2i + 1) = (gate_i, up_i) of the interleaved [gate|up] matrix
        if (r0 + 1 < a.rows) a.y[r0 >> 1] = silu_f(sum[0]) * sum[RPW - 1];
    } else {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (r0 + r < a.rows) a.y[r0 + r] = EPI == kEpiResidual ? cv.res[r] + sum[r] : sum[r];
    }
}

// RPW consecutive rows of one wave from `r0`. With PF the first pf_chunks(KC) chunks come
// from `pf` (loaded before the input prologue). With KC > 0 the width is KC * 512 and every
// chunk of the group is in flight at once.
template <int EPI, int RPW, int KC, bool PF>
__device__ __forceinline__ void row_group(const GemvArgs& a, const float* xs, int r0,
                                          const u32x4 (&pf)[pf_chunks(KC)][RPW], const ConvIn<RPW>& cv,
                                          int pos, float& bv, int& bi) {
    const int lane = threadIdx.x & 63;
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
    if (KC > 0) {
        u32x4 w[pf_chunks(KC)][RPW];
        if (PF) {
#pragma unroll
            for (int u = 0; u < pf_chunks(KC); ++u)
#pragma unroll
                for (int r = 0; r < RPW; ++r) w[u][r] = pf[u][r];
        } else {
            load_rows<RPW, KC>(a, r0, w);
        }
#pragma unroll
        for (int u = 0; u < pf_chunks(KC); ++u) {
            const int c = (u << 9) + lane * 8;
            const float4 x0 = *reinterpret_cast<const float4*>(xs + c);
            const float4 x1 = *reinterpret_cast<const float4*>(xs + c + 4);
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[r] = dot8(w[u][r], x0, x1, acc[r]);
        }
        store_rows<EPI, RPW>(a, r0, acc, cv, pos, bv, bi);
        return;
    }
    const int n = a.in_dim;
    const int nfull = n >> 9;           // 512-element chunks: 64 lanes x 8
    const int tail = n - (nfull << 9);  // multiple of 8
    const uint16_t* wr[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) wr[r] = a.W + static_cast<size_t>(min(r0 + r, a.rows - 1)) * n + lane * 8;
    int k = 0;
    if (PF) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (u < nfull) {
                const int c = (u << 9) + lane * 8;
                const float4 x0 = *reinterpret_cast<const float4*>(xs + c);
                const float4 x1 = *reinterpret_cast<const float4*>(xs + c + 4);
#pragma unroll
                for (int r = 0; r < RPW; ++r) acc[r] = dot8(pf[u][r], x0, x1, acc[r]);
            }
        }
        k = min(nfull, 4);
    }
    for (; k + 4 <= nfull; k += 4) {
        u32x4 w[4][RPW];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < RPW; ++r) w[u][r] = load_w(wr[r] + ((k + u) << 9));
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
    store_rows<EPI, RPW>(a, r0, acc, cv, pos, bv, bi);
}

// Input staged through registers (n <= 1024 NX): the input loads are issued first, then
// the first row group's weight loads, then the prologue arithmetic. Loads complete in
// order for the wait counter, so issuing the input first lets the prologue wait for the
// input alone while the weights are still in flight.
template <int PRO, int NX>
__device__ __forceinline__ void load_input(const GemvArgs& a, const uint16_t* erow, float4 (&xv)[NX],
                                           uint2 (&xe)[NX], float4 (&gv)[NX], float4 (&wv)[NX]) {
    const int tid = threadIdx.x, n = a.in_dim;
    // Unconditional loads (indices clamped into the vector, surplus lanes masked later): a
    // load under a branch makes the wait-count insertion fall back to waiting for every
    // outstanding load, the weight prefetch included. (`erow` is uniform over the grid; the
    // embedding's bf16 elements are widened in finish_input, so nothing here waits for them.)
#pragma unroll
    for (int j = 0; j < NX; ++j) {
        const int i = min((tid + j * 256) * 4, n - 4);
        if (PRO == kProRmsNorm && erow) xe[j] = *reinterpret_cast<const uint2*>(erow + i);
        else xv[j] = *reinterpret_cast<const float4*>(a.x + i);
        if (PRO == kProRmsNorm) wv[j] = *reinterpret_cast<const float4*>(a.norm_w + i);
        if (PRO == kProGatedNorm) {
            gv[j] = *reinterpret_cast<const float4*>(a.gate + i);
            wv[j] = *reinterpret_cast<const float4*>(a.norm_w + i % a.head_dim);
        }
    }
}

template <int PRO, int NX>
__device__ __forceinline__ void finish_input(const GemvArgs& a, const uint16_t* erow, float4 (&xv)[NX],
                                             const uint2 (&xe)[NX], const float4 (&gv)[NX],
                                             const float4 (&wv)[NX], float* xs) {
    const int tid = threadIdx.x, n = a.in_dim;
    __shared__ double red[4];
    if (PRO == kProRmsNorm && erow) {
#pragma unroll
        for (int j = 0; j < NX; ++j)
            xv[j] = make_float4(bf16_lo(xe[j].x), bf16_hi(xe[j].x), bf16_lo(xe[j].y), bf16_hi(xe[j].y));
    }
    // Every use below is unconditional (slots past the input are zeroed by a select and
    // stored to the spare slot xs[n .. n+3]): a use under a branch lets the compiler sink
    // the input loads behind the weight loads, and then staging waits for all of them.
#pragma unroll
    for (int j = 0; j < NX; ++j)
        if ((tid + j * 256) * 4 >= n) xv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (PRO == kProRmsNorm && a.x_out && blockIdx.x == 0) {  // the embedding row, as read
#pragma unroll
        for (int j = 0; j < NX; ++j)
            if ((tid + j * 256) * 4 < n) *reinterpret_cast<float4*>(a.x_out + (tid + j * 256) * 4) = xv[j];
    }
    if (PRO == kProRmsNorm) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < NX; ++j)
            ss += static_cast<double>(xv[j].x) * xv[j].x + static_cast<double>(xv[j].y) * xv[j].y +
                  static_cast<double>(xv[j].z) * xv[j].z + static_cast<double>(xv[j].w) * xv[j].w;
        ss = block_sum_once_256(ss, red);
        const float inv = 1.0f / sqrtf(static_cast<float>(ss / n) + a.eps);
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            xv[j].x = xv[j].x * inv * (1.0f + wv[j].x);
            xv[j].y = xv[j].y * inv * (1.0f + wv[j].y);
            xv[j].z = xv[j].z * inv * (1.0f + wv[j].z);
            xv[j].w = xv[j].w * inv * (1.0f + wv[j].w);
        }
    }
    if (PRO == kProGatedNorm) {
        // head_dim == 128: a head is 32 consecutive threads' float4s (half a wave)
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            double ss = static_cast<double>(xv[j].x) * xv[j].x + static_cast<double>(xv[j].y) * xv[j].y +
                        static_cast<double>(xv[j].z) * xv[j].z + static_cast<double>(xv[j].w) * xv[j].w;
            ss = half_wave_sum(ss);
            const float inv = 1.0f / sqrtf(static_cast<float>(ss / a.head_dim) + a.eps);
            xv[j].x = wv[j].x * (xv[j].x * inv) * silu_f(gv[j].x);
            xv[j].y = wv[j].y * (xv[j].y * inv) * silu_f(gv[j].y);
            xv[j].z = wv[j].z * (xv[j].z * inv) * silu_f(gv[j].z);
            xv[j].w = wv[j].w * (xv[j].w * inv) * silu_f(gv[j].w);
        }
    }
#pragma unroll
    for (int j = 0; j < NX; ++j) {
        const int i = (tid + j * 256) * 4;
        *reinterpret_cast<float4*>(xs + min(i, n)) = xv[j];
    }
    lds_barrier();
}

// The fields the first loads need come first as separate arguments: the library is built
// with kernarg preloading for them (k_gemv's build line), so the CP hands them over in
// SGPRs at wave launch and the input and weight loads do not wait for a kernarg load.
template <int PRO, int EPI, int RPW, int NX, int KC>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* W, const float* x, const float* norm_w,
                                                   const float* gate, const uint16_t* embed, int rows,
                                                   GemvArgs a) {
    a.W = W;
    a.x = x;
    a.norm_w = norm_w;
    a.gate = gate;
    a.embed = embed;
    a.rows = rows;
    // constants of this instantiation (the dispatch picks KC = in_dim / 512, and register
    // staging of the gated norm only for 128-wide heads)
    if (KC > 0) a.in_dim = KC * 512;
    if (PRO == kProGatedNorm && NX > 0) a.head_dim = 128;
    extern __shared__ float xs[];
    const int wave = threadIdx.x >> 6;
    const int row_step = gridDim.x * 4 * RPW;
    int r0 = (blockIdx.x * 4 + wave) * RPW;
    // the position and the token first (scalar loads: the ring and embedding loads below
    // depend on them, and waiting for them must not wait for the vector loads)
    const int pos = EPI == kEpiConvSilu ? *a.pos_dev : 0;
    const uint16_t* erow = PRO == kProRmsNorm && a.embed ? a.embed + static_cast<int64_t>(*a.token) * a.in_dim : nullptr;
    float4 xv[NX > 0 ? NX : 1], gv[NX > 0 ? NX : 1], wv[NX > 0 ? NX : 1];
    uint2 xe[NX > 0 ? NX : 1];
    if (NX > 0) load_input<PRO>(a, erow, xv, xe, gv, wv);
    // The first row group's weights do not depend on the input: their loads are in flight
    // while the prologue works.
    u32x4 pf[pf_chunks(KC)][RPW];
    load_rows<RPW, KC>(a, r0, pf);  // rows clamped: unconditional, see load_input
    // nothing after this point is scheduled before the weight loads (a wait for a kernarg
    // loaded later, e.g. the residual's pointer, would hold them back)
    __builtin_amdgcn_sched_barrier(0);
    ConvIn<RPW> cv;
    if (EPI == kEpiConvSilu) load_conv<RPW>(a, r0, pos, cv);
    if (EPI == kEpiResidual) load_resid<RPW>(a, r0, cv);
    if (NX > 0) finish_input<PRO>(a, erow, xv, xe, gv, wv, xs);
    else stage_input<PRO>(a, erow, xs);
    float bv = -INFINITY;  // argmax partial of this wave's rows (amax_part)
    int bi = INT_MAX;
    if (r0 < a.rows) {
        if (KC > 0) {
            // one register set: compute the group in `pf`, then load the next one into it
            for (;;) {
                row_group<EPI, RPW, KC, true>(a, xs, r0, pf, cv, pos, bv, bi);
                r0 += row_step;
                if (r0 >= a.rows) break;
                load_rows<RPW, KC>(a, r0, pf);
                if (EPI == kEpiConvSilu) load_conv<RPW>(a, r0, pos, cv);
                if (EPI == kEpiResidual) load_resid<RPW>(a, r0, cv);
            }
        } else {
            row_group<EPI, RPW, KC, true>(a, xs, r0, pf, cv, pos, bv, bi);
            for (r0 += row_step; r0 < a.rows; r0 += row_step) {
                if (EPI == kEpiConvSilu) load_conv<RPW>(a, r0, pos, cv);
                if (EPI == kEpiResidual) load_resid<RPW>(a, r0, cv);
                row_group<EPI, RPW, KC, false>(a, xs, r0, pf, cv, pos, bv, bi);
            }
        }
    }
    if (EPI == kEpiStore && a.amax_part) {  // uniform over the grid
        __shared__ float sv[4];
        __shared__ int si[4];
        if ((threadIdx.x & 63) == 0) {
            sv[wave] = bv;
            si[wave] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float v = sv[0];
            int i = si[0];
            for (int w = 1; w < 4; ++w)
                if (amax_better(sv[w], si[w], v, i)) {
                    v = sv[w];
                    i = si[w];
                }
            a.amax_part[blockIdx.x] = v;
            reinterpret_cast<int*>(a.amax_part + gridDim.x)[blockIdx.x] = i;
        }
    }
}

int gemv_max_blocks() {
    static const int v = [] {
        const char* e = getenv("Q35_GEMV_MAX_BLOCKS");
        const int x = e ? atoi(e) : 0;
        return x > 0 ? x : 2048;
    }();
    return v;
}

bool gemv_two_rows(int rows, int epilogue) { return epilogue == kEpiSwiGluPair || rows >= 8192; }

template <int PRO, int EPI, int NX, int KC>
hipError_t launch_kc(const GemvArgs& a, hipStream_t s) {
    const size_t lds = static_cast<size_t>(a.in_dim + 4) * sizeof(float);  // + the spare slot
    const int blocks = gemv_blocks(a, EPI);
    if (gemv_two_rows(a.rows, EPI))
        klaunch(gemv_kernel<PRO, EPI, 2, NX, KC>, blocks, 256, lds, s, a.W, a.x, a.norm_w, a.gate, a.embed, a.rows,
                a);
    else
        klaunch(gemv_kernel<PRO, EPI, 1, NX, KC>, blocks, 256, lds, s, a.W, a.x, a.norm_w, a.gate, a.embed, a.rows,
                a);
    return hipGetLastError();
}

// Widths of the model (2048, 4096, 6144) get compile-time chunk counts; the input is
// staged through registers for widths up to 2048 (the SwiGLU prologue, whose input is
// twice as wide, and wider inputs stage through LDS directly).
template <int PRO, int EPI>
hipError_t launch_rpw(const GemvArgs& a, hipStream_t s) {
    const bool gated_ok = PRO != kProGatedNorm || a.head_dim == 128;
    if (PRO != kProSwiGlu) {
        if (a.in_dim == 2048 && gated_ok) return launch_kc<PRO, EPI, 2, 4>(a, s);
        if (a.in_dim == 4096 && gated_ok) return launch_kc<PRO, EPI, 4, 8>(a, s);
        if (a.in_dim == 6144 && gated_ok) return launch_kc<PRO, EPI, 6, 12>(a, s);
        if (a.in_dim <= 2048 && gated_ok) return launch_kc<PRO, EPI, 2, 0>(a, s);
    }
    return launch_kc<PRO, EPI, 0, 0>(a, s);
}

template <int PRO>
hipError_t launch_pro(const GemvArgs& a, int epi, hipStream_t s) {
    if (epi == kEpiSwiGluPair) return launch_rpw<PRO, kEpiSwiGluPair>(a, s);
    if (epi == kEpiConvSilu) {
        if (PRO != kProRmsNorm || !a.conv_w || !a.conv_ring || !a.pos_dev || a.conv_rows <= 0 || a.conv_rows > a.rows)
            return hipErrorInvalidValue;
        return launch_rpw<kProRmsNorm, kEpiConvSilu>(a, s);
    }
    return a.resid ? launch_rpw<PRO, kEpiResidual>(a, s) : launch_rpw<PRO, kEpiStore>(a, s);
}

template <int PRO, int EPI>
hipError_t allow_wide() {
    const int bytes = (kGemvMaxIn + 4) * static_cast<int>(sizeof(float));
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<PRO, EPI, 1, 0, 0>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<PRO, EPI, 2, 0, 0>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    return e;
}

template <int PRO>
hipError_t allow_wide_pro() {
    hipError_t e = allow_wide<PRO, kEpiStore>();
    if (e == hipSuccess) e = allow_wide<PRO, kEpiResidual>();
    if (e == hipSuccess) e = allow_wide<PRO, kEpiSwiGluPair>();
    if (e == hipSuccess && PRO == kProRmsNorm) e = allow_wide<kProRmsNorm, kEpiConvSilu>();
    return e;
}

}  // namespace

hipError_t gemv_enable_wide_inputs() {
    static const hipError_t e = [] {
        hipError_t r = allow_wide_pro<kProPlain>();
        if (r == hipSuccess) r = allow_wide_pro<kProRmsNorm>();
        if (r == hipSuccess) r = allow_wide_pro<kProSwiGlu>();
        if (r == hipSuccess) r = allow_wide_pro<kProGatedNorm>();
        return r;
    }();
    return e;
}

int gemv_blocks(const GemvArgs& a, int epilogue) {
    if (epilogue == kEpiAuto) epilogue = a.resid ? kEpiResidual : kEpiStore;
    const int per = gemv_two_rows(a.rows, epilogue) ? 8 : 4;  // rows per workgroup and group
    const int blocks = min(gemv_max_blocks(), (a.rows + per - 1) / per);
    return a.amax_part ? min(blocks, kArgmaxParts) : blocks;
}

hipError_t launch_gemv(const GemvArgs& a, int prologue, hipStream_t s, int epilogue) {
    if ((a.embed && (prologue != kProRmsNorm || !a.token)) ||
        (a.amax_part && !(epilogue == kEpiStore || (epilogue == kEpiAuto && !a.resid))))
        return hipErrorInvalidValue;
    switch (prologue) {
        case kProPlain: return launch_pro<kProPlain>(a, epilogue, s);
        case kProRmsNorm: return launch_pro<kProRmsNorm>(a, epilogue, s);
        case kProSwiGlu: return launch_pro<kProSwiGlu>(a, epilogue, s);
        case kProGatedNorm: return launch_pro<kProGatedNorm>(a, epilogue, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace q35k
