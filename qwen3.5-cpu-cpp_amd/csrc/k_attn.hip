// Gated GQA attention decode over the fp32 KV cache (QwenModel::attn_step after its
// projections, src/qwen_model.cpp:119-150), in three launches:
//
//   prep     q_norm + RoPE of every query head, k_norm + RoPE of the new key, K/V append
//            at `pos` (rmsnorm (1+w) with the sum of squares in double; RoPE angles in
//            double, src/forward_pass.cpp:77-84,102-112).
//   partial  split-K over the cache: grid (n_splits, NKV). A workgroup owns a contiguous
//            range of positions of one kv head and serves all GRP = NQ/NKV query heads of
//            that group, so each K/V row is read from HBM once per token (the reference
//            re-reads it for every query head). The range is walked in sub-chunks of 32
//            positions; for each sub-chunk every K and V row load is issued up front
//            (16 float4 per lane), then the scores, a running-max softmax update and the
//            P.V accumulation run from registers. Writes the unnormalised partial output
//            and (max, sum) per query head.
//   combine  per query head: merge the splits with the usual max-rescaled sum, divide,
//            multiply by sigmoid(gate).
//
// Scores use LPP lanes per position (16 for GRP <= 4, 32 above), each lane holding
// 256/LPP dims of the query vectors; the GRP partial dots are reduced over the LPP lanes
// with a butterfly that halves the set of values carried at each exchange, ending with
// each lane owning the full dot of one query head. P.V uses 4 dims per lane over all 64
// lanes with the softmax weights broadcast from LDS.
#include <math.h>

#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

constexpr int kHD = 256;
constexpr int kChunk = kAttnChunk;

__device__ __forceinline__ int read_pos(const AttnDecodeArgs& a) {
    return a.pos_dev ? *a.pos_dev : a.pos_val;
}

// Positions per split: ceil(n / n_splits) rounded up to whole sub-chunks.
__device__ __forceinline__ int split_len(int n, int n_splits) {
    const int per = (n + n_splits - 1) / n_splits;
    return ((per + kChunk - 1) / kChunk) * kChunk;
}

__global__ __launch_bounds__(256) void attn_prep_kernel(AttnDecodeArgs a) {
    const int b = blockIdx.x, t = threadIdx.x;
    const int pos = read_pos(a);
    __shared__ float buf[kHD];
    __shared__ double red[4];
    const float* src;
    const float* w;
    float* dst;
    int kh = -1;
    if (b < a.NQ) {
        src = a.qg + static_cast<int64_t>(b) * 2 * kHD;
        w = a.q_norm;
        dst = a.q_work + static_cast<int64_t>(b) * kHD;
    } else {
        kh = b - a.NQ;
        src = a.k_new + static_cast<int64_t>(kh) * kHD;
        w = a.k_norm;
        dst = a.k_cache + (static_cast<int64_t>(kh) * a.max_ctx + pos) * kHD;
    }
    const float x = src[t];
    const double ss = block_sum(static_cast<double>(x) * x, red);
    const float inv = 1.0f / sqrtf(static_cast<float>(ss / kHD) + a.eps);
    float y = x * inv * (1.0f + w[t]);
    buf[t] = y;
    __syncthreads();
    const int half = a.ROT / 2;
    if (t < a.ROT) {
        const int i = t < half ? t : t - half;
        const double inv_freq = pow(a.theta, -static_cast<double>(2 * i) / a.ROT);
        const double ang = static_cast<double>(pos) * inv_freq;
        const float c = static_cast<float>(cos(ang)), s = static_cast<float>(sin(ang));
        const float x1 = buf[i], x2 = buf[i + half];
        y = t < half ? x1 * c - x2 * s : x2 * c + x1 * s;
    }
    dst[t] = y;
    if (kh >= 0)
        a.v_cache[(static_cast<int64_t>(kh) * a.max_ctx + pos) * kHD + t] =
            a.v_new[static_cast<int64_t>(kh) * kHD + t];
}

// Reduce GRP per-lane partial sums over groups of LPP lanes. On return lane l holds in v[0]
// the full sum of query head `head`.
template <int GRP, int LPP>
__device__ __forceinline__ void butterfly(float (&v)[GRP], int lane, int& head) {
    head = 0;
    int cnt = GRP;
#pragma unroll
    for (int o = LPP / 2; o >= 1; o >>= 1) {
        if (cnt > 1) {
            const int half = cnt / 2;
            const bool up = (lane & o) != 0;
#pragma unroll
            for (int i = 0; i < GRP / 2; ++i) {
                if (i < half) {
                    const float send = up ? v[i] : v[i + half];
                    const float keep = up ? v[i + half] : v[i];
                    v[i] = keep + __shfl_xor(send, o);
                }
            }
            if (up) head += half;
            cnt = half;
        } else {
            v[0] += __shfl_xor(v[0], o);
        }
    }
}

template <int GRP, int LPP>
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnDecodeArgs a) {
    constexpr int NF4 = 64 / LPP;            // float4 of one row per lane in the score phase
    constexpr int PPW = 64 / LPP;            // positions per wave per score pass
    constexpr int QIT = kChunk / (4 * PPW);  // score passes per sub-chunk
    constexpr int VIT = kChunk / 4;          // P.V rows per wave per sub-chunk
    constexpr int OWN = LPP / GRP;           // lanes sharing one head after the butterfly
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, kh = blockIdx.y;
    const int n = read_pos(a) + 1;
    const int per = split_len(n, a.n_splits);
    const int j0 = split * per;
    if (j0 >= n) return;
    const int j1 = min(n, j0 + per);

    const float* K = a.k_cache + static_cast<int64_t>(kh) * a.max_ctx * kHD;
    const float* V = a.v_cache + static_cast<int64_t>(kh) * a.max_ctx * kHD;
    const float* Q = a.q_work + static_cast<int64_t>(kh) * GRP * kHD;
    const float sc = 1.0f / sqrtf(static_cast<float>(kHD));

    __shared__ float s_l[kChunk][GRP];
    __shared__ float m_s[GRP], l_s[GRP], f_s[GRP];
    __shared__ float red[GRP][kHD];

    const int pl = lane % LPP, sub = lane / LPP;
    float4 qr[GRP][NF4];
#pragma unroll
    for (int h = 0; h < GRP; ++h)
#pragma unroll
        for (int m = 0; m < NF4; ++m)
            qr[h][m] = *reinterpret_cast<const float4*>(Q + h * kHD + pl * 4 + m * LPP * 4);
    if (tid < GRP) {
        m_s[tid] = -INFINITY;
        l_s[tid] = 0.0f;
    }
    float4 acc[GRP];
#pragma unroll
    for (int h = 0; h < GRP; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);

    for (int c0 = j0; c0 < j1; c0 += kChunk) {
        const int cn = min(kChunk, j1 - c0);
        float4 kr[QIT][NF4];
        float4 vr[VIT];
#pragma unroll
        for (int it = 0; it < QIT; ++it) {
            const int jl = it * 4 * PPW + wave * PPW + sub;
            const float* row = K + static_cast<int64_t>(c0 + min(jl, cn - 1)) * kHD + pl * 4;
#pragma unroll
            for (int m = 0; m < NF4; ++m) kr[it][m] = *reinterpret_cast<const float4*>(row + m * LPP * 4);
        }
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
            const int jl = it * 4 + wave;
            vr[it] = *reinterpret_cast<const float4*>(V + static_cast<int64_t>(c0 + min(jl, cn - 1)) * kHD + lane * 4);
        }
        // scores
#pragma unroll
        for (int it = 0; it < QIT; ++it) {
            const int jl = it * 4 * PPW + wave * PPW + sub;
            float p[GRP];
#pragma unroll
            for (int h = 0; h < GRP; ++h) {
                float t = 0.0f;
#pragma unroll
                for (int m = 0; m < NF4; ++m) {
                    t = fmaf(qr[h][m].x, kr[it][m].x, t);
                    t = fmaf(qr[h][m].y, kr[it][m].y, t);
                    t = fmaf(qr[h][m].z, kr[it][m].z, t);
                    t = fmaf(qr[h][m].w, kr[it][m].w, t);
                }
                p[h] = t;
            }
            int head;
            butterfly<GRP, LPP>(p, lane, head);
            if ((pl % OWN) == 0) s_l[jl][head] = jl < cn ? p[0] * sc : -INFINITY;
        }
        __syncthreads();
        // running-max softmax update, one wave per query head
        for (int h = wave; h < GRP; h += 4) {
            const float v = lane < kChunk ? s_l[lane][h] : -INFINITY;
            const float cmax = wave_max(v);
            const float m_old = m_s[h];
            const float m_new = fmaxf(m_old, cmax);
            const float e = (lane < kChunk && lane < cn) ? expf(v - m_new) : 0.0f;
            if (lane < kChunk) s_l[lane][h] = e;
            const float es = wave_sum(e);
            if (lane == 0) {
                const float f = expf(m_old - m_new);
                f_s[h] = f;
                m_s[h] = m_new;
                l_s[h] = l_s[h] * f + es;
            }
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < GRP; ++h) {
            const float f = f_s[h];
            acc[h].x *= f;
            acc[h].y *= f;
            acc[h].z *= f;
            acc[h].w *= f;
        }
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
            const int jl = it * 4 + wave;
#pragma unroll
            for (int h = 0; h < GRP; ++h) {
                const float e = s_l[jl][h];
                acc[h].x = fmaf(e, vr[it].x, acc[h].x);
                acc[h].y = fmaf(e, vr[it].y, acc[h].y);
                acc[h].z = fmaf(e, vr[it].z, acc[h].z);
                acc[h].w = fmaf(e, vr[it].w, acc[h].w);
            }
        }
        __syncthreads();
    }
    // fixed-order cross-wave sum of the P.V accumulators
    for (int w = 0; w < 4; ++w) {
        if (wave == w) {
#pragma unroll
            for (int h = 0; h < GRP; ++h) {
                float4* r = reinterpret_cast<float4*>(&red[h][lane * 4]);
                if (w == 0) {
                    *r = acc[h];
                } else {
                    float4 t = *r;
                    t.x += acc[h].x;
                    t.y += acc[h].y;
                    t.z += acc[h].z;
                    t.w += acc[h].w;
                    *r = t;
                }
            }
        }
        __syncthreads();
    }
    const int64_t base = (static_cast<int64_t>(kh) * a.n_splits + split) * GRP;
#pragma unroll
    for (int h = 0; h < GRP; ++h) a.part_o[(base + h) * kHD + tid] = red[h][tid];
    if (tid < GRP) {
        a.part_ml[(base + tid) * 2] = m_s[tid];
        a.part_ml[(base + tid) * 2 + 1] = l_s[tid];
    }
}

__global__ __launch_bounds__(256) void attn_combine_kernel(AttnDecodeArgs a) {
    const int h = blockIdx.x, t = threadIdx.x;
    const int grp = a.NQ / a.NKV, kh = h / grp, g = h - kh * grp;
    const int n = read_pos(a) + 1;
    const int per = split_len(n, a.n_splits);
    const int nact = (n + per - 1) / per;
    extern __shared__ float w_s[];
    __shared__ float redf[4];
    const int64_t base = static_cast<int64_t>(kh) * a.n_splits * grp + g;
    float mx = -INFINITY;
    for (int s = t; s < nact; s += 256) mx = fmaxf(mx, a.part_ml[(base + static_cast<int64_t>(s) * grp) * 2]);
    mx = wave_max(mx);
    if ((t & 63) == 0) redf[t >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
    __syncthreads();
    for (int s = t; s < nact; s += 256) {
        const float* ml = a.part_ml + (base + static_cast<int64_t>(s) * grp) * 2;
        const float w = expf(ml[0] - M);
        w_s[s] = w;
        w_s[a.n_splits + s] = ml[1] * w;
    }
    __syncthreads();
    float L = 0.0f, o = 0.0f;
    for (int s = 0; s < nact; ++s) {
        L += w_s[a.n_splits + s];
        o = fmaf(a.part_o[(base + static_cast<int64_t>(s) * grp) * kHD + t], w_s[s], o);
    }
    const float gate = a.qg[static_cast<int64_t>(h) * 2 * kHD + kHD + t];
    a.out[static_cast<int64_t>(h) * kHD + t] = (o / L) * sigmoid_f(gate);
}

template <int GRP>
hipError_t launch_partial_grp(const AttnDecodeArgs& a, hipStream_t s) {
    constexpr int LPP = GRP <= 4 ? 16 : 32;
    dim3 grid(a.n_splits, a.NKV);
    attn_partial_kernel<GRP, LPP><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_prep(const AttnDecodeArgs& a, hipStream_t s) {
    attn_prep_kernel<<<a.NQ + a.NKV, kHD, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_attn_partial(const AttnDecodeArgs& a, hipStream_t s) {
    switch (a.NQ / a.NKV) {
        case 1: return launch_partial_grp<1>(a, s);
        case 2: return launch_partial_grp<2>(a, s);
        case 4: return launch_partial_grp<4>(a, s);
        case 8: return launch_partial_grp<8>(a, s);
        case 16: return launch_partial_grp<16>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_combine(const AttnDecodeArgs& a, hipStream_t s) {
    const size_t lds = static_cast<size_t>(a.n_splits) * 2 * sizeof(float);
    attn_combine_kernel<<<a.NQ, kHD, lds, s>>>(a);
    return hipGetLastError();
}

}  // namespace q35k
