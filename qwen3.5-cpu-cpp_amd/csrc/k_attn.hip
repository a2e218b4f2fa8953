// Gated GQA attention decode over the fp32 KV cache (QwenModel::attn_step after its
// projections, src/qwen_model.cpp:119-150), in two launches:
//
//   partial  split-K over the cache, grid (n_splits, NKV), 8 waves per workgroup. A
//            workgroup owns a contiguous range of positions of one kv head and serves all
//            GRP = NQ/NKV query heads of the group, so each K/V row is read from HBM once per
//            token (the reference re-reads it for every query head). Prologue: rmsnorm (1+w)
//            + RoPE of its GRP query rows (sum of squares and rotation angles in double,
//            src/forward_pass.cpp:77-84,102-112); the workgroup holding position `pos` also
//            norms + rotates the new key and appends the K/V rows. Each wave then walks its
//            own sub-range in batches with no block barrier: the next batch's K and V rows
//            are requested before the current one is consumed (register double buffer), the
//            scores use LPP lanes per position (16 for GRP <= 4, 32 above) with the GRP partial
//            dots reduced by a butterfly that halves the carried set at each exchange, the
//            running max and sum of each head live in the lanes that own that head, and P.V
//            (4 dims per lane) takes each softmax weight as a scalar operand read from its
//            lane. The waves are merged once at the end (max-rescaled, fixed order).
//            Output: unnormalised partial output and (max, sum) per query head and split.
//            The cache holds fp32 or bf16 elements (bf16: rows rounded to nearest even when
//            appended, widened exactly when read).
//   combine  grid (NQ, HD/64): merges the splits with max-rescaled sums (the splits are
//            shared over the 4 waves, one dim per lane), divides, multiplies by
//            sigmoid(gate).
#include <math.h>

#include <cstdlib>
#include <type_traits>

#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

constexpr int kHD = 256;

__device__ __forceinline__ int read_pos(const AttnDecodeArgs& a) {
    return a.pos_dev ? *a.pos_dev : a.pos_val;
}

// The matrix-core decode kernels take the position and the pointers of their first loads as
// leading arguments, preloaded into SGPRs at wave launch (k_attn's build line): the
// position (device pointer and value), the query rows, the appended key / value and the two
// norm weights; they request the query-side rows before anything that depends on the
// position. The combine takes the position, the partials, the gate rows and the split and
// head counts.
__device__ __forceinline__ void set_lead(AttnDecodeArgs& a, const int* pos_dev, int pos_val, const float* qg,
                                         const float* k_new, const float* v_new, const float* q_norm,
                                         const float* k_norm) {
    a.pos_dev = pos_dev;
    a.pos_val = pos_val;
    a.qg = qg;
    a.k_new = k_new;
    a.v_new = v_new;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
}

__device__ __forceinline__ int split_len(int n, int n_splits) { return (n + n_splits - 1) / n_splits; }

// Reduce GRP per-lane partial sums over groups of LPP lanes. On return lane l holds in v[0]
// the full sum of query head `head`.
// Value of the partner lane of the butterfly stage on lane bit `o`. The partner differs
// from this lane in bit o (and for o = 4, 8 also in the lower bits: the half-row and row
// mirrors i <-> 7-i, i <-> 15-i); the pairings of the five stages (xor 16, 15, 7, 2, 1)
// span all 32 lanes of a group, so the butterfly still sums every lane exactly once.
// DPP and swizzle move data without the address arithmetic of a generic shuffle.
__device__ __forceinline__ float xchg(float v, int o) {
    const int x = __builtin_bit_cast(int, v);
    int r;
    switch (o) {
        case 1: r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); break;   // quad xor 1
        case 2: r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); break;   // quad xor 2
        case 4: r = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false); break;  // half-row mirror
        case 8: r = __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false); break;  // row mirror
        case 16: r = __builtin_amdgcn_ds_swizzle(x, 0x401F); break;                      // xor 16 in 32
        default: r = __builtin_bit_cast(int, __shfl_xor(v, o)); break;
    }
    return __builtin_bit_cast(float, r);
}

template <int N>
using fvec = float __attribute__((ext_vector_type(N)));

// Halving butterfly over lane bits O, O/2, ..., 1 (O = LPP / 2): each lane starts with the
// partial dots of N query heads; at each stage the lane keeps the half of the heads its
// bit selects, adds the partner's partials of that half and sends the other half. After
// log2(N) stages a lane holds one head (bits of the lane give its index), the remaining
// stages finish the sum over the LPP lanes. The halves are whole vectors selected by a
// scalar condition, so no per-element dynamic indexing is generated.
template <int N, int O>
__device__ __forceinline__ float butterfly(fvec<N> v, int lane) {
    if constexpr (O == 0) {
        return v[0];
    } else if constexpr (N == 1) {
        fvec<1> t;
        t[0] = v[0] + xchg(v[0], O);
        return butterfly<1, O / 2>(t, lane);
    } else {
        const bool up = (lane & O) != 0;
        const fvec<N / 2> lo = v.lo, hi = v.hi;
        const fvec<N / 2> send = up ? lo : hi;
        const fvec<N / 2> keep = up ? hi : lo;
        fvec<N / 2> r;
#pragma unroll
        for (int i = 0; i < N / 2; ++i) r[i] = keep[i] + xchg(send[i], O);
        return butterfly<N / 2, O / 2>(r, lane);
    }
}

constexpr int kWaves = 8;   // waves per workgroup

// lane holding the full score of query head h (for lane group `sub`) after the butterfly
template <int GRP, int LPP>
__device__ __forceinline__ constexpr int head_lane(int sub, int h) { return sub * LPP + h * (LPP / GRP); }

// K / V rows are streamed with non-temporal loads: they are read once per token, and
// allocating them in the caches evicts dirty lines whose write-back competes with the
// stream (measured: 2.7 TB/s with plain loads against 6.2 TB/s non-temporal for the same
// K + V stream behind a cache full of dirty data).
__device__ __forceinline__ float4 load_stream(const float* p) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// 4 consecutive bf16 cache elements (8 bytes), widened exactly
__device__ __forceinline__ float4 load_stream_bf16(const uint16_t* p) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    const u2 v = __builtin_nontemporal_load(reinterpret_cast<const u2*>(p));
    return make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

template <int GRP, int LPP, int kBatch, bool DBUF, bool KVB>
__global__ __launch_bounds__(512) void attn_partial_kernel(AttnDecodeArgs a) {
    attn_select_layer(a, blockIdx.z);
    constexpr int NF4 = 64 / LPP;   // float4 of one K row per lane in the score layout
    constexpr int PPW = 64 / LPP;   // positions per score pass (one per lane group)
    constexpr int QIT = kBatch / PPW;
    constexpr int OWN = LPP / GRP;  // lanes sharing one head after the butterfly
    constexpr int NROW = GRP + 1;   // normed rows: GRP queries (+ the new key)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, kh = blockIdx.y;
    const int pos = read_pos(a);
    const int n = pos + 1;
    const int per = split_len(n, a.n_splits);
    const int j0 = split * per;
    if (j0 >= n) return;
    const int j1 = min(n, j0 + per);
    const bool owns_new = j1 == n;  // this split holds position pos
    // each wave walks its own contiguous sub-range [w0, w1)
    const int wpe = (j1 - j0 + kWaves - 1) / kWaves;
    const int w0 = j0 + wave * wpe, w1 = min(j1, w0 + wpe);

    const int64_t hoff = static_cast<int64_t>(kh) * a.max_ctx * kHD;  // elements
    const float* K = a.k_cache + hoff;
    const float* V = a.v_cache + hoff;
    const uint16_t* Kb = reinterpret_cast<const uint16_t*>(a.k_cache) + hoff;
    const uint16_t* Vb = reinterpret_cast<const uint16_t*>(a.v_cache) + hoff;
    const float sc = 1.0f / sqrtf(static_cast<float>(kHD));

    __shared__ float rows_s[NROW][kHD];  // normed + rotated q rows, then the new key
    __shared__ float vnew_s[kHD];
    __shared__ float cs_s[2][kHD / 2];   // RoPE cos / sin of this position
    __shared__ float ml_s[kWaves][GRP][2];
    __shared__ float red[GRP][kHD];

    const int pl = lane % LPP, sub = lane / LPP;
    float4 kA[QIT][NF4], vA[kBatch];
    float4 kB[DBUF ? QIT : 1][NF4], vB[DBUF ? kBatch : 1];
    auto load = [&](float4 (&kr)[QIT][NF4], float4 (&vr)[kBatch], int b0) {
#pragma unroll
        for (int it = 0; it < QIT; ++it) {
            const int64_t off = static_cast<int64_t>(min(b0 + it * PPW + sub, w1 - 1)) * kHD + pl * 4;
#pragma unroll
            for (int m = 0; m < NF4; ++m)
                kr[it][m] = KVB ? load_stream_bf16(Kb + off + m * LPP * 4) : load_stream(K + off + m * LPP * 4);
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int64_t off = static_cast<int64_t>(min(b0 + j, w1 - 1)) * kHD + lane * 4;
            vr[j] = KVB ? load_stream_bf16(Vb + off) : load_stream(V + off);
        }
    };
    // ---- prologue loads, then the first two K / V batches, all unconditional (rows clamped
    // into valid ones): a load under a branch makes the wait-count insertion wait for every
    // outstanding load, so the prologue would wait for the K / V batches.
    const int half = a.ROT / 2;
    const int nrow = owns_new ? NROW : GRP;
    constexpr int RW = (NROW + kWaves - 1) / kWaves;  // prologue rows per wave
    float4 px[RW], pw[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const int r = min(wave + i * kWaves, nrow - 1);
        const bool is_q = r < GRP;
        const float* src = is_q ? a.qg + static_cast<int64_t>(kh * GRP + r) * 2 * kHD
                                : a.k_new + static_cast<int64_t>(kh) * kHD;
        const float* w = is_q ? a.q_norm : a.k_norm;
        px[i] = *reinterpret_cast<const float4*>(src + lane * 4);
        pw[i] = *reinterpret_cast<const float4*>(w + lane * 4);
    }
    const float4 vn4 = *reinterpret_cast<const float4*>(a.v_new + static_cast<int64_t>(kh) * kHD + lane * 4);
    float csv0 = 0.0f, csv1 = 0.0f;
    if (a.rope_cs) {  // uniform: the table row of this position
        const int i = min(lane, max(half - 1, 0));
        csv0 = a.rope_cs[static_cast<int64_t>(pos) * a.ROT + i];
        csv1 = a.rope_cs[static_cast<int64_t>(pos) * a.ROT + half + i];
    }
    load(kA, vA, w0);
    if constexpr (DBUF) load(kB, vB, w0 + kBatch);

    // ---- prologue: q_norm + RoPE of the GRP query rows (and k_norm + RoPE of the new key)
    if (tid < half) {
        if (a.rope_cs) {  // precomputed with the same double-precision formula
            cs_s[0][tid] = csv0;
            cs_s[1][tid] = csv1;
        } else {
            const double inv_freq = pow(a.theta, -static_cast<double>(2 * tid) / a.ROT);
            const double ang = static_cast<double>(pos) * inv_freq;
            cs_s[0][tid] = static_cast<float>(cos(ang));
            cs_s[1][tid] = static_cast<float>(sin(ang));
        }
    }
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const int r = wave + i * kWaves;
        const float4 x = px[i], wv = pw[i];
        double ss = static_cast<double>(x.x) * x.x + static_cast<double>(x.y) * x.y +
                    static_cast<double>(x.z) * x.z + static_cast<double>(x.w) * x.w;
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(static_cast<float>(ss / kHD) + a.eps);
        float4 y;
        y.x = x.x * inv * (1.0f + wv.x);
        y.y = x.y * inv * (1.0f + wv.y);
        y.z = x.z * inv * (1.0f + wv.z);
        y.w = x.w * inv * (1.0f + wv.w);
        if (r < nrow) *reinterpret_cast<float4*>(&rows_s[r][lane * 4]) = y;
    }
    if (owns_new && wave == 0) *reinterpret_cast<float4*>(&vnew_s[lane * 4]) = vn4;
    __syncthreads();
    for (int t = tid; t < nrow * half; t += kWaves * 64) {
        const int r = t / half, i = t - r * half;
        const float c = cs_s[0][i], s = cs_s[1][i];
        const float x1 = rows_s[r][i], x2 = rows_s[r][i + half];
        rows_s[r][i] = x1 * c - x2 * s;
        rows_s[r][i + half] = x2 * c + x1 * s;
    }
    __syncthreads();
    if (owns_new && tid < kHD) {  // append the new K / V rows
        const int64_t off = hoff + static_cast<int64_t>(pos) * kHD + tid;
        if constexpr (KVB) {
            // the cache holds the rounded row, and so does the score of position pos here
            const uint16_t kb = f32_to_bf16(rows_s[GRP][tid]), vb = f32_to_bf16(vnew_s[tid]);
            reinterpret_cast<uint16_t*>(a.k_cache)[off] = kb;
            reinterpret_cast<uint16_t*>(a.v_cache)[off] = vb;
            rows_s[GRP][tid] = bf16_to_f32(kb);
            vnew_s[tid] = bf16_to_f32(vb);
        } else {
            a.k_cache[off] = rows_s[GRP][tid];
            a.v_cache[off] = vnew_s[tid];
        }
    }
    if constexpr (KVB) __syncthreads();

    float4 qr[GRP][NF4];
#pragma unroll
    for (int h = 0; h < GRP; ++h)
#pragma unroll
        for (int m = 0; m < NF4; ++m) qr[h][m] = *reinterpret_cast<const float4*>(&rows_s[h][pl * 4 + m * LPP * 4]);
    float4 acc[GRP];
#pragma unroll
    for (int h = 0; h < GRP; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    float m_run = -INFINITY, l_run = 0.0f;  // running max / sum of this lane's head

    // one batch of kBatch positions starting at b0, from registers kr / vr
    auto consume = [&](float4 (&kr)[QIT][NF4], float4 (&vr)[kBatch], int b0) {
        float s[QIT];
#pragma unroll
        for (int it = 0; it < QIT; ++it) {
            const int p = b0 + it * PPW + sub;
            if (owns_new && min(p, w1 - 1) == pos)  // loaded before this workgroup appended it
#pragma unroll
                for (int m = 0; m < NF4; ++m)
                    kr[it][m] = *reinterpret_cast<const float4*>(&rows_s[GRP][pl * 4 + m * LPP * 4]);
            fvec<GRP> d;
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
                d[h] = t;
            }
            const float score = butterfly<GRP, LPP / 2>(d, lane);
            s[it] = p < w1 ? score * sc : -INFINITY;
        }
        float cmax = s[0];
#pragma unroll
        for (int it = 1; it < QIT; ++it) cmax = fmaxf(cmax, s[it]);
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, o));
        const float m_new = fmaxf(m_run, cmax);
        const float f = expf(m_run - m_new);
        float e[QIT], es = 0.0f;
#pragma unroll
        for (int it = 0; it < QIT; ++it) {
            e[it] = b0 + it * PPW + sub < w1 ? expf(s[it] - m_new) : 0.0f;
            es += e[it];
        }
#pragma unroll
        for (int o = LPP; o < 64; o <<= 1) es += __shfl_xor(es, o);
        l_run = l_run * f + es;
        m_run = m_new;
#pragma unroll
        for (int h = 0; h < GRP; ++h) {
            const float fh = readlane_f(f, head_lane<GRP, LPP>(0, h));
            acc[h].x *= fh;
            acc[h].y *= fh;
            acc[h].z *= fh;
            acc[h].w *= fh;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            if (owns_new && min(b0 + j, w1 - 1) == pos) vr[j] = *reinterpret_cast<const float4*>(&vnew_s[lane * 4]);
#pragma unroll
            for (int h = 0; h < GRP; ++h) {
                const float ev = readlane_f(e[j / PPW], head_lane<GRP, LPP>(j % PPW, h));
                acc[h].x = fmaf(ev, vr[j].x, acc[h].x);
                acc[h].y = fmaf(ev, vr[j].y, acc[h].y);
                acc[h].z = fmaf(ev, vr[j].z, acc[h].z);
                acc[h].w = fmaf(ev, vr[j].w, acc[h].w);
            }
        }
    };

    if constexpr (DBUF) {
        for (int b0 = w0; b0 < w1; b0 += 2 * kBatch) {
            const int b1 = b0 + kBatch;
            if (b0 != w0 && b1 < w1) load(kB, vB, b1);  // the first B batch is loaded above
            consume(kA, vA, b0);
            if (b1 >= w1) break;
            if (b1 + kBatch < w1) load(kA, vA, b1 + kBatch);
            consume(kB, vB, b1);
        }
    } else {
        for (int b0 = w0; b0 < w1; b0 += kBatch) {
            if (b0 != w0) load(kA, vA, b0);
            consume(kA, vA, b0);
        }
    }

    // ---- merge the waves: rescale each wave's P.V to the workgroup max, fixed-order sum
    if (sub == 0 && (pl % OWN) == 0) {
        ml_s[wave][pl / OWN][0] = m_run;
        ml_s[wave][pl / OWN][1] = l_run;
    }
    const int64_t base = (static_cast<int64_t>(kh) * a.n_splits + split) * GRP;
    if constexpr (GRP <= 8) {
        // every wave's accumulators to LDS, one barrier, each thread merges its outputs
        __shared__ float redw[kWaves][GRP][kHD];
#pragma unroll
        for (int h = 0; h < GRP; ++h) *reinterpret_cast<float4*>(&redw[wave][h][lane * 4]) = acc[h];
        __syncthreads();
        for (int i = tid; i < GRP * kHD; i += kWaves * 64) {
            const int h = i / kHD, dd = i - h * kHD;
            float M = ml_s[0][h][0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) M = fmaxf(M, ml_s[w][h][0]);
            float o = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float mw = ml_s[w][h][0];
                if (mw != -INFINITY) o = fmaf(redw[w][h][dd], expf(mw - M), o);
            }
            a.part_o[base * kHD + i] = o;
        }
    } else {
        __syncthreads();
#pragma unroll
        for (int h = 0; h < GRP; ++h) {
            float M = ml_s[0][h][0];
            for (int w = 1; w < kWaves; ++w) M = fmaxf(M, ml_s[w][h][0]);
            const float mw = ml_s[wave][h][0];
            const float g = mw == -INFINITY ? 0.0f : expf(mw - M);
            acc[h].x *= g;
            acc[h].y *= g;
            acc[h].z *= g;
            acc[h].w *= g;
        }
        for (int w = 0; w < kWaves; ++w) {
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
        for (int i = tid; i < GRP * kHD; i += kWaves * 64) a.part_o[base * kHD + i] = red[i / kHD][i % kHD];
    }
    if (tid < GRP) {
        float M = ml_s[0][tid][0];
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, ml_s[w][tid][0]);
        float L = 0.0f;
        for (int w = 0; w < kWaves; ++w) {
            const float mw = ml_s[w][tid][0];
            if (mw != -INFINITY) L += ml_s[w][tid][1] * expf(mw - M);
        }
        a.part_ml[(base + tid) * 2] = M;
        a.part_ml[(base + tid) * 2 + 1] = L;
    }
}

// ---------------------------------------------------------------- matrix-core partial kernel
// GQA group of 8 (the 2B shape), rotary dims a multiple of 32. Same split-K partials as
// attn_partial_kernel, with the dot products on v_mfma_f32_16x16x4f32 (fp32 operands, fp32
// accumulation): for a tile of 16 cache positions, S[16 pos][16 cols] = K_tile . Q^T with
// the 8 query heads in columns 0-7 (8-15 are zero), then O[16 rows][16 dims] += P . V_tile
// with the heads in rows 0-7. A lane l (column / row l % 16, group g = l / 16) holds
//   K operand   K[p0 + l%16][16c + 4g + i]              (float4 per c: 64 B per row / instr)
//   Q operand   Q[head l%16][16c + 4g + i]              (from LDS, same dim order)
//   scores      S[p0 + 4g + r][head l%16], r = 0..3     (the MFMA output registers)
//   P operand   P[head l%16][p0 + 4g + v] = score reg v  (no data movement)
//   V operand   V[p0 + 4g + v][64t + 4(l%16) + i]       (float4 per (v, t): 256 B per row)
//   O           O[head 4g + r][64t + 4(l%16) + i]        (16 accumulator tiles)
// so no lane exchange is needed between the two products; the softmax of a tile reduces
// over the 4 registers and the 4 lane groups (two exchanges). Four waves per workgroup
// walk whole tiles; their (m, l, O) are merged through LDS at the end.
// With a bf16 cache the products run on the bf16 matrix cores instead, exactly: Q and P are
// split into three bf16 parts each (hi + mid + lo = the fp32 value) and every bf16 x bf16
// product is exact in fp32. S = K . Q^T on v_mfma_f32_16x16x32_bf16 (K operand: 8 dims
// 32c + 8g .. + 7 of row p0 + l%16, one 16-byte load; Q parts from LDS in that order), and
// O += P . V on v_mfma_f32_16x16x16_bf16 (P operand: the 4 score registers of head l%16 =
// positions 4g .. 4g + 3; V operand: the same 4 positions of dim 64t + 4(l%16) + i,
// regrouped from the loaded rows). The scores and O keep the fp32 layouts above.
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kMW = 4;  // waves per workgroup of the matrix-core kernel

// four consecutive bf16 cache elements, read non-temporally and widened exactly
struct KvBf16 {
    using T = uint2;
    static __device__ __forceinline__ T load(const float* base, int64_t off) {
        typedef unsigned int u2 __attribute__((ext_vector_type(2)));
        const u2 v = __builtin_nontemporal_load(reinterpret_cast<const u2*>(reinterpret_cast<const uint16_t*>(base) + off));
        return make_uint2(v.x, v.y);
    }
    static __device__ __forceinline__ float4 f4(const T& v) {
        return make_float4(bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y));
    }
};

// rmsnorm (1 + w) + RoPE of one 256-vector held as 4 dims per lane (dims 4 lane .. + 3),
// sum of squares in double; cos / sin of dims (d mod ROT/2) for d < ROT from the table or
// from the double-precision angle (src/forward_pass.cpp:77-84,102-112).
__device__ __forceinline__ float4 norm_rope_row(float4 x, float4 w, float4 c, float4 sn, int lane, int ROT, float eps) {
    double ss = static_cast<double>(x.x) * x.x + static_cast<double>(x.y) * x.y + static_cast<double>(x.z) * x.z +
                static_cast<double>(x.w) * x.w;
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(static_cast<float>(ss / kHD) + eps);
    float4 y;
    y.x = x.x * inv * (1.0f + w.x);
    y.y = x.y * inv * (1.0f + w.y);
    y.z = x.z * inv * (1.0f + w.z);
    y.w = x.w * inv * (1.0f + w.w);
    const int hq = ROT / 8;  // lanes holding the first half of the rotated dims
    const int src = lane < hq ? lane + hq : lane - hq;
    float4 o;  // the partner dims d +- ROT/2
    o.x = __shfl(y.x, src);
    o.y = __shfl(y.y, src);
    o.z = __shfl(y.z, src);
    o.w = __shfl(y.w, src);
    if (lane < hq) {
        y.x = y.x * c.x - o.x * sn.x;
        y.y = y.y * c.y - o.y * sn.y;
        y.z = y.z * c.z - o.z * sn.z;
        y.w = y.w * c.w - o.w * sn.w;
    } else if (lane < 2 * hq) {
        y.x = y.x * c.x + o.x * sn.x;
        y.y = y.y * c.y + o.y * sn.y;
        y.z = y.z * c.z + o.z * sn.z;
        y.w = y.w * c.w + o.w * sn.w;
    }
    return y;
}

// weight of a wave's partial with maximum mw in a merge with maximum M (0 for an empty wave)
__device__ __forceinline__ float m_run_of(float mw, float M) { return mw == -INFINITY ? 0.0f : expf(mw - M); }

// bf16 caches, GQA 8: split-K over the cache, a workgroup of four waves per (kv head, range of
// positions) serving the 8 query heads from each K/V row. Each wave walks tiles of 16
// positions: S = K.Q^T on the 16x16x32 bf16 matrix cores against the three exact bf16 parts
// of Q, O += P.V on the 16x16x16 bf16 cores with the three exact parts of P (every bf16 x bf16
// product is exact in fp32); online softmax per head; waves merged once at the end.
// ML: several layers in one launch (grid.z); a single-layer launch reads no layer strides
template <bool ML>
__global__ __launch_bounds__(kMW * 64, 2) void attn_mfma_bf16_kernel(const int* pos_dev, int pos_val, const float* qg,
                                                            const float* k_new, const float* v_new,
                                                            const float* q_norm, const float* k_norm,
                                                            AttnDecodeArgs a) {
    set_lead(a, pos_dev, pos_val, qg, k_new, v_new, q_norm, k_norm);
    if (ML) attn_select_layer(a, blockIdx.z);
    using KV = KvBf16;
    using KT = typename KV::T;
    constexpr int GRP = 8, TP = 16;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loop bounds
    const int n16 = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, kh = blockIdx.y;
    // the query-side rows first (rows of this wave: q heads wave, wave + 4, and row 8 the
    // appended key); they do not depend on the position
    float4 px[3], pw[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int r = min(wave + i * kMW, GRP);  // row 8 = the new key
        const float* src = r < GRP ? a.qg + static_cast<int64_t>(kh * GRP + r) * 2 * kHD
                                   : a.k_new + static_cast<int64_t>(kh) * kHD;
        px[i] = *reinterpret_cast<const float4*>(src + lane * 4);
        pw[i] = *reinterpret_cast<const float4*>((r < GRP ? a.q_norm : a.k_norm) + lane * 4);
    }
    const float4 vn4 = *reinterpret_cast<const float4*>(a.v_new + static_cast<int64_t>(kh) * kHD + lane * 4);
    // the kernarg fields the K / V addresses need, requested now (with the position below
    // they arrive in one round trip); nothing below is scheduled before the loads above (a
    // wait for a kernarg field would hold them back)
    const int64_t hoff = static_cast<int64_t>(kh) * a.max_ctx * kHD;  // elements
    float *const kcache = a.k_cache, *const vcache = a.v_cache;
    const int ROT = a.ROT, half = ROT / 2;
    __builtin_amdgcn_sched_barrier(0);
    const int pos = read_pos(a);
    // (the fields are requested with the position, not after the split check below)
    asm volatile("" ::"s"(hoff), "s"(kcache), "s"(vcache), "s"(ROT));
    const int n = pos + 1;
    const int per = split_len(n, a.n_splits);
    const int j0 = split * per;
    if (j0 >= n) return;
    const int j1 = min(n, j0 + per);
    const bool owns_new = j1 == n;
    const int tpw = ((j1 - j0 + TP - 1) / TP + kMW - 1) / kMW;  // tiles per wave
    const int w0 = min(j1, j0 + wave * tpw * TP), w1 = min(j1, w0 + tpw * TP);
    // the wave ending at pos walks the cached positions only; the appended row is added at
    // the end from LDS (so nothing in the tile loop depends on where pos falls)
    const bool has_new = owns_new && w0 < w1 && w1 == n;  // empty waves also end at n
    const int wl = has_new ? w1 - 1 : w1;

    const float* Kc_ = reinterpret_cast<const float*>(reinterpret_cast<const uint16_t*>(kcache) + hoff);
    const float* Vc_ = reinterpret_cast<const float*>(reinterpret_cast<const uint16_t*>(vcache) + hoff);
    const float sc = 1.0f / sqrtf(static_cast<float>(kHD));

    __shared__ float4 qs[16][64];             // Q in fp32 (the appended row's score): [c][lane]
    // the three exact bf16 parts of Q as the B operand of the 16x16x32 products,
    // [part][c][lane] with lane 16 g + head holding dims 32 c + 8 g .. + 7
    __shared__ uint4 qsb[3][8][64];
    __shared__ float4 ks[kHD / 4], vs[kHD / 4];  // the appended rows (as the cache holds them)
    __shared__ float os[kMW][GRP][kHD];
    __shared__ float ml_s[kMW][GRP][2];

    // ---- prologue (the rows requested above: q heads wave, wave + 4 of this wave, the key
    // on wave 0 and the value on wave 1 of the workgroup holding pos): the RoPE table row,
    // then the first K / V tiles
    const int ci = (lane * 4) % max(half, 4);  // table column of this lane's first dim
    float4 cs4 = make_float4(1.f, 1.f, 1.f, 1.f), sn4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (a.rope_cs) {
        const float* t = a.rope_cs + static_cast<int64_t>(pos) * ROT;
        cs4 = *reinterpret_cast<const float4*>(t + min(ci, max(half - 4, 0)));
        sn4 = *reinterpret_cast<const float4*>(t + half + min(ci, max(half - 4, 0)));
    }
    // K rows as the A operand: 8 dims 32 c + 8 g .. per 16-byte register (8 per tile, the
    // 16x16x32 bf16 operand)
    using KOp = uint4;
    constexpr int NK = 8;
    KOp kA[NK];
    KT vr[4][4];
    // Loads are issued unconditionally (a load under a branch makes the wait-count pass wait
    // for all outstanding loads at the join); past the end of the range every lane reads the
    // same 16 bytes of row w1 - 1, which costs the memory pipeline almost nothing.
    const int last = max(wl - 1, 0);  // a valid row to clamp to
    auto loadK = [&](KOp (&kr)[NK], int p0) {
        const int mask = -static_cast<int>(p0 < wl);  // all ones while live (no branch)
        const int64_t row = min(p0 + n16, last);
        typedef unsigned int u4 __attribute__((ext_vector_type(4)));
        const uint16_t* Kb = reinterpret_cast<const uint16_t*>(Kc_);
#pragma unroll
        for (int c = 0; c < NK; ++c) {
            const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(Kb + row * kHD + ((32 * c + 8 * g) & mask)));
            kr[c] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };
    auto loadV = [&](int p0) {
        const int mask = -static_cast<int>(p0 < wl);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t row = min((p0 + 4 * g + v) & mask, last) | (last & ~mask);
#pragma unroll
            for (int t = 0; t < 4; ++t) vr[v][t] = KV::load(Vc_, row * kHD + ((64 * t + 4 * n16) & mask));
        }
    };
    loadK(kA, w0);
    loadV(w0);

    // ---- Q operand and the appended rows
    if (!a.rope_cs) rope_cs4(a.theta, ROT, pos, lane, cs4, sn4);  // double-precision angles
    for (int e = tid; e < 3 * 8 * 32; e += kMW * 64)  // columns 8-15: zero heads
            qsb[e >> 8][(e >> 5) & 7][16 * ((e >> 3) & 3) + 8 + (e & 7)] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int r = wave + i * kMW;
        if (r > GRP || (r == GRP && !owns_new)) continue;  // uniform per wave
        float4 y = norm_rope_row(px[i], pw[i], cs4, sn4, lane, ROT, a.eps);
        if (r < GRP) {
            qs[lane >> 2][16 * (lane & 3) + r] = y;  // dims 4 lane .. + 3 of head r
            {  // dims 4 lane .. + 3 = half (lane & 1) of the slot (lane >> 3, (lane >> 1) & 3)
                const float v4[4] = {y.x, y.y, y.z, y.w};
                uint32_t hh[4], mm[4], ll[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) split3(v4[e], hh[e], mm[e], ll[e]);
                uint2* slot0 = reinterpret_cast<uint2*>(&qsb[0][lane >> 3][16 * ((lane >> 1) & 3) + r]) + (lane & 1);
                uint2* slot1 = reinterpret_cast<uint2*>(&qsb[1][lane >> 3][16 * ((lane >> 1) & 3) + r]) + (lane & 1);
                uint2* slot2 = reinterpret_cast<uint2*>(&qsb[2][lane >> 3][16 * ((lane >> 1) & 3) + r]) + (lane & 1);
                *slot0 = make_uint2(hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16));
                *slot1 = make_uint2(mm[0] | (mm[1] << 16), mm[2] | (mm[3] << 16));
                *slot2 = make_uint2(ll[0] | (ll[1] << 16), ll[2] | (ll[3] << 16));
            }
        } else {
            const int64_t off = hoff + static_cast<int64_t>(pos) * kHD + lane * 4;
            const uint16_t b0 = f32_to_bf16(y.x), b1 = f32_to_bf16(y.y), b2 = f32_to_bf16(y.z), b3 = f32_to_bf16(y.w);
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.k_cache) + off) =
                make_uint2(b0 | (static_cast<uint32_t>(b1) << 16), b2 | (static_cast<uint32_t>(b3) << 16));
            y = make_float4(bf16_to_f32(b0), bf16_to_f32(b1), bf16_to_f32(b2), bf16_to_f32(b3));
            ks[lane] = y;
        }
    }
    if (owns_new && wave == 1) {
        const int64_t off = hoff + static_cast<int64_t>(pos) * kHD + lane * 4;
        const float4 y = vn4;
        const uint16_t b0 = f32_to_bf16(y.x), b1 = f32_to_bf16(y.y), b2 = f32_to_bf16(y.z), b3 = f32_to_bf16(y.w);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.v_cache) + off) =
            make_uint2(b0 | (static_cast<uint32_t>(b1) << 16), b2 | (static_cast<uint32_t>(b3) << 16));
        vs[lane] = make_float4(bf16_to_f32(b0), bf16_to_f32(b1), bf16_to_f32(b2), bf16_to_f32(b3));
    }
    // LDS-only barrier: the K / V tiles in flight are not waited for here
    lds_barrier();

    floatx4 O[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) O[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;  // of head n16 (same in the 4 lane groups)

    // one tile of positions p0 .. p0 + 15 from K registers kr and the V registers; the next
    // tile's rows are requested as soon as these registers are consumed
    auto tile = [&](KOp (&kr)[NK], int p0, auto more) {
        // bf16 K times the three exact bf16 parts of Q on the 16x16x32 bf16 matrix cores
        // (every product exact in fp32), one accumulation chain per part
        floatx4 S3[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) S3[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NK; ++c) {
            const bf16x8 kop = __builtin_bit_cast(bf16x8, kr[c]);
#pragma unroll
            for (int part = 0; part < 3; ++part)
                S3[part] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, __builtin_bit_cast(bf16x8, qsb[part][c][lane]),
                                                                   S3[part], 0, 0, 0);
            if ((c & 1) == 1) __builtin_amdgcn_sched_barrier(0);
        }
        const floatx4 S = (S3[2] + S3[1]) + S3[0];
        if constexpr (decltype(more)::value) loadK(kr, p0 + TP);
        float s[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = p0 + 4 * g + r < wl ? S[r] * sc : -INFINITY;
        float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        tm = fmaxf(tm, xchg(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        // the reference max moves only when a score exceeds it by more than 8 (the weights
        // exp(s - m) stay below e^8, far from overflow), so the accumulators are rarely rescaled
        const float m_new = tm > m_run + 8.0f ? tm : m_run;
        const float f = expf(m_run - m_new);
        float p[4], ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = n16 < GRP ? expf(s[r] - m_new) : 0.0f;
            ps += p[r];
        }
        ps += xchg(ps, 16);
        ps += __shfl_xor(ps, 32);
        l_run = l_run * f + ps;
        m_run = m_new;
        if (__any(f != 1.0f)) {  // rescale the accumulators of heads 4g + r
            float fh[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) fh[r] = __shfl(f, 4 * g + r);
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                O[t][0] *= fh[0];
                O[t][1] *= fh[1];
                O[t][2] *= fh[2];
                O[t][3] *= fh[3];
            }
        }
        // the three exact bf16 parts of P (A operand: head n16, positions 4g .. 4g + 3)
        // times bf16 V (B operand: those positions, dim 64t + 4 n16 + i) on the 16x16x16
        // bf16 matrix cores; V's 16-bit elements are regrouped from the rows as loaded
        typedef short short4_ __attribute__((ext_vector_type(4)));
        uint32_t hh[4], mm[4], ll[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) split3(p[v], hh[v], mm[v], ll[v]);
        const short4_ pp[3] = {
            __builtin_bit_cast(short4_, make_uint2(ll[0] | (ll[1] << 16), ll[2] | (ll[3] << 16))),
            __builtin_bit_cast(short4_, make_uint2(mm[0] | (mm[1] << 16), mm[2] | (mm[3] << 16))),
            __builtin_bit_cast(short4_, make_uint2(hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16)))};
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t e[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t w = i < 2 ? vr[v][t].x : vr[v][t].y;
                    e[v] = (i & 1) ? w >> 16 : w & 0xffffu;
                }
                const short4_ vb = __builtin_bit_cast(short4_, make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16)));
#pragma unroll
                for (int part = 0; part < 3; ++part)  // lo, mid, hi
                    O[4 * t + i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pp[part], vb, O[4 * t + i], 0, 0, 0);
            }
        if constexpr (decltype(more)::value) loadV(p0 + TP);
    };
    int p0 = w0;
    for (; p0 + TP < wl; p0 += TP) tile(kA, p0, std::true_type{});
    if (p0 < wl) tile(kA, p0, std::false_type{});  // the last tile requests nothing more

    if (has_new) {  // position pos: score of head h = lane & 7 over the 32 dims of chunk lane >> 3
        const int h = lane & 7, j = lane >> 3;
        float d = 0.0f;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                const float4 q = qs[2 * j + cc][16 * gg + h], kk = ks[4 * (2 * j + cc) + gg];
                d = fmaf(q.x, kk.x, d);
                d = fmaf(q.y, kk.y, d);
                d = fmaf(q.z, kk.z, d);
                d = fmaf(q.w, kk.w, d);
            }
        d += __shfl_xor(d, 8);
        d += __shfl_xor(d, 16);
        d += __shfl_xor(d, 32);
        const float sn = __shfl(d, n16 & 7) * sc;  // the score of head n16
        const float m_new = sn > m_run + 8.0f ? sn : m_run;
        const float f = expf(m_run - m_new);
        const float pn = n16 < GRP ? expf(sn - m_new) : 0.0f;
        l_run = l_run * f + pn;
        m_run = m_new;
        float fh[4], ph[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            fh[r] = __shfl(f, 4 * g + r);
            ph[r] = __shfl(pn, 4 * g + r);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float4 v = vs[16 * t + n16];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                O[4 * t + 0][r] = fmaf(ph[r], v.x, O[4 * t + 0][r] * fh[r]);
                O[4 * t + 1][r] = fmaf(ph[r], v.y, O[4 * t + 1][r] * fh[r]);
                O[4 * t + 2][r] = fmaf(ph[r], v.z, O[4 * t + 2][r] * fh[r]);
                O[4 * t + 3][r] = fmaf(ph[r], v.w, O[4 * t + 3][r] * fh[r]);
            }
        }
    }

    // ---- merge the waves: maxima first, then each wave rescales its own accumulators to the
    // workgroup maximum and the four are summed in a fixed order
    if (g == 0 && n16 < GRP) {
        ml_s[wave][n16][0] = m_run;
        ml_s[wave][n16][1] = l_run;
    }
    lds_barrier();
    if (g < 2) {
        float sc4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            float M = ml_s[0][h][0];
#pragma unroll
            for (int w = 1; w < kMW; ++w) M = fmaxf(M, ml_s[w][h][0]);
            sc4[r] = m_run_of(ml_s[wave][h][0], M);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<float4*>(&os[wave][4 * g + r][64 * t + 4 * n16]) =
                    make_float4(O[4 * t][r] * sc4[r], O[4 * t + 1][r] * sc4[r], O[4 * t + 2][r] * sc4[r],
                                O[4 * t + 3][r] * sc4[r]);
    }
    lds_barrier();
    const int64_t base = (static_cast<int64_t>(kh) * a.n_splits + split) * GRP;
#pragma unroll
    for (int it = 0; it < GRP * kHD / (4 * kMW * 64); ++it) {
        const int e = (it * kMW * 64 + tid) * 4, h = e / kHD, dd = e - h * kHD;
        float4 o = *reinterpret_cast<const float4*>(&os[0][h][dd]);
#pragma unroll
        for (int w = 1; w < kMW; ++w) {
            const float4 x = *reinterpret_cast<const float4*>(&os[w][h][dd]);
            o.x += x.x;
            o.y += x.y;
            o.z += x.z;
            o.w += x.w;
        }
        *reinterpret_cast<float4*>(a.part_o + base * kHD + e) = o;
    }
    if (tid < GRP) {
        float M = ml_s[0][tid][0];
        for (int w = 1; w < kMW; ++w) M = fmaxf(M, ml_s[w][tid][0]);
        float L = 0.0f;
        for (int w = 0; w < kMW; ++w) L += ml_s[w][tid][1] * m_run_of(ml_s[w][tid][0], M);
        a.part_ml[(base + tid) * 2] = M;
        a.part_ml[(base + tid) * 2 + 1] = L;
    }
}

// ---- fp32 caches, GQA 8: both products on v_mfma_f32_4x4x1_16b_f32 ----------------------
// 16x16x4 products would use 8 of their 16 columns (8 query heads); the 4x4x1 instruction
// holds 16 independent 4 x 4 blocks, so every lane carries a useful product. Lane l = 16 g + 4 pg + j (block b = l / 4 = pg + 4 g, A row / B column j):
//   S = K.Q^T: A = K[row 4 pg + j][dim], B = Q[head 4 hg + j][dim] for the dims 16 u + 4 g + e
//   (u = 0..15, e = 0..3) -- the K registers are the rows as the 16x16x4 kernel loads them --
//   so block (pg, g) accumulates positions 4 pg .. + 3 x heads 4 hg .. + 3 over a quarter of
//   the dims; the quarters are summed across lanes by the gfx950 16- and 32-lane swaps.
//   Result: lane l holds S[4 pg + i][4 hg + (l & 3)] in register i.
//   O += P.V: A = P[head 4 hg + (l & 3)][p] (every block), B = V[p][4 l + c] (component c of
//   the lane's float4 of row p: V rows are loaded as whole contiguous 1 KB rows), so
//   accumulator (hg, c) register i of lane l holds O[4 hg + i][4 l + c]: 8 x 4 registers for
//   the 8 heads x 256 dims. P goes from the score lanes to the A operand through 512 bytes of
//   LDS per wave.
// 256 products of 4x4x1 per 16-position tile against 128 of 16x16x4: measured about 10-11
// cycles against 32 per instruction, so each tile's products take ~2.5k cycles instead of ~4k.
__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}
// sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the 16- and 32-lane swaps of gfx950)
__device__ __forceinline__ float dimq_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    v = __builtin_bit_cast(float, static_cast<int>(r[0])) + __builtin_bit_cast(float, static_cast<int>(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, static_cast<int>(r[0])) + __builtin_bit_cast(float, static_cast<int>(r[1]));
}
// over the lanes l, l + 4, l + 8, l + 12 of a 16-lane row (DPP row rotations by 4 and 8)
__device__ __forceinline__ float pg_max(float v) {
    v = fmaxf(v, dpp_f<0x124>(v));
    return fmaxf(v, dpp_f<0x128>(v));
}
__device__ __forceinline__ float pg_sum(float v) {
    v += dpp_f<0x124>(v);
    return v + dpp_f<0x128>(v);
}

template <bool ML>
__global__ __launch_bounds__(kMW * 64, 2) void attn_mfma4_kernel(const int* pos_dev, int pos_val, const float* qg,
                                                            const float* k_new, const float* v_new,
                                                            const float* q_norm, const float* k_norm,
                                                            AttnDecodeArgs a) {
    set_lead(a, pos_dev, pos_val, qg, k_new, v_new, q_norm, k_norm);
    if (ML) attn_select_layer(a, blockIdx.z);
    constexpr int GRP = 8, TP = 16;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loop bounds
    const int n16 = lane & 15, g = lane >> 4, jj = lane & 3, pg = (lane >> 2) & 3;
    const int split = blockIdx.x, kh = blockIdx.y;
    // the query-side rows first (rows of this wave: q heads wave, wave + 4, and row 8 the
    // appended key); they do not depend on the position
    float4 px[3], pw[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int r = min(wave + i * kMW, GRP);  // row 8 = the new key
        const float* src = r < GRP ? a.qg + static_cast<int64_t>(kh * GRP + r) * 2 * kHD
                                   : a.k_new + static_cast<int64_t>(kh) * kHD;
        px[i] = *reinterpret_cast<const float4*>(src + lane * 4);
        pw[i] = *reinterpret_cast<const float4*>((r < GRP ? a.q_norm : a.k_norm) + lane * 4);
    }
    const float4 vn4 = *reinterpret_cast<const float4*>(a.v_new + static_cast<int64_t>(kh) * kHD + lane * 4);
    // the kernarg fields the K / V addresses need, requested now (with the position below
    // they arrive in one round trip); nothing below is scheduled before the loads above (a
    // wait for a kernarg field would hold them back)
    const int64_t hoff = static_cast<int64_t>(kh) * a.max_ctx * kHD;  // elements
    float *const kcache = a.k_cache, *const vcache = a.v_cache;
    const int ROT = a.ROT, half = ROT / 2;
    __builtin_amdgcn_sched_barrier(0);
    const int pos = read_pos(a);
    // (the fields are requested with the position, not after the split check below)
    asm volatile("" ::"s"(hoff), "s"(kcache), "s"(vcache), "s"(ROT));
    const int n = pos + 1;
    const int per = split_len(n, a.n_splits);
    const int j0 = split * per;
    if (j0 >= n) return;
    const int j1 = min(n, j0 + per);
    const bool owns_new = j1 == n;
    const int tpw = ((j1 - j0 + TP - 1) / TP + kMW - 1) / kMW;  // tiles per wave
    const int w0 = min(j1, j0 + wave * tpw * TP), w1 = min(j1, w0 + tpw * TP);
    // the wave ending at pos walks the cached positions only; the appended row is added at
    // the end from LDS (so nothing in the tile loop depends on where pos falls)
    const bool has_new = owns_new && w0 < w1 && w1 == n;  // empty waves also end at n
    const int wl = has_new ? w1 - 1 : w1;

    const float* Kc = kcache + hoff;
    const float* Vc = vcache + hoff;
    const float sc = 1.0f / sqrtf(static_cast<float>(kHD));

    __shared__ float4 qs[2][16][4][4];       // Q operand: [hg][u][j][g] = Q[4 hg + j][16 u + 4 g .. + 3]
    __shared__ float4 ks[kHD / 4], vs[kHD / 4];  // the appended rows
    __shared__ float4 pl[kMW][2][4][4];      // softmax weights of a tile: [hg][j][t] = P[4 hg + j][4 t .. + 3]
    __shared__ float os[kMW][GRP][kHD];
    __shared__ float ml_s[kMW][GRP][2];

    // ---- prologue (the rows requested above: q heads wave, wave + 4 of this wave, the key
    // on wave 0 and the value on wave 1 of the workgroup holding pos): the RoPE table row,
    // then the first K / V tiles
    const int ci = (lane * 4) % max(half, 4);  // table column of this lane's first dim
    float4 cs4 = make_float4(1.f, 1.f, 1.f, 1.f), sn4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (a.rope_cs) {
        const float* t = a.rope_cs + static_cast<int64_t>(pos) * ROT;
        cs4 = *reinterpret_cast<const float4*>(t + min(ci, max(half - 4, 0)));
        sn4 = *reinterpret_cast<const float4*>(t + half + min(ci, max(half - 4, 0)));
    }
    // K: row n16, dims 16 u + 4 g .. + 3 in register u; V: row p, dims 4 lane .. + 3 in
    // register p. Loads are issued unconditionally (a load under a branch makes the
    // wait-count pass wait for all outstanding loads at the join); past the end of the range
    // every lane reads the same 16 bytes of a valid row.
    float4 kA[16], vr[16];
    const int last = max(wl - 1, 0);  // a valid row to clamp to
    auto loadK = [&](float4 (&kr)[16], int p0) {
        const int mask = -static_cast<int>(p0 < wl);  // all ones while live (no branch)
        const int64_t row = min(p0 + n16, last);
#pragma unroll
        for (int u = 0; u < 16; ++u) kr[u] = load_stream(Kc + row * kHD + ((16 * u + 4 * g) & mask));
    };
    auto loadV = [&](int p0) {
        const int mask = -static_cast<int>(p0 < wl);
#pragma unroll
        for (int p = 0; p < TP; ++p) {
            const int64_t row = min((p0 + p) & mask, last) | (last & ~mask);
            vr[p] = load_stream(Vc + row * kHD + ((4 * lane) & mask));
        }
    };
    loadK(kA, w0);
    loadV(w0);

    // ---- Q operand and the appended rows
    if (!a.rope_cs) rope_cs4(a.theta, ROT, pos, lane, cs4, sn4);  // double-precision angles
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int r = wave + i * kMW;
        if (r > GRP || (r == GRP && !owns_new)) continue;  // uniform per wave
        const float4 y = norm_rope_row(px[i], pw[i], cs4, sn4, lane, ROT, a.eps);
        if (r < GRP) {
            qs[r >> 2][lane >> 2][r & 3][lane & 3] = y;  // dims 4 lane .. + 3 of head r
        } else {
            *reinterpret_cast<float4*>(a.k_cache + hoff + static_cast<int64_t>(pos) * kHD + lane * 4) = y;
            ks[lane] = y;
        }
    }
    if (owns_new && wave == 1) {
        *reinterpret_cast<float4*>(a.v_cache + hoff + static_cast<int64_t>(pos) * kHD + lane * 4) = vn4;
        vs[lane] = vn4;
    }
    // LDS-only barrier: the K / V tiles in flight are not waited for here
    lds_barrier();

    floatx4 O[2][4];  // [hg][c]: register i = O[4 hg + i][4 lane + c]
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int c = 0; c < 4; ++c) O[h][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};  // of heads jj + 4 hg

    // rescale the accumulators of heads 4 hg + i by the factors f of lanes i (heads i + 4 hg)
    auto rescale = [&](const float (&f)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float fh[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) fh[i] = __shfl(f[h], i);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) O[h][c][i] *= fh[i];
        }
    };

    auto tile = [&](float4 (&kr)[16], int p0, auto more) {
        floatx4 Sx[2][4];  // [hg][e]: eight independent accumulation chains
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) Sx[h][e] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const float4 k = kr[u];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float4 q = qs[h][u][jj][g];
                Sx[h][0] = mfma4(k.x, q.x, Sx[h][0]);
                Sx[h][1] = mfma4(k.y, q.y, Sx[h][1]);
                Sx[h][2] = mfma4(k.z, q.z, Sx[h][2]);
                Sx[h][3] = mfma4(k.w, q.w, Sx[h][3]);
            }
            // keep the Q operand reads close to their use (a few in flight, not all 32)
            if ((u & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (decltype(more)::value) loadK(kr, p0 + TP);
        // s[h][i]: position p0 + 4 pg + i, head 4 h + jj (the dim quarters summed)
        float s[2][4], tm[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const floatx4 S = (Sx[h][0] + Sx[h][1]) + (Sx[h][2] + Sx[h][3]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = dimq_sum(S[i]);
                s[h][i] = p0 + 4 * pg + i < wl ? v * sc : -INFINITY;
            }
            tm[h] = pg_max(fmaxf(fmaxf(s[h][0], s[h][1]), fmaxf(s[h][2], s[h][3])));
        }
        // the reference max moves only when a score exceeds it by more than 8 (the weights
        // exp(s - m) stay below e^8, far from overflow), so the accumulators are rarely rescaled
        float f[2], p[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float m_new = tm[h] > m_run[h] + 8.0f ? tm[h] : m_run[h];
            f[h] = expf(m_run[h] - m_new);
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[h][i] = expf(s[h][i] - m_new);
                ps += p[h][i];
            }
            l_run[h] = l_run[h] * f[h] + pg_sum(ps);
            m_run[h] = m_new;
        }
        if (__any(f[0] != 1.0f || f[1] != 1.0f)) rescale(f);
        // P to the A operand layout: the lanes of dim quarter 0 store their 4 positions of
        // heads jj, jj + 4; every lane reads the 16 positions of its heads (same wave: LDS
        // operations complete in order)
        if (g == 0) {
#pragma unroll
            for (int h = 0; h < 2; ++h) pl[wave][h][jj][pg] = make_float4(p[h][0], p[h][1], p[h][2], p[h][3]);
        }
        __builtin_amdgcn_wave_barrier();
        float4 pv[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int t = 0; t < 4; ++t) pv[h][t] = pl[wave][h][jj][t];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float4 v = vr[4 * t + e];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float pa = e == 0 ? pv[h][t].x : e == 1 ? pv[h][t].y : e == 2 ? pv[h][t].z : pv[h][t].w;
                    O[h][0] = mfma4(pa, v.x, O[h][0]);
                    O[h][1] = mfma4(pa, v.y, O[h][1]);
                    O[h][2] = mfma4(pa, v.z, O[h][2]);
                    O[h][3] = mfma4(pa, v.w, O[h][3]);
                }
            }
        if constexpr (decltype(more)::value) loadV(p0 + TP);
    };
    int p0 = w0;
    for (; p0 + TP < wl; p0 += TP) tile(kA, p0, std::true_type{});
    if (p0 < wl) tile(kA, p0, std::false_type{});  // the last tile requests nothing more

    if (has_new) {  // position pos: each lane's 4 dims for the 8 heads, then a halving butterfly
        const float4 kn = ks[lane];
        fvec<8> d;
#pragma unroll
        for (int h = 0; h < GRP; ++h) {
            const float4 q = qs[h >> 2][lane >> 2][h & 3][lane & 3];
            d[h] = ((q.x * kn.x + q.y * kn.y) + q.z * kn.z) + q.w * kn.w;
        }
        const float dh = butterfly<8, 32>(d, lane);  // head lane / 8 on every lane
        float f[2], pn[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float sn = __shfl(dh, 8 * (jj + 4 * h)) * sc;
            const float m_new = sn > m_run[h] + 8.0f ? sn : m_run[h];
            f[h] = expf(m_run[h] - m_new);
            pn[h] = expf(sn - m_new);
            l_run[h] = l_run[h] * f[h] + pn[h];
            m_run[h] = m_new;
        }
        rescale(f);
        const float4 v = vs[lane];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float ph = __shfl(pn[h], i);
                O[h][0][i] = fmaf(ph, v.x, O[h][0][i]);
                O[h][1][i] = fmaf(ph, v.y, O[h][1][i]);
                O[h][2][i] = fmaf(ph, v.z, O[h][2][i]);
                O[h][3][i] = fmaf(ph, v.w, O[h][3][i]);
            }
    }

    // ---- merge the waves: maxima first, then each wave rescales its own accumulators to the
    // workgroup maximum and the four are summed in a fixed order
    if (lane < 4) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            ml_s[wave][lane + 4 * h][0] = m_run[h];
            ml_s[wave][lane + 4 * h][1] = l_run[h];
        }
    }
    lds_barrier();
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hd = 4 * h + i;
            float M = ml_s[0][hd][0];
#pragma unroll
            for (int w = 1; w < kMW; ++w) M = fmaxf(M, ml_s[w][hd][0]);
            const float w8 = m_run_of(ml_s[wave][hd][0], M);
            *reinterpret_cast<float4*>(&os[wave][hd][4 * lane]) =
                make_float4(O[h][0][i] * w8, O[h][1][i] * w8, O[h][2][i] * w8, O[h][3][i] * w8);
        }
    lds_barrier();
    const int64_t base = (static_cast<int64_t>(kh) * a.n_splits + split) * GRP;
#pragma unroll
    for (int it = 0; it < GRP * kHD / (4 * kMW * 64); ++it) {
        const int e = (it * kMW * 64 + tid) * 4, h = e / kHD, dd = e - h * kHD;
        float4 o = *reinterpret_cast<const float4*>(&os[0][h][dd]);
#pragma unroll
        for (int w = 1; w < kMW; ++w) {
            const float4 x = *reinterpret_cast<const float4*>(&os[w][h][dd]);
            o.x += x.x;
            o.y += x.y;
            o.z += x.z;
            o.w += x.w;
        }
        *reinterpret_cast<float4*>(a.part_o + base * kHD + e) = o;
    }
    if (tid < GRP) {
        float M = ml_s[0][tid][0];
        for (int w = 1; w < kMW; ++w) M = fmaxf(M, ml_s[w][tid][0]);
        float L = 0.0f;
        for (int w = 0; w < kMW; ++w) L += ml_s[w][tid][1] * m_run_of(ml_s[w][tid][0], M);
        a.part_ml[(base + tid) * 2] = M;
        a.part_ml[(base + tid) * 2 + 1] = L;
    }
}

// grid (NQ, HD / 64), 256 threads, 64 dims per workgroup (one per lane). Every load is
// requested up front -- the (m, l) of split t on thread t and the o rows of splits
// 32 w .. 32 w + 31 on wave w -- so the merge waits for one memory round trip; the maximum
// and the split weights exp(m_s - M) go through LDS. Past 128 (o rows) or 256 ((m, l)
// pairs) active splits further passes follow.
__global__ __launch_bounds__(256) void attn_combine_kernel(const int* pos_dev, const float* part_ml,
                                                           const float* part_o, const float* qg, int n_splits,
                                                           int NQ, int NKV, AttnDecodeArgs a) {
    a.pos_dev = pos_dev;
    a.part_ml = const_cast<float*>(part_ml);
    a.part_o = const_cast<float*>(part_o);
    a.qg = qg;
    a.n_splits = n_splits;
    a.NQ = NQ;
    a.NKV = NKV;
    attn_select_layer(a, blockIdx.z);
    constexpr int kRW = 32;  // o rows per wave per pass
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d = blockIdx.y * 64 + lane;
    const int grp = a.NQ / a.NKV, kh = h / grp, g = h - kh * grp;
    const int n = read_pos(a) + 1;
    const int per = split_len(n, a.n_splits);
    const int nact = (n + per - 1) / per;
    const int64_t base = static_cast<int64_t>(kh) * a.n_splits * grp + g;  // split s: row base + s grp
    const float* po = a.part_o + base * kHD + d;
    const int64_t so = static_cast<int64_t>(grp) * kHD;
    __shared__ float w_s[256], red[4], o_s[4][64];

    // (m, l) first: loads complete in order for the wait counter, so the maximum and the
    // weights need not wait for the o rows, which stay in flight through the LDS-only
    // barriers until the weighted sum
    const float* ml = a.part_ml + (base + static_cast<int64_t>(min(tid, nact - 1)) * grp) * 2;
    float m_t = ml[0];
    const float l_t = ml[1];
    float ov[kRW];
#pragma unroll
    for (int u = 0; u < kRW; ++u) ov[u] = po[min(wave * kRW + u, nact - 1) * so];
    const float gate = a.qg[static_cast<int64_t>(h) * 2 * kHD + kHD + d];
    if (tid >= nact) m_t = -INFINITY;
    float mx = m_t;
    for (int s = tid + 256; s < nact; s += 256) mx = fmaxf(mx, a.part_ml[(base + static_cast<int64_t>(s) * grp) * 2]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    lds_barrier();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float L = 0.0f, o = 0.0f;
    for (int c0 = 0; c0 < nact; c0 += 256) {
        float w = 0.0f;
        if (c0 == 0) {
            if (tid < nact) {
                w = expf(m_t - M);
                L = l_t * w;
            }
        } else if (c0 + tid < nact) {
            const int64_t i = base + static_cast<int64_t>(c0 + tid) * grp;
            w = expf(a.part_ml[i * 2] - M);
            L = fmaf(a.part_ml[i * 2 + 1], w, L);
        }
        lds_barrier();  // the previous pass's weights (and the maxima) are consumed
        w_s[tid] = w;
        lds_barrier();
        for (int c1 = 0; c1 < 256 && c0 + c1 < nact; c1 += 4 * kRW) {
            if (c0 + c1 > 0) {
#pragma unroll
                for (int u = 0; u < kRW; ++u) ov[u] = po[min(c0 + c1 + wave * kRW + u, nact - 1) * so];
            }
            // rows past the last active split carry weight 0
#pragma unroll
            for (int u = 0; u < kRW; ++u) o = fmaf(ov[u], w_s[c1 + wave * kRW + u], o);
        }
    }
    o_s[wave][lane] = o;
    L = wave_sum(L);
    if (lane == 0) red[wave] = L;
    lds_barrier();
    if (wave == 0) {
        const float Lt = (red[0] + red[1]) + (red[2] + red[3]);
        const float ot = (o_s[0][lane] + o_s[1][lane]) + (o_s[2][lane] + o_s[3][lane]);
        a.out[static_cast<int64_t>(h) * kHD + d] = (ot / Lt) * sigmoid_f(gate);
    }
}

template <int GRP>
hipError_t launch_partial_grp(const AttnDecodeArgs& a, hipStream_t s) {
    if (GRP == 8 && a.ROT % 32 == 0 && a.ROT > 0 && !attn_force_valu()) {
        dim3 grid(a.n_splits, a.NKV, a.n_layers > 0 ? a.n_layers : 1);
        auto go = [&](auto k) {
            klaunch(k, grid, kMW * 64, 0, s, a.pos_dev, a.pos_val, a.qg, a.k_new, a.v_new, a.q_norm, a.k_norm, a);
        };
        const bool ml = grid.z > 1;
        if (a.kv_bf16) ml ? go(attn_mfma_bf16_kernel<true>) : go(attn_mfma_bf16_kernel<false>);
        else ml ? go(attn_mfma4_kernel<true>) : go(attn_mfma4_kernel<false>);
        return hipGetLastError();
    }
    constexpr int LPP = GRP <= 4 ? 16 : 32;
    dim3 grid(a.n_splits, a.NKV, a.n_layers > 0 ? a.n_layers : 1);
    constexpr int BATCH = GRP <= 4 ? 8 : GRP == 8 ? 4 : 2;
    if (a.kv_bf16) klaunch(attn_partial_kernel<GRP, LPP, BATCH, (GRP <= 8), true>, grid, kWaves * 64, 0, s, a);
    else klaunch(attn_partial_kernel<GRP, LPP, BATCH, (GRP <= 8), false>, grid, kWaves * 64, 0, s, a);
    return hipGetLastError();
}

}  // namespace

// Q35_ATTN_VALU=1 keeps the vector-ALU kernel for every group size (for comparisons).
bool attn_force_valu() {
    static const bool v = [] {
        const char* e = std::getenv("Q35_ATTN_VALU");
        return e && e[0] == '1';
    }();
    return v;
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

int device_cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    return n;
}

hipError_t launch_attn_combine(const AttnDecodeArgs& a, hipStream_t s) {
    dim3 grid(a.NQ, kHD / 64, a.n_layers > 0 ? a.n_layers : 1);
    klaunch(attn_combine_kernel, grid, 256, 0, s, a.pos_dev, a.part_ml, a.part_o, a.qg, a.n_splits, a.NQ, a.NKV, a);
    return hipGetLastError();
}

}  // namespace q35k
