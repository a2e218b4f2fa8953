// Whole-prompt mixers (QwenForward::mix_gdn src/qwen_forward.cpp:83-152 and
// QwenForward::mix_attention src/qwen_forward.cpp:20-80), on a block of T tokens that starts
// at position pos0 and continues from the model's state (so prefill and decode hand over).
//
// Gated DeltaNet, chunked (chunk C = 64, the WY form of the gated delta rule):
//   chunk    per (v-head, chunk), from the raw projection rows: conv window + SiLU per
//            channel (the three inputs before the block come from the conv ring), l2norm of
//            q and k per token, q scaled by DK^-1/2, beta = sigmoid(b),
//            g = -exp(A_log) softplus(a + dt_bias); rows past the block (padding to whole
//            chunks) have q = k = v = 0, beta = g = 0 and change nothing. q goes head-major to
//            the workspace for the output pass. gamma = cumsum(g) in double (every decay factor
//            below is e^(a difference of gammas) rounded once: an fp32 running sum would lose
//            ~1e-6 of each exponent to cancellation, gamma reaching -40 within a chunk); the
//            chunk's e^gamma and e^(gamma_last - gamma) go to the workspace for the later passes;
//            Q K^T and K K^T on the fp32 matrix cores (the 10 lower-triangle 16 x 16 blocks);
//              P[i][j] = q_i.k_j e^(gamma_i - gamma_j)      (j <= i)
//              A[i][j] = beta_i k_i.k_j e^(gamma_i - gamma_j)  (j < i)
//              [U | W] = (I + A)^-1 [beta v | beta e^gamma k]  (forward substitution, one
//                                                               column per thread, in registers)
//   ring     the last three raw inputs of the block go to their ring slots (after the chunk
//            pass, which reads the old ones).
//   state    per (v-head, 16-column slice of the state), sequential over the chunks, on the
//            fp32 matrix cores: store the chunk-start state S_c, v_new = U - W S,
//              S <- e^(gamma_last) S + K^T (e^(gamma_last - gamma) v_new)
//            The delta rule is column-separable, so the 8 slices of a head are independent.
//   output   per (v-head, chunk), in parallel: o = e^gamma (Q S_c) + P v_new on the matrix
//            cores, then rmsnorm_gated per (token, v-head) (src/forward_pass.cpp:86-93).
// Causal attention, flash form on the bf16 matrix cores:
//   prep     q_norm + RoPE of every query row (head-major), k_norm + RoPE of every key and
//            the values appended to the KV cache at pos0 + t (angles in double; a bf16 cache
//            stores them rounded to nearest even and the flash kernel widens them back).
//   flash    grid (query tiles of 128, NQ): 8 waves of 16 query rows with their q in
//            registers (as three bf16 parts); 32-position K / V tiles in LDS (split into
//            bf16 parts when staged); S = Q K^T and O += P V on the bf16 matrix cores from
//            six part products each; running max / sum per row; epilogue O / l * sigmoid(gate).
#include <math.h>

#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

constexpr int kD = 128;   // GDN head dim
constexpr int kC = 64;    // chunk length
constexpr int kHD = 256;  // attention head dim

// ring slots of the block's last three raw inputs
__global__ __launch_bounds__(256) void gdn_ring_kernel(GdnPrefillArgs a) {
    const int KD = a.KH * kD, VD = a.VH * kD, CONV = 2 * KD + VD;
    const int t0 = a.T > 3 ? a.T - 3 : 0;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < (a.T - t0) * CONV; i += gridDim.x * 256) {
        const int t = t0 + i / CONV, ch = i % CONV;
        a.conv_ring[static_cast<int64_t>((a.pos0 + t) & 3) * CONV + ch] = a.qkv[static_cast<int64_t>(t) * a.ld_qkv + ch];
    }
}

// v_mfma_f32_16x16x4_f32, one block: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16];
// result register v of lane l is D[4 (l / 16) + v][l % 16].
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ GDN chunk
// grid (VH, Tp / 64), 256 threads: the whole chunk pass of one (v-head, chunk of 64 tokens).
//   inputs   thread (run, quad) convolves channels 4 quad .. + 3 of the head's q and k over
//            tokens 8 run .. + 7 of the chunk (eleven raw rows, 16 bytes per load), and each
//            32-lane half-wave (one run) sums a token's squares for the l2norm (in double);
//            threads 0..127 convolve v channel tid over the 64 tokens (the column they solve
//            for below); wave 0 forms beta and g, thread 0 the cumulative sum.
//   products P and A on the fp32 matrix cores over the lower triangle of 16 x 16 blocks
//            (three block pairs per wave, the last wave one), K and Q rows padded to 132
//            floats so the 16 rows x 4 dims of an operand read fall in 64 distinct banks; A
//            takes the place of Q in LDS once the products are done (68 KB in all: two
//            workgroups per CU).
//   solve    threads 0..127 the columns of beta v, 128..255 those of beta e^gamma k; step i
//            requests row i + 1 of A before it computes, so it waits once per row.
constexpr int kLdC = kD + 4;
constexpr int kLdA = kC + 4;  // A rows: 16-byte aligned, read four entries at a time
constexpr int kRun = 8;       // tokens per q / k conv run
__global__ __launch_bounds__(256, 2) void gdn_chunk_kernel(GdnPrefillArgs a) {
    const int vh = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int rep = a.VH / a.KH, kh = vh / rep;
    const int KD = a.KH * kD, VD = a.VH * kD, CONV = 2 * KD + VD;
    const int t0 = c * kC;
    const int64_t row0 = t0;
    __shared__ __align__(16) float Ks[kC][kLdC];
    __shared__ __align__(16) float QA[kC * kLdC];
    float (*Qs)[kLdC] = reinterpret_cast<float (*)[kLdC]>(QA);
    float (*As)[kLdA] = reinterpret_cast<float (*)[kLdA]>(QA);
    __shared__ double gam[kC];
    __shared__ float beta[kC], gsh[kC], edl[kC];
    // raw input of block token s (s < 0: the conv ring; s >= T: a padding row, zeroed below)
    auto xin4 = [&](int s, int ch) -> float4 {
        if (s >= 0) return *reinterpret_cast<const float4*>(a.qkv + static_cast<int64_t>(min(s, a.T - 1)) * a.ld_qkv + ch);
        return *reinterpret_cast<const float4*>(a.conv_ring + static_cast<int64_t>((a.pos0 + s) & 3) * CONV + ch);
    };
    auto xin1 = [&](int s, int ch) -> float {
        if (s >= 0) return a.qkv[static_cast<int64_t>(min(s, a.T - 1)) * a.ld_qkv + ch];
        return a.conv_ring[static_cast<int64_t>((a.pos0 + s) & 3) * CONV + ch];
    };
    // every input requested up front: q / k runs, their taps, the v column and its taps
    const int run = tid >> 5, c4 = 4 * (tid & 31);
    const int ts0 = t0 + kRun * run;
    float4 xq[kRun + 3], xk[kRun + 3];
#pragma unroll
    for (int j = 0; j < kRun + 3; ++j) {
        xq[j] = xin4(ts0 - 3 + j, kh * kD + c4);
        xk[j] = xin4(ts0 - 3 + j, KD + kh * kD + c4);
    }
    float4 wq[4], wk[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        wq[e] = *reinterpret_cast<const float4*>(a.conv_w + static_cast<int64_t>(kh * kD + c4 + e) * 4);
        wk[e] = *reinterpret_cast<const float4*>(a.conv_w + static_cast<int64_t>(KD + kh * kD + c4 + e) * 4);
    }
    float xv[kC + 3];
    float4 wv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < kD) {
        const int ch = 2 * KD + vh * kD + tid;
#pragma unroll
        for (int j = 0; j < kC + 3; ++j) xv[j] = xin1(t0 - 3 + j, ch);
        wv = *reinterpret_cast<const float4*>(a.conv_w + static_cast<int64_t>(ch) * 4);
    }
    if (tid < kC) {
        const int t = t0 + tid;
        float bb = 0.0f, gg = 0.0f;
        if (t < a.T) {
            bb = sigmoid_f(a.b[static_cast<int64_t>(t) * a.ld_ba + vh]);
            gg = -expf(a.A_log[vh]) * softplus_f(a.a[static_cast<int64_t>(t) * a.ld_ba + vh] + a.dt_bias[vh]);
        }
        beta[tid] = bb;
        gsh[tid] = gg;
    }
    // causal conv + SiLU of four channels over a run (the reference's 4-tap window,
    // src/qwen_forward.cpp:109-118)
    auto conv_run = [&](const float4 (&x)[kRun + 3], const float4 (&w)[4], float (&y)[kRun][4]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float xs[kRun + 3];
#pragma unroll
            for (int j = 0; j < kRun + 3; ++j) xs[j] = e == 0 ? x[j].x : e == 1 ? x[j].y : e == 2 ? x[j].z : x[j].w;
#pragma unroll
            for (int j = 0; j < kRun; ++j) {
                float acc = 0.0f;
                acc += w[e].x * xs[j];
                acc += w[e].y * xs[j + 1];
                acc += w[e].z * xs[j + 2];
                acc += w[e].w * xs[j + 3];
                y[j][e] = silu_f(acc);
            }
        }
    };
    {
        // q: l2norm, scaled by DK^-1/2; to LDS and (once per k-head) to the workspace
        const bool write_q = vh % rep == 0;
        const float qs = 1.0f / sqrtf(static_cast<float>(kD));
        float y[kRun][4];
        conv_run(xq, wq, y);
#pragma unroll
        for (int j = 0; j < kRun; ++j) {
            double ss = 0.0;
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += static_cast<double>(y[j][e]) * y[j][e];
            ss = half_wave_sum(ss);
            const float inv = 1.0f / sqrtf(static_cast<float>(ss) + 1e-6f);
            float4 o = make_float4((y[j][0] * inv) * qs, (y[j][1] * inv) * qs, (y[j][2] * inv) * qs, (y[j][3] * inv) * qs);
            if (ts0 + j >= a.T) o = make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<float4*>(&Qs[kRun * run + j][c4]) = o;
            if (write_q) *reinterpret_cast<float4*>(a.Qg + (static_cast<int64_t>(kh) * a.Tp + ts0 + j) * kD + c4) = o;
        }
    }
    {
        float y[kRun][4];
        conv_run(xk, wk, y);
#pragma unroll
        for (int j = 0; j < kRun; ++j) {
            double ss = 0.0;
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += static_cast<double>(y[j][e]) * y[j][e];
            ss = half_wave_sum(ss);
            const float inv = 1.0f / sqrtf(static_cast<float>(ss) + 1e-6f);
            float4 o = make_float4(y[j][0] * inv, y[j][1] * inv, y[j][2] * inv, y[j][3] * inv);
            if (ts0 + j >= a.T) o = make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<float4*>(&Ks[kRun * run + j][c4]) = o;
        }
    }
    __syncthreads();  // Q, K, beta, g in LDS
    if (tid == 0) {
        double s = 0.0;
        for (int i = 0; i < kC; ++i) {
            s += static_cast<double>(gsh[i]);
            gam[i] = s;
        }
    }
    __syncthreads();
    if (tid < kC) {
        const int64_t r = static_cast<int64_t>(vh) * a.Tp + row0 + tid;
        a.Eg[r] = expf(static_cast<float>(gam[tid]));
        edl[tid] = expf(static_cast<float>(gam[kC - 1] - gam[tid]));
    }
    // P (j <= i) and A (j < i): Q K^T and K K^T over the 128 dims for the block pairs
    // (row block r, column block b <= r) of this wave: (3,0) (3,1) (3,2) | (3,3) (2,0) (2,1) |
    // (2,2) (1,0) (1,1) | (0,0); lane (lr, lg) ends with rows 16 r + 4 lg + v of column 16 b + lr
    {
        const int pr[3] = {wave < 2 ? 3 : wave == 2 ? 2 : 0, wave == 0 ? 3 : wave == 1 ? 2 : 1,
                           wave == 0 ? 3 : wave == 1 ? 2 : 1};
        const int pb[3] = {wave == 0 ? 0 : wave == 1 ? 3 : wave == 2 ? 2 : 0, wave == 0 ? 1 : 0,
                           wave == 0 ? 2 : 1};
        const bool three = wave < 3;
        floatx4 sq[3], sk[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) sq[p] = sk[p] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int k = 0; k < kD; k += 4) {
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                if (p > 0 && !three) break;
                const float aq = Qs[16 * pr[p] + lr][k + lg], ak = Ks[16 * pr[p] + lr][k + lg];
                const float bk = Ks[16 * pb[p] + lr][k + lg];
                sq[p] = mfma4(aq, bk, sq[p]);
                sk[p] = mfma4(ak, bk, sk[p]);
            }
        }
        lds_barrier();  // every wave is done reading Q: A takes its place
        // (P blocks above the diagonal are never read and are left unwritten)
        float* P = a.P + (static_cast<int64_t>(vh) * (a.Tp / kC) + c) * kC * kC;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            if (p > 0 && !three) break;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = 16 * pr[p] + 4 * lg + v;
                const int j = 16 * pb[p] + lr;
                const float dec = j <= i ? expf(static_cast<float>(gam[i] - gam[j])) : 0.0f;
                P[i * kC + j] = j <= i ? sq[p][v] * dec : 0.0f;
                As[i][j] = j < i ? beta[i] * sk[p][v] * dec : 0.0f;
            }
        }
    }
    __syncthreads();
    // forward substitution on [beta v | beta e^gamma k], one column per thread
    float col[kC];
    if (tid < kD) {
#pragma unroll
        for (int i = 0; i < kC; ++i) {
            float acc = 0.0f;
            acc += wv.x * xv[i];
            acc += wv.y * xv[i + 1];
            acc += wv.z * xv[i + 2];
            acc += wv.w * xv[i + 3];
            const float v = t0 + i < a.T ? silu_f(acc) : 0.0f;
            col[i] = beta[i] * v;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kC; ++i) col[i] = beta[i] * expf(static_cast<float>(gam[i])) * Ks[i][tid - kD];
    }
    float4 ar[2][16];
    ar[1][0] = *reinterpret_cast<const float4*>(&As[1][0]);
#pragma unroll
    for (int i = 1; i < kC; ++i) {
        if (i + 1 < kC) {
#pragma unroll
            for (int q = 0; q < 16; ++q)
                if (4 * q < i + 1) ar[(i + 1) & 1][q] = *reinterpret_cast<const float4*>(&As[i + 1][4 * q]);
        }
        __builtin_amdgcn_sched_barrier(0);
        float x = col[i];
#pragma unroll
        for (int k = 0; k < i; ++k) x = fmaf(-ar[i & 1][k >> 2][k & 3], col[k], x);
        col[i] = x;
        __builtin_amdgcn_sched_barrier(0);
    }
    float* dst = (tid < kD ? a.U : a.W) + (static_cast<int64_t>(vh) * a.Tp + row0) * kD + (tid & (kD - 1));
#pragma unroll
    for (int i = 0; i < kC; ++i) dst[static_cast<int64_t>(i) * kD] = col[i];
    // the decayed keys of the state update, transposed: Kd[d][t] = K[t][d] e^(gamma_last - gamma_t)
    float* kd = a.Kd + (static_cast<int64_t>(vh) * (a.Tp / kC) + c) * kD * kC;
    for (int e = tid; e < kD * kC; e += 256) kd[e] = Ks[e & (kC - 1)][e >> 6] * edl[e & (kC - 1)];
}

// ------------------------------------------------------------------ GDN state scan
constexpr int kSW = 16;         // state columns per state-scan workgroup
constexpr int kLdSt = kD + 4;   // state slice in LDS, one row per state column (k contiguous)
constexpr int kLdW = kD + 4;    // W rows
constexpr int kLdKt = kC + 4;   // decayed K, transposed: one row per dim (t contiguous)
constexpr int kLdV = kC + 4;    // v_new, transposed: one row per state column

// grid (VH, 128 / kSW), 512 threads: sequential over the chunks of one state column slice.
// Per chunk: store the chunk-start state, v_new = U - W S (written over U), then
// S <- e^(gamma_last) S + (K e^(gamma_last - gamma))^T v_new. Two barriers per chunk:
//   waves 0-3   v_new rows [16 w, 16 w + 16) over all 128 dims (the dim halves [0, 64) and
//               [64, 128) in separate accumulation chains, summed in a fixed order)
//   waves 4-7   meanwhile store the next chunk's W and decayed K (requested one chunk ago)
//               into the other of two LDS buffers, and request the chunk after it
//   all waves   the new state rows [16 w, 16 w + 16)
// Operand layout: every matrix-core operand is read 16 bytes at a time. MFMA i of a 64-deep
// product takes the reduction index 16 lg + i from lane group lg (i < 16), so a lane's
// operands for four consecutive MFMAs are four consecutive floats of one LDS row: W rows and
// the state slice (stored column-major) for v_new, the decayed K (transposed by the chunk
// pass) and v_new (stored column-major) for the state update.
constexpr int kSThreads = 512;
__global__ __launch_bounds__(kSThreads) void gdn_state_kernel(GdnPrefillArgs a) {
    const int vh = blockIdx.x, cs = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int col0 = cs * kSW;
    const int nchunk = a.Tp / kC;
    const bool stager = wave >= 4;  // uniform per wave
    const int st = tid & 255;       // thread index within the half
    __shared__ __align__(16) float St[kSW][kLdSt];
    __shared__ __align__(16) float Wl[2][kC][kLdW];
    __shared__ __align__(16) float Kt[2][kD][kLdKt];
    __shared__ __align__(16) float VNt[kSW][kLdV];
    __shared__ __align__(16) float Ul[2][kC][kSW];  // the chunk's U entries of this slice
    float* S = a.state + static_cast<int64_t>(vh) * kD * kD;
    for (int i = tid; i < kD * kSW; i += kSThreads) St[i & 15][i >> 4] = S[(i >> 4) * kD + col0 + (i & 15)];

    constexpr int NF = kC * kD / 4 / 256;  // float4 of W (and of Kd) per staging thread: 8
    floatx4 rw[NF], rk[NF], ru4;
    auto load_chunk = [&](int c) {  // staging waves: the chunk's W, decayed K and U entries
        const int64_t row0 = static_cast<int64_t>(c) * kC;
        const float* W = a.W + (static_cast<int64_t>(vh) * a.Tp + row0) * kD;
        const float* Kd = a.Kd + (static_cast<int64_t>(vh) * nchunk + c) * kD * kC;
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            const int f = st + 256 * i;
            rw[i] = *reinterpret_cast<const floatx4*>(W + f * 4);
            rk[i] = *reinterpret_cast<const floatx4*>(Kd + f * 4);
        }
        // U row st / 4, columns col0 + 4 (st % 4) .. + 3
        ru4 = *reinterpret_cast<const floatx4*>(a.U + (static_cast<int64_t>(vh) * a.Tp + row0 + (st >> 2)) * kD + col0 + 4 * (st & 3));
    };
    auto store_chunk = [&](int b) {
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            const int f = st + 256 * i;
            *reinterpret_cast<floatx4*>(&Wl[b][f >> 5][(f & 31) * 4]) = rw[i];
            *reinterpret_cast<floatx4*>(&Kt[b][f >> 4][(f & 15) * 4]) = rk[i];
        }
        *reinterpret_cast<floatx4*>(&Ul[b][st >> 2][4 * (st & 3)]) = ru4;
    };
    // chunk 0 into buffer 0 (the staging waves), chunk 1 requested
    if (stager) {
        load_chunk(0);
        store_chunk(0);
        load_chunk(min(1, nchunk - 1));
    }
    // e^(gamma_last) of each chunk through the constant address space: scalar loads, whose
    // waits are on the scalar / LDS counter. (A vector load of it one chunk ahead made the
    // loop's register copy wait for every vector load in flight -- the staged chunk too --
    // at the end of each step.)
    typedef __attribute__((address_space(4))) const float cfloat;
    const cfloat* eg_last = reinterpret_cast<const cfloat*>(
        reinterpret_cast<uintptr_t>(a.Eg + static_cast<int64_t>(vh) * a.Tp + kC - 1));
    __syncthreads();  // the state slice and chunk 0 are in LDS
    for (int i = tid; i < kD * kSW; i += kSThreads)
        a.Sc[static_cast<int64_t>(vh) * nchunk * kD * kD + (i >> 4) * kD + col0 + (i & 15)] = St[i & 15][i >> 4];
    // Phase 2 of chunk c: the new state rows [16 w, 16 w + 16) -- rows 16 w + 4 lg + v of
    // column lr in this lane -- to LDS
    auto phase2 = [&](int b, float elast) {
        floatx4 sn = *reinterpret_cast<const floatx4*>(&St[lr][16 * wave + 4 * lg]);
        sn = sn * elast;
        floatx4 ch[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 ka = *reinterpret_cast<const float4*>(&Kt[b][16 * wave + lr][16 * lg + 4 * q]);
            const float4 vv = *reinterpret_cast<const float4*>(&VNt[lr][16 * lg + 4 * q]);
            ch[0] = mfma4(ka.x, vv.x, ch[0]);
            ch[1] = mfma4(ka.y, vv.y, ch[1]);
            ch[0] = mfma4(ka.z, vv.z, ch[0]);
            ch[1] = mfma4(ka.w, vv.w, ch[1]);
        }
        sn = sn + (ch[0] + ch[1]);
        *reinterpret_cast<floatx4*>(&St[lr][16 * wave + 4 * lg]) = sn;
    };
    // The two roles run separate loops with the same barriers; the staging waves only load
    // from memory and the v_new waves only store (v_new, and the chunk-start states from LDS),
    // so no wait for a load one step old also waits for the stores issued since. (One loop
    // with a branch per role made each step wait for the previous step's stores.)
    if (!stager) {
        const int vb = wave;
        for (int c = 0; c < nchunk; ++c) {
            const int b = c & 1;
            const float elast = eg_last[static_cast<int64_t>(c) * kC];
            if (c > 0) {  // the chunk-start state S_c (chunk 0's went out before the loop)
                float* Sc = a.Sc + (static_cast<int64_t>(vh) * nchunk + c) * kD * kD + col0;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int i = tid + 256 * j, row = i >> 2, q = 4 * (i & 3);  // 16 bytes of row `row`
                    *reinterpret_cast<float4*>(Sc + row * kD + q) =
                        make_float4(St[q][row], St[q + 1][row], St[q + 2][row], St[q + 3][row]);
                }
            }
            // v_new rows [16 w, 16 w + 16) over dims [0, 64) and [64, 128): four chains each
            floatx4 part[2];
#pragma unroll
            for (int kq = 0; kq < 2; ++kq) {
                floatx4 ch[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) ch[q] = floatx4{0.f, 0.f, 0.f, 0.f};
                const int k0 = 64 * kq + 16 * lg;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 wa = *reinterpret_cast<const float4*>(&Wl[b][16 * vb + lr][k0 + 4 * q]);
                    const float4 sb = *reinterpret_cast<const float4*>(&St[lr][k0 + 4 * q]);
                    ch[0] = mfma4(wa.x, sb.x, ch[0]);
                    ch[1] = mfma4(wa.y, sb.y, ch[1]);
                    ch[2] = mfma4(wa.z, sb.z, ch[2]);
                    ch[3] = mfma4(wa.w, sb.w, ch[3]);
                }
                part[kq] = (ch[0] + ch[1]) + (ch[2] + ch[3]);
            }
            float* U = a.U + (static_cast<int64_t>(vh) * a.Tp + static_cast<int64_t>(c) * kC) * kD + col0;
            floatx4 x;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                x[v] = Ul[b][16 * vb + 4 * lg + v][lr] - (part[0][v] + part[1][v]);
                U[(16 * vb + 4 * lg + v) * kD + lr] = x[v];
            }
            *reinterpret_cast<floatx4*>(&VNt[lr][16 * vb + 4 * lg]) = x;
            lds_barrier();  // VNt and the next chunk's buffer written; every v_new read of St done
            phase2(b, elast);
            lds_barrier();  // the new state rows in LDS; every read of VNt and of buffer b done
        }
    } else {
        for (int c = 0; c < nchunk; ++c) {
            const int b = c & 1;
            const float elast = eg_last[static_cast<int64_t>(c) * kC];
            // chunk c + 1, requested one step ago, into the other buffer (after the last chunk:
            // the last one again, into the buffer nothing reads any more)
            store_chunk(b ^ 1);
            load_chunk(min(c + 2, nchunk - 1));
            lds_barrier();
            phase2(b, elast);
            lds_barrier();
        }
    }
    for (int i = tid; i < kD * kSW; i += kSThreads) S[(i >> 4) * kD + col0 + (i & 15)] = St[i & 15][i >> 4];
}

// ------------------------------------------------------------------ GDN chunk output
constexpr int kLdQ = kD + 4;    // Q rows (A operand)
constexpr int kLdS = kD + 16;   // state / v_new rows (B operand)

// grid (VH, Tp / 64), 256 threads: o = e^gamma (Q S_c) + P v_new for one chunk of one v-head,
// then the gated rmsnorm (src/forward_pass.cpp:86-93, sum of squares in double) or the raw
// readout. Wave w owns output rows [16w, 16w + 16), all 128 columns (8 blocks of 16).
// S_c goes through LDS in two halves of 64 rows (71 KB of LDS, two workgroups per CU); every
// operand is requested into registers at the start, so the later phases' loads (the second
// half of S_c, P and v_new, then the epilogue's gate and norm weight) arrive while the
// earlier phases multiply.
__global__ __launch_bounds__(256, 2) void gdn_out_kernel(GdnPrefillArgs a) {
    const int vh = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int kh = vh / (a.VH / a.KH);
    const int nchunk = a.Tp / kC;
    const int64_t row0 = static_cast<int64_t>(c) * kC;
    // Operand order: within each 16-deep block of the product, MFMA step j takes from lane
    // group lg the index 4 lg + j, so a lane's four A values of the block are one 16-byte
    // read of its row; B rows are stored with their columns permuted (column 16 b + r at
    // 8 r + b), so a lane's eight column blocks of one B row are two 16-byte reads.
    __shared__ __align__(16) float A_s[kC][kLdQ];   // Q, then P
    __shared__ __align__(16) float B_s[kC][kLdS];   // S_c rows [0, 64), then [64, 128), then v_new
    __shared__ float eg[kC];  // e^gamma of the chunk's rows
    const float* Q = a.Qg + (static_cast<int64_t>(kh) * a.Tp + row0) * kD;
    const float* Sc = a.Sc + (static_cast<int64_t>(vh) * nchunk + c) * kD * kD;
    const float* P = a.P + (static_cast<int64_t>(vh) * nchunk + c) * kC * kC;
    const float* Vn = a.U + (static_cast<int64_t>(vh) * a.Tp + row0) * kD;
    constexpr int NQ4 = kC * kD / 4 / 256;  // float4 per thread of a 64 x 128 tile (8)
    constexpr int NP4 = kC * kC / 4 / 256;  // of the 64 x 64 P tile (4)
    auto put_b = [&](int f, floatx4 v) {  // float4 f of a row-major 64 x 128 tile -> B_s, permuted
        const int r = f >> 5, c0 = (f & 31) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) B_s[r][((c0 + i) & 15) * 8 + ((c0 + i) >> 4)] = v[i];
    };
    floatx4 acc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) acc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
    // acc += A[rows 16 w ..][acol .. acol + 15] . B[brow .. brow + 15][all 128 columns]
    auto mma16 = [&](int acol, int brow) {
        const float4 a4 = *reinterpret_cast<const float4*>(&A_s[16 * wave + lr][acol + 4 * lg]);
        const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4* bp = reinterpret_cast<const float4*>(&B_s[brow + 4 * lg + j][lr * 8]);
            const float4 b0 = bp[0], b1 = bp[1];
            acc[0] = mfma4(av[j], b0.x, acc[0]);
            acc[1] = mfma4(av[j], b0.y, acc[1]);
            acc[2] = mfma4(av[j], b0.z, acc[2]);
            acc[3] = mfma4(av[j], b0.w, acc[3]);
            acc[4] = mfma4(av[j], b1.x, acc[4]);
            acc[5] = mfma4(av[j], b1.y, acc[5]);
            acc[6] = mfma4(av[j], b1.z, acc[6]);
            acc[7] = mfma4(av[j], b1.w, acc[7]);
        }
    };
    // every operand is requested up front (Q and S_c[0:64) first: loads complete in order
    // for the wait counter, so the first phase waits for those alone)
    // (vector-typed register arrays: arrays of float4 structs were placed in scratch)
    floatx4 rq[NQ4], rs0[NQ4], rs[NQ4], rp[NP4], rv[NQ4];
#pragma unroll
    for (int i = 0; i < NQ4; ++i) {
        rq[i] = *reinterpret_cast<const floatx4*>(Q + (tid + 256 * i) * 4);
        rs0[i] = *reinterpret_cast<const floatx4*>(Sc + (tid + 256 * i) * 4);
    }
#pragma unroll
    for (int i = 0; i < NQ4; ++i) rs[i] = *reinterpret_cast<const floatx4*>(Sc + kC * kD + (tid + 256 * i) * 4);
#pragma unroll
    for (int i = 0; i < NP4; ++i) rp[i] = *reinterpret_cast<const floatx4*>(P + (tid + 256 * i) * 4);
#pragma unroll
    for (int i = 0; i < NQ4; ++i) rv[i] = *reinterpret_cast<const floatx4*>(Vn + (tid + 256 * i) * 4);
    const float egv = a.Eg[static_cast<int64_t>(vh) * a.Tp + row0 + (tid & (kC - 1))];
#pragma unroll
    for (int i = 0; i < NQ4; ++i) {
        const int f = tid + 256 * i;
        *reinterpret_cast<floatx4*>(&A_s[f >> 5][(f & 31) * 4]) = rq[i];
        put_b(f, rs0[i]);
    }
    if (tid < kC) eg[tid] = egv;
    lds_barrier();  // LDS only: S_c[64:128), P and v_new stay in flight
    // the epilogue's gate z (this lane's 4 rows x 8 columns) and norm weight (8 columns),
    // requested now that the Q and S_c[0:64) registers are free (unconditional loads from a
    // valid address: a raw readout reads the S_c tile and ignores it)
    const bool gated = a.norm_w != nullptr;
    float zr[4][8], nw[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int64_t t = row0 + 16 * wave + 4 * lg + v;
        const int64_t tc = t < a.T ? t : a.T - 1;  // padding rows compute but store nothing
        const float* zrow = gated ? a.z + tc * a.ld_z + vh * kD : Sc;
#pragma unroll
        for (int b = 0; b < 8; ++b) zr[v][b] = zrow[16 * b + lr];
    }
    {
        const float* nwp = gated ? a.norm_w : Sc;
#pragma unroll
        for (int b = 0; b < 8; ++b) nw[b] = nwp[16 * b + lr];
    }
#pragma unroll
    for (int blk = 0; blk < kC / 16; ++blk) mma16(16 * blk, 16 * blk);
    lds_barrier();  // done with S_c[0:64)
#pragma unroll
    for (int i = 0; i < NQ4; ++i) put_b(tid + 256 * i, rs[i]);
    lds_barrier();
#pragma unroll
    for (int blk = 0; blk < kC / 16; ++blk) mma16(kC + 16 * blk, 16 * blk);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const float e = eg[16 * wave + 4 * lg + v];
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[b][v] *= e;
    }
    lds_barrier();  // done with Q and S_c
#pragma unroll
    for (int i = 0; i < NP4; ++i) {
        const int f = tid + 256 * i;
        *reinterpret_cast<floatx4*>(&A_s[f >> 4][(f & 15) * 4]) = rp[i];
    }
#pragma unroll
    for (int i = 0; i < NQ4; ++i) put_b(tid + 256 * i, rv[i]);
    lds_barrier();
    // P is lower triangular: the row block of wave w needs columns j < 16 (w + 1)
    for (int blk = 0; blk <= wave; ++blk) mma16(16 * blk, 16 * blk);
    // epilogue: rows 16w + 4 lg + v, columns 16 b + lr
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int64_t t = row0 + 16 * wave + 4 * lg + v;
        double ss = 0.0;
#pragma unroll
        for (int b = 0; b < 8; ++b) ss += static_cast<double>(acc[b][v]) * acc[b][v];
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o);  // the 16 lanes of the row
        const float inv = 1.0f / sqrtf(static_cast<float>(ss / kD) + a.eps);
        float* out = a.out + t * (a.VH * kD) + vh * kD;
        float mx = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const int col = 16 * b + lr;
            const float y = gated ? nw[b] * (acc[b][v] * inv) * silu_f(zr[v][b]) : acc[b][v];
            mx = fmaxf(mx, fabsf(y));
            if (t < a.T) {
                if (a.out_tiled) a.out[xt_off(t, vh * kD + col, a.VH * kD)] = y;
                else out[col] = y;
            }
        }
        if (a.omax) {  // uniform: the row's maximum over this v-head's 128 columns (16 lanes)
            mx = fmaxf(mx, __shfl_xor(mx, 1));
            mx = fmaxf(mx, __shfl_xor(mx, 2));
            mx = fmaxf(mx, __shfl_xor(mx, 4));
            mx = fmaxf(mx, __shfl_xor(mx, 8));
            if (lr == 0 && t < a.T) a.omax[t * a.VH + vh] = mx;
        }
    }
}

// ------------------------------------------------------------------ attention prep
// Any even rotary width: grid (T, NQ + NKV), one thread per dim.
__global__ __launch_bounds__(256) void attn_prefill_prep_any_kernel(AttnPrefillArgs a) {
    const int t = blockIdx.x, r = blockIdx.y, d = threadIdx.x;
    const int pos = a.pos0 + t;
    __shared__ float buf[kHD];
    __shared__ float cs[2][kHD / 2];
    __shared__ double red[4];
    const float* row = a.qkv + static_cast<int64_t>(t) * a.ld_qkv;
    const float* src;
    const float* w;
    const bool is_q = r < a.NQ;
    const int kh = r - a.NQ;
    const int64_t coff = (static_cast<int64_t>(kh) * a.max_ctx + pos) * kHD;  // cache row (keys)
    if (is_q) {
        src = row + static_cast<int64_t>(r) * 2 * kHD;
        w = a.q_norm;
    } else {
        src = row + static_cast<int64_t>(a.NQ) * 2 * kHD + kh * kHD;
        w = a.k_norm;
        const float v = row[static_cast<int64_t>(a.NQ) * 2 * kHD + static_cast<int64_t>(a.NKV) * kHD + kh * kHD + d];
        if (a.kv_bf16) reinterpret_cast<uint16_t*>(a.v_cache)[coff + d] = f32_to_bf16(v);
        else a.v_cache[coff + d] = v;
    }
    const int half = a.ROT / 2;
    if (d < half) {
        const double inv_freq = pow(a.theta, -static_cast<double>(2 * d) / a.ROT);
        const double ang = static_cast<double>(pos) * inv_freq;
        cs[0][d] = static_cast<float>(cos(ang));
        cs[1][d] = static_cast<float>(sin(ang));
    }
    const float x = src[d];
    const double ss = block_sum(static_cast<double>(x) * x, red);
    const float inv = 1.0f / sqrtf(static_cast<float>(ss / kHD) + a.eps);
    float y = x * inv * (1.0f + w[d]);
    buf[d] = y;
    __syncthreads();
    if (d < a.ROT) {
        const int i = d < half ? d : d - half;
        const float c = cs[0][i], s = cs[1][i];
        const float x1 = buf[i], x2 = buf[i + half];
        y = d < half ? x1 * c - x2 * s : x2 * c + x1 * s;
    }
    if (is_q) a.Qa[(static_cast<int64_t>(r) * a.T + t) * kHD + d] = y;
    else if (a.kv_bf16) reinterpret_cast<uint16_t*>(a.k_cache)[coff + d] = f32_to_bf16(y);
    else a.k_cache[coff + d] = y;
}

// One workgroup per token, all of its rows: the NQ query rows (rmsnorm (1 + q_norm) + RoPE
// -> Qa), the NKV key rows (k_norm + RoPE -> cache) and the NKV value rows (-> cache). A row
// is 4 dims per lane of one wave (sum of squares in double); the RoPE partner dims d +- ROT/2
// come from lane +- ROT/8; cos / sin from the table or from the double-precision angle.
__global__ __launch_bounds__(256) void attn_prefill_prep_kernel(AttnPrefillArgs a) {
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = a.pos0 + t;
    const int half = a.ROT / 2, hq = a.ROT / 8;
    const float* row = a.qkv + static_cast<int64_t>(t) * a.ld_qkv;
    // cos / sin of the 4 dims of this lane (dims d mod half, lanes < ROT / 4)
    float4 cs4 = make_float4(1.f, 1.f, 1.f, 1.f), sn4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const int ci = (lane * 4) % max(half, 4);
    if (a.rope_cs) {
        const float* tb = a.rope_cs + static_cast<int64_t>(pos) * a.ROT;
        const int c0 = min(ci, max(half - 4, 0));
        cs4 = *reinterpret_cast<const float4*>(tb + c0);
        sn4 = *reinterpret_cast<const float4*>(tb + half + c0);
    } else {
        rope_cs4(a.theta, a.ROT, pos, lane, cs4, sn4);  // double-precision angles
    }
    const int nrow = a.NQ + 2 * a.NKV;
    for (int r = wave; r < nrow; r += 4) {  // uniform per wave
        if (r >= a.NQ + a.NKV) {  // value row: copied to the cache
            const int kh = r - a.NQ - a.NKV;
            const float4 v = *reinterpret_cast<const float4*>(row + static_cast<int64_t>(a.NQ) * 2 * kHD +
                                                              static_cast<int64_t>(a.NKV + kh) * kHD + lane * 4);
            const int64_t off = (static_cast<int64_t>(kh) * a.max_ctx + pos) * kHD + lane * 4;
            if (a.kv_bf16) {
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.v_cache) + off) =
                    make_uint2(f32_to_bf16(v.x) | (static_cast<uint32_t>(f32_to_bf16(v.y)) << 16),
                               f32_to_bf16(v.z) | (static_cast<uint32_t>(f32_to_bf16(v.w)) << 16));
            } else {
                *reinterpret_cast<float4*>(a.v_cache + off) = v;
            }
            continue;
        }
        const bool is_q = r < a.NQ;
        const int kh = r - a.NQ;
        const float* src = is_q ? row + static_cast<int64_t>(r) * 2 * kHD
                                : row + static_cast<int64_t>(a.NQ) * 2 * kHD + static_cast<int64_t>(kh) * kHD;
        const float4 x = *reinterpret_cast<const float4*>(src + lane * 4);
        const float4 w = *reinterpret_cast<const float4*>((is_q ? a.q_norm : a.k_norm) + lane * 4);
        double ss = static_cast<double>(x.x) * x.x + static_cast<double>(x.y) * x.y + static_cast<double>(x.z) * x.z +
                    static_cast<double>(x.w) * x.w;
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(static_cast<float>(ss / kHD) + a.eps);
        float4 y;
        y.x = x.x * inv * (1.0f + w.x);
        y.y = x.y * inv * (1.0f + w.y);
        y.z = x.z * inv * (1.0f + w.z);
        y.w = x.w * inv * (1.0f + w.w);
        const int srcl = lane < hq ? lane + hq : lane - hq;
        float4 o;
        o.x = __shfl(y.x, srcl);
        o.y = __shfl(y.y, srcl);
        o.z = __shfl(y.z, srcl);
        o.w = __shfl(y.w, srcl);
        if (lane < hq) {
            y.x = y.x * cs4.x - o.x * sn4.x;
            y.y = y.y * cs4.y - o.y * sn4.y;
            y.z = y.z * cs4.z - o.z * sn4.z;
            y.w = y.w * cs4.w - o.w * sn4.w;
        } else if (lane < 2 * hq) {
            y.x = y.x * cs4.x + o.x * sn4.x;
            y.y = y.y * cs4.y + o.y * sn4.y;
            y.z = y.z * cs4.z + o.z * sn4.z;
            y.w = y.w * cs4.w + o.w * sn4.w;
        }
        if (is_q) {
            *reinterpret_cast<float4*>(a.Qa + (static_cast<int64_t>(r) * a.T + t) * kHD + lane * 4) = y;
        } else {
            const int64_t off = (static_cast<int64_t>(kh) * a.max_ctx + pos) * kHD + lane * 4;
            if (a.kv_bf16) {
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.k_cache) + off) =
                    make_uint2(f32_to_bf16(y.x) | (static_cast<uint32_t>(f32_to_bf16(y.y)) << 16),
                               f32_to_bf16(y.z) | (static_cast<uint32_t>(f32_to_bf16(y.w)) << 16));
            } else {
                *reinterpret_cast<float4*>(a.k_cache + off) = y;
            }
        }
    }
}

// ------------------------------------------------------------------ flash attention
constexpr int kFW = 8;            // waves per workgroup
constexpr int kQT = 16 * kFW;     // query rows per workgroup (16 per wave)
constexpr int kKT = 32;           // keys per tile
constexpr float kLog2e = 1.44269504088896341f;

// 128 query rows of one head per workgroup (16 per wave), causal, keys of earlier blocks from
// the cache, 32-key tiles staged through LDS (the next tile's rows are loaded into registers
// while the current one is multiplied), online softmax. One workgroup per CU (112 KB of LDS
// with three parts); causal work grows with the query block, and workgroups are dispatched
// in linear order, so block L takes the L-th longest item (query blocks from the last).
// Both products run on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16): every fp32 operand
// is the exact sum of three bf16 parts (hi + mid + lo, as in the bf16 path of the projection GEMM), and a
// product a.b is the sum of the six part products a_i b_j with i + j <= 2 (parts counted
// from 0): the three dropped ones (mid.lo, lo.mid, lo.lo) are below 2^-23 |a||b| together,
// the size of an fp32 rounding, and each bf16 x bf16 part product is exact in fp32. A bf16
// cache holds K and V exactly, so only Q and P are split (three products each).
//   S^T = K Q^T per 16-key half of the tile: keys as rows (K parts from LDS, 8 consecutive
//         dims per lane), the lane's own query row as the column (Q parts in registers, split
//         once); lane (r16, g) ends with keys 4g + v of each half for query r16.
//   O += P V, 32 keys deep: those eight scores are the A operand (query r16) without data
//         movement, taking the k slots 8g .. 8g + 7 of the product as keys 4g .. 4g + 3 of the
//         first half and of the second; the dim-major V rows in LDS store the keys in that
//         order (one 16-byte read per lane and dim block); lane (r16, g) ends with dims
//         16t + r16 of queries 4g + v. (16-key tiles would need the 16-deep bf16 product,
//         which the gfx950 matrix cores run at half the 32-deep one's rate.)
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// the three bf16 parts of four floats, each part as four packed bf16 (element 0 low)
__device__ __forceinline__ void split3_4(const float (&x)[4], uint2 (&part)[3]) {
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split3(x[e], h[e], m[e], l[e]);
    part[0] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    part[1] = make_uint2(m[0] | (m[1] << 16), m[2] | (m[3] << 16));
    part[2] = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
}

// eight floats as three 16-byte chunks, the exact bf16 parts of each (elements 0..7 in order)
__device__ __forceinline__ void split3_8(const float (&x)[8], uint4 (&c)[3]) {
    const float lo[4] = {x[0], x[1], x[2], x[3]}, hi[4] = {x[4], x[5], x[6], x[7]};
    uint2 p0[3], p1[3];
    split3_4(lo, p0);
    split3_4(hi, p1);
#pragma unroll
    for (int p = 0; p < 3; ++p) c[p] = make_uint4(p0[p].x, p0[p].y, p1[p].x, p1[p].y);
}

// The flash kernel's LDS image of one 32-key tile of an fp32 cache: K chunks Kc[3][2][32][16]
// then V chunks Vc[3][16][4][16] (the layouts described at that kernel), 16-byte chunks.
constexpr int kImgK = 3 * 2 * (kHD / 8) * 16;
constexpr int kImgTile = 2 * kImgK;
// key of slot 8 g + j of a V chunk: keys 4 g .. + 3 of the tile's first half, then the same
// four of its second half
__device__ __forceinline__ int vslot_key(int g, int j) { return (j < 4 ? 0 : 12) + 4 * g + j; }

// grid (tiles, NKV), 256 threads: writes the LDS image of every tile of keys [0, pos0 + T) of
// one kv head (rows past the last key are copies of it), so that the flash kernel stages a
// tile by a plain copy instead of splitting it again in every query-block workgroup.
__global__ __launch_bounds__(256) void attn_kv_image_kernel(AttnPrefillArgs a) {
    const int ti = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x;
    const int last = a.pos0 + a.T - 1;
    const int64_t hoff = static_cast<int64_t>(kh) * a.max_ctx * kHD;
    uint4* img = static_cast<uint4*>(a.kv_img) + (static_cast<int64_t>(kh) * gridDim.x + ti) * kImgTile;
    // K chunk (key, dims 8 dc ..): lanes walk the dim chunks of one key
    for (int e = tid; e < kKT * (kHD / 8); e += 256) {
        const int key = e >> 5, dc = e & 31;
        const float* src = a.k_cache + hoff + static_cast<int64_t>(min(ti * kKT + key, last)) * kHD + 8 * dc;
        const float4 u = *reinterpret_cast<const float4*>(src), w = *reinterpret_cast<const float4*>(src + 4);
        const float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
        uint4 c[3];
        split3_8(x, c);
#pragma unroll
        for (int p = 0; p < 3; ++p) img[((p * 2 + (key >> 4)) * (kHD / 8) + dc) * 16 + (key & 15)] = c[p];
    }
    // V chunk (dim d, slot chunk g): lanes walk the dims of the same eight keys
    for (int e = tid; e < kHD * 4; e += 256) {
        const int d = e & (kHD - 1), g = e >> 8;
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            x[j] = a.v_cache[hoff + static_cast<int64_t>(min(ti * kKT + vslot_key(g, j), last)) * kHD + d];
        uint4 c[3];
        split3_8(x, c);
#pragma unroll
        for (int p = 0; p < 3; ++p) img[kImgK + ((p * (kHD / 16) + (d >> 4)) * 4 + g) * 16 + ((d & 15) ^ (4 * g))] = c[p];
    }
}

// IMG (fp32 cache only): tiles are copied from the image attn_kv_image_kernel wrote.
template <bool KVB, bool IMG>
__global__ __launch_bounds__(kFW * 64, 1) void flash_attn_kernel(AttnPrefillArgs a) {
    static_assert(!(KVB && IMG), "the tile image holds the parts of an fp32 cache");
    constexpr int NP = KVB ? 1 : 3;  // parts of K and V
    const int nqt = gridDim.x;
    const int rank = blockIdx.x + blockIdx.y * nqt;
    const int qt = nqt - 1 - rank / a.NQ, h = rank % a.NQ;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = a.NQ / a.NKV, kh = h / grp;
    const int t0 = qt * kQT;
    const int r16 = lane & 15, g4 = lane >> 4;
    // LDS in 16-byte chunks (8 bf16) so that the 16 lanes of a lane group read one whole
    // 256-byte row of 16 chunks (any order within the row runs at full rate; rows of padded
    // or scattered chunks at 0.6 of it): K chunk (key, dims 8 dc ..) at Kc[p][key / 16][dc]
    // [key % 16], V chunk (dim, key slots 8 g ..) at Vc[p][dim / 16][g][(dim % 16) ^ 4 g]
    // (the XOR puts the 8 lanes of each staging store on distinct banks).
    __shared__ __align__(16) uint4 Kc[NP][2][kHD / 8][16];
    __shared__ __align__(16) uint4 Vc[NP][kHD / 16][4][16];
    const float sc = 1.0f / sqrtf(static_cast<float>(kHD));

    // this lane's query row, dims 32c + 8 g4 .. + 7, as three bf16 parts (the B operand)
    const int qrow = t0 + wave * 16 + r16;
    bf16x8 qp[3][8];
    {
        const float* src = a.Qa + (static_cast<int64_t>(h) * a.T + min(qrow, a.T - 1)) * kHD + 8 * g4;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 x0 = *reinterpret_cast<const float4*>(src + 32 * c);
            const float4 x1 = *reinterpret_cast<const float4*>(src + 32 * c + 4);
            const float v0[4] = {x0.x, x0.y, x0.z, x0.w}, v1[4] = {x1.x, x1.y, x1.z, x1.w};
            uint2 p0[3], p1[3];
            split3_4(v0, p0);
            split3_4(v1, p1);
#pragma unroll
            for (int p = 0; p < 3; ++p)
                qp[p][c] = __builtin_bit_cast(bf16x8, make_uint4(p0[p].x, p0[p].y, p1[p].x, p1[p].y));
        }
    }
    const int qpos = a.pos0 + qrow;
    // the wave's last query position: tiles starting past it hold no key its rows attend
    const int wlast = a.pos0 + min(t0 + wave * 16 + 15, a.T - 1);
    floatx4 o[16];  // dims 16 t + r16 of query rows 4 g4 + v
#pragma unroll
    for (int t = 0; t < 16; ++t) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;

    const int kv_end = a.pos0 + min(a.T, t0 + kQT);
    const int64_t hoff = static_cast<int64_t>(kh) * a.max_ctx * kHD;
    // staging of one tile, in registers while the previous tile is multiplied: K key
    // 8 (wave % 4) + lane % 8, dim chunks 8 c + lane / 8 for c = 2 (wave / 4) + i, i < 2 (two
    // float4 each); V dims 2 (tid / 4), + 1 of the eight keys of slot chunk g = tid % 4 (keys
    // 4 g .. + 3 and 16 + 4 g .. + 3, one float2 each); split (or widened) when stored to LDS
    const int ks_row = 8 * (wave & 3) + (lane & 7), ks_c0 = 16 * (wave >> 2) + (lane >> 3);
    const int vs_g = tid & 3, vs_d = (tid >> 2) * 2;
    float4 kst[IMG ? 1 : 4];
    float2 vst[IMG ? 1 : 8];
    // (vector-typed: an array of uint4 structs here was placed in scratch memory)
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 ist[IMG ? kImgTile / (kFW * 64) : 1];
    auto vkey = [&](int j) { return vslot_key(vs_g, j); };
    auto load_tile = [&](int kv0) {
        if constexpr (IMG) {  // tiles past the block's keys: the last one again (in the image)
            const u32x4* src = static_cast<const u32x4*>(a.kv_img) +
                               (static_cast<int64_t>(kh) * a.img_tiles + min(kv0, kv_end - 1) / kKT) * kImgTile;
#pragma unroll
            for (int j = 0; j < kImgTile / (kFW * 64); ++j) ist[j] = src[tid + kFW * 64 * j];
            return;
        }
        const bool live = kv0 < kv_end;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int pk = min(kv0 + ks_row, kv_end - 1);
            const int64_t ok = live ? static_cast<int64_t>(pk) * kHD + 8 * (ks_c0 + 8 * (j >> 1)) + 4 * (j & 1) : 0;
            if constexpr (KVB) {
                const uint2 kb = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.k_cache) + hoff + ok);
                kst[j] = make_float4(bf16_lo(kb.x), bf16_hi(kb.x), bf16_lo(kb.y), bf16_hi(kb.y));
            } else {
                kst[j] = *reinterpret_cast<const float4*>(a.k_cache + hoff + ok);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int pv = min(kv0 + vkey(j), kv_end - 1);
            const int64_t ov = live ? static_cast<int64_t>(pv) * kHD + vs_d : 0;
            if constexpr (KVB) {
                const uint32_t vb = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(a.v_cache) + hoff + ov);
                vst[j] = make_float2(bf16_lo(vb), bf16_hi(vb));
            } else {
                vst[j] = *reinterpret_cast<const float2*>(a.v_cache + hoff + ov);
            }
        }
    };
    // eight floats as NP 16-byte chunks: three exact bf16 parts, or (a bf16 cache) the values
    auto parts8 = [&](const float (&x)[8], uint4 (&c)[NP]) {
        if constexpr (KVB) {
            c[0] = make_uint4(__float_as_uint(x[0]) >> 16 | (__float_as_uint(x[1]) & 0xffff0000u),
                              __float_as_uint(x[2]) >> 16 | (__float_as_uint(x[3]) & 0xffff0000u),
                              __float_as_uint(x[4]) >> 16 | (__float_as_uint(x[5]) & 0xffff0000u),
                              __float_as_uint(x[6]) >> 16 | (__float_as_uint(x[7]) & 0xffff0000u));
        } else {
            split3_8(x, c);
        }
    };
    // Rows past the end of the keys are copies of the last one (finite): their scores are
    // masked to -inf, so their weights are exactly 0 and 0 * V adds nothing.
    auto store_tile = [&]() {
        if constexpr (IMG) {  // the image is the two arrays' contents, chunk for chunk
            constexpr int NJ = kImgTile / (kFW * 64);
#pragma unroll
            for (int j = 0; j < NJ / 2; ++j) reinterpret_cast<u32x4*>(&Kc[0][0][0][0])[tid + kFW * 64 * j] = ist[j];
#pragma unroll
            for (int j = 0; j < NJ / 2; ++j) reinterpret_cast<u32x4*>(&Vc[0][0][0][0])[tid + kFW * 64 * j] = ist[NJ / 2 + j];
            return;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float4 u = kst[2 * i], w = kst[2 * i + 1];
            const float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
            uint4 c[NP];
            parts8(x, c);
#pragma unroll
            for (int p = 0; p < NP; ++p) Kc[p][ks_row >> 4][ks_c0 + 8 * i][ks_row & 15] = c[p];
        }
        // V, dim-major: dims vs_d, vs_d + 1 get the eight keys of slot chunk vs_g
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = e ? vst[j].y : vst[j].x;
            uint4 c[NP];
            parts8(x, c);
            const int d = vs_d + e;
#pragma unroll
            for (int p = 0; p < NP; ++p) Vc[p][d >> 4][vs_g][(d & 15) ^ (4 * vs_g)] = c[p];
        }
    };
    load_tile(0);
    store_tile();
    lds_barrier();
    for (int kv0 = 0; kv0 < kv_end; kv0 += kKT) {
        load_tile(kv0 + kKT);  // in flight during this tile's products
        if (kv0 <= wlast) {    // uniform per wave
            // S^T[key 16 hf + 4 g4 + v][query r16]: the hi.hi products and the smaller part
            // products in separate accumulators, each split over even / odd dim blocks
            floatx4 St[2];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                floatx4 sa[2], sb[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) sa[e] = sb[e] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    bf16x8 kop[NP];
#pragma unroll
                    for (int p = 0; p < NP; ++p)
                        kop[p] = __builtin_bit_cast(bf16x8, Kc[p][hf][4 * c + g4][r16]);
                    floatx4& b = sb[c & 1];
                    if constexpr (KVB) {
                        b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[0], qp[2][c], b, 0, 0, 0);
                        b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[0], qp[1][c], b, 0, 0, 0);
                    } else {
                        b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[2 % NP], qp[0][c], b, 0, 0, 0);
                        b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[1 % NP], qp[1][c], b, 0, 0, 0);
                        b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[0], qp[2][c], b, 0, 0, 0);
                        b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[1 % NP], qp[0][c], b, 0, 0, 0);
                        b = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[0], qp[1][c], b, 0, 0, 0);
                    }
                    sa[c & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[0], qp[0][c], sa[c & 1], 0, 0, 0);
                }
                St[hf] = (sb[0] + sb[1]) + (sa[0] + sa[1]);
            }
            float sv[8];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int key = kv0 + 16 * hf + 4 * g4 + v;
                    sv[4 * hf + v] = key <= qpos && key < kv_end ? St[hf][v] * sc : -INFINITY;
                }
            float tm = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) tm = fmaxf(tm, sv[i]);
            tm = fmaxf(tm, __shfl_xor(tm, 16));
            tm = fmaxf(tm, __shfl_xor(tm, 32));
            // the reference max moves only when a score exceeds it by more than 8; a row with
            // no key yet keeps -inf and weight 0
            const float m_new = tm > m_run + 8.0f ? tm : m_run;
            const bool live = m_new != -INFINITY;
            // e^y as the native 2^(y log2 e): y = score - max is formed exactly as before, so
            // the product's rounding moves a weight by |y| 2^-24 relative (1 ulp of v_exp_f32
            // besides), negligible where the weights are large
            const float f = live ? __builtin_amdgcn_exp2f((m_run - m_new) * kLog2e) : 1.0f;
            float p[8], ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                p[i] = live ? __builtin_amdgcn_exp2f((sv[i] - m_new) * kLog2e) : 0.0f;
                ps += p[i];
            }
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            l_run = l_run * f + ps;
            m_run = m_new;
            if (__any(f != 1.0f)) {  // rescale output rows 4 g4 + r
                float fr[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) fr[rr] = __shfl(f, 4 * g4 + rr);
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    o[t][0] *= fr[0];
                    o[t][1] *= fr[1];
                    o[t][2] *= fr[2];
                    o[t][3] *= fr[3];
                }
            }
            // O[query 4 g4 + v][dim 16 t + r16] += P[query][keys] V[keys][dim], k slots
            // 8 g4 .. + 7 = keys 4 g4 .. + 3 of both halves
            bf16x8 pa[3];
            {
                const float p0[4] = {p[0], p[1], p[2], p[3]}, p1[4] = {p[4], p[5], p[6], p[7]};
                uint2 q0[3], q1[3];
                split3_4(p0, q0);
                split3_4(p1, q1);
#pragma unroll
                for (int q = 0; q < 3; ++q) pa[q] = __builtin_bit_cast(bf16x8, make_uint4(q0[q].x, q0[q].y, q1[q].x, q1[q].y));
            }
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                bf16x8 vb[NP];
#pragma unroll
                for (int q = 0; q < NP; ++q) vb[q] = __builtin_bit_cast(bf16x8, Vc[q][t][g4][r16 ^ (4 * g4)]);
                // the part products straight into the running output, smallest first
                if constexpr (KVB) {
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[2], vb[0], o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[1], vb[0], o[t], 0, 0, 0);
                } else {
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[2], vb[0], o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[1], vb[1 % NP], o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[0], vb[2 % NP], o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[1], vb[0], o[t], 0, 0, 0);
                    o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[0], vb[1 % NP], o[t], 0, 0, 0);
                }
                o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[0], vb[0], o[t], 0, 0, 0);
            }
        }
        lds_barrier();  // every wave is done with this tile
        if (kv0 + kKT < kv_end) {
            store_tile();
            lds_barrier();
        }
    }
    float lr[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) lr[rr] = __shfl(l_run, 4 * g4 + rr);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const int t = t0 + wave * 16 + 4 * g4 + rr;
        const int tc = min(t, a.T - 1);  // rows past the block compute but store nothing
        const float inv = 1.0f / lr[rr];
        const float* gate = a.qkv + static_cast<int64_t>(tc) * a.ld_qkv + static_cast<int64_t>(h) * 2 * kHD + kHD;
        float* out = a.out + static_cast<int64_t>(t) * (a.NQ * kHD) + static_cast<int64_t>(h) * kHD;
        float mx = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
            const int dd = 16 * tt + r16;
            const float y = (o[tt][rr] * inv) * sigmoid_f(gate[dd]);
            mx = fmaxf(mx, fabsf(y));
            if (t < a.T) {
                if (a.out_tiled) a.out[xt_off(t, h * kHD + dd, a.NQ * kHD)] = y;
                else out[dd] = y;
            }
        }
        if (a.omax) {  // uniform: the row's maximum over this head's 256 dims (16 lanes)
            mx = fmaxf(mx, __shfl_xor(mx, 1));
            mx = fmaxf(mx, __shfl_xor(mx, 2));
            mx = fmaxf(mx, __shfl_xor(mx, 4));
            mx = fmaxf(mx, __shfl_xor(mx, 8));
            if (r16 == 0 && t < a.T) a.omax[static_cast<int64_t>(t) * a.NQ + h] = mx;
        }
    }
}

// ------------------------------------------------------------------ small prefill helpers
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint16_t* embed, const int* ids, float* hidden, int T,
                                                         int H) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < static_cast<int64_t>(T) * H;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t t = i / H, c = i % H;
        hidden[i] = bf16_to_f32(embed[static_cast<int64_t>(ids[t]) * H + c]);
    }
}

int blocks_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return static_cast<int>(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

}  // namespace

int64_t gdn_prefill_workspace_floats(int KH, int VH, int T) {
    const int64_t Tp = (T + kC - 1) / kC * kC;
    return (KH + 2 * static_cast<int64_t>(VH)) * Tp * kD  // Qg U W
           + static_cast<int64_t>(VH) * Tp                 // Eg
           + static_cast<int64_t>(VH) * Tp * kD            // Kd
           + static_cast<int64_t>(VH) * Tp * kC            // P
           + static_cast<int64_t>(VH) * (Tp / kC) * kD * kD  // Sc (chunk-start states)
           + 64 * 6;                                       // alignment slack
}

void gdn_prefill_carve(GdnPrefillArgs& a, float* ws) {
    a.Tp = (a.T + kC - 1) / kC * kC;
    auto take = [&](int64_t n) {
        float* p = ws;
        ws += (n + 63) / 64 * 64;
        return p;
    };
    a.Qg = take(static_cast<int64_t>(a.KH) * a.Tp * kD);
    a.U = take(static_cast<int64_t>(a.VH) * a.Tp * kD);
    a.W = take(static_cast<int64_t>(a.VH) * a.Tp * kD);
    a.Eg = take(static_cast<int64_t>(a.VH) * a.Tp);
    a.Kd = take(static_cast<int64_t>(a.VH) * a.Tp * kD);
    a.P = take(static_cast<int64_t>(a.VH) * a.Tp * kC);
    a.Sc = take(static_cast<int64_t>(a.VH) * (a.Tp / kC) * kD * kD);
}

hipError_t launch_gdn_prefill(GdnPrefillArgs& a, hipStream_t s) {
    klaunch(gdn_chunk_kernel, dim3(a.VH, a.Tp / kC), 256, 0, s, a);
    klaunch(gdn_ring_kernel, blocks_for(3 * (2 * a.KH * kD + a.VH * kD)), 256, 0, s, a);
    klaunch(gdn_state_kernel, dim3(a.VH, kD / kSW), kSThreads, 0, s, a);
    klaunch(gdn_out_kernel, dim3(a.VH, a.Tp / kC), 256, 0, s, a);
    return hipGetLastError();
}

int64_t attn_prefill_workspace_floats(int NQ, int T) { return static_cast<int64_t>(NQ) * T * kHD + 64; }
int attn_prefill_image_tiles(int pos0, int T) { return (pos0 + T + kKT - 1) / kKT; }
int64_t attn_prefill_image_floats(int NKV, int pos0, int T) {
    return static_cast<int64_t>(NKV) * attn_prefill_image_tiles(pos0, T) * kImgTile * 4;
}

hipError_t launch_attn_prefill(const AttnPrefillArgs& in, hipStream_t s) {
    AttnPrefillArgs a = in;
    if (a.ROT % 8 == 0) klaunch(attn_prefill_prep_kernel, a.T, 256, 0, s, a);
    else klaunch(attn_prefill_prep_any_kernel, dim3(a.T, a.NQ + a.NKV), 256, 0, s, a);
    const dim3 grid((a.T + kQT - 1) / kQT, a.NQ);
    if (a.kv_bf16) {
        klaunch(flash_attn_kernel<true, false>, grid, kFW * 64, 0, s, a);
    } else if (a.kv_img) {
        a.img_tiles = attn_prefill_image_tiles(a.pos0, a.T);
        klaunch(attn_kv_image_kernel, dim3(a.img_tiles, a.NKV), 256, 0, s, a);
        klaunch(flash_attn_kernel<false, true>, grid, kFW * 64, 0, s, a);
    } else {
        klaunch(flash_attn_kernel<false, false>, grid, kFW * 64, 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_embed_rows(const uint16_t* embed, const int* ids, float* hidden, int T, int H, hipStream_t s) {
    klaunch(embed_rows_kernel, blocks_for(static_cast<int64_t>(T) * H), 256, 0, s, embed, ids, hidden, T, H);
    return hipGetLastError();
}

}  // namespace q35k
