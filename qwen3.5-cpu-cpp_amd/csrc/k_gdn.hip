// Gated-DeltaNet decode: one token through the conv window, q/k l2-normalisation, the
// decay + delta-rule update of the 128 x 128 fp32 state and the readout, for one or more
// layers in one launch (QwenModel::gdn_step after its projections,
// src/qwen_model.cpp:173-207).
//
// Work split: one 256-thread workgroup per (layer, v-head, column slice of CS state
// columns). The delta rule is column-separable -- for a state column vv,
//     S[:,vv] <- a S[:,vv];  d = (v[vv] - S[:,vv].k) b;  S[:,vv] += k d;  o[vv] = S[:,vv].q
// -- so a slice needs only k, q (shared by the head) and its own v entries. Each thread
// holds RPT = 128*CS/256 state values of one column in registers; the state is read from
// HBM once and written once, with CS consecutive floats per row (128 B for CS = 32). A
// launch of one layer uses CS = 32 (64 workgroups); a launch of many layers CS = 64.
// The two column dot products are reduced over the 256/CS row groups through LDS.
//
// Conv window: a ring of KER = 4 slots per channel in the state arena, the input of
// position t in slot t % 4. Step t reads slots (t-3..t-1) % 4 and writes slot t % 4, so
// the workgroups that share the q/k channels of a k-head can all read the window while
// one of them (v-head % rep == 0, slice 0) stores the new input, without a race.
//
// In the model's decode step the conv window already ran in the in-projection matvec's
// epilogue (conv_done): q, k and v arrive as SiLU(conv) outputs, and the ring is up to date.
// That step runs gdn_wave_kernel instead: one wave per 32-column slice, the reductions
// across lanes (DPP and the gfx950 lane swaps) instead of through LDS.
//
// With CS = 128 (one workgroup per head) the gated rmsnorm of the readout
// (src/forward_pass.cpp:86-93) is fused too; with CS = 32 the raw readout is written and
// the norm runs in the prologue of the out_proj matvec.
#include "dev_common.hpp"
#include "launch.hpp"

namespace q35k {
namespace {

constexpr int kD = 128;  // DK == DV

template <int CS, bool FUSE_NORM, bool CONVD>
__global__ __launch_bounds__(256) void gdn_decode_kernel(GdnDecodeArgs a) {
    constexpr int NSPLIT = kD / CS;
    constexpr int NRG = 256 / CS;
    constexpr int RPT = kD / NRG;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // workgroups are dispatched to the 8 XCDs in turn: in a launch of 32-column slices (one
    // layer, the decode step) with VH a multiple of 8, the slices of a head get ids of one
    // residue mod 8, so they run on one XCD and its L2 fetches the head's shared q / k rows
    // once (the 64-column launches of many layers run 6% faster without it)
    int vh, split;
    if (NSPLIT == 4 && (a.VH & 7) == 0) {
        const int xcd = blockIdx.x & 7, rest = blockIdx.x >> 3;
        split = rest % NSPLIT;
        vh = xcd + 8 * (rest / NSPLIT);
    } else {
        vh = blockIdx.x / NSPLIT;
        split = blockIdx.x - vh * NSPLIT;
    }
    const int layer = blockIdx.y;
    const int rep = a.VH / a.KH, kh = vh / rep;
    const int KD = a.KH * kD, VD = a.VH * kD, CONV = 2 * KD + VD;

    const float* qkv = a.qkv + layer * a.ls_qkv;
    const float* zin = a.z ? a.z + layer * a.ls_z : nullptr;
    const float* bin = a.b + layer * a.ls_ba;
    const float* ain = a.a + layer * a.ls_ba;
    const float* convw = a.conv_w + layer * a.ls_convw;
    const float* A_log = a.A_log + layer * a.ls_vh;
    const float* dt_bias = a.dt_bias + layer * a.ls_vh;
    float* ring = a.conv_ring + layer * a.ls_ring;
    float* S = a.state + layer * a.ls_state + static_cast<int64_t>(vh) * kD * kD;
    float* out = a.out + layer * a.ls_out;

    const int pos = a.pos_dev ? *a.pos_dev : a.pos_val;
    const int s_new = pos & 3, s_m1 = (pos + 3) & 3, s_m2 = (pos + 2) & 3, s_m3 = (pos + 1) & 3;

    __shared__ float q_s[kD], k_s[kD], v_s[CS], d_s[CS];
    __shared__ float part[NRG][CS];
    __shared__ double red[4];

    // Loads in the order they are needed (they complete in order for the wait counter): the
    // conv inputs of the 128 q, 128 k and this slice's v channels (every thread loads a v
    // channel, clamped to the slice, so no load sits under a branch), then the state slice
    // and the per-head scalars, which are first used after the l2norm. The barriers up to
    // there order LDS only, so the state loads stay in flight through the conv and the norm.
    const int chq = tid < kD ? kh * kD + tid : KD + kh * kD + (tid - kD);
    const int chv = 2 * KD + vh * kD + split * CS + (tid % CS);
    const float xq = qkv[chq];
    const float xv = qkv[chv];
    float4 wq{}, wv{};
    float rq3 = 0.f, rq2 = 0.f, rq1 = 0.f, rv3 = 0.f, rv2 = 0.f, rv1 = 0.f;
    if constexpr (!CONVD) {
        wq = *reinterpret_cast<const float4*>(convw + static_cast<int64_t>(chq) * 4);
        rq3 = ring[static_cast<int64_t>(s_m3) * CONV + chq];
        rq2 = ring[static_cast<int64_t>(s_m2) * CONV + chq];
        rq1 = ring[static_cast<int64_t>(s_m1) * CONV + chq];
        wv = *reinterpret_cast<const float4*>(convw + static_cast<int64_t>(chv) * 4);
        rv3 = ring[static_cast<int64_t>(s_m3) * CONV + chv];
        rv2 = ring[static_cast<int64_t>(s_m2) * CONV + chv];
        rv1 = ring[static_cast<int64_t>(s_m1) * CONV + chv];
    }
    const int c = tid % CS, rg = tid / CS, r0 = rg * RPT;
    float* Sc = S + split * CS + c;
    float s[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) s[i] = Sc[(r0 + i) * kD];
    const float A_v = A_log[vh], dt_v = dt_bias[vh], a_v = ain[vh], b_v = bin[vh];

    // causal conv (taps oldest first) + SiLU for the 128 q and 128 k channels of head kh ...
    {
        float y = xq;
        if constexpr (!CONVD) {
            float acc = 0.0f;
            acc += wq.x * rq3;
            acc += wq.y * rq2;
            acc += wq.z * rq1;
            acc += wq.w * xq;
            y = silu_f(acc);
            if (vh % rep == 0 && split == 0) ring[static_cast<int64_t>(s_new) * CONV + chq] = xq;
        }
        if (tid < kD) q_s[tid] = y;
        else k_s[tid - kD] = y;
    }
    // ... and for this slice's v channels
    {
        float y = xv;
        if constexpr (!CONVD) {
            float acc = 0.0f;
            acc += wv.x * rv3;
            acc += wv.y * rv2;
            acc += wv.z * rv1;
            acc += wv.w * xv;
            y = silu_f(acc);
            if (tid < CS) ring[static_cast<int64_t>(s_new) * CONV + chv] = xv;
        }
        if (tid < CS) v_s[tid] = y;
    }
    lds_barrier();

    // l2norm (eps 1e-6, sum of squares in double); q also scaled by DK^-1/2
    {
        const float v = tid < kD ? q_s[tid] : k_s[tid - kD];
        double ss = static_cast<double>(v) * v;
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        lds_barrier();
        const double sq = red[0] + red[1], sk = red[2] + red[3];
        if (tid < kD) {
            const float inv = 1.0f / sqrtf(static_cast<float>(sq) + 1e-6f);
            q_s[tid] = (v * inv) * (1.0f / sqrtf(static_cast<float>(kD)));
        } else {
            const float inv = 1.0f / sqrtf(static_cast<float>(sk) + 1e-6f);
            k_s[tid - kD] = v * inv;
        }
    }
    const float g = -expf(A_v) * softplus_f(a_v + dt_v);
    const float alpha = expf(g), beta = sigmoid_f(b_v);
    lds_barrier();

    // decay, S^T k, delta, rank-1 update, S^T q on the register-resident slice
    float km = 0.0f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        s[i] *= alpha;
        km += s[i] * k_s[r0 + i];
    }
    part[rg][c] = km;
    lds_barrier();
    if (tid < CS) {
        float t = 0.0f;
#pragma unroll
        for (int r = 0; r < NRG; ++r) t += part[r][tid];
        d_s[tid] = (v_s[tid] - t) * beta;
    }
    lds_barrier();
    const float dv = d_s[c];
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        s[i] += k_s[r0 + i] * dv;
        o += s[i] * q_s[r0 + i];
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) Sc[(r0 + i) * kD] = s[i];
    part[rg][c] = o;
    lds_barrier();

    float ov = 0.0f;
    if (tid < CS) {
#pragma unroll
        for (int r = 0; r < NRG; ++r) ov += part[r][tid];
    }
    if constexpr (FUSE_NORM) {
        // CS == 128: threads 0..127 hold the head's readout
        double ss = tid < kD ? static_cast<double>(ov) * ov : 0.0;
        ss = wave_sum(ss);
        lds_barrier();
        if (lane == 0) red[wave] = ss;
        lds_barrier();
        const double tot = red[0] + red[1];
        if (tid < kD) {
            const float inv = 1.0f / sqrtf(static_cast<float>(tot / kD) + a.eps);
            const float zz = zin[vh * kD + tid];
            out[vh * kD + tid] = a.norm_w[layer * a.ls_normw + tid] * (ov * inv) * silu_f(zz);
        }
    } else {
        if (tid < CS) out[vh * kD + split * CS + tid] = ov;
    }
}


// sum over the 8 lanes l, l ^ 8, ..., l ^ 56 (the row groups of one column quad): a DPP
// rotation by 8 within each 16-lane row, then the 16- and 32-lane swaps of gfx950
__device__ __forceinline__ float rowgroup_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    v = __builtin_bit_cast(float, static_cast<int>(r[0])) + __builtin_bit_cast(float, static_cast<int>(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, static_cast<int>(r[0])) + __builtin_bit_cast(float, static_cast<int>(r[1]));
}

// The model's decode step (inputs already convolved): one wave per (layer, v-head, slice of
// 32 state columns), no LDS and no barrier. Lane l holds rows 16 (l / 8) .. + 15 of columns
// 4 (l % 8) .. + 3 of the slice (16 float4, each row's 32 columns one 128-byte segment over 8
// lanes); the column dot products S^T k and S^T q reduce over the lane's 16 rows, then over
// the 8 row groups across lanes. Every lane forms the l2 norms of q and k itself (two
// channels each, a double-precision wave sum) and scales its own 16 rows. 3.5 us per layer
// against 4.0 us for the workgroup kernel with its five LDS barriers, same results to fp32
// rounding.
// The pointers and head counts the first loads need come first as separate arguments,
// preloaded into SGPRs at wave launch (k_gdn's build line); the per-layer strides are read
// only by launches of more than one layer.
__global__ __launch_bounds__(64) void gdn_wave_kernel(float* state, const float* qkv_in, const float* b_in,
                                                      const float* a_in, const float* A_log_in,
                                                      const float* dt_bias_in, int VH, int KH, GdnDecodeArgs a) {
    constexpr int CW = 32, RR = 16;
    const int lane = threadIdx.x;
    a.VH = VH;
    a.KH = KH;
    const int rg = lane >> 3, cq = lane & 7;
    // workgroups go to the 8 XCDs in turn: with VH a multiple of 8 the four slices of a head
    // get ids of one residue mod 8, so one L2 fetches the head's q / k rows for all four
    int vh, split;
    if ((a.VH & 7) == 0) {
        const int xcd = blockIdx.x & 7, rest = blockIdx.x >> 3;
        split = rest & 3;
        vh = xcd + 8 * (rest >> 2);
    } else {
        vh = blockIdx.x >> 2;
        split = blockIdx.x & 3;
    }
    const int layer = blockIdx.y;
    const int rep = a.VH / a.KH, kh = vh / rep;
    const int KD = a.KH * kD;
    const float *qkv = qkv_in, *bin = b_in, *ain = a_in, *A_log = A_log_in, *dt_bias = dt_bias_in;
    float* out = a.out;
    if (layer > 0) {  // uniform
        qkv += layer * a.ls_qkv;
        bin += layer * a.ls_ba;
        ain += layer * a.ls_ba;
        A_log += layer * a.ls_vh;
        dt_bias += layer * a.ls_vh;
        state += layer * a.ls_state;
        out += layer * a.ls_out;
    }
    float* S = state + static_cast<int64_t>(vh) * kD * kD;
    const int col0 = split * CW + 4 * cq;

    // inputs first, then the state slice (loads complete in order for the wait counter)
    const float A_v = A_log[vh], dt_v = dt_bias[vh], a_v = ain[vh], b_v = bin[vh];
    const float* qh = qkv + kh * kD;
    const float* kk = qkv + KD + kh * kD;
    const float2 qa = *reinterpret_cast<const float2*>(qh + 2 * lane);
    const float2 ka = *reinterpret_cast<const float2*>(kk + 2 * lane);
    float4 q4[RR / 4], k4[RR / 4];
#pragma unroll
    for (int j = 0; j < RR / 4; ++j) {
        q4[j] = *reinterpret_cast<const float4*>(qh + RR * rg + 4 * j);
        k4[j] = *reinterpret_cast<const float4*>(kk + RR * rg + 4 * j);
    }
    const float4 v4 = *reinterpret_cast<const float4*>(qkv + 2 * KD + vh * kD + col0);
    float4 s[RR];
#pragma unroll
    for (int i = 0; i < RR; ++i) s[i] = *reinterpret_cast<const float4*>(S + (RR * rg + i) * kD + col0);

    // l2norm (eps 1e-6, sums of squares in double); q also scaled by DK^-1/2
    double sq = static_cast<double>(qa.x) * qa.x + static_cast<double>(qa.y) * qa.y;
    double sk = static_cast<double>(ka.x) * ka.x + static_cast<double>(ka.y) * ka.y;
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    const float iq = 1.0f / sqrtf(static_cast<float>(sq) + 1e-6f), ik = 1.0f / sqrtf(static_cast<float>(sk) + 1e-6f);
    const float qsc = 1.0f / sqrtf(static_cast<float>(kD));
    float qn[RR], kn[RR];
#pragma unroll
    for (int j = 0; j < RR / 4; ++j) {
        qn[4 * j + 0] = (q4[j].x * iq) * qsc;
        qn[4 * j + 1] = (q4[j].y * iq) * qsc;
        qn[4 * j + 2] = (q4[j].z * iq) * qsc;
        qn[4 * j + 3] = (q4[j].w * iq) * qsc;
        kn[4 * j + 0] = k4[j].x * ik;
        kn[4 * j + 1] = k4[j].y * ik;
        kn[4 * j + 2] = k4[j].z * ik;
        kn[4 * j + 3] = k4[j].w * ik;
    }
    const float g = -expf(A_v) * softplus_f(a_v + dt_v);
    const float alpha = expf(g), beta = sigmoid_f(b_v);

    // decay, S^T k, delta, rank-1 update, S^T q
    float4 km = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RR; ++i) {
        s[i].x *= alpha;
        s[i].y *= alpha;
        s[i].z *= alpha;
        s[i].w *= alpha;
        km.x += s[i].x * kn[i];
        km.y += s[i].y * kn[i];
        km.z += s[i].z * kn[i];
        km.w += s[i].w * kn[i];
    }
    km.x = rowgroup_sum(km.x);
    km.y = rowgroup_sum(km.y);
    km.z = rowgroup_sum(km.z);
    km.w = rowgroup_sum(km.w);
    const float4 d = make_float4((v4.x - km.x) * beta, (v4.y - km.y) * beta, (v4.z - km.z) * beta, (v4.w - km.w) * beta);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RR; ++i) {
        s[i].x += kn[i] * d.x;
        s[i].y += kn[i] * d.y;
        s[i].z += kn[i] * d.z;
        s[i].w += kn[i] * d.w;
        o.x += s[i].x * qn[i];
        o.y += s[i].y * qn[i];
        o.z += s[i].z * qn[i];
        o.w += s[i].w * qn[i];
    }
#pragma unroll
    for (int i = 0; i < RR; ++i) *reinterpret_cast<float4*>(S + (RR * rg + i) * kD + col0) = s[i];
    o.x = rowgroup_sum(o.x);
    o.y = rowgroup_sum(o.y);
    o.z = rowgroup_sum(o.z);
    o.w = rowgroup_sum(o.w);
    if (rg == 0) *reinterpret_cast<float4*>(out + vh * kD + col0) = o;
}
}  // namespace

hipError_t launch_gdn_decode(const GdnDecodeArgs& in, bool fuse_norm, hipStream_t s) {
    GdnDecodeArgs a = in;
    const int64_t KD = static_cast<int64_t>(a.KH) * kD, VD = static_cast<int64_t>(a.VH) * kD;
    const int64_t CONV = 2 * KD + VD;
    if (!a.ls_qkv) a.ls_qkv = CONV;
    if (!a.ls_z) a.ls_z = VD;
    if (!a.ls_ba) a.ls_ba = a.VH;
    if (!a.ls_convw) a.ls_convw = CONV * 4;
    if (!a.ls_vh) a.ls_vh = a.VH;
    if (!a.ls_normw) a.ls_normw = kD;
    if (!a.ls_ring) a.ls_ring = CONV * 4;
    if (!a.ls_state) a.ls_state = static_cast<int64_t>(a.VH) * kD * kD;
    if (!a.ls_out) a.ls_out = VD;
    if (a.conv_done && !fuse_norm) {  // the model's decode step
        klaunch(gdn_wave_kernel, dim3(a.VH * 4, a.n_layers), 64, 0, s, a.state, a.qkv, a.b, a.a, a.A_log, a.dt_bias,
                a.VH, a.KH, a);
        return hipGetLastError();
    }
    if (fuse_norm) {
        dim3 grid(a.VH, a.n_layers);
        if (a.conv_done) klaunch(gdn_decode_kernel<128, true, true>, grid, 256, 0, s, a);
        else klaunch(gdn_decode_kernel<128, true, false>, grid, 256, 0, s, a);
    } else if (a.n_layers * a.VH * (kD / 64) >= 2 * device_cu_count()) {
        // several layers per launch: 64-column slices still give two workgroups per CU, and
        // fewer, fuller workgroups stream better (18 layers: 0.63 of HBM peak against 0.60
        // with 32 columns; 16 columns: 0.32)
        dim3 grid(a.VH * (kD / 64), a.n_layers);
        klaunch(gdn_decode_kernel<64, false, false>, grid, 256, 0, s, a);
    } else {
        dim3 grid(a.VH * (kD / 32), a.n_layers);
        klaunch(gdn_decode_kernel<32, false, false>, grid, 256, 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace q35k
