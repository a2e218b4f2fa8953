// Kernel-level C ABI on caller-owned device pointers: the forward_pass.h primitives
// (include/forward_pass.h:21-54) and the two decode mixers. Shapes are validated here so
// that no kernel is launched with an extent it does not support.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "../host/q35_internal.h"
#include "launch.hpp"

// Device memory of q35_attn_decode_static: the split-K partials of callers that cannot
// allocate. Every GPU the library runs on holds its own copy until the process ends. Host
// code never uses this name as an address (on the host it is only a stand-in for the
// symbol): the device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) float scratch[Q35_ATTN_STATIC_SCRATCH_BYTES / sizeof(float)];

namespace {

q35_status launched(hipError_t e, const char* what) {
    return e == hipSuccess ? Q35_OK : q35::fail(Q35_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t as_stream(q35_stream s) { return static_cast<hipStream_t>(s); }

// Device address of `scratch` on the current device (resolved at the first call on that
// device, with the device current, and kept).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

q35_status scratch_of_current_device(hipStream_t s, float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return q35::fail(Q35_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return q35::fail(Q35_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
    if (s) {
        int sdev = -1;
        e = hipStreamGetDevice(s, &sdev);
        if (e != hipSuccess) return q35::fail(Q35_ERR_HIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
        if (sdev != dev)
            return q35::fail(Q35_ERR_ARG, "the stream belongs to device %d but device %d is current", sdev, dev);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return q35::fail(Q35_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *out = static_cast<float*>(g_scratch_dev[dev]);
    return Q35_OK;
}

// Shared by q35_attn_decode (partials in the caller's workspace) and q35_attn_decode_static
// (partials in `scratch`): validates the arguments, then launches the split-K kernel and
// the combine with the partials at `part`.
q35_status attn_decode_checked(const q35_attn_decode_args* args, bool need_workspace, const char* who,
                               int* splits_out) {
    if (!args) return q35::fail(Q35_ERR_ARG, "%s: null args", who);
    const q35_attn_decode_args& g = *args;
    if (g.head_dim != 256) return q35::fail(Q35_ERR_UNSUPPORTED, "%s: head_dim must be 256", who);
    if (g.kv_heads <= 0 || g.q_heads % g.kv_heads != 0) return q35::fail(Q35_ERR_ARG, "%s: bad head counts", who);
    const int grp = g.q_heads / g.kv_heads;
    if (grp != 1 && grp != 2 && grp != 4 && grp != 8 && grp != 16)
        return q35::fail(Q35_ERR_UNSUPPORTED, "%s: GQA group %d", who, grp);
    if (g.rotary_dim < 0 || g.rotary_dim > 256 || (g.rotary_dim & 1))
        return q35::fail(Q35_ERR_ARG, "%s: rotary_dim %d", who, g.rotary_dim);
    if (g.pos < 0 || g.pos >= g.max_context)
        return q35::fail(Q35_ERR_RANGE, "%s: position %d outside [0, %lld)", who, g.pos,
                         static_cast<long long>(g.max_context));
    if (!g.qg || !g.k_new || !g.v_new || !g.q_norm || !g.k_norm || !g.k_cache || !g.v_cache || !g.out ||
        (need_workspace && !g.workspace))
        return q35::fail(Q35_ERR_ARG, "%s: null pointer", who);
    if (g.n_splits < 0 || g.n_splits > 4096) return q35::fail(Q35_ERR_ARG, "%s: n_splits %d", who, g.n_splits);
    if (g.kv_dtype != 0 && g.kv_dtype != 1) return q35::fail(Q35_ERR_ARG, "%s: kv_dtype %d", who, g.kv_dtype);
    *splits_out = g.n_splits > 0 ? g.n_splits
                                 : q35k::attn_default_splits(g.max_context, g.kv_heads * std::max(1, g.n_layers),
                                                             q35k::device_cu_count());
    return Q35_OK;
}

q35_status attn_decode_launch(const q35_attn_decode_args& g, int splits, float* part, hipStream_t st) {
    const int grp = g.q_heads / g.kv_heads;
    q35k::AttnDecodeArgs a{};
    a.NQ = g.q_heads;
    a.NKV = g.kv_heads;
    a.HD = 256;
    a.ROT = g.rotary_dim;
    a.pos_val = g.pos;
    a.max_ctx = g.max_context;
    a.n_splits = splits;
    a.theta = g.rope_theta;
    a.eps = g.eps;
    a.qg = g.qg;
    a.k_new = g.k_new;
    a.v_new = g.v_new;
    a.q_norm = g.q_norm;
    a.k_norm = g.k_norm;
    a.k_cache = g.k_cache;
    a.v_cache = g.v_cache;
    a.kv_bf16 = g.kv_dtype == 1;
    a.out = g.out;
    a.n_layers = g.n_layers > 0 ? g.n_layers : 1;
    a.part_o = part;
    a.part_ml = a.part_o + static_cast<int64_t>(a.n_layers) * g.kv_heads * splits * grp * 256;
    const q35_status r = launched(q35k::launch_attn_partial(a, st), "attn partial");
    if (r != Q35_OK) return r;
    return launched(q35k::launch_attn_combine(a, st), "attn combine");
}

}  // namespace

extern "C" {

q35_status q35_matmul_bf16(const uint16_t* W, const float* x, float* y, int32_t out_dim,
                           int32_t in_dim, q35_stream s) {
    if (!W || !x || !y || out_dim <= 0 || in_dim <= 0)
        return q35::fail(Q35_ERR_ARG, "q35_matmul_bf16: bad argument");
    if (in_dim % 8 != 0 || in_dim > q35k::kGemvMaxIn)
        return q35::fail(Q35_ERR_UNSUPPORTED, "q35_matmul_bf16: in_dim %d (needs %%8 == 0, <= %d)", in_dim,
                         q35k::kGemvMaxIn);
    if ((reinterpret_cast<uintptr_t>(W) & 15) || (reinterpret_cast<uintptr_t>(x) & 15))
        return q35::fail(Q35_ERR_ARG, "q35_matmul_bf16: W and x must be 16-byte aligned");
    if (in_dim > 16384 && q35k::gemv_enable_wide_inputs() != hipSuccess)
        return q35::fail(Q35_ERR_HIP, "q35_matmul_bf16: cannot enable %d-wide inputs", in_dim);
    q35k::GemvArgs a{};
    a.W = W;
    a.x = x;
    a.y = y;
    a.rows = out_dim;
    a.in_dim = in_dim;
    return launched(q35k::launch_gemv(a, q35k::kProPlain, as_stream(s)), "q35_matmul_bf16");
}

q35_status q35_matmul_f32(const float* W, const float* x, float* y, int32_t out_dim, int32_t in_dim,
                          q35_stream s) {
    if (!W || !x || !y || out_dim <= 0 || in_dim <= 0) return q35::fail(Q35_ERR_ARG, "q35_matmul_f32: bad argument");
    return launched(q35k::launch_matvec_f32(W, x, y, out_dim, in_dim, as_stream(s)), "q35_matmul_f32");
}

q35_status q35_gemm_bf16(const float* X, int64_t ldx, const uint16_t* W, int32_t M, int32_t N, int32_t K,
                         const float* R, int64_t ldr, float* Y, int64_t ldy, q35_stream s) {
    if (!X || !W || !Y || M <= 0 || N <= 0 || K <= 0 || ldx < K || ldy < N || (R && ldr < N))
        return q35::fail(Q35_ERR_ARG, "q35_gemm_bf16: bad argument");
    if (K % 8 != 0 || ldx % 4 != 0 || (reinterpret_cast<uintptr_t>(X) & 15) || (reinterpret_cast<uintptr_t>(W) & 15))
        return q35::fail(Q35_ERR_UNSUPPORTED, "q35_gemm_bf16: needs K %% 8 == 0, ldx %% 4 == 0, 16-byte aligned X/W");
    q35k::GemmArgs a{X, W, R, Y, M, N, K, ldx, R ? ldr : 0, ldy};
    return launched(q35k::launch_gemm(a, as_stream(s)), "q35_gemm_bf16");
}

namespace {
// workspace of q35_gemm_f16x2 (byte offsets, 256-B aligned): weight maximum, row maxima,
// the fp16 weight copy, the tiled activations
struct F16x2Plan {
    uint64_t xmax, wh, xt, bytes;
};
F16x2Plan f16x2_plan(int64_t M, int64_t N, int64_t K) {
    auto al = [](uint64_t x) { return (x + 255) / 256 * 256; };
    F16x2Plan p{};
    p.xmax = 256;
    p.wh = p.xmax + al(static_cast<uint64_t>(M) * 4);
    p.xt = p.wh + al(static_cast<uint64_t>(N) * K * 2);
    p.bytes = p.xt + al(static_cast<uint64_t>(q35k::rows_tiled(M)) * K * 4);
    return p;
}
}  // namespace

uint64_t q35_gemm_f16x2_workspace_bytes(int32_t M, int32_t N, int32_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return f16x2_plan(M, N, K).bytes;
}

q35_status q35_gemm_f16x2(const float* X, int64_t ldx, const uint16_t* W, int32_t M, int32_t N, int32_t K,
                          const float* R, int64_t ldr, float* Y, int64_t ldy, void* workspace, uint64_t workspace_bytes,
                          q35_stream s) {
    if (!X || !W || !Y || !workspace || M <= 0 || N <= 0 || K <= 0 || ldx < K || ldy < N || (R && ldr < N))
        return q35::fail(Q35_ERR_ARG, "q35_gemm_f16x2: bad argument");
    if (K % 32 != 0 || (reinterpret_cast<uintptr_t>(W) & 15) || (reinterpret_cast<uintptr_t>(workspace) & 255))
        return q35::fail(Q35_ERR_UNSUPPORTED, "q35_gemm_f16x2: needs K %% 32 == 0, 16-byte aligned W, 256-byte aligned workspace");
    const F16x2Plan p = f16x2_plan(M, N, K);
    if (workspace_bytes < p.bytes)
        return q35::fail(Q35_ERR_ARG, "q35_gemm_f16x2: workspace of %llu bytes, needs %llu",
                         static_cast<unsigned long long>(workspace_bytes), static_cast<unsigned long long>(p.bytes));
    const hipStream_t st = as_stream(s);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    unsigned* wmax = reinterpret_cast<unsigned*>(ws);
    float* xmax = reinterpret_cast<float*>(ws + p.xmax);
    uint16_t* wh = reinterpret_cast<uint16_t*>(ws + p.wh);
    float* xt = reinterpret_cast<float*>(ws + p.xt);
    const int64_t nw = static_cast<int64_t>(N) * K;
    // the weights' scale: 2^e with e = 15 - (exponent of max |w| as in frexp), as the model's
    // prefill makes its fp16 copies
    unsigned mx = 0;
    q35_status r = launched(q35k::launch_fill_f32(reinterpret_cast<float*>(wmax), 1, 0.0f, st), "q35_gemm_f16x2");
    if (r == Q35_OK) r = launched(q35k::launch_bf16_absmax(W, nw, wmax, st), "q35_gemm_f16x2");
    if (r == Q35_OK) r = launched(hipMemcpyAsync(&mx, wmax, 4, hipMemcpyDeviceToHost, st), "q35_gemm_f16x2");
    if (r == Q35_OK) r = launched(hipStreamSynchronize(st), "q35_gemm_f16x2");
    if (r != Q35_OK) return r;
    const uint32_t bits = mx << 16;
    float wm = 0.0f;
    std::memcpy(&wm, &bits, 4);
    int ex = 0;
    (void)std::frexp(wm, &ex);
    const int we = wm > 0.0f && std::isfinite(wm) ? std::min(std::max(15 - ex, -100), 100) : 0;
    r = launched(q35k::launch_bf16_to_f16(W, wh, nw, we, st), "q35_gemm_f16x2");
    if (r == Q35_OK) r = launched(q35k::launch_rows_to_tiled(X, ldx, M, K, xt, xmax, st), "q35_gemm_f16x2");
    if (r != Q35_OK) return r;
    q35k::GemmArgs g{xt, W, R, Y, M, N, K, K, R ? ldr : 0, ldy};
    g.Wh = wh;
    g.w_exp = we;
    g.xmax = xmax;
    g.xmax_n = 1;
    g.x_tiled = 1;
    return launched(q35k::launch_gemm(g, st), "q35_gemm_f16x2");
}

q35_status q35_rmsnorm(const float* x, const float* w, float* y, int32_t rows, int32_t n, float eps,
                       q35_stream s) {
    if (!x || !w || !y || rows <= 0 || n <= 0) return q35::fail(Q35_ERR_ARG, "q35_rmsnorm: bad argument");
    return launched(q35k::launch_rmsnorm_rows(x, w, y, rows, n, eps, 0, nullptr, as_stream(s)), "q35_rmsnorm");
}

q35_status q35_rmsnorm_gated(const float* x, const float* w, const float* gate, float* y, int32_t rows,
                             int32_t n, float eps, q35_stream s) {
    if (!x || !w || !gate || !y || rows <= 0 || n <= 0)
        return q35::fail(Q35_ERR_ARG, "q35_rmsnorm_gated: bad argument");
    return launched(q35k::launch_rmsnorm_rows(x, w, y, rows, n, eps, 1, gate, as_stream(s)), "q35_rmsnorm_gated");
}

q35_status q35_l2norm(float* x, int32_t rows, int32_t n, float eps, q35_stream s) {
    if (!x || rows <= 0 || n <= 0) return q35::fail(Q35_ERR_ARG, "q35_l2norm: bad argument");
    return launched(q35k::launch_l2norm_rows(x, rows, n, eps, as_stream(s)), "q35_l2norm");
}

q35_status q35_apply_rope(float* x, int32_t rows, int32_t head_dim, int32_t rotary_dim, const int32_t* pos,
                          int32_t pos0, double theta, q35_stream s) {
    if (!x || rows <= 0 || head_dim <= 0 || rotary_dim < 0 || rotary_dim > head_dim)
        return q35::fail(Q35_ERR_ARG, "q35_apply_rope: bad argument");
    return launched(q35k::launch_rope_rows(x, rows, head_dim, rotary_dim, pos, pos0, theta, as_stream(s)),
                    "q35_apply_rope");
}

q35_status q35_gdn_decode(const q35_gdn_decode_args* args, q35_stream s) {
    if (!args) return q35::fail(Q35_ERR_ARG, "q35_gdn_decode: null args");
    const q35_gdn_decode_args& g = *args;
    if (g.head_dim_k != 128 || g.head_dim_v != 128 || g.conv_kernel != 4)
        return q35::fail(Q35_ERR_UNSUPPORTED, "q35_gdn_decode: needs DK == DV == 128 and conv kernel 4");
    if (g.n_layers <= 0 || g.k_heads <= 0 || g.v_heads <= 0 || g.v_heads % g.k_heads != 0 || g.pos < 0)
        return q35::fail(Q35_ERR_ARG, "q35_gdn_decode: bad head counts or position");
    if (!g.qkv || !g.b || !g.a || !g.conv_w || !g.A_log || !g.dt_bias || !g.conv_ring || !g.state || !g.out)
        return q35::fail(Q35_ERR_ARG, "q35_gdn_decode: null pointer");
    if (g.norm_w && !g.z) return q35::fail(Q35_ERR_ARG, "q35_gdn_decode: the gated norm needs z");
    q35k::GdnDecodeArgs a{};
    a.n_layers = g.n_layers;
    a.KH = g.k_heads;
    a.VH = g.v_heads;
    a.KER = 4;
    a.pos_val = g.pos;
    a.eps = g.eps;
    a.qkv = g.qkv;
    a.z = g.z;
    a.b = g.b;
    a.a = g.a;
    a.conv_w = g.conv_w;
    a.A_log = g.A_log;
    a.dt_bias = g.dt_bias;
    a.norm_w = g.norm_w;
    a.conv_ring = g.conv_ring;
    a.state = g.state;
    a.out = g.out;
    return launched(q35k::launch_gdn_decode(a, g.norm_w != nullptr, as_stream(s)), "q35_gdn_decode");
}

uint64_t q35_attn_decode_workspace_bytes(const q35_attn_decode_args* args) {
    if (!args || args->kv_heads <= 0 || args->q_heads <= 0) return 0;
    const uint64_t layers = args->n_layers > 0 ? static_cast<uint64_t>(args->n_layers) : 1;
    const int splits = args->n_splits > 0 ? args->n_splits
                                          : q35k::attn_default_splits(args->max_context, args->kv_heads * static_cast<int>(layers),
                                                                      q35k::device_cu_count());
    return layers * static_cast<uint64_t>(q35k::attn_partial_floats(args->q_heads, args->kv_heads, args->head_dim, splits)) * 4;
}

q35_status q35_attn_decode(const q35_attn_decode_args* args, q35_stream s) {
    int splits = 0;
    const q35_status st = attn_decode_checked(args, true, "q35_attn_decode", &splits);
    if (st != Q35_OK) return st;
    const uint64_t need = q35_attn_decode_workspace_bytes(args);
    if (args->workspace_bytes < need)
        return q35::fail(Q35_ERR_ARG, "q35_attn_decode: workspace of %llu bytes, needs %llu",
                         static_cast<unsigned long long>(args->workspace_bytes), static_cast<unsigned long long>(need));
    return attn_decode_launch(*args, splits, static_cast<float*>(args->workspace), as_stream(s));
}

// The partials go to `scratch` instead of a workspace: nothing is allocated (no hipMalloc,
// no allocating library call). Every partial the combine reads is written by the same
// call's split-K kernel, so nothing needs clearing between calls.
q35_status q35_attn_decode_static(const q35_attn_decode_args* args, q35_stream s) {
    int splits = 0;
    q35_status st = attn_decode_checked(args, false, "q35_attn_decode_static", &splits);
    if (st != Q35_OK) return st;
    const uint64_t need = q35_attn_decode_workspace_bytes(args);
    if (need > Q35_ATTN_STATIC_SCRATCH_BYTES)
        return q35::fail(Q35_ERR_RANGE,
                         "q35_attn_decode_static: the split-K partials need %llu bytes, beyond the %llu of the "
                         "static scratch (use fewer splits or layers per call, or q35_attn_decode)",
                         static_cast<unsigned long long>(need),
                         static_cast<unsigned long long>(Q35_ATTN_STATIC_SCRATCH_BYTES));
    float* part = nullptr;
    st = scratch_of_current_device(as_stream(s), &part);
    if (st != Q35_OK) return st;
    return attn_decode_launch(*args, splits, part, as_stream(s));
}

uint64_t q35_gdn_prefill_workspace_bytes(const q35_gdn_prefill_args* args) {
    if (!args || args->k_heads <= 0 || args->v_heads <= 0 || args->n_tokens <= 0) return 0;
    return static_cast<uint64_t>(q35k::gdn_prefill_workspace_floats(args->k_heads, args->v_heads, args->n_tokens)) * 4;
}

q35_status q35_gdn_prefill(const q35_gdn_prefill_args* args, q35_stream s) {
    if (!args) return q35::fail(Q35_ERR_ARG, "q35_gdn_prefill: null args");
    const q35_gdn_prefill_args& g = *args;
    if (g.head_dim_k != 128 || g.head_dim_v != 128 || g.conv_kernel != 4)
        return q35::fail(Q35_ERR_UNSUPPORTED, "q35_gdn_prefill: needs DK == DV == 128 and conv kernel 4");
    if (g.n_tokens <= 0 || g.pos0 < 0 || g.k_heads <= 0 || g.v_heads <= 0 || g.v_heads % g.k_heads != 0)
        return q35::fail(Q35_ERR_ARG, "q35_gdn_prefill: bad token count, position or head counts");
    if (!g.qkv || !g.b || !g.a || !g.conv_w || !g.A_log || !g.dt_bias || !g.conv_ring || !g.state || !g.out ||
        !g.workspace)
        return q35::fail(Q35_ERR_ARG, "q35_gdn_prefill: null pointer");
    if (g.norm_w && !g.z) return q35::fail(Q35_ERR_ARG, "q35_gdn_prefill: the gated norm needs z");
    const int64_t CONV = 2LL * g.k_heads * 128 + g.v_heads * 128;
    if (g.ld_qkv < CONV || (g.z && g.ld_z < g.v_heads * 128LL) || g.ld_ba < g.v_heads)
        return q35::fail(Q35_ERR_ARG, "q35_gdn_prefill: leading dimension too small");
    // the conv pass reads qkv rows, the ring and the taps 16 bytes at a time, and carves the
    // workspace into float4-aligned arrays
    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (g.ld_qkv % 4 != 0 || !a16(g.qkv) || !a16(g.conv_ring) || !a16(g.conv_w) || !a16(g.workspace))
        return q35::fail(Q35_ERR_ARG, "q35_gdn_prefill: qkv, conv_ring, conv_w and workspace must be 16-byte aligned "
                                      "and ld_qkv a multiple of 4");
    if (g.workspace_bytes < q35_gdn_prefill_workspace_bytes(args))
        return q35::fail(Q35_ERR_ARG, "q35_gdn_prefill: workspace of %llu bytes, needs %llu",
                         static_cast<unsigned long long>(g.workspace_bytes),
                         static_cast<unsigned long long>(q35_gdn_prefill_workspace_bytes(args)));
    q35k::GdnPrefillArgs a{};
    a.T = g.n_tokens;
    a.KH = g.k_heads;
    a.VH = g.v_heads;
    a.pos0 = g.pos0;
    a.eps = g.eps;
    a.qkv = g.qkv;
    a.ld_qkv = g.ld_qkv;
    a.z = g.z;
    a.ld_z = g.ld_z;
    a.b = g.b;
    a.a = g.a;
    a.ld_ba = g.ld_ba;
    a.conv_w = g.conv_w;
    a.A_log = g.A_log;
    a.dt_bias = g.dt_bias;
    a.norm_w = g.norm_w;
    a.conv_ring = g.conv_ring;
    a.state = g.state;
    a.out = g.out;
    q35k::gdn_prefill_carve(a, static_cast<float*>(g.workspace));
    return launched(q35k::launch_gdn_prefill(a, as_stream(s)), "q35_gdn_prefill");
}

namespace {
// without the pre-split key / value tiles (the least q35_attn_prefill accepts)
uint64_t attn_prefill_min_bytes(const q35_attn_prefill_args& g) {
    return static_cast<uint64_t>(q35k::attn_prefill_workspace_floats(g.q_heads, g.n_tokens)) * 4;
}
}  // namespace

uint64_t q35_attn_prefill_workspace_bytes(const q35_attn_prefill_args* args) {
    if (!args || args->q_heads <= 0 || args->n_tokens <= 0) return 0;
    uint64_t n = attn_prefill_min_bytes(*args);
    if (args->kv_dtype == 0 && args->kv_heads > 0 && args->pos0 >= 0)
        n += static_cast<uint64_t>(q35k::attn_prefill_image_floats(args->kv_heads, args->pos0, args->n_tokens)) * 4;
    return n;
}

q35_status q35_attn_prefill(const q35_attn_prefill_args* args, q35_stream s) {
    if (!args) return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: null args");
    const q35_attn_prefill_args& g = *args;
    if (g.head_dim != 256) return q35::fail(Q35_ERR_UNSUPPORTED, "q35_attn_prefill: head_dim must be 256");
    if (g.kv_heads <= 0 || g.q_heads <= 0 || g.q_heads % g.kv_heads != 0)
        return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: bad head counts");
    if (g.rotary_dim < 0 || g.rotary_dim > 256 || (g.rotary_dim & 1))
        return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: rotary_dim %d", g.rotary_dim);
    if (g.n_tokens <= 0 || g.pos0 < 0 || g.pos0 + static_cast<int64_t>(g.n_tokens) > g.max_context)
        return q35::fail(Q35_ERR_RANGE, "q35_attn_prefill: positions [%d, %lld) outside [0, %lld)", g.pos0,
                         static_cast<long long>(g.pos0) + g.n_tokens, static_cast<long long>(g.max_context));
    if (!g.qkv || !g.q_norm || !g.k_norm || !g.k_cache || !g.v_cache || !g.out || !g.workspace)
        return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: null pointer");
    if (g.kv_dtype != 0 && g.kv_dtype != 1) return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: kv_dtype %d", g.kv_dtype);
    if (g.ld_qkv < 2LL * g.q_heads * 256 + 2LL * g.kv_heads * 256)
        return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: leading dimension too small");
    if (g.workspace_bytes < attn_prefill_min_bytes(g))
        return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: workspace of %llu bytes, needs %llu",
                         static_cast<unsigned long long>(g.workspace_bytes),
                         static_cast<unsigned long long>(attn_prefill_min_bytes(g)));
    if ((reinterpret_cast<uintptr_t>(g.workspace) & 15) != 0)
        return q35::fail(Q35_ERR_ARG, "q35_attn_prefill: workspace not 16-byte aligned");
    q35k::AttnPrefillArgs a{};
    a.T = g.n_tokens;
    a.NQ = g.q_heads;
    a.NKV = g.kv_heads;
    a.ROT = g.rotary_dim;
    a.pos0 = g.pos0;
    a.max_ctx = g.max_context;
    a.theta = g.rope_theta;
    a.eps = g.eps;
    a.qkv = g.qkv;
    a.ld_qkv = g.ld_qkv;
    a.q_norm = g.q_norm;
    a.k_norm = g.k_norm;
    a.k_cache = g.k_cache;
    a.v_cache = g.v_cache;
    a.kv_bf16 = g.kv_dtype == 1;
    a.Qa = static_cast<float*>(g.workspace);
    if (!a.kv_bf16 && g.workspace_bytes >= q35_attn_prefill_workspace_bytes(args))
        a.kv_img = a.Qa + q35k::attn_prefill_workspace_floats(a.NQ, a.T);
    a.out = g.out;
    return launched(q35k::launch_attn_prefill(a, as_stream(s)), "q35_attn_prefill");
}

}  // extern "C"
