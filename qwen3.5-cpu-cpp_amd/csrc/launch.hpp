#pragma once
// Host-side launchers of the gfx950 kernels. Each returns the hipError_t of its launch.
// Shapes are checked by the callers (c_api_kernels.hip, runtime.hip) before launching.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace q35k {

// Per-launch timing of a host thread. While launch_timer() is set, every launch records the
// kernel's own start (first launch) and end (every launch) in the two events, through
// hipExtLaunchKernelGGL: the events take the dispatch's begin / end timestamps, so the host
// and queue overheads between launches are not counted (what a kernel trace reports).
struct LaunchTimer {
    hipEvent_t start = nullptr, stop = nullptr;
    bool started = false;
};
LaunchTimer*& launch_timer();

template <typename... KArgs, typename... Args>
inline void klaunch(void (*k)(KArgs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Args... args) {
    if (LaunchTimer* t = launch_timer()) {
        hipExtLaunchKernelGGL(k, grid, block, lds, s, t->started ? nullptr : t->start, t->stop, 0u,
                              static_cast<KArgs>(args)...);
        t->started = true;
    } else {
        k<<<grid, block, lds, s>>>(static_cast<KArgs>(args)...);
    }
}

// ---------------------------------------------------------------- bf16 x fp32 matvec
// y[r] = (resid ? resid[r] : 0) + sum_i W[r][i] * x'[i] for r < rows, where x' is the input
// after the prologue:
enum GemvPrologue : int {
    kProPlain = 0,      // x' = x
    kProRmsNorm = 1,    // x' = x * rsqrt(mean(x^2) + eps) * (1 + norm_w)     (input norms)
    kProSwiGlu = 2,     // x' = silu(x[i]) * x[in_dim + i]                     (FFN down)
    kProGatedNorm = 3,  // x' = norm_w[i % hd] * (x * rsqrt(mean_head(x^2)+eps)) * silu(gate)
};
struct GemvArgs {
    const uint16_t* W;  // [rows][in_dim] bf16, 16-byte aligned rows (in_dim % 8 == 0)
    const float* x;
    const float* norm_w;
    const float* gate;
    const float* resid;  // may alias y
    float* y;
    int rows, in_dim, head_dim;
    float eps;
    // kEpiConvSilu: rows [0, conv_rows) are the GDN conv channels; the epilogue runs their
    // causal conv window (conv_w [conv_rows][4], ring [4][conv_rows], slot = position % 4 at
    // *pos_dev) and stores SiLU of it, and writes the raw projection into the ring
    const float* conv_w;
    float* conv_ring;
    const int* pos_dev;
    int conv_rows;
    // kProRmsNorm input from the embedding: x = bf16 row *token of embed (in_dim wide) in
    // place of x, and workgroup 0 stores it to x_out (the residual stream of the step)
    const uint16_t* embed = nullptr;
    const int* token = nullptr;
    float* x_out = nullptr;
    // kEpiStore: each workgroup also writes the largest output it stored and its row (the
    // first row of that value; NaN never wins): values amax_part[0 .. blocks), then the rows
    // as ints. The grid is gemv_blocks(); it is capped at kArgmaxParts when this is set.
    float* amax_part = nullptr;
};
// Epilogue: store y, add the residual (the default when resid is set), or, for an
// interleaved [gate_0; up_0; gate_1; up_1; ...] matrix, y[i] = silu(row 2i) * row 2i+1, or
// the GDN in-projection's conv window + SiLU on its conv rows (kEpiConvSilu).
enum GemvEpilogue : int { kEpiAuto = -1, kEpiStore = 0, kEpiResidual = 1, kEpiSwiGluPair = 2, kEpiConvSilu = 3 };
hipError_t launch_gemv(const GemvArgs& a, int prologue, hipStream_t s, int epilogue = kEpiAuto);
// Workgroups of a launch_gemv grid (the argmax partials of amax_part: one per workgroup).
constexpr int kArgmaxParts = 4096;
int gemv_blocks(const GemvArgs& a, int epilogue);
// Largest in_dim the matvec stages in LDS (128 KB of the 160 KB a gfx950 workgroup may use).
constexpr int kGemvMaxIn = 32768;
// Raises the dynamic-LDS limit of the matvec instantiations that stage inputs wider than
// 16384 (64 KB); once per process, before any launch is captured into a graph.
hipError_t gemv_enable_wide_inputs();

// ---------------------------------------------------------------- token-batched GEMM
// Y[M][N] = (R ? R : 0) + X[M][K] . W[N][K]^T; K % 8 == 0, ldx % 4 == 0, 16-byte aligned X.
struct GemmArgs {
    const float* X;
    const uint16_t* W;
    const float* R;  // may alias Y
    float* Y;
    int M, N, K;
    int64_t ldx, ldr, ldy;
    // W rows (2i, 2i + 1) are (gate_i, up_i), the interleaved gate/up projection: store
    // Y[m][i] = silu(gate_i) * up_i instead (Y is M x N/2, row stride ldy); R unused
    int swiglu = 0;
    // Two-part fp16 path (when Wh and xmax are set): Wh = W x 2^w_exp as fp16 (same layout),
    // xmax[r * xmax_n + j], j < xmax_n, partial maxima of |X| row r whose maximum scales the
    // row into [2^14, 2^15) before its split into two fp16 parts.
    const uint16_t* Wh = nullptr;
    int w_exp = 0;
    const float* xmax = nullptr;
    int xmax_n = 0;
    // SwiGLU output: the maximum |Y| of each row over each column tile (N / 128 wide rows:
    // ymax[r * ceil(N / 128) + tile]) for the next GEMM's two-part path (may be null)
    float* ymax = nullptr;
    // X (two-part path) and, for SwiGLU, Y in the tiled layout of xt_off (ldx / ldy unused;
    // rows padded to a multiple of 128, K to a multiple of 32)
    int x_tiled = 0, y_tiled = 0;
    // X already split (two-part path, x_tiled): X holds the fp16 parts of each row scaled by
    // 2^split_row_exp(row maximum of xmax) in the split-plane layout of xp_off
    int x_planes = 0;
};
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s);
// Tiled activation layout of the two-part GEMM's X operand: blocks of 16 rows x 32 k
// (512 floats), row block after row block and within one the k blocks in order; inside a
// block [h][r][g][e] for k = 8 g + 4 h + e of row r: the 16 bytes a lane of the matrix-core
// operand loads per instruction are contiguous, 1 KB per wave-wide load. K % 32 == 0.
__host__ __device__ inline int64_t xt_off(int64_t row, int k, int K) {
    return ((row >> 4) * (K >> 5) + (k >> 5)) * 512 + (((k & 7) >> 2) << 8) + ((row & 15) << 4) +
           (((k & 31) >> 3) << 2) + (k & 3);
}
inline int64_t rows_tiled(int64_t rows) { return (rows + 127) / 128 * 128; }
// Split-plane layout of the two-part GEMM's X operand (x_planes), in fp16 elements: the same
// blocks of 16 rows x 32 k as xt_off and the same 2 KB each, holding the 512 high parts and
// then the 512 low parts, each as [k / 8][row % 16][k % 8]: lane l of a wave-wide 16-byte
// load reads the 16 bytes at 16 l, its matrix-core operand (row l % 16, k = 8 (l / 16) .. + 7).
// (Rows kept whole, [row % 16][k / 8][k % 8], made the producer's stores contiguous and the
// GEMM's loads scattered over four 64-byte pieces per lane quad: 0.25% slower overall.)
__host__ __device__ inline int64_t xp_off(int64_t row, int k, int K, int part) {
    return ((row >> 4) * (K >> 5) + (k >> 5)) * 1024 + part * 512 + (((k & 31) >> 3) << 7) + ((row & 15) << 3) +
           (k & 7);
}
// Column tiles of the GEMM (the ymax row width)
inline int gemm_col_tiles(int N) { return (N + 127) / 128; }
// max |w| over n bf16 weights, into *out (a uint zeroed beforehand: the bits of the
// non-negative maximum); and wh = fp16(w x 2^e), round to nearest even
hipError_t launch_bf16_absmax(const uint16_t* w, int64_t n, unsigned* out, hipStream_t s);
hipError_t launch_bf16_to_f16(const uint16_t* w, uint16_t* wh, int64_t n, int e, hipStream_t s);
// row-major X -> tiled Xt (rows_tiled(M) rows, zero padding) and xmax[r] = max |X[r][:]|
hipError_t launch_rows_to_tiled(const float* X, int64_t ldx, int M, int K, float* Xt, float* xmax, hipStream_t s);

// ---------------------------------------------------------------- GDN decode
struct GdnDecodeArgs {
    int n_layers, KH, VH, KER;  // DK = DV = 128
    int pos_val;
    const int* pos_dev;         // position read on the device when non-null
    float eps;
    const float *qkv, *z, *b, *a;                 // per-layer contiguous inputs
    const float *conv_w, *A_log, *dt_bias, *norm_w;
    float *conv_ring, *state, *out;
    int conv_done;  // qkv already holds SiLU(conv) (the in-projection ran the window); no ring update
    // per-layer strides in elements (0 = derive the contiguous stride)
    int64_t ls_qkv, ls_z, ls_ba, ls_convw, ls_vh, ls_normw, ls_ring, ls_state, ls_out;
};
hipError_t launch_gdn_decode(const GdnDecodeArgs& a, bool fuse_norm, hipStream_t s);

// ---------------------------------------------------------------- attention decode
struct AttnDecodeArgs {
    int NQ, NKV, HD, ROT;       // HD = 256
    int pos_val;
    const int* pos_dev;
    int64_t max_ctx;
    int n_splits;               // splits per kv head (grid.x of the partial kernel)
    double theta;
    float eps;
    const float *qg, *k_new, *v_new, *q_norm, *k_norm;
    const float* rope_cs;       // optional [max_ctx][ROT]: cos (ROT/2) then sin (ROT/2) per position
    float *k_cache, *v_cache;   // [NKV][max_ctx][HD], fp32 or (kv_bf16) bf16 elements
    int kv_bf16;                // cache element: 0 = fp32, 1 = bf16 (round to nearest even)
    float* part_o;              // [NKV][n_splits][GRP][HD]
    float* part_ml;             // [NKV][n_splits][GRP][2]
    float* out;                 // [NQ][HD]
    // independent layers in one launch (grid.z); every array above repeats per layer with
    // its natural stride, the caches with stride ls_cache (0 = NKV * max_ctx * HD)
    int n_layers;
    int64_t ls_cache;
};
// Advances the per-layer pointers of `a` to layer l (device side).
__device__ __forceinline__ void attn_select_layer(AttnDecodeArgs& a, int l) {
    if (l == 0) return;
    const int grp = a.NQ / a.NKV;
    const int64_t lc = a.ls_cache ? a.ls_cache : static_cast<int64_t>(a.NKV) * a.max_ctx * a.HD;
    a.qg += static_cast<int64_t>(l) * 2 * a.NQ * a.HD;
    a.k_new += static_cast<int64_t>(l) * a.NKV * a.HD;
    a.v_new += static_cast<int64_t>(l) * a.NKV * a.HD;
    a.q_norm += static_cast<int64_t>(l) * a.HD;
    a.k_norm += static_cast<int64_t>(l) * a.HD;
    const int64_t lce = a.kv_bf16 ? lc / 2 : lc;  // in floats: a bf16 cache is half as long
    a.k_cache += l * lce;
    a.v_cache += l * lce;
    a.part_o += static_cast<int64_t>(l) * a.NKV * a.n_splits * grp * a.HD;
    a.part_ml += static_cast<int64_t>(l) * a.NKV * a.n_splits * grp * 2;
    a.out += static_cast<int64_t>(l) * a.NQ * a.HD;
}
// split-K partials, with the q/k norm + RoPE + K/V append of position pos folded in
hipError_t launch_attn_partial(const AttnDecodeArgs& a, hipStream_t s);
bool attn_force_valu();  // Q35_ATTN_VALU=1: no matrix-core kernel
hipError_t launch_attn_combine(const AttnDecodeArgs& a, hipStream_t s);
// workspace floats for part_o + part_ml
inline int64_t attn_partial_floats(int NQ, int NKV, int HD, int n_splits) {
    const int grp = NQ / NKV;
    return static_cast<int64_t>(NKV) * n_splits * grp * (HD + 2);
}
// Default splits per kv head: one workgroup per CU over all kv heads (of all layers in the
// launch: NKV counts them), and no split shorter than 64 positions at full context. When
// that leaves each range 8-63 tiles of 16 positions (2-15 per wave of the 4-wave
// matrix-core kernel), the tile loop is too short to hide the first loads and the uneven
// last tiles, and two workgroups per CU (the kernel's occupancy) are used instead -- as
// long as that stays within 64 splits per kv head, past which the combine's extra partials
// cost more than it gains. Measured: 6 layers x 2 kv heads at 8k, 42 splits 0.60 of HBM
// peak against 0.575 for 21; one layer at 32k, 256 splits 918 tok/s against 947 for 128.
inline int attn_default_splits(int64_t max_ctx, int NKV, int n_cu) {
    const int64_t want = (max_ctx + 63) / 64;
    const int64_t one = std::max<int64_t>(1, n_cu / std::max(1, NKV));
    const int64_t s = std::max<int64_t>(1, std::min<int64_t>(want, one));
    const int64_t tiles = (max_ctx + 16 * s - 1) / (16 * s);
    if (s == one && 2 * one <= 64 && tiles >= 8 && tiles < 64) return static_cast<int>(std::min<int64_t>(want, 2 * one));
    return static_cast<int>(s);
}
// Compute units of the current device (256 on MI355X when the query fails).
int device_cu_count();

// ---------------------------------------------------------------- whole-prompt mixers
// GDN over a block of T tokens at positions pos0 .. pos0 + T - 1, continuing from `state`
// and the conv ring (both updated in place). Inputs are token-major rows with leading
// dimensions; the workspace pointers (Qg .. O) are carved by gdn_prefill_carve.
struct GdnPrefillArgs {
    int T, Tp, KH, VH, pos0;  // Tp = T rounded up to whole chunks
    float eps;
    const float* qkv;  // [T][ld_qkv], CONV raw (pre-conv) channels
    int64_t ld_qkv;
    const float* z;    // [T][ld_z], VD
    int64_t ld_z;
    const float *b, *a;  // [T][ld_ba], VH each
    int64_t ld_ba;
    const float *conv_w, *A_log, *dt_bias, *norm_w;  // norm_w null: raw readout
    float *conv_ring, *state;
    float* out;        // [T][VH * 128]
    // workspace (head-major, padded to Tp rows): Qg the normalised, scaled q; Eg = e^gamma
    // of each row, gamma the chunk-local cumulative decay; Kd = K e^(gamma_last - gamma) per
    // (v-head, chunk), transposed ([128 dims][64 rows]); P the chunk's decayed Q K^T
    float *Qg, *U, *W, *Eg, *Kd, *P;
    float* Sc;         // [VH][Tp / 64][128][128] state at the start of each chunk
    float* omax = nullptr;  // maximum |out| of each (token, v-head): [T][VH] (may be null)
    int out_tiled = 0;      // out in the xt_off layout (K = VH * 128)
};
int64_t gdn_prefill_workspace_floats(int KH, int VH, int T);
void gdn_prefill_carve(GdnPrefillArgs& a, float* ws);
hipError_t launch_gdn_prefill(GdnPrefillArgs& a, hipStream_t s);

// Causal gated attention over a block of T tokens at positions pos0 ..: the block's keys and
// values are appended to the caches, every query attends to positions [0, pos0 + t].
struct AttnPrefillArgs {
    int T, NQ, NKV, ROT, pos0;  // HD = 256
    int64_t max_ctx;
    double theta;
    float eps;
    const float* qkv;  // [T][ld_qkv]: NQ x [q | gate] (2 HD each), NKV x k, NKV x v
    int64_t ld_qkv;
    const float *q_norm, *k_norm;
    float *k_cache, *v_cache;  // [NKV][max_ctx][HD], fp32 or (kv_bf16) bf16 elements
    int kv_bf16;
    float* Qa;                 // workspace [NQ][T][HD]
    float* out;                // [T][NQ * HD]
    const float* rope_cs;      // optional [max_ctx][ROT] cos | sin table (else computed)
    float* omax = nullptr;     // maximum |out| of each (token, head): [T][NQ] (may be null)
    int out_tiled = 0;         // out in the xt_off layout (K = NQ * HD)
    // optional (fp32 cache): attn_prefill_image_floats(NKV, pos0, T) floats, 16-byte aligned,
    // for the keys and values pre-split into the attention kernel's tile layout
    void* kv_img = nullptr;
    int img_tiles = 0;  // set by the launch
};
int64_t attn_prefill_workspace_floats(int NQ, int T);
int attn_prefill_image_tiles(int pos0, int T);
int64_t attn_prefill_image_floats(int NKV, int pos0, int T);
hipError_t launch_attn_prefill(const AttnPrefillArgs& a, hipStream_t s);
// h[t][i] = silu(gu[t][2i]) * gu[t][2i + 1] (gate / up columns interleaved)
// hidden[t][:] = bf16 embed[ids[t]][:]
hipError_t launch_embed_rows(const uint16_t* embed, const int* ids, float* hidden, int T, int H, hipStream_t s);

// ---------------------------------------------------------------- small kernels
// y = W x with fp32 weights [rows][n], any n
hipError_t launch_matvec_f32(const float* W, const float* x, float* y, int rows, int n, hipStream_t s);
// ymax (may be null): the maximum |y| of each row
// y_tiled: 0 row-major, 1 the tiled layout of xt_off, 2 split already for the two-part GEMM
// (the layout of xp_off; needs ymax, and n with rmsnorm_rows_splits(n))
hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* y, int rows, int n,
                               float eps, int gated, const float* gate, hipStream_t s, float* ymax = nullptr,
                               int y_tiled = 0);
inline bool rmsnorm_rows_splits(int n) { return n == 1024 || n == 2048 || n == 4096; }
hipError_t launch_l2norm_rows(float* x, int rows, int n, float eps, hipStream_t s);
hipError_t launch_rope_rows(float* x, int rows, int hd, int rot, const int* pos, int pos0,
                            double theta, hipStream_t s);
// hidden[i] = bf16 embed[token][i]; token read from token_dev
hipError_t launch_embed(const uint16_t* embed, const int* token_dev, float* hidden, int H,
                        hipStream_t s);
// argmax over n logits (first index of the maximum) in two passes through `part`
// (2 * kArgmaxBlocks words). The final pass writes the index to token_out; when pos is
// non-null it also stores the index at ids[*pos] (ids may be null) and increments *pos.
constexpr int kArgmaxBlocks = 256;
hipError_t launch_argmax(const float* logits, int n, void* part, int* token_out, int* ids,
                         int* pos, hipStream_t s);
// The final pass alone over n_parts (value, index) partials (a matvec's amax_part).
hipError_t launch_argmax_parts(const void* part, int n_parts, int* token_out, int* ids, int* pos,
                               hipStream_t s);
hipError_t launch_add_int(int* p, int v, hipStream_t s);
hipError_t launch_set_int(int* p, int v, hipStream_t s);
hipError_t launch_copy_f32(float* dst, const float* src, int64_t n, hipStream_t s);
hipError_t launch_fill_f32(float* dst, int64_t n, float v, hipStream_t s);
// dst[i] = std * N(0,1)(key, i); with bf16, dst holds bf16 elements rounded to nearest even
hipError_t launch_fill_normal(float* dst, int64_t n, uint64_t key, float std, hipStream_t s, bool bf16 = false);
// t[p][i] = cos(p * theta^(-2i/rot)), t[p][rot/2 + i] = sin(...) for i < rot/2, in double
// rounded to float (the apply_rope formula, src/forward_pass.cpp:102-112)
hipError_t launch_rope_table(float* t, int64_t n_pos, int rot, double theta, hipStream_t s);

}  // namespace q35k
