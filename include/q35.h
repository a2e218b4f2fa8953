/*
 * q35.h -- C ABI of the MI355X (gfx950) Qwen3.5 hybrid token-mixer library (libq35.so).
 *
 * Every entry point is plain C: pointers, sizes and status codes, no C++ or torch types.
 * Device pointers are HIP device allocations; `q35_stream` is a hipStream_t (NULL = the
 * default stream). Entry points never throw; a non-zero status comes with a message from
 * q35_last_error() (thread-local).
 *
 * Reference interfaces replaced (paths relative to the Qwen3.5-CPU-cpp tree):
 *   model level   -> include/qwen_model.h:21-32 (QwenModel), include/qwen_forward.h:18-25
 *                    (QwenForward::prefill)
 *   planning      -> include/memory_budget.h:6-62, include/model_config.h:11-63,
 *                    src/config_loader.cpp:59-108
 *   primitives    -> include/forward_pass.h:21-54 (matmul, rmsnorm, rmsnorm_gated, l2norm,
 *                    apply_rope) on device pointers
 *   mixers        -> QwenModel::gdn_step src/qwen_model.cpp:154-209,
 *                    QwenModel::attn_step src/qwen_model.cpp:106-152,
 *                    QwenForward::mix_gdn src/qwen_forward.cpp:83-152,
 *                    QwenForward::mix_attention src/qwen_forward.cpp:20-80
 */
#ifndef Q35_H
#define Q35_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t q35_status;
#define Q35_OK 0
#define Q35_ERR_ARG (-1)         /* bad argument (null pointer, size out of range) */
#define Q35_ERR_HIP (-2)         /* a HIP runtime call failed */
#define Q35_ERR_IO (-3)          /* file could not be read or written */
#define Q35_ERR_FORMAT (-4)      /* malformed config.json / safetensors header */
#define Q35_ERR_MISSING (-5)     /* a required weight tensor is absent */
#define Q35_ERR_RANGE (-6)       /* position / token id beyond the planned arenas */
#define Q35_ERR_UNSUPPORTED (-7) /* a shape or dtype the kernels are not built for */

typedef void *q35_stream; /* hipStream_t */

/* Architecture constants. Mirrors ModelConfig, include/model_config.h:11-63. */
typedef struct q35_dims {
    int32_t hidden_size;          /* hidden_size */
    int32_t n_layers_total;       /* num_hidden_layers */
    int32_t n_layers_gdn;         /* derived: total - total / attn_interval */
    int32_t n_layers_attn;        /* derived: total / attn_interval */
    int32_t gdn_k_heads;          /* linear_num_key_heads */
    int32_t gdn_v_heads;          /* linear_num_value_heads */
    int32_t gdn_k_head_dim;       /* linear_key_head_dim */
    int32_t gdn_v_head_dim;       /* linear_value_head_dim */
    int32_t gdn_conv_kernel;      /* linear_conv_kernel_dim */
    int32_t attn_q_heads;         /* num_attention_heads */
    int32_t attn_kv_heads;        /* num_key_value_heads */
    int32_t attn_head_dim;        /* head_dim */
    int32_t ffn_intermediate;     /* intermediate_size */
    int32_t vocab_size;           /* vocab_size */
    int64_t native_max_context;   /* max_position_embeddings */
    int64_t n_params;             /* rough count used by the budget display */
    double rope_theta;            /* rope_theta */
    float rms_norm_eps;           /* rms_norm_eps */
    float partial_rotary_factor;  /* partial_rotary_factor */
    int32_t attn_interval;        /* full_attention_interval */
    int32_t tie_word_embeddings;  /* tie_word_embeddings */
} q35_dims;

/* Bytes per arena. Mirrors MemoryBudget, include/memory_budget.h:6-19, plus the prompt arena
 * of the chunked prefill (activations of one block of prompt tokens and the fp16 copies of
 * the projection weights its GEMMs multiply), which the reference does not have:
 * q35_compute_budget leaves it 0, q35_model_budget reports the model's. */
typedef struct q35_budget {
    uint64_t weight_bytes;
    uint64_t gdn_state_bytes;
    uint64_t gdn_conv_bytes;
    uint64_t kv_cache_bytes;
    uint64_t activation_bytes;
    uint64_t vision_scratch_bytes;
    uint64_t prompt_arena_bytes;
} q35_budget;

/* ------------------------------------------------------------------------------------ */
/* errors / version                                                                     */
/* ------------------------------------------------------------------------------------ */
const char *q35_last_error(void);  /* message for the last failed call on this thread */
const char *q35_version(void);
/* Number of device allocations the library has made since load (they happen in
 * q35_model_open / q35_model_create, q35_model_reserve_context, the prompt arena of a
 * model's first prefill when none was planned, and the staging buffer of the forward_pass.h
 * functions' first call; a decode step must leave this unchanged). */
int64_t q35_device_alloc_count(void);

/* ------------------------------------------------------------------------------------ */
/* config + memory planning (host only)                                                 */
/* ------------------------------------------------------------------------------------ */
void q35_dims_default(q35_dims *d);                              /* model_config.h:11-63 */
q35_status q35_load_config(const char *path, q35_dims *d);       /* config_loader.cpp:59-108 */
int32_t q35_is_attention_layer(const q35_dims *d, int32_t layer);  /* model_config.h:60-62 */
uint64_t q35_gdn_conv_state_bytes(const q35_dims *d);            /* memory_budget.h:23-28 */
q35_status q35_compute_budget(const q35_dims *d, int32_t bytes_per_weight,
                              int64_t max_context, int32_t kv_bytes_per_elem,
                              int32_t max_vision_tiles, int32_t vit_dim,
                              q35_budget *out);                  /* memory_budget.cpp:30-54 */
int64_t q35_solve_max_context(const q35_dims *d, uint64_t ram_budget_bytes,
                              uint64_t weight_bytes, uint64_t gdn_state_bytes,
                              uint64_t activation_bytes, uint64_t vision_scratch_bytes,
                              uint64_t safety_margin_bytes,
                              int32_t kv_bytes_per_elem);        /* memory_budget.cpp:56-81 */

/* ------------------------------------------------------------------------------------ */
/* synthetic checkpoints (host only): deterministic counter-based N(0, std) weights      */
/* ------------------------------------------------------------------------------------ */
/* Writes <dir>/config.json and <dir>/model.safetensors (bf16, reference tensor names,
 * src/qwen_model.cpp:39-69). (1+w)-form norm weights are 0, the GDN gated-norm weight is 1,
 * every other tensor is N(0, std). `threads` <= 0 means all cores. */
q35_status q35_synth_write_model(const char *dir, const q35_dims *d, uint64_t seed,
                                 float std, int32_t threads);
/* n ids uniform in [0, vocab). */
q35_status q35_synth_token_ids(uint64_t seed, int32_t vocab, int32_t n, int32_t *ids);
/* Host fill: dst[i] = std * N(0,1) drawn from (seed, stream, i). */
q35_status q35_synth_normal(float *dst, int64_t n, uint64_t seed, uint64_t stream, float std,
                            int32_t threads);

/* ------------------------------------------------------------------------------------ */
/* model: the device-resident decoder (QwenModel, include/qwen_model.h:21-32)            */
/* ------------------------------------------------------------------------------------ */
typedef struct q35_model q35_model;

/* One tensor of a host weight table (a SafeTensors entry, include/safetensors_loader.h:26-33). */
typedef struct q35_tensor {
    const char *name;      /* HuggingFace tensor name */
    int32_t dtype;         /* 0 = BF16, 1 = F32 */
    int32_t ndim;
    int64_t shape[4];
    const void *data;      /* host pointer, read only during q35_model_create */
} q35_tensor;

/* Plans the four device arenas (weights, recurrent state, KV cache, scratch) with the
 * memory equation, makes one hipMalloc for each and uploads the weights. max_context is
 * the KV capacity in positions; max_context 0 plans it with solve_max_context
 * (src/memory_budget.cpp:56-81) against the device's memory: weights, state, scratch, a
 * planned prompt arena and a 1 GiB margin are fixed costs, the rest holds KV rows, up to
 * native_max_context (q35_model_max_context reports the result). */
q35_status q35_model_create(const q35_dims *d, const q35_tensor *tensors, int32_t n_tensors,
                            int64_t max_context, q35_model **out);
/* Creation options. kv_bytes_per_elem is memory_budget's KV element width
 * (include/memory_budget.h:37-42): 4 = fp32 cache (the reference's; the default), 2 = bf16
 * cache (rows rounded to nearest even when appended; half the KV bytes and bandwidth).
 * prefill_block > 0 plans the prompt arena at creation, for prefill blocks of up to that
 * many tokens (a fifth hipMalloc, reported in q35_budget.prompt_arena_bytes; larger blocks
 * are refused); 0 leaves it to the first prefill. prefill_exact = 1 runs the prefill's
 * projection GEMMs on three exact bf16 parts of each fp32 activation (full fp32 precision;
 * no fp16 weight copies, so the prompt arena is smaller by the projection weights' size in
 * fp16, 2.7 GiB at the 2B shape); 0 (default) on two row-scaled fp16 parts (about 22
 * significant bits of each activation) against fp16 copies of the weights, which is faster. */
typedef struct q35_model_options {
    int32_t kv_bytes_per_elem;
    int32_t prefill_block;
    int32_t prefill_exact;
    int32_t reserved[5];
} q35_model_options;
q35_status q35_model_create_opts(const q35_dims *d, const q35_tensor *tensors, int32_t n_tensors,
                                 int64_t max_context, const q35_model_options *opt, q35_model **out);
q35_status q35_model_open_opts(const char *model_dir, int64_t max_context,
                               const q35_model_options *opt, q35_model **out);
/* Same, reading <dir>/config.json and every <dir>/ *.safetensors shard. */
q35_status q35_model_open(const char *model_dir, int64_t max_context, q35_model **out);
void q35_model_destroy(q35_model *m);
q35_status q35_model_dims(const q35_model *m, q35_dims *out);
q35_status q35_model_budget(const q35_model *m, q35_budget *out);  /* QwenModel::budget */
int64_t q35_model_position(const q35_model *m);                    /* QwenModel::position */
int64_t q35_model_max_context(const q35_model *m);
q35_stream q35_model_stream(const q35_model *m);
q35_status q35_model_synchronize(q35_model *m);

/* QwenModel::reset (src/qwen_model.cpp:98-104): zero KV, GDN and conv state, pos = 0. */
q35_status q35_model_reset(q35_model *m);
/* QwenModel::step (src/qwen_model.cpp:211-239): one token through all layers.
 * logits_host (vocab floats) and argmax may each be NULL. Fails with Q35_ERR_RANGE when
 * the position has reached max_context or the token is outside [0, vocab). */
q35_status q35_model_step(q35_model *m, int32_t token, float *logits_host, int32_t *argmax);
/* QwenModel::generate_greedy (src/qwen_model.cpp:241-255): reset, ingest the prompt one
 * step at a time, then n_new greedy steps (first index of the maximum). out has n_new ids. */
q35_status q35_model_generate_greedy(q35_model *m, const int32_t *prompt, int32_t n_prompt,
                                     int32_t n_new, int32_t *out);
/* Greedy continuation from the current state without reset: n_new steps, the first fed
 * with `token`, each next one with the previous argmax. out has n_new ids (the argmax
 * after each step). All steps run back to back on the device with no host round trip. */
q35_status q35_model_decode_greedy(q35_model *m, int32_t token, int32_t n_new, int32_t *out);
/* Whole-prompt forward (QwenForward::prefill, src/qwen_forward.cpp:154-206): starts from a
 * zero state, runs the chunked GDN and flash attention prefill and leaves the model state
 * (GDN state, conv window, KV rows, pos = n) as n decode steps would. logits_host receives
 * n rows of q35_model_prefill_logits_width floats when not NULL. Without a prompt arena
 * planned at creation, the first call makes it (one more device allocation, kept for later
 * calls): activations for one block of tokens. */
q35_status q35_model_prefill(q35_model *m, const int32_t *ids, int32_t n, float *logits_host);
/* The same chunked path continuing from the current position: ids are placed at positions
 * pos .. pos + n - 1 (no reset). trace_host, when not NULL, receives the hidden state after
 * every layer for every token, [n][n_layers_total][hidden_size]. Afterwards the last
 * token's logits / argmax are where q35_model_step leaves them, so decoding continues with
 * q35_model_decode_greedy. */
q35_status q35_model_extend(q35_model *m, const int32_t *ids, int32_t n, float *logits_host,
                            float *trace_host);
/* Tokens per prefill block (0 = automatic: the planned block, else min(4096, max_context)).
 * Larger blocks make larger GEMMs and a larger prompt arena; a prompt arena planned at
 * creation serves every block up to its size and refuses larger ones (Q35_ERR_RANGE), one
 * made by a prefill is made again only for a larger block. */
q35_status q35_model_set_prefill_block(q35_model *m, int32_t tokens);
/* Output head of the prefill logits: Q35_HEAD_OUTPUT (the default) is the step's head
 * (lm_head when the checkpoint has one, else the tied embedding; vocab_size rows),
 * Q35_HEAD_EMBEDDING is QwenForward::prefill's rule (src/qwen_forward.cpp:193-199): the
 * embedding over all its rows. The width of each logits row is
 * q35_model_prefill_logits_width. Decoding after a prefill always uses the step's head. */
#define Q35_HEAD_OUTPUT 0
#define Q35_HEAD_EMBEDDING 1
q35_status q35_model_set_prefill_head(q35_model *m, int32_t head);
int64_t q35_model_prefill_logits_width(const q35_model *m);
/* Grows the KV capacity to max_context positions (no change when it is not larger): the KV
 * and scratch arenas are made again, the weights stay; the model is reset. For a caller
 * that learns the context it needs after creating the model (a longer prompt). */
q35_status q35_model_reserve_context(q35_model *m, int64_t max_context);

/* Decode-step execution options. */
q35_status q35_model_set_graph(q35_model *m, int32_t enable);        /* hipGraph replay */
q35_status q35_model_set_layer_trace(q35_model *m, int32_t enable);  /* record per-layer hidden */
/* Hidden state after every layer of the last step: n_layers_total * hidden_size floats. */
q35_status q35_model_read_layer_trace(q35_model *m, float *host);
/* Residual stream after the last layer of the last step (before the final norm). */
q35_status q35_model_read_hidden(q35_model *m, float *host);

/* Per-kernel-class device time of the decode steps and prefills run while timing is on
 * (hipEvents on the model stream around each launch; graph replay is bypassed while it is
 * on). */
#define Q35_KT_GEMV 0
#define Q35_KT_GDN_DECODE 1
#define Q35_KT_ATTN_DECODE 2   /* split-K kernel (q/k norm + RoPE + KV append folded in) */
#define Q35_KT_ATTN_COMBINE 3
#define Q35_KT_OTHER 4
#define Q35_KT_GEMM 5          /* prefill projections */
#define Q35_KT_GDN_PREFILL 6   /* one layer's chunked GDN (chunk pass, ring, scan, gated norm) */
#define Q35_KT_ATTN_PREFILL 7  /* one layer's q/k norm + RoPE + append and flash kernel */
#define Q35_KT_COUNT 8
q35_status q35_model_set_kernel_timing(q35_model *m, int32_t enable);
/* ms[Q35_KT_COUNT] total milliseconds, launches[Q35_KT_COUNT]; resets the counters. */
q35_status q35_model_kernel_times(q35_model *m, double *ms, int64_t *launches);
/* KV splits per kv head of the attention decode kernel (0 = the default for max_context);
 * at most 1024. A tuning knob: results are the same for every value. */
q35_status q35_model_set_attn_splits(q35_model *m, int32_t n_splits);

/* State access, in the reference layouts (src/qwen_model.cpp:50-61):
 * GDN state [VH][DK][DV], conv window [CONV][KER-1] oldest first, K/V rows [n][NKV][HD]. */
q35_status q35_model_read_gdn_state(q35_model *m, int32_t gdn_layer, float *host);
q35_status q35_model_write_gdn_state(q35_model *m, int32_t gdn_layer, const float *host);
q35_status q35_model_read_conv_state(q35_model *m, int32_t gdn_layer, float *host);
q35_status q35_model_write_conv_state(q35_model *m, int32_t gdn_layer, const float *host);
q35_status q35_model_read_kv(q35_model *m, int32_t attn_layer, int64_t pos0, int64_t n,
                             float *k_host, float *v_host);
q35_status q35_model_write_kv(q35_model *m, int32_t attn_layer, int64_t pos0, int64_t n,
                              const float *k_host, const float *v_host);
q35_status q35_model_set_position(q35_model *m, int64_t pos);
/* Synthetic prefilled cache: K/V rows [0, pos) ~ N(0,1), GDN state ~ N(0, state_std),
 * conv window 0, position = pos. Generated on the device from (seed). */
q35_status q35_model_fill_synthetic(q35_model *m, int64_t pos, uint64_t seed, float state_std);

/* ------------------------------------------------------------------------------------ */
/* primitives on device pointers (include/forward_pass.h:21-54)                           */
/* ------------------------------------------------------------------------------------ */
/* y = W x, W bf16 row-major [out_dim][in_dim] (forward_pass.cpp:65-75). in_dim % 8 == 0 and
 * in_dim <= 32768 (the input is staged in LDS); Q35_ERR_UNSUPPORTED otherwise. */
q35_status q35_matmul_bf16(const uint16_t *W, const float *x, float *y, int32_t out_dim,
                           int32_t in_dim, q35_stream s);
/* y = W x with fp32 W row-major [out_dim][in_dim], any in_dim (forward_pass.cpp:29-33, the
 * fp32 overload of matmul). */
q35_status q35_matmul_f32(const float *W, const float *x, float *y, int32_t out_dim, int32_t in_dim,
                          q35_stream s);
/* Token-batched matmul for the prefill: Y[M][N] = (R ? R : 0) + X[M][K] . W[N][K]^T, fp32 X /
 * R / Y with leading dimensions (elements), bf16 W row-major (forward_pass.cpp:65-75 for M
 * rows at once). Requires K % 8 == 0, ldx % 4 == 0 and a 16-byte aligned X. R may alias Y. */
q35_status q35_gemm_bf16(const float *X, int64_t ldx, const uint16_t *W, int32_t M, int32_t N,
                         int32_t K, const float *R, int64_t ldr, float *Y, int64_t ldy,
                         q35_stream s);
/* The same product on the model prefill's two-part fp16 path, from plain row-major inputs
 * (replaces forward_pass.cpp:65-75 for M rows at once, as q35_gemm_bf16): W is copied to fp16
 * scaled by 2^e so that its largest |w| lies in [2^14, 2^15) (exact for every bf16 weight
 * down to 2^-24 of the largest); each row of X is scaled by a power of two from its maximum
 * into (-2^15, 2^15) and split into h = fp16(x), l = fp16(x - h), |x - h - l| <= 2^-22 |x|
 * (about 22 significant bits of x); each fp16 x fp16 product is exact, accumulation is fp32
 * and both scales are undone exactly. Requires K % 32 == 0, a 16-byte aligned W and a
 * 256-byte aligned workspace of q35_gemm_f16x2_workspace_bytes(M, N, K) bytes (fp16 copy of
 * W, X in the GEMM's tiled layout, the maxima). Synchronizes the stream once (the weights'
 * maximum is read back to choose their scale). */
uint64_t q35_gemm_f16x2_workspace_bytes(int32_t M, int32_t N, int32_t K);
q35_status q35_gemm_f16x2(const float *X, int64_t ldx, const uint16_t *W, int32_t M, int32_t N,
                          int32_t K, const float *R, int64_t ldr, float *Y, int64_t ldy,
                          void *workspace, uint64_t workspace_bytes, q35_stream s);
/* Row-wise y = x * rsqrt(mean(x^2) + eps) * (1 + w) over rows of n (forward_pass.cpp:77-84). */
q35_status q35_rmsnorm(const float *x, const float *w, float *y, int32_t rows, int32_t n,
                       float eps, q35_stream s);
/* Row-wise y = w * (x * rsqrt(mean(x^2)+eps)) * silu(gate) (forward_pass.cpp:86-93). */
q35_status q35_rmsnorm_gated(const float *x, const float *w, const float *gate, float *y,
                             int32_t rows, int32_t n, float eps, q35_stream s);
/* Row-wise in place x *= 1/sqrt(sum(x^2) + eps) (forward_pass.cpp:95-100). */
q35_status q35_l2norm(float *x, int32_t rows, int32_t n, float eps, q35_stream s);
/* Partial rotate-half RoPE in place on rows of head_dim; row r is at position pos[r]
 * (device int32 array) or at pos0 when pos is NULL (forward_pass.cpp:102-112). Pairs
 * (i, i + rotary_dim / 2) for i < rotary_dim / 2: with an odd rotary_dim the last rotated
 * index stays as it is, as in the reference. */
q35_status q35_apply_rope(float *x, int32_t rows, int32_t head_dim, int32_t rotary_dim,
                          const int32_t *pos, int32_t pos0, double theta, q35_stream s);

/* ------------------------------------------------------------------------------------ */
/* mixer kernels on device pointers                                                      */
/* ------------------------------------------------------------------------------------ */
/* GDN decode for one token over n_layers independent layer states in one launch
 * (QwenModel::gdn_step after its input projections, src/qwen_model.cpp:173-207).
 * Layouts, per layer l (strides are whole layers):
 *   qkv [CONV] pre-conv projection, z [VD], b [VH], a [VH]     (inputs)
 *   conv_w [CONV][KER], A_log [VH], dt_bias [VH], norm_w [DV]  (weights)
 *   conv_ring [KER][CONV]: input of position t lives in slot t % KER
 *   state [VH][DK][DV]
 *   out [VD]: with norm_w != NULL the gated-rmsnorm output, else the raw S^T q readout.
 * Requires DK == DV == 128 and KER == 4. */
typedef struct q35_gdn_decode_args {
    int32_t n_layers, k_heads, v_heads, head_dim_k, head_dim_v, conv_kernel;
    int32_t pos;           /* position of this token (selects the conv ring slot) */
    float eps;             /* gated-norm eps */
    const float *qkv, *z, *b, *a;
    const float *conv_w, *A_log, *dt_bias, *norm_w;
    float *conv_ring, *state, *out;
} q35_gdn_decode_args;
q35_status q35_gdn_decode(const q35_gdn_decode_args *args, q35_stream s);

/* Gated GQA attention decode for one token (QwenModel::attn_step after its projections,
 * src/qwen_model.cpp:119-150) of n_layers independent layers in one launch: q_norm + RoPE
 * on q, k_norm + RoPE on the new key, K/V append at `pos`, softmax over positions 0..pos
 * (split-K over the cache with a combine pass), times sigmoid(gate). Per layer l (arrays
 * repeat with their natural stride):
 *   qg [NQ][2*HD] (per head: q then gate), k_new [NKV][HD], v_new [NKV][HD] (inputs)
 *   q_norm [HD], k_norm [HD]; k_cache, v_cache [NKV][max_context][HD]
 *   out [NQ][HD]; workspace: q35_attn_decode_workspace_bytes() bytes of device memory.
 * Requires HD == 256 and NQ / NKV in {1, 2, 4, 8, 16}. */
typedef struct q35_attn_decode_args {
    int32_t q_heads, kv_heads, head_dim, rotary_dim;
    int32_t pos;
    int32_t n_splits;      /* KV splits per kv head; 0 = automatic */
    int32_t n_layers;      /* independent layers in one launch (0 or 1 = one) */
    int32_t kv_dtype;      /* cache elements: 0 = fp32, 1 = bf16 (appended rows rounded to nearest even) */
    int64_t max_context;
    double rope_theta;
    float eps;
    const float *qg, *k_new, *v_new, *q_norm, *k_norm;
    float *k_cache, *v_cache, *out;
    void *workspace;
    uint64_t workspace_bytes;
} q35_attn_decode_args;
uint64_t q35_attn_decode_workspace_bytes(const q35_attn_decode_args *args);
q35_status q35_attn_decode(const q35_attn_decode_args *args, q35_stream s);

/* q35_attn_decode without a workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops or harnesses that forbid allocation). It has no
 * counterpart in the reference. The split-K partials live in a device array the library
 * owns, Q35_ATTN_STATIC_SCRATCH_BYTES on every GPU it runs on (held until the process ends):
 * args->workspace and workspace_bytes are ignored, and a call whose partials
 * (q35_attn_decode_workspace_bytes) exceed the array fails with Q35_ERR_RANGE. The call
 * allocates nothing. All calls on one GPU share its array: calls that overlap in time on
 * one GPU (other streams, other threads) race. The stream must belong to the current
 * device. Results equal q35_attn_decode's. */
#define Q35_ATTN_STATIC_SCRATCH_BYTES (8u << 20)
q35_status q35_attn_decode_static(const q35_attn_decode_args *args, q35_stream s);

/* GDN over a block of n_tokens prompt tokens at positions pos0 .. pos0 + n_tokens - 1, one
 * layer, chunked (WY form, chunk 64); the replacement of the sequential recurrence of
 * QwenForward::mix_gdn (src/qwen_forward.cpp:109-142). It continues from `state` and
 * `conv_ring` (zeros for a fresh prompt: the reference's left zero pad and S = 0) and leaves
 * them as n_tokens decode steps would. Token-major inputs with leading dimensions:
 *   qkv [n][ld_qkv] (CONV pre-conv channels), z [n][ld_z] (VD), b, a [n][ld_ba] (VH each)
 *   conv_w, A_log, dt_bias, norm_w, conv_ring, state as for q35_gdn_decode
 *   out [n][VD]: gated-rmsnorm output (raw readout when norm_w is NULL)
 * workspace: q35_gdn_prefill_workspace_bytes() bytes. Requires DK == DV == 128, KER == 4;
 * qkv, conv_ring, conv_w and workspace 16-byte aligned and ld_qkv a multiple of 4 (read 16
 * bytes at a time), else Q35_ERR_ARG. */
typedef struct q35_gdn_prefill_args {
    int32_t n_tokens, pos0, k_heads, v_heads, head_dim_k, head_dim_v, conv_kernel;
    float eps;
    const float *qkv, *z, *b, *a;
    int64_t ld_qkv, ld_z, ld_ba;
    const float *conv_w, *A_log, *dt_bias, *norm_w;
    float *conv_ring, *state, *out;
    void *workspace;
    uint64_t workspace_bytes;
} q35_gdn_prefill_args;
uint64_t q35_gdn_prefill_workspace_bytes(const q35_gdn_prefill_args *args);
q35_status q35_gdn_prefill(const q35_gdn_prefill_args *args, q35_stream s);

/* Causal gated attention over a block of n_tokens prompt tokens at positions pos0 .., one
 * layer (QwenForward::mix_attention, src/qwen_forward.cpp:20-80, after its projections):
 * q_norm + RoPE of every query, k_norm + RoPE of every key, the block's K / V rows appended
 * to the caches at pos0 + t, softmax over positions [0, pos0 + t], times sigmoid(gate).
 *   qkv [n][ld_qkv]: NQ x [q | gate] (2 HD each), then NKV x k, then NKV x v
 *   k_cache, v_cache [NKV][max_context][HD]; out [n][NQ * HD]
 * workspace (16-byte aligned): q35_attn_prefill_workspace_bytes() bytes. With an fp32 cache
 * that size includes the keys and values of positions [0, pos0 + n) pre-split into the
 * attention kernel's tile layout (3 KB per position and kv head); a workspace of at least
 * NQ * n * HD * 4 + 256 bytes but smaller than that is accepted, and the kernel then splits
 * every tile itself (slower, same results). Requires HD == 256. */
typedef struct q35_attn_prefill_args {
    int32_t n_tokens, pos0, q_heads, kv_heads, head_dim, rotary_dim;
    int32_t kv_dtype;      /* cache elements: 0 = fp32, 1 = bf16 (as q35_attn_decode_args) */
    int32_t reserved;
    int64_t max_context;
    double rope_theta;
    float eps;
    const float *qkv;
    int64_t ld_qkv;
    const float *q_norm, *k_norm;
    float *k_cache, *v_cache, *out;
    void *workspace;
    uint64_t workspace_bytes;
} q35_attn_prefill_args;
uint64_t q35_attn_prefill_workspace_bytes(const q35_attn_prefill_args *args);
q35_status q35_attn_prefill(const q35_attn_prefill_args *args, q35_stream s);

#ifdef __cplusplus
}
#endif
#endif /* Q35_H */
