/*
 * oracle.h -- CPU fp32 restatement of the Qwen3.5-CPU-cpp hybrid token-mixer path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the parity tests compare the HIP
 * path against, and the "port" CPU baseline of bench.py. Nothing in the shipped library
 * (libq35.so) links, loads or calls it.
 *
 * Every function follows a reference function (paths relative to the Qwen3.5-CPU-cpp
 * tree) and keeps its arithmetic: fp32 values, double-precision sums in the norms,
 * double-precision RoPE angles, the 4x8-lane dot-product accumulation of the AVX2 matvec.
 *
 * Layouts are the reference ones: GDN state [VH][DK][DV] (S[kk*DV+vv]), conv window
 * [CONV][KER-1] oldest first, KV cache [max_context][NKV][HD].
 */
#ifndef Q35_ORACLE_H
#define Q35_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_dims {
    int32_t hidden_size, n_layers_total, n_layers_gdn, n_layers_attn;
    int32_t gdn_k_heads, gdn_v_heads, gdn_k_head_dim, gdn_v_head_dim, gdn_conv_kernel;
    int32_t attn_q_heads, attn_kv_heads, attn_head_dim;
    int32_t ffn_intermediate, vocab_size;
    int64_t native_max_context, n_params;
    double rope_theta;
    float rms_norm_eps, partial_rotary_factor;
    int32_t attn_interval, tie_word_embeddings;
} orc_dims;

/* scalar activations: include/forward_pass.h:21-24 */
float orc_silu(float x);
float orc_sigmoid(float x);
float orc_softplus(float x);

/* primitives: src/forward_pass.cpp */
void orc_matmul_bf16(const uint16_t *W, const float *x, float *y, int out_dim, int in_dim);
void orc_matmul_bf16_rows(const uint16_t *W, const float *X, int64_t ldx, float *Y, int64_t ldy,
                          int n, int out_dim, int in_dim);
void orc_matmul_f32(const float *W, const float *x, float *y, int out_dim, int in_dim);
void orc_rmsnorm(const float *x, const float *w, float *y, int n, float eps);
void orc_rmsnorm_gated(const float *x, const float *w, const float *gate, float *y, int n,
                       float eps);
void orc_l2norm(float *x, int n, float eps);
void orc_apply_rope(float *vec, int rotary_dim, int pos, double theta);

/* config + memory plan: src/config_loader.cpp:59-108, src/memory_budget.cpp:30-81 */
void orc_dims_default(orc_dims *d);
int orc_load_config(const char *path, orc_dims *d); /* 0 ok */
int orc_is_attention_layer(const orc_dims *d, int layer);

/* GDN mixer after the projections, one token, one layer (src/qwen_model.cpp:173-207).
 * conv_win [CONV][KER-1] and S [VH][DK][DV] are updated in place. out_raw receives S^T q
 * per v-head, out receives rmsnorm_gated(out_raw, norm_w, z). Either may be NULL. */
void orc_gdn_core(const orc_dims *d, const float *qkv, const float *z, const float *b,
                  const float *a, const float *conv_w, const float *A_log,
                  const float *dt_bias, const float *norm_w, float *conv_win, float *S,
                  float *out_raw, float *out);

/* Attention mixer after the projections, one token, one layer (src/qwen_model.cpp:119-150).
 * Writes the normed+roped key and v_new to row pos of the caches [max][NKV][HD] and the
 * gated attention output [NQ*HD]. */
void orc_attn_core(const orc_dims *d, int pos, const float *qg, const float *k_new,
                   const float *v_new, const float *q_norm, const float *k_norm,
                   float *kcache, float *vcache, float *out);
/* Same with a bf16 cache (kv_bf16 = 1: the appended rows are stored rounded to the nearest
 * bf16, ties to even, before the attention reads them). append = 0 leaves row pos as the
 * caller put it (k_new / v_new / k_norm unused): the attention over given cache contents. */
void orc_attn_core_ex(const orc_dims *d, int pos, const float *qg, const float *k_new,
                      const float *v_new, const float *q_norm, const float *k_norm,
                      float *kcache, float *vcache, float *out, int kv_bf16, int append);
float orc_round_bf16(float x);
void orc_round_bf16_array(float *x, int64_t n);

/* whole model: src/qwen_model.cpp:12-255, src/qwen_forward.cpp:154-206 */
typedef struct orc_model orc_model;
orc_model *orc_open(const char *dir, int max_context);  /* NULL on failure */
void orc_close(orc_model *m);
void orc_set_kv_bf16(orc_model *m, int on); /* store cache rows rounded to bf16 from now on */
/* orc_prefill leaves its final state (GDN state, conv window, KV rows, residual, position) */
void orc_set_prefill_handoff(orc_model *m, int on);
const char *orc_error(void);
void orc_get_dims(const orc_model *m, orc_dims *d);
void orc_reset(orc_model *m);
int orc_step(orc_model *m, int token, float *logits);  /* logits may be NULL */
int orc_generate_greedy(orc_model *m, const int *prompt, int n_prompt, int n_new, int *out);
int orc_prefill(orc_model *m, const int *ids, int n, float *logits);  /* n * vocab */
int orc_position(const orc_model *m);
void orc_set_position(orc_model *m, int pos);
/* per-layer residual stream after each layer of every step: n_layers_total * H floats */
void orc_set_trace(orc_model *m, float *trace);
float *orc_hidden(orc_model *m);
float *orc_gdn_state(orc_model *m, int gdn_idx);
float *orc_conv_state(orc_model *m, int gdn_idx);
float *orc_kcache(orc_model *m, int attn_idx);
float *orc_vcache(orc_model *m, int attn_idx);
/* Weight pointers of one tensor (bf16 view of the file, or an fp32 copy). */
const uint16_t *orc_weight_bf16(orc_model *m, const char *name);
const float *orc_weight_f32(orc_model *m, const char *name);
/* Number of OpenMP threads the matvec uses (for the CPU baseline report). */
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
