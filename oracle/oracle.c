/*
 * oracle.c -- CPU fp32 restatement of the Qwen3.5-CPU-cpp hybrid token-mixer path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker of the parity tests and the "port" CPU baseline of
 * bench.py. The shipped library never links or calls it.
 *
 * Each function names the reference function it restates (file:line in the Qwen3.5-CPU-cpp
 * tree). The arithmetic is kept: fp32 values, sums of squares in double, RoPE angles in
 * double, the 4 x 8-lane fused-multiply-add accumulation of the AVX2 matvec followed by the
 * same horizontal reduction, and the scalar serial loops of the mixers.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <dirent.h>
#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <immintrin.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];
static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
const char *orc_error(void) { return g_err; }

int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------------------------- */
/* scalar activations: include/forward_pass.h:21-24                                    */
/* ---------------------------------------------------------------------------------- */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float orc_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

static inline float bf16f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16; /* include/safetensors_loader.h:69-74 */
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ---------------------------------------------------------------------------------- */
/* matvec: src/forward_pass.cpp:6-75. Four accumulators of eight lanes over 32-wide     */
/* blocks, one eight-lane accumulator over the following 8-wide blocks, the (lo+hi),    */
/* hadd, hadd horizontal sum, then a scalar tail.                                       */
/* ---------------------------------------------------------------------------------- */
/* Eight weights as fp32: bf16 widened exactly (<< 16), or fp32 as stored */
static inline __m256 w8(const uint16_t *wb, const float *wf, int i) {
    if (!wb) return _mm256_loadu_ps(wf + i);
    const __m256i h = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(wb + i)));
    return _mm256_castsi256_ps(_mm256_slli_epi32(h, 16));
}

static float dot_w(const uint16_t *wb, const float *wf, const float *x, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        a0 = _mm256_fmadd_ps(w8(wb, wf, i), _mm256_loadu_ps(x + i), a0);
        a1 = _mm256_fmadd_ps(w8(wb, wf, i + 8), _mm256_loadu_ps(x + i + 8), a1);
        a2 = _mm256_fmadd_ps(w8(wb, wf, i + 16), _mm256_loadu_ps(x + i + 16), a2);
        a3 = _mm256_fmadd_ps(w8(wb, wf, i + 24), _mm256_loadu_ps(x + i + 24), a3);
    }
    __m256 acc = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(w8(wb, wf, i), _mm256_loadu_ps(x + i), acc);
    /* lane l + lane l + 4, then ((s0 + s1) + (s2 + s3)) */
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    float r = _mm_cvtss_f32(s);
    for (; i < n; ++i) r += (wb ? bf16f(wb[i]) : wf[i]) * x[i];
    return r;
}

void orc_matmul_bf16(const uint16_t *W, const float *x, float *y, int out_dim, int in_dim) {
#pragma omp parallel for schedule(static)
    for (int o = 0; o < out_dim; ++o) y[o] = dot_w(W + (size_t)o * in_dim, NULL, x, in_dim);
}

/* The matvec above for n input rows at once: Y[t][o] = dot(W[o], X[t]), every output with
 * exactly the arithmetic of orc_matmul_bf16. Blocks of 64 input rows stay in cache while
 * each weight row is applied to all of them, so a whole prompt streams the weights once
 * per block instead of once per token. */
void orc_matmul_bf16_rows(const uint16_t *W, const float *X, int64_t ldx, float *Y, int64_t ldy,
                          int n, int out_dim, int in_dim) {
    for (int t0 = 0; t0 < n; t0 += 64) {
        const int t1 = t0 + 64 < n ? t0 + 64 : n;
#pragma omp parallel for schedule(static)
        for (int o = 0; o < out_dim; ++o)
            for (int t = t0; t < t1; ++t)
                Y[(size_t)t * ldy + o] = dot_w(W + (size_t)o * in_dim, NULL, X + (size_t)t * ldx, in_dim);
    }
}

void orc_matmul_f32(const float *W, const float *x, float *y, int out_dim, int in_dim) {
#pragma omp parallel for schedule(static)
    for (int o = 0; o < out_dim; ++o) y[o] = dot_w(NULL, W + (size_t)o * in_dim, x, in_dim);
}

/* src/forward_pass.cpp:77-84 -- (1 + w) form, sum of squares in double */
void orc_rmsnorm(const float *x, const float *w, float *y, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    float inv = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv * (1.0f + w[i]);
}

/* src/forward_pass.cpp:86-93 -- plain w, silu(gate) after the normalisation */
void orc_rmsnorm_gated(const float *x, const float *w, const float *gate, float *y, int n,
                       float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    float inv = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; ++i) y[i] = w[i] * (x[i] * inv) * orc_silu(gate[i]);
}

/* src/forward_pass.cpp:95-100 -- sum (not mean) of squares */
void orc_l2norm(float *x, int n, float eps) {
    double s = 0.0;
    for (int i = 0; i < n; ++i) s += (double)x[i] * x[i];
    float inv = 1.0f / sqrtf((float)s + eps);
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

/* src/forward_pass.cpp:102-112 -- rotate-half on [0, rotary_dim), angles in double */
void orc_apply_rope(float *vec, int rotary_dim, int pos, double theta) {
    int half = rotary_dim / 2;
    for (int i = 0; i < half; ++i) {
        double inv_freq = pow(theta, -(double)(2 * i) / rotary_dim);
        double ang = (double)pos * inv_freq;
        float c = (float)cos(ang), s = (float)sin(ang);
        float x1 = vec[i], x2 = vec[i + half];
        vec[i] = x1 * c - x2 * s;
        vec[i + half] = x2 * c + x1 * s;
    }
}

/* ---------------------------------------------------------------------------------- */
/* config: include/model_config.h:11-63 defaults, src/config_loader.cpp:59-108 reader   */
/* ---------------------------------------------------------------------------------- */
void orc_dims_default(orc_dims *d) {
    memset(d, 0, sizeof *d);
    d->hidden_size = 1024;
    d->n_layers_total = 24;
    d->n_layers_gdn = 18;
    d->n_layers_attn = 6;
    d->gdn_k_heads = 16;
    d->gdn_v_heads = 16;
    d->gdn_k_head_dim = 128;
    d->gdn_v_head_dim = 128;
    d->gdn_conv_kernel = 4;
    d->attn_q_heads = 8;
    d->attn_kv_heads = 2;
    d->attn_head_dim = 256;
    d->ffn_intermediate = 3584;
    d->vocab_size = 248320;
    d->native_max_context = 262144;
    d->n_params = 800000000LL;
    d->rope_theta = 10000000.0;
    d->rms_norm_eps = 1e-6f;
    d->partial_rotary_factor = 0.25f;
    d->attn_interval = 4;
    d->tie_word_embeddings = 1;
}

int orc_is_attention_layer(const orc_dims *d, int layer) {
    return ((layer + 1) % d->attn_interval) == 0;
}

/* brace-matched substring of the object that follows "key" (config_loader.cpp:12-25) */
static char *cfg_object(const char *s, const char *key) {
    char pat[128];
    snprintf(pat, sizeof pat, "\"%s\"", key);
    const char *k = strstr(s, pat);
    if (!k) return NULL;
    const char *b = strchr(k, '{');
    if (!b) return NULL;
    int depth = 0;
    for (const char *p = b; *p; ++p) {
        if (*p == '{') ++depth;
        else if (*p == '}' && --depth == 0) return strndup(b, (size_t)(p - b + 1));
    }
    return NULL;
}

/* first "key": number (config_loader.cpp:28-41) */
static int cfg_number(const char *s, const char *key, double *out) {
    char pat[128];
    snprintf(pat, sizeof pat, "\"%s\"", key);
    const char *k = strstr(s, pat);
    if (!k) return 0;
    const char *c = strchr(k, ':');
    if (!c) return 0;
    const char *p = c + 1;
    while (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r') ++p;
    const char *st = p;
    while ((*p >= '0' && *p <= '9') || *p == '-' || *p == '+' || *p == '.' || *p == 'e' ||
           *p == 'E')
        ++p;
    if (p == st) return 0;
    char buf[64];
    size_t len = (size_t)(p - st) < sizeof buf - 1 ? (size_t)(p - st) : sizeof buf - 1;
    memcpy(buf, st, len);
    buf[len] = 0;
    char *end = NULL;
    *out = strtod(buf, &end);
    return end != buf;
}

/* "true" before the next comma (config_loader.cpp:43-51) */
static int cfg_bool(const char *s, const char *key, int *out) {
    char pat[128];
    snprintf(pat, sizeof pat, "\"%s\"", key);
    const char *k = strstr(s, pat);
    if (!k) return 0;
    const char *c = strchr(k, ':');
    if (!c) return 0;
    const char *e = strchr(c, ',');
    const char *t = strstr(c, "true");
    *out = t && (!e || t < e);
    return 1;
}

static int cfg_int(const char *s, const char *key, int fallback) {
    double v;
    return cfg_number(s, key, &v) ? (int)(v + 0.5) : fallback;
}

int orc_load_config(const char *path, orc_dims *d) {
    FILE *f = fopen(path, "rb");
    if (!f) {
        set_err("cannot open %s", path);
        return -1;
    }
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *all = (char *)malloc((size_t)n + 1);
    if (fread(all, 1, (size_t)n, f) != (size_t)n) {
        fclose(f);
        free(all);
        set_err("read failed %s", path);
        return -1;
    }
    all[n] = 0;
    fclose(f);
    char *tc = cfg_object(all, "text_config");
    const char *s = tc ? tc : all;
    d->hidden_size = cfg_int(s, "hidden_size", d->hidden_size);
    d->n_layers_total = cfg_int(s, "num_hidden_layers", d->n_layers_total);
    d->attn_interval = cfg_int(s, "full_attention_interval", d->attn_interval);
    d->attn_q_heads = cfg_int(s, "num_attention_heads", d->attn_q_heads);
    d->attn_kv_heads = cfg_int(s, "num_key_value_heads", d->attn_kv_heads);
    d->attn_head_dim = cfg_int(s, "head_dim", d->attn_head_dim);
    d->gdn_k_heads = cfg_int(s, "linear_num_key_heads", d->gdn_k_heads);
    d->gdn_v_heads = cfg_int(s, "linear_num_value_heads", d->gdn_v_heads);
    d->gdn_k_head_dim = cfg_int(s, "linear_key_head_dim", d->gdn_k_head_dim);
    d->gdn_v_head_dim = cfg_int(s, "linear_value_head_dim", d->gdn_v_head_dim);
    d->gdn_conv_kernel = cfg_int(s, "linear_conv_kernel_dim", d->gdn_conv_kernel);
    d->ffn_intermediate = cfg_int(s, "intermediate_size", d->ffn_intermediate);
    d->vocab_size = cfg_int(s, "vocab_size", d->vocab_size);
    d->native_max_context = cfg_int(s, "max_position_embeddings", (int)d->native_max_context);
    d->n_layers_attn = d->n_layers_total / d->attn_interval;
    d->n_layers_gdn = d->n_layers_total - d->n_layers_attn;
    double v;
    if (cfg_number(s, "rms_norm_eps", &v)) d->rms_norm_eps = (float)v;
    if (cfg_number(s, "rope_theta", &v)) d->rope_theta = v;
    if (cfg_number(s, "partial_rotary_factor", &v)) d->partial_rotary_factor = (float)v;
    int b;
    if (cfg_bool(s, "tie_word_embeddings", &b)) d->tie_word_embeddings = b;
    d->n_params = (int64_t)d->vocab_size * d->hidden_size +
                  (int64_t)d->n_layers_total * 12 * d->hidden_size * d->hidden_size;
    free(tc);
    free(all);
    return 0;
}

/* ---------------------------------------------------------------------------------- */
/* safetensors: 8-byte little-endian header length, JSON header, raw data               */
/* (src/safetensors_loader.cpp:131-234). Files are memory-mapped read-only.            */
/* ---------------------------------------------------------------------------------- */
typedef struct st_entry {
    char *name;
    int dtype; /* 0 bf16, 1 f32, -1 other */
    int ndim;
    int64_t shape[8];
    const uint8_t *data;
    size_t nbytes;
} st_entry;

typedef struct st_file {
    void *map;
    size_t size;
} st_file;

typedef struct jp {
    const char *p, *e;
    int ok;
} jp;

static void jws(jp *j) {
    while (j->p < j->e && (*j->p == ' ' || *j->p == '\n' || *j->p == '\r' || *j->p == '\t'))
        ++j->p;
}
static int jexpect(jp *j, char c) {
    jws(j);
    if (j->p < j->e && *j->p == c) {
        ++j->p;
        return 1;
    }
    j->ok = 0;
    return 0;
}
static char *jstring(jp *j) {
    jws(j);
    if (j->p >= j->e || *j->p != '"') {
        j->ok = 0;
        return NULL;
    }
    ++j->p;
    size_t cap = 64, len = 0;
    char *s = (char *)malloc(cap);
    while (j->p < j->e && *j->p != '"') {
        char c = *j->p;
        if (c == '\\' && j->p + 1 < j->e) {
            ++j->p;
            c = *j->p == 'n' ? '\n' : *j->p == 't' ? '\t' : *j->p;
        }
        if (len + 2 > cap) s = (char *)realloc(s, cap *= 2);
        s[len++] = c;
        ++j->p;
    }
    if (j->p >= j->e) {
        j->ok = 0;
        free(s);
        return NULL;
    }
    ++j->p;
    s[len] = 0;
    return s;
}
static int64_t jint(jp *j) {
    jws(j);
    const char *st = j->p;
    if (j->p < j->e && (*j->p == '-' || *j->p == '+')) ++j->p;
    while (j->p < j->e && *j->p >= '0' && *j->p <= '9') ++j->p;
    if (j->p == st) {
        j->ok = 0;
        return 0;
    }
    return strtoll(st, NULL, 10);
}
static void jskip(jp *j) {
    jws(j);
    if (j->p >= j->e) {
        j->ok = 0;
        return;
    }
    char c = *j->p;
    if (c == '"') {
        free(jstring(j));
    } else if (c == '{' || c == '[') {
        char close = c == '{' ? '}' : ']';
        ++j->p;
        jws(j);
        if (j->p < j->e && *j->p == close) {
            ++j->p;
            return;
        }
        while (j->ok) {
            if (c == '{') {
                free(jstring(j));
                jexpect(j, ':');
            }
            jskip(j);
            jws(j);
            if (j->p < j->e && *j->p == ',') {
                ++j->p;
                continue;
            }
            break;
        }
        jexpect(j, close);
    } else {
        while (j->p < j->e && *j->p != ',' && *j->p != '}' && *j->p != ']') ++j->p;
    }
}

typedef struct st_set {
    st_file files[64];
    int nfiles;
    st_entry *ents;
    int nents, cap;
} st_set;

static int st_parse_file(st_set *S, const char *path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_err("cannot open %s", path);
        return -1;
    }
    struct stat sb;
    fstat(fd, &sb);
    size_t size = (size_t)sb.st_size;
    if (size < 8) {
        close(fd);
        set_err("file too small %s", path);
        return -1;
    }
    void *map = mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        set_err("mmap failed %s", path);
        return -1;
    }
    if (S->nfiles >= 64) {
        set_err("too many shards");
        return -1;
    }
    S->files[S->nfiles].map = map;
    S->files[S->nfiles].size = size;
    S->nfiles++;
    uint64_t hl;
    memcpy(&hl, map, 8);
    if (8 + hl > size) {
        set_err("header length exceeds file %s", path);
        return -1;
    }
    const uint8_t *base = (const uint8_t *)map + 8 + hl;
    jp j = {(const char *)map + 8, (const char *)map + 8 + hl, 1};
    if (!jexpect(&j, '{')) {
        set_err("bad header %s", path);
        return -1;
    }
    jws(&j);
    if (j.p < j.e && *j.p == '}') return 0;
    while (j.ok) {
        char *key = jstring(&j);
        jexpect(&j, ':');
        if (!j.ok) {
            free(key);
            break;
        }
        if (strcmp(key, "__metadata__") == 0) {
            jskip(&j);
            free(key);
        } else {
            st_entry e;
            memset(&e, 0, sizeof e);
            e.name = key;
            e.dtype = -1;
            int64_t o0 = 0, o1 = 0;
            jexpect(&j, '{');
            while (j.ok) {
                char *field = jstring(&j);
                jexpect(&j, ':');
                if (!field) break;
                if (strcmp(field, "dtype") == 0) {
                    char *dt = jstring(&j);
                    if (dt) e.dtype = strcmp(dt, "BF16") == 0 ? 0 : strcmp(dt, "F32") == 0 ? 1 : -1;
                    free(dt);
                } else if (strcmp(field, "shape") == 0 || strcmp(field, "data_offsets") == 0) {
                    int64_t v[8];
                    int nv = 0;
                    jexpect(&j, '[');
                    jws(&j);
                    if (j.p < j.e && *j.p == ']') {
                        ++j.p;
                    } else {
                        while (j.ok) {
                            int64_t x = jint(&j);
                            if (nv < 8) v[nv++] = x;
                            jws(&j);
                            if (j.p < j.e && *j.p == ',') {
                                ++j.p;
                                continue;
                            }
                            break;
                        }
                        jexpect(&j, ']');
                    }
                    if (field[0] == 's') {
                        e.ndim = nv;
                        for (int i = 0; i < nv; ++i) e.shape[i] = v[i];
                    } else if (nv == 2) {
                        o0 = v[0];
                        o1 = v[1];
                    }
                } else {
                    jskip(&j);
                }
                free(field);
                jws(&j);
                if (j.p < j.e && *j.p == ',') {
                    ++j.p;
                    continue;
                }
                break;
            }
            jexpect(&j, '}');
            if ((size_t)(8 + hl + o1) > size || o1 < o0) {
                set_err("tensor %s out of range", e.name);
                free(e.name);
                return -1;
            }
            e.data = base + o0;
            e.nbytes = (size_t)(o1 - o0);
            if (S->nents == S->cap) {
                S->cap = S->cap ? S->cap * 2 : 256;
                S->ents = (st_entry *)realloc(S->ents, sizeof(st_entry) * (size_t)S->cap);
            }
            S->ents[S->nents++] = e;
        }
        jws(&j);
        if (j.p < j.e && *j.p == ',') {
            ++j.p;
            continue;
        }
        break;
    }
    if (!jexpect(&j, '}')) {
        set_err("header parse error %s", path);
        return -1;
    }
    return 0;
}

static int cmpstr(const void *a, const void *b) {
    return strcmp(*(char *const *)a, *(char *const *)b);
}

static int st_load_dir(st_set *S, const char *dir) {
    DIR *dp = opendir(dir);
    if (!dp) {
        set_err("cannot open dir %s", dir);
        return -1;
    }
    char *names[64];
    int n = 0;
    struct dirent *de;
    while ((de = readdir(dp)) != NULL) {
        size_t L = strlen(de->d_name);
        if (L > 12 && strcmp(de->d_name + L - 12, ".safetensors") == 0 && n < 64)
            names[n++] = strdup(de->d_name);
    }
    closedir(dp);
    if (n == 0) {
        set_err("no .safetensors files in %s", dir);
        return -1;
    }
    qsort(names, (size_t)n, sizeof(char *), cmpstr);
    int rc = 0;
    for (int i = 0; i < n; ++i) {
        char path[4096];
        snprintf(path, sizeof path, "%s/%s", dir, names[i]);
        if (rc == 0 && st_parse_file(S, path) != 0) rc = -1;
        free(names[i]);
    }
    return rc;
}

static const st_entry *st_find(const st_set *S, const char *name) {
    for (int i = 0; i < S->nents; ++i)
        if (strcmp(S->ents[i].name, name) == 0) return &S->ents[i];
    return NULL;
}

static int64_t st_numel(const st_entry *e) {
    if (e->ndim == 0) return 0;
    int64_t n = 1;
    for (int i = 0; i < e->ndim; ++i) n *= e->shape[i];
    return n;
}

static void st_free(st_set *S) {
    for (int i = 0; i < S->nfiles; ++i) munmap(S->files[i].map, S->files[i].size);
    for (int i = 0; i < S->nents; ++i) free(S->ents[i].name);
    free(S->ents);
    memset(S, 0, sizeof *S);
}

/* ---------------------------------------------------------------------------------- */
/* isolated mixers                                                                     */
/* ---------------------------------------------------------------------------------- */

/* src/qwen_model.cpp:173-207 */
void orc_gdn_core(const orc_dims *d, const float *qkv, const float *z, const float *b,
                  const float *a, const float *conv_w, const float *A_log,
                  const float *dt_bias, const float *norm_w, float *conv_win, float *S,
                  float *out_raw, float *out) {
    const int KH = d->gdn_k_heads, VH = d->gdn_v_heads, DK = d->gdn_k_head_dim,
              DV = d->gdn_v_head_dim, KER = d->gdn_conv_kernel;
    const int KD = KH * DK, VD = VH * DV, CONV = 2 * KD + VD, rep = VH / KH;
    const float qs = 1.0f / sqrtf((float)DK);
    float *conv = (float *)malloc(sizeof(float) * (size_t)CONV);
    float *Q = (float *)malloc(sizeof(float) * (size_t)KD);
    float *K = (float *)malloc(sizeof(float) * (size_t)KD);
    float *km = (float *)malloc(sizeof(float) * (size_t)DV);
    float *dl = (float *)malloc(sizeof(float) * (size_t)DV);
    float *o = (float *)malloc(sizeof(float) * (size_t)DV);
    /* causal conv over the rolling window, then SiLU; shift the window (:173-183) */
    for (int c = 0; c < CONV; ++c) {
        const float *w4 = conv_w + (size_t)c * KER;
        float *st = conv_win + (size_t)c * (KER - 1);
        float acc = 0.0f;
        for (int k = 0; k < KER - 1; ++k) acc += w4[k] * st[k];
        acc += w4[KER - 1] * qkv[c];
        conv[c] = orc_silu(acc);
        for (int k = 0; k < KER - 2; ++k) st[k] = st[k + 1];
        st[KER - 2] = qkv[c];
    }
    /* l2norm q and k per k-head (eps 1e-6), scale q by DK^-1/2 (:185-190) */
    for (int h = 0; h < KH; ++h) {
        float *q = Q + (size_t)h * DK, *k = K + (size_t)h * DK;
        for (int i = 0; i < DK; ++i) {
            q[i] = conv[h * DK + i];
            k[i] = conv[KD + h * DK + i];
        }
        orc_l2norm(q, DK, 1e-6f);
        orc_l2norm(k, DK, 1e-6f);
        for (int i = 0; i < DK; ++i) q[i] *= qs;
    }
    const float *V = conv + 2 * KD;
    /* per v-head decay, delta rule, readout, gated norm (:193-207) */
    for (int vh = 0; vh < VH; ++vh) {
        const int kh = vh / rep;
        const float g = -expf(A_log[vh]) * orc_softplus(a[vh] + dt_bias[vh]);
        const float gt = expf(g), beta = orc_sigmoid(b[vh]);
        const float *q = Q + (size_t)kh * DK, *k = K + (size_t)kh * DK, *v = V + (size_t)vh * DV;
        float *Sh = S + (size_t)vh * DK * DV;
        for (size_t i = 0; i < (size_t)DK * DV; ++i) Sh[i] *= gt;
        for (int vv = 0; vv < DV; ++vv) {
            float m = 0.0f;
            for (int kk = 0; kk < DK; ++kk) m += Sh[(size_t)kk * DV + vv] * k[kk];
            km[vv] = m;
        }
        for (int vv = 0; vv < DV; ++vv) dl[vv] = (v[vv] - km[vv]) * beta;
        for (int kk = 0; kk < DK; ++kk) {
            const float kv = k[kk];
            float *row = Sh + (size_t)kk * DV;
            for (int vv = 0; vv < DV; ++vv) row[vv] += kv * dl[vv];
        }
        for (int vv = 0; vv < DV; ++vv) {
            float acc = 0.0f;
            for (int kk = 0; kk < DK; ++kk) acc += Sh[(size_t)kk * DV + vv] * q[kk];
            o[vv] = acc;
        }
        if (out_raw) memcpy(out_raw + (size_t)vh * DV, o, sizeof(float) * (size_t)DV);
        if (out) orc_rmsnorm_gated(o, norm_w, z + (size_t)vh * DV, out + (size_t)vh * DV, DV, d->rms_norm_eps);
    }
    free(conv);
    free(Q);
    free(K);
    free(km);
    free(dl);
    free(o);
}

/* fp32 -> nearest bf16 value (ties to even), returned widened. The reference keeps an fp32
 * cache (src/qwen_model.cpp:29-30); this is the rounding a bf16 cache applies to the rows it
 * stores, memory_budget's kv_bytes_per_elem = 2 (include/memory_budget.h:37-42). NaN stays
 * NaN; values that round past the largest bf16 become infinity. */
float orc_round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        u |= 0x00400000u; /* quiet NaN */
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
    }
    u &= 0xffff0000u;
    float y;
    memcpy(&y, &u, 4);
    return y;
}

void orc_round_bf16_array(float *x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_round_bf16(x[i]);
}

void orc_attn_core(const orc_dims *d, int pos, const float *qg, const float *k_new,
                   const float *v_new, const float *q_norm, const float *k_norm,
                   float *kcache, float *vcache, float *out) {
    orc_attn_core_ex(d, pos, qg, k_new, v_new, q_norm, k_norm, kcache, vcache, out, 0, 1);
}

/* src/qwen_model.cpp:119-150 */
void orc_attn_core_ex(const orc_dims *d, int pos, const float *qg, const float *k_new,
                      const float *v_new, const float *q_norm, const float *k_norm,
                      float *kcache, float *vcache, float *out, int kv_bf16, int append) {
    const int NQ = d->attn_q_heads, NKV = d->attn_kv_heads, HD = d->attn_head_dim,
              GRP = NQ / NKV;
    const int ROT = (int)(HD * d->partial_rotary_factor);
    const float eps = d->rms_norm_eps, sc = 1.0f / sqrtf((float)HD);
    float *Q = (float *)malloc(sizeof(float) * (size_t)NQ * HD);
    float *gate = (float *)malloc(sizeof(float) * (size_t)NQ * HD);
    float *sco = (float *)malloc(sizeof(float) * (size_t)(pos + 1));
    for (int h = 0; h < NQ; ++h) {
        const float *src = qg + (size_t)h * HD * 2;
        float *qd = Q + (size_t)h * HD;
        orc_rmsnorm(src, q_norm, qd, HD, eps);
        orc_apply_rope(qd, ROT, pos, d->rope_theta);
        for (int i = 0; i < HD; ++i) gate[(size_t)h * HD + i] = src[HD + i];
    }
    float *kslot = kcache + (size_t)pos * NKV * HD;
    float *vslot = vcache + (size_t)pos * NKV * HD;
    if (append) {
        for (int kh = 0; kh < NKV; ++kh) {
            float *kd = kslot + (size_t)kh * HD;
            orc_rmsnorm(k_new + (size_t)kh * HD, k_norm, kd, HD, eps);
            orc_apply_rope(kd, ROT, pos, d->rope_theta);
        }
        memcpy(vslot, v_new, sizeof(float) * (size_t)NKV * HD);
        if (kv_bf16) {
            orc_round_bf16_array(kslot, (int64_t)NKV * HD);
            orc_round_bf16_array(vslot, (int64_t)NKV * HD);
        }
    }
    for (int h = 0; h < NQ; ++h) {
        const int kh = h / GRP;
        const float *q = Q + (size_t)h * HD;
        float mx = -1e30f;
        for (int j = 0; j <= pos; ++j) {
            const float *k = kcache + ((size_t)j * NKV + kh) * HD;
            float s = 0.0f;
            for (int i = 0; i < HD; ++i) s += q[i] * k[i];
            s *= sc;
            sco[j] = s;
            if (s > mx) mx = s;
        }
        float sm = 0.0f;
        for (int j = 0; j <= pos; ++j) {
            sco[j] = expf(sco[j] - mx);
            sm += sco[j];
        }
        float *oh = out + (size_t)h * HD;
        for (int i = 0; i < HD; ++i) oh[i] = 0.0f;
        for (int j = 0; j <= pos; ++j) {
            const float p = sco[j] / sm;
            const float *v = vcache + ((size_t)j * NKV + kh) * HD;
            for (int i = 0; i < HD; ++i) oh[i] += p * v[i];
        }
    }
    for (int i = 0; i < NQ * HD; ++i) out[i] *= orc_sigmoid(gate[i]);
    free(Q);
    free(gate);
    free(sco);
}

/* ---------------------------------------------------------------------------------- */
/* model: src/qwen_model.cpp:12-255                                                     */
/* ---------------------------------------------------------------------------------- */
typedef struct orc_layer {
    int is_attn, idx;
    float *input_ln, *post_ln;
    const uint16_t *gate, *up, *down;
    const uint16_t *q, *k, *v, *o;
    float *q_norm, *k_norm;
    const uint16_t *in_qkv, *in_z, *in_b, *in_a, *out;
    float *conv1d, *dt_bias, *A_log, *gdn_norm;
} orc_layer;

typedef struct f32copy {
    char *name;
    float *data;
} f32copy;

struct orc_model {
    orc_dims d;
    int max_ctx, pos;
    st_set st;
    f32copy *copies;
    int ncopies;
    orc_layer *L;
    const uint16_t *embed, *head;
    int64_t embed_rows, head_rows;
    float *final_norm;
    float **kc, **vc, **S, **cw;
    float *hidden, *normed, *mix, *ff, *logits;
    float *trace;
    int ok;
    int kv_bf16; /* 1: cache rows stored rounded to bf16 */
    int handoff; /* 1: orc_prefill leaves its final state in the model (see below) */
};

void orc_set_kv_bf16(orc_model *m, int on) { m->kv_bf16 = on ? 1 : 0; }

/* The reference's QwenForward::prefill discards the recurrent state it builds (it starts
 * every call from S = 0, src/qwen_forward.cpp:129-142). With handoff on, orc_prefill keeps
 * it instead, as n token-serial steps would leave it: each GDN layer's final state and conv
 * window (the last KER - 1 pre-conv inputs, oldest first), each attention layer's K / V rows
 * at positions 0 .. n - 1, the residual of the last token, position n. The logits and the
 * per-layer hidden states are unchanged. */
void orc_set_prefill_handoff(orc_model *m, int on) { m->handoff = on ? 1 : 0; }

static const uint16_t *need_bf16(orc_model *m, const char *name) {
    const st_entry *e = st_find(&m->st, name);
    if (!e) {
        set_err("missing weight: %s", name);
        m->ok = 0;
        return NULL;
    }
    if (e->dtype != 0) {
        set_err("weight %s is not BF16", name);
        m->ok = 0;
        return NULL;
    }
    return (const uint16_t *)e->data;
}

static float *need_f32(orc_model *m, const char *name) {
    for (int i = 0; i < m->ncopies; ++i)
        if (strcmp(m->copies[i].name, name) == 0) return m->copies[i].data;
    const st_entry *e = st_find(&m->st, name);
    if (!e) {
        set_err("missing weight: %s", name);
        m->ok = 0;
        return NULL;
    }
    int64_t n = st_numel(e);
    float *buf = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    if (e->dtype == 1) memcpy(buf, e->data, (size_t)n * 4);
    else if (e->dtype == 0)
        for (int64_t i = 0; i < n; ++i) buf[i] = bf16f(((const uint16_t *)e->data)[i]);
    else {
        set_err("unsupported dtype for %s", name);
        m->ok = 0;
        free(buf);
        return NULL;
    }
    m->copies = (f32copy *)realloc(m->copies, sizeof(f32copy) * (size_t)(m->ncopies + 1));
    m->copies[m->ncopies].name = strdup(name);
    m->copies[m->ncopies].data = buf;
    m->ncopies++;
    return buf;
}

const uint16_t *orc_weight_bf16(orc_model *m, const char *name) {
    const st_entry *e = st_find(&m->st, name);
    return (e && e->dtype == 0) ? (const uint16_t *)e->data : NULL;
}
const float *orc_weight_f32(orc_model *m, const char *name) { return need_f32(m, name); }

#define LM "model.language_model."

orc_model *orc_open(const char *dir, int max_context) {
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    m->ok = 1;
    orc_dims_default(&m->d);
    char path[4096];
    snprintf(path, sizeof path, "%s/config.json", dir);
    orc_load_config(path, &m->d); /* absent config keeps the defaults, as the reference */
    if (st_load_dir(&m->st, dir) != 0) {
        orc_close(m);
        return NULL;
    }
    const orc_dims *d = &m->d;
    const int H = d->hidden_size, NKV = d->attn_kv_heads, HD = d->attn_head_dim;
    const int VH = d->gdn_v_heads, DK = d->gdn_k_head_dim, DV = d->gdn_v_head_dim,
              KER = d->gdn_conv_kernel;
    const int CONV = 2 * d->gdn_k_heads * DK + VH * DV;
    m->max_ctx = max_context;
    m->L = (orc_layer *)calloc((size_t)d->n_layers_total, sizeof(orc_layer));
    m->kc = (float **)calloc((size_t)d->n_layers_total, sizeof(float *));
    m->vc = (float **)calloc((size_t)d->n_layers_total, sizeof(float *));
    m->S = (float **)calloc((size_t)d->n_layers_total, sizeof(float *));
    m->cw = (float **)calloc((size_t)d->n_layers_total, sizeof(float *));
    int ai = 0, gi = 0;
    char n[512];
#define NM(suffix) (snprintf(n, sizeof n, LM "layers.%d.%s", l, suffix), n)
    for (int l = 0; l < d->n_layers_total; ++l) {
        orc_layer *L = &m->L[l];
        L->input_ln = need_f32(m, NM("input_layernorm.weight"));
        L->post_ln = need_f32(m, NM("post_attention_layernorm.weight"));
        L->gate = need_bf16(m, NM("mlp.gate_proj.weight"));
        L->up = need_bf16(m, NM("mlp.up_proj.weight"));
        L->down = need_bf16(m, NM("mlp.down_proj.weight"));
        if (orc_is_attention_layer(d, l)) {
            L->is_attn = 1;
            L->idx = ai++;
            L->q = need_bf16(m, NM("self_attn.q_proj.weight"));
            L->k = need_bf16(m, NM("self_attn.k_proj.weight"));
            L->v = need_bf16(m, NM("self_attn.v_proj.weight"));
            L->o = need_bf16(m, NM("self_attn.o_proj.weight"));
            L->q_norm = need_f32(m, NM("self_attn.q_norm.weight"));
            L->k_norm = need_f32(m, NM("self_attn.k_norm.weight"));
            m->kc[L->idx] = (float *)calloc((size_t)max_context * NKV * HD, sizeof(float));
            m->vc[L->idx] = (float *)calloc((size_t)max_context * NKV * HD, sizeof(float));
        } else {
            L->is_attn = 0;
            L->idx = gi++;
            L->in_qkv = need_bf16(m, NM("linear_attn.in_proj_qkv.weight"));
            L->in_z = need_bf16(m, NM("linear_attn.in_proj_z.weight"));
            L->in_b = need_bf16(m, NM("linear_attn.in_proj_b.weight"));
            L->in_a = need_bf16(m, NM("linear_attn.in_proj_a.weight"));
            L->conv1d = need_f32(m, NM("linear_attn.conv1d.weight"));
            L->dt_bias = need_f32(m, NM("linear_attn.dt_bias"));
            L->A_log = need_f32(m, NM("linear_attn.A_log"));
            L->gdn_norm = need_f32(m, NM("linear_attn.norm.weight"));
            L->out = need_bf16(m, NM("linear_attn.out_proj.weight"));
            m->S[L->idx] = (float *)calloc((size_t)VH * DK * DV, sizeof(float));
            m->cw[L->idx] = (float *)calloc((size_t)CONV * (KER - 1), sizeof(float));
        }
    }
#undef NM
    const st_entry *emb = st_find(&m->st, LM "embed_tokens.weight");
    m->embed = need_bf16(m, LM "embed_tokens.weight");
    m->embed_rows = emb && emb->ndim == 2 ? emb->shape[0] : 0;
    m->final_norm = need_f32(m, LM "norm.weight");
    /* untied head first, else the tied embedding (src/qwen_model.cpp:64-69) */
    const char *hn = st_find(&m->st, "lm_head.weight")        ? "lm_head.weight"
                     : st_find(&m->st, LM "lm_head.weight")   ? LM "lm_head.weight"
                                                              : LM "embed_tokens.weight";
    const st_entry *he = st_find(&m->st, hn);
    m->head = need_bf16(m, hn);
    m->head_rows = he && he->ndim == 2 ? he->shape[0] : 0;
    if (m->ok && m->head_rows < d->vocab_size) {
        set_err("output head has %lld rows < vocab %d", (long long)m->head_rows, d->vocab_size);
        m->ok = 0;
    }
    m->hidden = (float *)calloc((size_t)H, sizeof(float));
    m->normed = (float *)calloc((size_t)H, sizeof(float));
    m->mix = (float *)calloc((size_t)H, sizeof(float));
    m->ff = (float *)calloc((size_t)H, sizeof(float));
    m->logits = (float *)calloc((size_t)d->vocab_size, sizeof(float));
    if (!m->ok) {
        orc_close(m);
        return NULL;
    }
    return m;
}

void orc_close(orc_model *m) {
    if (!m) return;
    if (m->L)
        for (int l = 0; l < m->d.n_layers_total; ++l) {
            free(m->kc[l]);
            free(m->vc[l]);
            free(m->S[l]);
            free(m->cw[l]);
        }
    free(m->kc);
    free(m->vc);
    free(m->S);
    free(m->cw);
    free(m->L);
    for (int i = 0; i < m->ncopies; ++i) {
        free(m->copies[i].name);
        free(m->copies[i].data);
    }
    free(m->copies);
    free(m->hidden);
    free(m->normed);
    free(m->mix);
    free(m->ff);
    free(m->logits);
    st_free(&m->st);
    free(m);
}

void orc_get_dims(const orc_model *m, orc_dims *d) { *d = m->d; }
int orc_position(const orc_model *m) { return m->pos; }
void orc_set_position(orc_model *m, int pos) { m->pos = pos; }
void orc_set_trace(orc_model *m, float *trace) { m->trace = trace; }
float *orc_hidden(orc_model *m) { return m->hidden; }
float *orc_gdn_state(orc_model *m, int i) { return m->S[i]; }
float *orc_conv_state(orc_model *m, int i) { return m->cw[i]; }
float *orc_kcache(orc_model *m, int i) { return m->kc[i]; }
float *orc_vcache(orc_model *m, int i) { return m->vc[i]; }

/* src/qwen_model.cpp:98-104 */
void orc_reset(orc_model *m) {
    const orc_dims *d = &m->d;
    const size_t kv = (size_t)m->max_ctx * d->attn_kv_heads * d->attn_head_dim;
    const size_t st = (size_t)d->gdn_v_heads * d->gdn_k_head_dim * d->gdn_v_head_dim;
    const size_t cw = (size_t)(2 * d->gdn_k_heads * d->gdn_k_head_dim +
                               d->gdn_v_heads * d->gdn_v_head_dim) *
                      (d->gdn_conv_kernel - 1);
    m->pos = 0;
    for (int i = 0; i < d->n_layers_attn; ++i) {
        memset(m->kc[i], 0, kv * 4);
        memset(m->vc[i], 0, kv * 4);
    }
    for (int i = 0; i < d->n_layers_gdn; ++i) {
        memset(m->S[i], 0, st * 4);
        memset(m->cw[i], 0, cw * 4);
    }
}

/* QwenModel::attn_step, src/qwen_model.cpp:106-152 */
static void attn_step(orc_model *m, const orc_layer *L, float *out) {
    const orc_dims *d = &m->d;
    const int H = d->hidden_size, NQ = d->attn_q_heads, NKV = d->attn_kv_heads,
              HD = d->attn_head_dim;
    float *qg = (float *)malloc(sizeof(float) * (size_t)NQ * HD * 2);
    float *kn = (float *)malloc(sizeof(float) * (size_t)NKV * HD);
    float *vn = (float *)malloc(sizeof(float) * (size_t)NKV * HD);
    float *ac = (float *)malloc(sizeof(float) * (size_t)NQ * HD);
    orc_matmul_bf16(L->q, m->normed, qg, NQ * HD * 2, H);
    orc_matmul_bf16(L->k, m->normed, kn, NKV * HD, H);
    orc_matmul_bf16(L->v, m->normed, vn, NKV * HD, H);
    orc_attn_core_ex(d, m->pos, qg, kn, vn, L->q_norm, L->k_norm, m->kc[L->idx], m->vc[L->idx], ac,
                     m->kv_bf16, 1);
    orc_matmul_bf16(L->o, ac, out, H, NQ * HD);
    free(qg);
    free(kn);
    free(vn);
    free(ac);
}

/* QwenModel::gdn_step, src/qwen_model.cpp:154-209 */
static void gdn_step(orc_model *m, const orc_layer *L, float *out) {
    const orc_dims *d = &m->d;
    const int H = d->hidden_size, VH = d->gdn_v_heads;
    const int KD = d->gdn_k_heads * d->gdn_k_head_dim, VD = VH * d->gdn_v_head_dim;
    const int CONV = 2 * KD + VD;
    float *qkv = (float *)malloc(sizeof(float) * (size_t)CONV);
    float *z = (float *)malloc(sizeof(float) * (size_t)VD);
    float *b = (float *)malloc(sizeof(float) * (size_t)VH);
    float *a = (float *)malloc(sizeof(float) * (size_t)VH);
    float *gn = (float *)malloc(sizeof(float) * (size_t)VD);
    orc_matmul_bf16(L->in_qkv, m->normed, qkv, CONV, H);
    orc_matmul_bf16(L->in_z, m->normed, z, VD, H);
    orc_matmul_bf16(L->in_b, m->normed, b, VH, H);
    orc_matmul_bf16(L->in_a, m->normed, a, VH, H);
    orc_gdn_core(d, qkv, z, b, a, L->conv1d, L->A_log, L->dt_bias, L->gdn_norm, m->cw[L->idx],
                 m->S[L->idx], NULL, gn);
    orc_matmul_bf16(L->out, gn, out, H, VD);
    free(qkv);
    free(z);
    free(b);
    free(a);
    free(gn);
}

static void embed_row(const orc_model *m, int token, float *dst) {
    const uint16_t *row = m->embed + (size_t)token * m->d.hidden_size;
    for (int i = 0; i < m->d.hidden_size; ++i) dst[i] = bf16f(row[i]);
}

/* FFN block of one token (src/qwen_model.cpp:225-232, src/qwen_forward.cpp:185-191) */
static void ffn(const orc_model *m, const orc_layer *L, const float *x, float *out) {
    const int H = m->d.hidden_size, I = m->d.ffn_intermediate;
    float *g = (float *)malloc(sizeof(float) * (size_t)I);
    float *u = (float *)malloc(sizeof(float) * (size_t)I);
    orc_matmul_bf16(L->gate, x, g, I, H);
    orc_matmul_bf16(L->up, x, u, I, H);
    for (int i = 0; i < I; ++i) g[i] = orc_silu(g[i]) * u[i];
    orc_matmul_bf16(L->down, g, out, H, I);
    free(g);
    free(u);
}

/* The FFN block of n tokens at once (rows of H), each token as ffn() computes it */
static void ffn_rows(const orc_model *m, const orc_layer *L, const float *x, float *out, int n) {
    const int H = m->d.hidden_size, I = m->d.ffn_intermediate;
    float *g = (float *)malloc(sizeof(float) * (size_t)n * I);
    float *u = (float *)malloc(sizeof(float) * (size_t)n * I);
    orc_matmul_bf16_rows(L->gate, x, H, g, I, n, I, H);
    orc_matmul_bf16_rows(L->up, x, H, u, I, n, I, H);
    for (size_t i = 0; i < (size_t)n * I; ++i) g[i] = orc_silu(g[i]) * u[i];
    orc_matmul_bf16_rows(L->down, g, I, out, H, n, H, I);
    free(g);
    free(u);
}

/* QwenModel::step, src/qwen_model.cpp:211-239 */
int orc_step(orc_model *m, int token, float *logits) {
    const orc_dims *d = &m->d;
    const int H = d->hidden_size;
    const float eps = d->rms_norm_eps;
    if (token < 0 || token >= m->embed_rows) {
        set_err("token %d out of range", token);
        return -1;
    }
    if (m->pos >= m->max_ctx) {
        set_err("position %d >= max_context %d", m->pos, m->max_ctx);
        return -1;
    }
    embed_row(m, token, m->hidden);
    for (int l = 0; l < d->n_layers_total; ++l) {
        const orc_layer *L = &m->L[l];
        orc_rmsnorm(m->hidden, L->input_ln, m->normed, H, eps);
        if (L->is_attn) attn_step(m, L, m->mix);
        else gdn_step(m, L, m->mix);
        for (int i = 0; i < H; ++i) m->hidden[i] += m->mix[i];
        orc_rmsnorm(m->hidden, L->post_ln, m->normed, H, eps);
        ffn(m, L, m->normed, m->ff);
        for (int i = 0; i < H; ++i) m->hidden[i] += m->ff[i];
        if (m->trace) memcpy(m->trace + (size_t)l * H, m->hidden, sizeof(float) * (size_t)H);
    }
    orc_rmsnorm(m->hidden, m->final_norm, m->normed, H, eps);
    orc_matmul_bf16(m->head, m->normed, m->logits, d->vocab_size, H);
    m->pos++;
    if (logits) memcpy(logits, m->logits, sizeof(float) * (size_t)d->vocab_size);
    return 0;
}

/* QwenModel::generate_greedy, src/qwen_model.cpp:241-255 (first index of the maximum) */
int orc_generate_greedy(orc_model *m, const int *prompt, int n_prompt, int n_new, int *out) {
    orc_reset(m);
    for (int i = 0; i < n_prompt; ++i)
        if (orc_step(m, prompt[i], NULL) != 0) return -1;
    for (int i = 0; i < n_new; ++i) {
        int am = 0;
        for (int v = 1; v < m->d.vocab_size; ++v)
            if (m->logits[v] > m->logits[am]) am = v;
        out[i] = am;
        if (orc_step(m, am, NULL) != 0) return -1;
    }
    return 0;
}

/* QwenForward::mix_attention, src/qwen_forward.cpp:20-80 */
static void prefill_attention(orc_model *m, const orc_layer *L, const float *in, float *out,
                              int seq) {
    const orc_dims *d = &m->d;
    const int H = d->hidden_size, NQ = d->attn_q_heads, NKV = d->attn_kv_heads,
              HD = d->attn_head_dim, GRP = NQ / NKV;
    const int ROT = (int)(HD * d->partial_rotary_factor);
    const float eps = d->rms_norm_eps, sc = 1.0f / sqrtf((float)HD);
    float *Q = (float *)malloc(sizeof(float) * (size_t)seq * NQ * HD);
    float *Kc = (float *)malloc(sizeof(float) * (size_t)seq * NKV * HD);
    float *Vc = (float *)malloc(sizeof(float) * (size_t)seq * NKV * HD);
    float *gt = (float *)malloc(sizeof(float) * (size_t)seq * NQ * HD);
    /* q_proj / k_proj / v_proj of every token (each output a reference matvec) */
    float *qkv_all = (float *)malloc(sizeof(float) * (size_t)seq * NQ * HD * 2);
    float *kv_all = (float *)malloc(sizeof(float) * (size_t)seq * NKV * HD);
    orc_matmul_bf16_rows(L->q, in, H, qkv_all, (int64_t)NQ * HD * 2, seq, NQ * HD * 2, H);
    orc_matmul_bf16_rows(L->k, in, H, kv_all, (int64_t)NKV * HD, seq, NKV * HD, H);
    orc_matmul_bf16_rows(L->v, in, H, Vc, (int64_t)NKV * HD, seq, NKV * HD, H);
    for (int t = 0; t < seq; ++t) {
        const float *qkv = qkv_all + (size_t)t * NQ * HD * 2, *kv = kv_all + (size_t)t * NKV * HD;
        for (int h = 0; h < NQ; ++h) {
            const float *qgp = qkv + (size_t)h * HD * 2;
            float *qd = Q + ((size_t)t * NQ + h) * HD;
            orc_rmsnorm(qgp, L->q_norm, qd, HD, eps);
            orc_apply_rope(qd, ROT, t, d->rope_theta);
            memcpy(gt + ((size_t)t * NQ + h) * HD, qgp + HD, sizeof(float) * (size_t)HD);
        }
        for (int kh = 0; kh < NKV; ++kh) {
            float *kd = Kc + ((size_t)t * NKV + kh) * HD;
            orc_rmsnorm(kv + (size_t)kh * HD, L->k_norm, kd, HD, eps);
            orc_apply_rope(kd, ROT, t, d->rope_theta);
        }
    }
    /* The (token, query head) pairs are independent: they run in parallel, each with the
     * reference's serial score / softmax / P.V loops in the reference's order. */
    float *att = (float *)malloc(sizeof(float) * (size_t)seq * NQ * HD);
    float *sco_all = (float *)malloc(sizeof(float) * (size_t)seq * orc_threads());
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (int t = 0; t < seq; ++t) {
        for (int h = 0; h < NQ; ++h) {
#ifdef _OPENMP
            float *sco = sco_all + (size_t)omp_get_thread_num() * seq;
#else
            float *sco = sco_all;
#endif
            const int kh = h / GRP;
            const float *q = Q + ((size_t)t * NQ + h) * HD;
            float mx = -1e30f;
            for (int j = 0; j <= t; ++j) {
                const float *k = Kc + ((size_t)j * NKV + kh) * HD;
                float s = 0.0f;
                for (int i = 0; i < HD; ++i) s += q[i] * k[i];
                s *= sc;
                sco[j] = s;
                if (s > mx) mx = s;
            }
            float sm = 0.0f;
            for (int j = 0; j <= t; ++j) {
                sco[j] = expf(sco[j] - mx);
                sm += sco[j];
            }
            float *oh = att + ((size_t)t * NQ + h) * HD;
            for (int i = 0; i < HD; ++i) oh[i] = 0.0f;
            for (int j = 0; j <= t; ++j) {
                const float p = sco[j] / sm;
                const float *v = Vc + ((size_t)j * NKV + kh) * HD;
                for (int i = 0; i < HD; ++i) oh[i] += p * v[i];
            }
        }
    }
    for (int t = 0; t < seq; ++t) {
        float *ac = att + (size_t)t * NQ * HD;
        const float *g = gt + (size_t)t * NQ * HD;
        for (int i = 0; i < NQ * HD; ++i) ac[i] *= orc_sigmoid(g[i]);
    }
    orc_matmul_bf16_rows(L->o, att, (int64_t)NQ * HD, out, H, seq, H, NQ * HD);
    if (m->handoff) {
        const size_t row = (size_t)NKV * HD;
        memcpy(m->kc[L->idx], Kc, sizeof(float) * row * (size_t)seq);
        memcpy(m->vc[L->idx], Vc, sizeof(float) * row * (size_t)seq);
        if (m->kv_bf16) {
            orc_round_bf16_array(m->kc[L->idx], (int64_t)(row * (size_t)seq));
            orc_round_bf16_array(m->vc[L->idx], (int64_t)(row * (size_t)seq));
        }
    }
    free(Q);
    free(Kc);
    free(Vc);
    free(gt);
    free(qkv_all);
    free(kv_all);
    free(att);
    free(sco_all);
}

/* QwenForward::mix_gdn, src/qwen_forward.cpp:83-152 (needs KH == VH, DK == DV) */
static void prefill_gdn(orc_model *m, const orc_layer *L, const float *in, float *out, int seq) {
    const orc_dims *d = &m->d;
    const int H = d->hidden_size, NH = d->gdn_v_heads, D = d->gdn_v_head_dim;
    const int KD = NH * D, VD = NH * D, CONV = 2 * KD + VD, KER = d->gdn_conv_kernel;
    const float eps = d->rms_norm_eps, qs = 1.0f / sqrtf((float)D);
    float *qkv = (float *)malloc(sizeof(float) * (size_t)seq * CONV);
    float *zb = (float *)malloc(sizeof(float) * (size_t)seq * VD);
    float *beta = (float *)malloc(sizeof(float) * (size_t)seq * NH);
    float *g = (float *)malloc(sizeof(float) * (size_t)seq * NH);
    float *bt = (float *)malloc(sizeof(float) * (size_t)seq * NH);
    float *at = (float *)malloc(sizeof(float) * (size_t)seq * NH);
    orc_matmul_bf16_rows(L->in_qkv, in, H, qkv, CONV, seq, CONV, H);
    orc_matmul_bf16_rows(L->in_z, in, H, zb, VD, seq, VD, H);
    orc_matmul_bf16_rows(L->in_b, in, H, bt, NH, seq, NH, H);
    orc_matmul_bf16_rows(L->in_a, in, H, at, NH, seq, NH, H);
    for (int t = 0; t < seq; ++t) {
        for (int h = 0; h < NH; ++h) {
            beta[(size_t)t * NH + h] = orc_sigmoid(bt[(size_t)t * NH + h]);
            g[(size_t)t * NH + h] = -expf(L->A_log[h]) * orc_softplus(at[(size_t)t * NH + h] + L->dt_bias[h]);
        }
    }
    if (m->handoff) /* window [CONV][KER-1]: inputs of tokens seq-KER+1 .. seq-1, oldest first */
        for (int c = 0; c < CONV; ++c)
            for (int k = 0; k < KER - 1; ++k) {
                const int s = seq - (KER - 1) + k;
                m->cw[L->idx][(size_t)c * (KER - 1) + k] = s >= 0 ? qkv[(size_t)s * CONV + c] : 0.0f;
            }
    float *conv = (float *)malloc(sizeof(float) * (size_t)seq * CONV);
    for (int c = 0; c < CONV; ++c) {
        const float *w4 = L->conv1d + (size_t)c * KER;
        for (int t = 0; t < seq; ++t) {
            float acc = 0.0f;
            for (int k = 0; k < KER; ++k) {
                int s = t - (KER - 1) + k;
                if (s >= 0) acc += w4[k] * qkv[(size_t)s * CONV + c];
            }
            conv[(size_t)t * CONV + c] = orc_silu(acc);
        }
    }
    float *Q = (float *)malloc(sizeof(float) * (size_t)seq * KD);
    float *K = (float *)malloc(sizeof(float) * (size_t)seq * KD);
    float *V = (float *)malloc(sizeof(float) * (size_t)seq * VD);
    for (int t = 0; t < seq; ++t) {
        const float *c = conv + (size_t)t * CONV;
        for (int h = 0; h < NH; ++h) {
            float *q = Q + ((size_t)t * NH + h) * D, *k = K + ((size_t)t * NH + h) * D,
                  *v = V + ((size_t)t * NH + h) * D;
            for (int i = 0; i < D; ++i) {
                q[i] = c[h * D + i];
                k[i] = c[KD + h * D + i];
                v[i] = c[2 * KD + h * D + i];
            }
            orc_l2norm(q, D, 1e-6f);
            orc_l2norm(k, D, 1e-6f);
            for (int i = 0; i < D; ++i) q[i] *= qs;
        }
    }
    /* Heads are independent: each runs the reference's serial recurrence from S = 0, in the
     * reference's order, on a thread of its own. */
    float *core = (float *)malloc(sizeof(float) * (size_t)seq * VD);
#pragma omp parallel
    {
        float *S = (float *)malloc(sizeof(float) * (size_t)D * D);
        float *km = (float *)malloc(sizeof(float) * (size_t)D);
        float *dl = (float *)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
        for (int h = 0; h < NH; ++h) {
            memset(S, 0, sizeof(float) * (size_t)D * D);
            for (int t = 0; t < seq; ++t) {
                const float gtt = expf(g[(size_t)t * NH + h]), b = beta[(size_t)t * NH + h];
                const float *q = Q + ((size_t)t * NH + h) * D, *k = K + ((size_t)t * NH + h) * D,
                            *v = V + ((size_t)t * NH + h) * D;
                for (size_t i = 0; i < (size_t)D * D; ++i) S[i] *= gtt;
                for (int vv = 0; vv < D; ++vv) {
                    float acc = 0.0f;
                    for (int kk = 0; kk < D; ++kk) acc += S[(size_t)kk * D + vv] * k[kk];
                    km[vv] = acc;
                }
                for (int vv = 0; vv < D; ++vv) dl[vv] = (v[vv] - km[vv]) * b;
                for (int kk = 0; kk < D; ++kk) {
                    const float kv = k[kk];
                    float *row = S + (size_t)kk * D;
                    for (int vv = 0; vv < D; ++vv) row[vv] += kv * dl[vv];
                }
                float *o = core + ((size_t)t * NH + h) * D;
                for (int vv = 0; vv < D; ++vv) {
                    float acc = 0.0f;
                    for (int kk = 0; kk < D; ++kk) acc += S[(size_t)kk * D + vv] * q[kk];
                    o[vv] = acc;
                }
            }
            if (m->handoff)
                memcpy(m->S[L->idx] + (size_t)h * D * D, S, sizeof(float) * (size_t)D * D);
        }
        free(S);
        free(km);
        free(dl);
    }
    float *gn = (float *)malloc(sizeof(float) * (size_t)seq * VD);
    for (int t = 0; t < seq; ++t)
        for (int h = 0; h < NH; ++h)
            orc_rmsnorm_gated(core + ((size_t)t * NH + h) * D, L->gdn_norm,
                              zb + ((size_t)t * NH + h) * D, gn + ((size_t)t * NH + h) * D, D, eps);
    orc_matmul_bf16_rows(L->out, gn, VD, out, H, seq, H, VD);
    free(qkv);
    free(zb);
    free(beta);
    free(g);
    free(bt);
    free(at);
    free(conv);
    free(Q);
    free(K);
    free(V);
    free(core);
    free(gn);
}

/* QwenForward::prefill, src/qwen_forward.cpp:154-206 (stateless; vocab = embed rows) */
int orc_prefill(orc_model *m, const int *ids, int n, float *logits) {
    const orc_dims *d = &m->d;
    const int H = d->hidden_size;
    const float eps = d->rms_norm_eps;
    if (d->gdn_k_heads != d->gdn_v_heads || d->gdn_k_head_dim != d->gdn_v_head_dim) {
        set_err("prefill needs equal GDN key/value heads and dims");
        return -1;
    }
    if (m->handoff && n > m->max_ctx) {
        set_err("prefill of %d tokens exceeds max_context %d", n, m->max_ctx);
        return -1;
    }
    float *hidden = (float *)malloc(sizeof(float) * (size_t)n * H);
    float *normed = (float *)malloc(sizeof(float) * (size_t)n * H);
    float *mix = (float *)malloc(sizeof(float) * (size_t)n * H);
    float *ff = (float *)malloc(sizeof(float) * (size_t)H);
    for (int t = 0; t < n; ++t) {
        if (ids[t] < 0 || ids[t] >= m->embed_rows) {
            set_err("embedding lookup failed (id %d)", ids[t]);
            free(hidden);
            free(normed);
            free(mix);
            free(ff);
            return -1;
        }
        embed_row(m, ids[t], hidden + (size_t)t * H);
    }
    for (int l = 0; l < d->n_layers_total; ++l) {
        const orc_layer *L = &m->L[l];
        for (int t = 0; t < n; ++t)
            orc_rmsnorm(hidden + (size_t)t * H, L->input_ln, normed + (size_t)t * H, H, eps);
        if (L->is_attn) prefill_attention(m, L, normed, mix, n);
        else prefill_gdn(m, L, normed, mix, n);
        for (size_t i = 0; i < (size_t)n * H; ++i) hidden[i] += mix[i];
        for (int t = 0; t < n; ++t)
            orc_rmsnorm(hidden + (size_t)t * H, L->post_ln, normed + (size_t)t * H, H, eps);
        ffn_rows(m, L, normed, mix, n);
        for (size_t i = 0; i < (size_t)n * H; ++i) hidden[i] += mix[i];
        if (m->trace)
            for (int t = 0; t < n; ++t)
                memcpy(m->trace + ((size_t)t * d->n_layers_total + l) * H,
                       hidden + (size_t)t * H, sizeof(float) * (size_t)H);
    }
    if (logits) {
        const int64_t vocab = m->embed_rows;
        float *fn = (float *)malloc(sizeof(float) * (size_t)n * H);
        for (int t = 0; t < n; ++t) orc_rmsnorm(hidden + (size_t)t * H, m->final_norm, fn + (size_t)t * H, H, eps);
        orc_matmul_bf16_rows(m->embed, fn, H, logits, vocab, n, (int)vocab, H);
        free(fn);
    }
    if (m->handoff) {
        memcpy(m->hidden, hidden + (size_t)(n - 1) * H, sizeof(float) * (size_t)H);
        m->pos = n;
    }
    free(hidden);
    free(normed);
    free(mix);
    free(ff);
    return 0;
}
