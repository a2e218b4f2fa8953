// Device-resident decoder behind the model-level C ABI (QwenModel, src/qwen_model.cpp).
//
// Memory plan: four device arenas, one hipMalloc each, made when the model is created:
//   weights  every projection as bf16 (layer matrices fused row-wise where one matvec
//            serves several reference matmuls), small vectors widened to fp32
//   state    GDN states [L_gdn][VH][DK][DV] fp32, conv rings [L_gdn][4][CONV] fp32
//   kv       [L_attn][K|V][NKV][max_context][HD] fp32
//   scratch  per-step activations, split-K partials, logits, argmax partials, device
//            token / position, the greedy id history
// A decode step launches kernels only: no allocation, no host synchronisation. The
// position lives on the device, so a captured step graph replays unchanged every token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../host/memory_budget.h"
#include "../host/model_config.h"
#include "../host/q35_internal.h"
#include "../host/safetensors_loader.h"
#include "../host/synth.h"
#include "launch.hpp"

namespace {

std::atomic<int64_t> g_dev_allocs{0};

#define HIPCHK(expr)                                                                        \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return q35::fail(Q35_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));  \
    } while (0)

hipError_t dev_alloc(void** p, size_t bytes) {
    g_dev_allocs.fetch_add(1);
    return hipMalloc(p, bytes);
}

}  // namespace

void q35::count_device_alloc() { g_dev_allocs.fetch_add(1); }

namespace {

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// split-K workspace is sized for this many splits per kv head
constexpr int kMaxSplits = 1024;
// greedy runs replay a graph of this many consecutive steps (one launch per run)
constexpr int kGraphRun = 8;
// device memory left free when the KV capacity is planned from the device's memory
constexpr size_t kSolveMarginBytes = size_t{1} << 30;

struct LayerDev {
    bool attn = false;
    int idx = 0;
    const uint16_t* w_in = nullptr;   // GDN [qkv|z|b|a] or attention [q|k|v], rows x H
    const uint16_t* w_out = nullptr;  // out_proj / o_proj
    const uint16_t* w_gu = nullptr;   // gate / up rows interleaved, 2I x H
    const uint16_t* w_down = nullptr; // H x I
    const float* input_ln = nullptr;
    const float* post_ln = nullptr;
    const float* conv_w = nullptr;
    const float* A_log = nullptr;
    const float* dt_bias = nullptr;
    const float* gdn_norm = nullptr;
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    int in_rows = 0;
    // the prefill's fp16 copies of w_in, w_out, w_gu, w_down (in the prompt arena):
    // wh[i] = w x 2^we[i], wn[i] elements
    uint16_t* wh[4] = {nullptr, nullptr, nullptr, nullptr};
    int we[4] = {0, 0, 0, 0};
    int64_t wn[4] = {0, 0, 0, 0};
};

}  // namespace

struct q35_model {
    q35_dims d{};
    int64_t max_ctx = 0;
    hipStream_t stream = nullptr;
    uint8_t* w_arena = nullptr;
    size_t w_bytes = 0;
    float* state_arena = nullptr;
    size_t state_bytes = 0;
    float* kv_arena = nullptr;
    size_t kv_bytes = 0;
    int kv_elem = 4;  // bytes per KV cache element: 4 (fp32) or 2 (bf16)
    uint8_t* scratch = nullptr;
    size_t scratch_bytes = 0;

    std::vector<LayerDev> layers;
    const uint16_t* embed = nullptr;
    const uint16_t* head = nullptr;
    int64_t embed_rows = 0;
    const float* final_norm = nullptr;

    float* gdn_state = nullptr;  // inside state_arena
    float* conv_ring = nullptr;

    float *hidden = nullptr, *proj = nullptr, *mix = nullptr, *gu = nullptr;
    float *part_o = nullptr, *part_ml = nullptr, *logits = nullptr, *trace = nullptr;
    float* rope_cs = nullptr;  // [max_context][ROT] RoPE cos / sin table
    void* argmax_part = nullptr;
    int *token_dev = nullptr, *pos_dev = nullptr, *ids_dev = nullptr;
    int n_splits = 0;
    int n_cu = 256;

    int64_t pos = 0;  // host mirror of *pos_dev
    int32_t* pinned_token = nullptr;

    // prompt arena: token-block activations of the chunked prefill (one hipMalloc), planned
    // at creation for blocks of up to pf_planned tokens, or made by the first prefill when
    // none was planned (and made again only for a larger block)
    uint8_t* pf_arena = nullptr;
    size_t pf_bytes = 0;
    int pf_block = 0;    // requested block size (0 = automatic)
    int pf_planned = 0;  // block size planned at creation (0: none)
    int pf_exact = 0;    // prefill GEMMs on three exact bf16 parts (no fp16 weight copies)
    int prefill_head = 0;  // prefill logits: 0 = the step's output head, 1 = the embedding

    bool use_graph = true;
    bool graph_valid = false;
    bool trace_on = false;
    bool timing_on = false;
    hipGraph_t graph = nullptr;        // one step
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph_run = nullptr;    // kGraphRun steps back to back (greedy runs)
    hipGraphExec_t exec_run = nullptr;

    std::vector<hipEvent_t> ev;  // timing event pairs
    std::vector<int> ev_class;
    size_t ev_used = 0;
    double kt_ms[Q35_KT_COUNT] = {};
    int64_t kt_n[Q35_KT_COUNT] = {};

    q35_budget budget{};
};

namespace {

// ------------------------------------------------------------------ shape checks
q35_status check_dims(const q35_dims& d) {
    if (d.hidden_size <= 0 || d.n_layers_total <= 0 || d.attn_interval <= 0 || d.vocab_size <= 0)
        return q35::fail(Q35_ERR_ARG, "invalid dims");
    if (d.gdn_k_head_dim != 128 || d.gdn_v_head_dim != 128)
        return q35::fail(Q35_ERR_UNSUPPORTED, "GDN head dims must be 128 (got %d/%d)",
                         d.gdn_k_head_dim, d.gdn_v_head_dim);
    if (d.gdn_conv_kernel != 4)
        return q35::fail(Q35_ERR_UNSUPPORTED, "conv kernel must be 4 (got %d)", d.gdn_conv_kernel);
    if (d.gdn_k_heads <= 0 || d.gdn_v_heads % d.gdn_k_heads != 0 || d.gdn_v_heads > 64)
        return q35::fail(Q35_ERR_UNSUPPORTED, "GDN heads %d/%d unsupported", d.gdn_k_heads, d.gdn_v_heads);
    if (d.attn_head_dim != 256)
        return q35::fail(Q35_ERR_UNSUPPORTED, "attention head_dim must be 256 (got %d)", d.attn_head_dim);
    if (d.attn_kv_heads <= 0 || d.attn_q_heads % d.attn_kv_heads != 0)
        return q35::fail(Q35_ERR_UNSUPPORTED, "attention heads %d/%d", d.attn_q_heads, d.attn_kv_heads);
    const int grp = d.attn_q_heads / d.attn_kv_heads;
    if (grp != 1 && grp != 2 && grp != 4 && grp != 8 && grp != 16)
        return q35::fail(Q35_ERR_UNSUPPORTED, "GQA group %d not in {1,2,4,8,16}", grp);
    const int rot = static_cast<int>(d.attn_head_dim * d.partial_rotary_factor);
    if (rot < 0 || rot > d.attn_head_dim || (rot & 1))
        return q35::fail(Q35_ERR_UNSUPPORTED, "rotary dims %d", rot);
    const int H = d.hidden_size, I = d.ffn_intermediate;
    const int VD = d.gdn_v_heads * 128, QD = d.attn_q_heads * 256;
    for (int n : {H, I, VD, QD})
        if (n % 8 != 0 || n > q35k::kGemvMaxIn)
            return q35::fail(Q35_ERR_UNSUPPORTED, "matvec input width %d (needs %%8 == 0, <= %d)", n,
                             q35k::kGemvMaxIn);
    return Q35_OK;
}

int rot_dims(const q35_dims& d) { return static_cast<int>(d.attn_head_dim * d.partial_rotary_factor); }

// ------------------------------------------------------------------ weight arena layout
struct Piece {
    const q35_tensor* src;
    size_t off;   // byte offset in the arena
    bool to_f32;  // widen to fp32 (small vectors) instead of keeping bf16
    // rows interleaved with a second matrix of the same shape: src row i goes to arena row
    // 2i, partner row i to row 2i + 1
    const q35_tensor* partner = nullptr;
    int64_t cols = 0;
};

int64_t numel_of(const q35_tensor* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
    return t->ndim > 0 ? n : 0;
}

class ArenaPlanner {
public:
    explicit ArenaPlanner(const q35_tensor* ts, int n) : ts_(ts), n_(n) {}
    const q35_tensor* find(const std::string& name) const {
        for (int i = 0; i < n_; ++i)
            if (ts_[i].name && name == ts_[i].name) return &ts_[i];
        return nullptr;
    }
    // bf16 matrix rows x cols; returns arena offset or SIZE_MAX with the error set
    size_t mat(const std::vector<std::string>& names, int64_t cols, int64_t* rows_out, q35_status* st) {
        int64_t rows = 0;
        const size_t off = cursor_;
        for (const std::string& nm : names) {
            const q35_tensor* t = find(nm);
            if (!t) {
                *st = q35::fail(Q35_ERR_MISSING, "missing weight: %s", nm.c_str());
                return SIZE_MAX;
            }
            if (t->dtype != 0) {
                *st = q35::fail(Q35_ERR_UNSUPPORTED, "weight %s must be BF16", nm.c_str());
                return SIZE_MAX;
            }
            const int64_t n = numel_of(t);
            if (n % cols != 0 || t->shape[t->ndim - 1] != cols) {
                *st = q35::fail(Q35_ERR_FORMAT, "weight %s has %lld elements, not a multiple of %lld columns",
                                nm.c_str(), static_cast<long long>(n), static_cast<long long>(cols));
                return SIZE_MAX;
            }
            pieces_.push_back({t, cursor_ + static_cast<size_t>(rows * cols) * 2, false});
            rows += n / cols;
        }
        cursor_ = align256(cursor_ + static_cast<size_t>(rows * cols) * 2);
        if (rows_out) *rows_out = rows;
        return off;
    }
    // Two matrices of equal shape with their rows interleaved (a row, b row, a row, ...):
    // [gate_proj; up_proj] for the matvec whose epilogue is silu(gate_i) * up_i.
    size_t mat_interleaved(const std::string& a, const std::string& b, int64_t cols, int64_t* rows_out,
                           q35_status* st) {
        const q35_tensor* ta = find(a);
        const q35_tensor* tb = find(b);
        if (!ta || !tb) {
            *st = q35::fail(Q35_ERR_MISSING, "missing weight: %s", (ta ? b : a).c_str());
            return SIZE_MAX;
        }
        if (ta->dtype != 0 || tb->dtype != 0) {
            *st = q35::fail(Q35_ERR_UNSUPPORTED, "weights %s / %s must be BF16", a.c_str(), b.c_str());
            return SIZE_MAX;
        }
        const int64_t na = numel_of(ta), nb = numel_of(tb);
        if (na != nb || na % cols != 0 || ta->shape[ta->ndim - 1] != cols) {
            *st = q35::fail(Q35_ERR_FORMAT, "weights %s / %s: shapes differ or are not [rows][%lld]", a.c_str(),
                            b.c_str(), static_cast<long long>(cols));
            return SIZE_MAX;
        }
        const size_t off = cursor_;
        Piece pc{ta, off, false};
        pc.partner = tb;
        pc.cols = cols;
        pieces_.push_back(pc);
        cursor_ = align256(cursor_ + static_cast<size_t>(2 * na) * 2);
        if (rows_out) *rows_out = 2 * na / cols;
        return off;
    }
    size_t vec(const std::string& name, int64_t expect, q35_status* st) {
        const q35_tensor* t = find(name);
        if (!t) {
            *st = q35::fail(Q35_ERR_MISSING, "missing weight: %s", name.c_str());
            return SIZE_MAX;
        }
        if (t->dtype != 0 && t->dtype != 1) {
            *st = q35::fail(Q35_ERR_UNSUPPORTED, "weight %s: unsupported dtype", name.c_str());
            return SIZE_MAX;
        }
        if (numel_of(t) != expect) {
            *st = q35::fail(Q35_ERR_FORMAT, "weight %s has %lld elements, expected %lld", name.c_str(),
                            static_cast<long long>(numel_of(t)), static_cast<long long>(expect));
            return SIZE_MAX;
        }
        const size_t off = cursor_;
        pieces_.push_back({t, off, true});
        cursor_ = align256(cursor_ + static_cast<size_t>(expect) * 4);
        return off;
    }
    size_t bytes() const { return cursor_; }
    const std::vector<Piece>& pieces() const { return pieces_; }

private:
    const q35_tensor* ts_;
    int n_;
    size_t cursor_ = 0;
    std::vector<Piece> pieces_;
};

// Start of the cache rows of (attention layer, K = 0 / V = 1, kv head), whatever the element
// width (the kernels take the arena as float* and index it by elements of the cache type).
float* kv_ptr(const q35_model* m, int layer, int which, int kh) {
    const int64_t elems = ((static_cast<int64_t>(layer) * 2 + which) * m->d.attn_kv_heads + kh) * m->max_ctx *
                          m->d.attn_head_dim;
    return reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(m->kv_arena) + elems * m->kv_elem);
}

// ------------------------------------------------------------------ step enqueue
struct Launcher {
    q35_model* m;
    hipStream_t s;
    bool timed;
    q35_status st = Q35_OK;

    template <class F>
    void run(int cls, F&& f) {
        if (st != Q35_OK) return;
        if (timed) {
            if (m->ev_used + 2 > m->ev.size()) {
                hipEvent_t a = nullptr, b = nullptr;
                if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
                    st = q35::fail(Q35_ERR_HIP, "hipEventCreate failed");
                    return;
                }
                m->ev.push_back(a);
                m->ev.push_back(b);
                m->ev_class.push_back(cls);
            }
            m->ev_class[m->ev_used / 2] = cls;
        }
        // timed: the launches inside f() stamp the pair with their own start / end
        q35k::LaunchTimer timer{timed ? m->ev[m->ev_used] : nullptr, timed ? m->ev[m->ev_used + 1] : nullptr, false};
        if (timed) q35k::launch_timer() = &timer;
        const hipError_t e = f();
        if (timed) q35k::launch_timer() = nullptr;
        if (e != hipSuccess) st = q35::fail(Q35_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
        if (timed) {
            if (!timer.started && st == Q35_OK &&  // nothing launched: an empty interval
                (hipEventRecord(timer.start, s) != hipSuccess || hipEventRecord(timer.stop, s) != hipSuccess))
                st = q35::fail(Q35_ERR_HIP, "hipEventRecord failed");
            m->ev_used += 2;
        }
    }
};

q35_status enqueue_step(q35_model* m, hipStream_t s, bool timed) {
    const q35_dims& d = m->d;
    const int H = d.hidden_size, I = d.ffn_intermediate;
    const int KH = d.gdn_k_heads, VH = d.gdn_v_heads, KD = KH * 128, VD = VH * 128;
    const int CONV = 2 * KD + VD;
    const int NQ = d.attn_q_heads, NKV = d.attn_kv_heads, HD = d.attn_head_dim;
    Launcher L{m, s, timed};
    for (size_t li = 0; li < m->layers.size(); ++li) {
        const LayerDev& ly = m->layers[li];
        q35k::GemvArgs g{};
        g.W = ly.w_in;
        g.x = m->hidden;
        if (li == 0) {  // the token's embedding row is the first projection's input (and hidden)
            g.embed = m->embed;
            g.token = m->token_dev;
            g.x_out = m->hidden;
        }
        g.norm_w = ly.input_ln;
        g.y = m->proj;
        g.rows = ly.in_rows;
        g.in_dim = H;
        g.eps = d.rms_norm_eps;
        if (!ly.attn) {  // the conv window runs in the in-projection's epilogue
            g.conv_w = ly.conv_w;
            g.conv_ring = m->conv_ring + static_cast<int64_t>(ly.idx) * 4 * CONV;
            g.pos_dev = m->pos_dev;
            g.conv_rows = CONV;
        }
        L.run(Q35_KT_GEMV, [&] {
            return q35k::launch_gemv(g, q35k::kProRmsNorm, s, ly.attn ? q35k::kEpiAuto : q35k::kEpiConvSilu);
        });
        if (!ly.attn) {
            q35k::GdnDecodeArgs ga{};
            ga.n_layers = 1;
            ga.KH = KH;
            ga.VH = VH;
            ga.KER = 4;
            ga.pos_dev = m->pos_dev;
            ga.eps = d.rms_norm_eps;
            ga.qkv = m->proj;
            ga.z = m->proj + CONV;
            ga.b = m->proj + CONV + VD;
            ga.a = m->proj + CONV + VD + VH;
            ga.conv_w = ly.conv_w;
            ga.A_log = ly.A_log;
            ga.dt_bias = ly.dt_bias;
            ga.norm_w = ly.gdn_norm;
            ga.conv_ring = m->conv_ring + static_cast<int64_t>(ly.idx) * 4 * CONV;
            ga.state = m->gdn_state + static_cast<int64_t>(ly.idx) * VH * 128 * 128;
            ga.out = m->mix;
            ga.conv_done = 1;
            L.run(Q35_KT_GDN_DECODE, [&] { return q35k::launch_gdn_decode(ga, false, s); });
            q35k::GemvArgs o{};
            o.W = ly.w_out;
            o.x = m->mix;
            o.norm_w = ly.gdn_norm;
            o.gate = m->proj + CONV;
            o.head_dim = 128;
            o.resid = m->hidden;
            o.y = m->hidden;
            o.rows = H;
            o.in_dim = VD;
            o.eps = d.rms_norm_eps;
            L.run(Q35_KT_GEMV, [&] { return q35k::launch_gemv(o, q35k::kProGatedNorm, s); });
        } else {
            q35k::AttnDecodeArgs aa{};
            aa.NQ = NQ;
            aa.NKV = NKV;
            aa.HD = HD;
            aa.ROT = rot_dims(d);
            aa.pos_dev = m->pos_dev;
            aa.max_ctx = m->max_ctx;
            aa.n_splits = m->n_splits;
            aa.theta = d.rope_theta;
            aa.eps = d.rms_norm_eps;
            aa.qg = m->proj;
            aa.k_new = m->proj + 2 * NQ * HD;
            aa.v_new = m->proj + 2 * NQ * HD + NKV * HD;
            aa.q_norm = ly.q_norm;
            aa.k_norm = ly.k_norm;
            aa.rope_cs = m->rope_cs;
            aa.k_cache = kv_ptr(m, ly.idx, 0, 0);
            aa.v_cache = kv_ptr(m, ly.idx, 1, 0);
            aa.kv_bf16 = m->kv_elem == 2;
            aa.part_o = m->part_o;
            aa.part_ml = m->part_ml;
            aa.out = m->mix;
            aa.n_layers = 1;
            L.run(Q35_KT_ATTN_DECODE, [&] { return q35k::launch_attn_partial(aa, s); });
            L.run(Q35_KT_ATTN_COMBINE, [&] { return q35k::launch_attn_combine(aa, s); });
            q35k::GemvArgs o{};
            o.W = ly.w_out;
            o.x = m->mix;
            o.resid = m->hidden;
            o.y = m->hidden;
            o.rows = H;
            o.in_dim = NQ * HD;
            L.run(Q35_KT_GEMV, [&] { return q35k::launch_gemv(o, q35k::kProPlain, s); });
        }
        q35k::GemvArgs f1{};
        f1.W = ly.w_gu;
        f1.x = m->hidden;
        f1.norm_w = ly.post_ln;
        f1.y = m->gu;
        f1.rows = 2 * I;
        f1.in_dim = H;
        f1.eps = d.rms_norm_eps;
        L.run(Q35_KT_GEMV, [&] { return q35k::launch_gemv(f1, q35k::kProRmsNorm, s, q35k::kEpiSwiGluPair); });
        q35k::GemvArgs f2{};
        f2.W = ly.w_down;
        f2.x = m->gu;  // silu(gate) * up, I floats
        f2.resid = m->hidden;
        f2.y = m->hidden;
        f2.rows = H;
        f2.in_dim = I;
        L.run(Q35_KT_GEMV, [&] { return q35k::launch_gemv(f2, q35k::kProPlain, s); });
        if (m->trace_on)
            L.run(Q35_KT_OTHER, [&] {
                return q35k::launch_copy_f32(m->trace + li * H, m->hidden, H, s);
            });
    }
    q35k::GemvArgs hd{};
    hd.W = m->head;
    hd.x = m->hidden;
    hd.norm_w = m->final_norm;
    hd.y = m->logits;
    hd.rows = d.vocab_size;
    hd.in_dim = H;
    hd.eps = d.rms_norm_eps;
    hd.amax_part = static_cast<float*>(m->argmax_part);  // the argmax's first pass, per workgroup
    L.run(Q35_KT_GEMV, [&] { return q35k::launch_gemv(hd, q35k::kProRmsNorm, s, q35k::kEpiStore); });
    L.run(Q35_KT_OTHER, [&] {
        return q35k::launch_argmax_parts(m->argmax_part, q35k::gemv_blocks(hd, q35k::kEpiStore), m->token_dev,
                                         m->ids_dev, m->pos_dev, s);
    });
    return L.st;
}

void drop_graph(q35_model* m) {
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    if (m->exec_run) (void)hipGraphExecDestroy(m->exec_run);
    if (m->graph_run) (void)hipGraphDestroy(m->graph_run);
    m->exec = m->exec_run = nullptr;
    m->graph = m->graph_run = nullptr;
    m->graph_valid = false;
}

// `steps` consecutive decode steps captured into one graph. Every step reads its token and
// position from token_dev / pos_dev and leaves the next ones there, so the same graph
// serves any position.
q35_status capture_steps(q35_model* m, int steps, hipGraph_t* graph, hipGraphExec_t* exec) {
    HIPCHK(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    q35_status st = Q35_OK;
    for (int i = 0; i < steps && st == Q35_OK; ++i) st = enqueue_step(m, m->stream, false);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (st != Q35_OK) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return q35::fail(Q35_ERR_HIP, "graph capture failed: %s", hipGetErrorString(e));
    *graph = g;
    HIPCHK(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
    return Q35_OK;
}

q35_status build_graph(q35_model* m) {
    drop_graph(m);
    q35_status st = capture_steps(m, 1, &m->graph, &m->exec);
    if (st == Q35_OK) st = capture_steps(m, kGraphRun, &m->graph_run, &m->exec_run);
    if (st != Q35_OK) {
        drop_graph(m);
        return st;
    }
    m->graph_valid = true;
    return Q35_OK;
}

// Enqueue `steps` (1 or kGraphRun) steps for the token already in token_dev.
q35_status launch_steps(q35_model* m, int steps) {
    if (m->timing_on || m->trace_on || !m->use_graph) {
        for (int i = 0; i < steps; ++i) {
            const q35_status st = enqueue_step(m, m->stream, m->timing_on);
            if (st != Q35_OK) return st;
        }
    } else {
        if (!m->graph_valid) {
            const q35_status st = build_graph(m);
            if (st != Q35_OK) return st;
        }
        HIPCHK(hipGraphLaunch(steps == kGraphRun ? m->exec_run : m->exec, m->stream));
    }
    m->pos += steps;
    return Q35_OK;
}

q35_status launch_one_step(q35_model* m) { return launch_steps(m, 1); }

q35_status collect_timing(q35_model* m) {
    if (!m->timing_on || m->ev_used == 0) return Q35_OK;
    HIPCHK(hipStreamSynchronize(m->stream));
    for (size_t i = 0; i + 1 < m->ev_used; i += 2) {
        float ms = 0.0f;
        HIPCHK(hipEventElapsedTime(&ms, m->ev[i], m->ev[i + 1]));
        const int c = m->ev_class[i / 2];
        m->kt_ms[c] += ms;
        m->kt_n[c] += 1;
    }
    m->ev_used = 0;
    return Q35_OK;
}

void destroy(q35_model* m) {
    if (!m) return;
    // teardown: errors are not actionable here, each release is attempted
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    drop_graph(m);
    for (hipEvent_t e : m->ev) (void)hipEventDestroy(e);
    if (m->pinned_token) (void)hipHostFree(m->pinned_token);
    if (m->w_arena) (void)hipFree(m->w_arena);
    if (m->state_arena) (void)hipFree(m->state_arena);
    if (m->kv_arena) (void)hipFree(m->kv_arena);
    if (m->scratch) (void)hipFree(m->scratch);
    if (m->pf_arena) (void)hipFree(m->pf_arena);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

// ------------------------------------------------------------------ context arenas
// Scratch arena layout for a given KV capacity (byte offsets, 256-B aligned): the decode
// step's activations, split-K partials, logits, argmax partials, device token / position,
// and the two context-sized tables (greedy id history, RoPE cos / sin per position).
struct ScratchPlan {
    size_t hidden, proj, mix, gu, part, logits, trace, am, ints, ids, rope, bytes;
};

ScratchPlan scratch_plan(const q35_dims& d, int64_t max_ctx) {
    const int H = d.hidden_size, I = d.ffn_intermediate;
    const int KD = d.gdn_k_heads * 128, VD = d.gdn_v_heads * 128, VH = d.gdn_v_heads, CONV = 2 * KD + VD;
    const int NQ = d.attn_q_heads, NKV = d.attn_kv_heads, HD = d.attn_head_dim;
    const int64_t proj_n = std::max<int64_t>(static_cast<int64_t>(CONV) + VD + 2 * VH, 2LL * NQ * HD + 2LL * NKV * HD);
    ScratchPlan p{};
    size_t sc = 0;
    auto take = [&](size_t bytes) {
        const size_t o = sc;
        sc = align256(sc + bytes);
        return o;
    };
    p.hidden = take(static_cast<size_t>(H) * 4);
    p.proj = take(static_cast<size_t>(proj_n) * 4);
    p.mix = take(static_cast<size_t>(std::max(VD, NQ * HD)) * 4);
    p.gu = take(static_cast<size_t>(2) * I * 4);
    p.part = take(static_cast<size_t>(q35k::attn_partial_floats(NQ, NKV, HD, kMaxSplits)) * 4);
    p.logits = take(static_cast<size_t>(d.vocab_size) * 4);
    p.trace = take(static_cast<size_t>(d.n_layers_total) * H * 4);
    p.am = take(static_cast<size_t>(2) * std::max(q35k::kArgmaxBlocks, q35k::kArgmaxParts) * 4);
    p.ints = take(16 * 4);
    p.ids = take(static_cast<size_t>(max_ctx) * 4);
    p.rope = take(static_cast<size_t>(max_ctx) * std::max(1, rot_dims(d)) * 4);
    p.bytes = sc;
    return p;
}

size_t kv_arena_bytes(const q35_model* m, int64_t max_ctx) {
    const q35_dims& d = m->d;
    return static_cast<size_t>(d.n_layers_attn) * 2 * d.attn_kv_heads * static_cast<size_t>(max_ctx) *
           d.attn_head_dim * m->kv_elem;
}

// The KV and scratch arenas for max_ctx positions, both or neither (a failed second
// allocation frees the first).
hipError_t alloc_context_pair(const q35_model* m, int64_t max_ctx, void** kv, void** sc) {
    *kv = *sc = nullptr;
    hipError_t e = dev_alloc(kv, std::max<size_t>(kv_arena_bytes(m, max_ctx), 256));
    if (e == hipSuccess) e = dev_alloc(sc, scratch_plan(m->d, max_ctx).bytes);
    if (e != hipSuccess) {
        if (*kv) (void)hipFree(*kv);
        *kv = *sc = nullptr;
        (void)hipGetLastError();  // the failed allocation is reported by the caller
    }
    return e;
}

void release_context(q35_model* m) {
    if (m->kv_arena) (void)hipFree(m->kv_arena);
    if (m->scratch) (void)hipFree(m->scratch);
    m->kv_arena = nullptr;
    m->scratch = nullptr;
    m->max_ctx = 0;
    m->kv_bytes = 0;
    m->scratch_bytes = 0;
    m->pos = 0;
}

// The KV cache and scratch arenas exist (a failed q35_model_reserve_context that could not
// make any context arenas again leaves a model without them).
q35_status need_context(const q35_model* m) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    if (!m->scratch || !m->kv_arena)
        return q35::fail(Q35_ERR_RANGE, "the model has no context arenas (a context reservation failed)");
    return Q35_OK;
}

q35_status install_context(q35_model* m, int64_t max_ctx, void* kv, void* sc);

// (Re)makes the KV and scratch arenas for max_ctx positions (one hipMalloc each), zeroed,
// with the RoPE table filled; the model is at position 0 afterwards. The new arenas are
// made while the old ones still exist and replace them only when both were made; when they
// do not fit beside the old ones, the old ones are freed and the new size tried again, then
// the old size. Should even that fail, the model keeps no context arenas (max_context 0)
// and every call that needs them refuses with Q35_ERR_RANGE instead of touching them.
q35_status alloc_context(q35_model* m, int64_t max_ctx) {
    const int64_t old_ctx = m->scratch ? m->max_ctx : 0;
    void *kv = nullptr, *sc = nullptr;
    hipError_t e = alloc_context_pair(m, max_ctx, &kv, &sc);
    if (e != hipSuccess && old_ctx > 0) {
        release_context(m);
        e = alloc_context_pair(m, max_ctx, &kv, &sc);
        if (e != hipSuccess) {
            const hipError_t e_old = alloc_context_pair(m, old_ctx, &kv, &sc);
            if (e_old == hipSuccess) {
                const q35_status st = install_context(m, old_ctx, kv, sc);
                if (st != Q35_OK) return st;
                return q35::fail(Q35_ERR_HIP, "context arenas for %lld positions: %s (the %lld-position arenas were made again)",
                                 static_cast<long long>(max_ctx), hipGetErrorString(e), static_cast<long long>(old_ctx));
            }
        }
    }
    if (e != hipSuccess)
        return q35::fail(Q35_ERR_HIP, "context arenas for %lld positions: %s", static_cast<long long>(max_ctx),
                         hipGetErrorString(e));
    release_context(m);
    return install_context(m, max_ctx, kv, sc);
}

// Takes over kv / sc (made by alloc_context_pair for max_ctx) as the model's context arenas.
q35_status install_context(q35_model* m, int64_t max_ctx, void* kv, void* sc) {
    const q35_dims& d = m->d;
    m->kv_arena = static_cast<float*>(kv);
    m->scratch = static_cast<uint8_t*>(sc);
    m->max_ctx = max_ctx;
    m->kv_bytes = kv_arena_bytes(m, max_ctx);
    m->n_splits = q35k::attn_default_splits(max_ctx, d.attn_kv_heads, m->n_cu);
    const ScratchPlan sp = scratch_plan(d, max_ctx);
    m->scratch_bytes = sp.bytes;
    auto S32 = [&](size_t off) { return reinterpret_cast<float*>(m->scratch + off); };
    const int NQ = d.attn_q_heads, NKV = d.attn_kv_heads, HD = d.attn_head_dim;
    m->hidden = S32(sp.hidden);
    m->proj = S32(sp.proj);
    m->mix = S32(sp.mix);
    m->gu = S32(sp.gu);
    m->part_o = S32(sp.part);
    m->part_ml = m->part_o + static_cast<int64_t>(NKV) * kMaxSplits * (NQ / NKV) * HD;
    m->logits = S32(sp.logits);
    m->trace = S32(sp.trace);
    m->argmax_part = m->scratch + sp.am;
    int* ints = reinterpret_cast<int*>(m->scratch + sp.ints);
    m->token_dev = ints;
    m->pos_dev = ints + 1;
    m->ids_dev = reinterpret_cast<int*>(m->scratch + sp.ids);
    m->rope_cs = S32(sp.rope);
    HIPCHK(q35k::launch_fill_f32(m->kv_arena, static_cast<int64_t>(m->kv_bytes / 4), 0.0f, m->stream));
    HIPCHK(q35k::launch_fill_f32(reinterpret_cast<float*>(m->scratch), static_cast<int64_t>(m->scratch_bytes / 4), 0.0f,
                                 m->stream));
    HIPCHK(q35k::launch_rope_table(m->rope_cs, max_ctx, rot_dims(d), d.rope_theta, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    m->pos = 0;
    m->budget.kv_cache_bytes = m->kv_bytes;
    m->budget.activation_bytes = m->scratch_bytes;
    return Q35_OK;
}

// Layout of the prompt arena for blocks of `tb` tokens (offsets in floats, 256-B aligned).
// The logits rows are wide enough for either output head (vocab_size or the embedding's rows).
struct PrefillPlan {
    int tb = 0, lr = 0;  // tokens per block, logits rows per output-head pass
    int tiled = 0;       // xn, mix, hb in the tiled layout of the two-part GEMM (H, I % 32 == 0)
    int64_t hidden = 0, xn = 0, proj = 0, mix = 0, hb = 0, ws = 0, logits = 0, ids = 0, total = 0;
    int64_t ws_n = 0;  // floats at ws
    // row maxima of the GEMM inputs (xn, mix, hb), the weight maxima, the fp16 weights
    int64_t xn_max = 0, mix_max = 0, hb_max = 0, wmax = 0, wh = 0;
};

// Elements of the four projection matrices of layer l (w_in, w_out, w_gu, w_down).
void layer_matrix_sizes(const q35_dims& d, int l, int64_t (&n)[4]) {
    const int64_t H = d.hidden_size, I = d.ffn_intermediate;
    const int64_t KD = d.gdn_k_heads * 128LL, VD = d.gdn_v_heads * 128LL, VH = d.gdn_v_heads;
    const int64_t NQ = d.attn_q_heads, NKV = d.attn_kv_heads, HD = d.attn_head_dim;
    const bool attn = (l + 1) % d.attn_interval == 0;
    n[0] = (attn ? 2 * NQ * HD + 2 * NKV * HD : 2 * KD + VD + VD + 2 * VH) * H;
    n[1] = H * (attn ? NQ * HD : VD);
    n[2] = 2 * I * H;
    n[3] = H * I;
}

int64_t proj_width(const q35_dims& d) {
    const int64_t KD = d.gdn_k_heads * 128LL, VD = d.gdn_v_heads * 128LL;
    return std::max<int64_t>(2 * KD + VD + VD + 2LL * d.gdn_v_heads,
                             2LL * d.attn_q_heads * d.attn_head_dim + 2LL * d.attn_kv_heads * d.attn_head_dim);
}

PrefillPlan plan_prefill(const q35_dims& d, int tb, int64_t logits_width, bool exact) {
    PrefillPlan p;
    p.tb = tb;
    p.lr = std::min(tb, 256);
    p.tiled = !exact && d.hidden_size % 32 == 0 && d.ffn_intermediate % 32 == 0;
    const int64_t H = d.hidden_size, I = d.ffn_intermediate, T = tb;
    const int64_t VD = d.gdn_v_heads * 128LL, QD = static_cast<int64_t>(d.attn_q_heads) * d.attn_head_dim;
    int64_t cur = 0;
    auto take = [&](int64_t n) {
        const int64_t o = cur;
        cur += (n + 63) / 64 * 64;
        return o;
    };
    // xn, mix and hb feed the two-part GEMM in its tiled layout: rows padded to 128
    const int64_t TP = q35k::rows_tiled(T);
    p.hidden = take(T * H);
    p.xn = take(TP * H);
    p.proj = take(T * proj_width(d));
    p.mix = take(TP * std::max(VD, QD));
    p.hb = take(TP * I);
    p.ws_n = std::max(q35k::gdn_prefill_workspace_floats(d.gdn_k_heads, d.gdn_v_heads, tb),
                      q35k::attn_prefill_workspace_floats(d.attn_q_heads, tb));
    p.ws = take(p.ws_n);
    p.logits = take(static_cast<int64_t>(p.lr) * logits_width);
    p.ids = take(T);
    p.xn_max = take(T);
    p.mix_max = take(T * std::max(d.attn_q_heads, d.gdn_v_heads));
    p.hb_max = take(T * q35k::gemm_col_tiles(2 * d.ffn_intermediate));
    p.wmax = take(4LL * d.n_layers_total);
    if (p.tiled) {  // the fp16 weight copies of the two-part path
        int64_t wh = 0;
        for (int l = 0; l < d.n_layers_total; ++l) {
            int64_t n[4];
            layer_matrix_sizes(d, l, n);
            for (const int64_t x : n) wh += (x + 127) / 128 * 128;  // 256-B aligned fp16 matrices
        }
        p.wh = take(wh / 2);
    }
    p.total = cur;
    return p;
}

int64_t logits_width(const q35_model* m) { return std::max<int64_t>(m->d.vocab_size, m->embed_rows); }

size_t prompt_arena_bytes(const q35_model* m, int64_t tb) {
    return static_cast<size_t>(plan_prefill(m->d, static_cast<int>(tb), logits_width(m), m->pf_exact).total) * 4;
}

// The prefill's fp16 weight copies, in the prompt arena: per matrix its maximum |w| (one
// readback for all), then wh = fp16(w x 2^e) with e = 15 - (exponent of the maximum as in
// frexp), so the largest weight lies in [2^14, 2^15).
q35_status make_prefill_weights(q35_model* m, const PrefillPlan& p) {
    const int L = m->d.n_layers_total;
    unsigned* wmax = reinterpret_cast<unsigned*>(reinterpret_cast<float*>(m->pf_arena) + p.wmax);
    uint16_t* wh = reinterpret_cast<uint16_t*>(reinterpret_cast<float*>(m->pf_arena) + p.wh);
    HIPCHK(hipMemsetAsync(wmax, 0, sizeof(unsigned) * 4 * L, m->stream));
    for (int l = 0; l < L; ++l) {
        LayerDev& ly = m->layers[static_cast<size_t>(l)];
        layer_matrix_sizes(m->d, l, ly.wn);
        const uint16_t* src[4] = {ly.w_in, ly.w_out, ly.w_gu, ly.w_down};
        for (int i = 0; i < 4; ++i) {
            HIPCHK(q35k::launch_bf16_absmax(src[i], ly.wn[i], wmax + 4 * l + i, m->stream));
            ly.wh[i] = wh;
            wh += (ly.wn[i] + 127) / 128 * 128;
        }
    }
    std::vector<unsigned> mx(static_cast<size_t>(4) * L);
    HIPCHK(hipMemcpyAsync(mx.data(), wmax, mx.size() * sizeof(unsigned), hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    for (int l = 0; l < L; ++l) {
        LayerDev& ly = m->layers[static_cast<size_t>(l)];
        const uint16_t* src[4] = {ly.w_in, ly.w_out, ly.w_gu, ly.w_down};
        for (int i = 0; i < 4; ++i) {
            const uint32_t bits = mx[static_cast<size_t>(4 * l + i)] << 16;  // |bf16| -> fp32
            float w = 0.0f;
            std::memcpy(&w, &bits, 4);
            int ex = 0;
            (void)std::frexp(w, &ex);
            ly.we[i] = w > 0.0f && std::isfinite(w) ? std::min(std::max(15 - ex, -100), 100) : 0;
            HIPCHK(q35k::launch_bf16_to_f16(src[i], ly.wh[i], ly.wn[i], ly.we[i], m->stream));
        }
    }
    return Q35_OK;
}

q35_status make_prompt_arena(q35_model* m, int64_t tb) {
    if (m->pf_arena) {
        HIPCHK(hipStreamSynchronize(m->stream));
        HIPCHK(hipFree(m->pf_arena));
        m->pf_arena = nullptr;
        m->pf_bytes = 0;
    }
    void* p = nullptr;
    const size_t bytes = prompt_arena_bytes(m, tb);
    HIPCHK(dev_alloc(&p, bytes));
    m->pf_arena = static_cast<uint8_t*>(p);
    m->pf_bytes = bytes;
    m->budget.prompt_arena_bytes = bytes;
    const PrefillPlan plan = plan_prefill(m->d, static_cast<int>(tb), logits_width(m), m->pf_exact);
    return plan.tiled ? make_prefill_weights(m, plan) : Q35_OK;
}

int prefill_block_tokens(const q35_model* m) {
    const int64_t want = m->pf_block > 0 ? m->pf_block : m->pf_planned > 0 ? m->pf_planned : 4096;
    return static_cast<int>(std::min<int64_t>(want, m->max_ctx));
}

// The prompt arena for the current block size: the one planned at creation, or the one the
// last prefill made when it is large enough, else a new one (lazy mode only).
q35_status ensure_prefill_arena(q35_model* m, PrefillPlan* plan) {
    const int tb = prefill_block_tokens(m);
    *plan = plan_prefill(m->d, tb, logits_width(m), m->pf_exact);
    if (m->pf_arena && static_cast<size_t>(plan->total) * 4 <= m->pf_bytes) return Q35_OK;
    if (m->pf_planned > 0)
        return q35::fail(Q35_ERR_RANGE, "a prefill block of %d tokens exceeds the prompt arena planned for %d", tb,
                         m->pf_planned);
    const q35_status st = make_prompt_arena(m, tb);
    if (st == Q35_OK)
        std::cerr << "[q35] prompt arena: " << (m->pf_bytes >> 20) << " MiB for blocks of " << tb << " tokens\n";
    return st;
}

q35_status create_model(const q35_dims* dims, const q35_tensor* ts, int nt, int64_t max_ctx, int kv_elem,
                        int prefill_block, int prefill_exact, q35_model** out) {
    if (!dims || !ts || !out || nt <= 0) return q35::fail(Q35_ERR_ARG, "q35_model_create: null argument");
    *out = nullptr;
    if (max_ctx < 0 || max_ctx > (int64_t{1} << 30))
        return q35::fail(Q35_ERR_RANGE, "max_context %lld out of range", static_cast<long long>(max_ctx));
    if (prefill_block < 0 || prefill_block > (1 << 20))
        return q35::fail(Q35_ERR_RANGE, "prefill block %d out of range", prefill_block);
    if (kv_elem != 4 && kv_elem != 2)
        return q35::fail(Q35_ERR_UNSUPPORTED, "KV cache element of %d bytes (4 = fp32 or 2 = bf16)", kv_elem);
    if (prefill_exact != 0 && prefill_exact != 1)
        return q35::fail(Q35_ERR_ARG, "prefill_exact %d (0 or 1)", prefill_exact);
    q35_dims d = *dims;
    d.n_layers_attn = d.n_layers_total / d.attn_interval;
    d.n_layers_gdn = d.n_layers_total - d.n_layers_attn;
    q35_status st = check_dims(d);
    if (st != Q35_OK) return st;

    const int H = d.hidden_size, I = d.ffn_intermediate;
    const int KH = d.gdn_k_heads, VH = d.gdn_v_heads, KD = KH * 128, VD = VH * 128;
    const int CONV = 2 * KD + VD;
    const int NQ = d.attn_q_heads, NKV = d.attn_kv_heads, HD = d.attn_head_dim;
    const std::string lm = "model.language_model.";

    // weight arena plan
    ArenaPlanner plan(ts, nt);
    struct LayerOff {
        size_t w_in, w_out, w_gu, w_down, input_ln, post_ln, conv_w, A_log, dt_bias, gdn_norm, q_norm, k_norm;
        int64_t in_rows;
    };
    std::vector<LayerOff> lo(static_cast<size_t>(d.n_layers_total));
    auto bad = [](size_t o) { return o == SIZE_MAX; };
    for (int l = 0; l < d.n_layers_total; ++l) {
        const std::string p = lm + "layers." + std::to_string(l) + ".";
        LayerOff& o = lo[static_cast<size_t>(l)];
        o = LayerOff{};
        o.input_ln = plan.vec(p + "input_layernorm.weight", H, &st);
        if (bad(o.input_ln)) return st;
        o.post_ln = plan.vec(p + "post_attention_layernorm.weight", H, &st);
        if (bad(o.post_ln)) return st;
        int64_t r = 0;
        o.w_gu = plan.mat_interleaved(p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", H, &r, &st);
        if (bad(o.w_gu)) return st;
        if (r != 2 * I) return q35::fail(Q35_ERR_FORMAT, "layer %d: gate/up rows %lld != 2*%d", l, (long long)r, I);
        o.w_down = plan.mat({p + "mlp.down_proj.weight"}, I, &r, &st);
        if (bad(o.w_down)) return st;
        if (r != H) return q35::fail(Q35_ERR_FORMAT, "layer %d: down_proj rows %lld != %d", l, (long long)r, H);
        if ((l + 1) % d.attn_interval == 0) {
            const std::string a = p + "self_attn.";
            o.w_in = plan.mat({a + "q_proj.weight", a + "k_proj.weight", a + "v_proj.weight"}, H, &o.in_rows, &st);
            if (bad(o.w_in)) return st;
            if (o.in_rows != 2LL * NQ * HD + 2LL * NKV * HD)
                return q35::fail(Q35_ERR_FORMAT, "layer %d: q/k/v rows %lld", l, (long long)o.in_rows);
            o.w_out = plan.mat({a + "o_proj.weight"}, static_cast<int64_t>(NQ) * HD, &r, &st);
            if (bad(o.w_out)) return st;
            if (r != H) return q35::fail(Q35_ERR_FORMAT, "layer %d: o_proj rows %lld", l, (long long)r);
            o.q_norm = plan.vec(a + "q_norm.weight", HD, &st);
            if (bad(o.q_norm)) return st;
            o.k_norm = plan.vec(a + "k_norm.weight", HD, &st);
            if (bad(o.k_norm)) return st;
        } else {
            const std::string g = p + "linear_attn.";
            o.w_in = plan.mat({g + "in_proj_qkv.weight", g + "in_proj_z.weight", g + "in_proj_b.weight",
                               g + "in_proj_a.weight"},
                              H, &o.in_rows, &st);
            if (bad(o.w_in)) return st;
            if (o.in_rows != static_cast<int64_t>(CONV) + VD + 2 * VH)
                return q35::fail(Q35_ERR_FORMAT, "layer %d: GDN in-projection rows %lld", l, (long long)o.in_rows);
            o.w_out = plan.mat({g + "out_proj.weight"}, VD, &r, &st);
            if (bad(o.w_out)) return st;
            if (r != H) return q35::fail(Q35_ERR_FORMAT, "layer %d: out_proj rows %lld", l, (long long)r);
            o.conv_w = plan.vec(g + "conv1d.weight", static_cast<int64_t>(CONV) * 4, &st);
            if (bad(o.conv_w)) return st;
            o.dt_bias = plan.vec(g + "dt_bias", VH, &st);
            if (bad(o.dt_bias)) return st;
            o.A_log = plan.vec(g + "A_log", VH, &st);
            if (bad(o.A_log)) return st;
            o.gdn_norm = plan.vec(g + "norm.weight", 128, &st);
            if (bad(o.gdn_norm)) return st;
        }
    }
    const q35_tensor* emb_t = plan.find(lm + "embed_tokens.weight");
    if (!emb_t) return q35::fail(Q35_ERR_MISSING, "missing weight: %sembed_tokens.weight", lm.c_str());
    int64_t emb_rows = 0;
    const size_t emb_off = plan.mat({lm + "embed_tokens.weight"}, H, &emb_rows, &st);
    if (bad(emb_off)) return st;
    size_t head_off = emb_off;
    int64_t head_rows = emb_rows;
    for (const std::string& hn : {std::string("lm_head.weight"), lm + "lm_head.weight"}) {
        if (plan.find(hn)) {
            head_off = plan.mat({hn}, H, &head_rows, &st);
            if (bad(head_off)) return st;
            break;
        }
    }
    if (head_rows < d.vocab_size || emb_rows < d.vocab_size)
        return q35::fail(Q35_ERR_FORMAT, "embedding / output head rows %lld / %lld < vocab %d", (long long)emb_rows,
                         (long long)head_rows, d.vocab_size);
    const size_t fnorm_off = plan.vec(lm + "norm.weight", H, &st);
    if (bad(fnorm_off)) return st;

    std::unique_ptr<q35_model, void (*)(q35_model*)> m(new (std::nothrow) q35_model(), destroy);
    if (!m) return q35::fail(Q35_ERR_ARG, "out of host memory");
    m->d = d;
    m->max_ctx = max_ctx;
    HIPCHK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
    HIPCHK(q35k::gemv_enable_wide_inputs());  // before any launch is captured into a graph

    // state arena: GDN states and conv rings (fixed size)
    const size_t gdn_bytes = static_cast<size_t>(d.n_layers_gdn) * VH * 128 * 128 * 4;
    const size_t ring_bytes = static_cast<size_t>(d.n_layers_gdn) * 4 * CONV * 4;
    m->state_bytes = align256(gdn_bytes) + align256(ring_bytes);
    m->kv_elem = kv_elem;
    m->n_cu = q35k::device_cu_count();
    m->w_bytes = plan.bytes();
    m->embed_rows = emb_rows;
    m->pf_planned = prefill_block;
    m->pf_exact = prefill_exact;
    const size_t pf_bytes = prefill_block > 0 ? prompt_arena_bytes(m.get(), max_ctx > 0 ? std::min<int64_t>(prefill_block, max_ctx) : prefill_block) : 0;

    if (max_ctx == 0) {
        // KV capacity from the memory equation (src/memory_budget.cpp:56-81) against the
        // device's memory: weights, recurrent state, the context-independent scratch, the
        // planned prompt arena and a margin are fixed; the rest is KV, up to the model's
        // native context
        size_t free_b = 0, total_b = 0;
        HIPCHK(hipMemGetInfo(&free_b, &total_b));
        const size_t fixed = m->w_bytes + m->state_bytes + scratch_plan(d, 0).bytes + pf_bytes;
        int64_t ctx = q35_solve_max_context(&d, total_b, m->w_bytes, m->state_bytes,
                                            scratch_plan(d, 0).bytes + pf_bytes, 0, kSolveMarginBytes, kv_elem);
        if (ctx <= 0)
            return q35::fail(Q35_ERR_RANGE, "no KV capacity fits %zu bytes of device memory next to %zu of weights",
                             total_b, m->w_bytes);
        // the scratch also grows with the context (greedy ids, RoPE table): the equation's
        // per-token KV cost plus those bytes per position must fit as well
        const size_t per_pos = static_cast<size_t>(d.n_layers_attn) * 2 * NKV * HD * kv_elem +
                               (scratch_plan(d, 1).bytes - scratch_plan(d, 0).bytes);
        ctx = std::min<int64_t>(ctx, static_cast<int64_t>((total_b - fixed - kSolveMarginBytes) / per_pos));
        max_ctx = std::min<int64_t>(ctx, int64_t{1} << 30);
        std::cerr << "[q35] max_context " << max_ctx << " planned by the memory equation against "
                  << (total_b >> 20) << " MiB of device memory\n";
    }

    void* p = nullptr;
    HIPCHK(dev_alloc(&p, m->w_bytes));
    m->w_arena = static_cast<uint8_t*>(p);
    HIPCHK(dev_alloc(&p, m->state_bytes));
    m->state_arena = static_cast<float*>(p);
    HIPCHK(hipHostMalloc(reinterpret_cast<void**>(&m->pinned_token), 64, hipHostMallocDefault));

    // upload
    std::vector<float> tmp;
    for (const Piece& pc : plan.pieces()) {
        const int64_t n = numel_of(pc.src);
        if (pc.partner) {
            const int64_t rows = n / pc.cols;
            const auto* ra = static_cast<const uint16_t*>(pc.src->data);
            const auto* rb = static_cast<const uint16_t*>(pc.partner->data);
            std::vector<uint16_t> il(static_cast<size_t>(2 * n));
            for (int64_t r = 0; r < rows; ++r) {
                std::memcpy(il.data() + (2 * r) * pc.cols, ra + r * pc.cols, static_cast<size_t>(pc.cols) * 2);
                std::memcpy(il.data() + (2 * r + 1) * pc.cols, rb + r * pc.cols, static_cast<size_t>(pc.cols) * 2);
            }
            HIPCHK(hipMemcpy(m->w_arena + pc.off, il.data(), il.size() * 2, hipMemcpyHostToDevice));
        } else if (!pc.to_f32) {
            HIPCHK(hipMemcpy(m->w_arena + pc.off, pc.src->data, static_cast<size_t>(n) * 2, hipMemcpyHostToDevice));
        } else {
            tmp.resize(static_cast<size_t>(n));
            if (pc.src->dtype == 1) {
                std::memcpy(tmp.data(), pc.src->data, static_cast<size_t>(n) * 4);
            } else {
                const auto* b = static_cast<const uint16_t*>(pc.src->data);
                for (int64_t i = 0; i < n; ++i) tmp[static_cast<size_t>(i)] = bf16_to_f32(b[i]);
            }
            HIPCHK(hipMemcpy(m->w_arena + pc.off, tmp.data(), static_cast<size_t>(n) * 4, hipMemcpyHostToDevice));
        }
    }

    auto W16 = [&](size_t off) { return reinterpret_cast<const uint16_t*>(m->w_arena + off); };
    auto W32 = [&](size_t off) { return reinterpret_cast<const float*>(m->w_arena + off); };
    int ai = 0, gi = 0;
    m->layers.resize(static_cast<size_t>(d.n_layers_total));
    for (int l = 0; l < d.n_layers_total; ++l) {
        const LayerOff& o = lo[static_cast<size_t>(l)];
        LayerDev& ly = m->layers[static_cast<size_t>(l)];
        ly.attn = (l + 1) % d.attn_interval == 0;
        ly.idx = ly.attn ? ai++ : gi++;
        ly.w_in = W16(o.w_in);
        ly.w_out = W16(o.w_out);
        ly.w_gu = W16(o.w_gu);
        ly.w_down = W16(o.w_down);
        ly.input_ln = W32(o.input_ln);
        ly.post_ln = W32(o.post_ln);
        ly.in_rows = static_cast<int>(o.in_rows);
        if (ly.attn) {
            ly.q_norm = W32(o.q_norm);
            ly.k_norm = W32(o.k_norm);
        } else {
            ly.conv_w = W32(o.conv_w);
            ly.A_log = W32(o.A_log);
            ly.dt_bias = W32(o.dt_bias);
            ly.gdn_norm = W32(o.gdn_norm);
        }
    }
    m->embed = W16(emb_off);
    m->head = W16(head_off);
    m->final_norm = W32(fnorm_off);
    m->gdn_state = m->state_arena;
    m->conv_ring = m->state_arena + align256(gdn_bytes) / 4;
    HIPCHK(q35k::launch_fill_f32(m->state_arena, static_cast<int64_t>(m->state_bytes / 4), 0.0f, m->stream));

    m->budget.weight_bytes = m->w_bytes;
    m->budget.gdn_state_bytes = gdn_bytes;
    m->budget.gdn_conv_bytes = ring_bytes;
    m->budget.vision_scratch_bytes = 0;
    st = alloc_context(m.get(), max_ctx);
    if (st != Q35_OK) return st;
    if (prefill_block > 0) {
        // the block size the arena is made for: a block beyond max_context is never run, and
        // a later q35_model_reserve_context keeps blocks within this arena
        m->pf_planned = static_cast<int>(std::min<int64_t>(prefill_block, max_ctx));
        st = make_prompt_arena(m.get(), m->pf_planned);
        if (st != Q35_OK) return st;
    }
    std::cerr << "[q35] device arenas (max_context=" << max_ctx << "): weights " << (m->w_bytes >> 20)
              << " MiB, state " << (m->state_bytes >> 10) << " KiB, kv " << (m->kv_bytes >> 20)
              << " MiB, scratch " << (m->scratch_bytes >> 10) << " KiB";
    if (m->pf_arena) std::cerr << ", prompt " << (m->pf_bytes >> 20) << " MiB";
    std::cerr << "\n";
    *out = m.release();
    return Q35_OK;
}

hipError_t gemm(const float* X, int64_t ldx, const uint16_t* W, int M, int N, int K, const float* R, float* Y,
                int64_t ldy, hipStream_t s, bool swiglu = false) {
    q35k::GemmArgs g{X, W, R, Y, M, N, K, ldx, R ? ldy : 0, ldy};
    g.swiglu = swiglu;
    return q35k::launch_gemm(g, s);
}

// The same on the two-part fp16 path: weight matrix i of layer ly, the row maxima of X
// (xmax_n partial maxima per row), and for the SwiGLU GEMM the row maxima of its output.
// tiled: 0 row-major X (three exact bf16 parts), 1 tiled fp32 X, 2 X split by its producer.
hipError_t gemm_h(const float* X, int64_t ldx, const LayerDev& ly, int i, const float* xmax, int xmax_n, int M, int N,
                  int K, const float* R, float* Y, int64_t ldy, hipStream_t s, int tiled, float* ymax = nullptr) {
    const uint16_t* W[4] = {ly.w_in, ly.w_out, ly.w_gu, ly.w_down};
    q35k::GemmArgs g{X, W[i], R, Y, M, N, K, ldx, R ? ldy : 0, ldy};
    g.swiglu = ymax != nullptr;
    g.Wh = tiled ? ly.wh[i] : nullptr;  // row-major X: the three exact bf16 parts
    g.w_exp = ly.we[i];
    g.xmax = xmax;
    g.xmax_n = xmax_n;
    g.ymax = ymax;
    g.x_tiled = tiled != 0;
    g.x_planes = tiled == 2;
    g.y_tiled = tiled && ymax != nullptr;
    return q35k::launch_gemm(g, s);
}

// One block of T tokens at positions pos0 .. pos0 + T - 1 (ids already in the arena).
// Row r of the block is prompt row base + r of logits_host / trace_host.
q35_status prefill_block(q35_model* m, const PrefillPlan& p, int pos0, int T, int64_t base, float* logits_host,
                         float* trace_host) {
    const q35_dims& d = m->d;
    const hipStream_t s = m->stream;
    const int H = d.hidden_size, I = d.ffn_intermediate, L = d.n_layers_total;
    const int KH = d.gdn_k_heads, VH = d.gdn_v_heads, KD = KH * 128, VD = VH * 128, CONV = 2 * KD + VD;
    const int NQ = d.attn_q_heads, NKV = d.attn_kv_heads, HD = d.attn_head_dim;
    const float eps = d.rms_norm_eps;
    float* F = reinterpret_cast<float*>(m->pf_arena);
    float *hidden = F + p.hidden, *xn = F + p.xn, *proj = F + p.proj, *mix = F + p.mix;
    float *hb = F + p.hb, *ws = F + p.ws, *lg = F + p.logits;
    float *xn_max = F + p.xn_max, *mix_max = F + p.mix_max, *hb_max = F + p.hb_max;
    const int* ids = reinterpret_cast<const int*>(F + p.ids);
    // the input norms' rows feed only the in-projection and gate/up GEMMs: on the tiled
    // path they are written split for them (row widths the one-row-per-wave norm handles)
    const int xn_form = p.tiled ? (q35k::rmsnorm_rows_splits(H) ? 2 : 1) : 0;
    Launcher Lr{m, s, m->timing_on};

    Lr.run(Q35_KT_OTHER, [&] { return q35k::launch_embed_rows(m->embed, ids, hidden, T, H, s); });
    for (int li = 0; li < L; ++li) {
        const LayerDev& ly = m->layers[static_cast<size_t>(li)];
        Lr.run(Q35_KT_OTHER, [&] {
            return q35k::launch_rmsnorm_rows(hidden, ly.input_ln, xn, T, H, eps, 0, nullptr, s, xn_max, xn_form);
        });
        Lr.run(Q35_KT_GEMM, [&] { return gemm_h(xn, H, ly, 0, xn_max, 1, T, ly.in_rows, H, nullptr, proj, ly.in_rows, s, xn_form); });
        if (!ly.attn) {
            q35k::GdnPrefillArgs g{};
            g.T = T;
            g.KH = KH;
            g.VH = VH;
            g.pos0 = pos0;
            g.eps = eps;
            g.qkv = proj;
            g.ld_qkv = ly.in_rows;
            g.z = proj + CONV;
            g.ld_z = ly.in_rows;
            g.b = proj + CONV + VD;
            g.a = proj + CONV + VD + VH;
            g.ld_ba = ly.in_rows;
            g.conv_w = ly.conv_w;
            g.A_log = ly.A_log;
            g.dt_bias = ly.dt_bias;
            g.norm_w = ly.gdn_norm;
            g.conv_ring = m->conv_ring + static_cast<int64_t>(ly.idx) * 4 * CONV;
            g.state = m->gdn_state + static_cast<int64_t>(ly.idx) * VH * 128 * 128;
            g.out = mix;
            g.omax = mix_max;
            g.out_tiled = p.tiled;
            q35k::gdn_prefill_carve(g, ws);
            Lr.run(Q35_KT_GDN_PREFILL, [&] { return q35k::launch_gdn_prefill(g, s); });
            Lr.run(Q35_KT_GEMM, [&] { return gemm_h(mix, VD, ly, 1, mix_max, VH, T, H, VD, hidden, hidden, H, s, p.tiled); });
        } else {
            q35k::AttnPrefillArgs a{};
            a.T = T;
            a.NQ = NQ;
            a.NKV = NKV;
            a.ROT = rot_dims(d);
            a.pos0 = pos0;
            a.max_ctx = m->max_ctx;
            a.theta = d.rope_theta;
            a.eps = eps;
            a.qkv = proj;
            a.ld_qkv = ly.in_rows;
            a.q_norm = ly.q_norm;
            a.k_norm = ly.k_norm;
            a.k_cache = kv_ptr(m, ly.idx, 0, 0);
            a.v_cache = kv_ptr(m, ly.idx, 1, 0);
            a.kv_bf16 = m->kv_elem == 2;
            a.rope_cs = m->rope_cs;
            a.Qa = ws;
            // the pre-split key / value tiles where they fit in the rest of the workspace
            // (the GDN layers' share is the larger one at 2B shapes: up to ~35k keys)
            const int64_t qa_n = q35k::attn_prefill_workspace_floats(NQ, T);
            if (!a.kv_bf16 && qa_n + q35k::attn_prefill_image_floats(NKV, pos0, T) <= p.ws_n) a.kv_img = ws + qa_n;
            a.out = mix;
            a.omax = mix_max;
            a.out_tiled = p.tiled;
            Lr.run(Q35_KT_ATTN_PREFILL, [&] { return q35k::launch_attn_prefill(a, s); });
            Lr.run(Q35_KT_GEMM, [&] {
                return gemm_h(mix, NQ * HD, ly, 1, mix_max, NQ, T, H, NQ * HD, hidden, hidden, H, s, p.tiled);
            });
        }
        Lr.run(Q35_KT_OTHER, [&] {
            return q35k::launch_rmsnorm_rows(hidden, ly.post_ln, xn, T, H, eps, 0, nullptr, s, xn_max, xn_form);
        });
        // gate/up projection with silu(gate) * up in its epilogue: hb = T x I, with the row
        // maxima of hb per column tile for the down projection
        Lr.run(Q35_KT_GEMM, [&] { return gemm_h(xn, H, ly, 2, xn_max, 1, T, 2 * I, H, nullptr, hb, I, s, xn_form, hb_max); });
        Lr.run(Q35_KT_GEMM, [&] {
            return gemm_h(hb, I, ly, 3, hb_max, q35k::gemm_col_tiles(2 * I), T, H, I, hidden, hidden, H, s, p.tiled);
        });
        if (trace_host)
            Lr.run(Q35_KT_OTHER, [&] {
                return hipMemcpy2DAsync(trace_host + (base * L + li) * H, static_cast<size_t>(L) * H * 4, hidden,
                                        static_cast<size_t>(H) * 4, static_cast<size_t>(H) * 4,
                                        static_cast<size_t>(T), hipMemcpyDeviceToHost, s);
            });
    }
    if (logits_host) {
        // the step's output head over vocab_size rows, or (QwenForward::prefill's rule,
        // src/qwen_forward.cpp:193-199) the embedding over all its rows
        const int V = m->prefill_head ? static_cast<int>(m->embed_rows) : d.vocab_size;
        const uint16_t* head = m->prefill_head ? m->embed : m->head;
        for (int r0 = 0; r0 < T; r0 += p.lr) {
            const int rows = std::min(p.lr, T - r0);
            Lr.run(Q35_KT_OTHER, [&] {
                return q35k::launch_rmsnorm_rows(hidden + static_cast<int64_t>(r0) * H, m->final_norm, xn, rows, H,
                                                 eps, 0, nullptr, s);
            });
            Lr.run(Q35_KT_GEMM, [&] { return gemm(xn, H, head, rows, V, H, nullptr, lg, V, s); });
            Lr.run(Q35_KT_OTHER, [&] {
                return hipMemcpyAsync(logits_host + (base + r0) * V, lg, static_cast<size_t>(rows) * V * 4,
                                      hipMemcpyDeviceToHost, s);
            });
        }
    }
    // the block's last row becomes the decode residual (what the last step would leave)
    Lr.run(Q35_KT_OTHER, [&] { return q35k::launch_copy_f32(m->hidden, hidden + static_cast<int64_t>(T - 1) * H, H, s); });
    return Lr.st;
}

// Feeds ids[0 .. n) at positions pos .. pos + n - 1 through the chunked prefill and leaves the
// model as n decode steps would: state, conv ring, KV rows, position, the residual and
// logits of the last token, its argmax in token_dev and ids_dev[pos + n - 1].
q35_status extend(q35_model* m, const int32_t* ids, int32_t n, float* logits_host, float* trace_host) {
    if (!m || !ids || n <= 0) return q35::fail(Q35_ERR_ARG, "bad argument");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    if (m->pos + n > m->max_ctx)
        return q35::fail(Q35_ERR_RANGE, "position %lld + %d tokens exceeds max_context %lld", (long long)m->pos, n,
                         (long long)m->max_ctx);
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= m->d.vocab_size || ids[i] >= m->embed_rows)
            return q35::fail(Q35_ERR_RANGE, "token %d at %d outside [0, %d)", ids[i], i, m->d.vocab_size);
    PrefillPlan p;
    const q35_status pa = ensure_prefill_arena(m, &p);
    if (pa != Q35_OK) return pa;
    float* F = reinterpret_cast<float*>(m->pf_arena);
    const hipStream_t s = m->stream;
    const int64_t start = m->pos;
    for (int64_t r0 = 0; r0 < n; r0 += p.tb) {
        const int T = static_cast<int>(std::min<int64_t>(p.tb, n - r0));
        // the previous block's kernels read the ids buffer: order the upload after them
        HIPCHK(hipMemcpyAsync(F + p.ids, ids + r0, static_cast<size_t>(T) * 4, hipMemcpyHostToDevice, s));
        const q35_status st = prefill_block(m, p, static_cast<int>(start + r0), T, r0, logits_host, trace_host);
        if (st != Q35_OK) return st;
        HIPCHK(hipStreamSynchronize(s));  // host ids / logits buffers are reused per block
        const q35_status tt = collect_timing(m);
        if (tt != Q35_OK) return tt;
    }
    const q35_dims& d = m->d;
    q35k::GemvArgs hd{};
    hd.W = m->head;
    hd.x = m->hidden;
    hd.norm_w = m->final_norm;
    hd.y = m->logits;
    hd.rows = d.vocab_size;
    hd.in_dim = d.hidden_size;
    hd.eps = d.rms_norm_eps;
    HIPCHK(q35k::launch_gemv(hd, q35k::kProRmsNorm, s));
    HIPCHK(q35k::launch_set_int(m->pos_dev, static_cast<int>(start + n - 1), s));
    HIPCHK(q35k::launch_argmax(m->logits, d.vocab_size, m->argmax_part, m->token_dev, m->ids_dev, m->pos_dev, s));
    HIPCHK(hipStreamSynchronize(s));
    m->pos = start + n;
    return Q35_OK;
}

// reference window [CONV][KER-1] (oldest first) <-> ring slot (t % 4) for t = pos-3..pos-1
int64_t ring_slot(int64_t pos, int k) { return (((pos - 3 + k) % 4) + 4) % 4; }

q35_status check_model(const q35_model* m) {
    return m ? Q35_OK : q35::fail(Q35_ERR_ARG, "null model");
}

}  // namespace

extern "C" {

int64_t q35_device_alloc_count(void) { return g_dev_allocs.load(); }

q35_status q35_model_create(const q35_dims* d, const q35_tensor* tensors, int32_t n_tensors,
                            int64_t max_context, q35_model** out) {
    return create_model(d, tensors, n_tensors, max_context, 4, 0, 0, out);
}

q35_status q35_model_create_opts(const q35_dims* d, const q35_tensor* tensors, int32_t n_tensors,
                                 int64_t max_context, const q35_model_options* opt, q35_model** out) {
    return create_model(d, tensors, n_tensors, max_context, opt ? opt->kv_bytes_per_elem : 4,
                        opt ? opt->prefill_block : 0, opt ? opt->prefill_exact : 0, out);
}

q35_status q35_model_open(const char* model_dir, int64_t max_context, q35_model** out) {
    return q35_model_open_opts(model_dir, max_context, nullptr, out);
}

q35_status q35_model_open_opts(const char* model_dir, int64_t max_context, const q35_model_options* opt,
                               q35_model** out) {
    if (!model_dir || !out) return q35::fail(Q35_ERR_ARG, "q35_model_open: null argument");
    ModelConfig cfg;
    load_model_config(std::string(model_dir) + "/config.json", cfg);
    SafeTensors st;
    if (!st.load_model(model_dir)) return q35::fail(Q35_ERR_IO, "cannot load safetensors from %s", model_dir);
    std::vector<q35_tensor> table;
    st.device_table(&table);
    q35_dims d;
    q35::dims_from_config(cfg, &d);
    return create_model(&d, table.data(), static_cast<int32_t>(table.size()), max_context,
                        opt ? opt->kv_bytes_per_elem : 4, opt ? opt->prefill_block : 0, opt ? opt->prefill_exact : 0,
                        out);
}

void q35_model_destroy(q35_model* m) { destroy(m); }

q35_status q35_model_dims(const q35_model* m, q35_dims* out) {
    if (!m || !out) return q35::fail(Q35_ERR_ARG, "null argument");
    *out = m->d;
    return Q35_OK;
}

q35_status q35_model_budget(const q35_model* m, q35_budget* out) {
    if (!m || !out) return q35::fail(Q35_ERR_ARG, "null argument");
    *out = m->budget;
    return Q35_OK;
}

int64_t q35_model_position(const q35_model* m) { return m ? m->pos : -1; }
int64_t q35_model_max_context(const q35_model* m) { return m ? m->max_ctx : -1; }
q35_stream q35_model_stream(const q35_model* m) { return m ? m->stream : nullptr; }

q35_status q35_model_synchronize(q35_model* m) {
    if (check_model(m) != Q35_OK) return Q35_ERR_ARG;
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

q35_status q35_model_reset(q35_model* m) {
    const q35_status nc = need_context(m);
    if (nc != Q35_OK) return nc;
    HIPCHK(q35k::launch_fill_f32(m->state_arena, static_cast<int64_t>(m->state_bytes / 4), 0.0f, m->stream));
    HIPCHK(q35k::launch_fill_f32(m->kv_arena, static_cast<int64_t>(m->kv_bytes / 4), 0.0f, m->stream));
    HIPCHK(q35k::launch_set_int(m->pos_dev, 0, m->stream));
    m->pos = 0;
    return Q35_OK;
}

q35_status q35_model_step(q35_model* m, int32_t token, float* logits_host, int32_t* argmax) {
    const q35_status nc = need_context(m);
    if (nc != Q35_OK) return nc;
    if (token < 0 || token >= m->embed_rows || token >= m->d.vocab_size)
        return q35::fail(Q35_ERR_RANGE, "token %d outside [0, %d)", token, m->d.vocab_size);
    if (m->pos >= m->max_ctx)
        return q35::fail(Q35_ERR_RANGE, "position %lld reached max_context %lld", (long long)m->pos,
                         (long long)m->max_ctx);
    *m->pinned_token = token;
    HIPCHK(hipMemcpyAsync(m->token_dev, m->pinned_token, 4, hipMemcpyHostToDevice, m->stream));
    q35_status st = launch_one_step(m);
    if (st != Q35_OK) return st;
    if (logits_host)
        HIPCHK(hipMemcpyAsync(logits_host, m->logits, static_cast<size_t>(m->d.vocab_size) * 4,
                              hipMemcpyDeviceToHost, m->stream));
    if (argmax) HIPCHK(hipMemcpyAsync(argmax, m->token_dev, 4, hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return collect_timing(m);
}

}  // extern "C"

namespace {

// n_steps back-to-back steps on the device: the first fed with `token`, each next one with
// the argmax the previous step left in token_dev. ids_dev[p] receives the argmax after
// the step at position p.
q35_status run_greedy(q35_model* m, int32_t token, int32_t n_steps) {
    const q35_status nc = need_context(m);
    if (nc != Q35_OK) return nc;
    if (token < 0 || token >= m->d.vocab_size)
        return q35::fail(Q35_ERR_RANGE, "token %d outside [0, %d)", token, m->d.vocab_size);
    if (m->pos + n_steps > m->max_ctx)
        return q35::fail(Q35_ERR_RANGE, "position %lld + %d steps exceeds max_context %lld", (long long)m->pos,
                         n_steps, (long long)m->max_ctx);
    *m->pinned_token = token;
    HIPCHK(hipMemcpyAsync(m->token_dev, m->pinned_token, 4, hipMemcpyHostToDevice, m->stream));
    const bool runs = m->use_graph && !m->timing_on && !m->trace_on;
    for (int i = 0; i < n_steps;) {
        const int k = runs && n_steps - i >= kGraphRun ? kGraphRun : 1;
        const q35_status st = launch_steps(m, k);
        if (st != Q35_OK) return st;
        if (m->timing_on) {
            const q35_status t = collect_timing(m);
            if (t != Q35_OK) return t;
        }
        i += k;
    }
    return Q35_OK;
}

}  // namespace

extern "C" {

q35_status q35_model_decode_greedy(q35_model* m, int32_t token, int32_t n_new, int32_t* out) {
    if (!m || (n_new > 0 && !out) || n_new < 0) return q35::fail(Q35_ERR_ARG, "bad argument");
    if (n_new == 0) return Q35_OK;
    const int64_t p0 = m->pos;
    const q35_status st = run_greedy(m, token, n_new);
    if (st != Q35_OK) return st;
    HIPCHK(hipMemcpyAsync(out, m->ids_dev + p0, static_cast<size_t>(n_new) * 4, hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

// Same step sequence as the reference loop (src/qwen_model.cpp:241-255): every prompt token,
// then n_new greedy steps, the last of which is fed with the last emitted id.
q35_status q35_model_generate_greedy(q35_model* m, const int32_t* prompt, int32_t n_prompt,
                                     int32_t n_new, int32_t* out) {
    if (!m || (n_prompt > 0 && !prompt) || n_prompt < 0 || n_new < 0 || (n_new > 0 && !out))
        return q35::fail(Q35_ERR_ARG, "bad argument");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    if (n_prompt + static_cast<int64_t>(n_new) > m->max_ctx)
        return q35::fail(Q35_ERR_RANGE, "prompt + new tokens (%d + %d) exceed max_context %lld", n_prompt, n_new,
                         (long long)m->max_ctx);
    q35_status st = q35_model_reset(m);
    if (st != Q35_OK) return st;
    if (n_prompt == 0) return Q35_OK;  // the reference emits nothing without logits
    for (int i = 0; i + 1 < n_prompt; ++i) {
        st = q35_model_step(m, prompt[i], nullptr, nullptr);
        if (st != Q35_OK) return st;
    }
    int32_t am = 0;
    st = q35_model_step(m, prompt[n_prompt - 1], nullptr, &am);
    if (st != Q35_OK || n_new == 0) return st;
    st = run_greedy(m, am, n_new);
    if (st != Q35_OK) return st;
    HIPCHK(hipMemcpyAsync(out, m->ids_dev + (n_prompt - 1), static_cast<size_t>(n_new) * 4, hipMemcpyDeviceToHost,
                          m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

q35_status q35_model_set_graph(q35_model* m, int32_t enable) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    m->use_graph = enable != 0;
    return Q35_OK;
}

q35_status q35_model_set_attn_splits(q35_model* m, int32_t n_splits) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    if (n_splits < 0 || n_splits > kMaxSplits)
        return q35::fail(Q35_ERR_RANGE, "n_splits %d outside [0, %d]", n_splits, kMaxSplits);
    m->n_splits = n_splits > 0 ? n_splits : q35k::attn_default_splits(m->max_ctx, m->d.attn_kv_heads, m->n_cu);
    drop_graph(m);
    return Q35_OK;
}

q35_status q35_model_set_layer_trace(q35_model* m, int32_t enable) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    m->trace_on = enable != 0;
    return Q35_OK;
}

q35_status q35_model_read_layer_trace(q35_model* m, float* host) {
    if (!m || !host) return q35::fail(Q35_ERR_ARG, "null argument");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    HIPCHK(hipMemcpyAsync(host, m->trace, static_cast<size_t>(m->d.n_layers_total) * m->d.hidden_size * 4,
                          hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

q35_status q35_model_read_hidden(q35_model* m, float* host) {
    if (!m || !host) return q35::fail(Q35_ERR_ARG, "null argument");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    HIPCHK(hipMemcpyAsync(host, m->hidden, static_cast<size_t>(m->d.hidden_size) * 4, hipMemcpyDeviceToHost,
                          m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

q35_status q35_model_set_kernel_timing(q35_model* m, int32_t enable) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    m->timing_on = enable != 0;
    m->ev_used = 0;
    return Q35_OK;
}

q35_status q35_model_kernel_times(q35_model* m, double* ms, int64_t* launches) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    const q35_status st = collect_timing(m);
    if (st != Q35_OK) return st;
    for (int i = 0; i < Q35_KT_COUNT; ++i) {
        if (ms) ms[i] = m->kt_ms[i];
        if (launches) launches[i] = m->kt_n[i];
        m->kt_ms[i] = 0.0;
        m->kt_n[i] = 0;
    }
    return Q35_OK;
}

q35_status q35_model_read_gdn_state(q35_model* m, int32_t layer, float* host) {
    if (!m || !host || layer < 0 || layer >= m->d.n_layers_gdn) return q35::fail(Q35_ERR_ARG, "bad argument");
    const size_t n = static_cast<size_t>(m->d.gdn_v_heads) * 128 * 128;
    HIPCHK(hipMemcpyAsync(host, m->gdn_state + layer * n, n * 4, hipMemcpyDeviceToHost, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

q35_status q35_model_write_gdn_state(q35_model* m, int32_t layer, const float* host) {
    if (!m || !host || layer < 0 || layer >= m->d.n_layers_gdn) return q35::fail(Q35_ERR_ARG, "bad argument");
    const size_t n = static_cast<size_t>(m->d.gdn_v_heads) * 128 * 128;
    HIPCHK(hipMemcpyAsync(m->gdn_state + layer * n, host, n * 4, hipMemcpyHostToDevice, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

q35_status q35_model_read_conv_state(q35_model* m, int32_t layer, float* host) {
    if (!m || !host || layer < 0 || layer >= m->d.n_layers_gdn) return q35::fail(Q35_ERR_ARG, "bad argument");
    const int64_t conv = 2LL * m->d.gdn_k_heads * 128 + m->d.gdn_v_heads * 128;
    std::vector<float> ring(static_cast<size_t>(4 * conv));
    HIPCHK(hipMemcpyAsync(ring.data(), m->conv_ring + layer * 4 * conv, ring.size() * 4, hipMemcpyDeviceToHost,
                          m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    for (int64_t c = 0; c < conv; ++c)
        for (int k = 0; k < 3; ++k) host[c * 3 + k] = ring[static_cast<size_t>(ring_slot(m->pos, k) * conv + c)];
    return Q35_OK;
}

q35_status q35_model_write_conv_state(q35_model* m, int32_t layer, const float* host) {
    if (!m || !host || layer < 0 || layer >= m->d.n_layers_gdn) return q35::fail(Q35_ERR_ARG, "bad argument");
    const int64_t conv = 2LL * m->d.gdn_k_heads * 128 + m->d.gdn_v_heads * 128;
    std::vector<float> ring(static_cast<size_t>(4 * conv), 0.0f);
    for (int64_t c = 0; c < conv; ++c)
        for (int k = 0; k < 3; ++k) ring[static_cast<size_t>(ring_slot(m->pos, k) * conv + c)] = host[c * 3 + k];
    HIPCHK(hipMemcpyAsync(m->conv_ring + layer * 4 * conv, ring.data(), ring.size() * 4, hipMemcpyHostToDevice,
                          m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return Q35_OK;
}

q35_status q35_model_read_kv(q35_model* m, int32_t layer, int64_t pos0, int64_t n, float* k_host,
                             float* v_host) {
    if (!m || layer < 0 || layer >= m->d.n_layers_attn || pos0 < 0 || n < 0 || pos0 + n > m->max_ctx)
        return q35::fail(Q35_ERR_ARG, "bad argument");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    const int NKV = m->d.attn_kv_heads, HD = m->d.attn_head_dim, E = m->kv_elem;
    std::vector<uint16_t> tmp(m->kv_elem == 2 ? static_cast<size_t>(n) * NKV * HD : 0);
    for (int which = 0; which < 2; ++which) {
        float* dst = which == 0 ? k_host : v_host;
        if (!dst) continue;
        void* hdst = E == 2 ? static_cast<void*>(tmp.data()) : static_cast<void*>(dst);
        for (int kh = 0; kh < NKV; ++kh) {
            const uint8_t* src = reinterpret_cast<const uint8_t*>(kv_ptr(m, layer, which, kh)) + pos0 * HD * E;
            HIPCHK(hipMemcpy2DAsync(static_cast<uint8_t*>(hdst) + static_cast<size_t>(kh) * HD * E,
                                    static_cast<size_t>(NKV) * HD * E, src, static_cast<size_t>(HD) * E,
                                    static_cast<size_t>(HD) * E, static_cast<size_t>(n), hipMemcpyDeviceToHost,
                                    m->stream));
        }
        HIPCHK(hipStreamSynchronize(m->stream));
        if (E == 2)
            for (size_t i = 0; i < tmp.size(); ++i) dst[i] = bf16_to_f32(tmp[i]);
    }
    return Q35_OK;
}

// Host rows into the cache; a bf16 cache stores them rounded to nearest even.
q35_status q35_model_write_kv(q35_model* m, int32_t layer, int64_t pos0, int64_t n, const float* k_host,
                              const float* v_host) {
    if (!m || layer < 0 || layer >= m->d.n_layers_attn || pos0 < 0 || n < 0 || pos0 + n > m->max_ctx)
        return q35::fail(Q35_ERR_ARG, "bad argument");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    const int NKV = m->d.attn_kv_heads, HD = m->d.attn_head_dim, E = m->kv_elem;
    std::vector<uint16_t> tmp(m->kv_elem == 2 ? static_cast<size_t>(n) * NKV * HD : 0);
    for (int which = 0; which < 2; ++which) {
        const float* src = which == 0 ? k_host : v_host;
        if (!src) continue;
        if (E == 2)
            for (size_t i = 0; i < tmp.size(); ++i) tmp[i] = q35synth::f32_to_bf16(src[i]);
        const void* hsrc = E == 2 ? static_cast<const void*>(tmp.data()) : static_cast<const void*>(src);
        for (int kh = 0; kh < NKV; ++kh) {
            uint8_t* dst = reinterpret_cast<uint8_t*>(kv_ptr(m, layer, which, kh)) + pos0 * HD * E;
            HIPCHK(hipMemcpy2DAsync(dst, static_cast<size_t>(HD) * E,
                                    static_cast<const uint8_t*>(hsrc) + static_cast<size_t>(kh) * HD * E,
                                    static_cast<size_t>(NKV) * HD * E, static_cast<size_t>(HD) * E,
                                    static_cast<size_t>(n), hipMemcpyHostToDevice, m->stream));
        }
        HIPCHK(hipStreamSynchronize(m->stream));
    }
    return Q35_OK;
}

q35_status q35_model_set_position(q35_model* m, int64_t pos) {
    if (!m || pos < 0 || pos > m->max_ctx) return q35::fail(Q35_ERR_RANGE, "bad position");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    HIPCHK(q35k::launch_set_int(m->pos_dev, static_cast<int>(pos), m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    m->pos = pos;
    return Q35_OK;
}

q35_status q35_model_fill_synthetic(q35_model* m, int64_t pos, uint64_t seed, float state_std) {
    if (!m || pos < 0 || pos > m->max_ctx) return q35::fail(Q35_ERR_RANGE, "bad position");
    if (need_context(m) != Q35_OK) return Q35_ERR_RANGE;
    const int NKV = m->d.attn_kv_heads, HD = m->d.attn_head_dim;
    for (int l = 0; l < m->d.n_layers_attn; ++l)
        for (int which = 0; which < 2; ++which)
            for (int kh = 0; kh < NKV; ++kh) {
                float* dst = kv_ptr(m, l, which, kh);
                const uint64_t stream = 0x4b560000ULL + (static_cast<uint64_t>(l) << 8) + (which << 4) + kh;
                HIPCHK(q35k::launch_fill_normal(dst, pos * HD, q35synth::stream_key(seed, stream), 1.0f,
                                                m->stream, m->kv_elem == 2));
            }
    const int64_t ns = static_cast<int64_t>(m->d.n_layers_gdn) * m->d.gdn_v_heads * 128 * 128;
    HIPCHK(q35k::launch_fill_normal(m->gdn_state, ns, q35synth::stream_key(seed, 0x47444eULL), state_std, m->stream));
    const int64_t conv = 2LL * m->d.gdn_k_heads * 128 + m->d.gdn_v_heads * 128;
    HIPCHK(q35k::launch_fill_f32(m->conv_ring, static_cast<int64_t>(m->d.n_layers_gdn) * 4 * conv, 0.0f, m->stream));
    HIPCHK(q35k::launch_set_int(m->pos_dev, static_cast<int>(pos), m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    m->pos = pos;
    return Q35_OK;
}

q35_status q35_model_prefill(q35_model* m, const int32_t* ids, int32_t n, float* logits_host) {
    if (!m || !ids || n <= 0) return q35::fail(Q35_ERR_ARG, "bad argument");
    if (n > m->max_ctx) return q35::fail(Q35_ERR_RANGE, "prompt of %d exceeds max_context", n);
    const q35_status st = q35_model_reset(m);
    if (st != Q35_OK) return st;
    return extend(m, ids, n, logits_host, nullptr);
}

q35_status q35_model_extend(q35_model* m, const int32_t* ids, int32_t n, float* logits_host, float* trace_host) {
    return extend(m, ids, n, logits_host, trace_host);
}

q35_status q35_model_set_prefill_block(q35_model* m, int32_t tokens) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    if (tokens < 0 || tokens > (1 << 20)) return q35::fail(Q35_ERR_RANGE, "prefill block %d", tokens);
    if (m->pf_planned > 0 && tokens > m->pf_planned)
        return q35::fail(Q35_ERR_RANGE, "prefill block %d beyond the %d tokens the prompt arena was planned for", tokens,
                         m->pf_planned);
    m->pf_block = tokens;
    return Q35_OK;
}

q35_status q35_model_set_prefill_head(q35_model* m, int32_t head) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    if (head != Q35_HEAD_OUTPUT && head != Q35_HEAD_EMBEDDING) return q35::fail(Q35_ERR_ARG, "prefill head %d", head);
    m->prefill_head = head;
    return Q35_OK;
}

int64_t q35_model_prefill_logits_width(const q35_model* m) {
    if (!m) return -1;
    return m->prefill_head ? m->embed_rows : m->d.vocab_size;
}

q35_status q35_model_reserve_context(q35_model* m, int64_t max_context) {
    if (!m) return q35::fail(Q35_ERR_ARG, "null model");
    if (max_context <= 0 || max_context > (int64_t{1} << 30))
        return q35::fail(Q35_ERR_RANGE, "max_context %lld out of range", static_cast<long long>(max_context));
    if (max_context <= m->max_ctx) return Q35_OK;
    HIPCHK(hipStreamSynchronize(m->stream));
    drop_graph(m);
    const q35_status st = alloc_context(m, max_context);
    if (!m->scratch) return st;  // no context arenas: every call that needs them refuses
    // the recurrent state goes back to zero with the cache (also when a failed reservation
    // made the old arenas again): the model is reset
    HIPCHK(q35k::launch_fill_f32(m->state_arena, static_cast<int64_t>(m->state_bytes / 4), 0.0f, m->stream));
    HIPCHK(hipStreamSynchronize(m->stream));
    return st;
}

}  // extern "C"
