// engine.cpp -- MI355X decode engine behind include/atlas_engine.h.
//
// Host-side mirror of the reference's decode orchestration
// (crates/atlas-model/src/lib.rs: OlmoModel 1298-2009, TransformerBlock
// 982-1091, Attention 598-870, FeedForward 882-924; crates/atlas-infer:
// InferEngine::generate and StigmergicHook), re-laid out for one MI355X:
//
//  * weights live in HBM in the stored format (bf16 / int8 / int4), with
//    wq|wk|wv concatenated into one [d + 2*kv_dim, d] matrix and gate/up rows
//    interleaved (gate_i, up_i) so one GEMV launch yields silu(gate)*up;
//  * one decode step = embed gather, per layer {QKV GEMV, QK-norm+RoPE+KV
//    write, split-K attention, W_o GEMV, residual RMSNorm, SwiGLU GEMV,
//    W_down GEMV, residual RMSNorm}, final RMSNorm, lm_head GEMV and (greedy)
//    device argmax -- no per-op allocation (the reference allocates a fresh
//    buffer per op, crates/atlas-tensor/src/lib.rs:196-206);
//  * the step reads its token and position from device memory, so it is
//    captured once in a HIP graph and replayed per token; greedy decode needs
//    no host round trip per token (the reference downloads 401 KB of logits
//    per token, lib.rs:1504);
//  * sampling with temperature runs the reference's host pipeline on the
//    downloaded logits (lib.rs:1652-1711).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/atlas_engine.h"
#include "attention.hpp"
#include "common.hpp"
#include "fused.hpp"
#include "gemv.hpp"

using namespace atlas;

namespace {

// Context length from which decode steps give the fused attention (one
// launch per layer, split merge inside the kernel) up for three launches:
// QK-norm/RoPE/KV write, the split kernel and the split merge (the two-kernel
// path of atlas_decode_attention).  With the fused kernel's partials published
// by sc1 stores and its split count fitted per context it is the faster step
// at every measured context of the 7B bf16 decode (2.89 vs 2.99 ms/token at
// ctx 600, 2.93 vs 3.12 at 1200, 3.37 vs 3.52 at 4000), so the long-context
// step runs only from a position the caller sets.
constexpr int kLongAttnFrom = 1 << 30;
// The ragged batch's shared steps switch to the split kernel + merge from
// this position of their longest row (or the caller's long_from, if lower).
constexpr int kBatchLongAttnFrom = 512;
// Rows of the multi-row step, and prompt tokens per prefill step: the
// multi-row GEMV for 2-3 rows, the skinny MFMA kernel for 4-16.
constexpr int kPrefillChunk = 16;
constexpr int kMaxRows = kPrefillChunk;
// Prompt chunks of models whose GEMM inner dims are multiples of 128 go
// through the tiled MFMA GEMM (gemm_rows_launch), up to this many rows
// per step, replayed eagerly (the captured steps stop at kMaxRows rows).
constexpr int kPrefillBig = 128;
// ... and up to this many rows per step in all: the library GEMM (bf16, int8)
// takes them at once (at the 7B shapes the GEMMs of a layer cost 1.28 us per
// prompt token at 127 rows, 0.87 at 255 and 0.68 at 511, bf16; a 2047-token
// prompt took 76.8 ms in 512-row chunks and 68.9 in 1024), the tiled kernel
// (int4) in 128-row launches; the chunk's attention then runs on the matrix
// cores (above 128 rows).
constexpr int kPrefillLib = 1024;

struct DevMat {
    int fmt = WF_BF16;
    void* w = nullptr;
    float* scales = nullptr;
    int rows = 0, cols = 0, block = 0;
    size_t pitch = 0;        // bytes between rows in HBM; 0 = packed (row_bytes)
    size_t row_pitch() const { return pitch ? pitch : row_bytes(); }
    size_t row_bytes() const {
        switch (fmt) {
        case WF_F32: return (size_t)cols * 4;
        case WF_BF16: return (size_t)cols * 2;
        case WF_I8: return (size_t)cols;
        default: return (size_t)cols / 2;
        }
    }
    size_t scales_per_row() const {
        if (fmt == WF_I8) return 1;
        if (fmt == WF_I4) return (size_t)cols / block;
        return 0;
    }
    size_t data_bytes() const { return row_bytes() * rows; }     // algorithmic bytes
    size_t alloc_bytes() const { return row_pitch() * rows; }
    size_t scale_count() const { return scales_per_row() * rows; }
};

struct LayerW {
    DevMat qkv, wo, gu, down;
    float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float *kc = nullptr, *vc = nullptr;
    int window = 0;
};

// XorShift64 of the reference's sampling Rng (lib.rs:1190-1220)
struct Rng {
    uint64_t s;
    float next_f32() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return (float)(s >> 33) / (float)(1ULL << 31);
    }
};

}  // namespace

struct atlas_model {
    atlas_model_config cfg{};
    std::vector<uint8_t> sliding;
    int hd = 0, kvd = 0, qkv_rows = 0, B = 1;
    int R = 1;                       // rows of the multi-row step buffers: max(B, prefill chunk)
    int RF = 1;                      // rows with a fused attention, logits and a choice: max(B, 16 or 128)
    int prefill_chunk = kPrefillLib;     // prompt tokens per prefill step (1: token by token)
    bool big_prefill = false;            // chunks above 16 rows, up to kPrefillLib (prefill_cap)
    float scale = 1.f;
    std::vector<LayerW> L;
    uint16_t* embed = nullptr;
    DevMat lm_head;
    float* final_norm = nullptr;
    float *cos_tab = nullptr, *sin_tab = nullptr;
    float* rope_row = nullptr;           // the fused step's RoPE row at pos (embed writes it)
    float *x = nullptr, *xn = nullptr, *y = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr,
          *logits = nullptr;
    // fused step: residual ping-pong partner of x, the W_down output, split
    // partials and merge counters of the fused attention
    float *xb = nullptr, *y2 = nullptr;
    float* attn_part = nullptr;
    int* attn_counters = nullptr;
    // split-K partials of the multi-row GEMMs (ragged batch, prompt chunks):
    // the model's own, so captured steps never point at shared scratch
    float* gemm_part = nullptr;
    size_t gemm_part_bytes = 0;
    // bf16 / int8 prompt chunks (17..1024 rows): hipBLASLt context (null: the tiled kernel)
    BlasRows* blas = nullptr;
    bool fused = false;
    int *pos_dev = nullptr, *slot_dev = nullptr, *step_dev = nullptr, *hist_len = nullptr;
    uint32_t *tok_dev = nullptr, *hist = nullptr, *suppress_dev = nullptr, *choice_dev = nullptr;
    int suppress_cap = 0;
    SampleCfg* samp_cfg = nullptr;       // device sampling settings (mode 2)
    unsigned long long* rng_dev = nullptr;   // device XorShift64 state (mode 2)
    unsigned long long* argpart = nullptr;
    long slot_stride = 0;
    int attn_splits = 1;           // fused kernel: maximum (grid) split count
    int attn_splits_unfused = 1;
    int attn_splits_long = 1;      // long-context step: split kernel grid (adaptive)
    int attn_splits_batch[kMaxRows + 1] = {};   // two-kernel batch step of n rows: split grid
    int long_from = kLongAttnFrom; // positions >= this replay the long-context step
    int pos = 0;
    hipStream_t st = nullptr;
    bool use_graph = true;
    // captured decode steps per mode: 0 forward, 1 + greedy choice, 2 + sampled choice
    // step modes: 0 logits, 1 greedy choice, 2 device sampling, 3 logits plus
    // every layer's hidden state (hooked)
    hipGraphExec_t gexec[4] = {nullptr, nullptr, nullptr, nullptr};
    hipGraphExec_t gexec_long[4] = {nullptr, nullptr, nullptr, nullptr};
    hipGraphExec_t bgexec[kMaxRows + 1] = {};       // multi-row step per row count
    hipGraphExec_t bgexec_long[kMaxRows + 1] = {};  // ... its two-kernel attention variant
    hipGraphExec_t pgexec[kMaxRows + 1] = {};       // prefill step (no lm_head) per row count
    hipGraphExec_t pgexec_long[kMaxRows + 1] = {};
    // pinned staging ring for the batch step's tokens / positions / slots:
    // entry k is rewritten only after its event (the copies) completed
    static constexpr int kRing = 8;
    int* ring = nullptr;             // [kRing][3][kMaxRows]
    hipEvent_t ring_ev[kRing] = {};
    bool ring_used[kRing] = {};
    // [n_layers][d_model] of the hooked step's per-layer hidden states: on the
    // device (mode 3 copies them there) and pinned on the host
    float* hook_dev = nullptr;
    float* hook_stage = nullptr;
    // greedy choice settings baked into the captured graph
    float g_theta = 1.f;
    int g_window = 0, g_nsup = 0;
    std::vector<void*> allocs;
    Rng rng{0x517cc1b727220a95ULL};
};

namespace {

int dalloc(atlas_model* m, void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) return ATLAS_OK;
    if (dev_malloc(p, bytes) != hipSuccess || !*p) {
        (void)hipGetLastError();
        *p = nullptr;
        set_error(ATLAS_ENOMEM, "engine: device allocation of %zu bytes failed", bytes);
        return ATLAS_ENOMEM;
    }
    m->allocs.push_back(*p);
    return ATLAS_OK;
}

#define TRY(expr)                 \
    do {                          \
        int rc_ = (expr);         \
        if (rc_) return rc_;      \
    } while (0)

// Row pitch in HBM.  bf16 rows longer than 8 KB whose length is not a
// multiple of 4 KB (the 7B W_down: 22016 B) stream ~10% faster with one
// extra 256-byte gap per row; other rows are stored packed.
size_t pad_pitch(int fmt, int cols) {
    if (fmt != WF_BF16 || cols <= 4096) return 0;
    const size_t rb = (size_t)cols * 2;
    if (rb % 4096 == 0) return 0;
    return (rb + 255) / 256 * 256 + 256;
}

int alloc_mat(atlas_model* m, DevMat& d, int fmt, int rows, int cols, int block) {
    d.fmt = fmt;
    d.rows = rows;
    d.cols = cols;
    d.block = block;
    d.pitch = pad_pitch(fmt, cols);
    TRY(dalloc(m, &d.w, d.alloc_bytes()));
    if (d.scale_count()) TRY(dalloc(m, (void**)&d.scales, d.scale_count() * 4));
    return ATLAS_OK;
}

GemvArgs gemv_args(const DevMat& w, const float* x, float* y, int epi) {
    GemvArgs a{};
    a.fmt = w.fmt;
    a.w = w.w;
    a.scales = w.scales;
    a.block = w.block;
    a.x = x;
    a.y = y;
    a.M = w.rows;
    a.K = w.cols;
    a.epi = epi;
    a.N = 1;
    a.ldw = (long)w.pitch;
    return a;
}

int gemv(atlas_model* m, const DevMat& w, const float* x, float* y, int epi) {
    return gemv_launch(gemv_args(w, x, y, epi), m->st);
}

int skinny(atlas_model* m, const DevMat& w, const float* x, float* y, int n, int epi,
           int* defer_splits = nullptr) {
    GemvArgs a = gemv_args(w, x, y, epi);
    a.defer_splits = defer_splits;
    a.N = n;
    a.x_stride_n = w.cols;
    a.x_stride_k = 1;
    a.y_stride_n = epi == EPI_SILU_MUL ? w.rows / 2 : w.rows;
    a.y_stride_m = 1;
    a.partial = m->gemm_part;
    a.partial_bytes = m->gemm_part_bytes;
    a.blas = m->blas;
    return skinny_launch(a, m->st);
}

// ---- RoPE tables: RopeCache::new (crates/atlas-model/src/lib.rs:380-423) on
// the host with the same f32 libm calls, then uploaded (GpuRopeTables).
void rope_tables(const atlas_model_config& c, int hd, std::vector<float>& cs,
                 std::vector<float>& sn) {
    const int half = hd / 2;
    const float two_pi = 2.0f * 3.14159265358979323846f;
    std::vector<float> f(half);
    for (int i = 0; i < half; ++i) {
        const float base = 1.0f / powf(c.rope_theta, 2.0f * (float)i / (float)hd);
        float v = base;
        if (c.yarn) {
            const float wl = two_pi / base;
            const float low = (float)c.yarn_orig_max_pos / (two_pi * c.yarn_beta_slow);
            const float high = (float)c.yarn_orig_max_pos / (two_pi * c.yarn_beta_fast);
            if (wl < high) v = base;
            else if (wl > low) v = base / c.yarn_factor;
            else {
                const float alpha = (wl - high) / (low - high);
                v = base / (alpha * c.yarn_factor + (1.0f - alpha));
            }
        }
        f[i] = v;
    }
    cs.resize((size_t)c.max_seq * half);
    sn.resize((size_t)c.max_seq * half);
    for (int p = 0; p < c.max_seq; ++p)
        for (int i = 0; i < half; ++i) {
            cs[(size_t)p * half + i] = cosf((float)p * f[i]);
            sn[(size_t)p * half + i] = sinf((float)p * f[i]);
        }
}

// ---- one transformer layer, batch 1 -------------------------------------
int layer_step(atlas_model* m, int li) {
    const atlas_model_config& c = m->cfg;
    LayerW& L = m->L[li];
    const int d = c.d_model;
    const float* xin = m->x;
    if (!c.post_norm) {
        TRY(rmsnorm_launch(m->x, L.attn_norm, m->xn, d, 1, d, c.rms_eps, m->st));
        xin = m->xn;
    }
    TRY(gemv(m, L.qkv, xin, m->qkv, EPI_STORE));
    QkvPostArgs q{};
    q.qkv = m->qkv; q.qkv_stride = m->qkv_rows;
    q.q_norm = L.q_norm; q.k_norm = L.k_norm; q.qk_eps = 1e-6f;
    q.cos_tab = m->cos_tab; q.sin_tab = m->sin_tab;
    q.k_cache = L.kc; q.v_cache = L.vc; q.slot_stride = m->slot_stride;
    q.slot_dev = nullptr; q.pos_dev = m->pos_dev; q.pos = 0;
    q.n_heads = c.n_heads; q.n_kv = c.n_kv_heads; q.head_dim = m->hd;
    TRY(qkv_post_launch(q, 1, m->st));
    AttnArgs a{};
    a.q = m->qkv; a.k_cache = L.kc; a.v_cache = L.vc; a.out = m->att;
    a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = m->hd;
    a.pos = 0; a.pos_dev = m->pos_dev; a.scale = m->scale; a.window = L.window;
    a.max_rows = c.max_seq;
    // the model's own partials: a captured step must not point at library
    // scratch that another model's reservation may reallocate
    const size_t np = (size_t)c.n_heads * m->attn_splits_unfused;
    a.part_m = m->attn_part; a.part_l = m->attn_part + np; a.part_o = m->attn_part + 2 * np;
    TRY(attn_launch(a, m->attn_splits_unfused, m->st));
    TRY(gemv(m, L.wo, m->att, m->y, EPI_STORE));
    if (c.post_norm) {
        TRY(residual_rmsnorm_launch(m->x, m->y, L.attn_norm, d, 1, d, c.rms_eps, m->st));
        TRY(gemv(m, L.gu, m->x, m->h, EPI_SILU_MUL));
        TRY(gemv(m, L.down, m->h, m->y, EPI_STORE));
        TRY(residual_rmsnorm_launch(m->x, m->y, L.ffn_norm, d, 1, d, c.rms_eps, m->st));
    } else {
        TRY(ew_launch(EW_ADD, m->x, m->y, m->x, 0.f, d, m->st));
        TRY(rmsnorm_launch(m->x, L.ffn_norm, m->xn, d, 1, d, c.rms_eps, m->st));
        TRY(gemv(m, L.gu, m->xn, m->h, EPI_SILU_MUL));
        TRY(gemv(m, L.down, m->h, m->y, EPI_STORE));
        TRY(ew_launch(EW_ADD, m->x, m->y, m->x, 0.f, d, m->st));
    }
    return ATLAS_OK;
}

int head_step(atlas_model* m) {
    const atlas_model_config& c = m->cfg;
    TRY(rmsnorm_launch(m->x, m->final_norm, m->xn, c.d_model, 1, c.d_model, c.rms_eps, m->st));
    TRY(gemv(m, m->lm_head, m->xn, m->logits, EPI_STORE));
    return ATLAS_OK;
}

SampleArgs sample_args(atlas_model* m, int* pos_inc) {
    SampleArgs a{};
    a.x = m->logits; a.n = m->cfg.vocab; a.cfg = m->samp_cfg;
    a.suppress = m->suppress_dev;
    a.hist = m->hist; a.hist_len = m->hist_len; a.step = m->step_dev; a.pos_inc = pos_inc;
    a.rng = m->rng_dev; a.out_u32 = m->tok_dev; a.record = 1;
    return a;
}

int choose_step(atlas_model* m) {
    ArgmaxArgs g{};
    g.x = m->logits; g.n = m->cfg.vocab; g.part = m->argpart;
    g.out_u32 = m->tok_dev;
    g.suppress = m->g_nsup ? m->suppress_dev : nullptr; g.n_suppress = m->g_nsup;
    g.hist = m->hist; g.hist_len = m->hist_len; g.window = m->g_window; g.theta = m->g_theta;
    g.step = m->step_dev; g.record = 1;
    return argmax_launch(g, m->st);
}

GemvArgs pro_args(const DevMat& w, const float* x, float* y, int pro, const float* py,
                  const float* pw, float eps, float* pout) {
    GemvArgs a = gemv_args(w, x, y, EPI_STORE);
    a.pro = pro;
    a.pro_y = py;
    a.pro_w = pw;
    a.pro_eps = eps;
    a.pro_out = pout;
    return a;
}

// Attention of the long-context step: QK-norm + RoPE in place and the K/V
// cache write, then split kernel + merge with the split count of the live
// context (read on the device, so one captured step serves every position).
int enqueue_attn_long(atlas_model* m, const LayerW& L) {
    const atlas_model_config& c = m->cfg;
    QkvPostArgs q{};
    q.qkv = m->qkv; q.qkv_stride = m->qkv_rows;
    q.q_norm = L.q_norm; q.k_norm = L.k_norm; q.qk_eps = 1e-6f;
    q.cos_tab = m->cos_tab; q.sin_tab = m->sin_tab;
    q.k_cache = L.kc; q.v_cache = L.vc; q.slot_stride = m->slot_stride;
    q.slot_dev = nullptr; q.pos_dev = m->pos_dev; q.pos = 0;
    q.n_heads = c.n_heads; q.n_kv = c.n_kv_heads; q.head_dim = m->hd;
    TRY(qkv_post_launch(q, 1, m->st));
    AttnArgs a{};
    a.q = m->qkv; a.k_cache = L.kc; a.v_cache = L.vc; a.out = m->att;
    a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = m->hd;
    a.pos = 0; a.pos_dev = m->pos_dev; a.scale = m->scale; a.window = L.window;
    a.max_rows = c.max_seq;
    a.adaptive = 1;
    const size_t np = (size_t)c.n_heads * m->attn_splits_long;
    a.part_m = m->attn_part;
    a.part_l = m->attn_part + np;
    a.part_o = m->attn_part + 2 * np;
    return attn_launch(a, m->attn_splits_long, m->st);
}

// GU of the fused step: x'_l = x_l + rmsnorm(y1) * attn_norm_l materialised
// into xb, then h = silu(gate) * up in the epilogue.
int enqueue_gu_fused(atlas_model* m, const LayerW& L) {
    GemvArgs gu = pro_args(L.gu, m->x, m->h, PRO_RESNORM, m->y, L.attn_norm, m->cfg.rms_eps, m->xb);
    gu.epi = EPI_SILU_MUL;
    return gemv_launch(gu, m->st);
}

// DOWN of the fused step: y2 = W_down h.
int enqueue_down_fused(atlas_model* m, const LayerW& L) {
    return gemv(m, L.down, m->h, m->y2, EPI_STORE);
}

// The post-norm decode step with the norms folded into the GEMV prologues
// and one attention launch per layer (5 launches per layer):
//   QKV    x_l = x'_{l-1} + rmsnorm(y2) * ffn_norm_{l-1}   (layer 0: embedding)
//   ATTN   QK-norm + RoPE + KV write + split-K attention + merge
//   WO     y1 = W_o att
//   GU     x'_l = x_l + rmsnorm(y1) * attn_norm_l;  h = silu(gate) * up
//   DOWN   y2 = W_down h
// x_l lives in m->x, x'_l in m->xb.
int enqueue_step_fused(atlas_model* m, int mode, bool long_ctx) {
    const atlas_model_config& c = m->cfg;
    const int d = c.d_model;
    const float eps = c.rms_eps;
    RopeRowArgs rr;
    rr.pos_dev = m->pos_dev; rr.cos_tab = m->cos_tab; rr.sin_tab = m->sin_tab; rr.half = m->hd / 2;
    rr.out = long_ctx ? nullptr : m->rope_row;
    TRY(embed_launch(m->embed, c.vocab, d, m->tok_dev, 0, m->x, d, 1, m->st, rr));
    for (int li = 0; li < c.n_layers; ++li) {
        LayerW& L = m->L[li];
        if (li == 0)
            TRY(gemv_launch(pro_args(L.qkv, m->x, m->qkv, PRO_X, nullptr, nullptr, 0.f, nullptr), m->st));
        else
            TRY(gemv_launch(pro_args(L.qkv, m->xb, m->qkv, PRO_RESNORM, m->y2, m->L[li - 1].ffn_norm,
                                     eps, m->x), m->st));
        // the QKV prologue wrote the hidden state after layer li - 1 into x
        if (mode == 3 && li > 0)
            TRY(ew_launch(EW_COPY, m->x, nullptr, m->hook_dev + (size_t)(li - 1) * d, 0.f, d, m->st));
        if (long_ctx) {
            TRY(enqueue_attn_long(m, L));
        } else {
            AttnFusedArgs a{};
            a.qkv = m->qkv; a.qkv_stride = m->qkv_rows;
            a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.qk_eps = 1e-6f;
            a.cos_tab = m->cos_tab; a.sin_tab = m->sin_tab;
            a.k_cache = L.kc; a.v_cache = L.vc; a.slot_stride = m->slot_stride;
            a.slot_dev = nullptr; a.pos_dev = m->pos_dev;
            a.out = m->att; a.out_stride = d;
            a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = m->hd;
            a.scale = m->scale; a.window = L.window;
            a.part_m = m->attn_part;
            a.part_l = m->attn_part + (size_t)m->RF * c.n_heads * m->attn_splits;
            a.part_o = m->attn_part + (size_t)2 * m->RF * c.n_heads * m->attn_splits;
            a.counters = m->attn_counters;
            a.adaptive = 1; a.max_rows = c.max_seq;
            a.rope_row = m->rope_row;
            TRY(attn_fused_launch(a, m->attn_splits, 1, m->st));
        }
        TRY(gemv(m, L.wo, m->att, m->y, EPI_STORE));
        TRY(enqueue_gu_fused(m, L));
        TRY(enqueue_down_fused(m, L));
    }
    // lm_head with the last layer's residual and the final norm in its prologue:
    // x_L = x'_{L-1} + rmsnorm(y2) * ffn_norm_{L-1} (into the hook's last slot in
    // mode 3), logits = W_lm rmsnorm(x_L) * final_norm.  Shapes the decode GEMV
    // does not cover keep a residual launch and the final norm prologue.
    const bool penalties = m->g_nsup > 0 || m->g_theta != 1.0f;
    float* hook_last = mode == 3 ? m->hook_dev + (size_t)(c.n_layers - 1) * d : nullptr;
    GemvArgs h = pro_args(m->lm_head, m->xb, m->logits, PRO_RESNORM_NORM, m->y2,
                          m->L[c.n_layers - 1].ffn_norm, eps, hook_last);
    h.pro_w2 = m->final_norm;
    if (!gemv_resnorm_norm_ok(h)) {
        TRY(residual_rmsnorm_launch(m->xb, m->y2, m->L[c.n_layers - 1].ffn_norm, d, 1, d, eps,
                                    m->st));
        if (hook_last) TRY(ew_launch(EW_COPY, m->xb, nullptr, hook_last, 0.f, d, m->st));
        h = pro_args(m->lm_head, m->xb, m->logits, PRO_RMSNORM, nullptr, m->final_norm, eps, m->xn);
    }
    const bool fused_choice = mode == 1 && !penalties;
    if (fused_choice) {
        h.epi = EPI_ARGMAX;
        h.arg_part = m->argpart;
    }
    TRY(gemv_launch(h, m->st));
    if (mode == 1) {
        ArgmaxArgs g{};
        g.x = m->logits; g.n = c.vocab; g.part = m->argpart;
        g.out_u32 = m->tok_dev;
        g.suppress = m->g_nsup ? m->suppress_dev : nullptr; g.n_suppress = m->g_nsup;
        g.hist = m->hist; g.hist_len = m->hist_len; g.window = m->g_window; g.theta = m->g_theta;
        g.step = m->step_dev; g.record = 1;
        g.n_parts = fused_choice ? gemv_waves(h) : 0;
        g.pos_inc = m->pos_dev;
        TRY(argmax_launch(g, m->st));
    } else if (mode == 2) {
        TRY(sample_launch(sample_args(m, m->pos_dev), m->st));
    } else {
        TRY(add_int_launch(m->pos_dev, 1, 1, m->st));
    }
    return ATLAS_OK;
}

// mode 0: forward only; mode 1: forward + greedy choice into tok_dev/hist
int enqueue_step(atlas_model* m, int mode, bool long_ctx) {
    if (m->fused) return enqueue_step_fused(m, mode, long_ctx);
    const atlas_model_config& c = m->cfg;
    TRY(embed_launch(m->embed, c.vocab, c.d_model, m->tok_dev, 0, m->x, c.d_model, 1, m->st));
    for (int li = 0; li < c.n_layers; ++li) {
        TRY(layer_step(m, li));
        if (mode == 3)
            TRY(ew_launch(EW_COPY, m->x, nullptr, m->hook_dev + (size_t)li * c.d_model, 0.f,
                          c.d_model, m->st));
    }
    TRY(head_step(m));
    if (mode == 1) TRY(choose_step(m));
    if (mode == 2) TRY(sample_launch(sample_args(m, nullptr), m->st));
    TRY(add_int_launch(m->pos_dev, 1, 1, m->st));
    return ATLAS_OK;
}

void drop_graphs(atlas_model* m) {
    if (m->st) (void)hipStreamSynchronize(m->st);   // no replay of them still running
    for (auto& g : m->gexec)
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    for (auto& g : m->gexec_long)
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    for (auto& g : m->bgexec)
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    for (auto& g : m->bgexec_long)
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    for (auto* arr : {m->pgexec, m->pgexec_long})
        for (int k = 0; k <= kMaxRows; ++k)
            if (arr[k]) {
                (void)hipGraphExecDestroy(arr[k]);
                arr[k] = nullptr;
            }
}

int run_step(atlas_model* m, int mode) {
    ATLAS_REQUIRE(m->pos < m->cfg.max_seq, "position %d reaches max_seq %d", m->pos,
                  m->cfg.max_seq);
    // the host knows the position this step runs at: long contexts replay the
    // long-context step
    const bool long_ctx = m->fused && m->pos >= m->long_from;
    if (!m->use_graph) {
        TRY(enqueue_step(m, mode, long_ctx));
    } else {
        hipGraphExec_t& gx = long_ctx ? m->gexec_long[mode] : m->gexec[mode];
        if (!gx) {
            hipGraph_t g = nullptr;
            ATLAS_HIP(hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal));
            int rc = enqueue_step(m, mode, long_ctx);
            hipError_t e = hipStreamEndCapture(m->st, &g);
            if (rc) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            if (e != hipSuccess) {
                set_error(ATLAS_EHIP, "graph capture: %s", hipGetErrorString(e));
                return ATLAS_EHIP;
            }
            e = hipGraphInstantiate(&gx, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e != hipSuccess) {
                gx = nullptr;
                set_error(ATLAS_EHIP, "graph instantiate: %s", hipGetErrorString(e));
                return ATLAS_EHIP;
            }
        }
        ATLAS_HIP(hipGraphLaunch(gx, m->st));
    }
    m->pos += 1;
    return ATLAS_OK;
}

int set_token(atlas_model* m, uint32_t tok) {
    ATLAS_HIP(hipMemcpyAsync(m->tok_dev, &tok, 4, hipMemcpyHostToDevice, m->st));
    return ATLAS_OK;
}

int sync_pos(atlas_model* m) {
    int p = m->pos;
    ATLAS_HIP(hipMemcpyAsync(m->pos_dev, &p, 4, hipMemcpyHostToDevice, m->st));
    return ATLAS_OK;
}

int download_logits(atlas_model* m, float* host) {
    ATLAS_HIP(hipMemcpyAsync(host, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost,
                             m->st));
    ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}

// the step-0 suppression list on the device (a captured step holds the
// pointer, so growing it drops the graphs)
int upload_suppress(atlas_model* m, const atlas_sampling* s, int nsup) {
    if (nsup > m->suppress_cap) {
        void* p = nullptr;
        TRY(dalloc(m, &p, (size_t)nsup * 4));
        m->suppress_dev = (uint32_t*)p;
        m->suppress_cap = nsup;
        drop_graphs(m);
    }
    if (nsup)
        ATLAS_HIP(hipMemcpyAsync(m->suppress_dev, s->suppress_initial_tokens, (size_t)nsup * 4,
                                 hipMemcpyHostToDevice, m->st));
    return ATLAS_OK;
}

// ---- device sampling: which configurations the sampler kernel takes ----------
// temperature > 0 with 1 <= top_k <= SAMPLE_MAX_K (all of the vocabulary when
// it is smaller) or top_k = 0 with top_p off (the whole vocabulary), at most
// SAMPLE_MAX_HIST generated tokens when the frequency or presence penalty is
// on, and a repetition window of at most SAMPLE_MAX_HIST tokens.  Other
// configurations (top_k = 0 with top_p < 1) sample on the host.
bool sample_dev_ok(const atlas_sampling* s, int V, int max_hist) {
    if (!s || s->temperature <= 0.0f || s->temperature < 1e-6f) return false;
    const bool whole = s->top_k == 0 && !(s->top_p < 1.0f);
    if (!whole && (s->top_k < 1 || s->top_k > SAMPLE_MAX_K || (s->top_k >= V && V > SAMPLE_MAX_K)))
        return false;
    if ((s->frequency_penalty != 0.0f || s->presence_penalty != 0.0f) && max_hist > SAMPLE_MAX_HIST)
        return false;
    if (s->repetition_penalty != 1.0f && std::min(s->repetition_window, max_hist) > SAMPLE_MAX_HIST)
        return false;
    return true;
}

SampleCfg sample_cfg_of(const atlas_sampling* s) {
    SampleCfg c{};
    c.temperature = s->temperature;
    c.theta = s->repetition_penalty;
    c.freq = s->frequency_penalty;
    c.presence = s->presence_penalty;
    c.top_p = s->top_p;
    c.min_p = s->min_p;
    c.log_min_p = s->min_p > 0.0f ? logf(s->min_p) : 0.0f;     // the host's logf, as min_p's
    c.window = s->repetition_window;
    c.top_k = s->top_k;
    c.n_suppress = s->n_suppress > 0 && s->suppress_initial_tokens ? s->n_suppress : 0;
    return c;
}

// settings, suppression list and RNG state of the sampled step (mode 2): the
// captured step reads them from device memory
int set_sample_cfg(atlas_model* m, const atlas_sampling* s) {
    const SampleCfg c = sample_cfg_of(s);
    TRY(upload_suppress(m, s, c.n_suppress));
    ATLAS_HIP(hipMemcpyAsync(m->samp_cfg, &c, sizeof c, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipMemcpyAsync(m->rng_dev, &m->rng.s, 8, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipStreamSynchronize(m->st));     // c and the RNG state live on this frame
    return ATLAS_OK;
}

// ---- greedy settings baked into the graph --------------------------------
int set_greedy_cfg(atlas_model* m, const atlas_sampling* s) {
    float theta = 1.f;
    int window = 0, nsup = 0;
    if (s) {
        theta = s->repetition_penalty;
        window = s->repetition_window;
        nsup = s->n_suppress > 0 && s->suppress_initial_tokens ? s->n_suppress : 0;
    }
    TRY(upload_suppress(m, s, nsup));
    if (theta != m->g_theta || window != m->g_window || nsup != m->g_nsup) {
        m->g_theta = theta;
        m->g_window = window;
        m->g_nsup = nsup;
        for (hipGraphExec_t* g : {&m->gexec[1], &m->gexec_long[1]})
            if (*g) {
                (void)hipGraphExecDestroy(*g);
                *g = nullptr;
            }
    }
    return ATLAS_OK;
}

int reset_state(atlas_model* m) {
    m->pos = 0;
    int zeros[3] = {0, 0, 0};
    TRY(sync_pos(m));
    ATLAS_HIP(hipMemcpyAsync(m->step_dev, zeros, 4, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipMemcpyAsync(m->hist_len, zeros, 4, hipMemcpyHostToDevice, m->st));
    return ATLAS_OK;
}

bool is_stop(const atlas_sampling* s, uint32_t tok) {
    if (!s) return false;
    if (s->eos_token_id >= 0 && (int64_t)tok == s->eos_token_id) return true;
    for (int i = 0; i < s->n_extra_stop; ++i)
        if (s->extra_stop_tokens[i] == tok) return true;
    return false;
}

bool is_greedy(const atlas_sampling* s) {
    return !s || s->temperature <= 0.0f || s->temperature < 1e-6f;
}

// ---- host sampling pipeline (lib.rs:1624-1711, 2581-2722) ---------------------
int host_argmax(const float* x, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i) {
        const float a = x[best], b = x[i];
        const bool greater = !std::isnan(a) && !std::isnan(b) && a > b;
        if (!greater) best = i;
    }
    return n > 0 ? best : 0;
}

void rep_penalty(std::vector<float>& lg, const uint32_t* hist, size_t n_hist, int window,
                 float theta) {
    const size_t start = n_hist > (size_t)window ? n_hist - window : 0;
    for (size_t i = start; i < n_hist; ++i) {
        const uint32_t t = hist[i];
        if (t < lg.size()) {
            if (lg[t] > 0.0f) lg[t] /= theta;
            else lg[t] *= theta;
        }
    }
}

void top_k(std::vector<float>& lg, size_t k) {
    if (k == 0 || k >= lg.size()) return;
    std::vector<float> sorted(lg);
    std::sort(sorted.begin(), sorted.end(), [](float a, float b) { return a > b; });
    const float th = sorted[k - 1];
    size_t at_or_above = 0, above = 0;
    for (float v : lg) {
        if (v >= th) ++at_or_above;
        if (v > th) ++above;
    }
    if (at_or_above <= k) {
        for (float& v : lg)
            if (v < th) v = -INFINITY;
    } else {
        size_t need = k - above, kept = 0;
        for (float& v : lg) {
            if (v > th) continue;
            if (v == th && kept < need) { ++kept; continue; }
            v = -INFINITY;
        }
    }
}

void top_p(std::vector<float>& lg, float p) {
    const size_t n = lg.size();
    if (n == 0) return;
    float mx = -INFINITY;
    for (float v : lg) mx = std::isnan(v) ? mx : std::max(mx, v);
    std::vector<std::pair<size_t, float>> pr(n);
    float sum = 0.f;
    for (size_t i = 0; i < n; ++i) pr[i] = {i, expf(lg[i] - mx)};
    for (auto& e : pr) sum += e.second;
    if (sum <= 0.f) return;
    for (auto& e : pr) e.second /= sum;
    // The running sum goes over the probabilities in descending order (ties in
    // index order, as a stable sort leaves them) until it reaches p.  Only
    // that prefix is ordered: a selection brings the next largest entries to
    // the front, a sort orders them, and the prefix grows 8x until it covers
    // the cut (instead of sorting the whole vocabulary).
    const auto before = [](const std::pair<size_t, float>& a, const std::pair<size_t, float>& b) {
        return a.second > b.second || (a.second == b.second && a.first < b.first);
    };
    float cum = 0.f;
    size_t cut = n, done = 0, k = std::min(n, (size_t)1024);
    while (cut == n && done < n) {
        if (k < n) std::nth_element(pr.begin() + done, pr.begin() + k, pr.end(), before);
        std::sort(pr.begin() + done, pr.begin() + k, before);
        for (size_t i = done; i < k; ++i) {
            cum += pr[i].second;
            if (cum >= p) { cut = i + 1; break; }
        }
        done = k;
        k = std::min(n, k * 8);
    }
    for (size_t i = cut; i < n; ++i) lg[pr[i].first] = -INFINITY;
}

void min_p(std::vector<float>& lg, float mp) {
    if (mp <= 0.f) return;
    float mx = -INFINITY;
    for (float v : lg) mx = std::isnan(v) ? mx : std::max(mx, v);
    const float th = mx + logf(mp);
    for (float& v : lg)
        if (v < th) v = -INFINITY;
}

void softmax_host(std::vector<float>& x) {
    float mx = -INFINITY;
    for (float v : x) mx = std::isnan(v) ? mx : std::max(mx, v);
    float sum = 0.f;
    for (float& v : x) { v = expf(v - mx); sum += v; }
    const float inv = 1.0f / sum;
    for (float& v : x) v *= inv;
}

// One token choice over `logits` given the generated history (lib.rs:1623-1711).
uint32_t choose_token(const float* logits, int V, int step, const uint32_t* hist,
                      size_t n_hist, const atlas_sampling* s, Rng& rng) {
    std::vector<float> lg(logits, logits + V);
    if (s && step == 0)
        for (int i = 0; i < s->n_suppress; ++i)
            if (s->suppress_initial_tokens[i] < (uint32_t)V) lg[s->suppress_initial_tokens[i]] = -INFINITY;
    if (s && s->repetition_penalty != 1.0f && n_hist)
        rep_penalty(lg, hist, n_hist, s->repetition_window, s->repetition_penalty);
    if (is_greedy(s)) return (uint32_t)host_argmax(lg.data(), V);
    if (s->frequency_penalty != 0.0f && n_hist) {
        std::vector<std::pair<uint32_t, size_t>> counts;
        for (size_t j = 0; j < n_hist; ++j) {
            const uint32_t t = hist[j];
            auto it = std::find_if(counts.begin(), counts.end(),
                                   [t](const auto& e) { return e.first == t; });
            if (it != counts.end()) ++it->second;
            else counts.push_back({t, 1});
        }
        for (auto& e : counts)
            if (e.first < (uint32_t)V) lg[e.first] -= s->frequency_penalty * (float)e.second;
    }
    if (s->presence_penalty != 0.0f && n_hist) {
        std::vector<uint32_t> seen(hist, hist + n_hist);
        std::sort(seen.begin(), seen.end());
        seen.erase(std::unique(seen.begin(), seen.end()), seen.end());
        for (uint32_t t : seen)
            if (t < (uint32_t)V) lg[t] -= s->presence_penalty;
    }
    for (float& v : lg) v /= s->temperature;
    if (s->top_k > 0) top_k(lg, (size_t)s->top_k);
    if (s->top_p < 1.0f) top_p(lg, s->top_p);
    if (s->min_p > 0.0f) min_p(lg, s->min_p);
    softmax_host(lg);
    const float r = rng.next_f32();
    float cum = 0.f;
    for (int i = 0; i < V; ++i) {
        cum += lg[i];
        if (r < cum) return (uint32_t)i;
    }
    return (uint32_t)(V - 1);
}

uint32_t host_choose(atlas_model* m, const float* logits, int step,
                     const std::vector<uint32_t>& hist, const atlas_sampling* s) {
    return choose_token(logits, m->cfg.vocab, step, hist.data(), hist.size(), s, m->rng);
}

void seed_rng(atlas_model* m, const atlas_sampling* s) {
    if (s && s->rng_seed) {
        m->rng.s = s->rng_seed | 1ULL;
    } else {
        const uint64_t t = (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                               std::chrono::system_clock::now().time_since_epoch())
                               .count();
        m->rng.s = t ^ 0x517cc1b727220a95ULL;
    }
}

// ---- tensor placement ---------------------------------------------------------
// dst row r of the fused matrix <- src row r of the single matrix; the fused
// row index is base + r * stride (stride 2 interleaves gate/up).
int place_rows(atlas_model* m, DevMat& dst, int base, int stride, int rows, const void* data,
               const float* scales, bool upload) {
    const size_t rb = dst.row_bytes(), rp = dst.row_pitch();
    const size_t spr = dst.scales_per_row();
    const hipMemcpyKind kind = upload ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
    char* dptr = (char*)dst.w + (size_t)base * rp;
    if (upload)
        ATLAS_HIP(hipMemcpy2DAsync(dptr, rp * stride, data, rb, rb, rows, kind, m->st));
    else
        ATLAS_HIP(hipMemcpy2DAsync((void*)data, rb, dptr, rp * stride, rb, rows, kind, m->st));
    if (spr) {
        ATLAS_REQUIRE(scales, "tensor needs scales for format %d", dst.fmt);
        float* sptr = dst.scales + (size_t)base * spr;
        if (upload)
            ATLAS_HIP(hipMemcpy2DAsync(sptr, spr * 4 * stride, scales, spr * 4, spr * 4, rows, kind,
                                       m->st));
        else
            ATLAS_HIP(hipMemcpy2DAsync((void*)scales, spr * 4, sptr, spr * 4 * stride, spr * 4, rows,
                                       kind, m->st));
    }
    ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}

int tensor_io(atlas_model* m, int kind, int layer, void* data, float* scales, bool upload) {
    const atlas_model_config& c = m->cfg;
    const int d = c.d_model;
    auto vec_io = [&](float* dev, size_t n) -> int {
        ATLAS_REQUIRE(dev, "tensor kind %d is not present in this model", kind);
        if (upload) ATLAS_HIP(hipMemcpyAsync(dev, data, n * 4, hipMemcpyHostToDevice, m->st));
        else ATLAS_HIP(hipMemcpyAsync(data, dev, n * 4, hipMemcpyDeviceToHost, m->st));
        ATLAS_HIP(hipStreamSynchronize(m->st));
        return ATLAS_OK;
    };
    if (kind == ATLAS_T_EMBED) {
        const size_t bytes = (size_t)c.vocab * d * 2;
        if (upload) ATLAS_HIP(hipMemcpyAsync(m->embed, data, bytes, hipMemcpyHostToDevice, m->st));
        else ATLAS_HIP(hipMemcpyAsync(data, m->embed, bytes, hipMemcpyDeviceToHost, m->st));
        ATLAS_HIP(hipStreamSynchronize(m->st));
        return ATLAS_OK;
    }
    if (kind == ATLAS_T_LM_HEAD)
        return place_rows(m, m->lm_head, 0, 1, c.vocab, data, scales, upload);
    if (kind == ATLAS_T_FINAL_NORM) return vec_io(m->final_norm, d);
    ATLAS_REQUIRE(layer >= 0 && layer < c.n_layers, "layer %d out of range", layer);
    LayerW& L = m->L[layer];
    switch (kind) {
    case ATLAS_T_WQ: return place_rows(m, L.qkv, 0, 1, d, data, scales, upload);
    case ATLAS_T_WK: return place_rows(m, L.qkv, d, 1, m->kvd, data, scales, upload);
    case ATLAS_T_WV: return place_rows(m, L.qkv, d + m->kvd, 1, m->kvd, data, scales, upload);
    case ATLAS_T_WO: return place_rows(m, L.wo, 0, 1, d, data, scales, upload);
    case ATLAS_T_W_GATE: return place_rows(m, L.gu, 0, 2, c.ffn_hidden, data, scales, upload);
    case ATLAS_T_W_UP: return place_rows(m, L.gu, 1, 2, c.ffn_hidden, data, scales, upload);
    case ATLAS_T_W_DOWN: return place_rows(m, L.down, 0, 1, d, data, scales, upload);
    case ATLAS_T_ATTN_NORM: return vec_io(L.attn_norm, d);
    case ATLAS_T_FFN_NORM: return vec_io(L.ffn_norm, d);
    case ATLAS_T_Q_NORM: return vec_io(L.q_norm, (size_t)c.n_heads * m->hd);
    case ATLAS_T_K_NORM: return vec_io(L.k_norm, (size_t)m->kvd);
    }
    set_error(ATLAS_EINVAL, "unknown tensor kind %d", kind);
    return ATLAS_EINVAL;
}

// ---- tensors from device memory (the safetensors loader) ---------------------
// Where a tensor kind lives: rows [base, base + rows * stride) step stride of a
// matrix, a float vector, or the bf16 embedding.
struct TensorTarget {
    DevMat* mat = nullptr;
    int base = 0, stride = 1, rows = 0;
    float* vec = nullptr;
    size_t n = 0;                  // elements of the tensor
    bool embed = false;
};

int tensor_target(atlas_model* m, int kind, int layer, TensorTarget& t) {
    const atlas_model_config& c = m->cfg;
    const int d = c.d_model;
    auto mat = [&](DevMat& w, int base, int stride, int rows) {
        t.mat = &w; t.base = base; t.stride = stride; t.rows = rows;
        t.n = (size_t)rows * w.cols;
        return ATLAS_OK;
    };
    auto vec = [&](float* v, size_t n) {
        ATLAS_REQUIRE(v, "tensor kind %d is not present in this model", kind);
        t.vec = v; t.n = n;
        return ATLAS_OK;
    };
    switch (kind) {
    case ATLAS_T_EMBED: t.embed = true; t.n = (size_t)c.vocab * d; return ATLAS_OK;
    case ATLAS_T_LM_HEAD: return mat(m->lm_head, 0, 1, c.vocab);
    case ATLAS_T_FINAL_NORM: return vec(m->final_norm, d);
    }
    ATLAS_REQUIRE(layer >= 0 && layer < c.n_layers, "layer %d out of range", layer);
    LayerW& L = m->L[layer];
    switch (kind) {
    case ATLAS_T_WQ: return mat(L.qkv, 0, 1, d);
    case ATLAS_T_WK: return mat(L.qkv, d, 1, m->kvd);
    case ATLAS_T_WV: return mat(L.qkv, d + m->kvd, 1, m->kvd);
    case ATLAS_T_WO: return mat(L.wo, 0, 1, d);
    case ATLAS_T_W_GATE: return mat(L.gu, 0, 2, c.ffn_hidden);
    case ATLAS_T_W_UP: return mat(L.gu, 1, 2, c.ffn_hidden);
    case ATLAS_T_W_DOWN: return mat(L.down, 0, 1, d);
    case ATLAS_T_ATTN_NORM: return vec(L.attn_norm, d);
    case ATLAS_T_FFN_NORM: return vec(L.ffn_norm, d);
    case ATLAS_T_Q_NORM: return vec(L.q_norm, (size_t)c.n_heads * m->hd);
    case ATLAS_T_K_NORM: return vec(L.k_norm, (size_t)m->kvd);
    }
    set_error(ATLAS_EINVAL, "unknown tensor kind %d", kind);
    return ATLAS_EINVAL;
}

}  // namespace

// Device temporaries of set_tensor_dev, grown on demand.
struct atlas_load_scratch {
    void* conv = nullptr;          // bf16 conversion of an f32 matrix
    void* qdata = nullptr;         // quantised rows
    float* qscales = nullptr;
    size_t conv_bytes = 0, qdata_bytes = 0, qscale_bytes = 0;
};

namespace {

int grow(void** p, size_t* have, size_t need) {
    if (need <= *have) return ATLAS_OK;
    if (*p) {
        ATLAS_HIP(hipDeviceSynchronize());
        ATLAS_HIP(hipFree(*p));
        *p = nullptr;
        *have = 0;
    }
    if (dev_malloc(p, need) != hipSuccess) {
        (void)hipGetLastError();
        *p = nullptr;
        set_error(ATLAS_ENOMEM, "load scratch: %zu bytes", need);
        return ATLAS_ENOMEM;
    }
    *have = need;
    return ATLAS_OK;
}

// Converts a device tensor (f32 or bf16 elements) into the model's format and
// layout, on the model's stream, without waiting for it.
int set_tensor_dev(atlas_model* m, int kind, int layer, const void* src, int src_dtype, size_t n,
                   atlas_load_scratch& s) {
    ATLAS_REQUIRE(src, "set_tensor_dev: null source");
    ATLAS_REQUIRE(src_dtype == WF_F32 || src_dtype == WF_BF16,
                  "set_tensor_dev: source dtype %d (f32 or bf16)", src_dtype);
    TensorTarget t;
    TRY(tensor_target(m, kind, layer, t));
    ATLAS_REQUIRE(n == t.n, "set_tensor_dev: tensor kind %d has %zu elements, expected %zu", kind, n,
                  t.n);
    const bool bf16 = src_dtype == WF_BF16;
    if (t.vec) {
        if (bf16) return cvt_launch(CVT_BF16_F32, src, t.vec, (long)n, m->st);
        ATLAS_HIP(hipMemcpyAsync(t.vec, src, n * 4, hipMemcpyDeviceToDevice, m->st));
        return ATLAS_OK;
    }
    if (t.embed) {
        if (!bf16) return cvt_launch(CVT_F32_BF16, src, m->embed, (long)n, m->st);
        ATLAS_HIP(hipMemcpyAsync(m->embed, src, n * 2, hipMemcpyDeviceToDevice, m->st));
        return ATLAS_OK;
    }
    DevMat& w = *t.mat;
    const size_t rb = w.row_bytes(), rp = w.row_pitch(), spr = w.scales_per_row();
    char* dst = (char*)w.w + (size_t)t.base * rp;
    const void* rows_src = src;
    if (w.fmt == WF_BF16) {
        if (!bf16) {
            TRY(grow(&s.conv, &s.conv_bytes, n * 2));
            TRY(cvt_launch(CVT_F32_BF16, src, s.conv, (long)n, m->st));
            rows_src = s.conv;
        }
    } else {
        TRY(grow(&s.qdata, &s.qdata_bytes, rb * t.rows));
        TRY(grow((void**)&s.qscales, &s.qscale_bytes, spr * t.rows * 4));
        if (w.fmt == WF_I8)
            TRY(quant_i8_launch(src, bf16, t.rows, w.cols, (int8_t*)s.qdata, s.qscales, m->st));
        else
            TRY(quant_i4_launch(src, bf16, (long)n, w.block, (uint8_t*)s.qdata, s.qscales, m->st));
        rows_src = s.qdata;
        ATLAS_HIP(hipMemcpy2DAsync(w.scales + (size_t)t.base * spr, spr * 4 * t.stride, s.qscales,
                                   spr * 4, spr * 4, t.rows, hipMemcpyDeviceToDevice, m->st));
    }
    ATLAS_HIP(hipMemcpy2DAsync(dst, rp * t.stride, rows_src, rb, rb, t.rows, hipMemcpyDeviceToDevice,
                               m->st));
    return ATLAS_OK;
}

// ---- the ragged batch step ----------------------------------------------------
// n rows of activations through w: the batch-1 GEMV for one row, the skinny
// launcher for 2..16 (the multi-row GEMV for 2-3 rows, MFMA tiles above)
int bmm(atlas_model* m, const DevMat& w, const float* x, float* y, int n, int epi) {
    if (n == 1) return gemv(m, w, x, y, epi);
    return skinny(m, w, x, y, n, epi);
}

// y = w . x rows, then x += rmsnorm(y) * norm_w: where the GEMM splits K
// (the 2-8-row direct-load kernels), the norm sums its partials itself and
// the split-K reduce launch goes away (same y bit for bit)
int bmm_resnorm(atlas_model* m, const DevMat& w, const float* x, float* y, int n,
                const float* norm_w) {
    const atlas_model_config& c = m->cfg;
    int splits = 0;
    const bool fold = n > 1 && c.d_model <= 8192;
    if (!fold) TRY(bmm(m, w, x, y, n, EPI_STORE));
    else TRY(skinny(m, w, x, y, n, EPI_STORE, &splits));
    if (splits > 8) {
        // more partials than the folded norm unrolls: sum them as the reduce does
        GemvArgs a = gemv_args(w, x, y, EPI_STORE);
        a.N = n;
        a.y_stride_n = w.rows;
        a.y_stride_m = 1;
        TRY(skinny_reduce_launch(a, m->gemm_part, splits, m->st));
        splits = 0;
    }
    if (splits > 0)
        return residual_rmsnorm_parts_launch(m->x, m->gemm_part, splits, norm_w, c.d_model, n,
                                             c.d_model, c.rms_eps, m->st);
    return residual_rmsnorm_launch(m->x, y, norm_w, c.d_model, n, c.d_model, c.rms_eps, m->st);
}

// The hipBLASLt prompt GEMMs are used only when the environment sets
// ATLAS_PROMPT_BLAS=1 at model creation.
bool prompt_blas_opt_in() {
    const char* e = std::getenv("ATLAS_PROMPT_BLAS");
    return e && std::strcmp(e, "1") == 0;
}

// A prompt chunk of 17..1024 rows whose four GEMMs per layer all take the
// hipBLASLt path (post-norm): their activation split and product combine then
// live in the neighbouring kernels where those see whole rows -- the split of
// x in the residual RMSNorm that produces it (and once after the embedding),
// the QKV combine in qkv_post, the W_o / W_down combine in the residual
// RMSNorm that consumes it; for bf16 also the attention output's split in the
// prompt attention and the gate/up combine with its SwiGLU in one kernel that
// writes the W_down input split (int8 digits need a whole row's maximum, so
// those two keep their own split).  Same values as the separate kernels:
// every sum, product and rounding is the same.  Returns the weight format
// (WF_BF16 or WF_I8), or 0 when the chunk takes the unfused path.
int blas_chunk(atlas_model* m, int n) {
    if (!m->blas || !m->fused || !m->cfg.post_norm || n <= 16 || n > blas_rows_max_n(m->blas))
        return 0;
    const int fmt = m->L[0].qkv.fmt;
    if (fmt != WF_BF16 && fmt != WF_I8) return 0;
    for (const LayerW& L : m->L)
        for (const DevMat* w : {&L.qkv, &L.wo, &L.gu, &L.down}) {
            GemvArgs a = gemv_args(*w, m->x, m->y, w == &L.gu ? EPI_SILU_MUL : EPI_STORE);
            a.N = n;
            a.x_stride_n = w->cols;
            a.x_stride_k = 1;
            if (w->fmt != fmt || !gemm_rows_ok(a) || (fmt == WF_I8 && w->cols > kDigitsMaxK))
                return 0;
        }
    const bool ok = m->L[0].qkv.rows == m->qkv_rows && m->L[0].wo.rows == m->cfg.d_model &&
                    m->L[0].down.rows == m->cfg.d_model && m->L[0].gu.rows % 4 == 0 &&
                    m->cfg.d_model % 8 == 0 && (fmt != WF_I8 || m->cfg.d_model <= 8192);
    return ok ? fmt : 0;
}

// the library GEMM of w against the split rows in the context's staging rows
int blas_gemm(atlas_model* m, const DevMat& w, int n) {
    GemvArgs a = gemv_args(w, nullptr, nullptr, EPI_STORE);
    a.N = n;
    return blas_rows_gemm(m->blas, a, n, m->st);
}

// prompt_chunk = true: the n rows are ONE sequence's prompt tokens at
// consecutive positions pos_dev[0] .. + n - 1, all in slot slots[0] (only
// prefill_rows sets it); the step then skips the final norm, lm_head and
// choice, and its attention may take the query-tiled prompt kernel, which
// relies on exactly that layout.  Ragged rows (any other caller) pass false.
int batch_step(atlas_model* m, int n, const std::vector<int>& slots, bool long_ctx,
               bool prompt_chunk = false) {
    const atlas_model_config& c = m->cfg;
    const bool with_head = !prompt_chunk;
    const int d = c.d_model;
    const int bfmt = prompt_chunk && long_ctx ? blas_chunk(m, n) : 0;
    const bool bc = bfmt != 0, b8 = bfmt == WF_I8;
    uint16_t* xs = bc ? blas_rows_xs(m->blas) : nullptr;      // split GEMM input rows
    int8_t* xd = (int8_t*)xs;                                 // (int8: digit rows)
    float* xsc = bc ? blas_rows_xscale(m->blas) : nullptr;    // (int8: their row scales)
    float* dd = bc ? blas_rows_d(m->blas) : nullptr;          // product rows
    TRY(embed_launch(m->embed, c.vocab, d, m->tok_dev, 0, m->x, d, n, m->st));
    if (bc && b8) TRY(digits_rows_launch(m->x, d, n, d, xd, xsc, m->st));
    else if (bc) TRY(split_rows_launch(m->x, d, n, d, xs, m->st));
    for (int li = 0; li < c.n_layers; ++li) {
        LayerW& L = m->L[li];
        const float* xin = m->x;
        if (!c.post_norm) {
            TRY(rmsnorm_launch(m->x, L.attn_norm, m->xn, d, n, d, c.rms_eps, m->st));
            xin = m->xn;
        }
        // the separate-kernel path (long contexts) lets qkv_post sum the
        // QKV GEMM's split-K partials in place of the reduce launch
        int qkv_splits = 0;
        if (bc) TRY(blas_gemm(m, L.qkv, n));
        else if (m->fused && long_ctx && n > 1) TRY(skinny(m, L.qkv, xin, m->qkv, n, EPI_STORE, &qkv_splits));
        else TRY(bmm(m, L.qkv, xin, m->qkv, n, EPI_STORE));
        QkvPostArgs q{};
        if (qkv_splits > 0) {
            q.src_parts = m->gemm_part;
            q.src_splits = qkv_splits;
            q.src_stride = L.qkv.rows;
            q.src_lo = (long)n * L.qkv.rows;
        }
        if (bc) {
            if (b8) {
                q.src_d = (const int*)dd;
                q.src_ws = L.qkv.scales;
                q.src_xs = xsc;
            } else {
                q.src = dd;
            }
            q.src_stride = L.qkv.rows;
            q.src_lo = (long)n * L.qkv.rows;
        }
        q.qkv = m->qkv; q.qkv_stride = m->qkv_rows;
        q.q_norm = L.q_norm; q.k_norm = L.k_norm; q.qk_eps = 1e-6f;
        q.cos_tab = m->cos_tab; q.sin_tab = m->sin_tab;
        q.k_cache = L.kc; q.v_cache = L.vc; q.slot_stride = m->slot_stride;
        q.slot_dev = m->slot_dev; q.pos_dev = m->pos_dev;
        q.n_heads = c.n_heads; q.n_kv = c.n_kv_heads; q.head_dim = m->hd;
        if (m->fused && long_ctx) {
            // long contexts: QK-norm/RoPE/KV write, then the split kernel over
            // (KV head, split, sequence) and the split merge as a second
            // kernel (no per-block device-scope fence)
            TRY(qkv_post_launch(q, n, m->st));
            AttnArgs a{};
            a.q = m->qkv; a.q_stride = m->qkv_rows;
            a.k_cache = L.kc; a.v_cache = L.vc;
            a.slot_dev = m->slot_dev; a.slot_stride = m->slot_stride;
            a.pos_dev = m->pos_dev;
            a.out = m->att; a.out_stride = d;
            a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = m->hd;
            a.scale = m->scale; a.window = L.window; a.max_rows = c.max_seq;
            a.adaptive = 1;
            const int sp = n <= kMaxRows ? m->attn_splits_batch[n]
                                         : attn_batch_splits_for(c.n_kv_heads, n, c.max_seq);
            const size_t np = (size_t)n * c.n_heads * sp;
            a.part_m = m->attn_part; a.part_l = m->attn_part + np; a.part_o = m->attn_part + 2 * np;
            // a prompt chunk (one sequence, consecutive positions, one slot):
            // 16 rows share each K/V tile
            if (prompt_chunk && attn_prefill_ok(a)) {
                if (bc && !b8) {
                    a.out_split = xs;       // the W_o input rows, split
                    a.split_lo = (long)n * d;
                }
                TRY(attn_prefill_launch(a, n, m->st));
                if (b8) TRY(digits_rows_launch(m->att, d, n, d, xd, xsc, m->st));
            } else {
                TRY(attn_batch_launch(a, sp, n, m->st));
                if (b8) TRY(digits_rows_launch(m->att, d, n, d, xd, xsc, m->st));
                else if (bc) TRY(split_rows_launch(m->att, d, n, d, xs, m->st));
            }
        } else if (m->fused) {
            // one launch: every sequence's QK-norm/RoPE/KV write and attention
            AttnFusedArgs a{};
            a.qkv = m->qkv; a.qkv_stride = m->qkv_rows;
            a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.qk_eps = 1e-6f;
            a.cos_tab = m->cos_tab; a.sin_tab = m->sin_tab;
            a.k_cache = L.kc; a.v_cache = L.vc; a.slot_stride = m->slot_stride;
            a.slot_dev = m->slot_dev; a.pos_dev = m->pos_dev;
            a.out = m->att; a.out_stride = d;
            a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = m->hd;
            a.scale = m->scale; a.window = L.window;
            a.part_m = m->attn_part;
            a.part_l = m->attn_part + (size_t)m->RF * c.n_heads * m->attn_splits;
            a.part_o = m->attn_part + (size_t)2 * m->RF * c.n_heads * m->attn_splits;
            a.counters = m->attn_counters;
            a.adaptive = 1; a.max_rows = c.max_seq;
            TRY(attn_fused_launch(a, m->attn_splits, n, m->st));
        }
        if (!m->fused) TRY(qkv_post_launch(q, n, m->st));
        for (int i = 0; i < n && !m->fused; ++i) {
            AttnArgs a{};
            a.q = m->qkv + (size_t)i * m->qkv_rows;
            a.k_cache = L.kc + (size_t)slots[i] * m->slot_stride;
            a.v_cache = L.vc + (size_t)slots[i] * m->slot_stride;
            a.out = m->att + (size_t)i * d;
            a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.head_dim = m->hd;
            a.pos_dev = m->pos_dev + i; a.scale = m->scale; a.window = L.window;
            a.max_rows = c.max_seq;
            const size_t np = (size_t)c.n_heads * m->attn_splits_unfused;
            a.part_m = m->attn_part; a.part_l = m->attn_part + np; a.part_o = m->attn_part + 2 * np;
            TRY(attn_launch(a, m->attn_splits_unfused, m->st));
        }
        if (bc && b8) {
            const int h = L.gu.rows / 2;
            TRY(blas_gemm(m, L.wo, n));
            TRY(residual_rmsnorm_digits_launch(m->x, (const int*)dd, L.wo.scales, xsc, L.attn_norm, d,
                                               n, d, c.rms_eps, xd, m->st));
            TRY(blas_gemm(m, L.gu, n));
            TRY(combine_digits_launch((const int*)dd, n, L.gu.rows, L.gu.scales, xsc, EPI_SILU_MUL,
                                      m->h, h, 1, m->st));
            TRY(digits_rows_launch(m->h, h, n, h, xd, xsc, m->st));
            TRY(blas_gemm(m, L.down, n));
            TRY(residual_rmsnorm_digits_launch(m->x, (const int*)dd, L.down.scales, xsc, L.ffn_norm,
                                               d, n, d, c.rms_eps,
                                               li + 1 < c.n_layers ? xd : nullptr, m->st));
            continue;
        }
        if (bc) {
            TRY(blas_gemm(m, L.wo, n));
            TRY(residual_rmsnorm_rows_launch(m->x, dd, (long)n * d, L.attn_norm, d, n, d, c.rms_eps,
                                             xs, m->st));
            TRY(blas_gemm(m, L.gu, n));
            TRY(combine_split_launch(dd, n, L.gu.rows, xs, m->st));
            TRY(blas_gemm(m, L.down, n));
            TRY(residual_rmsnorm_rows_launch(m->x, dd, (long)n * d, L.ffn_norm, d, n, d, c.rms_eps,
                                             li + 1 < c.n_layers ? xs : nullptr, m->st));
            continue;
        }
        if (c.post_norm) {
            TRY(bmm_resnorm(m, L.wo, m->att, m->y, n, L.attn_norm));
            TRY(bmm(m, L.gu, m->x, m->h, n, EPI_SILU_MUL));
            TRY(bmm_resnorm(m, L.down, m->h, m->y, n, L.ffn_norm));
        } else {
            TRY(bmm(m, L.wo, m->att, m->y, n, EPI_STORE));
            TRY(ew_launch(EW_ADD, m->x, m->y, m->x, 0.f, (long)n * d, m->st));
            TRY(rmsnorm_launch(m->x, L.ffn_norm, m->xn, d, n, d, c.rms_eps, m->st));
            TRY(bmm(m, L.gu, m->xn, m->h, n, EPI_SILU_MUL));
            TRY(bmm(m, L.down, m->h, m->y, n, EPI_STORE));
            TRY(ew_launch(EW_ADD, m->x, m->y, m->x, 0.f, (long)n * d, m->st));
        }
    }
    if (!with_head) return ATLAS_OK;
    TRY(rmsnorm_launch(m->x, m->final_norm, m->xn, d, n, d, c.rms_eps, m->st));
    TRY(bmm(m, m->lm_head, m->xn, m->logits, n, EPI_STORE));
    // greedy choice of every row into choice_dev (last maximum wins): one
    // launch pair for all rows while their partial keys fit, else per row
    const int parts = std::min(512, (c.vocab + 255) / 256);
    if ((long)parts * n <= ARGMAX_MAX_PARTS)
        return argmax_rows_launch(m->logits, c.vocab, c.vocab, n, m->argpart, m->choice_dev, m->st);
    for (int j = 0; j < n; ++j) {
        ArgmaxArgs g{};
        g.x = m->logits + (size_t)j * c.vocab; g.n = c.vocab; g.part = m->argpart;
        g.out_u32 = m->choice_dev + j; g.theta = 1.0f;
        TRY(argmax_launch(g, m->st));
    }
    return ATLAS_OK;
}

// batch_step replayed from a graph captured per batch size and attention
// variant (fused models: tokens, positions and slots are read from device
// memory); long_ctx picks the long-context variant
int run_batch_step(atlas_model* m, int n, const std::vector<int>& slots, bool long_ctx,
                   bool prompt_chunk = false) {
    long_ctx = long_ctx && m->fused;
    const bool with_head = !prompt_chunk;
    if (!m->use_graph || !m->fused) return batch_step(m, n, slots, long_ctx, prompt_chunk);
    hipGraphExec_t& ge = with_head ? (long_ctx ? m->bgexec_long[n] : m->bgexec[n])
                                   : (long_ctx ? m->pgexec_long[n] : m->pgexec[n]);
    if (!ge) {
        hipGraph_t g = nullptr;
        ATLAS_HIP(hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal));
        int rc = batch_step(m, n, slots, long_ctx, prompt_chunk);
        hipError_t e = hipStreamEndCapture(m->st, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) {
            set_error(ATLAS_EHIP, "graph capture: %s", hipGetErrorString(e));
            return ATLAS_EHIP;
        }
        e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            ge = nullptr;
            set_error(ATLAS_EHIP, "graph instantiate: %s", hipGetErrorString(e));
            return ATLAS_EHIP;
        }
    }
    ATLAS_HIP(hipGraphLaunch(ge, m->st));
    return ATLAS_OK;
}

// Prompt tokens through the multi-row step, up to prefill_chunk at a time, at
// the single sequence's positions m->pos.. in KV slot 0 (fused models; others
// and lone tokens take the decode step).  Always the step's two-kernel
// attention variant: its QK-norm / RoPE / KV-write kernel stores every row's K
// and V before the split kernel's row j reads cache rows up to m->pos + j.
// (The fused attention kernel writes a row's K/V in the same launch that
// other rows read; the rows of a ragged batch live in different slots, the
// rows of a prefill chunk in one.)
// k >= 2 prompt tokens of the sequence in KV slot `slot` at positions
// pos0 .. pos0 + k - 1, as one multi-row step without the lm_head
// the most prompt rows one step of this model takes
int prefill_cap(const atlas_model* m) {
    if (!m->fused) return 1;
    if (!m->big_prefill) return std::min(m->R, kPrefillChunk);
    return std::min(m->R, kPrefillLib);
}

int prefill_rows(atlas_model* m, int slot, int pos0, const uint32_t* toks, int k) {
    ATLAS_REQUIRE(k >= 2 && k <= prefill_cap(m), "prefill: %d rows", k);
    ATLAS_REQUIRE(pos0 + k <= m->cfg.max_seq, "prefill: position %d + %d exceeds max_seq %d", pos0,
                  k, m->cfg.max_seq);
    static_assert(kPrefillLib >= kPrefillBig, "row caps");
    int host[3][kPrefillLib];
    for (int j = 0; j < k; ++j) {
        host[0][j] = (int)toks[j];
        host[1][j] = pos0 + j;
        host[2][j] = slot;
    }
    ATLAS_HIP(hipMemcpyAsync(m->tok_dev, host[0], (size_t)k * 4, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipMemcpyAsync(m->pos_dev, host[1], (size_t)k * 4, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipMemcpyAsync(m->slot_dev, host[2], (size_t)k * 4, hipMemcpyHostToDevice, m->st));
    // chunks beyond the captured row counts run eagerly: ~260 launches
    // queue while the first GEMMs run
    if (k > kMaxRows) TRY(batch_step(m, k, std::vector<int>(k, slot), true, /*prompt_chunk=*/true));
    else TRY(run_batch_step(m, k, std::vector<int>(k, slot), true, /*prompt_chunk=*/true));
    ATLAS_HIP(hipStreamSynchronize(m->st));      // host[] lives on this frame
    return ATLAS_OK;
}

int prefill(atlas_model* m, const uint32_t* toks, int n) {
    const int chunk = std::min(m->prefill_chunk, prefill_cap(m));
    int done = 0;
    while (done < n) {
        const int k = std::min(chunk, n - done);
        ATLAS_REQUIRE(m->pos + k <= m->cfg.max_seq, "prefill: position %d + %d exceeds max_seq %d",
                      m->pos, k, m->cfg.max_seq);
        if (k == 1) {
            TRY(sync_pos(m));
            TRY(set_token(m, toks[done]));
            TRY(run_step(m, 0));
            ++done;
            continue;
        }
        TRY(prefill_rows(m, 0, m->pos, toks + done, k));
        m->pos += k;
        done += k;
    }
    return sync_pos(m);                               // pos_dev[0] for the decode step
}

}  // namespace

// =============================================================================
// C ABI
// =============================================================================

ATLAS_API atlas_model* atlas_model_create(const atlas_model_config* cfg) {
    if (!cfg) {
        set_error(ATLAS_EINVAL, "atlas_model_create: null config");
        return nullptr;
    }
    const atlas_model_config& c = *cfg;
    if (c.vocab <= 0 || c.d_model <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 ||
        c.ffn_hidden <= 0 || c.max_seq <= 0 || c.d_model % c.n_heads || c.n_heads % c.n_kv_heads) {
        set_error(ATLAS_EINVAL, "atlas_model_create: inconsistent shape");
        return nullptr;
    }
    const int fmt = c.weight_format;
    if (fmt != WF_BF16 && fmt != WF_I8 && fmt != WF_I4) {
        set_error(ATLAS_EINVAL, "atlas_model_create: weight_format %d", fmt);
        return nullptr;
    }
    const int hd = c.d_model / c.n_heads;
    if (hd % 2 || hd > 256) {
        set_error(ATLAS_EINVAL, "atlas_model_create: head_dim %d", hd);
        return nullptr;
    }
    if (fmt == WF_I4 && (c.int4_block <= 0 || c.int4_block % 32 || c.d_model % c.int4_block ||
                         c.ffn_hidden % c.int4_block)) {
        set_error(ATLAS_EINVAL, "atlas_model_create: int4 block %d must be a multiple of 32 "
                  "dividing d_model and ffn_hidden", c.int4_block);
        return nullptr;
    }
    atlas_model* m = new atlas_model();
    m->cfg = c;
    m->sliding.assign(c.n_layers, 0);
    if (c.layer_sliding) std::memcpy(m->sliding.data(), c.layer_sliding, c.n_layers);
    m->cfg.layer_sliding = m->sliding.data();
    m->hd = hd;
    m->kvd = c.n_kv_heads * hd;
    m->qkv_rows = c.d_model + 2 * m->kvd;
    m->B = c.max_batch < 1 ? 1 : c.max_batch;
    // big prompt chunks: the fused (post-norm) step, every GEMM inner
    // dimension (d_model, n_heads * head_dim, ffn_hidden) a multiple of the
    // tiled GEMM's 128, and int4 blocks of 32 * 2^j
    const int i4_cpb = fmt == WF_I4 && c.int4_block > 0 ? c.int4_block / 32 : 1;
    m->big_prefill = (i4_cpb & (i4_cpb - 1)) == 0 && c.post_norm &&
                     attn_fused_supported(c.n_heads, c.n_kv_heads, hd) &&
                     attn_rows_fit(c.max_seq, c.n_kv_heads, hd) && c.d_model % 128 == 0 &&
                     (c.n_heads * hd) % 128 == 0 && c.ffn_hidden % 128 == 0;
    m->RF = std::max(m->B, m->big_prefill ? kPrefillBig : kPrefillChunk);
    // prompt chunks take up to kPrefillLib rows
    m->R = std::max(m->RF, m->big_prefill ? kPrefillLib : 0);
    // scale = attn_factor / sqrt(head_dim) (lib.rs:632, 1331-1335)
    m->scale = 1.0f / sqrtf((float)hd);
    const float af = c.yarn ? c.yarn_attn_factor : 1.0f;
    if (fabsf(af - 1.0f) > 1e-6f) m->scale *= af;

    auto fail = [&](atlas_model* mm) -> atlas_model* {
        atlas_model_destroy(mm);
        return nullptr;
    };
    if (hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking) != hipSuccess) {
        set_error(ATLAS_EHIP, "atlas_model_create: stream creation failed");
        m->st = nullptr;
        return fail(m);
    }
    const int d = c.d_model, B = m->B, blk = c.int4_block;
    m->slot_stride = (long)c.max_seq * m->kvd;
    m->L.resize(c.n_layers);
    for (int li = 0; li < c.n_layers; ++li) {
        LayerW& L = m->L[li];
        if (alloc_mat(m, L.qkv, fmt, m->qkv_rows, d, blk) || alloc_mat(m, L.wo, fmt, d, d, blk) ||
            alloc_mat(m, L.gu, fmt, 2 * c.ffn_hidden, d, blk) ||
            alloc_mat(m, L.down, fmt, d, c.ffn_hidden, blk) ||
            dalloc(m, (void**)&L.attn_norm, (size_t)d * 4) ||
            dalloc(m, (void**)&L.ffn_norm, (size_t)d * 4) ||
            dalloc(m, (void**)&L.kc, (size_t)B * m->slot_stride * 4) ||
            dalloc(m, (void**)&L.vc, (size_t)B * m->slot_stride * 4))
            return fail(m);
        if (c.qk_norm && (dalloc(m, (void**)&L.q_norm, (size_t)c.n_heads * hd * 4) ||
                          dalloc(m, (void**)&L.k_norm, (size_t)m->kvd * 4)))
            return fail(m);
        L.window = (m->sliding[li] && c.sliding_window > 0) ? c.sliding_window : 0;
    }
    if (dalloc(m, (void**)&m->embed, (size_t)c.vocab * d * 2) ||
        alloc_mat(m, m->lm_head, fmt, c.vocab, d, blk) ||
        dalloc(m, (void**)&m->final_norm, (size_t)d * 4))
        return fail(m);
    // scratch
    // activations of up to R rows (a ragged batch or a prefill chunk)
    const int big = std::max(c.ffn_hidden, d), R = m->R;
    if (dalloc(m, (void**)&m->x, (size_t)R * d * 4) || dalloc(m, (void**)&m->xn, (size_t)R * d * 4) ||
        dalloc(m, (void**)&m->y, (size_t)R * d * 4) ||
        dalloc(m, (void**)&m->qkv, (size_t)R * m->qkv_rows * 4) ||
        dalloc(m, (void**)&m->att, (size_t)R * d * 4) ||
        dalloc(m, (void**)&m->h, (size_t)R * 2 * big * 4) ||
        dalloc(m, (void**)&m->xb, (size_t)R * d * 4) || dalloc(m, (void**)&m->y2, (size_t)R * d * 4) ||
        dalloc(m, (void**)&m->logits, (size_t)m->RF * c.vocab * 4) ||
        dalloc(m, (void**)&m->pos_dev, (size_t)R * 4) || dalloc(m, (void**)&m->slot_dev, (size_t)R * 4) ||
        dalloc(m, (void**)&m->tok_dev, (size_t)R * 4) || dalloc(m, (void**)&m->step_dev, 4) ||
        dalloc(m, (void**)&m->hist_len, 4) ||
        dalloc(m, (void**)&m->hist, (size_t)(c.max_seq + 2) * 4) ||
        dalloc(m, (void**)&m->choice_dev, (size_t)m->RF * 4) ||
        dalloc(m, (void**)&m->argpart, (size_t)ARGMAX_MAX_PARTS * 8) ||
        dalloc(m, (void**)&m->samp_cfg, sizeof(SampleCfg)) || dalloc(m, (void**)&m->rng_dev, 8) ||
        dalloc(m, (void**)&m->suppress_dev, 64 * 4))
        return fail(m);
    m->suppress_cap = 64;     // a captured step holds the pointer: never null
    // RoPE tables
    {
        std::vector<float> cs, sn;
        rope_tables(c, hd, cs, sn);
        if (dalloc(m, (void**)&m->cos_tab, cs.size() * 4) ||
            dalloc(m, (void**)&m->sin_tab, sn.size() * 4) ||
            dalloc(m, (void**)&m->rope_row, (size_t)hd * 4))
            return fail(m);
        if (hipMemcpy(m->cos_tab, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(m->sin_tab, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            set_error(ATLAS_EHIP, "rope table upload failed");
            return fail(m);
        }
    }
    // Split counts.  The fused kernel sizes its grid for the longest context
    // and activates attn_fused_splits_for(n_kv * n_seq, ctx) of its splits at
    // the live context, so short contexts run one block per KV head and merge
    // nothing.  The unfused kernel's count is fixed at launch.
    m->attn_splits = attn_pick_splits(c.n_kv_heads, c.max_seq);
    m->attn_splits_unfused = m->attn_splits;
    m->attn_splits_long = attn_splits_for(c.n_kv_heads, c.max_seq);
    // split-K partials of the ragged batch's skinny GEMMs and the prompt
    // chunks' tiled GEMMs, allocated now so that no later launch (graph
    // capture included) allocates
    {
        const int nb = R < kMaxRows ? R : kMaxRows;
        const int shapes[5][2] = {{m->qkv_rows, d}, {d, c.n_heads * hd}, {2 * c.ffn_hidden, d},
                                  {d, c.ffn_hidden}, {c.vocab, d}};
        size_t need = 0;
        for (const auto& sh : shapes) {
            if (sh[1] % 32 == 0) need = std::max(need, skinny_partial_bytes(sh[0], nb, sh[1]));
            if (m->big_prefill)
                need = std::max(need, gemm_rows_partial_bytes(sh[0], kPrefillBig, sh[1]));
        }
        if (need && dalloc(m, (void**)&m->gemm_part, need)) return fail(m);
        m->gemm_part_bytes = need;
        // bf16 and int8 prompt chunks through hipBLASLt (bf16 1.6x the tiled
        // kernel's rate at 127 rows of the 7B shapes) only when the
        // environment sets ATLAS_PROMPT_BLAS=1.  Off by default: one process
        // that had created and destroyed two library contexts (and run an
        // int4 model between) saw the library report that it could not
        // initialise its kernel host, then crash, and the cause is not
        // known.  Without a library context the tiled kernel serves every
        // prompt chunk, as it serves int4.
        if (m->big_prefill && (fmt == WF_BF16 || fmt == WF_I8) && prompt_blas_opt_in()) {
            int max_m = 0, max_k = 0;
            for (const auto& sh : shapes) {
                max_m = std::max(max_m, sh[0]);
                max_k = std::max(max_k, sh[1]);
            }
            if (blas_rows_create(&m->blas, kPrefillLib, max_m, max_k) != ATLAS_OK) {
                m->blas = nullptr;
                if (atlas_last_error_code() == ATLAS_ENOMEM) return fail(m);
                atlas_clear_error();
            }

        }
    }
    // fused step: post-norm model whose attention shape the fused kernel
    // covers and whose GEMVs take the aligned fast path (d % 32 == 0)
    m->fused = c.post_norm && attn_fused_supported(c.n_heads, c.n_kv_heads, hd) &&
               attn_rows_fit(c.max_seq, c.n_kv_heads, hd) && d % 32 == 0 &&
               c.ffn_hidden % 32 == 0;
    // split partials: the fused kernel's B x n_heads x attn_splits, the
    // long-context step's n_heads x attn_splits_long, or the long-context
    // batch step's n x n_heads x attn_splits_batch[n]
    size_t part_slots = std::max((size_t)m->RF * c.n_heads * m->attn_splits,
                                 (size_t)c.n_heads * m->attn_splits_long);
    for (int n = 1; n <= R; ++n) {
        const int sp = attn_batch_splits_for(c.n_kv_heads, n, c.max_seq);
        if (n <= kMaxRows) m->attn_splits_batch[n] = sp;
        part_slots = std::max(part_slots, (size_t)n * c.n_heads * sp);
    }
    if (dalloc(m, (void**)&m->attn_part, part_slots * (hd + 2) * 4) ||
        dalloc(m, (void**)&m->attn_counters, (size_t)m->RF * c.n_kv_heads * 4))
        return fail(m);
    if (hipMemset(m->attn_counters, 0, (size_t)m->RF * c.n_kv_heads * 4) != hipSuccess) {
        set_error(ATLAS_EHIP, "counter init failed");
        return fail(m);
    }
    if (reset_state(m) || hipStreamSynchronize(m->st) != hipSuccess) return fail(m);
    return m;
}

ATLAS_API void atlas_model_destroy(atlas_model* m) {
    if (!m) return;
    if (m->st) (void)hipStreamSynchronize(m->st);
    drop_graphs(m);
    blas_rows_destroy(m->blas);
    for (void* p : m->allocs) (void)hipFree(p);
    for (auto& e : m->ring_ev)
        if (e) (void)hipEventDestroy(e);
    if (m->ring) (void)hipHostFree(m->ring);
    if (m->hook_stage) (void)hipHostFree(m->hook_stage);
    if (m->st) (void)hipStreamDestroy(m->st);
    delete m;
}

ATLAS_API int atlas_model_set_tensor(atlas_model* m, int kind, int layer, const void* data,
                                     const float* scales) {
    ATLAS_REQUIRE(m && data, "set_tensor: null argument");
    return tensor_io(m, kind, layer, const_cast<void*>(data), const_cast<float*>(scales), true);
}

ATLAS_API atlas_load_scratch* atlas_load_scratch_create(void) { return new atlas_load_scratch(); }

ATLAS_API void atlas_load_scratch_destroy(atlas_load_scratch* s) {
    if (!s) return;
    if (s->conv || s->qdata || s->qscales) (void)hipDeviceSynchronize();
    if (s->conv) (void)hipFree(s->conv);
    if (s->qdata) (void)hipFree(s->qdata);
    if (s->qscales) (void)hipFree(s->qscales);
    delete s;
}

ATLAS_API int atlas_model_set_tensor_dev(atlas_model* m, int kind, int layer, const void* src,
                                         int src_dtype, int64_t numel, atlas_load_scratch* scratch) {
    ATLAS_REQUIRE(m, "set_tensor_dev: null model");
    ATLAS_REQUIRE(numel >= 0, "set_tensor_dev: numel < 0");
    if (scratch) return set_tensor_dev(m, kind, layer, src, src_dtype, (size_t)numel, *scratch);
    atlas_load_scratch s;
    int rc = set_tensor_dev(m, kind, layer, src, src_dtype, (size_t)numel, s);
    if (hipStreamSynchronize(m->st) != hipSuccess && rc == ATLAS_OK) {
        set_error(ATLAS_EHIP, "set_tensor_dev: stream synchronisation failed");
        rc = ATLAS_EHIP;
    }
    if (s.conv) (void)hipFree(s.conv);
    if (s.qdata) (void)hipFree(s.qdata);
    if (s.qscales) (void)hipFree(s.qscales);
    return rc;
}

ATLAS_API int atlas_model_get_tensor(atlas_model* m, int kind, int layer, void* data,
                                     float* scales) {
    ATLAS_REQUIRE(m && data, "get_tensor: null argument");
    return tensor_io(m, kind, layer, data, scales, false);
}

ATLAS_API int atlas_model_init_random(atlas_model* m, uint64_t seed) {
    ATLAS_REQUIRE(m, "init_random: null model");
    const atlas_model_config& c = m->cfg;
    const int d = c.d_model;
    auto sub = [&](int kind, int layer) {
        uint64_t z = seed + 0x9E3779B97F4A7C15ULL * (uint64_t)(kind * 4096 + layer + 1);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    };
    // temporaries sized for the largest matrix
    const size_t max_el = std::max((size_t)c.vocab * d, (size_t)c.ffn_hidden * d);
    float* tmp = nullptr;
    void* qd = nullptr;
    float* qs = nullptr;
    if (dev_malloc(&tmp, max_el * 4) != hipSuccess) {
        (void)hipGetLastError();
        set_error(ATLAS_ENOMEM, "init_random: temporaries");
        return ATLAS_ENOMEM;
    }
    int rc = ATLAS_OK;
    const int fmt = c.weight_format;
    if (fmt != WF_BF16) {
        if (dev_malloc(&qd, max_el) != hipSuccess || dev_malloc(&qs, max_el / 8 * 4 + 64) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(tmp);
            if (qd) (void)hipFree(qd);
            set_error(ATLAS_ENOMEM, "init_random: temporaries");
            return ATLAS_ENOMEM;
        }
    }
    // matrix: generate into tmp (bf16 bits or f32), convert, place
    auto mat = [&](DevMat& dst, int base, int stride, int rows, int kind, int layer) -> int {
        const long n = (long)rows * dst.cols;
        if (fmt == WF_BF16) {
            TRY(init_launch(INIT_NORMAL_BF16, tmp, n, sub(kind, layer), 0.f, 0.02f, m->st));
            const size_t rb = dst.row_bytes(), rp = dst.row_pitch();
            ATLAS_HIP(hipMemcpy2DAsync((char*)dst.w + (size_t)base * rp, rp * stride, tmp, rb, rb, rows,
                                       hipMemcpyDeviceToDevice, m->st));
        } else {
            TRY(init_launch(INIT_NORMAL_F32, tmp, n, sub(kind, layer), 0.f, 0.02f, m->st));
            if (fmt == WF_I8) TRY(quant_i8_launch(tmp, 0, rows, dst.cols, (int8_t*)qd, qs, m->st));
            else TRY(quant_i4_launch(tmp, 0, n, dst.block, (uint8_t*)qd, qs, m->st));
            const size_t rb = dst.row_bytes(), rp = dst.row_pitch(), spr = dst.scales_per_row();
            ATLAS_HIP(hipMemcpy2DAsync((char*)dst.w + (size_t)base * rp, rp * stride, qd, rb, rb, rows,
                                       hipMemcpyDeviceToDevice, m->st));
            ATLAS_HIP(hipMemcpy2DAsync(dst.scales + (size_t)base * spr, spr * 4 * stride, qs, spr * 4,
                                       spr * 4, rows, hipMemcpyDeviceToDevice, m->st));
        }
        ATLAS_HIP(hipStreamSynchronize(m->st));
        return ATLAS_OK;
    };
    auto vec = [&](float* dst, long n, int kind, int layer) -> int {
        if (!dst) return ATLAS_OK;
        return init_launch(INIT_UNIFORM_F32, dst, n, sub(kind, layer), 0.5f, 1.5f, m->st);
    };
    for (int li = 0; li < c.n_layers && !rc; ++li) {
        LayerW& L = m->L[li];
        rc = mat(L.qkv, 0, 1, d, ATLAS_T_WQ, li);
        if (!rc) rc = mat(L.qkv, d, 1, m->kvd, ATLAS_T_WK, li);
        if (!rc) rc = mat(L.qkv, d + m->kvd, 1, m->kvd, ATLAS_T_WV, li);
        if (!rc) rc = mat(L.wo, 0, 1, d, ATLAS_T_WO, li);
        if (!rc) rc = mat(L.gu, 0, 2, c.ffn_hidden, ATLAS_T_W_GATE, li);
        if (!rc) rc = mat(L.gu, 1, 2, c.ffn_hidden, ATLAS_T_W_UP, li);
        if (!rc) rc = mat(L.down, 0, 1, d, ATLAS_T_W_DOWN, li);
        if (!rc) rc = vec(L.attn_norm, d, ATLAS_T_ATTN_NORM, li);
        if (!rc) rc = vec(L.ffn_norm, d, ATLAS_T_FFN_NORM, li);
        if (!rc) rc = vec(L.q_norm, (long)c.n_heads * m->hd, ATLAS_T_Q_NORM, li);
        if (!rc) rc = vec(L.k_norm, m->kvd, ATLAS_T_K_NORM, li);
    }
    if (!rc) rc = init_launch(INIT_NORMAL_BF16, m->embed, (long)c.vocab * d, sub(ATLAS_T_EMBED, 0), 0.f,
                              0.02f, m->st);
    if (!rc) rc = mat(m->lm_head, 0, 1, c.vocab, ATLAS_T_LM_HEAD, 0);
    if (!rc) rc = vec(m->final_norm, d, ATLAS_T_FINAL_NORM, 0);
    if (!rc && hipStreamSynchronize(m->st) != hipSuccess) {
        set_error(ATLAS_EHIP, "init_random: sync failed");
        rc = ATLAS_EHIP;
    }
    (void)hipFree(tmp);
    if (qd) (void)hipFree(qd);
    if (qs) (void)hipFree(qs);
    return rc;
}

ATLAS_API int atlas_model_reset(atlas_model* m) {
    ATLAS_REQUIRE(m, "reset: null model");
    TRY(reset_state(m));
    ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}

ATLAS_API int atlas_model_get_config(const atlas_model* m, atlas_model_config* out) {
    ATLAS_REQUIRE(m && out, "get_config: null argument");
    *out = m->cfg;
    return ATLAS_OK;
}

ATLAS_API int atlas_model_pos(const atlas_model* m) { return m ? m->pos : -1; }

ATLAS_API int atlas_model_set_kv_rows(atlas_model* m, int seq, int layer, int pos0, int n,
                                      const float* k, const float* v) {
    ATLAS_REQUIRE(m && k && v, "set_kv_rows: null argument");
    const atlas_model_config& c = m->cfg;
    ATLAS_REQUIRE(seq >= 0 && seq < m->B, "set_kv_rows: sequence %d outside 0..%d", seq, m->B - 1);
    ATLAS_REQUIRE(layer >= 0 && layer < c.n_layers, "set_kv_rows: layer %d", layer);
    ATLAS_REQUIRE(pos0 >= 0 && n >= 0 && (long)pos0 + n <= c.max_seq,
                  "set_kv_rows: rows [%d, %ld) outside the cache of %d", pos0, (long)pos0 + n,
                  c.max_seq);
    const size_t off = (size_t)seq * m->slot_stride + (size_t)pos0 * m->kvd;
    const size_t bytes = (size_t)n * m->kvd * 4;
    ATLAS_HIP(hipMemcpyAsync(m->L[layer].kc + off, k, bytes, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipMemcpyAsync(m->L[layer].vc + off, v, bytes, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}

ATLAS_API int atlas_model_set_pos(atlas_model* m, int pos) {
    ATLAS_REQUIRE(m, "set_pos: null model");
    ATLAS_REQUIRE(pos >= 0 && pos < m->cfg.max_seq, "set_pos: %d outside [0, %d)", pos,
                  m->cfg.max_seq);
    m->pos = pos;
    TRY(sync_pos(m));
    ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}
ATLAS_API float atlas_model_attn_scale(const atlas_model* m) { return m ? m->scale : 0.f; }
ATLAS_API void* atlas_model_stream(atlas_model* m) { return m ? (void*)m->st : nullptr; }
ATLAS_API const float* atlas_model_logits_dev(atlas_model* m) { return m ? m->logits : nullptr; }

ATLAS_API int atlas_model_set_long_context(atlas_model* m, int from_pos) {
    ATLAS_REQUIRE(m, "set_long_context: null model");
    ATLAS_REQUIRE(from_pos >= 0, "set_long_context: from_pos %d < 0", from_pos);
    m->long_from = from_pos;
    return ATLAS_OK;
}

ATLAS_API int atlas_model_set_prefill_chunk(atlas_model* m, int chunk) {
    ATLAS_REQUIRE(m, "set_prefill_chunk: null model");
    ATLAS_REQUIRE(chunk >= 1 && chunk <= kPrefillLib, "set_prefill_chunk: %d outside 1..%d", chunk,
                  kPrefillLib);
    m->prefill_chunk = chunk;
    return ATLAS_OK;
}

ATLAS_API int atlas_model_prefill(atlas_model* m, const uint32_t* tokens, int n) {
    ATLAS_REQUIRE(m && n >= 0 && (n == 0 || tokens), "prefill: bad arguments");
    TRY(prefill(m, tokens, n));
    ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}

ATLAS_API int atlas_model_use_graph(atlas_model* m, int enable) {
    ATLAS_REQUIRE(m, "use_graph: null model");
    m->use_graph = enable != 0;
    if (!m->use_graph) drop_graphs(m);
    return ATLAS_OK;
}

ATLAS_API int64_t atlas_model_weight_bytes(const atlas_model* m) {
    if (!m) return 0;
    int64_t b = 0;
    for (const auto& L : m->L)
        for (const DevMat* w : {&L.qkv, &L.wo, &L.gu, &L.down})
            b += (int64_t)w->data_bytes() + (int64_t)w->scale_count() * 4;
    b += (int64_t)m->lm_head.data_bytes() + (int64_t)m->lm_head.scale_count() * 4;
    return b;
}

ATLAS_API int atlas_model_forward_one(atlas_model* m, uint32_t token, float* logits) {
    ATLAS_REQUIRE(m, "forward_one: null model");
    TRY(sync_pos(m));
    TRY(set_token(m, token));
    TRY(run_step(m, 0));
    if (logits) TRY(download_logits(m, logits));
    else ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}

ATLAS_API int atlas_model_forward_one_hooked(atlas_model* m, uint32_t token, float* logits,
                                             float* hidden, atlas_hook_fn hook, void* user) {
    ATLAS_REQUIRE(m, "forward_one_hooked: null model");
    const atlas_model_config& c = m->cfg;
    const bool keep = hidden || hook;
    if (!keep) return atlas_model_forward_one(m, token, logits);
    // The hook only reads the hidden states (StigmergicHook::on_layer returns
    // a deposit; nothing flows back into the model), so the token runs as one
    // captured step that also copies every layer's hidden state aside (mode
    // 3); the hooks run in layer order once it is done -- one host round
    // trip per token instead of one per layer.
    const size_t hb = (size_t)c.n_layers * c.d_model * 4;
    if (!m->hook_dev) TRY(dalloc(m, (void**)&m->hook_dev, hb));
    if (!m->hook_stage && host_malloc_pinned(&m->hook_stage, hb) != hipSuccess) {
        (void)hipGetLastError();
        m->hook_stage = nullptr;
        set_error(ATLAS_ENOMEM, "forward_one_hooked: pinned staging of %zu bytes", hb);
        return ATLAS_ENOMEM;
    }
    TRY(sync_pos(m));
    TRY(set_token(m, token));
    TRY(run_step(m, 3));
    ATLAS_HIP(hipMemcpyAsync(m->hook_stage, m->hook_dev, hb, hipMemcpyDeviceToHost, m->st));
    if (logits) TRY(download_logits(m, logits));
    else ATLAS_HIP(hipStreamSynchronize(m->st));
    if (hidden) std::memcpy(hidden, m->hook_stage, hb);
    if (hook)
        for (int li = 0; li < c.n_layers; ++li) {
            float delta = 0.f;
            (void)hook(user, li, m->hook_stage + (size_t)li * c.d_model, c.d_model, &delta);
        }
    return ATLAS_OK;
}

namespace {

// Shared driver of generate / generate_streaming (lib.rs:1599-1732, 1853-1955).
int generate_impl(atlas_model* m, const uint32_t* prompt, int n_prompt, int max_new,
                  const atlas_sampling* s, uint32_t* out, int* n_out, atlas_token_fn on_token,
                  void* user) {
    ATLAS_REQUIRE(m && n_out && (out || on_token), "generate: null argument");
    ATLAS_REQUIRE(n_prompt >= 0 && max_new >= 0 && (n_prompt == 0 || prompt), "generate: bad prompt");
    *n_out = 0;
    const int V = m->cfg.vocab;
    TRY(reset_state(m));
    seed_rng(m, s);
    ATLAS_REQUIRE(n_prompt + max_new <= m->cfg.max_seq,
                  "generate: prompt %d + max_new %d exceeds max_seq %d", n_prompt, max_new,
                  m->cfg.max_seq);
    std::vector<uint32_t> gen;
    std::vector<float> logits((size_t)V, 0.0f);
    const bool greedy = is_greedy(s);
    const bool device_sample = !greedy && !on_token && sample_dev_ok(s, V, max_new);
    const bool device_choice = (greedy && !on_token) || device_sample;
    const int choose_mode = greedy ? 1 : 2;
    if (greedy && device_choice) TRY(set_greedy_cfg(m, s));

    // prompt: forward all but the last token without choosing
    if (n_prompt > 1) TRY(prefill(m, prompt, n_prompt - 1));
    if (max_new == 0) {
        if (n_prompt > 0) {
            TRY(set_token(m, prompt[n_prompt - 1]));
            TRY(run_step(m, 0));
        }
        ATLAS_HIP(hipStreamSynchronize(m->st));
        return ATLAS_OK;
    }

    if (device_choice && n_prompt > 0) {
        // choice on the device (greedy, or sampled from the device RNG state):
        // each replay forwards the last choice and chooses the next; check for
        // stop tokens every `chunk` replays.
        if (device_sample) TRY(set_sample_cfg(m, s));
        TRY(set_token(m, prompt[n_prompt - 1]));
        TRY(run_step(m, choose_mode));              // chooses t_1
        int issued = 1;                              // tokens chosen so far
        int forwarded = 0;                           // generated tokens forwarded
        std::vector<uint32_t> h;
        const int chunk = 16;
        while (true) {
            h.resize(issued);
            ATLAS_HIP(hipMemcpyAsync(h.data(), m->hist, (size_t)issued * 4, hipMemcpyDeviceToHost,
                                     m->st));
            ATLAS_HIP(hipStreamSynchronize(m->st));
            // the output is t_1..t_k: k = max_new, or t_{k+1} is a stop token
            gen.clear();
            bool determined = false;
            for (int j = 0; j < issued; ++j) {
                if ((int)gen.size() >= max_new || is_stop(s, h[j])) {
                    determined = true;
                    break;
                }
                gen.push_back(h[j]);
            }
            if ((int)gen.size() >= max_new) determined = true;
            const int k = (int)gen.size();
            if (determined && forwarded >= k) break;
            // each replay forwards the latest choice and chooses the next; the
            // forward of t_k is the reference's final forward (lib.rs:1725-1729)
            const int want = determined ? k - forwarded : std::min(chunk, max_new - forwarded);
            for (int r = 0; r < want; ++r) TRY(run_step(m, choose_mode));
            issued += want;
            forwarded += want;
        }
        // the reference forwarded exactly n_prompt + |gen| tokens; anything
        // beyond (a chunk that ran past a stop token) is never read again
        m->pos = n_prompt + (int)gen.size();
        TRY(sync_pos(m));
        for (size_t i = 0; i < gen.size(); ++i) out[i] = gen[i];
        *n_out = (int)gen.size();
        ATLAS_HIP(hipStreamSynchronize(m->st));
        return ATLAS_OK;
    }

    // host choice (sampling, streaming, or an empty prompt)
    if (n_prompt > 0) {
        TRY(set_token(m, prompt[n_prompt - 1]));
        TRY(run_step(m, 0));
        TRY(download_logits(m, logits.data()));
    }
    for (int step = 0; step < max_new; ++step) {
        const uint32_t tok = host_choose(m, logits.data(), step, gen, s);
        if (is_stop(s, tok)) break;
        gen.push_back(tok);
        if (out) out[gen.size() - 1] = tok;
        if (on_token && !on_token(user, tok)) break;
        TRY(set_token(m, tok));
        TRY(run_step(m, 0));
        TRY(download_logits(m, logits.data()));
    }
    *n_out = (int)gen.size();
    return ATLAS_OK;
}

}  // namespace

ATLAS_API int atlas_model_generate(atlas_model* m, const uint32_t* prompt, int n_prompt,
                                   int max_new, const atlas_sampling* s, uint32_t* out,
                                   int* n_out) {
    return generate_impl(m, prompt, n_prompt, max_new, s, out, n_out, nullptr, nullptr);
}

ATLAS_API int atlas_model_generate_streaming(atlas_model* m, const uint32_t* prompt, int n_prompt,
                                             int max_new, const atlas_sampling* s,
                                             atlas_token_fn on_token, void* user, int* n_out) {
    ATLAS_REQUIRE(on_token, "generate_streaming: null callback");
    std::vector<uint32_t> out((size_t)std::max(max_new, 1));
    return generate_impl(m, prompt, n_prompt, max_new, s, out.data(), n_out, on_token, user);
}

namespace {
struct HookAcc {
    atlas_hook_fn fn;
    void* user;
    float acc;
    uint32_t fired;
};
int acc_hook(void* u, int li, const float* hidden, int d, float* delta) {
    HookAcc* h = (HookAcc*)u;
    float dl = 0.f;
    if (h->fn(h->user, li, hidden, d, &dl)) {
        h->acc += dl > 0.f ? dl : 0.f;      // max(delta, 0): lib.rs:1839
        h->fired += 1;
    }
    *delta = dl;
    return 0;
}
}  // namespace

ATLAS_API int atlas_model_generate_hooked(atlas_model* m, const uint32_t* prompt, int n_prompt,
                                          int max_new, const atlas_sampling* s, atlas_hook_fn hook,
                                          void* user, uint32_t* out, float* total_delta,
                                          uint32_t* layers_fired, int* n_out) {
    ATLAS_REQUIRE(m && hook && out && n_out, "generate_hooked: null argument");
    ATLAS_REQUIRE(n_prompt >= 0 && max_new >= 0 && (n_prompt == 0 || prompt), "generate_hooked: bad prompt");
    *n_out = 0;
    const int V = m->cfg.vocab;
    TRY(reset_state(m));
    seed_rng(m, s);
    ATLAS_REQUIRE(n_prompt + max_new <= m->cfg.max_seq, "generate_hooked: exceeds max_seq");
    std::vector<float> logits((size_t)V, 0.0f);
    HookAcc acc{hook, user, 0.f, 0};
    // prefill: hook runs, deposits discarded (lib.rs:1763-1770)
    for (int i = 0; i < n_prompt; ++i)
        TRY(atlas_model_forward_one_hooked(m, prompt[i], logits.data(), nullptr, acc_hook, &acc));
    std::vector<uint32_t> gen;
    for (int step = 0; step < max_new; ++step) {
        const uint32_t tok = host_choose(m, logits.data(), step, gen, s);
        if (is_stop(s, tok)) break;
        gen.push_back(tok);
        out[gen.size() - 1] = tok;
        acc.acc = 0.f;
        acc.fired = 0;
        TRY(atlas_model_forward_one_hooked(m, tok, logits.data(), nullptr, acc_hook, &acc));
        if (total_delta) total_delta[gen.size() - 1] = acc.acc;
        if (layers_fired) layers_fired[gen.size() - 1] = acc.fired;
    }
    *n_out = (int)gen.size();
    return ATLAS_OK;
}

static int decode_greedy(atlas_model* m, uint32_t first_token, int n_steps, uint32_t* tokens,
                         float* step_ms) {
    ATLAS_REQUIRE(m && n_steps >= 0, "decode_greedy: bad arguments");
    ATLAS_REQUIRE(m->pos + n_steps <= m->cfg.max_seq, "decode_greedy: exceeds max_seq");
    TRY(set_greedy_cfg(m, nullptr));
    int zero = 0;
    ATLAS_HIP(hipMemcpyAsync(m->hist_len, &zero, 4, hipMemcpyHostToDevice, m->st));
    ATLAS_HIP(hipMemcpyAsync(m->step_dev, &zero, 4, hipMemcpyHostToDevice, m->st));
    TRY(sync_pos(m));
    TRY(set_token(m, first_token));
    // step_ms: an event after every step (and one before the first), on the
    // engine stream, so step i's GPU time is the span between two of them
    std::vector<hipEvent_t> ev;
    int rc = ATLAS_OK;
    // this function's own HIP calls record what failed; an error from
    // run_step keeps the message run_step recorded
    auto hip_ok = [&rc](hipError_t e, const char* what) {
        if (e == hipSuccess) return true;
        set_error(ATLAS_EHIP, "decode_greedy: %s: %s", what, hipGetErrorString(e));
        rc = ATLAS_EHIP;
        return false;
    };
    if (step_ms) {
        ev.resize((size_t)n_steps + 1, nullptr);
        for (auto& e : ev)
            if (!rc) hip_ok(hipEventCreate(&e), "hipEventCreate");
        if (!rc) hip_ok(hipEventRecord(ev[0], m->st), "hipEventRecord");
    }
    for (int i = 0; i < n_steps && !rc; ++i) {
        rc = run_step(m, 1);
        if (!rc && step_ms) hip_ok(hipEventRecord(ev[i + 1], m->st), "hipEventRecord");
    }
    if (!rc && tokens && n_steps > 0)
        hip_ok(hipMemcpyAsync(tokens, m->hist, (size_t)n_steps * 4, hipMemcpyDeviceToHost, m->st),
               "token download");
    {
        const hipError_t e = hipStreamSynchronize(m->st);
        if (!rc) hip_ok(e, "hipStreamSynchronize");
    }
    for (int i = 0; i < n_steps && !rc && step_ms; ++i)
        hip_ok(hipEventElapsedTime(&step_ms[i], ev[i], ev[i + 1]), "hipEventElapsedTime");
    for (auto e : ev)
        if (e) (void)hipEventDestroy(e);
    return rc;
}

ATLAS_API int atlas_model_decode_greedy(atlas_model* m, uint32_t first_token, int n_steps,
                                        uint32_t* tokens) {
    return decode_greedy(m, first_token, n_steps, tokens, nullptr);
}

ATLAS_API int atlas_model_decode_greedy_timed(atlas_model* m, uint32_t first_token, int n_steps,
                                              uint32_t* tokens, float* step_ms) {
    ATLAS_REQUIRE(step_ms, "decode_greedy_timed: null step_ms");
    return decode_greedy(m, first_token, n_steps, tokens, step_ms);
}

ATLAS_API int atlas_model_bench_gemv(atlas_model* m, int iters, int which, float* ms,
                                     int* launches, int64_t* bytes) {
    ATLAS_REQUIRE(m && iters > 0 && ms && launches && bytes && which >= 0 && which <= 6,
                  "bench_gemv: bad arguments");
    const float eps = m->cfg.rms_eps;
    auto mat_bytes = [](const DevMat& w, int64_t out) {
        return (int64_t)w.data_bytes() + (int64_t)w.scale_count() * 4 + (int64_t)w.cols * 4 + out * 4;
    };
    const bool k_set = which == 0 || which == 1, down_set = which == 0 || which == 2,
               gu_set = which == 0 || which == 3;
    const bool qkv_set = k_set || which == 4, wo_set = k_set || which == 5, lm_set = k_set || which == 6;
    int64_t b = 0;
    int n = 0;
    for (const auto& L : m->L) {
        if (qkv_set) {
            b += mat_bytes(L.qkv, L.qkv.rows);
            n += 1;
        }
        if (wo_set) {
            b += mat_bytes(L.wo, L.wo.rows);
            n += 1;
        }
        if (gu_set) {
            b += mat_bytes(L.gu, L.gu.rows / 2);
            n += 1;
        }
        if (down_set) {
            b += mat_bytes(L.down, L.down.rows);
            n += 1;
        }
    }
    if (lm_set) {
        b += mat_bytes(m->lm_head, m->lm_head.rows);
        n += 1;
    }
    hipEvent_t e0, e1;
    ATLAS_HIP(hipEventCreate(&e0));
    ATLAS_HIP(hipEventCreate(&e1));
    ATLAS_HIP(hipEventRecord(e0, m->st));
    for (int it = 0; it < iters; ++it) {
        for (size_t li = 0; li < m->L.size(); ++li) {
            LayerW& L = m->L[li];
            if (qkv_set) {
                if (m->fused)
                    TRY(gemv_launch(pro_args(L.qkv, m->xb, m->qkv, PRO_RESNORM, m->y2, L.ffn_norm, eps, m->x), m->st));
                else
                    TRY(gemv(m, L.qkv, m->x, m->qkv, EPI_STORE));
            }
            if (wo_set) TRY(gemv(m, L.wo, m->att, m->y, EPI_STORE));
            if (gu_set) {
                if (m->fused) TRY(enqueue_gu_fused(m, L));
                else TRY(gemv(m, L.gu, m->x, m->h, EPI_SILU_MUL));
            }
            if (down_set) {
                if (m->fused) TRY(enqueue_down_fused(m, L));
                else TRY(gemv(m, L.down, m->h, m->y, EPI_STORE));
            }
        }
        if (lm_set) {
            if (m->fused) {
                GemvArgs h = pro_args(m->lm_head, m->xb, m->logits, PRO_RESNORM_NORM, m->y2,
                                      m->L.back().ffn_norm, eps, nullptr);
                h.pro_w2 = m->final_norm;
                if (!gemv_resnorm_norm_ok(h))
                    h = pro_args(m->lm_head, m->xb, m->logits, PRO_RMSNORM, nullptr, m->final_norm,
                                 eps, m->xn);
                TRY(gemv_launch(h, m->st));
            }
            else
                TRY(gemv(m, m->lm_head, m->xn, m->logits, EPI_STORE));
        }
    }
    ATLAS_HIP(hipEventRecord(e1, m->st));
    ATLAS_HIP(hipEventSynchronize(e1));
    float t = 0.f;
    ATLAS_HIP(hipEventElapsedTime(&t, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms = t;
    *launches = n * iters;
    *bytes = b;
    return ATLAS_OK;
}

ATLAS_API int atlas_sample_host(const float* logits, int vocab, const uint32_t* hist, int n_hist,
                                int step, const atlas_sampling* s, uint64_t* rng_state,
                                uint32_t* token) {
    if (!logits || vocab <= 0 || n_hist < 0 || (n_hist && !hist) || !rng_state || !token ||
        (s && s->n_suppress > 0 && !s->suppress_initial_tokens))
        return ATLAS_EINVAL;
    Rng rng{*rng_state};
    *token = choose_token(logits, vocab, step, hist, (size_t)n_hist, s, rng);
    *rng_state = rng.s;
    return ATLAS_OK;
}

ATLAS_API int atlas_sample_device(const float* logits, int vocab, const uint32_t* hist,
                                  int n_hist, int step, const atlas_sampling* s,
                                  uint64_t* rng_state, uint32_t* token) {
    ATLAS_REQUIRE(logits && vocab > 0 && n_hist >= 0 && (n_hist == 0 || hist) && s && rng_state &&
                  token && step >= 0 && (s->n_suppress <= 0 || s->suppress_initial_tokens),
                  "sample_device: bad arguments");
    if (!sample_dev_ok(s, vocab, n_hist)) {
        set_error(ATLAS_EUNSUPPORTED, "sample_device: temperature %g, top_k %d, top_p %g, %d history "
                  "tokens: the device sampler needs temperature > 0 and 1 <= top_k <= %d, or "
                  "top_k = 0 with top_p = 1", s->temperature, s->top_k, s->top_p, n_hist,
                  (int)SAMPLE_MAX_K);
        return ATLAS_EUNSUPPORTED;
    }
    const SampleCfg c = sample_cfg_of(s);
    hipStream_t st = stream();
    // one device block: logits copy | history | suppression | settings | counters
    const size_t nh = (size_t)n_hist + 1, ns = (size_t)std::max(c.n_suppress, 1);
    const size_t off_h = (size_t)vocab * 4, off_s = off_h + nh * 4, off_c = off_s + ns * 4;
    const size_t off_i = (off_c + sizeof(SampleCfg) + 7) & ~(size_t)7;
    const size_t bytes = off_i + 32;
    char* d = nullptr;
    if (dev_malloc(&d, bytes) != hipSuccess) {
        (void)hipGetLastError();
        set_error(ATLAS_ENOMEM, "sample_device: %zu bytes", bytes);
        return ATLAS_ENOMEM;
    }
    int rc = ATLAS_OK;
    const int ints[4] = {n_hist, step, 0, 0};
    if (hipMemcpyAsync(d, logits, (size_t)vocab * 4, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        (n_hist && hipMemcpyAsync(d + off_h, hist, (size_t)n_hist * 4, hipMemcpyHostToDevice, st) != hipSuccess) ||
        (c.n_suppress && hipMemcpyAsync(d + off_s, s->suppress_initial_tokens, (size_t)c.n_suppress * 4,
                                        hipMemcpyHostToDevice, st) != hipSuccess) ||
        hipMemcpyAsync(d + off_c, &c, sizeof c, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(d + off_i, rng_state, 8, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipMemcpyAsync(d + off_i + 8, ints, 16, hipMemcpyHostToDevice, st) != hipSuccess) {
        set_error(ATLAS_EHIP, "sample_device: upload failed");
        rc = ATLAS_EHIP;
    }
    if (!rc) {
        SampleArgs a{};
        a.x = (float*)d; a.n = vocab; a.cfg = (const SampleCfg*)(d + off_c);
        a.suppress = (const uint32_t*)(d + off_s);
        a.hist = (uint32_t*)(d + off_h); a.hist_len = (int*)(d + off_i + 8);
        a.step = (int*)(d + off_i + 12); a.pos_inc = nullptr;
        a.rng = (unsigned long long*)(d + off_i); a.out_u32 = (uint32_t*)(d + off_i + 16);
        a.record = 0;
        rc = sample_launch(a, st);
    }
    if (!rc && (hipMemcpyAsync(rng_state, d + off_i, 8, hipMemcpyDeviceToHost, st) != hipSuccess ||
                hipMemcpyAsync(token, d + off_i + 16, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
                hipStreamSynchronize(st) != hipSuccess)) {
        set_error(ATLAS_EHIP, "sample_device: download failed");
        rc = ATLAS_EHIP;
    }
    (void)hipStreamSynchronize(st);
    (void)hipFree(d);
    return rc;
}

ATLAS_API int atlas_model_generate_batch(atlas_model* m, const uint32_t* prompts,
                                         const int* prompt_lens, int n_seqs, int max_new,
                                         const atlas_sampling* s, uint32_t* out, int* n_out) {
    ATLAS_REQUIRE(m && prompt_lens && out && n_out, "generate_batch: null argument");
    ATLAS_REQUIRE(n_seqs >= 1 && n_seqs <= m->B && n_seqs <= 8,
                  "generate_batch: n_seqs %d outside 1..min(max_batch %d, 8)", n_seqs, m->B);
    ATLAS_REQUIRE(max_new >= 0, "generate_batch: max_new < 0");
    const int V = m->cfg.vocab;
    std::vector<size_t> off(n_seqs + 1, 0);
    for (int i = 0; i < n_seqs; ++i) {
        ATLAS_REQUIRE(prompt_lens[i] >= 0, "generate_batch: negative prompt length");
        ATLAS_REQUIRE(prompt_lens[i] + max_new <= m->cfg.max_seq,
                      "generate_batch: sequence %d exceeds max_seq", i);
        off[i + 1] = off[i] + prompt_lens[i];
    }
    ATLAS_REQUIRE(off[n_seqs] == 0 || prompts, "generate_batch: null prompts");
    std::vector<int> cursor(n_seqs, 0), pos(n_seqs, 0);
    std::vector<std::vector<uint32_t>> gen(n_seqs);
    std::vector<bool> done(n_seqs, false);
    std::vector<uint32_t> pending(n_seqs, 0);   // token to feed next
    std::vector<bool> has_pending(n_seqs, false);
    std::vector<float> zero_logits((size_t)V, 0.f);
    const bool host_path = !is_greedy(s) || (s && (s->n_suppress > 0 || s->repetition_penalty != 1.0f));
    seed_rng(m, s);
    for (int i = 0; i < n_seqs; ++i) {
        n_out[i] = 0;
        if (max_new == 0) { done[i] = true; continue; }
        if (prompt_lens[i] == 0) {
            // choose from all-zero logits, as the reference does with an empty prompt
            const uint32_t t = host_choose(m, zero_logits.data(), 0, gen[i], s);
            if (is_stop(s, t)) { done[i] = true; continue; }
            gen[i].push_back(t);
            pending[i] = t;
            has_pending[i] = true;
            if ((int)gen[i].size() >= max_new) done[i] = true;
        }
    }
    std::vector<uint32_t> toks(kPrefillChunk), choice(kPrefillChunk);
    std::vector<int> slots(kPrefillChunk), poss(kPrefillChunk), idx(kPrefillChunk);
    std::vector<int> rows_of(n_seqs);
    std::vector<float> lg;
    if (!m->ring) {
        if (host_malloc_pinned(&m->ring, sizeof(int) * 3 * kMaxRows * atlas_model::kRing) != hipSuccess) {
            (void)hipGetLastError();
            m->ring = nullptr;
            set_error(ATLAS_ENOMEM, "generate_batch: pinned staging ring");
            return ATLAS_ENOMEM;
        }
        for (auto& e : m->ring_ev) ATLAS_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    int ring_next = 0;
    // Rows per step: one per live sequence (its pending token or next prompt
    // token); rows left over take further prompt tokens of the sequences with
    // the most prompt left, at consecutive positions of their own slot (up to
    // prefill_chunk rows per sequence).  Such a step takes the two-kernel
    // attention variant, which writes every row's K/V before any row attends.
    const int cap = std::min(kPrefillChunk, m->R);
    // Long prompts first take the tiled GEMM's big chunks, one sequence at a
    // time in its own slot, while more than kMaxRows of their tokens before
    // the last remain; the rest joins the shared steps below.
    if (m->fused && m->big_prefill && m->prefill_chunk > kMaxRows) {
        for (int i = 0; i < n_seqs; ++i) {
            if (done[i]) continue;
            while (prompt_lens[i] - 1 - cursor[i] > kMaxRows) {
                const int k = std::min(std::min(m->prefill_chunk, prefill_cap(m)),
                                       prompt_lens[i] - 1 - cursor[i]);
                TRY(prefill_rows(m, i, pos[i], prompts + off[i] + cursor[i], k));
                cursor[i] += k;
                pos[i] += k;
            }
        }
    }
    bool any_choice_row = false;
    while (true) {
        int n = 0;
        any_choice_row = false;
        for (int i = 0; i < n_seqs; ++i) {
            rows_of[i] = 0;
            if (done[i]) continue;
            uint32_t t;
            if (cursor[i] < prompt_lens[i]) t = prompts[off[i] + cursor[i]];
            else if (has_pending[i]) t = pending[i];
            else continue;
            toks[n] = t;
            slots[n] = i;
            poss[n] = pos[i];
            idx[n] = i;
            any_choice_row = any_choice_row || cursor[i] + 1 >= prompt_lens[i];
            rows_of[i] = 1;
            ++n;
        }
        if (n == 0) break;
        bool multi = false;
        while (n < cap && m->prefill_chunk > 1) {
            int best = -1, best_rem = 0;
            for (int i = 0; i < n_seqs; ++i) {
                if (done[i] || rows_of[i] == 0 || rows_of[i] >= m->prefill_chunk) continue;
                const int rem = prompt_lens[i] - cursor[i] - rows_of[i];
                if (rem > best_rem) { best = i; best_rem = rem; }
            }
            if (best < 0) break;
            const int r = rows_of[best];
            toks[n] = prompts[off[best] + cursor[best] + r];
            slots[n] = best;
            poss[n] = pos[best] + r;
            idx[n] = best;
            any_choice_row = any_choice_row || cursor[best] + r + 1 >= prompt_lens[best];
            rows_of[best] = r + 1;
            multi = true;
            ++n;
        }
        {
            // stage through the pinned ring: steps without a host round trip
            // may still be queued when the next step's values are written
            const int k = ring_next++ % atlas_model::kRing;
            if (m->ring_used[k]) ATLAS_HIP(hipEventSynchronize(m->ring_ev[k]));
            int* e = m->ring + (size_t)k * 3 * kMaxRows;
            for (int j = 0; j < n; ++j) {
                e[j] = (int)toks[j];
                e[kMaxRows + j] = poss[j];
                e[2 * kMaxRows + j] = slots[j];
            }
            ATLAS_HIP(hipMemcpyAsync(m->tok_dev, e, (size_t)n * 4, hipMemcpyHostToDevice, m->st));
            ATLAS_HIP(hipMemcpyAsync(m->pos_dev, e + kMaxRows, (size_t)n * 4, hipMemcpyHostToDevice,
                                     m->st));
            ATLAS_HIP(hipMemcpyAsync(m->slot_dev, e + 2 * kMaxRows, (size_t)n * 4,
                                     hipMemcpyHostToDevice, m->st));
            ATLAS_HIP(hipEventRecord(m->ring_ev[k], m->st));
            m->ring_used[k] = true;
        }
        std::vector<int> sl(slots.begin(), slots.begin() + n);
        int max_pos = 0;
        for (int j = 0; j < n; ++j) max_pos = std::max(max_pos, poss[j]);
        TRY(run_batch_step(m, n, sl,
                           multi || max_pos >= std::min(m->long_from, kBatchLongAttnFrom)));
        // a row chooses a token when it consumes its last prompt token or
        // generates; steps inside every row's prompt need no host round trip
        const bool any_choice = any_choice_row;
        if (!host_path) {
            if (any_choice) {
                ATLAS_HIP(hipMemcpyAsync(choice.data(), m->choice_dev, (size_t)n * 4,
                                         hipMemcpyDeviceToHost, m->st));
                ATLAS_HIP(hipStreamSynchronize(m->st));
            }
        } else {
            lg.resize((size_t)n * V);
            ATLAS_HIP(hipMemcpyAsync(lg.data(), m->logits, (size_t)n * V * 4, hipMemcpyDeviceToHost,
                                     m->st));
            ATLAS_HIP(hipStreamSynchronize(m->st));
        }
        for (int j = 0; j < n; ++j) {
            const int i = idx[j];
            pos[i] += 1;
            bool choose;
            if (cursor[i] < prompt_lens[i]) {
                cursor[i] += 1;
                choose = cursor[i] == prompt_lens[i];
            } else {
                choose = true;
            }
            if (!choose) continue;
            if ((int)gen[i].size() >= max_new) { done[i] = true; continue; }
            const uint32_t t = host_path
                ? host_choose(m, lg.data() + (size_t)j * V, (int)gen[i].size(), gen[i], s)
                : choice[j];
            if (is_stop(s, t)) { done[i] = true; continue; }
            gen[i].push_back(t);
            pending[i] = t;
            has_pending[i] = true;
            // the final forward of the last token changes no output: skip it
            if ((int)gen[i].size() >= max_new) done[i] = true;
        }
    }
    for (int i = 0; i < n_seqs; ++i) {
        n_out[i] = (int)gen[i].size();
        for (size_t k = 0; k < gen[i].size(); ++k) out[(size_t)i * max_new + k] = gen[i][k];
    }
    m->pos = 0;
    TRY(sync_pos(m));
    ATLAS_HIP(hipStreamSynchronize(m->st));
    return ATLAS_OK;
}
