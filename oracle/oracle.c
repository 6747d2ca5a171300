/*
 * oracle.c -- CPU restatement of the reference's single-token decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Restates, in plain C:
 *   crates/atlas-quant/src/lib.rs:43-168      Int8Tensor / Int4Tensor
 *   crates/atlas-model/src/lib.rs:335-357     rmsnorm / silu / softmax
 *   crates/atlas-model/src/lib.rs:380-437     RopeCache (YaRN) new / apply
 *   crates/atlas-model/src/lib.rs:487-499     Linear::forward (CPU dot)
 *   crates/atlas-model/src/lib.rs:539-542     Embedding::embed_token (clamp)
 *   crates/atlas-model/src/lib.rs:557-596     KvCache layout
 *   crates/atlas-model/src/lib.rs:648-727     Attention::forward_token
 *   crates/atlas-model/src/lib.rs:911-924     FeedForward::forward
 *   crates/atlas-model/src/lib.rs:982-1006    TransformerBlock::forward_token_cpu
 *   crates/atlas-model/src/lib.rs:1322-1353   OlmoModel::new (scale, SWA wiring)
 *   crates/atlas-model/src/lib.rs:1425-1445   forward_one_hooked
 *   crates/atlas-model/src/lib.rs:1599-1732   generate_with_sampling (greedy)
 *   crates/atlas-model/src/lib.rs:2581-2592   apply_repetition_penalty
 *   crates/atlas-model/src/lib.rs:2701-2706   argmax
 * Compiled with -O2 -ffp-contract=off: every f32 multiply and add is rounded
 * separately and sums run left to right, as Rust's non-fast-math code does.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* generator: SplitMix64 (state += gamma; mix) and Box-Muller in double      */
/* ------------------------------------------------------------------------ */
#define GOLDEN_GAMMA 0x9E3779B97F4A7C15ULL

uint64_t orc_splitmix64_at(uint64_t seed, uint64_t n) {
    uint64_t z = seed + (n + 1) * GOLDEN_GAMMA;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static double u01_open(uint64_t z) {          /* (0, 1] */
    return ((double)(z >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void orc_fill_normal(float* dst, size_t n, uint64_t seed, float mean, float std) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = u01_open(orc_splitmix64_at(seed, i));
        double u2 = u01_open(orc_splitmix64_at(seed, i + 1));
        double r = sqrt(-2.0 * log(u1));
        double a = two_pi * u2;
        dst[i] = (float)(mean + std * r * cos(a));
        if (i + 1 < n) dst[i + 1] = (float)(mean + std * r * sin(a));
    }
}

void orc_fill_uniform(float* dst, size_t n, uint64_t seed, float lo, float hi) {
    for (size_t i = 0; i < n; ++i) {
        double u = (double)(orc_splitmix64_at(seed, i) >> 11) * (1.0 / 9007199254740992.0);
        dst[i] = (float)(lo + (hi - lo) * u);
    }
}

/* ------------------------------------------------------------------------ */
/* formats                                                                   */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

void orc_bf16_from_f32(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = (uint16_t)(f2u(src[i]) >> 16);
}

void orc_bf16_to_f32(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = u2f((uint32_t)src[i] << 16);
}

/* Rust f32::max ignores a NaN operand; |x| of the reference data is never NaN */
static inline float rmax(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    return a > b ? a : b;
}

/* Rust `(v).clamp(lo, hi).round() as i8`: clamp, round half away from zero
 * (C roundf), saturating cast with NaN -> 0.                                 */
static inline int rust_clamp_round(float v, float lo, float hi) {
    if (isnan(v)) return 0;
    float c = v < lo ? lo : (v > hi ? hi : v);
    return (int)roundf(c);
}

/* crates/atlas-quant/src/lib.rs:43-63 */
void orc_int8_quantize(const float* w, size_t rows, size_t cols,
                       int8_t* data, float* scales) {
    for (size_t r = 0; r < rows; ++r) {
        const float* row = w + r * cols;
        float mx = 0.0f;
        for (size_t j = 0; j < cols; ++j) mx = rmax(mx, fabsf(row[j]));
        float s = mx > 0.0f ? mx / 127.0f : 1.0f;
        scales[r] = s;
        float inv = 1.0f / s;
        for (size_t j = 0; j < cols; ++j)
            data[r * cols + j] = (int8_t)rust_clamp_round(row[j] * inv, -127.0f, 127.0f);
    }
}

/* crates/atlas-quant/src/lib.rs:66-75 */
void orc_int8_dequantize(const int8_t* data, const float* scales,
                         size_t rows, size_t cols, float* out) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t j = 0; j < cols; ++j)
            out[r * cols + j] = (float)data[r * cols + j] * scales[r];
}

/* crates/atlas-quant/src/lib.rs:113-145: blocks over the flattened index,
 * even element -> high nibble, odd -> low nibble.                           */
void orc_int4_quantize(const float* w, size_t rows, size_t cols, size_t block,
                       uint8_t* data, float* scales) {
    size_t n = rows * cols;
    size_t n_blocks = (n + block - 1) / block;
    memset(data, 0, (n + 1) / 2);
    for (size_t b = 0; b < n_blocks; ++b) {
        size_t start = b * block;
        size_t end = start + block < n ? start + block : n;
        float mx = 0.0f;
        for (size_t i = start; i < end; ++i) mx = rmax(mx, fabsf(w[i]));
        float s = mx > 0.0f ? mx / 7.0f : 1.0f;
        scales[b] = s;
        float inv = 1.0f / s;
        for (size_t i = start; i < end; ++i) {
            int8_t q = (int8_t)rust_clamp_round(w[i] * inv, -7.0f, 7.0f);
            uint8_t nib = (uint8_t)(q & 0x0F);
            if (i % 2 == 0) data[i / 2] = (uint8_t)((data[i / 2] & 0x0F) | (nib << 4));
            else            data[i / 2] = (uint8_t)((data[i / 2] & 0xF0) | nib);
        }
    }
}

/* crates/atlas-quant/src/lib.rs:148-155 (dequant_nibble) */
static inline float int4_at(const uint8_t* data, const float* scales,
                            size_t i, size_t block) {
    uint8_t byte = data[i / 2];
    uint8_t nib = (i % 2 == 0) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0F);
    int sv = nib >= 8 ? (int)nib - 16 : (int)nib;
    return (float)sv * scales[i / block];
}

/* crates/atlas-quant/src/lib.rs:158-168 */
void orc_int4_dequantize(const uint8_t* data, const float* scales,
                         size_t rows, size_t cols, size_t block, float* out) {
    size_t n = rows * cols;
    for (size_t i = 0; i < n; ++i) out[i] = int4_at(data, scales, i, block);
}

void orc_mat_row(const orc_mat* m, int64_t r, float* out) {
    int64_t cols = m->cols;
    switch (m->fmt) {
    case ORC_F32:
        memcpy(out, (const float*)m->data + r * cols, (size_t)cols * 4);
        break;
    case ORC_BF16: {
        const uint16_t* p = (const uint16_t*)m->data + r * cols;
        for (int64_t j = 0; j < cols; ++j) out[j] = u2f((uint32_t)p[j] << 16);
        break;
    }
    case ORC_INT8: {
        const int8_t* p = (const int8_t*)m->data + r * cols;
        float s = m->scales[r];
        for (int64_t j = 0; j < cols; ++j) out[j] = (float)p[j] * s;
        break;
    }
    case ORC_INT4: {
        const uint8_t* p = (const uint8_t*)m->data;
        for (int64_t j = 0; j < cols; ++j)
            out[j] = int4_at(p, m->scales, (size_t)(r * cols + j), (size_t)m->block);
        break;
    }
    default:
        memset(out, 0, (size_t)cols * 4);
    }
}

/* ------------------------------------------------------------------------ */
/* Linear::forward (crates/atlas-model/src/lib.rs:495-498)                   */
/* ------------------------------------------------------------------------ */
static float dot_seq(const float* a, const float* b, int64_t n) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}

typedef struct {
    const orc_mat* m; const float* x; float* y; int64_t r0, r1;
} lin_job;

static void* lin_worker(void* arg) {
    lin_job* j = (lin_job*)arg;
    float* row = (float*)malloc((size_t)j->m->cols * 4);
    for (int64_t r = j->r0; r < j->r1; ++r) {
        orc_mat_row(j->m, r, row);
        j->y[r] = dot_seq(row, j->x, j->m->cols);
    }
    free(row);
    return NULL;
}

void orc_linear_rows(const orc_mat* m, const float* x, float* y,
                     int64_t r0, int64_t r1, int threads) {
    if (threads <= 1 || r1 - r0 < 64) {
        lin_job j = { m, x, y, r0, r1 };
        lin_worker(&j);
        return;
    }
    if (threads > 64) threads = 64;
    pthread_t th[64];
    lin_job jobs[64];
    int64_t n = r1 - r0;
    for (int t = 0; t < threads; ++t) {
        jobs[t].m = m; jobs[t].x = x; jobs[t].y = y;
        jobs[t].r0 = r0 + n * t / threads;
        jobs[t].r1 = r0 + n * (t + 1) / threads;
        pthread_create(&th[t], NULL, lin_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
}

void orc_linear(const orc_mat* m, const float* x, float* y) {
    orc_linear_rows(m, x, y, 0, m->rows, 1);
}

void orc_linear_batch(const orc_mat* m, const float* x, float* y, int n) {
    for (int i = 0; i < n; ++i)
        orc_linear_rows(m, x + (int64_t)i * m->cols, y + (int64_t)i * m->rows,
                        0, m->rows, 1);
}

/* ------------------------------------------------------------------------ */
/* norms / activations                                                       */
/* ------------------------------------------------------------------------ */
void orc_rmsnorm(float* x, const float* w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; ++i) ss += x[i] * x[i];
    ss = ss / (float)n;
    float inv = 1.0f / sqrtf(ss + eps);
    for (int i = 0; i < n; ++i) x[i] = x[i] * inv * w[i];
}

float orc_silu(float x) { return x / (1.0f + expf(-x)); }

void orc_softmax(float* x, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = rmax(mx, x[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) { x[i] = expf(x[i] - mx); sum += x[i]; }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

void orc_qk_norm(float* x, const float* w, int n_heads, int head_dim, float eps) {
    for (int h = 0; h < n_heads; ++h)
        orc_rmsnorm(x + h * head_dim, w + h * head_dim, head_dim, eps);
}

void orc_add(float* x, const float* y, int n) {
    for (int i = 0; i < n; ++i) x[i] += y[i];
}

/* ------------------------------------------------------------------------ */
/* RopeCache (crates/atlas-model/src/lib.rs:380-437)                         */
/* ------------------------------------------------------------------------ */
void orc_rope_tables(int head_dim, int max_seq, float theta,
                     const orc_rope_scaling* sc, float* cos_tab, float* sin_tab,
                     float* freqs_out) {
    int half = head_dim / 2;
    const float two_pi = 2.0f * 3.14159265358979323846f;
    float* freqs = (float*)malloc((size_t)(half > 0 ? half : 1) * 4);
    for (int i = 0; i < half; ++i) {
        float base = 1.0f / powf(theta, 2.0f * (float)i / (float)head_dim);
        float f = base;
        if (sc && sc->yarn) {
            float wavelength = two_pi / base;
            float low = (float)sc->orig_max_pos / (two_pi * sc->beta_slow);
            float high = (float)sc->orig_max_pos / (two_pi * sc->beta_fast);
            if (wavelength < high) {
                f = base;
            } else if (wavelength > low) {
                f = base / sc->factor;
            } else {
                float alpha = (wavelength - high) / (low - high);
                f = base / (alpha * sc->factor + (1.0f - alpha));
            }
        }
        freqs[i] = f;
        if (freqs_out) freqs_out[i] = f;
    }
    for (int p = 0; p < max_seq; ++p)
        for (int i = 0; i < half; ++i) {
            cos_tab[(size_t)p * half + i] = cosf((float)p * freqs[i]);
            sin_tab[(size_t)p * half + i] = sinf((float)p * freqs[i]);
        }
    free(freqs);
}

void orc_rope_apply(float* x, int head_dim, const float* c, const float* s) {
    int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        float x0 = x[i], x1 = x[i + half];
        x[i] = x0 * c[i] - x1 * s[i];
        x[i + half] = x0 * s[i] + x1 * c[i];
    }
}

/* ------------------------------------------------------------------------ */
/* Attention (crates/atlas-model/src/lib.rs:689-721)                         */
/* ------------------------------------------------------------------------ */
void orc_attention(const float* q, const float* k_cache, const float* v_cache,
                   float* out, int n_heads, int n_kv_heads, int head_dim,
                   int pos, float scale, int window) {
    int group = n_heads / n_kv_heads;
    float* sc = (float*)malloc((size_t)(pos + 1) * 4);
    memset(out, 0, (size_t)n_heads * head_dim * 4);
    for (int h = 0; h < n_heads; ++h) {
        int kvh = h / group;
        const float* qh = q + (size_t)h * head_dim;
        for (int t = 0; t <= pos; ++t) {
            if (window > 0 && pos - t >= window) { sc[t] = -INFINITY; continue; }
            const float* kt = k_cache + ((size_t)t * n_kv_heads + kvh) * head_dim;
            sc[t] = dot_seq(qh, kt, head_dim) * scale;
        }
        orc_softmax(sc, pos + 1);
        float* oh = out + (size_t)h * head_dim;
        for (int t = 0; t <= pos; ++t) {
            const float* vt = v_cache + ((size_t)t * n_kv_heads + kvh) * head_dim;
            float a = sc[t];
            for (int i = 0; i < head_dim; ++i) oh[i] += a * vt[i];
        }
    }
    free(sc);
}

/* ------------------------------------------------------------------------ */
/* OlmoModel CPU path                                                        */
/* ------------------------------------------------------------------------ */
typedef struct { float* k; float* v; } orc_kv;

struct orc_model {
    orc_config cfg;
    orc_mat embed, lm_head;
    orc_layer* layers;
    const float* final_norm;
    uint8_t* sliding;
    float* cos_tab; float* sin_tab;
    float scale;
    int threads;
    int n_slots, slot;
    orc_kv* kv;            /* [n_slots * n_layers] */
    int* pos;              /* [n_slots] */
    /* scratch */
    float *x, *q, *k, *v, *att, *o, *gate, *up, *hid, *ffo;
};

orc_model* orc_model_new_slots(const orc_config* cfg, const orc_mat* embed,
                               const orc_layer* layers, const float* final_norm,
                               const orc_mat* lm_head, int threads, int n_slots) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->cfg = *cfg;
    m->embed = *embed;
    m->lm_head = *lm_head;
    m->final_norm = final_norm;
    m->threads = threads < 1 ? 1 : threads;
    int L = cfg->n_layers, d = cfg->d_model, hd = cfg->d_model / cfg->n_heads;
    int kvd = cfg->n_kv_heads * hd;
    m->layers = (orc_layer*)malloc(sizeof(orc_layer) * (size_t)L);
    memcpy(m->layers, layers, sizeof(orc_layer) * (size_t)L);
    m->sliding = (uint8_t*)calloc((size_t)L, 1);
    if (cfg->layer_sliding) memcpy(m->sliding, cfg->layer_sliding, (size_t)L);
    m->cfg.layer_sliding = m->sliding;
    int half = hd / 2;
    m->cos_tab = (float*)malloc((size_t)cfg->max_seq * half * 4);
    m->sin_tab = (float*)malloc((size_t)cfg->max_seq * half * 4);
    orc_rope_tables(hd, cfg->max_seq, cfg->rope_theta, &cfg->rope,
                    m->cos_tab, m->sin_tab, NULL);
    /* lib.rs:632 then 1331-1335 */
    m->scale = 1.0f / sqrtf((float)hd);
    float af = cfg->rope.yarn ? cfg->rope.attn_factor : 1.0f;
    if (fabsf(af - 1.0f) > 1e-6f) m->scale *= af;
    m->n_slots = n_slots < 1 ? 1 : n_slots;
    m->kv = (orc_kv*)calloc((size_t)m->n_slots * L, sizeof(orc_kv));
    for (int i = 0; i < m->n_slots * L; ++i) {
        m->kv[i].k = (float*)calloc((size_t)cfg->max_seq * kvd, 4);
        m->kv[i].v = (float*)calloc((size_t)cfg->max_seq * kvd, 4);
    }
    m->pos = (int*)calloc((size_t)m->n_slots, sizeof(int));
    int big = cfg->ffn_hidden > d ? cfg->ffn_hidden : d;
    m->x = (float*)malloc((size_t)d * 4);
    m->q = (float*)malloc((size_t)d * 4);
    m->k = (float*)malloc((size_t)kvd * 4);
    m->v = (float*)malloc((size_t)kvd * 4);
    m->att = (float*)malloc((size_t)d * 4);
    m->o = (float*)malloc((size_t)d * 4);
    m->gate = (float*)malloc((size_t)big * 4);
    m->up = (float*)malloc((size_t)big * 4);
    m->hid = (float*)malloc((size_t)big * 4);
    m->ffo = (float*)malloc((size_t)d * 4);
    return m;
}

orc_model* orc_model_new(const orc_config* cfg, const orc_mat* embed,
                         const orc_layer* layers, const float* final_norm,
                         const orc_mat* lm_head, int threads) {
    return orc_model_new_slots(cfg, embed, layers, final_norm, lm_head, threads, 1);
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    for (int i = 0; i < m->n_slots * m->cfg.n_layers; ++i) { free(m->kv[i].k); free(m->kv[i].v); }
    free(m->kv); free(m->pos); free(m->layers); free(m->sliding);
    free(m->cos_tab); free(m->sin_tab);
    free(m->x); free(m->q); free(m->k); free(m->v); free(m->att); free(m->o);
    free(m->gate); free(m->up); free(m->hid); free(m->ffo);
    free(m);
}

void orc_model_select_slot(orc_model* m, int slot) {
    if (slot >= 0 && slot < m->n_slots) m->slot = slot;
}

/* reset(): pos = 0, caches not zeroed (lib.rs:1389-1392, 872-880) */
void orc_model_reset(orc_model* m) { m->pos[m->slot] = 0; }
int orc_model_pos(const orc_model* m) { return m->pos[m->slot]; }

/* Test seeding (no reference counterpart): cache rows [pos0, pos0 + n) of one
 * layer of the current slot, [n][n_kv * hd] each, copied in; then the
 * position.  Lets a parity test start decoding at a long position without
 * feeding every earlier token through both models. */
int orc_model_set_kv_rows(orc_model* m, int layer, int pos0, int n, const float* k,
                          const float* v) {
    int hd = m->cfg.d_model / m->cfg.n_heads, kvd = m->cfg.n_kv_heads * hd;
    if (layer < 0 || layer >= m->cfg.n_layers || pos0 < 0 || n < 0 || pos0 + n > m->cfg.max_seq)
        return -1;
    orc_kv* c = &m->kv[m->slot * m->cfg.n_layers + layer];
    memcpy(c->k + (size_t)pos0 * kvd, k, (size_t)n * kvd * 4);
    memcpy(c->v + (size_t)pos0 * kvd, v, (size_t)n * kvd * 4);
    return 0;
}

int orc_model_set_pos(orc_model* m, int pos) {
    if (pos < 0 || pos >= m->cfg.max_seq) return -1;
    m->pos[m->slot] = pos;
    return 0;
}
float orc_model_attn_scale(const orc_model* m) { return m->scale; }

static void lin(orc_model* m, const orc_mat* w, const float* x, float* y) {
    orc_linear_rows(w, x, y, 0, w->rows, m->threads);
}

/* Attention::forward_token: lib.rs:648-727 */
static void attn_forward(orc_model* m, int li, const float* x, int pos, float* result) {
    const orc_config* c = &m->cfg;
    const orc_layer* L = &m->layers[li];
    int hd = c->d_model / c->n_heads, half = hd / 2;
    orc_kv* kv = &m->kv[m->slot * c->n_layers + li];
    lin(m, &L->wq, x, m->q);
    lin(m, &L->wk, x, m->k);
    lin(m, &L->wv, x, m->v);
    if (L->q_norm) orc_qk_norm(m->q, L->q_norm, c->n_heads, hd, 1e-6f);
    if (L->k_norm) orc_qk_norm(m->k, L->k_norm, c->n_kv_heads, hd, 1e-6f);
    const float* cr = m->cos_tab + (size_t)pos * half;
    const float* sr = m->sin_tab + (size_t)pos * half;
    for (int h = 0; h < c->n_heads; ++h) orc_rope_apply(m->q + h * hd, hd, cr, sr);
    for (int h = 0; h < c->n_kv_heads; ++h) orc_rope_apply(m->k + h * hd, hd, cr, sr);
    size_t kvd = (size_t)c->n_kv_heads * hd;
    memcpy(kv->k + (size_t)pos * kvd, m->k, kvd * 4);
    memcpy(kv->v + (size_t)pos * kvd, m->v, kvd * 4);
    int window = (m->sliding[li] && c->sliding_window > 0) ? c->sliding_window : 0;
    orc_attention(m->q, kv->k, kv->v, m->att, c->n_heads, c->n_kv_heads, hd,
                  pos, m->scale, window);
    lin(m, &L->wo, m->att, result);
}

/* FeedForward::forward: lib.rs:911-924 */
static void ffn_forward(orc_model* m, int li, const float* x, float* out) {
    const orc_layer* L = &m->layers[li];
    int h = (int)L->w_gate.rows;
    lin(m, &L->w_gate, x, m->gate);
    lin(m, &L->w_up, x, m->up);
    for (int i = 0; i < h; ++i) m->hid[i] = orc_silu(m->gate[i]) * m->up[i];
    lin(m, &L->w_down, m->hid, out);
}

/* TransformerBlock::forward_token_cpu: lib.rs:982-1006 */
static void block_forward(orc_model* m, int li, float* x, int pos) {
    const orc_config* c = &m->cfg;
    const orc_layer* L = &m->layers[li];
    int d = c->d_model;
    if (c->post_norm) {
        attn_forward(m, li, x, pos, m->o);
        orc_rmsnorm(m->o, L->attn_norm, d, c->rms_eps);
        orc_add(x, m->o, d);
        ffn_forward(m, li, x, m->ffo);
        orc_rmsnorm(m->ffo, L->ffn_norm, d, c->rms_eps);
        orc_add(x, m->ffo, d);
    } else {
        float* xn = (float*)malloc((size_t)d * 4);
        memcpy(xn, x, (size_t)d * 4);
        orc_rmsnorm(xn, L->attn_norm, d, c->rms_eps);
        attn_forward(m, li, xn, pos, m->o);
        orc_add(x, m->o, d);
        memcpy(xn, x, (size_t)d * 4);
        orc_rmsnorm(xn, L->ffn_norm, d, c->rms_eps);
        ffn_forward(m, li, xn, m->ffo);
        orc_add(x, m->ffo, d);
        free(xn);
    }
}

/* forward_one_hooked: lib.rs:1425-1445; embed_token clamps: lib.rs:539-542 */
void orc_model_forward_one(orc_model* m, uint32_t token, float* logits,
                           float* hidden_out) {
    const orc_config* c = &m->cfg;
    int d = c->d_model;
    int pos = m->pos[m->slot];
    m->pos[m->slot] += 1;
    int64_t id = token < (uint32_t)c->vocab ? (int64_t)token : (int64_t)c->vocab - 1;
    orc_mat_row(&m->embed, id, m->x);
    for (int li = 0; li < c->n_layers; ++li) {
        block_forward(m, li, m->x, pos);
        if (hidden_out) memcpy(hidden_out + (size_t)li * d, m->x, (size_t)d * 4);
    }
    orc_rmsnorm(m->x, m->final_norm, d, c->rms_eps);
    lin(m, &m->lm_head, m->x, logits);
}

/* argmax: Iterator::max_by keeps the LAST of equal maxima (lib.rs:2701-2706).
 * partial_cmp == None (NaN) counts as Equal, which also moves to the later
 * element.                                                                   */
int orc_argmax(const float* x, int n) {
    if (n <= 0) return 0;
    int best = 0;
    for (int i = 1; i < n; ++i) {
        float a = x[best], b = x[i];
        /* max_by replaces the running max unless cmp(best, cur) == Greater */
        int greater = (!isnan(a) && !isnan(b) && a > b);
        if (!greater) best = i;
    }
    return best;
}

void orc_repetition_penalty(float* logits, int n, const uint32_t* toks,
                            int n_toks, float theta) {
    for (int i = 0; i < n_toks; ++i) {
        uint32_t t = toks[i];
        if (t < (uint32_t)n) {
            if (logits[t] > 0.0f) logits[t] /= theta;
            else logits[t] *= theta;
        }
    }
}

/* generate_with_sampling, greedy branch: lib.rs:1599-1646, 1713-1729 */
int orc_generate_greedy(orc_model* m, const uint32_t* prompt, int n_prompt,
                        int max_new, const uint32_t* suppress, int n_suppress,
                        float rep_penalty, int rep_window, int64_t eos,
                        const uint32_t* extra_stop, int n_extra,
                        uint32_t* out) {
    int V = m->cfg.vocab;
    float* last = (float*)calloc((size_t)V, 4);
    float* logits = (float*)malloc((size_t)V * 4);
    orc_model_reset(m);
    for (int i = 0; i < n_prompt; ++i) orc_model_forward_one(m, prompt[i], last, NULL);
    int n_out = 0;
    for (int step = 0; step < max_new; ++step) {
        memcpy(logits, last, (size_t)V * 4);
        if (step == 0)
            for (int i = 0; i < n_suppress; ++i)
                if (suppress[i] < (uint32_t)V) logits[suppress[i]] = -INFINITY;
        if (rep_penalty != 1.0f && n_out > 0) {
            int start = n_out > rep_window ? n_out - rep_window : 0;
            orc_repetition_penalty(logits, V, out + start, n_out - start, rep_penalty);
        }
        uint32_t tok = (uint32_t)orc_argmax(logits, V);
        if (eos >= 0 && (int64_t)tok == eos) break;
        int stop = 0;
        for (int i = 0; i < n_extra; ++i) if (extra_stop[i] == tok) stop = 1;
        if (stop) break;
        out[n_out++] = tok;
        orc_model_forward_one(m, tok, last, NULL);
    }
    free(last); free(logits);
    return n_out;
}


/* ---- temperature sampling ------------------------------------------------ */
float orc_rng_next(uint64_t* state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (float)(x >> 33) / (float)(1ULL << 31);
}

void orc_frequency_penalty(float* logits, int n, const uint32_t* toks,
                           const uint32_t* counts, int n_toks, float penalty) {
    for (int i = 0; i < n_toks; ++i)
        if (toks[i] < (uint32_t)n) logits[toks[i]] -= penalty * (float)counts[i];
}

void orc_presence_penalty(float* logits, int n, const uint32_t* toks, int n_toks,
                          float penalty) {
    for (int i = 0; i < n_toks; ++i)
        if (toks[i] < (uint32_t)n) logits[toks[i]] -= penalty;
}

static int cmp_desc_f32(const void* a, const void* b) {
    float x = *(const float*)a, y = *(const float*)b;
    return (x < y) - (x > y);
}

void orc_top_k(float* logits, int n, int k) {
    if (k <= 0 || k >= n) return;
    float* sorted = (float*)malloc((size_t)n * 4);
    memcpy(sorted, logits, (size_t)n * 4);
    qsort(sorted, (size_t)n, 4, cmp_desc_f32);
    float th = sorted[k - 1];
    free(sorted);
    int at_or_above = 0, above = 0;
    for (int i = 0; i < n; ++i) {
        if (logits[i] >= th) ++at_or_above;
        if (logits[i] > th) ++above;
    }
    if (at_or_above <= k) {
        for (int i = 0; i < n; ++i) if (logits[i] < th) logits[i] = -INFINITY;
    } else {
        int need = k - above, kept = 0;
        for (int i = 0; i < n; ++i) {
            if (logits[i] > th) continue;
            if (logits[i] == th && kept < need) { ++kept; continue; }
            logits[i] = -INFINITY;
        }
    }
}

typedef struct { int idx; float p; } orc_ip;

/* probability descending; equal probabilities keep index order */
static int cmp_ip(const void* a, const void* b) {
    const orc_ip* x = (const orc_ip*)a;
    const orc_ip* y = (const orc_ip*)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return (x->idx > y->idx) - (x->idx < y->idx);
}

void orc_top_p(float* logits, int n, float p) {
    if (n <= 0) return;
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = rmax(mx, logits[i]);
    orc_ip* pr = (orc_ip*)malloc((size_t)n * sizeof(orc_ip));
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) { pr[i].idx = i; pr[i].p = expf(logits[i] - mx); }
    for (int i = 0; i < n; ++i) sum += pr[i].p;
    if (sum <= 0.0f) { free(pr); return; }
    for (int i = 0; i < n; ++i) pr[i].p /= sum;
    qsort(pr, (size_t)n, sizeof(orc_ip), cmp_ip);
    float cum = 0.0f;
    int cut = n;
    for (int i = 0; i < n; ++i) {
        cum += pr[i].p;
        if (cum >= p) { cut = i + 1; break; }
    }
    for (int i = cut; i < n; ++i) logits[pr[i].idx] = -INFINITY;
    free(pr);
}

void orc_min_p(float* logits, int n, float min_p) {
    if (min_p <= 0.0f) return;
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = rmax(mx, logits[i]);
    float th = mx + logf(min_p);
    for (int i = 0; i < n; ++i) if (logits[i] < th) logits[i] = -INFINITY;
}

int orc_sample_from_probs(const float* probs, int n, float rand) {
    float cum = 0.0f;
    for (int i = 0; i < n; ++i) {
        cum += probs[i];
        if (rand < cum) return i;
    }
    return n - 1;
}

int orc_sample_step(const float* logits_in, int n, const uint32_t* hist, int n_hist, int step,
                    const orc_sampling* s, uint64_t* rng) {
    float* lg = (float*)malloc((size_t)n * 4);
    memcpy(lg, logits_in, (size_t)n * 4);
    /* step-0 suppression and the repetition penalty: lib.rs:1627-1644, 1649-1666 */
    if (step == 0)
        for (int i = 0; i < s->n_suppress; ++i)
            if (s->suppress[i] < (uint32_t)n) lg[s->suppress[i]] = -INFINITY;
    if (s->repetition_penalty != 1.0f && n_hist > 0) {
        int start = n_hist > s->repetition_window ? n_hist - s->repetition_window : 0;
        orc_repetition_penalty(lg, n, hist + start, n_hist - start, s->repetition_penalty);
    }
    int tok;
    if (s->temperature <= 0.0f || s->temperature < 1e-6f) {
        tok = orc_argmax(lg, n);                       /* lib.rs:1646 */
    } else {
        /* frequency penalty over (token, count) in first-seen order: lib.rs:1669-1680 */
        if (s->frequency_penalty != 0.0f && n_hist > 0) {
            uint32_t* tk = (uint32_t*)malloc((size_t)n_hist * 4);
            uint32_t* ct = (uint32_t*)malloc((size_t)n_hist * 4);
            int nu = 0;
            for (int i = 0; i < n_hist; ++i) {
                int j = 0;
                while (j < nu && tk[j] != hist[i]) ++j;
                if (j < nu) ++ct[j];
                else { tk[nu] = hist[i]; ct[nu] = 1; ++nu; }
            }
            orc_frequency_penalty(lg, n, tk, ct, nu, s->frequency_penalty);
            free(tk); free(ct);
        }
        /* presence penalty over the sorted, deduplicated history: lib.rs:1683-1688 */
        if (s->presence_penalty != 0.0f && n_hist > 0) {
            uint32_t* seen = (uint32_t*)malloc((size_t)n_hist * 4);
            memcpy(seen, hist, (size_t)n_hist * 4);
            for (int i = 1; i < n_hist; ++i)                 /* insertion sort */
                for (int j = i; j > 0 && seen[j - 1] > seen[j]; --j) {
                    uint32_t t = seen[j]; seen[j] = seen[j - 1]; seen[j - 1] = t;
                }
            int nu = 0;
            for (int i = 0; i < n_hist; ++i)
                if (nu == 0 || seen[nu - 1] != seen[i]) seen[nu++] = seen[i];
            orc_presence_penalty(lg, n, seen, nu, s->presence_penalty);
            free(seen);
        }
        for (int i = 0; i < n; ++i) lg[i] /= s->temperature;   /* lib.rs:1691-1693 */
        if (s->top_k > 0) orc_top_k(lg, n, s->top_k);             /* lib.rs:1696-1698 */
        if (s->top_p < 1.0f) orc_top_p(lg, n, s->top_p);          /* lib.rs:1701-1703 */
        if (s->min_p > 0.0f) orc_min_p(lg, n, s->min_p);          /* lib.rs:1706-1708 */
        orc_softmax(lg, n);                                      /* lib.rs:1711 */
        tok = orc_sample_from_probs(lg, n, orc_rng_next(rng));
    }
    free(lg);
    return tok;
}

int orc_generate_sampled(orc_model* m, const uint32_t* prompt, int n_prompt, int max_new,
                         const orc_sampling* s, uint64_t seed, int64_t eos,
                         const uint32_t* extra_stop, int n_extra, uint32_t* out) {
    int V = m->cfg.vocab;
    uint64_t rng = seed | 1ULL;
    float* last = (float*)calloc((size_t)V, 4);
    orc_model_reset(m);
    for (int i = 0; i < n_prompt; ++i) orc_model_forward_one(m, prompt[i], last, NULL);
    int n_out = 0;
    for (int step = 0; step < max_new; ++step) {
        uint32_t tok = (uint32_t)orc_sample_step(last, V, out, n_out, step, s, &rng);
        if (eos >= 0 && (int64_t)tok == eos) break;              /* lib.rs:1713-1718 */
        int stop = 0;
        for (int i = 0; i < n_extra; ++i) if (extra_stop[i] == tok) stop = 1;
        if (stop) break;
        out[n_out++] = tok;
        orc_model_forward_one(m, tok, last, NULL);
    }
    free(last);
    return n_out;
}
