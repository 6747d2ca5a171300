/*
 * oracle.h -- CPU restatement of the reference's decode-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product (atlas_amd/) never links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative
 * to the web3guru888/ATLAS source tree).  Build: oracle/Makefile
 * (gcc -O2 -ffp-contract=off, no fast-math), so that f32 products and sums
 * are rounded one at a time in source order, as the reference's Rust does.
 */
#ifndef ATLAS_ORACLE_H
#define ATLAS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic input generator (SplitMix64 + Box-Muller) --------------- */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t n);      /* n-th output   */
void orc_fill_normal(float* dst, size_t n, uint64_t seed, float mean, float std);
void orc_fill_uniform(float* dst, size_t n, uint64_t seed, float lo, float hi);

/* ---- formats ------------------------------------------------------------- */
/* f32 -> bf16 by truncation: crates/atlas-model/src/lib.rs:2274             */
void orc_bf16_from_f32(const float* src, uint16_t* dst, size_t n);
/* bf16 -> f32 = bits << 16: kernels/matmul.cu:321-323                        */
void orc_bf16_to_f32(const uint16_t* src, float* dst, size_t n);
/* Int8Tensor::quantize / dequantize: crates/atlas-quant/src/lib.rs:43-75     */
void orc_int8_quantize(const float* w, size_t rows, size_t cols,
                       int8_t* data, float* scales);
void orc_int8_dequantize(const int8_t* data, const float* scales,
                         size_t rows, size_t cols, float* out);
/* Int4Tensor::quantize / dequantize: crates/atlas-quant/src/lib.rs:113-168   */
void orc_int4_quantize(const float* w, size_t rows, size_t cols, size_t block,
                       uint8_t* data, float* scales);
void orc_int4_dequantize(const uint8_t* data, const float* scales,
                         size_t rows, size_t cols, size_t block, float* out);

/* ---- weight matrix view (any storage format) ----------------------------- */
enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_INT8 = 2, ORC_INT4 = 3 };
typedef struct {
    int fmt;                 /* ORC_*                                        */
    const void* data;        /* f32 / u16 / i8 / packed u8                   */
    const float* scales;     /* int8: [rows]; int4: [ceil(rows*cols/block)]  */
    int64_t rows, cols;      /* out x in, row-major                          */
    int64_t block;           /* int4 block size                              */
} orc_mat;

/* Dequantise row r of m into out[cols] (values identical to the reference's
 * full dequantize of that row).                                              */
void orc_mat_row(const orc_mat* m, int64_t r, float* out);

/* Linear::forward CPU dot: crates/atlas-model/src/lib.rs:487-499.
 * y[o] = sum_k W[o,k]*x[k], f32, left to right, starting at 0.               */
void orc_linear(const orc_mat* m, const float* x, float* y);
/* Same, rows [r0, r1) only, threads = worker count (1 = scalar).  Rows are
 * independent, so the result is bit-identical for any thread count.         */
void orc_linear_rows(const orc_mat* m, const float* x, float* y,
                     int64_t r0, int64_t r1, int threads);
/* Ragged batch: y[n*rows + o] for n < N input rows x[n*cols ...].             */
void orc_linear_batch(const orc_mat* m, const float* x, float* y, int n);

/* ---- elementwise / norm -------------------------------------------------- */
/* rmsnorm_inplace: crates/atlas-model/src/lib.rs:335-342                     */
void orc_rmsnorm(float* x, const float* w, int n, float eps);
/* silu: lib.rs:346-348                                                       */
float orc_silu(float x);
/* softmax_inplace: lib.rs:351-357                                            */
void orc_softmax(float* x, int n);
/* per-head QK-norm (eps 1e-6 at the call site): lib.rs:660-672               */
void orc_qk_norm(float* x, const float* w, int n_heads, int head_dim, float eps);
/* residual add of a normed branch (post-norm): lib.rs:985-993                */
void orc_add(float* x, const float* y, int n);

/* ---- RoPE / YaRN ------------------------------------------------------------ */
typedef struct {
    int   yarn;              /* 0 = RopeScaling::None                        */
    float factor;
    int   orig_max_pos;
    float attn_factor;
    float beta_fast, beta_slow;
} orc_rope_scaling;
/* RopeCache::new: lib.rs:380-423.  cos/sin are [max_seq x head_dim/2].       */
void orc_rope_tables(int head_dim, int max_seq, float theta,
                     const orc_rope_scaling* sc, float* cos_tab, float* sin_tab,
                     float* freqs_out /* [head_dim/2] or NULL */);
/* RopeCache::apply (rotate-half): lib.rs:428-437                             */
void orc_rope_apply(float* x, int head_dim, const float* cos_row,
                    const float* sin_row);

/* ---- attention ----------------------------------------------------------- */
/* Attention::forward_token scores/softmax/PV part: lib.rs:689-721.
 * q: [n_heads*hd] (after QK-norm + RoPE); caches [max_seq][n_kv][hd];
 * window 0 = full attention.  out: [n_heads*hd].                             */
void orc_attention(const float* q, const float* k_cache, const float* v_cache,
                   float* out, int n_heads, int n_kv_heads, int head_dim,
                   int pos, float scale, int window);

/* ---- full model (OlmoModel CPU path) ------------------------------------ */
typedef struct {
    int vocab, d_model, n_layers, n_heads, n_kv_heads, ffn_hidden, max_seq;
    float rope_theta, rms_eps;
    orc_rope_scaling rope;
    int sliding_window;              /* 0 = none                             */
    const uint8_t* layer_sliding;    /* [n_layers] 1 = Sliding (may be NULL) */
    int post_norm;                   /* 1 = OLMo-2/3 post-norm               */
} orc_config;

typedef struct {
    orc_mat wq, wk, wv, wo, w_gate, w_up, w_down;
    const float* attn_norm;          /* [d]                                  */
    const float* ffn_norm;           /* [d]                                  */
    const float* q_norm;             /* [n_heads*hd] or NULL                 */
    const float* k_norm;             /* [n_kv*hd] or NULL                    */
} orc_layer;

typedef struct orc_model orc_model;

/* Weights are referenced, not copied: the caller keeps them alive. */
orc_model* orc_model_new(const orc_config* cfg, const orc_mat* embed,
                         const orc_layer* layers, const float* final_norm,
                         const orc_mat* lm_head, int threads);
void  orc_model_free(orc_model* m);
void  orc_model_reset(orc_model* m);                  /* lib.rs:1389-1392   */
int   orc_model_pos(const orc_model* m);
float orc_model_attn_scale(const orc_model* m);       /* lib.rs:1331-1335   */
/* forward_one_hooked with a recording hook: lib.rs:1425-1445.  hidden_out
 * (may be NULL) receives the post-residual hidden state after every layer,
 * [n_layers x d].  logits: [vocab].                                          */
void  orc_model_forward_one(orc_model* m, uint32_t token, float* logits,
                            float* hidden_out);
/* Ragged step: token[i] at position pos_i of independent sequence i uses its
 * own KV cache.  Sequences are addressed by slot (0..n_slots-1) of a model
 * created with orc_model_new_slots.                                          */
orc_model* orc_model_new_slots(const orc_config* cfg, const orc_mat* embed,
                               const orc_layer* layers, const float* final_norm,
                               const orc_mat* lm_head, int threads, int n_slots);
void  orc_model_select_slot(orc_model* m, int slot);
/* Test seeding: copy n cache rows ([n][n_kv*hd] K and V) of one layer of the
 * current slot in at positions pos0.., and set the position; -1 when out of
 * range.  No reference counterpart. */
int   orc_model_set_kv_rows(orc_model* m, int layer, int pos0, int n, const float* k,
                            const float* v);
int   orc_model_set_pos(orc_model* m, int pos);

/* ---- token choice / greedy loop ----------------------------------------- */
/* argmax with Rust max_by semantics (last maximal index): lib.rs:2701-2706  */
int   orc_argmax(const float* x, int n);
/* apply_repetition_penalty: lib.rs:2581-2592                                 */
void  orc_repetition_penalty(float* logits, int n, const uint32_t* toks,
                             int n_toks, float theta);
/* generate_with_sampling, greedy branch: lib.rs:1599-1732.  Returns the
 * number of generated tokens written to out (EOS excluded); eos < 0 = none.
 * Optional: logits_out receives [max_new x vocab] pre-choice logits.        */
int   orc_generate_greedy(orc_model* m, const uint32_t* prompt, int n_prompt,
                          int max_new, const uint32_t* suppress, int n_suppress,
                          float rep_penalty, int rep_window, int64_t eos,
                          const uint32_t* extra_stop, int n_extra,
                          uint32_t* out);

/* ---- temperature sampling (generate_with_sampling's sampled branch) ----- */
/* Rng::next_f32, XorShift64: lib.rs:1208-1214 (state seeded as seed | 1,
 * Rng::from_seed lib.rs:1203-1206)                                          */
float orc_rng_next(uint64_t* state);
/* apply_frequency_penalty lib.rs:2598-2605 (counts in first-seen order),
 * apply_presence_penalty lib.rs:2610-2617                                    */
void  orc_frequency_penalty(float* logits, int n, const uint32_t* toks,
                            const uint32_t* counts, int n_toks, float penalty);
void  orc_presence_penalty(float* logits, int n, const uint32_t* toks, int n_toks,
                           float penalty);
/* apply_top_k lib.rs:2658-2689, apply_top_p lib.rs:2625-2655 (the
 * reference's unstable sort leaves the order of exactly equal
 * probabilities unspecified; this one keeps index order), apply_min_p
 * lib.rs:2692-2699, sample_from_probs lib.rs:2710-2717                      */
void  orc_top_k(float* logits, int n, int k);
void  orc_top_p(float* logits, int n, float p);
void  orc_min_p(float* logits, int n, float min_p);
int   orc_sample_from_probs(const float* probs, int n, float rand);

typedef struct {
    float temperature, repetition_penalty;
    int repetition_window;
    float frequency_penalty, presence_penalty, top_p;
    int top_k;
    float min_p;
    const uint32_t* suppress;
    int n_suppress;
} orc_sampling;

/* One token choice of generate_with_sampling (lib.rs:1623-1711): step-0
 * suppression, repetition / frequency / presence penalties over `hist`,
 * greedy argmax when temperature <= 0 or < 1e-6, else temperature, top-k,
 * top-p, min-p, softmax and a draw from *rng.  logits is copied.            */
int   orc_sample_step(const float* logits, int n, const uint32_t* hist, int n_hist, int step,
                      const orc_sampling* s, uint64_t* rng);
/* The whole loop (lib.rs:1599-1732) with an explicit RNG seed (state =
 * seed | 1); returns the generated count (EOS / stop tokens end it).        */
int   orc_generate_sampled(orc_model* m, const uint32_t* prompt, int n_prompt, int max_new,
                           const orc_sampling* s, uint64_t seed, int64_t eos,
                           const uint32_t* extra_stop, int n_extra, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
