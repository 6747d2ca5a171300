/*
 * atlas_engine.h -- C ABI of the MI355X decode engine: the `OlmoModel` /
 * `InferEngine` surface of the reference's decode path.
 *
 * Reference counterparts:
 *   ModelConfig            crates/atlas-model/src/lib.rs:58-84, 253-269
 *   SamplingConfig         crates/atlas-model/src/lib.rs:1223-1295
 *   OlmoModel::new / init_gpu_resources / reset      lib.rs:1322-1392
 *   OlmoModel::forward_one_gpu                       lib.rs:1463-1505
 *   OlmoModel::forward_one_hooked                    lib.rs:1425-1445
 *   OlmoModel::generate_with_sampling                lib.rs:1599-1732
 *   OlmoModel::generate_with_sampling_hooked         lib.rs:1745-1846
 *   OlmoModel::generate_streaming                    lib.rs:1853-1955
 *   InferEngine::generate / StigmergicHook / PheromoneDeposit
 *       crates/atlas-infer/src/engine.rs:51-163, crates/atlas-infer/src/hook.rs:58-100
 * The ragged batch (atlas_model_generate_batch) has no reference counterpart:
 * the reference decodes one sequence at a time (lib.rs:1298-1318).
 *
 * All entry points return 0 or a negative ATLAS_E* code (atlas_kernels.h);
 * atlas_last_error() has the message.
 */
#ifndef ATLAS_ENGINE_H
#define ATLAS_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "atlas_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct atlas_model atlas_model;

typedef struct {
    int vocab, d_model, n_layers, n_heads, n_kv_heads, ffn_hidden, max_seq;
    float rope_theta, rms_eps;
    /* RopeScaling::Yarn (lib.rs:35-53); yarn = 0 is RopeScaling::None */
    int yarn;
    float yarn_factor;
    int yarn_orig_max_pos;
    float yarn_attn_factor, yarn_beta_fast, yarn_beta_slow;
    int sliding_window;              /* 0 = None                                */
    const uint8_t* layer_sliding;    /* [n_layers], 1 = LayerType::Sliding      */
    int post_norm;                   /* 1 = OLMo-2/3 post-norm, 0 = Llama       */
    int qk_norm;                     /* 1 = per-head QK-norm weights            */
    int weight_format;               /* ATLAS_W_BF16 / ATLAS_W_INT8 / ATLAS_W_INT4 */
    int int4_block;                  /* Int4Tensor block size (multiple of 32)  */
    int max_batch;                   /* KV slots for the ragged batch (>= 1)    */
} atlas_model_config;

/* tensor kinds for atlas_model_set_tensor / atlas_model_get_tensor */
enum {
    ATLAS_T_WQ = 0, ATLAS_T_WK = 1, ATLAS_T_WV = 2, ATLAS_T_WO = 3,
    ATLAS_T_W_GATE = 4, ATLAS_T_W_UP = 5, ATLAS_T_W_DOWN = 6,
    ATLAS_T_ATTN_NORM = 7, ATLAS_T_FFN_NORM = 8, ATLAS_T_Q_NORM = 9, ATLAS_T_K_NORM = 10,
    ATLAS_T_EMBED = 11, ATLAS_T_LM_HEAD = 12, ATLAS_T_FINAL_NORM = 13
};

typedef struct {
    float temperature;               /* <= 0 or < 1e-6: greedy                  */
    float repetition_penalty;        /* 1 = off                                 */
    int repetition_window;
    float frequency_penalty, presence_penalty;
    float top_p;                     /* 1 = off                                 */
    int top_k;                       /* 0 = off                                 */
    float min_p;                     /* 0 = off                                 */
    const uint32_t* suppress_initial_tokens;
    int n_suppress;
    int64_t eos_token_id;            /* < 0 = none                              */
    const uint32_t* extra_stop_tokens;
    int n_extra_stop;
    uint64_t rng_seed;               /* 0 = seed from the clock, as the reference */
} atlas_sampling;

/* Per-layer hook: return 1 and set *delta for Some(delta), 0 for None. */
typedef int (*atlas_hook_fn)(void* user, int layer_idx, const float* hidden, int d_model,
                             float* delta);

atlas_model* atlas_model_create(const atlas_model_config* cfg);
void atlas_model_destroy(atlas_model* m);

/* Upload one tensor.  Matrices come in the model's weight_format: bf16 bits;
 * or int8 data + per-row scales; or int4 packed data + per-block scales
 * (Int4Tensor layout).  Norm vectors are f32; the embedding is bf16 bits.
 * layer is ignored for EMBED / LM_HEAD / FINAL_NORM.                        */
int atlas_model_set_tensor(atlas_model* m, int kind, int layer, const void* data,
                           const float* scales);
/* Download one tensor in the same layout. */
int atlas_model_get_tensor(atlas_model* m, int kind, int layer, void* data, float* scales);

/* Upload one tensor from device memory: numel f32 (ATLAS_W_F32) or bf16
 * (ATLAS_W_BF16) elements in the reference's row-major layout, converted on
 * the device to the model's weight_format (bf16 by truncation, lib.rs:2274;
 * int8 / int4 by the atlas-quant rules) and placed into the model's layout.
 * The checkpoint loader's building block; no reference counterpart (the
 * reference converts on the host, lib.rs:2271-2279).  With a scratch the
 * work is only enqueued on the model's stream (atlas_model_stream) and the
 * source must stay valid until it completes; with scratch == NULL the call
 * allocates its temporaries and waits.                                      */
typedef struct atlas_load_scratch atlas_load_scratch;
atlas_load_scratch* atlas_load_scratch_create(void);
void atlas_load_scratch_destroy(atlas_load_scratch* s);
int atlas_model_set_tensor_dev(atlas_model* m, int kind, int layer, const void* src,
                               int src_dtype, int64_t numel, atlas_load_scratch* scratch);
/* The model's configuration (after creation or loading); layer_sliding
 * points into the model and lives as long as it.                           */
int atlas_model_get_config(const atlas_model* m, atlas_model_config* out);
/* Random init on the device: projections, embedding and lm_head N(0, 0.02)
 * (bf16 by truncation, or quantised by the atlas-quant rules), norm and
 * QK-norm weights U(0.5, 1.5).                                               */
int atlas_model_init_random(atlas_model* m, uint64_t seed);

int atlas_model_reset(atlas_model* m);
int atlas_model_pos(const atlas_model* m);
/* Test helpers, no reference counterpart: write n rows of one layer's KV
 * cache of sequence slot seq (rows pos0.., each n_kv_heads * head_dim f32
 * for K and for V, from host memory; the layout of GpuKvCache,
 * crates/atlas-model/src/lib.rs:557-596), and set the decode position.
 * Parity tests use them to start decoding at a long position with the same
 * cache rows in the engine and in the CPU oracle.                          */
int atlas_model_set_kv_rows(atlas_model* m, int seq, int layer, int pos0, int n,
                            const float* k, const float* v);
int atlas_model_set_pos(atlas_model* m, int pos);
float atlas_model_attn_scale(const atlas_model* m);
/* forward_one_gpu: one token at the current position; pos += 1.  logits
 * (host, [vocab]) may be NULL (they stay on the device).                    */
int atlas_model_forward_one(atlas_model* m, uint32_t token, float* logits);
/* forward_one_hooked: also downloads the post-residual hidden state after
 * every layer into hidden ([n_layers x d_model], may be NULL) and calls
 * hook (may be NULL) with it.  The hook only reads (StigmergicHook::on_layer
 * returns a deposit, nothing flows back), so the layers run back to back and
 * the hooks run in layer order after the token's forward pass: one host
 * round trip per token.                                                     */
int atlas_model_forward_one_hooked(atlas_model* m, uint32_t token, float* logits, float* hidden,
                                   atlas_hook_fn hook, void* user);

/* Feed n tokens at the current position without choosing (the prompt part of
 * generate): up to `chunk` tokens per step through the multi-row step, whose
 * per-row causal attention reads exactly the cache rows the reference's
 * token-by-token loop (lib.rs:1612-1618) would.  Extension: the reference
 * feeds one token per forward.                                              */
int atlas_model_prefill(atlas_model* m, const uint32_t* tokens, int n);
/* Tokens per prefill step, 1..1024 (default 1024; 1 = token by token).
 * Chunks above 16 need GEMM inner dims that are multiples of 128 and, for
 * int4, blocks of 32 * 2^j; other models cap them at 16.  Their GEMMs run on
 * the library's own tiled kernel; ATLAS_PROMPT_BLAS=1 in the environment at
 * model creation sends bf16 / int8 chunks through hipBLASLt instead (off by
 * default: see INTEGRATION.md).                                             */
int atlas_model_set_prefill_chunk(atlas_model* m, int chunk);

/* generate_with_sampling: resets, feeds the prompt (atlas_model_prefill), then
 * generates up to max_new tokens (EOS / stop tokens end it and are not
 * emitted).  out: [max_new]; *n_out receives the count.                     */
int atlas_model_generate(atlas_model* m, const uint32_t* prompt, int n_prompt, int max_new,
                         const atlas_sampling* s, uint32_t* out, int* n_out);
/* generate_with_sampling_hooked (InferEngine::generate with a hook): per
 * generated token the sum of max(delta, 0) and the count of Some layers.    */
int atlas_model_generate_hooked(atlas_model* m, const uint32_t* prompt, int n_prompt,
                                int max_new, const atlas_sampling* s, atlas_hook_fn hook,
                                void* user, uint32_t* out, float* total_delta,
                                uint32_t* layers_fired, int* n_out);
/* generate_streaming: on_token(user, token) returning 0 stops early. */
typedef int (*atlas_token_fn)(void* user, uint32_t token);
int atlas_model_generate_streaming(atlas_model* m, const uint32_t* prompt, int n_prompt,
                                   int max_new, const atlas_sampling* s, atlas_token_fn on_token,
                                   void* user, int* n_out);

/* Ragged batch (extension): n_seqs <= max_batch independent greedy
 * sequences decoded together, one skinny-GEMM step per token position.
 * prompts: concatenated ids, prompt_lens[n_seqs]; out: [n_seqs x max_new];
 * n_out[n_seqs].  Each sequence's tokens equal its own generate().           */
int atlas_model_generate_batch(atlas_model* m, const uint32_t* prompts, const int* prompt_lens,
                               int n_seqs, int max_new, const atlas_sampling* s, uint32_t* out,
                               int* n_out);

/* One token choice of generate_with_sampling's loop on the host
 * (crates/atlas-model/src/lib.rs:1623-1711): step-0 suppression, repetition
 * penalty over the last repetition_window of hist, greedy argmax, or
 * frequency / presence penalties, temperature, top-k, top-p, min-p, softmax
 * and one draw of the XorShift64 Rng (lib.rs:1190-1214) whose state is
 * *rng_state (advanced in place).  The eos / stop / rng_seed fields are not
 * read.  Needs no device.                                                   */
int atlas_sample_host(const float* logits, int vocab, const uint32_t* hist, int n_hist, int step,
                      const atlas_sampling* s, uint64_t* rng_state, uint32_t* token);
/* The same token choice on the device, from device-resident logits (copied,
 * not modified): the sampler kernel the engine's generate loop replays for
 * temperature > 0 with 1 <= top_k <= 1024 (SamplingConfig::olmo3() among
 * them), or top_k = 0 with top_p = 1 (SamplingConfig::default()).  With
 * top_k >= 1 every sum runs in the reference's order; with top_k = 0 the
 * draw is placed by exact prefix sums and taken only where the reference's
 * f32 rounding cannot move it, else the sums are redone in its order.  The
 * choice equals the host's except where glibc's expf and a correctly rounded
 * exp differ (about 1e-4 of arguments, 1 ulp) and that ulp moves a
 * cumulative-probability boundary across the random draw.
 * ATLAS_EUNSUPPORTED for other settings.
 * No reference counterpart (the reference samples on the host).             */
int atlas_sample_device(const float* logits, int vocab, const uint32_t* hist, int n_hist,
                        int step, const atlas_sampling* s, uint64_t* rng_state, uint32_t* token);

/* Extension: position from which decode steps run the long-context attention
 * (QK-norm/RoPE/KV-write kernel, split kernel over up to 256 blocks, split
 * merge) instead of the one-launch fused attention; default: never (the
 * fused step is the faster one at every measured context).  Each path is
 * captured in its own graph; the choice is made per step on the host.      */
int atlas_model_set_long_context(atlas_model* m, int from_pos);

/* Benchmark helper: greedy decode of n_steps tokens continuing from the
 * current state, replaying the captured step with no host synchronisation
 * in between.  tokens (host, may be NULL) receives the chosen ids.          */
int atlas_model_decode_greedy(atlas_model* m, uint32_t first_token, int n_steps,
                              uint32_t* tokens);
/* Benchmark helper: atlas_model_decode_greedy that also writes each step's
 * GPU time (ms, between HIP events recorded on the engine stream after
 * every step) into step_ms[n_steps].                                       */
int atlas_model_decode_greedy_timed(atlas_model* m, uint32_t first_token, int n_steps,
                                    uint32_t* tokens, float* step_ms);
/* Benchmark helper: enqueue `iters` copies of the weight GEMV launches of one
 * decode step (same kernels, shapes, prologues and weights; activations from
 * the engine's scratch) and time them with HIP events on the engine stream.
 * which: 0 = all of them, 1 = QKV, W_o and lm_head, 2 = W_down, 3 = gate/up,
 * 4 = QKV, 5 = W_o, 6 = lm_head (for bf16 weights each of 1-3 is one kernel
 * instance).  *ms = elapsed
 * milliseconds, *launches = GEMV launches issued, *bytes = algorithmic bytes
 * of one copy (weights + scales + x + y).                                    */
int atlas_model_bench_gemv(atlas_model* m, int iters, int which, float* ms, int* launches,
                           int64_t* bytes);
/* 1 = capture the decode step in a HIP graph (default), 0 = plain launches */
int atlas_model_use_graph(atlas_model* m, int enable);
/* The engine's stream (for timing with events on the same stream). */
void* atlas_model_stream(atlas_model* m);
/* Device pointers of the live buffers (tests / profiling). */
const float* atlas_model_logits_dev(atlas_model* m);
/* Bytes of weights one decode step reads (algorithmic, for rooflines). */
int64_t atlas_model_weight_bytes(const atlas_model* m);

#ifdef __cplusplus
}
#endif
#endif
