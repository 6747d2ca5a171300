/*
 * atlas_kernels.h -- C ABI of the MI355X (gfx950) decode kernels.
 *
 * Drop-in boundary for the reference's `atlas-tensor` FFI.  Part 1 keeps the
 * exact names and signatures that crates/atlas-tensor/src/lib.rs:17-92
 * declares in its `extern "C"` block (int dims, raw device pointers, void
 * return), implemented in HIP for gfx950, so that block links unchanged.
 * Part 2 replaces the CUDA runtime calls that crates/atlas-tensor/src/lib.rs:
 * 151-161 makes directly (cudaMalloc / cudaFree / cudaMemcpy /
 * cudaMallocAsync / cudaFreeAsync).  Part 3 adds the entry points the
 * decode hot path needs beyond the reference (int8/int4 dequant-fused GEMV,
 * skinny ragged-batch GEMM, fused norm/RoPE/KV kernels, quantisers).
 *
 * Error behaviour: the reference's launches are unchecked and its Rust
 * wrappers fall back to the CPU when an allocation fails
 * (crates/atlas-tensor/src/lib.rs:193-207, 371-400).  Here every `int`
 * entry point returns 0 or a negative ATLAS_E* code, and the `void` ones of
 * Part 1 record failures the same way: atlas_last_error_code() /
 * atlas_last_error() report the most recent failure on the calling thread
 * (cleared by atlas_clear_error()).
 *
 * Streams: every launch, stream-ordered allocation and copy goes to the
 * library-wide stream set by atlas_set_stream (default = the null stream, as
 * in the reference, kernels/matmul.cu:17-23), from whichever thread it is
 * called.  A thread may override it for its own calls only
 * (atlas_set_thread_stream, undone by atlas_clear_thread_stream).  Launches
 * are asynchronous.
 *
 * Library scratch: entry points that need device scratch and are not handed
 * a workspace (atlas_decode_attention, atlas_gpu_argmax,
 * atlas_gemm_skinny_f32, atlas_attention_fused_f32) keep it per calling
 * thread, grow it on first use of a larger shape and free it when the
 * thread exits.  A call that would grow it while its stream is being
 * captured into a graph returns / records ATLAS_EUNSUPPORTED instead: warm
 * up with one call of the same shape before the capture, or use
 * atlas_decode_attention_noalloc.
 */
#ifndef ATLAS_KERNELS_H
#define ATLAS_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===== Part 1: reference FFI (crates/atlas-tensor/src/lib.rs:17-92) ======= */

/* lib.rs:21-24 -> kernels/matmul.cu:461-513.  C[m x n] = A[m x k] B[k x n],
 * all f32 row-major.  n == 1 runs the batch-1 GEMV kernel.                  */
void atlas_matmul_f32(const float* a, const float* b, float* c, int m, int n, int k);
/* lib.rs:25 -> matmul.cu:522-526 */
void atlas_vec_add_f32(const float* a, const float* b, float* out, int n);
/* lib.rs:26 -> matmul.cu:528-531 */
void atlas_scale_f32(const float* x, float s, float* out, int n);
/* lib.rs:27 -> matmul.cu:533-536 */
void atlas_relu_f32(const float* x, float* out, int n);
/* lib.rs:28 -> matmul.cu:538-542 (row softmax) */
void atlas_softmax_f32(const float* x, float* out, int rows, int cols);
/* lib.rs:29-30 -> matmul.cu:580-595.  Names keep the reference's spelling;
 * they report HIP devices.                                                  */
int atlas_cuda_available(void);
int atlas_cuda_device_count(void);
/* lib.rs:31-33 -> matmul.cu:597-605 */
void atlas_rmsnorm_f32(const float* x, const float* w, float* out, int n, float eps);
/* lib.rs:34 -> matmul.cu:607-612 */
void atlas_rope_apply_f32(float* x, int pos, int head_dim, float theta_base);
/* lib.rs:35 -> matmul.cu:614-618 */
void atlas_silu_mul_f32(const float* gate, const float* up, float* out, int n);
/* lib.rs:36 -> matmul.cu:620-626 */
void atlas_vram_copy_f32(const float* src, float* dst, int n);
/* lib.rs:37-41 -> matmul.cu:138-161, 546-557 (training; kept for ABI
 * completeness).  bc1/bc2 are 1/(1 - beta^t) as the caller passes them
 * (crates/atlas-optim/src/lib.rs:203-204) and multiply the moments;
 * param = param*(1 - lr*wd) - lr*m_hat/(sqrt(v_hat) + eps).  Returns with
 * the update complete (the current stream is synchronised).                 */
void atlas_adamw_step(float* param, float* m, float* v, const float* grad, float lr,
                      float beta1, float beta2, float eps, float wd, float bc1, float bc2,
                      int n);
/* lib.rs:44-47 -> matmul.cu:636-651.  A_bf16[m x k] (bf16 bits), B[k x n]
 * f32 row-major (column j = activation j), C[m x n].  n == 1: batch-1 GEMV;
 * 2 <= n <= 8: skinny MFMA GEMM; larger n: generic kernel.                  */
void atlas_sgemm_bf16_f32(const uint16_t* a_bf16, const float* b, float* c, int m, int n,
                          int k);
/* lib.rs:51 -> matmul.cu:450-459: drains the current device */
void atlas_sync(void);
/* lib.rs:56-59 -> matmul.cu:662-710 */
void atlas_qk_norm_inplace(float* x, const float* w, int n_heads, int head_dim, float eps);
/* lib.rs:64-68 -> matmul.cu:723-743, 898-907 */
void atlas_rope_precomputed(float* x, const float* cos_tab, const float* sin_tab, int n_heads,
                            int head_dim, int pos, int max_seq);
/* lib.rs:70-74 -> matmul.cu:752-766, 909-919 */
void atlas_kv_cache_write(float* k_cache, float* v_cache, const float* new_k,
                          const float* new_v, int pos, int n_kv_heads, int head_dim);
/* lib.rs:80-86 -> matmul.cu:786-933.  Split-K flash decode here; any
 * context length (no dynamic-LDS limit).  Up to 8 splits merge in the block
 * that finishes last (one launch), more in a second merge kernel.           */
void atlas_decode_attention(const float* q, const float* k_cache, const float* v_cache,
                            float* out, int n_heads, int n_kv_heads, int head_dim, int pos,
                            float scale, int window_size);
/* lib.rs:90 -> matmul.cu:997-1007.  Index written as f32.  Ties return the
 * LAST maximal index, the rule of the CPU path this feeds
 * (crates/atlas-model/src/lib.rs:2701-2706).                                */
void atlas_gpu_argmax(const float* x, float* out_f32, int n);

/* ===== Part 2: device memory (replaces crates/atlas-tensor/src/lib.rs:151-161) */

enum {
    ATLAS_OK = 0,
    ATLAS_EINVAL = -1,
    ATLAS_EHIP = -2,
    ATLAS_ENOMEM = -3,
    ATLAS_EUNSUPPORTED = -4,
    ATLAS_EIO = -5              /* file open / read / map failed (loader)      */
};

int atlas_last_error_code(void);
const char* atlas_last_error(void);
void atlas_clear_error(void);

/* Stream-ordered allocation on the current stream (cudaMallocAsync,
 * lib.rs:196-206), falling back to a synchronous allocation.               */
int atlas_dev_malloc(void** ptr, size_t bytes);
int atlas_dev_free(void* ptr);
/* Synchronous allocation for long-lived weights (cudaMalloc, lib.rs:254-258). */
int atlas_dev_malloc_sync(void** ptr, size_t bytes);
int atlas_dev_free_sync(void* ptr);
/* Copies; the d2h copy waits for the current stream (lib.rs:217-224).        */
int atlas_memcpy_h2d(void* dst, const void* src, size_t bytes);
int atlas_memcpy_d2h(void* dst, const void* src, size_t bytes);
int atlas_memcpy_d2d(void* dst, const void* src, size_t bytes);
int atlas_memset_zero(void* dst, size_t bytes);     /* fill kernel, graph-safe */

int atlas_set_device(int device);
int atlas_set_stream(void* hip_stream);               /* library-wide; NULL = null stream */
int atlas_set_thread_stream(void* hip_stream);        /* this thread only (NULL = null stream) */
int atlas_clear_thread_stream(void);                  /* back to the library-wide stream */
void* atlas_get_stream(void);                         /* the calling thread's effective stream */
int atlas_stream_sync(void);                          /* waits for that stream */
/* Bytes of library scratch the calling thread holds on the current device. */
int64_t atlas_thread_scratch_bytes(void);
/* Test hook, no reference counterpart: after `skip` more device or pinned-host
 * allocations of the library succeed, the next `count` fail as if the device
 * were out of memory (ATLAS_ENOMEM; the reference's Option/bool fallback
 * contract, crates/atlas-tensor/src/lib.rs:193-207, is tested with it).
 * count = 0 turns it off.  Process-wide.                                     */
int atlas_debug_fail_allocations(int skip, int count);
int atlas_device_cu_count(void);

/* ===== Part 3: decode hot-path extensions (no reference counterpart) ===== */

/* Weight storage formats of the GEMV family. */
enum {
    ATLAS_W_F32 = 0,     /* f32 row-major                                     */
    ATLAS_W_BF16 = 1,    /* bf16 bits row-major (GpuBufKind::BF16)            */
    ATLAS_W_INT8 = 2,    /* Int8Tensor: i8 row-major + f32 scale per row      */
    ATLAS_W_INT4 = 3     /* Int4Tensor: nibbles over the flattened index, even
                            element in the high nibble, f32 scale per block   */
};

/* y[m] = sum_k dequant(W)[m,k] x[k] (f32 accumulation).  Batch-1 decode GEMV
 * semantics of Linear::forward (crates/atlas-model/src/lib.rs:487-499) with
 * W stored per crates/atlas-quant/src/lib.rs:32-168.  scales: NULL for
 * f32/bf16; int8 [m]; int4 [ceil(m*k/block)].                               */
int atlas_gemv_f32(int fmt, const void* w, const float* scales, int block, const float* x,
                   float* y, int m, int k);
int atlas_gemv_bf16_f32(const uint16_t* w, const float* x, float* y, int m, int k);
int atlas_gemv_i8_f32(const int8_t* w, const float* scales, const float* x, float* y, int m,
                      int k);
int atlas_gemv_i4_f32(const uint8_t* w, const float* scales, int block, const float* x,
                      float* y, int m, int k);
/* Fused SwiGLU GEMV: W has 2*h rows interleaved (gate_0, up_0, gate_1, ...);
 * h_out[i] = silu(gate_i . x) * (up_i . x)  (FeedForward::forward,
 * crates/atlas-model/src/lib.rs:911-924).                                   */
int atlas_gemv_swiglu_f32(int fmt, const void* w, const float* scales, int block,
                          const float* x, float* h_out, int h, int k);

/* Batch-1 GEMV whose input is formed while it is loaded (one launch instead
 * of a norm kernel plus a GEMV):
 *   pro 0: x as given;
 *   pro 1: x' = x + rmsnorm(y) * w  (post-norm residual, crates/atlas-model/
 *          src/lib.rs:983-993); x' is also written to x_out (non-NULL,
 *          distinct from x and y);
 *   pro 2: x' = rmsnorm(x) * w  (x_out may be NULL);
 *   pro 3: x'[j] = silu(y[2j]) * y[2j+1]  (SwiGLU over interleaved gate/up
 *          outputs, lib.rs:918-921); x unused.
 * eps is the RMSNorm epsilon.  yout[m] = dequant(W) x'.                       */
int atlas_gemv_fused_f32(int fmt, const void* w, const float* scales, int block,
                         const float* x, float* yout, int m, int k, int pro, const float* y,
                         const float* norm_w, float eps, float* x_out);

/* Ragged micro-batch: Y[n, m] = sum_k dequant(W)[m,k] X[n,k] for 1 <= n <= 16
 * activation rows (X [n x k] row-major, Y [n x m] row-major).  MFMA bf16 with
 * hi/lo split activations.  fmt: BF16, INT8, INT4.  n >= 17 rows with
 * k % 128 == 0 (int4: blocks of 32 * 2^j) take the tiled MFMA GEMM of prompt
 * chunks (128 rows per launch); other shapes outside 1..16 return
 * ATLAS_EINVAL.                                                              */
int atlas_gemm_skinny_f32(int fmt, const void* w, const float* scales, int block,
                          const float* x, float* y, int m, int n, int k);
/* The same row counts with the SwiGLU epilogue: W has 2*h rows interleaved
 * (gate_0, up_0, gate_1, ...) and H[n, i] = silu(gate_i . X[n]) * (up_i . X[n])
 * (FeedForward::forward, crates/atlas-model/src/lib.rs:911-924), H [n x h]
 * row-major.  Extension: the ragged batch's and the prompt chunks' gate/up.  */
int atlas_gemm_skinny_swiglu_f32(int fmt, const void* w, const float* scales, int block,
                                 const float* x, float* h_out, int h, int n, int k);

/* out = rmsnorm(x) * w row-wise over `rows` rows of length n (ld = n).      */
int atlas_rmsnorm_rows_f32(const float* x, const float* w, float* out, int n, int rows,
                           float eps);
/* Post-norm residual: x += rmsnorm(y) * w  (crates/atlas-model/src/lib.rs:
 * 983-993), row-wise over `rows` rows.                                       */
int atlas_residual_rmsnorm_f32(float* x, const float* y, const float* w, int n, int rows,
                               float eps);
/* Fused per-head QK-norm (q_norm/k_norm may be NULL) + RoPE from the tables +
 * K/V cache write at pos.  qkv = [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)];
 * q is rotated in place; K, V land in the caches [max_seq][n_kv][hd].        */
int atlas_qkv_post_f32(float* qkv, const float* q_norm, const float* k_norm, float qk_eps,
                       const float* cos_tab, const float* sin_tab, float* k_cache,
                       float* v_cache, int n_heads, int n_kv, int head_dim, int pos);
/* Fused decode attention for one token: per-head QK-norm (norm weights may be
 * NULL) + RoPE of the raw qkv = [q | k | v] projections, K/V cache write at
 * pos, split-K GQA attention over [max(0, pos - window + 1), pos] and the
 * split merge, in one launch (atlas_qkv_post_f32 + atlas_decode_attention
 * semantics).  head_dim 64/128/256, n_heads / n_kv in {1, 2, 4, 8}.
 * n_splits <= 0 picks a split count for the context.  min_chunk > 0 makes
 * n_splits a maximum: the kernel uses min(n_splits, ceil(ctx / min_chunk))
 * splits for the live context length ctx (as a captured decode step does).  */
int atlas_attention_fused_f32(const float* qkv, const float* q_norm, const float* k_norm,
                              float qk_eps, const float* cos_tab, const float* sin_tab,
                              float* k_cache, float* v_cache, float* out, int n_heads, int n_kv,
                              int head_dim, int pos, float scale, int window, int n_splits,
                              int min_chunk);

/* No counterpart in the reference.  atlas_decode_attention for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): same arguments and results (to
 * float rounding: its splits always merge in a second kernel, with the
 * two-kernel split count), but the split partials live in a fixed 8 MiB device workspace
 * of the library (one per GPU, held until the process ends); no hipMalloc or
 * hipFree is made.  Shapes whose partials (n_heads x splits x (head_dim + 2)
 * floats) exceed the workspace return ATLAS_EINVAL.  Calls that overlap on
 * one GPU (two streams or threads) share the workspace and race: serialise
 * them.  Returns 0 or a negative ATLAS_E* code.                             */
int atlas_decode_attention_noalloc(const float* q, const float* k_cache, const float* v_cache,
                                   float* out, int n_heads, int n_kv_heads, int head_dim,
                                   int pos, float scale, int window_size);
/* Bytes of that workspace.                                                   */
int64_t atlas_decode_attention_noalloc_max_bytes(void);

/* Greedy choice: index of the last maximum of x[0..n) as u32 (device).      */
int atlas_argmax_u32(const float* x, int n, uint32_t* out_idx);

/* Device-side quantisers, bit-exact to Int8Tensor::quantize /
 * Int4Tensor::quantize (crates/atlas-quant/src/lib.rs:43-63, 113-145).
 * src_is_bf16 selects bf16-bits or f32 input.  int4 needs an even block.     */
int atlas_quantize_int8_dev(const void* src, int src_is_bf16, int rows, int cols,
                            int8_t* data, float* scales);
int atlas_quantize_int4_dev(const void* src, int src_is_bf16, int64_t n, int block,
                            uint8_t* data, float* scales);
/* Host-side quantisers (same rules; for callers holding host weights).      */
int atlas_quantize_int8_host(const float* w, int64_t rows, int64_t cols, int8_t* data,
                             float* scales);
int atlas_quantize_int4_host(const float* w, int64_t rows, int64_t cols, int64_t block,
                             uint8_t* data, float* scales);

/* Seeded synthetic fills on the device: SplitMix64 counter + Box-Muller.
 * kind 0: N(a, b) f32; 1: N(a, b) bf16 by truncation; 2: U(a, b) f32.        */
int atlas_fill_random(int kind, void* out, int64_t n, uint64_t seed, float a, float b);

/* Measurement only (no reference counterpart): the streaming floor of a
 * decode-GEMV-shaped launch.  Captures read-only launches of
 * bytes_per_launch bytes each (consecutive regions of buf, wrapping; a
 * multiple of 16 KiB, the bf16 decode GEMV's work split and load pattern,
 * blocks_per_cu 4-wave blocks per CU) in HIP graphs of `launches` and
 * 2 * `launches` kernels on the library's stream, replays them and stores
 * the difference of the best replay times per launch in microseconds (the
 * graph launch's own cost cancels).  bytes_per_launch 0 times an empty
 * kernel of the same grid (buf may be null): the launch floor itself.
 * What the decode GEMVs cost beyond the streaming floor is their own work. */
int atlas_bench_stream_floor(const void* buf, int64_t buf_bytes, int64_t bytes_per_launch,
                             int launches, int blocks_per_cu, float* us_per_launch);

#ifdef __cplusplus
}
#endif
#endif
