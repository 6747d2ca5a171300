// gemv.hpp -- launch interface of the decode GEMV kernels (internal).
#pragma once
#include "common.hpp"

namespace atlas {

enum { WF_F32 = 0, WF_BF16 = 1, WF_I8 = 2, WF_I4 = 3 };   // weight formats
enum { EPI_STORE = 0, EPI_SILU_MUL = 1, EPI_ARGMAX = 2 };  // epilogues
// prologues: how the GEMV input x is formed while it is loaded
enum {
    PRO_X = 0,        // x as given
    PRO_RESNORM = 1,  // x = x_in + (y * inv(y)) * w   (post-norm residual; materialised)
    PRO_RMSNORM = 2,  // x = (x_in * inv(x_in)) * w
    PRO_SILU = 3,     // x[k] = silu(y[2k]) * y[2k+1]   (SwiGLU of interleaved gate/up)
    PRO_RESNORM_NORM = 4   // h = x_in + (y * inv(y)) * w; x = (h * inv(h)) * w2 (the last
                           // layer's residual and the final norm; h materialised)
};

struct GemvArgs {
    int fmt;                 // WF_*
    const void* w;           // row-major [M x K] in the stored format
    const float* scales;     // int8: [M]; int4: [ceil(M*K/block)]
    const float* x;          // [K] (batch 1) or [N x K] (skinny)
    float* y;                // [M] or [M/2] (EPI_SILU_MUL); skinny: [N x M]
    int M, K;
    int block;               // int4 block size (multiple of 32 on the fast path)
    int bpr;                 // int4: blocks per row when K % block == 0, else 0
    int cpb;                 // int4: 32-element chunks per block
    int epi;                 // EPI_*
    int N;                   // skinny: number of activation rows (1..8)
    long x_stride_n, x_stride_k;   // skinny: x element (n, k) at n*sn + k*sk
    long y_stride_n, y_stride_m;   // skinny: y element (n, m) at n*sn + m*sm
    int x_vec;               // skinny: x rows 16-byte aligned with x_stride_k == 1
    int pro;                 // PRO_*
    const float* pro_y;      // RESNORM: normalised addend [K]; SILU: pairs [2K]
    const float* pro_w;      // RESNORM / RMSNORM / RESNORM_NORM: norm weight [K]
    const float* pro_w2;     // RESNORM_NORM: the second norm's weight [K]
    float pro_eps;
    float* pro_out;          // RESNORM / RMSNORM: x, RESNORM_NORM: h, written out by block 0
                             // (nullable)
    unsigned long long* arg_part;   // EPI_ARGMAX: per-wave (value, index) keys
    long ldw;                // bytes between weight rows (multiple of 16); 0 = packed rows
    float* partial;          // skinny / prompt GEMM split-K partials (null: the thread's scratch)
    size_t partial_bytes;    // ... their size
    // skinny_launch, host side: non-null with EPI_STORE and the caller's
    // partial buffer, a split-K launch of the 2-8-row direct-load kernels or
    // of the tiled prompt GEMM (17-128 rows, one launch) leaves its partials
    // in `partial` ([splits][N][M], summed in split order by the consumer)
    // and stores the split count here instead of launching the reduce; 0
    // when y was written.
    int* defer_splits;
    struct BlasRows* blas;   // 17+ rows of bf16 / int8 weights: the caller's hipBLASLt context, or
                             // null (the tiled MFMA kernel)
};

enum { GEMV_MAX_WAVES = 16384 };    // bound on persistent waves (argmax partials)

int gemv_fast_ok(int fmt, int K, int block);
int gemv_launch(const GemvArgs& a, hipStream_t st);     // N == 1
int gemv_waves(const GemvArgs& a);                       // persistent waves of gemv_launch
bool gemv_resnorm_norm_ok(const GemvArgs& a);             // PRO_RESNORM_NORM available for a
int skinny_launch(const GemvArgs& a, hipStream_t st);   // 1 <= N <= 8
// N = 2..kGemvMaxNx rows through the batch-1 GEMV (every weight load feeds
// all N rows); plain x, store / SwiGLU epilogues
constexpr int kGemvMaxNx = 4;
bool gemv_multi_ok(const GemvArgs& a);
int gemv_multi_launch(const GemvArgs& a, hipStream_t st);
size_t skinny_partial_bytes(int M, int N, int K);    // split-K partials of (M, N, K)
// y = the fixed-order sum of `splits` partials ([splits][N][M]), with a's epilogue
int skinny_reduce_launch(const GemvArgs& a, const float* partial, int splits, hipStream_t st);
// 17+ rows: the tiled MFMA GEMM (skinny_launch routes there; 128 rows per
// launch) or, with a library context, the hipBLASLt prompt GEMM
bool gemm_rows_ok(const GemvArgs& a);
int gemm_rows_launch(const GemvArgs& a, hipStream_t st);
size_t gemm_rows_partial_bytes(int M, int N, int K);
// The bf16 and int8 prompt GEMMs through hipBLASLt (blas.cpp): X's rows split
// into bf16 hi and lo rows (bf16 weights) or three int8 digit rows (int8
// weights), one library GEMM of the weights against all of them (the weights
// stream once), then y = the recombined products with the store or SwiGLU
// epilogue.  A context holds the library handle, its workspace and the
// staging buffers for up to max_n rows of K <= max_k, M <= max_m.
struct BlasRows;
int blas_rows_create(BlasRows** out, int max_n, int max_m, int max_k);
void blas_rows_destroy(BlasRows* b);
int blas_rows_launch(BlasRows* b, const GemvArgs& a, hipStream_t st);   // bf16/int8, gemm_rows_ok(a)
// The library GEMM alone, for callers that fuse the split and the combine into
// their neighbouring kernels: blas_rows_xs(b) holds X's split rows (K wide;
// bf16: hi rows 0..n-1, lo rows n..2n-1; int8: digit rows 0..3n-1 with the
// row scales in blas_rows_xscale(b)), blas_rows_d(b) receives the product
// rows (M wide; 2n f32 or 3n int32).  n <= blas_rows_max_n(b).
int blas_rows_gemm(BlasRows* b, const GemvArgs& a, int n, hipStream_t st);
uint16_t* blas_rows_xs(BlasRows* b);
float* blas_rows_d(BlasRows* b);
float* blas_rows_xscale(BlasRows* b);
int blas_rows_max_n(const BlasRows* b);
// the two element-wise halves (skinny.hip): rows n of x (f32, stride sn) ->
// out rows n (bf16 hi) and N + n (bf16 lo); y[n, m] = d[n, m] + d[N + n, m]
// (d rows of M f32) or the SwiGLU of the (gate, up) column pairs
int split_rows_launch(const float* x, long sn, int N, int K, uint16_t* out, hipStream_t st);
int combine_rows_launch(const float* d, int N, int M, int epi, float* y, long ysn, long ysm,
                        hipStream_t st);
// int8 weights: rows n of x -> three int8 digit rows (n, N + n, 2N + n; K
// wide) and the row scale xscale[n] = max|x[n]| / 127; y from the int32
// product rows d (M wide) times the weight row scales, store or SwiGLU
constexpr int kDigitsMaxK = 12288;      // digits_rows_launch: K <= this, K % 4 == 0
int digits_rows_launch(const float* x, long sn, int N, int K, int8_t* out, float* xscale,
                       hipStream_t st);
int combine_digits_launch(const int* d, int N, int M, const float* wscale, const float* xscale, int epi,
                          float* y, long ysn, long ysm, hipStream_t st);
// the SwiGLU of the (gate, up) pairs of d = hi + lo product rows, written
// straight as the split rows (M / 2 wide) of the next GEMM's input
int combine_split_launch(const float* d, int N, int M, uint16_t* out, hipStream_t st);
int gemm_generic_launch(int fmt, const void* A, const float* B, float* C, int m, int n, int k,
                        hipStream_t st);

// LDS bytes of the batch-1 GEMV's staged x: K / 4 pieces of 16 bytes plus
// one gap piece per 16
inline size_t gemv_x_lds_bytes(int K) {
    const size_t np = (size_t)K / 4;
    return (np + (np + 15) / 16) * 16;
}

// packed bytes of one weight row
inline long gemv_row_bytes(int fmt, int K) {
    return fmt == WF_F32 ? 4L * K : fmt == WF_BF16 ? 2L * K : fmt == WF_I8 ? (long)K : K / 2;
}

// a row pitch is 0 (packed) or a multiple of 16 bytes that holds the row
inline bool gemv_pitch_ok(const GemvArgs& a) {
    return a.ldw == 0 || (a.ldw % 16 == 0 && a.ldw >= gemv_row_bytes(a.fmt, a.K) &&
                          (a.fmt != WF_I4 || a.K % 2 == 0));
}

inline void gemv_fill_int4_index(GemvArgs& a) {
    a.bpr = 0;
    a.cpb = 1;
    if (a.fmt == WF_I4 && a.block > 0) {
        if (a.block % 32 == 0) a.cpb = a.block / 32;
        if (a.K % a.block == 0) a.bpr = a.K / a.block;
    }
}

// Measurement only: per-launch time of a graph of `launches` read-only
// launches of bytes_per_launch each with the bf16 decode GEMV's work split
// (consecutive regions of buf, wrapping); best of three replays.
int stream_floor_bench(const void* buf, long buf_bytes, long bytes_per_launch, int launches,
                       int blocks_per_cu, float* us_per_launch, hipStream_t st);

}  // namespace atlas
