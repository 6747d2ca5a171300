// fused.hpp -- launch interface of the small decode-step kernels (internal).
#pragma once
#include "common.hpp"

namespace atlas {

enum { EW_ADD = 0, EW_SCALE = 1, EW_RELU = 2, EW_SILU_MUL = 3, EW_COPY = 4, EW_FILL = 5 };
enum { INIT_NORMAL_F32 = 0, INIT_NORMAL_BF16 = 1, INIT_UNIFORM_F32 = 2 };
enum { ARGMAX_MAX_PARTS = 16384 };
enum { CVT_F16_F32 = 0, CVT_F32_BF16 = 1, CVT_BF16_F32 = 2 };

struct QkvPostArgs {
    float* qkv;              // per sequence: [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)]
    long qkv_stride;         // elements between sequences
    const float* q_norm;     // [n_heads*hd] or null (no QK-norm)
    const float* k_norm;     // [n_kv*hd] or null
    float qk_eps;
    const float* cos_tab;    // [max_seq x hd/2]
    const float* sin_tab;
    float* k_cache;          // [slots][max_seq][n_kv][hd]
    float* v_cache;
    long slot_stride;        // elements per slot
    const int* slot_dev;     // [n_seq] slot per sequence, or null (slot 0)
    const int* pos_dev;      // [n_seq] position per sequence, or null (use pos)
    int pos;
    int n_heads, n_kv, head_dim;
    // non-null: sequence s's q|k|v is src[s*src_stride + e] + src[src_lo + s*src_stride + e]
    // (the library GEMM's hi and lo product rows); q is written to qkv
    const float* src;
    long src_stride, src_lo;
    // non-null (src null): the int8 digit products instead, element e of
    // sequence s = (P0 + (P1 + P2 / 128) / 128) * src_xs[s] * src_ws[column]
    // with planes P0..P2 src_lo apart, as combine_digits_kernel forms it
    const int* src_d;
    const float* src_ws;
    const float* src_xs;
    // non-null (src, src_d null): split-K partials of the QKV GEMM instead,
    // element e of sequence s = the sum over p < src_splits, in p order, of
    // src_parts[p * src_lo + s * src_stride + e] (the split-K reduce's sum)
    const float* src_parts;
    int src_splits;
};

struct ArgmaxArgs {
    float* x;                      // logits (modified in place by penalties)
    int n;
    unsigned long long* part;      // scratch [ARGMAX_MAX_PARTS]
    float* out_f32;                // index as float (reference atlas_gpu_argmax)
    uint32_t* out_u32;             // index as u32
    const uint32_t* suppress;      // step-0 suppression list (device) or null
    int n_suppress;
    uint32_t* hist;                // generated-token history (device) or null
    int* hist_len;                 // its length (device)
    int window;                    // repetition window
    float theta;                   // repetition penalty (1 = off)
    int* step;                     // device step counter (step 0 = first token), or null
    int record;                    // append the choice to hist and bump hist_len
    int n_parts;                   // > 0: part[] already holds this many partial keys
    int* pos_inc;                  // device position bumped after the choice, or null
};

// Device-resident sampling settings (SamplingConfig, lib.rs:1223-1295).
struct SampleCfg {
    float temperature;             // > 0
    float theta;                   // repetition penalty (1 = off)
    float freq, presence;          // frequency / presence penalties (0 = off)
    float top_p;                   // 1 = off
    float min_p, log_min_p;        // min_p > 0: threshold max + logf(min_p) (host logf)
    int window;                    // repetition window
    int top_k;                     // 1 .. SAMPLE_MAX_K, or 0 (whole vocabulary; top_p off)
    int n_suppress;                // step-0 suppression list length
};
enum { SAMPLE_MAX_K = 1024, SAMPLE_MAX_HIST = 4096, SAMPLE_CAND = 4096 };

struct SampleArgs {
    float* x;                      // logits [n] (modified in place by the penalties)
    int n;
    const SampleCfg* cfg;          // device
    const uint32_t* suppress;      // device [cfg->n_suppress] or null
    uint32_t* hist;                // generated-token history (device)
    int* hist_len;                 // its length (device)
    int* step;                     // device step counter (step 0 = first token)
    int* pos_inc;                  // device position bumped after the choice, or null
    unsigned long long* rng;       // device XorShift64 state
    uint32_t* out_u32;             // the chosen token
    int record;                    // append the choice to hist and bump hist_len
};

int rmsnorm_launch(const float* x, const float* w, float* out, int n, int rows, long ld, float eps,
                   hipStream_t st);
int residual_rmsnorm_launch(float* x, const float* y, const float* w, int n, int rows, long ld,
                            float eps, hipStream_t st);
// x += rmsnorm(d_hi + d_lo) * w from the library GEMM's product rows (row b at
// d + b*n, its lo row lo_off further); with xs non-null the new x rows are
// also written as bf16 hi rows (xs row b) and lo rows (xs row rows + b)
int residual_rmsnorm_rows_launch(float* x, const float* d, long lo_off, const float* w, int n, int rows,
                                 long ld, float eps, uint16_t* xs, hipStream_t st);
// x += rmsnorm(y) * w with y from the int8 digit products (three int32 planes
// of rows x n, weight column scales ws, input row scales xscale); with xd
// non-null the new x rows are also written as int8 digit rows (xd rows b,
// rows + b, 2 rows + b) and xscale[b] becomes their scale
int residual_rmsnorm_digits_launch(float* x, const int* d, const float* ws, float* xscale,
                                   const float* w, int n, int rows, long ld, float eps, int8_t* xd,
                                   hipStream_t st);
// x += rmsnorm(y) * w with y the split-K partials ([splits][rows][n]) of the
// GEMM that produced it, summed in split order (splits <= 8, n <= 8192)
int residual_rmsnorm_parts_launch(float* x, const float* part, int splits, const float* w, int n,
                                  int rows, long ld, float eps, hipStream_t st);
int qkv_post_launch(const QkvPostArgs& a, int n_seq, hipStream_t st);
// greedy choice of each of `rows` logit rows (row r at x + r*ld, n logits)
// into out_u32[r], last maximal index on ties; part holds rows * min(512,
// ceil(n / 256)) <= ARGMAX_MAX_PARTS keys
int argmax_rows_launch(const float* x, int n, long ld, int rows, unsigned long long* part,
                       uint32_t* out_u32, hipStream_t st);
int qk_norm_launch(float* x, const float* w, int n_heads, int hd, float eps, hipStream_t st);
int rope_tab_launch(float* x, const float* c, const float* s, int n_heads, int hd, int pos,
                    int max_seq, hipStream_t st);
int rope_apply_launch(float* x, int pos, int hd, float theta, hipStream_t st);
int kv_write_launch(float* kc, float* vc, const float* nk, const float* nv, int pos, int n_kv,
                    int hd, hipStream_t st);
int ew_launch(int op, const float* a, const float* b, float* out, float s, long n, hipStream_t st);
int softmax_rows_launch(const float* x, float* out, int rows, int cols, hipStream_t st);
int adamw_launch(float* p, float* m, float* v, const float* g, float lr, float b1, float b2,
                 float eps, float wd, float bc1, float bc2, int n, hipStream_t st);
int argmax_launch(const ArgmaxArgs& a, hipStream_t st);
// one token of generate_with_sampling (temperature > 0, 1 <= top_k <= 1024)
int sample_launch(const SampleArgs& a, hipStream_t st);
// Optional copy of the RoPE tables' row at *pos_dev into out (cos[half] then
// sin[half]), made by the embedding gather that starts a decode step, so the
// step's attention launches read their rotation without waiting on pos.
struct RopeRowArgs {
    const int* pos_dev = nullptr;
    const float* cos_tab = nullptr;   // [max_seq x half]
    const float* sin_tab = nullptr;
    int half = 0;
    float* out = nullptr;             // null: no copy
};
int embed_launch(const uint16_t* table, int vocab, int d, const uint32_t* tok_dev, uint32_t tok,
                 float* out, long ld, int n_seq, hipStream_t st, const RopeRowArgs& rope = RopeRowArgs{});
int add_int_launch(int* p, int n, int v, hipStream_t st);
int init_launch(int kind, void* out, long n, unsigned long long seed, float a, float b,
                hipStream_t st);
int quant_i8_launch(const void* src, int src_bf16, int rows, int cols, int8_t* data, float* scales,
                    hipStream_t st);
int quant_i4_launch(const void* src, int src_bf16, long n, int block, uint8_t* data, float* scales,
                    hipStream_t st);
// element conversion (CVT_*): f16 -> f32, f32 -> bf16 (truncation), bf16 -> f32
int cvt_launch(int kind, const void* src, void* dst, long n, hipStream_t st);

}  // namespace atlas
