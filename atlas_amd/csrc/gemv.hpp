// gemv.hpp -- launch interface of the decode GEMV kernels (internal).
#pragma once
#include "common.hpp"

namespace atlas {

enum { WF_F32 = 0, WF_BF16 = 1, WF_I8 = 2, WF_I4 = 3 };   // weight formats
enum { EPI_STORE = 0, EPI_SILU_MUL = 1 };                 // epilogues

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
};

int gemv_fast_ok(int fmt, int K, int block);
int gemv_launch(const GemvArgs& a, hipStream_t st);     // N == 1
int skinny_launch(const GemvArgs& a, hipStream_t st);   // 1 <= N <= 8
int skinny_reserve(int M, int N, int K);
int gemm_generic_launch(int fmt, const void* A, const float* B, float* C, int m, int n, int k,
                        hipStream_t st);

inline void gemv_fill_int4_index(GemvArgs& a) {
    a.bpr = 0;
    a.cpb = 1;
    if (a.fmt == WF_I4 && a.block > 0) {
        if (a.block % 32 == 0) a.cpb = a.block / 32;
        if (a.K % a.block == 0) a.bpr = a.K / a.block;
    }
}

}  // namespace atlas
