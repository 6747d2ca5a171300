// gemv.hip -- batch-1 decode GEMV y = W x for bf16 / int8 / int4 / f32 weights.
//
// Semantics: y[m] = sum_k dequant(W)[m,k] * x[k] with f32 accumulation, the
// reference's Linear::forward (crates/atlas-model/src/lib.rs:487-499) over
// weights stored as in crates/atlas-tensor/src/lib.rs:242-292 (bf16 bits) and
// crates/atlas-quant/src/lib.rs:32-168 (int8 per-row scale, int4 per-block
// scale over the flattened index, even element in the high nibble).
//
// Design (gfx950, HBM-bound, no MFMA):
//  * a 256-thread block = 4 wave64s; each wave owns ROWS consecutive rows and
//    walks the whole K with 128-bit nontemporal loads (lane i reads the i-th
//    16-byte chunk of every row, so one instruction reads 1 KiB contiguous
//    per row);
//  * x is staged once per block in LDS as f32 in 16-byte pieces with one
//    empty piece after every 16 (xpad below), which keeps the per-lane
//    ds_read_b128 of consecutive chunks bank-conflict free;
//  * one x read feeds ROWS rows, so LDS traffic stays below HBM traffic even
//    for int4 (32 f32 of x per 16 bytes of weights);
//  * int8/int4 dequantise with one SDWA sign-extending convert per value;
//    int4 uses the byte trick (byte & 0xF0) == 16*q_even and
//    ((byte << 4) & 0xF0) == 16*q_odd, with 1/16 folded into the block scale;
//  * wave reduction with DPP (row swaps, mirrors, row broadcasts).
#include <mutex>

#include "common.hpp"
#include "gemv.hpp"

namespace atlas {

// x lives in LDS as 16-byte pieces with one empty piece after every 16
// (piece p at p + p / 16).  A lane's chunk reads PPC <= 8 consecutive pieces
// starting at a multiple of PPC, which never straddle a gap, so the reads
// take immediate offsets from one base address; the gaps spread the lanes
// of a 16-lane group over distinct banks for every PPC in {1, 2, 4, 8}.
__device__ __forceinline__ int xpad(int p) { return p + (p >> 4); }

template <int FMT> struct WT;
template <> struct WT<WF_F32>  { static constexpr int EPC = 4;  };   // elems per 16 B
template <> struct WT<WF_BF16> { static constexpr int EPC = 8;  };
template <> struct WT<WF_I8>   { static constexpr int EPC = 16; };
template <> struct WT<WF_I4>   { static constexpr int EPC = 32; };

// dot of one 16-byte weight chunk with its EPC x values (padded LDS layout;
// p0 is the chunk's first piece, a multiple of the pieces per chunk).
template <int FMT>
__device__ __forceinline__ float chunk_dot(const u32x4 w, const f32x4* __restrict__ xs_all,
                                           int p0, float acc) {
    int b = xpad(p0);
    asm volatile("" : "+v"(b));    // one base address; the pieces take immediate offsets
    const f32x4* __restrict__ xs = xs_all + b;
    if constexpr (FMT == WF_F32) {
        f32x4 x = xs[0];
        acc += __uint_as_float(w.x) * x.x;
        acc += __uint_as_float(w.y) * x.y;
        acc += __uint_as_float(w.z) * x.z;
        acc += __uint_as_float(w.w) * x.w;
    } else if constexpr (FMT == WF_BF16) {
        f32x4 x0 = xs[0], x1 = xs[1];
        acc += bf16_lo(w.x) * x0.x;  acc += bf16_hi(w.x) * x0.y;
        acc += bf16_lo(w.y) * x0.z;  acc += bf16_hi(w.y) * x0.w;
        acc += bf16_lo(w.z) * x1.x;  acc += bf16_hi(w.z) * x1.y;
        acc += bf16_lo(w.w) * x1.z;  acc += bf16_hi(w.w) * x1.w;
    } else if constexpr (FMT == WF_I8) {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4 x = xs[j];
            acc += s8_at(ww[j], 0) * x.x;
            acc += s8_at(ww[j], 1) * x.y;
            acc += s8_at(ww[j], 2) * x.z;
            acc += s8_at(ww[j], 3) * x.w;
        }
    } else {  // WF_I4: returns sum of (16*q) * x over the 32 elements
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t hi = ww[j] & 0xF0F0F0F0u;          // even elements * 16
            const uint32_t lo = (ww[j] << 4) & 0xF0F0F0F0u;   // odd elements * 16
            f32x4 xa = xs[2 * j], xb = xs[2 * j + 1];
            acc += s8_at(hi, 0) * xa.x;
            acc += s8_at(lo, 0) * xa.y;
            acc += s8_at(hi, 1) * xa.z;
            acc += s8_at(lo, 1) * xa.w;
            acc += s8_at(hi, 2) * xb.x;
            acc += s8_at(lo, 2) * xb.y;
            acc += s8_at(hi, 3) * xb.z;
            acc += s8_at(lo, 3) * xb.w;
        }
    }
    return acc;
}


// ---------------------------------------------------------------------------
// x staging with the fused prologues (all 256 threads of the block call it).
// PRO_RESNORM / PRO_RMSNORM follow rmsnorm_inplace (crates/atlas-model/src/
// lib.rs:335-342): inv = 1/sqrt(sum(v^2)/n + eps), v*inv*w, and the post-norm
// residual x + normed (lib.rs:985-993); PRO_SILU is FeedForward's
// silu(gate) * up (lib.rs:918-921) over interleaved (gate, up) pairs.
// ---------------------------------------------------------------------------
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) s += red[i];
    return s;
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// Staging comes in two halves: `*_issue` sends every global read of x (and
// of the prologue's vectors) and `*_finish` consumes them.  Where the first
// weight loads go relative to them is a per-format choice (the kernel body
// explains it).
//
// Register staging: a thread owns the 16-byte pieces p = tid + 256 j,
// j < PPT; a norm prologue costs one round trip, not two (sum of squares,
// then x, w).
template <int PPT>
struct XRegs { f32x4 x[PPT], y[PPT], w[PPT]; };

// guarded loads: only the vectors the prologue uses, only pieces below K
template <int PPT, int NT = 256, bool N2 = false>
__device__ __forceinline__ void stage_regs_issue(const GemvArgs& a, XRegs<PPT>& r, int K) {
    const int np = K >> 2;
    const f32x4* xin = reinterpret_cast<const f32x4*>(a.x);
    const f32x4* yin = reinterpret_cast<const f32x4*>(a.pro_y);
    const f32x4* win = reinterpret_cast<const f32x4*>(a.pro_w);
    const bool norm2 = N2 && a.pro == PRO_RESNORM_NORM;
    const bool res = a.pro == PRO_RESNORM || norm2, norm = res || a.pro == PRO_RMSNORM;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int p = threadIdx.x + NT * j;
        if (p < np) {
            r.x[j] = xin[p];
            if (res) r.y[j] = yin[p];
            if (norm) r.w[j] = win[p];
        }
    }
}

// unconditional buffer loads: a vector the prologue does not use gets an
// empty range and reads as zeros without touching memory, as do pieces past
// K.  Guarded loads split the issue into branches, after which the compiler
// waits for every load in flight, including weight loads issued between
// the two halves.
template <int PPT, int NT = 256, bool N2 = false>
__device__ __forceinline__ void stage_regs_issue_buf(const GemvArgs& a, XRegs<PPT>& r, int K) {
    const bool norm2 = N2 && a.pro == PRO_RESNORM_NORM;
    const bool res = a.pro == PRO_RESNORM || norm2, norm = res || a.pro == PRO_RMSNORM;
    const __amdgpu_buffer_rsrc_t xb =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.x), (short)0, K * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t yb = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(res ? a.pro_y : a.x), (short)0, res ? K * 4 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t wb = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(norm ? a.pro_w : a.x), (short)0, norm ? K * 4 : 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int off = (int)threadIdx.x * 16;
        r.x[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xb, off, NT * 16 * j, 0));
        r.y[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(yb, off, NT * 16 * j, 0));
        r.w[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wb, off, NT * 16 * j, 0));
    }
}

template <bool SWZ, int PPT, int NT = 256, bool N2 = false>
__device__ __forceinline__ void stage_regs_finish(const GemvArgs& a, XRegs<PPT>& r, f32x4* xs,
                                                  int K) {
    __shared__ float red[NT / 64], red2[NT / 64];
    const int np = K >> 2;
    const bool norm2 = N2 && a.pro == PRO_RESNORM_NORM;
    const bool res = a.pro == PRO_RESNORM || norm2, norm = res || a.pro == PRO_RMSNORM;
    const f32x4 (&xv)[PPT] = r.x;
    const f32x4 (&yv)[PPT] = r.y;
    const f32x4 (&wv)[PPT] = r.w;
    float inv = 1.0f;
    if (norm) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < PPT; ++j) {
            if (threadIdx.x + NT * j < np) {
                const f32x4 t = res ? yv[j] : xv[j];
                ss += t.x * t.x;
                ss += t.y * t.y;
                ss += t.z * t.z;
                ss += t.w * t.w;
            }
        }
        ss = block_sum<NT / 64>(ss, red);
        inv = 1.0f / sqrtf(ss / (float)K + a.pro_eps);
    }
    const bool write_out = a.pro_out && blockIdx.x == 0 && norm;
    f32x4 v[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        if (res) v[j] = xv[j] + (yv[j] * inv) * wv[j];
        else if (norm) v[j] = (xv[j] * inv) * wv[j];
        else v[j] = xv[j];
    }
    // RESNORM_NORM: the final norm of the residual-updated h (second reduction).
    // Its weight is loaded only now, into registers the first norm's inputs
    // have freed: loaded with them, it cost the kernel a block per CU of
    // occupancy (+16 VGPRs), more than this round trip costs the one launch.
    float inv2 = 1.0f;
    f32x4 w2[N2 ? PPT : 1];
    if constexpr (N2) {
        const __amdgpu_buffer_rsrc_t w2b = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(norm2 ? a.pro_w2 : a.x), (short)0, norm2 ? K * 4 : 0, 0x00020000);
#pragma unroll
        for (int j = 0; j < PPT; ++j)
            w2[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  w2b, (int)threadIdx.x * 16, NT * 16 * j, 0));
    }
    if constexpr (N2) if (norm2) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < PPT; ++j) {
            if (threadIdx.x + NT * j < np) {
                ss += v[j].x * v[j].x;
                ss += v[j].y * v[j].y;
                ss += v[j].z * v[j].z;
                ss += v[j].w * v[j].w;
            }
        }
        ss = block_sum<NT / 64>(ss, red2);
        inv2 = 1.0f / sqrtf(ss / (float)K + a.pro_eps);
    }
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int p = threadIdx.x + NT * j;
        if (p < np) {
            if constexpr (N2) xs[SWZ ? xpad(p) : p] = norm2 ? (v[j] * inv2) * w2[j] : v[j];
            else xs[SWZ ? xpad(p) : p] = v[j];
            if (write_out) reinterpret_cast<f32x4*>(a.pro_out)[p] = v[j];
        }
    }
}

// Plain x (no prologue) of up to 256 * PPT pieces, one round trip for any K
// the registers hold (PPT = 12: K <= 12288).  Buffer loads address all
// pieces from one VGPR offset (the piece stride goes in the SGPR offset),
// and reads past the end of x return zeros that are never stored.
template <int PPT, int NT = 256>
__device__ __forceinline__ void stage_plain_issue(const GemvArgs& a, f32x4 (&xv)[PPT], int K) {
    const __amdgpu_buffer_rsrc_t xb =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.x), (short)0, K * 4, 0x00020000);
#pragma unroll
    for (int j = 0; j < PPT; ++j)
        xv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              xb, (int)threadIdx.x * 16, NT * 16 * j, 0));
}

template <bool SWZ, int PPT, int NT = 256>
__device__ __forceinline__ void stage_plain_finish(const f32x4 (&xv)[PPT], f32x4* xs, int K) {
    const int np = K >> 2;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int p = threadIdx.x + NT * j;
        if (p < np) xs[SWZ ? xpad(p) : p] = xv[j];
    }
}

// Which staging a batch-1 launch takes.  The register staging also takes
// plain x at K <= 4096 (four loads per thread, where the plain path's
// twelve would mostly read past K).
enum { STAGE_REGS = 0, STAGE_PLAIN = 1, STAGE_LOOP = 2 };
__device__ __forceinline__ int stage_kind(const GemvArgs& a, int K) {
    if (a.pro != PRO_SILU && K <= 256 * 4 * 4) return STAGE_REGS;    // d_model <= 4096: 48 VGPRs
    if (a.pro == PRO_X && K <= 256 * 4 * 12) return STAGE_PLAIN;     // e.g. the W_down input
    return STAGE_LOOP;
}

// Looped staging: any K the LDS holds, and the SwiGLU prologue.
template <bool SWZ, int NT = 256, bool N2 = false>
__device__ __forceinline__ void stage_x_loop(const GemvArgs& a, f32x4* xs, int K) {
    __shared__ float red[NT / 64], red2[NT / 64];
    const int np = K >> 2;
    const f32x4* xin = reinterpret_cast<const f32x4*>(a.x);
    const bool norm2 = N2 && a.pro == PRO_RESNORM_NORM;
    const bool res = a.pro == PRO_RESNORM || norm2;
    float inv = 1.0f;
    if (res || a.pro == PRO_RMSNORM) {
        const f32x4* v = reinterpret_cast<const f32x4*>(res ? a.pro_y : a.x);
        float ss = 0.f;
        for (int p = threadIdx.x; p < np; p += NT) {
            const f32x4 t = v[p];
            ss += t.x * t.x;
            ss += t.y * t.y;
            ss += t.z * t.z;
            ss += t.w * t.w;
        }
        ss = block_sum<NT / 64>(ss, red);
        inv = 1.0f / sqrtf(ss / (float)K + a.pro_eps);
    }
    const bool write_out = a.pro_out && blockIdx.x == 0 && (res || a.pro == PRO_RMSNORM);
    float ss2 = 0.f;
    for (int p = threadIdx.x; p < np; p += NT) {
        f32x4 r;
        if (a.pro == PRO_X) {
            r = xin[p];
        } else if (res) {
            const f32x4 yi = reinterpret_cast<const f32x4*>(a.pro_y)[p];
            const f32x4 wi = reinterpret_cast<const f32x4*>(a.pro_w)[p];
            r = xin[p] + (yi * inv) * wi;
        } else if (a.pro == PRO_RMSNORM) {
            const f32x4 wi = reinterpret_cast<const f32x4*>(a.pro_w)[p];
            r = (xin[p] * inv) * wi;
        } else {   // PRO_SILU
            const f32x4* pr = reinterpret_cast<const f32x4*>(a.pro_y);
            const f32x4 g0 = pr[2 * p], g1 = pr[2 * p + 1];
            r = f32x4{silu_f(g0.x) * g0.y, silu_f(g0.z) * g0.w, silu_f(g1.x) * g1.y,
                      silu_f(g1.z) * g1.w};
        }
        xs[SWZ ? xpad(p) : p] = r;
        if (write_out) reinterpret_cast<f32x4*>(a.pro_out)[p] = r;
        if (norm2) ss2 += r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w;
    }
    if (norm2) {
        // the final norm of h, over the pieces this thread staged
        ss2 = block_sum<NT / 64>(ss2, red2);
        const float inv2 = 1.0f / sqrtf(ss2 / (float)K + a.pro_eps);
        for (int p = threadIdx.x; p < np; p += NT)
            xs[SWZ ? xpad(p) : p] = (xs[SWZ ? xpad(p) : p] * inv2) *
                                    reinterpret_cast<const f32x4*>(a.pro_w2)[p];
    }
}

// NX dot products of one 16-byte weight chunk with NX staged x vectors (the
// weights are dequantised once): acc[n] += sum_e w_e * x_n[e], x vector n at
// xs_all + n * npad.  The int4 path returns sums of 16 * q like chunk_dot.
template <int FMT, int NX>
__device__ __forceinline__ void chunk_dot_nx(const u32x4 w, const f32x4* __restrict__ xs_all,
                                             int npad, int p0, float (&acc)[NX]) {
    constexpr int EPC = WT<FMT>::EPC;
    float v[EPC];
    if constexpr (FMT == WF_F32) {
        v[0] = __uint_as_float(w.x); v[1] = __uint_as_float(w.y);
        v[2] = __uint_as_float(w.z); v[3] = __uint_as_float(w.w);
    } else if constexpr (FMT == WF_BF16) {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[2 * j] = bf16_lo(ww[j]); v[2 * j + 1] = bf16_hi(ww[j]); }
    } else if constexpr (FMT == WF_I8) {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * j + b] = s8_at(ww[j], b);
    } else {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t hi = ww[j] & 0xF0F0F0F0u;          // even elements * 16
            const uint32_t lo = (ww[j] << 4) & 0xF0F0F0F0u;   // odd elements * 16
#pragma unroll
            for (int b = 0; b < 4; ++b) { v[8 * j + 2 * b] = s8_at(hi, b); v[8 * j + 2 * b + 1] = s8_at(lo, b); }
        }
    }
    int base = xpad(p0);
    asm volatile("" : "+v"(base));
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        const f32x4* __restrict__ xs = xs_all + n * npad + base;
        float t = acc[n];
#pragma unroll
        for (int j = 0; j < EPC / 4; ++j) {
            const f32x4 x = xs[j];
            t += v[4 * j] * x.x;
            t += v[4 * j + 1] * x.y;
            t += v[4 * j + 2] * x.z;
            t += v[4 * j + 3] * x.w;
        }
        acc[n] = t;
    }
}

// Plain staging of NX x rows (row n at a.x + n * x_stride_n, 16-byte aligned)
// into the padded layout, row n at xs + n * npad.  One row's loads are all in
// flight before its stores.
template <int NX>
__device__ __forceinline__ void stage_xn(const GemvArgs& a, f32x4* xs, int K, int npad) {
    const int np = K >> 2;
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        const __amdgpu_buffer_rsrc_t xb = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(a.x + (long)n * a.x_stride_n), (short)0, K * 4, 0x00020000);
        f32x4 xv[12];
#pragma unroll
        for (int j = 0; j < 12; ++j)
            if (256 * j < np)
                xv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      xb, (int)threadIdx.x * 16, 4096 * j, 0));
#pragma unroll
        for (int j = 0; j < 12; ++j) {
            const int p = threadIdx.x + 256 * j;
            if (256 * j < np && p < np) xs[n * npad + xpad(p)] = xv[j];
        }
    }
}

// ordered (value, index) key: larger value wins, ties keep the larger index
__device__ __forceinline__ unsigned long long argkey_f(float v, int i) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)i;
}

template <int FMT, int ROWS, int UNROLL, int NX = 1>
__global__ __launch_bounds__(256) void gemv_n1_kernel(GemvArgs a) {
    // NX > 1: NX activation rows share every weight load (a small ragged
    // batch); plain x only, store / SwiGLU epilogues, y[n] at n * y_stride_n
    extern __shared__ f32x4 xs[];
    constexpr int EPC = WT<FMT>::EPC;
    constexpr int PPC = EPC / 4;                  // 16-byte x pieces per chunk
    constexpr int STEP = 64 * UNROLL;             // chunks per wave iteration
    const int K = a.K, M = a.M;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int chunks = K / EPC;                   // 16-byte chunks per row
    const long ldc = a.ldw > 0 ? a.ldw / 16 : chunks;   // chunks between rows
    const u32x4* W = reinterpret_cast<const u32x4*>(a.w);
    // One-row waves with the SwiGLU epilogue take a (gate, up) row pair one
    // row after the other (SEQ = 2): the pair's epilogue stays in the wave
    // without the registers of a two-row wave.
    const int SEQ = (ROWS == 1 && a.epi == EPI_SILU_MUL) ? 2 : 1;
    const int n_groups = ((M + ROWS - 1) / ROWS + SEQ - 1) / SEQ;
    // persistent waves: wave w of the grid takes row groups w, w + S, ...
    const int S = gridDim.x * 4;
    const int g0 = blockIdx.x * 4 + wave;
    const int iters = (chunks + STEP - 1) / STEP;
    const int my_groups = g0 < n_groups ? (n_groups - 1 - g0) / S + 1 : 0;
    const int total = my_groups * SEQ * iters;    // (group, row, k-slice) steps of this wave
    // first row of step `it`
    auto row_of = [&](int it) {
        return ((g0 + (it / (iters * SEQ)) * S) * SEQ + (it / iters) % SEQ) * ROWS;
    };

    // Weights (and raw int4 block scales) of step `it` into registers.  The
    // loads are unconditional (chunk and row clamped into the matrix; the
    // compute skips lanes past the row end) and nothing consumes them here,
    // so the prefetch never forces a wait on the loads in flight.
    auto load = [&](int it, u32x4 (&wb)[UNROLL][ROWS], float (&sb)[UNROLL][ROWS]) {
        const int g = row_of(it) / ROWS;
        const int c0 = lane + (it % iters) * STEP;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int c = min(c0 + 64 * u, chunks - 1);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const int row = g * ROWS + r < M ? g * ROWS + r : M - 1;
                wb[u][r] = ldg_stream(W + (long)row * ldc + c);
                if constexpr (FMT == WF_I4) {
                    long bi;
                    if (a.bpr > 0) bi = (long)row * a.bpr + (a.cpb == 1 ? c : c / a.cpb);
                    else bi = ((long)row * K + (long)c * EPC) / a.block;
                    sb[u][r] = a.scales[bi];
                }
            }
        }
    };

    u32x4 cur[UNROLL][ROWS];
    float scur[UNROLL][ROWS];
    // Where the first weight step goes relative to x's reads.  Vector loads
    // return in order, so x read after a grid-wide burst of weight loads
    // arrives only when that burst has, and the next weight step goes out
    // only then.  bf16 and int8 still do best with the weights first
    // (measured at the 7B shapes): their 16-byte loads per lane and step
    // keep HBM busy across the staging.  int4 waves read 4 bytes of weights
    // per 32 x values and gain from x first (4096 x 4096: 5.8 -> 5.3 us;
    // 11008 x 4096: 10.3 -> 9.4 us).  In that order the first weight step is
    // loaded even by a wave without rows (row and chunk are clamped into the
    // matrix): a load under a branch would make the compiler wait for it
    // before x's last piece is stored.
    const int npad = (K >> 2) + ((K >> 2) + 15) / 16;     // padded pieces per x row
    if constexpr (NX == 1) {
        const int kind = stage_kind(a, K);
        if constexpr (FMT == WF_I4) {
            if (kind == STAGE_REGS) {
                XRegs<4> r;
                stage_regs_issue_buf<4>(a, r, K);
                __builtin_amdgcn_sched_barrier(0);
                load(0, cur, scur);
                stage_regs_finish<true, 4>(a, r, xs, K);
            } else if (kind == STAGE_PLAIN) {
                f32x4 xv[12];
                stage_plain_issue<12>(a, xv, K);
                __builtin_amdgcn_sched_barrier(0);
                load(0, cur, scur);
                stage_plain_finish<true, 12>(xv, xs, K);
            } else {
                load(0, cur, scur);
                stage_x_loop<true>(a, xs, K);
            }
        } else {
            if (total > 0) load(0, cur, scur);
            if (kind == STAGE_REGS) {
                XRegs<4> r;
                stage_regs_issue<4>(a, r, K);
                stage_regs_finish<true, 4>(a, r, xs, K);
            } else if (kind == STAGE_PLAIN) {
                f32x4 xv[12];
                stage_plain_issue<12>(a, xv, K);
                stage_plain_finish<true, 12>(xv, xs, K);
            } else {
                stage_x_loop<true>(a, xs, K);
            }
        }
    } else {
        if (total > 0) load(0, cur, scur);
        stage_xn<NX>(a, xs, K, npad);
    }
    __syncthreads();

    float acc[ROWS][NX];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int n = 0; n < NX; ++n) acc[r][n] = 0.0f;
    unsigned long long best = 0;          // EPI_ARGMAX: best (logit, row) of this wave
    float gate[NX];                       // SEQ == 2: the pair's gate row
#pragma unroll
    for (int n = 0; n < NX; ++n) gate[n] = 0.0f;

    for (int it = 0; it < total; ++it) {
        u32x4 nxt[UNROLL][ROWS];
        float snx[UNROLL][ROWS];
        if (it + 1 < total) load(it + 1, nxt, snx);     // one step of prefetch
        const int ks = it % iters;
        const int c0 = lane + ks * STEP;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int c = c0 + 64 * u;
            if (c < chunks) {
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    if constexpr (NX == 1) {
                        if constexpr (FMT == WF_I4)
                            acc[r][0] += scur[u][r] * chunk_dot<FMT>(cur[u][r], xs, c * PPC, 0.0f);
                        else
                            acc[r][0] = chunk_dot<FMT>(cur[u][r], xs, c * PPC, acc[r][0]);
                    } else if constexpr (FMT == WF_I4) {
                        float t[NX];
#pragma unroll
                        for (int n = 0; n < NX; ++n) t[n] = 0.0f;
                        chunk_dot_nx<FMT, NX>(cur[u][r], xs, npad, c * PPC, t);
#pragma unroll
                        for (int n = 0; n < NX; ++n) acc[r][n] += scur[u][r] * t[n];
                    } else {
                        chunk_dot_nx<FMT, NX>(cur[u][r], xs, npad, c * PPC, acc[r]);
                    }
                }
            }
        }
        if (ks == iters - 1) {
            // end of this row group: reduce across the wave and store
            const int r0 = row_of(it);
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
#pragma unroll
                for (int n = 0; n < NX; ++n) acc[r][n] = wave_sum(acc[r][n]);
            if constexpr (FMT == WF_I4) {
                // the chunks hold 16 * q: one exact power-of-two rescale per row
#pragma unroll
                for (int r = 0; r < ROWS; ++r)
#pragma unroll
                    for (int n = 0; n < NX; ++n) acc[r][n] *= 0.0625f;
            }
            if constexpr (FMT == WF_I8) {
                // scalar loads (constant address space): no vector-memory wait
                const __attribute__((address_space(4))) float* cs =
                    (const __attribute__((address_space(4))) float*)a.scales;
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const float sc = cs[r0 + r < M ? r0 + r : M - 1];
#pragma unroll
                    for (int n = 0; n < NX; ++n) acc[r][n] *= sc;
                }
            }
            if constexpr (NX == 1) {
                if (a.epi == EPI_SILU_MUL) {
                    // rows (2i, 2i+1) = (gate_i, up_i): y[i] = silu(gate) * up
                    if constexpr (ROWS % 2 == 0) {
#pragma unroll
                        for (int r = 0; r < ROWS; r += 2)
                            if (lane == r && r0 + r + 1 < M)
                                a.y[(r0 + r) >> 1] = silu_f(acc[r][0]) * acc[r + 1][0];
                    } else if (ROWS == 1) {
                        if ((r0 & 1) == 0) gate[0] = acc[0][0];
                        else if (lane == 0 && r0 < M) a.y[r0 >> 1] = silu_f(gate[0]) * acc[0][0];
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < ROWS; ++r)
                        if (lane == r && r0 + r < M) a.y[r0 + r] = acc[r][0];
                    if (a.epi == EPI_ARGMAX) {
#pragma unroll
                        for (int r = 0; r < ROWS; ++r)
                            if (r0 + r < M) {
                                const unsigned long long k = argkey_f(acc[r][0], r0 + r);
                                best = k > best ? k : best;
                            }
                    }
                }
            } else {
                // lane n * ROWS + r stores (row r0 + r, sequence n)
                if (a.epi == EPI_SILU_MUL) {
                    if constexpr (ROWS % 2 == 0) {
#pragma unroll
                        for (int n = 0; n < NX; ++n)
#pragma unroll
                            for (int r = 0; r < ROWS; r += 2)
                                if (lane == n * ROWS + r && r0 + r + 1 < M)
                                    a.y[n * a.y_stride_n + (long)((r0 + r) >> 1) * a.y_stride_m] =
                                        silu_f(acc[r][n]) * acc[r + 1][n];
                    } else if (ROWS == 1) {
#pragma unroll
                        for (int n = 0; n < NX; ++n) {
                            if ((r0 & 1) == 0) gate[n] = acc[0][n];
                            else if (lane == n && r0 < M)
                                a.y[n * a.y_stride_n + (long)(r0 >> 1) * a.y_stride_m] =
                                    silu_f(gate[n]) * acc[0][n];
                        }
                    }
                } else {
#pragma unroll
                    for (int n = 0; n < NX; ++n)
#pragma unroll
                        for (int r = 0; r < ROWS; ++r)
                            if (lane == n * ROWS + r && r0 + r < M)
                                a.y[n * a.y_stride_n + (long)(r0 + r) * a.y_stride_m] = acc[r][n];
                }
            }
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
#pragma unroll
                for (int n = 0; n < NX; ++n) acc[r][n] = 0.0f;
        }
        if (it + 1 < total) {
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    cur[u][r] = nxt[u][r];
                    scur[u][r] = snx[u][r];
                }
        }
    }
    if (a.epi == EPI_ARGMAX && lane == 0) a.arg_part[blockIdx.x * 4 + wave] = best;
}

// ---------------------------------------------------------------------------
// The batch-1 decode GEMV.  Same work split, staging, prologues and
// epilogues as gemv_n1_kernel at NX = 1, with the inner loop rebuilt for
// instruction count (the VALU issue rate limits int4 and weighs on int8):
//  * a wave walks its (row group, k step) sequence with a cursor advanced
//    by adds (no divisions per step); row addresses are wave-uniform and
//    every row is its own buffer resource, so the loads take one VGPR of
//    lane offset, the step offset in an SGPR and the unroll offset as an
//    immediate, and chunks past a row's end read as zeros (no clamps: x's
//    LDS copy is zero-padded to whole steps, so those chunks add nothing);
//  * the x pieces of a chunk are read once from LDS for all ROWS rows;
//  * int4 nibbles become f16 by the magic-number trick and multiply f32 x
//    in v_fma_mix_f32 (one instruction per weight, conversion ~0.75 per
//    weight), with exact per-chunk offset corrections (below).
// ---------------------------------------------------------------------------

// int4 chunk (32 weights, 4 words; word j holds elements 8j..8j+7, the even
// element of a byte in its high nibble).  With n = s ^ 8 = q + 8 for the
// stored nibble s of the signed value q, (w & 0x000F000F) ^ 0x64086408 is
// the f16 pair (1024 + n1, 1024 + n5) of the word's odd elements in bytes 0
// and 2 (0x6400 = 1024 leaves the low mantissa bits free, so the XOR sets
// the exponent and flips the nibble's sign bit at once: one v_bitop3); with
// mask 0x00F000F0 and 0x64806480 the even elements give (1024 + 16 n0,
// 1024 + 16 n4); w >> 8 gives bytes 1 and 3.  Hence with sums acc_o over odd
// and acc_e over even elements,
//   sum_k q_k x_k = acc_e / 16 + acc_o - (72 S_even + 1032 S_odd),
// S_* the chunk's x sums, whose weighted sum `corr` is staged per chunk.
// Every f16 here is an exact integer; fma_mix rounds like an f32 FMA.
__device__ __forceinline__ void fma_mix_lo(float& acc, uint32_t pair, float x) {
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(pair), "v"(x));
}
__device__ __forceinline__ void fma_mix_hi(float& acc, uint32_t pair, float x) {
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "+v"(acc) : "v"(pair), "v"(x));
}

// one word (8 weights) of an int4 chunk into the odd / even sums
__device__ __forceinline__ void i4_word_mix(uint32_t w, const f32x4 xa, const f32x4 xb, float& ao,
                                            float& ae) {
    const uint32_t t8 = w >> 8;
    const uint32_t o15 = (w & 0x000F000Fu) ^ 0x64086408u;   // elements 1, 5
    const uint32_t e04 = (w & 0x00F000F0u) ^ 0x64806480u;   // elements 0, 4 (x16)
    const uint32_t o37 = (t8 & 0x000F000Fu) ^ 0x64086408u;  // elements 3, 7
    const uint32_t e26 = (t8 & 0x00F000F0u) ^ 0x64806480u;  // elements 2, 6 (x16)
    fma_mix_lo(ao, o15, xa.y);
    fma_mix_hi(ao, o15, xb.y);
    fma_mix_lo(ao, o37, xa.w);
    fma_mix_hi(ao, o37, xb.w);
    fma_mix_lo(ae, e04, xa.x);
    fma_mix_hi(ae, e04, xb.x);
    fma_mix_lo(ae, e26, xa.z);
    fma_mix_hi(ae, e26, xb.z);
}

// dot of a 16-byte chunk with its x pieces (bf16 / int8 / f32)
template <int FMT>
__device__ __forceinline__ float chunk_dot_x(const u32x4 w, const f32x4 (&x)[WT<FMT>::EPC / 4],
                                             float acc) {
    if constexpr (FMT == WF_F32) {
        acc += __uint_as_float(w.x) * x[0].x;
        acc += __uint_as_float(w.y) * x[0].y;
        acc += __uint_as_float(w.z) * x[0].z;
        acc += __uint_as_float(w.w) * x[0].w;
    } else if constexpr (FMT == WF_BF16) {
        acc += bf16_lo(w.x) * x[0].x;  acc += bf16_hi(w.x) * x[0].y;
        acc += bf16_lo(w.y) * x[0].z;  acc += bf16_hi(w.y) * x[0].w;
        acc += bf16_lo(w.z) * x[1].x;  acc += bf16_hi(w.z) * x[1].y;
        acc += bf16_lo(w.w) * x[1].z;  acc += bf16_hi(w.w) * x[1].w;
    } else {   // WF_I8
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc += s8_at(ww[j], 0) * x[j].x;
            acc += s8_at(ww[j], 1) * x[j].y;
            acc += s8_at(ww[j], 2) * x[j].z;
            acc += s8_at(ww[j], 3) * x[j].w;
        }
    }
    return acc;
}

// Pieces of x a row's steps read: whole steps, past K zero-filled.
__host__ __device__ inline int v4_pieces(int fmt, int K, int U) {
    const int epc = fmt == WF_F32 ? 4 : fmt == WF_BF16 ? 8 : fmt == WF_I8 ? 16 : 32;
    const int chunks = K / epc, step = 64 * U;
    return (chunks + step - 1) / step * step * (epc / 4);
}

// LDS bytes of the v4 kernel: padded x pieces, plus int4 per-chunk corrections
inline size_t v4_lds_bytes(int fmt, int K, int U) {
    const size_t np = (size_t)v4_pieces(fmt, K, U);
    size_t b = (np + (np + 15) / 16) * 16;
    if (fmt == WF_I4) b += np / 8 * 4;           // one float per 32-element chunk
    return b;
}

template <int FMT, int ROWS, int U, int NW, bool N2>
__global__ __launch_bounds__(64 * NW) void gemv_v4_kernel(GemvArgs a) {
    extern __shared__ f32x4 xs[];
    constexpr int NT = 64 * NW;               // threads per block
    constexpr int PR = 1024 / NT;             // register staging: 16-byte pieces per thread (K <= 4096)
    constexpr int PP = 3072 / NT;             // plain staging: pieces per thread (K <= 12288)
    static_assert(NW == 4 || NW == 8 || NW == 16, "4, 8 or 16 waves per block");
    constexpr int EPC = WT<FMT>::EPC;
    constexpr int PPC = EPC / 4;
    constexpr int STEP = 64 * U;
    const int K = a.K, M = a.M;
    const int lane = threadIdx.x & 63;
    // wave-uniform: the cursor, row addresses and buffer resources live in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int chunks = K / EPC;
    const int iters = (chunks + STEP - 1) / STEP;
    const uint32_t row_bytes = (uint32_t)(K / EPC) * 16u;
    const long pitch = a.ldw > 0 ? a.ldw : (long)row_bytes;
    const char* Wb = static_cast<const char*>(a.w);
    const int SEQ = (ROWS == 1 && a.epi == EPI_SILU_MUL) ? 2 : 1;
    const int n_groups = ((M + ROWS - 1) / ROWS + SEQ - 1) / SEQ;
    const int S = gridDim.x * NW;
    const int g0 = blockIdx.x * NW + wave;
    const int my_groups = g0 < n_groups ? (n_groups - 1 - g0) / S + 1 : 0;
    const int total = my_groups * SEQ * iters;
    // int4 block-scale indexing inside a row (K % block == 0, block = 32 * 2^sh):
    // chunk ch = ks * STEP + lane + 64 u uses scale (ch >> sh), split into a
    // uniform, a lane and an immediate part (STEP and 64 u are multiples of 2^sh)
    int sh = 0;
    if constexpr (FMT == WF_I4) while ((1 << sh) < a.cpb) ++sh;
    const int lane_soff = (lane >> sh) * 4;
    // x piece of chunk ch: xpad((ks * STEP + lane + 64 u) * PPC) splits the
    // same way (the step and unroll parts are multiples of 16 pieces)
    const int lane_x = xpad(lane * PPC);

    // ---- cursor over the wave's steps --------------------------------------
    struct Cur { int ks, sq, grp; };
    auto first_row = [&](const Cur& c) { return (c.grp * SEQ + c.sq) * ROWS; };
    auto advance = [&](Cur& c) {
        if (++c.ks == iters) {
            c.ks = 0;
            if (++c.sq == SEQ) { c.sq = 0; c.grp += S; }
        }
    };
    // one step's weights (and int4 raw block scales) for rows r0 .. r0+ROWS-1
    auto load = [&](const Cur& c, u32x4 (&wb)[U][ROWS], float (&sb)[U][ROWS]) {
        const int r0 = first_row(c);
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const int row = r0 + r;
            const bool ok = row < M;
            const char* rp = Wb + (long)(ok ? row : 0) * pitch;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                uniform_ptr(rp), (short)0,
                __builtin_amdgcn_readfirstlane(ok ? (int)row_bytes : 0), 0x00020000);
            const int soff = __builtin_amdgcn_readfirstlane(c.ks * STEP * 16);
#pragma unroll
            for (int u = 0; u < U; ++u)
                wb[u][r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         rs, lane * 16 + u * 1024, soff, 2));
            if constexpr (FMT == WF_I4) {
                const float* sp = a.scales + (long)(ok ? row : 0) * a.bpr;
                const __amdgpu_buffer_rsrc_t ss = __builtin_amdgcn_make_buffer_rsrc(
                    uniform_ptr(sp), (short)0, __builtin_amdgcn_readfirstlane(ok ? a.bpr * 4 : 0),
                    0x00020000);
                const int s_soff = __builtin_amdgcn_readfirstlane(((c.ks * STEP) >> sh) * 4);
#pragma unroll
                for (int u = 0; u < U; ++u)
                    sb[u][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                             ss, lane_soff + ((64 * u) >> sh) * 4, s_soff, 0));
            }
        }
    };

    // ---- x staging (as gemv_n1_kernel), zero tail, int4 corrections --------
    u32x4 bufA[U][ROWS], bufB[U][ROWS];
    float sA[U][ROWS], sB[U][ROWS];
    Cur cl{0, 0, g0};        // next step to load
    const int kind = stage_kind(a, K);
    if constexpr (FMT == WF_I4) {
        if (kind == STAGE_REGS) {
            XRegs<PR> r;
            stage_regs_issue_buf<PR, NT, N2>(a, r, K);
            __builtin_amdgcn_sched_barrier(0);
            load(cl, bufA, sA);
            stage_regs_finish<true, PR, NT, N2>(a, r, xs, K);
        } else if (kind == STAGE_PLAIN) {
            f32x4 xv[PP];
            stage_plain_issue<PP, NT>(a, xv, K);
            __builtin_amdgcn_sched_barrier(0);
            load(cl, bufA, sA);
            stage_plain_finish<true, PP, NT>(xv, xs, K);
        } else {
            load(cl, bufA, sA);
            stage_x_loop<true, NT, N2>(a, xs, K);
        }
    } else {
        load(cl, bufA, sA);
        if (kind == STAGE_REGS) {
            XRegs<PR> r;
            stage_regs_issue<PR, NT, N2>(a, r, K);
            stage_regs_finish<true, PR, NT, N2>(a, r, xs, K);
        } else if (kind == STAGE_PLAIN) {
            f32x4 xv[PP];
            stage_plain_issue<PP, NT>(a, xv, K);
            stage_plain_finish<true, PP, NT>(xv, xs, K);
        } else {
            stage_x_loop<true, NT, N2>(a, xs, K);
        }
    }
    advance(cl);
    const int np = K >> 2;
    const int np_all = iters * STEP * PPC;
    for (int p = np + (int)threadIdx.x; p < np_all; p += NT) xs[xpad(p)] = f32x4{0.f, 0.f, 0.f, 0.f};
    float* corr = nullptr;
    if constexpr (FMT == WF_I4) {
        __syncthreads();
        corr = reinterpret_cast<float*>(xs + (np_all + (np_all + 15) / 16));
        for (int c = threadIdx.x; c < iters * STEP; c += NT) {
            const int b = xpad(c * PPC);
            float se = 0.f, so = 0.f;
#pragma unroll
            for (int j = 0; j < PPC; ++j) {
                const f32x4 v = xs[b + j];
                se += v.x; so += v.y; se += v.z; so += v.w;
            }
            corr[c] = 72.0f * se + 1032.0f * so;
        }
    }
    __syncthreads();

    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
    unsigned long long best = 0;
    float gate = 0.0f;
    Cur cc{0, 0, g0};        // step being computed

    auto compute = [&](const Cur& c, const u32x4 (&wb)[U][ROWS], const float (&sb)[U][ROWS]) {
        const int xs_step = xpad(c.ks * STEP * PPC);             // uniform
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const f32x4* xb = xs + xs_step + xpad(64 * u * PPC) + lane_x;
            if constexpr (FMT == WF_I4) {
                // two x pieces (one word of every row) at a time
                float ao[ROWS], ae[ROWS];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) { ao[r] = 0.f; ae[r] = 0.f; }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 xa = xb[2 * j], xc = xb[2 * j + 1];
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) {
                        const u32x4 w = wb[u][r];
                        const uint32_t wj = j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w;
                        i4_word_mix(wj, xa, xc, ao[r], ae[r]);
                    }
                }
                const float cr = corr[c.ks * STEP + 64 * u + lane];
#pragma unroll
                for (int r = 0; r < ROWS; ++r)
                    acc[r] = fmaf(sb[u][r], fmaf(ae[r], 0.0625f, ao[r]) - cr, acc[r]);
            } else {
                f32x4 x[PPC];
#pragma unroll
                for (int j = 0; j < PPC; ++j) x[j] = xb[j];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) acc[r] = chunk_dot_x<FMT>(wb[u][r], x, acc[r]);
            }
        }
        if (c.ks == iters - 1) {
            const int r0 = first_row(c);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = wave_sum(acc[r]);
            if constexpr (FMT == WF_I8) {
                // row scales through the constant address space: wave-uniform
                // scalar loads (lgkmcnt), so no vector-memory wait here drains
                // the next buffer's weight loads
                const __attribute__((address_space(4))) float* cs =
                    (const __attribute__((address_space(4))) float*)a.scales;
#pragma unroll
                for (int r = 0; r < ROWS; ++r) acc[r] *= cs[r0 + r < M ? r0 + r : M - 1];
            }
            if (a.epi == EPI_SILU_MUL) {
                if constexpr (ROWS % 2 == 0) {
#pragma unroll
                    for (int r = 0; r < ROWS; r += 2)
                        if (lane == r && r0 + r + 1 < M) a.y[(r0 + r) >> 1] = silu_f(acc[r]) * acc[r + 1];
                } else if (ROWS == 1) {
                    if ((r0 & 1) == 0) gate = acc[0];
                    else if (lane == 0 && r0 < M) a.y[r0 >> 1] = silu_f(gate) * acc[0];
                }
            } else {
#pragma unroll
                for (int r = 0; r < ROWS; ++r)
                    if (lane == r && r0 + r < M) a.y[r0 + r] = acc[r];
                if (a.epi == EPI_ARGMAX) {
#pragma unroll
                    for (int r = 0; r < ROWS; ++r)
                        if (r0 + r < M) {
                            const unsigned long long k = argkey_f(acc[r], r0 + r);
                            best = k > best ? k : best;
                        }
                }
            }
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
        }
    };

    // Two register buffers, renamed by unrolling the step loop by two.  The
    // prefetch is unconditional: past the wave's last step the cursor names
    // rows >= M, whose buffer resources have size 0, so those loads return
    // zeros without touching memory.  A conditional prefetch would give the
    // compiler a path without the next buffer's loads, and the wait count it
    // merges for both paths (the smaller one) would then drain the prefetch
    // before every other step.
    for (int t = 0; t < total; t += 2) {
        load(cl, bufB, sB);
        advance(cl);
        compute(cc, bufA, sA);
        advance(cc);
        if (t + 1 >= total) break;
        load(cl, bufA, sA);
        advance(cl);
        compute(cc, bufB, sB);
        advance(cc);
    }
    if (a.epi == EPI_ARGMAX && lane == 0) a.arg_part[blockIdx.x * NW + wave] = best;
}

// Any-shape fallback (K not a multiple of the chunk width, tiny matrices):
// one wave per row, scalar loads.  Used for reference-API compatibility.
template <int FMT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.M) return;
    float acc = 0.0f;
    // rows start ldw bytes apart when ldw is set (f32 / bf16 / int8 only)
    constexpr int ESZ = FMT == WF_F32 ? 4 : FMT == WF_BF16 ? 2 : 1;
    const long rs = (FMT != WF_I4 && a.ldw > 0) ? a.ldw / ESZ : a.K;
    for (int k = lane; k < a.K; k += 64) {
        const long e = (long)row * a.K + k;
        float w;
        if constexpr (FMT == WF_F32) w = reinterpret_cast<const float*>(a.w)[(long)row * rs + k];
        else if constexpr (FMT == WF_BF16)
            w = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(a.w)[(long)row * rs + k]
                                << 16);
        else if constexpr (FMT == WF_I8)
            w = (float)reinterpret_cast<const int8_t*>(a.w)[(long)row * rs + k] * a.scales[row];
        else {
            const uint8_t b = reinterpret_cast<const uint8_t*>(a.w)[e >> 1];
            const int nib = (e & 1) ? (b & 0x0F) : (b >> 4);
            w = (float)(nib >= 8 ? nib - 16 : nib) * a.scales[e / a.block];
        }
        acc += w * a.x[k];
    }
    // every lane of the wave reaches this point (row is wave-uniform)
    acc = wave_sum(acc);
    if (lane == 0) a.y[row] = acc;
}

// Generic C[m x n] = A[m x k] B[k x n] (A f32 or bf16 bits, B/C f32
// row-major), 16x16 output tiles through LDS.  Reference-API compatibility
// for n > 8 (kernels/matmul.cu:51-87, 384-420 contracts).
template <int FMT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(const void* __restrict__ A,
                                                           const float* __restrict__ B,
                                                           float* __restrict__ C, int m, int n,
                                                           int k) {
    __shared__ float As[16][17], Bs[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
    float acc = 0.f;
    for (int k0 = 0; k0 < k; k0 += 16) {
        const int ka = k0 + tx, kb = k0 + ty;
        float av = 0.f;
        if (row < m && ka < k) {
            const long e = (long)row * k + ka;
            if constexpr (FMT == WF_F32) av = reinterpret_cast<const float*>(A)[e];
            else av = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(A)[e] << 16);
        }
        As[ty][tx] = av;
        Bs[ty][tx] = (kb < k && col < n) ? B[(long)kb * n + col] : 0.f;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 16; ++j) acc += As[ty][j] * Bs[j][tx];
        __syncthreads();
    }
    if (row < m && col < n) C[(long)row * n + col] = acc;
}

int gemm_generic_launch(int fmt, const void* A, const float* B, float* C, int m, int n, int k,
                        hipStream_t st) {
    ATLAS_REQUIRE(A && B && C && m >= 0 && n >= 0 && k >= 0, "gemm: bad arguments");
    ATLAS_REQUIRE(fmt == WF_F32 || fmt == WF_BF16, "gemm: format %d", fmt);
    if (m == 0 || n == 0) return ATLAS_OK;
    dim3 grid((n + 15) / 16, (m + 15) / 16);
    if (fmt == WF_F32) hipLaunchKernelGGL(gemm_generic_kernel<WF_F32>, grid, dim3(256), 0, st, A, B, C, m, n, k);
    else hipLaunchKernelGGL(gemm_generic_kernel<WF_BF16>, grid, dim3(256), 0, st, A, B, C, m, n, k);
    ATLAS_LAUNCH_CHECK("gemm_generic");
    return ATLAS_OK;
}

// ---------------------------------------------------------------------------

// Allow `kern` up to 160 KB of dynamic LDS (once per kernel) and return the
// blocks of it (`threads` threads, `lds` dynamic LDS bytes) one CU holds at
// once; cached per (kernel, LDS size).
static int resident_per_cu(const void* kern, size_t lds, int threads = 256) {
    struct Entry { const void* k; size_t lds; int n; };
    static std::mutex mu;
    static Entry cache[64];
    static int used = 0;
    static const void* raised[32];
    static int n_raised = 0;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
        if (cache[i].k == kern && cache[i].lds == lds) return cache[i].n;
    if (lds > 64 * 1024) {
        bool done = false;
        for (int i = 0; i < n_raised; ++i) done = done || raised[i] == kern;
        if (!done) {
            if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    160 * 1024) != hipSuccess) {
                (void)hipGetLastError();
                return 0;
            }
            if (n_raised < 32) raised[n_raised++] = kern;
        }
    }
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    if (used < 64) cache[used++] = Entry{kern, lds, n};
    return n;
}

// Persistent grid of the LDS-staged kernel (nw waves per block): every block
// resident at once (LDS and register occupancy bound the blocks per CU), at
// most blocks_per_cu of them per CU.  0 if the kernel cannot run at this K.
static int n1_blocks(const void* kern, int M, size_t lds, int rows, int blocks_per_cu, int nw = 4) {
    const int n_groups = (M + rows - 1) / rows;
    const int blocks = (n_groups + nw - 1) / nw;
    const int fit = resident_per_cu(kern, lds, 64 * nw);
    if (fit < 1) return 0;
    const int bpc = blocks_per_cu < fit ? blocks_per_cu : fit;
    const int cap = bpc * device_cu_count();
    return blocks > cap ? cap : blocks;
}

// rows one wave's group covers (the kernel's SEQ rule)
static int n1_group_rows(const GemvArgs& a, int rows) {
    return (rows == 1 && a.epi == EPI_SILU_MUL) ? 2 : rows;
}

template <int FMT, int ROWS, int UNROLL>
int launch_n1(const GemvArgs& a, hipStream_t st, int blocks_per_cu) {
    const size_t lds = gemv_x_lds_bytes(a.K);
    ATLAS_REQUIRE(lds <= 160 * 1024, "gemv: K=%d exceeds the LDS-staged limit", a.K);
    auto kern = gemv_n1_kernel<FMT, ROWS, UNROLL>;
    const int blocks = n1_blocks((const void*)kern, a.M, lds, n1_group_rows(a, ROWS), blocks_per_cu);
    ATLAS_REQUIRE(blocks > 0, "gemv: the kernel does not fit a CU at K=%d", a.K);
    if (a.epi == EPI_ARGMAX)
        ATLAS_REQUIRE(blocks * 4 <= GEMV_MAX_WAVES, "gemv: too many waves for argmax partials");
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, st, a);
    ATLAS_LAUNCH_CHECK("gemv_n1");
    return ATLAS_OK;
}

int gemv_fast_ok(int fmt, int K, int block) {
    switch (fmt) {
    case WF_F32:  return K % 4 == 0;
    case WF_BF16: return K % 8 == 0;
    case WF_I8:   return K % 16 == 0;
    case WF_I4:   return K % 32 == 0 && block > 0 && block % 32 == 0;
    }
    return 0;
}

// Launch shape per (format, K): rows per wave, chunk unroll, blocks per CU.
// Chosen by sweeping the 7B decode shapes on MI355X over >= 1.1 GB of
// rotating weights (rows = 1 wins at K = 4096: more waves in flight per CU;
// the bf16 W_down, 4096 x 11008 with padded rows, prefers two-row waves).
struct N1Shape { int rows, unroll, bpc, nw = 4; };
static N1Shape n1_shape(int fmt, int K, int epi) {
    // SwiGLU epilogue: bf16 and int4 two-row waves hold the (gate, up) pair;
    // int8 one-row waves take the pair in sequence (its two-row variant
    // needs ~170 VGPRs)
    if (epi == EPI_SILU_MUL)
        return fmt == WF_BF16 ? N1Shape{2, 4, 8} : fmt == WF_I8 ? N1Shape{1, 4, 8} : N1Shape{2, 2, 4};
    const bool big_k = K > 4096;
    switch (fmt) {
    case WF_BF16: return big_k ? N1Shape{2, 4, 3} : N1Shape{1, 4, 8};
    case WF_I8:   return big_k ? N1Shape{1, 4, 8} : N1Shape{1, 2, 8};
    case WF_I4:   return N1Shape{2, 2, 8};
    default:      return {1, 4, 8};
    }
}

// The instantiations gemv_launch dispatches to.
#define ATLAS_N1_LIST(X)                                                           \
    X(WF_BF16, 1, 4) X(WF_BF16, 2, 4)                                              \
    X(WF_I8, 1, 2) X(WF_I8, 1, 4)                                                  \
    X(WF_I4, 2, 2)                                                                 \
    X(WF_F32, 1, 4) X(WF_F32, 2, 4)

static const void* n1_kernel(int fmt, int rows, int unroll) {
#define ATLAS_N1_PTR(F, R, U) \
    if (fmt == F && rows == R && unroll == U) return (const void*)gemv_n1_kernel<F, R, U>;
    ATLAS_N1_LIST(ATLAS_N1_PTR)
#undef ATLAS_N1_PTR
    return nullptr;
}

// The decode kernel (gemv_v4_kernel) covers every fast-path shape except
// int4 blocks that straddle rows or are not 32 * 2^j elements.
static bool v4_ok(const GemvArgs& a, int unroll) {
    if (a.fmt == WF_I4 && (a.bpr <= 0 || (a.cpb & (a.cpb - 1)) != 0)) return false;
    return v4_lds_bytes(a.fmt, a.K, unroll) <= 160 * 1024;
}

// Launch shape of the decode kernel per (format, role): rows per wave,
// chunk unroll, blocks per CU.  From a sweep of rows 1/2/4, unroll 1-4 and
// 2-8 blocks per CU at the 7B shapes on MI355X over >= 1.2 GB of rotating
// weights, taken with the unconditional prefetch (the best shapes of a role
// lie within 1-4% of each other, except int4 QKV and W_o, where 4 rows per
// wave beat 2 by 7-9%).
static N1Shape v4_shape(int fmt, int M, int K, int epi) {
    const bool gu = epi == EPI_SILU_MUL, wide = K > 4096, huge = M >= 65536, tall = M >= 8192;
    switch (fmt) {
    case WF_BF16:
        if (gu) return {2, 4, 4};
        if (wide) return {1, 4, 3};
        if (huge) return {2, 4, 6};
        return tall ? N1Shape{2, 4, 3} : N1Shape{2, 4, 8};
    case WF_I8:
        if (gu) return {2, 2, 6};
        if (wide) return {1, 4, 2};
        if (huge) return {2, 4, 8};
        return tall ? N1Shape{2, 1, 4} : N1Shape{1, 2, 4};
    case WF_I4:
        if (gu) return {2, 1, 2};
        if (wide) return {2, 1, 3};
        if (huge) return {2, 1, 8};
        return {4, 1, 2};
    default:
        return {1, 4, 8};
    }
}

// (format, rows per wave, unroll, waves per block)
#ifndef ATLAS_V4_LIST
#define ATLAS_V4_LIST(X)                                                                  \
    X(WF_BF16, 1, 4, 4) X(WF_BF16, 2, 4, 4)                                               \
    X(WF_I8, 1, 2, 4) X(WF_I8, 1, 4, 4) X(WF_I8, 2, 1, 4) X(WF_I8, 2, 2, 4) X(WF_I8, 2, 4, 4) \
    X(WF_I4, 2, 1, 4) X(WF_I4, 4, 1, 4)                                                   \
    X(WF_F32, 1, 4, 4)
#endif

static const void* v4_kernel(int fmt, int rows, int unroll, int nw, bool n2) {
#define ATLAS_V4_PTR(F, R, U, W)                                                            \
    if (fmt == F && rows == R && unroll == U && nw == W)                                    \
        return n2 ? (const void*)gemv_v4_kernel<F, R, U, W, true>                           \
                  : (const void*)gemv_v4_kernel<F, R, U, W, false>;
    ATLAS_V4_LIST(ATLAS_V4_PTR)
#undef ATLAS_V4_PTR
    return nullptr;
}

bool gemv_resnorm_norm_ok(const GemvArgs& a_in) {
    GemvArgs a = a_in;
    gemv_fill_int4_index(a);
    const uintptr_t align = (uintptr_t)a.w | (uintptr_t)a.x | (uintptr_t)a.pro_y |
                            (uintptr_t)a.pro_w | (uintptr_t)a.pro_w2 | (uintptr_t)a.pro_out;
    if ((align & 15) || a.K % 4 || !gemv_fast_ok(a.fmt, a.K, a.block) ||
        gemv_x_lds_bytes(a.K) > 160 * 1024)
        return false;
    const N1Shape v4 = v4_shape(a.fmt, a.M, a.K, a.epi);
    return v4_ok(a, v4.unroll) && v4_kernel(a.fmt, v4.rows, v4.unroll, v4.nw, true) != nullptr;
}

// number of persistent waves gemv_launch uses (argmax partial count)
int gemv_waves(const GemvArgs& a_in) {
    GemvArgs a = a_in;
    gemv_fill_int4_index(a);
    const N1Shape v4 = v4_shape(a.fmt, a.M, a.K, a.epi);
    if (v4_ok(a, v4.unroll)) {
        const void* kern = v4_kernel(a.fmt, v4.rows, v4.unroll, v4.nw, a.pro == PRO_RESNORM_NORM);
        return kern ? v4.nw * n1_blocks(kern, a.M, v4_lds_bytes(a.fmt, a.K, v4.unroll),
                                        n1_group_rows(a, v4.rows), v4.bpc, v4.nw)
                    : 0;
    }
    const N1Shape sh = n1_shape(a.fmt, a.K, a.epi);
    const void* kern = n1_kernel(a.fmt, sh.rows, sh.unroll);
    return kern ? 4 * n1_blocks(kern, a.M, gemv_x_lds_bytes(a.K), n1_group_rows(a, sh.rows), sh.bpc)
                : 0;
}

template <int FMT, int ROWS, int UNROLL, int NW, bool N2>
int launch_v4(const GemvArgs& a, hipStream_t st, int blocks_per_cu) {
    const size_t lds = v4_lds_bytes(FMT, a.K, UNROLL);
    auto kern = gemv_v4_kernel<FMT, ROWS, UNROLL, NW, N2>;
    const int blocks =
        n1_blocks((const void*)kern, a.M, lds, n1_group_rows(a, ROWS), blocks_per_cu, NW);
    ATLAS_REQUIRE(blocks > 0, "gemv: the kernel does not fit a CU at K=%d", a.K);
    if (a.epi == EPI_ARGMAX)
        ATLAS_REQUIRE(blocks * NW <= GEMV_MAX_WAVES, "gemv: too many waves for argmax partials");
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * NW), lds, st, a);
    ATLAS_LAUNCH_CHECK("gemv_v4");
    return ATLAS_OK;
}

int gemv_launch(const GemvArgs& a_in, hipStream_t st) {
    GemvArgs a = a_in;
    gemv_fill_int4_index(a);
    ATLAS_REQUIRE(a.M >= 0 && a.K >= 0, "gemv: negative shape");
    if (a.M == 0) return ATLAS_OK;
    ATLAS_REQUIRE(a.w && a.y, "gemv: null pointer");
    ATLAS_REQUIRE(a.pro == PRO_SILU || a.x, "gemv: null x");
    ATLAS_REQUIRE(a.pro != PRO_RESNORM || (a.pro_y && a.pro_w), "gemv: residual norm needs y and w");
    ATLAS_REQUIRE(a.pro != PRO_RMSNORM || a.pro_w, "gemv: rmsnorm prologue needs w");
    ATLAS_REQUIRE(a.pro != PRO_RESNORM_NORM || (a.pro_y && a.pro_w && a.pro_w2),
                  "gemv: residual + final norm prologue needs y, w and w2");
    ATLAS_REQUIRE(a.pro != PRO_SILU || a.pro_y, "gemv: silu prologue needs the gate/up pairs");
    ATLAS_REQUIRE(a.pro_out == nullptr || (a.pro_out != a.x && a.pro_out != a.pro_y),
                  "gemv: the materialised x must not alias the prologue inputs");
    ATLAS_REQUIRE(a.fmt == WF_F32 || a.fmt == WF_BF16 || a.scales, "gemv: null scales");
    ATLAS_REQUIRE(a.fmt != WF_I4 || a.block > 0, "gemv: int4 block must be > 0");
    if (a.epi == EPI_SILU_MUL) ATLAS_REQUIRE(a.M % 2 == 0, "gemv: silu-mul needs even rows");
    if (a.epi == EPI_ARGMAX) ATLAS_REQUIRE(a.arg_part, "gemv: argmax epilogue needs partials");
    if (a.K == 0) {
        set_error(ATLAS_EUNSUPPORTED, "gemv: K == 0");
        return ATLAS_EUNSUPPORTED;
    }
    ATLAS_REQUIRE(gemv_pitch_ok(a), "gemv: row pitch %ld bytes for K %d", a.ldw, a.K);
    const uintptr_t align = (uintptr_t)a.w | (uintptr_t)a.x | (uintptr_t)a.pro_y |
                            (uintptr_t)a.pro_w | (uintptr_t)a.pro_w2 | (uintptr_t)a.pro_out;
    const bool fast = (align & 15) == 0 && a.K % 4 == 0 && gemv_fast_ok(a.fmt, a.K, a.block) &&
                      gemv_x_lds_bytes(a.K) <= 160 * 1024;
    if (fast) {
        const N1Shape v4 = v4_shape(a.fmt, a.M, a.K, a.epi);
        if (v4_ok(a, v4.unroll)) {
#define ATLAS_V4(F, R, U, W)                                                          \
            if (a.fmt == F && v4.rows == R && v4.unroll == U && v4.nw == W)                 \
                return a.pro == PRO_RESNORM_NORM ? launch_v4<F, R, U, W, true>(a, st, v4.bpc) \
                                                 : launch_v4<F, R, U, W, false>(a, st, v4.bpc);
            ATLAS_V4_LIST(ATLAS_V4)
#undef ATLAS_V4
        }
        ATLAS_REQUIRE(a.pro != PRO_RESNORM_NORM,
                      "gemv: the residual + final norm prologue needs the decode kernel's shapes");
        const N1Shape sh = n1_shape(a.fmt, a.K, a.epi);
#define ATLAS_N1(F, R, U) \
        if (a.fmt == F && sh.rows == R && sh.unroll == U) return launch_n1<F, R, U>(a, st, sh.bpc);
        ATLAS_N1_LIST(ATLAS_N1)
#undef ATLAS_N1
        set_error(ATLAS_EUNSUPPORTED, "gemv: no kernel for format %d", a.fmt);
        return ATLAS_EUNSUPPORTED;
    }
    ATLAS_REQUIRE(a.epi == EPI_STORE && a.pro == PRO_X,
                  "gemv: fused prologue/epilogue needs an aligned fast-path shape");
    ATLAS_REQUIRE(a.fmt != WF_I4 || a.ldw == 0, "gemv: int4 row pitch needs the fast path");
    const int blocks = (a.M + 3) / 4;
    switch (a.fmt) {
    case WF_F32:  hipLaunchKernelGGL(gemv_generic_kernel<WF_F32>, dim3(blocks), dim3(256), 0, st, a); break;
    case WF_BF16: hipLaunchKernelGGL(gemv_generic_kernel<WF_BF16>, dim3(blocks), dim3(256), 0, st, a); break;
    case WF_I8:   hipLaunchKernelGGL(gemv_generic_kernel<WF_I8>, dim3(blocks), dim3(256), 0, st, a); break;
    case WF_I4:   hipLaunchKernelGGL(gemv_generic_kernel<WF_I4>, dim3(blocks), dim3(256), 0, st, a); break;
    default: set_error(ATLAS_EINVAL, "gemv: unknown weight format %d", a.fmt); return ATLAS_EINVAL;
    }
    ATLAS_LAUNCH_CHECK("gemv_generic");
    return ATLAS_OK;
}

// ---- small ragged batch: N = 2..4 activation rows per weight load ----------
template <int FMT, int ROWS, int UNROLL, int NX>
static int launch_nx(const GemvArgs& a, hipStream_t st, int blocks_per_cu) {
    const size_t lds = (size_t)NX * gemv_x_lds_bytes(a.K);
    ATLAS_REQUIRE(lds <= 160 * 1024, "gemv: %d rows of K=%d exceed LDS", NX, a.K);
    auto kern = gemv_n1_kernel<FMT, ROWS, UNROLL, NX>;
    const int blocks = n1_blocks((const void*)kern, a.M, lds, n1_group_rows(a, ROWS), blocks_per_cu);
    ATLAS_REQUIRE(blocks > 0, "gemv: the kernel does not fit a CU at K=%d", a.K);
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, st, a);
    ATLAS_LAUNCH_CHECK("gemv_nx");
    return ATLAS_OK;
}

bool gemv_multi_ok(const GemvArgs& a) {
    const uintptr_t al = (uintptr_t)a.w | (uintptr_t)a.x;
    return a.N >= 2 && a.N <= kGemvMaxNx && a.M > 0 && a.K > 0 && (al & 15) == 0 &&
           a.pro == PRO_X && (a.epi == EPI_STORE || a.epi == EPI_SILU_MUL) &&
           a.x_stride_k == 1 && a.x_stride_n % 4 == 0 && a.K % 4 == 0 &&
           a.K <= 256 * 4 * 12 &&    // stage_xn: twelve 16-byte pieces per thread
           gemv_fast_ok(a.fmt, a.K, a.block) && gemv_pitch_ok(a) &&
           (size_t)a.N * gemv_x_lds_bytes(a.K) <= 160 * 1024 &&
           (a.epi != EPI_SILU_MUL || a.M % 2 == 0);
}

int gemv_multi_launch(const GemvArgs& a_in, hipStream_t st) {
    GemvArgs a = a_in;
    gemv_fill_int4_index(a);
    ATLAS_REQUIRE(a.w && a.x && a.y, "gemv: null pointer");
    ATLAS_REQUIRE(a.fmt == WF_F32 || a.fmt == WF_BF16 || a.scales, "gemv: null scales");
    ATLAS_REQUIRE(gemv_multi_ok(a), "gemv: %d rows need the aligned fast path", a.N);
    const N1Shape sh = n1_shape(a.fmt, a.K, a.epi);
#define ATLAS_NX(F, R, U)                                                            \
    if (a.fmt == F && sh.rows == R && sh.unroll == U) {                              \
        switch (a.N) {                                                               \
        case 2: return launch_nx<F, R, U, 2>(a, st, sh.bpc);                         \
        case 3: return launch_nx<F, R, U, 3>(a, st, sh.bpc);                         \
        case 4: return launch_nx<F, R, U, 4>(a, st, sh.bpc);                         \
        }                                                                            \
    }
    ATLAS_N1_LIST(ATLAS_NX)
#undef ATLAS_NX
    set_error(ATLAS_EUNSUPPORTED, "gemv: no %d-row kernel for format %d", a.N, a.fmt);
    return ATLAS_EUNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Measurement only: the streaming floor of a decode-GEMV-shaped launch.  The
// kernel reads `bytes` from `src` with the bf16 decode GEMV's work split and
// load pattern (8 KB rows in groups of two, groups round-robin over the
// waves, 1 KB per load instruction, 4 KB per row per step, two register
// buffers) and does no arithmetic on them beyond a checksum, so a graph of
// such launches measures what a launch of that many bytes costs before any
// GEMV work (launch gap, ramp, tail and streaming rate).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void stream_floor_kernel(const char* __restrict__ src, long bytes,
                                                           float* __restrict__ sink) {
    constexpr int U = 4, ROWS = 2;
    constexpr long ROW = 8192;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const long n_groups = bytes / (ROW * ROWS);
    const int S = gridDim.x * 4;
    const int g0 = blockIdx.x * 4 + wave;
    const int steps = g0 < n_groups ? (int)((n_groups - 1 - g0) / S + 1) * 2 : 0;   // 2 steps per group
    auto load = [&](int t, u32x4 (&r)[U][ROWS]) {
        const long g = g0 + (long)(t >> 1) * S;
        const bool ok = t < steps;
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const char* rp = src + (ok ? (g * ROWS + i) * ROW + (t & 1) * (ROW / 2) : 0);
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                uniform_ptr(rp), (short)0, __builtin_amdgcn_readfirstlane(ok ? (int)(ROW / 2) : 0),
                0x00020000);
#pragma unroll
            for (int u = 0; u < U; ++u)
                r[u][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16 + u * 1024, 0, 2));
        }
    };
    float acc = 0.f;
    auto use = [&](const u32x4 (&r)[U][ROWS]) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < ROWS; ++i) acc += __uint_as_float(r[u][i].x & 0x3f800000u);
    };
    u32x4 A[U][ROWS], B[U][ROWS];
    load(0, A);
    for (int t = 0; t < steps; t += 2) {
        load(t + 1, B);
        use(A);
        if (t + 1 >= steps) break;
        load(t + 2, A);
        use(B);
    }
    if (lane == 0) sink[blockIdx.x * 4 + wave] = acc;
}

__global__ __launch_bounds__(256) void empty_launch_kernel(float* __restrict__ sink, int never) {
    if (never == 1) sink[blockIdx.x] = 0.f;   // the host passes 0: no work, no memory access
}

// Best replay time (ms) of a graph of `n` floor launches (empty kernels when
// bytes_per_launch is 0) on stream st.
static int floor_graph_ms(const void* buf, long buf_bytes, long bytes_per_launch, int n, int blocks,
                          float* sink, hipStream_t st, float* best_ms) {
    const long per = bytes_per_launch > 0 ? buf_bytes / bytes_per_launch : 1;
    hipGraph_t g = nullptr;
    hipGraphExec_t gx = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = ATLAS_OK;
    if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) rc = ATLAS_EHIP;
    for (int k = 0; rc == ATLAS_OK && k < n; ++k) {
        if (bytes_per_launch > 0)
            hipLaunchKernelGGL(stream_floor_kernel, dim3(blocks), dim3(256), 0, st,
                               static_cast<const char*>(buf) + (k % per) * bytes_per_launch,
                               bytes_per_launch, sink);
        else
            hipLaunchKernelGGL(empty_launch_kernel, dim3(blocks), dim3(256), 0, st, sink, 0);
    }
    if (rc == ATLAS_OK && hipStreamEndCapture(st, &g) != hipSuccess) rc = ATLAS_EHIP;
    if (rc == ATLAS_OK && hipGraphInstantiate(&gx, g, nullptr, nullptr, 0) != hipSuccess) rc = ATLAS_EHIP;
    if (rc == ATLAS_OK && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
        rc = ATLAS_EHIP;
    float best = 0.f;
    for (int rep = 0; rc == ATLAS_OK && rep < 4; ++rep) {
        float ms = 0.f;
        if (hipEventRecord(e0, st) != hipSuccess || hipGraphLaunch(gx, st) != hipSuccess ||
            hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
            hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
            rc = ATLAS_EHIP;
            break;
        }
        if (rep == 1 || (rep > 1 && ms < best)) best = ms;   // replay 0 warms up
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (gx) (void)hipGraphExecDestroy(gx);
    if (g) (void)hipGraphDestroy(g);
    *best_ms = best;
    return rc;
}

int stream_floor_bench(const void* buf, long buf_bytes, long bytes_per_launch, int launches,
                       int blocks_per_cu, float* us_per_launch, hipStream_t st) {
    ATLAS_REQUIRE(us_per_launch && launches > 0 && blocks_per_cu > 0, "stream_floor: bad arguments");
    ATLAS_REQUIRE(bytes_per_launch == 0 || (buf && bytes_per_launch >= 16384 &&
                                            bytes_per_launch % 16384 == 0 &&
                                            bytes_per_launch <= buf_bytes),
                  "stream_floor: %ld bytes per launch", bytes_per_launch);
    ATLAS_REQUIRE(((uintptr_t)buf & 15) == 0, "stream_floor: 16-byte alignment");
    const int blocks = blocks_per_cu * device_cu_count();
    // captured and replayed on a stream of its own (the caller's may be the
    // legacy default stream, which cannot be captured), after the caller's work
    ATLAS_HIP(hipStreamSynchronize(st));
    ATLAS_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    float* sink = nullptr;
    if (dev_malloc(&sink, (size_t)blocks * 4 * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipStreamDestroy(st);
        set_error(ATLAS_ENOMEM, "stream_floor: sink allocation");
        return ATLAS_ENOMEM;
    }
    // graphs of n and 2n launches: the difference is n launches without the
    // graph launch's own fixed cost (~10 us, which a short graph would spread
    // over few launches)
    float t1 = 0.f, t2 = 0.f;
    int rc = floor_graph_ms(buf, buf_bytes, bytes_per_launch, launches, blocks, sink, st, &t1);
    if (rc == ATLAS_OK)
        rc = floor_graph_ms(buf, buf_bytes, bytes_per_launch, 2 * launches, blocks, sink, st, &t2);
    if (rc != ATLAS_OK) {
        (void)hipGetLastError();
        set_error(ATLAS_EHIP, "stream_floor: graph capture or replay failed");
    }
    (void)hipStreamSynchronize(st);
    (void)hipFree(sink);
    (void)hipStreamDestroy(st);
    *us_per_launch = (t2 - t1) * 1e3f / launches;
    return rc;
}

}  // namespace atlas
