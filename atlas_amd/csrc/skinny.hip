// skinny.hip -- small ragged batch GEMM Y[n, m] = sum_k W[m, k] X[n, k], 1 <= N <= 8.
//
// The reference has no batched decode (each sequence runs its own GEMV,
// crates/atlas-model/src/lib.rs:487-499).  With N decode rows packed
// together the weights are still read once, and the N products per weight
// go to the matrix cores: v_mfma_f32_16x16x32_bf16.
//
// Layout (per wave, per MFMA):
//  * A operand = activations: lane (i = lane % 16, g = lane / 16) supplies 8
//    values of activation column i for its k-set; column i = 2*s + part holds
//    sequence s split into a bf16 "hi" (truncation) and "lo" (RNE of the
//    exact remainder) part, so hi + lo carries 16 significant bits and the
//    f32-accumulated product matches an f32 GEMV to ~2^-16;
//  * B operand = weights: lane (r = lane % 16, g) supplies 8 values of weight
//    row r (bf16 as stored; int8/int4 sign-extended to f32 by SDWA converts
//    and truncated to bf16, which is exact for |16*q| <= 128);
//  * D: lane (r, g) holds D[4g + v][r] -> rows of the output for sequences
//    2g and 2g + 1, so every lane owns one weight row and a per-row or
//    per-(row, block) scale is a single value per lane.
//  * int4: one MFMA covers exactly one 32-element chunk of one row (lane
//    group g takes the chunk's 4-byte word g), so the block scale applies to
//    the MFMA result.
//  * split-K across blocks writes fp32 partials; a second kernel sums them in
//    a fixed order (deterministic) and applies the epilogue.
#include "common.hpp"
#include "gemv.hpp"

namespace atlas {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// bf16 bits (low 16) of the hi (part 0) or lo (part 1) component of v
__device__ __forceinline__ uint32_t split_part(float v, int part) {
    const uint32_t u = __float_as_uint(v);
    if (part == 0) return u >> 16;
    const float hi = __uint_as_float(u & 0xFFFF0000u);
    return bf16_rne_bits(v - hi);
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo16, uint32_t hi16) {
    return (lo16 & 0xFFFFu) | (hi16 << 16);
}

// exact f32 -> bf16 bits for values with <= 8 significant bits
__device__ __forceinline__ uint32_t pack_f32_pair(float a, float b) {
    return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xFFFF0000u);
}

template <int FMT> struct SK;
template <> struct SK<WF_BF16> { static constexpr int SEG = 32;  static constexpr int MF = 1; };
template <> struct SK<WF_I8>   { static constexpr int SEG = 64;  static constexpr int MF = 2; };
template <> struct SK<WF_I4>   { static constexpr int SEG = 128; static constexpr int MF = 4; };

// k offset (within a segment) of lane group g's 8 values for MFMA m
template <int FMT>
__device__ __forceinline__ int kset(int g, int m) {
    if constexpr (FMT == WF_BF16) return 8 * g;
    else if constexpr (FMT == WF_I8) return 16 * g + 8 * m;
    else return 32 * m + 8 * g;
}

template <int FMT, int TILES>
__global__ __launch_bounds__(256) void skinny_kernel(GemvArgs a, float* __restrict__ partial,
                                                     int splitk) {
    constexpr int SEG = SK<FMT>::SEG, MF = SK<FMT>::MF;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, g = lane >> 4;
    const int row0 = (blockIdx.x * 4 + wave) * (TILES * 16);
    if (row0 >= a.M) return;                       // wave-uniform
    const int M = a.M, K = a.K, N = a.N;
    const int nseg = K / SEG;
    const int ks = blockIdx.y;
    const int s0 = (int)((long)nseg * ks / splitk), s1 = (int)((long)nseg * (ks + 1) / splitk);

    // activation column handled by this lane in the A operand
    const int xs = lr >> 1, xpart = lr & 1;
    const bool xvalid = xs < N;
    const float* xrow = a.x + (xvalid ? (long)xs * a.x_stride_n : 0);

    int rows[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        const int r = row0 + t * 16 + lr;
        rows[t] = r < M ? r : M - 1;
    }

    f32x4 acc[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int seg = s0; seg < s1; ++seg) {
        const int kb = seg * SEG;
        // ---- weight fragments for every tile (issued first) --------------
        u32x4 wraw[TILES];
        uint32_t w4[TILES][MF];
        if constexpr (FMT == WF_BF16 || FMT == WF_I8) {
            const int eb = FMT == WF_BF16 ? 2 : 1;
#pragma unroll
            for (int t = 0; t < TILES; ++t) {
                const char* base = reinterpret_cast<const char*>(a.w) +
                                   ((long)rows[t] * K + kb + (FMT == WF_BF16 ? 8 : 16) * g) * eb;
                wraw[t] = ldg_stream(reinterpret_cast<const u32x4*>(base));
            }
        } else {
#pragma unroll
            for (int t = 0; t < TILES; ++t)
#pragma unroll
                for (int m = 0; m < MF; ++m) {
                    const uint32_t* base = reinterpret_cast<const uint32_t*>(
                        reinterpret_cast<const uint8_t*>(a.w) + ((long)rows[t] * K + kb + 32 * m) / 2);
                    w4[t][m] = __builtin_nontemporal_load(base + g);
                }
        }
        // ---- per MFMA ------------------------------------------------------
#pragma unroll
        for (int m = 0; m < MF; ++m) {
            const int k0 = kb + kset<FMT>(g, m);
            u32x4 xa = u32x4{0u, 0u, 0u, 0u};
            if (xvalid) {
                float v[8];
                if (a.x_vec) {
                    const f32x4 p0 = *reinterpret_cast<const f32x4*>(xrow + k0);
                    const f32x4 p1 = *reinterpret_cast<const f32x4*>(xrow + k0 + 4);
                    v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
                    v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = xrow[(long)(k0 + j) * a.x_stride_k];
                }
                xa.x = pack2(split_part(v[0], xpart), split_part(v[1], xpart));
                xa.y = pack2(split_part(v[2], xpart), split_part(v[3], xpart));
                xa.z = pack2(split_part(v[4], xpart), split_part(v[5], xpart));
                xa.w = pack2(split_part(v[6], xpart), split_part(v[7], xpart));
            }
            const bf16x8 A = __builtin_bit_cast(bf16x8, xa);
#pragma unroll
            for (int t = 0; t < TILES; ++t) {
                u32x4 wb;
                if constexpr (FMT == WF_BF16) {
                    wb = wraw[t];
                } else if constexpr (FMT == WF_I8) {
                    const uint32_t w0 = m == 0 ? wraw[t].x : wraw[t].z;
                    const uint32_t w1 = m == 0 ? wraw[t].y : wraw[t].w;
                    wb.x = pack_f32_pair(s8_at(w0, 0), s8_at(w0, 1));
                    wb.y = pack_f32_pair(s8_at(w0, 2), s8_at(w0, 3));
                    wb.z = pack_f32_pair(s8_at(w1, 0), s8_at(w1, 1));
                    wb.w = pack_f32_pair(s8_at(w1, 2), s8_at(w1, 3));
                } else {
                    const uint32_t hi = w4[t][m] & 0xF0F0F0F0u;          // 16 * even
                    const uint32_t lo = (w4[t][m] << 4) & 0xF0F0F0F0u;   // 16 * odd
                    wb.x = pack_f32_pair(s8_at(hi, 0), s8_at(lo, 0));
                    wb.y = pack_f32_pair(s8_at(hi, 1), s8_at(lo, 1));
                    wb.z = pack_f32_pair(s8_at(hi, 2), s8_at(lo, 2));
                    wb.w = pack_f32_pair(s8_at(hi, 3), s8_at(lo, 3));
                }
                const bf16x8 B = __builtin_bit_cast(bf16x8, wb);
                if constexpr (FMT == WF_I4) {
                    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        A, B, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    const int c = (kb >> 5) + m;              // chunk index in the row
                    long bi;
                    if (a.bpr > 0) bi = (long)rows[t] * a.bpr + (a.cpb == 1 ? c : c / a.cpb);
                    else bi = ((long)rows[t] * K + (long)c * 32) / a.block;
                    const float s = a.scales[bi] * 0.0625f;
                    acc[t] += d * s;
                } else {
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, acc[t], 0, 0, 0);
                }
            }
        }
    }

    // ---- epilogue: lane (r, g) owns row r, sequences 2g and 2g+1 -----------
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        const int r = row0 + t * 16 + lr;
        if (r >= M) continue;
        float y0 = acc[t].x + acc[t].y, y1 = acc[t].z + acc[t].w;
        if constexpr (FMT == WF_I8) {
            const float s = a.scales[r];
            y0 *= s;
            y1 *= s;
        }
        const int n0 = 2 * g, n1 = 2 * g + 1;
        if (n0 < N) partial[((long)ks * N + n0) * M + r] = y0;
        if (n1 < N) partial[((long)ks * N + n1) * M + r] = y1;
    }
}

__global__ __launch_bounds__(256) void skinny_reduce_kernel(GemvArgs a, const float* __restrict__ partial,
                                                            int splitk) {
    const int M = a.M, N = a.N;
    const int m_out = a.epi == EPI_SILU_MUL ? M / 2 : M;
    const long total = (long)N * m_out;
    for (long i = blockIdx.x * 256L + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
        const int n = (int)(i / m_out), mo = (int)(i % m_out);
        if (a.epi == EPI_SILU_MUL) {
            float gsum = 0.f, usum = 0.f;
            for (int s = 0; s < splitk; ++s) {
                gsum += partial[((long)s * N + n) * M + 2 * mo];
                usum += partial[((long)s * N + n) * M + 2 * mo + 1];
            }
            a.y[n * a.y_stride_n + (long)mo * a.y_stride_m] = gsum / (1.0f + expf(-gsum)) * usum;
        } else {
            float sum = 0.f;
            for (int s = 0; s < splitk; ++s) sum += partial[((long)s * N + n) * M + mo];
            a.y[n * a.y_stride_n + (long)mo * a.y_stride_m] = sum;
        }
    }
}

// scratch for split-K partials (grown on demand, never shrunk)
static float* g_partial = nullptr;
static size_t g_partial_bytes = 0;

static int ensure_partial(size_t bytes) {
    if (bytes <= g_partial_bytes) return ATLAS_OK;
    if (g_partial) {
        ATLAS_HIP(hipDeviceSynchronize());
        ATLAS_HIP(hipFree(g_partial));
        g_partial = nullptr;
        g_partial_bytes = 0;
    }
    ATLAS_HIP(hipMalloc((void**)&g_partial, bytes));
    g_partial_bytes = bytes;
    return ATLAS_OK;
}

int skinny_reserve(int M, int N, int K) {
    return ensure_partial((size_t)64 * N * M * sizeof(float));
}

template <int FMT, int TILES>
static int launch_skinny(const GemvArgs& a, hipStream_t st) {
    constexpr int SEG = SK<FMT>::SEG;
    const int rows_per_block = 4 * TILES * 16;
    const int bx = (a.M + rows_per_block - 1) / rows_per_block;
    const int nseg = a.K / SEG;
    const int waves = bx * 4;
    int splitk = (4 * device_cu_count() * 4 + waves - 1) / waves;   // >= 4 waves per SIMD
    if (splitk > nseg) splitk = nseg;
    if (splitk > 64) splitk = 64;
    if (splitk < 1) splitk = 1;
    int rc = ensure_partial((size_t)splitk * a.N * a.M * sizeof(float));
    if (rc) return rc;
    hipLaunchKernelGGL((skinny_kernel<FMT, TILES>), dim3(bx, splitk), dim3(256), 0, st, a,
                       g_partial, splitk);
    ATLAS_LAUNCH_CHECK("skinny");
    const long m_out = a.epi == EPI_SILU_MUL ? a.M / 2 : a.M;
    long rb = ((long)a.N * m_out + 255) / 256;
    if (rb > 4096) rb = 4096;
    hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, a, g_partial,
                       splitk);
    ATLAS_LAUNCH_CHECK("skinny_reduce");
    return ATLAS_OK;
}

int skinny_launch(const GemvArgs& a_in, hipStream_t st) {
    GemvArgs a = a_in;
    gemv_fill_int4_index(a);
    a.x_vec = a.x_stride_k == 1 && a.x_stride_n % 4 == 0 && ((uintptr_t)a.x & 15) == 0;
    ATLAS_REQUIRE(a.N >= 1 && a.N <= 8, "skinny: N=%d outside 1..8", a.N);
    ATLAS_REQUIRE(a.w && a.x && a.y, "skinny: null pointer");
    ATLAS_REQUIRE(a.fmt == WF_BF16 || a.scales, "skinny: null scales");
    if (a.epi == EPI_SILU_MUL) ATLAS_REQUIRE(a.M % 2 == 0, "skinny: silu-mul needs even rows");
    if (a.M == 0) return ATLAS_OK;
    switch (a.fmt) {
    case WF_BF16:
        ATLAS_REQUIRE(a.K % 32 == 0, "skinny bf16: K %% 32 != 0");
        return launch_skinny<WF_BF16, 2>(a, st);
    case WF_I8:
        ATLAS_REQUIRE(a.K % 64 == 0, "skinny int8: K %% 64 != 0");
        return launch_skinny<WF_I8, 2>(a, st);
    case WF_I4:
        ATLAS_REQUIRE(a.K % 128 == 0 && a.block % 32 == 0, "skinny int4: K %% 128 or block %% 32");
        return launch_skinny<WF_I4, 2>(a, st);
    }
    set_error(ATLAS_EUNSUPPORTED, "skinny: weight format %d", a.fmt);
    return ATLAS_EUNSUPPORTED;
}

}  // namespace atlas
