// fused.hip -- the small per-token kernels of the decode step.
//
//  * residual_rmsnorm: x += rmsnorm(y) * w   (post-norm block,
//    crates/atlas-model/src/lib.rs:983-993) -- one launch instead of the
//    reference's rmsnorm + vec_add pair (kernels/matmul.cu:241-283, 91-94);
//  * rmsnorm: out = x * (1/sqrt(mean(x^2)+eps)) * w  (lib.rs:335-342);
//  * qkv_post: per-head QK-norm (eps 1e-6, lib.rs:660-672) + rotate-half RoPE
//    from the precomputed tables (lib.rs:428-437) + K/V cache write at pos
//    (lib.rs:577-585) in one launch, for a batch of sequences;
//  * argmax with the reference's tie rule (last maximal index,
//    lib.rs:2701-2706), optionally after step-0 suppression and the
//    repetition penalty (lib.rs:1629-1646, 2581-2592);
//  * embedding gather with the token id clamp (lib.rs:539-542);
//  * seeded initialisers and device-side atlas-quant quantisers.
// Position and token ids may be read from device memory so that one
// captured decode step can be replayed for every token.
#include "common.hpp"
#include "fused.hpp"

namespace atlas {

// block-wide sum for blockDim.x <= 1024 (all threads must call)
__device__ float block_sum(float v) {
    __shared__ float red[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nw = (blockDim.x + 63) >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// ---- rmsnorm / residual ----------------------------------------------------

// out = rmsnorm(x) * w ; row b of a batch at x + b*ld, out + b*ld
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       float* __restrict__ out, int n, long ld,
                                                       float eps) {
    const float* xb = x + blockIdx.x * ld;
    float* ob = out + blockIdx.x * ld;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += xb[i] * xb[i];
    ss = block_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) ob[i] = xb[i] * inv * w[i];
}

// x += (y * inv) * w with inv = 1/sqrt(mean(y^2)+eps); batch row b at +b*ld
__global__ __launch_bounds__(1024) void residual_rmsnorm_kernel(float* __restrict__ x,
                                                                const float* __restrict__ y,
                                                                const float* __restrict__ w, int n,
                                                                long ld, float eps) {
    float* xb = x + blockIdx.x * ld;
    const float* yb = y + blockIdx.x * ld;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += yb[i] * yb[i];
    ss = block_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) xb[i] += yb[i] * inv * w[i];
}

// The prompt chunk's form of residual_rmsnorm_kernel: y = d_hi + d_lo (the
// two product rows of the library GEMM, n wide, row b at d + b*n and
// d + lo_off + b*n), the same sums and order as residual_rmsnorm_kernel reading
// that y; the updated x row is also written as the bf16 hi / lo split rows of
// the next GEMM's input (xs rows b and rows + b, n wide) when xs is non-null.
__global__ __launch_bounds__(1024) void residual_rmsnorm_rows_kernel(
    float* __restrict__ x, const float* __restrict__ d, long lo_off, const float* __restrict__ w, int n,
    long ld, float eps, uint16_t* __restrict__ xs) {
    const int b = blockIdx.x;
    float* xb = x + b * ld;
    const float* dh = d + (long)b * n;
    const float* dl = dh + lo_off;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float y = dh[i] + dl[i];
        ss += y * y;
    }
    ss = block_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    uint16_t* sh = xs ? xs + (long)b * n : nullptr;
    uint16_t* sl = xs ? xs + (long)(gridDim.x + b) * n : nullptr;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float y = dh[i] + dl[i];
        const float v = xb[i] + y * inv * w[i];
        xb[i] = v;
        if (xs) {
            const uint32_t u = __float_as_uint(v);
            const float r = v - __uint_as_float(u & 0xFFFF0000u);
            const uint32_t ur = __float_as_uint(r);
            sh[i] = (uint16_t)(u >> 16);
            sl[i] = (uint16_t)((ur + 0x7FFFu + ((ur >> 16) & 1u)) >> 16);
        }
    }
}

int residual_rmsnorm_rows_launch(float* x, const float* d, long lo_off, const float* w, int n, int rows,
                                 long ld, float eps, uint16_t* xs, hipStream_t st) {
    ATLAS_REQUIRE(x && d && w && n > 0 && rows > 0 && lo_off >= (long)rows * n,
                  "residual_rmsnorm_rows: bad arguments");
    const int threads = n >= 1024 ? 1024 : ((n + 63) / 64) * 64;
    hipLaunchKernelGGL(residual_rmsnorm_rows_kernel, dim3(rows), dim3(threads), 0, st, x, d, lo_off, w,
                       n, ld, eps, xs);
    ATLAS_LAUNCH_CHECK("residual_rmsnorm_rows");
    return ATLAS_OK;
}

// The int8 prompt chunk's form: y[i] = (D0 + (D1 + D2 / 128) / 128) * s_b * ws[i]
// from the library GEMM's three int32 product planes (row b at d + b*n, the
// planes `plane` apart; s_b = xscale[b], the input digits' row scale), formed
// as combine_digits_kernel forms it; then x += rmsnorm(y) * w as above, and,
// when xd is non-null, the new x row as three int8 digit rows (xd rows b,
// rows + b, 2 rows + b) with its scale replacing xscale[b], as
// digits_rows_kernel writes them.
template <int EPT>
__global__ __launch_bounds__(1024) void residual_rmsnorm_digits_kernel(
    float* __restrict__ x, const int* __restrict__ d, long plane, const float* __restrict__ ws,
    float* __restrict__ xscale, const float* __restrict__ w, int n, long ld, float eps,
    int8_t* __restrict__ xd) {
    __shared__ float redm[16];
    const int b = blockIdx.x, rows = gridDim.x;
    float* xb = x + b * ld;
    const int* d0 = d + (long)b * n;
    const float sb = xscale[b];          // read before any thread replaces it
    // every load of the thread's EPT elements before the first use
    int p0[EPT], p1[EPT], p2[EPT];
    float xv[EPT], wv[EPT], sv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = threadIdx.x + 1024 * j;
        const bool ok = i < n;
        p0[j] = ok ? d0[i] : 0;
        p1[j] = ok ? d0[i + plane] : 0;
        p2[j] = ok ? d0[i + 2 * plane] : 0;
        sv[j] = ok ? ws[i] : 0.f;
        xv[j] = ok ? xb[i] : 0.f;
        wv[j] = ok ? w[i] : 0.f;
    }
    float y[EPT];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const float lo = (float)p1[j] + (float)p2[j] * (1.0f / 128.f);
        y[j] = ((float)p0[j] + lo * (1.0f / 128.f)) * sb * sv[j];
        if (threadIdx.x + 1024 * j < n) ss += y[j] * y[j];
    }
    ss = block_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = threadIdx.x + 1024 * j;
        xv[j] = xv[j] + y[j] * inv * wv[j];
        if (i < n) {
            xb[i] = xv[j];
            mx = fmaxf(mx, fabsf(xv[j]));
        }
    }
    if (!xd) return;
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) redm[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = redm[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, redm[i]);
    const float dinv = mx > 0.f ? 127.0f / mx : 0.f;
    if (threadIdx.x == 0) xscale[b] = mx / 127.0f;
    auto digit = [](float f) { return (int8_t)(int)fminf(fmaxf(rintf(f), -127.f), 127.f); };
    int8_t* o0 = xd + (long)b * n;
    int8_t* o1 = xd + (long)(rows + b) * n;
    int8_t* o2 = xd + (long)(2 * rows + b) * n;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = threadIdx.x + 1024 * j;
        if (i >= n) break;
        const float u = xv[j] * dinv;
        const int8_t q0 = digit(u);
        const float r1 = (u - (float)q0) * 128.f;
        const int8_t q1 = digit(r1);
        const float r2 = (r1 - (float)q1) * 128.f;
        o0[i] = q0;
        o1[i] = q1;
        o2[i] = digit(r2);
    }
}

int residual_rmsnorm_digits_launch(float* x, const int* d, const float* ws, float* xscale,
                                   const float* w, int n, int rows, long ld, float eps, int8_t* xd,
                                   hipStream_t st) {
    ATLAS_REQUIRE(x && d && ws && xscale && w && n > 0 && n <= 8192 && rows > 0,
                  "residual_rmsnorm_digits: bad arguments (n %d)", n);
    if (n <= 4096)
        hipLaunchKernelGGL(residual_rmsnorm_digits_kernel<4>, dim3(rows), dim3(1024), 0, st, x, d,
                           (long)rows * n, ws, xscale, w, n, ld, eps, xd);
    else
        hipLaunchKernelGGL(residual_rmsnorm_digits_kernel<8>, dim3(rows), dim3(1024), 0, st, x, d,
                           (long)rows * n, ws, xscale, w, n, ld, eps, xd);
    ATLAS_LAUNCH_CHECK("residual_rmsnorm_digits");
    return ATLAS_OK;
}

// residual_rmsnorm_kernel reading y as the split-K partials of the GEMM
// that produced it: y[b][i] = sum over s of part[(s * rows + b) * n + i], in
// split order from 0.f as skinny_reduce_kernel sums them (so y, and all that
// follows, is bit-identical to the reduce-then-norm pair).  One block per row
// (the norm needs the whole row): a thread holds its EPT elements' y, x and w
// in registers, every load issued before the first sum (S splits unrolled),
// so the block waits for one round trip of loads instead of one per split.
template <int S, int EPT>
__global__ __launch_bounds__(1024) void residual_rmsnorm_parts_kernel(float* __restrict__ x,
                                                                      const float* __restrict__ part,
                                                                      const float* __restrict__ w, int n,
                                                                      long ld, float eps) {
    const int b = blockIdx.x, rows = gridDim.x;
    float* xb = x + b * ld;
    const float* pb = part + (long)b * n;
    const long plane = (long)rows * n;
    float pv[EPT][S], xv[EPT], wv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = threadIdx.x + 1024 * j;
        const bool ok = i < n;
#pragma unroll
        for (int sp = 0; sp < S; ++sp) pv[j][sp] = ok ? pb[sp * plane + i] : 0.f;
        xv[j] = ok ? xb[i] : 0.f;
        wv[j] = ok ? w[i] : 0.f;
    }
    float y[EPT];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        float sum = 0.f;
#pragma unroll
        for (int sp = 0; sp < S; ++sp) sum += pv[j][sp];
        y[j] = sum;
        if (threadIdx.x + 1024 * j < n) ss += sum * sum;
    }
    ss = block_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = threadIdx.x + 1024 * j;
        if (i < n) xb[i] = xv[j] + y[j] * inv * wv[j];
    }
}

template <int S>
static int parts_go(float* x, const float* part, const float* w, int n, int rows, long ld, float eps,
                    hipStream_t st) {
    if (n <= 4096)
        hipLaunchKernelGGL((residual_rmsnorm_parts_kernel<S, 4>), dim3(rows), dim3(1024), 0, st, x, part,
                           w, n, ld, eps);
    else
        hipLaunchKernelGGL((residual_rmsnorm_parts_kernel<S, 8>), dim3(rows), dim3(1024), 0, st, x, part,
                           w, n, ld, eps);
    ATLAS_LAUNCH_CHECK("residual_rmsnorm_parts");
    return ATLAS_OK;
}

int residual_rmsnorm_parts_launch(float* x, const float* part, int splits, const float* w, int n,
                                  int rows, long ld, float eps, hipStream_t st) {
    ATLAS_REQUIRE(x && part && w && splits >= 1 && splits <= 8 && n > 0 && n <= 8192 && rows > 0,
                  "residual_rmsnorm_parts: %d splits, n %d", splits, n);
    switch (splits) {
    case 1: return parts_go<1>(x, part, w, n, rows, ld, eps, st);
    case 2: return parts_go<2>(x, part, w, n, rows, ld, eps, st);
    case 3: return parts_go<3>(x, part, w, n, rows, ld, eps, st);
    case 4: return parts_go<4>(x, part, w, n, rows, ld, eps, st);
    case 5: return parts_go<5>(x, part, w, n, rows, ld, eps, st);
    case 6: return parts_go<6>(x, part, w, n, rows, ld, eps, st);
    case 7: return parts_go<7>(x, part, w, n, rows, ld, eps, st);
    default: return parts_go<8>(x, part, w, n, rows, ld, eps, st);
    }
}

int rmsnorm_launch(const float* x, const float* w, float* out, int n, int rows, long ld, float eps,
                   hipStream_t st) {
    ATLAS_REQUIRE(x && w && out && n > 0 && rows > 0, "rmsnorm: bad arguments");
    const int threads = n >= 1024 ? 1024 : ((n + 63) / 64) * 64;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(threads), 0, st, x, w, out, n, ld, eps);
    ATLAS_LAUNCH_CHECK("rmsnorm");
    return ATLAS_OK;
}

int residual_rmsnorm_launch(float* x, const float* y, const float* w, int n, int rows, long ld,
                            float eps, hipStream_t st) {
    ATLAS_REQUIRE(x && y && w && n > 0 && rows > 0, "residual_rmsnorm: bad arguments");
    // packed rows up to 8192: the register-cached kernel (one split), whose
    // loads all go out before the first sum (8 rows of 4096: 5.1 -> ~4 us)
    if (ld == n && n <= 8192) return residual_rmsnorm_parts_launch(x, y, 1, w, n, rows, ld, eps, st);
    const int threads = n >= 1024 ? 1024 : ((n + 63) / 64) * 64;
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(rows), dim3(threads), 0, st, x, y, w, n, ld,
                       eps);
    ATLAS_LAUNCH_CHECK("residual_rmsnorm");
    return ATLAS_OK;
}

// ---- QK-norm + RoPE + KV write ---------------------------------------------
// grid (n_heads + n_kv [+ n_kv for V], n_seq), block = 64 (one wave per head).
// Head vector element e = lane + 64*j lives in registers and in LDS for the
// rotate-half partner e +- half.
__global__ __launch_bounds__(64) void qkv_post_kernel(QkvPostArgs a) {
    __shared__ float hv[256];
    const int s = blockIdx.y;
    const int hidx = blockIdx.x;
    const int HD = a.head_dim, half = HD / 2, lane = threadIdx.x;
    const int pos = a.pos_dev ? a.pos_dev[s] : a.pos;
    float* qkv = a.qkv + (long)s * a.qkv_stride;
    const int nq = a.n_heads, nkv = a.n_kv;
    const int slot = a.slot_dev ? a.slot_dev[s] : 0;
    const long cache_off = (long)slot * a.slot_stride + ((long)pos * nkv) * HD;
    // element off of this sequence's q|k|v: in place, or hi + lo product rows
    const long src_off = (a.src || a.src_d || a.src_parts) ? (long)s * a.src_stride : 0;
    auto in = [&](long off) {
        if (a.src_parts) {
            float sum = 0.f;
            for (int p = 0; p < a.src_splits; ++p) sum += a.src_parts[p * a.src_lo + off];
            return sum;
        }
        if (a.src_d) {
            // int8 digit products: planes src_lo apart, scales per row and column
            const int* p = a.src_d + off;
            const float lo = (float)p[a.src_lo] + (float)p[2 * a.src_lo] * (1.0f / 128.f);
            return ((float)p[0] + lo * (1.0f / 128.f)) * a.src_xs[s] * a.src_ws[off - src_off];
        }
        return a.src ? a.src[off] + a.src[a.src_lo + off] : qkv[off];
    };

    if (hidx >= nq + nkv) {
        // V head: copy into the cache
        const int vh = hidx - nq - nkv;
        float* dst = a.v_cache + cache_off + (long)vh * HD;
        for (int e = lane; e < HD; e += 64) dst[e] = in(src_off + (long)(nq + nkv + vh) * HD + e);
        return;
    }
    const bool is_q = hidx < nq;
    float* xh = qkv + (long)hidx * HD;
    const float* nw = is_q ? (a.q_norm ? a.q_norm + (long)hidx * HD : nullptr)
                           : (a.k_norm ? a.k_norm + (long)(hidx - nq) * HD : nullptr);
    float v[4];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < HD ? in(src_off + (long)hidx * HD + e) : 0.f;
        ss += v[j] * v[j];
    }
    if (nw) {
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)HD + a.qk_eps);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            if (e < HD) v[j] = v[j] * inv * nw[e];
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        if (e < HD) hv[e] = v[j];
    }
    __syncthreads();
    const float* c = a.cos_tab + (long)pos * half;
    const float* sn = a.sin_tab + (long)pos * half;
    float* dst = is_q ? xh : a.k_cache + cache_off + (long)(hidx - nq) * HD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        if (e < HD) {
            float r;
            if (e < half) r = hv[e] * c[e] - hv[e + half] * sn[e];
            else r = hv[e - half] * sn[e - half] + hv[e] * c[e - half];
            dst[e] = r;
        }
    }
}

int qkv_post_launch(const QkvPostArgs& a, int n_seq, hipStream_t st) {
    ATLAS_REQUIRE(a.head_dim > 0 && a.head_dim <= 256 && a.head_dim % 2 == 0,
                  "qkv_post: head_dim %d", a.head_dim);
    ATLAS_REQUIRE(a.qkv && a.k_cache && a.v_cache && a.cos_tab && a.sin_tab, "qkv_post: null");
    ATLAS_REQUIRE(n_seq >= 1, "qkv_post: n_seq");
    hipLaunchKernelGGL(qkv_post_kernel, dim3(a.n_heads + 2 * a.n_kv, n_seq), dim3(64), 0, st, a);
    ATLAS_LAUNCH_CHECK("qkv_post");
    return ATLAS_OK;
}

// ---- reference-compatible single ops --------------------------------------

// qk_norm_inplace (kernels/matmul.cu:662-710 contract): grid n_heads
__global__ __launch_bounds__(64) void qk_norm_kernel(float* x, const float* w, int hd, float eps) {
    float* xh = x + (long)blockIdx.x * hd;
    const float* wh = w + (long)blockIdx.x * hd;
    float ss = 0.f;
    for (int e = threadIdx.x; e < hd; e += 64) ss += xh[e] * xh[e];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    for (int e = threadIdx.x; e < hd; e += 64) xh[e] = xh[e] * inv * wh[e];
}

int qk_norm_launch(float* x, const float* w, int n_heads, int hd, float eps, hipStream_t st) {
    ATLAS_REQUIRE(x && w && n_heads > 0 && hd > 0, "qk_norm: bad arguments");
    hipLaunchKernelGGL(qk_norm_kernel, dim3(n_heads), dim3(64), 0, st, x, w, hd, eps);
    ATLAS_LAUNCH_CHECK("qk_norm");
    return ATLAS_OK;
}

// rope_precomputed (kernels/matmul.cu:723-743 contract): grid n_heads
__global__ __launch_bounds__(64) void rope_tab_kernel(float* x, const float* c, const float* s,
                                                      int hd, int pos) {
    float* xh = x + (long)blockIdx.x * hd;
    const int half = hd / 2;
    const float* cr = c + (long)pos * half;
    const float* sr = s + (long)pos * half;
    for (int i = threadIdx.x; i < half; i += 64) {
        const float x0 = xh[i], x1 = xh[i + half];
        xh[i] = x0 * cr[i] - x1 * sr[i];
        xh[i + half] = x0 * sr[i] + x1 * cr[i];
    }
}

int rope_tab_launch(float* x, const float* c, const float* s, int n_heads, int hd, int pos,
                    int max_seq, hipStream_t st) {
    ATLAS_REQUIRE(x && c && s && n_heads > 0 && hd > 0 && hd % 2 == 0, "rope: bad arguments");
    ATLAS_REQUIRE(pos >= 0 && pos < max_seq, "rope: pos %d outside [0, %d)", pos, max_seq);
    hipLaunchKernelGGL(rope_tab_kernel, dim3(n_heads), dim3(64), 0, st, x, c, s, hd, pos);
    ATLAS_LAUNCH_CHECK("rope");
    return ATLAS_OK;
}

// rope_apply (kernels/matmul.cu:285-300 contract; lib.rs:570-587 CPU form)
__global__ void rope_apply_kernel(float* x, int pos, int hd, float theta) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2;
    if (i >= half) return;
    const float freq = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
    const float ang = (float)pos * freq;
    const float c = cosf(ang), s = sinf(ang);
    const float x0 = x[i], x1 = x[i + half];
    x[i] = x0 * c - x1 * s;
    x[i + half] = x0 * s + x1 * c;
}

int rope_apply_launch(float* x, int pos, int hd, float theta, hipStream_t st) {
    ATLAS_REQUIRE(x && hd > 0, "rope_apply: bad arguments");
    const int half = hd / 2;
    if (half == 0) return ATLAS_OK;
    hipLaunchKernelGGL(rope_apply_kernel, dim3((half + 63) / 64), dim3(64), 0, st, x, pos, hd, theta);
    ATLAS_LAUNCH_CHECK("rope_apply");
    return ATLAS_OK;
}

__global__ void kv_write_kernel(float* kc, float* vc, const float* nk, const float* nv, long off,
                                int total) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < total) { kc[off + i] = nk[i]; vc[off + i] = nv[i]; }
}

int kv_write_launch(float* kc, float* vc, const float* nk, const float* nv, int pos, int n_kv,
                    int hd, hipStream_t st) {
    ATLAS_REQUIRE(kc && vc && nk && nv && pos >= 0 && n_kv > 0 && hd > 0, "kv_write: bad arguments");
    const int total = n_kv * hd;
    hipLaunchKernelGGL(kv_write_kernel, dim3((total + 255) / 256), dim3(256), 0, st, kc, vc, nk, nv,
                       (long)pos * total, total);
    ATLAS_LAUNCH_CHECK("kv_write");
    return ATLAS_OK;
}

// ---- elementwise -------------------------------------------------------------
__global__ void ew_kernel(int op, const float* a, const float* b, float* out, float s, long n) {
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        switch (op) {
        case EW_ADD: out[i] = a[i] + b[i]; break;
        case EW_SCALE: out[i] = a[i] * s; break;
        case EW_RELU: out[i] = a[i] > 0.f ? a[i] : 0.f; break;
        case EW_SILU_MUL: { const float g = a[i]; out[i] = g / (1.0f + expf(-g)) * b[i]; } break;
        case EW_COPY: out[i] = a[i]; break;
        case EW_FILL: out[i] = s; break;
        }
    }
}

int ew_launch(int op, const float* a, const float* b, float* out, float s, long n, hipStream_t st) {
    ATLAS_REQUIRE(n >= 0 && out, "elementwise: bad arguments");
    if (n == 0) return ATLAS_OK;
    long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(ew_kernel, dim3((unsigned)blocks), dim3(256), 0, st, op, a, b, out, s, n);
    ATLAS_LAUNCH_CHECK("elementwise");
    return ATLAS_OK;
}

// row softmax (kernels/matmul.cu:96-134 contract): one block per row
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* x, float* out, int cols) {
    const float* xr = x + (long)blockIdx.x * cols;
    float* orow = out + (long)blockIdx.x * cols;
    __shared__ float red[4];
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < cols; i += 256) mx = fmaxf(mx, xr[i]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.f;
    for (int i = threadIdx.x; i < cols; i += 256) sum += expf(xr[i] - mx);
    sum = block_sum(sum);
    const float inv = 1.0f / sum;
    for (int i = threadIdx.x; i < cols; i += 256) orow[i] = expf(xr[i] - mx) * inv;
}

int softmax_rows_launch(const float* x, float* out, int rows, int cols, hipStream_t st) {
    ATLAS_REQUIRE(x && out && rows >= 0 && cols > 0, "softmax: bad arguments");
    if (rows == 0) return ATLAS_OK;
    hipLaunchKernelGGL(softmax_rows_kernel, dim3(rows), dim3(256), 0, st, x, out, cols);
    ATLAS_LAUNCH_CHECK("softmax");
    return ATLAS_OK;
}

// AdamW (kernels/matmul.cu:138-161 contract; training, kept for ABI parity).
// bc1/bc2 are the reciprocal bias corrections 1/(1 - beta^t) that the caller
// computes (crates/atlas-optim/src/lib.rs:203-204), so they multiply; weight
// decay is decoupled: p * (1 - lr*wd) - lr * m_hat / (sqrt(v_hat) + eps).
__global__ void adamw_kernel(float* p, float* m, float* v, const float* g, float lr, float b1,
                             float b2, float eps, float wd, float bc1, float bc2, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gi = g[i];
    const float mi = b1 * m[i] + (1.f - b1) * gi;
    const float vi = b2 * v[i] + (1.f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const float mh = mi * bc1, vh = vi * bc2;
    p[i] = p[i] * (1.f - lr * wd) - lr * mh / (sqrtf(vh) + eps);
}

int adamw_launch(float* p, float* m, float* v, const float* g, float lr, float b1, float b2,
                 float eps, float wd, float bc1, float bc2, int n, hipStream_t st) {
    ATLAS_REQUIRE(p && m && v && g && n >= 0, "adamw: bad arguments");
    if (n == 0) return ATLAS_OK;
    hipLaunchKernelGGL(adamw_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, m, v, g, lr, b1, b2,
                       eps, wd, bc1, bc2, n);
    ATLAS_LAUNCH_CHECK("adamw");
    // the reference returns with the update complete (kernels/matmul.cu:555-556)
    ATLAS_HIP(hipStreamSynchronize(st));
    return ATLAS_OK;
}

// ---- token choice --------------------------------------------------------------
// ordered key: larger float -> larger key; ties keep the larger index (last max)
__device__ __forceinline__ unsigned long long argkey(float v, int i) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)i;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
    for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
    }
    return k;
}

// Penalties are applied in place to the logits (the caller's buffer is a
// scratch copy, as the reference clones its logits before choosing).
__global__ __launch_bounds__(256) void penalize_kernel(float* logits, int n, const int* step_dev,
                                                       const uint32_t* suppress, int n_suppress,
                                                       const uint32_t* hist, const int* hist_len_dev,
                                                       int window, float theta) {
    if (blockIdx.x != 0) return;
    const int step = step_dev ? *step_dev : 0;
    if (step == 0)
        for (int i = threadIdx.x; i < n_suppress; i += 256)
            if (suppress[i] < (uint32_t)n) logits[suppress[i]] = -INFINITY;
    __syncthreads();
    if (theta != 1.0f && hist && hist_len_dev) {
        const int len = *hist_len_dev;
        const int start = len > window ? len - window : 0;
        // sequential in history order: a token seen twice is penalised twice
        if (threadIdx.x == 0)
            for (int i = start; i < len; ++i) {
                const uint32_t t = hist[i];
                if (t < (uint32_t)n) {
                    if (logits[t] > 0.f) logits[t] /= theta;
                    else logits[t] *= theta;
                }
            }
    }
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ x, int n,
                                                             unsigned long long* __restrict__ part) {
    __shared__ unsigned long long red[4];
    unsigned long long best = 0;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const unsigned long long k = argkey(x[i], i);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int w = 1; w < 4; ++w) b = red[w] > b ? red[w] : b;
        part[blockIdx.x] = b;
    }
}

// One block of 1024 threads; each thread issues all of its (at most 16)
// partial-key loads before the first compare, so the reduction costs one
// cache round trip rather than one per loop trip (8192 keys: 7.9 us with a
// 256-thread strided loop that waited on every load).
__global__ __launch_bounds__(1024) void argmax_final_kernel(const unsigned long long* __restrict__ part,
                                                            int nparts, float* out_f32,
                                                            uint32_t* out_u32, uint32_t* hist,
                                                            int* hist_len, int* step, int* pos_inc) {
    constexpr int PER = ARGMAX_MAX_PARTS / 1024;
    __shared__ unsigned long long red[16];
    unsigned long long k[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = threadIdx.x + 1024 * j;
        k[j] = i < nparts ? part[i] : 0ull;
    }
    unsigned long long best = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) best = k[j] > best ? k[j] : best;
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int w = 1; w < 16; ++w) b = red[w] > b ? red[w] : b;
        const uint32_t idx = (uint32_t)(b & 0xFFFFFFFFu);
        if (out_f32) *out_f32 = (float)idx;
        if (out_u32) *out_u32 = idx;
        if (hist && hist_len) { hist[*hist_len] = idx; *hist_len += 1; }
        if (step) *step += 1;
        if (pos_inc) *pos_inc += 1;
    }
}

// Greedy choice of `rows` logit rows (row r at x + r*ld) in two launches:
// argmax_partial_kernel over a (parts, rows) grid, then one final block per
// row writing out_u32[r]; the same keys and tie rule (last maximal index) as
// argmax_launch per row.
__global__ __launch_bounds__(256) void argmax_partial_rows_kernel(const float* __restrict__ x, int n,
                                                                  long ld,
                                                                  unsigned long long* __restrict__ part) {
    __shared__ unsigned long long red[4];
    const float* xr = x + blockIdx.y * ld;
    unsigned long long best = 0;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const unsigned long long k = argkey(xr[i], i);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int w = 1; w < 4; ++w) b = red[w] > b ? red[w] : b;
        part[(long)blockIdx.y * gridDim.x + blockIdx.x] = b;
    }
}

__global__ __launch_bounds__(1024) void argmax_final_rows_kernel(const unsigned long long* __restrict__ part,
                                                                 int nparts, uint32_t* __restrict__ out_u32) {
    __shared__ unsigned long long red[16];
    const unsigned long long* pr = part + (long)blockIdx.x * nparts;
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < nparts; i += 1024) best = pr[i] > best ? pr[i] : best;
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
        for (int w = 1; w < 16; ++w) b = red[w] > b ? red[w] : b;
        out_u32[blockIdx.x] = (uint32_t)(b & 0xFFFFFFFFu);
    }
}

int argmax_rows_launch(const float* x, int n, long ld, int rows, unsigned long long* part,
                       uint32_t* out_u32, hipStream_t st) {
    ATLAS_REQUIRE(x && part && out_u32 && n > 0 && rows > 0 && rows <= 65535, "argmax rows: bad arguments");
    int parts = (n + 255) / 256;
    if (parts > 512) parts = 512;
    ATLAS_REQUIRE((long)parts * rows <= ARGMAX_MAX_PARTS, "argmax rows: %d rows x %d partials exceed %d",
                  rows, parts, (int)ARGMAX_MAX_PARTS);
    hipLaunchKernelGGL(argmax_partial_rows_kernel, dim3(parts, rows), dim3(256), 0, st, x, n, ld, part);
    ATLAS_LAUNCH_CHECK("argmax_partial_rows");
    hipLaunchKernelGGL(argmax_final_rows_kernel, dim3(rows), dim3(1024), 0, st, part, parts, out_u32);
    ATLAS_LAUNCH_CHECK("argmax_final_rows");
    return ATLAS_OK;
}

int argmax_launch(const ArgmaxArgs& a, hipStream_t st) {
    ATLAS_REQUIRE(a.x && a.n > 0 && a.part, "argmax: bad arguments");
    if (a.n_parts <= 0 && (a.suppress || (a.theta != 1.0f && a.hist))) {
        hipLaunchKernelGGL(penalize_kernel, dim3(1), dim3(256), 0, st, (float*)a.x, a.n, a.step,
                           a.suppress, a.n_suppress, a.hist, a.hist_len, a.window, a.theta);
        ATLAS_LAUNCH_CHECK("penalize");
    }
    int blocks = a.n_parts;
    if (blocks <= 0) {
        // partials not precomputed (by a GEMV epilogue): reduce the logits here
        blocks = (a.n + 255) / 256;
        if (blocks > ARGMAX_MAX_PARTS) blocks = ARGMAX_MAX_PARTS;
        hipLaunchKernelGGL(argmax_partial_kernel, dim3(blocks), dim3(256), 0, st, a.x, a.n, a.part);
        ATLAS_LAUNCH_CHECK("argmax_partial");
    }
    ATLAS_REQUIRE(blocks <= ARGMAX_MAX_PARTS, "argmax: %d partials exceed %d", blocks,
                  (int)ARGMAX_MAX_PARTS);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, st, a.part, blocks, a.out_f32,
                       a.out_u32, a.record ? a.hist : nullptr, a.record ? a.hist_len : nullptr,
                       a.step, a.pos_inc);
    ATLAS_LAUNCH_CHECK("argmax_final");
    return ATLAS_OK;
}

// ---- device sampling: one token of generate_with_sampling (lib.rs:1623-1711) ------
// One block of 1024 threads.  After the penalties, every stage works on the
// top-k survivors compacted in index order: the reference's sums over the whole
// vocabulary add exact zeros for the other entries (expf(-inf) = 0), so the
// sequential loops here over the survivors give the same sums bit for bit.
// The one difference is expf: the reference calls glibc's, which is not
// correctly rounded for ~1e-4 of arguments; this computes exp in double and
// rounds once (correctly rounded up to double's own error).

// larger float -> larger key
__device__ __forceinline__ uint32_t sample_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float sample_exp(float x) { return (float)exp((double)x); }

__device__ float block_max1024(float v, float* sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < 16; ++i) r = fmaxf(r, sh[i]);
    __syncthreads();
    return r;
}

// exclusive prefix sum of v over the 1024 threads; *total receives the sum
__device__ int block_excl_scan1024(int v, int* sh, int* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int incl = v;
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
    }
    if (lane == 63) sh[w] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int i = 0; i < 16; ++i) {
            const int t = sh[i];
            sh[i] = acc;
            acc += t;
        }
        sh[16] = acc;
    }
    __syncthreads();
    const int r = sh[w] + incl - v;
    *total = sh[16];
    __syncthreads();
    return r;
}

// Wave 0: the bin of `bins` (counts, nb of them, top bin first in rank order)
// holding rank kk from the top, and the rank left inside that bin.
__device__ void radix_pick(const int* bins, int nb, int kk, int* out_bin, int* out_kk) {
    const int lane = threadIdx.x & 63;
    const int per = nb / 64;
    int sum = 0;
    for (int j = 0; j < per; ++j) sum += bins[nb - 1 - (lane * per + j)];
    int incl = sum;
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
    }
    const unsigned long long ball = __ballot(incl >= kk);
    const int first = ball ? __ffsll((long long)ball) - 1 : 63;
    if (lane == first) {
        int acc = incl - sum;
        int b = nb - 1 - lane * per - (per - 1), k2 = kk - acc;
        for (int j = 0; j < per; ++j) {
            const int bb = nb - 1 - (lane * per + j);
            if (acc + bins[bb] >= kk) {
                b = bb;
                k2 = kk - acc;
                break;
            }
            acc += bins[bb];
        }
        *out_bin = b;
        *out_kk = k2;
    }
}

__device__ __forceinline__ float sample_unkey(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

// The kk-th largest (1-based) of keys[0..cnt) in LDS, and how many entries
// equal to it rank within the first kk: radix select, 11 + 11 + 10 bits.
__device__ void lds_select(const uint32_t* keys, int cnt, int kk, int* bins, int* pick,
                           uint32_t* th, int* need) {
    uint32_t prefix = 0, mask = 0;
    for (int pass = 0; pass < 3; ++pass) {
        const int shift = pass == 0 ? 21 : pass == 1 ? 10 : 0;
        const int nb = pass == 2 ? 1024 : 2048;
        for (int i = threadIdx.x; i < nb; i += 1024) bins[i] = 0;
        __syncthreads();
        for (int i = threadIdx.x; i < cnt; i += 1024) {
            const uint32_t key = keys[i];
            if ((key & mask) == prefix) atomicAdd(&bins[(key >> shift) & (uint32_t)(nb - 1)], 1);
        }
        __syncthreads();
        if (threadIdx.x < 64) radix_pick(bins, nb, kk, &pick[0], &pick[1]);
        __syncthreads();
        prefix |= (uint32_t)pick[0] << shift;
        mask |= (uint32_t)(nb - 1) << shift;
        kk = pick[1];
        __syncthreads();
    }
    *th = prefix;
    *need = kk;
}

// ascending bitonic sort of s[0..np2) (np2 a power of two), all 1024 threads
__device__ void bitonic_u32(uint32_t* s, int np2) {
    for (int k2 = 2; k2 <= np2; k2 <<= 1)
        for (int j2 = k2 >> 1; j2 > 0; j2 >>= 1) {
            for (int i = threadIdx.x; i < np2; i += 1024) {
                const int p = i ^ j2;
                if (p > i) {
                    const bool up = (i & k2) == 0;
                    const uint32_t u = s[i], v = s[p];
                    if ((u > v) == up) { s[i] = v; s[p] = u; }
                }
            }
            __syncthreads();
        }
}

// hist[lo, hi) into s sorted ascending (padding 0xFFFFFFFF up to a power of two)
__device__ int sorted_tokens(const uint32_t* hist, int lo, int hi, uint32_t* s) {
    const int len = hi - lo;
    int np2 = 1;
    while (np2 < len) np2 <<= 1;
    for (int i = threadIdx.x; i < np2; i += 1024) s[i] = i < len ? hist[lo + i] : 0xFFFFFFFFu;
    __syncthreads();
    bitonic_u32(s, np2);
    return len;
}

// ---- top_k = 0 with top_p off: the whole vocabulary samples ----------------
// The reference sums p_i = exp(v_i - max) sequentially in f32, scales them by
// inv = 1 / sum and takes the first i whose sequential f32 running sum of
// p_i * inv exceeds the draw u (lib.rs:351-357, 2710-2717).  Here the running
// sums are exact prefix sums C_j in double (a block scan over contiguous
// segments, in index order), and the candidate j with C_{j-1} <= u < C_j is
// the reference's choice whenever u clears both boundaries by what rounding
// can move the f32 sums.  With g = gamma_{m-1} = (m-1)e / (1 - (m-1)e),
// e = 2^-24, for the m non-zero terms (the error bound of recursive summation
// of non-negative terms, Higham, "Accuracy and Stability of Numerical
// Algorithms", 2nd ed., sec. 4.2), the reference's sum lies within S(1 +- g),
// inv and each p_i * inv add one rounding each, and its running sum within
// another factor (1 +- g): every running sum lies in
// [C_j (1-e)^2 (1-g)/(1+g), C_j (1+e)^2 (1+g)/(1-g)], plus 2^-150 per term
// where products or sums underflow.  When u falls inside that band (about 2g
// of draws, g ~ 0.006 at a 100K vocabulary) the sums are redone sequentially
// in f32, exactly as the reference does them.

// exclusive prefix sums of v (double) over the 1024 threads into base[0..1024]
// (base[1024] = the total)
__device__ void block_scan1024_f64(double v, double* base, double* sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    double incl = v;
    for (int off = 1; off < 64; off <<= 1) {
        const double t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
    }
    double excl = __shfl_up(incl, 1, 64);
    if (lane == 0) excl = 0.0;
    if (lane == 63) sh[w] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        double acc = 0.0;
        for (int i = 0; i < 16; ++i) {
            const double t = sh[i];
            sh[i] = acc;
            acc += t;
        }
        base[1024] = acc;
    }
    __syncthreads();
    base[threadIdx.x] = sh[w] + excl;
    __syncthreads();
}

constexpr int kSampleStage = 16384;      // floats staged per chunk (64 KB of LDS)

// ---- the reference's sequential f32 running sums, computed in parallel -----
// While the running sum s stays in one binade [2^E, 2^(E+1)), every float there
// is a multiple of q = 2^(E-23), so fl(s + v) = s + r q with r = v / q rounded
// to nearest: independent of s except at an exact tie, which rounds to the
// even multiple and so depends on the parity of s / q.  Each value is thus a
// map of the running parity b to (r(b), parity after); these maps compose
// associatively, a block scan gives every running sum of a chunk exactly, up
// to the first value whose sum leaves the binade.  Thread 0 adds that one in
// f32 and the scan resumes after it with the new binade's grid.  The first
// kRunSeq values, where a small running sum changes binade often, are added
// by thread 0 in order.
struct RunMap {
    int r0, r1;              // units of q added from parity 0 / parity 1 (saturating at kRunSat)
    int p;                   // bit 0: parity after from 0, bit 1: parity after from 1
};
constexpr int kRunSeq = 256;
constexpr int kRunTop = 1 << 24;         // units of q at the binade's top
constexpr int kRunSat = 1 << 30;         // sums saturate here (>= kRunTop: leaves anyway)

__device__ __forceinline__ RunMap run_identity() { return {0, 0, 2}; }

__device__ __forceinline__ int run_add(int a, int b) { return a + b < kRunSat ? a + b : kRunSat; }

// a, then b
__device__ __forceinline__ RunMap run_compose(const RunMap& a, const RunMap& b) {
    const int a0 = a.p & 1, a1 = (a.p >> 1) & 1, b0 = b.p & 1, b1 = (b.p >> 1) & 1;
    RunMap m;
    m.r0 = run_add(a.r0, a0 ? b.r1 : b.r0);
    m.r1 = run_add(a.r1, a1 ? b.r1 : b.r0);
    m.p = (a0 ? b1 : b0) | ((a1 ? b1 : b0) << 1);
    return m;
}

// adding v (>= 0, finite) on the grid q = 2^(E - 23), from v's bits: v = m 2^(ev - 23)
// with m its 24-bit significand, so v / q = m 2^(ev - E)
__device__ __forceinline__ RunMap run_map(float v, int E) {
    const uint32_t u = __float_as_uint(v);
    const int be = (int)(u >> 23);
    const uint32_t m = be ? ((u & 0x7FFFFFu) | 0x800000u) : (u & 0x7FFFFFu);
    const int ev = be ? be - 127 : -126;
    const int d = E - ev;
    RunMap r;
    if (d <= 0) {                            // v / q is an integer, at least m
        const int f = -d >= 7 ? kRunSat : (int)min((uint32_t)kRunSat, m << -d);
        r.r0 = r.r1 = f;
        r.p = (f & 1) | (((f + 1) & 1) << 1);
        return r;
    }
    if (d > 25) {                            // v < q / 2: adds nothing
        r.r0 = r.r1 = 0;
        r.p = 2;
        return r;
    }
    const int f = (int)(m >> d);
    const uint32_t rem = m & ((1u << d) - 1), half = 1u << (d - 1);
    if (rem == half) {                       // a tie: to the even multiple
        r.r0 = f + (f & 1);
        r.r1 = f + ((f + 1) & 1);
        r.p = 0;
        return r;
    }
    const int g = rem > half ? f + 1 : f;
    r.r0 = r.r1 = g;
    r.p = (g & 1) | (((g + 1) & 1) << 1);
    return r;
}

// the binade of s (subnormals share the first normal binade's grid 2^-149)
// and s in units of its grid
__device__ __forceinline__ int run_binade(float s, int* K) {
    const uint32_t u = __float_as_uint(s);
    const int be = (int)(u >> 23);
    if (be <= 1) {                           // s < 2^-125: grid 2^-149, s = bits
        *K = (int)u;
        return -126;
    }
    *K = (int)((u & 0x7FFFFFu) | 0x800000u);
    return be - 127;
}

__device__ __forceinline__ float run_value(int K, int E) { return ldexpf((float)K, E - 23); }

__device__ __forceinline__ RunMap run_shfl_up(const RunMap& m, int d) {
    RunMap o;
    o.r0 = __shfl_up(m.r0, d, 64);
    o.r1 = __shfl_up(m.r1, d, 64);
    o.p = __shfl_up(m.p, d, 64);
    return o;
}

// the minima of a and of b over the block (sh: 32 ints)
__device__ __forceinline__ void block_min2_1024(int a, int b, int* sh, int* oa, int* ob) {
    for (int off = 32; off >= 1; off >>= 1) {
        a = min(a, __shfl_xor(a, off, 64));
        b = min(b, __shfl_xor(b, off, 64));
    }
    if ((threadIdx.x & 63) == 0) { sh[threadIdx.x >> 6] = a; sh[16 + (threadIdx.x >> 6)] = b; }
    __syncthreads();
    int ra = sh[0], rb = sh[16];
    for (int i = 1; i < 16; ++i) { ra = min(ra, sh[i]); rb = min(rb, sh[16 + i]); }
    __syncthreads();
    *oa = ra;
    *ob = rb;
}

// Running sums of v_i = x[i] (kind 0) or v_i = x[i] * inv (kind 1), i in [0, n),
// in order in f32, exactly as a sequential loop gives them.  kind 0: returns
// -1 and *sum the total.  kind 1: returns the first i with u < running sum
// (n - 1 if there is none, as sample_from_probs).  Spans start at 1024 values
// and double while no value leaves the binade (a small running sum changes
// binade often; a restart only redoes the rest of its span).
__device__ int exact_run(const float* x, int n, int kind, float inv, float u, float* buf, RunMap* sw,
                         int* si, float* sf, float* sum) {
#pragma clang fp contract(off)
    constexpr int PMAX = kSampleStage / 1024;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n0 = n < kRunSeq ? n : kRunSeq;
    for (int i = tid; i < n0; i += 1024) buf[i] = kind ? x[i] * inv : x[i];
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        int hit = -1;
        for (int i = 0; i < n0; ++i) {
            s += buf[i];
            if (kind && u < s) { hit = i; break; }
        }
        sf[0] = s;
        si[0] = hit;
    }
    __syncthreads();
    if (kind && si[0] >= 0) return si[0];
    int pos = n0, span = 1024;
    while (pos < n) {
        const int cnt = n - pos < span ? n - pos : span;
        const int per = (cnt + 1023) / 1024;
        for (int i = tid; i < cnt; i += 1024) buf[i] = kind ? x[pos + i] * inv : x[pos + i];
        __syncthreads();
        int K0;
        const int E = run_binade(sf[0], &K0);
        const int b0 = K0 & 1;
        // this thread's values [tid * per, +per), their maps and their composition
        RunMap mp[PMAX];
        RunMap m = run_identity();
#pragma unroll
        for (int j = 0; j < PMAX; ++j) {
            const int i = tid * per + j;
            mp[j] = (j < per && i < cnt) ? run_map(buf[i], E) : run_identity();
            m = run_compose(m, mp[j]);
        }
        // block scan: the map of every value before this thread's
        RunMap inc = m;
        for (int off = 1; off < 64; off <<= 1) {
            const RunMap t = run_shfl_up(inc, off);
            if (lane >= off) inc = run_compose(t, inc);
        }
        RunMap exc = run_shfl_up(inc, 1);
        if (lane == 0) exc = run_identity();
        if (lane == 63) sw[w] = inc;
        __syncthreads();
        if (tid == 0) {
            RunMap acc = run_identity();
            for (int i = 0; i < 16; ++i) {
                const RunMap t = sw[i];
                sw[i] = acc;
                acc = run_compose(acc, t);
            }
            sw[16] = acc;
        }
        __syncthreads();
        const RunMap pre = run_compose(sw[w], exc);
        // every running sum of this thread's values, exact until one leaves the binade
        int K = run_add(K0, b0 ? pre.r1 : pre.r0);
        int b = b0 ? (pre.p >> 1) & 1 : pre.p & 1;
        int cross = INT_MAX, hit = INT_MAX, Kc = 0;
#pragma unroll
        for (int j = 0; j < PMAX; ++j) {
            const int i = tid * per + j;
            if (j < per && i < cnt && cross == INT_MAX) {
                const int Ka = run_add(K, b ? mp[j].r1 : mp[j].r0);
                if (Ka >= kRunTop) {
                    cross = i;
                    Kc = K;
                } else if (kind && hit == INT_MAX && u < run_value(Ka, E)) {
                    hit = i;
                }
                K = Ka;
                b = b ? (mp[j].p >> 1) & 1 : mp[j].p & 1;
            }
        }
        int gc, gh;
        block_min2_1024(cross, hit, si + 4, &gc, &gh);
        if (gh < gc) return pos + gh;
        if (gc == INT_MAX) {                     // no value leaves the binade: the span's total
            if (tid == 0) {
                const RunMap t = sw[16];
                sf[0] = run_value(K0 + (b0 ? t.r1 : t.r0), E);
            }
            __syncthreads();
            pos += cnt;
            span = span * 2 < kSampleStage ? span * 2 : kSampleStage;
            continue;
        }
        if (cross == gc) {                       // the value that leaves it, added in f32
            const float sn = run_value(Kc, E) + buf[gc];
            sf[0] = sn;
            si[1] = kind && u < sn;
        }
        __syncthreads();
        if (si[1]) return pos + gc;
        pos += gc + 1;
        __syncthreads();
    }
    *sum = sf[0];
    return kind ? n - 1 : -1;
}

// One draw over the whole (penalised) vocabulary x[0..n); thread 0 returns it.
// x is overwritten with the unnormalised probabilities p_i.
__device__ uint32_t sample_all_vocab(float* x, int n, const SampleCfg& c, float u, float* buf,
                                     double* base, double* sh, float* red, int* flag, RunMap* rmaps,
                                     float* stmp) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const float T = c.temperature;
    // max of v = x / T (lib.rs:1684-1686): the max of x divided once (correctly
    // rounded division by T > 0 is monotone), 16 coalesced loads in flight
    float mxx = -INFINITY;
    for (int b0 = tid; b0 < n; b0 += 1024 * 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = x[b0 + k * 1024 < n ? b0 + k * 1024 : n - 1];
#pragma unroll
        for (int k = 0; k < 16; ++k) mxx = fmaxf(mxx, v[k]);
    }
    const float mx = block_max1024(mxx, red) / T;
    const float th = c.min_p > 0.0f ? mx + c.log_min_p : -INFINITY;    // min-p's threshold
    // p_i = exp(v_i - max) in place (0 below the threshold); their sum in
    // double (any order: S is only compared to within 1e-12) and the non-zero count
    double part = 0.0;
    int nz = 0;
    for (int b0 = tid; b0 < n; b0 += 1024 * 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = x[b0 + k * 1024 < n ? b0 + k * 1024 : n - 1];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int i = b0 + k * 1024;
            const float vt = v[k] / T;
            const float p = vt < th ? 0.0f : sample_exp(vt - mx);
            if (i < n) {
                x[i] = p;
                part += (double)p;
                nz += p != 0.0f;
            }
        }
    }
    int m;
    (void)block_excl_scan1024(nz, flag + 2, &m);
    block_scan1024_f64(part, base, sh);
    const double S = base[1024];
    const double target = (double)u * S;
    if (tid == 0) { flag[0] = 0; flag[1] = -1; }
    // the band's width at u (relative 2g + 4e): no interval C_j - C_(j-1) is
    // wider than p_max / S = 1 / S, so when that is well inside the band the
    // check cannot pass and the exact sums run at once
    const double e = 0x1p-24;
    const double kk = m > 1 ? (double)(m - 1) * e : 0.0;
    const double g = kk / (1.0 - kk);
    const double hi_f = (1.0 + e) * (1.0 + e) * (1.0 + g) / (1.0 - g) + 1e-12;
    const double lo_f = (1.0 - e) * (1.0 - e) * (1.0 - g) / (1.0 + g) - 1e-12;
    const bool try_band = 1.0 / S >= 0.5 * (double)u * (hi_f - lo_f);
    // the exact prefix sums C_j in index order, chunk by chunk through LDS
    // (each thread sums 16 consecutive values), up to the chunk holding the
    // crossing; its owner finds j and checks the band
    constexpr int PER = kSampleStage / 1024;
    double cbase = 0.0;
    for (int c0 = 0; c0 < n && try_band; c0 += kSampleStage) {
        const int cnt = n - c0 < kSampleStage ? n - c0 : kSampleStage;
        __syncthreads();
        for (int i = tid; i < cnt; i += 1024) buf[i] = x[c0 + i];
        __syncthreads();
        double mine = 0.0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = tid * PER + j;
            mine += i < cnt ? (double)buf[i] : 0.0;
        }
        block_scan1024_f64(mine, base, sh);
        const double lo_c = cbase + base[tid], hi_c = cbase + base[tid + 1];
        if (lo_c <= target && target < hi_c) {
            double pre = lo_c;
            for (int j = 0; j < PER; ++j) {
                const int i = tid * PER + j;
                if (i >= cnt) break;
                const double prev = pre;
                pre += (double)buf[i];
                if (pre > target) {
                    const double slack = 1e-35;
                    const double uu = (double)u;
                    flag[1] = c0 + i;
                    if ((prev / S) * hi_f + slack <= uu && uu < (pre / S) * lo_f - slack) flag[0] = 1;
                    break;
                }
            }
        }
        cbase += base[1024];
        __syncthreads();
        if (flag[1] >= 0 || cbase > target) break;
    }
    __syncthreads();
    if (flag[0]) return (uint32_t)flag[1];
    // ---- inside the band: the reference's sums, exactly (exact_run)
    float sum, last;
    (void)exact_run(x, n, 0, 0.0f, 0.0f, buf, rmaps, flag + 8, stmp, &sum);
    const float inv = 1.0f / sum;
    const int tok = exact_run(x, n, 1, inv, u, buf, rmaps, flag + 8, stmp, &last);
    if (tid == 0) flag[1] = tok;
    __syncthreads();
    return (uint32_t)flag[1];       // n - 1 when no running sum exceeds u
}

__global__ __launch_bounds__(1024) void sample_kernel(SampleArgs a) {
#pragma clang fp contract(off)
    __shared__ uint32_t s_hist[SAMPLE_MAX_HIST];
    __shared__ int s_bins[2048];
    __shared__ int s_idx[SAMPLE_MAX_K];
    __shared__ float s_val[SAMPLE_MAX_K];
    __shared__ float s_p[SAMPLE_MAX_K];
    __shared__ int s_ord[SAMPLE_MAX_K];
    __shared__ int s_scan[17];
    __shared__ uint32_t s_ck[SAMPLE_CAND];      // top-k candidates: keys, index order
    __shared__ int s_ci[SAMPLE_CAND];           // and their indices
    __shared__ int s_wbase[17];
    __shared__ float s_red[16];
    __shared__ int s_pick[2];
    __shared__ float s_sum;
    const SampleCfg c = *a.cfg;
    const int tid = threadIdx.x, n = a.n;
    float* x = a.x;
    const int step = a.step ? *a.step : 0;
    const int len = (a.hist && a.hist_len) ? *a.hist_len : 0;

    // ---- step-0 suppression, then the repetition penalty in history order
    if (step == 0 && a.suppress)
        for (int i = tid; i < c.n_suppress; i += 1024)
            if (a.suppress[i] < (uint32_t)n) x[a.suppress[i]] = -INFINITY;
    __syncthreads();
    // A token seen r times in the window is penalised r times in a row (the
    // reference's loop in history order); distinct tokens are independent, so
    // one thread per distinct token of the sorted window gives the same values.
    // The host admits windows of at most SAMPLE_MAX_HIST tokens on this path.
    if (c.theta != 1.0f && len > 0) {
        int start = len > c.window ? len - c.window : 0;
        if (len - start > SAMPLE_MAX_HIST) start = len - SAMPLE_MAX_HIST;
        const int wl = sorted_tokens(a.hist, start, len, s_hist);
        for (int i = tid; i < wl; i += 1024) {
            const uint32_t t = s_hist[i];
            if (i > 0 && s_hist[i - 1] == t) continue;
            int j = i + 1;
            while (j < wl && s_hist[j] == t) ++j;
            if (t < (uint32_t)n) {
                float v = x[t];
                for (int r = i; r < j; ++r) v = v > 0.0f ? v / c.theta : v * c.theta;
                x[t] = v;
            }
        }
        __syncthreads();
    }

    // ---- frequency (times seen) and presence penalties per distinct token; the
    // host admits at most SAMPLE_MAX_HIST history entries on this path
    const int hl = len < SAMPLE_MAX_HIST ? len : SAMPLE_MAX_HIST;
    if ((c.freq != 0.0f || c.presence != 0.0f) && hl > 0) {
        sorted_tokens(a.hist, 0, hl, s_hist);
        for (int i = tid; i < hl; i += 1024) {
            const uint32_t t = s_hist[i];
            if (i > 0 && s_hist[i - 1] == t) continue;
            int j = i + 1;
            while (j < hl && s_hist[j] == t) ++j;
            if (t < (uint32_t)n) {
                float v = x[t];
                if (c.freq != 0.0f) v -= c.freq * (float)(j - i);
                if (c.presence != 0.0f) v -= c.presence;
                x[t] = v;
            }
        }
        __syncthreads();
    }

    // ---- top_k = 0 (top_p off): every token competes
    if (c.top_k == 0) {
        __shared__ double s_base[1025];
        __shared__ double s_dsh[16];
        __shared__ float s_u;
        __shared__ int s_flag[48];
        __shared__ __attribute__((aligned(16))) float s_stage[kSampleStage];
        __shared__ RunMap s_rmaps[17];
        __shared__ float s_stmp[2];
        if (tid == 0) {
            unsigned long long r = *a.rng;
            r ^= r << 13;
            r ^= r >> 7;
            r ^= r << 17;
            *a.rng = r;
            s_u = (float)(uint32_t)(r >> 33) / 2147483648.0f;
        }
        __syncthreads();
        const uint32_t tok = sample_all_vocab(x, n, c, s_u, s_stage, s_base, s_dsh, s_red, s_flag,
                                              s_rmaps, s_stmp);
        if (tid == 0) {
            if (a.out_u32) *a.out_u32 = tok;
            if (a.record && a.hist && a.hist_len) { a.hist[len] = tok; *a.hist_len = len + 1; }
            if (a.step) *a.step = step + 1;
            if (a.pos_inc) *a.pos_inc += 1;
        }
        return;
    }

    // ---- top-k (x / T): threshold key th = the k-th largest, ties at th kept
    // first by index; survivors compacted in index order into s_idx / s_val
    const float T = c.temperature;
    int k = c.top_k < 1 ? 1 : c.top_k;
    if (k > SAMPLE_MAX_K) k = SAMPLE_MAX_K;
    if (k > n) k = n;
    const int lane = tid & 63, wv = tid >> 6;
    // (a) The k-th largest of the 1024 per-thread maxima is a lower bound L of
    // th: those k maxima are k distinct entries >= it.
    uint32_t kmax = 0;
    for (int base = tid; base < n; base += 1024 * 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = base + u * 1024;
            v[u] = x[i < n ? i : n - 1];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const uint32_t key = sample_key(v[u] / T);
            if (base + u * 1024 < n && key > kmax) kmax = key;
        }
    }
    s_hist[tid] = kmax;                          // the penalties are done with s_hist
    __syncthreads();
    uint32_t L, th;
    int need, m;
    lds_select(s_hist, 1024, k, s_bins, s_pick, &L, &need);
    // (b) entries with key >= L, counted then written in index order: wave wv
    // owns a contiguous range and takes 4 x 64 consecutive entries per step
    const int chunk = ((n + 15) / 16 + 255) & ~255;
    const int c_lo = wv * chunk < n ? wv * chunk : n;
    const int c_hi = c_lo + chunk < n ? c_lo + chunk : n;
    int wcount = 0;
    for (int b = c_lo; b < c_hi; b += 256) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = b + u * 64 + lane;
            v[u] = x[i < n ? i : n - 1];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = b + u * 64 + lane;
            wcount += __popcll(__ballot(i < c_hi && sample_key(v[u] / T) >= L));
        }
    }
    if (lane == 0) s_wbase[wv] = wcount;
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        for (int w = 0; w < 16; ++w) {
            const int t = s_wbase[w];
            s_wbase[w] = acc;
            acc += t;
        }
        s_wbase[16] = acc;
    }
    __syncthreads();
    const int n_cand = s_wbase[16];
    if (n_cand <= SAMPLE_CAND) {
        int pos = s_wbase[wv];
        for (int b = c_lo; b < c_hi; b += 256) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = b + u * 64 + lane;
                v[u] = x[i < n ? i : n - 1];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = b + u * 64 + lane;
                const uint32_t key = sample_key(v[u] / T);
                const bool in = i < c_hi && key >= L;
                const unsigned long long bal = __ballot(in);
                if (in) {
                    const int at = pos + __popcll(bal & ((1ull << lane) - 1));
                    s_ck[at] = key;
                    s_ci[at] = i;
                }
                pos += __popcll(bal);
            }
        }
        __syncthreads();
        lds_select(s_ck, n_cand, k, s_bins, s_pick, &th, &need);
        // (c) survivors among the candidates (index order), one segment each
        const int seg = (n_cand + 1023) / 1024;
        const int lo = tid * seg < n_cand ? tid * seg : n_cand;
        const int hi = lo + seg < n_cand ? lo + seg : n_cand;
        int gt = 0, eq = 0;
        for (int i = lo; i < hi; ++i) {
            gt += s_ck[i] > th;
            eq += s_ck[i] == th;
        }
        int tot;
        const int eq_base = block_excl_scan1024(eq, s_scan, &tot);
        int keep_eq = need - eq_base;
        keep_eq = keep_eq < 0 ? 0 : (keep_eq > eq ? eq : keep_eq);
        int o = block_excl_scan1024(gt + keep_eq, s_scan, &m);
        int tie = eq_base;
        for (int i = lo; i < hi; ++i) {
            const uint32_t key = s_ck[i];
            bool keep = key > th;
            if (key == th) keep = tie++ < need;
            if (keep && o < SAMPLE_MAX_K) {
                s_idx[o] = s_ci[i];
                s_val[o] = sample_unkey(key);
                ++o;
            }
        }
    } else {
        // more candidates than LDS holds (long runs of equal logits): radix
        // select and survivors over the whole vocabulary
        uint32_t prefix = 0, mask = 0;
        int kk = k;
        for (int pass = 0; pass < 3; ++pass) {
            const int shift = pass == 0 ? 21 : pass == 1 ? 10 : 0;
            const int nb = pass == 2 ? 1024 : 2048;
            for (int i = tid; i < nb; i += 1024) s_bins[i] = 0;
            __syncthreads();
            // 16 independent loads per thread in flight, then their keys
            for (int base = tid; base < n; base += 1024 * 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int i = base + u * 1024;
                    v[u] = x[i < n ? i : n - 1];
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const uint32_t key = sample_key(v[u] / T);
                    if (base + u * 1024 < n && (key & mask) == prefix)
                        atomicAdd(&s_bins[(key >> shift) & (uint32_t)(nb - 1)], 1);
                }
            }
            __syncthreads();
            if (tid < 64) radix_pick(s_bins, nb, kk, &s_pick[0], &s_pick[1]);
            __syncthreads();
            prefix |= (uint32_t)s_pick[0] << shift;
            mask |= (uint32_t)(nb - 1) << shift;
            kk = s_pick[1];
            __syncthreads();
        }
        th = prefix;
        need = kk;                                   // ties at th kept, first by index

        // ---- survivors in index order (each thread one contiguous segment)
        const int seg = (n + 1023) / 1024;
        const int lo = tid * seg < n ? tid * seg : n;
        const int hi = lo + seg < n ? lo + seg : n;
        int gt = 0, eq = 0;
        for (int b = lo; b < hi; b += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = x[b + u < hi ? b + u : hi - 1];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const uint32_t key = sample_key(v[u] / T);
                if (b + u < hi) {
                    gt += key > th;
                    eq += key == th;
                }
            }
        }
        int tot;
        const int eq_base = block_excl_scan1024(eq, s_scan, &tot);
        int keep_eq = need - eq_base;
        keep_eq = keep_eq < 0 ? 0 : (keep_eq > eq ? eq : keep_eq);
        int o = block_excl_scan1024(gt + keep_eq, s_scan, &m);
        int tie = eq_base;
        for (int b = lo; b < hi; b += 16) {
            float w[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) w[u] = x[b + u < hi ? b + u : hi - 1];
            for (int u = 0; u < 16 && b + u < hi; ++u) {
                const float v = w[u] / T;
                const uint32_t key = sample_key(v);
                bool keep = key > th;
                if (key == th) keep = tie++ < need;
                if (keep && o < SAMPLE_MAX_K) {
                    s_idx[o] = b + u;
                    s_val[o] = v;
                    ++o;
                }
            }
        }
    }
    if (m > SAMPLE_MAX_K) m = SAMPLE_MAX_K;
    __syncthreads();

    // ---- top-p: probabilities of the survivors, ordered by (p desc, index),
    // cut where the running sum first reaches top_p
    if (c.top_p < 1.0f) {
        const float mx = block_max1024(tid < m ? s_val[tid] : -INFINITY, s_red);
        if (tid < m) s_p[tid] = sample_exp(s_val[tid] - mx);
        __syncthreads();
        if (tid == 0) {
            float sum = 0.0f;
            for (int i = 0; i < m; ++i) sum += s_p[i];
            s_sum = sum;
        }
        __syncthreads();
        const float sum = s_sum;
        if (sum > 0.0f) {
            if (tid < m) s_p[tid] = s_p[tid] / sum;
            int np2 = 1;
            while (np2 < m) np2 <<= 1;
            s_ord[tid] = tid;                       // np2 <= 1024 positions
            __syncthreads();
            for (int k2 = 2; k2 <= np2; k2 <<= 1)
                for (int j2 = k2 >> 1; j2 > 0; j2 >>= 1) {
                    const int i = tid, p = i ^ j2;
                    if (i < np2 && p > i) {
                        const int u = s_ord[i], v = s_ord[p];
                        // u before v: larger p first, then lower index; padding last
                        const float pu = u < m ? s_p[u] : -1.0f, pv = v < m ? s_p[v] : -1.0f;
                        const int iu = u < m ? s_idx[u] : 0x7FFFFFFF, iv = v < m ? s_idx[v] : 0x7FFFFFFF;
                        const bool u_first = pu > pv || (pu == pv && iu < iv);
                        const bool up = (i & k2) == 0;
                        if (u_first != up) { s_ord[i] = v; s_ord[p] = u; }
                    }
                    __syncthreads();
                }
            if (tid == 0) {
                float cum = 0.0f;
                int cut = m;
                for (int r = 0; r < m; ++r) {
                    cum += s_p[s_ord[r]];
                    if (cum >= c.top_p) { cut = r + 1; break; }
                }
                s_pick[0] = cut;
            }
            __syncthreads();
            if (tid < m && tid >= s_pick[0]) s_val[s_ord[tid]] = -INFINITY;
            __syncthreads();
        }
    }

    // ---- min-p: drop logits below max + ln(min_p)
    if (c.min_p > 0.0f) {
        const float mx = block_max1024(tid < m ? s_val[tid] : -INFINITY, s_red);
        const float th2 = mx + c.log_min_p;
        if (tid < m && s_val[tid] < th2) s_val[tid] = -INFINITY;
        __syncthreads();
    }

    // ---- softmax and the inverse CDF in index order (sample_from_probs)
    const float mx = block_max1024(tid < m ? s_val[tid] : -INFINITY, s_red);
    if (tid < m) s_p[tid] = sample_exp(s_val[tid] - mx);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int i = 0; i < m; ++i) sum += s_p[i];
        const float inv = 1.0f / sum;
        unsigned long long r = *a.rng;
        r ^= r << 13;
        r ^= r >> 7;
        r ^= r << 17;
        const float u = (float)(uint32_t)(r >> 33) / 2147483648.0f;
        float cum = 0.0f;
        uint32_t tok = (uint32_t)(n - 1);
        for (int i = 0; i < m; ++i) {
            const float p = s_p[i] * inv;
            cum += p;
            if (u < cum) { tok = (uint32_t)s_idx[i]; break; }
        }
        *a.rng = r;
        if (a.out_u32) *a.out_u32 = tok;
        if (a.record && a.hist && a.hist_len) { a.hist[len] = tok; *a.hist_len = len + 1; }
        if (a.step) *a.step = step + 1;
        if (a.pos_inc) *a.pos_inc += 1;
    }
}

int sample_launch(const SampleArgs& a, hipStream_t st) {
    ATLAS_REQUIRE(a.x && a.n > 0 && a.cfg && a.rng && a.out_u32, "sample: bad arguments");
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(1024), 0, st, a);
    ATLAS_LAUNCH_CHECK("sample");
    return ATLAS_OK;
}

// ---- embedding gather -----------------------------------------------------------
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ table, int vocab,
                                                    int d, const uint32_t* tok_dev, uint32_t tok,
                                                    float* __restrict__ out, long ld, RopeRowArgs r) {
    const int s = blockIdx.y;
    uint32_t t = tok_dev ? tok_dev[s] : tok;
    if (t >= (uint32_t)vocab) t = (uint32_t)vocab - 1;
    const uint16_t* row = table + (long)t * d;
    float* o = out + (long)s * ld;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < d; i += gridDim.x * 256)
        o[i] = __uint_as_float((uint32_t)row[i] << 16);
    // the step's RoPE row: cos then sin at the live position
    if (r.out && blockIdx.x == 0 && s == 0) {
        const long p = *r.pos_dev;
        for (int i = threadIdx.x; i < r.half; i += 256) {
            r.out[i] = r.cos_tab[p * r.half + i];
            r.out[r.half + i] = r.sin_tab[p * r.half + i];
        }
    }
}

int embed_launch(const uint16_t* table, int vocab, int d, const uint32_t* tok_dev, uint32_t tok,
                 float* out, long ld, int n_seq, hipStream_t st, const RopeRowArgs& rope) {
    ATLAS_REQUIRE(table && out && vocab > 0 && d > 0 && n_seq > 0, "embed: bad arguments");
    ATLAS_REQUIRE(!rope.out || (rope.pos_dev && rope.cos_tab && rope.sin_tab && rope.half > 0),
                  "embed: RoPE row needs the position and the tables");
    const int bx = (d + 255) / 256 < 16 ? (d + 255) / 256 : 16;
    hipLaunchKernelGGL(embed_kernel, dim3(bx, n_seq), dim3(256), 0, st, table, vocab, d, tok_dev, tok,
                       out, ld, rope);
    ATLAS_LAUNCH_CHECK("embed");
    return ATLAS_OK;
}

// ---- device counters ---------------------------------------------------------
__global__ void add_int_kernel(int* p, int n, int v) {
    const int i = threadIdx.x;
    if (i < n) p[i] += v;
}

int add_int_launch(int* p, int n, int v, hipStream_t st) {
    ATLAS_REQUIRE(p && n > 0 && n <= 1024, "add_int: bad arguments");
    hipLaunchKernelGGL(add_int_kernel, dim3(1), dim3(n <= 64 ? 64 : 1024), 0, st, p, n, v);
    ATLAS_LAUNCH_CHECK("add_int");
    return ATLAS_OK;
}

// ---- seeded initialisers (SplitMix64 counter + Box-Muller) ---------------------
__device__ __forceinline__ unsigned long long splitmix_at(unsigned long long seed,
                                                          unsigned long long n) {
    unsigned long long z = seed + (n + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__global__ void init_kernel(int kind, void* out, long n, unsigned long long seed, float a, float b) {
    for (long i = (blockIdx.x * 256L + threadIdx.x) * 2; i < n; i += (long)gridDim.x * 512) {
        float v0, v1;
        if (kind == INIT_UNIFORM_F32) {
            const double u0 = (double)(splitmix_at(seed, i) >> 11) * (1.0 / 9007199254740992.0);
            const double u1 = (double)(splitmix_at(seed, i + 1) >> 11) * (1.0 / 9007199254740992.0);
            v0 = (float)(a + (b - a) * u0);
            v1 = (float)(a + (b - a) * u1);
        } else {
            const double u1 = ((double)(splitmix_at(seed, i) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
            const double u2 = ((double)(splitmix_at(seed, i + 1) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
            const double r = sqrt(-2.0 * log(u1));
            const double t = 6.283185307179586476925286766559 * u2;
            v0 = (float)(a + b * r * cos(t));
            v1 = (float)(a + b * r * sin(t));
        }
        if (kind == INIT_NORMAL_BF16) {
            uint16_t* o = reinterpret_cast<uint16_t*>(out);
            o[i] = (uint16_t)(__float_as_uint(v0) >> 16);
            if (i + 1 < n) o[i + 1] = (uint16_t)(__float_as_uint(v1) >> 16);
        } else {
            float* o = reinterpret_cast<float*>(out);
            o[i] = v0;
            if (i + 1 < n) o[i + 1] = v1;
        }
    }
}

int init_launch(int kind, void* out, long n, unsigned long long seed, float a, float b,
                hipStream_t st) {
    ATLAS_REQUIRE(out && n >= 0, "init: bad arguments");
    if (n == 0) return ATLAS_OK;
    long blocks = (n / 2 + 255) / 256 + 1;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(init_kernel, dim3((unsigned)blocks), dim3(256), 0, st, kind, out, n, seed, a, b);
    ATLAS_LAUNCH_CHECK("init");
    return ATLAS_OK;
}

// ---- element conversions of the safetensors loader ------------------------------
// F16 -> F32 follows f16_to_f32 (crates/atlas-model/src/lib.rs:2243-2263): zero
// and subnormals as (mant / 1024) * 2^-14 (exact), exponent 31 as +-inf or the
// canonical quiet NaN, else the rebiased bits.  F32 -> BF16 truncates
// (bits >> 16, lib.rs:2274); BF16 -> F32 shifts (bits << 16).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    if (ex == 0) {
        const float m = (float)mant * 5.9604644775390625e-8f;     // mant * 2^-24
        return sign ? -m : m;
    }
    if (ex == 31) {
        if (mant) return __uint_as_float(0x7FC00000u);
        return __uint_as_float(sign ? 0xFF800000u : 0x7F800000u);
    }
    return __uint_as_float((sign << 31) | ((ex + 112u) << 23) | (mant << 13));
}

__global__ void cvt_kernel(int kind, const void* __restrict__ src, void* __restrict__ dst, long n) {
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        if (kind == CVT_F16_F32)
            reinterpret_cast<float*>(dst)[i] =
                f16_bits_to_f32(reinterpret_cast<const uint16_t*>(src)[i]);
        else if (kind == CVT_F32_BF16)
            reinterpret_cast<uint16_t*>(dst)[i] =
                (uint16_t)(reinterpret_cast<const uint32_t*>(src)[i] >> 16);
        else
            reinterpret_cast<uint32_t*>(dst)[i] =
                (uint32_t)reinterpret_cast<const uint16_t*>(src)[i] << 16;
    }
}

int cvt_launch(int kind, const void* src, void* dst, long n, hipStream_t st) {
    ATLAS_REQUIRE(src && dst && n >= 0 && kind >= CVT_F16_F32 && kind <= CVT_BF16_F32,
                  "convert: bad arguments");
    if (n == 0) return ATLAS_OK;
    long blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(cvt_kernel, dim3((unsigned)blocks), dim3(256), 0, st, kind, src, dst, n);
    ATLAS_LAUNCH_CHECK("convert");
    return ATLAS_OK;
}

// ---- device quantisers, bit-exact to crates/atlas-quant/src/lib.rs:43-145 -------
// Rust `(v * inv).clamp(lo, hi).round() as i8`: clamp, round half away from zero.
__device__ __forceinline__ int clamp_round(float v, float lo, float hi) {
    if (v != v) return 0;
    const float c = v < lo ? lo : (v > hi ? hi : v);
    return (int)roundf(c);
}

// source: f32 (src_bf16 == 0) or bf16 bits (src_bf16 == 1); one block per row
__global__ __launch_bounds__(256) void quant_i8_kernel(const void* src, int src_bf16, int cols,
                                                       int8_t* data, float* scales) {
    const long r = blockIdx.x;
    auto at = [&](long j) -> float {
        const long e = r * cols + j;
        return src_bf16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(src)[e] << 16)
                        : reinterpret_cast<const float*>(src)[e];
    };
    float mx = 0.f;
    for (int j = threadIdx.x; j < cols; j += 256) mx = fmaxf(mx, fabsf(at(j)));
    __shared__ float red[4];
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = mx > 0.f ? mx / 127.0f : 1.0f;
    const float inv = 1.0f / s;
    if (threadIdx.x == 0) scales[r] = s;
    for (int j = threadIdx.x; j < cols; j += 256)
        data[r * cols + j] = (int8_t)clamp_round(at(j) * inv, -127.f, 127.f);
}

// one wave per block of `block` elements of the flattened tensor
__global__ __launch_bounds__(256) void quant_i4_kernel(const void* src, int src_bf16, long n,
                                                       int block, uint8_t* data, float* scales,
                                                       long n_blocks) {
    const long b = blockIdx.x * 4L + (threadIdx.x >> 6);
    if (b >= n_blocks) return;
    const int lane = threadIdx.x & 63;
    const long start = b * block;
    const long end = start + block < n ? start + block : n;
    auto at = [&](long e) -> float {
        return src_bf16 ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(src)[e] << 16)
                        : reinterpret_cast<const float*>(src)[e];
    };
    float mx = 0.f;
    for (long e = start + lane; e < end; e += 64) mx = fmaxf(mx, fabsf(at(e)));
    mx = wave_max(mx);
    const float s = mx > 0.f ? mx / 7.0f : 1.0f;
    const float inv = 1.0f / s;
    if (lane == 0) scales[b] = s;
    // each lane packs whole bytes (element pairs); block starts are even when
    // block is even, so a byte never straddles two blocks
    for (long e = start + 2 * lane; e < end; e += 128) {
        const int q0 = clamp_round(at(e) * inv, -7.f, 7.f);
        const int q1 = e + 1 < end ? clamp_round(at(e + 1) * inv, -7.f, 7.f) : 0;
        data[e >> 1] = (uint8_t)(((q0 & 0x0F) << 4) | (q1 & 0x0F));
    }
}

int quant_i8_launch(const void* src, int src_bf16, int rows, int cols, int8_t* data, float* scales,
                    hipStream_t st) {
    ATLAS_REQUIRE(src && data && scales && rows >= 0 && cols > 0, "quant_i8: bad arguments");
    if (rows == 0) return ATLAS_OK;
    hipLaunchKernelGGL(quant_i8_kernel, dim3(rows), dim3(256), 0, st, src, src_bf16, cols, data, scales);
    ATLAS_LAUNCH_CHECK("quant_i8");
    return ATLAS_OK;
}

int quant_i4_launch(const void* src, int src_bf16, long n, int block, uint8_t* data, float* scales,
                    hipStream_t st) {
    ATLAS_REQUIRE(src && data && scales && n >= 0 && block > 0, "quant_i4: bad arguments");
    ATLAS_REQUIRE(block % 2 == 0, "quant_i4: device quantiser needs an even block size");
    if (n == 0) return ATLAS_OK;
    const long nb = (n + block - 1) / block;
    hipLaunchKernelGGL(quant_i4_kernel, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, st, src, src_bf16,
                       n, block, data, scales, nb);
    ATLAS_LAUNCH_CHECK("quant_i4");
    return ATLAS_OK;
}

}  // namespace atlas
