// capi.cpp -- the extern "C" kernel entry points declared in
// include/atlas_kernels.h (reference FFI names of
// crates/atlas-tensor/src/lib.rs:17-92, and the hot-path extensions).
#include <cmath>

#include "attention.hpp"
#include "common.hpp"
#include "fused.hpp"
#include "gemv.hpp"

using namespace atlas;

// ---- Part 1: reference FFI ------------------------------------------------------

static int gemm_dispatch(int fmt, const void* w, const float* b, float* c, int m, int n, int k) {
    ATLAS_REQUIRE(m >= 0 && n >= 0 && k >= 0, "gemm: negative shape");
    if (m == 0 || n == 0) return ATLAS_OK;
    if (n == 1) {
        GemvArgs a{};
        a.fmt = fmt; a.w = w; a.x = b; a.y = c; a.M = m; a.K = k; a.epi = EPI_STORE; a.N = 1;
        return gemv_launch(a, stream());
    }
    if (fmt == WF_BF16 && n <= 8 && k % 32 == 0) {
        // B is [k x n] row-major: activation j = column j (x stride n along k)
        GemvArgs a{};
        a.fmt = fmt; a.w = w; a.x = b; a.y = c; a.M = m; a.K = k; a.N = n; a.epi = EPI_STORE;
        a.x_stride_n = 1; a.x_stride_k = n;
        a.y_stride_n = 1; a.y_stride_m = n;
        return skinny_launch(a, stream());
    }
    return gemm_generic_launch(fmt, w, b, c, m, n, k, stream());
}

ATLAS_API void atlas_matmul_f32(const float* a, const float* b, float* c, int m, int n, int k) {
    gemm_dispatch(WF_F32, a, b, c, m, n, k);
}

ATLAS_API void atlas_sgemm_bf16_f32(const uint16_t* a, const float* b, float* c, int m, int n,
                                    int k) {
    gemm_dispatch(WF_BF16, a, b, c, m, n, k);
}

ATLAS_API void atlas_vec_add_f32(const float* a, const float* b, float* out, int n) {
    ew_launch(EW_ADD, a, b, out, 0.f, n, stream());
}

ATLAS_API void atlas_scale_f32(const float* x, float s, float* out, int n) {
    ew_launch(EW_SCALE, x, nullptr, out, s, n, stream());
}

ATLAS_API void atlas_relu_f32(const float* x, float* out, int n) {
    ew_launch(EW_RELU, x, nullptr, out, 0.f, n, stream());
}

ATLAS_API void atlas_softmax_f32(const float* x, float* out, int rows, int cols) {
    softmax_rows_launch(x, out, rows, cols, stream());
}

ATLAS_API void atlas_rmsnorm_f32(const float* x, const float* w, float* out, int n, float eps) {
    rmsnorm_launch(x, w, out, n, 1, n, eps, stream());
}

ATLAS_API void atlas_rope_apply_f32(float* x, int pos, int head_dim, float theta) {
    rope_apply_launch(x, pos, head_dim, theta, stream());
}

ATLAS_API void atlas_silu_mul_f32(const float* gate, const float* up, float* out, int n) {
    ew_launch(EW_SILU_MUL, gate, up, out, 0.f, n, stream());
}

ATLAS_API void atlas_vram_copy_f32(const float* src, float* dst, int n) {
    ew_launch(EW_COPY, src, nullptr, dst, 0.f, n, stream());
}

ATLAS_API void atlas_adamw_step(float* p, float* m, float* v, const float* g, float lr, float b1,
                                float b2, float eps, float wd, float bc1, float bc2, int n) {
    adamw_launch(p, m, v, g, lr, b1, b2, eps, wd, bc1, bc2, n, stream());
}

ATLAS_API void atlas_qk_norm_inplace(float* x, const float* w, int n_heads, int head_dim,
                                     float eps) {
    qk_norm_launch(x, w, n_heads, head_dim, eps, stream());
}

ATLAS_API void atlas_rope_precomputed(float* x, const float* c, const float* s, int n_heads,
                                      int head_dim, int pos, int max_seq) {
    rope_tab_launch(x, c, s, n_heads, head_dim, pos, max_seq, stream());
}

ATLAS_API void atlas_kv_cache_write(float* kc, float* vc, const float* nk, const float* nv,
                                    int pos, int n_kv, int hd) {
    kv_write_launch(kc, vc, nk, nv, pos, n_kv, hd, stream());
}

ATLAS_API void atlas_decode_attention(const float* q, const float* k_cache, const float* v_cache,
                                      float* out, int n_heads, int n_kv, int head_dim, int pos,
                                      float scale, int window) {
    AttnArgs a{};
    a.q = q; a.k_cache = k_cache; a.v_cache = v_cache; a.out = out;
    a.n_heads = n_heads; a.n_kv = n_kv; a.head_dim = head_dim;
    a.pos = pos; a.pos_dev = nullptr; a.scale = scale; a.window = window;
    a.max_rows = pos + 1;
    const int ctx = (window > 0 && pos + 1 > window) ? window : pos + 1;
    // Up to 8 splits (the fused kernel's rule) merge in the block that
    // finishes last, in one launch; past that the merge kernel's one block
    // per query head is faster than one merging block per KV head (MI355X,
    // GQA 32/8/128 at ctx 512 / 4096 / 16384: 8.95 vs 9.2, 16.7 vs 14.7,
    // 33.3 vs 30.6 us).  The merge counters are the calling thread's (zeroed
    // when allocated, left at zero by every launch).
    int n_splits = attn_fused_splits_for(n_kv, ctx);
    if (n_splits > 8) {
        n_splits = attn_pick_splits_unfused(n_kv, ctx);
    } else if (n_splits > 1) {
        void* cnt = nullptr;
        if (thread_scratch(SCR_ATTN_CNT, (size_t)n_kv * sizeof(int), &cnt, true)) return;
        a.counters = static_cast<int*>(cnt);
    }
    attn_launch(a, n_splits, stream());
}

ATLAS_API int atlas_decode_attention_noalloc(const float* q, const float* k_cache,
                                             const float* v_cache, float* out, int n_heads,
                                             int n_kv, int head_dim, int pos, float scale,
                                             int window) {
    ATLAS_REQUIRE(pos >= 0, "decode_attention_noalloc: pos < 0");
    AttnArgs a{};
    a.q = q; a.k_cache = k_cache; a.v_cache = v_cache; a.out = out;
    a.n_heads = n_heads; a.n_kv = n_kv; a.head_dim = head_dim;
    a.pos = pos; a.pos_dev = nullptr; a.scale = scale; a.window = window;
    a.max_rows = pos + 1;
    const int ctx = (window > 0 && pos + 1 > window) ? window : pos + 1;
    // the two-kernel split merge (no counters to keep in the fixed workspace)
    return attn_launch_noalloc(a, attn_pick_splits_unfused(n_kv, ctx), stream());
}

ATLAS_API int64_t atlas_decode_attention_noalloc_max_bytes(void) {
    return (int64_t)attn_noalloc_max_bytes();
}

// per-block argmax keys in the calling thread's scratch
static unsigned long long* argmax_scratch() {
    void* p = nullptr;
    if (thread_scratch(SCR_ARGMAX, ARGMAX_MAX_PARTS * sizeof(unsigned long long), &p)) return nullptr;
    return static_cast<unsigned long long*>(p);
}

ATLAS_API void atlas_gpu_argmax(const float* x, float* out_f32, int n) {
    ArgmaxArgs a{};
    a.x = const_cast<float*>(x); a.n = n; a.part = argmax_scratch(); a.out_f32 = out_f32;
    a.theta = 1.0f;
    if (a.part) argmax_launch(a, stream());
}

// ---- Part 3: extensions --------------------------------------------------------

ATLAS_API int atlas_gemv_f32(int fmt, const void* w, const float* scales, int block,
                             const float* x, float* y, int m, int k) {
    GemvArgs a{};
    a.fmt = fmt; a.w = w; a.scales = scales; a.block = block; a.x = x; a.y = y;
    a.M = m; a.K = k; a.epi = EPI_STORE; a.N = 1;
    return gemv_launch(a, stream());
}

ATLAS_API int atlas_gemv_bf16_f32(const uint16_t* w, const float* x, float* y, int m, int k) {
    return atlas_gemv_f32(ATLAS_W_BF16, w, nullptr, 0, x, y, m, k);
}

ATLAS_API int atlas_gemv_i8_f32(const int8_t* w, const float* scales, const float* x, float* y,
                                int m, int k) {
    return atlas_gemv_f32(ATLAS_W_INT8, w, scales, 0, x, y, m, k);
}

ATLAS_API int atlas_gemv_i4_f32(const uint8_t* w, const float* scales, int block, const float* x,
                                float* y, int m, int k) {
    return atlas_gemv_f32(ATLAS_W_INT4, w, scales, block, x, y, m, k);
}

ATLAS_API int atlas_gemv_fused_f32(int fmt, const void* w, const float* scales, int block,
                                   const float* x, float* yout, int m, int k, int pro,
                                   const float* y, const float* norm_w, float eps, float* x_out) {
    ATLAS_REQUIRE(pro >= PRO_X && pro <= PRO_SILU, "gemv_fused: prologue %d", pro);
    ATLAS_REQUIRE(pro != PRO_RESNORM || x_out, "gemv_fused: residual prologue needs x_out");
    GemvArgs a{};
    a.fmt = fmt; a.w = w; a.scales = scales; a.block = block; a.x = x; a.y = yout;
    a.M = m; a.K = k; a.epi = EPI_STORE; a.N = 1;
    a.pro = pro; a.pro_y = y; a.pro_w = norm_w; a.pro_eps = eps; a.pro_out = x_out;
    return gemv_launch(a, stream());
}

ATLAS_API int atlas_gemv_swiglu_f32(int fmt, const void* w, const float* scales, int block,
                                    const float* x, float* h_out, int h, int k) {
    GemvArgs a{};
    a.fmt = fmt; a.w = w; a.scales = scales; a.block = block; a.x = x; a.y = h_out;
    a.M = 2 * h; a.K = k; a.epi = EPI_SILU_MUL; a.N = 1;
    return gemv_launch(a, stream());
}

ATLAS_API int atlas_gemm_skinny_f32(int fmt, const void* w, const float* scales, int block,
                                    const float* x, float* y, int m, int n, int k) {
    GemvArgs a{};
    a.fmt = fmt; a.w = w; a.scales = scales; a.block = block; a.x = x; a.y = y;
    a.M = m; a.K = k; a.N = n; a.epi = EPI_STORE;
    a.x_stride_n = k; a.x_stride_k = 1; a.y_stride_n = m; a.y_stride_m = 1;
    return skinny_launch(a, stream());
}

ATLAS_API int atlas_gemm_skinny_swiglu_f32(int fmt, const void* w, const float* scales,
                                           int block, const float* x, float* h_out, int h, int n,
                                           int k) {
    ATLAS_REQUIRE(h >= 0, "gemm_skinny_swiglu: h < 0");
    GemvArgs a{};
    a.fmt = fmt; a.w = w; a.scales = scales; a.block = block; a.x = x; a.y = h_out;
    a.M = 2 * h; a.K = k; a.N = n; a.epi = EPI_SILU_MUL;
    a.x_stride_n = k; a.x_stride_k = 1; a.y_stride_n = h; a.y_stride_m = 1;
    return skinny_launch(a, stream());
}

ATLAS_API int atlas_rmsnorm_rows_f32(const float* x, const float* w, float* out, int n, int rows,
                                     float eps) {
    return rmsnorm_launch(x, w, out, n, rows, n, eps, stream());
}

ATLAS_API int atlas_residual_rmsnorm_f32(float* x, const float* y, const float* w, int n,
                                         int rows, float eps) {
    return residual_rmsnorm_launch(x, y, w, n, rows, n, eps, stream());
}

ATLAS_API int atlas_qkv_post_f32(float* qkv, const float* q_norm, const float* k_norm,
                                 float qk_eps, const float* cos_tab, const float* sin_tab,
                                 float* k_cache, float* v_cache, int n_heads, int n_kv,
                                 int head_dim, int pos) {
    ATLAS_REQUIRE(pos >= 0, "qkv_post: pos < 0");
    QkvPostArgs a{};
    a.qkv = qkv; a.qkv_stride = 0; a.q_norm = q_norm; a.k_norm = k_norm; a.qk_eps = qk_eps;
    a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.k_cache = k_cache; a.v_cache = v_cache;
    a.slot_stride = 0; a.slot_dev = nullptr; a.pos_dev = nullptr; a.pos = pos;
    a.n_heads = n_heads; a.n_kv = n_kv; a.head_dim = head_dim;
    return qkv_post_launch(a, 1, stream());
}

ATLAS_API int atlas_attention_fused_f32(const float* qkv, const float* q_norm,
                                        const float* k_norm, float qk_eps, const float* cos_tab,
                                        const float* sin_tab, float* k_cache, float* v_cache,
                                        float* out, int n_heads, int n_kv, int head_dim, int pos,
                                        float scale, int window, int n_splits,
                                        int min_chunk) {
    ATLAS_REQUIRE(pos >= 0, "attention_fused: pos < 0");
    ATLAS_REQUIRE(attn_fused_supported(n_heads, n_kv, head_dim), "attention_fused: shape");
    const int ctx = (window > 0 && pos + 1 > window) ? window : pos + 1;
    if (n_splits <= 0) n_splits = attn_pick_splits(n_kv, ctx);
    ATLAS_REQUIRE(n_splits <= 1024, "attention_fused: n_splits %d", n_splits);
    // the calling thread's scratch: position, merge counters (cleared when
    // grown; the kernel leaves them at zero), split partials
    void *d_pos = nullptr, *d_cnt = nullptr, *d_part_v = nullptr;
    const size_t need = (size_t)n_heads * n_splits * (head_dim + 2) * sizeof(float);
    int rc = thread_scratch(SCR_FUSED_POS, sizeof(int), &d_pos);
    if (!rc) rc = thread_scratch(SCR_FUSED_CNT, (size_t)n_kv * sizeof(int), &d_cnt, true);
    if (!rc) rc = thread_scratch(SCR_FUSED_PART, need, &d_part_v);
    if (rc) return rc;
    float* d_part = static_cast<float*>(d_part_v);
    ATLAS_HIP(hipMemcpyAsync(d_pos, &pos, sizeof(int), hipMemcpyHostToDevice, stream()));
    AttnFusedArgs a{};
    a.qkv = qkv; a.qkv_stride = 0; a.q_norm = q_norm; a.k_norm = k_norm; a.qk_eps = qk_eps;
    a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.k_cache = k_cache; a.v_cache = v_cache;
    a.slot_stride = 0; a.slot_dev = nullptr; a.pos_dev = static_cast<const int*>(d_pos);
    a.out = out; a.out_stride = 0;
    a.n_heads = n_heads; a.n_kv = n_kv; a.head_dim = head_dim; a.scale = scale; a.window = window;
    a.part_m = d_part;
    a.part_l = d_part + (size_t)n_heads * n_splits;
    a.part_o = d_part + (size_t)2 * n_heads * n_splits;
    a.counters = static_cast<int*>(d_cnt);
    a.min_chunk = min_chunk > 0 ? min_chunk : 0;
    a.max_rows = pos + 1;
    return attn_fused_launch(a, n_splits, 1, stream());
}

ATLAS_API int atlas_argmax_u32(const float* x, int n, uint32_t* out_idx) {
    ArgmaxArgs a{};
    a.x = const_cast<float*>(x); a.n = n; a.part = argmax_scratch(); a.out_u32 = out_idx;
    a.theta = 1.0f;
    if (!a.part) return ATLAS_ENOMEM;
    return argmax_launch(a, stream());
}

ATLAS_API int atlas_quantize_int8_dev(const void* src, int src_is_bf16, int rows, int cols,
                                      int8_t* data, float* scales) {
    return quant_i8_launch(src, src_is_bf16, rows, cols, data, scales, stream());
}

ATLAS_API int atlas_quantize_int4_dev(const void* src, int src_is_bf16, int64_t n, int block,
                                      uint8_t* data, float* scales) {
    return quant_i4_launch(src, src_is_bf16, (long)n, block, data, scales, stream());
}

ATLAS_API int atlas_fill_random(int kind, void* out, int64_t n, uint64_t seed, float a, float b) {
    ATLAS_REQUIRE(kind >= 0 && kind <= 2, "fill_random: kind %d", kind);
    return init_launch(kind, out, (long)n, (unsigned long long)seed, a, b, stream());
}

ATLAS_API int atlas_bench_stream_floor(const void* buf, int64_t buf_bytes, int64_t bytes_per_launch,
                                       int launches, int blocks_per_cu, float* us_per_launch) {
    return stream_floor_bench(buf, (long)buf_bytes, (long)bytes_per_launch, launches, blocks_per_cu,
                              us_per_launch, stream());
}

// ---- host quantisers (crates/atlas-quant/src/lib.rs:43-63, 113-145) --------------
// Same arithmetic as the Rust: scale = absmax / 127 (or 7), 1.0 for an
// all-zero row/block, value * (1/scale), clamp, round half away from zero.

static inline int rust_clamp_round(float v, float lo, float hi) {
    if (std::isnan(v)) return 0;
    const float c = v < lo ? lo : (v > hi ? hi : v);
    return (int)std::round(c);
}

static inline float rust_max(float a, float b) {
    if (std::isnan(a)) return b;
    if (std::isnan(b)) return a;
    return a > b ? a : b;
}

ATLAS_API int atlas_quantize_int8_host(const float* w, int64_t rows, int64_t cols, int8_t* data,
                                       float* scales) {
    ATLAS_REQUIRE(w && data && scales && rows >= 0 && cols >= 0, "quantize_int8_host: bad args");
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = w + r * cols;
        float mx = 0.0f;
        for (int64_t j = 0; j < cols; ++j) mx = rust_max(mx, std::fabs(row[j]));
        const float s = mx > 0.0f ? mx / 127.0f : 1.0f;
        scales[r] = s;
        const float inv = 1.0f / s;
        for (int64_t j = 0; j < cols; ++j)
            data[r * cols + j] = (int8_t)rust_clamp_round(row[j] * inv, -127.0f, 127.0f);
    }
    return ATLAS_OK;
}

ATLAS_API int atlas_quantize_int4_host(const float* w, int64_t rows, int64_t cols, int64_t block,
                                       uint8_t* data, float* scales) {
    ATLAS_REQUIRE(w && data && scales && rows >= 0 && cols >= 0 && block > 0,
                  "quantize_int4_host: bad args");
    const int64_t n = rows * cols;
    const int64_t nb = (n + block - 1) / block;
    for (int64_t i = 0; i < (n + 1) / 2; ++i) data[i] = 0;
    for (int64_t b = 0; b < nb; ++b) {
        const int64_t start = b * block, end = start + block < n ? start + block : n;
        float mx = 0.0f;
        for (int64_t i = start; i < end; ++i) mx = rust_max(mx, std::fabs(w[i]));
        const float s = mx > 0.0f ? mx / 7.0f : 1.0f;
        scales[b] = s;
        const float inv = 1.0f / s;
        for (int64_t i = start; i < end; ++i) {
            const int q = rust_clamp_round(w[i] * inv, -7.0f, 7.0f);
            const uint8_t nib = (uint8_t)(q & 0x0F);
            if (i % 2 == 0) data[i / 2] = (uint8_t)((data[i / 2] & 0x0F) | (nib << 4));
            else data[i / 2] = (uint8_t)((data[i / 2] & 0xF0) | nib);
        }
    }
    return ATLAS_OK;
}
