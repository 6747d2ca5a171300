// blas.cpp -- the bf16 and int8 prompt GEMMs (17..1024 activation rows)
// through hipBLASLt.
//
// Y[n, m] = sum_k W[m, k] X[n, k] with W [M x K] (row pitch ldw) and X f32, as
// the tiled kernel gemm_rows_kernel computes it (the prompt-chunk form of
// Linear::forward, crates/atlas-model/src/lib.rs:487-499):
//  * bf16 weights: X's rows are split into bf16 hi and lo rows
//    (split_rows_kernel, the tiled kernel's split), one library GEMM at f32
//    accumulation multiplies the weights with all 2N rows, and
//    combine_rows_kernel adds the hi and lo products;
//  * int8 weights (one f32 scale per row, crates/atlas-quant/src/lib.rs:43-80):
//    X's rows become three int8 digit rows each (digits_rows_kernel, 2^-22 of
//    the row's largest element), one int8 GEMM sums q * d exactly in int32
//    over all 3N rows, and combine_digits_kernel recombines the digits and
//    applies both scales.
// The weights stream once per chunk; the combine applies the store or SwiGLU
// epilogue.  A plain library GEMM: the hand-written kernel keeps int4 (block
// dequantisation fused) and every shape this path does not take.  A model
// creates this context only when ATLAS_PROMPT_BLAS=1 (engine.cpp); otherwise
// the hand-written kernel serves every prompt chunk.
//
// Layouts in the library's column-major terms: W is K x M with leading
// dimension ldw / element size and is transposed (op T), the split rows are
// K x cols, and D = W^T X' is M x cols (row j of the row-major view = product
// row j).
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "gemv.hpp"

namespace atlas {

namespace {

struct Plan {
    int fmt, M, K, lda, N2;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

void destroy_plan(Plan& p) {
    if (p.la) (void)hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) (void)hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) (void)hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
    p = Plan{};
}

constexpr size_t kWorkspace = 32u << 20;
constexpr size_t kMaxPlans = 64;

#define TRY_RC(expr)              \
    do {                          \
        const int rc_ = (expr);   \
        if (rc_) return rc_;      \
    } while (0)

}  // namespace

struct BlasRows {
    hipblasLtHandle_t h = nullptr;
    int max_n = 0, max_m = 0, max_k = 0;
    void* ws = nullptr;           // library workspace
    uint16_t* xs = nullptr;       // split rows: [2 max_n][max_k] bf16 or [3 max_n][max_k] int8
    float* d = nullptr;           // products: [2 max_n][max_m] f32 or [3 max_n][max_m] int32
    float* xscale = nullptr;      // int8 digits: [max_n] row scales
    std::vector<Plan> plans;
    size_t next = 0;              // plan slot reused once kMaxPlans are held
    std::mutex mu;
};

int blas_rows_create(BlasRows** out, int max_n, int max_m, int max_k) {
    ATLAS_REQUIRE(out && max_n > 0 && max_m > 0 && max_k > 0, "blas rows: bad arguments");
    *out = nullptr;
    BlasRows* b = new BlasRows();
    b->max_n = max_n;
    b->max_m = max_m;
    b->max_k = max_k;
    if (hipblasLtCreate(&b->h) != HIPBLAS_STATUS_SUCCESS) {
        delete b;
        set_error(ATLAS_EUNSUPPORTED, "blas rows: hipBLASLt handle creation failed");
        return ATLAS_EUNSUPPORTED;
    }
    if (dev_malloc(&b->ws, kWorkspace) != hipSuccess ||
        dev_malloc(&b->xs, (size_t)2 * max_n * max_k * sizeof(uint16_t)) != hipSuccess ||
        dev_malloc(&b->d, (size_t)3 * max_n * max_m * sizeof(float)) != hipSuccess ||
        dev_malloc(&b->xscale, (size_t)max_n * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        blas_rows_destroy(b);
        set_error(ATLAS_ENOMEM, "blas rows: staging buffers");
        return ATLAS_ENOMEM;
    }
    *out = b;
    return ATLAS_OK;
}

void blas_rows_destroy(BlasRows* b) {
    if (!b) return;
    for (Plan& p : b->plans) destroy_plan(p);
    if (b->ws) (void)hipFree(b->ws);
    if (b->xs) (void)hipFree(b->xs);
    if (b->d) (void)hipFree(b->d);
    if (b->xscale) (void)hipFree(b->xscale);
    if (b->h) (void)hipblasLtDestroy(b->h);
    delete b;
}

// alpha = 1, beta = 0 in the plan's scale type
struct Scalars {
    float f1 = 1.f, f0 = 0.f;
    int32_t i1 = 1, i0 = 0;
    const void* one(int fmt) const { return fmt == WF_I8 ? (const void*)&i1 : (const void*)&f1; }
    const void* zero(int fmt) const { return fmt == WF_I8 ? (const void*)&i0 : (const void*)&f0; }
};

// The plan of (format, M, K, lda, columns): descriptors and the fastest of the
// library's first candidates, timed once on the caller's stream with the
// caller's weights w (the prompt GEMMs run eagerly, never under capture).
// bf16: bf16 x bf16 -> f32 at f32 accumulation; int8: int8 x int8 -> int32.
static int get_plan(BlasRows* b, const void* w, int fmt, int M, int K, int lda, int N2,
                    hipStream_t st, Plan** out) {
    for (Plan& p : b->plans)
        if (p.fmt == fmt && p.M == M && p.K == K && p.lda == lda && p.N2 == N2) {
            *out = &p;
            return ATLAS_OK;
        }
    Plan p{};
    p.fmt = fmt; p.M = M; p.K = K; p.lda = lda; p.N2 = N2;
    const bool i8 = fmt == WF_I8;
    const hipDataType in_t = i8 ? HIP_R_8I : HIP_R_16BF, out_t = i8 ? HIP_R_32I : HIP_R_32F;
    bool ok = hipblasLtMatmulDescCreate(&p.desc, i8 ? HIPBLAS_COMPUTE_32I : HIPBLAS_COMPUTE_32F,
                                        i8 ? HIP_R_32I : HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
                   HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
                   HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.la, in_t, K, M, lda) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.lb, in_t, K, N2, K) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.lc, out_t, M, N2, M) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulPreference_t pref = nullptr;
    ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
    const uint64_t wsz = kWorkspace;
    ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                     &wsz, sizeof(wsz)) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulHeuristicResult_t res[8];
    int n_res = 0;
    ok = ok && hipblasLtMatmulAlgoGetHeuristic(b->h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 8, res,
                                               &n_res) == HIPBLAS_STATUS_SUCCESS &&
         n_res > 0;
    if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (!ok) {
        destroy_plan(p);
        set_error(ATLAS_EUNSUPPORTED, "blas rows: no hipBLASLt %s algorithm for %d x %d x %d",
                  i8 ? "int8" : "bf16", M, N2, K);
        return ATLAS_EUNSUPPORTED;
    }
    // time up to four candidates on the staging buffers (their contents are
    // overwritten by the real call that follows): two warm-up calls (the first
    // loads the candidate's kernels), then the fastest of five single calls
    int best = 0;
    if (n_res > 1) {
        constexpr int kRuns = 5;
        hipEvent_t ev[kRuns + 1] = {};
        bool ev_ok = true;
        for (hipEvent_t& e : ev) ev_ok = ev_ok && hipEventCreate(&e) == hipSuccess;
        if (!ev_ok) {
            for (hipEvent_t e : ev)
                if (e) (void)hipEventDestroy(e);
            (void)hipGetLastError();
            destroy_plan(p);
            set_error(ATLAS_EHIP, "blas rows: event creation failed");
            return ATLAS_EHIP;
        }
        const Scalars sc;
        float best_ms = -1.f;
        for (int i = 0; i < n_res && i < 4; ++i) {
            auto run = [&] {
                return hipblasLtMatmul(b->h, p.desc, sc.one(fmt), w, p.la, b->xs, p.lb, sc.zero(fmt),
                                       b->d, p.lc, b->d, p.lc, &res[i].algo, b->ws, kWorkspace,
                                       st) == HIPBLAS_STATUS_SUCCESS;
            };
            bool ok_i = run() && run();
            for (int r = 0; r < kRuns && ok_i; ++r) ok_i = hipEventRecord(ev[r], st) == hipSuccess && run();
            ok_i = ok_i && hipEventRecord(ev[kRuns], st) == hipSuccess &&
                   hipEventSynchronize(ev[kRuns]) == hipSuccess;
            float ms = 1e30f;
            for (int r = 0; r < kRuns && ok_i; ++r) {
                float t = 0.f;
                ok_i = hipEventElapsedTime(&t, ev[r], ev[r + 1]) == hipSuccess;
                ms = std::min(ms, t);
            }
            if (ok_i && (best_ms < 0.f || ms < best_ms)) {
                best_ms = ms;
                best = i;
            }
            (void)hipGetLastError();
        }
        for (hipEvent_t e : ev) (void)hipEventDestroy(e);
    }
    p.algo = res[best].algo;
    if (b->plans.size() < kMaxPlans) {
        b->plans.push_back(p);
        *out = &b->plans.back();
    } else {
        Plan& slot = b->plans[b->next++ % kMaxPlans];
        destroy_plan(slot);
        slot = p;
        *out = &slot;
    }
    return ATLAS_OK;
}

// D[0 .. cols) = W . xs[0 .. cols)^T for the split rows already in b->xs
// (2n bf16 rows or 3n int8 digit rows)
static int matmul(BlasRows* b, const GemvArgs& a, int n, hipStream_t st) {
    const int esz = a.fmt == WF_I8 ? 1 : 2, cols = (a.fmt == WF_I8 ? 3 : 2) * n;
    const long pitch = a.ldw > 0 ? a.ldw : (long)a.K * esz;
    ATLAS_REQUIRE(pitch % esz == 0 && pitch / esz >= a.K, "blas rows: row pitch %ld", pitch);
    Plan* p = nullptr;
    TRY_RC(get_plan(b, a.w, a.fmt, a.M, a.K, (int)(pitch / esz), cols, st, &p));
    const Scalars sc;
    if (hipblasLtMatmul(b->h, p->desc, sc.one(a.fmt), a.w, p->la, b->xs, p->lb, sc.zero(a.fmt), b->d,
                        p->lc, b->d, p->lc, &p->algo, b->ws, kWorkspace, st) != HIPBLAS_STATUS_SUCCESS) {
        (void)hipGetLastError();
        set_error(ATLAS_EHIP, "blas rows: hipBLASLt matmul failed (%d x %d x %d)", a.M, cols, a.K);
        return ATLAS_EHIP;
    }
    return ATLAS_OK;
}

int blas_rows_launch(BlasRows* b, const GemvArgs& a, hipStream_t st) {
    ATLAS_REQUIRE(b && (a.fmt == WF_BF16 || (a.fmt == WF_I8 && a.scales)) && a.N > 0 && a.M > 0 &&
                      a.K > 0,
                  "blas rows: bad arguments");
    ATLAS_REQUIRE(a.M <= b->max_m && a.K <= b->max_k, "blas rows: %d x %d beyond the staging buffers",
                  a.M, a.K);
    ATLAS_REQUIRE(a.x_stride_k == 1 && a.x_stride_n % 4 == 0 && ((uintptr_t)a.x & 15) == 0,
                  "blas rows: x rows must be contiguous and 16-byte aligned");
    std::lock_guard<std::mutex> lock(b->mu);     // one set of staging buffers
    for (int n0 = 0; n0 < a.N; n0 += b->max_n) {
        const int n = std::min(b->max_n, a.N - n0);
        const float* x = a.x + (long)n0 * a.x_stride_n;
        float* y = a.y + (long)n0 * a.y_stride_n;
        if (a.fmt == WF_I8) {
            TRY_RC(digits_rows_launch(x, a.x_stride_n, n, a.K, (int8_t*)b->xs, b->xscale, st));
            TRY_RC(matmul(b, a, n, st));
            TRY_RC(combine_digits_launch((const int*)b->d, n, a.M, a.scales, b->xscale, a.epi, y,
                                         a.y_stride_n, a.y_stride_m, st));
        } else {
            TRY_RC(split_rows_launch(x, a.x_stride_n, n, a.K, b->xs, st));
            TRY_RC(matmul(b, a, n, st));
            TRY_RC(combine_rows_launch(b->d, n, a.M, a.epi, y, a.y_stride_n, a.y_stride_m, st));
        }
    }
    return ATLAS_OK;
}

int blas_rows_gemm(BlasRows* b, const GemvArgs& a, int n, hipStream_t st) {
    ATLAS_REQUIRE(b && (a.fmt == WF_BF16 || a.fmt == WF_I8) && n > 0 && n <= b->max_n && a.M > 0 &&
                      a.K > 0,
                  "blas rows: bad arguments");
    ATLAS_REQUIRE(a.M <= b->max_m && a.K <= b->max_k, "blas rows: %d x %d beyond the staging buffers",
                  a.M, a.K);
    std::lock_guard<std::mutex> lock(b->mu);
    return matmul(b, a, n, st);
}

uint16_t* blas_rows_xs(BlasRows* b) { return b ? b->xs : nullptr; }
float* blas_rows_d(BlasRows* b) { return b ? b->d : nullptr; }
float* blas_rows_xscale(BlasRows* b) { return b ? b->xscale : nullptr; }
int blas_rows_max_n(const BlasRows* b) { return b ? b->max_n : 0; }

}  // namespace atlas
