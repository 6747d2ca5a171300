// skinny.hip -- small ragged batch GEMM Y[n, m] = sum_k W[m, k] X[n, k], 1 <= N <= 16.
//
// The reference has no batched decode (each sequence runs its own GEMV,
// crates/atlas-model/src/lib.rs:487-499).  With N decode rows packed
// together the weights are still read once, and the N products per weight
// go to the matrix cores: v_mfma_f32_16x16x32_bf16.
//
// MFMA operands (lane = 16 g + i, g = lane / 16):
//  * A = activations: lane (g, i) supplies k = 8g..8g+7 of a 32-k tile for
//    A-row i = 2s + part: sequence s split into a bf16 "hi" (truncation) and
//    "lo" (RNE of the exact remainder) part, so hi + lo carries 16
//    significant bits and the f32-accumulated product matches an f32 GEMV
//    to ~2^-16.  Rows i >= 2N are zero.
//  * B = weights: lane (g, n) supplies the same 8 k of weight row n, as
//    stored (bf16) or dequantised exactly to bf16 (int8 q and int4 16*q have
//    at most 8 significant bits).  An int4 tile is one 32-element scale
//    block of each row, so the block scale applies to the tile's product.
//  * D: lane (g, n) holds D[4g + v][n]: sequences 2g, 2g+1 of row n.
//  * N > 8: NA = 2 A tiles (sequences 0-7 and 8-15) share every B operand;
//    a wave then keeps half as many k tiles (KTW = SK_KTW / NA), so the A
//    operands fit the 128 VGPRs of a 1024-thread block, and K splits twice
//    as often.
//
// Work split: a 1024-thread block (16 waves) owns a K-slice of at most 128
// tiles (4096 k); wave w owns a fixed run of <= 8 of its tiles and keeps
// their A operands in registers, converted once.  The block walks 16-row
// weight tiles (persistent over the grid) with the next tile's weights in
// flight; the 16 waves' partial D meet in LDS (double-buffered, one barrier
// per tile) and 128 threads apply the epilogue.  K > 4096 splits K across
// blocks into fp32 partials summed by skinny_reduce_kernel in a fixed order.
//
// int4 with 2..8 rows takes skinny_i4d_kernel instead: weights go straight
// from HBM into registers (a lane-row transpose gives the B layout), every
// block's loads are in flight at once, and the nibbles become bf16 operands
// by masks alone, with an exact offset correction per tile.  bf16 and int8
// at 2..8 rows take skinny_lds_kernel (K <= 4096: GEMV-style row loads into
// an LDS tile) or skinny_d_kernel (K > 4096: the loads are the B operands).
#include <type_traits>

#include "common.hpp"
#include "gemv.hpp"

namespace atlas {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int SK_WAVES = 16;        // waves per block
constexpr int SK_KTW = 8;           // max 32-k tiles per wave
constexpr int SK_KT_BLOCK = SK_WAVES * SK_KTW;

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// bf16 bits (low 16) of the hi (part 0) or lo (part 1) component of v;
// branch-free (part differs between neighbouring lanes)
__device__ __forceinline__ uint32_t split_part(float v, bool lo) {
    const uint32_t u = __float_as_uint(v);
    const float hi = __uint_as_float(u & 0xFFFF0000u);
    const uint32_t lb = bf16_rne_bits(v - hi);
    return lo ? lb : (u >> 16);
}

__device__ __forceinline__ uint32_t pack2(uint32_t lo16, uint32_t hi16) {
    return (lo16 & 0xFFFFu) | (hi16 << 16);
}

// two f32 with <= 8 significant bits -> packed bf16 pair (a low), exact
__device__ __forceinline__ uint32_t pack_f32_pair(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// one lane's weights of one 32-k tile
template <int FMT> struct SkFrag;
template <> struct SkFrag<WF_BF16> { u32x4 w; };
template <> struct SkFrag<WF_I8>   { uint32_t w0, w1; };
template <> struct SkFrag<WF_I4>   { uint32_t w; float s; };

// A weight row's base addresses (data, and int4 block scales; K % block == 0
// so every row starts a block).
struct SkRow { const uint8_t* w; const float* s; };

template <int FMT>
__device__ __forceinline__ SkRow sk_row(const GemvArgs& a, int row) {
    SkRow r;
    constexpr int NUM = FMT == WF_BF16 ? 2 : 1, DEN = FMT == WF_I4 ? 2 : 1;
    r.w = reinterpret_cast<const uint8_t*>(a.w) + (long)row * (a.ldw > 0 ? a.ldw : (long)a.K * NUM / DEN);
    r.s = FMT == WF_I4 ? a.scales + (long)row * a.bpr : nullptr;
    return r;
}

// Plain (temporal) loads: one load instruction covers 16 rows x 64 / 32 / 16
// bytes, a part of each row's 128-byte line whose rest the next k tiles read
// a little later.  With the non-temporal hint the line did not stay in L2 for
// them and came from HBM once per part (the 128-row prompt GEMM moved 1.3x
// its algorithmic bytes for bf16 and 2.2x for int4); cached, each line is
// fetched once (prefill of 127 tokens: bf16 -3%, int8 -7%, int4 -17%).
// fragment of 32-k tile kt; cpb_shift: log2 of the int4 chunks per block
template <int FMT>
__device__ __forceinline__ void sk_load(const SkRow& r, int kt, int g, int cpb_shift,
                                        SkFrag<FMT>& f) {
    if constexpr (FMT == WF_BF16) {
        f.w = *reinterpret_cast<const u32x4*>(r.w + (kt * 32 + 8 * g) * 2);
    } else if constexpr (FMT == WF_I8) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = *reinterpret_cast<const u32x2*>(r.w + kt * 32 + 8 * g);
        f.w0 = v.x;
        f.w1 = v.y;
    } else {
        f.w = *reinterpret_cast<const uint32_t*>(r.w + kt * 16 + 4 * g);
        f.s = r.s[kt >> cpb_shift] * 0.0625f;        // the tile holds 16 * q
    }
}

template <int FMT>
__device__ __forceinline__ bf16x8 sk_operand(const SkFrag<FMT>& f) {
    u32x4 b;
    if constexpr (FMT == WF_BF16) {
        b = f.w;
    } else if constexpr (FMT == WF_I8) {
        b.x = pack_f32_pair(s8_at(f.w0, 0), s8_at(f.w0, 1));
        b.y = pack_f32_pair(s8_at(f.w0, 2), s8_at(f.w0, 3));
        b.z = pack_f32_pair(s8_at(f.w1, 0), s8_at(f.w1, 1));
        b.w = pack_f32_pair(s8_at(f.w1, 2), s8_at(f.w1, 3));
    } else {
        const uint32_t hi = f.w & 0xF0F0F0F0u;            // 16 * even elements
        const uint32_t lo = (f.w << 4) & 0xF0F0F0F0u;     // 16 * odd elements
        b.x = pack_f32_pair(s8_at(hi, 0), s8_at(lo, 0));
        b.y = pack_f32_pair(s8_at(hi, 1), s8_at(lo, 1));
        b.z = pack_f32_pair(s8_at(hi, 2), s8_at(lo, 2));
        b.w = pack_f32_pair(s8_at(hi, 3), s8_at(lo, 3));
    }
    return __builtin_bit_cast(bf16x8, b);
}

// grid (tile blocks, K splits); block 1024 threads.  partial: [splits][N][M]
// (used when gridDim.y > 1).  kt_split: 32-k tiles per K split (<= 128).
template <int FMT, int NA>
__global__ __launch_bounds__(1024) void skinny_kernel(GemvArgs a, float* __restrict__ partial,
                                                      int kt_split, int cpb_shift) {
    constexpr int KTW = SK_KTW / NA;                             // k tiles per wave
    const int lane = threadIdx.x & 63;
    // wave-uniform by construction; readfirstlane lets the compiler see it
    // (per-lane branches around the loads would serialise them)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int M = a.M, N = a.N;
    const int kt_total = a.K / 32;
    const int kt0 = blockIdx.y * kt_split;
    const int kt1 = min(kt_total, kt0 + kt_split);
    const int per = (kt1 - kt0 + SK_WAVES - 1) / SK_WAVES;      // <= KTW
    const int w0 = kt0 + wave * per;
    const int nkt = max(0, min(per, kt1 - w0));                  // wave-uniform
    const int n_tiles = (M + 15) / 16;
    const int step = gridDim.x;
    const int t0 = blockIdx.x;

    // ---- x of this lane's A operands (tile na: sequence 8 na + li / 2),
    // every load issued before the weights', so the conversion waits for x
    // alone (lanes of rows i >= 2N read sequence 0 and are zeroed at
    // conversion, so no lane-divergent branch separates the loads from their use)
    const int s = li >> 1;
    const bool lo = li & 1;
    // Every one of the KTW slots is loaded and multiplied (straight-line
    // code keeps the wait counts exact); slots j >= nkt re-read a valid tile
    // and get a zero A operand.
    auto ktile = [&](int j) { return min(w0 + j, kt1 - 1); };
    float xv[NA][KTW][8];
#pragma unroll
    for (int na = 0; na < NA; ++na) {
        const bool real = 8 * na + s < N;
        const float* xr = a.x + (real ? (long)(8 * na + s) * a.x_stride_n : 0);
        if (a.x_vec) {
#pragma unroll
            for (int j = 0; j < KTW; ++j) {
                const long k = (long)ktile(j) * 32 + 8 * g;
                const f32x4 p0 = *reinterpret_cast<const f32x4*>(xr + k);
                const f32x4 p1 = *reinterpret_cast<const f32x4*>(xr + k + 4);
                xv[na][j][0] = p0.x; xv[na][j][1] = p0.y; xv[na][j][2] = p0.z; xv[na][j][3] = p0.w;
                xv[na][j][4] = p1.x; xv[na][j][5] = p1.y; xv[na][j][6] = p1.z; xv[na][j][7] = p1.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < KTW; ++j) {
                const long k = (long)ktile(j) * 32 + 8 * g;
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[na][j][e] = xr[(k + e) * a.x_stride_k];
            }
        }
    }

    __builtin_amdgcn_sched_barrier(0);

    // ---- weights of the first tile (one buffer, refilled in place)
    SkFrag<FMT> cur[KTW];
    {
        const SkRow r = sk_row<FMT>(a, min(t0 * 16 + li, M - 1));
#pragma unroll
        for (int j = 0; j < KTW; ++j) sk_load<FMT>(r, ktile(j), g, cpb_shift, cur[j]);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- A operands, converted once (rows i >= 2N stay zero)
    bf16x8 A[NA][KTW];
#pragma unroll
    for (int na = 0; na < NA; ++na)
#pragma unroll
        for (int j = 0; j < KTW; ++j) {
            if (8 * na + s >= N || j >= nkt) {
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[na][j][e] = 0.f;
            }
            u32x4 xa;
            xa.x = pack2(split_part(xv[na][j][0], lo), split_part(xv[na][j][1], lo));
            xa.y = pack2(split_part(xv[na][j][2], lo), split_part(xv[na][j][3], lo));
            xa.z = pack2(split_part(xv[na][j][4], lo), split_part(xv[na][j][5], lo));
            xa.w = pack2(split_part(xv[na][j][6], lo), split_part(xv[na][j][7], lo));
            A[na][j] = __builtin_bit_cast(bf16x8, xa);
        }

    __shared__ f32x4 red[2][NA][SK_WAVES][64];
    const bool split_out = gridDim.y > 1;
    int buf = 0;
    const int my_tiles = t0 < n_tiles ? (n_tiles - 1 - t0) / step + 1 : 0;
    int t = t0;
    for (int i = 0; i < my_tiles; ++i, t += step) {      // block-uniform trip count
        const SkRow rn = sk_row<FMT>(a, min((t + step) * 16 + li, M - 1));
        f32x4 acc[NA];
#pragma unroll
        for (int na = 0; na < NA; ++na) acc[na] = f32x4{0.f, 0.f, 0.f, 0.f};
        // MFMAs over the tile; with REFILL each fragment's buffer takes the
        // next tile's fragment as soon as it has become an operand (two
        // straight-line versions keep the wait counts exact)
        auto body = [&](auto refill) {
#pragma unroll
            for (int j = 0; j < KTW; ++j) {
                bf16x8 B = sk_operand<FMT>(cur[j]);
                if constexpr (FMT == WF_BF16) asm volatile("" : "+v"(B));
                float sc = 1.0f;
                if constexpr (FMT == WF_I4) sc = cur[j].s;
                if constexpr (decltype(refill)::value) sk_load<FMT>(rn, ktile(j), g, cpb_shift, cur[j]);
#pragma unroll
                for (int na = 0; na < NA; ++na) {
                    if constexpr (FMT == WF_I4) {
                        const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            A[na][j], B, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        acc[na] += d * sc;
                    } else {
                        acc[na] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[na][j], B, acc[na], 0, 0, 0);
                    }
                }
            }
        };
        if (i + 1 < my_tiles) body(std::true_type{});
        else body(std::false_type{});
#pragma unroll
        for (int na = 0; na < NA; ++na) red[buf][na][wave][lane] = acc[na];
        __syncthreads();
        if (threadIdx.x < 128 * NA) {
            // thread (na, sp, l): sequence 8 na + 2 (l / 16) + sp of row 16 t + l % 16
            const int l = threadIdx.x & 63, sp = (threadIdx.x >> 6) & 1, na = threadIdx.x >> 7;
            const int sq = 8 * na + 2 * (l >> 4) + sp, row = t * 16 + (l & 15);
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < SK_WAVES; ++w) {
                const f32x4 pr = red[buf][na][w][l];
                v += sp ? pr.z + pr.w : pr.x + pr.y;
            }
            if constexpr (FMT == WF_I8) v *= a.scales[min(row, M - 1)];
            if (split_out) {
                if (sq < N && row < M) partial[((long)blockIdx.y * N + sq) * M + row] = v;
            } else if (a.epi == EPI_SILU_MUL) {
                // rows (2i, 2i+1) = (gate_i, up_i) sit in adjacent lanes
                const float up = __shfl_xor(v, 1, 64);
                if ((row & 1) == 0 && sq < N && row + 1 < M)
                    a.y[sq * a.y_stride_n + (long)(row >> 1) * a.y_stride_m] =
                        v / (1.0f + expf(-v)) * up;
            } else if (sq < N && row < M) {
                a.y[sq * a.y_stride_n + (long)row * a.y_stride_m] = v;
            }
        }
        buf ^= 1;
    }
}

// ---------------------------------------------------------------------------
// int4 variant: a 16-row weight tile reaches LDS through contiguous 16-byte
// loads (two tiles in flight in registers) -- the MFMA layout would read 4
// bytes per lane scattered over 16 rows and as many scale words.  Rows are
// padded by 16 bytes so the fragment reads (16 rows apart) hit distinct
// banks.  The A operands, the wave's K range and the reduction are those of
// skinny_kernel.
constexpr int SKI4_MAX_ROWB = 2048;     // packed bytes of a row's K slice (4096 k)

template <int PFN, int WAVES, int NA>
__global__ __launch_bounds__(64 * WAVES) void skinny_i4_kernel(GemvArgs a, float* __restrict__ partial,
                                                               int kt_split, int cpb_shift) {
    constexpr int KTW = SK_KT_BLOCK / WAVES / NA;                // 32-k tiles per wave
    constexpr int THREADS = 64 * WAVES;
    constexpr int NPC = 16 * (SKI4_MAX_ROWB / 16) / THREADS;     // pieces per thread
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int M = a.M, N = a.N;
    const int kt_total = a.K / 32;
    const int kt0 = blockIdx.y * kt_split;
    const int kt1 = min(kt_total, kt0 + kt_split);
    const int nks = kt1 - kt0;                                   // chunks of the slice
    const int per = (nks + WAVES - 1) / WAVES;
    const int w0 = wave * per;                                   // slice-relative
    const int nkt = max(0, min(per, nks - w0));
    const int n_tiles = (M + 15) / 16;
    const int step = gridDim.x;
    const int t0 = blockIdx.x;
    const int rowb = nks * 16;                                   // slice bytes per row
    constexpr int ROWP = SKI4_MAX_ROWB + 16;                     // padded LDS row
    // scale words of the slice per row (block index range)
    const int sb0 = kt0 >> cpb_shift;
    const int nsc = ((kt1 - 1) >> cpb_shift) - sb0 + 1;

    __shared__ __align__(16) uint8_t wt[2][16 * ROWP];           // 2 x 33 KB
    __shared__ __align__(16) float sct[2][16][SKI4_MAX_ROWB / 16 + 4];
    __shared__ f32x4 red[2][NA][WAVES][64];

    // ---- this thread's pieces of every tile (fixed): 16-byte data pieces
    // q = 0, 1 and scale words q = 0, 1 as (row in tile, byte/word column);
    // pieces past the tile re-read its last piece and are not stored
    const int dpr = rowb >> 4;                                   // 16-B pieces per row
    int drow[NPC], dcol[NPC], srow[NPC], scol[NPC];
    bool dok[NPC], sok[NPC];
#pragma unroll
    for (int q = 0; q < NPC; ++q) {
        const int pd = (int)threadIdx.x + THREADS * q, ps = pd;
        dok[q] = pd < 16 * dpr;
        sok[q] = ps < 16 * nsc;
        const int cd = min(pd, 16 * dpr - 1), cs = min(ps, 16 * nsc - 1);
        drow[q] = cd / dpr;
        dcol[q] = (cd % dpr) * 16;
        srow[q] = cs / nsc;
        scol[q] = cs % nsc;
    }
    struct Pf { u32x4 d[NPC]; float s[NPC]; };
    const uint8_t* wbase = reinterpret_cast<const uint8_t*>(a.w) + kt0 * 16;
    const long wstride = a.ldw > 0 ? a.ldw : a.K / 2;
    auto fetch = [&](int t, Pf& f) {
#pragma unroll
        for (int q = 0; q < NPC; ++q) {
            const int r = min(t * 16 + drow[q], M - 1);
            f.d[q] = ldg_stream(reinterpret_cast<const u32x4*>(wbase + (long)r * wstride + dcol[q]));
        }
#pragma unroll
        for (int q = 0; q < NPC; ++q) {
            const int r = min(t * 16 + srow[q], M - 1);
            f.s[q] = a.scales[(long)r * a.bpr + sb0 + scol[q]] * 0.0625f;
        }
    };
    auto stash = [&](const Pf& f, int b) {
#pragma unroll
        for (int q = 0; q < NPC; ++q)
            if (dok[q]) *reinterpret_cast<u32x4*>(&wt[b][drow[q] * ROWP + dcol[q]]) = f.d[q];
#pragma unroll
        for (int q = 0; q < NPC; ++q)
            if (sok[q]) sct[b][srow[q]][scol[q]] = f.s[q];
    };

    // ---- the first PFN tiles' weights, then x in two halves of four A
    // operands (the staging overlaps the weights' latency and holds 32 VGPRs
    // of x at a time)
    Pf pf[PFN];
#pragma unroll
    for (int p = 0; p < PFN; ++p) fetch(min(t0 + p * step, n_tiles - 1), pf[p]);
    __builtin_amdgcn_sched_barrier(0);
    const int s = li >> 1;
    const bool lo = li & 1;
    auto ktile = [&](int j) { return kt0 + min(w0 + j, nks - 1); };
    bf16x8 A[NA][KTW];
#pragma unroll
    for (int na = 0; na < NA; ++na) {
        const bool real = 8 * na + s < N;
        const float* xr = a.x + (real ? (long)(8 * na + s) * a.x_stride_n : 0);
#pragma unroll
        for (int h = 0; h < KTW; h += KTW / 2) {
            float xv[KTW / 2][8];
#pragma unroll
            for (int j = 0; j < KTW / 2; ++j) {
                const long k = (long)ktile(h + j) * 32 + 8 * g;
                if (a.x_vec) {
                    const f32x4 p0 = *reinterpret_cast<const f32x4*>(xr + k);
                    const f32x4 p1 = *reinterpret_cast<const f32x4*>(xr + k + 4);
                    xv[j][0] = p0.x; xv[j][1] = p0.y; xv[j][2] = p0.z; xv[j][3] = p0.w;
                    xv[j][4] = p1.x; xv[j][5] = p1.y; xv[j][6] = p1.z; xv[j][7] = p1.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xv[j][e] = xr[(k + e) * a.x_stride_k];
                }
            }
#pragma unroll
            for (int j = 0; j < KTW / 2; ++j) {
                if (!real || h + j >= nkt) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xv[j][e] = 0.f;
                }
                u32x4 xa;
                xa.x = pack2(split_part(xv[j][0], lo), split_part(xv[j][1], lo));
                xa.y = pack2(split_part(xv[j][2], lo), split_part(xv[j][3], lo));
                xa.z = pack2(split_part(xv[j][4], lo), split_part(xv[j][5], lo));
                xa.w = pack2(split_part(xv[j][6], lo), split_part(xv[j][7], lo));
                A[na][h + j] = __builtin_bit_cast(bf16x8, xa);
            }
        }
    }

    const bool split_out = gridDim.y > 1;
    const int my_tiles = t0 < n_tiles ? (n_tiles - 1 - t0) / step + 1 : 0;
    // the LDS buffer b = i & 1 holds tile i; registers pf[i % PFN] hold tile
    // i until stashed, then take tile i + PFN
    auto tile = [&](int i, Pf& f) {
        const int t = t0 + i * step, b = i & 1;
        stash(f, b);
        if (i + PFN < my_tiles) fetch(t0 + (i + PFN) * step, f);
        __syncthreads();
        f32x4 acc[NA];
#pragma unroll
        for (int na = 0; na < NA; ++na) acc[na] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KTW; ++j) {
            const int c = min(w0 + j, nks - 1);                 // slice chunk
            const uint32_t w = *reinterpret_cast<const uint32_t*>(&wt[b][li * ROWP + c * 16 + 4 * g]);
            const float sc = sct[b][li][((kt0 + c) >> cpb_shift) - sb0];
            const uint32_t hi = w & 0xF0F0F0F0u;
            const uint32_t lw = (w << 4) & 0xF0F0F0F0u;
            u32x4 bb;
            bb.x = pack_f32_pair(s8_at(hi, 0), s8_at(lw, 0));
            bb.y = pack_f32_pair(s8_at(hi, 1), s8_at(lw, 1));
            bb.z = pack_f32_pair(s8_at(hi, 2), s8_at(lw, 2));
            bb.w = pack_f32_pair(s8_at(hi, 3), s8_at(lw, 3));
#pragma unroll
            for (int na = 0; na < NA; ++na) {
                const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    A[na][j], __builtin_bit_cast(bf16x8, bb), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                acc[na] += d * sc;
            }
        }
#pragma unroll
        for (int na = 0; na < NA; ++na) red[b][na][wave][lane] = acc[na];
        __syncthreads();
        if (threadIdx.x < 128 * NA) {
            const int l = threadIdx.x & 63, sp = (threadIdx.x >> 6) & 1, na = threadIdx.x >> 7;
            const int sq = 8 * na + 2 * (l >> 4) + sp, row = t * 16 + (l & 15);
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const f32x4 pr = red[b][na][w][l];
                v += sp ? pr.z + pr.w : pr.x + pr.y;
            }
            if (split_out) {
                if (sq < N && row < M) partial[((long)blockIdx.y * N + sq) * M + row] = v;
            } else if (a.epi == EPI_SILU_MUL) {
                const float up = __shfl_xor(v, 1, 64);
                if ((row & 1) == 0 && sq < N && row + 1 < M)
                    a.y[sq * a.y_stride_n + (long)(row >> 1) * a.y_stride_m] =
                        v / (1.0f + expf(-v)) * up;
            } else if (sq < N && row < M) {
                a.y[sq * a.y_stride_n + (long)row * a.y_stride_m] = v;
            }
        }
    };
    int i = 0;
    for (; i + PFN <= my_tiles; i += PFN) {
#pragma unroll
        for (int p = 0; p < PFN; ++p) tile(i + p, pf[p]);
    }
#pragma unroll
    for (int p = 0; p < PFN - 1; ++p)
        if (i + p < my_tiles) tile(i + p, pf[p]);
}

// ---------------------------------------------------------------------------
// int4, N <= 8 rows, weights straight from HBM into registers.  A block owns
// R <= RM 16-row groups (blockIdx.x + r * gridDim.x) of one K slice; wave w
// owns the slice's 32-k tiles 8w .. 8w+7 as two 4-tile chunks, so each
// (group, chunk) item is one 16-byte load per lane -- lane (j, n) takes tile
// 4c + j of row n -- plus the row's scales of those four tiles.  All items
// but the last U - 1 are in flight at once (x is issued before them), and a
// 4 x 4 transpose across 16-lane rows turns lane (g, n)'s register j into
// word g of tile 4c + j, the MFMA B operand; weights touch no LDS and the
// waves meet once, to add their k partials.
//
// A operands: lanes 2s and 2s + 1 (sequence s, hi and lo bf16 parts) each
// read four of the eight x values of a k group, split them into hi and lo,
// and trade halves through a lane swap.
//
// B operands without conversions: a weight word (elements e0..e7, e_2b in
// the high nibble of byte b) gives four bf16 pairs by one mask and XOR each
// (plus three shifts).  With m = s ^ 8 = q + 8 for the stored nibble s of
// the signed value q, (w & 0x000F000F) ^ 0x43084308 is (128 + m) for e1 and
// e5, the same of w >> 8 for e3 and e7, and ((w >> 1) & 0x00780078) ^
// 0x41C041C0 is (16 + m) for e0 and e4 (w >> 9: e2, e6) -- every value an
// exact bf16.  So the k slots of a lane hold e1 e5 e3 e7 e0 e4 e2 e6 (the A
// operands are built in that order) with offsets 136 on the first four and
// 24 on the last four: a tile's product is sum_k A q + corr(i), where
// corr(i) = sum_k off_k A(i, k) is one MFMA of the offsets against the A
// operand (as B); the scaled corrections of a chunk's four tiles are then
// one f32 MFMA (k = tile) subtracted from the accumulator.

// afterwards register j of 16-lane row g holds what register g of row j held
__device__ __forceinline__ void rows_transpose4(uint32_t& r0, uint32_t& r1, uint32_t& r2,
                                                uint32_t& r3) {
    const auto p02 = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
    const auto p13 = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
    const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
    const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
    r0 = q01[0];
    r1 = q01[1];
    r2 = q23[0];
    r3 = q23[1];
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// packed bf16 of (a, b): hi = truncation, lo = the rounded remainder
__device__ __forceinline__ uint32_t bf16_hi2(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}
__device__ __forceinline__ uint32_t bf16_lo2(float a, float b) {
    const float ra = a - __uint_as_float(__float_as_uint(a) & 0xFFFF0000u);
    const float rb = b - __uint_as_float(__float_as_uint(b) & 0xFFFF0000u);
    const bf16x2 v = {(__bf16)ra, (__bf16)rb};
    return __builtin_bit_cast(uint32_t, v);
}

constexpr int SKD_KTW = 8;          // 32-k tiles per wave

template <int RM, int U, bool SV>
__global__ __launch_bounds__(1024) void skinny_i4d_kernel(GemvArgs a, float* __restrict__ partial,
                                                          int kt_split, int cpb_shift) {
    constexpr int NI = 2 * RM;                                  // items (group, chunk)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int M = a.M, N = a.N;
    const int kt_total = a.K / 32;
    const int kt0 = blockIdx.y * kt_split;
    const int nks = min(kt_total, kt0 + kt_split) - kt0;       // tiles of the slice (<= 128)
    const int tw0 = wave * SKD_KTW;
    const int ntw = max(0, min(SKD_KTW, nks - tw0));           // this wave's tiles (uniform)
    const int n_groups = (M + 15) / 16;
    const int gx = __builtin_amdgcn_readfirstlane((int)gridDim.x), bx = blockIdx.x;
    const int R = bx < n_groups ? (n_groups - 1 - bx) / gx + 1 : 0;
    __shared__ f32x4 red[RM][16][64];

    // ---- x: lane (g, i), sequence s = i / 2, reads k = 8g + 4p .. + 3 (p = i & 1)
    // of each of the wave's tiles (tiles past the slice read its last one);
    // rows of sequences past N read sequence 0: they only reach D rows that
    // are never stored
    const int s = li >> 1, p = li & 1;
    const float* xr = a.x + (s < N ? (long)s * a.x_stride_n : 0);
    f32x4 xv[SKD_KTW];
#pragma unroll
    for (int j = 0; j < SKD_KTW; ++j) {
        const long k = (long)(kt0 + min(tw0 + j, nks - 1)) * 32 + 8 * g + 4 * p;
        if (a.x_vec) {
            xv[j] = *reinterpret_cast<const f32x4*>(xr + k);
        } else {
            xv[j] = f32x4{xr[k * a.x_stride_k], xr[(k + 1) * a.x_stride_k], xr[(k + 2) * a.x_stride_k],
                          xr[(k + 3) * a.x_stride_k]};
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- weights: item q = (group r = q / 2, chunk c = q % 2); past R the
    // last group is re-read and not used.  The group's scales come with its
    // chunk-0 item: lane (g, n) takes the four of chunk g & 1 (row n).
    // buffer resources over the whole matrix and its scales (both < 2 GB:
    // the launcher checks), 32-bit offsets
    const uint32_t wstride = a.ldw > 0 ? (uint32_t)a.ldw : (uint32_t)a.K / 2;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a.w), (short)0, __builtin_amdgcn_readfirstlane((int)(M * wstride)), 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a.scales), (short)0, __builtin_amdgcn_readfirstlane(M * a.bpr * 4), 0x00020000);
    auto load = [&](int q, u32x4& w, f32x4& sc) {
        const int r = min(q >> 1, max(R - 1, 0)), c = q & 1;
        const uint32_t row = (uint32_t)min((bx + r * gx) * 16 + li, M - 1);
        const int kt = kt0 + min(tw0 + 4 * c + g, nks - 1);
        // cached (policy 0): the two halves of each row's 128-byte line come
        // from two items of the wave, and a non-temporal first half made the
        // second fetch the line again
        w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          wres, (int)(row * wstride + (uint32_t)kt * 16u), 0, 0));
        if (c == 0) {
            const uint32_t so = row * (uint32_t)a.bpr;
            if constexpr (SV) {                                 // nks % 4 == 0, one scale per tile
                sc = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    sres, (int)((so + kt0 + min(tw0 + 4 * (g & 1), nks - 4)) * 4u), 0, 0));
            } else {
                const int kc = kt0 + min(tw0 + 4 * (g & 1), nks - 1), kl = kt0 + nks - 1;
                const float* sr = a.scales + so;
                sc = f32x4{sr[min(kc, kl) >> cpb_shift], sr[min(kc + 1, kl) >> cpb_shift],
                           sr[min(kc + 2, kl) >> cpb_shift], sr[min(kc + 3, kl) >> cpb_shift]};
            }
        }
    };
    if (ntw == 0) {                                             // a wave past the slice
#pragma unroll
        for (int r = 0; r < RM; ++r) red[r][wave][lane] = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
    u32x4 wb[U];
    f32x4 sb[(U + 1) / 2];
#pragma unroll
    for (int u = 0; u < U; ++u) load(u, wb[u], sb[(u >> 1) % ((U + 1) / 2)]);
    __builtin_amdgcn_sched_barrier(0);

    // ---- A operands from x (zero on tiles past the slice), k slots in the
    // B operands' order e1 e5 e3 e7 e0 e4 e2 e6
    bf16x8 A[SKD_KTW];
    // perm(own, other) selectors: lane 2s owns e0..e3 (bytes 4-7 of the
    // pair), lane 2s + 1 owns e4..e7
    const uint32_t sel_odd = p ? 0x07060302u : 0x03020706u;    // (e1, e5), (e3, e7)
    const uint32_t sel_even = p ? 0x05040100u : 0x01000504u;   // (e0, e4), (e2, e6)
#pragma unroll
    for (int j = 0; j < SKD_KTW; ++j) {
        f32x4 v = xv[j];
        if (j >= ntw) v = f32x4{0.f, 0.f, 0.f, 0.f};             // uniform
        const uint32_t h0 = bf16_hi2(v.x, v.y), h1 = bf16_hi2(v.z, v.w);
        const uint32_t l0 = bf16_lo2(v.x, v.y), l1 = bf16_lo2(v.z, v.w);
        // lane 2s keeps hi of its four and gets hi of the other four; lane
        // 2s + 1 the lo parts (DPP quad_perm [1, 0, 3, 2]: the pair swaps)
        const uint32_t o0 = p ? l0 : h0, o1 = p ? l1 : h1;
        const uint32_t t0 = __builtin_amdgcn_update_dpp(0u, p ? h0 : l0, 0xB1, 0xF, 0xF, false);
        const uint32_t t1 = __builtin_amdgcn_update_dpp(0u, p ? h1 : l1, 0xB1, 0xF, 0xF, false);
        u32x4 o;
        o.x = __builtin_amdgcn_perm(o0, t0, sel_odd);
        o.y = __builtin_amdgcn_perm(o1, t1, sel_odd);
        o.z = __builtin_amdgcn_perm(o0, t0, sel_even);
        o.w = __builtin_amdgcn_perm(o1, t1, sel_even);
        A[j] = __builtin_bit_cast(bf16x8, o);
    }
    // ---- offset corrections: lane (g, i) holds -corr of tile 4c + g, row i
    float corr[2];
    {
        const bf16x8 offs = __builtin_bit_cast(bf16x8, u32x4{0x43084308u, 0x43084308u, 0x41C041C0u,
                                                                0x41C041C0u});
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            float cg[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                cg[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(offs, A[4 * c + j],
                                                                f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0)[0];
            const float c01 = (g & 1) ? cg[1] : cg[0], c23 = (g & 1) ? cg[3] : cg[2];
            corr[c] = -((g & 2) ? c23 : c01);
        }
    }

    // ---- items in order; the group's partial goes to LDS after its chunk 1
    constexpr int NS = (U + 1) / 2;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float sj1[4];                                               // chunk 1's scales
#pragma unroll
    for (int q = 0; q < NI; ++q) {
        const int u = q % U;
        const u32x4 w = wb[u];
        float sj[4];
        const int c = q & 1;
        if (c == 0) {
            // rows g & 1 == 0 hold chunk 0's scales, the odd rows chunk 1's:
            // one 16-lane row swap gives every lane both
            const f32x4 sc = sb[(q >> 1) % NS];
            const float sv[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const auto e = __builtin_amdgcn_permlane16_swap(__float_as_uint(sv[j]),
                                                                __float_as_uint(sv[j]), false, false);
                sj[j] = __uint_as_float(e[0]);
                sj1[j] = __uint_as_float(e[1]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) sj[j] = sj1[j];
        }
        if (q + U < NI) load(q + U, wb[u], sb[((q + U) >> 1) % NS]);
        // no branches: A is zero on tiles past the slice, and groups past R
        // (re-read copies) are computed but never stored
        uint32_t wj[4] = {w.x, w.y, w.z, w.w};
        rows_transpose4(wj[0], wj[1], wj[2], wj[3]);
        f32x4 d[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t w = wj[j], w8 = w >> 8;
            const u32x4 b = {(w & 0x000F000Fu) ^ 0x43084308u, (w8 & 0x000F000Fu) ^ 0x43084308u,
                             ((w >> 1) & 0x00780078u) ^ 0x41C041C0u,
                             ((w >> 9) & 0x00780078u) ^ 0x41C041C0u};
            d[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[4 * c + j], __builtin_bit_cast(bf16x8, b),
                                                           f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc += d[j] * sj[j];
        // minus sum over the four tiles of corr(tile, i) * scale(tile, n)
        const float s01 = (g & 1) ? sj[1] : sj[0], s23 = (g & 1) ? sj[3] : sj[2];
        const float sg = (g & 2) ? s23 : s01;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(corr[c], sg, acc, 0, 0, 0);
        if (c == 1) {
            red[q >> 1][wave][lane] = acc;
            acc = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    }
    __syncthreads();

    // ---- thread (r, h, l): group r, lane l's D rows 2h, 2h + 1 (sequence
    // 2 (l / 16) + h: hi + lo) of weight row l % 16
    const bool split_out = gridDim.y > 1;
    for (int t = threadIdx.x; t < RM * 128; t += 1024) {
        const int r = t >> 7, h = (t >> 6) & 1, l = t & 63;
        float v = 0.f;
        if (r < R) {
#pragma unroll
            for (int w = 0; w < 16; ++w) {
                const f32x4 pr = red[r][w][l];
                v += h ? pr.z + pr.w : pr.x + pr.y;
            }
        }
        const int sq = 2 * (l >> 4) + h;
        const int row = (bx + r * gx) * 16 + (l & 15);
        const float up = __shfl_xor(v, 1, 64);                  // rows (2i, 2i + 1): (gate, up)
        if (r >= R || sq >= N) continue;
        if (split_out) {
            if (row < M) partial[((long)blockIdx.y * N + sq) * M + row] = v;
        } else if (a.epi == EPI_SILU_MUL) {
            if ((row & 1) == 0 && row + 1 < M)
                a.y[sq * a.y_stride_n + (long)(row >> 1) * a.y_stride_m] = v / (1.0f + expf(-v)) * up;
        } else if (row < M) {
            a.y[sq * a.y_stride_n + (long)row * a.y_stride_m] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// bf16 / int8 with N <= 8 rows, the same direct-load scheme without the int4
// layout work: a bf16 lane load (16 bytes = k 8g..8g+7 of one 32-k tile of
// row n) already is the MFMA B operand, and an int8 lane load (16 bytes, k
// 16g..16g+15 of a 64-k pair of tiles) is two B operands once converted --
// any k order inside an MFMA is fine when the scale is per row, so the A
// operands simply follow the loads.  The products accumulate in the MFMA
// itself (two accumulators alternate); int8's row scale applies in the
// epilogue.  Block / wave / group split, x handling and the epilogue are
// those of skinny_i4d_kernel.

// A operand of a lane pair from its four x values (lane 2s: k 0..3 of the
// group, hi parts; lane 2s + 1: k 4..7, lo parts), natural k order
__device__ __forceinline__ bf16x8 pair_operand(const f32x4 v, bool p) {
    const uint32_t h0 = bf16_hi2(v.x, v.y), h1 = bf16_hi2(v.z, v.w);
    const uint32_t l0 = bf16_lo2(v.x, v.y), l1 = bf16_lo2(v.z, v.w);
    const uint32_t t0 = __builtin_amdgcn_update_dpp(0u, p ? h0 : l0, 0xB1, 0xF, 0xF, false);
    const uint32_t t1 = __builtin_amdgcn_update_dpp(0u, p ? h1 : l1, 0xB1, 0xF, 0xF, false);
    u32x4 o;
    o.x = p ? t0 : h0;
    o.y = p ? t1 : h1;
    o.z = p ? l0 : t0;
    o.w = p ? l1 : t1;
    return __builtin_bit_cast(bf16x8, o);
}

template <int FMT, int RM, int U>
__global__ __launch_bounds__(1024) void skinny_d_kernel(GemvArgs a, float* __restrict__ partial,
                                                        int kt_split) {
    static_assert(FMT == WF_BF16 || FMT == WF_I8, "bf16 or int8");
    constexpr int IPG = FMT == WF_BF16 ? 8 : 4;                 // lane loads per group
    constexpr int NI = RM * IPG;
    constexpr int EB = FMT == WF_BF16 ? 2 : 1;                  // bytes per weight
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int M = a.M, N = a.N;
    const int kt_total = a.K / 32;
    const int kt0 = blockIdx.y * kt_split;
    const int nks = min(kt_total, kt0 + kt_split) - kt0;       // tiles of the slice (% 4 == 0)
    const int tw0 = wave * SKD_KTW;
    const int ntw = max(0, min(SKD_KTW, nks - tw0));           // 0, 4 or 8 (uniform)
    const int n_groups = (M + 15) / 16;
    const int gx = __builtin_amdgcn_readfirstlane((int)gridDim.x), bx = blockIdx.x;
    const int R = bx < n_groups ? (n_groups - 1 - bx) / gx + 1 : 0;
    __shared__ f32x4 red[RM][16][64];

    // slice-relative k of this lane's first x value for MFMA t (0..7)
    const int s = li >> 1, p = li & 1;
    auto kofs = [&](int t) {
        if constexpr (FMT == WF_BF16) return min(tw0 + t, nks - 1) * 32 + 8 * g + 4 * p;
        else return min(tw0 + 2 * (t >> 1), nks - 2) * 32 + 16 * g + 8 * (t & 1) + 4 * p;
    };
    const float* xr = a.x + (s < N ? (long)s * a.x_stride_n : 0);   // rows past N: never stored
    f32x4 xv[SKD_KTW];
#pragma unroll
    for (int t = 0; t < SKD_KTW; ++t) {
        const long k = (long)kt0 * 32 + kofs(t);
        if (a.x_vec) {
            xv[t] = *reinterpret_cast<const f32x4*>(xr + k);
        } else {
            xv[t] = f32x4{xr[k * a.x_stride_k], xr[(k + 1) * a.x_stride_k], xr[(k + 2) * a.x_stride_k],
                          xr[(k + 3) * a.x_stride_k]};
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    const uint32_t wstride = a.ldw > 0 ? (uint32_t)a.ldw : (uint32_t)a.K * EB;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a.w), (short)0, __builtin_amdgcn_readfirstlane((int)(M * wstride)), 0x00020000);
    // item q = (group r = q / IPG, load j = q % IPG)
    auto load = [&](int q) {
        const int r = min(q / IPG, max(R - 1, 0)), j = q % IPG;
        const uint32_t row = (uint32_t)min((bx + r * gx) * 16 + li, M - 1);
        uint32_t off;
        if constexpr (FMT == WF_BF16) off = (uint32_t)(kt0 + min(tw0 + j, nks - 1)) * 64u + 16u * g;
        else off = (uint32_t)(kt0 + min(tw0 + 2 * j, nks - 2)) * 32u + 16u * g;
        // cached, as in skinny_i4d_kernel: a load covers 16 rows x 64 bytes
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             wres, (int)(row * wstride + off), 0, 0));
    };
    if (ntw == 0) {                                             // a wave past the slice
#pragma unroll
        for (int r = 0; r < RM; ++r) red[r][wave][lane] = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
    u32x4 wb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) wb[u] = load(u);
    __builtin_amdgcn_sched_barrier(0);

    bf16x8 A[SKD_KTW];
#pragma unroll
    for (int t = 0; t < SKD_KTW; ++t) {
        f32x4 v = xv[t];
        if (FMT == WF_BF16 ? t >= ntw : 2 * (t >> 1) >= ntw) v = f32x4{0.f, 0.f, 0.f, 0.f};
        A[t] = pair_operand(v, p);
    }

    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NI; ++q) {
        const int u = q % U, j = q % IPG;
        const u32x4 w = wb[u];
        if (q + U < NI) wb[u] = load(q + U);
        if constexpr (FMT == WF_BF16) {
            if (j & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j], __builtin_bit_cast(bf16x8, w), acc1, 0, 0, 0);
            else acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[j], __builtin_bit_cast(bf16x8, w), acc0, 0, 0, 0);
        } else {
            SkFrag<WF_I8> f0, f1;
            f0.w0 = w.x; f0.w1 = w.y; f1.w0 = w.z; f1.w1 = w.w;
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2 * j], sk_operand<WF_I8>(f0), acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2 * j + 1], sk_operand<WF_I8>(f1), acc1, 0, 0, 0);
        }
        if (j == IPG - 1) {
            red[q / IPG][wave][lane] = acc0 + acc1;
            acc0 = f32x4{0.f, 0.f, 0.f, 0.f};
            acc1 = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    }
    __syncthreads();

    const bool split_out = gridDim.y > 1;
    for (int t = threadIdx.x; t < RM * 128; t += 1024) {
        const int r = t >> 7, h = (t >> 6) & 1, l = t & 63;
        const int sq = 2 * (l >> 4) + h;
        const int row = (bx + r * gx) * 16 + (l & 15);
        float v = 0.f;
        if (r < R) {
#pragma unroll
            for (int w = 0; w < 16; ++w) {
                const f32x4 pr = red[r][w][l];
                v += h ? pr.z + pr.w : pr.x + pr.y;
            }
            if constexpr (FMT == WF_I8) v *= a.scales[min(row, M - 1)];
        }
        const float up = __shfl_xor(v, 1, 64);                  // rows (2i, 2i + 1): (gate, up)
        if (r >= R || sq >= N) continue;
        if (split_out) {
            if (row < M) partial[((long)blockIdx.y * N + sq) * M + row] = v;
        } else if (a.epi == EPI_SILU_MUL) {
            if ((row & 1) == 0 && row + 1 < M)
                a.y[sq * a.y_stride_n + (long)(row >> 1) * a.y_stride_m] = v / (1.0f + expf(-v)) * up;
        } else if (row < M) {
            a.y[sq * a.y_stride_n + (long)row * a.y_stride_m] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// bf16 / int8 with N <= 8 rows and K <= 4096 through LDS: the block loads a
// 16-row group the way the batch-1 GEMV does (each wave instruction reads
// 1 KB of one row), with PF groups in flight in registers, stores it in LDS
// (rows padded by 16 bytes: the B reads of 16 rows at one offset fall on
// distinct banks) and reads the MFMA B operands from there.  The direct-load
// kernel's 16-rows x 64-byte instructions stream at ~4.5 TB/s at these
// shapes; these run at the GEMV's rate.  x, A operands and the epilogue are
// those of skinny_d_kernel; one barrier pair and one reduction per group.
// (Two groups in flight need more than 128 VGPRs for bf16 and spill for
// int8, so the launcher takes PF = 1.)
constexpr int SKL_ROWB = 8192;                  // bytes of a row (K <= 4096 bf16)
constexpr int SKL_ROWP = SKL_ROWB + 16;         // padded LDS row

template <int FMT, int PF>
__global__ __launch_bounds__(1024) void skinny_lds_kernel(GemvArgs a) {
    static_assert(FMT == WF_BF16 || FMT == WF_I8, "bf16 or int8");
    constexpr int EB = FMT == WF_BF16 ? 2 : 1;                  // bytes per weight
    constexpr int NPC = 16 * (SKL_ROWB / (2 / EB)) / 16 / 1024; // pieces per thread per group
    constexpr int ROWP = SKL_ROWB / (2 / EB) + 16;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int M = a.M, N = a.N;
    const int nks = a.K / 32;                                  // tiles (<= 128)
    const int tw0 = wave * SKD_KTW;
    const int ntw = max(0, min(SKD_KTW, nks - tw0));
    const int n_groups = (M + 15) / 16;
    const int gx = __builtin_amdgcn_readfirstlane((int)gridDim.x), bx = blockIdx.x;
    const int R = bx < n_groups ? (n_groups - 1 - bx) / gx + 1 : 0;
    const int dpr = nks * 2 * EB;                              // 16-byte pieces per row
    __shared__ __align__(16) uint8_t wt[16 * ROWP];
    __shared__ f32x4 red[16][64];

    // A operands of the wave's 8 tiles (natural k order; zero past K)
    const int s = li >> 1, p = li & 1;
    const float* xr = a.x + (s < N ? (long)s * a.x_stride_n : 0);   // rows past N: never stored
    bf16x8 A[SKD_KTW];
    {
        f32x4 xv[SKD_KTW];
#pragma unroll
        for (int t = 0; t < SKD_KTW; ++t) {
            const long k = (long)min(tw0 + t, nks - 1) * 32 + 8 * g + 4 * p;
            if (a.x_vec) {
                xv[t] = *reinterpret_cast<const f32x4*>(xr + k);
            } else {
                xv[t] = f32x4{xr[k * a.x_stride_k], xr[(k + 1) * a.x_stride_k],
                              xr[(k + 2) * a.x_stride_k], xr[(k + 3) * a.x_stride_k]};
            }
        }
#pragma unroll
        for (int t = 0; t < SKD_KTW; ++t) {
            f32x4 v = xv[t];
            if (t >= ntw) v = f32x4{0.f, 0.f, 0.f, 0.f};
            A[t] = pair_operand(v, p);
        }
    }

    const uint32_t wstride = a.ldw > 0 ? (uint32_t)a.ldw : (uint32_t)a.K * EB;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a.w), (short)0, __builtin_amdgcn_readfirstlane((int)(M * wstride)), 0x00020000);
    // piece q of this thread in a group: (row pc / dpr, 16-byte column pc % dpr);
    // past the group's pieces, or past R, a copy is read and not stored
    auto fetch = [&](int r, u32x4 (&f)[NPC]) {
        const int grp = bx + min(r, max(R - 1, 0)) * gx;
#pragma unroll
        for (int q = 0; q < NPC; ++q) {
            const int pc = min((int)threadIdx.x + 1024 * q, 16 * dpr - 1);
            const uint32_t row = (uint32_t)min(grp * 16 + pc / dpr, M - 1);
            f[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 wres, (int)(row * wstride + (uint32_t)(pc % dpr) * 16u), 0, 2));
        }
    };
    u32x4 pf[PF][NPC];
#pragma unroll
    for (int i = 0; i < PF; ++i) fetch(i, pf[i]);
    for (int r0 = 0; r0 < R; r0 += PF) {                       // block-uniform
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            const int r = r0 + i;
            if (r >= R) break;
            __syncthreads();                                   // the last group's B reads are done
#pragma unroll
            for (int q = 0; q < NPC; ++q) {
                const int pc = (int)threadIdx.x + 1024 * q;
                if (pc < 16 * dpr)
                    *reinterpret_cast<u32x4*>(&wt[(pc / dpr) * ROWP + (pc % dpr) * 16]) = pf[i][q];
            }
            if (r + PF < R) fetch(r + PF, pf[i]);
            __syncthreads();
            f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < SKD_KTW; ++t) {
                const int kt = min(tw0 + t, nks - 1);
                bf16x8 b;
                if constexpr (FMT == WF_BF16) {
                    b = *reinterpret_cast<const bf16x8*>(&wt[li * ROWP + kt * 64 + 16 * g]);
                } else {
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    const u32x2 w2 = *reinterpret_cast<const u32x2*>(&wt[li * ROWP + kt * 32 + 8 * g]);
                    SkFrag<WF_I8> f;
                    f.w0 = w2.x;
                    f.w1 = w2.y;
                    b = sk_operand<WF_I8>(f);
                }
                if (t & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t], b, acc1, 0, 0, 0);
                else acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[t], b, acc0, 0, 0, 0);
            }
            red[wave][lane] = acc0 + acc1;
            __syncthreads();
            if (threadIdx.x < 128) {
                const int h = threadIdx.x >> 6, l = threadIdx.x & 63;
                const int sq = 2 * (l >> 4) + h;
                const int row = (bx + r * gx) * 16 + (l & 15);
                float v = 0.f;
#pragma unroll
                for (int w = 0; w < 16; ++w) {
                    const f32x4 pr = red[w][l];
                    v += h ? pr.z + pr.w : pr.x + pr.y;
                }
                if constexpr (FMT == WF_I8) v *= a.scales[min(row, M - 1)];
                const float up = __shfl_xor(v, 1, 64);         // rows (2i, 2i + 1): (gate, up)
                if (sq < N) {
                    if (a.epi == EPI_SILU_MUL) {
                        if ((row & 1) == 0 && row + 1 < M)
                            a.y[sq * a.y_stride_n + (long)(row >> 1) * a.y_stride_m] =
                                v / (1.0f + expf(-v)) * up;
                    } else if (row < M) {
                        a.y[sq * a.y_stride_n + (long)row * a.y_stride_m] = v;
                    }
                }
            }
        }
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

int skinny_reduce_launch(const GemvArgs& a, const float* partial, int splits, hipStream_t st) {
    ATLAS_REQUIRE(partial && a.y && a.N > 0 && a.M > 0 && splits > 0, "skinny reduce: bad arguments");
    const long m_out = a.epi == EPI_SILU_MUL ? a.M / 2 : a.M;
    long rb = ((long)a.N * m_out + 255) / 256;
    if (rb > 4096) rb = 4096;
    hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, a, partial, splits);
    ATLAS_LAUNCH_CHECK("skinny_reduce");
    return ATLAS_OK;
}

// The caller takes the split-K sum over (GemvArgs.defer_splits): plain
// stores into its own partial buffer only.
static bool defer_ok(const GemvArgs& a) {
    return a.defer_splits && a.epi == EPI_STORE && a.partial && a.y_stride_m == 1 &&
           a.y_stride_n == a.M;
}

// Split-K partials: the caller's buffer (GemvArgs.partial, e.g. a model's,
// which a captured step may point at) or the calling thread's scratch.
static int partial_for(const GemvArgs& a, size_t bytes, float** out) {
    if (a.partial) {
        ATLAS_REQUIRE(bytes <= a.partial_bytes, "split-K partials: %zu bytes needed, %zu given",
                      bytes, a.partial_bytes);
        *out = a.partial;
        return ATLAS_OK;
    }
    void* p = nullptr;
    const int rc = thread_scratch(SCR_GEMM, bytes, &p);
    *out = static_cast<float*>(p);
    return rc;
}

// A tiles of an N-row launch, and the K splits it uses (a block covers
// SK_KT_BLOCK / NA k tiles)
static int skinny_na(int N) { return N > 8 ? 2 : 1; }
static int skinny_splits(int K, int N) {
    const int kt_total = K / 32, kt_block = SK_KT_BLOCK / skinny_na(N);
    return (kt_total + kt_block - 1) / kt_block;
}

// blocks of 1024 threads one CU holds for kernel `kern` (cached per kernel)
template <const void* (*KERN)()>
static int skinny_resident() {
    static int resident = 0;
    if (resident == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, KERN(), 1024, 0) != hipSuccess || n < 1) {
            (void)hipGetLastError();
            n = 1;
        }
        resident = n;
    }
    return resident;
}

template <int FMT, int NA>
static const void* skinny_kernel_ptr() {
    if constexpr (FMT == WF_I4) return (const void*)skinny_i4_kernel<1, 16, NA>;
    else return (const void*)skinny_kernel<FMT, NA>;
}

template <int FMT, int NA>
static int launch_skinny(const GemvArgs& a, hipStream_t st) {
    const int kt_total = a.K / 32;
    const int splits = skinny_splits(a.K, a.N);
    const int kt_split = (kt_total + splits - 1) / splits;
    const int n_tiles = (a.M + 15) / 16;
    int bx = skinny_resident<skinny_kernel_ptr<FMT, NA>>() * device_cu_count();
    if (bx > n_tiles) bx = n_tiles;
    float* partial = nullptr;
    if (splits > 1) {
        int rc = partial_for(a, (size_t)splits * a.N * a.M * sizeof(float), &partial);
        if (rc) return rc;
    }
    int cpb_shift = 0;
    while ((1 << cpb_shift) < a.cpb) ++cpb_shift;
    if constexpr (FMT == WF_I4)
        hipLaunchKernelGGL((skinny_i4_kernel<1, 16, NA>), dim3(bx, splits), dim3(1024), 0, st, a,
                           partial, kt_split, cpb_shift);
    else
        hipLaunchKernelGGL((skinny_kernel<FMT, NA>), dim3(bx, splits), dim3(1024), 0, st, a,
                           partial, kt_split, cpb_shift);
    ATLAS_LAUNCH_CHECK("skinny");
    if (splits > 1) {
        const long m_out = a.epi == EPI_SILU_MUL ? a.M / 2 : a.M;
        long rb = ((long)a.N * m_out + 255) / 256;
        if (rb > 4096) rb = 4096;
        hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, a,
                           partial, splits);
        ATLAS_LAUNCH_CHECK("skinny_reduce");
    }
    return ATLAS_OK;
}

// int4 with N <= 8 rows through skinny_i4d_kernel: a block per CU holding
// RM <= 8 groups of 16 rows (a larger M takes more blocks than CUs), K in
// slices of <= 128 tiles over blockIdx.y (a multiple of 4 tiles, so the
// slices' scales load as 16-byte vectors when a block covers one tile).
// Returns 1 when the shape does not fit (the caller takes skinny_i4_kernel).
// K splits: the fewest whose grid (one block per CU) gives the smallest
// per-block load (groups x tiles); a matrix too large for 8 groups per block
// on every CU takes more blocks than CUs
struct I4dPlan { int splits, kt_split, bx, rm; };
static I4dPlan i4d_plan(int M, int K, int cus) {
    const int kt_total = K / 32;
    const int n_groups = (M + 15) / 16;
    const int s_min = (kt_total + SK_KT_BLOCK - 1) / SK_KT_BLOCK;
    I4dPlan p{0, 0, 0, 0};
    long best = 0;
    for (int sp = s_min; sp <= s_min + 3; ++sp) {
        const int ks = ((kt_total + sp - 1) / sp + 3) & ~3;
        if (ks > SK_KT_BLOCK || (kt_total + ks - 1) / ks != sp) continue;   // an empty split
        const int b = std::min(n_groups, std::max(1, cus / sp));
        const int r = (n_groups + b - 1) / b;
        if (r > 8) continue;
        const long cost = (long)r * ks;
        if (p.splits == 0 || cost < best) {
            p = I4dPlan{sp, ks, b, r};
            best = cost;
        }
    }
    if (p.splits == 0) {
        p.splits = s_min;
        p.kt_split = ((kt_total + s_min - 1) / s_min + 3) & ~3;
        p.rm = 8;
        p.bx = (n_groups + 7) / 8;
    }
    return p;
}

// Bytes of split-K partials an (M, N, K) launch needs; an N-row size
// covers every smaller N.
size_t skinny_partial_bytes(int M, int N, int K) {
    int splits = skinny_splits(K, N);
    if (N > 8) splits = std::max(splits, skinny_splits(K, 8));
    else splits = std::max(splits, i4d_plan(M, K, device_cu_count()).splits);   // int4 rows
    if (splits <= 1) return 0;
    return (size_t)splits * N * M * sizeof(float);
}

template <int RM, int U>
static void i4d_go(const GemvArgs& a, bool sv, dim3 grid, hipStream_t st, float* partial, int kt_split,
                   int cpb_shift) {
    if (sv)
        hipLaunchKernelGGL((skinny_i4d_kernel<RM, U, true>), grid, dim3(1024), 0, st, a, partial,
                           kt_split, cpb_shift);
    else
        hipLaunchKernelGGL((skinny_i4d_kernel<RM, U, false>), grid, dim3(1024), 0, st, a, partial,
                           kt_split, cpb_shift);
}

static int launch_skinny_i4d(const GemvArgs& a, hipStream_t st) {
    const long wstride = a.ldw > 0 ? a.ldw : a.K / 2;
    if (a.N > 8 || ((uintptr_t)a.w & 15) || (wstride & 15) || (long)a.M * wstride >= (1L << 31) ||
        (long)a.M * a.bpr * 4 >= (1L << 31))
        return 1;
    const int kt_total = a.K / 32;
    const I4dPlan pl = i4d_plan(a.M, a.K, device_cu_count());
    const int splits = pl.splits, kt_split = pl.kt_split, bx = pl.bx, rm = pl.rm;
    const bool sv = a.cpb == 1 && a.bpr % 4 == 0 && kt_total % 4 == 0 && ((uintptr_t)a.scales & 15) == 0;
    float* partial = nullptr;
    if (splits > 1) {
        const int rc = partial_for(a, (size_t)splits * a.N * a.M * sizeof(float), &partial);
        if (rc) return rc;
    }
    int cpb_shift = 0;
    while ((1 << cpb_shift) < a.cpb) ++cpb_shift;
    const dim3 grid(bx, splits);
    switch (rm) {
    case 1: i4d_go<1, 2>(a, sv, grid, st, partial, kt_split, cpb_shift); break;
    case 2: i4d_go<2, 4>(a, sv, grid, st, partial, kt_split, cpb_shift); break;
    case 3: i4d_go<3, 6>(a, sv, grid, st, partial, kt_split, cpb_shift); break;
    case 4: i4d_go<4, 4>(a, sv, grid, st, partial, kt_split, cpb_shift); break;
    case 5: case 6: i4d_go<6, 4>(a, sv, grid, st, partial, kt_split, cpb_shift); break;
    default: i4d_go<8, 4>(a, sv, grid, st, partial, kt_split, cpb_shift); break;
    }
    ATLAS_LAUNCH_CHECK("skinny int4");
    if (splits > 1 && defer_ok(a)) {
        *a.defer_splits = splits;
        return ATLAS_OK;
    }
    if (splits > 1) {
        const long m_out = a.epi == EPI_SILU_MUL ? a.M / 2 : a.M;
        long rb = ((long)a.N * m_out + 255) / 256;
        if (rb > 4096) rb = 4096;
        hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, a, partial,
                           splits);
        ATLAS_LAUNCH_CHECK("skinny_reduce");
    }
    return ATLAS_OK;
}

// bf16 / int8 with N <= 8 rows through skinny_d_kernel, with the int4
// launcher's K splits and groups per block (K % 128 == 0: slices of whole
// 4-tile steps).  Returns 1 when the shape does not fit.
template <int FMT, int RM, int U>
static void d_go(const GemvArgs& a, dim3 grid, hipStream_t st, float* partial, int kt_split) {
    hipLaunchKernelGGL((skinny_d_kernel<FMT, RM, U>), grid, dim3(1024), 0, st, a, partial, kt_split);
}

template <int FMT>
static int launch_skinny_d(const GemvArgs& a, hipStream_t st) {
    constexpr long EB = FMT == WF_BF16 ? 2 : 1;
    const long wstride = a.ldw > 0 ? a.ldw : (long)a.K * EB;
    if (a.N > 8 || a.K % 128 || ((uintptr_t)a.w & 15) || (wstride & 15) ||
        (long)a.M * wstride >= (1L << 31))
        return 1;
    const I4dPlan pl = i4d_plan(a.M, a.K, device_cu_count());
    float* partial = nullptr;
    if (pl.splits > 1) {
        const int rc = partial_for(a, (size_t)pl.splits * a.N * a.M * sizeof(float), &partial);
        if (rc) return rc;
    }
    const dim3 grid(pl.bx, pl.splits);
    switch (pl.rm) {
    case 1: d_go<FMT, 1, FMT == WF_BF16 ? 8 : 4>(a, grid, st, partial, pl.kt_split); break;
    case 2: d_go<FMT, 2, 8>(a, grid, st, partial, pl.kt_split); break;
    case 3: d_go<FMT, 3, 8>(a, grid, st, partial, pl.kt_split); break;
    case 4: d_go<FMT, 4, 8>(a, grid, st, partial, pl.kt_split); break;
    case 5: case 6: d_go<FMT, 6, 8>(a, grid, st, partial, pl.kt_split); break;
    default: d_go<FMT, 8, 8>(a, grid, st, partial, pl.kt_split); break;
    }
    ATLAS_LAUNCH_CHECK(FMT == WF_BF16 ? "skinny bf16" : "skinny int8");
    if (pl.splits > 1 && defer_ok(a)) {
        *a.defer_splits = pl.splits;
        return ATLAS_OK;
    }
    if (pl.splits > 1) {
        const long m_out = a.epi == EPI_SILU_MUL ? a.M / 2 : a.M;
        long rb = ((long)a.N * m_out + 255) / 256;
        if (rb > 4096) rb = 4096;
        hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, a, partial,
                           pl.splits);
        ATLAS_LAUNCH_CHECK("skinny_reduce");
    }
    return ATLAS_OK;
}

// bf16 / int8 with N <= 8 rows and K <= 4096 through skinny_lds_kernel: one
// block of 1024 threads per CU (the LDS row tile), persistent over the
// 16-row groups.  Returns 1 when the shape does not fit.
template <int FMT>
static int launch_skinny_lds(const GemvArgs& a, hipStream_t st) {
    constexpr long EB = FMT == WF_BF16 ? 2 : 1;
    const long wstride = a.ldw > 0 ? a.ldw : (long)a.K * EB;
    if (a.N > 8 || a.K > 4096 || ((uintptr_t)a.w & 15) || (wstride & 15) ||
        (long)a.M * wstride >= (1L << 31))
        return 1;
    const int n_groups = (a.M + 15) / 16;
    const int bx = std::min(n_groups, device_cu_count());
    hipLaunchKernelGGL((skinny_lds_kernel<FMT, 1>), dim3(bx), dim3(1024), 0, st, a);
    ATLAS_LAUNCH_CHECK(FMT == WF_BF16 ? "skinny lds bf16" : "skinny lds int8");
    return ATLAS_OK;
}

// ---------------------------------------------------------------------------
// Prompt chunks: Y[n, m] = sum_k W[m, k] X[n, k] for 17 <= N <= 128 rows of
// bf16, int8 or int4 weights (dequantised to exact bf16 operands as in
// skinny_kernel: int8 row scales in the epilogue, int4 block scales on each
// 32-k step's product).  Same operand roles and hi/lo split as skinny_kernel, but
// every A fragment now feeds many weight tiles, so the matrix cores do the
// work and the weights stream once per chunk:
//  * a 256-thread block owns 128 weight rows (wave w: rows 32 w .. +31, two
//    B fragments per 32-k step) and all NT 16-row tiles of X;
//  * A fragments (X hi and lo, bf16) go through LDS, 2 k steps per chunk,
//    double-buffered: each chunk's global reads are issued one chunk ahead
//    and converted after the MFMAs of the current one;
//  * B fragments (16 B per lane, straight from HBM) are refilled in place
//    four k steps ahead, as soon as each has become an operand;
//  * K splits over blockIdx.y when the row blocks alone leave CUs idle;
//    partials are summed by skinny_reduce_kernel in a fixed order.
// Per 32-k step a wave issues NT x 2 x 2 MFMAs (tiles x B fragments x hi/lo).
constexpr int GR_ROWS = 128;        // weight rows per block
constexpr int GR_MAX_N = 128;       // activation rows per launch
// (k step, tile) items whose A fragments are read ahead of the current one
constexpr int GR_AHEAD = 4;

// hi / lo bf16 parts of 8 floats, packed as MFMA operands: hi = the high
// halves (truncation), lo = the remainder rounded to nearest even (one
// hardware conversion per pair)
__device__ __forceinline__ void split8(const f32x4 p0, const f32x4 p1, u32x4& hi, u32x4& lo) {
    hi = u32x4{bf16_hi2(p0.x, p0.y), bf16_hi2(p0.z, p0.w), bf16_hi2(p1.x, p1.y), bf16_hi2(p1.z, p1.w)};
    lo = u32x4{bf16_lo2(p0.x, p0.y), bf16_lo2(p0.z, p0.w), bf16_lo2(p1.x, p1.y), bf16_lo2(p1.z, p1.w)};
}

// int4 at eight tiles runs one block per CU: its per-step scaled products
// need ~370 registers (spilled 27 at two blocks per CU), and one 128-row
// launch that streams the weights once beats two 64-row launches that
// stream them twice (127-token int4 prefill 14.1 -> 12.6 ms)
template <int FMT, int NT>
__global__ __launch_bounds__(256, (FMT == WF_I4 && NT == 8) ? 1 : 2) void gemm_rows_kernel(GemvArgs a, float* __restrict__ partial,
                                                           int steps_per_split, int cpb_shift) {
    constexpr int ITEMS = 2 * NT * 64 / 256;      // A items (8 floats) per thread per chunk
    __shared__ u32x4 As[2][2][NT][2][64];         // [buf][k step][tile][hi/lo][lane]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, li = lane & 15;
    const int M = a.M, N = a.N;
    const int s0 = blockIdx.y * steps_per_split;
    const int s1 = min(a.K / 32, s0 + steps_per_split);   // s1 - s0: a multiple of 4
    const int m0 = blockIdx.x * GR_ROWS + wave * 32;
    SkRow wrow[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) wrow[j] = sk_row<FMT>(a, min(m0 + 16 * j + li, M - 1));
    // A item q of this thread: (k step st, tile t, row i, k group gg) of a chunk
    auto xload = [&](int chunk, int q, f32x4& p0, f32x4& p1) {
        const int it = (int)threadIdx.x + 256 * q;
        const int gg = it & 3, ii = (it >> 2) & 15, t = (it >> 6) % NT, st = it / (64 * NT);
        const int n = t * 16 + ii;
        const long k = (long)(s0 + 2 * chunk + st) * 32 + 8 * gg;
        const float* xr = a.x + (long)min(n, N - 1) * a.x_stride_n + k;
        p0 = *reinterpret_cast<const f32x4*>(xr);
        p1 = *reinterpret_cast<const f32x4*>(xr + 4);
        if (n >= N) p0 = p1 = f32x4{0.f, 0.f, 0.f, 0.f};
    };
    auto xstore = [&](int buf, int q, const f32x4& p0, const f32x4& p1) {
        const int it = (int)threadIdx.x + 256 * q;
        const int gg = it & 3, ii = (it >> 2) & 15, t = (it >> 6) % NT, st = it / (64 * NT);
        u32x4 hi, lo;
        split8(p0, p1, hi, lo);
        As[buf][st][t][0][16 * gg + ii] = hi;
        As[buf][st][t][1][16 * gg + ii] = lo;
    };

    const int nsteps = s1 - s0;                   // k steps of this split
    const int nchunks = nsteps / 2;
    f32x4 xr0[ITEMS], xr1[ITEMS];                 // the next chunk's A items
#pragma unroll
    for (int q = 0; q < ITEMS; ++q) xload(0, q, xr0[q], xr1[q]);
#pragma unroll
    for (int q = 0; q < ITEMS; ++q) xstore(0, q, xr0[q], xr1[q]);
#pragma unroll
    for (int q = 0; q < ITEMS; ++q) xload(min(1, nchunks - 1), q, xr0[q], xr1[q]);
    SkFrag<FMT> B[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j) sk_load<FMT>(wrow[j], s0 + u, g, cpb_shift, B[u][j]);
    __syncthreads();

    f32x4 acc[NT][2];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // One chunk (k steps 2c, 2c+1; B slots u0, u0+1) as 2 NT items (k step,
    // tile) in order.  Each item's A fragments are read from LDS GR_AHEAD
    // items before its MFMAs, and X item q of chunk c+1 is split into the
    // other LDS buffer (then its registers take chunk c+2's item) between the
    // MFMAs of items 4q and 4q+1; scheduling barriers hold that order, so the
    // LDS latency and the split's VALU work overlap the matrix cores instead
    // of preceding them.
    auto chunk_body = [&](int c, int buf, int u0) {
        const int cn = min(c + 2, nchunks - 1);
        if constexpr (FMT == WF_I4 && NT == 8) {
            // int4 at eight tiles keeps its per-step products in registers
            // already (one block per CU); the items' extra live fragments
            // would spill, so its A fragments are read as used, and X item q
            // of the next chunk is split between k step 0's tiles 2q and 2q+1
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int u = u0 + st, s = s0 + 2 * c + st;
                bf16x8 bb[2];
                float ss[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    bb[j] = sk_operand<FMT>(B[u][j]);
                    ss[j] = B[u][j].s;
                    sk_load<FMT>(wrow[j], min(s + 4, s1 - 1), g, cpb_shift, B[u][j]);   // refill: step s + 4
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (st == 0 && (t & 1)) {
                        const int q = t >> 1;
                        if (c + 1 < nchunks) xstore(buf ^ 1, q, xr0[q], xr1[q]);
                        xload(cn, q, xr0[q], xr1[q]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    const bf16x8 xh = __builtin_bit_cast(bf16x8, As[buf][st][t][0][lane]);
                    const bf16x8 xl = __builtin_bit_cast(bf16x8, As[buf][st][t][1][lane]);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, bb[j], f32x4{0.f, 0.f, 0.f, 0.f},
                                                                          0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, bb[j], d, 0, 0, 0);
                        acc[t][j] += d * ss[j];
                    }
                }
            }
            __syncthreads();
            return;
        }
        constexpr int NI = 2 * NT, D = GR_AHEAD < NI ? GR_AHEAD : NI;
        bf16x8 ah[NI], al[NI];
        bf16x8 b[2][2];
        float sc[2][2];
        auto aread = [&](int i) {
            const int st = i / NT, t = i % NT;
            ah[i] = __builtin_bit_cast(bf16x8, As[buf][st][t][0][lane]);
            al[i] = __builtin_bit_cast(bf16x8, As[buf][st][t][1][lane]);
        };
        auto bprep = [&](int st) {
            const int u = u0 + st, s = s0 + 2 * c + st;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                b[st][j] = sk_operand<FMT>(B[u][j]);
                if constexpr (FMT == WF_BF16) asm volatile("" : "+v"(b[st][j]));
                sc[st][j] = 1.0f;
                if constexpr (FMT == WF_I4) sc[st][j] = B[u][j].s;
                sk_load<FMT>(wrow[j], min(s + 4, s1 - 1), g, cpb_shift, B[u][j]);   // refill: step s + 4
            }
        };
        bprep(0);
#pragma unroll
        for (int i = 0; i < D; ++i) aread(i);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (i + D < NI) aread(i + D);
            if (i == NT) bprep(1);
            if (i % 4 == 1) {
                const int q = i / 4;                  // ITEMS = NI / 4
                if (c + 1 < nchunks) xstore(buf ^ 1, q, xr0[q], xr1[q]);
                xload(cn, q, xr0[q], xr1[q]);
            }
            __builtin_amdgcn_sched_barrier(0);
            const int st = i / NT, t = i % NT;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if constexpr (FMT == WF_I4) {
                    // the step is one scale block of the lane's row
                    f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], b[st][j],
                                                                      f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], b[st][j], d, 0, 0, 0);
                    acc[t][j] += d * sc[st][j];
                } else {
                    acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], b[st][j], acc[t][j], 0, 0, 0);
                    acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], b[st][j], acc[t][j], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    };
    // block-uniform trip count: four k steps (two chunks, buffers 0 and 1)
    for (int c = 0; c < nchunks; c += 2) {
        chunk_body(c, 0, 0);
        chunk_body(c + 1, 1, 2);
    }

    // ---- epilogue: lane (g, li) holds D[4 g + v][li] of tile (t, j)
    const bool split_out = gridDim.y > 1;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int m = m0 + 16 * j + li;
            float rs = 1.0f;                                   // int8 row scale
            if constexpr (FMT == WF_I8) rs = a.scales[min(m, M - 1)];
            const float vals[4] = {acc[t][j].x * rs, acc[t][j].y * rs, acc[t][j].z * rs,
                                   acc[t][j].w * rs};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = t * 16 + 4 * g + v;
                const float val = vals[v];
                if (split_out) {
                    if (n < N && m < M) partial[((long)blockIdx.y * N + n) * M + m] = val;
                } else if (a.epi == EPI_SILU_MUL) {
                    const float up = __shfl_xor(val, 1, 64);   // rows (2i, 2i+1) = (gate, up)
                    if ((m & 1) == 0 && n < N && m + 1 < M)
                        a.y[n * a.y_stride_n + (long)(m >> 1) * a.y_stride_m] =
                            val / (1.0f + expf(-val)) * up;
                } else if (n < N && m < M) {
                    a.y[n * a.y_stride_n + (long)m * a.y_stride_m] = val;
                }
            }
        }
}

// K splits of a rows launch: enough (row block, split) blocks for one per
// CU, each split a multiple of four k steps.  (Two per CU, the occupancy
// limit, measured 3% slower over the 7B GEMMs at 128 rows and 8% at 64:
// the extra partials and reduce cost more than the second block gains.)
// int4 (one block per CU at eight tiles) takes no K split once its row blocks
// alone cover 60% of the CUs: a second split's blocks would run as a second
// round, and its partials and reduce cost ~7 us (7B gate/up, 127-token int4
// prefill 12.0 -> 11.8 ms).  For bf16 and int8 (two blocks per CU) the split
// stays faster (8.0 against 7.8 ms, 8.1 against 7.5 ms).
static void gemm_rows_split(int M, int K, int& splits, int& steps, int fmt = WF_BF16) {
    const int bx = (M + GR_ROWS - 1) / GR_ROWS, ksteps = K / 32;
    const int cus = device_cu_count();
    int want = fmt == WF_I4 && 5 * bx >= 3 * cus ? 1 : (cus + bx - 1) / bx;
    want = std::max(1, std::min(want, ksteps / 4));
    steps = ((ksteps + want - 1) / want + 3) / 4 * 4;
    splits = (ksteps + steps - 1) / steps;
}

// a: after gemv_fill_int4_index (int4 bpr / cpb)
bool gemm_rows_ok(const GemvArgs& a) {
    const uintptr_t wa = (uintptr_t)a.w;
    const bool fmt_ok =
        a.fmt == WF_BF16 ? (wa & 15) == 0 && (a.ldw == 0 || a.ldw % 16 == 0)
        : a.fmt == WF_I8 ? a.scales && (wa & 7) == 0 && (a.ldw == 0 || a.ldw % 8 == 0)
        : a.fmt == WF_I4 ? a.scales && (wa & 3) == 0 && a.ldw == 0 && a.block % 32 == 0 &&
                               a.bpr > 0 && (a.cpb & (a.cpb - 1)) == 0
                         : false;
    return fmt_ok && a.N > 16 && a.K % 128 == 0 && a.M > 0 &&
           a.x_stride_k == 1 && a.x_stride_n % 4 == 0 && ((uintptr_t)a.x & 15) == 0 &&
           (a.epi == EPI_STORE || (a.epi == EPI_SILU_MUL && a.M % 2 == 0));
}

// 2, 4 or 8 16-row tiles per launch; more are refused rather than left
// unwritten (gemm_rows_launch splits chunks above 128 rows)
template <int FMT>
static int gemm_rows_go(const GemvArgs& a, float* partial, dim3 grid, int steps, int cpb_shift,
                        hipStream_t st) {
    const int nt = (a.N + 15) / 16;
    if (nt <= 2)
        hipLaunchKernelGGL((gemm_rows_kernel<FMT, 2>), grid, dim3(256), 0, st, a, partial, steps, cpb_shift);
    else if (nt <= 4)
        hipLaunchKernelGGL((gemm_rows_kernel<FMT, 4>), grid, dim3(256), 0, st, a, partial, steps, cpb_shift);
    else if (nt <= 8)
        hipLaunchKernelGGL((gemm_rows_kernel<FMT, 8>), grid, dim3(256), 0, st, a, partial, steps, cpb_shift);
    else {
        set_error(ATLAS_EUNSUPPORTED, "gemm rows: a launch takes at most 128 rows (got %d)", a.N);
        return ATLAS_EUNSUPPORTED;
    }
    return ATLAS_OK;
}

size_t gemm_rows_partial_bytes(int M, int N, int K) {
    int splits, steps;
    gemm_rows_split(M, K, splits, steps);
    if (splits <= 1) return 0;
    return (size_t)splits * N * M * sizeof(float);
}

// one launch (+ split-K reduce, unless a.defer_splits takes the split count)
// over all a.N <= 128 rows
static int gemm_rows_part(const GemvArgs& a, hipStream_t st) {
    int splits, steps;
    gemm_rows_split(a.M, a.K, splits, steps, a.fmt);
    float* partial = nullptr;
    if (splits > 1) {
        int rc = partial_for(a, (size_t)splits * a.N * a.M * sizeof(float), &partial);
        if (rc) return rc;
    }
    const dim3 grid((a.M + GR_ROWS - 1) / GR_ROWS, splits);
    int cpb_shift = 0;
    while ((1 << cpb_shift) < a.cpb) ++cpb_shift;
    int rc;
    if (a.fmt == WF_BF16) rc = gemm_rows_go<WF_BF16>(a, partial, grid, steps, cpb_shift, st);
    else if (a.fmt == WF_I8) rc = gemm_rows_go<WF_I8>(a, partial, grid, steps, cpb_shift, st);
    else rc = gemm_rows_go<WF_I4>(a, partial, grid, steps, cpb_shift, st);
    if (rc) return rc;
    ATLAS_LAUNCH_CHECK("gemm_rows");
    if (splits > 1 && defer_ok(a)) {
        *a.defer_splits = splits;             // the consumer sums the partials
        return ATLAS_OK;
    }
    if (splits > 1) {
        const long m_out = a.epi == EPI_SILU_MUL ? a.M / 2 : a.M;
        long rb = ((long)a.N * m_out + 255) / 256;
        if (rb > 4096) rb = 4096;
        hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)rb), dim3(256), 0, st, a, partial,
                           splits);
        ATLAS_LAUNCH_CHECK("gemm_rows_reduce");
    }
    return ATLAS_OK;
}

// ---- the element-wise halves of the hipBLASLt prompt GEMM ---------------------
// Thread per 8 consecutive k of one row: the split of the tiled kernel
// (hi = the top 16 bits, lo = the rest rounded to nearest even).
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ x, long sn, int N,
                                                         int K, uint16_t* __restrict__ out) {
    const int n = blockIdx.y;
    const int k8 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (k8 >= K) return;
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + (long)n * sn + k8);
    u32x4 hi, lo;
    split8(xr[0], xr[1], hi, lo);
    *reinterpret_cast<u32x4*>(out + (long)n * K + k8) = hi;
    *reinterpret_cast<u32x4*>(out + (long)(N + n) * K + k8) = lo;
}

// Thread per output element (or per (gate, up) pair with SwiGLU).
__global__ __launch_bounds__(256) void combine_rows_kernel(const float* __restrict__ d, int N, int M,
                                                           int epi, float* __restrict__ y, long ysn,
                                                           long ysm) {
    const int n = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const float* dh = d + (long)n * M;
    const float* dl = d + (long)(N + n) * M;
    if (epi == EPI_SILU_MUL) {
        if (2 * i + 1 >= M) return;
        const float g = dh[2 * i] + dl[2 * i], u = dh[2 * i + 1] + dl[2 * i + 1];
        y[n * ysn + (long)i * ysm] = g / (1.0f + expf(-g)) * u;
    } else {
        if (i >= M) return;
        y[n * ysn + (long)i * ysm] = dh[i] + dl[i];
    }
}

// Thread per two (gate, up) pairs: h = SwiGLU(hi + lo products) as the
// combine kernel computes it, then split as split_rows_kernel does.
__global__ __launch_bounds__(256) void combine_split_kernel(const float* __restrict__ d, int N, int M,
                                                            uint16_t* __restrict__ out) {
    const int n = blockIdx.y;
    const int j = (blockIdx.x * 256 + threadIdx.x) * 2;        // first of two outputs
    const int K2 = M / 2;
    if (j >= K2) return;
    const f32x4 ph = *reinterpret_cast<const f32x4*>(d + (long)n * M + 2 * j);
    const f32x4 pl = *reinterpret_cast<const f32x4*>(d + (long)(N + n) * M + 2 * j);
    const float g0 = ph.x + pl.x, u0 = ph.y + pl.y, g1 = ph.z + pl.z, u1 = ph.w + pl.w;
    const float h[2] = {g0 / (1.0f + expf(-g0)) * u0, g1 / (1.0f + expf(-g1)) * u1};
    uint32_t hb[2], lb[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t u = __float_as_uint(h[e]);
        hb[e] = u >> 16;
        lb[e] = bf16_rne_bits(h[e] - __uint_as_float(u & 0xFFFF0000u));
    }
    *reinterpret_cast<uint32_t*>(out + (long)n * K2 + j) = pack2(hb[0], hb[1]);
    *reinterpret_cast<uint32_t*>(out + (long)(N + n) * K2 + j) = pack2(lb[0], lb[1]);
}

int combine_split_launch(const float* d, int N, int M, uint16_t* out, hipStream_t st) {
    ATLAS_REQUIRE(d && out && N > 0 && N <= 65535 && M > 0 && M % 4 == 0 && ((uintptr_t)d & 15) == 0 &&
                      ((uintptr_t)out & 3) == 0,
                  "combine split: N %d M %d", N, M);
    hipLaunchKernelGGL(combine_split_kernel, dim3((M / 4 + 255) / 256, N), dim3(256), 0, st, d, N, M,
                       out);
    ATLAS_LAUNCH_CHECK("combine_split");
    return ATLAS_OK;
}

// int8 weights (W8A32): each activation row n becomes three int8 digit rows,
// x[n, k] = s_n (d0 + d1 / 128 + d2 / 16384) + e with s_n = max_k |x[n, k]| / 127
// and |e| <= s_n / 32768 (2^-22 of the row's largest element); the library's
// int8 GEMM sums q * d exactly in int32.  A 1024-thread block per row; a
// thread holds up to DR_PT groups of four consecutive elements in registers
// between the row maximum and the digits (K <= 4 * 1024 * DR_PT), and stores
// each digit plane's four bytes as one word.
constexpr int DR_PT = kDigitsMaxK / 4096;
__global__ __launch_bounds__(1024) void digits_rows_kernel(const float* __restrict__ x, long sn, int N,
                                                           int K, int8_t* __restrict__ out,
                                                           float* __restrict__ xscale) {
    __shared__ float red[16];
    const int n = blockIdx.x;
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + (long)n * sn);
    const int ng = K >> 2;
    f32x4 v[DR_PT];
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < DR_PT; ++j) {
        const int g = threadIdx.x + 1024 * j;
        v[j] = g < ng ? xr[g] : f32x4{0.f, 0.f, 0.f, 0.f};
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, red[i]);
    const float inv = mx > 0.f ? 127.0f / mx : 0.f;
    if (threadIdx.x == 0) xscale[n] = mx / 127.0f;
    uint32_t* o0 = reinterpret_cast<uint32_t*>(out + (long)n * K);
    uint32_t* o1 = reinterpret_cast<uint32_t*>(out + (long)(N + n) * K);
    uint32_t* o2 = reinterpret_cast<uint32_t*>(out + (long)(2 * N + n) * K);
    auto digit = [](float f) { return (uint32_t)((int)fminf(fmaxf(rintf(f), -127.f), 127.f) & 0xFF); };
#pragma unroll
    for (int j = 0; j < DR_PT; ++j) {
        const int g = threadIdx.x + 1024 * j;
        if (g >= ng) break;
        const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float u = e[c] * inv;
            const uint32_t b0 = digit(u);
            const float r1 = (u - (float)(int8_t)b0) * 128.f;
            const uint32_t b1 = digit(r1);
            const float r2 = (r1 - (float)(int8_t)b1) * 128.f;
            const uint32_t b2 = digit(r2);
            w0 |= b0 << (8 * c);
            w1 |= b1 << (8 * c);
            w2 |= b2 << (8 * c);
        }
        o0[g] = w0;
        o1[g] = w1;
        o2[g] = w2;
    }
}

// y[n, m] = wscale[m] * s_n * (D0 + D1 / 128 + D2 / 16384) from the int32
// product rows of the three digit rows (M wide), with the store or SwiGLU
// epilogue; thread per output element (or per (gate, up) pair).
__global__ __launch_bounds__(256) void combine_digits_kernel(const int* __restrict__ d, int N, int M,
                                                             const float* __restrict__ wscale,
                                                             const float* __restrict__ xscale, int epi,
                                                             float* __restrict__ y, long ysn, long ysm) {
    const int n = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    const long plane = (long)N * M;
    const int* dr = d + (long)n * M;
    const float s = xscale[n];
    auto val = [&](int m) {
        const float lo = (float)dr[m + plane] + (float)dr[m + 2 * plane] * (1.0f / 128.f);
        return ((float)dr[m] + lo * (1.0f / 128.f)) * s * wscale[m];
    };
    if (epi == EPI_SILU_MUL) {
        if (2 * i + 1 >= M) return;
        const float g = val(2 * i), u = val(2 * i + 1);
        y[n * ysn + (long)i * ysm] = g / (1.0f + expf(-g)) * u;
    } else {
        if (i >= M) return;
        y[n * ysn + (long)i * ysm] = val(i);
    }
}

int digits_rows_launch(const float* x, long sn, int N, int K, int8_t* out, float* xscale,
                       hipStream_t st) {
    ATLAS_REQUIRE(x && out && xscale && N > 0 && N <= 65535 && K > 0 && K % 4 == 0 &&
                      K <= kDigitsMaxK && sn % 4 == 0 && ((uintptr_t)x & 15) == 0 &&
                      ((uintptr_t)out & 3) == 0,
                  "digit rows: N %d K %d", N, K);
    hipLaunchKernelGGL(digits_rows_kernel, dim3(N), dim3(1024), 0, st, x, sn, N, K, out, xscale);
    ATLAS_LAUNCH_CHECK("digits_rows");
    return ATLAS_OK;
}

int combine_digits_launch(const int* d, int N, int M, const float* wscale, const float* xscale, int epi,
                          float* y, long ysn, long ysm, hipStream_t st) {
    ATLAS_REQUIRE(d && wscale && xscale && y && N > 0 && N <= 65535 && M > 0 &&
                      (epi == EPI_STORE || (epi == EPI_SILU_MUL && M % 2 == 0)),
                  "combine digits: N %d M %d epi %d", N, M, epi);
    const int cols = epi == EPI_SILU_MUL ? M / 2 : M;
    hipLaunchKernelGGL(combine_digits_kernel, dim3((cols + 255) / 256, N), dim3(256), 0, st, d, N, M,
                       wscale, xscale, epi, y, ysn, ysm);
    ATLAS_LAUNCH_CHECK("combine_digits");
    return ATLAS_OK;
}

int split_rows_launch(const float* x, long sn, int N, int K, uint16_t* out, hipStream_t st) {
    ATLAS_REQUIRE(x && out && N > 0 && N <= 65535 && K > 0 && K % 8 == 0 && sn % 4 == 0 &&
                      ((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0,
                  "split rows: N %d K %d", N, K);
    hipLaunchKernelGGL(split_rows_kernel, dim3((K / 8 + 255) / 256, N), dim3(256), 0, st, x, sn, N, K,
                       out);
    ATLAS_LAUNCH_CHECK("split_rows");
    return ATLAS_OK;
}

int combine_rows_launch(const float* d, int N, int M, int epi, float* y, long ysn, long ysm,
                        hipStream_t st) {
    ATLAS_REQUIRE(d && y && N > 0 && N <= 65535 && M > 0 && (epi == EPI_STORE ||
                                                             (epi == EPI_SILU_MUL && M % 2 == 0)),
                  "combine rows: N %d M %d epi %d", N, M, epi);
    const int cols = epi == EPI_SILU_MUL ? M / 2 : M;
    hipLaunchKernelGGL(combine_rows_kernel, dim3((cols + 255) / 256, N), dim3(256), 0, st, d, N, M, epi,
                       y, ysn, ysm);
    ATLAS_LAUNCH_CHECK("combine_rows");
    return ATLAS_OK;
}

int gemm_rows_launch(const GemvArgs& a, hipStream_t st) {
    ATLAS_REQUIRE(gemm_rows_ok(a), "gemm rows: unsupported shape (fmt %d, n %d, k %d)", a.fmt, a.N,
                  a.K);
    const int cap = GR_MAX_N;
    for (int n0 = 0; n0 < a.N; n0 += cap) {
        GemvArgs p = a;
        p.N = std::min(cap, a.N - n0);
        p.x = a.x + (long)n0 * a.x_stride_n;
        p.y = a.y + (long)n0 * a.y_stride_n;
        if (a.N > cap) p.defer_splits = nullptr;   // the parts share one partial buffer
        int rc = gemm_rows_part(p, st);
        if (rc) return rc;
    }
    return ATLAS_OK;
}

template <int FMT>
static int launch_skinny_n(const GemvArgs& a, hipStream_t st) {
    return a.N > 8 ? launch_skinny<FMT, 2>(a, st) : launch_skinny<FMT, 1>(a, st);
}

// Whether 9..16 rows run faster as two launches of the 2..8-row kernels
// (the weights stream twice) than through the 16-row MFMA tiles.  Measured at
// the 7B shapes on MI355X (us, 16 rows: MFMA tiles against two 8-row launches):
// int4 QKV 28.0 / 21.5, W_o 18.6 / 13.6, gate/up 40.2 / 32.2, W_down 49.6 /
// 27.3; int8 W_o 17.8 / 14.7, W_down 46.0 / 32.3, but gate/up 40.6 / 46.0 and
// QKV even; bf16 W_down 48.0 / 43.8, but QKV 31.9 / 40.6, gate/up 46.3 / 68.
static bool halves_pay(const GemvArgs& a) {
    if (a.N < 9 || a.N > 16) return false;
    if (a.fmt == WF_I4) return a.block % 32 == 0 && (a.cpb & (a.cpb - 1)) == 0 && a.bpr > 0;
    if (a.fmt == WF_I8) return a.K > 4096 || a.M <= 8192;
    return a.fmt == WF_BF16 && a.K > 4096;
}

int skinny_launch(const GemvArgs& a_in, hipStream_t st) {
    GemvArgs a = a_in;
    if (a.defer_splits) *a.defer_splits = 0;
    gemv_fill_int4_index(a);
    if (halves_pay(a)) {
        const int n0 = (a.N + 1) / 2;
        GemvArgs h = a;
        h.defer_splits = nullptr;        // two launches share the partial buffer
        h.N = n0;
        const int rc = skinny_launch(h, st);
        if (rc) return rc;
        h.N = a.N - n0;
        h.x = a.x + (long)n0 * a.x_stride_n;
        h.y = a.y + (long)n0 * a.y_stride_n;
        return skinny_launch(h, st);
    }
    a.x_vec = a.x_stride_k == 1 && a.x_stride_n % 4 == 0 && ((uintptr_t)a.x & 15) == 0;
    if (a.N > 16 && gemm_rows_ok(a))
        return a.blas && (a.fmt == WF_BF16 || (a.fmt == WF_I8 && a.K <= kDigitsMaxK))
                   ? blas_rows_launch(a.blas, a, st)
                   : gemm_rows_launch(a, st);
    ATLAS_REQUIRE(a.N >= 1 && a.N <= 16, "skinny: N=%d outside 1..16 (17+ rows need K %% 128 == 0 "
                  "and, for int4, blocks of 32 * 2^j)", a.N);
    ATLAS_REQUIRE(a.w && a.x && a.y, "skinny: null pointer");
    ATLAS_REQUIRE(a.fmt == WF_BF16 || a.scales, "skinny: null scales");
    if (a.epi == EPI_SILU_MUL) ATLAS_REQUIRE(a.M % 2 == 0, "skinny: silu-mul needs even rows");
    if (a.M == 0) return ATLAS_OK;
    ATLAS_REQUIRE(a.K % 32 == 0 && a.K > 0, "skinny: K %% 32 != 0");
    ATLAS_REQUIRE(gemv_pitch_ok(a), "skinny: row pitch %ld bytes for K %d", a.ldw, a.K);
    // int4 at 2-8 rows: the direct-load MFMA kernel (at the 7B shapes on
    // MI355X 0.55-0.8x the multi-row GEMV's time at two and three rows, and
    // 1.05-1.2x the batch-1 GEMV's from 11008 x 4096 up).
    if (a.fmt == WF_I4 && a.N >= 2 && a.N <= 8 && a.block % 32 == 0 && (a.cpb & (a.cpb - 1)) == 0 &&
        a.bpr > 0) {
        const int rc = launch_skinny_i4d(a, st);
        if (rc != 1) return rc;
    }
    // bf16 / int8 at 2-8 rows (MI355X, 7B shapes at 8 rows against the
    // batch-1 GEMV's time over the same weights):
    //  * K <= 4096: the LDS-staged kernel (bf16 gate/up 33.4 vs 29.1 us, QKV
    //    20.7 vs 18.0; int8 gate/up 22.0 vs 17.6), except bf16 at two rows,
    //    where the multi-row GEMV is faster (30.7 vs 33.2 us at gate/up);
    //  * K > 4096: the direct-load kernel over K splits (bf16 W_down 25.0 us,
    //    int8 17.9 us, against 36.0 and 33.1 for skinny_kernel).
    if (a.N >= 2 && a.N <= 8 && (a.fmt == WF_I8 || a.fmt == WF_BF16)) {
        int rc = 1;
        if (a.K > 4096)
            rc = a.fmt == WF_I8 ? launch_skinny_d<WF_I8>(a, st) : launch_skinny_d<WF_BF16>(a, st);
        else if (a.fmt == WF_I8 || a.N >= 3)
            rc = a.fmt == WF_I8 ? launch_skinny_lds<WF_I8>(a, st) : launch_skinny_lds<WF_BF16>(a, st);
        if (rc != 1) return rc;
    }
    // Two or three rows stream the weights once through the multi-row GEMV:
    // at the 7B shapes on MI355X it takes 0.55-0.75x the MFMA kernel's time
    // for two rows and 0.65-0.9x for three; from four rows on, the LDS reads
    // of the x rows per weight chunk make it no faster than the MFMA kernel.
    if (a.N <= 3 && gemv_multi_ok(a)) return gemv_multi_launch(a, st);
    // One row is the batch-1 GEMV (int4 11008 x 4096: 10 us against 15.6 us
    // for the MFMA tiles, whose 16 rows would be 15 / 16 padding).
    if (a.N == 1 && a.x_stride_k == 1 && a.y_stride_m == 1 && (a.epi == EPI_STORE ||
                                                               a.epi == EPI_SILU_MUL)) {
        const uintptr_t al = (uintptr_t)a.w | (uintptr_t)a.x;
        if ((al & 15) == 0 && a.K % 4 == 0 && gemv_fast_ok(a.fmt, a.K, a.block) &&
            gemv_x_lds_bytes(a.K) <= 160 * 1024) {
            GemvArgs g = a;
            g.N = 1;
            return gemv_launch(g, st);
        }
    }
    const uintptr_t al = (uintptr_t)a.w;
    switch (a.fmt) {
    case WF_BF16:
        ATLAS_REQUIRE((al & 15) == 0, "skinny bf16: weights not 16-byte aligned");
        return launch_skinny_n<WF_BF16>(a, st);
    case WF_I8:
        ATLAS_REQUIRE((al & 7) == 0, "skinny int8: weights not 8-byte aligned");
        return launch_skinny_n<WF_I8>(a, st);
    case WF_I4:
        ATLAS_REQUIRE((al & 3) == 0, "skinny int4: weights not 4-byte aligned");
        ATLAS_REQUIRE(a.block % 32 == 0 && (a.cpb & (a.cpb - 1)) == 0 && a.bpr > 0,
                      "skinny int4: block %d must be 32 * 2^j and divide K", a.block);
        return launch_skinny_n<WF_I4>(a, st);
    }
    set_error(ATLAS_EUNSUPPORTED, "skinny: weight format %d", a.fmt);
    return ATLAS_EUNSUPPORTED;
}

}  // namespace atlas
