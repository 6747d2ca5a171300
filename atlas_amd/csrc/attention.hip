// attention.hip -- GQA single-token decode attention over the f32 KV cache.
//
// Semantics (crates/atlas-model/src/lib.rs:689-721; GPU contract
// crates/atlas-tensor/src/lib.rs:743-770): for query head h with KV head
// kvh = h / (n_heads / n_kv), s_t = (q_h . k_t) * scale for t in [t_lo, pos]
// where t_lo = pos - window + 1 when window > 0 (positions with
// pos - t >= window are masked out), p = softmax(s), o_h = sum_t p_t v_t.
// Cache layout [max_seq][n_kv][head_dim] f32 (lib.rs:557-596).
//
// Design (split-K flash decode, HBM-bound):
//  * grid (n_kv, n_splits); a 256-thread block owns one KV head and one
//    contiguous slice of positions, and serves all G = n_heads / n_kv query
//    heads of that group from a single read of each K/V row (the reference
//    kernel re-reads K/V once per query head);
//  * 16 lanes per position (head_dim / 16 dims each, 128-bit loads); each of
//    the block's 16 lane groups keeps an online-softmax state (max, sum,
//    partial output) per head and scans its positions with the next step's
//    K/V rows already in flight (attn_scan);
//  * scores use exp2 with log2(e) folded into the scale; the SWA start index
//    is computed, not masked;
//  * per block, the 16 (wave, row) states merge through LDS into one partial
//    (m, l, o) per head and split; attn_combine merges the splits.
//  * the split count is fixed at launch and `pos` may come from device
//    memory, so the same launch can be captured once and replayed per token.
#include <algorithm>
#include <mutex>

#include "common.hpp"
#include "attention.hpp"

namespace atlas {

__device__ __forceinline__ int load_pos(const int* pos_dev, int pos) {
    return pos_dev ? *pos_dev : pos;
}

// ---- the K/V scan shared by the split and fused kernels --------------------
// A block has 16 (wave, row) groups of 16 lanes; a group owns one position at
// a time, each lane DPL = HD/16 dims of it.  Group w handles the P
// consecutive positions b0 + 16*P*s + w*P + i of step s, so one step issues
// 2*P*DPL/4 = 16 128-bit loads per lane (P = 8, 4, 2 for HD 64, 128, 256).
//
// Decode attention is latency-bound per block: a CU sees ~1 us of HBM latency
// and streams at most (bytes in flight) / latency.  The scan therefore keeps
// two register buffers and loads step s+1 while step s is scored, with a
// scheduling barrier after each batch of loads -- left alone, the compiler
// interleaves each load with its use to save registers and the block waits
// out one full latency per 16-byte load.  The loads are raw buffer loads: the
// K (V) rows of the block's KV head form one buffer resource whose size ends
// at row e1, so an address needs one 32-bit VGPR and rows past the end read
// as zero (and are scored as -inf) with no clamp or branch.
// P positions per 16-lane group per step.  For HD = 128, two positions
// instead of four halve the register buffers (GQA-4: 170 VGPRs instead of
// 238), which outweighs the shorter steps: the two-kernel path at ctx 4096 /
// 16384 runs 14.7 / 31.3 us instead of 15.8 / 32.9 us; the decode step is
// unchanged.
template <int HD> struct ScanShape {
    static constexpr int DPL = HD / 16;
    static constexpr int P = HD == 64 ? 8 : 2;
};
// Steps each scan keeps in flight (register buffers of 2 * P * HD / 16 floats
// each): the split kernel's, and the fused decode kernel's.
constexpr int kScanDepth = 2;
#ifndef ATLAS_FUSED_SCAN_DEPTH
#define ATLAS_FUSED_SCAN_DEPTH 3
#endif
constexpr int kFusedScanDepth = ATLAS_FUSED_SCAN_DEPTH;

// A lane of a 16-lane position group owns DPL = HD/16 dims in chunks of 4:
// chunk c holds dims c*64 + dl*4 .. +3.  One 16-byte load per chunk then
// covers 256 contiguous bytes of the row across the group (whole cache
// lines), where contiguous per-lane dims would touch each line twice.
__device__ __forceinline__ int lane_dim(int dl, int d) { return (d >> 2) * 64 + dl * 4 + (d & 3); }

struct ScanBufs {
    __amdgpu_buffer_rsrc_t k, v;
    uint32_t row_bytes;      // bytes between consecutive positions
    uint32_t lane_bytes;     // this lane's byte offset inside a row
};

// kb/vb point at dim 0 of the KV head in row 0; rows [0, e1) are readable.
// The caller guarantees e1 * row_bytes < 2^32.
__device__ __forceinline__ ScanBufs scan_bufs(const float* kb, const float* vb, long kv_stride,
                                              int e1, int lane_dims) {
    ScanBufs b;
    const uint32_t rb = __builtin_amdgcn_readfirstlane((uint32_t)(kv_stride * 4));
    const int n = __builtin_amdgcn_readfirstlane((int)((uint32_t)e1 * rb));
    b.k = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kb), (short)0, n, 0x00020000);
    b.v = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vb), (short)0, n, 0x00020000);
    b.row_bytes = rb;
    b.lane_bytes = (uint32_t)lane_dims * 4u;
    return b;
}

template <int HD>
__device__ __forceinline__ void scan_load(const ScanBufs& b, int t,
                                          float (&kf)[ScanShape<HD>::P][HD / 16],
                                          float (&vf)[ScanShape<HD>::P][HD / 16]) {
    constexpr int P = ScanShape<HD>::P, DPL = HD / 16;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const uint32_t off = (uint32_t)(t + i) * b.row_bytes + b.lane_bytes;
#pragma unroll
        for (int d = 0; d < DPL; d += 4) {
            const f32x4 kv = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(b.k, (int)(off + (d >> 2) * 256), 0, 0));
            const f32x4 vv = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(b.v, (int)(off + (d >> 2) * 256), 0, 0));
            kf[i][d] = kv.x; kf[i][d + 1] = kv.y; kf[i][d + 2] = kv.z; kf[i][d + 3] = kv.w;
            vf[i][d] = vv.x; vf[i][d + 1] = vv.y; vf[i][d + 2] = vv.z; vf[i][d + 3] = vv.w;
        }
    }
}

// Online-softmax update of a group's state with positions t .. t+P-1 (those
// >= end are masked).  q is pre-scaled by scale * log2(e).  A group may see
// steps with no valid position (the scan loop is block-uniform); its state
// then stays (m, l, o) = (-inf, 0, 0) with no NaN.
template <int HD, int G>
__device__ __forceinline__ void scan_update(const float (&q)[G][HD / 16], float (&m)[G],
                                            float (&l)[G], float (&o)[G][HD / 16],
                                            const float (&kf)[ScanShape<HD>::P][HD / 16],
                                            const float (&vf)[ScanShape<HD>::P][HD / 16], int t,
                                            int end) {
    constexpr int P = ScanShape<HD>::P, DPL = HD / 16;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float s[P];
        float smax = -INFINITY;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            float acc = 0.f;
#pragma unroll
            for (int d = 0; d < DPL; ++d) acc += q[h][d] * kf[i][d];
            acc = row16_sum(acc);
            s[i] = t + i < end ? acc : -INFINITY;
            smax = fmaxf(smax, s[i]);
        }
        const float mn = fmaxf(m[h], smax);
        const float corr = m[h] == -INFINITY ? 0.f : exp2f(m[h] - mn);
        float psum = 0.f, p[P];
#pragma unroll
        for (int i = 0; i < P; ++i) {
            p[i] = t + i < end ? exp2f(s[i] - mn) : 0.f;
            psum += p[i];
        }
        l[h] = l[h] * corr + psum;
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            float acc = o[h][d] * corr;
#pragma unroll
            for (int i = 0; i < P; ++i) acc += p[i] * vf[i][d];
            o[h][d] = acc;
        }
        m[h] = mn;
    }
}

// scan_update for rows loaded before the live range was known: positions
// outside [lo, end) are masked and their V rows zeroed first (rows past the
// live position may hold anything a previous sequence left there).
template <int HD, int G>
__device__ __forceinline__ void scan_update_masked(const float (&q)[G][HD / 16], float (&m)[G],
                                                   float (&l)[G], float (&o)[G][HD / 16],
                                                   const float (&kf)[ScanShape<HD>::P][HD / 16],
                                                   float (&vf)[ScanShape<HD>::P][HD / 16], int t,
                                                   int lo, int end) {
    constexpr int P = ScanShape<HD>::P, DPL = HD / 16;
    float kk[P][DPL];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const bool ok = t + i >= lo && t + i < end;
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            kk[i][d] = ok ? kf[i][d] : 0.f;
            vf[i][d] = ok ? vf[i][d] : 0.f;
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float s[P];
        float smax = -INFINITY;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            float acc = 0.f;
#pragma unroll
            for (int d = 0; d < DPL; ++d) acc += q[h][d] * kk[i][d];
            acc = row16_sum(acc);
            s[i] = (t + i >= lo && t + i < end) ? acc : -INFINITY;
            smax = fmaxf(smax, s[i]);
        }
        const float mn = fmaxf(m[h], smax);
        const float corr = m[h] == -INFINITY ? 0.f : exp2f(m[h] - mn);
        float psum = 0.f, p[P];
#pragma unroll
        for (int i = 0; i < P; ++i) {
            p[i] = (t + i >= lo && t + i < end) ? exp2f(s[i] - mn) : 0.f;
            psum += p[i];
        }
        l[h] = l[h] * corr + psum;
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            float acc = o[h][d] * corr;
#pragma unroll
            for (int i = 0; i < P; ++i) acc += p[i] * vf[i][d];
            o[h][d] = acc;
        }
        m[h] = mn;
    }
}

// Merge the online-softmax states of a wave's four 16-lane rows (lanes with
// the same dl hold the same dims in every row) by lane shuffles across rows;
// afterwards every row holds the wave's state.  An empty state (m = -inf)
// weighs 0.
template <int HD, int G>
__device__ __forceinline__ void merge_rows(float (&m)[G], float (&l)[G], float (&o)[G][HD / 16]) {
    constexpr int DPL = HD / 16;
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float m2 = __shfl_xor(m[h], sh, 64);
            const float l2 = __shfl_xor(l[h], sh, 64);
            const float mn = fmaxf(m[h], m2);
            const float c1 = m[h] == -INFINITY ? 0.f : exp2f(m[h] - mn);
            const float c2 = m2 == -INFINITY ? 0.f : exp2f(m2 - mn);
            l[h] = l[h] * c1 + l2 * c2;
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                const float o2 = __shfl_xor(o[h][d], sh, 64);
                o[h][d] = o[h][d] * c1 + o2 * c2;
            }
            m[h] = mn;
        }
    }
}

// States a block merges through LDS: its W waves' when the rows of each wave
// were merged by shuffles first (G <= 2: 10 shuffles per head and stage),
// else all 4 W (wave, row) states (at G = 4 the shuffle chains cost more
// than the LDS reads they save: the GQA 32/8/128 split kernel at ctx 512 /
// 4096 ran 0.8 / 0.7 us slower with them on MI355X).
template <int G, int W> constexpr int block_states() { return G <= 2 ? W : 4 * W; }

// Writes the block's states for the LDS merge: (m, l) per head and the
// partial output of every dim.
template <int HD, int G, int W, int NS = block_states<G, W>()>
__device__ __forceinline__ void stage_block_states(float (&m)[G], float (&l)[G], float (&o)[G][HD / 16],
                                                   int wave, int row, int dl, float (&s_m)[NS][G],
                                                   float (&s_l)[NS][G], float (&s_o)[NS][G][HD]) {
    constexpr int DPL = HD / 16;
    if constexpr (NS == W) merge_rows<HD, G>(m, l, o);
    const int st = NS == W ? wave : wave * 4 + row;
    if (NS == W && row != 0) return;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (dl == 0) { s_m[st][h] = m[h]; s_l[st][h] = l[h]; }
#pragma unroll
        for (int d = 0; d < DPL; ++d) s_o[st][h][lane_dim(dl, d)] = o[h][d];
    }
}

// Scan cache rows [b0, e1) into the (wave, row) group's state (NG groups per
// block).  kb/vb: dim 0 of the KV head in row 0, lane_dims: the lane's
// first dim (lane_dim(dl, 0)).  scan_start issues the first PD - 1 steps'
// loads; scan_run scores everything, issuing each step's loads PD - 1 steps
// ahead of its scoring.  A caller can put independent work (the fused
// kernel's QK-norm/RoPE prep) between them, so that work and the first
// loads' latency overlap.
template <int HD, int PD>
struct ScanState {
    static constexpr int P = ScanShape<HD>::P, DPL = HD / 16;
    ScanBufs b;
    int t, steps;
    float k[PD][P][DPL], v[PD][P][DPL];
};

template <int HD, int NG, int PD>
__device__ __forceinline__ void scan_start(ScanState<HD, PD>& s, const float* kb, const float* vb,
                                           long kv_stride, int lane_dims, int b0, int e1,
                                           int group) {
    constexpr int S = NG * ScanShape<HD>::P;
    // Block-uniform trip count and one exit, at the bottom of the loop: with a
    // divergent or mid-body exit the compiler must assume the other buffers'
    // loads may still be in flight at the loop head and waits for them there,
    // serialising the buffers again.
    s.steps = __builtin_amdgcn_readfirstlane(e1 > b0 ? (e1 - b0 + S - 1) / S : 0);
    s.t = b0 + group * ScanShape<HD>::P;
    // Unconditional, also for a slice with no rows (those loads lie past the
    // buffer's end: zeros, no traffic).  A return here would join two paths
    // with different loads in flight, and the wait count merged at the join
    // would make the caller's next use of its own, earlier loads wait for
    // every K/V load issued here.
    s.b = scan_bufs(kb, vb, kv_stride, e1 > 0 ? e1 : 0, lane_dims);
#pragma unroll
    for (int i = 0; i < PD - 1; ++i) scan_load<HD>(s.b, s.t + i * S, s.k[i], s.v[i]);
}

template <int HD, int G, int NG, int PD>
__device__ __forceinline__ void scan_run(ScanState<HD, PD>& s, int e1, const float (&q)[G][HD / 16],
                                         float (&m)[G], float (&l)[G], float (&o)[G][HD / 16]) {
    constexpr int S = NG * ScanShape<HD>::P;
    if (s.steps == 0) return;
    int t = s.t;
    // step j lives in buffer j % PD; before step j is scored, step j + PD - 1
    // goes out into the buffer step j - 1 has freed (past the end: zeros, no
    // traffic), then a scheduling barrier keeps those loads ahead of the
    // scoring
    const int full = s.steps / PD;
    for (int it = 0; it < full; ++it) {
#pragma unroll
        for (int i = 0; i < PD; ++i) {
            const int nb = (i + PD - 1) % PD;
            scan_load<HD>(s.b, t + (PD - 1) * S, s.k[nb], s.v[nb]);
            __builtin_amdgcn_sched_barrier(0);
            scan_update<HD, G>(q, m, l, o, s.k[i], s.v[i], t, e1);
            t += S;
        }
    }
    const int rem = s.steps - full * PD;
#pragma unroll
    for (int i = 0; i < PD - 1; ++i) {
        if (i < rem) {
            scan_update<HD, G>(q, m, l, o, s.k[i], s.v[i], t, e1);
            t += S;
        }
    }
}

// Split merge of the fused kernel (and of the split kernel's one-launch
// mode), run by the block that arrives last.  The
// partials of query head qh, split s sit at index qh * n_splits + s (o: times
// HD) of part_m / part_l / part_o; other XCDs wrote them, so they are read
// with sc1 loads (past this XCD's L2, which can still hold an earlier
// launch's lines).  A thread owns (head, dim) elements and reads the splits in
// groups of 8, every load of a group -- for all of its elements -- issued
// before the first is used, with a running maximum across groups: one memory
// round trip per 8 splits instead of one per split and element.  Empty splits carry (m, l, o) = (-inf, 0, 0) and weigh 0;
// the split holding pos is never empty, so the final maximum is finite.
template <int HD, int G, int NT>
__device__ __forceinline__ void merge_splits(const float* part_m, const float* part_l, const float* part_o,
                                             int n_splits, int kvh, float* out) {
    constexpr int SC1 = 16;                   // buffer cache policy: sc1
    constexpr int NE = (G * HD + NT - 1) / NT;   // (head, dim) elements per thread
    const int nh = n_splits * G;              // this kv head's (head, split) pairs
    const long h0 = (long)kvh * G * n_splits;
    const __amdgpu_buffer_rsrc_t rm =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(part_m + h0), (short)0, nh * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rl =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(part_l + h0), (short)0, nh * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t ro =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(part_o + h0 * HD), (short)0, nh * HD * 4, 0x00020000);
    float M[NE], L[NE], O[NE];
#pragma unroll
    for (int k = 0; k < NE; ++k) { M[k] = -INFINITY; L[k] = 0.f; O[k] = 0.f; }
    for (int s0 = 0; s0 < n_splits; s0 += 8) {
        // every load of this round, for all of the thread's elements, goes out
        // before the first is used: one memory round trip per 8 splits
        float mv[NE][8], lv[NE][8], ov[NE][8];
#pragma unroll
        for (int k = 0; k < NE; ++k) {
            const int e = min((int)threadIdx.x + k * NT, G * HD - 1);   // past the end: a copy
            const int h = e / HD, d = e % HD;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = h * n_splits + min(s0 + j, n_splits - 1);   // past the end: a copy
                mv[k][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, i * 4, 0, SC1));
                lv[k][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, i * 4, 0, SC1));
                ov[k][j] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(ro, (i * HD + d) * 4, 0, SC1));
            }
        }
#pragma unroll
        for (int k = 0; k < NE; ++k) {
            float cm = M[k];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (s0 + j >= n_splits) mv[k][j] = -INFINITY;               // ... which weighs 0
                cm = fmaxf(cm, mv[k][j]);
            }
            if (cm == -INFINITY) continue;   // every split so far is empty
            const float c = exp2f(M[k] - cm);    // 0 while M = -inf
            L[k] *= c;
            O[k] *= c;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float w = exp2f(mv[k][j] - cm);
                L[k] += lv[k][j] * w;
                O[k] += ov[k][j] * w;
            }
            M[k] = cm;
        }
    }
#pragma unroll
    for (int k = 0; k < NE; ++k) {
        const int e = threadIdx.x + k * NT;
        if (e < G * HD) out[(long)(kvh * G + e / HD) * HD + e % HD] = O[k] / L[k];
    }
}

template <int HD, int G, int W>
__global__ __launch_bounds__(64 * W) void attn_split_kernel(AttnArgs a) {
    constexpr int DPL = HD / 16;              // dims per lane
    constexpr float LOG2E = 1.4426950408889634f;
    const int kvh = blockIdx.x, split = blockIdx.y, seq = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = lane >> 4, dl = lane & 15;     // position row, dim group
    const int pos = a.pos_dev ? a.pos_dev[seq] : a.pos;
    const long cache0 = a.slot_dev ? (long)a.slot_dev[seq] * a.slot_stride : 0;
    const float* qs = a.q + (long)seq * a.q_stride;
    float* out = a.out + (long)seq * a.out_stride;
    const long pbase = (long)seq * a.n_heads * gridDim.y;
    const int t_lo = (a.window > 0 && pos >= a.window) ? pos - a.window + 1 : 0;
    const int ctx = pos - t_lo + 1;
    const int n_splits = a.adaptive
        ? min((int)gridDim.y, attn_batch_splits_for(a.n_kv, gridDim.z, ctx)) : gridDim.y;
    if (split >= n_splits) return;
    const int chunk = (ctx + n_splits - 1) / n_splits;
    const int b0 = t_lo + split * chunk;
    const int b1 = min(pos + 1, b0 + chunk);
    const long kv_stride = (long)a.n_kv * HD;
    const float sc = a.scale * LOG2E;
    // the scan's first K/V steps go out before q's loads
    ScanState<HD, kScanDepth> scan;
    scan_start<HD, 4 * W, kScanDepth>(scan, a.k_cache + cache0 + (long)kvh * HD,
                                      a.v_cache + cache0 + (long)kvh * HD, kv_stride, lane_dim(dl, 0),
                                      b0, b1, wave * 4 + row);
    __builtin_amdgcn_sched_barrier(0);

    // q for the G heads of this group, this lane's dims
    float q[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float* qh = qs + (long)(kvh * G + h) * HD;
#pragma unroll
        for (int d = 0; d < DPL; d += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(qh + lane_dim(dl, d));
            q[h][d] = v.x * sc; q[h][d + 1] = v.y * sc; q[h][d + 2] = v.z * sc; q[h][d + 3] = v.w * sc;
        }
    }
    float m[G], l[G], o[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY; l[h] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[h][d] = 0.f;
    }

    scan_run<HD, G, 4 * W, kScanDepth>(scan, b1, q, m, l, o);

    // ---- merge the block's 16 (wave, row) states (first by lane shuffles
    // within each wave when G is small) through LDS ------------------------------
    constexpr int NS = block_states<G, W>();
    __shared__ float s_m[NS][G], s_l[NS][G];
    __shared__ float s_o[NS][G][HD];
    stage_block_states<HD, G, W>(m, l, o, wave, row, dl, s_m, s_l, s_o);
    __syncthreads();
    // thread -> (head, dim) pairs
    for (int e = threadIdx.x; e < G * HD; e += 64 * W) {
        const int h = e / HD, d = e % HD;
        float mx = -INFINITY;
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) mx = fmaxf(mx, s_m[s2][h]);
        float lsum = 0.f, osum = 0.f;
        if (mx != -INFINITY) {
#pragma unroll
            for (int s2 = 0; s2 < NS; ++s2) {
                const float w = exp2f(s_m[s2][h] - mx);   // 0 for empty states
                lsum += s_l[s2][h] * w;
                osum += s_o[s2][h][d] * w;
            }
        }
        const int qh = kvh * G + h;
        if (n_splits == 1) {
            out[(long)qh * HD + d] = osum / lsum;
        } else if (a.counters) {
            // agent-scope (sc1) stores for the merging block on any XCD
            const long pi = pbase + (long)qh * n_splits + split;
            __hip_atomic_store(&a.part_o[pi * HD + d], osum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(&a.part_m[pi], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&a.part_l[pi], lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            const long pi = pbase + (long)qh * n_splits + split;
            a.part_o[pi * HD + d] = osum;
            if (d == 0) { a.part_m[pi] = mx; a.part_l[pi] = lsum; }
        }
    }
    if (n_splits == 1 || !a.counters) return;
    // ---- one launch: the last block of this (seq, kv head) merges ------------
    // (as in attn_fused_kernel: partial stores complete before the counter
    // bump; the merging block resets the counter for the next launch)
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0x0F70);        // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(&a.counters[seq * a.n_kv + kvh], 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == n_splits - 1;
    }
    __syncthreads();
    if (!s_last) return;
    merge_splits<HD, G, 64 * W>(a.part_m + pbase, a.part_l + pbase, a.part_o + pbase * HD, n_splits,
                                kvh, out);
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[seq * a.n_kv + kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split merge of the reference-ABI path: one block per query head.  The
// split maxima and weights go through LDS once; every (split, dim) partial is
// then an independent load, so the sum streams instead of waiting on each
// split in turn.  Empty splits carry (m, l, o) = (-inf, 0, 0) and weigh 0.


__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a, int n_splits, int hd) {
    __shared__ float s_w[kAttnMaxSplits];
    __shared__ float s_red[4];
    const int qh = blockIdx.x, seq = blockIdx.y;
    const long pbase = (long)seq * a.n_heads * n_splits;   // n_splits: the split grid
    float* out = a.out + (long)seq * a.out_stride;
    if (a.adaptive) {
        // the split kernel's active count for this sequence's live context
        const int pos = a.pos_dev ? a.pos_dev[seq] : a.pos;
        const int t_lo = (a.window > 0 && pos >= a.window) ? pos - a.window + 1 : 0;
        n_splits = min(n_splits, attn_batch_splits_for(a.n_kv, gridDim.y, pos - t_lo + 1));
        if (n_splits == 1) return;             // the split kernel wrote out
    }
    const long base = pbase + (long)qh * n_splits;
    float mx = -INFINITY;
    for (int s = threadIdx.x; s < n_splits; s += blockDim.x) mx = fmaxf(mx, a.part_m[base + s]);
    mx = wave_max(mx);
    const int nw = (blockDim.x + 63) >> 6;
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = s_red[0];
    for (int w = 1; w < nw; ++w) mx = fmaxf(mx, s_red[w]);
    for (int s = threadIdx.x; s < n_splits; s += blockDim.x)
        s_w[s] = exp2f(a.part_m[base + s] - mx);
    __syncthreads();
    float lsum = 0.f;
    for (int s = 0; s < n_splits; ++s) lsum += a.part_l[base + s] * s_w[s];
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float osum = 0.f;
#pragma unroll 8
        for (int s = 0; s < n_splits; ++s) osum += a.part_o[(base + s) * hd + d] * s_w[s];
        out[(long)qh * hd + d] = osum / lsum;
    }
}

// Any head_dim / group size: one block per query head, online softmax over
// all positions with a wave per position slice (used for small test shapes).
__global__ __launch_bounds__(256) void attn_generic_kernel(AttnArgs a, int hd) {
    const int h = blockIdx.x;
    const int group = a.n_heads / a.n_kv;
    const int kvh = h / group;
    const int pos = load_pos(a.pos_dev, a.pos);
    const int t_lo = (a.window > 0 && pos >= a.window) ? pos - a.window + 1 : 0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* qh = a.q + (long)h * hd;
    const long kv_stride = (long)a.n_kv * hd;
    __shared__ float s_m[4], s_l[4];
    __shared__ float s_o[4][256];
    // each wave handles positions t = t_lo + wave, +4, ...; lanes split dims
    float m = -INFINITY, l = 0.f;
    float o[4] = {0.f, 0.f, 0.f, 0.f};   // dims lane + 64*j (hd <= 256)
    for (int t = t_lo + wave; t <= pos; t += 4) {
        const float* kt = a.k_cache + (long)t * kv_stride + (long)kvh * hd;
        const float* vt = a.v_cache + (long)t * kv_stride + (long)kvh * hd;
        float part = 0.f;
        for (int d = lane; d < hd; d += 64) part += qh[d] * kt[d];
        const float s = wave_sum(part) * a.scale;
        const float mn = fmaxf(m, s);
        const float corr = expf(m - mn), p = expf(s - mn);
        l = l * corr + p;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            o[j] = o[j] * corr + (d < hd ? p * vt[d] : 0.f);
        }
        m = mn;
    }
    if (lane == 0) { s_m[wave] = m; s_l[wave] = l; }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < hd) s_o[wave][lane + 64 * j] = o[j];
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += 256) {
        float mx = -INFINITY;
        for (int w = 0; w < 4; ++w) mx = fmaxf(mx, s_m[w]);
        float ls = 0.f, os = 0.f;
        for (int w = 0; w < 4; ++w) {
            if (s_m[w] == -INFINITY) continue;
            const float wt = expf(s_m[w] - mx);
            ls += s_l[w] * wt;
            os += s_o[w][d] * wt;
        }
        a.out[(long)h * hd + d] = os / ls;
    }
}


// ---------------------------------------------------------------------------
// Fused decode attention for one layer: per-head QK-norm (eps 1e-6,
// crates/atlas-model/src/lib.rs:660-672) and rotate-half RoPE from the tables
// (lib.rs:428-437) of the raw q|k|v GEMV output, K/V cache write at pos
// (lib.rs:577-585), split-K attention (lib.rs:689-721) and the split merge,
// in one launch.  grid (n_kv, n_splits, n_seq).
//  * every block recomputes the normalised+rotated q of its G heads and k
//    (a few hundred flops) into LDS;
//  * the block whose slice contains pos writes k/v into the cache and scores
//    position pos from LDS, so no block reads a cache row written in this
//    launch;
//  * the splits of a (sequence, kv head) merge in the block that finishes
//    last: each block publishes its partial, fences, and bumps a counter; the
//    block that sees n_splits - 1 merges and resets the counter to 0 (no
//    waiting anywhere, and the counters are clean for the next launch).
// ---------------------------------------------------------------------------
// LIVE: the step provides its RoPE row (a.rope_row) and the launch is one
// sequence in slot 0; the prep then needs no position, and split 0 loads its
// first steps before the position arrives (the pre-scan).
template <int HD, int G, int W, int PD, bool LIVE>
__global__ __launch_bounds__(64 * W) void attn_fused_kernel(AttnFusedArgs a) {
    constexpr int DPL = HD / 16;
    constexpr int EPL = HD / 64;              // head elements per lane in the prep
    constexpr float LOG2E = 1.4426950408889634f;
    constexpr int S = 4 * W * ScanShape<HD>::P;   // positions per scan step
    if constexpr (LIVE) {
        // the arguments the loads before pos and the split rule after it
        // need, in SGPRs now, in one round of argument loads: fetched where
        // first used, they cost further dependent rounds between the prep's
        // loads and the pre-scan's, and after pos
        asm volatile("" ::"s"(a.k_cache), "s"(a.v_cache), "s"(a.max_rows), "s"(gridDim.y),
                     "s"(a.window), "s"(a.adaptive), "s"(a.qk_eps), "s"(a.scale));
    }
    const int kvh = blockIdx.x, split = blockIdx.y, seq = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = lane >> 4, dl = lane & 15;
    const long kv_stride = (long)a.n_kv * HD;
    const float* qkv = a.qkv + (long)seq * a.qkv_stride;

    // ---- loads that need no position, first: the prep's inputs (q / k / v
    // of the raw GEMV output and their QK-norm weights) and, when LIVE, the
    // step's RoPE row and -- for split 0, whose history always starts at row
    // 0 or later -- the first PD - 1 steps of rows from row 0 (the pre-scan;
    // rows outside the live range are masked once it is known).  The
    // position is a dependent device load (~1 us); everything that needs it
    // follows.  Vector loads return in order, so the prep waits only for the
    // loads issued before its own last one: without LIVE its table row goes
    // out after pos, and there is no pre-scan for it to wait behind.
    constexpr int NV = (G + 1 + W - 1) / W;   // prep vectors per wave
    float pv[NV][EPL], pn[NV][EPL], rc[EPL], rs[EPL];
    // Branch-free: every lane loads (a wave past the G + 1 vectors reloads k;
    // without norm weights the vector itself is loaded and ignored), so the
    // wait counts before the prep cover these loads only, not the K/V steps
    // issued after them.
    const float* nq = a.q_norm, *nk = a.k_norm;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int vi = min(wave + n * W, G);            // wave-uniform
        const bool isq = vi < G;
        const float* src = qkv + (isq ? (long)(kvh * G + vi) * HD : (long)(a.n_heads + kvh) * HD);
        const float* nw = isq ? (nq ? nq + (long)(kvh * G + vi) * HD : nullptr)
                              : (nk ? nk + (long)kvh * HD : nullptr);
        const float* nsrc = nw ? nw : src;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            pv[n][j] = src[lane + 64 * j];
            const float w = nsrc[lane + 64 * j];
            pn[n][j] = nw ? w : 1.f;
        }
    }
    const float vnew = qkv[(long)(a.n_heads + a.n_kv + kvh) * HD + (threadIdx.x & (HD - 1))];
    // the rotate-half partner table index of each of the lane's elements
    auto rope_idx = [&](int j) {
        const int e = lane + 64 * j;
        return e < HD / 2 ? e : e - HD / 2;
    };
    const bool pre_on = LIVE && split == 0;
    const int pre_rows = pre_on ? min((PD - 1) * S, a.max_rows) : 0;
    ScanState<HD, PD> pre;
    int pos;
    if constexpr (LIVE) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            rc[j] = a.rope_row[rope_idx(j)];
            rs[j] = a.rope_row[HD / 2 + rope_idx(j)];
        }
        // pos as a vector load behind the prep's loads and ahead of the
        // pre-scan's (loads return in order: it arrives before the K/V rows);
        // a scalar load would make the next scalar wait cover it
        const __amdgpu_buffer_rsrc_t pb =
            __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.pos_dev), (short)0, 4, 0x00020000);
        const int pos_v = __builtin_amdgcn_raw_buffer_load_b32(pb, 0, 0, 0);
        // unconditional (split > 0: an empty range, zeros, no traffic)
        __builtin_amdgcn_sched_barrier(0);
        scan_start<HD, 4 * W, PD>(pre, a.k_cache + (long)kvh * HD, a.v_cache + (long)kvh * HD,
                                  kv_stride, lane_dim(dl, 0), 0, pre_rows, wave * 4 + row);
        __builtin_amdgcn_sched_barrier(0);
        pos = __builtin_amdgcn_readfirstlane(pos_v);
    } else {
        pos = a.pos_dev[seq];
    }

    const int slot = LIVE ? 0 : (a.slot_dev ? a.slot_dev[seq] : 0);
    const int t_lo = (a.window > 0 && pos >= a.window) ? pos - a.window + 1 : 0;
    const int ctx = pos - t_lo + 1;
    // active splits: all gridDim.y, the measured rule for the live context,
    // or one per min_chunk positions of it (the grid is fixed when a decode
    // step is captured once and replayed at every position; surplus blocks
    // leave here)
    int n_splits = gridDim.y;
    if (a.adaptive)
        n_splits = min(n_splits, attn_fused_splits_for(a.n_kv * (LIVE ? 1 : (int)gridDim.z), ctx));
    else if (a.min_chunk > 0) n_splits = min(n_splits, max(1, (ctx + a.min_chunk - 1) / a.min_chunk));
    if (split >= n_splits) return;
    const int chunk = (ctx + n_splits - 1) / n_splits;
    const int b0 = t_lo + split * chunk;
    const int b1 = min(pos + 1, b0 + chunk);
    const bool owner = b0 <= pos && pos < b0 + chunk;
    const int e1 = min(b1, pos);              // cache rows [b0, e1) are read here
    float* kc = a.k_cache + (long)slot * a.slot_stride;
    float* vc = a.v_cache + (long)slot * a.slot_stride;

    if constexpr (!LIVE) {
        // the RoPE row of pos
        const float* cr = a.cos_tab + (long)pos * (HD / 2);
        const float* sr = a.sin_tab + (long)pos * (HD / 2);
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            rc[j] = cr[rope_idx(j)];
            rs[j] = sr[rope_idx(j)];
        }
    }
    // the history scan proper: rows [b0, e1), less the pre-scan's
    __builtin_amdgcn_sched_barrier(0);
    ScanState<HD, PD> scan;
    scan_start<HD, 4 * W, PD>(scan, kc + (long)kvh * HD, vc + (long)kvh * HD, kv_stride,
                              lane_dim(dl, 0), pre_on ? max(b0, pre_rows) : b0, e1, wave * 4 + row);
    __builtin_amdgcn_sched_barrier(0);

    __shared__ float sq[G][HD], sk[HD], sv[HD];
    // ---- prep: QK-norm + RoPE of the G q heads and k, wave per vector -----
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int vi = wave + n * W;
        if (vi >= G + 1) continue;                     // wave-uniform
        const bool isq = vi < G;
        const bool normed = isq ? nq != nullptr : nk != nullptr;
        float v[EPL];
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            v[j] = pv[n][j];
            ss += v[j] * v[j];
        }
        if (normed) {
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)HD + a.qk_eps);
#pragma unroll
            for (int j = 0; j < EPL; ++j) v[j] = v[j] * inv * pn[n][j];
        }
        float r[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            if constexpr (HD == 64) {
                const float other = __shfl_xor(v[j], 32, 64);   // partner e +- 32
                r[j] = lane < 32 ? v[j] * rc[j] - other * rs[j] : other * rs[j] + v[j] * rc[j];
            } else {
                constexpr int HJ = EPL / 2;                     // partner is j +- HJ
                r[j] = j < HJ ? v[j] * rc[j] - v[j + HJ] * rs[j]
                              : v[j - HJ] * rs[j] + v[j] * rc[j];
            }
        }
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            if (isq) sq[vi][e] = r[j] * (a.scale * LOG2E);
            else sk[e] = r[j];
        }
    }
    if (threadIdx.x < HD) sv[threadIdx.x] = vnew;
    __syncthreads();
    if (owner) {
        for (int e = threadIdx.x; e < HD; e += 64 * W) {
            kc[(long)pos * kv_stride + (long)kvh * HD + e] = sk[e];
            vc[(long)pos * kv_stride + (long)kvh * HD + e] = sv[e];
        }
    }

    float q[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < DPL; ++d) q[h][d] = sq[h][lane_dim(dl, d)];
    float m[G], l[G], o[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY; l[h] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[h][d] = 0.f;
    }

    if (LIVE && pre_on) {
#pragma unroll
        for (int i = 0; i < PD - 1; ++i)
            scan_update_masked<HD, G>(q, m, l, o, pre.k[i], pre.v[i], pre.t + i * S, b0, e1);
    }
    scan_run<HD, G, 4 * W, PD>(scan, e1, q, m, l, o);
    if (owner && wave == 0 && row == 0) {
        // position pos from LDS (the 16 lanes of row 0 of wave 0)
        constexpr int P = ScanShape<HD>::P;
        float kf[P][DPL], vf[P][DPL];
#pragma unroll
        for (int i = 0; i < P; ++i)
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                kf[i][d] = sk[lane_dim(dl, d)];
                vf[i][d] = sv[lane_dim(dl, d)];
            }
        scan_update<HD, G>(q, m, l, o, kf, vf, 0, 1);
    }

    // ---- merge the block's 16 (wave, row) states (first by lane shuffles
    // within each wave when G is small) through LDS ------------------------------
    constexpr int NS = block_states<G, W>();
    __shared__ float s_m[NS][G], s_l[NS][G];
    __shared__ float s_o[NS][G][HD];
    __shared__ int s_last;
    stage_block_states<HD, G, W>(m, l, o, wave, row, dl, s_m, s_l, s_o);
    __syncthreads();
    // each sequence owns n_heads * gridDim.y partial slots (its active split
    // count may be smaller and differs between sequences)
    const long pbase = (long)seq * a.n_heads * gridDim.y;
    for (int e = threadIdx.x; e < G * HD; e += 64 * W) {
        const int h = e / HD, d = e % HD;
        float mx = -INFINITY;
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) mx = fmaxf(mx, s_m[s2][h]);
        float lsum = 0.f, osum = 0.f;
        if (mx != -INFINITY) {
#pragma unroll
            for (int s2 = 0; s2 < NS; ++s2) {
                const float w = exp2f(s_m[s2][h] - mx);
                lsum += s_l[s2][h] * w;
                osum += s_o[s2][h][d] * w;
            }
        }
        const int qh = kvh * G + h;
        if (n_splits == 1) {
            a.out[(long)seq * a.out_stride + (long)qh * HD + d] = osum / lsum;
        } else {
            // agent-scope stores (sc1): they reach memory past this XCD's L2,
            // so a block on another XCD reads them without the L2 write-back
            // a device-scope release fence would cost
            const long pi = pbase + (long)qh * n_splits + split;
            __hip_atomic_store(&a.part_o[pi * HD + d], osum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(&a.part_m[pi], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&a.part_l[pi], lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (n_splits == 1) return;
    // ---- the last block of this (seq, kv head) merges the splits -------------
    // Every thread's partial stores have completed (vmcnt 0) before the block
    // bumps the counter, so the block that sees n_splits - 1 earlier arrivals
    // reads complete partials with agent-scope (sc1) loads.
    __builtin_amdgcn_s_waitcnt(0x0F70);        // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(&a.counters[seq * a.n_kv + kvh], 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == n_splits - 1;
    }
    __syncthreads();
    if (!s_last) return;
    merge_splits<HD, G, 64 * W>(a.part_m + pbase, a.part_l + pbase, a.part_o + pbase * HD, n_splits,
                                kvh, a.out + (long)seq * a.out_stride);
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[seq * a.n_kv + kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waves per block.  Measured on MI355X at the 7B and GQA-32/8 shapes, ctx
// 128..16384: 8-wave blocks (twice the K/V rows in flight per block) run
// 10-35% slower than 4-wave blocks at every split count, so 4 it is.
template <int HD, int G> constexpr int attn_waves() { return 4; }

template <int HD, int G>
static int launch_fused(const AttnFusedArgs& a, int n_splits, int n_seq, hipStream_t st) {
    constexpr int W = attn_waves<HD, G>();
    if (a.rope_row)
        hipLaunchKernelGGL((attn_fused_kernel<HD, G, W, kFusedScanDepth, true>),
                           dim3(a.n_kv, n_splits, n_seq), dim3(64 * W), 0, st, a);
    else
        hipLaunchKernelGGL((attn_fused_kernel<HD, G, W, kFusedScanDepth, false>),
                           dim3(a.n_kv, n_splits, n_seq), dim3(64 * W), 0, st, a);
    ATLAS_LAUNCH_CHECK("attn_fused");
    return ATLAS_OK;
}

bool attn_fused_supported(int n_heads, int n_kv, int head_dim) {
    if (n_kv <= 0 || n_heads % n_kv) return false;
    const int G = n_heads / n_kv;
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
           (G == 1 || G == 2 || G == 4 || G == 8) && !(head_dim == 256 && G == 8);
}

int attn_fused_launch(const AttnFusedArgs& a, int n_splits, int n_seq, hipStream_t st) {
    ATLAS_REQUIRE(attn_fused_supported(a.n_heads, a.n_kv, a.head_dim),
                  "attention: fused path needs head_dim 64/128/256 and group 1/2/4/8");
    ATLAS_REQUIRE(a.qkv && a.k_cache && a.v_cache && a.out && a.pos_dev && a.cos_tab && a.sin_tab,
                  "attention: null pointer");
    ATLAS_REQUIRE(n_splits == 1 || (a.part_m && a.part_l && a.part_o && a.counters),
                  "attention: split partials missing");
    ATLAS_REQUIRE(n_seq >= 1 && n_splits >= 1, "attention: empty grid");
    ATLAS_REQUIRE(!a.rope_row || (n_seq == 1 && !a.slot_dev),
                  "attention: a live RoPE row serves one sequence in slot 0");
    ATLAS_REQUIRE(n_splits <= kAttnFusedMaxSplits, "attention: %d splits > %d", n_splits,
                  kAttnFusedMaxSplits);
    ATLAS_REQUIRE(attn_rows_fit(a.max_rows, a.n_kv, a.head_dim),
                  "attention: %d cache rows of %d x %d exceed 32-bit offsets", a.max_rows, a.n_kv,
                  a.head_dim);
    const uintptr_t al = (uintptr_t)a.qkv | (uintptr_t)a.k_cache | (uintptr_t)a.v_cache;
    ATLAS_REQUIRE((al & 15) == 0 && a.qkv_stride % 4 == 0 && a.slot_stride % 4 == 0,
                  "attention: 16-byte alignment");
    const int G = a.n_heads / a.n_kv;
#define ATLAS_FUSED_CASE(HDV, GV) \
    if (a.head_dim == HDV && G == GV) return launch_fused<HDV, GV>(a, n_splits, n_seq, st);
    ATLAS_FUSED_CASE(128, 1) ATLAS_FUSED_CASE(128, 2) ATLAS_FUSED_CASE(128, 4) ATLAS_FUSED_CASE(128, 8)
    ATLAS_FUSED_CASE(64, 1)  ATLAS_FUSED_CASE(64, 2)  ATLAS_FUSED_CASE(64, 4)  ATLAS_FUSED_CASE(64, 8)
    ATLAS_FUSED_CASE(256, 1) ATLAS_FUSED_CASE(256, 2) ATLAS_FUSED_CASE(256, 4)
#undef ATLAS_FUSED_CASE
    set_error(ATLAS_EUNSUPPORTED, "attention: fused shape");
    return ATLAS_EUNSUPPORTED;
}

// ---------------------------------------------------------------------------

int attn_max_splits(int n_kv) {
    // At most 256 blocks: with the partials published by sc1 stores (no L2
    // write-back per block) the GQA 32/8/128 shape keeps gaining up to 32
    // splits at ctx 16384, and no measured shape gains past 256 blocks.
    const int s = 256 / (n_kv > 0 ? n_kv : 1);
    return s < 1 ? 1 : (s > kAttnFusedMaxSplits ? kAttnFusedMaxSplits : s);
}

int attn_pick_splits_unfused(int n_kv, int ctx) { return attn_splits_for(n_kv, ctx); }

int attn_pick_splits(int n_kv, int max_ctx) {
    // the fused rule at the longest context (its split count only grows with
    // ctx past the one-split range), within attn_max_splits
    const int s = attn_fused_splits_for(n_kv, max_ctx);
    const int cap = attn_max_splits(n_kv);
    return s < cap ? s : cap;
}

template <int HD, int G>
static int launch_split(AttnArgs a, int n_splits, hipStream_t st, int n_seq = 1) {
    constexpr int W = attn_waves<HD, G>();
    hipLaunchKernelGGL((attn_split_kernel<HD, G, W>), dim3(a.n_kv, n_splits, n_seq), dim3(64 * W),
                       0, st, a);
    ATLAS_LAUNCH_CHECK("attn_split");
    if (n_splits > 1 && !a.counters) {
        hipLaunchKernelGGL(attn_combine_kernel, dim3(a.n_heads, n_seq), dim3(HD < 256 ? HD : 256), 0, st,
                           a, n_splits, HD);
        ATLAS_LAUNCH_CHECK("attn_combine");
    }
    return ATLAS_OK;
}

int attn_launch(AttnArgs a, int n_splits, hipStream_t st) {
    ATLAS_REQUIRE(a.n_heads > 0 && a.n_kv > 0 && a.n_heads % a.n_kv == 0,
                  "attention: n_heads %d not a multiple of n_kv %d", a.n_heads, a.n_kv);
    ATLAS_REQUIRE(a.head_dim > 0 && a.head_dim <= 256, "attention: head_dim %d", a.head_dim);
    ATLAS_REQUIRE(a.pos_dev || a.pos >= 0, "attention: pos < 0");
    ATLAS_REQUIRE(a.q && a.k_cache && a.v_cache && a.out, "attention: null pointer");
    const int G = a.n_heads / a.n_kv;
    const bool aligned =
        (((uintptr_t)a.q | (uintptr_t)a.k_cache | (uintptr_t)a.v_cache) & 15) == 0;
    const bool fast = aligned && (a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256) &&
                      (G == 1 || G == 2 || G == 4 || G == 8) &&
                      attn_rows_fit(a.max_rows, a.n_kv, a.head_dim);
    if (!fast) {
        hipLaunchKernelGGL(attn_generic_kernel, dim3(a.n_heads), dim3(256), 0, st, a, a.head_dim);
        ATLAS_LAUNCH_CHECK("attn_generic");
        return ATLAS_OK;
    }
    if (n_splits < 1) n_splits = 1;
    if (n_splits > kAttnMaxSplits) n_splits = kAttnMaxSplits;
    if (n_splits > 1 && !a.part_m) {
        // the calling thread's scratch (no model owns this call)
        void* p = nullptr;
        const size_t need = (size_t)a.n_heads * n_splits * (a.head_dim + 2) * sizeof(float);
        int rc = thread_scratch(SCR_ATTN, need, &p);
        if (rc) return rc;
        float* part = static_cast<float*>(p);
        a.part_m = part;
        a.part_l = part + (size_t)a.n_heads * n_splits;
        a.part_o = part + (size_t)2 * a.n_heads * n_splits;
    }
    ATLAS_REQUIRE(n_splits == 1 || (a.part_l && a.part_o), "attention: partial buffers missing");
    ATLAS_REQUIRE(!a.counters || n_splits <= kAttnFusedMaxSplits,
                  "attention: %d splits > %d for the one-launch merge", n_splits, kAttnFusedMaxSplits);
#define ATLAS_ATTN_CASE(HDV, GV) \
    if (a.head_dim == HDV && G == GV) return launch_split<HDV, GV>(a, n_splits, st);
    ATLAS_ATTN_CASE(128, 1) ATLAS_ATTN_CASE(128, 2) ATLAS_ATTN_CASE(128, 4) ATLAS_ATTN_CASE(128, 8)
    ATLAS_ATTN_CASE(64, 1)  ATLAS_ATTN_CASE(64, 2)  ATLAS_ATTN_CASE(64, 4)  ATLAS_ATTN_CASE(64, 8)
    ATLAS_ATTN_CASE(256, 1) ATLAS_ATTN_CASE(256, 2) ATLAS_ATTN_CASE(256, 4)
#undef ATLAS_ATTN_CASE
    hipLaunchKernelGGL(attn_generic_kernel, dim3(a.n_heads), dim3(256), 0, st, a, a.head_dim);
    ATLAS_LAUNCH_CHECK("attn_generic");
    return ATLAS_OK;
}

// ---------------------------------------------------------------------------
// Prompt chunk attention: n query rows of ONE sequence at consecutive
// positions pos_dev[0] .. + n - 1, all in cache slot slot_dev[0], whose K/V
// rows are already in the cache (the QK-norm / RoPE / KV-write kernel ran).
// Row j attends to positions [t_lo(p_j), p_j] with the reference's causal and
// sliding-window rule (crates/atlas-model/src/lib.rs:689-721): the same
// online softmax as attn_scan, but a block of 16 rows shares every K/V tile
// (32 positions staged once in LDS), so the history is read once per 16 rows
// instead of once per row.  Grid (n_heads, ceil(n / 16)), 16 waves: wave w
// serves rows 16-lane group by group (w % 4: four rows) over the tile
// positions 8 (w / 4) .. + 7; the four partial states of a row meet in LDS at
// the end.  (With one 4-wave block per CU the dependent DPP / exp chains had
// nothing to hide behind: 166 us per launch at 2047-token prompts.)
constexpr int APF_ROWS = 16, APF_TK = 32, APF_KS = 4;

__global__ __launch_bounds__(1024) void attn_prefill_kernel(AttnArgs a, int n) {
    constexpr int HD = 128, DPL = HD / 16, PPS = APF_TK / APF_KS;   // positions per split
    constexpr float LOG2E = 1.4426950408889634f;
    __shared__ f32x4 tk[APF_TK][HD / 4], tv[APF_TK][HD / 4];
    __shared__ float s_m[APF_KS][APF_ROWS], s_l[APF_KS][APF_ROWS];
    __shared__ float s_o[APF_KS][APF_ROWS][HD];
    const int qh = blockIdx.x, G = a.n_heads / a.n_kv, kvh = qh / G;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int dl = lane & 15, gi = (wave & 3) * 4 + (lane >> 4), ks = wave >> 2;
    const int p0 = a.pos_dev[0];
    const long kv_stride = (long)a.n_kv * HD;
    const float* kb = a.k_cache + (long)a.slot_dev[0] * a.slot_stride + (long)kvh * HD;
    const float* vb = a.v_cache + (long)a.slot_dev[0] * a.slot_stride + (long)kvh * HD;
    const int r0 = blockIdx.y * APF_ROWS;
    const int j = r0 + gi;                                      // this group's row
    const int pj = p0 + min(j, n - 1);
    const int loj = (a.window > 0 && pj >= a.window) ? pj - a.window + 1 : 0;
    // the block's position range: the first row's window start .. its last row
    const int pf = p0 + r0, pl = p0 + min(r0 + APF_ROWS, n) - 1;
    const int lo_b = (a.window > 0 && pf >= a.window) ? pf - a.window + 1 : 0;
    const int ntiles = (pl - lo_b) / APF_TK + 1;

    // q of this row, scaled into exp2 space
    float q[DPL];
    {
        const float* qr = a.q + (long)min(j, n - 1) * a.q_stride + (long)qh * HD;
        const float sc = a.scale * LOG2E;
#pragma unroll
        for (int d = 0; d < DPL; d += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(qr + lane_dim(dl, d));
            q[d] = v.x * sc; q[d + 1] = v.y * sc; q[d + 2] = v.z * sc; q[d + 3] = v.w * sc;
        }
    }
    // tile loads: 2 x 32 rows x 32 pieces = 2048 pieces, 2 per thread
    f32x4 pre[2];
    auto fetch = [&](int t0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = (int)threadIdx.x + 1024 * i;
            const int r = (idx >> 5) & (APF_TK - 1), c = idx & 31;
            const long row = min(t0 + r, pl);                   // rows past pl: masked
            pre[i] = *reinterpret_cast<const f32x4*>((i == 0 ? kb : vb) + row * kv_stride + 4 * c);
        }
    };
    auto stash = [&]() {
        const int r = ((int)threadIdx.x >> 5) & (APF_TK - 1), c = threadIdx.x & 31;
        tk[r][c] = pre[0];
        tv[r][c] = pre[1];
    };
    float m = -INFINITY, l = 0.f, o[DPL];
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[d] = 0.f;
    fetch(lo_b);
    stash();
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {            // block-uniform trip count
        const int t0 = lo_b + it * APF_TK;
        if (it + 1 < ntiles) fetch(t0 + APF_TK);
#pragma unroll
        for (int s2 = ks * PPS; s2 < ks * PPS + PPS; s2 += 2) {
            float sv[2], vf[2][DPL];
            float smax = -INFINITY;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int t = t0 + s2 + i;
                const f32x4 k0 = tk[s2 + i][dl], k1 = tk[s2 + i][16 + dl];
                const f32x4 v0 = tv[s2 + i][dl], v1 = tv[s2 + i][16 + dl];
                float acc = q[0] * k0.x;
                acc += q[1] * k0.y; acc += q[2] * k0.z; acc += q[3] * k0.w;
                acc += q[4] * k1.x; acc += q[5] * k1.y; acc += q[6] * k1.z; acc += q[7] * k1.w;
                acc = row16_sum(acc);
                sv[i] = (t >= loj && t <= pj) ? acc : -INFINITY;
                smax = fmaxf(smax, sv[i]);
                vf[i][0] = v0.x; vf[i][1] = v0.y; vf[i][2] = v0.z; vf[i][3] = v0.w;
                vf[i][4] = v1.x; vf[i][5] = v1.y; vf[i][6] = v1.z; vf[i][7] = v1.w;
            }
            if (smax != -INFINITY) {
                const float mn = fmaxf(m, smax);
                const float corr = m == -INFINITY ? 0.f : exp2f(m - mn);
                const float e0 = sv[0] == -INFINITY ? 0.f : exp2f(sv[0] - mn);
                const float e1 = sv[1] == -INFINITY ? 0.f : exp2f(sv[1] - mn);
                l = l * corr + e0 + e1;
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[d] = o[d] * corr + e0 * vf[0][d] + e1 * vf[1][d];
                m = mn;
            }
        }
        __syncthreads();
        if (it + 1 < ntiles) {
            stash();
            __syncthreads();
        }
    }
    // ---- merge the four key splits of each row
    if (dl == 0) { s_m[ks][gi] = m; s_l[ks][gi] = l; }
#pragma unroll
    for (int d = 0; d < DPL; ++d) s_o[ks][gi][lane_dim(dl, d)] = o[d];
    __syncthreads();
    for (int e = threadIdx.x; e < APF_ROWS * HD; e += 1024) {
        const int r = e / HD, d = e % HD, jr = r0 + r;
        if (jr >= n) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int k2 = 0; k2 < APF_KS; ++k2) mx = fmaxf(mx, s_m[k2][r]);
        float lsum = 0.f, osum = 0.f;
#pragma unroll
        for (int k2 = 0; k2 < APF_KS; ++k2) {
            const float w = s_m[k2][r] == -INFINITY ? 0.f : exp2f(s_m[k2][r] - mx);
            lsum += s_l[k2][r] * w;
            osum += s_o[k2][r][d] * w;
        }
        const float v = osum / lsum;
        const long off = (long)jr * a.out_stride + (long)qh * HD + d;
        if (a.out_split) {
            // bf16 hi = the top 16 bits, lo = the rest rounded to nearest even
            const uint32_t u = __float_as_uint(v);
            const uint32_t ur = __float_as_uint(v - __uint_as_float(u & 0xFFFF0000u));
            a.out_split[off] = (uint16_t)(u >> 16);
            a.out_split[a.split_lo + off] = (uint16_t)((ur + 0x7FFFu + ((ur >> 16) & 1u)) >> 16);
        } else {
            a.out[off] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// The prompt chunk's attention on the matrix cores: f32 v_mfma_f32_16x16x4f32
// (exact f32 products, as the VALU kernel above), flash-attention style.
//  * a block of NW waves takes 16 NW consecutive rows of one query head (wave
//    w: rows 16 w .. 16 w + 15) and streams the K/V tiles of 32 positions its
//    rows need through LDS once for all its waves (NW = 4: the VALU kernel
//    re-reads every tile per 16 rows);
//  * S = Q K^T per tile: two 16 x 16 position blocks, 32 k steps of 4 dims
//    each.  The reduction over the 128 dims may go in any order, so k step s
//    takes dim 32 g + s from lane group g: a lane's Q stays in 32 registers and
//    its K row segment is 8 contiguous 16-byte LDS reads;
//  * online softmax per row in the accumulator layout (lane l holds rows
//    4 (l / 16) + i, i < 4, of column l % 16), with 16-lane DPP reductions;
//  * P goes through LDS to the A-operand layout, then O += P V: eight 16-dim
//    blocks, 8 k steps of 4 positions.
// Operand layouts (checked on MI355X): A lane l = A[l % 16][l / 16], B lane l =
// B[l / 16][l % 16], D lane l register i = D[4 (l / 16) + i][l % 16].
constexpr int APM_TK = 32;

__device__ __forceinline__ float row16_max(float v) {
    int x = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false)));
    x = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false)));
    x = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false)));
    x = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false)));
    return v;
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void attn_prefill_mfma_kernel(AttnArgs a, int n) {
    constexpr int HD = 128, TK = APM_TK, NT = 64 * NW, PER = 1024 / NT, ROWS = 16 * NW;
    constexpr int KP = HD + 4, VP = HD + 16, PP = TK + 4;          // padded LDS rows
    constexpr float LOG2E = 1.4426950408889634f;
    __shared__ __align__(16) float tk[TK][KP];
    __shared__ __align__(16) float tv[TK][VP];
    __shared__ __align__(16) float tp[NW][16][PP];
    const int qh = blockIdx.x, G = a.n_heads / a.n_kv, kvh = qh / G;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int p0 = a.pos_dev[0];
    const long kv_stride = (long)a.n_kv * HD;
    const float* kb = a.k_cache + (long)a.slot_dev[0] * a.slot_stride + (long)kvh * HD;
    const float* vb = a.v_cache + (long)a.slot_dev[0] * a.slot_stride + (long)kvh * HD;
    const int r0 = blockIdx.y * ROWS, rw = r0 + 16 * w;
    // the block's position range: its first row's window start .. its last row
    const int pf = p0 + r0, pl = p0 + min(r0 + ROWS, n) - 1;
    const int lo_b = (a.window > 0 && pf >= a.window) ? pf - a.window + 1 : 0;
    const int ntiles = (pl - lo_b) / TK + 1;

    // A operand of k step s: Q[row lr][32 lg + s], scaled into exp2 space
    float q[32];
    {
        const float* qr = a.q + (long)min(rw + lr, n - 1) * a.q_stride + (long)qh * HD + 32 * lg;
        const float sc = a.scale * LOG2E;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(qr + 4 * c);
            q[4 * c] = v.x * sc; q[4 * c + 1] = v.y * sc; q[4 * c + 2] = v.z * sc; q[4 * c + 3] = v.w * sc;
        }
    }
    // this lane's accumulator rows 4 lg + i: their positions and window starts
    int prow[4], lorow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        prow[i] = p0 + min(rw + 4 * lg + i, n - 1);
        lorow[i] = (a.window > 0 && prow[i] >= a.window) ? prow[i] - a.window + 1 : 0;
    }
    float m[4], l[4];
    f32x4 o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) { m[i] = -INFINITY; l[i] = 0.f; }
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

    // tile loads: 32 rows x 32 pieces of K and of V, PER + PER pieces per
    // thread; rows past pl read row pl (their scores are masked)
    f32x4 pk[PER], pv[PER];
    auto fetch = [&](int t0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = (int)threadIdx.x + NT * i;
            const int r = idx >> 5, c = idx & 31;
            const long row = min(t0 + r, pl);
            pk[i] = *reinterpret_cast<const f32x4*>(kb + row * kv_stride + 4 * c);
            pv[i] = *reinterpret_cast<const f32x4*>(vb + row * kv_stride + 4 * c);
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = (int)threadIdx.x + NT * i;
            const int r = idx >> 5, c = idx & 31;
            *reinterpret_cast<f32x4*>(&tk[r][4 * c]) = pk[i];
            *reinterpret_cast<f32x4*>(&tv[r][4 * c]) = pv[i];
        }
    };
    fetch(lo_b);
    stash();
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {            // block-uniform trip count
        const int t0 = lo_b + it * TK;
        if (it + 1 < ntiles) fetch(t0 + TK);
        // S = Q K^T over two 16-position blocks
        f32x4 sacc[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            sacc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
            const float* kr = &tk[16 * nt + lr][32 * lg];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const f32x4 kv4 = *reinterpret_cast<const f32x4*>(kr + 4 * c);
                sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * c], kv4.x, sacc[nt], 0, 0, 0);
                sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * c + 1], kv4.y, sacc[nt], 0, 0, 0);
                sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * c + 2], kv4.z, sacc[nt], 0, 0, 0);
                sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(q[4 * c + 3], kv4.w, sacc[nt], 0, 0, 0);
            }
        }
        // online softmax of rows 4 lg + i (columns: positions t0 + 16 nt + lr)
        float pr[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sv[2];
            float mx = -INFINITY;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int t = t0 + 16 * nt + lr;
                sv[nt] = (t >= lorow[i] && t <= prow[i]) ? sacc[nt][i] : -INFINITY;
                mx = fmaxf(mx, sv[nt]);
            }
            mx = row16_max(mx);
            const float mn = fmaxf(m[i], mx);
            float alpha = 1.f, ps = 0.f;
            if (mn != -INFINITY) {
                alpha = m[i] == -INFINITY ? 0.f : exp2f(m[i] - mn);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    pr[nt][i] = sv[nt] == -INFINITY ? 0.f : exp2f(sv[nt] - mn);
                    ps += pr[nt][i];
                }
                m[i] = mn;
            } else {
                pr[0][i] = 0.f;
                pr[1][i] = 0.f;
            }
            ps = row16_sum(ps);
            l[i] = l[i] * alpha + ps;
#pragma unroll
            for (int d = 0; d < 8; ++d) o[d][i] *= alpha;
        }
        // P (16 rows x 32 positions of this wave) to the A-operand layout
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) tp[w][4 * lg + i][16 * nt + lr] = pr[nt][i];
        __syncthreads();
        // O += P V: k step s takes positions 4 s .. 4 s + 3 (lane group lg: 4 s + lg)
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float pa = tp[w][lr][4 * s + lg];
            const float* vr = &tv[4 * s + lg][lr];
#pragma unroll
            for (int d = 0; d < 8; ++d)
                o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vr[16 * d], o[d], 0, 0, 0);
        }
        __syncthreads();                 // every wave is done with this tile's K, V and P
        if (it + 1 < ntiles) {
            stash();
            __syncthreads();
        }
    }
    // rows 4 lg + i of the wave, columns 16 d + lr
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int jr = rw + 4 * lg + i;
        if (jr >= n) continue;
        const float inv = 1.0f / l[i];
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const float v = o[d][i] * inv;
            const long off = (long)jr * a.out_stride + (long)qh * HD + 16 * d + lr;
            if (a.out_split) {
                const uint32_t u = __float_as_uint(v);
                const uint32_t ur = __float_as_uint(v - __uint_as_float(u & 0xFFFF0000u));
                a.out_split[off] = (uint16_t)(u >> 16);
                a.out_split[a.split_lo + off] = (uint16_t)((ur + 0x7FFFu + ((ur >> 16) & 1u)) >> 16);
            } else {
                a.out[off] = v;
            }
        }
    }
}

bool attn_prefill_ok(const AttnArgs& a) {
    const uintptr_t al = (uintptr_t)a.q | (uintptr_t)a.k_cache | (uintptr_t)a.v_cache |
                         (uintptr_t)a.out;
    return a.head_dim == 128 && a.n_kv > 0 && a.n_heads % a.n_kv == 0 && (al & 15) == 0 &&
           a.q_stride % 4 == 0 && a.out_stride % 4 == 0 && a.slot_stride % 4 == 0 &&
           a.pos_dev && a.slot_dev && attn_rows_fit(a.max_rows, a.n_kv, a.head_dim);
}

int attn_prefill_launch(const AttnArgs& a, int n, hipStream_t st) {
    ATLAS_REQUIRE(attn_prefill_ok(a) && n >= 1, "attention: prompt-chunk kernel needs head_dim 128, "
                  "16-byte alignment and device positions/slot (n %d)", n);
    // Chunks above 128 rows: the matrix-core kernel, 64 rows per block (7B
    // bf16, 2047-token prompt in 512-row chunks: 109.5 -> 76.3 ms).  Up to 128
    // rows the VALU kernel's 16-row blocks fill more of the chip: the MFMA
    // kernel with 64-, 32- or 16-row blocks made the 127-token prompt 0.1-0.3 ms
    // slower.
    if (n > 128)
        hipLaunchKernelGGL(attn_prefill_mfma_kernel<4>, dim3(a.n_heads, (n + 63) / 64), dim3(256), 0, st,
                           a, n);
    else
        hipLaunchKernelGGL(attn_prefill_kernel, dim3(a.n_heads, (n + APF_ROWS - 1) / APF_ROWS), dim3(1024),
                           0, st, a, n);
    ATLAS_LAUNCH_CHECK("attn_prefill");
    return ATLAS_OK;
}

int attn_batch_launch(const AttnArgs& a, int n_splits, int n_seq, hipStream_t st) {
    ATLAS_REQUIRE(attn_fused_supported(a.n_heads, a.n_kv, a.head_dim),
                  "attention: batch path needs head_dim 64/128/256 and group 1/2/4/8");
    ATLAS_REQUIRE(a.q && a.k_cache && a.v_cache && a.out && a.pos_dev, "attention: null pointer");
    ATLAS_REQUIRE(n_seq >= 1 && n_splits >= 1 && n_splits <= kAttnMaxSplits,
                  "attention: %d sequences x %d splits", n_seq, n_splits);
    ATLAS_REQUIRE(n_splits == 1 || (a.part_m && a.part_l && a.part_o),
                  "attention: split partials missing");
    ATLAS_REQUIRE(attn_rows_fit(a.max_rows, a.n_kv, a.head_dim),
                  "attention: %d cache rows of %d x %d exceed 32-bit offsets", a.max_rows, a.n_kv,
                  a.head_dim);
    const uintptr_t al = (uintptr_t)a.q | (uintptr_t)a.k_cache | (uintptr_t)a.v_cache;
    ATLAS_REQUIRE((al & 15) == 0 && a.q_stride % 4 == 0 && a.slot_stride % 4 == 0,
                  "attention: 16-byte alignment");
    const int G = a.n_heads / a.n_kv;
#define ATLAS_BATCH_CASE(HDV, GV) \
    if (a.head_dim == HDV && G == GV) return launch_split<HDV, GV>(a, n_splits, st, n_seq);
    ATLAS_BATCH_CASE(128, 1) ATLAS_BATCH_CASE(128, 2) ATLAS_BATCH_CASE(128, 4) ATLAS_BATCH_CASE(128, 8)
    ATLAS_BATCH_CASE(64, 1)  ATLAS_BATCH_CASE(64, 2)  ATLAS_BATCH_CASE(64, 4)  ATLAS_BATCH_CASE(64, 8)
    ATLAS_BATCH_CASE(256, 1) ATLAS_BATCH_CASE(256, 2) ATLAS_BATCH_CASE(256, 4)
#undef ATLAS_BATCH_CASE
    set_error(ATLAS_EUNSUPPORTED, "attention: batch shape");
    return ATLAS_EUNSUPPORTED;
}

// ---------------------------------------------------------------------------
// The no-allocation variant of atlas_decode_attention: its split partials live
// in `scratch`, a fixed device array of this file that every GPU holds until
// the process ends.  Host code never passes the array's name to a kernel (in
// host code it is only a stand-in for the symbol): the device address of each
// GPU's copy comes from hipGetSymbolAddress on the first call made on that
// device and is kept per device.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;     // 8 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kNoAllocDevices = 64;
static std::mutex g_noalloc_mu;
static float* g_noalloc_ptr[kNoAllocDevices] = {};

// device address of the current device's copy of `scratch` (resolved once)
static int noalloc_scratch(float** out) {
    int dev = 0;
    ATLAS_HIP(hipGetDevice(&dev));
    ATLAS_REQUIRE(dev >= 0 && dev < kNoAllocDevices, "decode_attention_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            set_error(ATLAS_EHIP, "decode_attention_noalloc: scratch symbol address: %s",
                      hipGetErrorString(e));
            return ATLAS_EHIP;
        }
        g_noalloc_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_noalloc_ptr[dev];
    return ATLAS_OK;
}

size_t attn_noalloc_max_bytes() { return kNoAllocScratchBytes; }

int attn_launch_noalloc(AttnArgs a, int n_splits, hipStream_t st) {
    if (n_splits < 1) n_splits = 1;
    if (n_splits > kAttnMaxSplits) n_splits = kAttnMaxSplits;
    if (n_splits > 1) {
        const size_t need = (size_t)a.n_heads * n_splits * (a.head_dim + 2) * sizeof(float);
        if (need > kNoAllocScratchBytes) {
            set_error(ATLAS_EINVAL,
                      "decode_attention_noalloc: %d heads x %d splits x (head_dim %d + 2) floats "
                      "need %zu bytes of partials, above the fixed %zu-byte workspace",
                      a.n_heads, n_splits, a.head_dim, need, kNoAllocScratchBytes);
            return ATLAS_EINVAL;
        }
        float* part = nullptr;
        const int rc = noalloc_scratch(&part);
        if (rc) return rc;
        a.part_m = part;
        a.part_l = part + (size_t)a.n_heads * n_splits;
        a.part_o = part + (size_t)2 * a.n_heads * n_splits;
    }
    return attn_launch(a, n_splits, st);
}

}  // namespace atlas
