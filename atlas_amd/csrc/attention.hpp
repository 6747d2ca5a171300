// attention.hpp -- launch interface of the decode attention kernels (internal).
#pragma once
#include "common.hpp"

namespace atlas {

struct AttnArgs {
    const float* q;          // [n_heads * head_dim]
    const float* k_cache;    // [max_seq][n_kv][head_dim]
    const float* v_cache;
    float* out;              // [n_heads * head_dim]
    int n_heads, n_kv, head_dim;
    int pos;                 // used when pos_dev == nullptr
    const int* pos_dev;      // device-resident position (graph replay)
    float scale;
    int window;              // 0 = full attention
    float* part_m;           // split partials: the caller's, or null for the calling thread's scratch
    float* part_l;
    float* part_o;
    int max_rows;            // cache rows that may be read (max_seq), > 0
    int adaptive;            // 1: active splits = min(grid, attn_batch_splits_for(n_kv,
                             // n_seq, ctx)) of the live context (a captured step
                             // replayed at any pos)
    // Batch (attn_batch_launch): sequence s reads q at q + s * q_stride, the
    // cache slot slot_dev[s] (k_cache + slot * slot_stride), position
    // pos_dev[s], and writes out + s * out_stride; its partials follow the
    // previous sequences' n_heads * n_splits slots.
    const int* slot_dev;
    long slot_stride;
    long q_stride, out_stride;
    // [n_seq][n_kv] merge counters, zero before the first launch, or null:
    // non-null, the splits merge in the block that finishes last (one launch,
    // at most kAttnFusedMaxSplits splits); null, attn_combine_kernel merges
    int* counters;
    // attn_prefill_launch only: non-null, row j's output goes instead to
    // out_split + j * out_stride (its bf16 hi part) and + split_lo (its lo
    // part), the input rows of the library GEMM that follows
    uint16_t* out_split;
    long split_lo;
};

// Fused QK-norm + RoPE + KV write + split-K attention + split merge.
struct AttnFusedArgs {
    const float* qkv;        // per sequence [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)]
    long qkv_stride;         // elements between sequences
    const float* q_norm;     // [n_heads*hd] or null
    const float* k_norm;     // [n_kv*hd] or null
    float qk_eps;
    const float* cos_tab;    // [max_seq x hd/2]
    const float* sin_tab;
    float* k_cache;          // [slots][max_seq][n_kv][hd]
    float* v_cache;
    long slot_stride;
    const int* slot_dev;     // [n_seq] or null (slot 0)
    const int* pos_dev;      // [n_seq]
    float* out;              // per sequence [n_heads*hd]
    long out_stride;
    int n_heads, n_kv, head_dim;
    float scale;
    int window;
    float* part_m;           // [n_seq][n_heads][n_splits]
    float* part_l;
    float* part_o;           // [n_seq][n_heads][n_splits][hd]
    int* counters;           // [n_seq][n_kv], zero before the first launch
    int min_chunk;           // > 0: active splits = min(grid, ceil(ctx / min_chunk))
    int adaptive;            // 1 (min_chunk ignored): active splits = min(grid,
                             // attn_fused_splits_for(n_kv * n_seq, ctx))
    int max_rows;            // cache rows per slot (max_seq), > 0
    const float* rope_row;   // [hd]: cos (hd/2) then sin (hd/2) at pos_dev[0], or null (the
                             // tables); one sequence in slot 0 only
};

// The scan addresses one KV head's rows with 32-bit byte offsets.
// Cache byte offsets are 32-bit.  A scan prefetches up to a few steps past
// its last row (those loads lie past the buffer's end and read zeros); the
// 1024 rows of headroom keep every such offset from wrapping around.
inline bool attn_rows_fit(long max_rows, int n_kv, int head_dim) {
    return max_rows > 0 && (max_rows + 1024) * (long)n_kv * head_dim * 4 <= 0xFFFFFFFFL;
}

// Positions per split below which another split costs more than it saves
// (one pipelined block scans ~512 rows in the time a split merge takes).
constexpr int kAttnSplitChunk = 512;

// split-count bounds: the two-kernel path's merge, and the fused kernel's
// in-kernel merge (its split weights live in LDS)
constexpr int kAttnMaxSplits = 256;
constexpr int kAttnFusedMaxSplits = 64;

// Split count of the two-kernel path for a live context ctx: at least ~128
// blocks while splits keep >= 32 positions, at most 512 positions per split,
// and at most 256 blocks (measured at the GQA 32/8/128 shape, ctx 512..16384).
__host__ __device__ inline int attn_splits_for(int n_kv, int ctx) {
    const int nkv = n_kv > 0 ? n_kv : 1;
    int s = (ctx + kAttnSplitChunk - 1) / kAttnSplitChunk;
    const int wide = 128 / nkv < (ctx + 31) / 32 ? 128 / nkv : (ctx + 31) / 32;
    if (wide > s) s = wide;
    const int cap = 256 / nkv > 1 ? 256 / nkv : 1;
    if (s > cap) s = cap;
    if (s > kAttnMaxSplits) s = kAttnMaxSplits;
    return s < 1 ? 1 : s;
}

// Split count of n_seq sequences of one batch step: one split per
// (sequence, KV head) once they make >= 128 blocks (then every extra split
// only adds merge work: measured at the 7B shape, 2..8 sequences, ctx
// 256..2048), else the single-sequence rule over the n_seq * n_kv streams.
__host__ __device__ inline int attn_batch_splits_for(int n_kv, int n_seq, int ctx) {
    if (n_seq <= 1) return attn_splits_for(n_kv, ctx);
    const int streams = n_kv * n_seq;
    return streams >= 128 ? 1 : attn_splits_for(streams, ctx);
}

// Split count of the fused kernel for a live context ctx over `streams`
// (sequence, KV head) pairs.  Fitted to a sweep on MI355X (the 7B shape
// 32/32/128 at ctx 150..4000, GQA 32/8/128 at ctx 512..16384): one split
// while 32+ streams each hold < 256 positions (the split merge then costs
// more than the scan it shortens), else one split per 512 positions, raised
// towards 128 blocks while splits keep >= 64 positions, at most 256 blocks.
__host__ __device__ inline int attn_fused_splits_for(int streams, int ctx) {
    const int ns = streams > 0 ? streams : 1;
    if (ns >= 32 && ctx < 256) return 1;
    int s = (ctx + kAttnSplitChunk - 1) / kAttnSplitChunk;
    const int wide = 128 / ns < ctx / 64 ? 128 / ns : ctx / 64;
    if (wide > s) s = wide;
    const int cap = 256 / ns > 1 ? 256 / ns : 1;
    if (s > cap) s = cap;
    if (s > kAttnFusedMaxSplits) s = kAttnFusedMaxSplits;
    return s < 1 ? 1 : s;
}

bool attn_fused_supported(int n_heads, int n_kv, int head_dim);
int attn_max_splits(int n_kv);
int attn_fused_launch(const AttnFusedArgs& a, int n_splits, int n_seq, hipStream_t st);
int attn_pick_splits(int n_kv, int max_ctx);
// split count of the two-kernel path (attn_launch) for a live context
int attn_pick_splits_unfused(int n_kv, int ctx);
int attn_launch(AttnArgs a, int n_splits, hipStream_t st);
// attn_launch with its split partials in the library's fixed device
// workspace (no allocation; concurrent calls on one GPU share it)
int attn_launch_noalloc(AttnArgs a, int n_splits, hipStream_t st);
size_t attn_noalloc_max_bytes();
// n_seq sequences of one batch step: split kernel (grid n_kv x n_splits x
// n_seq) and split merge, no generic fallback; partials are the caller's,
// [n_seq][n_heads][n_splits] (+ head_dim for part_o)
int attn_batch_launch(const AttnArgs& a, int n_splits, int n_seq, hipStream_t st);
// n prompt rows of one sequence at consecutive positions pos_dev[0].. in slot
// slot_dev[0] (q rows q_stride apart, out rows out_stride apart), K/V already
// written: query-tiled causal attention, head_dim 128
bool attn_prefill_ok(const AttnArgs& a);
int attn_prefill_launch(const AttnArgs& a, int n, hipStream_t st);

}  // namespace atlas
