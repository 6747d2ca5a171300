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
    float* part_m;           // split partials (library scratch)
    float* part_l;
    float* part_o;
};

int attn_pick_splits(int n_kv, int max_ctx);
int attn_reserve(int n_heads, int head_dim, int n_splits);
int attn_launch(AttnArgs a, int n_splits, hipStream_t st);

}  // namespace atlas
