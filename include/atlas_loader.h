/*
 * atlas_loader.h -- C ABI of the checkpoint loader: safetensors files and
 * HuggingFace config.json into device residency.
 *
 * Reference counterparts (crates/atlas-model/src/lib.rs):
 *   SafetensorsFile::open / from_bytes              2074-2125
 *   SafetensorsFile::tensor_names / len / contains / get_desc   2128-2150
 *   SafetensorsFile::get_bf16 / get_f32             2189-2239
 *   f16_to_f32                                      2243-2263
 *   load_model_from_safetensors                     2283-2359
 *   patch_config_from_hf_json                       2367-2432
 *   load_model_from_dir                             2437-2570
 * The JSON syntax and value semantics follow crates/atlas-json/src/lib.rs.
 *
 * Differences from the reference, all where it would panic or misbehave:
 * a data_offsets array with fewer than two entries, a byte range outside the
 * data section, a tensor whose element count does not match the model, and
 * QK-norm weights present for only some layers are errors (ATLAS_EINVAL)
 * instead of a panic or a silently inconsistent model, and so is JSON nested
 * deeper than 512 levels (the reference's recursive parser has no bound and
 * would overflow its stack).
 *
 * All entry points return 0 or a negative ATLAS_E* code (atlas_kernels.h);
 * atlas_last_error() has the message.
 */
#ifndef ATLAS_LOADER_H
#define ATLAS_LOADER_H

#include <stddef.h>
#include <stdint.h>

#include "atlas_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct atlas_st atlas_st;

/* SafetensorsFile::open: the file is memory-mapped (not read into memory). */
int atlas_st_open(const char* path, atlas_st** out);
/* SafetensorsFile::from_bytes: the bytes are copied. */
int atlas_st_from_bytes(const void* bytes, size_t n, atlas_st** out);
void atlas_st_close(atlas_st* st);
/* len(); -1 for NULL */
int atlas_st_count(const atlas_st* st);
/* index of the first tensor named `name` (contains / get_desc), or -1 */
int atlas_st_find(const atlas_st* st, const char* name);
/* TensorDesc of tensor `index` (header order); pointers live as long as st.
 * offsets: [start, end) within the data section.                           */
int atlas_st_desc(const atlas_st* st, int index, const char** name, const char** dtype,
                  int* ndim, const uint64_t** shape, uint64_t* offsets);
/* get_f32: F32, BF16 (bits << 16) or F16 (f16_to_f32) elements as f32.
 * out == NULL only reports the count in *n_out.                            */
int atlas_st_get_f32(const atlas_st* st, const char* name, float* out, size_t cap,
                     size_t* n_out);
/* get_bf16: the raw bf16 bits; ATLAS_EINVAL unless the dtype is BF16. */
int atlas_st_get_bf16(const atlas_st* st, const char* name, uint16_t* out, size_t cap,
                      size_t* n_out);
/* f16_to_f32 */
float atlas_f16_to_f32(uint16_t h);

/* patch_config_from_hf_json: overlays sliding_window, rope_scaling (YaRN),
 * rope_theta and rms_norm_eps onto *cfg.  layer_types: the first min(count,
 * cap) entries (1 = "sliding_attention", 0 = anything else) and the count in
 * *n_layer_types (-1 when the key is absent).  *eos_token_id is set when
 * eos_token_id is present (as u32), else left unchanged.                    */
int atlas_config_patch_hf_json(const char* path, atlas_model_config* cfg, uint8_t* layer_types,
                               int cap, int* n_layer_types, int64_t* eos_token_id);

/* load_model_from_safetensors: creates the model from *cfg with the
 * architecture the tensor names give -- post_norm when any name contains
 * "post_feedforward_layernorm", qk_norm when the layers hold
 * self_attn.{q,k}_norm.weight, vocab = embedding elements / d_model, the
 * lm_head tied to the embedding when the file has no lm_head.weight -- and
 * fills it (cfg->weight_format: bf16 bits stay exact, F32/F16 truncate to
 * bf16; int8/int4 quantise by the atlas-quant rules on the device).
 * Tensors the file lacks keep a random init; unknown names are ignored.     */
int atlas_model_load_safetensors(const char* path, const atlas_model_config* cfg,
                                 atlas_model** out);
/* load_model_from_dir: config.json (if present) patched over *cfg, then the
 * shards named in model.safetensors.index.json (every quoted string ending in
 * ".safetensors", sorted), or model.safetensors.  *eos_token_id receives
 * config.json's eos_token_id, or -1.                                        */
int atlas_model_load_dir(const char* dir, const atlas_model_config* cfg, atlas_model** out,
                         int64_t* eos_token_id);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_LOADER_H */
