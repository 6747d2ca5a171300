"""Test checkpoints: modelgen weights written as HuggingFace-named safetensors
files (the layout load_model_from_safetensors / load_model_from_dir read,
crates/atlas-model/src/lib.rs:2283-2570), with config.json and a shard index.

The writer is independent of the library's parser: header JSON from the
json module, data little-endian, offsets packed in the given order.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np


def safetensors_bytes(tensors, metadata=None) -> bytes:
    """tensors: [(name, dtype, shape, raw bytes)] in file order."""
    hdr, data = {}, bytearray()
    if metadata is not None:
        hdr["__metadata__"] = metadata
    for name, dtype, shape, raw in tensors:
        hdr[name] = {"dtype": dtype, "shape": list(shape),
                     "data_offsets": [len(data), len(data) + len(raw)]}
        data += raw
    h = json.dumps(hdr).encode()
    return struct.pack("<Q", len(h)) + h + bytes(data)


def _raw(arr, dtype):
    if dtype == "BF16":
        return np.ascontiguousarray(arr, "<u2").tobytes()
    if dtype == "F16":
        return np.ascontiguousarray(arr, "<f2").tobytes()
    return np.ascontiguousarray(arr, "<f4").tobytes()


def hf_tensors(W, naming="olmo3", tie=False, source="BF16", seed=0):
    """The model's tensors under HF names.  Matrices and the embedding:
    source "BF16" writes the bf16 bits; "F32" writes f32 values whose top 16
    bits are those bits (random low bits, so loading must truncate); "F16"
    writes float16(bf16 value).  Norm vectors are F32.  naming "olmo3":
    model.layers.N., post-norm names, QK-norm; "llama": layers.N.,
    input/post_attention norms, tok_embeddings / norm, no QK-norm."""
    rng = np.random.default_rng(seed)

    def mat(bits):
        bits = np.asarray(bits, np.uint16)
        if source == "BF16":
            return "BF16", bits
        if source == "F32":
            low = rng.integers(0, 1 << 16, bits.shape, dtype=np.uint32)
            return "F32", ((bits.astype(np.uint32) << 16) | low).view(np.float32)
        f = (bits.astype(np.uint32) << 16).view(np.float32)
        return "F16", f.astype(np.float16)

    out = []

    def put(name, kind_arr, shape):
        dt, arr = kind_arr
        out.append((name, dt, shape, _raw(arr, dt)))

    cfg = W["cfg"]
    d, V = cfg["d_model"], cfg["vocab"]
    pre = "model.layers." if naming == "olmo3" else "layers."
    put("model.embed_tokens.weight" if naming == "olmo3" else "tok_embeddings.weight",
        mat(W["embed_bits"]), (V, d))
    for li, lw in enumerate(W["layers"]):
        p = f"{pre}{li}."
        for n, hf in (("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"),
                      ("wv", "self_attn.v_proj"), ("wo", "self_attn.o_proj"),
                      ("w_gate", "mlp.gate_proj"), ("w_up", "mlp.up_proj"),
                      ("w_down", "mlp.down_proj")):
            bits = lw[n + "_stored"][1][0]
            put(p + hf + ".weight", mat(bits), bits.shape)
        if naming == "olmo3":
            put(p + "post_attention_layernorm.weight", ("F32", lw["attn_norm"]), (d,))
            put(p + "post_feedforward_layernorm.weight", ("F32", lw["ffn_norm"]), (d,))
            if lw["q_norm"] is not None:
                put(p + "self_attn.q_norm.weight", ("F32", lw["q_norm"]), lw["q_norm"].shape)
                put(p + "self_attn.k_norm.weight", ("F32", lw["k_norm"]), lw["k_norm"].shape)
        else:
            put(p + "input_layernorm.weight", ("F32", lw["attn_norm"]), (d,))
            put(p + "post_attention_layernorm.weight", ("F32", lw["ffn_norm"]), (d,))
    put("model.norm.weight" if naming == "olmo3" else "norm.weight", ("F32", W["final_norm"]), (d,))
    if not tie:
        put("lm_head.weight", mat(W["lm_head_stored"][1][0]), (V, d))
    return out


def olmo3_config_json(cfg, eos=None) -> dict:
    """config.json fields patch_config_from_hf_json reads (lib.rs:2367-2432)."""
    c = {"vocab_size": cfg["vocab"], "hidden_size": cfg["d_model"],
         "num_hidden_layers": cfg["n_layers"], "rope_theta": cfg["rope_theta"],
         "rms_norm_eps": cfg["rms_eps"],
         "layer_types": ["sliding_attention" if s else "full_attention"
                         for s in cfg["layer_sliding"]]}
    if cfg.get("sliding_window"):
        c["sliding_window"] = cfg["sliding_window"]
    y = cfg.get("yarn")
    if y:
        c["rope_scaling"] = {"rope_type": "yarn", "factor": y["factor"],
                             "original_max_position_embeddings": y["orig_max_pos"],
                             "attention_factor": y["attn_factor"], "beta_fast": y["beta_fast"],
                             "beta_slow": y["beta_slow"]}
    if eos is not None:
        c["eos_token_id"] = eos
    return c


def write_dir(path, tensors, shards=1, config=None):
    """model.safetensors, or `shards` files plus model.safetensors.index.json."""
    os.makedirs(path, exist_ok=True)
    if config is not None:
        with open(os.path.join(path, "config.json"), "w") as f:
            json.dump(config, f, indent=2)
    if shards == 1:
        with open(os.path.join(path, "model.safetensors"), "wb") as f:
            f.write(safetensors_bytes(tensors))
        return
    per = (len(tensors) + shards - 1) // shards
    wmap = {}
    for s in range(shards):
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = tensors[s * per:(s + 1) * per]
        with open(os.path.join(path, name), "wb") as f:
            f.write(safetensors_bytes(part))
        for t in part:
            wmap[t[0]] = name
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": sum(len(t[3]) for t in tensors)},
                   "weight_map": wmap}, f, indent=2)
