"""Writes tests/golden/fixtures.npz: small seeded input/output vectors of the
decode path, computed by the CPU oracle (oracle/, the restatement of the
reference's CPU path that tests/test_oracle.py pins against the reference's
literals, closed forms and float64 checks).

The fixtures freeze the oracle's outputs so that (a) a change of the oracle
shows up as a fixture mismatch on the CPU, and (b) the GPU parity tests can
compare the HIP path with stored vectors.  Inputs come from the shared
SplitMix64 + Box-Muller generator (oracle.normal / oracle.uniform) with fixed
seeds; the model fixture's weights come from tests/modelgen.py (numpy PCG64,
seed 29) and are checked by a SHA-256 of their bytes.

Run: python tests/golden/make_golden.py   (rewrites the file)
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

YARN = dict(factor=8.0, orig_max_pos=8192, attn_factor=1.2079441541679836, beta_fast=32.0,
            beta_slow=1.0)


SAMPLED_SEED = 0x243F6A8885A308D3


def sampled_config(suppress):
    """A sampling configuration with every stage of the pipeline active."""
    return dict(temperature=0.8, top_p=0.9, top_k=20, min_p=0.02, repetition_penalty=1.15,
                repetition_window=8, frequency_penalty=0.1, presence_penalty=0.2,
                suppress=list(suppress))


def model_config():
    import modelgen
    return modelgen.tiny_config(vocab=128, d_model=64, n_layers=2, n_heads=4, n_kv_heads=2,
                                ffn_hidden=128, max_seq=64, rope_theta=500000.0, rms_eps=1e-6,
                                yarn=YARN, sliding_window=8, layer_sliding=[1, 0],
                                post_norm=True, qk_norm=True)


def weight_digest(W) -> str:
    h = hashlib.sha256()
    h.update(W["embed_bits"].tobytes())
    h.update(W["lm_head_stored"][1][0].tobytes())
    h.update(W["final_norm"].tobytes())
    for lw in W["layers"]:
        for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            h.update(lw[n + "_stored"][1][0].tobytes())
        for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
            h.update(lw[n].tobytes())
    return h.hexdigest()


def compute() -> dict:
    import oracle as orc
    import modelgen
    f = {}
    # ---- quantisers: a row of exact half-way and clamp cases, a zero row,
    # and generator rows; int4 blocks cross row ends (5 x 40, block 32)
    w8 = orc.normal(8 * 40, 101, 0.0, 0.02).reshape(8, 40)
    w8[0, :6] = [0.5, -0.5, 1.5, -1.5, 127.0, -127.0]
    w8[1] = 0.0
    f["q8_w"] = w8.astype(np.float32)
    f["q8_data"], f["q8_scales"] = orc.int8_quantize(f["q8_w"])
    w4 = orc.normal(5 * 40, 102, 0.0, 0.02).reshape(5, 40).astype(np.float32)
    w4[2, :4] = [7.0, -7.0, 3.5, -3.5]
    f["q4_w"] = w4
    f["q4_data"], f["q4_scales"] = orc.int4_quantize(w4, 32)
    # ---- GEMVs 64 x 96 (int4 block 32: three blocks per row)
    M, K = 64, 96
    w = orc.normal(M * K, 103, 0.0, 0.02).reshape(M, K).astype(np.float32)
    x = orc.normal(K, 104).astype(np.float32)
    f["gemv_x"] = x
    f["gemv_bf16_w"] = orc.bf16_from_f32(w)
    f["gemv_bf16_y"] = orc.linear(orc.MatView.bf16(f["gemv_bf16_w"], M, K), x)
    f["gemv_i8_w"], f["gemv_i8_s"] = orc.int8_quantize(w)
    f["gemv_i8_y"] = orc.linear(orc.MatView.int8(f["gemv_i8_w"], f["gemv_i8_s"]), x)
    f["gemv_i4_w"], f["gemv_i4_s"] = orc.int4_quantize(w, 32)
    f["gemv_i4_y"] = orc.linear(orc.MatView.int4(f["gemv_i4_w"], f["gemv_i4_s"], M, K, 32), x)
    # ---- YaRN RoPE tables: head_dim 128, 16 positions
    cos, sin, _ = orc.rope_tables(128, 16, 500000.0, YARN)
    f["rope_cos"], f["rope_sin"] = cos, sin
    # ---- GQA attention: 4 query / 2 KV heads of 32, position 36, full and window 8
    H, KVH, hd, pos = 4, 2, 32, 36
    q = orc.normal(H * hd, 105).astype(np.float32)
    kc = orc.normal((pos + 1) * KVH * hd, 106).reshape(pos + 1, KVH, hd).astype(np.float32)
    vc = orc.normal((pos + 1) * KVH * hd, 107).reshape(pos + 1, KVH, hd).astype(np.float32)
    scale = 1.2079441541679836 / np.sqrt(hd)
    f["attn_q"], f["attn_k"], f["attn_v"] = q, kc, vc
    f["attn_out_full"] = orc.attention(q, kc, vc, H, KVH, hd, pos, scale, 0)
    f["attn_out_w8"] = orc.attention(q, kc, vc, H, KVH, hd, pos, scale, 8)
    # ---- a 2-layer OLMo-3-wired model (bf16): first-step logits, 16 greedy
    # and 24 sampled tokens after a 5-token prompt
    cfg = model_config()
    W = modelgen.make_weights(cfg, seed=29, fmt="bf16")
    o = modelgen.oracle_model(W)
    prompt = [3, 17, 42, 99, 5]
    o.reset()
    f["model_logits0"] = o.forward_one(prompt[0])
    f["model_prompt"] = np.array(prompt, np.uint32)
    f["model_tokens"] = np.array(o.generate_greedy(prompt, 16), np.uint32)
    # 24 sampled tokens, the greedy first token suppressed at step 0
    sc = orc.sampling(**sampled_config([int(f["model_tokens"][0])]))
    f["model_sampled_tokens"] = np.array(o.generate_sampled(prompt, 24, sc, SAMPLED_SEED),
                                         np.uint32)
    f["model_digest"] = np.frombuffer(bytes.fromhex(weight_digest(W)), np.uint8)
    return f


def main():
    f = compute()
    path = os.path.join(HERE, "fixtures.npz")
    np.savez_compressed(path, **f)
    print(f"wrote {path}: {os.path.getsize(path)} bytes, {len(f)} arrays")


if __name__ == "__main__":
    main()
