"""The reference's ``atlas infer`` report with its CPU-vs-GPU logits check
(crates/atlas-cli/src/main.rs:786-972): ``atlas_amd.cli.run_infer`` over the
MI355X engine, with the oracle (the C restatement of the reference's CPU
``forward_one``) as the CPU path, built from the tensors the engine holds
after loading, so both sides use the same bf16 / int8 / int4 weights.

Test infrastructure: it runs the oracle.

    python tests/infer_harness.py --weights DIR [--model olmo3-7b|auto]
        [--prompt TEXT] [--max-tokens N] [--temperature T]
        [--format bf16|int8|int4] [--threads N]
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)

from atlas_amd import cli  # noqa: E402
from atlas_amd import model as am  # noqa: E402


def oracle_from_engine(m, threads: int = 1, max_seq: int = 0):
    """An oracle.Model over the weights resident in engine model m."""
    import oracle as orc
    c = m.config
    d, hd = c.d_model, c.d_model // c.n_heads
    kv = c.n_kv_heads * hd
    fmt = m.weight_format
    blk = 32

    def mat(kind, li, rows, cols):
        if fmt == am.W_BF16:
            return orc.MatView.bf16(m.get_tensor(kind, li, (rows, cols), np.uint16), rows, cols)
        if fmt == am.W_INT8:
            q, sc = m.get_tensor(kind, li, (rows, cols), np.int8, n_scales=rows)
            return orc.MatView.int8(q, sc)
        q, sc = m.get_tensor(kind, li, (rows * cols // 2,), np.uint8, n_scales=rows * cols // blk)
        return orc.MatView.int4(q, sc, rows, cols, blk)

    shapes = {am.T_WQ: ("wq", d, d), am.T_WK: ("wk", kv, d), am.T_WV: ("wv", kv, d),
              am.T_WO: ("wo", d, d), am.T_W_GATE: ("w_gate", c.ffn_hidden, d),
              am.T_W_UP: ("w_up", c.ffn_hidden, d), am.T_W_DOWN: ("w_down", d, c.ffn_hidden)}
    layers = []
    for li in range(c.n_layers):
        ld = {name: mat(k, li, r, cc) for k, (name, r, cc) in shapes.items()}
        ld["attn_norm"] = m.get_tensor(am.T_ATTN_NORM, li, (d,), np.float32)
        ld["ffn_norm"] = m.get_tensor(am.T_FFN_NORM, li, (d,), np.float32)
        ld["q_norm"] = m.get_tensor(am.T_Q_NORM, li, (d,), np.float32) if c.qk_norm else None
        ld["k_norm"] = m.get_tensor(am.T_K_NORM, li, (kv,), np.float32) if c.qk_norm else None
        layers.append(ld)
    V = c.vocab_size
    y = c.rope_scaling
    ocfg = dict(vocab=V, d_model=d, n_layers=c.n_layers, n_heads=c.n_heads,
                n_kv_heads=c.n_kv_heads, ffn_hidden=c.ffn_hidden,
                max_seq=max_seq or c.max_seq_len, rope_theta=c.rope_theta,
                rms_eps=c.rms_norm_eps,
                yarn=dict(factor=y.factor, orig_max_pos=y.orig_max_pos, attn_factor=y.attn_factor,
                          beta_fast=y.beta_fast, beta_slow=y.beta_slow) if y else None,
                sliding_window=c.sliding_window or 0,
                layer_sliding=[1 if t == "sliding" else 0 for t in (c.layer_types or [])] or
                [0] * c.n_layers,
                post_norm=c.post_norm)
    w = dict(embed=orc.MatView.bf16(m.get_tensor(am.T_EMBED, 0, (V, d), np.uint16), V, d),
             lm_head=mat(am.T_LM_HEAD, 0, V, d),
             final_norm=m.get_tensor(am.T_FINAL_NORM, 0, (d,), np.float32), layers=layers)
    return orc.Model(ocfg, w, threads=threads)


def oracle_logits(threads: int = 1):
    """cpu_logits for run_infer: the oracle's logits at the last prompt
    position, token by token as cmd_infer's CPU pass does."""
    def fn(m, prompt):
        om = oracle_from_engine(m, threads, max_seq=len(prompt) + 1)
        lg = None
        for t in prompt:
            lg = om.forward_one(int(t))
        return lg
    return fn


def main(argv=None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    threads = 1
    if "--threads" in argv:
        i = argv.index("--threads")
        threads = int(argv[i + 1])
        del argv[i:i + 2]
    cli.run_infer(cli.parse_args(argv), cpu_logits=oracle_logits(threads))
    return 0


if __name__ == "__main__":
    sys.exit(main())
