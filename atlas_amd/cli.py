"""``python -m atlas_amd.cli infer``: the reference's ``atlas infer`` command
(crates/atlas-cli/src/main.rs:786-972) over the MI355X engine.

It loads a checkpoint directory (``model.safetensors`` or the shards of
``model.safetensors.index.json``, with its ``config.json``), encodes the
prompt with the directory's ``tokenizer.json`` (byte-level ids when there is
none), prints the top-10 logits at the last prompt position and their spread,
then times ``generate`` and decodes its tokens.

The reference also compares its CPU ``forward_one`` logits with its GPU ones
(top-1 and max-abs).  This package has no CPU model.  ``run_infer`` takes the
CPU side as a callable, and ``tests/infer_harness.py`` passes the oracle
restatement of the reference CPU path for it.

Extensions:
- ``--format bf16|int8|int4`` picks the weight residency (the reference's GPU
  path is bf16).
- ``--model auto`` takes the shapes from config.json instead of a preset.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from typing import Callable, List, Optional, Sequence

import numpy as np

from . import loader
from .model import W_BF16, W_INT4, W_INT8, ModelConfig

PRESETS = {
    "smollm2-1.7b": ModelConfig.smollm2_1b7,
    "smollm2-135m": ModelConfig.smollm2_135m,
    "olmo3-1b": ModelConfig.olmo3_1b,
    "olmo3-7b": ModelConfig.olmo3_actual_7b,
    "llama32-1b": ModelConfig.llama32_1b,
}
FORMATS = {"bf16": W_BF16, "int8": W_INT8, "int4": W_INT4}


def parse_args(argv: Sequence[str]) -> argparse.Namespace:
    ap = argparse.ArgumentParser(prog="atlas_amd.cli infer")
    ap.add_argument("--weights", required=True, help="checkpoint directory")
    ap.add_argument("--prompt", default="The capital of France is")
    ap.add_argument("--max-tokens", type=int, default=50)
    ap.add_argument("--temperature", type=float, default=0.0)
    ap.add_argument("--model", default="smollm2-1.7b",
                    help=f"one of {', '.join(PRESETS)}, or auto (shapes from config.json)")
    ap.add_argument("--format", default="bf16", choices=sorted(FORMATS))
    return ap.parse_args(list(argv))


def config_from_hf_json(path: str) -> ModelConfig:
    """Shapes of a HF-style config.json (the fields the loader's config patch
    does not set: heads, KV heads, FFN width, context length)."""
    with open(path) as f:
        j = json.load(f)
    heads = int(j["num_attention_heads"])
    return ModelConfig(vocab_size=int(j["vocab_size"]), d_model=int(j["hidden_size"]),
                       n_layers=int(j["num_hidden_layers"]), n_heads=heads,
                       n_kv_heads=int(j.get("num_key_value_heads", heads)),
                       ffn_hidden=int(j["intermediate_size"]),
                       max_seq_len=int(j.get("max_position_embeddings", 4096)),
                       rope_theta=float(j.get("rope_theta", 10000.0)),
                       rms_norm_eps=float(j.get("rms_norm_eps", 1e-5)))


def load_tokenizer(weights_dir: str):
    """The directory's tokenizer.json through the `tokenizers` package, or None
    (missing file or package): the caller falls back to byte-level ids."""
    path = os.path.join(weights_dir, "tokenizer.json")
    try:
        from tokenizers import Tokenizer
        return Tokenizer.from_file(path), None
    except Exception as e:                      # noqa: BLE001 (reported, then byte-level)
        return None, f"{e}"


def encode(tok, text: str) -> List[int]:
    if tok is not None:
        return list(tok.encode(text).ids)
    return list(text.encode("utf-8"))


def decode(tok, ids: Sequence[int]) -> str:
    if tok is not None:
        return tok.decode(list(ids))
    return bytes(int(t) % 256 for t in ids).decode("utf-8", errors="replace")


def top1_last(logits: np.ndarray) -> int:
    """Index of the maximum, the last one on ties (Iterator::max_by)."""
    return int(logits.size - 1 - np.argmax(logits[::-1]))


def run_infer(args: argparse.Namespace,
              cpu_logits: Optional[Callable[[object, List[int]], np.ndarray]] = None,
              out: Callable[[str], None] = print) -> dict:
    """cmd_infer's steps and report; returns the figures as a dict.
    cpu_logits(model, prompt_ids) -> logits at the last prompt position from a
    CPU path over the same weights (None: the comparison is skipped)."""
    wdir = args.weights.rstrip("/")
    out("┌─ ATLAS infer (MI355X) ─────────────────────────────────────────────")
    out(f"│  weights     = {wdir}")
    out(f"│  model       = {args.model}   format = {args.format}")
    out(f"│  prompt      = {args.prompt!r}")
    out(f"│  max_tokens  = {args.max_tokens}   temperature = {args.temperature}")
    out("└────────────────────────────────────────────────────────────────────")
    if args.model == "auto":
        cfg = config_from_hf_json(os.path.join(wdir, "config.json"))
    elif args.model in PRESETS:
        cfg = PRESETS[args.model]()
    else:
        raise SystemExit(f"atlas infer: unknown model {args.model!r}; available: "
                         f"{', '.join(PRESETS)}, auto")
    out(f"\n  Model config : {cfg.n_layers} layers, d={cfg.d_model}, {cfg.n_heads} heads, "
        f"vocab={cfg.vocab_size}")
    tok, err = load_tokenizer(wdir)
    if tok is not None:
        out(f"  Tokenizer    : loaded ({tok.get_vocab_size()} vocab) from {wdir}/tokenizer.json")
    else:
        out(f"  Tokenizer    : {err} -- falling back to byte-level encoding")
    prompt = encode(tok, args.prompt) or [0]
    out(f"  Prompt tokens: {len(prompt)} -> {prompt[:20]}")
    # the KV cache covers this run (the preset's context can be 128K)
    cfg.max_seq_len = min(cfg.max_seq_len, len(prompt) + args.max_tokens + 64)

    sharded = os.path.exists(os.path.join(wdir, "model.safetensors.index.json"))
    out(f"\n  Loading weights from {wdir} (sharded={sharded}) ...")
    t0 = time.perf_counter()
    m = loader.load_model_from_dir(wdir, cfg, weight_format=FORMATS[args.format])
    load_ms = (time.perf_counter() - t0) * 1e3
    out(f"  Weights loaded in {load_ms:.0f} ms ({m.weight_bytes() / 1e9:.2f} GB resident)")

    # logits at the last prompt position
    t0 = time.perf_counter()
    m.reset()
    if len(prompt) > 1:
        m.prefill(prompt[:-1])
    gpu = m.forward_one(prompt[-1])
    logit_ms = (time.perf_counter() - t0) * 1e3
    order = np.argsort(-gpu, kind="stable")
    out(f"  Top-10 logits (last prompt position, {logit_ms:.0f} ms):")
    for t in order[:10]:
        shown = f" = {decode(tok, [int(t)])!r}" if tok is not None else ""
        out(f"    token {int(t):6d}: {float(gpu[t]):8.4f}{shown}")
    spread = float(gpu[order[0]] - gpu[order[min(99, gpu.size - 1)]])
    out(f"\n  {'Logit spread' if spread >= 1.0 else 'WARNING: logit spread'} = {spread:.2f}"
        f"{' (healthy)' if spread >= 1.0 else ' (< 1.0): forward pass may be incorrect'}")

    report = dict(prompt_tokens=len(prompt), load_ms=load_ms, logit_ms=logit_ms, spread=spread,
                  gpu_top1=top1_last(gpu))
    if cpu_logits is not None:
        cpu = np.asarray(cpu_logits(m, prompt), np.float32)
        ct, gt = top1_last(cpu), top1_last(gpu)
        diff = float(np.max(np.abs(cpu - gpu)))
        out(f"\n  CPU top-1: token {ct} (logit {cpu[ct]:.4f})")
        out(f"  GPU top-1: token {gt} (logit {gpu[gt]:.4f})")
        out("  CPU/GPU agree on top token" if ct == gt else "  CPU/GPU DISAGREE on top token!")
        out(f"  Max logit abs diff: {diff:.6f}")
        report.update(cpu_top1=ct, top1_agrees=ct == gt, max_abs_diff=diff,
                      max_abs_logit=float(np.max(np.abs(cpu))))
    else:
        out("\n  CPU path: not in this package (tests/infer_harness.py compares the oracle)")

    out(f"\n  Generating {args.max_tokens} tokens (temperature={args.temperature}) ...")
    t0 = time.perf_counter()
    new = m.generate(prompt, args.max_tokens, args.temperature)
    gen_s = time.perf_counter() - t0
    tps = len(new) / max(gen_s, 1e-3)
    text = decode(tok, new)
    out("\n  --- Output -----------------------------------------------------------")
    out(f"  Prompt : {args.prompt!r}")
    out(f"  Output : {text!r}")
    out(f"  Full   : {args.prompt + text!r}")
    out("\n  --- Stats ------------------------------------------------------------")
    out(f"  Tokens generated : {len(new)}")
    out(f"  Generation time  : {gen_s * 1e3:.0f} ms")
    out(f"  Throughput       : {tps:.1f} tok/s")
    out(f"  Token IDs        : {new[:20]}")
    out("\n  atlas infer complete")
    report.update(tokens=new, gen_ms=gen_s * 1e3, tok_s=tps, text=text)
    m.close()
    return report


def main(argv: Optional[Sequence[str]] = None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] != "infer":
        print("usage: python -m atlas_amd.cli infer --weights DIR [--model NAME|auto] "
              "[--prompt TEXT] [--max-tokens N] [--temperature T] [--format bf16|int8|int4]",
              file=sys.stderr)
        return 1
    run_infer(parse_args(argv[1:]))
    return 0


if __name__ == "__main__":
    sys.exit(main())
