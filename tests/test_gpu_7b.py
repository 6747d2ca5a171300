"""BASELINE.json configs[4] at its real shape, on the MI355X.

The OLMo-3-7B decode shape: vocab 100278, d_model 4096, 32 layers, 32 query
and 32 KV heads of dim 128, MLP 11008 (SwiGLU), post-norm RMSNorm, per-head
QK-norm, YaRN RoPE, layers i % 4 != 3 sliding with window 4096
(crates/atlas-model/src/lib.rs:253-269 plus the OLMo-3 config.json
fields, lib.rs:2367-2432).  Weights are random-initialised on the device
(N(0, 0.02) projections, U(0.5, 1.5) norms), in bf16 and separately int8
and int4, then downloaded to build the oracle model of the same weights.

* Teacher forcing past position 0 in bf16, int8 and int4 (blocks of 32): a
  40-token prompt goes through the engine's prompt-chunk path (39 rows in one
  chunk, then the last token as a decode step), followed by 8 decode steps.
  At each of those 9 positions the logits must be within 1e-3 * max|logit|
  of the oracle (the reference's CPU path restated, row-threaded) and top-1
  must agree (a near-tie of the oracle's own top two is reported instead).
* Long positions: both models get the same seeded KV-cache rows and decode
  8 teacher-forced steps from position 300 and from 4100 (bf16 and int4).
* The ragged batch of 8 sequences with prompts of 16..2048 tokens and 256
  greedy tokens each: every sequence's tokens equal its own single-sequence
  greedy run (a divergence is accepted only at a near-tie, checked on the
  single run's logits at that step).
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
D, V, L, F = 4096, 100278, 32, 11008


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import atlas_amd
    if not atlas_amd.load().atlas_cuda_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")


def _threads():
    # the GPU box's CPU share is 16 cores, whatever os.cpu_count() reports
    return max(1, min(16, os.cpu_count() or 1))


def _engine(fmt: str, max_seq: int, max_batch: int = 1, seed: int = 2024):
    from atlas_amd import model as am
    cfg = am.ModelConfig.olmo3_actual_7b()
    cfg.max_seq_len = max_seq
    m = am.OlmoModel(cfg, weight_format={"bf16": am.W_BF16, "int8": am.W_INT8,
                                         "int4": am.W_INT4}[fmt],
                     int4_block=32, max_batch=max_batch)
    m.init_random(seed)
    return m


def _oracle_of(m, fmt: str, max_seq: int):
    """The oracle model over the engine's own weights (downloaded)."""
    import oracle as orc
    from atlas_amd import model as am
    shapes = {am.T_WQ: (D, D), am.T_WK: (D, D), am.T_WV: (D, D), am.T_WO: (D, D),
              am.T_W_GATE: (F, D), am.T_W_UP: (F, D), am.T_W_DOWN: (D, F)}
    names = {am.T_WQ: "wq", am.T_WK: "wk", am.T_WV: "wv", am.T_WO: "wo",
             am.T_W_GATE: "w_gate", am.T_W_UP: "w_up", am.T_W_DOWN: "w_down"}

    def mat(kind, li, shp):
        if fmt == "bf16":
            return orc.MatView.bf16(m.get_tensor(kind, li, shp, np.uint16), *shp)
        if fmt == "int4":
            # Int4Tensor: two weights per byte, one f32 scale per 32-weight
            # block of the flattened matrix (crates/atlas-quant/src/lib.rs:113-168)
            rows, cols = shp
            q, s = m.get_tensor(kind, li, (rows * cols // 2,), np.uint8,
                                n_scales=rows * cols // 32)
            return orc.MatView.int4(q, s, rows, cols, 32)
        q, s = m.get_tensor(kind, li, shp, np.int8, n_scales=shp[0])
        return orc.MatView.int8(q, s)

    layers = []
    for li in range(L):
        ld = {names[k]: mat(k, li, shp) for k, shp in shapes.items()}
        for k, n in ((am.T_ATTN_NORM, "attn_norm"), (am.T_FFN_NORM, "ffn_norm"),
                     (am.T_Q_NORM, "q_norm"), (am.T_K_NORM, "k_norm")):
            ld[n] = m.get_tensor(k, li, (D,), np.float32)
        layers.append(ld)
    emb = orc.MatView.bf16(m.get_tensor(am.T_EMBED, 0, (V, D), np.uint16), V, D)
    ocfg = dict(vocab=V, d_model=D, n_layers=L, n_heads=32, n_kv_heads=32, ffn_hidden=F,
                max_seq=max_seq, rope_theta=500000.0, rms_eps=1e-6,
                yarn=dict(factor=8.0, orig_max_pos=8192, attn_factor=1.2079441541679836,
                          beta_fast=32.0, beta_slow=1.0),
                sliding_window=4096, layer_sliding=[0 if i % 4 == 3 else 1 for i in range(L)],
                post_norm=True)
    w = dict(embed=emb, lm_head=mat(am.T_LM_HEAD, 0, (V, D)),
             final_norm=m.get_tensor(am.T_FINAL_NORM, 0, (D,), np.float32), layers=layers)
    return orc.Model(ocfg, w, threads=_threads())


def _rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / np.max(np.abs(b)))


def _top1(lg):
    return int(lg.size - 1 - np.argmax(lg[::-1]))      # last index on ties (lib.rs:2701-2706)


def _margin(lg):
    s = np.sort(lg)
    return float(s[-1] - s[-2])


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int4"])
def test_7b_teacher_forced(orc, fmt):
    max_seq = 64
    m = _engine(fmt, max_seq)
    o = _oracle_of(m, fmt, max_seq)
    rng = np.random.default_rng(17)
    prompt = [int(t) for t in rng.integers(0, V, 40)]
    m.reset()
    m.prefill(prompt[:-1])                       # one 39-row prompt chunk
    for t in prompt[:-1]:
        o.forward_one(t)
    assert m.pos == o.pos == 39
    tok = prompt[-1]
    worst = 0.0
    for step in range(9):
        lg, ref = m.forward_one(tok), o.forward_one(tok)
        err = _rel(lg, ref)
        worst = max(worst, err)
        print(f"7B {fmt} pos {m.pos - 1}: rel logit err {err:.2e}, top-1 {_top1(lg)} / "
              f"{_top1(ref)}, oracle margin {_margin(ref):.3g}", flush=True)
        assert err <= LOGIT_TOL, (step, err)
        if _top1(lg) != _top1(ref):
            assert _margin(ref) <= 2 * LOGIT_TOL * np.max(np.abs(ref)), (step, _margin(ref))
        tok = _top1(ref)                         # teacher: the oracle's choice
    assert m.pos == o.pos == 48
    print(f"7B {fmt}: worst rel logit err {worst:.2e} over positions 39..47", flush=True)


@pytest.mark.parametrize("fmt", ["bf16", "int4"])
def test_7b_long_positions(orc, fmt):
    """Decode steps at positions 300..307 (four attention splits merged by the
    last block) and 4100..4107 (eight splits; the sliding layers' window of
    4096 masks cache rows 4..11), teacher-forced against the oracle.  Both
    models get the same seeded cache rows (K, V ~ N(0, 1)) for every earlier
    position instead of a 4100-token prefill through the CPU path."""
    max_seq = 4120
    m = _engine(fmt, max_seq)
    o = _oracle_of(m, fmt, max_seq)
    kvd = 32 * 128
    rng = np.random.default_rng(31)
    for p0 in (300, 4100):
        for li in range(L):
            k = rng.standard_normal((p0, kvd), dtype=np.float32)
            v = rng.standard_normal((p0, kvd), dtype=np.float32)
            m.set_kv_rows(li, 0, k, v)
            o.set_kv_rows(li, 0, k, v)
        m.set_pos(p0)
        o.set_pos(p0)
        tok = int(rng.integers(0, V))
        worst = 0.0
        for step in range(8):
            lg, ref = m.forward_one(tok), o.forward_one(tok)
            err = _rel(lg, ref)
            worst = max(worst, err)
            print(f"7B {fmt} pos {m.pos - 1}: rel logit err {err:.2e}, top-1 {_top1(lg)} / "
                  f"{_top1(ref)}, oracle margin {_margin(ref):.3g}", flush=True)
            assert err <= LOGIT_TOL, (p0, step, err)
            if _top1(lg) != _top1(ref):
                assert _margin(ref) <= 2 * LOGIT_TOL * np.max(np.abs(ref)), (p0, step)
            tok = _top1(ref)
        assert m.pos == o.pos == p0 + 8
        print(f"7B {fmt}: worst rel logit err {worst:.2e} over positions {p0}..{p0 + 7}",
              flush=True)


def test_7b_ragged_batch_matches_single(orc):
    from atlas_amd.model import SamplingConfig
    lens = [16, 64, 128, 256, 512, 1024, 1536, 2048]
    max_new = 256
    m = _engine("bf16", max_seq=2048 + max_new + 8, max_batch=8)
    rng = np.random.default_rng(23)
    prompts = [[int(t) for t in rng.integers(0, V, n)] for n in lens]
    batch = m.generate_batch(prompts, max_new)
    assert [len(b) for b in batch] == [max_new] * 8
    greedy = SamplingConfig.greedy()
    for p, got in zip(prompts, batch):
        want = m.generate_with_sampling(p, max_new, greedy)
        if got != want:
            k = next(i for i in range(max_new) if got[i] != want[i])
            # the single run's logits where the two runs part: a near-tie only
            m.reset()
            m.prefill(p[:-1])
            lg = None
            for t in [p[-1]] + want[:k]:
                lg = m.forward_one(t)
            print(f"prompt {len(p)}: batch and single part at token {k}, "
                  f"margin {_margin(lg):.3g}", flush=True)
            assert _margin(lg) <= 2 * LOGIT_TOL * np.max(np.abs(lg)), (len(p), k)
        print(f"prompt {len(p)}: {max_new} batch tokens == single-sequence greedy", flush=True)
