"""Checkpoint loading on the MI355X (include/atlas_loader.h): HF-named
safetensors written by tests/ckptgen.py from modelgen weights, loaded into
device residency, checked tensor by tensor (bit-exact: bf16 bits, bf16
truncation of F32/F16 sources, atlas-quant int8/int4 of the widened values)
and end to end against the CPU oracle and the engine loaded through
set_tensor (identical logits: the device state is the same).
"""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import ckptgen  # noqa: E402
import modelgen  # noqa: E402

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import atlas_amd
    atlas_amd.load()
    from tests.gpu_util import lib
    if not lib().atlas_cuda_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")


def _base_cfg(cfg, **kw):
    """A caller configuration that only knows the shapes: the rest must come
    from config.json and the tensor names."""
    from atlas_amd import model as am
    c = am.ModelConfig(vocab_size=7, d_model=cfg["d_model"], n_layers=cfg["n_layers"],
                       n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"],
                       ffn_hidden=cfg["ffn_hidden"], max_seq_len=cfg["max_seq"],
                       rope_theta=cfg["rope_theta"], rms_norm_eps=cfg["rms_eps"],
                       post_norm=False, qk_norm=False)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def _bits(stored):
    return stored[1][0]


def _check_bf16_tensors(m, W, tied=False):
    from atlas_amd import model as am
    cfg = W["cfg"]
    shp, _ = modelgen.shapes(cfg)
    kinds = dict(wq=am.T_WQ, wk=am.T_WK, wv=am.T_WV, wo=am.T_WO, w_gate=am.T_W_GATE,
                 w_up=am.T_W_UP, w_down=am.T_W_DOWN)
    for li, lw in enumerate(W["layers"]):
        for n, k in kinds.items():
            assert np.array_equal(m.get_tensor(k, li, shp[n], np.uint16), _bits(lw[n + "_stored"])), (li, n)
        assert np.array_equal(m.get_tensor(am.T_ATTN_NORM, li, cfg["d_model"], np.float32),
                              lw["attn_norm"])
        assert np.array_equal(m.get_tensor(am.T_FFN_NORM, li, cfg["d_model"], np.float32),
                              lw["ffn_norm"])
    V, d = cfg["vocab"], cfg["d_model"]
    assert np.array_equal(m.get_tensor(am.T_EMBED, 0, (V, d), np.uint16), W["embed_bits"])
    lm = W["embed_bits"] if tied else _bits(W["lm_head_stored"])
    assert np.array_equal(m.get_tensor(am.T_LM_HEAD, 0, (V, d), np.uint16), lm)
    assert np.array_equal(m.get_tensor(am.T_FINAL_NORM, 0, d, np.float32), W["final_norm"])


def _teacher_forced(m, W, tokens):
    o = modelgen.oracle_model(W, threads=8)
    m.reset()
    worst = 0.0
    for t in tokens:
        lg, ref = m.forward_one(int(t)), o.forward_one(int(t))
        worst = max(worst, float(np.max(np.abs(lg.astype(np.float64) - ref)) / np.max(np.abs(ref))))
    return worst


def test_load_dir_olmo3_config_and_weights(tmp_path):
    # OLMo-3 wiring from config.json (layer types, window, YaRN, theta, eps,
    # eos) and from the names (post-norm, QK-norm, vocab); bf16 bits exact
    from atlas_amd import loader
    cfg = modelgen.olmo3_small_config(max_seq=64)
    W = modelgen.make_weights(cfg, seed=51, fmt="bf16")
    ckptgen.write_dir(str(tmp_path), ckptgen.hf_tensors(W),
                      config=ckptgen.olmo3_config_json(cfg, eos=17))
    base = _base_cfg(cfg, rope_theta=10000.0, rms_norm_eps=1e-5)
    m = loader.load_model_from_dir(str(tmp_path), base)
    c = m.config
    assert c.vocab_size == cfg["vocab"] and c.post_norm and c.qk_norm
    assert c.layer_types == ["sliding" if s else "full" for s in cfg["layer_sliding"]]
    assert c.sliding_window == cfg["sliding_window"] and c.rope_scaling.factor == 8.0
    assert c.rope_theta == np.float32(cfg["rope_theta"]) and m.eos_token_id == 17
    _check_bf16_tensors(m, W)
    for li, lw in enumerate(W["layers"]):
        from atlas_amd import model as am
        assert np.array_equal(m.get_tensor(am.T_Q_NORM, li, lw["q_norm"].size, np.float32),
                              lw["q_norm"])
    toks = np.random.default_rng(3).integers(0, cfg["vocab"], 12)
    assert _teacher_forced(m, W, toks) <= LOGIT_TOL
    # the same device state as weights uploaded through set_tensor
    ref = modelgen.engine_model(W)
    m.reset()
    ref.reset()
    for t in toks[:6]:
        assert np.array_equal(m.forward_one(int(t)), ref.forward_one(int(t)))


def test_load_sharded_llama_names_tied_embedding(tmp_path):
    # pre-norm names (input / post_attention layernorm), "layers.N." and
    # tok_embeddings / norm prefixes, no lm_head (tied), no QK-norm, two shards
    from atlas_amd import loader
    cfg = modelgen.tiny_config(post_norm=False, qk_norm=False, vocab=300)
    W = modelgen.make_weights(cfg, seed=52, fmt="bf16")
    ckptgen.write_dir(str(tmp_path), ckptgen.hf_tensors(W, naming="llama", tie=True), shards=2)
    assert os.path.exists(tmp_path / "model.safetensors.index.json")
    m = loader.load_model_from_dir(str(tmp_path), _base_cfg(cfg, post_norm=True, qk_norm=True))
    assert not m.config.post_norm and not m.config.qk_norm and m.eos_token_id is None
    _check_bf16_tensors(m, W, tied=True)
    Wt = dict(W)
    Wt["lm_head_stored"] = ("bf16", (W["embed_bits"],))
    toks = np.random.default_rng(4).integers(0, cfg["vocab"], 10)
    assert _teacher_forced(m, Wt, toks) <= LOGIT_TOL


@pytest.mark.parametrize("source", ["F32", "F16"])
def test_load_f32_f16_sources_truncate(tmp_path, source):
    # F32 values with random low bits truncate back to the bf16 bits; F16
    # values widen exactly (f16_to_f32) and then truncate
    from atlas_amd import loader
    from atlas_amd import model as am
    import oracle as orc
    cfg = modelgen.tiny_config()
    W = modelgen.make_weights(cfg, seed=53, fmt="bf16")
    p = str(tmp_path / "m.safetensors")
    with open(p, "wb") as f:
        f.write(ckptgen.safetensors_bytes(ckptgen.hf_tensors(W, source=source, seed=9)))
    m = loader.load_model_from_safetensors(p, _base_cfg(cfg))
    if source == "F32":
        _check_bf16_tensors(m, W)
        return
    shp, _ = modelgen.shapes(cfg)
    for n, k in (("wq", am.T_WQ), ("w_down", am.T_W_DOWN)):
        b = _bits(W["layers"][1][n + "_stored"])
        f16 = orc.bf16_to_f32(b).astype(np.float16).astype(np.float32)
        want = (f16.view(np.uint32) >> 16).astype(np.uint16)
        assert np.array_equal(m.get_tensor(k, 1, shp[n], np.uint16), want), n


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_load_quantised_residency(tmp_path, fmt):
    # bf16 checkpoint -> int8 / int4 on the device, bit-exact to the
    # atlas-quant rules applied to the widened values
    from atlas_amd import loader
    from atlas_amd import model as am
    import oracle as orc
    cfg = modelgen.olmo3_small_config(max_seq=48)
    W = modelgen.make_weights(cfg, seed=54, fmt="bf16")
    ckptgen.write_dir(str(tmp_path), ckptgen.hf_tensors(W),
                      config=ckptgen.olmo3_config_json(cfg))
    wf = am.W_INT8 if fmt == "int8" else am.W_INT4
    m = loader.load_model_from_dir(str(tmp_path), _base_cfg(cfg), weight_format=wf, int4_block=32)
    shp, _ = modelgen.shapes(cfg)
    kinds = dict(wq=am.T_WQ, wk=am.T_WK, wv=am.T_WV, wo=am.T_WO, w_gate=am.T_W_GATE,
                 w_up=am.T_W_UP, w_down=am.T_W_DOWN)
    Wq = modelgen.make_weights(cfg, seed=54, fmt="bf16")
    for li, lw in enumerate(W["layers"]):
        for n, k in kinds.items():
            r, c = shp[n]
            f = orc.bf16_to_f32(_bits(lw[n + "_stored"]))
            if fmt == "int8":
                q, s = orc.int8_quantize(f)
                got, gs = m.get_tensor(k, li, (r, c), np.int8, n_scales=r)
                Wq["layers"][li][n + "_stored"] = ("int8", (q, s))
            else:
                q, s = orc.int4_quantize(f, 32)
                got, gs = m.get_tensor(k, li, q.shape, np.uint8, n_scales=s.size)
                Wq["layers"][li][n + "_stored"] = ("int4", (q, s))
            assert np.array_equal(got.reshape(q.shape), q) and np.array_equal(gs, s), (li, n)
    Wq["fmt"], Wq["block"] = fmt, 32
    f = orc.bf16_to_f32(_bits(W["lm_head_stored"]))
    Wq["lm_head_stored"] = ("int8", orc.int8_quantize(f)) if fmt == "int8" else \
        ("int4", orc.int4_quantize(f, 32))
    toks = np.random.default_rng(5).integers(0, cfg["vocab"], 8)
    assert _teacher_forced(m, Wq, toks) <= LOGIT_TOL
