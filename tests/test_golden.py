"""Golden fixtures (tests/golden/fixtures.npz, written by
tests/golden/make_golden.py from the pinned CPU oracle).

CPU: the oracle still reproduces every fixture bit for bit, the model
generator still yields the same weights, and the library's host quantisers
match the stored quantisations.  GPU: the HIP kernels and the engine against
the stored vectors -- quantisation bit-exact, GEMV max-abs <= 1e-3 * max|y|,
attention <= 2e-3 * max|o|, greedy tokens identical.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = os.path.join(HERE, "golden", "fixtures.npz")
GEMV_TOL = 1e-3
ATTN_TOL = 2e-3


@pytest.fixture(scope="module")
def fx():
    with np.load(FIXTURES, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _make_golden():
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_golden
    return make_golden


def test_oracle_reproduces_fixtures(orc, fx):
    fresh = _make_golden().compute()
    assert set(fresh) == set(fx)
    for k, v in fresh.items():
        assert v.dtype == fx[k].dtype and v.shape == fx[k].shape, k
        assert np.array_equal(v, fx[k]), k


def test_fixture_inputs_hold_the_edge_cases(fx):
    # the int8 fixture row 0 holds half-way values (round away from zero) and
    # the clamp limits; row 1 is all zero (scale 1.0); int4 blocks cross rows
    assert fx["q8_scales"][1] == 1.0 and not fx["q8_data"][1].any()
    assert fx["q8_data"][0, 4] == 127 and fx["q8_data"][0, 5] == -127
    assert fx["q4_data"].size == (5 * 40 + 1) // 2 and fx["q4_scales"].size == (5 * 40 + 31) // 32
    assert len(fx["model_tokens"]) == 16


def test_host_quantisers_match_fixtures(fx):
    from atlas_amd.quant import Int4Tensor, Int8Tensor
    a = Int8Tensor.quantize(fx["q8_w"])
    assert np.array_equal(a.data.reshape(fx["q8_data"].shape), fx["q8_data"])
    assert np.array_equal(a.scales, fx["q8_scales"])
    b = Int4Tensor.quantize(fx["q4_w"], 32)
    assert np.array_equal(b.data, fx["q4_data"]) and np.array_equal(b.scales, fx["q4_scales"])


def test_sampled_fixture_survives_small_logit_errors(fx):
    # The GPU logits differ from the oracle's by ~1e-5 relative.  Replaying the
    # sampled fixture with teacher forcing, every step's choice must stay the
    # same under random logit errors of 1e-4 * max|logit|, so that the GPU test
    # below compares tokens rather than luck.
    import oracle as orc
    sys.path.insert(0, HERE)
    import modelgen
    mg = _make_golden()
    W = modelgen.make_weights(mg.model_config(), seed=29, fmt="bf16")
    o = modelgen.oracle_model(W)
    prompt = [int(t) for t in fx["model_prompt"]]
    toks = [int(t) for t in fx["model_sampled_tokens"]]
    sc = orc.sampling(**mg.sampled_config([int(fx["model_tokens"][0])]))
    rng = orc.Rng(mg.SAMPLED_SEED)
    noise = np.random.default_rng(3)
    o.reset()
    for t in prompt:
        logits = o.forward_one(t)
    for step, tok in enumerate(toks):
        state = rng.state.value
        assert orc.sample_step(logits, toks[:step], step, sc, rng) == tok
        eps = 1e-4 * float(np.max(np.abs(logits)))
        for _ in range(8):
            r = orc.Rng(0)
            r.state.value = state
            pert = logits + noise.uniform(-eps, eps, logits.size).astype(np.float32)
            assert orc.sample_step(pert, toks[:step], step, sc, r) == tok, step
        logits = o.forward_one(tok)


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------

def _gpu_ready():
    import atlas_amd
    atlas_amd.load()
    from tests.gpu_util import lib
    if not lib().atlas_cuda_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")


def _rel(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / np.max(np.abs(ref)))


@pytest.mark.gpu
def test_gpu_quantisers_match_fixtures(fx):
    _gpu_ready()
    from tests.gpu_util import Dev, lib
    # every device buffer stays referenced until the results are read back
    w8 = fx["q8_w"]
    dw8, dq, ds = Dev(w8), Dev.empty(w8.shape, np.int8), Dev.empty(w8.shape[0])
    assert lib().atlas_quantize_int8_dev(dw8.ptr, 0, w8.shape[0], w8.shape[1], dq.ptr,
                                         ds.ptr) == 0
    assert np.array_equal(dq.get(), fx["q8_data"]) and np.array_equal(ds.get(), fx["q8_scales"])
    w4 = fx["q4_w"]
    dw4 = Dev(w4)
    d4, d4s = Dev.empty(fx["q4_data"].shape, np.uint8), Dev.empty(fx["q4_scales"].shape)
    assert lib().atlas_quantize_int4_dev(dw4.ptr, 0, w4.size, 32, d4.ptr, d4s.ptr) == 0
    assert np.array_equal(d4.get(), fx["q4_data"]) and np.array_equal(d4s.get(), fx["q4_scales"])


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "int8", "int4"])
def test_gpu_gemv_matches_fixtures(fx, fmt):
    _gpu_ready()
    from tests.gpu_util import Dev, lib, sync
    M, K = 64, 96
    dx, dy = Dev(fx["gemv_x"]), Dev.empty(M)
    if fmt == "bf16":
        dw = Dev(fx["gemv_bf16_w"])
        assert lib().atlas_gemv_bf16_f32(dw.ptr, dx.ptr, dy.ptr, M, K) == 0
        ref = fx["gemv_bf16_y"]
    elif fmt == "int8":
        dw, dsc = Dev(fx["gemv_i8_w"]), Dev(fx["gemv_i8_s"])
        assert lib().atlas_gemv_i8_f32(dw.ptr, dsc.ptr, dx.ptr, dy.ptr, M, K) == 0
        ref = fx["gemv_i8_y"]
    else:
        dw, dsc = Dev(fx["gemv_i4_w"]), Dev(fx["gemv_i4_s"])
        assert lib().atlas_gemv_i4_f32(dw.ptr, dsc.ptr, 32, dx.ptr, dy.ptr, M, K) == 0
        ref = fx["gemv_i4_y"]
    sync()
    assert _rel(dy.get(), ref) <= GEMV_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("window", [0, 8])
def test_gpu_attention_matches_fixtures(fx, window):
    _gpu_ready()
    from tests.gpu_util import Dev, lib, sync
    H, KVH, hd, pos = 4, 2, 32, 36
    dq, dk, dv, do = Dev(fx["attn_q"]), Dev(fx["attn_k"]), Dev(fx["attn_v"]), Dev.empty(H * hd)
    lib().atlas_decode_attention(dq.ptr, dk.ptr, dv.ptr, do.ptr, H, KVH, hd, pos,
                                 C.c_float(1.2079441541679836 / np.sqrt(hd)), window)
    sync()
    ref = fx["attn_out_w8"] if window else fx["attn_out_full"]
    assert _rel(do.get(), ref) <= ATTN_TOL


@pytest.mark.gpu
def test_gpu_model_matches_fixtures(fx):
    _gpu_ready()
    sys.path.insert(0, HERE)
    import modelgen
    from atlas_amd.model import SamplingConfig
    mg = _make_golden()
    W = modelgen.make_weights(mg.model_config(), seed=29, fmt="bf16")
    assert mg.weight_digest(W) == bytes(fx["model_digest"]).hex()
    m = modelgen.engine_model(W)
    m.reset()
    logits = m.forward_one(int(fx["model_prompt"][0]))
    assert _rel(logits, fx["model_logits0"]) <= GEMV_TOL
    got = m.generate_with_sampling([int(t) for t in fx["model_prompt"]], 16,
                                   SamplingConfig.greedy())
    assert got == [int(t) for t in fx["model_tokens"]]


@pytest.mark.gpu
def test_gpu_model_sampled_matches_fixture(fx):
    _gpu_ready()
    sys.path.insert(0, HERE)
    import modelgen
    from atlas_amd.model import SamplingConfig
    mg = _make_golden()
    W = modelgen.make_weights(mg.model_config(), seed=29, fmt="bf16")
    m = modelgen.engine_model(W)
    c = mg.sampled_config([int(fx["model_tokens"][0])])
    cfg = SamplingConfig(temperature=c["temperature"], repetition_penalty=c["repetition_penalty"],
                         repetition_window=c["repetition_window"],
                         frequency_penalty=c["frequency_penalty"],
                         presence_penalty=c["presence_penalty"], top_p=c["top_p"],
                         top_k=c["top_k"], min_p=c["min_p"],
                         suppress_initial_tokens=c["suppress"])
    m.set_rng_seed(mg.SAMPLED_SEED)
    got = m.generate_with_sampling([int(t) for t in fx["model_prompt"]], 24, cfg)
    assert got == [int(t) for t in fx["model_sampled_tokens"]]
