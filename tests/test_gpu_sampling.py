"""The device sampler (atlas_sample_device, the kernel the engine's generate
loop replays for temperature > 0 with 1 <= top_k <= 1024, or top_k = 0 with
top_p = 1) against the host sampler atlas_sample_host, which tests/test_sampling.py pins bit for bit to the
oracle's restatement of lib.rs:1623-1711.

The two must choose the same token and leave the same RNG state.  Their only
arithmetic difference is expf (glibc's vs exp rounded once from double: 1 ulp
apart for ~1e-4 of arguments); a choice can flip only if that ulp moves a
cumulative-probability boundary across the random draw (~1e-7 per draw), so
every case here is asserted equal.
"""
import ctypes as C

import numpy as np
import pytest

from tests.gpu_util import Dev, lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import atlas_amd
    atlas_amd.load()
    if not lib().atlas_cuda_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")


def _cfg(**kw):
    from atlas_amd._lib import SamplingC
    sup = np.ascontiguousarray(kw.pop("suppress", []) or [0], np.uint32)
    n_sup = kw.pop("n_suppress", None)
    d = dict(temperature=1.0, repetition_penalty=1.0, repetition_window=64, frequency_penalty=0.0,
             presence_penalty=0.0, top_p=1.0, top_k=50, min_p=0.0)
    d.update(kw)
    s = SamplingC(d["temperature"], d["repetition_penalty"], d["repetition_window"],
                  d["frequency_penalty"], d["presence_penalty"], d["top_p"], d["top_k"], d["min_p"],
                  sup.ctypes.data, len(sup) if n_sup is None else n_sup, -1, None, 0, 0)
    return s, sup


def _both(logits, hist, step, s, seed):
    """(host token, host state), (device token, device state)"""
    lg = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(list(hist) or [0], np.uint32)
    out = []
    for fn in ("host", "device"):
        st, tok = C.c_uint64(seed), C.c_uint32(0)
        if fn == "host":
            rc = lib().atlas_sample_host(lg.ctypes.data, lg.size, h.ctypes.data, len(hist), step,
                                         C.byref(s), C.byref(st), C.byref(tok))
        else:
            d = Dev(lg)
            rc = lib().atlas_sample_device(d.ptr, lg.size, h.ctypes.data, len(hist), step,
                                           C.byref(s), C.byref(st), C.byref(tok))
        assert rc == 0, (fn, lib().atlas_last_error())
        out.append((int(tok.value), int(st.value)))
    return out


def _random_case(rng, V):
    kind = rng.integers(0, 3)
    if kind == 0:
        lg = rng.standard_normal(V).astype(np.float32) * rng.uniform(0.5, 8.0)
    elif kind == 1:
        # heavy ties: a few distinct values, so top-k thresholds and top-p
        # cut-offs fall inside runs of equal logits
        lg = rng.integers(-4, 4, V).astype(np.float32)
    else:
        lg = (rng.standard_normal(V) * 3).astype(np.float32)
        lg[rng.integers(0, V, 40)] += 12.0          # a peaked head
    n_hist = int(rng.integers(0, 300))
    hist = [int(t) for t in rng.integers(0, V, n_hist)]
    if n_hist and rng.random() < 0.5:
        hist += hist[: n_hist // 2]                 # repeats
    s, keep = _cfg(temperature=float(rng.choice([0.3, 0.7, 1.0, 1.6])),
                   repetition_penalty=float(rng.choice([1.0, 1.15, 1.3])),
                   repetition_window=int(rng.choice([8, 64, 256])),
                   frequency_penalty=float(rng.choice([0.0, 0.1, 0.5])),
                   presence_penalty=float(rng.choice([0.0, 0.2])),
                   top_p=float(rng.choice([1.0, 0.95, 0.8, 0.5])),
                   top_k=int(rng.choice([0, 0, 1, 2, 5, 20, 50, 200, 1024])),
                   min_p=float(rng.choice([0.0, 0.02, 0.05, 0.2])),
                   suppress=[int(t) for t in rng.integers(0, V, rng.integers(0, 4))])
    if s.top_k == 0:
        s.top_p = 1.0                               # the device's whole-vocabulary path
    step = int(rng.choice([0, 0, 1, 7]))
    return lg, hist, step, s, keep


@pytest.mark.parametrize("V", [100278, 4093, 600])
def test_device_sampler_matches_host_random(V):
    rng = np.random.default_rng(V)
    n = 60 if V > 50000 else 120
    for case in range(n):
        lg, hist, step, s, keep = _random_case(rng, V)
        seed = int(rng.integers(1, 2**63)) * 2 + 1
        (th, sh), (td, sd) = _both(lg, hist, step, s, seed)
        assert (td, sd) == (th, sh), (V, case, s.top_k, s.top_p, s.min_p)


def test_device_sampler_olmo3_preset_many_draws():
    # SamplingConfig::olmo3 (lib.rs:1278-1294) over a 7B vocabulary, one
    # logit vector and 200 consecutive RNG states
    rng = np.random.default_rng(7)
    lg = (rng.standard_normal(100278) * 2.5).astype(np.float32)
    hist = [int(t) for t in rng.integers(0, 100278, 120)]
    s, keep = _cfg(temperature=0.6, repetition_penalty=1.15, repetition_window=256, top_p=0.95,
                   top_k=50, min_p=0.05, suppress=[14023])
    state = 0x9E3779B97F4A7C15
    seen = set()
    for i in range(200):
        (th, sh), (td, sd) = _both(lg, hist, 1, s, state)
        assert (td, sd) == (th, sh), i
        seen.add(td)
        state = sh
    assert len(seen) > 3                      # the draws explore the nucleus


def test_device_sampler_top_k_covers_small_vocab_and_long_history():
    rng = np.random.default_rng(3)
    # top_k >= V with V <= 1024: every token survives
    lg = rng.standard_normal(700).astype(np.float32)
    s, keep = _cfg(top_k=1000, top_p=0.9, temperature=0.9)
    for seed in range(1, 40, 2):
        (th, sh), (td, sd) = _both(lg, [], 3, s, seed)
        assert (td, sd) == (th, sh)
    # 4096 history tokens with the frequency and presence penalties
    lg = rng.standard_normal(50000).astype(np.float32) * 2
    hist = [int(t) for t in rng.integers(0, 300, 4096)]
    s, keep = _cfg(top_k=64, frequency_penalty=0.3, presence_penalty=0.4, repetition_penalty=1.2,
                   repetition_window=512)
    for seed in (3, 5, 11, 99):
        (th, sh), (td, sd) = _both(lg, hist, 9, s, seed)
        assert (td, sd) == (th, sh)


def _xorshift_u(state):
    """Rng::next_f32 after one step of XorShift64 (lib.rs:1190-1214)."""
    m = (1 << 64) - 1
    r = state
    r ^= (r << 13) & m
    r ^= r >> 7
    r ^= (r << 17) & m
    return np.float32(np.float32(r >> 33) / np.float32(2147483648.0)), r


def test_device_sampler_whole_vocabulary_band_and_fast_path():
    # top_k = 0 (SamplingConfig::default(): temperature 1, no top-k / top-p).
    # Equal logits put a cumulative boundary every 1/V, inside the f32
    # rounding band around any draw: every draw takes the sequential path.
    # A peaked vocabulary leaves most draws outside the band (exact prefix
    # sums decide).  Both must equal the host sampler, token and RNG state.
    V = 100278
    flat = np.zeros(V, np.float32)
    s, keep = _cfg(top_k=0, temperature=1.0)
    for seed in (3, 77, 0x9E3779B97F4A7C15 | 1, 2**62 + 1):
        (th, sh), (td, sd) = _both(flat, [], 1, s, seed)
        assert (td, sd) == (th, sh), seed
        u, _ = _xorshift_u(seed)
        # near u * V: the f32 running sum of 1/V drifts by ~1e-3 over 1e5 adds
        assert abs(th - float(u) * V) <= 0.01 * V, (th, float(u))
    rng = np.random.default_rng(11)
    lg = (rng.standard_normal(V) * 1.5).astype(np.float32)
    lg[rng.integers(0, V, 30)] += 9.0
    state = 12345
    for i in range(100):
        (th, sh), (td, sd) = _both(lg, [], 1, s, state)
        assert (td, sd) == (th, sh), i
        state = sh
    # min-p and penalties on the whole-vocabulary path
    hist = [int(t) for t in rng.integers(0, V, 50)]
    s2, keep2 = _cfg(top_k=0, temperature=0.8, min_p=0.01, repetition_penalty=1.2,
                     frequency_penalty=0.2, presence_penalty=0.1, suppress=[int(lg.argmax())])
    for seed in range(1, 60, 2):
        (th, sh), (td, sd) = _both(lg, hist, 0, s2, seed)
        assert (td, sd) == (th, sh), seed


def test_device_sampler_rejects_what_it_does_not_cover():
    lg = Dev(np.zeros(2000, np.float32))
    st, tok = C.c_uint64(1), C.c_uint32(0)
    for kw in (dict(top_k=0, top_p=0.9), dict(top_k=1025), dict(temperature=0.0)):
        s, keep = _cfg(**kw)
        assert lib().atlas_sample_device(lg.ptr, 2000, None, 0, 0, C.byref(s), C.byref(st),
                                         C.byref(tok)) == -4
    h = np.zeros(4097, np.uint32)
    for kw in (dict(top_k=10, frequency_penalty=0.1),
               dict(top_k=10, repetition_penalty=1.1, repetition_window=5000)):
        s, keep = _cfg(**kw)
        assert lib().atlas_sample_device(lg.ptr, 2000, h.ctypes.data, 4097, 1, C.byref(s),
                                         C.byref(st), C.byref(tok)) == -4
    lib().atlas_clear_error()           # the expected refusals leave their message behind


def test_generate_device_sampling_matches_host_sampling():
    # generate_with_sampling (device sampler in the captured step) against
    # generate_streaming (host sampler per token) on the same model and seed
    import sys
    import os
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import modelgen
    from atlas_amd.model import SamplingConfig
    cfg = modelgen.olmo3_small_config(max_seq=96)
    W = modelgen.make_weights(cfg, seed=61)
    m = modelgen.engine_model(W)
    prompt = [5, 17, 200, 3, 44]
    for sc in (SamplingConfig(temperature=0.8, top_k=40, top_p=0.9, min_p=0.02,
                              repetition_penalty=1.1, repetition_window=16,
                              frequency_penalty=0.1, presence_penalty=0.1,
                              suppress_initial_tokens=[7]),
               SamplingConfig(temperature=1.3, top_k=5),
               SamplingConfig()):                     # top_k = 0: the whole vocabulary
        for seed in (11, 12345):
            m.set_rng_seed(seed)
            dev = m.generate_with_sampling(prompt, 40, sc)
            m.set_rng_seed(seed)
            host = []
            m.generate_streaming(prompt, 40, sc, lambda t: host.append(t) or True)
            assert dev == host, (seed, sc.top_k)
