"""Temperature sampling of generate_with_sampling (crates/atlas-model/src/lib.rs:1599-1732).

The oracle's restatement (oracle.c orc_rng_next ... orc_generate_sampled) is
pinned by the reference's own literal tests (lib.rs:2845-2985), by an
independent pure-Python XorShift64, by brute-force rules for the filters, by
tests whose outcome depends on the order of the pipeline's stages, and by a
chi-square test of the sampled distribution.  The library's host sampler
(atlas_sample_host) must then agree with the oracle bit for bit -- token and
RNG state -- on random configurations.  All of this runs on the CPU: the
sampler is host code (the logits are downloaded once per step).
"""
import math

import numpy as np
import pytest

import oracle as orc

NEG = float("-inf")


# ---- reference literal tests --------------------------------------------------

def test_ref_sample_from_probs_basic():
    # lib.rs:2868-2876
    p = [0.1, 0.2, 0.3, 0.4]
    assert [orc.sample_from_probs(p, r) for r in (0.0, 0.05, 0.15, 0.35, 0.95)] == [0, 0, 1, 2, 3]


def test_ref_repetition_penalty():
    # lib.rs:2880-2899
    lg = orc.repetition_penalty([1.0, 2.0, 3.0, -1.0], [1, 3], 1.5)
    assert lg[1] == np.float32(2.0) / np.float32(1.5) and lg[3] == -1.5
    assert lg[0] == 1.0 and lg[2] == 3.0
    orig = [1.0, 2.0, 3.0, -1.0]
    assert list(orc.repetition_penalty(orig, [0, 1, 2, 3], 1.0)) == orig


def test_ref_top_p():
    # lib.rs:2901-2920; probabilities ~[0.06, 0.11, 0.22, 0.60]: the top token
    # alone reaches p = 0.5, so it is the only survivor
    lg = orc.top_p([-1.0, 0.0, 0.7, 1.7], 0.5)
    assert lg[3] == np.float32(1.7) and all(v == NEG for v in lg[:3])
    assert np.all(orc.top_p([1.0, 2.0, 3.0, 4.0], 1.0) > NEG)


def test_ref_top_k():
    # lib.rs:2922-2941
    lg = orc.top_k([1.0, 5.0, 3.0, 2.0, 4.0], 3)
    assert list(lg) == [NEG, 5.0, 3.0, NEG, 4.0]
    assert list(orc.top_k([1.0, 5.0, 3.0, 2.0, 4.0], 0)) == [1.0, 5.0, 3.0, 2.0, 4.0]


def test_ref_min_p():
    # lib.rs:2943-2954
    assert list(orc.min_p([10.0, 0.0, -5.0, 9.0], 0.1)) == [10.0, NEG, NEG, 9.0]


def test_ref_frequency_and_presence():
    # lib.rs:2956-2975
    lg = orc.frequency_penalty([1.0, 2.0, 3.0], [1, 2], [3, 1], 0.5)
    assert list(lg) == [1.0, 0.5, 2.5]
    assert list(orc.presence_penalty([1.0, 2.0, 3.0], [0, 2], 0.5)) == [0.5, 2.0, 2.5]


def test_ref_sampling_config_presets():
    # lib.rs:2977-2990 and the presets at lib.rs:1250-1294
    from atlas_amd.model import SamplingConfig
    d = SamplingConfig()
    assert (d.temperature, d.repetition_penalty, d.repetition_window, d.top_p, d.top_k,
            d.min_p) == (1.0, 1.0, 64, 1.0, 0, 0.0)
    o = SamplingConfig.olmo3()
    assert abs(o.temperature - 0.6) < 0.01 and abs(o.repetition_penalty - 1.15) < 0.01


# ---- RNG ----------------------------------------------------------------------

def _xorshift(seed, n):
    s, out = (seed | 1) & (2**64 - 1), []
    for _ in range(n):
        s ^= (s << 13) & (2**64 - 1)
        s ^= s >> 7
        s ^= (s << 17) & (2**64 - 1)
        out.append(np.float32(s >> 33) / np.float32(2**31))
    return out


@pytest.mark.parametrize("seed", [0, 1, 42, 0xDEADBEEF, 2**63 + 5, 2**64 - 1])
def test_rng_matches_python_xorshift(seed):
    r = orc.Rng(seed)
    got = [r.next_f32() for _ in range(1000)]
    want = _xorshift(seed, 1000)
    assert [np.float32(g) for g in got] == want
    assert all(0.0 <= v < 1.0 for v in got)          # lib.rs:2845-2852 (bound 2.0)
    assert len(set(got)) > 990                          # lib.rs:2854-2866


# ---- brute-force rules of the filters ------------------------------------------

def test_top_k_keeps_the_first_k_by_value_then_index():
    rng = np.random.default_rng(5)
    for _ in range(300):
        n = int(rng.integers(1, 24))
        lg = rng.integers(-3, 4, n).astype(np.float32)        # many ties
        k = int(rng.integers(0, n + 2))
        got = orc.top_k(lg, k)
        if k == 0 or k >= n:
            assert np.array_equal(got, lg)
            continue
        keep = sorted(range(n), key=lambda i: (-lg[i], i))[:k]
        want = np.full(n, NEG, np.float32)
        want[keep] = lg[keep]
        assert np.array_equal(got, want)


def test_top_p_keeps_the_smallest_nucleus():
    rng = np.random.default_rng(6)
    checked = 0
    for _ in range(400):
        n = int(rng.integers(1, 40))
        lg = (rng.standard_normal(n) * 2).astype(np.float32)
        p = float(rng.uniform(0.05, 1.0))
        pr = np.exp(lg.astype(np.float64) - lg.max())
        pr /= pr.sum()
        order = np.argsort(-pr, kind="stable")
        cum = np.cumsum(pr[order])
        if np.min(np.abs(cum - p)) < 1e-5:
            continue                                    # float32 vs float64 decides
        cut = int(np.argmax(cum >= p)) + 1 if cum[-1] >= p else n
        want = np.full(n, NEG, np.float32)
        want[order[:cut]] = lg[order[:cut]]
        assert np.array_equal(orc.top_p(lg, p), want)
        checked += 1
    assert checked > 350


def test_min_p_threshold():
    rng = np.random.default_rng(7)
    for _ in range(300):
        n = int(rng.integers(1, 40))
        lg = (rng.standard_normal(n) * 3).astype(np.float32)
        mp = float(rng.uniform(0.0, 1.0))
        th = float(lg.max()) + math.log(mp) if mp > 0 else -math.inf
        if np.min(np.abs(lg - th)) < 1e-5:
            continue
        want = np.where(lg >= th, lg, NEG).astype(np.float32)
        assert np.array_equal(orc.min_p(lg, mp), want)
    assert np.array_equal(orc.min_p([1.0, -50.0], 0.0), np.float32([1.0, -50.0]))


def test_sample_from_probs_is_inverse_cdf():
    rng = np.random.default_rng(8)
    for _ in range(300):
        n = int(rng.integers(1, 30))
        p = rng.random(n).astype(np.float32)
        p /= p.sum()
        r = np.float32(rng.random())
        cum = np.cumsum(p, dtype=np.float32)            # sequential float32 sums
        idx = np.nonzero(r < cum)[0]
        assert orc.sample_from_probs(p, float(r)) == (int(idx[0]) if idx.size else n - 1)


# ---- the pipeline --------------------------------------------------------------

def _step(lg, hist=(), step=1, seed=3, **kw):
    # small seeds give a tiny first XorShift draw: spread them over 64 bits
    rng = orc.Rng(((seed + 1) * 0x9E3779B97F4A7C15) % 2**64)
    return orc.sample_step(np.float32(lg), list(hist), step, orc.sampling(**kw), rng)


def test_greedy_is_argmax_after_suppression_and_repetition():
    lg = [1.0, 4.0, 3.9, -2.0]
    assert _step(lg, temperature=0.0) == 1
    assert _step(lg, temperature=1e-7) == 1                 # below the 1e-6 threshold
    assert _step(lg, step=0, temperature=0.0, suppress=[1]) == 2
    assert _step(lg, step=1, temperature=0.0, suppress=[1]) == 1   # step 0 only
    # 4.0 / 1.1 < 3.9: the repeated token loses; outside the window it does not
    assert _step(lg, hist=[1], temperature=0.0, repetition_penalty=1.1) == 2
    assert _step(lg, hist=[1, 0, 0], temperature=0.0, repetition_penalty=1.1,
                 repetition_window=2) == 1
    # ties go to the last maximum (Iterator::max_by)
    assert _step([2.0, 5.0, 5.0, 1.0], temperature=0.0) == 2


def test_penalties_apply_before_temperature():
    # frequency: (2 - 0.5) / 0.5 < 1.9 / 0.5, but 2 / 0.5 - 0.5 > 1.9 / 0.5
    for seed in range(20):
        assert _step([2.0, 1.9], hist=[0], seed=seed, temperature=0.5,
                     frequency_penalty=0.5, top_k=1) == 1
        assert _step([2.0, 1.9], hist=[0, 0], seed=seed, temperature=0.5,
                     presence_penalty=0.5, top_k=1) == 1


def test_min_p_applies_after_temperature():
    # [0, -1] / 0.5 = [0, -2] and ln 0.3 = -1.20: token 1 is dropped only when
    # min_p sees the tempered logits
    seen = {_step([0.0, -1.0], seed=s, temperature=0.5, min_p=0.3) for s in range(200)}
    assert seen == {0}
    seen = {_step([0.0, -1.0], seed=s, temperature=1.0, min_p=0.3) for s in range(200)}
    assert seen == {0, 1}


def test_top_k_applies_before_top_p():
    # [3, 2.9, 2.8]: top_k=2 first leaves probabilities [0.525, 0.475], so
    # top_p=0.5 keeps token 0 alone; top_p over all three ([0.37, 0.33, 0.30])
    # would keep tokens 0 and 1
    seen = {_step([3.0, 2.9, 2.8], seed=s, top_k=2, top_p=0.5) for s in range(200)}
    assert seen == {0}
    seen = {_step([3.0, 2.9, 2.8], seed=s, top_p=0.5) for s in range(200)}
    assert seen == {0, 1}


def test_sampled_distribution_matches_tempered_softmax():
    lg = np.float32([1.0, 0.5, 0.0, -0.5, -1.0, 2.0, 0.25, -2.0])
    T, n = 0.7, 40000
    rng, s = orc.Rng(1234), orc.sampling(temperature=T)
    counts = np.zeros(lg.size)
    for _ in range(n):
        counts[orc.sample_step(lg, [], 1, s, rng)] += 1
    p = np.exp(lg.astype(np.float64) / T)
    p /= p.sum()
    chi2 = float(np.sum((counts - n * p) ** 2 / (n * p)))
    assert chi2 < 24.3            # chi-square, 7 dof, p = 0.001
    # the same draws at temperature 1 / 0.7 (multiplied instead of divided)
    # are far off
    q = np.exp(lg.astype(np.float64) * T)
    q /= q.sum()
    assert float(np.sum((counts - n * q) ** 2 / (n * q))) > 1000


# ---- the library's host sampler against the oracle ------------------------------

def _random_cfg(rng):
    from atlas_amd.model import SamplingConfig
    pick = lambda a, b, off: float(rng.uniform(a, b)) if rng.random() < 0.6 else off  # noqa: E731
    return SamplingConfig(
        temperature=float(rng.choice([0.0, 1e-7, 0.3, 0.6, 1.0, 1.7])),
        repetition_penalty=pick(1.01, 1.5, 1.0),
        repetition_window=int(rng.integers(1, 12)),
        frequency_penalty=pick(-0.5, 1.0, 0.0),
        presence_penalty=pick(-0.5, 1.0, 0.0),
        top_p=pick(0.05, 0.999, 1.0),
        top_k=int(rng.integers(1, 12)) if rng.random() < 0.5 else 0,
        min_p=pick(0.001, 0.5, 0.0),
        suppress_initial_tokens=[int(t) for t in rng.integers(0, 140, int(rng.integers(0, 4)))])


def test_library_sampler_matches_oracle():
    from atlas_amd.model import sample_host
    rng = np.random.default_rng(11)
    for case in range(600):
        V = int(rng.choice([1, 2, 7, 33, 128, 1000]))
        if rng.random() < 0.3:
            lg = rng.integers(-3, 3, V).astype(np.float32)          # ties
        else:
            lg = (rng.standard_normal(V) * 3).astype(np.float32)
        hist = [int(t) for t in rng.integers(0, V + 3, int(rng.integers(0, 20)))]
        step = int(rng.integers(0, 3))
        cfg = _random_cfg(rng)
        seed = int(rng.integers(0, 2**63))
        o = orc.Rng(seed)
        s = orc.sampling(cfg.temperature, cfg.top_p, cfg.top_k, cfg.min_p,
                         cfg.repetition_penalty, cfg.repetition_window, cfg.frequency_penalty,
                         cfg.presence_penalty, cfg.suppress_initial_tokens)
        want = orc.sample_step(lg, hist, step, s, o)
        got, state = sample_host(lg, hist, step, cfg, seed | 1)
        assert (got, state) == (want, o.state.value), (case, V, cfg)


def test_library_sampler_rejects_bad_arguments():
    import ctypes as C
    from atlas_amd import load
    from atlas_amd._lib import SamplingC
    L = load()
    st, tok = C.c_uint64(1), C.c_uint32(0)
    x = np.zeros(4, np.float32)
    s = SamplingC(1.0, 1.0, 64, 0.0, 0.0, 1.0, 0, 0.0, None, 0, -1, None, 0, 0)
    assert L.atlas_sample_host(x.ctypes.data, 0, None, 0, 0, C.byref(s), C.byref(st),
                               C.byref(tok)) < 0
    assert L.atlas_sample_host(x.ctypes.data, 4, None, 2, 0, C.byref(s), C.byref(st),
                               C.byref(tok)) < 0
    assert L.atlas_sample_host(x.ctypes.data, 4, None, 0, 0, None, C.byref(st),
                               C.byref(tok)) == 0 and tok.value == 3   # NULL config: greedy
