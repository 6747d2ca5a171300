"""CPU checks of the drop-in boundary: the C-ABI library loads, exports every
symbol include/*.h declares, and the host-side mirrors of atlas-quant are
bit-exact to the oracle.  No GPU calls."""
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        src = open(os.path.join(ROOT, "include", h)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names |= set(re.findall(r"\b(atlas_[a-z0-9_]+)\s*\(", src))
    return names


@pytest.fixture(scope="module")
def lib():
    import atlas_amd
    from atlas_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from atlas_amd import build
        build.build()
    return atlas_amd.load()


def test_library_exports_every_declared_symbol(lib):
    from atlas_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.split()[-1].startswith("atlas_")}
    declared = _declared()
    assert declared, "no declarations parsed"
    missing = declared - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    # the ctypes table covers exactly the declared surface
    assert set(_lib.SIGNATURES) == declared
    for name in declared:
        assert hasattr(lib, name)


def test_reference_ffi_names_present():
    # the 19 names crates/atlas-tensor/src/lib.rs:17-92 declares
    ref = ["atlas_matmul_f32", "atlas_vec_add_f32", "atlas_scale_f32", "atlas_relu_f32",
           "atlas_softmax_f32", "atlas_cuda_available", "atlas_cuda_device_count",
           "atlas_rmsnorm_f32", "atlas_rope_apply_f32", "atlas_silu_mul_f32",
           "atlas_vram_copy_f32", "atlas_adamw_step", "atlas_sgemm_bf16_f32", "atlas_sync",
           "atlas_qk_norm_inplace", "atlas_rope_precomputed", "atlas_kv_cache_write",
           "atlas_decode_attention", "atlas_gpu_argmax"]
    assert set(ref) <= _declared()


def test_no_device_means_no_gpu_work(lib):
    from atlas_amd import tensor as t
    if t.cuda_available():
        pytest.skip("a device is present")
    assert t.cuda_device_count() == 0
    m = t.GpuMatrix.upload(np.ones(12, np.float32), 4, 3)
    assert not m.is_on_gpu()
    out = np.zeros(4, np.float32)
    assert m.sgemm(np.ones(3, np.float32), 3, 1, out) is False     # lib.rs:371-400 contract
    assert t.GpuKvCache.new(8, 2, 4) is None


def test_host_quantisers_bit_exact(orc, lib):
    from atlas_amd.quant import Int4Tensor, Int8Tensor
    rng = np.random.default_rng(1)
    for shape in [(7, 33), (64, 256), (1, 1), (3, 5)]:
        w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        w[0, 0] = 0.0
        a = Int8Tensor.quantize(w)
        q, s = orc.int8_quantize(w)
        assert np.array_equal(a.data.reshape(shape), q) and np.array_equal(a.scales, s)
        assert np.array_equal(a.dequantize(), orc.int8_dequantize(q, s))
        for bs in (32, 64, 4, 3):
            b = Int4Tensor.quantize(w, bs)
            q4, s4 = orc.int4_quantize(w, bs)
            assert np.array_equal(b.data, q4) and np.array_equal(b.scales, s4)
            assert np.array_equal(b.dequantize(), orc.int4_dequantize(q4, s4, *shape, bs))
    z = Int8Tensor.quantize(np.zeros((2, 3), np.float32))
    assert list(z.scales) == [1.0, 1.0]
    assert Int8Tensor.quantize(np.ones((128, 128), np.float32)).compression_ratio() > 3.5
    assert Int4Tensor.quantize(np.ones((128, 128), np.float32), 64).compression_ratio() > 7.0


def test_model_config_presets():
    from atlas_amd.model import ModelConfig, SamplingConfig
    c = ModelConfig.olmo3_actual_7b()
    assert (c.vocab_size, c.d_model, c.n_layers, c.n_heads, c.n_kv_heads, c.ffn_hidden) == \
        (100278, 4096, 32, 32, 32, 11008)
    assert c.head_dim() == 128 and c.kv_dim() == 4096
    assert sum(1 for t in c.layer_types if t == "sliding") == 24
    assert [i for i, t in enumerate(c.layer_types) if t == "full"] == [3, 7, 11, 15, 19, 23, 27, 31]
    s = SamplingConfig.olmo3()
    assert s.suppress_initial_tokens == [14023] and s.top_k == 50


def test_stream_rule_library_wide_with_thread_override(lib):
    """atlas_set_stream is library-wide: another thread without an override
    sees it; atlas_set_thread_stream overrides it for the calling thread only.
    The handles are never used for work here (no HIP call takes them)."""
    import ctypes as C
    import threading
    a, b = C.c_void_p(0x1000), C.c_void_p(0x2000)
    seen = {}

    def other():
        seen["before"] = lib.atlas_get_stream()
        lib.atlas_set_thread_stream(b)
        seen["override"] = lib.atlas_get_stream()
        lib.atlas_clear_thread_stream()
        seen["cleared"] = lib.atlas_get_stream()

    try:
        assert lib.atlas_set_stream(a) == 0
        assert lib.atlas_get_stream() == 0x1000
        t = threading.Thread(target=other)
        t.start()
        t.join()
        assert seen == {"before": 0x1000, "override": 0x2000, "cleared": 0x1000}
        assert lib.atlas_get_stream() == 0x1000          # the override stayed on its thread
    finally:
        lib.atlas_set_stream(None)
    assert not lib.atlas_get_stream()
