"""CPU tests of the checkpoint loader's host side (include/atlas_loader.h):
safetensors parsing, f16/bf16 conversion, config.json overlay, and the
loader's checks that run before any device work.

The reference's own tests are restated first (crates/atlas-model/src/lib.rs:
safetensors_header_parse 3126-3153, f16_to_f32_conversion 3155-3197,
bf16_to_f32_conversion 3200-3236, safetensors_roundtrip 3308-3349,
config_json_parsing_olmo3_fields 3521-3591, test_olmo3_config_parsed
4383-4420).  f16_to_f32 is also checked against numpy's IEEE half
conversion for all 65536 bit patterns, and files are written by an
independent writer (tests/ckptgen.py, the json module).
"""
import json
import os
import struct
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import ckptgen  # noqa: E402


@pytest.fixture(scope="module")
def ld():
    import atlas_amd
    from atlas_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from atlas_amd import build
        build.build()
    atlas_amd.load()
    from atlas_amd import loader
    return loader


def _err(fn, *a):
    from atlas_amd._lib import AtlasError
    with pytest.raises(AtlasError) as e:
        fn(*a)
    return str(e.value)


# ---- the reference's tests ----------------------------------------------------

def test_safetensors_header_parse(ld):
    a = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0]
    b = [7.0, 8.0]
    st = ld.SafetensorsFile.from_bytes(ld.SafetensorsFile.build_f32([("weight_a", [2, 3], a),
                                                                      ("bias_b", [2], b)]))
    assert st.len() == 2
    assert "weight_a" in st.tensor_names() and "bias_b" in st.tensor_names()
    da = st.get_desc("weight_a")
    assert da.dtype == "F32" and da.shape == [2, 3]
    assert st.get_desc("bias_b").shape == [2]
    assert st.get_f32("weight_a").tolist() == a
    assert st.get_f32("bias_b").tolist() == b


def test_f16_to_f32_reference_literals(ld):
    f = ld.f16_to_f32
    assert abs(f(0x3C00) - 1.0) < 1e-6 and abs(f(0xBC00) + 1.0) < 1e-6
    assert f(0x0000) == 0.0 and np.signbit(f(0x8000)) and f(0x8000) == 0.0
    assert abs(f(0x3800) - 0.5) < 1e-6 and abs(f(0x7BFF) - 65504.0) < 1.0
    assert f(0x7C00) == float("inf") and f(0xFC00) == float("-inf") and np.isnan(f(0x7C01))
    assert 0.0 < f(0x0001) < 1e-6
    # an F16 tensor in a file
    raw = struct.pack("<HH", 0x3C00, 0x3800)
    st = ld.SafetensorsFile.from_bytes(ckptgen.safetensors_bytes([("x", "F16", [2], raw)]))
    assert st.get_f32("x").tolist() == [1.0, 0.5]


def test_f16_to_f32_all_bit_patterns(ld):
    # every half: numpy's IEEE conversion, except that every NaN becomes the
    # canonical quiet NaN (f32::NAN), as the reference returns
    h = np.arange(65536, dtype=np.uint16)
    st = ld.SafetensorsFile.from_bytes(ckptgen.safetensors_bytes([("h", "F16", [65536],
                                                                   h.tobytes())]))
    got = st.get_f32("h").view(np.uint32)
    want = h.view(np.float16).astype(np.float32).view(np.uint32).copy()
    nan = np.isnan(h.view(np.float16))
    want[nan] = 0x7FC00000
    assert np.array_equal(got, want)
    # the scalar entry point agrees
    for v in (0x0001, 0x03FF, 0x0400, 0x8001, 0x7BFF, 0xFBFF, 0x7E00, 0xFC01):
        assert np.float32(ld.f16_to_f32(v)).view(np.uint32) == got[v]


def test_bf16_to_f32_reference_literals(ld):
    bits = [0x3F80, 0xC000, 0x0000]
    st = ld.SafetensorsFile.from_bytes(ckptgen.safetensors_bytes(
        [("y", "BF16", [3], struct.pack("<3H", *bits))]))
    assert st.get_f32("y").tolist() == [1.0, -2.0, 0.0]
    assert st.get_bf16("y").tolist() == bits


def test_safetensors_roundtrip(ld):
    w1 = [0.1, -0.2, 0.3, 0.4, -0.5, 0.6]
    w2, w3 = [1.0, 2.0, 3.0], [-1.0]
    st = ld.SafetensorsFile.from_bytes(ld.SafetensorsFile.build_f32(
        [("layer.0.weight", [2, 3], w1), ("layer.1.bias", [3], w2), ("scalar", [1], w3)]))
    assert st.len() == 3
    assert st.contains("layer.0.weight") and st.contains("scalar")
    assert not st.contains("nonexistent")
    assert np.array_equal(st.get_f32("layer.0.weight"), np.float32(w1))
    assert st.get_f32("layer.1.bias").tolist() == w2 and st.get_f32("scalar").tolist() == w3
    assert st.get_desc("layer.0.weight").shape == [2, 3]
    assert st.get_desc("layer.1.bias").shape == [3]


OLMO3_LAYER_TYPES = (["sliding_attention"] * 3 + ["full_attention"]) * 8


def _patch(ld, tmp_path, obj, base=None):
    from atlas_amd.model import ModelConfig
    p = tmp_path / "config.json"
    p.write_text(obj if isinstance(obj, str) else json.dumps(obj))
    return ld.patch_config_from_hf_json(base or ModelConfig.olmo3_actual_7b(), str(p))


def test_config_json_olmo3_fields(ld, tmp_path):
    js = {"vocab_size": 100278, "hidden_size": 4096, "num_hidden_layers": 32,
          "num_attention_heads": 32, "num_key_value_heads": 32, "sliding_window": 4096,
          "rope_theta": 500000.0, "rms_norm_eps": 1e-06, "layer_types": OLMO3_LAYER_TYPES,
          "rope_scaling": {"rope_type": "yarn", "factor": 8.0,
                           "original_max_position_embeddings": 8192,
                           "attention_factor": 1.2079441541679836, "beta_fast": 32.0,
                           "beta_slow": 1.0}}
    from atlas_amd.model import ModelConfig
    base = ModelConfig.olmo3_actual_7b()
    base.layer_types, base.sliding_window, base.rope_scaling = [], None, None
    c = _patch(ld, tmp_path, js, base)
    assert len(c.layer_types) == 32
    assert c.layer_types.count("full") == 8 and c.layer_types.count("sliding") == 24
    assert all(c.layer_types[i] == "full" for i in (3, 7, 11, 15, 19, 23, 27, 31))
    assert c.sliding_window == 4096
    y = c.rope_scaling
    assert abs(y.factor - 8.0) < 1e-4 and y.orig_max_pos == 8192
    assert abs(y.attn_factor - 1.2079) < 1e-3 and y.beta_fast == 32.0 and y.beta_slow == 1.0
    assert abs(c.rope_theta - 500000.0) < 1.0 and c.rms_norm_eps < 1e-5


def test_olmo3_config_parsed_over_tiny(ld, tmp_path):
    from atlas_amd.model import ModelConfig
    text = """{
        "layer_types": ["sliding_attention","sliding_attention","sliding_attention","full_attention",
                        "sliding_attention","sliding_attention","sliding_attention","full_attention"],
        "sliding_window": 4096, "rope_theta": 500000, "rms_norm_eps": 1e-6,
        "rope_scaling": {"rope_type": "yarn", "factor": 8.0,
            "original_max_position_embeddings": 8192, "attention_factor": 1.2079441541679836,
            "beta_fast": 32.0, "beta_slow": 1.0}}"""
    c = _patch(ld, tmp_path, text, ModelConfig.tiny())
    assert len(c.layer_types) == 8 and c.layer_types[0] == "sliding" and c.layer_types[3] == "full"
    assert c.layer_types.count("sliding") == 6 and c.layer_types.count("full") == 2
    assert c.sliding_window == 4096 and abs(c.rope_theta - 500000.0) < 1.0
    assert abs(c.rms_norm_eps - np.float32(1e-6)) < 1e-10
    y = c.rope_scaling
    assert abs(y.factor - 8.0) < 1e-5 and y.orig_max_pos == 8192
    assert abs(y.attn_factor - 1.2079) < 1e-3 and y.beta_fast == 32.0 and y.beta_slow == 1.0
    # the other fields are the caller's
    assert c.d_model == 64 and c.n_layers == 2 and c.max_seq_len == 128


# ---- config.json semantics the reference's code fixes ---------------------------

def test_config_defaults_and_ignored_values(ld, tmp_path):
    from atlas_amd.model import ModelConfig
    base = ModelConfig.tiny()
    # YaRN without fields: factor 1, orig = the caller's max_seq_len, attn 1,
    # betas 32 / 1; an integer-valued float is a usize; eos as u32
    c = _patch(ld, tmp_path, {"rope_scaling": {"rope_type": "yarn"}, "sliding_window": 64.0,
                              "eos_token_id": 100257}, base)
    y = c.rope_scaling
    assert (y.factor, y.orig_max_pos, y.attn_factor, y.beta_fast, y.beta_slow) == \
        (1.0, base.max_seq_len, 1.0, 32.0, 1.0)
    assert c.sliding_window == 64 and c.eos_token_id == 100257
    # another rope_type, a negative window, a list-valued eos: no change;
    # non-string layer types are Full; absent keys keep the caller's values
    c = _patch(ld, tmp_path, {"rope_scaling": {"rope_type": "linear", "factor": 4.0},
                              "sliding_window": -1, "eos_token_id": [1, 2],
                              "layer_types": ["sliding_attention", 7, None]}, base)
    assert c.rope_scaling is None and c.sliding_window is None and c.eos_token_id is None
    assert c.layer_types == ["sliding", "full", "full"]
    assert c.rope_theta == base.rope_theta and c.rms_norm_eps == np.float32(base.rms_norm_eps)
    # a JSON error and a missing file are errors
    assert "parse" in _err(_patch, ld, tmp_path, '{"rope_theta": 1,}', base)
    assert "read" in _err(ld.patch_config_from_hf_json, base, str(tmp_path / "absent.json"))


# ---- safetensors parsing: errors and header semantics ----------------------------

def _hdr(obj_text: str, data=b""):
    h = obj_text.encode()
    return struct.pack("<Q", len(h)) + h + data


def header_error_cases():
    """Files SafetensorsFile.from_bytes rejects, with the message each gives
    (also the corpus of the sanitizer run, tests/test_loader_sanitize.py)."""
    raw = b'{"\xff": 1}'
    return [(b"\x01\x00", "too short"),
            (struct.pack("<Q", 100) + b"{}", "truncated"),
            (struct.pack("<Q", 2**64 - 1) + b"{}", "truncated"),
            (struct.pack("<Q", len(raw)) + raw, "UTF-8"),
            (_hdr('{"a": {"dtype": "F32",}}'), "JSON"),
            (_hdr('{"a": 1} x'), "JSON"),
            (_hdr('{"a": {"dtype": "F32", "shape": [1]}}'), "missing data_offsets"),
            (_hdr('{"a": {"data_offsets": [0]}}'), "two entries"),
            (_hdr("[" * 600 + "]" * 600), "nesting")]


def range_error_file():
    """A file that parses, whose tensors fail on read: an unsupported dtype, a
    range past the data section and a reversed range."""
    return _hdr('{"a": {"dtype": "I8", "shape": [4], "data_offsets": [0, 4]},'
                ' "b": {"dtype": "F32", "shape": [1], "data_offsets": [0, 8]},'
                ' "c": {"dtype": "F32", "shape": [1], "data_offsets": [4, 2]}}', b"\0" * 4)


def test_safetensors_errors(ld):
    fb = ld.SafetensorsFile.from_bytes
    for blob, msg in header_error_cases():
        assert msg in _err(fb, blob), msg
    st = fb(range_error_file())
    assert "unsupported dtype: I8" in _err(st.get_f32, "a")
    assert "not BF16" in _err(st.get_bf16, "a")
    assert "outside" in _err(st.get_f32, "b") and "outside" in _err(st.get_f32, "c")
    assert "not found" in _err(st.get_f32, "zz") and "not found" in _err(st.get_bf16, "zz")


def test_safetensors_header_semantics(ld):
    data = np.arange(6, dtype="<f4").tobytes()
    text = ('{"__metadata__": {"format": "pt"},'
            ' "w\\u0041\\ud83d\\ude00": {"shape": [2, -1, 3.9, "x"], "data_offsets": [0.0, 24.7]},'
            ' "dup": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},'
            ' "dup": {"dtype": "F32", "shape": [1], "data_offsets": [20, 24]},'
            ' "z": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 3]}}')
    st = ld.SafetensorsFile.from_bytes(_hdr(text, data))
    names = st.tensor_names()
    assert names == ["wA\U0001F600", "dup", "dup", "z"]        # header order, metadata skipped
    d = st.get_desc("wA\U0001F600")
    assert d.dtype == "F32"                                      # default dtype
    assert d.shape == [2, 3] and d.offsets == (0, 24)            # filter_map(as_usize)
    assert st.get_f32("wA\U0001F600").tolist() == [0, 1, 2, 3, 4, 5]
    assert st.get_f32("dup").tolist() == [0.0]                   # first match
    assert st.get_bf16("z").size == 1                            # chunks_exact(2) of 3 bytes
    # a root that is not an object has no tensors
    assert ld.SafetensorsFile.from_bytes(_hdr("[1, 2]")).is_empty()


def test_open_reads_a_file(ld, tmp_path):
    p = tmp_path / "m.safetensors"
    p.write_bytes(ld.SafetensorsFile.build_f32([("a", [2], [1.5, -2.5])]))
    st = ld.SafetensorsFile.open(str(p))
    assert st.get_f32("a").tolist() == [1.5, -2.5]
    from atlas_amd._lib import AtlasError
    with pytest.raises(AtlasError) as e:
        ld.SafetensorsFile.open(str(tmp_path / "none.safetensors"))
    assert e.value.code == -5


# ---- loader checks before any device work ------------------------------------------

def _tiny_w(**kw):
    import modelgen
    cfg = modelgen.tiny_config(**kw)
    return cfg, modelgen.make_weights(cfg, seed=5, fmt="bf16")


def _am_cfg(cfg):
    from atlas_amd import model as am
    return am.ModelConfig(vocab_size=cfg["vocab"], d_model=cfg["d_model"],
                          n_layers=cfg["n_layers"], n_heads=cfg["n_heads"],
                          n_kv_heads=cfg["n_kv_heads"], ffn_hidden=cfg["ffn_hidden"],
                          max_seq_len=cfg["max_seq"])


def test_loader_rejects_inconsistent_files(ld, tmp_path):
    cfg, W = _tiny_w()
    t = ckptgen.hf_tensors(W)
    # a matrix with the wrong element count
    bad = [(n, dt, sh, raw[:-4] if n.endswith("0.self_attn.q_proj.weight") else raw)
           for n, dt, sh, raw in t]
    ckptgen.write_dir(str(tmp_path / "a"), bad)
    assert "elements" in _err(ld.load_model_from_dir, str(tmp_path / "a"), _am_cfg(cfg))
    # a tensor no get_f32 can read, even under an unknown name
    ckptgen.write_dir(str(tmp_path / "b"), t + [("extra.counter", "I64", [1], b"\0" * 8)])
    assert "unsupported dtype" in _err(ld.load_model_from_dir, str(tmp_path / "b"), _am_cfg(cfg))
    # QK-norm weights for one layer only
    part = [x for x in t if not x[0].startswith("model.layers.1.self_attn.q_norm")]
    ckptgen.write_dir(str(tmp_path / "c"), part)
    assert "QK-norm" in _err(ld.load_model_from_dir, str(tmp_path / "c"), _am_cfg(cfg))
    # no model file
    os.makedirs(tmp_path / "d")
    assert "model.safetensors" in _err(ld.load_model_from_dir, str(tmp_path / "d"), _am_cfg(cfg))
    # a shard the index names is missing
    ckptgen.write_dir(str(tmp_path / "e"), t, shards=2)
    os.remove(tmp_path / "e" / "model-00002-of-00002.safetensors")
    assert "00002" in _err(ld.load_model_from_dir, str(tmp_path / "e"), _am_cfg(cfg))
