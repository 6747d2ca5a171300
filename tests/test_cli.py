"""Host logic of ``atlas_amd.cli`` (the ``atlas infer`` command,
crates/atlas-cli/src/main.rs:786-972): argument defaults, presets, shapes
from config.json, tokenizer loading and the byte-level fallback.  No GPU."""
import json

import pytest


def test_defaults_and_presets():
    from atlas_amd import cli
    a = cli.parse_args(["--weights", "/x"])
    assert (a.prompt, a.max_tokens, a.temperature, a.model, a.format) == (
        "The capital of France is", 50, 0.0, "smollm2-1.7b", "bf16")
    # main.rs:812-823 presets, lib.rs:109-205 / 253-269 shapes
    shapes = {k: (f().n_layers, f().d_model, f().n_heads, f().n_kv_heads, f().vocab_size)
              for k, f in cli.PRESETS.items()}
    assert shapes == {"smollm2-1.7b": (24, 2048, 32, 32, 49152),
                      "smollm2-135m": (30, 576, 9, 3, 49152),
                      "olmo3-1b": (16, 2048, 16, 16, 100352),
                      "olmo3-7b": (32, 4096, 32, 32, 100278),
                      "llama32-1b": (16, 2048, 32, 8, 128256)}
    assert cli.main([]) == 1


def test_config_from_hf_json(tmp_path):
    from atlas_amd import cli
    p = tmp_path / "config.json"
    p.write_text(json.dumps(dict(vocab_size=512, hidden_size=256, num_hidden_layers=4,
                                 num_attention_heads=8, intermediate_size=1024,
                                 rope_theta=1e6, rms_norm_eps=1e-6)))
    c = cli.config_from_hf_json(str(p))
    assert (c.vocab_size, c.d_model, c.n_layers, c.n_heads, c.n_kv_heads, c.ffn_hidden,
            c.max_seq_len, c.rope_theta, c.rms_norm_eps) == (512, 256, 4, 8, 8, 1024, 4096,
                                                              1e6, 1e-6)


def test_tokenizer_and_byte_fallback(tmp_path):
    from atlas_amd import cli
    tok, err = cli.load_tokenizer(str(tmp_path))
    assert tok is None and err
    assert cli.encode(None, "Hé") == [72, 195, 169]            # UTF-8 bytes (main.rs:846-849)
    assert cli.decode(None, [72, 195, 169, 256 + 33]) == "Hé!"  # t % 256 (main.rs:956-958)
    tokenizers = pytest.importorskip("tokenizers")
    vocab = {"[UNK]": 0, "the": 1, "capital": 2}
    t = tokenizers.Tokenizer(tokenizers.models.WordLevel(vocab, unk_token="[UNK]"))
    t.pre_tokenizer = tokenizers.pre_tokenizers.Whitespace()
    t.save(str(tmp_path / "tokenizer.json"))
    tok, err = cli.load_tokenizer(str(tmp_path))
    assert err is None and cli.encode(tok, "the capital x") == [1, 2, 0]
    assert cli.top1_last(__import__("numpy").array([1.0, 3.0, 3.0, 2.0])) == 2
