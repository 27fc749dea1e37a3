"""On-disk format: ``Qwen3Config.from_json`` (qwen3_naive.py:129-148) and
``load_weights`` (qwen3_naive.py:1682-1730), which packs the checkpoint's
separate q/k/v and gate/up matrices into the fused projections.

The packing is pinned against an independent implementation: a tiny
transformers ``Qwen3ForCausalLM`` whose weights are written in the published
Qwen3 safetensors naming (``q_proj``/``k_proj``/``v_proj``, ``gate_proj``/
``up_proj``, tied ``lm_head``); after loading, the product model's CPU forward
must give transformers' logits.  A transposed shard or a wrong offset moves
the logits by O(1)."""
import importlib
import json

import pytest
import torch

safetensors_torch = pytest.importorskip("safetensors.torch")


def _pkg():
    return importlib.import_module("qwen3-naive-inference_amd")


# Qwen3-0.6B's published config.json fields (the ones the reader uses).
QWEN3_06B = {
    "architectures": ["Qwen3ForCausalLM"], "attention_bias": False, "attention_dropout": 0.0,
    "bos_token_id": 151643, "eos_token_id": 151645, "head_dim": 128, "hidden_act": "silu",
    "hidden_size": 1024, "initializer_range": 0.02, "intermediate_size": 3072,
    "max_position_embeddings": 40960, "max_window_layers": 28, "model_type": "qwen3",
    "num_attention_heads": 16, "num_hidden_layers": 28, "num_key_value_heads": 8,
    "rms_norm_eps": 1e-06, "rope_scaling": None, "rope_theta": 1000000, "sliding_window": None,
    "tie_word_embeddings": True, "torch_dtype": "bfloat16", "use_cache": True,
    "use_sliding_window": False, "vocab_size": 151936,
}


def test_config_from_json_qwen3_06b(tmp_path):
    p = tmp_path / "config.json"
    p.write_text(json.dumps(QWEN3_06B))
    cfg = _pkg().Qwen3Config.from_json(str(p))
    assert cfg == _pkg().Qwen3Config()      # the defaults are Qwen3-0.6B
    assert (cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) == \
        (1024, 16, 8, 128)
    assert (cfg.intermediate_size, cfg.num_hidden_layers, cfg.vocab_size) == (3072, 28, 151936)
    assert cfg.rms_norm_eps == 1e-6 and cfg.rope_theta == 1000000 and cfg.tie_word_embeddings


def test_config_from_json_defaults(tmp_path):
    """Optional fields fall back as the reference's reader does: head_dim =
    hidden / heads, rope_theta 1e6, no attention bias, tied embeddings."""
    d = {k: QWEN3_06B[k] for k in ("hidden_size", "num_attention_heads", "num_key_value_heads",
                                   "intermediate_size", "num_hidden_layers", "vocab_size",
                                   "max_position_embeddings", "rms_norm_eps", "hidden_act")}
    d.update(hidden_size=2048, num_attention_heads=32)
    p = tmp_path / "config.json"
    p.write_text(json.dumps(d))
    cfg = _pkg().Qwen3Config.from_json(str(p))
    assert cfg.head_dim == 64 and cfg.rope_theta == 1000000
    assert cfg.attention_bias is False and cfg.tie_word_embeddings is True
    assert (cfg.bos_token_id, cfg.eos_token_id) == (151643, 151645)


def _hf_tiny():
    tr = pytest.importorskip("transformers")
    cfg = tr.Qwen3Config(vocab_size=320, hidden_size=128, intermediate_size=192,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                         head_dim=32, rms_norm_eps=1e-6, rope_theta=1e6,
                         tie_word_embeddings=True, max_position_embeddings=256,
                         attention_bias=False)
    torch.manual_seed(0)
    m = tr.Qwen3ForCausalLM(cfg).float().eval()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.uniform_(0.5, 1.5)
            else:
                p.normal_(0, 0.05 if p.dim() == 2 and "embed" not in name else 1.0)
    return m


def _write_checkpoint(hf, path, dtype):
    """The published checkpoint naming: separate q/k/v and gate/up, plus the
    tied lm_head (which the loader skips)."""
    sd = {k: v.detach().to(dtype).contiguous() for k, v in hf.state_dict().items()}
    sd["lm_head.weight"] = sd["model.embed_tokens.weight"].clone()
    safetensors_torch.save_file(sd, str(path))
    return sd


def _product_like(hf, dtype):
    c = hf.config
    pkg = _pkg()
    cfg = pkg.Qwen3Config(hidden_size=c.hidden_size, num_attention_heads=c.num_attention_heads,
                          num_key_value_heads=c.num_key_value_heads, head_dim=c.head_dim,
                          intermediate_size=c.intermediate_size,
                          num_hidden_layers=c.num_hidden_layers, vocab_size=c.vocab_size,
                          max_position_embeddings=c.max_position_embeddings)
    m = pkg.Qwen3ForCausalLM(cfg).to(dtype)
    with torch.no_grad():
        for p in m.parameters():
            p.fill_(float("nan"))             # anything the loader misses shows up
    return m


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_load_weights_packs_like_the_checkpoint(tmp_path, dtype):
    hf = _hf_tiny()
    path = tmp_path / "model.safetensors"
    sd = _write_checkpoint(hf, path, dtype)
    model = _product_like(hf, dtype)
    _pkg().load_weights(model, str(path))
    for i in range(hf.config.num_hidden_layers):
        a, m = f"model.layers.{i}.self_attn.", f"model.layers.{i}.mlp."
        qkv = model.get_parameter(a + "qkv_proj.weight")
        q, k, v = sd[a + "q_proj.weight"], sd[a + "k_proj.weight"], sd[a + "v_proj.weight"]
        assert qkv.shape[0] == q.shape[0] + k.shape[0] + v.shape[0]
        assert torch.equal(qkv[:q.shape[0]], q)
        assert torch.equal(qkv[q.shape[0]:q.shape[0] + k.shape[0]], k)
        assert torch.equal(qkv[q.shape[0] + k.shape[0]:], v)
        gu = model.get_parameter(m + "gate_up_proj.weight")
        g, u = sd[m + "gate_proj.weight"], sd[m + "up_proj.weight"]
        assert torch.equal(gu[:g.shape[0]], g) and torch.equal(gu[g.shape[0]:], u)
    for name, p in model.named_parameters():
        assert not torch.isnan(p).any(), f"{name} not loaded"
    assert model.lm_head.weight is model.model.embed_tokens.weight


def test_loaded_model_matches_transformers(tmp_path):
    hf = _hf_tiny()
    path = tmp_path / "model.safetensors"
    _write_checkpoint(hf, path, torch.float32)
    model = _product_like(hf, torch.float32).eval()
    _pkg().load_weights(model, str(path))
    ids = torch.randint(0, hf.config.vocab_size, (2, 29), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = hf(ids).logits
        got = model(ids)
    assert ref.abs().max() > 1.0
    torch.testing.assert_close(got, ref, atol=2e-4, rtol=2e-4)
