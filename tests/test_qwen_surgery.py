"""Model surgery of the Qwen3 drop-in on a tiny random Qwen3-MoE (CPU, no kernel calls):
replace / restore / idempotence (qwen_routed_attention.py:331-399), shared weights, argument
checks and the no-fallback rule."""
import pytest
import torch

transformers = pytest.importorskip("transformers")

from hierarchicalglobalattention_amd.qwen_routed_attention import (  # noqa: E402
    QwenRoutedAttention, replace_qwen_attention_with_router, restore_original_attention)


def _tiny_model():
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM
    torch.manual_seed(0)
    cfg = Qwen3MoeConfig(vocab_size=96, hidden_size=64, intermediate_size=64,
                         moe_intermediate_size=32, num_hidden_layers=3, num_attention_heads=4,
                         num_key_value_heads=2, head_dim=16, num_experts=4,
                         num_experts_per_tok=2, rms_norm_eps=1e-6, rope_theta=10000.0,
                         attention_bias=False, max_position_embeddings=1024)
    return Qwen3MoeForCausalLM(cfg).eval()


def test_replace_restore_idempotent():
    model = _tiny_model()
    origs = [layer.self_attn for layer in model.model.layers]
    n_params = sum(p.numel() for p in model.parameters())
    assert replace_qwen_attention_with_router(model, chunk_size=8, group_size=4) == 3
    attns = [layer.self_attn for layer in model.model.layers]
    assert all(isinstance(a, QwenRoutedAttention) for a in attns)
    assert [a.orig for a in attns] == origs                 # original modules kept by reference
    assert [a.layer_idx for a in attns] == [0, 1, 2]
    assert sum(p.numel() for p in model.parameters()) == n_params   # no new parameters
    # idempotent: a second replacement unwraps first instead of nesting
    assert replace_qwen_attention_with_router(model, chunk_size=8, group_size=4,
                                              topk_chunks=2, topk_groups=4) == 3
    assert all(a.orig is o for a, o in zip((l.self_attn for l in model.model.layers), origs))
    assert model.model.layers[0].self_attn._cfg.topk_chunks == 2
    assert restore_original_attention(model) == 3
    assert [layer.self_attn for layer in model.model.layers] == origs
    assert restore_original_attention(model) == 0


def test_config_and_arguments():
    model = _tiny_model()
    a = QwenRoutedAttention(model.model.layers[1].self_attn, model.config, chunk_size=8,
                            group_size=4, keep_first=1, keep_last=3, topk_chunks=5,
                            topk_groups=12)
    c = a._cfg
    assert (c.nhead, c.kv_heads, c.head_dim, c.chunk_size, c.group_size) == (4, 2, 16, 8, 4)
    assert (c.topk_chunks, c.topk_groups, c.theta) == (5, 12, 10000.0)
    assert (a._policy.keep_first, a._policy.keep_last, a._policy.first_token_level) == (1, 3, True)
    with pytest.raises(ValueError):
        QwenRoutedAttention(model.model.layers[0].self_attn, model.config, chunk_size=8,
                            dca_chunk=12)
    d = QwenRoutedAttention(model.model.layers[0].self_attn, model.config, chunk_size=8,
                            dca_chunk=40)
    assert (d.dca_local, d.dca_ceil) == (8, 48)
    # any location other than "vram" / "fs" takes the RAM tier (qwen_routed_attention.py:286-315)
    t = QwenRoutedAttention(model.model.layers[0].self_attn, model.config, cache_location="tape")
    assert type(t._make_store(1, torch.float32, torch.device("cpu"))).__name__ == "RamKVCacheStore"
    f = QwenRoutedAttention(model.model.layers[0].self_attn, model.config, cache_location="fs",
                            ram_budget_gb=0.5, fs_cache_dir="/tmp")
    assert (f.cache_location, f.ram_budget_gb, f.fs_cache_dir) == ("fs", 0.5, "/tmp")


def test_cpu_forward_raises():
    """No CPU fallback: the drop-in refuses host tensors."""
    model = _tiny_model()
    replace_qwen_attention_with_router(model, chunk_size=8, group_size=4)
    ids = torch.randint(0, 96, (1, 12))
    with pytest.raises(RuntimeError, match="GPU"):
        model(input_ids=ids)

