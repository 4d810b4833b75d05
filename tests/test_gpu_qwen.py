"""Qwen3 drop-in (qwen_routed_attention.py:94-325) on the GPU.

* RoPE with every step in the activation dtype is bit-identical to transformers'
  ``apply_rotary_pos_emb`` (computed on the CPU).
* The reference's wrapper self-test (test_qwen30b_routed.py:146-215): with everything kept local
  (``keep_last`` covering the sequence, no routed middle) ``QwenRoutedAttention`` equals the stock
  ``Qwen3MoeAttention`` (SDPA, CPU), for one forward and for cache-shared blocked forwards, in
  the reference's tiny fp32 and realistic bf16 shapes, VRAM and RAM tiers.
* With routing active the wrapper equals the oracle fed the same projections and HF RoPE.
* A tiny Qwen3-MoE model after ``replace_qwen_attention_with_router`` streams through the HF
  decoder (DynamicCache, position_ids) and matches the stock model at full coverage.
"""
import copy
import types

import numpy as np
import pytest
import torch

import oracle

transformers = pytest.importorskip("transformers")
pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def hga():
    import hierarchicalglobalattention_amd as m
    m.lib()
    return m


def _rot_table(theta, S, Dh, dtype, pos0=0, B=1):
    half = Dh // 2
    inv = 1.0 / (theta ** (torch.arange(half, dtype=torch.float32) / half))
    t = torch.arange(pos0, pos0 + S, dtype=torch.float32)
    emb = torch.cat([torch.outer(t, inv)] * 2, dim=-1)
    return emb.cos().to(dtype).expand(B, S, Dh).contiguous(), emb.sin().to(dtype).expand(B, S, Dh).contiguous()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S", [77, 32768])   # 32768: q takes four heads per thread
def test_rope_steps_match_hf(hga, dtype, S):
    from transformers.models.qwen3_moe.modeling_qwen3_moe import apply_rotary_pos_emb
    from hierarchicalglobalattention_amd import ops
    print(f"[qwen] rope steps {dtype} S={S}", flush=True)
    g = torch.Generator().manual_seed(3)
    B, H, KVH, Dh = 2, 4, 2, 128
    q = torch.randn(B, S, H, Dh, generator=g).to(dtype).transpose(1, 2)     # strided view
    k = torch.randn(B, KVH, S, Dh, generator=g).to(dtype)
    c1, s1 = _rot_table(1e6, S, Dh, dtype, pos0=5)
    c2, s2 = _rot_table(1e6, S, Dh, dtype, pos0=4000)
    cos, sin = torch.cat([c1, c2]), torch.cat([s1, s2])                    # per-batch positions
    qr, kr = apply_rotary_pos_emb(q, k, cos, sin)
    cfg = ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=64,
                          group_size=16, topk_chunks=4, topk_groups=8, keep_first=1,
                          keep_last=1, cutoff_pair=0, dtype=dtype)
    gq = ops.rope(cfg, q.to(DEV), cos.to(DEV), sin.to(DEV), steps_in_dtype=True)
    gk = ops.rope(cfg, k.to(DEV), cos.to(DEV), sin.to(DEV), steps_in_dtype=True)
    assert torch.equal(gq.cpu(), qr) and torch.equal(gk.cpu(), kr)
    if dtype == torch.bfloat16:   # the one-rounding mode differs from HF on bf16
        assert not torch.equal(ops.rope(cfg, q.to(DEV), cos.to(DEV), sin.to(DEV)).cpu(), qr)


def _qwen_attn(realistic):
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (Qwen3MoeAttention,
                                                                  Qwen3MoeRotaryEmbedding)
    torch.manual_seed(0)
    if realistic:
        cfg = Qwen3MoeConfig(hidden_size=2048, num_attention_heads=32, num_key_value_heads=4,
                             head_dim=128, num_hidden_layers=1, num_experts=4,
                             num_experts_per_tok=2, rms_norm_eps=1e-6, rope_theta=10_000_000.0,
                             attention_bias=False, max_position_embeddings=262144)
        S, C, gs, dtype, tol = 200, 64, 16, torch.bfloat16, 0.05
    else:
        cfg = Qwen3MoeConfig(hidden_size=128, num_attention_heads=8, num_key_value_heads=2,
                             head_dim=16, num_hidden_layers=1, num_experts=4,
                             num_experts_per_tok=2, rms_norm_eps=1e-6, rope_theta=10000.0,
                             attention_bias=False, max_position_embeddings=4096)
        S, C, gs, dtype, tol = 20, 8, 4, torch.float32, 1e-3
    cfg._attn_implementation = "sdpa"
    attn = Qwen3MoeAttention(cfg, layer_idx=0).to(dtype=dtype).eval()
    rot = Qwen3MoeRotaryEmbedding(cfg)
    return cfg, attn, rot, S, C, gs, dtype, tol


@pytest.mark.parametrize("loc", ["vram", "ram", "fs"])
@pytest.mark.parametrize("realistic", [False, True], ids=["tiny-fp32", "realistic-bf16"])
@torch.no_grad()
def test_wrapper_equals_qwen_full_coverage(hga, realistic, loc):
    print(f"[qwen] wrapper vs Qwen3MoeAttention realistic={realistic} {loc}", flush=True)
    cfg, attn, rot, S, C, gs, dtype, tol = _qwen_attn(realistic)
    x = torch.randn(1, S, cfg.hidden_size, dtype=dtype)
    pos = torch.arange(S).unsqueeze(0)
    cos, sin = rot(x, pos)
    causal = torch.triu(torch.full((S, S), float("-inf"), dtype=dtype), diagonal=1).view(1, 1, S, S)
    ref, _ = attn(x, position_embeddings=(cos, sin), attention_mask=causal, past_key_values=None)
    ga = copy.deepcopy(attn).to(DEV)
    xg, cg, sg = x.to(DEV), cos.to(DEV), sin.to(DEV)
    kw = dict(keep_first=0, keep_last=9999, topk_chunks=0, chunk_size=C, group_size=gs,
              cache_location=loc)
    w = hga.QwenRoutedAttention(ga, cfg, **kw)
    out, aux = w(xg, position_embeddings=(cg, sg), attention_mask=None, position_ids=pos.to(DEV))
    assert aux is None
    w2 = hga.QwenRoutedAttention(ga, cfg, **kw)
    pkv = types.SimpleNamespace()
    outs = []
    for s in range(0, S, 16):
        e = min(s + 16, S)
        pids = torch.arange(s, e).unsqueeze(0).to(DEV)
        ob, _ = w2(xg[:, s:e], position_embeddings=(cg[:, s:e], sg[:, s:e]), attention_mask=None,
                   past_key_values=pkv, position_ids=pids)
        outs.append(ob)
    assert hasattr(pkv, "_kv_router")
    out_blk = torch.cat(outs, dim=1)
    err = (out.float().cpu() - ref.float()).abs().max().item()
    err_blk = (out_blk.float().cpu() - ref.float()).abs().max().item()
    print(f"  single {err:.3e}  blocked {err_blk:.3e}  (ref scale {ref.abs().max().item():.2f})")
    assert err < tol and err_blk < tol


@torch.no_grad()
def test_wrapper_routing_vs_oracle(hga):
    """Routing active (bf16, Dh 128): the wrapper's output equals o_proj of the oracle's
    prefill over the same projections, RoPE'd the HF way."""
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (Qwen3MoeAttention,
                                                                  Qwen3MoeRotaryEmbedding,
                                                                  apply_rotary_pos_emb)
    print("[qwen] wrapper routing vs oracle", flush=True)
    torch.manual_seed(1)
    cfg = Qwen3MoeConfig(hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                         head_dim=128, num_hidden_layers=1, num_experts=4, num_experts_per_tok=2,
                         rms_norm_eps=1e-6, rope_theta=1_000_000.0, attention_bias=False,
                         max_position_embeddings=8192)
    S, C, gs, kf, kl, tc, tg = 1000, 64, 16, 1, 2, 3, 6
    attn = Qwen3MoeAttention(cfg, layer_idx=0).to(DEV, torch.bfloat16).eval()
    rot = Qwen3MoeRotaryEmbedding(cfg).to(DEV)
    x = torch.randn(1, S, cfg.hidden_size, device=DEV, dtype=torch.bfloat16)
    pos = torch.arange(S, device=DEV).unsqueeze(0)
    cos, sin = rot(x, pos)
    w = hga.QwenRoutedAttention(attn, cfg, chunk_size=C, group_size=gs, keep_first=kf,
                                keep_last=kl, topk_chunks=tc, topk_groups=tg)
    out, _ = w(x, position_embeddings=(cos, sin), position_ids=pos)
    H, KVH, Dh = 8, 2, 128
    q = attn.q_norm(attn.q_proj(x).view(1, S, H, Dh)).transpose(1, 2).cpu()
    k_raw = attn.k_norm(attn.k_proj(x).view(1, S, KVH, Dh)).transpose(1, 2).cpu()
    v = attn.v_proj(x).view(1, S, KVH, Dh).transpose(1, 2).cpu()
    qr, kr = apply_rotary_pos_emb(q, k_raw, cos.cpu(), sin.cpu())
    f = lambda t: t.float().contiguous().numpy()
    o_heads, r, _, _ = oracle.prefill(f(qr), f(kr), f(k_raw), f(v), f(cos[0].cpu()),
                                      f(sin[0].cpu()), C=C, gs=gs, keep_first=kf, keep_last=kl,
                                      topk_chunks=tc, topk_groups=tg, theta=1e6,
                                      dt=oracle.DT_BF16)
    assert (r["n_open"] > 0).any()
    oh = torch.from_numpy(o_heads).to(DEV, torch.bfloat16)
    ref = attn.o_proj(oh.transpose(1, 2).reshape(1, S, H * Dh))
    err = (out.float() - ref.float()).abs()
    print(f"  max {err.max().item():.3e} mean {err.mean().item():.3e}")
    assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3


@torch.no_grad()
def test_model_surgery_streams_through_decoder(hga):
    """Tiny Qwen3-MoE, attention replaced in every layer; blocked cached forward through the HF
    decoder (DynamicCache + position_ids, test_qwen30b_routed.py:331-351) equals the stock model
    at full coverage; restore gives the stock logits back."""
    from transformers import DynamicCache, Qwen3MoeConfig, Qwen3MoeForCausalLM
    print("[qwen] model surgery", flush=True)
    torch.manual_seed(0)
    cfg = Qwen3MoeConfig(vocab_size=128, hidden_size=128, intermediate_size=128,
                         moe_intermediate_size=64, num_hidden_layers=2, num_attention_heads=8,
                         num_key_value_heads=2, head_dim=16, num_experts=4, num_experts_per_tok=2,
                         rms_norm_eps=1e-6, rope_theta=10000.0, attention_bias=False,
                         max_position_embeddings=1024)
    cfg._attn_implementation = "sdpa"
    model = Qwen3MoeForCausalLM(cfg).eval()
    S = 40
    ids = torch.randint(0, 128, (1, S))
    ref = model(input_ids=ids).logits
    model = model.to(DEV)
    n = hga.replace_qwen_attention_with_router(model, keep_first=0, keep_last=9999,
                                               topk_chunks=0, chunk_size=8, group_size=4)
    assert n == 2
    cache, outs = DynamicCache(), []
    for s in range(0, S, 12):
        e = min(s + 12, S)
        cp = torch.arange(s, e, device=DEV)
        outs.append(model(input_ids=ids[:, s:e].to(DEV), past_key_values=cache, cache_position=cp,
                          position_ids=cp.unsqueeze(0), use_cache=True).logits)
    got = torch.cat(outs, dim=1).cpu()
    err = (got - ref).abs().max().item()
    print(f"  routed-model logits max err {err:.3e}")
    assert err < 1e-3
    assert hga.restore_original_attention(model) == 2
    back = model(input_ids=ids.to(DEV)).logits.cpu()
    assert (back - ref).abs().max().item() < 1e-3
