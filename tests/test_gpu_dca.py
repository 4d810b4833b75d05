"""Dual Chunk Attention on the GPU (qwen_routed_attention.py:209-283).

* ``hga_attend_decode_dca`` against the oracle with routing active, per key regime (intra /
  successive / inter DCA chunk), for the VRAM record, the pinned host record read in place and
  the staged (gathered) record -- the staged result equals the in-place one bit for bit.
* The reference's DCA self-test (test_qwen30b_routed.py:249-310): ``QwenRoutedAttention`` with
  ``dca_chunk`` and everything kept local equals dense DCA (float64 on the CPU), for one forward
  and for cache-shared blocked forwards, tiny fp32 and a Qwen3-30B-shaped bf16 layer.
"""
import types

import numpy as np
import pytest
import torch

import oracle
from test_gpu_decode import ATTN_CASES, BF16_MAX, BF16_MEAN, F32_TOL, _cfg, _history, _ring, \
    _summaries
from test_oracle_dca import _dense_dca

pytestmark = pytest.mark.gpu
hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402

DEV = "cuda"


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: f"B{c[0]}n{c[10]}c{c[11]}L{c[12]}"
                         f"{'bf16' if c[13] is torch.bfloat16 else 'f32'}")
@pytest.mark.parametrize("tier", ["vram", "ram", "gather"])
def test_attend_decode_dca_vs_oracle(case, tier):
    B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, c0, L, dt = case
    print(f"[dca] attend {tier} {case}", flush=True)
    M = C // gs
    L_c = 2 * C
    gen = torch.Generator().manual_seed(n_closed * 5 + c0 + 1)
    start = n_closed * C + c0
    T = start + L
    k, v = _history(gen, B, KVH, T, Dh, dt)
    qs = [torch.randn(B, H, L, Dh, generator=gen) for _ in range(3)]     # fp32 versions
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt)
    if n_closed:
        ck, gk = _summaries(gen, B, KVH, n_closed, M, Dh, dt)
        r = ops.route_decode(cfg, qs[0].to(dt).to(DEV), ck.to(DEV), gk.to(DEV), n_closed)
        og, ot, Kg = r["open_grp"], r["open_thr"], r["Kg"]
    else:
        og = ot = torch.full((B, H, 1), -1, dtype=torch.int32, device=DEV)
        Kg = 0
    qd = [x.to(DEV) for x in qs]
    dca = dict(q_succ=qd[1], q_inter=qd[2], chunk=L_c, open_pos=None)
    if tier == "vram":
        kd, vd = k.to(DEV), v.to(DEV)
        out = ops.attend_decode(cfg, qd[0], n_closed, start, kd, vd, 0, kd, vd, kd, vd, False,
                                og, ot, Kg, dca=dca)
    else:
        R = kl + 1 + 2
        rk, rv = _ring(k, n_closed, C, kf, kl, R), _ring(v, n_closed, C, kf, kl, R)
        fk = k[:, :, :max(kf, 1) * C].contiguous()
        fv = v[:, :, :max(kf, 1) * C].contiguous()
        hk = torch.zeros(B, KVH, (n_closed + 1) * C, Dh, dtype=dt, pin_memory=True)
        hv = torch.zeros_like(hk).pin_memory()
        hk[:, :, :n_closed * C] = k[:, :, :n_closed * C]
        hv[:, :, :n_closed * C] = v[:, :, :n_closed * C]
        srcs = (rk.to(DEV), rv.to(DEV), R, fk.to(DEV), fv.to(DEV))
        out = ops.attend_decode(cfg, qd[0], n_closed, start, *srcs, hk, hv, True, og, ot, Kg,
                                dca=dca)
        if tier == "gather":
            sk, sv, sg = ops.gather_decode(cfg, n_closed, og, ot, Kg, hk, hv, True,
                                           ops.DecodeStaging(), H)
            out_g = ops.attend_decode(cfg, qd[0], n_closed, start, *srcs, sk, sv, False, sg, ot,
                                      Kg, dca=dict(dca, open_pos=og))
            torch.cuda.synchronize()
            assert torch.equal(out_g, out)
    torch.cuda.synchronize()
    assert out.dtype == dt
    ref = oracle.attend_decode_dca(*(x.numpy() for x in qs), k.float().numpy(),
                                   v.float().numpy(), C, gs, kf, kl, n_closed, start,
                                   og.cpu().numpy(), ot.cpu().numpy(), oracle.attn_scale(Dh),
                                   oracle.DT_BF16 if dt is torch.bfloat16 else oracle.DT_F32, L_c)
    d = np.abs(out.float().cpu().numpy() - ref)
    if dt is torch.bfloat16:
        assert d.max() <= BF16_MAX and d.mean() <= BF16_MEAN, (d.max(), d.mean())
    else:
        assert d.max() <= F32_TOL, d.max()


def test_dca_rejects_bad_chunk():
    B, H, KVH, Dh, C, gs = 1, 4, 2, 64, 32, 8
    cfg = _cfg(B, H, KVH, Dh, C, gs, 2, 4, 1, 1, torch.float32)
    q = torch.zeros(B, H, 1, Dh, device=DEV)
    kv = torch.zeros(B, KVH, C, Dh, device=DEV)
    e = torch.full((B, H, 1), -1, dtype=torch.int32, device=DEV)
    with pytest.raises(hga.HgaError, match="multiple"):
        ops.attend_decode(cfg, q, 0, 0, kv, kv, 0, kv, kv, kv, kv, False, e, e, 0,
                          dca=dict(q_succ=q, q_inter=q, chunk=48))


def _qwen(realistic):
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (Qwen3MoeAttention,
                                                                  Qwen3MoeRotaryEmbedding)
    torch.manual_seed(0)
    if realistic:
        cfg = Qwen3MoeConfig(hidden_size=2048, num_attention_heads=32, num_key_value_heads=4,
                             head_dim=128, num_hidden_layers=1, num_experts=4,
                             num_experts_per_tok=2, rms_norm_eps=1e-6, rope_theta=10_000_000.0,
                             attention_bias=False, max_position_embeddings=262144)
        shape = dict(S=200, C=64, gs=16, L_c=64, local=16, dtype=torch.bfloat16, tol=0.05)
    else:
        cfg = Qwen3MoeConfig(hidden_size=128, num_attention_heads=8, num_key_value_heads=2,
                             head_dim=16, num_hidden_layers=1, num_experts=4,
                             num_experts_per_tok=2, rms_norm_eps=1e-6, rope_theta=10000.0,
                             attention_bias=False, max_position_embeddings=4096)
        shape = dict(S=40, C=8, gs=4, L_c=16, local=4, dtype=torch.float32, tol=1e-4)
    cfg._attn_implementation = "eager"
    attn = Qwen3MoeAttention(cfg, layer_idx=0).to(DEV, shape["dtype"]).eval()
    return cfg, attn, Qwen3MoeRotaryEmbedding(cfg).to(DEV), shape


@pytest.mark.parametrize("loc", ["vram", "ram", "fs"])
@pytest.mark.parametrize("realistic", [False, True], ids=["tiny-fp32", "realistic-bf16"])
@torch.no_grad()
def test_wrapper_dca_equals_dense(realistic, loc):
    print(f"[dca] wrapper realistic={realistic} {loc}", flush=True)
    cfg, attn, rot, sh = _qwen(realistic)
    S, C, gs, L_c, local, dt = sh["S"], sh["C"], sh["gs"], sh["L_c"], sh["local"], sh["dtype"]
    H, KVH, Dh = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    x = torch.randn(1, S, cfg.hidden_size, device=DEV, dtype=dt)
    pos = torch.arange(S, device=DEV).unsqueeze(0)
    cos, sin = rot(x, pos)
    q = attn.q_norm(attn.q_proj(x).view(1, S, H, Dh)).transpose(1, 2)
    k_raw = attn.k_norm(attn.k_proj(x).view(1, S, KVH, Dh)).transpose(1, 2)
    v = attn.v_proj(x).view(1, S, KVH, Dh).transpose(1, 2)
    f = lambda t: t.double().cpu().numpy()
    theta = float(cfg.rope_parameters["rope_theta"])
    heads = _dense_dca(f(q), f(k_raw), f(v), theta, L_c, L_c + local, Dh ** -0.5)
    ref = attn.o_proj(torch.from_numpy(heads).to(DEV, dt).transpose(1, 2).reshape(1, S, H * Dh))
    kw = dict(keep_first=0, keep_last=9999, topk_chunks=0, chunk_size=C, group_size=gs,
              dca_chunk=L_c, dca_local=local, cache_location=loc)
    w = hga.QwenRoutedAttention(attn, cfg, **kw)
    out, _ = w(x, position_embeddings=(cos, sin), attention_mask=None, position_ids=pos)
    w2 = hga.QwenRoutedAttention(attn, cfg, **kw)
    pkv, outs = types.SimpleNamespace(), []
    for s in range(0, S, L_c):
        e = min(s + L_c, S)
        pids = torch.arange(s, e, device=DEV).unsqueeze(0)
        ob, _ = w2(x[:, s:e], position_embeddings=(cos[:, s:e], sin[:, s:e]), attention_mask=None,
                   past_key_values=pkv, position_ids=pids)
        outs.append(ob)
    out_blk = torch.cat(outs, dim=1)
    err = (out.float() - ref.float()).abs().max().item()
    err_blk = (out_blk.float() - ref.float()).abs().max().item()
    print(f"  single {err:.3e} blocked {err_blk:.3e}")
    assert err < sh["tol"] and err_blk < sh["tol"]
