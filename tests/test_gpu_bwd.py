"""Backward of the routed prefill attention on the GPU (hga_attend_prefill_bwd) and training
through the drop-in module.

* ops level: dq, dk, dv against the oracle's exact gradient (itself pinned to torch float64
  autograd of the masked dense attention, test_oracle_bwd.py) on random routing lists: opened
  groups visible from a later row or never, ragged tails, GQA head sums, routing off -- with the
  rows' softmax statistics recomputed and taken from the forward (whose lse output is checked
  against float64 log-sum-exp for each forward kernel).
  Tolerances: fp32 1e-4 and bf16 2e-2 max / 1e-2 mean abs error, relative to the gradient's
  largest magnitude when that exceeds 1.
* module level: HierarchicalGlobalAttentionRouted forward + backward (RoPE transpose, routed
  attention backward, projections) against a float64 torch model of the same layer, with windows
  that cover the whole block (routed attention = causal attention), and with routing active
  against the float64 model under the routing mask the oracle's router gives.
"""
import numpy as np
import pytest
import torch

import oracle
from test_oracle_bwd import random_lists

pytestmark = pytest.mark.gpu
hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402

DEV = "cuda"


def _cfg(B, H, KVH, Dh, C, gs, kf, kl, tg, dtype):
    return ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                           group_size=gs, topk_chunks=max(1, tg), topk_groups=tg, keep_first=kf,
                           keep_last=kl, cutoff_pair=ops.mixed_cutoff_pair(1e4, C, Dh), dtype=dtype)


def _check(a, ref, dt, what):
    a = a.float().cpu().numpy()
    scale = max(1.0, float(np.abs(ref).max()))
    d = np.abs(a - ref) / scale
    if dt is torch.bfloat16:
        assert d.max() <= 2e-2 and d.mean() <= 1e-2, (what, d.max(), d.mean())
    else:
        assert d.max() <= 1e-4, (what, d.max())


BWD_CASES = [
    # B, H, KVH, S, Dh, C, gs, kf, kl, dtype
    (1, 4, 2, 300, 64, 64, 16, 1, 1, torch.float32),
    (2, 4, 1, 83, 16, 8, 4, 1, 2, torch.float32),
    (1, 2, 2, 160, 32, 32, 8, 0, 0, torch.float32),
    (1, 8, 2, 1000, 128, 64, 16, 2, 3, torch.bfloat16),
    (1, 4, 2, 333, 64, 32, 8, 1, 1, torch.bfloat16),
    (1, 4, 4, 200, 128, 64, 16, 1, 1, torch.float32),
]


@pytest.mark.parametrize("case", BWD_CASES, ids=lambda c: f"S{c[3]}D{c[4]}C{c[5]}gs{c[6]}"
                         f"{'bf16' if c[9] is torch.bfloat16 else 'f32'}")
@pytest.mark.parametrize("Kg", [0, 6])
@pytest.mark.parametrize("keep_lse", [False, True], ids=["recompute", "fwd-lse"])
def test_attend_prefill_bwd_vs_oracle(case, Kg, keep_lse):
    B, H, KVH, S, Dh, C, gs, kf, kl, dt = case
    print(f"[bwd] ops {case} Kg={Kg} lse={keep_lse}", flush=True)
    rng = np.random.default_rng(S + Dh + Kg)
    bf = oracle.bf16_round if dt is torch.bfloat16 else (lambda x: x)
    q = bf(rng.standard_normal((B, H, S, Dh)).astype(np.float32))
    k = bf(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    v = bf(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    dout = bf(rng.standard_normal((B, H, S, Dh)).astype(np.float32))
    og, ot = random_lists(rng, B, H, S, C, gs, kf, kl, Kg)
    cfg = _cfg(B, H, KVH, Dh, C, gs, kf, kl, Kg, dt)
    N, _, Kgc = ops.prefill_widths(cfg, S)
    og, ot = og[..., :max(Kgc, 1)], ot[..., :max(Kgc, 1)]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dt)
    I = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    qd, kd, vd, gd = T(q), T(k), T(v), T(dout)
    lse = torch.empty(B, H, S, device=DEV) if keep_lse else None
    out = ops.attend_prefill(cfg, qd, kd, vd, I(og), I(ot), Kgc, lse=lse)
    dq, dk, dv = ops.attend_prefill_bwd(cfg, qd, kd, vd, out, gd, I(og), I(ot), Kgc, lse=lse)
    torch.cuda.synchronize()
    ro = oracle.attend_prefill(q, k, v, C, gs, kf, kl, og, ot, oracle.attn_scale(Dh),
                               oracle.DT_BF16 if dt is torch.bfloat16 else oracle.DT_F32)
    _check(out, ro, dt, "out")
    rq, rk, rv = oracle.attend_prefill_bwd(q, k, v, dout, C, gs, kf, kl, og, ot,
                                           oracle.attn_scale(Dh))
    for a, ref, what in ((dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
        assert a.dtype == dt and a.shape == ref.shape
        _check(a, ref, dt, what)


@pytest.mark.parametrize("shape", [
    dict(S=300, Dh=128, C=64, gs=16, dt=torch.bfloat16),   # pipelined GQA MFMA kernel (v3)
    dict(S=150, Dh=64, C=32, gs=8, dt=torch.bfloat16),     # LDS-tiled MFMA kernel
    dict(S=83, Dh=16, C=8, gs=4, dt=torch.float32),        # VALU kernel
], ids=["v3", "lds", "valu"])
def test_forward_lse_is_logsumexp(shape):
    """The forward's lse output = log2 of the sum over the row's visible keys of
    2^(scale*log2(e)*q.k), float64 under the routing mask."""
    from test_oracle_bwd import routing_mask
    B, H, KVH, kf, kl, Kg = 1, 4, 2, 1, 1, 5
    S, Dh, C, gs, dt = shape["S"], shape["Dh"], shape["C"], shape["gs"], shape["dt"]
    rng = np.random.default_rng(S)
    bf = oracle.bf16_round if dt is torch.bfloat16 else (lambda x: x)
    q = bf(rng.standard_normal((B, H, S, Dh)).astype(np.float32))
    k = bf(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    v = bf(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    og, ot = random_lists(rng, B, H, S, C, gs, kf, kl, Kg)
    cfg = _cfg(B, H, KVH, Dh, C, gs, kf, kl, Kg, dt)
    _, _, Kgc = ops.prefill_widths(cfg, S)
    og, ot = og[..., :max(Kgc, 1)], ot[..., :max(Kgc, 1)]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dt)
    I = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    lse = torch.full((B, H, S), float("nan"), device=DEV)
    ops.attend_prefill(cfg, T(q), T(k), T(v), I(og), I(ot), Kgc, lse=lse)
    mask = routing_mask(B, H, S, C, gs, kf, kl, og, ot)
    s = np.einsum("bhsd,bhtd->bhst", q.astype(np.float64),
                  np.repeat(k, H // KVH, axis=1).astype(np.float64)) * oracle.attn_scale(Dh)
    s = np.where(mask, s, -np.inf)
    mx = s.max(-1, keepdims=True)
    ref = (mx[..., 0] + np.log(np.exp(s - mx).sum(-1))) * np.log2(np.e)
    np.testing.assert_allclose(lse.cpu().numpy(), ref, atol=1e-3, rtol=1e-5)


def test_attend_prefill_bwd_unaligned_rows_take_valu_kernel():
    """bf16 head_dim 128 rows that are not 16-byte aligned take the VALU backward kernel; its
    gradients match the oracle like the MFMA kernel's."""
    B, H, KVH, S, Dh, C, gs, kf, kl, Kg, dt = 1, 4, 2, 200, 128, 64, 16, 1, 1, 6, torch.bfloat16
    rng = np.random.default_rng(7)
    q = oracle.bf16_round(rng.standard_normal((B, H, S, Dh)).astype(np.float32))
    k = oracle.bf16_round(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    v = oracle.bf16_round(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    dout = oracle.bf16_round(rng.standard_normal((B, H, S, Dh)).astype(np.float32))
    og, ot = random_lists(rng, B, H, S, C, gs, kf, kl, Kg)
    cfg = _cfg(B, H, KVH, Dh, C, gs, kf, kl, Kg, dt)
    _, _, Kgc = ops.prefill_widths(cfg, S)
    og, ot = og[..., :max(Kgc, 1)], ot[..., :max(Kgc, 1)]
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dt)
    I = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    qd, kd, vd = T(q), T(k), T(v)
    out = ops.attend_prefill(cfg, qd, kd, vd, I(og), I(ot), Kgc)
    # the same q values one element into a larger buffer: rows 2 bytes off 16-byte alignment
    buf = torch.empty(qd.numel() + 8, dtype=dt, device=DEV)
    qu = buf[1:1 + qd.numel()].view(B, H, S, Dh)
    qu.copy_(qd)
    assert qu.data_ptr() % 16 != 0
    dq, dk, dv = ops.attend_prefill_bwd(cfg, qu, kd, vd, out, T(dout), I(og), I(ot), Kgc)
    torch.cuda.synchronize()
    rq, rk, rv = oracle.attend_prefill_bwd(q, k, v, dout, C, gs, kf, kl, og, ot,
                                           oracle.attn_scale(Dh))
    for a, ref, what in ((dq, rq, "dq"), (dk, rk, "dk"), (dv, rv, "dv")):
        _check(a, ref, dt, what)


def test_attend_prefill_bwd_rejects_wide_chunks():
    cfg = _cfg(1, 2, 1, 64, 128, 16, 1, 1, 0, torch.float32)
    q = torch.zeros(1, 2, 256, 64, device=DEV)
    kv = torch.zeros(1, 1, 256, 64, device=DEV)
    e = torch.full((1, 2, 2, 1), -1, dtype=torch.int32, device=DEV)
    with pytest.raises(hga.HgaError, match="chunk_size"):
        ops.attend_prefill_bwd(cfg, q, kv, kv, q, q, e, e, 0)


# ----------------------------------------------------------------------------------------------
# training through the module
# ----------------------------------------------------------------------------------------------
def _ref_layer(m, x, mask_fn):
    """float64 torch model of HierarchicalGlobalAttentionRouted.forward with the layer's weights;
    mask_fn(S) -> [B|1, H|1, S, S] bool visibility."""
    B, S, _ = x.shape
    H, KVH, Dh = m.nhead, m.kv_heads, m.head_dim
    W = {n: p.detach().double().cpu().requires_grad_(True) for n, p in m.named_parameters()}
    xd = x.detach().double().cpu().requires_grad_(True)
    lin = lambda t, name: t @ W[name + ".weight"].t()
    q = lin(xd, "q_proj").view(B, S, H, Dh).transpose(1, 2)
    k = lin(xd, "k_proj").view(B, S, KVH, Dh).transpose(1, 2)
    v = lin(xd, "v_proj").view(B, S, KVH, Dh).transpose(1, 2)
    half = Dh // 2
    inv = 1.0 / (m.theta ** (torch.arange(half, dtype=torch.float64) / half))
    f = torch.arange(S, dtype=torch.float64)[:, None] * inv[None]
    cos, sin = torch.cat([f, f], -1).cos(), torch.cat([f, f], -1).sin()
    rot = lambda t: torch.cat([-t[..., half:], t[..., :half]], -1)
    q, k = q * cos + rot(q) * sin, k * cos + rot(k) * sin
    k, v = k.repeat_interleave(H // KVH, 1), v.repeat_interleave(H // KVH, 1)
    s = (q @ k.transpose(-1, -2)) * Dh ** -0.5
    s = s.masked_fill(~mask_fn(S), float("-inf"))
    o = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B, S, H * Dh)
    return o @ W["o_proj.weight"].t(), xd, W


@pytest.mark.parametrize("routed", [False, True], ids=["dense-windows", "routed"])
def test_module_backward_vs_float64(routed):
    torch.manual_seed(3)
    B, S, d_model, H, KVH, C, gs = 1, 200, 128, 4, 2, 16, 4
    kw = dict(keep_first=1, keep_last=2, topk_chunks=3, topk_groups=5) if routed else \
        dict(keep_first=0, keep_last=64, topk_chunks=0, topk_groups=0)
    m = hga.HierarchicalGlobalAttentionRouted(d_model=d_model, nhead=H, kv_heads=KVH,
                                              chunk_size=C, group_size=gs, theta=1e4,
                                              **kw).to(DEV)
    x = torch.randn(B, S, d_model, device=DEV, requires_grad=True)
    print(f"[bwd] module routed={routed}", flush=True)
    out, _ = m(hidden_states=x)
    g = torch.randn_like(out)
    out.backward(g)
    if routed:
        # the routing the module used: the oracle's router on the module's own fp32 q/k
        # (routing sets are bit-exact to the oracle's, test_gpu_prefill.py)
        Dh = d_model // H
        with torch.no_grad():
            qr = m.q_proj(x).view(B, S, H, Dh).transpose(1, 2)
            kr = m.k_proj(x).view(B, S, KVH, Dh).transpose(1, 2)
            cos, sin = m._get_rotary(S, x.device)
            hc = ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                                 group_size=gs, topk_chunks=3, topk_groups=5, keep_first=1,
                                 keep_last=2, cutoff_pair=ops.mixed_cutoff_pair(1e4, C, Dh),
                                 dtype=torch.float32)
            qrope, krope = ops.rope(hc, qr, cos, sin), ops.rope(hc, kr, cos, sin)
            f = lambda t: t.float().cpu().numpy()
            cut = oracle.cutoff_pair(1e4, C, Dh)
            ck, gk = oracle.summarize(f(kr), f(krope), f(cos), f(sin), C, gs, cut,
                                      oracle.group_scale(gs), oracle.DT_F32)
            r = oracle.route_prefill(f(qrope), ck, gk, S, C, gs, 1, 2, 3, 5,
                                     oracle.attn_scale(Dh))
        from test_oracle_bwd import routing_mask
        mk = torch.from_numpy(routing_mask(B, H, S, C, gs, 1, 2, r["open_grp"], r["open_thr"]))
        mask_fn = lambda S_: mk
    else:
        mask_fn = lambda S_: torch.ones(S_, S_, dtype=torch.bool).tril()
    ref, xd, W = _ref_layer(m, x, mask_fn)
    ref.backward(g.double().cpu())
    np.testing.assert_allclose(out.detach().cpu().numpy(), ref.detach().numpy(), atol=1e-4)
    tol = lambda t: 1e-4 * max(1.0, float(t.abs().max()))
    assert (x.grad.cpu().double() - xd.grad).abs().max() <= tol(xd.grad)
    for n, p in m.named_parameters():
        assert (p.grad.cpu().double() - W[n].grad).abs().max() <= tol(W[n].grad), n


def test_module_decode_block_backward_raises():
    """Blocks that are not a fresh multi-chunk block have no backward; the module refuses them
    before routing, so the router's store is left as it was (a 16-token block would otherwise
    fill and close chunk 0)."""
    m = hga.HierarchicalGlobalAttentionRouted(d_model=64, nhead=2, kv_heads=1, chunk_size=16,
                                              group_size=4).to(DEV)
    for S in (5, 16):
        x = torch.randn(1, S, 64, device=DEV, requires_grad=True)
        with pytest.raises(NotImplementedError):
            m(hidden_states=x)
        assert m._kv_router.store.num_closed_chunks(0) == 0
