"""The reference's inner seams on this build's stores and router, on the GPU, against the oracle.

* ``KVCacheStore`` (kv_cache_store.py:26-82): closed chunks handed to every tier through
  ``append_closed_chunk``; ``chunk_summaries``, ``gather_tokens``, ``gather_group_summaries``,
  ``hot_tokens``, ``hot_group_summaries`` and ``prefetch`` read them back (tokens and key
  summaries bit for bit, group V summaries to rounding), and a decode block routed over the
  store matches the oracle's routing and attention.
* ``ChunkRouter.prefill`` (chunk_router.py:410-440): a prefix streamed chunk by chunk, against
  the oracle's decode segments.
* The reference's dense-equivalence check (KvRouter/Tests/test_router.py:37-62): every chunk in
  the first window, no routing -> causal attention (fp32 here; the reference runs it in fp64).
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import OracleModule, rope_torch, rotary_table

pytestmark = pytest.mark.gpu

hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402
from hierarchicalglobalattention_amd.router import (ChunkPlacementPolicy, ChunkRouter,  # noqa: E402
                                                    FsKVCacheStore, RamKVCacheStore,
                                                    RouterConfig, VramKVCacheStore)

DEV = "cuda"
THETA = 1e6
F32_TOL, BF16_MAX, BF16_MEAN = 1e-4, 2e-2, 1e-2


def _same_lists(a, b):
    a, b = np.asarray(a), np.asarray(b)
    w = max(a.shape[-1], b.shape[-1])
    pad = lambda x: np.concatenate(
        [x, np.full(x.shape[:-1] + (w - x.shape[-1],), -1, np.int32)], -1)
    np.testing.assert_array_equal(pad(a), pad(b))


def _store(tier, B, KVH, Dh, C, M, kf, kl, dt, tmp_path, cap=8):
    kw = dict(compute_device=torch.device(DEV),
              policy=ChunkPlacementPolicy(keep_first=kf, keep_last=kl, first_token_level=True),
              kv_heads=KVH, head_dim=Dh, chunk_size=C, groups_per_chunk=M, batch_size=B,
              dtype=dt, initial_capacity=cap)
    if tier == "vram":
        return VramKVCacheStore(**kw)
    if tier == "ram":
        return RamKVCacheStore(**kw)
    return FsKVCacheStore(fs_cache_dir=str(tmp_path), ram_cache_chunks=16, **kw)


def _index_tokens(x, chunk_idx, group_idx, C, gs, rep):
    """x [B, KVH, T, Dh] -> [B, H, K, gs, Dh] rows of the groups (chunk_idx, group_idx)."""
    B, H, K = chunk_idx.shape
    tok = (chunk_idx * C + group_idx * gs)[..., None] + torch.arange(gs)
    b = torch.arange(B).view(B, 1, 1, 1)
    kv = (torch.arange(H) // rep).view(1, H, 1, 1)
    return x[b, kv, tok]


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("tier", ["vram", "ram", "fs"])
def test_store_seam_vs_oracle(tier, dt, tmp_path):
    B, H, KVH, Dh, C, gs, kf, kl, tc, tg, N, L = 2, 4, 2, 64, 16, 4, 1, 2, 3, 6, 12, 5
    M, rep = C // gs, H // KVH
    print(f"[seam] store {tier} {dt}", flush=True)
    g = torch.Generator().manual_seed(17)
    T = N * C + L
    k_raw = torch.randn(B, KVH, T, Dh, generator=g).to(dt)
    v = torch.randn(B, KVH, T, Dh, generator=g).to(dt)
    cos, sin = rotary_table(T, Dh, THETA)
    k_rope = rope_torch(k_raw.float(), cos, sin).to(dt)
    q = rope_torch(torch.randn(B, H, L, Dh, generator=g), cos[N * C:], sin[N * C:]).to(dt)
    e = N * C
    ck, gk = oracle.summarize(k_raw[:, :, :e].float().numpy(), k_rope[:, :, :e].float().numpy(),
                              cos.numpy(), sin.numpy(), C, gs, oracle.cutoff_pair(THETA, C, Dh),
                              oracle.group_scale(gs),
                              oracle.DT_BF16 if dt is torch.bfloat16 else oracle.DT_F32)
    ck_t, gk_t = torch.from_numpy(ck).to(dt), torch.from_numpy(gk).to(dt)
    gscale = 1.0 / (gs + gs ** 0.5)
    gv_t = (v[:, :, :e].reshape(B, KVH, N, M, gs, Dh).sum(4) * gscale).to(dt)

    store = _store(tier, B, KVH, Dh, C, M, kf, kl, dt, tmp_path)
    for n in range(N):
        store.append_closed_chunk(0, ck_t[:, :, n].to(DEV), gk_t[:, :, n].to(DEV),
                                  gv_t[:, :, n].to(DEV), k_rope[:, :, n * C:(n + 1) * C].to(DEV),
                                  v[:, :, n * C:(n + 1) * C].to(DEV))
    assert store.num_closed_chunks(0) == N
    assert torch.equal(store.chunk_summaries(0).cpu(), ck_t)

    ci = torch.randint(0, N, (B, H, 7), generator=g)
    gi = torch.randint(0, M, (B, H, 7), generator=g)
    store.prefetch(0, ci.to(DEV))
    kg, vg = store.gather_tokens(0, ci.to(DEV), gi.to(DEV))
    assert kg.shape == (B, H, 7, gs, Dh)
    assert torch.equal(kg.cpu(), _index_tokens(k_rope, ci, gi, C, gs, rep))
    assert torch.equal(vg.cpu(), _index_tokens(v, ci, gi, C, gs, rep))

    cj = torch.randint(0, N, (B, H, 3), generator=g)
    gkg, gvg = store.gather_group_summaries(0, cj.to(DEV))
    b = torch.arange(B).view(B, 1, 1)
    kvh = (torch.arange(H) // rep).view(1, H, 1)
    assert torch.equal(gkg.cpu(), gk_t[b, kvh, cj])
    gv_ref = v[:, :, :e].float().reshape(B, KVH, N, M, gs, Dh).sum(4).numpy() * gscale
    tol = 1e-5 if dt is torch.float32 else 3e-2
    np.testing.assert_allclose(gvg.float().cpu().numpy(), gv_ref[b.numpy(), kvh.numpy(), cj.numpy()], atol=tol,
                               rtol=tol)

    for lo, hi in ((0, kf), (N - kl, N)):
        kh, vh = store.hot_tokens(0, lo, hi)
        assert torch.equal(kh.cpu(), k_rope[:, :, lo * C:hi * C].reshape(B, KVH, hi - lo, C, Dh))
        assert torch.equal(vh.cpu(), v[:, :, lo * C:hi * C].reshape(B, KVH, hi - lo, C, Dh))
        gkh, gvh = store.hot_group_summaries(0, lo, hi)
        assert torch.equal(gkh.cpu(), gk_t[:, :, lo:hi])
        np.testing.assert_allclose(gvh.float().cpu().numpy(), gv_ref[:, :, lo:hi], atol=tol,
                                   rtol=tol)
    with pytest.raises(ValueError):
        store.hot_tokens(0, kf, kf + 1)          # a routed chunk, in no window

    # a decode block routed over the seam-fed store
    rcfg = RouterConfig(nhead=H, kv_heads=KVH, head_dim=Dh, chunk_size=C, group_size=gs,
                        topk_chunks=tc, topk_groups=tg, theta=THETA)
    router = ChunkRouter(rcfg, store)
    routed = router.decode_block(0, q.to(DEV), k_rope[:, :, e:].to(DEV), k_raw[:, :, e:].to(DEV),
                                 v[:, :, e:].to(DEV), e)
    out = routed.attend(q.to(DEV))
    torch.cuda.synchronize()
    scale = oracle.attn_scale(Dh)
    o = oracle.route_decode(q.float().numpy(), ck_t.float().numpy(), gk_t.float().numpy(), N,
                            kf, kl, tc, tg, scale)
    for key in ("mid", "mid_thr", "open_grp", "open_thr"):
        _same_lists(routed.routing[key].cpu().numpy(), o[key])
    ref = oracle.attend_decode(q.float().numpy(), k_rope.float().numpy(), v.float().numpy(), C,
                               gs, kf, kl, N, e, o["open_grp"], o["open_thr"], scale,
                               oracle.DT_BF16 if dt is torch.bfloat16 else oracle.DT_F32)
    d = np.abs(out.float().cpu().numpy() - ref)
    if dt is torch.bfloat16:
        assert d.max() <= BF16_MAX and d.mean() <= BF16_MEAN, (d.max(), d.mean())
    else:
        assert d.max() <= F32_TOL, d.max()


@pytest.mark.parametrize("tier", ["vram", "ram", "fs"])
def test_chunk_router_prefill_vs_oracle(tier, tmp_path):
    """ChunkRouter.prefill streams 9 chunks and a partial one through decode_block; outputs and
    routing decisions equal the oracle's decode segments."""
    B, H, KVH, Dh, C, gs, kf, kl, tc, tg = 2, 4, 2, 64, 16, 4, 1, 2, 2, 4
    S = 9 * C + 7
    print(f"[seam] prefill {tier}", flush=True)
    g = torch.Generator().manual_seed(23)
    k_raw = torch.randn(B, KVH, S, Dh, generator=g)
    v = torch.randn(B, KVH, S, Dh, generator=g)
    cos, sin = rotary_table(S, Dh, THETA)
    k_rope = rope_torch(k_raw, cos, sin)
    q = rope_torch(torch.randn(B, H, S, Dh, generator=g), cos, sin)
    store = _store(tier, B, KVH, Dh, C, C // gs, kf, kl, torch.float32, tmp_path)
    router = ChunkRouter(RouterConfig(nhead=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                                      group_size=gs, topk_chunks=tc, topk_groups=tg,
                                      theta=THETA), store)
    seen = []
    real = ops.route_decode

    def spy(cfg, qq, ck, gk, n_closed):
        r = real(cfg, qq, ck, gk, n_closed)
        seen.append((n_closed, r["mid"].cpu().numpy(), r["open_grp"].cpu().numpy()))
        return r

    import hierarchicalglobalattention_amd.router as hrouter
    hrouter.ops.route_decode = spy
    try:
        out = router.prefill(0, q.to(DEV), k_rope.to(DEV), k_raw.to(DEV), v.to(DEV))
    finally:
        hrouter.ops.route_decode = real
    torch.cuda.synchronize()
    om = OracleModule(dict(H=H, KVH=KVH, Dh=Dh, C=C, gs=gs, theta=THETA, keep_first=kf,
                           keep_last=kl, topk_chunks=tc, topk_groups=tg), {})
    ref, p = [], 0
    while p < S:
        take = min(C - p % C, S - p)
        sl = slice(p, p + take)
        ref.append(om._decode_segment(q[:, :, sl].numpy(), k_rope[:, :, sl].numpy(),
                                      k_raw[:, :, sl].numpy(), v[:, :, sl].numpy(), p, cos, sin))
        p += take
    ref = np.concatenate(ref, axis=2)
    assert out.shape == (B, H, S, Dh)
    np.testing.assert_allclose(out.cpu().numpy(), ref, atol=F32_TOL, rtol=0)
    assert store.num_closed_chunks(0) == S // C
    assert len(seen) == len(om.decisions)
    for (ncl, mid, og), (oncl, r) in zip(seen, om.decisions):
        assert ncl == oncl
        _same_lists(mid, r["mid"])
        _same_lists(og, r["open_grp"])


def test_dense_equivalence():
    """KvRouter/Tests/test_router.py:37-62: keep_first beyond every chunk, token level, no
    routing -> ChunkRouter.prefill equals causal attention with GQA expansion (B2, S28: three
    full chunks and a partial one)."""
    cfg = RouterConfig(nhead=8, kv_heads=4, head_dim=16, chunk_size=8, group_size=4,
                       topk_chunks=0, topk_groups=0, current_group_summaries=False,
                       theta=10000.0)
    B, S = 2, 28
    g = torch.Generator().manual_seed(0)
    cos, sin = rotary_table(S, cfg.head_dim, cfg.theta)
    q = rope_torch(torch.randn(B, cfg.nhead, S, cfg.head_dim, generator=g), cos, sin)
    k_raw = torch.randn(B, cfg.kv_heads, S, cfg.head_dim, generator=g)
    v = torch.randn(B, cfg.kv_heads, S, cfg.head_dim, generator=g)
    k_rope = rope_torch(k_raw, cos, sin)
    policy = ChunkPlacementPolicy(keep_last=0, keep_first=999, first_token_level=True)
    store = RamKVCacheStore(compute_device=torch.device(DEV), policy=policy,
                            kv_heads=cfg.kv_heads, head_dim=cfg.head_dim,
                            chunk_size=cfg.chunk_size, groups_per_chunk=cfg.groups_per_chunk,
                            batch_size=B, dtype=torch.float32, pin_memory=False)
    out = ChunkRouter(cfg, store).prefill(0, q.to(DEV), k_rope.to(DEV), k_raw.to(DEV),
                                          v.to(DEV), start_pos=0)
    torch.cuda.synchronize()
    rep = cfg.nhead // cfg.kv_heads
    qd, kd, vd = q.double(), k_rope.double().repeat_interleave(rep, 1), \
        v.double().repeat_interleave(rep, 1)
    s = (qd @ kd.transpose(-1, -2)) * cfg.head_dim ** -0.5
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    ref = torch.softmax(s, -1) @ vd
    err = (out.cpu().double() - ref).abs().max().item()
    print(f"[seam] dense equivalence max abs err {err:.3e}", flush=True)
    assert err < 1e-5, err
