"""GPU parity at the shapes of the benchmark configurations, through the C ABI.

* c3 (Qwen3-30B-A3B layer, 32K prefill): every query chunk's routing pool from 0 to 502 chunks,
  so every stage-1 selection width of the prefill router runs (rows of 1..32 candidates per lane
  of a 16-lane row group); query heads reduced to 4 (one KV head) so the C oracle finishes in
  seconds.  Lists compared bit for bit in the fused and split MFMA-certified kernels and the
  canonical scoring mode,
  with and without exact ties at the wide pools; attention within the bf16 bar on a few query
  chunks.
* c5 (batched decode, B64 x 64K, topk 32/128, needle chunks): one decode step for all 64
  sequences, every head's whole pool in one segment; lists bit for bit, attention within the
  bf16 bar for a few sequences.
* c2 (40M-class 8-layer stack, 8K prefill, h <- h + attn(h)): the inputs each layer hands its
  router are captured and fed to the oracle; summaries and lists bit for bit, attention within
  the bf16 bar.

Routing references: vectorized.py:304-396 (prefill), chunk_router.py:187-277 (decode)."""
import numpy as np
import pytest
import torch

import oracle
from helpers import make_inputs, rope_torch, rotary_table

pytestmark = pytest.mark.gpu

hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402

DEV = "cuda"
BF16_MAX, BF16_MEAN = 2e-2, 1e-2


def _pad(a, w):
    a = np.asarray(a)
    return np.concatenate([a, np.full(a.shape[:-1] + (w - a.shape[-1],), -1, np.int32)], -1)


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    w = max(a.shape[-1], b.shape[-1])
    np.testing.assert_array_equal(_pad(a, w), _pad(b, w))


def _stage1_width(P):
    """Candidates per lane of the prefill router's stage-1 row groups for a pool of P chunks
    (16 lanes per row, widths 1, 2, 4, 8, 12, ..., 32)."""
    for jj in (1, 2, 4, 8, 12, 16, 20, 24, 28, 32):
        if P <= 16 * jj:
            return jj
    raise ValueError(P)


# ----------------------------------------------------------------------------------------------
# c3: Qwen3-30B-A3B layer, 32K prefill, reduced heads
# ----------------------------------------------------------------------------------------------
C3 = dict(B=1, H=4, KVH=1, S=32768, Dh=128, C=64, gs=16, kf=2, kl=8, tc=16, tg=64, theta=1e6)


@pytest.fixture(scope="module")
def c3():
    c = C3
    print("[headline] c3 inputs", flush=True)
    q_raw, k_raw, v = make_inputs(21, c["B"], c["H"], c["KVH"], c["S"], c["Dh"],
                                  torch.bfloat16, qk_rmsnorm=True)
    cos, sin = rotary_table(c["S"], c["Dh"], c["theta"])
    q = rope_torch(q_raw.float(), cos, sin).to(torch.bfloat16)
    k_rope = rope_torch(k_raw.float(), cos, sin).to(torch.bfloat16)
    cb, sb = cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float()
    cfg = ops.make_config(batch=c["B"], heads=c["H"], kv_heads=c["KVH"], head_dim=c["Dh"],
                          chunk_size=c["C"], group_size=c["gs"], topk_chunks=c["tc"],
                          topk_groups=c["tg"], keep_first=c["kf"], keep_last=c["kl"],
                          cutoff_pair=ops.mixed_cutoff_pair(c["theta"], c["C"], c["Dh"]),
                          dtype=torch.bfloat16)
    ck, gk = ops.summarize(cfg, k_raw.to(DEV), k_rope.to(DEV), cb.to(DEV), sb.to(DEV))
    f = lambda t: t.float().numpy()
    cut = oracle.cutoff_pair(c["theta"], c["C"], c["Dh"])
    o_ck, o_gk = oracle.summarize(f(k_raw), f(k_rope), cb.numpy(), sb.numpy(), c["C"], c["gs"],
                                  cut, oracle.group_scale(c["gs"]), oracle.DT_BF16)
    return dict(cfg=cfg, q=q, k_rope=k_rope, v=v, ck=ck, gk=gk, o_ck=o_ck, o_gk=o_gk)


def _route_c3(d, ck, gk, o_ck, o_gk):
    c = C3
    q = d["q"].to(DEV)
    stats = torch.zeros(4, dtype=torch.int32, device=DEV)
    r = ops.route_prefill(d["cfg"], q, ck, gk, stats=stats)
    rc = ops.route_prefill(d["cfg"], q, ck, gk, canonical=True)
    rs = ops.route_prefill(d["cfg"], q, ck, gk, split=True)
    torch.cuda.synchronize()
    o_r = oracle.route_prefill_heads(d["q"].float().numpy(), o_ck, o_gk, c["S"], c["C"], c["gs"],
                                     c["kf"], c["kl"], c["tc"], c["tg"],
                                     oracle.attn_scale(c["Dh"]))
    for rr in (r, rc, rs):      # fused, canonical, split
        _same(rr["sel_chunk"].cpu().numpy(), o_r["sel_chunk"])
        _same(rr["sel_thr"].cpu().numpy(), o_r["sel_thr"])
        _same(rr["open_grp"].cpu().numpy(), o_r["open_grp"])
        _same(rr["open_thr"].cpu().numpy(), o_r["open_thr"])
        np.testing.assert_array_equal(rr["n_sel"].cpu().numpy(), o_r["n_sel"])
        np.testing.assert_array_equal(rr["n_open"].cpu().numpy(), o_r["n_open"])
    return r, o_r, stats.cpu().tolist()


def test_c3_routing_every_pool_width(c3):
    """All 512 query chunks of the 32K block: pools of 0..502 chunks, so the stage-1 row groups
    run at every width; summaries and lists identical to the oracle's."""
    c = C3
    np.testing.assert_array_equal(c3["ck"].float().cpu().numpy(), c3["o_ck"])
    np.testing.assert_array_equal(c3["gk"].float().cpu().numpy(), c3["o_gk"])
    N = c["S"] // c["C"]
    pools = [max(0, oracle.windows(n, c["kf"], c["kl"])[1] - oracle.windows(n, c["kf"], c["kl"])[0])
             for n in range(N)]
    widths = sorted({_stage1_width(P) for P in pools if P > 0})
    print("[headline] c3 pool widths", min(pools), max(pools), "stage-1 lane widths", widths,
          flush=True)
    assert widths == [1, 2, 4, 8, 12, 16, 20, 24, 28, 32]
    _, o_r, stats = _route_c3(c3, c3["ck"], c3["gk"], c3["o_ck"], c3["o_gk"])
    print("[headline] c3 re-ranked rows / pools (stage 1, 2):", stats, flush=True)
    assert (o_r["n_sel"][..., 26:] == c["tc"]).all()   # pools of 16+ chunks from chunk 26 on


def test_c3_routing_ties_at_wide_pools(c3):
    """Exact score ties in pools of 130-502 chunks: a large-norm chunk summary copied into 35
    chunks past 150 (many rows rank the copies in their top 16, and no threshold separates 17..32
    keys, so those rows take the full-row search and the canonical re-rank over up to 8
    candidates per lane) and one group of every chunk copied into another (stage-2 ties)."""
    c = C3
    ck, gk = c3["ck"].clone(), c3["gk"].clone()
    ck[:, :, 2] *= 3
    for n in range(150, 500, 10):
        ck[:, :, n] = ck[:, :, 2]
    gk[:, :, :, 3] = gk[:, :, :, 1]
    f = lambda t: t.float().cpu().numpy()
    r, o_r, stats = _route_c3(c3, ck, gk, f(ck), f(gk))
    print("[headline] c3 ties: re-ranked rows / pools (stage 1, 2):", stats, flush=True)
    sel = o_r["sel_chunk"]
    assert np.isin(sel[:, :, 160:], np.arange(150, 500, 10)).any()
    assert stats[0] > 0 and stats[1] > 0


def test_c3_attention_on_sample_chunks(c3):
    """The 32K block's attention on query chunks at both ends and across the stage-1 width
    steps, against the oracle over the same lists (within the bf16 bar)."""
    c = C3
    q = c3["q"].to(DEV)
    kr, v = c3["k_rope"].to(DEV), c3["v"].to(DEV)
    r = ops.route_prefill(c3["cfg"], q, c3["ck"], c3["gk"])
    out = ops.attend_prefill(c3["cfg"], q, kr, v, r["open_grp"], r["open_thr"], r["Kg"])
    torch.cuda.synchronize()
    og, ot = r["open_grp"].cpu().numpy(), r["open_thr"].cpu().numpy()
    chunks = [0, 10, 137, 138, 300, 511]
    f = lambda t: t.float().numpy()
    o_out = oracle.attend_prefill(f(c3["q"]), f(c3["k_rope"]), f(c3["v"]), c["C"], c["gs"],
                                  c["kf"], c["kl"], og, ot, oracle.attn_scale(c["Dh"]),
                                  oracle.DT_BF16, chunks=chunks)
    rows = np.concatenate([np.arange(n * c["C"], (n + 1) * c["C"]) for n in chunks])
    err = np.abs(out.float().cpu().numpy()[:, :, rows] - o_out[:, :, rows])
    print("[headline] c3 attention max/mean abs err:", err.max(), err.mean(), flush=True)
    assert err.max() <= BF16_MAX and err.mean() <= BF16_MEAN


# ----------------------------------------------------------------------------------------------
# c5: batched decode B64 x 64K, topk 32 / 128, needle chunks in KV heads 0-1
# ----------------------------------------------------------------------------------------------
def test_c5_batched_decode_step():
    from hierarchicalglobalattention_amd.router import (ChunkPlacementPolicy, ChunkRouter,
                                                        RouterConfig, VramKVCacheStore,
                                                        rotary_for_positions)
    B, H, KVH, Dh, C, gs, kf, kl, tc, tg, theta = 64, 32, 4, 128, 64, 16, 2, 8, 32, 128, 1e6
    ctx = 65536
    T = ctx + 1
    print("[headline] c5 inputs", flush=True)
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(5)
    rms = lambda x: x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    k_raw = rms(torch.randn(B, KVH, T, Dh, device=dev, generator=g)).to(torch.bfloat16)
    gc = torch.Generator().manual_seed(6)
    needles = {}
    for b in range(B):
        for kvh in range(2):
            ids = torch.randperm(ctx // C, generator=gc)[:4].tolist()
            needles[(b, kvh)] = ids
            for n in ids:
                k_raw[b, kvh, n * C:(n + 1) * C] *= 8
    v = torch.randn(B, KVH, T, Dh, device=dev, generator=g).to(torch.bfloat16)
    q_raw = rms(torch.randn(B, H, 1, Dh, device=dev, generator=g)).to(torch.bfloat16)
    rcfg = RouterConfig(nhead=H, kv_heads=KVH, head_dim=Dh, chunk_size=C, group_size=gs,
                        topk_chunks=tc, topk_groups=tg, theta=theta)
    pol = ChunkPlacementPolicy(keep_first=kf, keep_last=kl, first_token_level=True)
    store = VramKVCacheStore(compute_device=dev, policy=pol, kv_heads=KVH, head_dim=Dh,
                             chunk_size=C, groups_per_chunk=C // gs, batch_size=B,
                             dtype=torch.bfloat16, initial_capacity=ctx // C + 2)
    router = ChunkRouter(rcfg, store)
    hc = router.hcfg(B, torch.bfloat16)
    cos, sin = rotary_for_positions(theta, Dh, 0, T, dev)
    k_rope = ops.rope(hc, k_raw, cos, sin)
    q = ops.rope(hc, q_raw, cos[ctx:], sin[ctx:])
    router.seed_store_from_block(0, k_rope[:, :, :ctx], k_raw[:, :, :ctx], v[:, :, :ctx])
    n_closed = ctx // C
    # one segment per head: the whole 1014-chunk pool is scored by one workgroup
    nb = ops.route_decode_workspace(hc, 1, n_closed)
    Kc, Kg = ops.decode_widths(hc, n_closed)
    assert (Kc, Kg) == (tc, tg)
    assert nb == B * H * Kc * 8, nb
    print("[headline] c5 decode step", flush=True)
    routed = router.decode_block(0, q, k_rope[:, :, ctx:], k_raw[:, :, ctx:], v[:, :, ctx:], ctx)
    out = routed.attend(q)
    torch.cuda.synchronize()
    st = store.layer(0)
    ck = st.chunk_k[:, :, :n_closed].float().cpu().numpy()
    gk = st.group_k[:, :, :n_closed].float().cpu().numpy()
    o = oracle.route_decode(q.float().cpu().numpy(), ck, gk, n_closed, kf, kl, tc, tg,
                            oracle.attn_scale(Dh))
    r = routed.routing
    for key in ("mid", "mid_thr", "open_grp", "open_thr"):
        _same(r[key].cpu().numpy(), o[key])
    np.testing.assert_array_equal(r["n_mid"].cpu().numpy(), o["n_mid"])
    # the needles win in KV heads 0-1: a query head there selects at least one needle chunk
    mid = o["mid"]
    hit = [any(c in needles[(b, h // (H // KVH))] for c in mid[b, h])
           for b in range(B) for h in range(H // 2)]
    print("[headline] c5 heads selecting a needle chunk:", sum(hit), "of", len(hit), flush=True)
    assert sum(hit) > len(hit) // 2
    og, ot = r["open_grp"].cpu().numpy(), r["open_thr"].cpu().numpy()
    for b in (0, 37, 63):
        kh = k_rope[b:b + 1].float().cpu().numpy()
        vh = v[b:b + 1].float().cpu().numpy()
        ref = oracle.attend_decode(q[b:b + 1].float().cpu().numpy(), kh, vh, C, gs, kf, kl,
                                   n_closed, ctx, og[b:b + 1], ot[b:b + 1],
                                   oracle.attn_scale(Dh), oracle.DT_BF16)
        d = np.abs(out[b:b + 1].float().cpu().numpy() - ref)
        print(f"[headline] c5 b{b} attention max/mean abs err:", d.max(), d.mean(), flush=True)
        assert d.max() <= BF16_MAX and d.mean() <= BF16_MEAN


# ----------------------------------------------------------------------------------------------
# c2: the 40M-class 8-layer stack, 8K prefill, layer by layer
# ----------------------------------------------------------------------------------------------
def test_c2_stack_layer_by_layer(monkeypatch):
    from hierarchicalglobalattention_amd import router as hrouter
    C, gs, kf, kl, tc, tg, theta, Dh = 64, 16, 2, 8, 16, 64, 1e4, 64
    S = 8192
    torch.manual_seed(0)
    layers = []
    for i in range(8):
        m = hga.HierarchicalGlobalAttentionRouted(d_model=512, nhead=8, kv_heads=2,
                                                  chunk_size=C, group_size=gs, topk_chunks=tc,
                                                  topk_groups=tg, keep_first=kf, keep_last=kl,
                                                  theta=theta, layer_idx=i)
        for prm in m.parameters():
            torch.nn.init.normal_(prm, std=0.02)
        layers.append(m.to(DEV, torch.bfloat16).eval())
    x = torch.randn(1, S, 512, device=DEV, dtype=torch.bfloat16)
    cap = {}
    real_sum, real_route, real_att = ops.summarize, ops.route_prefill, ops.attend_prefill

    def spy_sum(cfg, k_raw, k_rope, cos, sin, **kw):
        res = real_sum(cfg, k_raw, k_rope, cos, sin, **kw)
        cap["sum"] = [t.float().cpu().numpy() for t in (k_raw, k_rope, cos, sin)] + \
            [res[0].float().cpu().numpy(), res[1].float().cpu().numpy()]
        return res

    def spy_route(cfg, q, ck, gk, *a, **kw):
        res = real_route(cfg, q, ck, gk, *a, **kw)
        cap["q"] = q.float().cpu().numpy()
        cap["route"] = {k: v.cpu().numpy() for k, v in res.items() if torch.is_tensor(v)}
        return res

    def spy_att(cfg, q, k, v, og, ot, Kg, *a, **kw):
        res = real_att(cfg, q, k, v, og, ot, Kg, *a, **kw)
        cap["v"] = v.float().cpu().numpy()
        cap["out"] = res.float().cpu().numpy()
        return res

    monkeypatch.setattr(hrouter.ops, "summarize", spy_sum)
    monkeypatch.setattr(hrouter.ops, "route_prefill", spy_route)
    monkeypatch.setattr(hrouter.ops, "attend_prefill", spy_att)
    cut = oracle.cutoff_pair(theta, C, Dh)
    scale = oracle.attn_scale(Dh)
    chunks = [0, 1, 9, 10, 11, 64, 100, 127]
    rows = np.concatenate([np.arange(n * C, (n + 1) * C) for n in chunks])
    with torch.no_grad():
        for i, m in enumerate(layers):
            cap.clear()
            a, _ = m(hidden_states=x)
            x = x + a
            torch.cuda.synchronize()
            k_raw, k_rope, cos, sin, g_ck, g_gk = cap["sum"]
            o_ck, o_gk = oracle.summarize(k_raw, k_rope, cos, sin, C, gs, cut,
                                          oracle.group_scale(gs), oracle.DT_BF16)
            np.testing.assert_array_equal(g_ck, o_ck)
            np.testing.assert_array_equal(g_gk, o_gk)
            o_r = oracle.route_prefill_heads(cap["q"], o_ck, o_gk, S, C, gs, kf, kl, tc, tg,
                                             scale)
            for key in ("sel_chunk", "sel_thr", "open_grp", "open_thr"):
                _same(cap["route"][key], o_r[key])
            o_out = oracle.attend_prefill(cap["q"], k_rope, cap["v"], C, gs, kf, kl,
                                          o_r["open_grp"], o_r["open_thr"], scale,
                                          oracle.DT_BF16, chunks=chunks)
            err = np.abs(cap["out"][:, :, rows] - o_out[:, :, rows])
            print(f"[headline] c2 layer {i}: q std {cap['q'].std():.3g}, attention max/mean "
                  f"abs err {err.max():.3g} / {err.mean():.3g}", flush=True)
            assert err.max() <= BF16_MAX and err.mean() <= BF16_MEAN
