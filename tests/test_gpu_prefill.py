"""GPU parity of the prefill path through the C ABI: RoPE and summaries bit-exact against the
oracle, routing sets identical to the oracle (and to the reference's own fixtures for fp32),
attention within 1e-4 (fp32) / 2e-2 max, 1e-2 mean (bf16)."""
import numpy as np
import pytest
import torch

import oracle
from helpers import (dtype_table, load_case, make_inputs, oracle_prefill_case,
                     prefill_case_inputs, rope_torch, rotary_table)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hga():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import hierarchicalglobalattention_amd as h
    h.lib()
    return h


def _cfg(ops, *, B, H, KVH, Dh, C, gs, kf, kl, tc, tg, theta, dtype):
    return ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                           group_size=gs, topk_chunks=tc, topk_groups=tg, keep_first=kf,
                           keep_last=kl, cutoff_pair=ops.mixed_cutoff_pair(theta, C, Dh),
                           dtype=dtype)


def _cmp_sets(r, ref_id, ref_thr, key_id, key_thr):
    a_id = r[key_id].cpu().numpy()
    a_thr = r[key_thr].cpu().numpy()
    w = max(a_id.shape[-1], ref_id.shape[-1])
    pad = lambda x: np.concatenate([x, np.full(x.shape[:-1] + (w - x.shape[-1],), -1, np.int32)], -1)
    np.testing.assert_array_equal(pad(a_id), pad(np.asarray(ref_id)))
    np.testing.assert_array_equal(pad(a_thr), pad(np.asarray(ref_thr)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
# one head per thread; four heads per thread (taken once the grid has >= 2048 workgroups)
@pytest.mark.parametrize("B,X,S,Dh", [(2, 3, 77, 64), (1, 8, 32768, 128)])
def test_rope_bit_exact(hga, dtype, B, X, S, Dh):
    from hierarchicalglobalattention_amd import ops
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, S, X, Dh, generator=g).to(dtype).transpose(1, 2)   # strided view
    cos, sin = rotary_table(S, Dh, 1e4)
    ref = rope_torch(x.float(), cos, sin).to(dtype)
    cfg = _cfg(ops, B=B, H=X, KVH=X, Dh=Dh, C=8, gs=4, kf=0, kl=0, tc=0, tg=0, theta=1e4,
               dtype=dtype)
    out = ops.rope(cfg, x.cuda(), cos.cuda(), sin.cuda())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,KVH,S,Dh", [(2, 6, 3, 77, 64), (1, 32, 4, 32768, 128)])
@pytest.mark.parametrize("steps", [False, True])
def test_rope_qk_matches_two_ropes(hga, dtype, B, H, KVH, S, Dh, steps):
    """q and k in one launch (q's grid first, k's after) equal two separate rope calls bit for
    bit, and the fp32-rotation variant equals torch's."""
    from hierarchicalglobalattention_amd import ops
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, S, H, Dh, generator=g).to(dtype).transpose(1, 2).cuda()   # strided
    k = torch.randn(B, KVH, S, Dh, generator=g).to(dtype).cuda()
    cos, sin = rotary_table(S, Dh, 1e6)
    cfg = _cfg(ops, B=B, H=H, KVH=KVH, Dh=Dh, C=8, gs=4, kf=0, kl=0, tc=0, tg=0, theta=1e6,
               dtype=dtype)
    cos, sin = cos.cuda(), sin.cuda()
    qo, ko = ops.rope_qk(cfg, q, k, cos, sin, steps_in_dtype=steps)
    q1 = ops.rope(cfg, q, cos, sin, steps_in_dtype=steps)
    k1 = ops.rope(cfg, k, cos, sin, steps_in_dtype=steps)
    torch.cuda.synchronize()
    assert torch.equal(qo, q1) and torch.equal(ko, k1)
    if not steps:
        assert torch.equal(ko.cpu(), rope_torch(k.cpu().float(), cos.cpu(), sin.cpu()).to(dtype))


@pytest.mark.parametrize("name", ["c1_full", "c1_ragged", "forced_prev", "ref_shape", "wide_topk"])
def test_prefill_fp32_vs_reference(hga, name):
    from hierarchicalglobalattention_amd import ops
    meta, g = load_case(name)
    q, k_rope, k_raw, v, cos, sin = prefill_case_inputs(meta, g)
    dev = torch.device("cuda:0")
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    cfg = _cfg(ops, B=meta["B"], H=meta["H"], KVH=meta["KVH"], Dh=meta["Dh"], C=meta["C"],
               gs=meta["gs"], kf=meta["keep_first"], kl=meta["keep_last"],
               tc=meta["topk_chunks"], tg=meta["topk_groups"], theta=meta["theta"],
               dtype=torch.float32)
    ck, gk = ops.summarize(cfg, T(k_raw), T(k_rope), T(cos), T(sin))
    o_out, o_r, o_ck, o_gk = oracle_prefill_case(meta, g)
    np.testing.assert_array_equal(ck.cpu().numpy(), o_ck)
    np.testing.assert_array_equal(gk.cpu().numpy(), o_gk)
    r = ops.route_prefill(cfg, T(q), ck, gk)
    if meta["Kc"] > 0:
        _cmp_sets(r, g["sel_chunk"], g["sel_thr"], "sel_chunk", "sel_thr")
    if "open_grp" in g:
        _cmp_sets(r, g["open_grp"], g["open_thr"], "open_grp", "open_thr")
    out = ops.attend_prefill(cfg, T(q), T(k_rope), T(v), r["open_grp"], r["open_thr"], r["Kg"])
    o = out.cpu().numpy()
    st = meta["out_row_stride"]
    np.testing.assert_allclose(o[:, :, ::st], g["out"], atol=1e-4, rtol=0)
    np.testing.assert_allclose(o, o_out, atol=1e-4, rtol=0)


def _bf16_case(seed, B, H, KVH, S, Dh, C, gs, kf, kl, tc, tg, theta):
    q_raw, k_raw, v = make_inputs(seed, B, H, KVH, S, Dh, torch.bfloat16, qk_rmsnorm=True)
    cos, sin = rotary_table(S, Dh, theta)
    q = rope_torch(q_raw.float(), cos, sin).to(torch.bfloat16)
    k_rope = rope_torch(k_raw.float(), cos, sin).to(torch.bfloat16)
    return q, k_rope, k_raw, v, cos, sin


@pytest.mark.parametrize("shape", [
    dict(B=1, H=8, KVH=2, S=4096, Dh=128, C=64, gs=16, kf=2, kl=8, tc=16, tg=64, theta=1e6),
    dict(B=2, H=4, KVH=1, S=1500, Dh=64, C=64, gs=16, kf=1, kl=2, tc=4, tg=8, theta=1e4),
    dict(B=1, H=4, KVH=2, S=203, Dh=64, C=8, gs=4, kf=0, kl=0, tc=3, tg=6, theta=1e4),
    # shapes of the 16-key-block attention kernel: no windows, C=32, gs=32, one partial chunk
    dict(B=1, H=4, KVH=2, S=777, Dh=128, C=32, gs=16, kf=0, kl=0, tc=3, tg=5, theta=1e4),
    dict(B=2, H=4, KVH=2, S=640, Dh=64, C=64, gs=32, kf=1, kl=1, tc=2, tg=3, theta=1e4),
    dict(B=1, H=2, KVH=1, S=50, Dh=128, C=64, gs=16, kf=1, kl=1, tc=2, tg=4, theta=1e4),
])
def test_prefill_bf16_vs_oracle(hga, shape):
    from hierarchicalglobalattention_amd import ops
    q, k_rope, k_raw, v, cos, sin = _bf16_case(11, **shape)
    dev = torch.device("cuda:0")
    cfg = _cfg(ops, **{k: shape[k] for k in ("B", "H", "KVH", "Dh", "C", "gs", "kf", "kl",
                                             "tc", "tg", "theta")}, dtype=torch.bfloat16)
    cb, sb = cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float()
    ck, gk = ops.summarize(cfg, k_raw.to(dev), k_rope.to(dev), cb.to(dev), sb.to(dev))
    f = lambda t: t.float().numpy()
    cut = oracle.cutoff_pair(shape["theta"], shape["C"], shape["Dh"])
    o_ck, o_gk = oracle.summarize(f(k_raw), f(k_rope), cb.numpy(), sb.numpy(), shape["C"],
                                  shape["gs"], cut, oracle.group_scale(shape["gs"]),
                                  oracle.DT_BF16)
    np.testing.assert_array_equal(ck.float().cpu().numpy(), o_ck)
    np.testing.assert_array_equal(gk.float().cpu().numpy(), o_gk)
    stats = torch.zeros(4, dtype=torch.int32, device=dev)
    r = ops.route_prefill(cfg, q.to(dev), ck, gk, stats=stats)
    rc = ops.route_prefill(cfg, q.to(dev), ck, gk, canonical=True)
    rs = ops.route_prefill(cfg, q.to(dev), ck, gk, split=True)
    o_r = oracle.route_prefill(f(q), o_ck, o_gk, shape["S"], shape["C"], shape["gs"],
                               shape["kf"], shape["kl"], shape["tc"], shape["tg"],
                               oracle.attn_scale(shape["Dh"]))
    for rr in (r, rc, rs):      # fused (where eligible), canonical, split MFMA kernels
        _cmp_sets(rr, o_r["sel_chunk"], o_r["sel_thr"], "sel_chunk", "sel_thr")
        _cmp_sets(rr, o_r["open_grp"], o_r["open_thr"], "open_grp", "open_thr")
    print("ambiguous rows/pools:", stats.cpu().tolist())
    out = ops.attend_prefill(cfg, q.to(dev), k_rope.to(dev), v.to(dev), r["open_grp"],
                             r["open_thr"], r["Kg"])
    o_out = oracle.attend_prefill(f(q), f(k_rope), f(v), shape["C"], shape["gs"], shape["kf"],
                                  shape["kl"], o_r["open_grp"], o_r["open_thr"],
                                  oracle.attn_scale(shape["Dh"]), oracle.DT_BF16)
    err = np.abs(out.float().cpu().numpy() - o_out)
    print("bf16 attention max/mean abs err:", err.max(), err.mean())
    assert err.max() <= 2e-2 and err.mean() <= 1e-2


@pytest.mark.parametrize("Dh,gs", [(128, 16), (64, 16), (64, 4)])
def test_attend_prefill_routing_off(hga, Dh, gs):
    """Kg = 0 (1-element -1 lists): windows and the causal own chunk only."""
    from hierarchicalglobalattention_amd import ops
    B, H, KVH, S, C = 1, 4, 2, 1000, 64
    q, k_rope, k_raw, v, cos, sin = _bf16_case(3, B, H, KVH, S, Dh, C, gs, 1, 2, 0, 0, 1e4)
    dev = torch.device("cuda:0")
    cfg = _cfg(ops, B=B, H=H, KVH=KVH, Dh=Dh, C=C, gs=gs, kf=1, kl=2, tc=0, tg=0, theta=1e4,
               dtype=torch.bfloat16)
    N = (S + C - 1) // C
    e = torch.full((B, H, N, 1), -1, dtype=torch.int32)
    out = ops.attend_prefill(cfg, q.to(dev), k_rope.to(dev), v.to(dev), e.to(dev), e.to(dev), 0)
    f = lambda t: t.float().numpy()
    o_out = oracle.attend_prefill(f(q), f(k_rope), f(v), C, gs, 1, 2, e.numpy(), e.numpy(),
                                  oracle.attn_scale(Dh), oracle.DT_BF16)
    err = np.abs(out.float().cpu().numpy() - o_out)
    assert err.max() <= 2e-2 and err.mean() <= 1e-2, (err.max(), err.mean())


def test_route_exact_ties(hga):
    """Duplicated summaries give exactly tied scores; the lower chunk / group id must win in
    the MFMA path as in the canonical oracle."""
    from hierarchicalglobalattention_amd import ops
    B, H, KVH, S, Dh, C, gs = 1, 4, 2, 64 * 40, 128, 64, 16
    q, k_rope, k_raw, v, cos, sin = _bf16_case(5, B, H, KVH, S, Dh, C, gs, 1, 1, 4, 8, 1e6)
    dev = torch.device("cuda:0")
    cfg = _cfg(ops, B=B, H=H, KVH=KVH, Dh=Dh, C=C, gs=gs, kf=1, kl=1, tc=4, tg=8, theta=1e6,
               dtype=torch.bfloat16)
    cb, sb = cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float()
    ck, gk = ops.summarize(cfg, k_raw.to(dev), k_rope.to(dev), cb.to(dev), sb.to(dev))
    for c in range(3, 30, 2):          # chunks 3,5,..,29 copy chunk 2
        ck[:, :, c] = ck[:, :, 2]
        gk[:, :, c] = gk[:, :, 2]
    gk[:, :, :, 3] = gk[:, :, :, 1]    # group 3 of every chunk ties with group 1
    stats = torch.zeros(4, dtype=torch.int32, device=dev)
    r = ops.route_prefill(cfg, q.to(dev), ck, gk, stats=stats)
    stats_c = torch.zeros(4, dtype=torch.int32, device=dev)
    rc = ops.route_prefill(cfg, q.to(dev), ck, gk, canonical=True, stats=stats_c)
    rs = ops.route_prefill(cfg, q.to(dev), ck, gk, split=True)
    f = lambda t: t.float().cpu().numpy()
    o_r = oracle.route_prefill(f(q), f(ck), f(gk), S, C, gs, 1, 1, 4, 8, oracle.attn_scale(Dh))
    for rr in (r, rc, rs):               # fused MFMA-certified, canonical, split kernels
        _cmp_sets(rr, o_r["sel_chunk"], o_r["sel_thr"], "sel_chunk", "sel_thr")
        _cmp_sets(rr, o_r["open_grp"], o_r["open_thr"], "open_grp", "open_thr")
    print("ambiguous rows/pools:", stats.cpu().tolist(), "canonical:", stats_c.cpu().tolist())
    assert (o_r["sel_chunk"] == 2).sum() > 0
    assert stats[0].item() > 0           # the tie path really ran


def test_route_many_ties_full_search(hga):
    """41 copies of one chunk summary in pools of up to ~117 chunks with top-16: a row ranking
    the copied score among its top 16 has no threshold leaving 17..32 keys (the count jumps by
    41), so its row group takes the full-row search, and the boundary tie the canonical path;
    selections must still equal the oracle's."""
    from hierarchicalglobalattention_amd import ops
    B, H, KVH, S, Dh, C, gs = 1, 4, 2, 64 * 120, 128, 64, 16
    print("[prefill] many ties", flush=True)
    q, k_rope, k_raw, v, cos, sin = _bf16_case(9, B, H, KVH, S, Dh, C, gs, 1, 1, 16, 64, 1e6)
    dev = torch.device("cuda:0")
    cfg = _cfg(ops, B=B, H=H, KVH=KVH, Dh=Dh, C=C, gs=gs, kf=1, kl=1, tc=16, tg=64, theta=1e6,
               dtype=torch.bfloat16)
    cb, sb = cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float()
    ck, gk = ops.summarize(cfg, k_raw.to(dev), k_rope.to(dev), cb.to(dev), sb.to(dev))
    ck[:, :, 2] *= 3                   # large norm: the copies rank near the top of many rows
    for c in range(4, 84, 2):          # chunks 4, 6, .., 82 copy chunk 2
        ck[:, :, c] = ck[:, :, 2]
    stats = torch.zeros(4, dtype=torch.int32, device=dev)
    r = ops.route_prefill(cfg, q.to(dev), ck, gk, stats=stats)
    rc = ops.route_prefill(cfg, q.to(dev), ck, gk, canonical=True)
    rs = ops.route_prefill(cfg, q.to(dev), ck, gk, split=True)
    f = lambda t: t.float().cpu().numpy()
    o_r = oracle.route_prefill(f(q), f(ck), f(gk), S, C, gs, 1, 1, 16, 64, oracle.attn_scale(Dh))
    for rr in (r, rc, rs):
        _cmp_sets(rr, o_r["sel_chunk"], o_r["sel_thr"], "sel_chunk", "sel_thr")
        _cmp_sets(rr, o_r["open_grp"], o_r["open_thr"], "open_grp", "open_thr")
    print("ambiguous rows/pools:", stats.cpu().tolist())
    assert stats[0].item() > 0
