"""GPU parity of the decode path: routing of blocks inside the active chunk, the decode attention
over [first window | last window | opened groups | active chunk], the VRAM and pinned-RAM
stores, and whole-module decode against the reference module's recorded outputs.

Routing indices are compared bit-exactly with the oracle (fp32 canonical scores, ties to the
lower id); attention outputs within 1e-4 (fp32) or 2e-2 max / 1e-2 mean abs (bf16)."""
import numpy as np
import pytest
import torch

import oracle
from helpers import OracleModule, load_case

pytestmark = pytest.mark.gpu

hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402
from hierarchicalglobalattention_amd import router as hrouter  # noqa: E402

DEV = "cuda"
BF16_MAX, BF16_MEAN, F32_TOL = 2e-2, 1e-2, 1e-4


def _pad(a, w):
    a = np.asarray(a)
    return np.concatenate([a, np.full(a.shape[:-1] + (w - a.shape[-1],), -1, np.int32)], -1)


def _same_lists(a, b):
    w = max(a.shape[-1], b.shape[-1])
    np.testing.assert_array_equal(_pad(a, w), _pad(b, w))


# ----------------------------------------------------------------------------------------------
# whole module against the reference module's recorded decode runs
# ----------------------------------------------------------------------------------------------
def _module(meta, g, cache_location=None):
    m = hga.HierarchicalGlobalAttentionRouted(
        d_model=meta["d_model"], nhead=meta["H"], kv_heads=meta["KVH"], head_dim=meta["Dh"],
        chunk_size=meta["C"], group_size=meta["gs"], topk_chunks=meta["topk_chunks"],
        topk_groups=meta["topk_groups"], keep_first=meta["keep_first"],
        keep_last=meta["keep_last"], theta=meta["theta"], qk_norm=meta.get("qk_norm", False),
        cache_location=cache_location or meta.get("cache_location", "vram"))
    sd = {k[2:]: torch.from_numpy(v) for k, v in g.items() if k.startswith("w_")}
    m.load_state_dict(sd, strict=True)
    return m.to(DEV).eval()


class _Cache:
    pass


def _run_module(m, x, S, gen, block=1):
    """Prefill S tokens, then feed the rest in blocks of `block` tokens."""
    cache = _Cache()
    outs = []
    with torch.no_grad():
        o, _ = m(hidden_states=x[:, :S], past_key_value=cache,
                 cache_position=torch.arange(S, device=DEV))
        outs.append(o)
        p = S
        while p < S + gen:
            e = min(S + gen, p + block)
            o, _ = m(hidden_states=x[:, p:e], past_key_value=cache,
                     cache_position=torch.arange(p, e, device=DEV))
            outs.append(o)
            p = e
    torch.cuda.synchronize()
    return torch.cat(outs, 1).cpu().numpy()


@pytest.mark.parametrize("name", ["mod_decode", "mod_decode_prev", "mod_decode_ram"])
def test_module_decode_matches_reference(name, monkeypatch):
    meta, g = load_case(name)
    print(f"[decode] module {name}", flush=True)
    seen = []
    real = ops.route_decode

    def spy(cfg, q, ck, gk, n_closed):
        r = real(cfg, q, ck, gk, n_closed)
        seen.append((n_closed, r["mid"].cpu().numpy(), r["open_grp"].cpu().numpy()))
        return r

    monkeypatch.setattr(hrouter.ops, "route_decode", spy)
    m = _module(meta, g)
    x = torch.from_numpy(g["x"]).to(DEV)
    out = _run_module(m, x, meta["S"], meta["gen"])
    np.testing.assert_allclose(out, g["out"], atol=F32_TOL, rtol=0)
    assert len(seen) == meta["gen"]
    for i, (ncl, mid, og) in enumerate(seen):
        assert ncl == g["dec_n_closed"][i]
        _same_lists(mid, g["dec_sel"][i])
        _same_lists(og, g["dec_open"][i])


def _run_module_blocks(m, x, S, blocks):
    """Prefill S tokens, then blocks of the given token counts."""
    cache = _Cache()
    outs = []
    with torch.no_grad():
        o, _ = m(hidden_states=x[:, :S], past_key_value=cache,
                 cache_position=torch.arange(S, device=DEV))
        outs.append(o)
        p = S
        for L in blocks:
            o, _ = m(hidden_states=x[:, p:p + L], past_key_value=cache,
                     cache_position=torch.arange(p, p + L, device=DEV))
            outs.append(o)
            p += L
    torch.cuda.synchronize()
    return torch.cat(outs, 1).cpu().numpy()


@pytest.mark.parametrize("name,loc", [("mod_blocks", "vram"), ("mod_blocks", "ram"),
                                      ("mod_blocks", "fs"), ("mod_blocks64", "ram"),
                                      ("mod_blocks64", "vram")])
def test_module_multi_row_blocks_match_reference(name, loc, monkeypatch):
    """Blocks of 3, 11 and 64 tokens after a prefill, recorded from the reference module
    (tests/golden/make_golden.py): every decode segment's routing decision -- L rows pooled
    for the chunk selection, the groups requested over all rows, each id with its first
    visible row (chunk_router.py:187-277) -- bit for bit, and the outputs within fp32
    tolerance.  mod_blocks64 routes a whole 64-row chunk in one segment."""
    meta, g = load_case(name)
    print(f"[decode] blocks {name} {loc} {meta['blocks']}", flush=True)
    seen = []
    real = ops.route_decode

    def spy(cfg, q, ck, gk, n_closed):
        r = real(cfg, q, ck, gk, n_closed)
        seen.append((q.shape[2], {k: r[k].cpu().numpy() for k in
                                  ("mid", "mid_thr", "open_grp", "open_thr")}))
        return r

    monkeypatch.setattr(hrouter.ops, "route_decode", spy)
    m = _module(meta, g, loc)
    x = torch.from_numpy(g["x"]).to(DEV)
    out = _run_module_blocks(m, x, meta["S"], meta["blocks"])
    np.testing.assert_allclose(out, g["out"], atol=F32_TOL, rtol=0)
    assert len(seen) == len(g["blk_L"])
    for i, (L, r) in enumerate(seen):
        assert L == g["blk_L"][i]
        _same_lists(r["mid"], g["blk_sel"][i])
        _same_lists(r["mid_thr"], g["blk_sel_thr"][i])
        _same_lists(r["open_grp"], g["blk_open"][i])
        _same_lists(r["open_thr"], g["blk_open_thr"][i])


@pytest.mark.parametrize("loc", ["ram", "fs"])
def test_module_host_stores_equal_vram_store(loc):
    meta, g = load_case("mod_decode")
    x = torch.from_numpy(g["x"]).to(DEV)
    a = _run_module(_module(meta, g, "vram"), x, meta["S"], meta["gen"])
    b = _run_module(_module(meta, g, loc), x, meta["S"], meta["gen"])
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("loc", ["vram", "ram", "fs"])
@pytest.mark.parametrize("block", [3, 11])
def test_module_multi_token_blocks_vs_oracle(loc, block):
    """Blocks of several tokens over resident context -- inside one chunk, and crossing chunk
    boundaries (one decode segment per chunk, chunk_router.py:493-516) -- against the oracle
    module fed the same blocks; routing decisions compared bit-exactly."""
    meta, g = load_case("mod_decode_ram")
    print(f"[decode] multi-token blocks loc={loc} block={block}", flush=True)
    seen = []
    real = ops.route_decode

    def spy(cfg, q, ck, gk, n_closed):
        r = real(cfg, q, ck, gk, n_closed)
        seen.append((n_closed, r["mid"].cpu().numpy(), r["open_grp"].cpu().numpy()))
        return r

    x = torch.from_numpy(g["x"])
    S, gen = meta["S"], meta["gen"]
    om = OracleModule(meta, g)
    ref = [om.forward(x[:, :S], 0)]
    p = S
    while p < S + gen:
        e = min(S + gen, p + block)
        ref.append(om.forward(x[:, p:e], p))
        p = e
    ref = torch.cat(ref, 1).numpy()
    orig = hrouter.ops.route_decode
    hrouter.ops.route_decode = spy
    try:
        out = _run_module(_module(meta, g, loc), x.to(DEV), S, gen, block=block)
    finally:
        hrouter.ops.route_decode = orig
    np.testing.assert_allclose(out, ref, atol=F32_TOL, rtol=0)
    assert len(seen) == len(om.decisions)
    for (ncl, mid, og), (oncl, r) in zip(seen, om.decisions):
        assert ncl == oncl
        _same_lists(mid, r["mid"])
        _same_lists(og, r["open_grp"])


# ----------------------------------------------------------------------------------------------
# ops level: routing and attention against the oracle at c4-like shapes
# ----------------------------------------------------------------------------------------------
def _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dtype):
    return ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                           group_size=gs, topk_chunks=tc, topk_groups=tg, keep_first=kf,
                           keep_last=kl, cutoff_pair=ops.mixed_cutoff_pair(1e6, C, Dh),
                           dtype=dtype)


def _summaries(gen, B, KVH, cap, M, Dh, dtype, dup=False):
    ck = torch.randn(B, KVH, cap, Dh, generator=gen)
    gk = torch.randn(B, KVH, cap, M, Dh, generator=gen)
    if dup:   # exact score ties: every 3rd chunk/group repeats its predecessor
        ck[:, :, 3::3] = ck[:, :, 2:-1:3][:, :, :ck[:, :, 3::3].shape[2]]
        gk[:, :, :, 1::2] = gk[:, :, :, 0::2][:, :, :, :gk[:, :, :, 1::2].shape[3]]
    return ck.to(dtype), gk.to(dtype)


ROUTE_CASES = [
    # B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, L, dtype
    (2, 8, 2, 128, 64, 16, 16, 64, 2, 8, 40, 1, torch.bfloat16),
    (2, 8, 2, 128, 64, 16, 16, 64, 2, 8, 40, 7, torch.bfloat16),
    (1, 8, 2, 128, 64, 16, 16, 64, 2, 8, 511, 1, torch.bfloat16),     # 32K context
    (1, 4, 1, 128, 64, 16, 16, 64, 2, 8, 2047, 1, torch.bfloat16),    # 128K context
    (1, 4, 2, 128, 64, 16, 16, 64, 2, 8, 300, 5, torch.float32),
    (2, 4, 2, 64, 32, 8, 5, 9, 1, 3, 17, 3, torch.float32),
    (1, 4, 2, 64, 64, 16, 4, 64, 0, 0, 9, 2, torch.float32),          # tg > Kc*M, no windows
    (1, 4, 2, 128, 64, 16, 16, 64, 2, 8, 12, 1, torch.bfloat16),      # pool smaller than tc
    (1, 4, 2, 128, 64, 16, 16, 64, 2, 8, 6, 1, torch.bfloat16),       # everything in windows
    (1, 4, 1, 128, 64, 16, 16, 64, 2, 8, 8191, 1, torch.bfloat16),    # 512K context, 17 segments
    (1, 4, 2, 128, 64, 16, 16, 64, 2, 8, 2047, 64, torch.bfloat16),   # 128K context, 64-row block
    (1, 4, 2, 128, 64, 16, 64, 256, 2, 8, 1200, 64, torch.float32),   # Kc 64, fp32: short segments
    (1, 4, 2, 64, 64, 16, 4, 64, 0, 0, 1300, 2, torch.float32),       # forced previous, long pool
    (1, 2, 1, 128, 64, 16, 16, 64, 2, 8, 8191, 64, torch.bfloat16),   # 64 rows, 512K: merge of 2048
    (1, 4, 2, 64, 64, 16, 16, 64, 2, 8, 650, 16, torch.bfloat16),     # pool = 10 whole 64-segments
    (1, 4, 2, 64, 64, 16, 40, 160, 0, 3, 300, 5, torch.float32),      # 5 rows, Kc 40, one segment
]


@pytest.mark.parametrize("case", ROUTE_CASES, ids=lambda c: f"B{c[0]}H{c[1]}n{c[10]}L{c[11]}"
                         f"{'bf16' if c[12] is torch.bfloat16 else 'f32'}")
def test_route_decode_vs_oracle(case):
    B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, L, dt = case
    print(f"[decode] route {case}", flush=True)
    M = C // gs
    gen = torch.Generator().manual_seed(n_closed * 31 + L)
    cap = n_closed + 3
    ck, gk = _summaries(gen, B, KVH, cap, M, Dh, dt)
    q = torch.randn(B, H, L, Dh, generator=gen).to(dt)
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt)
    r = ops.route_decode(cfg, q.to(DEV), ck.to(DEV), gk.to(DEV), n_closed)
    torch.cuda.synchronize()
    o = oracle.route_decode(q.float().numpy(), ck.float().numpy(), gk.float().numpy(), n_closed,
                            kf, kl, tc, tg, oracle.attn_scale(Dh))
    for key in ("mid", "mid_thr", "open_grp", "open_thr"):
        _same_lists(r[key].cpu().numpy(), o[key])
    np.testing.assert_array_equal(r["n_mid"].cpu().numpy(), o["n_mid"])
    np.testing.assert_array_equal(r["n_open"].cpu().numpy(), o["n_open"])


@pytest.mark.parametrize("L", [1, 4])
def test_route_decode_exact_ties(L):
    B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed = 1, 8, 2, 128, 64, 16, 8, 16, 1, 2, 60
    M = C // gs
    gen = torch.Generator().manual_seed(77 + L)
    ck, gk = _summaries(gen, B, KVH, n_closed, M, Dh, torch.bfloat16, dup=True)
    q = torch.randn(B, H, L, Dh, generator=gen).to(torch.bfloat16)
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, torch.bfloat16)
    r = ops.route_decode(cfg, q.to(DEV), ck.to(DEV), gk.to(DEV), n_closed)
    o = oracle.route_decode(q.float().numpy(), ck.float().numpy(), gk.float().numpy(), n_closed,
                            kf, kl, tc, tg, oracle.attn_scale(Dh))
    for key in ("mid", "mid_thr", "open_grp", "open_thr"):
        _same_lists(r[key].cpu().numpy(), o[key])


@pytest.mark.parametrize("L", [1, 64])
def test_route_decode_periodic_pool(L):
    """Chunk and group summaries repeat with period 7 over a 1500-chunk pool: every selection
    boundary is a tie spread over all stage-1 segments, so the running lists must keep the lowest
    ids of each score class (chunk_router.py:227-231 take torch.topk over the whole pool)."""
    B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed = 1, 4, 2, 128, 64, 16, 16, 64, 2, 8, 1500
    M = C // gs
    print(f"[decode] route periodic L={L}", flush=True)
    gen = torch.Generator().manual_seed(1234 + L)
    base_c = torch.randn(B, KVH, 7, Dh, generator=gen)
    base_g = torch.randn(B, KVH, 7, M, Dh, generator=gen)
    idx = torch.arange(n_closed) % 7
    ck, gk = base_c[:, :, idx].to(torch.bfloat16), base_g[:, :, idx].to(torch.bfloat16)
    q = torch.randn(B, H, L, Dh, generator=gen).to(torch.bfloat16)
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, torch.bfloat16)
    r = ops.route_decode(cfg, q.to(DEV), ck.to(DEV), gk.to(DEV), n_closed)
    o = oracle.route_decode(q.float().numpy(), ck.float().numpy(), gk.float().numpy(), n_closed,
                            kf, kl, tc, tg, oracle.attn_scale(Dh))
    for key in ("mid", "mid_thr", "open_grp", "open_thr"):
        _same_lists(r[key].cpu().numpy(), o[key])
    # the pooled top-16 of a period-7 pool is the best class's 16 lowest-id members
    assert (o["mid"] < oracle.windows(n_closed, kf, kl)[0] + 7 * 16).all()


def _history(gen, B, KVH, T, Dh, dt):
    k = (torch.randn(B, KVH, T, Dh, generator=gen) * 0.5).to(dt)
    v = torch.randn(B, KVH, T, Dh, generator=gen).to(dt)
    return k, v


ATTN_CASES = [
    # B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, c0, L, dtype
    (2, 8, 2, 128, 64, 16, 16, 64, 2, 8, 40, 0, 1, torch.bfloat16),
    (2, 8, 2, 128, 64, 16, 16, 64, 2, 8, 40, 37, 7, torch.bfloat16),
    (1, 8, 2, 128, 64, 16, 16, 64, 2, 8, 511, 63, 1, torch.bfloat16),
    (1, 4, 2, 128, 64, 16, 16, 64, 2, 8, 300, 10, 5, torch.float32),
    (2, 4, 2, 64, 32, 8, 5, 9, 1, 3, 17, 30, 2, torch.float32),
    (1, 4, 2, 64, 64, 16, 4, 64, 0, 0, 9, 0, 2, torch.float32),
    (1, 4, 2, 32, 16, 4, 3, 5, 1, 1, 0, 5, 3, torch.float32),         # nothing closed yet
    # blocks of 8+ bf16 rows take the MFMA split kernel
    (1, 8, 2, 128, 64, 16, 16, 64, 2, 8, 200, 0, 64, torch.bfloat16),  # a whole 64-row chunk
    (2, 4, 2, 64, 32, 8, 5, 9, 1, 3, 40, 7, 20, torch.bfloat16),       # 20 rows from c0 7
    (1, 4, 1, 128, 64, 16, 16, 64, 2, 8, 3, 16, 48, torch.bfloat16),   # few closed chunks
]


def _ring(k, n_closed, C, kf, kl, R):
    """Ring of R chunk slots holding chunks [l_lo, n_closed] at slot c % R (other slots hold
    garbage that must never be read)."""
    B, KVH, T, Dh = k.shape
    ring = torch.full((B, KVH, R * C, Dh), float("nan"), dtype=k.dtype)
    l_lo = oracle.windows(n_closed, kf, kl)[1]
    for c in range(l_lo, n_closed + 1):
        a = c * C
        e = min(T, a + C)
        ring[:, :, (c % R) * C:(c % R) * C + e - a] = k[:, :, a:e]
    return ring


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: f"B{c[0]}n{c[10]}c{c[11]}L{c[12]}"
                         f"{'bf16' if c[13] is torch.bfloat16 else 'f32'}")
@pytest.mark.parametrize("tier", ["vram", "ram", "gather"])
def test_attend_decode_vs_oracle(case, tier):
    B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, c0, L, dt = case
    print(f"[decode] attend {tier} {case}", flush=True)
    M = C // gs
    gen = torch.Generator().manual_seed(n_closed * 7 + c0)
    start = n_closed * C + c0
    T = start + L
    k, v = _history(gen, B, KVH, T, Dh, dt)
    q = torch.randn(B, H, L, Dh, generator=gen).to(dt)
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt)
    if n_closed:
        ck, gk = _summaries(gen, B, KVH, n_closed, M, Dh, dt)
        r = ops.route_decode(cfg, q.to(DEV), ck.to(DEV), gk.to(DEV), n_closed)
        og, ot, Kg = r["open_grp"], r["open_thr"], r["Kg"]
    else:
        og = ot = torch.full((B, H, 1), -1, dtype=torch.int32, device=DEV)
        Kg = 0
    if tier == "vram":
        kd, vd = k.to(DEV), v.to(DEV)
        out = ops.attend_decode(cfg, q.to(DEV), n_closed, start, kd, vd, 0, kd, vd, kd, vd,
                                False, og, ot, Kg)
    else:
        R = kl + 1 + 2     # wider than needed: slot = chunk % R must be honoured
        rk, rv = _ring(k, n_closed, C, kf, kl, R), _ring(v, n_closed, C, kf, kl, R)
        fk = k[:, :, :max(kf, 1) * C].contiguous()
        fv = v[:, :, :max(kf, 1) * C].contiguous()
        hk = torch.zeros(B, KVH, (n_closed + 1) * C, Dh, dtype=dt, pin_memory=True)
        hv = torch.zeros_like(hk).pin_memory()
        hk[:, :, :n_closed * C] = k[:, :, :n_closed * C]
        hv[:, :, :n_closed * C] = v[:, :, :n_closed * C]
        out = ops.attend_decode(cfg, q.to(DEV), n_closed, start, rk.to(DEV), rv.to(DEV), R,
                                fk.to(DEV), fv.to(DEV), hk, hv, True, og, ot, Kg)
        if tier == "gather":
            # opened groups staged in device memory: the same keys in the same order, so the
            # result equals the zero-copy read bit for bit
            staged = ops.gather_decode(cfg, n_closed, og, ot, Kg, hk, hv, True,
                                       ops.DecodeStaging(), H)
            out_g = ops.attend_decode(cfg, q.to(DEV), n_closed, start, rk.to(DEV), rv.to(DEV),
                                      R, fk.to(DEV), fv.to(DEV), staged[0], staged[1], False,
                                      staged[2], ot, Kg)
            torch.cuda.synchronize()
            assert torch.equal(out_g, out)
    torch.cuda.synchronize()
    ref = oracle.attend_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), C, gs,
                               kf, kl, n_closed, start, og.cpu().numpy(), ot.cpu().numpy(),
                               oracle.attn_scale(Dh),
                               oracle.DT_BF16 if dt is torch.bfloat16 else oracle.DT_F32)
    d = np.abs(out.float().cpu().numpy() - ref)
    if dt is torch.bfloat16:
        assert d.max() <= BF16_MAX and d.mean() <= BF16_MEAN, (d.max(), d.mean())
    else:
        assert d.max() <= F32_TOL, d.max()


@pytest.mark.parametrize("on_host,n_closed", [(True, 40), (False, 40), (False, 8200)])
def test_gather_decode_contents(on_host, n_closed):
    """Staged groups are the record's groups, one slot per distinct (b, kv head, group) in
    ascending group order; every opened entry maps to its group's slot, padding to -1.  At 40
    closed chunks the plan and the copy run in one launch; at 8200 (a group bitmap of more than
    4096 words over the (b, kv head) pairs) they run as two."""
    B, H, KVH, Dh, C, gs, tc, tg, kf, kl = 2, 8, 2, 128, 64, 16, 8, 16, 1, 2
    dt = torch.bfloat16
    if n_closed > 1000:
        Dh = 64
    M = C // gs
    gen = torch.Generator().manual_seed(17)
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt)
    q = torch.randn(B, H, 1, Dh, generator=gen).to(dt)
    ck, gk = _summaries(gen, B, KVH, n_closed, M, Dh, dt)
    r = ops.route_decode(cfg, q.to(DEV), ck.to(DEV), gk.to(DEV), n_closed)
    og, ot, Kg = r["open_grp"], r["open_thr"], r["Kg"]
    k, v = _history(gen, B, KVH, n_closed * C, Dh, dt)
    if on_host:
        hk = torch.empty(B, KVH, n_closed * C, Dh, dtype=dt, pin_memory=True)
        hv = torch.empty_like(hk).pin_memory()
        hk.copy_(k)
        hv.copy_(v)
    else:
        hk, hv = k.to(DEV), v.to(DEV)
    sk, sv, sg = ops.gather_decode(cfg, n_closed, og, ot, Kg, hk, hv, on_host,
                                   ops.DecodeStaging(), H)
    torch.cuda.synchronize()
    og_, ot_, sg_ = og.cpu().numpy(), ot.cpu().numpy(), sg.cpu().numpy()
    sk_, sv_ = sk.cpu(), sv.cpu()
    rep = H // KVH
    for b in range(B):
        for kvh in range(KVH):
            ids = sorted({int(x) for h in range(kvh * rep, (kvh + 1) * rep)
                          for x, t in zip(og_[b, h, :Kg], ot_[b, h, :Kg]) if x >= 0 and t >= 0})
            for slot, grp in enumerate(ids):
                p0 = (grp // M) * C + (grp % M) * gs
                assert torch.equal(sk_[b, kvh, slot * gs:(slot + 1) * gs], k[b, kvh, p0:p0 + gs])
                assert torch.equal(sv_[b, kvh, slot * gs:(slot + 1) * gs], v[b, kvh, p0:p0 + gs])
            for h in range(kvh * rep, (kvh + 1) * rep):
                for i in range(Kg):
                    valid = og_[b, h, i] >= 0 and ot_[b, h, i] >= 0
                    want = ids.index(int(og_[b, h, i])) if valid else -1
                    assert sg_[b, h, i] == want


def test_attend_decode_rejects_bad_blocks():
    cfg = _cfg(1, 4, 2, 64, 64, 16, 4, 8, 1, 1, torch.float32)
    q = torch.zeros(1, 4, 2, 64, device=DEV)
    kv = torch.zeros(1, 2, 256, 64, device=DEV)
    e = torch.full((1, 4, 1), -1, dtype=torch.int32, device=DEV)
    with pytest.raises(hga.HgaError, match="not inside active chunk"):
        ops.attend_decode(cfg, q, 1, 64 + 63, kv, kv, 0, kv, kv, kv, kv, False, e, e, 0)
    with pytest.raises(hga.HgaError, match="ring"):
        ops.attend_decode(cfg, q, 3, 3 * 64, kv, kv, 1, kv, kv, kv, kv, False, e, e, 0)


# ----------------------------------------------------------------------------------------------
# token ingest: hga_write_tokens against torch's copies
# ----------------------------------------------------------------------------------------------
def _wcfg(B, KVH, Dh, dt):
    return ops.make_config(batch=B, heads=2 * KVH, kv_heads=KVH, head_dim=Dh, chunk_size=64,
                           group_size=16, topk_chunks=4, topk_groups=8, keep_first=1, keep_last=2,
                           cutoff_pair=3, dtype=dt)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L", [1, 7, 64])
def test_write_tokens_matches_copies(dt, L):
    """Strided sources (a [B, L, KVH, Dh] tensor seen as [B, KVH, L, Dh]) land bit-exactly in a
    record slice, a ring slice and an active-chunk slice; every other element stays as it was."""
    B, KVH, Dh = 2, 3, 64
    g = torch.Generator(device=DEV).manual_seed(11 + L)
    srcs = [torch.randn(B, L, KVH, Dh, generator=g, device=DEV).to(dt).transpose(1, 2)
            for _ in range(3)]
    rec = torch.randn(B, KVH, 300, Dh, generator=g, device=DEV).to(dt)
    ring = torch.randn(B, KVH, 192, Dh, generator=g, device=DEV).to(dt)
    act = torch.randn(B, KVH, 64, Dh, generator=g, device=DEV).to(dt)
    want = [t.clone() for t in (rec, ring, act)]
    p, s, c0 = 130, 64, 64 - L
    for w, src, a in zip(want, srcs, (p, s, c0)):
        w[:, :, a:a + L] = src
    ops.write_tokens(_wcfg(B, KVH, Dh, dt), L, [(srcs[0], rec[:, :, p:p + L]),
                                                (srcs[1], ring[:, :, s:s + L]),
                                                (srcs[2], act[:, :, c0:c0 + L])])
    torch.cuda.synchronize()
    for got, w in zip((rec, ring, act), want):
        assert torch.equal(got, w)


def test_write_tokens_past_2g_elements_and_skipped_sets():
    """Rows beyond element 2^31 of a record are addressed exactly (64-bit offsets): a record of
    two sequences whose batch stride exceeds 2^31 elements, rows written near the end of both,
    so the second sequence's b * d_sb term alone crosses 2^31 (and the whole offset 2^32).  A
    row set given as None is left out."""
    Dh, L, B = 64, 5, 2
    rows = (1 << 31) // Dh + 96
    rec = torch.empty(B, 1, rows, Dh, dtype=torch.bfloat16, device=DEV)
    assert rec.stride(0) > (1 << 31)
    try:
        g = torch.Generator(device=DEV).manual_seed(3)
        k = torch.randn(B, 1, L, Dh, generator=g, device=DEV).to(torch.bfloat16)
        raw = torch.randn(B, 1, L, Dh, generator=g, device=DEV).to(torch.bfloat16)
        act = torch.zeros(B, 1, 64, Dh, dtype=torch.bfloat16, device=DEV)
        pos = rows - 40
        before = rec[:, :, pos - 8:pos].clone()
        after = rec[:, :, pos + L:pos + L + 8].clone()
        ops.write_tokens(_wcfg(B, 1, Dh, torch.bfloat16), L,
                         [(k, rec[:, :, pos:pos + L]), None, (raw, act[:, :, 3:3 + L])])
        torch.cuda.synchronize()
        assert torch.equal(rec[:, :, pos:pos + L], k)
        assert torch.equal(rec[:, :, pos - 8:pos], before)
        assert torch.equal(rec[:, :, pos + L:pos + L + 8], after)
        assert torch.equal(act[:, :, 3:3 + L], raw)
        assert not act[:, :, :3].any() and not act[:, :, 3 + L:].any()
    finally:
        del rec
        torch.cuda.empty_cache()


def test_write_tokens_rejects_mismatches():
    cfg = _wcfg(1, 2, 64, torch.bfloat16)
    a = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(TypeError):
        ops.write_tokens(cfg, 4, [(a.float(), a.float())])
    with pytest.raises(ValueError):
        ops.write_tokens(cfg, 3, [(a, a)])
    with pytest.raises(RuntimeError):
        ops.write_tokens(cfg, 4, [(a.cpu(), a)])


@pytest.mark.parametrize("case", [c for c in ATTN_CASES if c[3] in (64, 128)],
                         ids=lambda c: f"B{c[0]}n{c[10]}c{c[11]}L{c[12]}"
                         f"{'bf16' if c[13] is torch.bfloat16 else 'f32'}")
def test_attend_decode_phases_equal_one_launch(case):
    """hga_attend_decode_phase: the windows and active chunk (phase 1) while the opened groups
    are gathered into device staging, then the opened groups (phase 2) from the staging --
    bit-identical to the one-launch attention over the host record (same split partition and
    combine)."""
    B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, c0, L, dt = case
    print(f"[decode] phases {case}", flush=True)
    M = C // gs
    gen = torch.Generator().manual_seed(n_closed * 5 + c0 + 1)
    start = n_closed * C + c0
    T = start + L
    k, v = _history(gen, B, KVH, T, Dh, dt)
    q = torch.randn(B, H, L, Dh, generator=gen).to(dt).to(DEV)
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt)
    if n_closed:
        ck, gk = _summaries(gen, B, KVH, n_closed, M, Dh, dt)
        r = ops.route_decode(cfg, q, ck.to(DEV), gk.to(DEV), n_closed)
        og, ot, Kg = r["open_grp"], r["open_thr"], r["Kg"]
    else:
        og = ot = torch.full((B, H, 1), -1, dtype=torch.int32, device=DEV)
        Kg = 0
    R = kl + 3
    rk, rv = _ring(k, n_closed, C, kf, kl, R).to(DEV), _ring(v, n_closed, C, kf, kl, R).to(DEV)
    fk = k[:, :, :max(kf, 1) * C].contiguous().to(DEV)
    fv = v[:, :, :max(kf, 1) * C].contiguous().to(DEV)
    hk = torch.zeros(B, KVH, (n_closed + 1) * C, Dh, dtype=dt, pin_memory=True)
    hv = torch.zeros_like(hk).pin_memory()
    hk[:, :, :n_closed * C] = k[:, :, :n_closed * C]
    hv[:, :, :n_closed * C] = v[:, :, :n_closed * C]
    one = ops.attend_decode(cfg, q, n_closed, start, rk, rv, R, fk, fv, hk, hv, True, og, ot, Kg)
    staged = ops.gather_decode(cfg, n_closed, og, ot, Kg, hk, hv, True, ops.DecodeStaging(), H)
    ws = ops.attend_decode_workspace(cfg, L, n_closed, start, Kg, q.device)
    out = ops.attend_decode(cfg, q, n_closed, start, rk, rv, R, fk, fv, staged[0], staged[1],
                            False, og, ot, Kg, phase=1, workspace=ws)
    out = ops.attend_decode(cfg, q, n_closed, start, rk, rv, R, fk, fv, staged[0], staged[1],
                            False, staged[2], ot, Kg, out=out, phase=2, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out, one)
