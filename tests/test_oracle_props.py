"""Pin the oracle with closed forms and invariants that the mathematics fixes."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from helpers import rope_torch, rotary_table


def _inputs(seed, B, H, KVH, S, Dh, theta):
    g = torch.Generator().manual_seed(seed)
    q_raw, k_raw, v = (torch.randn(B, X, S, Dh, generator=g) for X in (H, KVH, KVH))
    cos, sin = rotary_table(S, Dh, theta)
    return rope_torch(q_raw, cos, sin), rope_torch(k_raw, cos, sin), k_raw, v, cos, sin


@pytest.mark.parametrize("S,C,gs", [(28, 8, 4), (37, 8, 4), (300, 64, 16)])
def test_full_coverage_equals_causal_sdpa(S, C, gs):
    """topk 0 and a keep_last window covering every chunk reduce the routed attention to dense
    causal attention (the reference's own check, KvRouter/Tests/test_router.py:37-62 and
    Qwen3LongContext/test_qwen30b_routed.py:80-143)."""
    B, H, KVH, Dh = 2, 4, 2, 16
    q, k, k_raw, v, cos, sin = _inputs(0, B, H, KVH, S, Dh, 1e4)
    out, r, _, _ = oracle.prefill(q.numpy(), k.numpy(), k_raw.numpy(), v.numpy(), cos.numpy(),
                                  sin.numpy(), C=C, gs=gs, keep_first=0, keep_last=10_000,
                                  topk_chunks=0, topk_groups=0, theta=1e4, dt=oracle.DT_F32)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(H // KVH, 1),
                                         v.repeat_interleave(H // KVH, 1), is_causal=True)
    assert np.abs(out - ref.numpy()).max() < 1e-5


def test_summary_closed_forms():
    B, KVH, S, Dh, C, gs = 1, 2, 96, 16, 16, 4
    _, k_rope, k_raw, _, cos, sin = _inputs(1, B, 2, KVH, S, Dh, 1e4)
    kr, kp = k_raw.numpy(), k_rope.numpy()
    N, M = S // C, C // gs
    # cutoff = Dh/2: every pair token-wise -> plain sums of the roped keys (scaled for groups)
    ck, gk = oracle.summarize(kr, kp, cos.numpy(), sin.numpy(), C, gs, Dh // 2, 0.25,
                              oracle.DT_F32)
    np.testing.assert_allclose(ck, kp.reshape(B, KVH, N, C, Dh).sum(3), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gk, kp.reshape(B, KVH, N, M, gs, Dh).sum(4) * 0.25, rtol=1e-5,
                               atol=1e-5)
    # cutoff = 0: every pair anchor-rotated -> RoPE(sum of raw keys) at the middle token
    ck0, gk0 = oracle.summarize(kr, kp, cos.numpy(), sin.numpy(), C, gs, 0, 0.25, oracle.DT_F32)
    raw_sum = torch.from_numpy(kr.reshape(B, KVH, N, C, Dh).sum(3))
    mid = torch.arange(N) * C + (C - 1) // 2
    want = rope_torch(raw_sum, cos[mid], sin[mid]).numpy()
    np.testing.assert_allclose(ck0, want, rtol=1e-5, atol=1e-5)
    gmid = (torch.arange(N)[:, None] * C + torch.arange(M)[None] * gs + (gs - 1) // 2)
    graw = torch.from_numpy(kr.reshape(B, KVH, N, M, gs, Dh).sum(4) * 0.25)
    want = rope_torch(graw, cos[gmid], sin[gmid]).numpy()
    np.testing.assert_allclose(gk0, want, rtol=1e-5, atol=1e-5)
    # equal positions make token-wise and anchored sums agree (RoPE is linear)
    same = np.repeat(kr[:, :, :1], S, axis=2)
    cos1 = np.repeat(cos.numpy()[5:6], S, 0)
    sin1 = np.repeat(sin.numpy()[5:6], S, 0)
    rot = rope_torch(torch.from_numpy(same), torch.from_numpy(cos1), torch.from_numpy(sin1)).numpy()
    a, _ = oracle.summarize(same, rot, cos1, sin1, C, gs, Dh // 2, 0.25, oracle.DT_F32)
    b, _ = oracle.summarize(same, rot, cos1, sin1, C, gs, 0, 0.25, oracle.DT_F32)
    np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("kf,kl,tc,tg", [(1, 2, 4, 8), (0, 0, 3, 6), (2, 1, 16, 10), (1, 1, 2, 1)])
def test_routing_invariants(kf, kl, tc, tg):
    B, H, KVH, S, Dh, C, gs = 1, 4, 2, 40 * 16 + 7, 16, 16, 4
    q, k, k_raw, v, cos, sin = _inputs(2, B, H, KVH, S, Dh, 1e4)
    _, r, _, _ = oracle.prefill(q.numpy(), k.numpy(), k_raw.numpy(), v.numpy(), cos.numpy(),
                                sin.numpy(), C=C, gs=gs, keep_first=kf, keep_last=kl,
                                topk_chunks=tc, topk_groups=tg, theta=1e4, dt=oracle.DT_F32)
    N, M, Kc, Kg = oracle.sizes(S, C, gs, tc, tg)
    for h in range(H):
        for n in range(N):
            f_hi, l_lo = oracle.windows(n, kf, kl)
            pool = set(range(f_hi, l_lo))
            rows = min(C, S - n * C)
            sel = [(c, t) for c, t in zip(r["sel_chunk"][0, h, n], r["sel_thr"][0, h, n]) if c >= 0]
            ids = [c for c, _ in sel]
            assert ids == sorted(ids) and set(ids) <= pool
            assert len(ids) == min(Kc, len(pool))          # pool large enough, or all of it
            if kl == 0 and n - 1 in pool:
                assert (n - 1, 0) in sel                    # forced previous chunk
            assert all(0 <= t < rows for _, t in sel)
            thrA = dict(sel)
            opened = [(g, t) for g, t in zip(r["open_grp"][0, h, n], r["open_thr"][0, h, n]) if g >= 0]
            assert len(opened) <= Kg
            for g, t in opened:
                assert g // M in thrA and t >= thrA[g // M] and t < rows


def test_canonical_score_is_the_fma_chain():
    """The canonical score is a sequential fp32 FMA chain times the fp32 scale: it stays within
    the chain's rounding bound of the exact dot product."""
    rng = np.random.default_rng(0)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)
    import ctypes
    lib = oracle.lib()
    fp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    got = lib.orc_score(fp(q), fp(k), 64, ctypes.c_float(0.125))
    exact = float(np.dot(q.astype(np.float64), k.astype(np.float64))) * 0.125
    assert abs(got - exact) <= 64 * 2 ** -24 * float(np.abs(q * k).sum())


def test_per_head_routing_and_chunk_subset_attention_agree():
    """The test helpers that make the 32K cases fit in seconds: routing one query head per
    thread equals one call over all heads, and attention of a query-chunk subset equals those
    rows of the full attention (NaN elsewhere)."""
    B, H, KVH, S, Dh, C, gs = 2, 4, 2, 700, 32, 32, 8
    q, k, k_raw, v, cos, sin = _inputs(7, B, H, KVH, S, Dh, 1e4)
    out, r, ck, gk = oracle.prefill(q.numpy(), k.numpy(), k_raw.numpy(), v.numpy(), cos.numpy(),
                                    sin.numpy(), C=C, gs=gs, keep_first=1, keep_last=2,
                                    topk_chunks=3, topk_groups=5, theta=1e4, dt=oracle.DT_F32)
    rh = oracle.route_prefill_heads(q.numpy(), ck, gk, S, C, gs, 1, 2, 3, 5,
                                    oracle.attn_scale(Dh), threads=3)
    for key in r:
        np.testing.assert_array_equal(rh[key], r[key])
    chunks = [0, 5, 21]
    sub = oracle.attend_prefill(q.numpy(), k.numpy(), v.numpy(), C, gs, 1, 2, r["open_grp"],
                                r["open_thr"], oracle.attn_scale(Dh), oracle.DT_F32,
                                chunks=chunks)
    rows = np.concatenate([np.arange(n * C, min(S, (n + 1) * C)) for n in chunks])
    np.testing.assert_array_equal(sub[:, :, rows], out[:, :, rows])
    other = np.setdiff1d(np.arange(S), rows)
    assert np.isnan(sub[:, :, other]).all()
