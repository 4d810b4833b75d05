"""Pins the oracle's attention gradient (orc_attend_prefill_bwd) on the CPU.

The routed attention of a prefill block equals dense attention under a boolean mask (row (n, t)
sees the first window, the last window, the opened groups whose first visible row is <= t and
its own chunk causally).  The mask built here is first checked to reproduce the oracle's forward
(``attend_prefill``, itself pinned against the reference's fixtures); torch float64 autograd of
the masked dense attention then gives the exact gradients, which the oracle's hand-derived
formulas must match -- including GQA head sums, ragged tails, rows that see no routed group and
groups opened only from a later row.
"""
import numpy as np
import pytest
import torch

import oracle


def random_lists(rng, B, H, S, C, gs, kf, kl, Kg):
    """Valid routing lists: ascending distinct pool groups, first visible rows in [0, rows) or
    -1 (never visible), -1 padded at the end."""
    N, M = (S + C - 1) // C, C // gs
    og = np.full((B, H, N, max(Kg, 1)), -1, np.int32)
    ot = np.full_like(og, -1)
    for b in range(B):
        for h in range(H):
            for n in range(N):
                f_hi, l_lo = oracle.windows(n, kf, kl)
                pool = np.arange(f_hi * M, max(l_lo, f_hi) * M)
                if Kg == 0 or pool.size == 0:
                    continue
                take = np.sort(rng.choice(pool, size=min(Kg, pool.size), replace=False))
                take = take[: rng.integers(0, take.size + 1)]
                rows = min(C, S - n * C)
                thr = rng.integers(-1, rows, size=take.size)
                og[b, h, n, :take.size] = take
                ot[b, h, n, :take.size] = thr
    return og, ot


def routing_mask(B, H, S, C, gs, kf, kl, og, ot):
    N, M = (S + C - 1) // C, C // gs
    mask = np.zeros((B, H, S, S), bool)
    for b in range(B):
        for h in range(H):
            for n in range(N):
                f_hi, l_lo = oracle.windows(n, kf, kl)
                for t in range(min(C, S - n * C)):
                    i = n * C + t
                    mask[b, h, i, :f_hi * C] = True
                    mask[b, h, i, l_lo * C:n * C] = True
                    mask[b, h, i, n * C:i + 1] = True
                    for g, th in zip(og[b, h, n], ot[b, h, n]):
                        if g >= 0 and 0 <= th <= t:
                            c, m = divmod(int(g), M)
                            mask[b, h, i, c * C + m * gs:c * C + (m + 1) * gs] = True
    return mask


def dense_grads(q, k, v, dout, mask, scale):
    H, KVH = q.shape[1], k.shape[1]
    t = [torch.from_numpy(x.astype(np.float64)).requires_grad_(True) for x in (q, k, v)]
    ke = t[1].repeat_interleave(H // KVH, dim=1)
    ve = t[2].repeat_interleave(H // KVH, dim=1)
    s = (t[0] @ ke.transpose(-1, -2)) * scale
    s = s.masked_fill(~torch.from_numpy(mask), float("-inf"))
    o = torch.softmax(s, dim=-1) @ ve
    (o * torch.from_numpy(dout.astype(np.float64))).sum().backward()
    return o.detach().numpy(), [x.grad.numpy() for x in t]


@pytest.mark.parametrize("shape", [
    dict(B=1, H=4, KVH=2, S=83, Dh=16, C=8, gs=4, kf=1, kl=2, Kg=5),     # ragged tail, GQA 2
    dict(B=2, H=2, KVH=2, S=64, Dh=8, C=16, gs=4, kf=0, kl=0, Kg=6),     # no windows
    dict(B=1, H=6, KVH=1, S=50, Dh=16, C=8, gs=8, kf=2, kl=1, Kg=3),     # MQA, whole-chunk groups
    dict(B=1, H=2, KVH=1, S=40, Dh=16, C=8, gs=4, kf=1, kl=1, Kg=0),     # routing off
])
def test_oracle_bwd_equals_autograd(shape):
    rng = np.random.default_rng(sum(shape.values()))
    B, H, KVH, S, Dh, C, gs, kf, kl, Kg = (shape[x] for x in
                                           ("B", "H", "KVH", "S", "Dh", "C", "gs", "kf", "kl", "Kg"))
    q = rng.standard_normal((B, H, S, Dh)).astype(np.float32)
    k = rng.standard_normal((B, KVH, S, Dh)).astype(np.float32)
    v = rng.standard_normal((B, KVH, S, Dh)).astype(np.float32)
    dout = rng.standard_normal((B, H, S, Dh)).astype(np.float32)
    og, ot = random_lists(rng, B, H, S, C, gs, kf, kl, Kg)
    scale = oracle.attn_scale(Dh)
    mask = routing_mask(B, H, S, C, gs, kf, kl, og, ot)
    o_dense, (gq, gk, gv) = dense_grads(q, k, v, dout, mask, scale)
    o_orc = oracle.attend_prefill(q, k, v, C, gs, kf, kl, og, ot, scale, oracle.DT_F32)
    np.testing.assert_allclose(o_orc, o_dense, atol=2e-6, rtol=0)     # the mask is the key set
    dq, dk, dv = oracle.attend_prefill_bwd(q, k, v, dout, C, gs, kf, kl, og, ot, scale)
    for a, b in ((dq, gq), (dk, gk), (dv, gv)):
        np.testing.assert_allclose(a, b, atol=2e-5, rtol=1e-5)


def test_oracle_bwd_planted_error_fails():
    """A gradient with the D_i term dropped (a plausible mistake) is far outside the tolerance
    above, so the comparison can tell."""
    rng = np.random.default_rng(5)
    B, H, KVH, S, Dh, C, gs, kf, kl = 1, 2, 1, 32, 8, 8, 4, 1, 1
    q, k, v, dout = (rng.standard_normal(s).astype(np.float32) for s in
                     ((B, H, S, Dh), (B, KVH, S, Dh), (B, KVH, S, Dh), (B, H, S, Dh)))
    og, ot = random_lists(rng, B, H, S, C, gs, kf, kl, 2)
    scale = oracle.attn_scale(Dh)
    mask = routing_mask(B, H, S, C, gs, kf, kl, og, ot)
    _, (gq, _, _) = dense_grads(q, k, v, dout, mask, scale)
    # dq without the -D_i term: scale * sum_j p_j dp_j k_j
    t = [torch.from_numpy(x.astype(np.float64)) for x in (q, k, v, dout)]
    s = (t[0] @ t[1].repeat_interleave(H, 1).transpose(-1, -2)) * scale
    p = torch.softmax(s.masked_fill(~torch.from_numpy(mask), float("-inf")), -1)
    dp = t[3] @ t[2].repeat_interleave(H, 1).transpose(-1, -2)
    wrong = (scale * (p * dp) @ t[1].repeat_interleave(H, 1)).numpy()
    assert np.abs(wrong - gq).max() > 1e-2
