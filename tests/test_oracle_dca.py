"""Pins the oracle's Dual Chunk Attention decode (oracle.attend_decode_dca) on the CPU.

Closed form, as the reference's own check does (test_qwen30b_routed.py:218-246, 249-310): with
every key kept (``keep_last`` covering the sequence, no routed middle) the routed DCA path fed
chunk by chunk must equal dense DCA over all earlier keys -- keys RoPE'd at ``pos % L_c``, each
query RoPE'd at ``pos % L_c`` (same DCA chunk), ``min(pos % L_c + L_c, ceil)`` (previous chunk)
and ``ceil`` (older chunks), causal softmax.  The sequence spans five DCA chunks, so all three
regimes are exercised; the dense form here is float64 numpy written independently of the
oracle.  Also: with L_c beyond the sequence every key is intra and DCA equals plain decode
attention over keys and queries RoPE'd at their own positions.
"""
import numpy as np
import pytest

import oracle


def _rope_at(x, pos, theta):
    Dh = x.shape[-1]
    half = Dh // 2
    inv = 1.0 / (theta ** (np.arange(half, dtype=np.float64) / half))
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(np.concatenate([ang, ang], -1)), np.sin(np.concatenate([ang, ang], -1))
    x1, x2 = x[..., :half], x[..., half:]
    return x * c + np.concatenate([-x2, x1], -1) * s


def _dense_dca(q, k, v, theta, L_c, ceil, scale):
    B, H, S, Dh = q.shape
    rep = H // k.shape[1]
    pos = np.arange(S)
    kh = np.repeat(_rope_at(k, pos % L_c, theta), rep, axis=1)
    vh = np.repeat(v.astype(np.float64), rep, axis=1)
    qp = pos % L_c
    qi = _rope_at(q, qp, theta)
    qs = _rope_at(q, np.minimum(qp + L_c, ceil), theta)
    qt = _rope_at(q, np.full(S, ceil), theta)
    sc = {n: np.einsum("bhid,bhjd->bhij", qq, kh) * scale for n, qq in
          (("i", qi), ("s", qs), ("t", qt))}
    cq, ck = (pos // L_c)[:, None], (pos // L_c)[None, :]
    s = np.where(ck == cq, sc["i"], np.where(ck == cq - 1, sc["s"], sc["t"]))
    s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", p, vh)


def _routed_dca(q, k, v, theta, L_c, ceil, scale, C, gs, block):
    """Oracle DCA decode fed `block`-token blocks (each inside one chunk), keeping everything."""
    B, H, S, Dh = q.shape
    pos = np.arange(S)
    k_dca = _rope_at(k, pos % L_c, theta).astype(np.float32)
    out = np.zeros((B, H, S, Dh), np.float32)
    p = 0
    while p < S:
        take = min(block, C - p % C, S - p)
        sl = slice(p, p + take)
        qp = pos[sl] % L_c
        qi = _rope_at(q[:, :, sl], qp, theta).astype(np.float32)
        qs = _rope_at(q[:, :, sl], np.minimum(qp + L_c, ceil), theta).astype(np.float32)
        qt = _rope_at(q[:, :, sl], np.full(take, ceil), theta).astype(np.float32)
        none = -np.ones((B, H, 1), np.int32)
        out[:, :, sl] = oracle.attend_decode_dca(
            qi, qs, qt, k_dca[:, :, :p + take], v[:, :, :p + take].astype(np.float32), C, gs,
            0, 10_000, p // C, p, none, none, scale, oracle.DT_F32, L_c)
        p += take
    return out


@pytest.mark.parametrize("block", [1, 8])
def test_dca_full_coverage_equals_dense(block):
    rng = np.random.default_rng(0)
    B, H, KVH, S, Dh, C, gs, L_c, local = 1, 4, 2, 40, 16, 8, 4, 16, 4
    q = rng.standard_normal((B, H, S, Dh))
    k = rng.standard_normal((B, KVH, S, Dh))
    v = rng.standard_normal((B, KVH, S, Dh))
    scale = Dh ** -0.5
    ref = _dense_dca(q, k, v, 1e4, L_c, L_c + local, scale)
    got = _routed_dca(q, k, v, 1e4, L_c, L_c + local, scale, C, gs, block)
    assert np.abs(got - ref).max() < 1e-5
    # the regimes matter: scoring every key with the intra version differs
    assert np.abs(_dense_dca(q, k, v, 1e4, 10**6, 10**6, scale) - ref).max() > 1e-2


def test_dca_single_chunk_is_plain_rope_attention():
    rng = np.random.default_rng(1)
    B, H, KVH, S, Dh, C, gs = 1, 2, 1, 24, 16, 8, 4
    q = rng.standard_normal((B, H, S, Dh))
    k = rng.standard_normal((B, KVH, S, Dh))
    v = rng.standard_normal((B, KVH, S, Dh))
    scale = Dh ** -0.5
    got = _routed_dca(q, k, v, 1e4, 64, 80, scale, C, gs, 8)
    pos = np.arange(S)
    qr, kr = _rope_at(q, pos, 1e4), _rope_at(k, pos, 1e4)
    s = np.einsum("bhid,bjd->bhij", qr, kr[:, 0]) * scale
    s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("bhij,bjd->bhid", p, v[:, 0])
    assert np.abs(got - ref).max() < 1e-5
