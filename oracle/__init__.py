"""CPU oracle for the HGA routed-attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package.  The product path (``hierarchicalglobalattention_amd``) never does.

``hga_oracle.c`` is a single-threaded C restatement of the reference's prefill path
(``ExistingModelFineTuning/KvRouter/vectorized.py:189-492`` + ``chunk_router.py:139-162``) and
decode path (``chunk_router.py:187-407``), the Dual Chunk Attention decode
(``qwen_routed_attention.py:244-283``) and the gradient of the prefill attention (what autograd
computes through ``HierarchicalGlobalAttentionRouted.py:137-177``), with the canonical score/tie
rules documented at the top of that file.  This module wraps it for numpy float32 arrays (bf16 tensors are passed as
float32 arrays holding bf16-representable values) and restates the small host-side formulas
(cutoff pair, window ranges) independently of the product package.

``mirror.py`` (same package) is a separate op-by-op torch restatement used as the CPU baseline.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

DT_F32, DT_BF16 = 0, 1


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_score.restype = ctypes.c_float
        _lib.orc_bf16_round.restype = ctypes.c_float
        _lib.orc_bf16_round.argtypes = [ctypes.c_float]
    return _lib


def _f(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _i(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


# ----------------------------------------------------------------------------------------------
# host-side formulas, restated from the reference
# ----------------------------------------------------------------------------------------------
def cutoff_pair(theta: float, chunk_size: int, head_dim: int, threshold: float = 0.5,
                override=None) -> int:
    """``_mixed_cutoff_pair`` (vectorized.py:146-155; chunk_router.py:717-726)."""
    if override is not None:
        return int(override)
    half = head_dim // 2
    cut = 0
    for i in range(half):
        if max(1, chunk_size - 1) * (1.0 / (theta ** (i / half))) > threshold:
            cut = i + 1
    return cut


def group_scale(group_size: int) -> float:
    """``RouterConfig.group_kv_scale`` (chunk_router.py:87-90) as the fp32 factor torch uses."""
    return float(np.float32(1.0 / (group_size + math.sqrt(group_size))))


def attn_scale(head_dim: int) -> float:
    """``RouterConfig.scale`` (chunk_router.py:83-85) as the fp32 factor torch uses."""
    return float(np.float32(head_dim ** -0.5))


def windows(n: int, keep_first: int, keep_last: int):
    """(f_hi, l_lo) for a query chunk / decode step with ``n`` earlier chunks
    (vectorized.py:246-253; chunk_placement_policy.py:27-38)."""
    f_hi = min(keep_first, n) if keep_first > 0 else 0
    l_lo = min(max(keep_first, n - keep_last), n) if keep_last > 0 else n
    return f_hi, l_lo


def sizes(S, C, gs, topk_chunks, topk_groups):
    N = (S + C - 1) // C
    M = C // gs
    Kc = min(topk_chunks, N) if topk_chunks > 0 else 0
    T = Kc * M
    Kg = min(topk_groups, T) if topk_groups > 0 else 0
    return N, M, Kc, Kg


# ----------------------------------------------------------------------------------------------
# kernels
# ----------------------------------------------------------------------------------------------
def rope(x, cos, sin, dt):
    """x [B,X,S,Dh]; cos/sin [S,Dh] or [B,S,Dh] (fp32)."""
    x, px = _f(x)
    B, X, S, Dh = x.shape
    cos, pc = _f(cos)
    sin, ps = _f(sin)
    bstride = 0 if cos.ndim == 2 else S * Dh
    out = np.empty_like(x)
    lib().orc_rope(px, _f(out)[1], pc, ps, B, X, S, Dh, ctypes.c_long(bstride), dt)
    return out


def summarize(k_raw, k_rope, cos_tab, sin_tab, C, gs, cutoff, gscale, dt, pos0=0):
    """Mixed-RoPE chunk/group key summaries -> (chunk_k [B,KVH,N,Dh], group_k [B,KVH,N,M,Dh])."""
    k_raw, pr = _f(k_raw)
    k_rope, pp = _f(k_rope)
    cos_tab, pc = _f(cos_tab)
    sin_tab, ps = _f(sin_tab)
    B, KVH, S, Dh = k_raw.shape
    N, M = (S + C - 1) // C, C // gs
    ck = np.zeros((B, KVH, N, Dh), np.float32)
    gk = np.zeros((B, KVH, N, M, Dh), np.float32)
    lib().orc_summarize(pr, pp, pc, ps, ctypes.c_long(pos0), B, KVH, S, Dh, C, gs, cutoff,
                        ctypes.c_float(gscale), dt, _f(ck)[1], _f(gk)[1])
    return ck, gk


def route_prefill(q, chunk_k, group_k, S, C, gs, keep_first, keep_last, topk_chunks,
                  topk_groups, scale):
    q, pq = _f(q)
    chunk_k, pc = _f(chunk_k)
    group_k, pg = _f(group_k)
    B, H, _, Dh = q.shape
    KVH = chunk_k.shape[1]
    N, M, Kc, Kg = sizes(S, C, gs, topk_chunks, topk_groups)
    Kcw, Kgw = max(Kc, 1), max(Kg, 1)
    r = dict(sel_chunk=np.empty((B, H, N, Kcw), np.int32), sel_thr=np.empty((B, H, N, Kcw), np.int32),
             n_sel=np.empty((B, H, N), np.int32), open_grp=np.empty((B, H, N, Kgw), np.int32),
             open_thr=np.empty((B, H, N, Kgw), np.int32), n_open=np.empty((B, H, N), np.int32))
    lib().orc_route_prefill(pq, pc, pg, B, H, KVH, S, Dh, C, gs, keep_first, keep_last,
                            topk_chunks, topk_groups, ctypes.c_float(scale), Kcw, Kgw,
                            _i(r["sel_chunk"]), _i(r["sel_thr"]), _i(r["n_sel"]),
                            _i(r["open_grp"]), _i(r["open_thr"]), _i(r["n_open"]))
    return r


def attend_prefill(q, k, v, C, gs, keep_first, keep_last, open_grp, open_thr, scale, dt,
                   chunks=None):
    """Routed prefill attention; with ``chunks`` (query chunk ids) only those chunks' rows are
    computed and the other rows of the result are NaN."""
    q, pq = _f(q)
    k, pk = _f(k)
    v, pv = _f(v)
    B, H, S, Dh = q.shape
    KVH = k.shape[1]
    og = np.ascontiguousarray(open_grp, np.int32)
    ot = np.ascontiguousarray(open_thr, np.int32)
    out = np.full_like(q, np.nan)
    if chunks is None:
        lib().orc_attend_prefill(pq, pk, pv, B, H, KVH, S, Dh, C, gs, keep_first, keep_last,
                                 _i(og), _i(ot), og.shape[-1], ctypes.c_float(scale), dt,
                                 _f(out)[1])
    else:
        ch = np.ascontiguousarray(chunks, np.int32)
        lib().orc_attend_prefill_chunks(pq, pk, pv, B, H, KVH, S, Dh, C, gs, keep_first,
                                        keep_last, _i(og), _i(ot), og.shape[-1],
                                        ctypes.c_float(scale), dt, _i(ch), len(ch), _f(out)[1])
    return out


def route_prefill_heads(q, chunk_k, group_k, S, C, gs, keep_first, keep_last, topk_chunks,
                        topk_groups, scale, threads=None):
    """route_prefill with one oracle call per query head on a thread pool (the C oracle releases
    the GIL); results are identical to one call over all heads."""
    from concurrent.futures import ThreadPoolExecutor
    q = np.ascontiguousarray(q, np.float32)
    B, H = q.shape[:2]
    KVH = chunk_k.shape[1]
    rep = H // KVH
    n = threads or min(H, len(os.sched_getaffinity(0)))

    def one(h):
        kv = h // rep
        return route_prefill(q[:, h:h + 1], chunk_k[:, kv:kv + 1], group_k[:, kv:kv + 1], S, C,
                             gs, keep_first, keep_last, topk_chunks, topk_groups, scale)

    with ThreadPoolExecutor(n) as ex:
        parts = list(ex.map(one, range(H)))
    return {key: np.concatenate([p[key] for p in parts], axis=1) for key in parts[0]}


def attend_prefill_bwd(q, k, v, dout, C, gs, keep_first, keep_last, open_grp, open_thr, scale):
    """Exact (double) gradients (dq, dk, dv) of attend_prefill's attention for upstream dout."""
    q, pq = _f(q)
    k, pk = _f(k)
    v, pv = _f(v)
    dout, pg = _f(dout)
    B, H, S, Dh = q.shape
    KVH = k.shape[1]
    og = np.ascontiguousarray(open_grp, np.int32)
    ot = np.ascontiguousarray(open_thr, np.int32)
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib().orc_attend_prefill_bwd(pq, pk, pv, pg, B, H, KVH, S, Dh, C, gs, keep_first, keep_last,
                                 _i(og), _i(ot), og.shape[-1], ctypes.c_float(scale),
                                 _f(dq)[1], _f(dk)[1], _f(dv)[1])
    return dq, dk, dv


def route_decode(q, chunk_k, group_k, n_closed, keep_first, keep_last, topk_chunks,
                 topk_groups, scale):
    """q [B,H,L,Dh]; chunk_k [B,KVH,cap,Dh]; group_k [B,KVH,cap,M,Dh] (store layout)."""
    q, pq = _f(q)
    chunk_k, pc = _f(chunk_k)
    group_k, pg = _f(group_k)
    B, H, L, Dh = q.shape
    KVH, cap, M = group_k.shape[1], group_k.shape[2], group_k.shape[3]
    f_hi, l_lo = windows(n_closed, keep_first, keep_last)
    nmid = max(0, l_lo - f_hi)
    Kc = min(topk_chunks, nmid) if (topk_chunks > 0 and nmid > 0) else 0
    Kg = min(topk_groups, Kc * M) if topk_groups > 0 else 0
    Kcw, Kgw = max(Kc, 1), max(Kg, 1)
    r = dict(mid=np.empty((B, H, Kcw), np.int32), mid_thr=np.empty((B, H, Kcw), np.int32),
             n_mid=np.empty((B, H), np.int32), open_grp=np.empty((B, H, Kgw), np.int32),
             open_thr=np.empty((B, H, Kgw), np.int32), n_open=np.empty((B, H), np.int32))
    lib().orc_route_decode(pq, pc, pg, ctypes.c_long(cap), B, H, KVH, L, Dh, M, n_closed,
                           keep_first, keep_last, topk_chunks, topk_groups, ctypes.c_float(scale),
                           Kcw, Kgw, _i(r["mid"]), _i(r["mid_thr"]), _i(r["n_mid"]),
                           _i(r["open_grp"]), _i(r["open_thr"]), _i(r["n_open"]))
    return r


def attend_decode(q, k_hist, v_hist, C, gs, keep_first, keep_last, n_closed, start_pos,
                  open_grp, open_thr, scale, dt):
    """q [B,H,L,Dh]; k_hist/v_hist [B,KVH,T,Dh] token history including the active chunk."""
    q, pq = _f(q)
    k_hist, pk = _f(k_hist)
    v_hist, pv = _f(v_hist)
    B, H, L, Dh = q.shape
    KVH, T = k_hist.shape[1], k_hist.shape[2]
    og = np.ascontiguousarray(open_grp, np.int32)
    ot = np.ascontiguousarray(open_thr, np.int32)
    out = np.empty_like(q)
    lib().orc_attend_decode(pq, pk, pv, ctypes.c_long(T), B, H, KVH, L, Dh, C, gs, keep_first,
                            keep_last, n_closed, ctypes.c_long(start_pos), _i(og), _i(ot),
                            og.shape[-1], ctypes.c_float(scale), dt, _f(out)[1])
    return out


def attend_decode_dca(q_intra, q_succ, q_inter, k_hist, v_hist, C, gs, keep_first, keep_last,
                      n_closed, start_pos, open_grp, open_thr, scale, dt, dca_chunk):
    """Dual Chunk Attention decode (qwen_routed_attention.py:253-283): the three fp32 RoPE'd
    query versions [B,H,L,Dh]; k_hist holds the DCA-roped keys by absolute position."""
    q1, p1 = _f(q_intra)
    q2, p2 = _f(q_succ)
    q3, p3 = _f(q_inter)
    k_hist, pk = _f(k_hist)
    v_hist, pv = _f(v_hist)
    B, H, L, Dh = q1.shape
    KVH, T = k_hist.shape[1], k_hist.shape[2]
    og = np.ascontiguousarray(open_grp, np.int32)
    ot = np.ascontiguousarray(open_thr, np.int32)
    out = np.empty_like(q1)
    lib().orc_attend_decode_dca(p1, p2, p3, pk, pv, ctypes.c_long(T), B, H, KVH, L, Dh, C, gs,
                                keep_first, keep_last, n_closed, ctypes.c_long(start_pos),
                                _i(og), _i(ot), og.shape[-1], ctypes.c_float(scale), dt,
                                dca_chunk, _f(out)[1])
    return out


def prefill(q, k_rope, k_raw, v, cos_tab, sin_tab, *, C, gs, keep_first, keep_last,
            topk_chunks, topk_groups, theta, dt):
    """The whole vectorized prefill path for one block at position 0: summaries (with the
    ``cos_tab``/``sin_tab`` rows the reference's dtype table holds), routing, attention.
    Returns (out, routing dict, chunk_k, group_k)."""
    B, H, S, Dh = q.shape
    cut = cutoff_pair(theta, C, Dh)
    ck, gk = summarize(k_raw, k_rope, cos_tab, sin_tab, C, gs, cut, group_scale(gs), dt)
    r = route_prefill(q, ck, gk, S, C, gs, keep_first, keep_last, topk_chunks, topk_groups,
                      attn_scale(Dh))
    out = attend_prefill(q, k_rope, v, C, gs, keep_first, keep_last, r["open_grp"],
                         r["open_thr"], attn_scale(Dh), dt)
    return out, r, ck, gk
