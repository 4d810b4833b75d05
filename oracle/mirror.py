"""Op-by-op torch CPU restatement of the reference prefill path -- TEST INFRASTRUCTURE ONLY
(the CPU baseline of bench.py and a cross-check in tests/).

It follows the eager sequence of ExistingModelFineTuning/KvRouter/vectorized.py:189-492 and
RoutedKV.attend (chunk_router.py:149-158): summaries by masked sums at query-head granularity,
einsum scores, masked_fill(-1e4), per-row torch.topk, scatter_reduce(amax) pooling, pooled topk,
forced previous chunk by argmin replacement, cumsum visibility, stage-2 group routing, gathers of
the opened groups and windows into materialised token K/V + masks, and fp32 einsum/softmax
attention -- the same torch operations and dtypes, so its cost is the reference's CPU cost.
Query chunks are independent given the summaries, so the work can be run on a slab of query
chunks [n_lo, n_hi) with identical results for those chunks.
"""
from __future__ import annotations

import math
import time

import torch

NEG = -1.0e4


def _rot(x, cos, sin):
    h = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., h:], x[..., :h]), dim=-1) * sin


def _cutoff(theta, C, Dh, threshold=0.5):
    half = Dh // 2
    cut = 0
    for i in range(half):
        if max(1, C - 1) * (1.0 / (theta ** (i / half))) > threshold:
            cut = i + 1
    return cut


class Geometry:
    def __init__(self, S, C, gs, kf, kl):
        self.S, self.C, self.gs, self.M = S, C, gs, C // gs
        self.N = (S + C - 1) // C
        self.kf, self.kl = max(0, kf), max(0, kl)
        N, M = self.N, self.M
        self.valid = (torch.arange(N * C) < S).view(N, C)
        self.chunk_len = self.valid.sum(1)
        self.group_len = self.valid.view(N, M, gs).sum(-1)
        self.valid_groups = self.valid.view(N, M, gs).any(-1)
        qn = torch.arange(N)
        self.f_hi = torch.clamp(qn, max=self.kf) if self.kf > 0 else torch.zeros_like(qn)
        self.l_lo = torch.minimum(torch.clamp(qn - self.kl, min=self.kf), qn) if self.kl > 0 else qn
        cand = torch.arange(N)
        self.pool = (cand.view(1, N) < qn.view(N, 1)) & (cand.view(1, N) >= self.f_hi.view(N, 1)) \
            & (cand.view(1, N) < self.l_lo.view(N, 1))


def summaries(k_raw, k_rope, cos, sin, geo: Geometry, theta, gscale):
    """chunk_k [B,X,N,Dh], group_k [B,X,N,M,Dh] in the activation dtype."""
    B, X, S, Dh = k_raw.shape
    N, C, gs, M = geo.N, geo.C, geo.gs, geo.M
    dt = k_raw.dtype
    pad = N * C - S
    z = lambda t: torch.cat([t, t.new_zeros(B, X, pad, Dh)], 2) if pad else t
    kr, kp = z(k_raw).view(B, X, N, C, Dh), z(k_rope).view(B, X, N, C, Dh)
    cmask = geo.valid.view(1, 1, N, C, 1).to(dt)
    gmask = geo.valid.view(1, 1, N, M, gs, 1).to(dt)
    cut = _cutoff(theta, C, Dh)
    sel = torch.cat([torch.arange(Dh // 2) < cut] * 2).view(*([1] * 4), Dh)
    start = torch.arange(N) * C
    c_mid = (start + (geo.chunk_len.clamp_min(1) - 1) // 2).clamp_max(S - 1)
    g_start = start[:, None] + torch.arange(M)[None, :] * gs
    g_mid = (g_start + (geo.group_len.clamp_min(1) - 1) // 2).clamp_max(S - 1)

    def one(raw, rope, mask, dim, anchor, scale):
        raw_sum = (raw * mask).sum(dim=dim) * scale
        ac = cos[:, :, anchor.reshape(-1)].reshape(1, 1, *anchor.shape, Dh)
        asn = sin[:, :, anchor.reshape(-1)].reshape(1, 1, *anchor.shape, Dh)
        end = _rot(raw_sum.float(), ac, asn).to(raw_sum.dtype)
        tok = (rope * mask).sum(dim=dim) * scale
        s = sel.view(*([1] * (tok.ndim - 1)), Dh)
        return torch.where(s, tok, end)

    ck = one(kr, kp, cmask, 3, c_mid, 1.0)
    gk = one(kr.view(B, X, N, M, gs, Dh), kp.view(B, X, N, M, gs, Dh), gmask, 4, g_mid, gscale)
    return ck, gk


def _topk_all(x, k, sorted_=True):
    n = x.shape[-1]
    if k >= n:
        return x, torch.arange(n).expand(*x.shape[:-1], n)
    return torch.topk(x, k, dim=-1, sorted=sorted_)


def route_attend_slab(q, k_rope, v, ck, gk, geo: Geometry, tc, tg, scale, n_lo, n_hi):
    """Attention output [B,H,(n_hi-n_lo)*C,Dh] (rows past S are padding) for query chunks
    [n_lo, n_hi); q/k_rope/v/ck/gk at query-head granularity (repeated KV heads)."""
    B, H, S, Dh = q.shape
    N, C, gs, M = geo.N, geo.C, geo.gs, geo.M
    dt = q.dtype
    ns = n_hi - n_lo
    pad = N * C - S
    z = lambda t: torch.cat([t, t.new_zeros(B, H, pad, Dh)], 2) if pad else t
    qc = z(q).view(B, H, N, C, Dh)[:, :, n_lo:n_hi]
    kc = z(k_rope).view(B, H, N, C, Dh)
    vc = z(v).view(B, H, N, C, Dh)
    qvalid = geo.valid[n_lo:n_hi].view(1, 1, ns, C, 1)
    pool = geo.pool[n_lo:n_hi]
    f_hi, l_lo = geo.f_hi[n_lo:n_hi], geo.l_lo[n_lo:n_hi]
    qidx = torch.arange(n_lo, n_hi)
    Kc = min(tc, N) if tc > 0 else 0
    bh = torch.arange(B * H).view(B * H, 1)
    tok_k, tok_v, tok_m = [], [], []
    causal = torch.arange(C).view(1, C) <= torch.arange(C).view(C, 1)
    tok_k.append(kc[:, :, n_lo:n_hi]); tok_v.append(vc[:, :, n_lo:n_hi])
    tok_m.append((causal.view(1, 1, 1, C, C) & geo.valid[n_lo:n_hi].view(1, 1, ns, 1, C)
                  & qvalid).expand(B, H, ns, C, C))
    if Kc > 0:
        with torch.no_grad():
            sc = torch.einsum("bhncd,bhmd->bhncm", qc, ck) * scale
            sc = sc.masked_fill(~(pool.view(1, 1, ns, 1, N) & qvalid), NEG)
            rs, ri = _topk_all(sc, Kc)
            flat = B * H * ns
            pooled = torch.full((flat, N), NEG, dtype=sc.dtype)
            if ri.shape[-1] == N:
                pooled = rs.max(dim=-2).values.reshape(flat, N)
            else:
                pooled.scatter_reduce_(1, ri.reshape(flat, -1), rs.reshape(flat, -1), "amax",
                                       include_self=True)
            pooled = pooled.view(B, H, ns, N)
        tsc, tix = _topk_all(pooled, Kc, sorted_=False)
        qi = qidx.view(1, 1, ns, 1)
        prev = (qi - 1).clamp_min(0).expand(B, H, ns, 1)
        has_prev = (qi > 0).expand(B, H, ns, 1)
        prev_in = (prev >= f_hi.view(1, 1, ns, 1)) & (prev < l_lo.view(1, 1, ns, 1))
        missing = has_prev & prev_in & ~(tix == prev).any(-1, keepdim=True)
        at = tsc.argmin(-1, keepdim=True)
        tix = tix.scatter(-1, at, torch.where(missing, prev, tix.gather(-1, at)))
        vprev = pool.view(1, 1, ns, N).expand(B, H, ns, N).gather(-1, tix)
        req = (ri.unsqueeze(-1) == tix.unsqueeze(-2).unsqueeze(-3)).any(-2) & vprev.unsqueeze(3)
        cvis = (torch.cumsum(req.to(torch.int32), 3) > 0) & vprev.unsqueeze(3) & qvalid
        pslot = (tix == prev).unsqueeze(3)
        cvis = (cvis | (pslot & has_prev.unsqueeze(3) & qvalid)) & vprev.unsqueeze(3)
        T2 = Kc * M
        cg = gk.reshape(B * H, N, M, Dh)[bh, tix.reshape(B * H, -1)].reshape(B, H, ns, T2, Dh)
        cgv = (geo.valid_groups.view(1, 1, N, M).expand(B, H, N, M).reshape(B * H, N, M)
               [bh, tix.reshape(B * H, -1)].reshape(B, H, ns, Kc, M) & vprev.unsqueeze(-1))
        cgv = cgv.reshape(B, H, ns, T2)
        gmask = cvis.unsqueeze(-1).expand(B, H, ns, C, Kc, M).reshape(B, H, ns, C, T2) \
            & cgv.unsqueeze(3) & qvalid
        Kg = min(tg, T2) if tg > 0 else 0
        Kgr = min(tg // 2, T2) if tg > 0 else 0
        if Kg > 0 and Kgr > 0:
            with torch.no_grad():
                s2 = torch.einsum("bhncd,bhnrd->bhncr", qc, cg) * scale
                s2 = s2.masked_fill(~gmask, NEG)
                gs_, gi = _topk_all(s2, Kgr)
                flat = B * H * ns
                if gi.shape[-1] == T2:
                    p2 = gs_.max(dim=-2).values
                else:
                    p2 = torch.full((flat, T2), NEG, dtype=s2.dtype)
                    p2.scatter_reduce_(1, gi.reshape(flat, -1), gs_.reshape(flat, -1), "amax",
                                       include_self=True)
                    p2 = p2.view(B, H, ns, T2)
            _, tg_ = _topk_all(p2, Kg, sorted_=False)
            tgv = cgv.gather(-1, tg_)
            parent = tg_ // M
            pvis = cvis.gather(-1, parent.unsqueeze(3).expand(B, H, ns, C, Kg))
            greq = (gi.unsqueeze(-1) == tg_.unsqueeze(-2).unsqueeze(-3)).any(-2) \
                & tgv.unsqueeze(3) & pvis
            gvis = (torch.cumsum(greq.to(torch.int32), 3) > 0) & tgv.unsqueeze(3) & pvis & qvalid
            src_c = tix.gather(-1, parent)
            src_g = tg_ - parent * M
            kg = kc.reshape(B * H, N, M, gs, Dh)
            vg = vc.reshape(B * H, N, M, gs, Dh)
            fc, fg = src_c.reshape(B * H, -1), src_g.reshape(B * H, -1)
            tok_k.append(kg[bh, fc, fg].reshape(B, H, ns, Kg * gs, Dh))
            tok_v.append(vg[bh, fc, fg].reshape(B, H, ns, Kg * gs, Dh))
            om = gvis.unsqueeze(-1).expand(B, H, ns, C, Kg, gs).reshape(B, H, ns, C, Kg * gs)
            tok_m.append(om & qvalid)
    for kind in ("last", "first"):
        w = min(geo.kl if kind == "last" else geo.kf, N)
        if w <= 0:
            continue
        j = torch.arange(w)
        if kind == "last":
            cid = l_lo.view(ns, 1) + j.view(1, w)
            ok = cid < qidx.view(ns, 1)
        else:
            ok = j.view(1, w) < f_hi.view(ns, 1)
            cid = j.view(1, w).expand(ns, w)
        cid = torch.where(ok, cid, torch.zeros_like(cid))
        idx = cid.reshape(1, ns * w).expand(B * H, ns * w)
        tok_k.append(kc.reshape(B * H, N, C, Dh)[bh, idx].reshape(B, H, ns, w * C, Dh))
        tok_v.append(vc.reshape(B * H, N, C, Dh)[bh, idx].reshape(B, H, ns, w * C, Dh))
        src_ok = geo.valid[cid.reshape(-1)].view(1, 1, ns, 1, w, C)
        tok_m.append((ok.view(1, 1, ns, 1, w, 1) & src_ok & qvalid.view(1, 1, ns, C, 1, 1))
                     .expand(B, H, ns, C, w, C).reshape(B, H, ns, C, w * C))
    tk = torch.cat(tok_k, 3)
    tv = torch.cat(tok_v, 3)
    tm = torch.cat(tok_m, -1)
    s = torch.einsum("bhncd,bhnrd->bhncr", qc.float(), tk.float()) * scale
    s = s.masked_fill(~tm, NEG)
    p = torch.softmax(s, dim=-1)
    o = torch.einsum("bhncr,bhnrd->bhncd", p, tv.float())
    return o.reshape(B, H, ns * C, Dh).to(dt)


def prefill(q, k_rope, k_raw, v, cos, sin, *, C, gs, keep_first, keep_last, topk_chunks,
            topk_groups, theta, slab=None):
    """Whole block (KV-head inputs are repeated to query heads as the reference does)."""
    B, H, S, Dh = q.shape
    rep = H // k_rope.shape[1]
    r = lambda t: t.repeat_interleave(rep, dim=1) if rep > 1 else t
    kp, kr, vv = r(k_rope), r(k_raw), r(v)
    geo = Geometry(S, C, gs, keep_first, keep_last)
    ck, gk = summaries(kr, kp, cos, sin, geo, theta, 1.0 / (gs + math.sqrt(gs)))
    scale = Dh ** -0.5
    slab = slab or geo.N
    outs = [route_attend_slab(q, kp, vv, ck, gk, geo, topk_chunks, topk_groups, scale, a,
                              min(a + slab, geo.N)) for a in range(0, geo.N, slab)]
    return torch.cat(outs, 2)[:, :, :S]


def bench_c3_slab(cfg: dict, budget_s: float = 15.0, seed: int = 0) -> dict:
    """Times the mirror on the bench workload: summaries for the whole block, then slabs of 32
    consecutive query chunks (routed and attended together, as the reference's vectorized path
    batches chunks) in a strided order over the sequence until the budget is used; the layer
    time is summaries + the slabs' time scaled to all N chunks (exact when every slab ran)."""
    B, S, H, KVH, Dh = cfg["B"], cfg["S"], cfg["H"], cfg["KVH"], cfg["Dh"]
    C, gs = cfg["C"], cfg["gs"]
    g = torch.Generator().manual_seed(seed)
    rms = lambda x: x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    bf = torch.bfloat16
    q_raw = rms(torch.randn(B, H, S, Dh, generator=g)).to(bf)
    k_raw = rms(torch.randn(B, KVH, S, Dh, generator=g)).to(bf)
    v = torch.randn(B, KVH, S, Dh, generator=g).to(bf)
    half = Dh // 2
    inv = 1.0 / (cfg["theta"] ** (torch.arange(0, half, dtype=torch.float32) / half))
    e = torch.einsum("i,j->ij", torch.arange(S, dtype=torch.float32), inv)
    e = torch.cat((e, e), -1)
    cos, sin = e.cos()[None, None], e.sin()[None, None]
    t0 = time.perf_counter()
    q = _rot(q_raw.float(), cos, sin).to(bf)
    k_rope = _rot(k_raw.float(), cos, sin).to(bf)
    rep = H // KVH
    kp, kr, vv = (t.repeat_interleave(rep, 1) for t in (k_rope, k_raw, v))
    geo = Geometry(S, C, gs, cfg["kf"], cfg["kl"])
    ck, gk = summaries(kr, kp, cos.to(bf), sin.to(bf), geo, cfg["theta"],
                       1.0 / (gs + math.sqrt(gs)))
    t_sum = time.perf_counter() - t0
    scale = Dh ** -0.5
    slab = 32
    route_attend_slab(q, kp, vv, ck, gk, geo, cfg["tc"], cfg["tg"], scale, geo.N // 2,
                      geo.N // 2 + 1)   # warm-up
    starts = list(range(0, geo.N, slab))
    # every slab, in a strided order so that a budget cut still samples the whole sequence
    stride = next(x for x in (5, 7, 11, 13, 1) if math.gcd(x, len(starts)) == 1)
    order = [starts[(i * stride) % len(starts)] for i in range(len(starts))]
    times, done = [], 0
    deadline = time.perf_counter() + budget_s
    for n0 in order:
        if times and time.perf_counter() > deadline:
            break
        n1 = min(n0 + slab, geo.N)
        a = time.perf_counter()
        route_attend_slab(q, kp, vv, ck, gk, geo, cfg["tc"], cfg["tg"], scale, n0, n1)
        times.append(time.perf_counter() - a)
        done += n1 - n0
    layer_s = t_sum + geo.N * (sum(times) / done)
    return dict(tokens_per_s=B * S / layer_s, layer_s=layer_s,
                sample=(f"RoPE+summaries for all {geo.N} chunks ({t_sum:.2f} s) + {done} of "
                        f"{geo.N} query chunks in {len(times)} slabs of {slab} spread over the "
                        f"sequence, scaled to the full layer; bf16, torch {torch.__version__}, "
                        f"{torch.get_num_threads()} threads"))
