"""Shared test helpers: golden-fixture loading, the seeded input recipe, and an oracle-driven
CPU model of the whole module (projections in torch fp32 on the CPU, routed attention in the
C oracle).  Test infrastructure only."""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_case(name):
    d = dict(np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False))
    meta = json.loads(str(d.pop("meta")))
    return meta, d


def rotary_table(seq_len, head_dim, theta, device="cpu"):
    """cos/sin [seq_len, Dh] fp32, the rotate-half table of
    HierarchicalGlobalAttentionRouted._get_rotary (HierarchicalGlobalAttentionRouted.py:209-217)."""
    half = head_dim // 2
    inv = 1.0 / (theta ** (torch.arange(0, half, device=device, dtype=torch.float32) / half))
    t = torch.arange(seq_len, device=device, dtype=torch.float32)
    f = torch.einsum("i,j->ij", t, inv)
    e = torch.cat((f, f), dim=-1)
    return e.cos(), e.sin()


def rope_torch(x, cos, sin):
    half = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., half:], x[..., :half]), dim=-1) * sin


def make_inputs(seed, B, H, KVH, S, Dh, dtype, scale_inputs=None, qk_rmsnorm=False):
    """Same recipe as tests/golden/make_golden.py:make_inputs."""
    g = torch.Generator().manual_seed(seed)
    q_raw = torch.randn(B, H, S, Dh, generator=g)
    k_raw = torch.randn(B, KVH, S, Dh, generator=g)
    v = torch.randn(B, KVH, S, Dh, generator=g)
    if scale_inputs is not None:
        q_raw, k_raw, v = q_raw * scale_inputs, k_raw * scale_inputs, v * scale_inputs
    if qk_rmsnorm:
        q_raw = q_raw * torch.rsqrt(q_raw.pow(2).mean(-1, keepdim=True) + 1e-6)
        k_raw = k_raw * torch.rsqrt(k_raw.pow(2).mean(-1, keepdim=True) + 1e-6)
    return q_raw.to(dtype), k_raw.to(dtype), v.to(dtype)


def tdtype(name):
    return {"float32": torch.float32, "bfloat16": torch.bfloat16}[name]


def prefill_case_inputs(meta, arrs):
    """(q, k_rope, k_raw, v) float32 numpy + cos/sin tables for a prefill fixture; inputs are
    regenerated from the recipe when the fixture does not store them, and checked against the
    stored hash."""
    dt = tdtype(meta["dtype"])
    cos = torch.from_numpy(arrs["cos"])
    sin = torch.from_numpy(arrs["sin"])
    if "q" in arrs:
        q, k_rope, k_raw, v = (arrs[n] for n in ("q", "k_rope", "k_raw", "v"))
    else:
        q_raw, k_raw_t, v_t = make_inputs(meta["seed"], meta["B"], meta["H"], meta["KVH"],
                                          meta["S"], meta["Dh"], dt, meta["scale_inputs"],
                                          meta["qk_rmsnorm"])
        q_t = rope_torch(q_raw.float(), cos, sin).to(dt)
        kr_t = rope_torch(k_raw_t.float(), cos, sin).to(dt)
        q, k_rope, k_raw, v = (t.float().numpy() for t in (q_t, kr_t, k_raw_t, v_t))
    h = hashlib.sha256()
    for a in (q, k_raw, v):
        h.update(np.ascontiguousarray(a, np.float32).tobytes())
    assert h.hexdigest() == bytes(arrs["inputs_sha"]).decode(), "input recipe drifted"
    return q, k_rope, k_raw, v, cos.numpy(), sin.numpy()


def dt_code(name):
    return oracle.DT_BF16 if name == "bfloat16" else oracle.DT_F32


def dtype_table(tab, name):
    """The reference hands the vectorized path ``cos[:1].to(x.dtype)`` (Routed.py:168)."""
    return oracle.bf16_round(tab) if name == "bfloat16" else np.asarray(tab, np.float32)


def oracle_prefill_case(meta, arrs):
    q, k_rope, k_raw, v, cos, sin = prefill_case_inputs(meta, arrs)
    dtn = meta["dtype"]
    return oracle.prefill(q, k_rope, k_raw, v, dtype_table(cos, dtn), dtype_table(sin, dtn),
                          C=meta["C"], gs=meta["gs"], keep_first=meta["keep_first"],
                          keep_last=meta["keep_last"], topk_chunks=meta["topk_chunks"],
                          topk_groups=meta["topk_groups"], theta=meta["theta"],
                          dt=dt_code(dtn))


# ----------------------------------------------------------------------------------------------
# whole-module CPU model driven by the oracle
# ----------------------------------------------------------------------------------------------
class OracleModule:
    """HierarchicalGlobalAttentionRouted.forward (HierarchicalGlobalAttentionRouted.py:137-177)
    as the oracle computes it: fp32 torch projections, optional per-head RMSNorm, RoPE, the
    vectorized prefill for a fresh multi-chunk block, the decode path for blocks inside one
    chunk, and a VRAM-store model (record + summaries at KV-head granularity computed with the
    fp32 table, chunk_router.py:552-598, 631-657)."""

    def __init__(self, meta, arrs):
        self.m = meta
        self.w = {k[2:]: torch.from_numpy(v) for k, v in arrs.items() if k.startswith("w_")}
        self.H, self.KVH, self.Dh = meta["H"], meta["KVH"], meta["Dh"]
        self.C, self.gs = meta["C"], meta["gs"]
        self.M = self.C // self.gs
        self.theta = meta["theta"]
        self.reset()

    def reset(self):
        self.k_hist = None     # [B,KVH,T,Dh] rope keys
        self.kraw_hist = None
        self.v_hist = None
        self.n_closed = 0
        self.ck = None         # store summaries [B,KVH,n_closed,Dh]
        self.gk = None
        self.decisions = []

    def _lin(self, x, name):
        y = x @ self.w[name + ".weight"].t()
        if name + ".bias" in self.w:
            y = y + self.w[name + ".bias"]
        return y

    def _norm(self, x, name):
        if name + ".weight" not in self.w:
            return x
        xf = x.float()
        return (self.w[name + ".weight"].float() * xf *
                torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype)

    def _close_summaries(self, k_rope, k_raw, pos0, cos, sin):
        cut = oracle.cutoff_pair(self.theta, self.C, self.Dh)
        return oracle.summarize(k_raw, k_rope, cos.numpy(), sin.numpy(), self.C, self.gs, cut,
                                oracle.group_scale(self.gs), oracle.DT_F32, pos0=pos0)

    def _decode_segment(self, q, k_rope, k_raw, v, start_pos, cos_f, sin_f):
        """Rows inside one chunk: route against the closed chunks, attend, then close the chunk
        when it is full (chunk_router.py:279-407, 631-657)."""
        B, H = q.shape[:2]
        C = self.C
        kf, kl = self.m["keep_first"], self.m["keep_last"]
        tc, tg = self.m["topk_chunks"], self.m["topk_groups"]
        scale = oracle.attn_scale(self.Dh)
        cat = (lambda a, b: b) if self.k_hist is None else (
            lambda a, b: np.concatenate([a, b], axis=2))
        self.k_hist = cat(self.k_hist, k_rope)
        self.kraw_hist = cat(self.kraw_hist, k_raw)
        self.v_hist = cat(self.v_hist, v)
        r = None
        if self.n_closed > 0:
            r = oracle.route_decode(q, self.ck, self.gk, self.n_closed, kf, kl, tc, tg, scale)
            self.decisions.append((self.n_closed, r))
        og = r["open_grp"] if r is not None else np.full((B, H, 1), -1, np.int32)
        ot = r["open_thr"] if r is not None else np.full((B, H, 1), -1, np.int32)
        out = oracle.attend_decode(q, self.k_hist, self.v_hist, C, self.gs, kf, kl,
                                   self.n_closed, start_pos, og, ot, scale, oracle.DT_F32)
        T = self.k_hist.shape[2]
        if T == (self.n_closed + 1) * C:       # the segment filled the active chunk
            lo = self.n_closed * C
            ck, gk = self._close_summaries(self.k_hist[:, :, lo:], self.kraw_hist[:, :, lo:],
                                           lo, cos_f, sin_f)
            self.ck = ck if self.ck is None else np.concatenate([self.ck, ck], axis=2)
            self.gk = gk if self.gk is None else np.concatenate([self.gk, gk], axis=2)
            self.n_closed += 1
        return out

    def forward(self, x, start_pos):
        B, S, _ = x.shape
        H, KVH, Dh, C = self.H, self.KVH, self.Dh, self.C
        q_raw = self._norm(self._lin(x, "q_proj").view(B, S, H, Dh), "q_norm").transpose(1, 2)
        k_raw = self._norm(self._lin(x, "k_proj").view(B, S, KVH, Dh), "k_norm").transpose(1, 2)
        v = self._lin(x, "v_proj").view(B, S, KVH, Dh).transpose(1, 2)
        cos_f, sin_f = rotary_table(start_pos + S, Dh, self.theta)
        cos, sin = cos_f[start_pos:], sin_f[start_pos:]
        q = rope_torch(q_raw.float(), cos, sin).contiguous().numpy()
        k_rope = rope_torch(k_raw.float(), cos, sin).contiguous().numpy()
        k_raw = k_raw.contiguous().numpy()
        v = v.contiguous().numpy()
        kf, kl = self.m["keep_first"], self.m["keep_last"]
        tc, tg = self.m["topk_chunks"], self.m["topk_groups"]
        if start_pos == 0:
            self.reset()
        first_chunk, last_chunk = start_pos // C, (start_pos + S - 1) // C
        if first_chunk != last_chunk and start_pos == 0:
            out, r, _, _ = oracle.prefill(q, k_rope, k_raw, v, cos.numpy(), sin.numpy(), C=C,
                                          gs=self.gs, keep_first=kf, keep_last=kl,
                                          topk_chunks=tc, topk_groups=tg, theta=self.theta,
                                          dt=oracle.DT_F32)
            self.k_hist, self.kraw_hist, self.v_hist = k_rope, k_raw, v
            self.n_closed = S // C
            if self.n_closed:
                e = self.n_closed * C
                self.ck, self.gk = self._close_summaries(k_rope[:, :, :e], k_raw[:, :, :e], 0,
                                                         cos_f, sin_f)
        else:
            # one decode segment per chunk the block touches (chunk_router.py:493-516)
            out = np.empty_like(q)
            p, done = start_pos, 0
            while done < S:
                take = min(C - (p % C), S - done)
                sl = slice(done, done + take)
                out[:, :, sl] = self._decode_segment(q[:, :, sl], k_rope[:, :, sl],
                                                     k_raw[:, :, sl], v[:, :, sl], p, cos_f,
                                                     sin_f)
                p += take
                done += take
        o = torch.from_numpy(out).transpose(1, 2).reshape(B, S, H * Dh)
        return self._lin(o, "o_proj")
