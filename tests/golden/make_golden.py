"""Write golden vectors for the routed-attention path from the reference implementation.

Run ONCE, in the build container only (``python tests/golden/make_golden.py``); the
reference tree (``/root/reference``) exists there and nowhere else.  The script imports the
reference's own ``ChunkRouter`` / ``HierarchicalGlobalAttentionRouted`` (torch + stdlib only),
runs them on small seeded inputs on the CPU, and stores inputs and outputs as ``.npz``
fixtures next to this file.  Nothing here is imported by the library, the GPU tests,
``smoke()`` or ``bench.py``; the fixtures are plain data.

Selection sets are read back without re-deriving them: the script wraps the reference's
module-level gather helpers (``vectorized._gather_chunks`` / ``_gather_groups``,
``ExistingModelFineTuning/KvRouter/vectorized.py:65-89``) to record the index tensors the
reference passes them (``top_chunk_idx`` at ``vectorized.py:339`` and the opened
``source_chunk_idx``/``source_group_idx`` at ``:388``), and reads the per-row visibility from
the masks the reference returns (``vectorized.py:420-425``: summary columns
``[routed groups | current groups | ...]``, token columns ``[current C | opened Kg*gs | ...]``).
For decode it wraps ``ChunkRouter._route_decision`` (``chunk_router.py:187-277``).

Each fixture stores, per (b, h, query chunk n):
  * ``sel_chunk`` / ``sel_thr``  : routed chunks visible to some valid row, with the first such
    row (query-chunk-local), ascending by chunk id, padded with -1;
  * ``open_grp`` / ``open_thr``  : opened groups (absolute id ``chunk*M + group``) visible to
    some valid row, with that first row, ascending, padded with -1;
  * the attention output of ``RoutedKV.attend(use_summaries=False)`` (``chunk_router.py:139-162``).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

REF_ROOT = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REF_ROOT)
sys.path.insert(0, os.path.join(REF_ROOT, "ExistingModelFineTuning"))

from KvRouter import ChunkRouter, RouterConfig, VramKVCacheStore  # noqa: E402
from KvRouter.cache_store import ChunkPlacementPolicy  # noqa: E402
import KvRouter.vectorized as V  # noqa: E402
from HierarchicalGlobalAttentionRouted import HierarchicalGlobalAttentionRouted  # noqa: E402


def sha(*arrs) -> str:
    h = hashlib.sha256()
    for a in arrs:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def make_inputs(seed, B, H, KVH, S, Dh, theta, dtype, scale_inputs=None, qk_rmsnorm=False):
    """Seeded q/k/v generation recipe shared with the tests (torch CPU generator)."""
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


class Capture:
    """Records the index tensors the reference hands its gather helpers."""

    def __init__(self):
        self.gc, self.gg = [], []
        self._gc0, self._gg0 = V._gather_chunks, V._gather_groups

    def __enter__(self):
        def gc(t, idx):
            self.gc.append(idx.clone())
            return self._gc0(t, idx)

        def gg(t, cidx, gidx):
            self.gg.append((cidx.clone(), gidx.clone()))
            return self._gg0(t, cidx, gidx)

        V._gather_chunks, V._gather_groups = gc, gg
        return self

    def __exit__(self, *a):
        V._gather_chunks, V._gather_groups = self._gc0, self._gg0


def first_true_row(mask_cols, valid_rows):
    """mask_cols [..., C, K] bool -> first valid row index per column, or -1."""
    C = mask_cols.shape[-2]
    m = mask_cols & valid_rows.view(*([1] * (mask_cols.ndim - 2)), C, 1)
    any_ = m.any(dim=-2)
    first = torch.argmax(m.to(torch.int8), dim=-2)
    return torch.where(any_, first, torch.full_like(first, -1))


def pack_sets(ids, thr, width):
    """ids/thr [..., K] with thr=-1 for invisible -> ascending padded arrays [..., width]."""
    lead = ids.shape[:-1]
    out_id = np.full(lead + (width,), -1, np.int32)
    out_thr = np.full(lead + (width,), -1, np.int32)
    ids_n, thr_n = ids.numpy(), thr.numpy()
    for idx in np.ndindex(*lead):
        pairs = sorted({(int(i), int(t)) for i, t in zip(ids_n[idx], thr_n[idx]) if t >= 0})
        assert len({p[0] for p in pairs}) == len(pairs), "duplicate visible id"
        for j, (i, t) in enumerate(pairs):
            out_id[idx + (j,)] = i
            out_thr[idx + (j,)] = t
    return out_id, out_thr


def run_prefill_case(name, *, B, H, KVH, S, Dh, C, gs, kf, kl, tc, tg, theta, dtype, seed,
                     scale_inputs=None, qk_rmsnorm=False, store_inputs=True, out_row_stride=1):
    cfg = RouterConfig(nhead=H, kv_heads=KVH, head_dim=Dh, chunk_size=C, group_size=gs,
                       topk_chunks=tc, topk_groups=tg, theta=theta)
    policy = ChunkPlacementPolicy(keep_first=kf, keep_last=kl, first_token_level=True)
    mod = HierarchicalGlobalAttentionRouted(d_model=H * Dh, nhead=H, kv_heads=KVH, head_dim=Dh,
                                            theta=theta)
    q_raw, k_raw, v = make_inputs(seed, B, H, KVH, S, Dh, theta, dtype, scale_inputs, qk_rmsnorm)
    cos, sin = mod._get_rotary(S, torch.device("cpu"))            # fp32 [S, Dh]
    c4, s4 = cos[None, None], sin[None, None]
    q = mod._apply_rotary(q_raw.float(), c4, s4).to(dtype)
    k_rope = mod._apply_rotary(k_raw.float(), c4, s4).to(dtype)
    cos_r, sin_r = c4.to(dtype), s4.to(dtype)

    store = VramKVCacheStore(compute_device=torch.device("cpu"), policy=policy, kv_heads=KVH,
                             head_dim=Dh, chunk_size=C, groups_per_chunk=C // gs, batch_size=B,
                             dtype=dtype)
    router = ChunkRouter(cfg, store)
    router.reset()
    with Capture() as cap, torch.no_grad():
        segs = router.route_query_block(0, q, k_rope, k_raw, v, 0, cos=cos_r, sin=sin_r)
        (routed, lo, hi), = segs
        out = routed.attend(q, use_summaries=False)
    N = (S + C - 1) // C
    M = C // gs
    Kc = min(tc, N) if tc > 0 else 0
    Tgrp = Kc * M
    Kg = min(tg, Tgrp) if tg > 0 else 0
    valid = (torch.arange(N * C) < S).view(N, C)
    res = dict(meta=json.dumps(dict(name=name, B=B, H=H, KVH=KVH, S=S, Dh=Dh, C=C, gs=gs,
                                    keep_first=kf, keep_last=kl, topk_chunks=tc, topk_groups=tg,
                                    theta=theta, dtype=str(dtype).split(".")[-1], seed=seed,
                                    scale_inputs=scale_inputs, qk_rmsnorm=qk_rmsnorm,
                                    Kc=Kc, Kg=Kg, out_row_stride=out_row_stride)))
    vmask = valid.view(1, 1, N, C)
    if Kc > 0:
        top_chunk_idx = cap.gc[0]                                     # vectorized.py:339
        assert top_chunk_idx.shape == (B, H, N, Kc)
        sm = routed.summary_mask                                      # [B,H,N,C,Tgrp+M+...]
        slot_cols = sm[..., :Tgrp].reshape(B, H, N, C, Kc, M)[..., 0]  # chunk_visible per slot
        thr = torch.stack([first_true_row(slot_cols[:, :, n], valid[n]) for n in range(N)], 2)
        res["sel_chunk"], res["sel_thr"] = pack_sets(top_chunk_idx, thr, Kc)
    if Kg > 0 and min(tg // 2, Tgrp) > 0:
        src_c, src_g = cap.gg[0]                                      # vectorized.py:388
        assert src_c.shape == (B, H, N, Kg)
        tm = routed.token_mask                                        # [B,H,N,C,C+Kg*gs+...]
        op_cols = tm[..., C:C + Kg * gs].reshape(B, H, N, C, Kg, gs)[..., 0]
        thr = torch.stack([first_true_row(op_cols[:, :, n], valid[n]) for n in range(N)], 2)
        res["open_grp"], res["open_thr"] = pack_sets(src_c * M + src_g, thr, Kg)
    o = out.float().numpy()
    res["out"] = o[:, :, ::out_row_stride].copy()
    res["out_sum"] = np.array([o.astype(np.float64).sum(), np.abs(o.astype(np.float64)).sum()])
    if store_inputs:
        for nm, t in (("q", q), ("k_rope", k_rope), ("k_raw", k_raw), ("v", v)):
            res[nm] = t.float().numpy()
    res["inputs_sha"] = np.frombuffer(sha(q.float().numpy(), k_raw.float().numpy(),
                                          v.float().numpy()).encode(), dtype=np.uint8)
    res["cos"], res["sin"] = cos.numpy(), sin.numpy()
    del vmask
    return res


def run_summary_case(name, *, B, KVH, S, Dh, C, gs, theta, dtype, seed):
    """Summaries as the vectorized path computes them (``vectorized.py:275-287``), captured at
    KV-head granularity (H == KVH so no head expansion is involved)."""
    H = KVH
    cfg = RouterConfig(nhead=H, kv_heads=KVH, head_dim=Dh, chunk_size=C, group_size=gs,
                       topk_chunks=4, topk_groups=8, theta=theta)
    mod = HierarchicalGlobalAttentionRouted(d_model=H * Dh, nhead=H, kv_heads=KVH, head_dim=Dh,
                                            theta=theta)
    q_raw, k_raw, v = make_inputs(seed, B, H, KVH, S, Dh, theta, dtype)
    cos, sin = mod._get_rotary(S, torch.device("cpu"))
    c4, s4 = cos[None, None], sin[None, None]
    k_rope = mod._apply_rotary(k_raw.float(), c4, s4).to(dtype)
    got = []
    orig = V._rope_summary

    def rs(*a, **kw):
        r = orig(*a, **kw)
        got.append(r.clone())
        return r

    V._rope_summary = rs
    try:
        with torch.no_grad():
            V.assemble_routed_kv(cfg, k_rope, k_rope, k_raw, v, c4.to(dtype), s4.to(dtype),
                                 keep_first=1, keep_last=2)
    finally:
        V._rope_summary = orig
    chunk_k, group_k = got[0], got[1]
    # Store-side twin: fp32 anchor cos/sin (chunk_router.py:575-585, 693-709).
    store = VramKVCacheStore(compute_device=torch.device("cpu"),
                             policy=ChunkPlacementPolicy(keep_first=1, keep_last=2,
                                                         first_token_level=True),
                             kv_heads=KVH, head_dim=Dh, chunk_size=C, groups_per_chunk=C // gs,
                             batch_size=B, dtype=dtype)
    router = ChunkRouter(cfg, store)
    router._seed_store_from_block(0, k_rope, k_raw, v)
    n_closed = S // C
    st = store._layer(0)
    return dict(meta=json.dumps(dict(name=name, B=B, KVH=KVH, S=S, Dh=Dh, C=C, gs=gs, theta=theta,
                                     dtype=str(dtype).split(".")[-1], seed=seed)),
                k_raw=k_raw.float().numpy(), k_rope=k_rope.float().numpy(),
                cos=cos.numpy(), sin=sin.numpy(),
                chunk_k=chunk_k.float().numpy(), group_k=group_k.float().numpy(),
                store_chunk_k=st.chunk_k[:, :, :n_closed].float().numpy(),
                store_group_k=st.cpu_group_k[:, :, :n_closed].float().numpy())


def run_module_case(name, *, B, S, d_model, H, KVH, Dh, C, gs, kf, kl, tc, tg, theta, seed,
                    gen=0, cache_location="vram", qk_norm=False, blocks=None):
    """Full ``HierarchicalGlobalAttentionRouted.forward`` (HierarchicalGlobalAttentionRouted.py:137-177):
    a prefill of ``S`` tokens, then ``gen`` one-token decode steps through a cache object, or
    (``blocks``) blocks of the given token counts, each routed by the reference as decode
    segments of up to one chunk (chunk_router.py:493-516) -- L > 1 rows per routing decision."""
    if blocks is not None:
        gen = int(sum(blocks))
    torch.manual_seed(seed)
    mod = HierarchicalGlobalAttentionRouted(d_model=d_model, nhead=H, kv_heads=KVH, head_dim=Dh,
                                            chunk_size=C, group_size=gs, topk_chunks=tc,
                                            topk_groups=tg, keep_first=kf, keep_last=kl,
                                            theta=theta, cache_location=cache_location,
                                            qk_norm=qk_norm).eval()
    if qk_norm:   # non-trivial norm weights so the test sees them
        with torch.no_grad():
            mod.q_norm.weight.uniform_(0.5, 1.5)
            mod.k_norm.weight.uniform_(0.5, 1.5)
    x = torch.randn(B, S + gen, d_model, generator=torch.Generator().manual_seed(seed + 1))

    class _Cache:
        pass

    decisions = []
    orig = ChunkRouter._route_decision

    def rd(self, q, layer, n_closed):
        r = orig(self, q, layer, n_closed)
        mid_idx, _, _, mid_vis, oc, og, ov = r
        decisions.append(dict(n_closed=n_closed, mid_idx=mid_idx.clone(), mid_vis=mid_vis.clone(),
                              open_chunk=oc.clone(), open_grp=og.clone(), open_vis=ov.clone()))
        return r

    ChunkRouter._route_decision = rd
    outs = []
    try:
        cache = _Cache()
        with torch.no_grad():
            cp = torch.arange(S)
            o, _ = mod(hidden_states=x[:, :S], past_key_value=cache, cache_position=cp)
            outs.append(o)
            p = S
            for L in (blocks if blocks is not None else [1] * gen):
                o, _ = mod(hidden_states=x[:, p:p + L], past_key_value=cache,
                           cache_position=torch.arange(p, p + L))
                outs.append(o)
                p += L
    finally:
        ChunkRouter._route_decision = orig
    res = dict(meta=json.dumps(dict(name=name, B=B, S=S, d_model=d_model, H=H, KVH=KVH, Dh=Dh,
                                    C=C, gs=gs, keep_first=kf, keep_last=kl, topk_chunks=tc,
                                    topk_groups=tg, theta=theta, seed=seed, gen=gen,
                                    cache_location=cache_location, qk_norm=qk_norm,
                                    blocks=blocks)),
               x=x.numpy(), out=torch.cat(outs, dim=1).numpy())
    for k_, t in mod.state_dict().items():
        res["w_" + k_] = t.numpy()
    M = C // gs
    # Decode decisions: per step, routed chunks visible at L=1 and opened groups visible.
    dec = [d for d in decisions]
    if gen > 0 and blocks is None:
        Kmax = max([d["mid_idx"].shape[-1] for d in dec] + [1])
        Gmax = max([d["open_chunk"].shape[-1] for d in dec] + [1])
        sel = np.full((len(dec), B, H, Kmax), -1, np.int32)
        opn = np.full((len(dec), B, H, Gmax), -1, np.int32)
        ncl = np.zeros(len(dec), np.int32)
        for i, d in enumerate(dec):
            ncl[i] = d["n_closed"]
            if d["mid_idx"].shape[-1]:
                vis = d["mid_vis"][:, :, 0]                 # L == 1
                ids = torch.where(vis, d["mid_idx"], torch.full_like(d["mid_idx"], -1))
                s = np.sort(np.where(ids.numpy() < 0, 1 << 30, ids.numpy()), -1)
                sel[i, ..., :s.shape[-1]] = np.where(s == 1 << 30, -1, s)
            if d["open_chunk"].shape[-1]:
                vis = d["open_vis"][:, :, 0]
                g = d["open_chunk"] * M + d["open_grp"]
                ids = torch.where(vis, g, torch.full_like(g, -1)).numpy()
                s = np.sort(np.where(ids < 0, 1 << 30, ids), -1)
                opn[i, ..., :s.shape[-1]] = np.where(s == 1 << 30, -1, s)
        res["dec_n_closed"], res["dec_sel"], res["dec_open"] = ncl, sel, opn
    if blocks is not None:
        # L-row decisions: every id visible to some row, ascending, with its first such row
        # (chunk_router.py:225-276 -- the pool and the group requests span all L rows)
        def first_rows(ids, vis):
            """ids [B, H, K], vis [B, H, L, K] -> (sorted ids, first rows) padded with -1."""
            anyv = vis.any(dim=2)
            first = torch.argmax(vis.to(torch.int8), dim=2)
            out_id = np.full(ids.shape, -1, np.int32)
            out_thr = np.full(ids.shape, -1, np.int32)
            for b in range(ids.shape[0]):
                for h in range(ids.shape[1]):
                    keep = [(int(ids[b, h, j]), int(first[b, h, j])) for j in range(ids.shape[2])
                            if bool(anyv[b, h, j])]
                    keep.sort()
                    for j, (i_, t_) in enumerate(keep):
                        out_id[b, h, j], out_thr[b, h, j] = i_, t_
            return out_id, out_thr

        Kmax = max([d["mid_idx"].shape[-1] for d in dec] + [1])
        Gmax = max([d["open_chunk"].shape[-1] for d in dec] + [1])
        n = len(dec)
        bl = dict(L=np.zeros(n, np.int32), sel=np.full((n, B, H, Kmax), -1, np.int32),
                  sel_thr=np.full((n, B, H, Kmax), -1, np.int32),
                  open=np.full((n, B, H, Gmax), -1, np.int32),
                  open_thr=np.full((n, B, H, Gmax), -1, np.int32))
        for i, d in enumerate(dec):
            bl["L"][i] = d["mid_vis"].shape[2] if d["mid_idx"].shape[-1] else d["open_vis"].shape[2]
            if d["mid_idx"].shape[-1]:
                a, t = first_rows(d["mid_idx"], d["mid_vis"])
                bl["sel"][i, ..., :a.shape[-1]], bl["sel_thr"][i, ..., :a.shape[-1]] = a, t
            if d["open_chunk"].shape[-1]:
                a, t = first_rows(d["open_chunk"] * M + d["open_grp"], d["open_vis"])
                bl["open"][i, ..., :a.shape[-1]], bl["open_thr"][i, ..., :a.shape[-1]] = a, t
        for k_, v_ in bl.items():
            res["blk_" + k_] = v_
    return res


def main():
    torch.set_num_threads(8)
    cases = {}
    # c1 exactly; inputs regenerated by the tests from the recipe.
    cases["c1_full"] = run_prefill_case(
        "c1_full", B=1, H=8, KVH=2, S=2048, Dh=64, C=64, gs=16, kf=1, kl=2, tc=4, tg=8,
        theta=1e4, dtype=torch.float32, seed=0, scale_inputs=1.0 / 8.0, store_inputs=False,
        out_row_stride=16)
    # c1 shape with a ragged tail (partial last chunk and partial last group).
    cases["c1_ragged"] = run_prefill_case(
        "c1_ragged", B=1, H=8, KVH=2, S=1000, Dh=64, C=64, gs=16, kf=1, kl=2, tc=4, tg=8,
        theta=1e4, dtype=torch.float32, seed=1, scale_inputs=1.0 / 8.0, store_inputs=False,
        out_row_stride=4)
    # keep_first = keep_last = 0 -> the previous chunk is force-included (vectorized.py:314-337).
    cases["forced_prev"] = run_prefill_case(
        "forced_prev", B=2, H=4, KVH=2, S=203, Dh=16, C=8, gs=4, kf=0, kl=0, tc=3, tg=6,
        theta=1e4, dtype=torch.float32, seed=2)
    # reference test shape (KvRouter/Tests/test_routed_attention.py:36-46) with module defaults.
    cases["ref_shape"] = run_prefill_case(
        "ref_shape", B=2, H=4, KVH=2, S=37, Dh=16, C=8, gs=4, kf=1, kl=2, tc=3, tg=4,
        theta=1e4, dtype=torch.float32, seed=3)
    # topk >= pool: every pool chunk selected; groups Kg < Tgrp with Kg_request < Kg.
    cases["wide_topk"] = run_prefill_case(
        "wide_topk", B=1, H=2, KVH=1, S=160, Dh=32, C=16, gs=4, kf=1, kl=1, tc=16, tg=10,
        theta=1e4, dtype=torch.float32, seed=4)
    # bf16 c3-like miniature: selection in the reference is on bf16-rounded scores, so only
    # the attention output is used from this case (selection parity is defined in fp32).
    cases["bf16_mini"] = run_prefill_case(
        "bf16_mini", B=1, H=8, KVH=2, S=640, Dh=128, C=64, gs=16, kf=2, kl=2, tc=4, tg=8,
        theta=1e6, dtype=torch.bfloat16, seed=5, qk_rmsnorm=True, store_inputs=False,
        out_row_stride=4)
    cases["sum_bf16"] = run_summary_case("sum_bf16", B=1, KVH=2, S=300, Dh=64, C=64, gs=16,
                                         theta=1e4, dtype=torch.bfloat16, seed=6)
    cases["sum_f32"] = run_summary_case("sum_f32", B=2, KVH=2, S=45, Dh=16, C=8, gs=4,
                                        theta=1e4, dtype=torch.float32, seed=7)
    cases["mod_prefill"] = run_module_case(
        "mod_prefill", B=2, S=37, d_model=64, H=4, KVH=2, Dh=16, C=8, gs=4, kf=1, kl=2, tc=3,
        tg=4, theta=1e4, seed=8)
    cases["mod_decode"] = run_module_case(
        "mod_decode", B=1, S=60, d_model=64, H=4, KVH=2, Dh=16, C=8, gs=4, kf=1, kl=1, tc=3,
        tg=4, theta=1e4, seed=9, gen=24)
    cases["mod_decode_prev"] = run_module_case(
        "mod_decode_prev", B=1, S=44, d_model=64, H=4, KVH=2, Dh=16, C=8, gs=4, kf=0, kl=0,
        tc=2, tg=4, theta=1e4, seed=10, gen=20)
    cases["mod_decode_ram"] = run_module_case(
        "mod_decode_ram", B=2, S=52, d_model=64, H=4, KVH=2, Dh=16, C=8, gs=4, kf=1, kl=2,
        tc=3, tg=6, theta=1e4, seed=11, gen=14, cache_location="ram", qk_norm=True)
    # multi-row decode blocks (the chat feeds 64-token blocks, chat_qwen30b_fp8.py:67): blocks of
    # 3, 11 and 64 tokens after a prefill, crossing chunk boundaries (C 16) ...
    cases["mod_blocks"] = run_module_case(
        "mod_blocks", B=2, S=75, d_model=64, H=4, KVH=2, Dh=16, C=16, gs=4, kf=1, kl=2, tc=3,
        tg=6, theta=1e4, seed=12, blocks=[3, 11, 64, 3, 11])
    # ... and at C 64: the active chunk filled, then a whole 64-row chunk in one decode segment
    cases["mod_blocks64"] = run_module_case(
        "mod_blocks64", B=1, S=514, d_model=64, H=4, KVH=2, Dh=16, C=64, gs=16, kf=1, kl=1,
        tc=3, tg=8, theta=1e4, seed=13, blocks=[62, 64, 11, 3], cache_location="ram")
    only = sys.argv[1:]
    for name, res in cases.items():
        if only and name not in only:
            continue
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **res)
        print(f"wrote {path} ({os.path.getsize(path) / 1024:.1f} KiB)")


if __name__ == "__main__":
    main()
