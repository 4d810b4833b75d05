"""Router configuration, placement policy, KV store and the ``ChunkRouter`` seam.

Mirrors the reference's KvRouter interfaces (``RouterConfig``/``RoutedKV``/``ChunkRouter``,
ExistingModelFineTuning/KvRouter/chunk_router.py:58-162, 463-516; ``ChunkPlacementPolicy``,
chunk_placement_policy.py:12-38) with the same names and argument meaning, but a routing result
is a set of index lists on the GPU rather than materialised K/V + masks, and
``RoutedKV.attend`` launches the fused HIP attention kernel over those lists.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import ops


@dataclass
class RouterConfig:
    """Same fields and derived constants as the reference RouterConfig (chunk_router.py:58-90)."""

    nhead: int
    kv_heads: int
    head_dim: int
    chunk_size: int
    group_size: int
    topk_chunks: int = 20
    topk_groups: int = 32
    current_group_summaries: bool = True
    theta: float = 1_000_000.0
    mixed_rope_threshold: float = 0.5
    mixed_rope_cutoff_pair: Optional[int] = None

    @property
    def groups_per_chunk(self) -> int:
        return self.chunk_size // self.group_size

    @property
    def rep(self) -> int:
        return self.nhead // self.kv_heads

    @property
    def scale(self) -> float:
        return self.head_dim ** -0.5

    @property
    def group_kv_scale(self) -> float:
        return 1.0 / (self.group_size + math.sqrt(self.group_size))

    @property
    def cutoff_pair(self) -> int:
        return ops.mixed_cutoff_pair(self.theta, self.chunk_size, self.head_dim,
                                     self.mixed_rope_threshold, self.mixed_rope_cutoff_pair)


@dataclass(frozen=True)
class ChunkPlacementPolicy:
    """Always-resident windows (chunk_placement_policy.py:12-38)."""

    keep_last: int = 1
    keep_first: int = 0
    first_token_level: bool = False

    def hot_first_range(self, n_closed: int) -> Tuple[int, int]:
        return 0, min(self.keep_first, n_closed)

    def hot_last_range(self, n_closed: int) -> Tuple[int, int]:
        if self.keep_last <= 0:
            return n_closed, n_closed
        return min(max(self.keep_first, n_closed - self.keep_last), n_closed), n_closed


def rotary_for_positions(theta: float, head_dim: int, start: int, length: int,
                         device) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin [length, Dh] for absolute positions [start, start+length): the formula of
    ChunkRouter._rotary_for_positions (chunk_router.py:702-709)."""
    half = head_dim // 2
    inv = 1.0 / (theta ** (torch.arange(half, device=device, dtype=torch.float32) / half))
    pos = torch.arange(start, start + length, device=device, dtype=torch.float32)
    f = pos.unsqueeze(-1) * inv
    e = torch.cat((f, f), dim=-1)
    return e.cos(), e.sin()


class _LayerRecord:
    """Closed-chunk record of one layer on the compute device: store summaries (fp32-table
    anchors, chunk_router.py:552-598) and the RoPE'd token K / V history, capacity-doubling
    like RamKVCacheStore._ensure_capacity (ram_kv_cache_store.py:138-157)."""

    def __init__(self):
        self.chunk_k = None   # [B, KVH, cap, Dh]
        self.group_k = None   # [B, KVH, cap, M, Dh]
        self.tok_k = None     # [B, KVH, cap*C, Dh]
        self.tok_v = None
        self.n_closed = 0
        self.active_krope = None   # [B, KVH, cur, Dh] partial chunk
        self.active_kraw = None
        self.active_v = None


class VramKVCacheStore:
    """All-VRAM store (vram_kv_cache_store.py:15-50 semantics): chunk summaries and the full
    token record stay on the compute device."""

    def __init__(self, *, compute_device, policy: ChunkPlacementPolicy, kv_heads: int,
                 head_dim: int, chunk_size: int, groups_per_chunk: int, batch_size: int,
                 dtype=torch.float32, initial_capacity: int = 64):
        self.compute_device = torch.device(compute_device)
        self.policy = policy
        self.kvh, self.dh, self.C, self.M, self.B = kv_heads, head_dim, chunk_size, \
            groups_per_chunk, batch_size
        self.dtype = dtype
        self._init_cap = initial_capacity
        self._layers: Dict[int, _LayerRecord] = {}

    def reset(self) -> None:
        self._layers.clear()

    def layer(self, layer: int) -> _LayerRecord:
        st = self._layers.get(layer)
        if st is None:
            st = _LayerRecord()
            self._layers[layer] = st
        return st

    def num_closed_chunks(self, layer: int) -> int:
        return self.layer(layer).n_closed

    def ensure_capacity(self, layer: int, need: int) -> _LayerRecord:
        st = self.layer(layer)
        cur = 0 if st.chunk_k is None else st.chunk_k.shape[2]
        if need <= cur:
            return st
        cap = max(self._init_cap, cur * 2, need)
        B, KVH, D, C, M, dev, dt = self.B, self.kvh, self.dh, self.C, self.M, \
            self.compute_device, self.dtype
        ck = torch.zeros(B, KVH, cap, D, device=dev, dtype=dt)
        gk = torch.zeros(B, KVH, cap, M, D, device=dev, dtype=dt)
        tk = torch.zeros(B, KVH, cap * C, D, device=dev, dtype=dt)
        tv = torch.zeros(B, KVH, cap * C, D, device=dev, dtype=dt)
        if st.chunk_k is not None and st.n_closed:
            n = st.n_closed
            ck[:, :, :n] = st.chunk_k[:, :, :n]
            gk[:, :, :n] = st.group_k[:, :, :n]
            tk[:, :, :n * C] = st.tok_k[:, :, :n * C]
            tv[:, :, :n * C] = st.tok_v[:, :, :n * C]
        st.chunk_k, st.group_k, st.tok_k, st.tok_v = ck, gk, tk, tv
        return st

    def chunk_summaries(self, layer: int):
        st = self.layer(layer)
        return None if st.n_closed == 0 else st.chunk_k[:, :, :st.n_closed]


class RoutedKV:
    """Routing result of one block: the index lists the attention kernel reads -- no
    materialised K/V (compare RoutedKV, chunk_router.py:93-162).  ``attend`` computes the exact
    softmax attention over real tokens (``use_summaries=False``, the only mode of the exact
    routed path, HierarchicalGlobalAttentionRouted.py:172-174)."""

    def __init__(self, hcfg, k_rope, v, routing: dict, scale: float, chunk_size: int):
        self.hcfg = hcfg
        self.k_rope = k_rope
        self.v = v
        self.routing = routing
        self.scale = scale
        self.chunked = True
        self.chunk_size = chunk_size

    def attend(self, q: torch.Tensor, use_summaries: bool = False) -> torch.Tensor:
        if use_summaries:
            raise NotImplementedError("summary-attending routed attention is not part of the "
                                      "exact-token path")
        r = self.routing
        return ops.attend_prefill(self.hcfg, q, self.k_rope, self.v, r["open_grp"],
                                  r["open_thr"], r["Kg"])


class ChunkRouter:
    """Routing engine over a KV store (chunk_router.py:165-516).  Prefill of a fresh multi-chunk
    block runs the vectorized semantics through the HIP kernels; blocks inside one chunk go
    through the decode path."""

    def __init__(self, cfg: RouterConfig, store: VramKVCacheStore) -> None:
        self.cfg = cfg
        self.store = store
        self._hcfg_cache: Dict[Tuple[int, torch.dtype], object] = {}

    def reset(self) -> None:
        self.store.reset()

    def hcfg(self, B: int, dtype) -> object:
        key = (B, dtype)
        c = self._hcfg_cache.get(key)
        if c is None:
            cfg, pol = self.cfg, self.store.policy
            c = ops.make_config(batch=B, heads=cfg.nhead, kv_heads=cfg.kv_heads,
                                head_dim=cfg.head_dim, chunk_size=cfg.chunk_size,
                                group_size=cfg.group_size, topk_chunks=cfg.topk_chunks,
                                topk_groups=cfg.topk_groups, keep_first=pol.keep_first,
                                keep_last=pol.keep_last, cutoff_pair=cfg.cutoff_pair,
                                dtype=dtype)
            self._hcfg_cache[key] = c
        return c

    def route_query_block(self, layer: int, q: torch.Tensor, k_rope: torch.Tensor,
                          k_raw: torch.Tensor, v: torch.Tensor, start_pos: int,
                          cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                          populate_store: bool = True, max_chunks_at_once=None,
                          return_positions: bool = False) -> List[Tuple[RoutedKV, int, int]]:
        """Route a block of new queries (chunk_router.py:463-516): q [B,H,S,Dh] RoPE'd,
        k_rope/k_raw/v [B,KVH,S,Dh]; cos/sin the block's rotary rows in the activation dtype
        ([1,1,S,Dh] or [S,Dh]).  Returns [(routed, lo, hi)] segments."""
        if return_positions:
            raise NotImplementedError("token positions are only used by the DCA attend variant")
        C = self.cfg.chunk_size
        S = q.shape[2]
        first_chunk, last_chunk = start_pos // C, (start_pos + S - 1) // C
        if first_chunk == last_chunk:
            raise NotImplementedError("decode blocks are not built yet")
        if start_pos != 0:
            raise NotImplementedError("multi-chunk blocks over resident context are not built")
        return [(self._prefill(layer, q, k_rope, k_raw, v, cos, sin, populate_store), 0, S)]

    def _prefill(self, layer, q, k_rope, k_raw, v, cos, sin, populate_store) -> RoutedKV:
        cfg = self.cfg
        B, H, S, D = q.shape
        dev, dt = q.device, q.dtype
        hc = self.hcfg(B, dt)
        if cos is None or sin is None:
            cos, sin = rotary_for_positions(cfg.theta, D, 0, S, dev)
            cos, sin = cos.to(dt), sin.to(dt)
        cos_r = cos.reshape(-1, D)[:S].float()
        sin_r = sin.reshape(-1, D)[:S].float()
        n_closed = S // cfg.chunk_size
        need_store = populate_store and n_closed > 0
        if dt == torch.float32 or not need_store:
            ck, gk = ops.summarize(hc, k_raw, k_rope, cos_r, sin_r)
            ck_s, gk_s = ck, gk
        else:
            cf, sf = rotary_for_positions(cfg.theta, D, 0, S, dev)
            ck, gk, ck_s, gk_s = ops.summarize(hc, k_raw, k_rope, cos_r, sin_r, cos_b=cf, sin_b=sf)
        routing = ops.route_prefill(hc, q, ck, gk, S)
        if populate_store:
            self._seed_store(layer, k_rope, k_raw, v, ck_s, gk_s, n_closed)
        return RoutedKV(hc, k_rope, v, routing, cfg.scale, cfg.chunk_size)

    def _seed_store(self, layer, k_rope, k_raw, v, ck, gk, n_closed) -> None:
        """Closed chunks into the record, remainder kept as the active chunk
        (ChunkRouter._seed_store_from_block, chunk_router.py:552-598)."""
        C = self.cfg.chunk_size
        st = self.store.layer(layer)
        st.n_closed = 0
        if n_closed:
            st = self.store.ensure_capacity(layer, n_closed)
            e = n_closed * C
            st.chunk_k[:, :, :n_closed] = ck[:, :, :n_closed]
            st.group_k[:, :, :n_closed] = gk[:, :, :n_closed]
            st.tok_k[:, :, :e] = k_rope[:, :, :e]
            st.tok_v[:, :, :e] = v[:, :, :e]
            st.n_closed = n_closed
        S = k_rope.shape[2]
        rem = S - n_closed * C
        if rem > 0:
            st.active_krope = k_rope[:, :, n_closed * C:].contiguous()
            st.active_kraw = k_raw[:, :, n_closed * C:].contiguous()
            st.active_v = v[:, :, n_closed * C:].contiguous()
        else:
            st.active_krope = st.active_kraw = st.active_v = None
