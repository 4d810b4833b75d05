"""Router configuration, placement policy, KV store and the ``ChunkRouter`` seam.

Mirrors the reference's KvRouter interfaces (``RouterConfig``/``RoutedKV``/``ChunkRouter``,
ExistingModelFineTuning/KvRouter/chunk_router.py:58-162, 463-516; ``ChunkPlacementPolicy``,
chunk_placement_policy.py:12-38) with the same names and argument meaning, but a routing result
is a set of index lists on the GPU rather than materialised K/V + masks, and
``RoutedKV.attend`` launches the fused HIP attention kernel over those lists.
"""
from __future__ import annotations

import math
import os
import shutil
import tempfile
import weakref
from abc import ABC, abstractmethod
from collections import OrderedDict
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np
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
    """Per-layer store state: closed-chunk summary tables on the compute device (store anchors,
    fp32 table, chunk_router.py:552-598, 631-657), the token record, and the active chunk's raw
    keys (needed for its summaries when it closes).  Capacities double like
    RamKVCacheStore._ensure_capacity (ram_kv_cache_store.py:138-157)."""

    def __init__(self):
        self.cap = 0
        self.chunk_k = None      # [B, KVH, cap, Dh]
        self.group_k = None      # [B, KVH, cap, M, Dh]
        self.tok_k = None        # record [B, KVH, cap*C, Dh]: device (VRAM) or pinned host (RAM)
        self.tok_v = None
        self.first_k = None      # RAM tier: first window [B, KVH, kf*C, Dh] on device
        self.first_v = None
        self.ring_k = None       # RAM tier: last window + active chunk, ring of kl+1 chunks
        self.ring_v = None
        self.ring_R = 0
        self.act_kraw = None     # [B, KVH, C, Dh] raw keys of the active chunk
        self.n_closed = 0


class KVCacheStore(ABC):
    """The tiered KV store interface (kv_cache_store.py:26-82): one instance serves all layers;
    per layer it holds the closed chunks' summaries (chunk_k [B, KVH, Dh] on the compute device,
    the routing table), their group summaries and their tokens.  The router of this package
    reads the summary tables and the token sources directly (``layer``/``sources``); these
    methods are the reference's seam for callers that drive a store themselves."""

    def __init__(self, *, compute_device, policy: ChunkPlacementPolicy) -> None:
        self.compute_device = torch.device(compute_device)
        self.policy = policy

    @abstractmethod
    def reset(self) -> None: ...

    @abstractmethod
    def num_closed_chunks(self, layer: int) -> int: ...

    @abstractmethod
    def chunk_summaries(self, layer: int) -> Optional[torch.Tensor]:
        """[B, KVH, n_closed, Dh] on the compute device, or None."""

    @abstractmethod
    def append_closed_chunk(self, layer: int, chunk_k: torch.Tensor, group_k: torch.Tensor,
                            group_v: torch.Tensor, token_k: torch.Tensor,
                            token_v: torch.Tensor) -> None:
        """Store a freshly closed chunk: chunk_k [B, KVH, Dh], group_k/group_v [B, KVH, M, Dh],
        token_k/token_v [B, KVH, C, Dh]."""

    @abstractmethod
    def gather_group_summaries(self, layer: int, chunk_idx: torch.Tensor
                               ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Group K/V summaries of chunk_idx [B, H, *] -> [B, H, *, M, Dh] on the device."""

    @abstractmethod
    def gather_tokens(self, layer: int, chunk_idx: torch.Tensor, group_idx: torch.Tensor
                      ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Token K/V of the groups (chunk_idx, group_idx) [B, H, *] -> [B, H, *, gs, Dh]."""

    @abstractmethod
    def hot_group_summaries(self, layer: int, lo: int, hi: int
                            ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Group K/V summaries of the window chunks [lo, hi) -> [B, KVH, hi-lo, M, Dh]."""

    @abstractmethod
    def hot_tokens(self, layer: int, lo: int, hi: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Token K/V of the window chunks [lo, hi) -> [B, KVH, hi-lo, C, Dh]."""

    def prefetch(self, layer: int, chunk_idx: torch.Tensor) -> None:  # noqa: B027
        """Best-effort hint that chunk_idx will be gathered soon (no-op unless a tier reads
        from disk)."""


class _StoreBase(KVCacheStore):
    def __init__(self, *, compute_device, policy: ChunkPlacementPolicy, kv_heads: int,
                 head_dim: int, chunk_size: int, groups_per_chunk: int, batch_size: int,
                 dtype=torch.float32, initial_capacity: int = 64):
        super().__init__(compute_device=compute_device, policy=policy)
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

    def chunk_summaries(self, layer: int):
        st = self.layer(layer)
        return None if st.n_closed == 0 else st.chunk_k[:, :, :st.n_closed]

    def prepare_block(self, layer: int, first_chunk: int, last_chunk: int) -> None:
        """Reserve room for every chunk a block touches before any of its segments is routed,
        so routed segments keep reading the buffers they were routed against."""
        self.ensure_capacity(layer, last_chunk + 1)

    def _dev_zeros(self, *shape):
        return torch.zeros(*shape, device=self.compute_device, dtype=self.dtype)

    def ensure_capacity(self, layer: int, need: int) -> _LayerRecord:
        """Room for `need` chunks (closed + active) in the summary tables and the record."""
        st = self.layer(layer)
        if need <= st.cap:
            return st
        cap = max(self._init_cap, st.cap * 2, need)
        B, KVH, D, C, M = self.B, self.kvh, self.dh, self.C, self.M
        ck, gk = self._dev_zeros(B, KVH, cap, D), self._dev_zeros(B, KVH, cap, M, D)
        tk, tv = self._new_record(B, KVH, cap * C, D), self._new_record(B, KVH, cap * C, D)
        if st.cap:
            if not st.tok_k.is_cuda:   # pending async D2H copies into the old host record
                torch.cuda.current_stream(self.compute_device).synchronize()
            n = st.n_closed
            ck[:, :, :n] = st.chunk_k[:, :, :n]
            gk[:, :, :n] = st.group_k[:, :, :n]
            keep = self._record_len(st)
            tk[:, :, :keep].copy_(st.tok_k[:, :, :keep])
            tv[:, :, :keep].copy_(st.tok_v[:, :, :keep])
        st.chunk_k, st.group_k, st.tok_k, st.tok_v, st.cap = ck, gk, tk, tv, cap
        if st.act_kraw is None:
            st.act_kraw = self._dev_zeros(B, KVH, C, D)
        return st

    # -- the KVCacheStore seam ---------------------------------------------------------------
    # Group V summaries are not stored: the exact-token path never reads them, and they are a
    # function of the tokens the store holds (sum over the group's values x 1/(gs + sqrt(gs)),
    # chunk_router.py:641-642, 578), so the gathers below recompute them from the tokens.
    def _group_v(self, v: torch.Tensor) -> torch.Tensor:
        """[..., C, Dh] token values -> [..., M, Dh] group V summaries."""
        gs = self.C // self.M
        return v.reshape(*v.shape[:-2], self.M, gs, self.dh).sum(dim=-2) * \
            (1.0 / (gs + math.sqrt(gs)))

    def append_closed_chunk(self, layer: int, chunk_k, group_k, group_v, token_k,
                            token_v) -> None:
        """Chunk n_closed closes with the given summaries and tokens (its token rows are
        written as the active chunk's, then handed on as when the router closes a chunk).
        group_v is not kept (recomputed from token_v)."""
        st = self.layer(layer)
        n = st.n_closed
        B, KVH, C, D, M = self.B, self.kvh, self.C, self.dh, self.M
        if tuple(chunk_k.shape) != (B, KVH, D) or tuple(group_k.shape) != (B, KVH, M, D) or \
                tuple(token_k.shape) != (B, KVH, C, D) or token_v.shape != token_k.shape:
            raise ValueError("append_closed_chunk: chunk_k [B,KVH,Dh], group_k [B,KVH,M,Dh], "
                             "token_k/token_v [B,KVH,C,Dh] expected")
        self.prepare_block(layer, n, n + 1)
        st = self.layer(layer)
        dev = self.compute_device
        st.chunk_k[:, :, n] = chunk_k.detach().to(dev)
        st.group_k[:, :, n] = group_k.detach().to(dev)
        self.write_tokens(layer, n * C, token_k.detach().to(dev, self.dtype),
                          token_v.detach().to(dev, self.dtype))
        self.close_chunk(layer, n)
        st.n_closed = n + 1

    def seed_closed_chunks(self, layer: int, chunk_k, group_k, group_v, token_k,
                           token_v) -> None:
        """N closed chunks at once (ram_kv_cache_store.py:483-527): chunk_k [B,KVH,N,Dh],
        group_k/group_v [B,KVH,N,M,Dh], token_k/token_v [B,KVH,N,C,Dh]; replaces the layer's
        contents.  group_v is not kept."""
        B, KVH, N = token_k.shape[:3]
        C, D = self.C, self.dh
        st = self.layer(layer)
        st.n_closed = 0
        st = self.ensure_capacity(layer, N + 1)
        dev = self.compute_device
        st.chunk_k[:, :, :N] = chunk_k.detach().to(dev)
        st.group_k[:, :, :N] = group_k.detach().to(dev)
        self.seed(layer, token_k.detach().to(dev, self.dtype).reshape(B, KVH, N * C, D),
                  token_v.detach().to(dev, self.dtype).reshape(B, KVH, N * C, D), N)
        st.n_closed = N

    def _hot_chunk(self, layer: int, c: int):
        """Device views [B, KVH, C, Dh] of window chunk c's keys and values."""
        src = self.sources(layer)
        C = self.C
        n_closed = self.num_closed_chunks(layer)
        first = c < self.policy.hot_first_range(n_closed)[1]
        if not (first or self.policy.hot_last_range(n_closed)[0] <= c <= n_closed):
            raise ValueError(f"chunk {c} is not in a window of layer {layer} "
                             f"({n_closed} closed chunks)")
        if src["ring_chunks"] == 0:                       # record by position (VRAM tier)
            return src["recent_k"][:, :, c * C:(c + 1) * C], src["recent_v"][:, :, c * C:(c + 1) * C]
        if first:
            return src["first_k"][:, :, c * C:(c + 1) * C], src["first_v"][:, :, c * C:(c + 1) * C]
        s = (c % src["ring_chunks"]) * C
        return src["recent_k"][:, :, s:s + C], src["recent_v"][:, :, s:s + C]

    def hot_tokens(self, layer: int, lo: int, hi: int):
        if not 0 <= lo <= hi <= self.num_closed_chunks(layer):
            raise ValueError(f"window chunks [{lo}, {hi}) outside the closed chunks")
        if hi == lo:
            e = torch.empty(self.B, self.kvh, 0, self.C, self.dh, dtype=self.dtype,
                            device=self.compute_device)
            return e, e.clone()
        kv = [self._hot_chunk(layer, c) for c in range(lo, hi)]
        return (torch.stack([k for k, _ in kv], dim=2), torch.stack([v for _, v in kv], dim=2))

    def hot_group_summaries(self, layer: int, lo: int, hi: int):
        _, v = self.hot_tokens(layer, lo, hi)
        return self.layer(layer).group_k[:, :, lo:hi].clone(), self._group_v(v)

    def _gather_groups(self, layer: int, grp: torch.Tensor):
        """Token K/V [B, H, K, gs, Dh] of the global group ids grp [B, H, K] (chunk*M + group)
        of closed chunks, through the decode gather (one copy per distinct group and KV head,
        from whichever record the tier keeps)."""
        B, H, K = grp.shape
        gs, D = self.C // self.M, self.dh
        n_closed = self.num_closed_chunks(layer)
        cfg = ops.make_config(batch=B, heads=H, kv_heads=self.kvh, head_dim=D, chunk_size=self.C,
                              group_size=gs, topk_chunks=1, topk_groups=K,
                              keep_first=self.policy.keep_first, keep_last=self.policy.keep_last,
                              cutoff_pair=0, dtype=self.dtype)
        if int(grp.numel()) and (int(grp.min()) < 0 or int(grp.max()) >= n_closed * self.M):
            raise ValueError("group ids outside the closed chunks")
        src = self.sources(layer)
        og = grp.to(self.compute_device, torch.int32).contiguous()
        ot = torch.zeros_like(og)
        resolve = src.get("resolve")
        og_rec, n_rec, rk, rv = (resolve(og) if resolve is not None else
                                 (og, n_closed, src["record_k"], src["record_v"]))
        sk, sv, sg = ops.gather_decode(cfg, n_rec, og_rec, ot, K, rk, rv, src["record_on_host"],
                                       ops.DecodeStaging(), H)
        U = sk.shape[2] // gs
        b = torch.arange(B, device=og.device).view(B, 1, 1)
        kv = (torch.arange(H, device=og.device) // (H // self.kvh)).view(1, H, 1)
        slot = sg.long()
        return (sk.view(B, self.kvh, U, gs, D)[b, kv, slot],
                sv.view(B, self.kvh, U, gs, D)[b, kv, slot])

    def gather_tokens(self, layer: int, chunk_idx: torch.Tensor, group_idx: torch.Tensor):
        shape = tuple(chunk_idx.shape)
        B, H = shape[:2]
        grp = (chunk_idx.long() * self.M + group_idx.long()).reshape(B, H, -1)
        k, v = self._gather_groups(layer, grp)
        tail = (self.C // self.M, self.dh)
        return k.reshape(*shape, *tail), v.reshape(*shape, *tail)

    def gather_group_summaries(self, layer: int, chunk_idx: torch.Tensor):
        shape = tuple(chunk_idx.shape)
        B, H = shape[:2]
        dev = self.compute_device
        idx = chunk_idx.to(dev).long().reshape(B, H, -1)
        st = self.layer(layer)
        b = torch.arange(B, device=dev).view(B, 1, 1)
        kvh = (torch.arange(H, device=dev) // (H // self.kvh)).view(1, H, 1)
        gk = st.group_k[b, kvh, idx]                                        # [B, H, n, M, Dh]
        grp = (idx.unsqueeze(-1) * self.M + torch.arange(self.M, device=dev)).reshape(B, H, -1)
        _, v = self._gather_groups(layer, grp)                              # [B, H, n*M, gs, Dh]
        gv = v.sum(dim=-2) * (1.0 / (self.C // self.M + math.sqrt(self.C // self.M)))
        tail = (self.M, self.dh)
        return gk.reshape(*shape, *tail), gv.reshape(*shape, *tail)


class VramKVCacheStore(_StoreBase):
    """All-VRAM tier (vram_kv_cache_store.py:15-50): summaries and every token, closed and
    active, live on the compute device in one record addressed by absolute position."""

    def _new_record(self, *shape):
        return self._dev_zeros(*shape)

    def _record_len(self, st):
        return st.cap * self.C

    def token_rows(self, layer: int, pos: int, L: int):
        """Device views [B, KVH, L, Dh] that tokens pos..pos+L-1 (one active chunk) go to."""
        st = self.layer(layer)
        return st.tok_k[:, :, pos:pos + L], st.tok_v[:, :, pos:pos + L]

    def write_tokens(self, layer: int, pos: int, k_rope, v) -> None:
        kd, vd = self.token_rows(layer, pos, k_rope.shape[2])
        kd.copy_(k_rope)
        vd.copy_(v)

    def close_chunk(self, layer: int, n: int) -> None:
        pass

    def seed(self, layer: int, k_rope, v, n_closed: int) -> None:
        st = self.layer(layer)
        S = k_rope.shape[2]
        st.tok_k[:, :, :S] = k_rope
        st.tok_v[:, :, :S] = v

    def sources(self, layer: int):
        st = self.layer(layer)
        return dict(recent_k=st.tok_k, recent_v=st.tok_v, ring_chunks=0, first_k=st.tok_k,
                    first_v=st.tok_v, record_k=st.tok_k, record_v=st.tok_v, record_on_host=False)


class RamKVCacheStore(_StoreBase):
    """RAM tier (ram_kv_cache_store.py:29-619 semantics): the closed-token record lives in pinned
    host memory; only the summary tables, the first window and a ring holding the last window
    plus the active chunk live on the GPU.  Each decode step gathers its opened groups,
    deduplicated over the query heads of a KV head, from the host record into a device staging
    buffer (hga_gather_decode: coalesced 4 KiB group reads over PCIe), and attention reads them
    there, so only routed groups cross the link, once per KV head.
    The record must be pinned for that (the reference's module uses pageable memory,
    HierarchicalGlobalAttentionRouted.py:239); ``pin_memory`` is accepted for signature
    compatibility.  The reference's optional LRU VRAM banks (``vram_cache_chunks``,
    ``vram_summary_chunks``) are not needed: summaries stay resident and opened groups are read
    in place."""

    def __init__(self, *, pin_memory: bool = True, num_layers: int = 0, **kw):
        kw = {k: v for k, v in kw.items() if k in ("compute_device", "policy", "kv_heads",
                                                     "head_dim", "chunk_size",
                                                     "groups_per_chunk", "batch_size", "dtype",
                                                     "initial_capacity")}
        super().__init__(**kw)
        self.staging = ops.DecodeStaging()   # shared by all layers (stream-ordered reuse)

    def _new_record(self, *shape):
        return torch.zeros(*shape, dtype=self.dtype, pin_memory=True)

    def _record_len(self, st):
        return st.n_closed * self.C

    def _ring_slot(self, st, c: int) -> int:
        return c % st.ring_R

    def _ensure_hot(self, st, span: int = 1):
        """Device first-window buffer and a ring of keep_last + span chunk slots: the last window
        plus every chunk a block of `span` chunks writes, so that no segment of the block
        overwrites a chunk an earlier segment still attends to.  Growing re-lays the live chunks
        out for the new ring size."""
        B, KVH, D, C = self.B, self.kvh, self.dh, self.C
        R = max(self.policy.keep_last, 0) + max(span, 1)
        if st.ring_k is not None and st.ring_R >= R:
            return
        rk, rv = self._dev_zeros(B, KVH, R * C, D), self._dev_zeros(B, KVH, R * C, D)
        if st.ring_k is not None:
            lo = self.policy.hot_last_range(st.n_closed)[0]
            for c in range(lo, st.n_closed + 1):
                a, b = (c % st.ring_R) * C, (c % R) * C
                rk[:, :, b:b + C] = st.ring_k[:, :, a:a + C]
                rv[:, :, b:b + C] = st.ring_v[:, :, a:a + C]
        st.ring_k, st.ring_v, st.ring_R = rk, rv, R
        kf = max(self.policy.keep_first, 0)
        if kf and st.first_k is None:
            st.first_k = self._dev_zeros(B, KVH, kf * C, D)
            st.first_v = self._dev_zeros(B, KVH, kf * C, D)

    def prepare_block(self, layer: int, first_chunk: int, last_chunk: int) -> None:
        super().prepare_block(layer, first_chunk, last_chunk)
        self._ensure_hot(self.layer(layer), last_chunk - first_chunk + 1)

    def token_rows(self, layer: int, pos: int, L: int):
        """Ring views [B, KVH, L, Dh] that tokens pos..pos+L-1 (one active chunk) go to."""
        st = self.layer(layer)
        self._ensure_hot(st)
        C = self.C
        s = self._ring_slot(st, pos // C) * C + pos % C
        return st.ring_k[:, :, s:s + L], st.ring_v[:, :, s:s + L]

    def write_tokens(self, layer: int, pos: int, k_rope, v) -> None:
        kd, vd = self.token_rows(layer, pos, k_rope.shape[2])
        kd.copy_(k_rope)
        vd.copy_(v)

    def close_chunk(self, layer: int, n: int) -> None:
        """Chunk n left the active slot: copy it to the host record (async D2H into pinned
        memory) and, inside the first window, to the device first-window buffer."""
        st = self.layer(layer)
        C = self.C
        s = self._ring_slot(st, n) * C
        st.tok_k[:, :, n * C:(n + 1) * C].copy_(st.ring_k[:, :, s:s + C], non_blocking=True)
        st.tok_v[:, :, n * C:(n + 1) * C].copy_(st.ring_v[:, :, s:s + C], non_blocking=True)
        if n < self.policy.keep_first:
            st.first_k[:, :, n * C:(n + 1) * C] = st.ring_k[:, :, s:s + C]
            st.first_v[:, :, n * C:(n + 1) * C] = st.ring_v[:, :, s:s + C]

    def seed(self, layer: int, k_rope, v, n_closed: int) -> None:
        st = self.layer(layer)
        self._ensure_hot(st)
        C = self.C
        S = k_rope.shape[2]
        e = n_closed * C
        if e:
            st.tok_k[:, :, :e].copy_(k_rope[:, :, :e], non_blocking=True)
            st.tok_v[:, :, :e].copy_(v[:, :, :e], non_blocking=True)
        kf = min(self.policy.keep_first, n_closed)
        if kf:
            st.first_k[:, :, :kf * C] = k_rope[:, :, :kf * C]
            st.first_v[:, :, :kf * C] = v[:, :, :kf * C]
        lo = self.policy.hot_last_range(n_closed)[0]
        for c in range(lo, (S + C - 1) // C):
            a, b = c * C, min(S, (c + 1) * C)
            s = self._ring_slot(st, c) * C
            st.ring_k[:, :, s:s + b - a] = k_rope[:, :, a:b]
            st.ring_v[:, :, s:s + b - a] = v[:, :, a:b]

    def sources(self, layer: int):
        st = self.layer(layer)
        return dict(recent_k=st.ring_k, recent_v=st.ring_v, ring_chunks=st.ring_R,
                    first_k=st.first_k, first_v=st.first_v, record_k=st.tok_k,
                    record_v=st.tok_v, record_on_host=True, staging=self.staging)


class _FsLayer:
    """One layer of the on-disk tier: the layer file and its bounded pinned page cache."""

    def __init__(self, path: str, B: int, KVH: int, C: int, D: int, dtype, ram_cap: int):
        self.path = path
        self.fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o600)
        self.B, self.KVH, self.C, self.D, self.dtype = B, KVH, C, D, dtype
        self.esz = torch.tensor([], dtype=dtype).element_size()
        self.chunk_bytes = B * KVH * C * D * self.esz       # K (or V) of one chunk
        self.ram_cap = ram_cap
        self.cap = 0
        self.cache_k = self.cache_v = None                  # pinned [B, KVH, cap*C, D]
        self.slot: Dict[int, int] = {}                      # chunk -> cache slot
        self.lru: "OrderedDict[int, None]" = OrderedDict()
        self.free: List[int] = []
        self.bounce = torch.empty((2, B, KVH, C, D), dtype=dtype, pin_memory=True)
        self.reads = 0

    def close(self) -> None:
        if self.fd is not None:
            os.close(self.fd)
            self.fd = None
            try:
                os.unlink(self.path)
            except OSError:
                pass

    def write(self, c0: int, kv: torch.Tensor) -> None:
        """kv: contiguous host tensor [n, 2, B, KVH, C, D] of chunks c0 .. c0+n-1 (K then V)."""
        mv = memoryview(kv.view(torch.uint8).numpy().reshape(-1))
        off, n = c0 * 2 * self.chunk_bytes, 0
        while n < len(mv):
            n += os.pwrite(self.fd, mv[n:], off + n)
        if hasattr(os, "posix_fadvise"):   # written once, read rarely: keep the page cache small
            os.posix_fadvise(self.fd, off, len(mv), os.POSIX_FADV_DONTNEED)

    def _grow(self, need: int) -> None:
        cap = min(self.ram_cap, max(64, 2 * self.cap, need))
        shape = (self.B, self.KVH, cap * self.C, self.D)
        k = torch.empty(shape, dtype=self.dtype, pin_memory=True)
        v = torch.empty(shape, dtype=self.dtype, pin_memory=True)
        if self.cap:
            k[:, :, :self.cap * self.C].copy_(self.cache_k)
            v[:, :, :self.cap * self.C].copy_(self.cache_v)
        self.free.extend(range(self.cap, cap))
        self.cache_k, self.cache_v, self.cap = k, v, cap

    def ensure_resident(self, chunks: List[int]) -> None:
        """Every chunk of `chunks` in a cache slot; misses are read from the file, evicting the
        least recently used chunks that `chunks` does not need."""
        if len(chunks) > self.ram_cap:
            raise RuntimeError(f"a decode step needs {len(chunks)} distinct chunks, more than the "
                               f"{self.ram_cap}-chunk RAM cache holds; raise ram_budget_gb")
        missing = [c for c in chunks if c not in self.slot]
        if len(self.slot) + len(missing) > self.cap and self.cap < self.ram_cap:
            self._grow(len(self.slot) + len(missing))
        need = set(chunks)
        C = self.C
        for c in missing:
            if self.free:
                s = self.free.pop()
            else:
                victim = next(x for x in self.lru if x not in need)
                del self.lru[victim]
                s = self.slot.pop(victim)
            mv = memoryview(self.bounce.view(torch.uint8).numpy().reshape(-1))
            off, n = c * 2 * self.chunk_bytes, 0
            while n < len(mv):
                r = os.preadv(self.fd, [mv[n:]], off + n)
                if r == 0:
                    raise EOFError(f"chunk {c} is not on disk ({self.path})")
                n += r
            self.cache_k[:, :, s * C:(s + 1) * C].copy_(self.bounce[0])
            self.cache_v[:, :, s * C:(s + 1) * C].copy_(self.bounce[1])
            self.slot[c] = s
            self.reads += 1
        for c in chunks:
            self.lru[c] = None
            self.lru.move_to_end(c)


class FsKVCacheStore(RamKVCacheStore):
    """On-disk tier (fs_kv_cache_store.py:385-818): the closed-token record lives in one file per
    layer, chunk-major with K and V adjacent -- chunk c at byte offset c * 2 * chunk_bytes, its K
    [B, KVH, C, Dh] first, then its V (the reference's layout, :50-64) -- and host RAM holds a
    bounded pinned page cache of chunk slots (LRU).  As in the RAM tier, the GPU keeps the
    summaries, the first window and a ring of the last window.  A decode step makes the chunks of
    its opened groups resident (pread of the misses into the cache), maps group ids to cache
    slots and gathers them into device staging with the RAM tier's kernel.  Closed chunks are
    written once (immutable), so evicting them from RAM is free.  Files live in a private
    directory under ``fs_cache_dir`` (default: the system temporary directory), removed on reset
    and when the store is collected.  ``ram_budget_gb`` bounds the page caches of all
    ``num_layers`` layers together; ``ram_cache_chunks`` sets the per-layer slot count directly.
    The reference's VRAM bank knobs are accepted and unused (summaries are always resident)."""

    def __init__(self, *, ram_budget_gb: float = 12.0, fs_cache_dir: Optional[str] = None,
                 num_layers: int = 0, ram_cache_chunks: Optional[int] = None,
                 vram_cache_chunks: int = 256, vram_summary_chunks: int = 4096,
                 vram_cache_reserve_gb: float = 1.5, **kw):
        super().__init__(num_layers=num_layers, **kw)
        self.ram_budget_gb = ram_budget_gb
        self._dir = tempfile.mkdtemp(prefix="hga_kv_", dir=fs_cache_dir)
        self._finalizer = weakref.finalize(self, shutil.rmtree, self._dir, True)
        esz = torch.tensor([], dtype=self.dtype).element_size()
        chunk_kv = 2 * self.B * self.kvh * self.C * self.dh * esz
        if ram_cache_chunks is None:
            ram_cache_chunks = int(ram_budget_gb * (1 << 30)) // (max(num_layers, 1) * chunk_kv)
        self.ram_cap = max(1, int(ram_cache_chunks))
        self._fs: Dict[int, _FsLayer] = {}

    def fs_layer(self, layer: int) -> _FsLayer:
        f = self._fs.get(layer)
        if f is None:
            f = _FsLayer(os.path.join(self._dir, f"L{layer}.t"), self.B, self.kvh, self.C,
                         self.dh, self.dtype, self.ram_cap)
            self._fs[layer] = f
        return f

    def reset(self) -> None:
        super().reset()
        for f in self._fs.values():
            f.close()
        self._fs.clear()

    def close(self) -> None:
        self.reset()
        self._finalizer()

    def _new_record(self, *shape):   # no host record: the file is the record
        B, KVH, _, D = shape
        return torch.empty((B, KVH, 0, D), dtype=self.dtype)

    def _record_len(self, st):
        return 0

    def close_chunk(self, layer: int, n: int) -> None:
        """Chunk n left the active slot: write it to the layer file (and, inside the first
        window, copy it to the device first-window buffer)."""
        st = self.layer(layer)
        C = self.C
        s = self._ring_slot(st, n) * C
        f = self.fs_layer(layer)
        f.bounce[0].copy_(st.ring_k[:, :, s:s + C])
        f.bounce[1].copy_(st.ring_v[:, :, s:s + C])
        torch.cuda.current_stream(self.compute_device).synchronize()
        f.write(n, f.bounce.unsqueeze(0))
        if n < self.policy.keep_first:
            st.first_k[:, :, n * C:(n + 1) * C] = st.ring_k[:, :, s:s + C]
            st.first_v[:, :, n * C:(n + 1) * C] = st.ring_v[:, :, s:s + C]

    def seed(self, layer: int, k_rope, v, n_closed: int) -> None:
        st = self.layer(layer)
        self._ensure_hot(st)
        B, KVH, C, D = self.B, self.kvh, self.C, self.dh
        S = k_rope.shape[2]
        f = self.fs_layer(layer)
        for c0 in range(0, n_closed, 256):    # chunk-major K/V blocks, <= 256 chunks per write
            n = min(256, n_closed - c0)
            a, e = c0 * C, (c0 + n) * C
            kc = k_rope[:, :, a:e].reshape(B, KVH, n, C, D).permute(2, 0, 1, 3, 4)
            vc = v[:, :, a:e].reshape(B, KVH, n, C, D).permute(2, 0, 1, 3, 4)
            f.write(c0, torch.stack([kc, vc], 1).contiguous().cpu())
        kf = min(self.policy.keep_first, n_closed)
        if kf:
            st.first_k[:, :, :kf * C] = k_rope[:, :, :kf * C]
            st.first_v[:, :, :kf * C] = v[:, :, :kf * C]
        lo = self.policy.hot_last_range(n_closed)[0]
        for c in range((lo), (S + C - 1) // C):
            a, b = c * C, min(S, (c + 1) * C)
            s = self._ring_slot(st, c) * C
            st.ring_k[:, :, s:s + b - a] = k_rope[:, :, a:b]
            st.ring_v[:, :, s:s + b - a] = v[:, :, a:b]

    def prefetch(self, layer: int, chunk_idx: torch.Tensor) -> None:
        """Reads the chunks of chunk_idx that are not in the page cache (when they fit in it)."""
        n_closed = self.num_closed_chunks(layer)
        chunks = [c for c in np.unique(chunk_idx.detach().cpu().numpy()).tolist()
                  if 0 <= c < n_closed]
        f = self.fs_layer(layer)
        if chunks and len(chunks) <= f.ram_cap:
            f.ensure_resident(chunks)

    def _resolve(self, layer: int, open_grp: torch.Tensor):
        """Makes the opened groups' chunks resident and maps group ids (chunk*M + m) to cache
        ids (slot*M + m); returns the mapped list, the cache size in chunks and the cache's K/V
        tensors (the record the gather reads; growing the cache replaces them)."""
        M = self.M
        og = open_grp.cpu().numpy()                    # waits for routing (and earlier gathers)
        valid = og >= 0
        chunks = np.unique(og[valid] // M).tolist()
        f = self.fs_layer(layer)
        f.ensure_resident(chunks)
        mapped = np.full(og.shape, -1, dtype=np.int32)
        if chunks:
            table = np.full(int(max(chunks)) + 1, -1, dtype=np.int64)
            for c in chunks:
                table[c] = f.slot[c]
            mapped[valid] = (table[og[valid] // M] * M + og[valid] % M).astype(np.int32)
        return torch.from_numpy(mapped).to(open_grp.device), f.cap, f.cache_k, f.cache_v

    def sources(self, layer: int):
        st = self.layer(layer)
        f = self.fs_layer(layer)
        if f.cache_k is None:
            f._grow(1)
        return dict(recent_k=st.ring_k, recent_v=st.ring_v, ring_chunks=st.ring_R,
                    first_k=st.first_k, first_v=st.first_v, record_k=f.cache_k,
                    record_v=f.cache_v, record_on_host=True, staging=self.staging,
                    resolve=lambda og, _l=layer: self._resolve(_l, og))


class RoutedKV:
    """Routing result of one block: the index lists the attention kernel reads -- no
    materialised K/V (compare RoutedKV, chunk_router.py:93-162).  ``attend`` computes the exact
    softmax attention over real tokens.  This router builds no group-summary keys
    (``summary_k``/``summary_v``/``summary_mask`` are None, as for the reference's exact
    router), so ``use_summaries`` -- True by default, as in the reference -- selects nothing
    extra (chunk_router.py:128-136); the exact routed module passes False
    (HierarchicalGlobalAttentionRouted.py:172-174).  ``chunked`` results come from the
    vectorized prefill, the others from ``decode_block``."""

    summary_k = None
    summary_v = None
    summary_mask = None

    def __init__(self, hcfg, routing: dict, scale: float, chunk_size: int, *, chunked: bool,
                 k_rope=None, v=None, sources=None, n_closed: int = 0, start_pos: int = 0):
        self.hcfg = hcfg
        self.routing = routing
        self.scale = scale
        self.chunked = chunked
        self.chunk_size = chunk_size
        self.k_rope, self.v = k_rope, v
        self.sources = sources
        self.n_closed, self.start_pos = n_closed, start_pos

    def attend(self, q: torch.Tensor, use_summaries: bool = True) -> torch.Tensor:
        r = self.routing
        if self.chunked:
            return ops.attend_prefill(self.hcfg, q, self.k_rope, self.v, r["open_grp"],
                                      r["open_thr"], r["Kg"])
        src = dict(self.sources)
        staging = src.pop("staging", None)
        resolve = src.pop("resolve", None)
        og = r["open_grp"]
        if staging is None:
            return ops.attend_decode(self.hcfg, q, self.n_closed, self.start_pos, open_grp=og,
                                     open_thr=r["open_thr"], Kg=r["Kg"], **src)
        # host record (or its page cache): the opened groups are copied into device staging on a
        # side stream while the windows and the active chunk are attended on this one
        # (the reference's non-blocking group copy, ram_kv_cache_store.py:578-607)
        og_rec, n_rec, rk, rv = (resolve(og) if resolve is not None else
                                 (og, self.n_closed, src["record_k"], src["record_v"]))
        if self.hcfg.head_dim not in (64, 128):
            # the split kernels (and their phases) cover head_dim 64 and 128 only
            sk, sv, sg = ops.gather_decode(self.hcfg, n_rec, og_rec, r["open_thr"], r["Kg"], rk,
                                           rv, src["record_on_host"], staging, q.shape[1])
            src.update(record_k=sk, record_v=sv, record_on_host=False)
            return ops.attend_decode(self.hcfg, q, self.n_closed, self.start_pos, open_grp=sg,
                                     open_thr=r["open_thr"], Kg=r["Kg"], **src)
        # one library call: gather on its side stream, windows and active chunk meanwhile
        return ops.attend_decode_overlapped(
            self.hcfg, q, self.n_closed, self.start_pos, src["recent_k"], src["recent_v"],
            src["ring_chunks"], src["first_k"], src["first_v"], rk, rv, src["record_on_host"],
            n_rec, og_rec.contiguous(), og.contiguous(), r["open_thr"].contiguous(), r["Kg"],
            staging)

    def attend_dca(self, q_intra: torch.Tensor, q_succ: torch.Tensor, q_inter: torch.Tensor,
                   dca_chunk: int) -> torch.Tensor:
        """Dual Chunk Attention over this block's keys (QwenRoutedAttention._dca_attend,
        qwen_routed_attention.py:244-283): the fp32 query rows RoPE'd at the intra, successive
        and inter positions; each key is scored with the version its DCA chunk selects.  Keys
        are as stored (RoPE'd at pos % dca_chunk by the caller).  Decode-path results only."""
        if self.chunked:
            raise ValueError("DCA attends per chunk: route with return_positions=True")
        r = self.routing
        src = dict(self.sources)
        staging = src.pop("staging", None)
        resolve = src.pop("resolve", None)
        og, op = r["open_grp"], None
        if staging is not None:
            og_rec, n_rec, rk, rv = (resolve(og) if resolve is not None else
                                     (og, self.n_closed, src["record_k"], src["record_v"]))
            sk, sv, sg = ops.gather_decode(self.hcfg, n_rec, og_rec, r["open_thr"], r["Kg"], rk,
                                           rv, src["record_on_host"], staging, q_intra.shape[1])
            src.update(record_k=sk, record_v=sv, record_on_host=False)
            og, op = sg, og
        return ops.attend_decode(self.hcfg, q_intra, self.n_closed, self.start_pos, open_grp=og,
                                 open_thr=r["open_thr"], Kg=r["Kg"],
                                 dca=dict(q_succ=q_succ, q_inter=q_inter, chunk=dca_chunk,
                                          open_pos=op), **src)


class ChunkRouter:
    """Routing engine over a KV store (chunk_router.py:165-516).  Prefill of a fresh multi-chunk
    block runs the vectorized semantics through the HIP kernels; blocks inside one chunk go
    through the decode path."""

    def __init__(self, cfg: RouterConfig, store: KVCacheStore) -> None:
        if not store.policy.first_token_level:
            raise ValueError("ChunkRouter attends the first window at token level "
                             "(ChunkPlacementPolicy(first_token_level=True)); a summary-level "
                             "first window belongs to the summary-attending variant")
        self.cfg = cfg
        self.store = store
        self._hcfg_cache: Dict[Tuple[int, torch.dtype], object] = {}
        self._rot_cache: Dict[object, Tuple[torch.Tensor, torch.Tensor]] = {}   # fp32 rotary rows

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
        ([1,1,S,Dh] or [S,Dh]).  Returns [(routed, lo, hi)] segments: one decode segment for a
        block inside one chunk, one chunk-parallel segment for a fresh multi-chunk block, else
        one decode segment per chunk."""
        C = self.cfg.chunk_size
        S = q.shape[2]
        first_chunk, last_chunk = start_pos // C, (start_pos + S - 1) // C
        # return_positions (the DCA attend variant) takes the per-chunk path, as in the
        # reference (:503-506); key positions are implicit in the routing lists
        vectorized = start_pos == 0 and first_chunk != last_chunk and not return_positions
        if not vectorized:
            self.store.prepare_block(layer, first_chunk, last_chunk)
        if first_chunk == last_chunk:
            return [(self.decode_block(layer, q, k_rope, k_raw, v, start_pos), 0, S)]
        if vectorized:
            return [(self._prefill(layer, q, k_rope, k_raw, v, cos, sin, populate_store), 0, S)]
        segs, p, done = [], start_pos, 0
        while done < S:
            take = min(C - (p % C), S - done)
            sl = slice(done, done + take)
            segs.append((self.decode_block(layer, q[:, :, sl], k_rope[:, :, sl],
                                           k_raw[:, :, sl], v[:, :, sl], p), done, done + take))
            p += take
            done += take
        return segs

    def decode_block(self, layer: int, q: torch.Tensor, k_rope: torch.Tensor,
                     k_raw: torch.Tensor, v: torch.Tensor, start_pos: int) -> RoutedKV:
        """Route L new tokens that all fall inside the active chunk and register them
        (chunk_router.py:279-407); closes the chunk when its last token arrives."""
        cfg = self.cfg
        C = cfg.chunk_size
        B, H, L, D = q.shape
        n, c0 = start_pos // C, start_pos % C
        assert c0 + L <= C, "decode_block must stay within one chunk; feed chunk-by-chunk."
        st = self.store.layer(layer)
        n_closed = st.n_closed
        assert n_closed == n, f"active chunk {n} != closed {n_closed}; out-of-order block"
        st = self.store.ensure_capacity(layer, n_closed + 1)
        hc = self.hcfg(B, q.dtype)
        kd, vd = self.store.token_rows(layer, start_pos, L)
        ops.write_tokens(hc, L, [(k_rope, kd), (v, vd), (k_raw, st.act_kraw[:, :, c0:c0 + L])])
        if n_closed > 0:
            routing = ops.route_decode(hc, q, st.chunk_k, st.group_k, n_closed)
        else:
            e = torch.full((B, H, 1), -1, dtype=torch.int32, device=q.device)
            routing = dict(mid=e, mid_thr=e, open_grp=e, open_thr=e, Kc=0, Kg=0)
        routed = RoutedKV(hc, routing, cfg.scale, C, chunked=False,
                          sources=self.store.sources(layer), n_closed=n_closed,
                          start_pos=start_pos)
        if c0 + L == C:
            self._close_chunk(layer, n, k_rope_chunk=None)
        return routed

    @torch.no_grad()
    def prefill(self, layer: int, q: torch.Tensor, k_rope: torch.Tensor, k_raw: torch.Tensor,
                v: torch.Tensor, start_pos: int = 0) -> torch.Tensor:
        """Stream a prefix chunk by chunk through ``decode_block`` and return the attention
        output [B, H, S, Dh] (ChunkRouter.prefill, chunk_router.py:410-440): each piece ends at
        a chunk boundary, is routed against the chunks closed before it and attended."""
        C = self.cfg.chunk_size
        S = q.shape[2]
        outs, p, done = [], start_pos, 0
        while done < S:
            take = min(C - (p % C), S - done)
            sl = slice(done, done + take)
            routed = self.decode_block(layer, q[:, :, sl], k_rope[:, :, sl], k_raw[:, :, sl],
                                       v[:, :, sl], p)
            outs.append(routed.attend(q[:, :, sl]))
            p += take
            done += take
        return torch.cat(outs, dim=2)

    def _rotary_rows(self, start: int, length: int, device):
        """Rows [start, start + length) of the fp32 rotary table, sliced from a cached table
        (each row depends on its position only, so the values equal rotary_for_positions')."""
        cos, sin = self._rot_cache.get(device, (None, None))
        if cos is None or cos.shape[0] < start + length:
            n = max(2 * (cos.shape[0] if cos is not None else 0), start + length, 4096)
            cos, sin = rotary_for_positions(self.cfg.theta, self.cfg.head_dim, 0, n, device)
            self._rot_cache[device] = (cos, sin)
        return cos[start:start + length], sin[start:start + length]

    def _close_chunk(self, layer: int, n: int, k_rope_chunk=None) -> None:
        """Summaries of the full active chunk n with the fp32 anchor table, then hand it to the
        store (ChunkRouter._close_active_chunk, chunk_router.py:631-657)."""
        cfg = self.cfg
        C, D = cfg.chunk_size, cfg.head_dim
        st = self.store.layer(layer)
        src = self.store.sources(layer)
        if src["ring_chunks"]:
            s = (n % src["ring_chunks"]) * C
        else:
            s = n * C
        krope = src["recent_k"][:, :, s:s + C]
        cf, sf = self._rotary_rows(n * C, C, st.act_kraw.device)
        hc = self.hcfg(st.act_kraw.shape[0], st.act_kraw.dtype)
        ops.summarize(hc, st.act_kraw, krope, cf, sf, pos0=0, chunk_k=st.chunk_k[:, :, n:],
                      group_k=st.group_k[:, :, n:])
        self.store.close_chunk(layer, n)
        st.n_closed = n + 1

    @torch.no_grad()
    def _seed_store_from_block(self, layer: int, k_rope: torch.Tensor, k_raw: torch.Tensor,
                               v: torch.Tensor) -> None:
        """Populate the store from a block at position 0 without routing it
        (chunk_router.py:552-598): store summaries of the closed chunks with the fp32 anchor
        table, the token record, and the partial remainder as the active chunk."""
        cfg = self.cfg
        B, KVH, S, D = k_rope.shape
        C = cfg.chunk_size
        n_closed, N = S // C, (S + C - 1) // C
        st = self.store.layer(layer)
        st.n_closed = 0
        st = self.store.ensure_capacity(layer, N)
        if n_closed:
            e = n_closed * C
            cf, sf = rotary_for_positions(cfg.theta, D, 0, e, k_rope.device)
            ops.summarize(self.hcfg(B, k_rope.dtype), k_raw[:, :, :e], k_rope[:, :, :e], cf, sf,
                          chunk_k=st.chunk_k, group_k=st.group_k)
        self.store.seed(layer, k_rope, v, n_closed)
        if S > n_closed * C:
            st.act_kraw[:, :, :S - n_closed * C] = k_raw[:, :, n_closed * C:]
        st.n_closed = n_closed

    seed_store_from_block = _seed_store_from_block

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
        C = cfg.chunk_size
        n_closed = S // C
        N = (S + C - 1) // C
        pol = self.store.policy
        f_hi, l_lo = pol.hot_first_range(N - 1)[1], pol.hot_last_range(N - 1)[0]
        max_pool = ops.prefill_max_pool(hc)
        if l_lo - f_hi > max_pool:
            raise ValueError(
                f"a fresh block of {S} tokens routes query chunks over pools of up to "
                f"{l_lo - f_hi} chunks; the chunk-parallel router takes {max_pool}. "
                f"Feed the prompt in blocks (the first of at most "
                f"{(max_pool + 1 + max(pol.keep_first, 0) + max(pol.keep_last, 0)) * C} "
                f"tokens, later blocks are routed chunk by chunk).")
        if populate_store:
            st = self.store.layer(layer)
            st.n_closed = 0
            st = self.store.ensure_capacity(layer, N)
        if dt == torch.float32 or not populate_store:
            ck, gk = ops.summarize(hc, k_raw, k_rope, cos_r, sin_r)
            ck_s, gk_s = ck, gk
        else:
            # routing summaries with the activation-dtype table, store summaries with the fp32
            # table written straight into the store tables (one pass over the keys)
            cf, sf = rotary_for_positions(cfg.theta, D, 0, S, dev)
            # same strides as the store tables (one stride set for both output pairs)
            ck = torch.empty_like(st.chunk_k)[:, :, :N]
            gk = torch.empty_like(st.group_k)[:, :, :N]
            ck, gk, ck_s, gk_s = ops.summarize(hc, k_raw, k_rope, cos_r, sin_r, chunk_k=ck,
                                               group_k=gk, cos_b=cf, sin_b=sf,
                                               chunk_k_b=st.chunk_k[:, :, :N],
                                               group_k_b=st.group_k[:, :, :N])
        routing = ops.route_prefill(hc, q, ck, gk, S)
        if populate_store:
            if dt == torch.float32:
                st.chunk_k[:, :, :N] = ck
                st.group_k[:, :, :N] = gk
            self.store.seed(layer, k_rope, v, n_closed)
            rem = S - n_closed * C
            if rem:
                st.act_kraw[:, :, :rem] = k_raw[:, :, n_closed * C:]
            st.n_closed = n_closed
        return RoutedKV(hc, routing, cfg.scale, C, chunked=True, k_rope=k_rope, v=v)
