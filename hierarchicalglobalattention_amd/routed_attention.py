"""Drop-in ``HierarchicalGlobalAttentionRouted`` for MI355X.

Same constructor and ``forward`` contract as the reference module
(ExistingModelFineTuning/HierarchicalGlobalAttentionRouted.py:70-250): projections and optional
per-head RMSNorm in torch, then RoPE, key summaries, two-level routing and exact attention in
the HIP kernels of libhga, then ``o_proj``.  The router/store is attached to
``past_key_value._kv_router`` (or to the module when no cache is given) and reset when
``layer_idx == 0`` and the block starts at position 0, as in the reference (:160-166, :241-250).
"""
from __future__ import annotations

from typing import Any, Optional, Tuple

import torch
import torch.nn as nn

from . import ops
from .router import (ChunkPlacementPolicy, ChunkRouter, FsKVCacheStore, RamKVCacheStore,
                     RouterConfig, VramKVCacheStore)


class RMSNorm(nn.Module):
    """Per-head RMSNorm computed in fp32 (HierarchicalGlobalAttentionRouted.py:56-67)."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        out = self.weight.float() * xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return out.to(dtype=x.dtype)


class HierarchicalGlobalAttentionRouted(nn.Module):
    """Chunk-routed causal self-attention (exact tokens) on the MI355X kernels."""

    def __init__(self, d_model: int, nhead: int = 16, kv_heads: int = 8, dropout: float = 0.0,
                 use_bias_q: bool = False, use_bias_k: bool = False, use_bias_v: bool = False,
                 use_bias_o: bool = False, causal: bool = True, chunk_size: int = 64,
                 group_size: int = 16, topk_chunks: int = 20, topk_groups: int = 32,
                 keep_first: int = 1, keep_last: int = 2, head_dim: Optional[int] = None,
                 qk_norm: bool = False, norm_eps: float = 1e-6, theta: float = 1_000_000.0,
                 layer_idx: int = 0, cache_location: str = "vram", num_layers: int = 0,
                 **kwargs: Any) -> None:
        super().__init__()
        assert nhead % kv_heads == 0
        head_dim = d_model // nhead if head_dim is None else head_dim
        self.d_model, self.nhead, self.kv_heads, self.head_dim = d_model, nhead, kv_heads, head_dim
        self.theta = float(theta)
        self.dropout_p = dropout
        self.layer_idx = layer_idx
        self.cache_location = cache_location
        self.num_layers = num_layers
        self.chunk_size = chunk_size
        self.q_proj = nn.Linear(d_model, nhead * head_dim, bias=use_bias_q)
        self.k_proj = nn.Linear(d_model, kv_heads * head_dim, bias=use_bias_k)
        self.v_proj = nn.Linear(d_model, kv_heads * head_dim, bias=use_bias_v)
        self.o_proj = nn.Linear(nhead * head_dim, d_model, bias=use_bias_o)
        if qk_norm:
            self.q_norm: nn.Module = RMSNorm(head_dim, eps=norm_eps)
            self.k_norm: nn.Module = RMSNorm(head_dim, eps=norm_eps)
        else:
            self.q_norm = nn.Identity()
            self.k_norm = nn.Identity()
        self._cfg = RouterConfig(nhead=nhead, kv_heads=kv_heads, head_dim=head_dim,
                                 chunk_size=chunk_size, group_size=group_size,
                                 topk_chunks=topk_chunks, topk_groups=topk_groups, theta=theta)
        self._policy = ChunkPlacementPolicy(keep_first=keep_first, keep_last=keep_last,
                                            first_token_level=True)

    def forward(self, hidden_states: Optional[torch.Tensor] = None,
                position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                attention_mask: Optional[torch.Tensor] = None, past_key_value: Any = None,
                cache_position: Optional[torch.Tensor] = None, **kw: Any) -> Tuple[torch.Tensor, dict]:
        x = hidden_states
        if not x.is_cuda:
            raise RuntimeError("HierarchicalGlobalAttentionRouted (MI355X) needs GPU tensors")
        B, S, _ = x.shape
        H, KVH, Dh = self.nhead, self.kv_heads, self.head_dim
        q_raw = self.q_norm(self.q_proj(x).view(B, S, H, Dh)).transpose(1, 2)
        k_raw = self.k_norm(self.k_proj(x).view(B, S, KVH, Dh)).transpose(1, 2)
        v = self.v_proj(x).view(B, S, KVH, Dh).transpose(1, 2)

        cos, sin = self._get_rotary_for(position_embeddings, cache_position, B, S, x.device)
        router = self._get_router(past_key_value, B, x.dtype, x.device)
        start_pos = 0
        if cache_position is not None and cache_position.numel() > 0:
            start_pos = int(cache_position.reshape(-1)[0].item())
        if self.layer_idx == 0 and start_pos == 0:
            router.reset()
        hc = router.hcfg(B, x.dtype)
        # training: gradients flow through RoPE and the exact attention (hga_attend_prefill_bwd);
        # routing runs on detached tensors (top-k selections carry no gradient in the reference)
        train = torch.is_grad_enabled() and (q_raw.requires_grad or k_raw.requires_grad or
                                             v.requires_grad)
        if train:
            q_rope = ops.RopeFunction.apply(hc, q_raw, cos[:, 0], sin[:, 0])
            k_rope = ops.RopeFunction.apply(hc, k_raw, cos[:, 0], sin[:, 0])
        else:
            q_rope, k_rope = ops.rope_qk(hc, q_raw, k_raw, cos[:, 0], sin[:, 0])
        cos_r, sin_r = cos[:1].to(x.dtype), sin[:1].to(x.dtype)
        C = self.chunk_size
        if train and not (start_pos == 0 and (S - 1) // C > 0):
            # checked before routing, which writes tokens and may close chunks
            raise NotImplementedError(
                "backward is supported for a fresh multi-chunk block (start_pos 0, "
                "S > chunk_size); decode blocks run without gradients")
        with torch.no_grad():
            segments = router.route_query_block(self.layer_idx, q_rope.detach(), k_rope.detach(),
                                                k_raw.detach(), v.detach(), start_pos,
                                                cos=cos_r, sin=sin_r)
        if train:
            if len(segments) != 1 or not segments[0][0].chunked:
                raise NotImplementedError(
                    "backward is supported for a fresh multi-chunk block (start_pos 0, "
                    "S > chunk_size); decode blocks run without gradients")
            r = segments[0][0].routing
            out_heads = ops.RoutedAttentionFunction.apply(q_rope, k_rope, v, r["open_grp"],
                                                          r["open_thr"], r["Kg"], hc)
        else:
            out_heads = q_rope.new_empty(B, H, S, Dh)
            for routed, lo, hi in segments:
                out_heads[:, :, lo:hi] = routed.attend(q_rope[:, :, lo:hi], use_summaries=False)
        out = self.o_proj(out_heads.transpose(1, 2).contiguous().view(B, S, H * Dh))
        return out, {}

    def _get_rotary_for(self, position_embeddings, cache_position, B: int, S: int, device):
        """fp32 cos/sin [B|1, 1, S, Dh] (HierarchicalGlobalAttentionRouted.py:180-207)."""
        if position_embeddings is not None:
            cos, sin = position_embeddings
            cos = cos.to(device=device, dtype=torch.float32)
            sin = sin.to(device=device, dtype=torch.float32)
            if cos.dim() == 2:
                cos, sin = cos[None, None], sin[None, None]
            elif cos.dim() == 3:
                cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
            if cos.shape[-2] != S:
                cos, sin = cos[:, :, -S:, :], sin[:, :, -S:, :]
            return cos, sin
        pos_start = int(cache_position[0].item()) if cache_position is not None else 0
        cos_full, sin_full = self._get_rotary(pos_start + S, device)
        return cos_full[pos_start:][None, None], sin_full[pos_start:][None, None]

    def _get_rotary(self, seq_len: int, device):
        half = self.head_dim // 2
        inv_freq = 1.0 / (self.theta ** (torch.arange(0, half, device=device,
                                                      dtype=torch.float32) / half))
        t = torch.arange(seq_len, device=device, dtype=torch.float32)
        freqs = torch.einsum("i,j->ij", t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos(), emb.sin()

    def _make_store(self, B: int, dtype, device):
        """VRAM, pinned-RAM or on-disk token record (HierarchicalGlobalAttentionRouted.py:223-240);
        any other cache_location takes the RAM tier, as in the reference."""
        cls = {"vram": VramKVCacheStore, "fs": FsKVCacheStore}.get(self.cache_location,
                                                                   RamKVCacheStore)
        kw = dict(num_layers=self.num_layers) if cls is FsKVCacheStore else {}
        return cls(compute_device=device, policy=self._policy, kv_heads=self.kv_heads,
                   head_dim=self.head_dim, chunk_size=self.chunk_size,
                   groups_per_chunk=self._cfg.groups_per_chunk, batch_size=B, dtype=dtype, **kw)

    def _get_router(self, pkv: Any, B: int, dtype, device) -> ChunkRouter:
        holder = pkv if pkv is not None else self
        router = getattr(holder, "_kv_router", None)
        if router is None:
            router = ChunkRouter(self._cfg, self._make_store(B, dtype, device))
            setattr(holder, "_kv_router", router)
        return router
