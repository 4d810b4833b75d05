"""Drop-in routed attention for pretrained Qwen3 (MoE) models on MI355X.

Same classes and functions as the reference
(ExistingModelFineTuning/Qwen3LongContext/qwen_routed_attention.py:94-399):
``QwenRoutedAttention`` replaces a ``Qwen3MoeAttention`` and keeps the original projections and
q/k RMSNorms by reference (no new parameters); only what each query attends to changes.  RoPE
follows transformers' ``apply_rotary_pos_emb`` on the model's cos/sin (every step rounded to the
activation dtype, :176), then the block goes through ``ChunkRouter.route_query_block`` and
``RoutedKV.attend`` on the HIP kernels, then ``o_proj``.  ``replace_qwen_attention_with_router``
/ ``restore_original_attention`` do the model surgery (:331-399).

Cache tiers: ``"vram"`` (``VramKVCacheStore``), ``"ram"`` (``RamKVCacheStore``: the token
record in pinned host memory, each decode step's opened groups gathered over the host link) and
``"fs"`` (``FsKVCacheStore``: the record in per-layer files under ``fs_cache_dir`` with a
pinned page cache bounded by ``ram_budget_gb``).  The reference's VRAM-bank knobs
(``vram_cache_chunks``, ``vram_summary_chunks``, ``vram_cache_reserve_gb``) size VRAM LRU
caches this build has no use for (summaries stay resident); they are accepted and ignored.
"""
from __future__ import annotations

from typing import Any, Optional, Tuple

import torch
import torch.nn as nn

from . import ops
from .router import (ChunkPlacementPolicy, ChunkRouter, FsKVCacheStore, RamKVCacheStore,
                     RouterConfig, VramKVCacheStore)


def _rope_theta(config: Any) -> float:
    """The model's RoPE base: ``config.rope_theta`` (transformers 4) or
    ``config.rope_parameters["rope_theta"]`` (transformers 5), else 1e6 as in the reference
    (qwen_routed_attention.py:146)."""
    theta = getattr(config, "rope_theta", None)
    if theta is None:
        params = getattr(config, "rope_parameters", None) or {}
        theta = params.get("rope_theta", 1_000_000.0)
    return float(theta)


def _dca_rope(positions: torch.Tensor, head_dim: int, theta: float, device: torch.device,
              dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    """Default-RoPE cos/sin rows [len, Dh] for arbitrary (DCA-remapped) positions: the model's
    inv_freq = theta**-(2i/Dh) evaluated at the given positions, in ``dtype``
    (qwen_routed_attention.py:61-77)."""
    half = head_dim // 2
    inv = 1.0 / (theta ** (torch.arange(half, device=device, dtype=torch.float32) / half))
    freqs = positions.to(device=device, dtype=torch.float32).unsqueeze(-1) * inv
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


class QwenRoutedAttention(nn.Module):
    """Replacement for ``Qwen3MoeAttention`` routing through a shared ``ChunkRouter``
    (qwen_routed_attention.py:94-325).  Reuses ``orig``'s ``q_proj/k_proj/v_proj/o_proj`` and
    ``q_norm/k_norm``."""

    def __init__(self, orig: nn.Module, config: Any, *, chunk_size: int = 64,
                 group_size: int = 16, keep_first: int = 2, keep_last: int = 2,
                 topk_chunks: int = 8, topk_groups: int = 32, cache_location: str = "vram",
                 vram_cache_chunks: int = 256, vram_summary_chunks: int = 4096,
                 vram_cache_reserve_gb: float = 1.5, ram_budget_gb: float = 12.0,
                 fs_cache_dir: Optional[str] = None, dca_chunk: int = 0,
                 dca_local: int = 0) -> None:
        super().__init__()
        self.orig = orig
        self.layer_idx = int(getattr(orig, "layer_idx", 0))
        self.num_heads = int(getattr(config, "num_attention_heads"))
        self.num_kv_heads = int(getattr(config, "num_key_value_heads", self.num_heads))
        self.head_dim = int(getattr(config, "head_dim", config.hidden_size // self.num_heads))
        self.num_layers = int(getattr(config, "num_hidden_layers", 0))
        self.chunk_size = chunk_size
        self.cache_location = cache_location     # "vram", "fs", anything else: the RAM tier
        self.vram_cache_chunks = vram_cache_chunks
        self.vram_summary_chunks = vram_summary_chunks
        self.vram_cache_reserve_gb = vram_cache_reserve_gb
        self.ram_budget_gb = ram_budget_gb
        self.fs_cache_dir = fs_cache_dir
        # Dual Chunk Attention (qwen_routed_attention.py:134-141): L_c must be a multiple of the
        # routing chunk so a routing chunk never straddles a DCA boundary.
        if dca_chunk > 0 and dca_chunk % chunk_size != 0:
            raise ValueError(f"dca_chunk ({dca_chunk}) must be a multiple of chunk_size "
                             f"({chunk_size})")
        self.dca_chunk = int(dca_chunk)
        self.dca_local = int(dca_local) if dca_local > 0 else max(1, self.dca_chunk // 5)
        self.dca_ceil = self.dca_chunk + self.dca_local
        self._cfg = RouterConfig(nhead=self.num_heads, kv_heads=self.num_kv_heads,
                                 head_dim=self.head_dim, chunk_size=chunk_size,
                                 group_size=group_size, topk_chunks=topk_chunks,
                                 topk_groups=topk_groups, theta=_rope_theta(config))
        self._policy = ChunkPlacementPolicy(keep_last=keep_last, keep_first=keep_first,
                                            first_token_level=True)

    def forward(self, hidden_states: torch.Tensor,
                position_embeddings: Tuple[torch.Tensor, torch.Tensor],
                attention_mask: Optional[torch.Tensor] = None, past_key_values: Any = None,
                cache_position: Optional[torch.Tensor] = None,
                **kw: Any) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        o = self.orig
        x = hidden_states
        if not x.is_cuda:
            raise RuntimeError("QwenRoutedAttention (MI355X) needs GPU tensors")
        B, S, _ = x.shape
        H, KVH, Dh = self.num_heads, self.num_kv_heads, self.head_dim
        q = o.q_norm(o.q_proj(x).view(B, S, H, Dh)).transpose(1, 2)          # [B,H,S,Dh]
        k_raw = o.k_norm(o.k_proj(x).view(B, S, KVH, Dh)).transpose(1, 2)    # pre-RoPE
        v = o.v_proj(x).view(B, S, KVH, Dh).transpose(1, 2)

        # The decoder passes position_ids (not cache_position) to attention; either gives the
        # block's absolute start (qwen_routed_attention.py:178-186).
        start_pos = 0
        pos_ids = kw.get("position_ids", None)
        if cache_position is not None and cache_position.numel() > 0:
            start_pos = int(cache_position.reshape(-1)[0].item())
        elif pos_ids is not None and pos_ids.numel() > 0:
            start_pos = int(pos_ids.reshape(-1)[0].item())

        router = self._get_router(past_key_values, B, x.dtype, x.device)
        if self.layer_idx == 0 and start_pos == 0:
            router.reset()
        if self.dca_chunk > 0:
            return self._dca_forward(o, q, k_raw, v, start_pos, router, B, S)

        cos, sin = position_embeddings                                       # [B|1, S, Dh]
        cos = cos.reshape(-1, S, Dh)
        sin = sin.reshape(-1, S, Dh)
        hc = router.hcfg(B, x.dtype)
        q_rope, k_rope = ops.rope_qk(hc, q, k_raw, cos, sin, steps_in_dtype=True)
        # summaries anchor with the model's table in the activation dtype (:192-193)
        cos_r, sin_r = cos[:1].to(x.dtype), sin[:1].to(x.dtype)
        segments = router.route_query_block(self.layer_idx, q_rope, k_rope, k_raw, v, start_pos,
                                            cos=cos_r, sin=sin_r)
        out_heads = q_rope.new_empty(B, H, S, Dh)
        for routed, lo, hi in segments:
            out_heads[:, :, lo:hi] = routed.attend(q_rope[:, :, lo:hi], use_summaries=False)
        out = o.o_proj(out_heads.transpose(1, 2).reshape(B, S, H * Dh))
        return out, None

    def _dca_forward(self, o: nn.Module, q: torch.Tensor, k_raw: torch.Tensor, v: torch.Tensor,
                     start_pos: int, router: ChunkRouter, B: int,
                     S: int) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Dual Chunk Attention forward (qwen_routed_attention.py:209-242): keys RoPE'd at the
        intra-chunk position pos % L_c (and stored that way), routing with queries RoPE'd the
        same way, chunk by chunk; attention per key regime (intra / successive / inter)."""
        H, Dh = self.num_heads, self.head_dim
        L_c, ceil, theta = self.dca_chunk, self.dca_ceil, self._cfg.theta
        dev, dt = q.device, q.dtype
        hc = router.hcfg(B, dt)
        pos = torch.arange(start_pos, start_pos + S, device=dev)
        kcos, ksin = _dca_rope(pos % L_c, Dh, theta, dev, dt)
        q_sel, k_dca = ops.rope_qk(hc, q, k_raw, kcos, ksin, steps_in_dtype=True)
        segments = router.route_query_block(self.layer_idx, q_sel, k_dca, k_raw, v, start_pos,
                                            return_positions=True)
        # attention queries in fp32 (:259-266)
        hf = router.hcfg(B, torch.float32)
        qf = q.float()
        qp = pos % L_c
        versions = []
        for p_ in (qp, (qp + L_c).clamp(max=ceil), torch.full_like(qp, ceil)):
            c_, s_ = _dca_rope(p_, Dh, theta, dev, torch.float32)
            versions.append(ops.rope(hf, qf, c_, s_))
        out_heads = q.new_empty(B, H, S, Dh)
        for routed, lo, hi in segments:
            out_heads[:, :, lo:hi] = routed.attend_dca(*(x_[:, :, lo:hi] for x_ in versions),
                                                       L_c)
        out = o.o_proj(out_heads.transpose(1, 2).reshape(B, S, H * Dh))
        return out, None

    def _make_store(self, B: int, dtype: torch.dtype, device: torch.device):
        """VRAM, on-disk or (any other cache_location) pinned-RAM token record
        (qwen_routed_attention.py:286-315)."""
        kwargs = dict(compute_device=device, policy=self._policy, kv_heads=self.num_kv_heads,
                      head_dim=self.head_dim, chunk_size=self.chunk_size,
                      groups_per_chunk=self._cfg.groups_per_chunk, batch_size=B, dtype=dtype)
        if self.cache_location == "vram":
            return VramKVCacheStore(**kwargs)
        if self.cache_location == "fs":
            return FsKVCacheStore(ram_budget_gb=self.ram_budget_gb, fs_cache_dir=self.fs_cache_dir,
                                  num_layers=self.num_layers, **kwargs)
        return RamKVCacheStore(num_layers=self.num_layers, **kwargs)

    def _get_router(self, pkv: Any, B: int, dtype: torch.dtype,
                    device: torch.device) -> ChunkRouter:
        """One router/store shared by all layers, attached to ``past_key_values`` (or to this
        module when no cache object is passed), qwen_routed_attention.py:317-325."""
        holder = pkv if pkv is not None else self
        router = getattr(holder, "_kv_router", None)
        if router is None:
            router = ChunkRouter(self._cfg, self._make_store(B, dtype, device))
            setattr(holder, "_kv_router", router)
        return router


def _iter_attention_layers(model: nn.Module):
    core = getattr(model, "model", None)
    layers = getattr(core, "layers", None)
    if layers is None:
        raise RuntimeError("model.model.layers not found")
    for layer in layers:
        if hasattr(layer, "self_attn"):
            yield layer


def restore_original_attention(model: nn.Module) -> int:
    """Put the original ``self_attn`` modules back; returns how many were restored
    (qwen_routed_attention.py:342-350)."""
    n = 0
    for layer in _iter_attention_layers(model):
        a = layer.self_attn
        if isinstance(a, QwenRoutedAttention):
            layer.self_attn = a.orig
            n += 1
    return n


def replace_qwen_attention_with_router(model: nn.Module, *, keep_first: int = 2,
                                       keep_last: int = 2, topk_chunks: int = 8,
                                       topk_groups: int = 32, chunk_size: int = 64,
                                       group_size: int = 16, cache_location: str = "vram",
                                       vram_cache_chunks: int = 256,
                                       vram_summary_chunks: int = 4096,
                                       vram_cache_reserve_gb: float = 1.5,
                                       ram_budget_gb: float = 12.0,
                                       fs_cache_dir: Optional[str] = None, dca_chunk: int = 0,
                                       dca_local: int = 0) -> int:
    """Replace every ``self_attn`` of ``model.model.layers`` with a ``QwenRoutedAttention``
    (idempotent: earlier replacements are undone first); returns the number replaced
    (qwen_routed_attention.py:353-399)."""
    restore_original_attention(model)
    config = model.config
    count = 0
    for layer in _iter_attention_layers(model):
        layer.self_attn = QwenRoutedAttention(
            layer.self_attn, config, chunk_size=chunk_size, group_size=group_size,
            keep_first=keep_first, keep_last=keep_last, topk_chunks=topk_chunks,
            topk_groups=topk_groups, cache_location=cache_location,
            vram_cache_chunks=vram_cache_chunks, vram_summary_chunks=vram_summary_chunks,
            vram_cache_reserve_gb=vram_cache_reserve_gb, ram_budget_gb=ram_budget_gb,
            fs_cache_dir=fs_cache_dir, dca_chunk=dca_chunk, dca_local=dca_local)
        count += 1
    return count
