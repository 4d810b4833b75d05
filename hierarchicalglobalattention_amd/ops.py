"""Torch-facing wrappers of the libhga entry points.

Each function takes device tensors, checks shapes/dtypes on the host, and launches the HIP
kernel on torch's current stream through the C ABI.  There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import HgaConfig, check, lib

_DT = {torch.float32: _lib.HGA_DTYPE_F32, torch.bfloat16: _lib.HGA_DTYPE_BF16}


def mixed_cutoff_pair(theta: float, chunk_size: int, head_dim: int, threshold: float = 0.5,
                      override=None) -> int:
    """Number of low-index RoPE pairs whose summary is the plain sum of roped keys
    (``_mixed_cutoff_pair``, KvRouter/vectorized.py:146-155, chunk_router.py:717-726)."""
    if override is not None:
        return int(override)
    half = head_dim // 2
    cut = 0
    for i in range(half):
        if max(1, chunk_size - 1) * (1.0 / (theta ** (i / half))) > threshold:
            cut = i + 1
    return cut


def make_config(*, batch, heads, kv_heads, head_dim, chunk_size, group_size, topk_chunks,
                topk_groups, keep_first, keep_last, cutoff_pair, dtype) -> HgaConfig:
    """hga_config for one layer call.  ``scale``/``group_scale`` are the fp32 roundings of
    RouterConfig.scale / group_kv_scale (chunk_router.py:83-90), which is what torch multiplies
    fp32 and bf16 tensors by."""
    if dtype not in _DT:
        raise TypeError(f"unsupported activation dtype {dtype}")
    c = HgaConfig()
    c.batch, c.heads, c.kv_heads, c.head_dim = batch, heads, kv_heads, head_dim
    c.chunk_size, c.group_size = chunk_size, group_size
    c.topk_chunks, c.topk_groups = topk_chunks, topk_groups
    c.keep_first, c.keep_last = keep_first, keep_last
    c.cutoff_pair = cutoff_pair
    c.dtype = _DT[dtype]
    c.scale = float(torch.tensor(head_dim ** -0.5, dtype=torch.float32))
    c.group_scale = float(torch.tensor(1.0 / (group_size + math.sqrt(group_size)),
                                       dtype=torch.float32))
    return c


def _stream() -> int:
    """The current device's current stream (the one torch launches on), as a raw hipStream_t.
    Read through torch's C binding: torch.cuda.current_stream() re-checks device availability
    in Python on every call, several microseconds per launch on the decode path."""
    return torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("hierarchicalglobalattention_amd runs on the GPU only "
                               "(got a CPU tensor); there is no CPU fallback")


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _s4(t):
    """(b, x, s) element strides of a [B, X, S, D] view with a contiguous last dim."""
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError(f"expected a [B, X, S, D] view with contiguous D, got {tuple(t.shape)} "
                         f"strides {t.stride()}")
    return t.stride(0), t.stride(1), t.stride(2)


def prefill_widths(cfg: HgaConfig, S: int):
    n, kc, kg = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    check(lib().hga_prefill_widths(ctypes.byref(cfg), S, ctypes.byref(n), ctypes.byref(kc),
                                   ctypes.byref(kg)), "hga_prefill_widths")
    return n.value, kc.value, kg.value


ROPE_STEPS_IN_DTYPE = 1
# Longest routing pool (chunks) of a query chunk that hga_route_prefill takes: its stage-1 rows
# hold 8 candidates per lane of a wave in registers.  The fused bf16 router (head_dim 64 or 128,
# top-k chunks <= 16, at most 64 group candidates) takes pools of up to PREFILL_MAX_POOL_FUSED.
PREFILL_MAX_POOL = 512
PREFILL_MAX_POOL_FUSED = 2048


def prefill_max_pool(cfg: HgaConfig) -> int:
    """Longest routing pool (chunks) of a query chunk that ``route_prefill`` takes for cfg."""
    M = cfg.chunk_size // cfg.group_size
    fused = (cfg.dtype == _lib.HGA_DTYPE_BF16 and cfg.head_dim in (64, 128) and cfg.topk_chunks <= 16
             and cfg.topk_chunks * M <= 64)
    return PREFILL_MAX_POOL_FUSED if fused else PREFILL_MAX_POOL


def _rope_tables(cos: torch.Tensor, sin: torch.Tensor, B: int, S: int, D: int):
    """fp32 contiguous tables and their batch stride (0: one table shared by the batch).
    Accepted: [S, D] or [Bt, S, D] with Bt 1 or B, sin of cos's shape -- what torch's
    broadcasting of cos/sin against [B, X, S, D] accepts."""
    if tuple(sin.shape) != tuple(cos.shape):
        raise ValueError(f"rotary tables differ in shape: cos {tuple(cos.shape)}, "
                         f"sin {tuple(sin.shape)}")
    if cos.dim() not in (2, 3) or tuple(cos.shape[-2:]) != (S, D) or \
            (cos.dim() == 3 and cos.shape[0] not in (1, B)):
        raise ValueError(f"rotary table {tuple(cos.shape)} is not [{S}, {D}] or [1|{B}, {S}, {D}]")
    cb = 0 if cos.dim() == 2 or cos.shape[0] == 1 else S * D
    return cos.contiguous().float(), sin.contiguous().float(), cb


def rope(cfg: HgaConfig, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         out: torch.Tensor | None = None, steps_in_dtype: bool = False) -> torch.Tensor:
    """Rotate-half RoPE of x [B, X, S, Dh] with tables cos/sin [S, Dh] or [B, S, Dh] (any float
    dtype; used as fp32).  ``steps_in_dtype`` rounds x*cos, rotate_half(x)*sin and their sum to
    x's dtype one by one (transformers' apply_rotary_pos_emb on bf16 tensors); otherwise the
    rotation is computed in fp32 and rounded once."""
    _dev(x, cos, sin)
    B, X, S, D = x.shape
    if out is None:
        out = torch.empty((B, X, S, D), dtype=x.dtype, device=x.device)
    cos, sin, cb = _rope_tables(cos, sin, B, S, D)
    check(lib().hga_rope(ctypes.byref(cfg), X, S, _p(x), *_s4(x), _p(out), *_s4(out), _p(cos),
                         _p(sin), cb, ROPE_STEPS_IN_DTYPE if steps_in_dtype else 0, _stream()),
          "hga_rope")
    return out


def rope_qk(cfg: HgaConfig, q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
            sin: torch.Tensor, steps_in_dtype: bool = False):
    """rope of q [B, heads, S, Dh] and k [B, kv_heads, S, Dh] with the same tables in one
    launch; returns (q_rope, k_rope), equal to two rope calls."""
    _dev(q, k, cos, sin)
    B, H, S, D = q.shape
    if tuple(k.shape) != (B, cfg.kv_heads, S, D) or H != cfg.heads or k.dtype != q.dtype:
        raise ValueError(f"rope_qk: q {tuple(q.shape)} / k {tuple(k.shape)} {k.dtype} do not "
                         f"match the config")
    qo = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    ko = torch.empty(tuple(k.shape), dtype=k.dtype, device=k.device)
    cos, sin, cb = _rope_tables(cos, sin, B, S, D)
    check(lib().hga_rope_qk(ctypes.byref(cfg), S, _p(q), *_s4(q), _p(qo), *_s4(qo), _p(k),
                            *_s4(k), _p(ko), *_s4(ko), _p(cos), _p(sin), cb,
                            ROPE_STEPS_IN_DTYPE if steps_in_dtype else 0, _stream()),
          "hga_rope_qk")
    return qo, ko


def summarize(cfg: HgaConfig, k_raw: torch.Tensor, k_rope: torch.Tensor, cos_tab: torch.Tensor,
              sin_tab: torch.Tensor, pos0: int = 0, chunk_k=None, group_k=None, cos_b=None,
              sin_b=None, chunk_k_b=None, group_k_b=None):
    """Chunk/group key summaries of the block k_raw/k_rope [B, KVH, S, Dh] (block token 0 at
    absolute position pos0).  cos_tab/sin_tab: fp32 [*, Dh] indexed by absolute position.
    Output tensors (optional) are [B, KVH, N', Dh] and [B, KVH, N', M, Dh] views whose first
    N = ceil(S/C) chunk slots receive the block's summaries."""
    _dev(k_raw, k_rope, cos_tab, sin_tab)
    B, KVH, S, D = k_raw.shape
    C, gs = cfg.chunk_size, cfg.group_size
    N, M = (S + C - 1) // C, C // gs
    if chunk_k is None:
        chunk_k = torch.empty((B, KVH, N, D), dtype=k_raw.dtype, device=k_raw.device)
    if group_k is None:
        group_k = torch.empty((B, KVH, N, M, D), dtype=k_raw.dtype, device=k_raw.device)
    two = cos_b is not None
    if two and chunk_k_b is None:
        chunk_k_b = torch.empty_like(chunk_k)
        group_k_b = torch.empty_like(group_k)
    for t in (chunk_k, group_k) + ((chunk_k_b, group_k_b) if two else ()):
        if t.stride(-1) != 1:
            raise ValueError("summary outputs need a contiguous head dim")
    if chunk_k.stride(2) != D or group_k.stride(3) != D or group_k.stride(2) != M * D:
        raise ValueError("summary outputs must be chunk-contiguous")
    if two and (chunk_k_b.stride() != chunk_k.stride() or group_k_b.stride() != group_k.stride()):
        raise ValueError("second summary outputs must share the first ones' strides")
    cos_tab, sin_tab = cos_tab.contiguous().float(), sin_tab.contiguous().float()
    for tab in (cos_tab, sin_tab) + ((cos_b, sin_b) if two else ()):
        if tab.dim() != 2 or tab.shape[1] != D or tab.shape[0] < pos0 + S:
            raise ValueError(f"rotary table {tuple(tab.shape)} must be [>= {pos0 + S}, {D}]")
    if chunk_k.shape[2] < N or group_k.shape[2] < N:
        raise ValueError("summary outputs have fewer chunk slots than the block")
    if two:
        cos_b, sin_b = cos_b.contiguous().float(), sin_b.contiguous().float()
    check(lib().hga_summarize(
        ctypes.byref(cfg), S, pos0, _p(k_raw), *_s4(k_raw), _p(k_rope), *_s4(k_rope),
        _p(cos_tab), _p(sin_tab), _p(chunk_k), chunk_k.stride(0), chunk_k.stride(1),
        _p(group_k), group_k.stride(0), group_k.stride(1), _p(cos_b if two else None),
        _p(sin_b if two else None), _p(chunk_k_b if two else None),
        _p(group_k_b if two else None), _stream()), "hga_summarize")
    if two:
        return chunk_k, group_k, chunk_k_b, group_k_b
    return chunk_k, group_k


def route_prefill(cfg: HgaConfig, q: torch.Tensor, chunk_k: torch.Tensor,
                  group_k: torch.Tensor, S: int | None = None, canonical: bool = False,
                  stats: torch.Tensor | None = None, split: bool = False) -> dict:
    """Two-level routing of a fresh prefill block.  Returns int32 tensors
    sel_chunk/sel_thr [B,H,N,Kc], n_sel [B,H,N], open_grp/open_thr [B,H,N,Kg], n_open [B,H,N]
    (widths at least 1).  ``canonical`` scores every candidate with the fp32 FMA chain;
    ``split`` runs bf16 routing as two kernels instead of the fused one (same lists)."""
    _dev(q, chunk_k, group_k)
    B, H, Sq, D = q.shape
    S = Sq if S is None else S
    N, Kc, Kg = prefill_widths(cfg, S)
    dev = q.device
    r = dict(sel_chunk=torch.empty((B, H, N, max(Kc, 1)), dtype=torch.int32, device=dev),
             sel_thr=torch.empty((B, H, N, max(Kc, 1)), dtype=torch.int32, device=dev),
             n_sel=torch.empty((B, H, N), dtype=torch.int32, device=dev),
             open_grp=torch.empty((B, H, N, max(Kg, 1)), dtype=torch.int32, device=dev),
             open_thr=torch.empty((B, H, N, max(Kg, 1)), dtype=torch.int32, device=dev),
             n_open=torch.empty((B, H, N), dtype=torch.int32, device=dev))
    if chunk_k.stride(-1) != 1 or chunk_k.stride(2) != D or group_k.stride(3) != D or \
            group_k.stride(2) != group_k.shape[3] * D:
        raise ValueError("summaries must be chunk-contiguous with a contiguous head dim")
    flags = (_lib.HGA_ROUTE_CANONICAL if canonical else 0) | (_lib.HGA_ROUTE_SPLIT if split else 0)
    check(lib().hga_route_prefill(
        ctypes.byref(cfg), S, _p(q), *_s4(q), _p(chunk_k), chunk_k.stride(0), chunk_k.stride(1),
        _p(group_k), group_k.stride(0), group_k.stride(1), _p(r["sel_chunk"]), _p(r["sel_thr"]),
        _p(r["n_sel"]), _p(r["open_grp"]), _p(r["open_thr"]), _p(r["n_open"]), flags,
        _p(stats), _stream()), "hga_route_prefill")
    r["Kc"], r["Kg"] = Kc, Kg
    return r


def attend_prefill(cfg: HgaConfig, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   open_grp: torch.Tensor, open_thr: torch.Tensor, Kg: int,
                   out: torch.Tensor | None = None,
                   lse: torch.Tensor | None = None) -> torch.Tensor:
    """Exact attention of q [B,H,S,Dh] over the routed working set (RoPE'd k and v
    [B,KVH,S,Dh]); returns out [B,H,S,Dh] in q's dtype.  lse: optional fp32 [B,H,S] that
    receives each row's log-sum-exp (log2 units of scale*log2(e) scores) for the backward."""
    _dev(q, k, v, open_grp, open_thr, lse)
    B, H, S, D = q.shape
    if out is None:
        out = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    og = open_grp.contiguous()
    ot = open_thr.contiguous()
    ws = attend_prefill_workspace(cfg, S)
    wbuf = torch.empty(max(ws, 16), dtype=torch.uint8, device=q.device) if ws else None
    check(lib().hga_attend_prefill(
        ctypes.byref(cfg), S, _p(q), *_s4(q), _p(k), *_s4(k), _p(v), *_s4(v), _p(og), _p(ot),
        Kg, _p(out), *_s4(out), _p(lse), _p(wbuf), ws, _stream()), "hga_attend_prefill")
    return out


def attend_prefill_workspace(cfg: HgaConfig, S: int) -> int:
    """Scratch bytes hga_attend_prefill needs for a block of S tokens."""
    n = ctypes.c_int64()
    check(lib().hga_attend_prefill_workspace(ctypes.byref(cfg), S, ctypes.byref(n)),
          "hga_attend_prefill_workspace")
    return n.value


def attend_prefill_bwd(cfg: HgaConfig, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       out: torch.Tensor, dout: torch.Tensor, open_grp: torch.Tensor,
                       open_thr: torch.Tensor, Kg: int, lse: torch.Tensor | None = None):
    """Gradients (dq [B,H,S,Dh], dk, dv [B,KVH,S,Dh]) of attend_prefill's output `out` for the
    upstream gradient dout, in q's dtype; lse: attend_prefill's lse output for the same call
    (optional: recomputed when absent)."""
    _dev(q, k, v, out, dout, open_grp, open_thr, lse)
    B, H, S, D = q.shape
    dq = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=q.dtype, device=q.device)
    dv = torch.empty(v.shape, dtype=q.dtype, device=q.device)
    if dout.stride(-1) != 1:
        dout = dout.contiguous()
    og = open_grp.contiguous()
    ot = open_thr.contiguous()
    n = ctypes.c_int64()
    check(lib().hga_attend_prefill_bwd_workspace(ctypes.byref(cfg), S, ctypes.byref(n)),
          "hga_attend_prefill_bwd_workspace")
    ws = torch.empty(max(n.value, 16), dtype=torch.uint8, device=q.device)
    check(lib().hga_attend_prefill_bwd(
        ctypes.byref(cfg), S, _p(q), *_s4(q), _p(k), *_s4(k), _p(v), *_s4(v), _p(out), *_s4(out),
        _p(dout), *_s4(dout), _p(lse), _p(og), _p(ot), Kg, _p(dq), *_s4(dq), _p(dk), *_s4(dk),
        _p(dv),
        *_s4(dv), _p(ws), n.value, _stream()), "hga_attend_prefill_bwd")
    return dq, dk, dv


class RoutedAttentionFunction(torch.autograd.Function):
    """attend_prefill with a backward through hga_attend_prefill_bwd (routing lists are
    constants: the reference's top-k selections carry no gradient)."""

    @staticmethod
    def forward(ctx, q, k, v, open_grp, open_thr, Kg, cfg):
        B, H, S, _ = q.shape
        lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
        out = attend_prefill(cfg, q, k, v, open_grp, open_thr, Kg, lse=lse)
        ctx.save_for_backward(q, k, v, out, open_grp, open_thr, lse)
        ctx.Kg, ctx.cfg = Kg, cfg
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, og, ot, lse = ctx.saved_tensors
        dq, dk, dv = attend_prefill_bwd(ctx.cfg, q, k, v, out, dout, og, ot, ctx.Kg, lse=lse)
        return dq, dk, dv, None, None, None, None


class RopeFunction(torch.autograd.Function):
    """rope with its transpose as the backward: the rotation by -theta (cos, -sin)."""

    @staticmethod
    def forward(ctx, cfg, x, cos, sin):
        ctx.cfg = cfg
        ctx.save_for_backward(cos, sin)
        return rope(cfg, x, cos, sin)

    @staticmethod
    def backward(ctx, g):
        cos, sin = ctx.saved_tensors
        if g.stride(-1) != 1:
            g = g.contiguous()
        return None, rope(ctx.cfg, g, cos, -sin), None, None


def decode_widths(cfg: HgaConfig, n_closed: int):
    kc, kg = ctypes.c_int32(), ctypes.c_int32()
    check(lib().hga_decode_widths(ctypes.byref(cfg), n_closed, ctypes.byref(kc), ctypes.byref(kg)),
          "hga_decode_widths")
    return kc.value, kg.value


def route_decode_workspace(cfg: HgaConfig, L: int, n_closed: int) -> int:
    """Workspace bytes hga_route_decode needs for an L-row block over n_closed chunks."""
    nb = ctypes.c_int64()
    check(lib().hga_route_decode_workspace(ctypes.byref(cfg), L, n_closed, ctypes.byref(nb)),
          "hga_route_decode_workspace")
    return nb.value


def route_decode(cfg: HgaConfig, q: torch.Tensor, chunk_k: torch.Tensor, group_k: torch.Tensor,
                 n_closed: int) -> dict:
    """Decode routing of q [B,H,L,Dh] against the store tables chunk_k [B,KVH,cap,Dh] and
    group_k [B,KVH,cap,M,Dh] (first n_closed chunks valid).  Returns int32 tensors mid/mid_thr
    [B,H,Kc], n_mid [B,H], open_grp/open_thr [B,H,Kg], n_open [B,H] (widths >= 1)."""
    _dev(q, chunk_k, group_k)
    B, H, L, D = q.shape
    Kc, Kg = decode_widths(cfg, n_closed)
    dev = q.device
    r = dict(mid=torch.empty((B, H, max(Kc, 1)), dtype=torch.int32, device=dev),
             mid_thr=torch.empty((B, H, max(Kc, 1)), dtype=torch.int32, device=dev),
             n_mid=torch.empty((B, H), dtype=torch.int32, device=dev),
             open_grp=torch.empty((B, H, max(Kg, 1)), dtype=torch.int32, device=dev),
             open_thr=torch.empty((B, H, max(Kg, 1)), dtype=torch.int32, device=dev),
             n_open=torch.empty((B, H), dtype=torch.int32, device=dev))
    if chunk_k.stride(-1) != 1 or chunk_k.stride(2) != D or group_k.stride(3) != D or \
            group_k.stride(2) != group_k.shape[3] * D:
        raise ValueError("store tables must be chunk-contiguous with a contiguous head dim")
    nb = route_decode_workspace(cfg, L, n_closed)
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=dev)
    check(lib().hga_route_decode(
        ctypes.byref(cfg), L, n_closed, _p(q), *_s4(q), _p(chunk_k), chunk_k.stride(0),
        chunk_k.stride(1), _p(group_k), group_k.stride(0), group_k.stride(1), _p(r["mid"]),
        _p(r["mid_thr"]), _p(r["n_mid"]), _p(r["open_grp"]), _p(r["open_thr"]), _p(r["n_open"]),
        _p(ws), nb, _stream()), "hga_route_decode")
    r["Kc"], r["Kg"] = Kc, Kg
    return r


def gather_decode_sizes(cfg: HgaConfig, Kg: int) -> tuple[int, int, int]:
    """(stage_groups, stage_bytes, scratch_bytes) of hga_gather_decode."""
    u, sb, xb = ctypes.c_int32(), ctypes.c_int64(), ctypes.c_int64()
    check(lib().hga_gather_decode_sizes(ctypes.byref(cfg), Kg, ctypes.byref(u), ctypes.byref(sb),
                                        ctypes.byref(xb)), "hga_gather_decode_sizes")
    return u.value, sb.value, xb.value


class DecodeStaging:
    """Device staging for hga_gather_decode, reused across calls (stream-ordered): K/V
    [B, KVH, U, gs, Dh], staged group slots [B, H, Kg] and the int32 scratch; reallocated only
    when a call needs more."""

    def __init__(self):
        self.key = None

    def get(self, cfg: HgaConfig, Kg: int, H: int, dtype, device):
        U, sbytes, xbytes = gather_decode_sizes(cfg, Kg)
        B, KVH, gs, D = cfg.batch, cfg.kv_heads, cfg.group_size, cfg.head_dim
        key = (B, KVH, H, U, gs, D, max(Kg, 1), dtype, device)
        if self.key != key:
            self.k = torch.empty((B, KVH, U * gs, D), dtype=dtype, device=device)
            self.v = torch.empty_like(self.k)
            self.grp = torch.empty((B, H, max(Kg, 1)), dtype=torch.int32, device=device)
            self.scratch = torch.empty((xbytes + 3) // 4, dtype=torch.int32, device=device)
            self.key = key
        return U, self.k, self.v, self.grp, self.scratch


def gather_decode(cfg: HgaConfig, n_closed: int, open_grp: torch.Tensor, open_thr: torch.Tensor,
                  Kg: int, record_k: torch.Tensor, record_v: torch.Tensor, record_on_host: bool,
                  staging: DecodeStaging, H: int):
    """Copies the step's opened groups (deduplicated per KV head) from the record into device
    staging; returns (stage_k, stage_v, staged_grp): a [B, KVH, U*gs, Dh] record view and the
    open-group list to pass to attend_decode in place of the record and open_grp."""
    _dev(open_grp, open_thr)
    if record_on_host and not record_k.is_pinned():
        raise ValueError("a host record must be pinned memory")
    if record_k.stride() != record_v.stride():
        raise ValueError("K and V of the record must share strides")
    U, sk, sv, sg, scr = staging.get(cfg, Kg, H, record_k.dtype, open_grp.device)
    og = open_grp.contiguous()
    ot = open_thr.contiguous()
    check(lib().hga_gather_decode(
        ctypes.byref(cfg), n_closed, _p(og), _p(ot), Kg, _p(record_k), _p(record_v),
        *_s4(record_k)[:3], 1 if record_on_host else 0, _p(sk), _p(sv), U, _p(sg), _p(scr),
        scr.numel() * 4, _stream()), "hga_gather_decode")
    return sk, sv, sg


def write_tokens(cfg: HgaConfig, L: int, pairs) -> None:
    """One launch copying up to three (src, dst) row sets, each a [B, KVH, L, Dh] view of
    cfg's dtype with a contiguous last dim: a decode block's RoPE'd keys, values and raw keys
    into the token record or ring and the active-chunk buffer.  A pair may be None."""
    pairs = list(pairs)
    if len(pairs) > 3:
        raise ValueError("write_tokens takes at most three row sets")
    want = (cfg.batch, cfg.kv_heads, L, cfg.head_dim)
    src_args, dst_args = [], []
    for pr in pairs + [None] * (3 - len(pairs)):
        if pr is None:
            src_args += [ctypes.c_void_p(0), 0, 0, 0]
            dst_args += [ctypes.c_void_p(0), 0, 0, 0]
            continue
        src, dst = pr
        _dev(src, dst)
        if tuple(src.shape) != want or tuple(dst.shape) != want:
            raise ValueError(f"write_tokens: rows {tuple(src.shape)} -> {tuple(dst.shape)}, "
                             f"expected {want}")
        if src.dtype != dst.dtype or _DT.get(src.dtype) != cfg.dtype:
            raise TypeError(f"write_tokens: {src.dtype} -> {dst.dtype} under a config of "
                            f"another dtype")
        src_args += [_p(src), *_s4(src)]
        dst_args += [_p(dst), *_s4(dst)]
    check(lib().hga_write_tokens(ctypes.byref(cfg), L, *src_args, *dst_args, _stream()),
          "hga_write_tokens")


def attend_decode_overlapped(cfg: HgaConfig, q: torch.Tensor, n_closed: int, start_pos: int,
                             recent_k: torch.Tensor, recent_v: torch.Tensor, ring_chunks: int,
                             first_k, first_v, record_k: torch.Tensor, record_v: torch.Tensor,
                             record_on_host: bool, record_chunks: int, record_grp: torch.Tensor,
                             open_grp: torch.Tensor, open_thr: torch.Tensor, Kg: int,
                             staging: "DecodeStaging") -> torch.Tensor:
    """Decode attention over a host (or page-cache) record in one call
    (hga_attend_decode_overlapped): the opened groups (record_grp: ids into the record of
    record_chunks chunks) are copied into ``staging`` on the library's side stream while the
    windows and the active chunk are attended on the current stream; the staged groups are
    attended after the copy.  Equals attend_decode over the record.  head_dim 64 or 128."""
    _dev(q, recent_k, recent_v, open_grp, open_thr, record_grp)
    B, H, L, D = q.shape
    if first_k is None:
        first_k, first_v = recent_k, recent_v
    if record_on_host and not record_k.is_pinned():
        raise ValueError("a host record must be pinned memory")
    for a_, b_ in ((recent_k, recent_v), (first_k, first_v), (record_k, record_v)):
        if a_.stride() != b_.stride():
            raise ValueError("K and V of a source must share strides")
    if not (open_grp.is_contiguous() and open_thr.is_contiguous() and record_grp.is_contiguous()):
        raise ValueError("the routing lists must be contiguous")
    U, sk, sv, sg, scr = staging.get(cfg, Kg, H, record_k.dtype, q.device)
    out = torch.empty((B, H, L, D), dtype=q.dtype, device=q.device)
    ws = attend_decode_workspace(cfg, L, n_closed, start_pos, Kg, q.device)
    check(lib().hga_attend_decode_overlapped(
        ctypes.byref(cfg), L, n_closed, start_pos, _p(q), *_s4(q), _p(recent_k), _p(recent_v),
        *_s4(recent_k), ring_chunks, _p(first_k), _p(first_v), *_s4(first_k), _p(record_k),
        _p(record_v), *_s4(record_k), 1 if record_on_host else 0, record_chunks, _p(record_grp),
        _p(open_grp), _p(open_thr), Kg, _p(sk), _p(sv), U, _p(sg), _p(scr), scr.numel() * 4,
        _p(out), *_s4(out), _p(ws), ws.numel(), _stream()), "hga_attend_decode_overlapped")
    return out


def attend_decode_workspace(cfg: HgaConfig, L: int, n_closed: int, start_pos: int, Kg: int,
                            device) -> torch.Tensor:
    """A workspace for hga_attend_decode / hga_attend_decode_phase (bytes)."""
    nb = ctypes.c_int64()
    check(lib().hga_attend_decode_workspace(ctypes.byref(cfg), L, n_closed, start_pos, Kg,
                                            ctypes.byref(nb)), "hga_attend_decode_workspace")
    return torch.empty(max(nb.value, 16), dtype=torch.uint8, device=device)


def attend_decode_noalloc(cfg: HgaConfig, q: torch.Tensor, n_closed: int, start_pos: int,
                          recent_k: torch.Tensor, recent_v: torch.Tensor, ring_chunks: int,
                          first_k, first_v, record_k, record_v, record_on_host: bool,
                          open_grp: torch.Tensor, open_thr: torch.Tensor, Kg: int,
                          out: torch.Tensor) -> torch.Tensor:
    """attend_decode (phase 0, no DCA) through hga_attend_decode_noalloc: the split partials go
    to the library's static per-device scratch (32 MiB), so neither this call nor the library
    allocates device memory.  ``out`` is required, the lists must be contiguous; calls that
    overlap on one device race on the scratch."""
    _dev(q, recent_k, recent_v, open_grp, open_thr, out)
    B, H, L, D = q.shape
    if first_k is None:
        first_k, first_v = recent_k, recent_v
    if record_k is None:
        record_k, record_v = recent_k, recent_v
    if record_on_host and not record_k.is_pinned():
        raise ValueError("a host record must be pinned memory")
    if not record_on_host:
        _dev(first_k, first_v, record_k, record_v)
    for a_, b_ in ((recent_k, recent_v), (first_k, first_v), (record_k, record_v)):
        if a_.stride() != b_.stride():
            raise ValueError("K and V of a source must share strides")
    if not (open_grp.is_contiguous() and open_thr.is_contiguous()):
        raise ValueError("open_grp / open_thr must be contiguous")
    check(lib().hga_attend_decode_noalloc(
        ctypes.byref(cfg), L, n_closed, start_pos, _p(q), *_s4(q), _p(recent_k), _p(recent_v),
        *_s4(recent_k), ring_chunks, _p(first_k), _p(first_v), *_s4(first_k), _p(record_k),
        _p(record_v), *_s4(record_k), 1 if record_on_host else 0, _p(open_grp), _p(open_thr), Kg,
        _p(out), *_s4(out), _stream()), "hga_attend_decode_noalloc")
    return out




def attend_decode(cfg: HgaConfig, q: torch.Tensor, n_closed: int, start_pos: int,
                  recent_k: torch.Tensor, recent_v: torch.Tensor, ring_chunks: int,
                  first_k, first_v, record_k, record_v, record_on_host: bool,
                  open_grp: torch.Tensor, open_thr: torch.Tensor, Kg: int,
                  out: torch.Tensor | None = None, dca: dict | None = None, phase: int = 0,
                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention of q [B,H,L,Dh] (rows at start_pos..start_pos+L-1).  Token sources are
    [B,KVH,T,Dh] views: ``recent`` (positions >= the last window, optionally a ring of
    ring_chunks chunks), ``first`` (the first window) and ``record`` (the closed-token record
    read for opened groups; a pinned host tensor when record_on_host).

    ``dca`` selects Dual Chunk Attention: q is then the fp32 intra version and ``dca`` holds
    ``q_succ``/``q_inter`` (fp32, q's shape and strides), ``chunk`` (the DCA chunk length) and
    ``open_pos`` (the opened groups' own ids when open_grp indexes a staging record, else None);
    the output has the keys' dtype.

    ``phase`` 1 attends the windows and the active chunk into ``workspace`` (the record is not
    read), phase 2 (same workspace) the opened groups, and writes ``out``
    (hga_attend_decode_phase); 0 does both in one call."""
    _dev(q, recent_k, recent_v, open_grp, open_thr)
    B, H, L, D = q.shape
    if out is None:
        out = torch.empty((B, H, L, D), dtype=recent_k.dtype if dca else q.dtype,
                          device=q.device)
    if first_k is None:
        first_k, first_v = recent_k, recent_v
    if record_k is None:
        record_k, record_v = recent_k, recent_v
    if record_on_host and not record_k.is_pinned():
        raise ValueError("a host record must be pinned memory")
    if not record_on_host:
        _dev(first_k, first_v, record_k, record_v)
    for a_, b_ in ((recent_k, recent_v), (first_k, first_v), (record_k, record_v)):
        if a_.stride() != b_.stride():
            raise ValueError("K and V of a source must share strides")
    og = open_grp.contiguous()
    ot = open_thr.contiguous()
    ws = workspace if workspace is not None else attend_decode_workspace(
        cfg, L, n_closed, start_pos, Kg, q.device)
    src = (_p(recent_k), _p(recent_v), *_s4(recent_k), ring_chunks, _p(first_k), _p(first_v),
           *_s4(first_k), _p(record_k), _p(record_v), *_s4(record_k),
           1 if record_on_host else 0)
    if phase:
        if dca is not None:
            raise ValueError("phased decode attention is not available for DCA")
        check(lib().hga_attend_decode_phase(
            ctypes.byref(cfg), L, n_closed, start_pos, _p(q), *_s4(q), *src, _p(og), _p(ot), Kg,
            _p(out), *_s4(out), int(phase), _p(ws), ws.numel(), _stream()),
            "hga_attend_decode_phase")
        return out
    if dca is None:
        check(lib().hga_attend_decode(
            ctypes.byref(cfg), L, n_closed, start_pos, _p(q), *_s4(q), *src, _p(og), _p(ot), Kg,
            _p(out), *_s4(out), _p(ws), ws.numel(), _stream()), "hga_attend_decode")
        return out
    qs, qt = dca["q_succ"], dca["q_inter"]
    _dev(qs, qt)
    for t in (q, qs, qt):
        if t.dtype != torch.float32 or t.stride() != q.stride() or t.shape != q.shape:
            raise ValueError("DCA query versions must be fp32 views of one shape and strides")
    op = dca.get("open_pos")
    op = op.contiguous() if op is not None else None
    check(lib().hga_attend_decode_dca(
        ctypes.byref(cfg), L, n_closed, start_pos, _p(q), _p(qs), _p(qt), *_s4(q),
        int(dca["chunk"]), *src, _p(og), _p(op) if op is not None else None, _p(ot), Kg,
        _p(out), *_s4(out), _p(ws), ws.numel(), _stream()), "hga_attend_decode_dca")
    return out
