"""hga_attend_decode_noalloc, the decode attention entry point that allocates nothing (its split
partials live in a static per-device scratch array), against hga_attend_decode with a caller
workspace: bit-identical outputs on two calls in a row, the second on a smaller block (the
scratch keeps the first call's partials), and a clear error for blocks whose partials exceed
the scratch.  No counterpart in the reference: for callers that cannot allocate device memory
(graph capture, serving loops)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402

DEV = "cuda"


def _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt):
    return ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                           group_size=gs, topk_chunks=tc, topk_groups=tg, keep_first=kf,
                           keep_last=kl, cutoff_pair=ops.mixed_cutoff_pair(1e6, C, Dh), dtype=dt)


def _case(seed, B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, c0, L, dt):
    """Routed decode inputs on the device: history k/v, block q, opened lists."""
    gen = torch.Generator().manual_seed(seed)
    M = C // gs
    start = n_closed * C + c0
    T = start + L
    k = (torch.randn(B, KVH, T, Dh, generator=gen) * 0.5).to(dt).to(DEV)
    v = torch.randn(B, KVH, T, Dh, generator=gen).to(dt).to(DEV)
    q = torch.randn(B, H, L, Dh, generator=gen).to(dt).to(DEV)
    ck = torch.randn(B, KVH, n_closed, Dh, generator=gen).to(dt).to(DEV)
    gk = torch.randn(B, KVH, n_closed, M, Dh, generator=gen).to(dt).to(DEV)
    cfg = _cfg(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt)
    r = ops.route_decode(cfg, q, ck, gk, n_closed)
    return dict(cfg=cfg, q=q, k=k, v=v, n_closed=n_closed, start=start, og=r["open_grp"],
                ot=r["open_thr"], Kg=r["Kg"])


CASES = [
    # B, H, KVH, Dh, C, gs, tc, tg, kf, kl, n_closed, c0, L, dtype
    (2, 8, 2, 128, 64, 16, 16, 64, 2, 8, 200, 7, 20, torch.bfloat16),   # MFMA split kernel
    (1, 4, 2, 64, 32, 8, 5, 9, 1, 3, 40, 30, 1, torch.float32),          # smaller, one row
]


def test_noalloc_matches_workspace_entry_point_twice():
    outs = []
    for i, case in enumerate(CASES):
        print(f"[noalloc] call {i} {case}", flush=True)
        d = _case(100 + i, *case)
        q, k, v = d["q"], d["k"], d["v"]
        ref = ops.attend_decode(d["cfg"], q, d["n_closed"], d["start"], k, v, 0, k, v, k, v,
                                False, d["og"], d["ot"], d["Kg"])
        out = torch.full_like(q, float("nan"))
        ops.attend_decode_noalloc(d["cfg"], q, d["n_closed"], d["start"], k, v, 0, k, v, k, v,
                                  False, d["og"].contiguous(), d["ot"].contiguous(), d["Kg"], out)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert torch.equal(out, ref)
        outs.append(out)
    assert outs[1].numel() < outs[0].numel()


def test_noalloc_refuses_blocks_beyond_the_scratch():
    """B64 x H32 x 64 rows: about 450 MiB of partials, beyond the 32 MiB scratch; the call is
    refused before any kernel runs."""
    B, H, KVH, Dh, C, L, n_closed = 64, 32, 4, 128, 64, 64, 100
    cfg = _cfg(B, H, KVH, Dh, C, 16, 16, 64, 2, 8, torch.bfloat16)
    q = torch.zeros(B, H, L, Dh, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(B, KVH, C, Dh, dtype=torch.bfloat16, device=DEV)
    og = torch.full((B, H, 64), -1, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    with pytest.raises(RuntimeError, match="static scratch"):
        ops.attend_decode_noalloc(cfg, q, n_closed, n_closed * C, kv, kv, 0, kv, kv, kv, kv,
                                  False, og, og, 64, out)
