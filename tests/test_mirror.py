"""The op-faithful CPU mirror (the bench's CPU baseline) reproduces the reference's own outputs."""
import numpy as np
import pytest
import torch

from helpers import load_case, prefill_case_inputs
from oracle import mirror


@pytest.mark.parametrize("name", ["c1_ragged", "forced_prev", "ref_shape", "wide_topk", "bf16_mini"])
def test_mirror_matches_reference(name):
    meta, g = load_case(name)
    q, k_rope, k_raw, v, cos, sin = prefill_case_inputs(meta, g)
    dt = torch.bfloat16 if meta["dtype"] == "bfloat16" else torch.float32
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    c4 = torch.from_numpy(cos)[None, None].to(dt)
    s4 = torch.from_numpy(sin)[None, None].to(dt)
    out = mirror.prefill(T(q), T(k_rope), T(k_raw), T(v), c4, s4, C=meta["C"], gs=meta["gs"],
                         keep_first=meta["keep_first"], keep_last=meta["keep_last"],
                         topk_chunks=meta["topk_chunks"], topk_groups=meta["topk_groups"],
                         theta=meta["theta"], slab=3)
    o = out.float().numpy()[:, :, ::meta["out_row_stride"]]
    tol = 2e-2 if dt == torch.bfloat16 else 1e-5
    err = np.abs(o - g["out"])
    assert err.max() <= tol, err.max()


def test_mirror_bench_slab_runs():
    cfg = dict(B=1, S=2048, H=8, KVH=2, Dh=64, C=64, gs=16, kf=2, kl=8, tc=16, tg=64, theta=1e6)
    r = mirror.bench_c3_slab(cfg, budget_s=1.0)
    assert r["tokens_per_s"] > 0 and "query chunks" in r["sample"]
