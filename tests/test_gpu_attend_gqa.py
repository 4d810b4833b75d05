"""GPU parity of the bf16 prefill attention kernel that serves several query heads of one KV head
per workgroup (chunk and group sizes multiples of 16, head_dim 64/128), through the C ABI,
against the oracle's routed attention (oracle.attend_prefill, the restatement of
vectorized.py:404-490 / chunk_router.py:149-158) on random routing lists.

The cases cover what the kernel's step schedule depends on: head ratios 1, 2, 3 and 8 (one or two
heads per workgroup), chunks of one, three and four 16-key blocks (odd tile counts in the window
and own-chunk steps), groups of one and two blocks, ragged last chunks, lists of different
lengths within a workgroup's heads (down to none), entries never visible (-1), and both kernel
variants (with and without the log-sum-exp output).  Bar: 2e-2 max / 1e-2 mean abs error (bf16).
"""
import numpy as np
import pytest
import torch

import oracle
from test_oracle_bwd import random_lists

pytestmark = pytest.mark.gpu
hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402

DEV = "cuda"

CASES = [
    # B, H, KVH, S, Dh, C, gs, kf, kl, tg
    (1, 3, 1, 700, 128, 64, 16, 1, 2, 12),    # rep 3: one head per workgroup
    (2, 6, 3, 333, 64, 16, 16, 1, 3, 9),      # one block per chunk, rep 2
    (1, 4, 2, 1100, 128, 64, 32, 2, 2, 20),   # two blocks per group
    (1, 2, 2, 481, 64, 48, 16, 0, 1, 7),      # one head per KV head, three blocks per chunk
    (1, 8, 1, 517, 128, 32, 16, 1, 1, 16),    # rep 8
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"H{c[1]}KVH{c[2]}S{c[3]}D{c[4]}C{c[5]}gs{c[6]}")
@pytest.mark.parametrize("keep_lse", [False, True], ids=["plain", "lse"])
def test_gqa_attention_vs_oracle(case, keep_lse):
    B, H, KVH, S, Dh, C, gs, kf, kl, tg = case
    print(f"[gqa] case {case} lse={keep_lse}", flush=True)
    rng = np.random.default_rng(S + H)
    bf = oracle.bf16_round
    q = bf(rng.standard_normal((B, H, S, Dh)).astype(np.float32))
    k = bf(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    v = bf(rng.standard_normal((B, KVH, S, Dh)).astype(np.float32))
    cfg = ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                          group_size=gs, topk_chunks=max(1, tg), topk_groups=tg, keep_first=kf,
                          keep_last=kl, cutoff_pair=ops.mixed_cutoff_pair(1e4, C, Dh),
                          dtype=torch.bfloat16)
    _, _, Kg = ops.prefill_widths(cfg, S)
    og, ot = random_lists(rng, B, H, S, C, gs, kf, kl, Kg)
    og[:, 0], ot[:, 0] = -1, -1          # head 0 opens nothing; its partner heads do
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV, torch.bfloat16)
    I = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=DEV) if keep_lse else None
    out = ops.attend_prefill(cfg, T(q), T(k), T(v), I(og), I(ot), Kg, lse=lse)
    ref = oracle.attend_prefill(q, k, v, C, gs, kf, kl, og, ot, oracle.attn_scale(Dh),
                                oracle.DT_BF16)
    err = np.abs(out.float().cpu().numpy() - ref)
    assert err.max() <= 2e-2 and err.mean() <= 1e-2, (err.max(), err.mean())
    if keep_lse:
        assert torch.isfinite(lse).all()
