"""Fresh prefill blocks whose query chunks route over pools of more than 512 chunks, through the
C ABI.  The reference's vectorized router has no pool bound (vectorized.py:304-337); the fused
bf16 router takes pools of up to 2048 chunks, the query chunks with pools above 512 in a launch
of their own whose rows merge their survivor lists between 256-candidate segments.

* 64K tokens at C64 / Dh128 (pools up to 1014 chunks, four segments);
* 64K tokens at C32 / Dh64 (pools up to 2038 chunks, eight segments, rows of 32 queries);
* the same with exact ties among wide-pool summaries, so rows fall back to the canonical
  re-rank over their survivor lists and to the full canonical rescoring of a pool.

Lists compared bit for bit with the oracle (query heads reduced so that it finishes in
seconds); the canonical scoring mode, which has no long-pool variant, refuses such blocks."""
import numpy as np
import pytest
import torch

import oracle
from helpers import make_inputs, rope_torch, rotary_table

pytestmark = pytest.mark.gpu

hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import ops  # noqa: E402

DEV = "cuda"

CASES = {
    "64k_c64_dh128": dict(B=1, H=2, KVH=1, S=65536, Dh=128, C=64, gs=16, kf=2, kl=8, tc=16,
                          tg=64, theta=1e6),
    "64k_c32_dh64": dict(B=1, H=2, KVH=1, S=65536, Dh=64, C=32, gs=16, kf=2, kl=8, tc=16,
                         tg=32, theta=1e6),
}


def _pad(a, w):
    a = np.asarray(a)
    return np.concatenate([a, np.full(a.shape[:-1] + (w - a.shape[-1],), -1, np.int32)], -1)


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    w = max(a.shape[-1], b.shape[-1])
    np.testing.assert_array_equal(_pad(a, w), _pad(b, w))


_INPUTS = {}


def _inputs(name):
    if name in _INPUTS:
        return _INPUTS[name]
    c = CASES[name]
    print(f"[long] {name} inputs", flush=True)
    q_raw, k_raw, _ = make_inputs(31, c["B"], c["H"], c["KVH"], c["S"], c["Dh"], torch.bfloat16,
                                  qk_rmsnorm=True)
    cos, sin = rotary_table(c["S"], c["Dh"], c["theta"])
    q = rope_torch(q_raw.float(), cos, sin).to(torch.bfloat16)
    k_rope = rope_torch(k_raw.float(), cos, sin).to(torch.bfloat16)
    cb, sb = cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float()
    cfg = ops.make_config(batch=c["B"], heads=c["H"], kv_heads=c["KVH"], head_dim=c["Dh"],
                          chunk_size=c["C"], group_size=c["gs"], topk_chunks=c["tc"],
                          topk_groups=c["tg"], keep_first=c["kf"], keep_last=c["kl"],
                          cutoff_pair=ops.mixed_cutoff_pair(c["theta"], c["C"], c["Dh"]),
                          dtype=torch.bfloat16)
    ck, gk = ops.summarize(cfg, k_raw.to(DEV), k_rope.to(DEV), cb.to(DEV), sb.to(DEV))
    torch.cuda.synchronize()
    _INPUTS[name] = dict(cfg=cfg, q=q, ck=ck, gk=gk)
    return _INPUTS[name]


def _check(name, d, ck, gk):
    c = CASES[name]
    stats = torch.zeros(4, dtype=torch.int32, device=DEV)
    r = ops.route_prefill(d["cfg"], d["q"].to(DEV), ck, gk, stats=stats)
    torch.cuda.synchronize()
    print(f"[long] {name} routed; oracle", flush=True)
    f = lambda t: t.float().cpu().numpy()
    o_r = oracle.route_prefill_heads(d["q"].float().numpy(), f(ck), f(gk), c["S"], c["C"],
                                     c["gs"], c["kf"], c["kl"], c["tc"], c["tg"],
                                     oracle.attn_scale(c["Dh"]))
    for key in ("sel_chunk", "sel_thr", "open_grp", "open_thr"):
        _same(r[key].cpu().numpy(), o_r[key])
    for key in ("n_sel", "n_open"):
        np.testing.assert_array_equal(r[key].cpu().numpy(), o_r[key])
    return o_r, stats.cpu().tolist()


@pytest.mark.parametrize("name", list(CASES))
def test_long_fresh_block_routing_vs_oracle(name):
    """Every query chunk of a 64K fresh block, the long-pool launch included: lists identical
    to the oracle's."""
    c = CASES[name]
    d = _inputs(name)
    N = c["S"] // c["C"]
    pools = [max(0, oracle.windows(n, c["kf"], c["kl"])[1] - oracle.windows(n, c["kf"], c["kl"])[0])
             for n in range(N)]
    print(f"[long] {name} largest pool {max(pools)}, chunks over 512: "
          f"{sum(p > 512 for p in pools)}", flush=True)
    assert max(pools) > 512
    o_r, stats = _check(name, d, d["ck"], d["gk"])
    print(f"[long] {name} re-ranked rows / pools (stage 1, 2): {stats}", flush=True)
    assert (o_r["n_sel"][..., 30:] == c["tc"]).all()


def test_long_fresh_block_ties():
    """Exact ties among wide-pool summaries: a large-norm chunk summary copied into 60 chunks
    past 600, so rows rank the copies in their top 16 and segment lists hold more tied keys
    than a merge may keep (canonical re-rank over the survivors, or full canonical rescoring of
    pools of up to 2038 chunks), and one group of every chunk copied into another."""
    name = "64k_c32_dh64"
    d = _inputs(name)
    ck, gk = d["ck"].clone(), d["gk"].clone()
    ck[:, :, 2] *= 3
    for n in range(600, 1800, 20):
        ck[:, :, n] = ck[:, :, 2]
    gk[:, :, :, 1] = gk[:, :, :, 0]
    o_r, stats = _check(name, d, ck, gk)
    print(f"[long] ties: re-ranked rows / pools (stage 1, 2): {stats}", flush=True)
    assert np.isin(o_r["sel_chunk"][:, :, 700:], np.arange(600, 1800, 20)).any()
    assert stats[0] > 0


def test_long_pools_refused_by_canonical_and_split_modes():
    """The canonical scoring mode and the split kernels keep the 512-chunk bound and say so."""
    d = _inputs("64k_c64_dh128")
    q = d["q"].to(DEV)
    for kw in (dict(canonical=True), dict(split=True)):
        with pytest.raises(RuntimeError, match="pool"):
            ops.route_prefill(d["cfg"], q, d["ck"], d["gk"], **kw)
