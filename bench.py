"""Benchmark of the routed exact-token attention path on one MI355X.

Workload (the config the metric is quoted on): one Qwen3-30B-A3B
attention layer, prefill of a 32K-token context, all K/V resident in HBM: batch 1, 32 query
heads, 4 KV heads, head_dim 128, bf16, RoPE base 1e6, q/k ~ N(0,1) after per-head RMSNorm,
v ~ N(0,1); chunk 64, group 16, keep_first 2, keep_last 8, topk_chunks 16, topk_groups 64.

A step is one pass of the hot path over the block with inputs already in HBM: RoPE of q and k,
the module's router call (mixed-RoPE summaries for routing and for the store, two-level
routing, store seeding) and the exact routed attention -- what
HierarchicalGlobalAttentionRouted.forward runs between its projections and o_proj.

Prints one JSON line.  ``--gpus N`` with N > 1 exits: this build targets one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

CFG = dict(B=1, S=32768, H=32, KVH=4, Dh=128, C=64, gs=16, kf=2, kl=8, tc=16, tg=64, theta=1e6)
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16
HBM_PEAK_GBS = 8000.0


def make_inputs(cfg, dev, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    B, S, H, KVH, Dh = cfg["B"], cfg["S"], cfg["H"], cfg["KVH"], cfg["Dh"]

    def rms(x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)

    q_raw = rms(torch.randn(B, H, S, Dh, device=dev, generator=g)).to(torch.bfloat16)
    k_raw = rms(torch.randn(B, KVH, S, Dh, device=dev, generator=g)).to(torch.bfloat16)
    v = torch.randn(B, KVH, S, Dh, device=dev, generator=g).to(torch.bfloat16)
    return q_raw, k_raw, v


def useful_pairs(routing, cfg):
    """Sum over query rows of visible keys (windows + opened groups from their first row +
    causal own chunk), from the routing lists: the attention kernel's algorithmic work."""
    S, C, gs, kf, kl = cfg["S"], cfg["C"], cfg["gs"], cfg["kf"], cfg["kl"]
    N = (S + C - 1) // C
    n = torch.arange(N, device=routing["open_thr"].device)
    f_hi = torch.clamp(n, max=kf) if kf > 0 else torch.zeros_like(n)
    l_lo = torch.minimum(torch.clamp(n - kl, min=kf), n) if kl > 0 else n
    rows = torch.clamp(S - n * C, max=C)
    win = (f_hi + (n - l_lo)) * C * rows                               # [N]
    thr = routing["open_thr"].long()
    ok = thr >= 0
    opened = torch.where(ok, (rows.view(1, 1, N, 1) - thr) * gs, torch.zeros_like(thr)).sum(-1)
    own = rows * (rows + 1) // 2
    B, H = thr.shape[0], thr.shape[1]
    return int((win + own).sum().item()) * B * H + int(opened.sum().item())


def run_gpu(args):
    import hierarchicalglobalattention_amd as hga
    from hierarchicalglobalattention_amd import ops
    from hierarchicalglobalattention_amd.router import (ChunkPlacementPolicy, ChunkRouter,
                                                        RouterConfig, VramKVCacheStore,
                                                        rotary_for_positions)
    hga.lib()
    dev = torch.device("cuda:0")
    c = CFG
    q_raw, k_raw, v = make_inputs(c, dev)
    rcfg = RouterConfig(nhead=c["H"], kv_heads=c["KVH"], head_dim=c["Dh"], chunk_size=c["C"],
                        group_size=c["gs"], topk_chunks=c["tc"], topk_groups=c["tg"],
                        theta=c["theta"])
    pol = ChunkPlacementPolicy(keep_first=c["kf"], keep_last=c["kl"], first_token_level=True)
    store = VramKVCacheStore(compute_device=dev, policy=pol, kv_heads=c["KVH"],
                             head_dim=c["Dh"], chunk_size=c["C"],
                             groups_per_chunk=c["C"] // c["gs"], batch_size=c["B"],
                             dtype=torch.bfloat16)
    router = ChunkRouter(rcfg, store)
    hc = router.hcfg(c["B"], torch.bfloat16)
    cos, sin = rotary_for_positions(c["theta"], c["Dh"], 0, c["S"], dev)
    cos_r, sin_r = cos.to(torch.bfloat16), sin.to(torch.bfloat16)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    tsum = [0.0, 0.0, 0.0]
    state = {}

    def step(timed):
        if timed:
            ev[0].record()
        q = ops.rope(hc, q_raw, cos, sin)
        k_rope = ops.rope(hc, k_raw, cos, sin)
        if timed:
            ev[1].record()
        (routed, lo, hi), = router.route_query_block(0, q, k_rope, k_raw, v, 0, cos=cos_r,
                                                     sin=sin_r)
        if timed:
            ev[2].record()
        out = routed.attend(q)
        if timed:
            ev[3].record()
        state["routing"], state["out"] = routed.routing, out

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    # per-stage timing pass (events between stages), then the clean timed loop
    for _ in range(args.steps):
        step(True)
        torch.cuda.synchronize()
        for i in range(3):
            tsum[i] += ev[i].elapsed_time(ev[i + 1])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(False)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    st = [x / args.steps for x in tsum]
    pairs = useful_pairs(state["routing"], c)
    flops = 4.0 * c["Dh"] * pairs
    attn_tflops = flops / (st[2] * 1e-3) / 1e12
    tokens = c["B"] * c["S"]
    assert torch.isfinite(state["out"].float()).all()
    route_bytes = 2 * (c["B"] * c["H"] * c["S"] * c["Dh"]) + 2 * 2.5 * 2 ** 20
    return dict(ms=ms, stage_ms=st, pairs=pairs, flops=flops, attn_tflops=attn_tflops,
                tokens=tokens, route_bytes=route_bytes)


def cpu_baseline(budget_s: float):
    """The op-faithful torch CPU mirror of the reference path, on a bounded query-chunk slab of
    the same workload, scaled to tokens/s."""
    from oracle import mirror
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    r = mirror.bench_c3_slab(CFG, budget_s=budget_s)
    return dict(value=r["tokens_per_s"], unit="tokens/s", cores=threads, kind="port",
                sample=r["sample"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build targets a single MI355X; multi-GPU runs are out of scope "
              "(see DESIGN.md for how the path would shard)", file=sys.stderr)
        sys.exit(2)
    g = run_gpu(args)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_budget)
    rec = {
        "metric": "routed-attn tokens/s per GPU, Qwen3-30B layer @32K ctx; % HBM/MFMA roofline",
        "value": g["tokens"] / (g["ms"] * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": g["ms"],
        "us_per_layer": g["ms"] * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "qwen3-30b-a3b-attention-layer-prefill-32k", "batch": CFG["B"],
                   "seq_len": CFG["S"], "heads": CFG["H"], "kv_heads": CFG["KVH"],
                   "head_dim": CFG["Dh"], "chunk_size": CFG["C"], "group_size": CFG["gs"],
                   "keep_first": CFG["kf"], "keep_last": CFG["kl"],
                   "topk_chunks": CFG["tc"], "topk_groups": CFG["tg"], "rope_theta": CFG["theta"]},
        "stages_ms": {"rope_q_k": g["stage_ms"][0], "summaries_route_seed": g["stage_ms"][1],
                      "attention": g["stage_ms"][2]},
        "roofline": {"kernel": "attend_mfma_kernel<128>", "bound": "mfma",
                     "achieved": g["attn_tflops"], "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": g["attn_tflops"] / MFMA_BF16_PEAK_TFLOPS,
                     "traffic": None,
                     "algorithmic_flops": g["flops"], "visible_qk_pairs": g["pairs"]},
        "cpu_baseline": cpu,
        "host": {"cpu": platform.processor() or platform.machine(), "torch": torch.__version__},
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
