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
    state = {}

    def step():
        q, k_rope = ops.rope_qk(hc, q_raw, k_raw, cos, sin)
        (routed, lo, hi), = router.route_query_block(0, q, k_rope, k_raw, v, 0, cos=cos_r,
                                                     sin=sin_r)
        out = routed.attend(q)
        state["routing"], state["out"] = routed.routing, out

    # Per-kernel timing pass: the same launches as step(), issued op by op with HIP events in
    # between (torch's current stream, the stream every op launches on).
    B, S, D, C = c["B"], c["S"], c["Dh"], c["C"]
    N, M = (S + C - 1) // C, C // c["gs"]
    cos_rf, sin_rf = cos_r.float(), sin_r.float()
    names = ["rope_q_k", "summarize", "route", "store_seed", "attention"]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
    tsum = [0.0] * len(names)

    def step_timed():
        st = store.layer(0)
        store.ensure_capacity(0, N)
        ev[0].record()
        q, k_rope = ops.rope_qk(hc, q_raw, k_raw, cos, sin)
        ev[1].record()
        ck, gk, _, _ = ops.summarize(hc, k_raw, k_rope, cos_rf, sin_rf, cos_b=cos, sin_b=sin,
                                     chunk_k_b=st.chunk_k[:, :, :N], group_k_b=st.group_k[:, :, :N])
        ev[2].record()
        r = ops.route_prefill(hc, q, ck, gk, S)
        ev[3].record()
        store.seed(0, k_rope, v, S // C)
        ev[4].record()
        ops.attend_prefill(hc, q, k_rope, v, r["open_grp"], r["open_thr"], r["Kg"])
        ev[5].record()
        return r

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    for _ in range(args.steps):
        r_t = step_timed()
        torch.cuda.synchronize()
        for i in range(len(names)):
            tsum[i] += ev[i].elapsed_time(ev[i + 1])
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    st_ms = {n: x / args.steps for n, x in zip(names, tsum)}
    pairs = useful_pairs(state["routing"], c)
    flops = 4.0 * c["Dh"] * pairs
    assert torch.isfinite(state["out"].float()).all()
    # router: algorithmic HBM bytes (q rows, summaries, routing lists) and score FLOPs
    Kcw, Kgw = r_t["sel_chunk"].shape[-1], r_t["open_grp"].shape[-1]
    route_bytes = (2 * B * c["H"] * S * D + 2 * B * c["KVH"] * N * (1 + M) * D
                   + 4 * B * c["H"] * N * (2 * Kcw + 2 * Kgw + 2))
    n_idx = torch.arange(N)
    f_hi = torch.clamp(n_idx, max=c["kf"])
    l_lo = torch.minimum(torch.clamp(n_idx - c["kl"], min=c["kf"]), n_idx)
    pool = torch.clamp(l_lo - f_hi, min=0)
    rows = torch.clamp(S - n_idx * C, max=C)
    nsel = r_t["n_sel"].long().cpu().sum(dim=(0, 1))             # per chunk, summed over heads
    score_flops = float(2 * D * (c["H"] * B * (rows * pool).sum() + (rows * nsel * M).sum()))
    bwd = None
    if not args.no_backward:
        # training leg: gradient of the routed attention (hga_attend_prefill_bwd) for an upstream
        # gradient, same block and routing; 5 products per visible (query, key) pair
        q, k_rope = ops.rope_qk(hc, q_raw, k_raw, cos, sin)
        # as in training: the forward keeps each row's log-sum-exp for the backward
        lse = torch.empty(B, c["H"], S, dtype=torch.float32, device=dev)
        out = ops.attend_prefill(hc, q, k_rope, v, r_t["open_grp"], r_t["open_thr"], r_t["Kg"],
                                 lse=lse)
        dout = torch.randn_like(out)
        args_b = (hc, q, k_rope, v, out, dout, r_t["open_grp"], r_t["open_thr"], r_t["Kg"])
        ops.attend_prefill_bwd(*args_b, lse=lse)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 3
        e0.record()
        for _ in range(reps):
            ops.attend_prefill_bwd(*args_b, lse=lse)
        e1.record()
        torch.cuda.synchronize()
        bms = e0.elapsed_time(e1) / reps
        bflops = 10.0 * c["Dh"] * pairs
        bwd = {"kernel": "attend_bwd_mfma_kernel<128> (+ accumulator clear and conversion)",
               "ms": bms, "algorithmic_flops": bflops,
               "achieved": bflops / (bms * 1e-3) / 1e12, "unit": "TFLOP/s",
               "frac": bflops / (bms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS}
    return dict(ms=ms, stage_ms=st_ms, pairs=pairs, flops=flops, tokens=B * S,
                route_bytes=route_bytes, score_flops=score_flops, backward=bwd)


def run_c2(reps: int = 5, warmup: int = 2):
    """the 40M-class stack, 8 HGA attention layers (d_model 512, 8 query
    heads, 2 KV heads, head_dim 64, chunk 64, group 16, keep_first 2, keep_last 8, topk_chunks 16,
    topk_groups 64, bf16, projections ~ N(0, 0.02)), prefill of 8192 tokens with inputs ~ N(0,1),
    each layer adding its output to the residual stream that feeds the next (h <- h + attn(h)).  Times the layers' forward (projections, RoPE, router,
    attention, o_proj); the model's MLPs, norms and embeddings are not part of the path."""
    import hierarchicalglobalattention_amd as hga
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    layers = []
    for i in range(8):
        m = hga.HierarchicalGlobalAttentionRouted(d_model=512, nhead=8, kv_heads=2, chunk_size=64,
                                                  group_size=16, topk_chunks=16, topk_groups=64,
                                                  keep_first=2, keep_last=8, theta=1e4,
                                                  layer_idx=i)
        for prm in m.parameters():
            torch.nn.init.normal_(prm, std=0.02)
        layers.append(m.to(dev, torch.bfloat16).eval())
    x0 = torch.randn(1, 8192, 512, device=dev, dtype=torch.bfloat16)

    def stack():
        x = x0
        for m in layers:
            a, _ = m(hidden_states=x)
            x = x + a
        return x

    with torch.no_grad():
        for _ in range(warmup):
            stack()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            out = stack()
        e1.record()
        torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    ms = e0.elapsed_time(e1) / reps
    return dict(layers=8, seq_len=8192, ms_per_stack=ms, ms_per_layer=ms / 8,
                tokens_per_s=8192 / (ms * 1e-3),
                note="8 attention layers (projections + routed attention); the reference's "
                     "published 40M figure times the whole model on other hardware")


def copy_calibration(nbytes: int = 1 << 30, reps: int = 3):
    """A plain device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    dev = torch.device("cuda:0")
    a = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).normal_()
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "reps": reps}))


def h2d_dma_gbs(nbytes: int = 8 << 20, reps: int = 10) -> float:
    """Host-to-device rate of a contiguous copy from pinned memory (the link's DMA rate), the
    reference point for the RAM tier's gather of scattered 4 KiB groups."""
    dev = torch.device("cuda:0")
    h = torch.empty(nbytes * reps, dtype=torch.uint8, pin_memory=True)
    d = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    d.copy_(h[:nbytes], non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        d.copy_(h[i * nbytes:(i + 1) * nbytes], non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    return nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9


DEC_CFG = dict(H=32, KVH=4, Dh=128, C=64, gs=16, kf=2, kl=8, theta=1e6)


def _rms(x):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)


def run_decode(*, ctx, B, tc, tg, tier, steps, warmup, needles=False, seed=0, block=1):
    """Decode of `steps + warmup` steps of `block` tokens per sequence after a seeded c3-style
    context of `ctx` tokens (block 64: the Qwen chat's 64-token prompt blocks).  A step is one
    decode_block (token writes, decode routing, chunk close when the active chunk fills) plus the
    routed attention over its working set, for all B sequences.
    tier "ram": the closed-token record is pinned host memory (the GPU keeps summaries, the
    first window and a ring of last-window chunks); "vram": everything in HBM.  needles: KV heads
    0-1 of every sequence get 4 chunks of keys scaled x8 at seeded random chunk ids."""
    from hierarchicalglobalattention_amd import ops
    from hierarchicalglobalattention_amd.router import (ChunkPlacementPolicy, ChunkRouter,
                                                        RamKVCacheStore, RouterConfig,
                                                        VramKVCacheStore, rotary_for_positions)
    c = DEC_CFG
    dev = torch.device("cuda:0")
    H, KVH, Dh, C = c["H"], c["KVH"], c["Dh"], c["C"]
    T = ctx + (warmup + steps) * block
    g = torch.Generator(device=dev).manual_seed(seed)
    k_raw = _rms(torch.randn(B, KVH, T, Dh, device=dev, generator=g)).to(torch.bfloat16)
    if needles:
        gc = torch.Generator().manual_seed(seed + 1)
        for b in range(B):
            for kvh in range(min(2, KVH)):
                for n in torch.randperm(ctx // C, generator=gc)[:4].tolist():
                    k_raw[b, kvh, n * C:(n + 1) * C] *= 8
    v = torch.randn(B, KVH, T, Dh, device=dev, generator=g).to(torch.bfloat16)
    q_raw = _rms(torch.randn(B, H, (warmup + steps) * block, Dh, device=dev,
                             generator=g)).to(torch.bfloat16)
    rcfg = RouterConfig(nhead=H, kv_heads=KVH, head_dim=Dh, chunk_size=C, group_size=c["gs"],
                        topk_chunks=tc, topk_groups=tg, theta=c["theta"])
    pol = ChunkPlacementPolicy(keep_first=c["kf"], keep_last=c["kl"], first_token_level=True)
    cls = RamKVCacheStore if tier == "ram" else VramKVCacheStore
    store = cls(compute_device=dev, policy=pol, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                groups_per_chunk=C // c["gs"], batch_size=B, dtype=torch.bfloat16,
                initial_capacity=(T + C - 1) // C + 1)
    router = ChunkRouter(rcfg, store)
    hc = router.hcfg(B, torch.bfloat16)
    cos, sin = rotary_for_positions(c["theta"], Dh, 0, T, dev)
    k_rope = ops.rope(hc, k_raw, cos, sin)
    q = ops.rope(hc, q_raw, cos[ctx:], sin[ctx:])
    router.seed_store_from_block(0, k_rope[:, :, :ctx], k_raw[:, :, :ctx], v[:, :, :ctx])
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    stats = dict(open_groups=0, open_groups_union=0, samples=0, gather_ms=0.0, gather_bytes=0)
    gstage = ops.DecodeStaging()
    grp_bytes = c["gs"] * Dh * 2 * 2          # K and V of one 16-token group, bf16

    def step(i, timed):
        p = ctx + i * block
        sl = slice(p, p + block)
        qi = q[:, :, i * block:(i + 1) * block]
        if timed is not None:
            timed[0].record()
        routed = router.decode_block(0, qi, k_rope[:, :, sl], k_raw[:, :, sl], v[:, :, sl], p)
        if timed is not None:
            timed[1].record()
        out = routed.attend(qi)
        if timed is not None:
            timed[2].record()
        return routed, out

    for i in range(warmup):
        step(i, None)
    torch.cuda.synchronize()
    # pass 1: per-stage events; sampled routing statistics
    for j in range(steps):
        routed, out = step(warmup + j, ev[j])
        if j % max(1, steps // 8) == 0 and routed.routing["Kg"] > 0:
            og = routed.routing["open_grp"]
            n_open = int((og >= 0).sum().item())
            u = 0
            rep = H // KVH
            for kvh in range(KVH):
                grp = og[:, kvh * rep:(kvh + 1) * rep].reshape(B, -1)
                for b in range(B):
                    x = grp[b][grp[b] >= 0]
                    u += int(torch.unique(x).numel())
            stats["open_groups"] += n_open
            stats["open_groups_union"] += u
            stats["samples"] += 1
            if tier == "ram":
                # the step's gather again, alone on this stream: its deduplicated bytes (one
                # copy per distinct group and KV head) over its own time
                src = store.sources(0)
                g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                g0.record()
                ops.gather_decode(hc, routed.n_closed, og, routed.routing["open_thr"],
                                  routed.routing["Kg"], src["record_k"], src["record_v"], True,
                                  gstage, H)
                g1.record()
                torch.cuda.synchronize()
                stats["gather_ms"] += g0.elapsed_time(g1)
                stats["gather_bytes"] += u * grp_bytes
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    route_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    attn_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / steps
    # pass 2: clean wall-clock loop over fresh tokens would change the context; re-seed instead
    router.seed_store_from_block(0, k_rope[:, :, :ctx], k_raw[:, :, :ctx], v[:, :, :ctx])
    for i in range(warmup):
        step(i, None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for j in range(steps):
        step(warmup + j, None)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    ns = max(stats["samples"], 1)
    rd = stats["open_groups"] / ns * grp_bytes
    return dict(ctx=ctx, batch=B, block=block, topk_chunks=tc, topk_groups=tg, tier=tier,
                steps=steps, ms_per_step=ms, us_per_step_layer=ms * 1e3,
                tokens_per_s=B * block / (ms * 1e-3),
                device_ms=dict(decode_block=route_ms, attention=attn_ms),
                opened_group_bytes_per_step=rd,
                opened_group_bytes_per_step_dedup=stats["open_groups_union"] / ns * grp_bytes,
                gather_ms=stats["gather_ms"] / ns if tier == "ram" else None,
                h2d_gbs=(stats["gather_bytes"] / (stats["gather_ms"] * 1e-3) / 1e9)
                if tier == "ram" and stats["gather_ms"] > 0 else None)


def _cpu_model():
    """The host CPU's model name (/proc/cpuinfo), else the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _measured_traffic(kernel: str):
    """HBM bytes per launch of a c3 kernel ("route" or "attention"), from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, scaled by the same counters over a plain copy);
    None if absent."""
    path = os.path.join(HERE, "profiles", "c3_route_prefill_traffic.md")
    try:
        for line in open(path):
            if line.startswith(f"traffic_bytes_per_launch_{kernel}:"):
                return float(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


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
    ap.add_argument("--no-decode", action="store_true", help="skip the decode legs (c4, c5)")
    ap.add_argument("--no-backward", action="store_true", help="skip the attention backward leg")
    ap.add_argument("--no-c2", action="store_true", help="skip the 40M 8-layer prefill leg")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 1 GiB device copy (scales the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build targets a single MI355X; multi-GPU runs are out of scope "
              "(one GPU's throughput is the reported value)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    g = run_gpu(args)
    t_route, t_attn = g["stage_ms"]["route"], g["stage_ms"]["attention"]
    attn_tflops = g["flops"] / (t_attn * 1e-3) / 1e12
    route_gbs = g["route_bytes"] / (t_route * 1e-3) / 1e9
    roofline_route = {"kernel": "route_fused_kernel<128, false>",
                      "bound": "hbm",
                      "achieved": route_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": route_gbs / HBM_PEAK_GBS, "traffic": _measured_traffic("route"),
                      "algorithmic_bytes": g["route_bytes"],
                      "score_mfma_tflops": g["score_flops"] / (t_route * 1e-3) / 1e12,
                      "score_mfma_frac": g["score_flops"] / (t_route * 1e-3) / 1e12
                                         / MFMA_BF16_PEAK_TFLOPS}
    if t_route >= t_attn:
        roofline = roofline_route
    else:
        traffic = _measured_traffic("attention")
        roofline = {"kernel": "kv_block_kernel + attend_v3_kernel<128, 2>", "bound": "mfma",
                    "achieved": attn_tflops, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": attn_tflops / MFMA_BF16_PEAK_TFLOPS, "traffic": traffic}
    dec = None
    if not args.no_decode:
        ds = args.decode_steps
        dec = {
            "c4_32k_ram": run_decode(ctx=32768, B=1, tc=16, tg=64, tier="ram", steps=ds,
                                     warmup=8),
            "c4_128k_ram": run_decode(ctx=131072, B=1, tc=16, tg=64, tier="ram", steps=ds,
                                      warmup=8),
            "c5_b64_64k_vram": run_decode(ctx=65536, B=64, tc=32, tg=128, tier="vram",
                                          steps=max(ds // 8, 4), warmup=4, needles=True),
            "c4_32k_ram_64token_blocks": run_decode(ctx=32768, B=1, tc=16, tg=64, tier="ram",
                                                    steps=max(ds // 8, 4), warmup=4, block=64),
            "h2d_dma_gbs_contiguous_8mib": h2d_dma_gbs(),
        }
        torch.cuda.empty_cache()
    c2 = None if args.no_c2 else run_c2()
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
        "stages_ms": g["stage_ms"],
        "roofline": roofline,
        "roofline_route": roofline_route,
        "roofline_attention": {"kernel": "kv_block_kernel + attend_v3_kernel<128, 2>",
                               "bound": "mfma", "achieved": attn_tflops,
                               "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                               "frac": attn_tflops / MFMA_BF16_PEAK_TFLOPS,
                               "algorithmic_flops": g["flops"], "visible_qk_pairs": g["pairs"]},
        "decode": dec,
        "backward": g["backward"],
        "c2_40m_8layer_prefill_8k": c2,
        "cpu_baseline": cpu,
        "host": {"cpu": _cpu_model(), "torch": torch.__version__},
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
