"""On-disk KV tier (fs_kv_cache_store.py:385-818) on the GPU.

* The layer file holds chunk c at byte offset c * 2 * chunk_bytes, K [B, KVH, C, Dh] first, then
  V -- the reference's layout (:50-64).
* Prefill + many single-token decode steps through ChunkRouter with an FsKVCacheStore whose RAM
  cache holds fewer chunks than the context (so chunks are evicted and read back) give outputs
  bit-identical to the VRAM store's, and identical routing.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
hga = pytest.importorskip("hierarchicalglobalattention_amd")
from hierarchicalglobalattention_amd import router as hr  # noqa: E402

DEV = torch.device("cuda:0")


def _router(store_cls, **kw):
    cfg = hr.RouterConfig(nhead=8, kv_heads=2, head_dim=128, chunk_size=64, group_size=16,
                          topk_chunks=4, topk_groups=16, theta=1e6)
    pol = hr.ChunkPlacementPolicy(keep_first=1, keep_last=2, first_token_level=True)
    store = store_cls(compute_device=DEV, policy=pol, kv_heads=2, head_dim=128, chunk_size=64,
                      groups_per_chunk=4, batch_size=1, dtype=torch.bfloat16, **kw)
    return hr.ChunkRouter(cfg, store)


def _inputs(S, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, 8, S, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, S, 128, generator=g).to(torch.bfloat16)
    kr = torch.randn(1, 2, S, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 2, S, 128, generator=g).to(torch.bfloat16)
    return q.to(DEV), k.to(DEV), kr.to(DEV), v.to(DEV)


def _run(r, q, k, kr, v, S0, steps, spy):
    cos, sin = hr.rotary_for_positions(1e6, 128, 0, S0, DEV)
    outs = []
    with torch.no_grad():
        (rk, lo, hi), = r.route_query_block(0, q[:, :, :S0], k[:, :, :S0], kr[:, :, :S0],
                                            v[:, :, :S0], 0, cos=cos.to(torch.bfloat16),
                                            sin=sin.to(torch.bfloat16))
        outs.append(rk.attend(q[:, :, :S0]))
        for p in range(S0, S0 + steps):
            sl = slice(p, p + 1)
            (rk, lo, hi), = r.route_query_block(0, q[:, :, sl], k[:, :, sl], kr[:, :, sl],
                                                v[:, :, sl], p)
            spy.append(rk.routing["open_grp"].cpu().clone())
            outs.append(rk.attend(q[:, :, sl]))
    torch.cuda.synchronize()
    return torch.cat(outs, 2).cpu()


def test_fs_file_layout(tmp_path):
    r = _router(hr.FsKVCacheStore, fs_cache_dir=str(tmp_path), ram_cache_chunks=16)
    S0 = 64 * 10 + 17
    q, k, kr, v = _inputs(S0, 3)
    _run(r, q, k, kr, v, S0, 0, [])
    f = r.store.fs_layer(0)
    data = open(f.path, "rb").read()
    cb = 2 * 64 * 128 * 2                      # B * KVH * C * Dh * bf16
    assert len(data) == 10 * 2 * cb            # the 10 closed chunks
    raw = np.frombuffer(data, dtype=np.uint16).reshape(10, 2, 1, 2, 64, 128)
    kk = k.cpu().view(torch.int16).numpy().view(np.uint16)
    vv = v.cpu().view(torch.int16).numpy().view(np.uint16)
    for c in range(10):
        np.testing.assert_array_equal(raw[c, 0], kk[:, :, 64 * c:64 * (c + 1)])
        np.testing.assert_array_equal(raw[c, 1], vv[:, :, 64 * c:64 * (c + 1)])
    path = f.path
    r.store.reset()
    assert not os.path.exists(path)


def test_fs_decode_equals_vram(tmp_path):
    print("[fs] decode vs vram", flush=True)
    S0, steps = 64 * 120 + 5, 200
    q, k, kr, v = _inputs(S0 + steps, 7)
    ra = _router(hr.VramKVCacheStore)
    rb = _router(hr.FsKVCacheStore, fs_cache_dir=str(tmp_path), ram_cache_chunks=40)
    sa, sb = [], []
    a = _run(ra, q, k, kr, v, S0, steps, sa)
    b = _run(rb, q, k, kr, v, S0, steps, sb)
    for x, y in zip(sa, sb):
        assert torch.equal(x, y)
    assert torch.equal(a, b)
    f = rb.store.fs_layer(0)
    distinct = len({int(g) // 4 for s in sb for g in s.flatten().tolist() if g >= 0})
    print(f"  chunk reads {f.reads}, distinct chunks opened {distinct}, cache {f.cap} slots")
    assert f.cap == 40 and f.reads > distinct     # evicted chunks were read back
    # chunks closed during decode were written to the file
    assert os.path.getsize(f.path) == (S0 + steps) // 64 * 2 * (2 * 64 * 128 * 2)
