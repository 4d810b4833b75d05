"""CPU checks of the C ABI: the library loads, exports every function include/hga.h declares,
and its host-side validation and size logic behave (no kernel is launched)."""
import ctypes
import os
import re

import pytest

import oracle
from hierarchicalglobalattention_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "hga.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hga_[a-z_0-9]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert "hga_route_prefill" in names and len(names) >= 7
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/hga.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_widths():
    lib = _lib.lib()
    assert lib.hga_version() >= 100
    for S, C, gs, tc, tg in [(2048, 64, 16, 4, 8), (32768, 64, 16, 16, 64), (37, 8, 4, 3, 4),
                             (100, 64, 16, 0, 8), (64, 64, 16, 20, 32)]:
        cfg = ops.make_config(batch=1, heads=8, kv_heads=2, head_dim=64, chunk_size=C,
                              group_size=gs, topk_chunks=tc, topk_groups=tg, keep_first=1,
                              keep_last=2, cutoff_pair=3, dtype=__import__("torch").bfloat16)
        N, Kc, Kg = ops.prefill_widths(cfg, S)
        assert (N, Kc, Kg) == tuple(oracle.sizes(S, C, gs, tc, tg)[i] for i in (0, 2, 3))


def test_errors_reported_without_launch():
    import torch
    lib = _lib.lib()
    cfg = ops.make_config(batch=1, heads=6, kv_heads=4, head_dim=64, chunk_size=64,
                          group_size=16, topk_chunks=4, topk_groups=8, keep_first=1, keep_last=2,
                          cutoff_pair=3, dtype=torch.float32)
    rc = lib.hga_prefill_widths(ctypes.byref(cfg), 100, None, None, None)
    assert rc == -1 and b"kv_heads" in lib.hga_last_error()
    cfg.kv_heads = 2
    cfg.head_dim = 96
    assert lib.hga_prefill_widths(ctypes.byref(cfg), 100, None, None, None) == -2
    cfg.head_dim = 64
    z = ctypes.c_void_p(0)
    rc = lib.hga_rope(ctypes.byref(cfg), 2, 10, z, 0, 0, 0, z, 0, 0, 0, z, z, 0, 0, z)
    assert rc == -1 and b"NULL" in lib.hga_last_error()
    with pytest.raises(_lib.HgaError):
        _lib.check(lib.hga_rope(ctypes.byref(cfg), 2, 10, z, 0, 0, 0, z, 0, 0, 0, z, z, 0, 0, z),
                   "hga_rope")


def test_cpu_tensors_are_rejected():
    import torch
    cfg = ops.make_config(batch=1, heads=2, kv_heads=1, head_dim=64, chunk_size=64,
                          group_size=16, topk_chunks=4, topk_groups=8, keep_first=1, keep_last=2,
                          cutoff_pair=3, dtype=torch.float32)
    x = torch.zeros(1, 2, 8, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.rope(cfg, x, torch.zeros(8, 64), torch.zeros(8, 64))


def test_cutoff_pair_closed_forms():
    """Closed-form values of the mixed-RoPE cutoff (chunk_router.py:717-726)."""
    for theta, C, Dh, want in [(1e4, 64, 64, 17), (1e6, 64, 128, 23), (1e4, 8, 16, 3)]:
        assert ops.mixed_cutoff_pair(theta, C, Dh) == want
        assert oracle.cutoff_pair(theta, C, Dh) == want


def test_workspace_queries_and_checks_without_launch():
    """Host-side sizing of the decode router's and the backward's workspaces, and the argument
    checks that run before any kernel (fake device pointers are never dereferenced)."""
    import torch
    lib = _lib.lib()

    def cfg_of(B, H, KVH, Dh, C, gs, tc, tg, kf, kl, dt=torch.bfloat16):
        return ops.make_config(batch=B, heads=H, kv_heads=KVH, head_dim=Dh, chunk_size=C,
                               group_size=gs, topk_chunks=tc, topk_groups=tg, keep_first=kf,
                               keep_last=kl, cutoff_pair=3, dtype=dt)

    def route_ws(cfg, L, n):
        nb = ctypes.c_int64(-1)
        rc = lib.hga_route_decode_workspace(ctypes.byref(cfg), L, n, ctypes.byref(nb))
        return rc, nb.value

    cfg = cfg_of(1, 32, 4, 128, 64, 16, 16, 64, 2, 8)
    assert route_ws(cfg, 1, 10) == (0, 0)                 # pool inside the windows: nothing routed
    sizes = [route_ws(cfg, L, n)[1] for L, n in [(1, 511), (1, 2047), (64, 2047), (64, 8191)]]
    assert all(b > 0 for b in sizes) and sizes == sorted(sizes)
    # a multi-row block's scores of every pool chunk are part of it: at least B*H*L*pool floats
    assert sizes[2] >= 32 * 64 * (2047 - 10) * 4 > 2 * sizes[1]
    assert route_ws(cfg, 65, 100)[0] == -1                 # rows outside [1, 64]
    # too small a workspace is refused before anything is launched
    fake = ctypes.c_void_p(1 << 20)
    need = route_ws(cfg, 4, 700)[1]
    rc = lib.hga_route_decode(ctypes.byref(cfg), 4, 700, fake, 0, 0, 128, fake, 0, 0, fake, 0, 0,
                              fake, fake, fake, fake, fake, fake, fake, need - 4, None)
    assert rc == -1 and b"workspace" in lib.hga_last_error()

    # backward: fp32 dk/dv accumulators, 2*B*KVH*S*Dh floats
    for B, KVH, S, Dh in [(1, 4, 32768, 128), (2, 1, 77, 16)]:
        c = cfg_of(B, 4 * KVH, KVH, Dh, 64, 16, 16, 64, 2, 8)
        nb = ctypes.c_int64()
        assert lib.hga_attend_prefill_bwd_workspace(ctypes.byref(c), S, ctypes.byref(nb)) == 0
        assert nb.value == 2 * B * KVH * S * Dh * 4
    c = cfg_of(1, 2, 1, 64, 128, 16, 1, 0, 1, 1, torch.float32)
    args = [fake, 0, 0, 64] * 5
    rc = lib.hga_attend_prefill_bwd(ctypes.byref(c), 256, *args, None, fake, fake, 0,
                                    *([fake, 0, 0, 64] * 3), fake, 1 << 30, None)
    assert rc == -2 and b"chunk_size" in lib.hga_last_error()


def test_write_tokens_checks_without_launch():
    """hga_write_tokens refuses a half-given row set, unaligned rows and negative counts before
    launching; an empty block or no row set at all is a no-op."""
    import torch
    lib = _lib.lib()
    cfg = ops.make_config(batch=1, heads=8, kv_heads=2, head_dim=64, chunk_size=64,
                          group_size=16, topk_chunks=4, topk_groups=8, keep_first=1,
                          keep_last=2, cutoff_pair=3, dtype=torch.bfloat16)
    fake, odd, z = ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 20) + 8), ctypes.c_void_p(0)
    good = [fake, 128 * 64, 64 * 64, 64]

    def call(L, sets):
        args = [a for s in sets for a in s[0]] + [a for s in sets for a in s[1]]
        return lib.hga_write_tokens(ctypes.byref(cfg), L, *args, None)

    none = [z, 0, 0, 0]
    assert call(4, [(none, none)] * 3) == 0                       # nothing to copy
    assert call(0, [(good, good)] * 3) == 0                        # empty block
    assert call(-1, [(good, good)] * 3) == -1
    rc = call(4, [(good, none), (none, none), (none, none)])
    assert rc == -1 and b"half given" in lib.hga_last_error()
    rc = call(4, [(good, good), (good, [odd, 128 * 64, 64 * 64, 64]), (none, none)])
    assert rc == -1 and b"aligned" in lib.hga_last_error()
    rc = call(4, [(good, [fake, 128 * 64, 64 * 64, 68]), (none, none), (none, none)])
    assert rc == -1 and b"aligned" in lib.hga_last_error()


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="needs hipcc")
def test_host_checks_under_address_and_undefined_sanitizers(tmp_path):
    """The host side of the C ABI (config validation, width / workspace / size queries, every
    entry point's argument checks, tests/sanitize/capi_checks.cpp) built host-only with
    -fsanitize=address,undefined and run with boundary and invalid inputs: no report, every
    status as expected."""
    import subprocess
    csrc = os.path.join(ROOT, "hierarchicalglobalattention_amd", "csrc")
    b = subprocess.run(["make", "-s", "-j8", "-C", csrc, "sanitize"], capture_output=True,
                       text=True, timeout=600)
    assert b.returncode == 0, b.stdout[-2000:] + b.stderr[-2000:]
    exe = os.path.join(ROOT, "hierarchicalglobalattention_amd", "_build", "sanitize",
                       "capi_checks")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "capi_checks: ok" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr
