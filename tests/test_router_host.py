"""Host logic of the router that runs before any kernel (CPU, no GPU needed)."""
import types

import pytest
import torch

from hierarchicalglobalattention_amd.router import (ChunkPlacementPolicy, ChunkRouter,
                                                    RouterConfig)


@pytest.mark.parametrize("dtype,head_dim,limit", [(torch.float32, 16, 512),
                                                   (torch.bfloat16, 64, 2048)])
def test_long_fresh_block_error_names_the_limit(dtype, head_dim, limit):
    """A fresh block whose last query chunk routes over more chunks than the chunk-parallel
    router takes (512 for the split kernels and fp32; 2048 for the fused bf16 router) is refused
    with guidance before any kernel runs (no GPU needed: the check precedes the first launch).
    Blocks within the bound are routed on the GPU (tests/test_gpu_long_prefill.py)."""
    pol = ChunkPlacementPolicy(keep_first=2, keep_last=8, first_token_level=True)
    router = ChunkRouter(RouterConfig(nhead=2, kv_heads=1, head_dim=head_dim, chunk_size=8,
                                      group_size=4, topk_chunks=2, topk_groups=4, theta=1e4),
                         types.SimpleNamespace(policy=pol))
    S = (limit + 2 + 8 + 2) * 8                   # last query chunk's pool: limit + 1 chunks
    q = torch.zeros(1, 2, S, head_dim, dtype=dtype)
    kv = torch.zeros(1, 1, S, head_dim, dtype=dtype)
    with pytest.raises(ValueError, match=str(limit)):
        router._prefill(0, q, kv, kv, kv, None, None, populate_store=False)
