"""Physical KV block operations (rg_copy_blocks through railgun_amd.kv_pool) on the GPU.

Copies are bit-exact by construction, so every check is equality: copy-on-write inside the
per-layer fused pool against torch indexing on the CPU, GPU -> pinned host -> GPU swap
round trips (bf16 and fp16 pools), paged attention over swapped-in blocks equal to the
attention over the originals, and pageable host memory refused before any launch.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from railgun_amd import _lib
from railgun_amd.kv_pool import CpuBlockPool, GpuBlockPool

pytestmark = pytest.mark.gpu


def _pool(device, dtype, layers=3, nb=40, hkv=8, bs=16, d=64, seed=0):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return GpuBlockPool(layers, nb, hkv, bs, d, device, dtype, fill=g)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_copy_blocks_copy_on_write(device, dtype):
    pool = _pool(device, dtype)
    before = pool.storage.cpu()
    src, dst = [3, 17, 0, 39], [5, 2, 38, 11]
    pool.copy_blocks(src, dst)
    torch.cuda.synchronize()
    want = before.clone()
    want[:, dst] = before[:, src]
    assert torch.equal(pool.storage.cpu().view(torch.uint8), want.view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_swap_out_and_in_round_trip(device, dtype):
    pool = _pool(device, dtype, seed=1)
    host = CpuBlockPool(pool, 24)
    before = pool.storage.cpu()
    gpu_ids, cpu_ids = [7, 30, 1, 12, 25], [0, 23, 9, 4, 16]
    pool.swap_out(gpu_ids, host, cpu_ids)
    torch.cuda.synchronize()
    assert torch.equal(host.storage[:, cpu_ids].view(torch.uint8), before[:, gpu_ids].view(torch.uint8))
    # the GPU blocks are reused (overwritten), then the host copies come back elsewhere
    pool.storage[:, gpu_ids] = 0
    back = [2, 3, 33, 34, 39]
    pool.swap_in(host, cpu_ids, back)
    torch.cuda.synchronize()
    assert torch.equal(pool.storage[:, back].cpu().view(torch.uint8), before[:, gpu_ids].view(torch.uint8))


def test_decode_over_swapped_blocks_matches(device, kernels):
    """fp16 KV: attention over blocks swapped out and back in at other ids (block table
    rewritten) equals the attention over the original blocks, bit for bit."""
    H, hkv, d, bs = 32, 8, 64, 16
    pool = _pool(device, torch.float16, layers=1, nb=64, hkv=hkv, d=d, seed=2)
    host = CpuBlockPool(pool, 16)
    ctx = torch.tensor([100, 37, 160], dtype=torch.int32, device=device)
    bt = torch.tensor([[4, 9, 11, 20, 21, 22, 30, 0, 0, 0], [1, 2, 3, 0, 0, 0, 0, 0, 0, 0],
                       [40, 41, 42, 43, 44, 45, 46, 47, 48, 49]], dtype=torch.int32, device=device)
    q = torch.randn(3, H, d, device=device).half()
    out_a, out_b = torch.empty_like(q), torch.empty_like(q)
    mb = int(bt.shape[1])
    ws = torch.empty(kernels.v1_workspace_bytes(3, H, hkv, d, bs, mb), dtype=torch.uint8, device=device)
    kernels.launch_v1(q, pool.k_cache(0), pool.v_cache(0), bt, ctx, out_a, 0.125, H, hkv, d, bs, mb, 3, workspace=ws)
    used = [4, 9, 11, 20, 21, 22, 30]
    pool.swap_out(used, host, list(range(7)))
    new = [50, 51, 52, 53, 54, 55, 56]
    pool.swap_in(host, list(range(7)), new)
    bt2 = bt.clone()
    bt2[0, :7] = torch.tensor(new, dtype=torch.int32)
    pool.storage[:, used] = 0
    kernels.launch_v1(q, pool.k_cache(0), pool.v_cache(0), bt2, ctx, out_b, 0.125, H, hkv, d, bs, mb, 3, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)


def test_pageable_host_memory_is_refused(device):
    """The entry checks every pointer with the HIP runtime before it launches anything."""
    lib = _lib.load_library()
    pool = torch.zeros(4, 64, device=device)
    host = np.zeros((4, 64), np.float32)  # ordinary (pageable) numpy memory
    m = torch.tensor([[0, 1]], dtype=torch.int32, device=device)
    st = lib.rg_copy_blocks(pool.data_ptr(), host.ctypes.data, m.data_ptr(), 1, 256, 256, 256, 1, 0, 0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "pinned" in _lib.last_error()
    torch.cuda.synchronize()
