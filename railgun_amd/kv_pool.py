"""Paged KV pools and the physical block operations on them.

Railgun keeps every KV page of a GPU in one pre-allocated pool ``[NB, 2, H_kv, bs, D]``
(K at ``[:, 0]``, V at ``[:, 1]``, crates/vllm-paged-attention/src/block.rs:49-99) and a
host-side pool of the same block shape (block.rs:101-108).  Its allocator hands out block
ids, forks them for copy-on-write and "swaps" them between the two pools, but the swap moves
no data (crates/vllm-paged-attention/src/allocator.rs:102-153).  Here:

* :class:`GpuBlockPool` holds one such pool per layer, ``[layers, NB, 2, H_kv, bs, D]``
  (one pool shared by all layers is defect D11 of the reference), with the K / V views the
  kernels take (block stride ``2 H_kv bs D`` elements);
* :class:`CpuBlockPool` is the host pool in pinned memory, which the GPU reads and writes
  directly;
* :meth:`GpuBlockPool.swap_out`, :meth:`GpuBlockPool.swap_in` and
  :meth:`GpuBlockPool.copy_blocks` are the physical copies behind the allocator's swap and
  copy-on-write, each one ``rg_copy_blocks`` launch over all layers.

Block ids are pool indices (``BlockId.index()``); which ids are free is the allocator's
business and stays outside this module.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from .ops import PagedAttentionKernels


def _pairs(src: Sequence[int], dst: Sequence[int], nsrc: int, ndst: int, device) -> torch.Tensor:
    if len(src) != len(dst):
        raise ValueError("source and destination id lists differ in length")
    if any(not 0 <= int(b) < nsrc for b in src) or any(not 0 <= int(b) < ndst for b in dst):
        raise ValueError("block id outside its pool")
    if len(set(int(b) for b in dst)) != len(dst):
        raise ValueError("a destination block appears twice")
    m = torch.tensor([[int(a), int(b)] for a, b in zip(src, dst)], dtype=torch.int32).reshape(-1, 2)
    return m.to(device) if device is not None else m.pin_memory()


class GpuBlockPool:
    """Per-layer paged KV storage ``[layers, NB, 2, H_kv, bs, D]`` on one GPU."""

    def __init__(self, num_layers: int, num_blocks: int, num_kv_heads: int, block_size: int, head_dim: int,
                 device, dtype=torch.bfloat16, fill: Optional[torch.Generator] = None,
                 kernels: Optional[PagedAttentionKernels] = None):
        shape = (num_layers, num_blocks, 2, num_kv_heads, block_size, head_dim)
        if fill is None:
            self.storage = torch.zeros(shape, device=device, dtype=dtype)
        else:  # N(0, 1) contents, for measurements over a pre-filled context
            self.storage = torch.empty(shape, device=device, dtype=dtype)
            for layer in range(num_layers):
                self.storage[layer].copy_(torch.randn(shape[1:], generator=fill, device=device,
                                                      dtype=torch.float32).to(dtype))
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.device = self.storage.device
        self._kernels = kernels

    @staticmethod
    def for_model(cfg, num_blocks: int, block_size: int, device, dtype=torch.bfloat16,
                  fill: Optional[torch.Generator] = None) -> "GpuBlockPool":
        return GpuBlockPool(cfg.num_hidden_layers, num_blocks, cfg.num_key_value_heads, block_size, cfg.head_dim,
                            device, dtype, fill)

    @property
    def kernels(self) -> PagedAttentionKernels:
        if self._kernels is None:
            self._kernels = PagedAttentionKernels(self.device)
        return self._kernels

    def k_cache(self, layer: int) -> torch.Tensor:
        """block.rs:89-91: the K view [NB, H_kv, bs, D] of one layer."""
        return self.storage[layer, :, 0]

    def v_cache(self, layer: int) -> torch.Tensor:
        """block.rs:93-95: the V view [NB, H_kv, bs, D] of one layer."""
        return self.storage[layer, :, 1]

    def copy_blocks(self, src: Sequence[int], dst: Sequence[int]) -> None:
        """Copy-on-write: block dst[i] becomes a copy of block src[i], K and V, every layer."""
        if not len(src):
            return
        m = _pairs(src, dst, self.num_blocks, self.num_blocks, self.device)
        if set(int(b) for b in src) & set(int(b) for b in dst):
            raise ValueError("copy_blocks: a block is both a source and a destination")
        self.kernels.launch_copy_blocks(self.storage, self.storage, m, layered=True)

    def swap_out(self, gpu_ids: Sequence[int], cpu_pool: "CpuBlockPool", cpu_ids: Sequence[int]) -> None:
        """allocator.rs:102-131 with the data: GPU block gpu_ids[i] -> host block cpu_ids[i]."""
        if not len(gpu_ids):
            return
        cpu_pool.check_compatible(self)
        m = _pairs(gpu_ids, cpu_ids, self.num_blocks, cpu_pool.num_blocks, self.device)
        self.kernels.launch_copy_blocks(self.storage, cpu_pool.storage, m, layered=True)

    def swap_in(self, cpu_pool: "CpuBlockPool", cpu_ids: Sequence[int], gpu_ids: Sequence[int]) -> None:
        """allocator.rs:133-153 with the data: host block cpu_ids[i] -> GPU block gpu_ids[i]."""
        if not len(gpu_ids):
            return
        cpu_pool.check_compatible(self)
        m = _pairs(cpu_ids, gpu_ids, cpu_pool.num_blocks, self.num_blocks, self.device)
        self.kernels.launch_copy_blocks(cpu_pool.storage, self.storage, m, layered=True)


class CpuBlockPool:
    """Host pool of the same per-layer block shape, in pinned (device-accessible) memory."""

    def __init__(self, like: GpuBlockPool, num_blocks: int):
        shape = (like.storage.shape[0], num_blocks) + tuple(like.storage.shape[2:])
        self.storage = torch.zeros(shape, dtype=like.storage.dtype, pin_memory=True)
        self.num_blocks = num_blocks

    def check_compatible(self, gpu: GpuBlockPool) -> None:
        g, c = gpu.storage, self.storage
        if g.dtype != c.dtype or g.shape[0] != c.shape[0] or g.shape[2:] != c.shape[2:]:
            raise ValueError("host and GPU pools differ in layers, block shape or dtype")


__all__ = ["CpuBlockPool", "GpuBlockPool"]
