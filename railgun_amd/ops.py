"""Host-side mirror of Railgun's kernel launchers and custom op over the C ABI.

``PagedAttentionKernels`` mirrors ``crates/vllm-cuda/src/kernels/mod.rs:23-509`` (one
``launch_*`` method per launcher, same argument order and meaning) and
``PagedAttentionOp`` mirrors ``crates/vllm-cuda/src/kernels/paged_attn_op.rs:12-269``
(``execute`` with the v1/v2 dispatch rule, ``reshape_and_cache``, ``apply_rope``).  Device
buffers are torch tensors (PyTorch only supplies device memory and the current stream);
every launch goes through ``librailgun_hip.so``.  Errors surface as
:class:`railgun_amd.RailgunError` carrying the library's message, in the places the
reference returns ``CoreError`` / ``candle_core::Error::Msg``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import RailgunError, check, load_library

_DTYPES = {torch.float32: _lib.RG_DTYPE_F32, torch.bfloat16: _lib.RG_DTYPE_BF16, torch.float16: _lib.RG_DTYPE_F16}

# Dispatch threshold of PagedAttentionOp::execute (paged_attn_op.rs:89).
V1_MAX_CONTEXT = 4096
# Tokens per partition execute() uses for its v2 branch (the reference fixes 256,
# paged_attention_utils.cuh:10; any multiple of block_size gives the same result).
V2_PARTITION_SIZE = 512


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise RailgunError(_lib.RG_ERR_NOT_SUPPORTED, f"dtype {t.dtype} is not supported") from None


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_cuda(*tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "PagedAttentionOp requires GPU tensors")


def _require_i32(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise RailgunError(
                _lib.RG_ERR_INVALID_ARGUMENT,
                f"index tensors must be contiguous int32 (block ids are read as i32), got {t.dtype}",
            )


def cache_geometry(k_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple[int, int, int, int]:
    """(num_kv_heads, block_size, head_dim, kv_block_stride) of a [NB, H_kv, bs, D] cache view.

    Accepts Railgun's fused pool views ``storage[:, 0]`` / ``storage[:, 1]`` of a
    ``[NB, 2, H_kv, bs, D]`` tensor (crates/vllm-paged-attention/src/block.rs:70,89-95): each
    block's rows must be contiguous and both caches must share the block stride.
    """
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT,
                           f"caches must be [num_blocks, num_kv_heads, block_size, head_dim], got "
                           f"{tuple(k_cache.shape)} and {tuple(v_cache.shape)}")
    _, hkv, bs, d = k_cache.shape
    for c in (k_cache, v_cache):
        if c.stride(3) != 1 or c.stride(2) != d or c.stride(1) != bs * d:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "cache blocks must be contiguous [H_kv, bs, D]")
    if k_cache.stride(0) != v_cache.stride(0) or k_cache.dtype != v_cache.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "k and v caches must share dtype and block stride")
    return int(hkv), int(bs), int(d), int(k_cache.stride(0))


def rope_cos_sin_table(max_position: int, head_dim: int, theta: float,
                       device: Optional[torch.device] = None) -> torch.Tensor:
    """fp32 [max_position, head_dim] table: cos in [:, :D/2], sin in [:, D/2:] (HF Llama)."""
    lib = load_library()
    table = np.empty((max_position, head_dim), dtype=np.float32)
    check(lib.rg_rope_cos_sin_table(table.ctypes.data_as(_lib.f32p), max_position, head_dim, float(theta)))
    t = torch.from_numpy(table)
    return t.to(device) if device is not None else t


class PagedAttentionKernels:
    """Launchers of the attention hot path (crates/vllm-cuda/src/kernels/mod.rs:23-509).

    Construction checks the device (``PagedAttentionKernels::new``, mod.rs:57-190).  Every
    ``launch_*`` is asynchronous on the current torch stream of the tensors' device; none
    allocates.  The KV block stride is taken from ``key_cache.stride(0)``.
    """

    def __init__(self, device: int | torch.device = 0):
        self.lib = load_library()
        ordinal = device.index if isinstance(device, torch.device) else int(device)
        self.ordinal = 0 if ordinal is None else ordinal
        check(self.lib.rg_init(self.ordinal))

    # mod.rs:196-225
    def launch_rope(self, x, cos_sin, positions, num_heads: int, head_dim: int, num_tokens: int) -> None:
        _require_cuda(x, cos_sin, positions)
        _require_i32(positions)
        check(self.lib.rg_rope(x.data_ptr(), cos_sin.data_ptr(), positions.data_ptr(), num_heads, head_dim,
                               num_tokens, dtype_code(x), _stream(x)))

    # Opt-in index checks (no counterpart in mod.rs): synchronous, raise RailgunError naming the
    # first bad entry.
    def validate_block_tables(self, block_table, context_lens, block_size: int, num_blocks: int) -> None:
        _require_cuda(block_table, context_lens)
        _require_i32(block_table, context_lens)
        batch, max_blocks = int(block_table.shape[0]), int(block_table.shape[1])
        check(self.lib.rg_validate_block_tables(block_table.data_ptr(), context_lens.data_ptr(), batch, max_blocks,
                                                block_size, num_blocks, _stream(block_table)))

    def validate_slot_mapping(self, slot_mapping, num_slots: int) -> None:
        _require_cuda(slot_mapping)
        _require_i32(slot_mapping)
        check(self.lib.rg_validate_slot_mapping(slot_mapping.data_ptr(), int(slot_mapping.numel()), num_slots,
                                                _stream(slot_mapping)))

    # mod.rs:227-262
    def launch_reshape_and_cache(self, k, v, k_cache, v_cache, slot_mapping, num_kv_heads: int,
                                 head_dim: int, block_size: int, batch_size: int) -> None:
        _require_cuda(k, v, k_cache, v_cache, slot_mapping)
        _require_i32(slot_mapping)
        check(self.lib.rg_reshape_and_cache(k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                            slot_mapping.data_ptr(), num_kv_heads, head_dim, block_size,
                                            batch_size, dtype_code(k), k_cache.stride(0), _stream(k)))

    # mod.rs:264-303
    def launch_reshape_and_cache_isoquant(self, k, v, k_cache, v_cache, slot_mapping, rotation_metadata,
                                          num_kv_heads: int, head_dim: int, block_size: int,
                                          batch_size: int) -> None:
        _require_cuda(k, v, k_cache, v_cache, slot_mapping, rotation_metadata)
        _require_i32(slot_mapping)
        check(self.lib.rg_reshape_and_cache_isoquant(
            k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(),
            rotation_metadata.data_ptr(), num_kv_heads, head_dim, block_size, batch_size, dtype_code(k),
            k_cache.stride(0), _stream(k)))

    def v1_workspace_bytes(self, batch_size: int, num_heads: int, num_kv_heads: int, head_dim: int,
                           block_size: int, max_blocks_per_seq: int) -> int:
        return int(self.lib.rg_paged_attention_v1_workspace_bytes(batch_size, num_heads, num_kv_heads, head_dim,
                                                                  block_size, max_blocks_per_seq))

    # mod.rs:305-348 (+ optional workspace: the split-K form of the same computation)
    def launch_v1(self, query, key_cache, value_cache, block_table, context_lens, output, scale: float,
                  num_heads: int, num_kv_heads: int, head_dim: int, block_size: int, max_blocks_per_seq: int,
                  batch_size: int, workspace: Optional[torch.Tensor] = None) -> None:
        _require_cuda(query, key_cache, value_cache, block_table, context_lens, output, workspace)
        _require_i32(block_table, context_lens)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(self.lib.rg_paged_attention_v1(
            query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), output.data_ptr(), float(scale), num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, dtype_code(query), key_cache.stride(0),
            _ptr(workspace), ws_bytes, _stream(query)))

    def launch_rope_reshape_and_cache_v1(self, query, key, value, key_cache, value_cache, cos_sin, positions,
                                         slot_mapping, block_table, context_lens, output, scale: float,
                                         num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                                         max_blocks_per_seq: int, batch_size: int,
                                         workspace: torch.Tensor) -> None:
        """launch_rope_reshape_and_cache of one new token per sequence (key / value [batch, H_kv, D])
        followed by launch_v1, in the stream-K decode's launches
        (rg_rope_reshape_and_cache_paged_attention_v1): the same output and caches bit for bit,
        with query read and left unrotated."""
        _require_cuda(query, key, value, key_cache, value_cache, cos_sin, positions, slot_mapping, block_table,
                      context_lens, output, workspace)
        _require_i32(positions, slot_mapping, block_table, context_lens)
        for t in (query, key, value):
            if not t.is_contiguous():
                raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "query, key and value must be contiguous")
        check(self.lib.rg_rope_reshape_and_cache_paged_attention_v1(
            query.data_ptr(), key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
            cos_sin.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), output.data_ptr(), float(scale), num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, dtype_code(query), key_cache.stride(0),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(query)))

    def launch_v1_no_alloc(self, query, key_cache, value_cache, block_table, context_lens, output, scale: float,
                           num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                           max_blocks_per_seq: int, batch_size: int) -> None:
        """launch_v1 for callers that cannot allocate (graph capture, serving loops): the split-K
        partials go to the library's static per-device scratch (rg_paged_attention_v1_no_alloc).
        Calls that overlap in time on one device race on that scratch; one stream orders them."""
        _require_cuda(query, key_cache, value_cache, block_table, context_lens, output)
        _require_i32(block_table, context_lens)
        check(self.lib.rg_paged_attention_v1_no_alloc(
            query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), output.data_ptr(), float(scale), num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, dtype_code(query), key_cache.stride(0), _stream(query)))

    # mod.rs:350-399
    def launch_v1_plus(self, query, key_cache, value_cache, block_table, context_lens, output,
                       rotation_metadata, scale: float, num_heads: int, num_kv_heads: int, head_dim: int,
                       block_size: int, max_blocks_per_seq: int, batch_size: int,
                       workspace: Optional[torch.Tensor] = None) -> None:
        _require_cuda(query, key_cache, value_cache, block_table, context_lens, output, workspace)
        _require_i32(block_table, context_lens)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(self.lib.rg_paged_attention_v1_plus(
            query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), output.data_ptr(), _ptr(rotation_metadata), float(scale), num_heads,
            num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size, dtype_code(query),
            key_cache.stride(0), _ptr(workspace), ws_bytes, _stream(query)))

    # mod.rs:401-456
    def launch_v2_partition(self, query, key_cache, value_cache, block_table, context_lens, tmp_out, exp_sums,
                            max_logits, rotation_metadata, scale: float, num_heads: int, num_kv_heads: int,
                            head_dim: int, block_size: int, max_blocks_per_seq: int, num_partitions: int,
                            batch_size: int, partition_size: int = 256) -> None:
        _require_cuda(query, key_cache, value_cache, block_table, context_lens, tmp_out, exp_sums, max_logits)
        _require_i32(block_table, context_lens)
        check(self.lib.rg_paged_attention_v2_partition(
            query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), tmp_out.data_ptr(), exp_sums.data_ptr(), max_logits.data_ptr(),
            _ptr(rotation_metadata), float(scale), num_heads, num_kv_heads, head_dim, block_size,
            max_blocks_per_seq, num_partitions, batch_size, partition_size, dtype_code(query),
            key_cache.stride(0), _stream(query)))

    # mod.rs:458-508
    def launch_v2_reduce(self, output, exp_sums, max_logits, tmp_out, context_lens, rotation_metadata,
                         num_heads: int, head_dim: int, num_partitions: int, batch_size: int,
                         partition_size: int = 256) -> None:
        _require_cuda(output, exp_sums, max_logits, tmp_out, context_lens)
        _require_i32(context_lens)
        check(self.lib.rg_paged_attention_v2_reduce(
            output.data_ptr(), exp_sums.data_ptr(), max_logits.data_ptr(), tmp_out.data_ptr(),
            context_lens.data_ptr(), _ptr(rotation_metadata), num_heads, head_dim, num_partitions, batch_size,
            partition_size, dtype_code(output), _stream(output)))

    def launch_v2(self, query, key_cache, value_cache, block_table, context_lens, output, scale: float,
                  num_heads: int, num_kv_heads: int, head_dim: int, block_size: int, max_blocks_per_seq: int,
                  batch_size: int, max_context_len: int, partition_size: int, workspace: torch.Tensor) -> None:
        """v2 partition + reduce in one call, scratch carved from ``workspace``."""
        _require_cuda(query, key_cache, value_cache, block_table, context_lens, output, workspace)
        _require_i32(block_table, context_lens)
        check(self.lib.rg_paged_attention_v2(
            query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), output.data_ptr(), float(scale), num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, max_context_len, partition_size, dtype_code(query),
            key_cache.stride(0), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            _stream(query)))

    def v2_workspace_bytes(self, batch_size: int, num_heads: int, num_partitions: int, head_dim: int) -> int:
        return int(self.lib.rg_v2_workspace_bytes(batch_size, num_heads, num_partitions, head_dim))

    # New entries (no reference launcher): fused RoPE + cache write, packed causal prefill.
    def launch_rope_reshape_and_cache(self, q, k, v, k_cache, v_cache, cos_sin, positions, slot_mapping,
                                      num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                                      num_tokens: int) -> None:
        _require_cuda(q, k, v, k_cache, v_cache, cos_sin, positions, slot_mapping)
        _require_i32(positions, slot_mapping)
        check(self.lib.rg_rope_reshape_and_cache(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), cos_sin.data_ptr(),
            positions.data_ptr(), slot_mapping.data_ptr(), num_heads, num_kv_heads, head_dim, block_size,
            num_tokens, dtype_code(q), k_cache.stride(0), _stream(q)))

    def launch_qkv_rope_reshape_and_cache(self, qkv, q_out, k_cache, v_cache, cos_sin, positions, slot_mapping,
                                          num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                                          num_tokens: int) -> None:
        """Fused RoPE + cache write reading q/k/v from one fused projection output qkv
        [T, >= (H + 2 H_kv) D] (row stride qkv.stride(0)); rotated q goes to q_out [T, H, D]."""
        _require_cuda(qkv, q_out, k_cache, v_cache, cos_sin, positions, slot_mapping)
        _require_i32(positions, slot_mapping)
        if qkv.dim() != 2 or qkv.stride(1) != 1 or not q_out.is_contiguous():
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "qkv must be [T, N] with unit column stride and "
                                                             "q_out contiguous")
        check(self.lib.rg_qkv_rope_reshape_and_cache(
            qkv.data_ptr(), qkv.stride(0), q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            cos_sin.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(), num_heads, num_kv_heads, head_dim,
            block_size, num_tokens, dtype_code(qkv), k_cache.stride(0), _stream(qkv)))

    def launch_linear_qkv_rope_reshape_and_cache(self, x, weight_qkv, q_out, k_cache, v_cache, cos_sin, positions,
                                                 slot_mapping, num_heads: int, num_kv_heads: int, head_dim: int,
                                                 block_size: int, norm_weight=None, eps: float = 0.0) -> None:
        """The fused q/k/v projection x @ weight_qkv^T and launch_qkv_rope_reshape_and_cache in one
        pass (decode batches: x [T <= 128, K], head_dim 32 or 64); rotated q to q_out [T, H, D].
        With norm_weight, x is the residual stream and the RmsNorm in front of the attention is
        folded in (rg_rms_norm_linear_qkv_rope_reshape_and_cache)."""
        _require_cuda(x, weight_qkv, q_out, k_cache, v_cache, cos_sin, positions, slot_mapping)
        _require_i32(positions, slot_mapping)
        if x.dim() != 2 or x.stride(1) != 1 or not weight_qkv.is_contiguous() or not q_out.is_contiguous() or \
                x.dtype != weight_qkv.dtype:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "x must be [T, K] with unit column stride, weight_qkv "
                                                             "and q_out contiguous, one dtype")
        tokens, k = (int(d) for d in x.shape)
        # The entry derives N = (H + 2 H_kv) D from the head counts and reads that many weight
        # rows, writes T H D values of q and reads the cos/sin rows at head_dim floats each.
        n = (num_heads + 2 * num_kv_heads) * head_dim
        if weight_qkv.dim() != 2 or tuple(weight_qkv.shape) != (n, k):
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT,
                               f"weight_qkv must be [(H + 2 H_kv) D, K] = [{n}, {k}], got {tuple(weight_qkv.shape)}")
        if q_out.numel() < tokens * num_heads * head_dim or q_out.dtype != x.dtype:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT,
                               f"q_out must hold [T, H, D] = [{tokens}, {num_heads}, {head_dim}] of x's dtype")
        if cos_sin.dim() != 2 or int(cos_sin.shape[1]) != head_dim or cos_sin.dtype != torch.float32:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT,
                               f"cos_sin must be a float32 [max_position, head_dim = {head_dim}] table")
        if int(positions.numel()) < tokens or int(slot_mapping.numel()) < tokens:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "positions and slot_mapping need one entry per token")
        if norm_weight is not None:
            _require_cuda(norm_weight)
            if tuple(norm_weight.shape) != (k,) or not norm_weight.is_contiguous() or norm_weight.dtype != x.dtype:
                raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "norm_weight must be a contiguous [K] vector of "
                                                                 "x's dtype")
            check(self.lib.rg_rms_norm_linear_qkv_rope_reshape_and_cache(
                x.data_ptr(), norm_weight.data_ptr(), float(eps), weight_qkv.data_ptr(), q_out.data_ptr(),
                k_cache.data_ptr(), v_cache.data_ptr(), cos_sin.data_ptr(), positions.data_ptr(),
                slot_mapping.data_ptr(), tokens, num_heads, num_kv_heads, head_dim, block_size, k, x.stride(0),
                weight_qkv.stride(0), num_heads * head_dim, k_cache.stride(0), dtype_code(x), _stream(x)))
            return
        check(self.lib.rg_linear_qkv_rope_reshape_and_cache(
            x.data_ptr(), weight_qkv.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            cos_sin.data_ptr(), positions.data_ptr(), slot_mapping.data_ptr(), tokens, num_heads, num_kv_heads,
            head_dim, block_size, k, x.stride(0), weight_qkv.stride(0), num_heads * head_dim, k_cache.stride(0),
            dtype_code(x), _stream(x)))

    def launch_copy_blocks(self, src_pool: torch.Tensor, dst_pool: torch.Tensor, block_mapping: torch.Tensor,
                           layered: bool = False) -> None:
        """Whole-block copies (rg_copy_blocks): block ``m[i, 1]`` of ``dst_pool`` becomes block
        ``m[i, 0]`` of ``src_pool``, in every layer when ``layered``.

        Pools are ``[NB, ...]`` (``layered=False``) or ``[layers, NB, ...]`` with contiguous
        blocks and the same block shape and dtype on both sides; each may live on the device
        or in pinned host memory.  ``block_mapping`` is int32 ``[pairs, 2]`` of (source,
        destination) ids, on the device or pinned.  Asynchronous on the current stream of the
        device side's device.
        """
        bdim = 1 if layered else 0
        if src_pool.dtype != dst_pool.dtype or src_pool.dim() != dst_pool.dim() or src_pool.dim() < bdim + 1:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "copy_blocks: pools must share dtype and rank")
        if tuple(src_pool.shape[bdim + 1:]) != tuple(dst_pool.shape[bdim + 1:]) or \
                (layered and src_pool.shape[0] != dst_pool.shape[0]):
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "copy_blocks: block shapes or layer counts differ")
        for p in (src_pool, dst_pool):
            if not p[(0,) * (bdim + 1)].is_contiguous():
                raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "copy_blocks: blocks must be contiguous")
            if not (p.is_cuda or p.is_pinned()):
                raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "copy_blocks: pools must be on the GPU or pinned")
        m = block_mapping
        if m.dtype != torch.int32 or not m.is_contiguous() or m.dim() != 2 or m.shape[1] != 2 or \
                not (m.is_cuda or m.is_pinned()):
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT,
                               "copy_blocks: block_mapping must be contiguous int32 [pairs, 2], on the GPU or pinned")
        es = src_pool.element_size()
        block_bytes = src_pool[(0,) * (bdim + 1)].numel() * es
        dev = src_pool.device if src_pool.is_cuda else dst_pool.device
        stream = torch.cuda.current_stream(dev).cuda_stream if dev.type == "cuda" else 0
        check(self.lib.rg_copy_blocks(
            src_pool.data_ptr(), dst_pool.data_ptr(), m.data_ptr(), int(m.shape[0]), block_bytes,
            src_pool.stride(bdim) * es, dst_pool.stride(bdim) * es, int(src_pool.shape[0]) if layered else 1,
            src_pool.stride(0) * es if layered else 0, dst_pool.stride(0) * es if layered else 0, stream))

    def launch_prefill_packed(self, query, key_cache, value_cache, block_table, context_lens, cu_seqlens,
                              output, scale: float, num_heads: int, num_kv_heads: int, head_dim: int,
                              block_size: int, max_blocks_per_seq: int, num_seqs: int, num_tokens: int,
                              max_query_len: int) -> None:
        _require_cuda(query, key_cache, value_cache, block_table, context_lens, cu_seqlens, output)
        _require_i32(block_table, context_lens, cu_seqlens)
        check(self.lib.rg_prefill_packed(
            query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
            context_lens.data_ptr(), cu_seqlens.data_ptr(), output.data_ptr(), float(scale), num_heads,
            num_kv_heads, head_dim, block_size, max_blocks_per_seq, num_seqs, num_tokens, max_query_len,
            dtype_code(query), key_cache.stride(0), _stream(query)))


@dataclass
class PagedAttentionOp:
    """The custom op (crates/vllm-cuda/src/kernels/paged_attn_op.rs:12-19)."""

    scale: float
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    kernels: PagedAttentionKernels = field(repr=False)

    def execute(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                block_table: torch.Tensor, context_lens: torch.Tensor,
                rotation_metadata: Optional[torch.Tensor], max_context_len: int) -> torch.Tensor:
        """paged_attn_op.rs:45-166: q [B, H, D] -> new output [B, H, D].

        ``max_context_len <= 4096`` runs v1 (single pass per partition group), longer runs
        v2 split-K; both compute the same softmax attention.
        """
        if self.head_dim % 4 != 0:
            raise RailgunError(_lib.RG_ERR_NOT_SUPPORTED,
                               f"Head dimension ({self.head_dim}) must be a multiple of 4 for IsoQuant.")
        if q.dim() != 3:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, f"q must be [batch, heads, head_dim], got {tuple(q.shape)}")
        _require_cuda(q, k_cache, v_cache, block_table, context_lens)
        batch, num_heads, head_dim = (int(x) for x in q.shape)
        num_kv_heads, block_size, _, _ = cache_geometry(k_cache, v_cache)
        if num_kv_heads != self.num_kv_heads:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT,
                               f"cache has {num_kv_heads} kv heads, op expects {self.num_kv_heads}")
        max_blocks = int(block_table.shape[1])
        out = torch.zeros_like(q)
        k = self.kernels
        if max_context_len <= V1_MAX_CONTEXT:
            ws_bytes = k.v1_workspace_bytes(batch, num_heads, self.num_kv_heads, head_dim, block_size, max_blocks)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
            k.launch_v1_plus(q, k_cache, v_cache, block_table, context_lens, out, rotation_metadata, self.scale,
                             num_heads, self.num_kv_heads, head_dim, block_size, max_blocks, batch, workspace=ws)
        else:
            num_parts = math.ceil(max_context_len / V2_PARTITION_SIZE)
            ws_bytes = max(k.v2_workspace_bytes(batch, num_heads, num_parts, head_dim),
                           k.v1_workspace_bytes(batch, num_heads, self.num_kv_heads, head_dim, block_size, max_blocks))
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
            k.launch_v2(q, k_cache, v_cache, block_table, context_lens, out, self.scale, num_heads,
                        self.num_kv_heads, head_dim, block_size, max_blocks, batch, max_context_len,
                        V2_PARTITION_SIZE, ws)
        return out

    def reshape_and_cache(self, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                          slot_mapping: torch.Tensor, rotation_metadata: Optional[torch.Tensor],
                          use_isoquant: bool) -> None:
        """paged_attn_op.rs:168-233: k, v [T, H_kv, D] written into the caches in place."""
        batch, num_kv_heads, head_dim = (int(x) for x in k.shape)
        if use_isoquant:
            self.kernels.launch_reshape_and_cache_isoquant(k, v, k_cache, v_cache, slot_mapping, rotation_metadata,
                                                           num_kv_heads, head_dim, self.block_size, batch)
        else:
            self.kernels.launch_reshape_and_cache(k, v, k_cache, v_cache, slot_mapping, num_kv_heads, head_dim,
                                                  self.block_size, batch)

    def apply_rope(self, x: torch.Tensor, cos_sin: torch.Tensor, positions: torch.Tensor) -> None:
        """paged_attn_op.rs:236-268: in-place RoPE on x [T, H, D]."""
        num_tokens, num_heads, head_dim = (int(d) for d in x.shape)
        self.kernels.launch_rope(x, cos_sin, positions, num_heads, head_dim, num_tokens)

    def rope_reshape_and_cache(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                               v_cache: torch.Tensor, cos_sin: torch.Tensor, positions: torch.Tensor,
                               slot_mapping: torch.Tensor) -> None:
        """RoPE on q (in place) and k, then the cache write, in one pass over the new tokens."""
        num_tokens = int(q.shape[0])
        self.kernels.launch_rope_reshape_and_cache(q, k, v, k_cache, v_cache, cos_sin, positions, slot_mapping,
                                                   self.num_heads, self.num_kv_heads, self.head_dim,
                                                   self.block_size, num_tokens)

    def prefill_packed(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       block_table: torch.Tensor, context_lens: torch.Tensor, cu_seqlens: torch.Tensor,
                       max_query_len: int) -> torch.Tensor:
        """Causal attention of the packed new tokens q [T, H, D] over the paged cache."""
        num_tokens = int(q.shape[0])
        out = torch.empty_like(q)
        self.kernels.launch_prefill_packed(q, k_cache, v_cache, block_table, context_lens, cu_seqlens, out,
                                           self.scale, self.num_heads, self.num_kv_heads, self.head_dim,
                                           self.block_size, int(block_table.shape[1]), int(cu_seqlens.numel()) - 1,
                                           num_tokens, max_query_len)
        return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, eps: float,
             residual: Optional[torch.Tensor] = None) -> None:
    """Fused residual add + RMSNorm over the rows of x [rows, hidden] (rg_rms_norm): with a
    residual, residual <- residual + x and out <- rmsnorm(residual) * weight; without,
    out <- rmsnorm(x) * weight."""
    _require_cuda(x, weight, out, residual)
    for t in (x, weight, out, residual):
        if t is not None and (not t.is_contiguous() or t.dtype != x.dtype):
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "rms_norm: tensors must be contiguous and share a dtype")
    hidden = int(x.shape[-1])
    rows = x.numel() // hidden if hidden else 0
    if weight.numel() != hidden or out.shape != x.shape or (residual is not None and residual.shape != x.shape):
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "rms_norm: shape mismatch")
    check(load_library().rg_rms_norm(x.data_ptr(), _ptr(residual), weight.data_ptr(), out.data_ptr(), float(eps),
                                     rows, hidden, dtype_code(x), _stream(x)))


def silu_and_mul(gate_up: torch.Tensor, out: torch.Tensor) -> None:
    """out [rows, I] = silu(gate_up[:, :I]) * gate_up[:, I:] (rg_silu_and_mul)."""
    _require_cuda(gate_up, out)
    if not gate_up.is_contiguous() or not out.is_contiguous() or gate_up.dtype != out.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "silu_and_mul: tensors must be contiguous, one dtype")
    rows, inter = int(out.shape[0]), int(out.shape[-1])
    if tuple(gate_up.shape) != (rows, 2 * inter):
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "silu_and_mul: gate_up must be [rows, 2 * I]")
    check(load_library().rg_silu_and_mul(gate_up.data_ptr(), out.data_ptr(), rows, inter, dtype_code(out),
                                         _stream(out)))


# Rows up to which rg_linear serves a projection (decode batches); larger ones go to hipBLASLt.
LINEAR_MAX_ROWS = 128


def linear_workspace_bytes(rows: int, out_features: int, in_features: int) -> int:
    """Split-K workspace bytes rg_linear uses for this shape on the current device (0: unsplit)."""
    return int(load_library().rg_linear_workspace_bytes(rows, out_features, in_features))


def linear(x: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out [rows, N] = x [rows, K] @ weight [N, K]^T (rg_linear: the decode-step projection, fp32
    accumulation, one rounding).  x may be a row-strided view; weight and out rows contiguous.
    ``workspace`` (a uint8 tensor of at least linear_workspace_bytes) lets narrow or deep layers
    split K; when omitted, one is allocated for shapes that split."""
    _require_cuda(x, weight, out)
    if x.dim() != 2 or weight.dim() != 2 or x.stride(1) != 1 or not weight.is_contiguous() or x.dtype != weight.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "linear: x [rows, K] with unit column stride and a "
                                                         "contiguous weight [N, K] of the same dtype")
    rows, k = (int(d) for d in x.shape)
    n = int(weight.shape[0])
    if int(weight.shape[1]) != k:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, f"linear: x has {k} features, weight {int(weight.shape[1])}")
    if out is None:
        out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    elif tuple(out.shape) != (rows, n) or out.stride(1) != 1 or out.dtype != x.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "linear: out must be [rows, N] with unit column stride")
    if workspace is None:
        ws_bytes = linear_workspace_bytes(rows, n, k)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    ws_ptr, ws_len = (workspace.data_ptr(), workspace.numel() * workspace.element_size()) if workspace is not None \
        else (None, 0)
    check(load_library().rg_linear(x.data_ptr(), weight.data_ptr(), out.data_ptr(), rows, n, k, x.stride(0),
                                   weight.stride(0), out.stride(0), ws_ptr, ws_len, dtype_code(x), _stream(x)))
    return out


def interleave_gate_up(w_gate_up: torch.Tensor) -> torch.Tensor:
    """[2 I, K] gate/up weight (gate rows, then up rows) -> the layout rg_linear_silu_mul takes:
    gate and up rows interleaved in blocks of 16 (a copy)."""
    two_i, k = (int(d) for d in w_gate_up.shape)
    if two_i % 32 != 0:
        raise RailgunError(_lib.RG_ERR_NOT_SUPPORTED, "interleave_gate_up: intermediate size must be a multiple of 16")
    return w_gate_up.view(2, two_i // 32, 16, k).transpose(0, 1).contiguous().view(two_i, k)


def deinterleave_gate_up(y: torch.Tensor) -> torch.Tensor:
    """The inverse permutation of interleave_gate_up along the last dimension: [..., 2 I] with
    gate and up columns interleaved in blocks of 16 -> gate columns, then up columns (a copy).
    Applied to x @ weight_il^T it gives x @ w_gate_up^T; to weight_il itself, w_gate_up."""
    two_i = int(y.shape[-1])
    if two_i % 32 != 0:
        raise RailgunError(_lib.RG_ERR_NOT_SUPPORTED, "deinterleave_gate_up: intermediate size must be a multiple "
                                                      "of 16")
    lead = tuple(y.shape[:-1])
    return y.reshape(*lead, two_i // 32, 2, 16).transpose(-3, -2).reshape(*lead, two_i).contiguous()


def linear_silu_mul(x: torch.Tensor, weight_il: torch.Tensor, out: Optional[torch.Tensor] = None,
                    norm_weight: Optional[torch.Tensor] = None, eps: float = 0.0) -> torch.Tensor:
    """out [rows, I] = silu(x @ gate^T) * (x @ up^T), each step rounded as rg_linear followed by
    rg_silu_and_mul round it; weight_il from interleave_gate_up.  With norm_weight, x is the
    residual stream and the RmsNorm in front of the MLP is folded in
    (rg_rms_norm_linear_silu_mul)."""
    _require_cuda(x, weight_il, out)
    if x.dim() != 2 or weight_il.dim() != 2 or x.stride(1) != 1 or not weight_il.is_contiguous() or \
            x.dtype != weight_il.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "linear_silu_mul: x [rows, K] with unit column stride and a "
                                                         "contiguous interleaved weight [2 I, K] of the same dtype")
    rows, k = (int(d) for d in x.shape)
    inter = int(weight_il.shape[0]) // 2
    if int(weight_il.shape[1]) != k:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, f"linear_silu_mul: x has {k} features, weight "
                                                         f"{int(weight_il.shape[1])}")
    if out is None:
        out = torch.empty((rows, inter), dtype=x.dtype, device=x.device)
    elif tuple(out.shape) != (rows, inter) or out.stride(1) != 1 or out.dtype != x.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "linear_silu_mul: out must be [rows, I] with unit column stride")
    if norm_weight is not None:
        _require_cuda(norm_weight)
        if tuple(norm_weight.shape) != (k,) or not norm_weight.is_contiguous() or norm_weight.dtype != x.dtype:
            raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "linear_silu_mul: norm_weight must be a contiguous [K] "
                                                             "vector of x's dtype")
        check(load_library().rg_rms_norm_linear_silu_mul(
            x.data_ptr(), norm_weight.data_ptr(), float(eps), weight_il.data_ptr(), out.data_ptr(), rows, inter, k,
            x.stride(0), weight_il.stride(0), out.stride(0), dtype_code(x), _stream(x)))
        return out
    check(load_library().rg_linear_silu_mul(x.data_ptr(), weight_il.data_ptr(), out.data_ptr(), rows, inter, k,
                                            x.stride(0), weight_il.stride(0), out.stride(0), dtype_code(x), _stream(x)))
    return out


def linear_residual(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                    workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """residual += x @ weight^T in place, rounded as rg_linear followed by the residual add of
    rg_rms_norm (rg_linear_residual); the split-K workspace as for linear."""
    _require_cuda(x, weight, residual)
    if x.dim() != 2 or weight.dim() != 2 or x.stride(1) != 1 or not weight.is_contiguous() or x.dtype != weight.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "linear_residual: x [rows, K] with unit column stride and a "
                                                         "contiguous weight [N, K] of the same dtype")
    rows, k = (int(d) for d in x.shape)
    n = int(weight.shape[0])
    if int(weight.shape[1]) != k or tuple(residual.shape) != (rows, n) or residual.stride(1) != 1 or \
            residual.dtype != x.dtype:
        raise RailgunError(_lib.RG_ERR_INVALID_ARGUMENT, "linear_residual: weight [N, K] and residual [rows, N] with "
                                                         "unit column stride")
    if workspace is None:
        ws_bytes = linear_workspace_bytes(rows, n, k)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    ws_ptr, ws_len = (workspace.data_ptr(), workspace.numel() * workspace.element_size()) if workspace is not None \
        else (None, 0)
    check(load_library().rg_linear_residual(x.data_ptr(), weight.data_ptr(), residual.data_ptr(), rows, n, k,
                                            x.stride(0), weight.stride(0), residual.stride(0), ws_ptr, ws_len,
                                            dtype_code(x), _stream(x)))
    return residual


__all__ = ["LINEAR_MAX_ROWS", "PagedAttentionKernels", "PagedAttentionOp", "RailgunError", "cache_geometry",
           "deinterleave_gate_up", "dtype_code", "interleave_gate_up", "linear", "linear_residual",
           "linear_silu_mul", "linear_workspace_bytes", "rms_norm", "rope_cos_sin_table", "silu_and_mul",
           "V1_MAX_CONTEXT", "V2_PARTITION_SIZE"]
