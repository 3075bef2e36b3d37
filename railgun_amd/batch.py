"""Host-side packing of one engine step into the device metadata the kernels consume.

Railgun's scheduler emits prefill chunks and decode slots
(crates/vllm-scheduler/src/batch.rs:8-51) with one KV slot per token
(crates/vllm-scheduler/src/scheduler.rs:230-235 for prefill, :258-263 for decode), and the
engine flattens them into packed tensors (crates/vllm-engine/src/engine.rs:184-227):

* tokens: every prefill chunk's ids in order, then one id per decode slot;
* context length: ``position_start + len(chunk)`` for a prefill chunk, ``seq_len`` for a
  decode slot; ``max_context_len`` is their maximum;
* block table: row-major ``[requests, max_blocks]``, each row padded with block 0.

:func:`pack_step` reproduces that layout and adds what this build's kernels need on top
of it: the position of every token, ``cu_seqlens`` of the prefill rows and the split
point between prefill and decode rows.  Block ids are Railgun ``BlockId`` values (u32 whose
bit 31 marks a CPU-resident block, crates/vllm-paged-attention/src/block.rs:11-36); the
kernels read them as int32, so GPU ids must be below 2^31 (the reference builds u32
tensors and reads them as i32, which is the same bits for such ids).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

CPU_BLOCK_FLAG = 1 << 31  # BlockId bit 31: the block lives in host memory (block.rs:15-36)


@dataclass
class PrefillChunk:
    """batch.rs:23-34: a run of prompt tokens starting at ``position_start``."""

    token_ids: Sequence[int]
    position_start: int
    block_table: Sequence[int]


@dataclass
class DecodeSlot:
    """batch.rs:8-19: one new token; ``seq_len`` counts it (prompt + generated so far)."""

    last_token_id: int
    seq_len: int
    block_table: Sequence[int]


def slot_of(block_table: Sequence[int], pos: int, block_size: int) -> int:
    """scheduler.rs:230-235 / :258-263: block_table[pos / bs] * bs + pos % bs."""
    return int(block_table[pos // block_size]) * block_size + pos % block_size


@dataclass
class StepBatch:
    """Packed host metadata of one step (int32 numpy arrays, ready to copy to the device).

    Rows ``[0, num_prefill_tokens)`` are the prefill tokens of ``num_prefill_seqs``
    sequences (``cu_seqlens`` over them), rows after that one decode token each.  Request r
    (prefill chunks first) owns ``block_table[r]`` and ``context_lens[r]``.
    """

    tokens: np.ndarray          # int64 [T]
    positions: np.ndarray       # int32 [T]
    slot_mapping: np.ndarray    # int32 [T]
    context_lens: np.ndarray    # int32 [R]
    block_table: np.ndarray     # int32 [R, max_blocks]
    cu_seqlens: np.ndarray      # int32 [num_prefill_seqs + 1]
    num_prefill_seqs: int
    num_prefill_tokens: int
    max_context_len: int
    max_query_len: int
    last_rows: np.ndarray = field(default=None)  # int64 [R]: row of each request's last token

    @property
    def num_tokens(self) -> int:
        return int(self.tokens.shape[0])

    @property
    def num_requests(self) -> int:
        return int(self.context_lens.shape[0])

    @property
    def num_decode(self) -> int:
        return self.num_requests - self.num_prefill_seqs


def _check_ids(table: Sequence[int]) -> None:
    for b in table:
        if int(b) < 0 or int(b) & CPU_BLOCK_FLAG:
            raise ValueError(f"block id {int(b):#x} is not a GPU block (bit 31 marks CPU blocks, block.rs:15-36)")


def pack_step(prefill_chunks: Sequence[PrefillChunk], decode_slots: Sequence[DecodeSlot], block_size: int,
              max_blocks: Optional[int] = None) -> StepBatch:
    """engine.rs:184-227 plus positions / cu_seqlens; ``max_blocks`` (default: the longest
    table) fixes the padded row length, e.g. to keep one shape across steps."""
    tokens, positions, slots, ctx, tables = [], [], [], [], []
    cu = [0]
    for c in prefill_chunks:
        n = len(c.token_ids)
        if n == 0:
            raise ValueError("empty prefill chunk")
        _check_ids(c.block_table)
        end = c.position_start + n
        if (end + block_size - 1) // block_size > len(c.block_table):
            raise ValueError(f"prefill chunk ending at position {end} needs more than {len(c.block_table)} blocks")
        tokens.extend(int(t) for t in c.token_ids)
        for i in range(n):
            positions.append(c.position_start + i)
            slots.append(slot_of(c.block_table, c.position_start + i, block_size))
        ctx.append(end)
        tables.append(list(c.block_table))
        cu.append(cu[-1] + n)
    for d in decode_slots:
        if d.seq_len <= 0:
            raise ValueError("decode slot with seq_len <= 0")
        _check_ids(d.block_table)
        if (d.seq_len + block_size - 1) // block_size > len(d.block_table):
            raise ValueError(f"decode slot of length {d.seq_len} needs more than {len(d.block_table)} blocks")
        tokens.append(int(d.last_token_id))
        positions.append(d.seq_len - 1)
        slots.append(slot_of(d.block_table, d.seq_len - 1, block_size))
        ctx.append(d.seq_len)
        tables.append(list(d.block_table))
    widest = max((len(t) for t in tables), default=0)
    mb = widest if max_blocks is None else int(max_blocks)
    if mb < widest:
        raise ValueError(f"max_blocks {mb} is shorter than a block table of {widest}")
    bt = np.zeros((len(tables), mb), np.int32)
    for r, t in enumerate(tables):
        bt[r, :len(t)] = np.asarray(t, dtype=np.int64).astype(np.int32)
    lens = np.diff(np.asarray(cu))
    last = np.concatenate([np.asarray(cu[1:], np.int64) - 1,
                           cu[-1] + np.arange(len(decode_slots), dtype=np.int64)])
    return StepBatch(
        tokens=np.asarray(tokens, np.int64), positions=np.asarray(positions, np.int32),
        slot_mapping=np.asarray(slots, np.int32), context_lens=np.asarray(ctx, np.int32), block_table=bt,
        cu_seqlens=np.asarray(cu, np.int32), num_prefill_seqs=len(prefill_chunks), num_prefill_tokens=cu[-1],
        max_context_len=max(ctx, default=0), max_query_len=int(lens.max()) if len(lens) else 0, last_rows=last)


__all__ = ["CPU_BLOCK_FLAG", "DecodeSlot", "PrefillChunk", "StepBatch", "pack_step", "slot_of"]
