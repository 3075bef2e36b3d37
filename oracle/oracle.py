"""Python wrapper of the CPU oracle (oracle/oracle.c, built as oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the cpu_baseline
leg of bench.py import this module, and only as the checker; the product path
(railgun_amd/) never does.

Arrays are numpy.  Element types: ``"f32"`` (float32), ``"bf16"`` (bf16 bits held in a
uint16 array) and ``"f16"`` (float16).  Attention outputs are float32.

How each function is pinned independently of oracle.c (the checks live in
tests/test_oracle.py):

=====================================  =====================================================
function                               pinned by
=====================================  =====================================================
reshape_and_cache (+ isoquant meta)    numpy fancy-index scatter (bit-exact), untouched slots,
                                       slot = -1 skipped, fused-pool stride, metadata pattern
rope                                   numpy rotate_half in float64 (closed form); pos 0 is the
                                       identity; pair norms preserved; <R(m)q,R(n)k> depends on
                                       m-n only
rope_reshape_and_cache                 = rope on q and k followed by the scatter (composition)
paged_attention_v1 / v1_plus           float64 numpy softmax attention; torch SDPA (CPU, GQA);
                                       ctx = 1 returns V_0; constant scores give mean(V);
                                       permuted block table == sequential; GQA == repeated KV
paged_attention_v2_partition/reduce    v2(P) == v1 for several P; a planted wrong rescale in a
                                       copy of the merge maths is caught
prefill_packed                         torch SDPA is_causal (CPU, fp64); last row == decode
                                       with ctx = pos + 1
prefill_packed_rows                    == prefill_packed on the listed rows, rows not listed
                                       untouched
cpu_attention_gathered                 == paged_attention_v1_plus; float64 numpy attention
=====================================  =====================================================

bf16/f16 conversions are pinned against torch's own bfloat16/float16 casts.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int64, c_uint16, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

DT = {"f32": 0, "bf16": 1, "f16": 2}
NP_STORAGE = {"f32": np.float32, "bf16": np.uint16, "f16": np.float16}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        V, I, F, I64 = c_void_p, c_int, c_float, c_int64
        sig = {
            "or_bf16_to_f32": (c_float, [c_uint16]),
            "or_f32_to_bf16": (c_uint16, [c_float]),
            "or_f16_to_f32": (c_float, [c_uint16]),
            "or_f32_to_f16": (c_uint16, [c_float]),
            "or_reshape_and_cache": (None, [V, V, V, V, V, V, I, I, I, I, I, I64]),
            "or_rope": (None, [V, V, V, I, I, I, I]),
            "or_rope_reshape_and_cache": (None, [V, V, V, V, V, V, V, V, I, I, I, I, I, I, I64]),
            "or_paged_attention_v1": (None, [V, V, V, V, V, V, F, I, I, I, I, I, I, I, I64]),
            "or_paged_attention_v1_plus": (None, [V, V, V, V, V, V, F, I, I, I, I, I, I, I, I64]),
            "or_paged_attention_v2_partition": (None, [V, V, V, V, V, V, V, V, F, I, I, I, I, I, I, I, I, I, I64]),
            "or_paged_attention_v2_reduce": (None, [V, V, V, V, V, I, I, I, I, I]),
            "or_prefill_packed": (None, [V, V, V, V, V, V, V, F, I, I, I, I, I, I, I, I64]),
            "or_prefill_packed_rows": (None, [V, V, V, V, V, V, V, I, V, F, I, I, I, I, I, I, I, I64, I]),
            "or_cpu_attention_gathered": (None, [V, V, V, V, V, V, F, I, I, I, I, I, I, I, I64, I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _cache_base(c: np.ndarray) -> int:
    # Caches may be views with a larger block stride (fused pool); rows are contiguous.
    return c.ctypes.data


# ------------------------------------------------------------------ bf16 -----

def bf16_round(x) -> np.ndarray:
    """float32 -> bf16 bits (uint16), round to nearest even; NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f32(a: np.ndarray, dt: str) -> np.ndarray:
    if dt == "bf16":
        return bf16_to_f32(a)
    return np.asarray(a, dtype=np.float32)


def from_f32(a: np.ndarray, dt: str) -> np.ndarray:
    if dt == "bf16":
        return bf16_round(a)
    return np.ascontiguousarray(a, dtype=NP_STORAGE[dt])


# ------------------------------------------------------------- hot path -----

def reshape_and_cache(k, v, k_cache, v_cache, slot_mapping, dt: str, block_size: int,
                      kv_block_stride: int = 0, rotation_metadata=None) -> None:
    """In-place scatter of k, v [T, H_kv, D] into the caches (paged_attention.cu:121-137)."""
    T, hkv, d = k.shape
    slots = _i32(slot_mapping)
    meta = 0 if rotation_metadata is None else _p(rotation_metadata)
    lib().or_reshape_and_cache(_p(k), _p(v), _cache_base(k_cache), _cache_base(v_cache), _p(slots), meta or None,
                               T, hkv, d, block_size, DT[dt], kv_block_stride)


def rope(x, cos_sin, positions, dt: str) -> None:
    """In-place rotate-half RoPE on x [T, H, D] (rope.cu:18-41)."""
    T, h, d = x.shape
    pos = _i32(positions)
    cs = np.ascontiguousarray(cos_sin, dtype=np.float32)
    lib().or_rope(_p(x), _p(cs), _p(pos), T, h, d, DT[dt])


def rope_reshape_and_cache(q, k, v, k_cache, v_cache, cos_sin, positions, slot_mapping, dt: str,
                           block_size: int, kv_block_stride: int = 0) -> None:
    T, h, d = q.shape
    hkv = k.shape[1]
    cs = np.ascontiguousarray(cos_sin, dtype=np.float32)
    lib().or_rope_reshape_and_cache(_p(q), _p(k), _p(v), _cache_base(k_cache), _cache_base(v_cache), _p(cs),
                                    _p(_i32(positions)),
                                    _p(_i32(slot_mapping)), T, h, hkv, d, block_size, DT[dt], kv_block_stride)


def _decode_common(q, k_cache, block_table):
    B, H, D = q.shape
    _, hkv, bs, _ = k_cache.shape
    kv_stride = int(k_cache.strides[0] // k_cache.itemsize)
    return B, H, D, hkv, bs, int(block_table.shape[1]), kv_stride


def paged_attention_v1(q, k_cache, v_cache, block_table, context_lens, scale: float, dt: str) -> np.ndarray:
    """Two-pass decode of paged_attention.cu:33-107 -> float32 [B, H, D]."""
    B, H, D, hkv, bs, mb, stride = _decode_common(q, k_cache, block_table)
    out = np.zeros((B, H, D), np.float32)
    bt, cl = _i32(block_table), _i32(context_lens)
    lib().or_paged_attention_v1(_p(q), _cache_base(k_cache), _cache_base(v_cache), _p(bt), _p(cl), _p(out),
                                scale, B, H, hkv, D, bs, mb, DT[dt], stride)
    return out


def paged_attention_v1_plus(q, k_cache, v_cache, block_table, context_lens, scale: float, dt: str) -> np.ndarray:
    """Single-pass online-softmax decode of paged_attention_v1_plus.cu:37-105."""
    B, H, D, hkv, bs, mb, stride = _decode_common(q, k_cache, block_table)
    out = np.zeros((B, H, D), np.float32)
    bt, cl = _i32(block_table), _i32(context_lens)
    lib().or_paged_attention_v1_plus(_p(q), _cache_base(k_cache), _cache_base(v_cache), _p(bt), _p(cl), _p(out),
                                     scale, B, H, hkv, D, bs, mb, DT[dt], stride)
    return out


def paged_attention_v2_partition(q, k_cache, v_cache, block_table, context_lens, scale: float, dt: str,
                                 num_partitions: int, partition_size: int):
    """-> (tmp_out [B,H,NP,D], exp_sums [B,H,NP], max_logits [B,H,NP]); untouched entries stay 0."""
    B, H, D, hkv, bs, mb, stride = _decode_common(q, k_cache, block_table)
    tmp = np.zeros((B, H, num_partitions, D), np.float32)
    es = np.zeros((B, H, num_partitions), np.float32)
    ml = np.zeros((B, H, num_partitions), np.float32)
    bt, cl = _i32(block_table), _i32(context_lens)
    lib().or_paged_attention_v2_partition(_p(q), _cache_base(k_cache), _cache_base(v_cache), _p(bt), _p(cl),
                                          _p(tmp), _p(es), _p(ml), scale, B, H, hkv, D, bs, mb, num_partitions,
                                          partition_size, DT[dt], stride)
    return tmp, es, ml


def paged_attention_v2_reduce(tmp_out, exp_sums, max_logits, context_lens, partition_size: int) -> np.ndarray:
    B, H, NP, D = tmp_out.shape
    out = np.zeros((B, H, D), np.float32)
    lib().or_paged_attention_v2_reduce(_p(out), _p(np.ascontiguousarray(exp_sums, np.float32)),
                                       _p(np.ascontiguousarray(max_logits, np.float32)),
                                       _p(np.ascontiguousarray(tmp_out, np.float32)), _p(_i32(context_lens)),
                                       B, H, D, NP, partition_size)
    return out


def prefill_packed(q, k_cache, v_cache, block_table, context_lens, cu_seqlens, scale: float, dt: str) -> np.ndarray:
    """Textbook causal attention of the packed rows over the paged cache -> float32 [T, H, D]."""
    T, H, D = q.shape
    _, hkv, bs, _ = k_cache.shape
    stride = int(k_cache.strides[0] // k_cache.itemsize)
    S = len(cu_seqlens) - 1
    out = np.zeros((T, H, D), np.float32)
    lib().or_prefill_packed(_p(q), _cache_base(k_cache), _cache_base(v_cache), _p(_i32(block_table)),
                            _p(_i32(context_lens)), _p(_i32(cu_seqlens)), _p(out), scale, S, H, hkv, D, bs,
                            int(block_table.shape[1]), DT[dt], stride)
    return out


def prefill_packed_rows(q, k_cache, v_cache, block_table, context_lens, cu_seqlens, rows, scale: float, dt: str,
                        nthreads: int = 1) -> np.ndarray:
    """prefill_packed for the packed row indices `rows` only, threaded -> float32 [len(rows), H, D]
    (row i of the result is row rows[i] of prefill_packed's output)."""
    T, H, D = q.shape
    _, hkv, bs, _ = k_cache.shape
    stride = int(k_cache.strides[0] // k_cache.itemsize)
    S = len(cu_seqlens) - 1
    rows = _i32(rows)
    if rows.size and (rows.min() < 0 or rows.max() >= T):
        raise ValueError("row index outside the packed stream")
    out = np.zeros((T, H, D), np.float32)
    lib().or_prefill_packed_rows(_p(q), _cache_base(k_cache), _cache_base(v_cache), _p(_i32(block_table)),
                                 _p(_i32(context_lens)), _p(_i32(cu_seqlens)), _p(rows), int(rows.size), _p(out),
                                 scale, S, H, hkv, D, bs, int(block_table.shape[1]), DT[dt], stride, nthreads)
    return out[rows]


def cpu_attention_gathered(q, k_cache, v_cache, block_table, context_lens, scale: float, dt: str,
                           nthreads: int = 1) -> np.ndarray:
    """The reference CPU path (gather -> q.K^T*scale -> softmax -> .V), threaded."""
    B, H, D, hkv, bs, mb, stride = _decode_common(q, k_cache, block_table)
    out = np.zeros((B, H, D), np.float32)
    bt, cl = _i32(block_table), _i32(context_lens)
    lib().or_cpu_attention_gathered(_p(q), _cache_base(k_cache), _cache_base(v_cache), _p(bt), _p(cl), _p(out),
                                    scale, B, H, hkv, D, bs, mb, DT[dt], stride, nthreads)
    return out


def bf16_from_c(x: float) -> int:
    return int(lib().or_f32_to_bf16(float(x)))


def f16_from_c(x: float) -> int:
    return int(lib().or_f32_to_f16(float(x)))
