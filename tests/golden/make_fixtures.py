"""Writes the golden fixtures of tests/golden/ (run from the repository root).

The reference repository holds no golden vectors for this path, so the expected outputs
here come from textbook formulas evaluated in float64 numpy — independently of the C
oracle (oracle/oracle.c) and of the HIP kernels.  Inputs are not stored: they are
regenerated from the seeds below, and their SHA-256 is stored so that any drift of the
generator is detected before a comparison is made.

    python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import hashlib
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from railgun_amd import workloads as wl  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (NaN-free inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def bf16_to_f64(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


# ------------------------------------------------------------------ inputs ---

def config1_inputs():
    """Config 1: fp32, ctx 17/64/130/255, 32/8 heads, D 64, 256 blocks."""
    w = wl.config1()
    rng = np.random.default_rng(2001)
    q = rng.standard_normal((w.batch, w.num_heads, w.head_dim), dtype=np.float32)
    shape = (w.num_blocks, w.num_kv_heads, w.block_size, w.head_dim)
    kc = rng.standard_normal(shape, dtype=np.float32)
    vc = rng.standard_normal(shape, dtype=np.float32)
    k_new = rng.standard_normal((w.batch, w.num_kv_heads, w.head_dim), dtype=np.float32)
    v_new = rng.standard_normal((w.batch, w.num_kv_heads, w.head_dim), dtype=np.float32)
    return w, q, kc, vc, k_new, v_new


def small_bf16_inputs():
    """A small bf16 decode with the config-2 head shape (32/8 heads, D 128)."""
    rng = np.random.default_rng(2002)
    ctx = np.array([40, 1, 130, 77], np.int32)
    bt = wl.assign_blocks(ctx, 16, 24, 10, rng)
    q = bf16_round(rng.standard_normal((4, 32, 128), dtype=np.float32))
    kc = bf16_round(rng.standard_normal((24, 8, 16, 128), dtype=np.float32))
    vc = bf16_round(rng.standard_normal((24, 8, 16, 128), dtype=np.float32))
    return ctx, bt, q, kc, vc


def rope_inputs():
    rng = np.random.default_rng(2003)
    x = rng.standard_normal((7, 3, 128), dtype=np.float32)
    pos = np.array([0, 1, 2, 100, 511, 4095, 32767], np.int32)
    return x, pos


# -------------------------------------------------------------- references ---

def attention_f64(q, kc, vc, bt, ctx, scale, to64=lambda a: a.astype(np.float64)):
    """softmax(scale * q.K^T) V per (sequence, q-head), K/V gathered through the block table,
    q-head h reading kv-head h // (H / H_kv)."""
    B, H, D = q.shape
    hkv, bs = kc.shape[1], kc.shape[2]
    g = H // hkv
    out = np.zeros((B, H, D), np.float64)
    for s in range(B):
        n = int(ctx[s])
        if n == 0:
            continue
        tok = np.arange(n)
        blk = bt[s, tok // bs]
        off = tok % bs
        for h in range(H):
            K = to64(kc[blk, h // g, off])  # [n, D]
            V = to64(vc[blk, h // g, off])
            sc = K @ to64(q[s, h]) * scale
            p = np.exp(sc - sc.max())
            out[s, h] = (p / p.sum()) @ V
    return out


def rope_table_f64(max_pos: int, D: int, theta: float) -> np.ndarray:
    half = D // 2
    inv = theta ** (-2.0 * np.arange(half) / D)
    ang = np.arange(max_pos)[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1)


def main() -> None:
    w, q, kc, vc, k_new, v_new = config1_inputs()
    out = attention_f64(q, kc, vc, w.block_table, w.context_lens, w.scale)
    slots = w.slot_mapping
    kc2, vc2 = kc.copy(), vc.copy()
    for t, sl in enumerate(slots):
        kc2[sl // 16, :, sl % 16] = k_new[t]
        vc2[sl // 16, :, sl % 16] = v_new[t]
    slots_skip = slots.copy()
    slots_skip[2] = -1
    kc3, vc3 = kc.copy(), vc.copy()
    for t, sl in enumerate(slots_skip):
        if sl >= 0:
            kc3[sl // 16, :, sl % 16] = k_new[t]
            vc3[sl // 16, :, sl % 16] = v_new[t]
    np.savez_compressed(
        os.path.join(HERE, "config1_fp32.npz"),
        input_sha256=np.array(sha(q, kc, vc, w.block_table, w.context_lens, k_new, v_new)),
        context_lens=w.context_lens, block_table=w.block_table, scale=np.float64(w.scale),
        expected_out_f64=out, slot_mapping=slots, slot_mapping_skip=slots_skip,
        cache_after_sha256=np.array(sha(kc2, vc2)), cache_after_skip_sha256=np.array(sha(kc3, vc3)),
    )

    ctx, bt, qb, kcb, vcb = small_bf16_inputs()
    outb = attention_f64(qb, kcb, vcb, bt, ctx, 1.0 / math.sqrt(128), to64=bf16_to_f64)
    np.savez_compressed(os.path.join(HERE, "decode_bf16_small.npz"),
                        input_sha256=np.array(sha(qb, kcb, vcb, bt, ctx)), context_lens=ctx, block_table=bt,
                        expected_out_f64=outb)

    x, pos = rope_inputs()
    table = rope_table_f64(32768, 128, 500000.0)
    half = 64
    c, s_ = table[pos, :half][:, None, :], table[pos, half:][:, None, :]
    lo, hi = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    y = np.concatenate([lo * c - hi * s_, hi * c + lo * s_], axis=-1)
    np.savez_compressed(os.path.join(HERE, "rope_theta5e5.npz"), input_sha256=np.array(sha(x, pos)), positions=pos,
                        expected_out_f64=y, table_rows_f64=table[pos])
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
