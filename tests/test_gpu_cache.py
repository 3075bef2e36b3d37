"""reshape_and_cache, IsoQuant metadata, RoPE and fused RoPE + cache write on the GPU.

All of these are bit-exact against the oracle: the scatter is a copy
(crates/vllm-cuda/src/kernels/paged_attention.cu:121-137) and the RoPE arithmetic
(rope.cu:34-41) is evaluated with separately rounded products on both sides.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import from_dev, i32, normal, to_dev
from oracle import oracle as orc
from railgun_amd import workloads as wl
from railgun_amd.ops import rope_cos_sin_table

pytestmark = pytest.mark.gpu


def _slots(rng, T, nb, bs, with_skip=True):
    slots = rng.choice(nb * bs, size=T, replace=False).astype(np.int32)
    if with_skip and T > 1:
        slots[1] = -1
    return slots


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [64, 128, 6])
def test_reshape_and_cache_bit_exact(device, kernels, dt, D):
    rng = np.random.default_rng(D)
    T, hkv, bs, nb = 37, 8, 16, 12
    k, v = normal(rng, (T, hkv, D), dt), normal(rng, (T, hkv, D), dt)
    kc, vc = normal(rng, (nb, hkv, bs, D), dt), normal(rng, (nb, hkv, bs, D), dt)
    slots = _slots(rng, T, nb, bs)
    dkc, dvc = to_dev(kc, dt, device), to_dev(vc, dt, device)
    kernels.launch_reshape_and_cache(to_dev(k, dt, device), to_dev(v, dt, device), dkc, dvc, i32(slots, device),
                                     hkv, D, bs, T)
    torch.cuda.synchronize()
    orc.reshape_and_cache(k, v, kc, vc, slots, dt, bs)
    np.testing.assert_array_equal(from_dev(dkc, dt).view(np.uint8), kc.view(np.uint8))
    np.testing.assert_array_equal(from_dev(dvc, dt).view(np.uint8), vc.view(np.uint8))


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_reshape_and_cache_fused_pool_and_isoquant(device, kernels, dt):
    """Fused [NB, 2, H_kv, bs, D] pool (block.rs:70) and identity IsoQuant metadata."""
    rng = np.random.default_rng(3)
    T, hkv, bs, nb, D = 20, 4, 16, 6, 64
    k, v = normal(rng, (T, hkv, D), dt), normal(rng, (T, hkv, D), dt)
    pool = normal(rng, (nb, 2, hkv, bs, D), dt)
    slots = _slots(rng, T, nb, bs)
    # offset 0 of block 2 gets a token, so its metadata is written
    dup = np.nonzero(slots == 2 * bs)[0]
    if len(dup):
        slots[dup[0]] = slots[0]
    slots[0] = 2 * bs
    meta = np.full((nb, hkv, D // 4, 8), 7.0, np.float32)
    dpool = to_dev(pool, dt, device)
    dmeta = torch.from_numpy(meta.copy()).to(device)
    kernels.launch_reshape_and_cache_isoquant(to_dev(k, dt, device), to_dev(v, dt, device), dpool[:, 0],
                                              dpool[:, 1], i32(slots, device), dmeta, hkv, D, bs, T)
    torch.cuda.synchronize()
    orc.reshape_and_cache(k, v, pool[:, 0], pool[:, 1], slots, dt, bs, kv_block_stride=2 * hkv * bs * D,
                          rotation_metadata=meta)
    np.testing.assert_array_equal(from_dev(dpool, dt).view(np.uint8), pool.view(np.uint8))
    np.testing.assert_array_equal(dmeta.cpu().numpy(), meta)
    assert (meta[2].reshape(-1, 8) == np.array([0, 0, 0, 1, 0, 0, 0, 1], np.float32)).all()


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [64, 128, 6])
def test_rope_bit_exact(device, kernels, dt, D):
    rng = np.random.default_rng(100 + D)
    T, H = 29, 5
    x = normal(rng, (T, H, D), dt)
    pos = rng.integers(0, 4000, size=T).astype(np.int32)
    table = rope_cos_sin_table(4000, D, 500000.0)
    dx = to_dev(x, dt, device)
    kernels.launch_rope(dx, table.to(device), i32(pos, device), H, D, T)
    torch.cuda.synchronize()
    orc.rope(x, table.numpy(), pos, dt)
    np.testing.assert_array_equal(from_dev(dx, dt).view(np.uint8), x.view(np.uint8))


@pytest.mark.parametrize("which", ["config2", "config4", "small", "small_f16"])
def test_rope_reshape_and_cache_bit_exact(device, kernels, which):
    """Fused pass == rope(q), rope(k) + scatter, at the decode (T=64) and prefill (T~13k) sizes."""
    if which == "config2":
        w = wl.config2()
        T, H, hkv, D, bs, nb, dt = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, \
            w.num_blocks, "bf16"
        pos, slots = w.positions, w.slot_mapping
    elif which == "config4":
        w = wl.config4()
        T, H, hkv, D, bs, nb, dt = w.num_tokens, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, \
            w.num_blocks, "bf16"
        pos, slots = w.positions, w.slot_mapping
    elif which == "small_f16":  # the 16-byte kernel with D 64, f16, some padding slots
        T, H, hkv, D, bs, nb, dt = 37, 8, 2, 64, 16, 9, "f16"
        rng0 = np.random.default_rng(2)
        pos = rng0.integers(0, 300, size=T).astype(np.int32)
        slots = _slots(rng0, T, nb, bs)
        slots[[3, 17]] = -1
    else:
        T, H, hkv, D, bs, nb, dt = 9, 4, 2, 6, 4, 5, "f32"
        rng0 = np.random.default_rng(1)
        pos = rng0.integers(0, 50, size=T).astype(np.int32)
        slots = _slots(rng0, T, nb, bs)
    rng = np.random.default_rng(T)
    q, k, v = normal(rng, (T, H, D), dt), normal(rng, (T, hkv, D), dt), normal(rng, (T, hkv, D), dt)
    if which.startswith("small"):
        kc, vc = normal(rng, (nb, hkv, bs, D), dt), normal(rng, (nb, hkv, bs, D), dt)
    else:  # large pools: zero-filled, so untouched rows are checked against zeros
        kc = np.zeros((nb, hkv, bs, D), orc.NP_STORAGE[dt])
        vc = np.zeros_like(kc)
    table = rope_cos_sin_table(int(pos.max()) + 1, D, 500000.0)
    dq, dk = to_dev(q, dt, device), to_dev(k, dt, device)
    dkc, dvc = to_dev(kc, dt, device), to_dev(vc, dt, device)
    kernels.launch_rope_reshape_and_cache(dq, dk, to_dev(v, dt, device), dkc, dvc, table.to(device),
                                          i32(pos, device), i32(slots, device), H, hkv, D, bs, T)
    torch.cuda.synchronize()
    k_before = k.copy()
    orc.rope_reshape_and_cache(q, k, v, kc, vc, table.numpy(), pos, slots, dt, bs)
    np.testing.assert_array_equal(from_dev(dq, dt).view(np.uint8), q.view(np.uint8))
    np.testing.assert_array_equal(from_dev(dk, dt).view(np.uint8), k_before.view(np.uint8))
    np.testing.assert_array_equal(from_dev(dkc, dt).view(np.uint8), kc.view(np.uint8))
    np.testing.assert_array_equal(from_dev(dvc, dt).view(np.uint8), vc.view(np.uint8))
