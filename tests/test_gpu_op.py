"""PagedAttentionOp / PagedAttentionKernels used the way Railgun uses them.

``test_paged_attention_parity`` follows crates/vllm-cuda/tests/test_paged_attention.rs:8-204
(B=2, H=H_kv=4, D=64, bs=16, 64 blocks per sequence, ctx=512, sequential block table; v1 vs
v1+ vs v2 at 1e-4), with seeded inputs and an identity rotation (the reference passes zeroed
metadata, which makes its v1+/v2 outputs zero).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, dev_f32, from_dev, i32, normal, to_dev
from oracle import oracle as orc
from railgun_amd import workloads as wl
from railgun_amd.ops import PagedAttentionOp, RailgunError, rope_cos_sin_table

pytestmark = pytest.mark.gpu


def test_paged_attention_parity(device, kernels):
    batch_size, num_heads, num_kv_heads, head_dim, block_size = 2, 4, 4, 64, 16
    max_blocks_per_seq, context_len = 64, 512
    scale = 1.0 / math.sqrt(head_dim)
    g = torch.Generator(device="cpu").manual_seed(0)
    q = torch.randn((batch_size, num_heads, head_dim), generator=g).to(device)
    k_cache = torch.randn((max_blocks_per_seq * batch_size, num_kv_heads, block_size, head_dim), generator=g).to(device)
    v_cache = torch.randn((max_blocks_per_seq * batch_size, num_kv_heads, block_size, head_dim), generator=g).to(device)
    bt = torch.arange(batch_size * max_blocks_per_seq, dtype=torch.int32).reshape(batch_size, -1).to(device)
    context_lens = torch.full((batch_size,), context_len, dtype=torch.int32, device=device)
    rotation_metadata = torch.tensor([0, 0, 0, 1, 0, 0, 0, 1] * batch_size * num_heads, dtype=torch.float32,
                                     device=device)

    out_v1 = torch.zeros_like(q)
    out_v1_plus = torch.zeros_like(q)
    out_v2 = torch.zeros_like(q)
    kernels.launch_v1(q, k_cache, v_cache, bt, context_lens, out_v1, scale, num_heads, num_kv_heads, head_dim,
                      block_size, max_blocks_per_seq, batch_size)
    kernels.launch_v1_plus(q, k_cache, v_cache, bt, context_lens, out_v1_plus, rotation_metadata, scale,
                           num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size)
    num_partitions = (context_len + 255) // 256
    tmp_out = torch.zeros((batch_size * num_heads * num_partitions * head_dim,), device=device)
    exp_sums = torch.zeros((batch_size * num_heads * num_partitions,), device=device)
    max_logits = torch.zeros((batch_size * num_heads * num_partitions,), device=device)
    kernels.launch_v2_partition(q, k_cache, v_cache, bt, context_lens, tmp_out, exp_sums, max_logits,
                                rotation_metadata, scale, num_heads, num_kv_heads, head_dim, block_size,
                                max_blocks_per_seq, num_partitions, batch_size)
    kernels.launch_v2_reduce(out_v2, exp_sums, max_logits, tmp_out, context_lens, rotation_metadata, num_heads,
                             head_dim, num_partitions, batch_size)
    torch.cuda.synchronize()
    v1, v1p, v2 = (t.cpu().numpy().ravel() for t in (out_v1, out_v1_plus, out_v2))
    epsilon = 1e-4
    assert np.abs(v1 - v1p).max() <= epsilon
    assert np.abs(v1 - v2).max() <= epsilon
    want = orc.paged_attention_v1(q.cpu().numpy(), k_cache.cpu().numpy(), v_cache.cpu().numpy(), bt.cpu().numpy(),
                                  context_lens.cpu().numpy(), scale, "f32").ravel()
    assert np.abs(v1 - want).max() <= epsilon


@pytest.mark.parametrize("max_ctx", [300, 4096, 5000])
def test_execute_dispatch(device, kernels, max_ctx):
    """execute(): v1 for max_context_len <= 4096, v2 above (paged_attn_op.rs:89); same result."""
    rng = np.random.default_rng(max_ctx)
    ctx = np.array([max_ctx, 1, max_ctx // 3, 0], np.int32)
    H, hkv, D, bs = 16, 4, 128, 16
    need = int(sum((c + bs - 1) // bs for c in ctx))
    bt = wl.assign_blocks(ctx, bs, need + 2, (max_ctx + bs - 1) // bs, rng)
    q = normal(rng, (4, H, D), "bf16")
    kc, vc = normal(rng, (need + 2, hkv, bs, D), "bf16"), normal(rng, (need + 2, hkv, bs, D), "bf16")
    op = PagedAttentionOp(1 / math.sqrt(D), H, hkv, D, bs, kernels)
    out = op.execute(to_dev(q, "bf16", device), to_dev(kc, "bf16", device), to_dev(vc, "bf16", device),
                     i32(bt, device), i32(ctx, device), None, int(ctx.max()))
    torch.cuda.synchronize()
    want = orc.paged_attention_v1_plus(q, kc, vc, bt, ctx, 1 / math.sqrt(D), "bf16")
    assert_close(dev_f32(out), want, "bf16")


def test_op_cache_and_rope_methods(device, kernels):
    """reshape_and_cache (with and without IsoQuant) and apply_rope through the op."""
    rng = np.random.default_rng(9)
    T, H, hkv, D, bs, nb = 6, 8, 2, 64, 16, 4
    op = PagedAttentionOp(0.125, H, hkv, D, bs, kernels)
    k, v = normal(rng, (T, hkv, D), "bf16"), normal(rng, (T, hkv, D), "bf16")
    slots = np.array([0, 17, -1, 33, 48, 5], np.int32)
    for iso in (False, True):
        kc = torch.zeros((nb, hkv, bs, D), dtype=torch.bfloat16, device=device)
        vc = torch.zeros_like(kc)
        meta = torch.zeros((nb, hkv, D // 4, 8), dtype=torch.float32, device=device)
        op.reshape_and_cache(to_dev(k, "bf16", device), to_dev(v, "bf16", device), kc, vc, i32(slots, device),
                             meta, iso)
        hk = np.zeros((nb, hkv, bs, D), np.uint16)
        hv = np.zeros_like(hk)
        hm = np.zeros((nb, hkv, D // 4, 8), np.float32)
        orc.reshape_and_cache(k, v, hk, hv, slots, "bf16", bs, rotation_metadata=hm if iso else None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(kc, "bf16"), hk)
        np.testing.assert_array_equal(from_dev(vc, "bf16"), hv)
        np.testing.assert_array_equal(meta.cpu().numpy(), hm)
    x = normal(rng, (T, H, D), "bf16")
    pos = np.arange(T, dtype=np.int32) * 7
    table = rope_cos_sin_table(64, D, 10000.0)
    dx = to_dev(x, "bf16", device)
    op.apply_rope(dx, table.to(device), i32(pos, device))
    torch.cuda.synchronize()
    orc.rope(x, table.numpy(), pos, "bf16")
    np.testing.assert_array_equal(from_dev(dx, "bf16"), x)


def test_argument_errors(device, kernels):
    """Argument checks mirror CoreError::NotSupported / Tensor (mod.rs:42-54, 477-482)."""
    q = torch.zeros((1, 4, 66), device=device)
    kc = torch.zeros((2, 4, 16, 66), device=device)
    bt = torch.zeros((1, 2), dtype=torch.int32, device=device)
    cl = torch.ones((1,), dtype=torch.int32, device=device)
    with pytest.raises(RailgunError, match="head_dim must be a multiple of 4"):
        kernels.launch_v1_plus(q, kc, kc, bt, cl, q, None, 1.0, 4, 4, 66, 16, 2, 1)
    with pytest.raises(RailgunError, match="exceeds maximum block size"):
        kernels.launch_v2_reduce(q, cl.float(), cl.float(), q, cl, None, 4, 2048, 1, 1)
    ws = torch.empty(16, dtype=torch.uint8, device=device)
    q2 = torch.zeros((1, 4, 64), device=device)
    kc2 = torch.zeros((64, 4, 16, 64), device=device)
    bt2 = torch.zeros((1, 64), dtype=torch.int32, device=device)
    with pytest.raises(RailgunError, match="not a multiple of num_kv_heads"):
        kernels.launch_v1(q2, kc2, kc2, bt2, cl, q2, 1.0, 4, 3, 64, 16, 64, 1)
    with pytest.raises(RailgunError, match="workspace"):
        kernels.launch_v1(q2, kc2, kc2, bt2, cl, q2, 1.0, 4, 4, 64, 16, 64, 1, workspace=ws)
