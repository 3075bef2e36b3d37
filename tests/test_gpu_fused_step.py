"""rg_rope_reshape_and_cache_paged_attention_v1 (the decode step's RoPE + cache pass fused into
the stream-K decode) against the two-entry chain it replaces — rg_rope_reshape_and_cache on a
copy of q, then rg_paged_attention_v1 over the updated pool — on the same inputs: output and
both caches bit for bit, q left unrotated; and against the oracle's chain
(rope_reshape_and_cache, then the reference CPU path over the gathered blocks, which restates
crates/vllm-cuda/src/kernels/paged_attention.cu:33-107).

The cases put the sequence's new token where the fused kernel handles it differently: in the
first unit a worker loads (short contexts, the prologue's loads), in later sub-blocks of
four-block units (head_dim 64), at blocks of 32 tokens, in fused K/V pools, with padding
tokens (slot -1: nothing written, the stale row attended as the chain does), with RoPE
positions other than context_len - 1, and with more and fewer units than workers.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, dev_f32, from_dev, i32, normal, to_dev
from oracle import oracle as orc
from railgun_amd import workloads as wl
from railgun_amd._lib import RailgunError

pytestmark = pytest.mark.gpu


def make_step(device, ctx, dt="bf16", H=32, Hkv=8, D=128, bs=16, seed=0, fused_pool=False, pad=(),
              positions=None):
    """One decode step's inputs: pool, block tables, contexts (each including its new token), the
    new tokens' q / k / v, RoPE positions (default ctx - 1) and slots (the table's slot of
    position ctx - 1, -1 for the sequences in `pad`)."""
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int32)
    B = len(ctx)
    mb = max(1, max((int(c) + bs - 1) // bs for c in ctx))
    nb = int(sum((int(c) + bs - 1) // bs for c in ctx)) + 5
    bt = wl.assign_blocks(ctx, bs, nb, mb, rng)
    p = ctx - 1
    slots = np.array([int(bt[s, p[s] // bs]) * bs + int(p[s]) % bs for s in range(B)], np.int32)
    for s in pad:
        slots[s] = -1
    pos = p.copy() if positions is None else np.asarray(positions, np.int32)
    if fused_pool:
        pool = normal(rng, (nb, 2, Hkv, bs, D), dt)
        kc, vc = pool[:, 0], pool[:, 1]
    else:
        pool = None
        kc, vc = normal(rng, (nb, Hkv, bs, D), dt), normal(rng, (nb, Hkv, bs, D), dt)
    q = normal(rng, (B, H, D), dt)
    k = normal(rng, (B, Hkv, D), dt)
    v = normal(rng, (B, Hkv, D), dt)
    from railgun_amd.ops import rope_cos_sin_table

    table = rope_cos_sin_table(int(max(int(pos.max()) + 1, 1)), D, 500000.0)
    return dict(ctx=ctx, bt=bt, slots=slots, pos=pos, pool=pool, kc=kc, vc=vc, q=q, k=k, v=v, table=table,
                H=H, Hkv=Hkv, D=D, bs=bs, mb=mb, B=B, dt=dt, scale=1.0 / math.sqrt(D))


def device_pool(st, device):
    """Fresh device copies of the caches (views of one fused pool when the step has one)."""
    if st["pool"] is not None:
        dpool = to_dev(st["pool"], st["dt"], device)
        return dpool[:, 0], dpool[:, 1]
    return to_dev(st["kc"], st["dt"], device), to_dev(st["vc"], st["dt"], device)


def run_chain(kernels, st, device):
    dq = to_dev(st["q"], st["dt"], device)
    dkc, dvc = device_pool(st, device)
    kernels.launch_rope_reshape_and_cache(dq, to_dev(st["k"], st["dt"], device), to_dev(st["v"], st["dt"], device),
                                          dkc, dvc, st["table"].to(device), i32(st["pos"], device),
                                          i32(st["slots"], device), st["H"], st["Hkv"], st["D"], st["bs"], st["B"])
    out = torch.full_like(dq, float("nan"))
    ws = workspace(kernels, st, device)
    kernels.launch_v1(dq, dkc, dvc, i32(st["bt"], device), i32(st["ctx"], device), out, st["scale"], st["H"],
                      st["Hkv"], st["D"], st["bs"], st["mb"], st["B"], workspace=ws)
    torch.cuda.synchronize()
    return out, dkc, dvc


def workspace(kernels, st, device):
    n = kernels.v1_workspace_bytes(st["B"], st["H"], st["Hkv"], st["D"], st["bs"], st["mb"])
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


def run_fused(kernels, st, device, dq=None):
    dq = to_dev(st["q"], st["dt"], device) if dq is None else dq
    dkc, dvc = device_pool(st, device)
    out = torch.full_like(dq, float("nan"))
    kernels.launch_rope_reshape_and_cache_v1(
        dq, to_dev(st["k"], st["dt"], device), to_dev(st["v"], st["dt"], device), dkc, dvc, st["table"].to(device),
        i32(st["pos"], device), i32(st["slots"], device), i32(st["bt"], device), i32(st["ctx"], device), out,
        st["scale"], st["H"], st["Hkv"], st["D"], st["bs"], st["mb"], st["B"], workspace(kernels, st, device))
    torch.cuda.synchronize()
    return out, dkc, dvc, dq


def check_against_chain(kernels, st, device, what):
    print(f"fused step: {what}", flush=True)
    out_c, kc_c, vc_c = run_chain(kernels, st, device)
    out_f, kc_f, vc_f, dq = run_fused(kernels, st, device)
    dt = st["dt"]
    np.testing.assert_array_equal(from_dev(dq, dt), st["q"], err_msg=f"{what}: q must stay unrotated")
    np.testing.assert_array_equal(from_dev(kc_f, dt), from_dev(kc_c, dt), err_msg=f"{what}: key cache")
    np.testing.assert_array_equal(from_dev(vc_f, dt), from_dev(vc_c, dt), err_msg=f"{what}: value cache")
    np.testing.assert_array_equal(from_dev(out_f, dt), from_dev(out_c, dt), err_msg=f"{what}: attention output")
    return out_f


CASES = {
    # name: (contexts or (B, lo, hi), kwargs)
    "short_contexts_d128_g4": ((24, 1, 40), dict()),
    "short_contexts_d64_g4": ((24, 1, 90), dict(D=64)),
    "d64_four_block_units": ((16, 60, 700), dict(D=64, seed=3)),
    "block32_d128_g2": ((12, 1, 500), dict(H=16, Hkv=8, bs=32, seed=4)),
    "block64_d64_g1": ((10, 1, 400), dict(H=8, Hkv=8, D=64, bs=64, seed=5)),
    "g8_fused_pool": ((9, 30, 900), dict(H=32, Hkv=4, fused_pool=True, seed=6)),
    "padding_tokens": ((20, 1, 300), dict(pad=(0, 3, 7, 19), seed=7)),
    "f16_d128_g4": ((16, 1, 600), dict(dt="f16", seed=8)),
    "more_units_than_workers": ([5000, 7000, 4321], dict(seed=9)),
    "one_token_sequences": ([1] * 40, dict(seed=10)),
    "llama32_3b_g3_d128": ((20, 1, 900), dict(H=24, Hkv=8, seed=13)),
    "qwen2_7b_g7_d128": ((12, 1, 700), dict(H=28, Hkv=4, seed=14)),
    "g5_d64": ((16, 1, 500), dict(H=40, Hkv=8, D=64, seed=15)),
    "g6_d64_block32": ((14, 1, 400), dict(H=24, Hkv=4, D=64, bs=32, seed=16)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_fused_step_matches_chain(device, kernels, name):
    spec, kw = CASES[name]
    if isinstance(spec, tuple):
        B, lo, hi = spec
        ctx = np.random.default_rng(sum(map(ord, name))).integers(lo, hi + 1, size=B)
    else:
        ctx = spec
    st = make_step(device, ctx, **kw)
    check_against_chain(kernels, st, device, name)


def test_fused_step_rope_positions_not_at_the_end(device, kernels):
    """RoPE positions independent of the context length (the rotation reads positions[s] only)."""
    rng = np.random.default_rng(11)
    ctx = rng.integers(1, 400, size=18)
    st = make_step(device, ctx, positions=rng.integers(0, 9000, size=18), seed=11)
    check_against_chain(kernels, st, device, "positions")


def test_fused_step_config2_against_chain_and_oracle(device, kernels):
    """The bench's config-2 step at full size (64 sequences, contexts U[512, 4096], bf16, 32/8,
    D 128, block 16, theta 5e5): bit-equal to the chain, and within the bf16 tolerance of the
    oracle's chain."""
    w = wl.config2()
    st = make_step(device, w.context_lens, seed=w.seed + 7)
    out = check_against_chain(kernels, st, device, "config 2")
    q, kc, vc = st["q"].copy(), st["kc"].copy(), st["vc"].copy()
    orc.rope_reshape_and_cache(q, st["k"], st["v"], kc, vc, st["table"].numpy(), st["pos"], st["slots"], "bf16",
                               st["bs"])
    want = orc.cpu_attention_gathered(q, kc, vc, st["bt"], st["ctx"], st["scale"], "bf16", nthreads=8)
    assert_close(dev_f32(out), want, "bf16", "config-2 fused step vs the oracle's chain")


def test_fused_step_small_against_oracle(device, kernels):
    """A small step against the oracle's chain directly (short contexts, one padding token)."""
    st = make_step(device, [1, 17, 33, 5, 130, 64], H=8, Hkv=2, D=64, pad=(3,), seed=12)
    out, kc, vc, _ = run_fused(kernels, st, device)
    q, okc, ovc = st["q"].copy(), st["kc"].copy(), st["vc"].copy()
    orc.rope_reshape_and_cache(q, st["k"], st["v"], okc, ovc, st["table"].numpy(), st["pos"], st["slots"], "bf16",
                               st["bs"])
    np.testing.assert_array_equal(from_dev(kc, "bf16"), okc)
    np.testing.assert_array_equal(from_dev(vc, "bf16"), ovc)
    want = orc.cpu_attention_gathered(q, okc, ovc, st["bt"], st["ctx"], st["scale"], "bf16", nthreads=8)
    assert_close(dev_f32(out), want, "bf16", "small fused step vs the oracle")


@pytest.mark.parametrize("kw", [dict(dt="f32"), dict(H=32, Hkv=2), dict(D=256)])
def test_fused_step_rejects_other_shapes(device, kernels, kw):
    """fp32, GQA ratios above 8 and head_dim 256 are refused with RG_ERR_NOT_SUPPORTED
    (the chain of two entries covers them); nothing is launched."""
    st = make_step(device, [40, 70], **kw)
    with pytest.raises(RailgunError, match="not supported|runs at"):
        run_fused(kernels, st, device)
