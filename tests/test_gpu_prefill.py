"""Packed causal prefill on the GPU against the textbook oracle.

There is no reference prefill kernel (crates/vllm-models/src/llama/attention.rs:128-132 routes
prefill through the decode op), so the contract is textbook causal attention over the paged
cache, row j of sequence s at position ctx_s - L_s + j.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from helpers import TORCH_DT, assert_close, dev_f32, i32, normal, to_dev
from oracle import oracle as orc
from railgun_amd import workloads as wl
from railgun_amd.ops import rope_cos_sin_table

pytestmark = pytest.mark.gpu


def sample_rows(cu, stride: int = 61, edge: int = 32) -> np.ndarray:
    """Packed row indices of every sequence: its first and last `edge` rows and every
    `stride`-th row in between (all rows of a sequence shorter than 2 * edge)."""
    rows = []
    for s in range(len(cu) - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        r = set(range(a, min(b, a + edge))) | set(range(max(a, b - edge), b)) | set(range(a, b, stride))
        rows.extend(sorted(r))
    return np.array(rows, np.int32)


def _threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _run(device, kernels, w: wl.PrefillWorkload, seed: int, check_seqs=None, max_query_len=None,
         row_sample: bool = False, row_stride: int = 61):
    dt = w.dtype
    rng = np.random.default_rng(seed)
    T, H, hkv, D, bs = w.num_tokens, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    q = normal(rng, (T, H, D), dt)
    k, v = normal(rng, (T, hkv, D), dt), normal(rng, (T, hkv, D), dt)
    # prior context (if any) already sits in the cache: random pool
    kc = normal(rng, (w.num_blocks, hkv, bs, D), dt)
    vc = normal(rng, (w.num_blocks, hkv, bs, D), dt)
    table = rope_cos_sin_table(int(w.context_lens.max()), D, w.rope_theta)
    dq, dkc, dvc = to_dev(q, dt, device), to_dev(kc, dt, device), to_dev(vc, dt, device)
    pos, slots = w.positions, w.slot_mapping
    kernels.launch_rope_reshape_and_cache(dq, to_dev(k, dt, device), to_dev(v, dt, device), dkc, dvc,
                                          table.to(device), i32(pos, device), i32(slots, device), H, hkv, D, bs, T)
    out = torch.full_like(dq, float("nan"))
    cu = w.cu_seqlens
    kernels.launch_prefill_packed(dq, dkc, dvc, i32(w.block_table, device), i32(w.context_lens, device),
                                  i32(cu, device), out, w.scale, H, hkv, D, bs, w.max_blocks, w.num_seqs, T,
                                  int(w.seq_lens.max()) if max_query_len is None else max_query_len)
    torch.cuda.synchronize()
    got = dev_f32(out)
    orc.rope_reshape_and_cache(q, k, v, kc, vc, table.numpy(), pos, slots, dt, bs)
    if row_sample:
        rows = sample_rows(cu, stride=row_stride)
        want = orc.prefill_packed_rows(q, kc, vc, w.block_table, w.context_lens, cu, rows, w.scale, dt,
                                       nthreads=_threads())
        for s in range(w.num_seqs):
            sel = (rows >= cu[s]) & (rows < cu[s + 1])
            assert sel.sum() >= min(64, int(cu[s + 1] - cu[s]))
            assert_close(got[rows[sel]], want[sel], dt, f"sequence {s} ({int(cu[s + 1] - cu[s])} rows)")
        return got
    seqs = range(w.num_seqs) if check_seqs is None else check_seqs
    for s in seqs:
        rows = slice(int(cu[s]), int(cu[s + 1]))
        want = orc.prefill_packed(np.ascontiguousarray(q[rows]), kc, vc, w.block_table[s:s + 1],
                                  w.context_lens[s:s + 1], np.array([0, cu[s + 1] - cu[s]], np.int32), w.scale, dt)
        assert_close(got[rows], want, dt, f"sequence {s}")
    return got


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_prefill_small_with_prior_context(device, kernels, dt):
    """Fresh sequences and chunked ones (prior context already cached), GQA 4, D 64."""
    rng = np.random.default_rng(4)
    lens = np.array([1, 5, 17, 40, 64], np.int32)
    prior = np.array([0, 0, 30, 0, 100], np.int32)
    bt = wl.assign_blocks(prior + lens, 16, 40, 16, rng)
    w = wl.PrefillWorkload("small", dt, 8, 2, 64, 16, 40, lens, bt, 4, prior=prior)
    _run(device, kernels, w, seed=44)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_prefill_config4(device, kernels, dt):
    """Config 4 (12 seqs, L U[128,2048], 32/8, D 128) at the shape the bench times: every row
    of every sequence (11,471 rows, the longest sequence 1,890), all 32 heads, against the
    oracle.  bf16 is the bench's headline prefill (2e-2 abs / 1e-2 rel); fp32, the reference's
    element type, is the bench's fp32_prefill side figure (1e-4)."""
    import dataclasses

    w = wl.config4()
    assert w.num_seqs == 12 and int(w.seq_lens.max()) == 1890 and w.num_tokens == 11471
    if dt != w.dtype:
        w = dataclasses.replace(w, dtype=dt)
    _run(device, kernels, w, seed=w.seed, row_sample=True, row_stride=1)


def _gqa_workload(G: int, D: int, lens, prior, seed: int, H: int = 32, mb: int = 0, dt: str = "bf16",
                  bs: int = 16) -> wl.PrefillWorkload:
    rng = np.random.default_rng(seed)
    lens, prior = np.asarray(lens, np.int32), np.asarray(prior, np.int32)
    hkv = H // G
    need = int(((prior + lens + bs - 1) // bs).sum())
    mb = mb or int(((prior + lens + bs - 1) // bs).max())
    bt = wl.assign_blocks(prior + lens, bs, need + 4, mb, rng)
    return wl.PrefillWorkload(f"gqa{G}_d{D}", dt, H, hkv, D, bs, need + 4, lens, bt, seed, prior=prior)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 7, 8, 16])
@pytest.mark.parametrize("D", [64, 128])
def test_prefill_mfma_gqa_ratios(device, kernels, G, D, dt):
    """The MFMA prefill kernels (bf16 and fp32) beyond GQA 4: one head per workgroup on four
    32-row subtiles (G 1, 3, 5, 7), two heads on two (G 2, 6: three workgroups of two heads per
    kv-head), one or several head groups of one kv-head (G 4, 8, 16).  Ragged units (1 to 200
    rows, lengths around the 32 / 64 / 128-row unit sizes), prior context, a sequence whose
    rows end inside a unit's first subtile; every row against the oracle."""
    H = 16 if G == 1 else 32 if 32 % G == 0 else 4 * G
    w = _gqa_workload(G, D, [1, 31, 33, 64, 65, 100, 129, 200, 7], [0, 0, 40, 0, 17, 300, 0, 64, 1000],
                      seed=100 + G + D, H=H, dt=dt)
    _run(device, kernels, w, seed=200 + G + D, row_sample=True, row_stride=1)


@pytest.mark.parametrize("bs", [16, 32, 8])
def test_prefill_f32_long_and_block_sizes(device, kernels, bs):
    """The fp32 MFMA prefill on longer sequences (up to 1,200 rows after up to 2,000 cached
    positions, GQA 4, head_dim 128) and at block sizes 8 / 32 as well as 16 (its key tiles
    address any block size); every sequence on a row sample against the oracle."""
    w = _gqa_workload(4, 128, [1200, 700, 333, 64], [0, 2000, 5, 100], seed=500 + bs, dt="f32", bs=bs)
    _run(device, kernels, w, seed=600 + bs, row_sample=True)


@pytest.mark.parametrize("bs", [32, 64, 128, 256])
@pytest.mark.parametrize("D,G,dt", [(128, 4, "bf16"), (64, 8, "f16"), (128, 3, "bf16")])
def test_prefill_mfma_block_sizes(device, kernels, bs, D, G, dt):
    """The 16-bit MFMA prefill at KV blocks of 16 << j tokens (a block holds 2^j of the kernel's
    16-token sub-blocks; its block-table window holds sub-block addresses): sequences of up to
    1,200 rows after up to 2,600 cached positions (the window moves past 128 sub-blocks), a
    sequence whose rows end inside a block, every sequence on a row sample against the oracle."""
    w = _gqa_workload(G, D, [1200, 700, 33, 5, 257], [0, 2600, 17, 250, 100], seed=800 + bs + D + G,
                      H=8 * G, dt=dt, bs=bs)
    _run(device, kernels, w, seed=900 + bs + D, row_sample=True)


@pytest.mark.parametrize("pad", [0, 8])
def test_prefill_fused_pool_and_odd_stride(device, kernels, pad):
    """Caches that are views of a larger pool: Railgun's fused [NB, 2, H_kv, bs, D] pool (block
    stride 2 H_kv bs D, a multiple of 16 D: the MFMA kernel) and, with pad 8, blocks 8 elements
    apart beyond their rows (a stride the MFMA kernel's sub-block addressing cannot express:
    the generic kernel takes it).  bf16, block 32, GQA 4, head_dim 128, against the oracle."""
    rng = np.random.default_rng(60 + pad)
    lens = np.array([300, 45, 129], np.int32)
    prior = np.array([0, 500, 64], np.int32)
    bs, H, hkv, D = 32, 32, 8, 128
    bt = wl.assign_blocks(prior + lens, bs, 40, 20, rng)
    T = int(lens.sum())
    ctx = prior + lens
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q = normal(rng, (T, H, D), "bf16")
    blk = hkv * bs * D
    pool = normal(rng, (40, 2 * blk + pad), "bf16")
    kv = [pool[:, i * blk:(i + 1) * blk].reshape(40, hkv, bs, D) for i in (0, 1)]
    dpool = to_dev(pool, "bf16", device)
    dk, dv = (dpool[:, i * blk:(i + 1) * blk].view(40, hkv, bs, D) for i in (0, 1))
    assert dk.stride(0) == 2 * blk + pad
    out = torch.full((T, H, D), float("nan"), dtype=torch.bfloat16, device=device)
    scale = 1.0 / math.sqrt(D)
    kernels.launch_prefill_packed(to_dev(q, "bf16", device), dk, dv, i32(bt, device), i32(ctx, device),
                                  i32(cu, device), out, scale, H, hkv, D, bs, 20, len(lens), T, int(lens.max()))
    torch.cuda.synchronize()
    want = orc.prefill_packed(q, kv[0], kv[1], bt, ctx, cu, scale, "bf16")
    assert_close(dev_f32(out), want, "bf16", f"pad {pad}")


@pytest.mark.parametrize("max_query_len", [None, 1])
def test_prefill_f32_understated_max_query_len(device, kernels, max_query_len):
    """fp32: with max_query_len = 1 one workgroup per sequence and head group walks every unit
    of its sequence, which must give the same result as the full grid."""
    w = _gqa_workload(4, 64, [33, 170, 5, 96], [300, 2100, 0, 40], seed=71, dt="f32", H=16)
    _run(device, kernels, w, seed=72, max_query_len=max_query_len)


@pytest.mark.parametrize("G", [1, 2, 8])
def test_prefill_mfma_gqa_long(device, kernels, G):
    """Longer sequences (up to 1,200 rows and 2,000 cached positions) for GQA 1, 2 and 8 (64 q /
    8 kv heads, Llama-3-70B-like), bf16 head_dim 128: many units per workgroup, every sequence
    on a row sample against the oracle."""
    H = 8 * G
    w = _gqa_workload(G, 128, [1200, 700, 333, 1023, 64], [0, 2000, 5, 0, 100], seed=300 + G, H=H)
    _run(device, kernels, w, seed=400 + G, row_sample=True)


@pytest.mark.parametrize("H,Hkv", [(24, 8), (28, 4), (40, 8)])
def test_prefill_gqa_model_shapes(device, kernels, H, Hkv):
    """Packed prefill at the head counts of models whose GQA ratio is no power of two, bf16
    head_dim 128: Llama-3.2-3B (24 / 8), Qwen2-7B (28 / 4), Qwen2.5-14B (40 / 8); config 4's
    sequence lengths (12 sequences, up to 1,890 rows, many units per workgroup), every sequence
    on a row sample against the oracle."""
    G = H // Hkv
    c4 = wl.config4()
    w = _gqa_workload(G, 128, c4.seq_lens, np.zeros_like(c4.seq_lens), seed=H + Hkv, H=H)
    _run(device, kernels, w, seed=H * Hkv, row_sample=True)


@pytest.mark.parametrize("max_query_len", [None, 1])
def test_prefill_long_prior_context(device, kernels, max_query_len):
    """Chunks after up to 4000 cached positions (the block-table window of the MFMA kernel moves
    past 128 blocks), bf16 D 128; with max_query_len = 1 the last tile rank of each sequence
    takes every tile, which must give the same result."""
    rng = np.random.default_rng(7)
    lens = np.array([33, 70, 5, 96], np.int32)
    prior = np.array([3000, 2100, 4000, 0], np.int32)
    bt = wl.assign_blocks(prior + lens, 16, 1000, 260, rng)
    w = wl.PrefillWorkload("long_prior", "bf16", 32, 8, 128, 16, 1000, lens, bt, 4, prior=prior)
    _run(device, kernels, w, seed=77, max_query_len=max_query_len)


@pytest.mark.parametrize("nseq", [200, 300])
def test_prefill_many_sequences(device, kernels, nseq):
    """Many short sequences, bf16 D 64 GQA 4 (MFMA path): 200 use the work-sorted schedule
    (its sequence scan crosses several 64-lane chunks), 300 exceed its LDS table and run in
    rank order; both must match the oracle."""
    rng = np.random.default_rng(nseq)
    lens = rng.integers(1, 70, nseq).astype(np.int32)
    prior = np.where(rng.random(nseq) < 0.3, rng.integers(1, 90, nseq), 0).astype(np.int32)
    need = int(((prior + lens + 15) // 16).sum())
    bt = wl.assign_blocks(prior + lens, 16, need + 8, 12, rng)
    w = wl.PrefillWorkload(f"many{nseq}", "bf16", 8, 2, 64, 16, need + 8, lens, bt, 5, prior=prior)
    _run(device, kernels, w, seed=nseq + 1, check_seqs=list(range(0, nseq, 7)))


def test_prefill_wide_table_rank_order(device, kernels):
    """A block table padded to 2200 entries (35,200 positions) puts the work-key bound past the
    sorted schedule's LDS table: the rank-order path, with prior context, bf16 D 128."""
    rng = np.random.default_rng(9)
    lens = np.array([33, 170, 5, 96], np.int32)
    prior = np.array([300, 2100, 0, 40], np.int32)
    bt = wl.assign_blocks(prior + lens, 16, 400, 2200, rng)
    w = wl.PrefillWorkload("wide_table", "bf16", 32, 8, 128, 16, 400, lens, bt, 4, prior=prior)
    _run(device, kernels, w, seed=99)


def test_prefill_repeated_launches_and_streams(device, kernels):
    """Repeatability: 140 launches of the MFMA kernel into four rotating outputs, then launches
    alternating between two streams without waits between them, all bit-equal to the first
    launch, which matches the oracle (bf16 D 128, with prior context).  The kernel keeps no
    state between launches (its schedule is computed per workgroup from the arguments), so any
    difference would be a race inside a launch."""
    rng = np.random.default_rng(21)
    lens = np.array([300, 45, 129, 800, 7], np.int32)
    prior = np.array([0, 500, 64, 0, 1000], np.int32)
    bt = wl.assign_blocks(prior + lens, 16, 300, 120, rng)
    w = wl.PrefillWorkload("queue", "bf16", 32, 8, 128, 16, 300, lens, bt, 4, prior=prior)
    first = _run(device, kernels, w, seed=23)
    # the same device inputs again (same generator, same draw order as _run)
    drng = np.random.default_rng(23)
    T, H, hkv, D, bs = w.num_tokens, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    q = normal(drng, (T, H, D), "bf16")
    k, v = normal(drng, (T, hkv, D), "bf16"), normal(drng, (T, hkv, D), "bf16")
    kc, vc = normal(drng, (w.num_blocks, hkv, bs, D), "bf16"), normal(drng, (w.num_blocks, hkv, bs, D), "bf16")
    table = rope_cos_sin_table(int(w.context_lens.max()), D, w.rope_theta)
    dq, dkc, dvc = to_dev(q, "bf16", device), to_dev(kc, "bf16", device), to_dev(vc, "bf16", device)
    kernels.launch_rope_reshape_and_cache(dq, to_dev(k, "bf16", device), to_dev(v, "bf16", device), dkc, dvc,
                                          table.to(device), i32(w.positions, device), i32(w.slot_mapping, device),
                                          H, hkv, D, bs, T)
    bt_d, ctx_d, cu_d = i32(w.block_table, device), i32(w.context_lens, device), i32(w.cu_seqlens, device)
    maxq = int(w.seq_lens.max())

    def launch(out):
        kernels.launch_prefill_packed(dq, dkc, dvc, bt_d, ctx_d, cu_d, out, w.scale, H, hkv, D, bs, w.max_blocks,
                                      w.num_seqs, T, maxq)

    outs = [torch.full_like(dq, float("nan")) for _ in range(4)]
    for i in range(140):
        launch(outs[i % 4])
        if i % 4 == 3:
            torch.cuda.synchronize()
            for o in outs:
                assert np.array_equal(dev_f32(o), first), f"launch {i}"
    streams = [torch.cuda.Stream(device=device), torch.cuda.Stream(device=device)]
    sides = [[torch.full_like(dq, float("nan")) for _ in range(3)] for _ in streams]
    torch.cuda.synchronize()
    for i in range(3):
        for st, side in zip(streams, sides):
            with torch.cuda.stream(st):
                launch(side[i])
    torch.cuda.synchronize()
    for side in sides:
        for o in side:
            assert np.array_equal(dev_f32(o), first)


@pytest.mark.parametrize("D,G,dt", [(64, 4, "bf16"), (128, 4, "bf16"), (128, 1, "bf16"), (128, 3, "bf16"),
                                    (64, 2, "f16"), (128, 3, "f32"), (128, 1, "f32")])
def test_prefill_rows_without_position(device, kernels, D, G, dt):
    """Context lengths shorter than the chunk (row j of s has position ctx_s - L_s + j): rows
    with a negative position are zeros and the others attend to positions 0..pos, as in the
    oracle; a sequence with no cached position at all is zeros throughout (MFMA paths).  With
    G = 1, 2, 3 a unit holds several 32-row subtiles, whose waves stop computing after their own
    last row: here some subtiles have only rows without a position, or none at all."""
    rng = np.random.default_rng(31 + D + 7 * G)
    lens = np.array([40, 100, 70, 33, 5, 130], np.int32)
    ctx = np.array([25, 10, 0, 33, 64, 40], np.int32)
    hkv, bs, nb, mb = 2, 16, 64, 9
    H = G * hkv
    bt = np.stack([rng.permutation(nb)[:mb] for _ in lens]).astype(np.int32)
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q = normal(rng, (T, H, D), dt)
    kc, vc = normal(rng, (nb, hkv, bs, D), dt), normal(rng, (nb, hkv, bs, D), dt)
    out = torch.full((T, H, D), float("nan"), dtype=TORCH_DT[dt], device=device)
    scale = 1.0 / math.sqrt(D)
    kernels.launch_prefill_packed(to_dev(q, dt, device), to_dev(kc, dt, device), to_dev(vc, dt, device),
                                  i32(bt, device), i32(ctx, device), i32(cu, device), out, scale, H, hkv, D, bs, mb,
                                  len(lens), T, int(lens.max()))
    torch.cuda.synchronize()
    want = orc.prefill_packed(q, kc, vc, bt, ctx, cu, scale, dt)
    got = dev_f32(out)
    assert not np.isnan(got).any()
    assert_close(got, want, dt, "rows without a position")
    assert np.all(got[cu[2]:cu[3]] == 0)
    assert np.all(got[cu[5]:cu[5] + 90] == 0)  # positions -90 .. -1


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_prefill_rising_scores(device, kernels, dt):
    """Scores that climb along the keys (about 9 log2 units per 32-key tile on average, up to
    33 where the oscillation on top rises), so that the running maximum keeps moving: the MFMA
    kernel's lazy maximum, which moves only when a tile's maximum passes it by more than its
    slack of 8 log2 units, moves on most tiles here and rescales the accumulated output each
    time.  GQA 4, head_dim 128, prior context, every row against the oracle."""
    rng = np.random.default_rng(57)
    D, H, hkv, bs = 128, 32, 8, 16
    lens = np.array([300, 150, 64, 1], np.int32)
    prior = np.array([200, 0, 900, 700], np.int32)
    ctx = prior + lens
    need = int(((ctx + bs - 1) // bs).sum())
    mb = int(((ctx + bs - 1) // bs).max())
    bt = wl.assign_blocks(ctx, bs, need + 4, mb, rng)
    nb = need + 4
    u = rng.choice([-1.0, 1.0], size=(hkv, D)).astype(np.float32)
    kc = (0.3 * rng.standard_normal((nb, hkv, bs, D))).astype(np.float32)
    vc = rng.standard_normal((nb, hkv, bs, D)).astype(np.float32)
    for s in range(len(lens)):
        t = np.arange(int(ctx[s]))
        g = 0.0077 * t + 0.9 * np.sin(t / 31.0)
        blk, off = bt[s, t // bs], t % bs
        kc[blk, :, off, :] += g[:, None, None] * u[None, :, :]
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q = (2.0 * np.repeat(u, H // hkv, axis=0)[None] + 0.3 * rng.standard_normal((T, H, D))).astype(np.float32)
    q, kc, vc = (orc.from_f32(x, dt) for x in (q, kc, vc))
    scale = 1.0 / math.sqrt(D)
    out = torch.full((T, H, D), float("nan"), dtype=TORCH_DT[dt], device=device)
    kernels.launch_prefill_packed(to_dev(q, dt, device), to_dev(kc, dt, device), to_dev(vc, dt, device),
                                  i32(bt, device), i32(ctx, device), i32(cu, device), out, scale, H, hkv, D, bs, mb,
                                  len(lens), T, int(lens.max()))
    torch.cuda.synchronize()
    want = orc.prefill_packed(q, kc, vc, bt, ctx, cu, scale, dt)
    got = dev_f32(out)
    assert not np.isnan(got).any()
    assert_close(got, want, dt, "rising scores")


def test_prefill_column_schedule_past_64_rounds(device, kernels):
    """The column split of the sorted schedule past a column's first 64 rounds, which the
    weighted greedy does not cover (those rounds go to the three workgroups of a CU in turn):
    256 q-heads over 64 kv-heads (64 head groups of 4, so 4 columns on a 256-CU device), 36
    sequences of 256 rows, every other one after cached positions: 288 units per group, 72
    rounds per column.  Every output row is written (the output starts as NaN) and 3 rows of
    each sequence match the oracle at every head."""
    rng = np.random.default_rng(64)
    H, hkv, D, bs, dt = 256, 64, 64, 16, "bf16"
    lens = np.full(36, 256, np.int32)
    prior = np.where(np.arange(36) % 2 == 1, rng.integers(1, 300, 36), 0).astype(np.int32)
    ctx = prior + lens
    mb = int(((ctx + bs - 1) // bs).max())
    nb = int(((ctx + bs - 1) // bs).sum()) + 4
    bt = wl.assign_blocks(ctx, bs, nb, mb, rng)
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q = normal(rng, (T, H, D), dt)
    kc, vc = normal(rng, (nb, hkv, bs, D), dt), normal(rng, (nb, hkv, bs, D), dt)
    scale = 1.0 / math.sqrt(D)
    out = torch.full((T, H, D), float("nan"), dtype=TORCH_DT[dt], device=device)
    kernels.launch_prefill_packed(to_dev(q, dt, device), to_dev(kc, dt, device), to_dev(vc, dt, device),
                                  i32(bt, device), i32(ctx, device), i32(cu, device), out, scale, H, hkv, D, bs, mb,
                                  len(lens), T, int(lens.max()))
    torch.cuda.synchronize()
    assert not bool(torch.isnan(out).any()), "rows left unwritten"
    rows = np.array([r for s in range(len(lens)) for r in (cu[s], cu[s] + 131, cu[s + 1] - 1)], np.int32)
    want = orc.prefill_packed_rows(q, kc, vc, bt, ctx, cu, rows, scale, dt, nthreads=_threads())
    assert_close(dev_f32(out[torch.from_numpy(rows).long().to(device)]), want, dt, "sampled rows")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_prefill_mfma_head_dim256(device, kernels, dt, G):
    """head_dim 256 on the MFMA kernels (16-bit: one workgroup per CU, a four-stage ring; fp32:
    one workgroup per CU, two 64 KB K/V buffers), every GQA grouping (one, two and four heads
    per workgroup): fresh and chunked sequences, a row shorter than a tile, blocks of 16 and 32
    tokens, every row against the oracle."""
    hkv = 2
    lens = np.array([1, 33, 100, 250], np.int32)
    prior = np.array([0, 40, 0, 300], np.int32)
    ctx = prior + lens
    for bs in (16, 32):
        rng = np.random.default_rng(2560 + 10 * G + bs)
        mb = int(((ctx + bs - 1) // bs).max())
        nb = int(((ctx + bs - 1) // bs).sum()) + 3
        bt = wl.assign_blocks(ctx, bs, nb, mb, rng)
        w = wl.PrefillWorkload("d256", dt, hkv * G, hkv, 256, bs, nb, lens, bt, 256, prior=prior)
        _run(device, kernels, w, seed=2561 + G + bs)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_prefill_head_dim256_many_units(device, kernels, dt):
    """head_dim 256 with several units per workgroup (16-bit: 4 head groups, 64 persistent
    workgroups each on a 256-CU device): 16 / 4 heads, 8 sequences of 400-1,500 rows after up to
    500 cached positions (~220 units per group), sampled rows of every sequence against the
    oracle."""
    rng = np.random.default_rng(2562)
    lens = rng.integers(400, 1500, 8, endpoint=True).astype(np.int32)
    prior = rng.integers(0, 500, 8, endpoint=True).astype(np.int32)
    ctx = prior + lens
    mb = int(((ctx + 15) // 16).max())
    nb = int(((ctx + 15) // 16).sum()) + 8
    bt = wl.assign_blocks(ctx, 16, nb, mb, rng)
    w = wl.PrefillWorkload("d256_many", dt, 16, 4, 256, 16, nb, lens, bt, 2562, prior=prior)
    assert int(((lens + 31) // 32).sum()) > 3 * 64
    _run(device, kernels, w, seed=2563, row_sample=True, row_stride=97)


def test_prefill_random_shapes(device, kernels):
    """Twelve seeded random packed batches, every row against the oracle: 1-24 sequences of
    1-300 rows after 0-400 cached positions, GQA 1 / 2 / 3 / 4 / 8 over 1-4 kv-heads (head groups
    that divide the CU count take the column split, the others the snake), head_dim 64 / 128,
    blocks of 16 / 32 tokens, bf16, fp16 and fp32."""
    rng = np.random.default_rng(4096)
    for case in range(12):
        S = int(rng.integers(1, 25))
        G = int(rng.choice([1, 2, 3, 4, 8]))
        hkv = int(rng.choice([1, 2, 4]))
        D = int(rng.choice([64, 128]))
        bs = int(rng.choice([16, 32]))
        dt = ("bf16", "f16", "f32")[case % 3]
        lens = rng.integers(1, 300, S, endpoint=True).astype(np.int32)
        prior = np.where(rng.random(S) < 0.5, rng.integers(0, 400, S, endpoint=True), 0).astype(np.int32)
        ctx = prior + lens
        mb = int(((ctx + bs - 1) // bs).max())
        nb = int(((ctx + bs - 1) // bs).sum()) + 2
        bt = wl.assign_blocks(ctx, bs, nb, mb, rng)
        w = wl.PrefillWorkload(f"random{case}", dt, G * hkv, hkv, D, bs, nb, lens, bt, 4096 + case, prior=prior)
        _run(device, kernels, w, seed=5000 + case)
