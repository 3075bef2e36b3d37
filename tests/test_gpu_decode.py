"""Paged decode attention (v1, v1_plus, v2) on the GPU against the CPU oracle.

The oracle restates crates/vllm-cuda/src/kernels/paged_attention.cu:33-107 (v1),
paged_attention_v1_plus.cu:37-105 and paged_attention_v2_{partition,reduce}.cu; inputs are
seeded, bf16/f16 inputs are rounded once and the oracle sees the same bits.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from helpers import TORCH_DT, assert_close, dev_f32, from_dev, i32, normal, to_dev
from oracle import oracle as orc
from railgun_amd import workloads as wl

pytestmark = pytest.mark.gpu


def make_inputs(device, ctx, dt, H=32, Hkv=8, D=128, bs=16, seed=0, extra_blocks=3, fused=False, mb=None):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int32)
    need = int(sum((int(c) + bs - 1) // bs for c in ctx))
    nb = need + extra_blocks
    mb = mb or max(1, max((int(c) + bs - 1) // bs for c in ctx))
    bt = wl.assign_blocks(ctx, bs, nb, mb, rng)
    q = normal(rng, (len(ctx), H, D), dt)
    if fused:
        pool = normal(rng, (nb, 2, Hkv, bs, D), dt)
        kc, vc = pool[:, 0], pool[:, 1]
        dpool = to_dev(pool, dt, device)
        dkc, dvc = dpool[:, 0], dpool[:, 1]
    else:
        kc = normal(rng, (nb, Hkv, bs, D), dt)
        vc = normal(rng, (nb, Hkv, bs, D), dt)
        dkc, dvc = to_dev(kc, dt, device), to_dev(vc, dt, device)
    return dict(ctx=ctx, bt=bt, q=q, kc=kc, vc=vc, H=H, Hkv=Hkv, D=D, bs=bs, mb=mb, dt=dt,
                scale=1.0 / math.sqrt(D), dq=to_dev(q, dt, device), dkc=dkc, dvc=dvc,
                dbt=i32(bt, device), dctx=i32(ctx, device))


def oracle_v1_plus(inp):
    return orc.paged_attention_v1_plus(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"],
                                       inp["dt"])


def gpu_v1(kernels, inp, workspace: bool, entry: str = "v1"):
    B = len(inp["ctx"])
    out = torch.full_like(inp["dq"], float("nan"))
    ws = None
    if workspace:
        nbytes = kernels.v1_workspace_bytes(B, inp["H"], inp["Hkv"], inp["D"], inp["bs"], inp["mb"])
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=inp["dq"].device)
    args = (inp["dq"], inp["dkc"], inp["dvc"], inp["dbt"], inp["dctx"], out)
    tail = (inp["scale"], inp["H"], inp["Hkv"], inp["D"], inp["bs"], inp["mb"], B)
    if entry == "v1":
        kernels.launch_v1(*args, *tail, workspace=ws)
    else:
        kernels.launch_v1_plus(*args, None, *tail, workspace=ws)
    torch.cuda.synchronize()
    return dev_f32(out)


def gpu_v2(kernels, inp, P):
    B = len(inp["ctx"])
    out = torch.full_like(inp["dq"], float("nan"))
    max_ctx = int(inp["ctx"].max())
    np_ = max(1, math.ceil(max_ctx / P))
    ws = torch.empty(kernels.v2_workspace_bytes(B, inp["H"], np_, inp["D"]), dtype=torch.uint8,
                     device=inp["dq"].device)
    kernels.launch_v2(inp["dq"], inp["dkc"], inp["dvc"], inp["dbt"], inp["dctx"], out, inp["scale"], inp["H"],
                      inp["Hkv"], inp["D"], inp["bs"], inp["mb"], B, max_ctx, P, ws)
    torch.cuda.synchronize()
    return dev_f32(out)


def test_config1_fp32_all_entries(device, kernels):
    """Config 1 (fp32, ctx 17/64/130/255, 32/8 heads, D 64): every decode entry at 1e-4."""
    w = wl.config1()
    rng = np.random.default_rng(w.seed)
    inp = make_inputs(device, w.context_lens, "f32", H=32, Hkv=8, D=64, seed=w.seed)
    # The config's own table (256-block pool, seeded permutation) replaces the helper's.
    inp["kc"] = normal(rng, (w.num_blocks, 8, 16, 64), "f32")
    inp["vc"] = normal(rng, (w.num_blocks, 8, 16, 64), "f32")
    inp["bt"], inp["mb"] = w.block_table, w.max_blocks
    inp["dkc"], inp["dvc"] = to_dev(inp["kc"], "f32", device), to_dev(inp["vc"], "f32", device)
    inp["dbt"] = i32(w.block_table, device)
    want_v1 = orc.paged_attention_v1(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], "f32")
    want = oracle_v1_plus(inp)
    np.testing.assert_allclose(want_v1, want, atol=1e-5, rtol=1e-5)
    for ws in (False, True):
        for entry in ("v1", "v1_plus"):
            assert_close(gpu_v1(kernels, inp, ws, entry), want, "f32", f"{entry} ws={ws}")
    for P in (16, 64, 256):
        assert_close(gpu_v2(kernels, inp, P), want, "f32", f"v2 P={P}")


CTX_RAGGED = [1, 15, 16, 17, 33, 300, 0, 511, 1024]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 7, 8, 16])
def test_mfma_path_shapes(device, kernels, dt, D, G):
    """MFMA kernels (block 16): every GQA ratio (3, 5, 6, 7 fill the 16 operand rows unevenly:
    row m holds head m % G), ragged contexts incl. 0 and 1.  bf16 / f16 run the grid kernel
    without a workspace and stream-K with one; fp32 runs the generic kernel without a workspace
    and the fp32 stream-K tile (QK^T on fp32 MFMA) with one."""
    Hkv = 2
    inp = make_inputs(device, CTX_RAGGED, dt, H=Hkv * G, Hkv=Hkv, D=D, seed=10 * G + D)
    want = oracle_v1_plus(inp)
    for ws in (False, True):
        assert_close(gpu_v1(kernels, inp, ws), want, dt, f"ws={ws}")
    assert_close(gpu_v2(kernels, inp, 32), want, dt, "v2 P=32")


@pytest.mark.parametrize("D", [64, 128])
def test_stream_odd_blocks_full_row(device, kernels, D):
    """Stream-K units of several blocks (head_dim 64): sequences whose block count is no
    multiple of the unit fill the whole block-table row (19 blocks, max_blocks 19), so a
    segment's last unit is short and has no table entry after it; fused pool layout and 132
    sequences (the two-pass unit scan).  At head_dim 128 (one-block units) this makes more
    units than workers; at head_dim 64 (four-block units) fewer, which
    test_stream_head_dim64_many_units_per_worker covers."""
    ctx = [300, 289, 33, 300, 17, 300] * 22
    inp = make_inputs(device, ctx, "bf16", H=8, Hkv=2, D=D, seed=70 + D, fused=True, mb=19)
    assert inp["mb"] == 19 and max((c + 15) // 16 for c in ctx) == 19
    assert_close(gpu_v1(kernels, inp, True), oracle_v1_plus(inp), "bf16", "ws=True")


def _device_normal(shape, dt, seed, device):
    """N(0, 1) drawn on the device (pools of ~1 GB), and the same bits on the host."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(TORCH_DT[dt])
    return t, from_dev(t, dt)


def _stream_workers(device) -> int:
    """Workers of the stream-K decode: one wave per SIMD, four per CU."""
    return torch.cuda.get_device_properties(device).multi_processor_count * 4


def _stream_units(ctx, hkv: int, blocks_per_unit: int) -> int:
    blocks = (np.asarray(ctx, np.int64) + 15) // 16
    return int(((blocks + blocks_per_unit - 1) // blocks_per_unit).sum()) * hkv


def _big_decode_inputs(device, ctx, dt, H, Hkv, D, seed, mb, bs=16):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int32)
    need = int(((ctx.astype(np.int64) + bs - 1) // bs).sum())
    nb = need + 64
    bt = wl.assign_blocks(ctx, bs, nb, mb, rng)
    dkc, kc = _device_normal((nb, Hkv, bs, D), dt, seed + 1, device)
    dvc, vc = _device_normal((nb, Hkv, bs, D), dt, seed + 2, device)
    dq, q = _device_normal((len(ctx), H, D), dt, seed + 3, device)
    return dict(ctx=ctx, bt=bt, q=q, kc=kc, vc=vc, H=H, Hkv=Hkv, D=D, bs=bs, mb=mb, dt=dt, scale=1.0 / math.sqrt(D),
                dq=dq, dkc=dkc, dvc=dvc, dbt=i32(bt, device), dctx=i32(ctx, device))


def _threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.mark.parametrize("B", [60, 130])
def test_stream_cost_split_short_and_empty_sequences(device, kernels, B):
    """The stream-K split by cost (units plus a fixed cost per segment start) on short contexts
    U[1, 600] with a fifth of the sequences empty, 8 / 2 heads, D 128: batches of up to 64 (one
    pass over the context lengths) and above (chunked passes).  On a 256-CU device the shapes
    put 18 (B 60, where the cost caps the workers at 909) and 22 (B 130) workers' share
    boundaries past the last unit of a sequence, so that their ranges start at a later
    sequence, and send several workers across empty sequences.  Against the oracle."""
    rng = np.random.default_rng(B)
    ctx = rng.integers(1, 600, B, endpoint=True).astype(np.int32)
    ctx[rng.random(B) < 0.2] = 0
    inp = _big_decode_inputs(device, ctx, "bf16", 8, 2, 128, seed=B + 7, mb=64)
    assert _stream_units(ctx, 2, 1) > _stream_workers(device)
    want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], "bf16",
                                      nthreads=_threads())
    got = gpu_v1(kernels, inp, True)
    assert not np.isnan(got).any()
    assert_close(got, want, "bf16", f"B={B}")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_stream_head_dim64_many_units_per_worker(device, kernels, dt):
    """The attention of BASELINE config 5 (Llama-3.2-1B: 32 / 8 heads, head_dim 64, 128 sequences
    with its contexts U[64, 8192], block 16, 512-entry tables) through the stream-K decode,
    whose head_dim-64 units are four blocks: about 67.5 units per worker, so every worker runs
    whole rounds of its unit ring, crosses segments mid-range, and refills its 64-unit
    block-table window at least once (fp32: one-block units, about 270 per worker).  Against the
    oracle at 2e-2 / 1e-2 (bf16 / f16) and 1e-4 (fp32)."""
    w = wl.config5()
    ctx = w.context_lens
    inp = _big_decode_inputs(device, ctx, dt, 32, 8, 64, seed=500, mb=512)
    units, workers = _stream_units(ctx, 8, 1 if dt == "f32" else 4), _stream_workers(device)
    assert units > 64 * workers, (units, workers)
    want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], dt,
                                      nthreads=_threads())
    assert_close(gpu_v1(kernels, inp, True), want, dt, "stream-K v1")
    assert_close(gpu_v1(kernels, inp, True, "v1_plus"), want, dt, "stream-K v1_plus")


@pytest.mark.parametrize("G", [8, 16])
def test_stream_head_dim64_wide_groups(device, kernels, G):
    """head_dim 64 with 8 and 16 q-heads per kv-head (Llama-3-70B-like grouping): 128
    sequences with contexts U[64, 8192], several rounds of units per worker, bf16."""
    rng = np.random.default_rng(600 + G)
    ctx = rng.integers(64, 8192, 128, endpoint=True).astype(np.int32)
    Hkv = 2
    inp = _big_decode_inputs(device, ctx, "bf16", Hkv * G, Hkv, 64, seed=600 + G, mb=512)
    assert _stream_units(ctx, Hkv, 4) > 8 * _stream_workers(device)
    want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], "bf16",
                                      nthreads=_threads())
    assert_close(gpu_v1(kernels, inp, True), want, "bf16", f"G={G}")


def test_workspace_reused_across_calls(device, kernels):
    """One workspace serves calls of different shapes (GQA 4 and 8, head_dim 128 and 64, empty
    and long sequences) and a v2 call that falls back to partition + reduce on its front part:
    every call matches the oracle whatever the previous calls left in it."""
    shapes = [dict(ctx=CTX_RAGGED, G=4, D=128), dict(ctx=[2000, 37, 4096, 0, 900] * 6, G=4, D=128),
              dict(ctx=CTX_RAGGED[::-1], G=8, D=64)]
    inps = [make_inputs(device, sh["ctx"], "bf16", H=2 * sh["G"], Hkv=2, D=sh["D"], seed=40 + i)
            for i, sh in enumerate(shapes)]
    wants = [oracle_v1_plus(inp) for inp in inps]
    nbytes = max(kernels.v1_workspace_bytes(len(inp["ctx"]), inp["H"], inp["Hkv"], inp["D"], inp["bs"], inp["mb"])
                 for inp in inps)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    for i in (0, 1, 0, "v2", 2, 1, 2):
        if i == "v2":
            # v2 on the front of the same workspace, too small for the stream-K path: the
            # partition + reduce fallback
            inp, P = inps[0], 32
            np_ = math.ceil(int(inp["ctx"].max()) / P)
            need = kernels.v2_workspace_bytes(len(inp["ctx"]), inp["H"], np_, inp["D"])
            assert need < nbytes
            out = torch.full_like(inp["dq"], float("nan"))
            kernels.launch_v2(inp["dq"], inp["dkc"], inp["dvc"], inp["dbt"], inp["dctx"], out, inp["scale"],
                              inp["H"], inp["Hkv"], inp["D"], inp["bs"], inp["mb"], len(inp["ctx"]),
                              int(inp["ctx"].max()), P, ws[:need])
            torch.cuda.synchronize()
            assert_close(dev_f32(out), wants[0], "bf16", "v2 fallback")
            continue
        inp = inps[i]
        out = torch.full_like(inp["dq"], float("nan"))
        kernels.launch_v1(inp["dq"], inp["dkc"], inp["dvc"], inp["dbt"], inp["dctx"], out, inp["scale"], inp["H"],
                          inp["Hkv"], inp["D"], inp["bs"], inp["mb"], len(inp["ctx"]), workspace=ws)
        torch.cuda.synchronize()
        assert_close(dev_f32(out), wants[i], "bf16", f"shape {i}")


@pytest.mark.parametrize("dt,D,bs,G", [("f32", 128, 16, 4), ("bf16", 96, 16, 4), ("bf16", 256, 24, 2),
                                       ("f16", 32, 8, 3), ("bf16", 128, 24, 4), ("f32", 256, 8, 1),
                                       ("bf16", 128, 8, 4)])
def test_generic_path_shapes(device, kernels, dt, D, bs, G):
    """Shapes outside the MFMA kernels (fp32 without a workspace, head_dim 32/96/256, block 8 / 24,
    GQA 3)."""
    inp = make_inputs(device, [1, 7, 40, 129, 0], dt, H=2 * G, Hkv=2, D=D, bs=bs, seed=D + bs + G)
    want = oracle_v1_plus(inp)
    for ws in (False, True):
        assert_close(gpu_v1(kernels, inp, ws), want, dt, f"ws={ws}")
    assert_close(gpu_v2(kernels, inp, 2 * bs), want, dt, "v2")


@pytest.mark.parametrize("bs", [32, 64, 128, 256])
@pytest.mark.parametrize("dt,D,G", [("bf16", 128, 4), ("f16", 64, 8), ("f32", 128, 4), ("bf16", 64, 1)])
def test_mfma_path_block_sizes(device, kernels, dt, D, G, bs):
    """Block sizes 16 << j on the MFMA grid and stream-K kernels, which work in 16-token
    sub-blocks of each block (256 = 16 << 4, the largest shift they take): ragged contexts (0,
    1, sub-block and block boundaries), v1 without a workspace (grid kernel; generic for fp32),
    with one (stream-K), v2 with P = 2 bs, and the fused pool layout."""
    Hkv = 2
    for fused in (False, True):
        inp = make_inputs(device, CTX_RAGGED + [bs - 1, bs, bs + 1, 3 * bs + 16], dt, H=Hkv * G, Hkv=Hkv, D=D,
                          bs=bs, seed=bs + D + G, fused=fused)
        want = oracle_v1_plus(inp)
        for ws in (False, True):
            assert_close(gpu_v1(kernels, inp, ws), want, dt, f"fused={fused} ws={ws}")
        assert_close(gpu_v2(kernels, inp, 2 * bs), want, dt, f"fused={fused} v2")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("G", [1, 2, 4, 8, 16])
def test_mfma_head_dim256(device, kernels, dt, G):
    """head_dim 256 on the MFMA kernels (grid without a workspace, except G = 16, which the
    generic kernel serves; stream-K with one; v2) over ragged contexts, 16- and 32-token blocks.
    In fp32 (the reference's element type): the generic kernel without a workspace, the fp32
    stream-K tile with one."""
    Hkv = 2
    for bs in (16, 32):
        inp = make_inputs(device, CTX_RAGGED, dt, H=Hkv * G, Hkv=Hkv, D=256, bs=bs, seed=256 + G + bs)
        want = oracle_v1_plus(inp)
        for ws in (False, True):
            assert_close(gpu_v1(kernels, inp, ws), want, dt, f"bs={bs} ws={ws}")
        assert_close(gpu_v2(kernels, inp, 64), want, dt, f"bs={bs} v2")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("H,Hkv", [(24, 8), (28, 4), (40, 8), (48, 8)])
def test_stream_gqa_model_shapes(device, kernels, H, Hkv, dt):
    """Stream-K decode at the head counts of models whose GQA ratio is no power of two, head_dim
    128: Llama-3.2-3B (24 / 8, G 3), Qwen2-7B (28 / 4, G 7), Qwen2.5-14B (40 / 8, G 5), and
    48 / 8 (G 6); 64 sequences with contexts U[512, 4096] (config 2's load: many units per
    worker, segments crossed mid range, window refills), against the oracle."""
    rng = np.random.default_rng(H * 10 + Hkv)
    ctx = rng.integers(512, 4096, 64, endpoint=True).astype(np.int32)
    inp = _big_decode_inputs(device, ctx, dt, H, Hkv, 128, seed=H + Hkv, mb=256)
    assert _stream_units(ctx, Hkv, 1) > 16 * _stream_workers(device)
    want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], dt,
                                      nthreads=_threads())
    assert_close(gpu_v1(kernels, inp, True), want, dt, f"{H}/{Hkv} stream-K")
    if dt == "bf16":
        assert_close(gpu_v1(kernels, inp, False), want, dt, f"{H}/{Hkv} grid kernel")
        assert_close(gpu_v2(kernels, inp, 512), want, dt, f"{H}/{Hkv} v2")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_stream_head_dim256_many_units(device, kernels, dt):
    """head_dim 256, 16 / 4 heads (Gemma-like grouping), 96 sequences with contexts U[64, 4096],
    bf16 and fp32: tens of one-block units per worker, window refills, segments crossed mid
    range."""
    rng = np.random.default_rng(901)
    ctx = rng.integers(64, 4096, 96, endpoint=True).astype(np.int32)
    inp = _big_decode_inputs(device, ctx, dt, 16, 4, 256, seed=901, mb=256)
    assert _stream_units(ctx, 4, 1) > 16 * _stream_workers(device)
    want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], dt,
                                      nthreads=_threads())
    assert_close(gpu_v1(kernels, inp, True), want, dt, "D=256")


@pytest.mark.parametrize("bs", [32, 64, 256])
def test_stream_block_sizes_many_units(device, kernels, bs):
    """Stream-K with 32-, 64- and 256-token blocks at a config-5-like load (128 sequences,
    contexts U[64, 8192], 32 / 8 heads, head_dim 64, bf16): many units per worker, segments
    crossed mid range, block-table window refills, each window entry a (block, sub-block) pair
    (at 256, sixteen sub-blocks per block: the largest shift of the packing)."""
    rng = np.random.default_rng(700 + bs)
    ctx = rng.integers(64, 8192, 128, endpoint=True).astype(np.int32)
    inp = _big_decode_inputs(device, ctx, "bf16", 32, 8, 64, seed=700 + bs, mb=8192 // bs, bs=bs)
    assert _stream_units(ctx, 8, 4) > 48 * _stream_workers(device)
    want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], "bf16",
                                      nthreads=_threads())
    assert_close(gpu_v1(kernels, inp, True), want, "bf16", f"bs={bs}")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_fused_pool_layout(device, kernels, dt):
    """Railgun's fused [NB, 2, H_kv, bs, D] pool via kv_block_stride (block.rs:70,89-95)."""
    inp = make_inputs(device, [5, 70, 333], dt, seed=7, fused=True)
    want = oracle_v1_plus(inp)
    assert inp["dkc"].stride(0) == 2 * 8 * 16 * 128
    assert_close(gpu_v1(kernels, inp, True), want, dt)
    assert_close(gpu_v2(kernels, inp, 64), want, dt)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_tail_rows_never_leak(device, kernels, dt):
    """NaN in the unused rows of each sequence's last block must not reach the output."""
    inp = make_inputs(device, [3, 17, 250], dt, seed=11)
    clean = gpu_v1(kernels, inp, True)
    nan_bits = {"f32": np.float32(np.nan), "bf16": np.uint16(0x7FC0)}[dt]
    for s, c in enumerate(inp["ctx"]):
        c = int(c)
        if c % inp["bs"]:
            blk = int(inp["bt"][s, c // inp["bs"]])
            inp["kc"][blk, :, c % inp["bs"]:] = nan_bits
            inp["vc"][blk, :, c % inp["bs"]:] = nan_bits
    inp["dkc"], inp["dvc"] = to_dev(inp["kc"], dt, device), to_dev(inp["vc"], dt, device)
    for ws in (False, True):
        got = gpu_v1(kernels, inp, ws)
        assert np.isfinite(got).all()
        np.testing.assert_array_equal(got, clean) if ws else assert_close(got, clean, dt)
    assert np.isfinite(gpu_v2(kernels, inp, 32)).all()


@pytest.mark.parametrize("dt,bs", [("f32", 16), ("bf16", 32)])
def test_v2_partition_contract(device, kernels, dt, bs):
    """tmp_out / exp_sums / max_logits of v2_partition (P=256) against the oracle's: fp32 (the
    generic kernel) and bf16 with 32-token blocks (the MFMA grid kernel in partial mode)."""
    inp = make_inputs(device, [100, 256, 257, 700, 0], dt, H=8, Hkv=2, D=64, bs=bs, seed=5)
    P, NP = 256, 3
    B = len(inp["ctx"])
    tmp, es, ml = orc.paged_attention_v2_partition(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"],
                                                   inp["scale"], dt, NP, P)
    d_tmp = torch.zeros((B, 8, NP, 64), dtype=torch.float32, device=device)
    d_es = torch.zeros((B, 8, NP), dtype=torch.float32, device=device)
    d_ml = torch.zeros((B, 8, NP), dtype=torch.float32, device=device)
    kernels.launch_v2_partition(inp["dq"], inp["dkc"], inp["dvc"], inp["dbt"], inp["dctx"], d_tmp, d_es, d_ml,
                                None, inp["scale"], 8, 2, 64, bs, inp["mb"], NP, B, P)
    torch.cuda.synchronize()
    tol = 1e-4 if dt == "f32" else 2e-2
    np.testing.assert_allclose(dev_f32(d_ml), ml, atol=tol / 10, rtol=tol / 10)
    np.testing.assert_allclose(dev_f32(d_es), es, atol=tol, rtol=tol)
    np.testing.assert_allclose(dev_f32(d_tmp), tmp, atol=tol, rtol=tol)
    out = torch.zeros((B, 8, 64), dtype=TORCH_DT[dt], device=device)
    kernels.launch_v2_reduce(out, d_es, d_ml, d_tmp, inp["dctx"], None, 8, 64, NP, B, P)
    torch.cuda.synchronize()
    assert_close(dev_f32(out), oracle_v1_plus(inp), dt)


def _config_pool(w, device, seed_offset=0):
    rng = np.random.default_rng(w.seed + seed_offset)
    shape = (w.num_blocks, w.num_kv_heads, w.block_size, w.head_dim)
    kc, vc = normal(rng, shape, w.dtype), normal(rng, shape, w.dtype)
    q = normal(rng, (w.batch, w.num_heads, w.head_dim), w.dtype)
    return q, kc, vc


def test_config2_full_decode(device, kernels):
    """Config 2 at full size (B=64, ctx U[512,4096], bf16, D=128, 32/8): v1 vs oracle."""
    w = wl.config2()
    q, kc, vc = _config_pool(w, device)
    inp = dict(ctx=w.context_lens, bt=w.block_table, q=q, kc=kc, vc=vc, H=w.num_heads, Hkv=w.num_kv_heads,
               D=w.head_dim, bs=w.block_size, mb=w.max_blocks, dt=w.dtype, scale=w.scale,
               dq=to_dev(q, w.dtype, device), dkc=to_dev(kc, w.dtype, device), dvc=to_dev(vc, w.dtype, device),
               dbt=i32(w.block_table, device), dctx=i32(w.context_lens, device))
    want = orc.cpu_attention_gathered(q, kc, vc, w.block_table, w.context_lens, w.scale, w.dtype, nthreads=8)
    assert_close(gpu_v1(kernels, inp, True), want, "bf16", "v1 split")
    assert_close(gpu_v1(kernels, inp, False), want, "bf16", "v1 single")
    assert_close(gpu_v2(kernels, inp, 512), want, "bf16", "v2 P=512")


def test_config2_step_chain(device, kernels):
    """The bench's timed config-2 step end to end at full size (64 sequences, contexts U[512,
    4096], bf16, 32/8, D 128, block 16): rg_rope_reshape_and_cache of the 64 new tokens (RoPE
    theta 5e5 at position ctx - 1, the decode convention of scheduler.rs:258-263, written at
    their slots), then rg_paged_attention_v1 with its workspace over the updated pool.  The
    oracle runs the same chain: its rope_reshape_and_cache, then the reference CPU path over
    the gathered blocks.  Rotated q and both whole caches bit-exact; attention within the bf16
    tolerance (each sequence's last key is the token just written)."""
    from railgun_amd.ops import rope_cos_sin_table

    w = wl.config2()
    B, H, hkv, D, bs = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    rng = np.random.default_rng(w.seed + 7)
    shape = (w.num_blocks, hkv, bs, D)
    kc, vc = normal(rng, shape, "bf16"), normal(rng, shape, "bf16")
    q, k, v = normal(rng, (B, H, D), "bf16"), normal(rng, (B, hkv, D), "bf16"), normal(rng, (B, hkv, D), "bf16")
    pos, slots = w.positions, w.slot_mapping
    assert np.array_equal(pos, w.context_lens - 1)
    table = rope_cos_sin_table(int(w.context_lens.max()), D, w.rope_theta)
    dq, dkc, dvc = to_dev(q, "bf16", device), to_dev(kc, "bf16", device), to_dev(vc, "bf16", device)
    kernels.launch_rope_reshape_and_cache(dq, to_dev(k, "bf16", device), to_dev(v, "bf16", device), dkc, dvc,
                                          table.to(device), i32(pos, device), i32(slots, device), H, hkv, D, bs, B)
    out = torch.full_like(dq, float("nan"))
    ws = torch.empty(max(kernels.v1_workspace_bytes(B, H, hkv, D, bs, w.max_blocks), 1), dtype=torch.uint8,
                     device=device)
    kernels.launch_v1(dq, dkc, dvc, i32(w.block_table, device), i32(w.context_lens, device), out, w.scale, H, hkv,
                      D, bs, w.max_blocks, B, workspace=ws)
    torch.cuda.synchronize()
    orc.rope_reshape_and_cache(q, k, v, kc, vc, table.numpy(), pos, slots, "bf16", bs)
    np.testing.assert_array_equal(from_dev(dq, "bf16"), q, err_msg="rotated q")
    np.testing.assert_array_equal(from_dev(dkc, "bf16"), kc, err_msg="key cache after the step's write")
    np.testing.assert_array_equal(from_dev(dvc, "bf16"), vc, err_msg="value cache after the step's write")
    want = orc.cpu_attention_gathered(q, kc, vc, w.block_table, w.context_lens, w.scale, "bf16", nthreads=_threads())
    assert_close(dev_f32(out), want, "bf16", "config-2 step: RoPE + cache write, then v1")


def test_config3_v2_matches_v1(device, kernels):
    """Config 3 (B=8 x 32768, P=512) through the combined entries: rg_paged_attention_v2 with
    its full scratch takes the stream-K form (balanced split-K over all waves), as does v1 with
    a workspace, so the two agree by construction; the check that counts is against the oracle.
    The reference's own partition + reduce pair at P=512 is test_config3_v2_reference_contract."""
    w = wl.config3()
    q, kc, vc = _config_pool(w, device)
    inp = dict(ctx=w.context_lens, bt=w.block_table, q=q, kc=kc, vc=vc, H=w.num_heads, Hkv=w.num_kv_heads,
               D=w.head_dim, bs=w.block_size, mb=w.max_blocks, dt=w.dtype, scale=w.scale,
               dq=to_dev(q, w.dtype, device), dkc=to_dev(kc, w.dtype, device), dvc=to_dev(vc, w.dtype, device),
               dbt=i32(w.block_table, device), dctx=i32(w.context_lens, device))
    v2 = gpu_v2(kernels, inp, w.partition_size)
    v1 = gpu_v1(kernels, inp, True)
    assert_close(v2, v1, "bf16", "v2 vs v1")
    want = orc.cpu_attention_gathered(q, kc, vc, w.block_table, w.context_lens, w.scale, w.dtype, nthreads=8)
    assert_close(v2, want, "bf16", "v2 vs oracle")


def _golden(name):
    import os
    import sys

    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    if here not in sys.path:
        sys.path.insert(0, here)
    import make_fixtures  # noqa: E402

    return make_fixtures, np.load(os.path.join(here, name))


def test_config1_against_golden_fixture(device, kernels):
    """BASELINE configs[0] on the GPU against the committed float64 fixture: every decode entry
    at 1e-4, and reshape_and_cache of the 4 new tokens (with and without a slot of -1) bit-exact
    by the SHA-256 of the whole resulting caches."""
    import hashlib

    mf, f = _golden("config1_fp32.npz")
    w, q, kc, vc, k_new, v_new = mf.config1_inputs()
    assert mf.sha(q, kc, vc, w.block_table, w.context_lens, k_new, v_new) == str(f["input_sha256"])
    inp = dict(ctx=w.context_lens, bt=w.block_table, q=q, kc=kc, vc=vc, H=32, Hkv=8, D=64, bs=16, mb=w.max_blocks,
               dt="f32", scale=w.scale, dq=to_dev(q, "f32", device), dkc=to_dev(kc, "f32", device),
               dvc=to_dev(vc, "f32", device), dbt=i32(w.block_table, device), dctx=i32(w.context_lens, device))
    want = f["expected_out_f64"]
    for ws in (False, True):
        for entry in ("v1", "v1_plus"):
            assert_close(gpu_v1(kernels, inp, ws, entry), want, "f32", f"{entry} ws={ws}")
    assert_close(gpu_v2(kernels, inp, 64), want, "f32", "v2")
    for slots, key in ((f["slot_mapping"], "cache_after_sha256"), (f["slot_mapping_skip"], "cache_after_skip_sha256")):
        dkc, dvc = to_dev(kc, "f32", device), to_dev(vc, "f32", device)
        kernels.launch_reshape_and_cache(to_dev(k_new, "f32", device), to_dev(v_new, "f32", device), dkc, dvc,
                                         i32(slots, device), 8, 64, 16, 4)
        torch.cuda.synchronize()
        h = hashlib.sha256()
        h.update(np.ascontiguousarray(dkc.cpu().numpy()).tobytes())
        h.update(np.ascontiguousarray(dvc.cpu().numpy()).tobytes())
        assert h.hexdigest() == str(f[key])


def test_bf16_decode_against_golden_fixture(device, kernels):
    mf, f = _golden("decode_bf16_small.npz")
    ctx, bt, q, kc, vc = mf.small_bf16_inputs()
    assert mf.sha(q, kc, vc, bt, ctx) == str(f["input_sha256"])
    inp = dict(ctx=ctx, bt=bt, q=q, kc=kc, vc=vc, H=32, Hkv=8, D=128, bs=16, mb=bt.shape[1], dt="bf16",
               scale=1 / math.sqrt(128), dq=to_dev(q, "bf16", device), dkc=to_dev(kc, "bf16", device),
               dvc=to_dev(vc, "bf16", device), dbt=i32(bt, device), dctx=i32(ctx, device))
    for ws in (False, True):
        assert_close(gpu_v1(kernels, inp, ws), f["expected_out_f64"], "bf16", f"ws={ws}")
    assert_close(gpu_v2(kernels, inp, 32), f["expected_out_f64"], "bf16", "v2")


def test_config3_v2_reference_contract(device, kernels):
    """Config 3 through the reference's v2 launcher pair (paged_attn_op.rs:108-158):
    rg_paged_attention_v2_partition at P = 512 with NP = 64 partitions, then
    rg_paged_attention_v2_reduce.  The partials (tmp_out unnormalised, exp_sums, max_logits in
    natural-log units, paged_attention_v2_partition.cu:95-106) match the oracle's partition
    maths; the reduced output matches the oracle and the stream-K v1 output."""
    w = wl.config3()
    q, kc, vc = _config_pool(w, device)
    B, H, Hkv, D, P = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.partition_size
    NP = math.ceil(int(w.context_lens.max()) / P)
    assert (P, NP) == (512, 64)
    inp = dict(ctx=w.context_lens, bt=w.block_table, q=q, kc=kc, vc=vc, H=H, Hkv=Hkv, D=D, bs=w.block_size,
               mb=w.max_blocks, dt=w.dtype, scale=w.scale, dq=to_dev(q, w.dtype, device),
               dkc=to_dev(kc, w.dtype, device), dvc=to_dev(vc, w.dtype, device), dbt=i32(w.block_table, device),
               dctx=i32(w.context_lens, device))
    d_tmp = torch.full((B, H, NP, D), float("nan"), dtype=torch.float32, device=device)
    d_es = torch.full((B, H, NP), float("nan"), dtype=torch.float32, device=device)
    d_ml = torch.full((B, H, NP), float("nan"), dtype=torch.float32, device=device)
    kernels.launch_v2_partition(inp["dq"], inp["dkc"], inp["dvc"], inp["dbt"], inp["dctx"], d_tmp, d_es, d_ml, None,
                                w.scale, H, Hkv, D, w.block_size, w.max_blocks, NP, B, P)
    out = torch.full_like(inp["dq"], float("nan"))
    kernels.launch_v2_reduce(out, d_es, d_ml, d_tmp, inp["dctx"], None, H, D, NP, B, P)
    torch.cuda.synchronize()
    tmp, es, ml = orc.paged_attention_v2_partition(q, kc, vc, w.block_table, w.context_lens, w.scale, w.dtype, NP, P)
    # fp32 arithmetic on the same bf16 inputs on both sides: only summation order and the
    # exponential's rounding differ
    np.testing.assert_allclose(dev_f32(d_ml), ml, atol=1e-4, rtol=1e-5, err_msg="max_logits")
    np.testing.assert_allclose(dev_f32(d_es), es, atol=1e-3, rtol=1e-4, err_msg="exp_sums")
    np.testing.assert_allclose(dev_f32(d_tmp), tmp, atol=1e-3, rtol=1e-3, err_msg="tmp_out")
    got = dev_f32(out)
    want = orc.paged_attention_v2_reduce(tmp, es, ml, w.context_lens, P)
    assert_close(got, want, "bf16", "v2 partition + reduce vs oracle")
    assert_close(got, gpu_v1(kernels, inp, True), "bf16", "v2 partition + reduce vs stream-K v1")


def test_stream_fp32_config2_shape(device, kernels):
    """The reference's element type at config 2's shape (64 sequences, contexts U[512, 4096], 32 / 8
    heads, head_dim 128, block 16): the fp32 stream-K tile against the oracle at 1e-4, through v1,
    v1_plus and the combined v2."""
    w = wl.config2()
    inp = _big_decode_inputs(device, w.context_lens, "f32", 32, 8, 128, seed=800, mb=w.max_blocks)
    want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], "f32",
                                      nthreads=_threads())
    assert_close(gpu_v1(kernels, inp, True), want, "f32", "v1 stream-K")
    assert_close(gpu_v1(kernels, inp, True, "v1_plus"), want, "f32", "v1_plus stream-K")
    assert_close(gpu_v2(kernels, inp, 512), want, "f32", "v2")


def test_stream_random_shapes(device, kernels):
    """Twenty seeded random decode batches through the stream-K entry with a workspace, against
    the oracle: batch 1-150 (one pass over the context lengths and the chunked passes), a quarter
    of them with empty sequences, contexts up to 3,000 tokens, GQA 1 / 2 / 3 / 4 / 8, head_dim 64
    / 128, block sizes 16 / 32, bf16 and fp32 — loads from a few units per worker to tens, so the
    split by cost meets short segments, empty sequences and share boundaries at sequence ends."""
    rng = np.random.default_rng(2024)
    for case in range(20):
        B = int(rng.integers(1, 151))
        G = int(rng.choice([1, 2, 3, 4, 8]))
        Hkv = int(rng.choice([1, 2, 4]))
        D = int(rng.choice([64, 128]))
        bs = int(rng.choice([16, 32]))
        dt = "f32" if case % 4 == 3 else "bf16"
        ctx = rng.integers(1, int(rng.choice([40, 600, 3000])), B, endpoint=True).astype(np.int32)
        if case % 4 == 1:
            ctx[rng.random(B) < 0.3] = 0
        mb = int(max(1, (ctx.max() + bs - 1) // bs))
        inp = _big_decode_inputs(device, ctx, dt, G * Hkv, Hkv, D, seed=3000 + case, mb=mb, bs=bs)
        want = orc.cpu_attention_gathered(inp["q"], inp["kc"], inp["vc"], inp["bt"], inp["ctx"], inp["scale"], dt,
                                          nthreads=_threads())
        got = gpu_v1(kernels, inp, True)
        assert not np.isnan(got).any(), f"case {case}"
        assert_close(got, want, dt, f"case {case}: B={B} G={G} Hkv={Hkv} D={D} bs={bs} {dt}")
