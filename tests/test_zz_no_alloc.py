"""rg_paged_attention_v1_no_alloc, the decode entry that allocates nothing, on the GPU.

It runs the same stream-K kernels as rg_paged_attention_v1 with a workspace, on the
library's static per-device scratch.  Called through the C ABI (ctypes, no Python mirror in
between), two calls in a row — a config-2-sized batch, then a smaller one that leaves most of
the first call's partials in the scratch — must give exactly the output of
rg_paged_attention_v1 with a caller's workspace, which matches the oracle.  A shape whose
partials exceed the static scratch is refused before any launch.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, dev_f32, from_dev, i32
from oracle import oracle as orc
from railgun_amd import _lib
from railgun_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _inputs(device, ctx, H, Hkv, D, seed):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int32)
    mb = max(1, int(((ctx.max() + 15) // 16)))
    nb = int(((ctx.astype(np.int64) + 15) // 16).sum()) + 8
    bt = wl.assign_blocks(ctx, 16, nb, mb, rng)
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def normal(shape):
        return torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)

    return dict(q=normal((len(ctx), H, D)), kc=normal((nb, Hkv, 16, D)), vc=normal((nb, Hkv, 16, D)),
                bt=i32(bt, device), ctx=i32(ctx, device), hbt=bt, hctx=ctx, H=H, Hkv=Hkv, D=D, mb=mb,
                scale=1.0 / math.sqrt(D))


def _args(inp, out):
    return (inp["q"].data_ptr(), inp["kc"].data_ptr(), inp["vc"].data_ptr(), inp["bt"].data_ptr(),
            inp["ctx"].data_ptr(), out.data_ptr(), inp["scale"], inp["H"], inp["Hkv"], inp["D"], 16, inp["mb"],
            len(inp["hctx"]), _lib.RG_DTYPE_BF16, 0)


def _with_workspace(lib, inp):
    B = len(inp["hctx"])
    nbytes = lib.rg_paged_attention_v1_workspace_bytes(B, inp["H"], inp["Hkv"], inp["D"], 16, inp["mb"])
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=inp["q"].device)
    out = torch.full_like(inp["q"], float("nan"))
    st = lib.rg_paged_attention_v1(*_args(inp, out), ws.data_ptr(), ws.numel(), None)
    assert st == _lib.RG_OK, lib.rg_last_error()
    return out


def _no_alloc(lib, inp):
    out = torch.full_like(inp["q"], float("nan"))
    st = lib.rg_paged_attention_v1_no_alloc(*_args(inp, out), None)
    assert st == _lib.RG_OK, lib.rg_last_error()
    return out


def test_no_alloc_matches_workspace_entry(device, kernels):
    lib = kernels.lib
    big = _inputs(device, wl.config2().context_lens, 32, 8, 128, seed=71)               # 64 seqs, U[512, 4096]
    small = _inputs(device, [1, 17, 300, 0, 1000, 64], 32, 8, 64, seed=72)              # 6 seqs, head_dim 64
    first = _no_alloc(lib, big)
    second = _no_alloc(lib, small)
    torch.cuda.synchronize()
    for inp, got in ((big, first), (small, second)):
        want = _with_workspace(lib, inp)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), "differs from rg_paged_attention_v1"
    # the small call against the oracle as well (the big one is config 2, covered elsewhere)
    q, kc, vc = (from_dev(small[k], "bf16") for k in ("q", "kc", "vc"))
    oracle = orc.paged_attention_v1_plus(q, kc, vc, small["hbt"], small["hctx"], small["scale"], "bf16")
    assert_close(dev_f32(second), oracle, "bf16", "no_alloc vs oracle")


def test_no_alloc_refuses_shapes_beyond_the_scratch(device, kernels):
    """5000 sequences x 8 kv-heads need ~84 MB of partials: refused with RG_ERR_WORKSPACE and a
    message, nothing launched (the output keeps its contents)."""
    lib = kernels.lib
    B, H, Hkv, D = 5000, 32, 8, 128
    q = torch.zeros((B, H, D), dtype=torch.bfloat16, device=device)
    cache = torch.zeros((4, Hkv, 16, D), dtype=torch.bfloat16, device=device)
    bt = torch.zeros((B, 1), dtype=torch.int32, device=device)
    ctx = torch.ones(B, dtype=torch.int32, device=device)
    out = torch.full_like(q, 7.0)
    st = lib.rg_paged_attention_v1_no_alloc(q.data_ptr(), cache.data_ptr(), cache.data_ptr(), bt.data_ptr(),
                                            ctx.data_ptr(), out.data_ptr(), 0.1, H, Hkv, D, 16, 1, B,
                                            _lib.RG_DTYPE_BF16, 0, None)
    torch.cuda.synchronize()
    assert st == _lib.RG_ERR_WORKSPACE
    assert b"static scratch" in lib.rg_last_error()
    assert bool((out == 7.0).all())


def test_no_alloc_under_graph_capture(device, kernels):
    """The entry under HIP graph capture, as its header allows: captured once (torch's capture
    stream) and replayed four times, with eager work between the replays — a call of the same
    entry on other inputs, which rewrites the shared static scratch, and, before the third
    replay, a new q written into the captured input buffer.  Every replay is bit-equal to the
    eager call on the inputs the buffers then hold (the graph records only the two kernel
    launches: no allocation, no memset)."""
    lib = kernels.lib
    inp = _inputs(device, wl.config2().context_lens[:32], 32, 8, 128, seed=73)
    other = _inputs(device, [5, 900, 3000], 32, 8, 64, seed=74)
    want = _no_alloc(lib, inp)
    torch.cuda.synchronize()
    out = torch.full_like(inp["q"], float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = lib.rg_paged_attention_v1_no_alloc(*_args(inp, out), torch.cuda.current_stream().cuda_stream)
    assert st == _lib.RG_OK, lib.rg_last_error()
    torch.cuda.synchronize()
    g = torch.Generator(device=device)
    g.manual_seed(75)
    for i in range(4):
        _no_alloc(lib, other)
        if i == 2:
            inp["q"].copy_(torch.randn(inp["q"].shape, generator=g, device=device).to(torch.bfloat16))
            want = _no_alloc(lib, inp)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {i}"
