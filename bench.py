"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline workload: one Llama-3-8B-shaped bf16 decode step per
layer — batch 64, contexts U[512, 4096], 32 q / 8 kv heads, head_dim 128, block 16, shuffled
block tables — made of the fused RoPE + cache write of the 64 new tokens followed by paged
attention v1.  ``value`` is the step's algorithmic HBM bytes / step time (inputs resident in
HBM).  ``roofline`` is for the dominant call, paged attention v1 (partition + merge
kernels), timed with HIP events on the stream it is launched on.  Side figures: config 3
(v2 split-K, 8 x 32k) and config 4 (packed causal prefill, bf16 MFMA roofline).

Every timed region is preceded by ``SETTLE_MS`` of the same calls back to back (untimed, on
top of the warmup calls): the GPU's clocks ramp over the first ~10-20 ms of load (measured:
config 2's v1 call 114-115 us in its first 10 ms, 111-112 us after; config 4's prefill
158-187 us in its first rounds, 144 us after), and a figure timed inside that ramp is not the
steady state.

``cpu_baseline`` times the restated reference CPU path (gather -> q.K^T*scale -> softmax -> .V,
oracle/oracle.c) on every host core this process may use, over the whole config-2 batch.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "paged decode achieved HBM GB/s (% of peak) + prefill MFMA util, 1 GPU"
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2516.6
FP32_MFMA_PEAK_TFLOPS = 157.3
SETTLE_MS = 100.0  # back-to-back calls before each timed region (clock ramp, see above)


def measured_traffic(key: str):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (copy-calibrated) for
    this workload, as committed in profiles/traffic.json (key "commit": the commit they were
    measured at); None if absent."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-side", action="store_true", help="skip the config 3 / config 4 side figures")
    ap.add_argument("--only", choices=["decode", "v2", "fp32", "prefill", "model", "gemm", "copy"], default=None,
                    help="run one workload only and print its figures (for profiling); 'copy' is the plain "
                         "1 GiB device copy that calibrates the FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


def bf16_normal(shape, gen, device):
    import torch

    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)


def settle(fn, ms: float = SETTLE_MS) -> None:
    """Runs fn() back to back (synchronising after each batch of calls) until `ms` of wall time
    have passed, so that the GPU clocks have left their ramp before a timed region."""
    import torch

    t0 = time.perf_counter()
    n = 1
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        n = min(2 * n, 64)


def time_events(fn, steps: int, warmup: int):
    """Average ms per call of fn() over `steps` back-to-back calls, after `warmup` calls and the
    settle phase: one HIP event pair on the current stream (the stream every launch goes to)
    brackets them all, so no event record sits between two calls (a record between calls adds
    its own gap to the GPU timeline)."""
    import torch

    for _ in range(warmup):
        fn()
    settle(fn)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def decode_setup(w, device, gen):
    import torch

    from railgun_amd.ops import PagedAttentionKernels, PagedAttentionOp, rope_cos_sin_table

    kernels = PagedAttentionKernels(0)
    shape = (w.num_blocks, w.num_kv_heads, w.block_size, w.head_dim)
    st = dict(
        kernels=kernels,
        op=PagedAttentionOp(w.scale, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, kernels),
        kc=bf16_normal(shape, gen, device), vc=bf16_normal(shape, gen, device),
        q=bf16_normal((w.batch, w.num_heads, w.head_dim), gen, device),
        k=bf16_normal((w.batch, w.num_kv_heads, w.head_dim), gen, device),
        v=bf16_normal((w.batch, w.num_kv_heads, w.head_dim), gen, device),
        bt=torch.from_numpy(w.block_table).to(device), ctx=torch.from_numpy(w.context_lens).to(device),
        pos=torch.from_numpy(w.positions).to(device), slots=torch.from_numpy(w.slot_mapping).to(device),
    )
    st["out"] = torch.empty_like(st["q"])
    if w.rope_theta:
        st["cos_sin"] = rope_cos_sin_table(int(w.context_lens.max()), w.head_dim, w.rope_theta, device)
    nbytes = kernels.v1_workspace_bytes(w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, w.max_blocks)
    st["ws"] = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    return st


def v1_call(w, st):
    st["kernels"].launch_v1(st["q"], st["kc"], st["vc"], st["bt"], st["ctx"], st["out"], w.scale, w.num_heads,
                            w.num_kv_heads, w.head_dim, w.block_size, w.max_blocks, w.batch, workspace=st["ws"])


def fused_step_call(w, st):
    """The decode step through one entry: RoPE + cache write of the new tokens fused into the
    stream-K decode (q read unrotated)."""
    st["kernels"].launch_rope_reshape_and_cache_v1(
        st["q"], st["k"], st["v"], st["kc"], st["vc"], st["cos_sin"], st["pos"], st["slots"], st["bt"], st["ctx"],
        st["out"], w.scale, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, w.max_blocks, w.batch, st["ws"])


def rope_cache_call(w, st):
    st["op"].rope_reshape_and_cache(st["q"], st["k"], st["v"], st["kc"], st["vc"], st["cos_sin"], st["pos"],
                                    st["slots"])


def host_cores() -> tuple[int, str]:
    """Cores this process may run on: its CPU affinity, bounded by a cgroup CPU quota when one
    is set (cpu.max); and a description of both."""
    n = len(os.sched_getaffinity(0))
    note = f"{n} in the CPU affinity"
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            q = max(1, math.ceil(int(quota) / int(period)))
            note += f", cgroup quota {q}"
            n = min(n, q)
    except (OSError, ValueError):
        pass
    return n, note


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, seconds_target: float = 10.0) -> dict:
    """The restated reference CPU path (gather -> q.K^T*scale -> softmax -> .V, fp32, threaded
    over (sequence, kv-head)) on the whole config-2 batch: its 64 sequences, context lengths and
    block tables, over a pool of the same size (N(0, 1), bf16)."""
    import numpy as np

    from oracle import oracle as orc

    cores, core_note = host_cores()
    rng = np.random.default_rng(7)
    shape = (w.num_blocks, w.num_kv_heads, w.block_size, w.head_dim)
    kc = orc.bf16_round(rng.standard_normal(size=shape, dtype=np.float32))
    vc = orc.bf16_round(rng.standard_normal(size=shape, dtype=np.float32))
    q = orc.bf16_round(rng.standard_normal(size=(w.batch, w.num_heads, w.head_dim), dtype=np.float32))

    def run() -> float:
        t0 = time.perf_counter()
        orc.cpu_attention_gathered(q, kc, vc, w.block_table, w.context_lens, w.scale, "bf16", nthreads=cores)
        return time.perf_counter() - t0

    one = run()  # warm-up
    reps = max(10, min(100, int(seconds_target / max(one, 1e-3))))
    times = sorted(run() for _ in range(reps))
    med = times[len(times) // 2]
    return {"value": round(w.decode_bytes() / med / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"the whole config-2 batch ({w.batch} sequences, {int(w.context_lens.sum())} context tokens, "
                      f"32/8 heads, D 128, bf16 upcast to fp32), {w.decode_bytes() / 1e6:.1f} MB algorithmic bytes "
                      f"per run, median of {reps} runs after a warm-up, {cores} threads ({core_note})",
            "ms_per_run": round(med * 1e3, 2)}


def side_v2(device, gen, steps: int) -> dict:
    """Config 3 (8 x 32768, P = 512): the combined v2 entry with its full scratch, which runs the
    stream-K form (balanced split-K over all waves), and the reference's own launcher pair,
    rg_paged_attention_v2_partition over NP = 64 partitions + rg_paged_attention_v2_reduce
    (paged_attn_op.rs:108-158), timed on the same inputs."""
    import torch

    from railgun_amd import workloads as wl

    w = wl.config3()
    st = decode_setup(w, device, gen)
    P = w.partition_size
    np_ = math.ceil(int(w.context_lens.max()) / P)
    ws = torch.empty(st["kernels"].v2_workspace_bytes(w.batch, w.num_heads, np_, w.head_dim), dtype=torch.uint8,
                     device=device)

    def call():
        st["kernels"].launch_v2(st["q"], st["kc"], st["vc"], st["bt"], st["ctx"], st["out"], w.scale, w.num_heads,
                                w.num_kv_heads, w.head_dim, w.block_size, w.max_blocks, w.batch,
                                int(w.context_lens.max()), P, ws)

    tmp = torch.empty((w.batch, w.num_heads, np_, w.head_dim), dtype=torch.float32, device=device)
    es = torch.empty((w.batch, w.num_heads, np_), dtype=torch.float32, device=device)
    ml = torch.empty_like(es)

    def pair():
        k = st["kernels"]
        k.launch_v2_partition(st["q"], st["kc"], st["vc"], st["bt"], st["ctx"], tmp, es, ml, None, w.scale,
                              w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, w.max_blocks, np_, w.batch, P)
        k.launch_v2_reduce(st["out"], es, ml, tmp, st["ctx"], None, w.num_heads, w.head_dim, np_, w.batch, P)

    ms = time_events(call, steps, 3)
    ms_pair = time_events(pair, steps, 3)
    gbs = w.decode_bytes() / (ms * 1e-3) / 1e9
    gbs_pair = w.decode_bytes() / (ms_pair * 1e-3) / 1e9
    del st, ws, tmp, es, ml
    torch.cuda.empty_cache()
    return {"workload": w.name, "kernel": "rg_paged_attention_v2 (stream-K split over all waves + merge)",
            "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": w.decode_bytes(), "traffic": measured_traffic("paged_attention_v2_config3"),
            "reference_pair": {"kernel": f"rg_paged_attention_v2_partition (P {P}, NP {np_}) + "
                                         "rg_paged_attention_v2_reduce",
                               "us": round(ms_pair * 1e3, 2), "GB/s": round(gbs_pair, 1),
                               "frac_hbm_peak": round(gbs_pair / HBM_PEAK_GBS, 4)}}


def side_fp32(device, gen, steps: int, num_heads: int = 32) -> dict:
    """Config 2's decode (64 sequences, contexts U[512, 4096], 32 / 8 heads, head_dim 128) in fp32,
    the reference launchers' element type: paged attention v1 with its workspace (the fp32
    stream-K tile), K calls back to back.  Algorithmic bytes as for bf16, at 4 bytes per element.
    With num_heads 24 instead: the same load in bf16 at Llama-3.2-3B's heads (24 / 8, GQA 3)."""
    import dataclasses

    import torch

    from railgun_amd import workloads as wl
    from railgun_amd.ops import PagedAttentionKernels

    dt = torch.float32 if num_heads == 32 else torch.bfloat16
    w = dataclasses.replace(wl.config2(), dtype="f32" if dt == torch.float32 else "bf16", num_heads=num_heads)
    kernels = PagedAttentionKernels(0)
    shape = (w.num_blocks, w.num_kv_heads, w.block_size, w.head_dim)
    kc = torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(dt)
    vc = torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(dt)
    q = torch.randn((w.batch, w.num_heads, w.head_dim), generator=gen, device=device, dtype=torch.float32).to(dt)
    out = torch.empty_like(q)
    bt, ctx = torch.from_numpy(w.block_table).to(device), torch.from_numpy(w.context_lens).to(device)
    nbytes = kernels.v1_workspace_bytes(w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, w.max_blocks)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)

    def call():
        kernels.launch_v1(q, kc, vc, bt, ctx, out, w.scale, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size,
                          w.max_blocks, w.batch, workspace=ws)

    ms = time_events(call, steps, 3)
    gbs = w.decode_bytes() / (ms * 1e-3) / 1e9
    del kc, vc, ws
    torch.cuda.empty_cache()
    if dt == torch.bfloat16:
        return {"workload": f"config2_load_bf16_decode_{num_heads}q_{w.num_kv_heads}kv",
                "kernel": f"paged_attention_v1 (stream-K + merge, GQA {num_heads // w.num_kv_heads})",
                "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                "bytes": w.decode_bytes()}
    return {"workload": "config2_shape_fp32_decode", "kernel": "paged_attention_v1 (fp32 stream-K + merge)",
            "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": w.decode_bytes()}


def side_prefill(device, gen, steps: int, fp32: bool = False, num_heads: int = 32) -> dict:
    """Config 4's packed causal prefill (bf16; with fp32 the same shapes in the reference's
    element type, on the fp32 MFMA kernel, against the 157.3 TFLOP/s dense fp32 MFMA peak; with
    num_heads 24 the bf16 shapes at Llama-3.2-3B's heads, 24 / 8)."""
    import dataclasses

    import torch

    from railgun_amd import workloads as wl
    from railgun_amd.ops import PagedAttentionKernels, PagedAttentionOp, rope_cos_sin_table

    w = dataclasses.replace(wl.config4(), num_heads=num_heads)
    kernels = PagedAttentionKernels(0)
    op = PagedAttentionOp(w.scale, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size, kernels)
    T = w.num_tokens
    shape = (w.num_blocks, w.num_kv_heads, w.block_size, w.head_dim)
    mk = (lambda sh: bf16_normal(sh, gen, device).float()) if fp32 else (lambda sh: bf16_normal(sh, gen, device))
    kc, vc = mk(shape), mk(shape)
    q = mk((T, w.num_heads, w.head_dim))
    k = mk((T, w.num_kv_heads, w.head_dim))
    v = mk((T, w.num_kv_heads, w.head_dim))
    cs = rope_cos_sin_table(int(w.context_lens.max()), w.head_dim, w.rope_theta, device)
    i32 = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    pos, slots, bt, ctx, cu = (i32(a) for a in (w.positions, w.slot_mapping, w.block_table, w.context_lens,
                                                w.cu_seqlens))
    op.rope_reshape_and_cache(q, k, v, kc, vc, cs, pos, slots)
    out = torch.empty_like(q)
    maxq = int(w.seq_lens.max())

    def call():
        kernels.launch_prefill_packed(q, kc, vc, bt, ctx, cu, out, w.scale, w.num_heads, w.num_kv_heads,
                                      w.head_dim, w.block_size, w.max_blocks, w.num_seqs, T, maxq)

    ms = time_events(call, steps, 2)
    tflops = w.causal_flops() / (ms * 1e-3) / 1e12
    if fp32:
        return {"workload": "config4_shape_fp32_packed_prefill", "kernel": "prefill_f32_kernel "
                "(v_mfma_f32_32x32x2_f32)", "tokens": T, "us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 2),
                "frac_fp32_mfma_peak": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4), "flops": w.causal_flops()}
    if num_heads != 32:
        return {"workload": f"config4_shape_bf16_prefill_{num_heads}q_{w.num_kv_heads}kv", "tokens": T,
                "us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 2),
                "frac_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4), "flops": w.causal_flops()}
    return {"workload": w.name, "tokens": T, "us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 2),
            "frac_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4), "flops": w.causal_flops(),
            "traffic": measured_traffic("prefill_config4")}


def side_prefill_shapes(device, gen, steps: int) -> dict:
    """The bf16 packed prefill (config 4's heads, 32 / 8, D 128) on batches unlike config 4, side
    figures only: one long prompt, chunked prefill after a cached prefix (flops count the cached
    keys), and many short prompts.  Cache contents are N(0, 1) (the kernel's cost does not depend
    on them); tables drawn as config 4's."""
    import numpy as np
    import torch

    from railgun_amd import workloads as wl
    from railgun_amd.ops import PagedAttentionKernels

    kernels = PagedAttentionKernels(0)
    shapes = {"1x8192": ([8192], [0]), "4x2048_after_2048": ([2048] * 4, [2048] * 4),
              "16x512_after_4096": ([512] * 16, [4096] * 16), "64x128": ([128] * 64, [0] * 64)}
    out = {}
    for name, (lens, prior) in shapes.items():
        lens, prior = np.array(lens, np.int32), np.array(prior, np.int32)
        ctx = lens + prior
        mb = int(((ctx + 15) // 16).max())
        nb = int(((ctx + 15) // 16).sum()) + 8
        bt = wl.assign_blocks(ctx, 16, nb, mb, np.random.default_rng(1004))
        w = wl.PrefillWorkload(name, "bf16", 32, 8, 128, 16, nb, lens, bt, 1004, prior=prior)
        T = w.num_tokens
        shape = (w.num_blocks, w.num_kv_heads, w.block_size, w.head_dim)
        kc, vc = bf16_normal(shape, gen, device), bf16_normal(shape, gen, device)
        q = bf16_normal((T, w.num_heads, w.head_dim), gen, device)
        o = torch.empty_like(q)
        i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        btd, ctxd, cu = i32(w.block_table), i32(w.context_lens), i32(w.cu_seqlens)
        maxq = int(lens.max())

        def call():
            kernels.launch_prefill_packed(q, kc, vc, btd, ctxd, cu, o, w.scale, w.num_heads, w.num_kv_heads,
                                          w.head_dim, w.block_size, w.max_blocks, w.num_seqs, T, maxq)

        ms = time_events(call, steps, 2)
        tflops = w.causal_flops() / (ms * 1e-3) / 1e12
        out[name] = {"tokens": T, "cached": int(prior.sum()), "us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 2),
                     "frac_mfma_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4), "flops": w.causal_flops()}
        del kc, vc, q, o
        torch.cuda.empty_cache()
    return out


def side_model(device, steps: int) -> dict:
    """Config 5: one decode step of a random-init Llama-3.2-1B (16 layers, bf16 weights ~ N(0, 0.02))
    for 128 sequences with contexts U[64, 8192] over per-layer paged pools pre-filled with N(0, 1).
    The step runs as a captured HIP graph when its replays reproduce the eager logits bit for
    bit (eager otherwise); the attention share is the 16 layers' attention calls timed alone."""
    import numpy as np
    import torch

    from railgun_amd import workloads as wl
    from railgun_amd.batch import DecodeSlot, pack_step
    from railgun_amd.llama import LLAMA_3_2_1B as cfg
    from railgun_amd.kv_pool import GpuBlockPool
    from railgun_amd.llama import DeviceStep, LlamaWeights, RailgunLlama

    w = wl.config5()
    weights = LlamaWeights.random(cfg, 5, device)
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    pool = GpuBlockPool.for_model(cfg, w.num_blocks, w.block_size, device, fill=gen)
    model = RailgunLlama(cfg, weights, pool, max_position=int(w.context_lens.max()))
    rng = np.random.default_rng(w.seed)
    toks = rng.integers(0, cfg.vocab_size, w.batch)
    slots = [DecodeSlot(int(t), int(c), w.block_table[s, :(int(c) + w.block_size - 1) // w.block_size].tolist())
             for s, (t, c) in enumerate(zip(toks, w.context_lens))]
    st = DeviceStep.from_host(pack_step([], slots, w.block_size, max_blocks=w.block_table.shape[1]), device)

    eager_ms = time_events(lambda: model.forward(st), steps, 3)
    ref = model.forward(st)
    mode, step_ms = "eager", eager_ms
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        model.forward(st)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(graph):
        out = model.forward(st)
    same = True
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        same &= bool(torch.equal(out, ref))
        model.forward(st)  # eager work between replays
        torch.cuda.synchronize()
    if same:
        graph_ms = time_events(graph.replay, steps, 2)
        if graph_ms < eager_ms:
            mode, step_ms = "hip_graph", graph_ms
    # attention alone: the same 16 layers' decode attention calls back to back
    H, D = cfg.num_attention_heads, cfg.head_dim
    q = torch.randn((w.batch, H, D), device=device, dtype=torch.float32).to(torch.bfloat16)
    o = torch.empty_like(q)
    attn_ms = time_events(lambda: [model._attention(i, q, o, st) for i in range(cfg.num_hidden_layers)], steps, 2)
    kv = w.kv_bytes(cfg.num_hidden_layers, cfg.num_key_value_heads, D)
    step_bytes = weights.nbytes() + kv
    gemm = {f"{n}x{k}": "rg_linear" if v else "hipblaslt" for (_, n, k), v in model.linear_choice.items()}
    gemm["mlp"] = "fused gate/up + SiLU·mul" if model.mlp_choice.get(w.batch) else "gate/up + rg_silu_and_mul"
    gemm["qkv"] = ("fused qkv + RoPE + cache write" if model.qkv_choice.get(w.batch)
                   else "qkv + rg_qkv_rope_reshape_and_cache")
    fold = model.norm_chain.get(w.batch, (False, False))
    gemm["norms"] = {"input_norm": "folded into qkv (residual add in down_proj)" if fold[0] else "rg_rms_norm",
                     "post_attention_norm": "folded into gate/up (residual add in o_proj)" if fold[1]
                     else "rg_rms_norm"}
    del model, pool, weights, graph
    torch.cuda.empty_cache()
    return {"workload": w.name, "model": "llama-3.2-1b (random init, bf16)", "batch": w.batch,
            "context": "U[64,8192]", "context_tokens": int(w.context_lens.sum()), "mode": mode,
            "step_us": round(step_ms * 1e3, 1), "eager_step_us": round(eager_ms * 1e3, 1),
            "graph_matches_eager": same, "tokens_per_s": round(w.batch / (step_ms * 1e-3), 1),
            "attention_us": round(attn_ms * 1e3, 1), "attention_share": round(attn_ms / step_ms, 4),
            "gemm": gemm,
            "attention_GB/s": round(kv / (attn_ms * 1e-3) / 1e9, 1),
            "step_bytes": step_bytes, "step_GB/s": round(step_bytes / (step_ms * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(step_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def side_gemm(device) -> dict:
    """The Llama-3.2-1B decode projections (qkv, o_proj, gate/up, down, LM head) at 1 row and at
    config 5's 128 rows: rg_linear against hipBLASLt (torch F.linear), and at 128 rows the fused
    forms the model step runs (gate/up + SiLU·mul, q/k/v + RoPE + cache write, each with and
    without the folded RmsNorm; o_proj / down + residual add).  Each figure is the mean per call
    over HIP-graph replays of one call per copy of the weight, the copies totalling >= 600 MB, so
    that every call streams its weight from HBM as a decode step does (one weight timed in a loop
    would sit in the 256 MB last-level cache).  Weights bf16 ~ N(0, 0.02), activations N(0, 1)."""
    import torch
    import torch.nn.functional as F

    from railgun_amd.llama import graph_us
    from railgun_amd.ops import (PagedAttentionKernels, interleave_gate_up, linear, linear_residual,
                                 linear_silu_mul, linear_workspace_bytes, rope_cos_sin_table)

    shapes = {"qkv": (3072, 2048), "o_proj": (2048, 2048), "gate_up": (16384, 2048), "down": (2048, 8192),
              "lm_head": (128256, 2048)}
    g = torch.Generator(device=device)
    g.manual_seed(5)
    bf = torch.bfloat16

    def per_call(run, n):
        return graph_us(lambda: [run(j) for j in range(n)], calls=1, replays=5) / n

    def tb(n, k, us):
        return round(n * k * 2 / (us * 1e-6) / 1e12, 3)

    out = {}
    kern = PagedAttentionKernels(device)
    for rows in (1, 128):
        per = {}
        for name, (n, k) in shapes.items():
            copies = max(2, -(-600_000_000 // (n * k * 2)))
            x = torch.randn((rows, k), device=device, generator=g).to(bf)
            ws_ = [(0.02 * torch.randn((n, k), device=device, generator=g)).to(bf) for _ in range(copies)]
            o = torch.empty((rows, n), device=device, dtype=bf)
            wsp = torch.empty(max(16, linear_workspace_bytes(rows, n, k)), dtype=torch.uint8, device=device)
            t_rg = per_call(lambda j: linear(x, ws_[j], o, wsp), copies)
            t_blas = per_call(lambda j: F.linear(x, ws_[j]), copies)
            entry = {"rg_linear_us": round(t_rg, 2), "hipblaslt_us": round(t_blas, 2),
                     "rg_linear_weight_TB/s": tb(n, k, t_rg), "weight_copies": copies}
            if rows == 128 and name in ("o_proj", "down"):
                res = torch.randn((rows, n), device=device, generator=g).to(bf)
                t = per_call(lambda j: linear_residual(x, ws_[j], res, wsp), copies)
                entry["rg_linear_residual_us"] = round(t, 2)
            if rows == 128 and name == "gate_up":
                il = [interleave_gate_up(w) for w in ws_]
                nw = (1 + 0.1 * torch.randn((k,), device=device, generator=g)).to(bf)
                act = torch.empty((rows, n // 2), device=device, dtype=bf)
                entry["rg_linear_silu_mul_us"] = round(per_call(lambda j: linear_silu_mul(x, il[j], act), copies), 2)
                entry["rg_rms_norm_linear_silu_mul_us"] = round(
                    per_call(lambda j: linear_silu_mul(x, il[j], act, norm_weight=nw, eps=1e-5), copies), 2)
                del il
            if rows == 128 and name == "qkv":
                H, Hkv, D, bs = 32, 8, 64, 16
                q = torch.empty((rows, H, D), device=device, dtype=bf)
                pool = torch.zeros((64, 2, Hkv, bs, D), device=device, dtype=bf)
                cs = rope_cos_sin_table(4096, D, 500000.0, device)
                pos = torch.arange(rows, device=device, dtype=torch.int32)
                nw = (1 + 0.1 * torch.randn((k,), device=device, generator=g)).to(bf)

                def qkv(j, norm):
                    kern.launch_linear_qkv_rope_reshape_and_cache(x, ws_[j], q, pool[:, 0], pool[:, 1], cs, pos, pos,
                                                                  H, Hkv, D, bs, norm_weight=norm, eps=1e-5)
                entry["rg_linear_qkv_rope_reshape_and_cache_us"] = round(per_call(lambda j: qkv(j, None), copies), 2)
                entry["rg_rms_norm_linear_qkv_rope_reshape_and_cache_us"] = round(
                    per_call(lambda j: qkv(j, nw), copies), 2)
            per[name] = entry
            del x, ws_, o, wsp
            torch.cuda.empty_cache()
        out[f"rows_{rows}"] = per
    return out


def copy_calibration(device, steps: int) -> dict:
    """A plain device copy of 1 GiB (torch's copy kernel): reads and writes exactly 1 GiB per
    launch, which is what the HBM counters of a profile are scaled against."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    ms = time_events(lambda: dst.copy_(src), steps, 2)
    return {"workload": "copy_1GiB", "bytes_read": n, "bytes_written": n, "us": round(ms * 1e3, 2),
            "GB/s": round(2 * n / (ms * 1e-3) / 1e9, 1)}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(across GPUs the decode path would shard by sequence or kv-head with no exchange)"}))
        return 2
    import torch

    from railgun_amd import workloads as wl

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(1002)
    if args.only == "v2":
        print(json.dumps(side_v2(device, gen, args.steps)), flush=True)
        return 0
    if args.only == "fp32":
        print(json.dumps({"decode": side_fp32(device, gen, args.steps),
                          "prefill": side_prefill(device, gen, max(3, args.steps // 5), fp32=True)}), flush=True)
        return 0
    if args.only == "prefill":
        print(json.dumps(side_prefill(device, gen, args.steps)), flush=True)
        return 0
    if args.only == "model":
        print(json.dumps(side_model(device, args.steps)), flush=True)
        return 0
    if args.only == "copy":
        print(json.dumps(copy_calibration(device, args.steps)), flush=True)
        return 0
    if args.only == "gemm":
        print(json.dumps(side_gemm(device)), flush=True)
        return 0
    w = wl.config2()
    log(f"[bench] config2: B={w.batch} tokens={int(w.context_lens.sum())} pool={w.num_blocks} blocks")
    st = decode_setup(w, device, gen)

    def step():
        fused_step_call(w, st)

    def chain_step():
        rope_cache_call(w, st)
        v1_call(w, st)

    for _ in range(args.warmup):
        step()
    settle(step)
    torch.cuda.synchronize()
    # Timed region: exactly K whole steps, back to back, between one pair of events.
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for _ in range(args.steps):
        step()
    t_end.record()
    torch.cuda.synchronize()
    ms_step = t_start.elapsed_time(t_end) / args.steps
    # The same step as two entries (rg_rope_reshape_and_cache, then rg_paged_attention_v1).
    ms_chain = time_events(chain_step, args.steps, 2)
    # paged_attention_v1 alone (the roofline's kernel): K calls back to back, same inputs.
    ms_v1 = time_events(lambda: v1_call(w, st), args.steps, 2)
    value = w.fused_step_bytes() / (ms_step * 1e-3) / 1e9
    chain_bytes = w.decode_bytes() + w.rope_cache_bytes()
    achieved = w.decode_bytes() / (ms_v1 * 1e-3) / 1e9
    log(f"[bench] step {ms_step * 1e3:.1f} us (two entries {ms_chain * 1e3:.1f} us), v1 {ms_v1 * 1e3:.1f} us, "
        f"{achieved:.0f} GB/s")
    del st
    torch.cuda.empty_cache()

    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_ms": SETTLE_MS, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) q/k/v and pool, shuffled tables)",
        "config": {"workload": w.name, "batch": w.batch, "context": "U[512,4096]", "context_tokens":
                   int(w.context_lens.sum()), "heads": f"{w.num_heads}/{w.num_kv_heads}", "head_dim": w.head_dim,
                   "block_size": w.block_size, "pool_blocks": w.num_blocks,
                   "step": "RoPE(theta 5e5) + reshape_and_cache of the 64 new tokens fused into "
                           "paged_attention_v1 (rg_rope_reshape_and_cache_paged_attention_v1)"},
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "step_bytes": w.fused_step_bytes(),
        "step_traffic": measured_traffic("fused_decode_step_config2"),
        "two_entry_step": {"entries": "rg_rope_reshape_and_cache, then rg_paged_attention_v1",
                           "us": round(ms_chain * 1e3, 2), "bytes": chain_bytes,
                           "GBps": round(chain_bytes / (ms_chain * 1e-3) / 1e9, 1),
                           "frac_hbm_peak": round(chain_bytes / (ms_chain * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": "paged_attention_v1 (decode partition + merge)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("paged_attention_v1_config2"),
                     "traffic_source": "profiles/hbm_traffic_counters.txt (rocprofv3 FETCH_SIZE x2 + WRITE_SIZE, "
                                       f"measured at commit {measured_traffic('commit')})",
                     "algorithmic_bytes": w.decode_bytes(), "us_per_launch": round(ms_v1 * 1e3, 2)},
    }
    if args.only == "decode":
        print(json.dumps(result), flush=True)
        return 0
    if not args.no_side:
        log("[bench] config3 v2 ...")
        result["v2_long_context"] = side_v2(device, gen, max(3, args.steps // 5))
        log("[bench] config2 shape in fp32 ...")
        result["fp32_decode"] = side_fp32(device, gen, max(3, args.steps // 5))
        log("[bench] config4 prefill ...")
        result["prefill"] = side_prefill(device, gen, 10)
        log("[bench] config4 prefill in fp32 ...")
        result["fp32_prefill"] = side_prefill(device, gen, 3, fp32=True)
        log("[bench] GQA 3 (24 / 8 heads): config 2 decode load, config 4 prefill ...")
        result["gqa3"] = {"decode": side_fp32(device, gen, max(3, args.steps // 5), num_heads=24),
                          "prefill": side_prefill(device, gen, 10, num_heads=24)}
        log("[bench] config5 model step ...")
        result["model_step"] = side_model(device, 10)
        log("[bench] config5 projections ...")
        result["gemm"] = side_gemm(device)
        # Last: it launches config 4's prefill kernel on other shapes, and the profiles take
        # config 4's timed launches as the last of that kernel before the fp32 prefill leg.
        log("[bench] prefill on other batch shapes ...")
        result["prefill_shapes"] = side_prefill_shapes(device, gen, 10)
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
