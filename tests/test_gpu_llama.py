"""The model-step kernels and the Llama forward pass (railgun_amd.llama) on the GPU.

Kernel level: rg_rms_norm and rg_silu_and_mul against the same arithmetic on the CPU (the
residual add bit-exact, the normalised and gated outputs within one bf16 rounding);
rg_qkv_rope_reshape_and_cache bit-exact against rg_rope_reshape_and_cache on contiguous
copies of the same rows (the latter is bit-exact against the oracle, test_gpu_cache.py).

Model level: random-init tiny Llamas (weights from Hugging Face's initialiser, rounded to
bf16 on both sides) run a packed prefill, a decode step and a mixed chunked-prefill +
decode step through the GPU path, and the logits are compared with oracle/llama_ref.py
(pinned against transformers' LlamaForCausalLM in tests/test_llama_oracle.py).  bf16
activations make the GPU result drift from the float32 oracle; the bound is measured on the
CPU for each case: the oracle rerun with bf16 rounding at the same points (act_dtype) gives
the drift that rounding alone explains, and the GPU must stay within twice that (plus
1e-3) of the float32 oracle and agree with it to a cosine similarity of 0.999.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import llama_ref
from railgun_amd.batch import DecodeSlot, PrefillChunk, pack_step
from railgun_amd.kv_pool import GpuBlockPool
from railgun_amd.llama import DeviceStep, LlamaConfig, LlamaWeights, RailgunLlama
from railgun_amd.ops import deinterleave_gate_up, rms_norm, rope_cos_sin_table, silu_and_mul

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def _bf16_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


@pytest.mark.parametrize("hidden", [2048, 6144, 8200, 120, 100])  # 16-byte rows of 1-5 vectors per thread, a short row, scalar form
def test_rms_norm_residual(device, hidden):
    g = torch.Generator().manual_seed(hidden)
    rows = 37
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    r = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    w = (1 + 0.3 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    dx, dr, dw = x.to(device), r.clone().to(device), w.to(device)
    out = torch.empty_like(dx)
    rms_norm(dx, dw, out, 1e-5, residual=dr)
    torch.cuda.synchronize()
    s = (r.float() + x.float()).to(torch.bfloat16)            # residual add, rounded once
    assert torch.equal(dr.cpu(), s)
    sf = s.float()
    want = sf * torch.rsqrt(sf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.float()
    torch.testing.assert_close(out.cpu().float(), want, atol=0, rtol=2 ** -7)
    out2 = torch.empty_like(dx)
    rms_norm(dx, dw, out2, 1e-5)                               # no residual
    xf = x.float()
    want2 = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.float()
    torch.testing.assert_close(out2.cpu().float(), want2, atol=0, rtol=2 ** -7)


@pytest.mark.parametrize("inter", [8192, 200, 300])  # full and partial workgroups per row
def test_silu_and_mul(device, inter):
    g = torch.Generator().manual_seed(inter)
    gu = (3 * torch.randn(9, 2 * inter, generator=g)).to(torch.bfloat16)
    out = torch.empty(9, inter, dtype=torch.bfloat16, device=device)
    silu_and_mul(gu.to(device), out)
    a = _bf16_round(torch.nn.functional.silu(gu[:, :inter].float()))
    want = a * gu[:, inter:].float()
    torch.testing.assert_close(out.cpu().float(), want, atol=1e-6, rtol=2 ** -7)


@pytest.mark.parametrize("D,H,Hkv", [(64, 32, 8), (128, 8, 2)])
def test_qkv_rope_cache_matches_contiguous_entry(device, kernels, D, H, Hkv):
    g = torch.Generator().manual_seed(D)
    T, bs, nb = 29, 16, 40
    width = (H + 2 * Hkv) * D + 8                                # padded rows: stride > row
    qkv = torch.randn(T, width, generator=g).to(torch.bfloat16).to(device)
    pos = torch.randint(0, 500, (T,), generator=g, dtype=torch.int32).to(device)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    slots[3] = -1
    slots = slots.to(device)
    cs = rope_cos_sin_table(512, D, 500000.0, device)
    pool_a = torch.randn(nb, 2, Hkv, bs, D, generator=g).to(torch.bfloat16).to(device)
    pool_b = pool_a.clone()
    q_out = torch.empty(T, H, D, dtype=torch.bfloat16, device=device)
    kernels.launch_qkv_rope_reshape_and_cache(qkv[:, :width - 8], q_out, pool_a[:, 0], pool_a[:, 1], cs, pos, slots,
                                              H, Hkv, D, bs, T)
    q = qkv[:, :H * D].reshape(T, H, D).clone()
    k = qkv[:, H * D:(H + Hkv) * D].reshape(T, Hkv, D).contiguous()
    v = qkv[:, (H + Hkv) * D:(H + 2 * Hkv) * D].reshape(T, Hkv, D).contiguous()
    kernels.launch_rope_reshape_and_cache(q, k, v, pool_b[:, 0], pool_b[:, 1], cs, pos, slots, H, Hkv, D, bs, T)
    torch.cuda.synchronize()
    assert torch.equal(q_out.view(torch.int16), q.view(torch.int16))
    assert torch.equal(pool_a.view(torch.int16), pool_b.view(torch.int16))


# ------------------------------------------------------------------------ model ----

def _hf_state(cfg: LlamaConfig, seed: int) -> dict:
    hc = transformers.LlamaConfig(
        hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
        num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps,
        rope_theta=cfg.rope_theta, tie_word_embeddings=True, max_position_embeddings=8192, hidden_act="silu")
    torch.manual_seed(seed)
    m = transformers.LlamaForCausalLM(hc)
    sd = {}
    for k, v in m.state_dict().items():
        v = v.detach().float()
        if k.endswith("norm.weight"):
            v = v + 0.2 * torch.randn_like(v)
        sd[k] = _bf16_round(v)  # the GPU's bf16 weights, exactly
    return sd


def _tables(lens, bs, nb, seed):
    perm = np.random.default_rng(seed).permutation(nb)
    out, cur = [], 0
    for n in lens:
        k = (n + bs - 1) // bs
        out.append([int(b) for b in perm[cur:cur + k]])
        cur += k
    return out


def _check(gpu: torch.Tensor, ref32: torch.Tensor, ref16: torch.Tensor, what: str) -> None:
    gpu = gpu.float().cpu()
    drift = float((ref16 - ref32).abs().max())
    err = float((gpu - ref32).abs().max())
    cos = torch.nn.functional.cosine_similarity(gpu, ref32, dim=-1).min().item()
    assert err <= 2 * drift + 1e-3, f"{what}: |gpu - fp32 oracle| {err:.4g} vs bf16 drift {drift:.4g}"
    assert cos > 0.999, f"{what}: cosine similarity {cos}"


CONFIGS = {
    # MFMA paths: GQA 4, head_dim 64, block 16 (prefill MFMA tile, stream-K decode)
    "mfma_d64": LlamaConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=8,
                            num_key_value_heads=2, vocab_size=1000),
    # generic kernels: head_dim 32, GQA 2
    "generic_d32": LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=8,
                               num_key_value_heads=4, vocab_size=700),
}


class _AlwaysRgLinear(dict):
    """A projection choice table that sends every eligible shape to rg_linear."""

    def get(self, key, default=None):
        return True


class _Never(dict):
    """A choice table that declines every eligible shape (the RmsNorm-folded chain)."""

    def get(self, key, default=None):
        return False


class _Fixed(dict):
    """A choice table that answers every eligible shape with the same value."""

    def __init__(self, value):
        super().__init__()
        self.value = value

    def get(self, key, default=None):
        return self.value


@pytest.mark.parametrize("gemm", ["measured", "rg_linear", "norm_chain", "fold_attn_only", "fold_mlp_only",
                                  "choices_rg", "choices_blas"])
@pytest.mark.parametrize("name", list(CONFIGS))
def test_llama_prefill_decode_mixed(device, kernels, name, gemm):
    """Prefill, mixed and decode steps against the CPU model.  With gemm="rg_linear" every
    projection of the mixed (113 rows) and decode (4 rows) steps runs on rg_linear, the MLP's
    gate/up with SiLU·mul fused (rg_linear_silu_mul) and q/k/v with RoPE and the cache write
    fused (rg_linear_qkv_rope_reshape_and_cache); "norm_chain" also folds the RmsNorms into those
    projections and the residual adds into o_proj / down_proj (rg_rms_norm_linear_*,
    rg_linear_residual), "fold_attn_only" / "fold_mlp_only" one side of it; "measured" keeps the
    per-shape timing choice of normal use.  "choices_rg" / "choices_blas" are the constructor's
    fixed modes (every hand-written, fused and folded form; hipBLASLt and separate launches with
    the gate/up weight left stacked)."""
    _mixed_steps(device, kernels, CONFIGS[name], gemm, torch.bfloat16)


@pytest.mark.parametrize("gemm", ["measured", "norm_chain"])
def test_llama_f16_steps(device, kernels, gemm):
    """The same prefill, mixed and decode steps with fp16 weights, activations and KV pool (the
    oracle's weights rounded to fp16, its drift reference rounding to fp16)."""
    _mixed_steps(device, kernels, CONFIGS["mfma_d64"], gemm, torch.float16)


def _mixed_steps(device, kernels, cfg, gemm, dtype):
    bs, nb = 16, 96
    sd = _hf_state(cfg, 11)
    if dtype != torch.bfloat16:
        sd = {k: v.to(dtype).float() for k, v in sd.items()}
    w = LlamaWeights.from_state_dict(cfg, sd, device, dtype=dtype)
    pool = GpuBlockPool.for_model(cfg, nb, bs, device, dtype=dtype)
    mode = {"choices_rg": "rg", "choices_blas": "blas"}.get(gemm)
    model = RailgunLlama(cfg, w, pool, kernels, max_position=4096, choices=mode)
    assert w.layers[0].gate_up_interleaved == (mode != "blas")
    if gemm not in ("measured", "choices_rg", "choices_blas"):
        model.linear_choice = _AlwaysRgLinear()
        model.mlp_choice = _AlwaysRgLinear()
        model.qkv_choice = _AlwaysRgLinear()
        model.norm_chain = _Fixed({"rg_linear": (False, False), "norm_chain": (True, True),
                                   "fold_attn_only": (True, False), "fold_mlp_only": (False, True)}[gemm])
    ref32 = llama_ref.ReferenceLlama(cfg, sd, nb, bs)
    ref16 = llama_ref.ReferenceLlama(cfg, sd, nb, bs, act_dtype=dtype)
    rng = np.random.default_rng(7)
    lens = [40, 77, 130, 300]
    prompts = [rng.integers(0, cfg.vocab_size, n).tolist() for n in lens]
    bts = _tables(lens, bs, nb, 8)

    def run(step, what):
        got = model.forward(DeviceStep.from_host(step, device))
        torch.cuda.synchronize()
        _check(got, ref32.forward(step), ref16.forward(step), what)

    # step 1: prompts 0-2 prefilled whole but for the last token; prompt 3 its first 190 tokens
    run(pack_step([PrefillChunk(p[:-1], 0, bt) for p, bt in zip(prompts[:3], bts[:3])]
                  + [PrefillChunk(prompts[3][:190], 0, bts[3])], [], bs), "prefill")
    # step 2: prompt 3's second chunk (position_start 190) next to decode slots of prompts 0-2
    run(pack_step([PrefillChunk(prompts[3][190:], 190, bts[3])],
                  [DecodeSlot(p[-1], len(p), bt) for p, bt in zip(prompts[:3], bts[:3])], bs), "mixed")
    # step 3: decode only, every sequence one token further
    ext = [rng.integers(0, cfg.vocab_size) for _ in lens]
    run(pack_step([], [DecodeSlot(int(t), n + 1, bt) for t, n, bt in zip(ext, lens, bts)], bs), "decode")
    if mode is not None:
        made = model.choices()
        assert made["mode"] == mode
        want = mode == "rg"
        assert all(v == ("rg_linear" if want else "hipblaslt") for v in made["linear"].values())
        assert all(v == want for v in made["mlp_fused"].values()) and all(v == want for v in made["qkv_fused"].values())
        assert all(v == (want, want) for v in made["norms_folded"].values())


def _hf_state_of(cfg: LlamaConfig, w: LlamaWeights) -> dict:
    """Hugging Face-named float32 CPU copies of the GPU model's bf16 weights (the same values),
    split back into q/k/v and gate/up."""
    H, Hkv, D, inter = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size
    f = lambda t: t.float().cpu()  # noqa: E731
    sd = {"model.embed_tokens.weight": f(w.embed), "model.norm.weight": f(w.norm)}
    for i, L in enumerate(w.layers):
        p = f"model.layers.{i}."
        qkv = f(L.wqkv)
        # (the interleave permutes the weight's rows: de-interleave along dim 0)
        gu = f(deinterleave_gate_up(L.w_gate_up.t()).t() if L.gate_up_interleaved else L.w_gate_up)
        sd[p + "self_attn.q_proj.weight"] = qkv[:H * D]
        sd[p + "self_attn.k_proj.weight"] = qkv[H * D:(H + Hkv) * D]
        sd[p + "self_attn.v_proj.weight"] = qkv[(H + Hkv) * D:]
        sd[p + "self_attn.o_proj.weight"] = f(L.wo)
        sd[p + "mlp.gate_proj.weight"] = gu[:inter]
        sd[p + "mlp.up_proj.weight"] = gu[inter:]
        sd[p + "mlp.down_proj.weight"] = f(L.w_down)
        sd[p + "input_layernorm.weight"] = f(L.input_norm)
        sd[p + "post_attention_layernorm.weight"] = f(L.post_norm)
    return sd


def test_llama_config5_decode_step(device, kernels):
    """BASELINE config 5 at its own shape: random-init Llama-3.2-1B (16 layers, hidden 2048,
    32 / 8 heads, head_dim 64, intermediate 8192, vocab 128256, bf16 weights ~ N(0, 0.02), tied
    LM head), one decode step of 128 sequences with contexts U[64, 8192] over per-layer paged
    pools pre-filled with N(0, 1) (block 16, shuffled tables).  The logits of 8 sequences —
    the longest and the shortest among them — are compared with the float32 CPU model
    (oracle/llama_ref.py) run on those sequences alone: decode rows are independent, so the
    oracle gets a compact pool holding only their blocks, copied from the GPU pools."""
    from railgun_amd import workloads as wl
    from railgun_amd.llama import LLAMA_3_2_1B as cfg

    w = wl.config5()
    bs = w.block_size
    weights = LlamaWeights.random(cfg, 5, device)
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    pool = GpuBlockPool.for_model(cfg, w.num_blocks, bs, device, fill=gen)
    model = RailgunLlama(cfg, weights, pool, kernels, max_position=int(w.context_lens.max()))
    rng = np.random.default_rng(w.seed)
    toks = rng.integers(0, cfg.vocab_size, w.batch)
    nblk = [(int(c) + bs - 1) // bs for c in w.context_lens]
    slots = [DecodeSlot(int(t), int(c), w.block_table[s, :nblk[s]].tolist())
             for s, (t, c) in enumerate(zip(toks, w.context_lens))]
    logits = model.forward(DeviceStep.from_host(pack_step([], slots, bs, max_blocks=w.block_table.shape[1]), device))
    torch.cuda.synchronize()
    assert logits.shape == (128, 128256)

    order = np.argsort(w.context_lens, kind="stable")
    pick = sorted({int(order[i]) for i in np.linspace(0, w.batch - 1, 8).round().astype(int)})
    assert len(pick) == 8 and int(order[-1]) in pick and int(order[0]) in pick
    # compact pool: the picked sequences' blocks renumbered 0..n-1, every layer copied
    ids = np.concatenate([w.block_table[s, :nblk[s]] for s in pick]).astype(np.int64)
    assert len(set(ids.tolist())) == len(ids)
    sub_slots, cur = [], 0
    for s in pick:
        sub_slots.append(DecodeSlot(int(toks[s]), int(w.context_lens[s]), list(range(cur, cur + nblk[s]))))
        cur += nblk[s]
    sub_step = pack_step([], sub_slots, bs)
    sd = _hf_state_of(cfg, weights)
    ref32 = llama_ref.ReferenceLlama(cfg, sd, 1, bs)
    ref16 = llama_ref.ReferenceLlama(cfg, sd, 1, bs, act_dtype=torch.bfloat16)
    dev_ids = torch.from_numpy(ids).to(device)
    for layer in range(cfg.num_hidden_layers):
        blocks = pool.storage[layer].index_select(0, dev_ids).float().cpu()   # [n, 2, H_kv, bs, D]
        k, v = blocks[:, 0].contiguous(), blocks[:, 1].contiguous()
        # each reference writes its own new-token row before reading: sharing the pool is safe
        ref32.k[layer], ref32.v[layer] = k, v
        ref16.k[layer], ref16.v[layer] = k, v
    want32 = ref32.forward(sub_step)
    want16 = ref16.forward(sub_step)
    _check(logits[torch.as_tensor(pick, device=device)], want32, want16, "config 5 decode step")
