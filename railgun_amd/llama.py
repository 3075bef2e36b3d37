"""Llama forward pass (packed prefill + decode) over the attention hot path.

Mirrors Railgun's model code (crates/vllm-models/src/llama/architecture.rs:11-165,
attention.rs:85-155): ``RailgunLlama`` = embedding, ``LlamaLayer`` x N, final RMSNorm and
the (tied) LM head; a layer is RMSNorm -> ``PagedSelfAttention`` -> residual add ->
RMSNorm -> ``LlamaMLP`` (SwiGLU) -> residual add.  One engine step (prefill chunks first,
then decode slots, :mod:`railgun_amd.batch`) runs as:

* q, k and v from one GEMM with the concatenated projection weights, then
  ``rg_qkv_rope_reshape_and_cache``: RoPE on q and k, k and v into this layer's paged cache,
  one pass (the reference writes the cache but never applies RoPE, defect D10);
* attention: ``rg_prefill_packed`` for the prefill rows (causal, MFMA), the stream-K
  ``rg_paged_attention_v1`` for the decode rows (the reference sends prefill rows through
  the decode op, D7);
* ``rg_rms_norm`` fuses each residual add with the next RMSNorm; ``rg_silu_and_mul`` is the
  SwiGLU gate;
* the projections of decode-sized steps (at most 128 rows) run on ``rg_linear``, the skinny
  MFMA GEMM, unless hipBLASLt (``F.linear``) measured more than 5 % faster for that shape on
  this device: each (rows, out, in) shape is timed when an eager step first meets it (three
  interleaved graph-replay trials of each, medians compared).  Larger (prefill) steps use
  hipBLASLt.  The MLP's gate/up projection and SiLU·mul run as one ``rg_linear_silu_mul`` (the
  gate/up weight is held with its rows interleaved in blocks of 16, replaced in place) when that
  measured faster than the projection followed by ``rg_silu_and_mul``.  ``choices`` (or the
  ``RAILGUN_LLAMA_CHOICES`` environment variable) fixes these choices instead of timing them.

Every layer owns a KV pool in Railgun's fused layout ``[NB, 2, H_kv, bs, D]``
(crates/vllm-paged-attention/src/block.rs:70,89-95); the reference shares one pool across
layers (D11).  Activations are bf16 (or the weights' dtype), arithmetic inside each kernel
fp32, every op's result rounded once to the activation dtype, as in candle.
"""
from __future__ import annotations

import logging
import math
import os
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from .batch import StepBatch
from .kv_pool import GpuBlockPool
from .ops import (LINEAR_MAX_ROWS, PagedAttentionKernels, deinterleave_gate_up, interleave_gate_up, linear,
                  linear_residual, linear_silu_mul, linear_workspace_bytes, rms_norm, rope_cos_sin_table,
                  silu_and_mul)

log = logging.getLogger(__name__)

# How RailgunLlama picks between the equivalent forms of a step's projections (rg_linear or
# hipBLASLt, fused or separate SiLU·mul and RoPE + cache write, RmsNorm folded or not):
# "measured" times both once per shape on the device and keeps the faster (with a 5 % margin
# for the hand-written form), "rg" always takes the hand-written / fused / folded form where the
# shape allows it, "blas" always hipBLASLt and the separate launches.  The forms round
# differently, so a fixed mode makes the logits of a step the same in every process and on
# every box.  The constructor's `choices` argument wins over the environment variable.
CHOICE_MODES = ("measured", "rg", "blas")
CHOICES_ENV = "RAILGUN_LLAMA_CHOICES"


def graph_us(fn, calls: int = 10, replays: int = 3) -> float:
    """Mean device time of ``fn`` (a few launches) over graph replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                   # warm-up outside the capture (library set-up)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / (calls * replays)


@dataclass(frozen=True)
class LlamaConfig:
    """The fields of candle's llama Config the model reads (crates/vllm-models/src/config.rs:30-67)."""

    hidden_size: int = 2048
    intermediate_size: int = 8192
    num_hidden_layers: int = 16
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    vocab_size: int = 128256
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    tie_word_embeddings: bool = True

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def qkv_size(self) -> int:
        return (self.num_attention_heads + 2 * self.num_key_value_heads) * self.head_dim


LLAMA_3_2_1B = LlamaConfig()


@dataclass
class LayerWeights:
    input_norm: torch.Tensor   # [hidden]
    wqkv: torch.Tensor         # [(H + 2 H_kv) D, hidden]: q_proj, k_proj, v_proj stacked
    wo: torch.Tensor           # [hidden, H D]
    post_norm: torch.Tensor    # [hidden]
    w_gate_up: torch.Tensor    # [2 I, hidden]: gate_proj, up_proj stacked
    w_down: torch.Tensor       # [hidden, I]
    # True once RailgunLlama has replaced w_gate_up in place by its rows interleaved in blocks
    # of 16 (interleave_gate_up: the layout rg_linear_silu_mul reads), so that only one copy
    # of the weight is held; deinterleave_gate_up gives the stacked rows back.
    gate_up_interleaved: bool = False


@dataclass
class LlamaWeights:
    embed: torch.Tensor        # [vocab, hidden]
    layers: list
    norm: torch.Tensor         # [hidden]
    lm_head: torch.Tensor      # [vocab, hidden] (the embedding when tied)

    @staticmethod
    def random(cfg: LlamaConfig, seed: int, device, dtype=torch.bfloat16, std: float = 0.02,
               norm_jitter: float = 0.0) -> "LlamaWeights":
        """Random init: projections and embedding ~ N(0, std); norm weights 1 (+ N(0, jitter))."""
        g = torch.Generator(device=device)
        g.manual_seed(seed)

        def normal(*shape, s=std):
            return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * s).to(dtype)

        def norm_w():
            w = torch.ones(cfg.hidden_size, device=device, dtype=torch.float32)
            if norm_jitter:
                w += torch.randn(cfg.hidden_size, generator=g, device=device) * norm_jitter
            return w.to(dtype)

        hd, inter = cfg.hidden_size, cfg.intermediate_size
        embed = normal(cfg.vocab_size, hd)
        layers = [LayerWeights(norm_w(), normal(cfg.qkv_size, hd), normal(hd, cfg.num_attention_heads * cfg.head_dim),
                               norm_w(), normal(2 * inter, hd), normal(hd, inter))
                  for _ in range(cfg.num_hidden_layers)]
        norm = norm_w()
        lm_head = embed if cfg.tie_word_embeddings else normal(cfg.vocab_size, hd)
        return LlamaWeights(embed, layers, norm, lm_head)

    @staticmethod
    def from_state_dict(cfg: LlamaConfig, sd: dict, device, dtype=torch.bfloat16) -> "LlamaWeights":
        """From Hugging Face Llama parameter names (the names architecture.rs loads, :24-28, :101-118)."""
        def t(name):
            return sd[name].to(device=device, dtype=dtype).contiguous()

        layers = []
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            wqkv = torch.cat([t(p + "self_attn.q_proj.weight"), t(p + "self_attn.k_proj.weight"),
                              t(p + "self_attn.v_proj.weight")], 0).contiguous()
            wgu = torch.cat([t(p + "mlp.gate_proj.weight"), t(p + "mlp.up_proj.weight")], 0).contiguous()
            layers.append(LayerWeights(t(p + "input_layernorm.weight"), wqkv, t(p + "self_attn.o_proj.weight"),
                                       t(p + "post_attention_layernorm.weight"), wgu, t(p + "mlp.down_proj.weight")))
        embed = t("model.embed_tokens.weight")
        lm_head = embed if cfg.tie_word_embeddings or "lm_head.weight" not in sd else t("lm_head.weight")
        return LlamaWeights(embed, layers, t("model.norm.weight"), lm_head)

    def nbytes(self) -> int:
        """Bytes one forward reads: every weight once (the tied LM head counted again: the
        embedding gather touches only the batch's rows, the LM head reads the whole matrix)."""
        n = sum(w.numel() * w.element_size() for L in self.layers
                for w in (L.input_norm, L.wqkv, L.wo, L.post_norm, L.w_gate_up, L.w_down))
        return n + self.norm.numel() * self.norm.element_size() + self.lm_head.numel() * self.lm_head.element_size()


@dataclass
class DeviceStep:
    """A :class:`StepBatch` copied to the device, with the prefill / decode split views."""

    host: StepBatch
    tokens: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    context_lens: torch.Tensor
    block_table: torch.Tensor
    cu_seqlens: torch.Tensor
    last_rows: torch.Tensor

    @staticmethod
    def from_host(b: StepBatch, device) -> "DeviceStep":
        def d(a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device)

        return DeviceStep(b, d(b.tokens), d(b.positions), d(b.slot_mapping), d(b.context_lens), d(b.block_table),
                          d(b.cu_seqlens), d(b.last_rows))


class RailgunLlama:
    """architecture.rs:86-165 on the gfx950 kernels.  ``forward`` runs one packed engine
    step and returns the logits of each request's last token ``[requests, vocab]``
    (engine.rs:238-245 samples from those)."""

    def __init__(self, cfg: LlamaConfig, weights: LlamaWeights, pool: GpuBlockPool,
                 kernels: Optional[PagedAttentionKernels] = None, max_position: Optional[int] = None,
                 choices: Optional[str] = None):
        mode = choices or os.environ.get(CHOICES_ENV) or "measured"
        if mode not in CHOICE_MODES:
            raise ValueError(f"choices must be one of {CHOICE_MODES}, got {mode!r}")
        self.choice_mode = mode
        self.cfg = cfg
        self.w = weights
        self.pool = pool
        self.device = weights.embed.device
        self.dtype = weights.embed.dtype
        self.kernels = kernels or PagedAttentionKernels(self.device)
        max_pos = max_position or pool.num_blocks * pool.block_size
        self.cos_sin = rope_cos_sin_table(max_pos, cfg.head_dim, cfg.rope_theta, self.device)
        self.scale = 1.0 / math.sqrt(cfg.head_dim)  # attention.rs:69-70
        self._ws = torch.empty(0, dtype=torch.uint8, device=self.device)
        # (rows, out_features, in_features) -> True for rg_linear, False for hipBLASLt
        self.linear_choice: dict = {}
        # rows -> True for rg_linear_silu_mul, False for the projection + rg_silu_and_mul
        self.mlp_choice: dict = {}
        # The fused MLP form reads the gate/up weight with its rows interleaved in blocks of 16:
        # each layer's weight is replaced by that layout in place (one copy held, not two); the
        # separate form then de-interleaves the projection's output columns instead.
        self._w_gate_up_il: dict = {}  # layer -> interleaved copy, only for weights left stacked
        if mode != "blas" and self.dtype in (torch.bfloat16, torch.float16) and cfg.intermediate_size % 16 == 0:
            for L in weights.layers:
                if not L.gate_up_interleaved:
                    L.w_gate_up = interleave_gate_up(L.w_gate_up)
                    L.gate_up_interleaved = True
        # rows -> True for rg_linear_qkv_rope_reshape_and_cache, False for the projection +
        # rg_qkv_rope_reshape_and_cache
        self.qkv_choice: dict = {}
        # rows -> (input norm, post-attention norm): True where the RmsNorm is folded into the
        # projection after it (rg_rms_norm_linear_qkv_rope_reshape_and_cache with the residual add
        # in down_proj, rg_rms_norm_linear_silu_mul with the residual add in o_proj:
        # rg_linear_residual), False for rg_rms_norm + the projections above
        self.norm_chain: dict = {}
        # Hook for measurements: called as attention_hook("begin"/"end", layer) around each
        # layer's attention kernels (None in normal use).
        self.attention_hook = None

    def _workspace(self, nbytes: int) -> torch.Tensor:
        if self._ws.numel() < nbytes:
            self._ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self._ws

    def _attention(self, layer: int, q: torch.Tensor, out: torch.Tensor, st: DeviceStep) -> None:
        cfg, b, k = self.cfg, st.host, self.kernels
        kc, vc = self.pool.k_cache(layer), self.pool.v_cache(layer)
        H, Hkv, D, bs = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, self.pool.block_size
        mb = int(st.block_table.shape[1])
        P, TP = b.num_prefill_seqs, b.num_prefill_tokens
        if P:
            k.launch_prefill_packed(q[:TP], kc, vc, st.block_table[:P], st.context_lens[:P], st.cu_seqlens,
                                    out[:TP], self.scale, H, Hkv, D, bs, mb, P, TP, b.max_query_len)
        nd = b.num_decode
        if nd:
            ws = self._workspace(k.v1_workspace_bytes(nd, H, Hkv, D, bs, mb))
            k.launch_v1(q[TP:], kc, vc, st.block_table[P:], st.context_lens[P:], out[TP:], self.scale, H, Hkv, D,
                        bs, mb, nd, workspace=ws if ws.numel() else None)

    def _rg_linear_fits(self, x: torch.Tensor, weight: torch.Tensor) -> bool:
        rows, k = (int(d) for d in x.shape)
        n = int(weight.shape[0])
        return (0 < rows <= LINEAR_MAX_ROWS and n % 16 == 0 and k % 128 == 0 and x.stride(1) == 1
                and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and weight.is_contiguous()
                and weight.data_ptr() % 16 == 0 and x.dtype in (torch.bfloat16, torch.float16))

    def _peers(self, name: str) -> list:
        """The weight `name` of every layer (the LM head alone for "lm_head")."""
        if name == "lm_head":
            return [self.w.lm_head]
        return [getattr(L, name) for L in self.w.layers]

    @staticmethod
    def _time_pair(run_a, run_b, n: int) -> tuple:
        """Device times of run_a(j) and run_b(j) for j = 0 .. n - 1 under graph replay, medians of
        three interleaved trials (a clock or load change on the device hits both).  Each j is
        another layer's weight, so the weights stream from HBM as they do in a step rather than
        from the 256 MB last-level cache that a single weight timed in a loop would sit in."""
        calls = max(1, 20 // n)
        t_a, t_b = [], []
        for _ in range(3):
            t_a.append(graph_us(lambda: [run_a(j) for j in range(n)], calls=calls))
            t_b.append(graph_us(lambda: [run_b(j) for j in range(n)], calls=calls))
        return sorted(t_a)[1], sorted(t_b)[1]

    def _linear(self, x: torch.Tensor, name: str, layer: int = 0) -> torch.Tensor:
        """x @ weight^T for the weight `name` of `layer`, on rg_linear or hipBLASLt per the
        measured choice for the shape."""
        peers = self._peers(name)
        weight = peers[layer]
        if not self._rg_linear_fits(x, weight):
            return F.linear(x, weight)
        rows, k, n = int(x.shape[0]), int(x.shape[1]), int(weight.shape[0])
        key = (rows, n, k)
        use_rg = self.linear_choice.get(key)
        ws_bytes = linear_workspace_bytes(rows, n, k)
        if use_rg is None:
            if self._fixed() is not None:
                use_rg = self._fixed()
            elif torch.cuda.is_current_stream_capturing():
                use_rg = True                  # no timing inside a capture: the kernel built for it
            else:
                out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
                ws = self._workspace(ws_bytes)
                t_rg, t_blas = self._time_pair(lambda j: linear(x, peers[j], out, ws),
                                               lambda j: F.linear(x, peers[j]), len(peers))
                use_rg = not t_blas < 0.95 * t_rg
                log.info("projection %s: rg_linear %.2f us, hipBLASLt %.2f us -> %s", key, t_rg, t_blas,
                         "rg_linear" if use_rg else "hipBLASLt")
            self.linear_choice[key] = use_rg
        if not use_rg:
            return F.linear(x, weight)
        return linear(x, weight, workspace=self._workspace(ws_bytes) if ws_bytes else None)

    def _mlp_act(self, layer: int, h: torch.Tensor, act: torch.Tensor) -> None:
        """act = silu(h @ gate^T) * (h @ up^T), fused or as the projection + rg_silu_and_mul."""
        L = self.w.layers[layer]
        inter = int(act.shape[1])
        rows = int(h.shape[0])
        if not (self._rg_linear_fits(h, L.w_gate_up) and inter % 16 == 0):
            self._mlp_act_separate(layer, h, act)
            return
        fused = self.mlp_choice.get(rows)
        if fused is None:
            if self._fixed() is not None:
                fused = self._fixed()
            elif torch.cuda.is_current_stream_capturing():
                fused = True
            else:
                n = len(self.w.layers)
                self._linear(h, "w_gate_up", layer)  # settles the projection's own choice outside the timing
                t_f, t_s = self._time_pair(lambda j: linear_silu_mul(h, self._gate_up_il(j), act),
                                           lambda j: self._mlp_act_separate(j, h, act), n)
                fused = not t_s < 0.95 * t_f
                log.info("MLP at %d rows: fused gate/up + SiLU·mul %.2f us, separate %.2f us -> %s", rows, t_f,
                         t_s, "fused" if fused else "separate")
            self.mlp_choice[rows] = fused
        if fused:
            linear_silu_mul(h, self._gate_up_il(layer), act)
        else:
            self._mlp_act_separate(layer, h, act)

    def _mlp_act_separate(self, layer: int, h: torch.Tensor, act: torch.Tensor) -> None:
        """The gate/up projection, then rg_silu_and_mul over [gate | up] columns."""
        y = self._linear(h, "w_gate_up", layer)
        silu_and_mul(deinterleave_gate_up(y) if self.w.layers[layer].gate_up_interleaved else y, act)

    def _qkv_rope_cache(self, layer: int, h: torch.Tensor, q: torch.Tensor, st: DeviceStep) -> None:
        """q/k/v = h @ wqkv^T, RoPE on q and k, k and v into the paged cache: fused in the
        projection's epilogue or as the projection + rg_qkv_rope_reshape_and_cache."""
        cfg, L = self.cfg, self.w.layers[layer]
        H, Hkv, D, bs = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, self.pool.block_size
        kc, vc = self.pool.k_cache(layer), self.pool.v_cache(layer)
        rows = int(h.shape[0])
        peers = self._peers("wqkv")

        # Both forms write into this layer's cache; timed with another layer's weight they leave
        # other values at the step's slots, which the call below overwrites.
        def unfused(j):
            self.kernels.launch_qkv_rope_reshape_and_cache(self._linear(h, "wqkv", j), q, kc, vc, self.cos_sin,
                                                          st.positions, st.slot_mapping, H, Hkv, D, bs, rows)

        def fused(j):
            self.kernels.launch_linear_qkv_rope_reshape_and_cache(h, peers[j], q, kc, vc, self.cos_sin, st.positions,
                                                                  st.slot_mapping, H, Hkv, D, bs)

        if not (self._rg_linear_fits(h, L.wqkv) and D in (32, 64) and q.is_contiguous()):
            unfused(layer)
            return
        use_fused = self.qkv_choice.get(rows)
        if use_fused is None:
            if self._fixed() is not None:
                use_fused = self._fixed()
            elif torch.cuda.is_current_stream_capturing():
                use_fused = True
            else:
                self._linear(h, "wqkv", layer)  # settles the projection's own choice outside the timing
                t_f, t_u = self._time_pair(fused, unfused, len(peers))
                use_fused = not t_u < 0.95 * t_f
                log.info("q/k/v at %d rows: fused with RoPE + cache write %.2f us, separate %.2f us -> %s", rows,
                         t_f, t_u, "fused" if use_fused else "separate")
            self.qkv_choice[rows] = use_fused
        (fused if use_fused else unfused)(layer)

    def check_step(self, b: StepBatch) -> None:
        """The kernels trust their indices (as the reference's do): check them on the host."""
        if b.num_tokens and int(b.positions.max()) >= self.cos_sin.shape[0]:
            raise ValueError(f"position {int(b.positions.max())} beyond the RoPE table ({self.cos_sin.shape[0]})")
        if b.block_table.size and (int(b.block_table.max()) >= self.pool.num_blocks or int(b.block_table.min()) < 0):
            raise ValueError(f"block id outside the pool of {self.pool.num_blocks} blocks")
        if b.num_tokens and int(b.slot_mapping.max()) >= self.pool.num_blocks * self.pool.block_size:
            raise ValueError("slot outside the pool")

    def _norm_chain_fits(self, rows: int) -> bool:
        cfg = self.cfg
        return (0 < rows <= LINEAR_MAX_ROWS and cfg.head_dim in (32, 64) and cfg.hidden_size % 128 == 0
                and cfg.hidden_size <= 8192 and cfg.intermediate_size % 128 == 0
                and self.dtype in (torch.bfloat16, torch.float16))

    def _gate_up_il(self, layer: int) -> torch.Tensor:
        """Layer `layer`'s gate/up weight in the interleaved layout rg_linear_silu_mul reads: the
        weight itself once interleaved in place, else a copy kept beside it."""
        L = self.w.layers[layer]
        if L.gate_up_interleaved:
            return L.w_gate_up
        w_il = self._w_gate_up_il.get(layer)
        if w_il is None:
            w_il = self._w_gate_up_il[layer] = interleave_gate_up(L.w_gate_up)
        return w_il

    def _fixed(self) -> Optional[bool]:
        """The form a fixed choice mode takes (True: hand-written / fused / folded), None when
        the choices are measured."""
        return None if self.choice_mode == "measured" else self.choice_mode == "rg"

    def choices(self) -> dict:
        """The choices made so far, by kind and shape (for logs and reproducing a run)."""
        return {"mode": self.choice_mode,
                "linear": {f"{r}x{n}x{k}": "rg_linear" if v else "hipblaslt"
                           for (r, n, k), v in self.linear_choice.items()},
                "mlp_fused": dict(self.mlp_choice), "qkv_fused": dict(self.qkv_choice),
                "norms_folded": dict(self.norm_chain)}

    def _use_norm_chain(self, st: DeviceStep) -> tuple:
        """Which RmsNorms of this step's layers are folded into the projection after them, as
        (attention side, MLP side): the input norm into q/k/v (with the residual add of the MLP
        output moved into down_proj) and the post-attention norm into gate/up (with the residual
        add moved into o_proj).  Each side is measured once per row count against rg_rms_norm +
        the projections, over every layer's weights with scratch activations, before the step's
        first layer (so that the cache rows the timing writes are rewritten by the step itself)."""
        cfg = self.cfg
        rows = st.host.num_tokens
        if not self._norm_chain_fits(rows):
            return (False, False)
        use = self.norm_chain.get(rows)
        if use is not None:
            return (use, use) if isinstance(use, bool) else use
        if self._fixed() is not None:
            use = (self._fixed(), self._fixed())
        elif torch.cuda.is_current_stream_capturing():
            use = (True, True)
        else:
            H, D, eps = cfg.num_attention_heads, cfg.head_dim, cfg.rms_norm_eps
            Hkv, bs = cfg.num_key_value_heads, self.pool.block_size
            g = torch.Generator(device=self.device).manual_seed(0)
            x = torch.randn((rows, cfg.hidden_size), generator=g, device=self.device).to(self.dtype)
            delta = x.clone()
            h = torch.empty_like(x)
            q = torch.empty((rows, H, D), device=self.device, dtype=self.dtype)
            attn = torch.randn((rows, H * D), generator=g, device=self.device).to(self.dtype)
            act = torch.randn((rows, cfg.intermediate_size), generator=g, device=self.device).to(self.dtype)
            ws_o = self._workspace(max(linear_workspace_bytes(rows, cfg.hidden_size, H * D),
                                       linear_workspace_bytes(rows, cfg.hidden_size, cfg.intermediate_size)))
            layers = self.w.layers

            def attn_folded(j):
                self.kernels.launch_linear_qkv_rope_reshape_and_cache(
                    x, layers[j].wqkv, q, self.pool.k_cache(j), self.pool.v_cache(j), self.cos_sin, st.positions,
                    st.slot_mapping, H, Hkv, D, bs, norm_weight=layers[j].input_norm, eps=eps)
                linear_residual(act, layers[j].w_down, x, ws_o)

            def attn_unfolded(j):
                rms_norm(delta, layers[j].input_norm, h, eps, residual=x)
                self._qkv_rope_cache(j, h, q, st)
                delta.copy_(self._linear(act, "w_down", j))

            def mlp_folded(j):
                linear_residual(attn, layers[j].wo, x, ws_o)
                linear_silu_mul(x, self._gate_up_il(j), act, norm_weight=layers[j].post_norm, eps=eps)

            def mlp_unfolded(j):
                rms_norm(self._linear(attn, "wo", j), layers[j].post_norm, h, eps, residual=x)
                self._mlp_act(j, h, act)

            n = len(layers)
            t_af, t_au = self._time_pair(attn_folded, attn_unfolded, n)
            t_mf, t_mu = self._time_pair(mlp_folded, mlp_unfolded, n)
            use = (not t_au < 0.95 * t_af, not t_mu < 0.95 * t_mf)
            log.info("RmsNorm folds at %d rows: input norm %.2f / %.2f us, post-attention norm %.2f / %.2f us "
                     "(folded / separate) -> %s", rows, t_af, t_au, t_mf, t_mu, use)
        self.norm_chain[rows] = use
        return use

    @torch.no_grad()
    def forward(self, st: DeviceStep) -> torch.Tensor:
        cfg, w = self.cfg, self.w
        self.check_step(st.host)
        T = st.host.num_tokens
        H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        x = F.embedding(st.tokens, w.embed)                     # residual stream [T, hidden]
        h = torch.empty_like(x)
        q = torch.empty((T, H, D), device=self.device, dtype=self.dtype)
        attn = torch.empty_like(q)
        act = torch.empty((T, cfg.intermediate_size), device=self.device, dtype=self.dtype)
        delta = None                                            # projection output not yet added to x
        fold_attn, fold_mlp = self._use_norm_chain(st)
        ws_res = self._workspace(max(linear_workspace_bytes(T, cfg.hidden_size, H * D),
                                     linear_workspace_bytes(T, cfg.hidden_size, cfg.intermediate_size))) \
            if (fold_attn or fold_mlp) else None
        for i, L in enumerate(w.layers):
            if fold_attn:
                # input_layernorm folded into the q/k/v projection (+ RoPE, cache write); the
                # previous down_proj already added its output to x
                self.kernels.launch_linear_qkv_rope_reshape_and_cache(
                    x, L.wqkv, q, self.pool.k_cache(i), self.pool.v_cache(i), self.cos_sin, st.positions,
                    st.slot_mapping, H, Hkv, D, self.pool.block_size, norm_weight=L.input_norm, eps=eps)
            else:
                # input_layernorm (with the previous MLP's residual add), architecture.rs:49-50
                rms_norm(delta if delta is not None else x, L.input_norm, h, eps,
                         residual=x if delta is not None else None)
                self._qkv_rope_cache(i, h, q, st)               # q/k/v, RoPE, cache write
            if self.attention_hook:
                self.attention_hook("begin", i)
            self._attention(i, q, attn, st)
            if self.attention_hook:
                self.attention_hook("end", i)
            if fold_mlp:
                # o_proj + residual add, then post_attention_layernorm folded into gate/up + SiLU·mul
                linear_residual(attn.view(T, H * D), L.wo, x, ws_res)
                linear_silu_mul(x, self._gate_up_il(i), act, norm_weight=L.post_norm, eps=eps)
            else:
                delta = self._linear(attn.view(T, H * D), "wo", i)
                # residual add + post_attention_layernorm, architecture.rs:53-57
                rms_norm(delta, L.post_norm, h, eps, residual=x)
                self._mlp_act(i, h, act)                        # LlamaMLP, architecture.rs:80-84
            if fold_attn:
                linear_residual(act, L.w_down, x, ws_res)       # down_proj + residual add
                delta = None
            else:
                delta = self._linear(act, "w_down", i)
        # last residual add (unless down_proj made it) + model.norm
        rms_norm(delta if delta is not None else x, w.norm, h, eps, residual=x if delta is not None else None)
        return self._linear(h.index_select(0, st.last_rows), "lm_head")


__all__ = ["DeviceStep", "LLAMA_3_2_1B", "LayerWeights", "LlamaConfig", "LlamaWeights",
           "RailgunLlama", "graph_us"]
