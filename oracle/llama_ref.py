"""CPU restatement of Railgun's Llama forward step — TEST INFRASTRUCTURE ONLY.

Only tests/ import this module, as the checker of railgun_amd.llama; the product path never
does.  Plain torch on the CPU, float32 arithmetic throughout:

* layer (crates/vllm-models/src/llama/architecture.rs:38-59): x += attn(rmsnorm(x));
  x += mlp(rmsnorm(x)); final rmsnorm and the tied LM head (:101-118, :141-156);
* RMSNorm (candle_nn::RmsNorm): x / sqrt(mean(x^2) + eps) * w;
* MLP (:80-84): down(silu(gate(x)) * up(x));
* attention (attention.rs:85-155, with the defects the build fixes): q/k/v projections,
  rotate-half RoPE at each token's position (HF Llama convention, theta from the config),
  k/v written to the layer's paged cache at slot_mapping (paged_attention.cu:111-138), then
  for every token softmax(q k^T / sqrt(D)) v over cache positions 0..pos of its sequence,
  gathered through the block table (paged_attention.cu:55-62), q-head h on kv-head h/G;
* the step's packing follows engine.rs:184-227 (railgun_amd.batch.StepBatch).

``act_dtype=torch.bfloat16`` rounds every op result to bf16 at the points where the GPU path
stores a bf16 activation (after each GEMM, norm, residual add, RoPE, attention, SiLU and
product), so the rounding error of bf16 activations alone can be measured on the CPU.

Pinned by tests/test_llama_oracle.py: equal, within float32 rounding, to Hugging Face
transformers' LlamaForCausalLM (an independent implementation) on the same weights, for
whole prompts and for decode steps after a prefill.
"""
from __future__ import annotations

import math

import torch


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [T, D/2] of angle pos * theta^(-2i/D), computed in float64."""
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim)
    ang = positions.to(torch.float64)[:, None] * inv[None, :]
    return torch.cos(ang).float(), torch.sin(ang).float()


def rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half on x [T, heads, D] (rope.cu:34-41): (lo, hi) -> (lo c - hi s, hi c + lo s)."""
    half = x.shape[-1] // 2
    lo, hi = x[..., :half], x[..., half:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([lo * c - hi * s, hi * c + lo * s], dim=-1)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


class ReferenceLlama:
    """Weights as float32 CPU tensors with Hugging Face names; one float32 KV cache
    [NB, H_kv, bs, D] pair per layer."""

    def __init__(self, cfg, state_dict: dict, num_blocks: int, block_size: int, act_dtype=torch.float32):
        self.cfg = cfg
        self.w = {k: v.detach().to(torch.float32).cpu() for k, v in state_dict.items()}
        if "lm_head.weight" not in self.w or cfg.tie_word_embeddings:
            self.w["lm_head.weight"] = self.w["model.embed_tokens.weight"]
        shape = (num_blocks, cfg.num_key_value_heads, block_size, cfg.head_dim)
        self.k = [torch.zeros(shape) for _ in range(cfg.num_hidden_layers)]
        self.v = [torch.zeros(shape) for _ in range(cfg.num_hidden_layers)]
        self.block_size = block_size
        self.act = act_dtype

    def rd(self, t: torch.Tensor) -> torch.Tensor:
        return t if self.act == torch.float32 else t.to(self.act).to(torch.float32)

    def attention(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, batch) -> torch.Tensor:
        cfg, bs = self.cfg, self.block_size
        H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        G = H // Hkv
        kc, vc = self.k[layer], self.v[layer]
        for t, slot in enumerate(batch.slot_mapping.tolist()):  # reshape_and_cache, slot < 0 skipped
            if slot >= 0:
                kc[slot // bs, :, slot % bs] = k[t]
                vc[slot // bs, :, slot % bs] = v[t]
        out = torch.zeros_like(q)
        cu = batch.cu_seqlens.tolist()
        rows_of = [list(range(cu[r], cu[r + 1])) for r in range(batch.num_prefill_seqs)]
        rows_of += [[batch.num_prefill_tokens + i] for i in range(batch.num_decode)]
        for r, rows in enumerate(rows_of):
            ctx = int(batch.context_lens[r])
            blocks = torch.as_tensor(batch.block_table[r, : (ctx + bs - 1) // bs].astype("int64"))
            keys = kc[blocks].permute(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :ctx]   # [Hkv, ctx, D]
            vals = vc[blocks].permute(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :ctx]
            for t in rows:
                lim = self.keys_seen(int(batch.positions[t]), ctx)
                for h in range(H):
                    kvh = self.kv_head(h, G)
                    s = keys[kvh, :lim] @ q[t, h] / math.sqrt(D)
                    p = torch.softmax(s, dim=0)
                    out[t, h] = p @ vals[kvh, :lim]
        return out

    @staticmethod
    def kv_head(h: int, group: int) -> int:
        """q-head h reads kv-head h / G (paged_attention.cu:40)."""
        return h // group

    @staticmethod
    def keys_seen(pos: int, ctx: int) -> int:
        """A token at position pos attends to cache positions 0..pos (causal)."""
        return pos + 1

    @torch.no_grad()
    def forward(self, batch) -> torch.Tensor:
        """Logits [requests, vocab] of each request's last token for one packed step."""
        cfg, w, rd = self.cfg, self.w, self.rd
        H, Hkv, D, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rms_norm_eps
        T = batch.num_tokens
        cos, sin = rope_cos_sin(torch.as_tensor(batch.positions.astype("int64")), D, cfg.rope_theta)
        x = w["model.embed_tokens.weight"][torch.as_tensor(batch.tokens)]
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            h = rd(rms_norm(x, w[p + "input_layernorm.weight"], eps))
            q = rd(h @ w[p + "self_attn.q_proj.weight"].T).view(T, H, D)
            k = rd(h @ w[p + "self_attn.k_proj.weight"].T).view(T, Hkv, D)
            v = rd(h @ w[p + "self_attn.v_proj.weight"].T).view(T, Hkv, D)
            q, k = rd(rotate(q, cos, sin)), rd(rotate(k, cos, sin))
            a = rd(self.attention(i, q, k, v, batch)).reshape(T, H * D)
            x = rd(x + rd(a @ w[p + "self_attn.o_proj.weight"].T))
            h = rd(rms_norm(x, w[p + "post_attention_layernorm.weight"], eps))
            g = rd(h @ w[p + "mlp.gate_proj.weight"].T)
            u = rd(h @ w[p + "mlp.up_proj.weight"].T)
            m = rd(rd(torch.nn.functional.silu(g)) * u)
            x = rd(x + rd(m @ w[p + "mlp.down_proj.weight"].T))
        h = rd(rms_norm(x, w["model.norm.weight"], eps))
        return rd(h[torch.as_tensor(batch.last_rows)] @ w["lm_head.weight"].T)
