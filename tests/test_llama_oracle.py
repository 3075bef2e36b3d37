"""Pins oracle/llama_ref.py (the CPU restatement of Railgun's Llama step) and the host
batch packing (railgun_amd/batch.py) on the CPU.

The model oracle is compared with Hugging Face transformers' LlamaForCausalLM, an
independent implementation, on the same random weights: prompts prefilled in one packed
step must give HF's logits at each prompt's last position, a following decode step HF's
logits one position further, and a mixed step (a second prefill chunk with
position_start > 0 next to decode slots) the same.  Mistakes planted in copies of the
oracle (RoPE sign, GQA head mapping, causal limit) must make the comparison fail.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import llama_ref
from railgun_amd.batch import CPU_BLOCK_FLAG, DecodeSlot, PrefillChunk, pack_step, slot_of
from railgun_amd.llama import LlamaConfig

transformers = pytest.importorskip("transformers")

TINY = LlamaConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
                   num_key_value_heads=2, vocab_size=300, rms_norm_eps=1e-5, rope_theta=500000.0)


def hf_model(cfg: LlamaConfig, seed: int):
    hc = transformers.LlamaConfig(
        hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
        num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps,
        rope_theta=cfg.rope_theta, tie_word_embeddings=True, max_position_embeddings=4096, attention_bias=False,
        mlp_bias=False, hidden_act="silu")
    torch.manual_seed(seed)
    m = transformers.LlamaForCausalLM(hc).float().eval()
    with torch.no_grad():  # norm weights away from 1 so that a dropped weight shows
        for n, p in m.named_parameters():
            if n.endswith("norm.weight"):
                p.add_(0.2 * torch.randn_like(p))
    return m


def hf_logits(m, ids):
    with torch.no_grad():
        return m(torch.as_tensor([list(ids)])).logits[0].float()


def tables(lens, bs, nb, seed):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(nb)
    out, cur = [], 0
    for n in lens:
        k = (n + bs - 1) // bs
        out.append([int(b) for b in perm[cur:cur + k]])
        cur += k
    return out


@pytest.fixture(scope="module")
def setup():
    m = hf_model(TINY, 0)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, TINY.vocab_size, n).tolist() for n in (6, 17, 33)]
    full = [hf_logits(m, p) for p in prompts]
    return m, prompts, full


def run_prefill_then_decode(ref_cls, m, prompts, bs=16, nb=64):
    bts = tables([len(p) for p in prompts], bs, nb, 1)
    ref = ref_cls(TINY, m.state_dict(), nb, bs)
    step1 = pack_step([PrefillChunk(p[:-1], 0, bt) for p, bt in zip(prompts, bts)], [], bs)
    l1 = ref.forward(step1)
    step2 = pack_step([], [DecodeSlot(p[-1], len(p), bt) for p, bt in zip(prompts, bts)], bs)
    l2 = ref.forward(step2)
    return l1, l2


def test_oracle_matches_hf_prefill_and_decode(setup):
    m, prompts, full = setup
    l1, l2 = run_prefill_then_decode(llama_ref.ReferenceLlama, m, prompts)
    for r, p in enumerate(prompts):
        torch.testing.assert_close(l1[r], full[r][len(p) - 2], atol=2e-5, rtol=1e-4)
        torch.testing.assert_close(l2[r], full[r][len(p) - 1], atol=2e-5, rtol=1e-4)


def test_oracle_mixed_chunked_step(setup):
    """Prompt 2 prefilled in two chunks; the second chunk shares a step with decode slots."""
    m, prompts, full = setup
    bs, nb = 4, 64  # small blocks: chunks and tokens cross block boundaries
    bts = tables([len(p) for p in prompts], bs, nb, 2)
    ref = llama_ref.ReferenceLlama(TINY, m.state_dict(), nb, bs)
    a, b, c = prompts
    ref.forward(pack_step([PrefillChunk(a[:-1], 0, bts[0]), PrefillChunk(b[:-1], 0, bts[1]),
                           PrefillChunk(c[:13], 0, bts[2])], [], bs))
    step = pack_step([PrefillChunk(c[13:], 13, bts[2])],
                     [DecodeSlot(a[-1], len(a), bts[0]), DecodeSlot(b[-1], len(b), bts[1])], bs)
    out = ref.forward(step)
    torch.testing.assert_close(out[0], full[2][len(c) - 1], atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(out[1], full[0][len(a) - 1], atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(out[2], full[1][len(b) - 1], atol=2e-5, rtol=1e-4)


class _GqaModulo(llama_ref.ReferenceLlama):
    @staticmethod
    def kv_head(h, group):  # planted: q-head h on kv-head h % H_kv instead of h / G
        return h % TINY.num_key_value_heads


class _NotCausal(llama_ref.ReferenceLlama):
    @staticmethod
    def keys_seen(pos, ctx):  # planted: every row sees its whole context
        return ctx


@pytest.mark.parametrize("mistake", ["rope_sign", "gqa", "causal"])
def test_planted_mistakes_are_caught(setup, mistake, monkeypatch):
    m, prompts, full = setup
    cls = llama_ref.ReferenceLlama
    if mistake == "rope_sign":
        def bad_rotate(x, cos, sin):
            half = x.shape[-1] // 2
            lo, hi = x[..., :half], x[..., half:]
            return torch.cat([lo * cos[:, None] + hi * sin[:, None], hi * cos[:, None] - lo * sin[:, None]], -1)
        monkeypatch.setattr(llama_ref, "rotate", bad_rotate)
    else:
        cls = {"gqa": _GqaModulo, "causal": _NotCausal}[mistake]
    l1, l2 = run_prefill_then_decode(cls, m, prompts)
    worst = max(float((l2[r] - full[r][len(p) - 1]).abs().max()) for r, p in enumerate(prompts))
    worst = max(worst, max(float((l1[r] - full[r][len(p) - 2]).abs().max()) for r, p in enumerate(prompts)))
    assert worst > 1e-3, f"planted {mistake} not detected (max diff {worst})"


# ------------------------------------------------------------------ batch packing ----

def test_pack_step_layout_matches_engine_flatten():
    """engine.rs:184-227 on a hand-computed case: prefill chunks first, then decode slots;
    tables padded with block 0; ctx = position_start + len or seq_len; slots from
    scheduler.rs:230-235 / :258-263."""
    bs = 4
    st = pack_step([PrefillChunk([11, 12, 13], 2, [7, 3]), PrefillChunk([21], 0, [5])],
                   [DecodeSlot(99, 6, [9, 1]), DecodeSlot(98, 1, [4])], bs)
    assert st.tokens.tolist() == [11, 12, 13, 21, 99, 98]
    assert st.positions.tolist() == [2, 3, 4, 0, 5, 0]
    # pos 2 -> block 7 off 2 = 30; pos 3 -> 31; pos 4 -> block 3 off 0 = 12; 21 at pos 0 of block 5 = 20;
    # decode seq_len 6 -> pos 5 -> block 1 off 1 = 5; seq_len 1 -> pos 0 -> block 4 off 0 = 16
    assert st.slot_mapping.tolist() == [30, 31, 12, 20, 5, 16]
    assert st.context_lens.tolist() == [5, 1, 6, 1]
    assert st.block_table.tolist() == [[7, 3], [5, 0], [9, 1], [4, 0]]
    assert st.block_table.dtype == np.int32 and st.slot_mapping.dtype == np.int32
    assert st.cu_seqlens.tolist() == [0, 3, 4]
    assert (st.num_prefill_seqs, st.num_prefill_tokens, st.num_decode) == (2, 4, 2)
    assert st.max_context_len == 6 and st.max_query_len == 3
    assert st.last_rows.tolist() == [2, 3, 4, 5]


def test_pack_step_slots_against_formula():
    rng = np.random.default_rng(3)
    bs = 16
    lens = rng.integers(1, 200, 20)
    bts = tables(lens, bs, 400, 4)
    st = pack_step([], [DecodeSlot(1, int(n), bt) for n, bt in zip(lens, bts)], bs, max_blocks=16)
    for r, (n, bt) in enumerate(zip(lens, bts)):
        assert st.slot_mapping[r] == bt[(n - 1) // bs] * bs + (n - 1) % bs == slot_of(bt, int(n) - 1, bs)
        assert st.block_table[r, len(bt):].tolist() == [0] * (16 - len(bt))


def test_pack_step_rejects_bad_tables():
    with pytest.raises(ValueError):  # a CPU-resident block (BlockId bit 31)
        pack_step([], [DecodeSlot(1, 3, [CPU_BLOCK_FLAG | 2])], 16)
    with pytest.raises(ValueError):  # table too short for the context
        pack_step([], [DecodeSlot(1, 17, [0])], 16)
    with pytest.raises(ValueError):
        pack_step([PrefillChunk([], 0, [0])], [], 16)
    with pytest.raises(ValueError):
        pack_step([], [DecodeSlot(1, 20, [0, 1])], 16, max_blocks=1)
