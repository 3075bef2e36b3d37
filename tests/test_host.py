"""Host-side checks that need no GPU: the C ABI surface, argument validation, batch packing.

Argument checks return before any HIP call, so they run on a CPU-only machine; they mirror
the reference's CoreError::NotSupported / CoreError::Tensor cases
(crates/vllm-cuda/src/kernels/mod.rs:42-54, 477-482).
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

import railgun_amd
from railgun_amd import _lib
from railgun_amd import workloads as wl
from railgun_amd.ops import PagedAttentionOp, RailgunError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "railgun_hip.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(rg_[a-z0-9_]+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = railgun_amd.load_library()
    names = declared_symbols()
    assert len(names) >= 16, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/railgun_hip.h but not exported"
    # and the Python binding declares exactly the header's functions
    assert sorted(_lib.SIGNATURES) == names
    assert lib.rg_abi_version() == 1


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_header_compiles_standalone(lang, tmp_path):
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text('#include "railgun_hip.h"\nint main(void) { return RG_OK; }\n')
    cc = "gcc" if lang == "c" else "g++"
    r = subprocess.run([cc, "-Wall", "-Werror", "-fsyntax-only", f"-I{ROOT}/include", str(src)], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr


def test_cpp_mirror_header_compiles(tmp_path):
    """include/railgun_hip.hpp (the C++ mirror of PagedAttentionKernels / PagedAttentionOp)
    compiles standalone as C++17 against the HIP runtime headers."""
    src = tmp_path / "t.cpp"
    src.write_text('#include "railgun_hip.hpp"\nint main() { return railgun::dtype_size(railgun::DType::BF16) == 2 ? 0 : 1; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include", f"-I{ROOT}/include", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def call(name, *args):
    lib = railgun_amd.load_library()
    return getattr(lib, name)(*args), _lib.last_error()


def test_argument_checks_without_gpu():
    st, msg = call("rg_paged_attention_v1_plus", None, None, None, None, None, None, None, 1.0, 4, 4, 66, 16, 2, 1,
                   _lib.RG_DTYPE_F32, 0, None, 0, None)
    assert st == _lib.RG_ERR_NOT_SUPPORTED and "head_dim must be a multiple of 4 and <= 256, but got 66" in msg
    st, msg = call("rg_paged_attention_v1", None, None, None, None, None, None, 1.0, 4, 4, 512, 16, 2, 1,
                   _lib.RG_DTYPE_BF16, 0, None, 0, None)
    assert st == _lib.RG_ERR_NOT_SUPPORTED
    st, msg = call("rg_paged_attention_v2_reduce", None, None, None, None, None, None, 4, 2048, 1, 1, 256,
                   _lib.RG_DTYPE_F32, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "exceeds maximum block size" in msg
    st, msg = call("rg_paged_attention_v1", None, None, None, None, None, None, 1.0, 6, 4, 64, 16, 2, 1,
                   _lib.RG_DTYPE_F32, 0, None, 0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "not a multiple of num_kv_heads" in msg
    st, msg = call("rg_paged_attention_v2_partition", None, None, None, None, None, None, None, None, None, 1.0, 4,
                   4, 64, 16, 4, 2, 1, 24, _lib.RG_DTYPE_F32, 0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "multiple of block_size" in msg
    st, msg = call("rg_rope", None, None, None, 4, 7, 3, _lib.RG_DTYPE_F32, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT
    st, msg = call("rg_reshape_and_cache", None, None, None, None, None, 8, 128, 16, 0, _lib.RG_DTYPE_BF16, 0, None)
    assert st == _lib.RG_OK  # zero tokens: nothing to do
    st, msg = call("rg_reshape_and_cache", None, None, None, None, None, 8, 128, 16, 4, 9, 0, None)
    assert st == _lib.RG_ERR_NOT_SUPPORTED
    st, msg = call("rg_reshape_and_cache", None, None, None, None, None, 8, 128, 16, 4, _lib.RG_DTYPE_BF16, 100,
                   None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "kv_block_stride" in msg
    st, msg = call("rg_prefill_packed", None, None, None, None, None, None, None, 1.0, 32, 8, 128, 16, 8, 0, 5, 5,
                   _lib.RG_DTYPE_BF16, 0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "without sequences" in msg


def test_model_entry_argument_checks_without_gpu():
    """rg_copy_blocks / rg_rms_norm / rg_silu_and_mul / rg_qkv_rope_reshape_and_cache reject bad
    arguments before touching the GPU."""
    st, msg = call("rg_copy_blocks", None, None, None, -1, 16, 16, 16, 1, 0, 0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT
    st, msg = call("rg_copy_blocks", None, None, None, 0, 16, 16, 16, 1, 0, 0, None)
    assert st == _lib.RG_OK  # nothing to copy
    st, msg = call("rg_copy_blocks", None, None, None, 3, 16, 16, 16, 1, 0, 0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "null pointer" in msg
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    st, msg = call("rg_copy_blocks", p, p, p, 1, 32, 16, 32, 1, 0, 0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "stride smaller" in msg
    st, msg = call("rg_copy_blocks", p, p, p, 1, 24, 32, 32, 1, 0, 0, None)
    assert st == _lib.RG_ERR_NOT_SUPPORTED and "multiples of 16" in msg
    st, msg = call("rg_copy_blocks", p, p, p, 1, 32, 32, 32, 2, 0, 64, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "layer strides" in msg
    st, msg = call("rg_rms_norm", None, None, None, None, 1e-5, 4, 0, _lib.RG_DTYPE_BF16, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT
    st, msg = call("rg_rms_norm", None, None, None, None, 1e-5, 4, 64, _lib.RG_DTYPE_BF16, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "null pointer" in msg
    st, msg = call("rg_rms_norm", None, None, None, None, 1e-5, 0, 64, _lib.RG_DTYPE_BF16, None)
    assert st == _lib.RG_OK
    st, msg = call("rg_silu_and_mul", None, None, 70000, 64, _lib.RG_DTYPE_BF16, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT
    st, msg = call("rg_silu_and_mul", None, None, 2, 64, 7, None)
    assert st == _lib.RG_ERR_NOT_SUPPORTED
    st, msg = call("rg_qkv_rope_reshape_and_cache", p, 100, p, p, p, p, p, p, 32, 8, 64, 16, 4, _lib.RG_DTYPE_BF16,
                   0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "qkv_token_stride" in msg
    st, msg = call("rg_qkv_rope_reshape_and_cache", p, 3072, p, p, p, p, p, p, 30, 8, 64, 16, 4, _lib.RG_DTYPE_BF16,
                   0, None)
    assert st == _lib.RG_ERR_INVALID_ARGUMENT and "not a multiple" in msg


def test_workspace_queries():
    lib = railgun_amd.load_library()
    assert lib.rg_v2_workspace_bytes(8, 32, 64, 128) == 8 * 32 * 64 * 128 * 4 + 2 * 8 * 32 * 64 * 4
    assert lib.rg_v2_workspace_bytes(0, 32, 64, 128) == 0
    n = lib.rg_paged_attention_v1_workspace_bytes(64, 32, 8, 128, 16, 256)
    assert n > 0 and n % 256 == 0
    assert lib.rg_paged_attention_v1_workspace_bytes(64, 32, 7, 128, 16, 256) == 0  # bad GQA ratio


def test_rope_table_errors():
    lib = railgun_amd.load_library()
    t = np.zeros((4, 8), np.float32)
    assert lib.rg_rope_cos_sin_table(t.ctypes.data_as(_lib.f32p), 4, 7, 1e4) == _lib.RG_ERR_INVALID_ARGUMENT
    assert lib.rg_rope_cos_sin_table(t.ctypes.data_as(_lib.f32p), 4, 8, -1.0) == _lib.RG_ERR_INVALID_ARGUMENT
    assert lib.rg_rope_cos_sin_table(t.ctypes.data_as(_lib.f32p), 4, 8, 1e4) == _lib.RG_OK
    assert t[0, :4].tolist() == [1.0] * 4 and t[0, 4:].tolist() == [0.0] * 4


def test_op_rejects_host_tensors():
    class _NoKernels:  # the op checks its tensors before touching the launchers
        pass

    op = PagedAttentionOp(0.125, 4, 4, 64, 16, _NoKernels())
    q = torch.zeros((1, 4, 64))
    kc = torch.zeros((2, 4, 16, 64))
    bt = torch.zeros((1, 2), dtype=torch.int32)
    with pytest.raises(RailgunError, match="requires GPU tensors"):
        op.execute(q, kc, kc, bt, torch.ones(1, dtype=torch.int32), None, 1)
    bad = PagedAttentionOp(0.125, 4, 4, 66, 16, _NoKernels())
    with pytest.raises(RailgunError, match="multiple of 4"):
        bad.execute(q, kc, kc, bt, torch.ones(1, dtype=torch.int32), None, 1)


# ------------------------------------------------------------- batch packing --

def test_slot_mapping_follows_scheduler_formula():
    """slot = block_table[pos // bs] * bs + pos % bs, new token at pos = seq_len - 1
    (crates/vllm-scheduler/src/scheduler.rs:230-235, 258-263)."""
    w = wl.config2()
    slots = w.slot_mapping
    assert len(set(slots.tolist())) == w.batch  # distinct slots
    for s in range(w.batch):
        pos = int(w.context_lens[s]) - 1
        blk, off = divmod(int(slots[s]), w.block_size)
        assert blk == w.block_table[s, pos // w.block_size] and off == pos % w.block_size
    # prefill: every position of every sequence gets its own slot in its own blocks
    p = wl.config4()
    sl = p.slot_mapping
    assert len(sl) == p.num_tokens and len(set(sl.tolist())) == p.num_tokens
    cu = p.cu_seqlens
    for s in range(p.num_seqs):
        rows = sl[cu[s]:cu[s + 1]]
        assert set((rows // 16).tolist()) == set(p.block_table[s, :(p.seq_lens[s] + 15) // 16].tolist())
        np.testing.assert_array_equal(rows % 16, np.arange(p.seq_lens[s]) % 16)


def test_block_tables_are_padded_permutations():
    """Rows take distinct blocks from a shuffled pool and are 0-padded (engine.rs:217-226)."""
    for w in (wl.config1(), wl.config2(), wl.config3()):
        used = []
        for s in range(w.batch):
            n = (int(w.context_lens[s]) + w.block_size - 1) // w.block_size
            used += w.block_table[s, :n].tolist()
            assert (w.block_table[s, n:] == 0).all()
        assert len(set(used)) == len(used) and max(used) < w.num_blocks
    w = wl.config2()
    assert w.batch == 64 and w.context_lens.min() >= 512 and w.context_lens.max() <= 4096
    need = int(((w.context_lens + 15) // 16).sum())
    assert w.num_blocks == int(np.ceil(1.1 * need))
    p = wl.config4()
    assert p.num_seqs == 12 and p.seq_lens.min() >= 128 and p.seq_lens.max() <= 2048
    assert p.causal_flops() == 4 * 32 * 128 * int((p.seq_lens.astype(np.int64) * (p.seq_lens + 1) // 2).sum())


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stdout


def test_interleave_gate_up_layout():
    """interleave_gate_up puts gate rows 16j.. at rows 32j.. and up rows 16j.. at rows 32j + 16.."""
    import torch

    from railgun_amd.ops import interleave_gate_up
    inter, k = 48, 8
    w = torch.arange(2 * inter * k, dtype=torch.float32).view(2 * inter, k)
    il = interleave_gate_up(w)
    for j in range(inter // 16):
        assert torch.equal(il[32 * j:32 * j + 16], w[16 * j:16 * j + 16])
        assert torch.equal(il[32 * j + 16:32 * j + 32], w[inter + 16 * j:inter + 16 * j + 16])


def test_deinterleave_gate_up_inverts_the_layout():
    """deinterleave_gate_up undoes interleave_gate_up on the weight rows, and on the columns of
    a product: x @ interleaved^T, de-interleaved, is x @ w_gate_up^T exactly (a permutation of
    the same sums), which is what the model's separate MLP form relies on once the weight is
    held interleaved."""
    import torch

    from railgun_amd.ops import deinterleave_gate_up, interleave_gate_up
    g = torch.Generator().manual_seed(3)
    inter, k, rows = 64, 32, 5
    w = torch.randn(2 * inter, k, generator=g)
    il = interleave_gate_up(w)
    assert not torch.equal(il, w)
    assert torch.equal(deinterleave_gate_up(il.t()).t(), w)
    x = torch.randn(rows, k, generator=g)
    assert torch.equal(deinterleave_gate_up(x @ il.t()), x @ w.t())
