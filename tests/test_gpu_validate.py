"""The opt-in index checks (rg_validate_block_tables, rg_validate_slot_mapping): the decode and
cache kernels trust their indices, as the reference's do; these entries find the first bad one.
The planted bad values are handed to the checks only, never to a kernel that would use them."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from railgun_amd import _lib
from railgun_amd import workloads as wl
from railgun_amd.ops import RailgunError

pytestmark = pytest.mark.gpu


def _tables(device, ctx, bs, nb, mb, seed=3):
    rng = np.random.default_rng(seed)
    bt = wl.assign_blocks(np.asarray(ctx, np.int32), bs, nb, mb, rng)
    return torch.from_numpy(bt).to(device), torch.tensor(ctx, dtype=torch.int32, device=device)


def test_valid_tables_and_slots_pass(device, kernels):
    ctx = [0, 1, 16, 17, 300, 511]
    bt, cl = _tables(device, ctx, 16, 200, 32)
    kernels.validate_block_tables(bt, cl, 16, 200)
    slots = torch.tensor([-1, 0, 5, 3199, -7], dtype=torch.int32, device=device)   # negative: padding
    kernels.validate_slot_mapping(slots, 200 * 16)


def test_bad_block_number_is_named(device, kernels):
    ctx = [40, 300, 77]
    bt, cl = _tables(device, ctx, 16, 100, 32)
    bad = bt.clone()
    bad[1, 7] = 100                     # one past the pool
    bad[2, 3] = -2
    with pytest.raises(RailgunError) as e:
        kernels.validate_block_tables(bad, cl, 16, 100)
    assert e.value.code == _lib.RG_ERR_INVALID_ARGUMENT
    assert "block_table[1][7] = 100" in e.value.message      # the first bad entry in (seq, index) order
    ok = bt.clone()
    ok[1, 25] = 10_000                  # past the entries context 300 uses (19): never read
    kernels.validate_block_tables(ok, cl, 16, 100)


def test_bad_context_length_is_named(device, kernels):
    bt, cl = _tables(device, [40, 300], 16, 100, 32)
    for v in (32 * 16 + 1, -1):
        bad = cl.clone()
        bad[1] = v
        with pytest.raises(RailgunError) as e:
            kernels.validate_block_tables(bt, bad, 16, 100)
        assert f"context_lens[1] = {v}" in e.value.message


def test_bad_slot_is_named(device, kernels):
    slots = torch.arange(0, 5000, dtype=torch.int32, device=device)
    slots[4321] = 3200
    slots[4999] = 99_999
    with pytest.raises(RailgunError) as e:
        kernels.validate_slot_mapping(slots, 200 * 16)
    assert "slot_mapping[3200] = 3200" in e.value.message    # slots 3200.. are all past the pool
