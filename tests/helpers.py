"""Shared helpers of the test suite: seeded inputs, host<->device moves, tolerances."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as orc

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
# Attention tolerances: fp32 as the reference's own parity test (1e-4,
# crates/vllm-cuda/tests/test_paged_attention.rs:188); bf16/f16 outputs against the fp32
# oracle evaluated on the same bf16/f16-rounded inputs.
TOL = {"f32": dict(atol=1e-4, rtol=1e-4), "bf16": dict(atol=2e-2, rtol=1e-2), "f16": dict(atol=2e-2, rtol=1e-2)}


def normal(rng: np.random.Generator, shape, dt: str) -> np.ndarray:
    """N(0,1) values in the storage type of `dt` (bf16 as uint16 bits, rounded to nearest even)."""
    x = rng.standard_normal(size=shape, dtype=np.float32)
    return orc.from_f32(x, dt)


def to_dev(a: np.ndarray, dt: str, device) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if dt == "bf16":
        return torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)
    return torch.from_numpy(a).to(device)


def from_dev(t: torch.Tensor, dt: str) -> np.ndarray:
    if dt == "bf16":
        return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)
    return t.detach().cpu().numpy()


def dev_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def i32(a, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(device)


def assert_close(got: np.ndarray, want: np.ndarray, dt: str, what: str = "") -> None:
    np.testing.assert_allclose(got, want, err_msg=what, **TOL[dt])
