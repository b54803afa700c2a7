"""Tolerances used by the parity tests.

Activations are compared with a relative error that has an RMS floor, so that
entries near zero do not turn an absolute rounding difference into an infinite
relative one:

    |actual - expected| <= rtol * max(|expected|, rms(expected))   elementwise

rtol is 2e-2 for bf16/fp16 and 1e-5 for fp32 (the project's parity contract).
Integer and index outputs are compared bit-exactly with `torch.equal`.
"""
from __future__ import annotations

import torch

RTOL = {torch.bfloat16: 2e-2, torch.float16: 2e-2, torch.float32: 1e-5}


def rel_error(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """max_i |a_i - e_i| / max(|e_i|, rms(e)), computed in float64 on the CPU."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    if a.shape != e.shape:
        raise AssertionError(f"shape mismatch {tuple(a.shape)} vs {tuple(e.shape)}")
    if e.numel() == 0:
        return 0.0
    if not torch.isfinite(a).all():
        return float("inf")
    rms = e.pow(2).mean().sqrt().clamp_min(1e-30)
    scale = torch.maximum(e.abs(), rms)
    return float(((a - e).abs() / scale).max())


def assert_close(actual: torch.Tensor, expected: torch.Tensor, dtype: torch.dtype | None = None,
                 rtol: float | None = None, what: str = "") -> float:
    rtol = rtol if rtol is not None else RTOL[dtype or expected.dtype]
    err = rel_error(actual, expected)
    assert err <= rtol, f"{what} relative error {err:.3e} exceeds {rtol:.1e}"
    return err
