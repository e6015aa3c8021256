"""Shared helpers for the GPU parity tests: inputs are generated on the CPU RNG
(oracle.make_inputs), the oracle runs on the CPU, the kernels on cuda:0."""

from __future__ import annotations

import pytest
import torch

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X GPU")


def to_gpu(*ts, dtype=None):
    out = []
    for t in ts:
        t = t.to("cuda")
        out.append(t.to(dtype) if dtype is not None else t)
    return out


def max_abs(a, b) -> float:
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def mean_rel(a, b) -> float:
    a = a.double().cpu()
    b = b.double().cpu()
    return ((a - b).abs().mean() / b.abs().mean().clamp_min(1e-30)).item()
