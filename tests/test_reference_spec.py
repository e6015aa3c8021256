"""The public specification function ``dilution.kernels.dilution_attention_reference``
(the reference's kernels.py:40-68, exported because callers use it) against
the pinned CPU oracle: it is the spec the kernels are held to, so it is
itself held to the oracle's pins (fp64 loops through attention_f64, the
harmonic closed form)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dilution_oracle as orc


@pytest.mark.parametrize("t,d", [(1, 16), (33, 16), (200, 64)])
def test_public_reference_matches_oracle(t, d):
    from dilution import kernels

    q, k, v = orc.make_inputs((2, 3, t, d), seed=t + d)
    got = kernels.dilution_attention_reference(q, k, v)
    assert got.dtype == torch.float32 and got.shape == q.shape
    assert (got.double() - orc.attention_f64(q, k, v)).abs().max().item() < 2e-5
    # bf16 inputs are upcast, as in the reference
    qb, kb, vb = (x.to(torch.bfloat16) for x in (q, k, v))
    got_b = kernels.dilution_attention_reference(qb, kb, vb)
    assert (got_b.double() - orc.attention_f64(qb, kb, vb)).abs().max().item() < 2e-5


def test_public_reference_harmonic_closed_form():
    from dilution import kernels

    t = 120
    g = torch.Generator().manual_seed(3)
    v = torch.randn(1, 2, t, 8, generator=g)
    k = torch.randn(1, 2, t, 8, generator=g)
    want, _ = orc.harmonic_closed_form(t, v.double().numpy())
    got = kernels.dilution_attention_reference(torch.zeros_like(v), k, v)
    assert np.abs(got.double().numpy() - want).max() < 1e-5
