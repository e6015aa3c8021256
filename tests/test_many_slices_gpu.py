"""More (batch * head) slices than a grid's y dimension holds (65535): the
kernels that put the slice on grid y are launched in batches of slices.
Forward, backward and the decode step over 65600 slices of a short sequence
against the fp64 oracle (fp32 tolerances)."""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import max_abs, needs_gpu
from oracle import dilution_oracle as orc

pytestmark = [pytest.mark.gpu, needs_gpu]

SHAPE = (4, 16400, 8, 16)          # n = 65600 slices


def test_forward_backward_past_grid_y_limit():
    from dilution import kernels

    q, k, v, do = orc.make_inputs(SHAPE, seed=31, with_dout=True)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="ieee")
    out.backward(do.cuda())
    assert max_abs(out.detach(), orc.attention_f64(q, k, v)) < 1e-4
    want, _ = orc.grads_closed_form_f64(q.numpy(), k.numpy(), v.numpy(), do.numpy())
    for name, x, w in zip(("dq", "dk", "dv"), xs, want):
        assert max_abs(x.grad, torch.from_numpy(w)) < 1e-4, name


def test_decode_past_grid_y_limit():
    from dilution import kernels

    q, k, v = orc.make_inputs(SHAPE, seed=32)
    t = SHAPE[2]
    _, aux = kernels.dilution_attention_forward(q[:, :, :t - 1].cuda(), k[:, :, :t - 1].cuda(),
                                                v[:, :, :t - 1].cuda(), return_aux=True)
    committed = torch.zeros(*SHAPE[:2], t, device="cuda")
    committed[:, :, :t - 1] = aux["committed_total"]
    y = kernels.dilution_decode_step(q[:, :, t - 1:].contiguous().cuda(), k.cuda(), v.cuda(), committed, t)
    assert max_abs(y[:, :, 0], orc.attention_f64(q, k, v)[:, :, t - 1]) < 1e-4
    assert max_abs(committed, orc.demand_totals(q, k)) < 1e-5
