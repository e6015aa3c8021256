"""Gradient parity of the HIP backward against the CPU oracle.

Reference patterns: tests/test_kernels.py:109-127 (dq/dk/dv vs autograd
through the reference), :170-177 (finite grads), :180-202 (bf16 operands).
Tolerances: fp32 mode <= 1e-4 max-abs (north star); bf16 mode <= 5e-2
max-abs (north star) against the fp64 oracle on the bf16-rounded inputs, and
also within 1e-2 of the largest gradient with a mean error within 1e-2 of the
mean gradient.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import max_abs, needs_gpu
from oracle import dilution_oracle as orc

pytestmark = [pytest.mark.gpu, needs_gpu]


def _check_bf16(name, g, want):
    """A bf16-operand gradient against the fp64 oracle: the north-star 5e-2
    max-abs bound, within 1e-2 of the largest gradient, and a mean error
    within 1e-2 of the mean gradient (the measured errors are printed)."""
    w = torch.as_tensor(want).double()
    e = (g.double().cpu() - w).abs()
    err, wmax, merr, wmean = e.max().item(), w.abs().max().item(), e.mean().item(), w.abs().mean().item()
    print(f"{name}: max-abs {err:.3e} rel-to-max {err / wmax:.3e} mean-rel {merr / wmean:.3e}")
    assert err < 5e-2, f"{name} bf16 max abs err {err}"
    assert err < 1e-2 * wmax, f"{name} err {err} above 1e-2 of the largest gradient {wmax}"
    assert merr < 1e-2 * wmean, f"{name} mean err {merr} vs mean gradient {wmean}"


def _run(q, k, v, do, prec):
    from dilution import kernels

    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision=prec)
    out.backward(do.cuda())
    return out.detach(), [x.grad for x in xs]


@pytest.mark.parametrize("seq", [1, 8, 64, 257, 1024, 2049])
@pytest.mark.parametrize("prec", ["ieee", "tf32"])
def test_backward_fp32_matches_oracle(seq, prec):
    """fp32 operands ("ieee") and split bf16 operands ("tf32") both within the
    fp32-mode bound."""
    q, k, v, do = orc.make_inputs((2, 4, seq, 64), seed=seq, with_dout=True)
    out, grads = _run(q, k, v, do, prec)
    (dq, dk, dv), _ = orc.grads_closed_form_f64(q.numpy(), k.numpy(), v.numpy(), do.numpy())
    assert max_abs(out, orc.attention_f64(q, k, v)) < 1e-4
    for name, g, want in zip(("dq", "dk", "dv"), grads, (dq, dk, dv)):
        assert g.dtype == torch.float32
        assert torch.isfinite(g).all(), name
        err = max_abs(g, torch.from_numpy(want))
        assert err < 1e-4, f"{name} max abs err {err}"


@pytest.mark.parametrize("head_dim", [16, 32, 128])
@pytest.mark.parametrize("prec", ["ieee", "tf32"])
def test_backward_fp32_head_dims(head_dim, prec):
    q, k, v, do = orc.make_inputs((1, 2, 200, head_dim), seed=head_dim, with_dout=True)
    _, grads = _run(q, k, v, do, prec)
    want, _ = orc.grads_closed_form_f64(q.numpy(), k.numpy(), v.numpy(), do.numpy())
    for name, g, w in zip(("dq", "dk", "dv"), grads, want):
        assert max_abs(g, torch.from_numpy(w)) < 1e-4, name


@pytest.mark.parametrize("seq", [64, 257, 2048])
def test_backward_bf16_matches_oracle(seq):
    q, k, v, do = orc.make_inputs((2, 4, seq, 64), seed=11 + seq, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    out, grads = _run(q, k, v, do, "bf16")
    want, _ = orc.grads_closed_form_f64(*(t.double().numpy() for t in (q, k, v, do)))
    assert max_abs(out, orc.attention_f64(q, k, v)) < 2e-2
    for name, g, w in zip(("dq", "dk", "dv"), grads, want):
        assert g.dtype == torch.bfloat16
        assert torch.isfinite(g.float()).all(), name
        _check_bf16(name, g, w)


@pytest.mark.parametrize("head_dim", [16, 32, 128, 256])
def test_backward_bf16_head_dims(head_dim):
    # head_dim 16 and 32 run the parked row pass, 128 and 256 the register form
    q, k, v, do = orc.make_inputs((1, 2, 200, head_dim), seed=40 + head_dim, qk_scale=0.5,
                                  with_dout=True, dtype=torch.bfloat16)
    out, grads = _run(q, k, v, do, "bf16")
    want, _ = orc.grads_closed_form_f64(*(t.double().numpy() for t in (q, k, v, do)))
    assert max_abs(out, orc.attention_f64(q, k, v)) < 2e-2
    for name, g, w in zip(("dq", "dk", "dv"), grads, want):
        assert g.dtype == torch.bfloat16
        _check_bf16(name, g, w)


@pytest.mark.parametrize("seq", [4096, 4097])
def test_backward_bf16_long_rows(seq):
    # 128 and 129 row tiles: the LDS-parked row pass (three workgroups per CU)
    # over long key sweeps, against the oracle
    q, k, v, do = orc.make_inputs((1, 1, seq, 64), seed=seq, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    out, grads = _run(q, k, v, do, "bf16")
    want, _ = orc.grads_closed_form_f64(*(t.double().numpy() for t in (q, k, v, do)))
    for name, g, w in zip(("dq", "dk", "dv"), grads, want):
        assert torch.isfinite(g.float()).all(), name
        _check_bf16(name, g, w)


def test_backward_fp32_dout_with_bf16_inputs():
    """Under autocast the upstream gradient of the fp32 output is fp32 while
    q/k/v are bf16; gradients come back in the input dtype."""
    q, k, v, do = orc.make_inputs((1, 2, 300, 64), seed=5, qk_scale=0.5, with_dout=True)
    qb, kb, vb = (t.to(torch.bfloat16) for t in (q, k, v))
    _, grads = _run(qb, kb, vb, do, "bf16")
    want, _ = orc.grads_closed_form_f64(*(t.double().numpy() for t in (qb, kb, vb)), do.double().numpy())
    for name, g, w in zip(("dq", "dk", "dv"), grads, want):
        assert g.dtype == torch.bfloat16
        _check_bf16(name, g, w)


def test_backward_finite_and_shift_invariant():
    """out.sum().backward() (stride-0 upstream gradient); adding a constant to
    every key leaves the output unchanged, so sum_j dk_j = 0."""
    from dilution import kernels

    q, k, v = orc.make_inputs((1, 2, 96, 64), seed=1)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    kernels.dilution_attention(*xs, dot_precision="ieee").sum().backward()
    for x in xs:
        assert x.grad is not None and torch.isfinite(x.grad).all()
    assert xs[1].grad.sum(-2).abs().max().item() < 1e-4


def test_backward_grad_dtypes_follow_inputs():
    from dilution import kernels

    q, k, v = orc.make_inputs((1, 1, 70, 32), seed=2)
    xs = [q.cuda().half().requires_grad_(True), k.cuda().half().requires_grad_(True),
          v.cuda().half().requires_grad_(True)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(torch.ones_like(out))
    for x in xs:
        assert x.grad.dtype == torch.float16
        assert torch.isfinite(x.grad).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("head_dim", [32, 64, 128, 256])
def test_backward_converted_operands_match_oracle(dtype, head_dim):
    """fp32 or fp16 inputs with dot_precision="bf16": the backward converts q,
    k, v (and dO) to bf16 operands in its preparation launch (the z = 3 job
    picks V's copy).  Gradients against the closed-form oracle on the inputs
    as given, within the bf16 bound; gradients come back in the input dtype."""
    seq = 257
    q, k, v, do = orc.make_inputs((1, 3, seq, head_dim), seed=31 + head_dim, qk_scale=0.5,
                                  with_dout=True, dtype=dtype)
    out, grads = _run(q, k, v, do, "bf16")
    want, _ = orc.grads_closed_form_f64(*(t.double().numpy() for t in (q, k, v, do)))
    assert max_abs(out, orc.attention_f64(q, k, v)) < 5e-2
    for name, g, w in zip(("dq", "dk", "dv"), grads, want):
        assert g.dtype == dtype, name
        _check_bf16(name, g, w)


def test_backward_head_dim_256_many_key_tiles():
    """head_dim 256 over 1025 rows (33 key tiles, 33 row tiles: the suffix
    checkpoints, the diagonal peel and a ragged last tile) against the
    closed-form fp64 oracle at the bf16 bounds."""
    q, k, v, do = orc.make_inputs((1, 2, 1025, 256), seed=256, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    out, grads = _run(q, k, v, do, "bf16")
    want, _ = orc.grads_closed_form_f64(*(t.double().numpy() for t in (q, k, v, do)))
    assert max_abs(out, orc.attention_f64(q, k, v)) < 2e-2
    for name, g, w in zip(("dq", "dk", "dv"), grads, want):
        _check_bf16(name, g, w)
