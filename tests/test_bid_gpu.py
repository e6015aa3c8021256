"""Bid and share variants (dilution.kernels_bid) on the HIP kernels against
the fp64 oracle.

Reference patterns: tests/test_kernels.py:276-450 (forward and backward of
every bid with and without the share step, the softmax path equal to the
production operator, decode rows of every bid, the no-cumsum softmax equal to
plain attention, the exclusive share's identity collapse and first row).
Tolerances: fp32 forward 1e-4 max-abs and demand totals 1e-5 (the production
bounds; relu2 1e-3, the reference's bound for every bid forward: a diagonal key
with a tiny positive affinity bids relu(a)^2 ~ eps and, with no demand yet,
takes a share p / (p + eps) that the fp32 score moves by ~1e-3); gradients within the reference's relative bound (2e-3 of the
largest gradient, 5e-3 for relu2, kernels_bid's own test bounds); bf16
forward 2e-2 max-abs against the oracle on the bf16-rounded inputs.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import max_abs, needs_gpu
from oracle import dilution_oracle as orc

pytestmark = [pytest.mark.gpu, needs_gpu]

SHIFT = 3.0


def _inputs(seq, seed, shape=(2, 4)):
    return orc.make_inputs((*shape, seq, 64), seed=seed)


@pytest.mark.parametrize("bid", orc.BIDS)
@pytest.mark.parametrize("share", orc.SHARES, ids=str)
@pytest.mark.parametrize("seq", [64, 257])
def test_variant_forward_matches_oracle(bid, share, seq):
    from dilution import kernels_bid as kb

    q, k, v = _inputs(seq, seed=seq)
    got, aux = kb.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), bid=bid,
                                             share_cumsum=share, shift=SHIFT, return_aux=True)
    assert torch.isfinite(got).all()
    bound = 1e-3 if bid == "relu2" else 1e-4
    assert max_abs(got, orc.variant_attention_f64(q, k, v, bid, share, SHIFT)) < bound
    totals = orc.variant_demand_totals(q, k, bid, SHIFT)
    assert max_abs(aux["committed_total"], totals) < 1e-5 * max(1.0, totals.abs().max().item())


@pytest.mark.parametrize("bid", orc.BIDS)
@pytest.mark.parametrize("share", [True, False], ids=str)
@pytest.mark.parametrize("seq", [64, 257])
def test_variant_backward_matches_autograd(bid, share, seq):
    from dilution import kernels_bid as kb

    q, k, v, do = orc.make_inputs((2, 4, seq, 64), seed=100 + seq, with_dout=True)
    ref = [x.double().requires_grad_(True) for x in (q, k, v)]
    orc.variant_attention_f64(*ref, bid, share, SHIFT).backward(do.double())
    xs = [x.cuda().requires_grad_(True) for x in (q, k, v)]
    kb.dilution_attention(*xs, dot_precision="ieee", bid=bid, share_cumsum=share,
                          shift=SHIFT).backward(do.cuda())
    bound = 5e-3 if bid == "relu2" else 2e-3
    for name, r, x in zip(("dq", "dk", "dv"), ref, xs):
        scale = r.grad.abs().max().item() + 1e-6
        rel = max_abs(x.grad, r.grad) / scale
        assert rel < bound, f"{bid} {name} relative error {rel}"


@pytest.mark.parametrize("bid", orc.BIDS)
def test_variant_backward_bf16(bid):
    """bf16 operands (the ablation LM's training mode): gradients against the
    fp64 autograd oracle on the bf16-rounded inputs, relative to the largest
    gradient as in the fp32 variant test (minshift's gradients carry the
    1/eps-scale terms of a zero bid on an undemanded key): 1e-2, relu2 2.5e-2
    (the reference's 2.5x relu2 relaxation)."""
    from dilution import kernels_bid as kb

    q, k, v, do = (x.to(torch.bfloat16) for x in orc.make_inputs((1, 4, 200, 64), seed=41, qk_scale=0.5,
                                                                  with_dout=True))
    ref = [x.double().requires_grad_(True) for x in (q, k, v)]
    orc.variant_attention_f64(*ref, bid, True, SHIFT).backward(do.double())
    xs = [x.cuda().requires_grad_(True) for x in (q, k, v)]
    kb.dilution_attention(*xs, dot_precision="bf16", bid=bid, shift=SHIFT).backward(do.cuda())
    bound = 2.5e-2 if bid == "relu2" else 1e-2
    for name, r, x in zip(("dq", "dk", "dv"), ref, xs):
        assert x.grad.dtype == torch.bfloat16
        rel = max_abs(x.grad, r.grad) / (r.grad.abs().max().item() + 1e-6)
        assert rel < bound, f"{bid} {name} relative error {rel}"


@pytest.mark.parametrize("bid", orc.BIDS)
@pytest.mark.parametrize("share", [False, "exclusive"], ids=str)
def test_variant_backward_bf16_other_shares(bid, share):
    """bf16 operands at head_dim 64 (the one-pass backward) with no share step
    (dq, dk, dv) and with the exclusive share (dv only: its dq / dk cancel
    1e9-scale terms, see below), against the fp64 autograd oracle on the
    bf16-rounded inputs, relative to the largest gradient: 1e-2, relu2 2.5e-2."""
    from dilution import kernels_bid as kb

    q, k, v, do = (x.to(torch.bfloat16) for x in orc.make_inputs((1, 4, 200, 64), seed=43, qk_scale=0.5,
                                                                  with_dout=True))
    ref = [x.double().requires_grad_(True) for x in (q, k, v)]
    orc.variant_attention_f64(*ref, bid, share, SHIFT).backward(do.double())
    xs = [x.cuda().requires_grad_(True) for x in (q, k, v)]
    kb.dilution_attention(*xs, dot_precision="bf16", bid=bid, share_cumsum=share,
                          shift=SHIFT).backward(do.cuda())
    bound = 2.5e-2 if bid == "relu2" else 1e-2
    checked = ("dq", "dk", "dv") if share is False else ("dv",)
    for name, r, x in zip(("dq", "dk", "dv"), ref, xs):
        if name not in checked:
            continue
        rel = max_abs(x.grad, r.grad) / (r.grad.abs().max().item() + 1e-6)
        assert rel < bound, f"{bid} {share} {name} relative error {rel}"


@pytest.mark.parametrize("bid", ["softmax", "relu", "sigmoid"])
def test_variant_exclusive_backward_dv(bid):
    """The exclusive share's dq/dk are fp32 noise on cancelling 1e9-scale terms
    (the operator's property, kernels_bid tests note); dv is exact."""
    from dilution import kernels_bid as kb

    q, k, v, do = orc.make_inputs((1, 2, 96, 64), seed=7, with_dout=True)
    ref = [x.double().requires_grad_(True) for x in (q, k, v)]
    orc.variant_attention_f64(*ref, bid, "exclusive").backward(do.double())
    xs = [x.cuda().requires_grad_(True) for x in (q, k, v)]
    kb.dilution_attention(*xs, dot_precision="ieee", bid=bid, share_cumsum="exclusive").backward(do.cuda())
    assert max_abs(xs[2].grad, ref[2].grad) / (ref[2].grad.abs().max().item() + 1e-9) < 2e-3


@pytest.mark.parametrize("bid", orc.BIDS)
def test_variant_forward_bf16(bid):
    from dilution import kernels_bid as kb

    q, k, v = (x.to(torch.bfloat16) for x in _inputs(200, seed=11))
    got = kb.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), dot_precision="bf16", bid=bid,
                                        shift=SHIFT)
    assert max_abs(got, orc.variant_attention_f64(q, k, v, bid, True, SHIFT)) < 2e-2


def test_softmax_dilution_variant_is_the_production_operator():
    from dilution import kernels
    from dilution import kernels_bid as kb

    q, k, v = (x.cuda() for x in _inputs(200, seed=3))
    a = kernels.dilution_attention_forward(q, k, v)
    b = kb.dilution_attention_forward(q, k, v, bid="softmax", share_cumsum=True)
    assert torch.equal(a, b)


def test_no_share_softmax_is_plain_causal_attention():
    from dilution import kernels_bid as kb

    q, k, v = _inputs(200, seed=12)
    got = kb.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), bid="softmax", share_cumsum=False)
    s = torch.matmul(q.double(), k.double().transpose(-2, -1)) / 8.0
    causal = torch.ones(200, 200, dtype=torch.bool).tril()
    want = torch.matmul(torch.softmax(s.masked_fill(~causal, -float("inf")), -1), v.double())
    assert max_abs(got, want) < 1e-4


def test_exclusive_share_collapses_to_the_identity():
    from dilution import kernels_bid as kb

    q, k, v = _inputs(257, seed=13, shape=(1, 2))
    got = kb.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), share_cumsum="exclusive")
    assert max_abs(got, v) < 1e-3
    assert max_abs(got[:, :, 0], v[:, :, 0]) < 1e-6


@pytest.mark.parametrize("bid", orc.BIDS)
@pytest.mark.parametrize("share", orc.SHARES, ids=str)
def test_variant_decode_matches_full_rows(bid, share):
    """Prefix forward -> committed_total, then one decode step per token: each
    row equals the full-sequence row, the demand the full column totals."""
    from dilution import kernels_bid as kb

    b, h, t, prefix = 2, 3, 70, 62
    q, k, v = orc.make_inputs((b, h, t, 64), seed=17)
    full = orc.variant_attention_f64(q, k, v, bid, share, SHIFT)
    qg, kg, vg = (x.cuda() for x in (q, k, v))
    _, aux = kb.dilution_attention_forward(qg[:, :, :prefix], kg[:, :, :prefix], vg[:, :, :prefix],
                                           return_aux=True, bid=bid, share_cumsum=share, shift=SHIFT)
    committed = torch.zeros(b, h, t, device="cuda")
    committed[:, :, :prefix] = aux["committed_total"]
    for i in range(prefix, t):
        y = kb.dilution_decode_step(qg[:, :, i:i + 1].contiguous(), kg, vg, committed, i + 1, bid=bid,
                                    share_cumsum=share, shift=SHIFT)
        assert max_abs(y[:, :, 0], full[:, :, i]) < 1e-4, i
    totals = orc.variant_demand_totals(q, k, bid, SHIFT)
    assert max_abs(committed, totals) < 1e-5 * max(1.0, totals.abs().max().item())


_OTHER_DIM_CASES = [("relu", True), ("relu2", False), ("minshift", True), ("softplus", "exclusive"),
                    ("sigmoid", True), ("expshift", False), ("sigshift", "exclusive"), ("softmax", "exclusive")]


@pytest.mark.parametrize("head_dim", [16, 32, 128])
@pytest.mark.parametrize("bid,share", _OTHER_DIM_CASES, ids=lambda x: str(x))
def test_variant_other_head_dims(bid, share, head_dim):
    """Every variant is built for the production head dims: at 16, 32 and 128
    (ragged T = 97), the fp32 forward against the fp64 oracle (1e-4, relu2
    1e-3) with its demand totals (1e-5 relative), the gradients against fp64
    autograd (2e-3 of the largest, relu2 5e-3; only dv under the exclusive
    share, whose dq / dk cancel 1e9-scale terms), the bf16 forward (2e-2) and
    a decode step of the last row (1e-4)."""
    from dilution import kernels_bid as kb

    t = 97
    q, k, v, do = orc.make_inputs((1, 3, t, head_dim), seed=500 + head_dim, with_dout=True)
    kw = dict(bid=bid, share_cumsum=share, shift=SHIFT)
    want = orc.variant_attention_f64(q, k, v, bid, share, SHIFT)
    got, aux = kb.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), return_aux=True, **kw)
    bound = 1e-3 if bid == "relu2" else 1e-4
    assert max_abs(got, want) < bound
    totals = orc.variant_demand_totals(q, k, bid, SHIFT)
    assert max_abs(aux["committed_total"], totals) < 1e-5 * max(1.0, totals.abs().max().item())

    ref = [x.double().requires_grad_(True) for x in (q, k, v)]
    orc.variant_attention_f64(*ref, bid, share, SHIFT).backward(do.double())
    xs = [x.cuda().requires_grad_(True) for x in (q, k, v)]
    kb.dilution_attention(*xs, dot_precision="ieee", **kw).backward(do.cuda())
    gbound = 5e-3 if bid == "relu2" else 2e-3
    for name, r, x in zip(("dq", "dk", "dv"), ref, xs):
        if share == "exclusive" and name != "dv":
            continue
        rel = max_abs(x.grad, r.grad) / (r.grad.abs().max().item() + 1e-6)
        assert rel < gbound, f"{bid} {share} d{head_dim} {name} relative error {rel}"

    qb, kb16, vb = (x.to(torch.bfloat16) for x in (q, k, v))
    gotb = kb.dilution_attention_forward(qb.cuda(), kb16.cuda(), vb.cuda(), dot_precision="bf16", **kw)
    assert max_abs(gotb, orc.variant_attention_f64(qb, kb16, vb, bid, share, SHIFT)) < 2e-2

    committed = torch.zeros(1, 3, t, device="cuda")
    _, auxp = kb.dilution_attention_forward(q[:, :, :t - 1].cuda(), k[:, :, :t - 1].cuda(),
                                            v[:, :, :t - 1].cuda(), return_aux=True, **kw)
    committed[:, :, :t - 1] = auxp["committed_total"]
    y = kb.dilution_decode_step(q[:, :, t - 1:].contiguous().cuda(), k.cuda(), v.cuda(), committed, t, **kw)
    assert max_abs(y[:, :, 0], want[:, :, t - 1]) < 1e-4


def test_variant_argument_errors():
    from dilution import kernels_bid as kb

    q = torch.zeros(1, 1, 8, 48, device="cuda")
    with pytest.raises(ValueError):
        kb.dilution_attention_forward(q, q, q, bid="relu")          # head_dim 48: not built
    q64 = torch.zeros(1, 1, 8, 64, device="cuda")
    with pytest.raises(ValueError):
        kb.dilution_attention_forward(q64, q64, q64, bid="tanh")
    with pytest.raises(ValueError):
        kb.dilution_attention_forward(q64, q64, q64, bid="expshift", shift=0.0)
