"""Pin the CPU oracle (oracle/dilution_oracle.py) before trusting it.

Each check compares the oracle against something that is not a retyping of its
own formula: float64 brute-force loops, the q = 0 harmonic-number closed form,
finite differences (gradcheck), library routines (torch.softmax), causality and
shift invariance.  Planted mistakes in copies of the oracle formula must fail at
least one of these pins.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dilution_oracle as orc


def _rand(shape, seed, scale=1.0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(*shape, generator=g) * s).to(dtype) for s in (scale, scale, 1.0))


@pytest.mark.parametrize("t", [1, 2, 7, 33])
@pytest.mark.parametrize("d", [4, 16])
def test_fp32_restatement_matches_fp64_loops(t, d):
    q, k, v = _rand((2, 3, t, d), seed=100 + t + d)
    ref = orc.attention_loops_f64(q.numpy(), k.numpy(), v.numpy())
    got32 = orc.attention_fp32(q.float(), k.float(), v.float()).double().numpy()
    got64 = orc.attention_f64(q, k, v).numpy()
    assert np.abs(got64 - ref).max() < 1e-12
    assert np.abs(got32 - ref).max() < 2e-5


@pytest.mark.parametrize("t", [1, 5, 64, 300])
def test_harmonic_closed_form(t):
    """q = 0 makes every bid 1/(i+1); the operator reduces to harmonic numbers."""
    g = torch.Generator().manual_seed(t)
    v = torch.randn(1, 2, t, 8, generator=g, dtype=torch.float64)
    q = torch.zeros_like(v)
    k = torch.randn(1, 2, t, 8, generator=g, dtype=torch.float64)
    out_cf, totals_cf = orc.harmonic_closed_form(t, v.numpy())
    assert np.abs(orc.attention_f64(q, k, v).numpy() - out_cf).max() < 1e-12
    assert np.abs(orc.attention_fp32(q.float(), k.float(), v.float()).double().numpy() - out_cf).max() < 1e-5
    if t <= 64:
        assert np.abs(orc.attention_loops_f64(q, k, v) - out_cf).max() < 1e-12
    tot = orc.demand_totals(q, k).numpy()
    assert np.abs(tot - totals_cf).max() < 1e-12


@pytest.mark.parametrize("t,block", [(1, 4), (300, 64), (257, 100), (130, 512)])
def test_blocked_restatement_matches_fp64(t, block):
    """The row-blocked slice oracle (the full-size checker) against the dense
    fp64 formula, at ragged lengths and block sizes."""
    q, k, v = _rand((1, 1, t, 16), seed=400 + t)
    out, tot = orc.attention_blocked_f64(q[0, 0], k[0, 0], v[0, 0], block=block)
    assert np.abs(out - orc.attention_f64(q, k, v).numpy()[0, 0]).max() < 1e-12
    assert np.abs(tot - orc.demand_totals(q, k).numpy()[0, 0]).max() < 1e-10


def test_blocked_restatement_harmonic_closed_form():
    t = 3000
    g = torch.Generator().manual_seed(5)
    v = torch.randn(t, 8, generator=g, dtype=torch.float64)
    k = torch.randn(t, 8, generator=g, dtype=torch.float64)
    out_cf, totals_cf = orc.harmonic_closed_form(t, v.numpy())
    out, tot = orc.attention_blocked_f64(np.zeros((t, 8)), k, v, block=512)
    assert np.abs(out - out_cf).max() < 1e-10
    assert np.abs(tot - totals_cf).max() < 1e-10


def test_single_row_returns_first_value():
    """T = 1: share = p/(p+eps) ~ 1, so out_0 = v_0 up to eps."""
    q, k, v = _rand((1, 1, 1, 32), seed=3)
    out = orc.attention_f64(q, k, v)
    assert torch.allclose(out, v, atol=1e-8)


def test_causality_bit_identical_prefix():
    q, k, v = _rand((1, 2, 40, 16), seed=4, dtype=torch.float32)
    out = orc.attention_fp32(q, k, v)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[..., 25:, :] += 3.0
    k2[..., 25:, :] -= 2.0
    v2[..., 25:, :] *= 5.0
    out2 = orc.attention_fp32(q2, k2, v2)
    assert torch.equal(out[..., :25, :], out2[..., :25, :])
    assert not torch.equal(out[..., 25:, :], out2[..., 25:, :])


def test_shift_invariance_and_dk_sums_to_zero():
    q, k, v = _rand((1, 2, 24, 8), seed=5)
    out = orc.attention_f64(q, k, v)
    shifted = orc.attention_f64(q, k + torch.randn(1, 2, 1, 8, dtype=torch.float64), v)
    assert torch.allclose(out, shifted, atol=1e-12)
    do = torch.randn_like(q)
    dq, dk, dv = orc.grads_autograd(q, k, v, do)
    assert dk.sum(-2).abs().max().item() < 1e-12
    # rows of A sum to 1 - O(eps): sum_j dv_j == sum_i dO_i (to ~1e-8)
    assert torch.allclose(dv.sum(-2), do.sum(-2), atol=1e-6)


def test_gradcheck_of_restatement():
    q, k, v = _rand((1, 1, 6, 3), seed=6)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v)]
    assert torch.autograd.gradcheck(orc.attention_f64, xs, eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("t", [1, 9, 70])
def test_closed_form_backward_matches_autograd(t):
    q, k, v = _rand((2, 2, t, 16), seed=7 + t)
    do = torch.randn(2, 2, t, 16, dtype=torch.float64, generator=torch.Generator().manual_seed(t))
    ref = orc.grads_autograd(q, k, v, do)
    got, inter = orc.grads_closed_form_f64(q.numpy(), k.numpy(), v.numpy(), do.numpy())
    for r, g in zip(ref, got):
        assert np.abs(r.numpy() - g).max() < 1e-9
    assert np.abs(inter["out"] - orc.attention_f64(q, k, v).numpy()).max() < 1e-12


@pytest.mark.parametrize("t,block", [(1, 4), (33, 7), (100, 32), (257, 64), (130, 512)])
def test_blocked_backward_matches_closed_form(t, block):
    """The row-blocked backward (the full-length gradient checker) against the
    dense decomposition, itself pinned to autograd above, at ragged lengths
    and block sizes that do and do not divide T."""
    q, k, v = _rand((1, 1, t, 16), seed=500 + t, scale=0.7)
    do = torch.randn(t, 16, dtype=torch.float64, generator=torch.Generator().manual_seed(t))
    want, inter_w = orc.grads_closed_form_f64(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), do.numpy())
    got, inter = orc.grads_blocked_f64(q[0, 0], k[0, 0], v[0, 0], do, block=block)
    for w, g in zip(want, got):
        assert np.abs(g.numpy() - w).max() < 1e-10
    assert np.abs(inter["ghat"].numpy() - inter_w["ghat"]).max() < 1e-10
    assert np.abs(inter["out"].numpy() - inter_w["out"]).max() < 1e-12
    assert np.abs(inter["totals"].numpy() - orc.demand_totals(q, k)[0, 0].numpy()).max() < 1e-10
    # adding a constant to every key leaves the output unchanged: sum_j dk_j = 0
    assert got[1].sum(0).abs().max() < 1e-10 * (1.0 + got[1].abs().sum())


def test_blocked_backward_matches_autograd_directly():
    q, k, v = _rand((1, 1, 50, 8), seed=77)
    do = torch.randn(1, 1, 50, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(78))
    ref = orc.grads_autograd(q, k, v, do)
    got, _ = orc.grads_blocked_f64(q[0, 0], k[0, 0], v[0, 0], do[0, 0], block=16)
    for r, g in zip(ref, got):
        assert (r[0, 0] - g).abs().max() < 1e-10


@pytest.mark.parametrize("mutant", ["no_suffix_carry", "no_demand_carry"])
def test_blocked_backward_planted_mistakes_fail(mutant):
    q, k, v = _rand((1, 1, 90, 8), seed=79, scale=0.7)
    do = torch.randn(90, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(80))
    want, _ = orc.grads_closed_form_f64(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), do.numpy())
    got, _ = orc.grads_blocked_f64(q[0, 0], k[0, 0], v[0, 0], do, block=32, mutant=mutant)
    err = max(np.abs(g.numpy() - w).max() for w, g in zip(want, got))
    assert err > 1e-3, (mutant, err)


def test_row_stats_and_pk_match_library_softmax():
    q, k, v = _rand((1, 2, 50, 16), seed=8)
    rmax, rden = orc.row_stats(q, k)
    a = torch.matmul(q, k.transpose(-1, -2)) / 4.0
    causal = torch.ones(50, 50, dtype=torch.bool).tril()
    p = torch.softmax(a.masked_fill(~causal, -math.inf), -1)
    p2 = torch.exp2(a * orc.LOG2E - rmax[..., None]).masked_fill(~causal, 0) / rden[..., None]
    assert torch.allclose(p, p2, atol=1e-14)
    assert torch.allclose(orc.pk(q, k), (p @ k) / 4.0, atol=1e-14)


@pytest.mark.parametrize("block", [32, 64])
def test_carry_checkpoints_match_loop_sums(block):
    q, k, _ = _rand((1, 1, 150, 8), seed=9)
    p = orc.bids(q, k)[0, 0].numpy()
    carry = orc.carry_checkpoints(q, k, block)[0, 0].numpy()
    for rb in range(carry.shape[0]):
        want = np.zeros(150)
        for i in range(rb * block):
            want += p[i]
        assert np.abs(carry[rb] - want).max() < 1e-12
        assert (carry[rb, rb * block:] == 0).all()


def test_decode_chain_matches_full_rows_and_column_sums():
    q, k, v = _rand((2, 3, 45, 16), seed=10)
    full = orc.attention_loops_f64(q, k, v)
    prefix = 30
    cap = 48
    com = torch.zeros(2, 3, cap, dtype=torch.float64)
    com[..., :prefix] = orc.demand_totals(q[..., :prefix, :], k[..., :prefix, :])
    kc = torch.zeros(2, 3, cap, 16, dtype=torch.float64)
    vc = torch.zeros_like(kc)
    kc[..., :45, :] = k
    vc[..., :45, :] = v
    for t in range(prefix, 45):
        out, com = orc.decode_step(q[..., t:t + 1, :], kc, vc, com, t + 1)
        assert np.abs(out[..., 0, :].numpy() - full[..., t, :]).max() < 1e-12
    assert torch.allclose(com[..., :45], orc.demand_totals(q, k), atol=1e-12)
    assert (com[..., 45:] == 0).all()


def test_prefill_chunks_match_full_forward():
    q, k, v = _rand((1, 2, 100, 8), seed=11)
    full = orc.attention_f64(q, k, v).numpy()
    demand = torch.zeros(1, 2, 100, dtype=torch.float64)
    for start in range(0, 100, 32):
        stop = min(start + 32, 100)
        out, dem = orc.prefill_chunk(q[..., start:stop, :], k[..., :stop, :], v[..., :stop, :],
                                     demand, start)
        assert np.abs(out.numpy() - full[..., start:stop, :]).max() < 1e-12
        demand = torch.zeros(1, 2, 100, dtype=torch.float64)
        demand[..., :stop] = dem
    assert torch.allclose(demand, orc.demand_totals(q, k), atol=1e-12)


# --- planted mistakes: each mutant of the formula must fail a pin -------------

def _mutant(kind):
    def fwd(q, k, v):
        t, d = q.shape[-2], q.shape[-1]
        scale = 1.0 if kind == "no_scale" else 1.0 / math.sqrt(d)
        a = torch.matmul(q, k.transpose(-2, -1)) * scale
        causal = torch.ones(t, t, dtype=torch.bool).tril()
        p = torch.softmax(a.masked_fill(~causal, -math.inf), -1)
        if kind == "key_axis_cumsum":
            c = torch.cumsum(p, -1) - p
        elif kind == "inclusive_twice":
            c = torch.cumsum(p, -2)
        else:
            c = torch.cumsum(p, -2) - p
        den = c + EPS if kind == "exclusive_denominator" else c + p + EPS
        share = p / den
        if kind == "no_renormalise":
            a_ = share
        else:
            a_ = share / (share.sum(-1, keepdim=True) + EPS)
        return a_ @ v
    EPS = orc.EPS
    return fwd


@pytest.mark.parametrize("kind", ["no_scale", "key_axis_cumsum", "inclusive_twice",
                                  "exclusive_denominator", "no_renormalise"])
def test_planted_mistakes_fail_a_pin(kind):
    fwd = _mutant(kind)
    q, k, v = _rand((1, 2, 20, 8), seed=12)
    loops = orc.attention_loops_f64(q, k, v)
    err_loops = np.abs(fwd(q, k, v).numpy() - loops).max()
    z = torch.zeros_like(q)
    cf, _ = orc.harmonic_closed_form(20, v.numpy())
    err_cf = np.abs(fwd(z, k, v).numpy() - cf).max()
    assert max(err_loops, err_cf) > 1e-3, (kind, err_loops, err_cf)


# ---------------------------------------------------------------------------
# bid / share variants (kernels_bid.py)

UNIFORM_AT_ZERO = ("softmax", "relu", "relu2", "softplus", "minshift")   # q = 0 -> p = 1/(i+1)


@pytest.mark.parametrize("bid", orc.BIDS)
@pytest.mark.parametrize("share", orc.SHARES, ids=str)
def test_variant_restatement_matches_scalar_loops(bid, share):
    q, k, v = orc.make_inputs((1, 1, 13, 8), seed=5)
    got = orc.variant_attention_f64(q, k, v, bid, share, 3.0)[0, 0].numpy()
    want, demand = orc.variant_attention_loops(q[0, 0], k[0, 0], v[0, 0], bid, share, 3.0)
    assert np.abs(got - want).max() < 1e-12
    assert np.abs(orc.variant_demand_totals(q, k, bid, 3.0)[0, 0].numpy() - demand).max() < 1e-12


@pytest.mark.parametrize("bid", UNIFORM_AT_ZERO)
def test_variant_uniform_bids_closed_forms(bid):
    """q = 0: the uniform bid 1/(i+1) (softmax, softplus directly; relu, relu2,
    minshift through their empty-row rule) gives the harmonic closed form with
    the dilution share and the window mean with no share step."""
    t = 24
    _, k, v = orc.make_inputs((1, 1, t, 8), seed=6)
    q = torch.zeros_like(k)
    want, totals = orc.harmonic_closed_form(t, v[0, 0])
    got = orc.variant_attention_f64(q, k, v, bid, True)[0, 0].numpy()
    assert np.abs(got - want).max() < 1e-12
    assert np.abs(orc.variant_demand_totals(q, k, bid)[0, 0].numpy() - totals).max() < 1e-12
    mean = np.cumsum(v[0, 0].double().numpy(), 0) / np.arange(1, t + 1)[:, None]
    assert np.abs(orc.variant_attention_f64(q, k, v, bid, False)[0, 0].numpy() - mean).max() < 1e-12


@pytest.mark.parametrize("bid,c0", [("sigmoid", 0.5), ("sigshift", 1.0 / 4.0), ("expshift", 1.0 / 3.0)])
def test_variant_constant_bids_closed_form(bid, c0):
    """q = 0: the elementwise bids are a constant c0, the demand of key j at
    row i is c0 (i - j), the dilution share is 1/(i - j + 1) (eps aside), so
    row i averages v_j with weights 1/(i - j + 1) / H_{i+1}."""
    t = 20
    shift = 3.0 if bid != "sigmoid" else 1.0
    if bid == "sigshift":
        shift = 3.0                                    # 1 / (1 + 3)
    _, k, v = orc.make_inputs((1, 1, t, 8), seed=7)
    q = torch.zeros_like(k)
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    w = np.where(j <= i, 1.0 / (i - j + 1), 0.0)
    want = (w / w.sum(-1, keepdims=True)) @ v[0, 0].double().numpy()
    got = orc.variant_attention_f64(q, k, v, bid, True, shift)[0, 0].numpy()
    assert np.abs(got - want).max() < 1e-7
    totals = orc.variant_demand_totals(q, k, bid, shift)[0, 0].numpy()
    assert np.abs(totals - c0 * (t - np.arange(t))).max() < 1e-12


def test_variant_exclusive_share_collapses_to_identity():
    """share = p / (committed + eps): committed[i, i] is exactly 0, so every
    row's diagonal wins by 1/eps and the output is v itself; the first row is
    v_0 in every mode (kernels_bid.py's exclusive-history notes)."""
    q, k, v = orc.make_inputs((1, 2, 40, 8), seed=8)
    out = orc.variant_attention_f64(q, k, v, "softmax", "exclusive")
    assert (out - v.double()).abs().max() < 1e-4          # off-diagonal weight ~ eps / committed
    for share in orc.SHARES:
        row0 = orc.variant_attention_f64(q, k, v, "relu", share)[:, :, 0]
        assert (row0 - v[:, :, 0].double()).abs().max() < 1e-8    # eps in the normalisation


# minshift holds its row minimum constant in the backward (kernels_bid.py:13-16),
# which finite differences do not: its forward is pinned above, its backward
# shares the autograd path of the others
@pytest.mark.parametrize("bid,share", [("relu", True), ("softplus", "exclusive"), ("relu", False),
                                       ("sigshift", True), ("expshift", False), ("relu2", True),
                                       ("sigmoid", "exclusive")])
def test_variant_gradcheck(bid, share):
    q, k, v = (x.double().requires_grad_(True) for x in orc.make_inputs((1, 1, 5, 4), seed=9))
    assert torch.autograd.gradcheck(
        lambda a, b, c: orc.variant_attention_f64(a, b, c, bid, share, 2.0), (q, k, v), eps=1e-6,
        atol=1e-5)


def test_planted_variant_mistake_fails_a_pin():
    """A relu bid without the empty-row rule is NaN at q = 0: the closed form
    catches it."""
    t = 8
    _, k, v = orc.make_inputs((1, 1, t, 4), seed=10)
    q = torch.zeros_like(k)
    aff = torch.matmul(q.double(), k.double().transpose(-2, -1))
    causal = torch.ones(t, t, dtype=torch.bool).tril()
    num = aff.clamp_min(0.0) * causal
    p = num / num.sum(-1, keepdim=True)                     # no uniform fallback
    want, _ = orc.harmonic_closed_form(t, v[0, 0])
    before = torch.cumsum(p, -2) - p
    sh = p / (before + p + orc.EPS)
    got = ((sh / (sh.sum(-1, keepdim=True) + orc.EPS)) @ v.double())[0, 0].numpy()
    assert not np.abs(got - want).max() < 1e-6
