"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU tests: the oracle still reproduces every committed fixture, and the
fixtures are self-consistent with facts that hold independently of the oracle
(the q = 0 harmonic totals, prefix consistency between the forward, prefill
and decode fixtures' demand vectors).
GPU tests (marked gpu): the HIP kernels, called through the drop-in
`dilution.kernels` API, match the fixtures at the north-star tolerances.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from gpu_helpers import max_abs, needs_gpu
from oracle import dilution_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


# ---------------------------------------------------------------------------
# CPU: the oracle against the fixtures


def test_oracle_reproduces_forward_fixture():
    g = load("forward_t200_d64.npz")
    q, k, v = (t(g[x]).double() for x in "qkv")
    assert np.abs(orc.attention_f64(q, k, v).numpy() - g["out"]).max() < 1e-6
    assert np.abs(orc.demand_totals(q, k).numpy() - g["committed_total"]).max() < 1e-12
    assert np.abs(orc.carry_checkpoints(q, k, 32).numpy() - g["carry"]).max() < 1e-12
    assert np.abs(orc.pk(q, k).numpy() - g["pk"]).max() < 1e-6


def test_oracle_reproduces_backward_fixture():
    g = load("backward_t96_d32.npz")
    (dq, dk, dv), inter = orc.grads_closed_form_f64(g["q"], g["k"], g["v"], g["dout"])
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv), ("out", inter["out"]),
                      ("ghat", inter["ghat"])):
        assert np.abs(got - g[name]).max() < 1e-5, name
    # key-shift invariance of the fixture itself: sum over keys of dk is zero
    assert np.abs(g["dk"].astype(np.float64).sum(-2)).max() < 1e-4


def test_oracle_reproduces_decode_and_prefill_fixtures():
    g = load("decode_p40_d32.npz")
    q, k, v = (t(g[x]).double() for x in "qkv")
    full = orc.attention_f64(q, k, v).numpy()
    prefix = int(g["prefix"])
    assert np.abs(g["step_out"] - full[..., prefix:, :]).max() < 1e-6
    assert np.abs(g["committed"][..., :48] - orc.demand_totals(q, k).numpy()).max() < 1e-12
    assert (g["committed"][..., 48:] == 0).all()
    p = load("prefill_t150_c48_d64.npz")
    q, k, v = (t(p[x]).double() for x in "qkv")
    assert np.abs(p["out"] - orc.attention_f64(q, k, v).numpy()).max() < 1e-6
    assert np.abs(p["committed"] - orc.demand_totals(q, k).numpy()).max() < 1e-12


def test_harmonic_fixture_is_closed_form():
    g = load("harmonic_t64_d16.npz")
    harm = np.cumsum(1.0 / np.arange(1, 65))
    want = harm[-1] - np.concatenate([[0.0], harm[:-1]])      # H_T - H_j
    assert np.abs(g["committed_total"] - want).max() < 1e-12
    z = torch.zeros(1, 1, 64, 16, dtype=torch.float64)
    out = orc.attention_f64(z, t(g["k"]).double(), t(g["v"]).double()).numpy()
    assert np.abs(out - g["out"]).max() < 1e-6


# ---------------------------------------------------------------------------
# GPU: the HIP kernels against the fixtures


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("prec", ["ieee", "tf32", "bf16"])
def test_gpu_forward_fixture(prec):
    from dilution import kernels

    g = load("forward_t200_d64.npz")
    q, k, v = (t(g[x]).cuda() for x in "qkv")
    if prec == "bf16":
        q, k, v = (x.bfloat16() for x in (q, k, v))
    out, aux = kernels.dilution_attention_forward(q, k, v, dot_precision=prec, return_aux=True,
                                                  _save_pk=True)
    if prec in ("ieee", "tf32"):
        assert max_abs(out, t(g["out"])) < 1e-4
        assert max_abs(aux["committed_total"], t(g["committed_total"])) < 1e-5
        carry = aux["carry"].reshape(g["carry"].shape)
        nb, seq = carry.shape[-2:]
        for rb in range(nb):                 # the written (causal) keys of each block
            end = min(32 * (rb + 1), seq)
            assert max_abs(carry[..., rb, :end], t(g["carry"])[..., rb, :end]) < 1e-5, rb
        assert max_abs(aux["pk"].reshape(g["pk"].shape), t(g["pk"])) < 2e-5
    else:
        # bf16 operands on bf16-rounded inputs: compare with the oracle on the
        # same rounded values, at the bf16 tolerance
        want = orc.attention_fp32(*(x.float().cpu() for x in (q, k, v)))
        assert max_abs(out, want) < 2e-2


@pytest.mark.gpu
@needs_gpu
def test_gpu_backward_fixture():
    from dilution import kernels

    g = load("backward_t96_d32.npz")
    xs = [t(g[x]).cuda().requires_grad_(True) for x in "qkv"]
    out = kernels.dilution_attention(*xs, dot_precision="ieee")
    out.backward(t(g["dout"]).cuda())
    assert max_abs(out.detach(), t(g["out"])) < 1e-4
    for name, x in zip(("dq", "dk", "dv"), xs):
        assert max_abs(x.grad, t(g[name])) < 1e-4, name


@pytest.mark.gpu
@needs_gpu
def test_gpu_decode_fixture():
    from dilution import kernels

    g = load("decode_p40_d32.npz")
    q, k, v = (t(g[x]).cuda() for x in "qkv")
    prefix, cap = int(g["prefix"]), int(g["capacity"])
    _, aux = kernels.dilution_attention_forward(q[..., :prefix, :], k[..., :prefix, :],
                                                v[..., :prefix, :], return_aux=True)
    kc = torch.zeros(1, 2, cap, 32, device="cuda")
    vc = torch.zeros_like(kc)
    com = torch.zeros(1, 2, cap, device="cuda")
    kc[..., :prefix, :] = k[..., :prefix, :]
    vc[..., :prefix, :] = v[..., :prefix, :]
    com[..., :prefix] = aux["committed_total"]
    for i, tt in enumerate(range(prefix, 48)):
        kc[..., tt, :] = k[..., tt, :]
        vc[..., tt, :] = v[..., tt, :]
        y = kernels.dilution_decode_step(q[..., tt:tt + 1, :], kc, vc, com, tt + 1)
        assert max_abs(y[..., 0, :], t(g["step_out"][..., i, :])) < 1e-4, tt
    assert max_abs(com, t(g["committed"])) < 1e-5


@pytest.mark.gpu
@needs_gpu
def test_gpu_prefill_fixture():
    from dilution import kernels

    g = load("prefill_t150_c48_d64.npz")
    q, k, v = (t(g[x]).cuda() for x in "qkv")
    chunk = int(g["chunk"])
    kc, vc = k.contiguous(), v.contiguous()
    com = torch.zeros(1, 2, 150, device="cuda")
    outs = []
    for start in range(0, 150, chunk):
        stop = min(start + chunk, 150)
        outs.append(kernels.dilution_prefill_chunk(q[..., start:stop, :], kc, vc, com, start,
                                                   dot_precision="ieee"))
    assert max_abs(torch.cat(outs, dim=2), t(g["out"])) < 1e-4
    assert max_abs(com, t(g["committed"])) < 1e-5


@pytest.mark.gpu
@needs_gpu
def test_gpu_harmonic_fixture():
    from dilution import kernels

    g = load("harmonic_t64_d16.npz")
    k, v = t(g["k"]).cuda(), t(g["v"]).cuda()
    out, aux = kernels.dilution_attention_forward(torch.zeros_like(k), k, v, return_aux=True)
    assert max_abs(out, t(g["out"])) < 1e-4
    assert max_abs(aux["committed_total"], t(g["committed_total"])) < 1e-5
