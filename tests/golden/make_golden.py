"""Write the golden fixtures in this folder from the CPU oracle (float64).

    python tests/golden/make_golden.py

Each fixture is an .npz of inputs and expected outputs (no pickles).  The
reference repository holds no golden vectors for this path (its kernel tests
compare against the fp32 reference on freshly seeded inputs), so these are
produced by this repository's own restatement of the operator, which
tests/test_oracle.py pins against brute-force loops, the q = 0 harmonic closed
form, finite differences and planted mistakes.  The fixtures freeze those
numbers so that the GPU tests and any later change to the oracle are checked
against the same values.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import dilution_oracle as orc  # noqa: E402


def _inputs(shape, seed, scale=1.0, dout=False):
    g = torch.Generator().manual_seed(seed)
    out = [torch.randn(*shape, generator=g) * scale, torch.randn(*shape, generator=g) * scale,
           torch.randn(*shape, generator=g)]
    if dout:
        out.append(torch.randn(*shape, generator=g))
    return [t.float() for t in out]


def forward_fixture():
    """Forward, aux totals and carry checkpoints: B1 H2 T200 d64, N(0,1)."""
    q, k, v = _inputs((1, 2, 200, 64), seed=20261)
    qd, kd, vd = (t.double() for t in (q, k, v))
    return dict(q=q.numpy(), k=k.numpy(), v=v.numpy(),
                out=orc.attention_f64(qd, kd, vd).numpy(),
                committed_total=orc.demand_totals(qd, kd).numpy(),
                carry=orc.carry_checkpoints(qd, kd, 32).numpy(),
                pk=orc.pk(qd, kd).numpy())


def backward_fixture():
    """Gradients: B1 H2 T96 d32, q,k ~ 0.5 N(0,1), v, dO ~ N(0,1)."""
    q, k, v, do = _inputs((1, 2, 96, 32), seed=20262, scale=0.5, dout=True)
    (dq, dk, dv), inter = orc.grads_closed_form_f64(q.numpy(), k.numpy(), v.numpy(), do.numpy())
    return dict(q=q.numpy(), k=k.numpy(), v=v.numpy(), dout=do.numpy(), out=inter["out"],
                dq=dq, dk=dk, dv=dv, ghat=inter["ghat"])


def decode_fixture():
    """Prefix 40 then 8 decode steps: B1 H2 d32, N(0,1); outputs per step and
    the demand vector after the last step (capacity 52)."""
    q, k, v = _inputs((1, 2, 48, 32), seed=20263)
    qd, kd, vd = (t.double() for t in (q, k, v))
    cap, prefix = 52, 40
    kc = torch.zeros(1, 2, cap, 32, dtype=torch.float64)
    vc = torch.zeros_like(kc)
    kc[..., :48, :] = kd
    vc[..., :48, :] = vd
    com = torch.zeros(1, 2, cap, dtype=torch.float64)
    com[..., :prefix] = orc.demand_totals(qd[..., :prefix, :], kd[..., :prefix, :])
    outs = []
    for t in range(prefix, 48):
        o, com = orc.decode_step(qd[..., t:t + 1, :], kc, vc, com, t + 1)
        outs.append(o[..., 0, :].numpy())
    return dict(q=q.numpy(), k=k.numpy(), v=v.numpy(), prefix=np.int64(prefix), capacity=np.int64(cap),
                step_out=np.stack(outs, axis=2), committed=com.numpy())


def prefill_fixture():
    """Chunked prefill in chunks of 48 over T=150: B1 H2 d64, N(0,1)."""
    q, k, v = _inputs((1, 2, 150, 64), seed=20264)
    qd, kd, vd = (t.double() for t in (q, k, v))
    demand = torch.zeros(1, 2, 150, dtype=torch.float64)
    outs = []
    for start in range(0, 150, 48):
        stop = min(start + 48, 150)
        o, dem = orc.prefill_chunk(qd[..., start:stop, :], kd[..., :stop, :], vd[..., :stop, :],
                                   demand, start)
        outs.append(o.numpy())
        demand = torch.zeros(1, 2, 150, dtype=torch.float64)
        demand[..., :stop] = dem
    return dict(q=q.numpy(), k=k.numpy(), v=v.numpy(), chunk=np.int64(48),
                out=np.concatenate(outs, axis=2), committed=demand.numpy())


def harmonic_fixture():
    """q = 0 closed form (harmonic numbers): B1 H1 T64 d16."""
    g = torch.Generator().manual_seed(20265)
    k = torch.randn(1, 1, 64, 16, generator=g).float()
    v = torch.randn(1, 1, 64, 16, generator=g).float()
    out, totals = orc.harmonic_closed_form(64, v.double().numpy())
    return dict(k=k.numpy(), v=v.numpy(), out=out, committed_total=totals)


FIXTURES = {
    "forward_t200_d64.npz": forward_fixture,
    "backward_t96_d32.npz": backward_fixture,
    "decode_p40_d32.npz": decode_fixture,
    "prefill_t150_c48_d64.npz": prefill_fixture,
    "harmonic_t64_d16.npz": harmonic_fixture,
}


# Expected arrays compared at tolerances >= 1e-5 are stored as float32 (their
# rounding, ~1e-7 relative, is far below every tolerance); demand totals and
# checkpoints stay float64.
KEEP_F64 = {"committed_total", "committed", "carry"}


def main() -> None:
    for name, fn in FIXTURES.items():
        arrs = {key: (val.astype(np.float32) if val.dtype == np.float64 and key not in KEEP_F64 else val)
                for key, val in fn().items()}
        np.savez_compressed(os.path.join(HERE, name), **arrs)
        print("wrote", name)


if __name__ == "__main__":
    main()
