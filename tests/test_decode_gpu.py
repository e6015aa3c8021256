"""Cached decode parity (reference pattern: tests/test_kernels.py:205-241).

Token after token, the HIP decode step must reproduce the oracle's row t of
the full-sequence operator, advance the fp32 demand vector in place to the
column sums of p (within 1e-5 of the float64 oracle), and never touch the
spare capacity beyond `length`.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import max_abs, needs_gpu
from oracle import dilution_oracle as orc

pytestmark = [pytest.mark.gpu, needs_gpu]

TOL_OUT = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [16, 32, 64, 128])
def test_decode_matches_oracle_rows(dtype, head_dim):
    from dilution import kernels

    batch, heads, prefix, steps = 2, 4, 37, 6
    total = prefix + steps
    q, k, v = orc.make_inputs((batch, heads, total, head_dim), seed=1000 + head_dim)
    q, k, v = (x.to(dtype) for x in (q, k, v))           # the kernel's inputs
    full = orc.attention_f64(q, k, v)                     # oracle on the same (rounded) values
    prec = "bf16" if dtype == torch.bfloat16 else "ieee"
    qg, kg, vg = (x.cuda() for x in (q, k, v))
    _, aux = kernels.dilution_attention_forward(qg[:, :, :prefix], kg[:, :, :prefix],
                                                vg[:, :, :prefix], dot_precision=prec,
                                                return_aux=True)
    capacity = total + 3                                  # spare rows: never touched
    kc = torch.zeros(batch, heads, capacity, head_dim, device="cuda", dtype=dtype)
    vc = torch.zeros_like(kc)
    kc[:, :, :prefix] = kg[:, :, :prefix]
    vc[:, :, :prefix] = vg[:, :, :prefix]
    committed = torch.zeros(batch, heads, capacity, device="cuda")
    committed[:, :, :prefix] = aux["committed_total"]
    for t in range(prefix, total):
        kc[:, :, t] = kg[:, :, t]
        vc[:, :, t] = vg[:, :, t]
        out = kernels.dilution_decode_step(qg[:, :, t:t + 1], kc, vc, committed, t + 1)
        assert out.dtype == dtype and out.shape == (batch, heads, 1, head_dim)
        assert torch.isfinite(out).all()
        err = max_abs(out[:, :, 0], full[:, :, t])
        assert err < TOL_OUT[dtype], f"t={t} max abs err {err}"
    want = orc.demand_totals(q, k)
    assert max_abs(committed[:, :, :total], want) < 1e-5
    assert committed[:, :, total:].abs().max().item() == 0


@pytest.mark.parametrize("length", [1, 1023, 1024, 1025, 2047, 2048, 2049, 5000, 9000])
def test_decode_long_context_multi_chunk(length):
    """Lengths around the split-K decode's chunk boundaries (2048 keys per
    workgroup) and several chunks, with a synthetic non-negative demand vector."""
    from dilution import kernels

    batch, heads, d = 1, 3, 64
    g = torch.Generator().manual_seed(length)
    q = torch.randn(batch, heads, 1, d, generator=g)
    kc = torch.randn(batch, heads, length + 5, d, generator=g)
    vc = torch.randn(batch, heads, length + 5, d, generator=g)
    com = torch.rand(batch, heads, length + 5, generator=g) * 3.0
    com[..., length - 1:] = 0.0
    out_ref, com_ref = orc.decode_step(q, kc, vc, com, length)
    comg = com.cuda()
    out = kernels.dilution_decode_step(q.cuda(), kc.cuda(), vc.cuda(), comg, length)
    assert max_abs(out, out_ref) < 1e-4
    assert max_abs(comg, com_ref) < 1e-5
    assert comg[..., length:].abs().max().item() == 0


def test_decode_argument_errors():
    from dilution import kernels

    kc = torch.zeros(1, 1, 8, 64, device="cuda")
    com = torch.zeros(1, 1, 8, device="cuda")
    with pytest.raises(ValueError):
        kernels.dilution_decode_step(torch.zeros(1, 1, 2, 64, device="cuda"), kc, kc, com, 2)
    with pytest.raises(ValueError):
        kernels.dilution_decode_step(torch.zeros(1, 1, 1, 64, device="cuda"), kc, kc, com, 9)
    with pytest.raises(ValueError):
        kernels.dilution_decode_step(torch.zeros(1, 1, 1, 64, device="cuda"), kc, kc, com, 0)
    with pytest.raises(ValueError):
        bad = torch.zeros(1, 1, 8, 48, device="cuda")
        kernels.dilution_decode_step(torch.zeros(1, 1, 1, 48, device="cuda"), bad, bad, com, 2)


@pytest.mark.parametrize("qdt,cdt,tol", [(torch.float32, torch.bfloat16, 1e-4),
                                         (torch.bfloat16, torch.float32, 2e-2),
                                         (torch.float16, torch.bfloat16, 2e-3)])
def test_decode_query_keeps_its_dtype(qdt, cdt, tol):
    """q1 is read in its own dtype and the output stored in it, whatever the
    caches hold (reference kernels.py:953, 1029).  An fp32 query over bf16
    caches stays within the fp32 tolerance of the oracle on the same values:
    nothing on the query side is rounded to bf16."""
    from dilution import kernels

    batch, heads, length, d = 2, 3, 3000, 64
    g = torch.Generator().manual_seed(42)
    q = torch.randn(batch, heads, 1, d, generator=g).to(qdt)
    kc = torch.randn(batch, heads, length + 4, d, generator=g).to(cdt)
    vc = torch.randn(batch, heads, length + 4, d, generator=g).to(cdt)
    com = torch.rand(batch, heads, length + 4, generator=g) * 3.0
    com[..., length - 1:] = 0.0
    out_ref, com_ref = orc.decode_step(q, kc, vc, com, length)     # fp64 of the given values
    comg = com.cuda()
    out = kernels.dilution_decode_step(q.cuda(), kc.cuda(), vc.cuda(), comg, length)
    assert out.dtype == qdt
    err = max_abs(out, out_ref)
    assert err < tol, err
    assert max_abs(comg, com_ref) < 1e-5
    assert comg[..., length:].abs().max().item() == 0


@pytest.mark.parametrize("dtype,head_dim", [(torch.bfloat16, 64), (torch.float32, 128), (torch.bfloat16, 256)])
def test_device_length_decode_is_the_decode_step(dtype, head_dim):
    """decode_step_device_length (the length read from device memory, grid
    and workspace sized for max_length) against dilution_decode_step at the
    same live length: bitwise equal outputs and demand, around the 2048-key
    chunk boundaries; one workspace serves every length."""
    from dilution import kernels

    batch, heads, cap = 2, 3, 5000
    g = torch.Generator().manual_seed(11)
    kc = torch.randn(batch, heads, cap, head_dim, generator=g).to(dtype).cuda()
    vc = torch.randn(batch, heads, cap, head_dim, generator=g).to(dtype).cuda()
    base = torch.rand(batch, heads, cap, generator=g).cuda() * 3
    ws = kernels.decode_workspace(batch, heads, cap, head_dim, "cuda")
    out = torch.empty(batch, heads, head_dim, device="cuda", dtype=dtype)
    for length in (1, 2047, 2048, 2049, 4096, 4999, 5000):
        q1 = torch.randn(batch, heads, 1, head_dim, generator=g).to(dtype).cuda()
        c_ref = base.clone()
        c_ref[..., length - 1] = 0
        c_dev = c_ref.clone()
        want = kernels.dilution_decode_step(q1, kc, vc, c_ref, length)
        got = kernels.decode_step_device_length(q1, kc, vc, c_dev,
                                                torch.tensor([length], device="cuda"), cap,
                                                out=out, workspace=ws)
        assert torch.equal(got, want), length
        assert torch.equal(c_dev, c_ref), length


def test_device_length_decode_keeps_the_chunks_of_the_live_length():
    """B8 H16: the key chunks follow the batch and the live length (2048 keys
    at 16384, 1409 at 16900, where 2048-key chunks would leave a part-filled
    round; 513 at 2049).  The replayed form picks them from the device-resident
    length, so it stays bitwise equal to the host-length step at every length
    while its grid and workspace are sized once for the capacity."""
    from dilution import kernels

    batch, heads, cap, d = 8, 16, 17000, 64
    g = torch.Generator(device="cuda").manual_seed(21)
    kc = torch.randn(batch, heads, cap, d, device="cuda", generator=g).bfloat16()
    vc = torch.randn(batch, heads, cap, d, device="cuda", generator=g).bfloat16()
    base = torch.rand(batch, heads, cap, device="cuda", generator=g) * 3
    ws = kernels.decode_workspace(batch, heads, cap, d, "cuda")
    for length in (300, 2049, 8192, 16384, 16385, 16900, 17000):
        q1 = torch.randn(batch, heads, 1, d, device="cuda", generator=g).bfloat16()
        c_ref = base.clone()
        c_ref[..., length - 1] = 0
        c_dev = c_ref.clone()
        want = kernels.dilution_decode_step(q1, kc, vc, c_ref, length)
        got = kernels.decode_step_device_length(q1, kc, vc, c_dev, torch.tensor([length], device="cuda"), cap,
                                                workspace=ws)
        assert torch.equal(got, want), length
        assert torch.equal(c_dev, c_ref), length
        assert torch.equal(c_dev[..., length:], base[..., length:]), length


def test_device_length_decode_clamps_the_live_length():
    """A live length past max_length runs as max_length; 0 leaves the demand
    untouched and outputs zeros.  Nothing past max_length is read or written."""
    from dilution import kernels

    batch, heads, cap, d = 1, 2, 3000, 64
    g = torch.Generator().manual_seed(12)
    kc = torch.randn(batch, heads, cap, d, generator=g).bfloat16().cuda()
    vc = torch.randn(batch, heads, cap, d, generator=g).bfloat16().cuda()
    q1 = torch.randn(batch, heads, 1, d, generator=g).bfloat16().cuda()
    c0 = torch.rand(batch, heads, cap, generator=g).cuda()
    c0[..., 2499] = 0
    c_ref, c_dev = c0.clone(), c0.clone()
    want = kernels.dilution_decode_step(q1, kc, vc, c_ref, 2500)
    got = kernels.decode_step_device_length(q1, kc, vc, c_dev, torch.tensor([2600], device="cuda"), 2500)
    assert torch.equal(got, want) and torch.equal(c_dev, c_ref)
    c_zero = c0.clone()
    got0 = kernels.decode_step_device_length(q1, kc, vc, c_zero, torch.tensor([0], device="cuda"), 2500)
    assert torch.equal(c_zero, c0)
    assert (got0 == 0).all()
    with pytest.raises(ValueError):
        kernels.decode_step_device_length(q1, kc, vc, c_zero, torch.tensor([5], device="cuda"), cap + 1)
    with pytest.raises(ValueError):
        kernels.decode_step_device_length(q1, kc, vc, c_zero, torch.tensor([5.0], device="cuda"), 10)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_decode_head_dim_256_rows(dtype):
    """The decode step at head_dim 256 (every cache dtype) from a prefix
    demand the oracle supplies, step after step against the fp64 oracle of the
    whole sequence; the demand against the oracle's totals (1e-5); spare
    capacity untouched."""
    from dilution import kernels

    batch, heads, prefix, steps, d = 2, 2, 40, 5, 256
    total = prefix + steps
    q, k, v = orc.make_inputs((batch, heads, total, d), seed=2560)
    q, k, v = (x.to(dtype) for x in (q, k, v))
    full = orc.attention_f64(q, k, v)
    capacity = total + 3
    kc = torch.zeros(batch, heads, capacity, d, device="cuda", dtype=dtype)
    vc = torch.zeros_like(kc)
    committed = torch.zeros(batch, heads, capacity, device="cuda")
    committed[:, :, :prefix] = orc.demand_totals(q[:, :, :prefix], k[:, :, :prefix]).float().cuda()
    kc[:, :, :prefix], vc[:, :, :prefix] = k[:, :, :prefix].cuda(), v[:, :, :prefix].cuda()
    tol = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-3}[dtype]
    for t in range(prefix, total):
        kc[:, :, t], vc[:, :, t] = k[:, :, t].cuda(), v[:, :, t].cuda()
        out = kernels.dilution_decode_step(q[:, :, t:t + 1].cuda(), kc, vc, committed, t + 1)
        assert out.dtype == dtype and out.shape == (batch, heads, 1, d)
        assert max_abs(out[:, :, 0], full[:, :, t]) < tol, t
    assert max_abs(committed[:, :, :total], orc.demand_totals(q, k)) < 1e-5 * 4
    assert committed[:, :, total:].abs().max().item() == 0
