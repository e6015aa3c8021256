"""Parity at the benchmark's full sizes (C3 training, C4 prefill + decode,
decode at 128K), where the dense oracle does not fit: the row-blocked fp64
oracle on a few (batch, head) slices, plus size-independent properties on
every slice.

* C3, B1 H16 T16384 d64 bf16 (q, k ~ 0.5 N(0,1), v, dO ~ N(0,1)):
  - output rows of slices 0 and 15 against ``attention_blocked_f64`` on the
    bf16-rounded inputs (2e-2 max-abs, 1e-2 mean-rel: the bf16 bounds);
  - dq, dk, dv of slices 0 and 15 against the row-blocked fp64 backward
    ``grads_blocked_f64`` on the host, and of all 16 slices against the same
    function evaluated in float64 on the device: 5e-2 max-abs (the north-star
    bound), 1e-2 of the largest gradient, and a mean error within 1e-2 of the
    mean gradient (every bf16 gradient check in this file; the short-row test
    holds the largest error to 2e-2 of the largest gradient);
  - the first 4096 rows are bit-identical to the forward of the 4096-token
    prefix (causality, test_model.py:46-56);
  - rows of the attention matrix sum to one, so sum_j dv_j = sum_i dO_i.  The
    kernel rounds the share tile, dO / (S + eps) and dv to bf16 (relative
    error <= 2^-9 each), which bounds the gap by 2^-8 (sum |dv| + sum |dO|).
* The same shape through the key-parallel output pass (the default) and the
  three-pass forward (DILUTION_FORWARD_KEY_PASS=0): outputs of slices 0 and
  15 against the blocked oracle, every output of one against the other
  (1e-2), demand totals and checkpoints within fp32 summation-order
  differences (1e-5 relative), and dq, dk, dv of slices 0 and 15 against the
  device oracle.
* The same shape in fp32 operands: outputs and dq, dk, dv of slices 0 and 15
  against ``grads_blocked_f64`` on the host and of every slice on the device
  (1e-4 max-abs); sum_j dk_j = 0 (adding a constant to every key leaves each
  softmax row unchanged) within 1e-4 of sum_j |dk_j|, and the dv identity
  within 1e-5.
* C2, B8 H16 T2048 d64 bf16 (128 slices, 16 per XCD: the packed longest-first
  dispatch): outputs and gradients of every slice against
  ``grads_blocked_f64`` on the device, four slices on the host.
* Many slices of short rows, B32 H12 T1024 (the reference's published
  shape) and B4 H75 T1024 (300 slices, uneven over the XCDs), bf16: outputs
  and gradients of every slice against ``grads_blocked_f64`` on the device.
* T = 131072, one slice, bf16: outputs and gradients of every row and key
  against ``grads_blocked_f64`` in float64 on the device, with the middle
  4096 rows and keys reported on their own; and the far end in closed form.
* C4, B16 H16 d64 bf16: a 16384-token prompt prefilled in 8 chunks of 2048,
  then 256 decode steps to 16640.  Prefill rows, decode rows and the demand
  equal the one-call forward of all 16640 rows (2e-2 on bf16 outputs, 1e-5
  relative on the demand); every row's bids sum to one, so the final demand
  sums to 16640; slice (0, 0) against the blocked oracle.
* Decode at 128K (B16 H16 d64 bf16 caches): one step on every slice against
  a plain torch statement of the step (the output within 2e-2; each demand
  entry within one fp32 spacing of c + p plus the score's rounding bound),
  and against the fp64 decode oracle on two slices; positions past
  ``length`` stay bit-untouched.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import max_abs, mean_rel, needs_gpu
from oracle import dilution_oracle as orc

pytestmark = [pytest.mark.gpu, needs_gpu]


def _blocked(q, k, v):
    out, tot = orc.attention_blocked_f64(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                         v.float().cpu().numpy())
    return torch.from_numpy(out), torch.from_numpy(tot)


def _grads_oracle(q, k, v, do, sl, device, block=1024):
    """((dq, dk, dv), intermediates) of one slice sl = (b, h) from the
    row-blocked fp64 backward on `device` (the host, or the GPU where the host
    would take minutes); inputs are the bf16-rounded / fp32 values upcast."""
    args = [t[sl].to(device=device, dtype=torch.float64) for t in (q, k, v, do)]
    return orc.grads_blocked_f64(*args, block=block)


# bf16-operand gradients: besides the north-star 5e-2 max-abs bound, the
# largest error within 1e-2 of the largest gradient (the bound the ablation
# tests hold the same one-pass kernel to) and the mean error within 1e-2 of
# the mean gradient.  At C3 the mean |dq| is 0.029 and the largest 0.59, so a
# systematic error of a few percent of a typical gradient fails the mean
# bound.  Measured on MI355X: rel-to-max <= 7.6e-3 and mean-rel <= 3.3e-3 over
# C3, C2 and T = 131072.
BF16_REL_MAX = 1e-2
BF16_MEAN_REL = 1e-2


def _check_grads(got, want, tol, where, rel=None, mean_rel_tol=None):
    """max-abs error of dq, dk, dv below `tol`; with `rel`, also below `rel`
    times the largest |gradient|; with `mean_rel_tol`, the mean |error| below
    that fraction of the mean |gradient|.  The measured errors are printed."""
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        e = (g.double() - w.to(g.device)).abs()
        err, wmax = e.max().item(), w.abs().max().item()
        merr, wmean = e.mean().item(), w.abs().mean().item()
        print(f"{where} {name}: max-abs {err:.3e} rel-to-max {err / wmax:.3e} "
              f"mean-rel {merr / wmean:.3e}")
        assert err < tol, f"{where} {name} max abs err {err}"
        if rel is not None:
            assert err < rel * wmax, f"{where} {name} err {err} above {rel} of the largest gradient {wmax}"
        if mean_rel_tol is not None:
            assert merr < mean_rel_tol * wmean, f"{where} {name} mean err {merr} vs mean gradient {wmean}"


def _check_bf16_grads(got, want, where):
    _check_grads(got, want, 5e-2, where, rel=BF16_REL_MAX, mean_rel_tol=BF16_MEAN_REL)


def test_c3_training_bf16_full_size():
    from dilution import kernels

    q, k, v, do = orc.make_inputs((1, 16, 16384, 64), seed=2, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(do.cuda())
    out = out.detach()
    torch.cuda.synchronize()
    for h in (0, 15):
        want, _ = _blocked(q[0, h], k[0, h], v[0, h])
        assert max_abs(out[0, h], want) < 2e-2, h
        assert mean_rel(out[0, h], want) < 1e-2, h

    prefix = kernels.dilution_attention_forward(*(x.detach()[:, :, :4096] for x in xs), dot_precision="bf16")
    assert torch.equal(prefix, out[:, :, :4096])

    dv = xs[2].grad.double().cpu()
    dod = do.double()
    gap = (dv.sum(2) - dod.sum(2)).abs()
    bound = 2.0 ** -8 * (dv.abs().sum(2) + dod.abs().sum(2))
    assert (gap <= bound).all(), (gap / bound).max().item()

    grads = [x.grad for x in xs]
    for h in range(16):
        want, inter = _grads_oracle(q, k, v, do, (0, h), "cuda")
        _check_bf16_grads([g[0, h] for g in grads], want, f"slice {h} (device oracle)")
    for h in (0, 15):
        want, _ = _grads_oracle(q, k, v, do, (0, h), "cpu")
        _check_bf16_grads([g[0, h] for g in grads], want, f"slice {h} (host oracle)")


def test_c3_key_pass_full_size(monkeypatch):
    from dilution import kernels

    q, k, v, do = orc.make_inputs((1, 16, 16384, 64), seed=4, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    qg, kg, vg = (t.cuda() for t in (q, k, v))
    monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
    out0, aux0 = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16", return_aux=True)
    monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS")
    out1, aux1 = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16", return_aux=True)
    torch.cuda.synchronize()
    for h in (0, 15):
        want, tot = _blocked(q[0, h], k[0, h], v[0, h])
        assert max_abs(out1[0, h], want) < 2e-2, h
        assert mean_rel(out1[0, h], want) < 1e-2, h
        rel = (aux1["committed_total"][0, h].double().cpu() - tot).abs() / tot.abs().clamp(min=1.0)
        assert rel.max().item() < 1e-5, h
    assert max_abs(out1, out0) < 1e-2
    t0, t1 = aux0["committed_total"].double(), aux1["committed_total"].double()
    assert ((t1 - t0).abs() / t0.abs().clamp(min=1.0)).max().item() < 1e-5
    # checkpoints: the causal part of every 32-row block (keys before the block's end)
    c0 = aux0["carry"].reshape(1, 16, -1, 16384).double()
    c1 = aux1["carry"].reshape(1, 16, -1, 16384).double()
    keys = torch.arange(16384, device=c0.device)
    ends = 32 * (torch.arange(c0.shape[2], device=c0.device) + 1)
    causal = keys[None, :] < ends[:, None]
    diff = ((c1 - c0).abs() / c0.abs().clamp(min=1.0))[..., causal]
    assert diff.max().item() < 1e-5
    # gradients through the three-pass forward (the default path's are
    # checked on every slice by test_c3_training_bf16_full_size)
    monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(do.cuda())
    grads = [x.grad for x in xs]
    for h in (0, 15):
        want, _ = _grads_oracle(q, k, v, do, (0, h), "cuda")
        _check_bf16_grads([g[0, h] for g in grads], want, f"slice {h} (device oracle, three-pass forward)")


def test_c3_training_fp32_full_size():
    from dilution import kernels

    q, k, v, do = orc.make_inputs((1, 16, 16384, 64), seed=3, qk_scale=0.5, with_dout=True)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="ieee")
    out.backward(do.cuda())
    out = out.detach()
    grads = [x.grad for x in xs]
    for h in range(16):
        want, inter = _grads_oracle(q, k, v, do, (0, h), "cuda")
        assert max_abs(out[0, h], inter["out"]) < 1e-4, h
        _check_grads([g[0, h] for g in grads], want, 1e-4, f"slice {h} (device oracle)")
    for h in (0, 15):
        want, inter = _grads_oracle(q, k, v, do, (0, h), "cpu")
        assert max_abs(out[0, h], inter["out"]) < 1e-4, h
        _check_grads([g[0, h] for g in grads], want, 1e-4, f"slice {h} (host oracle)")
    dk = xs[1].grad.double().cpu()
    assert (dk.sum(2).abs() <= 1e-4 * dk.abs().sum(2)).all()
    dv = xs[2].grad.double().cpu()
    gap = (dv.sum(2) - do.double().sum(2)).abs()
    assert (gap <= 1e-5 * (dv.abs().sum(2) + do.double().abs().sum(2))).all()


def test_c3_training_tf32_full_size():
    """The "tf32" precision (fp32 values as split bf16 operands, three bf16
    products per product) at C3 shape within the fp32-mode bound."""
    from dilution import kernels

    q, k, v, do = orc.make_inputs((1, 16, 16384, 64), seed=4, qk_scale=0.5, with_dout=True)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="tf32")
    out.backward(do.cuda())
    out = out.detach()
    grads = [x.grad for x in xs]
    for h in (0, 5, 10, 15):
        want, inter = _grads_oracle(q, k, v, do, (0, h), "cuda")
        assert max_abs(out[0, h], inter["out"]) < 1e-4, h
        _check_grads([g[0, h] for g in grads], want, 1e-4, f"slice {h} (device oracle)")
    want, inter = _grads_oracle(q, k, v, do, (0, 15), "cpu")
    assert max_abs(out[0, 15], inter["out"]) < 1e-4
    _check_grads([g[0, 15] for g in grads], want, 1e-4, "slice 15 (host oracle)")


def test_c2_training_bf16_every_slice():
    """B8 H16 T2048 d64 bf16, q, k ~ 0.5 N(0,1), v, dO ~
    N(0,1).  128 slices put 16 on each XCD, the shape that dispatches every
    XCD's slices longest first (packed across slices)."""
    from dilution import kernels

    q, k, v, do = orc.make_inputs((8, 16, 2048, 64), seed=21, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(do.cuda())
    out = out.detach()
    grads = [x.grad for x in xs]
    worst = 0.0
    for b in range(8):
        for h in range(16):
            want, inter = _grads_oracle(q, k, v, do, (b, h), "cuda", block=512)
            assert max_abs(out[b, h], inter["out"]) < 2e-2, (b, h)
            assert mean_rel(out[b, h], inter["out"]) < 1e-2, (b, h)
            _check_bf16_grads([g[b, h] for g in grads], want, f"slice {(b, h)}")
            worst = max(worst, max((g[b, h].double().cpu() - w.cpu()).abs().max().item()
                                   for g, w in zip(grads, want)))
    for sl in ((0, 0), (3, 7), (5, 2), (7, 15)):
        want, inter = _grads_oracle(q, k, v, do, sl, "cpu", block=512)
        assert max_abs(out[sl], inter["out"]) < 2e-2, sl
        _check_bf16_grads([g[sl] for g in grads], want, f"slice {sl} (host oracle)")
    print(f"C2 worst gradient error {worst:.3e}")


@pytest.mark.parametrize("shape", [(32, 12, 1024), (4, 75, 1024)])
def test_short_rows_many_slices_every_slice(shape):
    """Many slices of short rows (more than 2^18 tokens, rows of at most 2048
    keys): every kernel dispatches longest first, per XCD for 384 slices (the
    reference's published B32 H12 T1024 shape) and spread over the chip for
    300 slices, which do not divide over the 8 XCDs.  Outputs and gradients of
    every slice against ``grads_blocked_f64`` on the device: the bf16 bounds
    of the other shapes, except that the largest gradient error is held to
    2e-2 of the slice's largest gradient (at T = 1024 the largest |dk| of a
    slice is ~0.3, and the bf16 rounding of the operands reached 1.03e-2 of
    it in one of the 684 slices, measured on MI355X; the worst of the other
    shape was 9.0e-3)."""
    from dilution import kernels

    q, k, v, do = orc.make_inputs((*shape, 64), seed=23, qk_scale=0.5, with_dout=True, dtype=torch.bfloat16)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(do.cuda())
    out = out.detach()
    grads = [x.grad for x in xs]
    worst = 0.0
    for b in range(shape[0]):
        for h in range(shape[1]):
            want, inter = _grads_oracle(q, k, v, do, (b, h), "cuda", block=512)
            assert max_abs(out[b, h], inter["out"]) < 2e-2, (b, h)
            assert mean_rel(out[b, h], inter["out"]) < 1e-2, (b, h)
            got = [g[b, h] for g in grads]
            _check_grads(got, want, 5e-2, f"slice {(b, h)}", rel=2e-2, mean_rel_tol=BF16_MEAN_REL)
            worst = max(worst, max((g.double() - w).abs().max().item() / w.abs().max().item()
                                   for g, w in zip(got, want)))
    print(f"{shape}: worst gradient error {worst:.3e} of the slice's largest gradient")


def test_c4_chunked_prefill_then_256_decode_steps():
    from dilution import cache as dcache
    from dilution import kernels

    b, h, d, t0, steps = 16, 16, 64, 16384, 256
    t1 = t0 + steps
    g = torch.Generator(device="cuda").manual_seed(4)
    q, k, v = (torch.randn(b, h, t1, d, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    full, aux = kernels.dilution_attention_forward(q, k, v, dot_precision="bf16", return_aux=True)
    y, cache = dcache.begin_cache(q[:, :, :t0], k[:, :, :t0].contiguous(), v[:, :, :t0].contiguous(),
                                  capacity=t1, chunk=2048)
    assert max_abs(y, full[:, :, :t0]) < 2e-2
    rows = []
    for t in range(t0, t1):
        rows.append(dcache.step_cache(q[:, :, t:t + 1], k[:, :, t:t + 1], v[:, :, t:t + 1], cache))
    dec = torch.cat(rows, dim=2)
    assert max_abs(dec, full[:, :, t0:]) < 2e-2
    com = cache["committed"]
    tot = aux["committed_total"]
    assert max_abs(com, tot) < 1e-5 * max(1.0, tot.abs().max().item())
    sums = com.double().sum(-1)
    assert (sums - t1).abs().max().item() < 1e-5 * t1

    want, want_tot = _blocked(q[0, 0], k[0, 0], v[0, 0])
    got = torch.cat([y[0, 0], dec[0, 0]], dim=0)
    assert max_abs(got, want) < 2e-2
    assert mean_rel(got, want) < 1e-2
    assert max_abs(com[0, 0], want_tot) < 1e-5 * max(1.0, want_tot.abs().max().item())


def test_decode_at_128k_context():
    from dilution import kernels

    b, h, d, length = 16, 16, 64, 131072
    cap = length + 64
    g = torch.Generator(device="cuda").manual_seed(6)
    kc = torch.randn(b, h, cap, d, device="cuda", generator=g).to(torch.bfloat16)
    vc = torch.randn(b, h, cap, d, device="cuda", generator=g).to(torch.bfloat16)
    q1 = torch.randn(b, h, 1, d, device="cuda", generator=g).to(torch.bfloat16)
    com = torch.rand(b, h, cap, device="cuda", generator=g) * 4.0
    com[..., length - 1] = 0.0
    before = com.clone()
    out = kernels.dilution_decode_step(q1, kc, vc, com, length)
    torch.cuda.synchronize()
    assert torch.equal(com[..., length:], before[..., length:])

    # every slice against a plain torch statement of the step (fp64 scores of
    # the bf16 values, so the reference's own rounding does not count)
    kd = kc[..., :length, :].double()
    aff = torch.matmul(q1.double(), kd.transpose(-1, -2).contiguous())[..., 0, :] / 8.0
    p = torch.softmax(aff, dim=-1)
    c = before[..., :length].double()
    share = p / (c + p + 1e-9)
    want = torch.matmul((share / (share.sum(-1, keepdim=True) + 1e-9))[..., None, :],
                        vc[..., :length, :].double())
    assert max_abs(out, want) < 2e-2
    # committed = fl(c + p_kernel).  The kernel's fp32 score of a 64-term dot
    # is off by at most 65 * 2^-24 * sum |q_d k_d| / 8 (the gamma_n bound of a
    # recursive fma sum); p moves by that relative to its own score and to the
    # row's normaliser, plus a few ulps of exp2 / rcp.
    err_a = 65 * 2.0 ** -24 * torch.matmul(q1.double().abs(), kd.abs().transpose(-1, -2).contiguous())[..., 0, :] / 8.0
    rel_p = 2 * err_a + 2 * err_a.amax(-1, keepdim=True) + 8 * 2.0 ** -24
    after = com[..., :length]
    spacing = (torch.nextafter(after, torch.full_like(after, float("inf"))) - after).double()
    assert ((after.double() - (c + p)).abs() <= spacing + p * rel_p).all()

    for bi, hi in ((0, 0), (15, 15)):
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        want64, want_com = orc.decode_step(q1[sl].cpu(), kc[sl].cpu(), vc[sl].cpu(), before[sl].cpu(), length)
        assert max_abs(out[sl], want64) < 2e-2
        assert max_abs(com[sl][..., :length], want_com[..., :length]) < 1e-5 * 4.0


def test_sequence_of_131072_gradients_against_blocked_oracle():
    """One slice at T = 131072 (bf16): every output row and every dq, dk, dv
    row against the row-blocked fp64 oracle evaluated on the device (the host
    would take hours), the middle 4096 rows / keys reported on their own --
    the suffix checkpoints and the row pass at 4096 row tiles, far past the
    benchmark's sizes."""
    from dilution import kernels

    seq, d = 131072, 64
    q, k, v, do = orc.make_inputs((1, 1, seq, d), seed=8, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(do.cuda())
    out = out.detach()
    grads = [x.grad[0, 0] for x in xs]
    torch.cuda.synchronize()
    want, inter = _grads_oracle(q, k, v, do, (0, 0), "cuda", block=2048)
    assert max_abs(out[0, 0], inter["out"]) < 2e-2
    assert mean_rel(out[0, 0], inter["out"]) < 1e-2
    mid = slice(seq // 2 - 2048, seq // 2 + 2048)
    _check_bf16_grads([g[mid] for g in grads], [w[mid] for w in want], "middle rows / keys")
    _check_bf16_grads(grads, want, "all rows / keys")


def test_key_pass_slice_batches_at_131072():
    """B1 H12 T = 131072 bf16, forward without aux (the long-context
    inference forward): one slice's key-pass partials take ~2.2 GB, so the
    24 GiB workspace holds 11 slices and the pass runs in two equal slice
    batches (6 + 6), writing no checkpoint array.  Slices are independent, so
    each equals, bit for bit, the forward of that slice alone (one batch): the
    first and last slices of each batch."""
    from dilution import _hip, kernels

    seq, heads, d = 131072, 12, 64
    lib = _hip.lib()
    assert lib.dil_forward_key_pass(seq, 0, d, 1, 2) == 1
    one_slice = lib.dil_forward_workspace_bytes(1, seq, d, 1, 2, 0)
    assert lib.dil_forward_workspace_bytes(heads, seq, d, 1, 2, 0) < heads * one_slice
    g = torch.Generator(device="cuda").manual_seed(9)
    q, k = ((torch.randn(1, heads, seq, d, device="cuda", generator=g) * 0.5).to(torch.bfloat16)
            for _ in range(2))
    v = torch.randn(1, heads, seq, d, device="cuda", generator=g).to(torch.bfloat16)
    out = kernels.dilution_attention_forward(q, k, v, dot_precision="bf16")
    assert torch.isfinite(out).all()
    for h in (0, 5, 6, 11):
        alone = kernels.dilution_attention_forward(*(x[:, h:h + 1].contiguous() for x in (q, k, v)),
                                                   dot_precision="bf16")
        assert torch.equal(alone, out[:, h:h + 1]), h


def test_sequence_of_131072_far_end_closed_forms():
    """One slice at T = 131072 (bf16), where (T/32) x T checkpoints and T x d
    offsets are far past the benchmark's sizes.  The oracle does not fit, but
    the far end of the sequence has closed forms in one row of scores:

    * the last row's committed demand plus its own bid is the key's demand
      total (c + p = total_j), so with the kernel's totals its output is
      sum_j p_j v_j / (total_j + eps), renormalised (kernels.py:59-68);
    * its suffix term is empty, so dp_j = ds_j (c_j + eps) / (total_j + eps)^2
      and dq_{T-1} = s sum_j p_j (dp_j - ghat) k_j; key T-1 is seen by row
      T-1 alone, which gives dk_{T-1} and dv_{T-1}
      (docs/kernels.md:62-84 restated);
    * the totals of the last 64 keys are column sums over the last 64 rows;
    * every row's bids sum to one, so the totals sum to T; the first 4096
      rows are bit-identical to the forward of the 4096-token prefix.
    """
    from dilution import kernels

    seq, d, eps = 131072, 64, 1e-9
    q, k, v, do = orc.make_inputs((1, 1, seq, d), seed=7, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(do.cuda())
    _, aux = kernels.dilution_attention_forward(*(x.detach() for x in xs), dot_precision="bf16",
                                                return_aux=True)
    prefix = kernels.dilution_attention_forward(*(x.detach()[:, :, :4096] for x in xs),
                                                dot_precision="bf16")
    torch.cuda.synchronize()
    assert torch.equal(prefix, out.detach()[:, :, :4096])
    out = out.detach()[0, 0].double().cpu().numpy()
    dq, dk, dv = (x.grad[0, 0].double().cpu().numpy() for x in xs)
    assert np.isfinite(dq).all() and np.isfinite(dk).all() and np.isfinite(dv).all()
    tot = aux["committed_total"][0, 0].double().cpu().numpy()
    assert abs(tot.sum() - seq) <= 1e-4 * seq

    Q, K, V, dO = (t[0, 0].double().numpy() for t in (q, k, v, do))
    s = d ** -0.5
    a = (Q[-64:] @ K.T) * s
    a[np.arange(64)[:, None] + seq - 64 < np.arange(seq)[None, :]] = -np.inf
    p64 = np.exp(a - a.max(1, keepdims=True))
    p64 /= p64.sum(1, keepdims=True)
    want_tot = p64[:, seq - 64:].sum(0)                     # masked: only rows i >= j
    assert np.abs(tot[seq - 64:] - want_tot).max() <= 1e-4 * want_tot.max() + 1e-7

    p = p64[-1]
    share = p / (tot + eps)
    S = share.sum()
    A = share / (S + eps)
    o = A @ V
    assert np.abs(out[-1] - o).max() < 2e-2
    ds = (V @ dO[-1] - dO[-1] @ o) / (S + eps)
    dp = ds * (tot - p + eps) / (tot + eps) ** 2
    da = p * (dp - (p * dp).sum())
    g_dq, g_dk, g_dv = s * (da @ K), s * da[-1] * Q[-1], A[-1] * dO[-1]
    scale = np.abs(g_dq).max()
    assert np.abs(dq[-1] - g_dq).max() < 5e-2 * max(scale, 1e-3), (np.abs(dq[-1] - g_dq).max(), scale)
    assert np.abs(dk[-1] - g_dk).max() < 5e-2 * max(np.abs(g_dk).max(), 1e-6) + 1e-6
    assert np.abs(dv[-1] - g_dv).max() < 5e-2 * max(np.abs(g_dv).max(), 1e-6) + 1e-6
