"""Forward parity of the HIP kernels against the CPU oracle.

Reference patterns: tests/test_kernels.py:19-75 (block scan, pk, forward),
:98-106 (bf16 inputs), :130-149 (checkpoints and totals).  Tolerances are the
north-star ones: fp32 mode <= 1e-4 max-abs; bf16 mode <= 2e-2 max-abs and
<= 1e-2 mean-relative against the fp32/fp64 oracle on the bf16-rounded inputs;
demand totals <= 1e-5.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import max_abs, mean_rel, needs_gpu
from oracle import dilution_oracle as orc

pytestmark = [pytest.mark.gpu, needs_gpu]


@pytest.mark.parametrize("seq", [1, 8, 33, 64, 128, 257, 1025])
@pytest.mark.parametrize("shape", [(1, 1), (2, 4)])
@pytest.mark.parametrize("prec", ["ieee", "tf32"])
def test_forward_fp32_matches_oracle(seq, shape, prec):
    from dilution import kernels

    batch, heads = shape
    q, k, v = orc.make_inputs((batch, heads, seq, 64), seed=seq)
    want = orc.attention_f64(q, k, v)
    got = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), dot_precision=prec)
    assert got.dtype == torch.float32 and got.shape == q.shape
    assert torch.isfinite(got).all()
    assert max_abs(got, want) < 1e-4


@pytest.mark.parametrize("head_dim", [16, 32, 128])
@pytest.mark.parametrize("prec", ["ieee", "tf32"])
def test_forward_fp32_head_dims(head_dim, prec):
    from dilution import kernels

    q, k, v = orc.make_inputs((2, 2, 200, head_dim), seed=head_dim)
    want = orc.attention_f64(q, k, v)
    got = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), dot_precision=prec)
    assert max_abs(got, want) < 1e-4


@pytest.mark.parametrize("seq", [1, 64, 257, 2048])
@pytest.mark.parametrize("head_dim", [32, 64, 128, 256])
def test_forward_bf16_matches_oracle(seq, head_dim):
    from dilution import kernels

    q, k, v = orc.make_inputs((2, 4, seq, head_dim), seed=7 * seq + head_dim, qk_scale=0.5,
                              dtype=torch.bfloat16)
    want = orc.attention_fp32(q, k, v)         # oracle on the bf16-rounded values
    got = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), dot_precision="bf16")
    assert torch.isfinite(got).all()
    assert max_abs(got, want) < 2e-2
    assert mean_rel(got, want) < 1e-2


def test_forward_fp32_inputs_bf16_operands():
    """fp32 tensors with dot_precision="bf16" (bf16 MFMA operands) stay within
    the bf16 tolerance of the fp32 oracle (reference test_kernels.py:98-106)."""
    from dilution import kernels

    q, k, v = orc.make_inputs((2, 4, 128, 64), seed=0)
    want = orc.attention_fp32(q, k, v)
    got = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), dot_precision="bf16")
    assert max_abs(got, want) < 5e-2


@pytest.mark.parametrize("seq", [1, 65, 257, 2049])
def test_checkpoints_totals_and_row_stats(seq):
    """aux["carry"] holds the demand entering every 32-row block,
    aux["committed_total"] the column totals of p (reference
    test_kernels.py:130-149; stricter tolerance)."""
    from dilution import kernels

    q, k, v = orc.make_inputs((1, 2, seq, 32), seed=seq)
    out, aux = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), return_aux=True,
                                                  _save_pk=True)
    assert max_abs(out, orc.attention_f64(q, k, v)) < 1e-4
    assert max_abs(aux["committed_total"], orc.demand_totals(q, k)) < 1e-5
    bm = aux["bwd_block_m"]
    assert bm == 32
    carry = orc.carry_checkpoints(q, k, bm).reshape(2, -1, seq)
    assert aux["carry"].shape == carry.shape
    for rb in range(carry.shape[1]):
        # only the block's causal keys are written (test_kernels.py:143-149)
        end = min((rb + 1) * bm, seq)
        assert max_abs(aux["carry"][:, rb, :end], carry[:, rb, :end]) < 1e-5, rb
    rmax, rden = orc.row_stats(q, k)
    assert max_abs(aux["rmax"], rmax.reshape(2, seq)) < 1e-4
    lse_got = aux["rmax"].double().cpu() + torch.log2(aux["rden"].double().cpu())
    lse_want = (rmax + torch.log2(rden)).reshape(2, seq)
    assert (lse_got - lse_want).abs().max().item() < 1e-5


def test_c1_exact_shape_fp32_forward():
    """BASELINE config 1 as stated: B1 H4 T512 d64, q, k, v ~ N(0,1) fp32,
    the reference's default ieee precision, scale 1/sqrt(d), eps 1e-9."""
    from dilution import kernels

    q, k, v = orc.make_inputs((1, 4, 512, 64), seed=1)
    got = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda())
    assert got.shape == (1, 4, 512, 64) and got.dtype == torch.float32
    assert max_abs(got, orc.attention_f64(q, k, v)) < 1e-4
    assert max_abs(got, orc.attention_fp32(q, k, v)) < 1e-4


def _forward_into(q, k, v, carry, prec=2):
    """dil_forward through the C ABI into a caller-owned carry buffer."""
    from dilution import _hip

    lib = _hip.lib()
    n, t, d = q.shape
    f32 = dict(device=q.device, dtype=torch.float32)
    out = torch.empty(n, t, d, **f32)
    stats = [torch.empty(n, t, **f32) for _ in range(4)]        # rmax rden ssum total
    dt = {torch.float32: 0, torch.bfloat16: 1}[q.dtype]
    ws = torch.empty(lib.dil_forward_workspace_bytes(n, t, d, dt, prec, 0), dtype=torch.uint8,
                     device=q.device)
    status = lib.dil_forward(q.data_ptr(), k.data_ptr(), v.data_ptr(), n, t, d, dt, prec,
                             out.data_ptr(), stats[0].data_ptr(), stats[1].data_ptr(),
                             stats[2].data_ptr(), carry.data_ptr(), stats[3].data_ptr(), None,
                             ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    _hip.check(status, "dil_forward")
    return out, stats


@pytest.mark.parametrize("seq", [1, 65, 257, 1025])
def test_carry_future_triangle_unwritten_and_unread(seq):
    """The forward neither writes nor reads the carry checkpoints past each
    block's causal keys (the reference's hygiene check, test_kernels.py:21-43,
    143-149): a carry buffer poisoned with NaN gives bit-identical outputs,
    the causal part is written, and the future triangle still holds NaN."""
    q, k, v = (t.reshape(2, seq, 64).cuda() for t in
               orc.make_inputs((1, 2, seq, 64), seed=seq, dtype=torch.bfloat16))
    nb = (seq + 31) // 32
    clean = torch.zeros(2, nb, seq, device="cuda")
    poisoned = torch.full((2, nb, seq), float("nan"), device="cuda")
    out_a, st_a = _forward_into(q, k, v, clean)
    out_b, st_b = _forward_into(q, k, v, poisoned)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    for a, b in zip(st_a, st_b):
        assert torch.equal(a, b)
    rows = torch.arange(nb, device="cuda")[:, None]
    keys = torch.arange(seq, device="cuda")[None, :]
    future = (keys >= 32 * (rows + 1)).expand(2, nb, seq)
    assert torch.equal(poisoned[~future], clean[~future])
    assert torch.isnan(poisoned[future]).all()


def test_backward_ignores_carry_future_triangle():
    """The backward reads only the causal checkpoints: NaN written into the
    future triangle of the saved carry leaves every gradient bit-identical."""
    from dilution import kernels

    seq = 300
    q, k, v, do = orc.make_inputs((1, 2, seq, 64), seed=5, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    qg, kg, vg, dog = (t.cuda() for t in (q, k, v, do))
    out, aux = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16", return_aux=True,
                                                  _save_pk=True)
    saved = [qg, kg, vg, out, aux["rmax"], aux["rden"], aux["carry"], aux["ssum"], aux["pk"]]
    clean = kernels._backward(saved, dog, "bf16", kernels._PRODUCTION)
    nb = aux["carry"].shape[1]
    rows = torch.arange(nb, device="cuda")[:, None]
    keys = torch.arange(seq, device="cuda")[None, :]
    poisoned = aux["carry"].clone()
    poisoned[(keys >= 32 * (rows + 1)).expand_as(poisoned)] = float("nan")
    saved[6] = poisoned
    dirty = kernels._backward(saved, dog, "bf16", kernels._PRODUCTION)
    for a, b in zip(clean, dirty):
        assert torch.equal(a, b)


@pytest.mark.parametrize("head_dim", [16, 32, 64, 128])
def test_saved_query_correction_pk(head_dim):
    """pk = (p @ k) / sqrt(d) (reference test_kernels.py:46-59)."""
    from dilution import kernels

    q, k, v = orc.make_inputs((1, 2, 257, head_dim), seed=head_dim)
    _, aux = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), return_aux=True,
                                                _save_pk=True)
    assert max_abs(aux["pk"].reshape(1, 2, 257, head_dim), orc.pk(q, k)) < 2e-5


def test_row_chunked_forward_is_identical():
    """A tiny scratch budget forces one (batch, head) slice per launch; slices
    are independent, so the result is bit-identical."""
    from dilution import kernels

    q, k, v = orc.make_inputs((2, 3, 300, 64), seed=3, dtype=torch.bfloat16)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    a = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16")
    b = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16", scratch_budget_gib=1e-9)
    assert torch.equal(a, b)


def test_causality_prefix_bit_identical():
    from dilution import kernels

    q, k, v = orc.make_inputs((1, 2, 200, 64), seed=4, dtype=torch.bfloat16)
    a = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), dot_precision="bf16")
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[..., 130:, :] += 1
    k2[..., 130:, :] -= 1
    v2[..., 130:, :] *= 3
    b = kernels.dilution_attention_forward(q2.cuda(), k2.cuda(), v2.cuda(), dot_precision="bf16")
    assert torch.equal(a[..., :128, :], b[..., :128, :])


def test_harmonic_closed_form_on_gpu():
    """q = 0: every bid is 1/(i+1); the kernel output must equal the
    harmonic-number closed form."""
    from dilution import kernels
    import numpy as np

    t = 300
    g = torch.Generator().manual_seed(9)
    v = torch.randn(1, 2, t, 64, generator=g)
    k = torch.randn(1, 2, t, 64, generator=g)
    q = torch.zeros_like(v)
    out, aux = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), return_aux=True)
    cf, totals = orc.harmonic_closed_form(t, v.numpy())
    assert np.abs(out.double().cpu().numpy() - cf).max() < 1e-4
    assert np.abs(aux["committed_total"].double().cpu().numpy() - totals).max() < 1e-5


@pytest.mark.parametrize("prec,dtype,tol", [("ieee", torch.float32, 1e-4),
                                            ("bf16", torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("chunk", [32, 100, 256])
def test_chunked_prefill_matches_full_forward(prec, dtype, tol, chunk):
    from dilution import kernels

    batch, heads, seq, d = 2, 2, 600, 64
    q, k, v = orc.make_inputs((batch, heads, seq, d), seed=chunk, dtype=dtype)
    full = orc.attention_f64(q, k, v)
    cap = seq + 7
    kc = torch.zeros(batch, heads, cap, d, dtype=dtype, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:, :, :seq] = k.cuda()
    vc[:, :, :seq] = v.cuda()
    committed = torch.zeros(batch, heads, cap, device="cuda")
    for start in range(0, seq, chunk):
        stop = min(start + chunk, seq)
        out = kernels.dilution_prefill_chunk(q[:, :, start:stop].cuda(), kc, vc, committed, start,
                                             dot_precision=prec)
        assert max_abs(out, full[:, :, start:stop]) < tol, start
    assert max_abs(committed[:, :, :seq], orc.demand_totals(q, k)) < 1e-5
    assert committed[:, :, seq:].abs().max().item() == 0


def test_precision_argument_errors():
    from dilution import kernels

    q = torch.zeros(1, 1, 4, 64, device="cuda")
    with pytest.raises(ValueError):
        kernels.dilution_attention_forward(q, q, q, dot_precision="fp8")
    with pytest.raises(ValueError):
        x = torch.zeros(1, 1, 4, 48, device="cuda")
        kernels.dilution_attention_forward(x, x, x)


@pytest.mark.parametrize("seq", [1, 33, 257, 1000, 2048])
def test_forward_key_pass_matches_three_pass(seq, monkeypatch):
    """The key-parallel output pass (fwd_keyout + fwd_out_reduce, the default
    for these calls) against the three-pass forward (DILUTION_FORWARD_KEY_PASS=0)
    and the oracle: bf16 outputs at the bf16 bounds, the demand checkpoints
    (causal part), totals and row sums of shares within fp32 summation-order
    differences; gradients through it within the bf16 gradient bound."""
    from dilution import kernels

    q, k, v, do = orc.make_inputs((2, 4, seq, 64), seed=300 + seq, qk_scale=0.5, with_dout=True,
                                  dtype=torch.bfloat16)
    qg, kg, vg = (x.cuda() for x in (q, k, v))
    monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
    out0, aux0 = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16", return_aux=True,
                                                    _save_pk=True)
    monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS")
    out1, aux1 = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16", return_aux=True,
                                                    _save_pk=True)
    want = orc.attention_fp32(q, k, v)
    assert max_abs(out1, want) < 2e-2 and mean_rel(out1, want) < 1e-2
    assert max_abs(out1, out0) < 1e-2
    assert max_abs(aux1["committed_total"], aux0["committed_total"]) < 1e-5
    # the two passes add each key's demand in a different fp32 order, so a
    # share on a bf16 rounding boundary may round to the other neighbour: the
    # row sums of the bf16 shares then differ by a few bf16 steps of a share
    assert max_abs(aux1["ssum"], aux0["ssum"]) < 2e-2
    carry0 = aux0["carry"].reshape(2, 4, -1, seq)
    carry1 = aux1["carry"].reshape(2, 4, -1, seq)
    for rb in range(carry0.shape[2]):
        end = min(32 * (rb + 1), seq)
        assert max_abs(carry1[:, :, rb, :end], carry0[:, :, rb, :end]) < 1e-5, rb
    xs = [t.cuda().requires_grad_(True) for t in (q, k, v)]
    out = kernels.dilution_attention(*xs, dot_precision="bf16")
    out.backward(do.cuda())
    (dq, dk, dv), _ = orc.grads_closed_form_f64(*(t.double().numpy() for t in (q, k, v, do)))
    for name, g, w in zip(("dq", "dk", "dv"), (x.grad for x in xs), (dq, dk, dv)):
        assert max_abs(g, torch.from_numpy(w)) < 5e-2, name


@pytest.mark.parametrize("chunk", [512, 1536])
def test_prefill_chunks_through_the_key_pass(chunk, monkeypatch):
    """Prefill chunks that start at a multiple of 512 rows run the
    key-parallel output pass with the carried demand as its starting point
    (keys before the chunk meet every row tile of it).  Chunk after chunk,
    against the same chunks through the three-pass forward
    (DILUTION_FORWARD_KEY_PASS=0) and the fp64 oracle of the whole sequence:
    outputs within bf16 rounding (1e-2 of each other, 2e-2 of the oracle), the
    carried demand and the causal checkpoints within fp32 summation-order
    differences (1e-5 relative), the row sums of shares within a few bf16
    steps; the last chunk is ragged (3100 rows)."""
    from dilution import kernels

    batch, heads, seq, d = 2, 3, 3100, 64
    q, k, v = orc.make_inputs((batch, heads, seq, d), seed=chunk + 5, qk_scale=0.5, dtype=torch.bfloat16)
    full = orc.attention_f64(q, k, v)
    cap = seq + 40
    kc = torch.zeros(batch, heads, cap, d, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:, :, :seq] = k.cuda()
    vc[:, :, :seq] = v.cuda()
    com = {m: torch.zeros(batch, heads, cap, device="cuda") for m in ("key", "three")}
    for start in range(0, seq, chunk):
        stop = min(start + chunk, seq)
        res = {}
        for mode in ("three", "key"):
            if mode == "three":
                monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
            else:
                monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS", raising=False)
            res[mode] = kernels.dilution_prefill_chunk(q[:, :, start:stop].cuda(), kc, vc, com[mode], start,
                                                       dot_precision="bf16", return_aux=True)
        (o1, a1), (o0, a0) = res["key"], res["three"]
        assert max_abs(o1, full[:, :, start:stop]) < 2e-2, start
        assert mean_rel(o1, full[:, :, start:stop]) < 1e-2, start
        assert max_abs(o1, o0) < 1e-2, start
        assert max_abs(a1["ssum"], a0["ssum"]) < 2e-2, start
        t0, t1 = com["three"][:, :, :stop].double(), com["key"][:, :, :stop].double()
        assert ((t1 - t0).abs() / t0.abs().clamp(min=1.0)).max().item() < 1e-5, start
        c0 = a0["carry"].reshape(batch, heads, -1, stop).double()
        c1 = a1["carry"].reshape(batch, heads, -1, stop).double()
        for rb in range(c0.shape[2]):
            end = min(start + 32 * (rb + 1), stop)
            diff = ((c1[:, :, rb, :end] - c0[:, :, rb, :end]).abs() / c0[:, :, rb, :end].abs().clamp(min=1.0))
            assert diff.max().item() < 1e-5, (start, rb)
    assert max_abs(com["key"][:, :, :seq], orc.demand_totals(q, k)) < 1e-5 * 8
    assert com["key"][:, :, seq:].abs().max().item() == 0


@pytest.mark.parametrize("seq", [33, 1000, 2048])
def test_forward_without_aux_keeps_no_checkpoints(seq):
    """Without aux the key-parallel forward writes no demand checkpoints (the
    carry array is an output only, for the backward): its outputs are the
    same bits as the aux forward's.  The autograd forward with no input
    needing a gradient takes that path, and the three-pass forward ("ieee")
    still runs without aux (it keeps its own checkpoint scratch)."""
    from dilution import _hip, kernels

    assert _hip.lib().dil_forward_key_pass(seq, 0, 64, 1, 2) == 1
    q, k, v = orc.make_inputs((2, 3, seq, 64), seed=40 + seq, qk_scale=0.5, dtype=torch.bfloat16)
    qg, kg, vg = (x.cuda() for x in (q, k, v))
    ref, aux = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16", return_aux=True)
    plain = kernels.dilution_attention_forward(qg, kg, vg, dot_precision="bf16")
    assert torch.equal(plain, ref)
    assert torch.equal(kernels.dilution_attention(qg, kg, vg, dot_precision="bf16"), ref)
    with torch.no_grad():
        assert torch.equal(kernels.dilution_attention(qg, kg, vg, dot_precision="bf16"), ref)
    want = orc.attention_fp32(q, k, v)
    assert max_abs(plain, want) < 2e-2 and mean_rel(plain, want) < 1e-2
    f32 = [x.float() for x in (qg, kg, vg)]
    ieee = kernels.dilution_attention_forward(*f32, dot_precision="ieee")
    assert max_abs(ieee, orc.attention_f64(q.float(), k.float(), v.float())) < 1e-4


@pytest.mark.parametrize("chunk", [512, 700])
def test_prefill_chunk_without_aux_is_identical(chunk):
    """A prefill chunk without aux writes no checkpoints on the key pass
    (starts at multiples of 512) and keeps them as scratch on the three-pass
    forward (other starts): outputs and the carried demand are the same bits
    as with aux, chunk after chunk."""
    from dilution import kernels

    batch, heads, seq, d = 1, 4, 2100, 64
    q, k, v = orc.make_inputs((batch, heads, seq, d), seed=chunk, qk_scale=0.5, dtype=torch.bfloat16)
    kc = torch.zeros(batch, heads, seq, d, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:], vc[:] = k.cuda(), v.cuda()
    com = [torch.zeros(batch, heads, seq, device="cuda") for _ in range(2)]
    for start in range(0, seq, chunk):
        stop = min(start + chunk, seq)
        qc = q[:, :, start:stop].cuda()
        a, _ = kernels.dilution_prefill_chunk(qc, kc, vc, com[0], start, dot_precision="bf16", return_aux=True)
        b = kernels.dilution_prefill_chunk(qc, kc, vc, com[1], start, dot_precision="bf16")
        assert torch.equal(a, b), start
        assert torch.equal(com[0], com[1]), start
    assert max_abs(com[1], orc.demand_totals(q, k)) < 1e-5 * 8


@pytest.mark.parametrize("chunk", [100, 512])
def test_head_dim_256_prefill_and_aux(chunk):
    """head_dim 256 (bf16 operands, the three-pass forward): chunked prefill
    chunk after chunk against the fp64 oracle of the whole sequence (bf16
    bounds), the carried demand against the oracle's totals (1e-5 relative),
    and the aux forward's pk, totals and causal checkpoints against the
    oracle (pk within bf16 rounding of p and k)."""
    from dilution import kernels

    batch, heads, seq, d = 1, 2, 700, 256
    q, k, v = orc.make_inputs((batch, heads, seq, d), seed=chunk + 256, qk_scale=0.5, dtype=torch.bfloat16)
    full = orc.attention_f64(q, k, v)
    kc, vc = (x.cuda().contiguous() for x in (k, v))
    com = torch.zeros(batch, heads, seq, device="cuda")
    for start in range(0, seq, chunk):
        stop = min(start + chunk, seq)
        out = kernels.dilution_prefill_chunk(q[:, :, start:stop].cuda(), kc, vc, com, start, dot_precision="bf16")
        assert max_abs(out, full[:, :, start:stop]) < 2e-2, start
        assert mean_rel(out, full[:, :, start:stop]) < 1e-2, start
    tot = orc.demand_totals(q, k)
    assert ((com.cpu().double() - tot.double()).abs() / tot.double().abs().clamp(min=1.0)).max().item() < 1e-5
    out, aux = kernels.dilution_attention_forward(q.cuda(), k.cuda(), v.cuda(), dot_precision="bf16",
                                                  return_aux=True, _save_pk=True)
    assert max_abs(out, full) < 2e-2
    assert max_abs(aux["committed_total"], tot) < 1e-5 * 8
    assert max_abs(aux["pk"].reshape(batch, heads, seq, d), orc.pk(q, k)) < 2e-2
    carry = aux["carry"].reshape(batch, heads, -1, seq)
    want = orc.carry_checkpoints(q, k, 32)
    for rb in range(carry.shape[2]):
        end = min(32 * (rb + 1), seq)
        assert max_abs(carry[:, :, rb, :end], want[:, :, rb, :end]) < 1e-5 * 8, rb
