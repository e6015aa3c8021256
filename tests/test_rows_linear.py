"""The decode step's few-row projections (dilution.lm.rows_linear, C ABI
dil_rows_linear) against the unfused torch ops they replace, and the LM's
decode step on them against the same step on torch's modules.

The kernel accumulates its dot products in fp32 in another order than
torch's GEMM, and rounds the same intermediates to bf16, so the bar is a
bf16-rounding bound, not bitwise.  An identity weight isolates the RMSNorm
stage: each output is then one staged, normalised activation (a dot product
with a single 1.0), which must equal torch's rms_norm to within one bf16 step
(the row's sum of squares is added in another order).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gpu_helpers import needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]


def _bf(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16).cuda()


def _check_close(out, ref, what):
    out, ref = out.float(), ref.float()
    err = (out - ref).abs()
    peak = ref.abs().max().item()
    # a few bf16 roundings of values up to `peak`, plus fp32 order effects
    assert err.max().item() <= 2.0 ** -6 * peak + 1e-6, (what, err.max().item(), peak)
    assert err.mean().item() <= 2.0 ** -8 * ref.abs().mean().item() + 1e-6, (what, err.mean().item())


@pytest.mark.parametrize("rows", [1, 5, 8])
@pytest.mark.parametrize("n,k", [(40, 256), (1000, 1024), (3072, 1024), (1024, 4096), (9000, 1024), (600, 2048),
                                 (2048, 1536), (8192, 4096)])
def test_plain_and_residual_match_torch(rows, n, k):
    from dilution.lm import rows_linear

    gen = torch.Generator().manual_seed(rows * 7 + n + k)
    x = _bf(rows, k, gen=gen)
    w = _bf(n, k, gen=gen, scale=0.02)
    resid = _bf(rows, n, gen=gen)
    _check_close(rows_linear(x, w, 0), F.linear(x, w), ("plain", rows, n, k))
    _check_close(rows_linear(x, w, 1, resid=resid), resid + F.linear(x, w), ("resid", rows, n, k))


@pytest.mark.parametrize("rows", [2, 8])
@pytest.mark.parametrize("n,k", [(3072, 1024), (50304, 1024), (64, 256), (1000, 2048), (5000, 4096), (9000, 3072)])
def test_norm_projection_matches_torch(rows, n, k):
    from dilution.lm import rows_linear

    gen = torch.Generator().manual_seed(rows + n)
    x = _bf(rows, k, gen=gen, scale=3.0)
    g = (1.0 + 0.1 * torch.randn(k, generator=gen)).to(torch.bfloat16).cuda()
    w = _bf(n, k, gen=gen, scale=0.02)
    ref = F.linear(F.rms_norm(x, (k,), g, 1e-5), w)
    _check_close(rows_linear(x, w, 2, g=g, eps=1e-5), ref, ("norm", rows, n, k))


@pytest.mark.parametrize("rows", [3, 8])
def test_norm_stage_equals_rms_norm(rows):
    """Identity weight: out = the staged rmsnorm(x) * g, within one bf16 step
    of torch's rms_norm, and equal to it almost everywhere (both round
    x / rms(x) * g once; the sum of squares is added in another order)."""
    from dilution.lm import rows_linear

    k = 1024
    gen = torch.Generator().manual_seed(rows)
    x = _bf(rows, k, gen=gen, scale=2.0)
    g = (1.0 + 0.3 * torch.randn(k, generator=gen)).to(torch.bfloat16).cuda()
    eye = torch.eye(k, dtype=torch.bfloat16, device="cuda")
    out = rows_linear(x, eye, 2, g=g, eps=1e-5).float()
    ref = F.rms_norm(x, (k,), g, 1e-5).float()
    ulp = ref.abs().clamp_min(1e-30) * 2.0 ** -7
    assert bool(((out - ref).abs() <= ulp).all())
    assert (out == ref).float().mean().item() > 0.95


@pytest.mark.parametrize("rows", [1, 8])
@pytest.mark.parametrize("n,k", [(4096, 1024), (1000, 1024), (2048, 4096)])
def test_swiglu_matches_torch(rows, n, k):
    from dilution.lm import rows_linear

    gen = torch.Generator().manual_seed(rows + n + 1)
    x = _bf(rows, k, gen=gen)
    g = (1.0 + 0.1 * torch.randn(k, generator=gen)).to(torch.bfloat16).cuda()
    w1 = _bf(n, k, gen=gen, scale=0.05)
    w2 = _bf(n, k, gen=gen, scale=0.05)
    r = F.rms_norm(x, (k,), g, 1e-5)
    ref = F.silu(F.linear(r, w1)) * F.linear(r, w2)
    _check_close(rows_linear(x, w1, 3, w2=w2, g=g, eps=1e-5), ref, ("swiglu", rows, n))


def test_rows_past_the_batch_are_untouched():
    """out has exactly `rows` rows: a poisoned buffer around a view is not written."""
    from dilution import _hip
    from dilution.lm import rows_linear  # noqa: F401  (loads the library)

    gen = torch.Generator().manual_seed(3)
    x = _bf(3, 256, gen=gen)
    w = _bf(48, 256, gen=gen, scale=0.1)
    buf = torch.full((5, 48), float("nan"), dtype=torch.bfloat16, device="cuda")
    out = buf[1:4]
    status = _hip.lib().dil_rows_linear(x.data_ptr(), w.data_ptr(), None, None, None, out.data_ptr(),
                                        3, 48, 256, 0, 1, 0.0, torch.cuda.current_stream().cuda_stream)
    assert status == 0
    torch.cuda.synchronize()
    assert bool(torch.isnan(buf[0]).all()) and bool(torch.isnan(buf[4]).all())
    _check_close(out, F.linear(x, w), "view")


@pytest.mark.parametrize("rows,heads", [(1, 16), (8, 16), (8, 32), (3, 64)])
@pytest.mark.parametrize("device_pos", [False, True])
def test_qkv_projection_writes_the_cache_row(rows, heads, device_pos):
    """rows_linear_qkv: q = the first third of rmsnorm(x) W^T; the k and v
    thirds land in row `pos` of the (B, H, capacity, D) caches, every other
    cache row untouched.  d_model 1024, 2048 and 4096 (N = 3 d_model from
    12288 takes the one-row-per-lane-group form)."""
    from dilution.lm import rows_linear_qkv

    hd, cap, pos = 64, 40, 17
    d = heads * hd
    gen = torch.Generator().manual_seed(rows + heads + 40)
    x = _bf(rows, d, gen=gen, scale=2.0)
    g = (1.0 + 0.1 * torch.randn(d, generator=gen)).to(torch.bfloat16).cuda()
    w = _bf(3 * d, d, gen=gen, scale=0.02)
    kc = _bf(rows, heads, cap, hd, gen=gen)
    vc = _bf(rows, heads, cap, hd, gen=gen)
    k0, v0 = kc.clone(), vc.clone()
    p = torch.tensor([pos], dtype=torch.int64, device="cuda") if device_pos else pos
    q = rows_linear_qkv(x, w, g, 1e-5, kc, vc, p)
    ref = F.linear(F.rms_norm(x, (d,), g, 1e-5), w)
    _check_close(q, ref[:, :d], ("q", rows))
    _check_close(kc[:, :, pos], ref[:, d:2 * d].view(rows, heads, hd), ("k", rows))
    _check_close(vc[:, :, pos], ref[:, 2 * d:].view(rows, heads, hd), ("v", rows))
    keep = torch.ones(cap, dtype=torch.bool)
    keep[pos] = False
    assert torch.equal(kc[:, :, keep], k0[:, :, keep]) and torch.equal(vc[:, :, keep], v0[:, :, keep])
    # the same product as the plain norm projection, bitwise (same kernel body)
    from dilution.lm import rows_linear
    full = rows_linear(x, w, 2, g=g, eps=1e-5)
    assert torch.equal(q, full[:, :d])
    assert torch.equal(kc[:, :, pos], full[:, d:2 * d].view(rows, heads, hd))


def test_qkv_device_position_outside_the_cache_stores_no_row():
    from dilution.lm import rows_linear_qkv

    heads, hd, cap, rows = 4, 64, 8, 3
    d = heads * hd
    gen = torch.Generator().manual_seed(7)
    x = _bf(rows, d, gen=gen)
    g = torch.ones(d, dtype=torch.bfloat16, device="cuda")
    w = _bf(3 * d, d, gen=gen, scale=0.05)
    kc = _bf(rows, heads, cap, hd, gen=gen)
    vc = _bf(rows, heads, cap, hd, gen=gen)
    k0, v0 = kc.clone(), vc.clone()
    for bad in (cap, -1):
        q = rows_linear_qkv(x, w, g, 1e-5, kc, vc, torch.tensor([bad], dtype=torch.int64, device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(kc, k0) and torch.equal(vc, v0), bad
        _check_close(q, F.linear(F.rms_norm(x, (d,), g, 1e-5), w)[:, :d], "q")


@pytest.mark.parametrize("rows,vocab,limit,offset", [(1, 50304, None, 0), (8, 50304, 50000, 0), (3, 1000, 999, 0),
                                                     (8, 4099, None, 0), (2, 64, 7, 3)])
def test_rows_argmax_is_torch_argmax(rows, vocab, limit, offset):
    """dil_rows_argmax against torch.argmax over the first `limit` logits:
    random rows, rows with a repeated maximum (the first index wins), a row
    whose maximum lies past the limit, a row with a NaN, and an unaligned
    view (offset columns: the scalar path)."""
    from dilution.lm import rows_argmax

    gen = torch.Generator().manual_seed(rows + vocab)
    full = _bf(rows, vocab + offset, gen=gen, scale=3.0)
    lg = full[:, offset:]
    lim = vocab if limit is None else limit
    if rows > 1:
        lg[1, 5] = lg[1, lim - 2] = 100.0                     # a tie: index 5 wins
    if rows > 2:
        lg[2, :] = -1.0
        lg[2, lim - 1] = float("nan")                          # a NaN counts as the largest
    if lim < vocab:
        lg[0, vocab - 1] = 1000.0                              # past the limit: ignored
    got = rows_argmax(lg, limit)
    want = lg[:, :lim].float().argmax(dim=-1, keepdim=True)
    assert torch.equal(got, want), (got.flatten().tolist(), want.flatten().tolist())
    if rows > 1:
        assert got[1, 0].item() == 5


def _lm():
    from dilution.lm import DilutionLM, LMConfig

    cfg = LMConfig(vocab_size=1000, n_layers=2, d_model=256, n_heads=4, prefill_chunk=32)
    torch.manual_seed(0)
    return DilutionLM(cfg).to(device="cuda", dtype=torch.bfloat16).eval()


def _clone_caches(caches):
    return [{key: (val.clone() if torch.is_tensor(val) else val) for key, val in c.items()} for c in caches]


def test_fused_decode_step_matches_torch_modules():
    """The bf16 decode step on rows_linear against the same step on torch's
    modules from the same caches, several steps in a row: logits within the
    bf16 bound of the last layer's inputs, identical caches growth."""
    model = _lm()
    assert model.fused_decode_eligible(3) and not model.fused_decode_eligible(9)
    gen = torch.Generator().manual_seed(11)
    idx = torch.randint(0, 1000, (3, 45), generator=gen).cuda()
    logits, caches_f = model.prefill(idx, capacity=45 + 6)
    caches_t = _clone_caches(caches_f)
    tok = logits[:, -1, :].float().argmax(dim=-1, keepdim=True)
    for step in range(6):
        lf = model.decode_step(tok, caches_f)
        lt = model.decode_step(tok, caches_t, fused=False)
        assert lf.shape == lt.shape == (3, 1, 1000)
        err = (lf.float() - lt.float()).abs().max().item()
        assert err <= 3e-2 * lt.float().abs().max().item(), (step, err)
        tok = lt[:, -1, :].float().argmax(dim=-1, keepdim=True)
    for cf, ct in zip(caches_f, caches_t):
        assert cf["len"] == ct["len"] == 45 + 6


def test_graph_decode_runs_fused_and_matches_eager_fused():
    """GraphDecoder on a fused-eligible model replays the fused step: every
    replay bitwise equal to the eager fused step (same kernels, same order)."""
    from dilution.lm import GraphDecoder

    model = _lm()
    gen = torch.Generator().manual_seed(12)
    idx = torch.randint(0, 1000, (2, 40), generator=gen).cuda()
    logits_e, caches_e = model.prefill(idx, capacity=48)
    _, caches_g = model.prefill(idx, capacity=48)
    tok = logits_e[:, -1, :].float().argmax(dim=-1, keepdim=True)
    dec = GraphDecoder(model, caches_g, tok)
    assert dec.fused
    for step in range(8):
        le = model.decode_step(tok, caches_e)
        tg = dec.step()
        torch.cuda.synchronize()
        assert torch.equal(dec.logits, le), step
        tok = le[:, -1, :].float().argmax(dim=-1, keepdim=True)
        assert torch.equal(tg, tok), step
