"""Prefill -> decode hand-off through the cache dict (dilution.cache).

Reference patterns: tests/test_kernels.py:205-273 (decode rows equal the
full-sequence rows, the demand vector equals the column sums, spare capacity
untouched) and tests/test_model.py:99-110 (cached decode == teacher-forced
full forward).  Here the prompt is prefilled in chunks (the C4 pattern, at a
small size), then decoded token by token, and every row is compared with the
float64 oracle of the whole sequence.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import max_abs, needs_gpu
from oracle import dilution_oracle as orc


def test_cache_requires_gpu_tensors():
    from dilution import cache as dc

    q = torch.zeros(1, 1, 4, 64)
    with pytest.raises(RuntimeError):
        dc.begin_cache(q, q, q)


def test_alloc_and_append_follow_the_reference_protocol():
    """Capacity rule max(capacity, T) and the error past capacity
    (model.py:76-93) are host logic: checked on CPU tensors."""
    from dilution import cache as dc

    k = torch.randn(1, 2, 5, 8)
    c = dc.alloc_cache(k, k, capacity=3)
    assert c["k"].shape[2] == 5 and c["len"] == 5 and c["committed"].dtype == torch.float32
    c = dc.alloc_cache(k, k, capacity=7)
    assert c["k"].shape[2] == 7
    one = torch.randn(1, 2, 1, 8)
    assert dc.append_kv(c, one, one) == 6
    assert torch.equal(c["k"][:, :, 5], one[:, :, 0])
    dc.append_kv(c, one, one)
    with pytest.raises(ValueError):
        dc.append_kv(c, one, one)


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("chunk", [None, 96, 256])
def test_chunked_prefill_then_decode_matches_full_rows(dtype, tol, chunk):
    """The cache prefills with the model's precision rule (model.py:203):
    bf16 operands for bf16 activations, "tf32" otherwise.  Split bf16
    operands ("tf32") leave p about 2^-17 relative off, so the fp32 demand
    totals (up to ~8 here) are held to 1e-5 of their magnitude; the bf16
    operands of bf16 inputs give exact products and keep 1e-5 absolute."""
    from dilution import cache as dc

    batch, heads, d, prompt, steps = 2, 4, 64, 600, 12
    total = prompt + steps
    q, k, v = orc.make_inputs((batch, heads, total, d), seed=31 + (chunk or 0))
    q, k, v = (x.to(dtype) for x in (q, k, v))
    full = orc.attention_f64(q, k, v)                   # oracle on the same (rounded) values
    qg, kg, vg = (x.cuda() for x in (q, k, v))
    y, cache = dc.begin_cache(qg[:, :, :prompt], kg[:, :, :prompt], vg[:, :, :prompt],
                              capacity=total + 5, chunk=chunk)
    assert y.dtype == dtype and cache["len"] == prompt
    assert max_abs(y, full[:, :, :prompt]) < tol
    want = orc.demand_totals(q[:, :, :prompt], k[:, :, :prompt])
    dtol = 1e-5 * (1.0 if dtype == torch.bfloat16 else max(1.0, float(want.abs().max())))
    assert max_abs(cache["committed"][:, :, :prompt], want) < dtol
    for t in range(prompt, total):
        out = dc.step_cache(qg[:, :, t:t + 1], kg[:, :, t:t + 1], vg[:, :, t:t + 1], cache)
        assert out.dtype == dtype
        assert max_abs(out[:, :, 0], full[:, :, t]) < tol, t
    assert max_abs(cache["committed"][:, :, :total], orc.demand_totals(q, k)) < dtol
    assert cache["committed"][:, :, total:].abs().max().item() == 0
    assert cache["len"] == total


@pytest.mark.gpu
@needs_gpu
def test_chunked_and_one_call_prefill_agree():
    """Chunked prefill reproduces the reference's one-call prefill: the same
    outputs (fp32 rounding apart) and the same demand buffer."""
    from dilution import cache as dc

    q, k, v = (x.cuda() for x in orc.make_inputs((1, 3, 777, 64), seed=41))
    y1, c1 = dc.begin_cache(q, k, v, capacity=800, dot_precision="ieee")
    y2, c2 = dc.begin_cache(q, k, v, capacity=800, chunk=100, dot_precision="ieee")
    assert max_abs(y1, y2) < 1e-5
    assert max_abs(c1["committed"], c2["committed"]) < 1e-5
    assert torch.equal(c1["k"], c2["k"]) and torch.equal(c1["v"], c2["v"])


@pytest.mark.gpu
@needs_gpu
def test_unwritten_cache_positions_are_never_read():
    """Cache rows past what is written (prefill: past start + C; decode: past
    length) and the demand past length hold NaN: outputs and demand are
    bit-identical to a clean cache, and the poisoned tail is left as it was
    (the reference's future-triangle poisoning, test_kernels.py:19-43)."""
    from dilution import kernels

    b, h, d, cap, chunk = 2, 3, 64, 96, 40
    q, k, v = (t.cuda() for t in orc.make_inputs((b, h, cap, d), seed=51))
    outs = []
    for poison in (False, True):
        kc, vc = torch.zeros_like(k), torch.zeros_like(v)
        com = torch.zeros(b, h, cap, device="cuda")
        if poison:
            kc.fill_(float("nan"))
            vc.fill_(float("nan"))
            com[..., chunk:] = float("nan")
        kc[:, :, :chunk] = k[:, :, :chunk]
        vc[:, :, :chunk] = v[:, :, :chunk]
        y = kernels.dilution_prefill_chunk(q[:, :, :chunk], kc, vc, com, 0, dot_precision="ieee")
        t = chunk + 1
        kc[:, :, t - 1] = k[:, :, t - 1]
        vc[:, :, t - 1] = v[:, :, t - 1]
        com[..., t - 1] = 0.0
        y1 = kernels.dilution_decode_step(q[:, :, t - 1:t].contiguous(), kc, vc, com, t)
        outs.append((y, y1, com.clone()))
    (y0, d0, c0), (y1, d1, c1) = outs
    assert torch.equal(y0, y1) and torch.equal(d0, d1)
    assert torch.equal(c0[..., :chunk + 1], c1[..., :chunk + 1])
    assert torch.isnan(c1[..., chunk + 1:]).all()
