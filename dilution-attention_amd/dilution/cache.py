"""Prefill -> decode state hand-off on the HIP kernels.

The reference keeps the decode state of one attention layer in a dict
``{"k", "v", "len", "committed"}``:

* k / v: ``(B, H, capacity, D)`` buffers allocated once and filled by slice
  assignment (src/dilution/model.py:76-83, ``_alloc_cache``);
* len: the number of valid positions;
* committed: the ``(B, H, capacity)`` fp32 demand -- column totals of the
  bids over every row seen so far (model.py:224-228).

``begin_cache`` prefills a prompt (model.py:198-229) and ``step_cache`` runs
one decode token (model.py:231-241, the kernel branch), with the same dict, the
same capacity rule (``max(capacity, prompt length)``, model.py:79) and the same
error past capacity (model.py:88-89).  Unlike the reference, which prefills the
whole prompt in one forward call, ``begin_cache(..., chunk=C)`` prefills it in
chunks of C rows through ``dilution_prefill_chunk``, writing K/V and the
demand straight into the cache buffers; with ``chunk=None`` it runs the
one-call forward as the reference does.  Both give the same outputs and demand.

The ablation variants (``bid`` / ``share_cumsum`` / ``shift`` keywords, the
operators of ``kernels_bid``) prefill in one call and decode through the
variant decode step (model.py:198-241 with ``_bid_kw``).
"""

from __future__ import annotations

import torch

from . import kernels
from . import kernels_bid


def _precision(dtype: torch.dtype) -> str:
    # model.py:203: bf16 activations use bf16 operands, anything else tf32
    return "bf16" if dtype == torch.bfloat16 else "tf32"


def alloc_cache(k: torch.Tensor, v: torch.Tensor, capacity: int | None = None) -> dict:
    """Cache buffers holding k, v (B, H, T, D) in positions [0, T) of a
    capacity of ``max(capacity, T)`` (model.py:76-83), with a zero demand."""
    batch, heads, seq, head_dim = k.shape
    capacity = max(capacity if capacity is not None else seq, seq)
    k_buf = k.new_zeros(batch, heads, capacity, head_dim)
    v_buf = v.new_zeros(batch, heads, capacity, head_dim)
    k_buf[:, :, :seq] = k
    v_buf[:, :, :seq] = v
    committed = torch.zeros(batch, heads, capacity, device=k.device, dtype=torch.float32)
    return {"k": k_buf, "v": v_buf, "len": seq, "committed": committed}


def append_kv(cache: dict, k1: torch.Tensor, v1: torch.Tensor) -> int:
    """Write one new position (k1, v1: (B, H, 1, D)) and return the new
    length (model.py:86-93)."""
    t = cache["len"]
    if t >= cache["k"].shape[2]:
        raise ValueError("decode step past the cache capacity (context_length)")
    cache["k"][:, :, t] = k1[:, :, 0]
    cache["v"][:, :, t] = v1[:, :, 0]
    cache["len"] = t + 1
    return t + 1


def begin_cache(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, capacity: int | None = None,
                chunk: int | None = None, dot_precision: str | None = None, **bid_kw):
    """Prefill a prompt: returns (y, cache) with y (B, H, T, D) in q.dtype.

    chunk=None runs the one-call forward and copies ``committed_total`` into
    the cache (model.py:202-228); chunk=C prefills C rows at a time with the
    demand carried in the cache's buffer.  ``bid_kw`` (bid, share_cumsum,
    shift) selects an ablation variant, always prefilled in one call.
    """
    prec = dot_precision or _precision(q.dtype)
    seq = q.shape[2]
    cache = alloc_cache(k, v, capacity)
    if bid_kw:
        y, aux = kernels_bid.dilution_attention_forward(q, k, v, dot_precision=prec, return_aux=True,
                                                        **bid_kw)
        cache["committed"][:, :, :seq] = aux["committed_total"]
        return y.to(q.dtype), cache
    if chunk is None:
        y, aux = kernels.dilution_attention_forward(q, k, v, dot_precision=prec, return_aux=True)
        cache["committed"][:, :, :seq] = aux["committed_total"]
        return y.to(q.dtype), cache
    if chunk < 1:
        raise ValueError("chunk must be positive")
    outs = []
    for start in range(0, seq, chunk):
        stop = min(start + chunk, seq)
        outs.append(kernels.dilution_prefill_chunk(q[:, :, start:stop], cache["k"], cache["v"],
                                                   cache["committed"], start, dot_precision=prec))
    return torch.cat(outs, dim=2).to(q.dtype), cache


def step_cache(q1: torch.Tensor, k1: torch.Tensor, v1: torch.Tensor, cache: dict, **bid_kw) -> torch.Tensor:
    """One decode token: append (k1, v1) and return the new row's output
    (B, H, 1, D) in q1.dtype, advancing the cache's demand in place
    (model.py:231-241); ``bid_kw`` as in ``begin_cache``."""
    t = append_kv(cache, k1, v1)
    if bid_kw:
        return kernels_bid.dilution_decode_step(q1, cache["k"], cache["v"], cache["committed"], t, **bid_kw)
    return kernels.dilution_decode_step(q1, cache["k"], cache["v"], cache["committed"], t)
