"""Dilution attention with a selectable bid function and share step, on MI355X.

Drop-in for the reference module ``dilution.kernels_bid``
(/root/reference/src/dilution/kernels_bid.py), the operator family of its bid
and share ablations (configs/bid_8192/*).  Same public names and signatures;
every launch goes to the HIP kernels of ``libdilution_hip.so``, compiled per
(bid, share) as template variants of the production kernels
(``dil_variants.hip``, head_dim 16, 32, 64 or 128, as the production operator).

Bids, with a = q.k / sqrt(d) on the causal window (kernels_bid.py:4-42):

    softmax   p = softmax(a)                    relu      p = relu(a) / rowsum
    relu2     p = relu(a)^2 / rowsum            softplus  p = softplus(a) / rowsum
    minshift  p = (a - min a) / rowsum          sigmoid   p = sigmoid(a)
    expshift  p = exp(a) / SHIFT                sigshift  p = 1 / (1 + SHIFT e^-a)

A row with no mass under relu / relu2 / softplus / minshift bids uniformly over
its window.  ``share_cumsum``: True -> p / (committed + p + eps) (dilution),
"exclusive" -> p / (committed + eps), False -> p (no share step); the shares
are then row-normalised and multiply V.  ``bid="softmax", share_cumsum=True``
is the production operator of ``dilution.kernels`` and runs its kernels.
"""

from __future__ import annotations

import math

import torch

from . import kernels as _k

HAS_HIP = _k.HAS_HIP

BID_TYPES = ("softmax", "relu", "relu2", "softplus", "minshift", "sigmoid", "expshift", "sigshift")

VARIANT_HEAD_DIMS = (16, 32, 64, 128)
"""head dims the ablation variants are built for (the production operator's in
every precision; it also takes 256 with bf16 operands, the variants do not)."""


def head_dim_supported(head_dim: int) -> bool:
    """Whether the variant kernels take this head width (16, 32, 64 or 128)."""
    return int(head_dim) in VARIANT_HEAD_DIMS


def _bid_code(bid: str) -> int:
    if bid not in BID_TYPES:
        raise ValueError(f"bid must be one of {BID_TYPES}")
    return BID_TYPES.index(bid)


def _share_code(share_cumsum) -> int:
    """True/1 -> inclusive dilution, "exclusive" -> history only, False/0 -> none
    (kernels_bid.py:123-127)."""
    if share_cumsum == "exclusive":
        return 2
    return int(bool(share_cumsum))


def _variant(bid: str, share_cumsum, shift: float, head_dim: int) -> tuple:
    code = (_bid_code(bid), _share_code(share_cumsum), float(shift))
    if not shift > 0:
        raise ValueError("shift must be positive")
    if head_dim not in VARIANT_HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {VARIANT_HEAD_DIMS}, got {head_dim}")
    return code


# numerators of the ratio bids (normalised by their row sum over the window)
_RATIO_NUMERATORS = {
    "relu": torch.relu,
    "relu2": lambda a: torch.relu(a).square(),
    "softplus": torch.nn.functional.softplus,
}


def bids_from_affinity(aff: torch.Tensor, causal: torch.Tensor, bid: str, shift: float = 1.0) -> torch.Tensor:
    """p from scaled affinities under the selected bid function, in plain
    torch (the behaviour of kernels_bid.py:94-121).  ``causal`` marks the
    visible keys; ``shift`` divides expshift and offsets sigshift."""
    _bid_code(bid)
    zero = torch.zeros((), dtype=aff.dtype, device=aff.device)
    if bid == "softmax":
        return torch.softmax(torch.where(causal, aff, torch.finfo(aff.dtype).min), dim=-1)
    if bid in ("sigmoid", "sigshift"):
        offset = math.log(float(shift)) if bid == "sigshift" else 0.0
        return torch.where(causal, torch.sigmoid(aff - offset), zero)
    if bid == "expshift":
        return torch.where(causal, torch.exp(aff) / float(shift), zero)
    if bid == "minshift":
        floor = torch.where(causal, aff, torch.inf).amin(dim=-1, keepdim=True).detach()
        num = aff - floor
    else:
        num = _RATIO_NUMERATORS[bid](aff)
    num = torch.where(causal, num, zero)
    mass = num.sum(dim=-1, keepdim=True)
    flat = causal.to(aff.dtype) / causal.sum(dim=-1, keepdim=True).to(aff.dtype)
    return torch.where(mass > 0, num / mass.clamp_min(1e-30), flat)


def dilution_attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bid: str = "softmax",
                                 share_cumsum=True, shift: float = 1.0) -> torch.Tensor:
    """The operator variant written plainly in fp32 torch (the behaviour of
    kernels_bid.py:130-165): the specification the kernels are tested
    against, not a kernel fallback."""
    seq, head_dim = q.shape[-2], q.shape[-1]
    aff = torch.matmul(q.float(), k.float().transpose(-1, -2)) * head_dim ** -0.5
    causal = torch.ones(seq, seq, dtype=torch.bool, device=q.device).tril()
    p = bids_from_affinity(aff, causal, bid, shift)
    mode = _share_code(share_cumsum)
    if mode == 0:
        weights = p / p.sum(dim=-1, keepdim=True)
    else:
        before = p.cumsum(dim=-2) - p                     # demand of the earlier queries
        shares = p / (before + 1e-9) if mode == 2 else p / (before + p + 1e-9)
        weights = shares / (shares.sum(dim=-1, keepdim=True) + 1e-9)
    return torch.matmul(weights, v.float())


def dilution_attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dot_precision: str = "ieee",
    block_m: int = 64,
    block_n: int = 64,
    return_aux: bool = False,
    num_warps: int = 4,
    num_stages: int = 2,
    bid: str = "softmax",
    share_cumsum=True,
    shift: float = 1.0,
):
    """Fused forward of the variant; returns fp32 outputs (kernels_bid.py:424-489).

    return_aux adds the reference's aux keys (``rmax, rden, carry, ssum,
    committed_total`` ...) plus ``bid, share_cumsum, shift``.  For the ratio
    bids rmax holds 0 (the row minimum for minshift) and rden the row sum of
    the numerators; for the elementwise bids rmax = 0 and rden = 1 (SHIFT for
    expshift), as in the reference.
    """
    variant = _variant(bid, share_cumsum, shift, q.shape[-1])
    res = _k.dilution_attention_forward(q, k, v, dot_precision=dot_precision, block_m=block_m,
                                        block_n=block_n, return_aux=return_aux, num_warps=num_warps,
                                        num_stages=num_stages, _variant=variant)
    if return_aux:
        out, aux = res
        aux.update(bid=bid, share_cumsum=share_cumsum, shift=shift)
        return out, aux
    return res


class _DilutionAttentionFn(torch.autograd.Function):
    """Forward + backward of the variant on the HIP kernels (kernels_bid.py:731-815);
    the same 15 positional arguments as the reference, tuning ones ignored."""

    @staticmethod
    def forward(ctx, q, k, v, dot_precision, block_m, block_n, num_warps, bwd_num_warps,
                bwd_num_stages, b3_block_n, b3_num_warps, b4_num_warps, bid, share_cumsum, shift):
        variant = _variant(bid, share_cumsum, shift, q.shape[-1])
        out, aux = _k.dilution_attention_forward(
            q, k, v, dot_precision=dot_precision, return_aux=True,
            _save_pk=any(ctx.needs_input_grad[:3]), _variant=variant)
        ctx.save_for_backward(q, k, v, out, aux["rmax"], aux["rden"], aux["carry"], aux["ssum"],
                              aux["pk"])
        ctx.dot_precision = dot_precision
        ctx.variant = variant
        return out

    @staticmethod
    def backward(ctx, dout):
        grads = _k._backward(ctx.saved_tensors, dout, ctx.dot_precision, ctx.variant)
        return (*grads,) + (None,) * 12


def dilution_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dot_precision: str = "bf16",
    block_m: int = 64,
    block_n: int = 64,
    num_warps: int = 4,
    bwd_num_warps: int = 4,
    bwd_num_stages: int = 1,
    b3_block_n: int | None = None,
    b3_num_warps: int | None = None,
    b4_num_warps: int | None = 4,
    bid: str = "softmax",
    share_cumsum=True,
    shift: float = 1.0,
) -> torch.Tensor:
    """Differentiable fused variant (kernels_bid.py:818-846)."""
    return _DilutionAttentionFn.apply(q, k, v, dot_precision, block_m, block_n, num_warps,
                                      bwd_num_warps, bwd_num_stages, b3_block_n, b3_num_warps,
                                      b4_num_warps, bid, share_cumsum, shift)


def dilution_decode_step(
    q1: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    committed: torch.Tensor,
    length: int,
    block_n: int = 512,
    num_warps: int = 8,
    bid: str = "softmax",
    share_cumsum=True,
    shift: float = 1.0,
) -> torch.Tensor:
    """Fused decode step of the variant (kernels_bid.py:962-1010): the new row's
    output (B, H, 1, D) in q1.dtype; ``committed`` advances by p in place in
    every share mode (kernels_bid.py:955)."""
    variant = _variant(bid, share_cumsum, shift, q1.shape[-1])
    return _k.dilution_decode_step(q1, k_cache, v_cache, committed, length, block_n=block_n,
                                   num_warps=num_warps, _variant=variant)
