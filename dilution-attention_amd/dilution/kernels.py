"""Dilution attention on MI355X (gfx950): reference, training, prefill and decode.

Drop-in for the reference module ``dilution.kernels``
(/root/reference/src/dilution/kernels.py).  The public functions keep the
reference signatures; behind them every launch goes to the hand-written HIP
kernels of ``libdilution_hip.so`` through its C ABI (include/dilution_hip.h).
There is no Triton and no CPU fallback: when the library cannot be loaded, or
the tensors are not on the GPU, the entry points raise.

    p         = causal_softmax(q k^T / sqrt(d))   # bids
    committed = exclusive_cumsum_cols(p)          # taken by earlier queries
    share     = p / (committed + p + eps)         # bid vs cumulative demand
    A         = share / rowsum(share);  out = A @ v

Kernel decomposition (csrc/): a row-statistics pass (row max, 2^-sum and the
saved p @ k), a key-parallel demand walk that writes the demand entering every
32-row block and the per-key totals (fp64 running sums), an output pass with
the in-tile demand scan on registers, the matching backward (a reverse
key-parallel walk for dv, dk and the demand adjoint, a row-parallel dq pass,
and the softmax-Jacobian correction of dk), and a split-K decode step.  Tuning
arguments of the Triton reference (block sizes, warps, stages) are accepted
and ignored: tiles are fixed for gfx950.
"""

from __future__ import annotations

import contextlib
import math

import torch

from . import _hip

HAS_HIP = _hip.available()
"""True when libdilution_hip.so is built and loadable (the test gate)."""

# The reference switches training above this length to its key-parallel
# forward (kernels.py:71-76).  Here one decomposition serves every length; the
# constant is kept so callers that read it keep working.
KEY_FORWARD_MIN_SEQ = 256

# Rows per demand checkpoint (aux["carry"] granularity, aux["bwd_block_m"]).
CHECKPOINT_ROWS = 32

_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
# operator variant (bid code, share code, shift); the production operator is
# softmax bids with the dilution share (the ablation variants are reached
# through dilution.kernels_bid)
_PRODUCTION = (0, 1, 1.0)
_PRECISIONS = {"ieee": 0, "tf32": 1, "bf16": 2}
_HEAD_DIMS = (16, 32, 64, 128, 256)
# The head widths the gfx950 kernels are built for.  The reference's model
# routes every power of two >= 16 to its kernels (model.py:158-165).  Here
# 16-128 run in every dot precision; 256 runs with bf16 operands (the forward,
# prefill and backward; the decode step takes every cache dtype), since the
# fp32 and split-operand tiles of the row-parallel output pass exceed the LDS
# at that width; 512 and wider are not built.  A caller narrows its routing
# with head_dim_supported(head_dim, dot_precision) and keeps its eager path
# for the rest.
SUPPORTED_HEAD_DIMS = _HEAD_DIMS
_BF16_ONLY_HEAD_DIMS = (256,)


def head_dim_supported(head_dim: int, dot_precision: str = "bf16") -> bool:
    """Whether the HIP kernels take this head width at this dot precision
    (16, 32, 64 or 128 in every precision; 256 with "bf16")."""
    head_dim = int(head_dim)
    if head_dim not in _HEAD_DIMS:
        return False
    return head_dim not in _BF16_ONLY_HEAD_DIMS or dot_precision == "bf16"


def dilution_attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """The operator written plainly in fp32 torch ops (kernels.py:40-68).

    q/k/v: (B, H, T, D).  Returns (B, H, T, D) fp32.  This is the spec the
    kernels are held to; it is never used as a kernel fallback.
    """
    seq, head_dim = q.shape[-2], q.shape[-1]
    aff = (q.float() @ k.float().transpose(-2, -1)) / math.sqrt(head_dim)
    mask = torch.tril(torch.ones(seq, seq, dtype=torch.bool, device=q.device))
    aff = aff.masked_fill(~mask, torch.finfo(torch.float32).min)
    p = aff.softmax(dim=-1)
    committed = p.cumsum(dim=-2) - p
    share = p / (committed + p + 1e-9)
    attn = share / (share.sum(dim=-1, keepdim=True) + 1e-9)
    return attn @ v.float()


# ---------------------------------------------------------------------------
# helpers


def _precision_code(dot_precision: str) -> int:
    """The C ABI's precision code (kernels.py:318-325): "ieee" fp32 MFMA
    operands; "tf32" fp32 values split into bf16 hi + lo operands, three bf16
    products per product (gfx950 has no tf32 MFMA; the split keeps about 16
    bits of each operand, more than tf32's 10); "bf16" bf16 MFMA operands."""
    if dot_precision not in _PRECISIONS:
        raise ValueError("dot_precision must be one of ieee, tf32, bf16")
    return _PRECISIONS[dot_precision]


def _check_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("dilution HIP kernels need tensors on the GPU (no CPU path)")
        if t.device != ts[0].device:
            raise ValueError(f"all tensors must be on one device, got {ts[0].device} and {t.device}")


def _check_cache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 committed: torch.Tensor) -> int:
    """Shapes of a decode / prefill call against its cache (kernels.py:1003-1021):
    contiguous (B, H, capacity, D) K and V, a contiguous (B, H, capacity) fp32
    demand, q of the same (B, H, ., D).  Returns the capacity."""
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must both be (B, H, capacity, D)")
    batch, heads, capacity, head_dim = k_cache.shape
    if q.dim() != 4 or (q.shape[0], q.shape[1], q.shape[3]) != (batch, heads, head_dim):
        raise ValueError(f"queries {tuple(q.shape)} do not match the cache {tuple(k_cache.shape)}")
    if tuple(committed.shape) != (batch, heads, capacity):
        raise ValueError(f"committed must be (B, H, capacity) = {(batch, heads, capacity)}, "
                         f"got {tuple(committed.shape)}")
    if committed.dtype != torch.float32:
        raise ValueError("committed must be float32")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous() and committed.is_contiguous()):
        raise ValueError("k_cache, v_cache and committed must be contiguous")
    return capacity


def _check_head_dim(head_dim: int, dot_precision: str | None = None) -> None:
    """ValueError unless the kernels take this width (at this dot precision;
    None: the decode step, which has none)."""
    if head_dim & (head_dim - 1):
        raise ValueError("head_dim must be a power of two")
    if head_dim not in _HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {_HEAD_DIMS} on the gfx950 kernels "
                         f"(head_dim_supported(); got {head_dim})")
    if dot_precision is not None and head_dim in _BF16_ONLY_HEAD_DIMS and dot_precision != "bf16":
        raise ValueError(f"head_dim {head_dim} runs with dot_precision='bf16' only on the gfx950 kernels "
                         f"(head_dim_supported(); got {dot_precision!r})")


def _common_dtype(*ts: torch.Tensor) -> torch.dtype:
    dt = ts[0].dtype
    for t in ts[1:]:
        dt = torch.promote_types(dt, t.dtype)
    if dt not in _DTYPES:
        dt = torch.float32
    return dt


def _rows(x: torch.Tensor, n: int, t: int, d: int, dtype: torch.dtype) -> torch.Tensor:
    """(n, t, d) contiguous view or copy in `dtype` (kernels.py:362-364)."""
    return x.reshape(n, t, d).to(dtype).contiguous()


def _stream(dev: torch.device) -> int:
    """The caller's current stream on the inputs' device; launches go there.
    (The raw handle, without building a torch Stream object: a decode step
    asks for it about 60 times.)"""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


_NO_SWITCH = contextlib.nullcontext()


def _on(dev: torch.device):
    """The inputs' device made current for a launch; no switch when it already is."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return _NO_SWITCH
    return torch.cuda.device(dev)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# forward


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
    _save_pk: bool = False,
    scratch_budget_gib: float = 16.0,
    _variant: tuple = _PRODUCTION,
):
    """Fused forward; returns fp32 outputs (kernels.py:328-455).

    With return_aux=True also returns the statistics the backward needs and
    the inclusive column totals of p (the cached-decode demand after this
    prefix), as the reference's aux dict: ``pk, rmax, rden, carry, ssum,
    bwd_block_m, block_m, block_n, dot_precision, num_warps,
    committed_total``.  ``carry`` holds the demand entering every 32-row block
    (``bwd_block_m`` = 32) for the block's causal keys ``j < 32 (b + 1)``; the
    entries past them are left unwritten, as in the reference
    (kernels.py:353-354; its tests read ``carry[:, b, :end]`` only).  Without
    return_aux no checkpoint is kept: the key-parallel pass (bf16 operands,
    head_dim 64) writes none, and the three-pass forward processes the
    (batch, head) slices in groups sized so its (rows, T/32, T) fp32
    checkpoint scratch stays under scratch_budget_gib; slices are independent,
    so results are identical either way.
    """
    prec = _precision_code(dot_precision)
    if q.dim() != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v must share one (B, H, T, D) shape, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    batch, heads, seq, head_dim = q.shape
    _check_head_dim(head_dim, dot_precision)
    _check_device(q, k, v)
    lib = _hip.lib()
    n = batch * heads
    dt = _common_dtype(q, k, v)
    qf, kf, vf = (_rows(x, n, seq, head_dim, dt) for x in (q, k, v))
    dev = q.device
    nb = (seq + CHECKPOINT_ROWS - 1) // CHECKPOINT_ROWS
    f32 = dict(device=dev, dtype=torch.float32)
    out = torch.empty(n, seq, head_dim, **f32)
    rmax = torch.empty(n, seq, **f32)
    rden = torch.empty(n, seq, **f32)
    ssum = torch.empty(n, seq, **f32)
    total = torch.empty(n, seq, **f32)
    pk = torch.empty(n, seq, head_dim, **f32) if _save_pk else None

    rows = n
    carry = None
    if return_aux:
        carry = torch.empty(n, nb, seq, **f32)
    elif tuple(_variant) != _PRODUCTION or not lib.dil_forward_key_pass(seq, 0, head_dim, _DTYPES[dt], prec):
        # the three-pass forward reads the checkpoints it writes: the slices go
        # in groups whose (rows, T/32, T) scratch fits the budget.  The key pass
        # writes none without aux and takes every slice in one call.
        per_row = nb * seq * 4
        rows = max(1, min(n, int(scratch_budget_gib * 2**30) // max(per_row, 1)))
        carry = torch.empty(rows, nb, seq, **f32)
    ws_bytes = lib.dil_forward_workspace_bytes(rows, seq, head_dim, _DTYPES[dt], prec, int(_save_pk))
    ws = _workspace(ws_bytes, dev)
    for a in range(0, n, rows):
        b = min(a + rows, n)
        head = (qf[a:b].data_ptr(), kf[a:b].data_ptr(), vf[a:b].data_ptr(), b - a, seq, head_dim,
                _DTYPES[dt], prec)
        tail = (out[a:b].data_ptr(), rmax[a:b].data_ptr(), rden[a:b].data_ptr(),
                ssum[a:b].data_ptr(), _ptr(carry), total[a:b].data_ptr(),
                None if pk is None else pk[a:b].data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
        with _on(dev):
            if tuple(_variant) == _PRODUCTION:
                status = lib.dil_forward(*head, *tail)
            else:
                status = lib.dil_forward_variant(*head, *_variant, *tail)
        _hip.check(status, "dil_forward")

    result = out.reshape(batch, heads, seq, head_dim)
    if return_aux:
        aux = dict(pk=pk, rmax=rmax, rden=rden, carry=carry, ssum=ssum, bwd_block_m=CHECKPOINT_ROWS,
                   block_m=block_m, block_n=block_n, dot_precision=dot_precision,
                   num_warps=num_warps, committed_total=total.reshape(batch, heads, seq))
        return result, aux
    return result


# ---------------------------------------------------------------------------
# training (autograd)


class _DilutionAttentionFn(torch.autograd.Function):
    """Forward + backward on the HIP kernels (kernels.py:829-903).

    Same 12 positional arguments as the reference; the tuning arguments are
    accepted and ignored.
    """

    @staticmethod
    def forward(ctx, q, k, v, dot_precision, block_m, block_n,
                num_warps, bwd_num_warps, bwd_num_stages, b3_block_n, b3_num_warps, b4_num_warps):
        if not any(ctx.needs_input_grad[:3]):
            # no backward can follow: nothing to save, no checkpoints to write
            return dilution_attention_forward(q, k, v, dot_precision=dot_precision, block_m=block_m,
                                              block_n=block_n, num_warps=num_warps)
        out, aux = dilution_attention_forward(
            q, k, v, dot_precision=dot_precision, block_m=block_m, block_n=block_n,
            return_aux=True, num_warps=num_warps, _save_pk=any(ctx.needs_input_grad[:3]),
        )
        ctx.save_for_backward(q, k, v, out, aux["rmax"], aux["rden"], aux["carry"], aux["ssum"],
                              aux["pk"])
        ctx.dot_precision = dot_precision
        return out

    @staticmethod
    def backward(ctx, dout):
        grads = _backward(ctx.saved_tensors, dout, ctx.dot_precision, _PRODUCTION)
        return (*grads, None, None, None, None, None, None, None, None, None)


def _backward(saved, dout, dot_precision: str, variant: tuple):
    """dq, dk, dv of the operator (variant) from the forward's saved tensors."""
    q, k, v, out, rmax, rden, carry, ssum, pk = saved
    lib = _hip.lib()
    batch, heads, seq, head_dim = q.shape
    n = batch * heads
    prec = _precision_code(dot_precision)
    dt = _common_dtype(q, k, v)
    qf, kf, vf = (_rows(x, n, seq, head_dim, dt) for x in (q, k, v))
    ddt = dout.dtype if dout.dtype in _DTYPES else torch.float32
    dof = _rows(dout, n, seq, head_dim, ddt)
    of = out.reshape(n, seq, head_dim)
    dev = q.device
    grads = []
    gdt = dt
    dq = torch.empty(n, seq, head_dim, device=dev, dtype=gdt)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    ws = _workspace(lib.dil_backward_workspace_bytes(n, seq, head_dim, _DTYPES[dt], prec), dev)
    head = (qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), dof.data_ptr(), of.data_ptr(),
            rmax.data_ptr(), rden.data_ptr(), ssum.data_ptr(), carry.data_ptr(), pk.data_ptr(),
            n, seq, head_dim, _DTYPES[dt], _DTYPES[ddt], _DTYPES[gdt], prec)
    tail = (dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
    with _on(dev):
        if tuple(variant) == _PRODUCTION:
            status = lib.dil_backward(*head, *tail)
        else:
            status = lib.dil_backward_variant(*head, *variant, *tail)
    _hip.check(status, "dil_backward")
    shape4 = (batch, heads, seq, head_dim)
    for g, ref in zip((dq, dk, dv), (q, k, v)):
        grads.append(g.reshape(shape4).to(ref.dtype))
    return tuple(grads)


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
) -> torch.Tensor:
    """Differentiable fused dilution attention (kernels.py:906-930).

    dot_precision "bf16" (default) uses bf16 MFMA operands for the score and
    value products with fp32 accumulation and fp32 demand/share math;
    "ieee" keeps fp32 operands; "tf32" runs fp32 values as split bf16
    operands (three bf16 products per product).
    """
    return _DilutionAttentionFn.apply(
        q, k, v, dot_precision, block_m, block_n,
        num_warps, bwd_num_warps, bwd_num_stages, b3_block_n, b3_num_warps, b4_num_warps,
    )


# ---------------------------------------------------------------------------
# chunked prefill (no reference counterpart; reference prefills in one call)


def dilution_prefill_chunk(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    committed: torch.Tensor,
    start: int,
    dot_precision: str = "bf16",
    return_aux: bool = False,
):
    """Rows [start, start + C) of the operator over the cached keys
    [0, start + C), carrying the fp32 demand vector across chunks.

    q: (B, H, C, D).  k_cache / v_cache: contiguous (B, H, capacity, D) with
    rows [0, start + C) written.  committed: contiguous (B, H, capacity) fp32
    holding the column totals of p over rows < start, zero on
    [start, start + C); advanced in place to the totals over rows < start + C
    (entries beyond start + C are not touched).  Returns the chunk's outputs
    (B, H, C, D) fp32, and with return_aux the chunk's rmax/rden/ssum/carry.
    Chaining chunks reproduces ``dilution_attention_forward`` row for row and
    its ``aux["committed_total"]``.
    """
    prec = _precision_code(dot_precision)
    capacity = _check_cache(q, k_cache, v_cache, committed)
    batch, heads, chunk, head_dim = q.shape
    _check_head_dim(head_dim, dot_precision)
    if start < 0 or start + chunk > capacity:
        raise ValueError(f"rows [{start}, {start + chunk}) outside cache capacity {capacity}")
    _check_device(q, k_cache, v_cache, committed)
    lib = _hip.lib()
    n = batch * heads
    dt = k_cache.dtype if k_cache.dtype in _DTYPES else torch.float32
    if v_cache.dtype != dt or k_cache.dtype != dt:
        raise ValueError("k_cache and v_cache must share a float dtype")
    kf = k_cache.view(n, capacity, head_dim)
    vf = v_cache.view(n, capacity, head_dim)
    cf = committed.view(n, capacity)
    qf = _rows(q, n, chunk, head_dim, dt)
    dev = q.device
    nb = (chunk + CHECKPOINT_ROWS - 1) // CHECKPOINT_ROWS
    f32 = dict(device=dev, dtype=torch.float32)
    out = torch.empty(n, chunk, head_dim, **f32)
    rmax = torch.empty(n, chunk, **f32)
    rden = torch.empty(n, chunk, **f32)
    ssum = torch.empty(n, chunk, **f32)
    # the key pass writes the checkpoints only for a caller that keeps them
    carry = None
    if return_aux or not lib.dil_forward_key_pass(chunk, start, head_dim, _DTYPES[dt], prec):
        carry = torch.empty(n, nb, start + chunk, **f32)
    ws = _workspace(lib.dil_prefill_workspace_bytes(n, chunk, start, head_dim, _DTYPES[dt], prec), dev)
    with _on(dev):
        status = lib.dil_prefill_chunk(
            qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), n, chunk, start, capacity, head_dim,
            _DTYPES[dt], prec, cf.data_ptr(), out.data_ptr(), rmax.data_ptr(), rden.data_ptr(),
            ssum.data_ptr(), _ptr(carry), ws.data_ptr(), ws.numel(), _stream(dev))
    _hip.check(status, "dil_prefill_chunk")
    result = out.reshape(batch, heads, chunk, head_dim)
    if return_aux:
        return result, dict(rmax=rmax, rden=rden, ssum=ssum, carry=carry,
                            bwd_block_m=CHECKPOINT_ROWS, dot_precision=dot_precision)
    return result


# ---------------------------------------------------------------------------
# cached decode


def dilution_decode_step(
    q1: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    committed: torch.Tensor,
    length: int,
    block_n: int = 512,
    num_warps: int = 8,
    _variant: tuple = _PRODUCTION,
) -> torch.Tensor:
    """Fused decode step; returns the new row's output (B, H, 1, D) in q1.dtype
    (kernels.py:994-1038).

    q1: (B, H, 1, D).  k_cache / v_cache: contiguous (B, H, capacity, D)
    buffers whose first `length` positions are valid, the new token already
    written at position length-1.  committed: contiguous (B, H, capacity) fp32
    accumulator (column totals of p over all previous rows; position length-1
    must be zero).  It is advanced in place to include this row; positions
    >= length are never touched.
    """
    batch, heads, one, head_dim = q1.shape
    if one != 1:
        raise ValueError("decode step takes exactly one query row per (batch, head)")
    if head_dim & (head_dim - 1):
        raise ValueError("head_dim must be a power of two")
    capacity = _check_cache(q1, k_cache, v_cache, committed)
    if not 1 <= length <= capacity:
        raise ValueError(f"length {length} outside cache capacity {capacity}")
    _check_head_dim(head_dim)
    _check_device(q1, k_cache, v_cache, committed)
    lib = _hip.lib()
    n = batch * heads
    dt = k_cache.dtype if k_cache.dtype in _DTYPES else torch.float32
    if v_cache.dtype != dt or k_cache.dtype != dt:
        raise ValueError("k_cache and v_cache must share a float dtype")
    kf = k_cache.view(n, capacity, head_dim)
    vf = v_cache.view(n, capacity, head_dim)
    cf = committed.view(n, capacity)
    # q1 keeps its own dtype: the kernels read it as fp32 and store the
    # output in it (kernels.py:953, 1029)
    qdt = q1.dtype if q1.dtype in _DTYPES else torch.float32
    qf = q1.reshape(n, head_dim).to(qdt).contiguous()
    out = torch.empty(n, head_dim, device=q1.device, dtype=qdt)
    ws = _workspace(lib.dil_decode_workspace_bytes(n, length, head_dim), q1.device)
    head = (qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), cf.data_ptr(), out.data_ptr(), n,
            capacity, length, head_dim, _DTYPES[dt], _DTYPES[qdt])
    tail = (ws.data_ptr(), ws.numel(), _stream(q1.device))
    with _on(q1.device):
        if tuple(_variant) == _PRODUCTION:
            status = lib.dil_decode_step(*head, *tail)
        else:
            status = lib.dil_decode_step_variant(*head, *_variant, *tail)
    _hip.check(status, "dil_decode_step")
    if out.dtype != q1.dtype:
        out = out.to(q1.dtype)
    return out.view(batch, heads, 1, head_dim)


def decode_step_device_length(q1: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                              committed: torch.Tensor, length: torch.Tensor, max_length: int,
                              out: torch.Tensor | None = None,
                              workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``dilution_decode_step`` with the length in device memory: ``length``
    is an int64 tensor of one element on the caches' device, read by the
    kernels when they run, so one captured HIP graph serves every decode step
    (no reference counterpart; the reference passes a Python int).
    ``max_length`` (<= capacity) sizes the grid and the workspace; a live
    length outside [0, max_length] is clamped.  ``out`` ((B, H, D) in q1's
    dtype) and ``workspace`` (``decode_workspace(...)``) may be given so that
    the call allocates nothing.  Results equal ``dilution_decode_step`` at the
    live length, bitwise."""
    batch, heads, one, head_dim = q1.shape
    if one != 1:
        raise ValueError("decode step takes exactly one query row per (batch, head)")
    capacity = _check_cache(q1, k_cache, v_cache, committed)
    if not 1 <= max_length <= capacity:
        raise ValueError(f"max_length {max_length} outside cache capacity {capacity}")
    if length.dtype != torch.int64 or length.numel() != 1 or length.device != k_cache.device:
        raise ValueError("length must be one int64 element on the caches' device")
    _check_head_dim(head_dim)
    _check_device(q1, k_cache, v_cache, committed)
    lib = _hip.lib()
    n = batch * heads
    dt = k_cache.dtype
    if dt not in _DTYPES or v_cache.dtype != dt:
        raise ValueError("k_cache and v_cache must share a float dtype")
    if q1.dtype not in _DTYPES:
        raise ValueError("q1 must be float32, bfloat16 or float16")
    qf = q1.reshape(n, head_dim)
    if not qf.is_contiguous():
        qf = qf.contiguous()
    if out is None:
        out = torch.empty(n, head_dim, device=q1.device, dtype=q1.dtype)
    elif out.dtype != q1.dtype or out.numel() != n * head_dim or not out.is_contiguous():
        raise ValueError("out must be a contiguous (B, H, D) tensor in q1's dtype")
    need = lib.dil_decode_workspace_bytes(n, max_length, head_dim)
    if workspace is None:
        workspace = _workspace(need, q1.device)
    elif workspace.numel() < need:
        raise ValueError(f"workspace of {workspace.numel()} bytes, {need} needed")
    status = lib.dil_decode_step_dlen(
        qf.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), committed.data_ptr(), out.data_ptr(),
        n, capacity, length.data_ptr(), max_length, head_dim, _DTYPES[dt], _DTYPES[q1.dtype],
        workspace.data_ptr(), workspace.numel(), _stream(q1.device))
    _hip.check(status, "dil_decode_step_dlen")
    return out.view(batch, heads, 1, head_dim)


def decode_workspace(batch: int, heads: int, max_length: int, head_dim: int, device) -> torch.Tensor:
    """A workspace for ``decode_step_device_length`` up to ``max_length``."""
    lib = _hip.lib()
    return _workspace(lib.dil_decode_workspace_bytes(batch * heads, max_length, head_dim), device)
