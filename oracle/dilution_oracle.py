"""CPU oracle for the dilution-attention hot path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for the CPU
baseline, as the thing timed on host cores).  The product path
(``dilution.kernels``) never imports it and has no CPU fallback.

Every function restates the reference operator from its published source, in
code written for this repository:

  reference operator            /root/reference/src/dilution/kernels.py:40-68
  operator definition           /root/reference/docs/operator.md:1-23
  row statistics (K1 sweep 1)   /root/reference/src/dilution/kernels.py:159-182
  saved query correction pk     /root/reference/src/dilution/kernels.py:166-182
  carry checkpoints / totals    /root/reference/tests/test_kernels.py:130-149
  cached decode step            /root/reference/src/dilution/kernels.py:937-991,
                                /root/reference/src/dilution/model.py:231-257
  prefill demand hand-off       /root/reference/src/dilution/model.py:198-229
  backward decomposition        /root/reference/docs/kernels.md:62-84,
                                /root/reference/src/dilution/kernels.py:678-775
  row-blocked reverse walk      /root/reference/src/dilution/kernels.py:736-770
  bid / share variants          /root/reference/src/dilution/kernels_bid.py:4-42,
                                :94-165 (bids, share modes), :853-960 (decode)

Pinning (each function is checked by something other than a retyping of its
own formula; see tests/test_oracle.py):

  attention_fp32          fp64 brute-force loops (attention_loops_f64), the
                          q = 0 harmonic-number closed form, T = 1, causality,
                          shift invariance, and planted-mistake variants that
                          must fail those checks.
  attention_blocked_f64   attention_f64 at ragged lengths and block sizes,
                          and the harmonic closed form at T = 3000.
  attention_loops_f64     the harmonic closed form (independent of softmax
                          and cumsum code) and agreement with attention_fp32.
  row_stats / bids        torch.softmax (a library routine) at fp64.
  demand_totals, carry    harmonic closed form H_T - H_j; fp64 loop sums.
  grads_autograd          torch.autograd.gradcheck (finite differences, fp64).
  grads_closed_form_f64   autograd through attention_fp32 at fp64.
  grads_blocked_f64       grads_closed_form_f64 at ragged lengths and block
                          sizes (and, through it, autograd); the key-shift
                          identity sum_j dk_j = 0; planted mistakes (the
                          demand or the suffix not carried across blocks)
                          that must fail the comparison.
  decode_step             the full-sequence rows of attention_loops_f64, token
                          after token, and the demand == column sums.
  prefill_chunk           the full-sequence rows and demand == column sums.
  pk                      (p @ k) / sqrt(d) via fp64 matmul of torch.softmax.
  variant_attention_f64   variant_attention_loops (scalar fp64 loops over
                          rows and keys, written independently), the q = 0
                          closed forms (uniform bids -> harmonic numbers;
                          sigmoid bids 1/2 -> 1/(i-j+1) weights; no share ->
                          window mean), the exclusive share's identity
                          collapse and softmax first row, and gradcheck.
  variant_demand_totals   the loops' running demand.

No function here is "parity unpinned".
"""

from __future__ import annotations

import math

import numpy as np
import torch

EPS = 1e-9          # kernels.py:66-67 (share denominator and row normalise)
LOG2E = 1.4426950408889634


# ---------------------------------------------------------------------------
# forward


def attention_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """fp32 restatement of dilution_attention_reference (kernels.py:40-68).

    q, k, v: (B, H, T, D) of any float dtype; math in fp32; returns fp32.
    """
    t, d = q.shape[-2], q.shape[-1]
    s = torch.matmul(q.float(), k.float().transpose(-2, -1)) / math.sqrt(d)
    causal = torch.ones(t, t, dtype=torch.bool, device=q.device).tril()
    s = s.masked_fill(~causal, torch.finfo(torch.float32).min)
    p = torch.softmax(s, dim=-1)
    demand_before = torch.cumsum(p, dim=-2) - p          # exclusive column sums
    share = p / (demand_before + p + EPS)
    a = share / (share.sum(dim=-1, keepdim=True) + EPS)
    return torch.matmul(a, v.float())


def attention_f64(q, k, v) -> torch.Tensor:
    """The same formula evaluated in float64 (used where fp32 rounding of the
    oracle itself would dominate a tolerance)."""
    t, d = q.shape[-2], q.shape[-1]
    q, k, v = (torch.as_tensor(x).double() for x in (q, k, v))
    s = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(d)
    causal = torch.ones(t, t, dtype=torch.bool).tril()
    s = s.masked_fill(~causal, -math.inf)
    p = torch.softmax(s, dim=-1)
    demand_before = torch.cumsum(p, dim=-2) - p
    share = p / (demand_before + p + EPS)
    a = share / (share.sum(dim=-1, keepdim=True) + EPS)
    return torch.matmul(a, v)


def attention_blocked_f64(q, k, v, block: int = 512) -> tuple[np.ndarray, np.ndarray]:
    """One (batch, head) slice at any length: q, k, v (T, D) -> (out (T, D),
    demand totals (T,)), float64, in row blocks of `block` with the demand
    carried from block to block, so memory is O(block T) rather than O(T^2).
    The same formula as attention_f64 (kernels.py:40-68), evaluated the way
    the eager prefill carries demand across prompts (model.py:209-222); what
    makes the full-size (T = 16384) parity checks affordable on host cores."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    t, d = q.shape
    out = np.empty((t, v.shape[1]))
    demand = np.zeros(t)
    for r0 in range(0, t, block):
        r1 = min(r0 + block, t)
        s = (q[r0:r1] @ k[:r1].T) / math.sqrt(d)                 # (rows, keys [0, r1))
        s[np.arange(r1)[None, :] > np.arange(r0, r1)[:, None]] = -np.inf
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        before = demand[:r1] + np.cumsum(p, axis=0) - p           # exclusive column sums
        share = p / (before + p + EPS)
        out[r0:r1] = (share / (share.sum(axis=1, keepdims=True) + EPS)) @ v[:r1]
        demand[:r1] += p.sum(axis=0)
    return out, demand


def attention_loops_f64(q, k, v) -> np.ndarray:
    """Brute-force float64 loops over (row, key): no softmax, cumsum or matmul
    library call.  For tiny T only (O(B H T^2 D) Python-level work is kept
    vectorised over B, H and D only)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, h, t, d = q.shape
    out = np.zeros((b, h, t, d))
    demand = np.zeros((b, h, t))           # running column totals, row by row
    for i in range(t):
        aff = np.stack([(q[:, :, i, :] * k[:, :, j, :]).sum(-1) for j in range(i + 1)], -1)
        aff = aff / math.sqrt(d)
        m = aff.max(-1, keepdims=True)
        e = np.exp(aff - m)
        p = e / e.sum(-1, keepdims=True)   # (b, h, i+1)
        share = np.empty_like(p)
        for j in range(i + 1):
            share[..., j] = p[..., j] / (demand[..., j] + p[..., j] + EPS)
        total = share.sum(-1, keepdims=True) + EPS
        for j in range(i + 1):
            out[:, :, i, :] += (share[..., j] / total[..., 0])[..., None] * v[:, :, j, :]
        demand[..., : i + 1] += p
    return out


def harmonic_closed_form(t: int, v) -> tuple[np.ndarray, np.ndarray]:
    """q = 0: every affinity is 0, so p_ij = 1/(i+1) for j <= i.

    Exclusive demand is H_i - H_j (H_m = sum_{s=1..m} 1/s), the share is
    (1/(i+1)) / (H_{i+1} - H_j + eps) and the decode totals are H_T - H_j.
    Returns (out (.., T, D) for the given v, totals (T,)).  Pure closed form:
    no softmax, no cumsum.
    """
    v = np.asarray(v, dtype=np.float64)
    harm = np.concatenate([[0.0], np.cumsum(1.0 / np.arange(1, t + 1, dtype=np.float64))])
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    share = np.where(j <= i, (1.0 / (i + 1)) / (harm[i + 1] - harm[j] + EPS), 0.0)
    a = share / (share.sum(-1, keepdims=True) + EPS)
    out = np.matmul(a, v)
    totals = harm[t] - harm[np.arange(t)]
    return out, totals


# ---------------------------------------------------------------------------
# statistics the kernels expose through aux


def bids(q, k, dtype=torch.float64) -> torch.Tensor:
    """Causal softmax bids p (B, H, T, T) (kernels.py:59-64)."""
    t, d = q.shape[-2], q.shape[-1]
    q = torch.as_tensor(q).to(dtype)
    k = torch.as_tensor(k).to(dtype)
    s = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(d)
    causal = torch.ones(t, t, dtype=torch.bool).tril()
    return torch.softmax(s.masked_fill(~causal, -math.inf), dim=-1)


def row_stats(q, k) -> tuple[torch.Tensor, torch.Tensor]:
    """(rmax, rden) as K1 defines them (kernels.py:159-182): rmax is the row
    max of the scaled affinities in the log2 domain and rden = sum 2^(a - rmax),
    so that p = 2^(a - rmax) / rden."""
    t, d = q.shape[-2], q.shape[-1]
    q = torch.as_tensor(q).double()
    k = torch.as_tensor(k).double()
    a = torch.matmul(q, k.transpose(-2, -1)) * (LOG2E / math.sqrt(d))
    causal = torch.ones(t, t, dtype=torch.bool).tril()
    a = a.masked_fill(~causal, -math.inf)
    rmax = a.max(-1).values
    rden = torch.exp2(a - rmax[..., None]).sum(-1)
    return rmax, rden


def demand_totals(q, k) -> torch.Tensor:
    """Inclusive column totals of p over all rows: aux["committed_total"],
    the decode accumulator after a prefix (kernels.py:451-453, 264)."""
    return bids(q, k).sum(-2)


def carry_checkpoints(q, k, block: int) -> torch.Tensor:
    """carry[:, :, rb, j] = sum_{i < rb*block} p_ij (test_kernels.py:143-149);
    keys j >= rb*block are exactly zero by causality."""
    p = bids(q, k)
    t = p.shape[-1]
    nb = (t + block - 1) // block
    incl = torch.cumsum(p, dim=-2)
    out = torch.zeros(*p.shape[:-2], nb, t, dtype=p.dtype)
    for rb in range(1, nb):
        out[..., rb, :] = incl[..., rb * block - 1, :]
    return out


def pk(q, k) -> torch.Tensor:
    """Saved query-side Jacobian correction (p @ k) / sqrt(d)
    (kernels.py:166-182; test_kernels.py:46-59)."""
    d = q.shape[-1]
    return torch.matmul(bids(q, k), torch.as_tensor(k).double()) / math.sqrt(d)


# ---------------------------------------------------------------------------
# prefill and decode


def prefill_chunk(q_chunk, k_all, v_all, demand_in, start: int):
    """Rows [start, start+C) of the operator given the keys [0, start+C) and
    the incoming demand D_j = sum_{i<start} p_ij (zero for j >= start).

    Returns (out (.., C, D) float64, demand_out (.., start+C) float64) where
    demand_out_j = D_j + sum_{start <= i < start+C} p_ij.  Follows the eager
    prefill (model.py:209-222) generalised to a carried-in demand.
    """
    qc = torch.as_tensor(q_chunk).double()
    ka = torch.as_tensor(k_all).double()
    va = torch.as_tensor(v_all).double()
    c, d = qc.shape[-2], qc.shape[-1]
    tk = start + c
    ka, va = ka[..., :tk, :], va[..., :tk, :]
    s = torch.matmul(qc, ka.transpose(-2, -1)) / math.sqrt(d)
    rows = torch.arange(start, start + c)[:, None]
    keys = torch.arange(tk)[None, :]
    s = s.masked_fill(keys > rows, -math.inf)
    p = torch.softmax(s, dim=-1)
    dem = torch.as_tensor(demand_in).double()[..., :tk].clone()
    before = dem[..., None, :] + torch.cumsum(p, dim=-2) - p
    share = p / (before + p + EPS)
    a = share / (share.sum(-1, keepdim=True) + EPS)
    return torch.matmul(a, va), dem + p.sum(-2)


def decode_step(q1, k_cache, v_cache, committed, length: int, dtype=torch.float64):
    """One cached decode row (kernels.py:937-991; eager twin model.py:242-257).

    q1: (B, H, 1, D); caches (B, H, cap, D); committed (B, H, cap) holding the
    column totals of p over earlier rows, with committed[..., length-1] == 0.
    Returns (out (B, H, 1, D), committed_new with the first `length` entries
    advanced by p and the rest unchanged), both in `dtype` (float64 for the
    parity checks; the bench's CPU baseline times float32).
    """
    q = torch.as_tensor(q1).to(dtype)
    k = torch.as_tensor(k_cache).to(dtype)[..., :length, :]
    v = torch.as_tensor(v_cache).to(dtype)[..., :length, :]
    com = torch.as_tensor(committed).to(dtype).clone()
    d = q.shape[-1]
    a = torch.matmul(q, k.transpose(-2, -1))[..., 0, :] / math.sqrt(d)
    p = torch.softmax(a, dim=-1)
    c = com[..., :length]
    share = p / (c + p + EPS)
    a_row = share / (share.sum(-1, keepdim=True) + EPS)
    out = torch.matmul(a_row[..., None, :], v)
    com[..., :length] = c + p
    return out, com


# ---------------------------------------------------------------------------
# backward


def grads_autograd(q, k, v, dout, dtype=torch.float64):
    """(dq, dk, dv) by autograd through the reference formula."""
    fn = attention_f64 if dtype == torch.float64 else attention_fp32
    xs = [torch.as_tensor(x).to(dtype).detach().clone().requires_grad_(True) for x in (q, k, v)]
    out = fn(*xs)
    out.backward(torch.as_tensor(dout).to(out.dtype))
    return tuple(x.grad for x in xs)


def grads_closed_form_f64(q, k, v, dout):
    """Backward by the published decomposition (docs/kernels.md:62-84,
    kernels.py:685-698), in float64 numpy.

        ds_ij   = (dO_i . v_j - dO_i . o_i) / (S_i + eps)
        inv_ij  = 1 / (c_ij + p_ij + eps)
        dp_ij   = ds_ij (c_ij + eps) inv_ij^2 - sum_{i' > i} ds_i'j p_i'j inv_i'j^2
        ghat_i  = sum_j p_ij dp_ij
        da_ij   = p_ij (dp_ij - ghat_i)
        dq = s da K,  dk = s da^T Q,  dv = A^T dO        (s = 1/sqrt(d))

    Also returns the intermediates (dict) so kernel-internal buffers (ghat,
    suffix checkpoints, dbar) can be checked.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(dout, dtype=np.float64)
    t, d = q.shape[-2], q.shape[-1]
    sc = 1.0 / math.sqrt(d)
    causal = np.tril(np.ones((t, t), dtype=bool))
    a = np.matmul(q, np.swapaxes(k, -1, -2)) * sc
    a = np.where(causal, a, -np.inf)
    a = a - a.max(-1, keepdims=True)
    e = np.exp(a)
    p = e / e.sum(-1, keepdims=True)
    c = np.cumsum(p, axis=-2) - p
    inv = np.where(causal, 1.0 / (c + p + EPS), 0.0)
    share = p * inv
    ssum = share.sum(-1, keepdims=True)
    attn = share / (ssum + EPS)
    o = np.matmul(attn, v)
    dbar = (do * o).sum(-1, keepdims=True)
    ds = np.where(causal, (np.matmul(do, np.swapaxes(v, -1, -2)) - dbar) / (ssum + EPS), 0.0)
    dk_share = -ds * p * inv * inv
    # suffix_ij = sum over later rows i' > i of dk_share_i'j
    rev = np.flip(np.cumsum(np.flip(dk_share, -2), axis=-2), -2)
    suffix = rev - dk_share
    dp = np.where(causal, ds * (c + EPS) * inv * inv + suffix, 0.0)
    ghat = (p * dp).sum(-1, keepdims=True)
    da = p * (dp - ghat)
    dq = np.matmul(da, k) * sc
    dk = np.matmul(np.swapaxes(da, -1, -2), q) * sc
    dv = np.matmul(np.swapaxes(attn, -1, -2), do)
    inter = dict(p=p, committed=c, ssum=ssum[..., 0], dbar=dbar[..., 0], ghat=ghat[..., 0],
                 suffix=suffix, out=o)
    return (dq, dk, dv), inter


def grads_blocked_f64(q, k, v, dout, block: int = 512, mutant: str | None = None):
    """Backward of one (batch, head) slice at any length, float64, in row
    blocks: q, k, v, dout (T, D) -> ((dq, dk, dv), intermediates).

    The same decomposition as grads_closed_form_f64 (docs/kernels.md:62-84),
    evaluated the way the reference's backward walks it
    (src/dilution/kernels.py:736-770): a forward sweep over row blocks that
    carries the column demand and records the demand entering each block, then
    a reverse sweep over the blocks that carries, per key, the suffix
    U_j = sum over later rows i' of ds_i'j p_i'j / (c_i'j + p_i'j + eps)^2.
    Memory is O(block T) instead of O(T^2), which makes gradient parity at
    T = 16384 affordable on host cores.  Runs on the device of the inputs
    (torch ops only), so a test may evaluate it in float64 on the GPU where
    the host would take too long.

    Intermediates: out, lse (natural log-sum-exp per row), ssum, ghat and the
    demand totals.  `mutant` plants a named mistake for the tests that show
    the pins catch it: "no_suffix_carry" drops the suffix carried between
    blocks, "no_demand_carry" the demand carried into each block.
    """
    dev = q.device if isinstance(q, torch.Tensor) else torch.device("cpu")
    q, k, v, do = (torch.as_tensor(x).to(device=dev, dtype=torch.float64) for x in (q, k, v, dout))
    t, d = q.shape
    sc = 1.0 / math.sqrt(d)
    nb = (t + block - 1) // block
    kt, vt = k.T.contiguous(), v.T.contiguous()      # right operands stored, not transposed views
    lse = torch.empty(t, dtype=torch.float64, device=dev)
    ssum = torch.empty(t, dtype=torch.float64, device=dev)
    out = torch.empty(t, v.shape[1], dtype=torch.float64, device=dev)
    carry = torch.zeros(nb, t, dtype=torch.float64, device=dev)   # demand entering block b
    demand = torch.zeros(t, dtype=torch.float64, device=dev)

    def block_bids(r0, r1):
        a = (q[r0:r1] @ kt[:, :r1]) * sc
        rows = torch.arange(r0, r1, device=dev)[:, None]
        keys = torch.arange(r1, device=dev)[None, :]
        a = a.masked_fill(keys > rows, -math.inf)
        m = a.max(dim=1, keepdim=True).values
        ls = m[:, 0] + torch.log(torch.exp(a - m).sum(dim=1))
        return torch.exp(a - ls[:, None]), ls

    for b in range(nb):
        r0, r1 = b * block, min(t, (b + 1) * block)
        if mutant != "no_demand_carry":
            carry[b] = demand
        p, lse[r0:r1] = block_bids(r0, r1)
        excl = carry[b, :r1] + torch.cumsum(p, dim=0) - p        # demand before each row
        sh = p / (excl + p + EPS)
        ssum[r0:r1] = sh.sum(dim=1)
        out[r0:r1] = (sh / (ssum[r0:r1, None] + EPS)) @ v[:r1]
        demand[:r1] += p.sum(dim=0)

    dbar = (do * out).sum(dim=1)
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    ghat = torch.empty(t, dtype=torch.float64, device=dev)
    suffix = torch.zeros(t, dtype=torch.float64, device=dev)      # U entering from below
    for b in reversed(range(nb)):
        r0, r1 = b * block, min(t, (b + 1) * block)
        a = (q[r0:r1] @ kt[:, :r1]) * sc
        rows = torch.arange(r0, r1, device=dev)[:, None]
        keys = torch.arange(r1, device=dev)[None, :]
        causal = keys <= rows
        p = torch.exp(a.masked_fill(~causal, -math.inf) - lse[r0:r1, None])
        excl = carry[b, :r1] + torch.cumsum(p, dim=0) - p
        inv = 1.0 / (excl + p + EPS)
        sh = p * inv
        sinv = 1.0 / (ssum[r0:r1, None] + EPS)
        ds = ((do[r0:r1] @ vt[:, :r1] - dbar[r0:r1, None]) * sinv).masked_fill(~causal, 0.0)
        g = ds * sh * inv                                          # ds p / (c + p + eps)^2
        later = torch.flip(torch.cumsum(torch.flip(g, (0,)), dim=0), (0,)) - g
        u = later + (0.0 if mutant == "no_suffix_carry" else suffix[:r1])
        dp = (ds * (excl + EPS) * inv * inv - u).masked_fill(~causal, 0.0)
        ghat[r0:r1] = (p * dp).sum(dim=1)
        da = p * (dp - ghat[r0:r1, None])
        dq[r0:r1] = (da @ k[:r1]) * sc
        dk[:r1] += (da.T @ q[r0:r1]) * sc
        dv[:r1] += (sh * sinv).T @ do[r0:r1]
        suffix[:r1] += g.sum(dim=0)
    inter = dict(out=out, lse=lse, ssum=ssum, ghat=ghat, totals=demand)
    return (dq, dk, dv), inter


# ---------------------------------------------------------------------------
# bid / share variants (kernels_bid.py)

BIDS = ("softmax", "relu", "relu2", "softplus", "minshift", "sigmoid", "expshift", "sigshift")
SHARES = (True, False, "exclusive")


def _variant_bids_f64(aff: torch.Tensor, bid: str, shift: float) -> torch.Tensor:
    """Bids (.., T, T) from fp64 affinities on the causal window
    (kernels_bid.py:94-121): row-normalised numerators for the ratio bids,
    with a uniform row where the numerators carry no mass."""
    t = aff.shape[-1]
    causal = torch.ones(t, t, dtype=torch.bool).tril()
    if bid == "softmax":
        return torch.softmax(aff.masked_fill(~causal, -math.inf), dim=-1)
    if bid == "sigmoid":
        return torch.sigmoid(aff) * causal
    if bid == "expshift":
        return torch.exp(aff) / shift * causal
    if bid == "sigshift":
        return torch.sigmoid(aff - math.log(shift)) * causal
    if bid == "relu":
        num = aff.clamp_min(0.0)
    elif bid == "relu2":
        num = aff.clamp_min(0.0) ** 2
    elif bid == "softplus":
        num = torch.nn.functional.softplus(aff)
    elif bid == "minshift":
        lo = aff.masked_fill(~causal, math.inf).amin(dim=-1, keepdim=True).detach()
        num = aff - lo
    else:
        raise ValueError(bid)
    num = num * causal
    mass = num.sum(dim=-1, keepdim=True)
    window = torch.arange(1, t + 1, dtype=aff.dtype)[:, None]
    return torch.where(mass > 0, num / mass.clamp_min(1e-300), causal / window)


def variant_attention_f64(q, k, v, bid: str = "softmax", share=True, shift: float = 1.0) -> torch.Tensor:
    """fp64 restatement of kernels_bid.dilution_attention_reference
    (kernels_bid.py:130-165): any bid, share True / "exclusive" / False.
    Differentiable (torch autograd) for the gradient checks."""
    t, d = q.shape[-2], q.shape[-1]
    q, k, v = (torch.as_tensor(x).double() for x in (q, k, v))
    aff = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(d)
    p = _variant_bids_f64(aff, bid, shift)
    if share is False:
        a = p / p.sum(dim=-1, keepdim=True)
    else:
        before = torch.cumsum(p, dim=-2) - p
        denom = before + EPS if share == "exclusive" else before + p + EPS
        sh = p / denom
        a = sh / (sh.sum(dim=-1, keepdim=True) + EPS)
    return torch.matmul(a, v)


def variant_demand_totals(q, k, bid: str = "softmax", shift: float = 1.0) -> torch.Tensor:
    """Column totals of the variant's bids (the decode demand), fp64."""
    d = q.shape[-1]
    q, k = (torch.as_tensor(x).double() for x in (q, k))
    aff = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(d)
    return _variant_bids_f64(aff, bid, shift).sum(dim=-2)


def variant_attention_loops(q, k, v, bid: str = "softmax", share=True, shift: float = 1.0):
    """Scalar fp64 loops over (row, key) for one (batch, head) slice: (T, D)
    arrays q, k, v.  Returns (out (T, D), demand totals (T,)).  Bids from
    math.exp / comparisons, demand accumulated row by row; tiny T only."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    t, d = q.shape
    out = np.zeros((t, d))
    demand = np.zeros(t)
    for i in range(t):
        a = [float(np.dot(q[i], k[j])) / math.sqrt(d) for j in range(i + 1)]
        if bid == "softmax":
            top = max(a)
            e = [math.exp(x - top) for x in a]
            p = [x / sum(e) for x in e]
        elif bid in ("sigmoid", "sigshift"):
            off = math.log(shift) if bid == "sigshift" else 0.0
            p = [1.0 / (1.0 + math.exp(-(x - off))) for x in a]
        elif bid == "expshift":
            p = [math.exp(x) / shift for x in a]
        else:
            if bid == "relu":
                num = [x if x > 0 else 0.0 for x in a]
            elif bid == "relu2":
                num = [x * x if x > 0 else 0.0 for x in a]
            elif bid == "softplus":
                num = [math.log1p(math.exp(x)) if x < 30 else x for x in a]
            else:
                lo = min(a)
                num = [x - lo for x in a]
            mass = sum(num)
            p = [x / mass for x in num] if mass > 0 else [1.0 / (i + 1)] * (i + 1)
        if share is False:
            w = p
        elif share == "exclusive":
            w = [p[j] / (demand[j] + EPS) for j in range(i + 1)]
        else:
            w = [p[j] / (demand[j] + p[j] + EPS) for j in range(i + 1)]
        tot = sum(w) + (0.0 if share is False else EPS)
        for j in range(i + 1):
            out[i] += (w[j] / tot) * v[j]
            demand[j] += p[j]
    return out, demand


# ---------------------------------------------------------------------------
# deterministic synthetic inputs (CPU RNG, so every device sees the same values)


def make_inputs(shape, seed: int, qk_scale: float = 1.0, with_dout: bool = False,
                dtype=torch.float32):
    """q, k ~ qk_scale * N(0,1), v ~ N(0,1) (and dO ~ N(0,1)) from a CPU
    generator, cast to `dtype`."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(*shape, generator=g) * qk_scale
    k = torch.randn(*shape, generator=g) * qk_scale
    v = torch.randn(*shape, generator=g)
    out = [q.to(dtype), k.to(dtype), v.to(dtype)]
    if with_dout:
        out.append(torch.randn(*shape, generator=g).to(dtype))
    return tuple(out)
