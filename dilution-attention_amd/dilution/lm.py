"""A decoder-only LM whose attention is the HIP dilution operator.

This is the whole-model harness for the operator: the caller side of the hot
path, at the shape of the model-level benchmark (12 layers, d_model 1024,
16 heads of 64, SwiGLU MLP, RMSNorm, no position encoding, vocab 50304, bf16
weights).  It follows the reference's module layout and cache protocol
(src/dilution/model.py):

* ``DilutionAttention``: fused q/k/v projection, the operator, output
  projection (model.py:120-257 with ``use_kernel`` on: training forward
  through ``kernels.dilution_attention``, no-grad forward through
  ``kernels.dilution_attention_forward``, prefill and cached decode through
  ``dilution.cache``); ``LMConfig.bid`` / ``share_cumsum`` select an ablation
  variant of the operator, which runs on ``kernels_bid`` with
  SHIFT = ``context_length`` (model.py:121-156);
* ``SoftmaxAttention``: the parameter-matched causal softmax control on
  torch SDPA, with a plain KV cache (model.py:96-117), selected per layer by
  ``LMConfig.attention`` / ``layer_attention`` as in the reference's
  ``ModelConfig.layer_kinds`` (config.py:134-137);
* ``Block``: pre-norm residual attention + MLP (model.py:317-339);
* ``DilutionLM``: embedding tied to the LM head, blocks, final norm;
  ``forward(idx, targets)`` -> (logits, loss), ``prefill``, ``decode_step``
  and cached greedy / sampled ``generate`` (model.py:342-512, sampling with
  ``filter_logits``, model.py:289-304);
* ``rows_linear``: the decode step's projections at M = batch (<= 8 rows) on
  the HIP library (``dil_rows_linear``), with the RMSNorms, the residual adds
  and the SwiGLU activation folded in: a bf16 model's cached decode step (eager
  and graph-replayed) runs four of them per layer instead of torch's GEMMs and
  elementwise ops, which read the weights at a fraction of HBM speed at M = 8.

The reference normalises with LayerNorm and sizes SwiGLU at 8/3 d_model; the
model-level benchmark configuration asks for RMSNorm and a 4x SwiGLU, which
``LMConfig`` selects here.  There is no eager fallback: the attention layers
run only on the HIP kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import _hip
from . import cache as dcache
from . import kernels
from . import kernels_bid

# dil_rows_linear modes
_LIN_PLAIN, _LIN_RESID, _LIN_NORM, _LIN_SWIGLU = 0, 1, 2, 3
_LIN_MAX_ROWS, _LIN_MAX_K = 8, 4096


def rows_linear(x: torch.Tensor, w1: torch.Tensor, mode: int, *, w2: torch.Tensor | None = None,
                g: torch.Tensor | None = None, resid: torch.Tensor | None = None,
                eps: float = 0.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """A few-row projection on the HIP library (``dil_rows_linear``): for
    bf16 x (rows, K) with rows <= 8 and nn.Linear weights (N, K), mode 0
    returns x W1^T, 1 resid + x W1^T, 2 rmsnorm(x; g, eps) W1^T, 3
    silu(r W1^T) * (r W2^T) with r = rmsnorm(x; g, eps), rounded to bf16 where
    the separate torch ops round.  (No reference counterpart: the reference
    model runs these through torch.nn.Linear, model.py:41-93.)"""
    if x.dim() != 2 or w1.dim() != 2:
        raise ValueError("rows_linear takes x (rows, K) and a weight (N, K)")
    rows, k = x.shape
    n = w1.shape[0]
    for t in (x, w1, w2, g, resid):
        if t is not None and (t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != x.device):
            raise ValueError("rows_linear takes contiguous bf16 tensors on one device")
    # the kernel indexes every operand with the rows, N and K given here
    if w1.shape[1] != k:
        raise ValueError(f"rows_linear: weight {tuple(w1.shape)} does not match x {tuple(x.shape)}")
    if w2 is not None and w2.shape != w1.shape:
        raise ValueError(f"rows_linear: w2 {tuple(w2.shape)} must have w1's shape {tuple(w1.shape)}")
    if g is not None and g.shape != (k,):
        raise ValueError(f"rows_linear: the norm weight must have shape ({k},), got {tuple(g.shape)}")
    if resid is not None and resid.shape != (rows, n):
        raise ValueError(f"rows_linear: resid must have shape ({rows}, {n}), got {tuple(resid.shape)}")
    if mode in (_LIN_NORM, _LIN_SWIGLU) and g is None:
        raise ValueError("rows_linear: the normed modes need the norm weight g")
    if mode == _LIN_SWIGLU and w2 is None:
        raise ValueError("rows_linear: the SwiGLU mode needs w2")
    if mode == _LIN_RESID and resid is None:
        raise ValueError("rows_linear: the residual mode needs resid")
    lib = _hip.lib()
    if out is None:
        out = torch.empty(rows, n, device=x.device, dtype=x.dtype)
    elif out.shape != (rows, n) or out.dtype != torch.bfloat16 or not out.is_contiguous() or out.device != x.device:
        raise ValueError("out must be a contiguous bf16 (rows, N) tensor on the inputs' device")
    status = lib.dil_rows_linear(x.data_ptr(), w1.data_ptr(), None if w2 is None else w2.data_ptr(),
                                 None if g is None else g.data_ptr(), None if resid is None else resid.data_ptr(),
                                 out.data_ptr(), rows, n, k, mode, 1, float(eps),
                                 kernels._stream(x.device))
    _hip.check(status, "dil_rows_linear")
    return out


def rows_linear_qkv(x: torch.Tensor, w: torch.Tensor, g: torch.Tensor, eps: float, k_cache: torch.Tensor,
                    v_cache: torch.Tensor, pos) -> torch.Tensor:
    """The decode step's RMSNorm + q/k/v projection with the cache append
    folded in (``dil_rows_linear_qkv``): [q | k | v] = rmsnorm(x; g, eps)
    w^T for c_attn's weight w (3 d_model, d_model); k and v go to row `pos`
    of the (B, H, capacity, D) caches, q is returned as (B, d_model).  `pos`
    is a Python int or a one-element int64 tensor on the device (read when
    the kernel runs, as in a graph replay).  (No reference counterpart: the
    reference projects with c_attn and writes its cache as separate ops,
    model.py:41-93.)"""
    if x.dim() != 2 or k_cache.dim() != 4:
        raise ValueError("rows_linear_qkv takes x (B, d_model) and (B, H, capacity, D) caches")
    rows, k = x.shape
    batch, heads, capacity, head_dim = k_cache.shape
    for t in (x, w, g, k_cache, v_cache):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != x.device:
            raise ValueError("rows_linear_qkv takes contiguous bf16 tensors on one device")
    if batch != rows or v_cache.shape != k_cache.shape or w.shape != (3 * heads * head_dim, k):
        raise ValueError("rows_linear_qkv: x, w and the caches disagree in shape")
    if g.shape != (k,):
        raise ValueError(f"rows_linear_qkv: the norm weight must have shape ({k},), got {tuple(g.shape)}")
    lib = _hip.lib()
    q = torch.empty(rows, heads * head_dim, device=x.device, dtype=x.dtype)
    if torch.is_tensor(pos):
        if pos.dtype != torch.int64 or pos.numel() != 1 or pos.device != x.device:
            raise ValueError("a device position is a one-element int64 tensor on the inputs' device")
        pos_dev, pos_host = pos.data_ptr(), 0
    else:
        pos_dev, pos_host = None, int(pos)
    status = lib.dil_rows_linear_qkv(x.data_ptr(), w.data_ptr(), g.data_ptr(), q.data_ptr(), k_cache.data_ptr(),
                                     v_cache.data_ptr(), rows, heads, head_dim, capacity, pos_dev, pos_host, k, 1,
                                     float(eps), kernels._stream(x.device))
    _hip.check(status, "dil_rows_linear_qkv")
    return q


def rows_argmax(logits: torch.Tensor, limit: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy tokens from bf16 logits (rows, V) on the HIP library
    (``dil_rows_argmax``): per row the index of the largest of the first
    ``limit`` (default V) values, as torch.argmax picks it; returned as an
    int64 (rows, 1) tensor, written into ``out`` when given.  (No reference
    counterpart: the reference's sampler calls torch.argmax,
    model.py:473-509.)"""
    rows, vocab = logits.shape
    limit = vocab if limit is None else int(limit)
    if logits.dtype != torch.bfloat16 or logits.stride(1) != 1 or not 0 < limit <= vocab:
        raise ValueError("rows_argmax takes bf16 (rows, V) logits with unit column stride and 0 < limit <= V")
    if out is None:
        out = torch.empty(rows, 1, device=logits.device, dtype=torch.int64)
    elif out.dtype != torch.int64 or out.numel() != rows or not out.is_contiguous() or out.device != logits.device:
        raise ValueError("out must be a contiguous int64 tensor of one element per row")
    status = _hip.lib().dil_rows_argmax(logits.data_ptr(), rows, logits.stride(0), limit, out.data_ptr(), 1,
                                        kernels._stream(logits.device))
    _hip.check(status, "dil_rows_argmax")
    return out

@dataclass
class LMConfig:
    vocab_size: int = 50304
    n_layers: int = 12
    d_model: int = 1024
    n_heads: int = 16
    mlp_ratio: float = 4.0          # SwiGLU hidden = mlp_ratio * d_model
    norm: str = "rms"               # "rms" or "layer"
    prefill_chunk: int | None = 2048
    attention: str = "dilution"     # default slot type: "dilution" or "softmax"
    layer_attention: list | None = None
    bid: str = "softmax"            # bid function of the dilution slots (kernels_bid.BID_TYPES)
    share_cumsum: bool | str = True # True: dilution share, "exclusive", False: no share step
    context_length: int = 16384     # the SHIFT of the expshift / sigshift bids (config.py:68-72)

    def __post_init__(self):
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        if self.norm not in ("rms", "layer"):
            raise ValueError("norm must be 'rms' or 'layer'")
        if self.layer_attention is not None and len(self.layer_attention) != self.n_layers:
            raise ValueError(f"layer_attention must list {self.n_layers} entries")
        bad = sorted(set(self.layer_kinds()) - set(ATTENTION_TYPES))
        if bad:
            raise ValueError(f"attention kinds must be in {ATTENTION_TYPES}; got {bad}")
        # config.py:111-116
        if not (isinstance(self.share_cumsum, bool) or self.share_cumsum == "exclusive"):
            raise ValueError('share_cumsum must be a boolean or "exclusive"')
        if self.bid not in kernels_bid.BID_TYPES:
            raise ValueError(f"bid must be one of {kernels_bid.BID_TYPES}; got {self.bid!r}")
        if not self.production_operator() and self.d_model // self.n_heads not in kernels_bid.VARIANT_HEAD_DIMS:
            raise ValueError(f"the bid / share ablations need head_dim in {kernels_bid.VARIANT_HEAD_DIMS}")

    def production_operator(self) -> bool:
        """softmax bids with the dilution share: the operator of ``kernels``."""
        return self.bid == "softmax" and self.share_cumsum is True

    def layer_kinds(self) -> list[str]:
        if self.layer_attention is not None:
            return list(self.layer_attention)
        return [self.attention] * self.n_layers


ATTENTION_TYPES = ("dilution", "softmax")


def _norm(cfg: LMConfig) -> nn.Module:
    if cfg.norm == "rms":
        return nn.RMSNorm(cfg.d_model, eps=1e-5)
    return nn.LayerNorm(cfg.d_model, eps=1e-5)


class _AttentionBase(nn.Module):
    """Fused q/k/v projection and output projection shared by both slot
    types (model.py:41-93)."""

    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.n_heads = cfg.n_heads
        self.d_model = cfg.d_model
        self.c_attn = nn.Linear(cfg.d_model, 3 * cfg.d_model, bias=False)
        self.c_proj = nn.Linear(cfg.d_model, cfg.d_model, bias=False)
        self.prefill_chunk = cfg.prefill_chunk

    def _split_heads(self, x: torch.Tensor):
        batch, seq, _ = x.shape
        q, k, v = self.c_attn(x).split(self.d_model, dim=2)
        shape = (batch, seq, self.n_heads, self.d_model // self.n_heads)
        return (t.view(shape).transpose(1, 2) for t in (q, k, v))

    def _merge_heads(self, y: torch.Tensor, batch: int, seq: int) -> torch.Tensor:
        return self.c_proj(y.transpose(1, 2).contiguous().view(batch, seq, self.d_model))


def _sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool) -> torch.Tensor:
    """torch SDPA; half-precision inputs are kept off the math backend, whose
    batched products take a transposed bf16 operand."""
    if q.dtype == torch.float32:
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal)


class SoftmaxAttention(_AttentionBase):
    """Causal softmax attention (torch SDPA): the parameter-matched control."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        batch, seq, _ = x.shape
        q, k, v = self._split_heads(x)
        return self._merge_heads(_sdpa(q, k, v, True), batch, seq)

    def begin_cache(self, x: torch.Tensor, capacity: int | None = None):
        batch, seq, _ = x.shape
        q, k, v = self._split_heads(x)
        y = self._merge_heads(_sdpa(q, k, v, True), batch, seq)
        return y, dcache.alloc_cache(k, v, capacity)

    def step_cache(self, x1: torch.Tensor, cache: dict) -> torch.Tensor:
        batch = x1.shape[0]
        q1, k1, v1 = self._split_heads(x1)
        t = dcache.append_kv(cache, k1, v1)
        y = _sdpa(q1, cache["k"][:, :, :t], cache["v"][:, :, :t], False)
        return self._merge_heads(y, batch, 1)


class DilutionAttention(_AttentionBase):
    """The dilution operator on the HIP kernels (model.py:120-257): the
    production operator through ``kernels``, an ablation variant (bid,
    share_cumsum) through ``kernels_bid`` (model.py:142-156)."""

    def __init__(self, cfg: LMConfig):
        super().__init__(cfg)
        self.production = cfg.production_operator()
        self.bid_kw = {} if self.production else {
            "bid": cfg.bid, "share_cumsum": cfg.share_cumsum, "shift": float(cfg.context_length)}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        batch, seq, _ = x.shape
        q, k, v = self._split_heads(x)
        prec = "bf16" if q.dtype == torch.bfloat16 else "tf32"
        ops = kernels if self.production else kernels_bid
        if torch.is_grad_enabled():
            y = ops.dilution_attention(q, k, v, dot_precision=prec, **self.bid_kw)
        else:
            y = ops.dilution_attention_forward(q, k, v, dot_precision=prec, **self.bid_kw)
        return self._merge_heads(y.to(x.dtype), batch, seq)

    def begin_cache(self, x: torch.Tensor, capacity: int | None = None):
        batch, seq, _ = x.shape
        q, k, v = self._split_heads(x)
        y, cache = dcache.begin_cache(q, k.contiguous(), v.contiguous(), capacity=capacity,
                                      chunk=self.prefill_chunk, **self.bid_kw)
        return self._merge_heads(y.to(x.dtype), batch, seq), cache

    def step_cache(self, x1: torch.Tensor, cache: dict) -> torch.Tensor:
        batch = x1.shape[0]
        q1, k1, v1 = self._split_heads(x1)
        y = dcache.step_cache(q1, k1, v1, cache, **self.bid_kw)
        return self._merge_heads(y.to(x1.dtype), batch, 1)


class SwiGLUMLP(nn.Module):
    def __init__(self, cfg: LMConfig):
        super().__init__()
        hidden = int(cfg.mlp_ratio * cfg.d_model)
        self.gate_proj = nn.Linear(cfg.d_model, hidden, bias=False)
        self.up_proj = nn.Linear(cfg.d_model, hidden, bias=False)
        self.down_proj = nn.Linear(hidden, cfg.d_model, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


_ATTENTION_CLASSES = {"dilution": DilutionAttention, "softmax": SoftmaxAttention}


class Block(nn.Module):
    def __init__(self, cfg: LMConfig, kind: str = "dilution"):
        super().__init__()
        self.ln_1 = _norm(cfg)
        self.attn = _ATTENTION_CLASSES[kind](cfg)
        self.ln_2 = _norm(cfg)
        self.mlp = SwiGLUMLP(cfg)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))

    def begin_cache(self, x: torch.Tensor, capacity: int | None = None):
        y, cache = self.attn.begin_cache(self.ln_1(x), capacity)
        x = x + y
        return x + self.mlp(self.ln_2(x)), cache

    def step_cache(self, x1: torch.Tensor, cache: dict) -> torch.Tensor:
        x1 = x1 + self.attn.step_cache(self.ln_1(x1), cache)
        return x1 + self.mlp(self.ln_2(x1))


class DilutionLM(nn.Module):
    """Decoder-only LM over dilution / softmax attention slots, tied
    embeddings, no position encoding (in dilution layers the demand cumsum
    supplies the order asymmetry)."""

    def __init__(self, cfg: LMConfig):
        super().__init__()
        self.cfg = cfg
        self.wte = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.h = nn.ModuleList([Block(cfg, kind) for kind in cfg.layer_kinds()])
        self.ln_f = _norm(cfg)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        self.wte.weight = self.lm_head.weight
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module: nn.Module) -> None:
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def num_parameters(self) -> int:
        return sum(p.numel() for p in self.parameters())

    def hidden_states(self, idx: torch.Tensor) -> torch.Tensor:
        """Final-norm hidden states (B, T, d_model) of one causal forward."""
        x = self.wte(idx)
        for block in self.h:
            x = block(x)
        return self.ln_f(x)

    def forward(self, idx: torch.Tensor, targets: torch.Tensor | None = None):
        x = self.hidden_states(idx)
        if targets is None:
            return self.lm_head(x[:, [-1], :]), None
        logits = self.lm_head(x)
        loss = F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.reshape(-1),
                               ignore_index=-100)
        return logits, loss

    @torch.no_grad()
    def prefill(self, idx: torch.Tensor, capacity: int | None = None):
        x = self.wte(idx)
        caches = []
        for block in self.h:
            x, cache = block.begin_cache(x, capacity)
            caches.append(cache)
        return self.lm_head(self.ln_f(x[:, [-1], :])), caches

    @torch.no_grad()
    def decode_step(self, token: torch.Tensor, caches, fused: bool = True) -> torch.Tensor:
        """Logits (B, 1, vocab) of the next position from the caches; a bf16
        model runs its projections on ``rows_linear`` (``fused=False`` keeps
        torch's modules, the same computation up to accumulation order)."""
        batch = token.shape[0]
        if fused and self.fused_decode_eligible(batch):
            def slot(i):
                cache = caches[i]
                t = cache["len"]
                if t >= cache["k"].shape[2]:
                    raise ValueError("decode step past the cache capacity (context_length)")
                cache["len"] = t + 1
                return cache["k"], cache["v"], t

            def attend(i, q1):
                c = caches[i]
                return kernels.dilution_decode_step(q1, c["k"], c["v"], c["committed"], c["len"])

            x2 = self._fused_layers(self.wte(token).view(batch, -1), slot, attend)
            return self._fused_head(x2)
        x = self.wte(token)
        for block, cache in zip(self.h, caches):
            x = block.step_cache(x, cache)
        return self.lm_head(self.ln_f(x))

    def graph_decode_eligible(self) -> bool:
        """Every layer runs the production dilution operator (the decode step
        GraphDecoder captures)."""
        return all(isinstance(b.attn, DilutionAttention) and b.attn.production for b in self.h)

    def fused_decode_eligible(self, batch: int) -> bool:
        """The cached decode step can run on ``rows_linear``: every layer on
        the production dilution operator, bf16 weights on the GPU, RMSNorm
        with weights, d_model and the MLP width multiples of 256 up to 4096,
        and at most 8 sequences."""
        cfg = self.cfg
        hidden = int(cfg.mlp_ratio * cfg.d_model)
        w = self.lm_head.weight
        return (self.graph_decode_eligible() and kernels.HAS_HIP and w.is_cuda and w.dtype == torch.bfloat16
                and cfg.norm == "rms" and self.ln_f.weight is not None
                and all(b.ln_1.weight is not None and b.ln_2.weight is not None for b in self.h)
                and cfg.d_model % 256 == 0 and cfg.d_model <= _LIN_MAX_K
                and hidden % 256 == 0 and hidden <= _LIN_MAX_K and 1 <= batch <= _LIN_MAX_ROWS)

    @staticmethod
    def _norm_eps(norm: nn.Module) -> float:
        return norm.eps if norm.eps is not None else torch.finfo(torch.bfloat16).eps

    def _fused_layers(self, x2: torch.Tensor, slot, attend) -> torch.Tensor:
        """The blocks of one decode step on ``rows_linear`` (B, d_model) ->
        (B, d_model): per layer norm + q/k/v projection with k and v written
        to ``slot(i)`` = (k_cache, v_cache, position) (an int or a device
        tensor), ``attend(i, q1)`` (the layer's decode step over the cache with
        the new row, (B, H, 1, D)), output projection + residual, norm +
        gate/up projections + SwiGLU, down projection + residual."""
        batch, d = x2.shape
        for i, block in enumerate(self.h):
            at, mlp = block.attn, block.mlp
            k_cache, v_cache, pos = slot(i)
            q = rows_linear_qkv(x2, at.c_attn.weight, block.ln_1.weight, self._norm_eps(block.ln_1), k_cache,
                                v_cache, pos)
            y = attend(i, q.view(batch, at.n_heads, 1, d // at.n_heads)).reshape(batch, d)
            x2 = rows_linear(y, at.c_proj.weight, _LIN_RESID, resid=x2)
            h = rows_linear(x2, mlp.gate_proj.weight, _LIN_SWIGLU, w2=mlp.up_proj.weight, g=block.ln_2.weight,
                            eps=self._norm_eps(block.ln_2))
            x2 = rows_linear(h, mlp.down_proj.weight, _LIN_RESID, resid=x2)
        return x2

    def _fused_head(self, x2: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        logits = rows_linear(x2, self.lm_head.weight, _LIN_NORM, g=self.ln_f.weight, eps=self._norm_eps(self.ln_f),
                             out=out)
        return logits.view(x2.shape[0], 1, -1)

    @torch.no_grad()
    def generate(self, idx: torch.Tensor, max_new_tokens: int, temperature: float = 0.0,
                 top_k: int | None = None, top_p: float | None = None,
                 generator: torch.Generator | None = None, vocab_limit: int | None = None,
                 graph: bool = False) -> torch.Tensor:
        """Cached generation with caches sized prompt + max_new_tokens
        (model.py:473-509): temperature 0 is greedy, otherwise a sample of
        softmax(logits / temperature) after top-k / nucleus truncation;
        ``generator`` makes sampling reproducible, ``vocab_limit`` keeps the
        new tokens below that id.  ``graph=True`` runs greedy decoding of an
        all-dilution production stack through ``GraphDecoder`` (the same
        tokens, one HIP graph replay per step)."""
        if vocab_limit is not None and not 0 < vocab_limit <= self.cfg.vocab_size:
            raise ValueError(f"vocab_limit must be in (0, {self.cfg.vocab_size}]")
        logits, caches = self.prefill(idx, capacity=idx.shape[1] + max_new_tokens)
        tokens = idx
        if graph and max_new_tokens > 0 and not (temperature and temperature > 0.0) and self.graph_decode_eligible():
            last = logits[:, -1, :].float()
            if vocab_limit is not None:
                last[:, vocab_limit:] = float("-inf")
            nxt = last.argmax(dim=-1, keepdim=True)
            out = [nxt]
            if max_new_tokens > 1:
                dec = GraphDecoder(self, caches, nxt, vocab_limit=vocab_limit)
                for _ in range(max_new_tokens - 1):
                    out.append(dec.step().clone())
            return torch.cat([tokens, *out], dim=1)
        for step in range(max_new_tokens):
            greedy = not (temperature and temperature > 0.0)
            if greedy and logits.dtype == torch.bfloat16 and logits.is_cuda and kernels.HAS_HIP:
                # torch.argmax's pick over the first vocab_limit logits, on the device
                nxt = rows_argmax(logits[:, -1, :], vocab_limit)
            else:
                last = logits[:, -1, :].float()
                if vocab_limit is not None:
                    last[:, vocab_limit:] = float("-inf")
                if greedy:
                    nxt = last.argmax(dim=-1, keepdim=True)
                else:
                    probs = filter_logits(last / temperature, top_k=top_k, top_p=top_p).softmax(dim=-1)
                    nxt = torch.multinomial(probs, 1, generator=generator)
            tokens = torch.cat([tokens, nxt], dim=1)
            if step + 1 < max_new_tokens:
                logits = self.decode_step(nxt, caches)
        return tokens


class GraphDecoder:
    """Greedy decoding of an all-dilution, production-operator LM with each
    token's step captured once as a HIP graph and replayed.

    One step is: the embedding of the last token; per layer the norm, the q/k/v
    projection, the cache append at a device-resident position
    (``index_copy_``), the decode step with its length in device memory
    (``kernels.decode_step_device_length``), the output projection and the
    MLP; then the head, the argmax that becomes the next step's token, and the
    position and length advanced by one on the device.  With nothing on the
    host changing from step to step, one capture serves every step up to the
    caches' capacity, and each step is a single graph launch.

    ``caches`` come from ``DilutionLM.prefill`` (sized for the whole
    generation); ``token`` (B, 1) is the token the first step consumes.  The
    first ``step()`` runs eagerly (the capture's warm-up, on a side stream) and
    then captures; later calls replay.  ``step()`` returns the (B, 1) token
    buffer the step wrote (overwritten by the next step: clone to keep it);
    ``logits`` holds that step's (B, 1, vocab) logits.  The caches' ``len``
    follows the steps taken.
    """

    def __init__(self, model: "DilutionLM", caches: list, token: torch.Tensor,
                 vocab_limit: int | None = None, fused: bool = True):
        if not model.graph_decode_eligible():
            raise ValueError("GraphDecoder needs every layer on the production dilution operator")
        self.model, self.caches = model, caches
        k0 = caches[0]["k"]
        self.batch, self.heads, self.capacity, self.head_dim = k0.shape
        self.len = caches[0]["len"]
        if any(c["len"] != self.len or c["k"].shape != k0.shape for c in caches):
            raise ValueError("every layer's cache must hold the same length and shape")
        dev = k0.device
        self.tok = token.detach().clone().to(device=dev, dtype=torch.long).view(self.batch, 1)
        self.pos = torch.full((1,), self.len, dtype=torch.long, device=dev)      # next write position
        self.live = torch.full((1,), self.len + 1, dtype=torch.long, device=dev)  # length after it
        qdt = model.lm_head.weight.dtype
        self.outs = [torch.empty(self.batch, self.heads, self.head_dim, device=dev, dtype=qdt)
                     for _ in caches]
        self.ws = kernels.decode_workspace(self.batch, self.heads, self.capacity, self.head_dim, dev)
        self.logits = torch.empty(self.batch, 1, model.cfg.vocab_size, device=dev, dtype=qdt)
        self.mask = None
        self.limit = model.cfg.vocab_size if vocab_limit is None else int(vocab_limit)
        if vocab_limit is not None:
            self.mask = torch.zeros(model.cfg.vocab_size, dtype=torch.bool, device=dev)
            self.mask[vocab_limit:] = True          # positions that never win (NaN included)
        self.fused = fused and model.fused_decode_eligible(self.batch)
        self.graph = None

    def _attend(self, i: int, q1, k1, v1) -> torch.Tensor:
        """Layer i's cache append at the device-resident position and its
        decode step at the device-resident length."""
        cache = self.caches[i]
        cache["k"].index_copy_(2, self.pos, k1)
        cache["v"].index_copy_(2, self.pos, v1)
        return kernels.decode_step_device_length(q1, cache["k"], cache["v"], cache["committed"], self.live,
                                                 self.capacity, out=self.outs[i], workspace=self.ws)

    def _slot(self, i: int):
        cache = self.caches[i]
        return cache["k"], cache["v"], self.pos

    def _attend_q(self, i: int, q1) -> torch.Tensor:
        cache = self.caches[i]
        return kernels.decode_step_device_length(q1, cache["k"], cache["v"], cache["committed"], self.live,
                                                 self.capacity, out=self.outs[i], workspace=self.ws)

    def _body(self) -> None:
        m = self.model
        if self.fused:
            # the head writes the logits buffer and the greedy pick the token
            # buffer directly: no copies, no fp32 logits
            x2 = m._fused_layers(m.wte(self.tok).view(self.batch, -1), self._slot, self._attend_q)
            m._fused_head(x2, out=self.logits.view(self.batch, -1))
            rows_argmax(self.logits.view(self.batch, -1), self.limit, out=self.tok)
        else:
            x = m.wte(self.tok)
            for i, block in enumerate(m.h):
                q1, k1, v1 = block.attn._split_heads(block.ln_1(x))
                y = self._attend(i, q1, k1, v1)
                x = x + block.attn._merge_heads(y.to(x.dtype), self.batch, 1)
                x = x + block.mlp(block.ln_2(x))
            logits = m.lm_head(m.ln_f(x))
            self.logits.copy_(logits)
            last = logits[:, -1, :].float()
            if self.mask is not None:
                last = last.masked_fill(self.mask, float("-inf"))
            self.tok.copy_(last.argmax(dim=-1, keepdim=True))
        self.pos.add_(1)
        self.live.add_(1)

    @torch.no_grad()
    def step(self) -> torch.Tensor:
        if self.len >= self.capacity:
            raise ValueError("decode step past the cache capacity (context_length)")
        if self.graph is None:
            side = torch.cuda.Stream(device=self.tok.device)
            side.wait_stream(torch.cuda.current_stream(self.tok.device))
            with torch.cuda.stream(side):
                self._body()                       # a real step: warms up the libraries
            torch.cuda.current_stream(self.tok.device).wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self._body()                       # recorded, not run
        else:
            self.graph.replay()
        self.len += 1
        for c in self.caches:
            c["len"] = self.len
        return self.tok


def filter_logits(logits: torch.Tensor, top_k: int | None = None, top_p: float | None = None) -> torch.Tensor:
    """Top-k, then nucleus (top-p) truncation of (..., vocab) logits; the
    dropped entries become -inf.  The nucleus is the shortest run of the most
    likely tokens whose probability reaches top_p; the most likely token always
    stays (model.py:289-304)."""
    out = logits
    if top_k is not None and top_k > 0:
        floor = out.topk(min(int(top_k), out.shape[-1]), dim=-1).values[..., -1:]
        out = out.masked_fill(out < floor, float("-inf"))
    if top_p is not None and top_p < 1.0:
        vals, order = out.sort(dim=-1, descending=True)
        probs = vals.softmax(dim=-1)
        mass_before = probs.cumsum(dim=-1) - probs
        vals = vals.masked_fill(mass_before >= top_p, float("-inf"))
        out = torch.empty_like(out).scatter_(-1, order, vals)
    return out
