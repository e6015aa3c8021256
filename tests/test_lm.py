"""Whole-model invariants of the LM harness (dilution.lm), the pattern of
the reference's tests/test_model.py:

* causality: logits at positions < t do not depend on tokens >= t
  (test_model.py:46-56);
* cached decode reproduces the teacher-forced full forward
  (test_model.py:99-110) -- here through chunked prefill and the HIP decode
  step, and through the softmax control's KV cache in mixed stacks;
* a bf16 training step produces a finite loss and finite gradients in
  every parameter;
* the bid / share ablations (``LMConfig.bid``, ``share_cumsum``): the model on
  the variant kernels matches the same model on the plain-torch variant
  specification (test_kernels.py:360-374, same 5e-2 logit bound), and their
  cached decode reproduces the full forward.
"""

from __future__ import annotations

import pytest
import torch

from gpu_helpers import needs_gpu


def _small(dtype=torch.float32, chunk=16, kinds=None, **variant):
    from dilution.lm import DilutionLM, LMConfig

    if variant:                                   # the ablation variants take head_dim 64
        cfg = LMConfig(vocab_size=97, n_layers=2, d_model=128, n_heads=2, prefill_chunk=chunk,
                       layer_attention=kinds, context_length=96, **variant)
    else:
        cfg = LMConfig(vocab_size=97, n_layers=2, d_model=64, n_heads=4, prefill_chunk=chunk,
                       layer_attention=kinds)
    torch.manual_seed(0)
    return DilutionLM(cfg).to(device="cuda", dtype=dtype).eval()


def test_rows_linear_rejects_mismatched_shapes():
    """The few-row projections check every operand's shape before a launch:
    the kernel indexes them with the rows, N and K of x and w1, so a
    mismatched weight, norm weight or residual raises ValueError on the host
    (CPU tensors: the checks run before the library is touched)."""
    from dilution.lm import rows_linear, rows_linear_qkv

    bf = torch.bfloat16
    x = torch.zeros(4, 256, dtype=bf)
    w = torch.zeros(512, 256, dtype=bf)
    g = torch.ones(256, dtype=bf)
    bad = [
        dict(w1=torch.zeros(512, 128, dtype=bf), mode=0),                          # K mismatch
        dict(w1=w, mode=3, w2=torch.zeros(256, 256, dtype=bf), g=g),              # w2 shape
        dict(w1=w, mode=2, g=torch.ones(128, dtype=bf)),                           # norm weight
        dict(w1=w, mode=1, resid=torch.zeros(4, 256, dtype=bf)),                   # resid shape
        dict(w1=w, mode=2),                                                        # no norm weight
        dict(w1=w, mode=3, g=g),                                                   # no w2
        dict(w1=w, mode=1),                                                        # no resid
        dict(w1=torch.zeros(512, 256, dtype=torch.float32), mode=0),               # dtype
    ]
    for kw in bad:
        w1, mode = kw.pop("w1"), kw.pop("mode")
        with pytest.raises(ValueError):
            rows_linear(x, w1, mode, **kw)
    kc = torch.zeros(4, 2, 32, 128, dtype=bf)
    with pytest.raises(ValueError):                                                # norm weight
        rows_linear_qkv(x, torch.zeros(768, 256, dtype=bf), torch.ones(255, dtype=bf), 1e-5, kc, kc.clone(), 0)
    with pytest.raises(ValueError):                                                # c_attn shape
        rows_linear_qkv(x, torch.zeros(512, 256, dtype=bf), g, 1e-5, kc, kc.clone(), 0)


def test_config_validation():
    from dilution.lm import LMConfig

    with pytest.raises(ValueError):
        LMConfig(d_model=100, n_heads=16)
    with pytest.raises(ValueError):
        LMConfig(norm="batch")
    with pytest.raises(ValueError):
        LMConfig(n_layers=2, layer_attention=["dilution"])
    with pytest.raises(ValueError):
        LMConfig(attention="linear")
    assert LMConfig(n_layers=2, layer_attention=["softmax", "dilution"]).layer_kinds() == [
        "softmax", "dilution"]
    with pytest.raises(ValueError):
        LMConfig(bid="tanh")
    with pytest.raises(ValueError):
        LMConfig(share_cumsum="inclusive")
    with pytest.raises(ValueError):
        LMConfig(d_model=384, n_heads=8, bid="relu")             # head_dim 48: no variant build
    assert not LMConfig(d_model=256, n_heads=8, bid="relu").production_operator()   # head_dim 32
    assert LMConfig(d_model=256, n_heads=8).production_operator()
    assert not LMConfig(d_model=256, n_heads=4, share_cumsum=False).production_operator()


def test_dilution_operator_is_parameter_free():
    """The dilution slot holds exactly the softmax control's parameters
    (test_model.py:184-195): the order asymmetry comes from the cumsum alone."""
    from dilution.lm import DilutionLM, LMConfig

    def count(kind):
        cfg = LMConfig(vocab_size=97, n_layers=2, d_model=64, n_heads=4, attention=kind)
        return sum(p.numel() for p in DilutionLM(cfg).parameters())

    assert count("dilution") == count("softmax")
    cfg = LMConfig(vocab_size=97, n_layers=1, d_model=64, n_heads=4)
    names = {n for n, _ in DilutionLM(cfg).h[0].attn.named_parameters()}
    assert names == {"c_attn.weight", "c_proj.weight"}, names


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("kinds", [None, ["softmax", "dilution"]])
def test_lm_causality(kinds):
    model = _small(kinds=kinds)
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, 97, (2, 40), generator=g).cuda()
    idx2 = idx.clone()
    idx2[:, 25:] = (idx2[:, 25:] + 7) % 97
    with torch.no_grad():
        x1 = model.ln_f(_hidden(model, idx))
        x2 = model.ln_f(_hidden(model, idx2))
    assert torch.allclose(x1[:, :25], x2[:, :25], atol=1e-5)
    assert not torch.allclose(x1[:, 25:], x2[:, 25:], atol=1e-3)


def _hidden(model, idx):
    x = model.wte(idx)
    for block in model.h:
        x = block(x)
    return x


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("chunk,kinds", [(None, None), (16, None), (16, ["dilution", "softmax"])])
def test_cached_decode_matches_full_forward(chunk, kinds):
    model = _small(chunk=chunk, kinds=kinds)
    g = torch.Generator().manual_seed(2)
    idx = torch.randint(0, 97, (2, 50), generator=g).cuda()
    prompt = 37
    with torch.no_grad():
        full = model.lm_head(model.ln_f(_hidden(model, idx)))
        logits, caches = model.prefill(idx[:, :prompt], capacity=idx.shape[1])
        assert torch.allclose(logits[:, 0], full[:, prompt - 1], atol=1e-4)
        for t in range(prompt, idx.shape[1]):
            logits = model.decode_step(idx[:, t:t + 1], caches)
            assert torch.allclose(logits[:, 0], full[:, t], atol=1e-4), t


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("kinds", [None, ["softmax", "dilution"]])
def test_training_step_bf16_finite(kinds):
    model = _small(dtype=torch.bfloat16, kinds=kinds).train()
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 97, (2, 64), generator=g).cuda()
    _, loss = model(idx[:, :-1], idx[:, 1:])
    loss.backward()
    assert torch.isfinite(loss)
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), name


@pytest.mark.gpu
@needs_gpu
def test_generate_extends_prompt():
    model = _small()
    idx = torch.zeros(1, 5, dtype=torch.long, device="cuda")
    out = model.generate(idx, 6)
    assert out.shape == (1, 11) and torch.equal(out[:, :5], idx)


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("bid", ["relu", "relu2", "softplus", "minshift", "sigmoid", "expshift", "sigshift"])
def test_variant_model_matches_torch_specification(bid, monkeypatch):
    from dilution import kernels_bid as kb
    from dilution import lm

    model = _small(kinds=["dilution", "softmax"], bid=bid)
    g = torch.Generator().manual_seed(7)
    idx = torch.randint(0, 97, (2, 96), generator=g).cuda()
    with torch.no_grad():
        fused = model.lm_head(model.ln_f(_hidden(model, idx)))
        spec = lambda q, k, v, dot_precision, **kw: kb.dilution_attention_reference(q, k, v, **kw)
        monkeypatch.setattr(lm.kernels_bid, "dilution_attention_forward", spec)
        eager = model.lm_head(model.ln_f(_hidden(model, idx)))
    assert (fused - eager).abs().max().item() < 5e-2


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("bid,share", [("relu2", True), ("minshift", "exclusive"), ("sigshift", False),
                                       ("expshift", True), ("softmax", "exclusive"), ("softmax", False)])
def test_variant_cached_decode_matches_full_forward(bid, share):
    model = _small(kinds=["dilution", "softmax"], bid=bid, share_cumsum=share)
    g = torch.Generator().manual_seed(8)
    idx = torch.randint(0, 97, (2, 50), generator=g).cuda()
    prompt = 37
    with torch.no_grad():
        full = model.lm_head(model.ln_f(_hidden(model, idx)))
        logits, caches = model.prefill(idx[:, :prompt], capacity=idx.shape[1])
        assert torch.allclose(logits[:, 0], full[:, prompt - 1], atol=1e-4)
        for t in range(prompt, idx.shape[1]):
            logits = model.decode_step(idx[:, t:t + 1], caches)
            assert torch.allclose(logits[:, 0], full[:, t], atol=1e-4), t


@pytest.mark.gpu
@needs_gpu
def test_variant_training_step_bf16_finite():
    model = _small(dtype=torch.bfloat16, bid="sigshift", share_cumsum=True).train()
    g = torch.Generator().manual_seed(9)
    idx = torch.randint(0, 97, (2, 64), generator=g).cuda()
    _, loss = model(idx[:, :-1], idx[:, 1:])
    loss.backward()
    assert torch.isfinite(loss)
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), name


def test_filter_logits():
    """Top-k keeps the k largest; the nucleus keeps the shortest most-likely
    prefix reaching top_p; the arg-max always survives."""
    from dilution.lm import filter_logits

    logits = torch.log(torch.tensor([[0.5, 0.2, 0.15, 0.1, 0.05]]))
    kept = lambda out: torch.isfinite(out[0]).nonzero().flatten().tolist()
    assert kept(filter_logits(logits, top_k=2)) == [0, 1]
    assert kept(filter_logits(logits, top_p=0.6)) == [0, 1]        # 0.5 < 0.6 <= 0.7
    assert kept(filter_logits(logits, top_p=0.69)) == [0, 1]       # mass before token 2 is 0.7
    assert kept(filter_logits(logits, top_p=0.01)) == [0]
    assert kept(filter_logits(logits[:, [3, 0, 4, 1, 2]], top_p=0.8)) == [1, 3, 4]   # order-independent
    assert kept(filter_logits(logits, top_k=4, top_p=0.99)) == [0, 1, 2, 3]
    assert torch.equal(filter_logits(logits), logits)


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_decode_replays_match_eager_decode(dtype):
    """Every replay of the captured decode step against the eager step from
    the same state: bitwise equal logits, tokens and caches (the device-length
    decode walks the same key chunks in the same order).  Eager work and a
    synchronisation separate the replays."""
    from dilution.lm import GraphDecoder

    model = _small(dtype=dtype)
    g = torch.Generator().manual_seed(5)
    idx = torch.randint(0, 97, (2, 37), generator=g).cuda()
    cap = 37 + 11
    logits_e, caches_e = model.prefill(idx, capacity=cap)
    logits_g, caches_g = model.prefill(idx, capacity=cap)
    assert torch.equal(logits_e, logits_g)
    tok = logits_e[:, -1, :].float().argmax(dim=-1, keepdim=True)
    dec = GraphDecoder(model, caches_g, tok)
    for step in range(11):
        le = model.decode_step(tok, caches_e)
        tg = dec.step()
        torch.cuda.synchronize()
        assert torch.equal(dec.logits, le), step
        tok = le[:, -1, :].float().argmax(dim=-1, keepdim=True)
        assert torch.equal(tg, tok), step
    for ce, cg in zip(caches_e, caches_g):
        assert cg["len"] == ce["len"] == 37 + 11
        for key in ("k", "v", "committed"):
            assert torch.equal(cg[key], ce[key]), key
    with pytest.raises(ValueError):
        dec.step()                                # the cache is full


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_generate_graph_matches_eager(dtype):
    """Greedy generation replayed and eager give the same tokens, also under a
    vocabulary limit.  A bf16 model's eager steps pick on the device
    (rows_argmax) while its replayed steps at this width take torch.argmax
    of the fp32 logits."""
    model = _small(dtype=dtype)
    idx = torch.zeros(2, 5, dtype=torch.long, device="cuda")
    assert torch.equal(model.generate(idx, 9, graph=True), model.generate(idx, 9))
    assert torch.equal(model.generate(idx, 9, graph=True, vocab_limit=10),
                       model.generate(idx, 9, vocab_limit=10))
    mixed = _small(kinds=["softmax", "dilution"])   # not eligible: the eager steps run
    assert not mixed.graph_decode_eligible()
    assert torch.equal(mixed.generate(idx, 6, graph=True), mixed.generate(idx, 6))
    # no new token returns the prompt, one new token the prefill's pick, on both paths
    for new in (0, 1):
        got, want = model.generate(idx, new, graph=True), model.generate(idx, new)
        assert got.shape == want.shape == (2, 5 + new)
        assert torch.equal(got, want)


@pytest.mark.gpu
@needs_gpu
def test_head_dim_256_bf16_model():
    """A bf16 model with head_dim 256 (d_model 512, 2 heads: the reference
    routes it to its kernels, model.py:158-165) runs on the HIP operator: a
    finite training step, cached decode against the full forward within bf16
    rounding of the logits, every replay of the captured decode step bitwise
    the eager step, and replayed greedy generation equal to eager."""
    from dilution.lm import DilutionLM, GraphDecoder, LMConfig

    cfg = LMConfig(vocab_size=97, n_layers=2, d_model=512, n_heads=2, prefill_chunk=16)
    torch.manual_seed(0)
    model = DilutionLM(cfg).to(device="cuda", dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(7)
    idx = torch.randint(0, 97, (2, 48), generator=g).cuda()
    _, loss = model.train()(idx[:, :-1], idx[:, 1:])
    loss.backward()
    assert torch.isfinite(loss)
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), name
    model.eval()
    prompt = 37
    with torch.no_grad():
        full = model.lm_head(model.ln_f(_hidden(model, idx))).float()
        scale = full.abs().max().item()
        logits, caches = model.prefill(idx[:, :prompt], capacity=idx.shape[1])
        assert (logits[:, 0].float() - full[:, prompt - 1]).abs().max().item() < 5e-2 * scale
        for t in range(prompt, idx.shape[1]):
            logits = model.decode_step(idx[:, t:t + 1], caches)
            assert (logits[:, 0].float() - full[:, t]).abs().max().item() < 5e-2 * scale, t
        logits_e, caches_e = model.prefill(idx[:, :prompt], capacity=prompt + 6)
        _, caches_g = model.prefill(idx[:, :prompt], capacity=prompt + 6)
        tok = logits_e[:, -1, :].float().argmax(dim=-1, keepdim=True)
        dec = GraphDecoder(model, caches_g, tok)
        for step in range(6):
            le = model.decode_step(tok, caches_e)
            dec.step()
            torch.cuda.synchronize()
            assert torch.equal(dec.logits, le), step
            tok = le[:, -1, :].float().argmax(dim=-1, keepdim=True)
    start = torch.zeros(2, 5, dtype=torch.long, device="cuda")
    assert torch.equal(model.generate(start, 7, graph=True), model.generate(start, 7))


@pytest.mark.gpu
@needs_gpu
def test_generate_sampling():
    model = _small()
    idx = torch.zeros(2, 5, dtype=torch.long, device="cuda")
    greedy = model.generate(idx, 6)
    assert torch.equal(model.generate(idx, 6, temperature=1.0, top_k=1), greedy)
    draw = lambda seed: model.generate(idx, 6, temperature=1.3, top_p=0.9,
                                       generator=torch.Generator(device="cuda").manual_seed(seed))
    assert torch.equal(draw(3), draw(3))
    limited = model.generate(idx, 8, temperature=2.0, vocab_limit=10,
                             generator=torch.Generator(device="cuda").manual_seed(4))
    assert (limited[:, 5:] < 10).all()
    with pytest.raises(ValueError):
        model.generate(idx, 2, vocab_limit=0)


# --- the production operator against its specification --------------------

def _spec_forward(q, k, v, dot_precision="ieee", return_aux=False, **_):
    """The operator as the fp32 oracle states it (kernels.py:40-68), with the
    demand totals a prefill hands to the decode cache."""
    from oracle import dilution_oracle as orc

    out = orc.attention_fp32(q.cpu(), k.cpu(), v.cpu()).to(q.device)
    if return_aux:
        return out, {"committed_total": orc.bids(q.float().cpu(), k.float().cpu()).sum(-2)
                     .float().to(q.device)}
    return out


def _spec_decode(q1, k_cache, v_cache, committed, length, **_):
    """The eager cached step (model.py:242-257), advancing the demand in place."""
    from oracle import dilution_oracle as orc

    out, com = orc.decode_step(q1.cpu(), k_cache.cpu(), v_cache.cpu(), committed.cpu(), length,
                               dtype=torch.float64)
    committed.copy_(com.float())
    return out.to(device=q1.device, dtype=q1.dtype)


@pytest.mark.gpu
@needs_gpu
@pytest.mark.parametrize("kinds", [None, ["dilution", "softmax"]])
def test_production_model_matches_specification(kinds, monkeypatch):
    """The model on the HIP operator against the same model on the operator's
    specification (reference test_kernels.py:79-95, whose bound is 2e-2 for
    tf32 noise; fp32 operands here)."""
    from dilution import lm

    model = _small(kinds=kinds)
    g = torch.Generator().manual_seed(11)
    idx = torch.randint(0, 97, (2, 96), generator=g).cuda()
    with torch.no_grad():
        fused = model.lm_head(model.ln_f(_hidden(model, idx)))
        monkeypatch.setattr(lm.kernels, "dilution_attention_forward", _spec_forward)
        spec = model.lm_head(model.ln_f(_hidden(model, idx)))
    assert torch.isfinite(fused).all()
    err = (fused - spec).abs().max().item()
    assert err < 1e-4, err


@pytest.mark.gpu
@needs_gpu
def test_production_cached_decode_matches_specification(monkeypatch):
    """Prefill + cached decode on the HIP kernels against the eager cached
    decode of the specification and against the full forward (reference
    test_kernels.py:245-273)."""
    from dilution import cache as dcache
    from dilution import lm

    model = _small(chunk=None)
    g = torch.Generator().manual_seed(12)
    tokens = torch.randint(0, 97, (2, 40), generator=g).cuda()
    prefix = 24

    def run():
        logits, caches = model.prefill(tokens[:, :prefix], capacity=tokens.shape[1])
        outs = [logits[:, -1]]
        for pos in range(prefix, tokens.shape[1]):
            outs.append(model.decode_step(tokens[:, pos:pos + 1], caches)[:, -1])
        return torch.stack(outs, dim=1)

    with torch.no_grad():
        fused = run()
        full = model.lm_head(model.ln_f(_hidden(model, tokens)))
        monkeypatch.setattr(dcache.kernels, "dilution_attention_forward", _spec_forward)
        monkeypatch.setattr(dcache.kernels, "dilution_decode_step", _spec_decode)
        eager = run()
    assert torch.isfinite(fused).all()
    assert (fused - eager).abs().max().item() < 1e-4
    assert (fused - full[:, prefix - 1:]).abs().max().item() < 1e-4


@pytest.mark.gpu
@needs_gpu
def test_c5_training_step_full_size():
    """BASELINE config 5's training step: 12 layers, d_model 1024, 16 heads of
    64, SwiGLU 4x, RMSNorm, vocab 50304, no position encoding, bf16 weights
    N(0, 0.02), uniform token ids, B4 T16384: a finite loss near ln(vocab)
    for a random init and finite gradients in every parameter."""
    import math

    from dilution.lm import DilutionLM, LMConfig

    cfg = LMConfig()                                   # the C5 defaults
    assert (cfg.n_layers, cfg.d_model, cfg.n_heads, cfg.vocab_size) == (12, 1024, 16, 50304)
    torch.manual_seed(0)
    model = DilutionLM(cfg).to(device="cuda", dtype=torch.bfloat16).train()
    g = torch.Generator(device="cuda").manual_seed(13)
    idx = torch.randint(0, cfg.vocab_size, (4, 16385), device="cuda", generator=g)
    _, loss = model(idx[:, :-1], idx[:, 1:])
    loss.backward()
    torch.cuda.synchronize()
    assert torch.isfinite(loss)
    assert abs(loss.item() - math.log(cfg.vocab_size)) < 1.0, loss.item()
    for name, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), name


@pytest.mark.gpu
@needs_gpu
def test_c5_inference_leg_full_size():
    """BASELINE config 5's inference leg at size: the 12-layer d1024 bf16 LM
    prefills a 16384-token prompt at B8 (2048-token chunks), then takes 512
    greedy tokens eagerly (model.decode_step + the device argmax, as
    generate() runs it) and through GraphDecoder's replayed steps from a copy
    of the same caches.  The two token streams are equal, every logit is
    finite, and after the last step every layer's demand vector sums to the
    context length (each row's bids sum to one; model.py:198-257, the
    generate loop of model.py:473-509)."""
    from dilution.lm import DilutionLM, GraphDecoder, LMConfig, rows_argmax

    cfg = LMConfig()
    torch.manual_seed(0)
    model = DilutionLM(cfg).to(device="cuda", dtype=torch.bfloat16).eval()
    assert model.fused_decode_eligible(8) and model.graph_decode_eligible()
    g = torch.Generator(device="cuda").manual_seed(17)
    prompt, new = 16384, 512
    idx = torch.randint(0, cfg.vocab_size, (8, prompt), device="cuda", generator=g)
    with torch.no_grad():
        logits, caches_e = model.prefill(idx, capacity=prompt + new)
    assert torch.isfinite(logits.float()).all()
    caches_g = [{key: (val.clone() if torch.is_tensor(val) else val) for key, val in c.items()}
                for c in caches_e]
    first = rows_argmax(logits[:, -1, :])
    finite = torch.ones((), dtype=torch.bool, device="cuda")
    eager = [first]
    nxt = first
    with torch.no_grad():
        for _ in range(new - 1):
            step_logits = model.decode_step(nxt, caches_e)
            finite &= torch.isfinite(step_logits.float()).all()
            nxt = rows_argmax(step_logits[:, -1, :])
            eager.append(nxt)
    dec = GraphDecoder(model, caches_g, first)
    replayed = [first]
    for _ in range(new - 1):
        replayed.append(dec.step().clone())
        finite &= torch.isfinite(dec.logits.float()).all()
    torch.cuda.synchronize()
    assert bool(finite)
    eager, replayed = torch.cat(eager, dim=1), torch.cat(replayed, dim=1)
    assert eager.shape == (8, new)
    assert torch.equal(eager, replayed)
    length = prompt + new - 1
    for i, (ce, cg) in enumerate(zip(caches_e, caches_g)):
        assert ce["len"] == cg["len"] == length, i
        for c in (ce, cg):
            sums = c["committed"][..., :length].double().sum(-1)
            assert (sums - length).abs().max().item() < 1e-5 * length, (i, sums)
            assert torch.equal(c["committed"][..., length:], torch.zeros_like(c["committed"][..., length:]))
