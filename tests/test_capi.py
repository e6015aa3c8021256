"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/dilution_hip.h declares, and its host-side argument checks and size
queries behave (no device call is made)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dilution_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dil_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from dilution import _hip

    return _hip.lib()


def test_header_declares_entry_points():
    syms = _declared_symbols()
    for name in ("dil_forward", "dil_backward", "dil_decode_step", "dil_prefill_chunk"):
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    from dilution import _hip

    raw = ctypes.CDLL(_hip.LIB_PATH)
    for name in _declared_symbols():
        assert hasattr(raw, name), name
    assert set(_declared_symbols()) == set(_hip.SIGNATURES)


def test_abi_version_and_status_strings(lib):
    assert lib.dil_abi_version() == 4
    assert lib.dil_status_string(0) == b"success"
    for code in (-1, -2, -3, -4, -5):
        assert lib.dil_status_string(code) != b"unknown status"


def test_workspace_queries(lib):
    assert lib.dil_decode_workspace_bytes(256, 131072, 64) >= 256 * 131072 * 4
    small = lib.dil_forward_workspace_bytes(4, 512, 64, 1, 2, 0)
    assert small > 0
    # fp32 inputs with bf16 operands need converted copies
    assert lib.dil_forward_workspace_bytes(4, 512, 64, 0, 2, 0) > small
    assert lib.dil_forward_workspace_bytes(4, 512, 64, 1, 2, 1) > small
    assert lib.dil_prefill_workspace_bytes(4, 256, 1024, 64, 1, 2) > 0
    assert lib.dil_backward_workspace_bytes(4, 512, 64, 1, 2) >= 0


def test_key_pass_switch_sizes_the_workspace(lib, monkeypatch):
    """The key-parallel output pass adds its partials to the forward's
    workspace for the calls that can take it (bf16 operands, head_dim 64, a
    chunk starting at a multiple of 512 rows: the full causal forward and
    aligned prefill chunks); DILUTION_FORWARD_KEY_PASS=0 turns it off.
    dil_forward reads the switch once for its size check and its launch: a
    workspace sized with the pass off is an error (-3) with it on, before any
    launch.  The stand-in addresses are never dereferenced."""
    monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
    off = lib.dil_forward_workspace_bytes(2, 300, 64, 1, 2, 1)
    off_pre = lib.dil_prefill_workspace_bytes(2, 300, 0, 64, 1, 2)
    assert off_pre == lib.dil_forward_workspace_bytes(2, 300, 64, 1, 2, 0)
    monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS", raising=False)
    on = lib.dil_forward_workspace_bytes(2, 300, 64, 1, 2, 1)
    assert on > off
    assert lib.dil_prefill_workspace_bytes(2, 300, 0, 64, 1, 2) > off_pre
    # not eligible: fp32 operands, head_dim 32, a prefill chunk at an unaligned start
    for args in ((2, 300, 64, 1, 0, 1), (2, 300, 32, 1, 2, 1)):
        monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
        base = lib.dil_forward_workspace_bytes(*args)
        monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS", raising=False)
        assert lib.dil_forward_workspace_bytes(*args) == base, args
    for start, eligible in ((300, False), (512, True), (1536, True), (1000, False)):
        monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
        base = lib.dil_prefill_workspace_bytes(2, 300, start, 64, 1, 2)
        monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS", raising=False)
        assert (lib.dil_prefill_workspace_bytes(2, 300, start, 64, 1, 2) > base) == eligible, start
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(12)]
    assert lib.dil_forward(*fake[:3], 2, 300, 64, 1, 2, *fake[3:9], fake[9], fake[10], off, None) == -3
    # only the exact value "0" turns it off
    monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "00")
    assert lib.dil_forward_workspace_bytes(2, 300, 64, 1, 2, 1) == on


def test_key_pass_query_and_optional_carry(lib, monkeypatch):
    """dil_forward_key_pass says which calls take the key-parallel pass (bf16
    operands, head_dim 64, a chunk starting at a multiple of 512 rows); only
    those may pass carry = NULL.  A NULL carry on a three-pass call is an
    argument error (-4) before any launch (the stand-in addresses are never
    dereferenced).  The forward workspace holds the key pass's partials for
    at most 24 GiB of slices: past that, the call runs in slice batches and
    the workspace stops growing with the batch."""
    monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS", raising=False)
    assert lib.dil_forward_key_pass(300, 0, 64, 1, 2) == 1
    assert lib.dil_forward_key_pass(300, 0, 64, 0, 2) == 1      # fp32 inputs, bf16 operands
    assert lib.dil_forward_key_pass(2048, 1536, 64, 1, 2) == 1
    for args in ((300, 0, 64, 1, 0), (300, 0, 64, 1, 1), (300, 0, 32, 1, 2), (300, 0, 128, 1, 2),
                 (2048, 1000, 64, 1, 2), (300, 0, 48, 1, 2), (0, 0, 64, 1, 2), (300, -512, 64, 1, 2)):
        assert lib.dil_forward_key_pass(*args) == 0, args
    monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
    assert lib.dil_forward_key_pass(300, 0, 64, 1, 2) == 0
    monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS")

    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(12)]
    q, k, v, out, rmax, rden, ssum, tot, ws = fake[:9]
    big = 1 << 40
    # fp32 operands: the three-pass forward needs the checkpoints
    assert lib.dil_forward(q, k, v, 2, 300, 64, 1, 0, out, rmax, rden, ssum, None, tot, None, ws, big,
                           None) == -4
    # a prefill chunk at an unaligned start takes the three-pass forward too
    assert lib.dil_prefill_chunk(q, k, v, 2, 300, 100, 1000, 64, 1, 2, tot, out, rmax, rden, ssum, None, ws,
                                 big, None) == -4

    # partial room: one 131072-row slice needs ~2.2 GB, so 24 GiB hold 11;
    # past that the slices go in equal batches (12 -> 6 + 6, 100 -> 10 x 10)
    def partial_room(n):
        monkeypatch.setenv("DILUTION_FORWARD_KEY_PASS", "0")
        off = lib.dil_forward_workspace_bytes(n, 131072, 64, 1, 2, 0)
        monkeypatch.delenv("DILUTION_FORWARD_KEY_PASS")
        return lib.dil_forward_workspace_bytes(n, 131072, 64, 1, 2, 0) - off

    one = partial_room(1)
    assert 2.1e9 < one < 2.3e9
    assert partial_room(5) >= 5 * one - 1024
    assert 11 * one - 1024 <= partial_room(11) <= 24 * 2**30
    assert partial_room(12) == partial_room(6)
    assert partial_room(100) == partial_room(10)


def test_argument_errors_before_any_launch(lib):
    # invalid head_dim / dtype / precision / shapes are rejected on the host
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 4, 48, 1, 1, None, 0, None) == -1
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 4, 64, 7, 1, None, 0, None) == -2
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 4, 64, 1, 5, None, 0, None) == -2
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 9, 64, 1, 1, None, 0, None) == -4
    assert lib.dil_forward(None, None, None, 1, 8, 64, 1, 9, None, None, None, None, None, None,
                           None, None, 0, None) == -5
    assert lib.dil_prefill_chunk(None, None, None, 1, 8, 4, 10, 64, 1, 2, None, None, None, None,
                                 None, None, None, 0, None) == -4


def test_rows_linear_argument_errors_before_any_launch(lib):
    """dil_rows_linear: bf16 only, 1-8 rows, K a multiple of 256 up to 4096,
    and the buffers its mode reads; the stand-in addresses are never
    dereferenced (every call returns before launching)."""
    f = [ctypes.c_void_p(4096 * (i + 1)) for i in range(6)]
    x, w1, w2, g, res, out = f
    ok = (8, 64, 1024)
    assert lib.dil_rows_linear(x, w1, None, None, None, out, *ok, 0, 0, 0.0, None) == -2      # fp32
    assert lib.dil_rows_linear(x, w1, None, None, None, out, 9, 64, 1024, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, w1, None, None, None, out, 0, 64, 1024, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, w1, None, None, None, out, 8, 64, 1000, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, w1, None, None, None, out, 8, 64, 8192, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, w1, None, None, None, out, 8, 0, 1024, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, w1, None, None, None, out, *ok, 4, 1, 0.0, None) == -4     # mode
    assert lib.dil_rows_linear(None, w1, None, None, None, out, *ok, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, None, None, None, None, out, *ok, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, w1, None, None, None, None, *ok, 0, 1, 0.0, None) == -4
    assert lib.dil_rows_linear(x, w1, None, None, None, out, *ok, 1, 1, 0.0, None) == -4     # resid
    assert lib.dil_rows_linear(x, w1, None, None, None, out, *ok, 2, 1, 1e-5, None) == -4    # g
    assert lib.dil_rows_linear(x, w1, None, g, None, out, *ok, 3, 1, 1e-5, None) == -4       # w2
    assert lib.dil_rows_linear(x, w1, None, g, None, out, *ok, 2, 1, -1.0, None) == -4       # eps


def test_rows_linear_qkv_argument_errors_before_any_launch(lib):
    """dil_rows_linear_qkv: the rows / K / dtype rules of dil_rows_linear,
    every buffer required, and a host position inside the cache; the stand-in
    addresses are never dereferenced."""
    x, w, g, q, kc, vc = (ctypes.c_void_p(4096 * (i + 1)) for i in range(6))
    bufs = [x, w, g, q, kc, vc]

    def call(*, b=bufs, rows=8, heads=16, hd=64, cap=100, pdev=None, pos=5, k=1024, dt=1, eps=1e-5):
        return lib.dil_rows_linear_qkv(*b, rows, heads, hd, cap, pdev, pos, k, dt, eps, None)

    assert call(dt=0) == -2
    assert call(rows=9) == -4 and call(rows=0) == -4 and call(k=1000) == -4 and call(k=8192) == -4
    assert call(heads=0) == -4 and call(hd=0) == -4 and call(cap=0) == -4
    assert call(pos=100) == -4 and call(pos=-1) == -4              # host position outside the cache
    assert call(eps=-1.0) == -4
    for hole in range(6):
        assert call(b=[None if i == hole else p for i, p in enumerate(bufs)]) == -4, hole


def test_rows_argmax_argument_errors_before_any_launch(lib):
    lg, out = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    assert lib.dil_rows_argmax(lg, 8, 100, 100, out, 0, None) == -2          # fp32
    assert lib.dil_rows_argmax(None, 8, 100, 100, out, 1, None) == -4
    assert lib.dil_rows_argmax(lg, 8, 100, 100, None, 1, None) == -4
    assert lib.dil_rows_argmax(lg, 0, 100, 100, out, 1, None) == -4
    assert lib.dil_rows_argmax(lg, 8, 100, 0, out, 1, None) == -4
    assert lib.dil_rows_argmax(lg, 8, 100, 101, out, 1, None) == -4         # limit past the row


def test_null_pointers_are_argument_errors(lib):
    """A NULL where the header requires a buffer is a status (-4) returned
    before any launch, never a device fault.  The stand-in addresses below are
    never dereferenced: every call returns before launching."""
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(16)]
    big = 1 << 40
    # decode: each required pointer in turn
    for hole in range(5):
        ptrs = [None if i == hole else fake[i] for i in range(5)]
        assert lib.dil_decode_step(*ptrs, 1, 8, 4, 64, 1, 1, fake[5], big, None) == -4, hole
    assert lib.dil_decode_step(*fake[:5], 1, 8, 4, 64, 1, 1, None, big, None) == -4
    # with every pointer set, the workspace size is the next check
    assert lib.dil_decode_step(*fake[:5], 1, 8, 4, 64, 1, 1, fake[5], 0, None) == -3
    # device-length decode: the five buffers and the length pointer
    for hole in range(6):
        ptrs = [None if i == hole else fake[i] for i in range(6)]
        assert lib.dil_decode_step_dlen(*ptrs[:5], 1, 8, ptrs[5], 4, 64, 1, 1, fake[6], big,
                                        None) == -4, hole
    assert lib.dil_decode_step_dlen(*fake[:5], 1, 8, fake[5], 9, 64, 1, 1, fake[6], big, None) == -4
    assert lib.dil_decode_step_dlen(*fake[:5], 1, 8, fake[5], 8, 64, 1, 1, fake[6], 0, None) == -3
    # forward: pk may be NULL, and carry on a key-pass call (bf16 operands at
    # head_dim 64), so its hole is tested on an "ieee" (three-pass) call
    fwd_ptrs = fake[:3]
    outs = fake[3:9]                              # out, rmax, rden, ssum, carry, committed_total
    for hole in range(6):
        o = [None if i == hole else outs[i] for i in range(6)]
        prec = 0 if hole == 4 else 2
        assert lib.dil_forward(*fwd_ptrs, 1, 8, 64, 1, prec, *o, None, fake[9], big, None) == -4, hole
    assert lib.dil_forward(None, *fake[1:3], 1, 8, 64, 1, 2, *outs, None, fake[9], big, None) == -4
    assert lib.dil_forward(*fwd_ptrs, 1, 8, 64, 1, 2, *outs, None, fake[9], 0, None) == -3
    # backward: pk is required there
    ins = fake[:10]                               # q k v dout out rmax rden ssum carry pk
    for hole in range(10):
        a = [None if i == hole else ins[i] for i in range(10)]
        assert lib.dil_backward(*a, 1, 8, 64, 1, 1, 1, 2, *fake[10:13], fake[13], big, None) == -4, hole
    for hole in range(3):
        g = [None if i == hole else fake[10 + i] for i in range(3)]
        assert lib.dil_backward(*ins, 1, 8, 64, 1, 1, 1, 2, *g, fake[13], big, None) == -4, hole
    # prefill
    pre = fake[:3]
    rest = fake[3:9]                              # committed out rmax rden ssum carry
    for hole in range(6):
        r = [None if i == hole else rest[i] for i in range(6)]
        assert lib.dil_prefill_chunk(*pre, 1, 8, 4, 16, 64, 1, 2, *r, fake[9], big, None) == -4, hole


def test_python_layer_raises_without_gpu_tensors():
    import torch
    from dilution import kernels

    x = torch.zeros(1, 1, 4, 64)
    with pytest.raises(RuntimeError):
        kernels.dilution_attention_forward(x, x, x)
    with pytest.raises(ValueError):
        kernels.dilution_attention_forward(x, x, x, dot_precision="fp16")
    with pytest.raises(ValueError):
        kernels.dilution_attention_forward(x, torch.zeros(1, 1, 5, 64), x)      # k of another length
    with pytest.raises(ValueError):
        kernels.dilution_attention_forward(x, x, torch.zeros(1, 1, 4, 32))      # v of another width


def test_cache_shape_errors_before_any_launch():
    """Decode / prefill reject caches that do not match the queries, a demand
    of the wrong shape or dtype, and non-contiguous buffers (kernels.py:1003-1021)
    with ValueError, before touching the device."""
    import torch
    from dilution import kernels

    b, h, cap, d = 2, 3, 16, 64
    q1 = torch.zeros(b, h, 1, d)
    kc = torch.zeros(b, h, cap, d)
    com = torch.zeros(b, h, cap)
    cases = [
        (q1, kc, torch.zeros(b, h, cap + 1, d), com),                    # V shape differs
        (torch.zeros(b, h + 1, 1, d), kc, kc, com),                       # heads differ
        (q1, kc, kc, torch.zeros(b, h, cap - 1)),                         # demand too short
        (q1, kc, kc, com.double()),                                       # demand not fp32
        (q1, kc.transpose(1, 2).contiguous().transpose(1, 2), kc, com),  # K not contiguous
    ]
    for q, k, v, c in cases:
        with pytest.raises(ValueError):
            kernels.dilution_decode_step(q, k, v, c, 4)
    with pytest.raises(ValueError):
        kernels.dilution_decode_step(q1, kc, kc, com, cap + 1)             # past capacity
    with pytest.raises(ValueError):
        kernels.dilution_prefill_chunk(torch.zeros(b, h, 8, d), kc, kc, com, 12)   # rows past capacity
    with pytest.raises(RuntimeError):
        kernels.dilution_decode_step(q1, kc, kc, com, 4)                    # valid, but no GPU tensors


def test_tensors_on_two_devices_are_rejected():
    """Every launch goes to the inputs' device and that device's current
    stream; inputs spread over two devices are a ValueError before any launch."""
    import types

    import torch
    from dilution import kernels

    on = lambda i: types.SimpleNamespace(is_cuda=True, device=torch.device("cuda", i))  # noqa: E731
    kernels._check_device(on(0), on(0), on(0))
    with pytest.raises(ValueError):
        kernels._check_device(on(0), on(1), on(0))
    with pytest.raises(RuntimeError):
        kernels._check_device(on(0), torch.zeros(1))


def test_head_dim_support_and_rejections_before_any_launch():
    """The reference's model routes every power-of-two head_dim >= 16 to its
    kernels (model.py:158-165).  The gfx950 kernels take 16-128 in every dot
    precision and 256 with bf16 operands (the decode step at 256 with any
    cache dtype); head_dim_supported(d, dot_precision) is the predicate a
    caller narrows its routing with.  Other widths, and 256 with "ieee" or
    "tf32", raise ValueError on the host (the reference model then keeps its
    eager path for them, model.py:182-257); the C ABI returns -1 before any
    launch (the stand-in addresses are never dereferenced)."""
    import ctypes

    import torch
    from dilution import _hip, kernels, kernels_bid

    assert kernels.SUPPORTED_HEAD_DIMS == (16, 32, 64, 128, 256)
    for prec in ("bf16", "tf32", "ieee"):
        assert all(kernels.head_dim_supported(d, prec) for d in (16, 32, 64, 128))
        assert not any(kernels.head_dim_supported(d, prec) for d in (8, 48, 512))
        assert kernels.head_dim_supported(256, prec) == (prec == "bf16")
    assert kernels.head_dim_supported(256)
    assert not kernels_bid.head_dim_supported(256)
    for d in (512, 8):
        x = torch.zeros(1, 2, 4, d)
        with pytest.raises(ValueError, match="head_dim"):
            kernels.dilution_attention_forward(x, x, x, dot_precision="bf16")
        with pytest.raises(ValueError, match="head_dim"):
            kernels.dilution_attention(x, x, x)
        kc, com = torch.zeros(1, 2, 8, d), torch.zeros(1, 2, 8)
        with pytest.raises(ValueError, match="head_dim"):
            kernels.dilution_decode_step(torch.zeros(1, 2, 1, d), kc, kc, com, 4)
        with pytest.raises(ValueError, match="head_dim"):
            kernels.dilution_prefill_chunk(x, kc, kc, com, 0)
    x = torch.zeros(1, 2, 4, 256)
    kc, com = torch.zeros(1, 2, 8, 256), torch.zeros(1, 2, 8)
    for prec in ("ieee", "tf32"):
        with pytest.raises(ValueError, match="head_dim 256"):
            kernels.dilution_attention_forward(x, x, x, dot_precision=prec)
        with pytest.raises(ValueError, match="head_dim 256"):
            kernels.dilution_attention(x, x, x, dot_precision=prec)
        with pytest.raises(ValueError, match="head_dim 256"):
            kernels.dilution_prefill_chunk(x, kc, kc, com, 0, dot_precision=prec)
    with pytest.raises(ValueError, match="head_dim"):
        kernels_bid.dilution_attention_forward(x, x, x, bid="relu")

    lib = _hip.lib()
    f = [ctypes.c_void_p(4096 * (i + 1)) for i in range(14)]
    big = 1 << 40
    for prec, want in ((0, -1), (1, -1)):
        assert lib.dil_forward(*f[:3], 1, 8, 256, 1, prec, *f[3:9], None, f[9], big, None) == want
        assert lib.dil_prefill_chunk(*f[:3], 1, 8, 0, 16, 256, 1, prec, *f[3:9], f[9], big, None) == want
        assert lib.dil_backward(*f[:10], 1, 8, 256, 1, 1, 1, prec, *f[10:13], f[13], big, None) == want
    assert lib.dil_decode_step(*f[:5], 1, 8, 4, 512, 1, 1, f[5], big, None) == -1
    # a bid / share variant at 256 (bf16 operands): its instantiations stop at 128
    assert lib.dil_forward_variant(*f[:3], 1, 8, 256, 1, 2, 1, 1, 1.0, *f[3:9], None, f[9], big,
                                   None) == -1
    assert lib.dil_decode_step_noalloc(*f[:5], 1, 8, 4, 512, 1, 1, None) == -1


def test_integration_loader_re_exports_the_module(monkeypatch):
    """The Option-A loader that INTEGRATION.md gives a maintainer (the body of
    the reference's src/dilution/kernels.py) runs as written: with
    DILUTION_AMD_ROOT pointing at this package it re-exports the operator's
    functions, the routing predicate and the test gate, and loads nothing
    from the reference."""
    import sys

    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    loader = next(b for b in blocks if "DILUTION_AMD_ROOT" in b)
    monkeypatch.setenv("DILUTION_AMD_ROOT", os.path.join(ROOT, "dilution-attention_amd"))
    ns = {"__name__": "reference_kernels_stand_in"}
    try:
        exec(compile(loader, "INTEGRATION.md", "exec"), ns)
        from dilution import kernels

        for name in ("dilution_attention_reference", "dilution_attention_forward", "dilution_attention",
                     "dilution_decode_step", "dilution_prefill_chunk", "head_dim_supported",
                     "_DilutionAttentionFn", "KEY_FORWARD_MIN_SEQ"):
            assert getattr(ns[name], "__name__", name) == getattr(getattr(kernels, name), "__name__", name), name
        assert ns["HAS_TRITON"] == kernels.HAS_HIP
        assert ns["head_dim_supported"](256, "bf16") and not ns["head_dim_supported"](256, "tf32")
    finally:
        for mod in [m for m in sys.modules if m == "dilution_amd" or m.startswith("dilution_amd.")]:
            del sys.modules[mod]
