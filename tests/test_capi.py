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
    assert lib.dil_abi_version() == 1
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


def test_argument_errors_before_any_launch(lib):
    # invalid head_dim / dtype / precision / shapes are rejected on the host
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 4, 48, 1, None, 0, None) == -1
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 4, 64, 7, None, 0, None) == -2
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 9, 64, 1, None, 0, None) == -4
    assert lib.dil_decode_step(None, None, None, None, None, 1, 8, 4, 64, 1, None, 0, None) == -3
    assert lib.dil_forward(None, None, None, 1, 8, 64, 1, 9, None, None, None, None, None, None,
                           None, None, 0, None) == -5
    assert lib.dil_prefill_chunk(None, None, None, 1, 8, 4, 10, 64, 1, 2, None, None, None, None,
                                 None, None, None, 0, None) == -4


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
