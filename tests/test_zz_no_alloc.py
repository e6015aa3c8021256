"""The allocation-free decode entry point (dil_decode_step_noalloc) against
dil_decode_step, both called through the C ABI: bit-identical outputs and
demand on two calls in a row, the second smaller than the first (the shared
scratch keeps the first call's contents, which must not leak into the
second), and a too-large call rejected before any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from gpu_helpers import needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]

DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _inputs(batch, heads, cap, length, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q1 = torch.randn(batch, heads, 1, d, generator=g).to(dtype)
    kc = torch.randn(batch, heads, cap, d, generator=g).to(dtype)
    vc = torch.randn(batch, heads, cap, d, generator=g).to(dtype)
    com = torch.rand(batch, heads, cap, generator=g) * 3.0
    com[..., length - 1:] = 0.0
    return [t.cuda() for t in (q1, kc, vc, com)]


def _both(lib, q1, kc, vc, com, length):
    """(out, demand) of dil_decode_step (torch workspace) and of the
    allocation-free entry point, each on its own copy of the demand."""
    batch, heads, cap, d = kc.shape
    n = batch * heads
    dt = DTYPES[kc.dtype]
    qdt = DTYPES[q1.dtype]
    stream = torch.cuda.current_stream().cuda_stream
    com_a, com_b = com.clone(), com.clone()
    out_a = torch.empty(n, d, device="cuda", dtype=q1.dtype)
    out_b = torch.full((n, d), float("nan"), device="cuda", dtype=q1.dtype)
    ws = torch.empty(lib.dil_decode_workspace_bytes(n, length, d), dtype=torch.uint8, device="cuda")
    st = lib.dil_decode_step(q1.data_ptr(), kc.data_ptr(), vc.data_ptr(), com_a.data_ptr(),
                             out_a.data_ptr(), n, cap, length, d, dt, qdt, ws.data_ptr(), ws.numel(),
                             stream)
    assert st == 0, st
    st = lib.dil_decode_step_noalloc(q1.data_ptr(), kc.data_ptr(), vc.data_ptr(), com_b.data_ptr(),
                                     out_b.data_ptr(), n, cap, length, d, dt, qdt, stream)
    assert st == 0, st
    torch.cuda.synchronize()
    return (out_a, com_a), (out_b, com_b)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 64), (torch.float32, 128)])
def test_noalloc_decode_matches_decode_step(dtype, d):
    from dilution import _hip

    lib = _hip.lib()
    # a larger call, then a smaller one (fewer slices, shorter context)
    for (batch, heads, cap, length), seed in (((4, 8, 9000, 8500), 1), ((2, 3, 1300, 777), 2)):
        q1, kc, vc, com = _inputs(batch, heads, cap, length, d, dtype, seed)
        (out_a, com_a), (out_b, com_b) = _both(lib, q1, kc, vc, com, length)
        assert torch.equal(out_a, out_b), (batch, heads, length)
        assert torch.equal(com_a, com_b), (batch, heads, length)
        assert torch.equal(com_b[..., length:], com[..., length:])


def test_noalloc_decode_rejects_calls_beyond_its_scratch():
    from dilution import _hip

    lib = _hip.lib()
    n, length, d = 256, 131072, 64
    assert lib.dil_decode_workspace_bytes(n, length, d) > 64 << 20
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(5)]     # never dereferenced
    assert lib.dil_decode_step_noalloc(*fake, n, length, length, d, 1, 1, None) == -7
    assert b"scratch" in lib.dil_status_string(-7)
    # still usable afterwards, on a call that fits
    q1, kc, vc, com = _inputs(1, 2, 600, 513, 64, torch.bfloat16, 3)
    (out_a, com_a), (out_b, com_b) = _both(lib, q1, kc, vc, com, 513)
    assert torch.equal(out_a, out_b) and torch.equal(com_a, com_b)
