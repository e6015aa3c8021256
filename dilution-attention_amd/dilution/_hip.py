"""ctypes binding of libdilution_hip.so (C ABI: include/dilution_hip.h).

The library is built in-tree by ``dilution-attention_amd/csrc/build.py`` (or
``__graft_entry__.build()``) and loaded from this package directory, or from
the path in the environment variable ``DILUTION_HIP_LIB`` when that is set (a
different build of the same sources).  There is no fallback: if the library is
missing, every entry point raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.environ.get("DILUTION_HIP_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libdilution_hip.so")

_c_int64 = ctypes.c_int64
_c_int = ctypes.c_int
_vp = ctypes.c_void_p

# name -> (restype, argtypes); must match include/dilution_hip.h
SIGNATURES = {
    "dil_abi_version": (_c_int, []),
    "dil_status_string": (ctypes.c_char_p, [_c_int]),
    "dil_forward_key_pass": (_c_int, [_c_int64, _c_int64, _c_int, _c_int, _c_int]),
    "dil_forward_workspace_bytes": (_c_int64, [_c_int64, _c_int64, _c_int, _c_int, _c_int, _c_int]),
    "dil_forward": (_c_int, [_vp, _vp, _vp, _c_int64, _c_int64, _c_int, _c_int, _c_int,
                             _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _vp]),
    "dil_prefill_workspace_bytes": (_c_int64, [_c_int64, _c_int64, _c_int64, _c_int, _c_int, _c_int]),
    "dil_prefill_chunk": (_c_int, [_vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _c_int64, _c_int,
                                   _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _vp]),
    "dil_backward_workspace_bytes": (_c_int64, [_c_int64, _c_int64, _c_int, _c_int, _c_int]),
    "dil_backward": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64,
                              _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _c_int64,
                              _vp]),
    "dil_forward_variant": (_c_int, [_vp, _vp, _vp, _c_int64, _c_int64, _c_int, _c_int, _c_int,
                                     _c_int, _c_int, ctypes.c_float,
                                     _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _vp]),
    "dil_backward_variant": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int64,
                                      _c_int64, _c_int, _c_int, _c_int, _c_int, _c_int,
                                      _c_int, _c_int, ctypes.c_float,
                                      _vp, _vp, _vp, _vp, _c_int64, _vp]),
    "dil_decode_step_variant": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64,
                                         _c_int, _c_int, _c_int, _c_int, _c_int, ctypes.c_float,
                                         _vp, _c_int64, _vp]),
    "dil_decode_workspace_bytes": (_c_int64, [_c_int64, _c_int64, _c_int]),
    "dil_decode_step": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _c_int,
                                 _c_int, _c_int, _vp, _c_int64, _vp]),
    "dil_decode_step_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64,
                                         _c_int, _c_int, _c_int, _vp]),
    "dil_decode_step_dlen": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _vp, _c_int64,
                                      _c_int, _c_int, _c_int, _vp, _c_int64, _vp]),
    "dil_rows_linear": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _c_int, _c_int,
                                 ctypes.c_float, _vp]),
    "dil_rows_linear_qkv": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _c_int64, _vp,
                                     _c_int64, _c_int64, _c_int, ctypes.c_float, _vp]),
    "dil_rows_argmax": (_c_int, [_vp, _c_int64, _c_int64, _c_int64, _vp, _c_int, _vp]),
    "dil_timing_enable": (_c_int, [_c_int]),
    "dil_timing_reset": (_c_int, []),
    "dil_timing_count": (_c_int, []),
    "dil_timing_read": (_c_int, [_c_int, ctypes.c_char_p, _c_int, ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(_c_int64)]),
}

ABI_VERSION = 4

_lib = None
_load_error: str | None = None


def _load():
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        _load_error = (f"{LIB_PATH} is not built; run `python dilution-attention_amd/csrc/build.py` "
                       "(or __graft_entry__.build())")
        return None
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as exc:  # missing ROCm runtime, wrong arch, ...
        _load_error = f"cannot load {LIB_PATH}: {exc}"
        return None
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.dil_abi_version() != ABI_VERSION:
        _load_error = f"{LIB_PATH} has ABI {lib.dil_abi_version()}, expected {ABI_VERSION}"
        return None
    _lib = lib
    return lib


def available() -> bool:
    return _load() is not None


def lib():
    """The loaded library, or RuntimeError explaining why it is unavailable."""
    handle = _load()
    if handle is None:
        raise RuntimeError(f"dilution HIP kernels are not available: {_load_error}")
    return handle


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().dil_status_string(status).decode()
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


class kernel_timing:
    """Context manager: per-kernel launch counts and summed HIP-event time of
    every library launch inside the block.

        with kernel_timing() as kt:
            ...
        kt.result  # {name: (launches, total_ms)}
    """

    def __enter__(self):
        handle = lib()
        check(handle.dil_timing_reset(), "dil_timing_reset")
        handle.dil_timing_enable(1)
        self.result = {}
        return self

    def __exit__(self, *exc):
        handle = lib()
        handle.dil_timing_enable(0)
        count = handle.dil_timing_count()
        name = ctypes.create_string_buffer(64)
        ms = ctypes.c_double()
        launches = _c_int64()
        for i in range(count):
            check(handle.dil_timing_read(i, name, 64, ctypes.byref(ms), ctypes.byref(launches)),
                  "dil_timing_read")
            self.result[name.value.decode()] = (int(launches.value), float(ms.value))
        check(handle.dil_timing_reset(), "dil_timing_reset")
        return False
