"""ctypes binding of ``libminiep_amd.so`` (the C ABI of include/miniep_amd.h).

The library is built in-tree by ``mini-ep_amd/build.py``.  Loading it does not
touch the GPU; every compute entry point needs ROCm device memory.  There is no
CPU fallback: if the library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libminiep_amd.so")
HEADER_PATH = Path(__file__).resolve().parents[2] / "include" / "miniep_amd.h"

DTYPE_F32 = 0
DTYPE_BF16 = 1

ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_WORKSPACE = -3
ERR_EXPERT_RANGE = -4
ERR_NOT_RESIDENT = -5
ERR_HIP = -6

DISPATCH_STATUS_RANGE = 1
DISPATCH_STATUS_NOT_RESIDENT = 2
DISPATCH_STATUS_REPLICAS = 4
DISPATCH_STATUS_BARRIER = 8

# sites of the give-up test hook (mep_test_force_giveup)
GIVEUP_NONE = 0
GIVEUP_DISPATCH = 1
GIVEUP_ROWS = 2
GIVEUP_CHUNK = 3
GIVEUP_COMBINE = 4
GIVEUP_ROUTED = 5


class MepError(RuntimeError):
    """A C-ABI call returned a nonzero status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed ({code}): {message}")
        self.fn, self.code, self.message = fn, code, message


class NotResidentError(MepError, AssertionError):
    """An entry was routed to this rank for an expert it does not hold
    (the condition miniep/ep.py:230 asserts on)."""


class ExpertRangeError(MepError, IndexError):
    """A routed expert id lies outside [0, n_experts)."""


_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_size = ctypes.c_size_t

_SIGNATURES = {
    "mep_last_error": (ctypes.c_char_p, []),
    "mep_abi_version": (ctypes.c_int, []),
    "mep_router_topk": (ctypes.c_int, [_c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32,
                                       _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "mep_topk_softmax": (ctypes.c_int, [_c_void_p, _i64, _i32, _i32, _i32, _c_void_p,
                                        _c_void_p, _c_void_p]),
    "mep_dispatch_workspace_size": (_size, [_i64, _i32, _i32, _i32, ctypes.POINTER(_i64)]),
    "mep_dispatch": (ctypes.c_int, [_c_void_p, _c_void_p, _i64, _i32, _i32,
                                    _c_void_p, _c_void_p, _i32, _i32, _c_void_p,
                                    ctypes.POINTER(_i64), _i32, _i32, _c_void_p, _i32,
                                    _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                    _c_void_p, _c_void_p, _size, _c_void_p]),
    "mep_dispatch_check": (ctypes.c_int, [_c_void_p, _c_void_p]),
    "mep_route_dispatch_workspace_size": (_size, [_i64, _i32]),
    "mep_route_dispatch": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32,
                                          _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                          _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "mep_dispatch_noalloc": (ctypes.c_int, [_c_void_p, _c_void_p, _i64, _i32, _i32,
                                            _c_void_p, _c_void_p, _i32, _i32, _c_void_p,
                                            ctypes.POINTER(_i64), _i32, _i32, _c_void_p, _i32,
                                            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                            _c_void_p, _c_void_p, _c_void_p]),
    "mep_experts_workspace_size": (_size, [_i64, _i32, _i32]),
    "mep_experts_queue_ints": (_size, [_i64, _i32]),
    "mep_experts_check": (ctypes.c_int, [_c_void_p, _c_void_p]),
    "mep_grouped_swiglu": (ctypes.c_int, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32,
                                          _i64, _c_void_p, _c_void_p, _i32, _i32, _i32,
                                          _c_void_p, _c_void_p, _size, _c_void_p, _size, _c_void_p]),
    "mep_grouped_swiglu_slots": (ctypes.c_int, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32,
                                                _i64, _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32,
                                                _c_void_p, _c_void_p, _size, _c_void_p, _size, _c_void_p]),
    "mep_grouped_swiglu_combine": (ctypes.c_int, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _c_void_p,
                                                  _c_void_p, _c_void_p, _i32, _i64, _c_void_p, _c_void_p, _i32,
                                                  _i32, _i32, _c_void_p, _c_void_p, _size, _c_void_p, _size,
                                                  _c_void_p, _c_void_p]),
    "mep_copy_experts": (ctypes.c_int, [_c_void_p, _c_void_p, _i32, _c_void_p, _c_void_p, _i32,
                                        ctypes.POINTER(_i32), ctypes.POINTER(_i32), _i32, _i32, _i32, _i32,
                                        _c_void_p]),
    "mep_swiglu_gate_up": (ctypes.c_int, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32, _i64,
                                          _c_void_p, _i32, _i32, _i32, _c_void_p, _size, _c_void_p, _size,
                                          _c_void_p]),
    "mep_swiglu_down": (ctypes.c_int, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32, _i64,
                                       _c_void_p, _i32, _i32, _i32, _c_void_p, _c_void_p, _size, _c_void_p]),
    "mep_combine": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
                                   _i32, _i32, _c_void_p, _c_void_p]),
    "mep_gather_rows": (ctypes.c_int, [_c_void_p, _i64, _i32, _c_void_p, _i64, _i32, _i32, _c_void_p,
                                       _c_void_p, _c_void_p, _c_void_p]),
    "mep_combine_rows": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
                                        _i32, _i32, _c_void_p, _c_void_p]),
    "mep_test_force_giveup": (ctypes.c_int, [_i32, _i32]),
    "mep_moe_layer_queue_ints": (_size, [_i64, _i32, _i32]),
    "mep_moe_layer": (ctypes.c_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32, _c_void_p,
                                     _c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                     _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p, _size,
                                     _c_void_p, _size, _c_void_p, _c_void_p]),
}

_LIB = None


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python mini-ep_amd/build.py` "
                "(the MoE hot path has no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def header_functions() -> list[str]:
    """Names of the functions declared in include/miniep_amd.h."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+(mep_[a-z_0-9]+)\(", text, re.M)))


def last_error() -> str:
    return lib().mep_last_error().decode(errors="replace")


def check(rc: int, fn: str) -> None:
    """Raise the MepError subclass matching a nonzero status."""
    if rc == 0:
        return
    msg = last_error()
    if rc == ERR_NOT_RESIDENT:
        raise NotResidentError(fn, rc, msg)
    if rc == ERR_EXPERT_RANGE:
        raise ExpertRangeError(fn, rc, msg)
    raise MepError(fn, rc, msg)
