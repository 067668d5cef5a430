"""ctypes binding of ``libdsv4moe.so`` (the C ABI of ``include/dsv4moe.h``).

The library is required: every device entry point of this package calls
through it, and there is no fallback implementation.  A missing library raises
``RuntimeError`` at the first call.  ``DSV4MOE_LIBRARY`` may name another build
of the same library (for example one built for a different target).
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("DSV4MOE_LIBRARY") or Path(__file__).resolve().with_name("libdsv4moe.so"))

DSV4MOE_OK = 0
DSV4MOE_EINVAL = 1
DSV4MOE_EHIP = 2

SCORE_FUNCS = {"sigmoid": 0, "softmax": 1, "sqrtsoftplus": 2}
PAIR_PLAIN = 0
PAIR_GATED = 1
WEIGHT_TILED = 0
WEIGHT_ROWMAJOR = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# the C ABI revision these signatures describe (dsv4moe_abi_version)
ABI_VERSION = 3

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "dsv4moe_last_error": (ctypes.c_char_p, []),
    "dsv4moe_abi_version": (_i32, []),
    "dsv4moe_profile_begin": (ctypes.c_int, [_i32]),
    "dsv4moe_profile_begin_stamps": (ctypes.c_int, [_i32, ctypes.c_uint32]),
    "dsv4moe_profile_end": (ctypes.c_int, [ctypes.POINTER(ctypes.c_float), _i32, ctypes.POINTER(_i32)]),
    "dsv4moe_block_size_m": (_i32, [_i64, _i32, _i32, _i32]),
    "dsv4moe_max_padded_tokens": (_i64, [_i64, _i32, _i32]),
    "dsv4moe_route_topk": (
        ctypes.c_int,
        [_p, _p, _i64, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p, _p],
    ),
    "dsv4moe_route_hash": (ctypes.c_int, [_p, _p, _i64, _p, _i64, _i32, _i32, _f32, _p, _p, _p, _p]),
    "dsv4moe_gate_logits": (ctypes.c_int, [_p, _p, _i64, _i32, _i32, _p, _p]),
    "dsv4moe_align": (ctypes.c_int, [_p, _i64, _i32, _i32, _i32, _p, _i64, _p, _i64, _p, _p]),
    "dsv4moe_align_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "dsv4moe_act_quant_block_fp8": (ctypes.c_int, [_p, _i32, _i64, _i64, _p, _p, _p]),
    "dsv4moe_block_fp8_split_k": (_i32, [_i64, _i64, _i64]),
    "dsv4moe_block_fp8_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "dsv4moe_block_fp8_gemm": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _p, _i32, _p, _i32, _p, _sz, _p, _p]),
    "dsv4moe_align_ws": (ctypes.c_int, [_p, _i64, _i32, _i32, _i32, _p, _i64, _p, _i64, _p, _p, _sz, _p]),
    "dsv4moe_pack_int4_g128": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i32, _p, _p, _p]),
    "dsv4moe_experts_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "dsv4moe_pack_int4_ratios": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _p]),
    "dsv4moe_experts_w4a16": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _i64, _p, _p, _i32,
         _f32, _p, _p, _sz, _p],
    ),
    "dsv4moe_layer_w4a16": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p, _p, _i32, _f32,
         _i32, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _sz, _p],
    ),
    "dsv4moe_layer_w4a16_noalloc": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p, _p, _i32, _f32,
         _i32, _p, _p, _p, _p, _i64, _p, _p, _p, _p],
    ),
    "dsv4moe_pack_mxfp4_g32": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i32, _p, _p, _p]),
    "dsv4moe_pack_mxfp4_g32_w4a8": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i32, _p, _p, _p]),
    "dsv4moe_experts_w4a8_mxfp4": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _i32, _p, _p, _i64, _p, _p, _i32,
         _f32, _p, _p, _sz, _p],
    ),
    "dsv4moe_layer_mxfp4": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _i32, _f32,
         _i32, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _sz, _p],
    ),
    "dsv4moe_layer_w4a8": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _i32, _f32,
         _i32, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _sz, _p],
    ),
    "dsv4moe_layer_w4a8_mxfp4": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _i32, _f32,
         _i32, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _sz, _p],
    ),
    "dsv4moe_experts_mxfp4": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _i32, _p, _p, _i64, _p, _p, _i32,
         _f32, _p, _p, _sz, _p],
    ),
    "dsv4moe_pack_int8": (ctypes.c_int, [_p, _i64, _i64, _p, _p]),
    "dsv4moe_decode_e8m0": (ctypes.c_int, [_p, _i64, _p, _p]),
    "dsv4moe_dequant_mxfp4": (ctypes.c_int, [_p, _p, _i64, _i64, _p, _p]),
    "dsv4moe_dequant_fp8_block": (ctypes.c_int, [_p, _i32, _p, _i64, _i64, _p, _p]),
    "dsv4moe_experts_w4a8_workspace_bytes": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "dsv4moe_experts_w4a8": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _i32, _p, _p, _i64, _p, _p, _i32,
         _f32, _p, _p, _sz, _p],
    ),
    "dsv4moe_act_quant_fp8": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _p]),
    "dsv4moe_w8a16_split_k": (_i32, [_i64, _i64, _i64]),
    "dsv4moe_w8a16_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "dsv4moe_w8a16_linear": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _i32, _p, _i32, _p, _sz, _p, _p]),
    "dsv4moe_w8a16_fp8_linear": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _i32, _p, _i32, _p, _sz, _p, _p]),
    "dsv4moe_shared_fp8_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "dsv4moe_shared_fp8_add": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p, _p, _p, ctypes.c_float, _p, _p, _sz,
                                              _p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class Dsv4MoEError(RuntimeError):
    """A HIP-side failure reported by the library (status DSV4MOE_EHIP)."""


def load() -> ctypes.CDLL:
    """Load and declare the library (once)."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built (expected at {LIB_PATH}); "
                    "run __graft_entry__.build() first"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.dsv4moe_abi_version.restype = _i32
            found = int(lib.dsv4moe_abi_version())
            if found != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has C ABI {found}, this binding needs {ABI_VERSION}: rebuild it")
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def is_loaded() -> bool:
    return _lib is not None


def last_error() -> str:
    msg = load().dsv4moe_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point and raise on failure.

    DSV4MOE_EINVAL -> ValueError (contract violation, nothing launched);
    DSV4MOE_EHIP -> Dsv4MoEError.
    """

    rc = getattr(load(), name)(*args)
    if rc == DSV4MOE_OK:
        return
    msg = last_error()
    if rc == DSV4MOE_EINVAL:
        raise ValueError(msg or f"{name}: invalid argument")
    raise Dsv4MoEError(msg or f"{name}: HIP error (status {rc})")


def ptr(tensor) -> int | None:
    """Device address of a tensor (None for None)."""

    return None if tensor is None else int(tensor.data_ptr())


def current_stream(device) -> int:
    import torch

    return int(torch.cuda.current_stream(device).cuda_stream)
