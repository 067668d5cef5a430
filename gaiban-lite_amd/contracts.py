"""Argument contracts of the host interface, checked before any launch.

A drop-in must fail the way the code it replaces fails: callers of
``runtime/dsv4_direct`` catch ``TypeError`` for an argument of the wrong kind
(not a tensor, wrong element type), ``ValueError`` for a wrong value (shape,
range, device, layout, aliasing, non-finite numbers) and ``RuntimeError`` for
lifecycle violations.  This module states each requirement once, as a small
set of composable checks, so every public entry of the package raises the
same exception class as the reference for the same violation; the wording of
the messages is this package's own.

Host reads of device data (``.item()``, ``.tolist()``) appear only in the
checks that need values (route tables, token ids, reserved scale bytes) and
are documented as synchronising; everything else looks at metadata only.
"""

from __future__ import annotations

import math
from collections.abc import Iterable, Mapping
from typing import Any

import torch

_DTYPE_SETS = (tuple, list, set, frozenset)


def _dtypes(dtype) -> tuple[torch.dtype, ...]:
    return tuple(dtype) if isinstance(dtype, _DTYPE_SETS) else (dtype,)


def _names(dtypes: tuple[torch.dtype, ...]) -> str:
    return " or ".join(str(d).replace("torch.", "") for d in dtypes)


def tensor(name: str, value: Any, *, dtype=None, shape=None, ndim: int | None = None, device=None,
           contiguous: bool = False, no_grad: bool = False, nonempty: bool = False,
           dtype_error: type[Exception] = TypeError, shape_error: type[Exception] = ValueError) -> torch.Tensor:
    """``value`` as a tensor meeting every given requirement, checked in the
    order kind, shape, element type, device, layout, autograd (the first
    violation decides the exception).

    Not a tensor: TypeError.  Shape / rank / emptiness: ``shape_error``.
    Element type outside ``dtype`` (one dtype or a collection):
    ``dtype_error``.  Device, layout and autograd: ValueError.
    """

    if not isinstance(value, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor, got {type(value).__name__}")
    if ndim is not None and value.ndim != ndim:
        raise shape_error(f"{name}: rank {value.ndim}, expected {ndim}")
    if shape is not None and tuple(value.shape) != tuple(shape):
        raise shape_error(f"{name}: shape {tuple(value.shape)}, expected {tuple(shape)}")
    if nonempty and value.numel() == 0:
        raise shape_error(f"{name}: must not be empty")
    if dtype is not None:
        allowed = _dtypes(dtype)
        if value.dtype not in allowed:
            raise dtype_error(f"{name}: element type {value.dtype} is not {_names(allowed)}")
    if device is not None and value.device != torch.device(device):
        raise ValueError(f"{name}: on {value.device}, expected {torch.device(device)}")
    if contiguous and not value.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if no_grad and value.requires_grad:
        raise ValueError(f"{name}: must not require gradients")
    return value


def positive_int(name: str, value: Any) -> int:
    """A positive Python int (bool excluded): ValueError otherwise."""

    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"{name}: expected a positive integer, got {value!r}")
    return value


def finite_positive(name: str, value: Any) -> float:
    """A finite, strictly positive real number: ValueError otherwise."""

    try:
        v = float(value)
    except (TypeError, ValueError):
        raise ValueError(f"{name}: expected a finite positive number, got {value!r}") from None
    if not math.isfinite(v) or v <= 0:
        raise ValueError(f"{name}: expected a finite positive number, got {value!r}")
    return v


def boolean(name: str, value: Any) -> bool:
    if not isinstance(value, bool):
        raise TypeError(f"{name}: expected bool, got {type(value).__name__}")
    return value


def same_device(name: str, tensors: Iterable[torch.Tensor]) -> torch.device:
    """The one device all ``tensors`` live on: ValueError when they differ."""

    devices = {t.device for t in tensors}
    if len(devices) != 1:
        raise ValueError(f"{name}: tensors span several devices {sorted(map(str, devices))}")
    return devices.pop()


def byte_spans_disjoint(tensors: Mapping[str, torch.Tensor], *, what: str = "tensors") -> torch.device:
    """Named contiguous tensors on one device whose byte ranges do not
    overlap (empty tensors occupy no bytes).  Returns the device."""

    if not isinstance(tensors, Mapping) or not tensors:
        raise ValueError(f"{what}: expected a non-empty mapping of named tensors")
    spans: list[tuple[int, int, str]] = []
    for name, t in tensors.items():
        if not isinstance(name, str) or not name:
            raise ValueError(f"{what}: tensor names must be non-empty strings")
        tensor(name, t, contiguous=True)
    device = same_device(what, tensors.values())
    for name, t in tensors.items():
        if t.numel():
            lo = int(t.data_ptr())
            spans.append((lo, lo + t.numel() * t.element_size(), name))
    spans.sort()
    for (lo_a, hi_a, a), (lo_b, _, b) in zip(spans, spans[1:]):
        if lo_b < hi_a:
            raise ValueError(f"{what}: {a} and {b} share memory")
    return device


def distinct_storages(tensors: Mapping[str, torch.Tensor], *, what: str) -> None:
    """No two tensors share an allocation: ValueError otherwise."""

    seen: dict[int, str] = {}
    for name, t in tensors.items():
        base = int(t.untyped_storage().data_ptr())
        if base in seen:
            raise ValueError(f"{what}: {seen[base]} and {name} share storage")
        seen[base] = name


def owns_whole_storage(name: str, t: torch.Tensor) -> None:
    """``t`` is its allocation from byte 0 to the end (not a view into a
    larger buffer): ValueError otherwise."""

    storage = t.untyped_storage()
    if t.storage_offset() != 0 or storage.nbytes() != t.numel() * t.element_size():
        raise ValueError(f"{name}: must own its complete storage, not view part of another")


def e8m0_codes(name: str, scale: torch.Tensor) -> torch.Tensor:
    """E8M0 scale bytes (``float8_e8m0fnu`` or ``uint8``) as uint8; TypeError
    for any other element type."""

    if scale.dtype == torch.float8_e8m0fnu:
        return scale.view(torch.uint8)
    if scale.dtype != torch.uint8:
        raise TypeError(f"{name}: E8M0 scales must be float8_e8m0fnu or uint8 bytes, got {scale.dtype}")
    return scale


def no_reserved_e8m0(name: str, scale: torch.Tensor) -> None:
    """Rejects the reserved E8M0 byte 0xFF (the reference decodes it as NaN,
    ``weight_only_linear.py:488-513``).  Reads the device: load time only."""

    if bool((e8m0_codes(name, scale) == 0xFF).any().item()):
        raise ValueError(f"{name}: contains the reserved E8M0 byte 255 (0xFF)")


def expert_table(name: str, ids: torch.Tensor, *, experts: int, unique_rows: bool = True) -> None:
    """Every id in ``[0, experts)`` and, with ``unique_rows``, no id twice in a
    row (ValueError).  Reads the device."""

    if ids.numel() == 0:
        return
    lo, hi = torch.stack(tuple(torch.aminmax(ids))).tolist()
    if lo < 0 or hi >= experts:
        raise ValueError(f"{name}: expert ids span [{lo}, {hi}], outside [0, {experts})")
    if unique_rows and ids.shape[-1] > 1:
        ordered = torch.sort(ids, dim=-1).values
        if bool((ordered[..., 1:] == ordered[..., :-1]).any().item()):
            raise ValueError(f"{name}: a row names the same expert twice")


def ids_below(name: str, ids: torch.Tensor, bound: int) -> None:
    """Every id in ``[0, bound)`` (ValueError).  Reads the device."""

    if ids.numel() == 0:
        return
    lo, hi = torch.stack(tuple(torch.aminmax(ids))).tolist()
    if lo < 0 or hi >= bound:
        raise ValueError(f"{name}: values span [{lo}, {hi}], outside [0, {bound})")


def route_weights(name: str, weights: torch.Tensor, *, row_sum: float | None) -> None:
    """Finite, strictly positive weights; with ``row_sum``, each row sums to
    it within 8 float32 epsilons of max(1, |row_sum|) (the invariant of a
    renormalised router, ``moe_runtime.py:463-475``).  ValueError; reads the
    device."""

    if not bool(torch.isfinite(weights).all().item()):
        raise ValueError(f"{name}: weights must be finite")
    if bool((weights <= 0).any().item()):
        raise ValueError(f"{name}: weights must be strictly positive")
    if row_sum is not None:
        err = float((weights.sum(dim=-1) - row_sum).abs().max().item())
        bound = 8.0 * torch.finfo(torch.float32).eps * max(1.0, abs(row_sum))
        if err > bound:
            raise ValueError(f"{name}: rows must sum to {row_sum} (off by up to {err:.3e} > {bound:.3e})")


__all__ = [
    "boolean",
    "byte_spans_disjoint",
    "distinct_storages",
    "e8m0_codes",
    "expert_table",
    "finite_positive",
    "ids_below",
    "no_reserved_e8m0",
    "owns_whole_storage",
    "positive_int",
    "route_weights",
    "same_device",
    "tensor",
]
