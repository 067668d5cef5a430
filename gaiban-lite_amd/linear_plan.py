"""Launch plans of the dense linears.

Both linear modules of the reference -- the checkpoint-FP8 weight-only linear
(``experiments/C1F-integrated-block/weight_only_linear.py:61-135,168-221``)
and the block-FP8 W8A8 linear (``runtime/dsv4_direct/fp8_linear.py:53-153,
166-234``) -- describe a call by the same frozen plan: (M, N, K, split_k)
plus a Triton tuning record, from which every caller-owned tensor shape
follows (activation [M, K], weight [N, K] with E8M0 block scales
[ceil(N/128), K/128], output [M, N], fp32 split-K workspace [split, M, N] or
the placeholder (0,) for one split).  The names and meanings of those fields
are the observable contract and are kept; this module states them once for
both modules.

What differs from the reference: the automatic split comes from this
library's policy for its own kernel tiles (``dsv4moe_w8a16_split_k`` /
``dsv4moe_block_fp8_split_k``), and the tuning record is carried for plan
identity only -- the HIP kernels choose their own tiles, so ``output_grid``
and ``gemm_grid`` describe the reference's Triton grid for that record, not
this library's launches.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Final

from . import contracts as C

BLOCK_K: Final = 128
WEIGHT_BLOCK_N: Final = 128
SUPPORTED_SPLIT_K: Final = (1, 2, 4, 8)


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


@dataclass(frozen=True)
class GemmTuning:
    """The reference's Triton tile record (its defaults: 32 x 64 tiles, 4
    warps, 3 stages).  Kept so plans compare and print like the reference's;
    the HIP kernels do not read it."""

    block_m: int = 32
    block_n: int = 64
    num_warps: int = 4
    num_stages: int = 3


DEFAULT_GEMM_TUNING: Final = GemmTuning()


@dataclass(frozen=True)
class GemmPlan:
    """One GEMM geometry and the shapes of its caller-owned tensors."""

    m: int
    n: int
    k: int
    split_k: int
    tuning: GemmTuning = DEFAULT_GEMM_TUNING

    # caller-owned tensors
    activation_shape = property(lambda self: (self.m, self.k))
    activation_scale_shape = property(lambda self: (self.m, self.k // BLOCK_K))
    weight_shape = property(lambda self: (self.n, self.k))
    weight_scale_shape = property(lambda self: (_cdiv(self.n, WEIGHT_BLOCK_N), self.k // BLOCK_K))
    output_shape = property(lambda self: (self.m, self.n))
    workspace_elements = property(lambda self: self.split_k * self.m * self.n if self.split_k > 1 else 0)
    workspace_bytes = property(lambda self: 4 * self.workspace_elements)

    @property
    def workspace_shape(self) -> tuple[int, ...]:
        return (self.split_k, self.m, self.n) if self.split_k > 1 else (0,)

    @property
    def dispatch(self) -> str:
        return "split_k_reduce" if self.split_k > 1 else "full_k"

    @property
    def k_blocks_per_split(self) -> int:
        return _cdiv(self.k // BLOCK_K, self.split_k)

    # the reference's Triton grid for this plan's tuning record
    @property
    def output_grid(self) -> tuple[int, int]:
        return (_cdiv(self.m, self.tuning.block_m), _cdiv(self.n, self.tuning.block_n))

    @property
    def gemm_grid(self) -> tuple[int, ...]:
        return self.output_grid + ((self.split_k,) if self.split_k > 1 else ())


# Values the reference's Triton launcher accepts for each tuning field
# (``weight_only_linear.py:147-165``; ``fp8_linear.py`` checks the same set).
TUNING_CHOICES: Final = {
    "block_m": (16, 32, 64),
    "block_n": (32, 64, 128),
    "num_warps": (4, 8),
    "num_stages": (2, 3, 4),
}
# Output channels per MFMA strip: every linear kernel here writes whole
# 16-channel strips, so N must be a multiple of this.
N_MULTIPLE: Final = 16


def validate_tuning(tuning: GemmTuning) -> None:
    """TypeError unless ``tuning`` is a GemmTuning; ValueError for a field that
    is not an int or not one of the reference's supported values, or a
    block_n that does not divide the 128-channel weight scale block."""

    if not isinstance(tuning, GemmTuning):
        raise TypeError(f"tuning: expected GemmTuning, got {type(tuning).__name__}")
    for field, allowed in TUNING_CHOICES.items():
        value = getattr(tuning, field)
        if isinstance(value, bool) or not isinstance(value, int):
            raise ValueError(f"tuning.{field} must be an int, got {value!r}")
        if value not in allowed:
            raise ValueError(f"tuning.{field}={value} is not one of {allowed}")
    if WEIGHT_BLOCK_N % tuning.block_n:
        raise ValueError(f"tuning.block_n={tuning.block_n} does not divide the {WEIGHT_BLOCK_N}-channel scale block")


def build_plan(m: int, n: int, k: int, *, split_k: int | None, tuning: GemmTuning,
               policy: Callable[[int, int, int], int]) -> GemmPlan:
    """A validated plan; ``policy`` picks the split when ``split_k`` is None.
    Every violation is a ValueError, as in both reference modules, except a
    tuning record of the wrong type (TypeError)."""

    dims = [C.positive_int(name, v) for name, v in (("m", m), ("n", n), ("k", k))]
    validate_tuning(tuning)
    if dims[2] % BLOCK_K:
        raise ValueError(f"k={k} is not a multiple of {BLOCK_K}")
    if dims[1] % N_MULTIPLE:
        raise ValueError(f"n={n} is not a multiple of {N_MULTIPLE}: the kernels store 16-channel strips")
    chosen = policy(*dims) if split_k is None else split_k
    if isinstance(chosen, bool) or chosen not in SUPPORTED_SPLIT_K:
        raise ValueError(f"split_k={chosen!r} is not one of {SUPPORTED_SPLIT_K}")
    if chosen > dims[2] // BLOCK_K:
        raise ValueError(f"split_k={chosen} exceeds the {dims[2] // BLOCK_K} K blocks of k={k}")
    return GemmPlan(*dims, split_k=chosen, tuning=tuning)


__all__ = ["BLOCK_K", "DEFAULT_GEMM_TUNING", "GemmPlan", "GemmTuning", "N_MULTIPLE", "SUPPORTED_SPLIT_K",
           "TUNING_CHOICES", "WEIGHT_BLOCK_N", "build_plan", "validate_tuning"]
