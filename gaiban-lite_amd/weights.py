"""Resident int4 group-128 MoE weights in the tiled device layout.

Counterpart of ``ResidentMoEWeights`` / ``MarlinRoutedWeights``
(``runtime/dsv4_direct/ops/marlin_moe.py:77-152``): all experts of one layer,
stacked over the expert axis, repacked once at load time by the HIP packer
(``dsv4moe_pack_int4_g128``) instead of vLLM's Marlin repack.  The shared
expert, when present, is stored as expert index ``experts`` in the same arrays
and runs inside the same grouped kernels with route weight 1.

Layout per expert (H = hidden, I = intermediate), pair-interleaved tiles of
16 rows x 128 K (see ``include/dsv4moe.h``, ``dsv4moe_pack_int4_g128``):
  w13_q  uint8 [E', I*H]        W13 [2I, H] (rows [0,I) gate w1, [I,2I) up w3),
                                gate strip p paired with up strip p
  w13_s  bf16  [E', 2I*H/128]
  w2_q   uint8 [E', H*I/2]      W2 [H, I], strips 2p and 2p+1 paired
  w2_s   bf16  [E', H*I/128]
with E' = experts + (1 if shared).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import contracts as C
from . import ops

GROUP = 128


@dataclass
class ResidentFP8SharedExpert:
    """The shared expert in the checkpoint's FP8 format (``SharedExpertSlice``,
    ``runtime/dsv4_direct/ops/marlin_moe.py:42-74``): E4M3 weights with one
    E8M0 scale per 128 x 128 block, repacked once into the W8A16 tile layout
    (``dsv4moe_pack_int8``, a byte permutation).  Runs as dense W8A16 linears
    (``dsv4moe_shared_fp8_add``), outside the grouped expert kernels.

      w13_q  uint8 [2I*H]           W13 = [W1; W3] [2I, H]
      w13_s  uint8 [2I/128, H/128]  E8M0 (W1's block rows, then W3's)
      w2_q   uint8 [H*I]            W2 [H, I]
      w2_s   uint8 [H/128, I/128]
    """

    w13_q: torch.Tensor
    w13_s: torch.Tensor
    w2_q: torch.Tensor
    w2_s: torch.Tensor
    hidden_size: int
    intermediate_size: int

    @property
    def device(self) -> torch.device:
        return self.w13_q.device

    @property
    def resident_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w13_q, self.w13_s, self.w2_q, self.w2_s))

    def validate(self) -> None:
        h, i = self.hidden_size, self.intermediate_size
        if h % GROUP or i % GROUP:
            raise ValueError("FP8 shared expert needs hidden and intermediate sizes that are multiples of 128")
        expected = {
            "w13_q": ((2 * i * h,), torch.uint8),
            "w13_s": ((2 * i // GROUP, h // GROUP), torch.uint8),
            "w2_q": ((h * i,), torch.uint8),
            "w2_s": ((h // GROUP, i // GROUP), torch.uint8),
        }
        for name, (shape, dtype) in expected.items():
            t = getattr(self, name)
            if tuple(t.shape) != shape or t.dtype != dtype:
                raise ValueError(f"{name} must be {dtype} {shape}, got {t.dtype} {tuple(t.shape)}")
            if not t.is_contiguous() or t.device != self.w13_q.device:
                raise ValueError(f"{name} must be contiguous on {self.w13_q.device}")

    @classmethod
    def from_checkpoint(cls, w1, s1, w3, s3, w2, s2) -> "ResidentFP8SharedExpert":
        """``w1``/``w3`` [I, H] and ``w2`` [H, I] float8_e4m3fn (or their uint8
        codes); ``s1``/``s3`` [I/128, H/128] and ``s2`` [H/128, I/128]
        float8_e8m0fnu (or uint8 codes).  Rejects the reserved E8M0 byte 255
        (a synchronising load-time check, as the reference's preflight)."""

        from .weight_only_linear import validate_e8m0_scale_values

        def codes(t):
            return t.view(torch.uint8) if t.dtype in (torch.float8_e4m3fn, torch.float8_e8m0fnu) else t

        w1, w3, w2 = codes(w1), codes(w3), codes(w2)
        s1, s3, s2 = codes(s1), codes(s3), codes(s2)
        for name, t in (("w1", w1), ("w3", w3), ("w2", w2), ("s1", s1), ("s3", s3), ("s2", s2)):
            if t.dtype != torch.uint8 or t.ndim != 2:
                raise TypeError(f"{name} must be a 2-D FP8 (or uint8) tensor")
        inter, hidden = w1.shape
        if w3.shape != (inter, hidden) or w2.shape != (hidden, inter):
            raise ValueError("w1/w3 must be [I, H] and w2 [H, I]")
        if inter % GROUP or hidden % GROUP:
            raise ValueError("hidden and intermediate sizes must be multiples of 128")
        for name, t, shape in (("s1", s1, (inter // GROUP, hidden // GROUP)), ("s3", s3, (inter // GROUP, hidden // GROUP)),
                               ("s2", s2, (hidden // GROUP, inter // GROUP))):
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} must be [{shape[0]}, {shape[1]}]")
            validate_e8m0_scale_values(name, t)
        w13 = torch.cat([w1, w3], dim=0).contiguous()
        out = cls(ops.pack_int8(w13.view(torch.int8)), torch.cat([s1, s3], dim=0).contiguous(),
                  ops.pack_int8(w2.contiguous().view(torch.int8)), s2.contiguous(), hidden, inter)
        out.validate()
        return out


def _validate_shared_fp8(resident) -> None:
    sh = resident.shared_fp8
    if sh is None:
        return
    if not isinstance(sh, ResidentFP8SharedExpert):
        raise TypeError("shared_fp8 must be ResidentFP8SharedExpert")
    if resident.has_shared:
        raise ValueError("a shared expert is either in the routed stack (has_shared) or in FP8, not both")
    if (sh.hidden_size, sh.intermediate_size) != (resident.hidden_size, resident.intermediate_size):
        raise ValueError("FP8 shared expert geometry does not match the routed experts")
    if sh.device != resident.w13_q.device:
        raise ValueError("FP8 shared expert must live on the routed experts' device")
    sh.validate()


def int4_g128_expert_bytes(hidden: int, inter: int) -> int:
    """Bytes of one expert's weights plus scales: 3*H*I/2 + 3*H*(I/128)*2."""

    return 3 * hidden * inter // 2 + 3 * hidden * (inter // GROUP) * 2


@dataclass
class ResidentInt4MoEWeights:
    w13_q: torch.Tensor
    w13_s: torch.Tensor
    w2_q: torch.Tensor
    w2_s: torch.Tensor
    experts: int
    hidden_size: int
    intermediate_size: int
    has_shared: bool
    layer_id: int | None = None
    checkpoint_id: str | None = None
    marlin_input_dtype: torch.dtype | None = None
    weight_format: str = "int4_g128"
    shared_fp8: ResidentFP8SharedExpert | None = None  # shared expert in the checkpoint FP8 format
    # fp32 ratios of consecutive group scales (ops.pack_int4_ratios), shaped as
    # w13_s / w2_s: the W4A16 prefill kernels' running-sum scaling reads them.
    # They are derived state: scale_ratios() recomputes them (in place, a
    # kernel launch, no allocation) whenever w13_s or w2_s was replaced or
    # written in place since, keyed on the scales' storage and version counter.
    w13_r: torch.Tensor | None = None
    w2_r: torch.Tensor | None = None
    _ratio_key: tuple | None = field(default=None, repr=False, compare=False)

    @property
    def device(self) -> torch.device:
        return self.w13_q.device

    @property
    def resident_bytes(self) -> int:
        tensors = [self.w13_q, self.w13_s, self.w2_q, self.w2_s]
        tensors += [t for t in (self.w13_r, self.w2_r) if t is not None]
        return sum(t.numel() * t.element_size() for t in tensors)

    def _scales_key(self) -> tuple:
        return tuple((t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape), t._version)
                     for t in (self.w13_s, self.w2_s))

    def scale_ratios(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(w13_r, w2_r), computed on the device from the packed scales: the
        first time into new tensors, later again into the same tensors when
        the scales changed since (new tensors, or an in-place write, which
        bumps their version counter).  Checking costs no device access; a
        recomputation is one kernel launch on the current stream, ordered
        before the work that follows it there."""

        key = self._scales_key()
        if self.w13_r is not None and self.w2_r is not None and key == self._ratio_key:
            return self.w13_r, self.w2_r
        if self.device.type != "cuda":
            raise ValueError("scale ratios are computed on the GPU; these weights live on the CPU")
        h, i = self.hidden_size, self.intermediate_size
        same_shape = (self.w13_r is not None and self.w2_r is not None
                      and self.w13_r.shape == self.w13_s.shape and self.w2_r.shape == self.w2_s.shape)
        self.w13_r = ops.pack_int4_ratios(self.w13_s, n=2 * i, k=h, out=self.w13_r if same_shape else None)
        self.w2_r = ops.pack_int4_ratios(self.w2_s, n=h, k=i, out=self.w2_r if same_shape else None)
        self._ratio_key = key
        return self.w13_r, self.w2_r

    @property
    def bytes_per_expert(self) -> int:
        return int4_g128_expert_bytes(self.hidden_size, self.intermediate_size)

    def validate(self) -> None:
        e_tot = self.experts + (1 if self.has_shared else 0)
        h, i = self.hidden_size, self.intermediate_size
        if h % GROUP or i % GROUP:
            raise ValueError("hidden and intermediate sizes must be multiples of 128")
        expected = {
            "w13_q": ((e_tot, i * h), torch.uint8),
            "w13_s": ((e_tot, 2 * i * (h // GROUP)), torch.bfloat16),
            "w2_q": ((e_tot, h * i // 2), torch.uint8),
            "w2_s": ((e_tot, h * (i // GROUP)), torch.bfloat16),
        }
        for name in ("w13_r", "w2_r"):
            if getattr(self, name) is not None:
                expected[name] = (expected[name.replace("_r", "_s")][0], torch.float32)
        for name, (shape, dtype) in expected.items():
            t = getattr(self, name)
            if tuple(t.shape) != shape or t.dtype != dtype:
                raise ValueError(f"{name} must be {dtype} {shape}, got {t.dtype} {tuple(t.shape)}")
            if not t.is_contiguous() or t.device != self.w13_q.device:
                raise ValueError(f"{name} must be contiguous on {self.w13_q.device}")
        _validate_shared_fp8(self)

    @classmethod
    def from_checkpoint_layout(
        cls,
        w13_packed: torch.Tensor,
        w13_scale: torch.Tensor,
        w2_packed: torch.Tensor,
        w2_scale: torch.Tensor,
        *,
        experts: int,
        has_shared: bool,
        layer_id: int | None = None,
        checkpoint_id: str | None = None,
        marlin_input_dtype: torch.dtype | None = None,
        shared_fp8: ResidentFP8SharedExpert | None = None,
    ) -> "ResidentInt4MoEWeights":
        """Repack stacked checkpoint-layout experts on the device.

        ``w13_packed`` [E', 2I, H/2] u8 (low nibble = even k, two's complement),
        ``w13_scale`` [E', 2I, H/128] bf16, ``w2_packed`` [E', H, I/2] u8,
        ``w2_scale`` [E', H, I/128] bf16.
        """

        e_tot, two_i, half_h = w13_packed.shape
        inter, hidden = two_i // 2, half_h * 2
        if w2_packed.shape != (e_tot, hidden, inter // 2):
            raise ValueError("w2_packed must be [E', H, I/2] matching w13_packed")
        if e_tot != experts + (1 if has_shared else 0):
            raise ValueError("expert count does not match the stacked tensors")
        q13, s13 = ops.pack_int4_g128(w13_packed.contiguous(), w13_scale.contiguous(), gated=True)
        q2, s2 = ops.pack_int4_g128(w2_packed.contiguous(), w2_scale.contiguous(), gated=False)
        out = cls(q13, s13, q2, s2, experts, hidden, inter, has_shared, layer_id, checkpoint_id,
                  marlin_input_dtype, shared_fp8=shared_fp8)
        if marlin_input_dtype is None:  # the W4A16 kernels' running-sum ratios
            out.scale_ratios()
        out.validate()
        return out


def mxfp4_g32_expert_bytes(hidden: int, inter: int) -> int:
    """Bytes of one MXFP4 expert: 3*H*I/2 E2M1 codes + 3*H*I/32 E8M0 scales."""

    return 3 * hidden * inter // 2 + 3 * hidden * inter // 32


@dataclass
class ResidentMXFP4MoEWeights:
    """MXFP4 experts (E2M1 codes, one E8M0 scale per 32 K): the checkpoint
    format of the reference's routed experts (``runtime/dsv4_direct/ops/
    marlin_moe.py:77-105,173-223``; ``moe_forward.py:126-155``), repacked once
    by ``dsv4moe_pack_mxfp4_g32`` into the tile geometry of the int4 layout.

      w13_q  uint8 [E', I*H]         W13 [2I, H], gate strip p paired with up strip p
      w13_s  uint8 [E', 2I*H/32]     E8M0 scales
      w2_q   uint8 [E', H*I/2]       W2 [H, I]
      w2_s   uint8 [E', H*I/32]
    """

    w13_q: torch.Tensor
    w13_s: torch.Tensor
    w2_q: torch.Tensor
    w2_s: torch.Tensor
    experts: int
    hidden_size: int
    intermediate_size: int
    has_shared: bool
    layer_id: int | None = None
    checkpoint_id: str | None = None
    marlin_input_dtype: torch.dtype | None = None
    weight_format: str = "mxfp4_g32"
    shared_fp8: ResidentFP8SharedExpert | None = None  # shared expert in the checkpoint FP8 format
    load_seconds: float | None = None  # set by the checkpoint loader
    # the tensor-parallel slice the loader took (world size 1: the whole layer)
    rank: int = 0
    world_size: int = 1
    intermediate_start: int | None = None
    intermediate_end: int | None = None

    @property
    def routed(self) -> "ResidentMXFP4MoEWeights":
        """The routed experts (this container), as the reference's resident
        record names them."""

        return self

    @property
    def shared(self) -> ResidentFP8SharedExpert | None:
        """The FP8 shared expert, as the reference's resident record names it."""

        return self.shared_fp8

    @property
    def device(self) -> torch.device:
        return self.w13_q.device

    @property
    def resident_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w13_q, self.w13_s, self.w2_q, self.w2_s))

    @property
    def bytes_per_expert(self) -> int:
        return mxfp4_g32_expert_bytes(self.hidden_size, self.intermediate_size)

    def validate(self) -> None:
        e_tot = self.experts + (1 if self.has_shared else 0)
        h, i = self.hidden_size, self.intermediate_size
        if h % 512 or i % 512:
            raise ValueError("MXFP4 experts need hidden and intermediate sizes that are multiples of 512")
        if self.marlin_input_dtype not in (None, torch.float8_e4m3fn):
            raise ValueError(f"MXFP4 experts run with bf16 or float8_e4m3fn activations, not {self.marlin_input_dtype}")
        expected = {
            "w13_q": ((e_tot, i * h), torch.uint8),
            "w13_s": ((e_tot, 2 * i * h // 32), torch.uint8),
            "w2_q": ((e_tot, h * i // 2), torch.uint8),
            "w2_s": ((e_tot, h * i // 32), torch.uint8),
        }
        for name, (shape, dtype) in expected.items():
            t = getattr(self, name)
            if tuple(t.shape) != shape or t.dtype != dtype:
                raise ValueError(f"{name} must be {dtype} {shape}, got {t.dtype} {tuple(t.shape)}")
            if not t.is_contiguous() or t.device != self.w13_q.device:
                raise ValueError(f"{name} must be contiguous on {self.w13_q.device}")
        _validate_shared_fp8(self)

    @classmethod
    def from_checkpoint_layout(
        cls,
        w13_packed: torch.Tensor,
        w13_scale: torch.Tensor,
        w2_packed: torch.Tensor,
        w2_scale: torch.Tensor,
        *,
        experts: int,
        has_shared: bool,
        layer_id: int | None = None,
        checkpoint_id: str | None = None,
        shared_fp8: ResidentFP8SharedExpert | None = None,
        marlin_input_dtype: torch.dtype | None = None,
    ) -> "ResidentMXFP4MoEWeights":
        """Repack stacked checkpoint-layout experts on the device.

        ``w13_packed`` [E', 2I, H/2] u8 (E2M1, low nibble = even k),
        ``w13_scale`` [E', 2I, H/32] u8 (E8M0, or torch.float8_e8m0fnu viewed as
        bytes), ``w2_packed`` [E', H, I/2] u8, ``w2_scale`` [E', H, I/32] u8.
        The reserved scale byte 255 (NaN in the reference's decode) is
        rejected with ValueError; the check reads the device (load time).
        ``marlin_input_dtype=torch.float8_e4m3fn`` packs for the W4A8 kernels
        (per-token e4m3 activations; the reference's ``is_a_8bit`` repack,
        ``ops/marlin_moe.py:197-222``): same bytes, another lane layout.
        """

        def as_u8(t):
            return t.view(torch.uint8) if t.dtype != torch.uint8 and t.element_size() == 1 else t

        e_tot, two_i, half_h = w13_packed.shape
        inter, hidden = two_i // 2, half_h * 2
        if w2_packed.shape != (e_tot, hidden, inter // 2):
            raise ValueError("w2_packed must be [E', H, I/2] matching w13_packed")
        if e_tot != experts + (1 if has_shared else 0):
            raise ValueError("expert count does not match the stacked tensors")
        C.no_reserved_e8m0("w13_scale", w13_scale)
        C.no_reserved_e8m0("w2_scale", w2_scale)
        if marlin_input_dtype not in (None, torch.float8_e4m3fn):
            raise ValueError(f"unsupported marlin_input_dtype {marlin_input_dtype!r}")
        a8 = marlin_input_dtype is not None
        q13, s13 = ops.pack_mxfp4_g32(as_u8(w13_packed).contiguous(), as_u8(w13_scale).contiguous(), gated=True,
                                      w4a8=a8)
        q2, s2 = ops.pack_mxfp4_g32(as_u8(w2_packed).contiguous(), as_u8(w2_scale).contiguous(), gated=False,
                                    w4a8=a8)
        out = cls(q13, s13, q2, s2, experts, hidden, inter, has_shared, layer_id, checkpoint_id,
                  marlin_input_dtype=marlin_input_dtype, shared_fp8=shared_fp8)
        out.validate()
        return out


__all__ = ["ResidentFP8SharedExpert", "ResidentInt4MoEWeights", "ResidentMXFP4MoEWeights",
           "int4_g128_expert_bytes", "mxfp4_g32_expert_bytes"]
