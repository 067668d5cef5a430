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

from dataclasses import dataclass

import torch

from . import ops

GROUP = 128


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

    @property
    def device(self) -> torch.device:
        return self.w13_q.device

    @property
    def resident_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w13_q, self.w13_s, self.w2_q, self.w2_s))

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
        for name, (shape, dtype) in expected.items():
            t = getattr(self, name)
            if tuple(t.shape) != shape or t.dtype != dtype:
                raise ValueError(f"{name} must be {dtype} {shape}, got {t.dtype} {tuple(t.shape)}")
            if not t.is_contiguous() or t.device != self.w13_q.device:
                raise ValueError(f"{name} must be contiguous on {self.w13_q.device}")

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
                  marlin_input_dtype)
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
        if self.marlin_input_dtype is not None:
            raise ValueError("MXFP4 experts run with bf16 activations (W4A16)")
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
    ) -> "ResidentMXFP4MoEWeights":
        """Repack stacked checkpoint-layout experts on the device.

        ``w13_packed`` [E', 2I, H/2] u8 (E2M1, low nibble = even k),
        ``w13_scale`` [E', 2I, H/32] u8 (E8M0, or torch.float8_e8m0fnu viewed as
        bytes), ``w2_packed`` [E', H, I/2] u8, ``w2_scale`` [E', H, I/32] u8.
        """

        def as_u8(t):
            return t.view(torch.uint8) if t.dtype != torch.uint8 and t.element_size() == 1 else t

        e_tot, two_i, half_h = w13_packed.shape
        inter, hidden = two_i // 2, half_h * 2
        if w2_packed.shape != (e_tot, hidden, inter // 2):
            raise ValueError("w2_packed must be [E', H, I/2] matching w13_packed")
        if e_tot != experts + (1 if has_shared else 0):
            raise ValueError("expert count does not match the stacked tensors")
        q13, s13 = ops.pack_mxfp4_g32(as_u8(w13_packed).contiguous(), as_u8(w13_scale).contiguous(), gated=True)
        q2, s2 = ops.pack_mxfp4_g32(as_u8(w2_packed).contiguous(), as_u8(w2_scale).contiguous(), gated=False)
        out = cls(q13, s13, q2, s2, experts, hidden, inter, has_shared, layer_id, checkpoint_id)
        out.validate()
        return out


__all__ = ["ResidentInt4MoEWeights", "ResidentMXFP4MoEWeights", "int4_g128_expert_bytes",
           "mxfp4_g32_expert_bytes"]
