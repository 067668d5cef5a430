"""Seeded synthetic inputs and weights for the benchmark configurations.

Distributions follow the benchmark definitions of this build (hidden states
bf16 ~ N(0,1); router logits fp32 ~ N(0,1); int4 values uniform in [-8, 7];
bf16 group scales ~ U(0.005, 0.02)) and the reference's routing pools
(``experiments/A3F-marlin-moe-flash/common.py:198-211``: uniform, Zipf via
Gumbel-top-k with p ~ rank^-alpha).  Generation runs with torch generators on
the target device; it is input preparation, not part of any timed path.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

GROUP = 128


@dataclass(frozen=True)
class LayerShape:
    experts: int
    hidden: int
    inter: int
    topk: int
    has_shared: bool

    @property
    def total_experts(self) -> int:
        return self.experts + (1 if self.has_shared else 0)


TINY = LayerShape(experts=8, hidden=1024, inter=512, topk=2, has_shared=False)
FLASH = LayerShape(experts=256, hidden=4096, inter=2048, topk=6, has_shared=True)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_checkpoint_experts(shape: LayerShape, *, seed: int = 0, device="cuda",
                            experts: range | None = None):
    """Checkpoint-layout int4-g128 weights for all (or a range of) experts.

    Returns (w13_packed [n, 2I, H/2] u8, w13_scale [n, 2I, H/128] bf16,
             w2_packed [n, H, I/2] u8, w2_scale [n, H, I/128] bf16).
    Each expert index e is generated from its own seeded stream
    (seed * 1_000_003 + e), so any subset reproduces the same bytes.
    """

    ids = range(shape.total_experts) if experts is None else experts
    n = len(ids)
    h, i = shape.hidden, shape.inter
    w13 = torch.empty((n, 2 * i, h // 2), dtype=torch.uint8, device=device)
    s13 = torch.empty((n, 2 * i, h // GROUP), dtype=torch.bfloat16, device=device)
    w2 = torch.empty((n, h, i // 2), dtype=torch.uint8, device=device)
    s2 = torch.empty((n, h, i // GROUP), dtype=torch.bfloat16, device=device)
    for slot, e in enumerate(ids):
        g = _gen(seed * 1_000_003 + e, device)
        w13[slot] = torch.randint(0, 256, (2 * i, h // 2), dtype=torch.uint8, device=device, generator=g)
        s13[slot] = (torch.rand((2 * i, h // GROUP), device=device, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
        w2[slot] = torch.randint(0, 256, (h, i // 2), dtype=torch.uint8, device=device, generator=g)
        s2[slot] = (torch.rand((h, i // GROUP), device=device, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    return w13, s13, w2, s2


def make_checkpoint_experts_mxfp4(shape: LayerShape, *, seed: int = 0, device="cuda",
                                  experts: range | None = None):
    """Checkpoint-layout MXFP4 weights (the reference's routed-expert format,
    ``moe_forward.py:126-155``) for all (or a range of) experts.

    Returns (w13_packed [n, 2I, H/2] u8, w13_scale [n, 2I, H/32] u8 E8M0,
             w2_packed [n, H, I/2] u8, w2_scale [n, H, I/32] u8 E8M0).
    Codes are uniform bytes (two E2M1 codes each); E8M0 scale bytes are
    uniform in [119, 122], i.e. 2^-8 .. 2^-5, which gives weights of the same
    magnitude as the int4-g128 generator.  Seeded per expert as
    ``make_checkpoint_experts``.
    """

    ids = range(shape.total_experts) if experts is None else experts
    n = len(ids)
    h, i = shape.hidden, shape.inter
    w13 = torch.empty((n, 2 * i, h // 2), dtype=torch.uint8, device=device)
    s13 = torch.empty((n, 2 * i, h // 32), dtype=torch.uint8, device=device)
    w2 = torch.empty((n, h, i // 2), dtype=torch.uint8, device=device)
    s2 = torch.empty((n, h, i // 32), dtype=torch.uint8, device=device)
    for slot, e in enumerate(ids):
        g = _gen(seed * 1_000_003 + e + 500_000, device)
        w13[slot] = torch.randint(0, 256, (2 * i, h // 2), dtype=torch.uint8, device=device, generator=g)
        s13[slot] = torch.randint(119, 123, (2 * i, h // 32), dtype=torch.uint8, device=device, generator=g)
        w2[slot] = torch.randint(0, 256, (h, i // 2), dtype=torch.uint8, device=device, generator=g)
        s2[slot] = torch.randint(119, 123, (h, i // 32), dtype=torch.uint8, device=device, generator=g)
    return w13, s13, w2, s2


def make_hidden(tokens: int, hidden: int, *, seed: int = 1, device="cuda") -> torch.Tensor:
    return torch.randn((tokens, hidden), device=device, generator=_gen(seed, device)).to(torch.bfloat16)


def make_logits(tokens: int, experts: int, *, seed: int = 2, device="cuda") -> torch.Tensor:
    return torch.randn((tokens, experts), device=device, generator=_gen(seed, device), dtype=torch.float32)


def zipf_ids(tokens: int, experts: int, topk: int, *, alpha: float = 1.1, seed: int = 4,
             device="cuda") -> torch.Tensor:
    """Gumbel-top-k (Plackett-Luce without replacement) with p ~ rank^-alpha
    (``common.py:202-206``); int32 [tokens, topk]."""

    g = _gen(seed, device)
    p = torch.arange(1, experts + 1, device=device, dtype=torch.float32) ** (-alpha)
    u = torch.rand((tokens, experts), device=device, generator=g).clamp_min(1e-20)
    logits = p.log() + (-torch.log(-torch.log(u)))
    return logits.topk(topk, dim=-1)[1].to(torch.int32)


def make_int8_linear(n: int, k: int, *, seed: int = 3, device="cuda"):
    """W8A16 weights: int8 uniform in [-127, 127] [n, k] and bf16 per-channel
    scales ~ U(0.005, 0.02) [n]."""

    g = _gen(seed * 1_000_003 + 77, device)
    q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=device, generator=g)
    s = (torch.rand((n,), device=device, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    return q, s


def make_fp8_block_linear(n: int, k: int, *, seed: int = 3, device="cuda", std: float = 0.02):
    """Checkpoint-style FP8 block weights: W ~ N(0, std^2) [n, k] quantised per
    128 x 128 block to E4M3 with the power-of-two E8M0 scale 2^ceil(log2(amax/448))
    (the block's largest magnitude maps into E4M3's range).  Returns
    (codes uint8 [n, k], scale codes uint8 [ceil(n/128), k/128])."""

    g = _gen(seed * 1_000_003 + 91, device)
    w = torch.randn((n, k), device=device, generator=g) * std
    nb, kb = (n + 127) // 128, k // 128
    pad = torch.zeros((nb * 128, k), device=device)
    pad[:n] = w
    amax = pad.abs().view(nb, 128, kb, 128).amax(dim=(1, 3)).clamp_min(1e-30)
    e = torch.ceil(torch.log2(amax / 448.0)).clamp(-127, 127)
    scale = torch.exp2(e)
    q = (pad.view(nb, 128, kb, 128) / scale[:, None, :, None]).view(nb * 128, k)[:n]
    codes = q.to(torch.float8_e4m3fn).view(torch.uint8)
    return codes.contiguous(), (e + 127).to(torch.uint8).contiguous()


__all__ = [
    "FLASH",
    "TINY",
    "LayerShape",
    "make_checkpoint_experts",
    "make_checkpoint_experts_mxfp4",
    "make_hidden",
    "make_fp8_block_linear",
    "make_int8_linear",
    "make_logits",
    "zipf_ids",
]
