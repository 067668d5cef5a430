"""Shared test helpers: moving device data to the oracle, tolerances, layouts."""

from __future__ import annotations

import numpy as np
import torch

import oracle as O

# Parity bar for bf16 layer outputs against the fp32 dequant oracle (north
# star: "within max relative error 1e-2 against an fp32 accumulation of the
# same dequantized weights"): both the normwise max error max|d| / max|ref|
# and the Frobenius relative error ||d|| / ||ref|| must be <= 1e-2.
MOE_TOL = 1e-2


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_np_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


class DeviceExpertSource(O.ExpertSource):
    """Oracle accessor over device-resident checkpoint-layout experts; each
    expert is copied to the host only when the oracle touches it."""

    def __init__(self, w13, s13, w2, s2, group: int = 128):
        super().__init__(w13, s13, w2, s2, group)
        self._cache: dict[tuple[str, int], np.ndarray] = {}

    def _get(self, which: str, e: int) -> np.ndarray:
        key = (which, e)
        if key not in self._cache:
            if which == "w13":
                v = O.dequant_int4_g128(self.w13_packed[e].cpu().numpy(), bf16_bits(self.w13_scale[e]), self.group)
            else:
                v = O.dequant_int4_g128(self.w2_packed[e].cpu().numpy(), bf16_bits(self.w2_scale[e]), self.group)
            if len(self._cache) > 64:
                self._cache.clear()
            self._cache[key] = v
        return self._cache[key]

    def w13(self, e: int) -> np.ndarray:
        return self._get("w13", e)

    def w2(self, e: int) -> np.ndarray:
        return self._get("w2", e)


class DeviceMXFP4Source(O.MXFP4ExpertSource):
    """Oracle accessor over device-resident MXFP4 experts (copied per expert)."""

    def __init__(self, w13, s13, w2, s2):
        super().__init__(w13, s13, w2, s2)
        self._cache: dict[tuple[str, int], np.ndarray] = {}

    def _get(self, which: str, e: int) -> np.ndarray:
        key = (which, e)
        if key not in self._cache:
            if len(self._cache) > 64:
                self._cache.clear()
            if which == "w13":
                v = O.dequant_mxfp4(self.w13_packed[e].cpu().numpy(), self.w13_scale[e].cpu().numpy())
            else:
                v = O.dequant_mxfp4(self.w2_packed[e].cpu().numpy(), self.w2_scale[e].cpu().numpy())
            self._cache[key] = v
        return self._cache[key]

    def w13(self, e: int) -> np.ndarray:
        return self._get("w13", e)

    def w2(self, e: int) -> np.ndarray:
        return self._get("w2", e)


def block_cover_rows(sorted_token_ids, num_tokens_post_padded: int, block_size: int, tokens: int,
                     topk: int) -> np.ndarray:
    """One token of every alignment block (its first real slot), plus the
    first and last token: a row set on which every expert block of the
    grouped kernels contributes to some checked output row."""

    s = np.asarray(sorted_token_ids)[:num_tokens_post_padded].reshape(-1, block_size)
    firsts = s[:, 0]
    assert (firsts < tokens * topk).all(), "an alignment block starts with padding"
    return np.unique(np.r_[firsts // topk, 0, tokens - 1])


def moe_errors(out, ref) -> dict:
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = o - r
    return {
        "max_rel": float(np.abs(d).max() / max(np.abs(r).max(), 1e-30)),
        "rel_fro": float(np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30)),
        "max_abs": float(np.abs(d).max()),
    }


def assert_moe_close(out, ref, tol: float = MOE_TOL, what: str = "") -> dict:
    err = moe_errors(out, ref)
    assert np.isfinite(np.asarray(out, dtype=np.float64)).all(), f"{what}: non-finite output"
    assert err["max_rel"] <= tol and err["rel_fro"] <= tol, f"{what}: {err}"
    return err


def np_tile_pack(canon: np.ndarray, scales_bits: np.ndarray, gated: bool = False):
    """Independent numpy statement of the pair-interleaved tiled int4 layout
    (see gaiban-lite_amd/csrc/pack.hip): returns (packed bytes [n*k/2],
    scales [n*k/128] as uint16)."""

    q = O.unpack_int4_rows(canon).astype(np.int32)  # [n, k]
    n, k = q.shape
    groups = k // 128
    pairs = n // 32
    lane = np.arange(64)
    # zero-scale groups: codes 0, scale = nearest nonzero of the row
    # (previous group first, else next, else bf16 1.0)
    sb = scales_bits.reshape(n, groups).copy()
    zero = (sb & 0x7FFF) == 0
    orig = sb.copy()
    for r, g in zip(*np.nonzero(zero)):
        q[r, g * 128:(g + 1) * 128] = 0
        prev = [h for h in range(g - 1, -1, -1) if not zero[r, h]]
        nxt = [h for h in range(g + 1, groups) if not zero[r, h]]
        sb[r, g] = orig[r, prev[0]] if prev else (orig[r, nxt[0]] if nxt else 0x3F80)
    u = (q + 8).astype(np.uint32)

    def row0(p, m):
        return (p * 16 + m * (n // 2)) if gated else ((2 * p + m) * 16)

    out = np.zeros((pairs, groups, 2, 64, 4), dtype=np.uint32)
    sc = np.zeros((pairs, groups, 4, 2, 4), dtype=np.uint16)
    for p in range(pairs):
        for m in range(2):
            rows = row0(p, m) + lane % 16
            for g in range(groups):
                for d in range(4):
                    k0 = g * 128 + 32 * d + 8 * (lane // 16)
                    word = np.zeros(64, dtype=np.uint32)
                    for j in range(4):
                        word |= u[rows, k0 + 2 * j] << np.uint32(4 * j)
                        word |= u[rows, k0 + 2 * j + 1] << np.uint32(16 + 4 * j)
                    out[p, g, m, :, d] = word
                for quad in range(4):
                    sc[p, g, quad, m, :] = sb[row0(p, m) + 4 * quad + np.arange(4), g]
    return out.reshape(-1).view(np.uint8), sc.reshape(-1)


def np_tile_pack_mxfp4(canon: np.ndarray, scale_codes: np.ndarray, gated: bool = False):
    """Independent numpy statement of the MXFP4 tile layout (see
    gaiban-lite_amd/csrc/pack.hip): returns (packed bytes [n*k/2], scale bytes
    [n*k/32])."""

    n, half_k = canon.shape
    k = half_k * 2
    groups = k // 128
    pairs = n // 32
    lane = np.arange(64)

    def row0(p, m):
        return (p * 16 + m * (n // 2)) if gated else ((2 * p + m) * 16)

    out = np.zeros((pairs, groups, 2, 64, 16), dtype=np.uint8)
    sc = np.zeros((pairs, groups, 16, 2, 4), dtype=np.uint8)
    for p in range(pairs):
        for m in range(2):
            rows = row0(p, m) + lane % 16
            for g in range(groups):
                for d in range(4):
                    b0 = (g * 128 + 32 * d + 8 * (lane // 16)) // 2
                    for j in range(4):
                        out[p, g, m, :, 4 * d + j] = canon[rows, b0 + j]
                for r16 in range(16):
                    sc[p, g, r16, m, :] = scale_codes[row0(p, m) + r16, 4 * g:4 * g + 4]
    return out.reshape(-1), sc.reshape(-1)
