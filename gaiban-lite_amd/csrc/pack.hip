// Load-time repack of int4 group-128 weights into the pair-interleaved tiled
// layout that the expert kernels stream contiguously.
//
// Checkpoint layout (the convention of runtime/dsv4_direct/moe_forward.py:126-131):
//   canon[n][k/2]: byte b holds k = 2b in its low nibble, k = 2b+1 in its high
//   nibble, two's complement q in [-8, 7]; scales[n][k/128] bf16.
//
// Tiled layout.  Rows are grouped in 16-row strips and strips in pairs; pair
// p has members m = 0, 1:
//   pairing 0 (plain): member m is strip 2p + m  (rows 32p + 16m ...);
//   pairing 1 (gated): member 0 is strip p of the first half of the rows and
//                      member 1 strip p of the second half (rows 16p and
//                      n/2 + 16p): the gate (w1) and up (w3) rows a SwiGLU
//                      output column needs.
// Tile (p, g, m) -- 16 rows x k in [128g, 128g+128) -- is stored at byte
// ((p*G + g)*2 + m) * 1024, so one pair's two tiles of a group are adjacent
// and a pair streams one contiguous region over K.  Inside a tile, lane L
// (0..63) owns bytes L*16..L*16+15; dword d (0..3) holds row L%16 of the strip,
// k0 = 128g + 32d + 8*(L/16): nibble slot j (bits 4j..) = k0+2j and slot 4+j
// (bits 16+4j..) = k0+2j+1, offset-binary (q + 8).
// Scales: element (((p*G + g)*4 + quad)*2 + m)*4 + i holds the scale of row
// 4*quad + i of member m, so one 16-byte load returns 4 rows of both members.
//
// Zero scales.  A group whose scale is +-0 contributes exactly zero; the
// packer stores its codes as q = 0 and gives it the nearest nonzero scale of
// the same row (the previous group's, else the next one's, else 1.0).  The
// product q * s is unchanged for every weight, and every packed scale is
// nonzero, which the prefill kernels rely on: they keep each row's running
// sum divided by the current group's scale and multiply it by the ratio of
// consecutive scales.
#include "common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

__device__ __forceinline__ int64_t member_row0(int64_t p, int m, int64_t n, int pairing) {
  return pairing == 0 ? (2 * p + m) * 16 : p * 16 + m * (n / 2);
}

__device__ __forceinline__ bool scale_is_zero(uint16_t bits) { return (bits & 0x7FFFu) == 0; }

__global__ __launch_bounds__(256) void pack_int4_kernel(const uint8_t* __restrict__ canon,
                                                        const uint16_t* __restrict__ canon_s,
                                                        uint8_t* __restrict__ packed,
                                                        int64_t n, int64_t k, int64_t batch,
                                                        int pairing) {
  const int64_t groups = k / kGroup;
  const int64_t tiles_per_mat = (n / 16) * groups;
  const int64_t total = batch * tiles_per_mat * 64;  // one thread per (tile, lane)
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const int64_t tile = idx >> 6;  // destination tile order: (mat, p, g, m)
    const int64_t mat = tile / tiles_per_mat;
    const int64_t tin = tile % tiles_per_mat;
    const int m = (int)(tin & 1);
    const int64_t g = (tin >> 1) % groups;
    const int64_t p = (tin >> 1) / groups;
    const int64_t row = member_row0(p, m, n, pairing) + (lane & 15);
    const uint8_t* src_row = canon + mat * n * (k / 2) + row * (k / 2);
    const bool zero_group = scale_is_zero(canon_s[mat * n * groups + row * groups + g]);
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int64_t k0 = g * kGroup + 32 * d + 8 * (lane >> 4);
      const uint32_t src = *reinterpret_cast<const uint32_t*>(src_row + k0 / 2);
      uint32_t w = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (src >> (8 * b)) & 0xFFu;
        w |= ((byte & 0xFu) ^ 0x8u) << (4 * b);
        w |= ((byte >> 4) ^ 0x8u) << (16 + 4 * b);
      }
      out[d] = zero_group ? 0x88888888u : w;  // q = 0 in every slot
    }
    *reinterpret_cast<u32x4*>(packed + mat * n * (k / 2) + tin * kTileBytes + lane * 16) = out;
  }
}

__global__ __launch_bounds__(256) void pack_scales_kernel(const uint16_t* __restrict__ canon_s,
                                                          uint16_t* __restrict__ packed_s,
                                                          int64_t n, int64_t k, int64_t batch,
                                                          int pairing) {
  const int64_t groups = k / kGroup;
  const int64_t total = batch * n * groups;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    // destination order (mat, p, g, quad, m, i)
    const int i = (int)(idx & 3);
    const int m = (int)((idx >> 2) & 1);
    const int quad = (int)((idx >> 3) & 3);
    const int64_t rest = idx >> 5;  // (mat, p, g)
    const int64_t g = rest % groups;
    const int64_t pm = rest / groups;
    const int64_t mat = pm / (n / 32);
    const int64_t p = pm % (n / 32);
    const int64_t row = member_row0(p, m, n, pairing) + 4 * quad + i;
    const uint16_t* srow = canon_s + mat * n * groups + row * groups;
    uint16_t v = srow[g];
    if (scale_is_zero(v)) {  // nearest nonzero scale of the row: earlier groups first
      v = 0x3F80u;           // 1.0 when the whole row is zero
      bool found = false;
      for (int64_t h = g - 1; h >= 0 && !found; --h)
        if (!scale_is_zero(srow[h])) { v = srow[h]; found = true; }
      for (int64_t h = g + 1; h < groups && !found; ++h)
        if (!scale_is_zero(srow[h])) { v = srow[h]; found = true; }
    }
    packed_s[idx] = v;
  }
}

// Group-scale ratios of the int4 prefill kernels, over the packed scales in
// their element order (mat, p, g, quad, m, i): r = s[g-1] / s[g] of the same
// row (32 elements back), correctly rounded in fp32, and 0 for g = 0.  The
// prefill kernels keep each accumulator divided by the current group's scale
// (a <- a * r + the next group's partial sums) and multiply by the last
// group's scale at the end.  Packed scales are never zero (see above), but a
// ratio, or the running sum it multiplies, can still leave the fp32 range
// when a row's scales spread widely (a group of 2^-100 after one of 2^100):
// pack_exact_flag_kernel marks such matrices for the exact-scaling path.
__global__ __launch_bounds__(256) void pack_ratio_kernel(const uint16_t* __restrict__ packed_s,
                                                         float* __restrict__ ratios, int64_t groups,
                                                         int64_t total) {
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = (idx >> 5) % groups;
    float r = 0.0f;
    if (g > 0) r = bf16_bits_to_float(packed_s[idx - 32]) / bf16_bits_to_float(packed_s[idx]);
    ratios[idx] = r;
  }
}

// MXFP4 (E2M1 codes, one E8M0 scale per 32 K; the reference checkpoint
// format, runtime/dsv4_direct/moe_forward.py:126-155).  Same tile geometry
// and pair interleave as the int4 layout; inside a tile lane L's dword d is
// the 4 checkpoint bytes of row L%16, k0 = 128g + 32d + 8*(L/16) .. k0+7
// (low nibble = even k), which is the byte order v_cvt_scalef32_pk_bf16_fp4
// consumes.  Scales: 128 bytes per (pair, group), byte (r16*2 + m)*4 + d
// holds the E8M0 scale of row r16 of member m for k in [128g + 32d, +32), so
// one 8-byte load gives a lane both members' four scales.
__global__ __launch_bounds__(256) void pack_mxfp4_kernel(const uint8_t* __restrict__ canon,
                                                         uint8_t* __restrict__ packed, int64_t n,
                                                         int64_t k, int64_t batch, int pairing) {
  const int64_t groups = k / kGroup;
  const int64_t tiles_per_mat = (n / 16) * groups;
  const int64_t total = batch * tiles_per_mat * 64;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const int64_t tile = idx >> 6;  // destination tile order: (mat, p, g, m)
    const int64_t mat = tile / tiles_per_mat;
    const int64_t tin = tile % tiles_per_mat;
    const int m = (int)(tin & 1);
    const int64_t g = (tin >> 1) % groups;
    const int64_t p = (tin >> 1) / groups;
    const int64_t row = member_row0(p, m, n, pairing) + (lane & 15);
    const uint8_t* src_row = canon + mat * n * (k / 2) + row * (k / 2);
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      out[d] = *reinterpret_cast<const uint32_t*>(src_row + (g * kGroup + 32 * d + 8 * (lane >> 4)) / 2);
    *reinterpret_cast<u32x4*>(packed + mat * n * (k / 2) + tin * kTileBytes + lane * 16) = out;
  }
}

// MXFP4 weights for the W4A8 kernels (block-scaled fp8 x fp4 MFMA): the same
// tile geometry, pair interleave and scale layout, but inside a tile lane L
// holds the 16 checkpoint bytes of row L%16 for k = 128g + 32*(L/16) .. +31:
// 32 E2M1 codes of one scale group, the MFMA's fp4 A operand as is.
__global__ __launch_bounds__(256) void pack_mxfp4_a8_kernel(const uint8_t* __restrict__ canon,
                                                            uint8_t* __restrict__ packed, int64_t n,
                                                            int64_t k, int64_t batch, int pairing) {
  const int64_t groups = k / kGroup;
  const int64_t tiles_per_mat = (n / 16) * groups;
  const int64_t total = batch * tiles_per_mat * 64;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const int64_t tile = idx >> 6;  // destination tile order: (mat, p, g, m)
    const int64_t mat = tile / tiles_per_mat;
    const int64_t tin = tile % tiles_per_mat;
    const int m = (int)(tin & 1);
    const int64_t g = (tin >> 1) % groups;
    const int64_t p = (tin >> 1) / groups;
    const int64_t row = member_row0(p, m, n, pairing) + (lane & 15);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(canon + mat * n * (k / 2) + row * (k / 2) +
                                                            (g * kGroup + 32 * (lane >> 4)) / 2);
    const u32x4 out = {src[0], src[1], src[2], src[3]};
    *reinterpret_cast<u32x4*>(packed + mat * n * (k / 2) + tin * kTileBytes + lane * 16) = out;
  }
}

__global__ __launch_bounds__(256) void pack_e8m0_kernel(const uint8_t* __restrict__ canon_s,
                                                        uint8_t* __restrict__ packed_s, int64_t n,
                                                        int64_t k, int64_t batch, int pairing) {
  const int64_t groups = k / kGroup;
  const int64_t total = batch * n * (k / 32);
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    // destination order (mat, p, g, r16, m, d)
    const int d = (int)(idx & 3);
    const int m = (int)((idx >> 2) & 1);
    const int r16 = (int)((idx >> 3) & 15);
    const int64_t rest = idx >> 7;  // (mat, p, g)
    const int64_t g = rest % groups;
    const int64_t pm = rest / groups;
    const int64_t mat = pm / (n / 32);
    const int64_t p = pm % (n / 32);
    const int64_t row = member_row0(p, m, n, pairing) + r16;
    packed_s[idx] = canon_s[mat * n * (k / 32) + row * (k / 32) + 4 * g + d];
  }
}

}  // namespace dsv4

using namespace dsv4;

int dsv4_launch_pack_mxfp4(const uint8_t* canon, const uint8_t* canon_scales, int64_t batch, int64_t n,
                           int64_t k, int pairing, uint8_t* packed, uint8_t* packed_scales,
                           hipStream_t stream) {
  const int64_t work = batch * (n / 16) * (k / kGroup) * 64;
  const int64_t blocks = (work + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 65535 * 16 ? blocks : 65535 * 16);
  if (work > 0) {
    hipLaunchKernelGGL(pack_mxfp4_kernel, dim3(grid), dim3(256), 0, stream, canon, packed, n, k, batch, pairing);
    DSV4_CHECK_LAUNCH("pack_mxfp4_kernel");
  }
  const int64_t swork = batch * n * (k / 32);
  const int64_t sblocks = (swork + 255) / 256;
  const unsigned sgrid = (unsigned)(sblocks < 65535 * 16 ? sblocks : 65535 * 16);
  if (swork > 0) {
    hipLaunchKernelGGL(pack_e8m0_kernel, dim3(sgrid), dim3(256), 0, stream, canon_scales, packed_scales, n, k,
                       batch, pairing);
    DSV4_CHECK_LAUNCH("pack_e8m0_kernel");
  }
  return DSV4MOE_OK;
}

int dsv4_launch_pack_mxfp4_a8(const uint8_t* canon, const uint8_t* canon_scales, int64_t batch, int64_t n,
                              int64_t k, int pairing, uint8_t* packed, uint8_t* packed_scales,
                              hipStream_t stream) {
  const int64_t work = batch * (n / 16) * (k / kGroup) * 64;
  const int64_t blocks = (work + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 65535 * 16 ? blocks : 65535 * 16);
  if (work > 0) {
    hipLaunchKernelGGL(pack_mxfp4_a8_kernel, dim3(grid), dim3(256), 0, stream, canon, packed, n, k, batch,
                       pairing);
    DSV4_CHECK_LAUNCH("pack_mxfp4_a8_kernel");
  }
  const int64_t swork = batch * n * (k / 32);
  const int64_t sblocks = (swork + 255) / 256;
  const unsigned sgrid = (unsigned)(sblocks < 65535 * 16 ? sblocks : 65535 * 16);
  if (swork > 0) {
    hipLaunchKernelGGL(pack_e8m0_kernel, dim3(sgrid), dim3(256), 0, stream, canon_scales, packed_scales, n, k,
                       batch, pairing);
    DSV4_CHECK_LAUNCH("pack_e8m0_kernel");
  }
  return DSV4MOE_OK;
}

// A matrix (one expert) needs the exact-scaling prefill path when one of its
// rows has a running-sum amplification max_g (s[0] + ... + s[g]) / s[g] above
// 2^64: the running sum after group g holds the scaled partial sums so far
// divided by s[g], so with the amplification bounded by 2^64 it stays finite
// while the partial sums stay below ~2^64 (activations up to ~2^50).  One
// thread per row scans its groups; a marked matrix gets 1.0 in its ratio
// element 0 (a group-0 ratio, 0 otherwise and multiplied by a zero
// accumulator, so the mark changes no product), and element 1 of the first
// matrix of the call (also a group-0 ratio) becomes 1.0 when any matrix of
// the call is marked, so the exact kernel's workgroups can leave after one
// load when none is.  Written after pack_ratio_kernel on the same stream;
// several threads may write the same 1.0.
constexpr float kExactAmplification = 18446744073709551616.0f;  // 2^64

__global__ __launch_bounds__(256) void pack_exact_flag_kernel(const uint16_t* __restrict__ packed_s,
                                                              float* __restrict__ ratios, int64_t n,
                                                              int64_t groups, int64_t batch) {
  const int64_t per_mat = n;  // rows
  const int64_t total = batch * per_mat;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t mat = idx / per_mat;
    const int64_t rin = idx % per_mat;
    const int64_t pair = rin / 32;
    const int64_t o = rin % 32;  // element of the row inside a (pair, group) block
    const uint16_t* base = packed_s + mat * n * groups + pair * groups * 32 + o;
    float sum = 0.0f, amp = 0.0f;
    for (int64_t g = 0; g < groups; ++g) {
      const float sg = fabsf(bf16_bits_to_float(base[g * 32]));
      sum += sg;
      amp = fmaxf(amp, sum / sg);  // inf or NaN compare as above the bound below
    }
    if (!(amp <= kExactAmplification)) {
      ratios[mat * n * groups] = 1.0f;
      ratios[1] = 1.0f;  // the stack holds a marked matrix (element 1: another group-0 ratio)
    }
  }
}

int dsv4_launch_pack_ratios(const uint16_t* packed_scales, int64_t batch, int64_t n, int64_t k, float* ratios,
                            hipStream_t stream) {
  const int64_t total = batch * n * (k / kGroup);
  const int64_t blocks = (total + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 65535 * 16 ? blocks : 65535 * 16);
  if (total > 0) {
    hipLaunchKernelGGL(pack_ratio_kernel, dim3(grid), dim3(256), 0, stream, packed_scales, ratios, k / kGroup,
                       total);
    DSV4_CHECK_LAUNCH("pack_ratio_kernel");
    const int64_t rows = batch * n;
    const int64_t fblocks = (rows + 255) / 256;
    hipLaunchKernelGGL(pack_exact_flag_kernel, dim3((unsigned)(fblocks < 65535 * 16 ? fblocks : 65535 * 16)),
                       dim3(256), 0, stream, packed_scales, ratios, n, k / kGroup, batch);
    DSV4_CHECK_LAUNCH("pack_exact_flag_kernel");
  }
  return DSV4MOE_OK;
}

int dsv4_launch_pack(const uint8_t* canon, const uint16_t* canon_scales, int64_t batch, int64_t n,
                     int64_t k, int pairing, uint8_t* packed, uint16_t* packed_scales,
                     hipStream_t stream) {
  const int64_t work = batch * (n / 16) * (k / kGroup) * 64;
  const int64_t blocks = (work + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 65535 * 16 ? blocks : 65535 * 16);
  if (work > 0) {
    hipLaunchKernelGGL(pack_int4_kernel, dim3(grid), dim3(256), 0, stream, canon, canon_scales, packed,
                       n, k, batch, pairing);
    DSV4_CHECK_LAUNCH("pack_int4_kernel");
  }
  const int64_t swork = batch * n * (k / kGroup);
  const int64_t sblocks = (swork + 255) / 256;
  const unsigned sgrid = (unsigned)(sblocks < 65535 * 16 ? sblocks : 65535 * 16);
  if (swork > 0) {
    hipLaunchKernelGGL(pack_scales_kernel, dim3(sgrid), dim3(256), 0, stream, canon_scales,
                       packed_scales, n, k, batch, pairing);
    DSV4_CHECK_LAUNCH("pack_scales_kernel");
  }
  return DSV4MOE_OK;
}
