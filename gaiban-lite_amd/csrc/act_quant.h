// Per-row e4m3 activation quantisation of the W4A8 paths, as a device
// function of one wavefront, shared by the quantiser kernel (experts_fp8.hip)
// and the prologue launches that run it beside the alignment (route.hip,
// align.hip).
//
// Restates the activation quantisation of vLLM's _fused_marlin_moe with
// input_dtype = float8_e4m3fn (runtime/dsv4_direct/moe_runtime.py:207-235):
// s = max(amax, 1e-12) / 448 and q = e4m3(clamp(v / s, -448, 448)), round to
// nearest even, saturating.
#pragma once

#include "common.h"

namespace dsv4 {

// Row `row` of x [rows][k] (k % 512 == 0) by the calling wavefront: writes the
// row scale and the codes, in one of two byte orders:
//  * NATURAL = false: each 128-K group in the order of the int4 W4A8 kernels'
//    nibble spread (32 bytes per lane group j, dword pair d holding K
//    32d + 8j + {0,4,1,5,2,6,3,7}), plus per group the fp32 sum of its 128
//    decoded e4m3 values (each lane adds its 8 values in K order, then a
//    fixed xor tree over 16 lanes);
//  * NATURAL = true: K order, no group sums (the MXFP4 W4A8 kernels' operand,
//    whose K order is the checkpoint's).
template <bool NATURAL>
__device__ __forceinline__ void act_quant_row(const uint16_t* __restrict__ x, int64_t row, int k,
                                              uint8_t* __restrict__ q, float* __restrict__ scale,
                                              float* __restrict__ gsum) {
  const int lane = threadIdx.x & 63;
  const uint16_t* src = x + row * k;
  const int iters = k / 512;
  float amax = 0.0f;
  for (int i = 0; i < iters; ++i) {
    const u32x4 v = load16(src + (lane + 64 * i) * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      amax = fmaxf(amax, fabsf(__uint_as_float(v[e] << 16)));
      amax = fmaxf(amax, fabsf(__uint_as_float(v[e] & 0xFFFF0000u)));
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float s = fmaxf(amax, 1e-12f) / 448.0f;
  if (lane == 0) scale[row] = s;

  const int groups = k / 128;
  for (int i = 0; i < iters; ++i) {
    const int o = lane + 64 * i;  // octet: K 8o .. 8o+7
    const u32x4 v = load16(src + o * 8);
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = __uint_as_float(v[e] << 16);
      f[2 * e + 1] = __uint_as_float(v[e] & 0xFFFF0000u);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(f[e] / s, -448.0f), 448.0f);
    if constexpr (NATURAL) {
      int lo = 0, hi = 0;
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], lo, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], lo, true);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4], f[5], hi, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6], f[7], hi, true);
      *reinterpret_cast<u32x2*>(q + row * k + o * 8) = u32x2{(uint32_t)lo, (uint32_t)hi};
      continue;
    }
    // output byte b holds K offset {0,4,1,5,2,6,3,7}[b]
    int lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[4], lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[1], f[5], lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[6], hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[3], f[7], hi, true);
    // decoded values in K order for the group sum
    float dq[8];
    dq[0] = __builtin_amdgcn_cvt_f32_fp8(lo, 0);
    dq[4] = __builtin_amdgcn_cvt_f32_fp8(lo, 1);
    dq[1] = __builtin_amdgcn_cvt_f32_fp8(lo, 2);
    dq[5] = __builtin_amdgcn_cvt_f32_fp8(lo, 3);
    dq[2] = __builtin_amdgcn_cvt_f32_fp8(hi, 0);
    dq[6] = __builtin_amdgcn_cvt_f32_fp8(hi, 1);
    dq[3] = __builtin_amdgcn_cvt_f32_fp8(hi, 2);
    dq[7] = __builtin_amdgcn_cvt_f32_fp8(hi, 3);
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += dq[e];
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    sum += __shfl_xor(sum, 8, 64);
    const int g = o >> 4;
    const int lo16 = o & 15;
    const int d = lo16 >> 2;
    const int j = lo16 & 3;
    *reinterpret_cast<u32x2*>(q + row * k + g * 128 + j * 32 + d * 8) = u32x2{(uint32_t)lo, (uint32_t)hi};
    if ((lane & 15) == 0) gsum[row * groups + g] = sum;
  }
}

// What the extra workgroups of a prologue launch (route.hip, align.hip) do
// with the activations beside the alignment.
enum ActPrepMode : int {
  kPrepNone = 0,
  kPrepRowSums = 1,      // 64-column row sums of x (the W4A16 decode kernels)
  kPrepQuantInt4 = 2,    // act_quant_row<false> (the int4 W4A8 kernels)
  kPrepQuantNatural = 3, // act_quant_row<true> (the MXFP4 W4A8 kernels)
  kPrepRowNc = 4         // per 128-column group, -136 * (sum of 64 + sum of 64) (the W4A16 prefill kernels)
};

struct ActPrep {
  int mode;
  const uint16_t* x;  // [tokens][hidden]
  int hidden;
  float* sums;        // row sums [tokens][hidden / 64], or per-group values [tokens][hidden / 128]
  uint8_t* q;         // e4m3 codes [tokens][hidden]
  float* qscale;      // [tokens]
};

// The W4A16 experts launcher takes the decode kernels for alignment blocks
// of at most 16 slots (H and I multiples of 512), else the prefill kernels;
// the two read the activation sums in different forms (kPrepRowSums /
// kPrepRowNc), so the producers choose by the same rule.
inline bool w4a16_decode_path(int block_size, int hidden, int inter) {
  return block_size <= 16 && hidden % 512 == 0 && inter % 512 == 0;
}

}  // namespace dsv4
