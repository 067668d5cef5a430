// Checkpoint-format dequantisers to fp32: the host helpers of the reference's
// moe_forward module (runtime/dsv4_direct/moe_forward.py:115-176) as
// HBM-bound streaming kernels.  Not on the layer's hot path (the expert and
// linear kernels dequantise in registers); these serve callers that want the
// dense fp32 weight, such as a dense reference executor.
//
//   decode_e8m0:   byte c -> 2^(c - 127) as fp32; c = 0 gives the subnormal
//                  2^-127 and c = 255 NaN, as torch's float8_e8m0fnu -> float.
//   mxfp4:         E2M1 codes (low nibble = even K) times one fp32 scale per
//                  32 K, one fp32 product per weight.
//   fp8_block:     a [rows, cols] weight (E4M3FN bytes, bf16, fp16 or fp32)
//                  times one fp32 scale per 128 x 128 block.
// The scales arrive decoded (fp32): the products are then the same IEEE fp32
// multiplications the reference's torch expression performs.
#include "common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

__device__ __forceinline__ float e8m0_to_float(uint32_t c) {
  const uint32_t bits = c == 0 ? 0x00400000u : (c == 255 ? 0x7FC00000u : c << 23);
  return __uint_as_float(bits);
}

// E2M1 code (sign, 2 exponent bits, 1 mantissa bit) -> fp32 value.  Code 8
// (negative zero) gives +0, as the reference's value table does.
__device__ __forceinline__ float e2m1_to_float(uint32_t code) {
  const uint32_t e = (code >> 1) & 3u, m = code & 1u;
  const uint32_t mag = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3F000000u : 0u);
  return __uint_as_float(mag | (mag ? (code & 8u) << 28 : 0u));
}

__global__ __launch_bounds__(256) void decode_e8m0_kernel(const uint8_t* __restrict__ codes, int64_t n,
                                                          float* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = e8m0_to_float(codes[i]);
}

// One thread per 32-K group: 16 code bytes in, 32 floats (8 x 16 B) out.
__global__ __launch_bounds__(256) void dequant_mxfp4_kernel(const uint8_t* __restrict__ packed,
                                                            const float* __restrict__ scale, int64_t groups,
                                                            float* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += stride) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(packed + g * 16);
    const float s = scale[g];
    f32x4* dst = reinterpret_cast<f32x4*>(out + g * 32);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t word = w[d];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = e2m1_to_float((word >> (16 * h + 4 * j)) & 0xFu) * s;
        dst[2 * d + h] = v;
      }
    }
  }
}

template <int kDtype>
__device__ __forceinline__ float weight_value(const void* w, int64_t i) {
  if constexpr (kDtype == DSV4MOE_DTYPE_FP8_E4M3) {
    const uint32_t byte = reinterpret_cast<const uint8_t*>(w)[i];
    return __builtin_amdgcn_cvt_f32_fp8((int)byte, 0);
  } else if constexpr (kDtype == DSV4MOE_DTYPE_BF16) {
    return bf16_bits_to_float(reinterpret_cast<const uint16_t*>(w)[i]);
  } else if constexpr (kDtype == DSV4MOE_DTYPE_FP16) {
    return (float)reinterpret_cast<const _Float16*>(w)[i];
  } else {
    return reinterpret_cast<const float*>(w)[i];
  }
}

// One thread per 4 consecutive elements of a row (cols % 4 == 0), or per
// element otherwise; each element times the scale of its 128 x 128 block.
template <int kDtype, int kVec>
__global__ __launch_bounds__(256) void dequant_fp8_block_kernel(const void* __restrict__ w,
                                                                const float* __restrict__ scale, int64_t rows,
                                                                int64_t cols, float* __restrict__ out) {
  const int64_t col_blocks = (cols + 127) / 128;
  const int64_t per_row = cols / kVec;
  const int64_t units = rows * per_row;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += stride) {
    const int64_t r = u / per_row;
    const int64_t c0 = (u - r * per_row) * kVec;
    const float s = scale[(r / 128) * col_blocks + c0 / 128];  // kVec divides 128: one block per unit
    const int64_t i0 = r * cols + c0;
    if constexpr (kVec == 4) {
      f32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = weight_value<kDtype>(w, i0 + j) * s;
      *reinterpret_cast<f32x4*>(out + i0) = v;
    } else {
      out[i0] = weight_value<kDtype>(w, i0) * s;
    }
  }
}

static unsigned stream_grid(int64_t units) {
  const int64_t blocks = (units + 255) / 256;
  return (unsigned)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

}  // namespace dsv4

using namespace dsv4;

int dsv4_launch_decode_e8m0(const uint8_t* codes, int64_t n, float* out, hipStream_t stream) {
  hipLaunchKernelGGL(decode_e8m0_kernel, dim3(stream_grid(n)), dim3(256), 0, stream, codes, n, out);
  DSV4_CHECK_LAUNCH("decode_e8m0_kernel");
  return DSV4MOE_OK;
}

int dsv4_launch_dequant_mxfp4(const uint8_t* packed, const float* scale, int64_t rows, int64_t k, float* out,
                              hipStream_t stream) {
  const int64_t groups = rows * (k / 32);
  hipLaunchKernelGGL(dequant_mxfp4_kernel, dim3(stream_grid(groups)), dim3(256), 0, stream, packed, scale, groups,
                     out);
  DSV4_CHECK_LAUNCH("dequant_mxfp4_kernel");
  return DSV4MOE_OK;
}

template <int kDtype>
static int launch_fp8_block(const void* w, const float* scale, int64_t rows, int64_t cols, float* out,
                            hipStream_t stream) {
  if (cols % 4 == 0) {
    hipLaunchKernelGGL((dequant_fp8_block_kernel<kDtype, 4>), dim3(stream_grid(rows * cols / 4)), dim3(256), 0,
                       stream, w, scale, rows, cols, out);
  } else {
    hipLaunchKernelGGL((dequant_fp8_block_kernel<kDtype, 1>), dim3(stream_grid(rows * cols)), dim3(256), 0,
                       stream, w, scale, rows, cols, out);
  }
  DSV4_CHECK_LAUNCH("dequant_fp8_block_kernel");
  return DSV4MOE_OK;
}

int dsv4_launch_dequant_fp8_block(const void* w, int32_t w_dtype, const float* scale, int64_t rows, int64_t cols,
                                  float* out, hipStream_t stream) {
  switch (w_dtype) {
    case DSV4MOE_DTYPE_FP8_E4M3: return launch_fp8_block<DSV4MOE_DTYPE_FP8_E4M3>(w, scale, rows, cols, out, stream);
    case DSV4MOE_DTYPE_BF16: return launch_fp8_block<DSV4MOE_DTYPE_BF16>(w, scale, rows, cols, out, stream);
    case DSV4MOE_DTYPE_FP16: return launch_fp8_block<DSV4MOE_DTYPE_FP16>(w, scale, rows, cols, out, stream);
    default: return launch_fp8_block<DSV4MOE_DTYPE_FP32>(w, scale, rows, cols, out, stream);
  }
}
