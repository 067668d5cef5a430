// Load-time repack of int4 group-128 weights into the tiled layout that the
// expert kernels stream with one 16-byte load per lane per group.
//
// Checkpoint layout (the convention of runtime/dsv4_direct/moe_forward.py:126-131):
//   canon[n][k/2]: byte b holds k = 2b in its low nibble, k = 2b+1 in its high
//   nibble, two's complement q in [-8, 7]; scales[n][k/128] bf16.
// Tiled layout: tile (s, g) = rows 16s..16s+15, k in [128g, 128g+128), stored
// at byte ((s*G + g) * 1024); inside, lane L (0..63) owns bytes L*16..L*16+15,
// dword d (0..3) of lane L holds row 16s + L%16, k0 = 128g + 32d + 8*(L/16):
// nibble slot j (bits 4j..) = k0+2j and slot 4+j (bits 16+4j..) = k0+2j+1,
// stored offset-binary (q + 8).  Scales: [n/16][k/128][16] bf16.
#include "common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

__global__ __launch_bounds__(256) void pack_int4_kernel(const uint8_t* __restrict__ canon,
                                                        uint8_t* __restrict__ packed,
                                                        int64_t n, int64_t k, int64_t batch) {
  const int64_t groups = k / kGroup;
  const int64_t tiles_per_mat = (n / 16) * groups;
  const int64_t total = batch * tiles_per_mat * 64;  // one thread per (tile, lane)
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const int64_t tile = idx >> 6;
    const int64_t mat = tile / tiles_per_mat;
    const int64_t tin = tile % tiles_per_mat;
    const int64_t strip = tin / groups;
    const int64_t g = tin % groups;
    const int64_t row = strip * 16 + (lane & 15);
    const uint8_t* src_row = canon + mat * n * (k / 2) + row * (k / 2);
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int64_t k0 = g * kGroup + 32 * d + 8 * (lane >> 4);
      const uint32_t src = *reinterpret_cast<const uint32_t*>(src_row + k0 / 2);
      uint32_t w = 0;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t byte = (src >> (8 * m)) & 0xFFu;
        const uint32_t lo = (byte & 0xFu) ^ 0x8u;
        const uint32_t hi = (byte >> 4) ^ 0x8u;
        w |= lo << (4 * m);
        w |= hi << (16 + 4 * m);
      }
      out[d] = w;
    }
    *reinterpret_cast<u32x4*>(packed + mat * n * (k / 2) + tile % tiles_per_mat * kTileBytes +
                              lane * 16) = out;
  }
}

__global__ __launch_bounds__(256) void pack_scales_kernel(const uint16_t* __restrict__ canon_s,
                                                          uint16_t* __restrict__ packed_s,
                                                          int64_t n, int64_t k, int64_t batch) {
  const int64_t groups = k / kGroup;
  const int64_t total = batch * n * groups;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    // destination order [mat][n/16][groups][16]
    const int64_t r16 = idx & 15;
    const int64_t rest = idx >> 4;
    const int64_t g = rest % groups;
    const int64_t strip_all = rest / groups;  // mat * (n/16) + strip
    const int64_t mat = strip_all / (n / 16);
    const int64_t strip = strip_all % (n / 16);
    const int64_t row = strip * 16 + r16;
    packed_s[idx] = canon_s[mat * n * groups + row * groups + g];
  }
}

}  // namespace dsv4

using namespace dsv4;

int dsv4_launch_pack(const uint8_t* canon, const uint16_t* canon_scales, int64_t batch, int64_t n,
                     int64_t k, uint8_t* packed, uint16_t* packed_scales, hipStream_t stream) {
  const int64_t work = batch * (n / 16) * (k / kGroup) * 64;
  const int64_t blocks = (work + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 65535 * 16 ? blocks : 65535 * 16);
  if (work > 0) {
    hipLaunchKernelGGL(pack_int4_kernel, dim3(grid), dim3(256), 0, stream, canon, packed, n, k,
                       batch);
    DSV4_CHECK_LAUNCH("pack_int4_kernel");
  }
  const int64_t swork = batch * n * (k / kGroup);
  const int64_t sblocks = (swork + 255) / 256;
  const unsigned sgrid = (unsigned)(sblocks < 65535 * 16 ? sblocks : 65535 * 16);
  if (swork > 0) {
    hipLaunchKernelGGL(pack_scales_kernel, dim3(sgrid), dim3(256), 0, stream, canon_scales,
                       packed_scales, n, k, batch);
    DSV4_CHECK_LAUNCH("pack_scales_kernel");
  }
  return DSV4MOE_OK;
}
