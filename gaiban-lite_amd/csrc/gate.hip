// Router logits = x . Wg^T on bf16 MFMA with fp32 accumulation.
// Restates F.linear(x.float(), weight.float()) of the learned gate
// (runtime/dsv4_direct/moe_forward.py:80, reference/inference/model.py:565):
// bf16 x bf16 products are exact in fp32, so only the summation order differs.
// Every summation order here is fixed, so the logits of a token do not depend
// on the other tokens of the batch or on the run; they can differ in the last
// bits between batches of up to kGateSplitMaxTokens tokens and larger ones,
// which run the other kernel (as a vendor GEMM changes its algorithm by M).
//
// Two kernels by batch size (Wg is [experts, hidden], experts = 256 at the
// Flash shape: 2 MiB of bf16):
//  * gate_logits_split_kernel (decode, up to kGateSplitMaxTokens tokens, and
//    any shape the tiled kernel does not take): one workgroup of 8
//    wavefronts per 16-expert x 16-token output tile; wavefront w sums K
//    range w of 8 (8 loads of each operand in flight per batch), and
//    the 8 partial tiles are added through LDS in wavefront order.  The
//    weight is streamed once per token tile, by 16 x (T/16) workgroups at a
//    time: bound by the bytes in flight per CU, not by the MFMAs.
//  * gate_logits_tile_kernel (prefill): 64 tokens x 64 experts per workgroup,
//    K in chunks of 128 copied into LDS by buffer_load ... lds (double
//    buffered, XOR-swizzled rows for conflict-free ds_read_b128); wavefront w
//    owns experts 16w .. 16w+15 of the tile against all 64 tokens, sharing
//    each weight fragment over 4 token fragments.
#include "common.h"
#include "experts_common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

constexpr int kGateSplitWaves = 8;
constexpr int kGateSplitBatch = 8;          // K steps (32 K each) loaded ahead per batch
constexpr int64_t kGateSplitMaxTokens = 512;

__global__ __launch_bounds__(64 * kGateSplitWaves) void gate_logits_split_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, int64_t tokens, int hidden, int experts,
    float* __restrict__ logits) {
  __shared__ f32x4 part[kGateSplitWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * 16;
  const int e0 = blockIdx.y * 16;
  const int e = e0 + (lane & 15);
  const int64_t t = t0 + (lane & 15);
  const bool e_ok = e < experts;
  const bool t_ok = t < tokens;
  // K steps of 32 (hidden % 32 == 0): wavefront w takes steps [w*per, min(steps, (w+1)*per))
  const int steps = hidden / 32;
  const int per = (steps + kGateSplitWaves - 1) / kGateSplitWaves;
  const int s_begin = wave * per;
  const int s_end = min(steps, s_begin + per);
  const int koff = 8 * (lane >> 4);
  const uint16_t* arow = wg + (int64_t)(e_ok ? e : 0) * hidden + koff;
  const uint16_t* brow = x + (t_ok ? t : 0) * hidden + koff;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = s_begin; s0 < s_end; s0 += kGateSplitBatch) {
    u32x4 a[kGateSplitBatch], b[kGateSplitBatch];
#pragma unroll
    for (int j = 0; j < kGateSplitBatch; ++j) {
      const bool in = s0 + j < s_end;
      a[j] = e_ok && in ? load16(arow + (s0 + j) * 32) : u32x4{0u, 0u, 0u, 0u};
      b[j] = t_ok && in ? load16(brow + (s0 + j) * 32) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < kGateSplitBatch; ++j)
      acc = mfma_bf16(__builtin_bit_cast(bf16x8, a[j]), __builtin_bit_cast(bf16x8, b[j]), acc);
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4 s = part[0][lane];
#pragma unroll
    for (int w = 1; w < kGateSplitWaves; ++w) {
      const f32x4 v = part[w][lane];
      s[0] += v[0]; s[1] += v[1]; s[2] += v[2]; s[3] += v[3];
    }
    if (t_ok) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int er = e0 + 4 * (lane >> 4) + i;
        if (er < experts) logits[t * experts + er] = s[i];
      }
    }
  }
}

constexpr int kGateTile = 64;   // tokens and experts per workgroup
constexpr int kGateChunk = 128; // K per LDS stage

__global__ __launch_bounds__(256, 2) void gate_logits_tile_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ wg,
                                                                  int64_t tokens, int hidden, int experts,
                                                                  float* __restrict__ logits) {
  // row r of a stage: 16 parts of 16 B (8 K each); part q stored at q ^ (r & 15)
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kGateTile * 256];
  __shared__ __attribute__((aligned(16))) uint8_t ws[2][kGateTile * 256];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * kGateTile;
  const int e0 = blockIdx.y * kGateTile;
  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)(tokens * hidden * 2), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wg, (short)0, (int)((int64_t)experts * hidden * 2), kRsrcFlags);
  // copy q (0..3) of wave w fills rows 16w + 4q + lane/16 of both tiles
  uint32_t xoff[4], woff[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 16 * wave + 4 * q + (lane >> 4);
    const int part = (lane & 15) ^ (row & 15);
    const int64_t t = t0 + row;
    const int e = e0 + row;
    xoff[q] = t < tokens ? (uint32_t)(t * hidden * 2 + part * 16) : kOobOffset;
    woff[q] = e < experts ? (uint32_t)((int64_t)e * hidden * 2 + part * 16) : kOobOffset;
  }
  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][16 * wave * 256]));
  const uint32_t ws_lds = __builtin_amdgcn_readfirstlane(lds_addr(&ws[0][16 * wave * 256]));
  auto issue = [&](int c, int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lds_copy16(x_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + q * 1024, xoff[q], c * kGateChunk * 2);
      lds_copy16(w_rsrc, ws_lds + buf * (uint32_t)sizeof(ws[0]) + q * 1024, woff[q], c * kGateChunk * 2);
    }
  };
  const int sw = lane & 15;
  f32x4 acc[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int chunks = hidden / kGateChunk;
  auto step = [&](int c, int u) {
    if (c + 1 < chunks) issue(c + 1, u ^ 1);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int part = ((4 * d + (lane >> 4)) ^ sw) * 16;
      const bf16x8 a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&ws[u][(16 * wave + sw) * 256 + part]));
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xs[u][(16 * ct + sw) * 256 + part]));
        acc[ct] = mfma_bf16(a, b, acc[ct]);
      }
    }
    lds_dma_wait_all();
    __syncthreads();
  };
  issue(0, 0);
  lds_dma_wait_all();
  __syncthreads();
  for (int c = 0; c < chunks; c += 2) {
    step(c, 0);
    if (c + 1 < chunks) step(c + 1, 1);
  }
  // acc[ct] lane l: expert e0 + 16w + 4(l/16) + i, token t0 + 16ct + l%16
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int64_t t = t0 + 16 * ct + sw;
    if (t >= tokens) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + 16 * wave + 4 * (lane >> 4) + i;
      if (e < experts) logits[t * experts + e] = acc[ct][i];
    }
  }
}

}  // namespace dsv4

using namespace dsv4;

int dsv4_launch_gate_logits(const uint16_t* x, const uint16_t* wg, int64_t tokens, int hidden,
                            int experts, float* logits, hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  const bool tiled = tokens > kGateSplitMaxTokens && hidden % kGateChunk == 0 &&
                     tokens * hidden * 2 < 0x7FFFFFFFLL && (int64_t)experts * hidden * 2 < 0x7FFFFFFFLL;
  if (!tiled) {
    const dim3 grid((unsigned)((tokens + 15) / 16), (unsigned)((experts + 15) / 16));
    hipLaunchKernelGGL(gate_logits_split_kernel, grid, dim3(64 * kGateSplitWaves), 0, stream, x, wg, tokens, hidden,
                       experts, logits);
    DSV4_CHECK_LAUNCH("gate_logits_split_kernel");
  } else {
    const dim3 grid((unsigned)((tokens + kGateTile - 1) / kGateTile), (unsigned)((experts + kGateTile - 1) / kGateTile));
    hipLaunchKernelGGL(gate_logits_tile_kernel, grid, dim3(256), 0, stream, x, wg, tokens, hidden, experts, logits);
    DSV4_CHECK_LAUNCH("gate_logits_tile_kernel");
  }
  return DSV4MOE_OK;
}
