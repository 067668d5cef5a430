// Router logits = x . Wg^T on bf16 MFMA with fp32 accumulation.
// Restates F.linear(x.float(), weight.float()) of the learned gate
// (runtime/dsv4_direct/moe_forward.py:80, reference/inference/model.py:565):
// bf16 x bf16 products are exact in fp32, so only the summation order differs.
// One wavefront computes a 16 (experts) x 16 (tokens) tile over all of K.
#include "common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

__global__ __launch_bounds__(256) void gate_logits_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wg,
                                                          int64_t tokens, int hidden, int experts,
                                                          float* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * 16;
  const int e0 = blockIdx.y * 64 + wave * 16;
  if (e0 >= experts) return;
  const int e = e0 + (lane & 15);
  const int64_t t = t0 + (lane & 15);
  const int koff = 8 * (lane >> 4);
  const bool e_ok = e < experts;
  const bool t_ok = t < tokens;
  const uint16_t* arow = wg + (int64_t)(e_ok ? e : 0) * hidden + koff;
  const uint16_t* brow = x + (t_ok ? t : 0) * hidden + koff;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int kk = 0; kk < hidden; kk += 32) {
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (e_ok) a = load16(arow + kk);
    if (t_ok) b = load16(brow + kk);
    acc = mfma_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc);
  }
  if (t_ok) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int er = e0 + 4 * (lane >> 4) + i;
      if (er < experts) logits[t * experts + er] = acc[i];
    }
  }
}

}  // namespace dsv4

using namespace dsv4;

int dsv4_launch_gate_logits(const uint16_t* x, const uint16_t* wg, int64_t tokens, int hidden,
                            int experts, float* logits, hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  const dim3 grid((unsigned)((tokens + 15) / 16), (unsigned)((experts + 63) / 64));
  hipLaunchKernelGGL(gate_logits_kernel, grid, dim3(256), 0, stream, x, wg, tokens, hidden,
                     experts, logits);
  DSV4_CHECK_LAUNCH("gate_logits_kernel");
  return DSV4MOE_OK;
}
