// The alignment kernel: one workgroup running align_block (align_impl.h).
#include "align_impl.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

__global__ __launch_bounds__(kAlignThreads) void align_kernel(
    const int32_t* __restrict__ ids, int64_t assignments, int experts, int expert_bits,
    int block_size, int32_t* __restrict__ sorted_ids, int64_t capacity,
    int32_t* __restrict__ expert_ids, int64_t num_blocks, int32_t* __restrict__ ntpp) {
  align_block(ids, assignments, experts, expert_bits, block_size, sorted_ids, capacity, expert_ids, num_blocks,
              ntpp);
}

}  // namespace dsv4

using namespace dsv4;

int dsv4_launch_align(const int32_t* ids, int64_t assignments, int32_t experts,
                      int32_t block_size, int32_t* sorted_ids, int64_t capacity,
                      int32_t* expert_ids, int64_t num_blocks, int32_t* ntpp,
                      hipStream_t stream) {
  int bits = 0;
  while ((1 << bits) < experts) ++bits;
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(kAlignThreads), 0, stream, ids, assignments,
                     experts, bits, block_size, sorted_ids, capacity, expert_ids, num_blocks, ntpp);
  DSV4_CHECK_LAUNCH("align_kernel");
  return DSV4MOE_OK;
}
