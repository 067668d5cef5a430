// The alignment kernels: one workgroup running align_block (align_impl.h) for
// few assignments, and a two-launch split over chunks of the flat ids for many:
//   align_count_kernel  workgroup c < chunks counts its chunk of ids into
//                       counts[c][experts] and flags an out-of-range id in
//                       bad[c]; workgroups past the chunks sum activation rows
//                       when a row-sum target is given;
//   align_place_kernel  workgroup c sums the counts of every chunk (totals)
//                       and of the chunks before its own (its starting
//                       cursors), runs the padded scan, writes its share of
//                       expert_ids and sentinels, and scatters its chunk.
// The scratch `counts` holds [chunks][experts] then [chunks] int32.  Each
// workgroup's result depends only on the ids, so the layout is the one the
// single workgroup writes, whatever the scheduling.
#include <algorithm>

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

__global__ __launch_bounds__(kAlignThreads) void align_count_kernel(
    const int32_t* __restrict__ ids, int64_t assignments, int experts, int64_t chunk, int chunks,
    int32_t* __restrict__ counts, ActPrep prep, int64_t tokens) {
  __shared__ int s_count[kAlignMaxExperts];
  __shared__ int s_bad;
  const int c = blockIdx.x;
  if (c < chunks) {
    const int64_t begin = (int64_t)c * chunk;
    align_histogram(s_count, &s_bad, ids, begin, std::min<int64_t>(begin + chunk, assignments), experts);
    for (int e = threadIdx.x; e < experts; e += kAlignThreads) counts[(int64_t)c * experts + e] = s_count[e];
    if (threadIdx.x == 0) counts[(int64_t)chunks * experts + c] = s_bad;
    return;
  }
  act_prep_part(prep, tokens, c - chunks, (int)gridDim.x - chunks);
}

__global__ __launch_bounds__(kAlignThreads) void align_place_kernel(
    const int32_t* __restrict__ ids, int64_t assignments, int experts, int expert_bits, int block_size,
    int64_t chunk, int chunks, const int32_t* __restrict__ counts, int32_t* __restrict__ sorted_ids,
    int64_t capacity, int32_t* __restrict__ expert_ids, int64_t num_blocks, int32_t* __restrict__ ntpp) {
  __shared__ AlignShared sh;
  const int tid = threadIdx.x;
  const int c = blockIdx.x;
  int bad = 0;
  for (int j = tid; j < chunks; j += kAlignThreads) bad |= counts[(int64_t)chunks * experts + j];
  if (__syncthreads_or(bad)) {
    // Contract violation: report through the padded total, touch nothing else.
    if (c == 0 && tid == 0) ntpp[0] = -1;
    return;
  }
  int before = 0;
  if (tid < experts) {
    int total = 0;
    for (int j = 0; j < chunks; ++j) {
      const int v = counts[(int64_t)j * experts + tid];
      before += j < c ? v : 0;
      total += v;
    }
    sh.count[tid] = total;
  }
  __syncthreads();
  align_scan(sh, experts, block_size, (int32_t)assignments, sorted_ids, capacity, expert_ids, num_blocks, ntpp, c,
             chunks);
  if (tid < experts) sh.cursor[tid] += before;
  __syncthreads();
  const int64_t begin = (int64_t)c * chunk;
  align_scatter(sh, ids, begin, std::min<int64_t>(begin + chunk, assignments), experts, expert_bits, sorted_ids);
}

}  // namespace dsv4

using namespace dsv4;

static int expert_bits_of(int experts) {
  int bits = 0;
  while ((1 << bits) < experts) ++bits;
  return bits;
}

// Chunking of the two-launch alignment: chunks of a multiple of 1024 flat ids,
// at least kAlignChunk of them, at most kAlignMaxChunks chunks.
void dsv4_align_chunks(int64_t assignments, int64_t* chunk, int* chunks) {
  int64_t n = std::min<int64_t>((assignments + kAlignChunk - 1) / kAlignChunk, kAlignMaxChunks);
  n = std::max<int64_t>(n, 1);
  int64_t c = (assignments + n - 1) / n;
  c = (c + kAlignThreads - 1) / kAlignThreads * kAlignThreads;
  *chunk = c;
  *chunks = (int)((assignments + c - 1) / c);
}

size_t dsv4_align_scratch_bytes(int64_t assignments, int32_t experts) {
  int64_t chunk;
  int chunks;
  dsv4_align_chunks(assignments, &chunk, &chunks);
  return sizeof(int32_t) * (size_t)chunks * (size_t)(experts + 1);
}

// Two-launch alignment [+ the activation work of `prep` beside the counting].
int dsv4_launch_align_multi(const int32_t* ids, int64_t assignments, int32_t experts, int32_t block_size,
                            int32_t* sorted_ids, int64_t capacity, int32_t* expert_ids, int64_t num_blocks,
                            int32_t* ntpp, int32_t* scratch, const ActPrep& prep, int64_t tokens,
                            hipStream_t stream) {
  int64_t chunk;
  int chunks;
  dsv4_align_chunks(assignments, &chunk, &chunks);
  const int sum_wgs = (int)act_prep_workgroups(prep, tokens, kAlignSumWorkgroups);
  hipLaunchKernelGGL(align_count_kernel, dim3((unsigned)(chunks + sum_wgs)), dim3(kAlignThreads), 0, stream, ids,
                     assignments, experts, chunk, chunks, scratch, prep, tokens);
  DSV4_CHECK_LAUNCH("align_count_kernel");
  hipLaunchKernelGGL(align_place_kernel, dim3((unsigned)chunks), dim3(kAlignThreads), 0, stream, ids, assignments,
                     experts, expert_bits_of(experts), block_size, chunk, chunks, scratch, sorted_ids, capacity,
                     expert_ids, num_blocks, ntpp);
  DSV4_CHECK_LAUNCH("align_place_kernel");
  return DSV4MOE_OK;
}

int dsv4_launch_align(const int32_t* ids, int64_t assignments, int32_t experts,
                      int32_t block_size, int32_t* sorted_ids, int64_t capacity,
                      int32_t* expert_ids, int64_t num_blocks, int32_t* ntpp,
                      hipStream_t stream) {
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(kAlignThreads), 0, stream, ids, assignments,
                     experts, expert_bits_of(experts), block_size, sorted_ids, capacity, expert_ids, num_blocks, ntpp);
  DSV4_CHECK_LAUNCH("align_kernel");
  return DSV4MOE_OK;
}
