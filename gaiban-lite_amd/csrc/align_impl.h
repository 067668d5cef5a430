// Deterministic expert alignment (expert histogram, padded prefix, stable
// permutation) in one workgroup.  Restates deterministic_moe_align_block_size
// (runtime/dsv4_direct/deterministic_moe_align.py:93-133):
//   * sorted_token_ids lists, expert by expert, the flat indices t*k+j routed to
//     that expert in ascending order, each expert's run padded to a multiple of
//     block_size with the sentinel T*k;
//   * expert_ids[b] = expert owning padded position b*block_size, -1 past the
//     padded total; num_tokens_post_padded = padded total.
// Stability without sorting: flat indices are processed in ascending chunks of
// 1024; inside a wavefront the rank among equal experts is a popcount over a
// ballot-built equality mask, across the 16 wavefronts of a chunk it is an LDS
// prefix of per-wave counts, and across chunks a running per-expert cursor.
#pragma once

#include "common.h"

namespace dsv4 {

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignMaxExperts = 1024;

// The whole alignment, run by one workgroup of kAlignThreads threads (every
// thread must call it).  `ids` may have been written by this workgroup just
// before (after a barrier).
__device__ __forceinline__ void align_block(const int32_t* __restrict__ ids, int64_t assignments, int experts,
                                            int expert_bits, int block_size, int32_t* __restrict__ sorted_ids,
                                            int64_t capacity, int32_t* __restrict__ expert_ids, int64_t num_blocks,
                                            int32_t* __restrict__ ntpp) {
  __shared__ int s_count[kAlignMaxExperts];
  __shared__ int s_pad_end[kAlignMaxExperts];
  __shared__ int s_cursor[kAlignMaxExperts];
  __shared__ uint16_t s_wave_cnt[kAlignWaves][kAlignMaxExperts];
  __shared__ int s_bad;
  __shared__ int s_scan[kAlignWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int32_t sentinel = (int32_t)assignments;

  for (int e = tid; e < experts; e += kAlignThreads) s_count[e] = 0;
  if (tid == 0) s_bad = 0;
  __syncthreads();

  // 1. histogram
  for (int64_t i = tid; i < assignments; i += kAlignThreads) {
    const int e = ids[i];
    if (e < 0 || e >= experts) {
      s_bad = 1;
    } else {
      atomicAdd(&s_count[e], 1);
    }
  }
  __syncthreads();
  if (s_bad) {
    // Contract violation: report through the padded total, touch nothing else.
    if (tid == 0) ntpp[0] = -1;
    return;
  }

  // 2. exclusive scan of padded counts over experts (experts <= 1024 = threads)
  int padded = 0;
  if (tid < experts) padded = (s_count[tid] + block_size - 1) / block_size * block_size;
  int incl = padded;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) s_scan[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int v = lane < kAlignWaves ? s_scan[lane] : 0;
    int w = v;
#pragma unroll
    for (int off = 1; off < kAlignWaves; off <<= 1) {
      const int u = __shfl_up(w, off, 64);
      if (lane >= off) w += u;
    }
    if (lane < kAlignWaves) s_scan[lane] = w - v;  // exclusive per-wave base
  }
  __syncthreads();
  const int pad_end = incl + s_scan[wave];
  if (tid < experts) {
    s_pad_end[tid] = pad_end;
    s_cursor[tid] = pad_end - padded;
  }
  __syncthreads();
  const int total = s_pad_end[experts - 1];

  // 3. per-block expert ids (searchsorted(padded_ends, start, right=True))
  for (int64_t b = tid; b < num_blocks; b += kAlignThreads) {
    const int64_t start = b * block_size;
    int32_t owner = -1;
    if (start < total) {
      int lo = 0, hi = experts;  // first e with pad_end[e] > start
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (s_pad_end[mid] > start) hi = mid; else lo = mid + 1;
      }
      owner = lo;
    }
    expert_ids[b] = owner;
  }
  // 4. sentinels: the tail past the total, and each expert's padding slots
  for (int64_t p = (int64_t)total + tid; p < capacity; p += kAlignThreads) sorted_ids[p] = sentinel;
  for (int e = tid; e < experts; e += kAlignThreads) {
    const int end = s_pad_end[e];
    const int used = (end - ((s_count[e] + block_size - 1) / block_size * block_size)) + s_count[e];
    for (int p = used; p < end; ++p) sorted_ids[p] = sentinel;
  }
  if (tid == 0) ntpp[0] = total;

  // 5. stable scatter
  for (int e = tid; e < experts; e += kAlignThreads)
    for (int w = 0; w < kAlignWaves; ++w) s_wave_cnt[w][e] = 0;
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t base = 0; base < assignments; base += kAlignThreads) {
    const int64_t i = base + tid;
    const bool active = i < assignments;
    const int e = active ? ids[i] : 0;
    uint64_t eq = __ballot(active);
    for (int b = 0; b < expert_bits; ++b) {
      const uint64_t bal = __ballot(active && ((e >> b) & 1));
      eq &= ((e >> b) & 1) ? bal : ~bal;
    }
    const int rank_in_wave = __popcll(eq & lt_mask);
    const bool leader = active && rank_in_wave == 0;
    if (leader) s_wave_cnt[wave][e] = (uint16_t)__popcll(eq);
    __syncthreads();
    if (active) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += s_wave_cnt[w][e];
      sorted_ids[s_cursor[e] + before + rank_in_wave] = (int32_t)i;
    }
    __syncthreads();
    for (int ex = tid; ex < experts; ex += kAlignThreads) {
      int sum = 0;
      for (int w = 0; w < kAlignWaves; ++w) {
        sum += s_wave_cnt[w][ex];
        s_wave_cnt[w][ex] = 0;
      }
      s_cursor[ex] += sum;
    }
    __syncthreads();
  }
}

}  // namespace dsv4
