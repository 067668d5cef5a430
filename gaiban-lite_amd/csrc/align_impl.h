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
//
// The phases (histogram, padded scan with block ids and sentinels, stable
// scatter over a range of flat indices) are separate device functions: one
// workgroup runs all of them (align_block), or, for many assignments, one
// launch per phase pair with the histogram and the scatter split over ranges
// of at least 4096 indices whose per-expert starting cursors come from the
// counts of the ranges before them.
#pragma once

#include "act_quant.h"
#include "common.h"

namespace dsv4 {

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kAlignMaxExperts = 1024;
// Two-launch alignment (align.hip): at least kAlignChunk flat ids per
// workgroup, at most kAlignMaxChunks workgroups (each sums the counts of all
// of them), and at most kAlignSumWorkgroups more workgroups for the
// activation work beside the counting (row sums or W4A8 quantisation).
constexpr int kAlignChunk = 4096;
constexpr int kAlignMaxChunks = 64;
constexpr int kAlignSumWorkgroups = 160;

// LDS of one alignment workgroup.
struct AlignShared {
  int count[kAlignMaxExperts];
  int pad_end[kAlignMaxExperts];
  int cursor[kAlignMaxExperts];
  uint16_t wave_cnt[kAlignWaves][kAlignMaxExperts];
  int scan[kAlignWaves];
  int bad;
};

// Phase 1: per-expert counts of ids[begin, end) into count[0, experts);
// *bad = 1 if an id lies outside [0, experts).  Ends with a barrier.
__device__ __forceinline__ void align_histogram(int* count, int* bad, const int32_t* __restrict__ ids,
                                                int64_t begin, int64_t end, int experts) {
  const int tid = threadIdx.x;
  for (int e = tid; e < experts; e += kAlignThreads) count[e] = 0;
  if (tid == 0) *bad = 0;
  __syncthreads();
  for (int64_t i = begin + tid; i < end; i += kAlignThreads) {
    const int e = ids[i];
    if (e < 0 || e >= experts) {
      *bad = 1;
    } else {
      atomicAdd(&count[e], 1);
    }
  }
  __syncthreads();
}

// Phase 2: from the per-expert totals in sh.count, the padded prefix
// (sh.pad_end, sh.cursor = start of each expert's run) and, for share `part`
// of `parts` workgroups, expert_ids per block, the sentinels of the padding
// slots and of the tail, and ntpp (share 0).  Ends with a barrier.
__device__ __forceinline__ void align_scan(AlignShared& sh, int experts, int block_size, int32_t sentinel,
                                           int32_t* __restrict__ sorted_ids, int64_t capacity,
                                           int32_t* __restrict__ expert_ids, int64_t num_blocks,
                                           int32_t* __restrict__ ntpp, int part, int parts) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // exclusive scan of padded counts over experts (experts <= 1024 = threads)
  int padded = 0;
  if (tid < experts) padded = (sh.count[tid] + block_size - 1) / block_size * block_size;
  int incl = padded;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) sh.scan[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int v = lane < kAlignWaves ? sh.scan[lane] : 0;
    int w = v;
#pragma unroll
    for (int off = 1; off < kAlignWaves; off <<= 1) {
      const int u = __shfl_up(w, off, 64);
      if (lane >= off) w += u;
    }
    if (lane < kAlignWaves) sh.scan[lane] = w - v;  // exclusive per-wave base
  }
  __syncthreads();
  const int pad_end = incl + sh.scan[wave];
  if (tid < experts) {
    sh.pad_end[tid] = pad_end;
    sh.cursor[tid] = pad_end - padded;
  }
  __syncthreads();
  const int total = sh.pad_end[experts - 1];

  // per-block expert ids (searchsorted(padded_ends, start, right=True))
  const int64_t first = (int64_t)part * kAlignThreads + tid;
  const int64_t stride = (int64_t)parts * kAlignThreads;
  for (int64_t b = first; b < num_blocks; b += stride) {
    const int64_t start = b * block_size;
    int32_t owner = -1;
    if (start < total) {
      int lo = 0, hi = experts;  // first e with pad_end[e] > start
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sh.pad_end[mid] > start) hi = mid; else lo = mid + 1;
      }
      owner = lo;
    }
    expert_ids[b] = owner;
  }
  // sentinels: the tail past the total, and each expert's padding slots
  for (int64_t p = (int64_t)total + first; p < capacity; p += stride) sorted_ids[p] = sentinel;
  for (int e = tid * parts + part; e < experts; e += kAlignThreads * parts) {
    const int end = sh.pad_end[e];
    const int used = (end - ((sh.count[e] + block_size - 1) / block_size * block_size)) + sh.count[e];
    for (int p = used; p < end; ++p) sorted_ids[p] = sentinel;
  }
  if (part == 0 && tid == 0) ntpp[0] = total;
  __syncthreads();
}

// Phase 3: stable scatter of the flat indices [begin, end) to
// sorted_ids[sh.cursor[e] + rank], advancing sh.cursor.
__device__ __forceinline__ void align_scatter(AlignShared& sh, const int32_t* __restrict__ ids, int64_t begin,
                                              int64_t end, int experts, int expert_bits,
                                              int32_t* __restrict__ sorted_ids) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  for (int e = tid; e < experts; e += kAlignThreads)
    for (int w = 0; w < kAlignWaves; ++w) sh.wave_cnt[w][e] = 0;
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t base = begin; base < end; base += kAlignThreads) {
    const int64_t i = base + tid;
    const bool active = i < end;
    const int e = active ? ids[i] : 0;
    uint64_t eq = __ballot(active);
    for (int b = 0; b < expert_bits; ++b) {
      const uint64_t bal = __ballot(active && ((e >> b) & 1));
      eq &= ((e >> b) & 1) ? bal : ~bal;
    }
    const int rank_in_wave = __popcll(eq & lt_mask);
    const bool leader = active && rank_in_wave == 0;
    if (leader) sh.wave_cnt[wave][e] = (uint16_t)__popcll(eq);
    __syncthreads();
    if (active) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += sh.wave_cnt[w][e];
      sorted_ids[sh.cursor[e] + before + rank_in_wave] = (int32_t)i;
    }
    __syncthreads();
    for (int ex = tid; ex < experts; ex += kAlignThreads) {
      int sum = 0;
      for (int w = 0; w < kAlignWaves; ++w) {
        sum += sh.wave_cnt[w][ex];
        sh.wave_cnt[w][ex] = 0;
      }
      sh.cursor[ex] += sum;
    }
    __syncthreads();
  }
}

// The whole alignment, run by one workgroup of kAlignThreads threads (every
// thread must call it).  `ids` may have been written by this workgroup just
// before (after a barrier).  A contract violation (an id outside [0, experts))
// is reported through ntpp = -1 and nothing else is written.
__device__ __forceinline__ void align_block(const int32_t* __restrict__ ids, int64_t assignments, int experts,
                                            int expert_bits, int block_size, int32_t* __restrict__ sorted_ids,
                                            int64_t capacity, int32_t* __restrict__ expert_ids, int64_t num_blocks,
                                            int32_t* __restrict__ ntpp) {
  __shared__ AlignShared sh;
  align_histogram(sh.count, &sh.bad, ids, 0, assignments, experts);
  if (sh.bad) {
    if (threadIdx.x == 0) ntpp[0] = -1;
    return;
  }
  align_scan(sh, experts, block_size, (int32_t)assignments, sorted_ids, capacity, expert_ids, num_blocks, ntpp, 0,
             1);
  align_scatter(sh, ids, 0, assignments, experts, expert_bits, sorted_ids);
}

// Per-64-column sums of the bf16 activation rows, xsum[r][c] = sum of
// x[r][64c .. 64c+63] in ascending column order (the order of the experts
// path's own row-sum kernel, so either producer gives the same bits); share
// `part` of `parts` workgroups of kAlignThreads threads.  The prologue
// launches run it beside the alignment.
__device__ __forceinline__ void row_sums_part(const uint16_t* __restrict__ x, int64_t tokens, int hidden,
                                              float* __restrict__ xsum, int part, int parts) {
  const int chunks = hidden / 64;
  const int64_t n = tokens * chunks;
  for (int64_t idx = (int64_t)part * kAlignThreads + threadIdx.x; idx < n; idx += (int64_t)parts * kAlignThreads) {
    const int64_t r = idx / chunks;
    const int c = (int)(idx % chunks);
    const uint16_t* src = x + r * hidden + c * 64;
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 64; e += 8) {
      const u32x4 v = load16(src + e);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sum += __uint_as_float(v[q] << 16);
        sum += __uint_as_float(v[q] & 0xFFFF0000u);
      }
    }
    xsum[idx] = sum;
  }
}

// The prefill form: per 128-column group g of row r, the two 64-column sums
// (each summed as in row_sums_part) combined into the start value of the
// group's MFMA chain, -136 * (s_lo + s_hi), stored at nc[r * (hidden / 128) + g].
__device__ __forceinline__ void row_nc_part(const uint16_t* __restrict__ x, int64_t tokens, int hidden,
                                           float* __restrict__ nc, int part, int parts) {
  const int groups = hidden / 128;
  const int64_t n = tokens * groups;
  for (int64_t idx = (int64_t)part * kAlignThreads + threadIdx.x; idx < n; idx += (int64_t)parts * kAlignThreads) {
    const int64_t r = idx / groups;
    const int g = (int)(idx % groups);
    const uint16_t* src = x + r * hidden + g * 128;
    float half[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 64; e += 8) {
        const u32x4 v = load16(src + 64 * h + e);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sum += __uint_as_float(v[q] << 16);
          sum += __uint_as_float(v[q] & 0xFFFF0000u);
        }
      }
      half[h] = sum;
    }
    nc[idx] = -kDequantBias * (half[0] + half[1]);
  }
}

// Share `part` of `parts` workgroups of kAlignThreads threads of the
// activation work of a prologue launch: the row sums above (either form),
// or the W4A8 quantiser with one wavefront per row (act_quant.h).
__device__ __forceinline__ void act_prep_part(const ActPrep& a, int64_t tokens, int part, int parts) {
  if (a.mode == kPrepRowSums) {
    row_sums_part(a.x, tokens, a.hidden, a.sums, part, parts);
    return;
  }
  if (a.mode == kPrepRowNc) {
    row_nc_part(a.x, tokens, a.hidden, a.sums, part, parts);
    return;
  }
  if (a.mode != kPrepQuantInt4 && a.mode != kPrepQuantNatural) return;
  const int wave = threadIdx.x >> 6;
  for (int64_t r = (int64_t)part * kAlignWaves + wave; r < tokens; r += (int64_t)parts * kAlignWaves) {
    if (a.mode == kPrepQuantInt4)
      act_quant_row<false>(a.x, r, a.hidden, a.q, a.qscale, a.sums);
    else
      act_quant_row<true>(a.x, r, a.hidden, a.q, a.qscale, nullptr);
  }
}

// Workgroups a prologue launch adds for `a` (at most `cap`): 1024 row sums
// or 16 quantised rows per workgroup and round.
inline int64_t act_prep_workgroups(const ActPrep& a, int64_t tokens, int64_t cap) {
  int64_t n = 0;
  if (a.mode == kPrepRowSums) n = (tokens * (a.hidden / 64) + kAlignThreads - 1) / kAlignThreads;
  else if (a.mode == kPrepRowNc) n = (tokens * (a.hidden / 128) + kAlignThreads - 1) / kAlignThreads;
  else if (a.mode == kPrepQuantInt4 || a.mode == kPrepQuantNatural) n = (tokens + kAlignWaves - 1) / kAlignWaves;
  return n < cap ? n : cap;
}

}  // namespace dsv4
