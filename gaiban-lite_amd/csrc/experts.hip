// Grouped expert GEMMs over tiled int4 group-128 weights on bf16 MFMA.
//
// Restates the two Marlin grouped GEMMs of vLLM's _fused_marlin_moe as called
// at runtime/dsv4_direct/moe_runtime.py:1829-1856, with the arithmetic of the
// reference torch path (runtime/dsv4_direct/ops/dense_moe.py:336-354):
//   stage 1: [g | u] = x[rows] . W13^T (fp32 accumulate), h = SiLU(min(g,L)) *
//            clamp(u,-L,L) in fp32, h rounded to bf16;  also writes the fp32
//            sum of each row's bf16 h over every 64-wide chunk of stage 2's K;
//   stage 2: y = h . W2^T (fp32 accumulate) * route_weight, written fp32 per
//            (token, k) slot (the shared expert uses weight 1);
//   combine: out[t] = bf16( sum_j y[t*k+j] + y_shared[t] ), one rounding
//            (moe_runtime.py:1857,1873 with a single fp32 accumulation).
//
// Arithmetic per quantisation group g (128 K values) of weight row n and
// token column t:  the MFMA chain starts from -136 * sum_g(x) (from the
// precomputed 64-wide row sums, added in a fixed order) and sums
// (q + 136) * x (dequant_biased), which leaves sum_g(q * x); the decode
// kernel accumulates s[n, g] times it in fp32, the prefill kernel keeps a
// running sum divided by the current group's scale (see there).
//
// Two kernels share this arithmetic:
//  * expert_decode_kernel (alignment blocks of <= 16 token slots): one
//    workgroup of 4 wavefronts per (expert block, N tile), two 16-row weight
//    strips per wavefront, weights prefetched two groups ahead, the block's
//    activations staged group by group in LDS one group ahead, loads issued in
//    an order that never makes the in-order vmcnt wait on a prefetch;  padded
//    token slots read zeros through out-of-range buffer loads (no branches in
//    the K loop).  Shared-expert blocks carry 16 tokens.
//  * expert_prefill_kernel (blocks of 32-64 slots): 64 token slots x 256
//    weight rows per workgroup, token tiles staged in LDS, XCD-aware order.
#include <algorithm>
#include <type_traits>

#include "act_quant.h"
#include "experts_common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

// ------------------------------------------------------------------ decode
// Persistent: the grid is sized to the resident workgroups; workgroup w takes
// items w, w + stride, ... of the active items (block, tile) -- routed
// blocks below ceil(ntpp / block_size), then the shared-expert blocks -- so no
// workgroup is launched for a padding block.  The K stream runs on across
// item boundaries: the next item's activation group and first two weight
// groups are fetched during the current item's last groups, and its metadata
// (expert, row ids) is loaded when the current item starts.
// STAGE 1: wave w owns gate strip n0/16 + w and up strip (inter + n0)/16 + w,
//          n0 = tile * 64 (one 64-row chunk of h per item).
// STAGE 2: wave w owns strips (n0 + 32 w)/16 + {0, 1}, n0 = tile * 128.
// The 16 token slots x 128 K of the current group live in LDS (double
// buffered, one barrier per group): every thread loads 16 bytes per group,
// every wavefront reads its four MFMA B fragments with ds_read_b128.

struct DecodeItem {
  const uint8_t* wq;   // this lane's 16 bytes of the pair's first tile
  const uint16_t* ws;  // this lane's 4 scales of the pair's first group
  uint32_t ld_base;    // loader thread: activation row offset of its slot (or out of range)
  uint32_t sum_base;   // lane: row-sum offset of its slot (or out of range)
  int64_t rowid;       // lane: row id of its slot, -1 if padded
  int n0;
  float wmul;          // 1, or NaN when the block names no valid expert (stage-2 multiplier)
  bool skip;           // PAIR: the block is the second of a pair, computed by the first
};

// `tid`: the thread's index in the 256 threads that compute the item.
template <int STAGE, bool PAIR>
__device__ __forceinline__ DecodeItem decode_item(const ExpertGemmParams& p, int item, int routed, int64_t tk,
                                                  int tid) {
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int bi, tile;
  decode_item_block(p, item, routed, bi, tile);
  const int blk = bi < routed ? bi : p.max_blocks + (bi - routed);
  const BlockInfo b = block_info(p, blk);
  const int groups = p.k_dim / kGroup;
  const int sums_per_row = p.k_dim / kSumChunk;
  DecodeItem it;
  const int span = decode_block_span<PAIR>(p, bi, routed);
  it.skip = span == 0;
  if (it.skip) return it;
  it.n0 = STAGE == 1 ? tile * 64 : tile * 128;
  const int pair = tile * 4 + wave;
  it.wq = p.wq + (int64_t)b.expert * p.wq_stride + (int64_t)pair * groups * 2048 + lane * 16;
  it.ws = p.ws + (int64_t)b.expert * p.ws_stride + (int64_t)pair * groups * 32 + 8 * (lane >> 4);
  it.wmul = b.poison ? __builtin_nanf("") : 1.0f;
  it.rowid = slot_rowid_span(p, b, lane & 15, tk, span);
  const int64_t arow = act_row_of<STAGE>(it.rowid, tk, p.topk);
  it.sum_base = arow >= 0 ? (uint32_t)(arow * sums_per_row * 4) : kOobOffset;
  const int ld_slot = tid >> 4;
  const int64_t ld_row = act_row_of<STAGE>(slot_rowid_span(p, b, ld_slot, tk, span), tk, p.topk);
  it.ld_base = ld_row >= 0 ? (uint32_t)(ld_row * p.k_dim * 2 + (tid & 15) * 16) : kOobOffset;
  return it;
}

// RING = 4: weights two groups ahead, four workgroups per CU.
// RING = 8: weights six groups ahead, three workgroups per CU (at most 168
// VGPRs; at 169 the occupancy drops to two and T=64 stage 1 takes 6% longer);
// K must be a multiple of 8 groups.  Stage 1 (w13, 256 KiB per item) streams faster with
// the deeper ring at every T measured; stage 2 (128 KiB items) keeps RING = 4
// unless its items fit one wave of resident workgroups (T ~ 1), where the
// bytes in flight per workgroup, not the workgroup count, bound the stream.
template <int STAGE, int RING, bool PAIR>
__global__ __launch_bounds__(256, RING == 4 ? 4 : 3) void expert_decode_kernel(ExpertGemmParams p) {
  constexpr int R = 2;
  constexpr int kAhead = RING - 2;
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][16 * 256];  // part q of slot s at q ^ s
  __shared__ float red[4][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t tk = p.tokens * p.topk;
  const int routed = decode_routed_blocks(p);
  const int n_items = decode_items(p, routed);
  const int stride = decode_stride(n_items);
  int item = blockIdx.x;
  if (item >= stride || item >= n_items) return;  // uniform per workgroup
  const int groups = p.k_dim / kGroup;
  const int sums_per_row = p.k_dim / kSumChunk;

  // Activations and their sums through buffer loads; padded slots read 0.
  const __amdgpu_buffer_rsrc_t act_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act, (short)0, (int)(p.act_rows * p.k_dim * 2), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t sum_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act_sum, (short)0, (int)(p.act_rows * sums_per_row * 4), kRsrcFlags);
  const int ld_slot = threadIdx.x >> 4;  // cooperative group load: slot, 16-byte part
  const int ld_lds = ld_slot * 256 + (((threadIdx.x & 15) ^ ld_slot) * 16);
  int rd_lds[4];  // K step d: part 4d + lane/16 of slot lane % 16
#pragma unroll
  for (int d = 0; d < 4; ++d) rd_lds[d] = (lane & 15) * 256 + (((4 * d + (lane >> 4)) ^ (lane & 15)) * 16);

  // this workgroup's next item from index i on (n_items when none is left),
  // passing over the items of paired second blocks
  auto fetch = [&](int i, DecodeItem& it) {
    for (; i < n_items; i += stride) {
      it = decode_item<STAGE, PAIR>(p, i, routed, tk, threadIdx.x);
      if (!it.skip) return i;
    }
    return n_items;
  };
  DecodeItem cur;
  item = fetch(item, cur);
  if (item >= n_items) return;  // uniform per workgroup
  DecodeItem nxt;
  int next = fetch(item + stride, nxt);
  if (next >= n_items) nxt = cur;

  // Weights kAhead groups ahead (ring RING), activations + sums one group
  // ahead (ring 2).  At the end of an item the prefetches continue with the
  // next item (or re-read the current one when there is none), so every load
  // is unconditional and the compiler's vmcnt waits stay exact.
  u32x4 W[RING][R];
  u32x4 S[RING];
  float CS[2][2];
  u32x4 xr;

  auto issue_w = [&](const DecodeItem& it, int g, u32x4 (&w)[R], u32x4& s) {
    w[0] = load16_nt(it.wq + g * 2048);
    w[1] = load16_nt(it.wq + g * 2048 + 1024);
    s = load16(it.ws + g * 32);  // 4 rows of both members
  };
  auto issue_x = [&](const DecodeItem& it, int g, float (&cs)[2]) {
    xr = __builtin_amdgcn_raw_buffer_load_b128(act_rsrc, it.ld_base + (uint32_t)(g * 256), 0, 0);
    cs[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sum_rsrc, it.sum_base + (uint32_t)(g * 8), 0, 0));
    cs[1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sum_rsrc, it.sum_base + (uint32_t)(g * 8 + 4), 0, 0));
  };

  const uint32_t magic = dequant_magic();
  issue_x(cur, 0, CS[0]);
#pragma unroll
  for (int a = 0; a < kAhead; ++a) issue_w(cur, a, W[a], S[a]);
  *reinterpret_cast<u32x4*>(&xs[0][ld_lds]) = xr;
  __syncthreads();

  for (;;) {
    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < groups; g0 += RING) {  // groups % RING == 0 (checked on the host)
#pragma unroll
      for (int u = 0; u < RING; ++u) {
        const int g = g0 + u;
        const bool xn = g + 1 >= groups;  // the activation prefetch crosses into the next item
        issue_x(xn ? nxt : cur, xn ? 0 : g + 1, CS[(u + 1) & 1]);
        const bool wn = g + kAhead >= groups;
        issue_w(wn ? nxt : cur, wn ? g + kAhead - groups : g + kAhead, W[(u + kAhead) % RING],
                S[(u + kAhead) % RING]);
        // the MFMA chain starts from -136 * sum_g(x): it yields sum_g(q * x) directly
        const float nc = -kDequantBias * (CS[u & 1][0] + CS[u & 1][1]);
        const f32x4 init = {nc, nc, nc, nc};
        f32x4 tmp[R];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const bf16x8 bfr = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xs[u & 1][rd_lds[d]]));
#pragma unroll
          for (int r = 0; r < R; ++r) tmp[r] = mfma_bf16(dequant_biased(W[u][r][d], magic), bfr, d == 0 ? init : tmp[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float sc[4];
          scale4(u32x2{S[u][2 * r], S[u][2 * r + 1]}, sc);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[r][i] += sc[i] * tmp[r][i];
        }
        *reinterpret_cast<u32x4*>(&xs[(u + 1) & 1][ld_lds]) = xr;
        __syncthreads();
      }
    }

    const int64_t rowid = cur.rowid;
    if constexpr (STAGE == 1) {
      const float lim = p.clamp_limit;
      uint32_t bits[4];
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gt = acc[0][i];
        float up = acc[1][i];
        if (lim > 0.0f) {
          gt = fminf(gt, lim);
          up = fminf(fmaxf(up, -lim), lim);
        }
        bits[i] = float_to_bf16_bits(silu_f(gt) * up);
        part += __uint_as_float(bits[i] << 16);
      }
      if (rowid >= 0) {
        const int n = cur.n0 + 16 * wave + 4 * (lane >> 4);
        u32x2 packed = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
        *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) = packed;
      }
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      if (lane < 16) red[wave][lane] = part;
      __syncthreads();
      if (threadIdx.x < 16 && rowid >= 0) {
        const float total = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
        p.hsum_out[rowid * (p.inter / kSumChunk) + cur.n0 / kSumChunk] = total;
      }
    } else {
      if (rowid >= 0) {
        const float wr = (rowid < tk ? p.route_w[rowid] : 1.0f) * cur.wmul;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int n = cur.n0 + 32 * wave + 16 * r + 4 * (lane >> 4);
          f32x4 v = acc[r];
          v[0] *= wr; v[1] *= wr; v[2] *= wr; v[3] *= wr;
          *reinterpret_cast<f32x4*>(p.contrib + rowid * p.out_cols + n) = v;
        }
      }
    }
    if (next >= n_items) break;  // uniform per workgroup; the last prefetches re-read cur
    item = next;
    cur = nxt;
    next = fetch(item + stride, nxt);
    if (next >= n_items) nxt = cur;
  }
}

// ------------------------------------------------------- decode, K split
// For launches with at most one decode item per CU (T = 1: 7 blocks x 32 N
// tiles = 224 items on 256 CUs).  There each item's four wavefronts walk the
// K groups of their strip pairs in sequence, one barrier per group, and that
// serial chain, not the memory system, bounds the stream (stage 1 at T = 1
// moved 59 MB in 21 us: 12-14 GB/s per CU).  Here eight wavefronts share an
// item: wavefronts w and w + 4 take the same strip pair, w the lower half of
// K and w + 4 the upper half, each with the deep ring of
// expert_decode_kernel (weights six groups ahead) and its own activation
// tile in LDS.  At the end the upper half's accumulators pass through LDS,
// the lower half adds them, and the epilogue is expert_decode_kernel's.  Each
// group's arithmetic is expert_decode_kernel's; the sum over groups is
// formed as (lower half) + (upper half), so the results can differ from
// that kernel's in the last bits.
// RESIDENT (K <= 4096: at most kKsplitResidentGroups groups per half): each
// half's activation rows (16 slots x its K range, 64 KiB) and their 64-column
// sums are copied into LDS once, before the K loop, so the loop holds only
// the weight ring and the MFMAs: no activation load, no LDS store and no
// barrier per group.  With a group's copy one group ahead and a barrier per
// group, the four wavefronts of a half waited on that copy every group (8
// MFMAs of work per group at one token), and the CU kept about 33 L1 -> L2
// requests in flight against ~90 in the persistent kernel at T = 64.  The
// same operations in the same order on every value: the same bits.
constexpr int kKsplitResidentGroups = 16;

template <int STAGE, bool RESIDENT>
__global__ __launch_bounds__(512, 1) void expert_decode_ksplit_kernel(ExpertGemmParams p) {
  constexpr int R = 2;
  constexpr int RING = 8;
  constexpr int kAhead = RING - 2;
  constexpr int kXsGroups = RESIDENT ? kKsplitResidentGroups : 2;
  // [half][group (RESIDENT) or buffer][slot x 256 B], part q of slot s at q ^ s
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kXsGroups][16 * 256];
  // RESIDENT: [half][64-column chunk of the half][slot] activation sums
  __shared__ float xsum[RESIDENT ? 2 : 1][RESIDENT ? 2 * kKsplitResidentGroups : 1][16];
  __shared__ f32x4 upper[4][R][64];
  __shared__ float red[4][16];
  const int tid = threadIdx.x & 255;
  const int half = threadIdx.x >> 8;  // wavefront-uniform
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t tk = p.tokens * p.topk;
  const int routed = decode_routed_blocks(p);
  const int n_items = decode_items(p, routed);
  const int item = blockIdx.x;
  if (item >= n_items) return;  // uniform per workgroup
  const DecodeItem cur = decode_item<STAGE, false>(p, item, routed, tk, tid);
  const int hg = p.k_dim / kGroup / 2;  // groups per half: a multiple of RING (checked on the host)
  const int gb = half * hg;             // this half's first group
  const int sums_per_row = p.k_dim / kSumChunk;

  const __amdgpu_buffer_rsrc_t act_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act, (short)0, (int)(p.act_rows * p.k_dim * 2), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t sum_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act_sum, (short)0, (int)(p.act_rows * sums_per_row * 4), kRsrcFlags);
  const int ld_slot = tid >> 4;
  const int ld_lds = ld_slot * 256 + (((tid & 15) ^ ld_slot) * 16);
  int rd_lds[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) rd_lds[d] = (lane & 15) * 256 + (((4 * d + (lane >> 4)) ^ (lane & 15)) * 16);

  u32x4 W[RING][R];
  u32x4 S[RING];
  float CS[2][2];
  u32x4 xr;
  auto issue_w = [&](int g, u32x4 (&w)[R], u32x4& sv) {
    w[0] = load16_nt(cur.wq + g * 2048);
    w[1] = load16_nt(cur.wq + g * 2048 + 1024);
    sv = load16(cur.ws + g * 32);
  };
  auto issue_x = [&](int g, float (&cs)[2]) {
    xr = __builtin_amdgcn_raw_buffer_load_b128(act_rsrc, cur.ld_base + (uint32_t)(g * 256), 0, 0);
    cs[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sum_rsrc, cur.sum_base + (uint32_t)(g * 8), 0, 0));
    cs[1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sum_rsrc, cur.sum_base + (uint32_t)(g * 8 + 4), 0, 0));
  };

  const uint32_t magic = dequant_magic();
  if constexpr (RESIDENT) {
    // the half's activation groups (padded slots read zeros) and sums, once
    u32x4 rows[kKsplitResidentGroups];
#pragma unroll
    for (int g = 0; g < kKsplitResidentGroups; ++g)
      if (g < hg) rows[g] = __builtin_amdgcn_raw_buffer_load_b128(act_rsrc, cur.ld_base + (uint32_t)((gb + g) * 256), 0, 0);
    const int chunk = tid >> 4;  // 0..15, and 16 + that
    float cs_lo = 0.0f, cs_hi = 0.0f;
    if (chunk < 2 * hg)
      cs_lo = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                            sum_rsrc, cur.sum_base + (uint32_t)((2 * gb + chunk) * 4), 0, 0));
    if (chunk + 16 < 2 * hg)
      cs_hi = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                            sum_rsrc, cur.sum_base + (uint32_t)((2 * gb + chunk + 16) * 4), 0, 0));
#pragma unroll
    for (int a = 0; a < kAhead; ++a) issue_w(gb + a, W[a], S[a]);
#pragma unroll
    for (int g = 0; g < kKsplitResidentGroups; ++g)
      if (g < hg) *reinterpret_cast<u32x4*>(&xs[half][g][ld_lds]) = rows[g];
    if (chunk < 2 * hg) xsum[half][chunk][tid & 15] = cs_lo;
    if (chunk + 16 < 2 * hg) xsum[half][chunk + 16][tid & 15] = cs_hi;
  } else {
    issue_x(gb, CS[0]);
#pragma unroll
    for (int a = 0; a < kAhead; ++a) issue_w(gb + a, W[a], S[a]);
    *reinterpret_cast<u32x4*>(&xs[half][0][ld_lds]) = xr;
  }
  __syncthreads();

  f32x4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int g0 = 0; g0 < hg; g0 += RING) {
#pragma unroll
    for (int u = 0; u < RING; ++u) {
      const int g = g0 + u;
      // prefetches past the half's end re-read its last group (unused), so
      // every load is unconditional and the compiler's vmcnt waits stay exact
      if constexpr (!RESIDENT) issue_x(gb + min(g + 1, hg - 1), CS[(u + 1) & 1]);
      issue_w(gb + min(g + kAhead, hg - 1), W[(u + kAhead) % RING], S[(u + kAhead) % RING]);
      float nc;
      if constexpr (RESIDENT)
        nc = -kDequantBias * (xsum[half][2 * g][lane & 15] + xsum[half][2 * g + 1][lane & 15]);
      else
        nc = -kDequantBias * (CS[u & 1][0] + CS[u & 1][1]);
      const f32x4 init = {nc, nc, nc, nc};
      const uint8_t* xg = RESIDENT ? &xs[half][min(g, kXsGroups - 1)][0] : &xs[half][u & 1][0];
      f32x4 tmp[R];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const bf16x8 bfr = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xg[rd_lds[d]]));
#pragma unroll
        for (int r = 0; r < R; ++r) tmp[r] = mfma_bf16(dequant_biased(W[u][r][d], magic), bfr, d == 0 ? init : tmp[r]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float sc[4];
        scale4(u32x2{S[u][2 * r], S[u][2 * r + 1]}, sc);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][i] += sc[i] * tmp[r][i];
      }
      if constexpr (!RESIDENT) {
        *reinterpret_cast<u32x4*>(&xs[half][(u + 1) & 1][ld_lds]) = xr;
        __syncthreads();
      }
    }
  }

  if (half == 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) upper[wave][r][lane] = acc[r];
  }
  __syncthreads();
  if (half == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f32x4 hi = upper[wave][r][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[r][i] += hi[i];
    }
  }

  const int64_t rowid = cur.rowid;
  if constexpr (STAGE == 1) {
    if (half == 0) {
      const float lim = p.clamp_limit;
      uint32_t bits[4];
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gt = acc[0][i];
        float up = acc[1][i];
        if (lim > 0.0f) {
          gt = fminf(gt, lim);
          up = fminf(fmaxf(up, -lim), lim);
        }
        bits[i] = float_to_bf16_bits(silu_f(gt) * up);
        part += __uint_as_float(bits[i] << 16);
      }
      if (rowid >= 0) {
        const int n = cur.n0 + 16 * wave + 4 * (lane >> 4);
        u32x2 packed = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
        *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) = packed;
      }
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      if (lane < 16) red[wave][lane] = part;
    }
    __syncthreads();
    if (threadIdx.x < 16 && rowid >= 0) {
      const float total = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
      p.hsum_out[rowid * (p.inter / kSumChunk) + cur.n0 / kSumChunk] = total;
    }
  } else {
    if (half == 0 && rowid >= 0) {
      const float wr = (rowid < tk ? p.route_w[rowid] : 1.0f) * cur.wmul;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = cur.n0 + 32 * wave + 16 * r + 4 * (lane >> 4);
        f32x4 v = acc[r];
        v[0] *= wr; v[1] *= wr; v[2] *= wr; v[3] *= wr;
        *reinterpret_cast<f32x4*>(p.contrib + rowid * p.out_cols + n) = v;
      }
    }
  }
}

// ----------------------------------------------------------------- prefill
// Alignment blocks of up to 64 token slots (block sizes 32/48/64).  Workgroup
// tile: 64 token slots x 256 weight rows; wavefront w owns 64 rows:
//   STAGE 1: gate strips (n0 + 32w)/16 + {0,1} and the matching up strips,
//            n0 = tile * 128 (the workgroup covers h columns [n0, n0+128));
//   STAGE 2: strips (n0 + 64w)/16 + {0..3}, n0 = tile * 256.
// Per group the 64 x 128 token tile, its 64 group sums and each wavefront's
// scale ratios are copied into LDS by buffer_load ... lds (double buffered,
// one group ahead); each wavefront's weight tiles are private to it and go
// straight into registers, one group ahead, so LDS carries only the shared
// operand.  Each wavefront reads 4 B fragments per K step and issues 16
// MFMAs.  Work items (block, tile) follow prefill_item: groups of
// consecutive blocks run tile by tile on one XCD, so a weight tile is
// fetched once for the group and a block's token rows stay in that XCD's L2
// across its tiles.  Three workgroups per CU (at most 168 VGPRs: the
// compiler spills a few setup values outside the K loops, none inside them);
// the third workgroup hides more of the issue stalls than it costs.
constexpr int kPfSlots = 64;

// An expert whose group scales spread too widely for the running-sum scaling
// (marked by dsv4moe_pack_int4_ratios: 1.0 in its ratio element 0, which is
// otherwise 0) is computed by expert_prefill_exact_kernel instead.
__device__ __forceinline__ bool expert_needs_exact(const ExpertGemmParams& p, int expert) {
  return __builtin_nontemporal_load(p.wr + (int64_t)expert * p.ws_stride) != 0.0f;
}

template <int STAGE>
__global__ __launch_bounds__(256, 3) void expert_prefill_kernel(ExpertGemmParams p, int total_blocks) {
  constexpr int R = 4;
  // Per group, copied into LDS by buffer_load ... lds (double buffered):
  //  * token tile: 64 slots x 256 B, 16-byte part p of slot s stored at part
  //    p ^ (s & 15) (conflict-free ds_read_b128 of the B fragments);
  //  * the 64 slots' start values -136 * sum_g(x) (the prefill form of the
  //    activation sums: row_nc_part, the stage-1 epilogues);
  //  * each wavefront's 16-row scale ratios (fp32, 256 B).
  // Padded slots read zeros (out-of-range buffer offsets).
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kPfSlots * 256];
  // 64 lanes x 4 B per ratio DMA: lanes 0..31 carry pair p0's 128-byte block,
  // lanes 32..63 pair p0 + 1's.
  __shared__ __attribute__((aligned(16))) uint8_t scl[2][4][256];
  __shared__ float xnc[2][kPfSlots];
  __shared__ float red[4][kPfSlots];  // stage-1 epilogue: per-wavefront column sums
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  int blk, tile;
  if (!prefill_item(p.n_tiles, total_blocks, blk, tile)) return;
  const int64_t tk = p.tokens * p.topk;
  const BlockInfo b = block_info(p, blk);
  if (!b.active) return;
  if (expert_needs_exact(p, b.expert)) return;  // expert_prefill_exact_kernel computes it

  const int groups = p.k_dim / kGroup;

  // wavefront w streams strip pairs p0 = tile*8 + 2w and p0 + 1; its strips
  // r = 2j + m are member m of pair p0 + j.  Stage 1: gate (m = 0) and up
  // (m = 1) rows of h columns n0 + 32w + 16j ..; stage 2: rows n0 + 64w + 16r.
  const int n0 = STAGE == 1 ? tile * 128 : tile * 256;
  const int p0 = tile * 8 + 2 * wave;

  const __amdgpu_buffer_rsrc_t act_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act, (short)0, (int)(p.act_rows * p.k_dim * 2), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t nc_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act_sum, (short)0, (int)(p.act_rows * groups * 4), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.wq + (int64_t)b.expert * p.wq_stride), (short)0, (int)p.wq_stride, kRsrcFlags);
  const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.ws + (int64_t)b.expert * p.ws_stride), (short)0, (int)(p.ws_stride * 2), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t r_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.wr + (int64_t)b.expert * p.ws_stride), (short)0, (int)(p.ws_stride * 4), kRsrcFlags);

  // token tile: DMA q (0..3) of wave w fills LDS rows 16w + 4q + lane/16
  uint32_t dma_off[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 16 * wave + 4 * q + (lane >> 4);
    const int64_t ar = act_row_of<STAGE>(slot_rowid(p, b, row, tk), tk, p.topk);
    const int part = (lane & 15) ^ (row & 15);
    dma_off[q] = ar >= 0 ? (uint32_t)(ar * p.k_dim * 2 + part * 16) : kOobOffset;
  }
  uint32_t nc_off = kOobOffset;
  if (wave == 0) {
    const int64_t ar = act_row_of<STAGE>(slot_rowid(p, b, lane, tk), tk, p.topk);
    if (ar >= 0) nc_off = (uint32_t)(ar * groups * 4);
  }
  // weight tiles: pair p, group g, member m at byte ((p*groups + g)*2 + m) * 1 KiB
  const uint32_t w_off0 = (uint32_t)(p0 * groups) * 2048 + lane * 16;
  const uint32_t w_off1 = (uint32_t)((p0 + 1) * groups) * 2048 + lane * 16;
  // ratios: 128 bytes per (pair, group), 32 lanes x 4 bytes per pair
  const uint32_t r_off = (uint32_t)((p0 + (lane >> 5)) * groups) * 128 + (lane & 31) * 4;

  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // here, plus constant offsets (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][16 * wave * 256]));
  const uint32_t scl_lds = __builtin_amdgcn_readfirstlane(lds_addr(&scl[0][wave][0]));
  const uint32_t xnc_lds = lds_addr(&xnc[0][0]);
  auto issue = [&](int g, int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      lds_copy16(act_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + q * 1024, dma_off[q], g * 256);
    lds_copy4(r_rsrc, scl_lds + buf * (uint32_t)sizeof(scl[0]), r_off, g * 128);
    if (wave == 0) lds_copy4(nc_rsrc, xnc_lds + buf * (uint32_t)sizeof(xnc[0]), nc_off, g * 4);
  };
  // The weight tiles are private to the wavefront: loaded straight into
  // registers, one group ahead, as inline asm -- the compiler neither counts
  // them in its own vmcnt waits nor lets their uses move above wait_weights,
  // which takes the registers as in/out operands.  The registers in flight
  // must not be touched in between: the kernel must compile without spills
  // (tests/test_kernel_resources.py checks the compiled code object).
  struct WRegs {
    u32x4 w[R];
  };
  auto load_weights = [&](int g, WRegs& o) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t gw = __builtin_amdgcn_readfirstlane((uint32_t)g * 2048u);
    const uint32_t w0b = w_off0 + kTileBytes, w1b = w_off1 + kTileBytes;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[0]) : "v"(w_off0), "s"(w_rsrc), "s"(gw));
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[1]) : "v"(w0b), "s"(w_rsrc), "s"(gw));
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[2]) : "v"(w_off1), "s"(w_rsrc), "s"(gw));
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[3]) : "v"(w1b), "s"(w_rsrc), "s"(gw));
#endif
  };
  auto wait_weights = [&](WRegs& o) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(o.w[0]), "+v"(o.w[1]), "+v"(o.w[2]), "+v"(o.w[3]) : : "memory");
#endif
  };

  // Token columns that hold a valid slot: the alignment pads each expert's
  // run at its end, so a block's valid slots come first.  The loop runs over
  // ceil(valid / 16) of the four 16-slot column tiles, at least two (the
  // MFMAs and scale FMAs of the empty tiles are skipped: partial blocks are
  // the last block of every expert, and most blocks when experts average
  // under 64 slots).
  const uint64_t valid = __ballot(slot_rowid(p, b, lane, tk) >= 0);
  const int used = valid ? 64 - __builtin_clzll(valid) : 0;

  auto body = [&](auto c_c) {
    constexpr int C = decltype(c_c)::value;
    // Running sum per accumulator element (row n, token column t): after group
    // g it holds sum_{g' <= g} s[n, g'] * sum_g'(q * x) divided by s[n, g].  At
    // the start of group g it is multiplied by r = s[n, g-1] / s[n, g] (fp32
    // ratios precomputed from the packed scales; r is 0 for g = 0, where the
    // accumulator is 0) and -136 * sum_g(x) is added, one FMA per element; the
    // MFMA chain then adds sum_g((q + 136) * x), leaving the quotient for group
    // g.  The last group's scale is applied in the epilogue.  One accumulator
    // set and no second pass over partial sums: the FMA of a tile waits only for
    // that tile's previous MFMA, 16 MFMAs earlier.
    f32x4 acc[R][C];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int ct = 0; ct < C; ++ct) acc[r][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int sw = lane & 15;  // swizzle key of this lane's slots (ct*16 + sw)
    const uint32_t magic = dequant_magic();
    // One group: optionally prefetch group g+1 into the other buffers and
    // registers, then the fold and 64 MFMAs.
    auto step = [&](int g, auto u_c, auto prefetch_c, const WRegs& cur, WRegs& nxt) {
      constexpr int u = decltype(u_c)::value;
      if constexpr (decltype(prefetch_c)::value) {
        issue(g + 1, (u + 1) & 1);
        load_weights(g + 1, nxt);
      }
      float nc[C];
#pragma unroll
      for (int ct = 0; ct < C; ++ct) nc[ct] = xnc[u][ct * 16 + sw];
      // ratios of strip r = 2j + m: pair j's block, element (quad * 2 + m) * 4 + i
      f32x4 ratio[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        ratio[r] = *reinterpret_cast<const f32x4*>(&scl[u][wave][(r >> 1) * 128 + ((lane >> 4) * 2 + (r & 1)) * 16]);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int part = ((4 * d + (lane >> 4)) ^ sw) * 16;
        bf16x8 bfr[C];
#pragma unroll
        for (int ct = 0; ct < C; ++ct)
          bfr[ct] = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const u32x4*>(&xs[u][(ct * 16 + sw) * 256 + part]));
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const bf16x8 a = dequant_biased(cur.w[r][d], magic);
#pragma unroll
          for (int ct = 0; ct < C; ++ct) {
            if (d == 0) {
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[r][ct][i] = __builtin_fmaf(acc[r][ct][i], ratio[r][i], nc[ct]);
            }
            acc[r][ct] = mfma_bf16(a, bfr[ct], acc[r][ct]);
          }
        }
      }
      if constexpr (decltype(prefetch_c)::value)
        wait_weights(nxt);  // this wavefront's copies and loads of group g + 1 have landed
      else
        lds_dma_wait_all();
      __syncthreads();     // ... and everyone's; buffer u is free again
    };
    using U0 = std::integral_constant<int, 0>;
    using U1 = std::integral_constant<int, 1>;
    using PF = std::true_type;
    using NOPF = std::false_type;

    WRegs wa, wb;
    issue(0, 0);
    load_weights(0, wa);
    wait_weights(wa);
    __syncthreads();
    // groups is even (checked on the host); the last group issues no prefetch,
    // so no copy or load is in flight when the workgroup leaves the loop.
    for (int g0 = 0; g0 + 2 < groups; g0 += 2) {
      step(g0, U0{}, PF{}, wa, wb);
      step(g0 + 1, U1{}, PF{}, wb, wa);
    }
    step(groups - 2, U0{}, PF{}, wa, wb);
    step(groups - 1, U1{}, NOPF{}, wb, wa);
    // the last group's scales (bf16, 4 rows of strip r per lane)
    float slast[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t off = (uint32_t)((p0 + (r >> 1)) * groups + groups - 1) * 64 + 16 * (lane >> 4) + 8 * (r & 1);
      scale4(__builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(s_rsrc, off, 0, 0)), slast[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int ct = 0; ct < C; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][ct][i] *= slast[r][i];

    if constexpr (STAGE == 1) {
      const float lim = p.clamp_limit;
#pragma unroll
      for (int ct = 0; ct < C; ++ct) {
        const int64_t rowid = slot_rowid(p, b, ct * 16 + sw, tk);
        float part = 0.0f;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          uint32_t bits[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float gt = acc[2 * s][ct][i];
            float up = acc[2 * s + 1][ct][i];
            if (lim > 0.0f) {
              gt = fminf(gt, lim);
              up = fminf(fmaxf(up, -lim), lim);
            }
            bits[i] = float_to_bf16_bits(silu_rcp(gt) * up);
            part += __uint_as_float(bits[i] << 16);
          }
          if (rowid >= 0) {
            const int n = n0 + 32 * wave + 16 * s + 4 * (lane >> 4);
            u32x2 packed = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
            *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) = packed;
          }
        }
        part += __shfl_xor(part, 16, 64);
        part += __shfl_xor(part, 32, 64);
        if (lane < 16) red[wave][ct * 16 + lane] = part;
      }
      __syncthreads();
      if (threadIdx.x < C * 16) {
        // stage 2's start value for K group `tile` (its 128 columns are this
        // workgroup's h columns): -136 * (sum of the two 64-column halves)
        const int col = threadIdx.x;
        const int64_t rid = slot_rowid(p, b, col, tk);
        if (rid >= 0) {
          const float lo = red[0][col] + red[1][col];
          const float hi = red[2][col] + red[3][col];
          p.hsum_out[rid * (p.inter / kGroup) + tile] = -kDequantBias * (lo + hi);
        }
      }
    } else {
#pragma unroll
      for (int ct = 0; ct < C; ++ct) {
        const int64_t rowid = slot_rowid(p, b, ct * 16 + sw, tk);
        if (rowid < 0) continue;
        const float wr = contrib_weight(p, b, rowid, tk);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int n = n0 + 64 * wave + 16 * r + 4 * (lane >> 4);
          f32x4 v = acc[r][ct];
          v[0] *= wr; v[1] *= wr; v[2] *= wr; v[3] *= wr;
          *reinterpret_cast<f32x4*>(p.contrib + rowid * p.out_cols + n) = v;
        }
      }
    }
  };
  if (used > 48)
    body(std::integral_constant<int, 4>{});
  else if (used > 32)
    body(std::integral_constant<int, 3>{});
  else
    body(std::integral_constant<int, 2>{});
}


// ----------------------------------------------------- exact prefill path
// The prefill blocks of experts marked for exact scaling (see
// expert_needs_exact), with each group's partial sums scaled by the group's
// own bf16 scale, as the decode kernels do: part = -136 * sum_g(x) + the MFMA
// chain of the group, then acc += s[n, g] * part.  Correctness only (such
// scale spreads do not occur in the benchmark weights): plain loads, one
// barrier pair per group, the same tile (64 slots x 256 rows, wavefront w on
// strip pairs tile*8 + 2w and + 1), the same K assignment and the same
// epilogue as expert_prefill_kernel.  Persistent over kExactGrid
// workgroups: each takes 256 blocks at a time, finds the marked ones with
// one load per thread and computes every N tile of each; with nothing
// marked every workgroup leaves after one round of loads.
constexpr int kExactGrid = 64;

template <int STAGE>
__global__ __launch_bounds__(256, 1) void expert_prefill_exact_kernel(ExpertGemmParams p, int total_blocks) {
  constexpr int R = 4, C = 4;
  __shared__ __attribute__((aligned(16))) uint8_t xs[kPfSlots * 256];  // slot s: its 128 K of bf16
  __shared__ float xsum_s[kPfSlots];
  __shared__ float red[4][kPfSlots];
  __shared__ int list[256];
  __shared__ int count;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sw = lane & 15;
  const int64_t tk = p.tokens * p.topk;
  const int groups = p.k_dim / kGroup;
  const uint32_t magic = dequant_magic();
  // element 1 of the stack's ratios: 1.0 when any expert of it is marked
  if (__builtin_nontemporal_load(p.wr + 1) == 0.0f) return;

  for (int base = (int)blockIdx.x * 256; base < total_blocks; base += (int)gridDim.x * 256) {
    if (threadIdx.x == 0) count = 0;
    __syncthreads();
    const int blk0 = base + (int)threadIdx.x;
    if (blk0 < total_blocks) {
      const BlockInfo bi = block_info(p, blk0);
      if (bi.active && expert_needs_exact(p, bi.expert)) list[atomicAdd(&count, 1)] = blk0;
    }
    __syncthreads();
    const int marked = count;
    for (int li = 0; li < marked; ++li) {
      const BlockInfo b = block_info(p, list[li]);
      const uint8_t* wexp = p.wq + (int64_t)b.expert * p.wq_stride;
      const uint16_t* sexp = p.ws + (int64_t)b.expert * p.ws_stride;
      // this thread's token-tile share: slot ts, 16-byte parts 4*tq .. 4*tq + 3
      const int ts = (int)threadIdx.x >> 2, tq = (int)threadIdx.x & 3;
      const int64_t tar = act_row_of<STAGE>(slot_rowid(p, b, ts, tk), tk, p.topk);
      for (int tile = 0; tile < p.n_tiles; ++tile) {
        const int n0 = STAGE == 1 ? tile * 128 : tile * 256;
        const int p0 = tile * 8 + 2 * wave;
        f32x4 acc[R][C];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int ct = 0; ct < C; ++ct) acc[r][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int g = 0; g < groups; ++g) {
          __syncthreads();  // the previous group's tile has been read
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int part = 4 * tq + e;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (tar >= 0) v = load16(p.act + tar * p.k_dim + g * kGroup + part * 8);
            *reinterpret_cast<u32x4*>(&xs[ts * 256 + part * 16]) = v;
          }
          if (threadIdx.x < kPfSlots) {
            const int64_t ar = act_row_of<STAGE>(slot_rowid(p, b, (int)threadIdx.x, tk), tk, p.topk);
            xsum_s[threadIdx.x] = ar >= 0 ? p.act_sum[ar * groups + g] : 0.0f;
          }
          __syncthreads();
          f32x4 part[R][C];
#pragma unroll
          for (int ct = 0; ct < C; ++ct) {
            const float nc = xsum_s[ct * 16 + sw];
#pragma unroll
            for (int r = 0; r < R; ++r) part[r][ct] = f32x4{nc, nc, nc, nc};
          }
          u32x4 wv[R];
          float sc[R][4];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int pair = p0 + (r >> 1);
            wv[r] = load16(wexp + ((int64_t)(pair * groups + g) * 2 + (r & 1)) * kTileBytes + lane * 16);
            const uint16_t* sp = sexp + (int64_t)(pair * groups + g) * 32 + 8 * (lane >> 4) + 4 * (r & 1);
            scale4(*reinterpret_cast<const u32x2*>(sp), sc[r]);
          }
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            bf16x8 bfr[C];
#pragma unroll
            for (int ct = 0; ct < C; ++ct)
              bfr[ct] = __builtin_bit_cast(
                  bf16x8, *reinterpret_cast<const u32x4*>(&xs[(ct * 16 + sw) * 256 + (4 * d + (lane >> 4)) * 16]));
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const bf16x8 a = dequant_biased(wv[r][d], magic);
#pragma unroll
              for (int ct = 0; ct < C; ++ct) part[r][ct] = mfma_bf16(a, bfr[ct], part[r][ct]);
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int ct = 0; ct < C; ++ct)
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[r][ct][i] = __builtin_fmaf(sc[r][i], part[r][ct][i], acc[r][ct][i]);
        }

        if constexpr (STAGE == 1) {
          const float lim = p.clamp_limit;
#pragma unroll
          for (int ct = 0; ct < C; ++ct) {
            const int64_t rowid = slot_rowid(p, b, ct * 16 + sw, tk);
            float partsum = 0.0f;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
              uint32_t bits[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                float gt = acc[2 * s2][ct][i];
                float up = acc[2 * s2 + 1][ct][i];
                if (lim > 0.0f) {
                  gt = fminf(gt, lim);
                  up = fminf(fmaxf(up, -lim), lim);
                }
                bits[i] = float_to_bf16_bits(silu_rcp(gt) * up);
                partsum += __uint_as_float(bits[i] << 16);
              }
              if (rowid >= 0) {
                const int n = n0 + 32 * wave + 16 * s2 + 4 * (lane >> 4);
                *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) =
                    u32x2{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
              }
            }
            partsum += __shfl_xor(partsum, 16, 64);
            partsum += __shfl_xor(partsum, 32, 64);
            if (lane < 16) red[wave][ct * 16 + lane] = partsum;
          }
          __syncthreads();
          if (threadIdx.x < C * 16) {
            const int col = (int)threadIdx.x;
            const int64_t rid = slot_rowid(p, b, col, tk);
            if (rid >= 0) {
              const float lo = red[0][col] + red[1][col];
              const float hi = red[2][col] + red[3][col];
              p.hsum_out[rid * (p.inter / kGroup) + n0 / kGroup] = -kDequantBias * (lo + hi);
            }
          }
        } else {
#pragma unroll
          for (int ct = 0; ct < C; ++ct) {
            const int64_t rowid = slot_rowid(p, b, ct * 16 + sw, tk);
            if (rowid < 0) continue;
            const float wr = contrib_weight(p, b, rowid, tk);
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const int n = n0 + 64 * wave + 16 * r + 4 * (lane >> 4);
              f32x4 v = acc[r][ct];
              v[0] *= wr; v[1] *= wr; v[2] *= wr; v[3] *= wr;
              *reinterpret_cast<f32x4*>(p.contrib + rowid * p.out_cols + n) = v;
            }
          }
        }
      }
    }
    __syncthreads();  // everyone is done with `list` and `count`
  }
}

// Per-row fp32 sums of bf16 activations over each 64-wide K chunk, summed in
// ascending k order.
// NC = false: out[r][c] = sum of x[r][64c .. 64c+63] (the decode kernels'
// form); NC = true: out[r][g] = -136 * (sum of the first 64 + sum of the last
// 64 columns of group g), each half summed as in the first form (the
// prefill kernels' form, as row_nc_part).
template <bool NC>
__global__ __launch_bounds__(256) void row_chunk_sum_kernel(const uint16_t* __restrict__ x,
                                                            int64_t rows, int k_dim,
                                                            float* __restrict__ out) {
  constexpr int kHalves = NC ? 2 : 1;
  const int chunks = k_dim / (kSumChunk * kHalves);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * chunks) return;
  const int64_t r = idx / chunks;
  const int c = (int)(idx % chunks);
  const uint16_t* src = x + r * k_dim + c * kSumChunk * kHalves;
  float half[kHalves];
#pragma unroll
  for (int h = 0; h < kHalves; ++h) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < kSumChunk; e += 8) {
      const u32x4 v = load16(src + h * kSumChunk + e);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s += __uint_as_float(v[q] << 16);
        s += __uint_as_float(v[q] & 0xFFFF0000u);
      }
    }
    half[h] = s;
  }
  if constexpr (NC)
    out[idx] = -kDequantBias * (half[0] + half[1]);
  else
    out[idx] = half[0];
}

// out[t][n] = bf16( sum_{j<k} contrib[t*k+j][n] + contrib[T*k+t][n] ).  The
// contributions are read once: nontemporal loads (T=8192: 195 -> 156 us).
// Up to kCombineBatch loads are issued before the first add instead of a
// loop of load, wait, add; the adds keep the slot order, so the result is the
// same bits.  Measured gain is small (T=64: 7.0 -> 6.7 us, against a ~6.4 us
// floor at T=1; T=8192 unchanged).
// An alignment that reports a negative padded count (the alignment kernel's
// answer to a route id outside [0, experts)) ran no routed block, so the
// contributions were never written: every output is NaN instead.
constexpr int kCombineBatch = 8;
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ contrib,
                                                      const int32_t* __restrict__ ntpp,
                                                      int64_t tokens, int topk, int hidden,
                                                      int has_shared, uint16_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int vec = hidden / 4;
  if (idx >= tokens * vec) return;
  const int64_t t = idx / vec;
  const int n = (int)(idx % vec) * 4;
  if (ntpp[0] < 0) {
    *reinterpret_cast<u32x2*>(out + t * hidden + n) = u32x2{0x7FC07FC0u, 0x7FC07FC0u};
    return;
  }
  const float* base = contrib + (t * topk) * hidden + n;
  f32x4 sh = {0.f, 0.f, 0.f, 0.f};
  if (has_shared)
    sh = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(contrib + (tokens * topk + t) * hidden + n));
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < topk; j0 += kCombineBatch) {
    f32x4 v[kCombineBatch];
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j)
      if (j0 + j < topk)
        v[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(base + (int64_t)(j0 + j) * hidden));
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) {
      if (j0 + j >= topk) break;
      if (j0 + j == 0) {
        s = v[0];
      } else {
        s[0] += v[j][0]; s[1] += v[j][1]; s[2] += v[j][2]; s[3] += v[j][3];
      }
    }
  }
  if (has_shared) {
    s[0] += sh[0]; s[1] += sh[1]; s[2] += sh[2]; s[3] += sh[3];
  }
  u32x2 o = {pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
  *reinterpret_cast<u32x2*>(out + t * hidden + n) = o;
}

}  // namespace dsv4

using namespace dsv4;


// Resident workgroups of a decode kernel on the current device (CUs x
// occupancy), cached per device: the persistent grid size.
template <int STAGE, int RING, bool PAIR>
static int decode_resident_grid() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, expert_decode_kernel<STAGE, RING, PAIR>, 256, 0) !=
            hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    cache[dev] = cus * per_cu;
  }
  return cache[dev];
}

// The decode launch of one stage: with at most one item per CU the K-split
// kernel (one item per workgroup); else the deep-ring kernel for stage 1,
// and for stage 2 when every item fits in one wave of resident workgroups,
// when K allows it; else the four-workgroups-per-CU kernel.  Either
// persistent grid is at most one wave of resident workgroups.  `blocks`
// bounds the active blocks (the kernels read the real count from the
// alignment on the device).
// Compute units of the current device, cached per device.
static int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

template <int STAGE, bool PAIR>
static void launch_decode_as(const ExpertGemmParams& p, int blocks, hipStream_t stream) {
  const int items = p.n_tiles * blocks;
  if (!PAIR && (p.k_dim / kGroup) % 16 == 0 && items <= device_cus()) {
    // at most one item per CU: eight wavefronts per item, K split in two,
    // each half's activations resident in LDS when they fit
    if (p.k_dim / kGroup / 2 <= kKsplitResidentGroups)
      hipLaunchKernelGGL((expert_decode_ksplit_kernel<STAGE, true>), dim3((unsigned)items), dim3(512), 0, stream, p);
    else
      hipLaunchKernelGGL((expert_decode_ksplit_kernel<STAGE, false>), dim3((unsigned)items), dim3(512), 0, stream, p);
    return;
  }
  if ((p.k_dim / kGroup) % 8 == 0 && (STAGE == 1 || items <= decode_resident_grid<STAGE, 8, PAIR>())) {
    const int grid = std::min(items, decode_resident_grid<STAGE, 8, PAIR>());
    hipLaunchKernelGGL((expert_decode_kernel<STAGE, 8, PAIR>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  } else {
    const int grid = std::min(items, decode_resident_grid<STAGE, 4, PAIR>());
    hipLaunchKernelGGL((expert_decode_kernel<STAGE, 4, PAIR>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  }
}

template <int STAGE>
static void launch_decode(const ExpertGemmParams& p, int blocks, hipStream_t stream) {
  if (decode_pairs(p)) launch_decode_as<STAGE, true>(p, blocks, stream);
  else launch_decode_as<STAGE, false>(p, blocks, stream);
}

size_t dsv4_experts_workspace_bytes(int64_t tokens, int topk, int hidden, int inter,
                                    int has_shared) {
  return carve_workspace(nullptr, tokens, topk, hidden, inter, has_shared).bytes;
}

// The activation row sums inside an experts workspace (written by the
// prologue launch when the caller fuses them there).
float* dsv4_experts_xsum(void* workspace, int64_t tokens, int topk, int hidden, int inter, int has_shared) {
  return carve_workspace(workspace, tokens, topk, hidden, inter, has_shared).xsum;
}

// Scratch for an alignment that runs before the experts: the contribution
// region, which the experts path writes only after it has read the alignment.
int32_t* dsv4_experts_align_scratch(void* workspace, int64_t tokens, int topk, int hidden, int inter,
                                    int has_shared, size_t* bytes) {
  const ExpertWorkspace w = carve_workspace(workspace, tokens, topk, hidden, inter, has_shared);
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);
  *bytes = sizeof(float) * (size_t)rows * hidden;
  return reinterpret_cast<int32_t*>(w.contrib);
}

int dsv4_launch_experts_w4a16(const uint16_t* x, int64_t tokens, int hidden, int inter,
                              int experts, int topk, const uint8_t* w13q, const uint16_t* w13s,
                              const uint8_t* w2q, const uint16_t* w2s, const float* w13r, const float* w2r,
                              int has_shared,
                              const float* weights, const int32_t* sorted, int64_t capacity,
                              const int32_t* expert_ids, const int32_t* ntpp, int block_size,
                              float clamp_limit, uint16_t* out, void* workspace,
                              hipStream_t stream, bool rowsums_ready) {
  if (tokens == 0) return DSV4MOE_OK;
  ExpertWorkspace ws = carve_workspace(workspace, tokens, topk, hidden, inter, has_shared);
  const int max_blocks = (int)((capacity + block_size - 1) / block_size);
  // decode kernel: blocks of <= 16 slots and K groups in multiples of 4
  const bool decode = w4a16_decode_path(block_size, hidden, inter);
  const int shared_bs = decode ? 16 : block_size;
  const int shared_blocks = has_shared ? (int)((tokens + shared_bs - 1) / shared_bs) : 0;
  const int blocks = max_blocks + shared_blocks;
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);

  if (!rowsums_ready) {
    // the activation sums in the form the chosen kernels read
    const int64_t n = tokens * (hidden / (decode ? kSumChunk : kGroup));
    if (decode)
      hipLaunchKernelGGL(row_chunk_sum_kernel<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                         stream, x, tokens, hidden, ws.xsum);
    else
      hipLaunchKernelGGL(row_chunk_sum_kernel<true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                         stream, x, tokens, hidden, ws.xsum);
    DSV4_CHECK_LAUNCH("row_chunk_sum_kernel");
  }
  dsv4host::prof_stamp(dsv4host::kStampRowSum, stream);
  ExpertGemmParams p{};
  p.sorted = sorted;
  p.expert_ids = expert_ids;
  p.ntpp = ntpp;
  p.block_size = block_size;
  p.shared_block_size = shared_bs;
  p.max_blocks = max_blocks;
  p.full_blocks = (int)(capacity / block_size);
  p.experts = experts;
  p.tokens = tokens;
  p.topk = topk;
  p.shared_expert = has_shared ? experts : -1;
  p.clamp_limit = clamp_limit;
  p.inter = inter;

  // stage 1: W13 [2I, H]
  p.wq = w13q;
  p.ws = w13s;
  p.wr = w13r;
  p.wq_stride = (int64_t)2 * inter * hidden / 2;
  p.ws_stride = (int64_t)2 * inter * (hidden / kGroup);
  p.k_dim = hidden;
  p.act = x;
  p.act_rows = tokens;
  p.act_sum = ws.xsum;
  p.h_out = ws.h;
  p.hsum_out = ws.hsum;
  if (decode) {
    p.n_tiles = inter / 64;
    launch_decode<1>(p, blocks, stream);
  } else {
    p.n_tiles = inter / 128;
    hipLaunchKernelGGL(expert_prefill_kernel<1>, dim3((unsigned)prefill_grid(blocks, p.n_tiles)),
                       dim3(256), 0, stream, p, blocks);
    hipLaunchKernelGGL(expert_prefill_exact_kernel<1>, dim3((unsigned)kExactGrid), dim3(256), 0, stream, p,
                       blocks);
  }
  DSV4_CHECK_LAUNCH("expert stage 1");
  dsv4host::prof_stamp(dsv4host::kStampStage1, stream);

  // stage 2: W2 [H, I]
  p.wq = w2q;
  p.ws = w2s;
  p.wr = w2r;
  p.wq_stride = (int64_t)hidden * inter / 2;
  p.ws_stride = (int64_t)hidden * (inter / kGroup);
  p.k_dim = inter;
  p.act = ws.h;
  p.act_rows = rows;
  p.act_sum = ws.hsum;
  p.route_w = weights;
  p.contrib = ws.contrib;
  p.out_cols = hidden;
  if (decode) {
    p.n_tiles = hidden / 128;
    launch_decode<2>(p, blocks, stream);
  } else {
    p.n_tiles = hidden / 256;
    hipLaunchKernelGGL(expert_prefill_kernel<2>, dim3((unsigned)prefill_grid(blocks, p.n_tiles)),
                       dim3(256), 0, stream, p, blocks);
    hipLaunchKernelGGL(expert_prefill_exact_kernel<2>, dim3((unsigned)kExactGrid), dim3(256), 0, stream, p,
                       blocks);
  }
  DSV4_CHECK_LAUNCH("expert stage 2");
  dsv4host::prof_stamp(dsv4host::kStampStage2, stream);

  const int rc = dsv4_launch_combine(ws.contrib, ntpp, tokens, topk, hidden, has_shared, out, stream);
  if (rc != DSV4MOE_OK) return rc;
  dsv4host::prof_stamp(dsv4host::kStampCombine, stream);
  return DSV4MOE_OK;
}

int dsv4_launch_combine(const float* contrib, const int32_t* ntpp, int64_t tokens, int topk, int hidden,
                        int has_shared, uint16_t* out, hipStream_t stream) {
  const int64_t n = tokens * (hidden / 4);
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     contrib, ntpp, tokens, topk, hidden, has_shared, out);
  DSV4_CHECK_LAUNCH("combine_kernel");
  return DSV4MOE_OK;
}
