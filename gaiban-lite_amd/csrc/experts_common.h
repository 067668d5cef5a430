// Helpers shared by the bf16 (W4A16) and fp8 (W4A8) grouped expert kernels:
// kernel parameters, alignment-block decoding and slot -> row mapping.
#pragma once

#include "common.h"

namespace dsv4 {

constexpr int kSumChunk = 64;            // granularity of the activation row sums
constexpr uint32_t kOobOffset = 0x80000000u;  // buffer offset past every resource
constexpr int kRsrcFlags = 0x00020000;    // raw buffer, gfx950 dword3
constexpr int kXcds = 8;                  // XCDs; workgroup id i runs on XCD i % 8

struct ExpertGemmParams {
  const uint8_t* wq;     // tiled int4, expert-major
  const uint16_t* ws;    // tiled scales
  const float* wr;       // int4 prefill: fp32 ratios of consecutive group scales, same order (ws_stride per expert)
  int64_t wq_stride;     // bytes per expert
  int64_t ws_stride;     // scale elements per expert
  int k_dim;             // K of the weight matrix
  int inter;             // stage 1: first up-projection row
  const uint16_t* act;   // stage 1: x [T][H]; stage 2: h [rows][I]
  int64_t act_rows;      // rows of `act`
  const float* act_sum;  // [act_rows][k_dim/64] row sums of `act`
  const int32_t* sorted;
  const int32_t* expert_ids;
  const int32_t* ntpp;
  int block_size;
  int shared_block_size; // token slots per shared-expert block
  int max_blocks;        // ceil(capacity / block_size): routed blocks before the shared ones
  int full_blocks;       // capacity / block_size: routed blocks that lie inside `sorted`
  int experts;           // routed experts: a block expert id outside [0, experts) is poisoned
  int n_tiles;
  int64_t tokens;
  int topk;
  int shared_expert;     // expert index of the shared expert, -1 if none
  float clamp_limit;
  const float* route_w;  // stage 2: [T*k]
  uint16_t* h_out;       // stage 1: [rows][I]
  float* hsum_out;       // stage 1: [rows][I/64]
  float* contrib;        // stage 2: [rows][H]
  int out_cols;          // stage 2: H
  const float* act_scale;  // fp8 kernels: per-row activation scale [act_rows]
  const uint8_t* ws8;      // MXFP4 kernels: tiled E8M0 scales (ws_stride bytes per expert)
};

struct BlockInfo {
  int expert;
  int64_t slot_base;
  bool shared;
  bool active;
  bool poison;  // the alignment names no valid expert: results of this block are NaN
};

// The alignment comes from the caller (or a caller's provider), so it is not
// trusted for addressing: a routed block is active only below both the padded
// count and the blocks that fit the capacity, and an active block whose expert
// id is outside [0, experts) reads expert 0's weights (in bounds) and marks its
// stage-2 contributions NaN, so the damage shows in the output.
__device__ __forceinline__ BlockInfo block_info(const ExpertGemmParams& p, int blk) {
  BlockInfo b;
  b.shared = blk >= p.max_blocks;
  b.active = true;
  b.poison = false;
  if (!b.shared) {
    const int total = p.ntpp[0];
    b.active = total > 0 && blk < p.full_blocks && (int64_t)blk * p.block_size < total;
    const int e = b.active ? p.expert_ids[blk] : 0;
    b.poison = (unsigned)e >= (unsigned)p.experts;
    b.expert = b.poison ? 0 : e;
    b.slot_base = (int64_t)blk * p.block_size;
  } else {
    b.expert = p.shared_expert;
    b.slot_base = (int64_t)(blk - p.max_blocks) * p.shared_block_size;
  }
  return b;
}

// Stage-2 multiplier of a contribution row: the route weight (1 for the
// shared expert), NaN in a poisoned block.
__device__ __forceinline__ float contrib_weight(const ExpertGemmParams& p, const BlockInfo& b, int64_t rowid,
                                               int64_t tk) {
  const float w = rowid < tk ? p.route_w[rowid] : 1.0f;
  return b.poison ? __builtin_nanf("") : w;
}

// Row id (index into h / contrib) of token column `col` of a block, -1 if padded.
__device__ __forceinline__ int64_t slot_rowid(const ExpertGemmParams& p, const BlockInfo& b, int col,
                                              int64_t tk) {
  if (col >= (b.shared ? p.shared_block_size : p.block_size)) return -1;
  if (!b.shared) {
    const int32_t f = p.sorted[b.slot_base + col];
    return (f >= 0 && f < tk) ? (int64_t)f : -1;
  }
  const int64_t t = b.slot_base + col;
  return t < p.tokens ? tk + t : -1;
}

// As slot_rowid for a routed block taken together with the next block of the
// same expert (`routed_slots` = twice the block size; the two blocks' slots
// are contiguous in sorted_token_ids).
__device__ __forceinline__ int64_t slot_rowid_span(const ExpertGemmParams& p, const BlockInfo& b, int col,
                                                   int64_t tk, int routed_slots) {
  if (b.shared) return slot_rowid(p, b, col, tk);
  if (col >= routed_slots) return -1;
  const int32_t f = p.sorted[b.slot_base + col];
  return (f >= 0 && f < tk) ? (int64_t)f : -1;
}

// Pairing of 8-slot decode blocks (PAIR, chosen at launch by decode_pairs):
// consecutive blocks of one expert pair up from the start of the expert's run
// of blocks, and the first block of a pair takes both blocks' 16 slots as one
// item, so the expert's weights stream once for them; the second block's
// items are skipped.  The position in the run is counted back over at most
// kPairScan blocks; blocks further into a long run stay unpaired, which keeps
// the pairs consistent (a block pairs with the next only while both
// positions are below kPairScan).
constexpr int kPairScan = 16;

// Routed slots of decode block `bi` (< routed: a routed block): the block
// size, twice it when the block leads a pair, 0 when it is a pair's second
// block; shared-expert blocks (bi >= routed) keep their own size.
template <bool PAIR>
__device__ __forceinline__ int decode_block_span(const ExpertGemmParams& p, int bi, int routed) {
  if (!PAIR || bi >= routed) return p.block_size;
  const int e = p.expert_ids[bi];
  int pos = 0;
  while (pos < kPairScan && pos < bi && p.expert_ids[bi - pos - 1] == e) ++pos;
  if (pos < kPairScan && (pos & 1)) return 0;
  if (pos + 1 < kPairScan && bi + 1 < routed && p.expert_ids[bi + 1] == e) return 2 * p.block_size;
  return p.block_size;
}

// Pairs of 8-slot blocks pay off once an expert often holds more than one
// block (on average at least 4 of its slots per 8-slot block); below that the
// extra expert-id reads per item cost more than they save.
inline bool decode_pairs(const ExpertGemmParams& p) {
  return p.block_size == 8 && p.tokens * p.topk >= 4 * (int64_t)p.experts;
}

template <int STAGE>
__device__ __forceinline__ int64_t act_row_of(int64_t rowid, int64_t tk, int topk) {
  if (rowid < 0) return -1;
  if (STAGE == 1) return rowid < tk ? (int64_t)((uint32_t)rowid / (uint32_t)topk) : rowid - tk;
  return rowid;
}

__device__ __forceinline__ void scale4(u32x2 sv, float (&sc)[4]) {
  sc[0] = __uint_as_float(sv[0] << 16);
  sc[1] = __uint_as_float(sv[0] & 0xFFFF0000u);
  sc[2] = __uint_as_float(sv[1] << 16);
  sc[3] = __uint_as_float(sv[1] & 0xFFFF0000u);
}

// Persistent decode kernels: active items (block, tile) are the shared-expert
// blocks and the routed blocks below ceil(ntpp / block_size), times the N
// tiles (order: decode_item_block).
__device__ __forceinline__ int decode_routed_blocks(const ExpertGemmParams& p) {
  const int total = p.ntpp[0];
  const int blocks = total > 0 ? (total + p.block_size - 1) / p.block_size : 0;
  return blocks < p.full_blocks ? blocks : p.full_blocks;
}

__device__ __forceinline__ int decode_shared_blocks(const ExpertGemmParams& p) {
  return p.shared_expert >= 0 ? (int)((p.tokens + p.shared_block_size - 1) / p.shared_block_size) : 0;
}

__device__ __forceinline__ int decode_items(const ExpertGemmParams& p, int routed) {
  return (routed + decode_shared_blocks(p)) * p.n_tiles;
}

// Block index bi (< routed: a routed block; routed + s: shared-expert block s)
// and N tile of decode item `item`: the S shared-expert blocks' items first,
// then the routed blocks', each block's n_tiles items in tile order.  The
// dispatcher sends workgroup i to XCD i % 8 and the persistent grid is a
// multiple of 8 (or covers every item), so item i runs on XCD i % 8; with
// n_tiles a multiple of 8 the S items of one shared-expert tile run on one
// XCD, in the first round of the persistent loop when S * n_tiles fits the
// grid, and stream that tile's weights through the XCD's L2 together.
__device__ __forceinline__ void decode_item_block(const ExpertGemmParams& p, int item, int routed, int& bi,
                                                  int& tile) {
  const int S = decode_shared_blocks(p);
  const int b = item / p.n_tiles;
  tile = item - b * p.n_tiles;
  bi = b < S ? routed + b : b - S;
}

// Workgroup stride over the items: the whole grid.  (Shrinking the grid so
// that the last round is full was measured slower: fewer workgroups keep
// fewer bytes in flight, which costs more than the partial last round.)
__device__ __forceinline__ int decode_stride(int) { return (int)gridDim.x; }

// Prefill work order.  Items are (alignment block, N tile).  Consecutive
// blocks, which mostly belong to the same expert, form groups of kBlkGroup;
// a group's items run tile by tile, so its workgroups stream the same weight
// tile together and its token rows stay in one L2.  The dispatcher sends
// workgroup id i to XCD i % 8; groups are dealt to the XCDs round-robin
// (group g on XCD g % 8), which keeps the XCDs balanced when the active
// blocks, the padding blocks and the shared-expert blocks sit in different
// parts of the block list.
constexpr int kBlkGroup = 4;

__host__ __device__ __forceinline__ int prefill_grid(int total_blocks, int n_tiles) {
  const int groups = (total_blocks + kBlkGroup - 1) / kBlkGroup;
  return (groups + kXcds - 1) / kXcds * kBlkGroup * n_tiles * kXcds;
}

__device__ __forceinline__ bool prefill_item(int n_tiles, int total_blocks, int& blk, int& tile) {
  const int xcd = (int)(blockIdx.x % kXcds);
  const int j = (int)(blockIdx.x / kXcds);
  const int span = kBlkGroup * n_tiles;
  const int g = (j / span) * kXcds + xcd;
  const int rem = j % span;
  tile = rem / kBlkGroup;
  blk = g * kBlkGroup + rem % kBlkGroup;
  return blk < total_blocks;
}

}  // namespace dsv4

// Workspace of the expert launchers (caller-owned, 256-byte aligned pieces):
// x row sums per 64 columns, h bf16 [rows][I], h row sums, fp32
// contributions [rows][H]; rows = T*k (+ T with the shared expert).
struct ExpertWorkspace {
  float* xsum;
  uint16_t* h;
  float* hsum;
  float* contrib;
  size_t bytes;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline ExpertWorkspace carve_workspace(void* base, int64_t tokens, int topk, int hidden, int inter,
                                       int has_shared) {
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);
  size_t off = 0;
  ExpertWorkspace w;
  char* b = static_cast<char*>(base);
  w.xsum = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)tokens * (hidden / dsv4::kSumChunk));
  w.h = reinterpret_cast<uint16_t*>(b + off);
  off += align256(sizeof(uint16_t) * (size_t)rows * inter);
  w.hsum = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)rows * (inter / dsv4::kSumChunk));
  w.contrib = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)rows * hidden);
  w.bytes = off;
  return w;
}

// Workspace of the W4A8 launchers (caller-owned, 256-byte aligned pieces):
// e4m3 x and its per-row scales and per-128-K sums, h bf16, e4m3 h with its
// scales and sums, fp32 contributions.  The MXFP4 W4A8 path carves the same
// pieces and leaves the sums unused.
struct Fp8Workspace {
  uint8_t* xq;
  float* xscale;
  float* xsum;
  uint16_t* h;
  uint8_t* hq;
  float* hscale;
  float* hsum;
  float* contrib;
  size_t bytes;
};

inline Fp8Workspace carve_fp8(void* base, int64_t tokens, int topk, int hidden, int inter, int has_shared) {
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);
  char* b = static_cast<char*>(base);
  size_t off = 0;
  Fp8Workspace w;
  w.xq = reinterpret_cast<uint8_t*>(b + off);
  off += align256((size_t)tokens * hidden);
  w.xscale = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)tokens);
  w.xsum = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)tokens * (hidden / dsv4::kGroup));
  w.h = reinterpret_cast<uint16_t*>(b + off);
  off += align256(sizeof(uint16_t) * (size_t)rows * inter);
  w.hq = reinterpret_cast<uint8_t*>(b + off);
  off += align256((size_t)rows * inter);
  w.hscale = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)rows);
  w.hsum = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)rows * (inter / dsv4::kGroup));
  w.contrib = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)rows * hidden);
  w.bytes = off;
  return w;
}

// Host launchers shared by the expert paths (experts.hip).
int dsv4_launch_combine(const float* contrib, const int32_t* ntpp, int64_t tokens, int topk, int hidden,
                        int has_shared, uint16_t* out, hipStream_t stream);
