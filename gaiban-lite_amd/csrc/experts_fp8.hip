// W4A8: grouped int4 expert GEMMs on the gfx950 fp8 MFMA (16x16x128 f8f6f4).
//
// Restates vLLM's _fused_marlin_moe with input_dtype = float8_e4m3fn as
// configured at runtime/dsv4_direct/moe_runtime.py:207-235,1829-1856: the
// expert inputs (x for stage 1, the bf16 SwiGLU output h for stage 2) are
// quantised per row to OCP e4m3 with s = max(amax, 1e-12) / 448 and
// q = e4m3(clamp(v / s, -448, 448)); the products accumulate in fp32 and the
// row scale multiplies the result.
//
// int4 weights enter the fp8 MFMA without a lookup: the offset-binary nibble
// u = q + 8 (0..15) placed in a byte is the e4m3 encoding of u * 2^-9 (bytes
// 0..7 are subnormals m * 2^-9, bytes 8..15 are (8 + m) * 2^-9).  Per
// quantisation group g of weight row n and activation row t the MFMA gives
// 2^-9 * sum(u * xq); minus sum_g(xq) / 64 that is 2^-9 * sum(q * xq) (the
// decode kernel starts the MFMA from -sum_g(xq) / 64, the prefill kernel
// subtracts it afterwards); the kernels add s[n, g] times that and the
// epilogue multiplies by 512 * s_row, which equals
// s_row * sum_g s[n, g] * sum(q * xq).
//
// Operand layout: a lane of the 16x16x128 MFMA holds 32 K values of one row
// (A) or column (B) in 8 dwords; both operands assign K values to (lane group,
// byte) the same way, so any fixed assignment gives the dot product.  The
// tiled int4 weights expand, per 16-byte lane chunk, dword d (8 nibbles, K
// k0 = 32d + 8j .. +7, slots as in the bf16 path) into the byte dwords
// (w & 0x0F0F0F0F, (w >> 4) & 0x0F0F0F0F) = K k0 + {0,4,1,5}, k0 + {2,6,3,7}.
// The activation quantiser writes each 128-K group in exactly that order: 32
// bytes per lane group j, dword pair d holding K 32d + 8j + {0,4,1,5,2,6,3,7}.
#include <algorithm>
#include <type_traits>

#include "act_quant.h"
#include "experts_common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

typedef __attribute__((ext_vector_type(8))) int i32x8;

__device__ __forceinline__ f32x4 mfma_fp8(i32x8 a, i32x8 b, f32x4 c) {
  // unit E8M0 block scales (127 = 2^0)
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// 16 bytes of tiled int4 (32 nibbles) -> 32 e4m3 bytes of u * 2^-9.
__device__ __forceinline__ i32x8 spread_nibbles(u32x4 w) {
  i32x8 a;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    a[2 * d] = (int)(w[d] & 0x0F0F0F0Fu);
    a[2 * d + 1] = (int)((w[d] >> 4) & 0x0F0F0F0Fu);
  }
  return a;
}

constexpr float kInvSum = 1.0f / 64.0f;  // 8 * 2^-9
constexpr float kUnScale = 512.0f;       // 2^9

// ------------------------------------------------------------ activation quant
// One wavefront per row (act_quant_row, act_quant.h), four rows per workgroup.
template <bool NATURAL>
__global__ __launch_bounds__(256) void act_quant_fp8_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                            int k, uint8_t* __restrict__ q,
                                                            float* __restrict__ scale,
                                                            float* __restrict__ gsum) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  act_quant_row<NATURAL>(x, row, k, q, scale, gsum);
}

// ------------------------------------------------------------------ decode
// Persistent, like the bf16 decode kernel: workgroup w takes items w, w +
// stride, ... of the active (block, tile) items, and the K stream (weights two
// groups ahead, activations one group ahead) runs on across item boundaries.
// Wavefront w streams strip pair tile*4 + w (stage 1: gate + up strip, h
// columns n0 + 16w ..; stage 2: strips (n0 + 32w)/16 + {0, 1}).  The 16 slots
// x 128 B of the current group are staged in LDS (part q of slot s at
// q ^ swz128(s)); the loader threads of slots 16..31 fill unused landing rows.

struct Fp8DecodeItem {
  const uint8_t* wq;
  const uint16_t* ws;
  uint32_t ld_base;   // loader thread: activation byte offset of its slot (or out of range)
  uint32_t sum_base;  // lane: group-sum offset of its slot (or out of range)
  int64_t rowid;      // lane: row id of its slot, -1 if padded
  int64_t arow;       // lane: activation row of its slot, -1 if padded
  int n0;
  float wmul;          // 1, or NaN when the block names no valid expert (stage-2 multiplier)
};

template <int STAGE>
__device__ __forceinline__ Fp8DecodeItem fp8_decode_item(const ExpertGemmParams& p, int item, int routed,
                                                         int64_t tk) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int bi, tile;
  decode_item_block(p, item, routed, bi, tile);
  const int blk = bi < routed ? bi : p.max_blocks + (bi - routed);
  const BlockInfo b = block_info(p, blk);
  const int groups = p.k_dim / kGroup;
  Fp8DecodeItem it;
  it.n0 = STAGE == 1 ? tile * 64 : tile * 128;
  const int pair = tile * 4 + wave;
  it.wq = p.wq + (int64_t)b.expert * p.wq_stride + (int64_t)pair * groups * 2048 + lane * 16;
  it.ws = p.ws + (int64_t)b.expert * p.ws_stride + (int64_t)pair * groups * 32 + 8 * (lane >> 4);
  it.wmul = b.poison ? __builtin_nanf("") : 1.0f;
  it.rowid = slot_rowid(p, b, lane & 15, tk);
  it.arow = act_row_of<STAGE>(it.rowid, tk, p.topk);
  it.sum_base = it.arow >= 0 ? (uint32_t)(it.arow * groups * 4) : kOobOffset;
  const int ld_slot = threadIdx.x >> 3;
  const int64_t ld_row =
      ld_slot < 16 ? act_row_of<STAGE>(slot_rowid(p, b, ld_slot, tk), tk, p.topk) : (int64_t)-1;
  it.ld_base = ld_row >= 0 ? (uint32_t)(ld_row * p.k_dim + (threadIdx.x & 7) * 16) : kOobOffset;
  return it;
}

template <int STAGE>
__global__ __launch_bounds__(256, 4) void expert_fp8_decode_kernel(ExpertGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][32 * 128];  // rows 16..31: unused landing rows
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t tk = p.tokens * p.topk;
  const int routed = decode_routed_blocks(p);
  const int n_items = decode_items(p, routed);
  const int stride = decode_stride(n_items);
  int item = blockIdx.x;
  if (item >= stride || item >= n_items) return;  // uniform per workgroup
  const int groups = p.k_dim / kGroup;

  const uint8_t* act = reinterpret_cast<const uint8_t*>(p.act);
  const __amdgpu_buffer_rsrc_t act_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)act, (short)0, (int)(p.act_rows * p.k_dim), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t sum_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act_sum, (short)0, (int)(p.act_rows * groups * 4), kRsrcFlags);
  const int ld_slot = threadIdx.x >> 3;
  const int ld_lds = ld_slot * 128 + (((threadIdx.x & 7) ^ swz128(ld_slot)) * 16);
  const int rd_lds0 = (lane & 15) * 128 + (((2 * (lane >> 4)) ^ swz128(lane & 15)) * 16);
  const int rd_lds1 = (lane & 15) * 128 + (((2 * (lane >> 4) + 1) ^ swz128(lane & 15)) * 16);

  Fp8DecodeItem cur = fp8_decode_item<STAGE>(p, item, routed, tk);
  int next = item + stride;
  Fp8DecodeItem nxt = next < n_items ? fp8_decode_item<STAGE>(p, next, routed, tk) : cur;

  u32x4 W[4][2];
  u32x4 S[4];
  float CS[2];
  u32x4 xr;
  auto issue_w = [&](const Fp8DecodeItem& it, int g, u32x4 (&w)[2], u32x4& s) {
    w[0] = load16_nt(it.wq + g * 2048);
    w[1] = load16_nt(it.wq + g * 2048 + 1024);
    s = load16(it.ws + g * 32);
  };
  auto issue_x = [&](const Fp8DecodeItem& it, int g, float& cs) {
    xr = __builtin_amdgcn_raw_buffer_load_b128(act_rsrc, it.ld_base + (uint32_t)(g * 128), 0, 0);
    cs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sum_rsrc, it.sum_base + (uint32_t)(g * 4), 0, 0));
  };

  issue_x(cur, 0, CS[0]);
  issue_w(cur, 0, W[0], S[0]);
  issue_w(cur, 1, W[1], S[1]);
  *reinterpret_cast<u32x4*>(&xs[0][ld_lds]) = xr;
  __syncthreads();

  for (;;) {
    f32x4 acc[2];
    acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < groups; g0 += 4) {  // groups % 4 == 0 (checked on the host)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int g = g0 + u;
        const bool xn = g + 1 >= groups;
        issue_x(xn ? nxt : cur, xn ? 0 : g + 1, CS[(u + 1) & 1]);
        const bool wn = g + 2 >= groups;
        issue_w(wn ? nxt : cur, wn ? g + 2 - groups : g + 2, W[(u + 2) & 3], S[(u + 2) & 3]);
        const u32x4 b0 = *reinterpret_cast<const u32x4*>(&xs[u & 1][rd_lds0]);
        const u32x4 b1 = *reinterpret_cast<const u32x4*>(&xs[u & 1][rd_lds1]);
        const i32x8 bf = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                          (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
        const float nc = -CS[u & 1] * kInvSum;
        const f32x4 init = {nc, nc, nc, nc};
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const f32x4 tmp = mfma_fp8(spread_nibbles(W[u][r]), bf, init);
          float sc[4];
          scale4(u32x2{S[u][2 * r], S[u][2 * r + 1]}, sc);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[r][i] += sc[i] * tmp[i];
        }
        *reinterpret_cast<u32x4*>(&xs[(u + 1) & 1][ld_lds]) = xr;
        __syncthreads();
      }
    }

    const int64_t rowid = cur.rowid;
    if (rowid >= 0) {
      const float mult = kUnScale * p.act_scale[cur.arow];
      if constexpr (STAGE == 1) {
        const float lim = p.clamp_limit;
        uint32_t bits[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float gt = acc[0][i] * mult;
          float up = acc[1][i] * mult;
          if (lim > 0.0f) {
            gt = fminf(gt, lim);
            up = fminf(fmaxf(up, -lim), lim);
          }
          bits[i] = float_to_bf16_bits(silu_f(gt) * up);
        }
        const int n = cur.n0 + 16 * wave + 4 * (lane >> 4);
        *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) =
            u32x2{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
      } else {
        const float wm = (rowid < tk ? p.route_w[rowid] : 1.0f) * cur.wmul * mult;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int n = cur.n0 + 32 * wave + 16 * r + 4 * (lane >> 4);
          const f32x4 v = {acc[r][0] * wm, acc[r][1] * wm, acc[r][2] * wm, acc[r][3] * wm};
          *reinterpret_cast<f32x4*>(p.contrib + rowid * p.out_cols + n) = v;
        }
      }
    }
    if (next >= n_items) break;  // uniform per workgroup; the last prefetches re-read cur
    item = next;
    cur = nxt;
    next = item + stride;
    nxt = next < n_items ? fp8_decode_item<STAGE>(p, next, routed, tk) : cur;
  }
}

// ----------------------------------------------------------------- prefill
// Blocks of up to 64 slots: workgroup tile 64 slots x 256 weight rows, the
// same strip assignment and work order as the bf16 prefill kernel.  Per
// group the 64 x 128 B token tile (16-byte part q of slot s at q ^ swz128(s)),
// the slots' group sums and each wavefront's 4 weight tiles and scales are
// copied into LDS by buffer_load ... lds in a three-buffer ring, two groups
// ahead of the compute (76 KiB per workgroup: still two per CU; one group of
// 16 MFMAs per wavefront is too short to cover a copy issued one group ahead).
constexpr int kF8Slots = 64;

template <int STAGE>
__global__ __launch_bounds__(256, 2) void expert_fp8_prefill_kernel(ExpertGemmParams p, int total_blocks) {
  constexpr int R = 4;
  constexpr int C = 4;
  __shared__ __attribute__((aligned(16))) uint8_t xs[3][kF8Slots * 128];
  __shared__ __attribute__((aligned(16))) uint8_t wts[3][4][R * kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t scl[3][4][256];
  __shared__ float xsum[3][kF8Slots];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  int blk, tile;
  if (!prefill_item(p.n_tiles, total_blocks, blk, tile)) return;
  const int64_t tk = p.tokens * p.topk;
  const BlockInfo b = block_info(p, blk);
  if (!b.active) return;

  const int groups = p.k_dim / kGroup;
  const int n0 = STAGE == 1 ? tile * 128 : tile * 256;
  const int p0 = tile * 8 + 2 * wave;

  const uint8_t* act = reinterpret_cast<const uint8_t*>(p.act);
  const __amdgpu_buffer_rsrc_t act_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)act, (short)0, (int)(p.act_rows * p.k_dim), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t sum_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act_sum, (short)0, (int)(p.act_rows * groups * 4), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.wq + (int64_t)b.expert * p.wq_stride), (short)0, (int)p.wq_stride, kRsrcFlags);
  const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.ws + (int64_t)b.expert * p.ws_stride), (short)0, (int)(p.ws_stride * 2), kRsrcFlags);

  // token tile: DMA q (0..1) of wave w fills slots 16w + 8q + lane/8
  uint32_t dma_off[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = 16 * wave + 8 * q + (lane >> 3);
    const int64_t ar = act_row_of<STAGE>(slot_rowid(p, b, row, tk), tk, p.topk);
    const int part = (lane & 7) ^ swz128(row);
    dma_off[q] = ar >= 0 ? (uint32_t)(ar * p.k_dim + part * 16) : kOobOffset;
  }
  uint32_t sum_off = kOobOffset;
  if (wave == 0) {
    const int64_t ar = act_row_of<STAGE>(slot_rowid(p, b, lane, tk), tk, p.topk);
    if (ar >= 0) sum_off = (uint32_t)(ar * groups * 4);
  }
  const uint32_t w_off0 = (uint32_t)(p0 * groups) * 2048 + lane * 16;
  const uint32_t w_off1 = (uint32_t)((p0 + 1) * groups) * 2048 + lane * 16;
  const uint32_t s_off = lane < 32 ? (uint32_t)((p0 + (lane >> 4)) * groups) * 64 + (lane & 15) * 4 : kOobOffset;

  // LDS copies of group g into buffer `buf` (inline-asm DMA, waited for
  // explicitly before the barrier that ends each step).  The destinations
  // are this wavefront's buffer-0 addresses, made scalar once here, plus
  // constant offsets, so the K loop sets M0 with scalar adds only.
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][16 * wave * 128]));
  const uint32_t wts_lds = __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][wave][0]));
  const uint32_t scl_lds = __builtin_amdgcn_readfirstlane(lds_addr(&scl[0][wave][0]));
  const uint32_t xsum_lds = lds_addr(&xsum[0][0]);
  auto issue = [&](int g, int buf) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      lds_copy16(act_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + q * 1024, dma_off[q], g * 128);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      lds_copy16(w_rsrc, wts_lds + buf * (uint32_t)sizeof(wts[0]) + t * kTileBytes,
                 (t < 2 ? w_off0 : w_off1) + (t & 1) * kTileBytes, g * 2048);
    lds_copy4(s_rsrc, scl_lds + buf * (uint32_t)sizeof(scl[0]), s_off, g * 64);
    if (wave == 0) lds_copy4(sum_rsrc, xsum_lds + buf * (uint32_t)sizeof(xsum[0]), sum_off, g * 4);
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int ct = 0; ct < C; ++ct) acc[r][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int sw = lane & 15;
  const int jg = lane >> 4;
  // copies one issue() makes per wavefront (wave 0 also the activation sums)
  constexpr int kLoads = 2 + 4 + 1;
  auto wait_step = [&]() {
    if (wave == 0) lds_dma_wait_keep<kLoads + 1>();
    else lds_dma_wait_keep<kLoads>();
  };
  // Step g: copy group g + 2 into buffer (u + 2) % 3 (released by step g - 1's
  // barrier), compute group g from buffer u, wait for group g + 1.
  auto step = [&](int g, auto u_c) {
    constexpr int u = decltype(u_c)::value;
    const bool issue2 = g + 2 < groups;
    if (issue2) issue(g + 2, (u + 2) % 3);
    i32x8 bfr[C];
#pragma unroll
    for (int ct = 0; ct < C; ++ct) {
      const int row = ct * 16 + sw;
      const u32x4 b0 = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + ((2 * jg) ^ swz128(row)) * 16]);
      const u32x4 b1 = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + ((2 * jg + 1) ^ swz128(row)) * 16]);
      bfr[ct] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    }
    // the MFMA starts from -sum_g(xq) / 64 of the lane's token (its four
    // outputs are four weight rows of one token), so one FMA per output
    // applies the group scale: acc += s * (2^-9 sum(u * xq) - sum_g(xq) / 64)
    f32x4 negcorr[C];
#pragma unroll
    for (int ct = 0; ct < C; ++ct) {
      const float c = -xsum[u][ct * 16 + sw] * kInvSum;
      negcorr[ct] = f32x4{c, c, c, c};
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const i32x8 a = spread_nibbles(*reinterpret_cast<const u32x4*>(&wts[u][wave][r * kTileBytes + lane * 16]));
      const u32x2 sv = *reinterpret_cast<const u32x2*>(&scl[u][wave][(r >> 1) * 64 + 16 * jg + 8 * (r & 1)]);
      float sc[4];
      scale4(sv, sc);
      f32x4 tmp[C];
#pragma unroll
      for (int ct = 0; ct < C; ++ct) tmp[ct] = mfma_fp8(a, bfr[ct], negcorr[ct]);
#pragma unroll
      for (int ct = 0; ct < C; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][ct][i] = __builtin_fmaf(sc[i], tmp[ct][i], acc[r][ct][i]);
    }
    if (issue2) wait_step();  // this wavefront's copies of group g + 1 have landed
    else lds_dma_wait_all();
    __syncthreads();          // ... and everyone's; buffer u is free again
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using U2 = std::integral_constant<int, 2>;

  issue(0, 0);
  if (groups > 1) {
    issue(1, 1);
    wait_step();
  } else {
    lds_dma_wait_all();
  }
  __syncthreads();
  // the last two steps copy nothing and the last waits for everything, so no
  // copy is outstanding at exit
  for (int g = 0; g < groups; g += 3) {
    step(g, U0{});
    if (g + 1 < groups) step(g + 1, U1{});
    if (g + 2 < groups) step(g + 2, U2{});
  }

#pragma unroll
  for (int ct = 0; ct < C; ++ct) {
    const int64_t rowid = slot_rowid(p, b, ct * 16 + sw, tk);
    if (rowid < 0) continue;
    const int64_t arow = act_row_of<STAGE>(rowid, tk, p.topk);
    const float mult = kUnScale * p.act_scale[arow];
    if constexpr (STAGE == 1) {
      const float lim = p.clamp_limit;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        uint32_t bits[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float gt = acc[2 * s][ct][i] * mult;
          float up = acc[2 * s + 1][ct][i] * mult;
          if (lim > 0.0f) {
            gt = fminf(gt, lim);
            up = fminf(fmaxf(up, -lim), lim);
          }
          bits[i] = float_to_bf16_bits(silu_rcp(gt) * up);
        }
        const int n = n0 + 32 * wave + 16 * s + 4 * jg;
        *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) =
            u32x2{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
      }
    } else {
      const float wm = contrib_weight(p, b, rowid, tk) * mult;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = n0 + 64 * wave + 16 * r + 4 * jg;
        const f32x4 v = {acc[r][ct][0] * wm, acc[r][ct][1] * wm, acc[r][ct][2] * wm, acc[r][ct][3] * wm};
        *reinterpret_cast<f32x4*>(p.contrib + rowid * p.out_cols + n) = v;
      }
    }
  }
}

static void launch_act_quant(const uint16_t* x, int64_t rows, int k, uint8_t* q, float* scale, float* gsum,
                             hipStream_t stream) {
  hipLaunchKernelGGL(act_quant_fp8_kernel<false>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, rows,
                     k, q, scale, gsum);
}

template <int STAGE>
static int fp8_decode_resident_grid() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, expert_fp8_decode_kernel<STAGE>, 256, 0) != hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    cache[dev] = cus * per_cu;
  }
  return cache[dev];
}

static void launch_fp8_stage(const ExpertGemmParams& p, bool decode, int stage, int blocks, hipStream_t stream) {
  if (decode) {
    if (stage == 1) {
      const dim3 grid((unsigned)std::min(p.n_tiles * blocks, fp8_decode_resident_grid<1>()));
      hipLaunchKernelGGL(expert_fp8_decode_kernel<1>, grid, dim3(256), 0, stream, p);
    } else {
      const dim3 grid((unsigned)std::min(p.n_tiles * blocks, fp8_decode_resident_grid<2>()));
      hipLaunchKernelGGL(expert_fp8_decode_kernel<2>, grid, dim3(256), 0, stream, p);
    }
  } else {
    const dim3 grid((unsigned)prefill_grid(blocks, p.n_tiles));
    if (stage == 1) hipLaunchKernelGGL(expert_fp8_prefill_kernel<1>, grid, dim3(256), 0, stream, p, blocks);
    else hipLaunchKernelGGL(expert_fp8_prefill_kernel<2>, grid, dim3(256), 0, stream, p, blocks);
  }
}

}  // namespace dsv4

using namespace dsv4;

size_t dsv4_experts_w4a8_workspace_bytes(int64_t tokens, int topk, int hidden, int inter, int has_shared) {
  return carve_fp8(nullptr, tokens, topk, hidden, inter, has_shared).bytes;
}

// The pieces of a W4A8 workspace a fused layer call fills before the experts
// launches: the quantised x (codes, row scales, group sums), written by the
// prologue beside the alignment, and the contribution region, which the
// experts path writes only after it has read the alignment (the split
// alignment's scratch).
void dsv4_experts_w4a8_pieces(void* workspace, int64_t tokens, int topk, int hidden, int inter, int has_shared,
                              uint8_t** xq, float** xscale, float** xsum, int32_t** scratch,
                              size_t* scratch_bytes) {
  const Fp8Workspace w = carve_fp8(workspace, tokens, topk, hidden, inter, has_shared);
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);
  *xq = w.xq;
  *xscale = w.xscale;
  *xsum = w.xsum;
  *scratch = reinterpret_cast<int32_t*>(w.contrib);
  *scratch_bytes = sizeof(float) * (size_t)rows * hidden;
}

// Per-row e4m3 quantisation in K order (no group sums): the activation
// operand of the MXFP4 W4A8 kernels.
int dsv4_launch_act_quant_fp8_rows(const uint16_t* x, int64_t rows, int k, uint8_t* q, float* scale,
                                   hipStream_t stream) {
  if (rows == 0) return DSV4MOE_OK;
  hipLaunchKernelGGL(act_quant_fp8_kernel<true>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, rows,
                     k, q, scale, nullptr);
  DSV4_CHECK_LAUNCH("act_quant_fp8_kernel (K order)");
  return DSV4MOE_OK;
}

int dsv4_launch_act_quant_fp8(const uint16_t* x, int64_t rows, int k, uint8_t* q, float* scale, float* gsum,
                              hipStream_t stream) {
  if (rows == 0) return DSV4MOE_OK;
  launch_act_quant(x, rows, k, q, scale, gsum, stream);
  DSV4_CHECK_LAUNCH("act_quant_fp8_kernel");
  return DSV4MOE_OK;
}

int dsv4_launch_experts_w4a8(const uint16_t* x, int64_t tokens, int hidden, int inter, int experts, int topk,
                             const uint8_t* w13q, const uint16_t* w13s, const uint8_t* w2q,
                             const uint16_t* w2s, int has_shared, const float* weights, const int32_t* sorted,
                             int64_t capacity, const int32_t* expert_ids, const int32_t* ntpp, int block_size,
                             float clamp_limit, uint16_t* out, void* workspace, hipStream_t stream,
                             bool x_ready) {
  if (tokens == 0) return DSV4MOE_OK;
  Fp8Workspace ws = carve_fp8(workspace, tokens, topk, hidden, inter, has_shared);
  const int max_blocks = (int)((capacity + block_size - 1) / block_size);
  const bool decode = block_size <= 16 && hidden % 512 == 0 && inter % 512 == 0;
  const int shared_bs = decode ? 16 : block_size;
  const int shared_blocks = has_shared ? (int)((tokens + shared_bs - 1) / shared_bs) : 0;
  const int blocks = max_blocks + shared_blocks;
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);

  if (!x_ready) {  // else a prologue launch quantised x beside the alignment
    launch_act_quant(x, tokens, hidden, ws.xq, ws.xscale, ws.xsum, stream);
    DSV4_CHECK_LAUNCH("act_quant_fp8_kernel (x)");
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

  p.wq = w13q;
  p.ws = w13s;
  p.wq_stride = (int64_t)2 * inter * hidden / 2;
  p.ws_stride = (int64_t)2 * inter * (hidden / kGroup);
  p.k_dim = hidden;
  p.act = reinterpret_cast<const uint16_t*>(ws.xq);
  p.act_rows = tokens;
  p.act_sum = ws.xsum;
  p.act_scale = ws.xscale;
  p.h_out = ws.h;
  p.n_tiles = decode ? inter / 64 : inter / 128;
  launch_fp8_stage(p, decode, 1, blocks, stream);
  DSV4_CHECK_LAUNCH("expert fp8 stage 1");

  launch_act_quant(ws.h, rows, inter, ws.hq, ws.hscale, ws.hsum, stream);
  DSV4_CHECK_LAUNCH("act_quant_fp8_kernel (h)");
  dsv4host::prof_stamp(dsv4host::kStampStage1, stream);

  p.wq = w2q;
  p.ws = w2s;
  p.wq_stride = (int64_t)hidden * inter / 2;
  p.ws_stride = (int64_t)hidden * (inter / kGroup);
  p.k_dim = inter;
  p.act = reinterpret_cast<const uint16_t*>(ws.hq);
  p.act_rows = rows;
  p.act_sum = ws.hsum;
  p.act_scale = ws.hscale;
  p.route_w = weights;
  p.contrib = ws.contrib;
  p.out_cols = hidden;
  p.n_tiles = decode ? hidden / 128 : hidden / 256;
  launch_fp8_stage(p, decode, 2, blocks, stream);
  DSV4_CHECK_LAUNCH("expert fp8 stage 2");
  dsv4host::prof_stamp(dsv4host::kStampStage2, stream);

  const int rc = dsv4_launch_combine(ws.contrib, ntpp, tokens, topk, hidden, has_shared, out, stream);
  if (rc != DSV4MOE_OK) return rc;
  dsv4host::prof_stamp(dsv4host::kStampCombine, stream);
  return DSV4MOE_OK;
}
