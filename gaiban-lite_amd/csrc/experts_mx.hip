// Grouped expert GEMMs over MXFP4 weights on bf16 MFMA: E2M1 codes with one
// E8M0 (power-of-two) scale per 32 K, the checkpoint format of the
// reference's routed experts (runtime/dsv4_direct/moe_forward.py:23-40,
// 115-155; flash-contract.txt:150-155).  Restates the two grouped GEMMs of
// the MXFP4 _fused_marlin_moe call (runtime/dsv4_direct/moe_runtime.py:
// 1829-1856) with the arithmetic of the reference's dense path
// (runtime/dsv4_direct/ops/dense_moe.py:41-68,336-354): dequantised weight x
// bf16 activation, fp32 accumulation, SwiGLU on the fp32 stage-1 result,
// h rounded to bf16, stage-2 result times the route weight.
//
// Dequantisation.  v_cvt_scalef32_pk_bf16_fp4 turns two E2M1 codes (one
// byte, low nibble first) into two bf16 values multiplied by the scale given
// by the exponent field of its fp32 operand.  An E8M0 scale byte e is passed
// as the float with bits e << 23, so the product 2^(e-127) * code is exact in
// bf16 and the whole group scale is applied inside the dequantisation: the
// MFMAs accumulate scaled products directly (no per-group rescaling and no
// offset correction, unlike the int4 path), 4 conversions per 8 weights.
// (Checked on gfx950 for every code, every byte position and power-of-two
// scales from 2^-127 to 2^20: exact.)
//
// Tile layout (dsv4moe_pack_mxfp4_g32): the int4 tile geometry, with lane L's
// dword d of a tile = the 4 checkpoint bytes of row L%16 for
// k = 128g + 32d + 8*(L/16) .. +7, and 128 scale bytes per (pair, group) at
// byte (r16*2 + m)*4 + d.
#include <algorithm>

#include "experts_common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// E8M0 byte d of `scales` as the fp32 operand of the scaled conversion.
__device__ __forceinline__ float e8m0_operand(uint32_t scales, int d) {
  return __uint_as_float(((scales >> (8 * d)) & 0xFFu) << 23);
}

// 8 E2M1 codes (4 bytes, k ascending) -> 8 bf16 MFMA operand values * scale.
__device__ __forceinline__ bf16x8 dequant_mxfp4(uint32_t w, float scale) {
  const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// ------------------------------------------------------------------ decode
// Persistent, as the int4 decode kernel: workgroup w takes items w, w +
// grid, ... of the active (block, tile) items; the K stream runs on across
// item boundaries (weights two groups ahead, activations one group ahead).
// STAGE 1: wave w owns gate strip tile*4 + w and the matching up strip (one
//          64-column chunk of h per item);
// STAGE 2: wave w owns strips 2(tile*4 + w) + {0, 1} (128 output rows per item).
struct MxItem {
  const uint8_t* wq;   // this lane's 16 bytes of the pair's first tile
  const uint8_t* ws;   // this lane's 8 scale bytes of the pair's first group
  uint32_t ld_base;    // loader thread: activation row offset of its slot (or out of range)
  int64_t rowid;       // lane: row id of its slot, -1 if padded
  int n0;
  float wmul;          // 1, or NaN when the block names no valid expert (stage-2 multiplier)
  bool skip;           // PAIR: the block is the second of a pair, computed by the first
};

template <int STAGE, bool PAIR>
__device__ __forceinline__ MxItem mx_item(const ExpertGemmParams& p, int item, int routed, int64_t tk) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int bi, tile;
  decode_item_block(p, item, routed, bi, tile);
  const int blk = bi < routed ? bi : p.max_blocks + (bi - routed);
  const BlockInfo b = block_info(p, blk);
  const int groups = p.k_dim / kGroup;
  MxItem it;
  const int span = decode_block_span<PAIR>(p, bi, routed);
  it.skip = span == 0;
  if (it.skip) return it;
  it.n0 = STAGE == 1 ? tile * 64 : tile * 128;
  const int pair = tile * 4 + wave;
  it.wq = p.wq + (int64_t)b.expert * p.wq_stride + (int64_t)pair * groups * 2048 + lane * 16;
  it.ws = p.ws8 + (int64_t)b.expert * p.ws_stride + (int64_t)pair * groups * 128 + (lane & 15) * 8;
  it.wmul = b.poison ? __builtin_nanf("") : 1.0f;
  it.rowid = slot_rowid_span(p, b, lane & 15, tk, span);
  const int ld_slot = threadIdx.x >> 4;
  const int64_t ld_row = act_row_of<STAGE>(slot_rowid_span(p, b, ld_slot, tk, span), tk, p.topk);
  it.ld_base = ld_row >= 0 ? (uint32_t)(ld_row * p.k_dim * 2 + (threadIdx.x & 15) * 16) : kOobOffset;
  return it;
}

template <int STAGE, bool PAIR>
__global__ __launch_bounds__(256, 4) void mx_decode_kernel(ExpertGemmParams p) {
  constexpr int R = 2;
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][16 * 256];  // part q of slot s at q ^ s
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t tk = p.tokens * p.topk;
  const int routed = decode_routed_blocks(p);
  const int n_items = decode_items(p, routed);
  const int stride = decode_stride(n_items);
  int item = blockIdx.x;
  if (item >= stride || item >= n_items) return;  // uniform per workgroup
  const int groups = p.k_dim / kGroup;

  const __amdgpu_buffer_rsrc_t act_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act, (short)0, (int)(p.act_rows * p.k_dim * 2), kRsrcFlags);
  const int ld_slot = threadIdx.x >> 4;
  const int ld_lds = ld_slot * 256 + (((threadIdx.x & 15) ^ ld_slot) * 16);
  int rd_lds[4];  // K step d: part 4d + lane/16 of slot lane % 16
#pragma unroll
  for (int d = 0; d < 4; ++d) rd_lds[d] = (lane & 15) * 256 + (((4 * d + (lane >> 4)) ^ (lane & 15)) * 16);

  // this workgroup's next item from index i on (n_items when none is left),
  // passing over the items of paired second blocks
  auto fetch = [&](int i, MxItem& it) {
    for (; i < n_items; i += stride) {
      it = mx_item<STAGE, PAIR>(p, i, routed, tk);
      if (!it.skip) return i;
    }
    return n_items;
  };
  MxItem cur;
  item = fetch(item, cur);
  if (item >= n_items) return;  // uniform per workgroup
  MxItem nxt;
  int next = fetch(item + stride, nxt);
  if (next >= n_items) nxt = cur;

  // Weights two groups ahead (ring 4), activations one group ahead (ring 2);
  // at the end of an item the prefetches continue with the next item (or
  // re-read the current one), so every load is unconditional.
  u32x4 W[4][R];
  u32x2 S[4];
  u32x4 xr;
  auto issue_w = [&](const MxItem& it, int g, u32x4 (&w)[R], u32x2& s) {
    w[0] = load16_nt(it.wq + g * 2048);
    w[1] = load16_nt(it.wq + g * 2048 + 1024);
    s = *reinterpret_cast<const u32x2*>(it.ws + g * 128);  // both members' 4 scales
  };
  auto issue_x = [&](const MxItem& it, int g) {
    xr = __builtin_amdgcn_raw_buffer_load_b128(act_rsrc, it.ld_base + (uint32_t)(g * 256), 0, 0);
  };

  issue_x(cur, 0);
  issue_w(cur, 0, W[0], S[0]);
  issue_w(cur, 1, W[1], S[1]);
  *reinterpret_cast<u32x4*>(&xs[0][ld_lds]) = xr;
  __syncthreads();

  for (;;) {
    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < groups; g0 += 4) {  // groups % 4 == 0 (checked on the host)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int g = g0 + u;
        const bool xn = g + 1 >= groups;
        issue_x(xn ? nxt : cur, xn ? 0 : g + 1);
        const bool wn = g + 2 >= groups;
        issue_w(wn ? nxt : cur, wn ? g + 2 - groups : g + 2, W[(u + 2) & 3], S[(u + 2) & 3]);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const bf16x8 bfr = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xs[u & 1][rd_lds[d]]));
#pragma unroll
          for (int r = 0; r < R; ++r)
            acc[r] = mfma_bf16(dequant_mxfp4(W[u][r][d], e8m0_operand(S[u][r], d)), bfr, acc[r]);
        }
        *reinterpret_cast<u32x4*>(&xs[(u + 1) & 1][ld_lds]) = xr;
        __syncthreads();
      }
    }

    const int64_t rowid = cur.rowid;
    if constexpr (STAGE == 1) {
      const float lim = p.clamp_limit;
      uint32_t bits[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gt = acc[0][i];
        float up = acc[1][i];
        if (lim > 0.0f) {
          gt = fminf(gt, lim);
          up = fminf(fmaxf(up, -lim), lim);
        }
        bits[i] = float_to_bf16_bits(silu_f(gt) * up);
      }
      if (rowid >= 0) {
        const int n = cur.n0 + 16 * wave + 4 * (lane >> 4);
        u32x2 packed = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
        *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) = packed;
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

// ----------------------------------------------------------------- prefill
// As the int4 prefill kernel: alignment blocks of up to 64 token slots,
// workgroup tile 64 slots x 256 weight rows (wavefront w: strip pairs
// p0 = tile*8 + 2w and p0 + 1), work items (block, tile) in XCD-grouped order
// (prefill_item).  The token tile is copied into LDS by inline-asm DMA,
// double buffered; each wavefront's weight tiles and scale words (private to
// it) are loaded straight into registers one group ahead, so LDS carries only
// the shared operand (32 KiB per workgroup, 160 VGPRs: three workgroups per
// CU).  One explicit wait and one barrier per group.  Per group a wavefront
// converts 16 weight operands (64 conversions)
// and issues 64 MFMAs into its 16 accumulator tiles.
template <int STAGE>
__global__ __launch_bounds__(256, 2) void mx_prefill_kernel(ExpertGemmParams p, int total_blocks) {
  constexpr int R = 4;
  constexpr int C = 4;
  constexpr int kSlots = 64;
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kSlots * 256];
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

  const __amdgpu_buffer_rsrc_t act_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.act, (short)0, (int)(p.act_rows * p.k_dim * 2), kRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.wq + (int64_t)b.expert * p.wq_stride), (short)0, (int)p.wq_stride, kRsrcFlags);
  const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.ws8 + (int64_t)b.expert * p.ws_stride), (short)0, (int)p.ws_stride, kRsrcFlags);

  // token tile: copy q (0..3) of wave w fills slots 16w + 4q + lane/16
  uint32_t dma_off[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 16 * wave + 4 * q + (lane >> 4);
    const int64_t ar = act_row_of<STAGE>(slot_rowid(p, b, row, tk), tk, p.topk);
    const int part = (lane & 15) ^ (row & 15);
    dma_off[q] = ar >= 0 ? (uint32_t)(ar * p.k_dim * 2 + part * 16) : kOobOffset;
  }
  // weight tiles: pair p, group g, member m at byte ((p*groups + g)*2 + m) * 1 KiB
  const uint32_t w_off0 = (uint32_t)(p0 * groups) * 2048 + lane * 16;
  const uint32_t w_off1 = (uint32_t)((p0 + 1) * groups) * 2048 + lane * 16;
  // scales: 128 bytes per (pair, group); strip r = 2j + m of this row at
  // byte 128 j + (r16*2 + m)*4 of the group's block: one 8-byte word per pair
  const uint32_t s_off0 = (uint32_t)(p0 * groups) * 128 + (lane & 15) * 8;
  const uint32_t s_off1 = (uint32_t)((p0 + 1) * groups) * 128 + (lane & 15) * 8;

  // copy destinations: this wavefront's buffer-0 address, made scalar once
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][16 * wave * 256]));
  auto issue = [&](int g, int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      lds_copy16(act_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + q * 1024, dma_off[q], g * 256);
  };
  // The weight tiles and scales are private to the wavefront: loaded straight
  // into registers, one group ahead (no LDS traffic for them).
  struct WRegs {
    u32x4 w[R];
    u32x2 s[2];
  };
  // Loads into registers as inline asm: the compiler neither counts them in
  // its own vmcnt waits (compiler-visible loads made it wait for the token
  // copies issued after them) nor lets uses move above wait_weights, which
  // takes the registers as in/out operands.  The registers in flight must not
  // be touched in between: the kernel must compile without spills
  // (tests/test_kernel_resources.py checks the compiled code object).
  auto load_weights = [&](int g, WRegs& o) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t gw = __builtin_amdgcn_readfirstlane((uint32_t)g * 2048u);
    const uint32_t gs = __builtin_amdgcn_readfirstlane((uint32_t)g * 128u);
    const uint32_t w0b = w_off0 + kTileBytes, w1b = w_off1 + kTileBytes;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[0]) : "v"(w_off0), "s"(w_rsrc), "s"(gw));
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[1]) : "v"(w0b), "s"(w_rsrc), "s"(gw));
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[2]) : "v"(w_off1), "s"(w_rsrc), "s"(gw));
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(o.w[3]) : "v"(w1b), "s"(w_rsrc), "s"(gw));
    asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen" : "=v"(o.s[0]) : "v"(s_off0), "s"(s_rsrc), "s"(gs));
    asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen" : "=v"(o.s[1]) : "v"(s_off1), "s"(s_rsrc), "s"(gs));
#endif
  };
  auto wait_weights = [&](WRegs& o) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(o.w[0]), "+v"(o.w[1]), "+v"(o.w[2]), "+v"(o.w[3]), "+v"(o.s[0]), "+v"(o.s[1])
                 :
                 : "memory");
#endif
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int ct = 0; ct < C; ++ct) acc[r][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int sw = lane & 15;
  // One group: prefetch group g+1 into the other buffers (unless last), then
  // 16 operand conversions and 64 MFMAs from buffer u.
  auto step = [&](int g, auto u_c, auto prefetch_c, const WRegs& cur, WRegs& nxt) {
    constexpr int u = decltype(u_c)::value;
    if constexpr (decltype(prefetch_c)::value) {
      issue(g + 1, (u + 1) & 1);
      load_weights(g + 1, nxt);
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int part = ((4 * d + (lane >> 4)) ^ sw) * 16;
      bf16x8 bfr[C];
#pragma unroll
      for (int ct = 0; ct < C; ++ct)
        bfr[ct] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xs[u][(ct * 16 + sw) * 256 + part]));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bf16x8 a = dequant_mxfp4(cur.w[r][d], e8m0_operand(cur.s[r >> 1][r & 1], d));
#pragma unroll
        for (int ct = 0; ct < C; ++ct) acc[r][ct] = mfma_bf16(a, bfr[ct], acc[r][ct]);
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
  // groups is even (checked on the host); the last group issues no prefetch
  for (int g0 = 0; g0 + 2 < groups; g0 += 2) {
    step(g0, U0{}, PF{}, wa, wb);
    step(g0 + 1, U1{}, PF{}, wb, wa);
  }
  step(groups - 2, U0{}, PF{}, wa, wb);
  step(groups - 1, U1{}, NOPF{}, wb, wa);

  if constexpr (STAGE == 1) {
    const float lim = p.clamp_limit;
#pragma unroll
    for (int ct = 0; ct < C; ++ct) {
      const int64_t rowid = slot_rowid(p, b, ct * 16 + sw, tk);
      if (rowid < 0) continue;
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
        }
        const int n = n0 + 32 * wave + 16 * s + 4 * (lane >> 4);
        u32x2 packed = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
        *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) = packed;
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

}  // namespace dsv4

using namespace dsv4;

// Resident workgroups of an MXFP4 decode kernel on the current device,
// cached per device: the persistent grid size.
template <int STAGE, bool PAIR>
static int mx_decode_resident_grid() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, mx_decode_kernel<STAGE, PAIR>, 256, 0) != hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    cache[dev] = cus * per_cu;
  }
  return cache[dev];
}

// One decode stage: persistent over at most one wave of resident
// workgroups, with pairs of 8-slot blocks when decode_pairs says so.
template <int STAGE>
static void launch_mx_decode(const ExpertGemmParams& p, int blocks, hipStream_t stream) {
  if (decode_pairs(p)) {
    const int grid = std::min(p.n_tiles * blocks, mx_decode_resident_grid<STAGE, true>());
    hipLaunchKernelGGL((mx_decode_kernel<STAGE, true>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  } else {
    const int grid = std::min(p.n_tiles * blocks, mx_decode_resident_grid<STAGE, false>());
    hipLaunchKernelGGL((mx_decode_kernel<STAGE, false>), dim3((unsigned)grid), dim3(256), 0, stream, p);
  }
}

int dsv4_launch_experts_mxfp4(const uint16_t* x, int64_t tokens, int hidden, int inter, int experts, int topk,
                              const uint8_t* w13q, const uint8_t* w13s, const uint8_t* w2q, const uint8_t* w2s,
                              int has_shared, const float* weights, const int32_t* sorted, int64_t capacity,
                              const int32_t* expert_ids, const int32_t* ntpp, int block_size, float clamp_limit,
                              uint16_t* out, void* workspace, hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  ExpertWorkspace ws = carve_workspace(workspace, tokens, topk, hidden, inter, has_shared);
  const int max_blocks = (int)((capacity + block_size - 1) / block_size);
  const bool decode = block_size <= 16;  // K groups in multiples of 4: checked by the caller
  const int shared_bs = decode ? 16 : block_size;
  const int shared_blocks = has_shared ? (int)((tokens + shared_bs - 1) / shared_bs) : 0;
  const int blocks = max_blocks + shared_blocks;
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);
  dsv4host::prof_stamp(dsv4host::kStampRowSum, stream);  // no activation sums on this path

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
  p.ws8 = w13s;
  p.wq_stride = (int64_t)2 * inter * hidden / 2;
  p.ws_stride = (int64_t)2 * inter * (hidden / 32);
  p.k_dim = hidden;
  p.act = x;
  p.act_rows = tokens;
  p.h_out = ws.h;
  if (decode) {
    p.n_tiles = inter / 64;
    launch_mx_decode<1>(p, blocks, stream);
  } else {
    p.n_tiles = inter / 128;
    hipLaunchKernelGGL(mx_prefill_kernel<1>, dim3((unsigned)prefill_grid(blocks, p.n_tiles)), dim3(256), 0,
                       stream, p, blocks);
  }
  DSV4_CHECK_LAUNCH("mxfp4 expert stage 1");
  dsv4host::prof_stamp(dsv4host::kStampStage1, stream);

  // stage 2: W2 [H, I]
  p.wq = w2q;
  p.ws8 = w2s;
  p.wq_stride = (int64_t)hidden * inter / 2;
  p.ws_stride = (int64_t)hidden * (inter / 32);
  p.k_dim = inter;
  p.act = ws.h;
  p.act_rows = rows;
  p.route_w = weights;
  p.contrib = ws.contrib;
  p.out_cols = hidden;
  if (decode) {
    p.n_tiles = hidden / 128;
    launch_mx_decode<2>(p, blocks, stream);
  } else {
    p.n_tiles = hidden / 256;
    hipLaunchKernelGGL(mx_prefill_kernel<2>, dim3((unsigned)prefill_grid(blocks, p.n_tiles)), dim3(256), 0,
                       stream, p, blocks);
  }
  DSV4_CHECK_LAUNCH("mxfp4 expert stage 2");
  dsv4host::prof_stamp(dsv4host::kStampStage2, stream);

  const int rc = dsv4_launch_combine(ws.contrib, ntpp, tokens, topk, hidden, has_shared, out, stream);
  if (rc != DSV4MOE_OK) return rc;
  dsv4host::prof_stamp(dsv4host::kStampCombine, stream);
  return DSV4MOE_OK;
}
