// W4A8 over the checkpoint's MXFP4 experts: E2M1 weight codes with E8M0
// per-32 scales against per-token e4m3 activations, on gfx950's block-scaled
// MFMA (v_mfma_scale_f32_16x16x128_f8f6f4 with an fp4 A operand).
//
// Restates vLLM's _fused_marlin_moe with input_dtype = float8_e4m3fn over the
// MXFP4 routed experts (runtime/dsv4_direct/ops/marlin_moe.py:197-222,
// moe_runtime.py:207-235,1829-1856): the expert inputs (x for stage 1, the
// bf16 SwiGLU output h for stage 2) are quantised per row to e4m3 with
// s = max(amax, 1e-12) / 448, the products of the exact E2M1 * 2^(e-127)
// weights and the e4m3 codes accumulate in fp32, and the row scale
// multiplies the result.
//
// No dequantisation work at all.  Operand layout of the 16x16x128 MFMA with
// an fp4 A and an fp8 B operand on gfx950 (any other K assignment or scale
// lane fails the per-32-group scale tests of tests/test_gpu_w4a8_mxfp4.py,
// whose scales differ per group): lane group j (lanes 16j .. 16j+15) of A holds K 32j .. 32j+31
// of its row, code i in nibble i (low nibble first), and the lane's E8M0
// scale byte multiplies exactly those 32 products; lane group j of B holds
// K 16j .. 16j+15 in bytes 0..15 and K 64+16j .. 64+16j+15 in bytes 16..31.
// So the weights are packed with the 16 checkpoint bytes of one 32-K scale
// group per lane (dsv4moe_pack_mxfp4_g32_w4a8) and that group's E8M0 byte as
// the lane's A scale; the activations are quantised in K order and lane
// group j reads the 16-byte parts j and j + 4 of each 128-K group; the B
// scale is 1 (byte 127).  The per-token scale is applied once, in the
// epilogue.
#include <algorithm>
#include <type_traits>

#include "experts_common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

typedef __attribute__((ext_vector_type(8))) int i32x8;

// 32 E2M1 codes (4 dwords, the lane's row and 32-K group) x 32 e4m3 codes.
// cbsz 4 = fp4 A operand (the compiler passes its first 4 dwords only),
// blgp 0 = e4m3 B operand; `scale` is the A operand's E8M0 byte.
__device__ __forceinline__ f32x4 mfma_fp4_fp8(u32x4 w, i32x8 x, int scale, f32x4 c) {
  const i32x8 a = {(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, x, c, 4, 0, 0, scale, 0, 127);
}

// The lane's E8M0 byte: byte j (its 32-K group within the 128-K group) of
// the member's scale word.
__device__ __forceinline__ int lane_scale(uint32_t word, int j) { return (int)((word >> (8 * j)) & 0xFFu); }

// ------------------------------------------------------------------ decode
// Persistent, as the int4 W4A8 decode kernel: workgroup w takes items w,
// w + grid, ... of the active (block, tile) items and the K stream runs on
// across item boundaries (weights and scale words two groups ahead, the
// activations one group ahead through LDS).  Wavefront w streams strip pair
// tile*4 + w (stage 1: gate + up strip of h columns n0 + 16w ..; stage 2:
// strips 2(tile*4 + w) + {0, 1}).
struct Fp4DecodeItem {
  const uint8_t* wq;  // this lane's 16 bytes of the pair's first tile
  const uint8_t* ws;  // this lane's 8 scale bytes (both members) of the pair's first group
  uint32_t ld_base;   // loader thread: activation byte offset of its slot (or out of range)
  int64_t rowid;      // lane: row id of its slot, -1 if padded
  int64_t arow;       // lane: activation row of its slot, -1 if padded
  int n0;
  float wmul;         // 1, or NaN when the block names no valid expert (stage-2 multiplier)
};

template <int STAGE>
__device__ __forceinline__ Fp4DecodeItem fp4_decode_item(const ExpertGemmParams& p, int item, int routed,
                                                         int64_t tk) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int bi, tile;
  decode_item_block(p, item, routed, bi, tile);
  const int blk = bi < routed ? bi : p.max_blocks + (bi - routed);
  const BlockInfo b = block_info(p, blk);
  const int groups = p.k_dim / kGroup;
  Fp4DecodeItem it;
  it.n0 = STAGE == 1 ? tile * 64 : tile * 128;
  const int pair = tile * 4 + wave;
  it.wq = p.wq + (int64_t)b.expert * p.wq_stride + (int64_t)pair * groups * 2048 + lane * 16;
  it.ws = p.ws8 + (int64_t)b.expert * p.ws_stride + (int64_t)pair * groups * 128 + (lane & 15) * 8;
  it.wmul = b.poison ? __builtin_nanf("") : 1.0f;
  it.rowid = slot_rowid(p, b, lane & 15, tk);
  it.arow = act_row_of<STAGE>(it.rowid, tk, p.topk);
  const int ld_slot = threadIdx.x >> 3;
  const int64_t ld_row =
      ld_slot < 16 ? act_row_of<STAGE>(slot_rowid(p, b, ld_slot, tk), tk, p.topk) : (int64_t)-1;
  it.ld_base = ld_row >= 0 ? (uint32_t)(ld_row * p.k_dim + (threadIdx.x & 7) * 16) : kOobOffset;
  return it;
}

template <int STAGE>
__global__ __launch_bounds__(256, 4) void expert_fp4_decode_kernel(ExpertGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][32 * 128];  // rows 16..31: unused landing rows
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int jg = lane >> 4;
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
  const int ld_slot = threadIdx.x >> 3;
  const int ld_lds = ld_slot * 128 + (((threadIdx.x & 7) ^ swz128(ld_slot)) * 16);
  // B operand: parts jg (K 16jg ..) and jg + 4 (K 64 + 16jg ..) of the slot's group
  const int rd_lds0 = (lane & 15) * 128 + ((jg ^ swz128(lane & 15)) * 16);
  const int rd_lds1 = (lane & 15) * 128 + (((jg + 4) ^ swz128(lane & 15)) * 16);

  Fp4DecodeItem cur = fp4_decode_item<STAGE>(p, item, routed, tk);
  int next = item + stride;
  Fp4DecodeItem nxt = next < n_items ? fp4_decode_item<STAGE>(p, next, routed, tk) : cur;

  u32x4 W[4][2];
  u32x2 S[4];
  u32x4 xr;
  auto issue_w = [&](const Fp4DecodeItem& it, int g, u32x4 (&w)[2], u32x2& s) {
    w[0] = load16_nt(it.wq + g * 2048);
    w[1] = load16_nt(it.wq + g * 2048 + 1024);
    s = *reinterpret_cast<const u32x2*>(it.ws + g * 128);
  };
  auto issue_x = [&](const Fp4DecodeItem& it, int g) {
    xr = __builtin_amdgcn_raw_buffer_load_b128(act_rsrc, it.ld_base + (uint32_t)(g * 128), 0, 0);
  };

  issue_x(cur, 0);
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
        issue_x(xn ? nxt : cur, xn ? 0 : g + 1);
        const bool wn = g + 2 >= groups;
        issue_w(wn ? nxt : cur, wn ? g + 2 - groups : g + 2, W[(u + 2) & 3], S[(u + 2) & 3]);
        const u32x4 b0 = *reinterpret_cast<const u32x4*>(&xs[u & 1][rd_lds0]);
        const u32x4 b1 = *reinterpret_cast<const u32x4*>(&xs[u & 1][rd_lds1]);
        const i32x8 bf = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3],
                          (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
#pragma unroll
        for (int r = 0; r < 2; ++r) acc[r] = mfma_fp4_fp8(W[u][r], bf, lane_scale(S[u][r], jg), acc[r]);
        *reinterpret_cast<u32x4*>(&xs[(u + 1) & 1][ld_lds]) = xr;
        __syncthreads();
      }
    }

    const int64_t rowid = cur.rowid;
    if (rowid >= 0) {
      const float mult = p.act_scale[cur.arow];
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
        const int n = cur.n0 + 16 * wave + 4 * jg;
        *reinterpret_cast<u32x2*>(p.h_out + rowid * p.inter + n) =
            u32x2{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
      } else {
        const float wm = (rowid < tk ? p.route_w[rowid] : 1.0f) * cur.wmul * mult;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int n = cur.n0 + 32 * wave + 16 * r + 4 * jg;
          const f32x4 v = {acc[r][0] * wm, acc[r][1] * wm, acc[r][2] * wm, acc[r][3] * wm};
          *reinterpret_cast<f32x4*>(p.contrib + rowid * p.out_cols + n) = v;
        }
      }
    }
    if (next >= n_items) break;  // uniform per workgroup; the last prefetches re-read cur
    item = next;
    cur = nxt;
    next = item + stride;
    nxt = next < n_items ? fp4_decode_item<STAGE>(p, next, routed, tk) : cur;
  }
}

// ----------------------------------------------------------------- prefill
// Blocks of up to 64 slots: workgroup tile 64 slots x 256 weight rows, the
// strip assignment and work order of the other prefill kernels.  Per group
// the 64 x 128 B token tile (16-byte part q of slot s at q ^ swz128(s)),
// each wavefront's 4 weight tiles and its two pairs' scale blocks are copied
// into LDS by buffer_load ... lds in a ring of RING buffers, RING - 1 groups
// ahead: 25 KiB per buffer, so RING = 2 runs three workgroups per CU and
// RING = 3 (copies two groups ahead) two.  Per group a wavefront issues 16
// MFMAs and no VALU work on the accumulators.
constexpr int kF4Slots = 64;
constexpr int kF4Ring = 2;

template <int STAGE, int RING>
__global__ __launch_bounds__(256, RING == 2 ? 3 : 2) void expert_fp4_prefill_kernel(ExpertGemmParams p,
                                                                                   int total_blocks) {
  static_assert(RING == 2 || RING == 3, "two or three buffers");
  constexpr int R = 4;
  constexpr int C = 4;
  __shared__ __attribute__((aligned(16))) uint8_t xs[RING][kF4Slots * 128];
  __shared__ __attribute__((aligned(16))) uint8_t wts[RING][4][R * kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t scl[RING][4][256];
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
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.wq + (int64_t)b.expert * p.wq_stride), (short)0, (int)p.wq_stride, kRsrcFlags);
  const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.ws8 + (int64_t)b.expert * p.ws_stride), (short)0, (int)p.ws_stride, kRsrcFlags);

  // token tile: DMA q (0..1) of wave w fills slots 16w + 8q + lane/8
  uint32_t dma_off[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = 16 * wave + 8 * q + (lane >> 3);
    const int64_t ar = act_row_of<STAGE>(slot_rowid(p, b, row, tk), tk, p.topk);
    const int part = (lane & 7) ^ swz128(row);
    dma_off[q] = ar >= 0 ? (uint32_t)(ar * p.k_dim + part * 16) : kOobOffset;
  }
  const uint32_t w_off0 = (uint32_t)(p0 * groups) * 2048 + lane * 16;
  const uint32_t w_off1 = (uint32_t)((p0 + 1) * groups) * 2048 + lane * 16;
  // scales: 128 bytes per (pair, group); lanes 0..31 copy pair p0's block,
  // lanes 32..63 pair p0 + 1's
  const uint32_t s_off = (uint32_t)((p0 + (lane >> 5)) * groups) * 128 + (lane & 31) * 4;

  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // here, plus constant offsets (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][16 * wave * 128]));
  const uint32_t wts_lds = __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][wave][0]));
  const uint32_t scl_lds = __builtin_amdgcn_readfirstlane(lds_addr(&scl[0][wave][0]));
  auto issue = [&](int g, int buf) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      lds_copy16(act_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + q * 1024, dma_off[q], g * 128);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      lds_copy16(w_rsrc, wts_lds + buf * (uint32_t)sizeof(wts[0]) + t * kTileBytes,
                 (t < 2 ? w_off0 : w_off1) + (t & 1) * kTileBytes, g * 2048);
    lds_copy4(s_rsrc, scl_lds + buf * (uint32_t)sizeof(scl[0]), s_off, g * 128);
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int ct = 0; ct < C; ++ct) acc[r][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int sw = lane & 15;
  const int jg = lane >> 4;
  constexpr int kLoads = 2 + 4 + 1;  // copies one issue() makes per wavefront
  // Step g: copy group g + RING - 1 into buffer (u + RING - 1) % RING
  // (released by step g - 1's barrier), compute group g from buffer u, wait
  // for group g + 1.
  auto step = [&](int g, auto u_c) {
    constexpr int u = decltype(u_c)::value;
    const bool issue2 = g + RING - 1 < groups;
    if (issue2) issue(g + RING - 1, (u + RING - 1) % RING);
    i32x8 bfr[C];
#pragma unroll
    for (int ct = 0; ct < C; ++ct) {
      const int row = ct * 16 + sw;
      // parts jg (K 16jg ..) and jg + 4 (K 64 + 16jg ..) of the token's group
      const u32x4 b0 = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + (jg ^ swz128(row)) * 16]);
      const u32x4 b1 = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + ((jg + 4) ^ swz128(row)) * 16]);
      bfr[ct] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(&wts[u][wave][r * kTileBytes + lane * 16]);
      // strip r = member (r & 1) of pair (r >> 1): byte (row*2 + m)*4 + j of the pair's block
      const int sc = scl[u][wave][(r >> 1) * 128 + (sw * 2 + (r & 1)) * 4 + jg];
#pragma unroll
      for (int ct = 0; ct < C; ++ct) acc[r][ct] = mfma_fp4_fp8(a, bfr[ct], sc, acc[r][ct]);
    }
    // this wavefront's copies of group g + 1 have landed (with three buffers
    // the newest group's copies stay in flight)
    if (RING == 3 && issue2) lds_dma_wait_keep<kLoads>();
    else lds_dma_wait_all();
    __syncthreads();  // ... and everyone's; buffer u is free again
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using U2 = std::integral_constant<int, 2>;

  issue(0, 0);
  if (RING == 3 && groups > 1) {
    issue(1, 1);
    lds_dma_wait_keep<kLoads>();
  } else {
    lds_dma_wait_all();
  }
  __syncthreads();
  // the last RING - 1 steps copy nothing and the last waits for everything,
  // so no copy is outstanding at exit
  for (int g = 0; g < groups; g += RING) {
    step(g, U0{});
    if (g + 1 < groups) step(g + 1, U1{});
    if constexpr (RING == 3)
      if (g + 2 < groups) step(g + 2, U2{});
  }

#pragma unroll
  for (int ct = 0; ct < C; ++ct) {
    const int64_t rowid = slot_rowid(p, b, ct * 16 + sw, tk);
    if (rowid < 0) continue;
    const int64_t arow = act_row_of<STAGE>(rowid, tk, p.topk);
    const float mult = p.act_scale[arow];
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

template <int STAGE>
static int fp4_decode_resident_grid() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, expert_fp4_decode_kernel<STAGE>, 256, 0) != hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    cache[dev] = cus * per_cu;
  }
  return cache[dev];
}

static void launch_fp4_stage(const ExpertGemmParams& p, bool decode, int stage, int blocks, hipStream_t stream) {
  if (decode) {
    if (stage == 1) {
      const dim3 grid((unsigned)std::min(p.n_tiles * blocks, fp4_decode_resident_grid<1>()));
      hipLaunchKernelGGL(expert_fp4_decode_kernel<1>, grid, dim3(256), 0, stream, p);
    } else {
      const dim3 grid((unsigned)std::min(p.n_tiles * blocks, fp4_decode_resident_grid<2>()));
      hipLaunchKernelGGL(expert_fp4_decode_kernel<2>, grid, dim3(256), 0, stream, p);
    }
  } else {
    const dim3 grid((unsigned)prefill_grid(blocks, p.n_tiles));
    if (stage == 1)
      hipLaunchKernelGGL((expert_fp4_prefill_kernel<1, kF4Ring>), grid, dim3(256), 0, stream, p, blocks);
    else
      hipLaunchKernelGGL((expert_fp4_prefill_kernel<2, kF4Ring>), grid, dim3(256), 0, stream, p, blocks);
  }
}

}  // namespace dsv4

using namespace dsv4;

int dsv4_launch_act_quant_fp8_rows(const uint16_t* x, int64_t rows, int k, uint8_t* q, float* scale,
                                   hipStream_t stream);

int dsv4_launch_experts_w4a8_mxfp4(const uint16_t* x, int64_t tokens, int hidden, int inter, int experts,
                                   int topk, const uint8_t* w13q, const uint8_t* w13s, const uint8_t* w2q,
                                   const uint8_t* w2s, int has_shared, const float* weights,
                                   const int32_t* sorted, int64_t capacity, const int32_t* expert_ids,
                                   const int32_t* ntpp, int block_size, float clamp_limit, uint16_t* out,
                                   void* workspace, hipStream_t stream, bool x_ready) {
  if (tokens == 0) return DSV4MOE_OK;
  Fp8Workspace ws = carve_fp8(workspace, tokens, topk, hidden, inter, has_shared);
  const int max_blocks = (int)((capacity + block_size - 1) / block_size);
  const bool decode = block_size <= 16;  // hidden, inter multiples of 512: checked by the caller
  const int shared_bs = decode ? 16 : block_size;
  const int shared_blocks = has_shared ? (int)((tokens + shared_bs - 1) / shared_bs) : 0;
  const int blocks = max_blocks + shared_blocks;
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);

  if (!x_ready) {  // else a prologue launch quantised x beside the alignment
    const int rc = dsv4_launch_act_quant_fp8_rows(x, tokens, hidden, ws.xq, ws.xscale, stream);
    if (rc != DSV4MOE_OK) return rc;
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
  p.ws8 = w13s;
  p.wq_stride = (int64_t)2 * inter * hidden / 2;
  p.ws_stride = (int64_t)2 * inter * hidden / 32;
  p.k_dim = hidden;
  p.act = reinterpret_cast<const uint16_t*>(ws.xq);
  p.act_rows = tokens;
  p.act_scale = ws.xscale;
  p.h_out = ws.h;
  p.n_tiles = decode ? inter / 64 : inter / 128;
  launch_fp4_stage(p, decode, 1, blocks, stream);
  DSV4_CHECK_LAUNCH("expert fp4 stage 1");

  int rc = dsv4_launch_act_quant_fp8_rows(ws.h, rows, inter, ws.hq, ws.hscale, stream);
  if (rc != DSV4MOE_OK) return rc;
  dsv4host::prof_stamp(dsv4host::kStampStage1, stream);

  p.wq = w2q;
  p.ws8 = w2s;
  p.wq_stride = (int64_t)hidden * inter / 2;
  p.ws_stride = (int64_t)hidden * inter / 32;
  p.k_dim = inter;
  p.act = reinterpret_cast<const uint16_t*>(ws.hq);
  p.act_rows = rows;
  p.act_scale = ws.hscale;
  p.route_w = weights;
  p.contrib = ws.contrib;
  p.out_cols = hidden;
  p.n_tiles = decode ? hidden / 128 : hidden / 256;
  launch_fp4_stage(p, decode, 2, blocks, stream);
  DSV4_CHECK_LAUNCH("expert fp4 stage 2");
  dsv4host::prof_stamp(dsv4host::kStampStage2, stream);

  rc = dsv4_launch_combine(ws.contrib, ntpp, tokens, topk, hidden, has_shared, out, stream);
  if (rc != DSV4MOE_OK) return rc;
  dsv4host::prof_stamp(dsv4host::kStampCombine, stream);
  return DSV4MOE_OK;
}
