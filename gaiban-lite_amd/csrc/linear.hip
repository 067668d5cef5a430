// Dense linears for gfx950 over 1-byte weights.
//
// W8A16: C[M,N] = bf16( A[M,K] . W[N,K]^T ), A bf16,
// fp32 accumulation, with W in one of two formats:
//   * int8 symmetric per output channel, W = Q * s[n] (s bf16);
//   * FP8 E4M3 with one E8M0 scale per 128 x 128 block, W = Q * 2^(e-127),
//     the reference checkpoint's format (weight_only_linear.py:488-513,
//     537-598; moe_forward.py:158-176).
//
// Restates the weight-only linear of experiments/C1F-integrated-block/
// weight_only_linear.py:537-702 (bf16 MMA over a weight reconstructed in
// registers, fp32 accumulate, optional split-K into an fp32 [split, M, N]
// workspace reduced in split order, one bf16 rounding) for the int8
// per-channel format: the scale factors out of the K sum and is applied once
// in the epilogue.  The FP8 weights convert with v_cvt_scalef32_pk_bf16_fp8,
// whose fp32 scale operand carries the E8M0 byte in its exponent field: the
// product is exact in bf16 (3 mantissa bits times a power of two), so the
// MFMA sees the reference's bf16(Q * scale) and no epilogue scale is needed.
// A 16-row strip and a 64-K window lie inside one 128 x 128 scale block.
//
// Weight layout (dsv4moe_pack_int8): 1 KiB tiles of 16 rows x 64 K, tile
// (strip, window) at byte (strip * K/64 + window) * 1024; lane l's 16 bytes are
// row 16*strip + l%16, K 64*window + 16*(l/16) .. +15.  A wavefront therefore
// streams one contiguous KiB per strip and window.  Each lane's 16 bytes feed
// two MFMA 16x16x32 steps (bytes 0-7: K 16j..16j+7, bytes 8-15: K 16j+8..+15,
// j = l/16); the activation fragments use the same K assignment, so the
// product is the plain dot product over a permuted K order.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

constexpr int kWin = 64;               // K per window
constexpr int kLinXcds = 8;
constexpr uint32_t kLinOob = 0x80000000u;
constexpr int kLinRsrcFlags = 0x00020000;

struct LinearParams {
  const uint16_t* a;
  int64_t m;
  int n;
  int k;
  const uint8_t* wq;
  const uint16_t* ws;    // int8 format: bf16 [N]
  const uint8_t* ws8;    // FP8 format: E8M0 [ceil(N/128)][K/128]
  int kblocks;           // K / 128
  int split;
  int win_per_split;
  int tiles_n;
  int tiles_m;
  uint16_t* out;
  float* partial;  // [split][M][N] when split > 1
  int accumulate;  // out = bf16(out + bf16(result)) instead of bf16(result)
  int w_rowmajor;  // weights as the checkpoint's row-major [N][K] bytes instead of 1 KiB tiles
};

// Byte offset of lane `lane`'s 16 weight bytes in 64-K window 0 of 16-row
// strip `strip`, in either weight layout: 1 KiB tiles (dsv4moe_pack_int8 /
// pack_fp8: the strip's tiles are contiguous, lane l at 16 l) or the
// checkpoint's row-major [N][K] bytes (lane l reads row 16 strip + l % 16,
// K 16 (l / 16) .. +15).  Both put the same bytes in the same LDS slots,
// since a buffer_load ... lds copy places lane l's 16 bytes at 16 l whatever
// address it read.  The step to the next window is weight_window_step.
__device__ __forceinline__ uint32_t weight_lane_offset(int rowmajor, int strip, int lane, int k, int wins) {
  return rowmajor ? (uint32_t)(((int64_t)strip * 16 + (lane & 15)) * k + (lane >> 4) * 16)
                  : (uint32_t)((int64_t)strip * wins * 1024 + lane * 16);
}
__device__ __forceinline__ int weight_window_step(int rowmajor) { return rowmajor ? 64 : 1024; }

// The bf16 written for result v: bf16(v), or with accumulation the bf16 sum
// of the existing output and bf16(v) (torch.add of two bf16 tensors).
__device__ __forceinline__ u32x2 finish_bf16x4(const float (&v)[4], const uint16_t* old, bool accumulate) {
  u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  if (accumulate) {
    const u32x2 prev = *reinterpret_cast<const u32x2*>(old);
    o[0] = pack_bf16x2(__uint_as_float(prev[0] << 16) + __uint_as_float(o[0] << 16),
                       __uint_as_float(prev[0] & 0xFFFF0000u) + __uint_as_float(o[0] & 0xFFFF0000u));
    o[1] = pack_bf16x2(__uint_as_float(prev[1] << 16) + __uint_as_float(o[1] << 16),
                       __uint_as_float(prev[1] & 0xFFFF0000u) + __uint_as_float(o[1] & 0xFFFF0000u));
  }
  return o;
}

// 8 int8 weights (two dwords, K order) -> 8 bf16.  Every int8 is exact in
// bf16; the signed byte converts through v_cvt_f32_i32 (SDWA byte select) and
// the bf16 is the upper half of the float (exact, no rounding).
__device__ __forceinline__ bf16x8 dequant_i8x8(uint32_t lo, uint32_t hi) {
  const uint32_t f0 = __float_as_uint((float)(int8_t)(lo));
  const uint32_t f1 = __float_as_uint((float)(int8_t)(lo >> 8));
  const uint32_t f2 = __float_as_uint((float)(int8_t)(lo >> 16));
  const uint32_t f3 = __float_as_uint((float)(int8_t)(lo >> 24));
  const uint32_t f4 = __float_as_uint((float)(int8_t)(hi));
  const uint32_t f5 = __float_as_uint((float)(int8_t)(hi >> 8));
  const uint32_t f6 = __float_as_uint((float)(int8_t)(hi >> 16));
  const uint32_t f7 = __float_as_uint((float)(int8_t)(hi >> 24));
  u32x4 p;
  p[0] = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
  p[1] = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
  p[2] = __builtin_amdgcn_perm(f5, f4, 0x07060302u);
  p[3] = __builtin_amdgcn_perm(f7, f6, 0x07060302u);
  return __builtin_bit_cast(bf16x8, p);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// 8 FP8 E4M3 weights (two dwords, K order, low byte first) -> 8 bf16 times
// the power of two whose exponent field `scale` carries.
__device__ __forceinline__ bf16x8 dequant_fp8x8(uint32_t lo, uint32_t hi, float scale) {
  const bf16x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, scale, false);
  const bf16x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, scale, true);
  const bf16x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, scale, false);
  const bf16x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, scale, true);
  return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Workgroup tile: 64*R output channels (wavefront w owns strips 4R*tn + R*w + r)
// x 16*C tokens, over one K split.  Per window, buffer_load ... lds copies the
// token tile (16C rows x 128 B, 16-byte part q of row t stored at
// q ^ swz128(t))
// and each wavefront's R weight tiles into LDS, double buffered.
template <int R, int C, bool FP8>
__global__ __launch_bounds__(256, 2) void w8a16_kernel(LinearParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][16 * C * 128];
  __shared__ __attribute__((aligned(16))) uint8_t wts[2][4][R * 1024];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // XCD-aware item order: workgroup id i runs on XCD i % 8; each XCD takes a
  // contiguous range of items, and items are split-major, then token tile,
  // then channel tile, so one XCD's L2 keeps sharing an activation tile.
  const int items = p.split * p.tiles_m * p.tiles_n;
  const int per_xcd = (items + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= items) return;
  const int tn = item % p.tiles_n;
  const int tm = (item / p.tiles_n) % p.tiles_m;
  const int sp = item / (p.tiles_n * p.tiles_m);

  const int wins = p.k / kWin;
  const int w_begin = sp * p.win_per_split;
  const int w_end = min(wins, w_begin + p.win_per_split);
  const int nw = w_end - w_begin;  // may be 0 for a trailing split: it writes zeros

  const int strips = p.n >> 4;
  const int strip0 = tn * 4 * R + wave * R;

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k * 2), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);

  // token tile: 2C DMAs of 1 KiB (8 rows of 128 B); wavefront w issues DMA q = w + 4i
  constexpr int kActDma = 2 * C;
  constexpr int kActPerWave = (kActDma + 3) / 4;
  uint32_t a_off[kActPerWave];
#pragma unroll
  for (int i = 0; i < kActPerWave; ++i) {
    const int q = wave + 4 * i;
    const int row = q * 8 + (lane >> 3);
    const int64_t tok = (int64_t)tm * 16 * C + row;
    const int part = (lane & 7) ^ swz128(row);
    a_off[i] = (q < kActDma && tok < p.m) ? (uint32_t)(tok * p.k * 2 + part * 16) : kLinOob;
  }
  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w_off[r] = strip0 + r < strips ? weight_lane_offset(p.w_rowmajor, strip0 + r, lane, p.k, wins) : kLinOob;
  // FP8: the wavefront's R strips lie in one 128-row scale block (R divides
  // 8); lane i holds the E8M0 bytes of K blocks i, 64 + i, 128 + i, 192 + i,
  // loaded before any copy is in flight (K <= 32768, checked on the host)
  uint32_t srow[4] = {0, 0, 0, 0};
  if constexpr (FP8) {
    const uint8_t* row = p.ws8 + (int64_t)(min(strip0, strips - 1) >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }

  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][wave * 1024]));
  const uint32_t wts_lds = __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][wave][0]));
  auto issue = [&](int win, int buf) {
#pragma unroll
    for (int i = 0; i < kActPerWave; ++i) {
      const int q = wave + 4 * i;
      if (q < kActDma)
        lds_dma16(a_rsrc, lds_ptr(xs_lds + buf * (uint32_t)sizeof(xs[0]) + i * 4096), a_off[i], win * 128);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
      lds_dma16(w_rsrc, lds_ptr(wts_lds + buf * (uint32_t)sizeof(wts[0]) + r * 1024), w_off[r], win * wstep);
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int n16 = lane & 15;
  const int j = lane >> 4;
  auto step = [&](int win, auto u_c, auto pf_c) {
    constexpr int u = decltype(u_c)::value;
    if constexpr (decltype(pf_c)::value) issue(win + 1, u ^ 1);
    u32x4 raw[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      raw[r] = *reinterpret_cast<const u32x4*>(&wts[u][wave][r * 1024 + lane * 16]);
    float bscale = 0.0f;  // FP8: E8M0 byte of (this wavefront's row block, K block) as an fp32 exponent field
    if constexpr (FP8) {
      const int kb = win >> 1;
      const uint32_t word = kb < 64 ? srow[0] : (kb < 128 ? srow[1] : (kb < 192 ? srow[2] : srow[3]));
      bscale = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)word, kb & 63) << 23);
    }
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      bf16x8 a[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (FP8)
          a[r] = dequant_fp8x8(raw[r][2 * d], raw[r][2 * d + 1], bscale);
        else
          a[r] = dequant_i8x8(raw[r][2 * d], raw[r][2 * d + 1]);
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int row = c * 16 + n16;
        const int part = (2 * j + d) ^ swz128(row);
        const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + part * 16]));
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][c] = mfma_bf16(a[r], b, acc[r][c]);
      }
    }
    __syncthreads();
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using PF = std::true_type;
  using NOPF = std::false_type;

  if (nw > 0) {
    issue(w_begin, 0);
    __syncthreads();
    int i = 0;
    for (; i + 2 < nw; i += 2) {
      step(w_begin + i, U0{}, PF{});
      step(w_begin + i + 1, U1{}, PF{});
    }
    // the last window issues no prefetch, so no LDS DMA is in flight at exit
    if (nw - i == 2) {
      step(w_begin + i, U0{}, PF{});
      step(w_begin + i + 1, U1{}, NOPF{});
    } else {
      step(w_begin + i, U0{}, NOPF{});
    }
  }

  // epilogue: lane holds channels 16*strip + 4*j + (0..3) of token c*16 + n16
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int strip = strip0 + r;
    if (strip >= strips) continue;
    const int n = strip * 16 + 4 * j;
    float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if constexpr (!FP8) {
      const u32x2 sv = *reinterpret_cast<const u32x2*>(p.ws + n);
      sc[0] = __uint_as_float(sv[0] << 16);
      sc[1] = __uint_as_float(sv[0] & 0xFFFF0000u);
      sc[2] = __uint_as_float(sv[1] << 16);
      sc[3] = __uint_as_float(sv[1] & 0xFFFF0000u);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t tok = (int64_t)tm * 16 * C + c * 16 + n16;
      if (tok >= p.m) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[r][c][e] * sc[e];
      if (p.split == 1) {
        uint16_t* dst = p.out + tok * p.n + n;
        *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, p.accumulate != 0);
      } else {
        float* dst = p.partial + ((int64_t)sp * p.m + tok) * p.n + n;
        *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

// 17..64 tokens: the tile of w8a16_kernel (64*R channels x 16*C tokens over
// one K split, the same partials, so the same bits), with each wavefront's
// weights straight to registers, D windows in flight, and the workgroup's
// token rows for the whole split copied into LDS first (DMAs issued before
// any weight load, so the waits for them are exact) -- the LDS copies of the
// weights, one or two windows deep, were what w8a16_kernel waited on.
// WPS > 0: WPS windows per split, straight-line code; WPS*16*C*128 bytes of
// LDS (<= 64 KiB, checked on the host).
template <int R, int C, int D, int WPS, bool FP8>
__global__ __launch_bounds__(256, 2) __attribute__((amdgpu_waves_per_eu(1, 2))) void w8a16_regw_kernel(
    LinearParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs_all[];  // [WPS][16C rows][128 B]
  constexpr int kRows = 16 * C;
  constexpr int kWinBytes = kRows * 128;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int items = p.split * p.tiles_m * p.tiles_n;
  const int per_xcd = (items + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= items) return;
  const int tn = item % p.tiles_n;
  const int tm = (item / p.tiles_n) % p.tiles_m;
  const int sp = item / (p.tiles_n * p.tiles_m);

  const int wins = p.k / kWin;
  const int w_begin = sp * WPS;
  const int w_end = min(wins, w_begin + WPS);
  const int strips = p.n >> 4;
  const int strip0 = tn * 4 * R + wave * R;
  const int n16 = lane & 15;
  const int j = lane >> 4;

  u32x2 sv[R];
  if constexpr (!FP8) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      sv[r] = *reinterpret_cast<const u32x2*>(p.ws + min(strip0 + r, strips - 1) * 16 + 4 * j);
  }
  uint32_t srow[4] = {0, 0, 0, 0};
  if constexpr (FP8) {
    const uint8_t* row = p.ws8 + (int64_t)(min(strip0, strips - 1) >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k * 2), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);

  // token rows of every window of the split: 2C DMAs of 1 KiB (8 rows x 128 B)
  // per window, DMA q = wave + 4i; part q of row t at q ^ swz128(t); rows past
  // M and windows past the split's end copy zeros
  constexpr int kActDma = 2 * C;
  static_assert(kActDma % 4 == 0, "every wavefront issues the same number of copies");
#pragma unroll
  for (int i = 0; i < kActDma / 4; ++i) {
    const int q = wave + 4 * i;
    const int row = q * 8 + (lane >> 3);
    const int64_t tok = (int64_t)tm * kRows + row;
    const int part = (lane & 7) ^ swz128(row);
    const uint32_t base = tok < p.m ? (uint32_t)(tok * p.k * 2 + part * 16) : kLinOob;
#pragma unroll
    for (int w = 0; w < WPS; ++w) {
      const int win = w_begin + w;
      lds_dma16(a_rsrc, (lds_void_ptr)&xs_all[w * kWinBytes + q * 1024], win < w_end ? base : kLinOob, win * 128);
    }
  }

  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w_off[r] = strip0 + r < strips ? weight_lane_offset(p.w_rowmajor, strip0 + r, lane, p.k, wins) : kLinOob;
  u32x4 wr[D][R];
  auto load = [&](int win, int t) {
    const bool in = win < w_end;
#pragma unroll
    for (int r = 0; r < R; ++r)
      wr[t][r] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, in ? w_off[r] : kLinOob, win * wstep, 0));
  };
  constexpr int kDepth = D < WPS ? D : WPS;
#pragma unroll
  for (int t = 0; t < kDepth; ++t) {
    load(w_begin + t, t);
    __builtin_amdgcn_sched_barrier(0);
  }
  // this wavefront's token copies have landed (only weight loads may remain), then everyone's
  lds_dma_wait_keep<kDepth * R>();
  __syncthreads();

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < WPS; ++i) {
    const int win = w_begin + i;
    const int t = i % kDepth;
    float bscale = 0.0f;
    if constexpr (FP8) {
      const int kb = min(win, wins - 1) >> 1;
      const uint32_t word = kb < 64 ? srow[0] : (kb < 128 ? srow[1] : (kb < 192 ? srow[2] : srow[3]));
      bscale = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)word, kb & 63) << 23);
    }
    const uint8_t* xw = &xs_all[i * kWinBytes];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      bf16x8 a[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (FP8)
          a[r] = dequant_fp8x8(wr[t][r][2 * d], wr[t][r][2 * d + 1], bscale);
        else
          a[r] = dequant_i8x8(wr[t][r][2 * d], wr[t][r][2 * d + 1]);
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int row = c * 16 + n16;
        const int part = (2 * j + d) ^ swz128(row);
        const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xw[row * 128 + part * 16]));
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][c] = mfma_bf16(a[r], b, acc[r][c]);
      }
    }
    if (i + kDepth < WPS) load(w_begin + i + kDepth, t);
    __builtin_amdgcn_sched_barrier(0);
  }

  // epilogue as w8a16_kernel: lane holds channels 16*strip + 4*j + (0..3) of token c*16 + n16
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int strip = strip0 + r;
    if (strip >= strips) continue;
    const int n = strip * 16 + 4 * j;
    float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if constexpr (!FP8) {
      sc[0] = __uint_as_float(sv[r][0] << 16);
      sc[1] = __uint_as_float(sv[r][0] & 0xFFFF0000u);
      sc[2] = __uint_as_float(sv[r][1] << 16);
      sc[3] = __uint_as_float(sv[r][1] & 0xFFFF0000u);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t tok = (int64_t)tm * kRows + c * 16 + n16;
      if (tok >= p.m) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[r][c][e] * sc[e];
      if (p.split == 1) {
        uint16_t* dst = p.out + tok * p.n + n;
        *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, p.accumulate != 0);
      } else {
        float* dst = p.partial + ((int64_t)sp * p.m + tok) * p.n + n;
        *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

// Up to 16 tokens with a K split: the split runs inside the workgroup.
// Workgroup tile: 16*R output channels x 16*C tokens; wavefront w of the
// `split` wavefronts computes split w's partial -- windows [w * wps,
// min(wins, (w + 1) * wps)), the same MFMA chain per (channel, token) as a
// split workgroup of w8a16_kernel -- scales it, and leaves it in LDS; the
// workgroup then sums the partials in split order (fp32, split 0 first) and
// rounds once, the additions of split_reduce_kernel, so the bits equal the
// two-launch result for the same split.  No workspace and no second launch.
// Operands go straight to registers (the lane's 16 weight bytes and 32
// activation bytes of a window are what its MFMAs use), D windows in flight
// per wavefront; windows past a split's end load out of range (zeros) and
// add exact zeros.  WPS > 0: the window count per split is WPS (checked on
// the host) and the window sequence is straight-line code, so each window
// waits only for its own loads; WPS = 0: a loop over groups of D windows.
// LDS_ACT (C = 1, WPS > 0, splits covering K exactly, M*K*2 <= 32 KiB):
// each wavefront first copies its split's activation rows (the M valid
// tokens, WPS*128 bytes each) into LDS with 1 KiB DMAs, every lane useful,
// and the MFMA operands come from there -- lanes of padding tokens read 32
// zero bytes -- instead of two 16-byte loads per window in which only the
// lanes of valid tokens fetch anything.
template <int R, int C, int D, int WPS, bool FP8, bool LDS_ACT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2))) void w8a16_wsplit_kernel(
    LinearParams p) {
  __shared__ __attribute__((aligned(16))) f32x4 red[8][R * C][64];
  extern __shared__ __attribute__((aligned(16))) uint8_t act_lds[];  // LDS_ACT: [split][M][WPS*128], [split][32] zeros
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // = split index (wavefront-uniform)
  const int tiles = p.tiles_m * p.tiles_n;
  const int per_xcd = (tiles + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= tiles) return;
  const int tn = item % p.tiles_n;
  const int tm = item / p.tiles_n;

  const int wins = p.k / kWin;
  const int w_begin = wave * p.win_per_split;
  const int w_end = min(wins, w_begin + p.win_per_split);
  const int strips = p.n >> 4;
  const int strip0 = tn * R;
  const int n16 = lane & 15;
  const int j = lane >> 4;

  // int8 format: the lane's 4 channel scales, loaded ahead of the weight stream
  u32x2 sv[R];
  if constexpr (!FP8) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      sv[r] = *reinterpret_cast<const u32x2*>(p.ws + min(strip0 + r, strips - 1) * 16 + 4 * j);
    __builtin_amdgcn_sched_barrier(0);
  }
  uint32_t srow[4] = {0, 0, 0, 0};
  if constexpr (FP8) {
    const uint8_t* row = p.ws8 + (int64_t)(min(strip0, strips - 1) >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k * 2), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);
  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w_off[r] = strip0 + r < strips ? weight_lane_offset(p.w_rowmajor, strip0 + r, lane, p.k, wins) : kLinOob;
  // lane's 32 activation bytes of a window: token tm*16C + 16c + n16, K 16j .. 16j+15
  uint32_t a_off[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t tok = (int64_t)tm * 16 * C + c * 16 + n16;
    a_off[c] = tok < p.m ? (uint32_t)(tok * p.k * 2 + j * 32) : kLinOob;
  }

  // LDS_ACT: this wavefront's rows, and the lane's read address for window w_begin
  constexpr int kRowBytes = WPS * 128;
  const uint8_t* act_row = nullptr;
  if constexpr (LDS_ACT) {
    static_assert(C == 1 && WPS > 0 && kRowBytes % 1024 == 0, "LDS activations: one token tile, whole KiB rows");
    const int m = (int)p.m;
    uint8_t* mine = act_lds + wave * m * kRowBytes;
    uint8_t* zeros = act_lds + p.split * m * kRowBytes + wave * 32;  // this wavefront's own: no barrier needed
    if (lane < 2) *reinterpret_cast<u32x4*>(zeros + 16 * lane) = u32x4{0, 0, 0, 0};
    for (int row = 0; row < m; ++row)
#pragma unroll
      for (int q = 0; q < kRowBytes / 1024; ++q)
        lds_dma16(a_rsrc, (lds_void_ptr)(mine + row * kRowBytes + q * 1024),
                  (uint32_t)(row * p.k * 2 + w_begin * 128 + lane * 16), q * 1024);
    act_row = n16 < m ? mine + n16 * kRowBytes + 32 * j : zeros;
  }

  u32x4 wr[D][R];
  u32x4 ar[D][C][2];
  // a window past the split's end reads at kLinOob + (small) soffset: out of range, zeros
  auto load = [&](int win, int t) {
    const bool in = win < w_end;
#pragma unroll
    for (int r = 0; r < R; ++r)
      wr[t][r] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, in ? w_off[r] : kLinOob, win * wstep, 0));
    if constexpr (!LDS_ACT) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const uint32_t off = in ? a_off[c] : kLinOob;
        ar[t][c][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off, win * 128, 0));
        ar[t][c][1] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off, win * 128 + 16, 0));
      }
    }
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto consume = [&](int win, int t) {
    float bscale = 0.0f;
    if constexpr (FP8) {
      const int kb = min(win, wins - 1) >> 1;
      const uint32_t word = kb < 64 ? srow[0] : (kb < 128 ? srow[1] : (kb < 192 ? srow[2] : srow[3]));
      bscale = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)word, kb & 63) << 23);
    }
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      bf16x8 a[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (FP8)
          a[r] = dequant_fp8x8(wr[t][r][2 * d], wr[t][r][2 * d + 1], bscale);
        else
          a[r] = dequant_i8x8(wr[t][r][2 * d], wr[t][r][2 * d + 1]);
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        bf16x8 b;
        if constexpr (LDS_ACT) {
          // padding lanes all read the zero block (one address: a broadcast)
          const int step = n16 < (int)p.m ? (win - w_begin) * 128 : 0;
          b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(act_row + step + 16 * d));
        } else {
          b = __builtin_bit_cast(bf16x8, ar[t][c][d]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][c] = mfma_bf16(a[r], b, acc[r][c]);
      }
    }
  };

  // sched_barrier keeps each group of loads where it stands: the scheduler
  // would otherwise sink loads toward their uses and shrink the ring
  if constexpr (WPS > 0) {
    constexpr int kDepth = D < WPS ? D : WPS;
#pragma unroll
    for (int t = 0; t < kDepth; ++t) {
      load(w_begin + t, t);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < WPS; ++i) {
      consume(w_begin + i, i % kDepth);
      if (i + kDepth < WPS) load(w_begin + i + kDepth, i % kDepth);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int t = 0; t < D; ++t) load(w_begin + t, t);
    for (int i = 0; i < p.win_per_split; i += D) {
#pragma unroll
      for (int t = 0; t < D; ++t) {
        consume(w_begin + i + t, t);
        load(w_begin + i + t + D, t);
      }
    }
  }

  // this split's scaled partial: lane holds channels 16*strip + 4*j + (0..3) of token c*16 + n16
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if constexpr (!FP8) {
      sc[0] = __uint_as_float(sv[r][0] << 16);
      sc[1] = __uint_as_float(sv[r][0] & 0xFFFF0000u);
      sc[2] = __uint_as_float(sv[r][1] << 16);
      sc[3] = __uint_as_float(sv[r][1] & 0xFFFF0000u);
    }
#pragma unroll
    for (int c = 0; c < C; ++c)
      red[wave][r * C + c][lane] = f32x4{acc[r][c][0] * sc[0], acc[r][c][1] * sc[1], acc[r][c][2] * sc[2],
                                         acc[r][c][3] * sc[3]};
  }
  __syncthreads();
  for (int q = threadIdx.x; q < R * C * 64; q += blockDim.x) {
    const int rc = q >> 6, l = q & 63;
    const int r = rc / C, c = rc % C;
    const int strip = strip0 + r;
    const int64_t tok = (int64_t)tm * 16 * C + c * 16 + (l & 15);
    if (strip >= strips || tok >= p.m) continue;
    f32x4 sum = red[0][rc][l];
    for (int w = 1; w < p.split; ++w) {
      const f32x4 v = red[w][rc][l];
      sum[0] += v[0];
      sum[1] += v[1];
      sum[2] += v[2];
      sum[3] += v[3];
    }
    const float v[4] = {sum[0], sum[1], sum[2], sum[3]};
    uint16_t* dst = p.out + tok * p.n + strip * 16 + 4 * (l >> 4);
    *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, p.accumulate != 0);
  }
}

// The same tile for 64 or more tokens (C >= 4), with the copies as inline
// asm into a three-buffer ring two windows ahead and one explicit wait per
// window (the compiler-visible copies of w8a16_kernel make every ds_read
// wait for the newest copy).  Used for the 256 x 64 tile (72 KiB of LDS, two
// workgroups per CU): M=8192, N=1024 65-78 us vs 72-96.  The 256 x 128 tile
// would need 96 KiB and run one workgroup per CU, which measured slower.
// Workgroup tile: 64*R output channels (wavefront w owns strips 4R*tn + R*w + r)
// x 16*C tokens, over one K split.  Per window, buffer_load ... lds copies the
// token tile (16C rows x 128 B, 16-byte part q of row t stored at
// q ^ swz128(t))
// and each wavefront's R weight tiles into LDS, double buffered.
template <int R, int C, bool FP8>
__global__ __launch_bounds__(256, 2) void w8a16_kernel3(LinearParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[3][16 * C * 128];
  __shared__ __attribute__((aligned(16))) uint8_t wts[3][4][R * 1024];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // XCD-aware item order: workgroup id i runs on XCD i % 8; each XCD takes a
  // contiguous range of items, and items are split-major, then token tile,
  // then channel tile, so one XCD's L2 keeps sharing an activation tile.
  const int items = p.split * p.tiles_m * p.tiles_n;
  const int per_xcd = (items + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= items) return;
  const int tn = item % p.tiles_n;
  const int tm = (item / p.tiles_n) % p.tiles_m;
  const int sp = item / (p.tiles_n * p.tiles_m);

  const int wins = p.k / kWin;
  const int w_begin = sp * p.win_per_split;
  const int w_end = min(wins, w_begin + p.win_per_split);
  const int nw = w_end - w_begin;  // may be 0 for a trailing split: it writes zeros

  const int strips = p.n >> 4;
  const int strip0 = tn * 4 * R + wave * R;

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k * 2), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);

  // token tile: 2C DMAs of 1 KiB (8 rows of 128 B); wavefront w issues DMA q = w + 4i
  constexpr int kActDma = 2 * C;
  constexpr int kActPerWave = (kActDma + 3) / 4;
  uint32_t a_off[kActPerWave];
#pragma unroll
  for (int i = 0; i < kActPerWave; ++i) {
    const int q = wave + 4 * i;
    const int row = q * 8 + (lane >> 3);
    const int64_t tok = (int64_t)tm * 16 * C + row;
    const int part = (lane & 7) ^ swz128(row);
    a_off[i] = (q < kActDma && tok < p.m) ? (uint32_t)(tok * p.k * 2 + part * 16) : kLinOob;
  }
  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w_off[r] = strip0 + r < strips ? weight_lane_offset(p.w_rowmajor, strip0 + r, lane, p.k, wins) : kLinOob;
  // FP8: the wavefront's R strips lie in one 128-row scale block (R divides
  // 8); lane i holds the E8M0 bytes of K blocks i, 64 + i, 128 + i, 192 + i,
  // loaded before any copy is in flight (K <= 32768, checked on the host)
  uint32_t srow[4] = {0, 0, 0, 0};
  if constexpr (FP8) {
    const uint8_t* row = p.ws8 + (int64_t)(min(strip0, strips - 1) >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }

  static_assert(kActDma % 4 == 0, "every wavefront issues the same number of copies");
  constexpr int kStepLoads = kActPerWave + R;
  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][wave * 1024]));
  const uint32_t wts_lds = __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][wave][0]));
  auto issue = [&](int win, int buf) {
#pragma unroll
    for (int i = 0; i < kActPerWave; ++i)
      lds_copy16(a_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + i * 4096, a_off[i], win * 128);
#pragma unroll
    for (int r = 0; r < R; ++r)
      lds_copy16(w_rsrc, wts_lds + buf * (uint32_t)sizeof(wts[0]) + r * 1024, w_off[r], win * wstep);
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int n16 = lane & 15;
  const int j = lane >> 4;
  // Step win: copy window win + 2 into buffer (u + 2) % 3 (released by the
  // previous step's barrier), compute window win from buffer u, then wait for
  // window win + 1 (this wavefront's copies; the barrier makes them everyone's).
  auto step = [&](int win, auto u_c) {
    constexpr int u = decltype(u_c)::value;
    const bool issue2 = win + 2 < w_end;
    if (issue2) issue(win + 2, (u + 2) % 3);
    u32x4 raw[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      raw[r] = *reinterpret_cast<const u32x4*>(&wts[u][wave][r * 1024 + lane * 16]);
    float bscale = 0.0f;  // FP8: E8M0 byte of (this wavefront's row block, K block) as an fp32 exponent field
    if constexpr (FP8) {
      const int kb = win >> 1;
      const uint32_t word = kb < 64 ? srow[0] : (kb < 128 ? srow[1] : (kb < 192 ? srow[2] : srow[3]));
      bscale = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)word, kb & 63) << 23);
    }
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      bf16x8 a[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (FP8)
          a[r] = dequant_fp8x8(raw[r][2 * d], raw[r][2 * d + 1], bscale);
        else
          a[r] = dequant_i8x8(raw[r][2 * d], raw[r][2 * d + 1]);
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int row = c * 16 + n16;
        const int part = (2 * j + d) ^ swz128(row);
        const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + part * 16]));
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][c] = mfma_bf16(a[r], b, acc[r][c]);
      }
    }
    if (issue2) lds_dma_wait_keep<kStepLoads>();
    else lds_dma_wait_all();
    __syncthreads();
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using U2 = std::integral_constant<int, 2>;

  if (nw > 0) {
    issue(w_begin, 0);
    if (nw > 1) {
      issue(w_begin + 1, 1);
      lds_dma_wait_keep<kStepLoads>();
    } else {
      lds_dma_wait_all();
    }
    __syncthreads();
    // the last two steps copy nothing and the last waits for everything
    for (int i = 0; i < nw; i += 3) {
      step(w_begin + i, U0{});
      if (i + 1 < nw) step(w_begin + i + 1, U1{});
      if (i + 2 < nw) step(w_begin + i + 2, U2{});
    }
  }

  // epilogue: lane holds channels 16*strip + 4*j + (0..3) of token c*16 + n16
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int strip = strip0 + r;
    if (strip >= strips) continue;
    const int n = strip * 16 + 4 * j;
    float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if constexpr (!FP8) {
      const u32x2 sv = *reinterpret_cast<const u32x2*>(p.ws + n);
      sc[0] = __uint_as_float(sv[0] << 16);
      sc[1] = __uint_as_float(sv[0] & 0xFFFF0000u);
      sc[2] = __uint_as_float(sv[1] << 16);
      sc[3] = __uint_as_float(sv[1] & 0xFFFF0000u);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t tok = (int64_t)tm * 16 * C + c * 16 + n16;
      if (tok >= p.m) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[r][c][e] * sc[e];
      if (p.split == 1) {
        uint16_t* dst = p.out + tok * p.n + n;
        *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, p.accumulate != 0);
      } else {
        float* dst = p.partial + ((int64_t)sp * p.m + tok) * p.n + n;
        *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

// Variant of w8a16_kernel3 for the 256 x 128 tile: the weights three buffers
// deep (two windows ahead: they come from HBM) and the tokens two (one window
// ahead: they are L2 hits), 80 KiB of LDS, still two workgroups per CU;
// inline-asm copies with one explicit wait per window.  M=8192, N=4096 /
// 16384: 6-11% faster than w8a16_kernel.  Tile and fragment layout as in
// w8a16_kernel.
template <int R, int C, bool FP8>
__global__ __launch_bounds__(256, 2) void w8a16_kernel_w3(LinearParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][16 * C * 128];
  __shared__ __attribute__((aligned(16))) uint8_t wts[3][4][R * 1024];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // XCD-aware item order: workgroup id i runs on XCD i % 8; each XCD takes a
  // contiguous range of items, and items are split-major, then token tile,
  // then channel tile, so one XCD's L2 keeps sharing an activation tile.
  const int items = p.split * p.tiles_m * p.tiles_n;
  const int per_xcd = (items + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= items) return;
  const int tn = item % p.tiles_n;
  const int tm = (item / p.tiles_n) % p.tiles_m;
  const int sp = item / (p.tiles_n * p.tiles_m);

  const int wins = p.k / kWin;
  const int w_begin = sp * p.win_per_split;
  const int w_end = min(wins, w_begin + p.win_per_split);
  const int nw = w_end - w_begin;  // may be 0 for a trailing split: it writes zeros

  const int strips = p.n >> 4;
  const int strip0 = tn * 4 * R + wave * R;

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k * 2), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);

  // token tile: 2C DMAs of 1 KiB (8 rows of 128 B); wavefront w issues DMA q = w + 4i
  constexpr int kActDma = 2 * C;
  constexpr int kActPerWave = (kActDma + 3) / 4;
  uint32_t a_off[kActPerWave];
#pragma unroll
  for (int i = 0; i < kActPerWave; ++i) {
    const int q = wave + 4 * i;
    const int row = q * 8 + (lane >> 3);
    const int64_t tok = (int64_t)tm * 16 * C + row;
    const int part = (lane & 7) ^ swz128(row);
    a_off[i] = (q < kActDma && tok < p.m) ? (uint32_t)(tok * p.k * 2 + part * 16) : kLinOob;
  }
  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w_off[r] = strip0 + r < strips ? weight_lane_offset(p.w_rowmajor, strip0 + r, lane, p.k, wins) : kLinOob;
  // FP8: the wavefront's R strips lie in one 128-row scale block (R divides
  // 8); lane i holds the E8M0 bytes of K blocks i, 64 + i, 128 + i, 192 + i,
  // loaded before any copy is in flight (K <= 32768, checked on the host)
  uint32_t srow[4] = {0, 0, 0, 0};
  if constexpr (FP8) {
    const uint8_t* row = p.ws8 + (int64_t)(min(strip0, strips - 1) >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }

  static_assert(kActDma % 4 == 0, "every wavefront issues the same number of copies");
  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][wave * 1024]));
  const uint32_t wts_lds = __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][wave][0]));
  auto issue_tok = [&](int win, int buf) {
#pragma unroll
    for (int i = 0; i < kActPerWave; ++i)
      lds_copy16(a_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + i * 4096, a_off[i], win * 128);
  };
  auto issue_w = [&](int win, int buf) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      lds_copy16(w_rsrc, wts_lds + buf * (uint32_t)sizeof(wts[0]) + r * 1024, w_off[r], win * wstep);
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int n16 = lane & 15;
  const int j = lane >> 4;
  // Step win: copy the tokens of window win + 1 (buffer t ^ 1) and the weights
  // of window win + 2 (buffer (u + 2) % 3), both released by the previous
  // step's barrier; compute window win from token buffer t and weight buffer
  // u; wait for window win + 1, keeping the newest weights in flight.
  auto step = [&](int win, auto t_c, auto u_c) {
    constexpr int t = decltype(t_c)::value;
    constexpr int u = decltype(u_c)::value;
    const bool next1 = win + 1 < w_end;
    const bool next2 = win + 2 < w_end;
    if (next1) issue_tok(win + 1, t ^ 1);
    if (next2) issue_w(win + 2, (u + 2) % 3);
    u32x4 raw[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      raw[r] = *reinterpret_cast<const u32x4*>(&wts[u][wave][r * 1024 + lane * 16]);
    float bscale = 0.0f;  // FP8: E8M0 byte of (this wavefront's row block, K block) as an fp32 exponent field
    if constexpr (FP8) {
      const int kb = win >> 1;
      const uint32_t word = kb < 64 ? srow[0] : (kb < 128 ? srow[1] : (kb < 192 ? srow[2] : srow[3]));
      bscale = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)word, kb & 63) << 23);
    }
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      bf16x8 a[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (FP8)
          a[r] = dequant_fp8x8(raw[r][2 * d], raw[r][2 * d + 1], bscale);
        else
          a[r] = dequant_i8x8(raw[r][2 * d], raw[r][2 * d + 1]);
      }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int row = c * 16 + n16;
        const int part = (2 * j + d) ^ swz128(row);
        const bf16x8 b = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&xs[t][row * 128 + part * 16]));
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][c] = mfma_bf16(a[r], b, acc[r][c]);
      }
    }
    if (next2) lds_dma_wait_keep<R>();  // the weights of window win + 2 stay in flight
    else lds_dma_wait_all();
    __syncthreads();
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using U2 = std::integral_constant<int, 2>;

  if (nw > 0) {
    issue_tok(w_begin, 0);
    issue_w(w_begin, 0);
    if (nw > 1) {
      issue_w(w_begin + 1, 1);
      lds_dma_wait_keep<R>();
    } else {
      lds_dma_wait_all();
    }
    __syncthreads();
    // token buffer = window % 2, weight buffer = window % 3 (six-step cycle);
    // the last step copies nothing and waits for everything
    for (int i = 0; i < nw; i += 6) {
      step(w_begin + i, U0{}, U0{});
      if (i + 1 < nw) step(w_begin + i + 1, U1{}, U1{});
      if (i + 2 < nw) step(w_begin + i + 2, U0{}, U2{});
      if (i + 3 < nw) step(w_begin + i + 3, U1{}, U0{});
      if (i + 4 < nw) step(w_begin + i + 4, U0{}, U1{});
      if (i + 5 < nw) step(w_begin + i + 5, U1{}, U2{});
    }
  }

  // epilogue: lane holds channels 16*strip + 4*j + (0..3) of token c*16 + n16
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int strip = strip0 + r;
    if (strip >= strips) continue;
    const int n = strip * 16 + 4 * j;
    float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if constexpr (!FP8) {
      const u32x2 sv = *reinterpret_cast<const u32x2*>(p.ws + n);
      sc[0] = __uint_as_float(sv[0] << 16);
      sc[1] = __uint_as_float(sv[0] & 0xFFFF0000u);
      sc[2] = __uint_as_float(sv[1] << 16);
      sc[3] = __uint_as_float(sv[1] & 0xFFFF0000u);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t tok = (int64_t)tm * 16 * C + c * 16 + n16;
      if (tok >= p.m) continue;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[r][c][e] * sc[e];
      if (p.split == 1) {
        uint16_t* dst = p.out + tok * p.n + n;
        *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, p.accumulate != 0);
      } else {
        float* dst = p.partial + ((int64_t)sp * p.m + tok) * p.n + n;
        *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

// out[m][n] = bf16(sum over splits, in split order, of partial[s][m][n]).
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* partial, int split, int64_t mn,
                                                           uint16_t* out, int accumulate) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 4 elements each
  if (q * 4 >= mn) return;
  f32x4 s = *reinterpret_cast<const f32x4*>(partial + q * 4);
  for (int i = 1; i < split; ++i) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(partial + (int64_t)i * mn + q * 4);
    s[0] += v[0];
    s[1] += v[1];
    s[2] += v[2];
    s[3] += v[3];
  }
  const float v[4] = {s[0], s[1], s[2], s[3]};
  *reinterpret_cast<u32x2*>(out + q * 4) = finish_bf16x4(v, out + q * 4, accumulate != 0);
}

// Shared-expert SwiGLU over bf16 linear outputs (shared_bf16_partial,
// runtime/dsv4_direct/moe_runtime.py:246-263): per row the first `inter`
// columns are the gate, the next `inter` the up projection;
// h = bf16(silu(min(gate, L)) * clamp(up, -L, L)) in fp32 (no clamp for L = 0).
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const uint16_t* __restrict__ gu, int64_t rows, int inter,
                                                          float clamp_limit, uint16_t* __restrict__ h) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 4 columns each
  const int quads = inter / 4;
  if (q >= rows * quads) return;
  const int64_t r = q / quads;
  const int c = (int)(q % quads) * 4;
  const u32x2 g = *reinterpret_cast<const u32x2*>(gu + r * 2 * inter + c);
  const u32x2 u = *reinterpret_cast<const u32x2*>(gu + r * 2 * inter + inter + c);
  float out[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t gw = g[e >> 1], uw = u[e >> 1];
    float gt = (e & 1) ? __uint_as_float(gw & 0xFFFF0000u) : __uint_as_float(gw << 16);
    float up = (e & 1) ? __uint_as_float(uw & 0xFFFF0000u) : __uint_as_float(uw << 16);
    if (clamp_limit > 0.0f) {
      gt = fminf(gt, clamp_limit);
      up = fminf(fmaxf(up, -clamp_limit), clamp_limit);
    }
    out[e] = silu_f(gt) * up;
  }
  *reinterpret_cast<u32x2*>(h + r * inter + c) = u32x2{pack_bf16x2(out[0], out[1]), pack_bf16x2(out[2], out[3])};
}

// Row-major int8 [N][K] -> 1 KiB tiles (16 rows x 64 K); one thread per 16 bytes.
__global__ __launch_bounds__(256) void pack_int8_kernel(const uint8_t* src, int64_t n, int64_t k, uint8_t* dst) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c * 16 >= n * k) return;
  const int64_t wins = k / kWin;
  const int64_t tile = c >> 6;
  const int lane = (int)(c & 63);
  const int64_t strip = tile / wins;
  const int64_t win = tile % wins;
  const int64_t row = strip * 16 + (lane & 15);
  const int64_t col = win * kWin + 16 * (lane >> 4);
  *reinterpret_cast<u32x4*>(dst + c * 16) = *reinterpret_cast<const u32x4*>(src + row * k + col);
}

// ------------------------------------------------------------ block-FP8 W8A8
// Restates runtime/dsv4_direct/fp8_linear.py:354-497: activations quantised
// per row and 128-K block to E4M3 with a power-of-two E8M0 scale, weights in
// the checkpoint's E4M3 / E8M0 128 x 128 block format, and per K block
// C += (A_blk . W_blk^T) * 2^(ea-127) * 2^(ew-127) in fp32, one bf16 rounding
// (split-K: fp32 partials reduced in split order).  gfx950 applies both block
// scales inside the MFMA: v_mfma_scale_f32_16x16x128_f8f6f4 takes one E8M0
// byte per lane for its row of A (weights: the row block's scale, uniform over
// the wavefront) and its column of B (tokens: the token's scale), so the MFMA
// adds exactly 2^(ea-127) * 2^(ew-127) times the block dot product.

typedef __attribute__((ext_vector_type(8))) int i32x8;

__device__ __forceinline__ f32x4 mfma_fp8_block(i32x8 w, i32x8 t, f32x4 c, int scale_w, int scale_t) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, t, c, 0, 0, 0, scale_w, 0, scale_t);
}

// Activation quantiser (fp8_linear.py:354-392): per row and 128-K block,
// s = max(amax, 1e-4) * fp32(1/448); its E8M0 exponent is rounded up to a
// power of two (biased exponent + 1 when the mantissa is nonzero, clamped to
// [1, 254]); q = e4m3(clamp(x / 2^(e-127), -448, 448)) (round to nearest
// even).  16 lanes per block, 8 K values per lane; X is bf16 (0), fp16 (1) or
// fp32 (2).
template <int X>
__device__ __forceinline__ void load_act8(const void* x, int64_t idx, float (&f)[8]) {
  if constexpr (X == 2) {
    const u32x4 a = load16(static_cast<const float*>(x) + idx);
    const u32x4 b = load16(static_cast<const float*>(x) + idx + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = __uint_as_float(a[e]);
      f[4 + e] = __uint_as_float(b[e]);
    }
  } else {
    const u32x4 v = load16(static_cast<const uint16_t*>(x) + idx);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (X == 0) {
        f[2 * e] = __uint_as_float(v[e] << 16);
        f[2 * e + 1] = __uint_as_float(v[e] & 0xFFFF0000u);
      } else {
        f[2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v[e] & 0xFFFFu));
        f[2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v[e] >> 16));
      }
    }
  }
}

template <int X>
__global__ __launch_bounds__(256) void act_quant_block_fp8_kernel(const void* __restrict__ x, int64_t m, int k,
                                                                  uint8_t* __restrict__ q,
                                                                  uint8_t* __restrict__ scale) {
  const int kblocks = k / 128;
  const int64_t blk = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;  // (row, K block)
  if (blk >= m * kblocks) return;  // 16-lane groups leave together
  const int sub = threadIdx.x & 15;
  const int64_t row = blk / kblocks;
  const int kb = (int)(blk % kblocks);
  const int64_t idx = row * k + kb * 128 + sub * 8;
  float f[8];
  load_act8<X>(x, idx, f);
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const uint32_t bits = __float_as_uint(fmaxf(amax, 1.0e-4f) * (1.0f / 448.0f));
  int e8 = (int)((bits >> 23) & 0xFF) + ((bits & 0x7FFFFF) != 0 ? 1 : 0);
  e8 = min(254, max(1, e8));
  const float s = __uint_as_float((uint32_t)e8 << 23);
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = fminf(fmaxf(f[e] / s, -448.0f), 448.0f);
  int lo = 0, hi = 0;
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], lo, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], lo, true);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4], f[5], hi, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6], f[7], hi, true);
  *reinterpret_cast<u32x2*>(q + idx) = u32x2{(uint32_t)lo, (uint32_t)hi};
  if (sub == 0) scale[row * kblocks + kb] = (uint8_t)e8;
}

struct BlockFp8Params {
  const uint8_t* a;    // E4M3 [M][K], row-major
  const uint8_t* as;   // E8M0 [M][K/128]
  int64_t m;
  int n;
  int k;
  const uint8_t* wq;   // E4M3 in 1 KiB tiles (16 rows x 64 K)
  const uint8_t* ws8;  // E8M0 [ceil(N/128)][K/128]
  int kblocks;
  int split;
  int kb_per_split;
  int tiles_n;
  int tiles_m;
  uint16_t* out;
  float* partial;      // [split][M][N] when split > 1
  int w_rowmajor;      // weights as the checkpoint's row-major [N][K] bytes instead of 1 KiB tiles
};

// Workgroup tile: 64*R output channels x 16*C tokens over one K split, one
// 128-K block per step.  Per step, buffer_load ... lds copies the token tile
// (16C rows x 128 B, part q of row t at q ^ swz128(t)) and each wavefront's R
// weight strips (two 1 KiB tiles each: K windows 2kb and 2kb+1) into LDS,
// double buffered.  A lane's 32-byte MFMA operand is K 16j..16j+15 and
// 64+16j..64+16j+15 of the block (j = lane/16) for both operands.
template <int R, int C>
__global__ __launch_bounds__(256, 2) void w8a8_block_kernel(BlockFp8Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][16 * C * 128];
  __shared__ __attribute__((aligned(16))) uint8_t wts[2][4][R * 2048];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // XCD-aware item order, as in w8a16_kernel
  const int items = p.split * p.tiles_m * p.tiles_n;
  const int per_xcd = (items + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= items) return;
  const int tn = item % p.tiles_n;
  const int tm = (item / p.tiles_n) % p.tiles_m;
  const int sp = item / (p.tiles_n * p.tiles_m);

  const int kb_begin = sp * p.kb_per_split;
  const int kb_end = min(p.kblocks, kb_begin + p.kb_per_split);
  const int nk = kb_end - kb_begin;  // may be 0 for a trailing split: it writes zeros
  const int wins = p.k / kWin;
  const int strips = p.n >> 4;
  const int strip0 = tn * 4 * R + wave * R;

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);

  constexpr int kActDma = 2 * C;
  constexpr int kActPerWave = (kActDma + 3) / 4;
  uint32_t a_off[kActPerWave];
#pragma unroll
  for (int i = 0; i < kActPerWave; ++i) {
    const int q = wave + 4 * i;
    const int row = q * 8 + (lane >> 3);
    const int64_t tok = (int64_t)tm * 16 * C + row;
    const int part = (lane & 7) ^ swz128(row);
    a_off[i] = (q < kActDma && tok < p.m) ? (uint32_t)(tok * p.k + part * 16) : kLinOob;
  }
  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w_off[r] = strip0 + r < strips ? weight_lane_offset(p.w_rowmajor, strip0 + r, lane, p.k, wins) : kLinOob;
  // the wavefront's R strips lie in one 128-row scale block (R divides 8);
  // lane i holds the E8M0 bytes of K blocks i, 64 + i, 128 + i, 192 + i
  uint32_t srow[4] = {0, 0, 0, 0};
  {
    const uint8_t* row = p.ws8 + (int64_t)(min(strip0, strips - 1) >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }
  const int n16 = lane & 15;
  const int j = lane >> 4;
  // activation scale rows of this lane's tokens (127 = 2^0 past the last token)
  const uint8_t* srow_t[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t tok = (int64_t)tm * 16 * C + c * 16 + n16;
    srow_t[c] = tok < p.m ? p.as + tok * p.kblocks : nullptr;
  }

  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][wave * 1024]));
  const uint32_t wts_lds = __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][wave][0]));
  auto issue = [&](int kb, int buf) {
#pragma unroll
    for (int i = 0; i < kActPerWave; ++i) {
      const int q = wave + 4 * i;
      if (q < kActDma)
        lds_dma16(a_rsrc, lds_ptr(xs_lds + buf * (uint32_t)sizeof(xs[0]) + i * 4096), a_off[i], kb * 128);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t wb = wts_lds + buf * (uint32_t)sizeof(wts[0]) + r * 2048;
      lds_dma16(w_rsrc, lds_ptr(wb), w_off[r], (2 * kb) * wstep);
      lds_dma16(w_rsrc, lds_ptr(wb + 1024), w_off[r], (2 * kb + 1) * wstep);
    }
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int kb, auto u_c, auto pf_c) {
    constexpr int u = decltype(u_c)::value;
    int st[C];  // token scales, loaded before this step's prefetch is issued
#pragma unroll
    for (int c = 0; c < C; ++c) st[c] = srow_t[c] != nullptr ? (int)srow_t[c][kb] : 127;
    if constexpr (decltype(pf_c)::value) issue(kb + 1, u ^ 1);
    const uint32_t word = kb < 64 ? srow[0] : (kb < 128 ? srow[1] : (kb < 192 ? srow[2] : srow[3]));
    const int sw = __builtin_amdgcn_readlane((int)word, kb & 63);
    i32x8 wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(&wts[u][wave][r * 2048 + lane * 16]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(&wts[u][wave][r * 2048 + 1024 + lane * 16]);
      wv[r] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int row = c * 16 + n16;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + ((j ^ swz128(row)) * 16)]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + (((4 + j) ^ swz128(row)) * 16)]);
      const i32x8 tv = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][c] = mfma_fp8_block(wv[r], tv, acc[r][c], sw, st[c]);
    }
    __syncthreads();
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using PF = std::true_type;
  using NOPF = std::false_type;

  if (nk > 0) {
    issue(kb_begin, 0);
    __syncthreads();
    int i = 0;
    for (; i + 2 < nk; i += 2) {
      step(kb_begin + i, U0{}, PF{});
      step(kb_begin + i + 1, U1{}, PF{});
    }
    // the last step issues no prefetch, so no LDS DMA is in flight at exit
    if (nk - i == 2) {
      step(kb_begin + i, U0{}, PF{});
      step(kb_begin + i + 1, U1{}, NOPF{});
    } else {
      step(kb_begin + i, U0{}, NOPF{});
    }
  }

  // epilogue: lane holds channels 16*strip + 4*j + (0..3) of token c*16 + n16
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int strip = strip0 + r;
    if (strip >= strips) continue;
    const int n = strip * 16 + 4 * j;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t tok = (int64_t)tm * 16 * C + c * 16 + n16;
      if (tok >= p.m) continue;
      const float v[4] = {acc[r][c][0], acc[r][c][1], acc[r][c][2], acc[r][c][3]};
      if (p.split == 1) {
        uint16_t* dst = p.out + tok * p.n + n;
        *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, false);
      } else {
        float* dst = p.partial + ((int64_t)sp * p.m + tok) * p.n + n;
        *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

// Up to 16 tokens with a K split: the split runs inside the workgroup, as in
// w8a16_wsplit_kernel.  Workgroup tile: one 16-channel strip x 16 tokens;
// wavefront w of the `split` wavefronts runs split w's K blocks [w * kbps,
// min(kblocks, (w + 1) * kbps)) -- the MFMA chain of a split workgroup of
// w8a8_block_kernel -- and the workgroup sums the partials through LDS in
// split order, the additions of split_reduce_kernel: the same bits as the
// two-launch path for the same split.  Per K block a lane loads its two
// 16-byte weight parts, its token's two 16-byte parts and its token's E8M0
// byte straight to registers, D blocks in flight; blocks past a split's end
// load out of range (zeros, and a zero scale byte, 2^-127, times zero).
// KPS > 0: KPS blocks per split (checked on the host), straight-line code.
// LDS_ACT (KPS > 0, splits covering K exactly, up to 4 tokens): the split's
// activation rows (KPS*128 bytes each, rows padded to whole KiB) are copied
// into LDS with 1 KiB DMAs first and the MFMA operands read from there, as in
// w8a16_wsplit_kernel.
template <int D, int KPS, bool LDS_ACT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2))) void w8a8_wsplit_kernel(
    BlockFp8Params p) {
  __shared__ __attribute__((aligned(16))) f32x4 red[8][64];
  extern __shared__ __attribute__((aligned(16))) uint8_t act_lds[];  // LDS_ACT: [split][M][stride], [split][32] zeros
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // = split index
  const int tiles = p.tiles_m * p.tiles_n;
  const int per_xcd = (tiles + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= tiles) return;
  const int strip = item % p.tiles_n;
  const int tm = item / p.tiles_n;

  const int kb_begin = wave * p.kb_per_split;
  const int kb_end = min(p.kblocks, kb_begin + p.kb_per_split);
  const int wins = p.k / kWin;
  const int strips = p.n >> 4;
  const int n16 = lane & 15;
  const int j = lane >> 4;

  // the strip's 128-row scale block: lane i holds the E8M0 bytes of K blocks i, 64 + i, 128 + i, 192 + i
  uint32_t srow[4] = {0, 0, 0, 0};
  {
    const uint8_t* row = p.ws8 + (int64_t)(strip >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.as, (short)0, (int)(p.m * p.kblocks), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);
  const int wstep = weight_window_step(p.w_rowmajor);
  const uint32_t w_off = weight_lane_offset(p.w_rowmajor, strip, lane, p.k, wins);
  const int64_t tok = (int64_t)tm * 16 + n16;
  const uint32_t a_off = tok < p.m ? (uint32_t)(tok * p.k + j * 16) : kLinOob;
  const uint32_t s_off = tok < p.m ? (uint32_t)(tok * p.kblocks) : kLinOob;

  constexpr int kRowBytes = KPS * 128;
  constexpr int kRowStride = (kRowBytes + 1023) / 1024 * 1024;
  const uint8_t* act_row = nullptr;
  if constexpr (LDS_ACT) {
    static_assert(KPS > 0, "LDS activations need a fixed block count per split");
    const int m = (int)p.m;
    uint8_t* mine = act_lds + wave * m * kRowStride;
    uint8_t* zeros = act_lds + p.split * m * kRowStride + wave * 32;  // this wavefront's own: no barrier needed
    if (lane < 2) *reinterpret_cast<u32x4*>(zeros + 16 * lane) = u32x4{0, 0, 0, 0};
    for (int row = 0; row < m; ++row)
#pragma unroll
      for (int q = 0; q < kRowStride / 1024; ++q) {
        const int byte = q * 1024 + lane * 16;  // padding past the row copies zeros
        lds_dma16(a_rsrc, (lds_void_ptr)(mine + row * kRowStride + q * 1024),
                  byte < kRowBytes ? (uint32_t)(row * p.k + kb_begin * 128 + byte) : kLinOob, 0);
      }
    act_row = n16 < m ? mine + n16 * kRowStride + 16 * j : zeros;
  }

  u32x4 wr[D][2];
  u32x4 ar[D][2];
  int st[D];
  // a block past the split's end reads at kLinOob + (small) soffset: out of range, zeros
  auto load = [&](int kb, int t) {
    const bool in = kb < kb_end;
    const uint32_t wo = in ? w_off : kLinOob;
    const uint32_t ao = in ? a_off : kLinOob;
    wr[t][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, wo, (2 * kb) * wstep, 0));
    wr[t][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, wo, (2 * kb + 1) * wstep, 0));
    if constexpr (!LDS_ACT) {
      ar[t][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, ao, kb * 128, 0));
      ar[t][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, ao, kb * 128 + 64, 0));
    }
    st[t] = (int)__builtin_amdgcn_raw_buffer_load_b8(s_rsrc, in ? s_off : kLinOob, kb, 0);
  };
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  auto consume = [&](int kb, int t) {
    const int kbc = min(kb, p.kblocks - 1);
    const uint32_t word = kbc < 64 ? srow[0] : (kbc < 128 ? srow[1] : (kbc < 192 ? srow[2] : srow[3]));
    const int sw = __builtin_amdgcn_readlane((int)word, kbc & 63);
    const i32x8 wv = {(int)wr[t][0][0], (int)wr[t][0][1], (int)wr[t][0][2], (int)wr[t][0][3],
                      (int)wr[t][1][0], (int)wr[t][1][1], (int)wr[t][1][2], (int)wr[t][1][3]};
    u32x4 lo, hi;
    if constexpr (LDS_ACT) {
      // padding lanes all read the zero block (one address: a broadcast)
      const int step = n16 < (int)p.m ? (kb - kb_begin) * 128 : 0;
      lo = *reinterpret_cast<const u32x4*>(act_row + step);
      hi = *reinterpret_cast<const u32x4*>(act_row + step + (n16 < (int)p.m ? 64 : 16));
    } else {
      lo = ar[t][0];
      hi = ar[t][1];
    }
    const i32x8 tv = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    acc = mfma_fp8_block(wv, tv, acc, sw, st[t]);
  };

  // sched_barrier keeps each group of loads where it stands (see w8a16_wsplit_kernel)
  if constexpr (KPS > 0) {
    constexpr int kDepth = D < KPS ? D : KPS;
#pragma unroll
    for (int t = 0; t < kDepth; ++t) {
      load(kb_begin + t, t);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < KPS; ++i) {
      consume(kb_begin + i, i % kDepth);
      if (i + kDepth < KPS) load(kb_begin + i + kDepth, i % kDepth);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int t = 0; t < D; ++t) load(kb_begin + t, t);
    for (int i = 0; i < p.kb_per_split; i += D) {
#pragma unroll
      for (int t = 0; t < D; ++t) {
        consume(kb_begin + i + t, t);
        load(kb_begin + i + t + D, t);
      }
    }
  }

  red[wave][lane] = acc;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int64_t t = (int64_t)tm * 16 + n16;
    if (t < p.m && strip < strips) {
      f32x4 sum = red[0][lane];
      for (int w = 1; w < p.split; ++w) {
        const f32x4 v = red[w][lane];
        sum[0] += v[0];
        sum[1] += v[1];
        sum[2] += v[2];
        sum[3] += v[3];
      }
      const float v[4] = {sum[0], sum[1], sum[2], sum[3]};
      uint16_t* dst = p.out + t * p.n + strip * 16 + 4 * j;
      *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, false);
    }
  }
}

// Many tokens: a three-stage pipeline through LDS.  Per K block, inline-asm
// buffer_load ... lds copies the token tile (16C rows x 128 B, part q of row t
// at q ^ swz128(t)), each wavefront's R weight strips (2 KiB each) and the
// tokens' E8M0 scale dwords (the 4-block group holding block kb; K % 512 == 0)
// two blocks ahead of the compute; one s_waitcnt vmcnt(n) (n = one step's
// copies, left in flight) and a barrier publish the next block.  No register
// holds data in flight, so nothing the compiler moves can read it early.
// H = 2: 8 wavefronts (two per SIMD) share each strip group's weights, wave
// w taking strip group w % 4 and token half w / 4; each copies one of the two
// 1 KiB weight tiles of its strips.
template <int R, int C, int H>
__global__ __launch_bounds__(256 * H, 1) void w8a8_block_prefill_kernel(BlockFp8Params p) {
  constexpr int kWaves = 4 * H;
  constexpr int kTokRows = 16 * C * H;
  constexpr int kTokBytes = kTokRows * 128;
  constexpr int kScaleTok = kTokRows / kWaves;  // tokens per wavefront's scale copy
  static_assert(kScaleTok <= 64, "one scale copy per wavefront");
  __shared__ __attribute__((aligned(16))) uint8_t xs[3][kTokBytes];
  __shared__ __attribute__((aligned(16))) uint8_t wts[3][4][R * 2048];
  __shared__ __attribute__((aligned(16))) uint32_t scs[3][kWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sg = wave & 3;   // strip group
  const int half = wave >> 2;  // token half (H = 2)

  const int items = p.split * p.tiles_m * p.tiles_n;
  const int per_xcd = (items + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= items) return;
  const int tn = item % p.tiles_n;
  const int tm = (item / p.tiles_n) % p.tiles_m;
  const int sp = item / (p.tiles_n * p.tiles_m);

  const int kb_begin = sp * p.kb_per_split;
  const int kb_end = min(p.kblocks, kb_begin + p.kb_per_split);
  const int nk = kb_end - kb_begin;
  const int wins = p.k / kWin;
  const int strips = p.n >> 4;
  const int strip0 = tn * 4 * R + sg * R;
  const int64_t tok0 = (int64_t)tm * kTokRows;

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t as_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.as, (short)0, (int)(p.m * p.kblocks), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);

  constexpr int kActDma = kTokRows / 8;
  static_assert(kActDma % kWaves == 0, "every wavefront issues the same number of token copies");
  constexpr int kActPerWave = kActDma / kWaves;
  uint32_t a_off[kActPerWave];
#pragma unroll
  for (int i = 0; i < kActPerWave; ++i) {
    const int q = wave + kWaves * i;
    const int row = q * 8 + (lane >> 3);
    const int64_t tok = tok0 + row;
    const int part = (lane & 7) ^ swz128(row);
    a_off[i] = tok < p.m ? (uint32_t)(tok * p.k + part * 16) : kLinOob;
  }
  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    w_off[r] = strip0 + r < strips ? weight_lane_offset(p.w_rowmajor, strip0 + r, lane, p.k, wins) : kLinOob;
  // scale dword of token tok0 + kScaleTok * wave + lane (lanes past kScaleTok
  // or past the last token read out of range into unused slots)
  const int64_t stok = tok0 + kScaleTok * wave + lane;
  const uint32_t s_off = (lane < kScaleTok && stok < p.m) ? (uint32_t)(stok * p.kblocks) : kLinOob;
  uint32_t srow[4] = {0, 0, 0, 0};
  {
    const uint8_t* row = p.ws8 + (int64_t)(min(strip0, strips - 1) >> 3) * p.kblocks;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (64 * q + lane < p.kblocks) srow[q] = row[64 * q + lane];
  }
  const int n16 = lane & 15;
  const int j = lane >> 4;

  constexpr int kStepLoads = kActPerWave + 2 * R / H + 1;
  static_assert(kStepLoads < 64, "vmcnt range");
  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][wave * 1024]));
  const uint32_t wts_lds = __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][sg][0]));
  const uint32_t scs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&scs[0][wave][0]));
  auto issue = [&](int kb, int buf) {
#pragma unroll
    for (int i = 0; i < kActPerWave; ++i)
      lds_copy16(a_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + i * kWaves * 1024, a_off[i], kb * 128);
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
        if (H == 1 || t == half)
          lds_copy16(w_rsrc, wts_lds + buf * (uint32_t)sizeof(wts[0]) + r * 2048 + t * 1024, w_off[r],
                     (2 * kb + t) * wstep);
    }
    lds_copy4(as_rsrc, scs_lds + buf * (uint32_t)sizeof(scs[0]), s_off, kb & ~3);
  };

  f32x4 acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Step kb: issue block kb + 2 into buffer (u + 2) % 3 (released by step
  // kb - 1's barrier), compute block kb from buffer u, wait for block kb + 1.
  auto step = [&](int kb, auto u_c) {
    constexpr int u = decltype(u_c)::value;
    const bool issue2 = kb + 2 < kb_end;
    if (issue2) issue(kb + 2, (u + 2) % 3);
    const uint32_t word = kb < 64 ? srow[0] : (kb < 128 ? srow[1] : (kb < 192 ? srow[2] : srow[3]));
    const int sw = __builtin_amdgcn_readlane((int)word, kb & 63);
    i32x8 wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(&wts[u][sg][r * 2048 + lane * 16]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(&wts[u][sg][r * 2048 + 1024 + lane * 16]);
      wv[r] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int row = half * 16 * C + c * 16 + n16;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + ((j ^ swz128(row)) * 16)]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + (((4 + j) ^ swz128(row)) * 16)]);
      const i32x8 tv = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      const int st = (int)((scs[u][row / kScaleTok][row % kScaleTok] >> (8 * (kb & 3))) & 0xFF);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][c] = mfma_fp8_block(wv[r], tv, acc[r][c], sw, st);
    }
    if (issue2)
      lds_dma_wait_keep<kStepLoads>();  // this wavefront's copies of block kb + 1 have landed
    else
      lds_dma_wait_all();
    __syncthreads();  // ... and everyone's; buffer u is free again
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using U2 = std::integral_constant<int, 2>;

  if (nk > 0) {
    issue(kb_begin, 0);
    if (nk > 1) {
      issue(kb_begin + 1, 1);
      lds_dma_wait_keep<kStepLoads>();
    } else {
      lds_dma_wait_all();
    }
    __syncthreads();
    // the last two steps issue nothing, and the last waits for everything,
    // so no copy is outstanding at exit
    for (int i = 0; i < nk; i += 3) {
      step(kb_begin + i, U0{});
      if (i + 1 < nk) step(kb_begin + i + 1, U1{});
      if (i + 2 < nk) step(kb_begin + i + 2, U2{});
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int strip = strip0 + r;
    if (strip >= strips) continue;
    const int n = strip * 16 + 4 * j;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t tok = tok0 + half * 16 * C + c * 16 + n16;
      if (tok >= p.m) continue;
      const float v[4] = {acc[r][c][0], acc[r][c][1], acc[r][c][2], acc[r][c][3]};
      if (p.split == 1) {
        uint16_t* dst = p.out + tok * p.n + n;
        *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, false);
      } else {
        float* dst = p.partial + ((int64_t)sp * p.m + tok) * p.n + n;
        *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

// Large grids without a K split: 256 tokens x CH (256 or 128) channels per
// workgroup, two stages through LDS.  Wavefront (wm, wn) owns the TM token
// tiles wm*TM .. (16 tokens each) and the TN strips wn*TN .. of the tile (at
// most 128 channels: inside one E8M0 row block, so its weight scale is one
// byte per K block); it keeps its TN weight fragments in registers for the
// block and streams its token fragments through.  With 256 x 256 a K block
// is 256 MFMAs per SIMD between two barriers (4x the 128 x 256 kernel above),
// so the barrier and the LDS read latency at the top of each block weigh
// less.  buffer_load ... lds copies block kb + 1 (256 token rows of 128 B,
// part q of row t at q ^ swz128(t); the strips' two 1 KiB weight tiles, or
// with row-major weights (RM) their CH rows like the token rows; the tokens'
// E8M0 dwords) while block kb is computed.  The work items go to the XCDs in
// contiguous runs, and inside a run groups of kGemmGroupM token tiles walk the
// channel tiles together, so one XCD's L2 serves each token tile and each
// weight tile to several workgroups.  The accumulation per output is the same
// chain of scaled MFMAs in K-block order as in the kernels above: same bits.
constexpr int kGemmGroupM = 4;
// The wavefront grid: WM x WN wavefronts (wave = wm * WN + wn), each TM =
// 16 / WM token tiles x TN = CH / 16 / WN strips.  4 x 2: 8 wavefronts, two
// per SIMD (each 64 tokens x 128 or 64 channels); 2 x 2: one per SIMD, 128 x
// 128 at 256 channels (456 registers, more of them copied around the MFMAs).
#ifndef DSV4_GEMM256_WM
#define DSV4_GEMM256_WM 4
#endif
#ifndef DSV4_GEMM256_WN
#define DSV4_GEMM256_WN 2
#endif
constexpr int kGemm256Wm = DSV4_GEMM256_WM;
constexpr int kGemm256Wn = DSV4_GEMM256_WN;

template <int WM, int WN, int CH, bool RM>
__global__ __launch_bounds__(64 * WM * WN, 1) void w8a8_gemm256_kernel(BlockFp8Params p) {
  constexpr int kWaves = WM * WN;
  constexpr int kTok = 256;
  constexpr int kStrips = CH / 16;
  constexpr int TM = 16 / WM;
  constexpr int TN = kStrips / WN;
  static_assert(kWaves == 4 || kWaves == 8, "4 or 8 wavefronts");
  static_assert(CH == 128 || CH == 256, "128 or 256 channels per workgroup");
  static_assert(16 % WM == 0 && kStrips % WN == 0 && TN * 16 <= 128, "a wavefront's strips lie in one scale block");
  static_assert(kStrips % kWaves == 0 && (CH / 8) % kWaves == 0, "every wavefront issues the same copies");
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kTok * 128];
  __shared__ __attribute__((aligned(16))) uint8_t wts[2][CH * 128];
  __shared__ __attribute__((aligned(16))) uint32_t scs[2][kTok];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;

  const int items = p.tiles_m * p.tiles_n;
  const int per_xcd = (items + kLinXcds - 1) / kLinXcds;
  const int item = (blockIdx.x % kLinXcds) * per_xcd + blockIdx.x / kLinXcds;
  if (item >= items) return;
  const int group = item / (kGemmGroupM * p.tiles_n);
  const int first_m = group * kGemmGroupM;
  const int gm = min(kGemmGroupM, p.tiles_m - first_m);
  const int in_group = item - group * kGemmGroupM * p.tiles_n;
  const int tm = first_m + in_group % gm;
  const int tn = in_group / gm;

  const int wins = p.k / kWin;
  const int strips = p.n >> 4;
  const int64_t tok0 = (int64_t)tm * kTok;

  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.a, (short)0, (int)(p.m * p.k), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t as_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.as, (short)0, (int)(p.m * p.kblocks), kLinRsrcFlags);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wq, (short)0, (int)((int64_t)p.n * p.k), kLinRsrcFlags);

  // token copies: copy q (0..31) fills rows 8q .. 8q + 7; wavefront w issues
  // q = w, w + kWaves, ...
  constexpr int kActPerWave = 32 / kWaves;
  uint32_t a_off[kActPerWave];
#pragma unroll
  for (int i = 0; i < kActPerWave; ++i) {
    const int row = (wave + kWaves * i) * 8 + (lane >> 3);
    const int64_t tok = tok0 + row;
    const int part = (lane & 7) ^ swz128(row);
    a_off[i] = tok < p.m ? (uint32_t)(tok * p.k + part * 16) : kLinOob;
  }
  // weight copies.  Tiled (RM = false): wavefront w copies strips w*kSpw ..
  // of the tile, both 1 KiB windows of the block each.  Row-major (RM): the
  // CH rows like the token rows, copy q = w, w + kWaves, .. filling rows
  // 8q .. 8q + 7 (part q of row t at q ^ swz128(t)), read back like the token
  // fragments.
  constexpr int kSpw = kStrips / kWaves;
  constexpr int kWCopies = RM ? CH / 8 / kWaves : 2 * kSpw;
  const int wstep = weight_window_step(p.w_rowmajor);
  uint32_t w_off[RM ? kWCopies : kSpw];
#pragma unroll
  for (int s = 0; s < (RM ? kWCopies : kSpw); ++s) {
    if constexpr (RM) {
      const int row = (wave + kWaves * s) * 8 + (lane >> 3);
      const int part = (lane & 7) ^ swz128(row);
      w_off[s] = (uint32_t)((int64_t)(tn * CH + row) * p.k + part * 16);
    } else {
      const int strip = tn * kStrips + wave * kSpw + s;
      w_off[s] = strip < strips ? weight_lane_offset(p.w_rowmajor, strip, lane, p.k, wins) : kLinOob;
    }
  }
  // scale dwords: wavefront w copies tokens 64 (w % 4) .. + 63 (with 8
  // wavefronts two copy the same bytes to the same place: no branch in the
  // loop body)
  const int64_t stok = tok0 + 64 * (wave & 3) + lane;
  const uint32_t s_off = stok < p.m ? (uint32_t)(stok * p.kblocks) : kLinOob;
  // this wavefront's weight scale row (host: N % CH == 0, so it exists;
  // K <= 8192, so lane kb holds block kb's byte)
  uint32_t srow = 0;
  if (lane < p.kblocks) srow = p.ws8[(int64_t)((tn * CH + wn * TN * 16) >> 7) * p.kblocks + lane];
  // A wait the compiler sees: its own wait before the first use of srow
  // would otherwise sit inside the K loop (the waits of the copies are
  // inline asm, which it does not count), where it also waits for the copies
  // issued just before it.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  const int n16 = lane & 15;
  const int j = lane >> 4;

  // copy destinations: this wavefront's buffer-0 addresses, made scalar once
  // (the K loop sets M0 with scalar adds only)
  const uint32_t xs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&xs[0][wave * 1024]));
  const uint32_t wts_lds =
      __builtin_amdgcn_readfirstlane(lds_addr(&wts[0][RM ? wave * 1024 : wave * kSpw * 2048]));
  const uint32_t scs_lds = __builtin_amdgcn_readfirstlane(lds_addr(&scs[0][64 * (wave & 3)]));
  auto issue = [&](int kb, int buf) {
#pragma unroll
    for (int i = 0; i < kActPerWave; ++i)
      lds_copy16(a_rsrc, xs_lds + buf * (uint32_t)sizeof(xs[0]) + i * kWaves * 1024, a_off[i], kb * 128);
#pragma unroll
    for (int s = 0; s < (RM ? kWCopies : kSpw); ++s) {
      if constexpr (RM) {
        lds_copy16(w_rsrc, wts_lds + buf * (uint32_t)sizeof(wts[0]) + s * kWaves * 1024, w_off[s], kb * 128);
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
          lds_copy16(w_rsrc, wts_lds + buf * (uint32_t)sizeof(wts[0]) + s * 2048 + t * 1024, w_off[s],
                     (2 * kb + t) * wstep);
      }
    }
    lds_copy4(as_rsrc, scs_lds + buf * (uint32_t)sizeof(scs[0]), s_off, kb & ~3);
  };

  f32x4 acc[TN][TM];
#pragma unroll
  for (int r = 0; r < TN; ++r)
#pragma unroll
    for (int c = 0; c < TM; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Step kb: issue block kb + 1 into the other buffer (released by step
  // kb - 1's barrier), compute block kb, wait for block kb + 1.
  auto step = [&](int kb, auto u_c) {
    constexpr int u = decltype(u_c)::value;
    // the last block re-copies itself into the idle buffer (no branch in the
    // loop body; nothing reads that buffer again)
    issue(min(kb + 1, p.kblocks - 1), u ^ 1);
    const int sw = __builtin_amdgcn_readlane((int)srow, kb);
    // the wavefront's TN weight fragments, kept for the block; the token
    // fragments stream through, one per TN MFMAs
    i32x8 wv[TN];
#pragma unroll
    for (int r = 0; r < TN; ++r) {
      u32x4 lo, hi;
      if constexpr (RM) {
        const int row = (wn * TN + r) * 16 + n16;
        lo = *reinterpret_cast<const u32x4*>(&wts[u][row * 128 + ((j ^ swz128(row)) * 16)]);
        hi = *reinterpret_cast<const u32x4*>(&wts[u][row * 128 + (((4 + j) ^ swz128(row)) * 16)]);
      } else {
        const uint8_t* wp = &wts[u][(wn * TN + r) * 2048 + lane * 16];
        lo = *reinterpret_cast<const u32x4*>(wp);
        hi = *reinterpret_cast<const u32x4*>(wp + 1024);
      }
      wv[r] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int c = 0; c < TM; ++c) {
      const int row = (wm * TM + c) * 16 + n16;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + ((j ^ swz128(row)) * 16)]);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(&xs[u][row * 128 + (((4 + j) ^ swz128(row)) * 16)]);
      const i32x8 tv = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      const int st = (int)((scs[u][row] >> (8 * (kb & 3))) & 0xFF);
#pragma unroll
      for (int r = 0; r < TN; ++r) acc[r][c] = mfma_fp8_block(wv[r], tv, acc[r][c], sw, st);
    }
    // the block's MFMAs stay ahead of the wait (the scheduler would otherwise
    // sink them past the barrier, leaving the wait right behind the copies)
    __builtin_amdgcn_sched_barrier(0);
    lds_dma_wait_all();  // this wavefront's copies of block kb + 1 have landed
    __syncthreads();     // ... and everyone's; buffer u is free again
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;

  issue(0, 0);
  lds_dma_wait_all();
  __syncthreads();
  // kblocks is a multiple of 4 (host check); the last step issues nothing
  for (int kb = 0; kb < p.kblocks; kb += 2) {
    step(kb, U0{});
    step(kb + 1, U1{});
  }

#pragma unroll
  for (int r = 0; r < TN; ++r) {
    const int n = (tn * kStrips + wn * TN + r) * 16 + 4 * j;
#pragma unroll
    for (int c = 0; c < TM; ++c) {
      const int64_t tok = tok0 + (wm * TM + c) * 16 + n16;
      if (tok >= p.m) continue;
      const float v[4] = {acc[r][c][0], acc[r][c][1], acc[r][c][2], acc[r][c][3]};
      uint16_t* dst = p.out + tok * p.n + n;
      *reinterpret_cast<u32x2*>(dst) = finish_bf16x4(v, dst, false);
    }
  }
}

// The channels per workgroup of the 256-token kernel (0: another kernel):
// no K split, K % 512 == 0, K <= 8192, N a multiple of the channel tile, and
// at least one workgroup per CU -- 256 channels where that fills the GPU,
// else 128.
static int gemm256_channels(int64_t m, int64_t n, int64_t k, int split) {
  if (split != 1 || k % 512 != 0 || k > 8192) return 0;
  const int64_t tiles_m = (m + 255) / 256;
  if (n % 256 == 0 && tiles_m * (n / 256) >= 256) return 256;
  if (n % 128 == 0 && tiles_m * (n / 128) >= 256) return 128;
  return 0;
}

static void launch_w8a8_block_kernel(const BlockFp8Params& p, int r, int c, hipStream_t stream) {
  const int items = p.split * p.tiles_m * p.tiles_n;
  const dim3 grid((unsigned)(((items + kLinXcds - 1) / kLinXcds) * kLinXcds));
  if (r == 4 && c == 8) hipLaunchKernelGGL((w8a8_block_prefill_kernel<4, 4, 2>), grid, dim3(512), 0, stream, p);
  else if (r == 4 && c == 4) hipLaunchKernelGGL((w8a8_block_prefill_kernel<4, 2, 2>), grid, dim3(512), 0, stream, p);
  else if (c == 1) hipLaunchKernelGGL((w8a8_block_kernel<2, 1>), grid, dim3(256), 0, stream, p);
  else if (c == 2) hipLaunchKernelGGL((w8a8_block_kernel<2, 2>), grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL((w8a8_block_kernel<2, 4>), grid, dim3(256), 0, stream, p);
}

// The in-workgroup split (w8a16_wsplit_kernel) for up to 16 tokens and 2..8
// splits, 16 channels per workgroup.  (17..64 tokens keep the split
// workgroups and the reduce launch: there the in-workgroup split measured
// 40-60% slower -- each wavefront re-reads its activations, no LDS sharing.)
static bool wsplit_geometry(int64_t m, int split, int* r, int* c) {
  if (m > 16 || split < 2 || split > 8) return false;
  *c = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
  *r = m <= 16 ? 1 : 2;
  return true;
}

template <bool FP8>
static void launch_w8a16_wsplit(const LinearParams& p, int r, int c, hipStream_t stream) {
  const int tiles = p.tiles_m * p.tiles_n;
  const dim3 grid((unsigned)(((tiles + kLinXcds - 1) / kLinXcds) * kLinXcds));
  const dim3 block((unsigned)(64 * p.split));
  const int wps = p.win_per_split;
  // activation rows through LDS: up to 4 tokens, splits covering K exactly, at most 32 KiB
  const bool lds = p.m <= 4 && wps * p.split == p.k / kWin && p.m * p.k * 2 <= 32768;
  const size_t lds_bytes = lds ? (size_t)(p.m * p.k * 2 + 32 * p.split) : 0;
  if (c == 1 && lds) {
    if (wps == 8) hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 8, FP8, true>), grid, block, lds_bytes, stream, p);
    else if (wps == 16)
      hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 16, FP8, true>), grid, block, lds_bytes, stream, p);
    else if (wps == 32)
      hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 32, FP8, true>), grid, block, lds_bytes, stream, p);
    else hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 0, FP8, false>), grid, block, 0, stream, p);
  } else if (c == 1) {
    if (wps == 8) hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 8, FP8, false>), grid, block, 0, stream, p);
    else if (wps == 16) hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 16, FP8, false>), grid, block, 0, stream, p);
    else if (wps == 32) hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 32, FP8, false>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((w8a16_wsplit_kernel<1, 1, 8, 0, FP8, false>), grid, block, 0, stream, p);
  } else if (c == 2) {
    hipLaunchKernelGGL((w8a16_wsplit_kernel<2, 2, 4, 0, FP8, false>), grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL((w8a16_wsplit_kernel<2, 4, 2, 0, FP8, false>), grid, block, 0, stream, p);
  }
}

template <bool FP8>
static void launch_w8a16_kernel(const LinearParams& p, int r, int c, hipStream_t stream) {
  const int items = p.split * p.tiles_m * p.tiles_n;
  const dim3 grid((unsigned)(((items + kLinXcds - 1) / kLinXcds) * kLinXcds));
  if (r == 4 && c == 8) hipLaunchKernelGGL((w8a16_kernel_w3<4, 8, FP8>), grid, dim3(256), 0, stream, p);
  else if (r == 4 && c == 4) hipLaunchKernelGGL((w8a16_kernel3<4, 4, FP8>), grid, dim3(256), 0, stream, p);
  else if (r == 2 && c == 8) hipLaunchKernelGGL((w8a16_kernel<2, 8, FP8>), grid, dim3(256), 0, stream, p);
  else if (c == 1) hipLaunchKernelGGL((w8a16_kernel<2, 1, FP8>), grid, dim3(256), 0, stream, p);
  else if ((c == 2 || c == 4) && (p.win_per_split == 8 || p.win_per_split == 4)) {
    // weights straight to registers, the split's token rows in LDS
    const size_t lds = (size_t)p.win_per_split * 16 * c * 128;
    if (c == 2 && p.win_per_split == 8)
      hipLaunchKernelGGL((w8a16_regw_kernel<2, 2, 8, 8, FP8>), grid, dim3(256), lds, stream, p);
    else if (c == 2)
      hipLaunchKernelGGL((w8a16_regw_kernel<2, 2, 8, 4, FP8>), grid, dim3(256), lds, stream, p);
    else if (p.win_per_split == 8)
      hipLaunchKernelGGL((w8a16_regw_kernel<2, 4, 8, 8, FP8>), grid, dim3(256), lds, stream, p);
    else
      hipLaunchKernelGGL((w8a16_regw_kernel<2, 4, 8, 4, FP8>), grid, dim3(256), lds, stream, p);
  }
  else if (c == 2) hipLaunchKernelGGL((w8a16_kernel<2, 2, FP8>), grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL((w8a16_kernel<2, 4, FP8>), grid, dim3(256), 0, stream, p);
}

}  // namespace dsv4

using namespace dsv4;

// Geometry of the instance chosen for (M, N): (R strips per wavefront, C
// token tiles).  Above 64 tokens the 256 x 128 tile, unless it leaves fewer
// than 512 workgroups (it would need a split-K reduction): then 256 x 64.
static void w8a16_geometry(int64_t m, int64_t n, int* r, int* c) {
  if (m <= 16) { *r = 2; *c = 1; }
  else if (m <= 32) { *r = 2; *c = 2; }
  else if (m <= 64) { *r = 2; *c = 4; }
  else if (((n + 255) / 256) * ((m + 127) / 128) >= 512) { *r = 4; *c = 8; }
  else { *r = 4; *c = 4; }
}

int32_t dsv4_w8a16_split_k(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return -1;
  int r, c;
  w8a16_geometry(m, n, &r, &c);
  const int64_t tiles = ((n + 64 * r - 1) / (64 * r)) * ((m + 16 * c - 1) / (16 * c));
  const int64_t wins = k / kWin;
  if (m <= 16) {
    // the in-workgroup split: 4 wavefronts, 8 from N = 8192 (K = 4096, M = 1..16:
    // N = 1024/4096 fastest at 4, N = 16384 at 8 -- the tiled weights 14.4 -> 11.7 us),
    // at least 4 windows each
    if (wins < 2) return 1;
    int split = n >= 8192 ? 8 : 4;
    while (split > 2 && wins / split < 4) split /= 2;
    return split;
  }
  int split = 1;
  // widen over K until about two workgroups per CU, keeping >= 4 windows per
  // split, at most 8 splits (16 measured slower at M = 1..64: the partial sums
  // and the fewer windows per split cost more than the extra workgroups gain)
  while (split < 8 && tiles * split < 512 && wins / (split * 2) >= 4) split *= 2;
  return split;
}

size_t dsv4_w8a16_workspace_bytes(int64_t m, int64_t n, int32_t split) {
  return split > 1 ? (size_t)split * (size_t)m * (size_t)n * sizeof(float) : 0;
}

int dsv4_launch_pack_int8(const int8_t* w, int64_t n, int64_t k, uint8_t* packed, hipStream_t stream) {
  const int64_t chunks = n * k / 16;
  const int64_t blocks = (chunks + 255) / 256;
  hipLaunchKernelGGL(pack_int8_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     reinterpret_cast<const uint8_t*>(w), n, k, packed);
  DSV4_CHECK_LAUNCH("pack_int8_kernel");
  return DSV4MOE_OK;
}

// ws (int8 format, bf16 [N]) or ws8 (FP8 format, E8M0 [ceil(N/128)][K/128]): exactly one is set.
int dsv4_launch_w8a16(const uint16_t* a, int64_t m, int64_t n, int64_t k, const uint8_t* wq,
                      const uint16_t* ws, const uint8_t* ws8, int32_t split, float* workspace, uint16_t* out,
                      hipStream_t stream, int accumulate, int w_rowmajor) {
  int r, c;
  const bool wsplit = wsplit_geometry(m, split, &r, &c);
  if (!wsplit) w8a16_geometry(m, n, &r, &c);
  LinearParams p;
  p.a = a;
  p.m = m;
  p.n = (int)n;
  p.k = (int)k;
  p.wq = wq;
  p.ws = ws;
  p.ws8 = ws8;
  p.kblocks = (int)(k / 128);
  p.split = split;
  const int wins = (int)(k / kWin);
  p.win_per_split = (wins + split - 1) / split;
  const int tile_n = wsplit ? 16 * r : 64 * r;
  p.tiles_n = (int)((n + tile_n - 1) / tile_n);
  p.tiles_m = (int)((m + 16 * c - 1) / (16 * c));
  p.out = out;
  p.partial = workspace;
  p.accumulate = accumulate;
  p.w_rowmajor = w_rowmajor;
  if (wsplit) {
    if (ws8 != nullptr)
      launch_w8a16_wsplit<true>(p, r, c, stream);
    else
      launch_w8a16_wsplit<false>(p, r, c, stream);
    DSV4_CHECK_LAUNCH("w8a16_wsplit_kernel");
    return DSV4MOE_OK;
  }
  if (ws8 != nullptr)
    launch_w8a16_kernel<true>(p, r, c, stream);
  else
    launch_w8a16_kernel<false>(p, r, c, stream);
  DSV4_CHECK_LAUNCH("w8a16_kernel");
  if (split > 1) {
    const int64_t quads = m * n / 4;
    hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                       workspace, split, m * n, out, accumulate);
    DSV4_CHECK_LAUNCH("split_reduce_kernel");
  }
  return DSV4MOE_OK;
}

// Block-FP8 W8A8 geometry: (R, C) = (2, 1 | 2 | 4) up to 64 tokens or when
// K % 512 != 0 (w8a8_block_kernel), then the three-stage kernel with 256
// channels x 128 tokens, or x 64 tokens when that leaves fewer than 512
// workgroups; split-K widened (powers of two up to 8, >= 2 K
// blocks per split) while the grid is below 512 workgroups.
static void w8a8_geometry(int64_t m, int64_t n, int64_t k, int* r, int* c) {
  *r = 2;
  if (m <= 16) *c = 1;
  else if (m <= 32) *c = 2;
  else if (m <= 64 || k % 512 != 0) *c = 4;
  else {
    *r = 4;
    *c = ((n + 255) / 256) * ((m + 127) / 128) >= 512 ? 8 : 4;
  }
}

int32_t dsv4_block_fp8_split_k(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return -1;
  int r, c;
  w8a8_geometry(m, n, k, &r, &c);
  const int64_t tiles = ((n + 64 * r - 1) / (64 * r)) * ((m + 16 * c - 1) / (16 * c));
  const int64_t kblocks = k / 128;
  if (m <= 16) {
    // the in-workgroup split, as for W8A16: 4 wavefronts, 8 from N = 8192 (K = 4096:
    // N = 16384 tiled 13.9 -> 11.1 us at 8), at least 2 K blocks each
    if (kblocks < 2) return 1;
    int split = n >= 8192 ? 8 : 4;
    while (split > 2 && kblocks / split < 2) split /= 2;
    return split;
  }
  int split = 1;
  while (split < 8 && tiles * split < 512 && kblocks / (split * 2) >= 2) split *= 2;
  return split;
}

int dsv4_launch_act_quant_block_fp8(const void* x, int32_t x_dtype, int64_t m, int64_t k, uint8_t* q, uint8_t* scale,
                                    hipStream_t stream) {
  const int64_t threads = m * (k / 128) * 16;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (x_dtype == 0)
    hipLaunchKernelGGL(act_quant_block_fp8_kernel<0>, grid, dim3(256), 0, stream, x, m, (int)k, q, scale);
  else if (x_dtype == 1)
    hipLaunchKernelGGL(act_quant_block_fp8_kernel<1>, grid, dim3(256), 0, stream, x, m, (int)k, q, scale);
  else
    hipLaunchKernelGGL(act_quant_block_fp8_kernel<2>, grid, dim3(256), 0, stream, x, m, (int)k, q, scale);
  DSV4_CHECK_LAUNCH("act_quant_block_fp8_kernel");
  return DSV4MOE_OK;
}

int dsv4_launch_block_fp8_gemm(const uint8_t* a, const uint8_t* as, int64_t m, int64_t n, int64_t k,
                               const uint8_t* wq, const uint8_t* ws8, int32_t split, float* workspace, uint16_t* out,
                               hipStream_t stream, int w_rowmajor) {
  int r, c;
  const bool wsplit = m <= 16 && split >= 2 && split <= 8;
  w8a8_geometry(m, n, k, &r, &c);
  BlockFp8Params p;
  p.a = a;
  p.as = as;
  p.m = m;
  p.n = (int)n;
  p.k = (int)k;
  p.wq = wq;
  p.ws8 = ws8;
  p.kblocks = (int)(k / 128);
  p.split = split;
  p.kb_per_split = (p.kblocks + split - 1) / split;
  p.tiles_n = (int)((n + 64 * r - 1) / (64 * r));
  p.tiles_m = (int)((m + 16 * c - 1) / (16 * c));
  p.out = out;
  p.partial = workspace;
  p.w_rowmajor = w_rowmajor;
  if (wsplit) {  // one strip x 16 tokens per workgroup, the split inside it
    p.tiles_n = (int)((n + 15) / 16);
    p.tiles_m = (int)((m + 15) / 16);
    const dim3 grid((unsigned)(((p.tiles_n * p.tiles_m + kLinXcds - 1) / kLinXcds) * kLinXcds));
    const dim3 block((unsigned)(64 * split));
    const int kbps = p.kb_per_split;
    const int stride = (kbps * 128 + 1023) / 1024 * 1024;
    // activation rows through LDS: up to 4 tokens, splits covering K exactly, at most 32 KiB
    const bool lds = m <= 4 && kbps * split == p.kblocks && split * m * stride <= 32768;
    const size_t lds_bytes = lds ? (size_t)(split * m * stride + 32 * split) : 0;
    if (lds && kbps == 4) hipLaunchKernelGGL((w8a8_wsplit_kernel<8, 4, true>), grid, block, lds_bytes, stream, p);
    else if (lds && kbps == 8) hipLaunchKernelGGL((w8a8_wsplit_kernel<8, 8, true>), grid, block, lds_bytes, stream, p);
    else if (lds && kbps == 16)
      hipLaunchKernelGGL((w8a8_wsplit_kernel<8, 16, true>), grid, block, lds_bytes, stream, p);
    else if (kbps == 4) hipLaunchKernelGGL((w8a8_wsplit_kernel<8, 4, false>), grid, block, 0, stream, p);
    else if (kbps == 8) hipLaunchKernelGGL((w8a8_wsplit_kernel<8, 8, false>), grid, block, 0, stream, p);
    else if (kbps == 16) hipLaunchKernelGGL((w8a8_wsplit_kernel<8, 16, false>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((w8a8_wsplit_kernel<4, 0, false>), grid, block, 0, stream, p);
    DSV4_CHECK_LAUNCH("w8a8_wsplit_kernel");
    return DSV4MOE_OK;
  }
  if (const int ch = gemm256_channels(m, n, k, split)) {
    p.tiles_m = (int)((m + 255) / 256);
    p.tiles_n = (int)(n / ch);
    const int items = p.tiles_m * p.tiles_n;
    const dim3 grid((unsigned)(((items + kLinXcds - 1) / kLinXcds) * kLinXcds));
    const dim3 block(64 * kGemm256Wm * kGemm256Wn);
    constexpr int WM = kGemm256Wm, WN = kGemm256Wn;
    if (ch == 256 && w_rowmajor) hipLaunchKernelGGL((w8a8_gemm256_kernel<WM, WN, 256, true>), grid, block, 0, stream, p);
    else if (ch == 256) hipLaunchKernelGGL((w8a8_gemm256_kernel<WM, WN, 256, false>), grid, block, 0, stream, p);
    else if (w_rowmajor) hipLaunchKernelGGL((w8a8_gemm256_kernel<WM, WN, 128, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((w8a8_gemm256_kernel<WM, WN, 128, false>), grid, block, 0, stream, p);
    DSV4_CHECK_LAUNCH("w8a8_gemm256_kernel");
    return DSV4MOE_OK;
  }
  launch_w8a8_block_kernel(p, r, c, stream);
  DSV4_CHECK_LAUNCH("w8a8_block_kernel");
  if (split > 1) {
    const int64_t quads = m * n / 4;
    hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                       workspace, split, m * n, out, 0);
    DSV4_CHECK_LAUNCH("split_reduce_kernel");
  }
  return DSV4MOE_OK;
}

// Workspace of the FP8-block shared expert: gate|up bf16 [T][2I], h bf16
// [T][I], split-K partials fp32 (the larger of the two linears' needs), each
// 256-byte aligned.
struct SharedFp8Workspace {
  uint16_t* gu;
  uint16_t* h;
  float* partial;
  int32_t split13, split2;
  size_t bytes;
};
static SharedFp8Workspace carve_shared_fp8(void* base, int64_t tokens, int hidden, int inter) {
  auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
  SharedFp8Workspace w{};
  w.split13 = dsv4_w8a16_split_k(tokens, 2 * (int64_t)inter, hidden);
  w.split2 = dsv4_w8a16_split_k(tokens, hidden, inter);
  const size_t gu = align((size_t)tokens * 2 * inter * 2);
  const size_t h = align((size_t)tokens * inter * 2);
  const size_t part = std::max(dsv4_w8a16_workspace_bytes(tokens, 2 * (int64_t)inter, w.split13),
                               dsv4_w8a16_workspace_bytes(tokens, hidden, w.split2));
  uint8_t* p = static_cast<uint8_t*>(base);
  w.gu = reinterpret_cast<uint16_t*>(p);
  w.h = reinterpret_cast<uint16_t*>(p + gu);
  w.partial = reinterpret_cast<float*>(p + gu + h);
  w.bytes = gu + h + align(part);
  return w;
}

size_t dsv4_shared_fp8_workspace_bytes(int64_t tokens, int hidden, int inter) {
  return tokens > 0 ? carve_shared_fp8(nullptr, tokens, hidden, inter).bytes : 0;
}

// out[T][H] (bf16, the routed sum) <- bf16(out + shared(x)), the shared expert
// as three dense steps over FP8-block weights: gate|up = bf16(x . W13^T),
// SwiGLU -> h bf16, bf16(h . W2^T) added into out.
int dsv4_launch_shared_fp8_add(const uint16_t* x, int64_t tokens, int hidden, int inter, const uint8_t* w13q,
                               const uint8_t* w13s8, const uint8_t* w2q, const uint8_t* w2s8, float clamp_limit,
                               uint16_t* out, void* workspace, hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  const SharedFp8Workspace w = carve_shared_fp8(workspace, tokens, hidden, inter);
  int rc = dsv4_launch_w8a16(x, tokens, 2 * (int64_t)inter, hidden, w13q, nullptr, w13s8, w.split13, w.partial, w.gu,
                             stream, 0, 0);
  if (rc != DSV4MOE_OK) return rc;
  const int64_t quads = tokens * (inter / 4);
  hipLaunchKernelGGL(swiglu_rows_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, w.gu, tokens,
                     inter, clamp_limit, w.h);
  DSV4_CHECK_LAUNCH("swiglu_rows_kernel");
  return dsv4_launch_w8a16(w.h, tokens, hidden, inter, w2q, nullptr, w2s8, w.split2, w.partial, out, stream, 1, 0);
}
