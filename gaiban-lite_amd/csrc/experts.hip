// Grouped expert GEMMs over tiled int4 group-128 weights on bf16 MFMA.
//
// Restates the two Marlin grouped GEMMs of vLLM's _fused_marlin_moe as called
// at runtime/dsv4_direct/moe_runtime.py:1829-1856, with the arithmetic of the
// reference torch path (runtime/dsv4_direct/ops/dense_moe.py:336-354):
//   stage 1: [g | u] = x[rows] . W13^T (fp32 accumulate), h = SiLU(min(g,L)) *
//            clamp(u,-L,L) in fp32, h rounded to bf16;  also writes the fp32
//            sum of each row's bf16 h over every 128-wide K group of stage 2;
//   stage 2: y = h . W2^T (fp32 accumulate) * route_weight, written fp32 per
//            (token, k) slot (the shared expert uses weight 1);
//   combine: out[t] = bf16( sum_j y[t*k+j] + y_shared[t] ), one rounding
//            (moe_runtime.py:1857,1873 with a single fp32 accumulation).
//
// Work decomposition.  One workgroup (4 wavefronts) per (expert block of the
// alignment, 128-row N tile).  The expert block supplies up to 16*C token
// slots (the MFMA N dimension); each wavefront owns R strips of 16 weight
// rows (the MFMA M dimension) and walks K one quantisation group at a time:
// per strip one 16-byte load per lane brings a 16x128 int4 tile, per K step
// of 32 the lane's dword is widened to 8 biased bf16 values in 5 ALU ops, and
// the group's partial sums are scaled by the bf16 group scale in fp32.
#include "common.h"
#include "../../include/dsv4moe.h"

namespace dsv4 {

struct ExpertGemmParams {
  const uint8_t* wq;     // tiled int4, expert-major
  const uint16_t* ws;    // tiled scales
  int64_t wq_stride;     // bytes per expert
  int64_t ws_stride;     // scale elements per expert
  int k_dim;             // K of the weight matrix
  int inter;             // stage 1: first up-projection row
  const uint16_t* act;   // stage 1: x [T][H]; stage 2: h [rows][I]
  const float* act_gsum; // per-row sums over each K group of `act`
  const int32_t* sorted;
  const int32_t* expert_ids;
  const int32_t* ntpp;
  int block_size;
  int max_blocks;
  int n_tiles;
  int64_t tokens;
  int topk;
  int shared_expert;     // expert index of the shared expert, -1 if none
  float clamp_limit;
  const float* route_w;  // stage 2: [T*k]
  uint16_t* h_out;       // stage 1: [rows][I]
  float* hsum_out;       // stage 1: [rows][I/128]
  float* contrib;        // stage 2: [rows][H]
  int out_cols;          // stage 2: H
};

template <int C, int R, int STAGE>
__global__ __launch_bounds__(256) void expert_gemm_kernel(ExpertGemmParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile = blockIdx.x % p.n_tiles;
  const int blk = blockIdx.x / p.n_tiles;
  const int64_t tk = p.tokens * p.topk;

  int expert;
  int64_t slot_base;
  bool shared_blk = blk >= p.max_blocks;
  if (!shared_blk) {
    const int total = p.ntpp[0];
    if (total <= 0 || (int64_t)blk * p.block_size >= total) return;
    expert = p.expert_ids[blk];
    slot_base = (int64_t)blk * p.block_size;
  } else {
    expert = p.shared_expert;
    slot_base = (int64_t)(blk - p.max_blocks) * p.block_size;
  }

  // Token slot of this lane for each column tile.
  int64_t rowid[C];
  int64_t in_row[C];
#pragma unroll
  for (int ct = 0; ct < C; ++ct) {
    const int col = ct * 16 + (lane & 15);
    rowid[ct] = -1;
    if (col < p.block_size) {
      if (!shared_blk) {
        const int32_t f = p.sorted[slot_base + col];
        if (f >= 0 && f < tk) rowid[ct] = f;
      } else {
        const int64_t t = slot_base + col;
        if (t < p.tokens) rowid[ct] = tk + t;
      }
    }
    if (STAGE == 1)
      in_row[ct] = rowid[ct] < 0 ? -1 : (rowid[ct] < tk ? rowid[ct] / p.topk : rowid[ct] - tk);
    else
      in_row[ct] = rowid[ct];
  }

  const int groups = p.k_dim / kGroup;
  const int n0 = tile * 128;
  int strip[R];
#pragma unroll
  for (int s = 0; s < R; ++s) {
    if (STAGE == 1)
      strip[s] = (s < R / 2) ? (n0 + 32 * wave) / 16 + s : (p.inter + n0 + 32 * wave) / 16 + (s - R / 2);
    else
      strip[s] = (n0 + 32 * wave) / 16 + s;
  }
  const uint8_t* wq = p.wq + (int64_t)expert * p.wq_stride + lane * 16;
  const uint16_t* ws = p.ws + (int64_t)expert * p.ws_stride + 4 * (lane >> 4);
  const int koff = 8 * (lane >> 4);

  f32x4 acc[R][C];
#pragma unroll
  for (int s = 0; s < R; ++s)
#pragma unroll
    for (int ct = 0; ct < C; ++ct) acc[s][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int g = 0; g < groups; ++g) {
    u32x4 wv[R];
    u32x2 sv[R];
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int64_t t_idx = (int64_t)strip[s] * groups + g;
      wv[s] = load16_nt(wq + (t_idx << 10));
      sv[s] = *reinterpret_cast<const u32x2*>(ws + t_idx * 16);
    }
    float corr[C];
#pragma unroll
    for (int ct = 0; ct < C; ++ct)
      corr[ct] = in_row[ct] >= 0 ? kDequantBias * p.act_gsum[in_row[ct] * groups + g] : 0.0f;

    f32x4 tmp[R][C];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      bf16x8 bfr[C];
#pragma unroll
      for (int ct = 0; ct < C; ++ct) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (in_row[ct] >= 0)
          v = load16(p.act + in_row[ct] * p.k_dim + g * kGroup + d * 32 + koff);
        bfr[ct] = __builtin_bit_cast(bf16x8, v);
      }
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const bf16x8 a = dequant_biased(wv[s][d]);
#pragma unroll
        for (int ct = 0; ct < C; ++ct)
          tmp[s][ct] = mfma_bf16(a, bfr[ct], d == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : tmp[s][ct]);
      }
    }
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const float sc0 = __uint_as_float(sv[s][0] << 16);
      const float sc1 = __uint_as_float(sv[s][0] & 0xFFFF0000u);
      const float sc2 = __uint_as_float(sv[s][1] << 16);
      const float sc3 = __uint_as_float(sv[s][1] & 0xFFFF0000u);
#pragma unroll
      for (int ct = 0; ct < C; ++ct) {
        acc[s][ct][0] += sc0 * (tmp[s][ct][0] - corr[ct]);
        acc[s][ct][1] += sc1 * (tmp[s][ct][1] - corr[ct]);
        acc[s][ct][2] += sc2 * (tmp[s][ct][2] - corr[ct]);
        acc[s][ct][3] += sc3 * (tmp[s][ct][3] - corr[ct]);
      }
    }
  }

  if constexpr (STAGE == 1) {
    // SwiGLU epilogue: strips [0, R/2) are gate rows, [R/2, R) the matching up rows.
    __shared__ float red[4][C * 16];
    const float lim = p.clamp_limit;
#pragma unroll
    for (int ct = 0; ct < C; ++ct) {
      float part = 0.0f;
#pragma unroll
      for (int s = 0; s < R / 2; ++s) {
        uint32_t bits[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float gt = acc[s][ct][i];
          float up = acc[s + R / 2][ct][i];
          if (lim > 0.0f) {
            gt = fminf(gt, lim);
            up = fminf(fmaxf(up, -lim), lim);
          }
          bits[i] = float_to_bf16_bits(silu_f(gt) * up);
          part += __uint_as_float(bits[i] << 16);
        }
        if (rowid[ct] >= 0) {
          const int n = n0 + 32 * wave + 16 * s + 4 * (lane >> 4);
          u32x2 packed = {bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
          *reinterpret_cast<u32x2*>(p.h_out + rowid[ct] * p.inter + n) = packed;
        }
      }
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      if (lane < 16) red[wave][ct * 16 + lane] = part;
    }
    __syncthreads();
    if (threadIdx.x < C * 16) {
      const int ct = threadIdx.x >> 4;
      const int col = threadIdx.x;  // == ct*16 + lane for lane < 16
      int64_t rid = -1;
      if (col < p.block_size) {
        if (!shared_blk) {
          const int32_t f = p.sorted[slot_base + col];
          if (f >= 0 && f < tk) rid = f;
        } else if (slot_base + col < p.tokens) {
          rid = tk + slot_base + col;
        }
      }
      if (rid >= 0) {
        const float total = ((red[0][col] + red[1][col]) + red[2][col]) + red[3][col];
        p.hsum_out[rid * (p.inter / kGroup) + n0 / kGroup] = total;
      }
      (void)ct;
    }
  } else {
#pragma unroll
    for (int ct = 0; ct < C; ++ct) {
      if (rowid[ct] < 0) continue;
      const float wr = rowid[ct] < tk ? p.route_w[rowid[ct]] : 1.0f;
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const int n = n0 + 32 * wave + 16 * s + 4 * (lane >> 4);
        f32x4 v = acc[s][ct];
        v[0] *= wr; v[1] *= wr; v[2] *= wr; v[3] *= wr;
        *reinterpret_cast<f32x4*>(p.contrib + rowid[ct] * p.out_cols + n) = v;
      }
    }
  }
}

// Per-row fp32 sums of bf16 activations over each 128-wide K group, summed in
// ascending k order.
__global__ __launch_bounds__(256) void row_group_sum_kernel(const uint16_t* __restrict__ x,
                                                            int64_t rows, int k_dim,
                                                            float* __restrict__ out) {
  const int groups = k_dim / kGroup;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * groups) return;
  const int64_t r = idx / groups;
  const int g = (int)(idx % groups);
  const uint16_t* src = x + r * k_dim + g * kGroup;
  float s = 0.0f;
#pragma unroll 4
  for (int c = 0; c < kGroup; c += 8) {
    const u32x4 v = load16(src + c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      s += __uint_as_float(v[q] << 16);
      s += __uint_as_float(v[q] & 0xFFFF0000u);
    }
  }
  out[idx] = s;
}

// out[t][n] = bf16( sum_{j<k} contrib[t*k+j][n] + contrib[T*k+t][n] ).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ contrib,
                                                      int64_t tokens, int topk, int hidden,
                                                      int has_shared, uint16_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int vec = hidden / 4;
  if (idx >= tokens * vec) return;
  const int64_t t = idx / vec;
  const int n = (int)(idx % vec) * 4;
  const float* base = contrib + (t * topk) * hidden + n;
  f32x4 s = *reinterpret_cast<const f32x4*>(base);
  for (int j = 1; j < topk; ++j) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(base + (int64_t)j * hidden);
    s[0] += v[0]; s[1] += v[1]; s[2] += v[2]; s[3] += v[3];
  }
  if (has_shared) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(contrib + (tokens * topk + t) * hidden + n);
    s[0] += v[0]; s[1] += v[1]; s[2] += v[2]; s[3] += v[3];
  }
  u32x2 o = {pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
  *reinterpret_cast<u32x2*>(out + t * hidden + n) = o;
}

}  // namespace dsv4

using namespace dsv4;

struct ExpertWorkspace {
  float* xsum;
  uint16_t* h;
  float* hsum;
  float* contrib;
  size_t bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static ExpertWorkspace carve_workspace(void* base, int64_t tokens, int topk, int hidden, int inter,
                                       int has_shared) {
  const int64_t rows = tokens * topk + (has_shared ? tokens : 0);
  size_t off = 0;
  ExpertWorkspace w;
  char* b = static_cast<char*>(base);
  w.xsum = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)tokens * (hidden / kGroup));
  w.h = reinterpret_cast<uint16_t*>(b + off);
  off += align256(sizeof(uint16_t) * (size_t)rows * inter);
  w.hsum = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)rows * (inter / kGroup));
  w.contrib = reinterpret_cast<float*>(b + off);
  off += align256(sizeof(float) * (size_t)rows * hidden);
  w.bytes = off;
  return w;
}

size_t dsv4_experts_workspace_bytes(int64_t tokens, int topk, int hidden, int inter,
                                    int has_shared) {
  return carve_workspace(nullptr, tokens, topk, hidden, inter, has_shared).bytes;
}

template <int STAGE>
static void launch_stage(int C, const ExpertGemmParams& p, unsigned grid, hipStream_t stream) {
  constexpr int R = STAGE == 1 ? 4 : 2;
  switch (C) {
    case 1: hipLaunchKernelGGL((expert_gemm_kernel<1, R, STAGE>), dim3(grid), dim3(256), 0, stream, p); break;
    case 2: hipLaunchKernelGGL((expert_gemm_kernel<2, R, STAGE>), dim3(grid), dim3(256), 0, stream, p); break;
    case 3: hipLaunchKernelGGL((expert_gemm_kernel<3, R, STAGE>), dim3(grid), dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL((expert_gemm_kernel<4, R, STAGE>), dim3(grid), dim3(256), 0, stream, p); break;
  }
}

int dsv4_launch_experts_w4a16(const uint16_t* x, int64_t tokens, int hidden, int inter,
                              int experts, int topk, const uint8_t* w13q, const uint16_t* w13s,
                              const uint8_t* w2q, const uint16_t* w2s, int has_shared,
                              const float* weights, const int32_t* sorted, int64_t capacity,
                              const int32_t* expert_ids, const int32_t* ntpp, int block_size,
                              float clamp_limit, uint16_t* out, void* workspace,
                              hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  ExpertWorkspace ws = carve_workspace(workspace, tokens, topk, hidden, inter, has_shared);
  const int max_blocks = (int)((capacity + block_size - 1) / block_size);
  const int shared_blocks = has_shared ? (int)((tokens + block_size - 1) / block_size) : 0;
  const int C = (block_size + 15) / 16;

  {
    const int64_t n = tokens * (hidden / kGroup);
    hipLaunchKernelGGL(row_group_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       stream, x, tokens, hidden, ws.xsum);
    DSV4_CHECK_LAUNCH("row_group_sum_kernel");
  }
  dsv4host::prof_stamp(dsv4host::kStampRowSum, stream);
  ExpertGemmParams p{};
  p.sorted = sorted;
  p.expert_ids = expert_ids;
  p.ntpp = ntpp;
  p.block_size = block_size;
  p.max_blocks = max_blocks;
  p.tokens = tokens;
  p.topk = topk;
  p.shared_expert = has_shared ? experts : -1;
  p.clamp_limit = clamp_limit;
  p.inter = inter;

  // stage 1: W13 [2I, H]
  p.wq = w13q;
  p.ws = w13s;
  p.wq_stride = (int64_t)2 * inter * hidden / 2;
  p.ws_stride = (int64_t)2 * inter * (hidden / kGroup);
  p.k_dim = hidden;
  p.act = x;
  p.act_gsum = ws.xsum;
  p.h_out = ws.h;
  p.hsum_out = ws.hsum;
  p.n_tiles = inter / 128;
  launch_stage<1>(C, p, (unsigned)(p.n_tiles * (max_blocks + shared_blocks)), stream);
  DSV4_CHECK_LAUNCH("expert_gemm_kernel<stage1>");
  dsv4host::prof_stamp(dsv4host::kStampStage1, stream);

  // stage 2: W2 [H, I]
  p.wq = w2q;
  p.ws = w2s;
  p.wq_stride = (int64_t)hidden * inter / 2;
  p.ws_stride = (int64_t)hidden * (inter / kGroup);
  p.k_dim = inter;
  p.act = ws.h;
  p.act_gsum = ws.hsum;
  p.route_w = weights;
  p.contrib = ws.contrib;
  p.out_cols = hidden;
  p.n_tiles = hidden / 128;
  launch_stage<2>(C, p, (unsigned)(p.n_tiles * (max_blocks + shared_blocks)), stream);
  DSV4_CHECK_LAUNCH("expert_gemm_kernel<stage2>");
  dsv4host::prof_stamp(dsv4host::kStampStage2, stream);

  {
    const int64_t n = tokens * (hidden / 4);
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       ws.contrib, tokens, topk, hidden, has_shared, out);
    DSV4_CHECK_LAUNCH("combine_kernel");
  }
  dsv4host::prof_stamp(dsv4host::kStampCombine, stream);
  return DSV4MOE_OK;
}
