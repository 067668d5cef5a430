// Router: scores (sigmoid / softmax / sqrt-softplus), top-(k+1) selection with
// a deterministic tie order, renormalised route weights and the top-k margin.
// Restates Gate.forward (reference/inference/model.py:564-584) and
// gate_forward_with_boundary (runtime/dsv4_direct/moe_forward.py:80-87).
//
// One 64-lane wavefront per token.  Expert e lives in lane e % 64, slot e / 64.
// The elementary functions below use a fixed sequence of IEEE fp32 operations
// (no contraction into FMA), so the scores are reproducible bit for bit by a
// CPU implementation of the same sequence:
//   exp   : Cody-Waite reduction x = n ln2 + r, degree-7 Taylor polynomial,
//           scale by 2^n; 0 for n <= -126, inf for n > 127.
//   log   : m in [sqrt(1/2), sqrt(2)), log m = 2 atanh((m-1)/(m+1)) (odd
//           series to s^9), plus e*ln2 split in two parts.
//   log1p : Goldberg's compensation log(w) * (u / (w - 1)), w = 1 + u.
#include <algorithm>

#include "common.h"
#include "align_impl.h"
#include "../../include/dsv4moe.h"

#pragma clang fp contract(off)

namespace dsv4 {

constexpr int kMaxTopk = 16;

__device__ __forceinline__ float exp_seq(float x) {
  x = fminf(fmaxf(x, -110.0f), 100.0f);
  const float n = rintf(x * 1.4426950408889634f);
  const float r = (x - n * 0.693359375f) - n * -2.12194440e-4f;
  float p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  const int ni = (int)n;
  const int nc = ni < -126 ? -126 : (ni > 127 ? 127 : ni);
  float out = p * __uint_as_float((uint32_t)(nc + 127) << 23);
  if (ni > 127) out = __builtin_huge_valf();
  if (ni <= -126) out = 0.0f;
  return out;
}

__device__ __forceinline__ float log_seq(float x) {  // x >= 1, finite
  const uint32_t bits = __float_as_uint(x);
  int e = (int)((bits >> 23) & 0xFFu) - 127;
  float m = __uint_as_float((bits & 0x7FFFFFu) | 0x3F800000u);
  if (m > 1.41421356237f) {
    m = m * 0.5f;
    e = e + 1;
  }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float t = 1.0f / 9.0f;
  t = t * s2 + 1.0f / 7.0f;
  t = t * s2 + 1.0f / 5.0f;
  t = t * s2 + 1.0f / 3.0f;
  t = t * s2;
  const float log_m = (s + s * t) * 2.0f;
  const float ef = (float)e;
  return ef * 0.693359375f + (ef * -2.12194440e-4f + log_m);
}

__device__ __forceinline__ float log1p_seq(float u) {  // u >= 0
  const float w = u + 1.0f;
  if (w == 1.0f) return u;
  return log_seq(w) * (u / (w - 1.0f));
}

__device__ __forceinline__ float sigmoid_seq(float x) { return 1.0f / (1.0f + exp_seq(-x)); }

__device__ __forceinline__ float sqrtsoftplus_seq(float x) {
  const float sp = x > 20.0f ? x : log1p_seq(exp_seq(fminf(x, 20.0f)));
  return __builtin_sqrtf(sp);
}

// Order-preserving image of a float as uint32 (-0.0 below +0.0).
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}

// Maximum of a 64-bit key over the wavefront, returned to every lane.  DPP
// steps (row_shr 1/2/4/8, then row_bcast 15/31) build an inclusive running
// maximum whose lane 63 covers all lanes; a lane whose DPP source is outside
// its row keeps its own value.  Plain VALU moves, no LDS round trips (the
// keys are distinct, so the reduction order cannot change the result).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_step(uint64_t v) {
  const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp((int)lo, (int)lo, CTRL, ROW_MASK, 0xF, false);
  const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp((int)hi, (int)hi, CTRL, ROW_MASK, 0xF, false);
  const uint64_t o = ((uint64_t)ohi << 32) | olo;
  return o > v ? o : v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = dpp_max_step<0x111, 0xF>(v);  // row_shr:1
  v = dpp_max_step<0x112, 0xF>(v);  // row_shr:2
  v = dpp_max_step<0x114, 0xF>(v);  // row_shr:4
  v = dpp_max_step<0x118, 0xF>(v);  // row_shr:8
  v = dpp_max_step<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_max_step<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

template <int SCORE>
__device__ __forceinline__ float score_of(float logit, float row_max, float row_sum) {
  if constexpr (SCORE == DSV4MOE_SCORE_SIGMOID) {
    return sigmoid_seq(logit);
  } else if constexpr (SCORE == DSV4MOE_SCORE_SQRTSOFTPLUS) {
    return sqrtsoftplus_seq(logit);
  } else {
    return exp_seq(logit - row_max) / row_sum;
  }
}

// Route NT tokens t0, t0 + tstride, ... (those below `tokens`) with one
// wavefront (every lane calls it).  The tokens are independent: their loads
// are issued together and their selection rounds interleave, so one memory
// latency and one dependency chain cover all of them.  Per token the
// operations and their order are those of a single-token route.
template <int SCORE, int EPL, int NT>
__device__ __forceinline__ void route_tokens(const float* __restrict__ logits, const float* __restrict__ bias,
                                             int64_t t0, int64_t tstride, int64_t tokens, int experts, int topk,
                                             float route_scale, int32_t* __restrict__ ids,
                                             float* __restrict__ weights, float* __restrict__ margin,
                                             int32_t* __restrict__ sel_ids, float* __restrict__ sel_scores) {
  const int lane = threadIdx.x & 63;
  bool valid[NT];
  const float* row[NT];
  float lg[NT][EPL];
  float sel[NT][EPL];
  uint32_t live[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    const int64_t t = t0 + u * tstride;
    valid[u] = t < tokens;
    row[u] = logits + (valid[u] ? t : 0) * experts;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      lg[u][j] = (valid[u] && e < experts) ? row[u][e] : 0.0f;
    }
  }
  float bv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    bv[j] = (bias != nullptr && e < experts) ? bias[e] : 0.0f;
  }

  float row_max[NT], row_sum[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    row_max[u] = 0.0f;
    row_sum[u] = 1.0f;
    if constexpr (SCORE == DSV4MOE_SCORE_SOFTMAX) {
      float m = -__builtin_huge_valf();
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (lane + 64 * j < experts) m = fmaxf(m, lg[u][j]);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
      row_max[u] = m;
      float part = 0.0f;
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (lane + 64 * j < experts) part = part + exp_seq(lg[u][j] - row_max[u]);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off, 64);
      row_sum[u] = part;
    }
    live[u] = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      if (e < experts) {
        float sc = score_of<SCORE>(lg[u][j], row_max[u], row_sum[u]);
        if (bias != nullptr) sc = sc + bv[j];
        sel[u][j] = sc;
        live[u] |= 1u << j;
      } else {
        sel[u][j] = 0.0f;
      }
    }
  }

  // Selection: round r takes the (score, -id)-largest live expert; lane r
  // keeps the id of round r, and rounds k-1 and k give the margin.
  const int depth = topk + 1 <= experts ? topk + 1 : experts;
  int my_id[NT];
  float kth[NT], nxt[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    my_id[u] = 0;
    kth[u] = 0.0f;
    nxt[u] = 0.0f;
  }
  for (int r = 0; r < depth; ++r) {
    uint64_t win[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
      uint64_t best = 0;
      int best_j = -1;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        if (live[u] & (1u << j)) {
          const int e = lane + 64 * j;
          const uint64_t c = ((uint64_t)order_key(sel[u][j]) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
          if (best_j < 0 || c > best) {
            best = c;
            best_j = j;
          }
        }
      }
      win[u] = wave_max_u64(best);
    }
#pragma unroll
    for (int u = 0; u < NT; ++u) {
      const int e_win = (int)(0xFFFFFFFFu - (uint32_t)(win[u] & 0xFFFFFFFFu));
      const float s_win = key_value((uint32_t)(win[u] >> 32));
      if ((e_win & 63) == lane) live[u] &= ~(1u << (e_win >> 6));
      if (lane == r) my_id[u] = e_win;
      if (r == topk - 1) kth[u] = s_win;
      if (r == topk) nxt[u] = s_win;
      if (valid[u] && lane == 0) {
        const int64_t t = t0 + u * tstride;
        if (sel_ids) sel_ids[t * depth + r] = e_win;
        if (sel_scores) sel_scores[t * depth + r] = s_win;
      }
    }
  }

  // Unbiased score of selected expert r, recomputed by lane r from its logit.
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    float my_score = 0.0f;
    if (valid[u] && lane < topk) my_score = score_of<SCORE>(row[u][my_id[u]], row_max[u], row_sum[u]);
    float w = my_score;
    if constexpr (SCORE != DSV4MOE_SCORE_SOFTMAX) {
      // sequential sum in selection order (lane r holds selected expert r)
      const int sbits = __float_as_int(my_score);
      float total = __int_as_float(__builtin_amdgcn_readlane(sbits, 0));
      for (int r = 1; r < topk; ++r) total = total + __int_as_float(__builtin_amdgcn_readlane(sbits, r));
      w = w / total;
    }
    w = w * route_scale;
    if (!valid[u]) continue;
    const int64_t t = t0 + u * tstride;
    if (lane < topk) {
      ids[t * topk + lane] = my_id[u];
      weights[t * topk + lane] = w;
    }
    if (lane == 0 && margin != nullptr) margin[t] = depth > topk ? kth[u] - nxt[u] : 0.0f;
  }
}

template <int SCORE, int EPL>
__global__ __launch_bounds__(256) void route_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int64_t tokens,
    int experts, int topk, float route_scale, int32_t* __restrict__ ids,
    float* __restrict__ weights, float* __restrict__ margin, int32_t* __restrict__ sel_ids,
    float* __restrict__ sel_scores) {
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (t >= tokens) return;
  route_tokens<SCORE, EPL, 1>(logits, bias, t, 0, tokens, experts, topk, route_scale, ids, weights, margin,
                              sel_ids, sel_scores);
}

// Layer prologue in one launch: workgroup 0 routes every token when `route`
// is set (wavefront w takes tokens w, w + 16, ...; used for T <= 16, since
// routing is VALU-bound and one workgroup runs on one CU) and then runs the
// alignment over the ids; workgroups 1.. do the activation work of `prep`
// (act_prep_part: the row sums in the decode or the prefill form, summed in
// ascending k as row_chunk_sum_kernel, or the W4A8 quantisation).
// Replaces the route, align and row-sum launches (or the last two).
struct PrologueArgs {
  const float* logits;
  const float* bias;
  int64_t tokens;
  int experts;
  int topk;
  float route_scale;
  int32_t* ids;
  float* weights;
  float* margin;
  int expert_bits;
  int block_size;
  int32_t* sorted_ids;
  int64_t capacity;
  int32_t* expert_ids;
  int64_t num_blocks;
  int32_t* ntpp;
  ActPrep prep;        // activation work of workgroups 1..
  int route;           // route in workgroup 0 (else ids are given)
};

// The alignment of one token's k distinct, valid expert ids in closed form
// (what align_block computes when every count is 0 or 1): the experts in
// ascending order each own one block, whose first slot holds the flat index
// j of the id and whose other slots, like every position past k blocks,
// hold the sentinel k; expert_ids[b] is the b-th smallest id, then -1; the
// padded total is k * block_size.  Returns false (nothing written) when an id
// is outside [0, experts) or repeats, which align_block handles.  Every
// thread of the workgroup calls it after the ids are visible to it.
__device__ __forceinline__ bool align_one_token(const int32_t* __restrict__ ids, int topk, int experts,
                                                int block_size, int32_t* __restrict__ sorted_ids, int64_t capacity,
                                                int32_t* __restrict__ expert_ids, int64_t num_blocks,
                                                int32_t* __restrict__ ntpp) {
  __shared__ int32_t order_flat[64];  // flat index j of the id of rank b
  __shared__ int32_t order_expert[64];
  __shared__ int ok;
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < 64) {
    const int id = lane < topk ? ids[lane] : 0;
    const bool in_range = lane >= topk || (id >= 0 && id < experts);
    int rank = 0;
    bool repeat = false;
    for (int i = 0; i < topk; ++i) {
      const int other = __shfl(id, i, 64);
      rank += other < id;
      repeat |= i != lane && other == id;
    }
    const bool lane_ok = lane >= topk || (in_range && !repeat);
    const uint64_t bad = __ballot(!lane_ok);
    if (lane < topk) {
      order_flat[rank] = lane;
      order_expert[rank] = id;
    }
    if (lane == 0) ok = bad == 0;
  }
  __syncthreads();
  if (!ok) return false;
  for (int64_t pos = threadIdx.x; pos < capacity; pos += blockDim.x) {
    const int64_t b = pos / block_size;
    sorted_ids[pos] = (pos % block_size == 0 && b < topk) ? order_flat[b] : topk;
  }
  for (int64_t b = threadIdx.x; b < num_blocks; b += blockDim.x) expert_ids[b] = b < topk ? order_expert[b] : -1;
  if (threadIdx.x == 0) ntpp[0] = topk * block_size;
  return true;
}

template <int SCORE, int EPL>
__global__ __launch_bounds__(kAlignThreads) void prologue_kernel(PrologueArgs a) {
  if (blockIdx.x == 0) {
    if (a.route) {
      for (int64_t t = threadIdx.x >> 6; t < a.tokens; t += kAlignWaves)
        route_tokens<SCORE, EPL, 1>(a.logits, a.bias, t, 0, a.tokens, a.experts, a.topk, a.route_scale, a.ids,
                                    a.weights, a.margin, nullptr, nullptr);
      __syncthreads();  // every id is written (workgroup-scope visibility)
      // one routed token (single-token decode): its k ids are distinct
      // experts, and their alignment needs none of align_block's phases
      if (a.tokens == 1 && a.topk <= 64 &&
          align_one_token(a.ids, a.topk, a.experts, a.block_size, a.sorted_ids, a.capacity, a.expert_ids,
                          a.num_blocks, a.ntpp))
        return;
    }
    align_block(a.ids, a.tokens * a.topk, a.experts, a.expert_bits, a.block_size, a.sorted_ids, a.capacity,
                a.expert_ids, a.num_blocks, a.ntpp);
    return;
  }
  act_prep_part(a.prep, a.tokens, blockIdx.x - 1, gridDim.x - 1);
}

__global__ __launch_bounds__(256) void route_hash_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ tid2eid, int64_t vocab,
    const int64_t* __restrict__ input_ids, int64_t tokens, int experts, int topk,
    float route_scale, int32_t* __restrict__ ids, float* __restrict__ weights,
    float* __restrict__ selected_scores) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (t >= tokens) return;
  int64_t tok = input_ids[t];
  const bool ok_tok = tok >= 0 && tok < vocab;
  int id = 0;
  float s = 0.0f;
  if (lane < topk && ok_tok) {
    const int64_t v = tid2eid[tok * topk + lane];
    id = (v >= 0 && v < experts) ? (int)v : -1;
    if (id >= 0) s = sqrtsoftplus_seq(logits[t * experts + id]);
  } else if (lane < topk) {
    id = -1;
  }
  float total = __shfl(s, 0, 64);
  for (int r = 1; r < topk; ++r) total = total + __shfl(s, r, 64);
  if (lane < topk) {
    ids[t * topk + lane] = id;
    weights[t * topk + lane] = (s / total) * route_scale;
    if (selected_scores != nullptr) selected_scores[t * topk + lane] = s;
  }
}

}  // namespace dsv4

using namespace dsv4;

template <int SCORE>
static int launch_route(const float* logits, const float* bias, int64_t tokens, int experts,
                        int topk, float route_scale, int32_t* ids, float* weights,
                        float* margin, int32_t* sel_ids, float* sel_scores, hipStream_t stream) {
  const int epl = (experts + 63) / 64;
  const dim3 block(256);
  const dim3 grid((unsigned)((tokens + 3) / 4));
#define DSV4_ROUTE_CASE(N)                                                                   \
  case N:                                                                                    \
    hipLaunchKernelGGL((route_topk_kernel<SCORE, N>), grid, block, 0, stream, logits, bias, \
                       tokens, experts, topk, route_scale, ids, weights, margin, sel_ids,    \
                       sel_scores);                                                          \
    break;
  switch (epl) {
    DSV4_ROUTE_CASE(1)
    DSV4_ROUTE_CASE(2)
    DSV4_ROUTE_CASE(4)
    DSV4_ROUTE_CASE(8)
    DSV4_ROUTE_CASE(16)
    case 3:
      hipLaunchKernelGGL((route_topk_kernel<SCORE, 4>), grid, block, 0, stream, logits, bias,
                         tokens, experts, topk, route_scale, ids, weights, margin, sel_ids,
                         sel_scores);
      break;
    default:
      if (epl <= 8) {
        hipLaunchKernelGGL((route_topk_kernel<SCORE, 8>), grid, block, 0, stream, logits, bias,
                           tokens, experts, topk, route_scale, ids, weights, margin, sel_ids,
                           sel_scores);
      } else {
        hipLaunchKernelGGL((route_topk_kernel<SCORE, 16>), grid, block, 0, stream, logits,
                           bias, tokens, experts, topk, route_scale, ids, weights, margin,
                           sel_ids, sel_scores);
      }
  }
#undef DSV4_ROUTE_CASE
  return DSV4MOE_OK;
}

int dsv4_launch_route_topk(const float* logits, const float* bias, int64_t tokens, int32_t experts,
                           int32_t topk, int32_t score_func, float route_scale, int32_t* ids,
                           float* weights, float* margin, int32_t* sel_ids, float* sel_scores,
                           hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  switch (score_func) {
    case DSV4MOE_SCORE_SIGMOID:
      launch_route<DSV4MOE_SCORE_SIGMOID>(logits, bias, tokens, experts, topk, route_scale, ids,
                                          weights, margin, sel_ids, sel_scores, stream);
      break;
    case DSV4MOE_SCORE_SOFTMAX:
      launch_route<DSV4MOE_SCORE_SOFTMAX>(logits, bias, tokens, experts, topk, route_scale, ids,
                                          weights, margin, sel_ids, sel_scores, stream);
      break;
    default:
      launch_route<DSV4MOE_SCORE_SQRTSOFTPLUS>(logits, bias, tokens, experts, topk, route_scale,
                                               ids, weights, margin, sel_ids, sel_scores, stream);
  }
  DSV4_CHECK_LAUNCH("route_topk_kernel");
  return DSV4MOE_OK;
}

int dsv4_launch_route_hash(const float* logits, const int64_t* tid2eid, int64_t vocab,
                           const int64_t* input_ids, int64_t tokens, int32_t experts,
                           int32_t topk, float route_scale, int32_t* ids, float* weights,
                           float* selected_scores, hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  hipLaunchKernelGGL(route_hash_kernel, dim3((unsigned)((tokens + 3) / 4)), dim3(256), 0, stream,
                     logits, tid2eid, vocab, input_ids, tokens, experts, topk, route_scale, ids,
                     weights, selected_scores);
  DSV4_CHECK_LAUNCH("route_hash_kernel");
  return DSV4MOE_OK;
}

// [Route +] align [+ the activation work of `prep`] as one launch.
int dsv4_launch_prologue(int32_t route, const float* logits, const float* bias, int64_t tokens, int32_t experts,
                         int32_t topk, int32_t score_func, float route_scale, int32_t* ids, float* weights,
                         float* margin, int32_t block_size, int32_t* sorted_ids, int64_t capacity,
                         int32_t* expert_ids, int64_t num_blocks, int32_t* ntpp, const ActPrep& prep,
                         hipStream_t stream) {
  if (tokens == 0) return DSV4MOE_OK;
  PrologueArgs a{logits, bias, tokens, experts, topk, route_scale, ids, weights, margin, 0, block_size,
                 sorted_ids, capacity, expert_ids, num_blocks, ntpp, prep, route};
  while ((1 << a.expert_bits) < experts) ++a.expert_bits;
  const unsigned grid = 1u + (unsigned)act_prep_workgroups(prep, tokens, 64);
  const int epl = (experts + 63) / 64;
#define DSV4_PROLOGUE(S, N) hipLaunchKernelGGL((prologue_kernel<S, N>), dim3(grid), dim3(kAlignThreads), 0, stream, a)
#define DSV4_PROLOGUE_EPL(S)          \
  if (epl <= 1) DSV4_PROLOGUE(S, 1);  \
  else if (epl <= 2) DSV4_PROLOGUE(S, 2); \
  else if (epl <= 4) DSV4_PROLOGUE(S, 4); \
  else if (epl <= 8) DSV4_PROLOGUE(S, 8); \
  else DSV4_PROLOGUE(S, 16);
  switch (score_func) {
    case DSV4MOE_SCORE_SIGMOID: DSV4_PROLOGUE_EPL(DSV4MOE_SCORE_SIGMOID) break;
    case DSV4MOE_SCORE_SOFTMAX: DSV4_PROLOGUE_EPL(DSV4MOE_SCORE_SOFTMAX) break;
    default: DSV4_PROLOGUE_EPL(DSV4MOE_SCORE_SQRTSOFTPLUS) break;
  }
#undef DSV4_PROLOGUE_EPL
#undef DSV4_PROLOGUE
  DSV4_CHECK_LAUNCH("prologue_kernel");
  return DSV4MOE_OK;
}
