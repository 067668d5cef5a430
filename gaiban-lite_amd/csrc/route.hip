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
#include "common.h"
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

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
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

template <int SCORE, int EPL>
__global__ __launch_bounds__(256) void route_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int64_t tokens,
    int experts, int topk, float route_scale, int32_t* __restrict__ ids,
    float* __restrict__ weights, float* __restrict__ margin, int32_t* __restrict__ sel_ids,
    float* __restrict__ sel_scores) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (t >= tokens) return;
  const float* row = logits + t * experts;

  float lg[EPL];
  float sel[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    lg[j] = e < experts ? row[e] : 0.0f;
  }

  float row_max = 0.0f, row_sum = 1.0f;
  if constexpr (SCORE == DSV4MOE_SCORE_SOFTMAX) {
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + 64 * j < experts) m = fmaxf(m, lg[j]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    row_max = m;
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + 64 * j < experts) part = part + exp_seq(lg[j] - row_max);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off, 64);
    row_sum = part;
  }

  uint32_t live = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    if (e < experts) {
      float s = score_of<SCORE>(lg[j], row_max, row_sum);
      if (bias != nullptr) s = s + bias[e];
      sel[j] = s;
      live |= 1u << j;
    } else {
      sel[j] = 0.0f;
    }
  }

  const int depth = topk + 1 <= experts ? topk + 1 : experts;
  int chosen_id[kMaxTopk + 1];
  float chosen_sel[kMaxTopk + 1];
#pragma unroll
  for (int r = 0; r < kMaxTopk + 1; ++r) {
    chosen_id[r] = 0;
    chosen_sel[r] = 0.0f;
    if (r >= depth) continue;
    uint64_t best = 0;
    int best_j = -1;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      if (live & (1u << j)) {
        const int e = lane + 64 * j;
        const uint64_t c = ((uint64_t)order_key(sel[j]) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
        if (best_j < 0 || c > best) {
          best = c;
          best_j = j;
        }
      }
    }
    const uint64_t win = wave_max_u64(best);
    const int e_win = (int)(0xFFFFFFFFu - (uint32_t)(win & 0xFFFFFFFFu));
    if ((e_win & 63) == lane) live &= ~(1u << (e_win >> 6));
    chosen_id[r] = e_win;
    chosen_sel[r] = key_value((uint32_t)(win >> 32));
  }

  // Unbiased score of selected expert r, recomputed by lane r from its logit.
  float my_score = 0.0f;
  int my_id = 0;
#pragma unroll
  for (int r = 0; r < kMaxTopk; ++r)
    if (r < topk && lane == r) my_id = chosen_id[r];
  if (lane < topk) my_score = score_of<SCORE>(row[my_id], row_max, row_sum);

  float w = my_score;
  if constexpr (SCORE != DSV4MOE_SCORE_SOFTMAX) {
    float total = __shfl(my_score, 0, 64);
    for (int r = 1; r < topk; ++r) total = total + __shfl(my_score, r, 64);
    w = w / total;
  }
  w = w * route_scale;
  if (lane < topk) {
    ids[t * topk + lane] = my_id;
    weights[t * topk + lane] = w;
  }
  if (lane == 0 && margin != nullptr) {
    float kth = 0.0f, next = 0.0f;
#pragma unroll
    for (int r = 0; r < kMaxTopk + 1; ++r) {
      if (r == topk - 1) kth = chosen_sel[r];
      if (r == topk) next = chosen_sel[r];
    }
    margin[t] = depth > topk ? kth - next : 0.0f;
  }
  if (sel_ids != nullptr || sel_scores != nullptr) {
#pragma unroll
    for (int r = 0; r < kMaxTopk + 1; ++r) {
      if (r < depth && lane == r) {
        if (sel_ids) sel_ids[t * depth + r] = chosen_id[r];
        if (sel_scores) sel_scores[t * depth + r] = chosen_sel[r];
      }
    }
  }
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
