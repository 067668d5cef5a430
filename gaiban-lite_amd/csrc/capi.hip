// extern "C" entry points of include/dsv4moe.h: argument validation (before
// any launch), dispatch to the kernels, and the thread-local error message.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "act_quant.h"
#include "common.h"
#include "../../include/dsv4moe.h"

namespace dsv4host {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(err));
    return DSV4MOE_EHIP;
  }
  return DSV4MOE_OK;
}

// Profiling state: one event per (call, stamp); a call is one layer/experts
// invocation, counted when its last stamp is recorded.  Process-global and
// not thread-safe: profile from one host thread.
struct ProfileState {
  std::vector<hipEvent_t> events;
  int max_calls = 0;
  int call = 0;
  uint32_t mask = 0;  // stamps recorded (bit i = stamp i)
  bool active = false;
};
static ProfileState g_prof;

void prof_stamp(int stamp, hipStream_t stream) {
  if (!g_prof.active || g_prof.call >= g_prof.max_calls) return;
  if (g_prof.mask & (1u << stamp))
    (void)hipEventRecord(g_prof.events[(size_t)g_prof.call * kNumStamps + stamp], stream);
  if (stamp == kNumStamps - 1) ++g_prof.call;
}

static void prof_release() {
  for (hipEvent_t e : g_prof.events)
    if (e != nullptr) (void)hipEventDestroy(e);
  g_prof.events.clear();
  g_prof.active = false;
  g_prof.call = 0;
  g_prof.max_calls = 0;
  g_prof.mask = 0;
}

}  // namespace dsv4host

// kernel launchers (one per translation unit)
int dsv4_launch_route_topk(const float*, const float*, int64_t, int32_t, int32_t, int32_t, float,
                           int32_t*, float*, float*, int32_t*, float*, hipStream_t);
int dsv4_launch_route_hash(const float*, const int64_t*, int64_t, const int64_t*, int64_t, int32_t,
                           int32_t, float, int32_t*, float*, float*, hipStream_t);
int dsv4_launch_gate_logits(const uint16_t*, const uint16_t*, int64_t, int, int, float*,
                            hipStream_t);
int dsv4_launch_align(const int32_t*, int64_t, int32_t, int32_t, int32_t*, int64_t, int32_t*,
                      int64_t, int32_t*, hipStream_t);
int dsv4_launch_pack_ratios(const uint16_t*, int64_t, int64_t, int64_t, float*, hipStream_t);
int dsv4_launch_pack(const uint8_t*, const uint16_t*, int64_t, int64_t, int64_t, int, uint8_t*,
                     uint16_t*, hipStream_t);
size_t dsv4_experts_workspace_bytes(int64_t, int, int, int, int);
int dsv4_launch_experts_w4a16(const uint16_t*, int64_t, int, int, int, int, const uint8_t*,
                              const uint16_t*, const uint8_t*, const uint16_t*, const float*, const float*, int,
                              const float*, const int32_t*, int64_t, const int32_t*, const int32_t*, int, float,
                              uint16_t*, void*, hipStream_t, bool rowsums_ready = false);
float* dsv4_experts_xsum(void*, int64_t, int, int, int, int);
int dsv4_launch_prologue(int32_t, const float*, const float*, int64_t, int32_t, int32_t, int32_t, float, int32_t*,
                         float*, float*, int32_t, int32_t*, int64_t, int32_t*, int64_t, int32_t*,
                         const dsv4::ActPrep&, hipStream_t);
// Largest token count routed inside the one-workgroup prologue (one token per
// wavefront); above it the wide route kernel runs first.
constexpr int64_t kPrologueRouteMaxTokens = 16;
int dsv4_launch_align_multi(const int32_t*, int64_t, int32_t, int32_t, int32_t*, int64_t, int32_t*, int64_t,
                            int32_t*, int32_t*, const dsv4::ActPrep&, int64_t, hipStream_t);
size_t dsv4_align_scratch_bytes(int64_t, int32_t);
int32_t* dsv4_experts_align_scratch(void*, int64_t, int, int, int, int, size_t*);
// Fewest flat route ids aligned by the two-launch split over chunks; below it
// one workgroup aligns them all in one launch.
constexpr int64_t kAlignMultiMinAssignments = 8192;

int dsv4_launch_pack_mxfp4(const uint8_t*, const uint8_t*, int64_t, int64_t, int64_t, int, uint8_t*, uint8_t*,
                           hipStream_t);
int dsv4_launch_experts_mxfp4(const uint16_t*, int64_t, int, int, int, int, const uint8_t*, const uint8_t*,
                              const uint8_t*, const uint8_t*, int, const float*, const int32_t*, int64_t,
                              const int32_t*, const int32_t*, int, float, uint16_t*, void*, hipStream_t);
int dsv4_launch_pack_mxfp4_a8(const uint8_t*, const uint8_t*, int64_t, int64_t, int64_t, int, uint8_t*,
                              uint8_t*, hipStream_t);
int dsv4_launch_experts_w4a8_mxfp4(const uint16_t*, int64_t, int, int, int, int, const uint8_t*, const uint8_t*,
                                   const uint8_t*, const uint8_t*, int, const float*, const int32_t*, int64_t,
                                   const int32_t*, const int32_t*, int, float, uint16_t*, void*, hipStream_t,
                                   bool x_ready = false);
size_t dsv4_experts_w4a8_workspace_bytes(int64_t, int, int, int, int);
void dsv4_experts_w4a8_pieces(void*, int64_t, int, int, int, int, uint8_t**, float**, float**, int32_t**, size_t*);
int dsv4_launch_act_quant_fp8(const uint16_t*, int64_t, int, uint8_t*, float*, float*, hipStream_t);
int dsv4_launch_experts_w4a8(const uint16_t*, int64_t, int, int, int, int, const uint8_t*,
                             const uint16_t*, const uint8_t*, const uint16_t*, int, const float*,
                             const int32_t*, int64_t, const int32_t*, const int32_t*, int, float,
                             uint16_t*, void*, hipStream_t, bool x_ready = false);
int32_t dsv4_w8a16_split_k(int64_t, int64_t, int64_t);
int32_t dsv4_block_fp8_split_k(int64_t, int64_t, int64_t);
int dsv4_launch_act_quant_block_fp8(const void*, int32_t, int64_t, int64_t, uint8_t*, uint8_t*, hipStream_t);
int dsv4_launch_block_fp8_gemm(const uint8_t*, const uint8_t*, int64_t, int64_t, int64_t, const uint8_t*,
                               const uint8_t*, int32_t, float*, uint16_t*, hipStream_t, int w_rowmajor);
size_t dsv4_w8a16_workspace_bytes(int64_t, int64_t, int32_t);
int dsv4_launch_pack_int8(const int8_t*, int64_t, int64_t, uint8_t*, hipStream_t);
int dsv4_launch_decode_e8m0(const uint8_t*, int64_t, float*, hipStream_t);
int dsv4_launch_dequant_mxfp4(const uint8_t*, const float*, int64_t, int64_t, float*, hipStream_t);
int dsv4_launch_dequant_fp8_block(const void*, int32_t, const float*, int64_t, int64_t, float*, hipStream_t);
int dsv4_launch_w8a16(const uint16_t*, int64_t, int64_t, int64_t, const uint8_t*, const uint16_t*,
                      const uint8_t*, int32_t, float*, uint16_t*, hipStream_t, int accumulate, int w_rowmajor);
size_t dsv4_shared_fp8_workspace_bytes(int64_t, int, int);
int dsv4_launch_shared_fp8_add(const uint16_t*, int64_t, int, int, const uint8_t*, const uint8_t*, const uint8_t*,
                               const uint8_t*, float, uint16_t*, void*, hipStream_t);

using dsv4host::clear_error;
using dsv4host::set_error;

static bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

static int64_t max_padded(int64_t a, int32_t e, int32_t bs) {
  if (a <= 0 || e <= 0 || bs <= 0) return -1;
  int64_t m = a + (int64_t)e * (bs - 1);
  if (a < e) {
    const int64_t alt = a * bs;
    if (alt < m) m = alt;
  }
  return m;
}

static bool valid_block_size(int32_t bs) {
  return bs == 8 || bs == 16 || bs == 32 || bs == 48 || bs == 64;
}

extern "C" {

const char* dsv4moe_last_error(void) { return dsv4host::g_error; }

int32_t dsv4moe_abi_version(void) { return 3; }

int dsv4moe_profile_begin(int32_t max_calls) {
  return dsv4moe_profile_begin_stamps(max_calls, (1u << dsv4host::kNumStamps) - 1u);
}

int dsv4moe_profile_begin_stamps(int32_t max_calls, uint32_t stamp_mask) {
  clear_error();
  DSV4_REQUIRE(max_calls > 0 && max_calls <= 100000, "profile_begin: max_calls must be in [1, 100000]");
  DSV4_REQUIRE(stamp_mask != 0 && (stamp_mask >> dsv4host::kNumStamps) == 0,
               "profile_begin: stamp_mask must select stamps 0..%d", dsv4host::kNumStamps - 1);
  dsv4host::prof_release();
  dsv4host::g_prof.events.resize((size_t)max_calls * dsv4host::kNumStamps);
  for (auto& e : dsv4host::g_prof.events) {
    if (hipEventCreate(&e) != hipSuccess) {
      e = nullptr;
      dsv4host::prof_release();
      set_error("profile_begin: hipEventCreate failed");
      return DSV4MOE_EHIP;
    }
  }
  dsv4host::g_prof.max_calls = max_calls;
  dsv4host::g_prof.call = 0;
  dsv4host::g_prof.mask = stamp_mask;
  dsv4host::g_prof.active = true;
  return DSV4MOE_OK;
}

int dsv4moe_profile_end(float* mean_ms, int32_t n_intervals, int32_t* calls_recorded) {
  clear_error();
  using dsv4host::g_prof;
  using dsv4host::kNumStamps;
  DSV4_REQUIRE(g_prof.active, "profile_end: profiling is not active");
  DSV4_REQUIRE(mean_ms && n_intervals == kNumStamps - 1, "profile_end: need %d output slots",
               kNumStamps - 1);
  const int calls = g_prof.call;
  const uint32_t mask = g_prof.mask;
  // intervals whose two stamps were not both recorded read -1
  for (int i = 1; i < kNumStamps; ++i)
    mean_ms[i - 1] = ((mask >> (i - 1)) & 3u) == 3u ? 0.0f : -1.0f;
  int last = kNumStamps - 1;
  while (!(mask & (1u << last))) --last;
  int rc = DSV4MOE_OK;
  if (calls > 0 && hipEventSynchronize(g_prof.events[(size_t)(calls - 1) * kNumStamps + last]) != hipSuccess) {
    set_error("profile_end: hipEventSynchronize failed");
    rc = DSV4MOE_EHIP;
  }
  for (int c = 0; c < calls && rc == DSV4MOE_OK; ++c) {
    for (int i = 1; i < kNumStamps; ++i) {
      if (((mask >> (i - 1)) & 3u) != 3u) continue;
      float ms = 0.0f;
      if (hipEventElapsedTime(&ms, g_prof.events[(size_t)c * kNumStamps + i - 1],
                              g_prof.events[(size_t)c * kNumStamps + i]) != hipSuccess) {
        set_error("profile_end: hipEventElapsedTime failed");
        rc = DSV4MOE_EHIP;
        break;
      }
      mean_ms[i - 1] += ms / (float)calls;
    }
  }
  if (calls_recorded) *calls_recorded = calls;
  dsv4host::prof_release();
  return rc;
}

int32_t dsv4moe_block_size_m(int64_t rows, int32_t topk, int32_t experts, int32_t act_itemsize) {
  if (rows <= 0 || topk <= 0 || experts <= 0) return -1;
  int32_t selected = 64;
  const int32_t cands[5] = {8, 16, 32, 48, 64};
  for (int i = 0; i < 5; ++i) {
    // rows*topk/experts/candidate < 0.9, evaluated as the reference's float division
    const double ratio = (double)rows * (double)topk / (double)experts / (double)cands[i];
    if (ratio < 0.9) {
      selected = cands[i];
      break;
    }
  }
  if (act_itemsize == 1 && selected < 16) selected = 16;
  return selected;
}

int64_t dsv4moe_max_padded_tokens(int64_t num_assignments, int32_t num_experts, int32_t block_size) {
  return max_padded(num_assignments, num_experts, block_size);
}

int dsv4moe_route_topk(const float* logits, const float* bias, int64_t tokens, int32_t experts,
                       int32_t topk, int32_t score_func, float route_scale, int32_t* ids,
                       float* weights, float* margin, int32_t* selection_ids,
                       float* selection_scores, void* stream) {
  clear_error();
  DSV4_REQUIRE(tokens >= 0, "route_topk: tokens must be >= 0");
  DSV4_REQUIRE(experts >= 1 && experts <= 1024, "route_topk: experts must be in [1, 1024]");
  DSV4_REQUIRE(topk >= 1 && topk <= experts && topk <= 16,
               "route_topk: topk must be in [1, min(experts, 16)]");
  DSV4_REQUIRE(score_func == DSV4MOE_SCORE_SIGMOID || score_func == DSV4MOE_SCORE_SOFTMAX ||
                   score_func == DSV4MOE_SCORE_SQRTSOFTPLUS,
               "route_topk: unknown score_func %d", score_func);
  DSV4_REQUIRE(route_scale > 0.0f && route_scale < 3.0e38f, "route_topk: route_scale must be finite and positive");
  if (tokens == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(logits && ids && weights, "route_topk: null logits/ids/weights");
  return dsv4_launch_route_topk(logits, bias, tokens, experts, topk, score_func, route_scale, ids,
                                weights, margin, selection_ids, selection_scores,
                                static_cast<hipStream_t>(stream));
}

int dsv4moe_route_hash(const float* logits, const int64_t* tid2eid, int64_t vocab,
                       const int64_t* input_ids, int64_t tokens, int32_t experts, int32_t topk,
                       float route_scale, int32_t* ids, float* weights,
                       float* selected_scores, void* stream) {
  clear_error();
  DSV4_REQUIRE(tokens >= 0 && vocab > 0, "route_hash: bad tokens/vocab");
  DSV4_REQUIRE(experts >= 1 && experts <= 1024, "route_hash: experts must be in [1, 1024]");
  DSV4_REQUIRE(topk >= 1 && topk < experts && topk <= 16, "route_hash: topk must be in [1, experts)");
  DSV4_REQUIRE(route_scale > 0.0f && route_scale < 3.0e38f, "route_hash: route_scale must be finite and positive");
  if (tokens == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(logits && tid2eid && input_ids && ids && weights, "route_hash: null pointer");
  return dsv4_launch_route_hash(logits, tid2eid, vocab, input_ids, tokens, experts, topk,
                                route_scale, ids, weights, selected_scores,
                                static_cast<hipStream_t>(stream));
}

int dsv4moe_gate_logits(const uint16_t* x, const uint16_t* wg, int64_t tokens, int32_t hidden,
                        int32_t experts, float* logits, void* stream) {
  clear_error();
  DSV4_REQUIRE(tokens >= 0, "gate_logits: tokens must be >= 0");
  DSV4_REQUIRE(hidden > 0 && hidden % 32 == 0, "gate_logits: hidden must be a positive multiple of 32");
  DSV4_REQUIRE(experts > 0 && experts <= 65535 * 64, "gate_logits: bad experts");
  if (tokens == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(x && wg && logits, "gate_logits: null pointer");
  DSV4_REQUIRE(aligned(x, 16) && aligned(wg, 16), "gate_logits: x and wg must be 16-byte aligned");
  return dsv4_launch_gate_logits(x, wg, tokens, hidden, experts, logits,
                                 static_cast<hipStream_t>(stream));
}

static int validate_align(const char* who, const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts,
                          int32_t block_size, const int32_t* sorted_token_ids, int64_t capacity,
                          const int32_t* expert_ids, int64_t num_blocks, const int32_t* num_tokens_post_padded) {
  DSV4_REQUIRE(tokens > 0 && topk > 0, "%s: route ids must be non-empty [tokens, topk]", who);
  DSV4_REQUIRE(experts >= 1 && experts <= 1024, "%s: experts must be in [1, 1024]", who);
  DSV4_REQUIRE(block_size > 0 && block_size <= 1024, "%s: bad block_size %d", who, block_size);
  const int64_t a = tokens * topk;
  DSV4_REQUIRE(a <= 0x7FFFFFFFLL, "%s: assignments exceed int32", who);
  const int64_t cap = max_padded(a, experts, block_size);
  DSV4_REQUIRE(cap <= 0x7FFFFFFFLL, "%s: capacity exceeds int32", who);
  DSV4_REQUIRE(capacity == cap, "%s: capacity %lld != max_padded_tokens %lld", who, (long long)capacity,
               (long long)cap);
  DSV4_REQUIRE(num_blocks == (cap + block_size - 1) / block_size, "%s: expert_ids length mismatch", who);
  DSV4_REQUIRE(ids && sorted_token_ids && expert_ids && num_tokens_post_padded, "%s: null pointer", who);
  return DSV4MOE_OK;
}

int dsv4moe_align(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts,
                  int32_t block_size, int32_t* sorted_token_ids, int64_t capacity,
                  int32_t* expert_ids, int64_t num_blocks, int32_t* num_tokens_post_padded,
                  void* stream) {
  clear_error();
  const int rc = validate_align("align", ids, tokens, topk, experts, block_size, sorted_token_ids, capacity,
                                expert_ids, num_blocks, num_tokens_post_padded);
  if (rc != DSV4MOE_OK) return rc;
  return dsv4_launch_align(ids, tokens * topk, experts, block_size, sorted_token_ids, capacity, expert_ids,
                           num_blocks, num_tokens_post_padded, static_cast<hipStream_t>(stream));
}

size_t dsv4moe_align_workspace_bytes(int64_t tokens, int32_t topk, int32_t experts) {
  if (tokens <= 0 || topk <= 0 || experts < 1 || experts > 1024) return 0;
  const int64_t a = tokens * topk;
  return a >= kAlignMultiMinAssignments ? dsv4_align_scratch_bytes(a, experts) : 0;
}

int dsv4moe_align_ws(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts, int32_t block_size,
                     int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids, int64_t num_blocks,
                     int32_t* num_tokens_post_padded, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  const int rc = validate_align("align_ws", ids, tokens, topk, experts, block_size, sorted_token_ids, capacity,
                                expert_ids, num_blocks, num_tokens_post_padded);
  if (rc != DSV4MOE_OK) return rc;
  const size_t need = dsv4moe_align_workspace_bytes(tokens, topk, experts);
  DSV4_REQUIRE(workspace_bytes >= need, "align_ws: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  DSV4_REQUIRE(need == 0 || (workspace && aligned(workspace, 4)), "align_ws: workspace must be 4-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (need == 0)
    return dsv4_launch_align(ids, tokens * topk, experts, block_size, sorted_token_ids, capacity, expert_ids,
                             num_blocks, num_tokens_post_padded, s);
  return dsv4_launch_align_multi(ids, tokens * topk, experts, block_size, sorted_token_ids, capacity, expert_ids,
                                 num_blocks, num_tokens_post_padded, static_cast<int32_t*>(workspace),
                                 dsv4::ActPrep{dsv4::kPrepNone, nullptr, 0, nullptr, nullptr, nullptr}, tokens, s);
}

int dsv4moe_pack_int4_g128(const uint8_t* canon, const uint16_t* canon_scales, int64_t batch,
                           int64_t n, int64_t k, int32_t pairing, uint8_t* packed,
                           uint16_t* packed_scales, void* stream) {
  clear_error();
  DSV4_REQUIRE(batch >= 0 && n >= 0 && k >= 0, "pack: negative size");
  DSV4_REQUIRE(n % 32 == 0, "pack: n=%lld must be a multiple of 32", (long long)n);
  DSV4_REQUIRE(pairing == DSV4MOE_PAIR_PLAIN || pairing == DSV4MOE_PAIR_GATED,
               "pack: unknown pairing %d", pairing);
  DSV4_REQUIRE(k % DSV4MOE_GROUP == 0, "pack: k=%lld must be a multiple of 128", (long long)k);
  if (batch == 0 || n == 0 || k == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(canon && canon_scales && packed && packed_scales, "pack: null pointer");
  DSV4_REQUIRE(aligned(canon, 4) && aligned(packed, 16), "pack: canon 4-byte / packed 16-byte alignment required");
  return dsv4_launch_pack(canon, canon_scales, batch, n, k, pairing, packed, packed_scales,
                          static_cast<hipStream_t>(stream));
}

int dsv4moe_pack_int4_ratios(const uint16_t* packed_scales, int64_t batch, int64_t n, int64_t k, float* ratios,
                             void* stream) {
  clear_error();
  DSV4_REQUIRE(batch >= 0 && n >= 0 && k >= 0, "pack_ratios: negative size");
  DSV4_REQUIRE(n % 32 == 0, "pack_ratios: n=%lld must be a multiple of 32", (long long)n);
  DSV4_REQUIRE(k % DSV4MOE_GROUP == 0, "pack_ratios: k=%lld must be a multiple of 128", (long long)k);
  if (batch == 0 || n == 0 || k == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(packed_scales && ratios, "pack_ratios: null pointer");
  DSV4_REQUIRE(aligned(packed_scales, 2) && aligned(ratios, 16),
               "pack_ratios: scales 2-byte / ratios 16-byte alignment required");
  return dsv4_launch_pack_ratios(packed_scales, batch, n, k, ratios, static_cast<hipStream_t>(stream));
}

size_t dsv4moe_experts_workspace_bytes(int64_t tokens, int32_t topk, int32_t hidden,
                                       int32_t inter, int32_t has_shared) {
  if (tokens < 0 || topk <= 0 || hidden <= 0 || inter <= 0) return 0;
  return dsv4_experts_workspace_bytes(tokens, topk, hidden, inter, has_shared ? 1 : 0);
}

// The W4A16 prefill kernels' group-scale ratios (dsv4moe_pack_int4_ratios).
static int validate_ratios(const char* who, const float* w13r, const float* w2r) {
  DSV4_REQUIRE(w13r && w2r, "%s: null scale-ratio pointer (dsv4moe_pack_int4_ratios)", who);
  DSV4_REQUIRE(aligned(w13r, 16) && aligned(w2r, 16), "%s: scale ratios must be 16-byte aligned", who);
  return DSV4MOE_OK;
}

static int validate_experts(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                            int32_t experts, int32_t topk, const uint8_t* w13q,
                            const uint16_t* w13s, const uint8_t* w2q, const uint16_t* w2s,
                            int64_t capacity, int32_t block_size, uint16_t* out, void* workspace,
                            size_t workspace_bytes, int32_t has_shared, const char* who,
                            bool a8 = false) {
  DSV4_REQUIRE(tokens >= 0, "%s: tokens must be >= 0", who);
  DSV4_REQUIRE(!a8 || (hidden % 512 == 0 && inter % 512 == 0),
               "%s: W4A8 needs hidden and inter to be multiples of 512 (got %d, %d)", who, hidden, inter);
  DSV4_REQUIRE(hidden > 0 && hidden % 256 == 0, "%s: hidden=%d must be a positive multiple of 256", who, hidden);
  DSV4_REQUIRE(inter > 0 && inter % 256 == 0, "%s: inter=%d must be a positive multiple of 256", who, inter);
  DSV4_REQUIRE(experts >= 1 && experts <= 1024, "%s: experts must be in [1, 1024]", who);
  DSV4_REQUIRE(topk >= 1 && topk <= experts, "%s: topk must be in [1, experts]", who);
  DSV4_REQUIRE(valid_block_size(block_size), "%s: block_size %d not in {8,16,32,48,64}", who, block_size);
  if (tokens == 0) return DSV4MOE_OK;
  const int64_t cap = max_padded(tokens * topk, experts, block_size);
  DSV4_REQUIRE(capacity == cap, "%s: capacity %lld != max_padded_tokens %lld", who,
               (long long)capacity, (long long)cap);
  DSV4_REQUIRE(x && w13q && w13s && w2q && w2s && out && workspace, "%s: null pointer", who);
  DSV4_REQUIRE(aligned(x, 16) && aligned(w13q, 16) && aligned(w2q, 16) && aligned(w13s, 8) &&
                   aligned(w2s, 8) && aligned(out, 8) && aligned(workspace, 256),
               "%s: alignment (x/w*q 16 B, scales/out 8 B, workspace 256 B)", who);
  const size_t need = a8 ? dsv4_experts_w4a8_workspace_bytes(tokens, topk, hidden, inter, has_shared ? 1 : 0)
                        : dsv4_experts_workspace_bytes(tokens, topk, hidden, inter, has_shared ? 1 : 0);
  DSV4_REQUIRE(workspace_bytes >= need, "%s: workspace %zu bytes < required %zu", who,
               workspace_bytes, need);
  const int64_t act_rows = tokens * topk + (has_shared ? tokens : 0);
  DSV4_REQUIRE(act_rows * (int64_t)(hidden > inter ? hidden : inter) * 4 < 0x7FFFFFFFLL,
               "%s: activation / intermediate arrays exceed 2 GiB (split the batch)", who);
  const int64_t blocks = (cap + block_size - 1) / block_size;
  const int64_t shared_blocks = has_shared ? (tokens + block_size - 1) / block_size : 0;
  const int64_t tiles = (int64_t)(hidden > inter ? hidden : inter) / 128;
  DSV4_REQUIRE((blocks + shared_blocks) * tiles < 0x7FFFFFFFLL, "%s: grid too large", who);
  return DSV4MOE_OK;
}

int dsv4moe_experts_w4a16(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                          int32_t experts, int32_t topk, const uint8_t* w13q,
                          const uint16_t* w13s, const uint8_t* w2q, const uint16_t* w2s,
                          const float* w13r, const float* w2r, int32_t has_shared, const float* weights,
                          const int32_t* sorted_token_ids, int64_t capacity,
                          const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                          int32_t block_size, float clamp_limit, uint16_t* out,
                          void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_experts(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s,
                            capacity, block_size, out, workspace, workspace_bytes, has_shared,
                            "experts_w4a16");
  if (rc != DSV4MOE_OK || tokens == 0) return rc;
  rc = validate_ratios("experts_w4a16", w13r, w2r);
  if (rc != DSV4MOE_OK) return rc;
  DSV4_REQUIRE(weights && sorted_token_ids && expert_ids && num_tokens_post_padded,
               "experts_w4a16: null route/alignment pointer");
  DSV4_REQUIRE(!(clamp_limit < 0.0f) && clamp_limit < 3.0e38f, "experts_w4a16: clamp_limit must be >= 0 and finite");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dsv4host::prof_stamp(dsv4host::kStampBegin, s);
  dsv4host::prof_stamp(dsv4host::kStampRoute, s);
  dsv4host::prof_stamp(dsv4host::kStampAlign, s);
  return dsv4_launch_experts_w4a16(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s, w13r, w2r,
                                   has_shared ? 1 : 0, weights, sorted_token_ids, capacity,
                                   expert_ids, num_tokens_post_padded, block_size, clamp_limit,
                                   out, workspace, static_cast<hipStream_t>(stream));
}

int dsv4moe_pack_mxfp4_g32(const uint8_t* canon, const uint8_t* canon_scales, int64_t batch, int64_t n,
                           int64_t k, int32_t pairing, uint8_t* packed, uint8_t* packed_scales, void* stream) {
  clear_error();
  DSV4_REQUIRE(batch >= 0 && n >= 0 && k >= 0, "pack_mxfp4: negative size");
  DSV4_REQUIRE(n % 32 == 0, "pack_mxfp4: n=%lld must be a multiple of 32", (long long)n);
  DSV4_REQUIRE(pairing == DSV4MOE_PAIR_PLAIN || pairing == DSV4MOE_PAIR_GATED,
               "pack_mxfp4: unknown pairing %d", pairing);
  DSV4_REQUIRE(k % DSV4MOE_GROUP == 0, "pack_mxfp4: k=%lld must be a multiple of 128", (long long)k);
  if (batch == 0 || n == 0 || k == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(canon && canon_scales && packed && packed_scales, "pack_mxfp4: null pointer");
  DSV4_REQUIRE(aligned(canon, 4) && aligned(packed, 16), "pack_mxfp4: canon 4-byte / packed 16-byte alignment required");
  return dsv4_launch_pack_mxfp4(canon, canon_scales, batch, n, k, pairing, packed, packed_scales,
                                static_cast<hipStream_t>(stream));
}

int dsv4moe_pack_mxfp4_g32_w4a8(const uint8_t* canon, const uint8_t* canon_scales, int64_t batch, int64_t n,
                                int64_t k, int32_t pairing, uint8_t* packed, uint8_t* packed_scales,
                                void* stream) {
  clear_error();
  DSV4_REQUIRE(batch >= 0 && n >= 0 && k >= 0, "pack_mxfp4_w4a8: negative size");
  DSV4_REQUIRE(n % 32 == 0, "pack_mxfp4_w4a8: n=%lld must be a multiple of 32", (long long)n);
  DSV4_REQUIRE(pairing == DSV4MOE_PAIR_PLAIN || pairing == DSV4MOE_PAIR_GATED,
               "pack_mxfp4_w4a8: unknown pairing %d", pairing);
  DSV4_REQUIRE(k % DSV4MOE_GROUP == 0, "pack_mxfp4_w4a8: k=%lld must be a multiple of 128", (long long)k);
  if (batch == 0 || n == 0 || k == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(canon && canon_scales && packed && packed_scales, "pack_mxfp4_w4a8: null pointer");
  DSV4_REQUIRE(aligned(canon, 4) && aligned(packed, 16),
               "pack_mxfp4_w4a8: canon 4-byte / packed 16-byte alignment required");
  return dsv4_launch_pack_mxfp4_a8(canon, canon_scales, batch, n, k, pairing, packed, packed_scales,
                                   static_cast<hipStream_t>(stream));
}

int dsv4moe_experts_w4a8_mxfp4(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                               int32_t experts, int32_t topk, const uint8_t* w13q, const uint8_t* w13s,
                               const uint8_t* w2q, const uint8_t* w2s, int32_t has_shared, const float* weights,
                               const int32_t* sorted_token_ids, int64_t capacity, const int32_t* expert_ids,
                               const int32_t* num_tokens_post_padded, int32_t block_size, float clamp_limit,
                               uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_experts(x, tokens, hidden, inter, experts, topk, w13q,
                            reinterpret_cast<const uint16_t*>(w13s), w2q, reinterpret_cast<const uint16_t*>(w2s),
                            capacity, block_size, out, workspace, workspace_bytes, has_shared,
                            "experts_w4a8_mxfp4", true);
  if (rc != DSV4MOE_OK || tokens == 0) return rc;
  DSV4_REQUIRE(weights && sorted_token_ids && expert_ids && num_tokens_post_padded,
               "experts_w4a8_mxfp4: null route/alignment pointer");
  DSV4_REQUIRE(!(clamp_limit < 0.0f) && clamp_limit < 3.0e38f,
               "experts_w4a8_mxfp4: clamp_limit must be >= 0 and finite");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dsv4host::prof_stamp(dsv4host::kStampBegin, s);
  dsv4host::prof_stamp(dsv4host::kStampRoute, s);
  dsv4host::prof_stamp(dsv4host::kStampAlign, s);
  return dsv4_launch_experts_w4a8_mxfp4(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s,
                                        has_shared ? 1 : 0, weights, sorted_token_ids, capacity, expert_ids,
                                        num_tokens_post_padded, block_size, clamp_limit, out, workspace, s);
}

int dsv4moe_experts_mxfp4(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                          int32_t experts, int32_t topk, const uint8_t* w13q, const uint8_t* w13s,
                          const uint8_t* w2q, const uint8_t* w2s, int32_t has_shared, const float* weights,
                          const int32_t* sorted_token_ids, int64_t capacity, const int32_t* expert_ids,
                          const int32_t* num_tokens_post_padded, int32_t block_size, float clamp_limit,
                          uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  DSV4_REQUIRE(hidden % 512 == 0 && inter % 512 == 0,
               "experts_mxfp4: hidden and inter must be multiples of 512 (got %d, %d)", hidden, inter);
  int rc = validate_experts(x, tokens, hidden, inter, experts, topk, w13q,
                            reinterpret_cast<const uint16_t*>(w13s), w2q, reinterpret_cast<const uint16_t*>(w2s),
                            capacity, block_size, out, workspace, workspace_bytes, has_shared, "experts_mxfp4");
  if (rc != DSV4MOE_OK || tokens == 0) return rc;
  DSV4_REQUIRE(weights && sorted_token_ids && expert_ids && num_tokens_post_padded,
               "experts_mxfp4: null route/alignment pointer");
  DSV4_REQUIRE(!(clamp_limit < 0.0f) && clamp_limit < 3.0e38f, "experts_mxfp4: clamp_limit must be >= 0 and finite");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dsv4host::prof_stamp(dsv4host::kStampBegin, s);
  dsv4host::prof_stamp(dsv4host::kStampRoute, s);
  dsv4host::prof_stamp(dsv4host::kStampAlign, s);
  return dsv4_launch_experts_mxfp4(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s,
                                   has_shared ? 1 : 0, weights, sorted_token_ids, capacity, expert_ids,
                                   num_tokens_post_padded, block_size, clamp_limit, out, workspace, s);
}

// Checks shared by the fused layer entries (who = entry name), after the
// experts checks.
static int validate_layer_route(const char* who, const float* logits, int32_t topk, int32_t score_func,
                                float route_scale, float clamp_limit, const int32_t* ids, const float* weights,
                                const int32_t* sorted_token_ids, const int32_t* expert_ids,
                                const int32_t* num_tokens_post_padded) {
  DSV4_REQUIRE(topk <= 16, "%s: topk must be <= 16", who);
  DSV4_REQUIRE(score_func == DSV4MOE_SCORE_SIGMOID || score_func == DSV4MOE_SCORE_SOFTMAX ||
                   score_func == DSV4MOE_SCORE_SQRTSOFTPLUS,
               "%s: unknown score_func %d", who, score_func);
  DSV4_REQUIRE(route_scale > 0.0f && route_scale < 3.0e38f, "%s: route_scale must be finite and positive", who);
  DSV4_REQUIRE(!(clamp_limit < 0.0f) && clamp_limit < 3.0e38f, "%s: clamp_limit must be >= 0 and finite", who);
  DSV4_REQUIRE(logits && ids && weights && sorted_token_ids && expert_ids && num_tokens_post_padded,
               "%s: null route/alignment pointer", who);
  return DSV4MOE_OK;
}

// Route and align a fused layer call, with the activation work of `prep`
// (row sums, W4A8 quantisation or none) beside the alignment, by token count:
// for T <= 16 one prologue launch routes, aligns and does `prep`; up to 8191
// route ids the route kernel, then the prologue (align + prep); from 8192 ids
// the route kernel, then the workgroup-split alignment with `prep` beside its
// counting and its scratch (`room` bytes) in the not yet used contribution
// region of the experts workspace.
static int layer_route_align(const char* who, const dsv4::ActPrep& prep, int32_t* scratch, size_t room,
                             const float* logits, const float* bias, int64_t tokens, int32_t experts, int32_t topk,
                             int32_t score_func, float route_scale, int32_t block_size, int32_t* ids, float* weights,
                             float* margin, int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                             int32_t* num_tokens_post_padded, hipStream_t s) {
  int rc = DSV4MOE_OK;
  const int64_t nblocks = (capacity + block_size - 1) / block_size;
  // (with routing in the prologue the route interval of the profile covers
  // the whole prologue, and the align interval is empty)
  const bool route_in_prologue = tokens <= kPrologueRouteMaxTokens;
  if (!route_in_prologue) {
    rc = dsv4_launch_route_topk(logits, bias, tokens, experts, topk, score_func, route_scale, ids,
                                weights, margin, nullptr, nullptr, s);
    if (rc != DSV4MOE_OK) return rc;
    dsv4host::prof_stamp(dsv4host::kStampRoute, s);
  }
  if (tokens * topk >= kAlignMultiMinAssignments) {
    DSV4_REQUIRE(room >= dsv4_align_scratch_bytes(tokens * topk, experts), "%s: align scratch too small", who);
    rc = dsv4_launch_align_multi(ids, tokens * topk, experts, block_size, sorted_token_ids, capacity, expert_ids,
                                 nblocks, num_tokens_post_padded, scratch, prep, tokens, s);
  } else {
    rc = dsv4_launch_prologue(route_in_prologue ? 1 : 0, logits, bias, tokens, experts, topk, score_func,
                              route_scale, ids, weights, margin, block_size, sorted_token_ids, capacity, expert_ids,
                              nblocks, num_tokens_post_padded, prep, s);
  }
  if (rc != DSV4MOE_OK) return rc;
  if (route_in_prologue) dsv4host::prof_stamp(dsv4host::kStampRoute, s);
  dsv4host::prof_stamp(dsv4host::kStampAlign, s);
  return DSV4MOE_OK;
}

int dsv4moe_layer_w4a16(const uint16_t* x, const float* logits, const float* bias,
                        int64_t tokens, int32_t hidden, int32_t inter, int32_t experts,
                        int32_t topk, int32_t score_func, float route_scale,
                        const uint8_t* w13q, const uint16_t* w13s, const uint8_t* w2q,
                        const uint16_t* w2s, const float* w13r, const float* w2r, int32_t has_shared,
                        float clamp_limit,
                        int32_t block_size, int32_t* ids, float* weights, float* margin,
                        int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                        int32_t* num_tokens_post_padded, uint16_t* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_experts(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s,
                            capacity, block_size, out, workspace, workspace_bytes, has_shared,
                            "layer_w4a16");
  if (rc != DSV4MOE_OK || tokens == 0) return rc;
  rc = validate_ratios("layer_w4a16", w13r, w2r);
  if (rc != DSV4MOE_OK) return rc;
  rc = validate_layer_route("layer_w4a16", logits, topk, score_func, route_scale, clamp_limit, ids, weights,
                            sorted_token_ids, expert_ids, num_tokens_post_padded);
  if (rc != DSV4MOE_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dsv4host::prof_stamp(dsv4host::kStampBegin, s);
  size_t room = 0;
  int32_t* scratch = dsv4_experts_align_scratch(workspace, tokens, topk, hidden, inter, has_shared ? 1 : 0, &room);
  const dsv4::ActPrep prep{dsv4::w4a16_decode_path(block_size, hidden, inter) ? dsv4::kPrepRowSums : dsv4::kPrepRowNc,
                           x, hidden, dsv4_experts_xsum(workspace, tokens, topk, hidden, inter, has_shared ? 1 : 0),
                           nullptr, nullptr};
  rc = layer_route_align("layer_w4a16", prep, scratch, room, logits, bias, tokens, experts, topk, score_func,
                         route_scale, block_size, ids, weights, margin, sorted_token_ids, capacity, expert_ids,
                         num_tokens_post_padded, s);
  if (rc != DSV4MOE_OK) return rc;
  return dsv4_launch_experts_w4a16(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s, w13r, w2r,
                                   has_shared ? 1 : 0, weights, sorted_token_ids, capacity, expert_ids,
                                   num_tokens_post_padded, block_size, clamp_limit, out, workspace, s,
                                   /*rowsums_ready=*/true);
}

int dsv4moe_layer_mxfp4(const uint16_t* x, const float* logits, const float* bias,
                        int64_t tokens, int32_t hidden, int32_t inter, int32_t experts,
                        int32_t topk, int32_t score_func, float route_scale,
                        const uint8_t* w13q, const uint8_t* w13s, const uint8_t* w2q,
                        const uint8_t* w2s, int32_t has_shared, float clamp_limit,
                        int32_t block_size, int32_t* ids, float* weights, float* margin,
                        int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                        int32_t* num_tokens_post_padded, uint16_t* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  clear_error();
  DSV4_REQUIRE(hidden % 512 == 0 && inter % 512 == 0,
               "layer_mxfp4: hidden and inter must be multiples of 512 (got %d, %d)", hidden, inter);
  int rc = validate_experts(x, tokens, hidden, inter, experts, topk, w13q, reinterpret_cast<const uint16_t*>(w13s),
                            w2q, reinterpret_cast<const uint16_t*>(w2s), capacity, block_size, out, workspace,
                            workspace_bytes, has_shared, "layer_mxfp4");
  if (rc != DSV4MOE_OK || tokens == 0) return rc;
  rc = validate_layer_route("layer_mxfp4", logits, topk, score_func, route_scale, clamp_limit, ids, weights,
                            sorted_token_ids, expert_ids, num_tokens_post_padded);
  if (rc != DSV4MOE_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dsv4host::prof_stamp(dsv4host::kStampBegin, s);
  // the MXFP4 kernels need no activation row sums (the E8M0 scale is exact
  // inside the conversion)
  size_t room = 0;
  int32_t* scratch = dsv4_experts_align_scratch(workspace, tokens, topk, hidden, inter, has_shared ? 1 : 0, &room);
  rc = layer_route_align("layer_mxfp4", dsv4::ActPrep{dsv4::kPrepNone, nullptr, 0, nullptr, nullptr, nullptr},
                         scratch, room, logits, bias, tokens, experts, topk, score_func, route_scale, block_size,
                         ids, weights, margin, sorted_token_ids, capacity, expert_ids, num_tokens_post_padded, s);
  if (rc != DSV4MOE_OK) return rc;
  return dsv4_launch_experts_mxfp4(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s,
                                   has_shared ? 1 : 0, weights, sorted_token_ids, capacity, expert_ids,
                                   num_tokens_post_padded, block_size, clamp_limit, out, workspace, s);
}

// The W4A8 fused layer calls: route -> align (with x quantised to e4m3 by the
// prologue's other workgroups) -> the W4A8 experts chain.  `mxfp4` picks the
// MXFP4 W4A8 kernels (x in K order) over the int4 ones.
static int layer_w4a8_common(const char* who, bool mxfp4, const uint16_t* x, const float* logits, const float* bias,
                             int64_t tokens, int32_t hidden, int32_t inter, int32_t experts, int32_t topk,
                             int32_t score_func, float route_scale, const uint8_t* w13q, const void* w13s,
                             const uint8_t* w2q, const void* w2s, int32_t has_shared, float clamp_limit,
                             int32_t block_size, int32_t* ids, float* weights, float* margin,
                             int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                             int32_t* num_tokens_post_padded, uint16_t* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_experts(x, tokens, hidden, inter, experts, topk, w13q, static_cast<const uint16_t*>(w13s), w2q,
                            static_cast<const uint16_t*>(w2s), capacity, block_size, out, workspace, workspace_bytes,
                            has_shared, who, true);
  if (rc != DSV4MOE_OK || tokens == 0) return rc;
  rc = validate_layer_route(who, logits, topk, score_func, route_scale, clamp_limit, ids, weights, sorted_token_ids,
                            expert_ids, num_tokens_post_padded);
  if (rc != DSV4MOE_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dsv4host::prof_stamp(dsv4host::kStampBegin, s);
  uint8_t* xq = nullptr;
  float* xscale = nullptr;
  float* xsum = nullptr;
  int32_t* scratch = nullptr;
  size_t room = 0;
  dsv4_experts_w4a8_pieces(workspace, tokens, topk, hidden, inter, has_shared ? 1 : 0, &xq, &xscale, &xsum,
                           &scratch, &room);
  const dsv4::ActPrep prep{mxfp4 ? dsv4::kPrepQuantNatural : dsv4::kPrepQuantInt4, x, hidden, xsum, xq, xscale};
  rc = layer_route_align(who, prep, scratch, room, logits, bias, tokens, experts, topk, score_func, route_scale,
                         block_size, ids, weights, margin, sorted_token_ids, capacity, expert_ids,
                         num_tokens_post_padded, s);
  if (rc != DSV4MOE_OK) return rc;
  if (mxfp4)
    return dsv4_launch_experts_w4a8_mxfp4(x, tokens, hidden, inter, experts, topk, w13q,
                                          static_cast<const uint8_t*>(w13s), w2q, static_cast<const uint8_t*>(w2s),
                                          has_shared ? 1 : 0, weights, sorted_token_ids, capacity, expert_ids,
                                          num_tokens_post_padded, block_size, clamp_limit, out, workspace, s,
                                          /*x_ready=*/true);
  return dsv4_launch_experts_w4a8(x, tokens, hidden, inter, experts, topk, w13q, static_cast<const uint16_t*>(w13s),
                                  w2q, static_cast<const uint16_t*>(w2s), has_shared ? 1 : 0, weights,
                                  sorted_token_ids, capacity, expert_ids, num_tokens_post_padded, block_size,
                                  clamp_limit, out, workspace, s, /*x_ready=*/true);
}

int dsv4moe_layer_w4a8(const uint16_t* x, const float* logits, const float* bias, int64_t tokens, int32_t hidden,
                       int32_t inter, int32_t experts, int32_t topk, int32_t score_func, float route_scale,
                       const uint8_t* w13q, const uint16_t* w13s, const uint8_t* w2q, const uint16_t* w2s,
                       int32_t has_shared, float clamp_limit, int32_t block_size, int32_t* ids, float* weights,
                       float* margin, int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                       int32_t* num_tokens_post_padded, uint16_t* out, void* workspace, size_t workspace_bytes,
                       void* stream) {
  return layer_w4a8_common("layer_w4a8", false, x, logits, bias, tokens, hidden, inter, experts, topk, score_func,
                           route_scale, w13q, w13s, w2q, w2s, has_shared, clamp_limit, block_size, ids, weights,
                           margin, sorted_token_ids, capacity, expert_ids, num_tokens_post_padded, out, workspace,
                           workspace_bytes, stream);
}

int dsv4moe_layer_w4a8_mxfp4(const uint16_t* x, const float* logits, const float* bias, int64_t tokens,
                             int32_t hidden, int32_t inter, int32_t experts, int32_t topk, int32_t score_func,
                             float route_scale, const uint8_t* w13q, const uint8_t* w13s, const uint8_t* w2q,
                             const uint8_t* w2s, int32_t has_shared, float clamp_limit, int32_t block_size,
                             int32_t* ids, float* weights, float* margin, int32_t* sorted_token_ids,
                             int64_t capacity, int32_t* expert_ids, int32_t* num_tokens_post_padded, uint16_t* out,
                             void* workspace, size_t workspace_bytes, void* stream) {
  return layer_w4a8_common("layer_w4a8_mxfp4", true, x, logits, bias, tokens, hidden, inter, experts, topk,
                           score_func, route_scale, w13q, w13s, w2q, w2s, has_shared, clamp_limit, block_size, ids,
                           weights, margin, sorted_token_ids, capacity, expert_ids, num_tokens_post_padded, out,
                           workspace, workspace_bytes, stream);
}

// ------------------------------------------------ allocation-free layer entry
// dsv4moe_layer_w4a16_noalloc keeps the experts workspace in this static
// device array instead of a caller buffer.  Every GPU the library runs on
// holds its own copy, at its own address, until the process ends.  In host
// code `scratch` names a host-side stand-in, never the device memory: the
// address passed to the kernels comes from hipGetSymbolAddress, taken once
// per device with that device current and kept in g_noalloc_scratch.  The
// array keeps the last call's contents; nothing in it needs to start at zero
// (each call writes every workspace region before reading it).  Calls that
// overlap on one GPU share the array and race.
static __device__ __align__(256) unsigned char scratch[DSV4MOE_NOALLOC_SCRATCH_BYTES];

static constexpr int kMaxScratchDevices = 64;
static std::mutex g_noalloc_mutex;
static void* g_noalloc_scratch[kMaxScratchDevices] = {};

// The device address of `scratch` on the device that runs `stream`.
static int noalloc_scratch_address(hipStream_t stream, void** address) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("layer_w4a16_noalloc: hipGetDevice: %s", hipGetErrorString(err));
    return DSV4MOE_EHIP;
  }
  if (stream != nullptr) {
    hipDevice_t stream_dev = -1;
    err = hipStreamGetDevice(stream, &stream_dev);
    if (err != hipSuccess) {
      set_error("layer_w4a16_noalloc: hipStreamGetDevice: %s", hipGetErrorString(err));
      return DSV4MOE_EHIP;
    }
    DSV4_REQUIRE(stream_dev == dev, "layer_w4a16_noalloc: the stream runs on device %d but device %d is current",
                 (int)stream_dev, dev);
  }
  DSV4_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "layer_w4a16_noalloc: device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_noalloc_mutex);
  if (g_noalloc_scratch[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      set_error("layer_w4a16_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(err));
      return DSV4MOE_EHIP;
    }
    g_noalloc_scratch[dev] = p;
  }
  *address = g_noalloc_scratch[dev];
  return DSV4MOE_OK;
}

int dsv4moe_layer_w4a16_noalloc(const uint16_t* x, const float* logits, const float* bias,
                                int64_t tokens, int32_t hidden, int32_t inter, int32_t experts,
                                int32_t topk, int32_t score_func, float route_scale,
                                const uint8_t* w13q, const uint16_t* w13s, const uint8_t* w2q,
                                const uint16_t* w2s, const float* w13r, const float* w2r, int32_t has_shared,
                                float clamp_limit, int32_t block_size, int32_t* ids, float* weights,
                                float* margin, int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                                int32_t* num_tokens_post_padded, uint16_t* out, void* stream) {
  clear_error();
  if (tokens == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(tokens > 0 && topk > 0 && hidden > 0 && inter > 0,
               "layer_w4a16_noalloc: tokens, topk, hidden and inter must be positive");
  const size_t need = dsv4_experts_workspace_bytes(tokens, topk, hidden, inter, has_shared ? 1 : 0);
  DSV4_REQUIRE(need <= (size_t)DSV4MOE_NOALLOC_SCRATCH_BYTES,
               "layer_w4a16_noalloc: %lld tokens need %zu bytes of workspace, more than the %zu-byte static "
               "scratch; call dsv4moe_layer_w4a16 with a caller workspace",
               (long long)tokens, need, (size_t)DSV4MOE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = noalloc_scratch_address(static_cast<hipStream_t>(stream), &ws);
  if (rc != DSV4MOE_OK) return rc;
  return dsv4moe_layer_w4a16(x, logits, bias, tokens, hidden, inter, experts, topk, score_func, route_scale, w13q,
                             w13s, w2q, w2s, w13r, w2r, has_shared, clamp_limit, block_size, ids, weights, margin,
                             sorted_token_ids, capacity, expert_ids, num_tokens_post_padded, out, ws,
                             (size_t)DSV4MOE_NOALLOC_SCRATCH_BYTES, stream);
}

int dsv4moe_pack_int8(const int8_t* w, int64_t n, int64_t k, uint8_t* packed, void* stream) {
  clear_error();
  DSV4_REQUIRE(n > 0 && n % 16 == 0, "pack_int8: n must be a positive multiple of 16, got %lld", (long long)n);
  DSV4_REQUIRE(k > 0 && k % 128 == 0, "pack_int8: k must be a positive multiple of 128, got %lld", (long long)k);
  DSV4_REQUIRE(n * k < (int64_t)1 << 31, "pack_int8: n*k must be below 2^31");
  DSV4_REQUIRE(w && packed, "pack_int8: null pointer");
  DSV4_REQUIRE(aligned(w, 16) && aligned(packed, 16), "pack_int8: buffers must be 16-byte aligned");
  return dsv4_launch_pack_int8(w, n, k, packed, static_cast<hipStream_t>(stream));
}

int dsv4moe_decode_e8m0(const uint8_t* codes, int64_t n, float* out, void* stream) {
  clear_error();
  DSV4_REQUIRE(n >= 0, "decode_e8m0: negative size");
  if (n == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(codes && out, "decode_e8m0: null pointer");
  DSV4_REQUIRE(aligned(out, 4), "decode_e8m0: out must be 4-byte aligned");
  return dsv4_launch_decode_e8m0(codes, n, out, static_cast<hipStream_t>(stream));
}

int dsv4moe_dequant_mxfp4(const uint8_t* packed, const float* scale, int64_t rows, int64_t k, float* out,
                          void* stream) {
  clear_error();
  DSV4_REQUIRE(rows >= 0, "dequant_mxfp4: negative row count");
  DSV4_REQUIRE(k > 0 && k % 32 == 0, "dequant_mxfp4: logical k must be a positive multiple of 32, got %lld",
               (long long)k);
  if (rows == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(packed && scale && out, "dequant_mxfp4: null pointer");
  DSV4_REQUIRE(aligned(packed, 16) && aligned(out, 16) && aligned(scale, 4),
               "dequant_mxfp4: packed and out must be 16-byte aligned, scale 4-byte aligned");
  return dsv4_launch_dequant_mxfp4(packed, scale, rows, k, out, static_cast<hipStream_t>(stream));
}

int dsv4moe_dequant_fp8_block(const void* w, int32_t w_dtype, const float* scale, int64_t rows, int64_t cols,
                              float* out, void* stream) {
  clear_error();
  DSV4_REQUIRE(w_dtype >= DSV4MOE_DTYPE_BF16 && w_dtype <= DSV4MOE_DTYPE_FP8_E4M3,
               "dequant_fp8_block: unknown w_dtype %d", (int)w_dtype);
  DSV4_REQUIRE(rows >= 0 && cols >= 0, "dequant_fp8_block: negative size");
  if (rows == 0 || cols == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(w && scale && out, "dequant_fp8_block: null pointer");
  const int elem = w_dtype == DSV4MOE_DTYPE_FP8_E4M3 ? 1 : (w_dtype == DSV4MOE_DTYPE_FP32 ? 4 : 2);
  DSV4_REQUIRE(aligned(w, elem) && aligned(scale, 4) && aligned(out, cols % 4 == 0 ? 16 : 4),
               "dequant_fp8_block: misaligned buffer (w to its element size, scale to 4 bytes, out to %d)",
               cols % 4 == 0 ? 16 : 4);
  return dsv4_launch_dequant_fp8_block(w, w_dtype, scale, rows, cols, out, static_cast<hipStream_t>(stream));
}

int32_t dsv4moe_w8a16_split_k(int64_t m, int64_t n, int64_t k) { return dsv4_w8a16_split_k(m, n, k); }

size_t dsv4moe_w8a16_workspace_bytes(int64_t m, int64_t n, int32_t split_k) {
  if (m < 0 || n <= 0 || split_k < 1) return 0;
  return dsv4_w8a16_workspace_bytes(m, n, split_k);
}

// Shared checks of the two W8A16 entry points (who = entry name).
static int validate_w8a16(const char* who, const uint16_t* a, int64_t m, int64_t n, int64_t k, const uint8_t* wq,
                          int32_t weight_layout, const void* scales, int32_t split_k, float* workspace,
                          size_t workspace_bytes, uint16_t* out) {
  DSV4_REQUIRE(m >= 0, "%s: m must be >= 0", who);
  DSV4_REQUIRE(weight_layout == DSV4MOE_WEIGHT_TILED || weight_layout == DSV4MOE_WEIGHT_ROWMAJOR,
               "%s: unknown weight_layout %d", who, weight_layout);
  DSV4_REQUIRE(n > 0 && n % 16 == 0, "%s: n must be a positive multiple of 16, got %lld", who, (long long)n);
  DSV4_REQUIRE(k > 0 && k % 128 == 0, "%s: k must be a positive multiple of 128, got %lld", who, (long long)k);
  DSV4_REQUIRE(split_k == 1 || split_k == 2 || split_k == 4 || split_k == 8 || split_k == 16,
               "%s: split_k must be one of 1, 2, 4, 8, 16, got %d", who, split_k);
  DSV4_REQUIRE(split_k <= k / 128, "%s: split_k=%d exceeds the K-block count %lld", who, split_k,
               (long long)(k / 128));
  DSV4_REQUIRE(m * k * 2 < (int64_t)1 << 31 && n * k < (int64_t)1 << 31,
               "%s: m*k*2 and n*k must be below 2^31", who);
  if (m == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(a && wq && scales && out, "%s: null pointer", who);
  DSV4_REQUIRE(aligned(a, 16) && aligned(wq, 16) && aligned(out, 8),
               "%s: a and wq must be 16-byte aligned, out 8-byte aligned", who);
  const size_t need = dsv4_w8a16_workspace_bytes(m, n, split_k);
  DSV4_REQUIRE(workspace_bytes >= need, "%s: workspace of %zu bytes is below the %zu needed", who,
               workspace_bytes, need);
  DSV4_REQUIRE(need == 0 || (workspace && aligned(workspace, 16)),
               "%s: split_k > 1 needs a 16-byte aligned workspace", who);
  return DSV4MOE_OK;
}

int dsv4moe_w8a16_linear(const uint16_t* a, int64_t m, int64_t n, int64_t k, const uint8_t* wq,
                         int32_t weight_layout, const uint16_t* ws, int32_t split_k, float* workspace,
                         size_t workspace_bytes, uint16_t* out, void* stream) {
  clear_error();
  int rc = validate_w8a16("w8a16_linear", a, m, n, k, wq, weight_layout, ws, split_k, workspace, workspace_bytes,
                          out);
  if (rc != DSV4MOE_OK || m == 0) return rc;
  DSV4_REQUIRE(aligned(ws, 8), "w8a16_linear: ws must be 8-byte aligned");
  return dsv4_launch_w8a16(a, m, n, k, wq, ws, nullptr, split_k, workspace, out,
                           static_cast<hipStream_t>(stream), 0, weight_layout == DSV4MOE_WEIGHT_ROWMAJOR);
}

int dsv4moe_w8a16_fp8_linear(const uint16_t* a, int64_t m, int64_t n, int64_t k, const uint8_t* wq,
                             int32_t weight_layout, const uint8_t* ws8, int32_t split_k, float* workspace,
                             size_t workspace_bytes, uint16_t* out, void* stream) {
  clear_error();
  int rc = validate_w8a16("w8a16_fp8_linear", a, m, n, k, wq, weight_layout, ws8, split_k, workspace,
                          workspace_bytes, out);
  if (rc != DSV4MOE_OK || m == 0) return rc;
  DSV4_REQUIRE(k <= 32768, "w8a16_fp8_linear: k must be <= 32768, got %lld", (long long)k);
  return dsv4_launch_w8a16(a, m, n, k, wq, nullptr, ws8, split_k, workspace, out,
                           static_cast<hipStream_t>(stream), 0, weight_layout == DSV4MOE_WEIGHT_ROWMAJOR);
}

int32_t dsv4moe_block_fp8_split_k(int64_t m, int64_t n, int64_t k) { return dsv4_block_fp8_split_k(m, n, k); }

size_t dsv4moe_block_fp8_workspace_bytes(int64_t m, int64_t n, int32_t split_k) {
  if (m <= 0 || n <= 0 || split_k <= 1) return 0;
  return (size_t)split_k * (size_t)m * (size_t)n * sizeof(float);
}

int dsv4moe_act_quant_block_fp8(const void* x, int32_t x_dtype, int64_t m, int64_t k, uint8_t* q, uint8_t* scale,
                                void* stream) {
  clear_error();
  DSV4_REQUIRE(x_dtype >= 0 && x_dtype <= 2, "act_quant_block_fp8: x_dtype must be 0 (bf16), 1 (fp16) or 2 (fp32)");
  DSV4_REQUIRE(m >= 0, "act_quant_block_fp8: m must be >= 0");
  DSV4_REQUIRE(k > 0 && k % 128 == 0, "act_quant_block_fp8: k must be a positive multiple of 128, got %lld",
               (long long)k);
  DSV4_REQUIRE(m * (k / 128) * 16 < (int64_t)1 << 38, "act_quant_block_fp8: m * k too large");
  if (m == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(x && q && scale, "act_quant_block_fp8: null pointer");
  DSV4_REQUIRE(aligned(x, 16) && aligned(q, 8), "act_quant_block_fp8: x 16-byte, q 8-byte aligned");
  return dsv4_launch_act_quant_block_fp8(x, x_dtype, m, k, q, scale, static_cast<hipStream_t>(stream));
}

int dsv4moe_block_fp8_gemm(const uint8_t* a, const uint8_t* a_scale, int64_t m, int64_t n, int64_t k,
                           const uint8_t* wq, int32_t weight_layout, const uint8_t* w_scale, int32_t split_k,
                           float* workspace, size_t workspace_bytes, uint16_t* out, void* stream) {
  clear_error();
  const char* who = "block_fp8_gemm";
  DSV4_REQUIRE(m >= 0, "%s: m must be >= 0", who);
  DSV4_REQUIRE(weight_layout == DSV4MOE_WEIGHT_TILED || weight_layout == DSV4MOE_WEIGHT_ROWMAJOR,
               "%s: unknown weight_layout %d", who, weight_layout);
  DSV4_REQUIRE(n > 0 && n % 16 == 0, "%s: n must be a positive multiple of 16, got %lld", who, (long long)n);
  DSV4_REQUIRE(k > 0 && k % 128 == 0 && k <= 32768, "%s: k must be a multiple of 128 in [128, 32768], got %lld", who,
               (long long)k);
  DSV4_REQUIRE(split_k == 1 || split_k == 2 || split_k == 4 || split_k == 8,
               "%s: split_k must be one of 1, 2, 4, 8, got %d", who, split_k);
  DSV4_REQUIRE(split_k <= k / 128, "%s: split_k=%d exceeds K-block count %lld", who, split_k, (long long)(k / 128));
  DSV4_REQUIRE(m * k < (int64_t)1 << 31 && n * k < (int64_t)1 << 31, "%s: m*k and n*k must be below 2^31", who);
  if (m == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(a && a_scale && wq && w_scale && out, "%s: null pointer", who);
  DSV4_REQUIRE(aligned(a, 16) && aligned(wq, 16) && aligned(out, 8) && aligned(a_scale, 4),
               "%s: a and wq must be 16-byte aligned, a_scale 4-byte, out 8-byte aligned", who);
  const size_t need = dsv4moe_block_fp8_workspace_bytes(m, n, split_k);
  DSV4_REQUIRE(workspace_bytes >= need, "%s: workspace of %zu bytes is below the %zu needed", who, workspace_bytes,
               need);
  DSV4_REQUIRE(need == 0 || (workspace && aligned(workspace, 16)), "%s: split_k > 1 needs a 16-byte aligned workspace",
               who);
  return dsv4_launch_block_fp8_gemm(a, a_scale, m, n, k, wq, w_scale, split_k, workspace, out,
                                    static_cast<hipStream_t>(stream), weight_layout == DSV4MOE_WEIGHT_ROWMAJOR);
}

size_t dsv4moe_shared_fp8_workspace_bytes(int64_t tokens, int32_t hidden, int32_t inter) {
  if (tokens < 0 || hidden <= 0 || inter <= 0 || hidden % 128 || inter % 128) return 0;
  return dsv4_shared_fp8_workspace_bytes(tokens, hidden, inter);
}

int dsv4moe_shared_fp8_add(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter, const uint8_t* w13q,
                           const uint8_t* w13s8, const uint8_t* w2q, const uint8_t* w2s8, float clamp_limit,
                           uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  DSV4_REQUIRE(tokens >= 0, "shared_fp8_add: tokens must be >= 0");
  DSV4_REQUIRE(hidden > 0 && hidden % 128 == 0 && hidden <= 32768 && inter > 0 && inter % 128 == 0 &&
                   inter <= 32768,
               "shared_fp8_add: hidden and inter must be multiples of 128 in [128, 32768], got %d, %d", hidden,
               inter);
  DSV4_REQUIRE(!(clamp_limit < 0.0f) && clamp_limit < 3.0e38f, "shared_fp8_add: clamp_limit must be >= 0 and finite");
  DSV4_REQUIRE(tokens * (int64_t)hidden * 2 < (int64_t)1 << 31 && tokens * (int64_t)inter * 4 < (int64_t)1 << 31 &&
                   (int64_t)hidden * inter * 2 < (int64_t)1 << 31,
               "shared_fp8_add: sizes must keep every operand below 2^31 bytes");
  if (tokens == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(x && w13q && w13s8 && w2q && w2s8 && out && workspace, "shared_fp8_add: null pointer");
  DSV4_REQUIRE(aligned(x, 16) && aligned(w13q, 16) && aligned(w2q, 16) && aligned(out, 8) && aligned(workspace, 256),
               "shared_fp8_add: x, w13q, w2q 16-byte aligned, out 8-byte, workspace 256-byte aligned");
  const size_t need = dsv4_shared_fp8_workspace_bytes(tokens, hidden, inter);
  DSV4_REQUIRE(workspace_bytes >= need, "shared_fp8_add: workspace of %zu bytes is below the %zu needed",
               workspace_bytes, need);
  return dsv4_launch_shared_fp8_add(x, tokens, hidden, inter, w13q, w13s8, w2q, w2s8, clamp_limit, out, workspace,
                                    static_cast<hipStream_t>(stream));
}

size_t dsv4moe_experts_w4a8_workspace_bytes(int64_t tokens, int32_t topk, int32_t hidden, int32_t inter,
                                            int32_t has_shared) {
  if (tokens < 0 || topk < 1 || hidden <= 0 || inter <= 0) return 0;
  return dsv4_experts_w4a8_workspace_bytes(tokens, topk, hidden, inter, has_shared ? 1 : 0);
}

int dsv4moe_act_quant_fp8(const uint16_t* x, int64_t rows, int32_t k, uint8_t* q, float* scale,
                          float* group_sums, void* stream) {
  clear_error();
  DSV4_REQUIRE(rows >= 0, "act_quant_fp8: rows must be >= 0");
  DSV4_REQUIRE(k > 0 && k % 512 == 0, "act_quant_fp8: k=%d must be a positive multiple of 512", k);
  DSV4_REQUIRE(rows * (int64_t)k * 2 < 0x7FFFFFFFLL, "act_quant_fp8: input exceeds 2 GiB");
  if (rows == 0) return DSV4MOE_OK;
  DSV4_REQUIRE(x && q && scale && group_sums, "act_quant_fp8: null pointer");
  DSV4_REQUIRE(aligned(x, 16) && aligned(q, 8) && aligned(scale, 4) && aligned(group_sums, 4),
               "act_quant_fp8: alignment (x 16 B, q 8 B)");
  return dsv4_launch_act_quant_fp8(x, rows, k, q, scale, group_sums, static_cast<hipStream_t>(stream));
}

int dsv4moe_experts_w4a8(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                         int32_t experts, int32_t topk, const uint8_t* w13q, const uint16_t* w13s,
                         const uint8_t* w2q, const uint16_t* w2s, int32_t has_shared,
                         const float* weights, const int32_t* sorted_token_ids, int64_t capacity,
                         const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                         int32_t block_size, float clamp_limit, uint16_t* out, void* workspace,
                         size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_experts(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s, capacity,
                            block_size, out, workspace, workspace_bytes, has_shared, "experts_w4a8", true);
  if (rc != DSV4MOE_OK || tokens == 0) return rc;
  DSV4_REQUIRE(weights && sorted_token_ids && expert_ids && num_tokens_post_padded,
               "experts_w4a8: null route/alignment pointer");
  DSV4_REQUIRE(!(clamp_limit < 0.0f) && clamp_limit < 3.0e38f, "experts_w4a8: clamp_limit must be >= 0 and finite");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dsv4host::prof_stamp(dsv4host::kStampBegin, s);
  dsv4host::prof_stamp(dsv4host::kStampRoute, s);
  dsv4host::prof_stamp(dsv4host::kStampAlign, s);
  return dsv4_launch_experts_w4a8(x, tokens, hidden, inter, experts, topk, w13q, w13s, w2q, w2s,
                                  has_shared ? 1 : 0, weights, sorted_token_ids, capacity, expert_ids,
                                  num_tokens_post_padded, block_size, clamp_limit, out, workspace, s);
}

}  // extern "C"
