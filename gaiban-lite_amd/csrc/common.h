// Shared device helpers and host error plumbing for the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace dsv4 {

// ---------------------------------------------------------------- vector types
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;   // MFMA 16x16x32 operand
typedef __attribute__((ext_vector_type(4))) float f32x4;     // MFMA 16x16 accumulator
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kGroup = 128;      // int4 quantisation group along K
constexpr int kTileBytes = 1024; // one packed tile: 16 rows x 128 K int4
constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 helpers
__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even float -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t float_to_bf16_bits(float v) {
  __bf16 b = (__bf16)v;
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return float_to_bf16_bits(lo) | (float_to_bf16_bits(hi) << 16);
}

// ---------------------------------------------------------------- int4 dequant
// A packed dword holds 8 offset-binary nibbles u = q + 8 of one row: nibble
// slot j (bits 4j..4j+3) is K offset 2j, slot 4+j (bits 16+4j..) is K offset
// 2j+1, j = 0..3.  OR-ing a nibble into the mantissa of bf16 128.0 (0x4300)
// gives exactly 128 + u = q + 136; the kernels remove the 136*sum(x) term with
// the per-group activation sums.
//
// `magic` is 0x43004300 held in a VGPR (dequant_magic()): with the mask as an
// SGPR constant each pair is then one v_and_or_b32 (gfx9 VOP3 encodings take
// no literals and one SGPR), instead of a v_and_b32 + v_or_b32 pair.
__device__ __forceinline__ uint32_t dequant_magic() {
  uint32_t m;
  asm("v_mov_b32 %0, 0x43004300" : "=v"(m));
  return m;
}
__device__ __forceinline__ bf16x8 dequant_biased(uint32_t w, uint32_t magic) {
  u32x4 p;
  p[0] = (w & 0x000F000Fu) | magic;
  p[1] = ((w >> 4) & 0x000F000Fu) | magic;
  p[2] = ((w >> 8) & 0x000F000Fu) | magic;
  p[3] = ((w >> 12) & 0x000F000Fu) | magic;
  return __builtin_bit_cast(bf16x8, p);
}
constexpr float kDequantBias = 136.0f;

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x4 load16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// LDS tiles of 16-row groups read with ds_read_b128 by lanes (row = lane % 16,
// part = f(lane / 16)) are swizzled so that every 8-lane and every 16-lane
// group of one read touches distinct 16-byte bank slots (measured with
// SQ_LDS_BANK_CONFLICT on gfx950; padding rows to 144 or 272 bytes does not
// achieve this):
//   256-byte rows: 16-byte part q of row r at q ^ (r & 15);
//   128-byte rows: part q of row r at q ^ swz128(r).
__device__ __forceinline__ int swz128(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// buffer_load ... lds of `size` bytes per lane (M0 = lds base, lane i writes
// base + i*size).  Wrapped in a plain function so that template kernels whose
// LDS arrays have template-dependent types still get their host-side launch
// stubs (a target builtin with dependent arguments fails host instantiation).
typedef __attribute__((address_space(3))) void* lds_void_ptr;
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, lds_void_ptr lds, uint32_t voffset,
                                          uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds, 16, voffset, soffset, 0, 0);
}

// The same copies issued as inline assembly.  The compiler does not see these
// as LDS writes, so it adds no vmcnt wait before ds_reads of *other* LDS
// buffers (it cannot tell the DMA destinations apart and would otherwise make
// every ds_read wait for the in-flight prefetch).  The caller must wait with
// lds_dma_wait_all() before the barrier that publishes the copied data.
// `lds` is the LDS byte address of lane 0's destination (M0); lane i writes
// lds + i*16 (dwordx4) or lds + i*4 (dword).
// (The asm bodies exist only in the device pass; the host pass of these
// device functions has no AMDGPU register constraints.)
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds, uint32_t voffset,
                                           uint32_t soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  // lds and soffset are wavefront-uniform; readfirstlane makes them scalar
  // for the compiler when it cannot prove it
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
#endif
}
__device__ __forceinline__ void lds_copy4(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds, uint32_t voffset,
                                          uint32_t soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
#endif
}
// Wait until at most N of this wavefront's vector-memory operations are
// outstanding (they complete in issue order).
template <int N>
__device__ __forceinline__ void lds_dma_wait_keep() {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
#endif
}
__device__ __forceinline__ void lds_dma_wait_all() {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
}
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)p;
}
// The LDS pointer of byte address `a` (a wavefront-uniform value stays scalar).
__device__ __forceinline__ lds_void_ptr lds_ptr(uint32_t a) { return (lds_void_ptr)(uintptr_t)a; }

// SiLU with the hardware reciprocal (v_rcp_f32, within an ulp) instead of
// the IEEE division: the prefill epilogues (32 per lane per work item, about
// 8 instructions less each; stage 1 1-1.5% faster).  The h it feeds is
// rounded to bf16; the decode kernels and the shared expert keep silu_f.
__device__ __forceinline__ float silu_rcp(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}
__device__ __forceinline__ float silu_f(float g) {
  return g / (1.0f + __expf(-g));
}

}  // namespace dsv4

// ------------------------------------------------------------------ host side
namespace dsv4host {
void set_error(const char* fmt, ...);
void clear_error();
int check_launch(const char* what);

// Optional per-kernel timing (dsv4moe_profile_begin/_end): stamp points of
// one layer call, recorded as HIP events on the launch stream.
enum Stamp {
  kStampBegin = 0,
  kStampRoute,
  kStampAlign,
  kStampRowSum,
  kStampStage1,
  kStampStage2,
  kStampCombine,
  kNumStamps
};
void prof_stamp(int stamp, hipStream_t stream);
}  // namespace dsv4host

#define DSV4_REQUIRE(cond, ...)            \
  do {                                      \
    if (!(cond)) {                          \
      ::dsv4host::set_error(__VA_ARGS__);   \
      return DSV4MOE_EINVAL;                \
    }                                       \
  } while (0)

#define DSV4_CHECK_LAUNCH(what)                          \
  do {                                                   \
    int _rc = ::dsv4host::check_launch(what);            \
    if (_rc != DSV4MOE_OK) return _rc;                   \
  } while (0)
