// Device helpers shared by the gfx950 (CDNA4) kernels of libkoptim.
//
// Storage type for bf16 is the raw 16-bit pattern (uint16_t); arithmetic is
// fp32. Conversions:
//   bf16 -> f32 : exact, a 16-bit left shift of the pattern.
//   f32 -> bf16 : round-to-nearest-even via the hardware v_cvt_pk_bf16_f32
//                 (the compiler lowers a cast to __bf16 to it on gfx950).
// Wavefronts are 64 lanes; a DPP "row" is 16 consecutive lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ko {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16hi(uint32_t packed) {
  return __uint_as_float(packed & 0xffff0000u);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}
// Round an fp32 value to the nearest bf16 and return it widened back to fp32
// (the ".to(bf16).to(fp32)" step of a cast chain).
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}
// Both halves rounded by one v_cvt_pk_bf16_f32 (a vector conversion; two
// scalar casts give one conversion per value and a pack).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  const bf16x2 v = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
  return __builtin_bit_cast(uint32_t, v);
}

// fp32 += a.lo*b.lo + a.hi*b.hi with bf16 pairs (v_dot2c_f32_bf16). The bf16
// products are exact in fp32; only the sums round.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), c, false);
}

// The loads below read device (global) memory; they address it as such
// whatever the caller's pointer provenance, so they compile to global_load
// with a scalar base where possible, never to flat_load.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4 g_u32x4;

__device__ __forceinline__ uint4 ldg16(const void* p) {
  const u32x4 v = *(g_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
// Streaming load: the data is read exactly once, so mark it non-temporal.
__device__ __forceinline__ uint4 ldg16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load((g_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte load at device (agent) scope: two relaxed agent-scope 8-byte atomic
// loads (global_load ... sc1), for data that other workgroups of the same
// launch wrote with agent-scope stores.
__device__ __forceinline__ uint4 ldg16_coherent(const void* p) {
  unsigned long long* q = reinterpret_cast<unsigned long long*>(const_cast<void*>(p));
  const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// ---- cross-lane reductions -------------------------------------------------
// Within each 16-lane DPP row: every lane ends with the row total.
// row_ror:n has DPP control 0x120 + n.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_f<0x128>(v);  // row_ror:8
  v += dpp_f<0x124>(v);  // row_ror:4
  v += dpp_f<0x122>(v);  // row_ror:2
  v += dpp_f<0x121>(v);  // row_ror:1
  return v;
}
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_f<0x128>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  v = fmaxf(v, dpp_f<0x122>(v));
  v = fmaxf(v, dpp_f<0x121>(v));
  return v;
}
// Sums/maxima with the lane 16 or 32 places away (the xor-16 / xor-32
// butterflies), on the VALU with the gfx950 permlane swaps instead of an LDS
// permute. v_permlane16_swap(x, y) exchanges the odd rows of x with the even
// rows of y; with x = y = v the two results hold v's rows {0, 0, 2, 2} and
// {1, 1, 3, 3}, so their sum is v[i] + v[i ^ 16] in every lane.
// v_permlane32_swap does the same with the two 32-lane halves.
__device__ __forceinline__ float sum_xor16(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)p[0]) + __builtin_bit_cast(float, (unsigned)p[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)p[0]) + __builtin_bit_cast(float, (unsigned)p[1]);
}
__device__ __forceinline__ float max_xor16(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)p[0]), __builtin_bit_cast(float, (unsigned)p[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)p[0]), __builtin_bit_cast(float, (unsigned)p[1]));
}

// Full 64-lane reductions (every lane ends with the total; call with all lanes
// active).
__device__ __forceinline__ float wave_sum(float v) { return sum_xor32(sum_xor16(row_sum16(v))); }
__device__ __forceinline__ float wave_max(float v) { return max_xor32(max_xor16(row_max16(v))); }

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
// Inclusive prefix sum over the 64 lanes (call with all lanes active):
// Hillis-Steele inside each 16-lane row with DPP row_shr:1/2/4/8 (lanes whose
// source falls outside the row read 0), then the totals of the rows below.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += dpp_i<0x111>(v);
  v += dpp_i<0x112>(v);
  v += dpp_i<0x114>(v);
  v += dpp_i<0x118>(v);
  const int t0 = __builtin_amdgcn_readlane(v, 15);
  const int t1 = __builtin_amdgcn_readlane(v, 31);
  const int t2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane_id() >> 4;
  return v + (row >= 1 ? t0 : 0) + (row >= 2 ? t1 : 0) + (row >= 3 ? t2 : 0);
}

__device__ __forceinline__ int readlane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float readlane(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

}  // namespace ko

// Status codes shared by every C entry point: 0 = success, a positive value is
// a hipError_t from the launch, a negative value is an argument error found on
// the host before anything was launched.
#define KO_OK 0
#define KO_EINVAL (-22)
#define KO_ERANGE (-34)
#define KO_ENOTSUP (-95)

#define KO_LAUNCH_STATUS() ((int)hipGetLastError())
