// Shared helpers for the gfx950 paged KV-cache kernels: status/error plumbing,
// bf16 bit tricks and wave64 DPP reductions.  Only CDNA4 (gfx950) is targeted.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "kvc.h"

namespace kvc {

// ---------------------------------------------------------------- errors ----
// Records the reason for a failed call; read back through kvc_last_error().
int set_error(int status, const std::string& msg);
inline int ok() { return KVC_OK; }

#define KVC_REQUIRE(cond, status, msg)                                      \
  do {                                                                      \
    if (!(cond)) return ::kvc::set_error((status), std::string(__func__) +  \
                                         ": " + (msg));                     \
  } while (0)

#define KVC_HIP_CHECK(expr)                                                  \
  do {                                                                       \
    hipError_t e_ = (expr);                                                  \
    if (e_ != hipSuccess)                                                    \
      return ::kvc::set_error(KVC_ERR_HIP, std::string(__func__) + ": " +    \
                              #expr + " -> " + hipGetErrorString(e_));       \
  } while (0)

#define KVC_LAUNCH_CHECK() KVC_HIP_CHECK(hipGetLastError())

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// ------------------------------------------------------------------ bf16 ----
// A 32-bit word holding two bf16 values (element 0 in the low half).
__device__ __forceinline__ float bf16lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16hi(uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}

// float -> bf16 bits, IEEE round-to-nearest-even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte loads/stores with the non-temporal hint (the `nt` bit): KV bytes
// are streamed once per kernel, and keeping them out of the L2's normal
// allocation is worth 10-50% of HBM throughput on gfx950 for the append,
// the gather and decode (measured).
__device__ __forceinline__ uint4 load_stream(const void* p) {
  return __builtin_bit_cast(uint4,
                            __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}
__device__ __forceinline__ void store_stream(void* p, uint4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(p));
}

// a.x*b.x + a.y*b.y + c with bf16 pairs and an fp32 accumulator
// (v_dot2c_f32_bf16; the bf16 products are exact in fp32).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

// ------------------------------------------------------------------- DPP ----
// DPP control words (CDNA ISA): quad_perm, row rotate right.
constexpr int kDppQuadSwap1 = 0xB1;  // quad_perm:[1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;  // quad_perm:[2,3,0,1]
constexpr int kDppRowRor4 = 0x124;   // row_ror:4
constexpr int kDppRowRor8 = 0x128;   // row_ror:8

template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), Ctrl,
                                         0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppQuadSwap1>(v);
  v += dpp<kDppQuadSwap2>(v);
  v += dpp<kDppRowRor4>(v);
  v += dpp<kDppRowRor8>(v);
  return v;
}

// Max over the 16 lanes of a DPP row; every lane of the row gets it.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp<kDppRowRor4>(v));
  v = fmaxf(v, dpp<kDppRowRor8>(v));
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float fast_log2(float x) {
  return __builtin_amdgcn_logf(x);
}

// Large negative finite stand-in for -inf in running maxima, so that
// exp2(m_old - m_new) never evaluates (-inf) - (-inf).
constexpr float kNegBig = -1.0e30f;

inline int cdiv(int64_t a, int64_t b) { return int((a + b - 1) / b); }

}  // namespace kvc
