// Shared device helpers for the gfx950 kernels of the GRPO rollout-and-loss path.
//
// Storage convention: every bf16 tensor crosses the C ABI as raw 16-bit words
// (uint16_t), and every kernel converts explicitly.  bf16 -> fp32 is exact
// (a shift into the high half of the word); fp32 -> bf16 uses the gfx950
// hardware round-to-nearest-even conversion (v_cvt_pk_bf16_f32), which is the
// rounding torch's `.to(torch.bfloat16)` applies.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/qwen3mi.h"

namespace qmi {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Finite stand-in for -inf in running maxima: keeps exp2(m_old - m_new)
// finite (0 or 1) when a row has not yet seen a valid score.
constexpr float kNegBig = -1.0e30f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// Two-element bf16 dot product with fp32 accumulation (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- cross-lane reductions (wave64) -------------------------------------
// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowRor8 = 0x128;     // row_ror:8: lane i of a 16-lane row reads lane i ^ 8

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_amdgcn_update_dpp(0.0f, x, CTRL, 0xf, 0xf, false);
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<kDppQuadXor1>(x);
  x += dpp_f32<kDppQuadXor2>(x);
  x += dpp_f32<kDppRowHalfMirror>(x);
  x += dpp_f32<kDppRowMirror>(x);
  return x;
}

__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f32<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_f32<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_f32<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp_f32<kDppRowMirror>(x));
  return x;
}

__device__ __forceinline__ float shfl_xor_f32(float x, int mask) {
  return __shfl_xor(x, mask, 64);
}

// Lane pairs {l, l ^ 16} and {l, l ^ 32} through the gfx950 VALU lane swaps
// (v_permlane16_swap / v_permlane32_swap, no LDS round trip): every lane gets
// the pair's two values as (lower lane's, upper lane's), so a commutative
// combine of the two gives bit-identical results on both lanes.
struct LanePair {
  float lo, hi;
};

__device__ __forceinline__ LanePair lane_pair16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}

__device__ __forceinline__ LanePair lane_pair32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one per DPP row).
__device__ __forceinline__ float rows4_max(float x) {
  LanePair p = lane_pair16(x);
  x = fmaxf(p.lo, p.hi);
  p = lane_pair32(x);
  return fmaxf(p.lo, p.hi);
}

__device__ __forceinline__ float rows4_sum(float x) {
  LanePair p = lane_pair16(x);
  x = p.lo + p.hi;
  p = lane_pair32(x);
  return p.lo + p.hi;
}

__device__ __forceinline__ float wave_sum(float x) { return rows4_sum(row16_sum(x)); }

__device__ __forceinline__ float wave_max(float x) { return rows4_max(row16_max(x)); }

// Merge two (max, sum-of-exp2) pairs kept in the log2 domain.
__device__ __forceinline__ void lse2_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  s = s * fast_exp2(m - mn) + s2 * fast_exp2(m2 - mn);
  m = mn;
}

__device__ __forceinline__ uint4 load_u4(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

// Streaming (non-temporal) 16-byte load for data read exactly once.
__device__ __forceinline__ uint4 load_u4_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers:
// as easy as 1, 2, 3", SC 2011): counter c, key (k0, k1).
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
    const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
    c = make_uint4(hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0);
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// Compute units of the current device (cached per device; 256 if the query
// fails).
inline int device_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Calls f(std::integral_constant<int, i>) for i = I .. N-1.
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

}  // namespace qmi

// Launch helper: returns the launch status as the C-ABI error code.
#define QMI_RETURN_LAUNCH_STATUS()                       \
  do {                                                   \
    hipError_t _e = hipGetLastError();                   \
    return _e == hipSuccess ? QMI_OK : (int)_e;          \
  } while (0)
