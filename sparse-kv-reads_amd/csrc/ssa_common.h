// Shared device helpers for the clustered sparse decode-attention kernels (gfx950).
//
// Canonical arithmetic. Every decision the index makes (which cluster a key joins, which
// clusters a query reads, which side of a split a key lands on) is a comparison of fp32
// values. To make those decisions bit-reproducible on any other IEEE machine, the kernels
// in index.hip compute them in one fixed order with no implicit FMA contraction (that
// file is built with -ffp-contract=off):
//   cdot(a, b)   8 interleaved fma chains (chain j takes elements j, j+8, ...), combined
//                ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7))
//   unit(x)      x_i / max(sqrt(cdot(x, x)), 1e-12)
//   q8(u)        (int8) floor(u*127 + 0.5), multiply and add rounded separately
//   cexp(x)      e^x for x <= 0: Cody-Waite reduction by ln2, degree-7 Taylor polynomial
//                in Horner form with fma, scaled by 2^k through the exponent bits;
//                0 below -87 (so every nonzero result is a normal fp32 number)
//   tree sums    pairwise halving over a power-of-two slot count
//   seq sums     left to right, starting from +0
// division and sqrt are the correctly rounded IEEE operations (hipcc's default for HIP).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace ssa {

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) { return __bfloat162float(x); }
__device__ __forceinline__ float to_f32(__half x) { return __half2float(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float x) { return __float2bfloat16(x); }
template <> __device__ __forceinline__ __half from_f32<__half>(float x) { return __float2half(x); }

// Load element i of a row stored as dtype `dt` (runtime tag) and widen to fp32 exactly.
__device__ __forceinline__ float load_as_f32(const void* base, int dt, int64_t i) {
  if (dt == kBF16) return __bfloat162float(reinterpret_cast<const __hip_bfloat16*>(base)[i]);
  if (dt == kF16) return __half2float(reinterpret_cast<const __half*>(base)[i]);
  return reinterpret_cast<const float*>(base)[i];
}

// ---- canonical fp32 arithmetic ------------------------------------------------------

// Canonical dot product of two fp32 vectors of length d (d a multiple of 8) read through
// accessor functors; see the file comment for the order.
template <typename FA, typename FB>
__device__ __forceinline__ float cdot(FA a, FB b, int d) {
  float c0 = 0.f, c1 = 0.f, c2 = 0.f, c3 = 0.f, c4 = 0.f, c5 = 0.f, c6 = 0.f, c7 = 0.f;
  for (int i = 0; i < d; i += 8) {
    c0 = __builtin_fmaf(a(i + 0), b(i + 0), c0);
    c1 = __builtin_fmaf(a(i + 1), b(i + 1), c1);
    c2 = __builtin_fmaf(a(i + 2), b(i + 2), c2);
    c3 = __builtin_fmaf(a(i + 3), b(i + 3), c3);
    c4 = __builtin_fmaf(a(i + 4), b(i + 4), c4);
    c5 = __builtin_fmaf(a(i + 5), b(i + 5), c5);
    c6 = __builtin_fmaf(a(i + 6), b(i + 6), c6);
    c7 = __builtin_fmaf(a(i + 7), b(i + 7), c7);
  }
  return ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
}

__device__ __forceinline__ float cdot_ptr(const float* a, const float* b, int d) {
  return cdot([&](int i) { return a[i]; }, [&](int i) { return b[i]; }, d);
}

__device__ __forceinline__ float cnorm_ptr(const float* a, int d) { return sqrtf(cdot_ptr(a, a, d)); }

__device__ __forceinline__ int8_t q8(float u) {
  float t = u * 127.0f;
  t = t + 0.5f;
  return (int8_t)floorf(t);
}

// e^x for x <= 0 (see the file comment).
__device__ __forceinline__ float cexp(float x) {
  if (!(x >= -87.0f)) return 0.0f;                  // also maps -inf and NaN to 0
  const float kLog2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;          // ln2 rounded to 16 significant bits, so k*hi is exact
  const float kLn2Lo = 1.42860682030941723e-06f;
  float k = rintf(x * kLog2e);
  float r = __builtin_fmaf(-k, kLn2Hi, x);
  r = __builtin_fmaf(-k, kLn2Lo, r);
  float p = 1.98412698412698413e-04f;               // 1/5040
  p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);  // 1/720
  p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);  // 1/120
  p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);  // 1/24
  p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);  // 1/6
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ki = (int)k;                                  // in [-126, 0]: 2^ki is a normal number
  float scale = __int_as_float((ki + 127) << 23);
  return p * scale;
}

// ---- wavefront / workgroup reductions -----------------------------------------------

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// DPP forms of the wave reductions (row_shr within 16-lane rows, then row_bcast:15 and
// row_bcast:31 across rows): a lane whose source is out of its row or in a disabled row takes
// the `old` operand.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_i(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}
// Maximum over the 64 lanes, returned to every lane (read from lane 63, which holds it).
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<0x111, 0xF>(v, v));      // row_shr:1
  v = fmaxf(v, dpp_f<0x112, 0xF>(v, v));      // row_shr:2
  v = fmaxf(v, dpp_f<0x114, 0xF>(v, v));      // row_shr:4
  v = fmaxf(v, dpp_f<0x118, 0xF>(v, v));      // row_shr:8
  v = fmaxf(v, dpp_f<0x142, 0xA>(v, v));      // row_bcast:15 into rows 1 and 3
  v = fmaxf(v, dpp_f<0x143, 0xC>(v, v));      // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_incl_scan_dpp(int v) {
  v += dpp_i<0x111, 0xF>(0, v);
  v += dpp_i<0x112, 0xF>(0, v);
  v += dpp_i<0x114, 0xF>(0, v);
  v += dpp_i<0x118, 0xF>(0, v);
  v += dpp_i<0x142, 0xA>(0, v);
  v += dpp_i<0x143, 0xC>(0, v);
  return v;
}

// (score, index) argmax with the lowest index winning ties; index -1 never wins.
__device__ __forceinline__ void argmax_merge(float& s, int& i, float s2, int i2) {
  bool take = (i < 0) || (i2 >= 0 && (s2 > s || (s2 == s && i2 < i)));
  if (take) { s = s2; i = i2; }
}
__device__ __forceinline__ void wave_argmax(float& s, int& i) {
  for (int o = 32; o > 0; o >>= 1) {
    float s2 = __shfl_xor(s, o, 64);
    int i2 = __shfl_xor(i, o, 64);
    argmax_merge(s, i, s2, i2);
  }
}
// (score, index) argmin with the lowest index winning ties.
__device__ __forceinline__ void argmin_merge(float& s, int& i, float s2, int i2) {
  bool take = (i < 0) || (i2 >= 0 && (s2 < s || (s2 == s && i2 < i)));
  if (take) { s = s2; i = i2; }
}
__device__ __forceinline__ void wave_argmin(float& s, int& i) {
  for (int o = 32; o > 0; o >>= 1) {
    float s2 = __shfl_xor(s, o, 64);
    int i2 = __shfl_xor(i, o, 64);
    argmin_merge(s, i, s2, i2);
  }
}

// Inclusive prefix count of `pred` over the 64 lanes of the wave.
__device__ __forceinline__ int wave_prefix_count(bool pred, int lane) {
  uint64_t b = __ballot(pred);
  uint64_t below = (lane == 0) ? 0ull : (b & (~0ull >> (64 - lane)));
  return __popcll(below) + (pred ? 1 : 0);
}

constexpr float kNeg = -1.0e30f;   // finite "-inf" for running maxima: exp(kNeg - kNeg) = 1, never NaN

}  // namespace ssa
