// Fused glue of the captured whole-model decode step (residual add + RMSNorm, per-head q/k
// RMSNorm + rotary embedding + KV-cache write, SwiGLU activation). A Qwen3 decode step is ~60
// element-wise launches per layer as separate tensor ops, and at batch 1-2 every launch costs a
// few microseconds of dependent-kernel latency whatever its size; these three kernels replace
// all of them, leaving per layer four GEMMs, three of these and the attention step.
//
// Each kernel reproduces the tensor-op sequence it replaces, including the rounding to the
// storage dtype between ops: RMSNorm is (x * rsqrt(mean(x^2) + eps)) * w in fp32 rounded once;
// the rotary embedding rotates pairs (x_i, x_{i+d/2}) of the normalised, rounded head by
// (cos, sin) of the position, x1*cos - x2*sin and x2*cos + x1*sin; SwiGLU is
// round(silu(g)) * up, each product rounded. Only the order of the mean's sum differs.
#include "ssa_common.h"
#include "../../include/ssa_hip.h"

#include <algorithm>

namespace ssa {
namespace {

template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }
template <typename T> __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = from_f32<T>(v); }
template <typename T> __device__ __forceinline__ float rnd(float v) { return to_f32(from_f32<T>(v)); }

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// h += delta (when given), x = rmsnorm(h) * w; one workgroup of 256 threads per row
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_add_kernel(T* __restrict__ h, const T* __restrict__ delta,
                                                          const T* __restrict__ w, T* __restrict__ x, int D,
                                                          float eps) {
  __shared__ float red[4];
  const int64_t row = (int64_t)blockIdx.x * D;
  const int tid = threadIdx.x;
  float ss = 0.f;
  for (int i = tid; i < D; i += 256) {
    float v = ld(h, row + i);
    if (delta) {
      v = rnd<T>(v + ld(delta, row + i));
      st(h, row + i, v);
    }
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float r = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  for (int i = tid; i < D; i += 256) {
    const float v = ld(h, row + i);
    st(x, row + i, (v * r) * ld(w, i));
  }
}

// qkv [B, (H + 2 Hk) d]: head slot j of sequence b is a query head (j < H), a key head
// (j < H + Hk) or a value head. Queries and keys: RMSNorm over d with their weight, then the
// rotary embedding at *pos; queries go to q_out [B H, d], keys to the cache at *pos, values are
// copied to the cache. One wave per (head slot, sequence); lane t owns pairs (t + 64 u, .. + d/2).
template <typename T>
__global__ __launch_bounds__(64) void qk_norm_rope_cache_kernel(const T* __restrict__ qkv, const T* __restrict__ qw,
                                                                const T* __restrict__ kw, const float* __restrict__ cos_t,
                                                                const float* __restrict__ sin_t,
                                                                const int64_t* __restrict__ pos_p, T* __restrict__ q_out,
                                                                T* __restrict__ kc, T* __restrict__ vc, int64_t s_cb,
                                                                int64_t s_ch, int64_t s_cl, int H, int Hk, int d,
                                                                float eps) {
  constexpr int kMaxPairs = 2;                      // d <= 256
  const int j = blockIdx.x, b = blockIdx.y, lane = threadIdx.x, half = d / 2;
  const int64_t pos = *pos_p;
  const T* src = qkv + ((int64_t)b * (H + 2 * Hk) + j) * d;
  if (j >= H + Hk) {                                // value head: copy into the cache
    T* dst = vc + b * s_cb + (int64_t)(j - H - Hk) * s_ch + pos * s_cl;
    for (int i = lane; i < d; i += 64) dst[i] = src[i];
    return;
  }
  const bool is_q = j < H;
  const T* w = is_q ? qw : kw;
  float x1[kMaxPairs], x2[kMaxPairs];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxPairs; ++u) {
    const int i = lane + 64 * u;
    x1[u] = i < half ? ld(src, i) : 0.f;
    x2[u] = i < half ? ld(src, i + half) : 0.f;
    ss += x1[u] * x1[u] + x2[u] * x2[u];
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)d + eps);
  T* dst = is_q ? q_out + ((int64_t)b * H + j) * d : kc + b * s_cb + (int64_t)(j - H) * s_ch + pos * s_cl;
#pragma unroll
  for (int u = 0; u < kMaxPairs; ++u) {
    const int i = lane + 64 * u;
    if (i >= half) continue;
    const float a = rnd<T>((x1[u] * r) * ld(w, i));
    const float c = rnd<T>((x2[u] * r) * ld(w, i + half));
    const float co = cos_t[pos * half + i], si = sin_t[pos * half + i];
    st(dst, i, a * co - c * si);
    st(dst, i + half, c * co + a * si);
  }
}

// out [rows, I] = round(silu(gate)) * up, gu [rows, 2 I] holding gate then up
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T* __restrict__ gu, T* __restrict__ out, int64_t rows,
                                                       int I) {
  const int64_t n = rows * I;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / I, i = e % I;
    const float g = ld(gu, r * 2 * I + i), u = ld(gu, r * 2 * I + I + i);
    const float s = rnd<T>(g / (1.0f + expf(-g)));
    st(out, e, s * u);
  }
}

// y [M, N] = x [M, K] . W[N, K]^T for a handful of rows M (decode batch): a weight-streaming
// kernel. Wave w of workgroup b owns output columns n0 = (4 b + w) R .. n0 + R; every lane
// reads 16 bytes (8 elements) of each of the R weight rows per k-step of 512 elements and dots
// them with the matching 8 elements of the M rows of x (fp32 accumulation), then the 64 lane
// partials are summed by a shuffle tree and rounded once to the output dtype.
template <typename T, int MM, int R>
__global__ __launch_bounds__(256) void skinny_kernel(const T* __restrict__ x, const T* __restrict__ W,
                                                     T* __restrict__ y, int M, int N, int K) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * R;
  if (n0 >= N) return;
  float acc[R][MM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;
  auto widen = [](const uint4& q, float (&f)[8]) {
    const T* h = reinterpret_cast<const T*>(&q);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = to_f32(h[e]);
  };
#pragma unroll 2
  for (int k0 = 8 * lane; k0 < K; k0 += 512) {
    uint4 wq[R], xq[MM];
#pragma unroll
    for (int r = 0; r < R; ++r)
      wq[r] = n0 + r < N ? *reinterpret_cast<const uint4*>(W + (int64_t)(n0 + r) * K + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int m = 0; m < MM; ++m)
      xq[m] = m < M ? *reinterpret_cast<const uint4*>(x + (int64_t)m * K + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float xf[8];
      widen(xq[m], xf);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float wf[8];
        widen(wq[r], wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][m] = __builtin_fmaf(wf[e], xf[e], acc[r][m]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float v = acc[r][m];
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      acc[r][m] = v;
    }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MM; ++m)
        if (m < M && n0 + r < N) st(y, (int64_t)m * N + n0 + r, acc[r][m]);
  }
}

template <typename F>
int by_dtype(int dtype, F f) {
  switch (dtype) {
    case kF32: return f(float{});
    case kBF16: return f(__hip_bfloat16{});
    case kF16: return f(__half{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace
}  // namespace ssa

using namespace ssa;

extern "C" int ssa_rmsnorm_add(void* h, const void* delta, const void* w, void* x, int32_t rows, int32_t D, float eps,
                               int32_t dtype, void* stream) {
  if (!h || !w || !x || rows < 0 || D < 1) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  return by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(rmsnorm_add_kernel<T>, dim3(rows), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<T*>(h), static_cast<const T*>(delta), static_cast<const T*>(w), static_cast<T*>(x),
                       D, eps);
    return (int)hipGetLastError();
  });
}

extern "C" int ssa_qk_norm_rope_cache(const void* qkv, const void* q_w, const void* k_w, const float* cos_t,
                                      const float* sin_t, const int64_t* pos, void* q_out, void* k_cache,
                                      void* v_cache, int64_t s_cb, int64_t s_ch, int64_t s_cl, int32_t B, int32_t H,
                                      int32_t Hk, int32_t d, float eps, int32_t dtype, void* stream) {
  if (!qkv || !q_w || !k_w || !cos_t || !sin_t || !pos || !q_out || !k_cache || !v_cache) return hipErrorInvalidValue;
  if (B < 1 || H < 1 || Hk < 1 || H % Hk || d < 2 || d > 256 || d % 2) return hipErrorInvalidValue;
  return by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(qk_norm_rope_cache_kernel<T>, dim3(H + 2 * Hk, B), dim3(64), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const T*>(qkv), static_cast<const T*>(q_w),
                       static_cast<const T*>(k_w), cos_t, sin_t, pos, static_cast<T*>(q_out), static_cast<T*>(k_cache),
                       static_cast<T*>(v_cache), s_cb, s_ch, s_cl, H, Hk, d, eps);
    return (int)hipGetLastError();
  });
}

extern "C" int ssa_silu_mul(const void* gu, void* out, int32_t rows, int32_t I, int32_t dtype, void* stream) {
  if (!gu || !out || rows < 0 || I < 1) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  const int64_t n = (int64_t)rows * I;
  const int grid = (int)std::min<int64_t>((n + 255) / 256, 4096);
  return by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(silu_mul_kernel<T>, dim3(grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const T*>(gu), static_cast<T*>(out), (int64_t)rows, I);
    return (int)hipGetLastError();
  });
}

extern "C" int ssa_linear_skinny(const void* x, const void* W, void* y, int32_t M, int32_t N, int32_t K, int32_t dtype,
                                 void* stream) {
  if (!x || !W || !y || M < 1 || M > 8 || N < 1 || K < 8 || K % 8) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W)) & 15) return hipErrorInvalidValue;
  if (dtype != kBF16 && dtype != kF16) return hipErrorInvalidValue;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto go = [&](auto tag, auto mm, auto rr) {
    using T = decltype(tag);
    constexpr int MM = decltype(mm)::value, R = decltype(rr)::value;
    const int grid = (N + 4 * R - 1) / (4 * R);
    hipLaunchKernelGGL((skinny_kernel<T, MM, R>), dim3(grid), dim3(256), 0, st, static_cast<const T*>(x),
                       static_cast<const T*>(W), static_cast<T*>(y), M, N, K);
    return (int)hipGetLastError();
  };
  // rows per wave: 4 when the columns give at least 1024 waves, else 1
  auto pick = [&](auto tag, auto mm) {
    if (N >= 4096) return go(tag, mm, std::integral_constant<int, 4>{});
    return go(tag, mm, std::integral_constant<int, 1>{});
  };
  auto bym = [&](auto tag) {
    if (M <= 1) return pick(tag, std::integral_constant<int, 1>{});
    if (M <= 2) return pick(tag, std::integral_constant<int, 2>{});
    if (M <= 4) return pick(tag, std::integral_constant<int, 4>{});
    return pick(tag, std::integral_constant<int, 8>{});
  };
  return dtype == kBF16 ? bym(__hip_bfloat16{}) : bym(__half{});
}

// out [M] int64 = argmax over each row of x [M, N] (first index of the maximum), one workgroup of
// 1024 threads per row.
template <typename T>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const T* __restrict__ x, int64_t* __restrict__ out, int N) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const int64_t row = (int64_t)blockIdx.x * N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -INFINITY;
  int bi = N;
  for (int i = tid; i < N; i += 1024) {
    const float v = ld(x, row + i);
    if (v > bv || (v == bv && i < bi) || (v != v && bi == N)) { bv = v; bi = i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    if (v2 > bv || (v2 == bv && i2 < bi)) { bv = v2; bi = i2; }
  }
  if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 16; ++w)
      if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) { bv = sv[w]; bi = si[w]; }
    out[blockIdx.x] = bi < N ? bi : 0;
  }
}

extern "C" int ssa_argmax_rows(const void* x, int64_t* out, int32_t M, int32_t N, int32_t dtype, void* stream) {
  if (!x || !out || M < 1 || N < 1) return hipErrorInvalidValue;
  return by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(argmax_rows_kernel<T>, dim3(M), dim3(1024), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const T*>(x), out, N);
    return (int)hipGetLastError();
  });
}
