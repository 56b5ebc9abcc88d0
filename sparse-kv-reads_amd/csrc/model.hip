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

// An fp32 value as computed, for the rounding to the storage dtype that follows: without it the
// compiler may fold the last multiply into the conversion (v_fma_mix* rounds the exact product
// once, straight to fp16), which differs from fp32-then-fp16 at fp16 midpoints, so that the same
// expression could round differently in two kernels.
__device__ __forceinline__ float f32_done(float v) {
  asm volatile("" : "+v"(v));
  return v;
}
template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }
template <typename T> __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = from_f32<T>(f32_done(v)); }
template <typename T> __device__ __forceinline__ float rnd(float v) { return to_f32(from_f32<T>(f32_done(v))); }

// The sums of squares of the RMSNorms load each thread's elements in rounds of kRmsU before
// adding them, in the order of the elements.
constexpr int kRmsU = 8;

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
  for (int i0 = tid; i0 < D; i0 += 256 * kRmsU) {
    float v[kRmsU], dv[kRmsU];
#pragma unroll
    for (int u = 0; u < kRmsU; ++u) {
      const int i = min(i0 + 256 * u, D - 1);     // in bounds for every lane: the loads issue together
      v[u] = ld(h, row + i);
      dv[u] = delta ? ld(delta, row + i) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kRmsU; ++u) {
      const int i = i0 + 256 * u;
      if (i < D) {
        if (delta) {
          v[u] = rnd<T>(v[u] + dv[u]);
          st(h, row + i, v[u]);
        }
        ss += v[u] * v[u];
      }
    }
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

// One query or key head of d entries (entry i read as load(i)): RMSNorm over d with weight w,
// then the rotary embedding at pos, stored to dst. One wave; lane t owns pairs (t + 64 u,
// t + 64 u + d/2).
template <typename T, typename F>
__device__ __forceinline__ void norm_rope_store(F load, const T* __restrict__ w, const float* __restrict__ cos_t,
                                                const float* __restrict__ sin_t, int64_t pos, T* __restrict__ dst,
                                                int d, float eps, int lane) {
  constexpr int kMaxPairs = 2;                      // d <= 256
  const int half = d / 2;
  // every input is loaded before the first use, in one round of loads
  float x1[kMaxPairs], x2[kMaxPairs], w1[kMaxPairs], w2[kMaxPairs], co[kMaxPairs], si[kMaxPairs];
#pragma unroll
  for (int u = 0; u < kMaxPairs; ++u) {
    const int i = lane + 64 * u;
    const bool ok = i < half;
    x1[u] = ok ? load(i) : 0.f;
    x2[u] = ok ? load(i + half) : 0.f;
    w1[u] = ok ? ld(w, i) : 0.f;
    w2[u] = ok ? ld(w, i + half) : 0.f;
    co[u] = ok ? cos_t[pos * half + i] : 0.f;
    si[u] = ok ? sin_t[pos * half + i] : 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxPairs; ++u) ss += x1[u] * x1[u] + x2[u] * x2[u];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)d + eps);
#pragma unroll
  for (int u = 0; u < kMaxPairs; ++u) {
    const int i = lane + 64 * u;
    if (i >= half) continue;
    const float a = rnd<T>((x1[u] * r) * w1[u]);
    const float c = rnd<T>((x2[u] * r) * w2[u]);
    st(dst, i, a * co[u] - c * si[u]);
    st(dst, i + half, c * co[u] + a * si[u]);
  }
}

// qkv [B, (H + 2 Hk) d]: head slot j of sequence b is a query head (j < H), a key head
// (j < H + Hk) or a value head. Queries and keys: RMSNorm over d with their weight, then the
// rotary embedding at *pos; queries go to q_out [B H, d], keys to the cache at *pos, values are
// copied to the cache. One wave per (head slot, sequence).
template <typename T>
__global__ __launch_bounds__(64) void qk_norm_rope_cache_kernel(const T* __restrict__ qkv, const T* __restrict__ qw,
                                                                const T* __restrict__ kw, const float* __restrict__ cos_t,
                                                                const float* __restrict__ sin_t,
                                                                const int64_t* __restrict__ pos_p, T* __restrict__ q_out,
                                                                T* __restrict__ kc, T* __restrict__ vc, int64_t s_cb,
                                                                int64_t s_ch, int64_t s_cl, int H, int Hk, int d,
                                                                float eps) {
  const int j = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int64_t pos = *pos_p;
  const T* src = qkv + ((int64_t)b * (H + 2 * Hk) + j) * d;
  if (j >= H + Hk) {                                // value head: copy into the cache
    T* dst = vc + b * s_cb + (int64_t)(j - H - Hk) * s_ch + pos * s_cl;
    for (int i = lane; i < d; i += 64) dst[i] = src[i];
    return;
  }
  const bool is_q = j < H;
  T* dst = is_q ? q_out + ((int64_t)b * H + j) * d : kc + b * s_cb + (int64_t)(j - H) * s_ch + pos * s_cl;
  norm_rope_store<T>([&](int i) { return ld(src, i); }, is_q ? qw : kw, cos_t, sin_t, pos, dst, d, eps, lane);
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

// The weight-streaming products of the decode step (a handful of rows M, the decode batch).
// A wave owns R weight rows; every lane reads 16 bytes (8 elements) of each of them per k-step
// of 512 elements and dots them with the matching 8 elements of the M rows of x in fp32, then the
// 64 lane partials are summed by a shuffle tree. Every kernel below uses these two functions, so
// an output column has the same bits whichever kernel computes it.
// row(r): the weight row of slot r, or -1 for none (its sums are left undefined).
// NORM: x holds the rows h and the dots take x = round((h * rs[m]) * nw) (nw: the RMSNorm weight),
// the bits of ssa_rmsnorm_add's output, computed element by element as the chunks are read.
// pro(): called by every thread once the first round of loads is issued (the NORM path
// computes rs there, so that its reads are in flight together with the weights').
template <typename T, int MM, int R, bool NORM, typename RowFn, typename Pro>
__device__ __forceinline__ void skinny_dots(const T* __restrict__ x, const T* __restrict__ W, int M, int K, int lane,
                                            RowFn row, float (&acc)[R][MM], const T* __restrict__ nw,
                                            const float* rs, Pro pro) {
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;
  auto widen = [](const uint4& q, float (&f)[8]) {
    const T* h = reinterpret_cast<const T*>(&q);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = to_f32(h[e]);
  };
  // Every load is unconditional, at an in-bounds address (slots without a row read row 0, rows
  // m >= M read row M - 1, lanes past K read the last chunk), so that a round of loads issues
  // at once; sums of such slots, rows and lanes are never stored or added.
  int64_t rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rows[r] = max(row(r), (int64_t)0);
  // Chunks of 8 columns at k and k + 512 per round, both loaded before either is used. The
  // unrolling is written out: the rounding barrier of the NORM path is an asm statement, which
  // the compiler treats as convergent and does not unroll over a runtime trip count.
  struct Chunk {
    uint4 w[R], x[MM], n;
  };
  auto load = [&](Chunk& c, int k0) {
    k0 = min(k0, K - 8);
#pragma unroll
    for (int r = 0; r < R; ++r) c.w[r] = *reinterpret_cast<const uint4*>(W + rows[r] * K + k0);
#pragma unroll
    for (int m = 0; m < MM; ++m) c.x[m] = *reinterpret_cast<const uint4*>(x + (int64_t)min(m, M - 1) * K + k0);
    if constexpr (NORM) c.n = *reinterpret_cast<const uint4*>(nw + k0);
  };
  auto dots = [&](const Chunk& c) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float xf[8];
      widen(c.x[m], xf);
      if constexpr (NORM) {
        float nf[8];
        widen(c.n, nf);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = rnd<T>((xf[e] * rs[m]) * nf[e]);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float wf[8];
        widen(c.w[r], wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][m] = __builtin_fmaf(wf[e], xf[e], acc[r][m]);
      }
    }
  };
  Chunk c0, c1;
  load(c0, 8 * lane);
  load(c1, 8 * lane + 512);
  __builtin_amdgcn_sched_barrier(0);        // the weights' loads issue first
  pro();
  for (int kb = 0;;) {                      // kb: the round's first column, the same in every lane
    const int k0 = kb + 8 * lane;
    if (k0 < K) dots(c0);
    if (k0 + 512 < K) dots(c1);
    kb += 1024;
    if (kb >= K) break;
    load(c0, kb + 8 * lane);
    load(c1, kb + 8 * lane + 512);
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float v = acc[r][m];
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      acc[r][m] = v;
    }
}

// 1 / sqrt(mean(h_m^2) + eps) of rows m < M of h [M, D], every thread of the workgroup taking
// part, in ssa_rmsnorm_add's order: thread t sums elements t, t + 256, ... left to right, then a
// wave tree, then the four waves in order. load() issues the loads of the first round (kRmsU
// elements of each row per thread), run() sums them and finishes.
template <typename T, int MM>
struct RowNorms {
  float v[MM][kRmsU];
  __device__ __forceinline__ void load(const T* __restrict__ h, int M, int D, int i0) {
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int u = 0; u < kRmsU; ++u) {
        // in-bounds addresses for every lane, so that the loads issue together
        const int i = min(i0 + 256 * u, D - 1);
        v[m][u] = ld(h, (int64_t)min(m, M - 1) * D + i);
      }
  }
  __device__ __forceinline__ void run(const T* __restrict__ h, int M, int D, float eps, float (&rs)[MM]) {
    __shared__ float red[MM][4];
    const int tid = threadIdx.x;
    float ss[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) ss[m] = 0.f;
    // b: the round's first element, the same in every thread. Every loaded value is used, so
    // that no load is moved behind a branch: rows m >= M sum copies of row M - 1 (not used), and
    // elements past D add +0, which leaves a sum of squares unchanged.
    auto add = [&](int b) {
#pragma unroll
      for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int u = 0; u < kRmsU; ++u) ss[m] += b + tid + 256 * u < D ? v[m][u] * v[m][u] : 0.f;
    };
    // the first round outside the loop: waits inside a loop would be sized for the loop's own
    // loads and so also cover every load still in flight when it is entered
    add(0);
    for (int b = 256 * kRmsU; b < D; b += 256 * kRmsU) {
      load(h, M, D, b + tid);
      add(b);
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      if (m < M) {
        const float t = wave_sum(ss[m]);
        if ((tid & 63) == 0) red[m][tid >> 6] = t;
      }
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MM; ++m)
      rs[m] = m < M ? 1.0f / sqrtf((red[m][0] + red[m][1] + red[m][2] + red[m][3]) / (float)D + eps) : 0.f;
  }
};

// y [M, N] = x [M, K] . W[N, K]^T, rounded once to the output dtype. Wave w of workgroup b owns
// output columns n0 = (4 b + w) R .. n0 + R.
// NORM: x holds rows h and the product is taken of rmsnorm(h) * nw (ssa_rmsnorm_add's bits).
// RES: y is the residual stream, y += round(product), rounded as ssa_rmsnorm_add's add.
template <typename T, int MM, int R, bool NORM = false, bool RES = false>
__global__ __launch_bounds__(256) void skinny_kernel(const T* __restrict__ x, const T* __restrict__ W,
                                                     T* __restrict__ y, int M, int N, int K,
                                                     const T* __restrict__ nw = nullptr, float eps = 0.f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * R;
  if (!NORM && n0 >= N) return;     // with NORM every wave takes part in the row norms
  float rs[MM], acc[R][MM];
  RowNorms<T, MM> norms;
  skinny_dots<T, MM, R, NORM>(
      x, W, M, K, lane, [&](int r) { return n0 + r < N ? (int64_t)(n0 + r) : (int64_t)-1; }, acc, nw, rs,
      [&] {
        if constexpr (NORM) {
          norms.load(x, M, K, threadIdx.x);
          norms.run(x, M, K, eps, rs);
        }
      });
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MM; ++m)
        if (m < M && n0 + r < N) {
          const int64_t o = (int64_t)m * N + n0 + r;
          if constexpr (RES) st(y, o, ld(y, o) + rnd<T>(acc[r][m]));
          else st(y, o, acc[r][m]);
        }
  }
}

// act [M, I] = round(silu(g)) * u with (g, u) = x . W[2 I, K]^T rounded to the dtype (gate rows
// first, then up rows): the gate/up projection with the SwiGLU activation as its epilogue, equal
// bit for bit to ssa_linear_skinny followed by ssa_silu_mul. Wave w of workgroup b owns
// activation columns c0 = 2 (4 b + w), c0 + 1: weight rows c0, c0 + 1, I + c0, I + c0 + 1.
// NORM: x holds rows h and the product is taken of rmsnorm(h) * nw (ssa_rmsnorm_add's bits).
template <typename T, int MM, bool NORM = false>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ x, const T* __restrict__ W,
                                                     T* __restrict__ act, int M, int I, int K,
                                                     const T* __restrict__ nw = nullptr, float eps = 0.f) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c0 = (blockIdx.x * 4 + wave) * 2;
  if (!NORM && c0 >= I) return;     // with NORM every wave takes part in the row norms
  float rs[MM], acc[4][MM];
  RowNorms<T, MM> norms;
  skinny_dots<T, MM, 4, NORM>(
      x, W, M, K, lane,
      [&](int r) {
        const int c = c0 + (r & 1);
        return c < I ? (int64_t)((r < 2 ? 0 : I) + c) : (int64_t)-1;
      },
      acc, nw, rs,
      [&] {
        if constexpr (NORM) {
          norms.load(x, M, K, threadIdx.x);
          norms.run(x, M, K, eps, rs);
        }
      });
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int m = 0; m < MM; ++m)
        if (m < M && c0 + q < I) {
          const float g = rnd<T>(acc[q][m]), u = rnd<T>(acc[2 + q][m]);
          const float sl = rnd<T>(g / (1.0f + expf(-g)));
          st(act, (int64_t)m * I + c0 + q, sl * u);
        }
  }
}

// h [rows, D] = embed[tok[row]], x = rmsnorm(h) * w (as ssa_rmsnorm_add without delta), and
// *n_out = *pos + 1 (the step's cache length): the first glue of a decode step.
template <typename T>
__global__ __launch_bounds__(256) void embed_rmsnorm_kernel(const int64_t* __restrict__ tok, const T* __restrict__ emb,
                                                            T* __restrict__ h, const T* __restrict__ w,
                                                            T* __restrict__ x, int D, int64_t vocab, float eps,
                                                            const int64_t* __restrict__ pos, int32_t* __restrict__ n_out) {
  __shared__ float red[4];
  const int64_t row = (int64_t)blockIdx.x * D;
  const int tid = threadIdx.x;
  const int64_t t = min(max(tok[blockIdx.x], (int64_t)0), vocab - 1);
  if (blockIdx.x == 0 && tid == 0 && n_out) *n_out = (int32_t)(*pos + 1);
  float ss = 0.f;
  for (int i = tid; i < D; i += 256) {
    const T e = emb[t * D + i];
    h[row + i] = e;
    const float v = to_f32(e);
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float r = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  for (int i = tid; i < D; i += 256) {
    const float v = to_f32(emb[t * D + i]);
    st(x, row + i, (v * r) * ld(w, i));
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

namespace {

template <bool NORM, bool RES>
int launch_skinny(const void* x, const void* W, void* y, int32_t M, int32_t N, int32_t K, int32_t dtype,
                  const void* nw, float eps, void* stream) {
  if (!x || !W || !y || M < 1 || M > 8 || N < 1 || K < 8 || K % 8 || (NORM && !nw)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(nw)) & 15)
    return hipErrorInvalidValue;
  if (dtype != kBF16 && dtype != kF16) return hipErrorInvalidValue;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto go = [&](auto tag, auto mm, auto rr) {
    using T = decltype(tag);
    constexpr int MM = decltype(mm)::value, R = decltype(rr)::value;
    const int grid = (N + 4 * R - 1) / (4 * R);
    hipLaunchKernelGGL((skinny_kernel<T, MM, R, NORM, RES>), dim3(grid), dim3(256), 0, st, static_cast<const T*>(x),
                       static_cast<const T*>(W), static_cast<T*>(y), M, N, K, static_cast<const T*>(nw), eps);
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

template <bool NORM>
int launch_swiglu(const void* x, const void* W, void* act, int32_t M, int32_t I, int32_t K, int32_t dtype,
                  const void* nw, float eps, void* stream) {
  if (!x || !W || !act || M < 1 || M > 8 || I < 1 || K < 8 || K % 8 || (NORM && !nw)) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(nw)) & 15)
    return hipErrorInvalidValue;
  if (dtype != kBF16 && dtype != kF16) return hipErrorInvalidValue;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto go = [&](auto tag, auto mm) {
    using T = decltype(tag);
    constexpr int MM = decltype(mm)::value;
    const int grid = (I + 7) / 8;
    hipLaunchKernelGGL((swiglu_kernel<T, MM, NORM>), dim3(grid), dim3(256), 0, st, static_cast<const T*>(x),
                       static_cast<const T*>(W), static_cast<T*>(act), M, I, K, static_cast<const T*>(nw), eps);
    return (int)hipGetLastError();
  };
  auto bym = [&](auto tag) {
    if (M <= 1) return go(tag, std::integral_constant<int, 1>{});
    if (M <= 2) return go(tag, std::integral_constant<int, 2>{});
    if (M <= 4) return go(tag, std::integral_constant<int, 4>{});
    return go(tag, std::integral_constant<int, 8>{});
  };
  return dtype == kBF16 ? bym(__hip_bfloat16{}) : bym(__half{});
}

}  // namespace

extern "C" int ssa_linear_skinny(const void* x, const void* W, void* y, int32_t M, int32_t N, int32_t K, int32_t dtype,
                                 void* stream) {
  return launch_skinny<false, false>(x, W, y, M, N, K, dtype, nullptr, 0.f, stream);
}

extern "C" int ssa_linear_skinny_res(const void* x, const void* W, void* h, int32_t M, int32_t N, int32_t K,
                                     int32_t dtype, void* stream) {
  return launch_skinny<false, true>(x, W, h, M, N, K, dtype, nullptr, 0.f, stream);
}

extern "C" int ssa_rmsnorm_linear_skinny(const void* h, const void* norm_w, float eps, const void* W, void* y,
                                         int32_t M, int32_t N, int32_t K, int32_t dtype, void* stream) {
  return launch_skinny<true, false>(h, W, y, M, N, K, dtype, norm_w, eps, stream);
}

// out [M] int64 = argmax over each row of x [M, N]: the first index of the maximum, a NaN counting
// as above every number (torch.argmax's rule). Grid (P, M): workgroup p scans the p-th of P
// slices of a row (16-byte loads of 8 elements when the dtype is 2 bytes, N a multiple of 8 and
// the rows 16-byte aligned), reduces to one (value, index) and folds it into the row's 64-bit key
// with an agent-scope atomic max; the key orders as arg_better does. The last workgroup of the row
// to count itself in writes the index and returns key and count to zero for the next call.
constexpr int kArgThreads = 256, kArgMaxParts = 64, kArgSlice = 2048;
__device__ __forceinline__ bool arg_better(float v2, int i2, float v1, int i1) {
  if (v2 != v2) return v1 == v1 || i2 < i1;
  if (v1 != v1) return false;
  return v2 > v1 || (v2 == v1 && i2 < i1);
}
// unsigned order of the key = arg_better's order: value bits made monotone (NaN above +inf, -0 as
// +0) above the complemented index
__device__ __forceinline__ unsigned long long arg_key(float v, int i) {
  unsigned int b;
  if (v != v) {
    b = 0xffffffffu;
  } else {
    const unsigned int f = __float_as_uint(v + 0.0f);
    b = (f & 0x80000000u) ? ~f : (f | 0x80000000u);
  }
  return ((unsigned long long)b << 32) | (unsigned long long)(~(unsigned int)i);
}

template <typename T>
__global__ __launch_bounds__(kArgThreads) void argmax_rows_kernel(const T* __restrict__ x, int64_t* __restrict__ out,
                                                                  int N, int vec, unsigned long long* __restrict__ key,
                                                                  unsigned int* __restrict__ cnt) {
  __shared__ float sv[kArgThreads / 64];
  __shared__ int si[kArgThreads / 64];
  const int r = blockIdx.y, P = gridDim.x, p = blockIdx.x;
  const T* row = x + (int64_t)r * N;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -INFINITY;
  int bi = N;
  const int units = vec ? N / 8 : N;                 // 8-element chunks or elements
  const int per = (units + P - 1) / P;
  const int u0 = min(p * per, units), u1 = min(u0 + per, units);
  if (vec) {
    const uint4* rv = reinterpret_cast<const uint4*>(row);
    for (int c0 = u0 + tid; c0 < u1; c0 += 4 * kArgThreads) {
      uint4 q[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int c = c0 + k * kArgThreads;
        q[k] = c < u1 ? rv[c] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int c = c0 + k * kArgThreads;
        if (c >= u1) break;
        const T* e = reinterpret_cast<const T*>(&q[k]);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float v = to_f32(e[t]);
          if (arg_better(v, 8 * c + t, bv, bi)) { bv = v; bi = 8 * c + t; }
        }
      }
    }
  } else {
    for (int i = u0 + tid; i < u1; i += kArgThreads) {
      const float v = ld(row, i);
      if (arg_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    if (arg_better(v2, i2, bv, bi)) { bv = v2; bi = i2; }
  }
  if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
  __syncthreads();
  if (tid != 0) return;
  for (int w = 1; w < kArgThreads / 64; ++w)
    if (arg_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
  // The max must have completed at the coherence point before this workgroup counts itself in:
  // both atomics are relaxed and go to different addresses, so nothing else orders them. The
  // asm wait is a hardware wait for every outstanding memory operation of this thread (the
  // atomic included) and, through its memory clobber, a compiler barrier.
  if (bi < N) (void)__hip_atomic_fetch_max(key + r, arg_key(bv, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const unsigned int old = __hip_atomic_fetch_add(cnt + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old != (unsigned int)(P - 1)) return;
  const unsigned long long k = __hip_atomic_load(key + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  out[r] = (int64_t)(~(unsigned int)(k & 0xffffffffull));
  __hip_atomic_store(key + r, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(cnt + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

extern "C" int ssa_argmax_rows(const void* x, int64_t* out, int32_t M, int32_t N, int32_t dtype, void* work,
                               void* stream) {
  if (!x || !out || !work || M < 1 || N < 1) return hipErrorInvalidValue;
  if (reinterpret_cast<uintptr_t>(work) & 7) return hipErrorInvalidValue;
  auto* key = static_cast<unsigned long long*>(work);
  auto* cnt = reinterpret_cast<unsigned int*>(key + M);
  return by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    const int vec = sizeof(T) == 2 && N % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const int parts = std::max(1, std::min(kArgMaxParts, (N + kArgSlice - 1) / kArgSlice));
    hipLaunchKernelGGL(argmax_rows_kernel<T>, dim3(parts, M), dim3(kArgThreads), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const T*>(x), out, N, vec, key, cnt);
    return (int)hipGetLastError();
  });
}

extern "C" int ssa_linear_swiglu(const void* x, const void* W, void* act, int32_t M, int32_t I, int32_t K,
                                 int32_t dtype, void* stream) {
  return launch_swiglu<false>(x, W, act, M, I, K, dtype, nullptr, 0.f, stream);
}

extern "C" int ssa_rmsnorm_linear_swiglu(const void* h, const void* norm_w, float eps, const void* W, void* act,
                                         int32_t M, int32_t I, int32_t K, int32_t dtype, void* stream) {
  return launch_swiglu<true>(h, W, act, M, I, K, dtype, norm_w, eps, stream);
}

extern "C" int ssa_embed_rmsnorm(const int64_t* tok, const void* embed, void* h, const void* w, void* x, int32_t rows,
                                 int32_t D, int64_t vocab, float eps, const int64_t* pos, int32_t* n_out,
                                 int32_t dtype, void* stream) {
  if (!tok || !embed || !h || !w || !x || rows < 1 || D < 1 || vocab < 1 || (n_out && !pos)) return hipErrorInvalidValue;
  return by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    hipLaunchKernelGGL(embed_rmsnorm_kernel<T>, dim3(rows), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), tok,
                       static_cast<const T*>(embed), static_cast<T*>(h), static_cast<const T*>(w), static_cast<T*>(x),
                       D, vocab, eps, pos, n_out);
    return (int)hipGetLastError();
  });
}
