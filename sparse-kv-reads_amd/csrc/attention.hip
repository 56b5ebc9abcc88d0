// Split-K decode attention over a KV cache read in place (gfx950).
//
//   out[h] = sum_j w[label_j] e^{s_j} v_j / sum_j w[label_j] e^{s_j},   s_j = q_h . k_j / sqrt(d)
//
// Reference behaviour: label_weighted_attention (src/ssa/attn/labeled.py:24-44), computed by the
// reference GPU path as compact_positions + _list_kernel + merge_splits
// (src/ssa/kernels/labeled_attn.py:166-278) and, for the dense baseline, _dense_dev_kernel
// (src/ssa/kernels/graph_kernels.py:28-59).
//
// Design (one kernel per call, no index list in HBM):
//   grid (S, Hk): workgroup (sp, h) owns positions [sp*chunk, (sp+1)*chunk) of KV head h.
//   Labelled mode scans its positions' 2-byte labels, looks their weights up in an LDS copy
//   of w, and compacts the selected positions into an LDS list (ballot + popcount), so only
//   selected K/V rows are ever fetched. Dense mode walks its rows directly.
//   Rows are read as 16-byte-per-lane loads: D/8 lanes cover one 128-dim bf16 row (256 B), so
//   one wave instruction reads 64*16 B of consecutive row bytes; each lane group keeps its own
//   online softmax (base-2, q pre-scaled by log2(e)/sqrt(d)) over the G query heads that share
//   the KV head, and issues U rows of K and V before it consumes any of them.
//   States merge across lane groups (DPP/shuffle), across waves (LDS), then across the S
//   workgroups of a head: the last workgroup to arrive (agent-scope fence + atomic counter,
//   reset by that workgroup for the next launch) combines the partials by log-sum-exp and
//   writes out[h*G + g] in the output dtype, plus the count of rows read.
#include "ssa_common.h"

namespace ssa {

struct DecodeParams {
  const void* q; int64_t s_qh; int q_dtype;
  const void* k; int64_t s_kh, s_kn;
  const void* v; int64_t s_vh, s_vn;
  const int16_t* labels; int64_t s_lh;
  const float* w; int64_t s_wr; int w_len; int per_head;
  const int32_t* n_dev; int n_host;
  float* part_m; float* part_l; float* part_a; int32_t* part_cnt;
  int32_t* counter;
  void* out; int64_t s_oh; int out_dtype;
  int32_t* cnt_out;
  int n_heads, G, S;
  float qscale;        // log2(e)/sqrt(d)
  int chunk_align;
};

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPage = 1024;          // positions compacted per pass
constexpr int kMaxW = 1025;          // weight slots (C + 1) held in LDS per row

template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  // Sum over the LPR consecutive lanes that hold one row (LPR a power of two, 2..32).
  if constexpr (LPR >= 2) x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));
  if constexpr (LPR >= 4) x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));
  if constexpr (LPR >= 8) x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, true));
  if constexpr (LPR >= 16) x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, true));
  if constexpr (LPR >= 32) x += __shfl_xor(x, 16, 64);
  return x;
}

template <typename T>
struct Row8 {   // 8 consecutive elements of a row, widened to fp32
  float f[8];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (sizeof(T) == 2) {
      uint4 r = *reinterpret_cast<const uint4*>(p);
      const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (std::is_same<T, __hip_bfloat16>::value) {
          f[2 * e] = __uint_as_float(u[e] << 16);
          f[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
        } else {
          __half2 h2 = *reinterpret_cast<const __half2*>(&u[e]);
          f[2 * e] = __low2float(h2);
          f[2 * e + 1] = __high2float(h2);
        }
      }
    } else {
      float4 a = *reinterpret_cast<const float4*>(p);
      float4 b = *reinterpret_cast<const float4*>(p + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = 0.f;
  }
};

__device__ __forceinline__ void store_out(void* out, int dt, int64_t i, float x) {
  if (dt == kBF16) reinterpret_cast<__hip_bfloat16*>(out)[i] = __float2bfloat16(x);
  else if (dt == kF16) reinterpret_cast<__half*>(out)[i] = __float2half(x);
  else reinterpret_cast<float*>(out)[i] = x;
}

// DENSE: every position in [0, n) is read with weight 1. Otherwise positions are selected by
// w[label] > 0 (any query head of the group, when w has one row per query head).
template <typename T, int D, int GMAX, bool DENSE>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeParams a) {
  constexpr int LPR = D / 8;           // lanes per row
  constexpr int RPI = 64 / LPR;        // rows per wave instruction
  constexpr int U = 4;                 // rows in flight per lane group
  constexpr int WROWS = DENSE ? 1 : GMAX;

  __shared__ float s_lw[DENSE ? 1 : WROWS][DENSE ? 1 : kMaxW];   // log2 w, -inf where w <= 0
  __shared__ int s_pos[DENSE ? 1 : kPage];
  __shared__ float s_rlw[DENSE ? 1 : WROWS][DENSE ? 1 : kPage];  // per listed row: log2 w per head row
  __shared__ int s_scan[kWaves];
  __shared__ float s_red_m[kWaves][GMAX], s_red_l[kWaves][GMAX];
  __shared__ float s_red_a[kWaves][GMAX][D];
  __shared__ int s_rows[kWaves];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane / LPR, li = lane % LPR;
  const int sp = blockIdx.x, h = blockIdx.y;
  const int G = a.G, S = a.S;
  const bool per_head = !DENSE && a.per_head;

  const int n = a.n_dev ? *a.n_dev : a.n_host;
  int chunk = (n + S - 1) / S;
  chunk = (chunk + a.chunk_align - 1) / a.chunk_align * a.chunk_align;
  const int s0 = min(sp * chunk, n);
  const int s1 = min(s0 + chunk, n);

  float qr[GMAX][8];
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      qr[g][e] = (g < G) ? load_as_f32(a.q, a.q_dtype, (int64_t)(h * G + g) * a.s_qh + li * 8 + e) * a.qscale : 0.f;

  if constexpr (!DENSE) {
    const int nrow = per_head ? G : 1;
    for (int r = 0; r < nrow; ++r) {
      const float* wr = a.w + (int64_t)(per_head ? h * G + r : h) * a.s_wr;
      for (int c = tid; c < a.w_len; c += kThreads) {
        float x = wr[c];
        s_lw[r][c] = x > 0.f ? __log2f(x) : -INFINITY;
      }
    }
  }

  float m_[GMAX], l_[GMAX];
  Row8<float> acc[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) { m_[g] = kNeg; l_[g] = 0.f; acc[g].zero(); }

  const T* kbase = reinterpret_cast<const T*>(a.k) + (int64_t)h * a.s_kh + li * 8;
  const T* vbase = reinterpret_cast<const T*>(a.v) + (int64_t)h * a.s_vh + li * 8;
  int rows_read = 0;

  for (int p0 = s0; p0 < s1; p0 += kPage) {
    const int pn = min(kPage, s1 - p0);
    int R;
    if constexpr (DENSE) {
      R = pn;
    } else {
      __syncthreads();   // s_lw ready / previous page's list consumed
      // Each thread owns 4 consecutive positions; the list keeps ascending position order.
      constexpr int PER = kPage / kThreads;
      const int16_t* lab = a.labels + (int64_t)h * a.s_lh + p0 + tid * PER;
      int lbl[PER];
      bool sel[PER];
      int cnt = 0;
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        int j = tid * PER + u;
        lbl[u] = (j < pn) ? min(max((int)lab[u], 0), a.w_len - 1) : 0;   // a bad label never leaves s_lw
        bool s = false;
        if (j < pn) {
          if (per_head) {
            for (int g = 0; g < G; ++g) s |= s_lw[g][lbl[u]] != -INFINITY;
          } else {
            s = s_lw[0][lbl[u]] != -INFINITY;
          }
        }
        sel[u] = s;
        cnt += s ? 1 : 0;
      }
      // workgroup exclusive scan of cnt
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      if (lane == 63) s_scan[wave] = incl;
      __syncthreads();
      int wbase = 0, total = 0;
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) {
        int c2 = s_scan[w2];
        if (w2 < wave) wbase += c2;
        total += c2;
      }
      int o = wbase + incl - cnt;
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        if (sel[u]) {
          s_pos[o] = p0 + tid * PER + u;
          if (per_head) {
            for (int g = 0; g < G; ++g) s_rlw[g][o] = s_lw[g][lbl[u]];
          } else {
            s_rlw[0][o] = s_lw[0][lbl[u]];
          }
          ++o;
        }
      }
      R = total;
      __syncthreads();
    }
    rows_read += R;

    // ---- attention over the R rows of this page -------------------------------------------
    for (int base = 0; base < R; base += kWaves * RPI * U) {
      Row8<float> kf[U], vf[U];
      int rr[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        rr[u] = base + u * kWaves * RPI + wave * RPI + lg;
        ok[u] = rr[u] < R;
        int pos = 0;
        if constexpr (DENSE) pos = p0 + rr[u];
        else pos = ok[u] ? s_pos[rr[u]] : 0;
        Row8<T> kt, vt;
        if (ok[u]) {
          kt.load(kbase + (int64_t)pos * a.s_kn);
          vt.load(vbase + (int64_t)pos * a.s_vn);
        } else {
          kt.zero();
          vt.zero();
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) { kf[u].f[e] = kt.f[e]; vf[u].f[e] = vt.f[e]; }
      }
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g >= G) break;
        float s[U];
        float mx = m_[g];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(qr[g][e], kf[u].f[e], d);
          d = row_sum<LPR>(d);
          float lw = 0.f;
          if constexpr (!DENSE) lw = ok[u] ? s_rlw[per_head ? g : 0][rr[u]] : -INFINITY;
          s[u] = ok[u] ? d + lw : -INFINITY;
          mx = fmaxf(mx, s[u]);
        }
        const float alpha = __builtin_amdgcn_exp2f(m_[g] - mx);
        float psum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g].f[e] *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float p = __builtin_amdgcn_exp2f(s[u] - mx);
          psum += p;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g].f[e] = fmaf(p, vf[u].f[e], acc[g].f[e]);
        }
        l_[g] = fmaf(l_[g], alpha, psum);
        m_[g] = mx;
      }
    }
  }

  // ---- merge the lane groups of each wave ---------------------------------------------------
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      float m2 = __shfl_xor(m_[g], o, 64);
      float l2 = __shfl_xor(l_[g], o, 64);
      float M = fmaxf(m_[g], m2);
      float f1 = __builtin_amdgcn_exp2f(m_[g] - M), f2 = __builtin_amdgcn_exp2f(m2 - M);
      l_[g] = l_[g] * f1 + l2 * f2;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a2 = __shfl_xor(acc[g].f[e], o, 64);
        acc[g].f[e] = acc[g].f[e] * f1 + a2 * f2;
      }
      m_[g] = M;
    }
  }
  if (lane < LPR) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (lane == 0) { s_red_m[wave][g] = m_[g]; s_red_l[wave][g] = l_[g]; }
#pragma unroll
      for (int e = 0; e < 8; ++e) s_red_a[wave][g][li * 8 + e] = acc[g].f[e];
    }
  }
  if (tid == 0) s_rows[0] = rows_read;
  __syncthreads();

  // ---- merge the waves; write this workgroup's partial --------------------------------------
  const int64_t pidx = (int64_t)h * S + sp;
  for (int t = tid; t < G * D; t += kThreads) {
    const int g = t / D, dd = t % D;
    float M = kNeg;
#pragma unroll
    for (int w2 = 0; w2 < kWaves; ++w2) M = fmaxf(M, s_red_m[w2][g]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kWaves; ++w2) {
      float f = __builtin_amdgcn_exp2f(s_red_m[w2][g] - M);
      L = fmaf(s_red_l[w2][g], f, L);
      A = fmaf(s_red_a[w2][g][dd], f, A);
    }
    a.part_a[(pidx * G + g) * D + dd] = A;
    if (dd == 0) { a.part_m[pidx * G + g] = M; a.part_l[pidx * G + g] = L; }
  }
  if (tid == 0) a.part_cnt[pidx] = s_rows[0];

  // ---- the last workgroup of head h merges the S partials ----------------------------------
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    int old = __hip_atomic_fetch_add(a.counter + h, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (old == S - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int64_t hb = (int64_t)h * S;
  for (int t = tid; t < G * D; t += kThreads) {
    const int g = t / D, dd = t % D;
    float M = kNeg;
    for (int s2 = 0; s2 < S; ++s2) M = fmaxf(M, __builtin_nontemporal_load(a.part_m + (hb + s2) * G + g));
    float num = 0.f, den = 0.f;
    for (int s2 = 0; s2 < S; ++s2) {
      float f = __builtin_amdgcn_exp2f(__builtin_nontemporal_load(a.part_m + (hb + s2) * G + g) - M);
      den = fmaf(f, __builtin_nontemporal_load(a.part_l + (hb + s2) * G + g), den);
      num = fmaf(f, __builtin_nontemporal_load(a.part_a + ((hb + s2) * G + g) * D + dd), num);
    }
    store_out(a.out, a.out_dtype, (int64_t)(h * G + g) * a.s_oh + dd, num / den);
  }
  if (tid == 0) {
    int tot = 0;
    for (int s2 = 0; s2 < S; ++s2) tot += __builtin_nontemporal_load(a.part_cnt + hb + s2);
    if (a.cnt_out) a.cnt_out[h] = tot;
    a.counter[h] = 0;
  }
}

// LSE merge of natural-log partials (m, l, a) [Hk, S, G(, D)] -> out [Hk*G, D].
// Reference: _merge_kernel / merge_splits (src/ssa/kernels/labeled_attn.py:124-151).
__global__ __launch_bounds__(256) void merge_kernel(const float* m, const float* l, const float* av,
                                                    int64_t s_mh, int64_t s_ms, int64_t s_ah, int64_t s_as,
                                                    int64_t s_ag, void* out, int64_t s_oh, int out_dtype,
                                                    int S, int G, int D) {
  const int h = blockIdx.x;
  for (int t = threadIdx.x; t < G * D; t += blockDim.x) {
    const int g = t / D, dd = t % D;
    float M = kNeg;
    for (int s = 0; s < S; ++s) M = fmaxf(M, m[h * s_mh + s * s_ms + g]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < S; ++s) {
      float f = expf(m[h * s_mh + s * s_ms + g] - M);
      den = fmaf(f, l[h * s_mh + s * s_ms + g], den);
      num = fmaf(f, av[h * s_ah + s * s_as + g * s_ag + dd], num);
    }
    store_out(out, out_dtype, (int64_t)(h * G + g) * s_oh + dd, num / den);
  }
}

// Ascending list of selected positions per KV head: two passes over blocks of 1024 labels
// (count, then place at the block's exclusive prefix), so the output order is deterministic.
// Reference: _compact_kernel / compact_positions (src/ssa/kernels/labeled_attn.py:166-199).
constexpr int kCompactBlock = 1024;

__device__ __forceinline__ bool selected(const int16_t* lab, const float* w, int64_t s_wr, int h, int G,
                                         int per_head, int j) {
  int c = lab[j];
  if (per_head) {
    for (int g = 0; g < G; ++g)
      if (w[(int64_t)(h * G + g) * s_wr + c] > 0.f) return true;
    return false;
  }
  return w[(int64_t)h * s_wr + c] > 0.f;
}

__global__ __launch_bounds__(256) void compact_count_kernel(const int16_t* labels, int64_t s_lh, const float* w,
                                                            int64_t s_wr, int G, int per_head, const int32_t* n_dev,
                                                            int n_host, int32_t* bcnt, int nblk) {
  const int b = blockIdx.x, h = blockIdx.y;
  const int n = n_dev ? *n_dev : n_host;
  const int16_t* lab = labels + (int64_t)h * s_lh;
  int c = 0;
  for (int j = b * kCompactBlock + threadIdx.x; j < min(n, (b + 1) * kCompactBlock); j += 256)
    c += selected(lab, w, s_wr, h, G, per_head, j) ? 1 : 0;
  c = wave_sum_i(c);
  __shared__ int s[4];
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) bcnt[(int64_t)h * nblk + b] = s[0] + s[1] + s[2] + s[3];
}

__global__ __launch_bounds__(256) void compact_place_kernel(const int16_t* labels, int64_t s_lh, const float* w,
                                                            int64_t s_wr, int G, int per_head, const int32_t* n_dev,
                                                            int n_host, const int32_t* bcnt, int nblk, int32_t* idx,
                                                            int64_t s_ih, int32_t* cnt) {
  const int b = blockIdx.x, h = blockIdx.y;
  const int n = n_dev ? *n_dev : n_host;
  const int16_t* lab = labels + (int64_t)h * s_lh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int s_base, s_w[4];
  if (tid == 0) {
    int base = 0, tot = 0;
    for (int i = 0; i < nblk; ++i) {
      int c = bcnt[(int64_t)h * nblk + i];
      if (i < b) base += c;
      tot += c;
    }
    s_base = base;
    if (b == 0 && cnt) cnt[h] = tot;
  }
  __syncthreads();
  int base = s_base;
  for (int j0 = b * kCompactBlock; j0 < min(n, (b + 1) * kCompactBlock); j0 += 256) {
    int j = j0 + tid;
    bool sel = j < n && selected(lab, w, s_wr, h, G, per_head, j);
    int incl = wave_prefix_count(sel, lane);
    if (lane == 63) s_w[wave] = incl;
    __syncthreads();
    int wb = 0, tot = 0;
    for (int i = 0; i < 4; ++i) { if (i < wave) wb += s_w[i]; tot += s_w[i]; }
    if (sel) idx[(int64_t)h * s_ih + base + wb + incl - 1] = j;
    base += tot;
    __syncthreads();
  }
}

}  // namespace ssa

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
#include "../../include/ssa_hip.h"

using namespace ssa;

namespace {

template <typename T, int D, int GMAX>
hipError_t launch_decode_t(const DecodeParams& p, bool dense, hipStream_t st) {
  dim3 grid(p.S, p.n_heads);
  if (dense) hipLaunchKernelGGL((decode_kernel<T, D, GMAX, true>), grid, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((decode_kernel<T, D, GMAX, false>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_decode_d(const DecodeParams& p, bool dense, hipStream_t st) {
  if (p.G <= 1) return launch_decode_t<T, D, 1>(p, dense, st);
  if (p.G <= 2) return launch_decode_t<T, D, 2>(p, dense, st);
  if (p.G <= 4) return launch_decode_t<T, D, 4>(p, dense, st);
  if (p.G <= 8) return launch_decode_t<T, D, 8>(p, dense, st);
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_decode_ty(const DecodeParams& p, int d, bool dense, hipStream_t st) {
  switch (d) {
    case 16: return launch_decode_d<T, 16>(p, dense, st);
    case 32: return launch_decode_d<T, 32>(p, dense, st);
    case 64: return launch_decode_d<T, 64>(p, dense, st);
    case 128: return launch_decode_d<T, 128>(p, dense, st);
    case 256: return launch_decode_d<T, 256>(p, dense, st);
  }
  return hipErrorInvalidValue;
}

int launch_decode(const ssa_attn_args_t* x, bool dense, void* stream) {
  if (!x || x->G < 1 || x->G > 8 || x->S < 1 || x->n_heads < 1) return hipErrorInvalidValue;
  if (!dense && (x->w_len < 1 || x->w_len > kMaxW)) return hipErrorInvalidValue;
  DecodeParams p{};
  p.q = x->q; p.s_qh = x->s_qh; p.q_dtype = x->q_dtype;
  p.k = x->k; p.s_kh = x->s_kh; p.s_kn = x->s_kn;
  p.v = x->v; p.s_vh = x->s_vh; p.s_vn = x->s_vn;
  p.labels = x->labels; p.s_lh = x->s_lh;
  p.w = x->w; p.s_wr = x->s_wr; p.w_len = x->w_len; p.per_head = x->per_head;
  p.n_dev = x->n_dev; p.n_host = x->n_host;
  p.part_m = x->part_m; p.part_l = x->part_l; p.part_a = x->part_a; p.part_cnt = x->part_cnt;
  p.counter = x->counter;
  p.out = x->out; p.s_oh = x->s_oh; p.out_dtype = x->out_dtype;
  p.cnt_out = x->cnt_out;
  p.n_heads = x->n_heads; p.G = x->G; p.S = x->S;
  p.qscale = (float)(1.4426950408889634 / __builtin_sqrt((double)x->d));
  p.chunk_align = x->chunk_align > 0 ? x->chunk_align : 64;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (x->kv_dtype) {
    case kBF16: return launch_decode_ty<__hip_bfloat16>(p, x->d, dense, st);
    case kF16: return launch_decode_ty<__half>(p, x->d, dense, st);
    case kF32: return launch_decode_ty<float>(p, x->d, dense, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

extern "C" int ssa_label_attention(const ssa_attn_args_t* args, void* stream) {
  return launch_decode(args, false, stream);
}

extern "C" int ssa_dense_attention(const ssa_attn_args_t* args, void* stream) {
  return launch_decode(args, true, stream);
}

extern "C" int ssa_merge_splits(const float* m, const float* l, const float* a, int64_t s_mh, int64_t s_ms,
                                int64_t s_ah, int64_t s_as, int64_t s_ag, int n_heads, int S, int G, int d,
                                void* out, int64_t s_oh, int out_dtype, void* stream) {
  if (n_heads < 1 || S < 1 || G < 1 || d < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(merge_kernel, dim3(n_heads), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), m, l, a,
                     s_mh, s_ms, s_ah, s_as, s_ag, out, s_oh, out_dtype, S, G, d);
  return hipGetLastError();
}

extern "C" int ssa_compact_positions(const int16_t* labels, int64_t s_lh, const float* w, int64_t s_wr,
                                     int n_heads, int G, int per_head, const int32_t* n_dev, int n_host,
                                     int capacity, int32_t* block_counts, int32_t* idx, int64_t s_ih,
                                     int32_t* cnt, void* stream) {
  if (n_heads < 1 || capacity < 1) return hipErrorInvalidValue;
  const int nblk = (capacity + kCompactBlock - 1) / kCompactBlock;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(compact_count_kernel, dim3(nblk, n_heads), dim3(256), 0, st, labels, s_lh, w, s_wr, G,
                     per_head, n_dev, n_host, block_counts, nblk);
  hipLaunchKernelGGL(compact_place_kernel, dim3(nblk, n_heads), dim3(256), 0, st, labels, s_lh, w, s_wr, G,
                     per_head, n_dev, n_host, block_counts, nblk, idx, s_ih, cnt);
  return hipGetLastError();
}

extern "C" const char* ssa_error_string(int err) { return hipGetErrorString(static_cast<hipError_t>(err)); }
