// Cluster index kernels (gfx950): per-step insertion with in-kernel splitting, cluster scoring
// and budget selection, and the prefill build (centring, cosine k-means, binning, summaries).
//
// Every decision is made in the canonical arithmetic described in ssa_common.h, and this file
// is compiled with -ffp-contract=off, so labels, selections and splits are reproducible bit
// for bit by a CPU restatement that follows the same order of operations.
//
// Reference behaviour:
//   insertion  _bin_kernel / _bin_dev_kernel    src/ssa/kernels/sphere_fused.py:171-227,
//                                               src/ssa/kernels/graph_kernels.py:63-130
//   split      _split_cluster                   src/ssa/kernels/sphere_fused.py:49-167
//              (rule of _bisect_padded,         src/ssa/attn/sphere_gpu.py:76-102)
//   selection  _score_kernel + _shared_pick     src/ssa/kernels/sphere_fused.py:231-313
//              SphereIndexGPU.labels_and_weights src/ssa/attn/sphere_gpu.py:402-442
//   prefill    SphereIndexGPU._build / _bin      src/ssa/attn/sphere_gpu.py:166-219
//              spherical_kmeans                  src/ssa/attn/clusterkv.py:27-46
//              _refresh8                         src/ssa/kernels/sphere_fused.py:394-405
//
// One workgroup owns one (layer, sequence, KV head) for insertion and selection, so every
// summary has a single writer and no float atomics are needed.
#include "insert.h"

namespace ssa {

constexpr int kKB = 256;      // keys per block of the prefill's blocked sums

struct IndexArgs {
  ssa_index_state_t st;
  ssa_insert_args_t ins;
  ssa_select_args_t sel;
  int do_insert, do_select;
};

struct IndexSmem : InsertBase {
  union {
    SelSmem<kMaxG> sel;
    SplitTile spl;
  } u;
};

// ---- selection -----------------------------------------------------------------------------

template <int D, int GMAX>
__device__ __forceinline__ void select_phase(IndexSmem& S, const IndexArgs& A, int h, int end) {
  const ssa_index_state_t& st = A.st;
  const ssa_select_args_t& sl = A.sel;
  const int tid = threadIdx.x, G = sl.G;
  const Head H = head_view(st, h);
  SelPre<D> pre;
  sel_prefetch<D>(pre, H, st.C);
  const int n_act = st.n_c[h];
  const bool per_head = sl.group == 1;
  if (sl.need_out && tid == 0) {
    const int nb = end - 1;
    const double need = nb > 0 ? ceil(sl.budget * (double)nb) : 0.0;
    sl.need_out[h] = (int32_t)fmin(need, 2147483647.0);
  }
  // the selection scratch sized for GMAX query rows (a prefix of the union's kMaxG-row one)
  SelSmem<GMAX>& sel = *reinterpret_cast<SelSmem<GMAX>*>(&S.u.sel);
  for (int e = tid; e < GMAX * D; e += kT) {
    const int g = e / D, i = e % D;
    sel.q[g][i] = g < G ? load_as_f32(sl.q, sl.q_dtype, (int64_t)(h * G + g) * sl.s_qh + i) : 0.f;
  }
  __syncthreads();
  float* w = sl.w;
  const int64_t s_wr = sl.s_wr;
  select_head<D, kT, GMAX>(sel, H, pre, st.C, n_act, end, G, sl.budget, sl.group, sl.scale,
                           [&](int r, int c, float x) { w[(int64_t)(per_head ? h * G + r : h) * s_wr + c] = x; });
}

template <int D, int GMAX>
__global__ __launch_bounds__(kT) void index_kernel(IndexArgs A) {
  __shared__ IndexSmem S;
  const int h = blockIdx.x;
  int end = 0;
  if (A.do_insert) {
    const int n = A.ins.n_dev ? *A.ins.n_dev : A.ins.n_host;
    InsPre<D> pre;
    insert_prefetch<D>(pre, A.st, A.ins, h, n);
    insert_phase<D>(S, A.st, A.ins, h, pre, n);
    end = S.scali[2];
  } else {
    end = A.st.end[h];
  }
  if (A.do_select) select_phase<D, GMAX>(S, A, h, end);
}

// ---- prefill ---------------------------------------------------------------------------------

struct BuildArgs {
  ssa_index_state_t st;
  ssa_build_args_t b;
  int nb, nblk;        // keys and blocks of the range; with a device plan, the maxima (scratch strides)
  // Device plan (ssa_maintain): the heads of this pass are b.heads[0, min(*dcount - dcount_off,
  // b.n_sel)) and the range is [b.start, *dend), both read by the kernels; the grids cover the
  // maxima and the workgroups past them return at once. The fit's cap, when set_cap, is
  // cap_keys if > 0 else cap_sf * nb / C_fit (in double, stored as float).
  const int32_t* dcount; int dcount_off;
  const int32_t* dend;
  int set_cap; float cap_keys; double cap_sf;
};

// The actual head count, range end, key count and block count of a build pass.
struct BuildDims {
  int nsel, end, nb, nblk;
};

__device__ __forceinline__ BuildDims build_dims(const BuildArgs& A) {
  BuildDims D;
  if (A.dend) {
    D.nsel = min(max(*A.dcount - A.dcount_off, 0), A.b.n_sel);
    D.end = min(*A.dend, A.b.start + A.nb);
    D.nb = max(D.end - A.b.start, 0);
    D.nblk = (D.nb + kKB - 1) / kKB;
  } else {
    D.nsel = A.b.n_sel;
    D.end = A.b.end;
    D.nb = A.nb;
    D.nblk = A.nblk;
  }
  return D;
}

__device__ __forceinline__ const char* head_keys(const BuildArgs& A, int h) {
  return reinterpret_cast<const char*>(A.b.k) + (int64_t)elem_size(A.b.k_dtype) * (int64_t)h * A.b.s_kh;
}

// Centre, stage 1: per block b of kKB consecutive keys of the range, the left-to-right sum of its
// keys, into part[s][b][0][:].
template <typename T>
__global__ __launch_bounds__(kT) void center_part_kernel(BuildArgs A, int ncl) {
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.y, b = blockIdx.x, tid = threadIdx.x, d = A.st.d;
  if (tid >= d || s >= Dm.nsel || b >= Dm.nblk) return;
  const int h = A.b.heads[s];
  KeysT<T> K{reinterpret_cast<const T*>(head_keys(A, h)), A.b.s_kn};
  const int p0 = A.b.start + b * kKB, p1 = min(p0 + kKB, Dm.end);
  // loads are issued 32 positions ahead of the adds
  float ks = 0.f;
  int p = p0;
  for (; p + 32 <= p1; p += 32) {
    float v[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) v[u] = K(p + u, tid);
#pragma unroll
    for (int u = 0; u < 32; ++u) ks = ks + v[u];
  }
  for (; p < p1; ++p) ks = ks + K(p, tid);
  A.b.part[(((int64_t)s * A.nblk + b) * ncl) * d + tid] = ks;
}

// Centre, stage 2: ksum = left-to-right sum of the block sums, mu = given or ksum / nb; reset the
// summaries.
__global__ __launch_bounds__(kT) void center_kernel(BuildArgs A, int ncl) {
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.x, tid = threadIdx.x;
  if (s >= Dm.nsel) return;
  const int h = A.b.heads[s];
  const int d = A.st.d, C = A.st.C, nb = Dm.nb;
  if (tid < d) {
    float ks = 0.f;
    for (int b = 0; b < Dm.nblk; ++b) ks = ks + A.b.part[(((int64_t)s * A.nblk + b) * ncl) * d + tid];
    A.st.ksum[(int64_t)h * d + tid] = ks;
    float mu;
    if (A.b.mu) mu = A.b.mu[(int64_t)s * d + tid];
    else mu = nb > 0 ? ks / (float)nb : 0.f;
    A.st.mu_ref[(int64_t)h * d + tid] = mu;
  }
  const int64_t cd = (int64_t)C * d;
  for (int64_t e = tid; e < cd; e += kT) A.st.sum_dir[(int64_t)h * cd + e] = 0.f;
  for (int c = tid; c < C; c += kT) {
    A.st.mmax[(int64_t)h * C + c] = 0.f;
    A.st.mmin[(int64_t)h * C + c] = INFINITY;
    A.st.count[(int64_t)h * C + c] = 0;
  }
  if (tid == 0) {
    A.st.end[h] = Dm.end;
    if (A.b.fit) {
      A.st.n_c[h] = A.b.C_fit;
      if (A.set_cap && nb > 0)
        A.st.cap[h] = A.cap_keys > 0.f ? A.cap_keys : (float)(A.cap_sf * (double)nb / (double)A.b.C_fit);
    }
  }
}

// Unit centred directions of the range's keys, their lengths and squared lengths.
// Also, per block of kKB (= kT) keys, the left-to-right sum of their squared lengths, into
// part[s][b][1][0].
template <typename T, int D>
__global__ __launch_bounds__(kT) void normalize_kernel(BuildArgs A, int ncl) {
  static_assert(kKB == kT, "one block of the squared-length sums per workgroup");
  __shared__ float s_sq[kT];
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.y;
  if (s >= Dm.nsel || (int)blockIdx.x >= Dm.nblk) return;   // uniform over the workgroup
  const int h = A.b.heads[s];
  const int j = blockIdx.x * kT + threadIdx.x;
  float sq = 0.f;
  if (j < Dm.nb) {
    KeysT<T> K{reinterpret_cast<const T*>(head_keys(A, h)), A.b.s_kn};
    const float* mu = A.st.mu_ref + (int64_t)h * D;
    const int p = A.b.start + j;
    float kr[D];
#pragma unroll
    for (int i = 0; i < D; ++i) kr[i] = K(p, i) - mu[i];
    sq = cdot([&](int i) { return kr[i]; }, [&](int i) { return kr[i]; }, D);
    const float mag = sqrtf(sq);
    const float magc = fmaxf(mag, 1e-12f);
    float4* x = reinterpret_cast<float4*>(A.b.xn + ((int64_t)s * A.nb + j) * D);
#pragma unroll
    for (int k = 0; k < D / 4; ++k)
      x[k] = make_float4(kr[4 * k] / magc, kr[4 * k + 1] / magc, kr[4 * k + 2] / magc, kr[4 * k + 3] / magc);
    A.b.mag[(int64_t)s * A.nb + j] = mag;
    A.b.sq[(int64_t)s * A.nb + j] = sq;
  }
  s_sq[threadIdx.x] = sq;
  __syncthreads();                                  // reached by every thread once
  if (threadIdx.x == 0) {
    const int nk = min(kT, Dm.nb - (int)blockIdx.x * kT);
    float t = 0.f;
    for (int u = 0; u < nk; ++u) t = t + s_sq[u];
    A.b.part[(((int64_t)s * A.nblk + blockIdx.x) * ncl + 1) * D] = t;
  }
}

// rbar = sqrt(left-to-right sum of the block sums of squared lengths / nb).
__global__ void rbar_kernel(BuildArgs A, int ncl) {
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.x;
  if (threadIdx.x != 0 || s >= Dm.nsel) return;
  const int h = A.b.heads[s];
  float t = 0.f;
  for (int b = 0; b < Dm.nblk; ++b) t = t + A.b.part[(((int64_t)s * A.nblk + b) * ncl + 1) * A.st.d];
  A.st.rbar[h] = Dm.nb > 0 ? sqrtf(t / (float)Dm.nb) : 0.f;
}

// k-means seed: centroid c is the unit direction of range member init_idx[c].
__global__ __launch_bounds__(kT) void kmeans_init_kernel(BuildArgs A) {
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.y, c = blockIdx.x, d = A.st.d;
  if (s >= Dm.nsel || Dm.nb <= 0) return;
  const int h = A.b.heads[s];
  const int j = A.b.init_idx[c];
  if (threadIdx.x < d)
    A.st.cent[((int64_t)h * A.st.C + c) * d + threadIdx.x] = A.b.xn[((int64_t)s * A.nb + j) * d + threadIdx.x];
}

// assign_j = argmax over the first n_c centroids of cdot(xn_j, cent_c), lowest index on ties.
// With write_labels the result also becomes the key's label.
//
// The contraction runs on the matrix cores: each wave scores 16 KG keys against every centroid
// with v_mfma_f32_16x16x32_bf16 on bf16 copies of the unit vectors (fp32 accumulation), the
// centroids staged through LDS in chunks of kAsgCH. Round-to-nearest bf16 copies (relative error
// at most 2^-9 per element) move the score of unit x and c by at most 2^-8 + 2^-18, and the two
// fp32 accumulations differ from the exact dot by under 2 d 2^-24: under 0.004 in all. So every
// centroid whose canonical dot equals the best lies within kAssignMargin = 0.01 > 2 * 0.004 of the
// best bf16 score. Pass 1 finds each key's best bf16 score; pass 2 lists the candidates (bf16
// score within the margin). A key with one candidate takes it; the candidates of the others are
// rescored with the canonical dot, 8 lanes per candidate (lane j runs chain j), and the best
// taken, lowest index on ties: the result is the canonical argmax.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr float kAssignMargin = 0.01f;
constexpr int kAsgCH = 64;                                   // centroids per LDS chunk
template <int D> constexpr int asg_groups() { return D <= 128 ? 4 : 2; }   // 16-key groups per wave
template <int D> constexpr int asg_keys() { return 16 * asg_groups<D>() * kW; }
// candidate list entries per wave: room for two tiles' worth (every lane a candidate of every key row)
template <int D> constexpr int asg_list() { return 2 * 64 * 4 * asg_groups<D>(); }

// 8 consecutive fp32 values [k0, k0 + 8) of a row of D, as bf16 (zeros past D)
template <int D>
__device__ __forceinline__ bf16x8 frag8(const float* row, int k0) {
  bf16x8 v;
  if (k0 < D) {
    const float4 x = *reinterpret_cast<const float4*>(row + k0);
    const float4 y = *reinterpret_cast<const float4*>(row + k0 + 4);
    v[0] = (__bf16)x.x; v[1] = (__bf16)x.y; v[2] = (__bf16)x.z; v[3] = (__bf16)x.w;
    v[4] = (__bf16)y.x; v[5] = (__bf16)y.y; v[6] = (__bf16)y.z; v[7] = (__bf16)y.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (__bf16)0.f;
  }
  return v;
}

// max / sum / min over the 16 lanes of a DPP row, on every lane of the row
template <typename T, typename F>
__device__ __forceinline__ T row16_reduce(T v, F op) {
  auto sh = [](T x, auto ctrl) {
    int b;
    __builtin_memcpy(&b, &x, 4);
    b = __builtin_amdgcn_mov_dpp(b, decltype(ctrl)::value, 0xF, 0xF, true);
    __builtin_memcpy(&x, &b, 4);
    return x;
  };
  v = op(v, sh(v, std::integral_constant<int, 0xB1>{}));
  v = op(v, sh(v, std::integral_constant<int, 0x4E>{}));
  v = op(v, sh(v, std::integral_constant<int, 0x141>{}));
  v = op(v, sh(v, std::integral_constant<int, 0x140>{}));
  return v;
}

template <int D>
__global__ __launch_bounds__(kT) void assign_kernel(BuildArgs A, int write_labels) {
  constexpr int KS = (D + 31) / 32;                      // MFMA k-steps
  constexpr int KG = asg_groups<D>();
  constexpr int NK = 16 * KG;                            // keys per wave
  constexpr int DP = 32 * KS + 8;                        // LDS row in bf16: 16 bytes of pad per row
  __shared__ __align__(16) __bf16 cl[kAsgCH * DP];
  constexpr int LIST = asg_list<D>();
  __shared__ int lst[kW][LIST];                      // candidates: key << 16 | centroid
  __shared__ unsigned long long rk[kW][NK];              // best (score desc, index asc) per key
  __shared__ int kcnt[kW][NK], kfirst[kW][NK];
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (s >= Dm.nsel || (int)blockIdx.x * asg_keys<D>() >= Dm.nb) return;   // uniform over the workgroup
  const int h = A.b.heads[s];
  const int nb = Dm.nb;
  const int nc = A.st.n_c[h];
  const float* cent = A.st.shared_dirs ? A.st.cent : A.st.cent + (int64_t)h * A.st.C * D;
  const float* xn = A.b.xn + (int64_t)s * A.nb * D;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int j0 = blockIdx.x * asg_keys<D>() + wave * NK;
  // A operands: key j0 + 16 g + r16, elements 32 ks + 8 g4 + [0, 8)
  bf16x8 af[KG][KS];
#pragma unroll
  for (int g = 0; g < KG; ++g) {
    const float* xa = xn + (int64_t)min(j0 + 16 * g + r16, nb - 1) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) af[g][ks] = frag8<D>(xa, 32 * ks + 8 * g4);
  }
  if (lane < NK) rk[wave][lane] = ~0ull;
  auto stage = [&](int c0) {
    __syncthreads();
    for (int e = tid; e < kAsgCH * 4 * KS; e += kT) {
      const int r = e / (4 * KS), k0 = 8 * (e % (4 * KS)), c = c0 + r;
      bf16x8 v;
      if (c < nc) v = frag8<D>(cent + (int64_t)c * D, k0);
      else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (__bf16)0.f;
      }
      *reinterpret_cast<bf16x8*>(cl + r * DP + k0) = v;
    }
    __syncthreads();
  };
  // scores of centroids c0 + 16 t + r16 against rows 4 g4 + i of every key group
  auto tile = [&](int t, f32x4 (&acc)[KG]) {
#pragma unroll
    for (int g = 0; g < KG; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(cl + (16 * t + r16) * DP + 32 * ks + 8 * g4);
#pragma unroll
      for (int g = 0; g < KG; ++g) acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[g][ks], b, acc[g], 0, 0, 0);
    }
  };
  // canonical rescoring of list entries [0, n): 8 lanes per entry; with `all` false only the
  // entries of keys with more than one candidate
  auto rescore = [&](int n, bool all) {
    const int q = lane >> 3, jc = lane & 7;
    for (int e0 = 0; e0 < n; e0 += 8) {
      const int ent = e0 + q < n ? lst[wave][e0 + q] : -1;
      const int kl = ent >> 16, c = ent & 0xFFFF;
      const bool go = ent >= 0 && (all || kcnt[wave][kl] > 1);
      float v = 0.f;
      if (go) {
        const float* xr = xn + (int64_t)(j0 + kl) * D + jc;
        const float* cr = cent + (int64_t)c * D + jc;
#pragma unroll 8
        for (int m = 0; m < D / 8; ++m) v = __builtin_fmaf(xr[8 * m], cr[8 * m], v);
      }
      v = group8_sum(v);
      if (go && jc == 0) atomicMin(&rk[wave][kl], rank_key(v, c));
    }
  };
  // pass 1: best bf16 score of every key
  float thr[KG][4];
#pragma unroll
  for (int g = 0; g < KG; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) thr[g][i] = -INFINITY;
  for (int c0 = 0; c0 < nc; c0 += kAsgCH) {
    stage(c0);
    const int nt = min(kAsgCH / 16, (nc - c0 + 15) / 16);
    for (int t = 0; t < nt; ++t) {
      f32x4 acc[KG];
      tile(t, acc);
      const bool ok = c0 + 16 * t + r16 < nc;
#pragma unroll
      for (int g = 0; g < KG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) thr[g][i] = fmaxf(thr[g][i], ok ? acc[g][i] : -INFINITY);
    }
  }
  auto fmax_op = [](float a, float b) { return fmaxf(a, b); };
#pragma unroll
  for (int g = 0; g < KG; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) thr[g][i] = row16_reduce(thr[g][i], fmax_op) - kAssignMargin;
  // pass 2: list the candidates; per lane, the count and the first candidate of its columns
  int cnt[KG][4], first[KG][4];
#pragma unroll
  for (int g = 0; g < KG; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) { cnt[g][i] = 0; first[g][i] = 0x7FFFFFFF; }
  int n = 0;
  bool flushed = false;
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int c0 = 0; c0 < nc; c0 += kAsgCH) {
    stage(c0);
    const int nt = min(kAsgCH / 16, (nc - c0 + 15) / 16);
    for (int t = 0; t < nt; ++t) {
      if (n > LIST - 64 * 4 * KG) {                    // room for one tile's worth
        rescore(n, true);
        n = 0;
        flushed = true;
      }
      f32x4 acc[KG];
      tile(t, acc);
      const int c = c0 + 16 * t + r16;
#pragma unroll
      for (int g = 0; g < KG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kl = 16 * g + 4 * g4 + i;
          const bool cand = c < nc && j0 + kl < nb && acc[g][i] >= thr[g][i];
          cnt[g][i] += cand ? 1 : 0;
          first[g][i] = cand ? min(first[g][i], c) : first[g][i];
          const unsigned long long m = __ballot(cand);
          if (cand) lst[wave][n + __popcll(m & below)] = (kl << 16) | c;
          n += __popcll(m);
        }
    }
  }
  auto add_op = [](int a, int b) { return a + b; };
  auto min_op = [](int a, int b) { return min(a, b); };
#pragma unroll
  for (int g = 0; g < KG; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tot = row16_reduce(cnt[g][i], add_op), fst = row16_reduce(first[g][i], min_op);
      if (r16 == i) { kcnt[wave][16 * g + 4 * g4 + i] = tot; kfirst[wave][16 * g + 4 * g4 + i] = fst; }
    }
  __syncthreads();
  rescore(n, flushed);
  __syncthreads();
  if (lane < NK) {
    const int j = j0 + lane;
    if (j < nb) {
      const int k = kcnt[wave][lane];
      // no candidate: every score of the key is NaN (a non-finite key); it joins cluster 0, the
      // first index, as torch.argmax picks on a row of NaNs
      const int c = k == 0 ? 0 : (k == 1 && !flushed) ? kfirst[wave][lane] : (int)(unsigned int)rk[wave][lane];
      A.b.assign[(int64_t)s * A.nb + j] = c;
      if (write_labels) A.st.labels[(int64_t)h * A.st.capacity + A.b.start + j] = (int16_t)c;
    }
  }
}

// Blocked sums, stage 1: for block b of kKB consecutive keys, per cluster, the ordered sum of its
// members' unit directions (members in position order) and the member count. With summaries,
// also fold the members' lengths into mmax / mmin (order-free max / min).
__global__ __launch_bounds__(kT) void block_sum_kernel(BuildArgs A, int ncl, int summaries) {
  __shared__ int s_as[kKB], s_order[kKB], s_start[kMaxC + 1], s_cnt[kMaxC];
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.y, b = blockIdx.x, tid = threadIdx.x, d = A.st.d;
  if (s >= Dm.nsel || b >= Dm.nblk) return;   // uniform over the workgroup
  const int h = A.b.heads[s];
  const int j0 = b * kKB, nk = min(kKB, Dm.nb - j0);
  const int* as = A.b.assign + (int64_t)s * A.nb + j0;
  for (int c = tid; c < ncl; c += kT) s_cnt[c] = 0;
  __syncthreads();
  for (int r = tid; r < nk; r += kT) {
    s_as[r] = as[r];
    atomicAdd(&s_cnt[s_as[r]], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int c = 0; c < ncl; ++c) { s_start[c] = acc; acc += s_cnt[c]; }
    s_start[ncl] = acc;
  }
  __syncthreads();
  for (int r = tid; r < nk; r += kT) {
    const int c = s_as[r];
    int rank = 0;
    for (int r2 = 0; r2 < r; ++r2) rank += (s_as[r2] == c) ? 1 : 0;
    s_order[s_start[c] + rank] = r;
  }
  __syncthreads();
  float* part = A.b.part + ((int64_t)s * A.nblk + b) * ncl * d;
  const float* xn = A.b.xn + ((int64_t)s * A.nb + j0) * d;
  for (int e = tid; e < ncl * d; e += kT) {
    const int c = e / d, i = e % d;
    float acc = 0.f;
    for (int t = s_start[c]; t < s_start[c + 1]; ++t) acc = acc + xn[(int64_t)s_order[t] * d + i];
    part[e] = acc;
  }
  for (int c = tid; c < ncl; c += kT) A.b.part_cnt[((int64_t)s * A.nblk + b) * ncl + c] = s_cnt[c];
  if (summaries) {
    const float* mg = A.b.mag + (int64_t)s * A.nb + j0;
    for (int r = tid; r < nk; r += kT) {
      const int c = s_as[r];
      const int bits = __float_as_int(mg[r]);   // lengths are >= 0, so int order is float order
      if (mg[r] != mg[r]) continue;             // a NaN length is ignored, as fmaxf / fminf do
      atomicMax(reinterpret_cast<int*>(A.st.mmax + (int64_t)h * A.st.C + c), bits);
      atomicMin(reinterpret_cast<int*>(A.st.mmin + (int64_t)h * A.st.C + c), bits);
    }
  }
}

// Blocked sums, stage 2: ordered sum over blocks. Centroid mode: cent_c = unit(sum) where the
// cluster has members (else unchanged). Summary mode: sum_dir_c = sum, count_c = members.
__global__ __launch_bounds__(kT) void block_reduce_kernel(BuildArgs A, int ncl, int summaries) {
  __shared__ float v[kMaxD];
  __shared__ float s_r;
  __shared__ int s_n;
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, d = A.st.d;
  if (s >= Dm.nsel) return;                         // uniform over the workgroup
  const int h = A.b.heads[s];
  const int nblk = Dm.nblk;
  if (tid == 0) s_n = 0;
  __syncthreads();
  if (tid < d) {
    // left to right over the blocks; loads are issued 16 blocks ahead of the adds
    const float* pp = A.b.part + ((int64_t)s * A.nblk * ncl + c) * d + tid;
    const int64_t st = (int64_t)ncl * d;
    float acc = 0.f;
    int b = 0;
    for (; b + 16 <= nblk; b += 16) {
      float x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = pp[(b + u) * st];
#pragma unroll
      for (int u = 0; u < 16; ++u) acc = acc + x[u];
    }
    for (; b < nblk; ++b) acc = acc + pp[b * st];
    v[tid] = acc;
  }
  int n = 0;                                        // integer counts: any order
  for (int b = tid; b < nblk; b += kT) n += A.b.part_cnt[((int64_t)s * A.nblk + b) * ncl + c];
  if (n) atomicAdd(&s_n, n);
  __syncthreads();
  const int64_t row = ((int64_t)h * A.st.C + c) * d;
  if (summaries) {
    if (tid < d) A.st.sum_dir[row + tid] = v[tid];
    if (tid == 0) A.st.count[(int64_t)h * A.st.C + c] = s_n;
    return;
  }
  if (s_n == 0) return;
  if (tid == 0) s_r = fmaxf(sqrtf(cdot_ptr(v, v, d)), 1e-12f);
  __syncthreads();
  if (tid < d) A.st.cent[row + tid] = v[tid] / s_r;
}

// int8 copies of every slot of the rebuilt heads: dir8 = q8(unit(sum_dir)), cent8 = q8(unit(cent)).
__global__ __launch_bounds__(kT) void refresh8_kernel(BuildArgs A) {
  __shared__ float v[kMaxD];
  __shared__ float s_r;
  const BuildDims Dm = build_dims(A);
  const int s = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, d = A.st.d;
  if (s >= Dm.nsel) return;                         // uniform over the workgroup
  const int h = A.b.heads[s];
  const int64_t row = ((int64_t)h * A.st.C + c) * d;
  for (int pass = 0; pass < 2; ++pass) {
    const float* src = pass == 0 ? A.st.sum_dir : A.st.cent;
    int8_t* dst = pass == 0 ? A.st.dir8 : A.st.cent8;
    if (!dst) continue;
    if (pass == 1 && A.st.shared_dirs) continue;
    __syncthreads();
    if (tid < d) v[tid] = src[row + tid];
    __syncthreads();
    if (tid == 0) s_r = fmaxf(sqrtf(cdot_ptr(v, v, d)), 1e-12f);
    __syncthreads();
    if (tid < d) dst[row + tid] = q8(v[tid] / s_r);
  }
}

// ---- division of over-cap clusters after a fit ------------------------------------------------
//
// Reference: SphereIndexGPU._split_overflow / _split_batch (src/ssa/attn/sphere_gpu.py:307-391)
// with _kmeans_padded (:56-73) for the first round and _bisect_padded (:76-102) after it. One
// workgroup per head takes that head's clusters over the cap in slot order, one at a time, so
// the spare slots are handed out in the reference's order.

constexpr int kKmax = 32;     // parts of one k-means division held in LDS; more use a->parts
constexpr int kMaxParts = kMaxC;

struct FitArgs {
  ssa_index_state_t st;
  ssa_split_args_t a;
};

struct FitSmem : InsertBase {
  float cent[kKmax][kMaxD];
  float sums[kKmax][kMaxD];
  float pmx[kMaxParts], pmn[kMaxParts];
  int cntp[kMaxParts], renum[kMaxParts], slot[kMaxParts];
  int list[kMaxC];
  int nlist, nz, bad;
  union {
    SplitTile spl;
  } u;
};

__device__ __forceinline__ float fit_cap(const FitArgs& A, int h) { return fmaxf(A.st.cap[h], A.a.cap_min); }

__device__ __forceinline__ bool fit_over(const FitArgs& A, int h, int c, float cap) {
  const int ct = A.st.count[(int64_t)h * A.st.C + c];
  return (float)ct > cap && ct >= 2;
}

// Clusters over the cap per head.
__global__ __launch_bounds__(kT) void fit_count_kernel(FitArgs A) {
  __shared__ int red[kW];
  const int s = blockIdx.x, h = A.a.heads[s];
  const float cap = fit_cap(A, h);
  const int n_act = min(A.st.n_c[h], A.st.C);
  int n = 0;
  for (int c = threadIdx.x; c < n_act; c += kT) n += fit_over(A, h, c, cap) ? 1 : 0;
  n = wave_sum_i(n);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = n;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < kW; ++w) t += red[w];
    A.a.over[s] = t;
  }
}

// Rows of the parts' centroids and sums: in LDS for up to kKmax parts, else in the caller's
// scratch (a->parts, [2, max_parts, d] per head); row p of each starts at p * stride.
struct PartRows {
  float* cent; float* sums; int stride;
  __device__ float* c(int p) const { return cent + (int64_t)p * stride; }
  __device__ float* s(int p) const { return sums + (int64_t)p * stride; }
};

// P.s(p) = ordered sum (members in position order) of the unit directions of the members in
// part p (H.side), S.cntp[p] their number, for p < k.
__device__ __forceinline__ void fit_sums(FitSmem& S, const PartRows& P, const Head& H, const Keys& K, int m, int k) {
  const int tid = threadIdx.x, d = H.d;
  for (int e = tid; e < k * d; e += kT) P.s(e / d)[e % d] = 0.f;
  for (int p = tid; p < k; p += kT) S.cntp[p] = 0;
  __syncthreads();
  // member tiles as in member_sums; the next tile's keys load while this one is summed
  const bool v16 = keys_vec16(K);
  const int rows = MemberTile::rows(d);
  MemberTile T;
  if (m > 0) T.fetch(H, K, v16, m, 0);
  for (int t0 = 0; t0 < m; t0 += rows) {
    const int nr = min(rows, m - t0);
    T.store(H, S.mu, S.u.spl.tile, m, t0);
    if (tid < nr) S.u.spl.tside[tid] = H.side[t0 + tid];
    __syncthreads();
    if (t0 + rows < m) T.fetch(H, K, v16, m, t0 + rows);
    if (tid < d)
      for (int r = 0; r < nr; ++r) {
        const int p = S.u.spl.tside[r];
        float* sp = P.s(p) + tid;
        *sp = *sp + S.u.spl.tile[r * d + tid];
      }
    if (tid == kT - 1)
      for (int r = 0; r < nr; ++r) S.cntp[S.u.spl.tside[r]] += 1;
    __syncthreads();
  }
}

// Cosine k-means of the m members into k parts (_kmeans_padded): centroids start at members
// j*m/k, `iters` updates (a part with members takes the unit of its ordered sum), then a final
// assignment; each member's part (the best canonical dot, lowest part on ties) goes to H.side.
__device__ __forceinline__ void fit_kmeans(FitSmem& S, const PartRows& P, const Head& H, const Keys& K, int m, int k,
                                           int iters) {
  const int tid = threadIdx.x, d = H.d;
  for (int e = tid; e < k * d; e += kT) {
    const int p = e / d, i = e % d;
    const int j = min((int)(((int64_t)p * m) / k), m - 1);
    P.c(p)[i] = (K(H.mem[j], i) - S.mu[i]) / fmaxf(H.smag[j], 1e-12f);
  }
  __syncthreads();
  for (int it = 0; it <= iters; ++it) {
    for (int j = tid; j < m; j += kT) {
      const int pos = H.mem[j];
      const float magc = fmaxf(H.smag[j], 1e-12f);
      auto kn = [&](int i) { return (K(pos, i) - S.mu[i]) / magc; };
      int best = 0;
      const float* c0 = P.c(0);
      float bs = cdot_rolled(kn, [&](int i) { return c0[i]; }, d);
      for (int p = 1; p < k; ++p) {
        const float* cp = P.c(p);
        const float sc = cdot_rolled(kn, [&](int i) { return cp[i]; }, d);
        if (sc > bs) { bs = sc; best = p; }
      }
      H.side[j] = best;
    }
    __syncthreads();
    if (it == iters) break;
    fit_sums(S, P, H, K, m, k);
    for (int p = 0; p < k; ++p)
      if (S.cntp[p] > 0) block_unit(S, P.s(p), P.c(p), d);
  }
}

// The range, cap floor, round kind and scratch slot of one head's division.
struct FitCtx {
  int start, end;
  float cap_min;
  int nmeans;
  int slot;       // row of a.mem / side / proj / smag and of a.parts used for this head
};

// One round of the division for head a.heads[s], whose first cluster over the cap has global
// rank r0 in the round. Returns the clusters divided, or -1 when a division found no room.
template <int D>
__device__ __forceinline__ int fit_split_head(FitSmem& S, const FitArgs& A, int s, int r0, const FitCtx& X) {
  const ssa_index_state_t& st = A.st;
  const ssa_split_args_t& a = A.a;
  const int h = a.heads[s], tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, C = st.C;
  const float cap = fmaxf(st.cap[h], X.cap_min);
  const int n_act0 = min(st.n_c[h], C);
  if (tid == 0) { S.nlist = 0; S.bad = 0; }
  __syncthreads();
  for (int c0 = 0; c0 < n_act0; c0 += kT) {
    const int c = c0 + tid;
    const bool hit = c < n_act0 && fit_over(A, h, c, cap);
    const int incl = wave_prefix_count(hit, lane);
    if (lane == 63) S.red_i[wave] = incl;
    __syncthreads();
    int wb = 0, tot = 0;
    for (int w2 = 0; w2 < kW; ++w2) { if (w2 < wave) wb += S.red_i[w2]; tot += S.red_i[w2]; }
    if (hit) S.list[S.nlist + wb + incl - 1] = c;
    __syncthreads();
    if (tid == 0) S.nlist += tot;
    __syncthreads();
  }
  Head H = head_view(st, h);
  H.mem = a.mem + (int64_t)X.slot * a.ms;
  H.side = a.side + (int64_t)X.slot * a.ms;
  H.proj = a.proj + (int64_t)X.slot * a.ms;
  H.smag = a.smag + (int64_t)X.slot * a.ms;
  H.ms = a.ms;
  Keys K;
  K.dt = a.k_dtype;
  K.s_kn = a.s_kn;
  K.base = reinterpret_cast<const char*>(a.k) + (int64_t)elem_size(a.k_dtype) * (int64_t)h * a.s_kh;
  if (tid < D) S.mu[tid] = st.mu_ref[(int64_t)h * D + tid];
  __syncthreads();
  const int nlist = S.nlist;
  int n_cur = n_act0, base = n_act0, done = 0;
  for (int i = 0; i < nlist; ++i) {
    const int c = S.list[i];
    if ((r0 + i) % 64 == 0) base = n_cur;                 // a new batch of 64
    if (!X.nmeans) {
      if (base + 1 <= C) {
        split_cluster(S, st, H, K, h, c, base, X.end);
        if (st.n_c[h] == base + 1) { n_cur = base + 1; ++done; }
      }
      base += 1;
      continue;
    }
    const int m = gather_members(S, H, c, X.start, X.end);
    for (int j = tid; j < m; j += kT) {
      const int pos = H.mem[j];
      auto kr = [&](int t) { return K(pos, t) - S.mu[t]; };
      H.smag[j] = sqrtf(cdot_rolled(kr, kr, D));
    }
    __syncthreads();
    const float kf = ceilf(((float)m * a.split_factor) / cap);
    int k = kf < 2.f ? 2 : (kf >= (float)kMaxParts ? kMaxParts + 1 : (int)kf);
    PartRows P{&S.cent[0][0], &S.sums[0][0], kMaxD};
    if (k > kKmax) {
      if (!a.parts || k > a.max_parts || k > kMaxParts) {
        // no room for the parts: the cluster is left whole and the round reports it (done = -1)
        if (tid == 0) S.bad = 1;
        __syncthreads();
        continue;
      }
      float* base_p = a.parts + (int64_t)X.slot * 2 * a.max_parts * D;
      P = PartRows{base_p, base_p + (int64_t)a.max_parts * D, D};
    }
    fit_kmeans(S, P, H, K, m, k, a.iters);
    fit_sums(S, P, H, K, m, k);                           // final parts: ordered sums and sizes
    if (tid == 0) {
      int nz = 0;
      for (int p = 0; p < k; ++p) S.renum[p] = S.cntp[p] > 0 ? nz++ : -1;
      for (int q = 0; q < nz; ++q) S.slot[q] = q == 0 ? c : base + q - 1;
      S.nz = nz;
      for (int q = 0; q < nz; ++q) { S.pmx[q] = 0.f; S.pmn[q] = INFINITY; }
      for (int j = 0; j < m; ++j) {
        const int q = S.renum[H.side[j]];
        S.pmx[q] = fmaxf(S.pmx[q], H.smag[j]);
        S.pmn[q] = fminf(S.pmn[q], H.smag[j]);
      }
    }
    __syncthreads();
    const int extra = S.nz - 1;
    if (extra > 0 && base + extra <= C) {
      for (int p = 0; p < k; ++p) {
        const int q = S.renum[p];
        if (q < 0) continue;
        const int row = S.slot[q];
        if (tid < D) H.sum_dir[(int64_t)row * D + tid] = P.s(p)[tid];
        block_unit(S, P.s(p), H.cent + (int64_t)row * D, D);
        if (tid == 0) {
          H.mmax[row] = S.pmx[q];
          H.mmin[row] = S.pmn[q];
          H.count[row] = S.cntp[p];
        }
      }
      for (int j = tid; j < m; j += kT) H.labels[H.mem[j]] = (int16_t)S.slot[S.renum[H.side[j]]];
      n_cur += extra;
      if (tid == 0) {
        st.n_c[h] = n_cur;
        st.nsplit[h] = st.nsplit[h] + extra;
      }
      ++done;
    }
    base += extra > 0 ? extra : 0;
    __syncthreads();
  }
  const int bad = S.bad;
  __syncthreads();                                     // S is reused by the caller
  return bad ? -1 : done;
}

template <int D>
__global__ __launch_bounds__(kT) void fit_split_kernel(FitArgs A) {
  __shared__ FitSmem S;
  const int s = blockIdx.x;
  // global rank of this head's first cluster over the cap: heads are taken in order
  int r0 = 0;
  for (int t = threadIdx.x; t < s; t += kT) r0 += A.a.over[t];
  r0 = block_sum_i(S, r0);
  const int done = fit_split_head<D>(S, A, s, r0, FitCtx{A.a.start, A.a.end, A.a.cap_min, A.a.nmeans, s});
  if (threadIdx.x == 0) A.a.done[s] = done;
}

// ---- maintenance on the device (ssa_maintain) -------------------------------------------------
//
// Reference: SphereIndexFused._check_flags / _act_on / _rebuild (src/ssa/kernels/sphere_fused.py:
// 434-464), SphereIndexGPU._reset_heads (src/ssa/attn/sphere_gpu.py:283-293) and
// SphereIndexGraph._refit (src/ssa/kernels/graph_kernels.py:270-279), acting on the flags at the
// check as the reference's synchronous check does. The plan kernel decides on the device which
// heads are rebuilt; every later launch reads that plan, so the sequence can be captured once.
//
// Plan words: [0] heads to recentre, [1] heads to refit, [2] binned end, [3] 1 if a division
// found no room for its parts, [4] heads recentred so far, [5] heads reset so far, [6] rounds
// of the last division, [7] heads whose int8 copies the division refreshes (all, or 0); then
// SSA_MAINT_PLAN_WORDS + [0, n): heads to recentre, + [n, 2n): heads to refit, + [2n, 3n): all.

struct MaintArgs {
  ssa_maint_args_t m;
  int n;                      // heads of the layer
};

__global__ __launch_bounds__(kT) void maint_plan_kernel(ssa_index_state_t st, MaintArgs M) {
  __shared__ int s_nrec;
  const int n = M.n, d = st.d, tid = threadIdx.x;
  int32_t* plan = M.m.plan;
  int32_t* rec = plan + SSA_MAINT_PLAN_WORDS;
  int32_t* ref = rec + n;
  int32_t* all = ref + n;
  const int end = st.end[0];
  const int nb = end - 1;
  if (tid == 0) {
    int a = 0, b = 0;
    for (int h = 0; h < n; ++h) {
      const int f = st.flags[h];
      if (M.m.refit && (M.m.refit_all || (f & 2))) ref[b++] = h;        // refit (bit 1 wins over bit 0)
      else if (!M.m.refit_all && !(f & 2) && (f & 1) && nb > 0) rec[a++] = h;
    }
    s_nrec = a;
    plan[0] = a;
    plan[1] = b;
    plan[2] = end;
    plan[3] = 0;
    plan[4] += a;
    if (!M.m.refit_all) plan[5] += b;                  // resets; refits of every head are counted by the host
    plan[7] = (b > 0 && M.m.split_factor > 0.f) ? n : 0;
  }
  for (int h = tid; h < n; h += kT) all[h] = h;
  __syncthreads();
  // the centring mean of a recentred head: its running key sum over the binned keys
  for (int e = tid; e < s_nrec * d; e += kT) {
    const int i = e / d, t = e % d;
    M.m.mu[(int64_t)i * d + t] = st.ksum[(int64_t)rec[i] * d + t] / (float)nb;
  }
  for (int h = tid; h < n; h += kT) st.flags[h] = 0;   // thread 0 read them before the barrier
}

// Seed members of a refit: init_idx[c] = torch.randperm(nb, generator seeded with seed)[c % nb]
// for c < C_init (src/ssa/attn/clusterkv.py:34-36). torch's CPU randperm is a Fisher-Yates
// shuffle driven by MT19937 seeded by init_genrand: step i swaps r[i] with r[i + (draw % (nb -
// i))], a draw being the next 32-bit tempered output. r[0, C) is final after C steps, and only
// the swapped positions are stored (a hash map in LDS; identity elsewhere). One thread; refits are
// rare.
constexpr int kPermMap = 4096;          // > 2 * 1024 swapped positions

__global__ __launch_bounds__(64) void maint_randperm_kernel(MaintArgs M) {
  __shared__ uint32_t mt[624];
  __shared__ int key[kPermMap], val[kPermMap];
  const int32_t* plan = M.m.plan;
  if (plan[1] == 0) return;
  const int nb = plan[2] - 1;
  if (nb <= 0) return;
  for (int i = threadIdx.x; i < kPermMap; i += 64) key[i] = -1;
  __syncthreads();
  if (threadIdx.x != 0) return;
  uint32_t x = (uint32_t)M.m.seed;
  mt[0] = x;
  for (int k = 1; k < 624; ++k) {
    x = 1812433253u * (x ^ (x >> 30)) + (uint32_t)k;
    mt[k] = x;
  }
  int mi = 624;
  auto draw = [&]() -> uint32_t {
    if (mi >= 624) {
      for (int k = 0; k < 624; ++k) {
        const uint32_t y = (mt[k] & 0x80000000u) | (mt[k + 1 < 624 ? k + 1 : 0] & 0x7fffffffu);
        mt[k] = mt[k + 397 < 624 ? k + 397 : k + 397 - 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
      }
      mi = 0;
    }
    uint32_t y = mt[mi++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
  };
  auto slot = [&](int pos) {
    unsigned h = ((unsigned)pos * 2654435761u) >> 20;
    while (key[h] != -1 && key[h] != pos) h = (h + 1) & (kPermMap - 1);
    return h;
  };
  auto get = [&](int pos) {
    const unsigned h = slot(pos);
    return key[h] == pos ? val[h] : pos;
  };
  auto put = [&](int pos, int v) {
    const unsigned h = slot(pos);
    key[h] = pos;
    val[h] = v;
  };
  const int C = M.m.C_init;
  const int steps = min(C, nb - 1);
  for (int i = 0; i < steps; ++i) {
    const int j = i + (int)(draw() % (uint32_t)(nb - i));
    const int vi = get(i), vj = get(j);
    put(i, vj);
    put(j, vi);
  }
  for (int c = 0; c < C; ++c) M.m.init_idx[c] = get(c % nb);
}

// The division after a refit: one workgroup runs the rounds of the host loop of
// SphereIndexFused._split_overflow (a k-means round, then bisection rounds, until no cluster is
// over its cap or a bisection round divides nothing) over every head of the layer, heads in order
// within a round (the global ranks of ssa_split_fit), one head's member scratch at a time.
template <int D>
__global__ __launch_bounds__(kT) void maint_divide_kernel(FitArgs A, MaintArgs M) {
  __shared__ FitSmem S;
  int32_t* plan = M.m.plan;
  if (plan[7] == 0) return;
  const int end = plan[2], start = 1, n = M.n;
  const float cap_min = (float)(M.m.capk * (double)(end - start));
  int nmeans = 1, rounds = 0;
  for (;;) {
    int over_tot = 0;
    for (int s2 = 0; s2 < n; ++s2) {
      const int h = A.a.heads[s2];
      const float cap = fmaxf(A.st.cap[h], cap_min);
      const int n_act = min(A.st.n_c[h], A.st.C);
      int c0 = 0;
      for (int c = threadIdx.x; c < n_act; c += kT) c0 += fit_over(A, h, c, cap) ? 1 : 0;
      c0 = block_sum_i(S, c0);
      if (threadIdx.x == 0) A.a.over[s2] = c0;
      over_tot += c0;
    }
    __syncthreads();                                   // A.a.over written
    int r0 = 0, done_tot = 0;
    bool bad = false;
    for (int s2 = 0; s2 < n && !bad; ++s2) {
      const int dn = fit_split_head<D>(S, A, s2, r0, FitCtx{start, end, cap_min, nmeans, 0});
      r0 += A.a.over[s2];
      if (dn < 0) bad = true;
      else done_tot += dn;
    }
    ++rounds;
    if (bad) {
      if (threadIdx.x == 0) plan[3] = 1;
      break;
    }
    if (over_tot == 0 || (done_tot == 0 && !nmeans)) break;
    nmeans = 0;
  }
  if (threadIdx.x == 0) plan[6] = rounds;
}

}  // namespace ssa

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
using namespace ssa;

namespace {

bool state_ok(const ssa_index_state_t* st) {
  return st && st->n_heads > 0 && st->C >= 1 && st->C <= kMaxC && (st->C & (st->C - 1)) == 0 && st->d >= 8 &&
         st->d <= kMaxD && st->d % 8 == 0 && st->heads_per_layer > 0 && st->capacity > 0;
}

template <int D>
hipError_t launch_index_d(const IndexArgs& A, hipStream_t s) {
  const dim3 g(A.st.n_heads), b(kT);
  const int G = A.do_select ? A.sel.G : 1;
  if (G <= 1) hipLaunchKernelGGL((index_kernel<D, 1>), g, b, 0, s, A);
  else if (G <= 2) hipLaunchKernelGGL((index_kernel<D, 2>), g, b, 0, s, A);
  else if (G <= 4) hipLaunchKernelGGL((index_kernel<D, 4>), g, b, 0, s, A);
  else hipLaunchKernelGGL((index_kernel<D, 8>), g, b, 0, s, A);
  return hipGetLastError();
}

int launch_index(const IndexArgs& A, hipStream_t s) {
  switch (A.st.d) {
    case 16: return launch_index_d<16>(A, s);
    case 32: return launch_index_d<32>(A, s);
    case 64: return launch_index_d<64>(A, s);
    case 128: return launch_index_d<128>(A, s);
    case 256: return launch_index_d<256>(A, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

extern "C" int ssa_split_fit(const ssa_index_state_t* st, const ssa_split_args_t* a, void* stream) {
  if (!state_ok(st) || !a || a->n_sel < 1 || !a->heads) return hipErrorInvalidValue;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->refresh_only) {
    BuildArgs B{};
    B.st = *st;
    B.b.heads = a->heads;
    B.b.n_sel = a->n_sel;
    if (st->dir8 || st->cent8) hipLaunchKernelGGL(refresh8_kernel, dim3(st->C, a->n_sel), dim3(kT), 0, s, B);
    return hipGetLastError();
  }
  if (!a->k || !a->mem || !a->side || !a->proj || !a->smag || !a->over || !a->done || a->ms < 1 || a->start < 1 ||
      a->end > st->capacity || a->iters < 0)
    return hipErrorInvalidValue;
  FitArgs A{};
  A.st = *st;
  A.a = *a;
  hipLaunchKernelGGL(fit_count_kernel, dim3(a->n_sel), dim3(kT), 0, s, A);
  switch (st->d) {
    case 16: hipLaunchKernelGGL(fit_split_kernel<16>, dim3(a->n_sel), dim3(kT), 0, s, A); break;
    case 32: hipLaunchKernelGGL(fit_split_kernel<32>, dim3(a->n_sel), dim3(kT), 0, s, A); break;
    case 64: hipLaunchKernelGGL(fit_split_kernel<64>, dim3(a->n_sel), dim3(kT), 0, s, A); break;
    case 128: hipLaunchKernelGGL(fit_split_kernel<128>, dim3(a->n_sel), dim3(kT), 0, s, A); break;
    case 256: hipLaunchKernelGGL(fit_split_kernel<256>, dim3(a->n_sel), dim3(kT), 0, s, A); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

extern "C" int ssa_insert(const ssa_index_state_t* st, const ssa_insert_args_t* ins, void* stream) {
  if (!state_ok(st) || !ins) return hipErrorInvalidValue;
  IndexArgs A{};
  A.st = *st;
  A.ins = *ins;
  A.do_insert = 1;
  A.do_select = 0;
  return launch_index(A, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ssa_select(const ssa_index_state_t* st, const ssa_insert_args_t* ins, const ssa_select_args_t* sel,
                          void* stream) {
  if (!state_ok(st) || !sel || sel->G < 1 || sel->G > kMaxG || sel->group < 0 || sel->group > 3)
    return hipErrorInvalidValue;
  IndexArgs A{};
  A.st = *st;
  if (ins) A.ins = *ins;
  A.sel = *sel;
  A.do_insert = ins ? 1 : 0;
  A.do_select = 1;
  return launch_index(A, reinterpret_cast<hipStream_t>(stream));
}

namespace {

// The kernels of a build pass over A's heads (centre, optionally fit, bin, summarise, and the
// int8 copies when refresh). With a device plan (A.dend) every kernel is launched for the
// maxima and reads the actual heads and range itself.
void launch_build(const BuildArgs& A, int fit, bool refresh, hipStream_t s) {
  const ssa_index_state_t* st = &A.st;
  const int n_sel = A.b.n_sel;
  const int ncl = st->C;                           // part[] holds at least C slots per block
  const bool dev = A.dend != nullptr;
  if (dev || A.nb > 0) {
    const dim3 gb(A.nblk, n_sel);
    switch (A.b.k_dtype) {
      case kBF16: hipLaunchKernelGGL(center_part_kernel<__hip_bfloat16>, gb, dim3(kT), 0, s, A, ncl); break;
      case kF16: hipLaunchKernelGGL(center_part_kernel<__half>, gb, dim3(kT), 0, s, A, ncl); break;
      default: hipLaunchKernelGGL(center_part_kernel<float>, gb, dim3(kT), 0, s, A, ncl); break;
    }
  }
  hipLaunchKernelGGL(center_kernel, dim3(n_sel), dim3(kT), 0, s, A, ncl);
  if (dev || A.nb > 0) {
    dim3 gk((A.nb + kT - 1) / kT, n_sel);
    auto normalize = [&](auto tag) {
      using T = decltype(tag);
      switch (st->d) {
        case 16: hipLaunchKernelGGL((normalize_kernel<T, 16>), gk, dim3(kT), 0, s, A, ncl); break;
        case 32: hipLaunchKernelGGL((normalize_kernel<T, 32>), gk, dim3(kT), 0, s, A, ncl); break;
        case 64: hipLaunchKernelGGL((normalize_kernel<T, 64>), gk, dim3(kT), 0, s, A, ncl); break;
        case 128: hipLaunchKernelGGL((normalize_kernel<T, 128>), gk, dim3(kT), 0, s, A, ncl); break;
        case 256: hipLaunchKernelGGL((normalize_kernel<T, 256>), gk, dim3(kT), 0, s, A, ncl); break;
      }
    };
    if (A.b.k_dtype == kBF16) normalize(__hip_bfloat16{});
    else if (A.b.k_dtype == kF16) normalize(__half{});
    else normalize(0.f);
    hipLaunchKernelGGL(rbar_kernel, dim3(n_sel), dim3(64), 0, s, A, ncl);
    auto assign = [&](int write_labels) {
      auto go = [&](auto kern, int keys) {
        hipLaunchKernelGGL(kern, dim3((A.nb + keys - 1) / keys, n_sel), dim3(kT), 0, s, A, write_labels);
      };
      switch (st->d) {
        case 16: go(assign_kernel<16>, asg_keys<16>()); break;
        case 32: go(assign_kernel<32>, asg_keys<32>()); break;
        case 64: go(assign_kernel<64>, asg_keys<64>()); break;
        case 128: go(assign_kernel<128>, asg_keys<128>()); break;
        case 256: go(assign_kernel<256>, asg_keys<256>()); break;
      }
    };
    if (fit && !st->shared_dirs) {
      hipLaunchKernelGGL(kmeans_init_kernel, dim3(A.b.C_fit, n_sel), dim3(kT), 0, s, A);
      for (int it = 0; it < A.b.iters; ++it) {
        assign(0);
        hipLaunchKernelGGL(block_sum_kernel, dim3(A.nblk, n_sel), dim3(kT), 0, s, A, A.b.C_fit, 0);
        hipLaunchKernelGGL(block_reduce_kernel, dim3(A.b.C_fit, n_sel), dim3(kT), 0, s, A, A.b.C_fit, 0);
      }
    }
    assign(1);
    hipLaunchKernelGGL(block_sum_kernel, dim3(A.nblk, n_sel), dim3(kT), 0, s, A, st->C, 1);
    hipLaunchKernelGGL(block_reduce_kernel, dim3(st->C, n_sel), dim3(kT), 0, s, A, st->C, 1);
  }
  if (refresh && (st->dir8 || st->cent8)) hipLaunchKernelGGL(refresh8_kernel, dim3(st->C, n_sel), dim3(kT), 0, s, A);
}

template <int D>
void launch_divide(const FitArgs& F, const MaintArgs& M, hipStream_t s) {
  hipLaunchKernelGGL(maint_divide_kernel<D>, dim3(1), dim3(kT), 0, s, F, M);
}

}  // namespace

extern "C" int ssa_build(const ssa_index_state_t* st, const ssa_build_args_t* b, void* stream) {
  if (!state_ok(st) || !b || b->n_sel < 1 || b->start < 0 || b->end < b->start || b->end > st->capacity)
    return hipErrorInvalidValue;
  if (b->fit && (b->C_fit < 1 || b->C_fit > st->C || b->C_fit > kKB * 4 || !b->init_idx)) return hipErrorInvalidValue;
  BuildArgs A{};
  A.st = *st;
  A.b = *b;
  A.nb = b->end - b->start;
  A.nblk = (A.nb + kKB - 1) / kKB;
  launch_build(A, b->fit, true, reinterpret_cast<hipStream_t>(stream));
  return hipGetLastError();
}

extern "C" int ssa_maintain(const ssa_index_state_t* st, const ssa_maint_args_t* a, void* stream) {
  if (!state_ok(st) || !a || st->n_heads != st->heads_per_layer || st->capacity > 65536 || st->capacity < 2 ||
      !a->k || !a->plan || !a->mu || !a->xn || !a->mag || !a->sq || !a->assign || !a->part || !a->part_cnt ||
      a->max_heads < 1)
    return hipErrorInvalidValue;
  if (a->refit && (st->shared_dirs || a->C_init < 1 || a->C_init > st->C || a->C_init > kKB * 4 || a->iters < 0 ||
                   !a->init_idx || !a->mem || !a->side || !a->proj || !a->smag || !a->parts || !a->over))
    return hipErrorInvalidValue;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int n = st->n_heads, P = min(a->max_heads, n), passes = (n + P - 1) / P;
  MaintArgs M{};
  M.m = *a;
  M.n = n;
  hipLaunchKernelGGL(maint_plan_kernel, dim3(1), dim3(kT), 0, s, *st, M);
  int32_t* rec = a->plan + SSA_MAINT_PLAN_WORDS;
  int32_t* ref = rec + n;
  int32_t* all = ref + n;
  BuildArgs B{};
  B.st = *st;
  B.b.k = a->k; B.b.k_dtype = a->k_dtype; B.b.s_kh = a->s_kh; B.b.s_kn = a->s_kn;
  B.b.start = 1;
  B.b.end = st->capacity;
  B.b.xn = a->xn; B.b.mag = a->mag; B.b.sq = a->sq; B.b.assign = a->assign;
  B.b.part = a->part; B.b.part_cnt = a->part_cnt;
  B.nb = st->capacity - 1;                           // scratch strides: the largest binned range
  B.nblk = (B.nb + kKB - 1) / kKB;
  B.dend = a->plan + 2;
  if (a->refit) {
    hipLaunchKernelGGL(maint_randperm_kernel, dim3(1), dim3(64), 0, s, M);
    B.b.fit = 1;
    B.b.C_fit = a->C_init;
    B.b.iters = a->iters;
    B.b.init_idx = a->init_idx;
    B.b.mu = nullptr;
    B.set_cap = a->split_factor > 0.f;
    B.cap_keys = a->cap_keys;
    B.cap_sf = (double)a->split_factor;
    B.dcount = a->plan + 1;
    const bool divide = a->split_factor > 0.f;
    for (int p = 0; p < passes; ++p) {
      B.b.heads = ref + p * P;
      B.b.n_sel = P;
      B.dcount_off = p * P;
      launch_build(B, 1, !divide, s);
    }
    if (divide) {
      FitArgs F{};
      F.st = *st;
      F.a.k = a->k; F.a.k_dtype = a->k_dtype; F.a.s_kh = a->s_kh; F.a.s_kn = a->s_kn;
      F.a.heads = all; F.a.n_sel = n;
      F.a.start = 1;
      F.a.split_factor = a->split_factor;
      F.a.iters = a->iters;
      F.a.mem = a->mem; F.a.side = a->side; F.a.proj = a->proj; F.a.smag = a->smag;
      F.a.ms = st->capacity;
      F.a.over = a->over;
      F.a.parts = a->parts;
      F.a.max_parts = kMaxParts;
      switch (st->d) {
        case 16: launch_divide<16>(F, M, s); break;
        case 32: launch_divide<32>(F, M, s); break;
        case 64: launch_divide<64>(F, M, s); break;
        case 128: launch_divide<128>(F, M, s); break;
        case 256: launch_divide<256>(F, M, s); break;
      }
      // the int8 copies of every head after the division (plan[7] is n when a head was refitted)
      BuildArgs R = B;
      R.b.heads = all;
      R.b.n_sel = n;
      R.dcount = a->plan + 7;
      R.dcount_off = 0;
      if (st->dir8 || st->cent8) hipLaunchKernelGGL(refresh8_kernel, dim3(st->C, n), dim3(kT), 0, s, R);
    }
  }
  // recentre: the flagged heads' centroids are kept (no fit), their mean is ksum / nb
  B.b.fit = 0;
  B.set_cap = 0;
  B.dcount = a->plan + 0;
  for (int p = 0; p < passes; ++p) {
    B.b.heads = rec + p * P;
    B.b.n_sel = P;
    B.dcount_off = p * P;
    B.b.mu = a->mu + (int64_t)p * P * st->d;
    launch_build(B, 0, true, s);
  }
  return hipGetLastError();
}
