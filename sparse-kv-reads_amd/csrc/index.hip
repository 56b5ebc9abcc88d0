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
#include "select.h"

namespace ssa {

constexpr int kT = 256;       // threads per workgroup
constexpr int kW = kT / 64;   // waves
constexpr int kTile = 16;     // member rows staged in LDS by the split's ordered sums
constexpr int kKB = 256;      // keys per block of the prefill's blocked sums

struct IndexArgs {
  ssa_index_state_t st;
  ssa_insert_args_t ins;
  ssa_select_args_t sel;
  int do_insert, do_select;
};

struct IndexSmem {
  float mu[kMaxD], kr[kMaxD], kn[kMaxD], sd[kMaxD];
  float va[kMaxD], vb[kMaxD], vs[kMaxD];
  float red_f[kW];
  int red_i[kW];
  float scal[4];
  int scali[4];
  union {
    SelSmem<kMaxG> sel;
    struct {
      float tile[kTile][kMaxD];
      int tside[kTile];
    } spl;
  } u;
};

__device__ __forceinline__ int elem_size(int dt) { return dt == kF32 ? 4 : 2; }

// ---- workgroup reductions (results are uniform across the workgroup) -----------------------

__device__ void block_argmax(IndexSmem& S, float& s, int& i) {
  wave_argmax(s, i);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { S.red_f[w] = s; S.red_i[w] = i; }
  __syncthreads();
  s = S.red_f[0]; i = S.red_i[0];
  for (int w2 = 1; w2 < kW; ++w2) argmax_merge(s, i, S.red_f[w2], S.red_i[w2]);
  __syncthreads();
}

__device__ void block_argmin(IndexSmem& S, float& s, int& i) {
  wave_argmin(s, i);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { S.red_f[w] = s; S.red_i[w] = i; }
  __syncthreads();
  s = S.red_f[0]; i = S.red_i[0];
  for (int w2 = 1; w2 < kW; ++w2) argmin_merge(s, i, S.red_f[w2], S.red_i[w2]);
  __syncthreads();
}

__device__ float block_max(IndexSmem& S, float v) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) S.red_f[w] = v;
  __syncthreads();
  float r = S.red_f[0];
  for (int w2 = 1; w2 < kW; ++w2) r = fmaxf(r, S.red_f[w2]);
  __syncthreads();
  return r;
}

__device__ int block_sum_i(IndexSmem& S, int v) {
  v = wave_sum_i(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) S.red_i[w] = v;
  __syncthreads();
  int r = 0;
  for (int w2 = 0; w2 < kW; ++w2) r += S.red_i[w2];
  __syncthreads();
  return r;
}

// Canonical unit vector of an LDS vector x (d entries) written to y (may alias x).
__device__ void block_unit(IndexSmem& S, const float* x, float* y, int d) {
  if (threadIdx.x < 64) {
    const float r = fmaxf(sqrtf(wave_cdot(x, x, d)), 1e-12f);
    if (threadIdx.x == 0) S.scal[3] = r;
  }
  __syncthreads();
  const float r = S.scal[3];
  if (threadIdx.x < d) y[threadIdx.x] = x[threadIdx.x] / r;
  __syncthreads();
}

// Key rows of one head's cache, element type T: element i of position p.
template <typename T>
struct KeysT {
  const T* base; int64_t s_kn;
  __device__ __forceinline__ float operator()(int p, int i) const { return to_f32(base[(int64_t)p * s_kn + i]); }
};

// Key rows of one head's cache, element type given at run time: element i of position p.
struct Keys {
  const char* base; int dt; int64_t s_kn;
  __device__ float operator()(int p, int i) const { return load_as_f32(base, dt, (int64_t)p * s_kn + i); }
};

// ---- in-kernel split (rule of _bisect_padded) ----------------------------------------------

// Ordered sums over the members of the cluster being split: for each dimension i (thread i),
// s1 = sum of kn_j[i] over members on side 1 and s0 over side 0, left to right in member order.
__device__ void member_sums(IndexSmem& S, const Head& H, const Keys& K, int m, float* s0_out, float* s1_out,
                            int& n1_out) {
  const int tid = threadIdx.x, d = H.d;
  float s0 = 0.f, s1 = 0.f;
  int n1 = 0;
  for (int t0 = 0; t0 < m; t0 += kTile) {
    const int nr = min(kTile, m - t0);
    for (int e = tid; e < nr * d; e += kT) {
      const int r = e / d, i = e % d, j = t0 + r;
      const float magc = fmaxf(H.smag[j], 1e-12f);
      S.u.spl.tile[r][i] = (K(H.mem[j], i) - S.mu[i]) / magc;
    }
    if (tid < nr) S.u.spl.tside[tid] = H.side[t0 + tid];
    __syncthreads();
    if (tid < d) {
      for (int r = 0; r < nr; ++r) {
        const float x = S.u.spl.tile[r][tid];
        if (S.u.spl.tside[r]) { s1 = s1 + x; ++n1; } else { s0 = s0 + x; }
      }
    }
    __syncthreads();
  }
  if (tid < d) { s0_out[tid] = s0; s1_out[tid] = s1; }
  if (tid == 0) S.scali[1] = n1;
  __syncthreads();
  n1_out = S.scali[1];
  __syncthreads();
}

// side_j = kn_j.b > kn_j.a for every member (canonical dots), stored in H.side; returns #side 1.
__device__ int member_sides(IndexSmem& S, const Head& H, const Keys& K, int m, bool with_proj) {
  const int tid = threadIdx.x, d = H.d;
  int n1 = 0;
  for (int j = tid; j < m; j += kT) {
    const int pos = H.mem[j];
    const float magc = fmaxf(H.smag[j], 1e-12f);
    auto kn = [&](int i) { return (K(pos, i) - S.mu[i]) / magc; };
    const float da = cdot(kn, [&](int i) { return S.va[i]; }, d);
    const float db = cdot(kn, [&](int i) { return S.vb[i]; }, d);
    const int one = db > da ? 1 : 0;
    H.side[j] = one;
    n1 += one;
    if (with_proj) H.proj[j] = cdot(kn, [&](int i) { return S.vs[i]; }, d);
  }
  return block_sum_i(S, n1);
}

__device__ void split_cluster(IndexSmem& S, const ssa_index_state_t& st, const Head& H, const Keys& K, int h,
                              int c, int nw, int stop) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, d = H.d;
  // 1. members in ascending position order
  int m = 0;
  for (int j0 = 1; j0 < stop; j0 += kT) {
    const int j = j0 + tid;
    const bool hit = j < stop && H.labels[j] == c;
    const int incl = wave_prefix_count(hit, lane);
    if (lane == 63) S.red_i[wave] = incl;
    __syncthreads();
    int wb = 0, tot = 0;
    for (int w2 = 0; w2 < kW; ++w2) { if (w2 < wave) wb += S.red_i[w2]; tot += S.red_i[w2]; }
    const int slot = m + wb + incl - 1;
    if (hit && slot < H.ms) H.mem[slot] = j;
    m += tot;
    __syncthreads();
  }
  m = min(m, H.ms);
  if (m < 2) return;   // labels and counts disagree: leave the cluster as it is
  // 2. lengths
  for (int j = tid; j < m; j += kT) {
    const int pos = H.mem[j];
    auto kr = [&](int i) { return K(pos, i) - S.mu[i]; };
    H.smag[j] = sqrtf(cdot(kr, kr, d));
  }
  __syncthreads();
  // 3. start from the first member and the member least similar to it
  if (tid < d) S.va[tid] = (K(H.mem[0], tid) - S.mu[tid]) / fmaxf(H.smag[0], 1e-12f);
  __syncthreads();
  float lo = 0.f;
  int far = -1;
  for (int j = tid; j < m; j += kT) {
    const int pos = H.mem[j];
    const float magc = fmaxf(H.smag[j], 1e-12f);
    auto kn = [&](int i) { return (K(pos, i) - S.mu[i]) / magc; };
    argmin_merge(lo, far, cdot(kn, [&](int i) { return S.va[i]; }, d), j);
  }
  block_argmin(S, lo, far);
  if (tid < d) S.vb[tid] = (K(H.mem[far], tid) - S.mu[tid]) / fmaxf(H.smag[far], 1e-12f);
  __syncthreads();
  // 4. 2-means on cosine similarity, 4 iterations
  int n1 = 0;
  for (int it = 0; it < 4; ++it) {
    member_sides(S, H, K, m, false);
    __syncthreads();
    member_sums(S, H, K, m, S.kr, S.sd, n1);
    if (m - n1 > 0) block_unit(S, S.kr, S.va, d);
    if (n1 > 0) block_unit(S, S.sd, S.vb, d);
  }
  // 5. final sides and projections on b - a
  if (tid < d) S.vs[tid] = S.vb[tid] - S.va[tid];
  __syncthreads();
  n1 = member_sides(S, H, K, m, true);
  const float mf = (float)m, n1f = (float)n1;
  if (n1f < 0.25f * mf || n1f > 0.75f * mf) {
    // lopsided: cut at the median projection (rank ties by member order)
    const int half = m / 2;
    for (int j = tid; j < m; j += kT) {
      const float pj = H.proj[j];
      int rank = 0;
      for (int i = 0; i < m; ++i) {
        const float pi = H.proj[i];
        rank += (pi < pj || (pi == pj && i < j)) ? 1 : 0;
      }
      H.side[j] = rank >= half ? 1 : 0;
    }
    __syncthreads();
  }
  // 6. both halves' summaries; relabel side 1
  member_sums(S, H, K, m, S.kr, S.sd, n1);
  float x0 = 0.f, x1 = 0.f, y0 = INFINITY, y1 = INFINITY;
  for (int j = tid; j < m; j += kT) {
    const float mg = H.smag[j];
    if (H.side[j]) { x1 = fmaxf(x1, mg); y1 = fminf(y1, mg); H.labels[H.mem[j]] = (int16_t)nw; }
    else { x0 = fmaxf(x0, mg); y0 = fminf(y0, mg); }
  }
  x0 = block_max(S, x0);
  x1 = block_max(S, x1);
  y0 = -block_max(S, -y0);
  y1 = -block_max(S, -y1);
  const int64_t r0 = (int64_t)c * d, r1 = (int64_t)nw * d;
  if (tid < d) { H.sum_dir[r0 + tid] = S.kr[tid]; H.sum_dir[r1 + tid] = S.sd[tid]; }
  block_unit(S, S.kr, S.va, d);
  block_unit(S, S.sd, S.vb, d);
  if (tid < d) {
    H.cent[r0 + tid] = S.va[tid];
    H.cent[r1 + tid] = S.vb[tid];
    if (H.dir8) { H.dir8[r0 + tid] = q8(S.va[tid]); H.dir8[r1 + tid] = q8(S.vb[tid]); }
    if (H.cent8) { H.cent8[r0 + tid] = q8(S.va[tid]); H.cent8[r1 + tid] = q8(S.vb[tid]); }
  }
  if (tid == 0) {
    H.mmax[c] = x0; H.mmax[nw] = x1;
    H.mmin[c] = y0; H.mmin[nw] = y1;
    H.count[c] = m - n1; H.count[nw] = n1;
    st.n_c[h] = nw + 1;
    st.nsplit[h] = st.nsplit[h] + 1;
  }
  __syncthreads();
}

// ---- insertion ---------------------------------------------------------------------------

template <int D>
__device__ void insert_phase(IndexSmem& S, const IndexArgs& A, int h) {
  const ssa_index_state_t& st = A.st;
  const ssa_insert_args_t& in = A.ins;
  const int tid = threadIdx.x, wave = tid >> 6, C = st.C;
  const Head H = head_view(st, h);
  const int n = in.n_dev ? *in.n_dev : in.n_host;
  const int old_end = st.end[h];
  const int new_end = max(max(n - in.window, 1), old_end);
  const int hpl = st.heads_per_layer;
  const int layer = h / hpl;
  Keys K;
  K.dt = in.k_dtype;
  K.s_kn = in.s_kn;
  K.base = reinterpret_cast<const char*>(in.k) +
           (int64_t)elem_size(in.k_dtype) * ((in.koff ? in.koff[layer] : 0) + (int64_t)(h % hpl) * in.s_kh);
  float mu_i = 0.f, ks_i = 0.f;
  if (tid < D) {
    mu_i = st.mu_ref[(int64_t)h * D + tid];
    ks_i = st.ksum[(int64_t)h * D + tid];
    S.mu[tid] = mu_i;
  }
  int n_act = st.n_c[h];
  const float cap = st.cap[h], vthr = st.vthr[h];
  __syncthreads();
  for (int p = old_end; p < new_end && n_act > 0; ++p) {
    if (tid < D) {
      const float kv = K(p, tid);
      ks_i = ks_i + kv;
      S.kr[tid] = kv - mu_i;
    }
    __syncthreads();
    if (wave == 0) {
      const float mag = sqrtf(wave_cdot(S.kr, S.kr, D));
      if (tid == 0) S.scal[0] = mag;
    }
    __syncthreads();
    const float mag = S.scal[0];
    const float magc = fmaxf(mag, 1e-12f);
    if (tid < D) S.kn[tid] = S.kr[tid] / magc;
    __syncthreads();
    float best = 0.f;
    int bi = -1;
    for (int c = tid; c < n_act; c += kT) {
      float x[D];
      if (H.q8cent) load_row<D>(H.cent8 + (int64_t)c * D, x);
      else load_row<D>(H.cent + (int64_t)c * D, x);
      const float sc = cdot([&](int i) { return x[i]; }, [&](int i) { return S.kn[i]; }, D);
      argmax_merge(best, bi, sc, c);
    }
    block_argmax(S, best, bi);
    const int row = bi;
    if (tid < D) {
      const float sd = H.sum_dir[(int64_t)row * D + tid] + S.kn[tid];
      H.sum_dir[(int64_t)row * D + tid] = sd;
      S.sd[tid] = sd;
    }
    __syncthreads();
    if (wave == 0) {
      const float sdsq = wave_cdot(S.sd, S.sd, D);
      if (tid == 0) {
        S.scal[1] = sqrtf(sdsq);
        H.mmax[row] = fmaxf(H.mmax[row], mag);
        H.mmin[row] = fminf(H.mmin[row], mag);
        const int cn = H.count[row] + 1;
        H.count[row] = cn;
        H.labels[p] = (int16_t)row;
        const float cnf = (float)cn;
        const bool wide = (1.0f - sdsq / (cnf * cnf) > vthr) && (cn >= in.var_min);
        const bool over = cnf > fmaxf(cap, in.capk * (float)p);
        S.scali[0] = ((over || wide) && n_act < C && cn >= 2 && cn <= H.ms) ? 1 : 0;
      }
    }
    __syncthreads();
    if (H.dir8 && tid < D) H.dir8[(int64_t)row * D + tid] = q8(S.sd[tid] / fmaxf(S.scal[1], 1e-12f));
    if (S.scali[0]) {
      __syncthreads();
      split_cluster(S, st, H, K, h, row, n_act, p + 1);
      n_act += 1;
    }
    __syncthreads();
  }
  // running mean vs the centring mean: drift flag; cluster count: reset flag
  const float nb = (float)(new_end - 1);
  if (tid < D) {
    st.ksum[(int64_t)h * D + tid] = ks_i;
    S.vs[tid] = ks_i / fmaxf(nb, 1.f) - mu_i;
  }
  __syncthreads();
  if (wave == 0) {
    const float dist = sqrtf(wave_cdot(S.vs, S.vs, D));
    if (tid == 0) {
      const bool moved = (dist > in.delta * st.rbar[h]) && (nb > 0.f);
      st.flags[h] = st.flags[h] | (moved ? 1 : 0) | ((n_act >= in.reset_at) ? 2 : 0);
      st.end[h] = new_end;
      S.scali[2] = new_end;
    }
  }
  __syncthreads();
}

// ---- selection -----------------------------------------------------------------------------

template <int D>
__device__ void select_phase(IndexSmem& S, const IndexArgs& A, int h, int end) {
  const ssa_index_state_t& st = A.st;
  const ssa_select_args_t& sl = A.sel;
  const int tid = threadIdx.x, G = sl.G;
  const Head H = head_view(st, h);
  const int n_act = st.n_c[h];
  const bool per_head = sl.group == 1;
  if (sl.need_out && tid == 0) {
    const int nb = end - 1;
    const double need = nb > 0 ? ceil(sl.budget * (double)nb) : 0.0;
    sl.need_out[h] = (int32_t)fmin(need, 2147483647.0);
  }
  for (int e = tid; e < G * D; e += kT) {
    const int g = e / D, i = e % D;
    S.u.sel.q[g][i] = load_as_f32(sl.q, sl.q_dtype, (int64_t)(h * G + g) * sl.s_qh + i);
  }
  __syncthreads();
  float* w = sl.w;
  const int64_t s_wr = sl.s_wr;
  select_head<D, kT, kMaxG>(S.u.sel, H, st.C, n_act, end, G, sl.budget, sl.group, sl.scale,
                            [&](int r, int c, float x) { w[(int64_t)(per_head ? h * G + r : h) * s_wr + c] = x; });
}

template <int D>
__global__ __launch_bounds__(kT) void index_kernel(IndexArgs A) {
  __shared__ IndexSmem S;
  const int h = blockIdx.x;
  int end = 0;
  if (A.do_insert) {
    insert_phase<D>(S, A, h);
    end = S.scali[2];
  } else {
    end = A.st.end[h];
  }
  if (A.do_select) select_phase<D>(S, A, h, end);
}

// ---- prefill ---------------------------------------------------------------------------------

struct BuildArgs {
  ssa_index_state_t st;
  ssa_build_args_t b;
  int nb, nblk;
  float cap_value;
};

__device__ __forceinline__ const char* head_keys(const BuildArgs& A, int h) {
  return reinterpret_cast<const char*>(A.b.k) + (int64_t)elem_size(A.b.k_dtype) * (int64_t)h * A.b.s_kh;
}

// Centre: ksum = ordered sum of the range's keys, mu = given or ksum / nb; reset the summaries.
template <typename T>
__global__ __launch_bounds__(kT) void center_kernel(BuildArgs A) {
  const int s = blockIdx.x, h = A.b.heads[s], tid = threadIdx.x;
  const int d = A.st.d, C = A.st.C, nb = A.nb;
  KeysT<T> K{reinterpret_cast<const T*>(head_keys(A, h)), A.b.s_kn};
  if (tid < d) {
    // left-to-right sum; loads are issued 32 positions ahead of the adds
    float ks = 0.f;
    int p = A.b.start;
    for (; p + 32 <= A.b.end; p += 32) {
      float v[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) v[u] = K(p + u, tid);
#pragma unroll
      for (int u = 0; u < 32; ++u) ks = ks + v[u];
    }
    for (; p < A.b.end; ++p) ks = ks + K(p, tid);
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
    A.st.end[h] = A.b.end;
    if (A.b.fit) {
      A.st.n_c[h] = A.b.C_fit;
      if (A.cap_value > 0.f) A.st.cap[h] = A.cap_value;
    }
  }
}

// Unit centred directions of the range's keys, their lengths and squared lengths.
template <typename T, int D>
__global__ __launch_bounds__(kT) void normalize_kernel(BuildArgs A) {
  const int s = blockIdx.y, h = A.b.heads[s];
  const int j = blockIdx.x * kT + threadIdx.x;
  if (j >= A.nb) return;
  KeysT<T> K{reinterpret_cast<const T*>(head_keys(A, h)), A.b.s_kn};
  const float* mu = A.st.mu_ref + (int64_t)h * D;
  const int p = A.b.start + j;
  float kr[D];
#pragma unroll
  for (int i = 0; i < D; ++i) kr[i] = K(p, i) - mu[i];
  const float sq = cdot([&](int i) { return kr[i]; }, [&](int i) { return kr[i]; }, D);
  const float mag = sqrtf(sq);
  const float magc = fmaxf(mag, 1e-12f);
  float4* x = reinterpret_cast<float4*>(A.b.xn + ((int64_t)s * A.nb + j) * D);
#pragma unroll
  for (int k = 0; k < D / 4; ++k)
    x[k] = make_float4(kr[4 * k] / magc, kr[4 * k + 1] / magc, kr[4 * k + 2] / magc, kr[4 * k + 3] / magc);
  A.b.mag[(int64_t)s * A.nb + j] = mag;
  A.b.sq[(int64_t)s * A.nb + j] = sq;
}

// rbar = sqrt(ordered sum of squared lengths / nb).
__global__ void rbar_kernel(BuildArgs A) {
  const int s = blockIdx.x, h = A.b.heads[s];
  if (threadIdx.x != 0) return;
  float t = 0.f;
  const float* sq = A.b.sq + (int64_t)s * A.nb;
  int j = 0;
  for (; j + 32 <= A.nb; j += 32) {
    float v[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) v[u] = sq[j + u];
#pragma unroll
    for (int u = 0; u < 32; ++u) t = t + v[u];
  }
  for (; j < A.nb; ++j) t = t + sq[j];
  A.st.rbar[h] = A.nb > 0 ? sqrtf(t / (float)A.nb) : 0.f;
}

// k-means seed: centroid c is the unit direction of range member init_idx[c].
__global__ __launch_bounds__(kT) void kmeans_init_kernel(BuildArgs A) {
  const int s = blockIdx.y, h = A.b.heads[s], c = blockIdx.x, d = A.st.d;
  const int j = A.b.init_idx[c];
  if (threadIdx.x < d)
    A.st.cent[((int64_t)h * A.st.C + c) * d + threadIdx.x] = A.b.xn[((int64_t)s * A.nb + j) * d + threadIdx.x];
}

// assign_j = argmax over the first n_c centroids of cdot(xn_j, cent_c), lowest index on ties.
// With write_labels the result also becomes the key's label.
template <int D>
__global__ __launch_bounds__(kT) void assign_kernel(BuildArgs A, int write_labels) {
  constexpr int CT = 32;
  __shared__ float tile[CT][D];
  const int s = blockIdx.y, h = A.b.heads[s], tid = threadIdx.x;
  const int j = blockIdx.x * kT + tid;
  const int nc = A.st.n_c[h];
  const float* cent = A.st.shared_dirs ? A.st.cent : A.st.cent + (int64_t)h * A.st.C * D;
  float x[D];
  const bool ok = j < A.nb;
  const float* xr = A.b.xn + ((int64_t)s * A.nb + (ok ? j : 0)) * D;
#pragma unroll
  for (int i = 0; i < D; ++i) x[i] = xr[i];
  float best = 0.f;
  int bi = -1;
  for (int c0 = 0; c0 < nc; c0 += CT) {
    const int nt = min(CT, nc - c0);
    __syncthreads();
    for (int e = tid; e < nt * D; e += kT) tile[e / D][e % D] = cent[(int64_t)(c0 + e / D) * D + e % D];
    __syncthreads();
    for (int r = 0; r < nt; ++r) {
      const float sc = cdot([&](int i) { return x[i]; }, [&](int i) { return tile[r][i]; }, D);
      if (bi < 0 || sc > best) { best = sc; bi = c0 + r; }
    }
  }
  if (!ok) return;
  A.b.assign[(int64_t)s * A.nb + j] = bi;
  if (write_labels) A.st.labels[(int64_t)h * A.st.capacity + A.b.start + j] = (int16_t)bi;
}

// Blocked sums, stage 1: for block b of kKB consecutive keys, per cluster, the ordered sum of its
// members' unit directions (members in position order) and the member count. With summaries,
// also fold the members' lengths into mmax / mmin (order-free max / min).
__global__ __launch_bounds__(kT) void block_sum_kernel(BuildArgs A, int ncl, int summaries) {
  __shared__ int s_as[kKB], s_order[kKB], s_start[kMaxC + 1], s_cnt[kMaxC];
  const int s = blockIdx.y, h = A.b.heads[s], b = blockIdx.x, tid = threadIdx.x, d = A.st.d;
  const int j0 = b * kKB, nk = min(kKB, A.nb - j0);
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
  const int s = blockIdx.y, h = A.b.heads[s], c = blockIdx.x, tid = threadIdx.x, d = A.st.d;
  if (tid < d) {
    float acc = 0.f;
    for (int b = 0; b < A.nblk; ++b) acc = acc + A.b.part[(((int64_t)s * A.nblk + b) * ncl + c) * d + tid];
    v[tid] = acc;
  }
  if (tid == 0) {
    int n = 0;
    for (int b = 0; b < A.nblk; ++b) n += A.b.part_cnt[((int64_t)s * A.nblk + b) * ncl + c];
    s_n = n;
  }
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
  const int s = blockIdx.y, h = A.b.heads[s], c = blockIdx.x, tid = threadIdx.x, d = A.st.d;
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

int launch_index(const IndexArgs& A, hipStream_t s) {
  const dim3 g(A.st.n_heads), b(kT);
  switch (A.st.d) {
    case 16: hipLaunchKernelGGL(index_kernel<16>, g, b, 0, s, A); break;
    case 32: hipLaunchKernelGGL(index_kernel<32>, g, b, 0, s, A); break;
    case 64: hipLaunchKernelGGL(index_kernel<64>, g, b, 0, s, A); break;
    case 128: hipLaunchKernelGGL(index_kernel<128>, g, b, 0, s, A); break;
    case 256: hipLaunchKernelGGL(index_kernel<256>, g, b, 0, s, A); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

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

extern "C" int ssa_build(const ssa_index_state_t* st, const ssa_build_args_t* b, void* stream) {
  if (!state_ok(st) || !b || b->n_sel < 1 || b->start < 0 || b->end < b->start || b->end > st->capacity)
    return hipErrorInvalidValue;
  if (b->fit && (b->C_fit < 1 || b->C_fit > st->C || b->C_fit > kKB * 4 || !b->init_idx)) return hipErrorInvalidValue;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  BuildArgs A{};
  A.st = *st;
  A.b = *b;
  A.nb = b->end - b->start;
  A.nblk = (A.nb + kKB - 1) / kKB;
  A.cap_value = 0.f;
  switch (b->k_dtype) {
    case kBF16: hipLaunchKernelGGL(center_kernel<__hip_bfloat16>, dim3(b->n_sel), dim3(kT), 0, s, A); break;
    case kF16: hipLaunchKernelGGL(center_kernel<__half>, dim3(b->n_sel), dim3(kT), 0, s, A); break;
    default: hipLaunchKernelGGL(center_kernel<float>, dim3(b->n_sel), dim3(kT), 0, s, A); break;
  }
  if (A.nb > 0) {
    dim3 gk((A.nb + kT - 1) / kT, b->n_sel);
    auto normalize = [&](auto tag) {
      using T = decltype(tag);
      switch (st->d) {
        case 16: hipLaunchKernelGGL((normalize_kernel<T, 16>), gk, dim3(kT), 0, s, A); break;
        case 32: hipLaunchKernelGGL((normalize_kernel<T, 32>), gk, dim3(kT), 0, s, A); break;
        case 64: hipLaunchKernelGGL((normalize_kernel<T, 64>), gk, dim3(kT), 0, s, A); break;
        case 128: hipLaunchKernelGGL((normalize_kernel<T, 128>), gk, dim3(kT), 0, s, A); break;
        case 256: hipLaunchKernelGGL((normalize_kernel<T, 256>), gk, dim3(kT), 0, s, A); break;
      }
    };
    if (b->k_dtype == kBF16) normalize(__hip_bfloat16{});
    else if (b->k_dtype == kF16) normalize(__half{});
    else normalize(0.f);
    hipLaunchKernelGGL(rbar_kernel, dim3(b->n_sel), dim3(64), 0, s, A);
    auto assign = [&](int write_labels) {
      switch (st->d) {
        case 16: hipLaunchKernelGGL(assign_kernel<16>, gk, dim3(kT), 0, s, A, write_labels); break;
        case 32: hipLaunchKernelGGL(assign_kernel<32>, gk, dim3(kT), 0, s, A, write_labels); break;
        case 64: hipLaunchKernelGGL(assign_kernel<64>, gk, dim3(kT), 0, s, A, write_labels); break;
        case 128: hipLaunchKernelGGL(assign_kernel<128>, gk, dim3(kT), 0, s, A, write_labels); break;
        case 256: hipLaunchKernelGGL(assign_kernel<256>, gk, dim3(kT), 0, s, A, write_labels); break;
      }
    };
    if (b->fit && !st->shared_dirs) {
      hipLaunchKernelGGL(kmeans_init_kernel, dim3(b->C_fit, b->n_sel), dim3(kT), 0, s, A);
      for (int it = 0; it < b->iters; ++it) {
        assign(0);
        hipLaunchKernelGGL(block_sum_kernel, dim3(A.nblk, b->n_sel), dim3(kT), 0, s, A, b->C_fit, 0);
        hipLaunchKernelGGL(block_reduce_kernel, dim3(b->C_fit, b->n_sel), dim3(kT), 0, s, A, b->C_fit, 0);
      }
    }
    assign(1);
    hipLaunchKernelGGL(block_sum_kernel, dim3(A.nblk, b->n_sel), dim3(kT), 0, s, A, st->C, 1);
    hipLaunchKernelGGL(block_reduce_kernel, dim3(st->C, b->n_sel), dim3(kT), 0, s, A, st->C, 1);
  }
  if (st->dir8 || st->cent8) hipLaunchKernelGGL(refresh8_kernel, dim3(st->C, b->n_sel), dim3(kT), 0, s, A);
  return hipGetLastError();
}
