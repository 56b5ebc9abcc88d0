// Insertion of keys into their nearest cluster and the in-kernel split of a cluster that
// passes its cap, for one (layer, sequence, KV head) per workgroup of kT threads. Used by the
// insertion kernel (index.hip) and by the tail of the fused decode step (decode.h).
//
// Reference behaviour:
//   insertion  _bin_kernel / _bin_dev_kernel    src/ssa/kernels/sphere_fused.py:171-227,
//                                               src/ssa/kernels/graph_kernels.py:63-130
//   split      _split_cluster                   src/ssa/kernels/sphere_fused.py:49-167
//              (rule of _bisect_padded,         src/ssa/attn/sphere_gpu.py:76-102)
// Every decision is made in the canonical arithmetic of ssa_common.h.
#pragma once

#include "select.h"

namespace ssa {

constexpr int kT = 256;       // threads per workgroup
constexpr int kW = kT / 64;   // waves
constexpr int kTile = 16;     // member rows of kMaxD staged in LDS by the split's ordered sums
constexpr int kTileFloats = kTile * kMaxD;   // a tile holds kTileFloats / d rows of d
constexpr int kGatherRun = 32;  // consecutive label positions per thread per pass of the member scan

// LDS of the insertion and split code. A kernel that runs them passes a struct with the members
// of InsertSmem (its own may add more to the union u, which must hold spl).
constexpr int kRankLds = 512;   // members whose projections a lopsided split ranks from LDS
static_assert(kRankLds <= kTileFloats, "the ranking reuses the tile");

struct SplitTile {
  union {
    float tile[kTileFloats];
    float rank[kRankLds];         // the lopsided split's projections (the tile is idle then)
  };
  int tside[kTileFloats / 8];
};

struct InsertBase {
  float mu[kMaxD], kr[kMaxD], kn[kMaxD], sd[kMaxD];
  float va[kMaxD], vb[kMaxD], vs[kMaxD];
  float red_f[kW];
  int red_i[kW];
  float scal[4];
  int scali[4];
  float rmx, rmn;          // summaries of the cluster a key joins
  int rcnt;
  int8_t d8[kMaxD];        // its new int8 direction, staged
};

struct InsertSmem : InsertBase {
  union {
    SplitTile spl;
  } u;
};

__device__ __forceinline__ int elem_size(int dt) { return dt == kF32 ? 4 : 2; }

// ---- workgroup reductions (results are uniform across the workgroup) -----------------------

template <class SM>
__device__ __forceinline__ void block_argmax(SM& S, float& s, int& i) {
  wave_argmax(s, i);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { S.red_f[w] = s; S.red_i[w] = i; }
  __syncthreads();
  s = S.red_f[0]; i = S.red_i[0];
  for (int w2 = 1; w2 < kW; ++w2) argmax_merge(s, i, S.red_f[w2], S.red_i[w2]);
  __syncthreads();
}

template <class SM>
__device__ __forceinline__ void block_argmin(SM& S, float& s, int& i) {
  wave_argmin(s, i);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { S.red_f[w] = s; S.red_i[w] = i; }
  __syncthreads();
  s = S.red_f[0]; i = S.red_i[0];
  for (int w2 = 1; w2 < kW; ++w2) argmin_merge(s, i, S.red_f[w2], S.red_i[w2]);
  __syncthreads();
}

template <class SM>
__device__ __forceinline__ float block_max(SM& S, float v) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) S.red_f[w] = v;
  __syncthreads();
  float r = S.red_f[0];
  for (int w2 = 1; w2 < kW; ++w2) r = fmaxf(r, S.red_f[w2]);
  __syncthreads();
  return r;
}

template <class SM>
__device__ __forceinline__ int block_sum_i(SM& S, int v) {
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
template <class SM>
__device__ __forceinline__ void block_unit(SM& S, const float* x, float* y, int d) {
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

// cdot with the loop over 8-element steps kept rolled (the split's operands are computed per
// element from the key cache, and unrolled copies of that would hold many registers).
template <typename FA, typename FB>
__device__ __forceinline__ float cdot_rolled(FA a, FB b, int d) {
  float c0 = 0.f, c1 = 0.f, c2 = 0.f, c3 = 0.f, c4 = 0.f, c5 = 0.f, c6 = 0.f, c7 = 0.f;
#pragma unroll 1
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

// Eight consecutive elements [i0, i0 + 8) of key row pos as fp32 (i0 a multiple of 8). With v16
// (16-byte aligned rows) one 16-byte load for 2-byte keys, two for fp32; else element loads.
__device__ __forceinline__ void load8(const Keys& K, bool v16, int pos, int i0, float (&x)[8]) {
  const int64_t off = (int64_t)pos * K.s_kn + i0;
  if (v16 && K.dt != kF32) {
    const uint4 r = *reinterpret_cast<const uint4*>(K.base + off * 2);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (K.dt == kBF16) {
        x[2 * k] = __uint_as_float(w[k] << 16);
        x[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
      } else {
        x[2 * k] = __half2float(__ushort_as_half((unsigned short)(w[k] & 0xffffu)));
        x[2 * k + 1] = __half2float(__ushort_as_half((unsigned short)(w[k] >> 16)));
      }
    }
  } else if (v16) {
    const float4 a = *reinterpret_cast<const float4*>(K.base + off * 4);
    const float4 b = *reinterpret_cast<const float4*>(K.base + off * 4 + 16);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = load_as_f32(K.base, K.dt, off + j);
  }
}

__device__ __forceinline__ bool keys_vec16(const Keys& K) {
  const int64_t es = elem_size(K.dt);
  return (reinterpret_cast<uintptr_t>(K.base) & 15) == 0 && ((K.s_kn * es) & 15) == 0;
}

// Canonical dots over one member's key row, two 8-element chunks loaded per round. With
// unit, kn = (K(pos, i) - mu[i]) / magc is dotted with each of the NV vectors v[0..NV);
// otherwise out[0] = dot(kr, kr) with kr = K(pos, i) - mu[i].
template <int NV, bool UNIT>
__device__ __forceinline__ void member_dots(const Keys& K, bool v16, int pos, const float* mu, float magc,
                                            const float* const (&v)[NV], int d, float (&out)[NV]) {
  float c[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) c[k][j] = 0.f;
#pragma unroll 1
  for (int i0 = 0; i0 < d; i0 += 16) {
    float x[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (i0 + 8 * u < d) load8(K, v16, pos, i0 + 8 * u, x[u]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (i0 + 8 * u < d) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int i = i0 + 8 * u + j;
          const float kr = x[u][j] - mu[i];
          if constexpr (UNIT) {
            const float kn = kr / magc;
#pragma unroll
            for (int k = 0; k < NV; ++k) c[k][j] = __builtin_fmaf(kn, v[k][i], c[k][j]);
          } else {
            c[0][j] = __builtin_fmaf(kr, kr, c[0][j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) out[k] = ((c[k][0] + c[k][1]) + (c[k][2] + c[k][3])) + ((c[k][4] + c[k][5]) + (c[k][6] + c[k][7]));
}

// The same dots over a member's staged unit direction (H.kn row j), for splits whose members'
// directions were computed once: the values are those member_dots computes, so are the dots.
template <int NV>
__device__ __forceinline__ void kn_dots(const Head& H, int j, const float* const (&v)[NV], int d, float (&out)[NV]) {
  float c[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) c[k][e] = 0.f;
  const float* r = H.kn + (int64_t)j * d;
#pragma unroll 1
  for (int i0 = 0; i0 < d; i0 += 16) {
    float4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i0 + 4 * u < d) x[u] = reinterpret_cast<const float4*>(r + i0)[u];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i0 + 4 * u < d) {
        const float xs[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = i0 + 4 * u + e;
#pragma unroll
          for (int k = 0; k < NV; ++k) c[k][(4 * u + e) & 7] = __builtin_fmaf(xs[e], v[k][i], c[k][(4 * u + e) & 7]);
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NV; ++k) out[k] = ((c[k][0] + c[k][1]) + (c[k][2] + c[k][3])) + ((c[k][4] + c[k][5]) + (c[k][6] + c[k][7]));
}

// Member tiles for the ordered sums: kMemberChunks 8-element chunks per thread, so a tile holds
// kT * 8 * kMemberChunks / d member rows of d. fetch loads a tile's raw keys into registers (the
// next tile's load overlaps the current tile's sums); store writes their unit directions
// kn = (k - mu) / max(|k - mu|, 1e-12) into LDS, row r at tile[r * d].
constexpr int kMemberChunks = 1;
static_assert(kT * 8 * kMemberChunks <= kTileFloats, "member tile too large for the LDS tile");

struct MemberTile {
  float x[kMemberChunks][8];
  __device__ __forceinline__ static int rows(int d) { return kT * 8 * kMemberChunks / d; }
  __device__ __forceinline__ void fetch(const Head& H, const Keys& K, bool v16, int m, int t0) {
    const int d = H.d, cpr = d / 8, nq = min(rows(d), m - t0) * cpr;
#pragma unroll
    for (int ch = 0; ch < kMemberChunks; ++ch) {
      const int q = threadIdx.x + ch * kT;
      if (q < nq) load8(K, v16, H.mem[t0 + q / cpr], 8 * (q % cpr), x[ch]);
    }
  }
  __device__ __forceinline__ void store(const Head& H, const float* mu, float* tile, int m, int t0) const {
    const int d = H.d, cpr = d / 8, nq = min(rows(d), m - t0) * cpr;
#pragma unroll
    for (int ch = 0; ch < kMemberChunks; ++ch) {
      const int q = threadIdx.x + ch * kT;
      if (q < nq) {
        const int r = q / cpr, i0 = 8 * (q % cpr);
        const float magc = fmaxf(H.smag[t0 + r], 1e-12f);
#pragma unroll
        for (int e = 0; e < 8; ++e) tile[r * d + i0 + e] = (x[ch][e] - mu[i0 + e]) / magc;
      }
    }
  }
};

// Side sums of the members' unit directions kn_j = (k_j - mu) / max(|k_j - mu|, 1e-12) for the
// cluster being split: members in blocks of kSumBlock (member order), each block's side sums left
// to right from +0, the block sums added left to right from +0 (s0: side 0, s1: side 1). A round
// takes as many blocks as their partials fit in the LDS tile; within it each thread owns one
// (block, 8-element chunk) and reads the chunk of every member of its block with 16-byte loads,
// then thread i adds the round's block partials of dimension i in block order.
constexpr int kSumBlock = 16;
template <class SM>
__device__ __forceinline__ void member_sums(SM& S, const Head& H, const Keys& K, bool v16, int m, float* s0_out,
                                            float* s1_out, int& n1_out, bool staged = false) {
  const int tid = threadIdx.x, d = H.d, cpr = d / 8;
  const int nbr = kTileFloats / (2 * d);
  float* part = S.u.spl.tile;                        // [2][nbr][d]
  float s0 = 0.f, s1 = 0.f;
  for (int j0 = 0; j0 < m; j0 += nbr * kSumBlock) {
    const int nb = min(nbr, (m - j0 + kSumBlock - 1) / kSumBlock);
    for (int it = tid; it < nb * cpr; it += kT) {
      const int b = it / cpr, i0 = 8 * (it % cpr);
      const int jb = j0 + b * kSumBlock, je = min(jb + kSumBlock, m);
      float a0[8], a1[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) { a0[e] = 0.f; a1[e] = 0.f; }
      if (staged) {
        // the members' unit directions, staged: 4 members' chunks in flight, added in member order
        for (int jb8 = jb; jb8 < je; jb8 += 4) {
          float4 xa[4], xb[4];
          bool one[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float* r = H.kn + (int64_t)min(jb8 + t, je - 1) * d + i0;
            xa[t] = reinterpret_cast<const float4*>(r)[0];
            xb[t] = reinterpret_cast<const float4*>(r)[1];
            one[t] = H.side[min(jb8 + t, je - 1)] != 0;
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if (jb8 + t < je) {
              const float kn[8] = {xa[t].x, xa[t].y, xa[t].z, xa[t].w, xb[t].x, xb[t].y, xb[t].z, xb[t].w};
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                if (one[t]) a1[e] = a1[e] + kn[e]; else a0[e] = a0[e] + kn[e];
              }
            }
          }
        }
      } else {
#pragma unroll 2
        for (int j = jb; j < je; ++j) {
          float x[8];
          load8(K, v16, H.mem[j], i0, x);
          const float magc = fmaxf(H.smag[j], 1e-12f);
          const bool one = H.side[j] != 0;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float kn = (x[e] - S.mu[i0 + e]) / magc;
            if (one) a1[e] = a1[e] + kn; else a0[e] = a0[e] + kn;
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        part[b * d + i0 + e] = a0[e];
        part[(nbr + b) * d + i0 + e] = a1[e];
      }
    }
    __syncthreads();
    if (tid < d)
      for (int b = 0; b < nb; ++b) {
        s0 = s0 + part[b * d + tid];
        s1 = s1 + part[(nbr + b) * d + tid];
      }
    __syncthreads();
  }
  int n1 = 0;
  for (int j = tid; j < m; j += kT) n1 += H.side[j] != 0 ? 1 : 0;
  n1 = block_sum_i(S, n1);
  if (tid < d) { s0_out[tid] = s0; s1_out[tid] = s1; }
  __syncthreads();
  n1_out = n1;
}

// side_j = kn_j.b > kn_j.a for every member (canonical dots), stored in H.side; returns #side 1.
template <class SM>
__device__ __forceinline__ int member_sides(SM& S, const Head& H, const Keys& K, bool v16, int m, bool with_proj,
                                            bool staged = false) {
  const int tid = threadIdx.x, d = H.d;
  int n1 = 0;
  for (int j = tid; j < m; j += kT) {
    int one;
    if (with_proj) {
      const float* const v[3] = {S.va, S.vb, S.vs};
      float o[3];
      if (staged) kn_dots<3>(H, j, v, d, o);
      else member_dots<3, true>(K, v16, H.mem[j], S.mu, fmaxf(H.smag[j], 1e-12f), v, d, o);
      one = o[1] > o[0] ? 1 : 0;
      H.proj[j] = o[2];
    } else {
      const float* const v[2] = {S.va, S.vb};
      float o[2];
      if (staged) kn_dots<2>(H, j, v, d, o);
      else member_dots<2, true>(K, v16, H.mem[j], S.mu, fmaxf(H.smag[j], 1e-12f), v, d, o);
      one = o[1] > o[0] ? 1 : 0;
    }
    H.side[j] = one;
    n1 += one;
  }
  return block_sum_i(S, n1);
}

// Positions of cluster c among [lo, hi), ascending, into H.mem[0 .. m) (at most H.ms); returns m.
// Each pass gives every thread kGatherRun consecutive positions (16-byte label loads where a
// chunk of 8 lies inside [lo, hi), element loads at the two ends), the threads' runs in order;
// an exclusive scan of the per-thread hit counts places every member.
template <class SM>
__device__ __forceinline__ int gather_members(SM& S, const Head& H, int c, int lo, int hi) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (lo >= hi) return 0;
  // the row starts `mis` positions past a 16-byte boundary; a0 <= lo is the aligned start
  const int mis = (int)((reinterpret_cast<uintptr_t>(H.labels) >> 1) & 7);
  const int a0 = lo - ((lo + mis) & 7);
  int m = 0;
  for (int p0 = a0; p0 < hi; p0 += kT * kGatherRun) {
    const int pb = p0 + tid * kGatherRun;
    unsigned int bits = 0;
#pragma unroll
    for (int q = 0; q < kGatherRun / 8; ++q) {
      const int ps = pb + 8 * q;
      int lab[8];
      if (ps >= lo && ps + 8 <= hi) {
        const uint4 r = *reinterpret_cast<const uint4*>(H.labels + ps);
        const int16_t* v = reinterpret_cast<const int16_t*>(&r);
#pragma unroll
        for (int e = 0; e < 8; ++e) lab[e] = v[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = ps + e;
          lab[e] = (j >= lo && j < hi) ? (int)H.labels[j] : -1;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) bits |= (lab[e] == c ? 1u : 0u) << (8 * q + e);
    }
    const int cnt = __popc(bits);
    const int incl = wave_incl_scan_dpp(cnt);
    if (lane == 63) S.red_i[wave] = incl;
    __syncthreads();
    int wb = 0, tot = 0;
#pragma unroll
    for (int w2 = 0; w2 < kW; ++w2) {
      const int v = S.red_i[w2];
      if (w2 < wave) wb += v;
      tot += v;
    }
    int slot = m + wb + incl - cnt;
    while (bits) {
      const int k = __ffs(bits) - 1;
      bits &= bits - 1;
      if (slot < H.ms) H.mem[slot] = pb + k;
      ++slot;
    }
    m += tot;
    __syncthreads();
  }
  return min(m, H.ms);
}

// Inlined (a call would put the caller's arguments and frame in scratch, whose set-up costs
// every launch of the kernel); its dot loops stay rolled to keep registers down.
template <class SM>
__device__ __forceinline__ void split_cluster(SM& S, const ssa_index_state_t& st, const Head& H, const Keys& K, int h,
                              int c, int nw, int stop) {
  const int tid = threadIdx.x, d = H.d;
  const bool v16 = keys_vec16(K);
  // 1. members in ascending position order
  const int m = gather_members(S, H, c, 1, stop);
  if (m < 2) return;   // labels and counts disagree: leave the cluster as it is
  // 2. lengths
  for (int j = tid; j < m; j += kT) {
    const float* const none[1] = {nullptr};
    float sq[1];
    member_dots<1, false>(K, v16, H.mem[j], S.mu, 1.f, none, d, sq);
    H.smag[j] = sqrtf(sq[0]);
  }
  __syncthreads();
  // With room in the state, every member's unit direction (k - mu) / max(|k - mu|, 1e-12) is
  // computed once here and read by the passes below, which otherwise divide every element again.
  const bool staged = H.kn && m <= H.kn_rows;
  if (staged) {
    const int cpr = d / 8, nq = m * cpr;
    for (int q0 = tid; q0 < nq; q0 += 2 * kT) {
      float x[2][8], magc[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {                   // two chunks' loads in flight
        const int q = min(q0 + t * kT, nq - 1);
        load8(K, v16, H.mem[q / cpr], 8 * (q % cpr), x[t]);
        magc[t] = fmaxf(H.smag[q / cpr], 1e-12f);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int q = q0 + t * kT;
        if (q < nq) {
          const int j = q / cpr, i0 = 8 * (q % cpr);
          float u[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) u[e] = (x[t][e] - S.mu[i0 + e]) / magc[t];
          float4* r = reinterpret_cast<float4*>(H.kn + (int64_t)j * d + i0);
          r[0] = make_float4(u[0], u[1], u[2], u[3]);
          r[1] = make_float4(u[4], u[5], u[6], u[7]);
        }
      }
    }
    __syncthreads();
  }
  // 3. start from the first member and the member least similar to it
  if (tid < d) S.va[tid] = staged ? H.kn[tid] : (K(H.mem[0], tid) - S.mu[tid]) / fmaxf(H.smag[0], 1e-12f);
  __syncthreads();
  float lo = 0.f;
  int far = -1;
  for (int j = tid; j < m; j += kT) {
    const float* const v[1] = {S.va};
    float o[1];
    if (staged) kn_dots<1>(H, j, v, d, o);
    else member_dots<1, true>(K, v16, H.mem[j], S.mu, fmaxf(H.smag[j], 1e-12f), v, d, o);
    argmin_merge(lo, far, o[0], j);
  }
  block_argmin(S, lo, far);
  if (tid < d)
    S.vb[tid] = staged ? H.kn[(int64_t)far * d + tid] : (K(H.mem[far], tid) - S.mu[tid]) / fmaxf(H.smag[far], 1e-12f);
  __syncthreads();
  // 4. 2-means on cosine similarity, 4 iterations
  int n1 = 0;
  for (int it = 0; it < 4; ++it) {
    member_sides(S, H, K, v16, m, false, staged);
    __syncthreads();
    member_sums(S, H, K, v16, m, S.kr, S.sd, n1, staged);
    if (m - n1 > 0) block_unit(S, S.kr, S.va, d);
    if (n1 > 0) block_unit(S, S.sd, S.vb, d);
  }
  // 5. final sides and projections on b - a
  if (tid < d) S.vs[tid] = S.vb[tid] - S.va[tid];
  __syncthreads();
  n1 = member_sides(S, H, K, v16, m, true, staged);
  const float mf = (float)m, n1f = (float)n1;
  if (n1f < 0.25f * mf || n1f > 0.75f * mf) {
    // lopsided: cut at the median projection (rank ties by member order)
    const int half = m / 2;
    // the projections in LDS for the m^2 comparisons when they fit
    const float* pr = H.proj;
    if (m <= kRankLds) {
      for (int j = tid; j < m; j += kT) S.u.spl.rank[j] = H.proj[j];
      __syncthreads();
      pr = S.u.spl.rank;
    }
    for (int j = tid; j < m; j += kT) {
      const float pj = pr[j];
      int rank = 0;
      for (int i = 0; i < m; ++i) {
        const float pi = pr[i];
        rank += (pi < pj || (pi == pj && i < j)) ? 1 : 0;
      }
      H.side[j] = rank >= half ? 1 : 0;
    }
    __syncthreads();
  }
  // 6. both halves' summaries; relabel side 1
  member_sums(S, H, K, v16, m, S.kr, S.sd, n1, staged);
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

// What an insertion reads before it knows the cluster a key joins, loaded in one round: the
// head's scalars, element threadIdx.x of the centring mean, of the running key sum and of the key
// at the expected position (the one that leaves the window when one key leaves per step), and
// the centroid row and summaries of cluster threadIdx.x.
template <int D>
struct InsPre {
  int old_end, n_act, flags;
  float cap, vthr, rbar;
  float mu, ks, kv;
  int4 c8[D / 16];
  int cnt;
  float mx, mn;
};

__device__ __forceinline__ Keys head_keys_of(const ssa_index_state_t& st, const ssa_insert_args_t& in, int h) {
  const int hpl = st.heads_per_layer;
  const int layer = h / hpl;
  Keys K;
  K.dt = in.k_dtype;
  K.s_kn = in.s_kn;
  K.base = reinterpret_cast<const char*>(in.k) +
           (int64_t)elem_size(in.k_dtype) * ((in.koff ? in.koff[layer] : 0) + (int64_t)(h % hpl) * in.s_kh);
  return K;
}

// Expected position of the key to insert at length n: the last one of [end, max(n - window, 1)).
__device__ __forceinline__ int expected_key(const ssa_insert_args_t& in, int n) { return max(n - in.window, 1) - 1; }

template <int D>
__device__ __forceinline__ void insert_prefetch(InsPre<D>& P, const ssa_index_state_t& st, const ssa_insert_args_t& in,
                                                int h, int n) {
  const int tid = threadIdx.x;
  const Head H = head_view(st, h);
  P.old_end = st.end[h];
  P.n_act = st.n_c[h];
  P.flags = st.flags[h];
  P.cap = st.cap[h];
  P.vthr = st.vthr[h];
  P.rbar = st.rbar[h];
  P.mu = 0.f; P.ks = 0.f; P.kv = 0.f;
  if (tid < D) {
    P.mu = st.mu_ref[(int64_t)h * D + tid];
    P.ks = st.ksum[(int64_t)h * D + tid];
    P.kv = head_keys_of(st, in, h)(expected_key(in, n), tid);
  }
  P.cnt = 0; P.mx = 0.f; P.mn = 0.f;
  if (tid < st.C) {
    P.cnt = H.count[tid];
    P.mx = H.mmax[tid];
    P.mn = H.mmin[tid];
    if (H.q8cent) {
#pragma unroll
      for (int k = 0; k < D / 16; ++k) P.c8[k] = reinterpret_cast<const int4*>(H.cent8 + (int64_t)tid * D)[k];
    }
  }
}

// Insert the keys of [end, max(n - window, 1)) of head h into their nearest clusters (lowest
// index on ties), splitting a cluster that passes its cap, then update end and the drift /
// reset flags. P holds insert_prefetch(st, in, h, n). With one key to insert (the usual decode
// step) the only load after P is the joined cluster's fp32 direction sum.
template <int D, class SM>
__device__ __forceinline__ void insert_phase(SM& S, const ssa_index_state_t& st, const ssa_insert_args_t& in, int h,
                             const InsPre<D>& P, int n) {
  const int tid = threadIdx.x, wave = tid >> 6, C = st.C;
  const Head H = head_view(st, h);
  const int old_end = P.old_end;
  const int new_end = max(max(n - in.window, 1), old_end);
  const int p_pre = expected_key(in, n);
  const Keys K = head_keys_of(st, in, h);
  const float mu_i = P.mu;
  float ks_i = P.ks;
  if (tid < D) S.mu[tid] = mu_i;
  int n_act = P.n_act;
  const float cap = P.cap, vthr = P.vthr;
  __syncthreads();
  for (int p = old_end; p < new_end && n_act > 0; ++p) {
    const bool first = p == old_end;          // nothing written yet: the prefetched rows are current
    if (tid < D) {
      const float kv = p == p_pre ? P.kv : K(p, tid);
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
    const float (*kn)[kMaxD] = reinterpret_cast<const float (*)[kMaxD]>(S.kn);
    // canonical dots <cent_c, kn> (the row's self-dot comes along unused); cluster threadIdx.x
    // first, from its prefetched row on the first key (outside the loop, so that the row's
    // conversion is not hoisted into registers for every iteration)
    if (tid < n_act) {
      float nrm2, sc[1];
      if (H.q8cent && first) {
        int4 raw[D / 16];
#pragma unroll
        for (int k = 0; k < D / 16; ++k) {
          raw[k] = P.c8[k];
          asm volatile("" : "+v"(raw[k].x), "+v"(raw[k].y), "+v"(raw[k].z), "+v"(raw[k].w));   // not hoisted
        }
        row_dots_raw<D, 1>(raw, kn, 1, nrm2, sc);
      } else if (H.q8cent) {
        row_dots<D, 1>(H.cent8 + (int64_t)tid * D, kn, 1, nrm2, sc);
      } else {
        row_dots<D, 1>(H.cent + (int64_t)tid * D, kn, 1, nrm2, sc);
      }
      argmax_merge(best, bi, sc[0], tid);
    }
    for (int c = tid + kT; c < n_act; c += kT) {
      float nrm2, sc[1];
      if (H.q8cent) row_dots<D, 1>(H.cent8 + (int64_t)c * D, kn, 1, nrm2, sc);
      else row_dots<D, 1>(H.cent + (int64_t)c * D, kn, 1, nrm2, sc);
      argmax_merge(best, bi, sc[0], c);
    }
    block_argmax(S, best, bi);
    const int row = bi;
    if (tid < D) {
      const float sd = H.sum_dir[(int64_t)row * D + tid] + S.kn[tid];
      H.sum_dir[(int64_t)row * D + tid] = sd;
      S.sd[tid] = sd;
    }
    // the joined cluster's summaries: from its thread's prefetch, else from memory
    const bool held = first && row < kT;
    if (held && tid == row) { S.rmx = P.mx; S.rmn = P.mn; S.rcnt = P.cnt; }
    if (!held && tid == 0) { S.rmx = H.mmax[row]; S.rmn = H.mmin[row]; S.rcnt = H.count[row]; }
    __syncthreads();
    if (wave == 0) {
      const float sdsq = wave_cdot(S.sd, S.sd, D);
      if (tid == 0) {
        S.scal[1] = sqrtf(sdsq);
        H.mmax[row] = fmaxf(S.rmx, mag);
        H.mmin[row] = fminf(S.rmn, mag);
        const int cn = S.rcnt + 1;
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
      const bool moved = (dist > in.delta * P.rbar) && (nb > 0.f);
      st.flags[h] = P.flags | (moved ? 1 : 0) | ((n_act >= in.reset_at) ? 2 : 0);
      st.end[h] = new_end;
      S.scali[2] = new_end;
    }
  }
  __syncthreads();
}

// ---- insertion staged beside the decode step ------------------------------------------------
//
// ssa_sparse_step's insert-ahead workgroup prepares the insertion of the next step's key while
// the attention workgroups of its head still read the index state: it writes what they do not
// read (the joined cluster's fp32 direction sum, the running key sum) and stages the rest in
// st.stage; the head's last workgroup, once every other one is done, commits the staged values
// (and runs a split, or the general insertion when the step is not the usual one key).
constexpr int kStageWords = SSA_STAGE_WORDS;
constexpr int kStageHead = 12;       // header words before the int8 direction row
enum StageStatus { kStageNone = 0, kStageOne = 1, kStageGeneral = 2, kStageSplit = 3 };
// header: [0] status, [1] cluster, [2] position, [3] new end, [4] count, [5] mmax, [6] mmin,
//         [7] clusters in use, [8] flags

__device__ __forceinline__ void stage_put(int32_t* stg, int i, int v) {
  __hip_atomic_store(stg + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int stage_get(const int32_t* stg, int i) {
  return __hip_atomic_load(stg + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stage the insertion at length n. Takes the one-key path when exactly the prefetched key
// leaves the window and scoring reads the int8 directions; anything else is left to the commit
// (kStageGeneral), which then runs insert_phase itself.
template <int D, class SM>
__device__ __forceinline__ void insert_stage(SM& S, const ssa_index_state_t& st, const ssa_insert_args_t& in, int h,
                                             const InsPre<D>& P, int n) {
  static_assert(kStageHead + D / 4 <= kStageWords, "stage row too short");
  const int tid = threadIdx.x, wave = tid >> 6, C = st.C;
  const Head H = head_view(st, h);
  int32_t* stg = st.stage + (int64_t)h * kStageWords;
  const int old_end = P.old_end;
  const int new_end = max(max(n - in.window, 1), old_end);
  const int n_act = P.n_act;
  const int p = old_end;
  if (!(new_end == old_end + 1 && n_act > 0 && H.q8dirs && p == expected_key(in, n))) {
    if (tid == 0) stage_put(stg, 0, kStageGeneral);
    return;
  }
  const float mu_i = P.mu;
  float ks_i = P.ks;
  if (tid < D) {
    ks_i = ks_i + P.kv;
    S.kr[tid] = P.kv - mu_i;
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
  const float (*kn)[kMaxD] = reinterpret_cast<const float (*)[kMaxD]>(S.kn);
  if (tid < n_act) {
    float nrm2, sc[1];
    if (H.q8cent) {
      int4 raw[D / 16];
#pragma unroll
      for (int k = 0; k < D / 16; ++k) raw[k] = P.c8[k];
      row_dots_raw<D, 1>(raw, kn, 1, nrm2, sc);
    } else {
      row_dots<D, 1>(H.cent + (int64_t)tid * D, kn, 1, nrm2, sc);
    }
    argmax_merge(best, bi, sc[0], tid);
  }
  for (int c = tid + kT; c < n_act; c += kT) {
    float nrm2, sc[1];
    if (H.q8cent) row_dots<D, 1>(H.cent8 + (int64_t)c * D, kn, 1, nrm2, sc);
    else row_dots<D, 1>(H.cent + (int64_t)c * D, kn, 1, nrm2, sc);
    argmax_merge(best, bi, sc[0], c);
  }
  block_argmax(S, best, bi);
  const int row = bi;
  if (tid < D) S.sd[tid] = H.sum_dir[(int64_t)row * D + tid] + S.kn[tid];
  if (row < kT && tid == row) { S.rmx = P.mx; S.rmn = P.mn; S.rcnt = P.cnt; }
  if (row >= kT && tid == 0) { S.rmx = H.mmax[row]; S.rmn = H.mmin[row]; S.rcnt = H.count[row]; }
  __syncthreads();
  if (wave == 0) {
    const float sdsq = wave_cdot(S.sd, S.sd, D);
    if (tid == 0) {
      S.scal[1] = sqrtf(sdsq);
      const int cn = S.rcnt + 1;
      const float cnf = (float)cn;
      const bool wide = (1.0f - sdsq / (cnf * cnf) > P.vthr) && (cn >= in.var_min);
      const bool over = cnf > fmaxf(P.cap, in.capk * (float)p);
      const bool split = (over || wide) && n_act < C && cn >= 2 && cn <= H.ms;
      S.scali[0] = split ? 1 : 0;
      stage_put(stg, 0, split ? kStageSplit : kStageOne);
      stage_put(stg, 1, row);
      stage_put(stg, 2, p);
      stage_put(stg, 3, new_end);
      stage_put(stg, 4, cn);
      stage_put(stg, 5, __float_as_int(fmaxf(S.rmx, mag)));
      stage_put(stg, 6, __float_as_int(fminf(S.rmn, mag)));
      stage_put(stg, 7, n_act);
    }
  }
  __syncthreads();
  // The fp32 direction sum is written now (the attention reads only the int8 copy) unless the
  // cluster splits: the commit's split then rewrites it, and a write from here could reach
  // memory after the split's (another XCD's L2 may write its line back later).
  if (tid < D && !S.scali[0]) H.sum_dir[(int64_t)row * D + tid] = S.sd[tid];
  if (tid < D) S.d8[tid] = q8(S.sd[tid] / fmaxf(S.scal[1], 1e-12f));
  // running mean vs the centring mean: drift flag; cluster count: reset flag
  const float nb = (float)(new_end - 1);
  if (tid < D) {
    st.ksum[(int64_t)h * D + tid] = ks_i;
    S.vs[tid] = ks_i / fmaxf(nb, 1.f) - mu_i;
  }
  __syncthreads();
  if (tid < D / 4) stage_put(stg, kStageHead + tid, reinterpret_cast<const int*>(S.d8)[tid]);
  if (wave == 0) {
    const float dist = sqrtf(wave_cdot(S.vs, S.vs, D));
    if (tid == 0) {
      const bool moved = (dist > in.delta * P.rbar) && (nb > 0.f);
      stage_put(stg, 8, P.flags | (moved ? 1 : 0) | ((n_act >= in.reset_at) ? 2 : 0));
    }
  }
}

// The staged words of head h, loaded by the committing workgroup as soon as it knows it commits
// (with the merge's loads, so that the commit does not wait for another round trip): header word
// threadIdx.x in the first 9 threads, word threadIdx.x of the int8 direction row in the first
// D/4. stage_publish puts the header into hdr (LDS) for every thread; a barrier must follow.
struct StagePre {
  int hw, d8w;
};

template <int D>
__device__ __forceinline__ void stage_prefetch(StagePre& T, const ssa_index_state_t& st, int h) {
  const int32_t* stg = st.stage + (int64_t)h * kStageWords;
  const int t = threadIdx.x;
  T.hw = t < 9 ? stage_get(stg, t) : 0;
  T.d8w = t < D / 4 ? stage_get(stg, kStageHead + t) : 0;
}

__device__ __forceinline__ void stage_publish(const StagePre& T, int* hdr) {
  if (threadIdx.x < 9) hdr[threadIdx.x] = T.hw;
}

// Commit what insert_stage staged for head h (called by the head's last workgroup, after every
// workgroup of the step has read the state; T and hdr hold stage_prefetch's words). A
// kStageGeneral stage runs the whole insertion.
template <int D, class SM>
__device__ __forceinline__ void insert_commit(SM& S, const ssa_index_state_t& st, const ssa_insert_args_t& in, int h,
                                              int n, const StagePre& T, const int* hdr) {
  const int tid = threadIdx.x;
  const Head H = head_view(st, h);
  int Th[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) Th[i] = hdr[i];
  const int status = Th[0];
  if (status == kStageGeneral) {
    InsPre<D> P;
    insert_prefetch<D>(P, st, in, h, n);
    insert_phase<D>(S, st, in, h, P, n);
    return;
  }
  if (status != kStageOne && status != kStageSplit) return;
  const int row = Th[1], p = Th[2], new_end = Th[3];
  const int cn = Th[4], n_act = Th[7], flags = Th[8];
  const float mx = __int_as_float(Th[5]), mn = __int_as_float(Th[6]);
  if (tid < D / 4) reinterpret_cast<int*>(H.dir8 + (int64_t)row * D)[tid] = T.d8w;
  if (tid == 0) {
    H.mmax[row] = mx;
    H.mmin[row] = mn;
    H.count[row] = cn;
    H.labels[p] = (int16_t)row;
    st.end[h] = new_end;
    st.flags[h] = flags;
  }
  if (status == kStageSplit) {
    if (tid < D) S.mu[tid] = st.mu_ref[(int64_t)h * D + tid];
    __syncthreads();                                     // the label and summaries above are written
    split_cluster(S, st, H, head_keys_of(st, in, h), h, row, n_act, p + 1);
    if (tid == 0 && n_act + 1 >= in.reset_at) st.flags[h] = flags | 2;
  }
}

}  // namespace ssa
