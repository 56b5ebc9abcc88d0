// Canonical cluster scoring and budget selection for one (sequence, KV head), shared by the
// selection kernel (index.hip) and the fused selection + attention kernel (attention.hip).
// Both files are compiled with -ffp-contract=off, so this code yields the same bits in both.
//
// Reference behaviour: SphereIndexGPU.labels_and_weights and _rank_mask
// (src/ssa/attn/sphere_gpu.py:402-442), _score_kernel / _shared_pick / _pick_kernel
// (src/ssa/kernels/sphere_fused.py:231-313). Scores e[g,c] = (p >= 0 ? mmax : mmin) * p with
// p = q_g . dir_c / |dir_c| over live clusters; sum_share ranks by the sum over the group's query
// heads of each head's softmax over clusters of e / sqrt(d); per_head ranks each head by e; max
// and max_rel by the largest (relative) z. A cluster is taken iff the live clusters ranked
// before it, by (key desc, index asc), hold fewer than need = ceil(budget * binned) keys.
#pragma once

#include "ssa_common.h"
#include "../../include/ssa_hip.h"

namespace ssa {

constexpr int kMaxD = 256;
constexpr int kMaxC = 1024;
constexpr int kMaxG = 8;

// One head's rows of the index state.
struct Head {
  int C, d, ms;
  float* sum_dir; int8_t* dir8; float* cent; int8_t* cent8;
  float* mmax; float* mmin; int32_t* count; int16_t* labels;
  int32_t* mem; float* proj; int32_t* side; float* smag;
  float* kn; int kn_rows;   // a split's member unit directions (rows of d), when the state has room
  bool q8dirs;    // scoring reads dir8
  bool q8cent;    // insertion reads cent8
};

__device__ __forceinline__ Head head_view(const ssa_index_state_t& st, int h) {
  Head H;
  H.C = st.C; H.d = st.d; H.ms = st.ms;
  const int64_t cd = (int64_t)st.C * st.d;
  H.sum_dir = st.sum_dir + h * cd;
  H.dir8 = st.dir8 ? st.dir8 + h * cd : nullptr;
  H.cent = st.shared_dirs ? st.cent : st.cent + h * cd;
  H.cent8 = st.cent8 ? st.cent8 + h * cd : nullptr;
  H.mmax = st.mmax + (int64_t)h * st.C;
  H.mmin = st.mmin + (int64_t)h * st.C;
  H.count = st.count + (int64_t)h * st.C;
  H.labels = st.labels + (int64_t)h * st.capacity;
  H.mem = st.mem ? st.mem + (int64_t)h * st.ms : nullptr;
  H.proj = st.proj ? st.proj + (int64_t)h * st.ms : nullptr;
  H.side = st.side ? st.side + (int64_t)h * st.ms : nullptr;
  H.smag = st.smag ? st.smag + (int64_t)h * st.ms : nullptr;
  H.kn = st.knbuf && st.kn_rows > 0 ? st.knbuf + (int64_t)h * st.kn_rows * st.d : nullptr;
  H.kn_rows = st.knbuf ? st.kn_rows : 0;
  H.q8dirs = st.summary_bits == 8 && st.dir8;
  H.q8cent = st.summary_bits == 8 && !st.shared_dirs && st.cent8;
  return H;
}

// One cluster row of D int8 or fp32 values widened into registers with 16-byte loads.
template <int D>
__device__ __forceinline__ void load_row(const int8_t* r, float (&x)[D]) {
#pragma unroll
  for (int k = 0; k < D / 16; ++k) {
    const int4 v = reinterpret_cast<const int4*>(r)[k];
    const int w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 16; ++e) x[16 * k + e] = (float)(int8_t)((w[e / 4] >> (8 * (e % 4))) & 0xff);
  }
}
template <int D>
__device__ __forceinline__ void load_row(const float* r, float (&x)[D]) {
#pragma unroll
  for (int k = 0; k < D / 4; ++k) {
    const float4 v = reinterpret_cast<const float4*>(r)[k];
    x[4 * k] = v.x; x[4 * k + 1] = v.y; x[4 * k + 2] = v.z; x[4 * k + 3] = v.w;
  }
}

// Canonical dot of two LDS vectors, computed by the calling wave: lanes 0..7 run the eight
// chains, then DPP moves combine them in the canonical tree (lane 0 adds lane 1, then lanes 2-3,
// then lane 7, which holds (c4+c5)+(c6+c7) by then); the result is read from lane 0, so every
// lane of the wave gets it. The whole wave must be active.
__device__ __forceinline__ float wave_cdot(const float* a, const float* b, int d) {
  const int lane = threadIdx.x & 63;
  float c = 0.f;
  if (lane < 8)
    for (int i = lane; i < d; i += 8) c = __builtin_fmaf(a[i], b[i], c);
  c = c + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(c), 0xB1, 0xF, 0xF, true));   // lane ^ 1
  c = c + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(c), 0x4E, 0xF, 0xF, true));   // lane ^ 2
  c = c + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(c), 0x141, 0xF, 0xF, true));  // 7 - lane
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(c)));
}

// Canonical dots of one cluster row with itself (nrm2) and with the GMAX query rows held in LDS
// (dot[g]; rows g >= G of q are zero and their dots unused), all in one pass over the row, 16
// elements at a time: chain j of every dot takes elements j, j+8, j+16, ... in increasing order,
// as cdot does, so the results are identical. int8 rows are loaded whole (one 16-byte load per
// 16 elements) before any use.
// An offset of 0 the compiler cannot see through: loads through a pointer moved by it are not
// hoisted out of loops or merged across calls, so a row of LDS that many loop iterations read
// is read per use instead of being held in registers.
__device__ __forceinline__ int opaque_zero() {
  int z = 0;
  asm volatile("" : "+v"(z));
  return z;
}

template <int D, int GMAX>
__device__ __forceinline__ void row_dots_raw(const int4 (&raw)[D / 16], const float (*q0)[kMaxD], int G, float& nrm2,
                                             float (&dot)[GMAX]) {
  const float (*q)[kMaxD] = q0 + opaque_zero();
  float cn[8], cq[GMAX][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    cn[j] = 0.f;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) cq[g][j] = 0.f;
  }
#pragma unroll
  for (int k = 0; k < D / 16; ++k) {
    __builtin_amdgcn_sched_barrier(0);     // keep this chunk's LDS reads of q inside the chunk
    const int w[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float x = (float)(int8_t)((w[e / 4] >> (8 * (e % 4))) & 0xff);
      const int j = e % 8, i = 16 * k + e;
      cn[j] = __builtin_fmaf(x, x, cn[j]);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) cq[g][j] = __builtin_fmaf(q[g][i], x, cq[g][j]);
    }
  }
  nrm2 = ((cn[0] + cn[1]) + (cn[2] + cn[3])) + ((cn[4] + cn[5]) + (cn[6] + cn[7]));
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
    dot[g] = ((cq[g][0] + cq[g][1]) + (cq[g][2] + cq[g][3])) + ((cq[g][4] + cq[g][5]) + (cq[g][6] + cq[g][7]));
}

template <int D, int GMAX>
__device__ __forceinline__ void row_dots(const int8_t* r, const float (*q)[kMaxD], int G, float& nrm2,
                                         float (&dot)[GMAX]) {
  int4 raw[D / 16];
#pragma unroll
  for (int k = 0; k < D / 16; ++k) raw[k] = reinterpret_cast<const int4*>(r)[k];
  row_dots_raw<D, GMAX>(raw, q, G, nrm2, dot);
}

template <int D, int GMAX>
__device__ __forceinline__ void row_dots(const float* r, const float (*q0)[kMaxD], int G, float& nrm2,
                                         float (&dot)[GMAX]) {
  const float (*q)[kMaxD] = q0 + opaque_zero();
  float cn[8], cq[GMAX][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    cn[j] = 0.f;
#pragma unroll
    for (int g = 0; g < GMAX; ++g) cq[g][j] = 0.f;
  }
#pragma unroll
  for (int k = 0; k < D / 16; ++k) {
    __builtin_amdgcn_sched_barrier(0);
    float x[16];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 f = reinterpret_cast<const float4*>(r)[4 * k + v];
      x[4 * v] = f.x; x[4 * v + 1] = f.y; x[4 * v + 2] = f.z; x[4 * v + 3] = f.w;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = e % 8, i = 16 * k + e;
      cn[j] = __builtin_fmaf(x[e], x[e], cn[j]);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) cq[g][j] = __builtin_fmaf(q[g][i], x[e], cq[g][j]);
    }
  }
  nrm2 = ((cn[0] + cn[1]) + (cn[2] + cn[3])) + ((cn[4] + cn[5]) + (cn[6] + cn[7]));
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
    dot[g] = ((cq[g][0] + cq[g][1]) + (cq[g][2] + cq[g][3])) + ((cq[g][4] + cq[g][5]) + (cq[g][6] + cq[g][7]));
}

constexpr int kBins = 1024;     // threshold buckets of the selection (top 10 bits of the rank key)

// CMAX: the largest slot count the selection is compiled for (a power of two, 256 or 1024); the
// per-slot arrays, the scoring rounds and the denominator tree are sized by it.
template <int GMAX, int CMAX = kMaxC>
struct SelSmem {
  float q[GMAX][kMaxD];             // the group's query rows, fp32
  float z[GMAX][CMAX];              // softmax terms, for the denominator tree
  float tree[GMAX];                 // softmax denominators
  float red[GMAX][16];              // per-wave maxima
  int hist[kBins];                  // keys per bucket
  int wsum[16];                     // per-wave bucket totals
  int bstar, base, nlist;           // crossing bucket, keys ranked before it, its member count
  unsigned long long lrk[CMAX];     // rank keys of the crossing bucket's clusters
  int lcnt[CMAX];                   // and their key counts
};

// The state a thread scores first (slot threadIdx.x), loaded at kernel start so that its
// memory latency overlaps the query and label loads.
template <int D>
struct SelPre {
  int4 raw[D / 16];                 // int8 chunks of the first round's 8 rows (8-bit summaries only)
  int cnt;                          // summaries of slot sel_slot(threadIdx.x, 0)
  float mx, mn;
};

// Scoring layout: 8 lanes score one cluster row together, lane j holding chain j (elements
// [j*D/8, (j+1)*D/8)). Lane group grp = t / 8 scores, in round k, the rows grp + 256k + 32i
// (i < 8), and afterwards thread t keeps the scores of slot grp + 256k + 32 * (t % 8).
__device__ __forceinline__ int sel_slot(int t, int k) { return (t >> 3) + 256 * k + 32 * (t & 7); }

// Lane j's int8 chunk of a row of D values: D/8 consecutive bytes.
template <int D>
__device__ __forceinline__ void load_chunk8(const int8_t* row, int j, int4* dst, int i) {
  constexpr int E = D / 8;
  const int8_t* p = row + j * E;
  if constexpr (E >= 16) {
#pragma unroll
    for (int n = 0; n < E / 16; ++n) dst[i * (E / 16) + n] = reinterpret_cast<const int4*>(p)[n];
  } else {
    // E bytes of chunk i go to bytes [i*E, (i+1)*E) of dst (E = 2, 4 or 8)
    int* w = reinterpret_cast<int*>(dst);
    if constexpr (E == 8) {
      const int2 v = *reinterpret_cast<const int2*>(p);
      w[2 * i] = v.x; w[2 * i + 1] = v.y;
    } else if constexpr (E == 4) {
      w[i] = *reinterpret_cast<const int*>(p);
    } else {
      const int v = *reinterpret_cast<const unsigned short*>(p);
      w[i / 2] = (i & 1) ? ((w[i / 2] & 0xffff) | (v << 16)) : v;
    }
  }
}

template <int D>
__device__ __forceinline__ void sel_prefetch(SelPre<D>& P, const Head& H, int C) {
  const int t = threadIdx.x, j = t & 7, grp = t >> 3;
  const int c = sel_slot(t, 0);
  P.cnt = 0; P.mx = 0.f; P.mn = 0.f;
  if (c < C) {
    P.cnt = H.count[c];
    P.mx = H.mmax[c];
    P.mn = H.mmin[c];
  }
  if (H.q8dirs) {
#pragma unroll
    for (int k = 0; k < D / 16; ++k) P.raw[k] = make_int4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) load_chunk8<D>(H.dir8 + (int64_t)min(grp + 32 * i, C - 1) * D, j, P.raw, i);
  }
}

// Sum of v over the 8 lanes of a lane group in the canonical tree ((c0+c1)+(c2+c3)) +
// ((c4+c5)+(c6+c7)), lane j holding c_j; every lane of the group gets the total.
__device__ __forceinline__ float group8_sum(float v) {
  v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));   // lane ^ 1
  v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));   // lane ^ 2
  v = v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));  // 7 - lane
  return v;
}

// Orderable bits of a key for the selection order: ascending bits = descending key; -0 and +0
// are one key (x + 0 maps -0 to +0); -inf sorts after every finite key.
__device__ __forceinline__ unsigned int desc_bits(float key) {
  const unsigned int u = __float_as_uint(key + 0.0f);
  const unsigned int asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~asc;
}

// Integer rank key of (key, slot): ascending order is (key desc, slot asc).
__device__ __forceinline__ unsigned long long rank_key(float key, int c) {
  return ((unsigned long long)desc_bits(key) << 32) | (unsigned int)c;
}

// Take cluster c iff it is live (cnt > 0) and the live clusters ranked before it, by (key desc,
// index asc), hold fewer than `need` keys: before(c) < need.
// Exact threshold search instead of a full ranking. The bucket of a key,
//   b(c) = min((desc_bits(key) - base) >> shift, kBins - 1)   (base <= desc_bits of every live key),
// is monotone in the rank order. With b* the first bucket where the running key count reaches
// need and cbase the count of all buckets before b*:
//   - a cluster of a bucket before b* has before(c) <= cbase - cnt(c) < need (taken);
//   - a cluster of a bucket after b* has before(c) >= cbase + count(b*) >= need (not taken);
//   - a cluster of bucket b* has before(c) = cbase + (its bucket's clusters ranked before it),
//     counted exactly.
// If all keys together are fewer than need, every live cluster is taken.
// On entry S.hist is zero and S.nlist is 0; both are so again on return.
template <int NT, int KPT, class SS, typename Emit>
__device__ __forceinline__ void bucket_take(SS& S, const float (&key)[KPT], const int (&cnt)[KPT], int C,
                                            int64_t need, unsigned int base, int shift, int row, Emit emit) {
  static_assert(kBins == 4 * NT, "one int4 of buckets per thread");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  unsigned int db[KPT], bk[KPT];
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    db[k] = desc_bits(key[k]);
    bk[k] = min((db[k] > base ? db[k] - base : 0u) >> shift, (unsigned int)(kBins - 1));
    if (cnt[k] > 0) atomicAdd(&S.hist[bk[k]], cnt[k]);
  }
  __syncthreads();
  const int4 hb = reinterpret_cast<const int4*>(S.hist)[tid];
  const int own = hb.x + hb.y + hb.z + hb.w;
  const int incl = wave_incl_scan_dpp(own);
  if (lane == 63) S.wsum[wave] = incl;
  __syncthreads();
  int wbase = 0, total = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const int v = S.wsum[w];
    if (w < wave) wbase += v;
    total += v;
  }
  const int64_t lo = wbase + incl - own, hi = wbase + incl;
  if (lo < need && need <= hi) {            // the crossing lies in this thread's four buckets
    const int v[4] = {hb.x, hb.y, hb.z, hb.w};
    int64_t cum = lo;
    int b = 4 * tid + 3;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (cum + v[e] >= need) { b = 4 * tid + e; break; }
      cum += v[e];
    }
    S.bstar = b;
    S.base = (int)cum;
  }
  if (tid == NT - 1 && (int64_t)total < need) { S.bstar = kBins; S.base = total; }
  reinterpret_cast<int4*>(S.hist)[tid] = make_int4(0, 0, 0, 0);     // this thread's buckets, read above
  __syncthreads();
  const unsigned int bstar = (unsigned int)S.bstar;
  const int64_t cbase = S.base;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    if (cnt[k] > 0 && bk[k] == bstar) {
      const int i = atomicAdd(&S.nlist, 1);
      S.lrk[i] = ((unsigned long long)db[k] << 32) | (unsigned int)sel_slot(tid, k);
      S.lcnt[i] = cnt[k];
    }
  }
  __syncthreads();
  const int nl = S.nlist;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const int c = sel_slot(tid, k);
    if (c >= C) continue;
    float x = 0.f;
    if (cnt[k] > 0) {
      const unsigned int b = bk[k];
      if (b < bstar) {
        x = 1.f;
      } else if (b == bstar) {
        const unsigned long long rk = ((unsigned long long)db[k] << 32) | (unsigned int)c;
        int64_t before = cbase;
        for (int i0 = 0; i0 < nl; i0 += 8) {
          unsigned long long r8[8];
          int n8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = min(i0 + e, nl - 1);
            r8[e] = S.lrk[i];
            n8[e] = S.lcnt[i];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) before += (i0 + e < nl && r8[e] < rk) ? n8[e] : 0;
        }
        x = before < need ? 1.f : 0.f;
      }
    }
    emit(row, c, x);
  }
  __syncthreads();
  if (tid == 0) S.nlist = 0;
}

// Selection for one head. S.q must hold the G query rows (fp32), rows G..GMAX-1 zero, and be
// visible (barrier) on entry; P holds slot threadIdx.x's state (sel_prefetch). emit(row, c, w) receives w for every
// slot c in [0, C] of every weight row (one row, or G rows for per_head); slot C, the
// always-read exact set, gets 1. Each thread scores slots threadIdx.x + k * NT and keeps their
// scores in registers.
template <int D, int NT, int GMAX, int CMAX = kMaxC, typename Emit>
__device__ __forceinline__ void select_head(SelSmem<GMAX, CMAX>& S, const Head& H, const SelPre<D>& P, int C, int n_act,
                                            int end, int G, double budget, int group, float scale, Emit emit) {
  static_assert(CMAX % NT == 0 && CMAX >= 64, "whole rounds of slots");
  constexpr int KPT = CMAX / NT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool per_head = group == 1;
  const int nrows = per_head ? G : 1;
  const int nb = end - 1;
  const double needd = nb > 0 ? ceil(budget * (double)nb) : 0.0;
  const int64_t need = needd > 9.0e18 ? (int64_t)9e18 : (int64_t)needd;
  if (tid < nrows) emit(tid, C, 1.f);
  if (nb <= 0 || need <= 0) {
    for (int r = 0; r < nrows; ++r)
      for (int c = tid; c < C; c += NT) emit(r, c, 0.f);
    return;
  }
  reinterpret_cast<int4*>(S.hist)[tid] = make_int4(0, 0, 0, 0);
  if (tid == 0) S.nlist = 0;
  // scores e[g] = (p >= 0 ? mmax : mmin) * p, p = q_g . dir / |dir|, scaled by 1/sqrt(d) unless
  // per_head; the dots are scoring dots (score_dots), 8 lanes per row
  float z[KPT][GMAX];
  int cnt[KPT];
  constexpr int E = D / 8;
  constexpr bool QREG = E * GMAX <= 64;        // the lane's query slices fit in registers
  const int jl = tid & 7, grp = tid >> 3;
  float qv[QREG ? GMAX : 1][QREG ? E : 1];
  if constexpr (QREG) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
#pragma unroll
      for (int e = 0; e < E; ++e) qv[g][e] = S.q[g][jl * E + e];
  }
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    if (256 * k >= min(C, n_act)) {             // no slot of this round is in use (uniform)
      cnt[k] = 0;
#pragma unroll
      for (int g = 0; g < GMAX; ++g) z[k][g] = -INFINITY;
      continue;
    }
    const int kact = min(C, n_act);
    const int c = sel_slot(tid, k);
    const bool used = c < C && c < n_act;
    // this round's summaries and rows (the first round's were prefetched), the rows in batches of
    // RB whose loads are all issued before the first dot of the batch waits on one (RB = 8 with
    // two query heads per KV head; 4 otherwise, which keeps the kernel at two waves per SIMD)
    constexpr int RB = GMAX == 2 ? 8 : 4;
    float mx = 0.f, mn = 0.f;
    int ct = 0;
    if (k == 0) {
      ct = P.cnt; mx = P.mx; mn = P.mn;
    } else if (used) {
      ct = H.count[c]; mx = H.mmax[c]; mn = H.mmin[c];
    }
    // lane j keeps the dots of row i = j of the round (every lane of a group gets each total)
    float nrm2 = 0.f, dot[GMAX];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) dot[g] = 0.f;
#pragma unroll
    for (int i0 = 0; i0 < 8; i0 += RB) {
      int4 rk[(E * RB + 15) / 16];             // the batch's chunks, E bytes each, packed
      if (k > 0 && H.q8dirs) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
          if (256 * k + 32 * (i0 + i) < kact)
            load_chunk8<D>(H.dir8 + (int64_t)min(grp + 256 * k + 32 * (i0 + i), C - 1) * D, jl, rk, i);
      }
#pragma unroll
      for (int i1 = 0; i1 < RB; ++i1) {
        const int i = i0 + i1;
        if (256 * k + 32 * i >= kact) continue;  // rows [256k + 32i, +32) hold no slot in use (uniform)
        const int cr = min(grp + 256 * k + 32 * i, C - 1);      // rows past C are never kept
        float x[E];
        if (H.q8dirs) {
          const int8_t* bytes = k == 0 ? reinterpret_cast<const int8_t*>(P.raw) + i * E
                                       : reinterpret_cast<const int8_t*>(rk) + i1 * E;
#pragma unroll
          for (int e = 0; e < E; ++e) x[e] = (float)bytes[e];
        } else {
          const float* rp = H.sum_dir + (int64_t)cr * D + jl * E;
#pragma unroll
          for (int e = 0; e < E; ++e) x[e] = rp[e];
        }
        float cn = 0.f, cq[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) cq[g] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          cn = __builtin_fmaf(x[e], x[e], cn);
#pragma unroll
          for (int g = 0; g < GMAX; ++g)
            cq[g] = __builtin_fmaf(QREG ? qv[QREG ? g : 0][QREG ? e : 0] : S.q[g][jl * E + e], x[e], cq[g]);
        }
        cn = group8_sum(cn);
        nrm2 = jl == i ? cn : nrm2;
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
          const float t = group8_sum(cq[g]);
          dot[g] = jl == i ? t : dot[g];
        }
      }
    }
    cnt[k] = used && ct > 0 ? ct : 0;
    const float nrm = fmaxf(sqrtf(nrm2), 1e-12f);
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      float e = -INFINITY;
      if (cnt[k] > 0 && g < G) {
        const float p = dot[g] / nrm;
        e = p >= 0.f ? mx * p : mn * p;
        if (!per_head) e = e * scale;
      }
      z[k][g] = e;
    }
  }
  if (per_head) {
    __syncthreads();                          // S.hist / S.nlist cleared
    for (int g = 0; g < G; ++g) {
      float key[KPT];
#pragma unroll
      for (int k = 0; k < KPT; ++k) {
        key[k] = -INFINITY;
#pragma unroll
        for (int g2 = 0; g2 < GMAX; ++g2)
          if (g2 == g) key[k] = z[k][g2];
      }
      bucket_take<NT, KPT>(S, key, cnt, C, need, 0u, 22, g, emit);
    }
    return;
  }
  // per-head maxima over live clusters (sum_share, max_rel)
  float zmx[GMAX];
  if (group == 0 || group == 3) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      float v = -INFINITY;
#pragma unroll
      for (int k = 0; k < KPT; ++k) v = fmaxf(v, z[k][g]);
      v = wave_max_dpp(v);
      if (lane == 0 && g < G) S.red[g][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      float r = -INFINITY;
      if (g < G) {
        r = S.red[g][0];
        for (int w2 = 1; w2 < NT / 64; ++w2) r = fmaxf(r, S.red[g][w2]);
      }
      zmx[g] = r;
    }
  } else {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) zmx[g] = 0.f;
  }
  float key[KPT];
  if (group == 0) {
    // sum_share: per head a softmax over live clusters, summed over the heads
    float t[KPT][GMAX];
    const int kact = min(C, n_act);             // rounds past the slots in use hold no live cluster
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      const int c = sel_slot(tid, k);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        t[k][g] = 0.f;
        if (256 * k < kact && cnt[k] > 0 && g < G) t[k][g] = cexp(z[k][g] - zmx[g]);
        if (g < G && c < C) S.z[g][c] = t[k][g];
      }
    }
    __syncthreads();
    // Pairwise halving tree over the C slots: tot = t[0] after t[c] += t[c + h] for h = C/2 .. 1.
    // Wave g computes head g's: lane l first folds its slots l, l+64, l+128, ... with the
    // strides >= 64 of the tree, then the strides 32 .. 1 run as shuffles. The terms are >= 0,
    // so lanes past C padded with +0 give the same bits as the tree over exactly C slots.
    for (int g = wave; g < G; g += NT / 64) {
      float u[CMAX / 64];
      // the strides of the tree over the C slots (C a power of two): lane l holds slots l + 64 k
      auto fold = [&](auto kc) {
        constexpr int KC = decltype(kc)::value;
#pragma unroll
        for (int k = 0; k < KC; ++k) u[k] = (lane + 64 * k < C) ? S.z[g][lane + 64 * k] : 0.f;
#pragma unroll
        for (int half = KC / 2; half >= 1; half >>= 1)
#pragma unroll
          for (int k = 0; k < half; ++k) u[k] = u[k] + u[k + half];
      };
      bool folded = false;
      if constexpr (CMAX > 512) {
        if (C > 512) { fold(std::integral_constant<int, 16>{}); folded = true; }
      }
      if constexpr (CMAX > 256) {
        if (!folded && C > 256) { fold(std::integral_constant<int, 8>{}); folded = true; }
      }
      if (!folded) {
        if (C > 128) fold(std::integral_constant<int, 4>{});
        else if (C > 64) fold(std::integral_constant<int, 2>{});
        else fold(std::integral_constant<int, 1>{});
      }
      // strides 32 and 16 by shuffles, 8 .. 1 by DPP row_shl (lane l reads lane l + h of its
      // row); only lanes below the stride keep meaningful sums
      float v = u[0];
      v = v + __shfl_down(v, 32, 64);
      v = v + __shfl_down(v, 16, 64);
      v = v + dpp_f<0x108, 0xF>(0.f, v);
      v = v + dpp_f<0x104, 0xF>(0.f, v);
      v = v + dpp_f<0x102, 0xF>(0.f, v);
      v = v + dpp_f<0x101, 0xF>(0.f, v);
      if (lane == 0) S.tree[g] = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      key[k] = -INFINITY;
      if (256 * k < kact && cnt[k] > 0) {
        float s = 0.f;
#pragma unroll
        for (int g = 0; g < GMAX; ++g)
          if (g < G) s = s + t[k][g] / S.tree[g];
        key[k] = s;
      }
    }
  } else {
    // max / max_rel
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      float s = -INFINITY;
#pragma unroll
      for (int g = 0; g < GMAX; ++g)
        if (g < G) s = fmaxf(s, z[k][g] - zmx[g]);
      key[k] = cnt[k] > 0 ? s : -INFINITY;
    }
    __syncthreads();                          // S.hist / S.nlist cleared
  }
  // sum_share keys lie in [0, G] (each head's share is at most 1): 32 buckets per binade below G
  if (group == 0) bucket_take<NT, KPT>(S, key, cnt, C, need, desc_bits((float)G), 18, 0, emit);
  else bucket_take<NT, KPT>(S, key, cnt, C, need, 0u, 22, 0, emit);
}

}  // namespace ssa
