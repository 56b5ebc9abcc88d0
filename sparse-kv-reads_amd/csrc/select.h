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

// Canonical dot of two LDS vectors, computed by the calling wave (lanes 0..7 run the eight
// chains, shuffles combine them in the canonical tree); every lane of the wave gets the result.
__device__ __forceinline__ float wave_cdot(const float* a, const float* b, int d) {
  const int lane = threadIdx.x & 63;
  float c = 0.f;
  if (lane < 8)
    for (int i = lane; i < d; i += 8) c = __builtin_fmaf(a[i], b[i], c);
  const float p = c + __shfl_xor(c, 1, 64);
  const float q = p + __shfl_xor(p, 2, 64);
  const float r = q + __shfl_xor(q, 4, 64);
  return __shfl(r, 0, 64);
}

// Canonical dots of one cluster row with itself (nrm2) and with the G query rows held in LDS
// (dot[g]), all in one pass over the row, 16 elements at a time: chain j of every dot takes
// elements j, j+8, j+16, ... in increasing order, as cdot does, so the results are identical.
// int8 rows are loaded whole (one 16-byte load per 16 elements) before any use.
template <int D, int GMAX>
__device__ __forceinline__ void row_dots(const int8_t* r, const float (*q)[kMaxD], int G, float& nrm2,
                                         float (&dot)[GMAX]) {
  int4 raw[D / 16];
#pragma unroll
  for (int k = 0; k < D / 16; ++k) raw[k] = reinterpret_cast<const int4*>(r)[k];
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
      for (int g = 0; g < GMAX; ++g)
        if (g < G) cq[g][j] = __builtin_fmaf(q[g][i], x, cq[g][j]);
    }
  }
  nrm2 = ((cn[0] + cn[1]) + (cn[2] + cn[3])) + ((cn[4] + cn[5]) + (cn[6] + cn[7]));
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
    dot[g] = ((cq[g][0] + cq[g][1]) + (cq[g][2] + cq[g][3])) + ((cq[g][4] + cq[g][5]) + (cq[g][6] + cq[g][7]));
}

template <int D, int GMAX>
__device__ __forceinline__ void row_dots(const float* r, const float (*q)[kMaxD], int G, float& nrm2,
                                         float (&dot)[GMAX]) {
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
      for (int g = 0; g < GMAX; ++g)
        if (g < G) cq[g][j] = __builtin_fmaf(q[g][i], x[e], cq[g][j]);
    }
  }
  nrm2 = ((cn[0] + cn[1]) + (cn[2] + cn[3])) + ((cn[4] + cn[5]) + (cn[6] + cn[7]));
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
    dot[g] = ((cq[g][0] + cq[g][1]) + (cq[g][2] + cq[g][3])) + ((cq[g][4] + cq[g][5]) + (cq[g][6] + cq[g][7]));
}

template <int GMAX>
struct SelSmem {
  float q[GMAX][kMaxD];     // the group's query rows, fp32
  float z[GMAX][kMaxC];     // scores, then softmax terms
  float key[kMaxC];         // ranking key per slot
  int cnt[kMaxC];           // keys per live slot (0 otherwise)
  float tree[GMAX][1];      // softmax denominators
  unsigned long long rk[kMaxC];   // rank keys: (score descending, index ascending) as one integer
  float red[GMAX][16];
};

// Per-row maxima over the slots of S.z[0..nrow): one pass, one pair of barriers.
template <int NT, int GMAX>
__device__ __forceinline__ void sel_row_max(SelSmem<GMAX>& S, int nrow, int C, float (&out)[GMAX]) {
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g >= nrow) break;
    float v = -INFINITY;
    for (int c = threadIdx.x; c < C; c += NT) v = fmaxf(v, S.z[g][c]);
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) S.red[g][w] = v;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g >= nrow) break;
    float r = S.red[g][0];
    for (int w2 = 1; w2 < NT / 64; ++w2) r = fmaxf(r, S.red[g][w2]);
    out[g] = r;
  }
}

// Integer rank key of a score: ascending order of the key is (score desc, slot asc); -0 and +0
// compare equal (x + 0 maps -0 to +0), -inf (dead slots) sorts after every finite score.
__device__ __forceinline__ unsigned long long rank_key(float key, int c) {
  const unsigned int u = __float_as_uint(key + 0.0f);
  const unsigned int asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)(~asc) << 32) | (unsigned int)c;
}

// Take cluster c iff it is live and the live clusters ranked before it, by (key desc, index
// asc), hold fewer than `need` keys. Slots past n_act have key -inf and count 0.
template <int NT, int GMAX, typename Emit>
__device__ __forceinline__ void rank_take(SelSmem<GMAX>& S, const float* key, int n_act, int C, int64_t need,
                                          int row, Emit emit) {
  for (int c = threadIdx.x; c < C; c += NT) S.rk[c] = rank_key(key[c], c);
  __syncthreads();
  const int jn = min(C, (n_act + 15) & ~15);
  for (int c = threadIdx.x; c < C; c += NT) {
    const bool live = c < n_act && S.cnt[c] > 0;
    const unsigned long long kc = S.rk[c];
    int before = 0;
    for (int j0 = 0; j0 < jn; j0 += 16) {
      // 16 slots per step: every LDS read of the step is issued before the compares
      unsigned long long k[16];
      int n[16];
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const int4 c4 = *reinterpret_cast<const int4*>(S.cnt + j0 + e);
        n[e] = c4.x; n[e + 1] = c4.y; n[e + 2] = c4.z; n[e + 3] = c4.w;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) k[e] = S.rk[j0 + e];
#pragma unroll
      for (int e = 0; e < 16; ++e) before += k[e] < kc ? n[e] : 0;
    }
    emit(row, c, (live && (int64_t)before < need) ? 1.f : 0.f);
  }
  __syncthreads();
}

// Selection for one head. S.q must hold the G query rows (fp32) and be visible (barrier) on
// entry. emit(row, c, w) receives w for every slot c in [0, C] of every weight row (one row, or
// G rows for per_head); slot C, the always-read exact set, gets 1.
template <int D, int NT, int GMAX, typename Emit>
__device__ void select_head(SelSmem<GMAX>& S, const Head& H, int C, int n_act, int end, int G, double budget,
                            int group, float scale, Emit emit) {
  const int tid = threadIdx.x;
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
  for (int c = tid; c < C; c += NT) {
    // every load of this slot is issued before the first use
    const bool used = c < n_act;
    const int cnt = used ? H.count[c] : 0;
    float mx = 0.f, mn = 0.f, nrm2 = 0.f, dot[GMAX];
    if (used) {
      mx = H.mmax[c];
      mn = H.mmin[c];
      if (H.q8dirs) row_dots<D, GMAX>(H.dir8 + (int64_t)c * D, S.q, G, nrm2, dot);
      else row_dots<D, GMAX>(H.sum_dir + (int64_t)c * D, S.q, G, nrm2, dot);
    }
    const bool live = cnt > 0;
    S.cnt[c] = live ? cnt : 0;
    if (live) {
      const float nrm = fmaxf(sqrtf(nrm2), 1e-12f);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g >= G) break;
        const float p = dot[g] / nrm;
        const float e = p >= 0.f ? mx * p : mn * p;
        S.z[g][c] = per_head ? e : e * scale;
      }
    } else {
      for (int g = 0; g < G; ++g) S.z[g][c] = -INFINITY;
    }
  }
  __syncthreads();
  if (per_head) {
    for (int g = 0; g < G; ++g) rank_take<NT>(S, S.z[g], n_act, C, need, g, emit);
    return;
  }
  float zmx[GMAX];
  if (group == 0) {
    // sum_share: per head a softmax over live clusters, summed over the heads (all heads at once)
    sel_row_max<NT>(S, G, C, zmx);
    for (int c = tid; c < C; c += NT) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g >= G) break;
        S.z[g][c] = S.cnt[c] > 0 ? cexp(S.z[g][c] - zmx[g]) : 0.f;
      }
    }
    __syncthreads();
    // Pairwise halving tree over the C slots: tot = t[0] after t[c] += t[c + h] for h = C/2 .. 1.
    // Wave g computes head g's: lane l first folds its slots l, l+64, l+128, ... with the
    // strides >= 64 of the tree, then the strides 32 .. 1 run as shuffles. The terms are >= 0,
    // so padding with +0 and folding from the largest stride gives the same bits as the tree
    // over exactly C slots.
    {
      const int w = tid >> 6, lane = tid & 63;
      for (int g = w; g < G; g += NT / 64) {
        float t[kMaxC / 64];
#pragma unroll
        for (int k = 0; k < kMaxC / 64; ++k) t[k] = (lane + 64 * k < C) ? S.z[g][lane + 64 * k] : 0.f;
#pragma unroll
        for (int half = kMaxC / 128; half >= 1; half >>= 1)
#pragma unroll
          for (int k = 0; k < half; ++k) t[k] = t[k] + t[k + half];
        float v = t[0];
#pragma unroll
        for (int h = 32; h >= 1; h >>= 1) {
          const float o = __shfl_down(v, h, 64);
          if (lane < h) v = v + o;
        }
        if (lane == 0) S.tree[g][0] = v;
      }
    }
    __syncthreads();
    for (int c = tid; c < C; c += NT) {
      float s = 0.f;
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g >= G) break;
        s = s + S.z[g][c] / S.tree[g][0];
      }
      S.key[c] = S.cnt[c] > 0 ? s : -INFINITY;
    }
  } else {
    // max / max_rel
    if (group == 3) sel_row_max<NT>(S, G, C, zmx);
    else
      for (int g = 0; g < GMAX; ++g) zmx[g] = 0.f;
    for (int c = tid; c < C; c += NT) {
      float s = -INFINITY;
      for (int g = 0; g < G; ++g) s = fmaxf(s, S.z[g][c] - zmx[g]);
      S.key[c] = S.cnt[c] > 0 ? s : -INFINITY;
    }
  }
  __syncthreads();
  rank_take<NT>(S, S.key, n_act, C, need, 0, emit);
}

}  // namespace ssa
