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
//   grid (S, Hk): workgroup (sp, h) owns positions [sp*chunk, (sp+1)*chunk) of KV head h (dense)
//   or its blocks of 256 positions b = sp (mod S) (label scans).
//   Labelled mode scans its positions' 2-byte labels, looks their weights up in an LDS copy
//   of w, and compacts the selected positions into an LDS list (ballot + popcount), so only
//   selected K/V rows are ever fetched. Dense mode walks its rows directly.
//   Rows are read as 16-byte-per-lane loads: D/8 lanes cover one 128-dim bf16 row (256 B), so
//   one wave instruction reads 64*16 B of consecutive row bytes; each lane group keeps its own
//   online softmax (base-2, q pre-scaled by log2(e)/sqrt(d)) over the G query heads that share
//   the KV head, and issues U rows of K and V before it consumes any of them.
//   States merge across lane groups (DPP/shuffle), across waves (LDS), then across the S
//   workgroups of a head: each writes its partial with agent-scope stores and counts itself in
//   on an agent-scope atomic counter; the last workgroup to arrive (which resets the counter
//   for the next launch) combines the partials by log-sum-exp and writes out[h*G + g] in the
//   output dtype, plus the count of rows read.
//   Fused mode (ssa_sparse_step) first computes the head's cluster selection in LDS
//   (select.h) and uses it as the weights.
#pragma once

#include "insert.h"

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
  // fused selection (ssa_sparse_step): the index state and the selection parameters
  ssa_index_state_t st;
  double budget; int group; float sel_scale;
  // insertion ahead (fused mode with AHEAD): after the merge, the last workgroup of each head
  // bins the keys that leave the window at length n + 1, as staged by an extra workgroup per
  // head or, with fold_stage (when the extra workgroups would not all be resident), by split S - 1
  ssa_insert_args_t ins;
  int fold_stage;
};

constexpr int kThreads = 256;
static_assert(kThreads == kT, "the insertion code runs on the decode kernel's workgroup");
constexpr int kWaves = kThreads / 64;
// positions compacted per pass: the selected-row list (position + GMAX weights per row) lives in
// LDS, so the page shrinks as the weight rows grow
template <int GMAX> constexpr int page_size() { return GMAX <= 4 ? 2048 : 1024; }
constexpr int kMaxW = kMaxC + 1;     // weight slots (C + 1) held in LDS per row

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

constexpr int kRowsInFlight = 8;     // rows of K (and of V) each lane group loads before using them

// 8 consecutive elements of a row in their storage type: 16 bytes for bf16/fp16, 32 for fp32.
struct F8 { float4 a, b; };
template <typename T> struct RawRow { using type = uint4; };
template <> struct RawRow<float> { using type = F8; };

__device__ __forceinline__ void widen8(const uint4& r, float (&f)[8], __hip_bfloat16*) {
  const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(u[e] << 16);
    f[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ void widen8(const uint4& r, float (&f)[8], __half*) {
  const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const __half2 h2 = *reinterpret_cast<const __half2*>(&u[e]);
    f[2 * e] = __low2float(h2);
    f[2 * e + 1] = __high2float(h2);
  }
}
__device__ __forceinline__ void widen8(const F8& r, float (&f)[8], float*) {
  f[0] = r.a.x; f[1] = r.a.y; f[2] = r.a.z; f[3] = r.a.w;
  f[4] = r.b.x; f[5] = r.b.y; f[6] = r.b.z; f[7] = r.b.w;
}

__device__ __forceinline__ void store_out(void* out, int dt, int64_t i, float x) {
  if (dt == kBF16) reinterpret_cast<__hip_bfloat16*>(out)[i] = __float2bfloat16(x);
  else if (dt == kF16) reinterpret_cast<__half*>(out)[i] = __float2half(x);
  else reinterpret_cast<float*>(out)[i] = x;
}

constexpr int kMaxS = 256;           // splits per head (host clamps)
// accumulator loads (float4) each merging thread issues at once: S = 32 splits of G x 128
// columns in one round up to G = 4
template <int GMAX> constexpr int merge_batch() { return GMAX >= 4 ? 16 : 8; }

// Agent-scope relaxed load: coherent with the agent-scope stores of other workgroups on any XCD.
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Four consecutive floats (16-byte aligned) as two 8-byte agent-scope relaxed loads.
__device__ __forceinline__ float4 load_coherent4(const float* p) {
  const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
  const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((unsigned int)a), __uint_as_float((unsigned int)(a >> 32)),
                     __uint_as_float((unsigned int)b), __uint_as_float((unsigned int)(b >> 32)));
}

// CMAX: the largest slot count of the fused selection (256 or 1024); the weight rows hold CMAX + 1
template <int D, int GMAX, bool DENSE, int CMAX = kMaxC>
struct DecodeSmem {
  static constexpr int kPage = page_size<GMAX>();
  static constexpr int kSelG = DENSE ? 1 : GMAX;
  float lw[DENSE ? 1 : GMAX][DENSE ? 1 : CMAX + 1];    // log2 w per weight row, -inf where w <= 0
  union {
    struct {
      int pos[DENSE ? 1 : kPage];                        // selected positions of the current page
      float rlw[GMAX][DENSE ? 1 : kPage];                // their log2 w per weight row
    } list;
    SelSmem<kSelG, CMAX> sel;                            // fused selection scratch
    InsertSmem tail;                                     // fused insertion ahead
    struct {
      float f[kMaxS * GMAX];                             // rescale factor per (split, head)
      float4 acc[kThreads];
    } mrg;
  } u;
  int scan[kPage / kThreads][kWaves];                 // selected positions per (page slice, wave)
  float red_m[kWaves][GMAX], red_l[kWaves][GMAX];
  float red_a[kWaves][GMAX][D];
  float gden[GMAX];
  int red_i[kWaves];
  int last;
  int stage_hdr[9];                                  // the staged insertion's header (commit)
};

// DENSE: every position in [0, n) is read with weight 1. Otherwise positions are selected by
// w[label] > 0 (any query head of the group, when w has one row per query head). SELECT: w is
// not read but computed by this workgroup from the index state (select.h), the same bits the
// selection kernel writes; workgroup 0 of each head also stores it.
template <typename T, int D, int GMAX, bool DENSE, bool SELECT = false, bool AHEAD = false, int CMAX = kMaxC>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeParams a) {
  constexpr int LPR = D / 8;           // lanes per row
  constexpr int RPI = 64 / LPR;        // rows per wave instruction
  constexpr int U = kRowsInFlight;     // rows in flight per lane group
  constexpr int kPage = page_size<GMAX>();
  constexpr int PER = kPage / kThreads;
  using Raw = typename RawRow<T>::type;
  __shared__ DecodeSmem<D, GMAX, DENSE, CMAX> sm;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane / LPR, li = lane % LPR;
  // XCD-aware placement: workgroups are dispatched to the 8 XCDs round robin by linear id, so
  // (when the head count allows) every workgroup of a head goes to the same XCD and the head's
  // index state, labels and partials are shared through one L2. Any mapping is correct; this one
  // is a permutation of the grid.
  int sp = blockIdx.x, h = blockIdx.y;
  if ((gridDim.y & 7) == 0) {
    const int lin = blockIdx.y * gridDim.x + blockIdx.x;
    const int j = lin >> 3;
    h = (lin & 7) + 8 * (j / gridDim.x);
    sp = j % gridDim.x;
  }
  const int G = a.G, S = a.S;
  const bool per_head = !DENSE && a.per_head;

  const int n = a.n_dev ? *a.n_dev : a.n_host;
  // Dense: workgroup sp owns the contiguous chunk [s0, s1). Label scans: it owns the blocks of
  // kThreads positions b = sp, sp + S, sp + 2S, ..., PER blocks per page, so that selected rows
  // that crowd into one stretch of positions (their clusters follow the position) still spread
  // over every workgroup of the head.
  int chunk = (n + S - 1) / S;
  chunk = (chunk + a.chunk_align - 1) / a.chunk_align * a.chunk_align;
  const int s0 = min(sp * chunk, n);
  const int s1 = min(s0 + chunk, n);
  auto block_pos = [&](int it, int u) { return (sp + S * (PER * it + u)) * kThreads; };
  const int16_t* labrow = DENSE ? nullptr : a.labels + (int64_t)h * a.s_lh;
  // AHEAD: the next step's insertion is staged by workgroup S of each head (one past the splits)
  // or, with fold_stage, by split S - 1 once its own attention is done
  const bool stager = AHEAD && !a.fold_stage && sp == S;
  if (!stager) {
    // Issue the selection state's and the first page's label loads before anything waits on memory.
    int n_act = 0, end_h = 0;
    uint32_t touch = 0;
    if constexpr (SELECT) {
      n_act = a.st.n_c[h];
      end_h = a.st.end[h];
    }
    SelPre<D> pre;
    if constexpr (SELECT) sel_prefetch<D>(pre, head_view(a.st, h), a.st.C);
    int lbl[PER];
    if constexpr (!DENSE) {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int j = block_pos(0, u) + tid;
        // fused mode: the labels are the state's rows of `capacity` (s_lh) entries, so the load
        // need not wait for n (positions >= n are masked by the scan)
        if constexpr (SELECT) lbl[u] = (int)labrow[min(j, (int)a.s_lh - 1)];
        else lbl[u] = j < n ? (int)labrow[j] : 0;
      }
      // One row per eighth of this head's K and V span, read now and consumed after the rows:
      // their address translations are then in place when the selected rows are read.
      if (tid < 16) {
        const int64_t span = (int64_t)max(n, 1);
        const int p = (int)min<int64_t>((int64_t)(tid & 7) * span / 8, span - 1);
        const T* tb = reinterpret_cast<const T*>(tid < 8 ? a.k : a.v) + (int64_t)h * (tid < 8 ? a.s_kh : a.s_vh);
        touch = *reinterpret_cast<const uint32_t*>(tb + (int64_t)p * (tid < 8 ? a.s_kn : a.s_vn));
      }
    }

    // q rows of the group: one uniform dtype branch, then 16-byte loads (rows 16-byte aligned)
    float qr[GMAX][8];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      const int64_t off = (int64_t)(h * G + min(g, G - 1)) * a.s_qh + li * 8;
      float r[8];
      if (a.q_dtype == kBF16) widen8(*reinterpret_cast<const uint4*>(reinterpret_cast<const __hip_bfloat16*>(a.q) + off), r, (__hip_bfloat16*)nullptr);
      else if (a.q_dtype == kF16) widen8(*reinterpret_cast<const uint4*>(reinterpret_cast<const __half*>(a.q) + off), r, (__half*)nullptr);
      else {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.q) + off);
        const float4 x = p[0], y = p[1];
        r[0] = x.x; r[1] = x.y; r[2] = x.z; r[3] = x.w; r[4] = y.x; r[5] = y.y; r[6] = y.z; r[7] = y.w;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) qr[g][e] = g < G ? r[e] * a.qscale : 0.f;
      if constexpr (SELECT) {
        // lane group 0 of wave 0 holds the whole row: the selection's fp32 copy (rows >= G zero)
        if (wave == 0 && lg == 0) {
          float4* dst = reinterpret_cast<float4*>(&sm.u.sel.q[g][li * 8]);
          dst[0] = g < G ? make_float4(r[0], r[1], r[2], r[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
          dst[1] = g < G ? make_float4(r[4], r[5], r[6], r[7]) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }

    if constexpr (SELECT) {
      // the head's selection, computed here while the label loads are in flight
      const int end = end_h;
      __syncthreads();
      float* wout = const_cast<float*>(a.w);
      const int64_t s_wr = a.s_wr;
      const bool store_w = sp == 0 && wout != nullptr;
      select_head<D, kThreads, GMAX, CMAX>(sm.u.sel, head_view(a.st, h), pre, a.st.C, n_act, end, G, a.budget, a.group,
                                     a.sel_scale, [&](int r, int c, float x) {
                                       sm.lw[r][c] = x > 0.f ? 0.f : -INFINITY;
                                       if (store_w) wout[(int64_t)(per_head ? h * G + r : h) * s_wr + c] = x;
                                     });
    } else if constexpr (!DENSE) {
      const int nrow = per_head ? G : 1;
      for (int r = 0; r < nrow; ++r) {
        const float* wr = a.w + (int64_t)(per_head ? h * G + r : h) * a.s_wr;
        float x[(CMAX + kThreads) / kThreads];
#pragma unroll
        for (int k = 0; k < (CMAX + kThreads) / kThreads; ++k) {
          const int c = tid + k * kThreads;
          x[k] = c < a.w_len ? wr[c] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < (CMAX + kThreads) / kThreads; ++k) {
          const int c = tid + k * kThreads;
          if (c < a.w_len) sm.lw[r][c] = x[k] > 0.f ? __log2f(x[k]) : -INFINITY;
        }
      }
    }

    float m_[GMAX], l_[GMAX], acc[GMAX][8];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      m_[g] = kNeg;
      l_[g] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    }

    const T* kbase = reinterpret_cast<const T*>(a.k) + (int64_t)h * a.s_kh + li * 8;
    const T* vbase = reinterpret_cast<const T*>(a.v) + (int64_t)h * a.s_vh + li * 8;
    int rows_read = 0;

    // Fused mode: the positions [ex0, n) not yet binned (label C, the exact set) are always read.
    // They are left out of the label scans and dealt round robin over the splits, appended to
    // each split's last scanned page, so that the recent window does not all fall to the split
    // owning the last block (at 20% that split read 64 rows above the ~210 of every other one, a
    // third batch of row loads that the merge waited for). Taken when it fits every split's last
    // page (every split has a block and no last page is full: the head's splits all decide
    // alike, from n, end and S); otherwise the exact set stays in the scans. Compiled up to two
    // query heads per KV head: past that the kernel has no registers to spare for it (it would
    // drop to one wave per SIMD).
    constexpr bool SPREAD = SELECT && GMAX <= 2;
    int ex0 = n;
    if constexpr (SPREAD) {
      const int e0 = min(max(end_h, 1), n);
      const int nb = (e0 + kThreads - 1) / kThreads, q = nb / S, r = nb % S;
      if (n - e0 <= kThreads * S && q >= 1 && q % PER != 0 && (r == 0 || (q + 1) % PER != 0)) ex0 = e0;
    }
    const int nblk = (ex0 + kThreads - 1) / kThreads;          // blocks the label scans cover
    const int nscan = DENSE ? 0 : max(0, (nblk - sp + S * PER - 1) / (S * PER));
    // pages: dense, kPage consecutive positions of [s0, s1); label scans, PER interleaved blocks
    for (int it = 0, p0 = s0; DENSE ? p0 < s1 : it < nscan; ++it, p0 += kPage) {
      const int pn = min(kPage, s1 - p0);
      int R;
      if constexpr (DENSE) {
        R = pn;
      } else {
        // lbl holds this page's labels: the first page's were loaded at the start, each later
        // page's while the previous page's rows were read
        __syncthreads();   // lw ready / previous page's list consumed
        // Position block_pos(it, u) + tid: the list in (u, wave, lane) order is ascending.
        bool sel[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int j = block_pos(it, u) + tid;
          lbl[u] = min(max(lbl[u], 0), a.w_len - 1);     // a bad label never indexes outside lw
          bool s = false;
          if (j < ex0) {
            if (per_head) {
              for (int g = 0; g < G; ++g) s |= sm.lw[g][lbl[u]] != -INFINITY;
            } else {
              s = sm.lw[0][lbl[u]] != -INFINITY;
            }
          }
          sel[u] = s;
        }
        const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        unsigned long long bal[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          bal[u] = __ballot(sel[u]);
          if (lane == 0) sm.scan[u][wave] = __popcll(bal[u]);
        }
        __syncthreads();
        int total = 0;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          int wbase = 0, tot_u = 0;
#pragma unroll
          for (int w2 = 0; w2 < kWaves; ++w2) {
            const int c2 = sm.scan[u][w2];
            if (w2 < wave) wbase += c2;
            tot_u += c2;
          }
          if (sel[u]) {
            const int o = total + wbase + __popcll(bal[u] & below);
            sm.u.list.pos[o] = block_pos(it, u) + tid;
            if (per_head) {
              for (int g = 0; g < G; ++g) sm.u.list.rlw[g][o] = sm.lw[g][lbl[u]];
            } else {
              sm.u.list.rlw[0][o] = sm.lw[0][lbl[u]];
            }
          }
          total += tot_u;
        }
        R = total;
        if constexpr (SPREAD) {
          if (it == nscan - 1 && ex0 < n) {   // room: the last page has at most kPage - kThreads positions
            const int nx = n > ex0 + sp ? (n - ex0 - sp + S - 1) / S : 0;
            const int cx = a.w_len - 1;                        // the exact set's slot
            for (int i = tid; i < nx; i += kThreads) {
              sm.u.list.pos[total + i] = ex0 + sp + S * i;
              if (per_head) {
                for (int g = 0; g < G; ++g) sm.u.list.rlw[g][total + i] = sm.lw[g][cx];
              } else {
                sm.u.list.rlw[0][total + i] = sm.lw[0][cx];
              }
            }
            R = total + nx;
          }
        }
        // the next page's labels load while this page's rows are read
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int j = block_pos(it + 1, u) + tid;
          lbl[u] = j < n ? (int)labrow[j] : 0;
        }
        __syncthreads();
      }
      rows_read += R;

      // ---- attention over the R rows of this page: every lane group issues U rows of K and V,
      // then consumes them; rows past R re-read the last row and are masked out.
      for (int base = 0; base < R; base += kWaves * RPI * U) {
        Raw kraw[U], vraw[U];
        int rr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          rr[u] = base + u * kWaves * RPI + wave * RPI + lg;
          const int rc = min(rr[u], R - 1);
          int pos;
          if constexpr (DENSE) pos = p0 + rc;
          else pos = sm.u.list.pos[rc];
          kraw[u] = *reinterpret_cast<const Raw*>(kbase + (int64_t)pos * a.s_kn);
          vraw[u] = *reinterpret_cast<const Raw*>(vbase + (int64_t)pos * a.s_vn);
        }
        float s[GMAX][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float kf[8];
          widen8(kraw[u], kf, (T*)nullptr);
          float lw0 = 0.f;
          if constexpr (!DENSE) lw0 = rr[u] < R ? sm.u.list.rlw[0][min(rr[u], R - 1)] : -INFINITY;
#pragma unroll
          for (int g = 0; g < GMAX; ++g) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) d = fmaf(qr[g][e], kf[e], d);
            d = row_sum<LPR>(d);
            float lw = lw0;
            if constexpr (!DENSE) {
              if (per_head && g < G) lw = rr[u] < R ? sm.u.list.rlw[g][min(rr[u], R - 1)] : -INFINITY;
            }
            s[g][u] = rr[u] < R ? d + lw : -INFINITY;
          }
        }
        float p[GMAX][U];
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
          float mx = m_[g];
#pragma unroll
          for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[g][u]);
          const float alpha = __builtin_amdgcn_exp2f(m_[g] - mx);
          float psum = 0.f;
#pragma unroll
          for (int u = 0; u < U; ++u) { p[g][u] = __builtin_amdgcn_exp2f(s[g][u] - mx); psum += p[g][u]; }
          l_[g] = fmaf(l_[g], alpha, psum);
          m_[g] = mx;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float vf[8];
          widen8(vraw[u], vf, (T*)nullptr);
#pragma unroll
          for (int g = 0; g < GMAX; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p[g][u], vf[e], acc[g][e]);
        }
      }
    }

    asm volatile("" ::"v"(touch));       // the translation touches above, long landed
    // ---- merge the lane groups of each wave ---------------------------------------------------
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        const float m2 = __shfl_xor(m_[g], o, 64);
        const float l2 = __shfl_xor(l_[g], o, 64);
        const float M = fmaxf(m_[g], m2);
        const float f1 = __builtin_amdgcn_exp2f(m_[g] - M), f2 = __builtin_amdgcn_exp2f(m2 - M);
        l_[g] = l_[g] * f1 + l2 * f2;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float a2 = __shfl_xor(acc[g][e], o, 64);
          acc[g][e] = acc[g][e] * f1 + a2 * f2;
        }
        m_[g] = M;
      }
    }
    if (lane < LPR) {
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (lane == 0) { sm.red_m[wave][g] = m_[g]; sm.red_l[wave][g] = l_[g]; }
#pragma unroll
        for (int e = 0; e < 8; ++e) sm.red_a[wave][g][li * 8 + e] = acc[g][e];
      }
    }
    __syncthreads();

    // ---- merge the waves; publish this workgroup's partial -------------------------------------
    // Partials are written with agent-scope stores (coherent across the XCDs' L2 caches), so the
    // workgroup only has to wait for its own stores before it counts itself in: no L2 write-back.
    const int64_t pidx = (int64_t)h * S + sp;
    for (int t = tid; t < G * D; t += kThreads) {
      const int g = t / D, dd = t % D;
      float M = kNeg;
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) M = fmaxf(M, sm.red_m[w2][g]);
      float L = 0.f, A = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) {
        const float f = __builtin_amdgcn_exp2f(sm.red_m[w2][g] - M);
        L = fmaf(sm.red_l[w2][g], f, L);
        A = fmaf(sm.red_a[w2][g][dd], f, A);
      }
      __hip_atomic_store(a.part_a + (pidx * G + g) * D + dd, A, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (dd == 0) {
        __hip_atomic_store(a.part_m + pidx * G + g, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.part_l + pidx * G + g, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (tid == 0) __hip_atomic_store(a.part_cnt + pidx, rows_read, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }  // attention workgroups
  if constexpr (AHEAD) {
    if (stager || (a.fold_stage && sp == S - 1)) {
      if (!stager) __syncthreads();    // the attention is done with sm.u
      InsPre<D> spre;
      insert_prefetch<D>(spre, a.st, a.ins, h, n + 1);
      insert_stage<D>(sm.u.tail, a.st, a.ins, h, spre, n + 1);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);       // this thread's stores have reached the coherence point
  __syncthreads();
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(a.counter + h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm.last = (old == S - 1 + (AHEAD && !a.fold_stage ? 1 : 0));
  }
  __syncthreads();
  if (!sm.last) return;
  // the staged insertion's words load beside the partials' (the stager's stores were
  // acknowledged before it counted in)
  StagePre stp;
  if constexpr (AHEAD) stage_prefetch<D>(stp, a.st, h);
  // ---- the last workgroup of head h merges the S partials ----------------------------------
  // One round of loads, all issued before the first wait: in wave 0, every split's (max, sum)
  // and row count spread over the lanes, first, so that the rescale factors can be computed
  // while the rest arrives; then this thread's accumulator columns (up to MB splits)
  // into registers. The partials are read with agent-scope loads (coherent across XCDs), so no
  // L2 invalidate is needed.
  const int64_t hb = (int64_t)h * S;
  const int cols4 = G * D / 4;
  const float* pa = a.part_a + hb * G * D;
  const int ncol0 = min(kThreads, cols4);
  const int nsg0 = kThreads / ncol0;
  const int sg0 = tid / ncol0, col0 = tid % ncol0;
  // wave 0: lane l holds head g = l % GMAX of splits l / GMAX + (64 / GMAX) * i
  constexpr int SPI = 64 / GMAX;                        // splits per round of lanes
  constexpr int kML = (kMaxS + SPI - 1) / SPI;
  const int gl = lane % GMAX;
  float mv[kML], lv[kML];
  int cpart = 0;
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < kML; ++i) {
      if (i * SPI < S) {                                // uniform
        const int s2 = lane / GMAX + SPI * i;
        const int e = min(s2, S - 1) * G + min(gl, G - 1);
        const float m0 = load_coherent(a.part_m + hb * G + e);
        const float l0 = load_coherent(a.part_l + hb * G + e);
        const bool ok = s2 < S && gl < G;
        mv[i] = ok ? m0 : kNeg;
        lv[i] = ok ? l0 : 0.f;
      }
    }
    for (int t = lane; t < S; t += 64)
      cpart += __hip_atomic_load(a.part_cnt + hb + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // branchless: out-of-range splits re-read split S-1 and get weight 0 below
  constexpr int MB = merge_batch<GMAX>();
  float4 va[MB];
#pragma unroll
  for (int k = 0; k < MB; ++k) {
    const int s2 = min(sg0 + k * nsg0, S - 1);
    va[k] = load_coherent4(pa + ((int64_t)s2 * cols4 + col0) * 4);
  }
  if (wave == 0) {
    const int g = gl;
    float M = kNeg;
#pragma unroll
    for (int i = 0; i < kML; ++i)
      if (i * SPI < S) M = fmaxf(M, mv[i]);
#pragma unroll
    for (int o = GMAX; o < 64; o <<= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < kML; ++i) {
      if (i * SPI < S) {
        const int s2 = lane / GMAX + SPI * i;
        const float f = __builtin_amdgcn_exp2f(mv[i] - M);
        if (s2 < S && g < G) sm.u.mrg.f[s2 * G + g] = f;
        den = fmaf(f, lv[i], den);
      }
    }
#pragma unroll
    for (int o = GMAX; o < 64; o <<= 1) den += __shfl_xor(den, o, 64);
    if (lane < G) sm.gden[lane] = den;
    cpart = wave_sum_i(cpart);
    if (lane == 0) sm.red_i[0] = cpart;
  }
  if constexpr (AHEAD) stage_publish(stp, sm.stage_hdr);
  __syncthreads();
  // Every workgroup of this head has read the index state and the labels (each counted itself in
  // after its scan, the stager after its stores), so the state may now move to the next step:
  // commit the staged insertion of the keys that leave the window at length n + 1, as ssa_insert
  // would bin them at the start of the next step. The one-key stage is a few stores that use no
  // LDS, issued here so that they overlap the merge; a split or a general stage runs after it.
  bool committed = false;
  if constexpr (AHEAD) {
    if (sm.stage_hdr[0] == kStageOne) {
      insert_commit<D>(sm.u.tail, a.st, a.ins, h, n + 1, stp, sm.stage_hdr);
      committed = true;
    }
  }
  // rescaled sum of the accumulators: float4 columns, splits strided over thread groups
  for (int c0 = 0; c0 < cols4; c0 += kThreads) {
    const int ncol = min(kThreads, cols4 - c0);
    const int nsg = kThreads / ncol;
    const int sg = tid / ncol, col = c0 + tid % ncol;
    float4 acc4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (sg < nsg) {
      const int g = col * 4 / D;
      int s2 = sg;
      if (c0 == 0) {                 // the batch already in registers
#pragma unroll
        for (int k = 0; k < MB; ++k) {
          const int sk = sg + k * nsg;
          const float f = sk < S ? sm.u.mrg.f[min(sk, S - 1) * G + g] : 0.f;
          acc4.x = fmaf(f, va[k].x, acc4.x); acc4.y = fmaf(f, va[k].y, acc4.y);
          acc4.z = fmaf(f, va[k].z, acc4.z); acc4.w = fmaf(f, va[k].w, acc4.w);
        }
        s2 = sg + MB * nsg;
      }
#pragma unroll 8
      for (; s2 < S; s2 += nsg) {
        const float f = sm.u.mrg.f[s2 * G + g];
        const float4 v4 = load_coherent4(pa + ((int64_t)s2 * cols4 + col) * 4);
        acc4.x = fmaf(f, v4.x, acc4.x); acc4.y = fmaf(f, v4.y, acc4.y);
        acc4.z = fmaf(f, v4.z, acc4.z); acc4.w = fmaf(f, v4.w, acc4.w);
      }
    }
    if (c0 > 0) __syncthreads();     // the previous chunk's sums have been read
    sm.u.mrg.acc[tid] = acc4;
    __syncthreads();
    if (tid < ncol) {
      float4 v = sm.u.mrg.acc[tid];
      for (int s3 = 1; s3 < nsg; ++s3) {
        const float4 w4 = sm.u.mrg.acc[s3 * ncol + tid];
        v.x += w4.x; v.y += w4.y; v.z += w4.z; v.w += w4.w;
      }
      const int e0 = (c0 + tid) * 4, g = e0 / D, dd = e0 % D;
      const float den = sm.gden[g];
      const int64_t o = (int64_t)(h * G + g) * a.s_oh + dd;
      store_out(a.out, a.out_dtype, o + 0, v.x / den);
      store_out(a.out, a.out_dtype, o + 1, v.y / den);
      store_out(a.out, a.out_dtype, o + 2, v.z / den);
      store_out(a.out, a.out_dtype, o + 3, v.w / den);
    }
  }
  if (tid == 0) {
    if (a.cnt_out) a.cnt_out[h] = sm.red_i[0];
    __hip_atomic_store(a.counter + h, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (AHEAD) {
    if (!committed) {
      __syncthreads();                                   // the merge is done with sm.u
      insert_commit<D>(sm.u.tail, a.st, a.ins, h, n + 1, stp, sm.stage_hdr);
    }
  }
}

enum Mode { kDense = 0, kLabelled = 1, kFused = 2, kFusedAhead = 3 };


// Slot counts up to 256 (one scoring round) have their own fused kernels at d = 128: the selection's
// per-slot registers, LDS and code then cover 256 slots instead of 1024.
template <typename T, int D, int GMAX>
hipError_t launch_decode_t(const DecodeParams& p, int mode, hipStream_t st) {
  dim3 grid(p.S + (mode == kFusedAhead && !p.fold_stage ? 1 : 0), p.n_heads);
  const bool small = D == 128 && p.st.C <= 256;
  if (mode == kDense) hipLaunchKernelGGL((decode_kernel<T, D, GMAX, true>), grid, dim3(kThreads), 0, st, p);
  else if (mode == kLabelled) hipLaunchKernelGGL((decode_kernel<T, D, GMAX, false>), grid, dim3(kThreads), 0, st, p);
  else if (mode == kFused && small)
    hipLaunchKernelGGL((decode_kernel<T, D, GMAX, false, true, false, (D == 128 ? 256 : kMaxC)>), grid, dim3(kThreads), 0, st, p);
  else if (mode == kFused) hipLaunchKernelGGL((decode_kernel<T, D, GMAX, false, true>), grid, dim3(kThreads), 0, st, p);
  else if (small)
    hipLaunchKernelGGL((decode_kernel<T, D, GMAX, false, true, true, (D == 128 ? 256 : kMaxC)>), grid, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((decode_kernel<T, D, GMAX, false, true, true>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_decode_d(const DecodeParams& p, int dense, hipStream_t st) {
  if (p.G <= 1) return launch_decode_t<T, D, 1>(p, dense, st);
  if (p.G <= 2) return launch_decode_t<T, D, 2>(p, dense, st);
  if (p.G <= 4) return launch_decode_t<T, D, 4>(p, dense, st);
  if (p.G <= 8) return launch_decode_t<T, D, 8>(p, dense, st);
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_decode_ty(const DecodeParams& p, int d, int dense, hipStream_t st) {
  switch (d) {
    case 16: return launch_decode_d<T, 16>(p, dense, st);
    case 32: return launch_decode_d<T, 32>(p, dense, st);
    case 64: return launch_decode_d<T, 64>(p, dense, st);
    case 128: return launch_decode_d<T, 128>(p, dense, st);
    case 256: return launch_decode_d<T, 256>(p, dense, st);
  }
  return hipErrorInvalidValue;
}

// One translation unit per KV dtype instantiates launch_decode_ty (decode_bf16.hip, decode_f16.hip,
// decode_f32.hip), so the kernel variants compile in parallel.
hipError_t launch_decode_bf16(const DecodeParams& p, int d, int mode, hipStream_t st);
hipError_t launch_decode_f16(const DecodeParams& p, int d, int mode, hipStream_t st);
hipError_t launch_decode_f32(const DecodeParams& p, int d, int mode, hipStream_t st);

}  // namespace ssa
