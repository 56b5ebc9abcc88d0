/* CPU oracle for the cluster index: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this file, as the
 * checker; the product (libssa_hip.so) never links or calls it.
 *
 * A scalar restatement of the reference's index algorithm in the fixed ("canonical") fp32
 * order of operations that the GPU kernels use, so that labels, selections and splits can be
 * compared bit for bit. It is written from the reference's semantics, not from the HIP code:
 *   insertion   _bin_kernel           src/ssa/kernels/sphere_fused.py:171-227
 *   split       _split_cluster        src/ssa/kernels/sphere_fused.py:49-167
 *               (= _bisect_padded     src/ssa/attn/sphere_gpu.py:76-102)
 *   selection   labels_and_weights    src/ssa/attn/sphere_gpu.py:412-442 and _rank_mask :402-410
 *               (sum_share / per_head / max / max_rel), _score_kernel src/ssa/kernels/sphere_fused.py:231-253
 *   prefill     _build / _bin         src/ssa/attn/sphere_gpu.py:166-219
 *               spherical_kmeans      src/ssa/attn/clusterkv.py:27-46
 *               _to8 / _refresh8      src/ssa/kernels/sphere_fused.py:394-405
 * Canonical order (the definition both sides implement):
 *   dot(a,b)   8 chains, chain j = fma over elements j, j+8, ...; ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7))
 *   scoring dot (selection scores only): 8 chains, chain j = fma over elements j*d/8 .. (j+1)*d/8-1
 *              in order, combined in the same tree
 *   unit(x)    x / max(sqrt(dot(x,x)), 1e-12)
 *   q8(u)      floor(u*127 + 0.5), multiply and add rounded separately
 *   exp(x<=0)  Cody-Waite by ln2 (hi 0.693145751953125, lo 1.42860682030941723e-6), degree-7
 *              Taylor in Horner form with fma, times 2^k; 0 below -87
 *   sums       left to right from +0; softmax denominators as a pairwise tree over the C slots;
 *              prefill sums (key sum, squared lengths, cluster sums) in blocks of 256 keys (each
 *              block left to right from +0), then the block sums left to right from +0
 * Build: oracle/Makefile (gcc -O3 -mfma -ffp-contract=off, so only the explicit fmaf are fused).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KB 256

float canon_dot(const float* a, const float* b, int d) {
  float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < d; i += 8)
    for (int j = 0; j < 8; ++j) c[j] = fmaf(a[i + j], b[i + j], c[j]);
  return ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
}

/* Scoring dot (the selection's scores): chain j sums elements [j*d/8, (j+1)*d/8) left to right
 * with fma; the chains are combined as in canon_dot. */
float canon_dot_chunked(const float* a, const float* b, int d) {
  float c[8];
  const int e = d / 8;
  for (int j = 0; j < 8; ++j) {
    c[j] = 0.f;
    for (int k = 0; k < e; ++k) c[j] = fmaf(a[j * e + k], b[j * e + k], c[j]);
  }
  return ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
}

static float dot_i8(const int8_t* a, const float* b, int d) {
  float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < d; i += 8)
    for (int j = 0; j < 8; ++j) c[j] = fmaf((float)a[i + j], b[i + j], c[j]);
  return ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
}

static void unit(const float* x, float* y, int d) {
  float r = fmaxf(sqrtf(canon_dot(x, x, d)), 1e-12f);
  for (int i = 0; i < d; ++i) y[i] = x[i] / r;
}

int8_t canon_q8(float u) {
  volatile float t = u * 127.0f;
  t = t + 0.5f;
  return (int8_t)floorf(t);
}

static void q8_unit(const float* x, int8_t* out, int d) {
  float r = fmaxf(sqrtf(canon_dot(x, x, d)), 1e-12f);
  for (int i = 0; i < d; ++i) out[i] = canon_q8(x[i] / r);
}

float canon_exp(float x) {
  if (!(x >= -87.0f)) return 0.0f;
  float k = rintf(x * 1.44269504088896341f);
  float r = fmaf(-k, 0.693145751953125f, x);
  r = fmaf(-k, 1.42860682030941723e-06f, r);
  float p = 1.98412698412698413e-04f;
  p = fmaf(p, r, 1.38888888888888889e-03f);
  p = fmaf(p, r, 8.33333333333333333e-03f);
  p = fmaf(p, r, 4.16666666666666667e-02f);
  p = fmaf(p, r, 1.66666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ki = (int)k;
  union { uint32_t u; float f; } s;
  s.u = (uint32_t)(ki + 127) << 23;
  return p * s.f;
}

/* One KV head's state; arrays are that head's rows. */
typedef struct {
  int C, d, ms, summary_bits, shared_dirs;
  int32_t* n_c;
  float* sum_dir; int8_t* dir8; float* cent; int8_t* cent8;
  float* mmax; float* mmin; int32_t* count;
  float* ksum; float* mu_ref; float* rbar; float* cap; float* vthr;
  int32_t* flags; int32_t* end; int32_t* nsplit;
  int16_t* labels;
} canon_head_t;

/* ---- split ------------------------------------------------------------------------------ */

static void kn_of(const float* K, int d, const float* mu, int pos, float magc, float* out) {
  for (int i = 0; i < d; ++i) out[i] = (K[(int64_t)pos * d + i] - mu[i]) / magc;
}

/* Side sums of the members' unit directions: members in blocks of SUM_BLOCK (in member order),
 * each block's side sums left to right from +0, then the block sums added left to right from +0. */
#define SUM_BLOCK 16
static void ordered_sums(const float* K, int d, const float* mu, const int* mem, const float* mag, const int* side,
                         int m, float* s0, float* s1, int* n1) {
  float* kn = (float*)malloc(sizeof(float) * d);
  float* b0 = (float*)malloc(sizeof(float) * d);
  float* b1 = (float*)malloc(sizeof(float) * d);
  for (int i = 0; i < d; ++i) { s0[i] = 0.f; s1[i] = 0.f; }
  *n1 = 0;
  for (int jb = 0; jb < m; jb += SUM_BLOCK) {
    for (int i = 0; i < d; ++i) { b0[i] = 0.f; b1[i] = 0.f; }
    for (int j = jb; j < m && j < jb + SUM_BLOCK; ++j) {
      kn_of(K, d, mu, mem[j], fmaxf(mag[j], 1e-12f), kn);
      if (side[j]) { for (int i = 0; i < d; ++i) b1[i] = b1[i] + kn[i]; ++*n1; }
      else for (int i = 0; i < d; ++i) b0[i] = b0[i] + kn[i];
    }
    for (int i = 0; i < d; ++i) { s0[i] = s0[i] + b0[i]; s1[i] = s1[i] + b1[i]; }
  }
  free(kn); free(b0); free(b1);
}

/* The bisection of _bisect_padded (src/ssa/attn/sphere_gpu.py:76-102) on the members mem[0..m)
 * (key rows of K, centred by mu, lengths mag): 2-means from the first member and the member least
 * similar to it, 4 updates, then the final sides; a result with fewer than 25% or more than 75% of
 * the members on side 1 is replaced by the cut at the median projection on b - a (stable order). */
void canon_bisect(const float* K, int d, const float* mu, const int* mem, const float* mag, int m, int* side) {
  float* proj = (float*)malloc(sizeof(float) * (size_t)(m > 0 ? m : 1));
  float* kn = (float*)malloc(sizeof(float) * d);
  float* a = (float*)malloc(sizeof(float) * d);
  float* b = (float*)malloc(sizeof(float) * d);
  float* s0 = (float*)malloc(sizeof(float) * d);
  float* s1 = (float*)malloc(sizeof(float) * d);
  float* vs = (float*)malloc(sizeof(float) * d);
  kn_of(K, d, mu, mem[0], fmaxf(mag[0], 1e-12f), a);
  float lo = 0.f;
  int far = -1;
  for (int j = 0; j < m; ++j) {
    kn_of(K, d, mu, mem[j], fmaxf(mag[j], 1e-12f), kn);
    float sim = canon_dot(kn, a, d);
    if (far < 0 || sim < lo) { lo = sim; far = j; }
  }
  kn_of(K, d, mu, mem[far], fmaxf(mag[far], 1e-12f), b);
  int n1 = 0;
  for (int it = 0; it < 4; ++it) {
    for (int j = 0; j < m; ++j) {
      kn_of(K, d, mu, mem[j], fmaxf(mag[j], 1e-12f), kn);
      side[j] = canon_dot(kn, b, d) > canon_dot(kn, a, d);
    }
    ordered_sums(K, d, mu, mem, mag, side, m, s0, s1, &n1);
    if (m - n1 > 0) unit(s0, a, d);
    if (n1 > 0) unit(s1, b, d);
  }
  for (int i = 0; i < d; ++i) vs[i] = b[i] - a[i];
  n1 = 0;
  for (int j = 0; j < m; ++j) {
    kn_of(K, d, mu, mem[j], fmaxf(mag[j], 1e-12f), kn);
    side[j] = canon_dot(kn, b, d) > canon_dot(kn, a, d);
    proj[j] = canon_dot(kn, vs, d);
    n1 += side[j];
  }
  float mf = (float)m, n1f = (float)n1;
  if (n1f < 0.25f * mf || n1f > 0.75f * mf) {
    int half = m / 2;
    for (int j = 0; j < m; ++j) {
      int rank = 0;
      for (int i = 0; i < m; ++i) rank += (proj[i] < proj[j] || (proj[i] == proj[j] && i < j));
      side[j] = rank >= half;
    }
  }
  free(proj); free(kn); free(a); free(b); free(s0); free(s1); free(vs);
}

static void split(canon_head_t* H, const float* K, int c, int nw, int stop) {
  const int d = H->d;
  int* mem = (int*)malloc(sizeof(int) * (size_t)(stop > 0 ? stop : 1));
  int m = 0;
  for (int j = 1; j < stop; ++j)
    if (H->labels[j] == c && m < H->ms) mem[m++] = j;
  if (m < 2) { free(mem); return; }
  float* mag = (float*)malloc(sizeof(float) * m);
  int* side = (int*)malloc(sizeof(int) * m);
  float* kr = (float*)malloc(sizeof(float) * d);
  float* a = (float*)malloc(sizeof(float) * d);
  float* b = (float*)malloc(sizeof(float) * d);
  float* s0 = (float*)malloc(sizeof(float) * d);
  float* s1 = (float*)malloc(sizeof(float) * d);
  for (int j = 0; j < m; ++j) {
    for (int i = 0; i < d; ++i) kr[i] = K[(int64_t)mem[j] * d + i] - H->mu_ref[i];
    mag[j] = sqrtf(canon_dot(kr, kr, d));
  }
  canon_bisect(K, d, H->mu_ref, mem, mag, m, side);
  int n1 = 0;
  ordered_sums(K, d, H->mu_ref, mem, mag, side, m, s0, s1, &n1);
  float x0 = 0.f, x1 = 0.f, y0 = INFINITY, y1 = INFINITY;
  for (int j = 0; j < m; ++j) {
    if (side[j]) { x1 = fmaxf(x1, mag[j]); y1 = fminf(y1, mag[j]); H->labels[mem[j]] = (int16_t)nw; }
    else { x0 = fmaxf(x0, mag[j]); y0 = fminf(y0, mag[j]); }
  }
  float* r0 = H->sum_dir + (int64_t)c * d;
  float* r1 = H->sum_dir + (int64_t)nw * d;
  memcpy(r0, s0, sizeof(float) * d);
  memcpy(r1, s1, sizeof(float) * d);
  unit(s0, a, d);
  unit(s1, b, d);
  memcpy(H->cent + (int64_t)c * d, a, sizeof(float) * d);
  memcpy(H->cent + (int64_t)nw * d, b, sizeof(float) * d);
  for (int i = 0; i < d; ++i) {
    if (H->dir8) { H->dir8[(int64_t)c * d + i] = canon_q8(a[i]); H->dir8[(int64_t)nw * d + i] = canon_q8(b[i]); }
    if (H->cent8) { H->cent8[(int64_t)c * d + i] = canon_q8(a[i]); H->cent8[(int64_t)nw * d + i] = canon_q8(b[i]); }
  }
  H->mmax[c] = x0; H->mmax[nw] = x1;
  H->mmin[c] = y0; H->mmin[nw] = y1;
  H->count[c] = m - n1; H->count[nw] = n1;
  *H->n_c = nw + 1;
  *H->nsplit += 1;
  free(mem); free(mag); free(side); free(kr); free(a); free(b); free(s0); free(s1);
}

/* ---- division after a fit ------------------------------------------------------------------ */
/* One round of SphereIndexGPU._split_overflow for one head (src/ssa/attn/sphere_gpu.py:307-391):
 * the clusters over the cap (count > cap_now, slot < n_c, count >= 2) are taken in slot order;
 * cluster i of the head has global rank rank0 + i in the round (heads in order), and spare
 * slots are handed out within batches of 64 ranks: base starts each batch at n_c and grows by
 * every cluster's new-part count, kept or not. nmeans: k = max(2, ceil(count * split_factor /
 * cap_now)) parts by cosine k-means from the members at j*m/k (_kmeans_padded :56-73), iters
 * updates then a final assignment (lowest part on ties); otherwise the bisection of the
 * insertion's split (_bisect_padded :76-102). Non-empty parts are numbered in order; part 0 keeps
 * the slot, part p > 0 takes base + p - 1; a cluster is split when all fit in C. Sums run over
 * members in position order. The int8 copies are left to a refresh. Returns the clusters split;
 * *n_over receives the number of clusters over the cap. */
/* Cosine k-means of the members into k parts (_kmeans_padded, src/ssa/attn/sphere_gpu.py:56-73):
 * seeds at members j*m/k, `iters` updates (an empty part keeps its centroid), then the final
 * assignment; argmax ties to the lowest part. part[j] receives member j's part. */
void canon_kmeans_parts(const float* K, int d, const float* mu, const int* mem, const float* mag, int m, int k,
                         int iters, int* part) {
  float* cent = (float*)malloc(sizeof(float) * (size_t)k * d);
  float* sums = (float*)malloc(sizeof(float) * (size_t)k * d);
  int* cnt = (int*)malloc(sizeof(int) * k);
  float* kn = (float*)malloc(sizeof(float) * d);
  for (int p = 0; p < k; ++p) {
    int j = (int)(((int64_t)p * m) / k);
    if (j > m - 1) j = m - 1;
    kn_of(K, d, mu, mem[j], fmaxf(mag[j], 1e-12f), cent + (int64_t)p * d);
  }
  for (int it = 0; it <= iters; ++it) {
    for (int j = 0; j < m; ++j) {
      kn_of(K, d, mu, mem[j], fmaxf(mag[j], 1e-12f), kn);
      int best = 0;
      float bs = canon_dot(kn, cent, d);
      for (int p = 1; p < k; ++p) {
        float sc = canon_dot(kn, cent + (int64_t)p * d, d);
        if (sc > bs) { bs = sc; best = p; }
      }
      part[j] = best;
    }
    if (it == iters) break;
    for (int p = 0; p < k; ++p) { cnt[p] = 0; for (int i = 0; i < d; ++i) sums[(int64_t)p * d + i] = 0.f; }
    for (int j = 0; j < m; ++j) {
      kn_of(K, d, mu, mem[j], fmaxf(mag[j], 1e-12f), kn);
      float* sp = sums + (int64_t)part[j] * d;
      for (int i = 0; i < d; ++i) sp[i] = sp[i] + kn[i];
      cnt[part[j]] += 1;
    }
    for (int p = 0; p < k; ++p)
      if (cnt[p] > 0) unit(sums + (int64_t)p * d, cent + (int64_t)p * d, d);
  }
  free(cent); free(sums); free(cnt); free(kn);
}

int canon_split_fit_head(canon_head_t* H, const float* K, int start, int end, float split_factor, float cap_now,
                         int nmeans, int iters, int rank0, int* n_over) {
  const int C = H->C, d = H->d;
  int* list = (int*)malloc(sizeof(int) * C);
  int no = 0;
  for (int c = 0; c < *H->n_c && c < C; ++c)
    if ((float)H->count[c] > cap_now && H->count[c] >= 2) list[no++] = c;
  *n_over = no;
  int n_cur = *H->n_c, base = n_cur, done = 0;
  int* mem = (int*)malloc(sizeof(int) * (size_t)(end > 0 ? end : 1));
  int* part = (int*)malloc(sizeof(int) * (size_t)(end > 0 ? end : 1));
  float* mag = (float*)malloc(sizeof(float) * (size_t)(end > 0 ? end : 1));
  float* kr = (float*)malloc(sizeof(float) * d);
  float* kn = (float*)malloc(sizeof(float) * d);
  float* sums = NULL;
  int* sizes = NULL; int* renum = NULL; int* slot = NULL;
  for (int i = 0; i < no; ++i) {
    const int c = list[i];
    if ((rank0 + i) % 64 == 0) base = n_cur;
    if (!nmeans) {
      /* bisection: the insertion's split, into slot base when it fits */
      if (base + 1 <= C) {
        split(H, K, c, base, end);
        if (*H->n_c == base + 1) { n_cur = base + 1; ++done; }
      }
      base += 1;
      continue;
    }
    int m = 0;
    for (int j = start; j < end; ++j)
      if (H->labels[j] == c) mem[m++] = j;
    for (int j = 0; j < m; ++j) {
      for (int t = 0; t < d; ++t) kr[t] = K[(int64_t)mem[j] * d + t] - H->mu_ref[t];
      mag[j] = sqrtf(canon_dot(kr, kr, d));
    }
    const float kf = ceilf(((float)m * split_factor) / cap_now);
    int k = kf < 2.f ? 2 : (int)kf;
    canon_kmeans_parts(K, d, H->mu_ref, mem, mag, m, k, iters, part);
    sums = (float*)realloc(sums, sizeof(float) * (size_t)k * d);
    sizes = (int*)realloc(sizes, sizeof(int) * (size_t)k);
    renum = (int*)realloc(renum, sizeof(int) * (size_t)k);
    slot = (int*)realloc(slot, sizeof(int) * (size_t)k);
    int nz = 0;
    for (int p = 0; p < k; ++p) sizes[p] = 0;
    for (int j = 0; j < m; ++j) sizes[part[j]] += 1;
    for (int p = 0; p < k; ++p) renum[p] = sizes[p] > 0 ? nz++ : -1;
    const int extra = nz - 1;
    if (extra > 0 && base + extra <= C) {
      for (int p = 0; p < nz; ++p) slot[p] = p == 0 ? c : base + p - 1;
      for (int p = 0; p < nz; ++p) {
        const int s = slot[p];
        for (int t = 0; t < d; ++t) sums[(int64_t)p * d + t] = 0.f;
        H->mmax[s] = 0.f; H->mmin[s] = INFINITY; H->count[s] = 0;
      }
      for (int j = 0; j < m; ++j) {
        const int p = renum[part[j]], s = slot[p];
        kn_of(K, d, H->mu_ref, mem[j], fmaxf(mag[j], 1e-12f), kn);
        float* sp = sums + (int64_t)p * d;
        for (int t = 0; t < d; ++t) sp[t] = sp[t] + kn[t];
        H->mmax[s] = fmaxf(H->mmax[s], mag[j]);
        H->mmin[s] = fminf(H->mmin[s], mag[j]);
        H->count[s] += 1;
        H->labels[mem[j]] = (int16_t)s;
      }
      for (int p = 0; p < nz; ++p) {
        const int s = slot[p];
        memcpy(H->sum_dir + (int64_t)s * d, sums + (int64_t)p * d, sizeof(float) * d);
        unit(sums + (int64_t)p * d, H->cent + (int64_t)s * d, d);
      }
      n_cur += extra;
      *H->n_c = n_cur;
      *H->nsplit += extra;
      ++done;
    }
    base += extra > 0 ? extra : 0;
  }
  free(list); free(mem); free(part); free(mag); free(kr); free(kn); free(sums); free(sizes); free(renum); free(slot);
  return done;
}

/* ---- insertion ---------------------------------------------------------------------------- */

/* K: this head's keys widened to fp32, [capacity, d]. */
void canon_insert(canon_head_t* H, const float* K, int n, int window, float delta, float capk, int reset_at,
                  int var_min) {
  const int d = H->d, C = H->C;
  int n_act = *H->n_c;
  const int old_end = *H->end;
  int new_end = n - window;
  if (new_end < 1) new_end = 1;
  if (new_end < old_end) new_end = old_end;
  float* ks = (float*)malloc(sizeof(float) * d);
  float* kr = (float*)malloc(sizeof(float) * d);
  float* kn = (float*)malloc(sizeof(float) * d);
  float* sd = (float*)malloc(sizeof(float) * d);
  memcpy(ks, H->ksum, sizeof(float) * d);
  const float cap = *H->cap, vthr = *H->vthr;
  for (int p = old_end; p < new_end && n_act > 0; ++p) {
    const float* k = K + (int64_t)p * d;
    for (int i = 0; i < d; ++i) { ks[i] = ks[i] + k[i]; kr[i] = k[i] - H->mu_ref[i]; }
    const float mag = sqrtf(canon_dot(kr, kr, d));
    const float magc = fmaxf(mag, 1e-12f);
    for (int i = 0; i < d; ++i) kn[i] = kr[i] / magc;
    float best = 0.f;
    int row = -1;
    for (int c = 0; c < n_act; ++c) {
      float sc = (H->summary_bits == 8 && !H->shared_dirs && H->cent8) ? dot_i8(H->cent8 + (int64_t)c * d, kn, d)
                                                                       : canon_dot(H->cent + (int64_t)c * d, kn, d);
      if (row < 0 || sc > best) { best = sc; row = c; }
    }
    float* sdr = H->sum_dir + (int64_t)row * d;
    for (int i = 0; i < d; ++i) { sdr[i] = sdr[i] + kn[i]; sd[i] = sdr[i]; }
    const float sdsq = canon_dot(sd, sd, d);
    const float sdn = sqrtf(sdsq);
    H->mmax[row] = fmaxf(H->mmax[row], mag);
    H->mmin[row] = fminf(H->mmin[row], mag);
    const int cn = H->count[row] + 1;
    H->count[row] = cn;
    H->labels[p] = (int16_t)row;
    const float cnf = (float)cn;
    const int wide = (1.0f - sdsq / (cnf * cnf) > vthr) && (cn >= var_min);
    const int over = cnf > fmaxf(cap, capk * (float)p);
    if (H->dir8)
      for (int i = 0; i < d; ++i) H->dir8[(int64_t)row * d + i] = canon_q8(sd[i] / fmaxf(sdn, 1e-12f));
    if ((over || wide) && n_act < C && cn >= 2 && cn <= H->ms) {
      split(H, K, row, n_act, p + 1);
      n_act += 1;
    }
  }
  const float nb = (float)(new_end - 1);
  for (int i = 0; i < d; ++i) { H->ksum[i] = ks[i]; kr[i] = ks[i] / fmaxf(nb, 1.f) - H->mu_ref[i]; }
  const float dist = sqrtf(canon_dot(kr, kr, d));
  const int moved = (dist > delta * *H->rbar) && (nb > 0.f);
  *H->flags = *H->flags | (moved ? 1 : 0) | ((n_act >= reset_at) ? 2 : 0);
  *H->end = new_end;
  free(ks); free(kr); free(kn); free(sd);
}

/* ---- selection ---------------------------------------------------------------------------- */

static void rank_take(const float* key, const int* cnt, int n_act, int C, int64_t need, float* w) {
  for (int c = 0; c < C; ++c) {
    int live = c < n_act && cnt[c] > 0;
    int64_t before = 0;
    if (live)
      for (int j = 0; j < n_act; ++j)
        if (key[j] > key[c] || (key[j] == key[c] && j < c)) before += cnt[j];
    w[c] = (live && before < need) ? 1.f : 0.f;
  }
}

/* q: this head's G query rows as fp32 [G, d]; w: [rows, C+1] (rows = G for per_head, else 1).
 * group: 0 sum_share, 1 per_head, 2 max, 3 max_rel. */
void canon_select(const canon_head_t* H, const float* q, int G, double budget, int group, float scale, float* w) {
  const int d = H->d, C = H->C;
  const int rows = group == 1 ? G : 1;
  const int nb = *H->end - 1;
  const double needd = nb > 0 ? ceil(budget * (double)nb) : 0.0;
  const int64_t need = (int64_t)needd;
  for (int r = 0; r < rows; ++r) {
    w[(int64_t)r * (C + 1) + C] = 1.f;
    if (nb <= 0 || need <= 0)
      for (int c = 0; c < C; ++c) w[(int64_t)r * (C + 1) + c] = 0.f;
  }
  if (nb <= 0 || need <= 0) return;
  const int n_act = *H->n_c;
  float* z = (float*)malloc(sizeof(float) * (size_t)G * C);
  float* key = (float*)malloc(sizeof(float) * C);
  float* t = (float*)malloc(sizeof(float) * C);
  float* dv = (float*)malloc(sizeof(float) * d);
  int* cnt = (int*)malloc(sizeof(int) * C);
  for (int c = 0; c < C; ++c) {
    const int live = c < n_act && H->count[c] > 0;
    cnt[c] = live ? H->count[c] : 0;
    if (!live) { for (int g = 0; g < G; ++g) z[(int64_t)g * C + c] = -INFINITY; continue; }
    for (int i = 0; i < d; ++i)
      dv[i] = (H->summary_bits == 8 && H->dir8) ? (float)H->dir8[(int64_t)c * d + i] : H->sum_dir[(int64_t)c * d + i];
    const float nrm = fmaxf(sqrtf(canon_dot_chunked(dv, dv, d)), 1e-12f);
    for (int g = 0; g < G; ++g) {
      const float p = canon_dot_chunked(q + (int64_t)g * d, dv, d) / nrm;
      const float e = p >= 0.f ? H->mmax[c] * p : H->mmin[c] * p;
      z[(int64_t)g * C + c] = group == 1 ? e : e * scale;
    }
  }
  if (group == 1) {
    for (int g = 0; g < G; ++g) rank_take(z + (int64_t)g * C, cnt, n_act, C, need, w + (int64_t)g * (C + 1));
  } else {
    if (group == 0) {
      for (int g = 0; g < G; ++g) {
        float* zg = z + (int64_t)g * C;
        float zm = -INFINITY;
        for (int c = 0; c < C; ++c) zm = fmaxf(zm, zg[c]);
        for (int c = 0; c < C; ++c) { zg[c] = cnt[c] > 0 ? canon_exp(zg[c] - zm) : 0.f; t[c] = zg[c]; }
        for (int half = C >> 1; half >= 1; half >>= 1)
          for (int c = 0; c < half; ++c) t[c] = t[c] + t[c + half];
        const float tot = t[0];
        for (int c = 0; c < C; ++c) zg[c] = zg[c] / tot;
      }
      for (int c = 0; c < C; ++c) {
        float s = 0.f;
        for (int g = 0; g < G; ++g) s = s + z[(int64_t)g * C + c];
        key[c] = cnt[c] > 0 ? s : -INFINITY;
      }
    } else {
      float zmx[64];
      for (int g = 0; g < G; ++g) {
        float zm = -INFINITY;
        for (int c = 0; c < C; ++c) zm = fmaxf(zm, z[(int64_t)g * C + c]);
        zmx[g] = group == 3 ? zm : 0.f;
      }
      for (int c = 0; c < C; ++c) {
        float s = -INFINITY;
        for (int g = 0; g < G; ++g) s = fmaxf(s, z[(int64_t)g * C + c] - zmx[g]);
        key[c] = cnt[c] > 0 ? s : -INFINITY;
      }
    }
    rank_take(key, cnt, n_act, C, need, w);
  }
  free(z); free(key); free(t); free(dv); free(cnt);
}

/* ---- prefill ------------------------------------------------------------------------------- */

/* Nearest centroid: argmax of the canonical dot, lowest index on ties; NaN scores never win, and
 * a key whose every score is NaN (a non-finite key) joins cluster 0, the index torch.argmax
 * returns on a row of NaNs. */
static void assign_all(const float* xn, int nb, int d, const float* cent, int nc, int* as) {
  for (int j = 0; j < nb; ++j) {
    float best = 0.f;
    int bi = -1;
    for (int c = 0; c < nc; ++c) {
      float sc = canon_dot(xn + (int64_t)j * d, cent + (int64_t)c * d, d);
      if (sc == sc && (bi < 0 || sc > best)) { best = sc; bi = c; }
    }
    as[j] = bi < 0 ? 0 : bi;
  }
}

/* Blocked sums of xn by cluster: per block of KB keys a left-to-right sum per cluster, then a
 * left-to-right sum over blocks. out [ncl, d], cnt [ncl]. */
static void blocked_sums(const float* xn, int nb, int d, const int* as, int ncl, float* out, int* cnt) {
  float* part = (float*)malloc(sizeof(float) * (size_t)ncl * d);
  memset(out, 0, sizeof(float) * (size_t)ncl * d);
  memset(cnt, 0, sizeof(int) * ncl);
  for (int b0 = 0; b0 < nb; b0 += KB) {
    memset(part, 0, sizeof(float) * (size_t)ncl * d);
    const int b1 = b0 + KB < nb ? b0 + KB : nb;
    for (int j = b0; j < b1; ++j) {
      float* pr = part + (int64_t)as[j] * d;
      for (int i = 0; i < d; ++i) pr[i] = pr[i] + xn[(int64_t)j * d + i];
      cnt[as[j]] += 1;
    }
    for (int64_t e = 0; e < (int64_t)ncl * d; ++e) out[e] = out[e] + part[e];
  }
  free(part);
}

/* (Re)build one head from K[start:end) (fp32 [capacity, d]). mu: centring mean or NULL.
 * fit: k-means with C_fit clusters from init_idx (offsets into the range) first. */
/* int8 copies of every slot: dir8 = q8(unit(sum_dir)), cent8 = q8(unit(cent)) (_refresh8,
 * src/ssa/kernels/sphere_fused.py:398-405). */
void canon_refresh8(canon_head_t* H) {
  const int C = H->C, d = H->d;
  for (int c = 0; c < C; ++c) {
    if (H->dir8) q8_unit(H->sum_dir + (int64_t)c * d, H->dir8 + (int64_t)c * d, d);
    if (H->cent8 && !H->shared_dirs) q8_unit(H->cent + (int64_t)c * d, H->cent8 + (int64_t)c * d, d);
  }
}

void canon_build(canon_head_t* H, const float* K, int start, int end, const float* mu, int fit, int C_fit, int iters,
                 const int32_t* init_idx) {
  const int d = H->d, C = H->C, nb = end - start;
  float* ks = H->ksum;
  /* ksum: per block of KB consecutive keys a left-to-right sum, then the block sums left to right */
  for (int i = 0; i < d; ++i) {
    float s = 0.f;
    for (int b0 = start; b0 < end; b0 += KB) {
      const int b1 = b0 + KB < end ? b0 + KB : end;
      float sb = 0.f;
      for (int p = b0; p < b1; ++p) sb = sb + K[(int64_t)p * d + i];
      s = s + sb;
    }
    ks[i] = s;
    H->mu_ref[i] = mu ? mu[i] : (nb > 0 ? s / (float)nb : 0.f);
  }
  memset(H->sum_dir, 0, sizeof(float) * (size_t)C * d);
  for (int c = 0; c < C; ++c) { H->mmax[c] = 0.f; H->mmin[c] = INFINITY; H->count[c] = 0; }
  *H->end = end;
  if (fit) *H->n_c = C_fit;
  if (nb > 0) {
    float* xn = (float*)malloc(sizeof(float) * (size_t)nb * d);
    float* mag = (float*)malloc(sizeof(float) * nb);
    float* kr = (float*)malloc(sizeof(float) * d);
    int* as = (int*)malloc(sizeof(int) * nb);
    float tsq = 0.f, tb = 0.f;     /* squared lengths: block sums of KB keys, added left to right */
    for (int j = 0; j < nb; ++j) {
      for (int i = 0; i < d; ++i) kr[i] = K[(int64_t)(start + j) * d + i] - H->mu_ref[i];
      const float sq = canon_dot(kr, kr, d);
      mag[j] = sqrtf(sq);
      const float magc = fmaxf(mag[j], 1e-12f);
      for (int i = 0; i < d; ++i) xn[(int64_t)j * d + i] = kr[i] / magc;
      tb = tb + sq;
      if ((j + 1) % KB == 0 || j + 1 == nb) { tsq = tsq + tb; tb = 0.f; }
    }
    *H->rbar = sqrtf(tsq / (float)nb);
    if (fit && !H->shared_dirs) {
      float* sums = (float*)malloc(sizeof(float) * (size_t)C_fit * d);
      int* cnt = (int*)malloc(sizeof(int) * C_fit);
      for (int c = 0; c < C_fit; ++c) memcpy(H->cent + (int64_t)c * d, xn + (int64_t)init_idx[c] * d, sizeof(float) * d);
      for (int it = 0; it < iters; ++it) {
        assign_all(xn, nb, d, H->cent, C_fit, as);
        blocked_sums(xn, nb, d, as, C_fit, sums, cnt);
        for (int c = 0; c < C_fit; ++c)
          if (cnt[c] > 0) unit(sums + (int64_t)c * d, H->cent + (int64_t)c * d, d);
      }
      free(sums); free(cnt);
    }
    assign_all(xn, nb, d, H->cent, *H->n_c, as);
    for (int j = 0; j < nb; ++j) H->labels[start + j] = (int16_t)as[j];
    blocked_sums(xn, nb, d, as, C, H->sum_dir, H->count);
    for (int j = 0; j < nb; ++j) {
      H->mmax[as[j]] = fmaxf(H->mmax[as[j]], mag[j]);
      H->mmin[as[j]] = fminf(H->mmin[as[j]], mag[j]);
    }
    free(xn); free(mag); free(kr); free(as);
  }
  canon_refresh8(H);
}
