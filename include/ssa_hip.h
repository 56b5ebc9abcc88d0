/* C ABI of libssa_hip.so: clustered sparse decode attention on AMD Instinct MI355X (gfx950).
 *
 * Every entry point takes device pointers, element strides, sizes and a hipStream_t passed as
 * void*, enqueues its kernels on that stream and returns a hipError_t value (0 = success). None
 * of them allocates device memory, synchronizes, or reads device memory on the host, so all of
 * them can be captured in a hipGraph. Lengths that change from step to step can be given in
 * device memory (n_dev, the index's end[]), which keeps a captured graph valid across steps.
 *
 * dtype tags: 0 = float32, 1 = bfloat16, 2 = float16.
 *
 * Layouts follow the reference's engine cache: K, V are [Hk, capacity, d] with a unit last
 * stride (Hk = batch x KV heads), q is [Hk*G, d], labels are int16 [Hk, capacity] with label C
 * marking the always-read exact set (token 0 and the recent window), w is fp32 [Hk or Hk*G, C+1].
 */
#ifndef SSA_HIP_H
#define SSA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Text of a hipError_t value returned by the entry points below. */
const char* ssa_error_string(int err);

/* ---- attention ----------------------------------------------------------------------------- */

typedef struct ssa_attn_args {
  const void* q; int64_t s_qh; int32_t q_dtype;
  const void* k; int64_t s_kh; int64_t s_kn;
  const void* v; int64_t s_vh; int64_t s_vn;
  int32_t kv_dtype;
  const int16_t* labels; int64_t s_lh;      /* labelled mode only */
  const float* w; int64_t s_wr; int32_t w_len; int32_t per_head;
  const int32_t* n_dev; int32_t n_host;      /* positions [0, n) are attended; n_dev wins if set */
  float* part_m; float* part_l;              /* [Hk, S, G] split partials (base-2 log domain) */
  float* part_a;                             /* [Hk, S, G, d], 16-byte aligned */
  int32_t* part_cnt;                         /* [Hk, S] rows read per split */
  int32_t* counter;                          /* [Hk] zero on first use; the kernel leaves it zero */
  void* out; int64_t s_oh; int32_t out_dtype;/* [Hk*G, d] */
  int32_t* cnt_out;                          /* optional [Hk]: rows read per KV head */
  int32_t n_heads; int32_t G; int32_t d; int32_t S;
  int32_t chunk_align;                       /* dense: split boundaries are multiples of it; label
                                                scans: split s reads blocks of 256 positions b = s mod S */
} ssa_attn_args_t;
/* q, k, v and part_a must be 16-byte aligned and every row stride (s_qh, s_kh, s_kn, s_vh, s_vn
 * times the element size, and d times the element size) a multiple of 16 bytes: rows are read
 * as 16-byte vectors. The attention entry points return hipErrorInvalidValue otherwise, before
 * anything is launched. */

/* Label-weighted split-K decode attention with the compaction fused in: positions whose label
 * has positive weight (for any query head of the group when per_head) are read, each with
 * weight w; the S partials of a head are merged by log-sum-exp in the same launch.
 * Replaces label_weighted_attention_compact (src/ssa/kernels/labeled_attn.py:248-278), i.e.
 * compact_positions + _list_kernel + merge_splits (:186, :203, :143), and the masked-scan
 * label_weighted_attention_triton (:88). Spec: label_weighted_attention (src/ssa/attn/labeled.py:24). */
int ssa_label_attention(const ssa_attn_args_t* args, void* stream);

/* Exact split-K decode attention over [0, n) (labels and w ignored).
 * Replaces DenseAttentionGraph.__call__ / _dense_dev_kernel (src/ssa/kernels/graph_kernels.py:28-59,171-189). */
int ssa_dense_attention(const ssa_attn_args_t* args, void* stream);

/* Log-sum-exp merge of natural-log split partials m, l [Hk, S, G] and a [Hk, S, G, d] into
 * out [Hk*G, d]. Replaces merge_splits / _merge_kernel (src/ssa/kernels/labeled_attn.py:124-151). */
int ssa_merge_splits(const float* m, const float* l, const float* a, int64_t s_mh, int64_t s_ms,
                     int64_t s_ah, int64_t s_as, int64_t s_ag, int n_heads, int S, int G, int d,
                     void* out, int64_t s_oh, int out_dtype, void* stream);

/* Ascending list of the selected positions {j < n : w[labels[j]] > 0} per KV head: idx
 * [Hk, >= n] (first cnt[h] valid), cnt [Hk]. block_counts is scratch of Hk*ceil(capacity/1024)
 * int32. Replaces compact_positions / _compact_kernel / _compact_dev_kernel
 * (src/ssa/kernels/labeled_attn.py:166-199; src/ssa/kernels/graph_kernels.py:145-155), with a
 * deterministic ascending order where the reference's atomics give an arbitrary one. */
int ssa_compact_positions(const int16_t* labels, int64_t s_lh, const float* w, int64_t s_wr,
                          int n_heads, int G, int per_head, const int32_t* n_dev, int n_host,
                          int capacity, int32_t* block_counts, int32_t* idx, int64_t s_ih,
                          int32_t* cnt, void* stream);

/* ---- cluster index ------------------------------------------------------------------------- */

/* Per-(sequence, KV head) cluster state, all device memory. With layers stacked, every array
 * holds n_heads = L * heads_per_layer rows. Reference state: SphereIndexGPU._alloc
 * (src/ssa/attn/sphere_gpu.py:145-164) and SphereIndexFused._alloc (src/ssa/kernels/sphere_fused.py:363-378). */
typedef struct ssa_index_state {
  int32_t n_heads, heads_per_layer, C, d, capacity, ms;
  int32_t summary_bits;     /* 8: scoring/insertion read the int8 copies; 32: the fp32 vectors */
  int32_t shared_dirs;      /* 1: cent is one [C, d] table shared by all heads (fixed random directions) */
  int32_t* n_c;             /* [n_heads] clusters in use */
  float* sum_dir;           /* [n_heads, C, d] sum of member unit directions */
  int8_t* dir8;             /* [n_heads, C, d] q8(unit(sum_dir)) */
  float* cent;              /* [n_heads, C, d] unit centroids ([C, d] if shared_dirs) */
  int8_t* cent8;            /* [n_heads, C, d] q8(unit(cent)) */
  float* mmax; float* mmin; /* [n_heads, C] longest / shortest centred key */
  int32_t* count;           /* [n_heads, C] keys per cluster */
  float* ksum; float* mu_ref;   /* [n_heads, d] running key sum, centring mean */
  float* rbar; float* cap; float* vthr;   /* [n_heads] */
  int32_t* flags;           /* [n_heads] bit0 drift, bit1 reset */
  int32_t* end;             /* [n_heads] binned positions are [1, end) */
  int32_t* nsplit;          /* [n_heads] splits done in kernels */
  int16_t* labels;          /* [n_heads, capacity] */
  int32_t* mem; float* proj; int32_t* side; float* smag;   /* [n_heads, ms] split scratch */
  int32_t* stage;           /* [n_heads, SSA_STAGE_WORDS] insertion staged by ssa_sparse_step's
                               insert-ahead workgroup, committed by the head's last workgroup */
  float* knbuf;             /* [n_heads, kn_rows, d] split scratch: the unit directions of the members of
                               a cluster being split, computed once per split (NULL: recomputed per pass) */
  int32_t kn_rows;          /* members knbuf holds per head; larger clusters recompute */
} ssa_index_state_t;

#define SSA_STAGE_WORDS 80  /* 8 header words + up to 256 int8 direction values */

typedef struct ssa_insert_args {
  const void* k; int32_t k_dtype; int64_t s_kh; int64_t s_kn;   /* cache of the first layer */
  const int64_t* koff;       /* [L] element offset of each layer's cache from k; NULL = one layer */
  const int32_t* n_dev; int32_t n_host;
  int32_t window; float delta; float capk; int32_t reset_at; int32_t var_min;
} ssa_insert_args_t;

typedef struct ssa_select_args {
  const void* q; int32_t q_dtype; int64_t s_qh; int32_t G;
  float* w; int64_t s_wr;    /* [Hk or Hk*G, C+1]; w[:, C] is set to 1 */
  double budget;             /* need = ceil(budget * (end - 1)) keys */
  int32_t group;             /* 0 sum_share, 1 per_head, 2 max, 3 max_rel */
  float scale;               /* 1/sqrt(d) */
  int32_t* need_out;         /* optional [Hk] */
} ssa_select_args_t;

/* Insert the keys that left the recent window since the last call into their nearest cluster
 * (lowest index on ties), split a cluster that passes its cap in the same kernel, update end,
 * and set the drift / reset flags; one workgroup per (layer, sequence, KV head).
 * Replaces _bin_kernel / _bin_dev_kernel / _split_cluster and AllLayerInsert
 * (src/ssa/kernels/sphere_fused.py:49-227; src/ssa/kernels/graph_kernels.py:63-130,286-325). */
int ssa_insert(const ssa_index_state_t* st, const ssa_insert_args_t* ins, void* stream);

/* Score every cluster from its summary for the G query heads of each KV head and choose clusters
 * in decreasing score, ties to the lowest index, until their keys reach the budget; writes w.
 * With ins non-NULL the insertion of ssa_insert runs first in the same kernel.
 * Replaces _score_kernel + _pick_kernel / _pick_dev_kernel (src/ssa/kernels/sphere_fused.py:231-313;
 * src/ssa/kernels/graph_kernels.py:134-141); oracle SphereIndexGPU.labels_and_weights
 * (src/ssa/attn/sphere_gpu.py:402-442). */
int ssa_select(const ssa_index_state_t* st, const ssa_insert_args_t* ins, const ssa_select_args_t* sel,
               void* stream);

/* One layer's decode step after insertion, in one launch: every workgroup of the attention grid
 * computes its head's selection exactly as ssa_select does (same bits, from the index state and
 * sel), then attends over the selected rows as ssa_label_attention does. args->labels must be
 * st->labels with args->s_lh = st->capacity (refused otherwise); sel->w, if non-NULL, receives
 * the selection (written by one workgroup per head).
 * With ins_ahead non-NULL (one layer's state, ins_ahead->k the attention's K, no koff), once
 * every workgroup of a head has read the state, the last one inserts the keys that leave the
 * window at length n + 1 (ins_ahead's n fields are ignored), splits included: the state is then
 * what ssa_insert would make of it at the start of the next step, so a decode loop that grows n
 * by one per step needs no insertion launch. The keys at positions < n + 1 - window must be in
 * the cache. The insertion is staged by one extra workgroup per head while Hk x (S + 1)
 * workgroups fit two per compute unit, otherwise by each head's split S - 1 after its attention
 * (no extra workgroups); either way the state and outputs are the same.
 * Replaces the per-layer bin + score + pick + compact + list + merge launches of
 * SphereIndexGraph.step (src/ssa/kernels/graph_kernels.py:220-244). */
int ssa_sparse_step(const ssa_index_state_t* st, const ssa_select_args_t* sel, const ssa_attn_args_t* args,
                    const ssa_insert_args_t* ins_ahead, void* stream);

/* Bytes of the split workspace held by the library for ssa_sparse_step_noalloc, per GPU. */
#define SSA_NOALLOC_SCRATCH_BYTES (4u << 20)

/* ssa_sparse_step without caller-supplied split buffers: no counterpart in the reference. It is
 * for callers that cannot allocate device memory (code under graph capture, serving loops,
 * harnesses that forbid hipMalloc). args->part_m, part_l, part_a, part_cnt and counter are
 * ignored (they may be NULL): the arrival counters and split partials live in a device array of
 * SSA_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, kept until the process ends. The
 * call allocates nothing; it enqueues a small kernel that clears the counters, then the step.
 * Layout, 256-byte aligned each: counters [Hk] int32, rows read [Hk, S] int32, m and l
 * [Hk, S, G] fp32, a [Hk, S, G, d] fp32; returns hipErrorInvalidValue before any launch when
 * they exceed SSA_NOALLOC_SCRATCH_BYTES (e.g. Hk = 8, S = 32, G = 2, d = 128 takes 0.27 MB).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, or
 * two graphs replayed concurrently) race, and must be serialised by the caller. The stream must
 * belong to the current device. Otherwise as ssa_sparse_step. */
int ssa_sparse_step_noalloc(const ssa_index_state_t* st, const ssa_select_args_t* sel, const ssa_attn_args_t* args,
                            const ssa_insert_args_t* ins_ahead, void* stream);

/* ---- prefill: fit, bin and summarise the prompt's keys ------------------------------------- */

typedef struct ssa_build_args {
  const void* k; int32_t k_dtype; int64_t s_kh; int64_t s_kn;   /* [Hk, capacity, d] */
  const int32_t* heads; int32_t n_sel;   /* heads to (re)build */
  int32_t start, end;                    /* binned range [start, end) */
  const float* mu;           /* [n_sel, d] centring mean, or NULL for the mean of the range */
  float* xn; float* mag;     /* scratch [n_sel, end-start, d] and [n_sel, end-start] */
  float* sq;                 /* scratch [n_sel, end-start] */
  int32_t* assign;           /* scratch [n_sel, end-start] */
  float* part;               /* scratch [n_sel, nblocks, max(C, C_fit), d], nblocks = ceil((end-start)/256) */
  int32_t* part_cnt;         /* scratch [n_sel, nblocks, max(C, C_fit)] */
  const int32_t* init_idx;   /* [C_fit] k-means seed members (offsets into the range) */
  int32_t fit;               /* 1: k-means fit of C_fit clusters first; 0: keep the centroids */
  int32_t C_fit; int32_t iters;
} ssa_build_args_t;

/* (Re)build heads: centre, optionally fit cosine k-means (assignment = argmax of the canonical
 * dot product, lowest index on ties; update = normalised blocked sums), label every key of the
 * range with its nearest centroid among the first n_c slots and rebuild the summaries and int8
 * copies. Replaces SphereIndexGPU._build / _bin / spherical_kmeans / _refresh8
 * (src/ssa/attn/sphere_gpu.py:166-219; src/ssa/attn/clusterkv.py:27-46;
 * src/ssa/kernels/sphere_fused.py:394-409). */
int ssa_build(const ssa_index_state_t* st, const ssa_build_args_t* b, void* stream);

/* ---- division of over-cap clusters after a fit -------------------------------------------- */

typedef struct ssa_split_args {
  const void* k; int32_t k_dtype; int64_t s_kh; int64_t s_kn;   /* [Hk, capacity, d] */
  const int32_t* heads; int32_t n_sel;   /* heads to divide */
  int32_t start, end;                    /* binned range [start, end) */
  float split_factor;
  float cap_min;             /* cap_now = max(cap[h], cap_min) */
  int32_t nmeans;            /* 1: k-means into max(2, ceil(count * split_factor / cap_now)) parts; 0: bisection */
  int32_t iters;             /* k-means updates */
  int32_t* mem; int32_t* side; float* proj; float* smag;   /* scratch [n_sel, ms] */
  int32_t ms;                /* members held per cluster (at least the largest cluster) */
  int32_t* over;             /* [n_sel] out: clusters over the cap at the start of the round */
  int32_t* done;             /* [n_sel] out: clusters divided in the round (-1: a division into more
                                than 32 parts found no room in parts, or asked for more than 1024) */
  int32_t refresh_only;      /* 1: only rebuild the int8 copies of the heads (after the last round) */
  float* parts;              /* scratch [n_sel, 2, max_parts, d] for k-means divisions into more than 32
                                parts (up to 32 are held on chip); NULL if none is expected */
  int32_t max_parts;         /* rows of parts per head, at most 1024 */
} ssa_split_args_t;

/* One round of the division of clusters over their cap after a k-means fit: the clusters with
 * count > cap_now, in slot order over the heads in order, each divided into parts (k-means from
 * members j*m/k, or the bisection of ssa_insert's split); non-empty parts are numbered in order,
 * part 0 keeps the slot and the others take spare slots handed out in order within batches of
 * 64 clusters. The caller repeats rounds (a k-means round, then bisection rounds) until no cluster
 * is over its cap or a bisection round divides nothing, then refreshes the int8 copies.
 * Replaces SphereIndexGPU._split_overflow / _split_batch / _kmeans_padded / _bisect_padded
 * (src/ssa/attn/sphere_gpu.py:56-102,307-391) and SphereIndexFused._split_overflow
 * (src/ssa/kernels/sphere_fused.py:411-413). */
int ssa_split_fit(const ssa_index_state_t* st, const ssa_split_args_t* a, void* stream);

/* ---- maintenance on the device: recentring, reset and refit ------------------------------- */

#define SSA_MAINT_PLAN_WORDS 8   /* header words of the plan, before its 3 * n_heads list words */

typedef struct ssa_maint_args {
  const void* k; int32_t k_dtype; int64_t s_kh; int64_t s_kn;   /* the layer's cache [Hk, capacity, d] */
  int32_t refit_all;         /* 1: refit every head (refit_every); 0: act on the flags */
  int32_t refit;             /* 1: refit the heads whose flag has bit 1 (with refit_all: every head);
                                0: bit 1 is cleared and ignored (no reset threshold) */
  int32_t C_init, iters, seed;   /* the fit's clusters, k-means updates, seed of its seed members */
  float split_factor;        /* > 0: the refit sets cap and divides clusters over it */
  float cap_keys;            /* > 0: the refit's cap, else split_factor * nb / C_init */
  double capk;               /* cap floor of the division: max(cap, capk * nb) */
  int32_t max_heads;         /* heads per build pass (rows of xn, mag, sq, assign, part, part_cnt) */
  int32_t* plan;             /* [SSA_MAINT_PLAN_WORDS + 3 * Hk], zero before the first call; plan[4] and
                                plan[5] count the heads recentred and reset (flag bit 1) so far */
  float* mu;                 /* [Hk, d] */
  float* xn; float* mag; float* sq; int32_t* assign;   /* [max_heads, capacity - 1 (, d)] */
  float* part; int32_t* part_cnt;   /* [max_heads, ceil((capacity - 1) / 256), C (, d)] */
  int32_t* init_idx;         /* [C_init] */
  int32_t* mem; int32_t* side; float* proj; float* smag;   /* [capacity]: the division, one head at a time */
  float* parts;              /* [2, 1024, d] */
  int32_t* over;             /* [Hk] */
} ssa_maint_args_t;

/* The recentring and refits the host check between graph replays performs, on the device and
 * with no host read: heads whose drift flag (bit 0) is set, and not bit 1, are rebuilt around
 * the mean of their binned keys with their centroids kept (labels, summaries, ksum, rbar, int8
 * copies); with refit, heads with bit 1 (or every head, with refit_all) are fitted again by
 * k-means from C_init clusters (seed members as torch.randperm on a CPU generator seeded with
 * seed), given a cap, and the clusters over it divided as after the prompt fit. Then all flags
 * are cleared. The state must be one layer's (n_heads == heads_per_layer), all heads with the
 * same binned length, capacity <= 65536. Every launch reads the flags and lengths from device
 * memory, so the call can be captured once and replayed every check_every steps.
 * Replaces SphereIndexFused._check_flags / _act_on / _rebuild (src/ssa/kernels/sphere_fused.py:
 * 434-464), SphereIndexGPU._reset_heads (src/ssa/attn/sphere_gpu.py:283-293) and
 * SphereIndexGraph.after_replay / _refit (src/ssa/kernels/graph_kernels.py:260-279), acting on
 * the flags as the reference's synchronous check (async_check=False) does. */
int ssa_maintain(const ssa_index_state_t* st, const ssa_maint_args_t* a, void* stream);

/* ---- glue of the captured whole-model decode step -----------------------------------------
 * These have no counterpart in the reference's path: its graph decoder runs the engine's own
 * torch modules between the attention calls (src/ssa/models/graph_decode.py:96-124). Here each
 * replaces a run of element-wise tensor ops of one Qwen3 layer, reproducing their rounding to
 * the storage dtype between ops. dtype: 0 fp32, 1 bf16, 2 fp16. */

/* h [rows, D] (updated in place), delta [rows, D] or NULL, w [D], x [rows, D]:
 * if delta, h = h + delta; then x = (h * rsqrt(mean(h^2) + eps)) * w (RMSNorm). */
int ssa_rmsnorm_add(void* h, const void* delta, const void* w, void* x, int32_t rows, int32_t D, float eps,
                    int32_t dtype, void* stream);

/* qkv [B, (H + 2 Hk) d] (query, key, value heads of each sequence). Query and key heads: RMSNorm
 * over d with q_w / k_w [d], then the half-split rotary embedding at position *pos (int64, device
 * memory) from cos / sin tables [max_pos, d/2] fp32; queries to q_out [B H, d], keys to
 * k_cache[b, h, *pos, :]; values copied to v_cache[b, h, *pos, :]. The caches are
 * [B, Hk, L, d] with element strides s_cb, s_ch, s_cl and unit last stride. d even, <= 256. */
int ssa_qk_norm_rope_cache(const void* qkv, const void* q_w, const void* k_w, const float* cos_t, const float* sin_t,
                           const int64_t* pos, void* q_out, void* k_cache, void* v_cache, int64_t s_cb, int64_t s_ch,
                           int64_t s_cl, int32_t B, int32_t H, int32_t Hk, int32_t d, float eps, int32_t dtype,
                           void* stream);

/* gu [rows, 2 I] (gate then up) -> out [rows, I] = round(silu(gate)) * up (SwiGLU). */
int ssa_silu_mul(const void* gu, void* out, int32_t rows, int32_t I, int32_t dtype, void* stream);

/* y [M, N] = x [M, K] W [N, K]^T for 1 <= M <= 8 (the decode batch), bf16 or fp16, fp32
 * accumulation rounded once: a weight-streaming kernel for the projections of a decode step,
 * where the library GEMM's tiles are mostly idle. K a multiple of 8; x and W 16-byte aligned. */
int ssa_linear_skinny(const void* x, const void* W, void* y, int32_t M, int32_t N, int32_t K, int32_t dtype,
                      void* stream);

/* out [M] int64 = the index of the first maximum of each row of x [M, N], a NaN counting as
 * above every number (greedy decoding). work: 12 M bytes of device memory, 8-byte aligned, zero
 * before the first call; every call leaves it zero. Calls that share a work buffer must not run
 * at the same time. */
int ssa_argmax_rows(const void* x, int64_t* out, int32_t M, int32_t N, int32_t dtype, void* work, void* stream);

/* act [M, I] = round(silu(g)) * u, (g, u) = x [M, K] W [2 I, K]^T rounded to the dtype (W holds
 * the gate rows, then the up rows): ssa_linear_skinny followed by ssa_silu_mul in one launch,
 * with the same bits. Same limits as ssa_linear_skinny. */
int ssa_linear_swiglu(const void* x, const void* W, void* act, int32_t M, int32_t I, int32_t K, int32_t dtype,
                      void* stream);

/* h [M, N] (the residual stream, updated in place) += x [M, K] W [N, K]^T: ssa_linear_skinny
 * followed by ssa_rmsnorm_add's add, in one launch with the same bits (the product rounded to
 * the dtype, then the sum). Same limits as ssa_linear_skinny; h need not be aligned. */
int ssa_linear_skinny_res(const void* x, const void* W, void* h, int32_t M, int32_t N, int32_t K, int32_t dtype,
                          void* stream);

/* y [M, N] = (RMSNorm(h) * norm_w) W [N, K]^T for rows h [M, K]: ssa_rmsnorm_add without delta
 * followed by ssa_linear_skinny, in one launch with the same bits (every workgroup reduces the
 * rows' squares itself, in ssa_rmsnorm_add's order). Same limits as ssa_linear_skinny; h and
 * norm_w 16-byte aligned. */
int ssa_rmsnorm_linear_skinny(const void* h, const void* norm_w, float eps, const void* W, void* y, int32_t M,
                              int32_t N, int32_t K, int32_t dtype, void* stream);

/* act [M, I] as ssa_linear_swiglu of x = RMSNorm(h) * norm_w for rows h [M, K]: ssa_rmsnorm_add
 * without delta followed by ssa_linear_swiglu, in one launch with the same bits. */
int ssa_rmsnorm_linear_swiglu(const void* h, const void* norm_w, float eps, const void* W, void* act, int32_t M,
                              int32_t I, int32_t K, int32_t dtype, void* stream);

/* h [rows, D] = embed [vocab, D] row tok[r] (int64, clamped to the table), then x = RMSNorm(h) * w
 * as ssa_rmsnorm_add without delta; if n_out, *n_out = *pos + 1 (int32, the step's cache length):
 * the first launch of a decode step. */
int ssa_embed_rmsnorm(const int64_t* tok, const void* embed, void* h, const void* w, void* x, int32_t rows, int32_t D,
                      int64_t vocab, float eps, const int64_t* pos, int32_t* n_out, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SSA_HIP_H */
