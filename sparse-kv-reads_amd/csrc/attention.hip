// C ABI of the attention entry points, and the standalone merge and compaction kernels of the
// reference's functional API. The decode kernel itself is in decode.h, instantiated once per KV
// dtype by decode_bf16.hip, decode_f16.hip and decode_f32.hip.
#include <atomic>
#include <mutex>

#include "decode.h"

namespace ssa {

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

// Clears n int32 values (the arrival counters of the no-alloc step): a kernel rather than a
// memset, so that a captured graph holds no memset node.
__global__ __launch_bounds__(256) void zero_i32_kernel(int32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += 256) p[i] = 0;
}

// Split workspace of ssa_sparse_step_noalloc: the arrival counters and split partials of one
// launch, in this file-scope device array instead of caller-supplied buffers. Each GPU the
// library runs on holds its own copy until the process ends. Host code never passes the array's
// name to a kernel (on the host it is a stand-in, not a device address): its device address is
// looked up once per device with hipGetSymbolAddress and kept in noalloc_base below.
static __device__ __align__(256) unsigned char scratch[SSA_NOALLOC_SCRATCH_BYTES];

}  // namespace ssa

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
using namespace ssa;

namespace {

int elem_size(int dt) { return dt == kF32 ? 4 : (dt == kBF16 || dt == kF16) ? 2 : 0; }

// The kernel reads q, K and V rows and the split accumulators as 16-byte vectors (and the
// accumulators with 8-byte atomic loads): every row it touches must start on a 16-byte boundary.
bool rows_aligned(const ssa_attn_args_t* x) {
  const int qe = elem_size(x->q_dtype), ke = elem_size(x->kv_dtype);
  if (!qe || !ke) return false;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  auto s16 = [](int64_t s, int e) { return (s * e) % 16 == 0; };
  return a16(x->q) && a16(x->k) && a16(x->v) && a16(x->part_a) && s16(x->s_qh, qe) && s16(x->s_kh, ke) &&
         s16(x->s_kn, ke) && s16(x->s_vh, ke) && s16(x->s_vn, ke) && (x->d * ke) % 16 == 0;
}

// Compute units of the current device (0 if unknown), looked up once per device.
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (c == 0 && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
    cus[dev].store(c, std::memory_order_relaxed);
  return c > 0 ? c : 0;
}

// zero_first: arrival counters to clear (a fill kernel on the same stream) once the arguments
// have been checked and before the decode kernel is launched; nullptr for none.
int launch_decode(const ssa_attn_args_t* x, int mode, void* stream, const ssa_index_state_t* st = nullptr,
                  const ssa_select_args_t* sel = nullptr, const ssa_insert_args_t* ins = nullptr,
                  int32_t* zero_first = nullptr) {
  if (!x || x->G < 1 || x->G > 8 || x->S < 1 || x->S > kMaxS || x->n_heads < 1) return hipErrorInvalidValue;
  if (!x->q || !x->k || !x->v || !x->out || !x->part_m || !x->part_l || !x->part_a || !x->part_cnt || !x->counter)
    return hipErrorInvalidValue;
  if (!rows_aligned(x)) return hipErrorInvalidValue;
  if (mode == kLabelled && (x->w_len < 1 || x->w_len > kMaxW)) return hipErrorInvalidValue;
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
  if (mode == kFused) {
    if (!st || !sel || st->C < 16 || st->C > kMaxC || (st->C & (st->C - 1)) || st->d != x->d || sel->G != x->G ||
        st->n_heads != x->n_heads || sel->group < 0 || sel->group > 3)
      return hipErrorInvalidValue;
    // the selection is computed from the state, so the labels scanned must be the state's own rows
    if (x->labels != st->labels || x->s_lh != st->capacity || st->capacity < 1) return hipErrorInvalidValue;
    p.st = *st;
    p.budget = sel->budget;
    p.group = sel->group;
    p.sel_scale = sel->scale;
    p.w = sel->w;
    p.s_wr = sel->s_wr;
    p.per_head = sel->group == 1;
    p.w_len = st->C + 1;
    if (ins) {
      if (st->heads_per_layer != st->n_heads || ins->koff || ins->k != x->k || ins->k_dtype != x->kv_dtype)
        return hipErrorInvalidValue;
      p.ins = *ins;
      mode = kFusedAhead;
      // An extra stager workgroup per head while heads x (S + 1) workgroups are all resident
      // (two per compute unit); past that, split S - 1 stages after its attention, which costs
      // less than a second round of workgroups. Both leave the same state.
      const int cus = device_cus();
      p.fold_stage = cus > 0 && (int64_t)x->n_heads * (x->S + 1) > 2 * (int64_t)cus;
    }
  }
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  if (zero_first) {
    hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(256), 0, hs, zero_first, x->n_heads);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  switch (x->kv_dtype) {
    case kBF16: return launch_decode_bf16(p, x->d, mode, hs);
    case kF16: return launch_decode_f16(p, x->d, mode, hs);
    case kF32: return launch_decode_f32(p, x->d, mode, hs);
  }
  return hipErrorInvalidValue;
}

// Byte offsets of the split workspace's arrays in the scratch array, each on a 256-byte boundary.
struct NoAllocLayout {
  size_t counter, part_cnt, part_m, part_l, part_a, total;
};

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

NoAllocLayout noalloc_layout(int n_heads, int S, int G, int d) {
  const size_t hs = (size_t)n_heads * (size_t)S, hsg = hs * (size_t)G;
  NoAllocLayout L;
  L.counter = 0;
  L.part_cnt = round256(sizeof(int32_t) * (size_t)n_heads);
  L.part_m = L.part_cnt + round256(sizeof(int32_t) * hs);
  L.part_l = L.part_m + round256(sizeof(float) * hsg);
  L.part_a = L.part_l + round256(sizeof(float) * hsg);
  L.total = L.part_a + round256(sizeof(float) * hsg * (size_t)d);
  return L;
}

// Device address of this device's scratch array, looked up on the first call made with the
// device current and kept per device.
constexpr int kMaxDevices = 64;
std::mutex noalloc_mu;
void* noalloc_base[kMaxDevices];

hipError_t noalloc_scratch(hipStream_t stream, unsigned char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return e;
    if (sdev != dev) return hipErrorInvalidValue;     // the stream must belong to the current device
  }
  std::lock_guard<std::mutex> lock(noalloc_mu);
  if (!noalloc_base[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    noalloc_base[dev] = p;
  }
  *out = static_cast<unsigned char*>(noalloc_base[dev]);
  return hipSuccess;
}

}  // namespace

extern "C" int ssa_label_attention(const ssa_attn_args_t* args, void* stream) {
  return launch_decode(args, kLabelled, stream);
}

extern "C" int ssa_dense_attention(const ssa_attn_args_t* args, void* stream) {
  return launch_decode(args, kDense, stream);
}

extern "C" int ssa_sparse_step(const ssa_index_state_t* st, const ssa_select_args_t* sel, const ssa_attn_args_t* args,
                               const ssa_insert_args_t* ins_ahead, void* stream) {
  return launch_decode(args, kFused, stream, st, sel, ins_ahead);
}

extern "C" int ssa_sparse_step_noalloc(const ssa_index_state_t* st, const ssa_select_args_t* sel,
                                       const ssa_attn_args_t* args, const ssa_insert_args_t* ins_ahead,
                                       void* stream) {
  if (!args || args->n_heads < 1 || args->S < 1 || args->S > kMaxS || args->G < 1 || args->G > 8 || args->d < 1)
    return hipErrorInvalidValue;
  const NoAllocLayout L = noalloc_layout(args->n_heads, args->S, args->G, args->d);
  if (L.total > (size_t)SSA_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;   // beyond the scratch array
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  unsigned char* base = nullptr;
  const hipError_t e = noalloc_scratch(hs, &base);
  if (e != hipSuccess) return e;
  ssa_attn_args_t x = *args;
  x.counter = reinterpret_cast<int32_t*>(base + L.counter);
  x.part_cnt = reinterpret_cast<int32_t*>(base + L.part_cnt);
  x.part_m = reinterpret_cast<float*>(base + L.part_m);
  x.part_l = reinterpret_cast<float*>(base + L.part_l);
  x.part_a = reinterpret_cast<float*>(base + L.part_a);
  // the counters are cleared by every call: the array keeps whatever the last call left in it
  return launch_decode(&x, kFused, stream, st, sel, ins_ahead, x.counter);
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
