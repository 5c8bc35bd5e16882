// Producers around the attention call for gfx950:
//   * the fog vectors -- the logit bias of the serving path
//     (_FogCache._compute_into, kessie_attention.py:114-139) and the V weights
//     (kessie_build_fog_weights, kessie_hip_kernels.py:403-413) -- computed in
//     one pass on the device instead of a chain of torch ops plus one
//     host-driven scalar write per recalled position;
//   * the slot-mapped write of new K/V rows into the paged cache (the step the
//     serving backend takes before attention: token t goes to page
//     slot[t] / P, offset slot[t] % P).
//
// The fog arithmetic follows the reference's op sequence as torch runs it on
// the device, rounding to the buffer dtype after every op:
//   pos = dtype(i)                      arange in the buffer dtype
//   x   = dtype(f32(pos) * (1/B))       tensor / python scalar: torch's device
//                                       kernel multiplies by the fp32 reciprocal
//   d   = dtype(1 - f32(x))
//   d2  = dtype(f32(d) * f32(d))        decay.mul_(decay)
//   b   = dtype(f32(d2) * f32(-alpha))  decay.mul_(-fog_alpha)
// and recalled positions are overwritten with dtype(recall_boost).
#include "common.h"

namespace kessie {
namespace cache {
namespace {

constexpr int kThreads = 256;

template <typename T>
__device__ __forceinline__ T round_to(float x) {
  return from_f32<T>(x);
}
template <>
__device__ __forceinline__ float round_to<float>(float x) {
  return x;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void fog_bias_kernel(T* buf, int kv_len, int boundary, float inv_b,
                                                            float neg_alpha, const int32_t* recall, int n_recall,
                                                            float boost) {
#pragma clang fp contract(off)
  // Recalled positions take the boost: the workgroup marks those inside its
  // own kThreads positions (a scan of the recall list into LDS flags), so
  // every position is written once, by one launch.
  __shared__ int marked[kThreads];
  const int lo = blockIdx.x * kThreads;
  const int i = lo + threadIdx.x;
  marked[threadIdx.x] = 0;
  if (n_recall > 0) {  // uniform
    __syncthreads();
    const int hi = min(lo + kThreads, kv_len);
    for (int r = threadIdx.x; r < n_recall; r += kThreads) {
      const int p = recall[r];
      if (p >= lo && p < hi) marked[p - lo] = 1;
    }
    __syncthreads();
  }
  if (i >= kv_len) return;
  T v = round_to<T>(0.0f);
  if (marked[threadIdx.x]) {
    v = round_to<T>(boost);
  } else if (i < boundary) {
    const T pos = round_to<T>((float)i);
    const T x = round_to<T>(to_f32(pos) * inv_b);
    const T d = round_to<T>(1.0f - to_f32(x));
    const T d2 = round_to<T>(to_f32(d) * to_f32(d));
    v = round_to<T>(to_f32(d2) * neg_alpha);
  }
  buf[i] = v;
}

// One row per sequence: row b is the vector above for kv_len = seq_lens[b]
// (its own fog boundary B_b = int(len * (1 - fog_start)), computed in double
// as in Python), every value rounded as in `T` and stored as fp32 -- the form
// the attention kernels read; positions at or past the row's length are 0.
template <typename T>
__global__ __launch_bounds__(kThreads) void fog_bias_rows_kernel(float* out, int64_t row_stride,
                                                                 const int32_t* seq_lens, int max_len,
                                                                 double one_minus_fs, float neg_alpha,
                                                                 const int32_t* recall, int n_recall, float boost) {
#pragma clang fp contract(off)
  __shared__ int marked[kThreads];  // recalled positions of this workgroup's range, as in fog_bias_kernel
  const int b = blockIdx.y;
  const int lo = blockIdx.x * kThreads;
  const int i = lo + threadIdx.x;
  const int len = min(max(seq_lens[b], 0), max_len);
  marked[threadIdx.x] = 0;
  if (n_recall > 0) {  // uniform
    __syncthreads();
    const int hi = min(lo + kThreads, len);
    for (int r = threadIdx.x; r < n_recall; r += kThreads) {
      const int p = recall[r];
      if (p >= lo && p < hi) marked[p - lo] = 1;
    }
    __syncthreads();
  }
  if (i >= max_len) return;
  const double bd = (double)len * one_minus_fs;
  const int64_t big_b = bd <= 0.0 ? 0 : (int64_t)bd;
  const int boundary = (int)(big_b < len ? big_b : len);
  float v = 0.0f;
  if (marked[threadIdx.x]) {
    v = to_f32(round_to<T>(boost));
  } else if (i < boundary) {
    const float inv_b = __frcp_rn((float)big_b);  // fp32 1/B, rounded to nearest as on the host
    const T pos = round_to<T>((float)i);
    const T x = round_to<T>(to_f32(pos) * inv_b);
    const T d = round_to<T>(1.0f - to_f32(x));
    const T d2 = round_to<T>(to_f32(d) * to_f32(d));
    v = to_f32(round_to<T>(to_f32(d2) * neg_alpha));
  }
  out[(int64_t)b * row_stride + i] = v;
}

template <typename T>
int fog_bias_rows_launch(float* out, int64_t row_stride, const int32_t* seq_lens, int rows, int max_len,
                         double one_minus_fs, float neg_alpha, const int32_t* recall, int n_recall, float boost,
                         hipStream_t s) {
  hipLaunchKernelGGL(fog_bias_rows_kernel<T>, dim3(div_up(max_len, kThreads), rows), dim3(kThreads), 0, s, out,
                     row_stride, seq_lens, max_len, one_minus_fs, neg_alpha, recall, n_recall > 0 ? n_recall : 0,
                     boost);
  return check_launch("fog bias rows");
}

// Exponent forms torch's device pow(tensor, scalar) special-cases, so the
// weights take the same arithmetic route (alpha > 0 only reaches here).
enum PowForm { kPowGeneral = 0, kPowOne = 1, kPowHalf = 2, kPowTwo = 3, kPowThree = 4 };

__global__ __launch_bounds__(kThreads) void fog_weights_kernel(float* w, int n, int clear_start, float inv_den,
                                                               float alpha, int form) {
#pragma clang fp contract(off)
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  float v = 1.0f;
  if (i < clear_start) {
    const float t = (float)i * inv_den;
    switch (form) {
      case kPowOne: v = t; break;
      case kPowHalf: v = sqrtf(t); break;
      case kPowTwo: v = t * t; break;
      case kPowThree: v = t * t * t; break;
      default: v = powf(t, alpha); break;
    }
  }
  w[i] = v;
}

template <typename T>
int fog_bias_launch(void* buf, int kv_len, int boundary, float inv_b, float neg_alpha, const int32_t* recall,
                    int n_recall, float boost, hipStream_t s) {
  T* b = static_cast<T*>(buf);
  hipLaunchKernelGGL(fog_bias_kernel<T>, dim3(div_up(kv_len, kThreads)), dim3(kThreads), 0, s, b, kv_len, boundary,
                     inv_b, neg_alpha, recall, n_recall > 0 ? n_recall : 0, boost);
  return check_launch("fog bias");
}

// ---- fog of the HF tiered cache (KeSSieCache, kessie_exp3.py:415-445) ------
// cc = max(1, int(N * fog_start)) clear tokens at the end, fc = N - cc fogged
// ones: w[p] = max(fp32(p) * fp32(1/max(fc-1,1)) ^ alpha, 0.01) for p < fc, 1
// otherwise (torch's device arange / division by a Python scalar / pow /
// clamp, in fp32), and V' = dtype(fp32(V) * w).

__device__ __forceinline__ float hf_fog_weight(int p, int fc, float inv_den, float alpha, int form) {
#pragma clang fp contract(off)
  if (p >= fc) return 1.0f;
  const float t = (float)p * inv_den;
  float w;
  switch (form) {
    case kPowOne: w = t; break;
    case kPowHalf: w = sqrtf(t); break;
    case kPowTwo: w = t * t; break;
    case kPowThree: w = t * t * t; break;
    default: w = powf(t, alpha); break;
  }
  return fmaxf(w, 0.01f);
}

__global__ __launch_bounds__(kThreads) void hf_fog_weights_kernel(float* w, int n, int fc, float inv_den, float alpha,
                                                                  int form) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < n) w[i] = hf_fog_weight(i, fc, inv_den, alpha, form);
}

// V' rows (b, h, t) = V rows * w[t]; one thread per 16-byte chunk.
template <typename T>
__global__ __launch_bounds__(kThreads) void hf_fog_apply_kernel(const T* __restrict__ v, T* __restrict__ out, int BH,
                                                                int H, int n, int D, int64_t v_bs, int64_t v_hs,
                                                                int64_t v_ts, int64_t o_bs, int64_t o_hs, int64_t o_ts,
                                                                int fc, float inv_den, float alpha, int form) {
#pragma clang fp contract(off)
  constexpr int N = 16 / (int)sizeof(T);
  const int chunks = D / N;
  const int64_t total = (int64_t)BH * n * chunks;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const int c = (int)(i % chunks);
  const int64_t r = i / chunks;
  const int t = (int)(r % n);
  const int bh = (int)(r / n);
  const int b = bh / H, h = bh - b * H;
  const float w = hf_fog_weight(t, fc, inv_den, alpha, form);
  typedef T V8 __attribute__((ext_vector_type(16 / sizeof(T))));
  const V8 x = *reinterpret_cast<const V8*>(v + b * v_bs + h * v_hs + t * v_ts + c * N);
  V8 y;
#pragma unroll
  for (int e = 0; e < N; ++e) y[e] = round_to<T>(to_f32(x[e]) * w);
  *reinterpret_cast<V8*>(out + b * o_bs + h * o_hs + t * o_ts + c * N) = y;
}

// Append + fog of one KeSSieCache layer in one pass: window tokens [0, n_old)
// come from the V arena; tokens [n_old, n_old + t_new) come from new_v, and
// those threads also write new_k / new_v into the arenas at window positions
// n_old.. .  V' (when vfog is set) = dtype(fp32(V) * w[t]) over all
// n_old + t_new tokens; without vfog only the new tokens are written.
template <typename T>
struct AppendFogArgs {
  T* k_arena;  // window start of the K arena
  T* v_arena;  // window start of the V arena (same strides)
  int64_t a_bs, a_hs, a_ts;
  const T* new_k;
  int64_t k_bs, k_hs, k_ts;
  const T* new_v;
  int64_t v_bs, v_hs, v_ts;
  T* vfog;
  int64_t o_bs, o_hs, o_ts;
  int H, n_old, t_new, D;
  int fc;
  float inv_den, alpha;
  int form;
};

// kAppendChunks 16-byte chunks per thread, a grid-stride apart (every load
// coalesced), all loaded before any V' store: 8K-token window, bf16, 8 heads:
// 7.22-7.25 us against 7.45-7.53 with one chunk per thread, 7.76 with four.
constexpr int kAppendChunks = 2;

template <typename T>
__global__ __launch_bounds__(kThreads) void hf_append_fog_kernel(AppendFogArgs<T> a) {
#pragma clang fp contract(off)
  constexpr int N = 16 / (int)sizeof(T);
  typedef T V8 __attribute__((ext_vector_type(16 / sizeof(T))));
  const int chunks = a.D / N;
  const int first = a.vfog ? 0 : a.n_old;
  const int n = a.n_old + a.t_new - first;
  const int64_t total = (int64_t)n * chunks;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t i0 = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int bh = blockIdx.y;  // one (batch, head) row
  const int b = bh / a.H, h = bh - b * a.H;
  V8 x[kAppendChunks];
  int tt[kAppendChunks], cc[kAppendChunks];
#pragma unroll
  for (int j = 0; j < kAppendChunks; ++j) {
    const int64_t i = i0 + j * stride;
    tt[j] = -1;
    if (i >= total) continue;
    const int c = (int)(i % chunks);
    const int t = first + (int)(i / chunks);
    tt[j] = t;
    cc[j] = c;
    const int64_t ao = b * a.a_bs + h * a.a_hs + (int64_t)t * a.a_ts + c * N;
    if (t >= a.n_old) {
      const int tn = t - a.n_old;
      x[j] = *reinterpret_cast<const V8*>(a.new_v + b * a.v_bs + h * a.v_hs + (int64_t)tn * a.v_ts + c * N);
      const V8 kx = *reinterpret_cast<const V8*>(a.new_k + b * a.k_bs + h * a.k_hs + (int64_t)tn * a.k_ts + c * N);
      *reinterpret_cast<V8*>(a.k_arena + ao) = kx;
      *reinterpret_cast<V8*>(a.v_arena + ao) = x[j];
    } else {
      x[j] = *reinterpret_cast<const V8*>(a.v_arena + ao);
    }
  }
  if (!a.vfog) return;
#pragma unroll
  for (int j = 0; j < kAppendChunks; ++j) {
    if (tt[j] < 0) continue;
    const float w = hf_fog_weight(tt[j], a.fc, a.inv_den, a.alpha, a.form);
    V8 y;
#pragma unroll
    for (int e = 0; e < N; ++e) y[e] = round_to<T>(to_f32(x[j][e]) * w);
    *reinterpret_cast<V8*>(a.vfog + b * a.o_bs + h * a.o_hs + (int64_t)tt[j] * a.o_ts + cc[j] * N) = y;
  }
}

struct HfFog {
  int fc;
  float inv_den;
  float alpha;
  int form;
};

HfFog hf_fog_params(int n, double fog_alpha, double fog_start) {
  // cc = max(1, int(N * fog_start)) (C's cast truncates toward zero like int());
  // fc <= 0 or fog_alpha <= 0 leaves V unweighted, as the reference does.
  const double prod = (double)n * fog_start;
  const int cc = prod >= (double)n ? n : (prod < 1.0 ? 1 : (int)prod);
  HfFog f{n - cc, 0.0f, (float)fog_alpha, kPowGeneral};
  if (f.fc < 0 || !(fog_alpha > 0.0)) f.fc = 0;
  f.inv_den = 1.0f / (float)(f.fc - 1 > 1 ? f.fc - 1 : 1);
  if (fog_alpha == 1.0) f.form = kPowOne;
  else if (fog_alpha == 0.5) f.form = kPowHalf;
  else if (fog_alpha == 2.0) f.form = kPowTwo;
  else if (fog_alpha == 3.0) f.form = kPowThree;
  return f;
}

// ---- slot-mapped K/V write -------------------------------------------------

struct WriteArgs {
  void* pool;
  int64_t page_stride, tok_stride, kv_stride, head_stride;
  const void* key;
  const void* value;
  int64_t k_ts, k_hs, v_ts, v_hs;  // source token / head strides (elements)
  const int64_t* slots;
  int T, H, D, page_size, num_pages;
};

// One thread per 16-byte chunk of one (token, head) row of K and of V.
template <typename T>
__global__ __launch_bounds__(kThreads) void kv_write_vec_kernel(WriteArgs a) {
  constexpr int N = 16 / (int)sizeof(T);
  const int chunks = a.D / N;
  const int64_t total = (int64_t)a.T * a.H * chunks;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const int c = (int)(i % chunks);
  const int64_t th = i / chunks;
  const int h = (int)(th % a.H);
  const int t = (int)(th / a.H);
  const int64_t slot = a.slots[t];
  if (slot < 0) return;
  const int64_t page = slot / a.page_size;
  if (page >= a.num_pages) return;
  T* pool = static_cast<T*>(a.pool);
  const int64_t dst = page * a.page_stride + (slot % a.page_size) * a.tok_stride + h * a.head_stride + c * N;
  const u32x4 kx = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.key) + t * a.k_ts + h * a.k_hs + c * N);
  const u32x4 vx = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.value) + t * a.v_ts + h * a.v_hs + c * N);
  *reinterpret_cast<u32x4*>(pool + dst) = kx;
  *reinterpret_cast<u32x4*>(pool + dst + a.kv_stride) = vx;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void kv_write_scalar_kernel(WriteArgs a) {
  const int64_t total = (int64_t)a.T * a.H * a.D;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const int d = (int)(i % a.D);
  const int64_t th = i / a.D;
  const int h = (int)(th % a.H);
  const int t = (int)(th / a.H);
  const int64_t slot = a.slots[t];
  if (slot < 0) return;
  const int64_t page = slot / a.page_size;
  if (page >= a.num_pages) return;
  T* pool = static_cast<T*>(a.pool);
  const int64_t dst = page * a.page_stride + (slot % a.page_size) * a.tok_stride + h * a.head_stride + d;
  pool[dst] = static_cast<const T*>(a.key)[t * a.k_ts + h * a.k_hs + d];
  pool[dst + a.kv_stride] = static_cast<const T*>(a.value)[t * a.v_ts + h * a.v_hs + d];
}

template <typename T>
int kv_write_launch(const WriteArgs& a, hipStream_t s) {
  constexpr int N = 16 / (int)sizeof(T);
  const bool vec = a.D % N == 0 && aligned16(a.pool) && aligned16(a.key) && aligned16(a.value) &&
                   a.page_stride % N == 0 && a.tok_stride % N == 0 && a.kv_stride % N == 0 && a.head_stride % N == 0 &&
                   a.k_ts % N == 0 && a.k_hs % N == 0 && a.v_ts % N == 0 && a.v_hs % N == 0;
  const int64_t items = (int64_t)a.T * a.H * (vec ? a.D / N : a.D);
  const int64_t grid = (items + kThreads - 1) / kThreads;
  KESSIE_REQUIRE(grid <= 0x7fffffff, KESSIE_ERR_UNSUPPORTED, "kv cache write: %lld items exceed one launch",
                 (long long)items);
  if (vec)
    hipLaunchKernelGGL(kv_write_vec_kernel<T>, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(kv_write_scalar_kernel<T>, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
  return check_launch("kv cache write");
}

}  // namespace
}  // namespace cache
}  // namespace kessie

using namespace kessie;
using namespace kessie::cache;

extern "C" int kessie_fog_bias_fill(void* buf, int dtype, int kv_len, double fog_alpha, double fog_start,
                                    const int32_t* recall_positions, int num_recall, double recall_boost,
                                    void* stream) {
  clear_error();
  KESSIE_REQUIRE(kv_len >= 0 && num_recall >= 0, KESSIE_ERR_INVALID, "fog bias: kv_len %d, num_recall %d", kv_len,
                 num_recall);
  if (kv_len == 0) return KESSIE_OK;
  KESSIE_REQUIRE(buf != nullptr, KESSIE_ERR_INVALID, "fog bias: null buffer");
  KESSIE_REQUIRE(num_recall == 0 || recall_positions != nullptr, KESSIE_ERR_INVALID, "fog bias: null recall list");
  // B = int(kv_len * (1.0 - fog_start)) in double, as the reference's Python
  // does; the decay divides by B itself and covers positions < min(B, kv_len).
  const double bd = (double)kv_len * (1.0 - fog_start);
  KESSIE_REQUIRE(bd < 2147483648.0, KESSIE_ERR_INVALID, "fog bias: fog boundary %.0f out of range", bd);
  const int64_t big_b = bd <= 0.0 ? 0 : (int64_t)bd;
  const int boundary = (int)(big_b < kv_len ? big_b : kv_len);
  const float inv_b = big_b > 0 ? 1.0f / (float)big_b : 0.0f;
  const float neg_alpha = (float)(-fog_alpha);
  const float boost = (float)recall_boost;
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case KESSIE_DTYPE_F32:
      return fog_bias_launch<float>(buf, kv_len, boundary, inv_b, neg_alpha, recall_positions, num_recall, boost, s);
    case KESSIE_DTYPE_BF16:
      return fog_bias_launch<bf16_t>(buf, kv_len, boundary, inv_b, neg_alpha, recall_positions, num_recall, boost, s);
    case KESSIE_DTYPE_F16:
      return fog_bias_launch<f16_t>(buf, kv_len, boundary, inv_b, neg_alpha, recall_positions, num_recall, boost, s);
  }
  set_error(KESSIE_ERR_UNSUPPORTED, "fog bias: dtype %d", dtype);
  return KESSIE_ERR_UNSUPPORTED;
}

extern "C" int kessie_fog_bias_fill_rows(float* out, int64_t row_stride, const int32_t* seq_lens, int num_rows,
                                         int max_len, int dtype, double fog_alpha, double fog_start,
                                         const int32_t* recall_positions, int num_recall, double recall_boost,
                                         void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_rows >= 0 && max_len >= 0 && num_recall >= 0 && row_stride >= max_len, KESSIE_ERR_INVALID,
                 "fog bias rows: rows %d, max_len %d, row_stride %lld, num_recall %d", num_rows, max_len,
                 (long long)row_stride, num_recall);
  if (num_rows == 0 || max_len == 0) return KESSIE_OK;
  KESSIE_REQUIRE(num_rows <= 65535, KESSIE_ERR_UNSUPPORTED, "fog bias rows: %d rows (at most 65,535)", num_rows);
  KESSIE_REQUIRE(out != nullptr && seq_lens != nullptr, KESSIE_ERR_INVALID, "fog bias rows: null pointer");
  KESSIE_REQUIRE(num_recall == 0 || recall_positions != nullptr, KESSIE_ERR_INVALID,
                 "fog bias rows: null recall list");
  KESSIE_REQUIRE((double)max_len * (1.0 - fog_start) < 2147483648.0, KESSIE_ERR_INVALID,
                 "fog bias rows: fog boundary out of range");
  const double omf = 1.0 - fog_start;
  const float neg_alpha = (float)(-fog_alpha);
  const float boost = (float)recall_boost;
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case KESSIE_DTYPE_F32:
      return fog_bias_rows_launch<float>(out, row_stride, seq_lens, num_rows, max_len, omf, neg_alpha,
                                         recall_positions, num_recall, boost, s);
    case KESSIE_DTYPE_BF16:
      return fog_bias_rows_launch<bf16_t>(out, row_stride, seq_lens, num_rows, max_len, omf, neg_alpha,
                                          recall_positions, num_recall, boost, s);
    case KESSIE_DTYPE_F16:
      return fog_bias_rows_launch<f16_t>(out, row_stride, seq_lens, num_rows, max_len, omf, neg_alpha,
                                         recall_positions, num_recall, boost, s);
  }
  set_error(KESSIE_ERR_UNSUPPORTED, "fog bias rows: dtype %d", dtype);
  return KESSIE_ERR_UNSUPPORTED;
}

extern "C" int kessie_fog_weights_fill(float* weights, int seq_len, double fog_alpha, double fog_start, void* stream) {
  clear_error();
  KESSIE_REQUIRE(seq_len >= 0, KESSIE_ERR_INVALID, "fog weights: seq_len %d", seq_len);
  if (seq_len == 0) return KESSIE_OK;
  KESSIE_REQUIRE(weights != nullptr, KESSIE_ERR_INVALID, "fog weights: null buffer");
  // c = int(N * (1.0 - fog_start)); c > N (fog_start < 0) is a shape error in
  // the reference and is clamped to N here.
  const double cd = (double)seq_len * (1.0 - fog_start);
  int clear_start = cd <= 0.0 ? 0 : (cd >= (double)seq_len ? seq_len : (int)cd);
  if (!(fog_alpha > 0.0)) clear_start = 0;  // weights stay 1
  const float inv_den = 1.0f / (float)(clear_start - 1 > 1 ? clear_start - 1 : 1);
  const float a = (float)fog_alpha;
  int form = kPowGeneral;
  if (fog_alpha == 1.0) form = kPowOne;
  else if (fog_alpha == 0.5) form = kPowHalf;
  else if (fog_alpha == 2.0) form = kPowTwo;
  else if (fog_alpha == 3.0) form = kPowThree;
  hipLaunchKernelGGL(fog_weights_kernel, dim3(div_up(seq_len, kThreads)), dim3(kThreads), 0, as_stream(stream),
                     weights, seq_len, clear_start, inv_den, a, form);
  return check_launch("fog weights");
}

extern "C" int kessie_kv_cache_write(void* kv_pool, int64_t page_stride, int64_t tok_stride, int64_t kv_stride,
                                     int64_t head_stride, const void* key, int64_t key_tok_stride,
                                     int64_t key_head_stride, const void* value, int64_t value_tok_stride,
                                     int64_t value_head_stride, const int64_t* slot_mapping, int num_tokens,
                                     int num_kv_heads, int head_dim, int page_size, int num_pages, int dtype,
                                     void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0 && page_size > 0 && num_pages >= 0,
                 KESSIE_ERR_INVALID, "kv cache write: bad sizes T=%d H=%d D=%d P=%d pages=%d", num_tokens,
                 num_kv_heads, head_dim, page_size, num_pages);
  if (num_tokens == 0 || num_pages == 0) return KESSIE_OK;
  KESSIE_REQUIRE(kv_pool && key && value && slot_mapping, KESSIE_ERR_INVALID, "kv cache write: null pointer");
  KESSIE_REQUIRE(head_stride >= head_dim && tok_stride >= (int64_t)num_kv_heads * head_stride && kv_stride > 0,
                 KESSIE_ERR_INVALID, "kv cache write: pool strides overlap");
  WriteArgs a{kv_pool, page_stride, tok_stride, kv_stride, head_stride, key, value, key_tok_stride, key_head_stride,
              value_tok_stride, value_head_stride, slot_mapping, num_tokens, num_kv_heads, head_dim, page_size,
              num_pages};
  const hipStream_t s = as_stream(stream);
  switch (dtype) {
    case KESSIE_DTYPE_BF16: return kv_write_launch<bf16_t>(a, s);
    case KESSIE_DTYPE_F16: return kv_write_launch<f16_t>(a, s);
    case KESSIE_DTYPE_F32: return kv_write_launch<float>(a, s);
  }
  set_error(KESSIE_ERR_UNSUPPORTED, "kv cache write: dtype %d", dtype);
  return KESSIE_ERR_UNSUPPORTED;
}

extern "C" int kessie_hf_fog_weights_fill(float* weights, int seq_len, double fog_alpha, double fog_start,
                                          void* stream) {
  clear_error();
  KESSIE_REQUIRE(seq_len >= 0, KESSIE_ERR_INVALID, "hf fog weights: seq_len %d", seq_len);
  if (seq_len == 0) return KESSIE_OK;
  KESSIE_REQUIRE(weights != nullptr, KESSIE_ERR_INVALID, "hf fog weights: null buffer");
  const HfFog f = hf_fog_params(seq_len, fog_alpha, fog_start);
  hipLaunchKernelGGL(hf_fog_weights_kernel, dim3(div_up(seq_len, kThreads)), dim3(kThreads), 0, as_stream(stream),
                     weights, seq_len, f.fc, f.inv_den, f.alpha, f.form);
  return check_launch("hf fog weights");
}

extern "C" int kessie_hf_fog_apply(const void* v, int64_t v_bs, int64_t v_hs, int64_t v_ts, void* out, int64_t o_bs,
                                   int64_t o_hs, int64_t o_ts, int batch, int num_heads, int seq_len, int head_dim,
                                   double fog_alpha, double fog_start, int dtype, void* stream) {
  clear_error();
  KESSIE_REQUIRE(batch >= 0 && num_heads > 0 && seq_len >= 0 && head_dim > 0, KESSIE_ERR_INVALID,
                 "hf fog apply: B=%d H=%d N=%d D=%d", batch, num_heads, seq_len, head_dim);
  if (batch == 0 || seq_len == 0) return KESSIE_OK;
  KESSIE_REQUIRE(v && out, KESSIE_ERR_INVALID, "hf fog apply: null pointer");
  const int esz = dtype_size(dtype);
  KESSIE_REQUIRE(esz > 0, KESSIE_ERR_UNSUPPORTED, "hf fog apply: dtype %d", dtype);
  const int N = 16 / esz;
  KESSIE_REQUIRE(head_dim % N == 0 && aligned16(v) && aligned16(out) && v_bs % N == 0 && v_hs % N == 0 &&
                     v_ts % N == 0 && o_bs % N == 0 && o_hs % N == 0 && o_ts % N == 0,
                 KESSIE_ERR_UNSUPPORTED, "hf fog apply: rows must be 16-byte aligned multiples of 16 bytes");
  const HfFog f = hf_fog_params(seq_len, fog_alpha, fog_start);
  const int64_t items = (int64_t)batch * num_heads * seq_len * (head_dim / N);
  const int64_t grid = (items + kThreads - 1) / kThreads;
  KESSIE_REQUIRE(grid <= 0x7fffffff, KESSIE_ERR_UNSUPPORTED, "hf fog apply: too large");
  const hipStream_t s = as_stream(stream);
  const int BH = batch * num_heads;
  switch (dtype) {
    case KESSIE_DTYPE_BF16:
      hipLaunchKernelGGL(hf_fog_apply_kernel<bf16_t>, dim3((unsigned)grid), dim3(kThreads), 0, s,
                         static_cast<const bf16_t*>(v), static_cast<bf16_t*>(out), BH, num_heads, seq_len, head_dim,
                         v_bs, v_hs, v_ts, o_bs, o_hs, o_ts, f.fc, f.inv_den, f.alpha, f.form);
      break;
    case KESSIE_DTYPE_F16:
      hipLaunchKernelGGL(hf_fog_apply_kernel<f16_t>, dim3((unsigned)grid), dim3(kThreads), 0, s,
                         static_cast<const f16_t*>(v), static_cast<f16_t*>(out), BH, num_heads, seq_len, head_dim,
                         v_bs, v_hs, v_ts, o_bs, o_hs, o_ts, f.fc, f.inv_den, f.alpha, f.form);
      break;
    case KESSIE_DTYPE_F32:
      hipLaunchKernelGGL(hf_fog_apply_kernel<float>, dim3((unsigned)grid), dim3(kThreads), 0, s,
                         static_cast<const float*>(v), static_cast<float*>(out), BH, num_heads, seq_len, head_dim,
                         v_bs, v_hs, v_ts, o_bs, o_hs, o_ts, f.fc, f.inv_den, f.alpha, f.form);
      break;
    default:
      set_error(KESSIE_ERR_UNSUPPORTED, "hf fog apply: dtype %d", dtype);
      return KESSIE_ERR_UNSUPPORTED;
  }
  return check_launch("hf fog apply");
}

template <typename T>
int hf_append_fog_launch(AppendFogArgs<T> a, int BH, hipStream_t s) {
  constexpr int N = 16 / (int)sizeof(T);
  const int n = a.vfog ? a.n_old + a.t_new : a.t_new;
  const int64_t items = (int64_t)n * (a.D / N);
  const int64_t gx = (items + (int64_t)kThreads * kAppendChunks - 1) / ((int64_t)kThreads * kAppendChunks);
  KESSIE_REQUIRE(gx <= 0x7fffffff && BH <= 65535, KESSIE_ERR_UNSUPPORTED, "hf append fog: too large");
  hipLaunchKernelGGL(hf_append_fog_kernel<T>, dim3((unsigned)gx, (unsigned)BH), dim3(kThreads), 0, s, a);
  return check_launch("hf append fog");
}

extern "C" int kessie_hf_append_fog(void* k_arena, void* v_arena, int64_t a_bs, int64_t a_hs, int64_t a_ts,
                                    const void* new_k, int64_t k_bs, int64_t k_hs, int64_t k_ts, const void* new_v,
                                    int64_t v_bs, int64_t v_hs, int64_t v_ts, void* vfog, int64_t o_bs, int64_t o_hs,
                                    int64_t o_ts, int batch, int num_heads, int n_old, int t_new, int head_dim,
                                    double fog_alpha, double fog_start, int dtype, void* stream) {
  clear_error();
  KESSIE_REQUIRE(batch >= 0 && num_heads > 0 && n_old >= 0 && t_new >= 0 && head_dim > 0, KESSIE_ERR_INVALID,
                 "hf append fog: B=%d H=%d n_old=%d t_new=%d D=%d", batch, num_heads, n_old, t_new, head_dim);
  KESSIE_REQUIRE((int64_t)n_old + t_new <= 0x7fffffff, KESSIE_ERR_INVALID, "hf append fog: window too long");
  if (batch == 0 || (t_new == 0 && (vfog == nullptr || n_old == 0))) return KESSIE_OK;
  KESSIE_REQUIRE(k_arena && v_arena && (t_new == 0 || (new_k && new_v)), KESSIE_ERR_INVALID,
                 "hf append fog: null pointer");
  const int esz = dtype_size(dtype);
  KESSIE_REQUIRE(esz > 0, KESSIE_ERR_UNSUPPORTED, "hf append fog: dtype %d", dtype);
  const int N = 16 / esz;
  const bool rows16 = head_dim % N == 0 && aligned16(k_arena) && aligned16(v_arena) && a_bs % N == 0 &&
                      a_hs % N == 0 && a_ts % N == 0 &&
                      (t_new == 0 || (aligned16(new_k) && aligned16(new_v) && k_bs % N == 0 && k_hs % N == 0 &&
                                      k_ts % N == 0 && v_bs % N == 0 && v_hs % N == 0 && v_ts % N == 0)) &&
                      (vfog == nullptr || (aligned16(vfog) && o_bs % N == 0 && o_hs % N == 0 && o_ts % N == 0));
  KESSIE_REQUIRE(rows16, KESSIE_ERR_UNSUPPORTED, "hf append fog: rows must be 16-byte aligned multiples of 16 bytes");
  const HfFog f = hf_fog_params(n_old + t_new, fog_alpha, fog_start);
  const hipStream_t s = as_stream(stream);
  const int BH = batch * num_heads;
#define KESSIE_AF_ARGS(T)                                                                                        \
  AppendFogArgs<T>{static_cast<T*>(k_arena), static_cast<T*>(v_arena), a_bs, a_hs, a_ts,                       \
                   static_cast<const T*>(new_k), k_bs, k_hs, k_ts, static_cast<const T*>(new_v), v_bs, v_hs, v_ts, \
                   static_cast<T*>(vfog), o_bs, o_hs, o_ts, num_heads, n_old, t_new, head_dim, f.fc, f.inv_den,  \
                   f.alpha, f.form}
  switch (dtype) {
    case KESSIE_DTYPE_BF16: return hf_append_fog_launch<bf16_t>(KESSIE_AF_ARGS(bf16_t), BH, s);
    case KESSIE_DTYPE_F16: return hf_append_fog_launch<f16_t>(KESSIE_AF_ARGS(f16_t), BH, s);
    case KESSIE_DTYPE_F32: return hf_append_fog_launch<float>(KESSIE_AF_ARGS(float), BH, s);
    default:
      set_error(KESSIE_ERR_UNSUPPORTED, "hf append fog: dtype %d", dtype);
      return KESSIE_ERR_UNSUPPORTED;
  }
#undef KESSIE_AF_ARGS
}
