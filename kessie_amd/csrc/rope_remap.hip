// RoPE position remap of recalled K, in place, for gfx950.
//
// Semantics (kessie_hip_kernels.py:596-606, _rope_remap_ref):
//   inv[j]  = host table 1/(theta ** (j/half))          (fp32, j < half)
//   ang     = float(tgt[t] - orig[t]) * inv[j]          (one fp32 multiply)
//   x1 = K[t,h,j], x2 = K[t,h,j+half]  (upcast to fp32)
//   K[t,h,j]      = round(x1*cos(ang) - x2*sin(ang))
//   K[t,h,j+half] = round(x1*sin(ang) + x2*cos(ang))
// Every product and sum is rounded separately (no FMA contraction), exactly
// as the reference's sequence of torch ops does, so that given the same
// cos/sin values the stored element is bit-identical.
//
// Design: HBM-bound (2 bytes read + 2 written per element, 4 flops).  A
// workgroup owns a tile of tokens.  Phase 1 evaluates cos/sin once per
// (token, frequency) into LDS, shared by all heads.  Phase 2 streams the K rows
// with 16-byte loads: each lane owns one chunk pair (8 elements of the first
// half of a head and the matching 8 of the second half), so a wave's loads
// cover whole 128-byte segments of a token's K row.
// The access pattern, not the arithmetic, bounds it.  In interleaved K/V
// pages K is the first 2 KiB of every 4 KiB token row of random 64 KiB pages:
// measured on MI355X with the measurement probes (bytes read + written per
// second), that half-row pattern reaches 4.8 TB/s updated in place and the
// same out of place, 5.9 TB/s when only read; whole rows 5.6 TB/s updated and
// 6.8 TB/s read.  A dense K tensor updated in place by this kernel with the
// rotation replaced by the identity reaches 6.0 TB/s; random 32 KiB K-only
// pages 4.7 TB/s.
#include "common.h"

namespace kessie {
namespace {

constexpr int kRemapThreads = 256;  // generic instances: 4 tokens per 256-thread workgroup
constexpr int kRemapTile = 4;
constexpr int kVecMaxHalf = 128;    // vectorised kernel: head_dim <= 256

// Byte-free addressing helper: element offset of token t's K row, or -1 when
// the token's page id is out of range.
__device__ __forceinline__ int64_t token_row(int t, const int32_t* __restrict__ page_list, int num_pages,
                                             int page_size, int64_t page_stride, int64_t tok_stride) {
  if (page_list == nullptr) return (int64_t)t * tok_stride;
  const int page = page_list[t / page_size];
  if (page < 0 || page >= num_pages) return -1;
  return (int64_t)page * page_stride + (int64_t)(t % page_size) * tok_stride;
}

__device__ __forceinline__ float inv_freq_at(const float* __restrict__ inv_freq, float theta, int j, int half) {
  if (inv_freq != nullptr) return inv_freq[j];
  // Legacy entry point: no host table was supplied.
  return 1.0f / powf(theta, (float)j / (float)half);
}

template <typename T>
struct Vec16;  // 16 bytes of T
template <>
struct Vec16<bf16_t> {
  static constexpr int N = 8;
  typedef bf16x8 type;
};
template <>
struct Vec16<f16_t> {
  static constexpr int N = 8;
  typedef f16x8 type;
};
template <>
struct Vec16<float> {
  static constexpr int N = 4;
  typedef f32x4 type;
};

// Vectorised kernel: 16-byte chunks.  Requires half % N == 0, 16-byte aligned
// rows and head starts.  The K chunks of a round are loaded into registers
// before the cos/sin phase, so HBM latency overlaps the trigonometry; the
// workgroup barrier that publishes cos/sin keeps those loads ahead of it.
// One chunk pair (two 16-byte loads) per thread per round.  Tile shape
// (measured, 65,536 bf16 tokens of 8 heads x 128 in random interleaved K/V
// 16-token pages): one page's 16 tokens per 1,024-thread workgroup
// 52.1-52.7 us; 8 tokens per 512 threads 54.3; 4 per 256 55.0-55.2; 1 per 64
// 53.7; 16 tokens with 2 or 4 pairs per thread 58.6-58.7; 32 tokens
// 57.4-59.7.  Exchanging chunk halves by lane shuffle (each wave reading 1 KiB
// contiguous) measured the same, and so did (or worse) persistent workgroups
// that load their next tile before rotating this one, and plain instead of
// non-temporal loads and stores (8-10 % slower), on every layout.
constexpr int kRemapItems = 1;  // chunk pairs per thread per round

// kHalf / kHeads / kPage > 0 fix head_dim/2, the head count and the page size
// at compile time (the index arithmetic then has no runtime divisions); 0
// takes them from the arguments.  kTile tokens per workgroup of kThreads.
template <typename T, int kHalf, int kHeads, int kPage, int kTile, int kThreads>
__global__ __launch_bounds__(kThreads) void rope_remap_vec(
    T* __restrict__ pool, int64_t page_stride, int64_t tok_stride, int64_t head_stride,
    const int32_t* __restrict__ page_list, int num_pages, const int32_t* __restrict__ orig_pos,
    const int32_t* __restrict__ tgt_pos, const float* __restrict__ inv_freq, float theta, int num_tokens,
    int num_heads_arg, int half_arg, int page_size_arg) {
#pragma clang fp contract(off)
  typedef typename Vec16<T>::type V;
  constexpr int N = Vec16<T>::N;
  __shared__ float2 cs[kTile * kVecMaxHalf];  // [token][j] = (cos, sin)
  const int half = kHalf > 0 ? kHalf : half_arg;
  const int num_heads = kHeads > 0 ? kHeads : num_heads_arg;
  const int page_size = kPage > 0 ? kPage : page_size_arg;

  const int t0 = blockIdx.x * kTile;
  const int ntok = min(kTile, num_tokens - t0);
  const int chunks = half / N;  // chunk pairs per head
  const int per_tok = num_heads * chunks;
  const int n_work = ntok * per_tok;

  for (int round = 0; round * kRemapItems * kThreads < n_work; ++round) {
    const int base = round * kRemapItems * kThreads;
    V a[kRemapItems], b[kRemapItems];
    T* p1[kRemapItems];
    int csi[kRemapItems];
#pragma unroll
    for (int it = 0; it < kRemapItems; ++it) {
      const int i = base + it * kThreads + threadIdx.x;
      p1[it] = nullptr;
      csi[it] = 0;
      if (i < n_work) {
        const int tt = i / per_tok;
        const int r = i - tt * per_tok;
        const int h = r / chunks;
        const int c = r - h * chunks;
        const int64_t row = token_row(t0 + tt, page_list, num_pages, page_size, page_stride, tok_stride);
        if (row >= 0) {
          p1[it] = pool + row + (int64_t)h * head_stride + c * N;
          // Streaming accesses: every byte is touched once, so non-temporal
          // loads/stores keep the in-place update from churning the caches.
          a[it] = __builtin_nontemporal_load(reinterpret_cast<const V*>(p1[it]));
          b[it] = __builtin_nontemporal_load(reinterpret_cast<const V*>(p1[it] + half));
          csi[it] = tt * half + c * N;
        }
      }
    }
    if (round == 0) {
      const int n_ang = ntok * half;
      for (int i = threadIdx.x; i < n_ang; i += kThreads) {
        const int tt = i / half;
        const int j = i - tt * half;
        const int t = t0 + tt;
        const float delta = (float)(tgt_pos[t] - orig_pos[t]);
        const float ang = delta * inv_freq_at(inv_freq, theta, j, half);
        float s, c;
        sincosf(ang, &s, &c);
        cs[i] = make_float2(c, s);
      }
      __syncthreads();
    }
#pragma unroll
    for (int it = 0; it < kRemapItems; ++it) {
      if (p1[it] == nullptr) continue;
      const float2* csr = cs + csi[it];
      V y1, y2;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float2 q = csr[e];
        const float x1 = to_f32(a[it][e]);
        const float x2 = to_f32(b[it][e]);
        const float u1 = x1 * q.x;
        const float u2 = x2 * q.y;
        const float w1 = x1 * q.y;
        const float w2 = x2 * q.x;
        y1[e] = from_f32<T>(u1 - u2);
        y2[e] = from_f32<T>(w1 + w2);
      }
      __builtin_nontemporal_store(y1, reinterpret_cast<V*>(p1[it]));
      __builtin_nontemporal_store(y2, reinterpret_cast<V*>(p1[it] + half));
    }
  }
}

// Scalar kernel for any even head_dim / alignment: one thread per
// (token, head, pair).
template <typename T>
__global__ __launch_bounds__(kRemapThreads) void rope_remap_scalar(
    T* __restrict__ pool, int64_t page_stride, int64_t tok_stride, int64_t head_stride,
    const int32_t* __restrict__ page_list, int num_pages, const int32_t* __restrict__ orig_pos,
    const int32_t* __restrict__ tgt_pos, const float* __restrict__ inv_freq, float theta, int num_tokens,
    int num_heads, int half, int page_size) {
#pragma clang fp contract(off)
  const int64_t gid = (int64_t)blockIdx.x * kRemapThreads + threadIdx.x;
  const int64_t total = (int64_t)num_tokens * num_heads * half;
  if (gid >= total) return;
  const int j = (int)(gid % half);
  const int64_t rem = gid / half;
  const int h = (int)(rem % num_heads);
  const int t = (int)(rem / num_heads);
  const int64_t row = token_row(t, page_list, num_pages, page_size, page_stride, tok_stride);
  if (row < 0) return;
  const float delta = (float)(tgt_pos[t] - orig_pos[t]);
  const float ang = delta * inv_freq_at(inv_freq, theta, j, half);
  float s, c;
  sincosf(ang, &s, &c);
  T* p1 = pool + row + (int64_t)h * head_stride + j;
  T* p2 = p1 + half;
  const float x1 = to_f32(*p1);
  const float x2 = to_f32(*p2);
  const float u1 = x1 * c;
  const float u2 = x2 * s;
  const float w1 = x1 * s;
  const float w2 = x2 * c;
  *p1 = from_f32<T>(u1 - u2);
  *p2 = from_f32<T>(w1 + w2);
}

template <typename T>
int launch_remap(void* pool, int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                 const int32_t* page_list, int num_pages, const int32_t* orig_pos, const int32_t* tgt_pos,
                 const float* inv_freq, float theta, int num_tokens, int num_heads, int head_dim,
                 int page_size, hipStream_t stream) {
  const int half = head_dim / 2;
  constexpr int N = Vec16<T>::N;
  const bool vec_ok = (half % N == 0) && (half <= kVecMaxHalf) && aligned16(pool) &&
                      (page_list == nullptr || page_stride % N == 0) && tok_stride % N == 0 &&
                      head_stride % N == 0;
  T* p = static_cast<T*>(pool);
  if (vec_ok) {
    // Specialised instances for the Llama-style K shape (8 kv heads x 128,
    // 16-token pages or dense rows), one chunk pair per thread (bf16/fp16;
    // fp32 rows hold twice the chunks and take two rounds).  The tile follows
    // the row layout (65,536 bf16 tokens, one MI355X): K rows that are the
    // first half of interleaved K/V token rows run best as one page's 16
    // tokens per 1,024-thread workgroup (54 us; 8 tokens per 512 threads 56);
    // contiguous K rows (a dense [T][H][D] tensor, K-only pages) as 8 tokens
    // per 512 threads (dense 45.5-46 us against 47 for the 16-token shape;
    // K-only pages 57 either way).
    const bool k_rows_contiguous = tok_stride == (int64_t)num_heads * head_stride;
    if (half == 64 && num_heads == 8 && (page_list == nullptr || page_size == 16) && k_rows_contiguous)
      hipLaunchKernelGGL((rope_remap_vec<T, 64, 8, 16, 8, 512>), dim3(div_up(num_tokens, 8)), dim3(512), 0,
                         stream, p, page_stride, tok_stride, head_stride, page_list, num_pages, orig_pos, tgt_pos,
                         inv_freq, theta, num_tokens, num_heads, half, page_size);
    else if (half == 64 && num_heads == 8 && (page_list == nullptr || page_size == 16))
      hipLaunchKernelGGL((rope_remap_vec<T, 64, 8, 16, 16, 1024>), dim3(div_up(num_tokens, 16)), dim3(1024), 0,
                         stream, p, page_stride, tok_stride, head_stride, page_list, num_pages, orig_pos, tgt_pos,
                         inv_freq, theta, num_tokens, num_heads, half, page_size);
    else
      hipLaunchKernelGGL((rope_remap_vec<T, 0, 0, 0, kRemapTile, kRemapThreads>), dim3(div_up(num_tokens, kRemapTile)),
                         dim3(kRemapThreads), 0, stream, p, page_stride, tok_stride, head_stride, page_list,
                         num_pages, orig_pos, tgt_pos, inv_freq, theta, num_tokens, num_heads, half, page_size);
  } else {
    const int64_t total = (int64_t)num_tokens * num_heads * half;
    const int64_t grid = (total + kRemapThreads - 1) / kRemapThreads;
    if (grid > 0x7fffffff) {
      set_error(KESSIE_ERR_UNSUPPORTED, "rope_remap: %lld elements exceed one launch", (long long)total);
      return KESSIE_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL(rope_remap_scalar<T>, dim3((unsigned)grid), dim3(kRemapThreads), 0, stream, p,
                       page_stride, tok_stride, head_stride, page_list, num_pages, orig_pos, tgt_pos, inv_freq,
                       theta, num_tokens, num_heads, half, page_size);
  }
  return check_launch("rope_remap");
}

int remap_dispatch(void* pool, int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                   const int32_t* page_list, int num_pages, const int32_t* orig_pos, const int32_t* tgt_pos,
                   const float* inv_freq, float theta, int num_tokens, int num_heads, int head_dim, int page_size,
                   int dtype, hipStream_t stream) {
  KESSIE_REQUIRE(num_tokens >= 0 && num_heads > 0 && head_dim > 0, KESSIE_ERR_INVALID,
                 "rope_remap: bad sizes T=%d H=%d D=%d", num_tokens, num_heads, head_dim);
  KESSIE_REQUIRE(head_dim % 2 == 0, KESSIE_ERR_INVALID, "rope_remap: head_dim %d must be even", head_dim);
  if (num_tokens == 0) return KESSIE_OK;
  KESSIE_REQUIRE(pool && orig_pos && tgt_pos, KESSIE_ERR_INVALID, "rope_remap: null pointer");
  KESSIE_REQUIRE(page_list == nullptr || (page_size > 0 && num_pages > 0), KESSIE_ERR_INVALID,
                 "rope_remap: page_size=%d num_pages=%d", page_size, num_pages);
  KESSIE_REQUIRE(tok_stride >= (int64_t)num_heads * head_stride && head_stride >= head_dim, KESSIE_ERR_INVALID,
                 "rope_remap: strides overlap (tok %lld head %lld)", (long long)tok_stride, (long long)head_stride);
  switch (dtype) {
    case KESSIE_DTYPE_BF16:
      return launch_remap<bf16_t>(pool, page_stride, tok_stride, head_stride, page_list, num_pages, orig_pos,
                                  tgt_pos, inv_freq, theta, num_tokens, num_heads, head_dim, page_size, stream);
    case KESSIE_DTYPE_F16:
      return launch_remap<f16_t>(pool, page_stride, tok_stride, head_stride, page_list, num_pages, orig_pos,
                                 tgt_pos, inv_freq, theta, num_tokens, num_heads, head_dim, page_size, stream);
    case KESSIE_DTYPE_F32:
      return launch_remap<float>(pool, page_stride, tok_stride, head_stride, page_list, num_pages, orig_pos,
                                 tgt_pos, inv_freq, theta, num_tokens, num_heads, head_dim, page_size, stream);
    default:
      set_error(KESSIE_ERR_UNSUPPORTED, "rope_remap: dtype %d", dtype);
      return KESSIE_ERR_UNSUPPORTED;
  }
}

}  // namespace
}  // namespace kessie

extern "C" int kessie_rope_remap_paged(void* kv_pool, int64_t page_stride, int64_t tok_stride,
                                       int64_t head_stride, const int32_t* page_list, int num_pages,
                                       const int32_t* orig_pos, const int32_t* tgt_pos, const float* inv_freq,
                                       int num_tokens, int num_heads, int head_dim, int page_size, int dtype,
                                       void* stream) {
  kessie::clear_error();
  KESSIE_REQUIRE(inv_freq != nullptr, KESSIE_ERR_INVALID, "rope_remap: inv_freq table is required");
  return kessie::remap_dispatch(kv_pool, page_stride, tok_stride, head_stride, page_list, num_pages, orig_pos,
                                tgt_pos, inv_freq, 0.0f, num_tokens, num_heads, head_dim, page_size, dtype,
                                kessie::as_stream(stream));
}

// Reference launcher signature (kessie_kernels_v2.hip:827-842): fp16 dense
// [T][H][2*half_dim]; the frequency table is evaluated on the device from
// rope_theta because this signature carries no table.
extern "C" void launch_kessie_rope_remap(void* k_data, const void* orig_positions, const void* target_positions,
                                         float rope_theta, int num_tokens, int num_heads, int half_dim,
                                         void* stream) {
  kessie::clear_error();
  const int head_dim = 2 * half_dim;
  kessie::remap_dispatch(k_data, 0, (int64_t)num_heads * head_dim, head_dim, nullptr, 0,
                         static_cast<const int32_t*>(orig_positions), static_cast<const int32_t*>(target_positions),
                         nullptr, rope_theta, num_tokens, num_heads, head_dim, 0, KESSIE_DTYPE_F16,
                         kessie::as_stream(stream));
}
