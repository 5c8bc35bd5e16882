// Semantic index query for gfx950: cosine similarity of one query embedding
// against every chunk embedding of the conversation index, then the exact
// top-k.  Replaces _kessie_index_query_kernel (kessie_hip_kernels.py:344-360)
// and the numpy / FAISS flat searches of VectorIndex.search
// (kessie_exp3.py:89-105).
//
// Similarity: sim_i = dot(q, e_i) * inv(|q|) * inv(|e_i|), fp32 accumulation
// (rows may be fp32, bf16 or fp16), with the normalisation of the call site
// being replaced (norm_mode):
//   0  inv(n) = 1 / sqrt(n^2 + 1e-8)       _kessie_index_query_kernel
//   1  inv(n) = 1 / (n + 1e-8)             the numpy searches, kessie_exp3.py:1866-1869
//   2  inv(n) = n < 1e-8 ? 1 : 1 / n       VectorIndex.rebuild / search, kessie_exp3.py:74-76,90-93  The scan is HBM-bound: 16 lanes own one row
// (16 bytes per lane per load, 256 contiguous bytes per 16 lanes), four rows
// per wave per step, the 16-lane dot / norm reductions on DPP row shuffles.
//
// Top-k order: score descending, ties by ascending chunk index -- a total
// order, encoded as the 64-bit key (~ordered(score) << 32 | index) sorted
// ascending.  Exact: each pass reduces groups of keys to their first k, sorted
// -- k <= 64: a wave per 512 keys, in registers (lane shuffles); larger k: a
// block per 2,048 keys, bitonic in LDS -- and passes repeat until one group
// remains, whose first k keys are the answer.
#include "common.h"

namespace kessie {
namespace attn {
int device_cus();  // compute units of the current device (fog_attention.hip)
}  // namespace attn
}  // namespace kessie

namespace kessie {
namespace index {
namespace {

constexpr int kScanThreads = 256;
constexpr int kSortN = 2048;  // keys per block in a top-k pass
constexpr int kSortThreads = 256;
constexpr int kMaxTopK = 1024;

template <typename T>
struct Row16;  // 16-byte vector of T and its element count
template <>
struct Row16<float> {
  typedef f32x4 type;
  static constexpr int N = 4;
};
template <>
struct Row16<bf16_t> {
  typedef bf16x8 type;
  static constexpr int N = 8;
};
template <>
struct Row16<f16_t> {
  typedef f16x8 type;
  static constexpr int N = 8;
};

__device__ __forceinline__ float inv_norm(float sumsq, int mode) {
  if (mode == 0) return 1.0f / sqrtf(sumsq + 1e-8f);
  const float n = sqrtf(sumsq);
  if (mode == 1) return 1.0f / (n + 1e-8f);
  return n < 1e-8f ? 1.0f : 1.0f / n;
}

__device__ __forceinline__ float sum16(float v) {
  // Reduce over the 16 lanes of a DPP row (xor 8, 4, 2, 1 within the row).
  v += __shfl_xor(v, 8, 16);
  v += __shfl_xor(v, 4, 16);
  v += __shfl_xor(v, 2, 16);
  v += __shfl_xor(v, 1, 16);
  return v;
}

// q_scale = inv(|q|), computed once per block from the query.
template <typename T>
__global__ __launch_bounds__(kScanThreads) void cosine_scan_kernel(const T* __restrict__ rows, int64_t row_stride,
                                                                   int n, int d, const float* __restrict__ q,
                                                                   float* __restrict__ sims, int mode) {
  typedef typename Row16<T>::type V;
  constexpr int N = Row16<T>::N;
  __shared__ float qs[1024];
  __shared__ float red[kScanThreads / 64];
  float part = 0.0f;
  for (int i = threadIdx.x; i < d; i += kScanThreads) {
    const float x = q[i];
    qs[i] = x;
    part += x * x;
  }
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
  __syncthreads();
  float qq = 0.0f;
#pragma unroll
  for (int w = 0; w < kScanThreads / 64; ++w) qq += red[w];
  const float q_scale = inv_norm(qq, mode);

  const int sub = threadIdx.x & 15;              // lane within the row group
  const int group = (blockIdx.x * kScanThreads + threadIdx.x) >> 4;
  const int groups = (gridDim.x * kScanThreads) >> 4;
  const int chunks = d / N;                      // 16-byte chunks per row
  for (int r = group; r < n; r += groups) {
    const T* row = rows + (int64_t)r * row_stride;
    float dot = 0.0f, ee = 0.0f;
    for (int c = sub; c < chunks; c += 16) {
      const V v = __builtin_nontemporal_load(reinterpret_cast<const V*>(row) + c);
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float x = to_f32(v[e]);
        dot += x * qs[c * N + e];
        ee += x * x;
      }
    }
    dot = sum16(dot);
    ee = sum16(ee);
    if (sub == 0) sims[r] = dot * q_scale * inv_norm(ee, mode);
  }
}

// Monotone map of a float to uint32 (ascending), -0 folded into +0.
__device__ __forceinline__ uint32_t ordered(float s) {
  uint32_t b = __float_as_uint(s == 0.0f ? 0.0f : s);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float unordered(uint32_t o) {
  const uint32_t b = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(b);
}

// Keys of the first pass: (~ordered(score) << 32) | index; ascending = best first.
__device__ __forceinline__ uint64_t make_key(float s, uint32_t i) {
  return ((uint64_t)(~ordered(s)) << 32) | i;
}

// One pass: block b sorts keys [b*kSortN, ...) (scores from `sims` when
// keys_in is null) and writes its first `keep` keys to keys_out[b*keep ...].
__global__ __launch_bounds__(kSortThreads) void topk_pass_kernel(const float* __restrict__ sims,
                                                                 const uint64_t* __restrict__ keys_in, int n,
                                                                 int keep, uint64_t* __restrict__ keys_out) {
  __shared__ uint64_t sk[kSortN];
  const int base = blockIdx.x * kSortN;
  for (int i = threadIdx.x; i < kSortN; i += kSortThreads) {
    const int g = base + i;
    uint64_t key = ~0ull;  // padding sorts last
    if (g < n) key = keys_in ? keys_in[g] : make_key(sims[g], (uint32_t)g);
    sk[i] = key;
  }
  __syncthreads();
  for (int size = 2; size <= kSortN; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < kSortN / 2; t += kSortThreads) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t a = sk[lo], b = sk[hi];
        if ((a > b) == up) {
          sk[lo] = b;
          sk[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < keep; i += kSortThreads) keys_out[(int64_t)blockIdx.x * keep + i] = sk[i];
}

// Small-k path (k <= 64): one key per lane, a wave holds its running best 64
// keys sorted across its lanes and folds in one 64-key segment at a time:
// sort the segment (bitonic, lane shuffles), take the lane-wise min against
// the running list reversed (that keeps the 64 smallest of the union, as a
// bitonic sequence), and re-sort it with the six merge stages.  No LDS, no
// barriers.  Each wave consumes kWaveKeys keys and writes its first `keep`
// (short chains: the shuffles are latency-bound, so more waves with fewer
// segments each).  The last pass (one wave) writes ids / scores directly.
constexpr int kWaveSegs = 2;
constexpr int kWaveKeys = 64 * kWaveSegs;
constexpr int kWaveThreads = 256;

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t x, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)x, m), hi = __shfl_xor((uint32_t)(x >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl64(uint64_t x, int src) {
  const uint32_t lo = __shfl((uint32_t)x, src), hi = __shfl((uint32_t)(x >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_sort64(uint64_t x, int lane) {
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t y = shfl_xor64(x, stride);
      const bool up = (lane & size) == 0 || size == 64;
      const bool lower = (lane & stride) == 0;
      x = (lower == up) ? (x < y ? x : y) : (x < y ? y : x);
    }
  return x;
}

__global__ __launch_bounds__(kWaveThreads) void topk_wave_kernel(const float* __restrict__ sims,
                                                                 const uint64_t* __restrict__ keys_in, int n,
                                                                 int keep, uint64_t* __restrict__ keys_out,
                                                                 int32_t* __restrict__ ids, float* __restrict__ scores,
                                                                 int top_k) {
  const int lane = threadIdx.x & 63;
  const int wave = (blockIdx.x * kWaveThreads + threadIdx.x) >> 6;
  const int64_t base = (int64_t)wave * kWaveKeys;
  if (base >= n) return;  // whole wave leaves together
  uint64_t best = ~0ull;
  for (int seg = 0; seg < kWaveSegs; ++seg) {
    const int64_t g = base + seg * 64 + lane;
    uint64_t x = ~0ull;
    if (g < n) x = keys_in ? keys_in[g] : make_key(sims[g], (uint32_t)g);
    x = wave_sort64(x, lane);
    const uint64_t rev = shfl64(x, 63 - lane);
    uint64_t m = best < rev ? best : rev;  // the 64 smallest of the union, bitonic
#pragma unroll
    for (int stride = 32; stride > 0; stride >>= 1) {
      const uint64_t y = shfl_xor64(m, stride);
      m = ((lane & stride) == 0) ? (m < y ? m : y) : (m < y ? y : m);
    }
    best = m;
  }
  if (top_k == 0) {
    if (lane < keep) keys_out[(int64_t)wave * keep + lane] = best;
    return;
  }
  for (int i = lane; i < top_k; i += 64) {  // final pass: i < keep only when i == lane
    const bool ok = i < keep;
    if (ids) ids[i] = ok ? (int32_t)(best & 0xffffffffu) : -1;
    if (scores) scores[i] = ok ? unordered(~(uint32_t)(best >> 32)) : -__builtin_huge_valf();
  }
}

__global__ void topk_unpack_kernel(const uint64_t* __restrict__ keys, int k, int n, int32_t* __restrict__ ids,
                                   float* __restrict__ scores) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= k) return;
  const bool ok = i < n;
  const uint64_t key = ok ? keys[i] : 0;
  if (ids) ids[i] = ok ? (int32_t)(key & 0xffffffffu) : -1;
  if (scores) scores[i] = ok ? unordered(~(uint32_t)(key >> 32)) : -__builtin_huge_valf();
}

// Fused path (k <= kFusedK): the scan keeps each workgroup's top-k.  A wave
// scans 16 rows, four per 16-lane group with their loads issued together;
// the workgroup's keys go to LDS, one per row, and every thread counts the
// keys below one of them over a segment of the others (LDS adds sum the
// counts), so each key's rank comes out with no selection rounds; the first
// k are written in order.  One workgroup then takes the first k of all
// workgroups' lists (the threshold pass of topk_merge_kernel, or selection
// rounds).  Per query at 78,125 x 256 fp32, back to back: 21.9 us with
// 64-bit selection rounds in both kernels, 21.2 with 32-bit rounds, 20.4 with
// the threshold merge, 20.2 with the scan's rank count, 19.9 with 10-wave
// workgroups (the scan alone, a plain grid-stride kernel: 14.9).  More rows
// per 16-lane group (8) or 64- and 256-row workgroups measured slower.
constexpr int kFusedK = 16;
constexpr int kFusedRowsGroup = 4;                                      // rows per 16-lane group
constexpr int kFusedRowsWave = 4 * kFusedRowsGroup;                     // 16 rows per wave
constexpr int kFusedWavesMin = 8;                                       // scan workgroups: 8 or 10 waves
constexpr int kFusedWavesMax = 10;
constexpr int kMergeThreads = 512;                                      // merge workgroup: 8 waves
constexpr int kMergeLoads = 6;                                          // keys a merge lane takes per pass

extern "C" __device__ unsigned int __ockl_wfred_min_u32(unsigned int);

// k rounds of selection over the keys the wave's lanes hold (x[0..M) each,
// unique but for the ~0 padding): round r takes the wave's smallest key out
// of its lane, and lane r keeps it.  Returns the lane's kept key (~0 for
// lanes >= k).  Every lane of the wave must take part.  A round reduces the
// keys' high words (the score) over the wave; when one slot of one lane holds
// that word, its low word (the chunk index) is read from there, and only on a
// tie (or when nothing but padding is left) do the low words of the tied
// slots take a second reduction -- two 32-bit reductions at most, against a
// 64-bit one whose compares and selects each take two instructions.
template <int M>
__device__ __forceinline__ uint64_t wave_select(const uint64_t (&x)[M], int k) {
  const int lane = threadIdx.x & 63;
  uint32_t hi[M], lo[M];
#pragma unroll
  for (int j = 0; j < M; ++j) {
    hi[j] = (uint32_t)(x[j] >> 32);
    lo[j] = (uint32_t)x[j];
  }
  uint64_t kept = ~0ull;
  for (int r = 0; r < k; ++r) {
    uint32_t lm = hi[0];
#pragma unroll
    for (int j = 1; j < M; ++j) lm = hi[j] < lm ? hi[j] : lm;
    const uint32_t mh = __ockl_wfred_min_u32(lm);
    uint64_t bal[M];
    int count = 0;
#pragma unroll
    for (int j = 0; j < M; ++j) {
      bal[j] = __builtin_amdgcn_ballot_w64(hi[j] == mh);
      count += __builtin_popcountll(bal[j]);
    }
    uint32_t ml;
    if (count == 1) {  // the one slot whose high word is mh: read its low word, take it out
      uint32_t t = 0;
      uint64_t any = 0;
#pragma unroll
      for (int j = 0; j < M; ++j) {
        t = hi[j] == mh ? lo[j] : t;
        any |= bal[j];
      }
      ml = (uint32_t)__builtin_amdgcn_readlane((int)t, __builtin_ctzll(any));
#pragma unroll
      for (int j = 0; j < M; ++j)
        if (hi[j] == mh) {
          hi[j] = ~0u;
          lo[j] = ~0u;
        }
    } else {
      uint32_t c = ~0u;
#pragma unroll
      for (int j = 0; j < M; ++j) c = hi[j] == mh && lo[j] < c ? lo[j] : c;
      ml = __ockl_wfred_min_u32(c);
#pragma unroll
      for (int j = 0; j < M; ++j)
        if (hi[j] == mh && lo[j] == ml) {
          hi[j] = ~0u;
          lo[j] = ~0u;
        }
    }
    if (lane == r) kept = ((uint64_t)mh << 32) | ml;
  }
  return kept;
}

template <typename T, int W>
__global__ __launch_bounds__(64 * W) void scan_topk_kernel(const T* __restrict__ rows, int64_t row_stride,
                                                                  int n, int d, const float* __restrict__ q,
                                                                  float* __restrict__ sims, int mode, int k,
                                                                  uint64_t* __restrict__ keys_out) {
  typedef typename Row16<T>::type V;
  constexpr int N = Row16<T>::N;
  constexpr int R = kFusedRowsGroup;
  constexpr int kFusedThreads = 64 * W, kFusedRowsWg = kFusedRowsWave * W;
  __shared__ float qs[1024];
  __shared__ float red[kFusedThreads / 64];
  __shared__ uint64_t wg_keys[kFusedRowsWg];
  __shared__ int wg_rank[kFusedRowsWg];
  static_assert(kFusedThreads % kFusedRowsWg == 0 && kFusedRowsWg % (kFusedThreads / kFusedRowsWg) == 0,
                "scan_topk_kernel: rank segments");
  if (threadIdx.x < kFusedRowsWg) wg_rank[threadIdx.x] = 0;
  float part = 0.0f;
  for (int i = threadIdx.x; i < d; i += kFusedThreads) {
    const float x = q[i];
    qs[i] = x;
    part += x * x;
  }
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
  __syncthreads();
  float qq = 0.0f;
#pragma unroll
  for (int w = 0; w < kFusedThreads / 64; ++w) qq += red[w];
  const float q_scale = inv_norm(qq, mode);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 15, grp = lane >> 4;
  // Rows of this wave's groups: r0 + R grp + u, u < R.
  const int64_t r0 = (int64_t)blockIdx.x * kFusedRowsWg + kFusedRowsWave * wave;
  const int chunks = d / N;
  float dot[R], ee[R];
  int64_t r[R];
#pragma unroll
  for (int u = 0; u < R; ++u) {
    dot[u] = 0.0f;
    ee[u] = 0.0f;
    r[u] = r0 + R * grp + u;
  }
  for (int c = sub; c < chunks; c += 16) {
    V v[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int64_t rr = r[u] < n ? r[u] : 0;
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const V*>(rows + rr * row_stride) + c);
    }
#pragma unroll
    for (int u = 0; u < R; ++u)
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float x = to_f32(v[u][e]);
        dot[u] += x * qs[c * N + e];
        ee[u] += x * x;
      }
  }
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const float dd = sum16(dot[u]), nn = sum16(ee[u]);
    const float sim = dd * q_scale * inv_norm(nn, mode);
    const bool in = r[u] < n;
    if (sub == 0) {
      if (in) sims[r[u]] = sim;
      // Rows past n: distinct keys above every row's (row indices stay below 2^31).
      const int at = kFusedRowsWave * wave + R * grp + u;
      wg_keys[at] = in ? make_key(sim, (uint32_t)r[u]) : ~0ull - (uint64_t)(kFusedRowsWg - 1 - at);
    }
  }
  __syncthreads();
  // Rank of each of the workgroup's (distinct) keys: thread t counts the keys
  // below key t % kFusedRowsWg in segment t / kFusedRowsWg (broadcast LDS reads).
  constexpr int kSeg = kFusedRowsWg * kFusedRowsWg / kFusedThreads;
  const int mine_at = threadIdx.x % kFusedRowsWg, seg = threadIdx.x / kFusedRowsWg;
  const uint64_t mine = wg_keys[mine_at];
  int below = 0;
#pragma unroll
  for (int j = 0; j < kSeg; ++j) below += wg_keys[seg * kSeg + j] < mine ? 1 : 0;
  atomicAdd(&wg_rank[mine_at], below);
  __syncthreads();
  if (threadIdx.x < kFusedRowsWg) {
    const int rank = wg_rank[threadIdx.x];
    if (rank < k) keys_out[(int64_t)blockIdx.x * k + rank] = mine;
  }
}

// The wave's smallest key (every lane takes part): the smallest high word,
// then the smallest low word among the lanes holding it.
__device__ __forceinline__ uint64_t wave_min_key(uint64_t x) {
  const uint32_t hi = (uint32_t)(x >> 32);
  const uint32_t mh = __ockl_wfred_min_u32(hi);
  const uint32_t ml = __ockl_wfred_min_u32(hi == mh ? (uint32_t)x : ~0u);
  return ((uint64_t)mh << 32) | ml;
}

// Writes ids / scores [0, top_k): rank r < k from key, the rest -1 / -inf.
__device__ __forceinline__ void store_result(int32_t* ids, float* scores, int i, uint64_t key) {
  const bool ok = key != ~0ull;
  if (ids) ids[i] = ok ? (int32_t)(key & 0xffffffffu) : -1;
  if (scores) scores[i] = ok ? unordered(~(uint32_t)(key >> 32)) : -__builtin_huge_valf();
}

// Threshold merge (k <= kThreshK, nkeys <= kMergeLoads * kMergeThreads): T =
// the largest of the W waves' smallest keys bounds the k-th smallest key from
// above (W >= k distinct keys are <= T), so the answer is the first k of the
// keys <= T -- typically a few dozen -- ranked by counting; more than
// kThreshCand of them (keys clustered in one wave's share) falls back to the
// selection rounds.
constexpr int kThreshK = kMergeThreads / 64;
constexpr int kThreshCand = 64;  // one per lane of the ranking wave

// The first k of nkeys keys: each wave selects the first k of its share,
// carried from pass to pass (kMergeLoads keys per lane per pass), then the
// first wave selects over the waves' lists and writes ids and scores.
__global__ __launch_bounds__(kMergeThreads) void topk_merge_kernel(const uint64_t* __restrict__ keys, int64_t nkeys,
                                                                   int k, int32_t* __restrict__ ids,
                                                                   float* __restrict__ scores, int top_k) {
  constexpr int W = kMergeThreads / 64;
  __shared__ uint64_t lists[W * kFusedK];
  __shared__ uint64_t cand[kThreshCand];
  __shared__ uint64_t wmin[W];
  __shared__ int ncand;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (k <= kThreshK && nkeys <= (int64_t)kMergeLoads * kMergeThreads) {  // uniform
    uint64_t x[kMergeLoads];
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j) {
      const int64_t i = (int64_t)j * kMergeThreads + threadIdx.x;
      x[j] = i < nkeys ? keys[i] : ~0ull;
    }
    if (threadIdx.x == 0) ncand = 0;
    if (wave == 0) cand[lane] = ~0ull;  // the rank count reads whole groups of 8
    uint64_t lm = x[0];
#pragma unroll
    for (int j = 1; j < kMergeLoads; ++j) lm = x[j] < lm ? x[j] : lm;
    const uint64_t wm = wave_min_key(lm);
    if (lane == 0) wmin[wave] = wm;
    __syncthreads();
    uint64_t t = wmin[0];
#pragma unroll
    for (int w = 1; w < W; ++w) t = wmin[w] > t ? wmin[w] : t;
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j) cnt += x[j] <= t ? 1 : 0;
    if (cnt > 0) {
      int at = atomicAdd(&ncand, cnt);
#pragma unroll
      for (int j = 0; j < kMergeLoads; ++j)
        if (x[j] <= t) {
          if (at < kThreshCand) cand[at] = x[j];
          ++at;
        }
    }
    __syncthreads();
    const int c = ncand;
    if (c <= kThreshCand) {  // uniform
      if (wave != 0) return;
      const uint64_t mine = lane < c ? cand[lane] : ~0ull;
      int rank = 0;
      const int c8 = (c + 7) & ~7;
      for (int j = 0; j < c8; ++j) rank += cand[j] < mine ? 1 : 0;
      if (lane < c && rank < k) store_result(ids, scores, rank, mine);
      for (int i = k + lane; i < top_k; i += 64) store_result(ids, scores, i, ~0ull);
      return;
    }
  }
  uint64_t kept = ~0ull;  // lane r < k: the wave's r-th key so far
  for (int64_t base = 0; base < nkeys; base += (int64_t)kMergeLoads * kMergeThreads) {  // uniform trip count
    uint64_t x[kMergeLoads + 1];
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j) {
      const int64_t i = base + (int64_t)j * kMergeThreads + threadIdx.x;
      x[j] = i < nkeys ? keys[i] : ~0ull;
    }
    x[kMergeLoads] = kept;
    kept = wave_select(x, k);
  }
  if (lane < kFusedK) lists[wave * kFusedK + lane] = kept;
  __syncthreads();
  if (wave != 0) return;
  uint64_t y[W * kFusedK / 64];
#pragma unroll
  for (int j = 0; j < W * kFusedK / 64; ++j) y[j] = lists[64 * j + lane];
  const uint64_t best = wave_select(y, k);
  for (int i = lane; i < top_k; i += 64) store_result(ids, scores, i, i == lane && lane < k ? best : ~0ull);
}

// Workgroups of the fused scan for n rows (each writes k keys).
inline int64_t fused_wgs(int64_t n, int waves) { return div_up(n, (int64_t)kFusedRowsWave * waves); }

// Scan workgroup size for n rows: 8 or 10 waves (128 or 160 rows), whichever
// leaves the fewest rows on the busiest CU of a one-round grid (78,125 rows
// on 256 CUs: 611 workgroups put three, 384 rows, on 99 CUs; 489 of 160 rows
// at most two, 320 rows -- 19.9 against 20.2 us per query); ties keep 8.
int fused_waves(int64_t n) {
  const int64_t cus = attn::device_cus();
  int best = kFusedWavesMin;
  int64_t best_rows = 0;
  for (int w : {kFusedWavesMin, kFusedWavesMax}) {
    const int64_t rows = div_up(fused_wgs(n, w), cus) * kFusedRowsWave * w;
    if (w == kFusedWavesMin || rows < best_rows) {
      best = w;
      best_rows = rows;
    }
  }
  return best;
}

template <typename T>
void launch_scan_topk(int waves, dim3 grid, hipStream_t s, const void* rows, int64_t stride, int n, int d,
                      const float* q, float* sims, int mode, int k, uint64_t* keys) {
  const T* r = static_cast<const T*>(rows);
  if (waves == kFusedWavesMax)
    hipLaunchKernelGGL((scan_topk_kernel<T, kFusedWavesMax>), grid, dim3(64 * kFusedWavesMax), 0, s, r, stride, n, d,
                       q, sims, mode, k, keys);
  else
    hipLaunchKernelGGL((scan_topk_kernel<T, kFusedWavesMin>), grid, dim3(64 * kFusedWavesMin), 0, s, r, stride, n, d,
                       q, sims, mode, k, keys);
}

// Keys written by pass p, and the number of passes, for n inputs and top k.
struct Plan {
  int passes;
  int64_t max_keys;  // largest intermediate key array
};

// Keys consumed per group (a wave on the small-k path, a block otherwise).
inline int group_keys(int k) { return k <= 64 ? kWaveKeys : kSortN; }

Plan plan_for(int n, int k) {
  Plan p{0, 0};
  int64_t cur = n;
  const int per = group_keys(k);
  do {
    const int64_t blocks = div_up(cur, (int64_t)per);
    cur = blocks * (int64_t)k;
    if (cur > p.max_keys) p.max_keys = cur;
    ++p.passes;
    if (blocks == 1) break;
  } while (true);
  return p;
}

template <typename T>
int scan_launch(const void* rows, int64_t stride, int n, int d, const float* q, float* sims, int mode,
                hipStream_t s) {
  // One 16-lane group per row, at most 4,096 workgroups (groups then loop).
  const int blocks = (int)std::min<int64_t>(div_up((int64_t)n * 16, (int64_t)kScanThreads), 4096);
  hipLaunchKernelGGL(cosine_scan_kernel<T>, dim3(blocks), dim3(kScanThreads), 0, s, static_cast<const T*>(rows),
                     stride, n, d, q, sims, mode);
  return check_launch("index query scan");
}

}  // namespace
}  // namespace index
}  // namespace kessie

using namespace kessie;
using namespace kessie::index;

extern "C" size_t kessie_index_query_workspace_bytes(int num_chunks, int top_k) {
  if (num_chunks <= 0 || top_k <= 0) return 0;
  const int k = top_k < num_chunks ? top_k : num_chunks;
  if (k <= kFusedK)  // sized for the smaller workgroups (the most lists)
    return (size_t)((fused_wgs(num_chunks, kFusedWavesMin) * k * sizeof(uint64_t) + 255) / 256 * 256);
  const Plan p = plan_for(num_chunks, k);
  // Two ping-pong key arrays.
  return 2 * (size_t)((p.max_keys * sizeof(uint64_t) + 255) / 256 * 256);
}

extern "C" int kessie_index_query(const void* index_embeds, int64_t row_stride, int num_chunks, int embed_dim,
                                  int dtype, int norm_mode, const float* query_embed, float* similarities, int top_k,
                                  int32_t* top_ids, float* top_scores, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_chunks >= 0 && embed_dim > 0 && embed_dim <= 1024 && top_k >= 0, KESSIE_ERR_INVALID,
                 "index query: num_chunks %d, embed_dim %d (1..1024), top_k %d", num_chunks, embed_dim, top_k);
  KESSIE_REQUIRE(top_k <= kMaxTopK, KESSIE_ERR_UNSUPPORTED, "index query: top_k %d above %d", top_k, kMaxTopK);
  if (num_chunks == 0 && top_k == 0) return KESSIE_OK;
  KESSIE_REQUIRE(num_chunks == 0 || (query_embed && similarities), KESSIE_ERR_INVALID,
                 "index query: null query or similarities");
  KESSIE_REQUIRE(num_chunks == 0 || index_embeds, KESSIE_ERR_INVALID, "index query: null index");
  KESSIE_REQUIRE(top_k == 0 || top_ids || top_scores, KESSIE_ERR_INVALID, "index query: no top-k output");
  const int esz = dtype_size(dtype);
  KESSIE_REQUIRE(esz > 0, KESSIE_ERR_UNSUPPORTED, "index query: dtype %d", dtype);
  KESSIE_REQUIRE((embed_dim * esz) % 16 == 0 && (row_stride * esz) % 16 == 0 && aligned16(index_embeds),
                 KESSIE_ERR_UNSUPPORTED, "index query: rows must be 16-byte aligned multiples of 16 bytes");
  KESSIE_REQUIRE(row_stride >= embed_dim, KESSIE_ERR_INVALID, "index query: row_stride %lld < embed_dim %d",
                 (long long)row_stride, embed_dim);
  KESSIE_REQUIRE(norm_mode >= 0 && norm_mode <= 2, KESSIE_ERR_INVALID, "index query: norm_mode %d", norm_mode);
  const hipStream_t s = as_stream(stream);
  const int kk = top_k < num_chunks ? top_k : num_chunks;
  if (kk > 0 && kk <= kFusedK) {
    // The scan keeps each workgroup's top-k, one workgroup merges them.
    const size_t need = kessie_index_query_workspace_bytes(num_chunks, kk);
    KESSIE_REQUIRE(workspace && workspace_bytes >= need, KESSIE_ERR_WORKSPACE,
                   "index query: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
    KESSIE_REQUIRE(aligned16(workspace), KESSIE_ERR_INVALID, "index query: workspace not 16-byte aligned");
    uint64_t* keys = static_cast<uint64_t*>(workspace);
    const int waves = fused_waves(num_chunks);
    const int64_t wgs = fused_wgs(num_chunks, waves);
    const dim3 grid((unsigned)wgs);
    switch (dtype) {
      case KESSIE_DTYPE_F32:
        launch_scan_topk<float>(waves, grid, s, index_embeds, row_stride, num_chunks, embed_dim, query_embed,
                                similarities, norm_mode, kk, keys);
        break;
      case KESSIE_DTYPE_BF16:
        launch_scan_topk<bf16_t>(waves, grid, s, index_embeds, row_stride, num_chunks, embed_dim, query_embed,
                                 similarities, norm_mode, kk, keys);
        break;
      default:
        launch_scan_topk<f16_t>(waves, grid, s, index_embeds, row_stride, num_chunks, embed_dim, query_embed,
                                similarities, norm_mode, kk, keys);
    }
    if (check_launch("index query scan + top-k") != KESSIE_OK) return last_status();
    hipLaunchKernelGGL(topk_merge_kernel, dim3(1), dim3(kMergeThreads), 0, s, keys, wgs * kk, kk, top_ids,
                       top_scores, top_k);
    return check_launch("index query top-k merge");
  }
  if (num_chunks > 0) {
    int st = KESSIE_OK;
    switch (dtype) {
      case KESSIE_DTYPE_F32: st = scan_launch<float>(index_embeds, row_stride, num_chunks, embed_dim, query_embed, similarities, norm_mode, s); break;
      case KESSIE_DTYPE_BF16: st = scan_launch<bf16_t>(index_embeds, row_stride, num_chunks, embed_dim, query_embed, similarities, norm_mode, s); break;
      case KESSIE_DTYPE_F16: st = scan_launch<f16_t>(index_embeds, row_stride, num_chunks, embed_dim, query_embed, similarities, norm_mode, s); break;
      default: st = KESSIE_ERR_UNSUPPORTED; set_error(st, "index query: dtype %d", dtype);
    }
    if (st != KESSIE_OK) return st;
  }
  if (top_k == 0) return KESSIE_OK;
  const int k = top_k < num_chunks ? top_k : num_chunks;
  if (k == 0) {  // nothing to rank: -1 / -inf
    hipLaunchKernelGGL(topk_unpack_kernel, dim3(div_up(top_k, 256)), dim3(256), 0, s, nullptr, top_k, 0, top_ids,
                       top_scores);
    return check_launch("index query top-k");
  }
  const size_t need = kessie_index_query_workspace_bytes(num_chunks, k);
  KESSIE_REQUIRE(workspace && workspace_bytes >= need, KESSIE_ERR_WORKSPACE,
                 "index query: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
  KESSIE_REQUIRE(aligned16(workspace), KESSIE_ERR_INVALID, "index query: workspace not 16-byte aligned");
  const Plan plan = plan_for(num_chunks, k);
  const size_t half = need / 2;
  uint64_t* buf[2] = {static_cast<uint64_t*>(workspace),
                      reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + half)};
  int64_t cur = num_chunks;
  const uint64_t* in = nullptr;
  const int per = group_keys(k);
  for (int pass = 0; pass < plan.passes; ++pass) {
    const int groups = (int)div_up(cur, (int64_t)per);
    uint64_t* out = buf[pass & 1];
    if (k <= 64) {
      const int blocks = div_up(groups, kWaveThreads / 64);
      const bool last = pass + 1 == plan.passes;
      hipLaunchKernelGGL(topk_wave_kernel, dim3(blocks), dim3(kWaveThreads), 0, s, similarities, in, (int)cur, k,
                         out, last ? top_ids : nullptr, last ? top_scores : nullptr, last ? top_k : 0);
      if (last) return check_launch("index query top-k");
    } else {
      hipLaunchKernelGGL(topk_pass_kernel, dim3(groups), dim3(kSortThreads), 0, s, similarities, in, (int)cur, k,
                         out);
    }
    in = out;
    cur = (int64_t)groups * k;
  }
  hipLaunchKernelGGL(topk_unpack_kernel, dim3(div_up(top_k, 256)), dim3(256), 0, s, in, top_k, k, top_ids,
                     top_scores);
  return check_launch("index query top-k");
}
