// Paged-KV management for gfx950: insert (optionally RoPE-remapping K),
// threshold eviction, score eviction, page-table compaction, valid-page lists
// and the page gather.
//
// Reference semantics:
//   threshold evict  valid==1 && pos < thr -> valid=0     (kessie_kernels_v2.hip:393-407)
//   insert           page = target[t/P], slot t%P; ids outside [0,pages)
//                    skipped; slot-0 token sets valid/position
//                                                          (kessie_kernels_v2.hip:414-456)
//   free-list order  evicted ids appended ascending        (kessie_hip_kernels.py:534-538)
//   gather order     valid ids ascending                   (kessie_hip_kernels.py:558-564)
// Every list this file produces is ordered by a prefix sum, never by atomics:
// count per block -> exclusive scan of the block counts -> each block writes
// its survivors at its offset in element order.  Atomics appear only in
// counters whose value does not depend on order (histograms, the legacy
// evict count).
#include <climits>
#include <cstdlib>

#include "common.h"

namespace kessie {
namespace pages {

constexpr int kThreads = 256;
constexpr int kItems = 8;                      // consecutive elements per thread
constexpr int kChunk = kThreads * kItems;      // elements per block in compaction
constexpr int kWaves = kThreads / 64;

// Exclusive scan of one int per thread across a 256-thread block.  `sm` needs
// kWaves + 1 ints.  Returns the thread's exclusive prefix; *total = block sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* total, int* sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sm[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int s = 0;
    for (int w = 0; w < kWaves; ++w) {
      const int t = sm[w];
      sm[w] = s;
      s += t;
    }
    sm[kWaves] = s;
  }
  __syncthreads();
  const int res = x - v + sm[wave];
  *total = sm[kWaves];
  __syncthreads();
  return res;
}

// ---------------------------------------------------------------------------
// Predicates for ordered compaction over page ids
// ---------------------------------------------------------------------------
enum PredKind : int {
  kPredValid = 0,      // valid[i] == 1
  kPredFreed = 1,      // (valid==1 && pos<thr) || (allocated && allocated[i] && valid!=1)
  kPredScoreEvict = 2  // valid==1 && key(i) <= threshold key (threshold in workspace)
};

struct PredArgs {
  int kind;
  const int8_t* valid;
  const int32_t* positions;
  const int8_t* allocated;
  int thr;
  const float* scores;
  const unsigned long long* key_thr;  // device, for kPredScoreEvict
  const int* k_dev;                   // device: number to evict (0 -> none)
};

__device__ __forceinline__ unsigned long long score_key(float s, int id) {
  if (s == 0.0f) s = 0.0f;  // -0 == +0
  const uint32_t bits = __float_as_uint(s);
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return ((unsigned long long)ord << 32) | (uint32_t)id;
}

__device__ __forceinline__ bool pred_eval(const PredArgs& a, int i) {
  switch (a.kind) {
    case kPredValid:
      return a.valid[i] == 1;
    case kPredFreed: {
      const bool v = a.valid[i] == 1;
      if (v && a.positions[i] < a.thr) return true;
      return a.allocated != nullptr && a.allocated[i] != 0 && !v;
    }
    case kPredScoreEvict:
      return a.valid[i] == 1 && *a.k_dev > 0 && score_key(a.scores[i], i) <= *a.key_thr;
  }
  return false;
}

__global__ __launch_bounds__(kThreads) void compact_count_kernel(PredArgs a, int n, int* block_counts) {
  __shared__ int sm[kWaves + 1];
  const int base = blockIdx.x * kChunk + threadIdx.x * kItems;
  int c = 0;
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    const int i = base + e;
    if (i < n && pred_eval(a, i)) ++c;
  }
  int total;
  block_exclusive_scan(c, &total, sm);
  if (threadIdx.x == 0) block_counts[blockIdx.x] = total;
}

// Exclusive scan of `n` ints by one 256-thread block (any n), total to *total.
__global__ __launch_bounds__(kThreads) void scan_counts_kernel(const int* counts, int n, int* offsets, int* total) {
  __shared__ int sm[kWaves + 1];
  int carry = 0;
  for (int base = 0; base < n; base += kThreads) {
    const int i = base + threadIdx.x;
    const int v = i < n ? counts[i] : 0;
    int tot;
    const int ex = block_exclusive_scan(v, &tot, sm);
    if (i < n) offsets[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0 && total) *total = carry;
}

// Writes the ids satisfying the predicate in element order; when clear_valid
// (clear_alloc) is set, each listed page also gets valid = 0 (allocated = 0):
// only the thread that evaluated a page's predicate touches its flags.
__global__ __launch_bounds__(kThreads) void compact_write_kernel(PredArgs a, int n, const int* block_offsets,
                                                                 int32_t* out, int8_t* clear_valid,
                                                                 int8_t* clear_alloc) {
  __shared__ int sm[kWaves + 1];
  const int base = blockIdx.x * kChunk + threadIdx.x * kItems;
  unsigned flags = 0;
  int c = 0;
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    const int i = base + e;
    if (i < n && pred_eval(a, i)) {
      flags |= 1u << e;
      ++c;
    }
  }
  int total;
  int pos = block_exclusive_scan(c, &total, sm) + block_offsets[blockIdx.x];
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    if (!(flags & (1u << e))) continue;
    out[pos++] = base + e;
    if (clear_valid) clear_valid[base + e] = 0;
    if (clear_alloc) clear_alloc[base + e] = 0;
  }
}

// ---------------------------------------------------------------------------
// Radix select: the key of rank k-1 among valid pages.  Keys are 64-bit
// (ordered score << 32 | page id), so they are unique and the k smallest form
// exactly the set the total order (score, id) puts first.  Five launches, no
// host round trip:
//   clear     zero the global 4096-bin histogram and counters (a fill kernel:
//             graph-capture safe);
//   hist      many workgroups histogram the top 12 bits of the ordered score
//             of valid pages in LDS and add them to the global histogram;
//   bucket    one workgroup derives k from the valid count and picks the bin
//             holding rank k-1 and the rank inside it;
//   collect   many workgroups append that bin's keys (low 20 score bits, page
//             id) to a candidate list, one atomic per workgroup tile;
//   resolve   one workgroup resolves the low 20 bits (two 10-bit passes) and,
//             when several candidates share that score, the page id (11+11+10
//             bits) on the candidates -- copied to LDS when they fit, read in
//             place otherwise (heavily tied scores).
// Histogram and list atomics only count; the result does not depend on their
// order.  (Folding bucket and resolve into the last workgroup of hist and
// collect measured slower: 46 us against 26 us for 65,536 pages.)
// ---------------------------------------------------------------------------
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelCap = 12288;   // candidate keys held in LDS
constexpr int kSelBins = 4096;
constexpr int kSelPer = 4;       // keys per thread per hist/collect tile
constexpr int kSelTile = kSelThreads * kSelPer;
constexpr int kSelMaxGrid = 1024;

struct SelectOut {
  unsigned long long key_thr;  // largest evicted key
  int k;                       // number evicted
  int n_valid;
};

struct SelScratch {
  int hist[kSelBins];
  int n_valid;
  int ncand;
  int k;      // keys to evict (0: nothing to resolve)
  int rank;   // rank of key k-1 inside bin `top`
  uint32_t top;
};

__device__ __forceinline__ uint32_t ordered_score(float s) {
  if (s == 0.0f) s = 0.0f;  // -0 == +0
  const uint32_t bits = __float_as_uint(s);
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

// Exclusive scan of one int per thread across the 1024-thread block.
__device__ __forceinline__ int sel_block_scan(int v, int* sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sm[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int w = 0; w < kSelWaves; ++w) {
      const int t = sm[w];
      sm[w] = acc;
      acc += t;
    }
    sm[kSelWaves] = acc;
  }
  __syncthreads();
  const int res = x - v + sm[wave];
  __syncthreads();
  return res;
}

// The bin of `bins[0..nb)` (nb = 1024, 2048 or 4096) whose cumulative count
// range holds `rank`, and the rank within it; every thread must call.
__device__ __forceinline__ void sel_pick(const int* bins, int nb, int rank, int* sm, int* s_digit, int* s_rank) {
  const int per = nb / kSelThreads;
  const int first = threadIdx.x * per;
  int c[4] = {0, 0, 0, 0};
  int sum = 0;
  for (int j = 0; j < per; ++j) {
    c[j] = bins[first + j];
    sum += c[j];
  }
  const int excl = sel_block_scan(sum, sm);
  if (rank >= excl && rank < excl + sum) {
    int r = rank - excl, d = first;
    for (int j = 0; j < per; ++j) {
      if (r < c[j]) break;
      r -= c[j];
      ++d;
    }
    *s_digit = d;
    *s_rank = r;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kThreads) void sel_clear_kernel(SelScratch* ss) {
  for (int e = threadIdx.x; e < kSelBins; e += kThreads) ss->hist[e] = 0;
  if (threadIdx.x == 0) {
    ss->n_valid = 0;
    ss->ncand = 0;
    ss->k = 0;
    ss->rank = 0;
    ss->top = 0;
  }
}

__global__ __launch_bounds__(kSelThreads) void sel_hist_kernel(const float* __restrict__ scores,
                                                               const int8_t* __restrict__ valid, int n,
                                                               SelScratch* ss) {
  __shared__ int hist[kSelBins];
  for (int e = threadIdx.x; e < kSelBins; e += kSelThreads) hist[e] = 0;
  __syncthreads();
  int c = 0;
  for (int64_t t0 = (int64_t)blockIdx.x * kSelTile; t0 < n; t0 += (int64_t)gridDim.x * kSelTile) {
    float sc[kSelPer];
    int8_t vv[kSelPer];
#pragma unroll
    for (int j = 0; j < kSelPer; ++j) {
      const int64_t i = t0 + j * kSelThreads + threadIdx.x;
      vv[j] = i < n ? valid[i] : (int8_t)0;
      sc[j] = i < n ? scores[i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kSelPer; ++j) {
      if (vv[j] != 1) continue;
      ++c;
      atomicAdd(&hist[ordered_score(sc[j]) >> 20], 1);
    }
  }
  for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
  if ((threadIdx.x & 63) == 0 && c) atomicAdd(&ss->n_valid, c);
  __syncthreads();
  for (int e = threadIdx.x; e < kSelBins; e += kSelThreads)
    if (hist[e]) atomicAdd(&ss->hist[e], hist[e]);
}

__global__ __launch_bounds__(kSelThreads) void sel_bucket_kernel(SelScratch* ss, int k_evict, float evict_fraction,
                                                                 SelectOut* out) {
  __shared__ int hist[kSelBins];
  __shared__ int sm[kSelWaves + 1];
  __shared__ int s_digit, s_rank;
  for (int e = threadIdx.x; e < kSelBins; e += kSelThreads) hist[e] = ss->hist[e];
  const int n_valid = ss->n_valid;
  long long k;
  if (k_evict >= 0) {
    k = min(k_evict, n_valid);
  } else {
    k = (long long)floor((double)evict_fraction * (double)n_valid);
    if (k < 0) k = 0;
    if (k > n_valid) k = n_valid;
  }
  __syncthreads();
  if (k == 0) {
    if (threadIdx.x == 0) {
      out->key_thr = 0;
      out->k = 0;
      out->n_valid = n_valid;
      ss->k = 0;
    }
    return;
  }
  sel_pick(hist, kSelBins, (int)k - 1, sm, &s_digit, &s_rank);
  if (threadIdx.x == 0) {
    ss->k = (int)k;
    ss->top = (uint32_t)s_digit;
    ss->rank = s_rank;
    out->k = (int)k;
    out->n_valid = n_valid;
  }
}

__global__ __launch_bounds__(kSelThreads) void sel_collect_kernel(const float* __restrict__ scores,
                                                                  const int8_t* __restrict__ valid, int n,
                                                                  SelScratch* ss, uint32_t* __restrict__ cand_s,
                                                                  uint32_t* __restrict__ cand_i) {
  __shared__ int sm[kSelWaves + 1];
  __shared__ int s_base;
  if (ss->k == 0) return;  // written by the previous launch; uniform
  const int tid = threadIdx.x;
  const uint32_t top = ss->top;
  for (int64_t t0 = (int64_t)blockIdx.x * kSelTile; t0 < n; t0 += (int64_t)gridDim.x * kSelTile) {
    uint32_t ks[kSelPer];
    int cnt = 0, mbits = 0;
#pragma unroll
    for (int j = 0; j < kSelPer; ++j) {
      const int64_t i = t0 + j * kSelThreads + tid;
      ks[j] = 0;
      if (i < n && valid[i] == 1) {
        ks[j] = ordered_score(scores[i]);
        if ((ks[j] >> 20) == top) {
          mbits |= 1 << j;
          ++cnt;
        }
      }
    }
    int pos = sel_block_scan(cnt, sm);
    if (tid == 0 && sm[kSelWaves] > 0) s_base = atomicAdd(&ss->ncand, sm[kSelWaves]);
    __syncthreads();
    pos += s_base;
#pragma unroll
    for (int j = 0; j < kSelPer; ++j) {
      if (!((mbits >> j) & 1)) continue;
      cand_s[pos] = ks[j] & 0xFFFFFu;
      cand_i[pos] = (uint32_t)(t0 + j * kSelThreads + tid);
      ++pos;
    }
    __syncthreads();  // s_base and sm are reused by the next tile
  }
}

__global__ __launch_bounds__(kSelThreads) void sel_resolve_kernel(const SelScratch* ss, const uint32_t* g_cand_s,
                                                                  const uint32_t* g_cand_i, SelectOut* out) {
  __shared__ int hist[2048];
  __shared__ uint32_t lds_s[kSelCap];  // low 20 bits of the ordered score
  __shared__ uint32_t lds_i[kSelCap];  // page id
  __shared__ int sm[kSelWaves + 1];
  __shared__ int s_digit, s_rank, s_id;
  if (ss->k == 0) return;
  const int tid = threadIdx.x;
  const int nc = ss->ncand;
  const uint32_t top = ss->top;
  int rank = ss->rank;
  const uint32_t* cs = g_cand_s;
  const uint32_t* ci = g_cand_i;
  if (nc <= kSelCap) {
    for (int q = tid; q < nc; q += kSelThreads) {
      lds_s[q] = g_cand_s[q];
      lds_i[q] = g_cand_i[q];
    }
    cs = lds_s;
    ci = lds_i;
  }
  __syncthreads();
  auto cand_score = [&](int q) { return cs[q]; };
  auto cand_id = [&](int q) { return ci[q]; };
  uint32_t low = 0;
  int ties = 0;
  for (int pass = 0; pass < 2; ++pass) {
    const int sh = 10 - 10 * pass;
    for (int e = tid; e < 1024; e += kSelThreads) hist[e] = 0;
    __syncthreads();
    for (int q = tid; q < nc; q += kSelThreads) {
      const uint32_t v = cand_score(q);
      if (pass == 0 || (v >> 10) == low) atomicAdd(&hist[(v >> sh) & 1023u], 1);
    }
    __syncthreads();
    sel_pick(hist, 1024, rank, sm, &s_digit, &s_rank);
    low = (low << 10) | (uint32_t)s_digit;
    rank = s_rank;
    ties = hist[s_digit];
    __syncthreads();
  }
  const uint32_t score = (top << 20) | low;
  uint32_t idp = 0;
  if (ties == 1) {
    for (int q = tid; q < nc; q += kSelThreads)
      if (cand_score(q) == low) s_id = (int)cand_id(q);
    __syncthreads();
    idp = (uint32_t)s_id;
  } else {
    for (int pass = 0; pass < 3; ++pass) {
      const int width = pass < 2 ? 11 : 10;
      const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      for (int e = tid; e < 2048; e += kSelThreads) hist[e] = 0;
      __syncthreads();
      for (int q = tid; q < nc; q += kSelThreads) {
        if (cand_score(q) != low) continue;
        const uint32_t id = cand_id(q);
        if (pass == 0 || (id >> (sh + width)) == idp) atomicAdd(&hist[(id >> sh) & ((1u << width) - 1u)], 1);
      }
      __syncthreads();
      sel_pick(hist, 2048, rank, sm, &s_digit, &s_rank);
      idp = (idp << width) | (uint32_t)s_digit;
      rank = s_rank;
      __syncthreads();
    }
  }
  if (tid == 0) out->key_thr = ((unsigned long long)score << 32) | idp;
}

// ---------------------------------------------------------------------------
// Table compaction
// ---------------------------------------------------------------------------
// One block per table row: survivors keep logical order; the rest of the row
// is filled with -1; new_lens[row] = survivors.
__global__ __launch_bounds__(kThreads) void compact_rows_kernel(const int32_t* tables, const int32_t* lens,
                                                                const int8_t* valid, int32_t* new_tables,
                                                                int32_t* new_lens, int table_stride, int num_pages) {
  __shared__ int sm[kWaves + 1];
  const int row = blockIdx.x;
  const int32_t* in = tables + (int64_t)row * table_stride;
  int32_t* outr = new_tables + (int64_t)row * table_stride;
  const int len = min(max(lens[row], 0), table_stride);
  int carry = 0;
  for (int base = 0; base < table_stride; base += kChunk) {
    const int first = base + threadIdx.x * kItems;
    unsigned flags = 0;
    int ids[kItems];
    int c = 0;
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
      const int j = first + e;
      ids[e] = -1;
      if (j < len) {
        const int id = in[j];
        ids[e] = id;
        if (id >= 0 && id < num_pages && valid[id] == 1) {
          flags |= 1u << e;
          ++c;
        }
      }
    }
    int total;
    int pos = carry + block_exclusive_scan(c, &total, sm);
#pragma unroll
    for (int e = 0; e < kItems; ++e)
      if (flags & (1u << e)) outr[pos++] = ids[e];
    carry += total;
  }
  __syncthreads();
  for (int j = carry + threadIdx.x; j < table_stride; j += kThreads) outr[j] = -1;
  if (threadIdx.x == 0) new_lens[row] = carry;
}

// gather_idx[row_off[row] + j] = new_tables[row][j], j < new_lens[row].
__global__ __launch_bounds__(kThreads) void flatten_rows_kernel(const int32_t* new_tables, const int32_t* new_lens,
                                                                const int* row_off, int table_stride,
                                                                int32_t* gather_idx) {
  const int row = blockIdx.x;
  const int n = new_lens[row];
  const int off = row_off[row];
  for (int j = threadIdx.x; j < n; j += kThreads) gather_idx[off + j] = new_tables[(int64_t)row * table_stride + j];
}

// ---------------------------------------------------------------------------
// Threshold evict (reference launcher semantics)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void threshold_evict_kernel(int8_t* valid, const int32_t* positions,
                                                                   int32_t* count, int thr, int n) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  int hit = 0;
  if (i < n && valid[i] == 1 && positions[i] < thr) {
    valid[i] = 0;
    hit = 1;
  }
  // One atomic per wave; the count does not depend on order.
  for (int o = 32; o >= 1; o >>= 1) hit += __shfl_xor(hit, o, 64);
  if ((threadIdx.x & 63) == 0 && hit) atomicAdd(count, hit);
}

// ---------------------------------------------------------------------------
// Gather: whole-page byte copies.  Each workgroup copies one 4 KiB tile of one
// page slot, one non-temporal 16-byte load and store per lane: a 64 KiB page is
// spread over 16 workgroups.  (Measured on 49,152 random 64 KiB pages: 0.99 ms
// against 1.17-1.21 ms for one workgroup per page at 1-8 chunks per lane.)
// The grid covers the slot capacity n while only *count_dev slots are live;
// slots are taken from kGatherRegions interleaved regions of [0, n), so the
// workgroups of dead slots (the tail of the capacity) are spread through the
// dispatch order instead of forming a tail of their own (49,152 live of 65,536:
// 1.03 ms against 1.07 ms; all live: within 0.5 %).
// ---------------------------------------------------------------------------
constexpr int kGatherThreads = 256;
constexpr int kGatherRegions = 32;

__global__ __launch_bounds__(kGatherThreads) void gather_kernel(const u32x4* __restrict__ src, int64_t page_vecs,
                                                                int tiles_per_page, int per_region,
                                                                const int32_t* __restrict__ idx,
                                                                const int32_t* __restrict__ count_dev, int n,
                                                                int num_pages, u32x4* __restrict__ dst) {
  const int j = blockIdx.x / tiles_per_page;
  const int i = (j % kGatherRegions) * per_region + j / kGatherRegions;  // slot
  if (i >= n) return;
  // The slot's page id and the device count are independent loads, issued
  // together: the data load then waits for one round trip, not two.
  const int pid = idx[i];
  const int cnt = count_dev ? min(n, *count_dev) : n;
  if (i >= cnt || pid < 0 || pid >= num_pages) return;
  const int64_t v = (int64_t)(blockIdx.x % tiles_per_page) * kGatherThreads + threadIdx.x;
  if (v < page_vecs)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + (int64_t)pid * page_vecs + v),
                                dst + (int64_t)i * page_vecs + v);
}

// ---------------------------------------------------------------------------
// Insert (optionally remapping K)
// ---------------------------------------------------------------------------
constexpr int kInsMaxHalf = 128;

template <typename T>
struct Vec16;
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

struct InsertArgs {
  void* pool;
  int64_t page_stride, tok_stride, kv_stride, head_stride;
  const void* new_k;
  const void* new_v;
  const int32_t* target_pages;
  int8_t* valid;
  int32_t* positions;
  int conv_pos;
  const int32_t* orig_pos;
  const int32_t* tgt_pos;
  const float* inv_freq;
  int T, H, D, page_size, num_pages;
};

// Element-wise insert, any layout/alignment: one thread per (token, head, d)
// for V and for K pairs.
template <typename T>
__global__ __launch_bounds__(kThreads) void insert_scalar_kernel(InsertArgs a) {
#pragma clang fp contract(off)
  const int half = a.D / 2;
  const bool remap = a.inv_freq != nullptr;
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t total = (int64_t)a.T * a.H * a.D;
  if (gid >= total) return;
  const int d = (int)(gid % a.D);
  const int64_t rem = gid / a.D;
  const int h = (int)(rem % a.H);
  const int t = (int)(rem / a.H);
  const int phys = a.target_pages[t / a.page_size];
  if (phys < 0 || phys >= a.num_pages) return;
  T* pool = static_cast<T*>(a.pool);
  const T* nk = static_cast<const T*>(a.new_k);
  const T* nv = static_cast<const T*>(a.new_v);
  const int64_t dst = (int64_t)phys * a.page_stride + (int64_t)(t % a.page_size) * a.tok_stride +
                      (int64_t)h * a.head_stride;
  const int64_t src = ((int64_t)t * a.H + h) * a.D;
  pool[dst + a.kv_stride + d] = nv[src + d];
  if (!remap) {
    pool[dst + d] = nk[src + d];
  } else if (d < half) {
    const float delta = (float)(a.tgt_pos[t] - a.orig_pos[t]);
    const float ang = delta * a.inv_freq[d];
    float s, c;
    sincosf(ang, &s, &c);
    const float x1 = to_f32(nk[src + d]);
    const float x2 = to_f32(nk[src + d + half]);
    const float u1 = x1 * c;
    const float u2 = x2 * s;
    const float w1 = x1 * s;
    const float w2 = x2 * c;
    pool[dst + d] = from_f32<T>(u1 - u2);
    pool[dst + d + half] = from_f32<T>(w1 + w2);
  }
  if (t % a.page_size == 0 && h == 0 && d == 0) {
    a.valid[phys] = 1;
    a.positions[phys] = a.conv_pos + t;
  }
}

// Vectorised insert: one token per workgroup.  Its H x half/N K chunk pairs
// (two 16-byte loads, rotated when remapping) and its H x D/N V chunks (one
// load) are separate items, one per lane (looping past 256 for large H x D);
// each lane issues its first item's non-temporal loads before the token's
// cos/sin are evaluated into LDS, so the trigonometry hides under the load
// latency.  (Measured, 65,536 bf16 tokens, 8 heads x 128, remap on: 93 us --
// the rate of a plain scatter of the same bytes into random pages -- against
// 103-106 us for 4-16-token workgroups with K and V pairs in one item.)
// kH / kChunks / kPage > 0 fix the head count, the chunk pairs per head and
// the page size at compile time (no runtime divisions in the index math, which
// with one item per lane would cost more than the copy); 0 reads them from the
// arguments.
template <typename T, int kH, int kChunks, int kPage>
__global__ __launch_bounds__(kThreads) void insert_vec_kernel(InsertArgs a) {
#pragma clang fp contract(off)
  typedef typename Vec16<T>::type V;
  constexpr int N = Vec16<T>::N;
  __shared__ float2 cs[kInsMaxHalf];
  const int H = kH > 0 ? kH : a.H;
  const int chunks = kChunks > 0 ? kChunks : a.D / 2 / N;  // chunk pairs per head
  const int page_size = kPage > 0 ? kPage : a.page_size;
  const int half = chunks * N;
  const int D = 2 * half;
  const bool remap = a.inv_freq != nullptr;
  const int t = blockIdx.x;
  const int kp = H * chunks;              // K pair items
  const int items = kp + 2 * kp;          // + V chunk items (H x D/N)
  const int nthr = blockDim.x;
  const int phys = a.target_pages[t / page_size];
  const bool ok = phys >= 0 && phys < a.num_pages;  // uniform
  T* pool = static_cast<T*>(a.pool);
  const T* nk = static_cast<const T*>(a.new_k);
  const T* nv = static_cast<const T*>(a.new_v);
  const int64_t dst_row = (int64_t)phys * a.page_stride + (int64_t)(t % page_size) * a.tok_stride;

  auto load = [&](int i, V& x1, V& x2) {
    if (i < kp) {
      const int h = i / chunks, c = i - h * chunks;
      const int64_t src = ((int64_t)t * H + h) * D + c * N;
      x1 = __builtin_nontemporal_load(reinterpret_cast<const V*>(nk + src));
      x2 = __builtin_nontemporal_load(reinterpret_cast<const V*>(nk + src + half));
    } else {
      const int q = i - kp;
      const int h = q / (2 * chunks), c = q - h * 2 * chunks;
      x1 = __builtin_nontemporal_load(reinterpret_cast<const V*>(nv + ((int64_t)t * H + h) * D + c * N));
    }
  };
  auto store = [&](int i, const V& x1, const V& x2) {
    if (i < kp) {
      const int h = i / chunks, c = i - h * chunks;
      V y1 = x1, y2 = x2;
      if (remap) {
        const float2* csr = cs + c * N;
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const float2 q = csr[e];
          const float v1 = to_f32(x1[e]);
          const float v2 = to_f32(x2[e]);
          const float u1 = v1 * q.x;
          const float u2 = v2 * q.y;
          const float w1 = v1 * q.y;
          const float w2 = v2 * q.x;
          y1[e] = from_f32<T>(u1 - u2);
          y2[e] = from_f32<T>(w1 + w2);
        }
      }
      T* d = pool + dst_row + (int64_t)h * a.head_stride + c * N;
      __builtin_nontemporal_store(y1, reinterpret_cast<V*>(d));
      __builtin_nontemporal_store(y2, reinterpret_cast<V*>(d + half));
    } else {
      const int q = i - kp;
      const int h = q / (2 * chunks), c = q - h * 2 * chunks;
      T* d = pool + dst_row + a.kv_stride + (int64_t)h * a.head_stride + c * N;
      __builtin_nontemporal_store(x1, reinterpret_cast<V*>(d));
    }
  };

  // The staging rows are always in bounds: load them without waiting for the
  // page id (a load that waited on it would add a round trip per token).
  V x1, x2;
  const int i0 = threadIdx.x;
  if (i0 < items) load(i0, x1, x2);
  if (remap) {
    const float delta = (float)(a.tgt_pos[t] - a.orig_pos[t]);
    for (int j = threadIdx.x; j < half; j += nthr) {
      const float ang = delta * a.inv_freq[j];
      float sn, cn;
      sincosf(ang, &sn, &cn);
      cs[j] = make_float2(cn, sn);
    }
    __syncthreads();
  }
  if (!ok) return;
  if (i0 < items) store(i0, x1, x2);
  for (int i = i0 + nthr; i < items; i += nthr) {
    V y1, y2;
    load(i, y1, y2);
    store(i, y1, y2);
  }
  if (threadIdx.x == 0 && t % page_size == 0) {
    a.valid[phys] = 1;
    a.positions[phys] = a.conv_pos + t;
  }
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
int num_blocks(int n) { return div_up(max(n, 1), kChunk); }

struct Workspace {
  SelectOut* sel;
  int* counts;
  int* offsets;
  int* rows;  // per-row offsets (table compaction)
  SelScratch* ss;
  uint32_t* cand_s;  // select candidates (n each)
  uint32_t* cand_i;
};

constexpr size_t round256(size_t b) { return (b + 255) / 256 * 256; }

size_t workspace_bytes(int n) {
  const size_t nb = (size_t)num_blocks(n);
  size_t b = 256;                                   // SelectOut + misc
  b += round256(nb * sizeof(int));                  // counts
  b += round256(nb * sizeof(int));                  // offsets
  b += round256(((size_t)n + 1) * sizeof(int));     // row offsets
  b += round256(sizeof(SelScratch));                // select histogram + counters
  b += 2 * round256((size_t)n * sizeof(uint32_t));  // select candidates
  return b;
}

Workspace carve(void* ws, int n) {
  Workspace w;
  char* c = static_cast<char*>(ws);
  const size_t nb = (size_t)num_blocks(n);
  w.sel = reinterpret_cast<SelectOut*>(c);
  c += 256;
  w.counts = reinterpret_cast<int*>(c);
  c += round256(nb * sizeof(int));
  w.offsets = reinterpret_cast<int*>(c);
  c += round256(nb * sizeof(int));
  w.rows = reinterpret_cast<int*>(c);
  c += round256(((size_t)n + 1) * sizeof(int));
  w.ss = reinterpret_cast<SelScratch*>(c);
  c += round256(sizeof(SelScratch));
  w.cand_s = reinterpret_cast<uint32_t*>(c);
  c += round256((size_t)n * sizeof(uint32_t));
  w.cand_i = reinterpret_cast<uint32_t*>(c);
  return w;
}

// Ordered compaction of page ids satisfying `a` into out[], count to *count.
int ordered_compact(const PredArgs& a, int n, int32_t* out, int32_t* count, Workspace& w, hipStream_t s,
                    int8_t* clear_valid = nullptr, int8_t* clear_alloc = nullptr) {
  const int nb = num_blocks(n);
  hipLaunchKernelGGL(compact_count_kernel, dim3(nb), dim3(kThreads), 0, s, a, n, w.counts);
  hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(kThreads), 0, s, w.counts, nb, w.offsets, count);
  hipLaunchKernelGGL(compact_write_kernel, dim3(nb), dim3(kThreads), 0, s, a, n, w.offsets, out, clear_valid,
                     clear_alloc);
  return check_launch("ordered compaction");
}

int check_ws(void* ws, size_t bytes, int n, const char* what) {
  const size_t need = workspace_bytes(n);
  KESSIE_REQUIRE(ws != nullptr && bytes >= need, KESSIE_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu",
                 what, need, bytes);
  KESSIE_REQUIRE(aligned16(ws), KESSIE_ERR_INVALID, "%s: workspace not 16-byte aligned", what);
  return KESSIE_OK;
}

template <typename T>
int launch_insert(InsertArgs& a, hipStream_t s) {
  constexpr int N = Vec16<T>::N;
  const int half = a.D / 2;
  const bool vec_ok = (a.D % 2 == 0) && (half % N == 0) && (half <= kInsMaxHalf) && aligned16(a.pool) &&
                      aligned16(a.new_k) && aligned16(a.new_v) && a.page_stride % N == 0 &&
                      a.tok_stride % N == 0 && a.head_stride % N == 0 && a.kv_stride % N == 0;
  if (vec_ok) {
    const int chunks = half / N;
    if (a.H == 8 && chunks == 8 && a.page_size == 16)  // 8 kv heads x 128, 16-token pages
      hipLaunchKernelGGL((insert_vec_kernel<T, 8, 8, 16>), dim3(a.T), dim3(3 * 8 * 8), 0, s, a);
    else
      hipLaunchKernelGGL((insert_vec_kernel<T, 0, 0, 0>), dim3(a.T), dim3(kThreads), 0, s, a);
  } else {
    const int64_t total = (int64_t)a.T * a.H * a.D;
    const int64_t grid = (total + kThreads - 1) / kThreads;
    KESSIE_REQUIRE(grid <= 0x7fffffff, KESSIE_ERR_UNSUPPORTED, "page insert: %lld elements exceed one launch",
                   (long long)total);
    hipLaunchKernelGGL(insert_scalar_kernel<T>, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
  }
  return check_launch("page insert");
}

int insert_dispatch(InsertArgs& a, int dtype, hipStream_t s) {
  KESSIE_REQUIRE(a.T >= 0 && a.H > 0 && a.D > 0 && a.page_size > 0 && a.num_pages >= 0, KESSIE_ERR_INVALID,
                 "page insert: bad sizes T=%d H=%d D=%d P=%d pages=%d", a.T, a.H, a.D, a.page_size, a.num_pages);
  if (a.T == 0 || a.num_pages == 0) return KESSIE_OK;
  KESSIE_REQUIRE(a.pool && a.new_k && a.new_v && a.target_pages && a.valid && a.positions, KESSIE_ERR_INVALID,
                 "page insert: null pointer");
  const bool any = a.orig_pos || a.tgt_pos || a.inv_freq;
  const bool all = a.orig_pos && a.tgt_pos && a.inv_freq;
  KESSIE_REQUIRE(!any || all, KESSIE_ERR_INVALID, "page insert: orig_pos, tgt_pos and inv_freq go together");
  KESSIE_REQUIRE(!all || a.D % 2 == 0, KESSIE_ERR_INVALID, "page insert: remap needs an even head_dim");
  KESSIE_REQUIRE(a.head_stride >= a.D && a.tok_stride >= (int64_t)a.H * a.head_stride, KESSIE_ERR_INVALID,
                 "page insert: strides overlap");
  switch (dtype) {
    case KESSIE_DTYPE_BF16: return launch_insert<bf16_t>(a, s);
    case KESSIE_DTYPE_F16: return launch_insert<f16_t>(a, s);
    case KESSIE_DTYPE_F32: return launch_insert<float>(a, s);
  }
  set_error(KESSIE_ERR_UNSUPPORTED, "page insert: dtype %d", dtype);
  return KESSIE_ERR_UNSUPPORTED;
}

}  // namespace pages
}  // namespace kessie

using namespace kessie;
using namespace kessie::pages;

extern "C" size_t kessie_page_workspace_bytes(int num_pages) { return pages::workspace_bytes(max(num_pages, 0)); }

extern "C" int kessie_page_insert_paged(void* kv_pool, int64_t page_stride, int64_t tok_stride, int64_t kv_stride,
                                        int64_t head_stride, const void* new_k, const void* new_v,
                                        const int32_t* target_pages, int8_t* page_valid, int32_t* page_positions,
                                        int conv_pos, const int32_t* orig_pos, const int32_t* tgt_pos,
                                        const float* inv_freq, int num_tokens, int num_heads, int head_dim,
                                        int page_size, int num_pages, int dtype, void* stream) {
  clear_error();
  InsertArgs a{kv_pool,  page_stride,    tok_stride, kv_stride, head_stride, new_k,     new_v,
               target_pages, page_valid, page_positions, conv_pos, orig_pos, tgt_pos, inv_freq,
               num_tokens, num_heads,     head_dim,   page_size, num_pages};
  return insert_dispatch(a, dtype, as_stream(stream));
}

extern "C" int kessie_page_evict_list(int8_t* page_valid, const int32_t* page_positions, int8_t* allocated,
                                      int evict_before_pos, int num_pages, int32_t* freed_list, int32_t* freed_count,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_pages >= 0, KESSIE_ERR_INVALID, "page evict: num_pages %d", num_pages);
  KESSIE_REQUIRE(page_valid && page_positions && freed_list && freed_count, KESSIE_ERR_INVALID,
                 "page evict: null pointer");
  int st = check_ws(workspace, workspace_bytes, num_pages, "page evict");
  if (st) return st;
  hipStream_t s = as_stream(stream);
  Workspace w = carve(workspace, num_pages);
  PredArgs a{kPredFreed, page_valid, page_positions, allocated, evict_before_pos, nullptr, nullptr, nullptr};
  return ordered_compact(a, num_pages, freed_list, freed_count, w, s, page_valid, allocated);
}

extern "C" int kessie_page_select_evict(const float* scores, int8_t* page_valid, int num_pages, int k_evict,
                                        float evict_fraction, int32_t* evict_list, int32_t* evict_count,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_pages >= 0, KESSIE_ERR_INVALID, "select evict: num_pages %d", num_pages);
  KESSIE_REQUIRE(scores && page_valid && evict_list && evict_count, KESSIE_ERR_INVALID, "select evict: null pointer");
  KESSIE_REQUIRE(k_evict >= 0 || (evict_fraction >= 0.0f && evict_fraction <= 1.0f), KESSIE_ERR_INVALID,
                 "select evict: evict_fraction %g outside [0,1]", (double)evict_fraction);
  int st = check_ws(workspace, workspace_bytes, num_pages, "select evict");
  if (st) return st;
  hipStream_t s = as_stream(stream);
  Workspace w = carve(workspace, num_pages);
  const int sg = max(1, min(kSelMaxGrid, div_up(num_pages, kSelTile)));
  hipLaunchKernelGGL(sel_clear_kernel, dim3(1), dim3(kThreads), 0, s, w.ss);
  hipLaunchKernelGGL(sel_hist_kernel, dim3(sg), dim3(kSelThreads), 0, s, scores, page_valid, num_pages, w.ss);
  hipLaunchKernelGGL(sel_bucket_kernel, dim3(1), dim3(kSelThreads), 0, s, w.ss, k_evict, evict_fraction, w.sel);
  hipLaunchKernelGGL(sel_collect_kernel, dim3(sg), dim3(kSelThreads), 0, s, scores, page_valid, num_pages, w.ss,
                     w.cand_s, w.cand_i);
  hipLaunchKernelGGL(sel_resolve_kernel, dim3(1), dim3(kSelThreads), 0, s, w.ss, w.cand_s, w.cand_i, w.sel);
  st = check_launch("select evict (radix select)");
  if (st) return st;
  PredArgs a{kPredScoreEvict, page_valid, nullptr, nullptr, 0, scores, &w.sel->key_thr, &w.sel->k};
  return ordered_compact(a, num_pages, evict_list, evict_count, w, s, page_valid);
}

extern "C" int kessie_page_compact(const int32_t* tables, const int32_t* lens, const int8_t* page_valid,
                                   int32_t* new_tables, int32_t* new_lens, int32_t* gather_idx, int32_t* gather_count,
                                   int num_seqs, int table_stride, int num_pages, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_seqs >= 0 && table_stride >= 0 && num_pages >= 0, KESSIE_ERR_INVALID,
                 "page compact: bad sizes S=%d W=%d pages=%d", num_seqs, table_stride, num_pages);
  KESSIE_REQUIRE((int64_t)num_seqs * table_stride <= INT_MAX, KESSIE_ERR_UNSUPPORTED, "page compact: table too big");
  if (num_seqs == 0) return KESSIE_OK;
  KESSIE_REQUIRE(tables && lens && page_valid && new_tables && new_lens && gather_idx && gather_count,
                 KESSIE_ERR_INVALID, "page compact: null pointer");
  KESSIE_REQUIRE(tables != new_tables, KESSIE_ERR_INVALID, "page compact: tables and new_tables must differ");
  const int n = num_seqs * table_stride;
  int st = check_ws(workspace, workspace_bytes, max(n, num_seqs), "page compact");
  if (st) return st;
  hipStream_t s = as_stream(stream);
  Workspace w = carve(workspace, max(n, num_seqs));
  hipLaunchKernelGGL(compact_rows_kernel, dim3(num_seqs), dim3(kThreads), 0, s, tables, lens, page_valid, new_tables,
                     new_lens, table_stride, num_pages);
  hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(kThreads), 0, s, new_lens, num_seqs, w.rows, gather_count);
  hipLaunchKernelGGL(flatten_rows_kernel, dim3(num_seqs), dim3(kThreads), 0, s, new_tables, new_lens, w.rows,
                     table_stride, gather_idx);
  return check_launch("page compact");
}

extern "C" int kessie_page_valid_list(const int8_t* page_valid, int num_pages, int32_t* out_idx, int32_t* out_count,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_pages >= 0, KESSIE_ERR_INVALID, "valid list: num_pages %d", num_pages);
  KESSIE_REQUIRE(page_valid && out_idx && out_count, KESSIE_ERR_INVALID, "valid list: null pointer");
  int st = check_ws(workspace, workspace_bytes, num_pages, "valid list");
  if (st) return st;
  Workspace w = carve(workspace, num_pages);
  PredArgs a{kPredValid, page_valid, nullptr, nullptr, 0, nullptr, nullptr, nullptr};
  return ordered_compact(a, num_pages, out_idx, out_count, w, as_stream(stream));
}

extern "C" int kessie_page_gather(const void* src_pool, int64_t page_bytes, const int32_t* idx,
                                  const int32_t* count_dev, int n, int num_pages, void* dst, void* stream) {
  clear_error();
  KESSIE_REQUIRE(n >= 0 && num_pages >= 0 && page_bytes > 0, KESSIE_ERR_INVALID,
                 "page gather: n=%d pages=%d page_bytes=%lld", n, num_pages, (long long)page_bytes);
  if (n == 0) return KESSIE_OK;
  KESSIE_REQUIRE(src_pool && idx && dst, KESSIE_ERR_INVALID, "page gather: null pointer");
  KESSIE_REQUIRE(page_bytes % 16 == 0 && aligned16(src_pool) && aligned16(dst), KESSIE_ERR_UNSUPPORTED,
                 "page gather: page_bytes and pointers must be 16-byte multiples/aligned");
  const int64_t page_vecs = page_bytes / 16;
  const int64_t tiles = div_up(page_vecs, (int64_t)kGatherThreads);
  const int per_region = div_up(n, kGatherRegions);
  const int64_t grid = tiles * per_region * kGatherRegions;
  KESSIE_REQUIRE(grid < (1LL << 31), KESSIE_ERR_UNSUPPORTED, "page gather: %d pages of %lld bytes is too large", n,
                 (long long)page_bytes);
  const u32x4* s = static_cast<const u32x4*>(src_pool);
  u32x4* d = static_cast<u32x4*>(dst);
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)grid), dim3(kGatherThreads), 0, as_stream(stream), s, page_vecs,
                     (int)tiles, per_region, idx, count_dev, n, num_pages, d);
  return check_launch("page gather");
}

// Reference launchers (kessie_kernels_v2.hip:753-782).
extern "C" void launch_kessie_page_evict(void* page_valid, const void* page_positions, void* evict_count,
                                         int evict_before_pos, int num_pages, void* stream) {
  clear_error();
  if (num_pages <= 0) return;
  if (!page_valid || !page_positions || !evict_count) {
    set_error(KESSIE_ERR_INVALID, "page evict: null pointer");
    return;
  }
  hipLaunchKernelGGL(threshold_evict_kernel, dim3(div_up(num_pages, kThreads)), dim3(kThreads), 0, as_stream(stream),
                     static_cast<int8_t*>(page_valid), static_cast<const int32_t*>(page_positions),
                     static_cast<int32_t*>(evict_count), evict_before_pos, num_pages);
  check_launch("page evict");
}

extern "C" void launch_kessie_page_insert(void* kv_cache, const void* new_keys, const void* new_values,
                                          const void* target_page_ids, void* page_valid, void* page_positions,
                                          int conv_pos, int num_tokens, int num_heads, int head_dim, int page_size,
                                          int max_pages, void* stream) {
  clear_error();
  const int64_t hs = head_dim;
  const int64_t kvs = (int64_t)num_heads * head_dim;
  const int64_t ts = 2 * kvs;
  const int64_t ps = (int64_t)page_size * ts;
  InsertArgs a{kv_cache,
               ps,
               ts,
               kvs,
               hs,
               new_keys,
               new_values,
               static_cast<const int32_t*>(target_page_ids),
               static_cast<int8_t*>(page_valid),
               static_cast<int32_t*>(page_positions),
               conv_pos,
               nullptr,
               nullptr,
               nullptr,
               num_tokens,
               num_heads,
               head_dim,
               page_size,
               max_pages};
  insert_dispatch(a, KESSIE_DTYPE_F16, as_stream(stream));
}
