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
  kPredValid = 0,  // valid[i] == 1
  kPredFreed = 1   // (valid==1 && pos<thr) || (allocated && allocated[i] && valid!=1)
};

struct PredArgs {
  int kind;
  const int8_t* valid;
  const int32_t* positions;
  const int8_t* allocated;
  int thr;
};

__device__ __forceinline__ bool pred_eval(const PredArgs& a, int i) {
  switch (a.kind) {
    case kPredValid:
      return a.valid[i] == 1;
    case kPredFreed: {
      const bool v = a.valid[i] == 1;
      if (v && a.positions[i] < a.thr) return true;
      return a.allocated != nullptr && a.allocated[i] != 0 && !v;
    }
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
// Score eviction: the key of rank k-1 among valid pages, then the ordered list
// of the keys up to it.  Keys are 64-bit (ordered score << 32 | page id), so
// they are unique and the k smallest are exactly the set the total order
// (score, id) puts first.  Two launches, no host round trip:
//   clear   a fill kernel zeroes the grid-barrier counter, the 4096-bin
//           histogram and the counters (graph-capture safe);
//   fused   G workgroups (G <= kFusedMaxG, one per CU at most: they are all
//           resident at once) that meet at three grid barriers:
//     P1  each workgroup histograms the top 12 bits of the ordered scores of
//         the valid pages of its tiles in LDS and adds them to the global
//         histogram;                                                    | B1
//     P2  every workgroup reads the histogram, derives k and the bin holding
//         rank k-1 and the rank inside it, and appends that bin's keys (low
//         20 score bits, page id) from its tiles to a candidate list, one
//         atomic per tile;                                              | B2
//     P3  every workgroup resolves the threshold key on the candidates (the
//         low 20 score bits in two 10-bit passes and, for tied scores, the
//         page id in 11+11+10 bits; the same result in every workgroup, so
//         no barrier is needed to share it), counts the pages of its tiles
//         it evicts and, in the fused evict + compact call, the survivors of
//         its table rows;                                               | B3
//     P4  prefix sums of those counts place each workgroup's evict-list
//         entries (ascending page id) and each table row's gather indices;
//         each workgroup writes its part and clears its evicted pages'
//         valid flags.
// A table entry survives when its page is valid and not evicted; the
// predicate reads page_valid, which other workgroups clear during P4 only for
// evicted pages, so it answers the same before or after their writes.  The
// histogram and candidate atomics only count: no result depends on their
// order.  Each barrier wait is bounded (~0.1 s); a wait that runs out (only
// possible if the device could not hold the G workgroups at once) marks the
// call failed and the evict count reads -1.  The mark is a bit of the barrier
// word itself, set by compare-and-swap only while the barrier is incomplete,
// so it precedes the last arrival in that word's modification order and every
// workgroup reads it after its last barrier: all of them see the failure, or
// none.  A failed call writes none of its outputs (page_valid, the evict
// list, the tables, the gather indices), so page_valid is left as it was and
// the call can be retried.
// Every workgroup loads its keys once, in P1 -- the 4,096 keys of its tile
// (4 per thread) and the page keys of its table-row entries (one 1,024-entry
// chunk per thread per row) -- and keeps them in registers, so P2-P4 touch
// memory only for the histogram, the candidates, the counts and the outputs.
// G = one workgroup per 4,096-key tile, at most 64: the barriers cost more
// with more workgroups (one contended counter; measured on 65,536 pages: 8
// workgroups 1.2 us per barrier, 16 2.8 us, 32-64 6-7 us), while the table
// rows spread over fewer workgroups take longer.  (Measured: five select
// launches + three compaction launches 35 us; one workgroup holding all
// 65,536 keys in registers 76 us -- a single CU is latency-bound in every
// phase.)
// ---------------------------------------------------------------------------
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelCap = 12288;                // candidate keys held in LDS
constexpr int kSelBins = 4096;
constexpr int kSelPer = 4;                    // consecutive keys per thread per tile
constexpr int kSelTile = kSelThreads * kSelPer;
constexpr int kFusedMaxG = 64;                // workgroups of the fused launch
constexpr int kFusedMaxRows = 8192;           // table rows whose offsets fit in LDS
constexpr int kSpinLimit = 1 << 21;           // barrier polls (s_sleep 2 each: ~0.1 s)
constexpr unsigned kBarFail = 0x80000000u;    // bit of FusedScratch::bar: a barrier wait ran out

// Scratch of the fused launch, at the start of the page workspace.  It is
// zero apart from `magic` between calls: kessie_page_workspace_init writes
// that state once, and each call's last workgroup to finish restores it, so
// no call needs a clearing launch of its own.
constexpr unsigned kScratchMagic = 0x4b535331u;
struct FusedScratch {
  unsigned magic;  // kScratchMagic once initialised
  unsigned bar;    // grid-barrier arrivals (| kBarFail once a wait ran out)
  unsigned done;   // workgroups past their last read of this scratch
  int unused;
  int n_valid;
  int ncand;
  int hist[kSelBins];
  int wg_evict[kFusedMaxG];  // evicted pages per workgroup (written before B3)
};

__device__ __forceinline__ uint32_t ordered_score(float s) {
  if (s == 0.0f) s = 0.0f;  // -0 == +0
  const uint32_t bits = __float_as_uint(s);
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

// Exclusive scan of one int per thread across the 1024-thread block; the
// block total is left in sm[kSelWaves] until the next call.
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

// sel_block_scan for 64-bit values (four 16-bit counts packed in one word);
// the block total is left in sm64[kSelWaves].
__device__ __forceinline__ unsigned long long sel_block_scan64(unsigned long long v, unsigned long long* sm64) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sm64[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long acc = 0;
    for (int w = 0; w < kSelWaves; ++w) {
      const unsigned long long t = sm64[w];
      sm64[w] = acc;
      acc += t;
    }
    sm64[kSelWaves] = acc;
  }
  __syncthreads();
  const unsigned long long res = x - v + sm64[wave];
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

__global__ __launch_bounds__(kThreads) void scratch_init_kernel(FusedScratch* fs) {
  for (int e = threadIdx.x; e < kSelBins; e += kThreads) fs->hist[e] = 0;
  if (threadIdx.x == 0) {
    fs->bar = 0;
    fs->done = 0;
    fs->unused = 0;
    fs->n_valid = 0;
    fs->ncand = 0;
    fs->magic = kScratchMagic;
  }
}

// All G workgroups arrive; returns once arrivals reach `target`, or once the
// bounded wait (`spin_limit` polls) has run out and the failure is recorded in
// fs->bar (or another workgroup recorded one).  The failure bit is set by
// compare-and-swap only on a value whose count is below `target`, so it is
// ordered before the barrier's last arrival: a workgroup that passes any later
// barrier, or reads fs->bar after its own last arrival, sees it.
// Release/acquire at agent scope make every write before the barrier visible
// to every workgroup after it.
__device__ __forceinline__ void grid_barrier(FusedScratch* fs, unsigned target, int spin_limit) {
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __hip_atomic_fetch_add(&fs->bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int spins = 0;
    unsigned v = __hip_atomic_load(&fs->bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Every pass either polls (at most spin_limit times), or attempts the
    // swap, which fails only when another arrival or failure changed fs->bar
    // (finitely many per call): the loop always ends.
    while ((v & ~kBarFail) < target && (v & kBarFail) == 0) {
      if (spins < spin_limit) {
        ++spins;
        __builtin_amdgcn_s_sleep(2);
        v = __hip_atomic_load(&fs->bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else if (__hip_atomic_compare_exchange_strong(&fs->bar, &v, v | kBarFail, __ATOMIC_RELAXED,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        break;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

struct FusedArgs {
  const float* scores;
  int8_t* valid;
  int n;
  int k_evict;
  float evict_fraction;
  int32_t* evict_list;
  int32_t* evict_count;
  // table compaction (tables == nullptr: select + evict only)
  const int32_t* tables;
  const int32_t* lens;
  int num_seqs;
  int table_stride;
  int32_t* new_tables;
  int32_t* new_lens;
  int32_t* gather_idx;
  int32_t* gather_count;
  // workspace
  FusedScratch* fs;
  uint32_t* cand_s;
  uint32_t* cand_i;
  int* row_count;
  int tiles_per_wg;
  int spin_limit;     // polls per barrier wait before the call is marked failed
  int extra_arrival;  // 1: the first barrier waits for one arrival more than the grid has (test hook)
};

// LDS of the fused kernel, in 32-bit words: P1/P2 use the first kSelBins as
// the histogram; P3 the 2048-bin resolve histogram plus the candidate copy;
// P4 the table row offsets.
constexpr int kFusedLdsWords = 2048 + 2 * kSelCap;
static_assert(kFusedLdsWords >= kSelBins && kFusedLdsWords >= kFusedMaxRows, "fused LDS layout");

// Buffer resources for the fused kernel's loads: dword-aligned raw buffers of
// `bytes` bytes (loads past the end read 0).  Every range is below 2^31 bytes
// (checked at the launch), so kOffNone, and any offset with bit 31 set, is
// past all of them.
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kOffNone = 0x7FFFFFF0;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t word_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}

constexpr int kTileRegs = 4;  // key tiles per workgroup held in registers (4 keys per thread each)
constexpr int kRowRegs = 4;   // 1,024-entry table-row chunks per workgroup held in registers

template <int kTR>
__global__ __launch_bounds__(kSelThreads) void sel_fused_kernel(FusedArgs a) {
  __shared__ uint32_t smem[kFusedLdsWords];
  __shared__ int sm[kSelWaves + 1];
  __shared__ int s_digit, s_rank, s_id, s_base, s_fail;
  FusedScratch* fs = a.fs;
  const int tid = threadIdx.x;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int ntiles = div_up(a.n, kSelTile);
  const int t_begin = min(ntiles, g * a.tiles_per_wg);
  const int t_end = min(ntiles, t_begin + a.tiles_per_wg);
  int* lhist = reinterpret_cast<int*>(smem);
  __shared__ unsigned long long sm64[kSelWaves + 1];
  // Read with the first input loads (one round trip for both); checked before
  // the first write to the scratch.
  const unsigned magic = __hip_atomic_load(&fs->magic, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // Key of page i: its ordered score when valid, ~0 otherwise (~0 sorts after
  // every valid key: the largest non-NaN ordered score is +inf's 0xFF800000).
  // Both loads are issued together (one round trip, not two).
  auto page_key = [&](int i) -> uint32_t {
    const float sc = a.scores[i];
    const int8_t v = a.valid[i];
    return v == 1 ? ordered_score(sc) : 0xFFFFFFFFu;
  };
  auto tile_key = [&](int t, int j) -> uint32_t {
    const int i = t * kSelTile + tid * kSelPer + j;
    return i < a.n ? page_key(i) : 0xFFFFFFFFu;
  };
  // Table rows: this workgroup owns rows g, g + G, ...; each row is cut into
  // chunks of 1,024 entries (one per thread); chunk c of the workgroup is
  // chunk c % cpr of its (c / cpr)-th row.
  const bool tables = a.tables != nullptr;
  const int cpr = tables ? max(1, div_up(a.table_stride, kSelThreads)) : 0;
  const int my_rows = tables && g < a.num_seqs ? div_up(a.num_seqs - g, G) : 0;
  const int my_chunks = my_rows * cpr;
  auto row_len = [&](int row) { return min(max(a.lens[row], 0), a.table_stride); };
  // Entry of chunk c for this thread: page id (-1 when absent) and the key of
  // that page when it is a valid page id (~0 otherwise).
  // The row length and the table entry are loaded together (every entry below
  // table_stride is in bounds), then the page's flag and score together: two
  // round trips, not three.
  auto chunk_entry = [&](int c, int* id_out) -> uint32_t {
    const int row = g + (c / cpr) * G;
    const int j = (c % cpr) * kSelThreads + tid;
    const int len = row_len(row);
    const int raw = j < a.table_stride ? a.tables[(int64_t)row * a.table_stride + j] : -1;
    const int id = j < len ? raw : -1;
    *id_out = id;
    return (id >= 0 && id < a.n) ? page_key(id) : 0xFFFFFFFFu;
  };

  // P1: load this workgroup's keys (tiles and table entries) into registers;
  // histogram the top 12 ordered-score bits of its valid pages.  The loads are
  // straight-line code with no branch between them (a load under a condition
  // turns the select on its value into a branch that waits for it): the
  // tiles' flags and scores and the rows' lengths and entries in one round
  // trip, then the flags and scores of the pages those entries name, which
  // are only needed after the first grid barrier and stay in flight through
  // the histogram.
  uint32_t tk[kTR][kSelPer];
  uint32_t rk[kRowRegs];
  int rid[kRowRegs];
  float rsc[kRowRegs];
  int rv[kRowRegs];
  {
    // Range-limited buffer resources: a load past the end reads 0 instead of
    // faulting, so absent tiles, rows and page ids need no clamp and no branch
    // (an absent slot loads at kOffNone, past every range; a 0 flag is not 1,
    // so its key is ~0).
    const auto sc_rs = word_rsrc(a.scores, (uint32_t)a.n * 4u);
    const auto va_rs = word_rsrc(a.valid, (uint32_t)a.n);
    float tsc[kTR][kSelPer];
    int tv[kTR][kSelPer];
#pragma unroll
    for (int u = 0; u < kTR; ++u)
#pragma unroll
      for (int j = 0; j < kSelPer; ++j) {
        const uint32_t i = (uint32_t)((t_begin + u) * kSelTile + tid * kSelPer + j);
        const bool in = t_begin + u < t_end;
        tsc[u][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sc_rs, in ? (int)(i * 4u) : kOffNone, 0, 0));
        tv[u][j] = __builtin_amdgcn_raw_buffer_load_b8(va_rs, in ? (int)i : kOffNone, 0, 0);
      }
    const auto ln_rs = word_rsrc(a.lens, tables ? (uint32_t)a.num_seqs * 4u : 0u);
    int rlen[kRowRegs], rraw[kRowRegs];
#pragma unroll
    for (int u = 0; u < kRowRegs; ++u) {
      const int row = g + (u / cpr) * G;
      const int j = (u % cpr) * kSelThreads + tid;
      const bool in = u < my_chunks;
      const auto tb_rs = word_rsrc(in ? a.tables + (int64_t)row * a.table_stride : nullptr,
                                   in ? (uint32_t)a.table_stride * 4u : 0u);
      rlen[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(ln_rs, in ? row * 4 : kOffNone, 0, 0);
      rraw[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(tb_rs, in ? j * 4 : kOffNone, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kRowRegs; ++u) {
      const int j = (u % cpr) * kSelThreads + tid;
      const int len = min(max(rlen[u], 0), a.table_stride);
      rid[u] = u < my_chunks && j < len ? rraw[u] : -1;
      // Out-of-range ids get bit 31 set: past every range (an offset select
      // here is split into two loads of one register, which then wait on
      // each other).
      const uint32_t out = (uint32_t)rid[u] < (uint32_t)a.n ? 0u : 0x80000000u;
      rsc[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sc_rs, (int)(((uint32_t)rid[u] * 4u) | out), 0, 0));
      rv[u] = __builtin_amdgcn_raw_buffer_load_b8(va_rs, (int)((uint32_t)rid[u] | out), 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kTR; ++u)
#pragma unroll
      for (int j = 0; j < kSelPer; ++j) tk[u][j] = tv[u][j] == 1 ? ordered_score(tsc[u][j]) : 0xFFFFFFFFu;
  }
  if (magic != kScratchMagic) {
    // The workspace was never initialised (kessie_page_workspace_init): touch
    // nothing.  `magic` is the same for every workgroup, so all return here.
    if (g == 0 && tid == 0) {
      *a.evict_count = -2;
      if (a.tables != nullptr) *a.gather_count = -2;
    }
    return;
  }
  for (int e = tid; e < kSelBins; e += kSelThreads) lhist[e] = 0;
  // (A call that has failed at a barrier may pick from incomplete counts, where
  // no bin holds the rank: the picks then keep these in-range values.)
  if (tid == 0) {
    s_digit = 0;
    s_rank = 0;
  }
  __syncthreads();
  int c = 0;
  for (int t = t_begin; t < t_end; ++t) {
#pragma unroll
    for (int j = 0; j < kSelPer; ++j) {
      uint32_t x = 0xFFFFFFFFu;
#pragma unroll
      for (int u = 0; u < kTR; ++u)
        if (t - t_begin == u) x = tk[u][j];
      if (t - t_begin >= kTR) x = tile_key(t, j);
      if (x != 0xFFFFFFFFu) {
        atomicAdd(&lhist[x >> 20], 1);
        ++c;
      }
    }
  }
  for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
  if ((tid & 63) == 0 && c) atomicAdd(&fs->n_valid, c);
  __syncthreads();
  if (t_end > t_begin)
    for (int e = tid; e < kSelBins; e += kSelThreads)
      if (lhist[e]) atomicAdd(&fs->hist[e], lhist[e]);
  grid_barrier(fs, (unsigned)(G + a.extra_arrival), a.spin_limit);
#pragma unroll
  for (int u = 0; u < kRowRegs; ++u)
    rk[u] = rid[u] >= 0 && rid[u] < a.n && rv[u] == 1 ? ordered_score(rsc[u]) : 0xFFFFFFFFu;

  // P2: k, the bin of rank k-1, and that bin's candidates.  (The histogram and
  // the valid count are read in one round trip: all loads, then the stores.)
  int n_valid;
  {
    static_assert(kSelBins % kSelThreads == 0, "histogram bins per thread");
    int hv[kSelBins / kSelThreads];
#pragma unroll
    for (int r = 0; r < kSelBins / kSelThreads; ++r)
      hv[r] = __hip_atomic_load(&fs->hist[tid + r * kSelThreads], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    n_valid = __hip_atomic_load(&fs->n_valid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int r = 0; r < kSelBins / kSelThreads; ++r) lhist[tid + r * kSelThreads] = hv[r];
  }
  long long kk;
  if (a.k_evict >= 0) {
    kk = min(a.k_evict, n_valid);
  } else {
    kk = (long long)floor((double)a.evict_fraction * (double)n_valid);
    kk = max(0LL, min(kk, (long long)n_valid));
  }
  const int k = (int)kk;
  __syncthreads();
  uint32_t top = 0;
  int rank = 0;
  if (k > 0) {
    sel_pick(lhist, kSelBins, k - 1, sm, &s_digit, &s_rank);
    top = (uint32_t)s_digit;
    rank = s_rank;
    for (int t = t_begin; t < t_end; ++t) {
      const int base = t * kSelTile + tid * kSelPer;
      uint32_t ks[kSelPer];
      int cnt = 0, mbits = 0;
#pragma unroll
      for (int j = 0; j < kSelPer; ++j) {
        uint32_t x = 0xFFFFFFFFu;
#pragma unroll
        for (int u = 0; u < kTR; ++u)
          if (t - t_begin == u) x = tk[u][j];
        if (t - t_begin >= kTR) x = tile_key(t, j);
        ks[j] = x;
        if (x != 0xFFFFFFFFu && (x >> 20) == top) {
          mbits |= 1 << j;
          ++cnt;
        }
      }
      int pos = sel_block_scan(cnt, sm);
      if (tid == 0 && sm[kSelWaves] > 0) s_base = atomicAdd(&fs->ncand, sm[kSelWaves]);
      __syncthreads();
      pos += s_base;
#pragma unroll
      for (int j = 0; j < kSelPer; ++j) {
        if (!((mbits >> j) & 1)) continue;
        a.cand_s[pos] = ks[j] & 0xFFFFFu;
        a.cand_i[pos] = (uint32_t)(base + j);
        ++pos;
      }
      __syncthreads();  // s_base and sm are reused by the next tile
    }
  }
  grid_barrier(fs, 2u * G, a.spin_limit);

  // P3: the threshold key (identical in every workgroup), then the counts.
  unsigned long long key_thr = 0;
  if (k > 0) {
    int* rhist = reinterpret_cast<int*>(smem);
    uint32_t* lds_s = smem + 2048;
    uint32_t* lds_i = smem + 2048 + kSelCap;
    const int nc = __hip_atomic_load(&fs->ncand, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t* cs = a.cand_s;
    const uint32_t* ci = a.cand_i;
    if (nc <= kSelCap) {
      for (int q = tid; q < nc; q += kSelThreads) {
        lds_s[q] = a.cand_s[q];
        lds_i[q] = a.cand_i[q];
      }
      cs = lds_s;
      ci = lds_i;
    }
    __syncthreads();
    uint32_t low = 0;
    int ties = 0;
    for (int pass = 0; pass < 2; ++pass) {
      const int sh = 10 - 10 * pass;
      for (int e = tid; e < 1024; e += kSelThreads) rhist[e] = 0;
      __syncthreads();
      for (int q = tid; q < nc; q += kSelThreads) {
        const uint32_t v = cs[q];
        if (pass == 0 || (v >> 10) == low) atomicAdd(&rhist[(v >> sh) & 1023u], 1);
      }
      __syncthreads();
      sel_pick(rhist, 1024, rank, sm, &s_digit, &s_rank);
      low = (low << 10) | (uint32_t)s_digit;
      rank = s_rank;
      ties = rhist[s_digit];
      __syncthreads();
    }
    uint32_t idp = 0;
    if (ties == 1) {
      for (int q = tid; q < nc; q += kSelThreads)
        if (cs[q] == low) s_id = (int)ci[q];
      __syncthreads();
      idp = (uint32_t)s_id;
    } else {
      for (int pass = 0; pass < 3; ++pass) {
        const int width = pass < 2 ? 11 : 10;
        const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
        for (int e = tid; e < 2048; e += kSelThreads) rhist[e] = 0;
        __syncthreads();
        for (int q = tid; q < nc; q += kSelThreads) {
          if (cs[q] != low) continue;
          const uint32_t id = ci[q];
          if (pass == 0 || (id >> (sh + width)) == idp) atomicAdd(&rhist[(id >> sh) & ((1u << width) - 1u)], 1);
        }
        __syncthreads();
        sel_pick(rhist, 2048, rank, sm, &s_digit, &s_rank);
        idp = (idp << width) | (uint32_t)s_digit;
        rank = s_rank;
        __syncthreads();
      }
    }
    key_thr = ((unsigned long long)((top << 20) | low) << 32) | idp;
  }
  // Evicted: a valid page whose (key, id) is <= the threshold (k > 0 only).
  auto evicted_key = [&](uint32_t x, int i) -> bool {
    return k > 0 && x != 0xFFFFFFFFu && (((unsigned long long)x << 32) | (uint32_t)i) <= key_thr;
  };
  auto tile_key_at = [&](int t, int j) -> uint32_t {
    uint32_t x = 0xFFFFFFFFu;
#pragma unroll
    for (int u = 0; u < kTR; ++u)
      if (t - t_begin == u) x = tk[u][j];
    if (t - t_begin >= kTR) x = tile_key(t, j);
    return x;
  };
  // Table entry of chunk c: survives when it names a valid page that is not evicted.
  auto chunk_survivor = [&](int cc, int* id_out) -> bool {
    int id = -1;
    uint32_t x = 0xFFFFFFFFu;
#pragma unroll
    for (int u = 0; u < kRowRegs; ++u)
      if (cc == u) {
        id = rid[u];
        x = rk[u];
      }
    if (cc >= kRowRegs) x = chunk_entry(cc, &id);
    *id_out = id;
    return x != 0xFFFFFFFFu && !evicted_key(x, id);
  };
  {
    int ce = 0;
    for (int t = t_begin; t < t_end; ++t)
#pragma unroll
      for (int j = 0; j < kSelPer; ++j) ce += evicted_key(tile_key_at(t, j), t * kSelTile + tid * kSelPer + j);
    for (int o = 32; o >= 1; o >>= 1) ce += __shfl_xor(ce, o, 64);
    if ((tid & 63) == 0) sm[tid >> 6] = ce;
    __syncthreads();
    if (tid == 0) {
      int s = 0;
      for (int w = 0; w < kSelWaves; ++w) s += sm[w];
      __hip_atomic_store(&fs->wg_evict[g], s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
  }
  // Rows of at most 1,024 entries, at most kRowRegs of them: all counted (and
  // later placed) by one packed scan, a 16-bit field per row.
  const bool packed_rows = cpr == 1 && my_rows <= kRowRegs;
  unsigned long long pk = 0;
  if (packed_rows) {
#pragma unroll
    for (int u = 0; u < kRowRegs; ++u) {
      int id;
      if (u < my_rows && chunk_survivor(u, &id)) pk += 1ull << (16 * u);
    }
    unsigned long long wsum = pk;  // pk itself is kept for the placing scan in P4
    for (int o = 32; o >= 1; o >>= 1) wsum += __shfl_xor(wsum, o, 64);
    if ((tid & 63) == 0) sm64[tid >> 6] = wsum;
    __syncthreads();
    if (tid < my_rows) {
      unsigned long long t = 0;
      for (int w = 0; w < kSelWaves; ++w) t += sm64[w];
      __hip_atomic_store(&a.row_count[g + tid * G], (int)((t >> (16 * tid)) & 0xFFFFull), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
  } else {
    for (int rr = 0; rr < my_rows; ++rr) {
      int cs = 0;
      for (int cc = rr * cpr; cc < (rr + 1) * cpr; ++cc) {
        int id;
        cs += chunk_survivor(cc, &id);
      }
      for (int o = 32; o >= 1; o >>= 1) cs += __shfl_xor(cs, o, 64);
      if ((tid & 63) == 0) sm[tid >> 6] = cs;
      __syncthreads();
      if (tid == 0) {
        int s = 0;
        for (int w = 0; w < kSelWaves; ++w) s += sm[w];
        __hip_atomic_store(&a.row_count[g + rr * G], s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
    }
  }
  grid_barrier(fs, 3u * G, a.spin_limit);

  // P4: read what the other workgroups published, leave the scratch, then
  // write the evict list (ascending ids, clearing the pages' valid flags) and
  // the compacted tables.
  // (Read by one thread: every workgroup reads fs->bar here after its own last
  // arrival, so all of them get the same answer.)
  if (tid == 0) s_fail = (__hip_atomic_load(&fs->bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kBarFail) != 0;
  __syncthreads();
  const bool failed = s_fail != 0;
  if (tid < 64) {
    int v = 0;
    if (tid < g) v = __hip_atomic_load(&fs->wg_evict[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if (tid == 0) s_base = v;
  }
  int* row_off = reinterpret_cast<int*>(smem);  // gather-list offset of every row
  int run = 0;
  if (tables) {
    for (int r0 = 0; r0 < a.num_seqs; r0 += kSelThreads) {
      const int r = r0 + tid;
      const int v = r < a.num_seqs ? __hip_atomic_load(&a.row_count[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : 0;
      const int ex = sel_block_scan(v, sm);
      if (r < a.num_seqs) row_off[r] = run + ex;
      run += sm[kSelWaves];
    }
  }
  __syncthreads();
  // The last workgroup out restores the scratch for the next call: every other
  // workgroup has passed its last barrier and its last read of it.
  if (tid == 0) s_id = (int)__hip_atomic_fetch_add(&fs->done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_id == G - 1) {
    for (int e = tid; e < kSelBins; e += kSelThreads)
      __hip_atomic_store(&fs->hist[e], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
      __hip_atomic_store(&fs->bar, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&fs->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&fs->n_valid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&fs->ncand, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (failed) {
    // Outputs untouched: only the counts report the failure.
    if (g == 0 && tid == 0) {
      if (tables) *a.gather_count = -1;
      *a.evict_count = -1;
    }
    return;
  }
  int carry = s_base;
  for (int t = t_begin; t < t_end; ++t) {
    const int base = t * kSelTile + tid * kSelPer;
    unsigned flags = 0;
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kSelPer; ++j)
      if (evicted_key(tile_key_at(t, j), base + j)) {
        flags |= 1u << j;
        ++cnt;
      }
    int pos = carry + sel_block_scan(cnt, sm);
    const int total = sm[kSelWaves];
#pragma unroll
    for (int j = 0; j < kSelPer; ++j) {
      if (!(flags & (1u << j))) continue;
      a.evict_list[pos++] = base + j;
      a.valid[base + j] = 0;
    }
    carry += total;
  }
  if (tables) {
    if (packed_rows) {
      const unsigned long long ex = sel_block_scan64(pk, sm64);
      const unsigned long long tot = sm64[kSelWaves];
#pragma unroll
      for (int u = 0; u < kRowRegs; ++u) {
        if (u >= my_rows) continue;
        const int row = g + u * G;
        int32_t* outr = a.new_tables + (int64_t)row * a.table_stride;
        int id;
        if (chunk_survivor(u, &id)) {
          const int pos = (int)((ex >> (16 * u)) & 0xFFFFull);
          outr[pos] = id;
          a.gather_idx[row_off[row] + pos] = id;
        }
        const int rc = (int)((tot >> (16 * u)) & 0xFFFFull);
        for (int j = rc + tid; j < a.table_stride; j += kSelThreads) outr[j] = -1;
        if (tid == 0) a.new_lens[row] = rc;
      }
    } else {
      for (int rr = 0; rr < my_rows; ++rr) {
        const int row = g + rr * G;
        int32_t* outr = a.new_tables + (int64_t)row * a.table_stride;
        const int off = row_off[row];
        int rc = 0;
        for (int cc = rr * cpr; cc < (rr + 1) * cpr; ++cc) {
          int id;
          const int sv = chunk_survivor(cc, &id) ? 1 : 0;
          const int pos = rc + sel_block_scan(sv, sm);
          rc += sm[kSelWaves];
          if (sv) {
            outr[pos] = id;
            a.gather_idx[off + pos] = id;
          }
        }
        for (int j = rc + tid; j < a.table_stride; j += kSelThreads) outr[j] = -1;
        if (tid == 0) a.new_lens[row] = rc;
      }
    }
    if (g == 0 && tid == 0) *a.gather_count = run;
  }
  if (g == 0 && tid == 0) *a.evict_count = k;
}

// ---------------------------------------------------------------------------
// Table compaction in one launch: one workgroup per table row; the row's
// offset in the gather list comes from a decoupled look-back over the rows
// before it (flags[row] = state << 62 | value, state 1 = the row's own count
// published, 2 = the inclusive prefix published), so no second pass and no
// second launch.  The flags must be zero on entry (the single-workgroup score
// eviction clears them in the fused call; kessie_page_compact launches a fill
// kernel first).  Workgroups only wait for lower-numbered rows, which were
// dispatched earlier and publish without waiting; each wait is bounded and a
// workgroup whose wait runs out counts the earlier rows itself, so the result
// never depends on the wait.
// ---------------------------------------------------------------------------
constexpr int kLbThreads = 256;
constexpr unsigned long long kLbAgg = 1ull << 62, kLbPre = 2ull << 62, kLbMask = (1ull << 62) - 1ull;

__device__ __forceinline__ bool lb_survives(int id, const int8_t* valid, int num_pages) {
  return id >= 0 && id < num_pages && valid[id] == 1;
}

__global__ __launch_bounds__(kLbThreads) void compact_lookback_kernel(
    const int32_t* __restrict__ tables, const int32_t* __restrict__ lens, const int8_t* __restrict__ valid,
    int32_t* __restrict__ new_tables, int32_t* __restrict__ new_lens, int32_t* __restrict__ gather_idx,
    int32_t* __restrict__ gather_count, int num_seqs, int table_stride, int num_pages,
    unsigned long long* flags) {
  __shared__ int sm[kWaves + 1];
  __shared__ long long s_prefix;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t* in = tables + (int64_t)row * table_stride;
  int32_t* outr = new_tables + (int64_t)row * table_stride;
  auto row_len = [&](int rr) { return min(max(lens[rr], 0), table_stride); };
  const int len = row_len(row);

  int cnt = 0;
  for (int j = tid; j < len; j += kLbThreads) cnt += lb_survives(in[j], valid, num_pages);
  int total;
  block_exclusive_scan(cnt, &total, sm);

  // Look-back by the first wave: lane l reads the flag of row (j_hi - l); the
  // nearest row that has published its inclusive prefix ends the walk (rows
  // before 0 read as an inclusive prefix of 0).
  if (tid < 64) {
    const int lane = tid;
    if (lane == 0)
      __hip_atomic_store(&flags[row], (row == 0 ? kLbPre : kLbAgg) | (unsigned long long)total, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    long long prefix = 0;
    int j_hi = row - 1, spins = 0;
    bool fallback = false;
    while (j_hi >= 0) {
      const int j = j_hi - lane;
      const unsigned long long f =
          j >= 0 ? __hip_atomic_load(&flags[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : kLbPre;
      const unsigned long long st = f & ~kLbMask;
      const unsigned long long pre = __builtin_amdgcn_ballot_w64(st == kLbPre);
      const unsigned long long nr = __builtin_amdgcn_ballot_w64(st != kLbPre && st != kLbAgg);
      const int stop = pre ? __builtin_ctzll(pre) : 64;               // nearest inclusive prefix
      const unsigned long long need = stop == 64 ? ~0ull : ((2ull << stop) - 1ull);  // lanes 0..stop
      if (nr & need) {  // a needed row has not published yet
        if (++spins > kSpinLimit) {
          fallback = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        continue;
      }
      long long v = ((need >> lane) & 1ull) ? (long long)(f & kLbMask) : 0;
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
      prefix += v;
      if (stop < 64) break;
      j_hi -= 64;
    }
    if (lane == 0) {
      if (fallback) {
        s_prefix = -1;  // counted below by the whole workgroup
      } else {
        s_prefix = prefix;
        if (row > 0)
          __hip_atomic_store(&flags[row], kLbPre | (unsigned long long)(prefix + total), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __syncthreads();
  long long prefix = s_prefix;
  if (prefix < 0) {  // bounded wait ran out: count the earlier rows directly
    int c = 0;
    for (int rr = 0; rr < row; ++rr) {
      const int l = row_len(rr);
      const int32_t* rin = tables + (int64_t)rr * table_stride;
      for (int j = tid; j < l; j += kLbThreads) c += lb_survives(rin[j], valid, num_pages);
    }
    int t2;
    block_exclusive_scan(c, &t2, sm);
    prefix = t2;
    if (tid == 0)
      __hip_atomic_store(&flags[row], kLbPre | (unsigned long long)(prefix + total), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }

  // Write the row: survivors in logical order, -1 after them.
  int rc = 0;
  for (int j0 = 0; j0 < len; j0 += kLbThreads) {
    const int j = j0 + tid;
    const int id = j < len ? in[j] : -1;
    const int sv = (j < len && lb_survives(id, valid, num_pages)) ? 1 : 0;
    int t3;
    const int pos = rc + block_exclusive_scan(sv, &t3, sm);
    if (sv) {
      outr[pos] = id;
      gather_idx[prefix + pos] = id;
    }
    rc += t3;
  }
  for (int j = rc + tid; j < table_stride; j += kLbThreads) outr[j] = -1;
  if (tid == 0) {
    new_lens[row] = rc;
    if (row == num_seqs - 1) *gather_count = (int32_t)(prefix + rc);
  }
}

__global__ __launch_bounds__(kThreads) void clear_flags_kernel(unsigned long long* flags, int n) {
  for (int j = blockIdx.x * kThreads + threadIdx.x; j < n; j += gridDim.x * kThreads) flags[j] = 0ull;
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
  int* counts;
  int* offsets;
  int* rows;                   // per-row counts (table compaction of the grid-barrier call)
  unsigned long long* flags;   // per-row look-back flags (same memory as rows)
  FusedScratch* fs;
  uint32_t* cand_s;  // select candidates (n each)
  uint32_t* cand_i;
};

constexpr size_t round256(size_t b) { return (b + 255) / 256 * 256; }

size_t workspace_bytes(int n) {
  const size_t nb = (size_t)num_blocks(n);
  size_t b = round256(sizeof(FusedScratch));        // fused-select scratch (first: its offset is fixed)
  b += round256(nb * sizeof(int));                  // counts
  b += round256(nb * sizeof(int));                  // offsets
  b += round256(((size_t)n + 1) * sizeof(unsigned long long));  // per-row counts / look-back flags
  b += 2 * round256((size_t)n * sizeof(uint32_t));  // select candidates
  return b;
}

Workspace carve(void* ws, int n) {
  Workspace w;
  char* c = static_cast<char*>(ws);
  const size_t nb = (size_t)num_blocks(n);
  w.fs = reinterpret_cast<FusedScratch*>(c);
  c += round256(sizeof(FusedScratch));
  w.counts = reinterpret_cast<int*>(c);
  c += round256(nb * sizeof(int));
  w.offsets = reinterpret_cast<int*>(c);
  c += round256(nb * sizeof(int));
  w.rows = reinterpret_cast<int*>(c);
  w.flags = reinterpret_cast<unsigned long long*>(c);
  c += round256(((size_t)n + 1) * sizeof(unsigned long long));
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

// Test hook: KESSIE_GRID_TEST_TIMEOUT=<polls> makes the fused launch's first
// grid barrier wait for one arrival more than the grid has, giving up after
// <polls> polls, so a test drives the failure path deterministically while
// every workgroup still exits normally.  Unset: the full bounded wait.
void grid_test_hook(int* spin_limit, int* extra_arrival) {
  const char* v = getenv("KESSIE_GRID_TEST_TIMEOUT");
  if (v == nullptr || *v == '\0') {
    *spin_limit = kSpinLimit;
    *extra_arrival = 0;
    return;
  }
  *spin_limit = min(max(0, atoi(v)), kSpinLimit);
  *extra_arrival = 1;
}

// Score eviction (+ table compaction when tables != nullptr): the fused launch.
int select_dispatch(const float* scores, int8_t* page_valid, int num_pages, int k_evict, float evict_fraction,
                    int32_t* evict_list, int32_t* evict_count, const int32_t* tables, const int32_t* lens,
                    int num_seqs, int table_stride, int32_t* new_tables, int32_t* new_lens, int32_t* gather_idx,
                    int32_t* gather_count, void* workspace, size_t workspace_bytes, hipStream_t s) {
  KESSIE_REQUIRE(num_pages >= 0, KESSIE_ERR_INVALID, "select evict: num_pages %d", num_pages);
  KESSIE_REQUIRE(scores && page_valid && evict_list && evict_count, KESSIE_ERR_INVALID, "select evict: null pointer");
  KESSIE_REQUIRE(num_pages < (1 << 29) && table_stride < (1 << 29), KESSIE_ERR_UNSUPPORTED,
                 "select evict: %d pages / %d table columns (at most 2^29 - 1 each)", num_pages, table_stride);
  KESSIE_REQUIRE(k_evict >= 0 || (evict_fraction >= 0.0f && evict_fraction <= 1.0f), KESSIE_ERR_INVALID,
                 "select evict: evict_fraction %g outside [0,1]", (double)evict_fraction);
  const int nws = max(num_pages, num_seqs);
  int st = check_ws(workspace, workspace_bytes, nws, "select evict");
  if (st) return st;
  Workspace w = carve(workspace, nws);
  const int ntiles = div_up(max(num_pages, 1), kSelTile);
  const int G = max(1, min(kFusedMaxG, ntiles));
  FusedArgs a{scores,       page_valid, num_pages, k_evict,  evict_fraction, evict_list, evict_count,
              tables,       lens,       num_seqs,  table_stride, new_tables, new_lens,   gather_idx,
              gather_count, w.fs,       w.cand_s,  w.cand_i,   w.rows,       div_up(ntiles, G),
              kSpinLimit,   0};
  grid_test_hook(&a.spin_limit, &a.extra_arrival);
  if (a.tiles_per_wg == 1)
    hipLaunchKernelGGL(sel_fused_kernel<1>, dim3(G), dim3(kSelThreads), 0, s, a);
  else
    hipLaunchKernelGGL(sel_fused_kernel<kTileRegs>, dim3(G), dim3(kSelThreads), 0, s, a);
  return check_launch("select evict");
}

}  // namespace pages
}  // namespace kessie

using namespace kessie;
using namespace kessie::pages;

extern "C" size_t kessie_page_workspace_bytes(int num_pages) { return pages::workspace_bytes(max(num_pages, 0)); }

extern "C" int kessie_page_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  KESSIE_REQUIRE(workspace != nullptr && workspace_bytes >= pages::workspace_bytes(0), KESSIE_ERR_WORKSPACE,
                 "page workspace init: %zu bytes (at least %zu)", workspace_bytes, pages::workspace_bytes(0));
  KESSIE_REQUIRE(aligned16(workspace), KESSIE_ERR_INVALID, "page workspace init: not 16-byte aligned");
  hipLaunchKernelGGL(scratch_init_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream),
                     static_cast<FusedScratch*>(workspace));
  return check_launch("page workspace init");
}

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
  PredArgs a{kPredFreed, page_valid, page_positions, allocated, evict_before_pos};
  return ordered_compact(a, num_pages, freed_list, freed_count, w, s, page_valid, allocated);
}

extern "C" int kessie_page_select_evict(const float* scores, int8_t* page_valid, int num_pages, int k_evict,
                                        float evict_fraction, int32_t* evict_list, int32_t* evict_count,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return pages::select_dispatch(scores, page_valid, num_pages, k_evict, evict_fraction, evict_list, evict_count,
                                nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr, nullptr, workspace,
                                workspace_bytes, as_stream(stream));
}

extern "C" int kessie_page_evict_compact(const float* scores, int8_t* page_valid, int num_pages, int k_evict,
                                         float evict_fraction, int32_t* evict_list, int32_t* evict_count,
                                         const int32_t* tables, const int32_t* lens, int num_seqs,
                                         int table_stride, int32_t* new_tables, int32_t* new_lens,
                                         int32_t* gather_idx, int32_t* gather_count, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  clear_error();
  KESSIE_REQUIRE(num_seqs >= 0 && table_stride >= 0, KESSIE_ERR_INVALID, "evict compact: S=%d W=%d", num_seqs,
                 table_stride);
  KESSIE_REQUIRE(num_seqs <= kFusedMaxRows, KESSIE_ERR_UNSUPPORTED,
                 "evict compact: %d sequences (at most %d; call select_evict + compact)", num_seqs, kFusedMaxRows);
  KESSIE_REQUIRE((int64_t)num_seqs * table_stride <= INT_MAX, KESSIE_ERR_UNSUPPORTED, "evict compact: table too big");
  KESSIE_REQUIRE(num_seqs == 0 || (tables && lens && new_tables && new_lens && gather_idx && gather_count),
                 KESSIE_ERR_INVALID, "evict compact: null table pointer");
  KESSIE_REQUIRE(tables == nullptr || tables != new_tables, KESSIE_ERR_INVALID,
                 "evict compact: tables and new_tables must differ");
  return pages::select_dispatch(scores, page_valid, num_pages, k_evict, evict_fraction, evict_list, evict_count,
                                num_seqs > 0 ? tables : nullptr, lens, num_seqs, table_stride, new_tables, new_lens,
                                gather_idx, gather_count, workspace, workspace_bytes, as_stream(stream));
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
  // A fill kernel zeroes the look-back flags (graph-capture safe), then one
  // workgroup per row compacts it and places it in the gather list.
  hipLaunchKernelGGL(clear_flags_kernel, dim3(max(1, min(64, div_up(num_seqs, kThreads)))), dim3(kThreads), 0, s,
                     w.flags, num_seqs);
  hipLaunchKernelGGL(compact_lookback_kernel, dim3(num_seqs), dim3(kLbThreads), 0, s, tables, lens, page_valid,
                     new_tables, new_lens, gather_idx, gather_count, num_seqs, table_stride, num_pages, w.flags);
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
  PredArgs a{kPredValid, page_valid, nullptr, nullptr, 0};
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
