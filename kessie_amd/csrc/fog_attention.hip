// Fog attention over paged KV for gfx950: decode, chunked prefill and the
// reference's dense launchers.
//
// Math (kessie_hip_kernels.py:577-593 and kessie_attention.py:114-139):
//   s_j = (q . k_j) * sm_scale + bias_j                (bias mode, optional)
//   keep j iff j < ctx, (!causal || j <= q_pos) and
//              (W == 0 || (0 <= q_pos - j < W))
//   o   = sum_j softmax(s)_j * w_j * v_j               (V mode, w optional,
//                                                       not renormalised)
// accumulated in fp32 with an online softmax; -inf masking with a guarded
// rescale, so a fully masked stretch contributes nothing.
//
// Kernels:
//   decode_mfma   bf16/f16 (fp32: decode_mfma_f32 on v_mfma_f32_16x16x4_f32,
//                 same decomposition), head_dim 128, pages of 16 * 2^k tokens
//                 (read as 16-token blocks).  One workgroup =
//                 one (sequence, split) x 2 kv heads, one wave per kv head; a
//                 wave streams its kv head's 256-byte K and V rows of every
//                 page in its split with 16-byte loads (register prefetch of
//                 PREF pages); QK^T and PV both on MFMA (P in the input
//                 dtype, accumulation in fp32), V transposed through LDS.
//   attn_generic  any dtype / head_dim <= 256 / page size / GQA ratio: K and
//                 V tiles staged in LDS as fp32, one workgroup per
//                 (row tile, kv head, sequence, split).  Serves the shapes the
//                 MFMA kernels do not take (fp32 prefill, other head_dims,
//                 page sizes and GQA ratios).
//   combine       merges the per-split (m, l, o) partials of either kernel.
#include <climits>
#include <cmath>
#include <cstdlib>

#include <atomic>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "attn_common.h"

namespace kessie {
namespace attn {

// ---------------------------------------------------------------------------
// Generic kernel
// ---------------------------------------------------------------------------
constexpr int kGenThreads = 256;
constexpr int kGenKT = 32;  // keys per LDS tile
constexpr int kGenRT = 16;  // query rows per workgroup
constexpr int kGenMaxD = 256;
constexpr int kGenAcc = kGenRT * kGenMaxD / kGenThreads;  // accumulators per thread

size_t generic_lds_bytes(int D) {
  return sizeof(float) * ((size_t)kGenRT * D + (size_t)kGenKT * (D + 1) + (size_t)kGenKT * D +
                          (size_t)kGenRT * kGenKT + 3 * kGenRT) +
         sizeof(int) * kGenRT + sizeof(int64_t) * kGenKT;
}

template <typename T>
__global__ __launch_bounds__(kGenThreads) void attn_generic_kernel(Params p) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int D = p.D;
  int64_t* off_s = reinterpret_cast<int64_t*>(smem_raw);  // [KT]
  float* q_s = reinterpret_cast<float*>(off_s + kGenKT);  // [RT][D]
  float* k_s = q_s + kGenRT * D;                          // [KT][D+1]
  float* v_s = k_s + kGenKT * (D + 1);                    // [KT][D]
  float* s_s = v_s + kGenKT * D;                          // [RT][KT]
  float* m_s = s_s + kGenRT * kGenKT;                     // [RT]
  float* l_s = m_s + kGenRT;                              // [RT]
  float* a_s = l_s + kGenRT;                              // [RT]
  int* pos_s = reinterpret_cast<int*>(a_s + kGenRT);      // [RT] query position, INT_MIN = no row

  const int tid = threadIdx.x;
  const int split = blockIdx.x;
  const int tile = blockIdx.y;
  const int b = blockIdx.z / p.Hkv;
  const int g = blockIdx.z % p.Hkv;
  const int ctx = seq_ctx(p, b);
  const int n_rows = p.C * p.G;
  const T* qbase = static_cast<const T*>(p.q);
  const T* kbase = static_cast<const T*>(p.k);
  const T* vbase = static_cast<const T*>(p.v);

  // Rows of this tile and their query positions.
  if (tid < kGenRT) {
    const int fr = tile * kGenRT + tid;
    int pos = INT_MIN;
    if (fr < n_rows) {
      const int i = fr / p.G;
      const int qp = ctx - p.C + i;
      if (qp >= 0) pos = qp;
    }
    pos_s[tid] = pos;
    m_s[tid] = kNegInf;
    l_s[tid] = 0.0f;
  }
  for (int e = tid; e < kGenRT * D; e += kGenThreads) {
    const int r = e / D, d = e - r * D;
    const int fr = tile * kGenRT + r;
    float x = 0.0f;
    if (fr < n_rows) {
      const int i = fr / p.G, hh = fr - i * p.G;
      x = to_f32(qbase[(int64_t)b * p.q_bs + (int64_t)i * p.q_is + (int64_t)(g * p.G + hh) * p.q_hs + d]);
    }
    q_s[e] = x;
  }
  __syncthreads();

  int qmin = INT_MAX, qmax = INT_MIN;
  for (int r = 0; r < kGenRT; ++r) {
    const int pos = pos_s[r];
    if (pos != INT_MIN) {
      qmin = min(qmin, pos);
      qmax = max(qmax, pos);
    }
  }
  int lo = 0, hi = 0;
  if (qmax != INT_MIN) key_range(p, ctx, qmin, qmax, &lo, &hi);
  const int per = (hi - lo + p.num_splits - 1) / p.num_splits;
  const int kb = lo + split * per;
  const int ke = min(hi, kb + per);

  float acc[kGenAcc];
#pragma unroll
  for (int a = 0; a < kGenAcc; ++a) acc[a] = 0.0f;

  for (int t0 = kb; t0 < ke; t0 += kGenKT) {
    if (tid < kGenKT) {
      const int t = t0 + tid;
      off_s[tid] = (t < ke) ? token_offset(p, b, t) : -1;
    }
    __syncthreads();
    for (int e = tid; e < kGenKT * D; e += kGenThreads) {
      const int tt = e / D, d = e - tt * D;
      const int64_t off = off_s[tt];
      float kx = 0.0f, vx = 0.0f;
      if (off >= 0) {
        kx = to_f32(kbase[off + (int64_t)g * p.head_stride + d]);
        vx = to_f32(vbase[off + (int64_t)g * p.head_stride + d]);
      }
      k_s[tt * (D + 1) + d] = kx;
      v_s[tt * D + d] = vx;
    }
    __syncthreads();
    for (int e = tid; e < kGenRT * kGenKT; e += kGenThreads) {
      const int r = e / kGenKT, j = e - r * kGenKT;
      const int t = t0 + j;
      const int pos = pos_s[r];
      float s = kNegInf;
      if (pos != INT_MIN && off_s[j] >= 0 && key_visible(pos, t, p.window, p.causal)) {
        float dot = 0.0f;
        const float* qr = q_s + r * D;
        const float* kr = k_s + j * (D + 1);
        for (int d = 0; d < D; ++d) dot += qr[d] * kr[d];
        s = dot * p.sm_scale;
        if (p.bias) s += p.bias[(int64_t)b * p.bias_bs + t];
      }
      s_s[e] = s;
    }
    __syncthreads();
    {
      // 16 threads per row, 2 keys each.
      const int r = tid >> 4, sub = tid & 15;
      const float s0 = s_s[r * kGenKT + sub];
      const float s1 = s_s[r * kGenKT + sub + 16];
      float mx = fmaxf(s0, s1);
#pragma unroll
      for (int w = 8; w >= 1; w >>= 1) mx = fmaxf(mx, __shfl_xor(mx, w, 16));
      const float mo = m_s[r];
      const float mn = fmaxf(mo, mx);
      const float p0 = (s0 == kNegInf) ? 0.0f : expf(s0 - mn);
      const float p1 = (s1 == kNegInf) ? 0.0f : expf(s1 - mn);
      float sum = p0 + p1;
#pragma unroll
      for (int w = 8; w >= 1; w >>= 1) sum += __shfl_xor(sum, w, 16);
      float w0 = 1.0f, w1 = 1.0f;
      if (p.vscale) {
        const int t_a = t0 + sub, t_b = t0 + sub + 16;
        w0 = (p0 != 0.0f) ? p.vscale[(int64_t)b * p.vs_bs + t_a] : 0.0f;
        w1 = (p1 != 0.0f) ? p.vscale[(int64_t)b * p.vs_bs + t_b] : 0.0f;
      }
      s_s[r * kGenKT + sub] = p0 * w0;
      s_s[r * kGenKT + sub + 16] = p1 * w1;
      __syncthreads();  // every thread has read m_s[r] before it changes
      if (sub == 0) {
        const float alpha = (mo == kNegInf) ? 0.0f : expf(mo - mn);
        l_s[r] = l_s[r] * alpha + sum;
        m_s[r] = mn;
        a_s[r] = alpha;
      }
    }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < kGenAcc; ++a) {
      const int e = tid + a * kGenThreads;
      if (e < kGenRT * D) {
        const int r = e / D, d = e - r * D;
        float o = acc[a] * a_s[r];
        const float* pr = s_s + r * kGenKT;
        for (int j = 0; j < kGenKT; ++j) o += pr[j] * v_s[j * D + d];
        acc[a] = o;
      }
    }
    __syncthreads();
  }

  // Epilogue: normalised output (one split) or partials.
#pragma unroll
  for (int a = 0; a < kGenAcc; ++a) {
    const int e = tid + a * kGenThreads;
    if (e >= kGenRT * D) continue;
    const int r = e / D, d = e - r * D;
    const int fr = tile * kGenRT + r;
    if (fr >= n_rows) continue;
    const int i = fr / p.G, h = g * p.G + (fr - i * p.G);
    if (p.direct_out) {
      const float l = l_s[r];
      store_out<T>(p, b, i, h, d, l > 0.0f ? acc[a] / l : 0.0f);
    } else {
      const int64_t row = row_id(p, b, i, h);
      p.ws_o[(row * p.num_splits + split) * D + d] = acc[a];
      if (d == 0) {
        p.ws_m[row * p.num_splits + split] = m_s[r];
        p.ws_l[row * p.num_splits + split] = l_s[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Split combine
// ---------------------------------------------------------------------------
constexpr int kCombineThreads = 256;
constexpr int kMaxSplits = 512;

// ---------------------------------------------------------------------------
// Balanced decode splits.  A decode launch has U = S * B workgroups per group
// of kv heads; with every sequence split S ways, a batch of one long context
// and many short ones leaves most of them idle while the long one streams.
// Instead the U units go to the batch's pages: P, the pages per unit, is the
// smallest value (at least ceil(max pages / kMaxSplits), so that no row has
// more partials than the combine takes) with sum_b ceil(pages_b / P) <= U,
// and sequence b gets ceil(pages_b / P) consecutive units.  A uniform batch
// gets S units per sequence, the page ranges of the plain split.  Unit u's
// partial of head h sits at slot h * U + u, so a row's partials are
// consecutive, as in the plain layout.  Each function is evaluated by a
// whole wave (lane b holds sequence b: batches of up to kBalSeqs) and returns
// the same value in every lane.
//
// Every wave of the launch runs this before its first page load, and its
// cost is mostly the fetch of its code (the caches hold none of it at the
// start of a launch): an unrolled form with four lengths per lane took
// 6-8 us per wave before the first page load, and a 4K-token decode ran 2.8
// times slower than with the plain split; a second pass over the same code in
// the same wave took 0.2 us.  So the code is kept short (one length per lane,
// reductions and the scan on the device library's DPP path), and
// decode_entry only chooses it for batches whose streaming time makes the
// rest negligible.
// ---------------------------------------------------------------------------
extern "C" __device__ int __ockl_wfscan_add_i32(int, bool);  // inclusive when the flag is set

constexpr int kBalSeqs = 64;  // batches the balanced split takes: one length per lane

// 16-token blocks a decode over ctx tokens reads: those of its window.
__device__ __forceinline__ int decode_pages(const Params& p, int ctx) {
  const int lo = p.window > 0 ? max(0, ctx - p.window) : 0;
  return ((ctx + 15) >> 4) - (lo >> 4);
}
struct BatchPages {
  int ctx;  // length of sequence `lane` (0 past the batch)
  int pg;   // its pages
  __device__ int seq_len(int b) const { return __builtin_amdgcn_readlane(ctx, b); }  // uniform b
  __device__ int seq_pages(int b) const { return __builtin_amdgcn_readlane(pg, b); }
};
__device__ __forceinline__ BatchPages batch_pages(const Params& p) {
  const int lane = threadIdx.x & 63;
  BatchPages bp;
  bp.ctx = lane < p.B ? clamp_ctx(p, p.ctx_lens ? p.ctx_lens[lane] : p.ctx_const) : 0;
  bp.pg = decode_pages(p, bp.ctx);
  return bp;
}
// P for S units per sequence of a B-sequence batch (U = S * B).
__device__ int decode_unit_pages(const BatchPages& bp, int S, int B) {
  const int lane = threadIdx.x & 63;
  const int mx = __ockl_wfred_max_i32(bp.pg);
  const int mn = __ockl_wfred_min_i32(lane < B ? bp.pg : INT_MAX);
  int lo = max(1, (mx + kMaxSplits - 1) / kMaxSplits);
  // Every sequence the same length: S units each, the plain split.
  if (mn == mx) return max(lo, (mx + S - 1) / S);
  const int tot = __ockl_wfred_add_i32(bp.pg);
  const int nz = __ockl_wfred_add_i32(bp.pg > 0 ? 1 : 0);
  const int U = S * B;
  // Bounds on the answer: a P that fits has tot / P <= U, so P >= ceil(tot / U);
  // P = mx fits (at most B <= U units), and so does ceil(tot / (U - nz)) when
  // U > nz, since sum ceil(pages / P) <= tot / P + nz.
  lo = max(lo, (tot + U - 1) / U);
  int hi = max(lo, mx);
  if (U > nz) hi = min(hi, max(lo, (tot + (U - nz) - 1) / (U - nz)));
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (__ockl_wfred_add_i32((bp.pg + mid - 1) / mid) <= U)
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo;
}
// The sequence and split of unit u (uniform u); false when u is past the
// batch's units.
__device__ bool decode_seq_of_unit(const BatchPages& bp, int P, int u, int* b_out, int* s_out) {
  const int n = (bp.pg + P - 1) / P;
  const int incl = __ockl_wfscan_add_i32(n, true);
  if (u >= __builtin_amdgcn_readlane(incl, 63)) return false;
  const int b = __ffsll((long long)__ballot(u < incl)) - 1;  // the first lane whose units reach past u
  *b_out = b;
  *s_out = u - __builtin_amdgcn_readlane(incl - n, b);
  return true;
}
// The first unit of sequence b (uniform b) and its number of units.
__device__ void decode_units_of_seq(const BatchPages& bp, int P, int b, int* u0, int* n) {
  const int lane = threadIdx.x & 63;
  *u0 = __ockl_wfred_add_i32(lane < b ? (bp.pg + P - 1) / P : 0);
  *n = (bp.seq_pages(b) + P - 1) / P;
}
// Workgroup (row, y) merges d in [y*D/Y, (y+1)*D/Y) of one row (Y =
// gridDim.y, 1 unless rows are few).  With an even chunk its 256 lanes are
// (split group, float2 column) pairs: each sums every groups-th split of its
// column, and the groups meet in LDS.  (One thread per d looping over every
// split was latency-bound: 25 us for one 128K sequence's 32 rows x 256 splits,
// against 89 us for the whole partials kernel.)
// Sum over the split groups of column col of a combine workgroup (thread
// tid = group * cols + col, cols a power of two).  TREE: the groups inside a
// wave by shuffles (lane bits from cols up), then the waves' sums in order
// through LDS -- a few steps where adding the groups one by one took a chain
// of dependent LDS reads (one combine of the fp32 4K decode: 32 groups).  Not
// TREE: the groups added one by one in increasing order, which with at most
// one split per group is the splits in increasing order whatever cols is --
// so a varlen prefill and its per-sequence launches (different row counts,
// hence different head_dim splits) give the same bits.  Both combine kernels
// sum this way for a given TREE, so their results are the same bits.  The
// result is valid in threads tid < cols.
template <bool TREE>
__device__ __forceinline__ float2 sum_groups(float ax, float ay, int tid, int cols, int groups, float2* part) {
  if (!TREE) {
    part[tid] = make_float2(ax, ay);
    __syncthreads();
    float2 acc = make_float2(0.0f, 0.0f);
    if (tid < cols) {
      acc = part[tid];
      for (int g = 1; g < groups; ++g) {
        acc.x += part[g * cols + tid].x;
        acc.y += part[g * cols + tid].y;
      }
    }
    return acc;
  }
  for (int off = cols; off < 64; off <<= 1) {
    ax += __shfl_xor(ax, off, 64);
    ay += __shfl_xor(ay, off, 64);
  }
  const int lane = tid & 63;
  const int q_n = cols < 64 ? kCombineThreads / 64 : groups;  // partial sums per column
  if (cols >= 64)
    part[tid] = make_float2(ax, ay);
  else if (lane < cols)
    part[(tid >> 6) * cols + lane] = make_float2(ax, ay);
  __syncthreads();
  float2 acc = make_float2(0.0f, 0.0f);
  if (tid < cols) {
    acc = part[tid];
    for (int q = 1; q < q_n; ++q) {
      acc.x += part[q * cols + tid].x;
      acc.y += part[q * cols + tid].y;
    }
  }
  return acc;
}

template <typename T, bool TREE>
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(Params p) {
  __shared__ float e_s[kMaxSplits];
  __shared__ float2 part[kCombineThreads];
  __shared__ float inv_l;
  const int64_t row = blockIdx.x;  // (b*C + i)*Hq + h
  const int S = p.num_splits;
  const int D = p.D;
  const int h = (int)(row % p.Hq);
  const int64_t bi = row / p.Hq;
  int i = (int)(bi % p.C);
  int b = (int)(bi / p.C);
  if (p.q_start) {  // varlen prefill: rows past the chunk have no partials
    const int s0 = p.q_start[b] - p.q_start[0];
    if (i >= p.q_start[b + 1] - p.q_start[b]) return;  // uniform, before any barrier (i < max_query_len)
    i += s0;
    b = 0;
  }
  const int tid = threadIdx.x, lane = tid & 63;
  // The row's partials: S of them at row * S + s, or, with balanced decode
  // splits, n_s at h * S * B + u0 + s (its sequence's units).
  __shared__ int s_first, s_count;
  int64_t first = row * S;
  int n_s = S;
  if (p.balanced) {
    if (tid < 64) {
      const BatchPages bp = batch_pages(p);
      const int P = decode_unit_pages(bp, S, p.B);
      int u0, n;
      decode_units_of_seq(bp, P, b, &u0, &n);
      if (tid == 0) {
        s_first = u0;
        s_count = n;
      }
    }
    __syncthreads();
    first = (int64_t)h * S * p.B + s_first;
    n_s = s_count;
  }
  i += p.q0_off;  // rows of a dense split start at position q0_off
  const float* m = p.ws_m + first;
  const float* l = p.ws_l + first;
  if (tid < 64) {
    float mx = kNegInf;
    for (int s = lane; s < n_s; s += 64) mx = fmaxf(mx, m[s]);
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) mx = fmaxf(mx, __shfl_xor(mx, w, 64));
    float sum = 0.0f;
    for (int s = lane; s < n_s; s += 64) {
      const float ms = m[s];
      const float e = (ms == kNegInf) ? 0.0f : expf(ms - mx);
      e_s[s] = e;
      sum += e * l[s];
    }
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) sum += __shfl_xor(sum, w, 64);
    if (lane == 0) inv_l = sum > 0.0f ? 1.0f / sum : 0.0f;
  }
  __syncthreads();
  const float il = inv_l;
  const int chunk = D / gridDim.y;
  const int d0 = blockIdx.y * chunk;
  const float* o = p.ws_o + first * D + d0;
  if ((chunk & 1) == 0 && kCombineThreads % (chunk / 2) == 0) {
    const int cols = chunk / 2;                // float2 columns
    const int groups = kCombineThreads / cols;
    const int col = tid % cols, grp = tid / cols;
    float ax = 0.0f, ay = 0.0f;
#pragma unroll 4
    for (int s = grp; s < n_s; s += groups) {
      const float e = e_s[s];
      const float2 v = *reinterpret_cast<const float2*>(o + (int64_t)s * D + 2 * col);
      ax += e * v.x;
      ay += e * v.y;
    }
    const float2 acc = sum_groups<TREE>(ax, ay, tid, cols, groups, part);
    if (tid < cols) {
      store_out<T>(p, b, i, h, d0 + 2 * tid, acc.x * il);
      store_out<T>(p, b, i, h, d0 + 2 * tid + 1, acc.y * il);
    }
  } else {
    for (int d = tid; d < chunk; d += kCombineThreads) {
      float acc = 0.0f;
      for (int s = 0; s < n_s; ++s) acc += e_s[s] * o[(int64_t)s * D + d];
      store_out<T>(p, b, i, h, d0 + d, acc * il);
    }
  }
}

// Workgroups per row of the combine: split head_dim into up to eight even
// chunks when the rows alone would leave the chip mostly idle.
inline int combine_dsplit(int64_t rows, int D) {
  int y = 1;
  while (y < 8 && rows * y < 256 && D % (4 * y) == 0) y *= 2;  // the chunk D/y stays even
  return y;
}

// combine_kernel with every load issued first (S <= 256 splits, at most
// kAheadLoads per thread, plain split layout): lane s of wave 0 holds (m, l)
// of splits s, s + 64, ..., and each thread the float2 column of its split
// group, all requested before the first use, where combine_kernel waits for
// the maxima, then for (m, l) again, then for the partials (three round trips
// instead of one; a 4K-token decode's combine is latency-bound).  The same
// arithmetic in the same order as combine_kernel's fast path -- max and sum
// over lanes s, s + 64, ... then the same butterfly, each group's splits
// summed in increasing order, the groups met by the same sum_groups -- so the
// two give the same bits.
constexpr int kAheadLoads = 8;

template <typename T, bool TREE>
__global__ __launch_bounds__(kCombineThreads) void combine_ahead_kernel(Params p) {
  __shared__ float e_s[256];
  __shared__ float2 part[kCombineThreads];
  __shared__ float inv_l;
  const int64_t row = blockIdx.x;  // (b*C + i)*Hq + h
  const int S = p.num_splits;
  const int D = p.D;
  const int h = (int)(row % p.Hq);
  const int64_t bi = row / p.Hq;
  int i = (int)(bi % p.C);
  int b = (int)(bi / p.C);
  if (p.q_start) {  // varlen prefill: rows past the chunk have no partials
    const int s0 = p.q_start[b] - p.q_start[0];
    if (i >= p.q_start[b + 1] - p.q_start[b]) return;  // uniform, before any barrier
    i += s0;
    b = 0;
  }
  i += p.q0_off;
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t first = row * S;
  const int chunk = D / gridDim.y;
  const int d0 = blockIdx.y * chunk;
  const int cols = chunk / 2, groups = kCombineThreads / cols;
  const int col = tid % cols, grp = tid / cols;
  const float* o = p.ws_o + first * D + d0 + 2 * col;
  float2 v[kAheadLoads];
#pragma unroll
  for (int j = 0; j < kAheadLoads; ++j) {
    const int sp = grp + j * groups;
    v[j] = sp < S ? *reinterpret_cast<const float2*>(o + (int64_t)sp * D) : make_float2(0.0f, 0.0f);
  }
  float mv[4], lv[4];
  if (tid < 64) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int sp = lane + 64 * k;
      mv[k] = sp < S ? p.ws_m[first + sp] : kNegInf;
      lv[k] = sp < S ? p.ws_l[first + sp] : 0.0f;
    }
    float mx = kNegInf;
#pragma unroll
    for (int k = 0; k < 4; ++k) mx = fmaxf(mx, mv[k]);
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) mx = fmaxf(mx, __shfl_xor(mx, w, 64));
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int sp = lane + 64 * k;
      if (sp < S) {
        const float ms = mv[k];
        const float e = (ms == kNegInf) ? 0.0f : expf(ms - mx);
        e_s[sp] = e;
        sum += e * lv[k];
      }
    }
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) sum += __shfl_xor(sum, w, 64);
    if (lane == 0) inv_l = sum > 0.0f ? 1.0f / sum : 0.0f;
  }
  __syncthreads();
  const float il = inv_l;
  float ax = 0.0f, ay = 0.0f;
#pragma unroll
  for (int j = 0; j < kAheadLoads; ++j) {
    const int sp = grp + j * groups;
    if (sp < S) {
      const float e = e_s[sp];
      ax += e * v[j].x;
      ay += e * v[j].y;
    }
  }
  const float2 acc = sum_groups<TREE>(ax, ay, tid, cols, groups, part);
  if (tid < cols) {
    store_out<T>(p, b, i, h, d0 + 2 * tid, acc.x * il);
    store_out<T>(p, b, i, h, d0 + 2 * tid + 1, acc.y * il);
  }
}

// The per-row merge of split partials: combine_ahead_kernel where its loads
// fit (plain split layout, S <= 256, an even chunk dividing the workgroup,
// S <= groups * kAheadLoads), else combine_kernel.  Same bits either way.
// Decode sums the split groups as a tree; the prefill combines (TREE false)
// in split order, which keeps varlen and per-sequence launches bit-equal.
template <typename T, bool TREE = true>
void launch_row_combine(const Params& p, int64_t rows, hipStream_t s) {
  const int y = combine_dsplit(rows, p.D);
  const int chunk = p.D / y;
  const int S = p.num_splits;
  bool ahead = !p.balanced && S <= 256 && (chunk & 1) == 0 && kCombineThreads % (chunk / 2) == 0;
  if (ahead) ahead = S <= (kCombineThreads / (chunk / 2)) * kAheadLoads;
  if (ahead)
    hipLaunchKernelGGL((combine_ahead_kernel<T, TREE>), dim3((unsigned)rows, y), dim3(kCombineThreads), 0, s, p);
  else
    hipLaunchKernelGGL((combine_kernel<T, TREE>), dim3((unsigned)rows, y), dim3(kCombineThreads), 0, s, p);
}

// Two consecutive outputs of lane-owned columns: one 8-byte store for
// fp32, one packed 4-byte store for bf16/fp16 (rows start on even columns).
template <typename T>
__device__ __forceinline__ void store2(T* dst, float a, float b);
template <>
__device__ __forceinline__ void store2<float>(float* dst, float a, float b) {
  *reinterpret_cast<float2*>(dst) = make_float2(a, b);
}
template <>
__device__ __forceinline__ void store2<bf16_t>(bf16_t* dst, float a, float b) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<bf2*>(dst) = bf2{from_f32<bf16_t>(a), from_f32<bf16_t>(b)};
}
template <>
__device__ __forceinline__ void store2<f16_t>(f16_t* dst, float a, float b) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<h2*>(dst) = h2{from_f32<f16_t>(a), from_f32<f16_t>(b)};
}

// Combine for many rows (split prefill and the dense launchers: a row per
// query position and head), S <= 16: each wave merges four rows, lane 16r + s
// holding (m, l) of split s of row r and every lane D / 64 columns of all
// four rows, with all of the wave's loads issued before any use.  The
// per-row workgroups of combine_kernel are dispatch- and latency-bound at
// these counts (65,536 rows: 97 us).  The same merge, summed in the same
// order, as combine_kernel (max and sum over the splits by the same butterfly
// -- its first two steps, across halves and quarters of the wave, only add
// zeros there -- and the columns in GR groups of every GR-th split, added in
// group order), so the two kernels give the same bits.  SM bounds the split
// count of an instance (4, 8 or 16): the partial registers are sized by it,
// so S <= 4 (the dense launchers, most split prefills) runs at 8 waves per
// SIMD instead of the 3 that room for 16 splits leaves.
constexpr int kCombRows = 4;                   // rows per wave
constexpr int kCombRowsPerWg = 4 * kCombRows;  // four waves

template <typename T, int D, int SM>
__global__ __launch_bounds__(256) void combine_rows_kernel(Params p, int64_t rows) {
  constexpr int NC = D / 64;                       // columns per lane
  constexpr int GR = kCombineThreads / (D / 2);    // combine_kernel's split groups
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kCombRows;
  if (row0 >= rows) return;  // uniform per wave; no barriers
  const int S = p.num_splits;
  // (m, l) of split lane % 16 of row row0 + lane / 16.
  const int64_t mr = min(row0 + lane / 16, rows - 1);
  const bool mok = (lane & 15) < S && row0 + lane / 16 < rows;
  const float m = mok ? p.ws_m[mr * S + (lane & 15)] : kNegInf;
  const float l = mok ? p.ws_l[mr * S + (lane & 15)] : 0.0f;
  // Partials: v[r][sp][c] of row row0 + r (clamped into range), split sp < S,
  // NC columns per load.
  typedef float fNC __attribute__((ext_vector_type(NC)));
  fNC v[kCombRows][SM];
#pragma unroll
  for (int r = 0; r < kCombRows; ++r) {
    const float* o = p.ws_o + min(row0 + r, rows - 1) * S * D + NC * lane;
#pragma unroll
    for (int sp = 0; sp < SM; ++sp)
      v[r][sp] = sp < S ? *reinterpret_cast<const fNC*>(o + (int64_t)sp * D) : fNC{};
  }
  float mx = m;
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  const float e = m == kNegInf ? 0.0f : expf(m - mx);
  float sum = e * l;
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
#pragma unroll
  for (int r = 0; r < kCombRows; ++r) {
    const int64_t row = row0 + r;
    if (row >= rows) break;  // uniform
    float part[GR][NC];
#pragma unroll
    for (int g = 0; g < GR; ++g)
#pragma unroll
      for (int c = 0; c < NC; ++c) part[g][c] = 0.0f;
#pragma unroll
    for (int sp = 0; sp < SM; ++sp) {
      if (sp < S) {  // uniform
        const float es = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), 16 * r + sp));
#pragma unroll
        for (int c = 0; c < NC; ++c) part[sp % GR][c] += es * v[r][sp][c];
      }
    }
    const float sr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sum), 16 * r));
    const float il = sr > 0.0f ? 1.0f / sr : 0.0f;
    const int h = (int)(row % p.Hq);
    const int64_t bi = row / p.Hq;
    int i = (int)(bi % p.C), b = (int)(bi / p.C);
    if (p.q_start) {  // varlen prefill: rows past the chunk have no partials
      if (i >= p.q_start[b + 1] - p.q_start[b]) continue;
      i += p.q_start[b] - p.q_start[0];
      b = 0;
    }
    i += p.q0_off;  // rows of a dense split start at position q0_off
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      acc[c] = part[0][c];
#pragma unroll
      for (int g = 1; g < GR; ++g) acc[c] += part[g][c];
    }
    T* dst = static_cast<T*>(p.out) + (int64_t)b * p.o_bs + (int64_t)i * p.o_is + (int64_t)h * p.o_hs + NC * lane;
    if constexpr (NC == 2)
      store2<T>(dst, acc[0] * il, acc[1] * il);
    else
      dst[0] = from_f32<T>(acc[0] * il);
  }
}

// Launches the merge of split partials into the output: combine_rows_kernel
// for many rows, combine_kernel otherwise.
template <typename T>
void launch_combine(const Params& p, int64_t rows, hipStream_t s) {
  const bool even = ((p.o_bs | p.o_is | p.o_hs) & 1) == 0 && ((uintptr_t)p.out & 3) == 0;  // packed stores
  if (rows >= 4096 && !p.balanced && p.num_splits <= 16 && (p.D == 128 || p.D == 64) && even) {
    const dim3 grid((unsigned)div_up(rows, (int64_t)kCombRowsPerWg));
    const int sm = p.num_splits <= 4 ? 4 : p.num_splits <= 8 ? 8 : 16;
    if (p.D == 128) {
      if (sm == 4)
        hipLaunchKernelGGL((combine_rows_kernel<T, 128, 4>), grid, dim3(256), 0, s, p, rows);
      else if (sm == 8)
        hipLaunchKernelGGL((combine_rows_kernel<T, 128, 8>), grid, dim3(256), 0, s, p, rows);
      else
        hipLaunchKernelGGL((combine_rows_kernel<T, 128, 16>), grid, dim3(256), 0, s, p, rows);
    } else {
      if (sm == 4)
        hipLaunchKernelGGL((combine_rows_kernel<T, 64, 4>), grid, dim3(256), 0, s, p, rows);
      else if (sm == 8)
        hipLaunchKernelGGL((combine_rows_kernel<T, 64, 8>), grid, dim3(256), 0, s, p, rows);
      else
        hipLaunchKernelGGL((combine_rows_kernel<T, 64, 16>), grid, dim3(256), 0, s, p, rows);
    }
    return;
  }
  launch_row_combine<T, false>(p, rows, s);
}


// ---------------------------------------------------------------------------
// MFMA decode (bf16 / f16, head_dim 128, pages of 16 * 2^k tokens)
//
// One workgroup = (split of one sequence's pages) x kDecWaves kv heads, one
// wave per kv head, no workgroup barriers.  Per page a wave:
//   * loads its kv head's K rows (16 tokens x 256 B) straight into the A
//     operand layout of MFMA 16x16x32 (lane = token l%16, 16 bytes of d), and
//     its V rows with 16-byte loads (lane group q = tokens 4q..4q+3, chunk
//     l%16), PREF pages ahead in registers;
//   * S^T = K Q^T on MFMA (B operand = the GQA group's query rows, head =
//     column l%16).  The accumulator layout puts head l%16's scores for tokens
//     4q..4q+3 in lane l, so the online softmax is lane-local plus two
//     cross-row reductions, and p (times the fog weight) is already the B
//     operand layout of MFMA 16x16x16 for PV -- no shuffles;
//   * V goes through a per-wave LDS tile (row stride 272 B: the four token
//     rows a read touches land on different banks) and is read back
//     transposed as the A operand: O^T[d][h] += V^T[d][t] P^T[t][h];
//   * the O^T accumulators are rescaled only when some head's running max
//     moved on that page.
// ---------------------------------------------------------------------------
constexpr int kDecWaves = 2;     // kv heads (waves) per decode workgroup
constexpr int kDecPref = 2;      // pages in flight per wave
constexpr int kDecWgsPerCu = 4;  // 2 waves/SIMD x 4 SIMDs / kDecWaves: one round of the grid
constexpr int kVRow = 128 + 8;  // LDS row stride of the V and Q tiles (elements)

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  typedef bf16x8 vec8;
  typedef bf16x4 vec4;
  static __device__ __forceinline__ f32x4 mma32(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
  }
};
template <>
struct Mfma<f16_t> {
  typedef f16x8 vec8;
  typedef f16x4 vec4;
  static __device__ __forceinline__ f32x4 mma32(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};

// Orders this wave's LDS writes before its later LDS reads (and the reads of
// one page before the writes of the next): wait for outstanding LDS traffic
// and keep the compiler from moving LDS accesses across.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// FOG: which per-token fog vectors the instance reads (bit 0 the logit bias,
// bit 1 the V-scale); each one read costs a register per prefetched page.
constexpr int kFogBias = 1, kFogVs = 2;

template <typename T, int G, int PREF, int W, int FOG>
// Two waves per SIMD (256 VGPRs; ~160 used with two pages of K and V in flight).
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_mfma_kernel(Params p) {
  typedef typename Mfma<T>::vec8 vec8;
  typedef typename Mfma<T>::vec4 vec4;
  __shared__ __align__(16) T vtile_all[W][16 * kVRow];
  __shared__ __align__(16) T qtile_all[W][16 * kVRow];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = blockIdx.z * W + wave;
  if (g >= p.Hkv) return;  // no workgroup barriers below
  T* vtile = vtile_all[wave];
  T* qtile = qtile_all[wave];
  const int S = p.num_splits;
  const int unit = blockIdx.y * S + blockIdx.x;  // balanced splits: this workgroup's unit
  int b = blockIdx.y, split = blockIdx.x, per = 0;
  int ctx;
  if (p.balanced) {
    const BatchPages bp = batch_pages(p);
    per = decode_unit_pages(bp, S, p.B);
    if (!decode_seq_of_unit(bp, per, unit, &b, &split)) return;  // past the batch's units: no partial to write
    // Wave-uniform results, kept in scalar registers so that the page loop's
    // bounds and page-table reads stay scalar (as vector loads they would
    // queue behind the page prefetch).
    per = __builtin_amdgcn_readfirstlane(per);
    b = __builtin_amdgcn_readfirstlane(b);
    split = __builtin_amdgcn_readfirstlane(split);
    ctx = bp.seq_len(b);
  } else {
    ctx = seq_ctx(p, b);
  }
  const int row = lane & 15;  // MFMA row / column index: token (K rows), head (scores), d (O^T)
  const int grp = lane >> 4;  // lane group: k-block slot, token quad

  const int lo = p.window > 0 ? max(0, ctx - p.window) : 0;
  const int pg_lo = lo >> 4;
  const int pg_hi = (ctx + 15) >> 4;
  if (!p.balanced) per = (pg_hi - pg_lo + S - 1) / S;
  const int p0 = pg_lo + split * per;
  const int p1 = min(pg_hi, p0 + per);

  const T* kbase = static_cast<const T*>(p.k) + (int64_t)g * p.head_stride;
  const T* vbase = static_cast<const T*>(p.v) + (int64_t)g * p.head_stride;
  const int32_t* table = p.page_table + (int64_t)b * p.table_stride;
  const int64_t ts = p.tok_stride;
  // The loop runs over 16-token blocks; a page of 16 * 2^psh tokens holds
  // 2^psh of them, block lp at rows 16 * (lp & pmask) of page table[lp >> psh].
  const int psh = __builtin_ctz((unsigned)p.page_size) - 4;
  const int pmask = (1 << psh) - 1;
  const int64_t koff = (int64_t)row * ts + 8 * grp;        // + 32*kb
  const int64_t voff = (int64_t)(4 * grp) * ts + 8 * row;  // + i*ts

  // B operand of S^T = K Q^T: the GQA group's query rows (column = head),
  // kept in this wave's LDS tile (zero rows past G) and read per page, which
  // leaves the registers to the page prefetch.
  {
    const T* qrow = static_cast<const T*>(p.q) + (int64_t)b * p.q_bs + (int64_t)(g * G + row) * p.q_hs;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      vec8 x;
      if (row < G) {
        x = *reinterpret_cast<const vec8*>(qrow + 32 * kb + 8 * grp);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = static_cast<T>(0.0f);
      }
      *reinterpret_cast<vec8*>(qtile + row * kVRow + 32 * kb + 8 * grp) = x;
    }
    wave_lds_sync();
  }

  f32x4 oacc[8];  // O^T[d = 16*blk + 4*grp + i][head = row]
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) oacc[blk] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegInf, l_run = 0.0f;  // softmax state of head `row`

  vec8 kreg[PREF][4], vreg[PREF][4];
  int pid_s[PREF];
  // Per-token fog values of the next page to compute, lane t (< 16) holding
  // token 16*lp + t (0 outside [lo, ctx)).  They are loaded when the previous
  // page is done, before the K/V prefetch issued then, so waiting for them never
  // waits for that prefetch (a load issued at use would: vector loads complete
  // in order).
  float fb_cur = 0.0f, fv_cur = 0.0f;
  const float* fog_b = (FOG & kFogBias) ? p.bias + (int64_t)b * p.bias_bs : nullptr;
  const float* fog_v = (FOG & kFogVs) ? p.vscale + (int64_t)b * p.vs_bs : nullptr;
  auto load_fog = [&](int lp) {
    const int tl = 16 * lp + lane;
    const bool in = lane < 16 && tl >= lo && tl < ctx;
    if (FOG & kFogBias) fb_cur = in ? fog_b[tl] : 0.0f;
    if (FOG & kFogVs) fv_cur = in ? fog_v[tl] : 0.0f;
  };

  auto issue = [&](int st, int lp) {
    const int pid = table[lp >> psh];
    pid_s[st] = pid;
    if (pid >= 0 && pid < p.num_pages) {
      const int64_t at = (int64_t)pid * p.page_stride + (int64_t)((lp & pmask) << 4) * ts;
      const T* kp = kbase + at;
      const T* vp = vbase + at;
      // Non-temporal: each K/V byte is read once per launch (measured 9 % faster
      // than plain loads for this access pattern).
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        kreg[st][kb] = __builtin_nontemporal_load(reinterpret_cast<const vec8*>(kp + koff + 32 * kb));
#pragma unroll
      for (int i = 0; i < 4; ++i) vreg[st][i] = __builtin_nontemporal_load(reinterpret_cast<const vec8*>(vp + voff + i * ts));
    }
  };

#pragma unroll
  for (int st = 0; st < PREF; ++st)
    if (p0 + st < p1) issue(st, p0 + st);
  if (FOG && p0 < p1) load_fog(p0);

  for (int base = p0; base < p1; base += PREF) {
#pragma unroll
    for (int st = 0; st < PREF; ++st) {
      const int lp = base + st;
      if (lp >= p1) break;
      const int pid = pid_s[st];
      if (pid < 0 || pid >= p.num_pages) {  // masked page: contributes nothing
        if (FOG && lp + 1 < p1) load_fog(lp + 1);
        if (lp + PREF < p1) issue(st, lp + PREF);
        continue;
      }
      const int t_page = lp << 4;
      const bool full = t_page >= lo && t_page + 16 <= ctx;
      // Scores: lane (grp, row) holds head `row`, tokens t_page + 4*grp + i.
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const vec8 qv = *reinterpret_cast<const vec8*>(qtile + row * kVRow + 32 * kb + 8 * grp);
        acc = Mfma<T>::mma32(kreg[st][kb], qv, acc);
      }
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t_page + 4 * grp + i;
        const bool ok = full || (t >= lo && t < ctx);
        float s = acc[i] * p.sm_scale;
        if (FOG & kFogBias) s += __shfl(fb_cur, 4 * grp + i);
        sc[i] = ok ? s : kNegInf;
      }
      float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      const float mnew = fmaxf(m_run, mloc);
      const float alpha = (m_run == kNegInf) ? 0.0f : __expf(m_run - mnew);
      float pr[4];
      float psum = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = (sc[i] == kNegInf) ? 0.0f : __expf(sc[i] - mnew);
        psum += pr[i];
      }
      psum += __shfl_xor(psum, 16);
      psum += __shfl_xor(psum, 32);
      l_run = l_run * alpha + psum;
      m_run = mnew;
      if (FOG & kFogVs) {
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] *= __shfl(fv_cur, 4 * grp + i);
      }
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) oacc[blk] *= alpha;
      }
      // V rows of this lane's token quad -> LDS tile (masked tokens as zeros).
      if (!full) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = t_page + 4 * grp + i;
          if (!(t >= lo && t < ctx)) {
#pragma unroll
            for (int e = 0; e < 8; ++e) vreg[st][i][e] = static_cast<T>(0.0f);
          }
        }
      }
      wave_lds_sync();  // the previous page's transposed reads are done
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<vec8*>(vtile + (4 * grp + i) * kVRow + 8 * row) = vreg[st][i];
      wave_lds_sync();
      vec4 pb;
#pragma unroll
      for (int i = 0; i < 4; ++i) pb[i] = static_cast<T>(pr[i]);
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
        vec4 va;
#pragma unroll
        for (int i = 0; i < 4; ++i) va[i] = vtile[(4 * grp + i) * kVRow + 16 * blk + row];
        oacc[blk] = Mfma<T>::mma16(va, pb, oacc[blk]);
      }
      if (FOG && lp + 1 < p1) load_fog(lp + 1);
      if (lp + PREF < p1) issue(st, lp + PREF);
    }
  }

  // Lane (grp, row) holds head `row`, d = 16*blk + 4*grp + i.
  if (row >= G) return;
  const int head = g * G + row;
  if (p.direct_out) {
    const float il = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    T* dst = static_cast<T*>(p.out) + (int64_t)b * p.o_bs + (int64_t)head * p.o_hs + 4 * grp;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      vec4 ov;
#pragma unroll
      for (int i = 0; i < 4; ++i) ov[i] = from_f32<T>(oacc[blk][i] * il);
      *reinterpret_cast<vec4*>(dst + 16 * blk) = ov;
    }
  } else {
    const int64_t slot = p.balanced ? (int64_t)head * S * p.B + unit : row_id(p, b, 0, head) * S + split;
    float* dst = p.ws_o + slot * 128 + 4 * grp;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) *reinterpret_cast<f32x4*>(dst + 16 * blk) = oacc[blk];
    if (grp == 0) {
      p.ws_m[slot] = m_run;
      p.ws_l[slot] = l_run;
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 decode on MFMA (head_dim 128, pages of 16 * 2^k tokens) for GQA ratios
// 8 and 16 (up to 4: decode_f32_4x4_kernel below): the bf16 kernel's
// decomposition with v_mfma_f32_16x16x4_f32 and the probabilities kept in
// fp32 (no rounding of p, so fp32 inputs meet a 1e-5 tolerance).
//   * K: lane (grp, row) loads token `row`'s d = 32*grp .. 32*grp+31 (128
//     contiguous bytes, eight 16-byte loads); MFMA kb (0..31) takes d =
//     32*grp + kb of that token as its A element, and the query element of the
//     same d as B (held in 32 registers), so the 32 MFMAs cover all 128 d;
//   * scores land in the same layout as the bf16 kernel's (lane: head `row`,
//     tokens 4*grp + i), so the softmax is identical;
//   * PV k-step ks takes tokens 4*grp' + ks over the four k lanes: each lane's
//     own p[ks] is its B element with no exchange, and V (staged in LDS as
//     token rows of 132 floats -- two token rows read by one half-wave fall on
//     different banks) supplies A = V[4*grp + ks][16*blk + row].
// ---------------------------------------------------------------------------
constexpr int kVRowF = 132;  // LDS row stride of the fp32 V tile (floats)

template <int G, int PREF, int W, int FOG>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_mfma_f32_kernel(
    Params p) {
  __shared__ __align__(16) float vtile_all[W][16 * kVRowF];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = blockIdx.z * W + wave;
  if (g >= p.Hkv) return;  // no workgroup barriers below
  float* vtile = vtile_all[wave];
  const int S = p.num_splits;
  const int unit = blockIdx.y * S + blockIdx.x;  // balanced splits: this workgroup's unit
  int b = blockIdx.y, split = blockIdx.x, per = 0;
  int ctx;
  if (p.balanced) {
    const BatchPages bp = batch_pages(p);
    per = decode_unit_pages(bp, S, p.B);
    if (!decode_seq_of_unit(bp, per, unit, &b, &split)) return;  // past the batch's units: no partial to write
    // Wave-uniform results, kept in scalar registers so that the page loop's
    // bounds and page-table reads stay scalar (as vector loads they would
    // queue behind the page prefetch).
    per = __builtin_amdgcn_readfirstlane(per);
    b = __builtin_amdgcn_readfirstlane(b);
    split = __builtin_amdgcn_readfirstlane(split);
    ctx = bp.seq_len(b);
  } else {
    ctx = seq_ctx(p, b);
  }
  const int row = lane & 15;
  const int grp = lane >> 4;

  const int lo = p.window > 0 ? max(0, ctx - p.window) : 0;
  const int pg_lo = lo >> 4;
  const int pg_hi = (ctx + 15) >> 4;
  if (!p.balanced) per = (pg_hi - pg_lo + S - 1) / S;
  const int p0 = pg_lo + split * per;
  const int p1 = min(pg_hi, p0 + per);

  const float* kbase = static_cast<const float*>(p.k) + (int64_t)g * p.head_stride;
  const float* vbase = static_cast<const float*>(p.v) + (int64_t)g * p.head_stride;
  const int32_t* table = p.page_table + (int64_t)b * p.table_stride;
  const int64_t ts = p.tok_stride;
  // The loop runs over 16-token blocks; a page of 16 * 2^psh tokens holds
  // 2^psh of them, block lp at rows 16 * (lp & pmask) of page table[lp >> psh].
  const int psh = __builtin_ctz((unsigned)p.page_size) - 4;
  const int pmask = (1 << psh) - 1;
  const int64_t koff = (int64_t)row * ts + 32 * grp;
  const int64_t voff = (int64_t)(4 * grp) * ts + 8 * row;  // + i*ts, +4

  // B operand of QK^T: query element d = 32*grp + kb of head `row` (zero past G).
  f32x4 qreg[8];
  {
    const float* qrow = static_cast<const float*>(p.q) + (int64_t)b * p.q_bs + (int64_t)(g * G + row) * p.q_hs;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      qreg[j] = row < G ? *reinterpret_cast<const f32x4*>(qrow + 32 * grp + 4 * j) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  f32x4 oacc[8];  // O^T[d = 16*blk + 4*grp + i][head = row]
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) oacc[blk] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegInf, l_run = 0.0f;

  f32x4 kreg[PREF][8], vreg[PREF][8];
  int pid_s[PREF];
  float fb_cur = 0.0f, fv_cur = 0.0f;
  const float* fog_b = (FOG & kFogBias) ? p.bias + (int64_t)b * p.bias_bs : nullptr;
  const float* fog_v = (FOG & kFogVs) ? p.vscale + (int64_t)b * p.vs_bs : nullptr;
  auto load_fog = [&](int lp) {
    const int tl = 16 * lp + lane;
    const bool in = lane < 16 && tl >= lo && tl < ctx;
    if (FOG & kFogBias) fb_cur = in ? fog_b[tl] : 0.0f;
    if (FOG & kFogVs) fv_cur = in ? fog_v[tl] : 0.0f;
  };
  auto issue = [&](int st, int lp) {
    const int pid = table[lp >> psh];
    pid_s[st] = pid;
    if (pid >= 0 && pid < p.num_pages) {
      const int64_t at = (int64_t)pid * p.page_stride + (int64_t)((lp & pmask) << 4) * ts;
      const float* kp = kbase + at;
      const float* vp = vbase + at;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        kreg[st][j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(kp + koff + 4 * j));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        vreg[st][2 * i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(vp + voff + i * ts));
        vreg[st][2 * i + 1] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(vp + voff + i * ts + 4));
      }
    }
  };

#pragma unroll
  for (int st = 0; st < PREF; ++st)
    if (p0 + st < p1) issue(st, p0 + st);
  if (FOG && p0 < p1) load_fog(p0);

  for (int base = p0; base < p1; base += PREF) {
#pragma unroll
    for (int st = 0; st < PREF; ++st) {
      const int lp = base + st;
      if (lp >= p1) break;
      const int pid = pid_s[st];
      if (pid < 0 || pid >= p.num_pages) {
        if (FOG && lp + 1 < p1) load_fog(lp + 1);
        if (lp + PREF < p1) issue(st, lp + PREF);
        continue;
      }
      const int t_page = lp << 4;
      const bool full = t_page >= lo && t_page + 16 <= ctx;
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kreg[st][j][e], qreg[j][e], acc, 0, 0, 0);
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t_page + 4 * grp + i;
        const bool ok = full || (t >= lo && t < ctx);
        float s = acc[i] * p.sm_scale;
        if (FOG & kFogBias) s += __shfl(fb_cur, 4 * grp + i);
        sc[i] = ok ? s : kNegInf;
      }
      float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      const float mnew = fmaxf(m_run, mloc);
      const float alpha = (m_run == kNegInf) ? 0.0f : __expf(m_run - mnew);
      float pr[4];
      float psum = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = (sc[i] == kNegInf) ? 0.0f : __expf(sc[i] - mnew);
        psum += pr[i];
      }
      psum += __shfl_xor(psum, 16);
      psum += __shfl_xor(psum, 32);
      l_run = l_run * alpha + psum;
      m_run = mnew;
      if (FOG & kFogVs) {
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] *= __shfl(fv_cur, 4 * grp + i);
      }
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) oacc[blk] *= alpha;
      }
      if (!full) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = t_page + 4 * grp + i;
          if (!(t >= lo && t < ctx)) {
            vreg[st][2 * i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            vreg[st][2 * i + 1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
        }
      }
      wave_lds_sync();  // the previous page's reads are done
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *reinterpret_cast<f32x4*>(vtile + (4 * grp + i) * kVRowF + 8 * row) = vreg[st][2 * i];
        *reinterpret_cast<f32x4*>(vtile + (4 * grp + i) * kVRowF + 8 * row + 4) = vreg[st][2 * i + 1];
      }
      wave_lds_sync();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int blk = 0; blk < 8; ++blk)
          oacc[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(vtile[(4 * grp + ks) * kVRowF + 16 * blk + row], pr[ks],
                                                           oacc[blk], 0, 0, 0);
      if (FOG && lp + 1 < p1) load_fog(lp + 1);
      if (lp + PREF < p1) issue(st, lp + PREF);
    }
  }

  // Lane (grp, row) holds head `row`, d = 16*blk + 4*grp + i.
  if (row >= G) return;
  const int head = g * G + row;
  if (p.direct_out) {
    const float il = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    float* dst = static_cast<float*>(p.out) + (int64_t)b * p.o_bs + (int64_t)head * p.o_hs + 4 * grp;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) *reinterpret_cast<f32x4*>(dst + 16 * blk) = oacc[blk] * il;
  } else {
    const int64_t slot = p.balanced ? (int64_t)head * S * p.B + unit : row_id(p, b, 0, head) * S + split;
    float* dst = p.ws_o + slot * 128 + 4 * grp;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) *reinterpret_cast<f32x4*>(dst + 16 * blk) = oacc[blk];
    if (grp == 0) {
      p.ws_m[slot] = m_run;
      p.ws_l[slot] = l_run;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Compute units of the current device, cached per device.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Number of key splits per (sequence, kv-head group); identical for the
// workspace query and the launch.  The default targets kDecWgsPerCu
// workgroups per CU, so the decode grid runs as a single round (at batch 16
// with 8 kv heads on 256 CUs: 16 splits of 512 pages; 32 splits, two rounds,
// measured 3 % slower).
int decode_splits(int B, int Hkv, int max_ctx, int page_size) {
  const int target = env_int("KESSIE_DECODE_WGS", kDecWgsPerCu * device_cus());
  const int units = B * div_up(Hkv, kDecWaves);
  // Counted in 16-token blocks, the unit the MFMA decode streams (pages of
  // 16 * 2^k tokens hold 2^k of them); smaller pages count as they are.
  const int pages = div_up(max(max_ctx, 1), max(min(page_size, 16), 1));
  int s = div_up(target, max(units, 1));
  // At least 2 pages per split: short contexts are latency-bound, so more,
  // shorter splits win (one 4K sequence: bf16 step 23.0 -> 17.8 us, fp32
  // 76.8 -> 56.3 us, against 8 pages per split; one page per split is no
  // better for bf16 and loses the fp32 gain).
  s = min(s, max(1, pages / 2));
  s = min(s, kMaxSplits);
  return max(s, 1);
}

// Key splits of the MFMA prefill: enough workgroups for one per CU (one fits a
// CU at a time: 106.5 KiB of LDS), at least 8 key tiles (512 keys) per split.
// A 2,048-query chunk at GQA 4 and 8 kv heads already has 256 workgroups: no
// split.  Under causal masking the chunk's query tiles see max_ctx - C/2 keys
// on average (half the context for a fresh prompt), and the per-split minimum
// counts those: a fresh 1,024-token prompt (128 workgroups) ran 39.5 us
// unsplit against 44.5 us in two splits.  causal false gives the largest
// count, which sizes the workspace.  KESSIE_PREFILL_SPLITS > 0 forces the
// count.
int prefill_mfma_splits(int B, int C, int Hkv, int G, int max_ctx, bool causal) {
  const int forced = env_int("KESSIE_PREFILL_SPLITS", 0);  // 0: sized to fill the chip
  if (forced > 0) return min(forced, kMaxSplits);
  const int per_wg = 256 / max(G, 1);  // query positions per workgroup
  const int units = B * Hkv * div_up(max(C, 1), per_wg);
  const int keys = causal ? max_ctx - max(C, 0) / 2 : max_ctx;
  const int tiles = div_up(max(keys, 1), 64);
  int s = div_up(device_cus(), max(units, 1));
  s = min(s, max(1, tiles / 8));
  s = min(s, kMaxSplits);
  return max(s, 1);
}

int prefill_splits(int B, int C, int Hkv, int G, int max_ctx, int page_size) {
  const int target = env_int("KESSIE_PREFILL_WGS", 1024);
  const int units = B * Hkv * div_up(C * G, kGenRT);
  const int pages = div_up(max(max_ctx, 1), max(min(page_size, 16), 1));  // 16-token blocks, as in decode_splits
  int s = div_up(target, max(units, 1));
  s = min(s, max(1, pages / 8));
  s = min(s, kMaxSplits);
  return max(s, 1);
}


template <typename T>
int launch_generic(Params& p, hipStream_t stream) {
  const int tiles = div_up(p.C * p.G, kGenRT);
  const size_t lds = generic_lds_bytes(p.D);
  if (lds > 48 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(attn_generic_kernel<T>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
      set_error(KESSIE_ERR_HIP, "fog attention: %zu bytes of LDS unavailable for head_dim %d", lds, p.D);
      return KESSIE_ERR_HIP;
    }
  }
  dim3 grid(p.num_splits, tiles, p.B * p.Hkv);
  hipLaunchKernelGGL(attn_generic_kernel<T>, grid, dim3(kGenThreads), lds, stream, p);
  if (check_launch("fog attention (generic)") != KESSIE_OK) return KESSIE_ERR_HIP;
  if (!p.direct_out && p.launch_combine) {
    launch_combine<T>(p, (int64_t)p.B * p.C * p.Hq, stream);
    return check_launch("fog attention (combine)");
  }
  return KESSIE_OK;
}

template <typename T, int G>
int launch_decode_mfma(Params& p, hipStream_t stream) {
  // Two kv heads per workgroup, two pages in flight per wave, two waves per
  // SIMD (measured at batch 16, 128K context: 1.308 ms against 1.314 ms with
  // four pages in flight -- which also cost one sequence 3-9 % -- and 1.398 ms
  // with two pages at three waves per SIMD).
  dim3 grid(p.num_splits, p.B, div_up(p.Hkv, kDecWaves));
  const int fog = (p.bias ? kFogBias : 0) | (p.vscale ? kFogVs : 0);
  const dim3 block(kDecWaves * 64);
  switch (fog) {
    case 0: hipLaunchKernelGGL((decode_mfma_kernel<T, G, kDecPref, kDecWaves, 0>), grid, block, 0, stream, p); break;
    case kFogBias: hipLaunchKernelGGL((decode_mfma_kernel<T, G, kDecPref, kDecWaves, kFogBias>), grid, block, 0, stream, p); break;
    case kFogVs: hipLaunchKernelGGL((decode_mfma_kernel<T, G, kDecPref, kDecWaves, kFogVs>), grid, block, 0, stream, p); break;
    default:
      hipLaunchKernelGGL((decode_mfma_kernel<T, G, kDecPref, kDecWaves, kFogBias | kFogVs>), grid, block, 0, stream, p);
  }
  if (check_launch("fog decode (mfma)") != KESSIE_OK) return KESSIE_ERR_HIP;
  if (!p.direct_out && p.launch_combine) {
    const int64_t rows = (int64_t)p.B * p.Hq;
    launch_row_combine<T>(p, rows, stream);
    return check_launch("fog decode (combine)");
  }
  return KESSIE_OK;
}

// ---------------------------------------------------------------------------
// fp32 decode for GQA ratios up to 4 on v_mfma_f32_4x4x1_16b_f32: 16
// independent 4x4x1 products per instruction, block b = lane / 4; lane 4b + j
// receives column j of block b's result (register r: row r), A comes from
// lane 4b + r and B from lane 4b + j.  The 16x16x4 instance fills 16 head
// columns of which G are live; here every column is:
//   * S: block b = (d-quarter b / 4, token group b % 4), A = K (row r: token
//     4 (b % 4) + r -- the token lane l & 15 loads, d = 32 (l >> 4) + step:
//     the 16x16x4 instance's K loads unchanged), B = Q (column j: head j, zero
//     from G on); 32 steps run through a d-quarter and two shuffles add the
//     quarters, leaving lane l with head l & 3's scores of tokens
//     4 ((l >> 2) & 3) + r in its registers r;
//   * PV: A = p (row r: head r; each lane reads its head's 16 probabilities
//     from a 64-float LDS slot of its wave), B = V (column: d = l in the first
//     product, 64 + l in the second), read from global memory one dword per
//     lane and token, so V needs no transpose; lane l ends with O[head r][l]
//     and O[head r][64 + l] in its registers r.
// ---------------------------------------------------------------------------
template <int G, int PREF, int W, int FOG>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_f32_4x4_kernel(
    Params p) {
  static_assert(G >= 1 && G <= 4, "decode_f32_4x4_kernel: GQA ratio up to 4");
  __shared__ __align__(16) float pslot_all[W][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = blockIdx.z * W + wave;
  if (g >= p.Hkv) return;  // no workgroup barriers below
  float* pslot = pslot_all[wave];
  const int S = p.num_splits;
  const int unit = blockIdx.y * S + blockIdx.x;  // balanced splits: this workgroup's unit
  int b = blockIdx.y, split = blockIdx.x, per = 0;
  int ctx;
  if (p.balanced) {
    const BatchPages bp = batch_pages(p);
    per = decode_unit_pages(bp, S, p.B);
    if (!decode_seq_of_unit(bp, per, unit, &b, &split)) return;  // past the batch's units: no partial to write
    per = __builtin_amdgcn_readfirstlane(per);
    b = __builtin_amdgcn_readfirstlane(b);
    split = __builtin_amdgcn_readfirstlane(split);
    ctx = bp.seq_len(b);
  } else {
    ctx = seq_ctx(p, b);
  }
  const int x = lane & 3;          // head of this lane's scores and probabilities
  const int tg = (lane >> 2) & 3;  // its token group: tokens 4 tg + r
  const int row = lane & 15;       // K: the token it loads
  const int grp = lane >> 4;       // K and Q: its d-quarter

  const int lo = p.window > 0 ? max(0, ctx - p.window) : 0;
  const int pg_lo = lo >> 4;
  const int pg_hi = (ctx + 15) >> 4;
  if (!p.balanced) per = (pg_hi - pg_lo + S - 1) / S;
  const int p0 = pg_lo + split * per;
  const int p1 = min(pg_hi, p0 + per);

  const float* kbase = static_cast<const float*>(p.k) + (int64_t)g * p.head_stride;
  const float* vbase = static_cast<const float*>(p.v) + (int64_t)g * p.head_stride;
  const int32_t* table = p.page_table + (int64_t)b * p.table_stride;
  const int64_t ts = p.tok_stride;
  const int psh = __builtin_ctz((unsigned)p.page_size) - 4;
  const int pmask = (1 << psh) - 1;
  const int64_t koff = (int64_t)row * ts + 32 * grp;

  // B operand of S: Q[head x][d = 32 grp + 4 j + e] (zero from G on).
  f32x4 qreg[8];
  {
    const float* qrow =
        static_cast<const float*>(p.q) + (int64_t)b * p.q_bs + (int64_t)(g * G + min(x, G - 1)) * p.q_hs;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      qreg[j] = x < G ? *reinterpret_cast<const f32x4*>(qrow + 32 * grp + 4 * j) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  f32x4 oacc[2];  // O[head r][d = l + 64 h]
  oacc[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  oacc[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegInf, l_run = 0.0f;  // head x's

  f32x4 kreg[PREF][8];
  float vreg[PREF][32];  // V[token t][d = lane] at t, V[t][64 + lane] at 16 + t
  int pid_s[PREF];
  float fb_cur = 0.0f, fv_cur = 0.0f;
  const float* fog_b = (FOG & kFogBias) ? p.bias + (int64_t)b * p.bias_bs : nullptr;
  const float* fog_v = (FOG & kFogVs) ? p.vscale + (int64_t)b * p.vs_bs : nullptr;
  auto load_fog = [&](int lp) {
    const int tl = 16 * lp + lane;
    const bool in = lane < 16 && tl >= lo && tl < ctx;
    if (FOG & kFogBias) fb_cur = in ? fog_b[tl] : 0.0f;
    if (FOG & kFogVs) fv_cur = in ? fog_v[tl] : 0.0f;
  };
  auto issue = [&](int st, int lp) {
    const int pid = table[lp >> psh];
    pid_s[st] = pid;
    if (pid >= 0 && pid < p.num_pages) {
      const int64_t at = (int64_t)pid * p.page_stride + (int64_t)((lp & pmask) << 4) * ts;
      const float* kp = kbase + at;
      const float* vp = vbase + at + lane;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        kreg[st][j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(kp + koff + 4 * j));
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        vreg[st][t] = __builtin_nontemporal_load(vp + t * ts);
        vreg[st][16 + t] = __builtin_nontemporal_load(vp + t * ts + 64);
      }
    }
  };

#pragma unroll
  for (int st = 0; st < PREF; ++st)
    if (p0 + st < p1) issue(st, p0 + st);
  if (FOG && p0 < p1) load_fog(p0);

  for (int base = p0; base < p1; base += PREF) {
#pragma unroll
    for (int st = 0; st < PREF; ++st) {
      const int lp = base + st;
      if (lp >= p1) break;
      const int pid = pid_s[st];
      if (pid < 0 || pid >= p.num_pages) {
        if (FOG && lp + 1 < p1) load_fog(lp + 1);
        if (lp + PREF < p1) issue(st, lp + PREF);
        continue;
      }
      const int t_page = lp << 4;
      const bool full = t_page >= lo && t_page + 16 <= ctx;
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc = __builtin_amdgcn_mfma_f32_4x4x1f32(kreg[st][j][e], qreg[j][e], acc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {  // the four d-quarters
        acc[r] += __shfl_xor(acc[r], 16);
        acc[r] += __shfl_xor(acc[r], 32);
      }
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t_page + 4 * tg + r;
        const bool ok = full || (t >= lo && t < ctx);
        float s = acc[r] * p.sm_scale;
        if (FOG & kFogBias) s += __shfl(fb_cur, 4 * tg + r);
        sc[r] = ok ? s : kNegInf;
      }
      float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 4));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 8));
      const float mnew = fmaxf(m_run, mloc);
      const float alpha = (m_run == kNegInf) ? 0.0f : __expf(m_run - mnew);
      float pr[4];
      float psum = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = (sc[r] == kNegInf) ? 0.0f : __expf(sc[r] - mnew);
        psum += pr[r];
      }
      psum += __shfl_xor(psum, 4);
      psum += __shfl_xor(psum, 8);
      l_run = l_run * alpha + psum;
      m_run = mnew;
      if (FOG & kFogVs) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] *= __shfl(fv_cur, 4 * tg + r);
      }
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // head r's factor, from lane r
          const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), r));
          oacc[0][r] *= a;
          oacc[1][r] *= a;
        }
      }
      if (!full) {  // tokens outside [lo, ctx) may hold anything: zero their V
#pragma unroll
        for (int t = 0; t < 16; ++t)
          if (!(t_page + t >= lo && t_page + t < ctx)) {
            vreg[st][t] = 0.0f;
            vreg[st][16 + t] = 0.0f;
          }
      }
      // p to the wave's LDS slot ([head][token]); each lane reads its head's 16.
      wave_lds_sync();  // the previous block's reads are done
      if (grp == 0) *reinterpret_cast<f32x4*>(pslot + 16 * x + 4 * tg) = f32x4{pr[0], pr[1], pr[2], pr[3]};
      wave_lds_sync();
      f32x4 pt[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) pt[k] = *reinterpret_cast<const f32x4*>(pslot + 16 * x + 4 * k);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        oacc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(pt[t >> 2][t & 3], vreg[st][t], oacc[0], 0, 0, 0);
        oacc[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(pt[t >> 2][t & 3], vreg[st][16 + t], oacc[1], 0, 0, 0);
      }
      if (FOG && lp + 1 < p1) load_fog(lp + 1);
      if (lp + PREF < p1) issue(st, lp + PREF);
    }
  }

  // Lane l holds O[head r][l] and O[head r][64 + l] (r < G live); lane r holds
  // head r's running max and sum.
#pragma unroll
  for (int r = 0; r < G; ++r) {
    const int head = g * G + r;
    if (p.direct_out) {
      const float lr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_run), r));
      const float il = lr > 0.0f ? 1.0f / lr : 0.0f;
      float* dst = static_cast<float*>(p.out) + (int64_t)b * p.o_bs + (int64_t)head * p.o_hs;
      dst[lane] = oacc[0][r] * il;
      dst[64 + lane] = oacc[1][r] * il;
    } else {
      const int64_t slot = p.balanced ? (int64_t)head * S * p.B + unit : row_id(p, b, 0, head) * S + split;
      float* dst = p.ws_o + slot * 128;
      dst[lane] = oacc[0][r];
      dst[64 + lane] = oacc[1][r];
      if (lane == r) {
        p.ws_m[slot] = m_run;
        p.ws_l[slot] = l_run;
      }
    }
  }
}

template <int G, int PREF, int FOG>
void launch_f32_instance(const Params& p, dim3 grid, dim3 block, hipStream_t stream) {
  if constexpr (G <= 4)
    hipLaunchKernelGGL((decode_f32_4x4_kernel<G, PREF, kDecWaves, FOG>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((decode_mfma_f32_kernel<G, PREF, kDecWaves, FOG>), grid, block, 0, stream, p);
}

template <int G>
int launch_decode_mfma_f32(Params& p, hipStream_t stream) {
  dim3 grid(p.num_splits, p.B, div_up(p.Hkv, kDecWaves));
  const int fog = (p.bias ? kFogBias : 0) | (p.vscale ? kFogVs : 0);
  const dim3 block(kDecWaves * 64);
  // Splits of at most two 16-token blocks (short contexts) take the
  // one-block-in-flight instance: less code to fetch, and a 4K-token step
  // 1 us faster although its two blocks then load one after the other.
  const int per = div_up(div_up(max(p.max_ctx, 1), 16), max(p.num_splits, 1));
  if (!p.balanced && per <= 2) {
    switch (fog) {
      case 0: launch_f32_instance<G, 1, 0>(p, grid, block, stream); break;
      case kFogBias: launch_f32_instance<G, 1, kFogBias>(p, grid, block, stream); break;
      case kFogVs: launch_f32_instance<G, 1, kFogVs>(p, grid, block, stream); break;
      default: launch_f32_instance<G, 1, kFogBias | kFogVs>(p, grid, block, stream);
    }
  } else {
    switch (fog) {
      case 0: launch_f32_instance<G, kDecPref, 0>(p, grid, block, stream); break;
      case kFogBias: launch_f32_instance<G, kDecPref, kFogBias>(p, grid, block, stream); break;
      case kFogVs: launch_f32_instance<G, kDecPref, kFogVs>(p, grid, block, stream); break;
      default: launch_f32_instance<G, kDecPref, kFogBias | kFogVs>(p, grid, block, stream);
    }
  }
  if (check_launch("fog decode (mfma fp32)") != KESSIE_OK) return KESSIE_ERR_HIP;
  if (!p.direct_out && p.launch_combine) {
    const int64_t rows = (int64_t)p.B * p.Hq;
    launch_row_combine<float>(p, rows, stream);
    return check_launch("fog decode (combine)");
  }
  return KESSIE_OK;
}

int run_decode_mfma_f32(Params& p, hipStream_t s) {
  switch (p.G) {
    case 1: return launch_decode_mfma_f32<1>(p, s);
    case 2: return launch_decode_mfma_f32<2>(p, s);
    case 4: return launch_decode_mfma_f32<4>(p, s);
    case 8: return launch_decode_mfma_f32<8>(p, s);
    case 16: return launch_decode_mfma_f32<16>(p, s);
  }
  set_error(KESSIE_ERR_UNSUPPORTED, "fog decode: GQA ratio %d", p.G);
  return KESSIE_ERR_UNSUPPORTED;
}

int run_generic(int dtype, Params& p, hipStream_t s) {
  switch (dtype) {
    case KESSIE_DTYPE_F32: return launch_generic<float>(p, s);
    case KESSIE_DTYPE_BF16: return launch_generic<bf16_t>(p, s);
    case KESSIE_DTYPE_F16: return launch_generic<f16_t>(p, s);
  }
  set_error(KESSIE_ERR_UNSUPPORTED, "fog attention: dtype %d", dtype);
  return KESSIE_ERR_UNSUPPORTED;
}

bool decode_mfma_ok(const Params& p, int dtype) {
  if (env_int("KESSIE_FORCE_GENERIC", 0)) return false;
  if (dtype != KESSIE_DTYPE_BF16 && dtype != KESSIE_DTYPE_F16 && dtype != KESSIE_DTYPE_F32) return false;
  // Pages of 16 * 2^k tokens (vLLM's 16, 32, 64, ... token blocks).
  if (p.D != 128 || p.page_size < 16 || (p.page_size & (p.page_size - 1)) != 0 || p.page_table == nullptr)
    return false;
  if (!(p.G == 1 || p.G == 2 || p.G == 4 || p.G == 8 || p.G == 16)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  // 16-byte rows: 8 elements of bf16/fp16, 4 of fp32.
  const int64_t vec = dtype == KESSIE_DTYPE_F32 ? 4 : 8;
  if (p.page_stride % vec || p.tok_stride % vec || p.head_stride % vec || p.q_bs % vec || p.q_hs % vec ||
      p.o_bs % vec || p.o_hs % vec)
    return false;
  return true;
}

template <typename T>
int run_decode_mfma(Params& p, hipStream_t s) {
  switch (p.G) {
    case 1: return launch_decode_mfma<T, 1>(p, s);
    case 2: return launch_decode_mfma<T, 2>(p, s);
    case 4: return launch_decode_mfma<T, 4>(p, s);
    case 8: return launch_decode_mfma<T, 8>(p, s);
    case 16: return launch_decode_mfma<T, 16>(p, s);
  }
  set_error(KESSIE_ERR_UNSUPPORTED, "fog decode: GQA ratio %d", p.G);
  return KESSIE_ERR_UNSUPPORTED;
}

int validate_common(const Params& p, int dtype) {
  KESSIE_REQUIRE(dtype_size(dtype) > 0, KESSIE_ERR_UNSUPPORTED, "fog attention: dtype %d", dtype);
  KESSIE_REQUIRE(p.B >= 0 && p.Hq > 0 && p.Hkv > 0 && p.D > 0, KESSIE_ERR_INVALID,
                 "fog attention: bad sizes B=%d Hq=%d Hkv=%d D=%d", p.B, p.Hq, p.Hkv, p.D);
  KESSIE_REQUIRE(p.Hq % p.Hkv == 0, KESSIE_ERR_INVALID, "fog attention: Hq=%d not a multiple of Hkv=%d", p.Hq,
                 p.Hkv);
  KESSIE_REQUIRE(p.D <= kGenMaxD, KESSIE_ERR_UNSUPPORTED, "fog attention: head_dim %d > %d", p.D, kGenMaxD);
  KESSIE_REQUIRE(p.window >= 0 && p.max_ctx >= 0, KESSIE_ERR_INVALID, "fog attention: window=%d max_ctx=%d",
                 p.window, p.max_ctx);
  KESSIE_REQUIRE(p.q && p.k && p.v && p.out, KESSIE_ERR_INVALID, "fog attention: null q/kv/out");
  KESSIE_REQUIRE(p.page_table == nullptr || (p.page_size > 0 && p.num_pages > 0 && p.table_stride > 0),
                 KESSIE_ERR_INVALID, "fog attention: page_size=%d num_pages=%d table_stride=%lld", p.page_size,
                 p.num_pages, (long long)p.table_stride);
  KESSIE_REQUIRE(p.head_stride >= p.D && p.tok_stride >= (int64_t)p.Hkv * p.head_stride, KESSIE_ERR_INVALID,
                 "fog attention: strides overlap (tok %lld head %lld)", (long long)p.tok_stride,
                 (long long)p.head_stride);
  return KESSIE_OK;
}

}  // namespace attn
}  // namespace kessie

using kessie::attn::Params;

extern "C" size_t kessie_fog_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                                    int max_ctx, int page_size, int dtype) {
  (void)dtype;
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  const int S = kessie::attn::decode_splits(batch, num_kv_heads, max_ctx, page_size);
  return kessie::attn::partial_bytes((int64_t)batch * num_q_heads, S, head_dim);
}

namespace kessie {
namespace attn {

// Shared body of the decode entry points.  partials_only: write (m, l, o) per
// split into the workspace and skip the combine.
static int decode_entry(const void* q, const void* kv_pool, int num_pages, int64_t page_stride, int64_t tok_stride,
                        int64_t kv_stride, int64_t head_stride, const int32_t* page_table, int64_t table_stride,
                        const int32_t* ctx_lens, const float* fog_vscale, int64_t fog_vscale_bstride,
                        const float* fog_bias, int64_t fog_bias_bstride, void* out, int batch, int num_q_heads,
                        int num_kv_heads, int head_dim, int page_size, int max_ctx, int window, float sm_scale,
                        int dtype, void* workspace, size_t workspace_bytes, void* stream, bool partials_only) {
  clear_error();
  Params p{};
  const int es = dtype_size(dtype);
  p.q = q;
  p.q_bs = (int64_t)num_q_heads * head_dim;
  p.q_is = 0;
  p.q_hs = head_dim;
  p.out = partials_only ? const_cast<void*>(q) : out;  // validated non-null; never written in that mode
  p.o_bs = p.q_bs;
  p.o_is = 0;
  p.o_hs = head_dim;
  p.k = kv_pool;
  p.v = kv_pool ? static_cast<const char*>(kv_pool) + kv_stride * es : nullptr;
  p.num_pages = num_pages;
  p.page_stride = page_stride;
  p.tok_stride = tok_stride;
  p.head_stride = head_stride;
  p.page_size = page_size;
  p.page_table = page_table;
  p.table_stride = table_stride;
  p.ctx_lens = ctx_lens;
  p.ctx_const = max_ctx;
  p.max_ctx = max_ctx;
  p.vscale = fog_vscale;
  p.vs_bs = fog_vscale_bstride;
  p.bias = fog_bias;
  p.bias_bs = fog_bias_bstride;
  p.B = batch;
  p.C = 1;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.G = num_kv_heads > 0 ? num_q_heads / num_kv_heads : 0;
  p.D = head_dim;
  p.window = window;
  p.causal = 1;
  p.sm_scale = sm_scale;
  int st = validate_common(p, dtype);
  if (st != KESSIE_OK) return st;
  KESSIE_REQUIRE(page_table != nullptr && ctx_lens != nullptr, KESSIE_ERR_INVALID,
                 "fog decode: page_table and ctx_lens are required");
  KESSIE_REQUIRE(kv_stride >= 0, KESSIE_ERR_INVALID, "fog decode: kv_stride %lld", (long long)kv_stride);
  if (batch == 0) return KESSIE_OK;
  p.num_splits = decode_splits(batch, num_kv_heads, max_ctx, page_size);
  p.direct_out = (!partials_only && p.num_splits == 1) ? 1 : 0;
  p.launch_combine = partials_only ? 0 : 1;
  if (!p.direct_out) {
    const size_t need = partial_bytes((int64_t)batch * num_q_heads, p.num_splits, head_dim);
    KESSIE_REQUIRE(workspace != nullptr && workspace_bytes >= need, KESSIE_ERR_WORKSPACE,
                   "fog decode: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
    KESSIE_REQUIRE(aligned16(workspace), KESSIE_ERR_INVALID, "fog decode: workspace not 16-byte aligned");
    carve_workspace(p, workspace, (int64_t)batch * num_q_heads);
  }
  hipStream_t s = as_stream(stream);
  if (decode_mfma_ok(p, dtype)) {
    // Split partials merged here: assign the splits by pages across the batch
    // (the partials-only form keeps the plain row * S + split layout).  Its
    // set-up costs each wave ~1 us before the first page load, so it is taken
    // for batches of 2..kBalSeqs sequences whose bound on the K/V bytes (B *
    // max_ctx tokens) streams for at least ~40 us, 256 MiB; one sequence, or a
    // batch that small, gets the plain split.
    const double kv_bound = (double)batch * max_ctx * num_kv_heads * head_dim * 2.0 * dtype_size(dtype);
    p.balanced = (!partials_only && !p.direct_out && batch >= 2 && batch <= kBalSeqs &&
                  kv_bound >= 256.0 * 1024 * 1024) ? 1 : 0;
    if (dtype == KESSIE_DTYPE_F32) return run_decode_mfma_f32(p, s);
    return dtype == KESSIE_DTYPE_BF16 ? run_decode_mfma<bf16_t>(p, s) : run_decode_mfma<f16_t>(p, s);
  }
  return run_generic(dtype, p, s);
}

}  // namespace attn
}  // namespace kessie

extern "C" int kessie_fog_decode_paged(const void* q, const void* kv_pool, int num_pages, int64_t page_stride,
                                       int64_t tok_stride, int64_t kv_stride, int64_t head_stride,
                                       const int32_t* page_table, int64_t table_stride, const int32_t* ctx_lens,
                                       const float* fog_vscale, int64_t fog_vscale_bstride, const float* fog_bias,
                                       int64_t fog_bias_bstride, void* out, int batch, int num_q_heads,
                                       int num_kv_heads, int head_dim, int page_size, int max_ctx, int window,
                                       float sm_scale, int dtype, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  return kessie::attn::decode_entry(q, kv_pool, num_pages, page_stride, tok_stride, kv_stride, head_stride,
                                    page_table, table_stride, ctx_lens, fog_vscale, fog_vscale_bstride, fog_bias,
                                    fog_bias_bstride, out, batch, num_q_heads, num_kv_heads, head_dim, page_size,
                                    max_ctx, window, sm_scale, dtype, workspace, workspace_bytes, stream, false);
}

extern "C" int kessie_fog_decode_partials(const void* q, const void* kv_pool, int num_pages, int64_t page_stride,
                                          int64_t tok_stride, int64_t kv_stride, int64_t head_stride,
                                          const int32_t* page_table, int64_t table_stride, const int32_t* ctx_lens,
                                          const float* fog_vscale, int64_t fog_vscale_bstride,
                                          const float* fog_bias, int64_t fog_bias_bstride, int batch,
                                          int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                          int max_ctx, int window, float sm_scale, int dtype, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  return kessie::attn::decode_entry(q, kv_pool, num_pages, page_stride, tok_stride, kv_stride, head_stride,
                                    page_table, table_stride, ctx_lens, fog_vscale, fog_vscale_bstride, fog_bias,
                                    fog_bias_bstride, nullptr, batch, num_q_heads, num_kv_heads, head_dim,
                                    page_size, max_ctx, window, sm_scale, dtype, workspace, workspace_bytes, stream,
                                    true);
}

// ---------------------------------------------------------------------------
// Decode that allocates nothing: the split partials go to a file-scope device
// array instead of a caller workspace (for callers that cannot allocate:
// code under graph capture, tight serving loops).  Each GPU holds its own copy
// of the array, at its own address, until the process ends; host code uses
// that address (from hipGetSymbolAddress, once per device), never the array's
// name.  Calls that overlap on one GPU share the array and race.  The decode
// kernels write every partial of every (row, split) on each call, so nothing
// needs clearing between calls.
// ---------------------------------------------------------------------------
namespace {
static __device__ __align__(256) unsigned char scratch[KESSIE_DECODE_NOALLOC_SCRATCH_BYTES];
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];  // device address of `scratch`, per device ordinal

// Address of this device's copy of `scratch` (looked up on the first call on
// the device, with that device current), or nullptr with the error recorded.
void* device_scratch() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    kessie::set_error(KESSIE_ERR_HIP, "fog decode (no-alloc): hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= 64) {
    kessie::set_error(KESSIE_ERR_UNSUPPORTED, "fog decode (no-alloc): device ordinal %d", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      kessie::set_error(KESSIE_ERR_HIP, "fog decode (no-alloc): hipGetSymbolAddress: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int kessie_fog_decode_paged_noalloc(const void* q, const void* kv_pool, int num_pages,
                                               int64_t page_stride, int64_t tok_stride, int64_t kv_stride,
                                               int64_t head_stride, const int32_t* page_table, int64_t table_stride,
                                               const int32_t* ctx_lens, const float* fog_vscale,
                                               int64_t fog_vscale_bstride, const float* fog_bias,
                                               int64_t fog_bias_bstride, void* out, int batch, int num_q_heads,
                                               int num_kv_heads, int head_dim, int page_size, int max_ctx,
                                               int window, float sm_scale, int dtype, void* stream) {
  using namespace kessie;
  clear_error();
  if (batch > 0 && num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0) {
    const int S = attn::decode_splits(batch, num_kv_heads, max_ctx, page_size);
    const size_t need = S > 1 ? attn::partial_bytes((int64_t)batch * num_q_heads, S, head_dim) : 0;
    KESSIE_REQUIRE(need <= (size_t)KESSIE_DECODE_NOALLOC_SCRATCH_BYTES, KESSIE_ERR_WORKSPACE,
                   "fog decode (no-alloc): %zu bytes of split partials needed for B=%d Hq=%d ctx=%d, more than "
                   "the %zu-byte static scratch; call kessie_fog_decode_paged with a workspace",
                   need, batch, num_q_heads, max_ctx, (size_t)KESSIE_DECODE_NOALLOC_SCRATCH_BYTES);
  }
  void* ws = device_scratch();
  if (ws == nullptr) return last_status();
  return attn::decode_entry(q, kv_pool, num_pages, page_stride, tok_stride, kv_stride, head_stride, page_table,
                            table_stride, ctx_lens, fog_vscale, fog_vscale_bstride, fog_bias, fog_bias_bstride, out,
                            batch, num_q_heads, num_kv_heads, head_dim, page_size, max_ctx, window, sm_scale, dtype,
                            ws, KESSIE_DECODE_NOALLOC_SCRATCH_BYTES, stream, false);
}

extern "C" int kessie_fog_decode_num_splits(int batch, int num_kv_heads, int max_ctx, int page_size) {
  if (batch <= 0 || num_kv_heads <= 0) return 0;
  return kessie::attn::decode_splits(batch, num_kv_heads, max_ctx, page_size);
}

extern "C" int kessie_fog_decode_combine(const void* workspace, size_t workspace_bytes, void* out, int batch,
                                         int num_q_heads, int num_kv_heads, int head_dim, int max_ctx,
                                         int page_size, int dtype, void* stream) {
  using namespace kessie;
  using namespace kessie::attn;
  clear_error();
  KESSIE_REQUIRE(batch >= 0 && num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0, KESSIE_ERR_INVALID,
                 "fog decode combine: bad sizes");
  KESSIE_REQUIRE(dtype_size(dtype) > 0, KESSIE_ERR_UNSUPPORTED, "fog decode combine: dtype %d", dtype);
  if (batch == 0) return KESSIE_OK;
  KESSIE_REQUIRE(out != nullptr, KESSIE_ERR_INVALID, "fog decode combine: null output");
  Params p{};
  p.out = out;
  p.o_bs = (int64_t)num_q_heads * head_dim;
  p.o_is = 0;
  p.o_hs = head_dim;
  p.B = batch;
  p.C = 1;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.D = head_dim;
  p.num_splits = decode_splits(batch, num_kv_heads, max_ctx, page_size);
  const int64_t rows = (int64_t)batch * num_q_heads;
  const size_t need = partial_bytes(rows, p.num_splits, head_dim);
  KESSIE_REQUIRE(workspace != nullptr && workspace_bytes >= need, KESSIE_ERR_WORKSPACE,
                 "fog decode combine: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
  carve_workspace(p, const_cast<void*>(workspace), rows);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case KESSIE_DTYPE_F32: launch_row_combine<float>(p, rows, s); break;
    case KESSIE_DTYPE_BF16: launch_row_combine<bf16_t>(p, rows, s); break;
    default: launch_row_combine<f16_t>(p, rows, s); break;
  }
  return check_launch("fog decode combine");
}

extern "C" size_t kessie_fog_prefill_workspace_bytes(int batch, int num_q_tokens, int num_q_heads, int num_kv_heads,
                                                     int head_dim, int max_ctx, int page_size, int dtype) {
  (void)dtype;
  if (batch <= 0 || num_q_tokens <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  const int G = num_q_heads / num_kv_heads;
  const int S = max(max(kessie::attn::prefill_splits(batch, num_q_tokens, num_kv_heads, G, max_ctx, page_size),
                        kessie::attn::prefill_mfma_splits(batch, num_q_tokens, num_kv_heads, G, max_ctx, false)),
                    kessie::attn::prefill_f32_splits(batch, num_q_tokens, num_kv_heads, G, max_ctx));
  return kessie::attn::partial_bytes((int64_t)batch * num_q_tokens * num_q_heads, S, head_dim);
}

// MFMA prefill for p.B sequences of up to p.C queries: one pass over the keys;
// split-K (partials + combine) when the chunks alone would leave CUs idle.
// Partial rows are (b*C + i)*Hq + h; with q_start the combine skips rows past a
// sequence's chunk and writes the rest at its packed offset.
// fp32 chunked prefill on the fp32 MFMA kernel (per-sequence or varlen
// batches alike): key splits when the chunks alone leave CUs idle, their
// partials merged by the combine.
static int run_prefill_f32(kessie::attn::Params& p, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace kessie;
  using namespace kessie::attn;
  p.num_splits = prefill_f32_splits(p.B, p.C, p.Hkv, p.G, p.max_ctx);
  p.direct_out = p.num_splits == 1 ? 1 : 0;
  const int64_t rows = (int64_t)p.B * p.C * p.Hq;
  if (!p.direct_out) {
    const size_t need = partial_bytes(rows, p.num_splits, p.D);
    KESSIE_REQUIRE(workspace != nullptr && workspace_bytes >= need, KESSIE_ERR_WORKSPACE,
                   "fog prefill: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
    KESSIE_REQUIRE(aligned16(workspace), KESSIE_ERR_INVALID, "fog prefill: workspace not 16-byte aligned");
    carve_workspace(p, workspace, rows);
  }
  const hipStream_t s = as_stream(stream);
  const int st = prefill_f32(p, s);
  if (st != KESSIE_OK || p.direct_out) return st;
  launch_combine<float>(p, rows, s);
  return check_launch("fog prefill (combine)");
}

static int run_prefill_mfma(kessie::attn::Params& p, int dtype, void* workspace, size_t workspace_bytes,
                            void* stream) {
  using namespace kessie;
  using namespace kessie::attn;
  p.num_splits = prefill_mfma_splits(p.B, p.C, p.Hkv, p.G, p.max_ctx, p.causal != 0);
  p.direct_out = p.num_splits == 1 ? 1 : 0;
  p.launch_combine = 0;
  // Longest query tiles first when the causal triangle dominates (the chunk is
  // at least half its context) and the grid takes more than one round: +4-11 %
  // on fresh prompts; with one round it only costs.
  const int64_t wgs = (int64_t)div_up(p.C, 256 / p.G) * p.Hkv * p.B;
  p.reverse_q = p.causal && p.direct_out && !p.q_start && wgs > device_cus() && 2 * (int64_t)p.C >= p.max_ctx;
  const int64_t rows = (int64_t)p.B * p.C * p.Hq;
  if (!p.direct_out) {
    const size_t need = partial_bytes(rows, p.num_splits, p.D);
    KESSIE_REQUIRE(workspace != nullptr && workspace_bytes >= need, KESSIE_ERR_WORKSPACE,
                   "fog prefill: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
    KESSIE_REQUIRE(aligned16(workspace), KESSIE_ERR_INVALID, "fog prefill: workspace not 16-byte aligned");
    carve_workspace(p, workspace, rows);
  }
  const hipStream_t s = as_stream(stream);
  const int st = prefill_mfma(p, dtype, s);
  if (st != KESSIE_OK || p.direct_out) return st;
  if (dtype == KESSIE_DTYPE_BF16)
    launch_combine<bf16_t>(p, rows, s);
  else
    launch_combine<f16_t>(p, rows, s);
  return check_launch("fog prefill (combine)");
}

extern "C" int kessie_fog_prefill_paged(const void* q, const void* kv_pool, int num_pages, int64_t page_stride,
                                        int64_t tok_stride, int64_t kv_stride, int64_t head_stride,
                                        const int32_t* page_table, int64_t table_stride, const int32_t* ctx_lens,
                                        const float* fog_vscale, int64_t fog_vscale_bstride, const float* fog_bias,
                                        int64_t fog_bias_bstride, void* out, int batch, int num_q_tokens,
                                        int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                        int max_ctx, int window, float sm_scale, int causal, int dtype,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  using namespace kessie;
  using namespace kessie::attn;
  clear_error();
  Params p{};
  const int es = dtype_size(dtype);
  p.q = q;
  p.q_bs = (int64_t)num_q_tokens * num_q_heads * head_dim;
  p.q_is = (int64_t)num_q_heads * head_dim;
  p.q_hs = head_dim;
  p.out = out;
  p.o_bs = p.q_bs;
  p.o_is = p.q_is;
  p.o_hs = head_dim;
  p.k = kv_pool;
  p.v = kv_pool ? static_cast<const char*>(kv_pool) + kv_stride * es : nullptr;
  p.num_pages = num_pages;
  p.page_stride = page_stride;
  p.tok_stride = tok_stride;
  p.head_stride = head_stride;
  p.page_size = page_size;
  p.page_table = page_table;
  p.table_stride = table_stride;
  p.ctx_lens = ctx_lens;
  p.ctx_const = max_ctx;
  p.max_ctx = max_ctx;
  p.vscale = fog_vscale;
  p.vs_bs = fog_vscale_bstride;
  p.bias = fog_bias;
  p.bias_bs = fog_bias_bstride;
  p.B = batch;
  p.C = num_q_tokens;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.G = num_kv_heads > 0 ? num_q_heads / num_kv_heads : 0;
  p.D = head_dim;
  p.window = window;
  p.causal = causal ? 1 : 0;
  p.sm_scale = sm_scale;
  int st = validate_common(p, dtype);
  if (st != KESSIE_OK) return st;
  KESSIE_REQUIRE(num_q_tokens > 0, KESSIE_ERR_INVALID, "fog prefill: num_q_tokens %d", num_q_tokens);
  KESSIE_REQUIRE(page_table != nullptr && ctx_lens != nullptr, KESSIE_ERR_INVALID,
                 "fog prefill: page_table and ctx_lens are required");
  KESSIE_REQUIRE(kv_stride >= 0, KESSIE_ERR_INVALID, "fog prefill: kv_stride %lld", (long long)kv_stride);
  if (batch == 0) return KESSIE_OK;
  if (prefill_mfma_ok(p, dtype)) return run_prefill_mfma(p, dtype, workspace, workspace_bytes, stream);
  if (prefill_f32_ok(p, dtype)) return run_prefill_f32(p, workspace, workspace_bytes, stream);
  p.num_splits = prefill_splits(batch, num_q_tokens, num_kv_heads, p.G, max_ctx, page_size);
  p.direct_out = p.num_splits == 1 ? 1 : 0;
  p.launch_combine = 1;
  const int64_t rows = (int64_t)batch * num_q_tokens * num_q_heads;
  const size_t need = partial_bytes(rows, p.num_splits, head_dim);
  if (!p.direct_out) {
    KESSIE_REQUIRE(workspace != nullptr && workspace_bytes >= need, KESSIE_ERR_WORKSPACE,
                   "fog prefill: workspace of %zu bytes needed, got %zu", need, workspace_bytes);
    KESSIE_REQUIRE(aligned16(workspace), KESSIE_ERR_INVALID, "fog prefill: workspace not 16-byte aligned");
    carve_workspace(p, workspace, rows);
  }
  return run_generic(dtype, p, as_stream(stream));
}

extern "C" int kessie_fog_prefill_varlen(const void* q, const int32_t* query_start_loc, int max_query_len,
                                         const void* kv_pool, int num_pages, int64_t page_stride, int64_t tok_stride,
                                         int64_t kv_stride, int64_t head_stride, const int32_t* page_table,
                                         int64_t table_stride, const int32_t* ctx_lens, const float* fog_vscale,
                                         int64_t fog_vscale_bstride, const float* fog_bias, int64_t fog_bias_bstride,
                                         void* out, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                         int page_size, int max_ctx, int window, float sm_scale, int causal,
                                         int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace kessie;
  using namespace kessie::attn;
  clear_error();
  Params p{};
  const int es = dtype_size(dtype);
  p.q = q;
  p.q_is = (int64_t)num_q_heads * head_dim;
  p.q_hs = head_dim;
  p.out = out;
  p.o_is = p.q_is;
  p.o_hs = head_dim;
  p.k = kv_pool;
  p.v = kv_pool ? static_cast<const char*>(kv_pool) + kv_stride * es : nullptr;
  p.num_pages = num_pages;
  p.page_stride = page_stride;
  p.tok_stride = tok_stride;
  p.head_stride = head_stride;
  p.page_size = page_size;
  p.page_table = page_table;
  p.table_stride = table_stride;
  p.ctx_lens = ctx_lens;
  p.ctx_const = max_ctx;
  p.max_ctx = max_ctx;
  p.vscale = fog_vscale;
  p.vs_bs = fog_vscale_bstride;
  p.bias = fog_bias;
  p.bias_bs = fog_bias_bstride;
  p.B = batch;
  p.C = max_query_len;
  p.q_start = query_start_loc;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.G = num_kv_heads > 0 ? num_q_heads / num_kv_heads : 0;
  p.D = head_dim;
  p.window = window;
  p.causal = causal ? 1 : 0;
  p.sm_scale = sm_scale;
  int st = validate_common(p, dtype);
  if (st != KESSIE_OK) return st;
  KESSIE_REQUIRE(max_query_len >= 0, KESSIE_ERR_INVALID, "fog prefill varlen: max_query_len %d", max_query_len);
  KESSIE_REQUIRE(page_table != nullptr && ctx_lens != nullptr && query_start_loc != nullptr, KESSIE_ERR_INVALID,
                 "fog prefill varlen: page_table, ctx_lens and query_start_loc are required");
  KESSIE_REQUIRE(kv_stride >= 0, KESSIE_ERR_INVALID, "fog prefill varlen: kv_stride %lld", (long long)kv_stride);
  if (batch == 0 || max_query_len == 0) return KESSIE_OK;
  if (prefill_f32_ok(p, dtype)) return run_prefill_f32(p, workspace, workspace_bytes, stream);
  KESSIE_REQUIRE(prefill_mfma_ok(p, dtype), KESSIE_ERR_UNSUPPORTED,
                 "fog prefill varlen: shape not taken by the MFMA kernels (bf16/fp16: head_dim 128, pages of 16*2^k "
                 "tokens, GQA 1/2/4/8/16; fp32: head_dim 128, pages of 16*2^k tokens, GQA up to 128; 16-byte aligned "
                 "rows)");
  return run_prefill_mfma(p, dtype, workspace, workspace_bytes, stream);
}

// Reference launchers (kessie_kernels_v2.hip:716-751, 788-825): dense fp16
// [B,H,N,D], no GQA, every position a query.  One split, so no workspace.
namespace kessie {
namespace attn {
namespace {
// Key splits of the dense launchers' MFMA kernel.  Every position is a query,
// so with causal masking a query tile's key tiles grow with its position: the
// longest tile (dispatched first) can take twice the chip's average share,
// and a small B*H leaves most CUs without a tile at all.  Each query tile's
// keys are split S ways, from the longest tile's key tiles over the per-CU
// share of all key tiles, with at least 2 key tiles per split; 1 when the
// grid alone balances (B=1 H=32 N=8,192 causal: 1,024 workgroups over 256
// CUs).  Returns S and, in *split_q0, the first position of the split tiles.
// KESSIE_DENSE_SPLITS > 0 forces the count (tests).
int dense_splits(int B, int H, int N, int window, int causal, int* split_q0) {
  *split_q0 = 0;
  const int kt = div_up(N, 64);  // key tiles of the whole sequence
  const int nq = div_up(N, 256);
  std::vector<int> tiles(nq);
  int64_t total = 0;
  int longest = 0;
  for (int t = 0; t < nq; ++t) {
    const int q0 = 256 * t, q1 = min(N, q0 + 256) - 1;
    int hi = causal ? q1 + 1 : N;
    int lo = 0;
    if (window > 0) {
      lo = max(0, q0 - window + 1);
      hi = min(hi, q1 + 1);
    }
    tiles[t] = hi > lo ? div_up(hi, 64) - lo / 64 : 0;
    total += tiles[t];
    longest = max(longest, tiles[t]);
  }
  total *= (int64_t)B * H;
  const double share = (double)total / device_cus();
  // Every query tile is split (split_q0 0).  Splitting only the tiles longer
  // than the share saves their partial rows but dispatches the long tiles'
  // later splits behind whole short tiles: N=8,192 ran 245-256 us against
  // 230 us.
  const int forced = env_int("KESSIE_DENSE_SPLITS", 0);  // testing: > 0 forces the count
  if (forced > 0) return min(forced, min(kt, kMaxSplits));
  if (longest <= 0 || share <= 0.0) return 1;
  // Each split adds a partial row per query of a split tile (written, then
  // read by the combine), which outweighs the balance gained past a few
  // splits: on the reference's benchmark (B=1, H=8, causal; forced counts 1,
  // 2, 4, 8) the best were 2 where the longest tile is 1.9-3.8 times the
  // share (N=4,096-8,192 full, N=4,096 W=1,024) and 4 from 5.3 times on
  // (N=512-2,048, full and W=1,024), down to 2 key tiles per split (N=512:
  // 22.4 us against 24.1 with 4 tiles per split).
  const double ratio = longest / share;
  if (ratio < 1.5) return 1;
  int s = ratio >= 5.0 ? 4 : 2;
  s = min(s, max(1, longest / 2));
  s = min(s, min(kt, kMaxSplits));
  return max(s, 1);
}

// Device buffer for the dense launchers' split partials, per device and
// stream (calls on one stream run in order, so they can share it), allocated
// on first need and kept until the process ends; an outgrown buffer is kept
// too (a graph captured with it may replay).  Under stream capture nothing is
// allocated: nullptr unless the stream's buffer is already large enough.
std::mutex g_dense_mu;
std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> g_dense_ws;
std::vector<void*> g_dense_retired;

void* dense_workspace(size_t bytes, hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_dense_mu);
  auto& e = g_dense_ws[{dev, s}];
  if (e.first != nullptr && e.second >= bytes) return e.first;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
  void* ptr = nullptr;
  if (hipMalloc(&ptr, bytes) != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (e.first != nullptr) g_dense_retired.push_back(e.first);
  e = {ptr, bytes};
  return ptr;
}
}  // namespace
}  // namespace attn
}  // namespace kessie

static void dense_fp16(const void* Q, const void* K, const void* V, void* O, const void* fog, float sm_scale,
                       int B, int H, int N, int D, int window, int causal, void* stream) {
  using namespace kessie;
  using namespace kessie::attn;
  clear_error();
  Params p{};
  const int64_t bs = (int64_t)H * N * D;
  p.q = Q;
  p.q_bs = bs;
  p.q_is = D;
  p.q_hs = (int64_t)N * D;
  p.out = O;
  p.o_bs = bs;
  p.o_is = D;
  p.o_hs = (int64_t)N * D;
  p.k = K;
  p.v = V;
  p.num_pages = B;
  p.page_stride = bs;
  p.tok_stride = D;
  p.head_stride = (int64_t)N * D;
  p.page_size = N;
  p.page_table = nullptr;
  p.ctx_const = N;
  p.max_ctx = N;
  p.vscale = static_cast<const float*>(fog);
  p.vs_bs = 0;
  p.B = B;
  p.C = N;
  p.Hq = H;
  p.Hkv = H;
  p.G = 1;
  p.D = D;
  p.window = window;
  p.causal = causal ? 1 : 0;
  p.sm_scale = sm_scale;
  p.num_splits = 1;
  p.direct_out = 1;
  p.launch_combine = 0;
  if (D != 64 && D != 128) {
    set_error(KESSIE_ERR_UNSUPPORTED, "dense attention: head_dim=%d unsupported (64 or 128)", D);
    return;
  }
  if (B <= 0 || H <= 0 || N <= 0) {
    if (B < 0 || H < 0 || N < 0) set_error(KESSIE_ERR_INVALID, "dense attention: B=%d H=%d N=%d", B, H, N);
    return;
  }
  // validate_common requires tok_stride >= Hkv*head_stride, which the
  // head-major dense layout does not satisfy; check what applies here.
  if (!Q || !K || !V || !O || window < 0) {
    set_error(KESSIE_ERR_INVALID, "dense attention: null pointer or window %d", window);
    return;
  }
  // head_dim 128 or 64: the MFMA prefill kernel, reading the dense tensors as
  // table-less 16-token pages (page b*H*N/16 + j = tokens 16j..16j+15 of every
  // head of sequence b, heads N*D apart; H*N a multiple of 16 keeps sequences
  // on whole pages, and the kernel reads no token past N).  Key splits
  // (partials merged by the combine kernel) when the grid alone would leave
  // CUs idle, in the library's per-stream buffer (these launchers take no
  // workspace); without one, a single split.
  const int64_t dense_pages = (int64_t)B * H * N / 16;
  if (((int64_t)H * N) % 16 == 0 && dense_pages <= INT_MAX) {
    Params m = p;
    m.page_size = 16;
    m.page_stride = 16 * (int64_t)D;
    m.num_pages = (int)dense_pages;
    m.dense_ppb = (int)(((int64_t)H * N) / 16);
    if (prefill_mfma_ok(m, KESSIE_DTYPE_F16)) {
      const hipStream_t s = as_stream(stream);
      int split_q0 = 0;
      const int S = dense_splits(B, H, N, window, causal, &split_q0);
      const int64_t rows = (int64_t)B * (N - split_q0) * H;  // partial rows: the split tiles' queries
      const size_t need = partial_bytes(rows, S, D);
      void* ws = S > 1 && need <= ((size_t)1 << 30) ? dense_workspace(need, s) : nullptr;
      if (ws != nullptr) {
        m.num_splits = S;
        m.split_q0 = split_q0;
        m.direct_out = 0;
        carve_workspace(m, ws, rows);
        if (prefill_mfma(m, KESSIE_DTYPE_F16, s) != KESSIE_OK) return;  // error recorded
        Params c = m;  // the combine's rows: positions split_q0 .. N-1
        c.C = N - split_q0;
        c.q0_off = split_q0;
        launch_combine<f16_t>(c, rows, s);
        check_launch("dense attention (combine)");
        return;
      }
      prefill_mfma(m, KESSIE_DTYPE_F16, s);  // records any launch error
      return;
    }
  }
  // Testing switch: KESSIE_REQUIRE_MFMA=1 makes a shape that would fall back
  // to the generic kernel an error instead (the tests use it to show which
  // route ran).
  if (env_int("KESSIE_REQUIRE_MFMA", 0)) {
    set_error(KESSIE_ERR_UNSUPPORTED, "dense attention: B=%d H=%d N=%d D=%d runs on the generic kernel", B, H, N, D);
    return;
  }
  launch_generic<f16_t>(p, as_stream(stream));
}

extern "C" void launch_kessie_windowed_attn(const void* Q, const void* K, const void* V, void* O, float sm_scale,
                                            int batch_size, int num_heads, int seq_len, int head_dim,
                                            int window_size, int is_causal, void* stream) {
  dense_fp16(Q, K, V, O, nullptr, sm_scale, batch_size, num_heads, seq_len, head_dim, window_size, is_causal,
             stream);
}

extern "C" void launch_kessie_fused_fog_attn(const void* Q, const void* K, const void* V, void* O,
                                             const void* fog_weights, float sm_scale, int batch_size, int num_heads,
                                             int seq_len, int head_dim, int window_size, int is_causal,
                                             void* stream) {
  if (fog_weights == nullptr) {
    kessie::clear_error();
    kessie::set_error(KESSIE_ERR_INVALID, "fused fog attention: fog_weights is null");
    return;
  }
  dense_fp16(Q, K, V, O, fog_weights, sm_scale, batch_size, num_heads, seq_len, head_dim, window_size, is_causal,
             stream);
}
