// Chunked-prefill fog attention in fp32 on MFMA for gfx950 (head_dim 128,
// pages of 16 * 2^k tokens, any GQA ratio up to 128).  The reference's own
// attention path computes in fp32 (callers upcast, kessie_hip_kernels.py:632,
// 652); this serves those inputs at the fp32 tolerance without the scalar
// generic kernel.
//
// Math: the last C rows of kessie_hip_kernels.py:577-593 over ctx = L + C
// tokens (query i at position ctx-C+i, causal, window, fog weights scaling V
// or a logit bias), fp32 throughout, online softmax in natural units.
//
// Work decomposition: one workgroup = 128 query rows (128/G positions x the
// G heads of one kv head) of one sequence; 8 waves x 16 rows.  Varlen batches
// (query_start_loc) number the live (sequence, query tile) pairs along x.  The workgroup
// streams its kv head's 16-token blocks through a two-stage LDS ring (K and V
// rows, and the block's fog values): every thread loads 16 bytes of K and of
// V of the next block while the waves compute the current one, then stores
// them; one barrier per block.  Per wave and block, on v_mfma_f32_16x16x4_f32
// (as the fp32 decode):
//   S^T (16 keys x 16 rows) = K Q^T: 32 MFMAs, lane (grp, col) reading key
//     col's d = 32 grp .. 32 grp + 31 (contiguous in LDS) against query row
//     col's same d (held in registers), so the 32 MFMAs cover all 128 d; the
//     result puts keys 4 grp + i of row col in lane (grp, col);
//   O^T (128 d x 16 rows) += V^T P^T: 32 MFMAs, k-step ks taking keys
//     4 grp + ks -- each lane's own probability is its B element.
// Rows see a per-row key interval (causal, window); blocks inside every row's
// interval skip the mask.  Split-K (grid z): split s takes blocks s, s + S,
// ... of the workgroup's range and stores unnormalised partials for the
// combine kernel.
#include "attn_common.h"

namespace kessie {
namespace attn {
namespace {

constexpr int kF32Waves = 8;
constexpr int kF32Threads = kF32Waves * 64;
constexpr int kF32Rows = kF32Waves * 16;  // query rows (position, head) per workgroup
constexpr int kF32Row = 128 + 4;          // LDS row stride of the K and V tiles (floats)

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr float kF32RescaleSlack = 5.545177444479562f;  // 8 ln 2

template <int FOG, bool kSplit>
__global__ __launch_bounds__(kF32Threads) void prefill_f32_kernel(Params p) {
  constexpr bool kBias = (FOG & 1) != 0, kVs = (FOG & 2) != 0;
  __shared__ __align__(16) float ks[2][16 * kF32Row];
  __shared__ __align__(16) float vs[2][16 * kF32Row];
  __shared__ float fvs[2][16], fbs[2][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int g = blockIdx.x % p.Hkv;
  int qtile = blockIdx.x / p.Hkv;
  int b = blockIdx.y;
  const int S = kSplit ? (int)gridDim.z : 1, split = kSplit ? (int)blockIdx.z : 0;
  const int G = p.G;
  const int kpos = kF32Rows / G;  // query positions per workgroup
  if (p.q_start) {
    // Varlen: x / Hkv numbers the live (sequence, query tile) pairs in order
    // (the grid's surplus workgroups at its end exit at once); each wave
    // scans query_start_loc 64 sequences at a time (prefix sum by shuffles).
    int found = -1, before = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
      const int bb = b0 + lane;
      const int nt = bb < p.B ? div_up(min(max(p.q_start[bb + 1] - p.q_start[bb], 0), p.C), kpos) : 0;
      int inc = nt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(inc, o, 64);
        if (lane >= o) inc += y;
      }
      const int total = __builtin_amdgcn_readlane(inc, 63);
      if (qtile < before + total) {
        const int l = __ffsll((unsigned long long)__ballot(before + inc > qtile)) - 1;
        found = b0 + l;
        qtile -= before + __builtin_amdgcn_readlane(inc - nt, l);
        break;
      }
      before += total;
    }
    if (found < 0) return;  // uniform, before any barrier
    b = found;
  }
  const int ctx = seq_ctx(p, b);
  int C = p.C;  // this sequence's queries, and where its rows start
  int64_t q_off = (int64_t)b * p.q_bs, o_off = (int64_t)b * p.o_bs;
  if (p.q_start) {
    const int s0 = p.q_start[b] - p.q_start[0];
    C = min(max(p.q_start[b + 1] - p.q_start[b], 0), p.C);  // partial rows are indexed by max_query_len
    q_off = (int64_t)s0 * p.q_is;
    o_off = (int64_t)s0 * p.o_is;
  }

  const int qi_first = qtile * kpos;
  const int qi_last = min(C, qi_first + kpos) - 1;
  if (qi_last < qi_first) return;  // uniform, before any barrier
  const int qmin = max(ctx - C + qi_first, 0), qmax = ctx - C + qi_last;
  int lo = 0, hi = 0;
  if (qmax >= 0) key_range(p, ctx, qmin, qmax, &lo, &hi);
  const int blk_lo = lo >> 4;
  const int nblk_all = hi > lo ? ((hi + 15) >> 4) - blk_lo : 0;
  const int nblk = nblk_all > split ? (nblk_all - split + S - 1) / S : 0;  // blocks split, split + S, ...

  // This lane's query row: row col of the wave.
  const int frow = wave * 16 + col;
  const int qi = qi_first + frow / G;
  const int head = g * G + frow % G;
  const int q_pos = ctx - C + qi;
  const bool row_ok = frow < kpos * G && qi <= qi_last && q_pos >= 0;
  int klo_r = lo, khi_r = hi;  // this row's visible keys
  if (p.causal || p.window > 0) khi_r = min(khi_r, q_pos + 1);
  if (p.window > 0) klo_r = max(klo_r, q_pos - p.window + 1);
  if (!row_ok) khi_r = klo_r;
  // Blocks inside every row's interval: [in_lo, in_hi) in key positions.
  const int in_lo = p.window > 0 ? max(lo, qmax - p.window + 1) : lo;
  const int in_hi = min(hi, qmin + 1);

  // B operand of S^T: query row d = 32 grp + 4 j + e (zero for an invalid row).
  f32x4v qreg[8];
  {
    const float* qr = static_cast<const float*>(p.q) + q_off + (int64_t)min(max(qi, 0), qi_last) * p.q_is +
                      (int64_t)head * p.q_hs;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      qreg[j] = row_ok ? *reinterpret_cast<const f32x4v*>(qr + 32 * grp + 4 * j) : f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // Loader: thread tid moves 16 bytes of K and of V of key tid / 32 of a
  // block (d chunk tid % 32); threads 0..15 the block's fog values.
  const int lkey = tid >> 5, lch = tid & 31;
  const int psh = __builtin_ctz((unsigned)p.page_size) - 4;
  const int pmask = (1 << psh) - 1;
  const int32_t* table = p.page_table + (int64_t)b * p.table_stride;
  const float* kpool = static_cast<const float*>(p.k) + (int64_t)g * p.head_stride;
  const float* vpool = static_cast<const float*>(p.v) + (int64_t)g * p.head_stride;
  const float* fog_v = kVs ? p.vscale + (int64_t)b * p.vs_bs : nullptr;
  const float* fog_b = kBias ? p.bias + (int64_t)b * p.bias_bs : nullptr;
  f32x4v kl, vl;
  float fvl = 1.0f, fbl = 0.0f;
  auto load = [&](int i) {  // block i of this split: key block blk_lo + split + i * S
    const int blk = blk_lo + split + i * S;
    const int t = 16 * blk + lkey;
    const int pid = table[blk >> psh];
    const bool ok = (uint32_t)pid < (uint32_t)p.num_pages && t >= lo && t < hi;
    const int64_t at = (int64_t)pid * p.page_stride + (int64_t)(((blk & pmask) << 4) + lkey) * p.tok_stride + 4 * lch;
    kl = ok ? __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(kpool + at)) : f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
    vl = ok ? __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(vpool + at)) : f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
    if (tid < 16) {
      const int tf = 16 * blk + tid;
      const bool fin = tf >= lo && tf < hi;
      if (kVs) fvl = fin ? fog_v[tf] : 0.0f;
      if (kBias) fbl = fin ? fog_b[tf] : 0.0f;
    }
  };
  auto store = [&](int st) {
    *reinterpret_cast<f32x4v*>(&ks[st][lkey * kF32Row + 4 * lch]) = kl;
    *reinterpret_cast<f32x4v*>(&vs[st][lkey * kF32Row + 4 * lch]) = vl;
    if (tid < 16) {
      if (kVs) fvs[st][tid] = fvl;
      if (kBias) fbs[st][tid] = fbl;
    }
  };

  f32x4v oacc[8];  // O^T[d = 16 blk + 4 grp + i][row col]
#pragma unroll
  for (int i = 0; i < 8; ++i) oacc[i] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = kNegInf, l_run = 0.0f;

  if (nblk > 0) {
    load(0);
    store(0);
    __syncthreads();
  }
  for (int i = 0; i < nblk; ++i) {
    const int st = i & 1;
    if (i + 1 < nblk) load(i + 1);
    const int t0 = 16 * (blk_lo + split + i * S);
    const float* kt = ks[st];
    const float* vt = vs[st];
    // S^T = K Q^T.
    f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4v kv = *reinterpret_cast<const f32x4v*>(kt + col * kF32Row + 32 * grp + 4 * j);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[e], qreg[j][e], acc, 0, 0, 0);
    }
    // Scores of keys t0 + 4 grp + i for row col.
    const bool interior = t0 >= in_lo && t0 + 16 <= in_hi && (uint32_t)table[(t0 >> 4) >> psh] < (uint32_t)p.num_pages;
    float sc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = t0 + 4 * grp + e;
      float s = acc[e] * p.sm_scale;
      if (kBias) s += fbs[st][4 * grp + e];
      sc[e] = interior || (t >= klo_r && t < khi_r) ? s : kNegInf;
    }
    if (!interior) {
      // A block past the pool (invalid page id) contributes nothing.
      const int pid = table[(t0 >> 4) >> psh];
      if ((uint32_t)pid >= (uint32_t)p.num_pages) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[e] = kNegInf;
      }
    }
    float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    // The reference max moves only when a row's max rises by more than
    // kF32RescaleSlack (natural units, 8 ln 2): until then p <= 2^8 and the O
    // accumulators are left alone.
    const float mnew = mloc > m_run + kF32RescaleSlack ? mloc : m_run;
    const float alpha = mnew == m_run ? 1.0f : (m_run == kNegInf ? 0.0f : __expf(m_run - mnew));
    float pr[4];
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pr[e] = sc[e] == kNegInf ? 0.0f : __expf(sc[e] - mnew);
      psum += pr[e];
    }
    psum += __shfl_xor(psum, 16);
    psum += __shfl_xor(psum, 32);
    l_run = l_run * alpha + psum;
    m_run = mnew;
    if (kVs) {
#pragma unroll
      for (int e = 0; e < 4; ++e) pr[e] *= fvs[st][4 * grp + e];
    }
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k) oacc[k] *= alpha;
    }
    // O^T += V^T P^T.
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4)
#pragma unroll
      for (int blk = 0; blk < 8; ++blk)
        oacc[blk] =
            __builtin_amdgcn_mfma_f32_16x16x4f32(vt[(4 * grp + k4) * kF32Row + 16 * blk + col], pr[k4], oacc[blk], 0, 0, 0);
    if (i + 1 < nblk) store(st ^ 1);
    __syncthreads();
  }

  // Lane (grp, col) holds row frow at d = 16 blk + 4 grp + e.
  if (!row_ok) return;
  if (kSplit) {
    // Partial: unnormalised O, the running max (natural units) and the sum.
    const int64_t r = row_id(p, b, qi, head) * S + split;
    float* dst = p.ws_o + r * 128 + 4 * grp;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) *reinterpret_cast<f32x4v*>(dst + 16 * blk) = oacc[blk];
    if (grp == 0) {
      p.ws_m[r] = m_run;
      p.ws_l[r] = l_run;
    }
    return;
  }
  const float il = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  float* dst = static_cast<float*>(p.out) + o_off + (int64_t)qi * p.o_is + (int64_t)head * p.o_hs + 4 * grp;
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) *reinterpret_cast<f32x4v*>(dst + 16 * blk) = oacc[blk] * il;
}

template <bool kSplit>
void launch_f32(const Params& p, dim3 grid, hipStream_t s) {
  const int fog = (p.bias ? 1 : 0) | (p.vscale ? 2 : 0);
  switch (fog) {
    case 0: hipLaunchKernelGGL((prefill_f32_kernel<0, kSplit>), grid, dim3(kF32Threads), 0, s, p); break;
    case 1: hipLaunchKernelGGL((prefill_f32_kernel<1, kSplit>), grid, dim3(kF32Threads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((prefill_f32_kernel<2, kSplit>), grid, dim3(kF32Threads), 0, s, p); break;
    default: hipLaunchKernelGGL((prefill_f32_kernel<3, kSplit>), grid, dim3(kF32Threads), 0, s, p); break;
  }
}

}  // namespace

// Key splits of the fp32 prefill: two workgroups per CU (34 KiB of LDS, 512
// threads each), at least 4 key blocks per split (forced counts 1-32 on
// 32q/8kv chunks from 64 queries on 8K to fresh 1K prompts: this rule picks
// the fastest or within 1 % of it everywhere but fresh 1,024-token prompts,
// 178 us in two splits against 154 in four; 8 blocks per split kept a fresh
// 256-token prompt at two splits, 37.0 us against 33.9).
int prefill_f32_splits(int B, int C, int Hkv, int G, int max_ctx) {
  const int forced = env_int("KESSIE_PREFILL_SPLITS", 0);
  if (forced > 0) return min(forced, 512);
  const int per_wg = max(1, kF32Rows / max(G, 1));
  const int units = B * Hkv * div_up(max(C, 1), per_wg);
  const int blocks = div_up(max(max_ctx, 1), 16);
  int s = div_up(2 * device_cus(), max(units, 1));
  s = min(s, max(1, blocks / 4));
  s = min(s, 512);
  return max(s, 1);
}

bool prefill_f32_ok(const Params& p, int dtype) {
  if (env_int("KESSIE_FORCE_GENERIC", 0)) return false;
  if (dtype != KESSIE_DTYPE_F32 || p.D != 128 || p.page_table == nullptr) return false;
  if (p.page_size < 16 || (p.page_size & (p.page_size - 1)) != 0) return false;
  if (p.G < 1 || p.G > kF32Rows) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  if (p.page_stride % 4 || p.tok_stride % 4 || p.head_stride % 4 || p.q_bs % 4 || p.q_is % 4 || p.q_hs % 4 ||
      p.o_bs % 4 || p.o_is % 4 || p.o_hs % 4)
    return false;
  return true;
}

// p.num_splits (> 1: partials in p.ws_*, merged by the caller) set by the caller.
int prefill_f32(const Params& p, hipStream_t s) {
  const int kpos = max(1, kF32Rows / p.G);
  const dim3 grid(div_up(p.C, kpos) * p.Hkv * (p.q_start ? p.B : 1), p.q_start ? 1 : p.B, max(p.num_splits, 1));
  if (p.num_splits > 1)
    launch_f32<true>(p, grid, s);
  else
    launch_f32<false>(p, grid, s);
  return check_launch("fog prefill (fp32 mfma)");
}

}  // namespace attn
}  // namespace kessie
