// Chunked-prefill fog attention on MFMA for gfx950 (bf16 / f16, head_dim 128,
// pages of 16 * 2^k tokens, GQA ratio 1/2/4/8/16, sm_scale > 0).
//
// Math: the last C rows of kessie_hip_kernels.py:577-593 over ctx = L + C
// tokens (query i at position ctx-C+i, causal, window, fog weights scaling V
// rows or a logit bias), fp32 accumulation, online softmax in base 2.
//
// Work decomposition: one workgroup = 256 query rows (256/G positions x the G
// heads of one kv head) of one sequence; 8 waves x 32 rows.  The workgroup
// streams its kv head's keys in tiles of 64 (4 pages) through a four-stage
// LDS ring (stage = tile & 3), one barrier per tile:
//   iteration t:  buffer loads of tile t+3 into one of two register sets
//                 (page ids fetched two iterations earlier, wave-uniform);
//                 the softmax of tile t (VALU) interleaved with S^T(t+1) =
//                 K Q^T on MFMA, which does not depend on it; O^T += V^T
//                 P^T(t) interleaved with the store of tile t+2 (loaded one
//                 iteration earlier) from the other set to LDS; barrier.
// Per wave and tile: S^T (64 keys x 32 rows) on v_mfma_f32_32x32x16 (16
// MFMAs) and O^T (128 d x 32 rows) likewise (16 MFMAs).  Key j of a 32-key
// block sits in LDS row swap23(j), so register v of lane l of the S^T
// accumulator holds key 16(v/8) + 8(l/32) + (v%8) of row l%32: the softmax is
// lane-local plus one half-wave swap, and p is already in the B-operand
// layout of PV.  V is stored transposed ([d][key], key pairs packed into
// 32-bit words, already scaled by the V-fog weights) with the 16-byte key
// chunks XOR-swizzled by d/16 and rows of 40 words: of the row strides and
// swizzles measured on gfx950 (LDS bank-conflict counters) this one leaves the
// 16-byte operand reads without conflicts and the transposing 4-byte stores
// with the fewest; the K rows are padded to 68 words, also conflict-free.  The softmax sum is taken from p as rounded for PV.
// Grid index x = qtile * Hkv + g, so with 8 kv heads (and the hardware's
// round-robin of workgroups over the 8 XCDs) every workgroup of kv head g
// sits on one XCD and the query tiles of that head share its keys in L2.
//
// Variants (template and Params):
//   kSplit   grid z splits each query tile's key tiles (split s takes tiles
//            s, s + S, ...); every split stores unnormalised partials (O,
//            max, sum) merged by the combine kernel -- used when the chunks
//            alone would leave CUs idle;
//   q_start  varlen batch: x / Hkv numbers the live (sequence, query tile)
//            pairs, each chunk's queries packed at query_start_loc;
//   kMode    0 paged; 1 table-less pages (page b * dense_ppb + j) for the
//            reference's dense [B][H][N][D] launchers, query tiles longest
//            first (split: only the tiles from split_q0 on, S units each,
//            numbered along x split-major with the unsplit tiles, which
//            store their output directly); 2 paged with query tiles longest first (a causal chunk
//            that is most of its context and takes several grid rounds); 3
//            paged with pages of 32, 64, ... tokens, read as 16-token blocks.
#include "attn_common.h"

namespace kessie {
namespace attn {
namespace {

constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * 64;
constexpr int kPfRows = kPfWaves * 32;  // query rows (position, head) per workgroup
constexpr int kPfKT = 64;               // keys per tile (4 pages)
constexpr int kPfStages = 4;            // LDS ring depth (a power of two)
constexpr int kVRowW = kPfKT / 2 + 8;   // V^T tile row stride (32-bit words)
// LDS geometry for head_dim D: 128, or 64 (the dense launchers only).
template <int D>
struct PfGeom {
  static constexpr int kKRow = D + 8;            // K tile row stride (elements)
  static constexpr int kKStage = kPfKT * kKRow;  // elements per K stage
  static constexpr int kVStage = D * kVRowW;     // words per V^T stage
  static constexpr size_t kLdsBytes = (size_t)kPfStages * (kKStage * 2 + kVStage * 4 + kPfKT * 4);
};
constexpr float kLog2e = 1.4426950408889634f;
// Word 3 of a raw (unformatted, stride 0) buffer resource on gfx9-family parts.
constexpr int kRsrcWord3 = 0x00020000;
constexpr float kLn2 = 0.6931471805599453f;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mma32;
template <>
struct Mma32<bf16_t> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mma32<f16_t> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ int swap23(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

template <typename T>
__device__ __forceinline__ uint32_t bits16(T x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to nearest-even and packed into one operand dword (one
// v_cvt_pk per pair, where element-wise stores left shuffles behind).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}

// max(a, b, c) in one instruction.  fmaxf on MFMA results first quiets each
// input (one extra v_max per score); scores hold no signalling NaN, so the
// raw instruction gives the same result.  Being inline assembly, it gets no
// wait states from the compiler's MFMA hazard checks: a VALU read of a 32x32
// MFMA's result needs 18 (ISA), and every use here reads scores whose MFMAs
// were issued in the previous iteration, hundreds of instructions earlier.
// (Reading them right after their MFMAs returned stale registers, seen as
// results that changed from run to run.)
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// max over lanes l and l ^ 32: v_permlane32_swap exchanges the two halves of
// the wave in registers (no LDS round trip).  Written as inline assembly: the
// builtin, given one value for both operands, is folded as if both results
// were that value, which drops the exchange.  (s_nop 1: the two wait states
// the swap needs after a VALU write of its operands.)
__device__ __forceinline__ float max_xor32(float x) {
  float a = x, b = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return max3(a, b, b);
}

// acc + lo + hi of two packed T values (one v_dot2 against (1, 1)).
template <typename T>
__device__ __forceinline__ float sum2(uint32_t w, float acc);
template <>
__device__ __forceinline__ float sum2<bf16_t>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3f803f80u), acc,
                                         false);
}
template <>
__device__ __forceinline__ float sum2<f16_t>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, 0x3c003c00u), acc, false);
}


// Headroom of the lazy rescale, in log2 units: probabilities up to 2^8.
constexpr float kRescaleSlack = 8.0f;

template <typename T, int G, bool kBias, bool kVs, bool kSplit, int kMode, int kD>
__global__ __launch_bounds__(kPfThreads) void prefill_mfma_kernel(Params p) {
  static_assert(kD == 128 || kD == 64, "head_dim 128, or 64 on table-less pages");
  constexpr bool kDense = kMode == 1;
  constexpr bool kBig = kMode == 3;  // pages of 16 * 2^k tokens, k >= 1
  constexpr int kKRow = PfGeom<kD>::kKRow;
  constexpr int kKStage = PfGeom<kD>::kKStage;
  constexpr int kVStage = PfGeom<kD>::kVStage;
  constexpr int kDS = kD / 16;  // QK d-steps (B operand registers)
  constexpr int kDB = kD / 32;  // PV d-blocks (O accumulators)
  typedef typename Mma32<T>::v8 v8;
  typedef typename Mma32<T>::v4 v4;
  constexpr int kPos = kPfRows / G;  // query positions per workgroup
  extern __shared__ __align__(16) unsigned char smem[];
  T* ks = reinterpret_cast<T*>(smem);                                                // [stage][64][kKRow]
  uint32_t* vts = reinterpret_cast<uint32_t*>(smem + (size_t)kPfStages * kKStage * 2);  // [stage][128][kVRowW]
  float* fbs = reinterpret_cast<float*>(vts + kPfStages * kVStage);                   // [stage][64] bias*log2(e)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int g = blockIdx.x % p.Hkv;
  int qtile = blockIdx.x / p.Hkv;
  int b = blockIdx.y;
  // Split instances: S workgroups per query tile along grid z, each taking
  // its share of the key tiles.  The dense split instead numbers (tile, split)
  // units along x, longest tile first: the S splits of each tile from
  // position split_q0 on, then the shorter tiles, one workgroup each.
  int S = kSplit ? (int)gridDim.z : 1, split = kSplit ? (int)blockIdx.z : 0;
  bool part_out = kSplit;  // this workgroup stores split partials
  if (kDense && kSplit) {
    // Split-major order, as a grid z of splits would dispatch: pass 0 holds
    // every query tile, longest first -- split 0 of a split tile, or all of a
    // tile that is not split (its output stored directly) -- and pass s >= 1
    // split s of the split tiles, longest first.  The tiles of a head in a
    // pass stream their keys upward from the same start, sharing them in L2
    // (units sorted by size instead ran N=8,192 5 % slower).
    const int nq = div_up(p.C, kPfRows);
    const int t0 = p.split_q0 / kPfRows;  // first split tile
    if (qtile < nq) {
      qtile = nq - 1 - qtile;
      split = 0;
      if (qtile >= t0) {
        S = p.num_splits;
      } else {
        S = 1;
        part_out = false;
      }
    } else {
      const int k = qtile - nq, nl = nq - t0;
      S = p.num_splits;
      split = 1 + k / nl;
      qtile = nq - 1 - k % nl;
    }
  } else if ((kDense && p.causal) || kMode == 2) {
    // Dense causal (every position a query): later query tiles see more keys;
    // dispatching them first keeps the short ones for the tail of the grid
    // (+15-19 %).  Not in the paged instances: there the same two lines cost
    // the long-context shape 1-2 % through code generation.
    qtile = (int)(gridDim.x / p.Hkv) - 1 - qtile;
  }
  if (p.q_start) {
    // Varlen: x / Hkv numbers the live (sequence, query tile) pairs in order,
    // so the grid's surplus workgroups all sit at its end and exit at once
    // (left among the live ones, they unbalanced the placement of those).
    // Each wave scans query_start_loc 64 sequences at a time.
    int found = -1, before = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
      const int bb = b0 + lane;
      const int nt = bb < p.B ? div_up(min(max(p.q_start[bb + 1] - p.q_start[bb], 0), p.C), kPos) : 0;
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
    if (found < 0) return;
    b = found;
  }
  const int ctx = seq_ctx(p, b);
  int C = p.C;  // this sequence's queries, and where they start (uniform)
  int64_t q_off = (int64_t)b * p.q_bs, o_off = (int64_t)b * p.o_bs;
  if (p.q_start) {
    const int s0 = p.q_start[b] - p.q_start[0];
    // Chunks are clamped to [0, max_query_len]: partial rows (split) are
    // indexed by it, so a longer chunk must not reach past them.
    C = min(max(p.q_start[b + 1] - p.q_start[b], 0), p.C);
    q_off = (int64_t)s0 * p.q_is;
    o_off = (int64_t)s0 * p.o_is;
  }

  // Rows of the workgroup and the key range they see (uniform).
  const int qi_first = qtile * kPos;
  const int qi_last = min(C, qi_first + kPos) - 1;
  const int qmin = max(ctx - C + qi_first, 0);
  const int qmax = ctx - C + qi_last;
  if (qi_last < qi_first) return;
  // Rows before position 0 (a chunk longer than its context) see no keys:
  // they still run, with no tiles, and store zeros (or empty partials).
  int lo = 0, hi = 0;
  if (qmax >= 0) key_range(p, ctx, qmin, qmax, &lo, &hi);
  const int tile_lo = lo / kPfKT;
  int n_tiles = hi > tile_lo * kPfKT ? div_up(hi - tile_lo * kPfKT, kPfKT) : 0;
  // Split-K: split s takes key tiles s, s + S, s + 2S, ... of the range
  // (possibly none: it still writes an empty partial for its rows).
  // Interleaved, the splits that run at one time all stream a head's keys
  // upward from its first tile, sharing them in L2 (contiguous thirds or
  // halves started the later splits at staggered keys: dense B=1 H=8 N=8,192
  // split in two ran each key tile ~30 % slower than unsplit).
  int first = 0, kstep = kPfKT;  // first tile, key positions between consecutive tiles
  if (kSplit && S > 1) {
    // (The division runs on the vector unit; readfirstlane returns the
    // uniform bounds to scalar registers.)
    first = split;
    n_tiles = __builtin_amdgcn_readfirstlane(n_tiles > split ? (n_tiles - split + S - 1) / S : 0);
    kstep = S * kPfKT;
  }
  const int t_begin = (tile_lo + first) * kPfKT;
  const int n_tab = div_up(hi, 16);  // table entries that may be read

  // This lane's query row.
  const int frow = wave * 32 + col;
  const int qi = qi_first + frow / G;
  const int head = g * G + frow % G;
  const int q_pos = ctx - C + qi;
  const bool row_ok = qi <= qi_last && q_pos >= 0;

  // B operand of S^T = K Q^T: d-step s holds d = 16s + 8*half .. +8.
  v8 qv[kDS];
  {
    const T* qr = static_cast<const T*>(p.q) + q_off + (int64_t)min(qi, qi_last) * p.q_is +
                  (int64_t)head * p.q_hs;
#pragma unroll
    for (int s = 0; s < kDS; ++s) {
      if (row_ok) {
        qv[s] = *reinterpret_cast<const v8*>(qr + 16 * s + 8 * half);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[s][e] = static_cast<T>(0.0f);
      }
    }
  }

  // Loader.  Head_dim 128: wave w loads page slot w/2 of the tile, K and V
  // alike (one page id per wave): K rows rr and rr+8 of the page and the V row
  // pair (2rr, 2rr+1), rr = lane/16 + 4(w%2), 16-byte chunk kc = lane%16 of the
  // 256-byte token row.  Head_dim 64: K row kr = tid/8 of the tile (page slot
  // w/2), V rows 2kr and 2kr+1 by waves 0-3 (page slot w), chunk kc of the
  // 128-byte row.
  constexpr int kCh = kD / 8;  // 16-byte chunks per token row
  const int kc = tid & (kCh - 1);
  const int rr = kD == 128 ? (lane >> 4) + 4 * (wave & 1) : tid / kCh;
  const int kslot = wave >> 1;                      // K page slot
  const int vslot = kD == 128 ? wave >> 1 : wave;   // V page slot
  const int kp = kD == 128 ? 8 * vslot + rr : rr;  // V key pair of the tile (keys 2kp, 2kp+1)
  auto krow = [&](int r) { return kD == 128 ? 16 * kslot + rr + 8 * r : rr; };  // K key of the tile
  auto krow_lds = [&](int r) { return (krow(r) & 32) | swap23(krow(r) & 31); };  // its LDS row
  const int32_t* table = kDense ? nullptr : p.page_table + (int64_t)b * p.table_stride;
  const int dense0 = kDense ? b * p.dense_ppb : 0;  // table-less pages: sequence b's first
  const bool vload = kD == 128 || wave < 4;
  const int vkey_off = 2 * kp;  // this thread's first V key in a tile

  // The loop runs over 16-token blocks.  With pages of 16 * 2^psh tokens
  // (kBig), block j is rows 16 * (j & pmask) of page table[j >> psh], and its
  // id is (page << psh) | (j & pmask), or -1 for an invalid page; otherwise the
  // id is the page id.  (A separate instance: the extra scalar work per tile
  // cost the 16-token instances 3-4.5 %.)
  const int psh = kBig ? __builtin_ctz((unsigned)p.page_size) - 4 : 0;
  const int pmask = (1 << psh) - 1;
  const uint32_t n_ids = kBig ? (uint32_t)p.num_pages << psh : (uint32_t)p.num_pages;
  // Page ids of a tile (4 uniform values; -1 past the end).  The table index
  // is clamped into the readable entries and the value replaced afterwards, so
  // the four scalar loads issue back to back with no branch around them.
  auto fetch_ids = [&](int tile) {
    const int pg0 = (t_begin + tile * kstep) >> 4;
    i32x4 ids;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = tile < n_tiles && pg0 + j < n_tab;
      if constexpr (kDense) {
        ids[j] = in ? dense0 + pg0 + j : -1;
      } else if constexpr (kBig) {
        const int e = table[min(pg0 + j, n_tab - 1) >> psh];
        ids[j] = in && (uint32_t)e < (uint32_t)p.num_pages ? (e << psh) | ((pg0 + j) & pmask) : -1;
      } else {
        const int e = table[min(pg0 + j, n_tab - 1)];
        ids[j] = in ? e : -1;
      }
    }
    return ids;
  };

  auto valid_mask = [&](i32x4 ids) {
    int m = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) m |= (uint32_t)uniform(ids[j]) < n_ids ? (1 << j) : 0;
    return m;
  };
  auto slot_id = [&](i32x4 ids, int slot) {
    return uniform(slot & 2 ? (slot & 1 ? ids[3] : ids[2]) : (slot & 1 ? ids[1] : ids[0]));
  };
  // A tile's page ids and this wave's own (page slot kslot).  Every tile
  // but the last has its four entries in range: one base, four consecutive
  // words (one scalar load of 16 bytes) and the wave's own word, instead of
  // four clamped addresses and a select chain over the slot.
  struct TileIds {
    i32x4 ids;
    int own;
  };
  auto fetch_tile = [&](int tile) {
    TileIds r;
    const int pg0 = (t_begin + tile * kstep) >> 4;
    if constexpr (!kDense && !kBig) {
      if (tile < n_tiles && pg0 + 3 < n_tab) {
        const int32_t* e = table + pg0;
        r.ids = i32x4{e[0], e[1], e[2], e[3]};
        r.own = e[kslot];
        return r;
      }
    }
    r.ids = fetch_ids(tile);
    if constexpr (kDense) {
      r.own = tile < n_tiles && pg0 + kslot < n_tab ? dense0 + pg0 + kslot : -1;
    } else if constexpr (kBig) {
      const int j = pg0 + kslot;
      const int e = table[min(j, n_tab - 1) >> psh];
      r.own = tile < n_tiles && j < n_tab && (uint32_t)e < (uint32_t)p.num_pages ? (e << psh) | (j & pmask) : -1;
    } else {
      r.own = slot_id(r.ids, kslot);
    }
    return r;
  };

  // Global loads go through buffer resources whose record count covers only
  // the page's rows inside the key range (none for an invalid page id), so
  // rows past the range, past a dense tensor's end or of an invalid page read
  // as zero with no branch: every tile issues the same loads, and the wait
  // for one tile's data does not wait for the next tile's loads.  All
  // offsets are in the per-lane offset, which the range check covers.
  constexpr int kKL = kD == 128 ? 2 : 1;  // K rows loaded per thread per tile
  const int ts_b = (int)p.tok_stride * (int)sizeof(T);
  constexpr int kRowB = kD * (int)sizeof(T);
  const char* kpool = static_cast<const char*>(p.k) + (int64_t)g * p.head_stride * (int64_t)sizeof(T);
  const char* vpool = static_cast<const char*>(p.v) + (int64_t)g * p.head_stride * (int64_t)sizeof(T);
  uint32_t koff[kKL];
#pragma unroll
  for (int r = 0; r < kKL; ++r) koff[r] = (uint32_t)((krow(r) & 15) * ts_b + 16 * kc);
  const uint32_t voff0 = (uint32_t)((vkey_off & 15) * ts_b + 16 * kc), voff1 = voff0 + (uint32_t)ts_b;
  // A page's place in its pool (bytes) and the bytes of its rows inside the
  // key range: 0 and 0 for an invalid page id or no rows in range, so its
  // loads read zeros.  With head_dim 128 a wave's K and V share the page, and
  // the span is computed once for both.
  // (A page's stride in bytes is below 2^32, checked on the host, so its
  // offset is one 32 x 32 -> 64-bit product.)
  const uint32_t pstride_b = (uint32_t)(p.page_stride * (int64_t)sizeof(T));
  auto page_span = [&](int pid, int first_tok, int64_t& off, int& bytes) {
    const int nrows = min(max(hi - first_tok, 0), 16);
    const bool ok = (uint32_t)pid < n_ids && nrows > 0;
    const uint32_t upid = ok ? (uint32_t)pid : 0u;
    uint64_t at = (uint64_t)upid * pstride_b;
    if constexpr (kBig)
      at = (uint64_t)(upid >> psh) * pstride_b + (uint64_t)(((upid & (uint32_t)pmask) << 4) * (uint32_t)ts_b);
    off = (int64_t)at;
    bytes = ok ? (nrows - 1) * ts_b + kRowB : 0;
  };
  auto span_rsrc = [&](const char* pool, int64_t off, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(pool + off), (short)0, bytes, kRsrcWord3);
  };
  // Rows of V weights and of the bias: keys past the range read as zero.
  // (The second weight goes through a resource starting one key later, so the
  // two loads are not merged into one 8-byte load, which would straddle the
  // range's end for the last key.)
  float* const fw_row = kVs ? const_cast<float*>(p.vscale + (int64_t)b * p.vs_bs) : nullptr;
  const auto fw_rsrc = __builtin_amdgcn_make_buffer_rsrc(fw_row, (short)0, kVs ? hi * 4 : 0, kRsrcWord3);
  const auto fw1_rsrc = __builtin_amdgcn_make_buffer_rsrc(kVs ? fw_row + 1 : nullptr, (short)0,
                                                          kVs ? max(hi - 1, 0) * 4 : 0, kRsrcWord3);
  const auto fb_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      kBias ? const_cast<float*>(p.bias + (int64_t)b * p.bias_bs) : nullptr, (short)0, kBias ? hi * 4 : 0, kRsrcWord3);

  // Two register sets: the loads of tile t+3 go out in iteration t, one
  // iteration before their stage store, and land behind a whole iteration.
  v8 kreg[2][kKL], vreg[2][2];
  float fw0[2] = {1.0f, 1.0f}, fw1[2] = {1.0f, 1.0f}, fb_r[2] = {0.0f, 0.0f};
  auto issue = [&](int tile, const TileIds& tid_s, int set) {
    const int t0 = t_begin + tile * kstep;
    int64_t k_at;
    int k_bytes;
    page_span(tid_s.own, t0 + 16 * kslot, k_at, k_bytes);
    const auto krs = span_rsrc(kpool, k_at, k_bytes);
#pragma unroll
    for (int r = 0; r < kKL; ++r)
      kreg[set][r] = __builtin_bit_cast(v8, __builtin_amdgcn_raw_buffer_load_b128(krs, (int)koff[r], 0, 0));
    if (vload) {
      int64_t v_at = k_at;
      int v_bytes = k_bytes;
      if constexpr (kD != 128) page_span(slot_id(tid_s.ids, vslot), t0 + 16 * vslot, v_at, v_bytes);
      const auto vrs = span_rsrc(vpool, v_at, v_bytes);
      vreg[set][0] = __builtin_bit_cast(v8, __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)voff0, 0, 0));
      vreg[set][1] = __builtin_bit_cast(v8, __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)voff1, 0, 0));
      if (kVs) {
        const int o = (t0 + vkey_off) * 4;
        fw0[set] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(fw_rsrc, o, 0, 0));
        fw1[set] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(fw1_rsrc, o, 0, 0));
      }
    }
    if (kBias)
      fb_r[set] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(fb_rsrc, (t0 + (tid & 63)) * 4, 0, 0));
  };
  // V-fog: V rows are scaled by their fog weights here, rounded to T, as the
  // reference scales V before its product (v * fog_weights), so the
  // probabilities stay unscaled and the softmax sum can be taken from them.
  auto store = [&](int stage, int set) {
    T* kd = ks + stage * kKStage + 8 * kc;
#pragma unroll
    for (int r = 0; r < kKL; ++r) *reinterpret_cast<v8*>(kd + krow_lds(r) * kKRow) = kreg[set][r];
    if (vload) {
      uint32_t* vd = vts + stage * kVStage + 4 * ((kp >> 2) ^ (kc >> 1)) + (kp & 3);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vd[(8 * kc + e) * kVRowW] = kVs ? pack2<T>(to_f32(vreg[set][0][e]) * fw0[set], to_f32(vreg[set][1][e]) * fw1[set])
                                        : bits16(vreg[set][0][e]) | (bits16(vreg[set][1][e]) << 16);
    }
    if (kBias && tid < kPfKT) fbs[stage * kPfKT + tid] = fb_r[set] * kLog2e;
  };

  // Slice i of n (n >= 8) of store(): V^T word i for i < 8, then the K rows
  // and the bias at slice n-1 -- spread over the PV MFMAs.  With no tile
  // t+2 it rewrites a stage that no later tile reads.
  auto store_slice = [&](int stage, int i, int n, int set) {
    if (vload && i < 8) {
      uint32_t* vd = vts + stage * kVStage + 4 * ((kp >> 2) ^ (kc >> 1)) + (kp & 3);
      vd[(8 * kc + i) * kVRowW] = kVs ? pack2<T>(to_f32(vreg[set][0][i]) * fw0[set], to_f32(vreg[set][1][i]) * fw1[set])
                                      : bits16(vreg[set][0][i]) | (bits16(vreg[set][1][i]) << 16);
    }
    if (i == n - 1) {
      T* kd = ks + stage * kKStage + 8 * kc;
#pragma unroll
      for (int r = 0; r < kKL; ++r) *reinterpret_cast<v8*>(kd + krow_lds(r) * kKRow) = kreg[set][r];
      if (kBias && tid < kPfKT) fbs[stage * kPfKT + tid] = fb_r[set] * kLog2e;
    }
  };
  // S^T of the tile in a stage: lane (col, half) reads K row 32kb + col.
  const T* kread = ks + col * kKRow + 8 * half;
  auto qk = [&](int stage, f32x16 (&s)[2]) {
    const T* kb0 = kread + stage * kKStage;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = f32x16{};
#pragma unroll
      for (int st = 0; st < kDS; ++st)
        s[kb] = Mma32<T>::mma(*reinterpret_cast<const v8*>(kb0 + 32 * kb * kKRow + 16 * st), qv[st], s[kb]);
    }
  };
  // V^T operand: lane reads row d = 32db + col, key chunk (2s + half) stored
  // at chunk (2s + half) ^ (d / 16) = 2(s ^ db) + (half ^ col / 16).
  const uint32_t* vread = vts + col * kVRowW + 4 * (half ^ (col >> 4));

  f32x16 oacc[kDB];
#pragma unroll
  for (int i = 0; i < kDB; ++i) oacc[i] = f32x16{};
  float m_run = kNegInf, l_half = 0.0f;
  const float c2 = p.sm_scale * kLog2e;

  // Tiles whose 64 keys all lie in [lo, hi) and are visible to every row of
  // the workgroup (causal: none after the first row's position; window: none
  // before the last row's window start): [ti_lo, ti_hi), uniform.
  int ti_lo, ti_hi;
  {
    const int klo = p.window > 0 ? max(lo, qmax - p.window + 1) : lo;
    const int khi = min(hi, qmin + 1);
    // Tile t covers keys [t_begin + t * kstep, + kPfKT).
    const int dlo = klo - t_begin, dhi = khi - t_begin;
    ti_lo = dlo <= 0 ? 0 : (dlo + kstep - 1) / kstep;
    ti_hi = dhi < kPfKT ? 0 : (dhi - kPfKT) / kstep + 1;
  }

  TileIds ids_a, ids_b;          // page ids of tiles t+3 and t+4
  int pm0 = 0, pm1 = 0, pm2 = 0;  // valid-page masks of tiles t, t+1 and t+2
  // Scores in three 16-register buffers: a tile's two 32-key blocks in two of
  // them, the next tile's second block built in the third while the first
  // is still read, its first block then built in the first buffer once that
  // buffer's exponentials are done (16 registers fewer than two full sets).
  f32x16 sA, sB, sC;
  // One tile: sc holds its scores, sn receives the next tile's.  The next
  // tile's S^T MFMAs do not depend on this tile's softmax, so they share one
  // scheduling region with its exponentials and are interleaved with them:
  // the wave keeps the matrix pipe busy while its VALU works (and the other
  // wave of the SIMD fills what is left of either).
  // set: the register set receiving tile t+3 (= (t+1) & 1); the other one
  // holds tile t+2, stored to its stage in this iteration.
  auto step = [&](int t, f32x16& c0, f32x16& c1, f32x16& x, int set) {
    auto sc = [&](int kb) -> f32x16& { return kb ? c1 : c0; };
    const int t0 = t_begin + t * kstep;
    const int st_cur = t & (kPfStages - 1);
    const int st_nxt = (t + 1) & (kPfStages - 1);
    const int st_new = (t + 2) & (kPfStages - 1);
    // Tile t+3's global loads (none past the last tile: its ids are -1).
    const int pm3 = valid_mask(ids_a.ids);
    issue(t + 3, ids_a, set);
    ids_a = ids_b;
    ids_b = fetch_tile(t + 5);

    const bool interior = pm0 == 0xF && t >= ti_lo && t < ti_hi;
    const float* fbt = fbs + st_cur * kPfKT + 8 * half;
    // Base-2 logits y = x * c2 (+ bias * log2 e); the tile max of y.
    if (!interior) {
      // This lane's keys of the tile form one interval of key offsets,
      // [klo_r, khi_r) relative to this lane's first key, intersected with
      // the valid pages: one unsigned compare per key.
      const int kbase = t0 + 8 * half;
      int klo_r = lo, khi_r = hi;
      if (p.causal || p.window > 0) khi_r = min(khi_r, q_pos + 1);
      if (p.window > 0) klo_r = max(klo_r, q_pos - p.window + 1);
      if (!row_ok) khi_r = klo_r;
      const int off = klo_r - kbase;
      const uint32_t len = (uint32_t)max(khi_r - klo_r, 0);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int kl = 32 * kb + 16 * (v >> 3) + (v & 7);  // key offset minus 8 * half
          const bool ok = ((uint32_t)(kl - off) < len) & (((pm0 >> (2 * kb + (v >> 3))) & 1) != 0);
          float y = kBias ? fmaf(sc(kb)[v], c2, fbt[32 * kb + 16 * (v >> 3) + (v & 7)]) : sc(kb)[v];
          sc(kb)[v] = ok ? y : kNegInf;
        }
    } else if (kBias) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) sc(kb)[v] = fmaf(sc(kb)[v], c2, fbt[32 * kb + 16 * (v >> 3) + (v & 7)]);
    }
    float ma = kNegInf, mb = kNegInf;  // two chains of max3
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; v += 4) {
        ma = max3(ma, sc(kb)[v], sc(kb)[v + 1]);
        mb = max3(mb, sc(kb)[v + 2], sc(kb)[v + 3]);
      }
    float mloc = max_xor32(fmaxf(ma, mb));
    if (!kBias) mloc *= c2;  // without a bias, y = x * c2 and c2 > 0
    // The reference max moves only when a row's max rises by more than
    // kRescaleSlack (log2 units); until then p = 2^(y - m_run) <= 2^kRescaleSlack,
    // as exact in T as any p <= 1, and the O accumulators are left alone.
    const float mnew = mloc > m_run + kRescaleSlack ? mloc : m_run;
    const float muse = mnew == kNegInf ? 0.0f : mnew;
    const float alpha = mnew == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - mnew);
    // (Rescaled before the exponentials, so that they, the next scores and PV
    // form one branch-free region.)
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int i = 0; i < kDB; ++i) oacc[i] *= alpha;
    }
    // The next tile's scores, this tile's exponentials and PV, and the stage
    // store of tile t+2 in one branch-free region, in a fixed order: step i
    // issues MFMA i (QK steps first, then PV), the LDS operand read of MFMA
    // i+2, and a share of the VALU work -- one or two exponential pairs per
    // QK step, one slice of the stage store per PV step -- so the wave keeps
    // the matrix pipe busy while its VALU works.
    constexpr int kQ = 2 * kDS;   // S^T MFMAs
    constexpr int kPV = 4 * kDB;  // O^T MFMAs
    constexpr int kPairsPer = 16 / kQ;
    const T* kb0 = kread + st_nxt * kKStage;
    const uint32_t* vr = vread + st_cur * kVStage;
    auto op_read = [&](int i) {
      if (i < kQ) return *reinterpret_cast<const v8*>(kb0 + 32 * (i < kDS ? 1 : 0) * kKRow + 16 * (i % kDS));
      const int s = (i - kQ) / kDB, db = (i - kQ) % kDB;
      return *reinterpret_cast<const v8*>(vr + 32 * db * kVRowW + 8 * (s ^ db));
    };
    float ps0 = 0.0f, ps1 = 0.0f;  // the softmax sum, from p as rounded for PV
    u32x4 pb[4];                   // p as the PV B operand, two keys per dword
    auto exp_pair = [&](int j) {   // keys 2j, 2j+1 of this lane's 32
      const int kb = j >> 3, v = 2 * (j & 7);
      const float y0 = sc(kb)[v], y1 = sc(kb)[v + 1];
      const float p0 = __builtin_amdgcn_exp2f(kBias ? y0 - muse : fmaf(y0, c2, -muse));
      const float p1 = __builtin_amdgcn_exp2f(kBias ? y1 - muse : fmaf(y1, c2, -muse));
      const uint32_t w = pack2<T>(p0, p1);
      pb[j >> 2][j & 3] = w;
      if (j & 1)
        ps1 = sum2<T>(w, ps1);
      else
        ps0 = sum2<T>(w, ps0);
    };
    v8 op[3];
    op[0] = op_read(0);
    op[1] = op_read(1);
#pragma unroll
    for (int i = 0; i < kQ + kPV; ++i) {
      if (i < kQ) {
        // The next tile's second block into x, then its first into c0
        // (whose exponentials, the first eight pairs, are issued by then).
        if (i < kDS)
          x = Mma32<T>::mma(op[i % 3], qv[i], i == 0 ? f32x16{} : x);
        else
          c0 = Mma32<T>::mma(op[i % 3], qv[i - kDS], i == kDS ? f32x16{} : c0);
      } else {
        const int s = (i - kQ) / kDB, db = (i - kQ) % kDB;
        oacc[db] = Mma32<T>::mma(op[i % 3], __builtin_bit_cast(v8, pb[s]), oacc[db]);
      }
      if (i + 2 < kQ + kPV) op[(i + 2) % 3] = op_read(i + 2);
      if (i < kQ) {
#pragma unroll
        for (int j = 0; j < kPairsPer; ++j) exp_pair(i * kPairsPer + j);
      } else {
        store_slice(st_new, i - kQ, kPV, set ^ 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l_half = l_half * alpha + (ps0 + ps1);
    m_run = mnew;
    pm0 = pm1;
    pm1 = pm2;
    pm2 = pm3;
    __syncthreads();
  };
  if (n_tiles > 0) {
    const TileIds ids0 = fetch_tile(0), ids1 = fetch_tile(1), ids2 = fetch_tile(2);
    pm0 = valid_mask(ids0.ids);
    pm1 = valid_mask(ids1.ids);
    pm2 = valid_mask(ids2.ids);
    issue(0, ids0, 0);
    store(0, 0);
    issue(1, ids1, 1);
    store(1, 1);
    issue(2, ids2, 0);
    ids_a = fetch_tile(3);
    ids_b = fetch_tile(4);
    __syncthreads();
    {
      f32x16 s0[2];
      qk(0, s0);
      sA = s0[0];
      sB = s0[1];
    }
    // Unrolled by two so the score buffers alternate instead of being copied.
    // (Inside the prologue's branch, so the wait for the query loads stays
    // here and not in every iteration, where it would also wait for the
    // tile loads just issued.)
    for (int t = 0; t < n_tiles; t += 2) {
      step(t, sA, sB, sC, 1);
      if (t + 1 < n_tiles) step(t + 1, sA, sC, sB, 0);
    }
  }

  // Lane (col, half) holds row frow at d = 32*db + 8*(v/4) + 4*half + (v%4).
  const float l = l_half + __shfl_xor(l_half, 32);
  if (!row_ok) return;
  if (kSplit && part_out) {
    // Split partial: unnormalised O, the running max in natural-log units
    // (the softmax here is base 2) and the sum, merged by the combine kernel.
    const int64_t r = (kDense ? ((int64_t)b * (p.C - p.split_q0) + (qi - p.split_q0)) * p.Hq + head
                              : row_id(p, b, qi, head)) * S + split;
    float* dst = p.ws_o + r * kD + 4 * half;
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int vq = 0; vq < 4; ++vq)
        *reinterpret_cast<f32x4*>(dst + 32 * db + 8 * vq) =
            f32x4{oacc[db][4 * vq], oacc[db][4 * vq + 1], oacc[db][4 * vq + 2], oacc[db][4 * vq + 3]};
    if (half == 0) {
      p.ws_m[r] = m_run == kNegInf ? kNegInf : m_run * kLn2;
      p.ws_l[r] = l;
    }
    return;
  }
  const float il = l > 0.0f ? 1.0f / l : 0.0f;
  T* orow = static_cast<T*>(p.out) + o_off + (int64_t)qi * p.o_is + (int64_t)head * p.o_hs;
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int vq = 0; vq < 4; ++vq) {
      v4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = from_f32<T>(oacc[db][4 * vq + e] * il);
      *reinterpret_cast<v4*>(orow + 32 * db + 8 * vq + 4 * half) = o;
    }
}

template <typename T, int G, bool kBias, bool kVs, bool kSplit, int kMode = 0, int kD = 128>
int launch_one(const Params& p, dim3 grid, hipStream_t stream) {
  static bool lds_set[64] = {};  // per instance and device
  constexpr size_t lds = PfGeom<kD>::kLdsBytes;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  const void* fn = reinterpret_cast<const void*>(prefill_mfma_kernel<T, G, kBias, kVs, kSplit, kMode, kD>);
  if (!lds_set[dev]) {
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
      set_error(KESSIE_ERR_HIP, "fog prefill (mfma): %zu bytes of LDS unavailable", lds);
      return KESSIE_ERR_HIP;
    }
    lds_set[dev] = true;
  }
  hipLaunchKernelGGL((prefill_mfma_kernel<T, G, kBias, kVs, kSplit, kMode, kD>), grid, dim3(kPfThreads), lds, stream,
                     p);
  return check_launch("fog prefill (mfma)");
}

template <typename T, int G, bool kSplit, int kMode = 0>
int launch_fog(const Params& p, dim3 grid, hipStream_t stream) {
  if (p.bias)
    return p.vscale ? launch_one<T, G, true, true, kSplit, kMode>(p, grid, stream)
                    : launch_one<T, G, true, false, kSplit, kMode>(p, grid, stream);
  return p.vscale ? launch_one<T, G, false, true, kSplit, kMode>(p, grid, stream)
                  : launch_one<T, G, false, false, kSplit, kMode>(p, grid, stream);
}

// The split and longest-first instances are separate: the plain loop keeps the
// register allocation it was tuned with (folding either into it cost the
// V-fog long-context shape 1-6 %).
template <typename T, int G>
int launch_split(const Params& p, dim3 grid, hipStream_t stream) {
  if (p.page_size > 16)  // pages of 16 * 2^k tokens (in query order)
    return p.direct_out ? launch_fog<T, G, false, 3>(p, grid, stream) : launch_fog<T, G, true, 3>(p, grid, stream);
  if (!p.direct_out) return launch_fog<T, G, true>(p, grid, stream);
  return p.reverse_q ? launch_fog<T, G, false, 2>(p, grid, stream) : launch_fog<T, G, false>(p, grid, stream);
}

template <typename T>
int launch_prefill(Params& p, hipStream_t stream) {
  const int kpos = kPfRows / p.G;
  // Varlen: the live (sequence, query tile) pairs are numbered along x.
  dim3 grid(div_up(p.C, kpos) * p.Hkv * (p.q_start ? p.B : 1), p.q_start ? 1 : p.B, max(p.num_splits, 1));
  // (The dense split instance numbers its (tile, split) units along x.)
  if (p.page_table == nullptr) {  // table-less pages (dense launchers): G 1, no bias
    if (p.num_splits > 1) {  // (tile, split) units along x (kernel header)
      const int nq = div_up(p.C, kPfRows), t0 = p.split_q0 / kPfRows;
      grid = dim3((unsigned)((t0 + (nq - t0) * p.num_splits) * p.Hkv), p.B, 1);
      if (p.D == 64)
        return p.vscale ? launch_one<T, 1, false, true, true, 1, 64>(p, grid, stream)
                        : launch_one<T, 1, false, false, true, 1, 64>(p, grid, stream);
      return p.vscale ? launch_one<T, 1, false, true, true, 1>(p, grid, stream)
                      : launch_one<T, 1, false, false, true, 1>(p, grid, stream);
    }
    if (p.D == 64)
      return p.vscale ? launch_one<T, 1, false, true, false, 1, 64>(p, grid, stream)
                      : launch_one<T, 1, false, false, false, 1, 64>(p, grid, stream);
    return p.vscale ? launch_one<T, 1, false, true, false, 1>(p, grid, stream)
                    : launch_one<T, 1, false, false, false, 1>(p, grid, stream);
  }
  switch (p.G) {
    case 1: return launch_split<T, 1>(p, grid, stream);
    case 2: return launch_split<T, 2>(p, grid, stream);
    case 4: return launch_split<T, 4>(p, grid, stream);
    case 8: return launch_split<T, 8>(p, grid, stream);
    case 16: return launch_split<T, 16>(p, grid, stream);
    default:
      set_error(KESSIE_ERR_UNSUPPORTED, "fog prefill (mfma): GQA ratio %d", p.G);
      return KESSIE_ERR_UNSUPPORTED;
  }
}

}  // namespace

bool prefill_mfma_ok(const Params& p, int dtype) {
  if (env_int("KESSIE_FORCE_GENERIC", 0)) return false;
  if (dtype != KESSIE_DTYPE_BF16 && dtype != KESSIE_DTYPE_F16) return false;
  // Head_dim 64 only on table-less pages (the dense launchers).
  if (!(p.D == 128 || (p.D == 64 && p.page_table == nullptr))) return false;
  // Pages of 16 * 2^k tokens (table-less pages: 16), block ids (page << k) below 2^31.
  if (p.page_size < 16 || (p.page_size & (p.page_size - 1)) != 0 || (p.page_table == nullptr && p.page_size != 16))
    return false;
  if (((int64_t)p.num_pages << (__builtin_ctz((unsigned)p.page_size) - 4)) >= (int64_t)1 << 31) return false;
  // Table-less pages: instantiated for the dense launchers' form only.
  if (p.page_table == nullptr && (p.dense_ppb <= 0 || p.G != 1 || p.bias)) return false;
  if (!(p.G == 1 || p.G == 2 || p.G == 4 || p.G == 8 || p.G == 16)) return false;
  if (!(p.sm_scale > 0.0f)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  if (p.page_stride % 8 || p.tok_stride % 8 || p.head_stride % 8) return false;
  // A page's stride in bytes below 2^32 (the kernel forms page offsets as 32 x 32-bit products).
  if (p.page_stride < 0 || p.page_stride * 2 >= ((int64_t)1 << 32)) return false;
  if (p.q_bs % 8 || p.q_is % 8 || p.q_hs % 8 || p.o_bs % 4 || p.o_is % 4 || p.o_hs % 4) return false;
  return true;
}

int prefill_mfma(Params& p, int dtype, hipStream_t stream) {
  if (!prefill_mfma_ok(p, dtype)) {
    set_error(KESSIE_ERR_UNSUPPORTED, "fog prefill (mfma): unsupported shape");
    return KESSIE_ERR_UNSUPPORTED;
  }
  return dtype == KESSIE_DTYPE_BF16 ? launch_prefill<bf16_t>(p, stream) : launch_prefill<f16_t>(p, stream);
}

}  // namespace attn
}  // namespace kessie
