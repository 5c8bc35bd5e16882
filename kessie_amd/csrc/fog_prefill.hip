// Chunked-prefill fog attention on MFMA for gfx950 (bf16 / f16, head_dim 128,
// 16-token pages, GQA ratio G dividing 32).
//
// Math: the last C rows of kessie_hip_kernels.py:577-593 over ctx = L + C
// tokens (query i at position ctx-C+i, causal, window, fog weights scaling V
// rows or a logit bias), fp32 accumulation, online softmax.
//
// Work decomposition: one workgroup = 256 query rows (256/G positions x the G
// heads of one kv head) of one sequence; 8 waves x 32 rows.  The workgroup
// streams its kv head's keys in tiles of 64 (4 pages): K row-major and V
// transposed ([d][key], key pairs packed into 32-bit LDS writes) into LDS,
// the next tile's global loads in flight while the current one is consumed.
// Per wave and tile:
//   S^T (64 keys x 32 rows) = K Q^T   on v_mfma_f32_32x32x16 (16 MFMAs);
//     row i of a 32-key A operand is key swap23(i), so the accumulator's
//     register v of lane l holds key 16(v/8) + 8(l/32) + (v%8) of row l%32:
//     the softmax is lane-local plus one xor-32 shuffle, and p is already in
//     the B-operand layout of PV (8 consecutive keys per lane half);
//   O^T (128 d x 32 rows) += V^T P^T  on v_mfma_f32_32x32x16 (16 MFMAs),
//     the V^T A operand is one 16-byte LDS read.
// Grid index x = qtile * Hkv + g, so with 8 kv heads (and the hardware's
// round-robin of workgroups over the 8 XCDs) every workgroup of kv head g
// sits on one XCD and the query tiles of that head share its keys in L2.
#include "attn_common.h"

namespace kessie {
namespace attn {
namespace {

constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * 64;
constexpr int kPfRows = kPfWaves * 32;  // query rows (position, head) per workgroup
constexpr int kPfKT = 64;               // keys per tile (4 pages)
constexpr int kPfKRow = 128 + 8;        // K tile row stride (elements)
constexpr int kPfVRow = kPfKT + 8;      // V^T tile row stride (elements)

typedef float f32x16 __attribute__((ext_vector_type(16)));

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

template <typename T, int G>
__global__ __launch_bounds__(kPfThreads) void prefill_mfma_kernel(Params p) {
  typedef typename Mma32<T>::v8 v8;
  typedef typename Mma32<T>::v4 v4;
  constexpr int kPos = kPfRows / G;  // query positions per workgroup
  __shared__ __align__(16) T ks[kPfKT * kPfKRow];
  __shared__ __align__(16) T vts[128 * kPfVRow];
  __shared__ float fws[kPfKT];  // fog weight per key of the tile (V mode)
  __shared__ float fbs[kPfKT];  // fog bias per key of the tile
  __shared__ int kok[kPfKT];    // key present (in range, valid page)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int g = blockIdx.x % p.Hkv;
  const int qtile = blockIdx.x / p.Hkv;
  const int b = blockIdx.y;
  const int ctx = seq_ctx(p, b);

  // Rows of the workgroup and the key range they see (uniform).
  const int qi_first = qtile * kPos;
  const int qi_last = min(p.C, qi_first + kPos) - 1;
  const int qmin = max(ctx - p.C + qi_first, 0);
  const int qmax = ctx - p.C + qi_last;
  if (qi_last < qi_first || qmax < 0) return;
  int lo = 0, hi = 0;
  key_range(p, ctx, qmin, qmax, &lo, &hi);
  const int t_begin = (lo / kPfKT) * kPfKT;
  const int n_tiles = hi > t_begin ? div_up(hi - t_begin, kPfKT) : 0;

  // This lane's query row.
  const int frow = wave * 32 + col;
  const int qi = qi_first + frow / G;
  const int head = g * G + frow % G;
  const int q_pos = ctx - p.C + qi;
  const bool row_ok = qi <= qi_last && q_pos >= 0;

  // B operand of S^T = K Q^T: d-step s holds d = 16s + 8*half .. +8.
  v8 qv[8];
  {
    const T* qr = static_cast<const T*>(p.q) + (int64_t)b * p.q_bs + (int64_t)min(qi, qi_last) * p.q_is +
                  (int64_t)head * p.q_hs;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (row_ok) {
        qv[s] = *reinterpret_cast<const v8*>(qr + 16 * s + 8 * half);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[s][e] = static_cast<T>(0.0f);
      }
    }
  }

  // Loader mapping: K rows kr and kr+32, V key pair (2kr, 2kr+1), chunk kc.
  const int kc = tid & 15, kr = tid >> 4;
  const T* kbase = static_cast<const T*>(p.k) + (int64_t)g * p.head_stride + 8 * kc;
  const T* vbase = static_cast<const T*>(p.v) + (int64_t)g * p.head_stride + 8 * kc;
  const int32_t* table = p.page_table + (int64_t)b * p.table_stride;
  auto key_off = [&](int key) -> int64_t {
    if (key < lo || key >= hi) return -1;
    const int pid = table[key >> 4];
    if (pid < 0 || pid >= p.num_pages) return -1;
    return (int64_t)pid * p.page_stride + (int64_t)(key & 15) * p.tok_stride;
  };
  v8 kreg[2], vreg[2];
  float fw_r = 0.0f, fb_r = 0.0f;
  int ok_r = 0;
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int64_t o = key_off(t0 + kr + 32 * r);
      if (o >= 0) {
        kreg[r] = *reinterpret_cast<const v8*>(kbase + o);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) kreg[r][e] = static_cast<T>(0.0f);
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int64_t o = key_off(t0 + 2 * kr + r);
      if (o >= 0) {
        vreg[r] = *reinterpret_cast<const v8*>(vbase + o);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) vreg[r][e] = static_cast<T>(0.0f);
      }
    }
    if (tid < kPfKT) {
      const int key = t0 + tid;
      ok_r = key_off(key) >= 0 ? 1 : 0;
      fw_r = (ok_r && p.vscale) ? p.vscale[(int64_t)b * p.vs_bs + key] : 1.0f;
      fb_r = (ok_r && p.bias) ? p.bias[(int64_t)b * p.bias_bs + key] : 0.0f;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int r = 0; r < 2; ++r) *reinterpret_cast<v8*>(ks + (kr + 32 * r) * kPfKRow + 8 * kc) = kreg[r];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t packed = bits16(vreg[0][e]) | (bits16(vreg[1][e]) << 16);
      *reinterpret_cast<uint32_t*>(vts + (8 * kc + e) * kPfVRow + 2 * kr) = packed;
    }
    if (tid < kPfKT) {
      fws[tid] = fw_r;
      fbs[tid] = fb_r;
      kok[tid] = ok_r;
    }
  };

  f32x16 oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16{};
  float m_run = kNegInf, l_run = 0.0f;
  const float scale = p.sm_scale;

  if (n_tiles > 0) {
    load_tile(t_begin);
    store_tile();
  }
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int t0 = t_begin + t * kPfKT;
    const bool more = t + 1 < n_tiles;
    if (more) load_tile(t0 + kPfKT);
    // Interior tile: every key present and visible to every row of the
    // workgroup (uniform), so no per-element mask.
    bool pages_ok = t0 >= lo && t0 + kPfKT <= hi;
    if (pages_ok) {
#pragma unroll
      for (int pg = 0; pg < kPfKT / 16; ++pg) {
        const int pid = table[(t0 >> 4) + pg];
        pages_ok = pages_ok && pid >= 0 && pid < p.num_pages;
      }
    }
    const bool interior = pages_ok && t0 + kPfKT - 1 <= qmin && (p.window == 0 || t0 > qmax - p.window);

    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = f32x16{};
      const T* krow = ks + (32 * kb + swap23(col)) * kPfKRow + 8 * half;
#pragma unroll
      for (int s = 0; s < 8; ++s) sacc[kb] = Mma32<T>::mma(*reinterpret_cast<const v8*>(krow + 16 * s), qv[s], sacc[kb]);
    }
    // Scores of this lane's row for keys 32kb + 16(v/8) + 8*half + (v%8).
    float mloc = kNegInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kl = 32 * kb + 16 * (v >> 3) + 8 * half + (v & 7);
        float s = sacc[kb][v] * scale;
        if (p.bias) s += fbs[kl];
        if (!(interior && row_ok)) {
          const bool ok = row_ok && kok[kl] && key_visible(q_pos, t0 + kl, p.window, p.causal);
          s = ok ? s : kNegInf;
        }
        sacc[kb][v] = s;
        mloc = fmaxf(mloc, s);
      }
    if (!row_ok) mloc = kNegInf;
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float mnew = fmaxf(m_run, mloc);
    const float alpha = (m_run == kNegInf) ? 0.0f : __expf(m_run - mnew);
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float s = sacc[kb][v];
        const float pr = (s == kNegInf) ? 0.0f : __expf(s - mnew);
        psum += pr;
        const int kl = 32 * kb + 16 * (v >> 3) + 8 * half + (v & 7);
        sacc[kb][v] = p.vscale ? pr * fws[kl] : pr;
      }
    psum += __shfl_xor(psum, 32);
    l_run = l_run * alpha + psum;
    m_run = mnew;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[i] *= alpha;
    }
    // O^T += V^T P^T over four 16-key steps.
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      v8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = static_cast<T>(sacc[s >> 1][8 * (s & 1) + e]);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const v8 a = *reinterpret_cast<const v8*>(vts + (32 * db + col) * kPfVRow + 16 * s + 8 * half);
        oacc[db] = Mma32<T>::mma(a, pb, oacc[db]);
      }
    }
    __syncthreads();  // every wave is done with this tile's LDS
    if (more) store_tile();
    __syncthreads();
  }

  // Lane (col, half) holds row frow at d = 32*db + 8*(v/4) + 4*half + (v%4).
  if (!row_ok) return;
  const float il = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  T* orow = static_cast<T*>(p.out) + (int64_t)b * p.o_bs + (int64_t)qi * p.o_is + (int64_t)head * p.o_hs;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int vq = 0; vq < 4; ++vq) {
      v4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = from_f32<T>(oacc[db][4 * vq + e] * il);
      *reinterpret_cast<v4*>(orow + 32 * db + 8 * vq + 4 * half) = o;
    }
}

template <typename T>
int launch_prefill(Params& p, hipStream_t stream) {
  const int kpos = kPfRows / p.G;
  dim3 grid(div_up(p.C, kpos) * p.Hkv, p.B);
  switch (p.G) {
    case 1: hipLaunchKernelGGL((prefill_mfma_kernel<T, 1>), grid, dim3(kPfThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL((prefill_mfma_kernel<T, 2>), grid, dim3(kPfThreads), 0, stream, p); break;
    case 4: hipLaunchKernelGGL((prefill_mfma_kernel<T, 4>), grid, dim3(kPfThreads), 0, stream, p); break;
    case 8: hipLaunchKernelGGL((prefill_mfma_kernel<T, 8>), grid, dim3(kPfThreads), 0, stream, p); break;
    default:
      set_error(KESSIE_ERR_UNSUPPORTED, "fog prefill (mfma): GQA ratio %d", p.G);
      return KESSIE_ERR_UNSUPPORTED;
  }
  return check_launch("fog prefill (mfma)");
}

}  // namespace

bool prefill_mfma_ok(const Params& p, int dtype) {
  if (env_int("KESSIE_FORCE_GENERIC", 0)) return false;
  if (dtype != KESSIE_DTYPE_BF16 && dtype != KESSIE_DTYPE_F16) return false;
  if (p.D != 128 || p.page_size != 16 || p.page_table == nullptr) return false;
  if (!(p.G == 1 || p.G == 2 || p.G == 4 || p.G == 8)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  if (p.page_stride % 8 || p.tok_stride % 8 || p.head_stride % 8) return false;
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
