// Shared by the attention translation units: the parameter block every
// attention kernel takes, masking / addressing helpers, and the split-K
// partial workspace layout.
#pragma once

#include <cstdlib>

#include "common.h"

namespace kessie {
namespace attn {

constexpr float kNegInf = -__builtin_huge_valf();

struct Params {
  // Query row (b, i, h) at q + b*q_bs + i*q_is + h*q_hs; output likewise.
  const void* q;
  int64_t q_bs, q_is, q_hs;
  void* out;
  int64_t o_bs, o_is, o_hs;
  // Key/value element (page, slot, h, d) at k + page*page_stride +
  // slot*tok_stride + h*head_stride + d (v likewise).  page_table == nullptr:
  // dense, sequence b's token t at b*page_stride + t*tok_stride.
  const void* k;
  const void* v;
  int num_pages;
  int64_t page_stride, tok_stride, head_stride;
  int page_size;
  const int32_t* page_table;
  int64_t table_stride;
  const int32_t* ctx_lens;  // nullptr: every sequence has ctx_const tokens
  int ctx_const;
  int max_ctx;
  const float* vscale;
  int64_t vs_bs;
  const float* bias;
  int64_t bias_bs;
  int B, C, Hq, Hkv, G, D;
  // Variable-length prefill (nullptr: every sequence has C queries at
  // q + b*q_bs): sequence b's queries are tokens q_start[b] - q_start[0] ..
  // q_start[b+1] - q_start[0] - 1 of q (and of out), C the longest of them.
  const int32_t* q_start;
  // Table-less 16-token pages (page_table == nullptr, MFMA prefill only):
  // page j of sequence b is page b * dense_ppb + j, as in a dense [B][H][N][D]
  // tensor with page_stride = 16 * D and head_stride = N * D.
  int dense_ppb;
  // Causal chunk covering most of its context over several grid rounds: the
  // MFMA prefill dispatches its query tiles longest first (host-set).
  int reverse_q;
  int window, causal;
  float sm_scale;
  int num_splits;
  // Dense launchers' split (table-less pages, split instance): query tiles
  // from position split_q0 on (the longest ones) take num_splits workgroups,
  // the others one; partial rows cover positions split_q0 .. C-1 only.  The
  // combine writes its row (b, i, h) at position i + q0_off.
  int split_q0;
  int q0_off;
  int direct_out;      // 1: the main kernel writes the normalised output
  int launch_combine;  // host side: follow the main kernel with the combine
  int balanced;        // decode split partials: units assigned by pages (decode_seq_of_unit)
  float* ws_o;  // [B*C*Hq][S][D]
  float* ws_m;  // [B*C*Hq][S]
  float* ws_l;  // [B*C*Hq][S]
};

// A sequence length as the kernels use it: at most max_ctx and the page
// table's capacity, at least 0.
__device__ __forceinline__ int clamp_ctx(const Params& p, int ctx) {
  ctx = min(ctx, p.max_ctx);
  if (p.page_table) {
    const int64_t cap = p.table_stride * (int64_t)p.page_size;
    if ((int64_t)ctx > cap) ctx = (int)cap;
  }
  return max(ctx, 0);
}
__device__ __forceinline__ int seq_ctx(const Params& p, int b) {
  return clamp_ctx(p, p.ctx_lens ? p.ctx_lens[b] : p.ctx_const);
}

// Element offset of token t of sequence b, or -1 when its page id is invalid.
__device__ __forceinline__ int64_t token_offset(const Params& p, int b, int t) {
  if (p.page_table == nullptr) return (int64_t)b * p.page_stride + (int64_t)t * p.tok_stride;
  const int pid = p.page_table[(int64_t)b * p.table_stride + t / p.page_size];
  if (pid < 0 || pid >= p.num_pages) return -1;
  return (int64_t)pid * p.page_stride + (int64_t)(t % p.page_size) * p.tok_stride;
}

__device__ __forceinline__ bool key_visible(int q_pos, int t, int window, int causal) {
  const int dist = q_pos - t;
  if (causal && dist < 0) return false;
  if (window > 0 && (dist < 0 || dist >= window)) return false;
  return true;
}

// Row index into the partial workspace / output for (b, i, h).
__device__ __forceinline__ int64_t row_id(const Params& p, int b, int i, int h) {
  return ((int64_t)b * p.C + i) * p.Hq + h;
}

template <typename T>
__device__ __forceinline__ void store_out(const Params& p, int b, int i, int h, int d, float val) {
  T* o = static_cast<T*>(p.out);
  o[(int64_t)b * p.o_bs + (int64_t)i * p.o_is + (int64_t)h * p.o_hs + d] = from_f32<T>(val);
}

// Key range [lo, hi) a set of query positions [qmin, qmax] can see.
__device__ __forceinline__ void key_range(const Params& p, int ctx, int qmin, int qmax, int* lo, int* hi) {
  int h = p.causal ? min(ctx, qmax + 1) : ctx;
  int l = 0;
  if (p.window > 0) {
    l = max(0, qmin - p.window + 1);
    h = min(h, qmax + 1);
  }
  *lo = l;
  *hi = max(h, l);
}

// Split-K partials: o[rows][S][D] fp32, then m[rows][S] and l[rows][S], each
// starting on a 256-byte boundary.
inline size_t partial_bytes(int64_t rows, int S, int D) {
  const size_t o = (size_t)rows * S * D * sizeof(float);
  const size_t ml = (size_t)rows * S * sizeof(float);
  return o + 2 * ((ml + 255) / 256 * 256);
}

inline void carve_workspace(Params& p, void* ws, int64_t rows) {
  char* c = static_cast<char*>(ws);
  p.ws_o = reinterpret_cast<float*>(c);
  c += (size_t)rows * p.num_splits * p.D * sizeof(float);
  p.ws_m = reinterpret_cast<float*>(c);
  c += ((size_t)rows * p.num_splits * sizeof(float) + 255) / 256 * 256;
  p.ws_l = reinterpret_cast<float*>(c);
}

inline int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  if (v == nullptr || *v == '\0') return dflt;
  return atoi(v);
}

// MFMA chunked prefill (fog_prefill.hip).  Returns KESSIE_ERR_UNSUPPORTED
// without launching when the shape is not one it handles.
int prefill_mfma(Params& p, int dtype, hipStream_t stream);
bool prefill_mfma_ok(const Params& p, int dtype);

// fp32 chunked prefill on MFMA (fog_prefill_f32.hip): p.num_splits from
// prefill_f32_splits; with more than one the partials go to p.ws_* for the
// caller's combine.
bool prefill_f32_ok(const Params& p, int dtype);
int prefill_f32_splits(int B, int C, int Hkv, int G, int max_ctx);
int prefill_f32(const Params& p, hipStream_t stream);
int device_cus();

}  // namespace attn
}  // namespace kessie
