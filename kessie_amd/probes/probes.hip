// HBM ceiling probes for gfx950 (measurement only; built into
// libkessie_probes.so, never into the product library).  Each measures the
// practical bandwidth of an access pattern the hot-path kernels use, with no
// arithmetic in the way, so a kernel's achieved GB/s can be set against what
// its pattern allows on the same device (the spec peak is the other reference
// point).
//   stream read   16-byte non-temporal loads over a contiguous buffer
//   copy          the same loads, each stored to a second buffer
//   page rows     for every token row of every page in a list, read
//                 `row_bytes` at the row start of the source pool and write
//                 them (each 32-bit word + 1) to the same offset of the
//                 destination pool; source == destination is the RoPE remap's
//                 in-place read-modify-write, row_bytes == row stride the
//                 whole-row form, a sorted list the page-ordered form.
// One 256-thread workgroup per tile of kU x 256 16-byte chunks (no grid-stride
// loop); the page-rows probe's tiles lie inside one page and kU is an argument
// (1, 2, 4 or 8 chunks per thread: at the remap's shape 8 is one whole page's
// K half per workgroup, read completely before any of it is written).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kessie_probes.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kReadU = 4;
constexpr int kCopyU = 1;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t grid_for(int64_t items, int per_thread) {
  return (items + (int64_t)per_thread * kThreads - 1) / ((int64_t)per_thread * kThreads);
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : KESSIE_PROBE_ERR_HIP; }

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n,
                                                               uint32_t* __restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * (kReadU * kThreads) + threadIdx.x;
  u32x4 v[kReadU];
#pragma unroll
  for (int k = 0; k < kReadU; ++k) {
    const int64_t i = base + k * kThreads;
    v[k] = i < n ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
  }
  u32x4 acc = v[0];
#pragma unroll
  for (int k = 1; k < kReadU; ++k) acc ^= v[k];
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[0] = x;  // keeps the loads; practically never taken
}

__global__ __launch_bounds__(kThreads) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                        int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// One workgroup per tile of kU x 256 sixteen-byte chunks of one listed page
// (grid = n_pages x tiles_per_page, the decomposition of the page gather):
// chunk c of the page's row-major work list is chunk (c & (2^log2_chunks - 1))
// of token row (c >> log2_chunks).  Page ids outside [0, num_pages) are
// skipped.  Every load of a thread is issued before its first store; with
// dst == nullptr the chunks are only read (folded into `sink`).
template <int kU>
__global__ __launch_bounds__(kThreads) void page_rows_kernel(const char* src, char* dst, int64_t page_bytes,
                                                             int64_t row_stride, int log2_chunks, int per_page,
                                                             int tiles_per_page, const int32_t* __restrict__ pages,
                                                             int num_pages, uint32_t* __restrict__ sink) {
  const int page = blockIdx.x / tiles_per_page;
  const int tile = blockIdx.x - page * tiles_per_page;
  const int pid = pages[page];
  if (pid < 0 || pid >= num_pages) return;
  const char* sbase = src + (int64_t)pid * page_bytes;
  const int cmask = (1 << log2_chunks) - 1;
  u32x4 v[kU];
  int64_t off[kU];
#pragma unroll
  for (int k = 0; k < kU; ++k) {
    const int c = (tile * kU + k) * kThreads + threadIdx.x;
    off[k] = -1;
    if (c < per_page) {
      off[k] = (int64_t)(c >> log2_chunks) * row_stride + 16 * (c & cmask);
      v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(sbase + off[k]));
    }
  }
  if (dst == nullptr) {
    u32x4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < kU; ++k)
      if (off[k] >= 0) acc ^= v[k];
    const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (x == 0x9e3779b9u) sink[0] = x;  // keeps the loads; practically never taken
    return;
  }
  char* dbase = dst + (int64_t)pid * page_bytes;
#pragma unroll
  for (int k = 0; k < kU; ++k)
    if (off[k] >= 0) __builtin_nontemporal_store(v[k] + 1u, reinterpret_cast<u32x4*>(dbase + off[k]));
}

int log2_exact(int64_t x) {
  int l = 0;
  while (((int64_t)1 << l) < x) ++l;
  return ((int64_t)1 << l) == x ? l : -1;
}

}  // namespace

extern "C" int kessie_probe_stream_read(const void* buf, int64_t bytes, void* sink, void* stream) {
  if (!buf || !sink || bytes <= 0 || bytes % 16 != 0 || !aligned16(buf)) return KESSIE_PROBE_ERR_INVALID;
  const int64_t n = bytes / 16;
  const int64_t grid = grid_for(n, kReadU);
  if (grid >= (1LL << 31)) return KESSIE_PROBE_ERR_INVALID;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const u32x4*>(buf), n,
                     static_cast<uint32_t*>(sink));
  return launched();
}

extern "C" int kessie_probe_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  if (!dst || !src || bytes <= 0 || bytes % 16 != 0 || !aligned16(dst) || !aligned16(src))
    return KESSIE_PROBE_ERR_INVALID;
  const int64_t n = bytes / 16;
  const int64_t grid = grid_for(n, kCopyU);
  if (grid >= (1LL << 31)) return KESSIE_PROBE_ERR_INVALID;
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)grid), dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n);
  return launched();
}

extern "C" int kessie_probe_page_rows(const void* src_pool, void* dst_pool, int64_t page_bytes,
                                      int64_t row_stride_bytes, int rows_per_page, int row_bytes,
                                      const int32_t* pages, int n_pages, int num_pages, int chunks_per_thread,
                                      void* sink, void* stream) {
  const int log2_chunks = log2_exact(row_bytes / 16);
  if (!src_pool || !pages || (!dst_pool && !sink) || n_pages < 0 || num_pages <= 0 || rows_per_page <= 0 ||
      row_bytes <= 0 || row_bytes % 16 != 0 || log2_chunks < 0 || page_bytes % 16 != 0 ||
      row_stride_bytes % 16 != 0 || !aligned16(src_pool) || (dst_pool && !aligned16(dst_pool)) ||
      (int64_t)(rows_per_page - 1) * row_stride_bytes + row_bytes > page_bytes ||
      (int64_t)rows_per_page * (row_bytes / 16) > (1 << 30))
    return KESSIE_PROBE_ERR_INVALID;
  if (n_pages == 0) return 0;
  const int per_page = rows_per_page * (row_bytes / 16);
  const int tiles = (int)grid_for(per_page, chunks_per_thread);
  const int64_t grid = (int64_t)n_pages * tiles;
  if (grid >= (1LL << 31)) return KESSIE_PROBE_ERR_INVALID;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const char* src = static_cast<const char*>(src_pool);
  char* dst = static_cast<char*>(dst_pool);
  uint32_t* sk = static_cast<uint32_t*>(sink);
  switch (chunks_per_thread) {
    case 1:
      hipLaunchKernelGGL(page_rows_kernel<1>, dim3((unsigned)grid), dim3(kThreads), 0, s, src, dst, page_bytes,
                         row_stride_bytes, log2_chunks, per_page, tiles, pages, num_pages, sk);
      break;
    case 2:
      hipLaunchKernelGGL(page_rows_kernel<2>, dim3((unsigned)grid), dim3(kThreads), 0, s, src, dst, page_bytes,
                         row_stride_bytes, log2_chunks, per_page, tiles, pages, num_pages, sk);
      break;
    case 4:
      hipLaunchKernelGGL(page_rows_kernel<4>, dim3((unsigned)grid), dim3(kThreads), 0, s, src, dst, page_bytes,
                         row_stride_bytes, log2_chunks, per_page, tiles, pages, num_pages, sk);
      break;
    case 8:
      hipLaunchKernelGGL(page_rows_kernel<8>, dim3((unsigned)grid), dim3(kThreads), 0, s, src, dst, page_bytes,
                         row_stride_bytes, log2_chunks, per_page, tiles, pages, num_pages, sk);
      break;
    default:
      return KESSIE_PROBE_ERR_INVALID;
  }
  return launched();
}
