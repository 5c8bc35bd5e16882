// HBM ceiling probes for gfx950: the practical bandwidth of the access
// patterns the hot-path kernels use, measured with no arithmetic in the way,
// so each kernel's achieved GB/s can be set against what its pattern allows on
// the same device (the spec peak is the other reference point).
//   stream read   16-byte non-temporal loads over a contiguous buffer
//   copy          the same loads, each stored to a second buffer (read + write)
//   page RMW      the RoPE remap's pattern: for every token row of every page in
//                 a list, read and rewrite `row_bytes` (the K half of the row),
//                 16-byte non-temporal accesses, each 32-bit word incremented so
//                 the store is not a no-op
// Each probe launches one 256-thread workgroup per tile of kU x 256 16-byte
// chunks (no grid-stride loop): the fastest shape of a sweep over chunks per
// thread {1, 2, 4, 8} and workgroups per CU {4, 8, 16, 32, one per tile} on
// MI355X -- read 4 per thread, copy 1, page RMW 2.
#include "common.h"

namespace kessie {
namespace probe {
namespace {

constexpr int kThreads = 256;
constexpr int kReadU = 4;
constexpr int kCopyU = 1;
constexpr int kRmwU = 2;

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

// Chunk i of the work is chunk (i % chunks) of token row ((i / chunks) % rows)
// of page pages[i / (rows * chunks)]; invalid page ids are skipped.
__global__ __launch_bounds__(kThreads) void page_rmw_kernel(char* __restrict__ pool, int64_t page_bytes,
                                                            int64_t row_stride, int rows, int row_bytes,
                                                            const int32_t* __restrict__ pages, int n_pages,
                                                            int num_pages) {
  const int chunks = row_bytes / 16;
  const int per_page = rows * chunks;
  const int64_t total = (int64_t)n_pages * per_page;
  const int64_t base = (int64_t)blockIdx.x * (kRmwU * kThreads) + threadIdx.x;
  u32x4 v[kRmwU];
  u32x4* q[kRmwU];
#pragma unroll
  for (int k = 0; k < kRmwU; ++k) {
    const int64_t i = base + k * kThreads;
    q[k] = nullptr;
    if (i < total) {
      const int pid = pages[i / per_page];
      const int r = (int)(i % per_page);
      if (pid >= 0 && pid < num_pages) {
        q[k] = reinterpret_cast<u32x4*>(pool + (int64_t)pid * page_bytes + (int64_t)(r / chunks) * row_stride +
                                        16 * (r % chunks));
        v[k] = __builtin_nontemporal_load(q[k]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kRmwU; ++k)
    if (q[k]) __builtin_nontemporal_store(v[k] + 1u, q[k]);
}

int grid_for(int64_t items, int per_thread) {
  return (int)div_up(items, (int64_t)per_thread * kThreads);
}

}  // namespace
}  // namespace probe
}  // namespace kessie

using namespace kessie;
using namespace kessie::probe;

extern "C" int kessie_probe_stream_read(const void* buf, int64_t bytes, void* sink, void* stream) {
  clear_error();
  KESSIE_REQUIRE(buf && sink && bytes > 0 && bytes % 16 == 0 && aligned16(buf), KESSIE_ERR_INVALID,
                 "probe read: %lld bytes", (long long)bytes);
  const int64_t n = bytes / 16;
  KESSIE_REQUIRE(div_up(n, (int64_t)kReadU * kThreads) < (1LL << 31), KESSIE_ERR_INVALID, "probe read: too large");
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid_for(n, kReadU)), dim3(kThreads), 0, as_stream(stream),
                     static_cast<const u32x4*>(buf), n, static_cast<uint32_t*>(sink));
  return check_launch("probe read");
}

extern "C" int kessie_probe_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  clear_error();
  KESSIE_REQUIRE(dst && src && bytes > 0 && bytes % 16 == 0 && aligned16(dst) && aligned16(src), KESSIE_ERR_INVALID,
                 "probe copy: %lld bytes", (long long)bytes);
  const int64_t n = bytes / 16;
  KESSIE_REQUIRE(div_up(n, (int64_t)kCopyU * kThreads) < (1LL << 31), KESSIE_ERR_INVALID, "probe copy: too large");
  hipLaunchKernelGGL(copy_kernel, dim3(grid_for(n, kCopyU)), dim3(kThreads), 0, as_stream(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n);
  return check_launch("probe copy");
}

extern "C" int kessie_probe_page_rmw(void* pool, int64_t page_bytes, int64_t row_stride_bytes, int rows_per_page,
                                     int row_bytes, const int32_t* pages, int n_pages, int num_pages, void* stream) {
  clear_error();
  KESSIE_REQUIRE(pool && pages && n_pages >= 0 && rows_per_page > 0 && row_bytes > 0 && row_bytes % 16 == 0 &&
                     page_bytes % 16 == 0 && row_stride_bytes % 16 == 0 && aligned16(pool) &&
                     (int64_t)(rows_per_page - 1) * row_stride_bytes + row_bytes <= page_bytes,
                 KESSIE_ERR_INVALID, "probe page rmw: bad geometry");
  if (n_pages == 0) return KESSIE_OK;
  const int64_t items = (int64_t)n_pages * rows_per_page * (row_bytes / 16);
  KESSIE_REQUIRE(div_up(items, (int64_t)kRmwU * kThreads) < (1LL << 31), KESSIE_ERR_INVALID,
                 "probe page rmw: too large");
  hipLaunchKernelGGL(page_rmw_kernel, dim3(grid_for(items, kRmwU)), dim3(kThreads), 0, as_stream(stream),
                     static_cast<char*>(pool), page_bytes, row_stride_bytes, rows_per_page, row_bytes, pages, n_pages,
                     num_pages);
  return check_launch("probe page rmw");
}
