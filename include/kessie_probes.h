/*
 * kessie_probes.h -- C ABI of libkessie_probes.so, the measurement-only
 * companion of libkessie_mi355x.so.  Nothing here is part of the product
 * library or of the reference's interface: these kernels measure the
 * practical HBM bandwidth of the hot path's access patterns on the device
 * (no arithmetic in the way), so that each product kernel's achieved GB/s
 * can be compared with what its pattern allows.  bench.py builds and loads
 * it for its HBM-ceiling line.
 *
 * All pointers are device pointers; `stream` is a hipStream_t passed as
 * void*.  Each call returns 0, or a KESSIE_PROBE_ERR_* code having launched
 * nothing (bad argument) or after a failed launch.
 */
#ifndef KESSIE_PROBES_H
#define KESSIE_PROBES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility push(default)
#endif

#define KESSIE_PROBE_ERR_INVALID 1
#define KESSIE_PROBE_ERR_HIP 4

/* Read `bytes` (multiple of 16, 16-byte aligned) with 16-byte non-temporal
 * loads; `sink` is one uint32 the kernel may write. */
int kessie_probe_stream_read(const void* buf, int64_t bytes, void* sink, void* stream);

/* Copy `bytes` from src to dst with 16-byte non-temporal loads and stores. */
int kessie_probe_copy(void* dst, const void* src, int64_t bytes, void* stream);

/* For each page id p of pages[0..n_pages) inside [0, num_pages) and each row
 * r < rows_per_page: read row_bytes (16 x a power of two) at src_pool +
 * p*page_bytes + r*row_stride_bytes and write them, every 32-bit word
 * incremented by one, to the same offset of dst_pool (dst_pool == src_pool:
 * in place; dst_pool == NULL: read only, `sink` one uint32 the kernel may
 * write).  One 256-thread workgroup per chunks_per_thread x 256 sixteen-byte
 * chunks of one page (chunks_per_thread in {1, 2, 4, 8}); non-temporal
 * accesses, each thread's loads all issued before its stores. */
int kessie_probe_page_rows(const void* src_pool, void* dst_pool, int64_t page_bytes, int64_t row_stride_bytes,
                           int rows_per_page, int row_bytes, const int32_t* pages, int n_pages, int num_pages,
                           int chunks_per_thread, void* sink, void* stream);

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* KESSIE_PROBES_H */
