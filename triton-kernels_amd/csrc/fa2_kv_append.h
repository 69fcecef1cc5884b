// fa2_kv_append.h - writes new K/V rows into paged caches (the producer side
// of the paged layout the attention kernels read).
//
// Sequence b's new rows k_new[indptr[b] + j] (j < indptr[b+1] - indptr[b])
// go to logical position n = start[b] + j of that sequence, i.e. to cache
// row table[b][n / P] * P + n % P - the page arithmetic of the paged
// attention kernels (attention.py:575-594, decode.py:130-149), the format
// the reference builds on the host in tests/test_attention.py:101-134 and
// benchmarks/attention.py:351-431.
//
// A pure copy, bound by HBM: each row is read once and written once.
// Workgroup = 256 threads over 64 new rows: the lanes of the first wave
// locate one row each (binary search of indptr, then the table entry) into
// LDS; then all 256 lanes copy 16-byte pieces of K and V, several in
// flight per lane.  A row whose logical page lies outside the table width,
// or whose table entry is outside [0, num_pages), is not written (a caller
// error must not become an out-of-bounds store).  Without v_new only K is
// written.
#pragma once

#include "fa2_device.h"

namespace fa2 {

constexpr int kAppendRows = 64;
constexpr int kAppendThreads = 256;

struct AppendArgs {
  const char* k_new;
  const char* v_new;
  char* k_cache;
  char* v_cache;
  const int32_t* indptr;
  const int32_t* start;  // may be null: every sequence starts at 0
  const int32_t* k_table;
  const int32_t* v_table;
  int64_t new_ts, new_hs;      // byte strides (row, head) of k_new / v_new
  int64_t cache_ts, cache_hs;  // byte strides (row, head) of the caches
  int64_t k_table_stride, v_table_stride;
  int64_t num_pages;
  int32_t batch, heads, row_chunks, head_chunks;  // 16-byte pieces per row / per head
  int32_t num_rows, page_size, table_width;
};

__global__ __launch_bounds__(kAppendThreads) void fa2_kv_append_kernel(AppendArgs a) {
  __shared__ int64_t src_off[kAppendRows];
  __shared__ int64_t dk_off[kAppendRows];
  __shared__ int64_t dv_off[kAppendRows];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * kAppendRows;

  if (tid < kAppendRows) {
    const int t = r0 + tid;
    int64_t so = -1, dk = -1, dv = -1;
    if (t < a.num_rows) {
      // sequence of row t: the last b with indptr[b] <= t
      int lo = 0, hi = a.batch - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.indptr[mid] <= t) lo = mid;
        else hi = mid - 1;
      }
      const int b = lo;
      const int j = t - a.indptr[b];
      const int n = (a.start ? a.start[b] : 0) + j;
      const int lp = n / a.page_size;
      if (j >= 0 && t < a.indptr[b + 1] && n >= 0 && lp < a.table_width) {
        const int64_t pk = a.k_table[b * a.k_table_stride + lp];
        const int64_t pv = a.v_new ? a.v_table[b * a.v_table_stride + lp] : -1;
        const int64_t off = n - static_cast<int64_t>(lp) * a.page_size;
        so = static_cast<int64_t>(t) * a.new_ts;
        if (pk >= 0 && pk < a.num_pages) dk = (pk * a.page_size + off) * a.cache_ts;
        if (pv >= 0 && pv < a.num_pages) dv = (pv * a.page_size + off) * a.cache_ts;
      }
    }
    src_off[tid] = so;
    dk_off[tid] = dk;
    dv_off[tid] = dv;
  }
  __syncthreads();

  const int rows = min(kAppendRows, a.num_rows - r0);
  const int total = rows * a.row_chunks;
  // Every byte is read once and written once: non-temporal loads and stores
  // (a1: 4.70 -> 4.86 TB/s in alternating runs on one box).
  constexpr int kUnroll = 4;
  for (int base = 0; base < total; base += kAppendThreads * kUnroll) {
    u32x4 kx[kUnroll], vx[kUnroll];
    int64_t kd[kUnroll], vd[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int idx = base + u * kAppendThreads + tid;
      kd[u] = vd[u] = -1;
      if (idx < total) {
        const int r = idx / a.row_chunks;
        const int c = idx - r * a.row_chunks;
        const int h = c / a.head_chunks;
        const int64_t col = static_cast<int64_t>(c - h * a.head_chunks) * 16;
        const int64_t so = src_off[r];
        if (so >= 0) {
          const int64_t s = so + h * a.new_hs + col;
          if (dk_off[r] >= 0) {
            kx[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.k_new + s));
            kd[u] = dk_off[r] + h * a.cache_hs + col;
          }
          if (dv_off[r] >= 0) {
            vx[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.v_new + s));
            vd[u] = dv_off[r] + h * a.cache_hs + col;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (kd[u] >= 0) __builtin_nontemporal_store(kx[u], reinterpret_cast<u32x4*>(a.k_cache + kd[u]));
      if (vd[u] >= 0) __builtin_nontemporal_store(vx[u], reinterpret_cast<u32x4*>(a.v_cache + vd[u]));
    }
  }
}

}  // namespace fa2
