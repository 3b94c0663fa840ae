// Device metadata and request routing for the verify step: everything that turns
// a host routing descriptor (mapped pinned memory or a device copy) into the
// per-row tables, lengths and KV write addresses the attention and KV writers
// read, plus the per-slot hidden-state / token gathers and scatters.  All launches
// have grids fixed by tensor capacities and read counts only from memory, so a
// HIP graph captured once replays with new descriptor contents.
//
//  * rlt_route_slots_kernel       -- vllm_rlt/kernels/routing.py:7-11 slots_kernel
//  * rlt_route_metadata_kernel    -- routing.py:14-49 metadata_kernel
//  * rlt_route_rows_kernel        -- routing.py:52-82 gather_kernel / scatter_kernel
//  * rlt_route_segments_kernel    -- routing.py:85-144 gather_segments_kernel /
//                                    scatter_segments_kernel
//  * rlt_expand_kv_kernel         -- vllm_rlt/kernels/metadata.py:7-24 expand_kv_addresses
//  * rlt_depth_tables_kernel      -- the per-row depth-table gather of
//                                    vllm_rlt/worker/async_speculative.py:449-470
//
// Every index read from memory (slot, plane, position, segment bounds) is checked
// against the buffer it addresses: an out-of-range gather source reads zeros, an
// out-of-range destination is skipped, and a block address that cannot be formed
// is -1 (which the KV writers skip).  Rows move as the widest unit (16, 8, 4, 2 or
// 1 bytes) that the row size, strides and base addresses allow.

#include "common.h"
#include "rlt_mi355x.h"

namespace {

constexpr int kThreads = 256;

// Copies (or, with src == nullptr, zero-fills) one unit of `unit` bytes.
__device__ __forceinline__ void move_unit(uint8_t* dst, const uint8_t* src, int unit) {
  switch (unit) {
    case 16: *(uint4*)dst = src ? *(const uint4*)src : make_uint4(0, 0, 0, 0); break;
    case 8: *(uint2*)dst = src ? *(const uint2*)src : make_uint2(0, 0); break;
    case 4: *(uint32_t*)dst = src ? *(const uint32_t*)src : 0u; break;
    case 2: *(uint16_t*)dst = src ? *(const uint16_t*)src : (uint16_t)0; break;
    default: *dst = src ? *src : (uint8_t)0; break;
  }
}

__global__ __launch_bounds__(kThreads) void rlt_route_slots_kernel(
    const int64_t* __restrict__ desc, int64_t* __restrict__ slots, int64_t count, int64_t size) {
  const int64_t row = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (row < size) slots[row] = row < count ? desc[3 * row] : 0;
}

// One workgroup per output row (size rows; the first `count` are live).
__global__ __launch_bounds__(kThreads) void rlt_route_metadata_kernel(
    const int64_t* __restrict__ desc, const int32_t* __restrict__ tables, int64_t table_rows,
    int width, int page, int planes, int64_t* __restrict__ slots, int64_t* __restrict__ positions,
    int32_t* __restrict__ lengths, int64_t* __restrict__ blocks, int64_t* __restrict__ offsets,
    int32_t* __restrict__ out_tables, int64_t out_stride, int out_width, int64_t count) {
  const int64_t row = blockIdx.x;
  const bool live = row < count;
  const int64_t slot = live ? desc[3 * row] : 0;
  const int64_t depth = live ? desc[3 * row + 1] : 0;
  const int64_t pos = live ? desc[3 * row + 2] : 0;
  const int64_t plane = planes > 1 ? depth : 0;
  const int64_t trow = slot * planes + plane;
  const bool table_ok = live && slot >= 0 && plane >= 0 && plane < planes && trow < table_rows;
  const int32_t* table = tables + trow * width;
  if (threadIdx.x == 0) {
    slots[row] = slot;
    positions[row] = pos;
    lengths[row] = live ? (int32_t)(pos + 1) : 0;
    if (live) {
      const bool page_ok = table_ok && pos >= 0 && pos / page < width;
      blocks[row] = page_ok ? (int64_t)table[pos / page] : -1;
      offsets[row] = pos % page;
    }
  }
  for (int col = threadIdx.x; col < out_width; col += kThreads)
    out_tables[row * out_stride + col] = table_ok ? table[col] : 0;
}

// Row gather (kScatter false): out[row] = pool[slots[row]] for row < count, zeros
// for count <= row < size.  Row scatter (kScatter true): pool[slots[row]] = in[row]
// for row < count.  Grid (rows, spans of kThreads units).
template <bool kScatter>
__global__ __launch_bounds__(kThreads) void rlt_route_rows_kernel(
    const uint8_t* __restrict__ src, int64_t src_stride, uint8_t* __restrict__ dst,
    int64_t dst_stride, const int64_t* __restrict__ slots, int64_t pool_rows, int64_t count,
    int64_t row_bytes, int unit) {
  const int64_t row = blockIdx.x;
  const int64_t o = ((int64_t)blockIdx.y * kThreads + threadIdx.x) * unit;
  if (o >= row_bytes) return;
  if (kScatter) {
    const int64_t slot = slots[row];
    if (slot < 0 || slot >= pool_rows) return;
    move_unit(dst + slot * dst_stride + o, src + row * src_stride + o, unit);
  } else {
    int64_t slot = row < count ? slots[row] : -1;
    const bool ok = slot >= 0 && slot < pool_rows;
    move_unit(dst + row * dst_stride + o, ok ? src + slot * src_stride + o : nullptr, unit);
  }
}

// Segments int64 [S, 5] = (slot, row offset in the slot, row count, batch row start,
// keep).  Gather: out[start + r] = pool[slot * rows_per_slot + offset + r].  Scatter
// (kept segments only): pool[slot * rows_per_slot + offset + r] = in[start + r].
// Grid (segments, max_rows, spans).
template <bool kScatter>
__global__ __launch_bounds__(kThreads) void rlt_route_segments_kernel(
    const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, const int64_t* __restrict__ seg,
    int64_t pool_slots, int64_t rows_per_slot, int64_t pool_stride, int64_t batch_rows,
    int64_t batch_stride, int64_t row_bytes, int unit) {
  const int64_t* s = seg + 5 * (int64_t)blockIdx.x;
  const int64_t r = blockIdx.y;
  const int64_t o = ((int64_t)blockIdx.z * kThreads + threadIdx.x) * unit;
  if (o >= row_bytes) return;
  const int64_t slot = s[0], offset = s[1], n = s[2], start = s[3];
  if (r >= n || (kScatter && s[4] == 0)) return;
  const int64_t prow = offset + r, brow = start + r;
  if (slot < 0 || slot >= pool_slots || prow < 0 || prow >= rows_per_slot || brow < 0 ||
      brow >= batch_rows)
    return;
  const int64_t p = (slot * rows_per_slot + prow) * pool_stride + o;
  const int64_t b = brow * batch_stride + o;
  if (kScatter)
    move_unit(dst + p, src + b, unit);
  else
    move_unit(dst + b, src + p, unit);
}

__global__ __launch_bounds__(kThreads) void rlt_expand_kv_kernel(
    const int64_t* __restrict__ positions, const int32_t* __restrict__ sequences,
    const int32_t* __restrict__ tables, int64_t num_sequences, int width, int page,
    int64_t* __restrict__ blocks, int64_t* __restrict__ offsets, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t pos = positions[i];
  const int64_t seq = sequences[i];
  const bool ok = seq >= 0 && seq < num_sequences && pos >= 0 && pos / page < width;
  blocks[i] = ok ? (int64_t)tables[seq * width + pos / page] : -1;
  offsets[i] = pos % page;
}

// One workgroup per row: table = tables[row, depth[row]], the write address of
// positions[row] in it, and lengths = pos + 1 (0 for inactive rows).  Offsets use
// the floor modulo of the torch formula.
__global__ __launch_bounds__(kThreads) void rlt_depth_tables_kernel(
    const int32_t* __restrict__ tables, int64_t row_stride, int64_t plane_stride, int planes,
    int width, const int64_t* __restrict__ depth, const int64_t* __restrict__ positions,
    const uint8_t* __restrict__ active, int block_size, int32_t* __restrict__ out_table,
    int64_t out_stride, int64_t* __restrict__ blocks, int64_t* __restrict__ offsets,
    int32_t* __restrict__ lengths) {
  const int64_t row = blockIdx.x;
  const int64_t d = depth[row];
  const int64_t pos = positions[row];
  const bool ok = d >= 0 && d < planes;
  const int32_t* table = tables + row * row_stride + d * plane_stride;
  if (threadIdx.x == 0) {
    int64_t page = pos / block_size, off = pos % block_size;
    if (off < 0) {  // floor division and modulo, as torch's // and %
      off += block_size;
      page -= 1;
    }
    blocks[row] = ok && page >= 0 && page < width ? (int64_t)table[page] : -1;
    offsets[row] = off;
    lengths[row] = (active && !active[row]) ? 0 : (int32_t)(pos + 1);
  }
  for (int col = threadIdx.x; col < width; col += kThreads)
    out_table[row * out_stride + col] = ok ? table[col] : 0;
}

// Widest unit dividing the row size, both strides and both base addresses.
inline int unit_for(int64_t row_bytes, int64_t a_stride, int64_t b_stride, const void* a,
                    const void* b) {
  const uint64_t all = (uint64_t)row_bytes | (uint64_t)a_stride | (uint64_t)b_stride |
                       (uint64_t)(uintptr_t)a | (uint64_t)(uintptr_t)b;
  for (int u = 16; u > 1; u >>= 1)
    if (all % u == 0) return u;
  return 1;
}

inline bool grid_ok(int64_t x, int64_t y, int64_t z = 1) {
  return x > 0 && x <= 0x7fffffff && y > 0 && y <= 65535 && z > 0 && z <= 65535;
}

}  // namespace

extern "C" {

int rlt_route_slots(const int64_t* descriptor, int64_t* slots, int64_t count, int64_t size,
                    hipStream_t stream) {
  if (count < 0 || size < 0 || count > size) return RLT_ERR_ARGUMENT;
  if (size == 0) return RLT_OK;
  if (!slots || (count > 0 && !descriptor)) return RLT_ERR_ARGUMENT;
  hipLaunchKernelGGL(rlt_route_slots_kernel, dim3((unsigned)((size + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, descriptor, slots, count, size);
  return rlt_launch_status();
}

int rlt_route_metadata(const int64_t* descriptor, const int32_t* tables, int64_t table_rows,
                       int32_t width, int32_t page, int32_t planes, int64_t* slots,
                       int64_t* positions, int32_t* lengths, int64_t* blocks, int64_t* offsets,
                       int32_t* out_tables, int64_t out_stride, int32_t out_width, int64_t count,
                       int64_t size, hipStream_t stream) {
  if (count < 0 || size < 0 || count > size || table_rows < 0 || width < 1 || page < 1 ||
      planes < 1 || out_width < 0 || out_width > width || out_stride < out_width)
    return RLT_ERR_ARGUMENT;
  if (size == 0) return RLT_OK;
  if (!slots || !positions || !lengths || !blocks || !offsets || !out_tables ||
      (count > 0 && (!descriptor || !tables)))
    return RLT_ERR_ARGUMENT;
  if (size > 0x7fffffff) return RLT_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(rlt_route_metadata_kernel, dim3((unsigned)size), dim3(kThreads), 0, stream,
                     descriptor, tables, table_rows, width, page, planes, slots, positions,
                     lengths, blocks, offsets, out_tables, out_stride, out_width, count);
  return rlt_launch_status();
}

int rlt_route_gather(const void* pool, int64_t pool_rows, int64_t pool_stride,
                     const int64_t* slots, void* out, int64_t out_stride, int64_t count,
                     int64_t size, int64_t row_elems, int32_t elt_bytes, hipStream_t stream) {
  if (pool_rows < 0 || count < 0 || size < 0 || count > size || row_elems < 0 || elt_bytes < 1 ||
      pool_stride < 0 || out_stride < row_elems)
    return RLT_ERR_ARGUMENT;
  if (size == 0 || row_elems == 0) return RLT_OK;
  if (!out || (count > 0 && (!pool || !slots))) return RLT_ERR_ARGUMENT;
  const int64_t row_bytes = row_elems * elt_bytes;
  const int unit = unit_for(row_bytes, pool_stride * elt_bytes, out_stride * elt_bytes, pool, out);
  const int64_t spans = (row_bytes / unit + kThreads - 1) / kThreads;
  if (!grid_ok(size, spans)) return RLT_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(rlt_route_rows_kernel<false>, dim3((unsigned)size, (unsigned)spans),
                     dim3(kThreads), 0, stream, (const uint8_t*)pool, pool_stride * elt_bytes,
                     (uint8_t*)out, out_stride * elt_bytes, slots, pool_rows, count, row_bytes,
                     unit);
  return rlt_launch_status();
}

int rlt_route_scatter(const void* values, int64_t values_stride, const int64_t* slots, void* pool,
                      int64_t pool_rows, int64_t pool_stride, int64_t count, int64_t row_elems,
                      int32_t elt_bytes, hipStream_t stream) {
  if (pool_rows < 0 || count < 0 || row_elems < 0 || elt_bytes < 1 || values_stride < 0 ||
      pool_stride < row_elems)
    return RLT_ERR_ARGUMENT;
  if (count == 0 || row_elems == 0) return RLT_OK;
  if (!values || !slots || !pool) return RLT_ERR_ARGUMENT;
  const int64_t row_bytes = row_elems * elt_bytes;
  const int unit =
      unit_for(row_bytes, values_stride * elt_bytes, pool_stride * elt_bytes, values, pool);
  const int64_t spans = (row_bytes / unit + kThreads - 1) / kThreads;
  if (!grid_ok(count, spans)) return RLT_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(rlt_route_rows_kernel<true>, dim3((unsigned)count, (unsigned)spans),
                     dim3(kThreads), 0, stream, (const uint8_t*)values, values_stride * elt_bytes,
                     (uint8_t*)pool, pool_stride * elt_bytes, slots, pool_rows, count, row_bytes,
                     unit);
  return rlt_launch_status();
}

static int route_segments(bool scatter, const void* src, void* dst, const int64_t* segments,
                          int64_t num_segments, int64_t max_rows, int64_t pool_slots,
                          int64_t rows_per_slot, int64_t pool_stride, int64_t batch_rows,
                          int64_t batch_stride, int64_t row_elems, int32_t elt_bytes,
                          const void* pool, const void* batch, hipStream_t stream) {
  if (num_segments < 0 || max_rows < 0 || pool_slots < 0 || rows_per_slot < 0 ||
      batch_rows < 0 || row_elems < 0 || elt_bytes < 1 || pool_stride < row_elems ||
      batch_stride < row_elems)
    return RLT_ERR_ARGUMENT;
  if (num_segments == 0 || max_rows == 0 || row_elems == 0) return RLT_OK;
  if (!src || !dst || !segments) return RLT_ERR_ARGUMENT;
  const int64_t row_bytes = row_elems * elt_bytes;
  const int unit = unit_for(row_bytes, pool_stride * elt_bytes, batch_stride * elt_bytes, pool,
                            batch);
  const int64_t spans = (row_bytes / unit + kThreads - 1) / kThreads;
  if (!grid_ok(num_segments, max_rows, spans)) return RLT_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)num_segments, (unsigned)max_rows, (unsigned)spans);
  if (scatter)
    hipLaunchKernelGGL(rlt_route_segments_kernel<true>, grid, dim3(kThreads), 0, stream,
                       (const uint8_t*)src, (uint8_t*)dst, segments, pool_slots, rows_per_slot,
                       pool_stride * elt_bytes, batch_rows, batch_stride * elt_bytes, row_bytes,
                       unit);
  else
    hipLaunchKernelGGL(rlt_route_segments_kernel<false>, grid, dim3(kThreads), 0, stream,
                       (const uint8_t*)src, (uint8_t*)dst, segments, pool_slots, rows_per_slot,
                       pool_stride * elt_bytes, batch_rows, batch_stride * elt_bytes, row_bytes,
                       unit);
  return rlt_launch_status();
}

int rlt_route_gather_segments(const void* pool, int64_t pool_slots, int64_t rows_per_slot,
                              int64_t pool_stride, const int64_t* segments, int64_t num_segments,
                              int64_t max_rows, void* out, int64_t out_rows, int64_t out_stride,
                              int64_t row_elems, int32_t elt_bytes, hipStream_t stream) {
  return route_segments(false, pool, out, segments, num_segments, max_rows, pool_slots,
                        rows_per_slot, pool_stride, out_rows, out_stride, row_elems, elt_bytes,
                        pool, out, stream);
}

int rlt_route_scatter_segments(const void* values, int64_t values_rows, int64_t values_stride,
                               const int64_t* segments, int64_t num_segments, int64_t max_rows,
                               void* pool, int64_t pool_slots, int64_t rows_per_slot,
                               int64_t pool_stride, int64_t row_elems, int32_t elt_bytes,
                               hipStream_t stream) {
  return route_segments(true, values, pool, segments, num_segments, max_rows, pool_slots,
                        rows_per_slot, pool_stride, values_rows, values_stride, row_elems,
                        elt_bytes, pool, values, stream);
}

int rlt_expand_kv_addresses(const int64_t* positions, const int32_t* sequences,
                            const int32_t* tables, int64_t num_sequences, int32_t width,
                            int32_t page, int64_t* blocks, int64_t* offsets, int64_t n,
                            hipStream_t stream) {
  if (n < 0 || num_sequences < 0 || width < 1 || page < 1) return RLT_ERR_ARGUMENT;
  if (n == 0) return RLT_OK;
  if (!positions || !sequences || !tables || !blocks || !offsets) return RLT_ERR_ARGUMENT;
  if (n > 0x7fffffffLL * kThreads) return RLT_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(rlt_expand_kv_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, positions, sequences, tables, num_sequences, width,
                     page, blocks, offsets, n);
  return rlt_launch_status();
}

int rlt_depth_tables(const int32_t* tables, int64_t row_stride, int64_t plane_stride,
                     int32_t planes, int32_t width, const int64_t* depth,
                     const int64_t* positions, const uint8_t* active, int32_t block_size,
                     int32_t* out_table, int64_t out_stride, int64_t* blocks, int64_t* offsets,
                     int32_t* lengths, int64_t n, hipStream_t stream) {
  if (n < 0 || planes < 1 || width < 1 || block_size < 1 || out_stride < width)
    return RLT_ERR_ARGUMENT;
  if (n == 0) return RLT_OK;
  if (!tables || !depth || !positions || !out_table || !blocks || !offsets || !lengths)
    return RLT_ERR_ARGUMENT;
  if (n > 0x7fffffff) return RLT_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(rlt_depth_tables_kernel, dim3((unsigned)n), dim3(kThreads), 0, stream,
                     tables, row_stride, plane_stride, planes, width, depth, positions, active,
                     block_size, out_table, out_stride, blocks, offsets, lengths);
  return rlt_launch_status();
}

}  // extern "C"
