// KV write side of the paged pool on MI355X (gfx950): the step that precedes
// attention in every layer.
//
//  * rlt_kv_store_kernel: scatter of [rows, kv_heads, head_dim] K and V rows into
//    one layer's pool view [block, token, kv_head, dim] at (blocks[r], offsets[r]),
//    skipping rows whose mask entry is false or that lie at or past *active.
//    Replaces vllm_rlt/kernels/routing.py:183-223 masked_kv_store,
//    vllm_rlt/kernels/graph_kv.py write_graph_kv and the index_put of
//    vllm_rlt/core/kv_cache_manager.py:893-895.
//  * rlt_kv_store_fp8_kernel: the same scatter into an FP8 e4m3 pool with per-vector
//    scales: scale = max(amax * (1/448), FLT_MIN) (or a fixed scale), codes =
//    clamp(x / scale, +-448) with IEEE division, converted to e4m3fn by
//    round-to-nearest-even.  Bitwise equal to vllm_rlt/core/kv_cache_manager.py:50-61
//    quantize_fp8; replaces vllm_rlt/kernels/triton_attention.py:505-623 store_fp8.
//  * rlt_kv_finalize_kernel: the LAST_EXITED finalize copy.  For every descriptor
//    (slot, exit depth, position), every layer's K and V at the position's page
//    offset are copied from the exit plane's block to the same offset of the block
//    of every deeper plane.  Replaces vllm_rlt/kernels/routing.py:147-180
//    finalize_kernel (and the host form kv_cache_manager.py:1053-1076).
//
// All three are bandwidth-bound copies; workgroups move 16-byte vectors where the
// element counts and addresses allow it.  Rows or descriptors that address memory
// outside the pool (block ids, offsets, slots or positions out of range) are
// skipped: nothing is written there (the reference's kernels would write out of
// bounds).

#include "common.h"
#include "fp8_codec.h"
#include "rlt_mi355x.h"

#include <math.h>

namespace {

using rlt_fp8::nan_max;

// One workgroup of 256 threads per (row, 16-byte-vector span); each thread moves
// one 16-byte vector of K and one of V when kVec, else one element.
template <bool kVec>
__global__ __launch_bounds__(256) void rlt_kv_store_kernel(
    const uint8_t* __restrict__ k, const uint8_t* __restrict__ v, int64_t k_row, int64_t k_head,
    int64_t v_row, int64_t v_head, uint8_t* __restrict__ kc, uint8_t* __restrict__ vc,
    int64_t c_block, int64_t c_token, int64_t c_head, const int64_t* __restrict__ blocks,
    const int64_t* __restrict__ offsets, const uint8_t* __restrict__ mask,
    const int32_t* __restrict__ active, int heads, int row_bytes, int elt, int64_t num_blocks,
    int block_size) {
  const int64_t r = blockIdx.x;
  if (active && r >= (int64_t)*active) return;
  if (mask && !mask[r]) return;
  const int64_t blk = blocks[r], off = offsets[r];
  if (blk < 0 || blk >= num_blocks || off < 0 || off >= block_size) return;  // outside the pool
  const int unit = kVec ? 16 : elt;
  const int per_head = row_bytes / unit;
  const int i = (int)(blockIdx.y * blockDim.x + threadIdx.x);
  if (i >= heads * per_head) return;
  const int h = i / per_head;
  const int o = (i - h * per_head) * unit;
  const int64_t dst = (blk * c_block + off * c_token + h * c_head) * elt + o;
  const int64_t ks = (r * k_row + h * k_head) * elt + o;
  const int64_t vs = (r * v_row + h * v_head) * elt + o;
  if (kVec) {
    *(uint4*)(kc + dst) = *(const uint4*)(k + ks);
    *(uint4*)(vc + dst) = *(const uint4*)(v + vs);
  } else {
    for (int b = 0; b < elt; ++b) {
      kc[dst + b] = k[ks + b];
      vc[dst + b] = v[vs + b];
    }
  }
}

// One wave per (row, kv head): K then V of the vector, quantized and scattered.
template <int DT>
__global__ __launch_bounds__(256) void rlt_kv_store_fp8_kernel(
    const void* __restrict__ k, const void* __restrict__ v, int64_t k_row, int64_t k_head,
    int64_t v_row, int64_t v_head, uint8_t* __restrict__ kc, uint8_t* __restrict__ vc,
    int64_t c_block, int64_t c_token, int64_t c_head, float* __restrict__ ks,
    float* __restrict__ vs, int64_t s_block, int64_t s_token, int64_t s_head,
    const int64_t* __restrict__ blocks, const int64_t* __restrict__ offsets,
    const uint8_t* __restrict__ mask, const int32_t* __restrict__ active, int64_t rows,
    int heads, int dim, int fixed, float fixed_scale, int64_t num_blocks, int block_size) {
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (item >= rows * heads) return;
  const int64_t r = item / heads;
  const int h = (int)(item - r * heads);
  if (active && r >= (int64_t)*active) return;
  if (mask && !mask[r]) return;
  const int64_t blk = blocks[r], off = offsets[r];
  if (blk < 0 || blk >= num_blocks || off < 0 || off >= block_size) return;  // outside the pool
  const int64_t c_at = blk * c_block + off * c_token + h * c_head;
  const int64_t s_at = blk * s_block + off * s_token + h * s_head;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const void* src = which ? v : k;
    const int64_t base = which ? (r * v_row + h * v_head) : (r * k_row + h * k_head);
    uint8_t* codes = which ? vc : kc;
    float* scales = which ? vs : ks;
    float x[4];
    float amax = 0.f;  // NaN-propagating, as torch's amax
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = lane + 64 * e;
      x[e] = d < dim ? load_as_f32<DT>(src, base + d) : 0.f;
      amax = nan_max(amax, fabsf(x[e]));
    }
    for (int o = 32; o >= 1; o >>= 1) amax = nan_max(amax, __shfl_xor(amax, o, RLT_WAVE));
    const float scale = fixed ? fixed_scale : rlt_fp8::dynamic_scale(amax);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = lane + 64 * e;
      if (d < dim) codes[c_at + d] = (uint8_t)rlt_fp8::encode(x[e], scale);
    }
    if (lane == 0) scales[s_at] = scale;
  }
}

// grid (descriptors, planes, spans): for target plane > exit depth, copies
// `channels` bytes per layer from the exit plane's block to the target plane's
// block at the position's page offset.
__global__ __launch_bounds__(256) void rlt_kv_finalize_kernel(
    const int64_t* __restrict__ desc, const int32_t* __restrict__ tables, int64_t slots,
    int width, int planes, int block_size, int layers, int64_t num_blocks,
    uint8_t* __restrict__ kc, uint8_t* __restrict__ vc, int64_t block_stride,
    int64_t layer_stride, int64_t token_stride, int64_t bytes_per_token, int vec) {
  const int64_t d = blockIdx.x;
  const int target = blockIdx.y;
  const int64_t slot = desc[3 * d];
  const int64_t depth = desc[3 * d + 1];
  const int64_t pos = desc[3 * d + 2];
  if (target <= depth || target >= planes || depth < 0) return;
  if (slot < 0 || slot >= slots || pos < 0 || pos >= (int64_t)width * block_size) return;
  const int64_t page = pos / block_size;
  const int64_t src_blk = tables[(slot * planes + depth) * width + page];
  const int64_t dst_blk = tables[(slot * planes + target) * width + page];
  // table entries outside the pool (unallocated pages) copy nothing
  if (src_blk < 0 || src_blk >= num_blocks || dst_blk < 0 || dst_blk >= num_blocks) return;
  const int64_t per_layer = bytes_per_token / vec;
  const int64_t i = (int64_t)blockIdx.z * blockDim.x + threadIdx.x;
  if (i >= (int64_t)layers * per_layer) return;
  const int64_t layer = i / per_layer;
  const int64_t o = (i - layer * per_layer) * vec;
  const int64_t rel = layer * layer_stride + (pos % block_size) * token_stride + o;
  const int64_t s = src_blk * block_stride + rel, t = dst_blk * block_stride + rel;
  if (vec == 16) {
    *(uint4*)(kc + t) = *(const uint4*)(kc + s);
    *(uint4*)(vc + t) = *(const uint4*)(vc + s);
  } else {
    for (int b = 0; b < vec; ++b) {
      kc[t + b] = kc[s + b];
      vc[t + b] = vc[s + b];
    }
  }
}

inline int elt_size(int dtype) {
  return dtype == RLT_F32 ? 4 : dtype == RLT_FP8_E4M3 ? 1 : 2;
}

}  // namespace

extern "C" {

int rlt_kv_store(const void* k, const void* v, int64_t k_row_stride, int64_t k_head_stride,
                 int64_t v_row_stride, int64_t v_head_stride, void* key_cache, void* value_cache,
                 int64_t c_block_stride, int64_t c_token_stride, int64_t c_head_stride,
                 int64_t num_blocks, int32_t block_size, const int64_t* blocks,
                 const int64_t* offsets, const uint8_t* mask, const int32_t* active, int64_t rows,
                 int32_t kv_heads, int32_t head_dim, int32_t dtype, hipStream_t stream) {
  if (rows < 0 || kv_heads < 1 || head_dim < 1 || dtype < RLT_F32 || dtype > RLT_FP8_E4M3 ||
      num_blocks < 0 || block_size < 1)
    return RLT_ERR_ARGUMENT;
  if (rows == 0) return RLT_OK;
  if (!k || !v || !key_cache || !value_cache || !blocks || !offsets) return RLT_ERR_ARGUMENT;
  if (rows > 0x7fffffff) return RLT_ERR_UNSUPPORTED;
  const int elt = elt_size(dtype);
  const int row_bytes = head_dim * elt;
  // 16-byte vectors when every row / head / token start is 16-byte aligned
  const bool vec = row_bytes % 16 == 0 && ((k_row_stride | k_head_stride | v_row_stride |
                                            v_head_stride | c_block_stride | c_token_stride |
                                            c_head_stride) * elt) % 16 == 0 &&
                   ((uintptr_t)k | (uintptr_t)v | (uintptr_t)key_cache | (uintptr_t)value_cache) % 16 == 0;
  const int unit = vec ? 16 : elt;
  const int64_t items = (int64_t)kv_heads * (row_bytes / unit);
  const dim3 grid((unsigned)rows, (unsigned)((items + 255) / 256));
  if (vec)
    hipLaunchKernelGGL(rlt_kv_store_kernel<true>, grid, dim3(256), 0, stream, (const uint8_t*)k,
                       (const uint8_t*)v, k_row_stride, k_head_stride, v_row_stride, v_head_stride,
                       (uint8_t*)key_cache, (uint8_t*)value_cache, c_block_stride, c_token_stride,
                       c_head_stride, blocks, offsets, mask, active, kv_heads, row_bytes, elt,
                       num_blocks, block_size);
  else
    hipLaunchKernelGGL(rlt_kv_store_kernel<false>, grid, dim3(256), 0, stream, (const uint8_t*)k,
                       (const uint8_t*)v, k_row_stride, k_head_stride, v_row_stride, v_head_stride,
                       (uint8_t*)key_cache, (uint8_t*)value_cache, c_block_stride, c_token_stride,
                       c_head_stride, blocks, offsets, mask, active, kv_heads, row_bytes, elt,
                       num_blocks, block_size);
  return rlt_launch_status();
}

int rlt_kv_store_fp8(const void* k, const void* v, int32_t src_dtype, int64_t k_row_stride,
                     int64_t k_head_stride, int64_t v_row_stride, int64_t v_head_stride,
                     void* key_codes, void* value_codes, int64_t c_block_stride,
                     int64_t c_token_stride, int64_t c_head_stride, float* key_scale,
                     float* value_scale, int64_t s_block_stride, int64_t s_token_stride,
                     int64_t s_head_stride, int64_t num_blocks, int32_t block_size,
                     const int64_t* blocks, const int64_t* offsets, const uint8_t* mask,
                     const int32_t* active, int64_t rows, int32_t kv_heads, int32_t head_dim,
                     int32_t has_fixed_scale, float fixed_scale, hipStream_t stream) {
  if (rows < 0 || kv_heads < 1 || head_dim < 1 || num_blocks < 0 || block_size < 1)
    return RLT_ERR_ARGUMENT;
  if (rows == 0) return RLT_OK;
  if (!k || !v || !key_codes || !value_codes || !key_scale || !value_scale || !blocks || !offsets)
    return RLT_ERR_ARGUMENT;
  if (head_dim > 256 || rows > 0x7fffffff || rows * kv_heads > 0x1fffffffLL)
    return RLT_ERR_UNSUPPORTED;  // one wave holds 256 elements; the grid's x extent
  const int64_t items = rows * kv_heads;
  const dim3 grid((unsigned)((items + 3) / 4));
#define RLT_FP8_STORE(DT)                                                                         \
  hipLaunchKernelGGL(rlt_kv_store_fp8_kernel<DT>, grid, dim3(256), 0, stream, k, v, k_row_stride, \
                     k_head_stride, v_row_stride, v_head_stride, (uint8_t*)key_codes,             \
                     (uint8_t*)value_codes, c_block_stride, c_token_stride, c_head_stride,        \
                     key_scale, value_scale, s_block_stride, s_token_stride, s_head_stride,       \
                     blocks, offsets, mask, active, rows, kv_heads, head_dim,                     \
                     has_fixed_scale != 0, fixed_scale, num_blocks, block_size)
  switch (src_dtype) {
    case RLT_F32: RLT_FP8_STORE(RLT_F32); break;
    case RLT_BF16: RLT_FP8_STORE(RLT_BF16); break;
    case RLT_F16: RLT_FP8_STORE(RLT_F16); break;
    default: return RLT_ERR_UNSUPPORTED;
  }
#undef RLT_FP8_STORE
  return rlt_launch_status();
}

int rlt_kv_finalize(const int64_t* descriptors, int64_t count, const int32_t* tables,
                    int64_t slots, int32_t width, int32_t planes, int32_t block_size,
                    int32_t layers, int64_t num_blocks, void* key_pool, void* value_pool,
                    int64_t block_stride, int64_t layer_stride, int64_t token_stride,
                    int64_t bytes_per_token, int32_t elt_bytes, hipStream_t stream) {
  if (count < 0 || slots < 0 || width < 1 || planes < 1 || block_size < 1 || layers < 1 ||
      num_blocks < 0 || bytes_per_token < 1 || elt_bytes < 1)
    return RLT_ERR_ARGUMENT;
  if (count == 0 || planes == 1) return RLT_OK;
  if (!descriptors || !tables || !key_pool || !value_pool) return RLT_ERR_ARGUMENT;
  if (count > 0x7fffffff) return RLT_ERR_UNSUPPORTED;
  const int64_t bs = block_stride * elt_bytes, ls = layer_stride * elt_bytes,
                ts = token_stride * elt_bytes;
  const bool vec = bytes_per_token % 16 == 0 && (bs | ls | ts) % 16 == 0 &&
                   ((uintptr_t)key_pool | (uintptr_t)value_pool) % 16 == 0;
  const int unit = vec ? 16 : 1;
  const int64_t items = (int64_t)layers * (bytes_per_token / unit);
  const dim3 grid((unsigned)count, (unsigned)planes, (unsigned)((items + 255) / 256));
  hipLaunchKernelGGL(rlt_kv_finalize_kernel, grid, dim3(256), 0, stream, descriptors, tables,
                     slots, width, planes, block_size, layers, num_blocks, (uint8_t*)key_pool,
                     (uint8_t*)value_pool, bs, ls, ts, bytes_per_token, unit);
  return rlt_launch_status();
}

}  // extern "C"
