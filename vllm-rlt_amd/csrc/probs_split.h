// Row-split form of the sampling-distribution kernel for calls without top-k or
// top-p (gfx950).
//
// rlt_probs_kernel (probabilities.hip) gives each logits row one 1024-thread
// workgroup, so a launch of n rows keeps at most n CUs busy, every row streams at the
// rate one CU pulls, and rows beyond one per CU run in further rounds.  Without a
// filter a row needs no selection, only its max and total, so the split form
// spreads each row over S workgroups of kThreads threads, each owning one contiguous
// slice (slice length L = kThreads * E, E elements per thread in registers), in two
// launches:
//
//   1. rlt_probs_slice_kernel, one workgroup per (row, slice): for every 4096-column
//      block b of the slice, its max m_b, NaN flag and float64 mass
//      z_b = sum exp2((l - m_b) c) (c = log2(e) / T), plus the slice's argmax key;
//   2. rlt_probs_write_kernel, one workgroup per (row, slice): the row max lmax and the
//      total z = sum_b z_b 2^((m_b - lmax) c), summed over the row's blocks by a fixed
//      lane tree, then out = exp2((l - lmax) c) / z for the slice, NaN rows as NaN.
//
// A block's statistics depend only on its own columns (thread t holds the same
// columns of a block whatever the slice length), so the results do not depend on
// the slicing; they equal the single-workgroup form's up to the order of the
// float64 total's summation.  Argmax-only rows (greedy targets next to the
// distributions) are extra slices of launch 1, finished in launch 2; the acceptance
// sampler's draft-row partial sums can ride as extra workgroups of launch 1, and the
// written rows' partial sums are formed in launch 2.  Included inside
// probabilities.hip's anonymous namespace, after the order-key helpers.

#pragma once

namespace split {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / RLT_WAVE;
constexpr int kMaxSlices = 16;
constexpr int kBlockCols = 4096;   // statistics block: 16 elements per thread
constexpr int kMaxBlocks = 64;     // V <= 262144: one lane per block in the row total

struct BlockStat {
  float m;                  // block max logit (NaN ignored)
  uint32_t nan;             // the block holds a NaN
  double z;                 // sum of exp2((l - m) c) (0 when m is not finite)
  unsigned long long best;  // argmax key of the slice, (order key, NaN highest) << 32 |
                            // ~column, in the slice's first block (0 in the others)
};

// Workspace view and the call's shape.
struct View {
  BlockStat* stats;  // [(n_dist + n_arg) * NB]
  int S, L, NB;      // slices per row, slice length, blocks per row
  int64_t n_dist;    // distribution rows
  int64_t n_arg;     // argmax-only rows (their statistics follow)
  int64_t* targets;  // argmax outputs, or nullptr
  int fused;         // distribution row r's argmax goes to targets[r]
  float* pm_out;     // torch-order row-sum partials of the written rows, or nullptr
                     // (row r, group g at pm_out + (r groups + g) 32; L % 8192 == 0)
  double* tile_sum;    // float64 totals of the written rows' 4096-column tiles, or
  uint32_t* tile_flags;  // nullptr (row r, tile k at [r tiles + k]; L % 4096 == 0)
  int tiles;           // tiles per row
  int skip_drawn;      // argmax-only rows listed in rows[] (n_dist <= kMaxDrawnScan) are
                       // skipped: the categorical draws that follow write their outputs
};

constexpr int kMaxDrawnScan = 4 * kThreads;  // rows[] entries an argmax slice scans

__device__ __forceinline__ int64_t argmax_column(unsigned long long best) {
  return (int64_t)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
}

// targets[i] for argmax-only row i from its blocks' keys (one thread per row).
// A skipped row (skip_drawn) has every key 0, which no scanned slice leaves (its first
// block's key holds ~column, nonzero), and keeps the output its draw writes.
__device__ __forceinline__ void finish_argmax_row(const View& v, int64_t i) {
  if (i >= v.n_arg || !v.targets) return;
  const BlockStat* st = v.stats + (v.n_dist + i) * v.NB;
  unsigned long long best = 0;
  for (int b = 0; b < v.NB; ++b) best = st[b].best > best ? st[b].best : best;
  if (v.skip_drawn && best == 0) return;
  v.targets[i] = argmax_column(best);
}

// ---------------------------------------------------------------- slice loads

// Element j of thread t in slice s: column s L + 4 (kThreads (j / 4) + t) + j % 4, so
// every group of four is one 16-byte (fp32) or 8-byte (16-bit) load.
template <int E>
__device__ __forceinline__ int64_t slice_col(int64_t c0, int j) {
  return c0 + 4 * ((int64_t)kThreads * (j >> 2) + threadIdx.x) + (j & 3);
}

// kVec: V % 4 == 0 and the row base aligned to four elements.  Padding reads NaN.
template <int DT, int E, bool kVec>
__device__ __forceinline__ void load_slice(const void* __restrict__ src, int64_t c0, int V,
                                           float (&x)[E]) {
  static_assert(E % 4 == 0, "four elements per load");
#pragma unroll
  for (int q = 0; q < E / 4; ++q) {
    const int64_t col = slice_col<E>(c0, 4 * q);
    if (kVec) {
      if (col < V) {
        if (DT == RLT_F32) {
          const float4 f = *(const float4*)((const float*)src + col);
          x[4 * q] = f.x;
          x[4 * q + 1] = f.y;
          x[4 * q + 2] = f.z;
          x[4 * q + 3] = f.w;
        } else {
          const uint2 u = *(const uint2*)((const uint16_t*)src + col);
          const uint16_t h[4] = {(uint16_t)(u.x & 0xffff), (uint16_t)(u.x >> 16),
                                 (uint16_t)(u.y & 0xffff), (uint16_t)(u.y >> 16)};
#pragma unroll
          for (int k = 0; k < 4; ++k)
            x[4 * q + k] = DT == RLT_BF16 ? bf16_bits_to_f32(h[k]) : f16_bits_to_f32(h[k]);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) x[4 * q + k] = NAN;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        x[4 * q + k] = col + k < V ? load_as_f32<DT>(src, col + k) : NAN;
    }
  }
}

// ---------------------------------------------------------------- block reductions

template <int N>
struct ReduceShared {
  float f[kWaves][N];
  double d[kWaves][N];
  uint32_t u[kWaves];
  uint32_t flag[kWaves];
};

// Block max of N floats and OR of a flag (every thread gets the results).
template <int N>
__device__ __forceinline__ void block_max_or(ReduceShared<N>& sh, float (&fm)[N], bool& flag) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < N; ++i)
    for (int off = 32; off >= 1; off >>= 1) fm[i] = fmaxf(fm[i], __shfl_xor(fm[i], off, RLT_WAVE));
  const bool any = __ballot(flag) != 0;
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < N; ++i) sh.f[w][i] = fm[i];
    sh.flag[w] = any;
  }
  __syncthreads();
  flag = false;
#pragma unroll
  for (int i = 0; i < N; ++i) fm[i] = sh.f[0][i];
  for (int k = 0; k < kWaves; ++k) {
#pragma unroll
    for (int i = 0; i < N; ++i) fm[i] = fmaxf(fm[i], sh.f[k][i]);
    flag |= sh.flag[k] != 0;
  }
  __syncthreads();
}

template <int N>
__device__ __forceinline__ uint32_t block_min_u32(ReduceShared<N>& sh, uint32_t x) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int off = 32; off >= 1; off >>= 1) x = min(x, (uint32_t)__shfl_xor(x, off, RLT_WAVE));
  if (lane == 0) sh.u[w] = x;
  __syncthreads();
  x = sh.u[0];
  for (int i = 1; i < kWaves; ++i) x = min(x, sh.u[i]);
  __syncthreads();
  return x;
}

// float64 sums of N values in a fixed order (lane tree, then waves in order).
template <int N>
__device__ __forceinline__ void block_sum(ReduceShared<N>& sh, double (&x)[N]) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < N; ++i)
    for (int off = 32; off >= 1; off >>= 1) x[i] += __shfl_xor(x[i], off, RLT_WAVE);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < N; ++i) sh.d[w][i] = x[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    x[i] = sh.d[0][i];
    for (int k = 1; k < kWaves; ++k) x[i] += sh.d[k][i];
  }
  __syncthreads();
}

// ---------------------------------------------------------------- launch 1

// Column of element j of this thread: base = c0 + 4 t (32 bits: V < 2^31).
template <int E>
__device__ __forceinline__ uint32_t elem_col(uint32_t base, int j) {
  return base + (uint32_t)(4 * kThreads * (j >> 2) + (j & 3));
}

// One slice's block statistics.  Element j lies in block j / 16 of the slice.  kFull:
// every element of the slice is a column of the row (no bounds tests).
template <int DT, int E, bool kVec, bool kFull>
__device__ __forceinline__ void slice_body(ReduceShared<E / 16>& sh, const void* __restrict__ src,
                                           int64_t c0, int V, bool dist, bool need_argmax,
                                           float temp, BlockStat* __restrict__ out, int nb_here) {
  constexpr int NB = E / 16;
  const int t = threadIdx.x;
  const uint32_t base = (uint32_t)(c0 + 4 * t);
  auto ok = [&](int j) { return kFull || (int64_t)elem_col<E>(base, j) < V; };
  float x[E];
  load_slice<DT, E, kVec>(src, c0, V, x);
  float m[NB];
  bool nan = false;
#pragma unroll
  for (int b = 0; b < NB; ++b) m[b] = -INFINITY;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    if (!ok(j)) continue;
    nan |= x[j] != x[j];
    m[j / 16] = fmaxf(m[j / 16], x[j]);  // NaN ignored
  }
  block_max_or<NB>(sh, m, nan);
  // argmax key: the first column holding the slice max (the first NaN when there is one)
  unsigned long long best = 0;
  if (need_argmax) {
    float ms = m[0];
#pragma unroll
    for (int b = 1; b < NB; ++b) ms = fmaxf(ms, m[b]);
    uint32_t col = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const bool hit = ok(j) && (nan ? x[j] != x[j] : x[j] == ms);
      col = hit ? min(col, elem_col<E>(base, j)) : col;
    }
    col = block_min_u32<NB>(sh, col);
    const uint32_t key = nan ? 0xffffffffu : order_key(ms);
    best = ((unsigned long long)key << 32) | (0xffffffffu - col);
  }
  double z[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) z[b] = 0.0;
  const float c = 1.44269504088896341f / temp;
  if (dist && isfinite(c) && !nan) {
#pragma unroll
    for (int j = 0; j < E; ++j)
      if (ok(j) && isfinite(m[j / 16]))
        z[j / 16] += (double)__builtin_amdgcn_exp2f((x[j] - m[j / 16]) * c);
    block_sum<NB>(sh, z);
  }
  if (t < nb_here) {
    // thread b writes block b's record (the slice's blocks that hold columns)
    float mb = m[0];
    double zb = z[0];
#pragma unroll
    for (int b = 1; b < NB; ++b) {
      mb = t == b ? m[b] : mb;
      zb = t == b ? z[b] : zb;
    }
    out[t].m = mb;
    out[t].nan = nan;
    out[t].z = isfinite(mb) ? zb : 0.0;
    out[t].best = t == 0 ? best : 0ull;
  }
}

// Workgroups [0, (n_dist + n_arg) S): slice statistics of distribution row r < n_dist
// (logits row rows[r], or r) or of argmax-only logits row r - n_dist; then the draft
// rows' float32 row-sum partials of the acceptance sampler (two 8192-float groups per
// workgroup) when qm_src is set.
template <int DT, int E, bool kVec>
__global__ __launch_bounds__(kThreads) void rlt_probs_slice_kernel(
    const void* __restrict__ logits, const int64_t* __restrict__ rows, int64_t n_src,
    int64_t row_stride, int V, const float* __restrict__ temperature, View v,
    const float* __restrict__ qm_src, int64_t qm_rows, float* __restrict__ qm_out) {
  __shared__ union {
    ReduceShared<E / 16> red;
    cascade::ChunkSums cs[kThreads / cascade::kGroupThreads];
  } lds;
  const int t = threadIdx.x;
  const int64_t n_slices = (v.n_dist + v.n_arg) * v.S;
  if ((int64_t)blockIdx.x >= n_slices) {
    const cascade::RowGeom geo = cascade::row_geom(V);
    const int sub = t / cascade::kGroupThreads, st = t % cascade::kGroupThreads;
    const int64_t task = ((int64_t)blockIdx.x - n_slices) * (kThreads / cascade::kGroupThreads) + sub;
    const int64_t qrow = geo.groups > 0 ? task / geo.groups : qm_rows;
    const int64_t g = geo.groups > 0 ? task % geo.groups : 0;
    const bool live = qrow < qm_rows;
    const float* x = qm_src + qrow * V;
    if (live) {
      if (V % 4 == 0 && (uintptr_t)qm_src % 16 == 0)
        cascade::group_chunk_sums<true>(x, g, geo.full_chunks, st, lds.cs[sub]);
      else
        cascade::group_chunk_sums<false>(x, g, geo.full_chunks, st, lds.cs[sub]);
    }
    __syncthreads();
    if (live)
      cascade::group_stream_sums(g, geo.full_chunks, st, lds.cs[sub],
                                 qm_out + (qrow * geo.groups + g) * cascade::kStreams);
    return;
  }
  const int64_t r = (int64_t)blockIdx.x / v.S;
  const int s = (int)((int64_t)blockIdx.x % v.S);
  const bool dist = r < v.n_dist;
  if (!dist && v.skip_drawn && rows) {
    // an argmax-only row that is also drawn: empty keys, no logits read
    int hit = 0;
    for (int64_t i = t; i < v.n_dist; i += kThreads) hit |= rows[i] == r - v.n_dist;
    if (__syncthreads_or(hit)) {
      BlockStat* out = v.stats + r * v.NB + (int64_t)s * (E / 16);
      if (t < min(E / 16, v.NB - s * (E / 16))) out[t] = BlockStat{-INFINITY, 0u, 0.0, 0ull};
      return;
    }
  }
  int64_t src_r = dist ? (rows ? rows[r] : r) : r - v.n_dist;
  if (src_r < 0 || src_r >= n_src) src_r = 0;  // the row is written as NaN (launch 2)
  const int64_t c0 = (int64_t)s * v.L;
  const void* src = (const char*)logits + src_r * row_stride * (DT == RLT_F32 ? 4 : 2);
  const bool need_argmax = !dist || (v.fused && v.targets);
  const float temp = dist ? temperature[r] : 1.f;
  BlockStat* out = v.stats + r * v.NB + (int64_t)s * (E / 16);
  const int nb_here = min(E / 16, v.NB - s * (E / 16));
  if (c0 + v.L <= V)
    slice_body<DT, E, kVec, true>(lds.red, src, c0, V, dist, need_argmax, temp, out, nb_here);
  else
    slice_body<DT, E, kVec, false>(lds.red, src, c0, V, dist, need_argmax, temp, out, nb_here);
}

// ---------------------------------------------------------------- launch 2

// The float32 row-sum partials (torch's CPU order, cascade.h) of the values y of this
// slice, one 8192-float group at a time staged through LDS; the same arithmetic as the
// acceptance sampler's mass kernel over the written row.
template <int E>
__device__ __forceinline__ void slice_partials(float (&y)[E], int64_t c0, int V, float* stage,
                                               cascade::ChunkSums* cs, float* __restrict__ pm) {
  constexpr int kGroups = E * kThreads / cascade::kGroupFloats;  // groups per slice
  constexpr int kQPerGroup = cascade::kGroupFloats / (4 * kThreads);
  static_assert(kGroups >= 1 && cascade::kGroupFloats % (4 * kThreads) == 0, "whole groups");
  const int t = threadIdx.x;
  const cascade::RowGeom geo = cascade::row_geom(V);
  const int64_t g0 = c0 / cascade::kGroupFloats;
#pragma unroll
  for (int gl = 0; gl < kGroups; ++gl) {
    if (gl > 0) __syncthreads();  // the previous group's readers are done with stage
#pragma unroll
    for (int q = 0; q < kQPerGroup; ++q) {
      const int qq = gl * kQPerGroup + q;
      *(float4*)(stage + 4 * (kThreads * q + t)) =
          make_float4(y[4 * qq], y[4 * qq + 1], y[4 * qq + 2], y[4 * qq + 3]);
    }
    __syncthreads();
    const int64_t g = g0 + gl;
    const int sub = t / cascade::kGroupThreads, st = t % cascade::kGroupThreads;
    const int64_t fc = geo.full_chunks - g * cascade::kGroupChunks;  // chunks of group g on
    if (sub == 0 && fc > 0) cascade::group_chunk_sums<true>(stage, 0, fc, st, *cs);
    __syncthreads();
    if (sub == 0 && fc > 0)
      cascade::group_stream_sums(0, fc, st, *cs, pm + g * cascade::kStreams);
  }
}

// The categorical draw's tile totals (float64) and flag bits (1 NaN, 2 +inf,
// 4 negative, 8 positive) of this slice's written values.  Quad q of a thread holds
// columns c0 + 4 (kThreads q + t) .. +3, so tile kt of the slice is quads 4kt..4kt+3.
// The draw certifies its crossing against a bound that holds for every float64
// summation order (and otherwise replays torch's sequential cumsum), so these totals
// need not repeat the tile kernel's order: the drawn index is the same.
template <int E, bool kFull>
__device__ __forceinline__ void slice_tiles(const float (&y)[E], int64_t c0, int V,
                                            double* __restrict__ ts,
                                            uint32_t* __restrict__ tf, int64_t tile0,
                                            int tiles) {
  constexpr int kT = E / 16;
  __shared__ double wsum[kT][kWaves];
  __shared__ uint32_t wflag[kT][kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
#pragma unroll
  for (int kt = 0; kt < kT; ++kt) {
    double d = 0.0;
    uint32_t f = 0;
#pragma unroll
    for (int j = 16 * kt; j < 16 * kt + 16; ++j) {
      const float x = y[j];
      if (!kFull && (int64_t)elem_col<E>((uint32_t)(c0 + 4 * t), j) >= V) continue;
      if (isnan(x)) f |= 1u;
      else if (isinf(x) && x > 0.f) f |= 2u;
      if (x < 0.f) f |= 4u;
      if (x > 0.f) f |= 8u;
      d += (double)x;
    }
    for (int off = 32; off >= 1; off >>= 1) d += __shfl_xor(d, off, RLT_WAVE);
    const uint32_t wf = (__ballot(f & 1u) ? 1u : 0u) | (__ballot(f & 2u) ? 2u : 0u) |
                        (__ballot(f & 4u) ? 4u : 0u) | (__ballot(f & 8u) ? 8u : 0u);
    if (lane == 0) {
      wsum[kt][wave] = d;
      wflag[kt][wave] = wf;
    }
  }
  __syncthreads();
  if (t < kT && tile0 + t < tiles) {
    double d = 0.0;
    uint32_t f = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      d += wsum[t][w];
      f |= wflag[t][w];
    }
    ts[tile0 + t] = d;
    tf[tile0 + t] = f;
  }
}

typedef float f32v4 __attribute__((ext_vector_type(4)));

template <int DT, int E, bool kVec, bool kFull>
__device__ __forceinline__ void write_body(const void* __restrict__ src, int64_t c0, int V,
                                           bool nan_row, float lmax, float c, float inv,
                                           float* __restrict__ dst, bool out_vec,
                                           float* __restrict__ pm, double* __restrict__ ts,
                                           uint32_t* __restrict__ tf, int tiles) {
  const uint32_t base = (uint32_t)(c0 + 4 * threadIdx.x);
  float y[E];
  if (nan_row) {
#pragma unroll
    for (int j = 0; j < E; ++j) y[j] = NAN;
  } else {
    float x[E];
    load_slice<DT, E, kVec>(src, c0, V, x);
#pragma unroll
    for (int j = 0; j < E; ++j) y[j] = __builtin_amdgcn_exp2f((x[j] - lmax) * c) * inv;
  }
#pragma unroll
  for (int q = 0; q < E / 4; ++q) {
    const uint32_t col = elem_col<E>(base, 4 * q);
    // streamed stores: no pass of the launch reads the row back (the partials and
    // tile totals come from y), and lines left dirty in the L2 would be written back
    // at the kernel boundary, ahead of the next launch's work
    if (kVec && out_vec) {
      if (kFull || (int64_t)col < V)
        __builtin_nontemporal_store(f32v4{y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]},
                                    (f32v4*)(dst + col));
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (kFull || (int64_t)col + k < V) __builtin_nontemporal_store(y[4 * q + k], dst + col + k);
    }
  }
  if (ts) slice_tiles<E, kFull>(y, c0, V, ts, tf, c0 / (16 * kThreads), tiles);
  if constexpr (E * kThreads % cascade::kGroupFloats == 0) {
    if (pm) {
      __shared__ float stage[cascade::kGroupFloats];
      __shared__ cascade::ChunkSums cs;
      slice_partials<E>(y, c0, V, stage, &cs, pm);
    }
  }
}

// Workgroups [0, n_dist S): slice s of distribution row r, normalized by the row's
// total from its blocks; workgroups past n_dist S finish the argmax-only rows (one
// thread per row).  out_vec: out rows aligned to four floats (vector stores).
template <int DT, int E, bool kVec>
__global__ __launch_bounds__(kThreads) void rlt_probs_write_kernel(
    const void* __restrict__ logits, const int64_t* __restrict__ rows, int64_t n_src,
    int64_t row_stride, int V, const float* __restrict__ temperature, View v,
    float* __restrict__ out, int64_t out_stride, int out_vec) {
  const int t = threadIdx.x, lane = t & 63;
  const int64_t n_slices = v.n_dist * v.S;
  if ((int64_t)blockIdx.x >= n_slices) {
    finish_argmax_row(v, ((int64_t)blockIdx.x - n_slices) * kThreads + t);
    return;
  }
  const int64_t r = (int64_t)blockIdx.x / v.S;
  const int s = (int)((int64_t)blockIdx.x % v.S);
  const int64_t src_r = rows ? rows[r] : r;
  const bool src_ok = src_r >= 0 && src_r < n_src;
  const float temp = temperature[r];
  const float c = 1.44269504088896341f / temp;
  // the row's max, NaN state, argmax and total: lane b holds block b; every wave
  // computes the same values (the lane tree's pairings do not depend on the wave)
  BlockStat b{-INFINITY, 0u, 0.0, 0ull};
  if (lane < v.NB) b = v.stats[r * v.NB + lane];
  float lmax = b.m;
  unsigned long long best = b.best;
  for (int off = 32; off >= 1; off >>= 1) {
    lmax = fmaxf(lmax, __shfl_xor(lmax, off, RLT_WAVE));
    const unsigned long long o = __shfl_xor(best, off, RLT_WAVE);
    best = o > best ? o : best;
  }
  const bool bad = __ballot(b.nan != 0) != 0;
  if (v.fused && v.targets && s == 0 && t == 0) v.targets[r] = argmax_column(best);
  const bool nan_row = bad || !src_ok || !isfinite(lmax) || !(temp > 0.f) || !isfinite(c);
  float inv = 0.f;
  if (!nan_row) {
    double term = lane < v.NB && isfinite(b.m)
                      ? b.z * exp2(((double)b.m - (double)lmax) * (double)c) : 0.0;
    for (int off = 32; off >= 1; off >>= 1) term += __shfl_xor(term, off, RLT_WAVE);
    inv = (float)(1.0 / term);
  }
  const int64_t c0 = (int64_t)s * v.L;
  const void* src =
      (const char*)logits + (src_ok ? src_r : 0) * row_stride * (DT == RLT_F32 ? 4 : 2);
  float* dst = out + r * out_stride;
  float* pm = v.pm_out ? v.pm_out + r * cascade::row_geom(V).groups * cascade::kStreams : nullptr;
  double* ts = v.tile_sum ? v.tile_sum + r * v.tiles : nullptr;
  uint32_t* tf = v.tile_sum ? v.tile_flags + r * v.tiles : nullptr;
  if (c0 + v.L <= V)
    write_body<DT, E, kVec, true>(src, c0, V, nan_row, lmax, c, inv, dst, out_vec != 0, pm, ts,
                                  tf, v.tiles);
  else
    write_body<DT, E, kVec, false>(src, c0, V, nan_row, lmax, c, inv, dst, out_vec != 0, pm, ts,
                                   tf, v.tiles);
}

}  // namespace split
