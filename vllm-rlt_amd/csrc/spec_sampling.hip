// Acceptance / rejection sampler for speculative verification on MI355X (gfx950).
//
// Replaces the eager torch chain of vllm_rlt/worker/speculative_sampling.py:59-181
// (``categorical`` and ``speculative_accept``) with three launches that are
// bit-exact against the torch-CPU arithmetic the reference defines:
//
//  1. rlt_mass_groups_kernel -- every p and q row of the batch, split into
//     8192-float groups across the whole GPU: each group's per-stream partial of
//     torch's fp32 cascade row sum (the HBM-bound pass: p and q read once).
//  2. rlt_accept_tiles_kernel -- (request, 4096-token tile) workgroups: the exact
//     fp32 row masses from the partials, the accept chain (px >= qx or
//     u*qx < px), stop point s and validity (recomputed identically by every tile
//     of a request), then the tile's float64 total of the final distribution
//     (p[s]/mass at the end of the drafts, else clamp_min(p[s]/pm - q[s]/qm, 0))
//     with NaN / +inf / negative / positive flags.
//  3. rlt_accept_draw_kernel -- one workgroup per request: the inverse-CDF draw.
//     It locates the tile and token where the float64 CDF crosses t = u * mass,
//     certifies the crossing against a bound on the difference between any
//     float64 summation order and torch's sequential cumsum, and otherwise replays
//     the sequential cumsum on one lane (exact by construction); then tokens /
//     accepted / final / error.
//
// ``categorical`` runs the same tile totals and draw on raw weights: a (row, tile) grid
// for the totals, then one draw workgroup per row.
//
// torch's fp32 row-sum order (what ``p.sum(-1, dtype=float32)`` computes on CPU):
// 32 streams, stream s = 8k + l owns elements 32*i + s (8-lane vectors, 4 in
// flight); each stream is a 4-level cascade: 16 elements per chunk (level 0),
// chunks summed sequentially into level 1, flushed to level 2 every 16 chunks
// (one "group" = 16 chunks = 8192 floats of the row), level 2 flushed to level 3
// every 16 groups; leftovers per the final combine in rlt_row_mass_finish().

#include "cascade.h"
#include "common.h"
#include "rlt_mi355x.h"

#include <math.h>

#include <mutex>

namespace {

using cascade::kChunkSteps;
using cascade::kGroupChunks;
using cascade::kGroupFloats;
using cascade::kStreams;
using cascade::row_geom;
using cascade::RowGeom;
constexpr int kDrawThreads = 512;
constexpr int kDrawWaves = kDrawThreads / 64;
constexpr int kElems = 8;                           // weights per thread per tile
constexpr int kTile = kDrawThreads * kElems;        // 4096 tokens
constexpr int kMaxTiles = 512;                      // V <= 2M on the fast path
constexpr int kMaxW1 = 32;


// ------------------------------------------------------------------ kernel 1

// grid (groups, rows), 128 threads: thread t sums chunk t/8 of the group for the
// four streams 4*(t%8)..+3 (16 sequential fp32 adds each), then 32 threads add the
// chunk sums of their stream in order (level-1 accumulator).
template <bool kVec4>
__global__ __launch_bounds__(128) void rlt_mass_groups_kernel(const float* __restrict__ p,
                                                              const float* __restrict__ q,
                                                              int64_t p_rows, int64_t V,
                                                              int64_t groups, int64_t full_chunks,
                                                              float* __restrict__ out) {
  __shared__ cascade::ChunkSums chunk_sum;
  const int64_t row = blockIdx.y;
  const int64_t g = blockIdx.x;
  const float* x = row < p_rows ? p + row * V : q + (row - p_rows) * V;
  const int t = threadIdx.x;
  cascade::group_chunk_sums<kVec4>(x, g, full_chunks, t, chunk_sum);
  __syncthreads();
  cascade::group_stream_sums(g, full_chunks, t, chunk_sum, out + (row * groups + g) * kStreams);
}

// Exact torch-CPU fp32 row sum of x[0..V) from the group partials (nullptr when
// the row has no complete chunk).  Called by one full wave; valid in every lane.
__device__ float rlt_row_mass_finish(const float* __restrict__ x, int64_t V,
                                     const float* __restrict__ partials) {
  const int lane = threadIdx.x & 63;
  if (V < 8) {
    // scalar ILP-4 form (no vector step): stream k owns x[4i + k].
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
    const int64_t si = V / 4;
    for (int64_t i = 0; i < si; ++i)
      for (int k = 0; k < 4; ++k) ps[k] += x[4 * i + k];
    for (int64_t i = si * 4; i < V; ++i) ps[0] += x[i];
    return ((ps[0] + ps[1]) + ps[2]) + ps[3];
  }
  const RowGeom geo = row_geom(V);
  float st = 0.f;  // this lane's stream total (lanes < 32)
  if (lane < kStreams) {
    const int s = lane;
    float acc2 = 0.f, acc3 = 0.f, acc1 = 0.f;
    const int64_t complete = geo.full_chunks / kGroupChunks;
    int64_t g = 0;
    for (; g + 8 <= complete; g += 8) {  // 8 independent loads in flight
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = partials[(g + u) * kStreams + s];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        acc2 += v[u];
        if ((g + u + 1) % 16 == 0) {
          acc3 += acc2;
          acc2 = 0.f;
        }
      }
    }
    for (; g < complete; ++g) {
      acc2 += partials[g * kStreams + s];
      if ((g + 1) % 16 == 0) {
        acc3 += acc2;
        acc2 = 0.f;
      }
    }
    if (geo.full_chunks % kGroupChunks) acc1 = partials[complete * kStreams + s];
    float acc0 = 0.f;
    for (int64_t i = geo.full_chunks * kChunkSteps; i < geo.si; ++i) acc0 += x[32 * i + s];
    st = ((acc0 + acc1) + acc2) + acc3;
    // Leftover whole vectors go lane-wise into the first ILP accumulator.
    if (s < 8)
      for (int64_t v = geo.si * 4; v < geo.vs; ++v) st += x[v * 8 + s];
  }
  // lanes[l] = ((st[l] + st[8+l]) + st[16+l]) + st[24+l]
  const float s8 = __shfl(st, (lane + 8) & 63, RLT_WAVE);
  const float s16 = __shfl(st, (lane + 16) & 63, RLT_WAVE);
  const float s24 = __shfl(st, (lane + 24) & 63, RLT_WAVE);
  const float lanes = ((st + s8) + s16) + s24;
  float f = 0.f;
  for (int64_t e = geo.vs * 8; e < V; ++e) f += x[e];
  for (int l = 0; l < 8; ++l) f += __shfl(lanes, l, RLT_WAVE);
  return f;
}

// Same as rlt_row_mass_finish for one 32-lane half of a wave (lanes 32h..32h+31
// serve row x): two rows per wave at once.  Valid in every lane of the half.
__device__ float rlt_row_mass_half(const float* __restrict__ x, int64_t V,
                                   const float* __restrict__ partials) {
  const int lane = threadIdx.x & 63;
  const int s = lane & 31;
  const int base = lane & 32;
  if (V < 8) {
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
    const int64_t si = V / 4;
    for (int64_t i = 0; i < si; ++i)
      for (int k = 0; k < 4; ++k) ps[k] += x[4 * i + k];
    for (int64_t i = si * 4; i < V; ++i) ps[0] += x[i];
    return ((ps[0] + ps[1]) + ps[2]) + ps[3];
  }
  const RowGeom geo = row_geom(V);
  float acc2 = 0.f, acc3 = 0.f, acc1 = 0.f;
  const int64_t complete = geo.full_chunks / kGroupChunks;
  for (int64_t g = 0; g < complete; g += 8) {  // up to 8 independent loads in flight
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = g + u < complete ? partials[(g + u) * kStreams + s] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (g + u >= complete) break;
      acc2 += v[u];
      if ((g + u + 1) % 16 == 0) {
        acc3 += acc2;
        acc2 = 0.f;
      }
    }
  }
  if (geo.full_chunks % kGroupChunks) acc1 = partials[complete * kStreams + s];
  float acc0 = 0.f;
  for (int64_t i = geo.full_chunks * kChunkSteps; i < geo.si; ++i) acc0 += x[32 * i + s];
  float st = ((acc0 + acc1) + acc2) + acc3;
  if (s < 8)
    for (int64_t v = geo.si * 4; v < geo.vs; ++v) st += x[v * 8 + s];
  const float s8 = __shfl(st, base + ((s + 8) & 31), RLT_WAVE);
  const float s16 = __shfl(st, base + ((s + 16) & 31), RLT_WAVE);
  const float s24 = __shfl(st, base + ((s + 24) & 31), RLT_WAVE);
  const float lanes = ((st + s8) + s16) + s24;
  float f = 0.f;
  for (int64_t e = geo.vs * 8; e < V; ++e) f += x[e];
  for (int l = 0; l < 8; ++l) f += __shfl(lanes, base + l, RLT_WAVE);
  return f;
}

__device__ __forceinline__ bool finite_pos(float m) { return isfinite(m) && m > 0.f; }

// ------------------------------------------------------------------ wave scans

// A float64 moved across lanes by a DPP pattern (both 32-bit halves).
template <int kCtrl>
__device__ __forceinline__ double dpp_move(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, kCtrl, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), kCtrl, 0xf, 0xf, false);
  return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

// Inclusive prefix sum over the 64 lanes in a fixed order: Hillis-Steele steps
// within each 16-lane row (row_shr 1, 2, 4, 8), then row 0 -> 1 and 2 -> 3
// (row_bcast 15), then lanes 0..31 -> 32..63 (row_bcast 31).
__device__ __forceinline__ double wave_inclusive_sum(double x) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  double y;
  y = dpp_move<0x111>(x);
  if (r >= 1) x += y;
  y = dpp_move<0x112>(x);
  if (r >= 2) x += y;
  y = dpp_move<0x114>(x);
  if (r >= 4) x += y;
  y = dpp_move<0x118>(x);
  if (r >= 8) x += y;
  y = dpp_move<0x142>(x);
  if (lane & 16) x += y;
  y = dpp_move<0x143>(x);
  if (lane >= 32) x += y;
  return x;
}

// The value of lane 63 in every lane.
__device__ __forceinline__ double lane63(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)b, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// OR of the flag bits (1 NaN, 2 +inf, 4 negative, 8 positive) over the wave.
__device__ __forceinline__ uint32_t wave_or_flags(uint32_t fl) {
  uint32_t r = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b)
    if (__builtin_amdgcn_ballot_w64((fl >> b) & 1u)) r |= 1u << b;
  return r;
}

// ------------------------------------------------------------------ weights

struct WeightRow {
  const float* a;  // p[s] row (or the raw weight row)
  const float* b;  // q[s] row, residual mode only
  float am, bm;
  bool residual;
  bool raw;
};

// The fp32 weight of one token exactly as torch computes it:
//   at_end: p/pm; else (p/pm - q/qm).clamp_min(0) (NaN propagates).
__device__ __forceinline__ float weight_of(float a, float b, const WeightRow& w) {
  if (w.raw) return a;
  const float pa = __fdiv_rn(a, w.am);
  if (!w.residual) return pa;
  const float r = pa - __fdiv_rn(b, w.bm);
  return r < 0.f ? 0.f : r;
}

// This thread's kElems raw floats [base, base + kElems) of a row (zero past V).
__device__ __forceinline__ void load_raw(const float* row, int64_t V, int64_t base, bool vec_ok,
                                         float out[kElems]) {
  if (vec_ok && base + kElems <= V) {
    const float4 a0 = *(const float4*)(row + base);
    const float4 a1 = *(const float4*)(row + base + 4);
    out[0] = a0.x; out[1] = a0.y; out[2] = a0.z; out[3] = a0.w;
    out[4] = a1.x; out[5] = a1.y; out[6] = a1.z; out[7] = a1.w;
  } else {
#pragma unroll
    for (int e = 0; e < kElems; ++e) out[e] = base + e < V ? row[base + e] : 0.f;
  }
}

// This thread's kElems weights of tile `tile` (zero past V).
__device__ __forceinline__ void load_weights(const WeightRow& w, int64_t V, int64_t tile, int t,
                                             bool vec_ok, float out[kElems]) {
  const int64_t base = tile * kTile + (int64_t)t * kElems;
  float av[kElems], bv[kElems];
  load_raw(w.a, V, base, vec_ok, av);
  if (w.residual) load_raw(w.b, V, base, vec_ok, bv);
#pragma unroll
  for (int e = 0; e < kElems; ++e) out[e] = base + e < V ? weight_of(av[e], w.residual ? bv[e] : 0.f, w) : 0.f;
}

// Sequential float64 replay of torch's cumsum + searchsorted(right=True) on one
// lane: exact by construction.  reference: speculative_sampling.py:74-84.
__device__ int64_t slow_draw(const WeightRow& w, int64_t V, float u, bool* valid_out) {
  double mass = 0.0;
  bool neg = false;
  for (int64_t k = 0; k < V; ++k) {
    const float x = weight_of(w.a[k], w.residual ? w.b[k] : 0.f, w);
    neg |= x < 0.f;
    mass += (double)x;
  }
  const bool valid = isfinite(mass) && mass > 0.0;
  *valid_out = valid;
  if (!valid) return 0;
  double t = (double)u * mass;
  const double below = nextafter(mass, 0.0);
  t = (isnan(t) || isnan(below)) ? (double)NAN : (below < t ? below : t);
  int64_t lo = 0;
  if (!neg) {
    // monotone cdf: upper_bound == index of the first entry > t
    double c = 0.0;
    lo = V;
    for (int64_t k = 0; k < V; ++k) {
      c += (double)weight_of(w.a[k], w.residual ? w.b[k] : 0.f, w);
      if (c > t) {
        lo = k;
        break;
      }
    }
  } else {
    // non-monotone cdf: replay torch's binary search, recomputing each probe.
    int64_t hi = V;
    while (lo < hi) {
      const int64_t mid = lo + ((hi - lo) >> 1);
      double c = 0.0;
      for (int64_t k = 0; k <= mid; ++k)
        c += (double)weight_of(w.a[k], w.residual ? w.b[k] : 0.f, w);
      if (!(c > t)) lo = mid + 1;
      else hi = mid;
    }
  }
  return lo > V - 1 ? V - 1 : lo;
}

// ------------------------------------------------------------------ draw

struct DrawScratch {
  double tile_total[kMaxTiles];
  uint32_t tile_flags[kMaxTiles];  // per-tile flag bits (accept draw only)
  double wave_sum[kDrawWaves];
  int64_t cand[kDrawWaves];  // per wave: first token whose cumulative weight exceeds t, or -1
  double cand_before[kDrawWaves], cand_at[kDrawWaves];
  int decision;  // 0 fast, 1 exact replay, 2 invalid row
  int64_t tile;
  double tile_start, t, margin;
};

// Inverse-CDF draw given the float64 tile totals (in ds.tile_total) and the row's
// flags.  Called by all kDrawThreads threads; the result is valid in thread 0.
// Locates the tile and token where the float64 CDF crosses t = u * mass and
// certifies the crossing against a bound on the difference between any float64
// summation order and torch's sequential cumsum; otherwise (or for out-of-contract
// inputs) replays torch's sequential cumsum + right bisect on one lane.
__device__ void draw_from_tiles(const WeightRow& w, int64_t V, float u, int64_t tiles, uint32_t flags,
                                bool flags_in_lds, bool vec_ok, DrawScratch& ds,
                                int32_t* slow_count, int64_t* index_out, bool* valid_out) {
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  if (wave == 0) {
    if (flags_in_lds) {
      uint32_t f = 0;
      for (int64_t k = lane; k < tiles && k < kMaxTiles; k += 64) f |= ds.tile_flags[k];
      flags = wave_or_flags(f);
    }
    const bool any_nan = flags & 1u, any_inf = flags & 2u, any_neg = flags & 4u, any_pos = flags & 8u;
    // wave 0: inclusive scan of the tile totals (64 tiles per pass, fixed order)
    // gives the mass and the first tile whose cumulative total exceeds t = u*mass
    int decision = 0;
    if (tiles > kMaxTiles || any_neg || !(u >= 0.f && u < 1.f)) decision = 1;
    else if (any_nan || any_inf || !any_pos) decision = 2;
    double m = 0.0;
    if (decision == 0) {
      for (int64_t k0 = 0; k0 < tiles; k0 += 64) {
        double v = k0 + lane < tiles ? ds.tile_total[k0 + lane] : 0.0;
        v = wave_inclusive_sum(v);
        if (k0 + lane < tiles) ds.tile_total[k0 + lane] = m + v;  // cumulative total
        m += lane63(v);
      }
    }
    const double tt = (double)u * m;
    int64_t tile = -1;
    if (decision == 0) {
      for (int64_t k0 = 0; k0 < tiles && tile < 0; k0 += 64) {
        const bool over = k0 + lane < tiles && ds.tile_total[k0 + lane] > tt;
        const uint64_t mask = __builtin_amdgcn_ballot_w64(over);
        if (mask) tile = k0 + __builtin_ctzll(mask);
      }
      if (tile < 0) decision = 1;
    }
    if (lane == 0) {
      // |any float64 summation order - torch's sequential cumsum| <= (#adds) * 2^-53
      // * mass per side; doubled for t's own dependence on the mass, plus the
      // rounding of u * mass.
      ds.margin = (4.0 * (double)V + 64.0) * 0x1p-52 * m;
      ds.t = tt;
      ds.tile = tile;
      ds.tile_start = tile > 0 ? ds.tile_total[tile - 1] : 0.0;
      ds.decision = decision;
    }
  }
  __syncthreads();
  int decision = ds.decision;
  int64_t index = 0;
  bool valid = decision != 2;
  if (decision == 0) {
    float wv[kElems];
    load_weights(w, V, ds.tile, t, vec_ok, wv);
    double local = 0.0;
#pragma unroll
    for (int e = 0; e < kElems; ++e) local += (double)wv[e];
    // exclusive scan of thread partials in index order: wave scan, then wave offsets
    const double incl = wave_inclusive_sum(local);
    if (lane == 63) ds.wave_sum[wave] = incl;
    __syncthreads();
    double wave_off = 0.0;
    for (int wv2 = 0; wv2 < wave; ++wv2) wave_off += ds.wave_sum[wv2];
    const double tt = ds.t;
    double run = ds.tile_start + (wave_off + (incl - local));
    int e_hit = -1;
    double before = 0.0, at = 0.0;
#pragma unroll
    for (int e = 0; e < kElems; ++e) {
      const double next = run + (double)wv[e];
      if (e_hit < 0 && next > tt) {
        e_hit = e;
        before = run;
        at = next;
      }
      run = next;
    }
    // each wave reports its first hit; the first reporting wave holds the crossing
    const uint64_t hits = __builtin_amdgcn_ballot_w64(e_hit >= 0);
    if (hits == 0) {
      if (lane == 0) ds.cand[wave] = -1;
    } else if (lane == __builtin_ctzll(hits)) {
      ds.cand[wave] = ds.tile * kTile + (int64_t)t * kElems + e_hit;
      ds.cand_before[wave] = before;
      ds.cand_at[wave] = at;
    }
    __syncthreads();
    if (t != 0) return;
    decision = 1;
    for (int wv2 = 0; wv2 < kDrawWaves; ++wv2) {
      if (ds.cand[wv2] < 0) continue;
      index = ds.cand[wv2];
      const bool ok = ds.cand_before[wv2] <= tt - ds.margin && ds.cand_at[wv2] > tt + ds.margin;
      decision = ok ? 0 : 1;
      break;
    }
  }
  if (t != 0) return;
  if (decision == 1) {
    bool v;
    index = slow_draw(w, V, u, &v);
    valid = v;
    atomicAdd(slow_count, 1);
  }
  if (!valid) index = 0;
  if (index > V - 1) index = V - 1;
  if (index < 0) index = 0;
  *index_out = index;
  *valid_out = valid;
}

// This thread's tile weights -> (wave-reduced float64 sum in every lane, flag bits).
__device__ __forceinline__ double tile_partial(const float wv[kElems], uint32_t& flags) {
  double local = 0.0;
#pragma unroll
  for (int e = 0; e < kElems; ++e) {
    const float x = wv[e];
    if (isnan(x)) flags |= 1u;
    else if (isinf(x) && x > 0.f) flags |= 2u;
    if (x < 0.f) flags |= 4u;
    if (x > 0.f) flags |= 8u;
    local += (double)x;
  }
  return lane63(wave_inclusive_sum(local));
}

// ------------------------------------------------------------------ categorical

struct CatShared {
  DrawScratch ds;
  double wave_tile[kMaxTiles][kDrawWaves];
  uint32_t flags;
};

// grid (m), kDrawThreads threads: one row of raw weights (row i at weights + i *
// w_stride) per workgroup.  The index goes to out_index[i], or with a scatter list
// to out_index[scatter[i]] when that lies in [0, n_out); out_valid may be null.
__global__ __launch_bounds__(kDrawThreads) void rlt_categorical_kernel(
    const float* __restrict__ weights, int64_t V, int64_t w_stride, const float* __restrict__ u,
    int64_t* __restrict__ out_index, uint8_t* __restrict__ out_valid,
    const int64_t* __restrict__ scatter, int64_t n_out, int32_t* __restrict__ slow_count) {
  __shared__ CatShared sh;
  const int64_t i = blockIdx.x;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  if (t == 0) sh.flags = 0;
  WeightRow w;
  w.a = weights + i * w_stride;
  w.b = nullptr;
  w.am = w.bm = 1.f;
  w.residual = false;
  w.raw = true;
  const bool vec_ok = (V % 4 == 0) && ((uintptr_t)w.a % 16 == 0);
  const int64_t tiles = (V + kTile - 1) / kTile;
  __syncthreads();
  if (tiles <= kMaxTiles) {
    uint32_t fl = 0;
    for (int64_t k0 = 0; k0 < tiles; k0 += 4) {
      float wv[4][kElems];
#pragma unroll
      for (int uu = 0; uu < 4; ++uu)
        if (k0 + uu < tiles) load_weights(w, V, k0 + uu, t, vec_ok, wv[uu]);
#pragma unroll
      for (int uu = 0; uu < 4; ++uu) {
        if (k0 + uu >= tiles) break;
        const double part = tile_partial(wv[uu], fl);
        if (lane == 0) sh.wave_tile[k0 + uu][wave] = part;
      }
    }
    fl = wave_or_flags(fl);
    if (lane == 0 && fl) atomicOr(&sh.flags, fl);
  }
  __syncthreads();
  for (int64_t k = t; k < tiles && k < kMaxTiles; k += kDrawThreads) {
    double tk = 0.0;
    for (int wv = 0; wv < kDrawWaves; ++wv) tk += sh.wave_tile[k][wv];
    sh.ds.tile_total[k] = tk;
  }
  __syncthreads();
  const uint32_t f = sh.flags;
  int64_t index;
  bool valid;
  draw_from_tiles(w, V, u[i], tiles, f, false, vec_ok, sh.ds, slow_count, &index, &valid);
  if (t == 0) {
    if (!scatter) {
      out_index[i] = index;
    } else {
      const int64_t d = scatter[i];
      if (d >= 0 && d < n_out) out_index[d] = index;
    }
    if (out_valid) out_valid[i] = valid;
  }
}

// Two-launch categorical (V <= kMaxTiles tiles): grid (m, tiles) tile totals, then
// grid (m) draws.  The tile totals are the single-workgroup kernel's bits (wave
// partials summed in wave order), so both forms draw the same index.
__global__ __launch_bounds__(kDrawThreads) void rlt_categorical_tiles_kernel(
    const float* __restrict__ weights, int64_t V, int64_t w_stride, double* __restrict__ tile_sum,
    uint32_t* __restrict__ tile_flags) {
  __shared__ double wave_part[kDrawWaves];
  __shared__ uint32_t wave_flags[kDrawWaves];
  const int64_t i = blockIdx.x;
  const int64_t k = blockIdx.y;
  const int64_t tiles = gridDim.y;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  WeightRow w;
  w.a = weights + i * w_stride;
  w.b = nullptr;
  w.am = w.bm = 1.f;
  w.residual = false;
  w.raw = true;
  const bool vec_ok = (V % 4 == 0) && ((uintptr_t)w.a % 16 == 0);
  float wv[kElems];
  load_weights(w, V, k, t, vec_ok, wv);
  uint32_t fl = 0;
  const double part = tile_partial(wv, fl);
  fl = wave_or_flags(fl);
  if (lane == 0) {
    wave_part[wave] = part;
    wave_flags[wave] = fl;
  }
  __syncthreads();
  if (t == 0) {
    double tk = 0.0;
    uint32_t f = 0;
    for (int v = 0; v < kDrawWaves; ++v) {
      tk += wave_part[v];
      f |= wave_flags[v];
    }
    tile_sum[i * tiles + k] = tk;
    tile_flags[i * tiles + k] = f;
  }
}

__global__ __launch_bounds__(kDrawThreads) void rlt_categorical_draw_kernel(
    const float* __restrict__ weights, int64_t V, int64_t w_stride, int64_t tiles,
    const float* __restrict__ u, const double* __restrict__ tile_sum,
    const uint32_t* __restrict__ tile_flags, int64_t* __restrict__ out_index,
    uint8_t* __restrict__ out_valid, const int64_t* __restrict__ scatter, int64_t n_out,
    int32_t* __restrict__ slow_count) {
  __shared__ DrawScratch ds;
  const int64_t i = blockIdx.x;
  const int t = threadIdx.x;
  for (int64_t k = t; k < tiles; k += kDrawThreads) {
    ds.tile_total[k] = tile_sum[i * tiles + k];
    ds.tile_flags[k] = tile_flags[i * tiles + k];
  }
  WeightRow w;
  w.a = weights + i * w_stride;
  w.b = nullptr;
  w.am = w.bm = 1.f;
  w.residual = false;
  w.raw = true;
  const bool vec_ok = (V % 4 == 0) && ((uintptr_t)w.a % 16 == 0);
  __syncthreads();
  int64_t index;
  bool valid;
  draw_from_tiles(w, V, u[i], tiles, 0u, true, vec_ok, ds, slow_count, &index, &valid);
  if (t != 0) return;
  if (!scatter) {
    out_index[i] = index;
  } else {
    const int64_t d = scatter[i];
    if (d >= 0 && d < n_out) out_index[d] = index;
  }
  if (out_valid) out_valid[i] = valid;
}

// ------------------------------------------------------------------ accept

// Stop state of one request, written by its tile-0 workgroup for the draw kernel.
struct StopState {
  int32_t s;        // leading valid accepts
  int32_t at_end;   // s == d: the final draw is the bonus from p[s]
  int32_t stop_ok;  // the stop point is numerically valid
  int32_t err0;     // drafts outside [0, W1]
  float pm, qm;     // masses of p[s] and q[s] (qm only for a residual)
  int64_t tok[kMaxW1];
};

struct AcceptShared {
  float pm[kMaxW1 + 1], qm[kMaxW1];
  float px_raw[kMaxW1], qx_raw[kMaxW1], ua[kMaxW1];
  int64_t tok[kMaxW1];
  int64_t drafts;
  double wave_part[kDrawWaves];
  uint32_t wave_flags[kDrawWaves];
  int s, at_end, stop_ok, err0;
};

__device__ __forceinline__ WeightRow stop_weights(const float* p, const float* q, int64_t i, int W1,
                                                  int64_t V, int s, bool at_end, float pm, float qm) {
  WeightRow w;
  w.a = p + (i * (W1 + 1) + s) * V;
  w.am = pm;
  w.residual = !at_end;
  w.b = w.residual ? q + (i * W1 + s) * V : nullptr;
  w.bm = w.residual ? qm : 1.f;
  w.raw = false;
  return w;
}

// grid (n, tiles), kDrawThreads threads.  Each workgroup recomputes its request's
// stop state from the mass partials (cheap and identical in every workgroup) and
// totals its 4096-token tile of the final weights; tile 0 also publishes the stop
// reference: speculative_sampling.py:136-172.
__global__ __launch_bounds__(kDrawThreads) void rlt_accept_tiles_kernel(
    const float* __restrict__ p, const float* __restrict__ q, int W1, int64_t V, int64_t n,
    const float* __restrict__ partials, int64_t groups, const int64_t* __restrict__ draft_tokens,
    const int64_t* __restrict__ drafts, const float* __restrict__ u_accept,
    double* __restrict__ tile_sum, uint32_t* __restrict__ tile_flags,
    StopState* __restrict__ stop, int64_t tiles, int tiles_per_group) {
  __shared__ AcceptShared sh;
  __shared__ double wave_part[2][kDrawWaves];
  __shared__ uint32_t wave_flags[2][kDrawWaves];
  const int64_t i = blockIdx.x;
  const int64_t k0 = (int64_t)blockIdx.y * tiles_per_group;
  const int64_t k1 = min(k0 + tiles_per_group, tiles);
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  // draft tokens, uniforms and the gathers p[x], q[x]: issued first, one lane each
  if (t < W1) {
    const int64_t tok = draft_tokens[i * W1 + t];
    const int64_t x = tok < 0 ? 0 : (tok > V - 1 ? V - 1 : tok);
    sh.tok[t] = tok;
    sh.ua[t] = u_accept[i * W1 + t];
    sh.px_raw[t] = p[(i * (W1 + 1) + t) * V + x];
    sh.qx_raw[t] = q[(i * W1 + t) * V + x];
  }
  if (t == kDrawThreads - 1) sh.drafts = drafts[i];
  // ---- exact masses: rows 0..W1 of p, then 0..W1-1 of q, one half-wave per row
  const int rows = 2 * W1 + 1;
  for (int r = 2 * wave + (lane >> 5); r < rows; r += 2 * kDrawWaves) {
    const bool is_p = r <= W1;
    const int j = is_p ? r : r - W1 - 1;
    const int64_t row = is_p ? i * (W1 + 1) + j : i * W1 + j;
    const float* x = is_p ? p + row * V : q + row * V;
    const int64_t prow = is_p ? row : n * (W1 + 1) + row;
    const float m = rlt_row_mass_half(x, V, partials ? partials + prow * groups * kStreams : nullptr);
    if ((lane & 31) == 0) {
      if (is_p) sh.pm[j] = m;
      else sh.qm[j] = m;
    }
  }
  __syncthreads();
  // ---- accept chain: lane j decides draft j; s = leading accepts (ballot)
  if (wave == 0) {
    const int64_t dr = sh.drafts;
    const int64_t d = dr < 0 ? 0 : (dr > W1 ? W1 : dr);
    bool accept = false, invalid = false;
    if (lane < W1) {
      const int j = lane;
      const int64_t tok = sh.tok[j];
      const bool in_range = tok >= 0 && tok < V;
      const float pmj = sh.pm[j], qmj = sh.qm[j];
      const float px = __fdiv_rn(sh.px_raw[j], pmj);
      const float qx = __fdiv_rn(sh.qx_raw[j], qmj);
      invalid = !(finite_pos(pmj) && finite_pos(qmj) && in_range && isfinite(px) && isfinite(qx) &&
                  qx > 0.f);
      accept = !invalid && ((px >= qx) || (sh.ua[j] * qx < px)) && (j < d);
    }
    const uint64_t am = __builtin_amdgcn_ballot_w64(accept);
    const uint64_t im = __builtin_amdgcn_ballot_w64(invalid);
    const int s = __builtin_ctzll(~am);  // <= W1
    if (lane == 0) {
      const bool at_end = s == d;
      sh.s = s;
      sh.at_end = at_end;
      // invalid_at_s is meaningful only when s < d (the first rejected draft)
      sh.stop_ok = at_end ? finite_pos(sh.pm[s]) : !((im >> s) & 1u);
      sh.err0 = dr != d;
    }
  }
  __syncthreads();
  const int s = sh.s;
  const bool at_end = sh.at_end;
  const WeightRow w = stop_weights(p, q, i, W1, V, s, at_end, sh.pm[s], at_end ? 1.f : sh.qm[s]);
  const bool vec_ok =
      (V % 4 == 0) && ((((uintptr_t)w.a) | ((uintptr_t)(w.b ? w.b : w.a))) % 16 == 0);
  // ---- this workgroup's tiles of the final weights (the stop state above is paid
  // once for all of them); the next tile's loads are in flight while one is reduced,
  // and the wave partials alternate between two buffers (one barrier per tile)
  float cur[kElems];
  load_weights(w, V, k0, t, vec_ok, cur);
  for (int64_t k = k0; k < k1; ++k) {
    float nxt[kElems];
    if (k + 1 < k1) load_weights(w, V, k + 1, t, vec_ok, nxt);
    uint32_t fl = 0;
    const double part = tile_partial(cur, fl);
    fl = wave_or_flags(fl);
    const int b = (int)((k - k0) & 1);
    if (lane == 0) {
      wave_part[b][wave] = part;
      wave_flags[b][wave] = fl;
    }
    __syncthreads();
    if (t == 0) {
      double tk = 0.0;
      uint32_t f = 0;
      for (int wv = 0; wv < kDrawWaves; ++wv) {
        tk += wave_part[b][wv];
        f |= wave_flags[b][wv];
      }
      tile_sum[i * tiles + k] = tk;
      tile_flags[i * tiles + k] = f;
    }
#pragma unroll
    for (int e = 0; e < kElems; ++e) cur[e] = nxt[e];
  }
  if (k0 == 0) {
    StopState& st = stop[i];
    if (t < W1) st.tok[t] = sh.tok[t];
    if (t == 0) {
      st.s = s;
      st.at_end = at_end;
      st.stop_ok = sh.stop_ok;
      st.err0 = sh.err0;
      st.pm = sh.pm[s];
      st.qm = at_end ? 1.f : sh.qm[s];
    }
  }
}

// grid (n), kDrawThreads threads: the inverse-CDF draw and the outputs of request i.
// reference: speculative_sampling.py:174-181.
__global__ __launch_bounds__(kDrawThreads) void rlt_accept_draw_kernel(
    const float* __restrict__ p, const float* __restrict__ q, int W1, int64_t V, int64_t tiles,
    const float* __restrict__ u_final, const double* __restrict__ tile_sum,
    const uint32_t* __restrict__ tile_flags, const StopState* __restrict__ stop,
    int64_t* __restrict__ final_token, int64_t* __restrict__ tokens,
    int64_t* __restrict__ accepted, uint8_t* __restrict__ error, int32_t* __restrict__ slow_count) {
  __shared__ DrawScratch ds;
  const int64_t i = blockIdx.x;
  const int t = threadIdx.x;
  const StopState& st = stop[i];
  for (int64_t k = t; k < tiles && k < kMaxTiles; k += kDrawThreads) {
    ds.tile_total[k] = tile_sum[i * tiles + k];
    ds.tile_flags[k] = tile_flags[i * tiles + k];
  }
  const WeightRow w = stop_weights(p, q, i, W1, V, st.s, st.at_end, st.pm, st.qm);
  const bool vec_ok =
      (V % 4 == 0) && ((((uintptr_t)w.a) | ((uintptr_t)(w.b ? w.b : w.a))) % 16 == 0);
  __syncthreads();
  int64_t index;
  bool valid;
  draw_from_tiles(w, V, u_final[i], tiles, 0u, true, vec_ok, ds, slow_count, &index, &valid);
  if (t != 0) return;
  const bool err = st.err0 || !(st.stop_ok && valid);
  const int64_t fin = err ? 0 : index;
  final_token[i] = fin;
  error[i] = err;
  accepted[i] = st.s;
  for (int j = 0; j <= W1; ++j) {
    int64_t v = 0;
    if (j < st.s) {
      const int64_t tok = st.tok[j];
      v = tok < 0 ? 0 : (tok > V - 1 ? V - 1 : tok);
    } else if (j == st.s) {
      v = fin;
    }
    tokens[i * (W1 + 1) + j] = v;
  }
}

__global__ __launch_bounds__(64) void rlt_row_mass_kernel(const float* __restrict__ x, int64_t V,
                                                          const float* __restrict__ partials,
                                                          int64_t groups, float* __restrict__ out) {
  const int64_t r = blockIdx.x;
  const float m =
      rlt_row_mass_finish(x + r * V, V, partials ? partials + r * groups * kStreams : nullptr);
  if (threadIdx.x == 0) out[r] = m;
}

// ------------------------------------------------------------------ workspace

struct Layout {
  size_t partials, tile_sum, tile_flags, stop, slow, total;
};

Layout layout_for(int64_t rows, int64_t n, int64_t V) {
  const RowGeom geo = row_geom(V);
  const int64_t tiles = (V + kTile - 1) / kTile;
  Layout l;
  size_t off = 0;
  l.partials = off;
  off = rlt_align_up(off + sizeof(float) * rows * geo.groups * kStreams, 256);
  l.tile_sum = off;
  off = rlt_align_up(off + sizeof(double) * n * tiles, 256);
  l.tile_flags = off;
  off = rlt_align_up(off + sizeof(uint32_t) * n * tiles, 256);
  l.stop = off;
  off = rlt_align_up(off + sizeof(StopState) * n, 256);
  l.slow = off;
  off = rlt_align_up(off + sizeof(int32_t), 256);
  l.total = off;
  return l;
}

void launch_mass_groups(const float* p, const float* q, int64_t p_rows, int64_t rows, int64_t V,
                        float* partials, hipStream_t stream) {
  const RowGeom geo = row_geom(V);
  if (geo.groups == 0 || rows == 0) return;
  const bool vec = (V % 4 == 0) && ((uintptr_t)p % 16 == 0) && (q == nullptr || (uintptr_t)q % 16 == 0);
  dim3 grid((unsigned)geo.groups, (unsigned)rows);
  if (vec)
    rlt_mass_groups_kernel<true><<<grid, 128, 0, stream>>>(p, q, p_rows, V, geo.groups,
                                                           geo.full_chunks, partials);
  else
    rlt_mass_groups_kernel<false><<<grid, 128, 0, stream>>>(p, q, p_rows, V, geo.groups,
                                                            geo.full_chunks, partials);
}

// Categorical draws of m weight rows (w_stride floats apart): tile totals over the
// whole GPU, then one draw workgroup per row; rows of more than kMaxTiles tiles run
// the single-workgroup kernel (its draw replays them exactly).
// tiles_ready: the workspace already holds the tile totals and flags (written with
// the weights; rows of at most kMaxTiles tiles only).
int launch_categorical(const float* weights, int64_t w_stride, const float* u, int64_t m,
                       int64_t vocab, int64_t* index, uint8_t* valid, const int64_t* scatter,
                       int64_t n_out, void* workspace, size_t workspace_bytes,
                       hipStream_t stream, bool tiles_ready = false) {
  const Layout l = layout_for(0, m, vocab);
  if (!workspace || workspace_bytes < l.total) return RLT_ERR_WORKSPACE;
  char* ws = (char*)workspace;
  int32_t* slow = (int32_t*)(ws + l.slow);
  const int64_t tiles = (vocab + kTile - 1) / kTile;
  if (tiles > kMaxTiles) {
    if (tiles_ready) return RLT_ERR_ARGUMENT;
    rlt_categorical_kernel<<<(unsigned)m, kDrawThreads, 0, stream>>>(
        weights, vocab, w_stride, u, index, valid, scatter, n_out, slow);
    return rlt_launch_status();
  }
  double* tile_sum = (double*)(ws + l.tile_sum);
  uint32_t* tile_flags = (uint32_t*)(ws + l.tile_flags);
  if (!tiles_ready)
    rlt_categorical_tiles_kernel<<<dim3((unsigned)m, (unsigned)tiles), kDrawThreads, 0,
                                   stream>>>(weights, vocab, w_stride, tile_sum, tile_flags);
  rlt_categorical_draw_kernel<<<(unsigned)m, kDrawThreads, 0, stream>>>(
      weights, vocab, w_stride, tiles, u, tile_sum, tile_flags, index, valid, scatter, n_out,
      slow);
  return rlt_launch_status();
}

// speculative_accept; with q_partials_ready the workspace already holds the mass
// partials of the q rows (written alongside the target distributions) and only the
// p rows are summed here.
int accept_launch(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                  const float* p, const float* u_accept, const float* u_final, int64_t n,
                  int32_t w1, int64_t vocab, int64_t* tokens, int64_t* accepted,
                  int64_t* final_token, uint8_t* error, void* workspace, size_t workspace_bytes,
                  int partials_ready, hipStream_t stream) {
  if (n < 0 || w1 < 0 || w1 > kMaxW1 || vocab < 1) return RLT_ERR_ARGUMENT;
  if (vocab >= ((int64_t)1 << 25)) return RLT_ERR_UNSUPPORTED;
  if (n == 0) return RLT_OK;
  const int64_t rows = n * (2 * (int64_t)w1 + 1);
  const Layout l = layout_for(rows, n, vocab);
  if (!workspace || workspace_bytes < l.total) return RLT_ERR_WORKSPACE;
  char* ws = (char*)workspace;
  float* partials = (float*)(ws + l.partials);
  double* tile_sum = (double*)(ws + l.tile_sum);
  uint32_t* tile_flags = (uint32_t*)(ws + l.tile_flags);
  StopState* stop = (StopState*)(ws + l.stop);
  int32_t* slow = (int32_t*)(ws + l.slow);
  const RowGeom geo = row_geom(vocab);
  const int64_t tiles = (vocab + kTile - 1) / kTile;
  if (tiles > 65535) return RLT_ERR_UNSUPPORTED;  // grid.y of the tile kernel
  const int64_t p_rows = n * (w1 + 1);
  // partials_ready: 0 none, 1 the q rows', 2 the p and q rows'
  if (partials_ready == 1)
    launch_mass_groups(p, nullptr, p_rows, p_rows, vocab, partials, stream);
  else if (partials_ready == 0)
    launch_mass_groups(p, w1 > 0 ? q : nullptr, p_rows, rows, vocab, partials, stream);
  // tiles per workgroup: enough workgroups to fill the GPU twice, the stop state (row
  // masses, accept chain) paid once per workgroup
  const int64_t tpg = std::max<int64_t>(1, std::min<int64_t>(tiles, n * tiles / 512));
  const int64_t groups_y = (tiles + tpg - 1) / tpg;
  rlt_accept_tiles_kernel<<<dim3((unsigned)n, (unsigned)groups_y), kDrawThreads, 0, stream>>>(
      p, q, w1, vocab, n, geo.groups > 0 ? partials : nullptr, geo.groups, draft_tokens, drafts,
      u_accept, tile_sum, tile_flags, stop, tiles, (int)tpg);
  rlt_accept_draw_kernel<<<(unsigned)n, kDrawThreads, 0, stream>>>(
      p, q, w1, vocab, tiles, u_final, tile_sum, tile_flags, stop, final_token, tokens, accepted,
      error, slow);
  return rlt_launch_status();
}

}  // namespace

// The mass partials of the p rows inside an acceptance workspace (p row r at
// partials + r * groups * 32), for a launch that computes them.
float* rlt_accept_p_partials(void* workspace, int64_t n, int32_t w1, int64_t vocab) {
  const Layout l = layout_for(n * (2 * (int64_t)w1 + 1), n, vocab);
  return (float*)((char*)workspace + l.partials);
}

// The mass partials of the q rows inside an acceptance workspace (q row r at
// partials + r * groups * 32), for a launch that computes them.
float* rlt_accept_q_partials(void* workspace, int64_t n, int32_t w1, int64_t vocab) {
  const Layout l = layout_for(n * (2 * (int64_t)w1 + 1), n, vocab);
  return (float*)((char*)workspace + l.partials) +
         n * (w1 + 1) * row_geom(vocab).groups * kStreams;
}

// speculative_accept after the q rows' partials were written into the workspace.
int rlt_accept_after_q_partials(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                                const float* p, const float* u_accept, const float* u_final,
                                int64_t n, int32_t w1, int64_t vocab, int64_t* tokens,
                                int64_t* accepted, int64_t* final_token, uint8_t* error,
                                void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return accept_launch(draft_tokens, drafts, q, p, u_accept, u_final, n, w1, vocab, tokens,
                       accepted, final_token, error, workspace, workspace_bytes, 1, stream);
}

// speculative_accept after the p and q rows' partials were written into the workspace.
int rlt_accept_after_pq_partials(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                                 const float* p, const float* u_accept, const float* u_final,
                                 int64_t n, int32_t w1, int64_t vocab, int64_t* tokens,
                                 int64_t* accepted, int64_t* final_token, uint8_t* error,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return accept_launch(draft_tokens, drafts, q, p, u_accept, u_final, n, w1, vocab, tokens,
                       accepted, final_token, error, workspace, workspace_bytes, 2, stream);
}

// ------------------------------------------------------------ no-allocation form

namespace {

// The acceptance workspace of rlt_speculative_accept_noalloc: one copy per GPU,
// held until the process ends.  Host code never passes this name to a kernel (on
// the host it is only a stand-in for the symbol); it passes the device address
// hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up once per device with that device
// current; nullptr on failure.
void* scratch_for_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

size_t rlt_speculative_accept_workspace_size(int64_t n, int32_t w1, int64_t vocab) {
  return layout_for(n * (2 * (int64_t)w1 + 1), n, vocab).total;
}

size_t rlt_categorical_workspace_size(int64_t m, int64_t vocab) {
  return layout_for(0, m, vocab).total;
}

int rlt_speculative_accept(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                           const float* p, const float* u_accept, const float* u_final, int64_t n,
                           int32_t w1, int64_t vocab, int64_t* tokens, int64_t* accepted,
                           int64_t* final_token, uint8_t* error, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  return accept_launch(draft_tokens, drafts, q, p, u_accept, u_final, n, w1, vocab, tokens,
                       accepted, final_token, error, workspace, workspace_bytes, 0, stream);
}

size_t rlt_speculative_accept_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

int rlt_speculative_accept_noalloc(const int64_t* draft_tokens, const int64_t* drafts,
                                   const float* q, const float* p, const float* u_accept,
                                   const float* u_final, int64_t n, int32_t w1, int64_t vocab,
                                   int64_t* tokens, int64_t* accepted, int64_t* final_token,
                                   uint8_t* error, hipStream_t stream) {
  if (n < 0 || w1 < 0 || w1 > kMaxW1 || vocab < 1) return RLT_ERR_ARGUMENT;
  if (n == 0) return RLT_OK;
  // Every kernel writes the parts of the workspace it later reads (the one counter
  // it only increments is diagnostic), so the array needs no clearing between calls.
  const size_t need = layout_for(n * (2 * (int64_t)w1 + 1), n, vocab).total;
  if (need > kNoAllocScratchBytes) return RLT_ERR_WORKSPACE;
  void* ws = scratch_for_current_device();
  if (!ws) return RLT_ERR_LAUNCH;
  return accept_launch(draft_tokens, drafts, q, p, u_accept, u_final, n, w1, vocab, tokens,
                       accepted, final_token, error, ws, kNoAllocScratchBytes, 0, stream);
}

int rlt_categorical(const float* weights, const float* u, int64_t m, int64_t vocab,
                    int64_t* index, uint8_t* valid, void* workspace, size_t workspace_bytes,
                    hipStream_t stream) {
  if (m < 0 || vocab < 1) return RLT_ERR_ARGUMENT;
  if (m == 0) return RLT_OK;
  return launch_categorical(weights, vocab, u, m, vocab, index, valid, nullptr, m, workspace,
                            workspace_bytes, stream);
}

size_t rlt_row_mass_workspace_size(int64_t rows, int64_t vocab) {
  return layout_for(rows, 0, vocab).total;
}

int rlt_row_mass_f32(const float* x, int64_t rows, int64_t vocab, float* out, void* workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  if (rows < 0 || vocab < 1) return RLT_ERR_ARGUMENT;
  if (vocab >= ((int64_t)1 << 25)) return RLT_ERR_UNSUPPORTED;
  if (rows == 0) return RLT_OK;
  const Layout l = layout_for(rows, 0, vocab);
  if (!workspace || workspace_bytes < l.total) return RLT_ERR_WORKSPACE;
  float* partials = (float*)((char*)workspace + l.partials);
  const RowGeom geo = row_geom(vocab);
  launch_mass_groups(x, nullptr, rows, rows, vocab, partials, stream);
  rlt_row_mass_kernel<<<(unsigned)rows, 64, 0, stream>>>(x, vocab, geo.groups > 0 ? partials : nullptr,
                                                         geo.groups, out);
  return rlt_launch_status();
}

}  // extern "C"

// Categorical draws over strided weight rows, scattered into out_index (used by the
// draft proposal in probabilities.hip); the workspace is rlt_categorical's.
int rlt_categorical_rows(const float* weights, int64_t w_stride, const float* u, int64_t m,
                         int64_t vocab, int64_t* out_index, const int64_t* scatter, int64_t n_out,
                         void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || vocab < 1 || w_stride < vocab) return RLT_ERR_ARGUMENT;
  if (m == 0) return RLT_OK;
  return launch_categorical(weights, w_stride, u, m, vocab, out_index, nullptr, scatter, n_out,
                            workspace, workspace_bytes, stream);
}

// The tile totals and flags inside a categorical workspace of m rows (row i, tile k
// at [i tiles + k]; tiles = ceil(vocab / 4096)), for a launch that writes them with the
// weights; nullptr when rows of this vocabulary do not take the two-launch form.
double* rlt_categorical_tile_sums(void* workspace, int64_t m, int64_t vocab) {
  if ((vocab + kTile - 1) / kTile > kMaxTiles) return nullptr;
  return (double*)((char*)workspace + layout_for(0, m, vocab).tile_sum);
}

uint32_t* rlt_categorical_tile_flags(void* workspace, int64_t m, int64_t vocab) {
  if ((vocab + kTile - 1) / kTile > kMaxTiles) return nullptr;
  return (uint32_t*)((char*)workspace + layout_for(0, m, vocab).tile_flags);
}

// rlt_categorical_rows after a launch that wrote the tile totals and flags of the
// weight rows into the workspace (rlt_categorical_tile_sums): the draws only.
int rlt_categorical_rows_after_tiles(const float* weights, int64_t w_stride, const float* u,
                                     int64_t m, int64_t vocab, int64_t* out_index,
                                     const int64_t* scatter, int64_t n_out, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || vocab < 1 || w_stride < vocab) return RLT_ERR_ARGUMENT;
  if (m == 0) return RLT_OK;
  return launch_categorical(weights, w_stride, u, m, vocab, out_index, nullptr, scatter, n_out,
                            workspace, workspace_bytes, stream, true);
}

// ============================================================ random-round merge

namespace {

constexpr int kMergeThreads = 1024;

// One workgroup, three phases separated by workgroup barriers (global writes are
// visible to the whole workgroup after __syncthreads): copy the greedy round's
// values, overlay the random requests' outcomes, then form the slot values.
// Indices outside their ranges are skipped and fail the whole round.
__global__ __launch_bounds__(kMergeThreads) void rlt_merge_random_round_kernel(
    const int64_t* __restrict__ target, int64_t num_rows, const int64_t* __restrict__ accepted,
    const int64_t* __restrict__ next_tokens, const int64_t* __restrict__ starts,
    const int64_t* __restrict__ input_tokens, int64_t n, const int64_t* __restrict__ tokens,
    int32_t width, const int64_t* __restrict__ r_accepted, const int64_t* __restrict__ r_final,
    const uint8_t* __restrict__ r_error, const int64_t* __restrict__ random_requests, int64_t r,
    const int64_t* __restrict__ verify_rows, const int64_t* __restrict__ verify_ranks,
    const int64_t* __restrict__ verify_offsets, int64_t num_verify, int64_t* rows_out,
    int64_t* accepted_out, int64_t* next_tokens_out, int64_t* next_positions_out,
    int64_t* next_values_out, int64_t* error_out) {
  __shared__ int bad_plan;
  const int t = threadIdx.x;
  if (t == 0) bad_plan = 0;
  for (int64_t i = t; i < num_rows; i += kMergeThreads) rows_out[i] = target[i];
  for (int64_t i = t; i < n; i += kMergeThreads) {
    accepted_out[i] = accepted[i];
    next_tokens_out[i] = next_tokens[i];
    error_out[i] = 0;
  }
  __syncthreads();
  for (int64_t k = t; k < num_verify; k += kMergeThreads) {
    const int64_t row = verify_rows[k], rank = verify_ranks[k], off = verify_offsets[k];
    if (row >= 0 && row < num_rows && rank >= 0 && rank < r && off >= 0 && off < width)
      rows_out[row] = tokens[rank * width + off];
    else
      bad_plan = 1;
  }
  for (int64_t k = t; k < r; k += kMergeThreads) {
    const int64_t req = random_requests[k];
    if (req >= 0 && req < n) {
      accepted_out[req] = r_accepted[k];
      next_tokens_out[req] = r_final[k];
      error_out[req] = r_error[k] ? 1 : 0;
    } else {
      bad_plan = 1;
    }
  }
  __syncthreads();
  // An index outside its range (where the reference's indexing raises) fails the
  // whole round: every request reports an error and keeps its slot values.
  const bool bad = bad_plan != 0;
  for (int64_t i = t; i < n; i += kMergeThreads) {
    const int64_t pos = starts[i] + accepted_out[i] + 1;
    next_positions_out[i] = pos;
    if (bad) error_out[i] = 1;
    const bool failed = error_out[i] != 0;
    next_values_out[2 * i] = failed ? input_tokens[i] : next_tokens_out[i];
    next_values_out[2 * i + 1] = failed ? starts[i] : pos;
  }
}

}  // namespace

extern "C" {

int rlt_merge_random_round(const int64_t* target, int64_t num_rows, const int64_t* accepted,
                           const int64_t* next_tokens, const int64_t* starts,
                           const int64_t* input_tokens, int64_t n, const int64_t* tokens,
                           int32_t width, const int64_t* r_accepted, const int64_t* r_final,
                           const uint8_t* r_error, const int64_t* random_requests, int64_t r,
                           const int64_t* verify_rows, const int64_t* verify_ranks,
                           const int64_t* verify_offsets, int64_t num_verify, int64_t* rows_out,
                           int64_t* accepted_out, int64_t* next_tokens_out,
                           int64_t* next_positions_out, int64_t* next_values_out,
                           int64_t* error_out, hipStream_t stream) {
  if (num_rows < 0 || n < 0 || r < 0 || num_verify < 0 || width < 0) return RLT_ERR_ARGUMENT;
  if (num_rows == 0 && n == 0) return RLT_OK;
  rlt_merge_random_round_kernel<<<1, kMergeThreads, 0, stream>>>(
      target, num_rows, accepted, next_tokens, starts, input_tokens, n, tokens, width, r_accepted,
      r_final, r_error, random_requests, r, verify_rows, verify_ranks, verify_offsets, num_verify,
      rows_out, accepted_out, next_tokens_out, next_positions_out, next_values_out, error_out);
  return rlt_launch_status();
}

}  // extern "C"

// ============================================================ sync-mode rejection

// Per-token rejection sampling of the synchronous runner
// (vllm_rlt/worker/speculative.py:56-72 rejection_sample, driven by _collect_round
// :574-625), for a batch of requests in three launches:
//
//  1. rlt_reject_chain_kernel -- grid (n, tiles): every workgroup walks its
//     request's drafts in order (candidate range, q[x] > 0, u * q[x] < p[x]) up to
//     the first event, and on a rejection writes its tile of the residual
//     clamp_min(p - q, 0) of that draft's rows; tile 0 records the event.
//  2. rlt_reject_groups_kernel -- grid (groups, chunks, n): the float32 cascade
//     partials of the residual rows, per summation chunk.
//  3. rlt_reject_scale_kernel -- grid (n, tiles): the residual total in torch's
//     order for a whole 1-D tensor (`residual.sum()`), its validity, and the
//     residual divided by it; tile 0 writes status and accepted.
//
// torch sums a contiguous 1-D float32 tensor serially (the row cascade) when it
// has fewer than 32768 elements or runs on one thread; otherwise in
// c = min(threads, ceil(V / 32768)) chunks of ceil(V / c), each summed with the
// row cascade into a `threads`-long zero buffer that is then summed the same way.

namespace {

constexpr int kRejThreads = 256;
constexpr int kRejTile = kRejThreads * 4;  // residual elements per workgroup
constexpr int64_t kSumGrain = 32768;
constexpr int kMaxSumThreads = 256;

enum RejectStatus : int32_t {
  kRejAllAccepted = 0,  // every draft accepted: the bonus comes from p[count]
  kRejRejected = 1,     // rejected at `accepted`: the residual row is normalized
  kRejZeroMass = 2,     // q[x] is not > 0 at `accepted` (the reference raises ValueError)
  kRejBadResidual = 3,  // residual total not finite and > 0 (RuntimeError)
  kRejBadToken = 4,     // candidate outside [-V, V) at `accepted` (IndexError)
};

struct RejectState {
  int32_t status;
  int32_t s;  // drafts accepted before the event
};

struct SumGeom {
  int64_t chunks, size;  // summation chunks of the row and their length
};

SumGeom sum_geom(int64_t V, int threads) {
  SumGeom g;
  if (V < kSumGrain || threads <= 1) {
    g.chunks = 1;
    g.size = V;
  } else {
    g.chunks = min((V + kSumGrain - 1) / kSumGrain, (int64_t)threads);
    g.size = (V + g.chunks - 1) / g.chunks;
  }
  return g;
}

// The reference's draft loop for request i up to its first event.
__device__ RejectState reject_chain(const int64_t* cand, int64_t K, int64_t d, const float* p,
                                    const float* q, const float* u, int64_t i, int64_t V) {
  RejectState r;
  for (int64_t j = 0; j < d; ++j) {
    const int64_t c = cand[i * K + j];
    r.s = (int32_t)j;
    if (c < -V || c >= V) {
      r.status = kRejBadToken;
      return r;
    }
    const int64_t x = c < 0 ? c + V : c;
    const float mass = q[(i * K + j) * V + x];
    if (!(mass > 0.f)) {
      r.status = kRejZeroMass;
      return r;
    }
    const float prod = u[i * K + j] * mass;
    if (!(prod < p[(i * (K + 1) + j) * V + x])) {
      r.status = kRejRejected;
      return r;
    }
  }
  r.status = kRejAllAccepted;
  r.s = (int32_t)d;
  return r;
}

__global__ __launch_bounds__(kRejThreads) void rlt_reject_chain_kernel(
    const int64_t* __restrict__ cand, const int64_t* __restrict__ counts, const float* __restrict__ p,
    const float* __restrict__ q, const float* __restrict__ u, int64_t K, int64_t V,
    float* __restrict__ residual, RejectState* __restrict__ state) {
  __shared__ RejectState sh;
  const int64_t i = blockIdx.x;
  if (threadIdx.x == 0) {
    const int64_t dc = counts[i];
    sh = reject_chain(cand, K, dc < 0 ? 0 : (dc > K ? K : dc), p, q, u, i, V);
    if (blockIdx.y == 0) state[i] = sh;
  }
  __syncthreads();
  if (sh.status != kRejRejected) return;
  const float* pr = p + (i * (K + 1) + sh.s) * V;
  const float* qr = q + (i * K + sh.s) * V;
  float* out = residual + i * V;
  const int64_t base = (int64_t)blockIdx.y * kRejTile;
  for (int e = threadIdx.x; e < kRejTile; e += kRejThreads) {
    const int64_t k = base + e;
    if (k < V) {
      const float r = pr[k] - qr[k];
      out[k] = r < 0.f ? 0.f : r;  // clamp_min(0): NaN stays NaN
    }
  }
}

// grid (groups of the longest chunk, chunks, n), 128 threads.
template <bool kVec4>
__global__ __launch_bounds__(128) void rlt_reject_groups_kernel(
    const float* __restrict__ residual, const RejectState* __restrict__ state, int64_t V,
    int64_t size, int64_t gmax, float* __restrict__ partials) {
  __shared__ cascade::ChunkSums chunk_sum;
  const int64_t i = blockIdx.z, c = blockIdx.y, g = blockIdx.x;
  if (state[i].status != kRejRejected) return;
  const int64_t b = c * size;
  const int64_t len = min(size, V - b);
  const RowGeom geo = row_geom(len);
  if (g >= geo.groups) return;
  const int t = threadIdx.x;
  cascade::group_chunk_sums<kVec4>(residual + i * V + b, g, geo.full_chunks, t, chunk_sum);
  __syncthreads();
  cascade::group_stream_sums(g, geo.full_chunks, t, chunk_sum,
                             partials + ((i * gridDim.y + c) * gmax + g) * kStreams);
}

__global__ __launch_bounds__(kRejThreads) void rlt_reject_scale_kernel(
    float* __restrict__ residual, const RejectState* __restrict__ state, int64_t V, int64_t chunks,
    int64_t size, int64_t gmax, const float* __restrict__ partials, int threads,
    int32_t* __restrict__ status_out, int64_t* __restrict__ accepted_out) {
  __shared__ float buf[kMaxSumThreads];
  __shared__ float total_sh;
  const int64_t i = blockIdx.x;
  const RejectState st = state[i];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  if (st.status != kRejRejected) {
    if (blockIdx.y == 0 && t == 0) {
      status_out[i] = st.status;
      accepted_out[i] = st.s;
    }
    return;
  }
  float* row = residual + i * V;
  const float* part = partials + i * chunks * gmax * kStreams;
  if (chunks == 1) {
    if (wave == 0) {
      const float s = rlt_row_mass_finish(row, V, row_geom(V).groups > 0 ? part : nullptr);
      if (lane == 0) total_sh = 0.f + s;
    }
  } else {
    for (int c = t; c < threads; c += kRejThreads) buf[c] = 0.f;
    __syncthreads();
    for (int64_t c = wave; c < chunks; c += kRejThreads / 64) {
      const int64_t b = c * size;
      const int64_t len = min(size, V - b);
      const float s = rlt_row_mass_finish(row + b, len,
                                          row_geom(len).groups > 0 ? part + c * gmax * kStreams : nullptr);
      if (lane == 0) buf[c] = 0.f + s;
    }
    __syncthreads();
    if (wave == 0) {
      const float s = rlt_row_mass_finish(buf, threads, nullptr);
      if (lane == 0) total_sh = 0.f + s;
    }
  }
  __syncthreads();
  const float total = total_sh;
  const bool ok = isfinite(total) && total > 0.f;
  if (blockIdx.y == 0 && t == 0) {
    status_out[i] = ok ? kRejRejected : kRejBadResidual;
    accepted_out[i] = st.s;
  }
  const int64_t base = (int64_t)blockIdx.y * kRejTile;
  for (int e = t; e < kRejTile; e += kRejThreads) {
    const int64_t k = base + e;
    if (k < V) row[k] = __fdiv_rn(row[k], total);
  }
}

struct RejectLayout {
  size_t state, partials, total;
};

RejectLayout reject_layout(int64_t n, int64_t V, int threads) {
  const SumGeom sg = sum_geom(V, threads);
  const int64_t gmax = row_geom(sg.size).groups;
  RejectLayout l;
  l.state = 0;
  size_t off = rlt_align_up(sizeof(RejectState) * n, 256);
  l.partials = off;
  off = rlt_align_up(off + sizeof(float) * n * sg.chunks * gmax * kStreams, 256);
  l.total = off;
  return l;
}

}  // namespace

extern "C" {

size_t rlt_rejection_sample_workspace_size(int64_t n, int64_t vocab, int32_t sum_threads) {
  return reject_layout(n, vocab, sum_threads).total;
}

int rlt_rejection_sample(const int64_t* candidates, const int64_t* counts, const float* target,
                         const float* proposal, const float* uniforms, int64_t n, int32_t k,
                         int64_t vocab, int32_t sum_threads, int32_t* status, int64_t* accepted,
                         float* residual, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  if (n < 0 || k < 0 || vocab < 1 || sum_threads < 1) return RLT_ERR_ARGUMENT;
  if (sum_threads > kMaxSumThreads || vocab >= ((int64_t)1 << 31)) return RLT_ERR_UNSUPPORTED;
  if (n == 0) return RLT_OK;
  const RejectLayout l = reject_layout(n, vocab, sum_threads);
  if (!workspace || workspace_bytes < l.total) return RLT_ERR_WORKSPACE;
  const int64_t tiles = (vocab + kRejTile - 1) / kRejTile;
  if (n >= ((int64_t)1 << 31) || tiles > 65535) return RLT_ERR_UNSUPPORTED;
  RejectState* state = (RejectState*)((char*)workspace + l.state);
  float* partials = (float*)((char*)workspace + l.partials);
  const SumGeom sg = sum_geom(vocab, sum_threads);
  const int64_t gmax = row_geom(sg.size).groups;
  rlt_reject_chain_kernel<<<dim3((unsigned)n, (unsigned)tiles), kRejThreads, 0, stream>>>(
      candidates, counts, target, proposal, uniforms, k, vocab, residual, state);
  if (gmax > 0) {
    if (n > 65535) return RLT_ERR_UNSUPPORTED;  // grid.z
    const dim3 grid((unsigned)gmax, (unsigned)sg.chunks, (unsigned)n);
    const bool vec = vocab % 4 == 0 && sg.size % 4 == 0 && (uintptr_t)residual % 16 == 0;
    if (vec)
      rlt_reject_groups_kernel<true><<<grid, 128, 0, stream>>>(residual, state, vocab, sg.size,
                                                               gmax, partials);
    else
      rlt_reject_groups_kernel<false><<<grid, 128, 0, stream>>>(residual, state, vocab, sg.size,
                                                                gmax, partials);
  }
  rlt_reject_scale_kernel<<<dim3((unsigned)n, (unsigned)tiles), kRejThreads, 0, stream>>>(
      residual, state, vocab, sg.chunks, sg.size, gmax, partials, sum_threads, status, accepted);
  return rlt_launch_status();
}

}  // extern "C"
