// Acceptance / rejection sampler for speculative verification on MI355X (gfx950).
//
// Replaces the eager torch chain of vllm_rlt/worker/speculative_sampling.py:59-181
// (``categorical`` and ``speculative_accept``) with four vocab-wide passes that are
// bit-exact against the torch-CPU arithmetic the reference defines:
//
//  1. rlt_mass_groups_kernel  -- every p and q row, split into 8192-float groups:
//     each group's per-stream partial of torch's fp32 cascade row sum.
//  2. rlt_accept_stop_kernel  -- one wave per request: finishes the exact fp32
//     masses, then the accept chain (px >= qx or u*qx < px), the stop point s and
//     the stop-point validity.
//  3. rlt_weight_tiles_kernel -- the final distribution (p[s]/mass at the end of
//     the drafts, else clamp_min(p[s]/pm - q[s]/qm, 0)) in 2048-token tiles:
//     per-tile float64 totals plus non-finite / negative / positive flags.
//  4. rlt_draw_kernel         -- per request: locates the tile and token where the
//     float64 CDF crosses t = u * mass, certifies the crossing against a bound on
//     the difference between any float64 summation order and torch's sequential
//     cumsum, and otherwise replays the sequential cumsum on one lane (exact by
//     construction).  Writes tokens / accepted / final / error.
//
// The standalone ``categorical`` runs passes 3 and 4 on raw weights.
//
// torch's fp32 row-sum order (what ``p.sum(-1, dtype=float32)`` computes on CPU):
// 32 streams, stream s = 8k + l owns elements 32*i + s (8-lane vectors, 4 in
// flight); each stream is a 4-level cascade: 16 elements per chunk (level 0),
// chunks summed sequentially into level 1, flushed to level 2 every 16 chunks
// (one "group" = 16 chunks = 8192 floats of the row), level 2 flushed to level 3
// every 16 groups; leftovers per the final combine in rlt_row_mass_finish().

#include "common.h"
#include "rlt_mi355x.h"

#include <math.h>

namespace {

constexpr int kStreams = 32;          // 8 lanes x ILP 4
constexpr int kChunkSteps = 16;       // stream steps per level-0 chunk
constexpr int kGroupChunks = 16;      // chunks per level-1 group
constexpr int kGroupFloats = kStreams * kChunkSteps * kGroupChunks;  // 8192
constexpr int kTileThreads = 256;
constexpr int kTileElems = 8;                              // per thread
constexpr int kTile = kTileThreads * kTileElems;           // 2048 tokens
constexpr int kMaxTiles = 1024;                            // V <= 2M on the fast path

struct RowGeom {
  int64_t vs;  // whole 8-lane vectors
  int64_t si;  // steps per stream
  int64_t full_chunks;
  int64_t groups;  // level-1 groups holding >= 1 full chunk
};

__host__ __device__ inline RowGeom row_geom(int64_t V) {
  RowGeom g;
  g.vs = V / 8;
  g.si = g.vs / 4;
  g.full_chunks = g.si / kChunkSteps;
  g.groups = (g.full_chunks + kGroupChunks - 1) / kGroupChunks;
  return g;
}

// ------------------------------------------------------------------ pass 1

// grid (groups, rows), 128 threads: thread t sums chunk t/8 of the group for the
// four streams 4*(t%8)..+3 (16 sequential fp32 adds each), then 32 threads add the
// chunk sums of their stream in order (level-1 accumulator).
template <bool kVec4>
__global__ __launch_bounds__(128) void rlt_mass_groups_kernel(const float* __restrict__ p,
                                                              const float* __restrict__ q,
                                                              int64_t p_rows, int64_t V,
                                                              int64_t groups, int64_t full_chunks,
                                                              float* __restrict__ out) {
  __shared__ float chunk_sum[kGroupChunks][kStreams + 1];
  const int64_t row = blockIdx.y;
  const int64_t g = blockIdx.x;
  const float* x = row < p_rows ? p + row * V : q + (row - p_rows) * V;
  const int t = threadIdx.x;
  const int cc = t >> 3;
  const int quad = t & 7;
  const int64_t chunks_here = min<int64_t>(kGroupChunks, full_chunks - g * kGroupChunks);
  if (cc < chunks_here) {
    const float* base = x + g * kGroupFloats + (int64_t)cc * (kStreams * kChunkSteps) + quad * 4;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (kVec4) {
      float4 v[kChunkSteps];
#pragma unroll
      for (int e = 0; e < kChunkSteps; ++e) v[e] = *(const float4*)(base + e * kStreams);
#pragma unroll
      for (int e = 0; e < kChunkSteps; ++e) {
        a0 += v[e].x; a1 += v[e].y; a2 += v[e].z; a3 += v[e].w;
      }
    } else {
#pragma unroll 4
      for (int e = 0; e < kChunkSteps; ++e) {
        a0 += base[e * kStreams + 0];
        a1 += base[e * kStreams + 1];
        a2 += base[e * kStreams + 2];
        a3 += base[e * kStreams + 3];
      }
    }
    chunk_sum[cc][quad * 4 + 0] = a0;
    chunk_sum[cc][quad * 4 + 1] = a1;
    chunk_sum[cc][quad * 4 + 2] = a2;
    chunk_sum[cc][quad * 4 + 3] = a3;
  }
  __syncthreads();
  if (t < kStreams) {
    float acc1 = 0.f;
    for (int c = 0; c < chunks_here; ++c) acc1 += chunk_sum[c][t];
    out[(row * groups + g) * kStreams + t] = acc1;
  }
}

// Exact torch-CPU fp32 row sum of x[0..V) from the group partials (or from
// memory alone when V < 32 / partials == nullptr).  Called by one full wave; the
// result is valid in every lane.
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
    for (int64_t g = 0; g < complete; ++g) {
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

__device__ __forceinline__ bool finite_pos(float m) { return isfinite(m) && m > 0.f; }

// ------------------------------------------------------------------ pass 2

struct StopState {
  int32_t s;        // leading valid accepts
  int32_t at_end;   // s == d: the final draw is the bonus from p[s]
  int32_t stop_ok;  // the stop point is numerically valid
  int32_t err0;     // drafts out of [0, W1]
  float pm;         // p[s] mass
  float qm;         // q[s] mass (residual only)
  int32_t pad[2];
};

// grid (n), 64 threads.  reference: speculative_sampling.py:136-172.
__global__ __launch_bounds__(64) void rlt_accept_stop_kernel(
    const int64_t* __restrict__ draft_tokens, const int64_t* __restrict__ drafts,
    const float* __restrict__ q, const float* __restrict__ p, const float* __restrict__ u_accept,
    int64_t n, int W1, int64_t V, const float* __restrict__ partials, int64_t groups,
    StopState* __restrict__ state) {
  const int64_t i = blockIdx.x;
  const int lane = threadIdx.x;
  // Masses: rows j of p (W1 + 1) and q (W1), exact torch order.
  __shared__ float pm_s[33], qm_s[32];
  for (int j = 0; j <= W1; ++j) {
    const int64_t row = i * (W1 + 1) + j;
    float m = rlt_row_mass_finish(p + row * V, V, partials ? partials + row * groups * kStreams : nullptr);
    if (lane == 0) pm_s[j] = m;
  }
  for (int j = 0; j < W1; ++j) {
    const int64_t row = i * W1 + j;
    const int64_t prow = n * (W1 + 1) + row;
    float m = rlt_row_mass_finish(q + row * V, V, partials ? partials + prow * groups * kStreams : nullptr);
    if (lane == 0) qm_s[j] = m;
  }
  __syncthreads();
  if (lane != 0) return;
  const int64_t dr = drafts[i];
  const int64_t d = dr < 0 ? 0 : (dr > W1 ? W1 : dr);
  int s = 0;
  bool chain = true;
  bool invalid_at_s = false;
  for (int j = 0; j < W1; ++j) {
    const int64_t tok = draft_tokens[i * W1 + j];
    const bool in_range = tok >= 0 && tok < V;
    const int64_t x = tok < 0 ? 0 : (tok > V - 1 ? V - 1 : tok);
    const float pmj = pm_s[j], qmj = qm_s[j];
    const float px = __fdiv_rn(p[(i * (W1 + 1) + j) * V + x], pmj);
    const float qx = __fdiv_rn(q[(i * W1 + j) * V + x], qmj);
    const bool invalid = !(finite_pos(pmj) && finite_pos(qmj) && in_range && isfinite(px) &&
                           isfinite(qx) && qx > 0.f);
    const float ua = u_accept[i * W1 + j];
    const bool accept = !invalid && ((px >= qx) || (ua * qx < px)) && (j < d);
    if (chain) {
      if (accept) {
        ++s;
      } else {
        chain = false;
        invalid_at_s = invalid;  // meaningful only when s < d
      }
    }
  }
  const bool at_end = s == d;
  StopState st;
  st.s = s;
  st.at_end = at_end;
  st.stop_ok = at_end ? finite_pos(pm_s[s]) : !invalid_at_s;
  st.err0 = dr != d;
  st.pm = pm_s[s];
  st.qm = at_end ? 1.f : qm_s[s];
  st.pad[0] = st.pad[1] = 0;
  state[i] = st;
}

// ------------------------------------------------------------------ weights

struct WeightRow {
  const float* a;  // p[s] row (or the raw weight row)
  const float* b;  // q[s] row, residual mode only
  float am, bm;
  bool residual;
  bool raw;
};

__device__ __forceinline__ WeightRow weight_row(int mode, int64_t i, const float* p, const float* q,
                                                int W1, int64_t V, const StopState* state) {
  WeightRow w;
  if (mode == 0) {
    w.a = p + i * V;
    w.b = nullptr;
    w.am = w.bm = 1.f;
    w.residual = false;
    w.raw = true;
    return w;
  }
  const StopState st = state[i];
  w.a = p + (i * (W1 + 1) + st.s) * V;
  w.am = st.pm;
  w.residual = !st.at_end;
  w.b = w.residual ? q + (i * W1 + st.s) * V : nullptr;
  w.bm = st.qm;
  w.raw = false;
  return w;
}

// The fp32 weight of token k exactly as torch computes it:
//   at_end: p/pm; else (p/pm - q/qm).clamp_min(0) (NaN propagates).
__device__ __forceinline__ float weight_of(float a, float b, const WeightRow& w) {
  if (w.raw) return a;
  const float pa = __fdiv_rn(a, w.am);
  if (!w.residual) return pa;
  const float r = pa - __fdiv_rn(b, w.bm);
  return r < 0.f ? 0.f : r;
}

struct TileFlags {
  uint32_t nan_or_inf;  // bit0: NaN seen, bit1: +inf seen
  uint32_t neg;         // a negative weight (or -inf) seen
  uint32_t pos;         // a positive weight seen
};

// Loads this thread's 8 weights of tile `tile` (zero past V).
__device__ __forceinline__ void load_weights(const WeightRow& w, int64_t V, int64_t tile, int t,
                                             bool vec_ok, float out[kTileElems]) {
  const int64_t base = tile * kTile + (int64_t)t * kTileElems;
  if (vec_ok && base + kTileElems <= V) {
    const float4 a0 = *(const float4*)(w.a + base);
    const float4 a1 = *(const float4*)(w.a + base + 4);
    float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    float bv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (w.residual) {
      const float4 b0 = *(const float4*)(w.b + base);
      const float4 b1 = *(const float4*)(w.b + base + 4);
      bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w;
      bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
    }
#pragma unroll
    for (int e = 0; e < kTileElems; ++e) out[e] = weight_of(av[e], bv[e], w);
  } else {
#pragma unroll
    for (int e = 0; e < kTileElems; ++e) {
      const int64_t k = base + e;
      out[e] = k < V ? weight_of(w.a[k], w.residual ? w.b[k] : 0.f, w) : 0.f;
    }
  }
}

// Deterministic block sum of one double per thread (fixed tree over 256 lanes).
__device__ double block_sum_f64(double v, double* scratch) {
  const int t = threadIdx.x;
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, RLT_WAVE);
  if ((t & 63) == 0) scratch[t >> 6] = v;
  __syncthreads();
  const double r = ((scratch[0] + scratch[1]) + scratch[2]) + scratch[3];
  __syncthreads();
  return r;
}

// ------------------------------------------------------------------ pass 3

// grid (tiles, n), 256 threads: per-tile float64 total of the final weights.
__global__ __launch_bounds__(kTileThreads) void rlt_weight_tiles_kernel(
    int mode, const float* __restrict__ p, const float* __restrict__ q, int W1, int64_t V,
    const StopState* __restrict__ state, int64_t tiles, double* __restrict__ tile_sum,
    TileFlags* __restrict__ tile_flags) {
  __shared__ double red[4];
  __shared__ uint32_t fl[3];
  const int64_t i = blockIdx.y;
  const int64_t tile = blockIdx.x;
  const int t = threadIdx.x;
  if (t < 3) fl[t] = 0;
  const WeightRow w = weight_row(mode, i, p, q, W1, V, state);
  const bool vec_ok = (V % 4 == 0) && ((((uintptr_t)w.a) | ((uintptr_t)(w.b ? w.b : w.a))) % 16 == 0);
  float wv[kTileElems];
  load_weights(w, V, tile, t, vec_ok, wv);
  double local = 0.0;
  uint32_t nf = 0, neg = 0, pos = 0;
#pragma unroll
  for (int e = 0; e < kTileElems; ++e) {
    const float x = wv[e];
    if (isnan(x)) nf |= 1u;
    else if (isinf(x) && x > 0.f) nf |= 2u;
    if (x < 0.f) neg = 1;
    if (x > 0.f) pos = 1;
    local += (double)x;
  }
  __syncthreads();
  if (nf) atomicOr(&fl[0], nf);
  if (neg) atomicOr(&fl[1], 1u);
  if (pos) atomicOr(&fl[2], 1u);
  const double total = block_sum_f64(local, red);
  if (t == 0) {
    tile_sum[i * tiles + tile] = total;
    TileFlags f;
    f.nan_or_inf = fl[0];
    f.neg = fl[1];
    f.pos = fl[2];
    tile_flags[i * tiles + tile] = f;
  }
}

// ------------------------------------------------------------------ pass 4

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

// grid (n), 256 threads.
__global__ __launch_bounds__(kTileThreads) void rlt_draw_kernel(
    int mode, const float* __restrict__ p, const float* __restrict__ q, int W1, int64_t V,
    const float* __restrict__ u_final, const int64_t* __restrict__ draft_tokens,
    const StopState* __restrict__ state, int64_t tiles, const double* __restrict__ tile_sum,
    const TileFlags* __restrict__ tile_flags, int64_t* __restrict__ out_index,
    uint8_t* __restrict__ out_valid, int64_t* __restrict__ tokens, int64_t* __restrict__ accepted,
    uint8_t* __restrict__ error, int32_t* __restrict__ slow_count) {
  __shared__ double scan[kTileThreads];
  __shared__ int s_decision;  // 0 fast, 1 slow, 2 invalid (index 0)
  __shared__ int64_t s_tile;
  __shared__ double s_tilestart, s_t, s_margin;
  __shared__ int64_t s_best;
  __shared__ double s_before, s_at;
  const int64_t i = blockIdx.x;
  const int t = threadIdx.x;
  const WeightRow w = weight_row(mode, i, p, q, W1, V, state);
  const float u = u_final[i];
  if (t == 0) {
    bool any_nan = false, any_inf = false, any_neg = false, any_pos = false;
    double m = 0.0;
    for (int64_t k = 0; k < tiles; ++k) {
      const TileFlags f = tile_flags[i * tiles + k];
      any_nan |= (f.nan_or_inf & 1u) != 0;
      any_inf |= (f.nan_or_inf & 2u) != 0;
      any_neg |= f.neg != 0;
      any_pos |= f.pos != 0;
      m += tile_sum[i * tiles + k];
    }
    int decision = 0;
    if (any_neg || !(u >= 0.f && u < 1.f) || tiles > kMaxTiles) {
      decision = 1;  // out-of-contract input: exact replay
    } else if (any_nan || any_inf || !any_pos) {
      decision = 2;  // mass NaN / inf / zero: invalid row
    }
    const double tt = (double)u * m;
    // |any float64 order - sequential cumsum| <= (#adds) * 2^-53 * mass per side;
    // doubled for t's own dependence on the mass, plus rounding of u * mass.
    const double margin = (4.0 * (double)V + 64.0) * 0x1p-52 * m;
    int64_t tile = -1;
    double start = 0.0;
    if (decision == 0) {
      double acc = 0.0;
      for (int64_t k = 0; k < tiles; ++k) {
        const double nx = acc + tile_sum[i * tiles + k];
        if (nx > tt) {
          tile = k;
          start = acc;
          break;
        }
        acc = nx;
      }
      if (tile < 0) decision = 1;
    }
    s_decision = decision;
    s_tile = tile;
    s_tilestart = start;
    s_t = tt;
    s_margin = margin;
    s_best = INT64_MAX;
  }
  __syncthreads();
  int decision = s_decision;
  int64_t index = 0;
  bool valid = decision != 2;
  if (decision == 0) {
    const bool vec_ok =
        (V % 4 == 0) && ((((uintptr_t)w.a) | ((uintptr_t)(w.b ? w.b : w.a))) % 16 == 0);
    float wv[kTileElems];
    load_weights(w, V, s_tile, t, vec_ok, wv);
    double local = 0.0;
#pragma unroll
    for (int e = 0; e < kTileElems; ++e) local += (double)wv[e];
    // exclusive scan of thread partials in index order (Hillis-Steele in LDS)
    scan[t] = local;
    __syncthreads();
    for (int off = 1; off < kTileThreads; off <<= 1) {
      const double add = t >= off ? scan[t - off] : 0.0;
      __syncthreads();
      scan[t] += add;
      __syncthreads();
    }
    double run = s_tilestart + (scan[t] - local);
    const double tt = s_t;
    for (int e = 0; e < kTileElems; ++e) {
      run += (double)wv[e];
      if (run > tt) {
        const int64_t k = s_tile * kTile + (int64_t)t * kTileElems + e;
        atomicMin((unsigned long long*)&s_best, (unsigned long long)k);
        break;
      }
    }
    __syncthreads();
    // the owner of the crossing publishes its neighbours' prefix values
    const int64_t best = s_best;
    if (best != INT64_MAX && (best - s_tile * kTile) / kTileElems == t) {
      double r = s_tilestart + (scan[t] - local);
      const int e_best = (int)((best - s_tile * kTile) % kTileElems);
      for (int e = 0; e < e_best; ++e) r += (double)wv[e];
      s_before = r;
      s_at = r + (double)wv[e_best];
    }
    __syncthreads();
    if (t == 0) {
      const bool ok = best != INT64_MAX && s_before <= tt - s_margin && s_at > tt + s_margin;
      s_decision = ok ? 0 : 1;
    }
    __syncthreads();
    decision = s_decision;
    index = best;
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
  if (mode == 0) {
    out_index[i] = index;
    out_valid[i] = valid;
    return;
  }
  const StopState st = state[i];
  const bool err = st.err0 || !(st.stop_ok && valid);
  const int64_t fin = err ? 0 : index;
  out_index[i] = fin;
  error[i] = err;
  accepted[i] = st.s;
  for (int j = 0; j <= W1; ++j) {
    int64_t v = 0;
    if (j < st.s) {
      const int64_t tok = draft_tokens[i * W1 + j];
      v = tok < 0 ? 0 : (tok > V - 1 ? V - 1 : tok);
    } else if (j == st.s) {
      v = fin;
    }
    tokens[i * (W1 + 1) + j] = v;
  }
}

// ------------------------------------------------------------------ workspace

struct AcceptLayout {
  size_t partials, state, tile_sum, tile_flags, slow, total;
};

AcceptLayout accept_layout(int64_t n, int W1, int64_t V) {
  const RowGeom geo = row_geom(V);
  const int64_t rows = n * (2 * W1 + 1);
  const int64_t tiles = (V + kTile - 1) / kTile;
  AcceptLayout l;
  size_t off = 0;
  l.partials = off;
  off = rlt_align_up(off + sizeof(float) * rows * geo.groups * kStreams, 256);
  l.state = off;
  off = rlt_align_up(off + sizeof(StopState) * n, 256);
  l.tile_sum = off;
  off = rlt_align_up(off + sizeof(double) * n * tiles, 256);
  l.tile_flags = off;
  off = rlt_align_up(off + sizeof(TileFlags) * n * tiles, 256);
  l.slow = off;
  off = rlt_align_up(off + sizeof(int32_t), 256);
  l.total = off;
  return l;
}

}  // namespace

extern "C" {

size_t rlt_speculative_accept_workspace_size(int64_t n, int32_t w1, int64_t vocab) {
  return accept_layout(n, w1, vocab).total;
}

size_t rlt_categorical_workspace_size(int64_t m, int64_t vocab) {
  return accept_layout(m, 0, vocab).total;
}

int rlt_speculative_accept(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                           const float* p, const float* u_accept, const float* u_final, int64_t n,
                           int32_t w1, int64_t vocab, int64_t* tokens, int64_t* accepted,
                           int64_t* final_token, uint8_t* error, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  if (n < 0 || w1 < 0 || w1 > 32 || vocab < 1) return RLT_ERR_ARGUMENT;
  if (vocab >= ((int64_t)1 << 25)) return RLT_ERR_UNSUPPORTED;
  if (n == 0) return RLT_OK;
  const AcceptLayout l = accept_layout(n, w1, vocab);
  if (!workspace || workspace_bytes < l.total) return RLT_ERR_WORKSPACE;
  char* ws = (char*)workspace;
  float* partials = (float*)(ws + l.partials);
  StopState* state = (StopState*)(ws + l.state);
  double* tile_sum = (double*)(ws + l.tile_sum);
  TileFlags* tile_flags = (TileFlags*)(ws + l.tile_flags);
  int32_t* slow = (int32_t*)(ws + l.slow);
  const RowGeom geo = row_geom(vocab);
  const int64_t rows = n * (2 * w1 + 1);
  const int64_t p_rows = n * (w1 + 1);
  if (geo.groups > 0) {
    const bool vec = (vocab % 4 == 0) && ((uintptr_t)p % 16 == 0) && ((uintptr_t)q % 16 == 0 || w1 == 0);
    dim3 grid((unsigned)geo.groups, (unsigned)rows);
    if (vec)
      rlt_mass_groups_kernel<true><<<grid, 128, 0, stream>>>(p, q, p_rows, vocab, geo.groups,
                                                             geo.full_chunks, partials);
    else
      rlt_mass_groups_kernel<false><<<grid, 128, 0, stream>>>(p, q, p_rows, vocab, geo.groups,
                                                              geo.full_chunks, partials);
  }
  rlt_accept_stop_kernel<<<(unsigned)n, 64, 0, stream>>>(
      draft_tokens, drafts, q, p, u_accept, n, w1, vocab, geo.groups > 0 ? partials : nullptr,
      geo.groups, state);
  const int64_t tiles = (vocab + kTile - 1) / kTile;
  rlt_weight_tiles_kernel<<<dim3((unsigned)tiles, (unsigned)n), kTileThreads, 0, stream>>>(
      1, p, q, w1, vocab, state, tiles, tile_sum, tile_flags);
  rlt_draw_kernel<<<(unsigned)n, kTileThreads, 0, stream>>>(
      1, p, q, w1, vocab, u_final, draft_tokens, state, tiles, tile_sum, tile_flags, final_token,
      nullptr, tokens, accepted, error, slow);
  return rlt_launch_status();
}

int rlt_categorical(const float* weights, const float* u, int64_t m, int64_t vocab,
                    int64_t* index, uint8_t* valid, void* workspace, size_t workspace_bytes,
                    hipStream_t stream) {
  if (m < 0 || vocab < 1) return RLT_ERR_ARGUMENT;
  if (m == 0) return RLT_OK;
  const AcceptLayout l = accept_layout(m, 0, vocab);
  if (!workspace || workspace_bytes < l.total) return RLT_ERR_WORKSPACE;
  char* ws = (char*)workspace;
  double* tile_sum = (double*)(ws + l.tile_sum);
  TileFlags* tile_flags = (TileFlags*)(ws + l.tile_flags);
  int32_t* slow = (int32_t*)(ws + l.slow);
  const int64_t tiles = (vocab + kTile - 1) / kTile;
  rlt_weight_tiles_kernel<<<dim3((unsigned)tiles, (unsigned)m), kTileThreads, 0, stream>>>(
      0, weights, nullptr, 0, vocab, nullptr, tiles, tile_sum, tile_flags);
  rlt_draw_kernel<<<(unsigned)m, kTileThreads, 0, stream>>>(
      0, weights, nullptr, 0, vocab, u, nullptr, nullptr, tiles, tile_sum, tile_flags, index,
      valid, nullptr, nullptr, nullptr, slow);
  return rlt_launch_status();
}

// Exact torch-CPU fp32 row sums (``x.sum(-1, dtype=float32)``) of a contiguous
// [rows, V] fp32 matrix; exposed for tests and for callers that need the masses.
int rlt_row_mass_f32(const float* x, int64_t rows, int64_t vocab, float* out, void* workspace,
                     size_t workspace_bytes, hipStream_t stream);

}  // extern "C"

namespace {
__global__ __launch_bounds__(64) void rlt_row_mass_kernel(const float* __restrict__ x, int64_t V,
                                                          const float* __restrict__ partials,
                                                          int64_t groups, float* __restrict__ out) {
  const int64_t r = blockIdx.x;
  const float m = rlt_row_mass_finish(x + r * V, V, partials ? partials + r * groups * kStreams : nullptr);
  if (threadIdx.x == 0) out[r] = m;
}
}  // namespace

extern "C" size_t rlt_row_mass_workspace_size(int64_t rows, int64_t vocab) {
  const RowGeom geo = row_geom(vocab);
  return rlt_align_up(sizeof(float) * rows * geo.groups * kStreams + 1, 256);
}

extern "C" int rlt_row_mass_f32(const float* x, int64_t rows, int64_t vocab, float* out,
                                void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (rows < 0 || vocab < 1) return RLT_ERR_ARGUMENT;
  if (vocab >= ((int64_t)1 << 25)) return RLT_ERR_UNSUPPORTED;
  if (rows == 0) return RLT_OK;
  const RowGeom geo = row_geom(vocab);
  if (workspace_bytes < rlt_row_mass_workspace_size(rows, vocab) || !workspace)
    return RLT_ERR_WORKSPACE;
  float* partials = (float*)workspace;
  if (geo.groups > 0) {
    const bool vec = (vocab % 4 == 0) && ((uintptr_t)x % 16 == 0);
    dim3 grid((unsigned)geo.groups, (unsigned)rows);
    if (vec)
      rlt_mass_groups_kernel<true><<<grid, 128, 0, stream>>>(x, x, rows, vocab, geo.groups,
                                                             geo.full_chunks, partials);
    else
      rlt_mass_groups_kernel<false><<<grid, 128, 0, stream>>>(x, x, rows, vocab, geo.groups,
                                                              geo.full_chunks, partials);
  }
  rlt_row_mass_kernel<<<(unsigned)rows, 64, 0, stream>>>(x, vocab, geo.groups > 0 ? partials : nullptr,
                                                         geo.groups, out);
  return rlt_launch_status();
}
