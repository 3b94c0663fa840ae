// torch-CPU's float32 row-sum order, shared by the acceptance sampler
// (spec_sampling.hip) and the distribution kernel (probabilities.hip), which can
// compute the draft rows' partial sums on otherwise idle CUs of its launch.
//
// `x.sum(-1, dtype=float32)` on CPU runs 32 streams, stream s = 8k + l owning the
// elements 32 i + s (8-lane vectors, 4 in flight); each stream is a 4-level cascade:
// 16 elements per chunk (level 0), chunks summed sequentially into level 1, flushed
// to level 2 every 16 chunks (one "group" = 16 chunks = 8192 floats of the row),
// level 2 flushed to level 3 every 16 groups; the row's leftovers follow the final
// combine (spec_sampling.hip, rlt_row_mass_finish).  The functions below give one
// group's level-1 value of every stream; callers put a workgroup barrier between the
// two phases.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cascade {

constexpr int kStreams = 32;      // 8 lanes x ILP 4
constexpr int kChunkSteps = 16;   // stream steps per level-0 chunk
constexpr int kGroupChunks = 16;  // chunks per level-1 group
constexpr int kGroupFloats = kStreams * kChunkSteps * kGroupChunks;  // 8192
constexpr int kGroupThreads = 128;

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

typedef float ChunkSums[kGroupChunks][kStreams + 1];

// Phase 1 (t in [0, 128)): thread t sums chunk t / 8 of group g of row x for the four
// streams 4 (t % 8) .. + 3, 16 sequential float32 adds each, into cs.
template <bool kVec4>
__device__ __forceinline__ void group_chunk_sums(const float* __restrict__ x, int64_t g,
                                                 int64_t full_chunks, int t, ChunkSums& cs) {
  const int cc = t >> 3;
  const int quad = t & 7;
  const int64_t chunks_here = min((int64_t)kGroupChunks, full_chunks - g * kGroupChunks);
  if (cc >= chunks_here) return;
  const float* base = x + g * kGroupFloats + (int64_t)cc * (kStreams * kChunkSteps) + quad * 4;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if (kVec4) {
    float4 v[kChunkSteps];
#pragma unroll
    for (int e = 0; e < kChunkSteps; ++e) v[e] = *(const float4*)(base + e * kStreams);
#pragma unroll
    for (int e = 0; e < kChunkSteps; ++e) {
      a0 += v[e].x;
      a1 += v[e].y;
      a2 += v[e].z;
      a3 += v[e].w;
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
  cs[cc][quad * 4 + 0] = a0;
  cs[cc][quad * 4 + 1] = a1;
  cs[cc][quad * 4 + 2] = a2;
  cs[cc][quad * 4 + 3] = a3;
}

// Phase 2 (after a barrier; t in [0, 128)): stream t < 32 adds the group's chunk sums
// in order (the level-1 accumulator) and stores it to out[t].
__device__ __forceinline__ void group_stream_sums(int64_t g, int64_t full_chunks, int t,
                                                  const ChunkSums& cs, float* __restrict__ out) {
  const int64_t chunks_here = min((int64_t)kGroupChunks, full_chunks - g * kGroupChunks);
  if (t >= kStreams || chunks_here <= 0) return;
  float acc1 = 0.f;
  for (int c = 0; c < chunks_here; ++c) acc1 += cs[c][t];
  out[t] = acc1;
}

}  // namespace cascade
