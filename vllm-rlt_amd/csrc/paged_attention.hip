// Depth-aware paged-KV attention for speculative verification on MI355X (gfx950).
//
// One kernel family serves both forms of the reference attention boundary:
//  * per-row decode / verify (``AttentionBackend.__call__``,
//    vllm_rlt/kernels/paged_attention.py:13-47, triton_attention.py:176-246): every
//    q row has its own block table and context length;
//  * packed verify window (``AttentionBackend.prefill``, triton_attention.py:386-404):
//    sequence s owns q rows cu[s]:cu[s+1], one block table, and query i sees keys
//    < len - q_len + i + 1 (bottom-right aligned causal window).
// The per-row form is the packed form with q_len = 1 per row.
//
// Work decomposition (static grids, graph-capturable: no host-side length reads):
//  The unit of work is (sequence x row-group, kv head, chunk), a chunk being
//  512 absolute key positions [512c, 512c + 512) (1024 for fp8 KV on the MFMA path)
//  processed in 16-position tiles by two waves (one for fp8 KV) whose states combine
//  in a fixed order.  Every row of the sequence (q_len window rows x GQA group)
//  that attends to the kv head is in the unit's row-group, so each KV byte is read
//  once per (sequence, kv head) instead of once per q row.  On the MFMA path one
//  persistent 8-wave workgroup per CU enumerates the active units from the
//  sequence lengths and takes an equal share of them; the vector path runs one
//  4-wave workgroup per (row-group, kv head, chunk) with the chunk split between
//  waves.  Partial (max, sum, unnormalized output) per (row, head, chunk) go to a
//  workspace; rlt_merge_kernel combines a row's chunks in chunk order.
//
// A row's arithmetic depends only on its own length, the absolute tile / chunk
// boundaries and its own q vector -- never on which other rows share its
// workgroup -- so packed verify equals per-row decode bit for bit and results are
// batch invariant (the reference's ``packed_matches_decode`` contract,
// vllm_rlt/attention/backend.py:25-27).  The one exception is a packed call whose
// longest window reaches kPfMinQ = 64 rows (prompt prefill: no verify window is that
// long), which takes the prefill tiling further down (rlt_prefill_kernel).
//
// Math paths of the split kernels (chosen by dtype and head_dim only, never by row count):
//  * MFMA (q bf16/fp16, KV same type or fp8-e4m3, head_dim % 32 == 0, <= 256):
//    S^T = K Q^T with v_mfma_f32_16x16x32_{bf16,f16} straight from global memory
//    (the contraction order is permuted so that each lane's eight elements per
//    step are contiguous in memory: the A-operand layout), online softmax in fp32
//    (log2 domain), then O^T = V^T P^T with v_mfma_f32_16x16x16: the P^T operand
//    is exactly the S^T accumulator layout, and the output dimensions are permuted
//    so that V^T operands are contiguous loads too (no LDS transpose).
//  * vector (fp32 q, or any other head_dim <= 256): fp32 FMA dot products.

#include "common.h"
#include "fp8_codec.h"
#include "rlt_mi355x.h"

#include <climits>
#include <math.h>

#include <type_traits>

namespace {

constexpr int kChunk = 512;       // key positions per workgroup (split unit)
constexpr int kWaves = 4;
constexpr int kWaveSpan = kChunk / kWaves;  // 128 positions per wave
constexpr int kTileTok = 16;
constexpr int kStages = 2;  // KV tiles in flight per wave (MFMA path)
// Waves per work unit on the MFMA path (equal position spans combined in a fixed
// order): two for 16-bit KV; one for fp8 KV, whose 512-position unit is half the bytes
// (one wave streams it alone faster than two that wait at the combine).  Fixed per
// dtype pair, so a row's result never depends on the batch.
template <int QT, int KVT>
constexpr int unit_split() { return KVT == QT ? 2 : 1; }
// Key positions per chunk on the MFMA path: 512 for 16-bit KV, 1024 for fp8 KV (whose
// chunk is the same bytes; one wave streams it).  Fixed per dtype pair, like the split.
template <int QT, int KVT>
constexpr int unit_chunk() { return KVT == QT ? kChunk : 2 * kChunk; }
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
  int chunk_log2;  // log2 of the chunk (split unit) in key positions: 9 or 10
  const void* q;
  int64_t q_row_stride, q_head_stride;
  const void* k;
  const void* v;
  int64_t k_block_stride, k_token_stride, k_head_stride;
  int64_t v_block_stride, v_token_stride, v_head_stride;
  const int32_t* tables;
  int64_t table_stride;
  int32_t table_width;
  int32_t num_blocks;  // physical blocks in the pool: out-of-range table entries read block 0
  const int32_t* lengths;
  const int32_t* cu_q;  // nullptr: per-row form
  const int32_t* row_len;  // packed form: explicit key count of each q row (nullptr: causal window)
  const float* k_scale;
  const float* v_scale;
  int64_t s_block_stride, s_token_stride, s_head_stride;
  int32_t scale_mode;  // 0 none, 1 per-tensor (0-d), 2 per-vector [blk, tok, kvh]
  int32_t compensate;  // MFMA path: P V also with the bits P loses in its 16-bit cast
  int32_t num_seqs;
  int32_t num_rows;  // total q rows
  int32_t hq, hkv, group, head_dim, block_size;
  int32_t window;  // 0: full context
  int32_t max_q;   // longest q window of a sequence (merge grid)
  int32_t rows_per_rg;
  int32_t rowgroups;
  int32_t head_groups;   // kv heads per grid row of work_item (one head per workgroup)
  int32_t persistent;    // MFMA path: one persistent workgroup per CU
  int32_t max_chunks;
  float qk_scale_log2;  // log2(e) / sqrt(head_dim)
  void* out;
  int64_t out_row_stride, out_head_stride;
  float* part_ml;  // [rows][hq][max_chunks][2]  (max in log2 units, sum)
  float* part_o;   // [rows][hq][max_chunks][head_dim]
  // packed form with the window rows' own keys / values to store first (nullptr: none):
  // row r of [rows, kv_heads, head_dim] (strides in elements) goes to its window
  // position through the block table
  const void* new_k;
  const void* new_v;
  int64_t new_row_stride, new_head_stride;
};

struct SeqView {
  int32_t q_begin, q_len, kv_len;
};

// Work item of a flat workgroup id.  Consecutive ids go to different XCDs (the
// dispatcher deals workgroups round-robin over the 8 XCDs), so the chunk index is
// rotated by the (sequence, row-group, kv head) index: every sequence's chunks then
// spread evenly over all XCDs whatever the mix of sequence lengths.
struct WorkItem {
  int seq, rg, hg, chunk;  // hg: kv-head group (heads_per_wg heads)
};

__device__ __forceinline__ WorkItem work_item(const AttnParams& P, int64_t id) {
  WorkItem w;
  const int64_t pair = id / P.max_chunks;
  const int j = (int)(id % P.max_chunks);
  w.chunk = (int)((j + pair) % P.max_chunks);
  w.hg = (int)(pair % P.head_groups);
  const int64_t sr = pair / P.head_groups;
  w.rg = (int)(sr % P.rowgroups);
  w.seq = (int)(sr / P.rowgroups);
  return w;
}

__device__ __forceinline__ SeqView seq_view(const AttnParams& P, int seq) {
  SeqView s;
  if (P.cu_q) {
    s.q_begin = P.cu_q[seq];
    s.q_len = P.cu_q[seq + 1] - s.q_begin;
  } else {
    s.q_begin = seq;
    s.q_len = 1;
  }
  s.kv_len = P.lengths[seq];
  return s;
}

// Row (window index qi) of a sequence: visible key range [lo, hi).
__device__ __forceinline__ void row_range(const AttnParams& P, const SeqView& s, int qi, int& lo,
                                          int& hi) {
  hi = P.row_len ? P.row_len[s.q_begin + qi] : s.kv_len - s.q_len + 1 + qi;
  if (hi < 0) hi = 0;
  // Never read past the row's block table (a length beyond it is a caller error).
  const int cap = P.table_width * P.block_size;
  if (hi > cap) hi = cap;
  lo = P.window > 0 ? max(0, hi - P.window) : 0;
}

// Bounds over the rows [rg_begin, rg_begin + rg_rows) of a sequence (row rho is
// window index rho / group): every row's visible range lies in [lo_min, hi_max),
// and positions in [lo_max, hi_min) are visible to every row.  The causal window's
// ranges grow with the window index, so its first and last rows give the bounds;
// explicit row lengths may come in any order and every row is visited.
__device__ __forceinline__ void group_range(const AttnParams& P, const SeqView& s, int rg_begin,
                                            int rg_rows, int& lo_min, int& hi_min, int& lo_max,
                                            int& hi_max) {
  const int q0 = rg_begin / P.group, q1 = (rg_begin + rg_rows - 1) / P.group;
  row_range(P, s, q0, lo_min, hi_min);
  row_range(P, s, q1, lo_max, hi_max);
  if (P.row_len) {
    if (lo_max < lo_min) {
      const int t = lo_min; lo_min = lo_max; lo_max = t;
    }
    if (hi_max < hi_min) {
      const int t = hi_min; hi_min = hi_max; hi_max = t;
    }
    for (int qi = q0 + 1; qi < q1; ++qi) {
      int lo, hi;
      row_range(P, s, qi, lo, hi);
      lo_min = min(lo_min, lo);
      lo_max = max(lo_max, lo);
      hi_min = min(hi_min, hi);
      hi_max = max(hi_max, hi);
    }
  }
}

// Physical block of key position `pos`; entries outside the pool read block 0
// so that a corrupt table can never address memory outside the KV pool.
__device__ __forceinline__ int64_t block_of(const AttnParams& P, int seq, int pos) {
  const int32_t blk = P.tables[(int64_t)seq * P.table_stride + pos / P.block_size];
  return (blk >= 0 && blk < P.num_blocks) ? (int64_t)blk : 0;
}

__device__ __forceinline__ int64_t kv_token_base(const AttnParams& P, int seq, int pos,
                                                 int64_t block_stride, int64_t token_stride) {
  const int64_t blk = block_of(P, seq, pos);
  return (int64_t)blk * block_stride + (int64_t)(pos % P.block_size) * token_stride;
}

__device__ __forceinline__ float scale_at(const AttnParams& P, const float* s, int seq, int pos,
                                          int kvh) {
  const int64_t blk = block_of(P, seq, pos);
  return s[blk * P.s_block_stride + (int64_t)(pos % P.block_size) * P.s_token_stride +
           (int64_t)kvh * P.s_head_stride];
}

// Merge two online-softmax states (log2 domain) in a fixed operand order.
__device__ __forceinline__ void merge_scales(float m1, float m2, float& mo, float& s1, float& s2) {
  mo = fmaxf(m1, m2);
  s1 = m1 == -INFINITY ? 0.f : exp2f(m1 - mo);
  s2 = m2 == -INFINITY ? 0.f : exp2f(m2 - mo);
}

// ============================================================ MFMA path

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int QT>
struct Mfma;

template <>
struct Mfma<RLT_BF16> {
  __device__ static f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    bf16x8 av, bv;
    __builtin_memcpy(&av, &a, 16);
    __builtin_memcpy(&bv, &b, 16);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
  }
  __device__ static f32x4 pv(uint2 a, uint2 b, f32x4 c) {
    s16x4 av, bv;
    __builtin_memcpy(&av, &a, 8);
    __builtin_memcpy(&bv, &b, 8);
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, c, 0, 0, 0);
  }
  __device__ static uint16_t from_f32(float x) { return f32_to_bf16_bits(x); }
  // the two values of a packed pair, exactly
  __device__ static float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // two floats -> packed pair (v_cvt_pk_bf16_f32, round to nearest even)
  __device__ static uint32_t pack2(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <>
struct Mfma<RLT_F16> {
  __device__ static f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    f16x8 av, bv;
    __builtin_memcpy(&av, &a, 16);
    __builtin_memcpy(&bv, &b, 16);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c, 0, 0, 0);
  }
  __device__ static f32x4 pv(uint2 a, uint2 b, f32x4 c) {
    f16x4 av, bv;
    __builtin_memcpy(&av, &a, 8);
    __builtin_memcpy(&bv, &b, 8);
    return __builtin_amdgcn_mfma_f32_16x16x16f16(av, bv, c, 0, 0, 0);
  }
  __device__ static uint16_t from_f32(float x) { return f32_to_f16_bits(x); }
  __device__ static float lo_f32(uint32_t w) { return f16_bits_to_f32((uint16_t)(w & 0xffffu)); }
  __device__ static float hi_f32(uint32_t w) { return f16_bits_to_f32((uint16_t)(w >> 16)); }
  __device__ static uint32_t pack2(float a, float b) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <bool B>
struct Flag {
  static constexpr bool value = B;
};

// Four fp8 codes -> four 16-bit values of the MFMA type (exact for e4m3).
template <int QT>
__device__ __forceinline__ uint2 fp8x4_to_16(uint32_t w) {
  const float2 lo = fp8x2_to_f32<false>(w);
  const float2 hi = fp8x2_to_f32<true>(w);
  uint2 r;
  if (QT == RLT_BF16) {
    // e4m3 values are exact in bf16: truncation of the fp32 bits is exact.
    r.x = (__float_as_uint(lo.x) >> 16) | (__float_as_uint(lo.y) & 0xffff0000u);
    r.y = (__float_as_uint(hi.x) >> 16) | (__float_as_uint(hi.y) & 0xffff0000u);
  } else {
    r.x = (uint32_t)f32_to_f16_bits(lo.x) | ((uint32_t)f32_to_f16_bits(lo.y) << 16);
    r.y = (uint32_t)f32_to_f16_bits(hi.x) | ((uint32_t)f32_to_f16_bits(hi.y) << 16);
  }
  return r;
}

// One lane's raw key elements, as loaded from HBM: for contraction step s the
// eight elements [32 s + 8 g, + 8) of its position (g = lane group), so the four
// lane groups of one load instruction read 64 (32 for fp8) contiguous bytes of
// each position.  Conversion to the MFMA element type happens at use, so a load
// in flight never forces a wait.
template <int QT, int KVT, int D>
struct RawSlice {
  static constexpr int kElt = KVT == QT ? 2 : 1;
  static constexpr int kSteps = D / 32;
  static constexpr int kWords = kSteps * 2 * kElt;  // 8 elements per step
  // fp8 keys with an even step count load 16 bytes per lane: steps 2j and 2j + 1 of
  // lane group g take elements [64 j + 16 g, + 16), so one load instruction reads
  // 64 contiguous bytes of each position (8-byte loads read 32)
  static constexpr bool kWide = kElt == 1 && kSteps % 2 == 0;
  static constexpr int kGroupElems = kWide ? 16 : 8;  // elements between lane groups
  uint32_t w[kWords];

  // Element of step s, lane group g, slot e (0..7) in the head vector: the
  // contraction order q must follow too.
  __device__ static constexpr int element(int s, int g) {
    return kWide ? 64 * (s / 2) + 16 * g + 8 * (s % 2) : 32 * s + 8 * g;
  }

  // p: element kGroupElems * g of the position's head vector
  __device__ __forceinline__ void load(const uint8_t* p) {
    if (kWide) {
#pragma unroll
      for (int j = 0; j < kSteps / 2; ++j) {
        const uint4 v = *(const uint4*)(p + j * 64);
        w[4 * j] = v.x; w[4 * j + 1] = v.y; w[4 * j + 2] = v.z; w[4 * j + 3] = v.w;
      }
      return;
    }
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      if (kElt == 2) {
        const uint4 v = *(const uint4*)(p + s * 32 * kElt);
        w[4 * s] = v.x; w[4 * s + 1] = v.y; w[4 * s + 2] = v.z; w[4 * s + 3] = v.w;
      } else {
        const uint2 v = *(const uint2*)(p + s * 32 * kElt);
        w[2 * s] = v.x; w[2 * s + 1] = v.y;
      }
    }
  }
  // The eight elements of step s as MFMA operand bits;
  // zeros when `ok` is false (positions past the sequence may hold any bits).
  __device__ __forceinline__ uint4 op(int s, bool ok) const {
    uint4 r;
    if (KVT == QT) {
      r = make_uint4(w[4 * s], w[4 * s + 1], w[4 * s + 2], w[4 * s + 3]);
    } else {
      const uint2 a = fp8x4_to_16<QT>(w[2 * s]);
      const uint2 b = fp8x4_to_16<QT>(w[2 * s + 1]);
      r = make_uint4(a.x, a.y, b.x, b.y);
    }
    if (!ok) r = make_uint4(0, 0, 0, 0);
    return r;
  }
};

// Four key positions' value slices of one lane for O^T = V^T P^T.  The output
// dimension of accumulator row m of column tile dt is DPL * m + dt (DPL =
// head_dim / 16), so lane (m = lane % 16, group g = lane / 16) needs dims
// [DPL m, DPL m + DPL) of positions 4g .. 4g + 3: one contiguous DPL-element
// load per position, and no transpose through LDS.
template <int QT, int KVT, int D>
struct ValueQuad {
  static constexpr int DPL = D / 16;
  static constexpr bool kFp8 = KVT != QT;
  static constexpr int kBytes = DPL * (kFp8 ? 1 : 2);
  static constexpr bool kHalfWords = kBytes % 4 != 0;  // fp8 with head_dim 96
  static constexpr int kUnits = kHalfWords ? kBytes / 2 : kBytes / 4;
  uint32_t w[4][kUnits];

  __device__ __forceinline__ void load(int i, const uint8_t* p) {
    if (kHalfWords) {
#pragma unroll
      for (int j = 0; j < kUnits; ++j) w[i][j] = ((const uint16_t*)p)[j];
    } else if (kBytes % 16 == 0) {
#pragma unroll
      for (int j = 0; j < kUnits / 4; ++j) {
        const uint4 v = ((const uint4*)p)[j];
        w[i][4 * j] = v.x; w[i][4 * j + 1] = v.y; w[i][4 * j + 2] = v.z; w[i][4 * j + 3] = v.w;
      }
    } else if (kBytes % 8 == 0) {
#pragma unroll
      for (int j = 0; j < kUnits / 2; ++j) {
        const uint2 v = ((const uint2*)p)[j];
        w[i][2 * j] = v.x; w[i][2 * j + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kUnits; ++j) w[i][j] = ((const uint32_t*)p)[j];
    }
  }
  __device__ __forceinline__ void zero(int i) {
#pragma unroll
    for (int j = 0; j < kUnits; ++j) w[i][j] = 0;
  }
  // A operands of the column tiles 2k and 2k + 1: four 16-bit values each, of
  // positions 0..3 at that tile's dimension.
  template <int K>
  __device__ __forceinline__ void op2(uint2& a0, uint2& a1) const {
    if (!kFp8) {
      // element pair k of each position is word k: low half -> tile 2k, high -> 2k + 1
      a0.x = __builtin_amdgcn_perm(w[1][K], w[0][K], 0x05040100u);
      a1.x = __builtin_amdgcn_perm(w[1][K], w[0][K], 0x07060302u);
      a0.y = __builtin_amdgcn_perm(w[3][K], w[2][K], 0x05040100u);
      a1.y = __builtin_amdgcn_perm(w[3][K], w[2][K], 0x07060302u);
    } else {
      float2 f[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (kHalfWords) f[i] = fp8x2_to_f32<false>(w[i][K]);
        else f[i] = (K & 1) ? fp8x2_to_f32<true>(w[i][K / 2]) : fp8x2_to_f32<false>(w[i][K / 2]);
      }
      if (QT == RLT_BF16) {
        // e4m3 values are exact in bf16: the high half of the fp32 bits
        a0.x = __builtin_amdgcn_perm(__float_as_uint(f[1].x), __float_as_uint(f[0].x), 0x07060302u);
        a1.x = __builtin_amdgcn_perm(__float_as_uint(f[1].y), __float_as_uint(f[0].y), 0x07060302u);
        a0.y = __builtin_amdgcn_perm(__float_as_uint(f[3].x), __float_as_uint(f[2].x), 0x07060302u);
        a1.y = __builtin_amdgcn_perm(__float_as_uint(f[3].y), __float_as_uint(f[2].y), 0x07060302u);
      } else {
        a0.x = (uint32_t)f32_to_f16_bits(f[0].x) | ((uint32_t)f32_to_f16_bits(f[1].x) << 16);
        a1.x = (uint32_t)f32_to_f16_bits(f[0].y) | ((uint32_t)f32_to_f16_bits(f[1].y) << 16);
        a0.y = (uint32_t)f32_to_f16_bits(f[2].x) | ((uint32_t)f32_to_f16_bits(f[3].x) << 16);
        a1.y = (uint32_t)f32_to_f16_bits(f[2].y) | ((uint32_t)f32_to_f16_bits(f[3].y) << 16);
      }
    }
  }
};

template <int ND, int NT, class F, int K = 0>
__device__ __forceinline__ void for_pairs(F&& f) {
  if constexpr (K < ND / 2) {
    f(std::integral_constant<int, K>{});
    for_pairs<ND, NT, F, K + 1>(static_cast<F&&>(f));
  }
}

// Row maximum / sum over the four lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48)
// with the gfx950 lane-swap instructions; every lane gets the same bits.
__device__ __forceinline__ float group_max(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Running state of one wave over its part of a unit: the online-softmax
// accumulators of the row-group's rows (one row per 16-row tile and lane) and
// what the partial write needs.
template <int NT, int ND>
struct UnitState {
  f32x4 oacc[NT][ND];
  float m_run[NT], l_run[NT];
  int row_lo[NT], row_hi[NT];
  int rg_begin, rg_rows, q_begin;
  float v_mul;
  bool active;  // the unit has rows and visible positions in this chunk
};

// The verify window's own keys and values of kv head kvh whose positions lie in
// [p0, p1), written into the pool through the sequence's block table.  Row i of the
// sequence sits at position row_len[i] - 1 with explicit row lengths, else at
// kv_len - q_len + i.  Every wave that reads a window position stores it first
// (identical bytes when several do, the quantization being deterministic), so no wave
// depends on another's store.  Positions whose block index lies beyond the table, or
// whose table entry lies outside the pool, are not written.  16-bit pools receive the
// rows as they are, half a wave per row; an fp8-e4m3 pool receives the codes of
// rlt_fp8::encode with the per-tensor scale (SM 1) or with a per-vector scale stored
// into the scale pool (SM 2), bitwise the scatter kernel's quantize-store, one row per
// wave (lanes 0-31 key, 32-63 value).  Returns whether this wave stored anything.
// The stores of window rows [i_lo, i_hi) whose positions lie in [p0, p1), on one wave;
// whether this lane stored anything.
template <int QT, int KVT, int D, int SM>
__device__ __forceinline__ bool store_rows(const AttnParams& P, int seq, int kvh,
                                           const SeqView& sv, int i_lo, int i_hi, int p0, int p1) {
  const int lane = threadIdx.x & 63;
  const int piece = lane & 31;
  const int base_pos = sv.kv_len - sv.q_len;  // position of window row 0 (causal form)
  auto position = [&](int i) { return P.row_len ? P.row_len[sv.q_begin + i] - 1 : base_pos + i; };
  auto block = [&](int pos) {
    const int idx = pos / P.block_size;
    return idx < P.table_width ? P.tables[(int64_t)seq * P.table_stride + idx] : -1;
  };
  bool stored = false;
  if constexpr (KVT == QT) {
    constexpr int kPieces = D * 2 / 16;  // 16-byte pieces of one (row, kv head)
    for (int i = i_lo + (lane >> 5); i < i_hi; i += 2) {
      const int pos = position(i);
      if (pos < p0 || pos >= p1 || pos < 0) continue;
      const int32_t e = block(pos);
      if (piece < kPieces && e >= 0 && e < P.num_blocks) {
        const int64_t row = (int64_t)(sv.q_begin + i) * P.new_row_stride + (int64_t)kvh * P.new_head_stride;
        const int64_t off = (int64_t)(pos % P.block_size);
        const uint4 kx = ((const uint4*)((const uint16_t*)P.new_k + row))[piece];
        const uint4 vx = ((const uint4*)((const uint16_t*)P.new_v + row))[piece];
        ((uint4*)((uint16_t*)P.k + (int64_t)e * P.k_block_stride + off * P.k_token_stride +
                  (int64_t)kvh * P.k_head_stride))[piece] = kx;
        ((uint4*)((uint16_t*)P.v + (int64_t)e * P.v_block_stride + off * P.v_token_stride +
                  (int64_t)kvh * P.v_head_stride))[piece] = vx;
        stored = true;
      }
    }
  } else {
    constexpr int kPieces = D / 8;  // 8-element pieces: 16 bytes of the row, 8 of codes
    const bool is_v = lane >= 32;
    const uint16_t* src = (const uint16_t*)(is_v ? P.new_v : P.new_k);
    uint8_t* pool = (uint8_t*)(is_v ? P.v : P.k);
    const int64_t b_stride = is_v ? P.v_block_stride : P.k_block_stride;
    const int64_t t_stride = is_v ? P.v_token_stride : P.k_token_stride;
    const int64_t h_stride = is_v ? P.v_head_stride : P.k_head_stride;
    float* scales = const_cast<float*>(is_v ? P.v_scale : P.k_scale);
    const float fixed = SM == 1 ? scales[0] : 0.f;
    for (int i = i_lo; i < i_hi; ++i) {  // wave-uniform: the lanes reduce together
      const int pos = position(i);
      if (pos < p0 || pos >= p1 || pos < 0) continue;
      const int32_t e = block(pos);
      if (e < 0 || e >= P.num_blocks) continue;
      float x[8];
      float amax = 0.f;
      if (piece < kPieces) {
        const int64_t row = (int64_t)(sv.q_begin + i) * P.new_row_stride + (int64_t)kvh * P.new_head_stride;
        const uint4 raw = ((const uint4*)(src + row))[piece];
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (QT == RLT_BF16) {
            x[2 * u] = __uint_as_float(w4[u] << 16);
            x[2 * u + 1] = __uint_as_float(w4[u] & 0xffff0000u);
          } else {
            x[2 * u] = f16_bits_to_f32((uint16_t)(w4[u] & 0xffffu));
            x[2 * u + 1] = f16_bits_to_f32((uint16_t)(w4[u] >> 16));
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) amax = rlt_fp8::nan_max(amax, fabsf(x[u]));
      }
      // the row's maximum over the 32 lanes of its half of the wave
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) amax = rlt_fp8::nan_max(amax, __shfl_xor(amax, o, RLT_WAVE));
      const float scale = SM == 2 ? rlt_fp8::dynamic_scale(amax) : fixed;
      const int64_t off = (int64_t)(pos % P.block_size);
      if (piece < kPieces) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          lo |= rlt_fp8::encode(x[u], scale) << (8 * u);
          hi |= rlt_fp8::encode(x[4 + u], scale) << (8 * u);
        }
        *(uint2*)(pool + (int64_t)e * b_stride + off * t_stride + (int64_t)kvh * h_stride + 8 * piece) =
            make_uint2(lo, hi);
      }
      if (SM == 2 && piece == 0)
        scales[(int64_t)e * P.s_block_stride + off * P.s_token_stride + (int64_t)kvh * P.s_head_stride] = scale;
      stored = true;
    }
  }
  return stored;
}

template <int QT, int KVT, int D, int SM>
__device__ __forceinline__ bool store_window(const AttnParams& P, int seq, int kvh,
                                             const SeqView& sv, int p0, int p1) {
  const int base_pos = sv.kv_len - sv.q_len;
  // rows to visit: every row with explicit row lengths (any order), else the range
  // whose positions meet [p0, p1)
  const int i_lo = P.row_len ? 0 : max(0, p0 - base_pos);
  const int i_hi = P.row_len ? sv.q_len : min(sv.q_len, p1 - base_pos);
  return __builtin_amdgcn_ballot_w64(store_rows<QT, KVT, D, SM>(P, seq, kvh, sv, i_lo, i_hi, p0, p1)) != 0;
}

// Part `part` (of KS = unit_split equal spans) of one work unit -- (sequence,
// row-group, kv head, chunk) -- on one wave: the wave streams the kv head over
// positions [512c + part * 512 / KS, + 512 / KS) for every row of the row-group.
// tbl_lds: this wave's 512-entry LDS slice for the chunk's block ids.
// SM: FP8 scale mode (0 none, 1 per-tensor, 2 per-vector).  UB: block_size is a
// multiple of 16, so the 16 positions of a tile share one block.
template <int QT, int KVT, int D, int NT, int SM, bool UB, bool CP>
__device__ __forceinline__ void attend_span(const AttnParams& P, int seq, int rg, int kvh, int chunk,
                                            int part, int32_t* tbl_lds,
                                            UnitState<NT, D / 16>& st) {
  using M = Mfma<QT>;
  using Raw = RawSlice<QT, KVT, D>;
  using VQ = ValueQuad<QT, KVT, D>;
  constexpr int NQS = D / 32;  // 32-wide contraction slices
  constexpr int ND = D / 16;   // 16-wide output column tiles (= dims per lane)
  constexpr int KV_ELT = KVT == QT ? 2 : 1;
  constexpr int CH = unit_chunk<QT, KVT>();
  constexpr int kSpan = CH / unit_split<QT, KVT>();
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15;
  const int grp = lane >> 4;
  const int c_begin = chunk * CH;
  const int w_begin = c_begin + part * kSpan;

  auto& oacc = st.oacc;
  auto& m_run = st.m_run;
  auto& l_run = st.l_run;
  auto& row_lo = st.row_lo;
  auto& row_hi = st.row_hi;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.f;
    row_lo[nt] = row_hi[nt] = 0;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) oacc[nt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  st.active = false;

  // Block ids of the chunk's positions (one per tile when blocks hold whole
  // tiles).  Table indices are clamped into the table and every entry is range
  // checked, so each stored id addresses memory inside the pool.
  for (int i = part * kSpan + (UB ? lane * kTileTok : lane); i < (part + 1) * kSpan;
       i += UB ? 64 * kTileTok : 64) {
    const int idx = min((c_begin + i) / P.block_size, P.table_width - 1);
    const int32_t e = P.tables[(int64_t)seq * P.table_stride + idx];
    tbl_lds[i] = (e >= 0 && e < P.num_blocks) ? e : 0;
  }
  __builtin_amdgcn_wave_barrier();

  SeqView sv = seq_view(P, seq);
  const int rows_total = sv.q_len * P.group;
  const int rg_begin = rg * P.rows_per_rg;
  if (rg_begin >= rows_total) return;
  const int rg_rows = min(P.rows_per_rg, rows_total - rg_begin);
  int lo_first, hi_first, lo_last, hi_last;
  group_range(P, sv, rg_begin, rg_rows, lo_first, hi_first, lo_last, hi_last);
  if (c_begin >= hi_last || c_begin + CH <= lo_first) return;
  st.active = true;
  st.rg_begin = rg_begin;
  st.rg_rows = rg_rows;
  st.q_begin = sv.q_begin;

  // Tiles: absolute 16-aligned positions [w_begin + 16t, +16), t in [t0, t1).
  const int span_lo = max(w_begin, lo_first & ~(kTileTok - 1));
  const int span_hi = min(w_begin + kSpan, hi_last);
  // wave-uniform (scalar) bounds: keeps the tile loop free of divergent branches
  const int t0 = __builtin_amdgcn_readfirstlane(
      span_lo <= w_begin ? 0 : (span_lo - w_begin) / kTileTok);
  const int t1 = __builtin_amdgcn_readfirstlane(
      span_hi <= w_begin ? 0 : (span_hi - w_begin + kTileTok - 1) / kTileTok);

  // This lane's rows (one per 16-row tile): B operand of S^T = K Q^T.
  uint4 qreg[NT][NQS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rho = rg_begin + nt * 16 + l16;
    if (nt * 16 + l16 < rg_rows) {
      const int qi = rho / P.group;
      const int head = kvh * P.group + rho % P.group;
      row_range(P, sv, qi, row_lo[nt], row_hi[nt]);
      const uint16_t* qp = (const uint16_t*)P.q + (int64_t)(sv.q_begin + qi) * P.q_row_stride +
                           (int64_t)head * P.q_head_stride;
#pragma unroll
      for (int s = 0; s < NQS; ++s) qreg[nt][s] = *(const uint4*)(qp + Raw::element(s, grp));
    } else {
      row_lo[nt] = 0;
      row_hi[nt] = 0;
#pragma unroll
      for (int s = 0; s < NQS; ++s) qreg[nt][s] = make_uint4(0, 0, 0, 0);
    }
  }

  float qk_scale = P.qk_scale_log2;
  st.v_mul = 1.f;
  if (SM == 1) {
    qk_scale *= P.k_scale[0];
    st.v_mul = P.v_scale[0];
  }

  if (P.new_k && t0 < t1) {
    // The window rows' own keys and values, stored through the block table before any
    // tile of this span is read; the wait makes this wave's stores visible to its own
    // loads.
    if (store_window<QT, KVT, D, SM>(P, seq, kvh, sv, w_begin + t0 * kTileTok,
                                     w_begin + t1 * kTileTok))
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  if (t0 < t1) {
    Raw kb[kStages];
    VQ vq[kStages];
    float ksc[kStages][4], vsc[kStages][4];
    bool okk[kStages];
    uint32_t okv[kStages];  // bit i: value position 4 * grp + i is inside the sequence
    const int64_t k_head = (int64_t)kvh * P.k_head_stride + grp * Raw::kGroupElems;
    const int64_t v_head = (int64_t)kvh * P.v_head_stride + l16 * ND;
    const int32_t* tbl = tbl_lds - c_begin;  // tbl[pos] for pos in the chunk
    // Loads of tile t into stage b.  Branch-free: every address is inside the
    // pool, and positions outside the sequence are zeroed at use.
    auto issue = [&](int t, int b) {
      const int tb = w_begin + t * kTileTok;
      okk[b] = tb + l16 < hi_last;
      uint32_t m4 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) m4 |= (tb + 4 * grp + i < hi_last) ? (1u << i) : 0u;
      okv[b] = m4;
      if (UB) {
        const int64_t bk = __builtin_amdgcn_readfirstlane(tbl[tb]);
        const int in_blk = tb % P.block_size;
        const uint8_t* kp = (const uint8_t*)P.k +
            (bk * P.k_block_stride + (int64_t)(in_blk + l16) * P.k_token_stride + k_head) * KV_ELT;
        kb[b].load(kp);
        const uint8_t* vbase = (const uint8_t*)P.v + (bk * P.v_block_stride + v_head) * KV_ELT;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          vq[b].load(i, vbase + (int64_t)(in_blk + 4 * grp + i) * P.v_token_stride * KV_ELT);
      } else {
        const int64_t bk = tbl[tb + l16];
        const uint8_t* kp = (const uint8_t*)P.k +
            (bk * P.k_block_stride + (int64_t)((tb + l16) % P.block_size) * P.k_token_stride + k_head) *
                KV_ELT;
        kb[b].load(kp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int pv = tb + 4 * grp + i;
          const int64_t bv = tbl[pv];
          const uint8_t* vp = (const uint8_t*)P.v +
              (bv * P.v_block_stride + (int64_t)(pv % P.block_size) * P.v_token_stride + v_head) * KV_ELT;
          vq[b].load(i, vp);
        }
      }
      if (SM == 2) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p4 = tb + 4 * grp + r;
          // with whole tiles per block only the tile's first entry is stored
          const int64_t so = (int64_t)tbl[UB ? tb : p4] * P.s_block_stride +
                             (int64_t)(p4 % P.block_size) * P.s_token_stride +
                             (int64_t)kvh * P.s_head_stride;
          const bool ok4 = p4 < hi_last;
          ksc[b][r] = ok4 ? P.k_scale[so] : 0.f;
          vsc[b][r] = ok4 ? P.v_scale[so] : 0.f;
        }
      }
    };
    // Wave-uniform fast-path bound: a tile inside [lo of the last row, hi of the
    // first row) is visible to every row of the row-group and fully stored, so
    // it needs no position masks.  Both paths compute identical bits for a row.
    const int full_lo = lo_last;
    const int full_hi = hi_first;
    auto compute = [&](int t, int b, auto full_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
      const int tb = w_begin + t * kTileTok;
      const bool okv_k = FULL ? true : okk[b];
      // ---- S^T = K Q^T : lane holds (positions tb + 4*grp + r, row l16 of tile nt)
      f32x4 sc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) sc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NQS; ++s) {
        const uint4 a = kb[b].op(s, okv_k);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) sc[nt] = M::qk(a, qreg[nt][s], sc[nt]);
      }
      // positions past the sequence may hold any bits (NaN included): zero them
      if (!FULL) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!(okv[b] >> i & 1u)) vq[b].zero(i);
      }
      // ---- online softmax (log2 domain) and the P^T operand
      uint2 pop[NT];
      uint2 plo[CP ? NT : 1];
      bool rescale = false;
      float corr[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float sv4[4];
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = sc[nt][r];
          if (SM == 2) x *= ksc[b][r];
          x *= qk_scale;
          if (!FULL) {
            const int pos = tb + 4 * grp + r;
            x = (pos >= row_lo[nt] && pos < row_hi[nt]) ? x : -INFINITY;
          }
          sv4[r] = x;
          mx = fmaxf(mx, x);
        }
        mx = group_max(mx);
        const float m_new = fmaxf(m_run[nt], mx);
        // a row that has seen no visible key keeps m = -inf and weights 0
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        corr[nt] = m_new == m_run[nt] ? 1.f : __builtin_amdgcn_exp2f(m_run[nt] - m_use);
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f(sv4[r] - m_use);
        rescale |= corr[nt] != 1.f;
        const float rs = group_sum(((pr[0] + pr[1]) + pr[2]) + pr[3]);
        l_run[nt] = l_run[nt] * corr[nt] + rs;
        m_run[nt] = m_new;
        if (SM == 2) {
#pragma unroll
          for (int r = 0; r < 4; ++r) pr[r] *= vsc[b][r];
        }
        pop[nt].x = M::pack2(pr[0], pr[1]);
        pop[nt].y = M::pack2(pr[2], pr[3]);
        if (CP) {
          // what the cast dropped, as a second 16-bit operand (the reference's
          // compensated dot, vllm_rlt/kernels/triton_attention.py:368-371)
          plo[nt].x = M::pack2(pr[0] - M::lo_f32(pop[nt].x), pr[1] - M::hi_f32(pop[nt].x));
          plo[nt].y = M::pack2(pr[2] - M::lo_f32(pop[nt].y), pr[3] - M::hi_f32(pop[nt].y));
        }
      }
      // multiplying by exactly 1 changes no bit: skip the rescale when no row's
      // running max moved in this tile (wave-uniform vote)
      if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int dt = 0; dt < ND; ++dt) oacc[nt][dt] *= corr[nt];
      }
      // ---- O^T += V^T P^T : A = V^T (dims ND * l16 + dt, positions 4grp..+3)
      for_pairs<ND, NT>([&](auto kc) {
        constexpr int K = decltype(kc)::value;
        uint2 a0, a1;
        vq[b].template op2<K>(a0, a1);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          oacc[nt][2 * K] = M::pv(a0, pop[nt], oacc[nt][2 * K]);
          oacc[nt][2 * K + 1] = M::pv(a1, pop[nt], oacc[nt][2 * K + 1]);
          if (CP) {
            oacc[nt][2 * K] = M::pv(a0, plo[nt], oacc[nt][2 * K]);
            oacc[nt][2 * K + 1] = M::pv(a1, plo[nt], oacc[nt][2 * K + 1]);
          }
        }
      });
    };
    auto step = [&](int t, int b) {
      const int tb = w_begin + t * kTileTok;
      const bool full = tb >= full_lo && tb + kTileTok <= full_hi;
      if (full) compute(t, b, Flag<true>{});
      else compute(t, b, Flag<false>{});
    };
    // kStages-deep pipeline: tile t + kStages is issued into the stage tile t just freed.
    // Issues are unconditional -- past the last tile the last tile is re-read (a
    // cache hit) -- so no branch merges pending loads and the wait counts stay exact.
    const int tl = t1 - 1;
#pragma unroll
    for (int b = 0; b < kStages; ++b) issue(min(t0 + b, tl), b);
    for (int t = t0; t < t1; t += kStages) {
#pragma unroll
      for (int b = 0; b < kStages; ++b) {
        if (b == 0 || t + b < t1) step(t + b, b);
        issue(min(t + b + kStages, tl), b);
      }
    }
  }

}

// Chunk partial (max, sum, unnormalized output) of the unit's rows whose merge
// range contains the chunk.
template <int D, int NT, int CH>
__device__ __forceinline__ void write_partial(const AttnParams& P, int kvh, int chunk,
                                              const UnitState<NT, D / 16>& st) {
  constexpr int ND = D / 16;
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15;
  const int grp = lane >> 4;
  const auto& oacc = st.oacc;
  const float v_mul = st.v_mul;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r_local = nt * 16 + l16;
    if (r_local >= st.rg_rows) continue;
    const int lo_c = st.row_lo[nt] / CH;
    const int hi_c = (st.row_hi[nt] + CH - 1) / CH;
    if (chunk < lo_c || chunk >= hi_c) continue;
    const int rho = st.rg_begin + r_local;
    const int qrow = st.q_begin + rho / P.group;
    const int head = kvh * P.group + rho % P.group;
    const int64_t slot = ((int64_t)qrow * P.hq + head) * P.max_chunks + chunk;
    if (grp == 0) {
      P.part_ml[2 * slot] = st.m_run[nt];
      P.part_ml[2 * slot + 1] = st.l_run[nt];
    }
    float* po = P.part_o + slot * D;
    // accumulator element r of column tile dt is dim ND * (4 * grp + r) + dt
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = po + ND * (4 * grp + r);
      if (ND % 4 == 0) {
#pragma unroll
        for (int d4 = 0; d4 < ND; d4 += 4)
          *(float4*)(dst + d4) = make_float4(oacc[nt][d4][r] * v_mul, oacc[nt][d4 + 1][r] * v_mul,
                                             oacc[nt][d4 + 2][r] * v_mul, oacc[nt][d4 + 3][r] * v_mul);
      } else {
#pragma unroll
        for (int d2 = 0; d2 < ND; d2 += 2)
          *(float2*)(dst + d2) = make_float2(oacc[nt][d2][r] * v_mul, oacc[nt][d2 + 1][r] * v_mul);
      }
    }
  }
}

// LDS hand-over of a part's state to the wave that owns the unit.
template <int NT, int ND>
struct PartBuffer {
  f32x4 o[NT * ND][64];
  float ml[NT * 16][2];
};

template <int NT, int ND>
__device__ __forceinline__ void publish_part(const UnitState<NT, ND>& st, PartBuffer<NT, ND>& buf) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if (lane < 16) {
      buf.ml[nt * 16 + lane][0] = st.m_run[nt];
      buf.ml[nt * 16 + lane][1] = st.l_run[nt];
    }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) buf.o[nt * ND + dt][lane] = st.oacc[nt][dt];
  }
}

// st = st (+) buffer, in that operand order.
template <int NT, int ND>
__device__ __forceinline__ void absorb_part(UnitState<NT, ND>& st, const PartBuffer<NT, ND>& buf) {
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float m2 = buf.ml[nt * 16 + l16][0];
    const float l2 = buf.ml[nt * 16 + l16][1];
    float mo, s1, s2;
    merge_scales(st.m_run[nt], m2, mo, s1, s2);
    st.m_run[nt] = mo;
    st.l_run[nt] = st.l_run[nt] * s1 + l2 * s2;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) st.oacc[nt][dt] = st.oacc[nt][dt] * s1 + buf.o[nt * ND + dt][lane] * s2;
  }
}

// Active chunk range [c0, c1) of (sequence, row-group) pair p: the chunks that
// hold a position some row of the row-group sees.
template <int CH>
__device__ __forceinline__ void pair_chunks(const AttnParams& P, int p, int& c0, int& c1) {
  const int seq = p / P.rowgroups;
  const int rg = p - seq * P.rowgroups;
  const SeqView sv = seq_view(P, seq);
  const int rows_total = sv.q_len * P.group;
  const int rg_begin = rg * P.rows_per_rg;
  c0 = c1 = 0;
  if (rg_begin >= rows_total) return;
  const int rg_rows = min(P.rows_per_rg, rows_total - rg_begin);
  int lo_first, hi_first, lo_last, hi_last;
  group_range(P, sv, rg_begin, rg_rows, lo_first, hi_first, lo_last, hi_last);
  if (hi_last <= lo_first) return;
  c0 = lo_first / CH;
  c1 = (hi_last + CH - 1) / CH;
}

constexpr int kPersistWaves = 8;     // waves of a persistent workgroup (one per CU)
constexpr int kMaxPairs = 8192;      // (sequence, row-group) pairs the persistent kernel indexes

// KS: waves per unit; the workgroup runs kPersistWaves / KS units at a time; CH: chunk
template <int NT, int ND, int KS, int CH>
struct PersistShared {
  static constexpr int kSlots = kPersistWaves / KS;
  int32_t first[kMaxPairs + 1];  // units before pair p (prefix sum)
  int32_t c0[kMaxPairs];         // first active chunk of pair p
  int32_t tbl[kPersistWaves][CH];
  PartBuffer<NT, ND> part[KS > 1 ? kSlots : 1][KS > 1 ? KS / 2 : 1];
  int32_t wave_total[kPersistWaves];
};

// Unit u of the persistent list -> (sequence, row-group, kv head, chunk).
__device__ __forceinline__ void unit_of(const AttnParams& P, const int32_t* first, const int32_t* c0s,
                                        int pairs, int u, int& seq, int& rg, int& kvh, int& chunk) {
  // pair of unit u: the last p with first[p] <= u
  int lo = 0, hi = pairs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (first[mid] <= u) lo = mid;
    else hi = mid - 1;
  }
  const int j = u - first[lo];
  seq = lo / P.rowgroups;
  rg = lo - seq * P.rowgroups;
  // the kv head is rotated by the chunk so that every XCD (workgroup b runs on
  // XCD b % 8, and so takes units u = b mod 8) serves every kv head
  const int cj = j / P.hkv;
  kvh = (j - cj * P.hkv + cj) % P.hkv;
  chunk = c0s[lo] + cj;
}

// Persistent MFMA attention: one 8-wave workgroup per CU.  Every workgroup lists
// the active units -- (pair, chunk, kv head) -- from the sequence lengths, and
// workgroup b takes units b, b + G, b + 2G, ... (G = workgroups), so every CU
// gets the same number of units whatever the mix of sequence lengths (a grid of
// one workgroup per unit leaves the placement of the busy workgroups to the
// dispatcher, and CUs end up with 1 to 8 of them).  kSlots units run at a time,
// each on KS waves that split its positions and combine through LDS in a
// fixed order, so a unit's arithmetic never depends on the assignment.
template <int QT, int KVT, int D, int NT, int SM, bool UB, bool CP>
__global__ __launch_bounds__(64 * kPersistWaves) void rlt_attn_mfma_kernel(AttnParams P) {
  constexpr int ND = D / 16;
  constexpr int KS = unit_split<QT, KVT>();
  constexpr int CH = unit_chunk<QT, KVT>();
  constexpr int kSlots = kPersistWaves / KS;
  __shared__ PersistShared<NT, ND, KS, CH> sh;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int slot = wave / KS;
  const int part = wave - slot * KS;
  const int pairs = P.num_seqs * P.rowgroups;
  // units per pair, summed per thread over a contiguous run of pairs
  const int per = (pairs + 64 * kPersistWaves - 1) / (64 * kPersistWaves);
  const int p_lo = t * per;
  const int p_hi = min(pairs, p_lo + per);
  int run = 0;
  for (int p = p_lo; p < p_hi; ++p) {
    int c0, c1;
    pair_chunks<CH>(P, p, c0, c1);
    sh.c0[p] = c0;
    sh.first[p] = run;  // local prefix for now
    run += (c1 - c0) * P.hkv;
  }
  // exclusive scan of the thread totals: wave scans, then wave offsets
  int incl = run;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, RLT_WAVE);
    if (lane >= off) incl += y;
  }
  if (lane == 63) sh.wave_total[wave] = incl;
  __syncthreads();
  int base = incl - run;
  for (int w = 0; w < wave; ++w) base += sh.wave_total[w];
  for (int p = p_lo; p < p_hi; ++p) sh.first[p] += base;
  if (t == 64 * kPersistWaves - 1) sh.first[pairs] = base + run;
  __syncthreads();
  const int units = sh.first[pairs];
  const int G = gridDim.x;
  const int mine = (int)blockIdx.x < units ? (units - (int)blockIdx.x + G - 1) / G : 0;
  const int rounds = (mine + kSlots - 1) / kSlots;  // the same in every wave
  for (int r = 0; r < rounds; ++r) {
    const int k = slot + kSlots * r;  // this slot's unit: the k-th of the workgroup
    const int u = (int)blockIdx.x + G * k;
    UnitState<NT, ND> st;
    int seq = 0, rg = 0, kvh = 0, chunk = 0;
    if (k < mine) {
      unit_of(P, sh.first, sh.c0, pairs, u, seq, rg, kvh, chunk);
      attend_span<QT, KVT, D, NT, SM, UB, CP>(P, seq, rg, kvh, chunk, part, sh.tbl[wave], st);
    } else {
      st.active = false;
    }
    // tree combine of the unit's parts: part p absorbs part p + h, h = KS/2 .. 1
#pragma unroll
    for (int h = KS / 2; h >= 1; h /= 2) {
      if (part >= h && part < 2 * h && st.active) publish_part(st, sh.part[slot][part - h]);
      __syncthreads();
      if (part < h && st.active) absorb_part(st, sh.part[slot][part]);
      __syncthreads();  // the buffers are reused by the next level / round
    }
    if (part == 0 && st.active) write_partial<D, NT, CH>(P, kvh, chunk, st);
  }
}

// Fallback for batches with more than kMaxPairs pairs: one KS-wave workgroup
// per (sequence, row-group, kv head, chunk), the same per-unit arithmetic.
template <int QT, int KVT, int D, int NT, int SM, bool UB, bool CP>
__global__ __launch_bounds__((64 * unit_split<QT, KVT>())) void rlt_attn_mfma_grid_kernel(AttnParams P) {
  constexpr int ND = D / 16;
  constexpr int KS = unit_split<QT, KVT>();
  constexpr int CH = unit_chunk<QT, KVT>();
  __shared__ int32_t tbl[KS][CH];
  __shared__ PartBuffer<NT, ND> buf[KS > 1 ? KS / 2 : 1];
  const int part = threadIdx.x >> 6;
  const WorkItem wi = work_item(P, blockIdx.x);
  UnitState<NT, ND> st;
  attend_span<QT, KVT, D, NT, SM, UB, CP>(P, wi.seq, wi.rg, wi.hg, wi.chunk, part, tbl[part], st);
#pragma unroll
  for (int h = KS / 2; h >= 1; h /= 2) {
    if (part >= h && part < 2 * h && st.active) publish_part(st, buf[part - h]);
    __syncthreads();
    if (part < h && st.active) absorb_part(st, buf[part]);
    __syncthreads();
  }
  if (part == 0 && st.active) write_partial<D, NT, CH>(P, wi.hg, wi.chunk, st);
}

// ============================================================ vector path

constexpr int kVecRows = 8;  // rows per row-group on the vector path

struct VecShared {
  float q[kVecRows][256];
  float p[kWaves][kVecRows][kTileTok];
  float ml[2][kVecRows][2];
  float o[2][kVecRows][256];
};

// Scores: lane (position l16, dim quarter grp) dots its quarter with every row's
// q (LDS broadcast) and reduces across quarters.  P * V: lane owns dims
// lane + 64e and reads the tile's 16 value vectors straight from memory.
template <int QT, int KVT>
__global__ __launch_bounds__(256) void rlt_attn_vec_kernel(AttnParams P) {
  __shared__ VecShared sh;
  const int D = P.head_dim;
  const int DQ = (D + 3) / 4;
  const WorkItem wi = work_item(P, blockIdx.x);
  const int seq = wi.seq;
  const int rg = wi.rg;
  const int kvh = wi.hg;  // one kv head per workgroup on this path
  const int chunk = wi.chunk;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15;
  const int grp = lane >> 4;

  const SeqView sv = seq_view(P, seq);
  const int rows_total = sv.q_len * P.group;
  const int rg_begin = rg * kVecRows;
  if (rg_begin >= rows_total) return;
  const int rg_rows = min(kVecRows, rows_total - rg_begin);
  int lo_first, hi_first, lo_last, hi_last;
  group_range(P, sv, rg_begin, rg_rows, lo_first, hi_first, lo_last, hi_last);
  const int c_begin = chunk * kChunk;
  if (c_begin >= hi_last || c_begin + kChunk <= lo_first) return;

  int rlo[kVecRows], rhi[kVecRows];
#pragma unroll
  for (int r = 0; r < kVecRows; ++r) {
    if (r < rg_rows) row_range(P, sv, (rg_begin + r) / P.group, rlo[r], rhi[r]);
    else rlo[r] = rhi[r] = 0;
  }
  for (int idx = threadIdx.x; idx < kVecRows * D; idx += blockDim.x) {
    const int r = idx / D, d = idx % D;
    float x = 0.f;
    if (r < rg_rows) {
      const int rho = rg_begin + r;
      const int head = kvh * P.group + rho % P.group;
      x = load_as_f32<QT>(P.q, (int64_t)(sv.q_begin + rho / P.group) * P.q_row_stride +
                                   (int64_t)head * P.q_head_stride + d);
    }
    sh.q[r][d] = x;
  }
  __syncthreads();

  float qk_scale = P.qk_scale_log2;
  float v_mul = 1.f;
  if (P.scale_mode == 1) {
    qk_scale *= P.k_scale[0];
    v_mul = P.v_scale[0];
  }
  float m_run[kVecRows], l_run[kVecRows], acc[kVecRows][4];
#pragma unroll
  for (int r = 0; r < kVecRows; ++r) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[r][e] = 0.f;
  }
  const int w_begin = c_begin + wave * kWaveSpan;
  const int span_lo = max(w_begin, lo_first & ~(kTileTok - 1));
  const int span_hi = min(w_begin + kWaveSpan, hi_last);
  const int t0 = span_lo <= w_begin ? 0 : (span_lo - w_begin) / kTileTok;
  const int t1 = span_hi <= w_begin ? 0 : (span_hi - w_begin + kTileTok - 1) / kTileTok;
  for (int t = t0; t < t1; ++t) {
    const int tb = w_begin + t * kTileTok;
    const int pos = tb + l16;
    const bool ok = pos < hi_last;
    int64_t kb = 0;
    float ksc = 1.f;
    if (ok) {
      kb = kv_token_base(P, seq, pos, P.k_block_stride, P.k_token_stride) + (int64_t)kvh * P.k_head_stride;
      if (P.scale_mode == 2) ksc = scale_at(P, P.k_scale, seq, pos, kvh);
    }
    float s_row[kVecRows];
#pragma unroll
    for (int r = 0; r < kVecRows; ++r) s_row[r] = 0.f;
    for (int e = 0; e < DQ; ++e) {
      const int d = grp * DQ + e;
      if (d < D) {
        const float kx = ok ? load_as_f32<KVT>(P.k, kb + d) * ksc : 0.f;
#pragma unroll
        for (int r = 0; r < kVecRows; ++r) s_row[r] = fmaf(kx, sh.q[r][d], s_row[r]);
      }
    }
    float corr[kVecRows];
#pragma unroll
    for (int r = 0; r < kVecRows; ++r) {
      float s = s_row[r];
      s += __shfl_xor(s, 16, RLT_WAVE);
      s += __shfl_xor(s, 32, RLT_WAVE);
      const bool vis = pos >= rlo[r] && pos < rhi[r];
      s = vis ? s * qk_scale : -INFINITY;
      float mx = s;
      for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, RLT_WAVE));
      const float m_new = fmaxf(m_run[r], mx);
      float pr = 0.f;
      corr[r] = 1.f;
      if (m_new != -INFINITY) {
        corr[r] = exp2f(m_run[r] - m_new);
        pr = exp2f(s - m_new);
      }
      float rs = pr;
      for (int off = 1; off < 16; off <<= 1) rs += __shfl_xor(rs, off, RLT_WAVE);
      l_run[r] = l_run[r] * corr[r] + rs;
      m_run[r] = m_new;
      if (grp == 0) sh.p[wave][r][l16] = pr;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < kVecRows; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[r][e] *= corr[r];
    // P * V over the tile's 16 positions; lane owns dims lane + 64e.
    for (int j = 0; j < kTileTok; ++j) {
      const int pj = tb + j;
      if (pj >= hi_last) break;
      const int64_t vb =
          kv_token_base(P, seq, pj, P.v_block_stride, P.v_token_stride) + (int64_t)kvh * P.v_head_stride;
      const float vsc = P.scale_mode == 2 ? scale_at(P, P.v_scale, seq, pj, kvh) : 1.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) {
          const float vx = load_as_f32<KVT>(P.v, vb + d) * vsc;
#pragma unroll
          for (int r = 0; r < kVecRows; ++r) acc[r][e] = fmaf(sh.p[wave][r][j], vx, acc[r][e]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  auto publish = [&](int buf) {
    if (lane < kVecRows) {
      float mv = 0.f, lv = 0.f;
#pragma unroll
      for (int r = 0; r < kVecRows; ++r)
        if (r == lane) { mv = m_run[r]; lv = l_run[r]; }
      sh.ml[buf][lane][0] = mv;
      sh.ml[buf][lane][1] = lv;
    }
#pragma unroll
    for (int r = 0; r < kVecRows; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) sh.o[buf][r][d] = acc[r][e];
      }
  };
  auto absorb = [&](int buf) {
#pragma unroll
    for (int r = 0; r < kVecRows; ++r) {
      float mo, s1, s2;
      merge_scales(m_run[r], sh.ml[buf][r][0], mo, s1, s2);
      m_run[r] = mo;
      l_run[r] = l_run[r] * s1 + sh.ml[buf][r][1] * s2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) acc[r][e] = acc[r][e] * s1 + sh.o[buf][r][d] * s2;
      }
    }
  };
  __syncthreads();
  if (wave >= 2) publish(wave - 2);
  __syncthreads();
  if (wave < 2) absorb(wave);
  __syncthreads();
  if (wave == 1) publish(0);
  __syncthreads();
  if (wave != 0) return;
  absorb(0);
#pragma unroll
  for (int r = 0; r < kVecRows; ++r) {
    if (r >= rg_rows) continue;
    const int lo_c = rlo[r] / kChunk;
    const int hi_c = (rhi[r] + kChunk - 1) / kChunk;
    if (chunk < lo_c || chunk >= hi_c) continue;
    const int rho = rg_begin + r;
    const int qrow = sv.q_begin + rho / P.group;
    const int head = kvh * P.group + rho % P.group;
    const int64_t slot = ((int64_t)qrow * P.hq + head) * P.max_chunks + chunk;
    if (lane == 0) {
      P.part_ml[2 * slot] = m_run[r];
      P.part_ml[2 * slot + 1] = l_run[r];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = lane + 64 * e;
      if (d < D) P.part_o[slot * D + d] = acc[r][e] * v_mul;
    }
  }
}

// ============================================================ merge

// grid (sequences x max_q, ceil(hq / 4)), 256 threads: one wave per (row, head).
// Combines the row's chunks: the (max, sum) of up to kMergeBatch chunks and
// their head-dim values are loaded together (one memory round trip), the scale
// exp2(m_c - M) of chunk c comes from lane c, and every lane accumulates its dims
// over the chunks in chunk order.  The order depends only on the row's own chunk
// range.  reference: triton_attention.py:145-173 (empty rows give zeros; 1e-30
// floor).
constexpr int kMergeBatch = 16;

// Lane c's value of x in every lane (c wave-uniform).
__device__ __forceinline__ float lane_value(float x, int c) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), c));
}

// E: head dims per lane (ceil(head_dim / 64)).
template <int OT, int E>
__global__ __launch_bounds__(256) void rlt_merge_kernel(AttnParams P) {
  const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (head >= P.hq) return;
  int seq, qi;
  if (P.cu_q) {
    seq = blockIdx.x / P.max_q;
    qi = blockIdx.x % P.max_q;
  } else {
    seq = blockIdx.x;
    qi = 0;
  }
  const SeqView sv = seq_view(P, seq);
  if (qi >= sv.q_len) return;
  const int row = sv.q_begin + qi;
  int lo, hi;
  row_range(P, sv, qi, lo, hi);
  const int c0 = lo >> P.chunk_log2, c1 = (hi + (1 << P.chunk_log2) - 1) >> P.chunk_log2;
  const int nc = c1 - c0;
  const int64_t base = ((int64_t)row * P.hq + head) * P.max_chunks + c0;
  const int64_t out_off = (int64_t)row * P.out_row_stride + (int64_t)head * P.out_head_stride;
  const int D = P.head_dim;
  if (nc <= 0) {
    for (int d = lane; d < D; d += 64) store_from_f32<OT>(P.out, out_off + d, 0.f);
    return;
  }
  if (nc <= kMergeBatch) {
    // statistics (lane c) and values (every lane, dims lane + 64e) of all chunks
    float m = -INFINITY, l = 0.f;
    if (lane < nc) {
      m = P.part_ml[2 * (base + lane)];
      l = P.part_ml[2 * (base + lane) + 1];
    }
    float v[kMergeBatch][E];
#pragma unroll
    for (int c = 0; c < kMergeBatch; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int d = lane + 64 * e;
        v[c][e] = (c < nc && d < D) ? P.part_o[(base + c) * D + d] : 0.f;
      }
    float mmax = -INFINITY;
    for (int c = 0; c < nc; ++c) mmax = fmaxf(mmax, lane_value(m, c));
    const float sc = (lane < nc && m != -INFINITY) ? exp2f(m - mmax) : 0.f;
    float lsum = 0.f;
    const float ls = l * sc;
    for (int c = 0; c < nc; ++c) lsum += lane_value(ls, c);
    const float inv_den = 1.f / fmaxf(lsum, 1.0e-30f);
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.f;
    // chunks past nc have scale 0 and values 0: adding them changes nothing
#pragma unroll
    for (int c = 0; c < kMergeBatch; ++c) {
      const float sv = lane_value(sc, c);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] += v[c][e] * sv;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = lane + 64 * e;
      if (d < D) store_from_f32<OT>(P.out, out_off + d, acc[e] * inv_den);
    }
    return;
  }
  // long rows: chunk statistics 64 at a time, then values chunk by chunk
  float mmax = -INFINITY;
  for (int c = lane; c < nc; c += 64) mmax = fmaxf(mmax, P.part_ml[2 * (base + c)]);
  for (int off = 32; off >= 1; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off, RLT_WAVE));
  float l = 0.f;
  for (int c0p = 0; c0p < nc; c0p += 64) {
    const int c = c0p + lane;
    float part = 0.f;
    if (c < nc) {
      const float m = P.part_ml[2 * (base + c)];
      const float s = m == -INFINITY ? 0.f : exp2f(m - mmax);
      part = P.part_ml[2 * (base + c) + 1] * s;
    }
    for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, RLT_WAVE);
    l += part;
  }
  const float inv_den = 1.f / fmaxf(l, 1.0e-30f);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int c0p = 0; c0p < nc; c0p += 64) {
    const int cn = min(64, nc - c0p);
    float my_s = 0.f;
    if (lane < cn) {
      const float m = P.part_ml[2 * (base + c0p + lane)];
      my_s = m == -INFINITY ? 0.f : exp2f(m - mmax);
    }
    int c = 0;
    for (; c + 4 <= cn; c += 4) {  // four chunks of loads in flight
      float v[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = lane + 64 * e;
          v[u][e] = d < D ? P.part_o[(base + c0p + c + u) * D + d] : 0.f;
        }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float s = __shfl(my_s, c + u, RLT_WAVE);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += v[u][e] * s;
      }
    }
    for (; c < cn; ++c) {
      const float s = __shfl(my_s, c, RLT_WAVE);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) acc[e] += P.part_o[(base + c0p + c) * D + d] * s;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = lane + 64 * e;
    if (d < D) store_from_f32<OT>(P.out, out_off + d, acc[e] * inv_den);
  }
}

// ============================================================ long-prompt prefill
//
// Calls whose longest q window reaches kPfMinQ rows (prompt prefill, long chunks)
// take a tiling built for many rows per sequence: one 256-thread workgroup per
// (sequence, 128-row group, kv head), each wave owning 32 rows (two 16-row MFMA
// tiles).  64-position K and V tiles are staged once per workgroup in LDS (K as
// [position][dim], V transposed to [dim][position] while it is stored) and shared
// by the four waves, double-buffered with the next tile's global loads in
// registers.  The math is the verify kernel's (S^T = K Q^T, online softmax in the
// log2 domain, O^T = V^T P^T), with both products on v_mfma_f32_16x16x32: the
// P^T operand of a key-tile pair is the two S^T accumulators of the lane, and the
// contraction order over the pair's 32 positions is permuted to match.  The
// output is normalized in the kernel (no split, no merge launch).  Rows of such a
// call are equal to the per-row form within floating-point tolerance, not bit for
// bit (the tile boundaries differ).
constexpr int kPfNT = 2;        // 16-row MFMA tiles per wave
constexpr int kPfWaves = 4;     // waves per workgroup (sharing each staged tile)
constexpr int kPfRows = kPfWaves * 16 * kPfNT;  // q rows per workgroup
constexpr int kPfKeys = 64;     // key positions per LDS tile
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfMinQ = 64;     // q window length from which a call takes this path
constexpr float kPfLazy = 8.f;  // log2 headroom before the running max moves

// LDS row width in dims: D = 96 rows take a 128-dim row whose last four 16-byte slots
// (their place moves with the swizzle) are never loaded nor read
template <int D>
constexpr int pf_row_dims() { return D == 96 ? 128 : D; }

template <int D>
struct PrefillLds {
  static constexpr int kRowB = pf_row_dims<D>() * 2;  // bytes per position row (XOR-swizzled slots)
  uint8_t k[2][kPfKeys * kRowB];
  uint8_t v[2][kPfKeys * kRowB];
  float ks[2][kPfKeys];  // per-vector fp8 scales of the tile's positions (SM 2)
  float vs[2][kPfKeys];
};

typedef __attribute__((address_space(3))) void lds_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));

// 16-byte slot of piece `piece` (8 dims) in row r of a staged tile.  K rows XOR the
// slot with r mod SLOTS, so the S^T operand reads (16 lanes = 16 rows of one piece
// column) meet distinct bank groups; V rows XOR it with 2 (r & 3), which keeps each piece
// pair adjacent for the transpose reads (16 lanes = 4 rows x one 32-byte pair) and puts
// the four rows on distinct bank groups, and with 8 in rows with bit 2 set (16 slots), so
// the next 16 lanes (rows 4 further on) use the other half of the banks.
template <int SLOTS>
__device__ __forceinline__ int k_slot(int r, int piece) { return piece ^ (r & (SLOTS - 1)); }
template <int SLOTS>
__device__ __forceinline__ int v_slot(int r, int piece) {
  return piece ^ (2 * (r & 3)) ^ (SLOTS >= 16 ? 8 * ((r >> 2) & 1) : 0);
}

// UB: block_size % 16 == 0, so each 16-position group of a tile lies in one block
// and its address comes from one wave-uniform table lookup (16-bit pools).
// KVT: the pool type, QT's own or fp8-e4m3 with scale mode SM (1 per-tensor, 2
// per-vector).  FP8 tiles are staged through registers: each thread loads 8-code pieces
// (item e = 256 j + t: LDS slot e % SLOTS of row e / SLOTS, holding the piece the
// swizzle puts there) while the previous tile is in use, then widens them to QT (exact
// for e4m3) into the same swizzled LDS layout, each wave writing contiguous slots; the
// per-tensor key scale folds into the score scale and the value scale into the output,
// per-vector scales multiply each position's score and (for P V only) its weight.
template <int QT, int KVT, int D, int SM, bool UB>
__global__ __launch_bounds__(kPfThreads, kPfNT > 2 || kPfWaves > 4 ? 1 : 2) void rlt_prefill_kernel(AttnParams P) {
  using M = Mfma<QT>;
  using L = PrefillLds<D>;
  constexpr int NT = kPfNT;
  constexpr int NQS = D / 32;       // 32-wide contraction slices of S^T
  constexpr int ND = D / 16;        // 16-wide dim tiles of O^T
  constexpr int PIECES = D / 8;     // 16-byte pieces of a position row in the pool
  constexpr int SLOTS = pf_row_dims<D>() / 8;  // 16-byte slots per LDS row (>= PIECES)
  constexpr int ROWS_PER_LD = 64 / SLOTS;                // rows one wave-wide direct load fills
  constexpr int LDS_PER_WAVE = kPfKeys / ROWS_PER_LD / kPfWaves;  // direct loads per wave per tile (K, V each)
  static_assert(LDS_PER_WAVE * ROWS_PER_LD * kPfWaves == kPfKeys, "the waves' loads cover a tile");
  static_assert(16 % ROWS_PER_LD == 0, "a direct load's rows stay in one 16-position group");
  constexpr bool FP8 = KVT != QT;
  static_assert(!FP8 || KVT == RLT_FP8_E4M3, "16-bit pools match q");
  static_assert(FP8 == (SM != 0), "scale modes are for fp8 pools");
  constexpr int FJ = kPfKeys * SLOTS / kPfThreads;  // fp8 LDS slots per thread per tile (K, V each)
  static_assert(FJ * kPfThreads == kPfKeys * SLOTS, "the threads' fp8 slots cover a tile");
  __shared__ L sh;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, l16 = lane & 15, grp = lane >> 4;

  // heaviest row-groups (latest positions) first across the whole batch: the
  // row-group index is outermost, then the sequence, then the kv head
  const int64_t id = blockIdx.x;
  const int kvh = (int)(id % P.hkv);
  const int64_t sr = id / P.hkv;
  const int seq = (int)(sr % P.num_seqs);
  const int rg = P.rowgroups - 1 - (int)(sr / P.num_seqs);
  const SeqView sv = seq_view(P, seq);
  const int rows_total = sv.q_len * P.group;
  const int rg_begin = rg * kPfRows;
  if (rg_begin >= rows_total) return;  // uniform over the workgroup
  const int rg_rows = min(kPfRows, rows_total - rg_begin);
  int lo_first, hi_first, lo_last, hi_last;
  group_range(P, sv, rg_begin, rg_rows, lo_first, hi_first, lo_last, hi_last);

  // this lane's rows (one per 16-row tile): B operand of S^T = K Q^T
  uint4 qreg[NT][NQS];
  int row_lo[NT], row_hi[NT];
  // the wave's common visible range: tiles inside [wlo, whi) need no position masks
  // (rows past the group are not stored and do not narrow it)
  int wlo = -(1 << 30), whi = 1 << 30;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int local = w * 16 * NT + nt * 16 + l16;
    if (local < rg_rows) {
      const int rho = rg_begin + local;
      const int qi = rho / P.group;
      const int head = kvh * P.group + rho % P.group;
      row_range(P, sv, qi, row_lo[nt], row_hi[nt]);
      wlo = max(wlo, row_lo[nt]);
      whi = min(whi, row_hi[nt]);
      const uint16_t* qp = (const uint16_t*)P.q + (int64_t)(sv.q_begin + qi) * P.q_row_stride +
                           (int64_t)head * P.q_head_stride + grp * 8;
#pragma unroll
      for (int s = 0; s < NQS; ++s) qreg[nt][s] = *(const uint4*)(qp + 32 * s);
    } else {
      row_lo[nt] = row_hi[nt] = 0;
#pragma unroll
      for (int s = 0; s < NQS; ++s) qreg[nt][s] = make_uint4(0, 0, 0, 0);
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    wlo = max(wlo, __shfl_xor(wlo, off, RLT_WAVE));
    whi = min(whi, __shfl_xor(whi, off, RLT_WAVE));
  }
  wlo = __builtin_amdgcn_readfirstlane(wlo);
  whi = __builtin_amdgcn_readfirstlane(whi);

  f32x4 oacc[NT][ND];
  float m_run[NT], l_run[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) oacc[nt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- global -> LDS staging of one 64-position tile by direct loads: wave w's j-th
  // load fills rows ROWS_PER_LD (LDS_PER_WAVE w + j) + [0, ROWS_PER_LD); lane L takes row
  // + L / SLOTS and LDS slot L % SLOTS, into which it loads the row's swizzled piece
  const int ld_row = lane / SLOTS;
  const int ld_slot = lane % SLOTS;
  const int64_t k_head = (int64_t)kvh * P.k_head_stride;
  const int64_t v_head = (int64_t)kvh * P.v_head_stride;
  // (block id, offset) of position pos: block ids outside the pool read block 0
  auto block_of = [&](int pos, int64_t& blk, int& off) {
    const int idx = min(pos / P.block_size, P.table_width - 1);
    const int32_t e = P.tables[(int64_t)seq * P.table_stride + idx];
    blk = (e >= 0 && e < P.num_blocks) ? e : 0;
    off = pos % P.block_size;
  };
  uint2 kraw[FP8 ? FJ : 1], vraw[FP8 ? FJ : 1];
  float sraw = 0.f;
  auto load = [&](int tile, int b) {
    const int base = tile * kPfKeys;
    if constexpr (FP8) {
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        // item e: LDS slot e % SLOTS of row e / SLOTS, so each wave's LDS writes are
        // contiguous (scattered 16-byte writes of permuted slots conflicted); the slot
        // holds the row's piece k_slot / v_slot (an involution), loaded here
        const int e = j * kPfThreads + t;
        const int r = e / SLOTS, sl = e % SLOTS;
        const int kpc = k_slot<SLOTS>(r, sl), vpc = v_slot<SLOTS>(r, sl);
        int64_t blk;
        int off;
        block_of(base + r, blk, off);
        if (PIECES == SLOTS || kpc < PIECES)
          kraw[j] = *(const uint2*)((const uint8_t*)P.k + blk * P.k_block_stride +
                                    (int64_t)off * P.k_token_stride + k_head + kpc * 8);
        if (PIECES == SLOTS || vpc < PIECES)
          vraw[j] = *(const uint2*)((const uint8_t*)P.v + blk * P.v_block_stride +
                                    (int64_t)off * P.v_token_stride + v_head + vpc * 8);
      }
      if (SM == 2 && t < 2 * kPfKeys) {  // threads 0-63 key scales, 64-127 value scales
        const int pos = base + (t & (kPfKeys - 1));
        int64_t blk;
        int off;
        block_of(pos, blk, off);
        const float x = (t < kPfKeys ? P.k_scale : P.v_scale)[blk * P.s_block_stride +
                                                              (int64_t)off * P.s_token_stride +
                                                              (int64_t)kvh * P.s_head_stride];
        sraw = pos < hi_last ? x : 0.f;
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < LDS_PER_WAVE; ++j) {
      const int r0 = ROWS_PER_LD * (LDS_PER_WAVE * w + j);  // wave-uniform
      const int r = r0 + ld_row;
      int64_t blk;
      int off;
      if (UB) {
        block_of(__builtin_amdgcn_readfirstlane(base + (r0 & ~15)), blk, off);
        off += r & 15;
      } else {
        block_of(base + r, blk, off);
      }
      // (the slot of lane ld_slot holds piece k_slot / v_slot of row r: an involution)
      const int kpc = k_slot<SLOTS>(r, ld_slot);
      const int vpc = v_slot<SLOTS>(r, ld_slot);
      const uint16_t* kp = (const uint16_t*)P.k + blk * P.k_block_stride +
                           (int64_t)off * P.k_token_stride + k_head + kpc * 8;
      const uint16_t* vp = (const uint16_t*)P.v + blk * P.v_block_stride +
                           (int64_t)off * P.v_token_stride + v_head + vpc * 8;
      // padded rows: lanes whose slot holds a piece past the row load nothing
      if (PIECES == SLOTS || kpc < PIECES)
        __builtin_amdgcn_global_load_lds((const void*)kp, (lds_void*)(sh.k[b] + r0 * L::kRowB), 16, 0, 0);
      if (PIECES == SLOTS || vpc < PIECES)
        __builtin_amdgcn_global_load_lds((const void*)vp, (lds_void*)(sh.v[b] + r0 * L::kRowB), 16, 0, 0);
    }
  };
  // After this wave's loads of tile `tile` into buffer b landed: its V rows past the
  // sequence may hold any bits (NaN included) and are zeroed, since their weight 0
  // times NaN would not vanish.  Only the tiles that reach past hi_last do work.
  auto settle = [&](int tile, int b) {
    const int base = tile * kPfKeys;
    if constexpr (FP8) {
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const int e = j * kPfThreads + t;
        const int r = e / SLOTS, sl = e % SLOTS;
        // (pad slots of 96-dim rows are never read: left unwritten)
        if (PIECES == SLOTS || k_slot<SLOTS>(r, sl) < PIECES) {
          const uint2 k0 = fp8x4_to_16<QT>(kraw[j].x), k1 = fp8x4_to_16<QT>(kraw[j].y);
          // two 8-byte halves: 16-byte LDS writes of a whole wave conflicted (the counters
          // read 4x the cycles of an ideal write)
          uint2* kd = (uint2*)(sh.k[b] + r * L::kRowB + sl * 16);
          kd[0] = make_uint2(k0.x, k0.y);
          kd[1] = make_uint2(k1.x, k1.y);
        }
        if (PIECES == SLOTS || v_slot<SLOTS>(r, sl) < PIECES) {
          uint4 vx = make_uint4(0, 0, 0, 0);
          if (base + r < hi_last) {
            const uint2 v0 = fp8x4_to_16<QT>(vraw[j].x), v1 = fp8x4_to_16<QT>(vraw[j].y);
            vx = make_uint4(v0.x, v0.y, v1.x, v1.y);
          }
          uint2* vd = (uint2*)(sh.v[b] + r * L::kRowB + sl * 16);
          vd[0] = make_uint2(vx.x, vx.y);
          vd[1] = make_uint2(vx.z, vx.w);
        }
      }
      if (SM == 2 && t < 2 * kPfKeys) (t < kPfKeys ? sh.ks[b] : sh.vs[b])[t & (kPfKeys - 1)] = sraw;
      return;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (base + kPfKeys > hi_last) {
#pragma unroll
      for (int j = 0; j < LDS_PER_WAVE; ++j) {
        const int r = ROWS_PER_LD * (LDS_PER_WAVE * w + j) + ld_row;
        if (base + r >= hi_last)
          *(uint4*)(sh.v[b] + r * L::kRowB + ld_slot * 16) = make_uint4(0, 0, 0, 0);
      }
    }
  };

  // S^T operand reads: row kt 16 + l16, piece 4 s + grp at slot (4 s + grp) ^ (l16 mod SLOTS)
  const int k_lane = l16 * L::kRowB;
  // V^T operand reads (transpose loads): lane (l16, grp) of the 16-lane group grp reads
  // row 32 c + 4 grp + (l16 >> 2) (+16 for the second half) at dims 16 dt + 4 (l16 & 3),
  // piece 2 dt + ((l16 >> 1) & 1) -> slot 2 (dt ^ m) + ((l16 >> 1) & 1), m = (l16 >> 2) & 3
  // (^ 4 for odd grp when rows have 16 slots: the slot's bit-3 flip)
  const int vm = ((l16 >> 2) & 3) ^ (SLOTS >= 16 ? 4 * (grp & 1) : 0);
  const int v_lane = (4 * grp + (l16 >> 2)) * L::kRowB + ((l16 >> 1) & 1) * 16 + (l16 & 1) * 8;

  float qk_scale = P.qk_scale_log2;
  float v_mul = 1.f;
  if (SM == 1) {
    qk_scale *= P.k_scale[0];
    v_mul = P.v_scale[0];
  }
  auto compute = [&](int tile, int b, auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    const int base = tile * kPfKeys;
    const uint8_t* kb = sh.k[b];
    const uint8_t* vb = sh.v[b];
    // per-vector scales of the lane's positions 16 kt + 4 grp + i
    f32x4 ksv[SM == 2 ? 4 : 1], vsv[SM == 2 ? 4 : 1];
    if constexpr (SM == 2) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        ksv[kt] = *(const f32x4*)(sh.ks[b] + 16 * kt + 4 * grp);
        vsv[kt] = *(const f32x4*)(sh.vs[b] + 16 * kt + 4 * grp);
      }
    }
    // ---- S^T = K Q^T for the tile's four 16-position sub-tiles
    f32x4 sc[4][NT];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) sc[kt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NQS; ++s)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const uint4 a = *(const uint4*)(kb + kt * 16 * L::kRowB + k_lane +
                                        (((4 * s + grp) ^ (l16 & (SLOTS - 1))) * 16));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) sc[kt][nt] = M::qk(a, qreg[nt][s], sc[kt][nt]);
      }
    // ---- online softmax (log2 domain); lane holds positions base + 16 kt + 4 grp + i.
    // The running max m moves only when a tile's max exceeds it by more than kPfLazy
    // (weights stay below 2^kPfLazy), so the accumulators are rarely rescaled; the
    // scale enters as one fma per score (qk_scale > 0: the max of raw scores scales).
    uint4 pop[2][NT];
    bool rescale = false;
    float corr[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float x[4][4];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = sc[kt][nt][i];
          if constexpr (SM == 2) v *= ksv[kt][i];
          if (FULL) {
            x[kt][i] = v;
          } else {
            const int pos = base + kt * 16 + 4 * grp + i;
            x[kt][i] = (pos >= row_lo[nt] && pos < row_hi[nt]) ? v : -INFINITY;
          }
          mx = fmaxf(mx, x[kt][i]);
        }
      const float mxs = group_max(mx) * qk_scale;
      const bool grow = mxs > m_run[nt] + kPfLazy;
      const float m_new = grow ? mxs : m_run[nt];
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      corr[nt] = grow ? __builtin_amdgcn_exp2f(m_run[nt] - m_use) : 1.f;
      rescale |= grow;
      float rs = 0.f;
      float pr[4][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[kt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[kt][i], qk_scale, -m_use));
          rs += pr[kt][i];
        }
      l_run[nt] = l_run[nt] * corr[nt] + group_sum(rs);
      m_run[nt] = m_new;
      if constexpr (SM == 2) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) pr[kt][i] *= vsv[kt][i];
      }
#pragma unroll
      for (int c = 0; c < 2; ++c)
        pop[c][nt] = make_uint4(M::pack2(pr[2 * c][0], pr[2 * c][1]),
                                M::pack2(pr[2 * c][2], pr[2 * c][3]),
                                M::pack2(pr[2 * c + 1][0], pr[2 * c + 1][1]),
                                M::pack2(pr[2 * c + 1][2], pr[2 * c + 1][3]));
    }
    if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) oacc[nt][dt] *= corr[nt];
    }
    // ---- O^T += V^T P^T over the sub-tile pairs (2c, 2c + 1): contraction slot
    // 8 grp + j is position 16 (2c) + 4 grp + j for j < 4, else 16 (2c + 1) + 4 grp + j - 4
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const uint8_t* vr = vb + 32 * c * L::kRowB + v_lane + 32 * (dt ^ vm);
        const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(lds_void*)vr);
        const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(lds_void*)(vr + 16 * L::kRowB));
        uint4 a;
        __builtin_memcpy(&a, &x0, 8);
        __builtin_memcpy((char*)&a + 8, &x1, 8);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) oacc[nt][dt] = M::qk(a, pop[c][nt], oacc[nt][dt]);
      }
  };

  const int kt0 = lo_first / kPfKeys;
  const int kt1 = (hi_last + kPfKeys - 1) / kPfKeys;
  if (kt0 < kt1) {
    auto step = [&](int tile, auto full_tag) {
      const int b = (tile - kt0) & 1;
      const bool more = tile + 1 < kt1;
      // buffer b ^ 1 was last read in the previous iteration, before its barrier
      if (more) load(tile + 1, b ^ 1);
      compute(tile, b, full_tag);
      if (more) settle(tile + 1, b ^ 1);
      __syncthreads();
    };
    // tiles [fa, fb) lie inside every row's visible range: three loops, so that no
    // branch between the two compute forms sits inside one (its join would copy the
    // accumulators)
    const int fa = min(kt1, max(kt0, (max(wlo, 0) + kPfKeys - 1) / kPfKeys));
    const int fb = max(fa, min(kt1, whi / kPfKeys));
    load(kt0, 0);
    settle(kt0, 0);
    __syncthreads();
    for (int tile = kt0; tile < fa; ++tile) step(tile, Flag<false>{});
    for (int tile = fa; tile < fb; ++tile) step(tile, Flag<true>{});
    for (int tile = fb; tile < kt1; ++tile) step(tile, Flag<false>{});
  }

  // ---- normalized output: lane holds dims 16 dt + 4 grp + i of its rows
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int local = w * 16 * NT + nt * 16 + l16;
    if (local >= rg_rows) continue;
    const int rho = rg_begin + local;
    const int qi = rho / P.group;
    const int head = kvh * P.group + rho % P.group;
    const int64_t off = (int64_t)(sv.q_begin + qi) * P.out_row_stride + (int64_t)head * P.out_head_stride;
    const float inv = v_mul / fmaxf(l_run[nt], 1.0e-30f);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) store_from_f32<QT>(P.out, off + dt * 16 + 4 * grp + i, oacc[nt][dt][i] * inv);
  }
}

// Window store ahead of the prefill tiling (a store-and-attend call whose window takes
// it): one 256-thread workgroup per (64 window rows, sequence, kv head), 16 rows per
// wave, the verify kernels' fused per-row stores (store_rows).
template <int QT, int KVT, int D, int SM>
__global__ __launch_bounds__(256) void rlt_window_store_kernel(AttnParams P) {
  const int64_t id = blockIdx.x;
  const int kvh = (int)(id % P.hkv);
  const int64_t sr = id / P.hkv;
  const int seq = (int)(sr % P.num_seqs);
  const int i0 = (int)(sr / P.num_seqs) * 64 + (int)(threadIdx.x >> 6) * 16;
  const SeqView sv = seq_view(P, seq);
  if (i0 >= sv.q_len) return;  // wave-uniform; no barriers follow
  store_rows<QT, KVT, D, SM>(P, seq, kvh, sv, i0, min(sv.q_len, i0 + 16), 0, INT_MAX);
}

// ============================================================ dispatch

template <int QT, int KVT, int D, int SM, bool UB, bool CP, int NT>
void launch_mfma_nt(const AttnParams& P, dim3 grid, hipStream_t stream) {
  if (P.persistent)
    rlt_attn_mfma_kernel<QT, KVT, D, NT, SM, UB, CP><<<grid, 64 * kPersistWaves, 0, stream>>>(P);
  else
    rlt_attn_mfma_grid_kernel<QT, KVT, D, NT, SM, UB, CP><<<grid, 64 * unit_split<QT, KVT>(), 0, stream>>>(P);
}

template <int QT, int KVT, int D, int SM, bool UB, bool CP>
int launch_mfma_ub(const AttnParams& P, dim3 grid, int nt, hipStream_t stream) {
  if (nt == 1) launch_mfma_nt<QT, KVT, D, SM, UB, CP, 1>(P, grid, stream);
  else if (D <= 128) launch_mfma_nt<QT, KVT, D, SM, UB, CP, (D <= 128 ? 2 : 1)>(P, grid, stream);
  else return RLT_ERR_UNSUPPORTED;
  return RLT_OK;
}

// Compensated P V is built for blocks holding whole 16-position tiles (the reference
// pools' block size 16 and its multiples).
template <int QT, int KVT, int D, int SM>
int launch_mfma_sm(const AttnParams& P, dim3 grid, int nt, hipStream_t stream) {
  const bool ub = P.block_size % kTileTok == 0;
  if (P.compensate) {
    if (!ub) return RLT_ERR_UNSUPPORTED;
    return launch_mfma_ub<QT, KVT, D, SM, true, true>(P, grid, nt, stream);
  }
  if (ub) return launch_mfma_ub<QT, KVT, D, SM, true, false>(P, grid, nt, stream);
  return launch_mfma_ub<QT, KVT, D, SM, false, false>(P, grid, nt, stream);
}

template <int QT, int KVT, int D>
int launch_mfma_d(const AttnParams& P, dim3 grid, int nt, hipStream_t stream) {
  // 16-bit pools are read unscaled (scale_mode applies to fp8 pools only)
  if constexpr (KVT == QT) {
    return launch_mfma_sm<QT, KVT, D, 0>(P, grid, nt, stream);
  } else {
    if (P.scale_mode == 1) return launch_mfma_sm<QT, KVT, D, 1>(P, grid, nt, stream);
    return launch_mfma_sm<QT, KVT, D, 2>(P, grid, nt, stream);
  }
}

template <int QT, int KVT>
int launch_mfma(const AttnParams& P, dim3 grid, int nt, hipStream_t stream) {
  switch (P.head_dim) {
    case 64: return launch_mfma_d<QT, KVT, 64>(P, grid, nt, stream);
    case 96: return launch_mfma_d<QT, KVT, 96>(P, grid, nt, stream);
    case 128: return launch_mfma_d<QT, KVT, 128>(P, grid, nt, stream);
    case 256: return launch_mfma_d<QT, KVT, 256>(P, grid, nt, stream);
    default: return RLT_ERR_UNSUPPORTED;
  }
}

bool mfma_head_dim(int d) { return d == 64 || d == 96 || d == 128 || d == 256; }

template <int QT>
int launch_vec_q(const AttnParams& P, int kv_dtype, dim3 grid, hipStream_t stream) {
  switch (kv_dtype) {
    case RLT_F32: rlt_attn_vec_kernel<QT, RLT_F32><<<grid, 256, 0, stream>>>(P); break;
    case RLT_F16: rlt_attn_vec_kernel<QT, RLT_F16><<<grid, 256, 0, stream>>>(P); break;
    case RLT_BF16: rlt_attn_vec_kernel<QT, RLT_BF16><<<grid, 256, 0, stream>>>(P); break;
    case RLT_FP8_E4M3: rlt_attn_vec_kernel<QT, RLT_FP8_E4M3><<<grid, 256, 0, stream>>>(P); break;
    default: return RLT_ERR_ARGUMENT;
  }
  return RLT_OK;
}

template <int QT, int KVT, int D, int SM>
void launch_prefill_sm(const AttnParams& P, dim3 grid, dim3 sgrid, hipStream_t stream) {
  if (P.new_k) rlt_window_store_kernel<QT, KVT, D, SM><<<sgrid, 256, 0, stream>>>(P);
  // (fp8 pools are staged per position: the whole-tile block form is for direct loads)
  if constexpr (KVT == QT) {
    if (P.block_size % 16 == 0) {
      rlt_prefill_kernel<QT, KVT, D, SM, true><<<grid, kPfThreads, 0, stream>>>(P);
      return;
    }
  }
  rlt_prefill_kernel<QT, KVT, D, SM, false><<<grid, kPfThreads, 0, stream>>>(P);
}

template <int QT, int KVT, int D>
void launch_prefill_d(const AttnParams& P, dim3 grid, dim3 sgrid, hipStream_t stream) {
  if constexpr (KVT == QT) launch_prefill_sm<QT, KVT, D, 0>(P, grid, sgrid, stream);
  else if (P.scale_mode == 1) launch_prefill_sm<QT, KVT, D, 1>(P, grid, sgrid, stream);
  else launch_prefill_sm<QT, KVT, D, 2>(P, grid, sgrid, stream);
}

// sgrid: the window store's grid (launched first when the call stores its rows)
template <int QT, int KVT>
void launch_prefill(const AttnParams& P, int head_dim, dim3 grid, dim3 sgrid, hipStream_t stream) {
  if (head_dim == 64) launch_prefill_d<QT, KVT, 64>(P, grid, sgrid, stream);
  else if (head_dim == 96) launch_prefill_d<QT, KVT, 96>(P, grid, sgrid, stream);
  else launch_prefill_d<QT, KVT, 128>(P, grid, sgrid, stream);
}

template <int OT>
void launch_merge(const AttnParams& P, dim3 grid, hipStream_t stream) {
  switch ((P.head_dim + 63) / 64) {
    case 1: rlt_merge_kernel<OT, 1><<<grid, 256, 0, stream>>>(P); break;
    case 2: rlt_merge_kernel<OT, 2><<<grid, 256, 0, stream>>>(P); break;
    case 3: rlt_merge_kernel<OT, 3><<<grid, 256, 0, stream>>>(P); break;
    default: rlt_merge_kernel<OT, 4><<<grid, 256, 0, stream>>>(P); break;
  }
}

// Compute units of the current device (cached per device).
int compute_units() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev < 64) cached[dev] = n;
  return n;
}

int max_chunks_for(int32_t table_width, int32_t block_size, int chunk = kChunk) {
  const int64_t tokens = (int64_t)table_width * block_size;
  return (int)((tokens + chunk - 1) / chunk);
}

}  // namespace

extern "C" {

int rlt_abi_version(void) { return RLT_MI355X_ABI_VERSION; }

int rlt_paged_attention_uses_mfma(int32_t q_dtype, int32_t kv_dtype, int32_t head_dim) {
  const bool qok = q_dtype == RLT_BF16 || q_dtype == RLT_F16;
  const bool kvok = kv_dtype == q_dtype || kv_dtype == RLT_FP8_E4M3;
  return qok && kvok && mfma_head_dim(head_dim);
}

int rlt_paged_attention_uses_prefill(int32_t q_dtype, int32_t kv_dtype, int32_t head_dim,
                                     int32_t max_q_len) {
  return rlt_paged_attention_uses_mfma(q_dtype, kv_dtype, head_dim) &&
         (head_dim == 64 || head_dim == 96 || head_dim == 128) && max_q_len >= kPfMinQ;
}

size_t rlt_paged_attention_workspace_size(int32_t num_q_rows, int32_t num_q_heads, int32_t head_dim,
                                          int32_t table_width, int32_t block_size) {
  const int64_t slots = (int64_t)num_q_rows * num_q_heads * max_chunks_for(table_width, block_size);
  return rlt_align_up(sizeof(float) * slots * 2, 256) + rlt_align_up(sizeof(float) * slots * head_dim, 256);
}

}  // extern "C"

namespace {

struct WindowStore {
  const void* k;
  const void* v;
  int64_t row_stride, head_stride;
};

int attention_impl(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                             const void* key_cache, const void* value_cache, int64_t k_block_stride,
                             int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                             int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
                             const int32_t* block_tables, int64_t table_stride, int32_t table_width,
                             const int32_t* context_lengths, const int32_t* row_lengths,
                             const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t max_q_len,
                             int32_t num_q_rows, const float* key_scale, const float* value_scale,
                             int32_t scale_mode, int64_t s_block_stride, int64_t s_token_stride,
                             int64_t s_head_stride, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t block_size, int32_t q_dtype, int32_t kv_dtype,
                             int32_t window, int32_t flags, void* out, int64_t out_row_stride,
                             int64_t out_head_stride, void* workspace, size_t workspace_bytes,
                             hipStream_t stream, const WindowStore* store) {
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return RLT_ERR_ARGUMENT;
  if (head_dim <= 0 || head_dim > 256 || block_size <= 0 || window < 0) return RLT_ERR_ARGUMENT;
  if (num_seqs < 0 || num_q_rows < 0 || max_q_len < 0 || table_width < 0) return RLT_ERR_ARGUMENT;
  if (scale_mode < 0 || scale_mode > 2 || (scale_mode && (!key_scale || !value_scale)))
    return RLT_ERR_ARGUMENT;
  if (kv_dtype == RLT_FP8_E4M3 && scale_mode == 0) return RLT_ERR_ARGUMENT;
  if (q_dtype == RLT_FP8_E4M3) return RLT_ERR_ARGUMENT;
  if (flags & ~RLT_ATTN_COMPENSATE) return RLT_ERR_ARGUMENT;
  if (num_blocks <= 0) return RLT_ERR_ARGUMENT;
  if (num_q_rows == 0 || num_seqs == 0) return RLT_OK;
  if (!cu_seqlens_q && num_seqs != num_q_rows) return RLT_ERR_ARGUMENT;
  if (cu_seqlens_q && max_q_len <= 0) return RLT_ERR_ARGUMENT;
  if (row_lengths && !cu_seqlens_q) return RLT_ERR_ARGUMENT;
  const size_t need = rlt_paged_attention_workspace_size(num_q_rows, num_q_heads, head_dim,
                                                         table_width, block_size);
  if (!workspace || workspace_bytes < need) return RLT_ERR_WORKSPACE;

  AttnParams P;
  P.q = q;
  P.q_row_stride = q_row_stride;
  P.q_head_stride = q_head_stride;
  P.k = key_cache;
  P.v = value_cache;
  P.k_block_stride = k_block_stride;
  P.k_token_stride = k_token_stride;
  P.k_head_stride = k_head_stride;
  P.v_block_stride = v_block_stride;
  P.v_token_stride = v_token_stride;
  P.v_head_stride = v_head_stride;
  P.tables = block_tables;
  P.table_stride = table_stride;
  P.table_width = table_width;
  P.num_blocks = num_blocks;
  P.lengths = context_lengths;
  P.cu_q = cu_seqlens_q;
  P.row_len = row_lengths;
  P.k_scale = key_scale;
  P.v_scale = value_scale;
  P.s_block_stride = s_block_stride;
  P.s_token_stride = s_token_stride;
  P.s_head_stride = s_head_stride;
  P.scale_mode = scale_mode;
  P.compensate = (flags & RLT_ATTN_COMPENSATE) ? 1 : 0;
  P.num_seqs = num_seqs;
  P.num_rows = num_q_rows;
  P.hq = num_q_heads;
  P.hkv = num_kv_heads;
  P.group = num_q_heads / num_kv_heads;
  P.head_dim = head_dim;
  P.block_size = block_size;
  P.window = window;
  // chunk size: 1024 for fp8 KV on the MFMA path (unit_chunk), 512 otherwise; the
  // workspace query sizes the partials for 512, an upper bound
  const bool fp8_mfma = kv_dtype == RLT_FP8_E4M3 && rlt_paged_attention_uses_mfma(q_dtype, kv_dtype, head_dim);
  P.chunk_log2 = fp8_mfma ? 10 : 9;
  P.max_chunks = max_chunks_for(table_width, block_size, 1 << P.chunk_log2);
  P.qk_scale_log2 = kLog2e / sqrtf((float)head_dim);
  P.out = out;
  P.out_row_stride = out_row_stride;
  P.out_head_stride = out_head_stride;
  const int64_t slots = (int64_t)num_q_rows * num_q_heads * P.max_chunks;
  P.part_ml = (float*)workspace;
  P.part_o = (float*)((char*)workspace + rlt_align_up(sizeof(float) * slots * 2, 256));
  if (P.max_chunks == 0) P.max_chunks = 1;  // zero-width tables: every row is empty
  P.new_k = store ? store->k : nullptr;
  P.new_v = store ? store->v : nullptr;
  P.new_row_stride = store ? store->row_stride : 0;
  P.new_head_stride = store ? store->head_stride : 0;
  if (store) {
    // the fused window store, on the verify kernels only: 16-bit pools (no scales), or
    // fp8 pools with per-tensor or per-vector scales; the rows are bf16 / fp16 like q
    const bool fp8 = kv_dtype == RLT_FP8_E4M3;
    if (!cu_seqlens_q || (q_dtype != RLT_BF16 && q_dtype != RLT_F16) ||
        !(kv_dtype == q_dtype || fp8) ||
        !rlt_paged_attention_uses_mfma(q_dtype, kv_dtype, head_dim))
      return RLT_ERR_UNSUPPORTED;
    if (fp8 != (scale_mode != 0)) return RLT_ERR_ARGUMENT;
    const int64_t piece = fp8 ? 8 : 16;  // bytes each lane stores into the pool
    const int64_t elt = fp8 ? 1 : 2;
    if (!store->k || !store->v || ((uintptr_t)store->k | (uintptr_t)store->v) % 16 ||
        (store->row_stride * 2) % 16 || (store->head_stride * 2) % 16 ||
        (k_token_stride * elt) % piece || (v_token_stride * elt) % piece ||
        (k_head_stride * elt) % piece || (v_head_stride * elt) % piece ||
        (k_block_stride * elt) % piece || (v_block_stride * elt) % piece)
      return RLT_ERR_ARGUMENT;
  }

  const int rows_per_seq = max_q_len * P.group;
  const bool mfma = rlt_paged_attention_uses_mfma(q_dtype, kv_dtype, head_dim);
  int st = RLT_OK;
  if (mfma) {
    // 16-byte vector loads of q and of every lane's KV slice.
    const int64_t kv_elt = kv_dtype == RLT_FP8_E4M3 ? 1 : 2;
    // (fp8 keys with head_dim % 64 == 0 are read 16 bytes per lane: RawSlice::kWide)
    const int64_t kv_align = kv_dtype == RLT_FP8_E4M3 && head_dim % 64 != 0 ? 8 : 16;
    const bool aligned =
        ((uintptr_t)q % 16 == 0) && (q_row_stride * 2) % 16 == 0 && (q_head_stride * 2) % 16 == 0 &&
        ((uintptr_t)key_cache % 16 == 0) && ((uintptr_t)value_cache % 16 == 0) &&
        (k_block_stride * kv_elt) % kv_align == 0 && (k_token_stride * kv_elt) % kv_align == 0 &&
        (k_head_stride * kv_elt) % kv_align == 0 && (v_block_stride * kv_elt) % kv_align == 0 &&
        (v_token_stride * kv_elt) % kv_align == 0 && (v_head_stride * kv_elt) % kv_align == 0;
    if (!aligned) return RLT_ERR_ARGUMENT;
    // (compensated calls stay on the verify kernels at every q_len)
    if (cu_seqlens_q && !row_lengths && !P.compensate &&
        rlt_paged_attention_uses_prefill(q_dtype, kv_dtype, head_dim, max_q_len)) {
      // long q windows: the prefill tiling, normalized in one launch
      P.rows_per_rg = kPfRows;
      P.rowgroups = (rows_per_seq + kPfRows - 1) / kPfRows;
      const int64_t wgs = (int64_t)num_seqs * P.rowgroups * num_kv_heads;
      if (wgs >= ((int64_t)1 << 31)) return RLT_ERR_UNSUPPORTED;
      const dim3 grid((unsigned)wgs);
      const int64_t swgs = (int64_t)num_seqs * num_kv_heads * ((max_q_len + 63) / 64);
      if (swgs >= ((int64_t)1 << 31)) return RLT_ERR_UNSUPPORTED;
      const dim3 sgrid((unsigned)swgs);
      const bool fp8 = kv_dtype == RLT_FP8_E4M3;
      if (q_dtype == RLT_BF16) {
        if (fp8) launch_prefill<RLT_BF16, RLT_FP8_E4M3>(P, head_dim, grid, sgrid, stream);
        else launch_prefill<RLT_BF16, RLT_BF16>(P, head_dim, grid, sgrid, stream);
      } else {
        if (fp8) launch_prefill<RLT_F16, RLT_FP8_E4M3>(P, head_dim, grid, sgrid, stream);
        else launch_prefill<RLT_F16, RLT_F16>(P, head_dim, grid, sgrid, stream);
      }
      return rlt_launch_status();
    }
    const int nt = (rows_per_seq > 16 && head_dim <= 128) ? 2 : 1;
    P.rows_per_rg = 16 * nt;
    P.rowgroups = (rows_per_seq + P.rows_per_rg - 1) / P.rows_per_rg;
    if (P.rowgroups < 1) P.rowgroups = 1;
    // Persistent workgroups, one per CU, unless the pair index does not fit in LDS.
    P.head_groups = num_kv_heads;
    const int64_t pairs = (int64_t)num_seqs * P.rowgroups;
    P.persistent = pairs <= kMaxPairs;
    int64_t wgs = (int64_t)num_seqs * P.rowgroups * num_kv_heads * P.max_chunks;
    if (P.persistent) wgs = compute_units();
    if (wgs >= ((int64_t)1 << 31)) return RLT_ERR_UNSUPPORTED;
    dim3 grid((unsigned)wgs);
    if (q_dtype == RLT_BF16)
      st = kv_dtype == RLT_BF16 ? launch_mfma<RLT_BF16, RLT_BF16>(P, grid, nt, stream)
                                : launch_mfma<RLT_BF16, RLT_FP8_E4M3>(P, grid, nt, stream);
    else
      st = kv_dtype == RLT_F16 ? launch_mfma<RLT_F16, RLT_F16>(P, grid, nt, stream)
                               : launch_mfma<RLT_F16, RLT_FP8_E4M3>(P, grid, nt, stream);
  } else {
    P.rows_per_rg = kVecRows;
    P.rowgroups = (rows_per_seq + kVecRows - 1) / kVecRows;
    if (P.rowgroups < 1) P.rowgroups = 1;
    P.head_groups = num_kv_heads;
    P.persistent = 0;
    const int64_t wgs = (int64_t)num_seqs * P.rowgroups * P.head_groups * P.max_chunks;
    if (wgs >= ((int64_t)1 << 31)) return RLT_ERR_UNSUPPORTED;
    dim3 grid((unsigned)wgs);
    switch (q_dtype) {
      case RLT_F32: st = launch_vec_q<RLT_F32>(P, kv_dtype, grid, stream); break;
      case RLT_F16: st = launch_vec_q<RLT_F16>(P, kv_dtype, grid, stream); break;
      case RLT_BF16: st = launch_vec_q<RLT_BF16>(P, kv_dtype, grid, stream); break;
      default: st = RLT_ERR_ARGUMENT;
    }
  }
  if (st != RLT_OK) return st;
  P.max_q = cu_seqlens_q ? max_q_len : 1;
  const int64_t merge_rows = cu_seqlens_q ? (int64_t)num_seqs * max_q_len : num_q_rows;
  if (merge_rows >= ((int64_t)1 << 31)) return RLT_ERR_UNSUPPORTED;
  dim3 mgrid((unsigned)merge_rows, (unsigned)((num_q_heads + 3) / 4));
  switch (q_dtype) {
    case RLT_F32: launch_merge<RLT_F32>(P, mgrid, stream); break;
    case RLT_F16: launch_merge<RLT_F16>(P, mgrid, stream); break;
    case RLT_BF16: launch_merge<RLT_BF16>(P, mgrid, stream); break;
  }
  return rlt_launch_status();
}

}  // namespace

extern "C" {

int rlt_paged_attention_rows(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                             const void* key_cache, const void* value_cache, int64_t k_block_stride,
                             int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                             int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
                             const int32_t* block_tables, int64_t table_stride, int32_t table_width,
                             const int32_t* context_lengths, const int32_t* row_lengths,
                             const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t max_q_len,
                             int32_t num_q_rows, const float* key_scale, const float* value_scale,
                             int32_t scale_mode, int64_t s_block_stride, int64_t s_token_stride,
                             int64_t s_head_stride, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t block_size, int32_t q_dtype, int32_t kv_dtype,
                             int32_t window, int32_t flags, void* out, int64_t out_row_stride,
                             int64_t out_head_stride, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  return attention_impl(q, q_row_stride, q_head_stride, key_cache, value_cache, k_block_stride,
                        k_token_stride, k_head_stride, v_block_stride, v_token_stride,
                        v_head_stride, num_blocks, block_tables, table_stride, table_width,
                        context_lengths, row_lengths, cu_seqlens_q, num_seqs, max_q_len,
                        num_q_rows, key_scale, value_scale, scale_mode, s_block_stride,
                        s_token_stride, s_head_stride, num_q_heads, num_kv_heads, head_dim,
                        block_size, q_dtype, kv_dtype, window, flags, out, out_row_stride,
                        out_head_stride, workspace, workspace_bytes, stream, nullptr);
}

int rlt_paged_attention_store(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                              void* key_cache, void* value_cache, int64_t k_block_stride,
                              int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                              int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
                              const int32_t* block_tables, int64_t table_stride,
                              int32_t table_width, const int32_t* context_lengths,
                              const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t max_q_len,
                              int32_t num_q_rows, int32_t num_q_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t block_size, int32_t dtype,
                              const void* new_k, const void* new_v, int64_t new_row_stride,
                              int64_t new_head_stride, void* out, int64_t out_row_stride,
                              int64_t out_head_stride, void* workspace, size_t workspace_bytes,
                              hipStream_t stream) {
  const WindowStore st{new_k, new_v, new_row_stride, new_head_stride};
  return attention_impl(q, q_row_stride, q_head_stride, key_cache, value_cache, k_block_stride,
                        k_token_stride, k_head_stride, v_block_stride, v_token_stride,
                        v_head_stride, num_blocks, block_tables, table_stride, table_width,
                        context_lengths, nullptr, cu_seqlens_q, num_seqs, max_q_len, num_q_rows,
                        nullptr, nullptr, 0, 0, 0, 0, num_q_heads, num_kv_heads, head_dim,
                        block_size, dtype, dtype, 0, 0, out, out_row_stride, out_head_stride,
                        workspace, workspace_bytes, stream, &st);
}

int rlt_paged_attention_store_scaled(
    const void* q, int64_t q_row_stride, int64_t q_head_stride, void* key_cache,
    void* value_cache, int64_t k_block_stride, int64_t k_token_stride, int64_t k_head_stride,
    int64_t v_block_stride, int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
    const int32_t* block_tables, int64_t table_stride, int32_t table_width,
    const int32_t* context_lengths, const int32_t* row_lengths, const int32_t* cu_seqlens_q,
    int32_t num_seqs, int32_t max_q_len, int32_t num_q_rows, float* key_scale, float* value_scale,
    int32_t scale_mode, int64_t s_block_stride, int64_t s_token_stride, int64_t s_head_stride,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int32_t q_dtype, int32_t kv_dtype, int32_t flags, const void* new_k, const void* new_v,
    int64_t new_row_stride, int64_t new_head_stride, void* out, int64_t out_row_stride,
    int64_t out_head_stride, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const WindowStore st{new_k, new_v, new_row_stride, new_head_stride};
  return attention_impl(q, q_row_stride, q_head_stride, key_cache, value_cache, k_block_stride,
                        k_token_stride, k_head_stride, v_block_stride, v_token_stride,
                        v_head_stride, num_blocks, block_tables, table_stride, table_width,
                        context_lengths, row_lengths, cu_seqlens_q, num_seqs, max_q_len,
                        num_q_rows, key_scale, value_scale, scale_mode, s_block_stride,
                        s_token_stride, s_head_stride, num_q_heads, num_kv_heads, head_dim,
                        block_size, q_dtype, kv_dtype, 0, flags, out, out_row_stride,
                        out_head_stride, workspace, workspace_bytes, stream, &st);
}

int rlt_paged_attention(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                        const void* key_cache, const void* value_cache, int64_t k_block_stride,
                        int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                        int64_t v_token_stride, int64_t v_head_stride, int32_t num_blocks,
                        const int32_t* block_tables, int64_t table_stride, int32_t table_width,
                        const int32_t* context_lengths,
                        const int32_t* cu_seqlens_q, int32_t num_seqs, int32_t max_q_len,
                        int32_t num_q_rows, const float* key_scale, const float* value_scale,
                        int32_t scale_mode, int64_t s_block_stride, int64_t s_token_stride,
                        int64_t s_head_stride, int32_t num_q_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t block_size, int32_t q_dtype, int32_t kv_dtype,
                        int32_t window, void* out, int64_t out_row_stride, int64_t out_head_stride,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return rlt_paged_attention_rows(
      q, q_row_stride, q_head_stride, key_cache, value_cache, k_block_stride, k_token_stride,
      k_head_stride, v_block_stride, v_token_stride, v_head_stride, num_blocks, block_tables,
      table_stride, table_width, context_lengths, nullptr, cu_seqlens_q, num_seqs, max_q_len,
      num_q_rows, key_scale, value_scale, scale_mode, s_block_stride, s_token_stride,
      s_head_stride, num_q_heads, num_kv_heads, head_dim, block_size, q_dtype, kv_dtype, window, 0,
      out, out_row_stride, out_head_stride, workspace, workspace_bytes, stream);
}

}  // extern "C"
