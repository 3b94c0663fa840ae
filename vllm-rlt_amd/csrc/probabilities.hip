// Sampling distributions from logits, and the greedy verify round, on MI355X (gfx950).
//
// rlt_probs_kernel replaces the eager torch chain of
// vllm_rlt/worker/speculative_sampling.py:8-56 ``batched_probabilities`` (row form
// vllm_rlt/worker/sampler.py:28-55): x = logits / T, strict top-k by index, strict
// top-p (sorted softmax cumulative mass > p, shifted by one so the crossing token
// stays), softmax.  No sort over the vocabulary is performed.  One 1024-thread
// workgroup owns a row and keeps it in registers and LDS (element j of thread t
// is column 1024 j + t).
//
// Order.  x = l / T is monotone in the logit l for T > 0, so the kernel orders
// tokens by (l descending, column ascending): a descending order of x in which
// tokens tied in x are ordered by l, then by column (the reference leaves the
// surviving index of a tie unspecified).  Every cut below is a threshold in this
// total order: a token is kept iff it precedes the cut token.
//
// Masses.  A token's mass is e = 2^((l - lmax) log2(e) / T) (hardware exp2): the
// softmax numerator exp(x - max x) to ~1e-6 relative.  e is non-decreasing in l,
// so bins taken from the float bits of e are ordered like the tokens: 64 bins per
// binade for e in (2^-16, 1], 4 per binade below (filled only when a cut falls
// there).  Masses are summed in 2^-40 fixed point (64-bit integers: exact and
// order-independent).
//
// Selection (top-k: the k-th token; top-p: the first token whose cumulative mass
// exceeds p Z, Z the total):
//   1. one pass computes e (stored in place of l), the float64 total, and the
//      count / mass histogram of the top bins;
//   2. a block scan finds the bin where the criterion is crossed;
//   3. the bin's tokens (few: a bin spans 1.1% in mass) are gathered into an LDS
//      list of (logit key, column), with their logits re-read, and bitonic-sorted;
//      a scan over the sorted list gives the cut token.  A row whose cut falls in
//      a bin holding more tokens than the list takes the exact path (probs_exact.h:
//      key-range histograms over the re-read logits, ties ranked by column).
// Top-p after top-k runs on the same histogram with the top-k cut bin reduced to
// its kept tokens.  Outputs are e * 2^40 / Z_kept, Z_kept the exact fixed-point
// total of the kept tokens; unfiltered rows sum e in float64.
//
// torch compares a float32 cumsum of float32 softmax values (whose total is 1 +-
// ~1e-5 at V = 65536) with p, so the two top-p cuts can differ only for tokens
// whose preceding mass lies that close to p Z.  A row holding NaN, with a
// non-finite max, or with T not > 0 is written as NaN (torch's softmax gives NaN
// for such rows).
//
// rlt_argmax_rows_kernel + rlt_greedy_match_kernel replace the device greedy round
// of vllm_rlt/worker/async_speculative.py:706-720 (targets = argmax per verify row,
// accepted = leading matches of draft j against target j, next = targets[accepted])
// with the host rule of vllm_rlt/worker/speculative.py:41-53.  argmax takes the first
// maximal column; NaN counts as the maximum (torch's argmax rule).

#include "cascade.h"
#include "common.h"
#include "rlt_mi355x.h"

#include <math.h>
#include <stdlib.h>

#include <type_traits>

namespace {

// ------------------------------------------------------------------ lane exchanges
//
// The value of lane ^ J, J a power of two below 64, without an LDS round trip (a
// ds_bpermute per 32 bits): DPP within 16-lane rows for J <= 8 (quad permutations for
// 1 and 2, the two 4-lane row shifts selected by lane bit 2 for 4, a rotation by 8 for
// 8), the gfx950 lane-swap instructions for 16 and 32.  Reductions built on them keep
// the xor-tree order of the shuffles they replace, so every sum has the same bits.
// Used by the distribution variants with more than 16 register chunks (V > 49152) and
// the long-row variant, where they shorten the selection's reductions (by ~6 us of a
// 65 us launch at V = 65536); the smaller variants measured slightly slower with them
// (code placement) and keep the shuffles.
template <int J>
__device__ __forceinline__ uint32_t xor_lane(uint32_t x) {
  static_assert(J == 1 || J == 2 || J == 4 || J == 8 || J == 16 || J == 32, "lane distance");
  const int lane = threadIdx.x & 63;
  const int v = (int)x;
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);  // [1,0,3,2]
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);  // [2,3,0,1]
  } else if constexpr (J == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xf, 0xf, false);  // lane + 4
    const int dn = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // lane - 4
    return (uint32_t)((lane & 4) ? dn : up);
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false);  // ror 8
  } else if constexpr (J == 16) {
    const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? a[0] : a[1];
  } else {
    const auto a = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? a[0] : a[1];
  }
}

template <int J, typename T>
__device__ __forceinline__ T xor_val(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "lane value");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, xor_lane<J>(__builtin_bit_cast(uint32_t, v)));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = xor_lane<J>((uint32_t)b), hi = xor_lane<J>((uint32_t)(b >> 32));
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}

// The value of lane ^ j (j a power of two below 64): lane exchanges (kFast) or a shuffle.
template <bool kFast, typename T>
__device__ __forceinline__ T xor_at(T v, int j) {
  if constexpr (!kFast) {
    return __shfl_xor(v, j, RLT_WAVE);
  } else {
    switch (j) {
      case 1: return xor_val<1>(v);
      case 2: return xor_val<2>(v);
      case 4: return xor_val<4>(v);
      case 8: return xor_val<8>(v);
      case 16: return xor_val<16>(v);
      default: return xor_val<32>(v);
    }
  }
}

// A 32- or 64-bit value moved by a DPP row pattern (lanes without a source read 0).
template <int kCtrl, typename T>
__device__ __forceinline__ T dpp_val(T v) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(
        T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
  } else {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo =
        (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, kCtrl, 0xf, 0xf, false);
    const uint64_t hi =
        (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), kCtrl, 0xf, 0xf, false);
    return __builtin_bit_cast(T, (hi << 32) | lo);
  }
}

// Inclusive prefix sum of an integer over the 64 lanes (the same value in any order).
// kFast: steps within each 16-lane row (row_shr 1, 2, 4, 8), then rows 0 -> 1 and
// 2 -> 3 (row_bcast 15), then lanes 0..31 -> 32..63 (row_bcast 31); else shuffles.
template <bool kFast, typename T>
__device__ __forceinline__ T wave_incl_scan(T x) {
  static_assert(std::is_integral<T>::value, "integer scan");
  const int lane = threadIdx.x & 63;
  if constexpr (!kFast) {
    for (int off = 1; off < 64; off <<= 1) {
      const T y = __shfl_up(x, off, RLT_WAVE);
      if (lane >= off) x += y;
    }
    return x;
  } else {
    const int r = lane & 15;
    T y = dpp_val<0x111>(x);
    if (r >= 1) x += y;
    y = dpp_val<0x112>(x);
    if (r >= 2) x += y;
    y = dpp_val<0x114>(x);
    if (r >= 4) x += y;
    y = dpp_val<0x118>(x);
    if (r >= 8) x += y;
    y = dpp_val<0x142>(x);
    if (lane & 16) x += y;
    y = dpp_val<0x143>(x);
    if (lane >= 32) x += y;
    return x;
  }
}

#include "probs_exact.h"

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / RLT_WAVE;
constexpr int kMaxRegChunks = 64;       // V <= 65536 keeps the row on chip
constexpr int kMaxStreamChunks = 256;   // V <= 262144: the first chunks on chip, the rest re-read
// On-chip chunks of rows longer than kMaxRegChunks (the exact path then needs tie
// tables for 256 chunks, which leaves room for 24 LDS chunks)
constexpr int kTailReg = 16, kTailLds = 24;
constexpr double kFixScale = 1099511627776.0;  // 2^40

// Histogram bins over the float bits of e in [0, 1].
constexpr uint32_t kOneBits = 0x3f800000u;  // 1.0f
constexpr int kTopBins = 1024;
constexpr uint32_t kFloor8 = 0x3b800000u;   // bits of 2^-8
constexpr uint32_t kFloor16 = 0x37800000u;  // bits of 2^-16
constexpr int kTailShift = 21;              // 4 bins per binade
constexpr int kBins = kTopBins + 512;       // tail: 445 bins used
constexpr int kBinsPerThread = (kBins + kThreads - 1) / kThreads;
constexpr unsigned long long kCutNone = ~0ull;  // "after every token"

// Bin of a token from the bits of its mass e in [0, 1]: 64 bins per binade over
// (2^-16, 1], 4 per binade below.  Non-increasing in e, hence in the logit.
__device__ __forceinline__ int bin_of(uint32_t b) {
  return b > kFloor16 ? (int)((kOneBits - b) >> 17) : kTopBins + (int)((kFloor16 - b) >> kTailShift);
}

// The float bits of the masses in bin b: [lo, hi] (the inverse of bin_of).
__device__ __forceinline__ void bin_bits(int b, uint32_t& lo, uint32_t& hi) {
  if (b < kTopBins) {
    hi = kOneBits - ((uint32_t)b << 17);
    lo = hi - (1u << 17) + 1u;
  } else {
    const int64_t k = b - kTopBins;
    const int64_t h = (int64_t)kFloor16 - (k << kTailShift);
    const int64_t l = h - (1ll << kTailShift) + 1;
    hi = h < 0 ? 0u : (uint32_t)h;
    lo = h < 0 ? 1u : l < 0 ? 0u : (uint32_t)l;  // bins past bin_of(0) are empty
  }
}

// Order-preserving key of a float (NaN excluded by the callers); -0 maps to +0.
__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t b = __float_as_uint(x);
  if ((b & 0x7fffffffu) == 0) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Position of a token in the total order (ascending = l descending, column
// ascending).
__device__ __forceinline__ unsigned long long composite(uint32_t key, uint32_t col) {
  return ((unsigned long long)(~key) << 32) | col;
}

// floor(e * 2^40) for e in [0, 1], from the float's bits (e = m24 * 2^(E - 150)).
__device__ __forceinline__ unsigned long long fixed_mass(float e) {
  const uint32_t b = __float_as_uint(e);
  const int s = (int)(b >> 23) - 110;
  const unsigned long long m24 = (b & 0x7fffffu) | 0x800000u;
  return s >= 0 ? (m24 << s) : (s > -24 ? (m24 >> -s) : 0ull);
}

// Mass of histogram bin b in 2^-40 fixed point.  With Shared::kF64Top the top bins (e in
// (2^-16, 1]) hold the float64 sum of their tokens' e, added by the mass pass with LDS
// float64 atomics: a top bin's tokens are within a factor of two of each other, each a
// multiple of 2^-40 with 24 significant bits, at most 2^18 of them, so their sum needs at
// most 43 significant bits: exact in any order, and equal to the fixed-point sum.  Other
// bins hold fixed-point sums.
template <class Shared>
__device__ __forceinline__ unsigned long long bin_mass(const Shared& sh, int b) {
  const unsigned long long raw = sh.mass[b];
  if (Shared::kF64Top && b < kTopBins)
    return (unsigned long long)(__longlong_as_double((long long)raw) * kFixScale);
  return raw;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

template <typename T, bool kFast = false>
__device__ __forceinline__ T wave_sum(T v) {
  if constexpr (kFast) {
    v += xor_val<32>(v);
    v += xor_val<16>(v);
    v += xor_val<8>(v);
    v += xor_val<4>(v);
    v += xor_val<2>(v);
    v += xor_val<1>(v);
  } else {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, RLT_WAVE);
  }
  return v;
}

#include "probs_split.h"

template <int CAP, bool F64TOP = false, bool FAST_LANES = false>
struct SharedT {
  static constexpr int kCap = CAP;
  // the selection's reductions and scans by lane exchanges (xor_lane, wave_incl_scan)
  static constexpr bool kFastLanes = FAST_LANES;
  // the top bins' masses as float64 sums (bin_mass); kernels whose registers are all
  // taken keep fixed-point sums (the float64 conversion costs them spills)
  static constexpr bool kF64Top = F64TOP;
  unsigned long long mass[kBins];
  uint32_t cnt[kBins];
  unsigned long long list[CAP];  // tokens of the crossing bin (columns, then composites)
  uint32_t wave_u32[kWaves];
  unsigned long long wave_u64[kWaves];
  double wave_f64[kWaves];
  double wave_f64x3[3][kWaves];
  // selection results broadcast to the block
  int sel_bin;
  uint32_t sel_cnt_before;
  unsigned long long sel_mass_before;
  uint32_t sel_bin_cnt;
  unsigned long long sel_bin_mass;
  uint32_t list_n;
  uint32_t gather_n;  // tokens gathered by the current selection
  uint32_t sel_kept_in_bin;
  unsigned long long sel_kept_mass;
};

// Block-wide sum of a u32 and a u64 (every thread gets the totals).
template <class Shared>
__device__ __forceinline__ void block_sum2(Shared& sh, uint32_t& a, unsigned long long& b) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  a = wave_sum<uint32_t, Shared::kFastLanes>(a);
  b = wave_sum<unsigned long long, Shared::kFastLanes>(b);
  if (lane == 0) {
    sh.wave_u32[w] = a;
    sh.wave_u64[w] = b;
  }
  __syncthreads();
  a = 0;
  b = 0;
  for (int i = 0; i < kWaves; ++i) {
    a += sh.wave_u32[i];
    b += sh.wave_u64[i];
  }
  __syncthreads();
}

template <class Shared>
__device__ __forceinline__ double block_sum_f64(Shared& sh, double v) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v = wave_sum<double, Shared::kFastLanes>(v);
  if (lane == 0) sh.wave_f64[w] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < kWaves; ++i) s += sh.wave_f64[i];  // fixed order
  __syncthreads();
  return s;
}

// Block min and max of u32 keys (identity 0xffffffff / 0 for non-members).
template <class Shared>
__device__ __forceinline__ void block_minmax(Shared& sh, uint32_t& lo, uint32_t& hi) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (Shared::kFastLanes) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      lo = min(lo, xor_at<true>(lo, off));
      hi = max(hi, xor_at<true>(hi, off));
    }
  } else {
    for (int off = 32; off >= 1; off >>= 1) {
      lo = min(lo, (uint32_t)__shfl_xor(lo, off, RLT_WAVE));
      hi = max(hi, (uint32_t)__shfl_xor(hi, off, RLT_WAVE));
    }
  }
  if (lane == 0) {
    sh.wave_u32[w] = lo;
    sh.wave_u64[w] = hi;
  }
  __syncthreads();
  lo = 0xffffffffu;
  hi = 0;
  for (int i = 0; i < kWaves; ++i) {
    lo = min(lo, sh.wave_u32[i]);
    hi = max(hi, (uint32_t)sh.wave_u64[i]);
  }
  __syncthreads();
}

// Inclusive block scan over nb histogram bins (thread t owns bins kBinsPerThread t
// + i), then the thread owning the first bin that satisfies the criterion
// publishes it (sel_bin = -1 if none).  kMass: before + cumulative mass > limit;
// else before + cumulative count >= limit.
template <bool kMass, class Shared>
__device__ __forceinline__ void scan_select(Shared& sh, int nb, uint32_t cnt_before,
                                            unsigned long long mass_before,
                                            unsigned long long limit) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  uint32_t c_own[kBinsPerThread];
  unsigned long long m_own[kBinsPerThread];
  uint32_t c = 0;
  unsigned long long m = 0;
#pragma unroll
  for (int i = 0; i < kBinsPerThread; ++i) {
    const int bin = t * kBinsPerThread + i;
    c_own[i] = bin < nb ? sh.cnt[bin] : 0u;
    m_own[i] = bin < nb ? bin_mass(sh, bin) : 0ull;
    c += c_own[i];
    m += m_own[i];
  }
  const uint32_t c_run = c;
  const unsigned long long m_run = m;
  if constexpr (Shared::kFastLanes) {
    c = wave_incl_scan<true>(c);
    m = wave_incl_scan<true>(m);
  } else {
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t cy = __shfl_up(c, off, RLT_WAVE);
      const unsigned long long my = __shfl_up(m, off, RLT_WAVE);
      if (lane >= off) {
        c += cy;
        m += my;
      }
    }
  }
  if (t == 0) {
    sh.sel_bin = -1;
    sh.gather_n = 0;  // for the gather that follows a selection (no reader before)
  }
  if (lane == 63) {
    sh.wave_u32[w] = c;
    sh.wave_u64[w] = m;
  }
  __syncthreads();
  uint32_t cp = cnt_before + c - c_run;
  unsigned long long mp = mass_before + m - m_run;
  for (int i = 0; i < w; ++i) {
    cp += sh.wave_u32[i];
    mp += sh.wave_u64[i];
  }
#pragma unroll
  for (int i = 0; i < kBinsPerThread; ++i) {
    const uint32_t c_incl = cp + c_own[i];
    const unsigned long long m_incl = mp + m_own[i];
    const bool hit = kMass ? (m_incl > limit && !(mp > limit)) : (c_incl >= limit && !(cp >= limit));
    if (hit) {
      sh.sel_bin = t * kBinsPerThread + i;
      sh.sel_cnt_before = cp;
      sh.sel_mass_before = mp;
      sh.sel_bin_cnt = c_own[i];
      sh.sel_bin_mass = m_own[i];
    }
    cp = c_incl;
    mp = m_incl;
  }
  __syncthreads();
}

// Bitonic sort (ascending) of sh.list[0, p), p a power of two; entries past the
// gathered count hold kCutNone.
template <class Shared>
__device__ __forceinline__ void sort_list(Shared& sh, int p) {
  for (int k = 2; k <= p; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < p; i += kThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long a = sh.list[i], b = sh.list[ixj];
          if ((a > b) == ((i & k) == 0)) {
            sh.list[i] = b;
            sh.list[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Result of one selection: tokens of bins before `bin` are kept, and of `bin`
// (whose tokens sit sorted in sh.list) the first kept_in_bin; `kept` is the kept
// tokens' fixed-point mass.  bin = -1: crowded, left to the exact path.
struct Cut {
  int bin;
  uint32_t kept_in_bin;
  unsigned long long kept;
};

// One row's logits.  Chunks j < NREG sit in registers, the next NLDS chunks in
// LDS (xl, chunk-major, conflict-free); NREG = NLDS = 0 re-reads the logits on
// every pass.  After the mass pass the on-chip slots hold e instead of l.
// Columns past V read as NaN: rows holding a real NaN are finished before any
// pass that tests `v == v` for validity, which keeps per-chunk bounds masks out of
// the scalar registers.
template <int DT, int NREG, int NLDS, bool kTail = false>
struct Row {
  static constexpr int kNpt = NREG + NLDS;
  static constexpr int kDtype = DT;
  const void* src;
  int V;
  int npt;  // chunks per thread
  float lmax, c;
  float* xl;
  float xr[NREG > 0 ? NREG : 1];

  // Column of chunk j of this thread: 1024 j + t, except the sixteen register chunks
  // of a kSeq row, which hold the first 16384 columns as whole streams of torch-CPU's
  // float32 row-sum cascade (512-column chunks, 32 streams of 16 steps): register chunk
  // e of thread t is step e of stream t % 32 of cascade chunk 2 (t / 64) + (t / 32) % 2,
  // column 512 c + 32 e + s.  A thread then sums its own register chunks in stream
  // order, and every other cascade chunk lies in LDS in column order.
  static constexpr bool kSeq = NREG == 16 && NLDS > 0 && NLDS % 16 == 0 && !kTail;
  __device__ __forceinline__ int64_t col(int j) const {
    const int t = threadIdx.x;
    if (kSeq && j < 16) return (t >> 6) * 1024 + ((t >> 5) & 1) * 512 + j * 32 + (t & 31);
    return (int64_t)j * kThreads + t;
  }
  __device__ __forceinline__ bool valid(int j) const { return col(j) < V; }
  // chunks past the on-chip ones (kTail: rows longer than kNpt chunks) are re-read
  __device__ __forceinline__ bool on_chip(int j) const { return kNpt > 0 && (!kTail || j < kNpt); }
  __device__ __forceinline__ void set(int j, float v) {
    if (j < NREG) xr[j] = v;
    else if (on_chip(j)) xl[(j - NREG) * kThreads + threadIdx.x] = v;
  }
  // the on-chip value of chunk j (l before the mass pass, e after), or the logit
  // re-read from memory (re-reading variant, and the tail of a kTail row)
  __device__ __forceinline__ float x(int j) const {
    float v;
    if (j < NREG) v = xr[j];
    else if (on_chip(j)) v = xl[(j - NREG) * kThreads + threadIdx.x];
    else v = logit(j);
    // opaque copy: values derived from v are recomputed in each pass instead of
    // being kept live across passes, which would spill
    asm volatile("" : "+v"(v));
    return v;
  }
  // the on-chip value of chunk j without the opaque copy (batched reads: the copies
  // follow all the reads of a batch, so one wait covers them)
  __device__ __forceinline__ float x_raw(int j) const {
    return j < NREG ? xr[j] : xl[(j - NREG) * kThreads + threadIdx.x];
  }
  __device__ __forceinline__ static void opaque(float& v) { asm volatile("" : "+v"(v)); }
  __device__ __forceinline__ float logit(int j) const {
    return valid(j) ? load_as_f32<DT>(src, col(j)) : NAN;
  }
  __device__ __forceinline__ float mass(float l) const {
    return __builtin_amdgcn_exp2f((l - lmax) * c);
  }
  // e of chunk j after the mass pass (NaN for padding)
  __device__ __forceinline__ float e(int j) const {
    if (on_chip(j)) return x(j);
    const float l = x(j);
    return l == l ? mass(l) : NAN;
  }
  // f(j, e(j)) for every chunk with the values of four LDS chunks read before their
  // four calls (the output pass: its global stores do not wait for the next LDS reads).
  template <class F>
  __device__ __forceinline__ void for_chunks_e4(F f) const {
#pragma unroll
    for (int j = 0; j < NREG; ++j) f(j, e(j));
    if (kNpt > 0) {
      const int end = kTail ? kNpt : npt;
      int j = NREG;
#pragma unroll 1
      for (; j + 4 <= end; j += 4) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = x_raw(j + u);  // on chip: e is the slot
#pragma unroll
        for (int u = 0; u < 4; ++u) opaque(v[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u) f(j + u, v[u]);
      }
#pragma unroll 1
      for (; j < end; ++j) f(j, e(j));
    }
    if (kNpt == 0 || kTail) {
      int j = kNpt;
#pragma unroll 1
      for (; j + 4 <= npt; j += 4) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = e(j + u);
#pragma unroll
        for (int u = 0; u < 4; ++u) f(j + u, v[u]);
      }
#pragma unroll 1
      for (; j < npt; ++j) f(j, e(j));
    }
  }
  // f(j, x(j)) for every chunk (l before the mass pass), LDS chunks read four at a time
  // before their four calls (one LDS round trip per four chunks, not per chunk).
  template <class F>
  __device__ __forceinline__ void for_chunks_x4(F f) const {
#pragma unroll
    for (int j = 0; j < NREG; ++j) f(j, x(j));
    if (kNpt > 0) {
      const int end = kTail ? kNpt : npt;
      int j = NREG;
#pragma unroll 1
      for (; j + 4 <= end; j += 4) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = x_raw(j + u);
#pragma unroll
        for (int u = 0; u < 4; ++u) opaque(v[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u) f(j + u, v[u]);
      }
#pragma unroll 1
      for (; j < end; ++j) f(j, x(j));
    }
    if (kNpt == 0 || kTail) {
      int j = kNpt;
#pragma unroll 1
      for (; j + 4 <= npt; j += 4) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = x(j + u);
#pragma unroll
        for (int u = 0; u < 4; ++u) f(j + u, v[u]);
      }
#pragma unroll 1
      for (; j < npt; ++j) f(j, x(j));
    }
  }
  // f(j) for every chunk: register chunks unrolled (static register indices),
  // LDS chunks in a rolled loop, re-read chunks four at a time (loads in flight).
  // Calls are wave-uniform (ballots allowed).
  template <class F>
  __device__ __forceinline__ void for_chunks(F f) const {
#pragma unroll
    for (int j = 0; j < NREG; ++j) f(j);
    if (kNpt > 0) {
#pragma unroll 1
      for (int j = NREG; j < (kTail ? kNpt : npt); ++j) f(j);
    }
    if (kNpt == 0 || kTail) {
      int j = kNpt;
#pragma unroll 1
      for (; j + 4 <= npt; j += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) f(j + u);
      }
#pragma unroll 1
      for (; j < npt; ++j) f(j);
    }
  }
};

// Adds (1, fm) of every lane with `take` to its bin.
template <class Shared>
__device__ __forceinline__ void hist_add(Shared& sh, bool take, int bin, unsigned long long fm) {
  if (take) {
    atomicAdd(&sh.cnt[bin], 1u);
    atomicAdd(&sh.mass[bin], fm);
  }
}

template <class Shared>
__device__ __forceinline__ void clear_hist(Shared& sh, int from, int to) {
  for (int i = from + (int)threadIdx.x; i < to; i += kThreads) {
    sh.cnt[i] = 0;
    sh.mass[i] = 0;
  }
}

// Histogram stages: the tokens with e in (2^-8, 1] (stage 0), (2^-16, 2^-8]
// (stage 1) and [0, 2^-16] (stage 2); admit_stages adds stages [s0, s1).
template <class Shared, class R>
__device__ __forceinline__ void admit_stages(Shared& sh, const R& row, int s0, int s1) {
  const uint32_t lo = s1 == 1 ? kFloor8 + 1u : s1 == 2 ? kFloor16 + 1u : 0u;
  const uint32_t hi = s0 == 0 ? 0xffffffffu : s0 == 1 ? kFloor8 : kFloor16;
  row.for_chunks([&](int j) {
    const float e = row.e(j);
    const uint32_t bits = __float_as_uint(e);
    const bool take = e == e && bits >= lo && bits <= hi;
    hist_add(sh, take, take ? bin_of(bits) : 0, take ? fixed_mass(e) : 0ull);
  });
  __syncthreads();
}

// Selection over the histogram in sh, admitting histogram stages as needed.  Members: every token of a bin < mbin, and in
// bin mbin the first mlist entries of the (sorted) list left by the previous
// selection; (kBins, 0) takes all.
//   kMass: the cut token is the first whose cumulative member mass exceeds limit;
//   else the cut follows the limit-th member.
// Leaves the crossing bin's tokens sorted in sh.list[0, sh.list_n).
template <bool kMass, class Shared, class R>
__device__ __forceinline__ Cut select(Shared& sh, const R& row, unsigned long long limit,
                                      int& stages, int mbin, uint32_t mlist) {
  const int t = threadIdx.x, lane = t & 63;
  // the histogram holds stages [0, stages); admit further tokens by mass range until
  // the criterion is crossed: e > 2^-8 and (2^-16, 2^-8] (both admitted by the mass
  // pass), then the rest (each stage a prefix of the order, so a scan over the
  // admitted bins is exact for the cuts they contain)
  scan_select<kMass>(sh, kBins, 0, 0, limit);
  while (sh.sel_bin < 0 && stages < 3) {
    __syncthreads();
    admit_stages(sh, row, stages, stages + 1);
    ++stages;
    scan_select<kMass>(sh, kBins, 0, 0, limit);
  }
  const int bin = sh.sel_bin;  // >= 0: the region holds the cut by construction
  const uint32_t cnt_before = sh.sel_cnt_before;
  const unsigned long long mass_before = sh.sel_mass_before;
  const uint32_t n = sh.sel_bin_cnt;
  // (sel_* are rewritten only by a later selection, after further barriers)

  Cut out;
  out.bin = bin;
  int nl;
  const bool member = bin >= 0 && bin == mbin;
  if (member) {
    nl = (int)mlist;  // the members are the sorted prefix already in the list
  } else {
    if (bin < 0 || n > (uint32_t)Shared::kCap) {
      // crowded bin: the row goes to the exact path (block-uniform)
      out.bin = -1;
      return out;
    }
    // gather the bin's columns (all members: bin < mbin) into the list (gather_n was
    // zeroed by the scan)
    uint32_t blo, bhi;
    bin_bits(bin, blo, bhi);
    row.for_chunks_e4([&](int j, float e) {
      // the bin's bit range (NaN padding lies above every bin's range)
      const uint32_t bits = __float_as_uint(e);
      const bool take = bits >= blo && bits <= bhi;
      const uint64_t m = __ballot(take);
      if (m == 0) return;
      uint32_t base = 0;
      if (lane == 0) base = atomicAdd(&sh.gather_n, (uint32_t)__popcll(m));
      base = __shfl(base, 0, RLT_WAVE);
      const uint32_t pos = base + __popcll(m & lanemask_lt());
      if (take && pos < (uint32_t)Shared::kCap) sh.list[pos] = (uint32_t)row.col(j);
    });
    __syncthreads();
    // (a top-p selection without a top-k cut has no bin counts: n = 0 above)
    if (sh.gather_n > (uint32_t)Shared::kCap) {
      out.bin = -1;  // crowded: the exact path (block-uniform)
      return out;
    }
    nl = (int)sh.gather_n;
  }
  if (nl <= RLT_WAVE) {
    // one wave: the gathered columns' logits, a bitonic sort in registers, and the scan
    // of the sorted members; one barrier publishes the result
    if (t < RLT_WAVE) {
      unsigned long long v = kCutNone;
      if (lane < nl) {
        v = sh.list[lane];
        if (!member) {
          const uint32_t col = (uint32_t)v;
          v = composite(order_key(load_as_f32<R::kDtype>(row.src, col)), col);
        }
      }
      if (!member) {
#pragma unroll
        for (int k = 2; k <= RLT_WAVE; k <<= 1) {
#pragma unroll
          for (int j = k >> 1; j > 0; j >>= 1) {
            const unsigned long long o = xor_at<Shared::kFastLanes>(v, j);
            const bool keep_min = ((lane & k) == 0) == ((lane & j) == 0);
            v = keep_min ? (o < v ? o : v) : (o < v ? v : o);
          }
        }
        if (lane < nl) sh.list[lane] = v;
        if (lane == 0) sh.list_n = (uint32_t)nl;
      }
      // masses recomputed from the keys (the mass pass's arithmetic); members kept
      // while the cut criterion is not reached
      const unsigned long long fm =
          lane < nl ? fixed_mass(row.mass(key_value(~(uint32_t)(v >> 32)))) : 0ull;
      const unsigned long long incl = wave_incl_scan<Shared::kFastLanes>(fm);
      const unsigned long long before = mass_before + incl - fm;
      const bool keep =
          lane < nl && (kMass ? before <= limit : (uint32_t)lane < limit - cnt_before);
      const unsigned long long km =
          wave_sum<unsigned long long, Shared::kFastLanes>(keep ? fm : 0ull);
      const uint32_t kn = (uint32_t)__popcll(__ballot(keep));  // (the whole wave votes)
      if (lane == 0) {
        sh.sel_kept_in_bin = kn;
        sh.sel_kept_mass = km;
      }
    }
    __syncthreads();
    out.kept_in_bin = sh.sel_kept_in_bin;
    out.kept = mass_before + sh.sel_kept_mass;
    return out;
  }
  if (!member) {
    if (t == 0) sh.list_n = (uint32_t)nl;  // (read after the barriers below)
    int p = 1;
    while (p < nl) p <<= 1;
    for (int i = t; i < p; i += kThreads) {
      unsigned long long v = kCutNone;
      if (i < nl) {
        const uint32_t col = (uint32_t)sh.list[i];
        v = composite(order_key(load_as_f32<R::kDtype>(row.src, col)), col);
      }
      sh.list[i] = v;
    }
    __syncthreads();
    sort_list(sh, p);
  }
  // scan the sorted members: masses recomputed from the keys (same arithmetic as
  // the mass pass), kept while the cut criterion is not reached
  constexpr int kPer = (Shared::kCap + kThreads - 1) / kThreads;
  unsigned long long fm[kPer];
  unsigned long long run = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int idx = t * kPer + i;
    fm[i] = 0;
    if (idx < nl) fm[i] = fixed_mass(row.mass(key_value(~(uint32_t)(sh.list[idx] >> 32))));
    run += fm[i];
  }
  const unsigned long long incl = wave_incl_scan<Shared::kFastLanes>(run);
  if (lane == 63) sh.wave_u64[t >> 6] = incl;
  __syncthreads();
  unsigned long long before = mass_before + incl - run;
  for (int i = 0; i < (t >> 6); ++i) before += sh.wave_u64[i];
  uint32_t kept_here = 0;
  unsigned long long kept_mass = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int idx = t * kPer + i;
    const bool keep = idx < nl && (kMass ? before <= limit : (uint32_t)idx < limit - cnt_before);
    kept_here += keep;
    kept_mass += keep ? fm[i] : 0ull;
    before += fm[i];
  }
  block_sum2(sh, kept_here, kept_mass);
  out.kept_in_bin = kept_here;
  out.kept = mass_before + kept_mass;
  return out;
}

// Workgroup barrier that orders LDS accesses only: the row's global stores stay in
// flight (a __syncthreads() would wait for every one of them to complete).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Store of a written probability, streamed (non-temporal) when no pass of the launch
// reads the row back: the next launch at most reads it, and lines left dirty in the L2
// would be written back at the kernel boundary, ahead of that launch's own work.  (A
// compile-time choice: a runtime branch between the two stores is merged into one
// plain store by the compiler.)
template <bool kStream, class P>
__device__ __forceinline__ void put(P dst, float v) {
  if constexpr (kStream) __builtin_nontemporal_store(v, dst);
  else *dst = v;
}

// What a written row holds, per token: e * inv above the cut bin (bits > chi), 0 below
// it (bits < clo), and in the cut bin e * inv for the first kept_n tokens of the
// sorted list, 0 for the others.
struct Written {
  float inv;
  uint32_t clo, chi;
  uint32_t kept_n;
};

// The last passes of a kSeq row whose acceptance partials are wanted (pm): every on-chip
// value becomes the written one in place (e * inv, 0, or for the cut bin's tokens e * inv
// when the sorted list keeps them; the kept tokens are first marked in their owners'
// chunk masks), the row-sum partials are formed from those values (the register chunks'
// streams by their own threads, the LDS chunks' streams read across threads; chunk sums
// meet in LDS, then stream s of group g adds its chunks in order), and only then is the
// row stored (streamed), so no barrier waits behind the stores.  `cut` false: an
// unfiltered row.
template <class Shared, class R>
__device__ __forceinline__ void seq_finish(Shared& sh, R& row, const Written& wr, bool cut,
                                           float* __restrict__ pm, float* __restrict__ dst) {
  static_assert(R::kNpt <= 64 && kThreads <= kBins, "chunk masks");
  const int t = threadIdx.x;
  const cascade::RowGeom geo = cascade::row_geom(row.V);
  lds_barrier();  // the selection's histogram is no longer read
  unsigned long long km = 0;
  if (cut) {
    sh.mass[t] = 0;
    lds_barrier();
    for (uint32_t i = t; i < wr.kept_n; i += kThreads) {
      // owner of column x: below 16384 thread 64 w + 32 h + s, chunk e for x = 1024 w +
      // 512 h + 32 e + s; above, thread x % 1024, chunk x / 1024
      const uint32_t x = (uint32_t)sh.list[i];
      const uint32_t owner = x < 16384u ? (((x >> 4) & 0x3e0u) | (x & 31u)) : (x & 1023u);
      const uint32_t j = x < 16384u ? ((x >> 5) & 15u) : (x >> 10);
      atomicOr(&sh.mass[owner], 1ull << j);
    }
    lds_barrier();
    km = sh.mass[t];
  }
  auto written = [&](int j, float m) {
    const bool keep = !cut || __float_as_uint(m) > wr.chi || ((km >> j) & 1ull);
    return keep ? m * wr.inv : 0.f;  // (padding: NaN stays NaN)
  };
#pragma unroll
  for (int j = 0; j < 16; ++j) row.xr[j] = written(j, row.xr[j]);
  const int npt = row.npt;  // a multiple of 16
  for (int j0 = 16; j0 < npt; j0 += 8) {
    // eight slots read at once (one wait), then rewritten
    float* slot = row.xl + (j0 - 16) * kThreads + t;
    float m[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) m[u] = slot[u * kThreads];
#pragma unroll
    for (int u = 0; u < 8; ++u) R::opaque(m[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u) slot[u * kThreads] = written(j0 + u, m[u]);
  }
  lds_barrier();  // the LDS chunks hold the written values; the masks are consumed
  float(*cs)[cascade::kStreams + 1] = reinterpret_cast<float(*)[cascade::kStreams + 1]>(&sh);
  const int s = t & 31;
  const int c_thread = 2 * (t >> 6) + ((t >> 5) & 1);
  if (c_thread < geo.full_chunks) {
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) a += row.xr[e];
    cs[c_thread][s] = a;
  }
  for (int c = 32 + c_thread; c < geo.full_chunks; c += 32) {
    // LDS slot of column 16384 + i is i (chunk 16 + i / 1024, thread i % 1024)
    const float* x = row.xl + (c - 32) * 512 + s;
    float m[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) m[e] = x[32 * e];
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) a += m[e];
    cs[c][s] = a;
  }
  lds_barrier();
  if (pm) {
    for (int i = t; i < geo.groups * cascade::kStreams; i += kThreads) {
      const int g = i / cascade::kStreams, st = i % cascade::kStreams;
      const int c_end = (int)min((int64_t)(g + 1) * cascade::kGroupChunks, geo.full_chunks);
      float acc1 = 0.f;
      for (int c = g * cascade::kGroupChunks; c < c_end; ++c) acc1 += cs[c][st];
      pm[i] = acc1;
    }
  }
  __attribute__((address_space(1))) float* gdst = (__attribute__((address_space(1))) float*)dst;
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (row.xr[j] == row.xr[j]) put<true>(&gdst[row.col(j)], row.xr[j]);
  for (int j0 = 16; j0 < npt; j0 += 8) {
    const float* slot = row.xl + (j0 - 16) * kThreads + t;
    float m[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) m[u] = slot[u * kThreads];
#pragma unroll
    for (int u = 0; u < 8; ++u) R::opaque(m[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (m[u] == m[u]) put<true>(&gdst[(int64_t)(j0 + u) * kThreads + t], m[u]);
  }
}

// Top-k / top-p cut and the output of one row.  Returns false, having written
// nothing, when a cut falls in a bin more crowded than the list (the caller then
// runs the exact path).
template <class Shared, class R>
__device__ __forceinline__ bool filter_row(Shared& sh, const R& row, float* __restrict__ dst,
                                           bool do_k, bool do_p, unsigned long long kk, float p,
                                           double z, float* __restrict__ pm, bool stream) {
  const int t = threadIdx.x;
  int stages = 2;  // histogram stages admitted so far (0 and 1 by the mass pass)

  Cut cut;
  if (do_k) {
    // top-k (reference: speculative_sampling.py:39-48): keeps min(k_eff, max_top_k)
    cut = select<false>(sh, row, kk, stages, kBins, 0u);
    if (cut.bin < 0) return false;
  }
  if (do_p) {
    // top-p (reference: speculative_sampling.py:49-55) over the top-k survivors:
    // kept prefix = every token whose preceding mass is <= p Z (p <= 0 keeps one)
    const unsigned long long zk = do_k ? cut.kept : (unsigned long long)(z * kFixScale);
    const unsigned long long limit = p > 0.f ? (unsigned long long)((double)p * (double)zk) : 0ull;
    if (do_k) {
      // histogram of the survivors: bins before the top-k bin unchanged, the
      // top-k bin reduced to its kept tokens, later bins empty
      const Cut ck = cut;
      if (t == 0) {
        unsigned long long before = 0;
        for (int i = 0; i < ck.bin; ++i) before += bin_mass(sh, i);
        sh.cnt[ck.bin] = ck.kept_in_bin;
        const unsigned long long kb = ck.kept - before;  // exact in float64 (as above)
        sh.mass[ck.bin] = Shared::kF64Top && ck.bin < kTopBins
                              ? (unsigned long long)__double_as_longlong((double)kb / kFixScale)
                              : kb;
      }
      clear_hist(sh, ck.bin + 1, kBins);
      __syncthreads();
      stages = 3;  // bins up to the top-k bin are complete; later ones hold no survivor
      cut = select<true>(sh, row, limit, stages, ck.bin, ck.kept_in_bin);
    } else {
      cut = select<true>(sh, row, limit, stages, kBins, 0u);
    }
    if (cut.bin < 0) return false;
  }

  // ---- softmax over the kept tokens, normalized by their exact fixed-point total:
  // bins before the cut bin kept, later bins dropped, the cut bin's tokens written
  // from the sorted list (its first kept_in_bin kept)
  const float inv = (float)(kFixScale / (double)cut.kept);
  uint32_t clo, chi;
  bin_bits(cut.bin, clo, chi);
  if constexpr (R::kSeq) {
    if (pm) {
      seq_finish(sh, const_cast<R&>(row), Written{inv, clo, chi, cut.kept_in_bin}, true, pm, dst);
      return true;
    }
  }
  // stores through a global-space pointer: they cannot alias the row's LDS chunks, so
  // the next chunks' LDS reads need not wait for them
  __attribute__((address_space(1))) float* gdst = (__attribute__((address_space(1))) float*)dst;
  auto output = [&](auto stream_tag) {
    constexpr bool kStream = decltype(stream_tag)::value;
    row.for_chunks_e4([&](int j, float e) {
      // bins before the cut bin hold larger masses (kept), later bins smaller ones; the
      // cut bin's tokens are written from the list below (NaN: padding); one store
      const uint32_t bits = __float_as_uint(e);
      const float v = bits > chi ? e * inv : 0.f;
      if (e == e && (bits > chi || bits < clo)) put<kStream>(&gdst[row.col(j)], v);
    });
    const int nl = min((int)sh.list_n, Shared::kCap);
    for (int i = t; i < nl; i += kThreads) {
      const unsigned long long v = sh.list[i];
      const float e = row.mass(key_value(~(uint32_t)(v >> 32)));
      put<kStream>(&dst[(uint32_t)v], (uint32_t)i < cut.kept_in_bin ? e * inv : 0.f);
    }
  };
  if (stream) output(std::true_type{});
  else output(std::false_type{});
  return true;
}

// First maximal column of logits row r (NaN counts as the maximum, torch's argmax
// rule) into targets[r]; one 1024-thread workgroup.
template <int DT>
__device__ __forceinline__ void argmax_row(const void* __restrict__ logits, int64_t row_stride,
                                           int V, int64_t r, int64_t* __restrict__ targets,
                                           unsigned long long* wave_best) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const char* src = (const char*)logits + r * row_stride * (DT == RLT_F32 ? 4 : 2);
  // packed key: (order key of the value, NaN = all ones) << 32 | ~column
  unsigned long long best = 0;
  auto take = [&](float x, int64_t i) {
    const uint32_t key = x != x ? 0xffffffffu : order_key(x);
    const unsigned long long packed = ((unsigned long long)key << 32) | (0xffffffffu - (uint32_t)i);
    best = packed > best ? packed : best;
  };
  // eight loads in flight per thread, then the remainder
  constexpr int kU = 8;
  int64_t i0 = t;
  for (; i0 + (kU - 1) * kThreads < V; i0 += kU * kThreads) {
    float x[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) x[u] = load_as_f32<DT>(src, i0 + u * kThreads);
#pragma unroll
    for (int u = 0; u < kU; ++u) take(x[u], i0 + u * kThreads);
  }
  for (; i0 < V; i0 += kThreads) take(load_as_f32<DT>(src, i0), i0);
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, RLT_WAVE);
    best = o > best ? o : best;
  }
  if (lane == 0) wave_best[w] = best;
  __syncthreads();
  if (t == 0) {
    unsigned long long b = 0;
    for (int i = 0; i < kWaves; ++i) b = wave_best[i] > b ? wave_best[i] : b;
    targets[r] = (int64_t)(0xffffffffu - (uint32_t)(b & 0xffffffffu));
  }
}

// Output row r (blockIdx.x) is the distribution of logits row rows[r] (rows ==
// nullptr: row r) of n_src; temperature / top_k / top_p are indexed by r.  A source
// row outside [0, n_src) gives an all-NaN output row.
template <int DT, int NREG, int NLDS, bool kTail>
__global__ __launch_bounds__(kThreads) void rlt_probs_kernel(
    const void* __restrict__ logits, const int64_t* __restrict__ rows, int64_t n_src,
    int64_t row_stride, int V,
    const float* __restrict__ temperature, const int64_t* __restrict__ top_k,
    const float* __restrict__ top_p, int max_top_k, int apply_top_p, float* __restrict__ out,
    int64_t out_stride, int64_t* __restrict__ argmax_out, int64_t argmax_rows,
    const float* __restrict__ qm_src, int64_t qm_rows, float* __restrict__ qm_out,
    int64_t qm_blocks, float* __restrict__ pm_out) {
  constexpr int NPT = NREG + NLDS;
  // the exact path (crowded rows) reuses the fast path's LDS
  constexpr int kCapV = NLDS > 32 ? 512 : NLDS == 32 ? 1024 : 2048;
  constexpr int kTC = NPT > 0 && !kTail ? NPT : kMaxStreamChunks;
  union Lds {
    SharedT<kCapV, (NREG <= 16), (NREG > 16 || kTail)> fast;
    exact::SharedT<kTC> ex;
  };
  __shared__ Lds lds;
  auto& sh = lds.fast;
  // blocks past the distribution rows take the argmax of logits rows 0..argmax_rows-1
  // (greedy proposals and targets, run alongside the distributions), then the float32
  // row-sum partials of the qm_rows draft rows for the acceptance sampler, eight
  // 8192-float groups per workgroup, on CUs the distributions leave idle
  const int64_t n_dist = (int64_t)gridDim.x - argmax_rows - qm_blocks;
  if ((int64_t)blockIdx.x >= n_dist + argmax_rows) {
    static_assert(sizeof(Lds) >= 8 * sizeof(cascade::ChunkSums), "group staging");
    cascade::ChunkSums* cs = reinterpret_cast<cascade::ChunkSums*>(&lds);
    const cascade::RowGeom geo = cascade::row_geom(V);
    const int t = threadIdx.x;
    const int sub = t / cascade::kGroupThreads, st = t % cascade::kGroupThreads;
    const int64_t task = ((int64_t)blockIdx.x - n_dist - argmax_rows) *
                             (kThreads / cascade::kGroupThreads) + sub;
    const int64_t qrow = geo.groups > 0 ? task / geo.groups : qm_rows;
    const int64_t g = geo.groups > 0 ? task % geo.groups : 0;
    const bool live = qrow < qm_rows;
    const float* x = qm_src + qrow * V;
    if (live) {
      if (V % 4 == 0 && (uintptr_t)qm_src % 16 == 0)
        cascade::group_chunk_sums<true>(x, g, geo.full_chunks, st, cs[sub]);
      else
        cascade::group_chunk_sums<false>(x, g, geo.full_chunks, st, cs[sub]);
    }
    __syncthreads();
    if (live)
      cascade::group_stream_sums(g, geo.full_chunks, st, cs[sub],
                                 qm_out + (qrow * geo.groups + g) * cascade::kStreams);
    return;
  }
  if ((int64_t)blockIdx.x >= n_dist) {
    argmax_row<DT>(logits, row_stride, V, (int64_t)blockIdx.x - n_dist, argmax_out,
                   reinterpret_cast<unsigned long long*>(&lds));
    return;
  }
  __shared__ float xlds[NLDS > 0 ? NLDS * kThreads : 1];
  // the p row's acceptance partials formed on chip (kSeq rows), else read back below
  constexpr bool kSeq = Row<DT, NREG, NLDS, kTail>::kSeq;
  float* const pm_row =
      kSeq && pm_out ? pm_out + (int64_t)blockIdx.x * cascade::row_geom(V).groups * cascade::kStreams
                     : nullptr;
  bool pm_done = false;
  do {
  const int64_t r = blockIdx.x;
  const int64_t src_r = rows ? rows[r] : r;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  Row<DT, NREG, NLDS, kTail> row;
  row.xl = xlds;
  row.V = V;
  const bool src_ok = src_r >= 0 && src_r < n_src;
  row.src = (const char*)logits + (src_ok ? src_r : 0) * row_stride * (DT == RLT_F32 ? 4 : 2);
  row.npt = NPT > 0 && !kTail ? NPT : (V + kThreads - 1) / kThreads;
  float* dst = out + r * out_stride;
  const float temp = temperature[r];
  row.c = 1.44269504088896341f / temp;  // log2(e) / T

  // ---- row max and NaN detection (padding stored as NaN)
  float lmax = -INFINITY;
  bool nan = false;
  auto take_raw = [&](int j, float l) {
    const bool ok = row.valid(j);
    nan |= ok && l != l;
    row.set(j, ok ? l : NAN);
    lmax = ok ? fmaxf(lmax, l) : lmax;
  };
  auto fetch = [&](int j) {
    return row.valid(j) ? load_as_f32<DT>(row.src, row.col(j)) : 0.f;
  };
  if constexpr (DT == RLT_F32 && NLDS > 0 && !kTail && NREG <= 16) {
    // every chunk in flight at once: register chunks into VGPRs, LDS chunks copied
    // straight into their LDS slots (each lane's dword lands at its own slot), then
    // the maximum and NaN test of the LDS chunks read back by their own lanes (the
    // variants with more register chunks keep the batched form below: the copies'
    // addresses cost them spills)
    typedef __attribute__((address_space(3))) void lds_void_t;
    float raw[NREG > 0 ? NREG : 1];
#pragma unroll
    for (int j = 0; j < NREG; ++j) raw[j] = fetch(j);
#pragma unroll
    for (int jj = 0; jj < NLDS; ++jj) {
      const int j = NREG + jj;
      if (row.valid(j))
        __builtin_amdgcn_global_load_lds(
            (const void*)((const float*)row.src + row.col(j)),
            (lds_void_t*)(xlds + jj * kThreads + w * 64), 4, 0, 0);
      else
        xlds[jj * kThreads + t] = NAN;
    }
#pragma unroll
    for (int j = 0; j < NREG; ++j) take_raw(j, raw[j]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll 8
    for (int jj = 0; jj < NLDS; ++jj) {
      const float l = xlds[jj * kThreads + t];
      nan |= row.valid(NREG + jj) && l != l;
      lmax = fmaxf(lmax, l);  // padding holds NaN, which fmaxf ignores
    }
  } else if (NPT > 0) {
    // every register chunk and the first LDS batch in flight at once; each LDS
    // batch is consumed while the next one loads
    constexpr int kB = 16;
    float raw[NREG > 0 ? NREG : 1];
    float cur[kB];
#pragma unroll
    for (int j = 0; j < NREG; ++j) raw[j] = fetch(j);
#pragma unroll
    for (int u = 0; u < kB; ++u) cur[u] = NREG + u < NPT ? fetch(NREG + u) : 0.f;
#pragma unroll
    for (int j = 0; j < NREG; ++j) take_raw(j, raw[j]);
#pragma unroll 1
    for (int j0 = NREG; j0 < NPT; j0 += kB) {
      float nxt[kB];
#pragma unroll
      for (int u = 0; u < kB; ++u) nxt[u] = j0 + kB + u < NPT ? fetch(j0 + kB + u) : 0.f;
#pragma unroll
      for (int u = 0; u < kB; ++u)
        if (j0 + u < NPT) take_raw(j0 + u, cur[u]);
#pragma unroll
      for (int u = 0; u < kB; ++u) cur[u] = nxt[u];
    }
    if (kTail) {
      // the re-read tail: maximum and NaN only (nothing stored)
#pragma unroll 1
      for (int j0 = NPT; j0 < row.npt; j0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = j0 + u < row.npt ? row.logit(j0 + u) : NAN;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          nan |= row.valid(j0 + u) && v[u] != v[u];
          lmax = fmaxf(lmax, v[u]);  // padding reads NaN, which fmaxf ignores
        }
      }
    }
  } else {
    row.for_chunks([&](int j) {
      const float l = row.x(j);
      nan |= row.valid(j) && l != l;
      lmax = fmaxf(lmax, l);  // padding reads NaN, which fmaxf ignores
    });
  }
  if constexpr (decltype(lds.fast)::kFastLanes) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) lmax = fmaxf(lmax, xor_at<true>(lmax, off));
  } else {
    for (int off = 32; off >= 1; off >>= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, off, RLT_WAVE));
  }
  const uint64_t nan_b = __ballot(nan);
  if (lane == 0) {
    sh.wave_f64[w] = lmax;
    sh.wave_u32[w] = nan_b != 0;
  }
  clear_hist(sh, 0, kBins);  // stages 0 and 1 are admitted by the mass pass
  __syncthreads();
  lmax = -INFINITY;
  int bad = 0;
  for (int i = 0; i < kWaves; ++i) {
    lmax = fmaxf(lmax, (float)sh.wave_f64[i]);
    bad |= sh.wave_u32[i];
  }
  __syncthreads();
  if (bad || !src_ok || !isfinite(lmax) || !(temp > 0.f) || !isfinite(row.c)) {
    for (int64_t i = t; i < V; i += kThreads) dst[i] = NAN;
    break;
  }
  row.lmax = lmax;

  const int64_t k_req = top_k[r];
  const int64_t k_eff = (k_req > 0 && k_req < V) ? k_req : (int64_t)V;
  const bool do_k = max_top_k > 0 && k_eff < V;
  const float p = top_p[r];
  const bool do_p = apply_top_p && p < 1.f;

  // ---- mass pass: e in place of l, the float64 total, and histogram stages 0 and 1
  // (the tokens with e > 2^-16: a few percent of a row; where top-p cuts the
  // distributions of a verify step)
  double zs = 0.0;
  row.for_chunks_x4([&](int j, float l) {
    // padding (NaN; rows holding a real NaN have left) keeps e = NaN in its slot and
    // counts as 0: fmaxf returns the number of a (NaN, number) pair
    const float e = row.mass(l);
    if (NPT > 0) row.set(j, e);
    const float e0 = fmaxf(e, 0.f);
    zs += (double)e0;
    const uint32_t bits = __float_as_uint(e0);
    if (bits > kFloor16) {
      const int b = bin_of(bits);
      // counts only for a top-k cut: a top-p selection scans masses, and its gather
      // counts the crossing bin's tokens itself
      if (do_k) atomicAdd(&sh.cnt[b], 1u);
      if constexpr (decltype(lds.fast)::kF64Top)
        atomicAdd(reinterpret_cast<double*>(&sh.mass[b]), (double)e0);  // a top bin
      else
        atomicAdd(&sh.mass[b], fixed_mass(e0));
    }
  });
  const double z = block_sum_f64(sh, zs);
  if (!do_k && !do_p) {
    const float inv = (float)(1.0 / z);
    if constexpr (kSeq) {
      if (pm_row) {
        seq_finish(sh, row, Written{inv, 0u, 0u, 0u}, false, pm_row, dst);
        pm_done = true;
        break;
      }
    }
    auto output = [&](auto stream_tag) {
      constexpr bool kStream = decltype(stream_tag)::value;
      row.for_chunks_e4([&](int j, float e) {
        if (e == e) put<kStream>(&dst[row.col(j)], e * inv);
      });
    };
    if (pm_out == nullptr) output(std::true_type{});  // (nothing reads the row back)
    else output(std::false_type{});
    break;
  }

  const unsigned long long kk =
      (unsigned long long)(k_eff < (int64_t)max_top_k ? k_eff : (int64_t)max_top_k);
  if (!filter_row(sh, row, dst, do_k, do_p, kk, p, z, pm_row, pm_out == nullptr)) {
    __syncthreads();
    exact::exact_row<DT, kTC>(lds.ex, logits, src_r, row_stride, V, temperature, top_k, top_p,
                              max_top_k, apply_top_p, out, out_stride);
  } else {
    pm_done = pm_row != nullptr;
  }
  } while (0);
  if (pm_out && !pm_done) {
    // the written row's float32 row-sum partials for the acceptance sampler (p row r
    // at pm_out + r * groups * 32) where seq_finish did not form them (rows of the
    // other variants, the exact path, rows written as NaN): the row is read back after
    // the barrier, which makes every wave's stores visible to the workgroup; eight
    // 8192-float groups per pass, staged like the q rows' blocks above
    __syncthreads();
    cascade::ChunkSums* cs = reinterpret_cast<cascade::ChunkSums*>(&lds);
    const cascade::RowGeom geo = cascade::row_geom(V);
    const int t = threadIdx.x;
    const int sub = t / cascade::kGroupThreads, st = t % cascade::kGroupThreads;
    const float* x = out + (int64_t)blockIdx.x * out_stride;
    constexpr int kPer = kThreads / cascade::kGroupThreads;
    for (int64_t g0 = 0; g0 < geo.groups; g0 += kPer) {
      const int64_t g = g0 + sub;
      if (g < geo.groups) {
        if (out_stride % 4 == 0 && (uintptr_t)out % 16 == 0)
          cascade::group_chunk_sums<true>(x, g, geo.full_chunks, st, cs[sub]);
        else
          cascade::group_chunk_sums<false>(x, g, geo.full_chunks, st, cs[sub]);
      }
      __syncthreads();
      if (g < geo.groups)
        cascade::group_stream_sums(g, geo.full_chunks, st, cs[sub],
                                   pm_out + ((int64_t)blockIdx.x * geo.groups + g) * cascade::kStreams);
      __syncthreads();
    }
  }
}

// ------------------------------------------------------------------ greedy round

// One workgroup per verify row: first maximal column (NaN is the maximum).
template <int DT>
__global__ __launch_bounds__(kThreads) void rlt_argmax_rows_kernel(const void* __restrict__ logits,
                                                                   int64_t row_stride, int V,
                                                                   int64_t* __restrict__ targets) {
  __shared__ unsigned long long wave_best[kWaves];
  argmax_row<DT>(logits, row_stride, V, blockIdx.x, targets, wave_best);
}

// One lane per request: leading matches of draft j against target row j.
__global__ void rlt_greedy_match_kernel(const int64_t* __restrict__ draft_tokens,
                                        const int64_t* __restrict__ drafts,
                                        const int64_t* __restrict__ targets, int64_t n, int w1,
                                        int64_t* __restrict__ accepted,
                                        int64_t* __restrict__ next_token) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t d = drafts[i];
  int64_t a = 0;
  for (int j = 0; j < w1; ++j) {
    if (j >= d || draft_tokens[i * w1 + j] != targets[i * (w1 + 1) + j]) break;
    ++a;
  }
  accepted[i] = a;
  next_token[i] = targets[i * (w1 + 1) + a];
}

template <int DT, int NREG, int NLDS, bool kTail = false>
void launch_probs(int64_t n, const void* logits, const int64_t* rows, int64_t n_src,
                  int64_t row_stride, int V, const float* temperature, const int64_t* top_k,
                  const float* top_p, int max_top_k, int apply_top_p, float* out,
                  int64_t out_stride, hipStream_t stream, int64_t* argmax_out,
                  int64_t argmax_rows, const float* qm_src, int64_t qm_rows, float* qm_out,
                  float* pm_out) {
  const cascade::RowGeom geo = cascade::row_geom(V);
  const int64_t per_block = kThreads / cascade::kGroupThreads;
  const int64_t qm_blocks = qm_src ? (qm_rows * geo.groups + per_block - 1) / per_block : 0;
  hipLaunchKernelGGL((rlt_probs_kernel<DT, NREG, NLDS, kTail>),
                     dim3((unsigned)(n + argmax_rows + qm_blocks)), dim3(kThreads), 0, stream,
                     logits, rows, n_src, row_stride, V, temperature, top_k, top_p, max_top_k,
                     apply_top_p, out, out_stride, argmax_out, argmax_rows, qm_src, qm_rows,
                     qm_out, qm_blocks, pm_out);
}

// Row placement by chunks per thread: registers first (at most 32, beyond which
// the kernel spills), then LDS (at most 128 KiB); longer rows keep their first 40
// chunks on chip and re-read the rest on every pass.
template <int DT>
void dispatch_probs(int64_t n, const void* logits, const int64_t* rows, int64_t n_src,
                    int64_t row_stride, int V,
                    const float* temperature, const int64_t* top_k, const float* top_p,
                    int max_top_k, int apply_top_p, float* out, int64_t out_stride,
                    hipStream_t stream, int64_t* argmax_out = nullptr, int64_t argmax_rows = 0,
                    const float* qm_src = nullptr, int64_t qm_rows = 0,
                    float* qm_out = nullptr, float* pm_out = nullptr) {
  const int chunks = (V + kThreads - 1) / kThreads;
#define RLT_PROBS_CASE(R, L)                                                                  \
  launch_probs<DT, R, L>(n, logits, rows, n_src, row_stride, V, temperature, top_k, top_p,     \
                         max_top_k, apply_top_p, out, out_stride, stream, argmax_out,         \
                         argmax_rows, qm_src, qm_rows, qm_out, pm_out)
  if (chunks <= 4) RLT_PROBS_CASE(4, 0);
  else if (chunks <= 16) RLT_PROBS_CASE(8, 8);
  else if (chunks <= 32) RLT_PROBS_CASE(16, 16);
  else if (chunks <= 48) RLT_PROBS_CASE(16, 32);
  else if (chunks <= 56) RLT_PROBS_CASE(24, 32);
  else if (chunks <= 58) RLT_PROBS_CASE(26, 32);
  else if (chunks <= 60) RLT_PROBS_CASE(28, 32);
  else if (chunks <= kMaxRegChunks) RLT_PROBS_CASE(30, 34);
  else
    launch_probs<DT, kTailReg, kTailLds, true>(n, logits, rows, n_src, row_stride, V,
                                               temperature, top_k, top_p, max_top_k,
                                               apply_top_p, out, out_stride, stream, argmax_out,
                                               argmax_rows, qm_src, qm_rows, qm_out, pm_out);
#undef RLT_PROBS_CASE
}

// ------------------------------------------------------------------ split form (host)

// The split form (probs_split.h) serves calls that filter no row (max_top_k == 0 and
// no top-p).  E elements per thread: the smallest of 16 (68 VGPRs, seven waves per
// SIMD), 32 (113 VGPRs) and 64 (217 VGPRs, two waves per SIMD) whose slice count fits
// kMaxSlices and min_e (the written rows' partial sums need whole 8192-column groups).
// 1280 rows of 65536: 187 us at E = 16, 196 at 32, 206 at 64.
struct SplitPlan {
  int E, S;
};

bool split_plan(int64_t n_dist, int V, SplitPlan& p, int min_e = 16) {
  auto slices = [&](int e) { return (V + split::kThreads * e - 1) / (split::kThreads * e); };
  int pick = min_e <= 16 && slices(16) <= split::kMaxSlices ? 16 : 32;
  if (slices(pick) > split::kMaxSlices) pick = 64;
  if (slices(pick) > split::kMaxSlices) return false;
  p.E = pick;
  p.S = slices(pick);
  return true;
}

size_t split_bytes(int64_t n_dist, int64_t n_arg, int V) {
  const int64_t nb = (V + split::kBlockCols - 1) / split::kBlockCols;
  return rlt_align_up((size_t)(n_dist + n_arg) * nb * sizeof(split::BlockStat), 256);
}

// The split form's two launches.  targets: argmax outputs -- of the distribution rows
// when fused, else of logits rows [0, n_arg).  pm_out: the written rows' row-sum
// partials (plans with E >= 32).
template <int DT, int E>
void launch_split_e(const SplitPlan& pl, int64_t n_dist, const void* logits, const int64_t* rows,
                    int64_t n_src, int64_t row_stride, int V, const float* temperature,
                    float* out, int64_t out_stride, hipStream_t stream, int64_t* targets,
                    int64_t n_arg, bool fused, const float* qm_src, int64_t qm_rows,
                    float* qm_out, void* ws, float* pm_out, double* tile_sum,
                    uint32_t* tile_flags, bool skip_drawn) {
  split::View v;
  v.stats = (split::BlockStat*)ws;
  v.S = pl.S;
  v.L = split::kThreads * E;
  v.NB = (V + split::kBlockCols - 1) / split::kBlockCols;
  v.n_dist = n_dist;
  v.n_arg = fused ? 0 : n_arg;
  v.targets = targets;
  v.fused = fused;
  v.pm_out = pm_out;
  v.tile_sum = tile_sum;
  v.tile_flags = tile_flags;
  v.tiles = (V + split::kBlockCols - 1) / split::kBlockCols;
  v.skip_drawn = skip_drawn && rows && !fused && n_dist <= split::kMaxDrawnScan;
  const int esz = DT == RLT_F32 ? 4 : 2;
  const bool vec = V % 4 == 0 && row_stride % 4 == 0 && (uintptr_t)logits % (4 * esz) == 0;
  const bool out_vec = out_stride % 4 == 0 && (uintptr_t)out % 16 == 0;
  const cascade::RowGeom geo = cascade::row_geom(V);
  const int64_t per_block = split::kThreads / cascade::kGroupThreads;
  const int64_t qm_blocks = qm_src ? (qm_rows * geo.groups + per_block - 1) / per_block : 0;
  const int64_t g1 = (n_dist + v.n_arg) * pl.S + qm_blocks;
  const int64_t g2 = n_dist * pl.S + (v.n_arg + split::kThreads - 1) / split::kThreads;
#define RLT_SPLIT_LAUNCH(VEC)                                                                  \
  hipLaunchKernelGGL((split::rlt_probs_slice_kernel<DT, E, VEC>), dim3((unsigned)g1),          \
                     dim3(split::kThreads), 0, stream, logits, rows, n_src, row_stride, V,       \
                     temperature, v, qm_src, qm_rows, qm_out);                                   \
  hipLaunchKernelGGL((split::rlt_probs_write_kernel<DT, E, VEC>), dim3((unsigned)g2),          \
                     dim3(split::kThreads), 0, stream, logits, rows, n_src, row_stride, V,       \
                     temperature, v, out, out_stride, (int)out_vec)
  if (vec) {
    RLT_SPLIT_LAUNCH(true);
  } else {
    RLT_SPLIT_LAUNCH(false);
  }
#undef RLT_SPLIT_LAUNCH
}

template <int DT>
void launch_split(const SplitPlan& pl, int64_t n_dist, const void* logits, const int64_t* rows,
                  int64_t n_src, int64_t row_stride, int V, const float* temperature, float* out,
                  int64_t out_stride, hipStream_t stream, int64_t* targets, int64_t n_arg,
                  bool fused, const float* qm_src, int64_t qm_rows, float* qm_out, void* ws,
                  float* pm_out = nullptr, double* tile_sum = nullptr,
                  uint32_t* tile_flags = nullptr, bool skip_drawn = false) {
#define RLT_SPLIT_E(EE)                                                                         \
  launch_split_e<DT, EE>(pl, n_dist, logits, rows, n_src, row_stride, V, temperature, out,      \
                         out_stride, stream, targets, n_arg, fused, qm_src, qm_rows, qm_out, ws, \
                         pm_out, tile_sum, tile_flags, skip_drawn)
  if (pl.E == 16) RLT_SPLIT_E(16);
  else if (pl.E == 32) RLT_SPLIT_E(32);
  else RLT_SPLIT_E(64);
#undef RLT_SPLIT_E
}

}  // namespace

// spec_sampling.hip: the acceptance workspace's p-row and q-row partials, and the
// acceptance launches that use them instead of summing q (and p) again.
float* rlt_accept_p_partials(void* workspace, int64_t n, int32_t w1, int64_t vocab);
float* rlt_accept_q_partials(void* workspace, int64_t n, int32_t w1, int64_t vocab);
double* rlt_categorical_tile_sums(void* workspace, int64_t m, int64_t vocab);
uint32_t* rlt_categorical_tile_flags(void* workspace, int64_t m, int64_t vocab);
int rlt_categorical_rows_after_tiles(const float* weights, int64_t w_stride, const float* u,
                                     int64_t m, int64_t vocab, int64_t* out_index,
                                     const int64_t* scatter, int64_t n_out, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream);
int rlt_accept_after_pq_partials(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                                 const float* p, const float* u_accept, const float* u_final,
                                 int64_t n, int32_t w1, int64_t vocab, int64_t* tokens,
                                 int64_t* accepted, int64_t* final_token, uint8_t* error,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream);
int rlt_accept_after_q_partials(const int64_t* draft_tokens, const int64_t* drafts, const float* q,
                                const float* p, const float* u_accept, const float* u_final,
                                int64_t n, int32_t w1, int64_t vocab, int64_t* tokens,
                                int64_t* accepted, int64_t* final_token, uint8_t* error,
                                void* workspace, size_t workspace_bytes, hipStream_t stream);

// spec_sampling.hip: categorical draws over strided rows with a scatter list.
int rlt_categorical_rows(const float* weights, int64_t w_stride, const float* u, int64_t m,
                         int64_t vocab, int64_t* out_index, const int64_t* scatter, int64_t n_out,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

extern "C" {

size_t rlt_probabilities_workspace_size(int64_t rows, int64_t argmax_rows, int64_t vocab) {
  SplitPlan pl;
  if (rows < 0 || argmax_rows < 0 || vocab < 1 || vocab > 0x7fffffff ||
      !split_plan(rows, (int)vocab, pl))
    return 0;
  return split_bytes(rows, argmax_rows, (int)vocab);
}

int rlt_batched_probabilities(const void* logits, int32_t logits_dtype, int64_t row_stride,
                              int64_t n, int64_t vocab, const float* temperature,
                              const int64_t* top_k, const float* top_p, int64_t max_top_k,
                              int32_t apply_top_p, float* out, int64_t out_stride,
                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (n < 0 || vocab < 1 || max_top_k < 0 || row_stride < vocab || out_stride < vocab)
    return RLT_ERR_ARGUMENT;
  if (n == 0) return RLT_OK;
  if (!logits || !temperature || !top_k || !top_p || !out) return RLT_ERR_ARGUMENT;
  if (vocab > (int64_t)kMaxStreamChunks * kThreads || n > 0x7fffffff) return RLT_ERR_UNSUPPORTED;
  const int mtk = max_top_k > vocab ? (int)vocab : (int)max_top_k;
  const int V = (int)vocab;
  // the row-split form for calls that filter no row, when a workspace is given
  SplitPlan pl;
  const bool sp = workspace && mtk == 0 && !apply_top_p && split_plan(n, V, pl);
  if (sp && workspace_bytes < split_bytes(n, 0, V)) return RLT_ERR_WORKSPACE;
#define RLT_PROBS(DT)                                                                          \
  do {                                                                                         \
    if (sp)                                                                                    \
      launch_split<DT>(pl, n, logits, nullptr, n, row_stride, V, temperature, out, out_stride, \
                       stream, nullptr, 0, false, nullptr, 0, nullptr, workspace);             \
    else                                                                                       \
      dispatch_probs<DT>(n, logits, nullptr, n, row_stride, V, temperature, top_k, top_p, mtk, \
                         apply_top_p != 0, out, out_stride, stream);                           \
  } while (0)
  switch (logits_dtype) {
    case RLT_F32: RLT_PROBS(RLT_F32); break;
    case RLT_BF16: RLT_PROBS(RLT_BF16); break;
    case RLT_F16: RLT_PROBS(RLT_F16); break;
    default: return RLT_ERR_UNSUPPORTED;
  }
#undef RLT_PROBS
  return rlt_launch_status();
}

int rlt_greedy_accept(const int64_t* draft_tokens, const int64_t* drafts, const void* target_logits,
                      int32_t logits_dtype, int64_t row_stride, int64_t n, int32_t w1,
                      int64_t vocab, int64_t* targets, int64_t* accepted, int64_t* next_token,
                      hipStream_t stream) {
  if (n < 0 || w1 < 0 || vocab < 1 || vocab > 0x7fffffff || row_stride < vocab)
    return RLT_ERR_ARGUMENT;
  if (n == 0) return RLT_OK;
  if (!draft_tokens || !drafts || !target_logits || !targets || !accepted || !next_token)
    return RLT_ERR_ARGUMENT;
  const int64_t rows = n * (w1 + 1);
  if (rows > 0x7fffffff) return RLT_ERR_UNSUPPORTED;
  switch (logits_dtype) {
    case RLT_F32:
      hipLaunchKernelGGL(rlt_argmax_rows_kernel<RLT_F32>, dim3((unsigned)rows), dim3(kThreads), 0,
                         stream, target_logits, row_stride, (int)vocab, targets);
      break;
    case RLT_BF16:
      hipLaunchKernelGGL(rlt_argmax_rows_kernel<RLT_BF16>, dim3((unsigned)rows), dim3(kThreads), 0,
                         stream, target_logits, row_stride, (int)vocab, targets);
      break;
    case RLT_F16:
      hipLaunchKernelGGL(rlt_argmax_rows_kernel<RLT_F16>, dim3((unsigned)rows), dim3(kThreads), 0,
                         stream, target_logits, row_stride, (int)vocab, targets);
      break;
    default:
      return RLT_ERR_UNSUPPORTED;
  }
  const int threads = 256;
  hipLaunchKernelGGL(rlt_greedy_match_kernel, dim3((unsigned)((n + threads - 1) / threads)),
                     dim3(threads), 0, stream, draft_tokens, drafts, targets, n, w1, accepted,
                     next_token);
  return rlt_launch_status();
}

size_t rlt_propose_drafts_workspace_size(int64_t m, int64_t r, int64_t vocab) {
  if (m < 0 || r < 0) return 0;
  return rlt_align_up(r > 0 ? rlt_categorical_workspace_size(r, vocab) : 0, 256) +
         (r > 0 ? rlt_probabilities_workspace_size(r, m, vocab) : 0);
}

int rlt_propose_drafts(const void* logits, int32_t logits_dtype, int64_t row_stride, int64_t m,
                       int64_t vocab, const int64_t* random_rows, int64_t r,
                       const float* temperature, const int64_t* top_k, const float* top_p,
                       int64_t max_top_k, int32_t apply_top_p, const float* u, float* q_out,
                       int64_t q_stride, int64_t* proposed, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || r < 0 || vocab < 1 || vocab > 0x7fffffff || row_stride < vocab ||
      max_top_k < 0 || (r > 0 && q_stride < vocab))
    return RLT_ERR_ARGUMENT;
  if (m == 0 && r == 0) return RLT_OK;
  if (!logits || !proposed) return RLT_ERR_ARGUMENT;
  if (r > 0 && (!random_rows || !temperature || !top_k || !top_p || !u || !q_out))
    return RLT_ERR_ARGUMENT;
  if (vocab > (int64_t)kMaxStreamChunks * kThreads || m > 0x7fffffff || r > 0x7fffffff)
    return RLT_ERR_UNSUPPORTED;
  if (r > 0 && (!workspace || workspace_bytes < rlt_categorical_workspace_size(r, vocab)))
    return RLT_ERR_WORKSPACE;
  const int V = (int)vocab;
  const int mtk = max_top_k > vocab ? V : (int)max_top_k;
  // the split form when the workspace holds its part too
  const size_t cat_bytes = r > 0 ? rlt_align_up(rlt_categorical_workspace_size(r, vocab), 256) : 0;
  SplitPlan pl;
  const bool sp = r > 0 && mtk == 0 && !apply_top_p && split_plan(r, V, pl) &&
                  workspace_bytes >= cat_bytes + split_bytes(r, m, V);
  // the split form also writes the draws' tile totals (rows of at most 2M columns)
  double* tsum = sp ? rlt_categorical_tile_sums(workspace, r, vocab) : nullptr;
  uint32_t* tflags = sp ? rlt_categorical_tile_flags(workspace, r, vocab) : nullptr;
  // greedy proposals for every row (extra workgroups of the distribution launch when
  // there are random rows; the split form skips the rows the draws overwrite), then
  // the random rows' draws
#define RLT_PROPOSE(DT)                                                                       \
  do {                                                                                        \
    if (r == 0)                                                                               \
      hipLaunchKernelGGL(rlt_argmax_rows_kernel<DT>, dim3((unsigned)m), dim3(kThreads), 0,    \
                         stream, logits, row_stride, V, proposed);                            \
    else if (sp)                                                                              \
      launch_split<DT>(pl, r, logits, random_rows, m, row_stride, V, temperature, q_out,      \
                       q_stride, stream, proposed, m, false, nullptr, 0, nullptr,             \
                       (char*)workspace + cat_bytes, nullptr, tsum, tflags, true);            \
    else                                                                                      \
      dispatch_probs<DT>(r, logits, random_rows, m, row_stride, V, temperature, top_k, top_p, \
                         mtk, apply_top_p != 0, q_out, q_stride, stream, proposed, m);        \
  } while (0)
  switch (logits_dtype) {
    case RLT_F32: RLT_PROPOSE(RLT_F32); break;
    case RLT_BF16: RLT_PROPOSE(RLT_BF16); break;
    case RLT_F16: RLT_PROPOSE(RLT_F16); break;
    default: return RLT_ERR_UNSUPPORTED;
  }
#undef RLT_PROPOSE
  if (r == 0) return rlt_launch_status();
  const int st = rlt_launch_status();
  if (st != RLT_OK) return st;
  if (tsum)
    return rlt_categorical_rows_after_tiles(q_out, q_stride, u, r, vocab, proposed, random_rows,
                                            m, workspace, workspace_bytes, stream);
  return rlt_categorical_rows(q_out, q_stride, u, r, vocab, proposed, random_rows, m, workspace,
                              workspace_bytes, stream);
}

int rlt_verify_distributions(const void* logits, int32_t logits_dtype, int64_t row_stride,
                             int64_t m, int64_t vocab, const int64_t* random_rows, int64_t r,
                             const float* temperature, const int64_t* top_k, const float* top_p,
                             int64_t max_top_k, int32_t apply_top_p, float* p_out,
                             int64_t p_stride, int64_t* targets, void* workspace,
                             size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || r < 0 || vocab < 1 || vocab > 0x7fffffff || row_stride < vocab ||
      max_top_k < 0 || (r > 0 && p_stride < vocab))
    return RLT_ERR_ARGUMENT;
  if (m == 0 && r == 0) return RLT_OK;
  if (!logits || (m > 0 && !targets)) return RLT_ERR_ARGUMENT;
  if (r > 0 && (!random_rows || !temperature || !top_k || !top_p || !p_out))
    return RLT_ERR_ARGUMENT;
  if (vocab > (int64_t)kMaxStreamChunks * kThreads || m > 0x7fffffff || r > 0x7fffffff)
    return RLT_ERR_UNSUPPORTED;
  const int V = (int)vocab;
  const int mtk = max_top_k > vocab ? V : (int)max_top_k;
  SplitPlan pl;
  const bool sp = r > 0 && workspace && mtk == 0 && !apply_top_p && split_plan(r, V, pl);
  if (sp && workspace_bytes < split_bytes(r, m, V)) return RLT_ERR_WORKSPACE;
  // targets of every row as extra workgroups of the distribution launch (split form:
  // extra slices of launch 1, finished by launch 2 or 3)
#define RLT_VERIFY(DT)                                                                        \
  do {                                                                                        \
    if (r == 0)                                                                               \
      hipLaunchKernelGGL(rlt_argmax_rows_kernel<DT>, dim3((unsigned)m), dim3(kThreads), 0,    \
                         stream, logits, row_stride, V, targets);                             \
    else if (sp)                                                                              \
      launch_split<DT>(pl, r, logits, random_rows, m, row_stride, V, temperature, p_out,      \
                       p_stride, stream, targets, m, false, nullptr, 0, nullptr, workspace);  \
    else                                                                                      \
      dispatch_probs<DT>(r, logits, random_rows, m, row_stride, V, temperature, top_k, top_p, \
                         mtk, apply_top_p != 0, p_out, p_stride, stream, targets, m);         \
  } while (0)
  switch (logits_dtype) {
    case RLT_F32: RLT_VERIFY(RLT_F32); break;
    case RLT_BF16: RLT_VERIFY(RLT_BF16); break;
    case RLT_F16: RLT_VERIFY(RLT_F16); break;
    default: return RLT_ERR_UNSUPPORTED;
  }
#undef RLT_VERIFY
  return rlt_launch_status();
}

size_t rlt_verify_accept_workspace_size(int64_t n, int32_t w1, int64_t vocab) {
  if (n < 0 || w1 < 0) return 0;
  return rlt_align_up(rlt_speculative_accept_workspace_size(n, w1, vocab), 256) +
         rlt_probabilities_workspace_size(n * (w1 + 1), 0, vocab);
}

int rlt_verify_accept(const void* target_logits, int32_t logits_dtype, int64_t row_stride,
                      const float* temperature, const int64_t* top_k, const float* top_p,
                      int64_t max_top_k, int32_t apply_top_p, const int64_t* draft_tokens,
                      const int64_t* drafts, const float* q, const float* u_accept,
                      const float* u_final, int64_t n, int32_t w1, int64_t vocab,
                      int64_t* targets, float* p_out, int64_t* tokens, int64_t* accepted,
                      int64_t* final_token, uint8_t* error, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  if (n < 0 || w1 < 0 || vocab < 1 || row_stride < vocab || max_top_k < 0) return RLT_ERR_ARGUMENT;
  if (n == 0) return RLT_OK;
  if (!target_logits || !temperature || !top_k || !top_p || !drafts || !u_final || !targets ||
      !p_out || !tokens || !accepted || !final_token || !error ||
      (w1 > 0 && (!draft_tokens || !q || !u_accept)))
    return RLT_ERR_ARGUMENT;
  const int64_t rows = n * (w1 + 1);
  if (vocab > (int64_t)kMaxStreamChunks * kThreads || rows > 0x7fffffff || w1 > 32 ||
      vocab >= ((int64_t)1 << 25))
    return RLT_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < rlt_speculative_accept_workspace_size(n, w1, vocab))
    return RLT_ERR_WORKSPACE;
  float* qm_out = rlt_accept_q_partials(workspace, n, w1, vocab);
  const int64_t q_rows = n * (int64_t)w1;
  const int V = (int)vocab;
  const int mtk = max_top_k > vocab ? V : (int)max_top_k;
  // the split form when the workspace holds its part too
  const size_t acc_bytes =
      rlt_align_up(rlt_speculative_accept_workspace_size(n, w1, vocab), 256);
  SplitPlan pl;
  const bool sp = mtk == 0 && !apply_top_p && split_plan(rows, V, pl, 32) &&
                  workspace_bytes >= acc_bytes + split_bytes(rows, 0, V);
  // both forms write the p rows' row-sum partials alongside the distributions
  float* pm_out = rlt_accept_p_partials(workspace, n, w1, vocab);
  // distributions of every verify row, their argmax targets, and the draft rows'
  // row-sum partials (one launch, or the split form's launches); then the acceptance
  // sums only p
#define RLT_VERIFY_ACCEPT(DT)                                                                 \
  do {                                                                                        \
    if (sp)                                                                                   \
      launch_split<DT>(pl, rows, target_logits, nullptr, rows, row_stride, V, temperature,    \
                       p_out, vocab, stream, targets, rows, true, q_rows > 0 ? q : nullptr,   \
                       q_rows, qm_out, (char*)workspace + acc_bytes, pm_out);                 \
    else                                                                                      \
      dispatch_probs<DT>(rows, target_logits, nullptr, rows, row_stride, V, temperature,      \
                         top_k, top_p, mtk, apply_top_p != 0, p_out, vocab, stream, targets,  \
                         rows, q_rows > 0 ? q : nullptr, q_rows, qm_out, pm_out);             \
  } while (0)
  switch (logits_dtype) {
    case RLT_F32: RLT_VERIFY_ACCEPT(RLT_F32); break;
    case RLT_BF16: RLT_VERIFY_ACCEPT(RLT_BF16); break;
    case RLT_F16: RLT_VERIFY_ACCEPT(RLT_F16); break;
    default: return RLT_ERR_UNSUPPORTED;
  }
#undef RLT_VERIFY_ACCEPT
  const int st = rlt_launch_status();
  if (st != RLT_OK) return st;
  return rlt_accept_after_pq_partials(draft_tokens, drafts, q, p_out, u_accept, u_final, n, w1,
                                      vocab, tokens, accepted, final_token, error, workspace,
                                      workspace_bytes, stream);
}

}  // extern "C"
