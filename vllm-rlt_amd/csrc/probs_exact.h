// Exact-selection path of the sampling-distribution kernel (gfx950).
//
// exact::exact_row computes, inside rlt_probs_kernel (probabilities.hip;
// reference vllm_rlt/worker/speculative_sampling.py:8-56), the rows whose top-k or
// top-p cut falls inside a mass bin holding more tokens than the fast path's
// on-chip list (near-uniform rows, large tie groups).  It re-reads the row on every pass and selects on x = logits / T
// (IEEE division, as torch) with expf masses:
//
//   * pass 0 bins every candidate by its distance below the row max, in steps of
//     1/16 logit (1024 bins, the last one open-ended); a block scan of the per-bin
//     (count, mass) finds the bin where the criterion is crossed: count >= k for
//     top-k, cumulative mass > p Z for top-p;
//   * later passes re-bin only the crossing bin's members by the order-preserving
//     32-bit key of x, in power-of-two key bins below the bin's largest key; each
//     pass shrinks the key range at least 512-fold, so at most five passes end on
//     a single value v (the cut);
//   * every element above v is kept; of the elements equal to v, the first t in
//     column order are kept, where t is what the count or mass rule leaves room
//     for.
//
// Masses are exp(x - max) in 2^-40 fixed point, summed as 64-bit integers: exact
// and order-independent.  Included inside probabilities.hip's anonymous
// namespace; it shares the fast path's LDS (the row is re-read from memory).

#pragma once

namespace exact {


constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / RLT_WAVE;
constexpr int kBins = 1024;
constexpr float kBinsPerLogit = 16.f;
constexpr int kMaxRegChunks = 64;       // V <= 65536 keeps the row in registers
constexpr int kMaxStreamChunks = 256;   // V <= 262144 on the re-reading variant
constexpr double kFixScale = 1099511627776.0;  // 2^40

// Order-preserving key of a float (NaN excluded by the callers); -0 maps to +0.
__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t b = __float_as_uint(x);
  if ((b & 0x7fffffffu) == 0) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint64_t fixed_mass(float e) {
  return (uint64_t)((double)e * kFixScale);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, RLT_WAVE);
  return v;
}

template <int TC>
struct SharedT {
  static constexpr int kTieChunks = TC;
  uint32_t cnt[kBins];
  unsigned long long mass[kBins];
  uint32_t wave_u32[kWaves];
  unsigned long long wave_u64[kWaves];
  double wave_f64[kWaves];
  uint32_t tie_base[2][TC * kWaves];
  // selection results broadcast to the block
  int sel_bin;
  uint32_t sel_cnt_before;
  unsigned long long sel_mass_before;
  uint32_t sel_bin_cnt;
  unsigned long long sel_bin_mass;
  uint32_t klo, khi;
  float row_max;
  int bad_row;
};

// Block-wide sum of a u32 and a u64 (every thread gets the totals).
template <class Shared>
__device__ __forceinline__ void block_sum2(Shared& sh, uint32_t& a, unsigned long long& b) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  a = wave_sum(a);
  b = wave_sum(b);
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
  v = wave_sum(v);
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
  for (int off = 32; off >= 1; off >>= 1) {
    lo = min(lo, (uint32_t)__shfl_xor(lo, off, RLT_WAVE));
    hi = max(hi, (uint32_t)__shfl_xor(hi, off, RLT_WAVE));
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

// Inclusive block scan over the histogram (thread t owns bin t), then the thread
// whose bin first satisfies the criterion publishes it.  kMass: criterion is
// before + cumulative mass > limit; else before + cumulative count >= limit.
template <bool kMass, class Shared>
__device__ __forceinline__ void scan_select(Shared& sh, uint32_t cnt_before, unsigned long long mass_before,
                            unsigned long long limit) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const uint32_t c_own = sh.cnt[t];
  const unsigned long long m_own = sh.mass[t];
  uint32_t c = c_own;
  unsigned long long m = m_own;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t cy = __shfl_up(c, off, RLT_WAVE);
    const unsigned long long my = __shfl_up(m, off, RLT_WAVE);
    if (lane >= off) {
      c += cy;
      m += my;
    }
  }
  if (lane == 63) {
    sh.wave_u32[w] = c;
    sh.wave_u64[w] = m;
  }
  __syncthreads();
  uint32_t cp = cnt_before;
  unsigned long long mp = mass_before;
  for (int i = 0; i < w; ++i) {
    cp += sh.wave_u32[i];
    mp += sh.wave_u64[i];
  }
  const uint32_t c_incl = cp + c, c_excl = c_incl - c_own;
  const unsigned long long m_incl = mp + m, m_excl = m_incl - m_own;
  const bool hit = kMass ? (m_incl > limit && !(m_excl > limit))
                         : (c_incl >= limit && !(c_excl >= limit));
  if (hit) {
    sh.sel_bin = t;
    sh.sel_cnt_before = c_excl;
    sh.sel_mass_before = m_excl;
    sh.sel_bin_cnt = c_own;
    sh.sel_bin_mass = m_own;
  }
  __syncthreads();
}

// Per-row state of one selection: elements with key > key are above the cut,
// `take` of the elements equal to key (in column order) are kept.
struct Cut {
  uint32_t key;
  uint32_t take;   // kept elements at key
  uint32_t ties;   // elements at key (members of the selection)
  bool partial;    // take < ties: column ranks needed
};

// One row's x = logits / T.  Chunks j < NREG sit in registers, the next NLDS
// chunks in LDS (xl, chunk-major, conflict-free); NREG = NLDS = 0 re-reads the
// logits on every pass.
template <int DT, int NREG, int NLDS>
struct Row {
  static constexpr int kNpt = NREG + NLDS;
  const void* src;
  int V;
  float temp;
  int npt;  // chunks per thread
  float* xl;
  float xr[NREG > 0 ? NREG : 1];

  __device__ __forceinline__ bool valid(int j) const {
    return (int64_t)j * kThreads + threadIdx.x < V;
  }
  __device__ __forceinline__ void set(int j, float v) {
    if (j < NREG) xr[j] = v;
    else if (kNpt > 0) xl[(j - NREG) * kThreads + threadIdx.x] = v;
  }
  __device__ __forceinline__ float x(int j) const {
    float v;
    if (j < NREG) v = xr[j];
    else if (kNpt > 0) v = xl[(j - NREG) * kThreads + threadIdx.x];
    else v = valid(j) ? load_as_f32<DT>(src, (int64_t)j * kThreads + threadIdx.x) / temp : -INFINITY;
    // opaque copy: values derived from x (key, exp, mass) are recomputed in each
    // pass instead of being kept live across passes, which would spill
    asm volatile("" : "+v"(v));
    return v;
  }
  // f(j) for every chunk: register chunks unrolled (static register indices),
  // the others in a rolled loop.  Calls are wave-uniform (ballots allowed).
  template <class F>
  __device__ __forceinline__ void for_chunks(F f) const {
#pragma unroll
    for (int j = 0; j < NREG; ++j) f(j);
#pragma unroll 1
    for (int j = NREG; j < npt; ++j) f(j);
  }
};

// Column rank of each tie (elements with member && key == cut) in column order:
// table[j * kWaves + w] = number of ties in chunks < j, plus ties of chunk j in
// waves < w; rank = table entry + ties in lower lanes of the same wave.
template <class Shared, class R, class Member>
__device__ __forceinline__ void build_tie_table(Shared& sh, const R& row, uint32_t key, int which,
                                                Member member) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint32_t* table = sh.tie_base[which];
  row.for_chunks([&](int j) {
    const bool tie = row.valid(j) && member(j) && order_key(row.x(j)) == key;
    const uint64_t b = __ballot(tie);
    if (lane == 0) table[j * kWaves + w] = __popcll(b);
  });
  __syncthreads();
  // exclusive scan of npt * kWaves entries: thread t owns a run of `per` entries
  const int entries = row.npt * kWaves;
  const int per = (entries + kThreads - 1) / kThreads;
  const int t = threadIdx.x;
  constexpr int kPerMax = (Shared::kTieChunks * kWaves + kThreads - 1) / kThreads;
  uint32_t vals[kPerMax];
  uint32_t run = 0;
#pragma unroll
  for (int e = 0; e < kPerMax; ++e) {
    const int idx = t * per + e;
    vals[e] = (e < per && idx < entries) ? table[idx] : 0u;
    run += vals[e];
  }
  uint32_t incl = run;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(incl, off, RLT_WAVE);
    if (lane >= off) incl += y;
  }
  if (lane == 63) sh.wave_u32[w] = incl;
  __syncthreads();
  uint32_t base = incl - run;
  for (int i = 0; i < w; ++i) base += sh.wave_u32[i];
#pragma unroll
  for (int e = 0; e < kPerMax; ++e) {
    const int idx = t * per + e;
    if (e < per && idx < entries) table[idx] = base;
    base += vals[e];
  }
  __syncthreads();
}

template <class Shared>
__device__ __forceinline__ uint32_t tie_rank(const Shared& sh, int which, int j, bool tie) {
  const uint64_t b = __ballot(tie);
  return sh.tie_base[which][j * kWaves + (threadIdx.x >> 6)] + __popcll(b & lanemask_lt());
}

// Bin of x in a pass: pass 0 by distance below the max in 1/16-logit steps,
// later passes by key offset below khi in 2^shift-key steps.
__device__ __forceinline__ int bin_of(float x, uint32_t key, float m, bool value_bins, uint32_t khi,
                                      int shift) {
  if (value_bins) {
    const float d = m - x;
    return d < (float)(kBins - 1) / kBinsPerLogit ? (int)(d * kBinsPerLogit) : kBins - 1;
  }
  return (int)((khi - key) >> shift);
}

// Finds the cut of one selection.  kMass: members carry mass fixed_mass(exp(x-m))
// and the cut is where the cumulative mass first exceeds `limit`; else every
// member counts 1 and the cut is the `limit`-th largest member.
template <bool kMass, class Shared, class R, class Member>
__device__ __forceinline__ Cut select_cut(Shared& sh, const R& row, float m,
                                          unsigned long long limit, Member member) {
  uint32_t cnt_before = 0;
  unsigned long long mass_before = 0;
  uint32_t klo = 0, khi = 0xffffffffu;
  for (int pass = 0; pass < 7; ++pass) {
    const bool value_bins = pass == 0;
    sh.cnt[threadIdx.x] = 0;
    sh.mass[threadIdx.x] = 0;
    __syncthreads();
    // key bins: the smallest power-of-two width that maps [klo, khi] to <= kBins bins
    const uint32_t span = khi - klo;
    const int shift = span < (uint32_t)kBins ? 0 : 22 - __clz(span);  // bit length - 10
    row.for_chunks([&](int j) {
      if (!row.valid(j) || !member(j)) return;
      const float x = row.x(j);
      const uint32_t key = order_key(x);
      if (key < klo || key > khi) return;
      const int bin = bin_of(x, key, m, value_bins, khi, shift);
      atomicAdd(&sh.cnt[bin], 1u);
      if (kMass) atomicAdd(&sh.mass[bin], (unsigned long long)fixed_mass(expf(x - m)));
    });
    __syncthreads();
    scan_select<kMass>(sh, cnt_before, mass_before, limit);
    const int b = sh.sel_bin;
    cnt_before = sh.sel_cnt_before;
    mass_before = sh.sel_mass_before;
    const uint32_t bin_cnt = sh.sel_bin_cnt;
    const unsigned long long bin_mass = sh.sel_bin_mass;
    // key range of the crossing bin's members
    uint32_t lo = 0xffffffffu, hi = 0;
    row.for_chunks([&](int j) {
      if (!row.valid(j) || !member(j)) return;
      const float x = row.x(j);
      const uint32_t key = order_key(x);
      if (key < klo || key > khi) return;
      if (bin_of(x, key, m, value_bins, khi, shift) == b) {
        lo = min(lo, key);
        hi = max(hi, key);
      }
    });
    block_minmax(sh, lo, hi);
    klo = lo;
    khi = hi;
    if (klo == khi) {
      Cut c;
      c.key = klo;
      c.ties = bin_cnt;
      if (kMass) {
        // every tie carries the same mass; tie i (0-based) is kept while the mass
        // above it is <= limit
        const unsigned long long each = bin_mass / bin_cnt;
        const unsigned long long t = (limit - mass_before) / each + 1ull;
        c.take = t < bin_cnt ? (uint32_t)t : bin_cnt;
      } else {
        c.take = (uint32_t)limit - cnt_before;
      }
      c.partial = c.take < c.ties;
      return c;
    }
  }
  // unreachable: five key passes reduce any 32-bit range to one key
  Cut c;
  c.key = klo;
  c.take = c.ties = 0xffffffffu;
  c.partial = false;
  return c;
}

// One row (block r = blockIdx.x, logits row src_r) on the re-reading variant; sh is
// the caller's LDS.
template <int DT, int TC>
__device__ __forceinline__ void exact_row(SharedT<TC>& sh, const void* __restrict__ logits,
                                          int64_t src_r, int64_t row_stride, int V,
                                          const float* __restrict__ temperature,
                                          const int64_t* __restrict__ top_k,
                                          const float* __restrict__ top_p, int max_top_k,
                                          int apply_top_p, float* __restrict__ out,
                                          int64_t out_stride) {
  constexpr int NREG = 0, NLDS = 0, NPT = 0;
  (void)NREG;
  (void)NLDS;
  float* const xlds = nullptr;
  const int64_t r = blockIdx.x;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  Row<DT, NREG, NLDS> row;
  row.xl = xlds;
  row.V = V;
  row.src = (const char*)logits + src_r * row_stride * (DT == RLT_F32 ? 4 : 2);
  row.temp = temperature[r];
  row.npt = NPT > 0 ? NPT : (V + kThreads - 1) / kThreads;
  float* dst = out + r * out_stride;

  // x = logits / T (IEEE division, as torch), row max, NaN detection
  float m = -INFINITY;
  bool nan = false;
  row.for_chunks([&](int j) {
    float x = -INFINITY;
    if (row.valid(j)) {
      x = load_as_f32<DT>(row.src, (int64_t)j * kThreads + t) / row.temp;
      nan |= x != x;
    }
    row.set(j, x);
    m = fmaxf(m, x);
  });
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, RLT_WAVE));
  const uint64_t nan_b = __ballot(nan);
  if (lane == 0) {
    sh.wave_f64[w] = m;
    sh.wave_u32[w] = nan_b != 0;
  }
  __syncthreads();
  m = -INFINITY;
  int bad = 0;
  for (int i = 0; i < kWaves; ++i) {
    m = fmaxf(m, (float)sh.wave_f64[i]);
    bad |= sh.wave_u32[i];
  }
  __syncthreads();
  if (bad || !isfinite(m)) {
    for (int64_t i = t; i < V; i += kThreads) dst[i] = NAN;
    return;
  }

  // top-k (reference: speculative_sampling.py:39-48): keeps min(k_eff, max_top_k)
  const int64_t k_req = top_k[r];
  const int64_t k_eff = (k_req > 0 && k_req < V) ? k_req : (int64_t)V;
  Cut ck;
  ck.key = 0;
  ck.take = ck.ties = 0xffffffffu;
  ck.partial = false;
  auto all = [](int) { return true; };
  if (max_top_k > 0 && k_eff < V) {
    const int64_t kk = k_eff < (int64_t)max_top_k ? k_eff : (int64_t)max_top_k;
    ck = select_cut<false>(sh, row, m, (unsigned long long)kk, all);
    if (ck.partial) build_tie_table(sh, row, ck.key, 0, all);
  }
  // top-k survivor test of a valid element (wave-uniform: ballot inside)
  auto kept_k = [&](int j, float x) {
    const uint32_t key = order_key(x);
    if (!ck.partial) return key >= ck.key;
    const uint32_t rank = tie_rank(sh, 0, j, key == ck.key);
    return key > ck.key || (key == ck.key && rank < ck.take);
  };

  // top-p (reference: speculative_sampling.py:49-55) over the top-k survivors
  const float p = top_p[r];
  const bool do_p = apply_top_p && p < 1.f;
  Cut cp = ck;
  if (do_p) {
    // members: survivors with nonzero fixed mass (zero-mass tokens can never be
    // the crossing and sit below it); z = their total mass
    uint64_t memb = 0;
    uint32_t dummy = 0;
    unsigned long long z = 0;
    row.for_chunks([&](int j) {
      const float x = row.x(j);
      const bool in = row.valid(j) && kept_k(j, x);
      const unsigned long long fm = in ? fixed_mass(expf(x - m)) : 0ull;
      if (fm && j < 64) memb |= 1ull << j;
      z += fm;
    });
    block_sum2(sh, dummy, z);
    // kept prefix: every token whose preceding mass is <= p z (p <= 0 keeps one)
    const unsigned long long limit = p > 0.f ? (unsigned long long)((double)p * (double)z) : 0ull;
    if (NPT > 0) {
      auto member = [&](int j) { return ((memb >> j) & 1ull) != 0; };
      cp = select_cut<true>(sh, row, m, limit, member);
      if (cp.partial) build_tie_table(sh, row, cp.key, 1, member);
    } else {
      auto member = [&](int j) {
        const float x = row.x(j);
        return kept_k(j, x) && fixed_mass(expf(x - m)) != 0ull;
      };
      cp = select_cut<true>(sh, row, m, limit, member);
      if (cp.partial) build_tie_table(sh, row, cp.key, 1, member);
    }
  }

  // softmax over the kept set: everything above cp.key, the first cp.take ties
  const int which = do_p ? 1 : 0;
  auto keep_of = [&](int j, float x) {
    const uint32_t key = order_key(x);
    if (!cp.partial) return row.valid(j) && key >= cp.key;
    const uint32_t rank = tie_rank(sh, which, j, row.valid(j) && key == cp.key);
    return row.valid(j) && (key > cp.key || (key == cp.key && rank < cp.take));
  };
  double zs = 0.0;
  row.for_chunks([&](int j) {
    const float x = row.x(j);
    const float e = keep_of(j, x) ? expf(x - m) : 0.f;
    if (NPT > 0) row.set(j, e);
    zs += (double)e;
  });
  const float inv = 1.f / (float)block_sum_f64(sh, zs);
  row.for_chunks([&](int j) {
    float e;
    if (NPT > 0) {
      e = row.x(j);
    } else {
      const float x = row.x(j);
      e = keep_of(j, x) ? expf(x - m) : 0.f;
    }
    if (row.valid(j)) dst[(int64_t)j * kThreads + t] = e * inv;
  });
}

}  // namespace exact
