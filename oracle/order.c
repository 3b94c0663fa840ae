/*
 * Independent C model of the two torch-CPU summation orders that the
 * bit-exact acceptance contract rests on.  TEST INFRASTRUCTURE ONLY.
 *
 * 1. fp32 row sum, ``Tensor.sum(-1, dtype=torch.float32)`` on a contiguous
 *    row of a multi-row tensor (called at
 *    vllm_rlt/worker/speculative_sampling.py:138,146).  torch 2.x routes it to
 *    its cascade-sum kernel compiled for 8-wide fp32 vectors (the AVX2 build,
 *    also used on AVX512 hosts): the row is read as vectors of 8 lanes, four
 *    vectors per step (ILP 4), giving 32 independent streams; stream
 *    s = 8*k + l owns elements 32*i + s.  Each stream is summed with a
 *    4-level cascade whose level step is 2^max(4, ceil_log2(steps)/4): 16
 *    consecutive elements into level 0, flushed into level 1 after every
 *    chunk, level 1 into level 2 every 16 chunks, level 2 into level 3 every
 *    256 chunks; the remainder of the stream goes into level 0 and the four
 *    levels are added in order.  Leftover whole vectors are added lane-wise
 *    into the first ILP accumulator, the four ILP accumulators are added
 *    lane-wise, then a scalar starts at 0, adds the leftover scalar tail in
 *    order and then the 8 lanes in order.  Rows shorter than 8 take the
 *    scalar form of the same ILP-4 cascade.
 * 2. fp32 sum of a whole 1-D tensor (``oracle_sum_1d_f32``): the same row
 *    cascade over thread chunks, then over the per-thread partials.
 * 3. categorical draw (speculative_sampling.py:74-84): sequential float64
 *    cumsum from 0, mass = last entry, valid = finite and > 0,
 *    t = min(u * mass, nextafter(mass, 0)), index = torch's upper_bound
 *    binary search over the cdf, 0 when invalid, clamped to [0, V - 1].
 *
 * tests/test_oracle_order.py checks both models against torch bit for bit on
 * random, skewed, subnormal and non-finite rows.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static int64_t ceil_log2(int64_t x) {
    if (x <= 2) return 1;
    int64_t r = 0;
    uint64_t v = (uint64_t)(x - 1);
    while (v) { r++; v >>= 1; }
    return r;
}

/* Cascade over `size` steps of `width` parallel accumulators; element for
 * (step i, accumulator a) is x[i * step_stride + a].  Result in out[a]. */
static void cascade(const float *x, int64_t size, int64_t step_stride, int width, float *out) {
    float acc[4][32];
    memset(acc, 0, sizeof(acc));
    int64_t lp = ceil_log2(size) / 4;
    if (lp < 4) lp = 4;
    const int64_t step = (int64_t)1 << lp, mask = step - 1;
    int64_t i = 0;
    while (i + step <= size) {
        for (int64_t j = 0; j < step; ++j, ++i)
            for (int a = 0; a < width; ++a) acc[0][a] += x[i * step_stride + a];
        for (int j = 1; j < 4; ++j) {
            for (int a = 0; a < width; ++a) { acc[j][a] += acc[j - 1][a]; acc[j - 1][a] = 0.0f; }
            if (i & (mask << (j * lp))) break;
        }
    }
    for (; i < size; ++i)
        for (int a = 0; a < width; ++a) acc[0][a] += x[i * step_stride + a];
    for (int j = 1; j < 4; ++j)
        for (int a = 0; a < width; ++a) acc[0][a] += acc[j][a];
    for (int a = 0; a < width; ++a) out[a] = acc[0][a];
}

float oracle_row_sum_f32(const float *x, int64_t n) {
    if (n < 8) {
        /* scalar ILP-4 form: 4 streams of stride-4 scalars */
        float ps[4] = {0, 0, 0, 0};
        int64_t si = n / 4;
        if (si > 0) cascade(x, si, 4, 4, ps);
        for (int64_t i = si * 4; i < n; ++i) ps[0] += x[i];
        return ((ps[0] + ps[1]) + ps[2]) + ps[3];
    }
    const int64_t vs = n / 8, si = vs / 4;
    float st[32];
    memset(st, 0, sizeof(st));
    if (si > 0) cascade(x, si, 32, 32, st);
    for (int64_t v = si * 4; v < vs; ++v)
        for (int l = 0; l < 8; ++l) st[l] += x[v * 8 + l];
    float lanes[8];
    for (int l = 0; l < 8; ++l) lanes[l] = ((st[l] + st[8 + l]) + st[16 + l]) + st[24 + l];
    float f = 0.0f;
    for (int64_t e = vs * 8; e < n; ++e) f += x[e];
    for (int l = 0; l < 8; ++l) f += lanes[l];
    return f;
}

/* fp32 sum of a whole 1-D tensor, ``x.sum()`` (the residual total at
 * vllm_rlt/worker/speculative.py:66).  torch reduces a contiguous tensor to one
 * value serially when it has fewer than 32768 elements or one thread; otherwise
 * it splits it into c = min(threads, ceil(n / 32768)) chunks of ceil(n / c)
 * elements, sums each chunk with the row cascade into its own slot of a
 * `threads`-long zero buffer, and reduces that buffer with the row cascade.
 * The output starts at 0 and accumulates (0 + sum). */
float oracle_sum_1d_f32(const float *x, int64_t n, int threads) {
    const int64_t grain = 32768;
    if (n < grain || threads <= 1) return 0.0f + oracle_row_sum_f32(x, n);
    int64_t chunks = (n + grain - 1) / grain;
    if (chunks > threads) chunks = threads;
    const int64_t size = (n + chunks - 1) / chunks;
    float buf[1024];
    if (threads > 1024) return NAN;
    for (int i = 0; i < threads; ++i) buf[i] = 0.0f;
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t b = c * size;
        if (b >= n) break;
        const int64_t e = b + size < n ? b + size : n;
        buf[c] = 0.0f + oracle_row_sum_f32(x + b, e - b);
    }
    return 0.0f + oracle_row_sum_f32(buf, threads);
}

void oracle_row_sums_f32(const float *x, int64_t rows, int64_t n, float *out) {
    for (int64_t r = 0; r < rows; ++r) out[r] = oracle_row_sum_f32(x + r * n, n);
}

/* Sequential float64 prefix sum up to and including index k. */
static double prefix(const float *w, int64_t k) {
    double c = 0.0;
    for (int64_t i = 0; i <= k; ++i) c += (double)w[i];
    return c;
}

int64_t oracle_categorical(const float *w, int64_t n, float u, uint8_t *valid_out) {
    double mass = prefix(w, n - 1);
    int valid = isfinite(mass) && mass > 0.0;
    *valid_out = (uint8_t)valid;
    double t = (double)u * mass;
    double below = nextafter(mass, 0.0);
    /* torch.minimum propagates NaN from either side */
    if (isnan(t) || isnan(below)) t = NAN; else if (below < t) t = below;
    /* upper_bound: first index whose cdf value is > t */
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        int64_t mid = lo + ((hi - lo) >> 1);
        if (!(prefix(w, mid) > t)) lo = mid + 1; else hi = mid;
    }
    int64_t idx = valid ? lo : 0;
    if (idx < 0) idx = 0;
    if (idx > n - 1) idx = n - 1;
    return idx;
}

void oracle_categorical_rows(const float *w, int64_t rows, int64_t n, const float *u,
                             int64_t *idx, uint8_t *valid) {
    for (int64_t r = 0; r < rows; ++r) idx[r] = oracle_categorical(w + r * n, n, u[r], valid + r);
}
