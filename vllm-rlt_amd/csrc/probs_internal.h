// Internal interface between the two sampling-distribution kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Written by rlt_probs_kernel into the first output element of a row it hands
// over to rlt_probs_exact_kernel (a NaN payload no computed output carries: NaN
// rows are written with the canonical NaN).
constexpr uint32_t kCrowdedRowMark = 0x7fc0c0deu;

// Launches rlt_probs_exact_kernel over n rows (the arguments of
// rlt_batched_probabilities); rows without the marker return at once.
void rlt_probs_exact_launch(int32_t dtype, int64_t n, const void* logits, int64_t row_stride,
                            int V, const float* temperature, const int64_t* top_k,
                            const float* top_p, int max_top_k, int apply_top_p, float* out,
                            int64_t out_stride, hipStream_t stream);
