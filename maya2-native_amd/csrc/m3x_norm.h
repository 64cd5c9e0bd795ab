// Row normalisation shared by the norm kernels and the depth sampler's fused next-level input.
//
// Reduction order (the one the C oracle restates; bit-exactness depends on it): a row of N elements is read
// as N/8 groups of 8 contiguous elements, one group per thread. A thread sums its 8 terms left to right
// (each product and each sum rounded to fp32), then the N/8 partials are folded in half repeatedly:
// p[g] = p[g] + p[g + s] for s = N/16, N/32, ..., 1. Folds across waves go through LDS; within a wave the fold
// runs on permlane swaps (s = 32, 16) and DPP row shifts (s <= 8), which give lane g < s exactly
// p[g] + p[g + s] (fold_half_sum).
#pragma once
#include "m3x_common.h"

enum { M3X_NORM_LAYER = 0, M3X_NORM_RMS = 1 };

// fold-in-half tree over TPR threads per row; rows are packed 256/TPR per block. Returns the row total in
// every thread of the row. Every thread of the block calls it (it holds block barriers).
template <int TPR>
__device__ __forceinline__ float row_tree_sum(float p, float* red, float* bcast) {
  const int t = threadIdx.x % TPR;
  const int rb = threadIdx.x / TPR;
  if constexpr (TPR > 64) {
    red[threadIdx.x] = p;
    __syncthreads();
#pragma unroll
    for (int s = TPR / 2; s >= 64; s >>= 1) {
      if (t < s) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + s];
      __syncthreads();
    }
    p = red[threadIdx.x];
  }
  p = fold_half_sum<(TPR < 64 ? TPR : 64)>(p);
  if (t == 0) bcast[rb] = p;
  __syncthreads();
  float r = bcast[rb];
  __syncthreads();
  return r;
}

// y for one thread's 8 elements v of a row of N = 8*TPR (serve/fast_depth_kernels.py:14-45 _add_ln and its RMS
// twin):
//   LayerNorm  y = dt((v - mean) / sqrt(var + eps) * w + b)   (mean, var over the row, fp32)
//   RMSNorm    y = dt(dt(v * (1 / sqrt(mean(v^2) + eps))) * w)
// Threads of inactive rows pass v = 0 and discard the result. Every thread of the block calls it.
template <int TPR, int DT>
__device__ __forceinline__ V8<DT> norm_vec(const float (&v)[8], const V8<DT>& wv, const V8<DT>& bv, int kind, float eps,
                                          float* red, float* bcast) {
  constexpr int N = TPR * 8;
  V8<DT> yv;
  float p;
  if (kind == M3X_NORM_LAYER) {
    p = v[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p = p + v[e];
    const float mean = row_tree_sum<TPR>(p, red, bcast) / (float)N;
    float d[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = v[e] - mean;
    p = d[0] * d[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p = p + d[e] * d[e];
    const float var = row_tree_sum<TPR>(p, red, bcast) / (float)N;
    const float sd = sqrtf(var + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) yv.v[e] = E<DT>::from_f(d[e] / sd * E<DT>::to_f(wv.v[e]) + E<DT>::to_f(bv.v[e]));
  } else {
    p = v[0] * v[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p = p + v[e] * v[e];
    const float ss = row_tree_sum<TPR>(p, red, bcast);
    const float inv = 1.0f / sqrtf(ss / (float)N + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) yv.v[e] = E<DT>::from_f(rnd<DT>(v[e] * inv) * E<DT>::to_f(wv.v[e]));
  }
  return yv;
}
