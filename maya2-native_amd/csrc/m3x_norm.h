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

// Per-head q/k RMSNorm + RoPE of one head row (serve/fast_backbone.py:61-92, rounding points :77-81), for the D/8
// threads that hold it, thread t holding elements 8t .. 8t+7 (x: the bf16 values of the projection, as floats):
//   y = bf16(bf16(x * inv) * w);  first half: o = y*c - y'*s;  second half: o = y*c + y'*s  (y' = rotate partner)
// For D = 128 the 16 threads must be one DPP row (lanes 16k .. 16k+15); for D = 64, 8 adjacent lanes. Every
// thread of those lanes calls it (the reductions are lane exchanges).
template <int D>
__device__ __forceinline__ u16x8 qk_norm_rope8(const float (&x)[8], const u16x8& wv, const u16x8& cv, const u16x8& sv,
                                               float eps, int t) {
  constexpr int TPI = D / 8;
  float p = x[0] * x[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) p = p + x[e] * x[e];
  if constexpr (TPI == 16) {
    p = dppf<DPP_ROW_NEWBCAST(0)>(fold_half_sum<16>(p));  // one DPP row per head: its total, from its first lane
  } else {
#pragma unroll
    for (int s = TPI / 2; s > 0; s >>= 1) p = p + __shfl_xor(p, s, 64);
  }
  const float inv = 1.0f / sqrtf(p / (float)D + eps);
  float yv[8], yp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) yv[e] = bf2f(f2bf(bf2f(f2bf(x[e] * inv)) * bf2f(wv.v[e])));
#pragma unroll
  for (int e = 0; e < 8; ++e)  // the rotate partner, lane t ^ TPI/2
    yp[e] = TPI == 16 ? dppf<DPP_ROW_ROR(8)>(yv[e]) : __shfl_xor(yv[e], TPI / 2, 64);
  const bool first = t < TPI / 2;
  u16x8 ov;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float a1 = yv[e] * bf2f(cv.v[e]);
    float a2 = yp[e] * bf2f(sv.v[e]);
    ov.v[e] = f2bf(first ? a1 - a2 : a1 + a2);
  }
  return ov;
}
