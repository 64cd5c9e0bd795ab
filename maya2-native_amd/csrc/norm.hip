// Row-normalisation kernels of the frame step.
//
// The reduction order every kernel here follows (row_tree_sum, m3x_norm.h) is the one the C oracle restates.
#include "m3x_norm.h"

// ---------------------------------------------------------------------------------------------------------
// K3: h' = bf16(h + a); y = bf16(bf16(h' * (1/sqrt(mean(h'^2) + eps))) * w).  a == nullptr: plain RMSNorm of h.
// serve/fast_backbone.py:95-104 (_add_rms) and HF Qwen3RMSNorm for the layer-0 input norm (:190).
template <int TPR>
__global__ __launch_bounds__(256) void add_rms_kernel(const uint16_t* __restrict__ h, long s_h,
                                                      const uint16_t* __restrict__ a, long s_a, uint16_t* ho,
                                                      long s_ho, uint16_t* __restrict__ y, long s_y,
                                                      const uint16_t* __restrict__ w, float eps, int rows) {
  constexpr int N = TPR * 8;
  constexpr int RPB = 256 / TPR;
  __shared__ float red[TPR > 64 ? 256 : 1];
  __shared__ float bcast[RPB];
  const int t = threadIdx.x % TPR;
  const int row = blockIdx.x * RPB + threadIdx.x / TPR;
  const bool active = row < rows;
  float x[8];
  float p = 0.f;
  u16x8 wv;
  if (active) {
    u16x8 hv = ld16(h + (long)row * s_h + 8 * t);
    u16x8 av;
    if (a) av = ld16(a + (long)row * s_a + 8 * t);
    wv = ld16(w + 8 * t);  // after the row's loads: it arrives while the reduction runs
    if (a) {
      u16x8 sv;
#pragma unroll
      for (int e = 0; e < 8; ++e) sv.v[e] = f2bf(bf2f(hv.v[e]) + bf2f(av.v[e]));
      if (ho) st16(ho + (long)row * s_ho + 8 * t, sv);
      hv = sv;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = bf2f(hv.v[e]);
    p = x[0] * x[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p = p + x[e] * x[e];
  }
  float ss = row_tree_sum<TPR>(p, red, bcast);
  if (!active) return;
  const float inv = 1.0f / sqrtf(ss / (float)N + eps);
  u16x8 yv;
#pragma unroll
  for (int e = 0; e < 8; ++e) yv.v[e] = f2bf(bf2f(f2bf(x[e] * inv)) * bf2f(wv.v[e]));
  st16(y + (long)row * s_y + 8 * t, yv);
}

// Row counts up to which the one-wave-per-row kernels run (measured: below it they save a block barrier chain).
constexpr int WAVE_ROWS_MAX = 16;

// ---------------------------------------------------------------------------------------------------------
// One wave per row of 1024, for a handful of rows (a one-row step is a chain of launches, and a lone row needs
// no block barrier): lane l holds groups l and l + 64 (8 elements each), whose partials it adds as the first
// fold (s = 64) of the same fold-in-half tree; the rest of the tree is fold_half_sum and lane 0's total is read
// back with readlane. Same arithmetic, so the same bits, as the block kernels.
template <int DT>
__device__ __forceinline__ float wave_row_total(float p) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fold_half_sum<64>(p)), 0));
}
template <int DT>
__device__ __forceinline__ void norm_pair_wave(const float (&v0)[8], const float (&v1)[8], const V8<DT>& w0,
                                               const V8<DT>& w1, const V8<DT>& b0, const V8<DT>& b1, int kind, float eps,
                                               V8<DT>& y0, V8<DT>& y1) {
  constexpr float N = 1024.0f;
  if (kind == M3X_NORM_LAYER) {
    float p0 = v0[0], p1 = v1[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p0 = p0 + v0[e], p1 = p1 + v1[e];
    const float mean = wave_row_total<DT>(p0 + p1) / N;
    float d0[8], d1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) d0[e] = v0[e] - mean, d1[e] = v1[e] - mean;
    p0 = d0[0] * d0[0];
    p1 = d1[0] * d1[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p0 = p0 + d0[e] * d0[e], p1 = p1 + d1[e] * d1[e];
    const float var = wave_row_total<DT>(p0 + p1) / N;
    const float sd = sqrtf(var + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y0.v[e] = E<DT>::from_f(d0[e] / sd * E<DT>::to_f(w0.v[e]) + E<DT>::to_f(b0.v[e]));
      y1.v[e] = E<DT>::from_f(d1[e] / sd * E<DT>::to_f(w1.v[e]) + E<DT>::to_f(b1.v[e]));
    }
  } else {
    float p0 = v0[0] * v0[0], p1 = v1[0] * v1[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p0 = p0 + v0[e] * v0[e], p1 = p1 + v1[e] * v1[e];
    const float inv = 1.0f / sqrtf(wave_row_total<DT>(p0 + p1) / N + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y0.v[e] = E<DT>::from_f(rnd<DT>(v0[e] * inv) * E<DT>::to_f(w0.v[e]));
      y1.v[e] = E<DT>::from_f(rnd<DT>(v1[e] * inv) * E<DT>::to_f(w1.v[e]));
    }
  }
}

// add_rms_kernel's contract for n = 1024, one 64-thread workgroup per row.
__global__ __launch_bounds__(64) void add_rms_wave_kernel(const uint16_t* __restrict__ h, long s_h,
                                                          const uint16_t* __restrict__ a, long s_a, uint16_t* ho,
                                                          long s_ho, uint16_t* __restrict__ y, long s_y,
                                                          const uint16_t* __restrict__ w, float eps) {
  const long row = blockIdx.x;
  const int l = threadIdx.x;
  u16x8 h0 = ld16(h + row * s_h + 8 * l), h1 = ld16(h + row * s_h + 8 * (l + 64));
  u16x8 a0, a1;
  if (a) a0 = ld16(a + row * s_a + 8 * l), a1 = ld16(a + row * s_a + 8 * (l + 64));
  const u16x8 w0 = ld16(w + 8 * l), w1 = ld16(w + 8 * (l + 64));
  if (a) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h0.v[e] = f2bf(bf2f(h0.v[e]) + bf2f(a0.v[e]));
      h1.v[e] = f2bf(bf2f(h1.v[e]) + bf2f(a1.v[e]));
    }
    if (ho) st16(ho + row * s_ho + 8 * l, h0), st16(ho + row * s_ho + 8 * (l + 64), h1);
  }
  float v0[8], v1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v0[e] = bf2f(h0.v[e]), v1[e] = bf2f(h1.v[e]);
  u16x8 y0, y1;
  norm_pair_wave<M3X_BF16>(v0, v1, w0, w1, w0, w1, M3X_NORM_RMS, eps, y0, y1);
  st16(y + row * s_y + 8 * l, y0);
  st16(y + row * s_y + 8 * (l + 64), y1);
}

M3X_API int m3x_add_rms(const void* h, long s_h, const void* a, long s_a, void* h_out, long s_ho, void* y, long s_y,
                        const void* w, float eps, int rows, int n, void* stream) {
  if (rows < 0) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!h || !y || !w) return M3X_ENULL;
  if ((s_h | s_y | (a ? s_a : 0) | (h_out ? s_ho : 0)) & 7) return M3X_EINVAL;
  if (!m3x_aligned16(h) || !m3x_aligned16(y) || !m3x_aligned16(w) || (a && !m3x_aligned16(a)) ||
      (h_out && !m3x_aligned16(h_out)))
    return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *H = (const uint16_t*)h, *A = (const uint16_t*)a, *Wt = (const uint16_t*)w;
  uint16_t *HO = (uint16_t*)h_out, *Y = (uint16_t*)y;
  if (n == 1024 && rows <= WAVE_ROWS_MAX) {
    hipLaunchKernelGGL(add_rms_wave_kernel, dim3(rows), dim3(64), 0, st, H, s_h, A, s_a, HO, s_ho, Y, s_y, Wt, eps);
    M3X_CHECK_LAUNCH();
    return M3X_OK;
  }
  switch (n) {
#define M3X_ADD_RMS_CASE(NN)                                                                                   \
  case NN: {                                                                                                   \
    constexpr int TPR = NN / 8;                                                                                \
    hipLaunchKernelGGL(add_rms_kernel<TPR>, dim3(m3x_ceil_div(rows, 256 / TPR)), dim3(256), 0, st, H, s_h, A, \
                       s_a, HO, s_ho, Y, s_y, Wt, eps, rows);                                                  \
    break;                                                                                                     \
  }
    M3X_ADD_RMS_CASE(512)
    M3X_ADD_RMS_CASE(1024)
    M3X_ADD_RMS_CASE(2048)
#undef M3X_ADD_RMS_CASE
    default:
      return M3X_EUNSUPPORTED;
  }
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// K2: per-head q/k RMSNorm + RoPE, query heads to q_out, key heads into the static cache at [slot, kh, pos],
// value heads copied verbatim. serve/fast_backbone.py:61-92 (_qk_norm_rope_cache), rounding points :77-81.
// One item = (row, j) with j < H a query head and H <= j < H+KV a key head; D/8 threads per item (qk_norm_rope8).
template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_cache_kernel(
    const uint16_t* __restrict__ qkv, long s_qkv, uint16_t* __restrict__ qo, long s_qo_b, long s_qo_h,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, long sk_s, long sk_h, long sk_t,
    const int64_t* __restrict__ slots, const int32_t* __restrict__ pos, const uint16_t* __restrict__ cosb,
    const uint16_t* __restrict__ sinb, long s_cos, const uint16_t* __restrict__ wq, const uint16_t* __restrict__ wk,
    float eps, int rows, int H, int KV, int cap) {
  constexpr int TPI = D / 8;  // threads per item
  constexpr int IPB = 256 / TPI;
  const int t = threadIdx.x % TPI;
  const long item = (long)blockIdx.x * IPB + threadIdx.x / TPI;
  const int NH = H + KV;
  const int row = (int)(item / NH);
  const int j = (int)(item % NH);
  const bool active = row < rows;
  // Every load is issued up front from clamped (valid) addresses, so one memory latency covers them all;
  // only cos/sin wait for the position. Inactive items compute on row 0 and store nothing.
  const int r = active ? row : 0;
  // the host guarantees 0 <= pos < cap; the clamp keeps the cache write inside the slot's rows whatever pos holds
  const int ps = min(max(pos[r], 0), cap - 1);
  const long slot = slots[r];
  const u16x8 xv = ld16(qkv + (long)r * s_qkv + (long)j * D + 8 * t);
  const u16x8 wv = ld16((j < H ? wq : wk) + 8 * t);
  const int kh = j < H ? 0 : j - H;
  const u16x8 vv = ld16(qkv + (long)r * s_qkv + (long)(H + KV + kh) * D + 8 * t);
  const u16x8 cv = ld16(cosb + (long)ps * s_cos + 8 * t);
  const u16x8 sv = ld16(sinb + (long)ps * s_cos + 8 * t);
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = bf2f(xv.v[e]);
  const u16x8 ov = qk_norm_rope8<D>(x, wv, cv, sv, eps, t);
  if (!active) return;
  if (j < H) {
    st16(qo + (long)row * s_qo_b + (long)j * s_qo_h + 8 * t, ov);
  } else {
    const long off = slot * sk_s + (long)kh * sk_h + (long)ps * sk_t + 8 * t;
    st16(kc + off, ov);
    st16(vc + off, vv);
  }
}

M3X_API int m3x_qk_norm_rope_cache(const void* qkv, long s_qkv, void* q_out, long s_qo_b, long s_qo_h, void* k_cache,
                                   void* v_cache, long sk_s, long sk_h, long sk_t, const int64_t* slots,
                                   const int32_t* pos, const void* cos, const void* sin, long s_cos, const void* wq,
                                   const void* wk, float eps, int rows, int heads, int kv_heads, int head_dim,
                                   int cap, void* stream) {
  if (rows < 0 || heads <= 0 || kv_heads <= 0 || cap <= 0) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!qkv || !q_out || !k_cache || !v_cache || !slots || !pos || !cos || !sin || !wq || !wk) return M3X_ENULL;
  if ((s_qkv | s_qo_b | s_qo_h | sk_s | sk_h | sk_t | s_cos) & 7) return M3X_EINVAL;
  if (!m3x_aligned16(qkv) || !m3x_aligned16(q_out) || !m3x_aligned16(k_cache) || !m3x_aligned16(v_cache) ||
      !m3x_aligned16(cos) || !m3x_aligned16(sin) || !m3x_aligned16(wq) || !m3x_aligned16(wk))
    return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const long items = (long)rows * (heads + kv_heads);
#define M3X_QKN_ARGS                                                                                              \
  (const uint16_t*)qkv, s_qkv, (uint16_t*)q_out, s_qo_b, s_qo_h, (uint16_t*)k_cache, (uint16_t*)v_cache, sk_s, sk_h, \
      sk_t, slots, pos, (const uint16_t*)cos, (const uint16_t*)sin, s_cos, (const uint16_t*)wq, (const uint16_t*)wk,  \
      eps, rows, heads, kv_heads, cap
  if (head_dim == 128) {
    hipLaunchKernelGGL(qk_norm_rope_cache_kernel<128>, dim3(m3x_ceil_div(items, 16)), dim3(256), 0, st, M3X_QKN_ARGS);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL(qk_norm_rope_cache_kernel<64>, dim3(m3x_ceil_div(items, 32)), dim3(256), 0, st, M3X_QKN_ARGS);
  } else {
    return M3X_EUNSUPPORTED;
  }
#undef M3X_QKN_ARGS
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Depth residual + norm: x' = dt(x + a) [then dt(x' + c[row / T])]; x' stored to xo (if given);
// y = LayerNorm(x') (fp32 statistics, affine w/b) or RMSNorm(x') (bf16(bf16(x*inv)*w), Qwen3 convention).
// serve/fast_depth_kernels.py:14-45 (_add_ln); the RMS variant serves the SwiGLU/RMSNorm depth trunk.
// a == nullptr: x' = x (plain norm of the input, serve/fast_depth.py:164).

template <int TPR, int DT>
__global__ __launch_bounds__(256) void add_norm_kernel(const Elt<DT>* __restrict__ x, long sxb, long sxt,
                                                       const Elt<DT>* __restrict__ a, long sab, long sat,
                                                       const Elt<DT>* __restrict__ c, long s_c, Elt<DT>* xo,
                                                       Elt<DT>* __restrict__ y, const Elt<DT>* __restrict__ w,
                                                       const Elt<DT>* __restrict__ b, float eps, int rows, int T,
                                                       int kind) {
  constexpr int N = TPR * 8;
  constexpr int RPB = 256 / TPR;
  __shared__ float red[TPR > 64 ? 256 : 1];
  __shared__ float bcast[RPB];
  const int t = threadIdx.x % TPR;
  const int row = blockIdx.x * RPB + threadIdx.x / TPR;
  const bool active = row < rows;
  const int rb = active ? row / T : 0, rt = active ? row % T : 0;
  float v[8];
  V8<DT> wv = zero_v8<DT>(), bv = zero_v8<DT>();
  if (active) {
    V8<DT> xv = ldv<DT>(x + rb * sxb + rt * sxt + 8 * t);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = E<DT>::to_f(xv.v[e]);
    if (a) {
      V8<DT> av = ldv<DT>(a + rb * sab + rt * sat + 8 * t);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = rnd<DT>(v[e] + E<DT>::to_f(av.v[e]));
    }
    if (c) {
      V8<DT> cv = ldv<DT>(c + (long)rb * s_c + 8 * t);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = rnd<DT>(v[e] + E<DT>::to_f(cv.v[e]));
    }
    // affine parameters after the row's own loads: they arrive while the reductions run
    wv = ldv<DT>(w + 8 * t);
    if (kind == M3X_NORM_LAYER) bv = ldv<DT>(b + 8 * t);
    if (xo) {
      V8<DT> ov;
#pragma unroll
      for (int e = 0; e < 8; ++e) ov.v[e] = E<DT>::from_f(v[e]);
      stv<DT>(xo + (long)row * N + 8 * t, ov);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
  }
  const V8<DT> yv = norm_vec<TPR, DT>(v, wv, bv, kind, eps, red, bcast);
  if (!active) return;
  stv<DT>(y + (long)row * N + 8 * t, yv);
}

// add_norm_kernel's contract for n = 1024, one 64-thread workgroup per row.
template <int DT>
__global__ __launch_bounds__(64) void add_norm_wave_kernel(const Elt<DT>* __restrict__ x, long sxb, long sxt,
                                                           const Elt<DT>* __restrict__ a, long sab, long sat,
                                                           const Elt<DT>* __restrict__ c, long s_c, Elt<DT>* xo,
                                                           Elt<DT>* __restrict__ y, const Elt<DT>* __restrict__ w,
                                                           const Elt<DT>* __restrict__ b, float eps, int T,
                                                           int kind) {
  const int row = blockIdx.x;
  const int l = threadIdx.x;
  const long rb = row / T, rt = row % T;
  const Elt<DT>* xr = x + rb * sxb + rt * sxt;
  V8<DT> x0 = ldv<DT>(xr + 8 * l), x1 = ldv<DT>(xr + 8 * (l + 64));
  V8<DT> a0, a1, c0, c1, b0 = zero_v8<DT>(), b1 = zero_v8<DT>();
  if (a) a0 = ldv<DT>(a + rb * sab + rt * sat + 8 * l), a1 = ldv<DT>(a + rb * sab + rt * sat + 8 * (l + 64));
  if (c) c0 = ldv<DT>(c + rb * s_c + 8 * l), c1 = ldv<DT>(c + rb * s_c + 8 * (l + 64));
  const V8<DT> w0 = ldv<DT>(w + 8 * l), w1 = ldv<DT>(w + 8 * (l + 64));
  if (kind == M3X_NORM_LAYER) b0 = ldv<DT>(b + 8 * l), b1 = ldv<DT>(b + 8 * (l + 64));
  float v0[8], v1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v0[e] = E<DT>::to_f(x0.v[e]);
    v1[e] = E<DT>::to_f(x1.v[e]);
    if (a) v0[e] = rnd<DT>(v0[e] + E<DT>::to_f(a0.v[e])), v1[e] = rnd<DT>(v1[e] + E<DT>::to_f(a1.v[e]));
    if (c) v0[e] = rnd<DT>(v0[e] + E<DT>::to_f(c0.v[e])), v1[e] = rnd<DT>(v1[e] + E<DT>::to_f(c1.v[e]));
  }
  if (xo) {
    V8<DT> o0, o1;
#pragma unroll
    for (int e = 0; e < 8; ++e) o0.v[e] = E<DT>::from_f(v0[e]), o1.v[e] = E<DT>::from_f(v1[e]);
    stv<DT>(xo + (long)row * 1024 + 8 * l, o0);
    stv<DT>(xo + (long)row * 1024 + 8 * (l + 64), o1);
  }
  V8<DT> y0, y1;
  norm_pair_wave<DT>(v0, v1, w0, w1, b0, b1, kind, eps, y0, y1);
  stv<DT>(y + (long)row * 1024 + 8 * l, y0);
  stv<DT>(y + (long)row * 1024 + 8 * (l + 64), y1);
}

template <int DT>
static bool launch_add_norm(const void* x, long sxb, long sxt, const void* a, long sab, long sat, const void* c,
                            long s_c, void* x_out, void* y, const void* w, const void* b, float eps, int rows, int T,
                            int n, int kind, hipStream_t st) {
  const Elt<DT> *X = (const Elt<DT>*)x, *A = (const Elt<DT>*)a, *C = (const Elt<DT>*)c;
  const Elt<DT> *Wt = (const Elt<DT>*)w, *Bt = (const Elt<DT>*)b;
  Elt<DT> *XO = (Elt<DT>*)x_out, *Y = (Elt<DT>*)y;
  if (n == 1024 && rows <= WAVE_ROWS_MAX) {
    hipLaunchKernelGGL(add_norm_wave_kernel<DT>, dim3(rows), dim3(64), 0, st, X, sxb, sxt, A, sab, sat, C, s_c, XO, Y,
                       Wt, Bt, eps, T, kind);
    return true;
  }
#define M3X_ADD_NORM_LAUNCH(NN)                                                                                  \
  hipLaunchKernelGGL((add_norm_kernel<NN / 8, DT>), dim3(m3x_ceil_div(rows, 256 / (NN / 8))), dim3(256), 0, st, X, \
                     sxb, sxt, A, sab, sat, C, s_c, XO, Y, Wt, Bt, eps, rows, T, kind)
  if (n == 512) M3X_ADD_NORM_LAUNCH(512);
  else if (n == 1024) M3X_ADD_NORM_LAUNCH(1024);
  else if (n == 2048) M3X_ADD_NORM_LAUNCH(2048);
  else return false;
#undef M3X_ADD_NORM_LAUNCH
  return true;
}

// Row r = (b, t) = (r / T, r % T) of x is read at x + b*sxb + t*sxt (likewise a); x_out and y are contiguous
// [rows, n]; c is indexed by b with stride s_c (s_c = 0 broadcasts one vector).
M3X_API int m3x_add_norm(const void* x, long sxb, long sxt, const void* a, long sab, long sat, const void* c, long s_c,
                         void* x_out, void* y, const void* w, const void* b, float eps, int rows, int T, int n,
                         int kind, int dtype, void* stream) {
  if (rows < 0 || T <= 0) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!x || !y || !w) return M3X_ENULL;
  if (kind == M3X_NORM_LAYER && !b) return M3X_ENULL;
  if (kind != M3X_NORM_LAYER && kind != M3X_NORM_RMS) return M3X_EINVAL;
  if ((sxb | sxt | (a ? (sab | sat) : 0) | (c ? s_c : 0)) & 7) return M3X_EINVAL;
  if (!m3x_aligned16(x) || !m3x_aligned16(y) || !m3x_aligned16(w) || (a && !m3x_aligned16(a)) ||
      (c && !m3x_aligned16(c)) || (x_out && !m3x_aligned16(x_out)) || (b && !m3x_aligned16(b)))
    return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  bool ok;
  if (dtype == M3X_BF16)
    ok = launch_add_norm<M3X_BF16>(x, sxb, sxt, a, sab, sat, c, s_c, x_out, y, w, b, eps, rows, T, n, kind, st);
  else if (dtype == M3X_F16)
    ok = launch_add_norm<M3X_F16>(x, sxb, sxt, a, sab, sat, c, s_c, x_out, y, w, b, eps, rows, T, n, kind, st);
  else if (dtype == M3X_F32)
    ok = launch_add_norm<M3X_F32>(x, sxb, sxt, a, sab, sat, c, s_c, x_out, y, w, b, eps, rows, T, n, kind, st);
  else
    return M3X_EUNSUPPORTED;
  if (!ok) return M3X_EUNSUPPORTED;
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// out[r] = dt(x[r] + bias[r * ld_bias]) for rows of n elements (ld_bias = 0 broadcasts one vector).
// Replaces `d.in_proj(h) + self.level0` (serve/fast_depth.py:150).
template <int DT>
__global__ __launch_bounds__(256) void add_rows_kernel(const Elt<DT>* __restrict__ x, long ld_x,
                                                       const Elt<DT>* __restrict__ bias, long ld_b,
                                                       Elt<DT>* __restrict__ out, long ld_o, int rows, int nvec) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)rows * nvec) return;
  const int r = (int)(i / nvec), v = (int)(i % nvec);
  V8<DT> xv = ldv<DT>(x + r * ld_x + 8 * v), bv = ldv<DT>(bias + r * ld_b + 8 * v), ov;
#pragma unroll
  for (int e = 0; e < 8; ++e) ov.v[e] = E<DT>::from_f(E<DT>::to_f(xv.v[e]) + E<DT>::to_f(bv.v[e]));
  stv<DT>(out + r * ld_o + 8 * v, ov);
}

M3X_API int m3x_add_rows(const void* x, long ld_x, const void* bias, long ld_bias, void* out, long ld_out, int rows,
                         int n, int dtype, void* stream) {
  if (rows < 0 || n <= 0 || (n & 7) || ((ld_x | ld_bias | ld_out) & 7)) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!x || !bias || !out) return M3X_ENULL;
  if (!m3x_aligned16(x) || !m3x_aligned16(bias) || !m3x_aligned16(out)) return M3X_EINVAL;
  const long total = (long)rows * (n / 8);
  hipStream_t st = (hipStream_t)stream;
#define M3X_ADD_ROWS(DTT)                                                                                 \
  hipLaunchKernelGGL(add_rows_kernel<DTT>, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, st, (const Elt<DTT>*)x, \
                     ld_x, (const Elt<DTT>*)bias, ld_bias, (Elt<DTT>*)out, ld_out, rows, n / 8)
  if (dtype == M3X_BF16) M3X_ADD_ROWS(M3X_BF16);
  else if (dtype == M3X_F16) M3X_ADD_ROWS(M3X_F16);
  else if (dtype == M3X_F32) M3X_ADD_ROWS(M3X_F32);
  else return M3X_EUNSUPPORTED;
#undef M3X_ADD_ROWS
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Feedback embedding for the next backbone step: e = sum_l table[codes[b,l] + n_codes*l] (fp32, l ascending),
// rounded to dt, divided by sqrt(n_q) (rounded), then RMSNorm in fp32 with one final rounding:
// y = dt((x * (1/sqrt(mean x^2 + eps))) * w). serve/fast_depth.py:200-203, tts/model/audio_io.py:27-35
// (nn.RMSNorm with eps = finfo(dtype).eps when the module was built with eps=None).
// Codes outside [0, n_codes) are clamped (the reference trusts its sampler; a clamp keeps the gather in bounds).
template <int TPR, int DT>
__global__ __launch_bounds__(256) void feedback_kernel(const Elt<DT>* __restrict__ table,
                                                       const int32_t* __restrict__ codes, long s_codes,
                                                       Elt<DT>* __restrict__ out, long s_out,
                                                       const Elt<DT>* __restrict__ w, float eps, float scale, int B,
                                                       int n_q, int n_codes) {
  constexpr int N = TPR * 8;
  constexpr int RPB = 256 / TPR;
  __shared__ float red[TPR > 64 ? 256 : 1];
  __shared__ float bcast[RPB];
  const int t = threadIdx.x % TPR;
  const int row = blockIdx.x * RPB + threadIdx.x / TPR;
  const bool active = row < B;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = 0.f;
  float p = 0.f;
  const V8<DT> wv = ldv<DT>(w + 8 * t);  // requested first: its latency overlaps the gathers
  if (active) {
    // 32 codebooks at a time: their codes in one round trip, then their rows GB at a time, every load issued
    // before the first add (codebooks past n_q re-read the last valid row and are not added: no load sits in a
    // branch, which would make the compiler wait for it there); the sum runs over the codebooks in ascending order
    constexpr int GB = sizeof(Elt<DT>) == 4 ? 16 : 32;
    for (int l0 = 0; l0 < n_q; l0 += 32) {
      int cd[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int c = codes[(long)row * s_codes + min(l0 + i, n_q - 1)];
        cd[i] = c < 0 ? 0 : (c >= n_codes ? n_codes - 1 : c);
      }
#pragma unroll
      for (int h = 0; h < 32; h += GB) {
        V8<DT> tv[GB];
#pragma unroll
        for (int i = 0; i < GB; ++i)
          tv[i] = ldv<DT>(table + ((long)cd[h + i] + (long)n_codes * min(l0 + h + i, n_q - 1)) * N + 8 * t);
#pragma unroll
        for (int i = 0; i < GB; ++i)
          if (l0 + h + i < n_q) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = v[e] + E<DT>::to_f(tv[i].v[e]);
          }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = rnd<DT>(rnd<DT>(v[e]) / scale);
    p = v[0] * v[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) p = p + v[e] * v[e];
  }
  const float ss = row_tree_sum<TPR>(p, red, bcast);
  if (!active) return;
  const float inv = 1.0f / sqrtf(ss / (float)N + eps);
  V8<DT> yv;
#pragma unroll
  for (int e = 0; e < 8; ++e) yv.v[e] = E<DT>::from_f(v[e] * inv * E<DT>::to_f(wv.v[e]));
  stv<DT>(out + (long)row * s_out + 8 * t, yv);
}

M3X_API int m3x_feedback(const void* table, const int32_t* codes, long s_codes, void* out, long s_out, const void* w,
                         float eps, float scale, int B, int n, int n_q, int n_codes, int dtype, void* stream) {
  if (B < 0 || n_q <= 0 || n_codes <= 0) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!table || !codes || !out || !w) return M3X_ENULL;
  if (s_out & 7) return M3X_EINVAL;
  if (!m3x_aligned16(table) || !m3x_aligned16(out) || !m3x_aligned16(w)) return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
#define M3X_FB_LAUNCH(NN, DTT)                                                                                   \
  hipLaunchKernelGGL((feedback_kernel<NN / 8, DTT>), dim3(m3x_ceil_div(B, 256 / (NN / 8))), dim3(256), 0, st,   \
                     (const Elt<DTT>*)table, codes, s_codes, (Elt<DTT>*)out, s_out, (const Elt<DTT>*)w, eps, scale,    \
                     B, n_q, n_codes)
  if (dtype == M3X_BF16 && n == 1024) M3X_FB_LAUNCH(1024, M3X_BF16);
  else if (dtype == M3X_F16 && n == 1024) M3X_FB_LAUNCH(1024, M3X_F16);
  else if (dtype == M3X_BF16 && n == 2048) M3X_FB_LAUNCH(2048, M3X_BF16);
  else if (dtype == M3X_F16 && n == 2048) M3X_FB_LAUNCH(2048, M3X_F16);
  else if (dtype == M3X_F32 && n == 1024) M3X_FB_LAUNCH(1024, M3X_F32);
  else if (dtype == M3X_F32 && n == 2048) M3X_FB_LAUNCH(2048, M3X_F32);
  else return M3X_EUNSUPPORTED;
#undef M3X_FB_LAUNCH
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}
