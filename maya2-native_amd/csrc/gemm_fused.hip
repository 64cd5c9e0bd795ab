// Projections fused with the residual stream: the producer of a residual add (o and down projections) adds its
// output into the stream and writes the statistics of each 16-column tile of the new row; the consumer (the
// q|k|v, gate|up and head projections) multiplies the raw rows by a weight with the norm's affine terms folded in
// and applies each row's scale (and shift) from those statistics in its epilogue. The separate add+norm launch
// between the two disappears (serve/fast_backbone.py:95-104,236-240 _add_rms;
// serve/fast_depth_kernels.py:14-45 _add_ln). Kernels and plans: m3x_gemm.h.
#include "m3x_gemm.h"

namespace {

bool aligned(const void* p, uintptr_t a) { return (((uintptr_t)p) & (a - 1)) == 0; }

template <int DT>
bool resid_launch(const LinearPlan& p, hipStream_t st, const void* x, long ldx, const void* w, void* h_out, long ld_out,
                  int M, int N, int K, const ResidOut& ro) {
  return launch_linear<DT, EPI_RESID>(p, st, (const uint16_t*)x, ldx, (const uint16_t*)w, nullptr,
                                      (uint16_t*)h_out, ld_out, M, N, K, NormIn{}, ro);
}

template <int DT>
bool normed_launch(const LinearPlan& p, hipStream_t st, const void* x, long ldx, const void* wg, const void* wu,
                   void* y, long ldy, int M, int N, int K, int act, const NormIn& ni) {
  const uint16_t *X = (const uint16_t*)x, *W = (const uint16_t*)wg, *W2 = (const uint16_t*)wu;
  uint16_t* Y = (uint16_t*)y;
  if (act == M3X_ACT_SWIGLU) return launch_linear<DT, EPI_SWIGLU, true>(p, st, X, ldx, W, W2, Y, ldy, M, N, K, ni);
  if (act == M3X_ACT_GELU) return launch_linear<DT, EPI_GELU, true>(p, st, X, ldx, W, nullptr, Y, ldy, M, N, K, ni);
  return launch_linear<DT, EPI_NONE, true>(p, st, X, ldx, W, nullptr, Y, ldy, M, N, K, ni);
}

}  // namespace

M3X_API int m3x_linear_resid(const void* x, long ldx, const void* w_packed, const void* h, long ldh, const void* c,
                             long ldc, int tc, void* h_out, long ld_out, void* part, int M, int N, int K,
                             int norm_kind, int dtype, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || tc <= 0 || ldc < 0) return M3X_EINVAL;
  if (M == 0) return M3X_OK;
  if (!x || !w_packed || !h || !h_out || !part) return M3X_ENULL;
  if (norm_kind != M3X_NORM_LAYER && norm_kind != M3X_NORM_RMS) return M3X_EINVAL;
  if (K % 32 || N % 16 || (ldx & 7) || ldx < K || ldh < N || ld_out < N || (ldh & 3) || (ld_out & 3) || (ldc & 3))
    return M3X_EINVAL;
  if (!aligned(x, 16) || !aligned(w_packed, 16) || !aligned(h, 8) || !aligned(h_out, 8) || (c && !aligned(c, 8)) ||
      !aligned(part, 8))
    return M3X_EINVAL;
  if (dtype != M3X_BF16 && dtype != M3X_F16) return M3X_EUNSUPPORTED;
  const LinearPlan p = linear_plan(M, N, K, false, ldx);
  if ((long)m3x_ceil_div(p.nblk, 8) * 8 * p.mblk > 0x7fffffffL) return M3X_EINVAL;
  const ResidOut ro{(const uint16_t*)h, ldh, (const uint16_t*)c, ldc, tc, (float2*)part, norm_kind};
  hipStream_t st = (hipStream_t)stream;
  const bool ok = dtype == M3X_BF16 ? resid_launch<M3X_BF16>(p, st, x, ldx, w_packed, h_out, ld_out, M, N, K, ro)
                                    : resid_launch<M3X_F16>(p, st, x, ldx, w_packed, h_out, ld_out, M, N, K, ro);
  if (!ok) return M3X_EUNSUPPORTED;
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

M3X_API int m3x_linear_normed(const void* x, long ldx, const void* part, const float* u, const float* v, float eps,
                              int norm_kind, const void* wg_packed, const void* wu_packed, void* y, long ldy, int M,
                              int N, int K, int act, int dtype, void* stream) {
  if (M < 0 || N <= 0) return M3X_EINVAL;
  if (M == 0) return M3X_OK;
  if (!x || !part || !wg_packed || !y) return M3X_ENULL;
  if (norm_kind == M3X_NORM_LAYER && (!u || !v)) return M3X_ENULL;
  if (act == M3X_ACT_SWIGLU && !wu_packed) return M3X_ENULL;
  if (norm_kind != M3X_NORM_LAYER && norm_kind != M3X_NORM_RMS) return M3X_EINVAL;
  if (act != M3X_ACT_NONE && act != M3X_ACT_SWIGLU && act != M3X_ACT_GELU) return M3X_EINVAL;
  if (K != PRO_K || (ldx & 7) || ldx < K || ldy < N) return M3X_EINVAL;
  if (!aligned(x, 16) || !aligned(part, 16) ||
      !aligned(wg_packed, 16) || (wu_packed && !aligned(wu_packed, 16)) || !aligned(y, 2))
    return M3X_EINVAL;
  if (dtype != M3X_BF16 && dtype != M3X_F16) return M3X_EUNSUPPORTED;
  const LinearPlan p = linear_plan(M, N, K, act == M3X_ACT_SWIGLU, ldx);
  if ((long)m3x_ceil_div(p.nblk, 8) * 8 * p.mblk > 0x7fffffffL) return M3X_EINVAL;
  const NormIn ni{(const float2*)part, u, v, eps, norm_kind};
  hipStream_t st = (hipStream_t)stream;
  const bool ok = dtype == M3X_BF16
                      ? normed_launch<M3X_BF16>(p, st, x, ldx, wg_packed, wu_packed, y, ldy, M, N, K, act, ni)
                      : normed_launch<M3X_F16>(p, st, x, ldx, wg_packed, wu_packed, y, ldy, M, N, K, act, ni);
  if (!ok) return M3X_EUNSUPPORTED;
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// norm.hip
M3X_API int m3x_qk_norm_rope_cache(const void* qkv, long s_qkv, void* q_out, long s_qo_b, long s_qo_h, void* k_cache,
                                   void* v_cache, long sk_s, long sk_h, long sk_t, const int64_t* slots,
                                   const int32_t* pos, const void* cos, const void* sin, long s_cos, const void* wq,
                                   const void* wk, float eps, int rows, int heads, int kv_heads, int head_dim,
                                   int cap, void* stream);

// The q|k|v projection (plain, or with the input norm folded in when part is given: m3x_linear_normed with
// RMSNorm) followed by m3x_qk_norm_rope_cache on its output, in one launch when the row count's plan holds whole
// heads per workgroup (193..256 rows and above 512 at N = 4096); otherwise the two launches in turn, through qkv.
// Same bits either way.
M3X_API int m3x_linear_qk_rope(const void* x, long ldx, const void* part, float eps_in, const void* w_packed, void* qkv,
                               long ld_qkv, void* q_out, long s_qo_b, long s_qo_h, void* k_cache, void* v_cache,
                               long sk_s, long sk_h, long sk_t, const int64_t* slots, const int32_t* pos,
                               const void* cos, const void* sin, long s_cos, const void* wq, const void* wk, float eps,
                               int M, int K, int heads, int kv_heads, int head_dim, int cap, void* stream) {
  if (M < 0 || K <= 0 || heads <= 0 || kv_heads <= 0 || cap <= 0) return M3X_EINVAL;
  if (M == 0) return M3X_OK;
  if (!x || !w_packed || !qkv || !q_out || !k_cache || !v_cache || !slots || !pos || !cos || !sin || !wq || !wk)
    return M3X_ENULL;
  if (head_dim != 128) return M3X_EUNSUPPORTED;
  const int N = (heads + 2 * kv_heads) * head_dim;
  if (K % 32 || (ldx & 7) || ldx < K || ld_qkv < N || (ld_qkv & 7) || (part && K != PRO_K)) return M3X_EINVAL;
  if ((s_qo_b | s_qo_h | sk_s | sk_h | sk_t | s_cos) & 7) return M3X_EINVAL;
  if (!aligned(x, 16) || !aligned(w_packed, 16) || !aligned(qkv, 16) || !aligned(q_out, 16) ||
      !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(cos, 16) || !aligned(sin, 16) || !aligned(wq, 16) ||
      !aligned(wk, 16) || (part && !aligned(part, 16)))
    return M3X_EINVAL;
  const LinearPlan p = linear_plan(M, N, K, false, ldx);
  if ((long)m3x_ceil_div(p.nblk, 8) * 8 * p.mblk > 0x7fffffffL) return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const NormIn ni{(const float2*)part, nullptr, nullptr, eps_in, M3X_NORM_RMS};
  const QkOut qk{(uint16_t*)q_out, s_qo_b, s_qo_h, (uint16_t*)k_cache, (uint16_t*)v_cache, sk_s, sk_h, sk_t, slots, pos,
                 (const uint16_t*)cos, (const uint16_t*)sin, s_cos, (const uint16_t*)wq, (const uint16_t*)wk, eps,
                 heads, kv_heads, cap};
  const uint16_t* X = (const uint16_t*)x;
  const uint16_t* W = (const uint16_t*)w_packed;
  uint16_t* Y = (uint16_t*)qkv;
  const bool fused = part ? launch_linear<M3X_BF16, EPI_QKR, true>(p, st, X, ldx, W, nullptr, Y, ld_qkv, M, N, K, ni,
                                                                   ResidOut{}, qk)
                          : launch_linear<M3X_BF16, EPI_QKR, false>(p, st, X, ldx, W, nullptr, Y, ld_qkv, M, N, K,
                                                                    ni, ResidOut{}, qk);
  if (fused) {
    M3X_CHECK_LAUNCH();
    return M3X_OK;
  }
  const bool ok = part ? launch_linear<M3X_BF16, EPI_NONE, true>(p, st, X, ldx, W, nullptr, Y, ld_qkv, M, N, K, ni)
                       : launch_linear<M3X_BF16, EPI_NONE, false>(p, st, X, ldx, W, nullptr, Y, ld_qkv, M, N, K);
  if (!ok) return M3X_EUNSUPPORTED;
  M3X_CHECK_LAUNCH();
  return m3x_qk_norm_rope_cache(qkv, ld_qkv, q_out, s_qo_b, s_qo_h, k_cache, v_cache, sk_s, sk_h, sk_t, slots, pos, cos,
                                sin, s_cos, wq, wk, eps, M, heads, kv_heads, head_dim, cap, stream);
}
