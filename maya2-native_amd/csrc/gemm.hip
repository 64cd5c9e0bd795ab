// Projections: y[M, N] = x[M, K] . W[N, K]^T (nn.Linear layout), 16-bit inputs, fp32 accumulation on MFMA,
// with optional fused gated epilogues.
// serve/fast_backbone.py:193,200-202 (q|k|v, o, gate|up + silu*mul, down), the cb0 head
// (tts/model/backbone.py:135-136) and the depth trunk/heads (serve/fast_depth.py:104,122-125,167,185-191).
//
// The decode shapes are skinny (M = seats, 1..2264). W is the MFMA A operand (16 weight rows per wave,
// 16 contiguous bytes per lane per 32-k step), the activations the B operand (16*MT rows per wave). A workgroup
// has 4 waves arranged as NW weight-row tiles x KW = 4/NW slices of K; the KW partial sums meet in LDS and are
// added in slice order, so the result does not depend on scheduling and no second launch or workspace is needed.
// The k loop keeps the next 4 k-steps of loads in flight while the current 4 run on the MFMAs.
// Blocks are ordered m-fastest, so the M tiles that share a weight slab are dispatched together.
//
// Epilogues (each rounds exactly where the reference's eager ops round):
//   EPI_NONE    y = dt(acc)
//   EPI_SWIGLU  y = dt(dt(silu(dt(acc_gate))) * dt(acc_up)), gate rows from W, up rows from W2
//               (F.linear -> chunk -> F.silu(g)*u, serve/fast_backbone.py:201-202)
//   EPI_GELU    y = dt(gelu(dt(acc)))  (F.gelu(f1(x)), serve/fast_depth.py:123,186; exact erf form)
#include "m3x_common.h"

enum { EPI_NONE = 0, EPI_SWIGLU = 1, EPI_GELU = 2 };

template <int DT, int MT, int NW, int EPI>
__global__ __launch_bounds__(256) void linear_kernel(const uint16_t* __restrict__ X, long ldx,
                                                     const uint16_t* __restrict__ W, const uint16_t* __restrict__ W2,
                                                     long ldw, uint16_t* __restrict__ Y, long ldy, int M, int N,
                                                     int K, int mfast) {
  constexpr int KW = 4 / NW;
  constexpr int U = 4;
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NA = DUAL ? 2 : 1;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wn = wave % NW;
  const int wk = wave / NW;
  const int mblock = mfast ? blockIdx.x : blockIdx.y;
  const int nblock = mfast ? blockIdx.y : blockIdx.x;
  const int n0 = (nblock * NW + wn) * 16;
  const int mbase = mblock * (16 * MT);
  const int ksteps = K / 32;
  const int per = (ksteps + KW - 1) / KW;
  const int s0 = wk * per;
  const int s1 = min(ksteps, s0 + per);

  const int nrow = n0 + li;
  const bool nvalid = nrow < N;
  const uint16_t* wp[NA];
  wp[0] = W + (long)(nvalid ? nrow : 0) * ldw + 8 * lg;
  if constexpr (DUAL) wp[NA - 1] = W2 + (long)(nvalid ? nrow : 0) * ldw + 8 * lg;
  const uint16_t* xp[MT];
  bool mvalid[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = mbase + 16 * t + li;
    mvalid[t] = m < M;
    xp[t] = X + (long)(mvalid[t] ? m : 0) * ldx + 8 * lg;
  }
  // Rows past N or M read a valid (clamped) row and their results are never stored, so no loaded value is
  // ever inspected before its MFMA: the loads of the next group stay in flight behind the current group.
  f32x4_t acc[NA][MT];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[a][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto load = [&](int st, u16x8(&A)[U][NA], u16x8(&Bv)[U][MT]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (st + u) * 32;
#pragma unroll
      for (int a = 0; a < NA; ++a) A[u][a] = ld16(wp[a] + k);
#pragma unroll
      for (int t = 0; t < MT; ++t) Bv[u][t] = ld16(xp[t] + k);
    }
  };
  auto compute = [&](const u16x8(&A)[U][NA], const u16x8(&Bv)[U][MT]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[a][t] = mfma16x16x32<DT>(A[u][a], Bv[u][t], acc[a][t]);
  };
  // two register buffers in ping-pong: group g+1 loads while group g multiplies; no copies between them
  const int nfull = max(s1 - s0, 0) / U;
  int s = s0;
  u16x8 A0[U][NA], B0[U][MT], A1[U][NA], B1[U][MT];
  if (nfull > 0) load(s0, A0, B0);
  int g = 0;
  for (; g + 1 < nfull; g += 2) {
    load(s + U, A1, B1);
    compute(A0, B0);
    s += U;
    load(g + 2 < nfull ? s + U : s, A0, B0);  // past the end: reload this group (in bounds, unused)
    compute(A1, B1);
    s += U;
  }
  if (g < nfull) {
    compute(A0, B0);
    s += U;
  }
  for (; s < s1; ++s) {
    u16x8 a1[NA], b1[MT];
#pragma unroll
    for (int a = 0; a < NA; ++a) a1[a] = ld16(wp[a] + s * 32);
#pragma unroll
    for (int t = 0; t < MT; ++t) b1[t] = ld16(xp[t] + s * 32);
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[a][t] = mfma16x16x32<DT>(a1[a], b1[t], acc[a][t]);
  }

  // ---- the KW slices of one weight tile meet in LDS, summed in slice order by slice 0
  if constexpr (KW > 1) {
    __shared__ f32x4_t red[KW - 1][NW][NA * MT][64];
    if (wk > 0) {
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < MT; ++t) red[wk - 1][wn][a * MT + t][lane] = acc[a][t];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int j = 0; j < KW - 1; ++j)
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const f32x4_t v = red[j][wn][a * MT + t][lane];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[a][t][r] = acc[a][t][r] + v[r];
        }
  }

  // ---- epilogue: lane holds weight rows n0 + 4*lg + r of activation row mbase + 16*t + li
  const int n = n0 + 4 * lg;
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)Y) & 7) == 0 && n + 3 < N;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = mbase + 16 * t + li;
    if (m >= M) continue;
    uint16_t o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = rnd<DT>(acc[0][t][r]);
      if constexpr (EPI == EPI_SWIGLU) {
        const float g = v;
        const float u = rnd<DT>(acc[NA - 1][t][r]);
        v = rnd<DT>(g / (1.0f + expf(-g))) * u;
      } else if constexpr (EPI == EPI_GELU) {
        v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
      }
      o[r] = E<DT>::from_f(v);
    }
    uint16_t* yp = Y + (long)m * ldy + n;
    if (vec) {
      uint2 pk;
      pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
      pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
      *reinterpret_cast<uint2*>(yp) = pk;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) yp[r] = o[r];
    }
  }
}

// Launch geometry: MT activation tiles of 16 rows per wave; NW weight tiles per workgroup (4 / NW K slices).
// The widest NW that still gives about one workgroup per CU keeps the whole K of a tile in one wave.
struct LinearPlan {
  int mt, nw, mblk, nblk, mfast;
};

static LinearPlan linear_plan(int M, int N, int K) {
  LinearPlan p;
  p.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.mblk = m3x_ceil_div(M, 16 * p.mt);
  const int ksteps = K / 32;
  p.nw = 1;
  for (int nw = 4; nw >= 1; nw >>= 1) {
    const long blocks = (long)m3x_ceil_div(N, 16 * nw) * p.mblk;
    if (blocks >= 240 || nw == 1) {
      p.nw = nw;
      break;
    }
  }
  // keep at least 4 k-steps per slice
  while (p.nw < 4 && ksteps / (4 / p.nw) < 4) p.nw <<= 1;
  p.nblk = m3x_ceil_div(N, 16 * p.nw);
  p.mfast = 1;
  return p;
}

template <int DT, int EPI>
static void launch_linear(const LinearPlan& p, hipStream_t st, const uint16_t* X, long ldx, const uint16_t* W,
                          const uint16_t* W2, long ldw, uint16_t* Y, long ldy, int M, int N, int K) {
  dim3 grid(p.mfast ? p.mblk : p.nblk, p.mfast ? p.nblk : p.mblk);
#define M3X_LIN(MTT, NWW)                                                                                       \
  hipLaunchKernelGGL((linear_kernel<DT, MTT, NWW, EPI>), grid, dim3(256), 0, st, X, ldx, W, W2, ldw, Y, ldy, M, N, \
                     K, p.mfast)
#define M3X_LIN_NW(MTT)          \
  if (p.nw == 4) M3X_LIN(MTT, 4); \
  else if (p.nw == 2) M3X_LIN(MTT, 2); \
  else M3X_LIN(MTT, 1);
  if (p.mt == 1) {
    M3X_LIN_NW(1)
  } else if (p.mt == 2) {
    M3X_LIN_NW(2)
  } else {
    M3X_LIN_NW(4)
  }
#undef M3X_LIN_NW
#undef M3X_LIN
}

static int linear_common(const void* x, long ldx, const void* w, const void* w2, long ldw, void* y, long ldy, int M,
                         int N, int K, int epi, int dtype, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return M3X_EINVAL;
  if (M == 0) return M3X_OK;
  if (!x || !w || !y || (epi == EPI_SWIGLU && !w2)) return M3X_ENULL;
  if (K % 32 || (ldx & 7) || (ldw & 7) || ldx < K || ldw < K || ldy < N) return M3X_EINVAL;
  if (!m3x_aligned16(x) || !m3x_aligned16(w) || (w2 && !m3x_aligned16(w2)) || (((uintptr_t)y) & 1))
    return M3X_EINVAL;
  const LinearPlan p = linear_plan(M, N, K);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *X = (const uint16_t*)x, *Wt = (const uint16_t*)w, *W2 = (const uint16_t*)w2;
  uint16_t* Y = (uint16_t*)y;
  if (dtype == M3X_BF16) {
    if (epi == EPI_NONE) launch_linear<M3X_BF16, EPI_NONE>(p, st, X, ldx, Wt, W2, ldw, Y, ldy, M, N, K);
    else if (epi == EPI_SWIGLU) launch_linear<M3X_BF16, EPI_SWIGLU>(p, st, X, ldx, Wt, W2, ldw, Y, ldy, M, N, K);
    else launch_linear<M3X_BF16, EPI_GELU>(p, st, X, ldx, Wt, W2, ldw, Y, ldy, M, N, K);
  } else if (dtype == M3X_F16) {
    if (epi == EPI_NONE) launch_linear<M3X_F16, EPI_NONE>(p, st, X, ldx, Wt, W2, ldw, Y, ldy, M, N, K);
    else if (epi == EPI_SWIGLU) launch_linear<M3X_F16, EPI_SWIGLU>(p, st, X, ldx, Wt, W2, ldw, Y, ldy, M, N, K);
    else launch_linear<M3X_F16, EPI_GELU>(p, st, X, ldx, Wt, W2, ldw, Y, ldy, M, N, K);
  } else {
    return M3X_EUNSUPPORTED;
  }
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

M3X_API int m3x_linear(const void* x, long ldx, const void* w, long ldw, void* y, long ldy, int M, int N, int K,
                       int dtype, void* stream) {
  return linear_common(x, ldx, w, nullptr, ldw, y, ldy, M, N, K, EPI_NONE, dtype, stream);
}

// kind 0 (SwiGLU): y[:, :I] = dt(silu(x.Wg^T)) * (x.Wu^T) with gate rows w_gate[I, K], up rows w_up[I, K];
// kind 1 (GELU): y[:, :I] = gelu(x.Wg^T) (w_up unused).
M3X_API int m3x_linear_act(const void* x, long ldx, const void* w_gate, const void* w_up, long ldw, void* y, long ldy,
                           int M, int I, int K, int kind, int dtype, void* stream) {
  if (kind != 0 && kind != 1) return M3X_EINVAL;
  return linear_common(x, ldx, w_gate, kind == 0 ? w_up : nullptr, ldw, y, ldy, M, I, K,
                       kind == 0 ? EPI_SWIGLU : EPI_GELU, dtype, stream);
}

// ---------------------------------------------------------------------------------------------------------
// Stand-alone gated activations on a [rows, 2*I] gate|up buffer (SwiGLU) or [rows, I] (GELU), for callers that
// hold the projection output already.
enum { M3X_ACT_SWIGLU = 0, M3X_ACT_GELU = 1 };

template <int DT>
__global__ __launch_bounds__(256) void act_kernel(const uint16_t* __restrict__ in, long ld_in, uint16_t* __restrict__ out,
                                                  long ld_out, int rows, int I, int kind) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)rows * I) return;
  const int r = (int)(i / I), c = (int)(i % I);
  const float g = E<DT>::to_f(in[(long)r * ld_in + c]);
  float y;
  if (kind == M3X_ACT_SWIGLU) {
    const float u = E<DT>::to_f(in[(long)r * ld_in + I + c]);
    const float sg = rnd<DT>(g / (1.0f + expf(-g)));
    y = sg * u;
  } else {
    y = 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
  }
  out[(long)r * ld_out + c] = E<DT>::from_f(y);
}

M3X_API int m3x_act(const void* in, long ld_in, void* out, long ld_out, int rows, int I, int kind, int dtype,
                    void* stream) {
  if (rows < 0 || I <= 0) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!in || !out) return M3X_ENULL;
  if (kind != M3X_ACT_SWIGLU && kind != M3X_ACT_GELU) return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const long total = (long)rows * I;
  if (dtype == M3X_BF16)
    hipLaunchKernelGGL(act_kernel<M3X_BF16>, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, st, (const uint16_t*)in,
                       ld_in, (uint16_t*)out, ld_out, rows, I, kind);
  else if (dtype == M3X_F16)
    hipLaunchKernelGGL(act_kernel<M3X_F16>, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, st, (const uint16_t*)in,
                       ld_in, (uint16_t*)out, ld_out, rows, I, kind);
  else
    return M3X_EUNSUPPORTED;
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}
