// Projections: the pack kernel, the fp32 projection kernel and the C entry points of the plain and gated
// projections (the 16-bit kernels and their plans are in m3x_gemm.h).
#include "m3x_gemm.h"

template <int DT>
__global__ __launch_bounds__(256) void pack_weight_kernel(const Elt<DT>* __restrict__ W, long ldw, int N, int K,
                                                          Elt<DT>* __restrict__ out) {
  const long v = (long)blockIdx.x * 256 + threadIdx.x;  // one 8-element lane vector of the packed layout
  const int ks = K >> 5;
  const long total = (long)((N + 15) >> 4) * ks * 64;
  if (v >= total) return;
  const int lane = (int)(v & 63);
  const long f = v >> 6;
  const int s = (int)(f % ks);
  const int n = (int)(f / ks) * 16 + (lane & 15);
  const V8<DT> x = n < N ? ldv<DT>(W + (long)n * ldw + s * 32 + 8 * (lane >> 4)) : zero_v8<DT>();
  stv<DT>(out + v * 8, x);
}

// fp32 projections (the fp32 compute paths: FastDepth and StaticMimi built with dtype=float32). The packed layout
// is the 16-bit one with 4-byte elements (a fragment is 2 KB, lane l's 8 values at + 8 l), so one pack serves
// both; each k step of 32 is eight v_mfma_f32_16x16x4_f32 (mfma16x16x32_f32). A workgroup of 4 waves = NW weight
// tiles x KW = 4 / NW slices of K walks its slice in chunks of 32 U (U = 4 k steps for 16- and 32-row tiles, 2 for
// 64-row ones): the chunk's activation rows are staged in LDS (row stride 32 U + 4 floats), the next chunk's rows and
// weight fragments load into registers while the
// current one multiplies. The KW slice partials meet in LDS and are added in slice order (deterministic).
// Epilogues in fp32: EPI_NONE y = acc; EPI_SWIGLU y = silu(g) * u; EPI_GELU y = gelu(acc) (erf form).
template <int MT, int NW, int EPI>
__global__ __launch_bounds__(256) void linear_f32_kernel(const float* __restrict__ X, long ldx,
                                                         const float* __restrict__ Wp, const float* __restrict__ W2p,
                                                         float* __restrict__ Y, long ldy, int M, int N, int K,
                                                         int mblk, int nblk) {
  constexpr int KW = 4 / NW;
  constexpr int ROWS = 16 * MT;
  static_assert(MT * KW <= 4, "activation chunks must fit the LDS budget");
  // k steps (of 32) per chunk: 4 for the tiles of one or two 16-row blocks (few rows, latency-bound: half the
  // chunks, half the load round trips), 2 for the 64-row tiles; each wave still adds its slice's steps in order, so
  // U does not change the bits
  constexpr int U = MT <= 2 ? 4 : 2;
  constexpr int LDR = 32 * U + 4;   // LDS row stride in floats
  constexpr int GPR = 8 * U;        // 16-byte granules per row per chunk
  constexpr int NVEC = KW * ROWS * GPR;
  constexpr int VPT = (NVEC + 255) / 256;
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NA = DUAL ? 2 : 1;
  constexpr int XS = KW * ROWS * LDR;
  constexpr int RED = (KW - 1) * NW * NA * MT * 64 * 4;  // floats of slice partials
  __shared__ __align__(16) float xs[XS > RED ? XS : RED];

  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int nb = (slot / mblk) * 8 + xcd;
  const int mb = slot - (slot / mblk) * mblk;
  if (nb >= nblk) return;  // padding block: the whole workgroup leaves before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches around the MFMAs
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wn = wave % NW;
  const int wk = wave / NW;
  const int ntiles = (N + 15) >> 4;
  const int n0 = (nb * NW + wn) * 16;
  const int nt = min(nb * NW + wn, ntiles - 1);  // tiles past N read a valid tile; nothing of them is stored
  const int m0 = mb * ROWS;
  const int ksteps = K >> 5;
  const int nch = ((ksteps + KW - 1) / KW + U - 1) / U;  // chunks per slice (equal for all slices)
  const int span = nch * U;
  const int s0 = wk * span;
  const int s1 = min(ksteps, s0 + span);

  const float* wp[NA];
  wp[0] = Wp + ((long)nt * ksteps * 64 + lane) * 8;
  if constexpr (DUAL) wp[NA - 1] = W2p + ((long)nt * ksteps * 64 + lane) * 8;

  // activation granule v = tid + 256 j -> slice q, row r, granule g (4 floats) of the chunk; rows past M and
  // steps past a slice keep earlier finite values, whose products are never stored
  float4 Xr[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) Xr[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  auto xload = [&](int c) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = tid + 256 * j;
      if (NVEC % 256 == 0 || v < NVEC) {
        const int q = v / (ROWS * GPR);
        const int rem = v - q * (ROWS * GPR);
        const int r = rem / GPR;
        const int g = rem - r * GPR;
        const int m = m0 + r;
        const int step = q * span + c * U + (g >> 3);
        if (m < M && step < min(ksteps, (q + 1) * span))
          Xr[j] = *reinterpret_cast<const float4*>(X + (long)m * ldx + step * 32 + (g & 7) * 4);
      }
    }
  };
  auto xstore = [&]() {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = tid + 256 * j;
      if (NVEC % 256 == 0 || v < NVEC) {
        const int q = v / (ROWS * GPR);
        const int rem = v - q * (ROWS * GPR);
        const int r = rem / GPR;
        const int g = rem - r * GPR;
        *reinterpret_cast<float4*>(&xs[(q * ROWS + r) * LDR + g * 4]) = Xr[j];
      }
    }
  };
  f32x8 Wc[U][NA], Wn[U][NA];
  auto wload = [&](int c, f32x8(&Wr)[U][NA]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = min(s0 + c * U + u, ksteps - 1);  // past the slice: a valid fragment, never multiplied
#pragma unroll
      for (int a = 0; a < NA; ++a) Wr[u][a] = ldv<M3X_F32>(wp[a] + (long)s * 512);
    }
  };
  f32x4_t acc[NA][MT];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[a][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  xload(0);
  wload(0, Wc);
  for (int c = 0; c < nch; ++c) {
    __syncthreads();  // every wave is done reading the previous chunk
    xstore();
    __syncthreads();
    if (c + 1 < nch) {
      xload(c + 1);
      wload(c + 1, Wn);
    }
    const float* xb = &xs[(wk * ROWS + li) * LDR + 8 * lg];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + c * U + u < s1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const f32x8 b = ldv<M3X_F32>(xb + t * 16 * LDR + u * 32);
#pragma unroll
          for (int a = 0; a < NA; ++a) acc[a][t] = mfma16x16x32_f32(Wc[u][a], b, acc[a][t]);
        }
      }
    }
    if (c + 1 < nch) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int a = 0; a < NA; ++a) Wc[u][a] = Wn[u][a];
    }
  }

  // slice partials meet in LDS, added in slice order by slice 0
  f32x4_t* red = reinterpret_cast<f32x4_t*>(xs);
  if constexpr (KW > 1) {
    __syncthreads();
    if (wk > 0) {
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < MT; ++t) red[(((wk - 1) * NW + wn) * NA * MT + a * MT + t) * 64 + lane] = acc[a][t];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int j = 0; j < KW - 1; ++j)
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const f32x4_t v = red[((j * NW + wn) * NA * MT + a * MT + t) * 64 + lane];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[a][t][r] = acc[a][t][r] + v[r];
        }
  }
  const int n = n0 + 4 * lg;
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)Y) & 15) == 0 && n + 3 < N;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = m0 + 16 * t + li;
    if (m >= M) continue;
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = acc[0][t][r];
      if constexpr (EPI == EPI_SWIGLU) {
        v = v / (1.0f + expf(-v)) * acc[NA - 1][t][r];
      } else if constexpr (EPI == EPI_GELU) {
        v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
      }
      o[r] = v;
    }
    float* yp = Y + (long)m * ldy + n;
    if (vec) {
      *reinterpret_cast<float4*>(yp) = make_float4(o[0], o[1], o[2], o[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) yp[r] = o[r];
    }
  }
}

// fp32 tile choice: the largest tile (most operand reuse) that still gives at least 256 workgroups; small grids
// split K four ways.
template <int EPI>
static bool launch_linear_f32(hipStream_t st, const float* X, long ldx, const float* W, const float* W2, float* Y,
                              long ldy, int M, int N, int K) {
  const int ntiles = m3x_ceil_div(N, 16);
  const int cand[6][2] = {{4, 4}, {2, 4}, {2, 2}, {1, 4}, {1, 2}, {1, 1}};
  int mt = 1, nw = 1;
  for (const auto& c : cand) {
    if ((long)m3x_ceil_div(M, 16 * c[0]) * m3x_ceil_div(ntiles, c[1]) >= 256) {
      mt = c[0];
      nw = c[1];
      break;
    }
  }
  const int mblk = m3x_ceil_div(M, 16 * mt), nblk = m3x_ceil_div(ntiles, nw);
  if ((long)m3x_ceil_div(nblk, 8) * 8 * mblk > 0x7fffffffL) return false;
  const dim3 grid(m3x_ceil_div(nblk, 8) * 8 * mblk);
#define M3X_LF(MTT, NWW)                                                                                     \
  hipLaunchKernelGGL((linear_f32_kernel<MTT, NWW, EPI>), grid, dim3(256), 0, st, X, ldx, W, W2, Y, ldy, M, N, K, \
                     mblk, nblk)
  switch (mt * 10 + nw) {
    case 44: M3X_LF(4, 4); return true;
    case 24: M3X_LF(2, 4); return true;
    case 22: M3X_LF(2, 2); return true;
    case 14: M3X_LF(1, 4); return true;
    case 12: M3X_LF(1, 2); return true;
    default: M3X_LF(1, 1); return true;
  }
#undef M3X_LF
}

static int linear_common(const void* x, long ldx, const void* w, const void* w2, void* y, long ldy, int M, int N,
                         int K, int epi, int dtype, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return M3X_EINVAL;
  if (M == 0) return M3X_OK;
  if (!x || !w || !y || (epi == EPI_SWIGLU && !w2)) return M3X_ENULL;
  if (K % 32 || (ldx & 7) || ldx < K || ldy < N) return M3X_EINVAL;
  if (!m3x_aligned16(x) || !m3x_aligned16(w) || (w2 && !m3x_aligned16(w2)) || (((uintptr_t)y) & 1))
    return M3X_EINVAL;
  if (dtype == M3X_F32) {
    if ((((uintptr_t)y) & 3) || (ldx & 3)) return M3X_EINVAL;
    hipStream_t st = (hipStream_t)stream;
    const float *X = (const float*)x, *Wt = (const float*)w, *W2 = (const float*)w2;
    float* Y = (float*)y;
    bool ok;
    if (epi == EPI_NONE) ok = launch_linear_f32<EPI_NONE>(st, X, ldx, Wt, W2, Y, ldy, M, N, K);
    else if (epi == EPI_SWIGLU) ok = launch_linear_f32<EPI_SWIGLU>(st, X, ldx, Wt, W2, Y, ldy, M, N, K);
    else ok = launch_linear_f32<EPI_GELU>(st, X, ldx, Wt, W2, Y, ldy, M, N, K);
    if (!ok) return M3X_EINVAL;
    M3X_CHECK_LAUNCH();
    return M3X_OK;
  }
  const LinearPlan p = linear_plan(M, N, K, epi == EPI_SWIGLU, ldx);
  if ((long)m3x_ceil_div(p.nblk, 8) * 8 * p.mblk > 0x7fffffffL) return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *X = (const uint16_t*)x, *Wt = (const uint16_t*)w, *W2 = (const uint16_t*)w2;
  uint16_t* Y = (uint16_t*)y;
  bool ok;
  if (dtype == M3X_BF16) {
    if (epi == EPI_NONE) ok = launch_linear<M3X_BF16, EPI_NONE>(p, st, X, ldx, Wt, W2, Y, ldy, M, N, K);
    else if (epi == EPI_SWIGLU) ok = launch_linear<M3X_BF16, EPI_SWIGLU>(p, st, X, ldx, Wt, W2, Y, ldy, M, N, K);
    else ok = launch_linear<M3X_BF16, EPI_GELU>(p, st, X, ldx, Wt, W2, Y, ldy, M, N, K);
  } else if (dtype == M3X_F16) {
    if (epi == EPI_NONE) ok = launch_linear<M3X_F16, EPI_NONE>(p, st, X, ldx, Wt, W2, Y, ldy, M, N, K);
    else if (epi == EPI_SWIGLU) ok = launch_linear<M3X_F16, EPI_SWIGLU>(p, st, X, ldx, Wt, W2, Y, ldy, M, N, K);
    else ok = launch_linear<M3X_F16, EPI_GELU>(p, st, X, ldx, Wt, W2, Y, ldy, M, N, K);
  } else {
    return M3X_EUNSUPPORTED;
  }
  if (!ok) return M3X_EUNSUPPORTED;
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// Elements of the packed form of an [N, K] weight: N rounded up to 16 rows, times K.
M3X_API long m3x_packed_weight_elems(int N, int K) {
  if (N <= 0 || K <= 0 || K % 32) return -1;
  return (long)m3x_ceil_div(N, 16) * 16 * K;
}

M3X_API int m3x_pack_weight(const void* w, long ldw, int N, int K, void* out, int dtype, void* stream) {
  if (N <= 0 || K <= 0 || K % 32 || ldw < K || (ldw & 7)) return M3X_EINVAL;
  if (!w || !out) return M3X_ENULL;
  if (!m3x_aligned16(w) || !m3x_aligned16(out)) return M3X_EINVAL;
  const long total = (long)m3x_ceil_div(N, 16) * (K / 32) * 64;
  const dim3 grid(m3x_ceil_div(total, 256));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == M3X_F32)
    hipLaunchKernelGGL(pack_weight_kernel<M3X_F32>, grid, dim3(256), 0, st, (const float*)w, ldw, N, K, (float*)out);
  else if (dtype == M3X_BF16 || dtype == M3X_F16)  // the layout moves bit patterns: one instance serves both
    hipLaunchKernelGGL(pack_weight_kernel<M3X_BF16>, grid, dim3(256), 0, st, (const uint16_t*)w, ldw, N, K,
                       (uint16_t*)out);
  else
    return M3X_EUNSUPPORTED;
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

M3X_API int m3x_linear(const void* x, long ldx, const void* w_packed, void* y, long ldy, int M, int N, int K,
                       int dtype, void* stream) {
  return linear_common(x, ldx, w_packed, nullptr, y, ldy, M, N, K, EPI_NONE, dtype, stream);
}

// kind 0 (SwiGLU): y[:, :I] = dt(silu(x.Wg^T)) * (x.Wu^T) with packed gate rows wg[I, K] and up rows wu[I, K];
// kind 1 (GELU): y[:, :I] = gelu(x.Wg^T) (wu unused).
M3X_API int m3x_linear_act(const void* x, long ldx, const void* wg_packed, const void* wu_packed, void* y, long ldy,
                           int M, int I, int K, int kind, int dtype, void* stream) {
  if (kind != 0 && kind != 1) return M3X_EINVAL;
  return linear_common(x, ldx, wg_packed, kind == 0 ? wu_packed : nullptr, y, ldy, M, I, K,
                       kind == 0 ? EPI_SWIGLU : EPI_GELU, dtype, stream);
}

// ---------------------------------------------------------------------------------------------------------
// Stand-alone gated activations on a [rows, 2*I] gate|up buffer (SwiGLU) or [rows, I] (GELU), for callers that
// hold the projection output already.

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
    const float sg = rnd<DT>(silu16(g));
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
