// Projections: y[M, N] = x[M, K] . W[N, K]^T (nn.Linear layout), 16-bit inputs, fp32 accumulation on MFMA.
// serve/fast_backbone.py:193,200-202 (q|k|v, o, gate|up, down), the cb0 head (tts/model/backbone.py:135-136) and
// the depth trunk/heads (serve/fast_depth.py:104,122-125,167,185-191).
//
// The decode shapes are skinny (M = seats, 1..2264) and, below M of a few hundred, bound by streaming W from
// HBM. W is therefore the MFMA A operand (16 weight rows per wave, 16 contiguous bytes per lane per 32-k step)
// and the activations are the B operand; a workgroup of 4 waves covers 64 weight rows and 16*MT activation rows,
// so every W byte is read once per M tile. Small grids split K; the fp32 partials are summed by
// linear_reduce_kernel in split order, so results do not depend on scheduling.
#include "m3x_common.h"

template <int DT, int MT>
__global__ __launch_bounds__(256) void linear_kernel(const uint16_t* __restrict__ X, long ldx,
                                                     const uint16_t* __restrict__ W, long ldw, uint16_t* __restrict__ Y,
                                                     long ldy, float* __restrict__ part, int M, int N, int K,
                                                     int kchunk) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int nrow = blockIdx.x * 64 + wave * 16 + li;
  const bool nvalid = nrow < N;
  const int mbase = blockIdx.y * (16 * MT);
  const int k0 = blockIdx.z * kchunk;
  const int k1 = min(K, k0 + kchunk);
  const uint16_t* wp = W + (long)(nvalid ? nrow : 0) * ldw + 8 * lg;
  const uint16_t* xp[MT];
  bool mvalid[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = mbase + 16 * t + li;
    mvalid[t] = m < M;
    xp[t] = X + (long)(mvalid[t] ? m : 0) * ldx + 8 * lg;
  }
  f32x4_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const u16x8 zero = {};
  for (int k = k0; k < k1; k += 32) {
    u16x8 a = ld16(wp + k);
    if (!nvalid) a = zero;
    u16x8 b[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      b[t] = ld16(xp[t] + k);
      if (!mvalid[t]) b[t] = zero;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = mfma16x16x32<DT>(a, b[t], acc[t]);
  }
  // D[i][j]: i = weight row 4*lg + r of this wave's 16, j = activation row li of tile t
  const int n = blockIdx.x * 64 + wave * 16 + 4 * lg;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = mbase + 16 * t + li;
    if (m >= M) continue;
    if (gridDim.z == 1) {
      if (n + 3 < N) {
        uint16_t o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = E<DT>::from_f(acc[t][r]);
        uint2 pk;
        pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
        pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
        *reinterpret_cast<uint2*>(Y + (long)m * ldy + n) = pk;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) Y[(long)m * ldy + n + r] = E<DT>::from_f(acc[t][r]);
      }
    } else {
      float* pp = part + ((long)blockIdx.z * M + m) * N + n;
      if (n + 3 < N && (N & 3) == 0) {
        *reinterpret_cast<float4*>(pp) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) pp[r] = acc[t][r];
      }
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void linear_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ Y,
                                                            long ldy, int M, int N, int splits) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)M * N) return;
  const int m = (int)(i / N), n = (int)(i % N);
  float s = part[i];
  for (int z = 1; z < splits; ++z) s = s + part[(long)z * M * N + i];
  Y[(long)m * ldy + n] = E<DT>::from_f(s);
}

// Launch geometry shared by the launcher and the workspace query.
struct LinearPlan {
  int mt, nblk, mblk, splits, kchunk;
};

static LinearPlan linear_plan(int M, int N, int K, int splits_hint) {
  LinearPlan p;
  p.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.nblk = m3x_ceil_div(N, 64);
  p.mblk = m3x_ceil_div(M, 16 * p.mt);
  const int ksteps = K / 32;
  int s = splits_hint;
  if (s <= 0) {
    // aim for >= 512 workgroups (two per CU) without cutting K below 128 per split
    const int tiles = p.nblk * p.mblk;
    s = tiles >= 512 ? 1 : (512 + tiles - 1) / tiles;
    const int smax = ksteps / 4 > 0 ? ksteps / 4 : 1;
    if (s > smax) s = smax;
  }
  if (s < 1) s = 1;
  if (s > ksteps) s = ksteps;
  p.kchunk = 32 * m3x_ceil_div(ksteps, s);
  p.splits = m3x_ceil_div(K, p.kchunk);
  return p;
}

M3X_API size_t m3x_linear_workspace(int M, int N, int K, int splits_hint) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 32) return 0;
  LinearPlan p = linear_plan(M, N, K, splits_hint);
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

// splits_hint: 0 = choose from the shape; otherwise the number of K splits wanted.
M3X_API int m3x_linear(const void* x, long ldx, const void* w, long ldw, void* y, long ldy, int M, int N, int K,
                       int splits_hint, void* workspace, size_t ws_bytes, int dtype, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return M3X_EINVAL;
  if (M == 0) return M3X_OK;
  if (!x || !w || !y) return M3X_ENULL;
  if (K % 32 || (ldx & 7) || (ldw & 7) || (ldy & 3) || ldx < K || ldw < K || ldy < N) return M3X_EINVAL;
  if (!m3x_aligned16(x) || !m3x_aligned16(w) || (((uintptr_t)y) & 7)) return M3X_EINVAL;
  LinearPlan p = linear_plan(M, N, K, splits_hint);
  if (p.splits > 1) {
    if (!workspace) return M3X_ENULL;
    if (ws_bytes < (size_t)p.splits * M * N * sizeof(float) || !m3x_aligned16(workspace)) return M3X_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(p.nblk, p.mblk, p.splits);
  const uint16_t *X = (const uint16_t*)x, *Wt = (const uint16_t*)w;
  uint16_t* Y = (uint16_t*)y;
  float* P = (float*)workspace;
#define M3X_LIN(DTT, MTT) \
  hipLaunchKernelGGL((linear_kernel<DTT, MTT>), grid, dim3(256), 0, st, X, ldx, Wt, ldw, Y, ldy, P, M, N, K, p.kchunk)
  if (dtype == M3X_BF16) {
    if (p.mt == 1) M3X_LIN(M3X_BF16, 1);
    else if (p.mt == 2) M3X_LIN(M3X_BF16, 2);
    else M3X_LIN(M3X_BF16, 4);
  } else if (dtype == M3X_F16) {
    if (p.mt == 1) M3X_LIN(M3X_F16, 1);
    else if (p.mt == 2) M3X_LIN(M3X_F16, 2);
    else M3X_LIN(M3X_F16, 4);
  } else {
    return M3X_EUNSUPPORTED;
  }
#undef M3X_LIN
  if (p.splits > 1) {
    const long total = (long)M * N;
    if (dtype == M3X_BF16)
      hipLaunchKernelGGL(linear_reduce_kernel<M3X_BF16>, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, st, P, Y, ldy,
                         M, N, p.splits);
    else
      hipLaunchKernelGGL(linear_reduce_kernel<M3X_F16>, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, st, P, Y, ldy,
                         M, N, p.splits);
  }
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Gated activations on a [rows, 2*I] gate|up buffer (serve/fast_backbone.py:201-202: silu(g)*u with the bf16
// rounding of two eager ops) and GELU on [rows, I] (serve/fast_depth.py:123,186: F.gelu, exact erf form).
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
