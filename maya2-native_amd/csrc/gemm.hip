// Projections: y[M, N] = x[M, K] . W[N, K]^T (nn.Linear layout), 16-bit inputs, fp32 accumulation on MFMA,
// with optional fused gated epilogues.
// serve/fast_backbone.py:193,200-202 (q|k|v, o, gate|up + silu*mul, down), the cb0 head
// (tts/model/backbone.py:135-136) and the depth trunk/heads (serve/fast_depth.py:104,122-125,167,185-191).
//
// Weights are packed once (m3x_pack_weight) into MFMA fragment order: the 16 x 32 fragment (row tile nt, k step s)
// occupies 1 KB at element offset (nt * K/32 + s) * 512 and lane l's 8 elements sit at + 8 l, holding
// W[16 nt + l % 16][32 s + 8 (l / 16) + e] - exactly the A operand of v_mfma_f32_16x16x32. A wave reads a
// fragment as one contiguous 1 KB (16 bytes per lane, in lane order), which the vector L1 serves as 16 cache-line
// accesses; the row-major operand pattern (16 rows per instruction) costs 64.
//
// Activations are the B operand. A workgroup (4 waves = NW weight tiles x KW = 4/NW slices of K) stages the
// 16*MT activation rows of each 128-wide K chunk in LDS with row-contiguous loads, double-buffered, and every
// wave reads its fragments from there. Weight fragments run two chunks ahead in registers, activations three.
// The KW partial sums meet in LDS and are added in slice order: the result is independent of scheduling.
// Workgroups are numbered so that the row blocks sharing one weight slab run on one XCD (ids equal mod 8) and
// the slab is fetched into that XCD's L2 once.
//
// Epilogues (each rounds exactly where the reference's eager ops round):
//   EPI_NONE    y = dt(acc)
//   EPI_SWIGLU  y = dt(dt(silu(dt(acc_gate))) * dt(acc_up)), gate rows from W, up rows from W2
//               (F.linear -> chunk -> F.silu(g)*u, serve/fast_backbone.py:201-202)
//   EPI_GELU    y = dt(gelu(dt(acc)))  (F.gelu(f1(x)), serve/fast_depth.py:123,186; exact erf form)
#include "m3x_common.h"

enum { EPI_NONE = 0, EPI_SWIGLU = 1, EPI_GELU = 2 };

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

// The KW K-slice partials of one weight tile meet in LDS (`red`, free when this runs) and are added in slice
// order by slice 0, which then applies the epilogue. Lane (li, lg) holds weight rows n0 + 4*lg + r of
// activation row m0 + 16*t + li.
template <int DT, int MT, int NW, int KW, int EPI>
__device__ __forceinline__ void linear_finish(f32x4_t (&acc)[EPI == EPI_SWIGLU ? 2 : 1][MT], f32x4_t* red, int wn,
                                              int wk, int lane, int n0, int m0, uint16_t* __restrict__ Y, long ldy,
                                              int M, int N) {
  constexpr int NA = EPI == EPI_SWIGLU ? 2 : 1;
  const int li = lane & 15;
  const int lg = lane >> 4;
  if constexpr (KW > 1) {
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
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)Y) & 7) == 0 && n + 3 < N;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = m0 + 16 * t + li;
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

template <int DT, int MT, int NW, int EPI>
__global__ __launch_bounds__(256) void linear_kernel(const uint16_t* __restrict__ X, long ldx,
                                                     const uint16_t* __restrict__ Wp,
                                                     const uint16_t* __restrict__ W2p, uint16_t* __restrict__ Y,
                                                     long ldy, int M, int N, int K, int mblk, int nblk) {
  constexpr int KW = 4 / NW;
  static_assert(MT * KW <= 4, "activation chunks must fit the LDS budget");
  constexpr int U = 4;                 // k steps (of 32) per chunk
  constexpr int ROWS = 16 * MT;
  constexpr int LDR = 32 * U + 8;      // LDS row stride in halfwords: 272 bytes, conflict-free fragment reads
  constexpr int VPR = 4 * U;           // 16-byte vectors per row per chunk
  constexpr int NVEC = KW * ROWS * VPR;
  constexpr int VPT = (NVEC + 255) / 256;
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NA = DUAL ? 2 : 1;
  __shared__ __align__(16) uint16_t xs[2][KW * ROWS * LDR];

  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int nb = (slot / mblk) * 8 + xcd;
  const int mb = slot - (slot / mblk) * mblk;
  if (nb >= nblk) return;  // padding block: the whole workgroup leaves before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
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

  const uint16_t* wp[NA];
  wp[0] = Wp + ((long)nt * ksteps * 64 + lane) * 8;
  if constexpr (DUAL) wp[NA - 1] = W2p + ((long)nt * ksteps * 64 + lane) * 8;

  // Activation vectors: v = tid + 256 j -> slice q, row r, 16-byte column c16 of the chunk. Rows past M and
  // steps past a slice are not loaded: their registers keep finite earlier values, whose products are never
  // stored.
  u16x8 X0[VPT], X1[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) X0[j].v[e] = X1[j].v[e] = 0;
  auto xload = [&](int c, u16x8(&Xr)[VPT]) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = tid + 256 * j;
      if (NVEC % 256 == 0 || v < NVEC) {
        const int q = v / (ROWS * VPR);
        const int rem = v - q * (ROWS * VPR);
        const int r = rem / VPR;
        const int c16 = rem - r * VPR;
        const int m = m0 + r;
        const int step = q * span + c * U + (c16 >> 2);
        if (m < M && step < min(ksteps, (q + 1) * span)) Xr[j] = ld16(X + (long)m * ldx + step * 32 + (c16 & 3) * 8);
      }
    }
  };
  auto xstore = [&](int buf, const u16x8(&Xr)[VPT]) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int v = tid + 256 * j;
      if (NVEC % 256 == 0 || v < NVEC) {
        const int q = v / (ROWS * VPR);
        const int rem = v - q * (ROWS * VPR);
        const int r = rem / VPR;
        const int c16 = rem - r * VPR;
        st16(&xs[buf][(q * ROWS + r) * LDR + c16 * 8], Xr[j]);
      }
    }
  };
  u16x8 W0[U][NA], W1[U][NA];
  auto wload = [&](int c, u16x8(&Wr)[U][NA]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = min(s0 + c * U + u, ksteps - 1);  // past the slice: a valid fragment, never multiplied
#pragma unroll
      for (int a = 0; a < NA; ++a) Wr[u][a] = ld16(wp[a] + (long)s * 512);
    }
  };
  f32x4_t acc[NA][MT];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[a][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int c, int buf, const u16x8(&Wr)[U][NA]) {
    const uint16_t* xb = &xs[buf][(wk * ROWS + li) * LDR + 8 * lg];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + c * U + u < s1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const u16x8 b = *reinterpret_cast<const u16x8*>(xb + t * 16 * LDR + u * 32);
#pragma unroll
          for (int a = 0; a < NA; ++a) acc[a][t] = mfma16x16x32<DT>(Wr[u][a], b, acc[a][t]);
        }
      }
    }
  };

  // chunk c: LDS buffer c & 1, weight registers W(c & 1), activation registers X(c & 1)
  xload(0, X0);
  wload(0, W0);
  if (nch > 1) {
    xload(1, X1);
    wload(1, W1);
  }
  xstore(0, X0);
  if (nch > 2) xload(2, X0);
  __syncthreads();
  for (int c = 0; c < nch; c += 2) {
    compute(c, 0, W0);
    if (c + 1 < nch) xstore(1, X1);
    if (c + 3 < nch) xload(c + 3, X1);
    if (c + 2 < nch) wload(c + 2, W0);
    __syncthreads();
    if (c + 1 >= nch) break;
    compute(c + 1, 1, W1);
    if (c + 2 < nch) xstore(0, X0);
    if (c + 4 < nch) xload(c + 4, X0);
    if (c + 3 < nch) wload(c + 3, W1);
    __syncthreads();
  }

  linear_finish<DT, MT, NW, KW, EPI>(acc, reinterpret_cast<f32x4_t*>(&xs[0][0]), wn, wk, lane, n0, m0, Y, ldy, M,
                                     N);
}

// One-shot variant: every weight fragment of the wave's K slice (S steps of 32) and the workgroup's whole
// activation block are loaded at once, so the kernel pays one memory latency instead of one per chunk. A
// workgroup is NWAVES waves = NW weight tiles x KW = NWAVES / NW slices of K. With 8 or 16 waves the block may
// take up to 128 KB of gfx950's 160 KB LDS; one such workgroup per CU then streams its whole weight slab at
// once. The block sits in LDS unpadded when a slice row is a multiple of 16 granules of 16 bytes, with granule
// g of row r stored at g ^ (r % 16), so the 16 rows a fragment read touches fall in 16 different bank groups;
// otherwise rows are padded by 16 bytes.
template <int DT, int MT, int NW, int NWAVES, int EPI, int S>
__global__ __launch_bounds__(64 * NWAVES) void linear_oneshot_kernel(const uint16_t* __restrict__ X, long ldx,
                                                                     const uint16_t* __restrict__ Wp,
                                                                     const uint16_t* __restrict__ W2p,
                                                                     uint16_t* __restrict__ Y, long ldy, int M, int N,
                                                                     int K, int mblk, int nblk) {
  constexpr int NT = 64 * NWAVES;
  constexpr int KW = NWAVES / NW;
  constexpr int ROWS = 16 * MT;
  constexpr int KS = 32 * S;          // k per slice
  constexpr int GR = 4 * S;           // 16-byte granules per row of a slice
  constexpr bool SWZ = GR % 16 == 0;
  constexpr int LDR = SWZ ? KS : KS + 8;
  constexpr int NVEC = KW * ROWS * GR;
  constexpr int VPT = (NVEC + NT - 1) / NT;
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NA = DUAL ? 2 : 1;
  static_assert(KW * NW == NWAVES, "one-shot geometry");
  static_assert((KW - 1) * NW * NA * MT * 1024 <= KW * ROWS * LDR * 2, "slice partials must fit the block");
  __shared__ __align__(16) uint16_t xs[KW * ROWS * LDR];

  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int nb = (slot / mblk) * 8 + xcd;
  const int mb = slot - (slot / mblk) * mblk;
  if (nb >= nblk) return;  // padding block: the whole workgroup leaves before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wn = wave % NW;
  const int wk = wave / NW;
  const int ntiles = (N + 15) >> 4;
  const int n0 = (nb * NW + wn) * 16;
  const int nt = min(nb * NW + wn, ntiles - 1);
  const int m0 = mb * ROWS;
  const int ksteps = K >> 5;
  const int s0 = wk * S;

  u16x8 Wr[S][NA];
  {
    const uint16_t* w0 = Wp + ((long)nt * ksteps * 64 + lane) * 8;
    const uint16_t* w1 = DUAL ? W2p + ((long)nt * ksteps * 64 + lane) * 8 : w0;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      Wr[s][0] = ld16(w0 + (long)(s0 + s) * 512);
      if constexpr (DUAL) Wr[s][NA - 1] = ld16(w1 + (long)(s0 + s) * 512);
    }
  }
  // activation vector v = tid + NT j -> slice q, row r, granule g
  u16x8 Xr[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int v = tid + NT * j;
    const int q = v / (ROWS * GR);
    const int rem = v - q * (ROWS * GR);
    const int r = rem / GR;
    const int g = rem - r * GR;
    const int m = m0 + r;
#pragma unroll
    for (int e = 0; e < 8; ++e) Xr[j].v[e] = 0;
    if ((NVEC % NT == 0 || v < NVEC) && m < M) Xr[j] = ld16(X + (long)m * ldx + q * KS + g * 8);
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int v = tid + NT * j;
    const int q = v / (ROWS * GR);
    const int rem = v - q * (ROWS * GR);
    const int r = rem / GR;
    const int g = rem - r * GR;
    if (NVEC % NT == 0 || v < NVEC) st16(&xs[(q * ROWS + r) * LDR + ((SWZ ? g ^ (r & 15) : g) << 3)], Xr[j]);
  }
  __syncthreads();

  f32x4_t acc[NA][MT];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[a][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* xb = &xs[(wk * ROWS + li) * LDR];
#pragma unroll
  for (int s = 0; s < S; ++s) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int gi = SWZ ? (4 * s + lg) ^ li : 4 * s + lg;
      const u16x8 b = *reinterpret_cast<const u16x8*>(xb + t * 16 * LDR + (gi << 3));
#pragma unroll
      for (int a = 0; a < NA; ++a) acc[a][t] = mfma16x16x32<DT>(Wr[s][a], b, acc[a][t]);
    }
  }
  __syncthreads();  // every wave is done with the block before it holds the slice partials
  linear_finish<DT, MT, NW, KW, EPI>(acc, reinterpret_cast<f32x4_t*>(xs), wn, wk, lane, n0, m0, Y, ldy, M, N);
}

// Large-M projections (M > 512 rows: steps with inline prefills). A workgroup of 8 waves owns a 2-D tile of 128
// activation rows x 128 weight rows (for SwiGLU: 64 gate rows from W and the same 64 up rows from W2, i.e. 64
// output columns) and walks K in stages of 64. The packed weight fragments of a stage are copied to LDS as they are
// (16 fragments of 1 KB: every fragment read is one contiguous 1 KB); the activation rows sit row-major with a
// 144-byte row stride, so the 16 rows of a fragment read fall in 16 different bank groups and a row's 8 stores in
// distinct banks. The waves are 2 x 4 blocks of 64 activation rows x 32 weight rows (4 x 2 MFMA tiles; with
// SwiGLU a wave holds one gate tile and the matching up tile). Stages are double-buffered in LDS: the next stage's
// global loads are in flight while the current one multiplies, with one barrier per stage. Every weight byte is
// read by ceil(M / 128) workgroups and every activation byte by ceil(N / 128), against 36 and 64 for the 64 x 64
// chunked tiles at 2264 rows.
template <int DT, int EPI>
__global__ __launch_bounds__(512, 2) void linear_tiled_kernel(const uint16_t* __restrict__ X, long ldx,
                                                              const uint16_t* __restrict__ Wp,
                                                              const uint16_t* __restrict__ W2p,
                                                              uint16_t* __restrict__ Y, long ldy, int M, int N, int K,
                                                              int mblk, int nblk) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int BM = 128;
  constexpr int LDA = 72;  // activation row stride in LDS, halfwords
  __shared__ __align__(16) uint16_t lw[2][16 * 512];
  __shared__ __align__(16) uint16_t la[2][BM * LDA];

  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int nb = (slot / mblk) * 8 + xcd;
  const int mb = slot - (slot / mblk) * mblk;
  if (nb >= nblk) return;  // padding block: the whole workgroup leaves before any barrier

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wm = wave & 1;   // activation tiles 4 wm .. 4 wm + 3
  const int wn = wave >> 1;  // weight tiles (below)
  const int ksteps = K >> 5;
  const int ntiles = (N + 15) >> 4;
  const int m0 = mb * BM;

  // per-thread load slots: vector v = tid + 512 j of a stage; weights: fragment f = v / 64 = tid / 64 + 8 j (tile
  // t = f / 2, step f % 2), lane v % 64, at LDS 8 v; activations: row v / 8 = tid / 8 + 64 j, 16-byte column v % 8.
  // Offsets are 32-bit element offsets; with SwiGLU, slot j = 0 holds gate rows and j = 1 up rows.
  int gw[2], ga[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int f = (tid >> 6) + 8 * j;
    const int t = f >> 1, st = f & 1;
    const int tt = min(DUAL ? nb * 4 + (t & 3) : nb * 8 + t, ntiles - 1);  // tiles past N: valid, never stored
    gw[j] = (tt * ksteps + st) * 512 + (tid & 63) * 8;
    ga[j] = min(m0 + (tid >> 3) + 64 * j, M - 1) * (int)ldx + 8 * (tid & 7);  // rows past M: re-read, never stored
  }
  const int la0 = (tid >> 3) * LDA + 8 * (tid & 7);
  // the wave's 2 weight tiles: plain 2 wn + i; SwiGLU gate wn and up 4 + wn
  int wt[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) wt[i] = DUAL ? (i == 0 ? wn : 4 + wn) : 2 * wn + i;

  f32x4_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  u16x8 rw[2], ra[2];
  auto gload = [&](int stg) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      rw[j] = ld16((DUAL && j == 1 ? W2p : Wp) + gw[j] + stg * 1024);
      ra[j] = ld16(X + ga[j] + stg * 64);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      st16(&lw[buf][tid * 8 + 4096 * j], rw[j]);
      st16(&la[buf][la0 + 64 * j * LDA], ra[j]);
    }
  };
  const int nst = K >> 6;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int stg = 0; stg < nst; ++stg) {
    const int buf = stg & 1;
    if (stg + 1 < nst) gload(stg + 1);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      u16x8 a[2], b[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const u16x8*>(&lw[buf][(wt[i] * 2 + s) * 512 + lane * 8]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const u16x8*>(&la[buf][(16 * (4 * wm + j) + li) * LDA + 32 * s + 8 * lg]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32<DT>(a[i], b[j], acc[i][j]);
    }
    if (stg + 1 < nst) lstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane (li, lg) of tile pair (i, j) holds weight rows 4 lg + r of tile wt[i] for activation row
  // m0 + 16 (4 wm + j) + li
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)Y) & 7) == 0;
  constexpr int NI = DUAL ? 1 : 2;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int n = DUAL ? (nb * 4 + wn) * 16 + 4 * lg : (nb * 8 + wt[i]) * 16 + 4 * lg;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + 16 * (4 * wm + j) + li;
      if (m >= M) continue;
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = rnd<DT>(acc[i][j][r]);
        if constexpr (DUAL) {
          const float g = v;
          const float u = rnd<DT>(acc[1][j][r]);
          v = rnd<DT>(g / (1.0f + expf(-g))) * u;
        } else if constexpr (EPI == EPI_GELU) {
          v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
        }
        o[r] = E<DT>::from_f(v);
      }
      uint16_t* yp = Y + (long)m * ldy + n;
      if (vec && n + 3 < N) {
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
}

// fp32 projections (the fp32 compute paths: FastDepth and StaticMimi built with dtype=float32). The packed layout
// is the 16-bit one with 4-byte elements (a fragment is 2 KB, lane l's 8 values at + 8 l), so one pack serves
// both; each k step of 32 is eight v_mfma_f32_16x16x4_f32 (mfma16x16x32_f32). A workgroup of 4 waves = NW weight
// tiles x KW = 4 / NW slices of K walks its slice in chunks of 64 (2 k steps): the chunk's activation rows are
// staged in LDS (row stride 68 floats), the next chunk's rows and weight fragments load into registers while the
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
  constexpr int U = 2;              // k steps (of 32) per chunk
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

// Launch geometry: MT activation tiles of 16 rows per workgroup; NW weight tiles per workgroup; NWAVES waves
// (NWAVES / NW K slices).
struct LinearPlan {
  int mt, nw, mblk, nblk;
  int nwaves;   // 4 for the chunked kernel and the small one-shot; 8 or 16 for the wide one-shot
  int oneshot;  // steps per K slice for the one-shot kernel, 0 for the chunked kernel
  int tiled;    // 1: linear_tiled_kernel (M > 512, K % 64 == 0)
};

// Small one-shot (4 waves): each of the 4/nw K slices is exactly 8 or 16 steps of 32 and the activation block
// (16*mt rows x K) fits in 64 KB of LDS.
static int oneshot_steps(int mt, int nw, int K) {
  const int kw = 4 / nw;
  if (K % (32 * kw)) return 0;
  const int s = K / 32 / kw;
  if ((s != 8 && s != 16) || (long)16 * mt * K * 2 > 65536) return 0;
  return s;
}

// Wide one-shot plans (measured on MI355X, graph-timed, 64..256 rows; 20-30 % under the chunked kernel on the
// decode shapes; up to 16 rows: 0.1-1.7 us under the 4-wave kernels). K = 1024: the first (MT, NW) of (2,2), (2,4), (3,4), (2,8) whose grid fits one workgroup per
// CU (<= 256); 8 waves. K = 2048, 2816, 3072: 16-row blocks, 16 waves, NW = 4 above 160 rows, else 2.
// Returns false when no instantiated plan covers (M, N, K).
static bool wide_plan(int M, int N, int K, bool dual, LinearPlan& p) {
  if (M <= 16 && (K == 1024 || K == 2048 || K == 2816 || K == 3072)) {
    // one 16-row block: 8 waves, each a K/8 slice of one weight tile (3.7 against 5.3 us at 1 x 1024 x 2816)
    p.mt = 1;
    p.nw = 1;
    p.nwaves = 8;
    p.oneshot = K / 256;
    return true;
  }
  if (M < 64 || M > 256) return false;
  const int ntiles = m3x_ceil_div(N, 16);
  if (K == 1024) {
    const int cand[4][2] = {{2, 2}, {2, 4}, {3, 4}, {2, 8}};
    for (const auto& c : cand) {
      if (dual && c[1] == 8) continue;  // the gate/up pair of 8 tiles does not fit the register file
      const long wgs = (long)m3x_ceil_div(M, 16 * c[0]) * m3x_ceil_div(ntiles, c[1]);
      if (wgs <= 256) {
        p.mt = c[0];
        p.nw = c[1];
        p.nwaves = 8;
        p.oneshot = K / 32 / (8 / c[1]);
        return true;
      }
    }
    return false;
  }
  if ((K == 2048 || K == 2816 || K == 3072) && !dual) {
    p.mt = 1;
    p.nw = M > 160 ? 4 : 2;
    p.nwaves = 16;
    p.oneshot = K / 32 / (16 / p.nw);
    return true;
  }
  return false;
}

// Chunked / small one-shot tile choice, measured on MI355X (graph-timed sweep over the decode shapes,
// M = 1..2264): the best plan is the largest tile that still gives at least ~400 workgroups; MT = 2 pays off
// only above ~112 rows.
static LinearPlan linear_plan(int M, int N, int K, bool dual, long ldx) {
  const int ntiles = m3x_ceil_div(N, 16);
  const int ksteps = K / 32;
  auto blocks = [&](int mt, int nw) { return (long)m3x_ceil_div(M, 16 * mt) * m3x_ceil_div(ntiles, nw); };
  LinearPlan p;
  p.nwaves = 4;
  p.tiled = 0;
  // tiled: 32-bit element offsets into the packed weight and the activations
  if (M > 512 && K % 64 == 0 && (long)ntiles * 16 * K < (1L << 31) && (long)M * ldx < (1L << 31)) {
    p.tiled = 1;
    p.mt = 8;
    p.nw = dual ? 4 : 8;
    p.oneshot = 0;
    p.mblk = m3x_ceil_div(M, 128);
    p.nblk = m3x_ceil_div(ntiles, p.nw);
    return p;
  }
  if (wide_plan(M, N, K, dual, p)) {
    p.mblk = m3x_ceil_div(M, 16 * p.mt);
    p.nblk = m3x_ceil_div(ntiles, p.nw);
    return p;
  }
  if (M > 512) {
    p.mt = 4;
    p.nw = 4;
  } else if (M > 112 && blocks(2, 2) >= 400) {
    p.mt = 2;
    p.nw = blocks(2, 4) >= 400 ? 4 : 2;
  } else {
    p.mt = 1;
    p.nw = blocks(1, 4) >= 400 ? 4 : (blocks(1, 2) >= 400 ? 2 : 1);
  }
  while (p.nw < 4 && ksteps / (4 / p.nw) < 4) p.nw <<= 1;  // at least one chunk per K slice
  // Small weights (N <= 2048, K <= 1024) at up to 512 rows: 16-row blocks through the one-shot kernel.
  if (M > 112 && M <= 512 && N <= 2048 && K <= 1024 && oneshot_steps(1, 2, K)) {
    p.mt = 1;
    p.nw = blocks(1, 2) >= 400 || !oneshot_steps(1, 1, K) ? 2 : 1;
  }
  p.mblk = m3x_ceil_div(M, 16 * p.mt);
  p.nblk = m3x_ceil_div(ntiles, p.nw);
  // One-shot when its activation block leaves room for several workgroups per CU (<= 32 KB), or when only a
  // handful of rows exist (a 64 KB block then costs nothing in latency): measured on the decode shapes, the
  // one-shot kernel is 0.5-1.1 us faster in those cases and slower with 32-row blocks of 64 KB.
  p.oneshot = oneshot_steps(p.mt, p.nw, K);
  if (p.oneshot && (long)16 * p.mt * K * 2 > 32768 && M > 16) p.oneshot = 0;
  return p;
}

// Launches the plan's kernel; false (nothing launched) for a plan no kernel instance covers.
template <int DT, int EPI>
static bool launch_linear(const LinearPlan& p, hipStream_t st, const uint16_t* X, long ldx, const uint16_t* W,
                          const uint16_t* W2, uint16_t* Y, long ldy, int M, int N, int K) {
  const dim3 grid(m3x_ceil_div(p.nblk, 8) * 8 * p.mblk);
  if (p.tiled) {
    hipLaunchKernelGGL((linear_tiled_kernel<DT, EPI>), grid, dim3(512), 0, st, X, ldx, W, W2, Y, ldy, M, N, K, p.mblk,
                       p.nblk);
    return true;
  }
#define M3X_ONE(MTT, NWW, NWV, SS)                                                                         \
  hipLaunchKernelGGL((linear_oneshot_kernel<DT, MTT, NWW, NWV, EPI, SS>), grid, dim3(64 * NWV), 0, st, X, \
                     ldx, W, W2, Y, ldy, M, N, K, p.mblk, p.nblk)
  if (p.oneshot) {
    const long key = ((p.mt * 10L + p.nw) * 100 + p.nwaves) * 100 + p.oneshot;
    switch (key) {
      case 120416: M3X_ONE(1, 2, 4, 16); return true;
      case 120408: M3X_ONE(1, 2, 4, 8); return true;
      case 110416: M3X_ONE(1, 1, 4, 16); return true;
      case 110408: M3X_ONE(1, 1, 4, 8); return true;
      case 140416: M3X_ONE(1, 4, 4, 16); return true;
      case 140408: M3X_ONE(1, 4, 4, 8); return true;
      case 220416: M3X_ONE(2, 2, 4, 16); return true;
      case 220408: M3X_ONE(2, 2, 4, 8); return true;
      case 240416: M3X_ONE(2, 4, 4, 16); return true;
      case 240408: M3X_ONE(2, 4, 4, 8); return true;
      case 210408: M3X_ONE(2, 1, 4, 8); return true;
      // up to 16 rows, K = 1024 / 2048 / 2816 / 3072
      case 110804: M3X_ONE(1, 1, 8, 4); return true;
      case 110808: M3X_ONE(1, 1, 8, 8); return true;
      case 110811: M3X_ONE(1, 1, 8, 11); return true;
      case 110812: M3X_ONE(1, 1, 8, 12); return true;
      // wide, K = 1024
      case 220808: M3X_ONE(2, 2, 8, 8); return true;
      case 240816: M3X_ONE(2, 4, 8, 16); return true;
      case 340816: M3X_ONE(3, 4, 8, 16); return true;
      case 280832: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(2, 8, 8, 32); return true; } return false;
      // wide, K = 2048 / 2816 / 3072
      case 141616: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 4, 16, 16); return true; } return false;
      case 121608: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 2, 16, 8); return true; } return false;
      case 141622: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 4, 16, 22); return true; } return false;
      case 121611: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 2, 16, 11); return true; } return false;
      case 141624: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 4, 16, 24); return true; } return false;
      case 121612: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 2, 16, 12); return true; } return false;
      default: return false;
    }
  }
#undef M3X_ONE
#define M3X_LIN(MTT, NWW)                                                                                           \
  hipLaunchKernelGGL((linear_kernel<DT, MTT, NWW, EPI>), grid, dim3(256), 0, st, X, ldx, W, W2, Y, ldy, M, N, K, \
                     p.mblk, p.nblk)
  const int key = p.mt * 10 + p.nw;
  switch (key) {
    case 14: M3X_LIN(1, 4); return true;
    case 12: M3X_LIN(1, 2); return true;
    case 11: M3X_LIN(1, 1); return true;
    case 24: M3X_LIN(2, 4); return true;
    case 22: M3X_LIN(2, 2); return true;
    case 44: M3X_LIN(4, 4); return true;
    default: return false;
  }
#undef M3X_LIN
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
