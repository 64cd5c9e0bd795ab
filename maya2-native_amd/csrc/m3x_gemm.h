// 16-bit projection kernels (bf16 / fp16 storage, fp32 accumulation on MFMA) and their launch plans, shared by
// gemm.hip (plain and gated projections) and gemm_fused.hip (projections fused with the residual add and the
// norm that follows it).
//
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
//   EPI_RESID   y = dt(h + dt(acc)) [then dt(y + c[m / tc])]: the projection joins the residual stream, and the
//               workgroup also writes the statistics of every 16-column tile of the stored row for the norm that
//               follows (the add of _add_rms / _add_ln, serve/fast_backbone.py:95-104, serve/fast_depth_kernels.py:
//               14-45; the norm itself is folded into the consumer, below)
//   EPI_QKR     the q|k|v projection's values (rounded to bf16 as EPI_NONE stores them) go through the per-head
//               q/k RMSNorm + RoPE and into the caches (m3x_qk_norm_rope_cache's arithmetic, qk_norm_rope8):
//               query heads to q_out, key and value heads into the static cache at [slot, head, pos]. Needs whole
//               heads per workgroup: the large-M tiled plan (128 x 128 tiles) and the one-shot plan with NW = 8 and
//               one K slice (128 columns).
//
// Folded norm (PRO): the consumer of a residual row multiplies the raw row and applies the norm to the product.
// A norm's elementwise weight w (and LayerNorm bias b) is folded into the consumer's weight when it is packed:
// Wf[n, k] = dt(W[n, k] * w[k]), u[n] = sum_k Wf[n, k], v[n] = sum_k b[k] W[n, k] (fp32). Then
//   RMSNorm:   norm(x) . W[n]^T = inv_rms * (x . Wf[n]^T)
//   LayerNorm: norm(x) . W[n]^T = rstd * (x . Wf[n]^T) - rstd * mean * u[n] + v[n]
// with the row's inv_rms, or mean and rstd = 1 / sqrt(var + eps), merged from the producer's tile statistics
// ((sum, sum of squares) per 16 columns for RMSNorm, (sum, squared deviations from the tile mean) for LayerNorm,
// combined in a fixed order: Chan's pairwise combination for the variance). The prologue only loads and merges the
// statistics of the workgroup's rows; the activations go to the MFMAs as stored, and the epilogue applies the row
// scale (and shift) before its own rounding. Against the reference's order (normalised row rounded to the storage
// type, then multiplied) this moves the rounding from the normalised activation to the folded weight: the same
// one-rounding error at the storage precision, on the other operand.
#pragma once
#include "m3x_common.h"
#include "m3x_norm.h"

enum { EPI_NONE = 0, EPI_SWIGLU = 1, EPI_GELU = 2, EPI_RESID = 3, EPI_QKR = 4 };
enum { M3X_ACT_NONE = -1, M3X_ACT_SWIGLU = 0, M3X_ACT_GELU = 1 };  // the C ABI's gated-activation kinds

// Folded input norm of a PRO projection: the statistics part[m * (K / 16) + j] of row m's 16-column tiles j, and
// for LayerNorm the column vectors u, v of the folded weight (N entries; with SwiGLU 2N: the gate's, then the
// up projection's).
struct NormIn {
  const float2* part;
  const float* u;
  const float* v;
  float eps;
  int kind;  // M3X_NORM_LAYER or M3X_NORM_RMS
};

// Residual epilogue: row m of the output is dt(h[m] + dt(acc)) [+ c[m / tc], rounded]; part[m * (N / 16) + j]
// receives the statistics of the stored row's tile j for a norm of kind `kind`.
struct ResidOut {
  const uint16_t* h;
  long ldh;
  const uint16_t* c;
  long ldc;
  int tc;
  float2* part;
  int kind;
};

// EPI_QKR's outputs: q_out rows [m * s_qb + head * s_qh], the caches at [slot * sk_s + head * sk_h + pos * sk_t]
// (slots[m], pos[m] < cap), cos/sin rows of s_cos halfwords, the q/k norm weights wq/wk (D = 128).
struct QkOut {
  uint16_t* q;
  long s_qb, s_qh;
  uint16_t* kc;
  uint16_t* vc;
  long sk_s, sk_h, sk_t;
  const int64_t* slots;
  const int32_t* pos;
  const uint16_t* cosb;
  const uint16_t* sinb;
  long s_cos;
  const uint16_t* wq;
  const uint16_t* wk;
  float eps;
  int H, KV, cap;
};

// Row scale and shift of a PRO row from its tile statistics: 8 consecutive lanes per row, TPT tiles per lane
// (K = 128 TPT). Every lane of the row's group returns (rstd, -mean * rstd) for LayerNorm and (1 / rms, 0) for
// RMSNorm; the sums over the group's lanes are group_sum<8> butterflies, so all eight lanes hold the same bits.
template <int TPT>
__device__ __forceinline__ float2 norm_row_stats(const float2 (&p)[TPT], int K, int kind, float eps) {
  if (kind == M3X_NORM_RMS) {
    float q = p[0].y;
#pragma unroll
    for (int j = 1; j < TPT; ++j) q = q + p[j].y;
    q = group_sum<8>(q);
    return make_float2(1.0f / sqrtf(q / (float)K + eps), 0.f);
  }
  float s = p[0].x;
#pragma unroll
  for (int j = 1; j < TPT; ++j) s = s + p[j].x;
  const float mean = group_sum<8>(s) / (float)K;
  float m2 = 0.f;
#pragma unroll
  for (int j = 0; j < TPT; ++j) {
    const float d = p[j].x * 0.0625f - mean;  // tile mean - row mean
    m2 = m2 + (p[j].y + 16.0f * d * d);
  }
  m2 = group_sum<8>(m2);
  const float rstd = 1.0f / sqrtf(m2 / (float)K + eps);
  return make_float2(rstd, -mean * rstd);
}

// PRO statistics, in two halves around the kernel's main loop. load issues the loads of the tile statistics of rows
// m0 .. m0 + ROWS - 1 (8 threads per row, NT threads, PASSES rounds) before the kernel's own loads; finish, after
// the main loop, merges them into the row scale and shift st[ROWS] in LDS. The caller then waits at a barrier
// before the epilogue reads them. Rows past M get (0, 0) and are never stored.
template <int ROWS, int NT, int TPT>
struct NormStage {
  static constexpr int PASSES = (ROWS * 8 + NT - 1) / NT;
  float2 p[PASSES][TPT];
  // with fewer rows than 8 lanes per row need, only the first ROWS / 8 waves hold statistics (a wave-uniform test:
  // the other waves issue no loads)
  static __device__ __forceinline__ bool active() {
    return ROWS * 8 >= NT || __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < ROWS / 8;
  }
  __device__ __forceinline__ void load(const NormIn& ni, int m0, int M, int K) {
    if (!active()) return;
    const int tid = threadIdx.x;
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      // clamped to a valid row: no branch around the loads (a divergent join would wait for every load in
      // flight); rows past M and threads past the block are never stored
      const int r = min((tid + ps * NT) >> 3, ROWS - 1);
      const int m = min(m0 + r, M - 1);
      const float4* src = reinterpret_cast<const float4*>(ni.part + (long)m * (K >> 4) + (tid & 7) * TPT);
#pragma unroll
      for (int j = 0; j < TPT / 2; ++j) {
        const float4 v = src[j];
        p[ps][2 * j] = make_float2(v.x, v.y);
        p[ps][2 * j + 1] = make_float2(v.z, v.w);
      }
    }
  }
  __device__ __forceinline__ void finish(const NormIn& ni, int m0, int M, int K, float2* st) {
    if (!active()) return;
    const int tid = threadIdx.x;
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int r = (tid + ps * NT) >> 3;
      const float2 v = norm_row_stats<TPT>(p[ps], K, ni.kind, ni.eps);
      if (r < ROWS && (tid & 7) == 0) st[r] = m0 + r < M ? v : make_float2(0.f, 0.f);
    }
  }
};

// The folded norm on one lane's 4 accumulators of row slot `row` (columns n .. n + 3 of weight a: 0 = W, 1 = W2):
// acc = scale * acc [+ shift * u[n] + v[n]].
__device__ __forceinline__ void norm_apply(f32x4_t& acc, const float2* pst, int row, const NormIn& ni, int n, int N,
                                           int a) {
  const float2 st = pst[row];
  if (ni.kind == M3X_NORM_LAYER) {
    const float* u = ni.u + a * N;
    const float* v = ni.v + a * N;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = min(n + r, N - 1);  // columns past N: any finite value, never stored
      acc[r] = st.x * acc[r] + (st.y * u[c] + v[c]);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = st.x * acc[r];
  }
}

// The residual operands of one lane's 4 outputs (columns n .. n + 3 of row m), loaded when the kernel starts so
// that the epilogue does not wait on them: h[m, n ..] and, with a per-seat constant, c[m / tc, n ..].
struct ResidPre {
  uint2 h, c;
};
// Addresses are clamped to valid elements (values of rows past M or columns past N are never stored), and the
// constant falls back to h's element when absent, so the loads sit in no branch.
__device__ __forceinline__ ResidPre resid_prefetch(const ResidOut& ro, int m, int n, int M, int N) {
  const int mc = min(m, M - 1), nc = min(n, N - 4);
  const uint16_t* hp = ro.h + (long)mc * ro.ldh + nc;
  const uint16_t* cp = ro.c ? ro.c + (long)(mc / ro.tc) * ro.ldc + nc : hp;
  return ResidPre{*reinterpret_cast<const uint2*>(hp), *reinterpret_cast<const uint2*>(cp)};
}

// EPI_RESID for one lane's 4 outputs (columns n .. n + 3 of row m, acc as accumulated, pre its prefetched
// operands): stores the residual row's values and, with the other 3 lanes of the 16-column tile (lanes
// li + 16 lg'), the tile's statistics part[m * (N / 16) + tile]. Every lane of the wave calls it (cross-lane
// sums); rows past M store nothing.
template <int DT>
__device__ __forceinline__ void resid_quad(const f32x4_t& acc, const ResidPre& pre, int m, int n, int tile, int M,
                                           int N, int lg, const ResidOut& ro, uint16_t* __restrict__ Y, long ldy) {
  const bool valid = m < M && n < N;  // N % 16 == 0: a tile is wholly inside or wholly past N
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (valid) {
    const uint2 hh = pre.h;
    const uint16_t h4[4] = {(uint16_t)hh.x, (uint16_t)(hh.x >> 16), (uint16_t)hh.y, (uint16_t)(hh.y >> 16)};
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = rnd<DT>(E<DT>::to_f(h4[r]) + rnd<DT>(acc[r]));
    if (ro.c) {
      const uint2 cc = pre.c;
      const uint16_t c4[4] = {(uint16_t)cc.x, (uint16_t)(cc.x >> 16), (uint16_t)cc.y, (uint16_t)(cc.y >> 16)};
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = rnd<DT>(v[r] + E<DT>::to_f(c4[r]));
    }
    uint2 pk;
    pk.x = (uint32_t)E<DT>::from_f(v[0]) | ((uint32_t)E<DT>::from_f(v[1]) << 16);
    pk.y = (uint32_t)E<DT>::from_f(v[2]) | ((uint32_t)E<DT>::from_f(v[3]) << 16);
    *reinterpret_cast<uint2*>(Y + (long)m * ldy + n) = pk;
  }
  float s = v[0] + v[1] + v[2] + v[3];
  s = xor32_sum(xor16_sum(s));
  float q;
  if (ro.kind == M3X_NORM_RMS) {
    q = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  } else {
    const float mt = s * 0.0625f;
    const float d0 = v[0] - mt, d1 = v[1] - mt, d2 = v[2] - mt, d3 = v[3] - mt;
    q = d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
  }
  q = xor32_sum(xor16_sum(q));
  if (valid && lg == 0) ro.part[(long)m * (N >> 4) + tile] = make_float2(s, q);
}

// The KW K-slice partials of one weight tile meet in LDS (`red`, free when this runs) and are added in slice
// order by slice 0, which then applies the epilogue. Lane (li, lg) holds weight rows n0 + 4*lg + r of
// activation row m0 + 16*t + li.
template <int DT, int MT, int NW, int KW, int EPI, bool PRO>
__device__ __forceinline__ void linear_finish(f32x4_t (&acc)[EPI == EPI_SWIGLU ? 2 : 1][MT], f32x4_t* red, int wn,
                                              int wk, int lane, int n0, int m0, uint16_t* __restrict__ Y, long ldy,
                                              int M, int N, const ResidOut& ro, const ResidPre* pre,
                                              const float2* pst, const NormIn& ni) {
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
  if constexpr (PRO) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int a = 0; a < NA; ++a) norm_apply(acc[a][t], pst, 16 * t + li, ni, n, N, a);
  }
  if constexpr (EPI == EPI_RESID) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
      resid_quad<DT>(acc[0][t], pre[t], m0 + 16 * t + li, n, n0 >> 4, M, N, lg, ro, Y, ldy);
    return;
  }
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
        v = rnd<DT>(silu16(g)) * u;
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

// linear_finish for the one-shot plans with several K slices and a plain, gated or GELU epilogue, with the work
// spread over every wave of the weight tile: each of the KW waves stores its partial tiles to LDS (`red`, free when
// this runs), then lane T = 64 wk + lane of the tile's waves takes elements e = T + 64 KW j of the MT x 16 x 16
// block (row-major, so a row's 16 columns sit in 16 adjacent lanes), adds their KW partials in slice order (the sum
// linear_finish forms), and applies the epilogue and a 2-byte store. Instead of one wave per tile doing all 4 MT
// elements per lane while the others wait, every wave does 4 MT / KW (rounded up; past the block, whole waves
// skip).
template <int DT, int MT, int NW, int KW, int EPI, bool PRO>
__device__ __forceinline__ void linear_finish_spread(f32x4_t (&acc)[EPI == EPI_SWIGLU ? 2 : 1][MT], float* red,
                                                     int wn, int wk, int lane, int n0, int m0,
                                                     uint16_t* __restrict__ Y, long ldy, int M, int N,
                                                     const float2* pst, const NormIn& ni) {
  constexpr int NA = EPI == EPI_SWIGLU ? 2 : 1;
  constexpr int EPL = (4 * MT + KW - 1) / KW;  // elements per lane (with KW > 4 MT, waves 4 MT.. have none)
  static_assert(KW > 1, "several K slices");
  static_assert(EPI == EPI_NONE || EPI == EPI_SWIGLU || EPI == EPI_GELU, "plain, gated or GELU epilogue");
  const int li = lane & 15;
  const int lg = lane >> 4;
  // partial (slice q, weight a, row tile t) of tile wn: element (row, col) at red[base(q, a, t) + 16 row + col]
  auto base = [&](int q, int a, int t) { return (((wn * KW + q) * NA + a) * MT + t) * 256; };
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int t = 0; t < MT; ++t) *reinterpret_cast<f32x4_t*>(&red[base(wk, a, t) + 16 * li + 4 * lg]) = acc[a][t];
  __syncthreads();
  const int T = 64 * wk + lane;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = T + 64 * KW * j;
    if (e >= 256 * MT) break;  // wave-uniform: 256 MT is a multiple of 64
    const int t = e >> 8;
    const int row = (e >> 4) & 15;
    const int n = n0 + (e & 15);
    const int m = m0 + 16 * t + row;
    float v[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      float x = red[base(0, a, t) + (e & 255)];
#pragma unroll
      for (int q = 1; q < KW; ++q) x = x + red[base(q, a, t) + (e & 255)];
      if constexpr (PRO) {
        const float2 st = pst[16 * t + row];
        if (ni.kind == M3X_NORM_LAYER) {
          const int c = min(n, N - 1);  // columns past N: any finite value, never stored
          x = st.x * x + (st.y * ni.u[a * N + c] + ni.v[a * N + c]);
        } else {
          x = st.x * x;
        }
      }
      v[a] = x;
    }
    float o = rnd<DT>(v[0]);
    if constexpr (EPI == EPI_SWIGLU) {
      o = rnd<DT>(silu16(o)) * rnd<DT>(v[NA - 1]);
    } else if constexpr (EPI == EPI_GELU) {
      o = 0.5f * o * (1.0f + erff(o * 0.70710678118654752f));
    }
    if (m < M && n < N) Y[(long)m * ldy + n] = E<DT>::from_f(o);
  }
}

// linear_finish for the one-shot plans with 2 <= KW <= MT and a plain, gated or GELU epilogue: row tile t is finished
// by the waves of K slice t % KW, so every wave of the weight tile takes MT / KW of the tiles instead of slice 0
// taking all MT. The other slices' partials of a tile meet in LDS (`red`, free when this runs) and are added in
// slice order with the finishing wave's own (the sum linear_finish forms); the epilogue and stores are
// linear_finish's.
template <int DT, int MT, int NW, int KW, int EPI, bool PRO>
__device__ __forceinline__ void linear_finish_tiles(f32x4_t (&acc)[EPI == EPI_SWIGLU ? 2 : 1][MT], f32x4_t* red,
                                                    int wn, int wk, int lane, int n0, int m0,
                                                    uint16_t* __restrict__ Y, long ldy, int M, int N,
                                                    const float2* pst, const NormIn& ni) {
  constexpr int NA = EPI == EPI_SWIGLU ? 2 : 1;
  static_assert(KW > 1 && KW <= MT, "a row tile per slice");
  static_assert(EPI == EPI_NONE || EPI == EPI_SWIGLU || EPI == EPI_GELU, "plain, gated or GELU epilogue");
  const int li = lane & 15;
  const int lg = lane >> 4;
  auto slot = [&](int q, int a, int t) { return (((wn * KW + q) * NA + a) * MT + t) * 64 + lane; };
#pragma unroll
  for (int t = 0; t < MT; ++t)
    if (t % KW != wk) {
#pragma unroll
      for (int a = 0; a < NA; ++a) red[slot(wk, a, t)] = acc[a][t];
    }
  __syncthreads();
  const int n = n0 + 4 * lg;
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)Y) & 7) == 0 && n + 3 < N;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    if (t % KW != wk) continue;  // wave-uniform
    f32x4_t sum[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      sum[a] = wk == 0 ? acc[a][t] : red[slot(0, a, t)];
#pragma unroll
      for (int q = 1; q < KW; ++q) {
        const f32x4_t v = q == wk ? acc[a][t] : red[slot(q, a, t)];
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[a][r] = sum[a][r] + v[r];
      }
      if constexpr (PRO) norm_apply(sum[a], pst, 16 * t + li, ni, n, N, a);
    }
    const int m = m0 + 16 * t + li;
    if (m >= M) continue;
    uint16_t o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = rnd<DT>(sum[0][r]);
      if constexpr (EPI == EPI_SWIGLU) {
        v = rnd<DT>(silu16(v)) * rnd<DT>(sum[NA - 1][r]);
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

// EPI_QKR's second half: the workgroup's ROWS rows x HPW whole heads of the projection, rounded to bf16, sit in LDS
// (`tile`, row stride LDT halfwords, head hh of the workgroup at column 128 hh; workgroup nb holds heads
// nb * HPW ..). Each 16-lane DPP row takes one (row, head) item at a time: a query or key head through
// qk_norm_rope8 into q_out or the key cache, a value head into the value cache as is.
template <int ROWS, int HPW, int NT>
__device__ __forceinline__ void qk_items(const uint16_t* tile, int LDT, int nb, int m0, int M, const QkOut& qk) {
  constexpr int HD = 128;
  const int tid = threadIdx.x;
  const int t = tid & 15;
  for (int it = tid >> 4; it < ROWS * HPW; it += NT / 16) {
    const int r = it / HPW;
    const int hh = it - r * HPW;
    const int j = nb * HPW + hh;  // head of q|k|v (uniform in the DPP row)
    const int m = min(m0 + r, M - 1);
    // the host guarantees 0 <= pos < cap (lengths and offsets are non-negative, contexts are checked against the
    // capacity); the clamp keeps the write inside the slot's rows whatever pos holds
    const int ps = min(max(qk.pos[m], 0), qk.cap - 1);
    const long slot = qk.slots[m];
    const u16x8 xv = *reinterpret_cast<const u16x8*>(&tile[r * LDT + HD * hh + 8 * t]);
    if (j >= qk.H + qk.KV) {
      if (m0 + r < M) st16(qk.vc + slot * qk.sk_s + (long)(j - qk.H - qk.KV) * qk.sk_h + (long)ps * qk.sk_t + 8 * t, xv);
      continue;
    }
    const u16x8 wv = ld16((j < qk.H ? qk.wq : qk.wk) + 8 * t);
    const u16x8 cv = ld16(qk.cosb + (long)ps * qk.s_cos + 8 * t);
    const u16x8 sv = ld16(qk.sinb + (long)ps * qk.s_cos + 8 * t);
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = bf2f(xv.v[e]);
    const u16x8 ov = qk_norm_rope8<HD>(x, wv, cv, sv, qk.eps, t);
    if (m0 + r >= M) continue;
    if (j < qk.H)
      st16(qk.q + (long)(m0 + r) * qk.s_qb + (long)j * qk.s_qh + 8 * t, ov);
    else
      st16(qk.kc + slot * qk.sk_s + (long)(j - qk.H) * qk.sk_h + (long)ps * qk.sk_t + 8 * t, ov);
  }
}

// qk_items for a kernel that staged each row's clamped position and slot in LDS at its start (sps, ssl). DPP row g
// (of NT / 16) takes head g % HPW of rows g / HPW + (NT / 16 / HPW) k, and loads every cos/sin row of its items
// before the first is used: one round trip for all of them rather than a dependent pos -> cos/sin pair per item.
// Same arithmetic per item as qk_items.
template <int ROWS, int HPW, int NT>
__device__ __forceinline__ void qk_items_staged(const uint16_t* tile, int LDT, int nb, int m0, int M,
                                                const QkOut& qk, const int* sps, const long* ssl) {
  constexpr int HD = 128;
  constexpr int G = NT / 16;
  static_assert(G % HPW == 0 && (ROWS * HPW) % G == 0, "whole rows per DPP row");
  constexpr int IPG = ROWS * HPW / G;  // items per DPP row
  constexpr int RS = G / HPW;          // row stride between them
  const int tid = threadIdx.x;
  const int t = tid & 15;
  const int g = tid >> 4;
  const int hh = g % HPW;
  const int r0 = g / HPW;
  const int j = nb * HPW + hh;  // head of q|k|v (uniform in the DPP row)
  if (j >= qk.H + qk.KV) {
#pragma unroll
    for (int k = 0; k < IPG; ++k) {
      const int r = r0 + RS * k;
      if (m0 + r < M)
        st16(qk.vc + ssl[r] * qk.sk_s + (long)(j - qk.H - qk.KV) * qk.sk_h + (long)sps[r] * qk.sk_t + 8 * t,
             *reinterpret_cast<const u16x8*>(&tile[r * LDT + HD * hh + 8 * t]));
    }
    return;
  }
  const u16x8 wv = ld16((j < qk.H ? qk.wq : qk.wk) + 8 * t);
  u16x8 cv[IPG], sv[IPG];
#pragma unroll
  for (int k = 0; k < IPG; ++k) {
    const long ps = sps[r0 + RS * k];
    cv[k] = ld16(qk.cosb + ps * qk.s_cos + 8 * t);
    sv[k] = ld16(qk.sinb + ps * qk.s_cos + 8 * t);
  }
#pragma unroll
  for (int k = 0; k < IPG; ++k) {
    const int r = r0 + RS * k;
    const u16x8 xv = *reinterpret_cast<const u16x8*>(&tile[r * LDT + HD * hh + 8 * t]);
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = bf2f(xv.v[e]);
    const u16x8 ov = qk_norm_rope8<HD>(x, wv, cv[k], sv[k], qk.eps, t);
    if (m0 + r >= M) continue;
    if (j < qk.H)
      st16(qk.q + (long)(m0 + r) * qk.s_qb + (long)j * qk.s_qh + 8 * t, ov);
    else
      st16(qk.kc + ssl[r] * qk.sk_s + (long)(j - qk.H) * qk.sk_h + (long)sps[r] * qk.sk_t + 8 * t, ov);
  }
}

// One lane's 4 outputs (columns c .. c + 3 of the workgroup, row r) rounded to bf16 into the staged tile.
__device__ __forceinline__ void qk_stage(uint16_t* tile, int LDT, int r, int c, const f32x4_t& acc) {
  uint2 pk;
  pk.x = (uint32_t)f2bf(acc[0]) | ((uint32_t)f2bf(acc[1]) << 16);
  pk.y = (uint32_t)f2bf(acc[2]) | ((uint32_t)f2bf(acc[3]) << 16);
  *reinterpret_cast<uint2*>(&tile[r * LDT + c]) = pk;
}

// EPI_QKR epilogue of a one-shot workgroup with one K slice and NW = 8 HPW weight tiles (HPW whole heads of 128
// columns): the wave's tiles, with the folded norm applied, are staged in LDS (`tile`, free when this runs), then
// qk_items.
template <int MT, int NW, int NT, bool PRO>
__device__ __forceinline__ void qk_finish(f32x4_t (&acc)[1][MT], uint16_t* tile, int wn, int lane, int nb, int m0,
                                          int M, int N, const float2* pst, const NormIn& ni, const QkOut& qk) {
  static_assert(NW % 8 == 0, "whole heads per workgroup");
  constexpr int LDT = 16 * NW + 8;  // staged row stride, halfwords
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int n = (nb * NW + wn) * 16 + 4 * lg;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    if constexpr (PRO) norm_apply(acc[0][t], pst, 16 * t + li, ni, n, N, 0);
    qk_stage(tile, LDT, 16 * t + li, 16 * wn + 4 * lg, acc[0][t]);
  }
  __syncthreads();
  qk_items<16 * MT, NW / 8, NT>(tile, LDT, nb, m0, M, qk);
}

// PRO: the input rows' folded norm (NormIn; K == PRO_K): statistics loaded in the prologue, applied in the epilogue.
constexpr int PRO_K = 1024;

template <int DT, int MT, int NW, int EPI, bool PRO>
__global__ __launch_bounds__(256) void linear_kernel(const uint16_t* __restrict__ X, long ldx,
                                                     const uint16_t* __restrict__ Wp,
                                                     const uint16_t* __restrict__ W2p, uint16_t* __restrict__ Y,
                                                     long ldy, int M, int N, int K, int mblk, int nblk, NormIn ni,
                                                     ResidOut ro) {
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
  __shared__ float2 pst[PRO ? ROWS : 1];

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
  NormStage<ROWS, 256, PRO_K / 128> ns;
  if constexpr (PRO) ns.load(ni, m0, M, PRO_K);
  const int nch = ((ksteps + KW - 1) / KW + U - 1) / U;  // chunks per slice (equal for all slices)
  const int span = nch * U;
  const int s0 = wk * span;
  const int s1 = min(ksteps, s0 + span);

  const uint16_t* wp[NA];
  wp[0] = Wp + ((long)nt * ksteps * 64 + lane) * 8;
  if constexpr (DUAL) wp[NA - 1] = W2p + ((long)nt * ksteps * 64 + lane) * 8;

  // Activation vectors: v = tid + 256 j -> slice q, row r, 16-byte column c16 of the chunk.
  u16x8 X0[VPT], X1[VPT];
  auto xload = [&](int c, u16x8(&Xr)[VPT]) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      // clamped addresses, no branch (rows past M re-read row M - 1, steps past K the last step: never stored or
      // never multiplied)
      const int v = NVEC % 256 == 0 ? tid + 256 * j : min(tid + 256 * j, NVEC - 1);
      const int q = v / (ROWS * VPR);
      const int rem = v - q * (ROWS * VPR);
      const int r = rem / VPR;
      const int c16 = rem - r * VPR;
      const int m = min(m0 + r, M - 1);
      const int step = min(q * span + c * U + (c16 >> 2), ksteps - 1);
      Xr[j] = ld16(X + (long)m * ldx + step * 32 + (c16 & 3) * 8);
    }
  };
  auto xstore = [&](int buf, int c, const u16x8(&Xr)[VPT]) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      // threads past the block repeat the last vector's store (same value, same place): no branch
      const int v = NVEC % 256 == 0 ? tid + 256 * j : min(tid + 256 * j, NVEC - 1);
      const int q = v / (ROWS * VPR);
      const int rem = v - q * (ROWS * VPR);
      const int r = rem / VPR;
      const int c16 = rem - r * VPR;
      st16(&xs[buf][(q * ROWS + r) * LDR + c16 * 8], Xr[j]);
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
  ResidPre pre[MT];
  if constexpr (EPI == EPI_RESID) {
    if (wk == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) pre[t] = resid_prefetch(ro, m0 + 16 * t + li, n0 + 4 * lg, M, N);
    }
  }
  xstore(0, 0, X0);
  if (nch > 2) xload(2, X0);
  __syncthreads();
  for (int c = 0; c < nch; c += 2) {
    compute(c, 0, W0);
    if (c + 1 < nch) xstore(1, c + 1, X1);
    if (c + 3 < nch) xload(c + 3, X1);
    if (c + 2 < nch) wload(c + 2, W0);
    __syncthreads();
    if (c + 1 >= nch) break;
    compute(c + 1, 1, W1);
    if (c + 2 < nch) xstore(0, c + 2, X0);
    if (c + 4 < nch) xload(c + 4, X0);
    if (c + 3 < nch) wload(c + 3, W1);
    __syncthreads();
  }

  if constexpr (PRO) {  // the rows' scale and shift, from statistics that arrived long ago
    ns.finish(ni, m0, M, PRO_K, pst);
    __syncthreads();
  }
  linear_finish<DT, MT, NW, KW, EPI, PRO>(acc, reinterpret_cast<f32x4_t*>(&xs[0][0]), wn, wk, lane, n0, m0, Y,
                                          ldy, M, N, ro, pre, pst, ni);
}

// One-shot variant: every weight fragment of the wave's K slice (S steps of 32) and the workgroup's whole
// activation block are loaded at once, so the kernel pays one memory latency instead of one per chunk. A
// workgroup is NWAVES waves = NW weight tiles x KW = NWAVES / NW slices of K. With 8 or 16 waves the block may
// take up to 128 KB of gfx950's 160 KB LDS; one such workgroup per CU then streams its whole weight slab at
// once. The block sits in LDS unpadded when a slice row is a multiple of 16 granules of 16 bytes, with granule
// g of row r stored at g ^ (r % 16), so the 16 rows a fragment read touches fall in 16 different bank groups;
// otherwise rows are padded by 16 bytes.
// PRO (K == PRO_K): the tile statistics are requested before the activation block and merged into the rows' scale
// and shift after the products; the epilogue applies them. EPI_RESID: the residual operands are requested after the
// weight fragments.
template <int DT, int MT, int NW, int NWAVES, int EPI, int S, bool PRO>
__global__ __launch_bounds__(64 * NWAVES) void linear_oneshot_kernel(const uint16_t* __restrict__ X, long ldx,
                                                                     const uint16_t* __restrict__ Wp,
                                                                     const uint16_t* __restrict__ W2p,
                                                                     uint16_t* __restrict__ Y, long ldy, int M, int N,
                                                                     int K, int mblk, int nblk, NormIn ni,
                                                                     ResidOut ro, QkOut qk) {
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
  static_assert(!PRO || KW * KS == PRO_K, "the norm prologue covers K = PRO_K");
  __shared__ __align__(16) uint16_t xs[KW * ROWS * LDR];
  __shared__ float2 pst[PRO ? ROWS : 1];

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
  NormStage<ROWS, NT, PRO_K / 128> ns;
  if constexpr (PRO) ns.load(ni, m0, M, PRO_K);

  // The activation block is requested first and the weight fragments after it, in k order: the block's LDS store
  // then waits for the activations only, and the MFMAs of step s wait only for the fragments up to s (memory
  // returns in issue order), so the products run while the rest of the slab is still arriving. Measured at
  // 224 rows: 5-24 % faster than weights first (224 x 1024 x 3072: 9.2 -> 7.0 us).
  // activation vector v = tid + NT j -> slice q, row r, granule g
  // Loads come from addresses clamped into the block and below M (rows past M re-read row M - 1, whose products
  // in those columns are never stored): no branch around them, so no join waits for the loads in flight.
  u16x8 Xr[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int v = NVEC % NT == 0 ? tid + NT * j : min(tid + NT * j, NVEC - 1);
    const int q = v / (ROWS * GR);
    const int rem = v - q * (ROWS * GR);
    const int r = rem / GR;
    const int g = rem - r * GR;
    const int m = min(m0 + r, M - 1);
    Xr[j] = ld16(X + (long)m * ldx + q * KS + g * 8);
  }
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
  // the 16-wave plans over K >= 2816 have no registers to spare for the residual operands before the products:
  // they load them after
  constexpr bool EARLY = !(NWAVES == 16 && S > 16);
  ResidPre pre[MT];
  if constexpr (EPI == EPI_RESID && EARLY) {
    if (wk == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) pre[t] = resid_prefetch(ro, m0 + 16 * t + li, n0 + 4 * lg, M, N);
    }
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    // threads past the block repeat the last vector's store (same value, same place): no branch
    const int v = NVEC % NT == 0 ? tid + NT * j : min(tid + NT * j, NVEC - 1);
    const int q = v / (ROWS * GR);
    const int rem = v - q * (ROWS * GR);
    const int r = rem / GR;
    const int g = rem - r * GR;
    st16(&xs[(q * ROWS + r) * LDR + ((SWZ ? g ^ (r & 15) : g) << 3)], Xr[j]);
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
  if constexpr (PRO) ns.finish(ni, m0, M, PRO_K, pst);  // the rows' scale and shift, read after the barrier
  if constexpr (EPI == EPI_RESID && !EARLY) {
    if (wk == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) pre[t] = resid_prefetch(ro, m0 + 16 * t + li, n0 + 4 * lg, M, N);
    }
  }
  __syncthreads();  // every wave is done with the block before it holds the slice partials
  if constexpr (EPI == EPI_QKR) {
    static_assert(KW == 1 && DT == M3X_BF16, "one K slice, bf16");
    static_assert(ROWS * (16 * NW + 8) <= KW * ROWS * LDR, "the staged tile fits the block");
    qk_finish<MT, NW, NT, PRO>(acc, xs, wn, lane, nb, m0, M, N, pst, ni, qk);
  } else if constexpr (KW > 1 && KW <= MT && EPI != EPI_RESID) {
    static_assert(NW * KW * NA * MT * 1024 <= KW * ROWS * LDR * 2, "the partial tiles fit the block");
    linear_finish_tiles<DT, MT, NW, KW, EPI, PRO>(acc, reinterpret_cast<f32x4_t*>(xs), wn, wk, lane, n0, m0, Y, ldy, M,
                                                  N, pst, ni);
  } else if constexpr (KW >= 4 && EPI != EPI_RESID) {
    static_assert(NW * KW * NA * MT * 1024 <= KW * ROWS * LDR * 2, "the partial tiles fit the block");
    linear_finish_spread<DT, MT, NW, KW, EPI, PRO>(acc, reinterpret_cast<float*>(xs), wn, wk, lane, n0, m0, Y, ldy, M,
                                                   N, pst, ni);
  } else {
    linear_finish<DT, MT, NW, KW, EPI, PRO>(acc, reinterpret_cast<f32x4_t*>(xs), wn, wk, lane, n0, m0, Y, ldy, M, N,
                                            ro, pre, pst, ni);
  }
}

// Large-M projections (M > 512 rows: steps with inline prefills). A workgroup of 8 waves owns a 2-D tile of 128 (or
// 96: RT = 3) activation rows x 128 weight rows (for SwiGLU: 64 gate rows from W and the same 64 up rows from W2, i.e. 64
// output columns) and walks K in stages of 64. The packed weight fragments of a stage are copied to LDS as they are
// (16 fragments of 1 KB: every fragment read is one contiguous 1 KB); the activation rows sit row-major with a
// 144-byte row stride, so the 16 rows of a fragment read fall in 16 different bank groups and a row's 8 stores in
// distinct banks. The waves are 2 x 4 blocks of 16 RT activation rows x 32 weight rows (RT x 2 MFMA tiles; with
// SwiGLU a wave holds one gate tile and the matching up tile). Stages are double-buffered in LDS: the next stage's
// global loads are in flight while the current one multiplies, with one barrier per stage. Every weight byte is
// read by ceil(M / 32 RT) workgroups and every activation byte by ceil(N / 128), against 36 and 64 for the 64 x 64
// chunked tiles at 2264 rows. Global loads run two stages ahead of the products (three register sets in turn):
// measured 2-10 % faster than one stage ahead, most on the N = 1024 shapes whose grid has one workgroup per CU.
// PRO (K == PRO_K): the rows' folded norm, applied in the epilogue; its statistics (and EPI_RESID's operands) load
// after the products.
template <int DT, int EPI, bool PRO, int RT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void linear_tiled_kernel(const uint16_t* __restrict__ X, long ldx,
                                                              const uint16_t* __restrict__ Wp,
                                                              const uint16_t* __restrict__ W2p,
                                                              uint16_t* __restrict__ Y, long ldy, int M, int N, int K,
                                                              int mblk, int nblk, NormIn ni, ResidOut ro, QkOut qk) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int BM = 32 * RT;  // activation rows: 2 wave rows x RT tiles of 16
  static_assert(RT == 3 || RT == 4, "96- or 128-row blocks");
  constexpr int LDA = 72;  // activation row stride in LDS, halfwords
  __shared__ __align__(16) uint16_t lw[2][16 * 512];
  __shared__ __align__(16) uint16_t la[2][BM * LDA];
  __shared__ float2 pst[PRO ? BM : 1];

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
  const int wm = wave & 1;   // activation tiles RT wm .. RT wm + RT - 1
  const int wn = wave >> 1;  // weight tiles (below)
  const int ksteps = K >> 5;
  const int ntiles = (N + 15) >> 4;
  const int m0 = mb * BM;
  NormStage<BM, 512, PRO_K / 128> ns;

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
    // rows past M: re-read, never stored; with 96-row blocks the second slot's rows past the block repeat its
    // last row (the same value to the same LDS place)
    ga[j] = min(m0 + min((tid >> 3) + 64 * j, BM - 1), M - 1) * (int)ldx + 8 * (tid & 7);
  }
  int la0[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) la0[j] = min((tid >> 3) + 64 * j, BM - 1) * LDA + 8 * (tid & 7);
  // the wave's 2 weight tiles: plain 2 wn + i; SwiGLU gate wn and up 4 + wn
  int wt[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) wt[i] = DUAL ? (i == 0 ? wn : 4 + wn) : 2 * wn + i;

  f32x4_t acc[2][RT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < RT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // a stage's loads in r[0..1] (weight fragments) and r[2..3] (activation rows); stages past the end re-read the
  // last stage (valid addresses, never stored)
  const int nst = K >> 6;
  auto gload = [&](int stg, u16x8(&r)[4]) {
    const int sc = min(stg, nst - 1);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      r[j] = ld16((DUAL && j == 1 ? W2p : Wp) + gw[j] + sc * 1024);
      r[2 + j] = ld16(X + ga[j] + sc * 64);
    }
  };
  auto lstore = [&](int buf, const u16x8(&r)[4]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      st16(&lw[buf][tid * 8 + 4096 * j], r[j]);
      st16(&la[buf][la0[j]], r[2 + j]);
    }
  };
  auto compute = [&](int buf) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      u16x8 a[2], b[RT];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const u16x8*>(&lw[buf][(wt[i] * 2 + s) * 512 + lane * 8]);
#pragma unroll
      for (int j = 0; j < RT; ++j)
        b[j] = *reinterpret_cast<const u16x8*>(&la[buf][(16 * (RT * wm + j) + li) * LDA + 32 * s + 8 * lg]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < RT; ++j) acc[i][j] = mfma16x16x32<DT>(a[i], b[j], acc[i][j]);
    }
  };
  u16x8 R0[4], R1[4], R2[4];
  gload(0, R0);
  gload(1, R1);
  lstore(0, R0);
  __syncthreads();
  // Stage s issues the loads of stage s + 2, multiplies stage s from LDS buffer s % 2 and stores stage s + 1
  // (loaded during stage s - 1) to the other buffer: every load has two stages of products to arrive in. Three
  // register sets rotate with the stage, so the loop is unrolled by 6 (register set s % 3, buffer s % 2).
#define M3X_TILED_STAGE(S, RN, RS, BUF)        \
  if (s0 + S < nst) {                          \
    gload(s0 + S + 2, RN);                     \
    compute(BUF);                              \
    if (s0 + S + 1 < nst) lstore(BUF ^ 1, RS); \
    __syncthreads();                           \
  }
  for (int s0 = 0; s0 < nst; s0 += 6) {
    M3X_TILED_STAGE(0, R2, R1, 0)
    M3X_TILED_STAGE(1, R0, R2, 1)
    M3X_TILED_STAGE(2, R1, R0, 0)
    M3X_TILED_STAGE(3, R2, R1, 1)
    M3X_TILED_STAGE(4, R0, R2, 0)
    M3X_TILED_STAGE(5, R1, R0, 1)
  }
#undef M3X_TILED_STAGE

  // the epilogue's operands load after the products: held across the long K loop they would cost the registers
  // of a second workgroup per CU
  ResidPre pre[2][RT];
  if constexpr (EPI == EPI_RESID) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < RT; ++j)
        pre[i][j] = resid_prefetch(ro, m0 + 16 * (RT * wm + j) + li, (nb * 8 + wt[i]) * 16 + 4 * lg, M, N);
  }
  if constexpr (PRO) ns.load(ni, m0, M, PRO_K);

  if constexpr (PRO) {
    ns.finish(ni, m0, M, PRO_K, pst);  // the rows' scale and shift, from statistics that arrived long ago
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int n = DUAL ? (nb * 4 + wn) * 16 + 4 * lg : (nb * 8 + wt[i]) * 16 + 4 * lg;
#pragma unroll
      for (int j = 0; j < RT; ++j) norm_apply(acc[i][j], pst, 16 * (RT * wm + j) + li, ni, n, N, DUAL ? i : 0);
    }
  }
  if constexpr (EPI == EPI_RESID) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int tile = nb * 8 + wt[i];
#pragma unroll
      for (int j = 0; j < RT; ++j)
        resid_quad<DT>(acc[i][j], pre[i][j], m0 + 16 * (RT * wm + j) + li, tile * 16 + 4 * lg, tile, M, N, lg, ro, Y,
                       ldy);
    }
    return;
  }
  if constexpr (EPI == EPI_QKR) {
    // the workgroup's 128 columns are one head: stage the 128 x 128 tile in the activation buffers (free after the
    // loop's last barrier), then the per-head norm, RoPE and cache writes
    static_assert(DT == M3X_BF16 && BM * (128 + 8) <= 2 * BM * LDA, "the staged tile fits the activation buffers");
    constexpr int LDT = 128 + 8;
    uint16_t* tile = &la[0][0];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < RT; ++j) qk_stage(tile, LDT, 16 * (RT * wm + j) + li, 16 * wt[i] + 4 * lg, acc[i][j]);
    __syncthreads();
    qk_items<BM, 1, 512>(tile, LDT, nb, m0, M, qk);
    return;
  }

  // epilogue: lane (li, lg) of tile pair (i, j) holds weight rows 4 lg + r of tile wt[i] for activation row
  // m0 + 16 (RT wm + j) + li
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)Y) & 7) == 0;
  constexpr int NI = DUAL ? 1 : 2;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int n = DUAL ? (nb * 4 + wn) * 16 + 4 * lg : (nb * 8 + wt[i]) * 16 + 4 * lg;
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int m = m0 + 16 * (RT * wm + j) + li;
      if (m >= M) continue;
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = rnd<DT>(acc[i][j][r]);
        if constexpr (DUAL) {
          const float g = v;
          const float u = rnd<DT>(acc[1][j][r]);
          v = rnd<DT>(silu16(g)) * u;
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

// Large-M projections in bf16, column strips (M > 512 rows; preferred over linear_tiled_kernel where an instance
// exists). A workgroup of 4 waves owns BM = 16 RT activation rows x 4 strips of NG weight tiles: wave w's strip is
// tiles (4 nb + w) NG .. + NG - 1 (16 NG columns; with SwiGLU NG gate tiles and the same NG up tiles). A wave loads
// its strip's packed fragments from global memory straight into its registers (a fragment is one contiguous 1 KB
// that no other wave of the workgroup reads), two K stages of 64 ahead in three register sets; only the activation
// rows pass through LDS (double-buffered, 144-byte row stride), where all 4 waves read them. Against the 2-D tiles
// of linear_tiled_kernel, where every wave reads both operands from LDS, this cuts the LDS traffic per product by
// more than half (measured at 2264 rows: waves waiting on LDS issue 27 % -> 3 % of their cycles; q|k|v 34 -> 27.5
// us, gate|up + SwiGLU 47 -> 40 us, down 38 -> 28 us with its substep-pipelined reads). Products accumulate in the same K order with the same MFMA as
// linear_tiled_kernel, so the two kernels give the same bits. Epilogues as linear_tiled_kernel's; EPI_QKR needs
// BN = 64 NG to hold whole heads of 128 columns (2 per workgroup at NG = 4).
template <int DT, int EPI, bool PRO, int RT, int NG>
__global__ __launch_bounds__(256) void linear_strip_kernel(const uint16_t* __restrict__ X, long ldx,
                                                          const uint16_t* __restrict__ Wp,
                                                          const uint16_t* __restrict__ W2p, uint16_t* __restrict__ Y,
                                                          long ldy, int M, int N, int K, int mblk, int nblk,
                                                          NormIn ni, ResidOut ro, QkOut qk) {
  constexpr bool DUAL = EPI == EPI_SWIGLU;
  constexpr int NA = DUAL ? 2 : 1;           // weight operands (gate, up)
  constexpr int BM = 16 * RT;                // activation rows per workgroup
  constexpr int LDA = 72;                    // activation row stride in LDS, halfwords
  constexpr int CPT = (BM * 8 + 255) / 256;  // 16-byte activation chunks per thread and stage
  constexpr int BN = 64 * NG;                // columns per workgroup
  constexpr int LDT = BN + 8;                // EPI_QKR's staged tile row stride, halfwords
  constexpr int LDS_A = 2 * BM * LDA;
  constexpr int LDS_T = EPI == EPI_QKR ? BM * LDT : 0;
  __shared__ __align__(16) uint16_t smem[LDS_A > LDS_T ? LDS_A : LDS_T];
  __shared__ float2 pst[PRO ? BM : 1];
  __shared__ int sps[EPI == EPI_QKR ? BM : 1];    // EPI_QKR: the rows' clamped positions
  __shared__ long ssl[EPI == EPI_QKR ? BM : 1];   // and slots
  uint16_t* const la0 = smem;
  uint16_t* const la1 = smem + BM * LDA;

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
  const int ksteps = K >> 5;
  const int ntiles = (N + 15) >> 4;
  const int m0 = mb * BM;
  const int t0 = (nb * 4 + wave) * NG;  // the wave's first weight tile
  NormStage<BM, 256, PRO_K / 128> ns;

  // 32-bit element offsets (the host checks that both operands fit). Tiles past N and rows past M are read at a
  // valid clamped place and never stored; activation chunks past the block repeat row BM - 1 (the same value to
  // the same LDS place).
  int wo[NG];
#pragma unroll
  for (int i = 0; i < NG; ++i) wo[i] = min(t0 + i, ntiles - 1) * ksteps * 512 + lane * 8;
  int ga[CPT], lo[CPT];
#pragma unroll
  for (int q = 0; q < CPT; ++q) {
    const int c = tid + 256 * q;
    const int r = min(c >> 3, BM - 1);
    ga[q] = min(m0 + r, M - 1) * (int)ldx + 8 * (c & 7);
    lo[q] = r * LDA + 8 * (c & 7);
  }

  f32x4_t acc[NA][NG][RT];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int j = 0; j < RT; ++j) acc[a][i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // stages past the end re-read the last stage (valid addresses, never used)
  const int nst = K >> 6;
  auto wload = [&](int stg, u16x8(&w)[NA][NG][2]) {
    const int sc = min(stg, nst - 1);
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int s = 0; s < 2; ++s) w[a][i][s] = ld16((a ? W2p : Wp) + wo[i] + (2 * sc + s) * 512);
  };
  auto aload = [&](int stg, u16x8(&r)[CPT]) {
    const int sc = min(stg, nst - 1);
#pragma unroll
    for (int q = 0; q < CPT; ++q) r[q] = ld16(X + ga[q] + sc * 64);
  };
  auto astore = [&](uint16_t* buf, const u16x8(&r)[CPT]) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) st16(buf + lo[q], r[q]);
  };
  auto compute = [&](const uint16_t* buf, const u16x8(&w)[NA][NG][2]) {
    if constexpr (NA * NG <= 2) {
      // two products per activation fragment leave its LDS latency exposed: substep 0's fragments are read
      // first, then substep 1's reads go out under substep 0's products (measured at 2264 rows: o 24.1 -> 21.8 us,
      // down 31.8 -> 28.3 us; with 4 products per fragment the extra registers cost the second workgroup per CU)
      u16x8 b0[RT], b1[RT];
#pragma unroll
      for (int j = 0; j < RT; ++j) b0[j] = *reinterpret_cast<const u16x8*>(buf + (16 * j + li) * LDA + 8 * lg);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < RT; ++j) b1[j] = *reinterpret_cast<const u16x8*>(buf + (16 * j + li) * LDA + 32 + 8 * lg);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int i = 0; i < NG; ++i) acc[a][i][j] = mfma16x16x32<DT>(w[a][i][0], b0[j], acc[a][i][j]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int i = 0; i < NG; ++i) acc[a][i][j] = mfma16x16x32<DT>(w[a][i][1], b1[j], acc[a][i][j]);
    } else {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < RT; ++j) {
          const u16x8 b = *reinterpret_cast<const u16x8*>(buf + (16 * j + li) * LDA + 32 * s + 8 * lg);
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int i = 0; i < NG; ++i) acc[a][i][j] = mfma16x16x32<DT>(w[a][i][s], b, acc[a][i][j]);
        }
    }
  };
  // The epilogue's row operands are read here, with the first stages' loads, and kept in LDS, so that no global
  // round trip is left after the products: EPI_QKR's positions and slots (loads clamped to valid rows, no branch
  // around them) and PRO's row scale and shift (measured at 2264 rows inside the mixed step: gate|up + SwiGLU +
  // norm 45.9 -> 43.0 us, q|k|v + norm + RoPE + cache 38.5 -> 33.0 us).
  int qps = 0;
  long qsl = 0;
  if constexpr (EPI == EPI_QKR) {
    const int m = min(m0 + min(tid, BM - 1), M - 1);
    qps = min(max(qk.pos[m], 0), qk.cap - 1);  // 0 <= pos < cap from the host; the clamp keeps writes in the slot
    qsl = qk.slots[m];
  }
  if constexpr (PRO) ns.load(ni, m0, M, PRO_K);
  u16x8 W0[NA][NG][2], W1[NA][NG][2], W2[NA][NG][2];
  u16x8 A0[CPT], A1[CPT];
  wload(0, W0);
  aload(0, A0);
  wload(1, W1);
  aload(1, A1);
  if constexpr (EPI == EPI_QKR) {
    if (tid < BM) {
      sps[tid] = qps;
      ssl[tid] = qsl;
    }
  }
  if constexpr (PRO) ns.finish(ni, m0, M, PRO_K, pst);
  astore(la0, A0);
  __syncthreads();
  // Stage s issues the weights (register set s + 2 mod 3) and activations (set s mod 2, stored to LDS during stage
  // s - 1) of stage s + 2, multiplies stage s (weights from set s mod 3, activations from LDS buffer s mod 2),
  // stores stage s + 1's activations to the other buffer, then meets the workgroup: unrolled by 6.
#define M3X_STRIP_STAGE(S, WN, WC, AN, AS, BUF, OBUF) \
  if (s0 + S < nst) {                                 \
    wload(s0 + S + 2, WN);                            \
    aload(s0 + S + 2, AN);                            \
    compute(BUF, WC);                                 \
    if (s0 + S + 1 < nst) astore(OBUF, AS);           \
    __syncthreads();                                  \
  }
  for (int s0 = 0; s0 < nst; s0 += 6) {
    M3X_STRIP_STAGE(0, W2, W0, A0, A1, la0, la1)
    M3X_STRIP_STAGE(1, W0, W1, A1, A0, la1, la0)
    M3X_STRIP_STAGE(2, W1, W2, A0, A1, la0, la1)
    M3X_STRIP_STAGE(3, W2, W0, A1, A0, la1, la0)
    M3X_STRIP_STAGE(4, W0, W1, A0, A1, la0, la1)
    M3X_STRIP_STAGE(5, W1, W2, A1, A0, la1, la0)
  }
#undef M3X_STRIP_STAGE

  // the epilogue's operands load after the products, as in linear_tiled_kernel
  ResidPre pre[EPI == EPI_RESID ? NG : 1][RT];
  if constexpr (EPI == EPI_RESID) {
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int j = 0; j < RT; ++j) pre[i][j] = resid_prefetch(ro, m0 + 16 * j + li, (t0 + i) * 16 + 4 * lg, M, N);
  }
  if constexpr (PRO) {
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int j = 0; j < RT; ++j) norm_apply(acc[a][i][j], pst, 16 * j + li, ni, (t0 + i) * 16 + 4 * lg, N, a);
  }
  if constexpr (EPI == EPI_RESID) {
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int j = 0; j < RT; ++j)
        resid_quad<DT>(acc[0][i][j], pre[i][j], m0 + 16 * j + li, (t0 + i) * 16 + 4 * lg, t0 + i, M, N, lg, ro, Y,
                       ldy);
    return;
  }
  if constexpr (EPI == EPI_QKR) {
    static_assert(DT == M3X_BF16 && BN % 128 == 0, "bf16, whole heads per workgroup");
    // the workgroup's BN columns are BN / 128 heads: stage the tile in LDS (free after the loop's last barrier),
    // then the per-head norm, RoPE and cache writes
    uint16_t* tile = smem;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int j = 0; j < RT; ++j) qk_stage(tile, LDT, 16 * j + li, 16 * (wave * NG + i) + 4 * lg, acc[0][i][j]);
    __syncthreads();
    qk_items_staged<BM, BN / 128, 256>(tile, LDT, nb, m0, M, qk, sps, ssl);
    return;
  }
  // lane (li, lg) of tile (i, j) holds columns 4 lg + r of weight tile t0 + i for activation row m0 + 16 j + li
  const bool vec = (ldy & 3) == 0 && (((uintptr_t)Y) & 7) == 0;
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const int n = (t0 + i) * 16 + 4 * lg;
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int m = m0 + 16 * j + li;
      if (m >= M) continue;
      uint16_t o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = rnd<DT>(acc[0][i][j][r]);
        if constexpr (DUAL) {
          const float u = rnd<DT>(acc[1][i][j][r]);
          v = rnd<DT>(silu16(v)) * u;
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

// The strip plan's geometry: 80-row blocks (RT = 5; measured best of 5, 8, 9 and 15 at 2264 and 4096 rows, with two
// workgroups per CU), 4 weight tiles per wave (2 gate + 2 up pairs with SwiGLU, 2 for the residual projections,
// whose N = 1024 otherwise leaves too few workgroups).
constexpr int STRIP_RT = 5;
template <int EPI>
constexpr int strip_ng() {
  return EPI == EPI_SWIGLU || EPI == EPI_RESID ? 2 : 4;
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
    p.nw = dual ? 4 : 8;
    p.oneshot = 0;
    p.nblk = m3x_ceil_div(ntiles, p.nw);
    // 96- or 128-row blocks, whichever gives the fewer rows per CU over the rounds of two workgroups per CU
    // (measured at 2264 rows: 96 is 9-11 % faster for q|k|v, o and down, 11 % slower for gate|up's 1,152 blocks)
    const long w6 = (long)m3x_ceil_div(M, 96) * p.nblk, w8 = (long)m3x_ceil_div(M, 128) * p.nblk;
    p.mt = (w6 + 511) / 512 * 96 < (w8 + 511) / 512 * 128 ? 6 : 8;
    p.mblk = m3x_ceil_div(M, 16 * p.mt);
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

// Launches the plan's kernel; false (nothing launched) for a plan no kernel instance covers. PRO instances exist
// for K = PRO_K only, EPI_RESID instances without PRO.
template <int DT, int EPI, bool PRO = false>
static bool launch_linear(const LinearPlan& p, hipStream_t st, const uint16_t* X, long ldx, const uint16_t* W,
                          const uint16_t* W2, uint16_t* Y, long ldy, int M, int N, int K, const NormIn& ni = NormIn{},
                          const ResidOut& ro = ResidOut{}, const QkOut& qk = QkOut{}) {
  static_assert(!(PRO && EPI == EPI_RESID), "a residual projection takes its input as is");
  const dim3 grid(m3x_ceil_div(p.nblk, 8) * 8 * p.mblk);
  if constexpr (DT == M3X_BF16) {
    // the tiled plan's shapes in bf16 take the strip kernel (EPI_QKR: when its 256-column blocks hold whole heads)
    constexpr int NG = strip_ng<EPI>();
    if (p.tiled && (EPI != EPI_QKR || N % (64 * NG) == 0)) {
      const int nblk = m3x_ceil_div(m3x_ceil_div(N, 16), 4 * NG);
      const int mblk = m3x_ceil_div(M, 16 * STRIP_RT);
      hipLaunchKernelGGL((linear_strip_kernel<DT, EPI, PRO, STRIP_RT, NG>), dim3(m3x_ceil_div(nblk, 8) * 8 * mblk),
                         dim3(256), 0, st, X, ldx, W, W2, Y, ldy, M, N, K, mblk, nblk, ni, ro, qk);
      return true;
    }
  }
  if constexpr (EPI == EPI_QKR) {
    // whole heads per workgroup: the tiled plan (128 columns) or the one-shot plan of 8 weight tiles in one K slice
    if (p.tiled) {
      if (p.mt == 6)
        hipLaunchKernelGGL((linear_tiled_kernel<DT, EPI_QKR, PRO, 3>), grid, dim3(512), 0, st, X, ldx, W, W2, Y, ldy,
                           M, N, K, p.mblk, p.nblk, ni, ro, qk);
      else
        hipLaunchKernelGGL((linear_tiled_kernel<DT, EPI_QKR, PRO, 4>), grid, dim3(512), 0, st, X, ldx, W, W2, Y, ldy,
                           M, N, K, p.mblk, p.nblk, ni, ro, qk);
      return true;
    }
    if (!p.oneshot || p.mt != 2 || p.nw != 8 || p.nwaves != 8 || p.oneshot != 32) return false;
    hipLaunchKernelGGL((linear_oneshot_kernel<DT, 2, 8, 8, EPI_QKR, 32, PRO>), grid, dim3(512), 0, st, X, ldx, W, W2,
                       Y, ldy, M, N, K, p.mblk, p.nblk, ni, ro, qk);
    return true;
  } else {
  if (p.tiled) {
    if (p.mt == 6)
      hipLaunchKernelGGL((linear_tiled_kernel<DT, EPI, PRO, 3>), grid, dim3(512), 0, st, X, ldx, W, W2, Y, ldy, M, N,
                         K, p.mblk, p.nblk, ni, ro, qk);
    else
      hipLaunchKernelGGL((linear_tiled_kernel<DT, EPI, PRO, 4>), grid, dim3(512), 0, st, X, ldx, W, W2, Y, ldy, M, N,
                         K, p.mblk, p.nblk, ni, ro, qk);
    return true;
  }
#define M3X_ONE(MTT, NWW, NWV, SS)                                                                              \
  if constexpr (!PRO || (NWV / NWW) * SS * 32 == PRO_K) {                                                     \
    hipLaunchKernelGGL((linear_oneshot_kernel<DT, MTT, NWW, NWV, EPI, SS, PRO>), grid, dim3(64 * NWV), 0, st, X, \
                       ldx, W, W2, Y, ldy, M, N, K, p.mblk, p.nblk, ni, ro, qk);                              \
    return true;                                                                                              \
  }                                                                                                           \
  return false
  if (p.oneshot) {
    const long key = ((p.mt * 10L + p.nw) * 100 + p.nwaves) * 100 + p.oneshot;
    switch (key) {
      case 120416: M3X_ONE(1, 2, 4, 16);
      case 120408: M3X_ONE(1, 2, 4, 8);
      case 110416: M3X_ONE(1, 1, 4, 16);
      case 110408: M3X_ONE(1, 1, 4, 8);
      case 140416: M3X_ONE(1, 4, 4, 16);
      case 140408: M3X_ONE(1, 4, 4, 8);
      case 220416: M3X_ONE(2, 2, 4, 16);
      case 220408: M3X_ONE(2, 2, 4, 8);
      case 240416: M3X_ONE(2, 4, 4, 16);
      case 240408: M3X_ONE(2, 4, 4, 8);
      case 210408: M3X_ONE(2, 1, 4, 8);
      // up to 16 rows, K = 1024 / 2048 / 2816 / 3072
      case 110804: M3X_ONE(1, 1, 8, 4);
      case 110808: M3X_ONE(1, 1, 8, 8);
      case 110811: M3X_ONE(1, 1, 8, 11);
      case 110812: M3X_ONE(1, 1, 8, 12);
      // wide, K = 1024
      case 220808: M3X_ONE(2, 2, 8, 8);
      case 240816: M3X_ONE(2, 4, 8, 16);
      case 340816: M3X_ONE(3, 4, 8, 16);
      case 280832: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(2, 8, 8, 32); } return false;
      // wide, K = 2048 / 2816 / 3072
      case 141616: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 4, 16, 16); } return false;
      case 121608: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 2, 16, 8); } return false;
      case 141622: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 4, 16, 22); } return false;
      case 121611: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 2, 16, 11); } return false;
      case 141624: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 4, 16, 24); } return false;
      case 121612: if constexpr (EPI != EPI_SWIGLU) { M3X_ONE(1, 2, 16, 12); } return false;
      default: return false;
    }
  }
#undef M3X_ONE
#define M3X_LIN(MTT, NWW)                                                                                    \
  hipLaunchKernelGGL((linear_kernel<DT, MTT, NWW, EPI, PRO>), grid, dim3(256), 0, st, X, ldx, W, W2, Y, ldy, M, N, \
                     K, p.mblk, p.nblk, ni, ro)
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
}
