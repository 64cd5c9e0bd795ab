// Mimi one-frame decode (serve/fast_codec.py StaticMimi, :32-277): the kernels around the projections and
// convolutions, which run as GEMMs on m3x_linear. Activations are time-major [rows = seat * T + t, channels] in
// 16-bit with fp32 arithmetic. Every stateful layer keeps one row per slot (the reference's conv_flat / kv /
// key_pos rows); several padding seats of a batch may name the one dummy slot, whose rows are scratch.
#include "m3x_common.h"

// Stateful kernels split a seat's rows over workgroups (blockIdx.y); the chunk is at least the state's depth, so
// only chunk 0 reads the old state, and chunk 0 alone writes the new state after a barrier. A thread keeps at
// most CODEC_KEEP state values across that barrier.
constexpr int CODEC_THREADS = 256;
constexpr int CODEC_KEEP = 16;
constexpr long NEVER_POS = -(1L << 40);  // key_pos of an empty ring entry

// ELU (alpha 1). 16-bit storage: the hardware exp, exp(v) - 1 for v <= 0, absolute error ~1e-7, below the storage
// step of every value it produces. fp32 storage: expm1f, accurate to an ulp of the result near 0 as well.
template <int DT> __device__ __forceinline__ float elu(float v) {
  if constexpr (DT == M3X_F32) return v > 0.f ? v : expm1f(v);
  else return v > 0.f ? v : __expf(v) - 1.f;
}

// ---------------------------------------------------------------------------------------------------------
// RVQ decode (:134-149; transformers MimiSplitResidualVectorQuantizer.decode): out[b, :dim] = table_0[code_0]
// (the semantic codebook), out[b, dim:] = dt(table_1[code_1] + ... + table_{nq-1}[code_{nq-1}]) summed in fp32 in
// that order. A GEMM with [W_semantic | W_acoustic] then applies both 1x1 output projections and their sum.
// Codes outside [0, n_codes) are clamped into it (the reference's embedding lookup raises on them).
template <int DT>
__global__ __launch_bounds__(256) void rvq_decode_kernel(const int64_t* __restrict__ codes, long ld_codes,
                                                         const Elt<DT>* __restrict__ tables, Elt<DT>* __restrict__ out,
                                                         long ld_out, int nq, int n_codes, int dim) {
  const int b = blockIdx.x;
  const int64_t* c = codes + (long)b * ld_codes;
  auto code = [&](int q) -> long { return (long)min(max(c[q], (int64_t)0), (int64_t)(n_codes - 1)); };
  for (int d = threadIdx.x; d < dim; d += blockDim.x) {
    out[(long)b * ld_out + d] = tables[code(0) * dim + d];
    float s = 0.f;
    int q = 1;
    for (; q + 8 <= nq; q += 8) {  // eight rows' loads in flight, then added in codebook order
      Elt<DT> v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = tables[((long)(q + u) * n_codes + code(q + u)) * dim + d];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += E<DT>::to_f(v[u]);
    }
    for (; q < nq; ++q) s += E<DT>::to_f(tables[((long)q * n_codes + code(q)) * dim + d]);
    out[(long)b * ld_out + dim + d] = E<DT>::from_f(s);
  }
}

// ---------------------------------------------------------------------------------------------------------
// Upsample (:186-188 -> :112-130): depthwise transposed conv with kernel k <= 2 s, stride s, no bias, one input
// frame per seat: out[b * s + j, c] = x[b, c] w[c, j] + tail[slot, j, c] (j < k - s); the new tail[slot, j - s, c]
// = x[b, c] w[c, j] for j >= s. Each thread owns channels, so its tail reads precede its tail writes.
template <int DT>
__global__ __launch_bounds__(256) void dwconvt_kernel(const Elt<DT>* __restrict__ x, long ld_x,
                                                      const Elt<DT>* __restrict__ w, Elt<DT>* tail, long ld_tail,
                                                      const int64_t* __restrict__ slots, Elt<DT>* __restrict__ out,
                                                      int C, int k, int s) {
  const int b = blockIdx.x;
  Elt<DT>* tl = tail + slots[b] * ld_tail;  // [k - s][C]
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    const float xv = E<DT>::to_f(x[(long)b * ld_x + c]);
    for (int j = 0; j < s; ++j) {
      const float prev = j < k - s ? E<DT>::to_f(tl[(long)j * C + c]) : 0.f;
      out[((long)b * s + j) * C + c] = E<DT>::from_f(xv * E<DT>::to_f(w[(long)c * k + j]) + prev);
    }
    for (int j = s; j < k; ++j) tl[(long)(j - s) * C + c] = E<DT>::from_f(xv * E<DT>::to_f(w[(long)c * k + j]));
  }
}

// ---------------------------------------------------------------------------------------------------------
// Causal conv input as GEMM rows (:104-111): cols[b * T + t, j * C + c] = joined[t + j * dil][c], where joined =
// the slot's pad = (k - 1) * dil stored frames followed by act(x[b * T + 0 .. T)), act = ELU (alpha 1) when
// use_elu, the ELU module in front of the conv. The slot's state becomes joined's last pad frames (post-ELU, as
// the reference stores the conv's own input). Grid (B, ceil(T / chunk)), chunk >= pad; 8 channels per thread.
// cols == NULL only advances the history (after an m3x_conv_gemm that read it in place of the gathered rows).
template <int DT>
__device__ __forceinline__ V8<DT> joined8(const Elt<DT>* st, const Elt<DT>* x, long ld_x, long row0, int pad, int i,
                                         int c, int C, int use_elu) {
  if (i < pad) return ldv<DT>(st + (long)i * C + c);
  V8<DT> v = ldv<DT>(x + (row0 + i - pad) * ld_x + c);
  if (use_elu) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v.v[e] = E<DT>::from_f(elu<DT>(E<DT>::to_f(v.v[e])));
  }
  return v;
}

template <int DT>
__global__ __launch_bounds__(CODEC_THREADS) void conv_gather_kernel(const Elt<DT>* __restrict__ x, long ld_x,
                                                                    Elt<DT>* state, long ld_state,
                                                                    const int64_t* __restrict__ slots,
                                                                    Elt<DT>* __restrict__ cols, long ld_cols, int T,
                                                                    int C, int k, int dil, int use_elu, int chunk) {
  const int b = blockIdx.x;
  const int t0 = blockIdx.y * chunk, t1 = min(T, t0 + chunk);
  const int pad = (k - 1) * dil;
  const long row0 = (long)b * T;
  Elt<DT>* st = pad ? state + slots[b] * ld_state : nullptr;  // [pad][C]
  const int cv = C / 8, kcv = k * cv;
  for (int e = threadIdx.x; cols && e < (t1 - t0) * kcv; e += CODEC_THREADS) {
    const int t = t0 + e / kcv;
    const int r = e - (t - t0) * kcv;
    const int j = r / cv, c = 8 * (r - j * cv);
    stv<DT>(cols + (row0 + t) * ld_cols + (long)j * C + c, joined8<DT>(st, x, ld_x, row0, pad, t + j * dil, c, C, use_elu));
  }
  if (!pad || blockIdx.y) return;
  V8<DT> keep[CODEC_KEEP / 8];  // constant indices: registers, not a private or LDS array
#pragma unroll
  for (int p = 0; p < CODEC_KEEP / 8; ++p) {
    const int e = threadIdx.x + CODEC_THREADS * p;
    if (e < pad * cv) keep[p] = joined8<DT>(st, x, ld_x, row0, pad, T + e / cv, 8 * (e % cv), C, use_elu);
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < CODEC_KEEP / 8; ++p) {
    const int e = threadIdx.x + CODEC_THREADS * p;
    if (e < pad * cv) stv<DT>(st + 8 * e, keep[p]);
  }
}

// ---------------------------------------------------------------------------------------------------------
// Row op: out = act(res + scale * (g + bias)); bias, scale, res may be NULL; act = ELU (alpha 1) when use_elu.
// Serves the conv biases (with the resnet shortcut and the ELU that follows it) and the transformer's
// layer-scaled residuals. C % 8 == 0, 16-byte rows.
template <int DT>
__global__ __launch_bounds__(256) void rows_op_kernel(const Elt<DT>* __restrict__ g, long ld_g,
                                                      const Elt<DT>* __restrict__ bias,
                                                      const Elt<DT>* __restrict__ scale, const Elt<DT>* res,
                                                      long ld_res, Elt<DT>* out, long ld_out, int rows, int C,
                                                      int use_elu) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int cv = C / 8;
  if (i >= (long)rows * cv) return;
  const long r = i / cv;
  const int c = 8 * (int)(i - r * cv);
  const V8<DT> gv = ldv<DT>(g + r * ld_g + c);
  V8<DT> bv = zero_v8<DT>(), sv = zero_v8<DT>(), rv = zero_v8<DT>(), ov;
  if (bias) bv = ldv<DT>(bias + c);
  if (scale) sv = ldv<DT>(scale + c);
  if (res) rv = ldv<DT>(res + r * ld_res + c);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float v = E<DT>::to_f(gv.v[e]);
    if (bias) v = v + E<DT>::to_f(bv.v[e]);
    if (scale) v = E<DT>::to_f(sv.v[e]) * v;
    if (res) v = E<DT>::to_f(rv.v[e]) + v;
    if (use_elu) v = elu<DT>(v);
    ov.v[e] = E<DT>::from_f(v);
  }
  stv<DT>(out + r * ld_out + c, ov);
}

// ---------------------------------------------------------------------------------------------------------
// Layer-scaled residual then LayerNorm over rows of 512: h = dt(h + scale * a) (the arithmetic of m3x_rows_op),
// y = dt((h - mean) / sqrt(var + eps) * w + b) with fp32 statistics. One wave per row. Serves the decoder
// transformer's `h = h + layer_scale(a)` followed by the next LayerNorm (serve/fast_codec.py:181-182,172,182).
constexpr int RLN_N = 512;
template <int DT>
__global__ __launch_bounds__(256) void resid_ln_kernel(Elt<DT>* h, long ld_h, const Elt<DT>* __restrict__ a,
                                                       long ld_a, const Elt<DT>* __restrict__ scale,
                                                       const Elt<DT>* __restrict__ w, const Elt<DT>* __restrict__ b,
                                                       Elt<DT>* __restrict__ y, long ld_y, float eps, int rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // a whole wave; the kernel has no block barrier
  const int c = 8 * (threadIdx.x & 63);
  const V8<DT> hv = ldv<DT>(h + row * ld_h + c), av = ldv<DT>(a + row * ld_a + c), sv = ldv<DT>(scale + c);
  float v[8];
  V8<DT> ho;
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float t = E<DT>::to_f(sv.v[e]) * E<DT>::to_f(av.v[e]);
    t = E<DT>::to_f(hv.v[e]) + t;
    ho.v[e] = E<DT>::from_f(t);
    v[e] = E<DT>::to_f(ho.v[e]);
    sum += v[e];
  }
  stv<DT>(h + row * ld_h + c, ho);
  const float mean = wave_sum_xor(sum, 64) / (float)RLN_N;
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v[e] = v[e] - mean;
    sq += v[e] * v[e];
  }
  const float inv = 1.f / sqrtf(wave_sum_xor(sq, 64) / (float)RLN_N + eps);
  const V8<DT> wv = ldv<DT>(w + c), bv = ldv<DT>(b + c);
  V8<DT> yo;
#pragma unroll
  for (int e = 0; e < 8; ++e) yo.v[e] = E<DT>::from_f(v[e] * inv * E<DT>::to_f(wv.v[e]) + E<DT>::to_f(bv.v[e]));
  stv<DT>(y + row * ld_y + c, yo);
}

// ---------------------------------------------------------------------------------------------------------
// Thin GEMM with the conv epilogue, for the SEANet convs with at most 128 output channels:
// y[m, n] = act(res[m, n] + (dt(x[m, :] . w[n, :]) + bias[n])) (m3x_linear's product, then m3x_rows_op's
// arithmetic), w packed by m3x_pack_weight, N = 16 NT, K % 32 == 0; bias and res optional, act = ELU when use_elu.
// Each wave owns 16 MT rows and the 16 NT columns of its column group (blockIdx.y; one group unless the rows alone
// make a small grid): the activation fragments are loaded straight into the MFMA's B operand (read once per column
// group), the weight fragments (cache resident) into A. A column group does not change any output's K order.
// Gathered form (G = 1): the conv's rows are read in place of a gathered copy. Row m = b * T + t, column
// kk = j * C + c of the product is joined[t + j * dil][c] (m3x_conv_gather's rows: the slot's pad stored frames,
// then x with ELU when pre_elu); the caller advances the history afterwards.
struct ConvSrc {
  const void* state;  // Elt<DT> rows
  long ld_state;
  const int64_t* slots;
  int T, C, dil, pad, pre_elu;
};

template <int DT, int NT, int MT, int G>
__global__ __launch_bounds__(256) void conv_gemm_kernel(const Elt<DT>* __restrict__ X, long ldx,
                                                        const Elt<DT>* __restrict__ Wp,
                                                        const Elt<DT>* __restrict__ bias, const Elt<DT>* res,
                                                        long ld_res, Elt<DT>* Y, long ldy, int M, int K,
                                                        int use_elu, ConvSrc cs) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, li = l & 15, lg = l >> 4;
  const long m0 = ((long)blockIdx.x * 4 + wave) * (16 * MT);
  if (m0 >= M) return;  // wave-uniform
  {  // column group blockIdx.y: columns 16 NT y .. 16 NT (y + 1) - 1
    const int n0 = 16 * NT * (int)blockIdx.y;
    Wp += (long)n0 * K;  // NT tiles of K / 32 fragments of 512 elements
    if (bias) bias += n0;
    if (res) res += n0;
    Y += n0;
  }
  f32x4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[t][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int ks = K / 32;
  // the fragments of step s + 1 are in flight while step s multiplies
  V8<DT> a[2][NT], b[2][MT];
  // gathered form: each row's seat, time and history row
  long xrow0[MT];
  int tt[MT];
  const Elt<DT>* hist[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const long row = m0 + 16 * j + li;
    xrow0[j] = 0, tt[j] = 0, hist[j] = nullptr;
    if (G && row < M) {
      const long bs = row / cs.T;
      tt[j] = (int)(row - bs * cs.T);
      xrow0[j] = bs * cs.T;
      hist[j] = cs.pad ? (const Elt<DT>*)cs.state + cs.slots[bs] * cs.ld_state : nullptr;
    }
  }
  auto load = [&](int s, int buf) {
    const int kk = 32 * s + 8 * lg;
    const int tap = G ? kk / cs.C : 0, c = G ? kk - tap * cs.C : 0;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const long row = m0 + 16 * j + li;
      b[buf][j] = zero_v8<DT>();
      if (row < M) {
        if (!G) {
          b[buf][j] = ldv<DT>(X + row * ldx + kk);
        } else {
          const int i = tt[j] + tap * cs.dil;
          if (i < cs.pad) {
            b[buf][j] = ldv<DT>(hist[j] + (long)i * cs.C + c);
          } else {
            b[buf][j] = ldv<DT>(X + (xrow0[j] + i - cs.pad) * ldx + c);
            if (cs.pre_elu) {
#pragma unroll
              for (int e = 0; e < 8; ++e) b[buf][j].v[e] = E<DT>::from_f(elu<DT>(E<DT>::to_f(b[buf][j].v[e])));
            }
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) a[buf][t] = ldv<DT>(Wp + ((long)t * ks + s) * 512 + 8 * l);
  };
  load(0, 0);
  for (int s = 0; s < ks; s += 2) {
    if (s + 1 < ks) load(s + 1, 1);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[t][j] = mfma_k32<DT>(a[0][t], b[0][j], acc[t][j]);
    if (s + 1 >= ks) break;
    if (s + 2 < ks) load(s + 2, 0);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[t][j] = mfma_k32<DT>(a[1][t], b[1][j], acc[t][j]);
  }
  // lane (li, lg) holds columns 16 t + 4 lg + r of row m0 + 16 j + li. res may be y itself (in place): every
  // residual and bias value of the lane is read before its first store.
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const long m = m0 + 16 * j + li;
    if (m >= M) continue;
    if constexpr (DT == M3X_F32) {
      float4 bb[NT], rr[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int n = 16 * t + 4 * lg;
        bb[t] = bias ? *reinterpret_cast<const float4*>(bias + n) : make_float4(0.f, 0.f, 0.f, 0.f);
        rr[t] = res ? *reinterpret_cast<const float4*>(res + m * ld_res + n) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int n = 16 * t + 4 * lg;
        const float bv[4] = {bb[t].x, bb[t].y, bb[t].z, bb[t].w}, rv[4] = {rr[t].x, rr[t].y, rr[t].z, rr[t].w};
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = acc[t][j][r];
          if (bias) v = v + bv[r];
          if (res) v = rv[r] + v;
          if (use_elu) v = elu<DT>(v);
          o[r] = v;
        }
        *reinterpret_cast<float4*>(Y + m * ldy + n) = make_float4(o[0], o[1], o[2], o[3]);
      }
    } else {
      uint2 bb[NT], rr[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int n = 16 * t + 4 * lg;
        bb[t] = bias ? *reinterpret_cast<const uint2*>(bias + n) : uint2{0, 0};
        rr[t] = res ? *reinterpret_cast<const uint2*>(res + m * ld_res + n) : uint2{0, 0};
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int n = 16 * t + 4 * lg;
        const uint16_t* bv = reinterpret_cast<const uint16_t*>(&bb[t]);
        const uint16_t* rv = reinterpret_cast<const uint16_t*>(&rr[t]);
        uint16_t o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = rnd<DT>(acc[t][j][r]);
          if (bias) v = v + E<DT>::to_f(bv[r]);
          if (res) v = E<DT>::to_f(rv[r]) + v;
          if (use_elu) v = elu<DT>(v);
          o[r] = E<DT>::from_f(v);
        }
        *reinterpret_cast<uint2*>(Y + m * ldy + n) = *reinterpret_cast<const uint2*>(o);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Transposed conv overlap-add (:112-130). cols[b * Tin + t, j * C + c] = x[b, t] . W[:, c, j] comes from the GEMM;
// output frame o < Tin * s of seat b is the sum of its contributions (t, j = o - t s, 0 <= j < k) + tail[slot, o, c]
// (o < k - s) + bias[c]; the new tail[slot, i, c] = the contributions to frame Tin * s + i, without bias (the
// reference stores its tail bias-free). Grid (B, ceil(Tin * s / chunk)), chunk >= k - s; 8 channels per thread.
template <int DT>
__device__ __forceinline__ void convt_frame8(const Elt<DT>* cols, long ld_cols, long row0, int o, int c, int Tin,
                                             int C, int k, int s, float (&v)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = 0.f;
  for (int t = min(o / s, Tin - 1); t >= 0 && o - t * s < k; --t) {
    const V8<DT> w = ldv<DT>(cols + (row0 + t) * ld_cols + (long)(o - t * s) * C + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += E<DT>::to_f(w.v[e]);
  }
}

template <int DT>
__global__ __launch_bounds__(CODEC_THREADS) void convt_overlap_kernel(const Elt<DT>* __restrict__ cols, long ld_cols,
                                                                      Elt<DT>* tail, long ld_tail,
                                                                      const int64_t* __restrict__ slots,
                                                                      const Elt<DT>* __restrict__ bias,
                                                                      Elt<DT>* __restrict__ out, long ld_out, int Tin,
                                                                      int C, int k, int s, int chunk) {
  const int b = blockIdx.x;
  const int nout = Tin * s, ov = k - s;
  const int o0 = blockIdx.y * chunk, o1 = min(nout, o0 + chunk);
  const long row0 = (long)b * Tin;
  Elt<DT>* tl = tail + slots[b] * ld_tail;  // [k - s][C]
  const int cv = C / 8;
  for (int e = threadIdx.x; e < (o1 - o0) * cv; e += CODEC_THREADS) {
    const int o = o0 + e / cv, c = 8 * (e % cv);
    float v[8];
    convt_frame8<DT>(cols, ld_cols, row0, o, c, Tin, C, k, s, v);
    V8<DT> tv = zero_v8<DT>(), bv = zero_v8<DT>(), r;
    if (o < ov) tv = ldv<DT>(tl + (long)o * C + c);
    if (bias) bv = ldv<DT>(bias + c);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float y = v[i];
      if (o < ov) y += E<DT>::to_f(tv.v[i]);
      if (bias) y += E<DT>::to_f(bv.v[i]);
      r.v[i] = E<DT>::from_f(y);
    }
    stv<DT>(out + ((long)b * nout + o) * ld_out + c, r);
  }
  if (blockIdx.y) return;
  V8<DT> keep[CODEC_KEEP / 8];  // constant indices: registers, not a private or LDS array
#pragma unroll
  for (int p = 0; p < CODEC_KEEP / 8; ++p) {
    const int e = threadIdx.x + CODEC_THREADS * p;
    if (e < ov * cv) {
      float v[8];
      convt_frame8<DT>(cols, ld_cols, row0, nout + e / cv, 8 * (e % cv), Tin, C, k, s, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) keep[p].v[i] = E<DT>::from_f(v[i]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < CODEC_KEEP / 8; ++p) {
    const int e = threadIdx.x + CODEC_THREADS * p;
    if (e < ov * cv) stv<DT>(tl + 8 * e, keep[p]);
  }
}

// ---------------------------------------------------------------------------------------------------------
// Decoder transformer attention (:151-184) for T new tokens per seat at positions p = tokens[slot] + t: q and k
// get RoPE (rotate_half; angle p * inv_freq[i] in fp32, cos and sin times rope_scale), k (post-RoPE) and v go to
// the slot's ring entry p % ring with key_pos[slot, p % ring] = p; query p attends the entries with
// p - window < key_pos <= p, softmax at scale 1/sqrt(64). qkv rows [q heads | k heads | v heads] (as many kv heads
// as heads), head_dim 64.
// TM bounds T at compile time, which keeps the unrolled code small.
// One 4-wave workgroup per (seat, head). Thread j owns ring entry j for the scores (its key row read whole, the
// queries read from LDS as broadcasts); the softmax is block-wide; for P.V wave w sums entries 64 w .. 64 w + 63
// with lane (g, d8) taking keys g (mod 8) and dims 8 d8 .. + 7, all loads in flight at once and no branch around
// them (masked entries have probability 0); the 8 key groups meet by shuffles and the 4 waves in LDS. Each key
// and value row is read once for all T queries. The head-0 workgroup records key_pos; every workgroup knows the
// positions of the entries this call writes, so none depends on another's key_pos write.
constexpr int RA_HD = 64;
constexpr int RA_RING = 256;
constexpr int RA_T = 2;  // tokens per call: Mimi's upsample makes 2 per frame
static_assert(RA_T <= 4, "one wave of the 4-wave workgroup per token");
template <int DT, int TM>
__global__ __launch_bounds__(256) void ring_attn_kernel(const Elt<DT>* __restrict__ qkv, long ld_qkv,
                                                        Elt<DT>* kring, Elt<DT>* vring, int64_t* key_pos,
                                                        const int64_t* __restrict__ tokens,
                                                        const int64_t* __restrict__ slots,
                                                        const float* __restrict__ inv_freq, float rope_scale,
                                                        Elt<DT>* __restrict__ out, long ld_out, int T, int H, int ring,
                                                        int window) {
  __shared__ float qs[TM][RA_HD];
  __shared__ float pw[TM][RA_RING];
  __shared__ float red[2][TM][4];
  __shared__ float part[4][TM][RA_HD];
  __shared__ __align__(16) Elt<DT> knew[TM][RA_HD];  // this call's keys (post-RoPE) and values, stored to the
  __shared__ __align__(16) Elt<DT> vnew[TM][RA_HD];  // ring only at the end: reads of them come from here
  const int b = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  const long slot = slots[b];
  // wave w < T handles token w: its q, k, v elements do not depend on the position, so they load first
  const int half = RA_HD / 2;
  const int partner = l < half ? l + half : l - half;
  float q_l = 0.f, q_p = 0.f, k_l = 0.f, k_p = 0.f;
  Elt<DT> v_l = 0;
  if (wave < T) {
    const Elt<DT>* r = qkv + ((long)b * T + wave) * ld_qkv;
    q_l = E<DT>::to_f(r[h * RA_HD + l]);
    q_p = E<DT>::to_f(r[h * RA_HD + partner]);
    k_l = E<DT>::to_f(r[(H + h) * RA_HD + l]);
    k_p = E<DT>::to_f(r[(H + h) * RA_HD + partner]);
    v_l = r[(2 * H + h) * RA_HD + l];
  }
  const long p0 = tokens[slot];
  Elt<DT>* kr = kring + slot * (long)ring * H * RA_HD;  // [ring][H][hd]
  Elt<DT>* vr = vring + slot * (long)ring * H * RA_HD;
  int64_t* kp = key_pos + slot * (long)ring;
  const int lo = (int)(p0 % ring);  // ring entry of token 0; token t sits at (lo + t) % ring
  // the older entries' keys, positions and values load now, while RoPE runs; this call's own rows come from LDS
  // after the barrier. Thread j owns entry j for the scores; for P.V lane (g, d8) of wave w takes entries
  // 64 w + g + 8 i, dims 8 d8 .. + 7.
  const int j = tid;
  const int dd = (j - lo + ring) % ring;  // entries this call writes hold p0 + dd, dd < T
  long kj = NEVER_POS;
  V8<DT> k8[RA_HD / 8];
#pragma unroll
  for (int d = 0; d < RA_HD / 8; ++d) k8[d] = zero_v8<DT>();
  if (j < ring && dd >= T) {
    const Elt<DT>* krow = kr + ((long)j * H + h) * RA_HD;
#pragma unroll
    for (int d = 0; d < RA_HD / 8; ++d) k8[d] = ldv<DT>(krow + 8 * d);
    kj = kp[j];
  }
  const int g = l >> 3, dc = 8 * (l & 7);
  V8<DT> vv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int jj = 64 * wave + g + 8 * i;
    vv[i] = zero_v8<DT>();
    if (jj < ring && (jj - lo + ring) % ring >= T) vv[i] = ldv<DT>(vr + ((long)jj * H + h) * RA_HD + dc);
  }
  if (wave < T) {  // RoPE of token `wave`
    const float f = inv_freq[l < half ? l : l - half];
    const float sgn = l < half ? -1.f : 1.f;
    const float ang = (float)(p0 + wave) * f;
    const float cs = cosf(ang) * rope_scale, sn = sinf(ang) * rope_scale;
    qs[wave][l] = q_l * cs + sgn * q_p * sn;
    knew[wave][l] = E<DT>::from_f(k_l * cs + sgn * k_p * sn);
    vnew[wave][l] = v_l;
  }
  __syncthreads();  // queries and this call's rows are in LDS
  if (j < ring && dd < T) {
    kj = p0 + dd;
#pragma unroll
    for (int d = 0; d < RA_HD / 8; ++d) k8[d] = *reinterpret_cast<const V8<DT>*>(&knew[dd][8 * d]);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int jj = 64 * wave + g + 8 * i;
    const int dn = (jj - lo + ring) % ring;
    if (jj < ring && dn < T) vv[i] = *reinterpret_cast<const V8<DT>*>(&vnew[dn][dc]);
  }
  float sc[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    sc[t] = -INFINITY;
    if (t >= T) continue;
    float acc = 0.f;
#pragma unroll
    for (int d = 0; d < RA_HD / 8; ++d) {
      const float4 qa = *reinterpret_cast<const float4*>(&qs[t][8 * d]);
      const float4 qb = *reinterpret_cast<const float4*>(&qs[t][8 * d + 4]);
      acc += qa.x * E<DT>::to_f(k8[d].v[0]) + qa.y * E<DT>::to_f(k8[d].v[1]) + qa.z * E<DT>::to_f(k8[d].v[2]) +
             qa.w * E<DT>::to_f(k8[d].v[3]) + qb.x * E<DT>::to_f(k8[d].v[4]) + qb.y * E<DT>::to_f(k8[d].v[5]) +
             qb.z * E<DT>::to_f(k8[d].v[6]) + qb.w * E<DT>::to_f(k8[d].v[7]);
    }
    const long pos = p0 + t;
    if (kj <= pos && kj > pos - window) sc[t] = acc * 0.125f;  // NEVER_POS and j >= ring never qualify
  }
  // block-wide softmax per query
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    if (t >= T) break;
    const float m = wave_max_xor(sc[t], 64);
    if (l == 0) red[0][t][wave] = m;
  }
  __syncthreads();
  float mx[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    if (t >= T) break;
    mx[t] = fmaxf(fmaxf(red[0][t][0], red[0][t][1]), fmaxf(red[0][t][2], red[0][t][3]));  // finite: own key
    const float pe = sc[t] == -INFINITY ? 0.f : expf(sc[t] - mx[t]);
    if (j < ring) pw[t][j] = pe;
    const float sm = wave_sum_xor(pe, 64);
    if (l == 0) red[1][t][wave] = sm;
  }
  __syncthreads();
  // P.V over this wave's 64 entries (values loaded above)
  float o[TM][8];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[t][e] = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int jj = 64 * wave + g + 8 * i;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      if (t >= T) continue;
      const float pj = jj < ring ? pw[t][jj] : 0.f;  // 0 for masked entries, whose values are finite
#pragma unroll
      for (int e = 0; e < 8; ++e) o[t][e] += pj * E<DT>::to_f(vv[i].v[e]);
    }
  }
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    if (t >= T) break;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = o[t][e];
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      o[t][e] = v;
    }
    if (g == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[wave][t][dc + e] = o[t][e];
    }
  }
  __syncthreads();
  for (int i = tid; i < T * RA_HD; i += 256) {
    const int t = i / RA_HD, d = i % RA_HD;
    const float sum = red[1][t][0] + red[1][t][1] + red[1][t][2] + red[1][t][3];
    const float v = part[0][t][d] + part[1][t][d] + part[2][t][d] + part[3][t][d];
    out[((long)b * T + t) * ld_out + h * RA_HD + d] = E<DT>::from_f(v / sum);
    // this call's rows into the ring (no thread of this workgroup reads them from global memory)
    const long e = (lo + t) % ring;
    kr[(e * H + h) * RA_HD + d] = knew[t][d];
    vr[(e * H + h) * RA_HD + d] = vnew[t][d];
    if (h == 0 && d == 0) kp[e] = p0 + t;
  }
}

// Seats' token counters advance by T after the transformer (:183-184); the dummy slot's counter returns to 0. One
// thread per seat (the seats' slots other than the dummy are distinct, so no two threads touch one counter).
__global__ void advance_tokens_kernel(int64_t* tokens, const int64_t* __restrict__ slots, int B, int T, int dummy) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) {
    const int64_t s = slots[b];
    if (s != dummy) tokens[s] += T;
  }
  if (b == 0) tokens[dummy] = 0;
}

// ---------------------------------------------------------------------------------------------------------
// Last conv to PCM (decoder.layers[-1], C -> 1 channel, kernel k, causal) in fp32 with fp32 weights:
// pcm[b, t] = bias + sum_j sum_c w[j * C + c] joined[t + j][c], joined = the slot's k - 1 stored frames then x
// (ELU already applied by the producing row op); the state becomes joined's last k - 1 frames.
// Grid (B, ceil(T / chunk)), chunk >= k - 1; one thread per output sample (rows read as 16-byte vectors,
// weights from LDS); k * C <= 4096.
constexpr int FC_W = 4096;
template <int DT>
__global__ __launch_bounds__(CODEC_THREADS) void final_conv_kernel(const Elt<DT>* __restrict__ x, long ld_x,
                                                                   Elt<DT>* state, long ld_state,
                                                                   const int64_t* __restrict__ slots,
                                                                   const float* __restrict__ w, float bias,
                                                                   float* __restrict__ pcm, long ld_pcm, int T, int C,
                                                                   int k, int chunk) {
  __shared__ float ws[FC_W];
  const int b = blockIdx.x;
  const int t0 = blockIdx.y * chunk, t1 = min(T, t0 + chunk);
  const int pad = k - 1;
  const long row0 = (long)b * T;
  Elt<DT>* st = pad ? state + slots[b] * ld_state : nullptr;
  for (int i = threadIdx.x; i < k * C; i += CODEC_THREADS) ws[i] = w[i];
  __syncthreads();
  const int cv = C / 8;
  for (int t = t0 + threadIdx.x; t < t1; t += CODEC_THREADS) {
    float acc = 0.f;
    for (int j = 0; j < k; ++j) {
      const int i = t + j;
      const Elt<DT>* row = i < pad ? st + (long)i * C : x + (row0 + i - pad) * ld_x;
      const float* wj = ws + j * C;
      for (int c8 = 0; c8 < cv; ++c8) {
        const V8<DT> v = ldv<DT>(row + 8 * c8);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += wj[8 * c8 + e] * E<DT>::to_f(v.v[e]);
      }
    }
    pcm[(long)b * ld_pcm + t] = acc + bias;
  }
  if (!pad || blockIdx.y) return;
  V8<DT> keep[CODEC_KEEP / 8];  // constant indices: registers, not a private or LDS array
#pragma unroll
  for (int p = 0; p < CODEC_KEEP / 8; ++p) {
    const int e = threadIdx.x + CODEC_THREADS * p;
    if (e < pad * cv) keep[p] = joined8<DT>(st, x, ld_x, row0, pad, T + e / cv, 8 * (e % cv), C, 0);
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < CODEC_KEEP / 8; ++p) {
    const int e = threadIdx.x + CODEC_THREADS * p;
    if (e < pad * cv) stv<DT>(st + 8 * e, keep[p]);
  }
}

// final_conv_kernel for the codec's shape (C <= 64 channels, k <= 9 taps), FCS_CHUNK samples per workgroup: the
// chunk's input rows and the k - 1 before it (the slot's stored frames for the first chunk) are staged in LDS as
// fp32 with every 16-byte load issued before the first store (clamped indices, no branch around the loads); then
// one thread per sample sums taps j and channels c in the same order as final_conv_kernel, so the two give the same
// bits. One thread per sample reading its rows from memory made every load touch 64 cache lines (180 us for 224
// seats of one frame).
constexpr int FCS_CHUNK = 128, FCS_C = 64, FCS_K = 9, FCS_LD = FCS_C + 4;
template <int DT>
__global__ __launch_bounds__(CODEC_THREADS) void final_conv_staged_kernel(const Elt<DT>* __restrict__ x, long ld_x,
                                                                          Elt<DT>* state, long ld_state,
                                                                          const int64_t* __restrict__ slots,
                                                                          const float* __restrict__ w, float bias,
                                                                          float* __restrict__ pcm, long ld_pcm, int T,
                                                                          int C, int k) {
  __shared__ __align__(16) float ws[FCS_K * FCS_C];
  __shared__ __align__(16) float xs[(FCS_CHUNK + FCS_K - 1) * FCS_LD];
  const int b = blockIdx.x;
  const int t0 = blockIdx.y * FCS_CHUNK, t1 = min(T, t0 + FCS_CHUNK);
  const int pad = k - 1;
  const long row0 = (long)b * T;
  Elt<DT>* st = pad ? state + slots[b] * ld_state : nullptr;
  for (int i = threadIdx.x; i < k * C; i += CODEC_THREADS) ws[i] = w[i];
  const int cv = C / 8;
  const int nvec = (t1 - t0 + pad) * cv;  // staged row r is the joined row t0 + r
  constexpr int VPT = ((FCS_CHUNK + FCS_K - 1) * (FCS_C / 8) + CODEC_THREADS - 1) / CODEC_THREADS;
  V8<DT> v[VPT];
#pragma unroll
  for (int p = 0; p < VPT; ++p) {
    const int e = min((int)threadIdx.x + CODEC_THREADS * p, nvec - 1);
    const int r = e / cv, q = e - (e / cv) * cv;
    const int i = t0 + r;
    v[p] = ldv<DT>(i < pad ? st + (long)i * C + 8 * q : x + (row0 + i - pad) * ld_x + 8 * q);
  }
#pragma unroll
  for (int p = 0; p < VPT; ++p) {
    const int e = min((int)threadIdx.x + CODEC_THREADS * p, nvec - 1);  // repeats store the same values
    const int r = e / cv, q = e - (e / cv) * cv;
    float* d = xs + r * FCS_LD + 8 * q;
    *reinterpret_cast<float4*>(d) =
        make_float4(E<DT>::to_f(v[p].v[0]), E<DT>::to_f(v[p].v[1]), E<DT>::to_f(v[p].v[2]), E<DT>::to_f(v[p].v[3]));
    *reinterpret_cast<float4*>(d + 4) =
        make_float4(E<DT>::to_f(v[p].v[4]), E<DT>::to_f(v[p].v[5]), E<DT>::to_f(v[p].v[6]), E<DT>::to_f(v[p].v[7]));
  }
  __syncthreads();
  for (int t = t0 + threadIdx.x; t < t1; t += CODEC_THREADS) {
    float acc = 0.f;
    for (int j = 0; j < k; ++j) {
      const float* row = xs + (t - t0 + j) * FCS_LD;
      const float* wj = ws + j * C;
      for (int c = 0; c < C; c += 4) {
        const float4 xv = *reinterpret_cast<const float4*>(row + c);
        acc += wj[c] * xv.x;
        acc += wj[c + 1] * xv.y;
        acc += wj[c + 2] * xv.z;
        acc += wj[c + 3] * xv.w;
      }
    }
    pcm[(long)b * ld_pcm + t] = acc + bias;
  }
  if (!pad || blockIdx.y) return;
  // the new history: pad * C / 8 <= 64 vectors, at most one per thread (a register, not a private array)
  const int e = threadIdx.x;
  V8<DT> keep = zero_v8<DT>();
  if (e < pad * cv) keep = joined8<DT>(st, x, ld_x, row0, pad, T + e / cv, 8 * (e % cv), C, 0);
  __syncthreads();
  if (e < pad * cv) stv<DT>(st + 8 * e, keep);
}

// ---------------------------------------------------------------------------------------------------------
// C ABI
// The arguments name the element type ET, which each branch binds to its dtype's storage type.
#define CODEC_LAUNCH(KERNEL, GRID, BLOCK, ...)                                                   \
  do {                                                                                           \
    if (dtype == M3X_BF16) {                                                                     \
      using ET = uint16_t;                                                                        \
      hipLaunchKernelGGL(KERNEL<M3X_BF16>, GRID, BLOCK, 0, (hipStream_t)stream, __VA_ARGS__);    \
    } else if (dtype == M3X_F16) {                                                               \
      using ET = uint16_t;                                                                        \
      hipLaunchKernelGGL(KERNEL<M3X_F16>, GRID, BLOCK, 0, (hipStream_t)stream, __VA_ARGS__);     \
    } else if (dtype == M3X_F32) {                                                               \
      using ET = float;                                                                            \
      hipLaunchKernelGGL(KERNEL<M3X_F32>, GRID, BLOCK, 0, (hipStream_t)stream, __VA_ARGS__);     \
    } else {                                                                                     \
      return M3X_EUNSUPPORTED;                                                                   \
    }                                                                                            \
    M3X_CHECK_LAUNCH();                                                                          \
  } while (0)

M3X_API int m3x_rvq_decode(const int64_t* codes, long ld_codes, const void* tables, void* out, long ld_out, int B,
                           int nq, int n_codes, int dim, int dtype, void* stream) {
  if (B < 0 || nq < 1 || n_codes < 1 || dim < 1 || ld_codes < nq || ld_out < 2L * dim) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!codes || !tables || !out) return M3X_ENULL;
  CODEC_LAUNCH(rvq_decode_kernel, dim3(B), dim3(256), codes, ld_codes, (const ET*)tables, (ET*)out,
               ld_out, nq, n_codes, dim);
  return M3X_OK;
}

M3X_API int m3x_dwconvt(const void* x, long ld_x, const void* w, void* tail, long ld_tail, const int64_t* slots,
                        void* out, int B, int C, int k, int s, int dtype, void* stream) {
  if (B < 0 || C < 1 || s < 1 || k < s || k > 2 * s || ld_x < C || ld_tail < (long)(k - s) * C) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!x || !w || !tail || !slots || !out) return M3X_ENULL;
  CODEC_LAUNCH(dwconvt_kernel, dim3(B), dim3(256), (const ET*)x, ld_x, (const ET*)w, (ET*)tail,
               ld_tail, slots, (ET*)out, C, k, s);
  return M3X_OK;
}

M3X_API int m3x_conv_gather(const void* x, long ld_x, void* state, long ld_state, const int64_t* slots, void* cols,
                            long ld_cols, int B, int T, int C, int k, int dil, int use_elu, int chunk, int dtype,
                            void* stream) {
  const int pad = (k - 1) * dil;
  if (B < 0 || T < 1 || C < 8 || C % 8 || k < 1 || dil < 1 || ld_x < C || (cols && ld_cols < (long)k * C) ||
      chunk < max(pad, 1) || ((ld_x | (cols ? ld_cols : 0) | (pad ? ld_state : 0)) & 7))
    return M3X_EINVAL;
  if (!m3x_aligned16(x) || (cols && !m3x_aligned16(cols)) || (pad && !m3x_aligned16(state))) return M3X_EINVAL;
  if (pad && (ld_state < (long)pad * C || pad * C > CODEC_KEEP * CODEC_THREADS)) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!x || !slots || (pad && !state)) return M3X_ENULL;
  if (!cols && !pad) return M3X_OK;
  CODEC_LAUNCH(conv_gather_kernel, dim3(B, m3x_ceil_div(T, chunk)), dim3(CODEC_THREADS), (const ET*)x, ld_x,
               (ET*)state, ld_state, slots, (ET*)cols, ld_cols, T, C, k, dil, use_elu, chunk);
  return M3X_OK;
}

M3X_API int m3x_rows_op(const void* g, long ld_g, const void* bias, const void* scale, const void* res, long ld_res,
                        void* out, long ld_out, int rows, int C, int use_elu, int dtype, void* stream) {
  if (rows < 0 || C < 8 || C % 8 || ld_g < C || ld_out < C || (res && ld_res < C)) return M3X_EINVAL;
  if ((ld_g | ld_out | (res ? ld_res : 0)) & 7) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!g || !out) return M3X_ENULL;
  if (!m3x_aligned16(g) || !m3x_aligned16(out) || (bias && !m3x_aligned16(bias)) ||
      (scale && !m3x_aligned16(scale)) || (res && !m3x_aligned16(res)))
    return M3X_EINVAL;
  CODEC_LAUNCH(rows_op_kernel, dim3(m3x_ceil_div((long)rows * (C / 8), 256)), dim3(256), (const ET*)g, ld_g,
               (const ET*)bias, (const ET*)scale, (const ET*)res, ld_res, (ET*)out, ld_out,
               rows, C, use_elu);
  return M3X_OK;
}

M3X_API int m3x_convt_overlap(const void* cols, long ld_cols, void* tail, long ld_tail, const int64_t* slots,
                              const void* bias, void* out, long ld_out, int B, int Tin, int C, int k, int s, int chunk,
                              int dtype, void* stream) {
  if (B < 0 || Tin < 1 || C < 8 || C % 8 || s < 1 || k <= s || k > 2 * s || ld_cols < (long)k * C || ld_out < C ||
      chunk < k - s || ((ld_cols | ld_tail | ld_out) & 7))
    return M3X_EINVAL;
  if (!m3x_aligned16(cols) || !m3x_aligned16(tail) || !m3x_aligned16(out) || (bias && !m3x_aligned16(bias)))
    return M3X_EINVAL;
  if (ld_tail < (long)(k - s) * C || (k - s) * C > CODEC_KEEP * CODEC_THREADS) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!cols || !tail || !slots || !out) return M3X_ENULL;
  CODEC_LAUNCH(convt_overlap_kernel, dim3(B, m3x_ceil_div((long)Tin * s, chunk)), dim3(CODEC_THREADS),
               (const ET*)cols, ld_cols, (ET*)tail, ld_tail, slots, (const ET*)bias, (ET*)out,
               ld_out, Tin, C, k, s, chunk);
  return M3X_OK;
}

M3X_API int m3x_ring_attn(const void* qkv, long ld_qkv, void* kring, void* vring, int64_t* key_pos,
                          const int64_t* tokens, const int64_t* slots, const float* inv_freq, float rope_scale,
                          void* out, long ld_out, int B, int T, int H, int head_dim, int ring, int window, int dtype,
                          void* stream) {
  if (B < 0 || T < 1 || T > RA_T || H < 1 || H > 8 || head_dim != RA_HD || ring < 1 || ring > RA_RING ||
      window < 1 || ring < window + T - 1 || ring < T || ld_qkv < 3L * H * RA_HD || ld_out < (long)H * RA_HD || (ld_qkv & 7))
    return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!qkv || !kring || !vring || !key_pos || !tokens || !slots || !inv_freq || !out) return M3X_ENULL;
  if (!m3x_aligned16(qkv) || !m3x_aligned16(kring)) return M3X_EINVAL;
  if (!m3x_aligned16(out) || (ld_out & 7)) return M3X_EINVAL;
#define RA_LAUNCH(DTT, TMM)                                                                                    \
  hipLaunchKernelGGL((ring_attn_kernel<DTT, TMM>), dim3(B, H), dim3(256), 0, (hipStream_t)stream,                  \
                     (const Elt<DTT>*)qkv, ld_qkv, (Elt<DTT>*)kring, (Elt<DTT>*)vring, key_pos, tokens, slots,      \
                     inv_freq, rope_scale, (Elt<DTT>*)out, ld_out, T, H, ring, window)
  if (dtype == M3X_F16) RA_LAUNCH(M3X_F16, RA_T);
  else if (dtype == M3X_BF16) RA_LAUNCH(M3X_BF16, RA_T);
  else if (dtype == M3X_F32) RA_LAUNCH(M3X_F32, RA_T);
  else return M3X_EUNSUPPORTED;
#undef RA_LAUNCH
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

M3X_API int m3x_advance_tokens(int64_t* tokens, const int64_t* slots, int B, int T, int dummy, void* stream) {
  if (B < 0 || T < 0 || dummy < 0) return M3X_EINVAL;
  if (!tokens || (B && !slots)) return M3X_ENULL;
  hipLaunchKernelGGL(advance_tokens_kernel, dim3(m3x_ceil_div(std::max(B, 1), 256)), dim3(256), 0, (hipStream_t)stream,
                     tokens, slots, B, T, dummy);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

M3X_API int m3x_final_conv(const void* x, long ld_x, void* state, long ld_state, const int64_t* slots, const float* w,
                           float bias, float* pcm, long ld_pcm, int B, int T, int C, int k, int chunk, int dtype,
                           void* stream) {
  if (B < 0 || T < 1 || C < 8 || C % 8 || k < 1 || ld_x < C || ld_pcm < T || chunk < max(k - 1, 1) ||
      ((ld_x | (k > 1 ? ld_state : 0)) & 7))
    return M3X_EINVAL;
  if (!m3x_aligned16(x) || (k > 1 && !m3x_aligned16(state))) return M3X_EINVAL;
  if (k > 1 && (ld_state < (long)(k - 1) * C || (k - 1) * C > CODEC_KEEP * CODEC_THREADS)) return M3X_EINVAL;
  if ((long)k * C > FC_W) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!x || !slots || !w || !pcm || (k > 1 && !state)) return M3X_ENULL;
  if (C <= FCS_C && k <= FCS_K) {  // the codec's shape: rows staged in LDS (chunk is the general path's)
    CODEC_LAUNCH(final_conv_staged_kernel, dim3(B, m3x_ceil_div(T, FCS_CHUNK)), dim3(CODEC_THREADS), (const ET*)x,
                 ld_x, (ET*)state, ld_state, slots, w, bias, pcm, ld_pcm, T, C, k);
    return M3X_OK;
  }
  CODEC_LAUNCH(final_conv_kernel, dim3(B, m3x_ceil_div(T, chunk)), dim3(CODEC_THREADS), (const ET*)x, ld_x,
               (ET*)state, ld_state, slots, w, bias, pcm, ld_pcm, T, C, k, chunk);
  return M3X_OK;
}

M3X_API int m3x_resid_ln(void* h, long ld_h, const void* a, long ld_a, const void* scale, const void* w,
                         const void* b, void* y, long ld_y, float eps, int rows, int n, int dtype, void* stream) {
  if (rows < 0 || n != RLN_N || ld_h < n || ld_a < n || ld_y < n || ((ld_h | ld_a | ld_y) & 7)) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!h || !a || !scale || !w || !b || !y) return M3X_ENULL;
  if (!m3x_aligned16(h) || !m3x_aligned16(a) || !m3x_aligned16(scale) || !m3x_aligned16(w) || !m3x_aligned16(b) ||
      !m3x_aligned16(y))
    return M3X_EINVAL;
  CODEC_LAUNCH(resid_ln_kernel, dim3(m3x_ceil_div(rows, 4)), dim3(256), (ET*)h, ld_h, (const ET*)a, ld_a,
               (const ET*)scale, (const ET*)w, (const ET*)b, (ET*)y, ld_y, eps, rows);
  return M3X_OK;
}

M3X_API int m3x_conv_gemm(const void* x, long ldx, const void* w_packed, const void* bias, const void* res,
                          long ld_res, void* y, long ldy, int M, int N, int K, int use_elu, const void* state,
                          long ld_state, const int64_t* slots, int T, int C, int dil, int pre_elu, int dtype,
                          void* stream) {
  // gathered form when C > 0: K = k * C, x rows [M, C], the slot's history of pad = (k - 1) * dil frames
  ConvSrc cs{state, ld_state, slots, T, C, dil, 0, pre_elu};
  const int G = C > 0;
  if (G) {
    if (T < 1 || C % 8 || K % C || M % T || dil < 1 || ldx < C || (ldx & 7)) return M3X_EINVAL;
    cs.pad = (K / C - 1) * dil;
    if (cs.pad && (!state || !slots)) return M3X_ENULL;
    if (cs.pad && (ld_state < (long)cs.pad * C || (ld_state & 7) || !m3x_aligned16(state))) return M3X_EINVAL;
  }
  if (M < 0 || K < 32 || K % 32 || (N != 16 && N != 32 && N != 64 && N != 128) || (!G && ldx < K) || ldy < N || (res && ld_res < N) || ((ldx | ldy | (res ? ld_res : 0)) & 7))
    return M3X_EINVAL;
  if (M == 0) return M3X_OK;
  if (!x || !w_packed || !y) return M3X_ENULL;
  if (!m3x_aligned16(x) || !m3x_aligned16(w_packed) || !m3x_aligned16(y) || (res && !m3x_aligned16(res)) ||
      (bias && (((uintptr_t)bias) & 7)))
    return M3X_EINVAL;
  const int mt = M >= 64 * 1024 ? 2 : 1;  // two row tiles per wave once the grid fills the chip anyway
  // few rows (one seat): the columns split into up to N / 16 groups until 128 workgroups run
  const int gx = m3x_ceil_div(M, 4 * 16 * mt);
  int ny = 1;
  while (ny < N / 16 && (long)gx * ny < 128) ny *= 2;
  const int nt = N / 16 / ny;
  const dim3 grid(gx, ny);
  if (dtype == M3X_F32 && bias && !m3x_aligned16(bias)) return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
#define CG_CASE(DTT, NTT, MTT)                                                                                   \
  if (dtype == DTT && nt == NTT && mt == MTT) {                                                              \
    using ET = Elt<DTT>;                                                                                         \
    const ET *X = (const ET*)x, *W = (const ET*)w_packed, *Bi = (const ET*)bias, *R = (const ET*)res;                 \
    if (G)                                                                                                       \
      hipLaunchKernelGGL((conv_gemm_kernel<DTT, NTT, MTT, 1>), grid, dim3(256), 0, st, X, ldx, W, Bi, R, ld_res, \
                         (ET*)y, ldy, M, K, use_elu, cs);                                                         \
    else                                                                                                         \
      hipLaunchKernelGGL((conv_gemm_kernel<DTT, NTT, MTT, 0>), grid, dim3(256), 0, st, X, ldx, W, Bi, R, ld_res, \
                         (ET*)y, ldy, M, K, use_elu, cs);                                                         \
    M3X_CHECK_LAUNCH();                                                                                          \
    return M3X_OK;                                                                                               \
  }
  CG_CASE(M3X_F16, 1, 1) CG_CASE(M3X_F16, 2, 1) CG_CASE(M3X_F16, 4, 1) CG_CASE(M3X_F16, 8, 1)
  CG_CASE(M3X_F16, 1, 2) CG_CASE(M3X_F16, 2, 2) CG_CASE(M3X_F16, 4, 2) CG_CASE(M3X_F16, 8, 2)
  CG_CASE(M3X_BF16, 1, 1) CG_CASE(M3X_BF16, 2, 1) CG_CASE(M3X_BF16, 4, 1) CG_CASE(M3X_BF16, 8, 1)
  CG_CASE(M3X_BF16, 1, 2) CG_CASE(M3X_BF16, 2, 2) CG_CASE(M3X_BF16, 4, 2) CG_CASE(M3X_BF16, 8, 2)
  CG_CASE(M3X_F32, 1, 1) CG_CASE(M3X_F32, 2, 1) CG_CASE(M3X_F32, 4, 1) CG_CASE(M3X_F32, 8, 1)
  CG_CASE(M3X_F32, 1, 2) CG_CASE(M3X_F32, 2, 2) CG_CASE(M3X_F32, 4, 2) CG_CASE(M3X_F32, 8, 2)
#undef CG_CASE
  return M3X_EUNSUPPORTED;
}
