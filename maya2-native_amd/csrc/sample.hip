// Codebook samplers driven by caller-supplied uniforms, and the counter-based uniform generator.
//
// Sampling contract (one row of V logits, one uniform u in [0,1)):
//   x_i      = transform(logit_i)                      (depth: logit*inv_temp; cb0: logit/temp + bias - penalty)
//   kth      = the k-th largest x (counting repeats)   (torch topk(k).values[-1])
//   kept     = { i : x_i >= kth }                      (ties kept: serve/fast_depth_kernels.py:55-56,
//                                                       maya3/engine.py:666-668)
//   order    = kept sorted by x descending, index ascending (+0 before -0)
//   w_j      = m3x_expf(x_j - x_first)                 (Cody-Waite exp shared with the oracle)
//   S        = w_0 + w_1 + ... in order (sequential fp32), t = u * S
//   sample   = first j in order with (w_0 + ... + w_j) > t, else the last kept
//   greedy   = the first in order (argmax, lowest index on ties)
// This is inverse-CDF sampling of the top-k renormalised softmax, the distribution the reference draws with
// Gumbel/exponential races (serve/fast_depth_kernels.py:60-68, maya3/engine.py:687-688).
//
// Selection inside one 256-thread workgroup per row: the row max m, a 256-bin histogram of the bucket
// floor(32*(m - x)) (bin 255 = everything 8 or more below the max, not counted), the first bin b* at which the
// cumulative count reaches k, then every x with bucket <= b* is a candidate. The bucket is monotone in x, so
// the candidates contain the top k and all its ties. When fewer than k elements lie within 8 of the max (a peaked
// row), a radix select over the ordered keys finds the exact k-th largest instead, and the candidates are the
// elements >= it. Candidates are ordered by rank placement (at most 256) or a bitonic sort.
#include "m3x_sample.h"

// ---------------------------------------------------------------------------------------------------------
// Depth codebook sampler (serve/fast_depth_kernels.py:48-79 _topk_sample; unfused twin serve/fast_depth.py:125-132):
// x = float(logit) * inv_temp. Writes the code of row b to out[b * ld_out] (int32, or int64 if out_i64).
//
// With TPR > 0 the workgroup also builds the next level's input from the code it drew (serve/fast_depth.py:
// 137-138 and the first norm of the next level, :164): e = table[code] is written to prefix[b]; with y given,
// xo[b] = e and y[b] = norm(e) (norm_vec over 8*TPR elements, the add+norm kernel's arithmetic with no addend),
// which replaces a row copy and a norm launch per codebook.
// Rows of the kernel's storage type (Elt<DT>); kept untyped here so one struct serves every dtype.
struct EmbedArgs {
  const void* table;
  long ld_table, table_rows;
  void* prefix;
  long ld_prefix;
  void* xo;
  void* y;
  const void* w;
  const void* b;
  float eps;
  int kind;
};

template <int DT, int TPR, int NE>
__global__ __launch_bounds__(ST) void topk_sample_kernel(const Elt<DT>* __restrict__ logits, long ld_l, int V,
                                                         const float* __restrict__ u, long ld_u, float inv_temp,
                                                         int top_k, int greedy, void* out, long ld_out, int out_i64,
                                                         EmbedArgs ea) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.x;
  const float ur = greedy ? 0.f : u[(long)row * ld_u];  // loaded first: its latency overlaps the selection
  // every element's load issued before the first is used (indices past V re-read element V - 1 and are masked
  // after: a load under a condition would make the compiler wait for it there, one round trip per element)
  Elt<DT> raw[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) raw[e] = logits[(long)row * ld_l + min((int)threadIdx.x + ST * e, V - 1)];
  float x[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) x[e] = (int)threadIdx.x + ST * e < V ? E<DT>::to_f(raw[e]) * inv_temp : -INFINITY;
  topk_select(x, V, top_k, sm);
  if (TPR == 0 && threadIdx.x >= 64) return;  // wave 0 draws
  if (threadIdx.x < 64) {
    int code = cand_index(sm.cand[0]);
    if (!greedy) {
      const int c = pick(sm, sm.nkeep, ur, -1);
      if (c >= 0) code = c;
    }
    if (threadIdx.x == 0) {
      if (out_i64)
        ((int64_t*)out)[(long)row * ld_out] = code;
      else
        ((int32_t*)out)[(long)row * ld_out] = code;
      sm.code = code;
    }
  }
  if constexpr (TPR > 0) {
    constexpr int N = 8 * TPR;
    __shared__ float red[256];
    __shared__ float bcast[ST / TPR];
    __syncthreads();
    const int t = threadIdx.x % TPR;
    const bool act = threadIdx.x < TPR;
    long cr = sm.code;
    cr = cr < 0 ? 0 : (cr >= ea.table_rows ? ea.table_rows - 1 : cr);
    float v[8];
    using T = Elt<DT>;
    V8<DT> wv = zero_v8<DT>(), bv = zero_v8<DT>();
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
    if (act) {
      const V8<DT> ev = ldv<DT>((const T*)ea.table + cr * ea.ld_table + 8 * t);
      if (ea.y) {
        wv = ldv<DT>((const T*)ea.w + 8 * t);
        if (ea.kind == M3X_NORM_LAYER) bv = ldv<DT>((const T*)ea.b + 8 * t);
      }
      stv<DT>((T*)ea.prefix + (long)row * ea.ld_prefix + 8 * t, ev);
      if (ea.xo) stv<DT>((T*)ea.xo + (long)row * N + 8 * t, ev);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = E<DT>::to_f(ev.v[e]);
    }
    if (ea.y) {
      const V8<DT> yv = norm_vec<TPR, DT>(v, wv, bv, ea.kind, ea.eps, red, bcast);
      if (act) stv<DT>((T*)ea.y + (long)row * N + 8 * t, yv);
    }
  }
}

M3X_API int m3x_topk_sample(const void* logits, long ld_l, int V, const float* u, long ld_u, float inv_temp,
                            int top_k, int greedy, void* out, long ld_out, int out_i64, int B, int dtype,
                            void* stream) {
  if (B < 0 || V <= 0 || V > SMAXV || top_k <= 0) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!logits || !out || (!greedy && !u)) return M3X_ENULL;
  hipStream_t st = (hipStream_t)stream;
  const EmbedArgs ea{};
#define M3X_TS(DTT, NEE)                                                                                             \
  hipLaunchKernelGGL((topk_sample_kernel<DTT, 0, NEE>), dim3(B), dim3(ST), 0, st, (const Elt<DTT>*)logits, ld_l, V, \
                     u, ld_u, inv_temp, top_k, greedy, out, ld_out, out_i64, ea)
  if (dtype == M3X_BF16 && V <= 2048) M3X_TS(M3X_BF16, 8);
  else if (dtype == M3X_BF16) M3X_TS(M3X_BF16, 16);
  else if (dtype == M3X_F16 && V <= 2048) M3X_TS(M3X_F16, 8);
  else if (dtype == M3X_F16) M3X_TS(M3X_F16, 16);
  else if (dtype == M3X_F32 && V <= 2048) M3X_TS(M3X_F32, 8);
  else if (dtype == M3X_F32) M3X_TS(M3X_F32, 16);
  else return M3X_EUNSUPPORTED;
#undef M3X_TS
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// m3x_topk_sample, then per row b: prefix[b * ld_prefix + j] = table[code_b * ld_table + j] for j < n, and, when
// y is given, x_out[b * n + j] = the same row and y[b * n + j] = its LayerNorm (kind 0, w and bias) or RMSNorm
// (kind 1, w). Codes are clamped to [0, table_rows). n is 1024 or 2048.
M3X_API int m3x_topk_sample_embed(const void* logits, long ld_l, int V, const float* u, long ld_u, float inv_temp,
                                  int top_k, int greedy, void* out, long ld_out, int out_i64, int B,
                                  const void* table, long ld_table, long table_rows, void* prefix, long ld_prefix,
                                  void* x_out, void* y, const void* w, const void* b, float eps, int kind, int n,
                                  int dtype, void* stream) {
  if (B < 0 || V <= 0 || V > SMAXV || top_k <= 0 || table_rows <= 0) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!logits || !out || (!greedy && !u) || !table || !prefix) return M3X_ENULL;
  if (y && (!w || (kind == M3X_NORM_LAYER && !b))) return M3X_ENULL;
  if (y && kind != M3X_NORM_LAYER && kind != M3X_NORM_RMS) return M3X_EINVAL;
  if (((ld_table | ld_prefix) & 7) || ld_table < n) return M3X_EINVAL;
  if (!m3x_aligned16(table) || !m3x_aligned16(prefix) || (x_out && !m3x_aligned16(x_out)) ||
      (y && !m3x_aligned16(y)) || (w && !m3x_aligned16(w)) || (b && !m3x_aligned16(b)))
    return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const EmbedArgs ea{table, ld_table, table_rows, prefix, ld_prefix, y ? x_out : nullptr, y, w, b, eps, kind};
#define M3X_TSE(DTT, TT)                                                                                      \
  do {                                                                                                     \
    if (V <= 2048)                                                                                         \
      hipLaunchKernelGGL((topk_sample_kernel<DTT, TT, 8>), dim3(B), dim3(ST), 0, st, (const Elt<DTT>*)logits,  \
                         ld_l, V, u, ld_u, inv_temp, top_k, greedy, out, ld_out, out_i64, ea);               \
    else                                                                                                   \
      hipLaunchKernelGGL((topk_sample_kernel<DTT, TT, 16>), dim3(B), dim3(ST), 0, st, (const Elt<DTT>*)logits, \
                         ld_l, V, u, ld_u, inv_temp, top_k, greedy, out, ld_out, out_i64, ea);               \
  } while (0)
  if (dtype == M3X_BF16 && n == 1024) M3X_TSE(M3X_BF16, 128);
  else if (dtype == M3X_F16 && n == 1024) M3X_TSE(M3X_F16, 128);
  else if (dtype == M3X_BF16 && n == 2048) M3X_TSE(M3X_BF16, 256);
  else if (dtype == M3X_F16 && n == 2048) M3X_TSE(M3X_F16, 256);
  else if (dtype == M3X_F32 && n == 1024) M3X_TSE(M3X_F32, 128);
  else if (dtype == M3X_F32 && n == 2048) M3X_TSE(M3X_F32, 256);
  else return M3X_EUNSUPPORTED;
#undef M3X_TSE
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// cb0 step: controlled stop + codebook-0 sampling for each seat (maya3/engine.py:652-694, Engine._cb0).
// Per row b with slot s = slots[b] (per-slot tensors are indexed by s, like the engine's [max_seats+1] state):
//   x_i = float(logit_i) / temp[s];  x_aeos += aeos_bias[s];  x_i -= rep[s] for every i != aeos seen in
//   hist[s, :] (entries >= 0);  top-k (k = topk[s], clamped to [1, V]) as in the contract above; then, with
//   top_p = topp[s] < 1, the kept set is cut to its top-p prefix (top_p_keep).
//   With an AEOS class (aeos >= 0): probs = w / S over the kept set; pa = w_aeos / S; arg = first in order;
//   can = frames[s] >= min_frames[s]; hz = can ? 1 - (1 - hazard[s]) * (1 - pa) : hazard[s];
//   stop = can & arg==aeos ? 2 : can & pa>=0.35 ? 3 : can & hz>=0.6 ? 4 : 0;
//   cb0 = inverse-CDF pick over the kept set without aeos (0 if nothing else is kept).
//   State: ctr[s] += 1, hist[s] shifts left and appends cb0, hazard[s] = hz, frames[s] += 1.
// Per-slot pointers may be null: temp/topk fall back to the scalars, no bias/penalty, no stop logic/state.
struct Cb0Args {
  const uint16_t* logits;
  long ld_l;
  int V;
  int aeos;
  const int64_t* slots;
  const float* u;
  long ld_u;
  const float* temp_t;
  float temp;
  const int64_t* topk_t;
  int top_k;
  const float* topp_t;
  float top_p;
  const float* aeos_bias;
  const float* rep_t;
  int64_t* hist_t;
  int hist_w;
  int64_t* frames_t;
  const int64_t* min_t;
  float* hazard_t;
  int32_t* ctr_t;
  int64_t* cb0_out;    // [B] int64 or null
  int32_t* cb0_i32;    // [B * ld_cb0_i32] or null (column 0 of the frame's code matrix)
  long ld_cb0_i32;
  int64_t* stop_out;   // [B] int64 or null
};

constexpr int CB0_HMAX = 256;  // the longest repetition-penalty history a row stages in LDS
// A per-slot value, or dflt when the table is absent: the load is unconditional (an absent table reads `dummy`,
// any valid 8-byte word), so it does not wait at a branch of its own.
template <class T>
__device__ __forceinline__ T slot_or(const T* p, long i, const void* dummy, T dflt) {
  const T v = *reinterpret_cast<const T*>(p ? (const void*)(p + i) : dummy);
  return p ? v : dflt;
}

__global__ __launch_bounds__(ST) void cb0_sample_kernel(Cb0Args a) {
  __shared__ SampleSmem sm;
  __shared__ int64_t hist[CB0_HMAX];
  const int row = blockIdx.x;
  // the logits first, every element's load issued before any is used (indices past V re-read element V - 1 and are
  // masked below: a load under a condition would make the compiler wait for it there, one round trip per element)
  uint16_t raw[SMAXV / ST];
#pragma unroll
  for (int e = 0; e < SMAXV / ST; ++e) raw[e] = a.logits[(long)row * a.ld_l + min((int)threadIdx.x + ST * e, a.V - 1)];
  const long s = a.slots[row];
  // the slot's settings and state in one round trip
  const void* dm = a.slots + row;
  const float temp = slot_or(a.temp_t, s, dm, a.temp);
  int k = (int)slot_or<int64_t>(a.topk_t, s, dm, a.top_k);
  k = k < 1 ? 1 : (k > a.V ? a.V : k);
  const float bias = slot_or(a.aeos_bias, s, dm, 0.f);
  const float rep = slot_or(a.rep_t, s, dm, 0.f);
  const float top_p = slot_or(a.topp_t, s, dm, a.top_p);
  const bool stop_rule = a.frames_t && a.min_t && a.hazard_t;
  const int64_t frames = slot_or<int64_t>(a.frames_t, s, dm, 0), min_frames = slot_or<int64_t>(a.min_t, s, dm, 0);
  const float hz0 = slot_or(a.hazard_t, s, dm, 0.f);
  const int32_t ctr = slot_or<int32_t>(a.ctr_t, s, dm, 0);
  const float uu = a.u[(long)row * a.ld_u];  // loaded first: its latency overlaps the selection
  // the slot's recent codes, staged once in LDS: the repetition penalty reads them, and wave 0 writes them back
  // shifted by one with the drawn code last
  const int hw = a.hist_t ? a.hist_w : 0;  // <= CB0_HMAX (checked on the host)
  const bool pen = hw > 0 && a.rep_t;
  for (int j = threadIdx.x; j < hw; j += ST) hist[j] = a.hist_t[s * a.hist_w + j];
  __syncthreads();
  float x[SMAXV / ST];
#pragma unroll
  for (int e = 0; e < SMAXV / ST; ++e) {
    const int i = threadIdx.x + ST * e;
    float v = -INFINITY;
    if (i < a.V) {
      v = bf2f(raw[e]) / temp;
      if (i == a.aeos) v = v + bias;
      if (pen && i != a.aeos) {
        bool seen = false;
        for (int j = 0; j < hw; ++j) seen |= hist[j] == (int64_t)i;
        if (seen) v = v - rep;
      }
    }
    x[e] = v;
  }
  topk_select(x, a.V, k, sm);
  if (threadIdx.x >= 64) return;  // wave 0 draws (every lane holds the code); lane 0 writes the rest
  int n = sm.nkeep;
  if (top_p < 1.0f) n = top_p_keep(sm, n, top_p);
  int cb0;
  int64_t stop = 0;
  float hz = hz0;
  if (a.aeos >= 0) {
    float wa = 0.f;  // weight of the AEOS candidate (indices are distinct: at most one)
    for (int j0 = 0; j0 < n; j0 += 64) {
      const int j = j0 + (int)(threadIdx.x & 63);
      const unsigned long long m = __ballot(j < n && cand_index(sm.cand[j]) == a.aeos);
      if (m) wa = sm.w[j0 + __ffsll((long long)m) - 1];
    }
    float S = 0.f;  // every kept weight in order (sequential fp32), read before pick reuses sm.w
    for (int j0 = 0; j0 < n; j0 += 64) {
      const int j = j0 + (int)(threadIdx.x & 63);
      const float wj = j < n ? sm.w[j] : 0.f;
#pragma unroll
      for (int q = 0; q < 64; ++q) S = S + lanef(wj, q);
    }
    const float pa = wa / S;
    const int c = pick(sm, n, uu, a.aeos);
    const int arg = cand_index(sm.cand[0]);
    if (stop_rule) {
      const bool can = frames >= min_frames;
      hz = can ? 1.0f - (1.0f - hz0) * (1.0f - pa) : hz0;
      if (can && arg == a.aeos) stop = 2;
      else if (can && pa >= 0.35f) stop = 3;
      else if (can && hz >= 0.6f) stop = 4;
    }
    cb0 = c < 0 ? 0 : c;
  } else {
    const int c = pick(sm, n, uu, -1);
    cb0 = c < 0 ? cand_index(sm.cand[0]) : c;
  }
  for (int j = threadIdx.x; j < hw; j += 64) a.hist_t[s * a.hist_w + j] = j + 1 < hw ? hist[j + 1] : (int64_t)cb0;
  if (threadIdx.x != 0) return;
  if (a.aeos >= 0 && stop_rule) {
    a.hazard_t[s] = hz;
    a.frames_t[s] = frames + 1;
  }
  if (a.ctr_t) a.ctr_t[s] = ctr + 1;
  if (a.cb0_out) a.cb0_out[row] = cb0;
  if (a.cb0_i32) a.cb0_i32[(long)row * a.ld_cb0_i32] = cb0;
  if (a.stop_out) a.stop_out[row] = stop;
}

M3X_API int m3x_cb0_sample(const void* logits, long ld_l, int V, int aeos, const int64_t* slots, const float* u,
                           long ld_u, const float* temp_t, float temp, const int64_t* topk_t, int top_k,
                           const float* topp_t, float top_p, const float* aeos_bias, const float* rep_t, int64_t* hist_t, int hist_w, int64_t* frames_t,
                           const int64_t* min_t, float* hazard_t, int32_t* ctr_t, int64_t* cb0_out, int32_t* cb0_i32,
                           long ld_cb0_i32, int64_t* stop_out, int B, void* stream) {
  if (B < 0 || V <= 0 || V > SMAXV || aeos >= V || hist_w < 0 || hist_w > CB0_HMAX) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!logits || !slots || !u) return M3X_ENULL;
  if (!temp_t && !(temp > 0.f)) return M3X_EINVAL;
  Cb0Args a{(const uint16_t*)logits, ld_l, V, aeos, slots, u, ld_u, temp_t, temp, topk_t, top_k, topp_t, top_p,
            aeos_bias, rep_t,
            hist_t, hist_w, frames_t, min_t, hazard_t, ctr_t, cb0_out, cb0_i32, ld_cb0_i32, stop_out};
  hipLaunchKernelGGL(cb0_sample_kernel, dim3(B), dim3(ST), 0, (hipStream_t)stream, a);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Counter-based uniforms: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC11), counter = (ctr[s], level, 0, 0), key = (seed[s], 0); u = (word0 >> 8) * 2^-24 in [0, 1).
// One draw per (seat, level): the per-request streams the engine keys by (seed, frame counter, level)
// (maya3/engine.py:436-437, serve/fast_depth_kernels.py:63,90).
__device__ __forceinline__ uint32_t philox_word0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                                 uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

__global__ void philox_uniforms_kernel(const int32_t* __restrict__ seeds, const int32_t* __restrict__ ctrs,
                                       const int64_t* __restrict__ slots, float* __restrict__ out, long ld_out,
                                       int level0, int nlevels, int B) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * nlevels) return;
  const int b = (int)(i / nlevels), j = (int)(i % nlevels);
  const long s = slots[b];
  const uint32_t w = philox_word0((uint32_t)ctrs[s], (uint32_t)(level0 + j), 0u, 0u, (uint32_t)seeds[s], 0u);
  out[(long)b * ld_out + j] = (float)(w >> 8) * 5.9604644775390625e-8f;
}

M3X_API int m3x_philox_uniforms(const int32_t* seeds, const int32_t* ctrs, const int64_t* slots, float* out,
                                long ld_out, int level0, int nlevels, int B, void* stream) {
  if (B < 0 || nlevels <= 0 || level0 < 0) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!seeds || !ctrs || !slots || !out) return M3X_ENULL;
  const long total = (long)B * nlevels;
  hipLaunchKernelGGL(philox_uniforms_kernel, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, seeds,
                     ctrs, slots, out, ld_out, level0, nlevels, B);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// Per-row Exp(1) noise: out[b, c] = -log(max(u, 1e-12)), u from counter (ctrs[b], level, c, 0), key (seeds[b], 0).
// Surface of row_exponential (serve/fast_depth_kernels.py:82-98) for callers that still take argmax(q/E).
__global__ void philox_exponential_kernel(const int32_t* __restrict__ seeds, const int32_t* __restrict__ ctrs,
                                          float* __restrict__ out, long ld_out, int level, int V, int B) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * V) return;
  const int b = (int)(i / V), c = (int)(i % V);
  const uint32_t w = philox_word0((uint32_t)ctrs[b], (uint32_t)level, (uint32_t)c, 0u, (uint32_t)seeds[b], 0u);
  const float u = (float)(w >> 8) * 5.9604644775390625e-8f;
  out[(long)b * ld_out + c] = -logf(fmaxf(u, 1e-12f));
}

M3X_API int m3x_philox_exponential(const int32_t* seeds, const int32_t* ctrs, float* out, long ld_out, int level,
                                   int V, int B, void* stream) {
  if (B < 0 || V <= 0 || level < 0) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!seeds || !ctrs || !out) return M3X_ENULL;
  const long total = (long)B * V;
  hipLaunchKernelGGL(philox_exponential_kernel, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream,
                     seeds, ctrs, out, ld_out, level, V, B);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// raw Philox4x32-10 block (known-answer tests), out[0..3] for counter c[0..3] and key k[0..1]
__global__ void philox_block_kernel(const uint32_t* c, const uint32_t* k, uint32_t* out) {
  uint32_t c0 = c[0], c1 = c[1], c2 = c[2], c3 = c[3], k0 = k[0], k1 = k[1];
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

M3X_API int m3x_philox_block(const uint32_t* counter, const uint32_t* key, uint32_t* out, void* stream) {
  if (!counter || !key || !out) return M3X_ENULL;
  hipLaunchKernelGGL(philox_block_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, counter, key, out);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}
