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
// the candidates contain the top k and all its ties; a bitonic sort of the candidates gives the exact order.
#include "m3x_norm.h"

namespace {
constexpr int ST = 256;      // threads per row
constexpr int SMAXV = 4096;  // largest vocabulary
constexpr int SEPT = SMAXV / ST;

__device__ __forceinline__ uint32_t ordkey(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ordkey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct SampleSmem {
  unsigned long long cand[SMAXV];
  float w[SMAXV];
  unsigned int hist[256];
  float red[ST / 64];
  int wtot[ST / 64];  // candidates per wave, for the compaction offsets
  int nkeep, bstar;
  int code;  // the drawn code, for the waves that build the next level's input
};

// every lane gets the wave's maximum (DPP within rows, permlane swaps across them; max is exact in any order)
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dppf<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dppf<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dppf<0x141>(v));  // row_half_mirror: the partner quad's maximum
  v = fmaxf(v, dppf<0x140>(v));  // row_mirror: the partner half-row's maximum
  return xor32_max(xor16_max(v));
}

// inclusive prefix sum of an integer over the 64 lanes (integer adds: any order gives the same sums). DPP row
// shifts build the sums within each row of 16, then row broadcasts carry the row totals forward.
__device__ __forceinline__ unsigned int wave_incl_scan(unsigned int x) {
  unsigned int v = x;
  v = v + (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, true);  // row_shr:1
  v = v + (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, true);  // row_shr:2
  v = v + (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x113, 0xf, 0xf, true);  // row_shr:3
  v = v + (unsigned int)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xe, false);  // row_shr:4, lanes 4..15
  v = v + (unsigned int)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xc, false);  // row_shr:8, lanes 8..15
  v = v + (unsigned int)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1, 3
  v = v + (unsigned int)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2, 3
  return v;
}

__device__ float block_max(float v, float* red) {
  v = wave_max_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < ST / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

// After this returns, sm.cand[0 .. sm.nkeep) holds the kept candidates in sampling order and sm.w their weights.
// x[] holds this thread's elements i = tid + 256*e (e < NE, NE * 256 >= V) of the transformed row.
template <int NE>
__device__ void topk_select(const float (&x)[NE], int V, int k, SampleSmem& sm) {
  const int tid = threadIdx.x;
  const float NEG = -INFINITY;
  sm.hist[tid] = 0;  // ordered before the histogram by block_max's barriers
  if (tid == 0) sm.nkeep = 0;
  float lm = NEG;
#pragma unroll
  for (int e = 0; e < NE; ++e)
    if (tid + ST * e < V) lm = fmaxf(lm, x[e]);
  const float m = block_max(lm, sm.red);
  int bk[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    bk[e] = 256;
    if (tid + ST * e < V) {
      const float d = (m - x[e]) * 32.0f;
      bk[e] = (d >= 255.0f || d != d) ? 255 : (int)d;
      if (bk[e] < 255) atomicAdd(&sm.hist[bk[e]], 1u);
    }
  }
  __syncthreads();
  if (tid < 64) {
    // lane owns bins 4*lane .. 4*lane+3 (bin 255 is excluded from the count)
    unsigned int c[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int bin = 4 * tid + i;
      c[i] = bin < 255 ? sm.hist[bin] : 0u;
      s += c[i];
    }
    const unsigned int incl = wave_incl_scan(s);
    unsigned int run = incl - s;
    int found = 255;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      run += c[i];
      if (found == 255 && run >= (unsigned)k && 4 * tid + i < 255) found = 4 * tid + i;
    }
    // first lane (lowest bin) that found it
    unsigned long long mask = __ballot(found < 255);
    if (tid == 0) sm.bstar = mask ? 0 : 255;
    if (mask) {
      const int first = __ffsll((long long)mask) - 1;
      const int b = __shfl(found, first, 64);
      if (tid == 0) sm.bstar = b;
    }
  }
  __syncthreads();
  const int bstar = sm.bstar;
  // compaction: each wave's count through LDS, a wave's base = the counts of the waves before it (candidates
  // land in wave order); lanes take consecutive places by ballot rank
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const unsigned long long below = (1ull << lane) - 1ull;
  unsigned long long masks[NE];
  int total = 0;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    masks[e] = __ballot(tid + ST * e < V && bk[e] <= bstar);
    total += __popcll(masks[e]);
  }
  if (lane == 0) sm.wtot[wave] = total;
  __syncthreads();
  int base = 0, ncand = 0;
#pragma unroll
  for (int w = 0; w < ST / 64; ++w) {
    const int c = sm.wtot[w];
    base += w < wave ? c : 0;
    ncand += c;
  }
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int i = tid + ST * e;
    if ((masks[e] >> lane) & 1ull)
      sm.cand[base + __popcll(masks[e] & below)] =
          ((unsigned long long)ordkey(x[e]) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)i);
    base += __popcll(masks[e]);
  }
  __syncthreads();
  const int nc = ncand;
  int P2 = 2;
  while (P2 < nc) P2 <<= 1;
  if (nc <= ST) {
    // The usual case (top-k of a peaked row): rank placement. Keys are distinct (the index is part of the key),
    // so candidate t goes to position #{j : key_j > key_t}; the reads of key_j are LDS broadcasts.
    const unsigned long long key = tid < nc ? sm.cand[tid] : 0ull;
    int rank = 0;
    if ((tid & ~63) < nc) {  // waves holding no candidate skip the count
      for (int j = 0; j < nc; j += 16) {  // sixteen broadcast reads in flight per step (clamped, masked)
        unsigned long long c16[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) c16[q] = sm.cand[min(j + q, nc - 1)];
#pragma unroll
        for (int q = 0; q < 16; ++q) rank += (j + q < nc && c16[q] > key) ? 1 : 0;
      }
    }
    __syncthreads();
    if (tid < nc) sm.cand[rank] = key;
    __syncthreads();
  } else {
  for (int i = nc + tid; i < P2; i += ST) sm.cand[i] = 0ull;
  __syncthreads();
  for (int kk = 2; kk <= P2; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int t = tid; t < (P2 >> 1); t += ST) {
        const int i = ((t & ~(j - 1)) << 1) | (t & (j - 1));
        const int p = i | j;
        const unsigned long long a = sm.cand[i], b = sm.cand[p];
        const bool desc = (i & kk) == 0;
        if (desc ? (a < b) : (a > b)) {
          sm.cand[i] = b;
          sm.cand[p] = a;
        }
      }
      __syncthreads();
    }
  }
  }
  const int kk = k < nc ? k : nc;
  const float kth = ordkey_inv((uint32_t)(sm.cand[kk - 1] >> 32));
  const float x0 = ordkey_inv((uint32_t)(sm.cand[0] >> 32));
  // the kept set (x >= kth) is a prefix of the sorted order: its last member records the length
  for (int j = tid; j < nc; j += ST) {
    const float xj = ordkey_inv((uint32_t)(sm.cand[j] >> 32));
    if (xj >= kth) {
      sm.w[j] = m3x_expf(xj - x0);
      if (j + 1 == nc || !(ordkey_inv((uint32_t)(sm.cand[j + 1] >> 32)) >= kth)) sm.nkeep = j + 1;
    }
  }
  __syncthreads();
}

__device__ __forceinline__ int cand_index(unsigned long long c) { return (int)(0xffffffffu - (uint32_t)c); }

__device__ __forceinline__ float lanef(float v, int q) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), q));
}

// Running sums of the weights of cand[0..n) in order, skipping index `skip` (-1: none), by one wave: the weights of
// 64 candidates sit one per lane (a skipped or absent one as +0.0) and are broadcast in order through readlane;
// lane j adds weight q through fmaf(w_q, f, c) with f = 1 for q <= j and 0 after, so it holds exactly the
// sequential fp32 sum w_0 + ... + w_j (fmaf(w, 1, c) rounds c + w once; fmaf(w, 0, c) = c), and lane 63 holds
// the chunk's total, carried into the next chunk. No lane-dependent select is needed, so the chain is 64
// independent-operand fmas. Running sums of chunks after the first are stored over their weights in sm.w.
// Returns the total (same value in every lane); *last = position of the last term, -1 if none; *first_use /
// *first_run = the first chunk's ballot of terms and this lane's running sum.
__device__ float wave_prefix(SampleSmem& sm, int n, int skip, int* last, unsigned long long* first_use,
                             float* first_run) {
  const int lane = threadIdx.x & 63;
  const float lf = (float)lane;
  float carry = 0.f;
  int l = -1;
  for (int j0 = 0; j0 < n; j0 += 64) {
    const int j = j0 + lane;
    const bool in = j < n && cand_index(sm.cand[j]) != skip;
    const float wsel = in ? sm.w[j] : 0.f;
    const unsigned long long use = __ballot(in);
    float c = carry;
#pragma unroll
    for (int q = 0; q < 64; ++q)
      c = fmaf(lanef(wsel, q), __builtin_amdgcn_fmed3f(lf - (float)q + 1.0f, 0.0f, 1.0f), c);
    carry = lanef(c, 63);
    if (use) l = j0 + 63 - __clzll((long long)use);
    if (j0 == 0) {
      *first_use = use;
      *first_run = c;
    } else if (j < n) {
      sm.w[j] = c;
    }
  }
  *last = l;
  return carry;
}

// Inverse-CDF pick over cand[0..n) skipping index `skip`: the first position whose running sum (the same
// sequential fp32 order as the total S) exceeds u * S, else the last term; -1 when the weights sum to 0.
// Called by one whole wave; every lane returns the same index. Overwrites sm.w past the first 64 candidates.
__device__ int pick(SampleSmem& sm, int n, float u, int skip) {
  const int lane = threadIdx.x & 63;
  int last;
  unsigned long long use0 = 0;
  float run0 = 0.f;
  const float S = wave_prefix(sm, n, skip, &last, &use0, &run0);
  if (last < 0 || !(S > 0.f)) return -1;
  const float t = u * S;
  unsigned long long hit = use0 & __ballot(run0 > t);
  if (hit) return cand_index(sm.cand[__ffsll((long long)hit) - 1]);
  for (int j0 = 64; j0 < n; j0 += 64) {
    const int j = j0 + lane;
    hit = __ballot(j < n && cand_index(sm.cand[j]) != skip && sm.w[j] > t);
    if (hit) return cand_index(sm.cand[j0 + __ffsll((long long)hit) - 1]);
  }
  return cand_index(sm.cand[last]);
}

// Top-p cut of the kept set cand[0..n) (maya3/engine.py:669-672: a candidate is dropped when the probability mass
// sorted before it exceeds top_p): position j stays while run_(j-1) / S <= top_p, where run is the sequential fp32
// running sum of the weights in order (the fmaf broadcast of wave_prefix) and S their total in the same order.
// The kept set stays a prefix of the order. Called by one whole wave; leaves sm.w unchanged; returns the new
// length (>= 1) in every lane.
__device__ int top_p_keep(const SampleSmem& sm, int n, float top_p) {
  const float lf = (float)(threadIdx.x & 63);
  auto chunk_runs = [&](int j0, float carry) {
    const int j = j0 + (int)(threadIdx.x & 63);
    const float wj = j < n ? sm.w[j] : 0.f;
    float c = carry;
#pragma unroll
    for (int q = 0; q < 64; ++q) c = fmaf(lanef(wj, q), __builtin_amdgcn_fmed3f(lf - (float)q + 1.0f, 0.0f, 1.0f), c);
    return c;
  };
  float S = 0.f;
  for (int j0 = 0; j0 < n; j0 += 64) S = lanef(chunk_runs(j0, S), 63);
  float carry = 0.f;
  for (int j0 = 0; j0 < n; j0 += 64) {
    const float c = chunk_runs(j0, carry);  // lane l: run_(j0 + l)
    carry = lanef(c, 63);
    const unsigned long long cut = __ballot(j0 + (int)(threadIdx.x & 63) + 1 < n && c / S > top_p);
    if (cut) return j0 + __ffsll((long long)cut);  // first j with run_j / S > top_p keeps 0..j
  }
  return n;
}
}  // namespace

// ---------------------------------------------------------------------------------------------------------
// Depth codebook sampler (serve/fast_depth_kernels.py:48-79 _topk_sample; unfused twin serve/fast_depth.py:125-132):
// x = float(logit) * inv_temp. Writes the code of row b to out[b * ld_out] (int32, or int64 if out_i64).
//
// With TPR > 0 the workgroup also builds the next level's input from the code it drew (serve/fast_depth.py:
// 137-138 and the first norm of the next level, :164): e = table[code] is written to prefix[b]; with y given,
// xo[b] = e and y[b] = norm(e) (norm_vec over 8*TPR elements, the add+norm kernel's arithmetic with no addend),
// which replaces a row copy and a norm launch per codebook.
struct EmbedArgs {
  const uint16_t* table;
  long ld_table, table_rows;
  uint16_t* prefix;
  long ld_prefix;
  uint16_t* xo;
  uint16_t* y;
  const uint16_t* w;
  const uint16_t* b;
  float eps;
  int kind;
};

template <int DT, int TPR, int NE>
__global__ __launch_bounds__(ST) void topk_sample_kernel(const uint16_t* __restrict__ logits, long ld_l, int V,
                                                         const float* __restrict__ u, long ld_u, float inv_temp,
                                                         int top_k, int greedy, void* out, long ld_out, int out_i64,
                                                         EmbedArgs ea) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.x;
  const float ur = greedy ? 0.f : u[(long)row * ld_u];  // loaded first: its latency overlaps the selection
  float x[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int i = threadIdx.x + ST * e;
    x[e] = i < V ? E<DT>::to_f(logits[(long)row * ld_l + i]) * inv_temp : -INFINITY;
  }
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
    u16x8 wv = {}, bv = {};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
    if (act) {
      const u16x8 ev = ld16(ea.table + cr * ea.ld_table + 8 * t);
      if (ea.y) {
        wv = ld16(ea.w + 8 * t);
        if (ea.kind == M3X_NORM_LAYER) bv = ld16(ea.b + 8 * t);
      }
      st16(ea.prefix + (long)row * ea.ld_prefix + 8 * t, ev);
      if (ea.xo) st16(ea.xo + (long)row * N + 8 * t, ev);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = E<DT>::to_f(ev.v[e]);
    }
    if (ea.y) {
      const u16x8 yv = norm_vec<TPR, DT>(v, wv, bv, ea.kind, ea.eps, red, bcast);
      if (act) st16(ea.y + (long)row * N + 8 * t, yv);
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
  hipLaunchKernelGGL((topk_sample_kernel<DTT, 0, NEE>), dim3(B), dim3(ST), 0, st, (const uint16_t*)logits, ld_l, V, \
                     u, ld_u, inv_temp, top_k, greedy, out, ld_out, out_i64, ea)
  if (dtype == M3X_BF16 && V <= 2048) M3X_TS(M3X_BF16, 8);
  else if (dtype == M3X_BF16) M3X_TS(M3X_BF16, 16);
  else if (dtype == M3X_F16 && V <= 2048) M3X_TS(M3X_F16, 8);
  else if (dtype == M3X_F16) M3X_TS(M3X_F16, 16);
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
  const EmbedArgs ea{(const uint16_t*)table, ld_table, table_rows, (uint16_t*)prefix, ld_prefix,
                     y ? (uint16_t*)x_out : nullptr, (uint16_t*)y, (const uint16_t*)w, (const uint16_t*)b, eps, kind};
#define M3X_TSE(DTT, TT)                                                                                      \
  do {                                                                                                     \
    if (V <= 2048)                                                                                         \
      hipLaunchKernelGGL((topk_sample_kernel<DTT, TT, 8>), dim3(B), dim3(ST), 0, st, (const uint16_t*)logits, \
                         ld_l, V, u, ld_u, inv_temp, top_k, greedy, out, ld_out, out_i64, ea);               \
    else                                                                                                   \
      hipLaunchKernelGGL((topk_sample_kernel<DTT, TT, 16>), dim3(B), dim3(ST), 0, st, (const uint16_t*)logits, \
                         ld_l, V, u, ld_u, inv_temp, top_k, greedy, out, ld_out, out_i64, ea);               \
  } while (0)
  if (dtype == M3X_BF16 && n == 1024) M3X_TSE(M3X_BF16, 128);
  else if (dtype == M3X_F16 && n == 1024) M3X_TSE(M3X_F16, 128);
  else if (dtype == M3X_BF16 && n == 2048) M3X_TSE(M3X_BF16, 256);
  else if (dtype == M3X_F16 && n == 2048) M3X_TSE(M3X_F16, 256);
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

__global__ __launch_bounds__(ST) void cb0_sample_kernel(Cb0Args a) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.x;
  const long s = a.slots[row];
  const float temp = a.temp_t ? a.temp_t[s] : a.temp;
  int k = a.topk_t ? (int)a.topk_t[s] : a.top_k;
  k = k < 1 ? 1 : (k > a.V ? a.V : k);
  const float bias = a.aeos_bias ? a.aeos_bias[s] : 0.f;
  const float rep = a.rep_t ? a.rep_t[s] : 0.f;
  const float top_p = a.topp_t ? a.topp_t[s] : a.top_p;
  const float uu = a.u[(long)row * a.ld_u];  // loaded first: its latency overlaps the selection
  float x[SEPT];
#pragma unroll
  for (int e = 0; e < SEPT; ++e) {
    const int i = threadIdx.x + ST * e;
    float v = -INFINITY;
    if (i < a.V) {
      v = bf2f(a.logits[(long)row * a.ld_l + i]) / temp;
      if (i == a.aeos) v = v + bias;
      if (a.hist_t && a.rep_t && i != a.aeos) {
        bool seen = false;
        for (int j = 0; j < a.hist_w; ++j) seen |= a.hist_t[s * a.hist_w + j] == (int64_t)i;
        if (seen) v = v - rep;
      }
    }
    x[e] = v;
  }
  topk_select(x, a.V, k, sm);
  if (threadIdx.x >= 64) return;  // wave 0 draws; lane 0 writes
  int n = sm.nkeep;
  if (top_p < 1.0f) n = top_p_keep(sm, n, top_p);
  int cb0;
  int64_t stop = 0;
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
    if (threadIdx.x != 0) return;
    const int arg = cand_index(sm.cand[0]);
    if (a.frames_t && a.min_t && a.hazard_t) {
      const bool can = a.frames_t[s] >= a.min_t[s];
      const float hz0 = a.hazard_t[s];
      const float hz = can ? 1.0f - (1.0f - hz0) * (1.0f - pa) : hz0;
      if (can && arg == a.aeos) stop = 2;
      else if (can && pa >= 0.35f) stop = 3;
      else if (can && hz >= 0.6f) stop = 4;
      a.hazard_t[s] = hz;
      a.frames_t[s] = a.frames_t[s] + 1;
    }
    cb0 = c < 0 ? 0 : c;
  } else {
    const int c = pick(sm, n, uu, -1);
    if (threadIdx.x != 0) return;
    cb0 = c < 0 ? cand_index(sm.cand[0]) : c;
  }
  if (a.ctr_t) a.ctr_t[s] = a.ctr_t[s] + 1;
  if (a.hist_t && a.hist_w > 0) {
    for (int j = 0; j + 1 < a.hist_w; ++j) a.hist_t[s * a.hist_w + j] = a.hist_t[s * a.hist_w + j + 1];
    a.hist_t[s * a.hist_w + a.hist_w - 1] = cb0;
  }
  if (a.cb0_out) a.cb0_out[row] = cb0;
  if (a.cb0_i32) a.cb0_i32[(long)row * a.ld_cb0_i32] = cb0;
  if (a.stop_out) a.stop_out[row] = stop;
}

M3X_API int m3x_cb0_sample(const void* logits, long ld_l, int V, int aeos, const int64_t* slots, const float* u,
                           long ld_u, const float* temp_t, float temp, const int64_t* topk_t, int top_k,
                           const float* topp_t, float top_p, const float* aeos_bias, const float* rep_t, int64_t* hist_t, int hist_w, int64_t* frames_t,
                           const int64_t* min_t, float* hazard_t, int32_t* ctr_t, int64_t* cb0_out, int32_t* cb0_i32,
                           long ld_cb0_i32, int64_t* stop_out, int B, void* stream) {
  if (B < 0 || V <= 0 || V > SMAXV || aeos >= V || hist_w < 0) return M3X_EINVAL;
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
