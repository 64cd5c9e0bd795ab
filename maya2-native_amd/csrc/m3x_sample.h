// Top-k selection and inverse-CDF draw inside one 256-thread workgroup per row, shared by the samplers of
// sample.hip and the depth frame kernel (depth.hip). The sampling contract is stated at the top of sample.hip.
#pragma once
#include "m3x_norm.h"

namespace {
constexpr int ST = 256;      // threads per row
constexpr int SMAXV = 4096;  // largest vocabulary

__device__ __forceinline__ uint32_t ordkey(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ordkey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// CAP: the most candidates a row can have (its vocabulary size)
template <int CAP>
struct SampleSmemT {
  unsigned long long cand[CAP];
  float w[CAP];
  unsigned int hist[256];
  float red[ST / 64];
  int wtot[ST / 64];  // candidates per wave, for the compaction offsets
  int nkeep, bstar;
  int code;  // the drawn code, for the waves that build the next level's input
};
using SampleSmem = SampleSmemT<SMAXV>;

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
template <int NE, class SM>
__device__ void topk_select(const float (&x)[NE], int V, int k, SM& sm) {
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
template <class SM>
__device__ float wave_prefix(SM& sm, int n, int skip, int* last, unsigned long long* first_use, float* first_run) {
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
template <class SM>
__device__ int pick(SM& sm, int n, float u, int skip) {
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
template <class SM>
__device__ int top_p_keep(const SM& sm, int n, float top_p) {
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
