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
  int nkeep;
  int ncand;  // candidates placed so far
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

// The first of 256 bins (lane l holds the counts c[0..3] of its 4 bins, in the order they are scanned) at which the
// running count reaches kk, with the count before that bin; every lane of the wave gets the result. (-1, 0) when
// the total stays below kk (or kk is 0).
__device__ __forceinline__ void wave_find_bin(const unsigned int (&c)[4], unsigned int kk, int& idx, unsigned int& before) {
  const int lane = threadIdx.x & 63;
  const unsigned int s = c[0] + c[1] + c[2] + c[3];
  const unsigned int incl = wave_incl_scan(s);
  unsigned int run = incl - s;
  int found = -1;
  unsigned int bef = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (found < 0 && kk > 0 && run + c[i] >= kk) {
      found = 4 * lane + i;
      bef = run;
    }
    run += c[i];
  }
  const unsigned long long mk = __ballot(found >= 0);
  const int fl = mk ? __ffsll((long long)mk) - 1 : 0;
  idx = mk ? __builtin_amdgcn_readlane(found, fl) : -1;
  before = mk ? (unsigned int)__builtin_amdgcn_readlane((int)bef, fl) : 0u;
}

// The k-th largest of the valid elements (i < V, not NaN) of a row, counting repeats, by an MSB-first radix select
// over their ordered keys, 8 bits a pass: each pass histograms the next byte of the keys that share the bytes fixed
// so far, and every wave finds the bin where the count from the top reaches the remaining rank. With fewer than k
// valid elements it returns the smallest; with none, NaN. Called by every thread with a block-uniform k, before
// the candidates are placed: the three histograms (used in turn, each cleared two passes ahead, so one barrier a
// pass) live in sm.cand after the coarse histogram of topk_select.
template <int NE, class SM>
__device__ float radix_kth(const float (&x)[NE], int V, int k, SM& sm) {
  static_assert(sizeof(sm.cand) >= 4 * 256 * sizeof(unsigned int), "histograms in sm.cand");
  unsigned int* hb = reinterpret_cast<unsigned int*>(sm.cand) + 256;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  uint32_t key[NE];
  bool ok[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    ok[e] = tid + ST * e < V && x[e] == x[e];
    key[e] = ordkey(x[e]);
  }
  hb[tid] = 0;
  hb[256 + tid] = 0;
  __syncthreads();
  uint32_t pre = 0;
  unsigned int kr = (unsigned int)k;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int sh = 24 - 8 * pass;
    const uint32_t hm = pass == 0 ? 0u : ~0u << (sh + 8);
    unsigned int* h = hb + 256 * (pass % 3);
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const bool in = ok[e] && (key[e] & hm) == pre;
      const uint32_t d = (key[e] >> sh) & 255u;
      // the keys of a row mostly share their top bytes: the lanes holding the wave's first live digit add their
      // count with one atomic, the others one each
      const unsigned long long live = __ballot(in);
      if (live) {
        const int first = __ffsll((long long)live) - 1;
        const uint32_t d0 = (uint32_t)__builtin_amdgcn_readlane((int)d, first);
        const unsigned long long same = __ballot(in && d == d0);
        if (lane == first) atomicAdd(&h[d0], (unsigned int)__popcll(same));
        if (in && d != d0) atomicAdd(&h[d], 1u);
      }
    }
    __syncthreads();
    if (pass < 2) hb[256 * ((pass + 2) % 3) + tid] = 0;  // last read two passes back, next written after a barrier
    // lane l scans bins 255 - 4 l .. 252 - 4 l: descending key order
    unsigned int c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = h[255 - 4 * lane - i];
    int idx;
    unsigned int before;
    if (pass == 0) {
      const unsigned int total = (unsigned int)__builtin_amdgcn_readlane(
          (int)wave_incl_scan(c[0] + c[1] + c[2] + c[3]), 63);
      if (total < kr) kr = total;  // fewer valid elements than k: the smallest of them
    }
    wave_find_bin(c, kr, idx, before);
    if (idx < 0) {  // no valid element (block-uniform)
      __syncthreads();
      return __uint_as_float(0x7fc00000u);
    }
    pre |= (uint32_t)(255 - idx) << sh;
    kr -= before;
  }
  __syncthreads();  // every wave's last scan precedes the candidate stores into sm.cand
  return ordkey_inv(pre);
}

// After this returns, sm.cand[0 .. sm.nkeep) holds the kept candidates in sampling order and sm.w their weights.
// x[] holds this thread's elements i = tid + 256*e (e < NE, NE * 256 >= V) of the transformed row.
template <int NE, class SM>
__device__ void topk_select(const float (&x)[NE], int V, int k, SM& sm) {
  const int tid = threadIdx.x;
  const float NEG = -INFINITY;
  sm.hist[tid] = 0;  // ordered before the histograms by the max's barrier
  unsigned int* h2 = reinterpret_cast<unsigned int*>(sm.cand);  // the coarse histogram (candidates come later)
  h2[tid] = 0;
  if (tid == 0) {
    sm.nkeep = 0;
    sm.ncand = 0;
  }
  float lm = NEG;
#pragma unroll
  for (int e = 0; e < NE; ++e)
    if (tid + ST * e < V) lm = fmaxf(lm, x[e]);
  // row max: wave maxima meet in LDS behind one barrier (sm.red is next written by a later call, after further
  // barriers)
  lm = wave_max_dpp(lm);
  if ((tid & 63) == 0) sm.red[tid >> 6] = lm;
  __syncthreads();
  float m = sm.red[0];
#pragma unroll
  for (int i = 1; i < ST / 64; ++i) m = fmaxf(m, sm.red[i]);
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
  // every wave finds b* itself from the histogram (no barrier): lane l holds bins 4 l .. 4 l + 3; bin 255 (8 or
  // more below the max) is not counted
  int bstar;
  unsigned int near = 0;  // elements within 8 of the max, when fewer than k
  {
    const int lane = tid & 63;
    unsigned int c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = 4 * lane + i < 255 ? sm.hist[4 * lane + i] : 0u;
    int idx;
    unsigned int before;
    wave_find_bin(c, (unsigned int)k, idx, before);
    bstar = idx < 0 ? 255 : idx;
    if (idx < 0) near = (unsigned int)__builtin_amdgcn_readlane((int)wave_incl_scan(c[0] + c[1] + c[2] + c[3]), 63);
  }
  // Fewer than k elements within 8 of the max (a peaked row, the usual case for a confident model): a coarse
  // histogram of the rest, 0.5 wide bins from 255/32 below the max (bin 255: 135 or more below, not counted), finds
  // the bin b2 where the count reaches k; the candidates are then the near elements and those in coarse bins <= b2.
  int b2 = 0;
  int cb[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) cb[e] = 255;
  if (bstar == 255) {
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      if (tid + ST * e < V && bk[e] == 255) {
        const float d2 = ((m - x[e]) * 32.0f - 255.0f) * 0.0625f;
        cb[e] = (d2 >= 255.0f || d2 != d2) ? 255 : (int)d2;
        if (cb[e] < 255) atomicAdd(&h2[cb[e]], 1u);
      }
    }
    __syncthreads();
    const int lane = tid & 63;
    unsigned int c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = 4 * lane + i < 255 ? h2[4 * lane + i] : 0u;
    unsigned int before;
    wave_find_bin(c, (unsigned int)k - near, b2, before);
    __syncthreads();  // every wave's scan of the coarse histogram precedes the candidate stores over it
  }

  // Fewer than k elements within 135 of the max (or -inf / NaN among the top k): the candidates are the elements
  // >= the exact k-th largest (all elements when no valid one exists), found by radix select, rather than the
  // whole row, so the rank placement below still applies.
  const bool radix = bstar == 255 && b2 < 0;
  const float kth_sel = radix ? radix_kth<NE>(x, V, k, sm) : 0.f;
  const bool all = kth_sel != kth_sel;
  // compaction: one LDS atomic per wave reserves the wave's places (their order does not matter: the candidates
  // are ranked by key below); lanes take consecutive places by ballot rank
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const unsigned long long below = (1ull << lane) - 1ull;
  unsigned long long masks[NE];
  int total = 0;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const bool near_e = bstar < 255 ? bk[e] <= bstar : (bk[e] < 255 || cb[e] <= b2);
    masks[e] = __ballot(tid + ST * e < V && (radix ? (all || x[e] >= kth_sel) : near_e));
    total += __popcll(masks[e]);
  }
  int base = 0;
  if (lane == 0 && total > 0) base = (int)atomicAdd((unsigned int*)&sm.ncand, (unsigned int)total);
  base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int i = tid + ST * e;
    if ((masks[e] >> lane) & 1ull)
      sm.cand[base + __popcll(masks[e] & below)] =
          ((unsigned long long)ordkey(x[e]) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)i);
    base += __popcll(masks[e]);
  }
  __syncthreads();
  const int nc = sm.ncand;
  int P2 = 2;
  while (P2 < nc) P2 <<= 1;
  if (nc <= 64) {
    // The usual case: rank placement with the count split over the waves. Keys are distinct (the index is part
    // of the key), so candidate l goes to position #{j : key_j > key_l}; wave w counts the keys j in
    // [16 w, 16 w + 16) (LDS broadcast reads), the four partial counts meet in sm.hist (free by now).
    const unsigned long long key = lane < nc ? sm.cand[lane] : 0ull;
    const int j0 = 16 * wave;
    int part = 0;
    if (j0 < nc) {
      unsigned long long c16[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) c16[q] = sm.cand[min(j0 + q, nc - 1)];
#pragma unroll
      for (int q = 0; q < 16; ++q) part += (j0 + q < nc && c16[q] > key) ? 1 : 0;
    }
    sm.hist[tid] = (unsigned int)part;
    __syncthreads();
    if (tid < nc) sm.cand[sm.hist[lane] + sm.hist[64 + lane] + sm.hist[128 + lane] + sm.hist[192 + lane]] = key;
    __syncthreads();
  } else if (nc <= ST) {
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
