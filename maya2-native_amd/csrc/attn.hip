// Attention kernels.
//
// decode_attn: GQA decode attention over the static KV cache, in place (serve/fast_backbone.py:31-58, launcher
// :242-247). Cache layout [slots, kv_heads, cap, D] bf16 (serve/fast_backbone.py:146-148). Row r attends keys
// 0..pos[r] of slot slots[r]; scale = D^-1/2; online softmax in fp32; output bf16.
//
// Mapping: one workgroup = (split c, row r, kv head kh) and handles the G query heads that share kh, so each K/V
// byte of a (row, kv head) is read once. The keys of a row are cut into splits of `chunk` keys (a multiple of
// 128); each of the 4 waves takes every 4th 32-key tile of its split. Per tile:
//   QK: S^T[key][head] = K[key][:] . Q^T  -> 2 x 4 MFMA 16x16x32 (K is the A operand: the tile's rows are loaded
//       16 lanes per 256-byte row, like V, into a wave-private LDS tile and read back in the A layout).
//   PV: O[head][dim] += P[head][key] . V[key][dim] -> 8 MFMAs. The P operand is exactly the S^T accumulator a
//       lane already holds (keys 4g..4g+3 of both 16-key halves); the V operand needs 8 keys of one dim per lane,
//       so a lane loads 8 full 16-byte key-row pieces and transposes 8x8 bf16 in registers (V stays out of LDS).
//       Output tile T holds dims {8c+T : c = 0..15}.
// The 4 waves merge through LDS; a split that is not the whole row writes (m, l, acc) partials and
// decode_attn_combine folds them in split order (deterministic).
#include "m3x_common.h"

#include <algorithm>
#include <queue>
#include <vector>
#include <mutex>

// K rows through a wave-private LDS tile (coalesced loads; bit-identical results): 1-2 % faster at 224 rows and
// 7 % at one row than loading the MFMA A layout straight from memory (KL = 0).
#ifndef M3X_ATTN_KL
#define M3X_ATTN_KL 1
#endif

namespace {
constexpr int AD = 128;       // head dim of the decode kernel
constexpr int PART_STRIDE = 264;  // floats per (row, kv head, split) partial: m[2] l[2] pad[4] o[2][128]
}

// K and V are read with the non-temporal hint: each cache byte is read once per step.
#ifndef M3X_ATTN_NT
#define M3X_ATTN_NT 1
#endif
__device__ __forceinline__ u16x8 kv_load(const uint16_t* p) {
  if constexpr (M3X_ATTN_NT) return ld16_nt(p);
  else return ld16(p);
}

// Three workgroups per CU (<= 168 VGPRs, no spill): measured 2 % faster than the unconstrained 190 VGPRs.
#ifndef M3X_ATTN_MINB
#define M3X_ATTN_MINB 3
#endif
template <int G, int KL>
__global__ __launch_bounds__(256, M3X_ATTN_MINB) void decode_attn_kernel(
    const uint16_t* __restrict__ q, long sq_b, long sq_h, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, long sk_s, long sk_h, long sk_t, uint16_t* __restrict__ out, long so_b,
    long so_h, const int64_t* __restrict__ slots, const int32_t* __restrict__ pos, float scale_log2, int chunk,
    float* __restrict__ part, int max_splits, int cap) {
  // rows vary fastest: consecutive workgroups (dispatched round-robin over the 8 XCDs) are live work, and the
  // splits past a row's context, which exit at once, gather in the last grid slices
  const int row = blockIdx.x;
  const int kh = blockIdx.y;
  const int split = blockIdx.z;
  const int KV = gridDim.y;
  const int ps = min(pos[row], cap - 1);  // the host guarantees pos < cap; the clamp keeps every access in the slot
  const int kstart = split * chunk;
  if (kstart > ps) return;  // this split is past the row's context (uniform per block)
  const int kend = min(kstart + chunk, ps + 1);
  const int nsplit = min((ps + chunk) / chunk, max_splits);  // ceil((ps + 1) / chunk)

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar branches
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;  // MFMA row/col index
  const int lg = lane >> 4;  // MFMA k group

  const long slot = slots[row];
  const uint16_t* kbase = kc + slot * sk_s + (long)kh * sk_h;
  const uint16_t* vbase = vc + slot * sk_s + (long)kh * sk_h;

  // Q^T operand: lane holds q[head li][32kk + 8lg .. +8] for li < G, zero otherwise.
  u16x8 qop[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    if (li < G) {
      qop[kk] = ld16(q + (long)row * sq_b + (long)(kh * G + li) * sq_h + 32 * kk + 8 * lg);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qop[kk].v[e] = 0;
    }
  }

  float m_run = -INFINITY, l_run = 0.f;  // per head li (meaningful for li < G), equal across lanes of one li
  f32x4_t acc[8];
#pragma unroll
  for (int T = 0; T < 8; ++T) acc[T] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // KL = 1: K rows are loaded like V (16 lanes per 256-byte row, 4 rows per instruction: one cache-line access
  // per 64 bytes) into a wave-private LDS tile and read back in the MFMA A layout; KL = 0 loads the A layout
  // straight from memory (each lane's 16 bytes a separate access).
  constexpr int KT_LD = 136;  // LDS row stride in halfwords (272 bytes: the 16 rows of a fragment read hit 16 bank groups)
  __shared__ __align__(16) uint16_t ktile[KL ? 4 : 1][KL ? 32 * KT_LD : 8];
  for (int k0 = kstart + 32 * wave; k0 < kend; k0 += 128) {
    // ---- loads: K rows k0 + 16*g2 + li (A operand), V rows key(lg, e) = k0 + 16*(e/4) + 4*lg + e%4
    u16x8 kop[2][4];
    u16x8 kld[KL ? 8 : 1];
    if constexpr (KL) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        kld[e] = kv_load(kbase + (long)(k0 + 16 * (e >> 2) + 4 * lg + (e & 3)) * sk_t + 8 * li);
    } else {
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        const uint16_t* kr = kbase + (long)(k0 + 16 * g2 + li) * sk_t + 8 * lg;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) kop[g2][kk] = kv_load(kr + 32 * kk);
      }
    }
    u16x8 vld[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vld[e] = kv_load(vbase + (long)(k0 + 16 * (e >> 2) + 4 * lg + (e & 3)) * sk_t + 8 * li);
    if constexpr (KL) {
      uint16_t* kt = ktile[wave];
#pragma unroll
      for (int e = 0; e < 8; ++e) st16(kt + (16 * (e >> 2) + 4 * lg + (e & 3)) * KT_LD + 8 * li, kld[e]);
      // wave-private tile: the LDS writes above complete before these reads (same wave, in-order LDS queue)
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          kop[g2][kk] = *reinterpret_cast<const u16x8*>(kt + (16 * g2 + li) * KT_LD + 32 * kk + 8 * lg);
    }

    // ---- scores S^T[key][head]: lane holds keys k0 + 16*g2 + 4*lg + r for head li
    f32x4_t s[2];
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      s[g2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) s[g2] = mfma16x16x32<M3X_BF16>(kop[g2][kk], qop[kk], s[g2]);
    }
    const bool tail = k0 + 32 > kend;
    float sv[8];
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 16 * g2 + 4 * lg + r;
        const float x = s[g2][r] * scale_log2;
        sv[4 * g2 + r] = (tail && key >= kend) ? -INFINITY : x;
      }
    float tmax = sv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) tmax = fmaxf(tmax, sv[e]);
    tmax = xor32_max(xor16_max(tmax));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp2f(m_run - m_new);
    float p[8], psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = (li < G) ? exp2f(sv[e] - m_new) : 0.f;
      psum += p[e];
    }
    psum = xor32_sum(xor16_sum(psum));
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // ---- rescale the accumulator rows (heads 0..G-1 live in lanes 0..15, register = head)
    float al[G];
#pragma unroll
    for (int h = 0; h < G; ++h) al[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), h));
#pragma unroll
    for (int T = 0; T < 8; ++T)
#pragma unroll
      for (int h = 0; h < G; ++h) acc[T][h] *= al[h];

    // ---- P operand (bf16): element e = 4*g2 + r is key k0 + 16*g2 + 4*lg + r
    u16x8 pop;
#pragma unroll
    for (int e = 0; e < 8; ++e) pop.v[e] = f2bf(p[e]);

    // ---- V operand: zero keys past the context in the tail tile (stale cache rows may hold anything)
    if (tail) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = k0 + 16 * (e >> 2) + 4 * lg + (e & 3);
        if (key >= kend) {
#pragma unroll
          for (int x = 0; x < 8; ++x) vld[e].v[x] = 0;
        }
      }
    }
#pragma unroll
    for (int T = 0; T < 8; ++T) {
      u16x8 vop;
#pragma unroll
      for (int e = 0; e < 8; ++e) vop.v[e] = vld[e].v[T];
      acc[T] = mfma16x16x32<M3X_BF16>(pop, vop, acc[T]);
    }
  }

  // ---- merge the 4 waves: lds_o[wave][h][dim], lds_ml[wave][h] = (m, l)
  __shared__ float lds_o[4][G][AD];
  __shared__ float lds_m[4][G], lds_l[4][G];
  if (lane < 16) {
#pragma unroll
    for (int T = 0; T < 8; ++T)
#pragma unroll
      for (int h = 0; h < G; ++h) lds_o[wave][h][8 * lane + T] = acc[T][h];
  }
  if (lane < G) {
    lds_m[wave][lane] = m_run;
    lds_l[wave][lane] = l_run;
  }
  __syncthreads();
  if (threadIdx.x >= G * AD) return;
  const int h = threadIdx.x / AD;
  const int d = threadIdx.x % AD;
  float M = lds_m[0][h];
#pragma unroll
  for (int w = 1; w < 4; ++w) M = fmaxf(M, lds_m[w][h]);
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float f = exp2f(lds_m[w][h] - M);  // 0 for a wave that saw no tile (m = -inf)
    L += lds_l[w][h] * f;
    O += lds_o[w][h][d] * f;
  }
  if (nsplit == 1) {
    out[(long)row * so_b + (long)(kh * G + h) * so_h + d] = f2bf(O / L);
  } else {
    float* pp = part + (((long)row * KV + kh) * max_splits + split) * PART_STRIDE;
    if (d == 0) {
      pp[h] = M;
      pp[2 + h] = L;
    }
    pp[8 + h * AD + d] = O;
  }
}

// One item of attn_block_kernel: rows row .. row + nb - 1, kv head kh, keys [kstart, kend) of split `split`. The
// rows are NB blocks of QB = 16 / G rows (NB = 2: a second block's 16 query vectors share every K/V tile the waves
// load, so a prefill makes one pass over its keys per 2 QB rows); each query vector sees the same tiles on the same
// wave and the same merge whatever NB, so its bits do not depend on the block it sits in.
template <int G, int NB>
__device__ __forceinline__ void attn_block_item(
    const uint16_t* __restrict__ q, long sq_b, long sq_h, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, long sk_s, long sk_h, long sk_t, uint16_t* __restrict__ out, long so_b,
    long so_h, const int64_t* __restrict__ slots, const int32_t* __restrict__ pos, float scale_log2, int chunk,
    float* __restrict__ part, int max_splits, int cap, int row, int nb, int kh, int KV, int split, int kstart,
    int kend, unsigned char* lds) {
  constexpr int QB = 16 / G;
  constexpr int KT_LD = 136;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;  // query vector (column) of S^T: block row li / G, head li % G
  const int lg = lane >> 4;
  const int jq = li / G;
  bool qlive[NB];
  int pq[NB];  // the vector's own position: it sees keys <= pq
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    qlive[b] = b * QB + jq < nb;
    pq[b] = qlive[b] ? min(pos[row + b * QB + jq], cap - 1) : -1;
  }

  const long slot = slots[row];
  const uint16_t* kbase = kc + slot * sk_s + (long)kh * sk_h;
  const uint16_t* vbase = vc + slot * sk_s + (long)kh * sk_h;
  u16x8 qop[NB][4];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (qlive[b]) {
        qop[b][kk] =
            ld16(q + (long)(row + b * QB + jq) * sq_b + (long)(kh * G + li % G) * sq_h + 32 * kk + 8 * lg);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qop[b][kk].v[e] = 0;
      }
    }
  float m_run[NB], l_run[NB];  // of vector li, equal across the 4 lanes of one li
  f32x4_t acc[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    m_run[b] = -INFINITY;
    l_run[b] = 0.f;
#pragma unroll
    for (int T = 0; T < 8; ++T) acc[b][T] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  uint16_t* kt = reinterpret_cast<uint16_t*>(lds) + wave * 32 * KT_LD;
  for (int k0 = kstart + 32 * wave; k0 < kend; k0 += 128) {
    u16x8 kld[8], vld[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      kld[e] = kv_load(kbase + (long)(k0 + 16 * (e >> 2) + 4 * lg + (e & 3)) * sk_t + 8 * li);
#pragma unroll
    for (int e = 0; e < 8; ++e) vld[e] = kv_load(vbase + (long)(k0 + 16 * (e >> 2) + 4 * lg + (e & 3)) * sk_t + 8 * li);
#pragma unroll
    for (int e = 0; e < 8; ++e) st16(kt + (16 * (e >> 2) + 4 * lg + (e & 3)) * KT_LD + 8 * li, kld[e]);
    f32x4_t sb[NB][2];
    if constexpr (NB == 1) {  // the whole tile's K operand read at once
      u16x8 kop[2][4];
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          kop[g2][kk] = *reinterpret_cast<const u16x8*>(kt + (16 * g2 + li) * KT_LD + 32 * kk + 8 * lg);
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        sb[0][g2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) sb[0][g2] = mfma16x16x32<M3X_BF16>(kop[g2][kk], qop[0][kk], sb[0][g2]);
      }
    } else {
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {  // one 16-key half of the tile at a time, shared by the blocks
        u16x8 kop[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          kop[kk] = *reinterpret_cast<const u16x8*>(kt + (16 * g2 + li) * KT_LD + 32 * kk + 8 * lg);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          sb[b][g2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) sb[b][g2] = mfma16x16x32<M3X_BF16>(kop[kk], qop[b][kk], sb[b][g2]);
        }
      }
    }
    u16x8 pop[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const f32x4_t* s = sb[b];
      // mask: keys past the split or the block, and keys after the vector's own position (causal); dead vectors
      // see nothing
      const int klim = min(kend - 1, pq[b]);
      float sv[8];
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 16 * g2 + 4 * lg + r;
          sv[4 * g2 + r] = (qlive[b] && key <= klim) ? s[g2][r] * scale_log2 : -INFINITY;
        }
      float tmax = sv[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) tmax = fmaxf(tmax, sv[e]);
      tmax = xor32_max(xor16_max(tmax));
      const float m_new = fmaxf(m_run[b], tmax);
      // a vector with no visible key yet keeps m = -inf: its weights are 0 and its rescale 1
      const float alpha = m_new == -INFINITY ? 1.f : exp2f(m_run[b] - m_new);
      float p[8], psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = sv[e] == -INFINITY ? 0.f : exp2f(sv[e] - m_new);
        psum += p[e];
      }
      psum = xor32_sum(xor16_sum(psum));
      l_run[b] = l_run[b] * alpha + psum;
      m_run[b] = m_new;
      // O rows are vectors 4 * lg + r: their rescale comes from lane 4 * lg + r
      float al[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, 4 * lg + r, 64);
#pragma unroll
      for (int T = 0; T < 8; ++T)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[b][T][r] *= al[r];
#pragma unroll
      for (int e = 0; e < 8; ++e) pop[b].v[e] = f2bf(p[e]);
    }
    if (k0 + 32 > kend) {  // zero V rows past the block's context in the tail tile
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = k0 + 16 * (e >> 2) + 4 * lg + (e & 3);
        if (key >= kend) {
#pragma unroll
          for (int x = 0; x < 8; ++x) vld[e].v[x] = 0;
        }
      }
    }
#pragma unroll
    for (int T = 0; T < 8; ++T) {
      u16x8 vop;
#pragma unroll
      for (int e = 0; e < 8; ++e) vop.v[e] = vld[e].v[T];
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[b][T] = mfma16x16x32<M3X_BF16>(pop[b], vop, acc[b][T]);
    }
  }

  // ---- merge the 4 waves (the K tiles are dead after the barrier)
  __syncthreads();
  float* lo = reinterpret_cast<float*>(lds);  // [4][16 NB][AD]
  float* lm = lo + 4 * 16 * NB * AD;          // [4][16 NB]
  float* ll = lm + 4 * 16 * NB;               // [4][16 NB]
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int T = 0; T < 8; ++T)
#pragma unroll
      for (int r = 0; r < 4; ++r) lo[((wave * NB + b) * 16 + 4 * lg + r) * AD + 8 * li + T] = acc[b][T][r];
    if (lg == 0) {
      lm[(wave * NB + b) * 16 + li] = m_run[b];
      ll[(wave * NB + b) * 16 + li] = l_run[b];
    }
  }
  __syncthreads();
  // thread t: vector t / 16 of each block, dims 8 * (t % 16) .. + 7
  const int c = threadIdx.x >> 4;
  const int d0 = 8 * (threadIdx.x & 15);
  const int h = c % G;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int j = b * QB + c / G;
    if (j >= nb) continue;
    const int pj = min(pos[row + j], cap - 1);
    const int nsplit = min((pj + chunk) / chunk, max_splits);
    if (split >= nsplit) continue;  // this row has no keys in this split (the caller's barrier follows)
    float M = lm[b * 16 + c];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, lm[(w * NB + b) * 16 + c]);
    float f[4], L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      f[w] = exp2f(lm[(w * NB + b) * 16 + c] - M);  // 0 for a wave that saw no visible key (m = -inf)
      L += ll[(w * NB + b) * 16 + c] * f[w];
    }
    float O[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      O[e] = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) O[e] += lo[((w * NB + b) * 16 + c) * AD + d0 + e] * f[w];
    }
    if (nsplit == 1) {
      u16x8 ov;
#pragma unroll
      for (int e = 0; e < 8; ++e) ov.v[e] = f2bf(O[e] / L);
      st16(out + (long)(row + j) * so_b + (long)(kh * G + h) * so_h + d0, ov);
    } else {
      float* pp = part + (((long)(row + j) * KV + kh) * max_splits + split) * PART_STRIDE;
      if (d0 == 0) {
        pp[h] = M;
        pp[2 + h] = L;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) pp[8 + h * AD + d0 + e] = O[e];
    }
  }
}

// Steps that hold inline prefill rows (serve/fast_backbone.py:326-359). The rows of one prefill are one slot at
// consecutive positions, and the caller groups them into items of up to IB = min(16, 2 QB) rows, QB = 16 / G (a
// decode row is an item of one row). One workgroup takes an item: each block of QB rows gives 16 query vectors
// (row j, head h), column j * G + h, that fill all 16 columns of the MFMA query operand, and an item's one or two
// blocks share each K/V tile, so a prefill costs one pass over its slot's keys per IB rows. Same tile
// pipeline as decode_attn_kernel (K through the wave-private LDS tile, V in registers, S^T = K . Q^T,
// O += P . V) and the same arithmetic per query vector, so every row gets the bits decode_attn_kernel would give
// it; the differences are the causal mask (vector j sees keys <= pos[row + j]) and the per-vector rescale (O rows
// are vectors 4 * lg + r, whose running max lives in lane 4 * lg + r). Rows whose context spans several splits
// write partials for decode_attn_combine_kernel.
// The grid is one workgroup per bin per kv head, 2 workgroups per CU whatever the item count (a workgroup
// launched only to exit costs a CU slot for microseconds). An item is one split of its rows' keys, so a long
// context is cut into several items that the bins balance. The caller deals the items into the bins (longest
// processing time first balances them) and lists them bin by bin:
//   items = [bins, start[0], ..., start[bins], code[0], code[1], ...], bin b = codes start[b] .. start[b + 1] - 1,
// each code = 2048 * (first row) + 32 * split + (rows of the item).
template <int G>
__global__ __launch_bounds__(256, 2) void attn_block_kernel(
    const uint16_t* __restrict__ q, long sq_b, long sq_h, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, long sk_s, long sk_h, long sk_t, uint16_t* __restrict__ out, long so_b,
    long so_h, const int64_t* __restrict__ slots, const int32_t* __restrict__ pos, float scale_log2, int chunk,
    float* __restrict__ part, int max_splits, int cap, const int32_t* __restrict__ items, int rows) {
  constexpr int QB = 16 / G;
  constexpr int NB = 2 * QB <= 16 ? 2 : 1;  // blocks per item
  const int kh = blockIdx.y;
  const int KV = gridDim.y;
  const int bins = items[0];
  if ((int)blockIdx.x >= bins || bins > rows) return;  // an item list sized for another grid does nothing
  const int i0 = max(items[1 + blockIdx.x], 0), i1 = min(items[2 + blockIdx.x], rows * max_splits);
  const int32_t* codes = items + 2 + bins;
  // LDS: the wave-private K tiles during the key loop, then the wave merge (after a barrier)
  constexpr int KTILE_BYTES = 4 * 32 * 136 * 2;
  constexpr int MERGE_BYTES = (4 * 16 * NB * AD + 2 * 4 * 16 * NB) * 4;
  __shared__ __align__(16) unsigned char lds[KTILE_BYTES > MERGE_BYTES ? KTILE_BYTES : MERGE_BYTES];
  for (int it = i0; it < i1; ++it) {
    const int code = codes[it];
    const int row = code >> 11;
    const int split = (code >> 5) & 63;
    if (row < 0 || row >= rows || split >= max_splits) continue;
    const int nb = min(min(code & 31, NB * QB), rows - row);
    if (nb <= 0) continue;
    int plast = 0;
#pragma unroll
    for (int j = 0; j < NB * QB; ++j) plast = max(plast, min(pos[row + min(j, nb - 1)], cap - 1));
    const int kstart = split * chunk;
    if (kstart > plast) continue;  // past the item's context (uniform per workgroup)
    const int kend = min(kstart + chunk, plast + 1);
    if (NB == 2 && nb > QB)
      attn_block_item<G, NB>(q, sq_b, sq_h, kc, vc, sk_s, sk_h, sk_t, out, so_b, so_h, slots, pos, scale_log2, chunk,
                             part, max_splits, cap, row, nb, kh, KV, split, kstart, kend, lds);
    else
      attn_block_item<G, 1>(q, sq_b, sq_h, kc, vc, sk_s, sk_h, sk_t, out, so_b, so_h, slots, pos, scale_log2, chunk,
                            part, max_splits, cap, row, nb, kh, KV, split, kstart, kend, lds);
    __syncthreads();  // the next item's K tiles reuse the merge area
  }
}

// Bins of an item launch: 2 workgroups per CU over the kv heads (one round at the kernel's 2 waves per SIMD), at
// most one per row. Measured on MI355X, 2264-row mixed step at 8 kv heads (graph-timed): 512 workgroups 205 us,
// 448 206, 384 220, 256 220, 576 245, 768 229.
static int attn_item_bins(int rows, int kv_heads) { return std::max(1, std::min(rows, 512 / kv_heads)); }

M3X_API int m3x_decode_attn_item_bins(int rows, int kv_heads, int max_ctx, int chunk) {
  if (rows <= 0 || kv_heads <= 0 || max_ctx <= 0 || chunk <= 0) return 0;
  return attn_item_bins(rows, kv_heads);
}

// Host side: the work items of an item launch for rows laid out as runs (first row, rows, first position): each run
// cut into blocks of up to min(16, 2 * (16 / (heads / kv_heads))) rows (the rows one workgroup attends in one pass
// over their keys), each block's keys into splits of `chunk`; an item is one
// split of one block, cost = its keys + 64. Items are dealt into `bins` bins longest processing time first (stable
// by item index on equal costs), each to the least loaded bin (the lowest index on equal loads). Writes
// [bins, start[0..bins], codes bin by bin] with code = 2048 * first_row + 32 * split + rows and returns the count.
M3X_API long m3x_decode_attn_items(const int32_t* runs, int nruns, int heads, int kv_heads, int bins, int chunk,
                                   int32_t* out, long out_cap) {
  if (!runs || !out) return M3X_ENULL;
  if (nruns < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || bins <= 0 || chunk <= 0) return M3X_EINVAL;
  const int qb = std::min(16, 2 * std::max(1, 16 / (heads / kv_heads)));
  std::vector<long> cost;
  std::vector<int32_t> code;
  cost.reserve(nruns * 2);
  code.reserve(nruns * 2);
  for (int i = 0; i < nruns; ++i) {
    const long r0 = runs[3 * i], n = runs[3 * i + 1], p0 = runs[3 * i + 2];
    if (r0 < 0 || n < 0 || p0 < 0 || r0 + n > (1L << 20)) return M3X_EINVAL;
    for (long s = 0; s < n; s += qb) {
      const long m = std::min<long>(qb, n - s);
      const long keys = p0 + s + m;  // the block's last row attends keys 0 .. keys - 1
      const long nsp = (keys + chunk - 1) / chunk;
      if (nsp > 64) return M3X_EINVAL;
      for (long sp = 0; sp < nsp; ++sp) {
        cost.push_back(std::min<long>(chunk, keys - sp * chunk) + 64);
        code.push_back((int32_t)(2048 * (r0 + s) + 32 * sp + m));
      }
    }
  }
  const long nitems = (long)code.size();
  if (out_cap < 2 + bins + nitems) return M3X_EINVAL;
  std::vector<long> order(nitems);
  for (long i = 0; i < nitems; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](long a, long b) { return cost[a] > cost[b]; });
  // the bin of the j-th item in dealing order, then the codes placed bin by bin in that order
  std::vector<int> bin_of(nitems);
  std::vector<long> count(bins, 0);
  using Load = std::pair<long, int>;
  std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
  const long k = std::min<long>(bins, nitems);
  for (long b = 0; b < k; ++b) {
    bin_of[b] = (int)b;
    heap.push(Load(cost[order[b]], (int)b));
  }
  for (long j = k; j < nitems; ++j) {
    const Load top = heap.top();
    heap.pop();
    bin_of[j] = top.second;
    heap.push(Load(top.first + cost[order[j]], top.second));
  }
  for (long j = 0; j < nitems; ++j) ++count[bin_of[j]];
  out[0] = bins;
  out[1] = 0;
  long acc = 0;
  for (int b = 0; b < bins; ++b) {
    const long c = count[b];
    count[b] = 2 + bins + acc;  // the bin's next write position
    acc += c;
    out[2 + b] = (int32_t)acc;
  }
  for (long j = 0; j < nitems; ++j) out[count[bin_of[j]]++] = code[order[j]];
  return 2 + bins + nitems;
}

template <int G>
__global__ __launch_bounds__(256) void decode_attn_combine_kernel(uint16_t* __restrict__ out, long so_b, long so_h,
                                                                  const int32_t* __restrict__ pos, int chunk,
                                                                  const float* __restrict__ part, int max_splits,
                                                                  int cap) {
  const int row = blockIdx.x;
  const int kh = blockIdx.y;
  const int KV = gridDim.y;
  const int nsplit = min((min(pos[row], cap - 1) + chunk) / chunk, max_splits);
  if (nsplit <= 1 || threadIdx.x >= G * AD) return;
  const int h = threadIdx.x / AD;
  const int d = threadIdx.x % AD;
  const float* pp = part + ((long)row * KV + kh) * max_splits * PART_STRIDE;
  // splits SB at a time, every load of a block issued before its first use (indices clamped, always in bounds);
  // the max and the sums still run over the splits in order
  constexpr int SB = 16;
  float M = -INFINITY;
  for (int s0 = 0; s0 < nsplit; s0 += SB) {
    float mv[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) mv[i] = pp[min(s0 + i, nsplit - 1) * PART_STRIDE + h];
#pragma unroll
    for (int i = 0; i < SB; ++i)
      if (s0 + i < nsplit) M = fmaxf(M, mv[i]);
  }
  float L = 0.f, O = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += SB) {
    float mv[SB], lv[SB], ov[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const float* ps = pp + min(s0 + i, nsplit - 1) * PART_STRIDE;
      mv[i] = ps[h];
      lv[i] = ps[2 + h];
      ov[i] = ps[8 + h * AD + d];
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      if (s0 + i < nsplit) {
        const float f = exp2f(mv[i] - M);
        L += lv[i] * f;
        O += ov[i] * f;
      }
    }
  }
  out[(long)row * so_b + (long)(kh * G + h) * so_h + d] = f2bf(O / L);
}

M3X_API size_t m3x_decode_attn_workspace(int rows, int kv_heads, int max_ctx, int chunk) {
  if (rows <= 0 || kv_heads <= 0 || max_ctx <= 0 || chunk <= 0) return 0;
  const long splits = (max_ctx + chunk - 1) / chunk;
  return (size_t)rows * kv_heads * splits * PART_STRIDE * sizeof(float);
}

// max_ctx: an upper bound on pos[r] + 1 for every row (the caller's context bucket); it sizes the grid.
// chunk: keys per split, a multiple of 128. cap (the cache's per-slot capacity) must be a multiple of 32 so the
// last 32-key tile of a row stays inside its slot. items (nullable): the step's work items (attn_block_kernel);
// with it, one launch of attn_block_kernel attends every row, the rows of an inline prefill QB at a time.
M3X_API int m3x_decode_attn(const void* q, long sq_b, long sq_h, const void* k_cache, const void* v_cache, long sk_s,
                            long sk_h, long sk_t, int cap, void* out, long so_b, long so_h, const int64_t* slots,
                            const int32_t* pos, const int32_t* items, float scale, int rows, int heads, int kv_heads,
                            int head_dim, int max_ctx, int chunk, void* workspace, size_t ws_bytes, void* stream) {
  if (rows < 0 || heads <= 0 || kv_heads <= 0 || max_ctx <= 0) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!q || !k_cache || !v_cache || !out || !slots || !pos) return M3X_ENULL;
  if (head_dim != AD || heads % kv_heads) return M3X_EUNSUPPORTED;
  const int G = heads / kv_heads;
  if (G != 1 && G != 2) return M3X_EUNSUPPORTED;
  if (chunk <= 0 || chunk % 128 || cap % 32 || max_ctx > cap) return M3X_EINVAL;
  if ((sq_b | sq_h | sk_s | sk_h | sk_t) & 7) return M3X_EINVAL;
  if (!m3x_aligned16(q) || !m3x_aligned16(k_cache) || !m3x_aligned16(v_cache)) return M3X_EINVAL;
  if (items && (((so_b | so_h) & 7) || !m3x_aligned16(out))) return M3X_EINVAL;  // item rows store 16 bytes
  const int max_splits = (max_ctx + chunk - 1) / chunk;
  if (max_splits > 1) {
    if (!workspace) return M3X_ENULL;
    if (ws_bytes < m3x_decode_attn_workspace(rows, kv_heads, max_ctx, chunk)) return M3X_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  const float scale_log2 = scale * 1.44269504088896341f;
  if (rows > 65535 * 64 || kv_heads > 65535) return M3X_EINVAL;
  dim3 grid(rows, kv_heads, max_splits);
  if (items && (rows >= (1 << 20) || max_splits > 64)) return M3X_EINVAL;  // item codes: row < 2^20, split < 64
  const dim3 igrid(attn_item_bins(rows, kv_heads), kv_heads, 1);
#define M3X_ATTN_LAUNCH(GG)                                                                                          \
  if (items)                                                                                                         \
    hipLaunchKernelGGL((attn_block_kernel<GG>), igrid, dim3(256), 0, st, (const uint16_t*)q, sq_b, sq_h,            \
                       (const uint16_t*)k_cache, (const uint16_t*)v_cache, sk_s, sk_h, sk_t, (uint16_t*)out, so_b,   \
                       so_h, slots, pos, scale_log2, chunk, (float*)workspace, max_splits, cap, items, rows);       \
  else                                                                                                               \
    hipLaunchKernelGGL((decode_attn_kernel<GG, M3X_ATTN_KL>), grid, dim3(256), 0, st, (const uint16_t*)q, sq_b,     \
                       sq_h, (const uint16_t*)k_cache, (const uint16_t*)v_cache, sk_s, sk_h, sk_t, (uint16_t*)out,   \
                       so_b, so_h, slots, pos, scale_log2, chunk, (float*)workspace, max_splits, cap);              \
  if (max_splits > 1)                                                                                                \
    hipLaunchKernelGGL(decode_attn_combine_kernel<GG>, dim3(rows, kv_heads), dim3(256), 0, st, (uint16_t*)out, so_b, \
                       so_h, pos, chunk, (const float*)workspace, max_splits, cap)
  if (G == 2) {
    M3X_ATTN_LAUNCH(2);
  } else {
    M3X_ATTN_LAUNCH(1);
  }
#undef M3X_ATTN_LAUNCH
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Allocation-free decode attention for callers that cannot allocate (code under graph capture, tight serving
// loops): the split partials go to `scratch`, a file-scope device array of M3X_NOALLOC_SCRATCH_BYTES that every
// GPU the library runs on holds until the process ends. In host code the array's name is only a stand-in: its
// device address is taken once per device with hipGetSymbolAddress, on that device's first call, and only that
// address reaches a kernel. Calls that overlap on one GPU share the array and race; the partials need no clearing
// (the combine reads only the splits the same call wrote).
#define M3X_NOALLOC_SCRATCH_BYTES (4u << 20)
#define M3X_NOALLOC_MAX_DEVICES 64
static __device__ __align__(256) unsigned char scratch[M3X_NOALLOC_SCRATCH_BYTES];
static void* g_scratch_addr[M3X_NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_address(void** addr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return M3X_ELAUNCH;
  if (dev < 0 || dev >= M3X_NOALLOC_MAX_DEVICES) return M3X_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return M3X_ELAUNCH;
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return M3X_OK;
}

M3X_API int m3x_decode_attn_noalloc(const void* q, long sq_b, long sq_h, const void* k_cache, const void* v_cache,
                                    long sk_s, long sk_h, long sk_t, int cap, void* out, long so_b, long so_h,
                                    const int64_t* slots, const int32_t* pos, const int32_t* items, float scale,
                                    int rows, int heads, int kv_heads, int head_dim, int max_ctx, int chunk,
                                    void* stream) {
  if (rows < 0 || kv_heads <= 0 || max_ctx <= 0 || chunk <= 0) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  const bool split = (max_ctx + chunk - 1) / chunk > 1;
  const size_t need = split ? m3x_decode_attn_workspace(rows, kv_heads, max_ctx, chunk) : 0;
  if (need > M3X_NOALLOC_SCRATCH_BYTES) return M3X_EWORKSPACE;
  void* ws = nullptr;
  if (split) {
    const int st = scratch_address(&ws);
    if (st != M3X_OK) return st;
  }
  return m3x_decode_attn(q, sq_b, sq_h, k_cache, v_cache, sk_s, sk_h, sk_t, cap, out, so_b, so_h, slots, pos, items,
                         scale, rows, heads, kv_heads, head_dim, max_ctx, chunk, ws, split ? M3X_NOALLOC_SCRATCH_BYTES : 0,
                         stream);
}

// ---------------------------------------------------------------------------------------------------------
// Depth-transformer self-attention over one frame's positions (serve/fast_depth.py:102-121, SDPA causal at a
// group start, incremental over the within-group KV otherwise).
// qkv rows (b, t) at positions p0 + t, read at qkv + b*sqb + t*sqt, laid out q | k | v with heads inside
// (view(B,T,3,H,hd)). kd/vd: per-frame scratch [B, H, np, hd]. If write_kv, the T new K/V rows are stored at
// positions p0..p0+T-1. Queries t in [tq0, T) attend keys 0..p0+t; output row (b, t - tq0) at out + b*sob + tq*sot.
// One wave per (b, head); HD in {64, 128}, np <= 64. The wave reads K and V rows RPI = 512/HD at a time, each
// row as HD/8 adjacent 16-byte lane pieces, so a load instruction covers whole rows (lane = row r in the group x
// piece c). Scores: a lane's 8-element partial dot product, summed over the row's lanes with DPP moves.
// P.V: each lane accumulates p_j * V[j][8c..8c+7] over its rows, then the row groups are summed with DPP and
// permlane swaps.
// Every K and V load of a query is issued before the first wait: NG row groups (a power of two covering the
// longest query's keys) are loaded unconditionally, rows past the query's last key clamped to it, because a
// conditional load whose register is merged after the branch makes the compiler wait for it there.
// With write_kv the keys and values of this call's own positions are read from qkv, and the last query's
// registers, which hold every one of them, are what is stored to the scratch.
template <int DT, int HD, int NG>
__global__ __launch_bounds__(64) void depth_attn_kernel(const Elt<DT>* __restrict__ qkv, long sqb, long sqt,
                                                        Elt<DT>* kd, Elt<DT>* vd, Elt<DT>* __restrict__ out,
                                                        long sob, long sot, int T, int p0, int tq0, int H, int np,
                                                        float scale, int write_kv) {
  constexpr int PPR = HD / 8;   // 16-byte pieces per row
  constexpr int RPI = 64 / PPR; // rows per load instruction
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int r = lane / PPR, c = lane % PPR;
  Elt<DT>* kb = kd + ((long)b * H + h) * np * HD;
  Elt<DT>* vb = vd + ((long)b * H + h) * np * HD;
  const Elt<DT>* qb = qkv + (long)b * sqb + (long)h * HD;  // q of row t at qb + t*sqt; k at +H*HD; v at +2*H*HD
  // key/value row j of this (b, h): the scratch below p0 (or always without write_kv), else this call's qkv row
  const int own = write_kv ? p0 : np;
  auto krow = [&](int j) { return j < own ? kb + (long)j * HD : qb + (long)(j - p0) * sqt + (long)H * HD; };
  auto vrow = [&](int j) { return j < own ? vb + (long)j * HD : qb + (long)(j - p0) * sqt + 2L * H * HD; };
  for (int t = tq0; t < T; ++t) {
    const int nk = p0 + t + 1;
    const int ng = (nk + RPI - 1) / RPI;
    const V8<DT> qv = ldv<DT>(qb + (long)t * sqt + 8 * c);
    V8<DT> kv[NG], vv[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int j = min(g * RPI + r, nk - 1);
      kv[g] = ldv<DT>(krow(j) + 8 * c);
      vv[g] = ldv<DT>(vrow(j) + 8 * c);
    }
    float qf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[e] = E<DT>::to_f(qv.v[e]);
    float s[NG];
    float m = -INFINITY;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      s[g] = -INFINITY;
      if (g < ng) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a = fmaf(qf[e], E<DT>::to_f(kv[g].v[e]), a);
        a = group_sum<PPR>(a);
        s[g] = g * RPI + r < nk ? a * scale : -INFINITY;
        m = fmaxf(m, s[g]);
      }
    }
    m = across_max<PPR>(m);
    float l = 0.f;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
        const float p = g * RPI + r < nk ? expf(s[g] - m) : 0.f;
        l = l + p;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(p, E<DT>::to_f(vv[g].v[e]), acc[e]);
      }
    }
    l = across_sum<PPR>(l);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = across_sum<PPR>(acc[e]);
    if (r == 0) {
      V8<DT> ov;
#pragma unroll
      for (int e = 0; e < 8; ++e) ov.v[e] = E<DT>::from_f(acc[e] / l);
      stv<DT>(out + (long)b * sob + (long)(t - tq0) * sot + (long)h * HD + 8 * c, ov);
    }
    // the last query has loaded every new row (keys p0..p0+T-1, from qkv): store them to the scratch
    if (write_kv && t == T - 1) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const int j = g * RPI + r;
        if (j >= p0 && j < nk) {
          stv<DT>(kb + (long)j * HD + 8 * c, kv[g]);
          stv<DT>(vb + (long)j * HD + 8 * c, vv[g]);
        }
      }
    }
  }
}

M3X_API int m3x_depth_attn(const void* qkv, long sqb, long sqt, void* kd, void* vd, void* out, long sob, long sot,
                           int B, int T, int p0, int tq0, int heads, int head_dim, int np, float scale, int write_kv,
                           int dtype, void* stream) {
  if (B < 0 || T <= 0 || p0 < 0 || tq0 < 0 || tq0 >= T || heads <= 0) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!qkv || !kd || !vd || !out) return M3X_ENULL;
  if (p0 + T > np || np > 64) return M3X_EINVAL;
  if (head_dim != 64 && head_dim != 128) return M3X_EUNSUPPORTED;
  if (((sqb | sqt | sob | sot) & 7) || !m3x_aligned16(qkv) || !m3x_aligned16(kd) || !m3x_aligned16(vd) ||
      !m3x_aligned16(out))
    return M3X_EINVAL;
  hipStream_t st = (hipStream_t)stream;
#define M3X_DA(DTT, HDD, NGG)                                                                                     \
  hipLaunchKernelGGL((depth_attn_kernel<DTT, HDD, NGG>), dim3(B, heads), dim3(64), 0, st, (const Elt<DTT>*)qkv,    \
                     sqb, sqt, (Elt<DTT>*)kd, (Elt<DTT>*)vd, (Elt<DTT>*)out, sob, sot, T, p0, tq0, heads, np,        \
                     scale, write_kv)
#define M3X_DA_NG(DTT, HDD)                                                        \
  do {                                                                             \
    const int groups = m3x_ceil_div(p0 + T, 512 / HDD);                            \
    if (groups <= 1) M3X_DA(DTT, HDD, 1);                                          \
    else if (groups <= 2) M3X_DA(DTT, HDD, 2);                                     \
    else if (groups <= 4) M3X_DA(DTT, HDD, 4);                                     \
    else if (groups <= 8) M3X_DA(DTT, HDD, 8);                                     \
    else M3X_DA(DTT, HDD, 16);                                                     \
  } while (0)
  if (dtype == M3X_BF16 && head_dim == 128) M3X_DA_NG(M3X_BF16, 128);
  else if (dtype == M3X_BF16) M3X_DA_NG(M3X_BF16, 64);
  else if (dtype == M3X_F16 && head_dim == 128) M3X_DA_NG(M3X_F16, 128);
  else if (dtype == M3X_F16) M3X_DA_NG(M3X_F16, 64);
  else if (dtype == M3X_F32 && head_dim == 128) M3X_DA_NG(M3X_F32, 128);
  else if (dtype == M3X_F32) M3X_DA_NG(M3X_F32, 64);
  else return M3X_EUNSUPPORTED;
#undef M3X_DA_NG
#undef M3X_DA
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}
