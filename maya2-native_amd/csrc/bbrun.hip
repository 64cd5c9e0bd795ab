// The 28-layer backbone decode of ONE row (the one-seat frame) as ONE persistent kernel
// (serve/fast_backbone.py:176-234, the fuse_rope branch :187-203 and the decode attention :31-58).
//
// Launched one kernel per step, a layer of the one-row backbone is 7 dependent launches (q|k|v, q/k norm + RoPE +
// cache write, split attention, its combine, o, gate|up, down) of 3-6 us each, almost all of it launch and cold
// memory latency. Here one workgroup per CU stays resident for all layers, and the steps hand over through LL words
// in global memory (m3x_ll.h):
//   S1 q|k|v     every workgroup: one 16-column tile of the 4096, from the residual row it keeps in LDS (the input
//                RMSNorm applied explicitly at layer 0, folded into the packed weight after it, as the launch path);
//   S2 attention every workgroup: one (kv head, split) item of 8 x 32: the two q heads and the new key of its kv head
//                normed and rotated (qk_norm_rope8, the launch kernels' arithmetic), the new key and value written
//                to the cache by the item that holds the row's position, fp32 scores / softmax / P.V over the
//                split's keys; the split's partial (max, sum, 128 values per q head) goes out;
//   S3 combine   workgroups 0..15: one q head each, its 32 partials folded in split order;
//   S4 o         workgroups 192..255: one 16-column tile of the o projection (K = 2048);
//   S5 residual  every workgroup: x = dt(x + o), then workgroups 0..191: one gate|up tile pair with the
//                post-attention RMSNorm folded, SwiGLU;
//   S6 down      workgroups 192..255: one 16-column tile of the down projection (K = 3072);
//   S7 residual  every workgroup: x = dt(x + down), the next layer's S1.
// A step's weights (and an attention item's cached keys and values) are loaded before the step waits for its
// input, so the weight stream and the cache reads overlap the chain of handovers. The split size follows the row's
// position (32 splits of ceil((pos + 1) / 32) keys rounded up to 16), so every workgroup attends about the same
// number of keys. After the last layer workgroup 0 stores the residual row; the caller's final norm reads it.
// Every wait is bounded by the run's spin limit: a workgroup whose input never arrives sets the error word and
// skips the rest, so the grid always drains (the output row is then not written).
#include "m3x_ll.h"
#include "m3x_norm.h"

// Arguments of one run (plain pointers and sizes; include/m3x.h declares the same layout).
struct M3xBackboneLayer {
  const void* wqkv;  // packed [4096, 1024]: plain at layer 0, the input RMSNorm weight folded in after it
  const void* wo;    // packed [1024, 2048]
  const void* wg;    // packed [3072, 1024], the post-attention RMSNorm weight folded in
  const void* wu;    // packed [3072, 1024], likewise
  const void* wd;    // packed [1024, 3072]
  const void* wq;    // q_norm weight [128]
  const void* wk;    // k_norm weight [128]
  void* kc;          // key cache [slots][8][cap][128]
  void* vc;          // value cache
};
struct M3xBackboneRun {
  const M3xBackboneLayer* layer;  // device array [layers]
  int layers, cap, nwg, probe;
  unsigned spin_limit;
  float eps, scale;
  const void* x;                  // [1024] the row's input
  void* h_out;                    // [1024] the last layer's residual
  const int64_t* slots;           // [1]
  const int32_t* pos;             // [1]
  const void* cos;
  const void* sin;
  long s_cos;
  const void* w_in0;              // layer 0's input RMSNorm weight [1024]
  long sk_s, sk_h, sk_t;
  uint64_t* xchg;
  int32_t* sync;                  // [0] epoch, [1] workgroups done, [2] error
  uint64_t* prof;                 // optional [256][512] real-time stamps of each workgroup's steps (profiling)
};

namespace bb {
using ll::ll_poll16;
using ll::ll_poll8;
using ll::ll_st8;
using ll::ro_rsrc;
using ll::bld16;

constexpr int NT = 256;                 // threads per workgroup
constexpr int NWG = 256;                // workgroups: one per CU
constexpr int DM = 1024, H = 16, KV = 8, HD = 128, FF = 3072;
constexpr int NQKV = (H + 2 * KV) * HD; // 4096: one q|k|v tile per workgroup
constexpr int SPLITS = NWG / KV;        // 32 attention splits per kv head
constexpr int SMAX = 128;               // keys per split at most (positions below 4096)
constexpr int KS = HD + 8;              // LDS row stride of the split's keys and values: 16 lanes hit 16 bank groups
constexpr int PW = 2 * (HD + 2);        // partial words per item: per q head its max, its sum and 128 values
constexpr int NOD = 64;                 // workgroups 192..255 own the o and down tiles
constexpr int NGU = FF / 16;            // workgroups 0..191 own the gate|up tile pairs

// exchange buffers (8-byte words, 4 bytes of payload each); two copies alternating by layer
constexpr long W_QKV = NQKV / 2, W_PART = (long)NWG * PW, W_ATT = H * HD / 2, W_O = DM / 2, W_GU = FF / 2,
               W_DN = DM / 2;
constexpr long O_QKV = 0, O_PART = O_QKV + 2 * W_QKV, O_ATT = O_PART + 2 * W_PART, O_O = O_ATT + 2 * W_ATT,
               O_GU = O_O + 2 * W_O, O_DN = O_GU + 2 * W_GU, X_WORDS = O_DN + 2 * W_DN;
constexpr int STEPS = 6;                // tags per layer: q|k|v, partials, attention, o, gate|up, down

struct Smem {
  uint16_t x[DM];                       // the residual row
  uint16_t b[FF + 8];                   // the B operand row of the step's tile
  union {
    struct {
      uint16_t kt[SMAX][KS];            // the split's keys
      uint16_t vt[SMAX][KS];            // and values
    } kv;
    float comb[SPLITS][HD + 2];         // a combine workgroup's 32 partials of its q head
  } u;
  uint16_t raw[4 * HD];                 // q heads 2h, 2h+1, then the new key and value, as projected
  uint16_t qb[2][HD];                   // the q heads, normed and rotated
  float cw[SPLITS];                     // a combine workgroup's split weights exp(m_s - M)
  uint16_t kn[HD];                      // the new key, normed and rotated
  float sc[2][SMAX];                    // scores, then probabilities
  float part[2][4][16];                 // per-wave partial tiles (gate, up)
  float red[2][4];                      // per-wave reductions
  float inv;                            // the residual row's 1 / rms
  ll::Sync sync;
};

// a 16-column weight tile: wave w takes K slice w of 4 (NF fragments of 32)
template <int NF>
struct WT {
  u16x8 f[NF];
};
template <int NF>
__device__ __forceinline__ void load_wt(WT<NF>& t, const void* w, int tile, int K) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t r = ro_rsrc(w);
  const int s0 = (tile * 16 * K + wave * NF * 512) * 2;  // uniform: scalar offset
#pragma unroll
  for (int f = 0; f < NF; ++f) t.f[f] = bld16(r, 16 * lane, s0 + f * 1024);
}
// W tile x b^T for the single row b (the MFMA's other 15 rows are zero: lanes l % 16 != 0 feed zeros)
template <int NF>
__device__ __forceinline__ f32x4_t mma_row(const WT<NF>& t, const uint16_t* b) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool live = (lane & 15) == 0;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int k = (wave * NF + f) * 32 + 8 * (lane >> 4);
    const u16x8 bv = *reinterpret_cast<const u16x8*>(&b[live ? k : 0]);
    acc = mfma16x16x32<M3X_BF16>(t.f[f], live ? bv : u16x8{}, acc);
  }
  return acc;
}
// the four waves' partials of column c (slot order, fp32): thread c < 16 gets the tile's column c
__device__ __forceinline__ void put_part(Smem& sm, int a, f32x4_t acc) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if ((lane & 15) == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.part[a][wave][4 * (lane >> 4) + r] = acc[r];
  }
}
__device__ __forceinline__ float get_part(const Smem& sm, int a, int c) {
  return ((sm.part[a][0][c] + sm.part[a][1][c]) + sm.part[a][2][c]) + sm.part[a][3][c];
}
// LL store of a tile's 16 bf16 outputs (thread c < 16 holds column c): 8 words from the even threads
__device__ __forceinline__ void st_tile(__amdgpu_buffer_rsrc_t rs, int base, int tile, uint16_t v, uint32_t tag) {
  const int c = threadIdx.x;
  const uint32_t nb = (uint32_t)__shfl_down((int)v, 1, 64);
  if (c < 16 && (c & 1) == 0) ll_st8(rs, base + tile * 8 + c / 2, (uint32_t)v | (nb << 16), tag);
}

// x = dt(x + a) with a from an LL buffer of DM bf16 (one 16-byte chunk of 4 per thread), then sm.inv = its 1 / rms
// (fp32 sum of squares: each thread's 4 in order, the wave's xor tree, then the 4 waves in order)
__device__ __forceinline__ bool add_row(Smem& sm, int& vph, __amdgpu_buffer_rsrc_t rs, int base, uint32_t tag,
                                        int probe, float eps) {
  const int t = threadIdx.x;
  const bool ok = ll_poll16<1>(
      sm.sync, vph, rs, base + 2 * t, [](int) { return 0; }, 1, probe, [](int) { return true; }, tag,
      [&](int, uint32_t p0, uint32_t p1) {
        const uint16_t av[4] = {(uint16_t)(p0 & 0xffff), (uint16_t)(p0 >> 16), (uint16_t)(p1 & 0xffff),
                                (uint16_t)(p1 >> 16)};
#pragma unroll
        for (int e = 0; e < 4; ++e) sm.x[4 * t + e] = f2bf(bf2f(sm.x[4 * t + e]) + bf2f(av[e]));
      });
  return ok;
}
__device__ __forceinline__ void row_inv(Smem& sm, float eps) {
  const int t = threadIdx.x;
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float v = bf2f(sm.x[4 * t + e]);
    q = q + v * v;
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) q = q + __shfl_xor(q, o, 64);
  if ((t & 63) == 0) sm.red[0][t >> 6] = q;
  __syncthreads();
  if (t == 0) sm.inv = 1.0f / sqrtf((((sm.red[0][0] + sm.red[0][1]) + sm.red[0][2]) + sm.red[0][3]) / (float)DM + eps);
  __syncthreads();
}
}  // namespace bb

using namespace bb;

__global__ __launch_bounds__(NT, 1) void backbone_run_kernel(const M3xBackboneRun a) {
  __shared__ Smem sm;
  const int wg = blockIdx.x, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const uint32_t epoch = (uint32_t)a.sync[0];
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(a.xchg, 0, (int)(X_WORDS * 8), 0x00020000);
  const bool od = wg >= NWG - NOD;    // an o / down workgroup
  const int t_od = wg - (NWG - NOD);  // its tile
  const bool gu = wg < NGU;           // a gate|up workgroup
  const int ih = wg / SPLITS, is = wg % SPLITS;  // the attention item: kv head, split
  // the row's slot and position (the host guarantees 0 <= pos < cap; the clamp keeps every access in the slot)
  const long slot = a.slots[0];
  const int pos = min(max(a.pos[0], 0), a.cap - 1);
  const int S = max(16, (((pos + 1 + SPLITS - 1) / SPLITS) + 15) / 16 * 16);
  const int k0 = is * S, n = max(min(k0 + S, pos + 1) - k0, 0);  // the item's keys k0 .. k0 + n - 1
  const bool own_pos = k0 <= pos && pos < k0 + S;
  const float scale = a.scale;
  bool ok = true;
  int vph = 0;
  // stamp k of layer l at slot 16 l + k (profiling only)
  auto stamp = [&](int slot) {
    if (a.prof && tid == 0) a.prof[(long)wg * 512 + slot] = __builtin_amdgcn_s_memrealtime();
  };

  if (tid == 0) sm.sync.spin = a.spin_limit ? a.spin_limit : ll::SPIN_LIMIT;
  for (int i = tid; i < DM / 8; i += NT)
    *reinterpret_cast<u16x8*>(&sm.x[8 * i]) = ld16((const uint16_t*)a.x + 8 * i);
  __syncthreads();

  for (int l = 0; l < a.layers && ok; ++l) {
    const M3xBackboneLayer L = a.layer[l];
    const int par = l & 1;
    const uint32_t s0 = 1u + (uint32_t)(STEPS * l);
    const uint32_t t_qkv = (epoch << 12) | s0, t_part = t_qkv + 1, t_att = t_qkv + 2, t_o = t_qkv + 3,
                   t_gu = t_qkv + 4, t_dn = t_qkv + 5;
    const int b_qkv = O_QKV + par * W_QKV, b_part = O_PART + par * W_PART, b_att = O_ATT + par * W_ATT,
              b_o = O_O + par * W_O, b_gu = O_GU + par * W_GU, b_dn = O_DN + par * W_DN;

    // ---- S1: the layer's input row -> q|k|v tile wg
    {
      WT<8> wt;
      load_wt<8>(wt, L.wqkv, wg, DM);
      stamp(16 * l + 0);
      if (l > 0) {
        const uint32_t t_prev = (epoch << 12) | (s0 - 1);
        ok = add_row(sm, vph, rs, O_DN + (1 - par) * W_DN, t_prev, a.probe, a.eps);
        if (!ok) break;
      }
      stamp(16 * l + 1);
      row_inv(sm, a.eps);
      const float inv = sm.inv;
      if (l == 0) {
        // the input RMSNorm applied to the row (the packed weight of layer 0 is the plain one)
        const __amdgpu_buffer_rsrc_t rw = ro_rsrc(a.w_in0);
        for (int i = tid; i < DM / 8; i += NT) {
          const u16x8 w8 = bld16(rw, 16 * i, 0);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            sm.b[8 * i + e] = f2bf(bf2f(f2bf(bf2f(sm.x[8 * i + e]) * inv)) * bf2f(w8.v[e]));
        }
      } else {
        for (int i = tid; i < DM / 8; i += NT)
          *reinterpret_cast<u16x8*>(&sm.b[8 * i]) = *reinterpret_cast<const u16x8*>(&sm.x[8 * i]);
      }
      __syncthreads();
      put_part(sm, 0, mma_row<8>(wt, sm.b));
      __syncthreads();
      uint16_t v = 0;
      if (tid < 16) {
        const float s = get_part(sm, 0, tid);
        v = f2bf(l == 0 ? s : inv * s);  // the folded norm's row scale (the plain weight at layer 0)
      }
      st_tile(rs, b_qkv, wg, v, t_qkv);
      stamp(16 * l + 2);
    }

    // ---- S2: attention item (ih, is): keys k0 .. k0 + n - 1 of the slot's kv head ih
    {
      // the split's cached keys and values load first (rows past the item clamp to the position: valid, unused)
      const uint16_t* kb = (const uint16_t*)L.kc + slot * a.sk_s + (long)ih * a.sk_h;
      const uint16_t* vb = (const uint16_t*)L.vc + slot * a.sk_s + (long)ih * a.sk_h;
      u16x8 kr[SMAX * HD / 8 / NT], vr[SMAX * HD / 8 / NT];
#pragma unroll
      for (int i = 0; i < SMAX * HD / 8 / NT; ++i) {
        const int c = tid + NT * i, j = c / (HD / 8), d = 8 * (c % (HD / 8));
        const long p = min(k0 + j, pos);
        kr[i] = ld16(kb + p * a.sk_t + d);
        vr[i] = ld16(vb + p * a.sk_t + d);
      }
      // q heads 2 ih, 2 ih + 1, the key and the value of kv head ih, as projected
      const int part = tid >> 5, c4 = tid & 31;  // 16-byte chunks: q 0..63, k 64..95, v 96..127
      const int col = part < 2 ? 2 * ih * HD + 4 * tid : (part == 2 ? H * HD + ih * HD : (H + KV) * HD + ih * HD) + 4 * c4;
      ok = ll_poll16<1>(
          sm.sync, vph, rs, b_qkv + col / 2, [](int) { return 0; }, 1, a.probe, [&](int) { return tid < 128; }, t_qkv,
          [&](int, uint32_t p0, uint32_t p1) {
            *reinterpret_cast<uint2*>(&sm.raw[4 * tid]) = uint2{p0, p1};
          });
      if (!ok) break;
      stamp(16 * l + 3);
#pragma unroll
      for (int i = 0; i < SMAX * HD / 8 / NT; ++i) {
        const int c = tid + NT * i, j = c / (HD / 8), d = 8 * (c % (HD / 8));
        *reinterpret_cast<u16x8*>(&sm.u.kv.kt[j][d]) = kr[i];
        *reinterpret_cast<u16x8*>(&sm.u.kv.vt[j][d]) = vr[i];
      }
      __syncthreads();
      stamp(16 * l + 13);
      // q/k norm + RoPE: lanes 0-15 q head 2 ih, 16-31 q head 2 ih + 1, 32-47 the key (one DPP row each)
      if (wave == 0) {
        const int grp = lane >> 4, t16 = lane & 15;
        const int g3 = min(grp, 2);
        float xv[8];
        const u16x8 r8 = *reinterpret_cast<const u16x8*>(&sm.raw[g3 * HD + 8 * t16]);
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = bf2f(r8.v[e]);
        const u16x8 wv = ld16((const uint16_t*)(g3 < 2 ? L.wq : L.wk) + 8 * t16);
        const u16x8 cv = ld16((const uint16_t*)a.cos + (long)pos * a.s_cos + 8 * t16);
        const u16x8 sv = ld16((const uint16_t*)a.sin + (long)pos * a.s_cos + 8 * t16);
        const u16x8 ov = qk_norm_rope8<HD>(xv, wv, cv, sv, a.eps, t16);
        if (grp < 2) {
          *reinterpret_cast<u16x8*>(&sm.qb[grp][8 * t16]) = ov;
        } else if (grp == 2) {
          *reinterpret_cast<u16x8*>(&sm.kn[8 * t16]) = ov;
        }
      }
      __syncthreads();
      stamp(16 * l + 14);
      // the new key and value into the cache, by the item that holds the position
      if (own_pos && tid < 32) {
        const int d = 8 * (tid & 15);
        if (tid < 16) st16((uint16_t*)L.kc + slot * a.sk_s + (long)ih * a.sk_h + (long)pos * a.sk_t + d,
                           *reinterpret_cast<const u16x8*>(&sm.kn[d]));
        else st16((uint16_t*)L.vc + slot * a.sk_s + (long)ih * a.sk_h + (long)pos * a.sk_t + d,
                  *reinterpret_cast<const u16x8*>(&sm.raw[3 * HD + d]));
      }
      // scores: thread t takes q head t / 128 and key t % 128 (the new key at the position)
      const int g = tid >> 7, jl = tid & (SMAX - 1);
      {
        float s = -INFINITY;
        if (jl < n) {
          const uint16_t* kp = (k0 + jl == pos) ? sm.kn : &sm.u.kv.kt[jl][0];
          float d = 0.f;
#pragma unroll
          for (int c = 0; c < HD / 8; ++c) {
            const u16x8 k8 = *reinterpret_cast<const u16x8*>(&kp[8 * c]);
            const u16x8 q8 = *reinterpret_cast<const u16x8*>(&sm.qb[g][8 * c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) d = fmaf(bf2f(q8.v[e]), bf2f(k8.v[e]), d);
          }
          s = d * scale;
        }
        float m = s;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (lane == 0) sm.red[0][wave] = m;
        __syncthreads();
        m = fmaxf(sm.red[0][2 * g], sm.red[0][2 * g + 1]);
        const float p = jl < n ? expf(s - m) : 0.f;
        sm.sc[g][jl] = p;
        float sum = p;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) sum = sum + __shfl_xor(sum, o, 64);
        if (lane == 0) sm.red[1][wave] = sum;
        __syncthreads();
        sum = sm.red[1][2 * g] + sm.red[1][2 * g + 1];
        // P.V: thread t takes q head t / 128 and dimension t % 128 (the new value at the position)
        const int d = jl;
        // the new value stands in the tile's row pos - k0 (the tile's own row there is the cache's stale entry)
        if (own_pos && tid < HD) sm.u.kv.vt[pos - k0][tid] = sm.raw[3 * HD + tid];
        __syncthreads();
        stamp(16 * l + 15);
        // four running sums over keys j = 4 i + r (a fixed order), so four loads are in flight at once
        float ac[4] = {0.f, 0.f, 0.f, 0.f};
        const int n4 = n & ~3;
        for (int j = 0; j < n4; j += 4) {
#pragma unroll
          for (int r = 0; r < 4; ++r) ac[r] = fmaf(sm.sc[g][j + r], bf2f(sm.u.kv.vt[j + r][d]), ac[r]);
        }
        for (int j = n4; j < n; ++j) ac[j & 3] = fmaf(sm.sc[g][j], bf2f(sm.u.kv.vt[j][d]), ac[j & 3]);
        const float acc = (ac[0] + ac[1]) + (ac[2] + ac[3]);
        const int w0 = b_part + wg * PW + g * (HD + 2);
        if (d == 0) {
          ll_st8(rs, w0, __float_as_uint(n > 0 ? m : -INFINITY), t_part);
          ll_st8(rs, w0 + 1, __float_as_uint(n > 0 ? sum : 0.f), t_part);
        }
        ll_st8(rs, w0 + 2 + d, __float_as_uint(acc), t_part);
      }
      __syncthreads();  // the K/V area is reused by the combine
      stamp(16 * l + 4);
    }

    // ---- S3: combine of q head wg (workgroups 0..15): its 32 partials in split order
    if (wg < H) {
      // thread t reads split t / 8, words t % 8 + 8 i of the q head's 130 (i < 17)
      const int hk = wg >> 1, gq = wg & 1, sp = tid >> 3, k8 = tid & 7;
      constexpr int NW = (HD + 2 + 7) / 8;
      ok = ll_poll8<NW>(
          sm.sync, vph, rs, b_part + (hk * SPLITS + sp) * PW + gq * (HD + 2) + k8, [](int i) { return 8 * i; }, NW,
          a.probe, [&](int i) { return k8 + 8 * i < HD + 2; }, t_part,
          [&](int i, uint32_t p) { sm.u.comb[sp][k8 + 8 * i] = __uint_as_float(p); });
      if (!ok) break;
      stamp(16 * l + 5);
      // the splits' weights exp(m_s - M) once per split (M the largest m_s of the non-empty ones)
      if (tid < SPLITS) {
        float M = sm.u.comb[tid][0];
#pragma unroll
        for (int o = 1; o < SPLITS; o <<= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        sm.cw[tid] = sm.u.comb[tid][1] > 0.f ? expf(sm.u.comb[tid][0] - M) : 0.f;
      }
      __syncthreads();
      if (tid < HD) {
        float L = 0.f, o = 0.f;
        for (int s = 0; s < SPLITS; ++s) {
          const float w = sm.cw[s];
          L = L + sm.u.comb[s][1] * w;
          o = o + sm.u.comb[s][2 + tid] * w;
        }
        const uint16_t v = f2bf(o / L);
        const uint32_t nb = (uint32_t)__shfl_down((int)v, 1, 64);
        if ((tid & 1) == 0) ll_st8(rs, b_att + (wg * HD + tid) / 2, (uint32_t)v | (nb << 16), t_att);
      }
      __syncthreads();
      stamp(16 * l + 6);
    }

    // ---- S4: o projection tile (workgroups 192..255), K = 2048
    if (od) {
      WT<16> wt;
      load_wt<16>(wt, L.wo, t_od, H * HD);
      ok = ll_poll16<2>(
          sm.sync, vph, rs, b_att + 2 * tid, [](int i) { return 2 * NT * i; }, 2, a.probe,
          [](int) { return true; }, t_att, [&](int i, uint32_t p0, uint32_t p1) {
            *reinterpret_cast<uint2*>(&sm.b[4 * (tid + NT * i)]) = uint2{p0, p1};
          });
      if (!ok) break;
      stamp(16 * l + 7);
      __syncthreads();
      put_part(sm, 0, mma_row<16>(wt, sm.b));
      __syncthreads();
      st_tile(rs, b_o, t_od, tid < 16 ? f2bf(get_part(sm, 0, tid)) : (uint16_t)0, t_o);
      stamp(16 * l + 8);
    }

    // ---- S5: x += o (every workgroup), gate|up tile pair wg with the folded norm and SwiGLU (0..191)
    {
      WT<8> wg_, wu_;
      if (gu) {
        load_wt<8>(wg_, L.wg, wg, DM);
        load_wt<8>(wu_, L.wu, wg, DM);
      }
      ok = add_row(sm, vph, rs, b_o, t_o, a.probe, a.eps);
      if (!ok) break;
      stamp(16 * l + 9);
      row_inv(sm, a.eps);
      if (gu) {
        const float inv = sm.inv;
        put_part(sm, 0, mma_row<8>(wg_, sm.x));
        put_part(sm, 1, mma_row<8>(wu_, sm.x));
        __syncthreads();
        uint16_t v = 0;
        if (tid < 16) {
          const float gt = rnd<M3X_BF16>(inv * get_part(sm, 0, tid));
          const float u = rnd<M3X_BF16>(inv * get_part(sm, 1, tid));
          v = f2bf(rnd<M3X_BF16>(silu16(gt)) * u);
        }
        st_tile(rs, b_gu, wg, v, t_gu);
        stamp(16 * l + 10);
      }
    }

    // ---- S6: down projection tile (workgroups 192..255), K = 3072
    if (od) {
      WT<24> wt;
      load_wt<24>(wt, L.wd, t_od, FF);
      ok = ll_poll16<3>(
          sm.sync, vph, rs, b_gu + 2 * tid, [](int i) { return 2 * NT * i; }, 3, a.probe,
          [](int) { return true; }, t_gu, [&](int i, uint32_t p0, uint32_t p1) {
            *reinterpret_cast<uint2*>(&sm.b[4 * (tid + NT * i)]) = uint2{p0, p1};
          });
      if (!ok) break;
      stamp(16 * l + 11);
      __syncthreads();
      put_part(sm, 0, mma_row<24>(wt, sm.b));
      __syncthreads();
      st_tile(rs, b_dn, t_od, tid < 16 ? f2bf(get_part(sm, 0, tid)) : (uint16_t)0, t_dn);
      stamp(16 * l + 12);
    }
  }

  // ---- the last layer's x += down, and workgroup 0 stores the row
  if (ok) {
    const int lp = a.layers - 1;
    ok = add_row(sm, vph, rs, O_DN + (lp & 1) * W_DN, (epoch << 12) | (uint32_t)(STEPS * lp + STEPS), a.probe,
                 a.eps);
    if (ok && wg == 0) {
      for (int i = tid; i < DM / 8; i += NT)
        st16((uint16_t*)a.h_out + 8 * i, *reinterpret_cast<const u16x8*>(&sm.x[8 * i]));
    }
  }

  // ---- the run's end: failures are recorded, and the last workgroup out advances the epoch
  if (!ok && tid == 0) atomicOr(&a.sync[2], 1);
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&a.sync[1], 1);
    if (prev == (int)gridDim.x - 1) {
      a.sync[1] = 0;
      a.sync[0] = (int)((epoch + 1) & 0xFFFFF);
    }
  }
}

M3X_API size_t m3x_backbone_run_xchg_bytes(void) { return (size_t)X_WORDS * 8; }
M3X_API size_t m3x_backbone_run_args_bytes(void) { return sizeof(M3xBackboneRun); }
M3X_API size_t m3x_backbone_run_layer_bytes(void) { return sizeof(M3xBackboneLayer); }

// the whole grid must be resident at once: the device's CUs times the kernel's workgroups per CU cover NWG
static bool bb_resident_ok() {
  constexpr int MAXDEV = 64;
  static int ok_dev[MAXDEV];  // 0: not checked, 1: resident, -1: not
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return false;
  if (ok_dev[dev] == 0) {
    int cus = 0, per = 0;
    const bool q = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                   hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, backbone_run_kernel, NT, 0) == hipSuccess;
    ok_dev[dev] = q && (long)cus * per >= NWG ? 1 : -1;
  }
  return ok_dev[dev] == 1;
}

M3X_API int m3x_backbone_run(const M3xBackboneRun* args, void* stream) {
  if (!args) return M3X_ENULL;
  const M3xBackboneRun& a = *args;
  if (a.layers <= 0 || a.layers > 600 || a.cap <= 0 || a.cap > SPLITS * SMAX || a.nwg != NWG) return M3X_EINVAL;
  if (!a.layer || !a.x || !a.h_out || !a.slots || !a.pos || !a.cos || !a.sin || !a.w_in0 || !a.xchg || !a.sync)
    return M3X_ENULL;
  if ((a.sk_s | a.sk_h | a.sk_t | a.s_cos) & 7) return M3X_EINVAL;
  if (!bb_resident_ok()) return M3X_EUNSUPPORTED;
  hipLaunchKernelGGL(backbone_run_kernel, dim3(NWG), dim3(NT), 0, (hipStream_t)stream, a);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}
