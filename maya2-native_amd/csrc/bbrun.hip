// The 28-layer backbone decode of ONE row (the one-seat frame) as ONE persistent kernel
// (serve/fast_backbone.py:176-234, the fuse_rope branch :187-203 and the decode attention :31-58).
//
// Launched one kernel per step, a layer of the one-row backbone is 7 dependent launches (q|k|v, q/k norm + RoPE +
// cache write, split attention, its combine, o, gate|up, down) of 3-6 us each, almost all of it launch and cold
// memory latency. Here one workgroup per CU stays resident for all layers, and the steps hand over through LL words
// in global memory (m3x_ll.h). A handover costs one device-scope round trip (~0.3 us) only if nothing else is in
// flight in the polling wave: a wave's vector memory counter retires in order, so a poll issued behind a weight
// load waits for that load too. The waves therefore split by role:
//   - waves 0-3 project: they hold the workgroup's weight tiles and its attention split's cached keys and values in
//     registers, each loaded ahead of its use (right after the slot's previous tile is used), run the MFMA tiles
//     and store each tile's outputs;
//   - waves 4-7 only poll, reduce, attend and combine: nothing of theirs is in flight when they poll. The
//     attention and the combine sync these waves alone (an LDS arrival counter), so a burst of the projecting
//     waves' loads never holds them up.
// The two roles run their own loop over the layers and meet at the same workgroup barriers.
// Per layer (every workgroup unless said otherwise):
//   S1 q|k|v     x += the previous layer's down (its two K-half partials summed in order, rounded, added), the
//                row's RMS; one 16-column tile of the 4096 (the input RMSNorm applied explicitly at layer 0, folded
//                into the packed weight after it, as the launch path); the 32 tiles of kv head h sit on XCD h;
//   S2 attention item (kv head wg % 8, split wg / 8): the two q heads and the new key of its kv head normed and
//                rotated (qk_norm_rope8, the launch kernels' arithmetic), the new key and value written to the cache
//                by the item that holds the row's position, scores and P.V on MFMA (fp32 sums, P as a bf16 hi/lo
//                pair), fp32 softmax; the split's partial (max, sum, 128 values per q head) goes out;
//   S3 combine   workgroups 0..15: one q head each (on its kv head's XCD), its 32 partials folded in split order;
//   S4 o         workgroups 0..127: one (16-column tile, K half) unit of the o projection, an fp32 partial;
//   S5 gate|up   x += o (the two partials summed in order, rounded, added), the row's RMS; workgroups 0..191: one
//                gate|up tile pair with the post-attention RMSNorm folded, SwiGLU;
//   S6 down      workgroups 128..255: one (16-column tile, K half) unit of the down projection, an fp32 partial.
// The K halves spread the o and down weights, so no workgroup streams more than ~144 KB a layer, and a consumer of
// a K half polls only that half of its input. The split size follows the row's position (32 splits of
// ceil((pos + 1) / 32) keys rounded up to 16), so every workgroup attends about the same number of keys. After the
// last layer workgroup 0 stores the residual row and its final RMSNorm, and the row's length moves on. Every wait
// is bounded by the run's spin limit: a workgroup whose input never arrives sets the error word and skips the rest,
// so the grid always drains (the output rows are then not written).
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
  const void* w_fin;              // the final RMSNorm weight [1024]
  void* y_out;                    // [1024] the final norm of the last layer's residual
  int64_t* lengths;               // lengths[slots[0]] += real[0] at the run's end (the step's length update)
  const int64_t* real;
};

namespace bb {
using ll::ll_poll16_w;
using ll::ll_poll8_w;
using ll::ll_st8;
using ll::ro_rsrc;
using ll::bld16;
using ll::wg_all;

constexpr int NT = 512;                 // threads per workgroup
constexpr int NM = 256;                 // waves 0-3: the projecting waves; waves 4-7: the io waves
constexpr int NWG = 256;                // workgroups: one per CU
constexpr int DM = 1024, H = 16, KV = 8, HD = 128, FF = 3072;
constexpr int NQKV = (H + 2 * KV) * HD; // 4096: one q|k|v tile per workgroup
constexpr int SPLITS = NWG / KV;        // 32 attention splits per kv head
constexpr int SMAX = 128;               // keys per split at most (positions below 4096)
constexpr int KS = HD + 8;              // LDS row stride of the split's keys and values: 16 lanes hit 16 bank groups
constexpr int PW = 2 * (HD + 2);        // partial words per item: per q head its max, its sum and 128 values
constexpr int KQ = 2;                   // K halves of the o and down projections
constexpr int KO = H * HD / KQ;         // 1024: an o unit's K (workgroups 0..127)
constexpr int KD = FF / KQ;             // 1536: a down unit's K (workgroups 128..255)
constexpr int NOD = NWG / 2;            // o units, then down units
constexpr int NGU = FF / 16;            // workgroups 0..191 own the gate|up tile pairs
constexpr int KVN = SMAX * HD / 8 / NM; // 16-byte chunks of the split's keys (and of its values) per projecting thread

// exchange buffers (8-byte words, 4 bytes of payload each); two copies alternating by layer. The o and down
// partials are fp32 words [K half][1024]; q|k|v, attention and gate|up carry two bf16 per word.
constexpr long W_QKV = NQKV / 2, W_PART = (long)NWG * PW, W_ATT = H * HD / 2, W_O = (long)KQ * DM, W_GU = FF / 2,
               W_DN = (long)KQ * DM;
constexpr long O_QKV = 0, O_PART = O_QKV + 2 * W_QKV, O_ATT = O_PART + 2 * W_PART, O_O = O_ATT + 2 * W_ATT,
               O_GU = O_O + 2 * W_O, O_DN = O_GU + 2 * W_GU, X_WORDS = O_DN + 2 * W_DN;
constexpr int STEPS = 6;                // tags per layer: q|k|v, partials, attention, o, gate|up, down

struct Smem {
  alignas(16) uint16_t x[DM];           // the residual row
  alignas(16) uint16_t b[KD + 8];       // the B operand row of a K-sliced tile (layer 0's normed row, o's, down's)
  alignas(16) uint16_t kt[SMAX][KS];    // the split's keys, a row per key
  alignas(16) uint16_t vt[HD][KS];      // and its values, transposed: a row per dimension (the P.V B operand)
  alignas(16) float comb[SPLITS][HD + 2];  // a combine workgroup's 32 partials of its q head
  alignas(16) uint16_t raw[4 * HD];     // q heads 2h, 2h+1, then the new key and value, as projected
  alignas(16) uint16_t qb[2][HD];       // the q heads, normed and rotated
  alignas(16) uint16_t kn[HD];          // the new key, normed and rotated
  alignas(16) uint16_t pb[4][SMAX];     // probabilities of q heads 0, 1 (bf16), then what bf16 left of them
  alignas(16) uint16_t nw[2][HD];       // the layer's q_norm and k_norm weights
  alignas(16) uint16_t cs[2][HD];       // cos and sin at the row's position
  float cw[SPLITS];                     // a combine workgroup's split weights exp(m_s - M)
  float part[2][4][16];                 // per-wave partial tiles (gate, up)
  float red[2][8];                      // per-io-wave reductions (two q heads each)
  float rq[2][4];                       // per-io-wave sums of squares, alternating with the votes
  int iob;                              // the io waves' own barrier: arrivals so far
  ll::Sync sync;
};

// the layer table through the constant address space: scalar loads (a generic load of it would be a vector load,
// since the kernel's own stores might alias it, and would then wait behind every weight load in flight)
__device__ __forceinline__ M3xBackboneLayer layer_at(const M3xBackboneLayer* t, int l) {
  typedef const uint64_t __attribute__((address_space(4)))* CW;
  static_assert(sizeof(M3xBackboneLayer) == 9 * sizeof(uint64_t), "nine pointers");
  const CW p = (CW)(t + l);
  uint64_t w[9];
#pragma unroll
  for (int i = 0; i < 9; ++i) w[i] = p[i];
  M3xBackboneLayer L;
  __builtin_memcpy(&L, w, sizeof L);
  return L;
}

// the q|k|v tile of workgroup wg: XCD x = wg % 8 holds q heads 2x, 2x+1 (tiles 16x ..), key head x, value head x
__device__ __forceinline__ int qkv_tile(int wg) {
  const int x = wg & 7, j = wg >> 3;
  return j < 16 ? 16 * x + j : (j < 24 ? 128 + 8 * x + (j - 16) : 192 + 8 * x + (j - 24));
}

// a 16-column weight tile over fragments f0 .. f0 + 4 NF - 1 of its K (32 each): projecting wave w takes NF of them
// A load that is not needed (no next layer, no gate|up pair) still issues, through an empty buffer resource: it
// moves no data and returns zeros, and every path keeps the same count of loads in flight, so the compiler's wait
// before each use stays exact (a conditional load would make it wait for everything issued since).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t opt_rsrc(const void* p, bool on) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, on ? 0x7fffffff : 0, 0x00020000);
}
template <int NF>
__device__ __forceinline__ void load_wt(u16x8* t, const void* w, int tile, int K, int f0, bool on = true) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t r = opt_rsrc(w, on);
  const int s0 = (tile * 16 * K + (f0 + wave * NF) * 512) * 2;  // uniform: scalar offset
#pragma unroll
  for (int f = 0; f < NF; ++f) t[f] = bld16(r, 16 * lane, s0 + f * 1024);
}
// W tile x b^T for the single row b (the MFMA's other 15 rows are zero: lanes l % 16 != 0 feed zeros)
template <int NF>
__device__ __forceinline__ f32x4_t mma_row(const u16x8* t, const uint16_t* b) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool live = (lane & 15) == 0;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int k = (wave * NF + f) * 32 + 8 * (lane >> 4);
    const u16x8 bv = *reinterpret_cast<const u16x8*>(&b[live ? k : 0]);
    acc = mfma16x16x32<M3X_BF16>(t[f], live ? bv : u16x8{}, acc);
  }
  return acc;
}
// the four projecting waves' partials of column c (slot order, fp32): io thread c < 16 gets the tile's column c
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
// the workgroup's o unit (workgroups 0..127: 8 fragments per projecting wave, the rest read as zeros) or down unit
// (128..255: 12 fragments), in one register slot
constexpr int NOD_F = KD / 32 / 4;  // 12
__device__ __forceinline__ void load_od(u16x8 (&t)[NOD_F], const M3xBackboneLayer& L, bool ow, int tu, int kh) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  constexpr int NOF = KO / 32 / 4;  // 8
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(ow ? L.wo : L.wd), 0, ow ? DM * H * HD * 2 : DM * FF * 2, 0x00020000);
  const int s0 = ow ? (tu * 16 * (H * HD) + (kh * (KO / 32) + wave * NOF) * 512) * 2
                    : (tu * 16 * FF + (kh * (KD / 32) + wave * NOD_F) * 512) * 2;
#pragma unroll
  for (int f = 0; f < NOD_F; ++f) t[f] = bld16(r, 16 * lane + (ow && f >= NOF ? ll::OOB : 0), s0 + f * 1024);
}

// the split's cached keys and values: rows past the split's n keys read as zeros (an out-of-range offset: no
// traffic), so the P.V tile's unused keys are zero times zero
__device__ __forceinline__ void load_kv(u16x8 (&kr)[KVN], u16x8 (&vr)[KVN], const M3xBackboneLayer& L, long off,
                                        long sk_t, int cap, int k0, int n, bool on = true) {
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((uint16_t*)L.kc + off, 0,
                                                                      on ? (int)(cap * sk_t * 2) : 0, 0x00020000),
                               rv = __builtin_amdgcn_make_buffer_rsrc((uint16_t*)L.vc + off, 0,
                                                                      on ? (int)(cap * sk_t * 2) : 0, 0x00020000);
#pragma unroll
  for (int i = 0; i < KVN; ++i) {
    const int c = threadIdx.x + NM * i, j = c / (HD / 8), d = 8 * (c % (HD / 8));
    const int o = j < n ? (int)(((long)(k0 + j) * sk_t + d) * 2) : ll::OOB;
    kr[i] = bld16(rk, o, 0);
    vr[i] = bld16(rv, o, 0);
  }
}
// the layer's q_norm weight (8 per projecting thread 0-15) and k_norm weight (16-31); zeros elsewhere
__device__ __forceinline__ void load_nw(u16x8& nq, u16x8& nk, const M3xBackboneLayer& L, bool on) {
  const int t = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(L.wq), 0, on ? HD * 2 : 0,
                                                                      0x00020000),
                               rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(L.wk), 0, on ? HD * 2 : 0,
                                                                      0x00020000);
  nq = bld16(rq, t < 16 ? 16 * t : ll::OOB, 0);
  nk = bld16(rk, t >= 16 && t < 32 ? 16 * (t - 16) : ll::OOB, 0);
}

// One barrier: every wave's vote (true iff every wave's ok) and, from the io waves, the row's sum of squares (each io
// thread's 4 in order, the wave's xor tree, the 4 io waves in order); every thread (both roles) gets 1 / rms in inv.
template <bool IO>
__device__ __forceinline__ bool vote_rms(Smem& sm, int& ph, bool ok, float q, float eps, float& inv) {
  const int w = threadIdx.x >> 6;
  const bool bad = __ballot(!ok) != 0;
  if (IO) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) q = q + __shfl_xor(q, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    sm.sync.vote[ph][w] = bad;
    if (IO) sm.rq[ph][w - NM / 64] = q;
  }
  __syncthreads();
  int any = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) any |= sm.sync.vote[ph][i];
  inv = 1.0f / sqrtf((((sm.rq[ph][0] + sm.rq[ph][1]) + sm.rq[ph][2]) + sm.rq[ph][3]) / (float)DM + eps);
  ph ^= 1;
  return __builtin_amdgcn_readfirstlane(!any) != 0;
}

// The io waves' own barrier (the projecting waves take no part, so a burst of their loads never holds it up): an
// LDS arrival counter that only grows; the call returns once all four io waves have arrived k times. LDS writes
// before it are visible after it (each wave's writes are done before its arrival). False after `limit` rounds.
__device__ __forceinline__ bool io_bar(Smem& sm, int& k, unsigned limit) {
  k += NM / 64;
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  if ((threadIdx.x & 63) == 0) atomicAdd(&sm.iob, 1);
  for (unsigned s = 0;; ++s) {
    if (__hip_atomic_load(&sm.iob, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= k) break;
    if (s >= limit) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
  return true;
}

// io thread ti: x[4 ti .. 4 ti + 3] += dt(the K-half partials summed in order); returns their sum of squares
__device__ __forceinline__ float add_quarters(Smem& sm, int ti, const float (&pv)[KQ][4]) {
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float o = pv[0][e];
#pragma unroll
    for (int h = 1; h < KQ; ++h) o = o + pv[h][e];
    const uint16_t xv = f2bf(bf2f(sm.x[4 * ti + e]) + bf2f(f2bf(o)));
    sm.x[4 * ti + e] = xv;
    const float v = bf2f(xv);
    q = q + v * v;
  }
  return q;
}
__device__ __forceinline__ float row_sq(const Smem& sm, int ti) {
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float v = bf2f(sm.x[4 * ti + e]);
    q = q + v * v;
  }
  return q;
}
// io wave: poll the K-half partials of columns 4 ti .. 4 ti + 3 (two 16-byte chunks per half)
__device__ __forceinline__ bool poll_quarters(unsigned limit, __amdgpu_buffer_rsrc_t rs, int base, int ti, int probe,
                                              uint32_t tag, float (&pv)[KQ][4]) {
  return ll_poll16_w<2 * KQ>(
      limit, rs, base + 4 * ti, [](int i) { return (i >> 1) * DM + 2 * (i & 1); }, 2 * KQ, probe,
      [](int) { return true; }, tag, [&](int i, uint32_t p0, uint32_t p1) {
        pv[i >> 1][2 * (i & 1)] = __uint_as_float(p0);
        pv[i >> 1][2 * (i & 1) + 1] = __uint_as_float(p1);
      });
}
// projecting wave 0: LL store of a tile's 16 bf16 outputs (thread c < 16 holds column c): 8 words from the even
// threads. The tiles' outputs leave from the projecting waves, which never poll, so no poll waits behind a store.
__device__ __forceinline__ void st_tile(__amdgpu_buffer_rsrc_t rs, int base, int tile, uint16_t v, uint32_t tag) {
  const int t = threadIdx.x;
  const uint32_t nb = (uint32_t)__shfl_down((int)v, 1, 64);
  if (t < 16 && (t & 1) == 0) ll_st8(rs, base + tile * 8 + t / 2, (uint32_t)v | (nb << 16), tag);
}
}  // namespace bb

using namespace bb;

__global__ __launch_bounds__(NT, 1) void backbone_run_kernel(const M3xBackboneRun a) {
  __shared__ Smem sm;
  const int wg = blockIdx.x, tid = threadIdx.x;
  const uint32_t epoch = (uint32_t)a.sync[0];
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(a.xchg, 0, (int)(X_WORDS * 8), 0x00020000);
  const bool gu = wg < NGU;              // a gate|up workgroup
  const bool ow = wg < NOD, dw = !ow;    // an o unit's, else a down unit's workgroup
  const int tq = qkv_tile(wg);           // its q|k|v tile
  const int tu = (wg % NOD) >> 1, kh = wg & 1;  // its o or down unit: 16-column tile, K half
  const int ih = wg & (KV - 1), is = wg / KV;   // its attention item: kv head (= its XCD), split
  // the row's slot and position (the host guarantees 0 <= pos < cap; the clamp keeps every access in the slot)
  const long slot = a.slots[0];
  const int pos = min(max(a.pos[0], 0), a.cap - 1);
  const int S = max(16, (((pos + 1 + SPLITS - 1) / SPLITS) + 15) / 16 * 16);
  const int k0 = is * S, n = max(min(k0 + S, pos + 1) - k0, 0);  // the item's keys k0 .. k0 + n - 1
  const bool own_pos = k0 <= pos && pos < k0 + S;
  const long kvoff = slot * a.sk_s + (long)ih * a.sk_h;
  bool ok = true;
  int vph = 0;

  if (tid == 0) {
    ll::sync_init(sm.sync, a.spin_limit);
    sm.iob = 0;
  }
  if (tid >= NM) {
    const int ti = tid - NM;
    *reinterpret_cast<uint2*>(&sm.x[4 * ti]) = *reinterpret_cast<const uint2*>((const uint16_t*)a.x + 4 * ti);
    if (ti < 32)  // cos and sin at the position, for every layer
      *reinterpret_cast<u16x8*>(&sm.cs[ti >> 4][8 * (ti & 15)]) =
          ld16((const uint16_t*)(ti < 16 ? a.cos : a.sin) + (long)pos * a.s_cos + 8 * (ti & 15));
  }

  if (__builtin_amdgcn_readfirstlane(tid) < NM) {
    // ================= projecting waves: the MFMA tiles and their epilogues, the weights and the split's keys and
    // values in registers ahead of use. Refills (each after its slot's tile is used) go right before the io waves'
    // longest stretches, since a burst of loads holds the issuing wave until the memory system takes it:
    //   after S1: the next layer's q|k|v and q/k norm weights, this layer's gate|up pair and o or down unit;
    //   after S5: the next layer's keys and values, which go to LDS after S6.
    // Registers (per projecting thread, 16 B each): q|k|v 8, the o or down unit 12, one 16-chunk slot shared by
    // the split's keys / values (until S6) and the gate|up pair (S1..S5), the norm weights 2 (no array indexed by a
    // thread-dependent value: that would move it to LDS).
    u16x8 wq[8], wod[NOD_F], ka[KVN], va[KVN], nq, nk;
    {
      const M3xBackboneLayer L = layer_at(a.layer, 0);
      load_kv(ka, va, L, kvoff, a.sk_t, a.cap, k0, n);
      load_nw(nq, nk, L, true);
      load_wt<8>(wq, L.wqkv, tq, DM, 0);
#pragma unroll
      for (int i = 0; i < KVN; ++i) {
        const int c = tid + NM * i, j = c / (HD / 8), d = 8 * (c % (HD / 8));
        *reinterpret_cast<u16x8*>(&sm.kt[j][d]) = ka[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) sm.vt[d + e][j] = va[i].v[e];
      }
      if (tid < 16) *reinterpret_cast<u16x8*>(&sm.nw[0][8 * tid]) = nq;
      else if (tid < 32) *reinterpret_cast<u16x8*>(&sm.nw[1][8 * (tid - 16)]) = nk;
    }
    __syncthreads();  // the set-up's LDS
    float inv = 0.f;
    for (int l = 0; l < a.layers; ++l) {
      const bool nx = l + 1 < a.layers;
      const M3xBackboneLayer L = layer_at(a.layer, l), N = layer_at(a.layer, nx ? l + 1 : l);
      const int par = l & 1;
      const uint32_t t_qkv = (epoch << 12) | (1u + (uint32_t)(STEPS * l));
      const int b_qkv = O_QKV + par * W_QKV, b_o = O_O + par * W_O, b_gu = O_GU + par * W_GU, b_dn = O_DN + par * W_DN;
      // S1
      if (!(ok = vote_rms<false>(sm, vph, true, 0.f, a.eps, inv))) break;
      if (l == 0) __syncthreads();  // the normed row in sm.b
      put_part(sm, 0, mma_row<8>(wq, l == 0 ? sm.b : sm.x));
      __syncthreads();
      {
        uint16_t v = 0;
        if (tid < 16) {
          const float s = get_part(sm, 0, tid);
          v = f2bf(l == 0 ? s : inv * s);  // the folded norm's row scale (the plain weight at layer 0)
        }
        st_tile(rs, b_qkv, tq, v, t_qkv);
      }
      load_wt<8>(wq, N.wqkv, tq, DM, 0, nx);
      load_nw(nq, nk, N, nx);
      load_wt<8>(ka, L.wg, gu ? wg : 0, DM, 0, gu);
      load_wt<8>(va, L.wu, gu ? wg : 0, DM, 0, gu);
      load_od(wod, L, ow, tu, kh);
      // S2, S3: io waves only
      // S4 (o units)
      if (ow) {
        if (!(ok = wg_all(sm.sync, true, vph))) break;
        put_part(sm, 0, mma_row<KO / 32 / 4>(wod, sm.b));
        __syncthreads();
        if (tid < 16) ll_st8(rs, b_o + kh * DM + 16 * tu + tid, __float_as_uint(get_part(sm, 0, tid)), t_qkv + 3);
      }
      // S5: the gate|up pair (a workgroup without one multiplies the zeros its empty loads returned: every path
      // then waits for the same loads); the sm.x reads end before the io waves pass the barrier below
      if (!(ok = vote_rms<false>(sm, vph, true, 0.f, a.eps, inv))) break;
      put_part(sm, 0, mma_row<8>(ka, sm.x));
      put_part(sm, 1, mma_row<8>(va, sm.x));
      if (gu) {
        __syncthreads();
        uint16_t v = 0;
        if (tid < 16) {
          const float gt = rnd<M3X_BF16>(inv * get_part(sm, 0, tid));
          const float u = rnd<M3X_BF16>(inv * get_part(sm, 1, tid));
          v = f2bf(rnd<M3X_BF16>(silu16(gt)) * u);
        }
        st_tile(rs, b_gu, wg, v, t_qkv + 4);
      }
      load_kv(ka, va, N, kvoff, a.sk_t, a.cap, k0, n, nx);
      // S6 (down units)
      if (dw) {
        if (!(ok = wg_all(sm.sync, true, vph))) break;
        put_part(sm, 0, mma_row<NOD_F>(wod, sm.b));
        __syncthreads();
        if (tid < 16) ll_st8(rs, b_dn + kh * DM + 16 * tu + tid, __float_as_uint(get_part(sm, 0, tid)), t_qkv + 5);
      }
      // the next layer's keys (rows), values (transposed) and norm weights into LDS: the io waves finished this
      // layer's attention before the S5 barrier, and start the next one after the next S1 barrier
#pragma unroll
      for (int i = 0; i < KVN; ++i) {
        const int c = tid + NM * i, j = c / (HD / 8), d = 8 * (c % (HD / 8));
        *reinterpret_cast<u16x8*>(&sm.kt[j][d]) = ka[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) sm.vt[d + e][j] = va[i].v[e];
      }
      if (tid < 16) *reinterpret_cast<u16x8*>(&sm.nw[0][8 * tid]) = nq;
      else if (tid < 32) *reinterpret_cast<u16x8*>(&sm.nw[1][8 * (tid - 16)]) = nk;
    }
    if (ok) ok = wg_all(sm.sync, true, vph);  // the last layer's down
  } else {
    // ================= io waves: polls, norms, attention, combine
    const int ti = tid - NM, iw = ti >> 6, lane = ti & 63, l16 = lane & 15, lg = lane >> 4;
    __syncthreads();  // the set-up's LDS
    const unsigned limit = __builtin_amdgcn_readfirstlane(sm.sync.spin);
    const int probe = a.probe;
    const float scale = a.scale;
    int kb = 0;  // io_bar arrivals
    auto stamp = [&](int s) {  // stamp s of layer l at slot 16 l + s (profiling only)
      if (a.prof && ti == 0) a.prof[(long)wg * 512 + s] = __builtin_amdgcn_s_memrealtime();
    };
    for (int l = 0; l < a.layers; ++l) {
      const M3xBackboneLayer L = layer_at(a.layer, l);
      const int par = l & 1;
      const uint32_t s0 = 1u + (uint32_t)(STEPS * l);
      const uint32_t t_qkv = (epoch << 12) | s0, t_part = t_qkv + 1, t_att = t_qkv + 2, t_o = t_qkv + 3,
                     t_gu = t_qkv + 4;
      const int b_qkv = O_QKV + par * W_QKV, b_part = O_PART + par * W_PART, b_att = O_ATT + par * W_ATT,
                b_o = O_O + par * W_O, b_gu = O_GU + par * W_GU;
      bool okc = true;  // polls and io barriers between two votes
      stamp(16 * l + 0);

      // ---- S1: x += the previous layer's down, the row's RMS (the q|k|v tile and its epilogue run in the
      // projecting waves)
      float inv;
      {
        bool okw = true;
        float q;
        if (l > 0) {
          float pv[KQ][4];
          okw = poll_quarters(limit, rs, O_DN + (1 - par) * W_DN, ti, probe, (epoch << 12) | (s0 - 1), pv);
          q = okw ? add_quarters(sm, ti, pv) : 0.f;
        } else {
          q = row_sq(sm, ti);
        }
        if (!(ok = vote_rms<true>(sm, vph, okw, q, a.eps, inv))) break;
      }
      stamp(16 * l + 1);
      if (l == 0) {
        // the input RMSNorm applied to the row (the packed weight of layer 0 is the plain one)
        const uint2 w4 = *reinterpret_cast<const uint2*>((const uint16_t*)a.w_in0 + 4 * ti);
        const uint16_t wv[4] = {(uint16_t)(w4.x & 0xffff), (uint16_t)(w4.x >> 16), (uint16_t)(w4.y & 0xffff),
                                (uint16_t)(w4.y >> 16)};
#pragma unroll
        for (int e = 0; e < 4; ++e) sm.b[4 * ti + e] = f2bf(bf2f(f2bf(bf2f(sm.x[4 * ti + e]) * inv)) * bf2f(wv[e]));
        __syncthreads();
      }
      __syncthreads();  // the projecting waves' partials (their x and sm.b reads end here)

      // ---- S2: attention item (ih, is): keys k0 .. k0 + n - 1 of the slot's kv head ih (io waves only)
      {
        // q heads 2 ih, 2 ih + 1, the key and the value of kv head ih, as projected
        const int part = ti >> 5, c4 = ti & 31;  // 16-byte chunks: q 0..63, k 64..95, v 96..127
        const int col = part < 2 ? 2 * ih * HD + 4 * ti
                                 : (part == 2 ? H * HD + ih * HD : (H + KV) * HD + ih * HD) + 4 * c4;
        okc = ll_poll16_w<1>(
            limit, rs, b_qkv + col / 2, [](int) { return 0; }, 1, probe, [&](int) { return ti < 128; }, t_qkv,
            [&](int, uint32_t p0, uint32_t p1) { *reinterpret_cast<uint2*>(&sm.raw[4 * ti]) = uint2{p0, p1}; });
        okc = io_bar(sm, kb, limit) && okc;
      }
      stamp(16 * l + 3);
      // q/k norm + RoPE: lanes 0-15 q head 2 ih, 16-31 q head 2 ih + 1, 32-47 the key (one DPP row each)
      if (iw == 0) {
        const int g3 = min(lg, 2);
        float xv[8];
        const u16x8 r8 = *reinterpret_cast<const u16x8*>(&sm.raw[g3 * HD + 8 * l16]);
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = bf2f(r8.v[e]);
        const u16x8 wv = *reinterpret_cast<const u16x8*>(&sm.nw[g3 < 2 ? 0 : 1][8 * l16]);
        const u16x8 cv = *reinterpret_cast<const u16x8*>(&sm.cs[0][8 * l16]);
        const u16x8 sv = *reinterpret_cast<const u16x8*>(&sm.cs[1][8 * l16]);
        const u16x8 ov = qk_norm_rope8<HD>(xv, wv, cv, sv, a.eps, l16);
        if (lg < 2) {
          *reinterpret_cast<u16x8*>(&sm.qb[lg][8 * l16]) = ov;
        } else if (lg == 2) {
          *reinterpret_cast<u16x8*>(&sm.kn[8 * l16]) = ov;
        }
      }
      // the new value stands in the tile's column pos - k0 (the tile's own entry there is the cache's stale one)
      if (own_pos && ti < HD) sm.vt[ti][pos - k0] = sm.raw[3 * HD + ti];
      okc = io_bar(sm, kb, limit) && okc;
      stamp(16 * l + 13);
      // the new key and value into the cache, by the item that holds the position
      if (own_pos && ti < 32) {
        const int d = 8 * (ti & 15);
        if (ti < 16) st16((uint16_t*)L.kc + kvoff + (long)pos * a.sk_t + d, *reinterpret_cast<const u16x8*>(&sm.kn[d]));
        else st16((uint16_t*)L.vc + kvoff + (long)pos * a.sk_t + d, *reinterpret_cast<const u16x8*>(&sm.raw[3 * HD + d]));
      }
      {
        // scores on MFMA: io wave w takes key blocks w and w + 4 (16 keys each); A = the two q heads (rows 0, 1),
        // B = the block's keys (the new key at the position); lanes 0-15 end with key l16's two scores
        float sc[2][2];
#pragma unroll
        for (int bs = 0; bs < 2; ++bs) {
          const int b = iw + 4 * bs, j = 16 * b + l16;
          sc[bs][0] = sc[bs][1] = -INFINITY;
          if (16 * b < n) {
            const uint16_t* kp = (k0 + j == pos) ? sm.kn : &sm.kt[j][0];
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < HD / 32; ++kc) {
              const u16x8 qa = l16 < 2 ? *reinterpret_cast<const u16x8*>(&sm.qb[l16 & 1][32 * kc + 8 * lg]) : u16x8{};
              const u16x8 kv8 = *reinterpret_cast<const u16x8*>(&kp[32 * kc + 8 * lg]);
              acc = mfma16x16x32<M3X_BF16>(qa, kv8, acc);
            }
            if (lane < 16 && j < n) {
              sc[bs][0] = acc[0] * scale;
              sc[bs][1] = acc[1] * scale;
            }
          }
        }
        float m0 = fmaxf(sc[0][0], sc[1][0]), m1 = fmaxf(sc[0][1], sc[1][1]);
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          m0 = fmaxf(m0, __shfl_xor(m0, o, 64));
          m1 = fmaxf(m1, __shfl_xor(m1, o, 64));
        }
        if (lane == 0) {
          sm.red[0][2 * iw] = m0;
          sm.red[0][2 * iw + 1] = m1;
        }
        okc = io_bar(sm, kb, limit) && okc;
        const float M0 = fmaxf(fmaxf(sm.red[0][0], sm.red[0][2]), fmaxf(sm.red[0][4], sm.red[0][6]));
        const float M1 = fmaxf(fmaxf(sm.red[0][1], sm.red[0][3]), fmaxf(sm.red[0][5], sm.red[0][7]));
        // probabilities in fp32; the P.V operand carries each as a bf16 pair (hi, lo = what bf16 left), so P.V is
        // the fp32 product to ~16 bits; every block 0..7 is written (zeros past the split's keys)
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int bs = 0; bs < 2; ++bs) {
          const int j = 16 * (iw + 4 * bs) + l16;
          const bool live = lane < 16 && j < n;
          const float p0 = live ? expf(sc[bs][0] - M0) : 0.f, p1 = live ? expf(sc[bs][1] - M1) : 0.f;
          if (lane < 16) {
            const uint16_t h0 = f2bf(p0), h1 = f2bf(p1);
            sm.pb[0][j] = h0;
            sm.pb[1][j] = h1;
            sm.pb[2][j] = f2bf(p0 - bf2f(h0));
            sm.pb[3][j] = f2bf(p1 - bf2f(h1));
          }
          s0 = s0 + p0;
          s1 = s1 + p1;
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          s0 = s0 + __shfl_xor(s0, o, 64);
          s1 = s1 + __shfl_xor(s1, o, 64);
        }
        if (lane == 0) {
          sm.red[1][2 * iw] = s0;
          sm.red[1][2 * iw + 1] = s1;
        }
        okc = io_bar(sm, kb, limit) && okc;
        stamp(16 * l + 15);
        // P.V on MFMA: io wave w takes dimensions 16 w .. and 16 (w + 4) ..; A = P's four rows, B = the values'
        // transposed tile; lanes 0-15 end with dimension l16's sums: rows 0 + 2 for head 0, 1 + 3 for head 1
        const int w0 = b_part + wg * PW;
        const int nk = (n + 31) & ~31;
#pragma unroll
        for (int ds = 0; ds < 2; ++ds) {
          const int db = iw + 4 * ds;
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
          for (int kc = 0; kc < nk; kc += 32) {
            const u16x8 pa = l16 < 4 ? *reinterpret_cast<const u16x8*>(&sm.pb[l16 & 3][kc + 8 * lg]) : u16x8{};
            const u16x8 vb = *reinterpret_cast<const u16x8*>(&sm.vt[16 * db + l16][kc + 8 * lg]);
            acc = mfma16x16x32<M3X_BF16>(pa, vb, acc);
          }
          if (lane < 16) {
            ll_st8(rs, w0 + 2 + 16 * db + l16, __float_as_uint(acc[0] + acc[2]), t_part);
            ll_st8(rs, w0 + (HD + 2) + 2 + 16 * db + l16, __float_as_uint(acc[1] + acc[3]), t_part);
          }
        }
        if (ti < 2) {
          const float M = ti == 0 ? M0 : M1;
          const float Ls = ti == 0 ? ((sm.red[1][0] + sm.red[1][2]) + sm.red[1][4]) + sm.red[1][6]
                                   : ((sm.red[1][1] + sm.red[1][3]) + sm.red[1][5]) + sm.red[1][7];
          ll_st8(rs, w0 + ti * (HD + 2), __float_as_uint(n > 0 ? M : -INFINITY), t_part);
          ll_st8(rs, w0 + ti * (HD + 2) + 1, __float_as_uint(n > 0 ? Ls : 0.f), t_part);
        }
      }
      stamp(16 * l + 4);

      // ---- S3: combine of q head 2 hk + gq (workgroups 0..15, on kv head hk's XCD): its 32 partials
      if (wg < H) {
        // io thread t reads split t / 8, words t % 8 + 8 i of the q head's 130 (i < 17)
        const int hk = wg & (KV - 1), gq = wg / KV, sp = ti >> 3, k8 = ti & 7;
        constexpr int NW = (HD + 2 + 7) / 8;
        okc = ll_poll8_w<NW>(
                  limit, rs, b_part + (hk + KV * sp) * PW + gq * (HD + 2) + k8, [](int i) { return 8 * i; }, NW,
                  probe, [&](int i) { return k8 + 8 * i < HD + 2; }, t_part,
                  [&](int i, uint32_t p) { sm.comb[sp][k8 + 8 * i] = __uint_as_float(p); }) &&
              okc;
        okc = io_bar(sm, kb, limit) && okc;
        stamp(16 * l + 5);
        // the splits' weights exp(m_s - M) (M the largest m_s; empty splits weigh 0)
        if (ti < SPLITS) {
          float M = sm.comb[ti][0];
#pragma unroll
          for (int o = 1; o < SPLITS; o <<= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
          sm.cw[ti] = sm.comb[ti][1] > 0.f ? expf(sm.comb[ti][0] - M) : 0.f;
        }
        okc = io_bar(sm, kb, limit) && okc;
        if (ti < HD) {
          // four chains over the splits s = 4 i + r (a fixed order), so the LDS reads pipeline
          float Lr[4] = {0.f, 0.f, 0.f, 0.f}, orr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < SPLITS; ++s) {
            const float w = sm.cw[s];
            Lr[s & 3] = Lr[s & 3] + sm.comb[s][1] * w;
            orr[s & 3] = orr[s & 3] + sm.comb[s][2 + ti] * w;
          }
          const float Ls = (Lr[0] + Lr[1]) + (Lr[2] + Lr[3]), o = (orr[0] + orr[1]) + (orr[2] + orr[3]);
          const uint16_t v = f2bf(o / Ls);
          const uint32_t nb = (uint32_t)__shfl_down((int)v, 1, 64);
          if ((ti & 1) == 0) ll_st8(rs, b_att + ((2 * hk + gq) * HD + ti) / 2, (uint32_t)v | (nb << 16), t_att);
        }
        stamp(16 * l + 6);
      }

      // ---- S4 (o units, workgroups 0..127): tile tu's K half kh, the half's 8 heads of the attention output
      if (ow) {
        okc = ll_poll16_w<1>(
                  limit, rs, b_att + kh * (KO / 2) + 2 * ti, [](int) { return 0; }, 1, probe, [](int) { return true; },
                  t_att, [&](int, uint32_t p0, uint32_t p1) { *reinterpret_cast<uint2*>(&sm.b[4 * ti]) = uint2{p0, p1}; }) &&
              okc;
        if (!(ok = wg_all(sm.sync, okc, vph))) break;
        okc = true;
        stamp(16 * l + 7);
        __syncthreads();  // the projecting waves' partials
        stamp(16 * l + 8);
      }

      // ---- S5: x += o, the row's RMS (gate|up tile pair and SwiGLU in the projecting waves)
      {
        float pv[KQ][4];
        const bool okw = poll_quarters(limit, rs, b_o, ti, probe, t_o, pv);
        const float q = okw ? add_quarters(sm, ti, pv) : 0.f;
        if (!(ok = vote_rms<true>(sm, vph, okw && okc, q, a.eps, inv))) break;
      }
      stamp(16 * l + 9);
      if (gu) {
        __syncthreads();  // the projecting waves' partials (their sm.x reads end here)
        stamp(16 * l + 10);
      }

      // ---- S6 (down units, workgroups 128..255): tile tu's K half kh, the half's 1536 gate|up outputs
      if (dw) {
        const bool okw = ll_poll16_w<2>(
            limit, rs, b_gu + kh * (KD / 2) + 2 * ti, [](int i) { return 2 * NT / 2 * i; }, 2, probe,
            [&](int i) { return i == 0 || ti < (KD / 4 - NM); }, t_gu,
            [&](int i, uint32_t p0, uint32_t p1) { *reinterpret_cast<uint2*>(&sm.b[4 * ti + 4 * NM * i]) = uint2{p0, p1}; });
        if (!(ok = wg_all(sm.sync, okw, vph))) break;
        stamp(16 * l + 11);
        __syncthreads();  // the projecting waves' partials (their sm.b reads end here)
        stamp(16 * l + 12);
      }
    }
    // ---- the last layer's x += down, and workgroup 0 stores the row
    if (ok) {
      const int lp = a.layers - 1;
      float pv[KQ][4];
      const bool okw = poll_quarters(limit, rs, O_DN + (lp & 1) * W_DN, ti, probe,
                                     (epoch << 12) | (uint32_t)(STEPS * lp + STEPS), pv);
      if (okw) add_quarters(sm, ti, pv);
      ok = wg_all(sm.sync, okw, vph);
      if (ok && wg == 0) {
        *reinterpret_cast<uint2*>((uint16_t*)a.h_out + 4 * ti) = *reinterpret_cast<const uint2*>(&sm.x[4 * ti]);
        if (iw == 0) {
          // the final RMSNorm in the add+norm kernels' order: lane t sums groups t and t + 64 (8 elements each,
          // left to right), the two partials add, then the wave's fold-in-half tree; y = dt(dt(x / rms) * w)
          float v[2][8], p[2];
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            const u16x8 x8 = *reinterpret_cast<const u16x8*>(&sm.x[8 * (lane + 64 * m)]);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[m][e] = bf2f(x8.v[e]);
            p[m] = v[m][0] * v[m][0];
#pragma unroll
            for (int e = 1; e < 8; ++e) p[m] = p[m] + v[m][e] * v[m][e];
          }
          const float sum = __builtin_bit_cast(
              float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fold_half_sum<64>(p[0] + p[1]))));
          const float sc = 1.0f / sqrtf(sum / (float)DM + a.eps);
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            const u16x8 w8 = ld16((const uint16_t*)a.w_fin + 8 * (lane + 64 * m));
            u16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o.v[e] = f2bf(rnd<M3X_BF16>(v[m][e] * sc) * bf2f(w8.v[e]));
            st16((uint16_t*)a.y_out + 8 * (lane + 64 * m), o);
          }
        }
      }
    }
  }

  // ---- the run's end: failures are recorded, and the last workgroup out advances the epoch
  if (!ok && tid == 0) atomicOr(&a.sync[2], 1);
  if (wg == 0 && tid == 0) a.lengths[slot] += a.real[0];  // as the launch path, whether or not the run failed
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
  if (!a.layer || !a.x || !a.h_out || !a.slots || !a.pos || !a.cos || !a.sin || !a.w_in0 || !a.xchg || !a.sync ||
      !a.w_fin || !a.y_out || !a.lengths || !a.real)
    return M3X_ENULL;
  if ((a.sk_s | a.sk_h | a.sk_t | a.s_cos) & 7) return M3X_EINVAL;
  if (!bb_resident_ok()) return M3X_EUNSUPPORTED;
  hipLaunchKernelGGL(backbone_run_kernel, dim3(NWG), dim3(NT), 0, (hipStream_t)stream, a);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}
