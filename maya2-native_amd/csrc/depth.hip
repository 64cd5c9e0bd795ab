// The depth frame over a run of levels that continue one weight group, as ONE persistent kernel
// (serve/fast_depth.py:143-203: the incremental levels, :150-155, with their sampling, :191-198).
//
// A level is a chain of ~22 dependent steps: per trunk layer q|k|v, attention, o, gate|up (+SwiGLU or GELU) and
// down, then the codebook head and the sampler. Launched one kernel per step, each step pays a launch and a cold
// memory round trip (~3.5 us per step at one seat, ~107 us per level). Here one workgroup per CU stays resident
// for the whole run:
//   - the first 192 workgroups project the residual stream (q|k|v, gate|up and head tiles): each keeps that stream,
//     and its norm, in LDS across the layers and the codebooks; each of them also owns up to one (seat, head)
//     pair, whose depth K/V history it keeps in LDS across the codebooks;
//   - the last 64 workgroups own the o and down tiles; the down tile's input (16 rows x the FFN width) lands in
//     their LDS, which holds nothing else;
//   - a step's weights are loaded before the step waits for its input, so the weight stream overlaps the chain;
//   - steps hand their outputs over through global memory in LL form: an 8-byte word carries 4 bytes of payload
//     (two 16-bit values, one code, ...) and a 4-byte tag, written and read with device-scope (sc1) accesses that
//     stay coherent across the XCDs' L2s. A consumer polls exactly the words it needs until each carries the
//     step's tag (the launch's epoch << 12 | the step's number). A word is its own flag, so no barrier, fence or
//     cache flush is needed, and a word read before its producer wrote it is simply read again.
// Every wait is bounded: a workgroup whose input does not arrive within the run's spin limit (SPIN_LIMIT polls
// unless the caller sets a smaller one) sets the error word and skips the rest of the run, so the grid always
// drains; m3x_depth_run_void, launched after the run, then overwrites the run's codes with -1 so every consumer
// of the codes sees the failure. The grid is at most one workgroup per CU (LDS use
// forces one per CU), so every workgroup is resident and every wait can be satisfied.
//
// Numerics follow the launch path step for step: norms in the add+norm kernels' reduction order (bit-identical
// rows), GEMM tiles accumulate in fp32 over four K slices summed in slice order with one rounding, the gated
// epilogues round where the reference rounds (serve/fast_backbone.py:201-202, serve/fast_depth.py:123,186),
// attention in fp32 with one rounding of the output, the sampler is m3x_sample.h's.
#include "m3x_ll.h"
#include "m3x_sample.h"

namespace dk {
constexpr int NT = 256;     // threads per workgroup
constexpr int RB = 16;      // seats per run (one MFMA row block)
constexpr int DM = 1024;    // trunk width
constexpr int XS = DM + 8;  // LDS row stride of the residual and its norm: a 16-byte offset per row
constexpr int NPOS = 32;    // positions of a frame
constexpr int MAXL = 4;     // trunk layers
constexpr int VMAX = 2048;  // codebook size
constexpr int FMAX = 3072;  // FFN width
constexpr int HDMAX = 128;  // head dim

// exchange buffers, in 8-byte words; two copies of each, alternating by layer (by level for head and codes)
constexpr long W_QKV = (long)RB * 3 * DM / 2, W_ATT = (long)RB * DM / 2, W_GU = (long)RB * FMAX / 2,
               W_LOG = (long)RB * VMAX / 2, W_CODE = RB;
constexpr long O_QKV = 0, O_ATT = O_QKV + 2 * W_QKV, O_O = O_ATT + 2 * W_ATT, O_GU = O_O + 2 * W_ATT,
               O_DN = O_GU + 2 * W_GU, O_LOG = O_DN + 2 * W_ATT, O_CODE = O_LOG + 2 * W_LOG,
               O_DUMMY = O_CODE + 2 * W_CODE, X_WORDS = O_DUMMY + 8;
}  // namespace dk

// Arguments of one run (a plain struct of pointers and sizes; the host fills it from m3x_depth_run's caller).
struct M3xDepthRun {
  int B, L0, L1, layers, H, hd, F, V, act, norm_kind, dtype, nwg;
  float inv_temp;
  int top_k, greedy;
  float eps1[dk::MAXL], eps2[dk::MAXL], eps_f;
  const void* n1w[dk::MAXL];
  const void* n1b[dk::MAXL];
  const void* n2w[dk::MAXL];
  const void* n2b[dk::MAXL];
  const void* fw;
  const void* fb;
  const void* wqkv[dk::MAXL];
  const void* wo[dk::MAXL];
  const void* wg[dk::MAXL];
  const void* wu[dk::MAXL];
  const void* wd[dk::MAXL];
  const void* heads[31];
  const void* embed;  // [31][V][DM]: prefix row of level L+1 = embed[L][code]
  const void* cross;  // [B][layers * DM] speaker constants, or null
  long ld_cross;
  void* prefix;       // row b, position p at prefix + b * ld_prefix + p * DM
  long ld_prefix;
  int32_t* codes;
  long ld_codes;
  const float* u;     // u[b * ld_u + L - 1]
  long ld_u;
  const void* kd[dk::MAXL];  // [B][H][32][hd] per layer: the group's K/V at positions < L0
  const void* vd[dk::MAXL];
  long kv_sb, kv_sh;
  uint64_t* xchg;     // dk::X_WORDS words, zeroed once
  int32_t* sync;      // [0] epoch, [1] workgroups done, [2] error
  void* logits_out;   // optional [31][B][V] copy of every level's head output (tests)
  uint64_t* prof;     // optional [nwg][2048] real-time stamps of each workgroup's steps (profiling)
  int probe;          // a poll with more chunks per thread than this waits on one chunk first
  unsigned spin_limit;  // polling rounds before a wait gives up (0: SPIN_LIMIT)
};

namespace dk {
using ll::u32x2;
using ll::u32x4;
using ll::SC1;
using ll::SPIN_LIMIT;
using ll::ll_poll16;
using ll::ll_poll8;
using ll::ll_st16;
using ll::ll_st8;
using ll::ro_rsrc;
using ll::bld16;

constexpr int NXM = 3 * DM / 16;  // workgroups that keep the residual stream (one q|k|v tile each)
constexpr int NOD = DM / 16;      // workgroups of the o and down tiles
constexpr int AS = FMAX + 8;      // LDS row stride of the down tile's input

struct SmemXM {
  uint16_t x[RB][XS];                 // the residual stream of every seat
  union {
    uint16_t y[RB][XS];               // its norm: the B operand of the q|k|v, gate|up and head tiles
    SampleSmemT<VMAX> smp;            // the sampler's candidates (the head's input is dead by then)
  } u;
  uint16_t kv[MAXL][2][NPOS][HDMAX];  // this workgroup's (seat, head) K and V history
};
struct Smem {
  union {
    SmemXM m;
    uint16_t act[RB][AS];             // o/down workgroups: the down tile's input
  };
  float part[2][4][256];              // per-wave partial tiles (gate, up)
  float qv[HDMAX];
  float pr[NPOS];
  int codes[RB];
  int seat_codes[NPOS];               // a sampler workgroup's codes of its seat, for the prefix rows at the end
  ll::Sync sync;                      // the polls' votes and spin limit
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// ---- norms of the resident stream. A row's 1024 elements are 128 groups of 8 (group g = columns 8 g .. 8 g + 7);
// the add+norm kernels sum each group left to right and fold the 128 partials in half (p[g] + p[g + s] for
// s = 64, 32, ..., 1). Here a row has one wave: lane t holds the groups t and t + 64, folds them (s = 64), and
// the wave folds the rest with fold_half_sum<64> (lane 0 ends with the tree's sum), so the rows are those kernels'
// bits. Wave w takes the rows w, w + 4, ... below B, interleaved.
__device__ __forceinline__ float row_fold(float p0, float p1) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fold_half_sum<64>(p0 + p1))));
}
__device__ __forceinline__ int norm_group(int m) { return (threadIdx.x & 63) + 64 * m; }

// the affine terms of a norm, as norm_rows' threads use them (loaded before a step waits for its input; the kind
// is a compile-time constant of the kernel, so an RMS norm holds no bias registers)
template <int NK>
struct NormW {
  u16x8 w[2], b[NK == M3X_NORM_LAYER ? 2 : 1];
};
template <int NK>
__device__ __forceinline__ void load_norm(NormW<NK>& n, const void* w, const void* b) {
  const __amdgpu_buffer_rsrc_t rw = ro_rsrc(w);
#pragma unroll
  for (int m = 0; m < 2; ++m) n.w[m] = bld16(rw, 16 * norm_group(m), 0);
  if constexpr (NK == M3X_NORM_LAYER) {
    const __amdgpu_buffer_rsrc_t rb = ro_rsrc(b);
#pragma unroll
    for (int m = 0; m < 2; ++m) n.b[m] = bld16(rb, 16 * norm_group(m), 0);
  }
}

// y[r] = norm(x[r]) for the rows r < B (x, y in LDS; the affine terms preloaded): wave w takes rows w + 4 k, k < R
template <int DT, int NK, int R>
__device__ __forceinline__ void norm_rows_r(Smem& sm, int B, const NormW<NK>& nw, float eps) {
  const int w = threadIdx.x >> 6, g0 = norm_group(0), g1 = norm_group(1);
  float v[R][2][8];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const u16x8 x0 = *reinterpret_cast<const u16x8*>(&sm.m.x[w + 4 * k][8 * g0]);
    const u16x8 x1 = *reinterpret_cast<const u16x8*>(&sm.m.x[w + 4 * k][8 * g1]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[k][0][e] = E<DT>::to_f(x0.v[e]);
      v[k][1][e] = E<DT>::to_f(x1.v[e]);
    }
  }
  float sc[R];  // LayerNorm: the standard deviation; RMSNorm: 1 / rms
  if constexpr (NK == M3X_NORM_LAYER) {
    float mean[R];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      float p[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        p[m] = v[k][m][0];
#pragma unroll
        for (int e = 1; e < 8; ++e) p[m] = p[m] + v[k][m][e];
      }
      mean[k] = row_fold(p[0], p[1]) / (float)DM;
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      float p[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][m][e] = v[k][m][e] - mean[k];
        p[m] = v[k][m][0] * v[k][m][0];
#pragma unroll
        for (int e = 1; e < 8; ++e) p[m] = p[m] + v[k][m][e] * v[k][m][e];
      }
      sc[k] = sqrtf(row_fold(p[0], p[1]) / (float)DM + eps);
    }
  } else {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      float p[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        p[m] = v[k][m][0] * v[k][m][0];
#pragma unroll
        for (int e = 1; e < 8; ++e) p[m] = p[m] + v[k][m][e] * v[k][m][e];
      }
      sc[k] = 1.0f / sqrtf(row_fold(p[0], p[1]) / (float)DM + eps);
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int r = w + 4 * k;
    if (r < B) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        u16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (NK == M3X_NORM_LAYER)
            o.v[e] = E<DT>::from_f(v[k][m][e] / sc[k] * E<DT>::to_f(nw.w[m].v[e]) + E<DT>::to_f(nw.b[m].v[e]));
          else
            o.v[e] = E<DT>::from_f(rnd<DT>(v[k][m][e] * sc[k]) * E<DT>::to_f(nw.w[m].v[e]));
        }
        *reinterpret_cast<u16x8*>(&sm.m.u.y[r][8 * (m ? g1 : g0)]) = o;
      }
    }
  }
  __syncthreads();
}
template <int DT, int NK>
__device__ __forceinline__ void norm_rows(Smem& sm, int B, const NormW<NK>& nw, float eps) {
  if (B <= 4) norm_rows_r<DT, NK, 1>(sm, B, nw, eps);
  else if (B <= 8) norm_rows_r<DT, NK, 2>(sm, B, nw, eps);
  else if (B <= 12) norm_rows_r<DT, NK, 3>(sm, B, nw, eps);
  else norm_rows_r<DT, NK, 4>(sm, B, nw, eps);
}

// x[r] = dt(dt(x[r] + a[r]) + c[r]) for r < B with a from an LL buffer [RB][DM] (c optional, global [B][ld_c]):
// thread t takes columns 4 t .. 4 t + 3 of every row, so a row is one 16-byte chunk per thread
template <int DT>
__device__ __forceinline__ bool add_rows(Smem& sm, int& vph, __amdgpu_buffer_rsrc_t rs, int base, uint32_t tag,
                                         int B, const uint16_t* c, long ld_c, int probe) {
  const int t = threadIdx.x;
  uint2 cv[RB];
  if (c) {
    const __amdgpu_buffer_rsrc_t rc = ro_rsrc(c);
#pragma unroll
    for (int i = 0; i < RB; ++i)
      if (i < B) {
        const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(rc, 8 * t, 2 * i * (int)ld_c, 0);
        cv[i] = uint2{q.x, q.y};
      }
  }
  const bool ok = ll_poll16<RB>(
      sm.sync, vph, rs, base + 2 * t, [](int i) { return i * (DM / 2); }, B, probe, [](int) { return true; }, tag,
      [&](int i, uint32_t p0, uint32_t p1) {
        uint16_t* xp = &sm.m.x[i][4 * t];
        const uint16_t av[4] = {(uint16_t)(p0 & 0xffff), (uint16_t)(p0 >> 16), (uint16_t)(p1 & 0xffff),
                                (uint16_t)(p1 >> 16)};
        const uint16_t cc[4] = {(uint16_t)(cv[i].x & 0xffff), (uint16_t)(cv[i].x >> 16), (uint16_t)(cv[i].y & 0xffff),
                                (uint16_t)(cv[i].y >> 16)};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = rnd<DT>(E<DT>::to_f(xp[e]) + E<DT>::to_f(av[e]));
          if (c) v = rnd<DT>(v + E<DT>::to_f(cc[e]));
          xp[e] = E<DT>::from_f(v);
        }
      });
  __syncthreads();
  return ok;
}

// rows [RB][K] of an LL buffer into sm.act (rows >= B stay as they are), in two halves of RB / 2 rows so that at
// most half the chunks are in flight beside the down tile's prefetched weights: chunk c = tid + NT i of half h
// holds columns 4 (c % (K / 4)) .. + 3 of row h RB / 2 + c / (K / 4), at word 2 c of the half; a half's first
// (its live rows) K / 4 chunks are live, and a half with no live row is skipped
template <int K>
__device__ __forceinline__ bool stage_act(Smem& sm, int& vph, __amdgpu_buffer_rsrc_t rs, int base, uint32_t tag,
                                          int B, int probe) {
  constexpr int CPR = K / 4, HR = RB / 2, N = HR * CPR / NT;
  static_assert(HR * CPR % NT == 0, "chunks per thread");
  bool ok = true;
  for (int h = 0; h < 2 && ok; ++h) {
    const int rows = min(max(B - h * HR, 0), HR), nlive = rows * CPR;
    if (rows == 0) break;
    ok = ll_poll16<N>(
        sm.sync, vph, rs, base + h * HR * CPR * 2 + 2 * (int)threadIdx.x, [](int i) { return 2 * NT * i; },
        (nlive + NT - 1) / NT, probe, [&](int i) { return (int)threadIdx.x + NT * i < nlive; }, tag,
        [&](int i, uint32_t p0, uint32_t p1) {
          const int cc = threadIdx.x + NT * i;
          *reinterpret_cast<uint2*>(&sm.act[h * HR + cc / CPR][4 * (cc % CPR)]) = uint2{p0, p1};
        });
  }
  __syncthreads();
  return ok;
}

// ---- GEMM tiles: 16 output columns x 16 seat rows; wave w reduces K slice w of 4 (NF fragments of 32)
template <int NF>
struct WTile {
  u16x8 f[NF];
};
template <int NF>
__device__ __forceinline__ void load_tile(WTile<NF>& t, const uint16_t* w, int tile, int K) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t r = ro_rsrc(w);
  const int s0 = (tile * 16 * K + wave * NF * 512) * 2;  // uniform: scalar offset
#pragma unroll
  for (int f = 0; f < NF; ++f) t.f[f] = bld16(r, 16 * lane, s0 + f * 1024);
}
// W tile x y^T, y the residual's norm in LDS
template <int DT, int NF>
__device__ __forceinline__ f32x4_t mma_y(const WTile<NF>& t, const Smem& sm) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = lane & 15, kg = lane >> 4;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int k = (wave * NF + f) * 32 + 8 * kg;
    acc = mfma16x16x32<DT>(t.f[f], *reinterpret_cast<const u16x8*>(&sm.m.u.y[row][k]), acc);
  }
  return acc;
}
// W tile x act^T, act staged in LDS
template <int DT, int NF>
__device__ __forceinline__ f32x4_t mma_act(const WTile<NF>& t, const Smem& sm) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = lane & 15, kg = lane >> 4;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int k = (wave * NF + f) * 32 + 8 * kg;
    acc = mfma16x16x32<DT>(t.f[f], *reinterpret_cast<const u16x8*>(&sm.act[row][k]), acc);
  }
  return acc;
}

// Sum the four waves' partial tiles (slice order, one rounding) and store the 16 x 16 tile to an LL buffer
// row-major [RB][N] at column tile `tile`: EPI 0 plain, 1 SwiGLU (acc = gate, acc2 = up), 2 GELU. dbg (optional):
// a plain row-major copy [B][ld_dbg].
template <int DT, int EPI>
__device__ __forceinline__ void finish_tile(Smem& sm, f32x4_t acc, f32x4_t acc2, __amdgpu_buffer_rsrc_t rs, int base,
                                            int N, int tile, uint32_t tag, int B, uint16_t* dbg, long ld_dbg) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sm.part[0][wave][(4 * kg + i) * 16 + row] = acc[i];
    if constexpr (EPI == 1) sm.part[1][wave][(4 * kg + i) * 16 + row] = acc2[i];
  }
  __syncthreads();
  if (wave == 0 && row < B) {
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = (4 * kg + i) * 16 + row;
      float v = rnd<DT>(((sm.part[0][0][idx] + sm.part[0][1][idx]) + sm.part[0][2][idx]) + sm.part[0][3][idx]);
      if constexpr (EPI == 1) {
        const float g = v;
        const float uu =
            rnd<DT>(((sm.part[1][0][idx] + sm.part[1][1][idx]) + sm.part[1][2][idx]) + sm.part[1][3][idx]);
        v = rnd<DT>(silu16(g)) * uu;
      } else if constexpr (EPI == 2) {
        v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
      }
      o[i] = E<DT>::from_f(v);
    }
    const int col = 16 * tile + 4 * kg;
    ll_st16(rs, base + row * (N / 2) + col / 2, pack2(o[0], o[1]), pack2(o[2], o[3]), tag);
    if (dbg) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dbg[(long)row * ld_dbg + col + i] = o[i];
    }
  }
  __syncthreads();
}
// The draw of one seat's code from its head row (x = logits / temp as the launch path's sampler forms them, one
// element i = tid + 256 e per thread): a separate function so that the selection's registers do not add to the
// rest of the run's. Every thread calls it; the code is returned in every thread.
__device__ __attribute__((noinline)) int draw_code(SampleSmemT<VMAX>& sp, int* code_slot, float x0, float x1,
                                                   float x2, float x3, float x4, float x5, float x6, float x7,
                                                   int top_k, int greedy, float u) {
  const float xv[VMAX / NT] = {x0, x1, x2, x3, x4, x5, x6, x7};
  topk_select<VMAX / NT>(xv, VMAX, top_k, sp);
  if (threadIdx.x < 64) {
    int code = cand_index(sp.cand[0]);
    if (!greedy) {
      const int cp = pick(sp, sp.nkeep, u, -1);
      if (cp >= 0) code = cp;
    }
    if (threadIdx.x == 0) *code_slot = code;
  }
  __syncthreads();
  return *code_slot;
}
}  // namespace dk

using namespace dk;

template <int DT, int ACT, int HD>
__global__ __launch_bounds__(NT, 1) void depth_run_kernel(const M3xDepthRun a) {
  __shared__ Smem sm;
  // the norm kind goes with the activation: RMSNorm in the SwiGLU trunks, LayerNorm in the GELU ones
  constexpr int NK = ACT == 1 ? M3X_NORM_RMS : M3X_NORM_LAYER;
  const int wg = blockIdx.x, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int B = a.B, H = a.H, layers = a.layers;
  const uint32_t epoch = (uint32_t)a.sync[0];
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(a.xchg, 0, (int)(X_WORDS * 8), 0x00020000);
  // roles: workgroup w < NXM keeps the residual stream and owns q|k|v tile w, gate|up tile w (if any), head tile
  // w (if any) and the (seat, head) pair NXM - 1 - w (if any); workgroup NXM + t owns o tile t and down tile t
  const int U_GU = a.F / 16, U_HEAD = a.V / 16;
  const bool xm = wg < NXM;
  const bool do_gu = xm && wg < U_GU, do_head = xm && wg < U_HEAD;
  const int u_od = wg - NXM;
  const bool do_od = u_od >= 0 && u_od < NOD;
  const int pair = NXM - 1 - wg;
  const bool has_pair = xm && pair < B * H;
  const int pb = has_pair ? pair / H : 0, ph = has_pair ? pair % H : 0;
  const int steps_per_level = 5 * layers + 2;
  const float scale = 1.0f / sqrtf((float)HD);
  bool ok = true;
  int vph = 0;  // wg_all's vote buffer
  // stamp k of (level li, layer l): slot li * 64 + l * 12 + k; the level's head and sampler at li * 64 + 48 + k
  auto stamp = [&](int slot) {
    if (a.prof && tid == 0) a.prof[(long)wg * 2048 + slot] = __builtin_amdgcn_s_memrealtime();
  };

  // ---- set-up: zeroed LDS rows, the residual at L0 from the prefix, the pair's K/V history
  if (tid == 0) ll::sync_init(sm.sync, a.spin_limit);
  if (xm) {
    for (int i = tid; i < RB * XS / 8; i += NT) {
      reinterpret_cast<u16x8*>(&sm.m.x[0][0])[i] = u16x8{};
      reinterpret_cast<u16x8*>(&sm.m.u.y[0][0])[i] = u16x8{};
    }
  } else {
    for (int i = tid; i < RB * AS / 8; i += NT) reinterpret_cast<u16x8*>(&sm.act[0][0])[i] = u16x8{};
  }
  __syncthreads();
  if (xm) {
    const uint16_t* pre = (const uint16_t*)a.prefix;
    for (int i = tid; i < B * DM / 8; i += NT) {
      const int r = i / (DM / 8), c = 8 * (i % (DM / 8));
      *reinterpret_cast<u16x8*>(&sm.m.x[r][c]) = ld16(pre + (long)r * a.ld_prefix + (long)a.L0 * DM + c);
    }
  }
  if (has_pair) {
    for (int l = 0; l < layers; ++l) {
      const uint16_t* kb = (const uint16_t*)a.kd[l] + (long)pb * a.kv_sb + (long)ph * a.kv_sh;
      const uint16_t* vb = (const uint16_t*)a.vd[l] + (long)pb * a.kv_sb + (long)ph * a.kv_sh;
      for (int i = tid; i < a.L0 * HD / 8; i += NT) {
        const int p = i / (HD / 8), c = 8 * (i % (HD / 8));
        *reinterpret_cast<u16x8*>(&sm.m.kv[l][0][p][c]) = ld16(kb + (long)p * HD + c);
        *reinterpret_cast<u16x8*>(&sm.m.kv[l][1][p][c]) = ld16(vb + (long)p * HD + c);
      }
    }
  }
  __syncthreads();

  for (int L = a.L0; L < a.L1 && ok; ++L) {
    const int li = L - a.L0;
    const uint32_t lvl_seq = 1u + (uint32_t)(li * steps_per_level);
    const int lpar = li & 1;
    for (int l = 0; l < layers && ok; ++l) {
      const int par = (li * layers + l) & 1;
      const uint32_t s0 = lvl_seq + 5u * l;  // steps q|k|v .. down of this layer: s0 .. s0 + 4
      const uint32_t t_qkv = (epoch << 12) | s0, t_att = t_qkv + 1, t_o = t_qkv + 2, t_gu = t_qkv + 3,
                     t_dn = t_qkv + 4;
      const int b_qkv = O_QKV + par * W_QKV, b_att = O_ATT + par * W_ATT, b_o = O_O + par * W_ATT,
                b_gu = O_GU + par * W_GU, b_dn = O_DN + par * W_ATT;
      // ---- step 1: the layer's input (the level's prefix row, or x + f + c of the previous layer) -> norm -> q|k|v
      if (xm) {
        WTile<8> wt;
        load_tile<8>(wt, (const uint16_t*)a.wqkv[l], wg, DM);
        NormW<NK> nw;
        load_norm<NK>(nw, a.n1w[l], a.n1b[l]);
        if (l == 0 && L > a.L0) {
          // the previous level's codes; this level's input rows are their prefix rows
          const uint32_t t_code = (epoch << 12) | (lvl_seq - 1);
          const int b_code = O_CODE + (1 - lpar) * W_CODE;
          ok = ll_poll8<1>(
              sm.sync, vph, rs, b_code + tid, [](int) { return 0; }, 1, a.probe, [&](int) { return tid < B; }, t_code,
              [&](int, uint32_t p) { sm.codes[tid] = (int)p; });
          stamp(li * 64 + 52);
          __syncthreads();
          const __amdgpu_buffer_rsrc_t re = ro_rsrc((const uint16_t*)a.embed + (long)(L - 1) * a.V * DM);
          for (int i = tid; i < B * DM / 8; i += NT) {
            const int r = i / (DM / 8), c = 8 * (i % (DM / 8));
            const int code = min(max(sm.codes[r], 0), a.V - 1);
            *reinterpret_cast<u16x8*>(&sm.m.x[r][c]) = bld16(re, 2 * (code * DM + c), 0);
          }
          __syncthreads();
        } else if (l > 0) {
          const int b_prev = O_DN + ((li * layers + l - 1) & 1) * W_ATT;
          const uint16_t* c = a.cross ? (const uint16_t*)a.cross + (long)(l - 1) * DM : nullptr;
          ok = add_rows<DT>(sm, vph, rs, b_prev, t_qkv - 1, B, c, a.ld_cross, a.probe);
        }
        stamp(li * 64 + l * 12 + 0);
        norm_rows<DT, NK>(sm, B, nw, a.eps1[l]);
        stamp(li * 64 + l * 12 + 10);
        if (ok) finish_tile<DT, 0>(sm, mma_y<DT, 8>(wt, sm), f32x4_t{}, rs, b_qkv, 3 * DM, wg, t_qkv, B, nullptr, 0);
        stamp(li * 64 + l * 12 + 1);
      }
      // ---- step 2: attention of this workgroup's (seat, head) at position L over the group's keys 0..L
      if (ok && has_pair) {
        constexpr int per = HD / 4;  // 16-byte chunks of each of q, k and v of one head
        const int part = tid / per, c = tid % per;
        const int w0 = b_qkv + pb * (3 * DM / 2) + (part * DM + ph * HD) / 2 + 2 * c;
        ok = ll_poll16<1>(sm.sync, vph, rs, w0, [](int) { return 0; }, 1, a.probe, [&](int) { return tid < 3 * per; }, t_qkv,
                          [&](int, uint32_t p0, uint32_t p1) {
                            const uint16_t v4[4] = {(uint16_t)(p0 & 0xffff), (uint16_t)(p0 >> 16),
                                                    (uint16_t)(p1 & 0xffff), (uint16_t)(p1 >> 16)};
                            if (part == 0) {
#pragma unroll
                              for (int e = 0; e < 4; ++e) sm.qv[4 * c + e] = E<DT>::to_f(v4[e]);
                            } else {
#pragma unroll
                              for (int e = 0; e < 4; ++e) sm.m.kv[l][part - 1][L][4 * c + e] = v4[e];
                            }
                          });
        stamp(li * 64 + l * 12 + 2);
        // scores: thread t takes key j = t / 8 and dims (t % 8) HD / 8 .. + HD / 8 - 1, summed over the 8 lanes
        {
          constexpr int DS = HD / 8;
          const int j = tid >> 3, s8 = tid & 7;
          float d = 0.f;
          if (j <= L) {
#pragma unroll
            for (int g = 0; g < DS / 8; ++g) {
              const u16x8 k8 = *reinterpret_cast<const u16x8*>(&sm.m.kv[l][0][j][s8 * DS + 8 * g]);
#pragma unroll
              for (int e = 0; e < 8; ++e) d = fmaf(sm.qv[s8 * DS + 8 * g + e], E<DT>::to_f(k8.v[e]), d);
            }
          }
          d += __shfl_xor(d, 1, 64);
          d += __shfl_xor(d, 2, 64);
          d += __shfl_xor(d, 4, 64);
          if (s8 == 0) sm.pr[j] = j <= L ? d * scale : -INFINITY;
        }
        __syncthreads();
        {
          // the softmax's max and sum, in every wave (lane j < NPOS holds key j's score)
          const float sj = lane < NPOS ? sm.pr[lane] : -INFINITY;
          float m = sj;
          for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
          float sum = lane <= L ? expf(sj - m) : 0.f;
          for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
          // P V: thread t takes dims 4 (t % DG) .. + 3 over the keys j = t / DG + PG i, then the PG partial
          // rows are summed, first across the lanes of a wave, then across the four waves
          constexpr int DG = HD / 4, PG = NT / DG;
          const int dg = tid % DG;
          float o4[4] = {0.f, 0.f, 0.f, 0.f};
          for (int j = tid / DG; j <= L; j += PG) {
            const float pj = expf(sm.pr[j] - m) / sum;
            const uint2 vv = *reinterpret_cast<const uint2*>(&sm.m.kv[l][1][j][4 * dg]);
            const uint16_t v4[4] = {(uint16_t)(vv.x & 0xffff), (uint16_t)(vv.x >> 16), (uint16_t)(vv.y & 0xffff),
                                    (uint16_t)(vv.y >> 16)};
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = fmaf(pj, E<DT>::to_f(v4[e]), o4[e]);
          }
#pragma unroll
          for (int o = DG; o < 64; o <<= 1)
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] += __shfl_xor(o4[e], o, 64);
          if (lane < DG) {
#pragma unroll
            for (int e = 0; e < 4; ++e) sm.part[0][wave][4 * lane + e] = o4[e];
          }
          __syncthreads();
          if (tid < DG) {
            float r4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int i = 4 * tid + e;
              r4[e] = ((sm.part[0][0][i] + sm.part[0][1][i]) + sm.part[0][2][i]) + sm.part[0][3][i];
            }
            ll_st16(rs, b_att + pb * (DM / 2) + (ph * HD + 4 * tid) / 2,
                    pack2(E<DT>::from_f(r4[0]), E<DT>::from_f(r4[1])),
                    pack2(E<DT>::from_f(r4[2]), E<DT>::from_f(r4[3])), t_att);
          }
          __syncthreads();
        }
        stamp(li * 64 + l * 12 + 3);
      }
      // ---- step 3: o projection of the attention rows
      if (ok && do_od) {
        WTile<8> wt;
        load_tile<8>(wt, (const uint16_t*)a.wo[l], u_od, DM);
        ok = stage_act<DM>(sm, vph, rs, b_att, t_att, B, a.probe);
        stamp(li * 64 + l * 12 + 4);
        if (ok) finish_tile<DT, 0>(sm, mma_act<DT, 8>(wt, sm), f32x4_t{}, rs, b_o, DM, u_od, t_o, B, nullptr, 0);
        stamp(li * 64 + l * 12 + 5);
      }
      // ---- step 4: x += o -> norm -> gate|up with the activation
      if (ok && xm) {
        WTile<8> wg_, wu_;
        if (do_gu) {
          load_tile<8>(wg_, (const uint16_t*)a.wg[l], wg, DM);
          if constexpr (ACT == 1) load_tile<8>(wu_, (const uint16_t*)a.wu[l], wg, DM);
        }
        NormW<NK> nw;
        load_norm<NK>(nw, a.n2w[l], a.n2b[l]);
        ok = add_rows<DT>(sm, vph, rs, b_o, t_o, B, nullptr, 0, a.probe);
        stamp(li * 64 + l * 12 + 6);
        norm_rows<DT, NK>(sm, B, nw, a.eps2[l]);
        stamp(li * 64 + l * 12 + 11);
        if (ok && do_gu) {
          if constexpr (ACT == 1)
            finish_tile<DT, 1>(sm, mma_y<DT, 8>(wg_, sm), mma_y<DT, 8>(wu_, sm), rs, b_gu, a.F, wg, t_gu, B, nullptr,
                               0);
          else
            finish_tile<DT, 2>(sm, mma_y<DT, 8>(wg_, sm), f32x4_t{}, rs, b_gu, a.F, wg, t_gu, B, nullptr, 0);
        }
        stamp(li * 64 + l * 12 + 7);
      }
      // ---- step 5: down projection of the activation (staged in LDS)
      if (ok && do_od) {
        f32x4_t acc;
        if constexpr (ACT == 1) {
          WTile<22> wt;
          load_tile<22>(wt, (const uint16_t*)a.wd[l], u_od, 2816);
          ok = stage_act<2816>(sm, vph, rs, b_gu, t_gu, B, a.probe);
          stamp(li * 64 + l * 12 + 8);
          acc = mma_act<DT, 22>(wt, sm);
        } else {
          WTile<24> wt;
          load_tile<24>(wt, (const uint16_t*)a.wd[l], u_od, 3072);
          ok = stage_act<3072>(sm, vph, rs, b_gu, t_gu, B, a.probe);
          acc = mma_act<DT, 24>(wt, sm);
        }
        if (ok) finish_tile<DT, 0>(sm, acc, f32x4_t{}, rs, b_dn, DM, u_od, t_dn, B, nullptr, 0);
        stamp(li * 64 + l * 12 + 9);
      }
    }
    if (!ok) break;
    // ---- the codebook head of level L over the final norm of x + f + c
    const uint32_t t_log = (epoch << 12) | (lvl_seq + 5u * layers), t_code = t_log + 1;
    const int b_log = O_LOG + lpar * W_LOG, b_code = O_CODE + lpar * W_CODE;
    if (xm) {
      WTile<8> wt;
      if (do_head) load_tile<8>(wt, (const uint16_t*)a.heads[L - 1], wg, DM);
      NormW<NK> nw;
      load_norm<NK>(nw, a.fw, a.fb);
      const int b_prev = O_DN + ((li * layers + layers - 1) & 1) * W_ATT;
      const uint16_t* c = a.cross ? (const uint16_t*)a.cross + (long)(layers - 1) * DM : nullptr;
      ok = add_rows<DT>(sm, vph, rs, b_prev, t_log - 1, B, c, a.ld_cross, a.probe);
      stamp(li * 64 + 48);
      norm_rows<DT, NK>(sm, B, nw, a.eps_f);
      if (ok && do_head) {
        uint16_t* dbg = a.logits_out ? (uint16_t*)a.logits_out + (long)(L - 1) * B * a.V : nullptr;
        finish_tile<DT, 0>(sm, mma_y<DT, 8>(wt, sm), f32x4_t{}, rs, b_log, a.V, wg, t_log, B, dbg, a.V);
      }
      stamp(li * 64 + 49);
    }
    // ---- sampling of seat wg's code (the launch path's sampler, on the LL copy of the head row)
    if (ok && wg < B) {
      const int r = wg;
      constexpr int NE = VMAX / NT;
      const float ur = a.greedy ? 0.f : a.u[(long)r * a.ld_u + L - 1];
      float xv[NE];
      // one workgroup per seat polls its row: every word each round (no probe word first), which costs little
      // traffic here and saves the round trip after the probe (0.6-0.9 us a level at one seat)
      ok = ll_poll8<NE>(sm.sync, vph, rs, b_log + r * (VMAX / 2) + tid / 2, [](int e) { return NT / 2 * e; }, NE, NE,
                        [&](int) { return true; }, t_log, [&](int e, uint32_t p) {
                          const uint16_t h16 = (uint16_t)((tid & 1) ? (p >> 16) : (p & 0xffff));
                          xv[e] = E<DT>::to_f(h16) * a.inv_temp;
                        });
      stamp(li * 64 + 50);
      const int code = draw_code(sm.m.u.smp, &sm.codes[0], xv[0], xv[1], xv[2], xv[3], xv[4], xv[5],
                                 xv[6], xv[7], a.top_k, a.greedy, ur);
      if (tid == 0) {
        a.codes[(long)r * a.ld_codes + L] = code;
        ll_st8(rs, b_code + r, (uint32_t)code, t_code);
        sm.seat_codes[L] = code;
      }
      stamp(li * 64 + 51);
      __syncthreads();
    }
  }

  // ---- the prefix rows of the levels sampled here (prefix position L + 1 = embed[L][code of level L]), for a
  // later group start that recomputes the whole prefix; written once at the end, off the levels' chain
  if (ok && wg < B) {
    const int nl = min(a.L1, NPOS - 1) - a.L0;
    for (int i = tid; i < nl * (DM / 8); i += NT) {
      const int L = a.L0 + i / (DM / 8), c = 8 * (i % (DM / 8));
      const long cc = min(max(sm.seat_codes[L], 0), VMAX - 1);
      st16((uint16_t*)a.prefix + (long)wg * a.ld_prefix + (long)(L + 1) * DM + c,
           ld16((const uint16_t*)a.embed + ((long)L * VMAX + cc) * DM + c));
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

// After a run: when its error word is set, codes[b][L0 .. L1-1] = -1 for b < B (a failed run's codes are void; the
// code consumers clamp codes, so -1 reads a valid row, and the host checks see the sentinel). One workgroup.
__global__ __launch_bounds__(256) void depth_run_void_kernel(const int32_t* __restrict__ sync, int32_t* codes,
                                                             long ld_codes, int B, int L0, int L1) {
  if (sync[2] == 0) return;
  const int n = L1 - L0;
  for (int i = threadIdx.x; i < B * n; i += blockDim.x) codes[(long)(i / n) * ld_codes + L0 + i % n] = -1;
}

M3X_API size_t m3x_depth_run_xchg_bytes(void) { return (size_t)X_WORDS * 8; }
M3X_API size_t m3x_depth_run_args_bytes(void) { return sizeof(M3xDepthRun); }

// Every workgroup of a run waits on others, so the whole grid must be resident at once: the device's CUs times
// the kernel instance's workgroups per CU must cover nwg (checked once per device and instance).
template <int DT, int ACT, int HD>
static int resident_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, depth_run_kernel<DT, ACT, HD>, NT, 0) != hipSuccess) return 0;
  return n;
}
static bool resident_grid_ok(const M3xDepthRun& a) {
  constexpr int MAXDEV = 64;
  static int cus[MAXDEV], per[MAXDEV][4];  // 0: not queried yet; -1: query failed
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return false;
  if (cus[dev] == 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? n : -1;
  }
  const int inst = (a.dtype == M3X_F16 ? 2 : 0) + (a.act == 1 ? 1 : 0);
  if (per[dev][inst] == 0) {
    int n = 0;
    if (inst == 0) n = resident_per_cu<M3X_BF16, 1, 128>();
    else if (inst == 1) n = resident_per_cu<M3X_BF16, 2, 64>();
    else if (inst == 2) n = resident_per_cu<M3X_F16, 1, 128>();
    else n = resident_per_cu<M3X_F16, 2, 64>();
    per[dev][inst] = n > 0 ? n : -1;
  }
  return cus[dev] > 0 && per[dev][inst] > 0 && (long)cus[dev] * per[dev][inst] >= a.nwg;
}

M3X_API int m3x_depth_run_void(const int32_t* sync, int32_t* codes, long ld_codes, int B, int L0, int L1,
                               void* stream) {
  if (!sync || !codes) return M3X_ENULL;
  if (B <= 0 || L0 < 0 || L1 <= L0 || ld_codes < L1) return M3X_EINVAL;
  hipLaunchKernelGGL(depth_run_void_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, sync, codes, ld_codes, B,
                     L0, L1);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

M3X_API int m3x_depth_run(const M3xDepthRun* args, void* stream) {
  if (!args) return M3X_ENULL;
  const M3xDepthRun& a = *args;
  if (a.B <= 0 || a.B > RB || a.L0 < 2 || a.L1 > NPOS || a.L0 >= a.L1 || a.layers <= 0 || a.layers > MAXL)
    return M3X_EINVAL;
  if (a.H * a.hd != DM || (a.hd != 64 && a.hd != 128) || a.V != VMAX || a.top_k <= 0) return M3X_EUNSUPPORTED;
  if (!((a.act == 0 && a.F == 2816 && a.norm_kind == M3X_NORM_RMS) ||
        (a.act == 1 && a.F == 3072 && a.norm_kind == M3X_NORM_LAYER)))
    return M3X_EUNSUPPORTED;
  if (a.nwg != NXM + NOD || a.B * a.H > NXM) return M3X_EINVAL;
  if (!resident_grid_ok(a)) return M3X_EUNSUPPORTED;
  if (!a.xchg || !a.sync || !a.embed || !a.prefix || !a.codes || (!a.greedy && !a.u) || !a.fw) return M3X_ENULL;
  if (a.norm_kind == M3X_NORM_LAYER && !a.fb) return M3X_ENULL;
  for (int l = 0; l < a.layers; ++l) {
    if (!a.wqkv[l] || !a.wo[l] || !a.wg[l] || !a.wd[l] || !a.n1w[l] || !a.n2w[l] || !a.kd[l] || !a.vd[l])
      return M3X_ENULL;
    if (a.act == 0 && !a.wu[l]) return M3X_ENULL;
    if (a.norm_kind == M3X_NORM_LAYER && (!a.n1b[l] || !a.n2b[l])) return M3X_ENULL;
  }
  for (int L = a.L0; L < a.L1; ++L)
    if (!a.heads[L - 1]) return M3X_ENULL;
  hipStream_t st = (hipStream_t)stream;
#define M3X_DR(DTT, ACTT, HDD) \
  hipLaunchKernelGGL((depth_run_kernel<DTT, ACTT, HDD>), dim3(a.nwg), dim3(NT), 0, st, a)
  // ACT template: 1 = SwiGLU pair (act 0 in the host's numbering), 2 = GELU
  if (a.dtype == M3X_BF16 && a.act == 0 && a.hd == 128) M3X_DR(M3X_BF16, 1, 128);
  else if (a.dtype == M3X_BF16 && a.act == 1 && a.hd == 64) M3X_DR(M3X_BF16, 2, 64);
  else if (a.dtype == M3X_F16 && a.act == 0 && a.hd == 128) M3X_DR(M3X_F16, 1, 128);
  else if (a.dtype == M3X_F16 && a.act == 1 && a.hd == 64) M3X_DR(M3X_F16, 2, 64);
  else return M3X_EUNSUPPORTED;
#undef M3X_DR
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}
