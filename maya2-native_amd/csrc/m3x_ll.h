// LL handovers between the resident workgroups of a persistent kernel (one workgroup per CU, every workgroup
// resident at once). An 8-byte word carries 4 bytes of payload and a 4-byte tag (the launch's epoch << 12 | the step),
// written and read with device-scope (sc1) accesses that stay coherent across the XCDs' L2s. A consumer polls exactly
// the words it needs until each carries the step's tag: a word is its own flag, so no barrier, fence or cache flush
// is needed, and a word read before its producer wrote it is simply read again. Every wait is bounded by the run's
// spin limit, so a workgroup whose input never arrives gives up and the grid still drains.
#pragma once
#include "m3x_common.h"

namespace ll {
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr unsigned SPIN_LIMIT = 1u << 19;
constexpr int SC1 = 16;  // cache-policy bit of a device-scope access (gfx950 SC1)

// per-workgroup LDS state of the polls: wg_all's per-wave votes (alternating buffers, up to 16 waves) and the run's
// spin limit; sync_init (thread 0, before the first barrier) sets the limit and clears every vote slot, so slots of
// waves the workgroup does not have read as "no failure"
struct Sync {
  int vote[2][16];
  unsigned spin;
};
__device__ __forceinline__ void sync_init(Sync& sy, unsigned spin_limit) {
  sy.spin = spin_limit ? spin_limit : SPIN_LIMIT;
#pragma unroll
  for (int i = 0; i < 16; ++i) sy.vote[0][i] = sy.vote[1][i] = 0;
}

// true in every thread iff v is true in every thread: one barrier; the two vote buffers alternate, so a wave that
// runs ahead into the next call writes the other buffer while a slower one still reads this one
__device__ __forceinline__ bool wg_all(Sync& sy, bool v, int& phase) {
  const bool any_false = __ballot(!v) != 0;
  if ((threadIdx.x & 63) == 0) sy.vote[phase][threadIdx.x >> 6] = any_false;
  __syncthreads();
  int any = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) any |= sy.vote[phase][w];
  const int r = !any;
  phase ^= 1;
  return __builtin_amdgcn_readfirstlane(r) != 0;
}

__device__ __forceinline__ u32x4 ll_ld16(__amdgpu_buffer_rsrc_t r, int word) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, word * 8, 0, SC1);
}
__device__ __forceinline__ u32x2 ll_ld8(__amdgpu_buffer_rsrc_t r, int word) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, word * 8, 0, SC1);
}
__device__ __forceinline__ void ll_st16(__amdgpu_buffer_rsrc_t r, int word, uint32_t p0, uint32_t p1, uint32_t tag) {
  const u32x4 v = {p0, tag, p1, tag};
  __builtin_amdgcn_raw_buffer_store_b128(v, r, word * 8, 0, SC1);
}
__device__ __forceinline__ void ll_st8(__amdgpu_buffer_rsrc_t r, int word, uint32_t p, uint32_t tag) {
  const u32x2 v = {p, tag};
  __builtin_amdgcn_raw_buffer_store_b64(v, r, word * 8, 0, SC1);
}

// Read-only tensors through buffer resources: the base stays in scalar registers and a load takes one 32-bit
// offset register, so loop-invariant addressing does not pin 64-bit vector address pairs for the whole run.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ro_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ u16x8 bld16(__amdgpu_buffer_rsrc_t r, int voff_bytes, int soff_bytes) {
  return __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff_bytes, soff_bytes, 0));
}

// Polling. A consumer reads exactly the words it needs until each carries the step's tag. Each wave polls its own
// threads' chunks, with no workgroup barrier per round; the workgroup meets once at the end (which also makes the
// sinks' LDS writes visible). A compiler-only memory clobber in every polling round keeps identical polls from
// being merged or hoisted out of the loop (the loads stay device-scope, sc1).
constexpr int OOB = 1 << 30;  // a byte offset past every exchange buffer: such a load returns zeros, no traffic
constexpr int VOL = SC1;
#define M3X_POLL_CLOBBER() asm volatile("" ::: "memory")

// One 16-byte chunk per lane (live lanes at byte offset `off`) until both words of every live lane of the wave
// carry `tag` (a lane that has its chunk polls out of bounds). The chunk's value lands in `out`; false after
// `limit` rounds.
__device__ __forceinline__ bool wave_poll1(__amdgpu_buffer_rsrc_t r, int off, bool live, uint32_t tag, u32x4& out,
                                           unsigned limit) {
  bool got = !live;
  for (unsigned it = 0; it < limit; ++it) {
    M3X_POLL_CLOBBER();
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, got ? OOB : off, 0, VOL);
    if (!got && a.y == tag && a.w == tag) {
      out = a;
      got = true;
    }
    if (__builtin_amdgcn_ballot_w64(!got) == 0) return true;
  }
  return false;
}
// the same for one 8-byte word per lane (payload in out.x)
__device__ __forceinline__ bool wave_poll1w(__amdgpu_buffer_rsrc_t r, int off, bool live, uint32_t tag, u32x2& out,
                                            unsigned limit) {
  bool got = !live;
  for (unsigned it = 0; it < limit; ++it) {
    M3X_POLL_CLOBBER();
    const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(r, got ? OOB : off, 0, VOL);
    if (!got && a.y == tag) {
      out = a;
      got = true;
    }
    if (__builtin_amdgcn_ballot_w64(!got) == 0) return true;
  }
  return false;
}

// This thread's chunks i < nit (16 bytes, two words each; nit uniform across the wave, at most N), handing each
// live chunk's two payloads to sink(i, p0, p1) once. Chunk i sits at word base + U(i), base per thread and U(i) a
// constant, so the loads take one address register and constant offsets. With more than `probe` chunks per thread,
// chunk 0 is polled first (a probe: one chunk per thread while the producers still run, which then mostly finds the
// rest already there); rounds read the chunks still missing, skipping chunks i >= nit by uniform branches and
// pushing arrived ones out of bounds. Wave-level: false (in every lane) if the wave gave up after `limit` rounds.
template <int N, class U, class Live, class Sink>
__device__ __forceinline__ bool ll_poll16_w(unsigned limit, __amdgpu_buffer_rsrc_t r, int base, U uoff, int nit,
                                            int probe, Live live, uint32_t tag, Sink sink) {
  static_assert(N <= 64, "chunks per thread");
  uint64_t pending = 0;
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (i < nit && live(i)) pending |= 1ull << i;
  bool ok = true;
  if (nit > probe) {
    const bool l0 = pending & 1ull;
    u32x4 v0;
    ok = wave_poll1(r, base * 8 + uoff(0) * 8, l0, tag, v0, limit);
    if (ok && l0) {
      sink(0, v0.x, v0.z);
      pending &= ~1ull;
    }
  }
  for (unsigned it = 0; ok; ++it) {
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (it >= limit) {
      ok = false;
      break;
    }
    M3X_POLL_CLOBBER();
    u32x4 v[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (i < nit)
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, base * 8 + (((pending >> i) & 1) ? 0 : OOB), uoff(i) * 8, VOL);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i < nit && ((pending >> i) & 1) && v[i].y == tag && v[i].w == tag) {
        sink(i, v[i].x, v[i].z);
        pending &= ~(1ull << i);
      }
    }
  }
  return ok;
}
// the same for single words (8-byte loads); sink(i, payload)
template <int N, class U, class Live, class Sink>
__device__ __forceinline__ bool ll_poll8_w(unsigned limit, __amdgpu_buffer_rsrc_t r, int base, U uoff, int nit,
                                           int probe, Live live, uint32_t tag, Sink sink) {
  static_assert(N <= 32, "words per thread");
  uint32_t pending = 0;
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (i < nit && live(i)) pending |= 1u << i;
  bool ok = true;
  if (nit > probe) {
    const bool l0 = pending & 1u;
    u32x2 v0;
    ok = wave_poll1w(r, base * 8 + uoff(0) * 8, l0, tag, v0, limit);
    if (ok && l0) {
      sink(0, v0.x);
      pending &= ~1u;
    }
  }
  for (unsigned it = 0; ok; ++it) {
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (it >= limit) {
      ok = false;
      break;
    }
    M3X_POLL_CLOBBER();
    u32x2 v[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (i < nit)
        v[i] = __builtin_amdgcn_raw_buffer_load_b64(r, base * 8 + (((pending >> i) & 1) ? 0 : OOB), uoff(i) * 8, VOL);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i < nit && ((pending >> i) & 1) && v[i].y == tag) {
        sink(i, v[i].x);
        pending &= ~(1u << i);
      }
    }
  }
  return ok;
}

// Workgroup-collective forms (every thread calls them): the wave-level poll, then one vote over the workgroup
// (which also makes the sinks' LDS writes visible); false if any wave gave up after the run's spin limit (sy.spin).
template <int N, class U, class Live, class Sink>
__device__ __forceinline__ bool ll_poll16(Sync& sy, int& vph, __amdgpu_buffer_rsrc_t r, int base, U uoff, int nit,
                                          int probe, Live live, uint32_t tag, Sink sink) {
  const unsigned limit = __builtin_amdgcn_readfirstlane(sy.spin);
  return wg_all(sy, ll_poll16_w<N>(limit, r, base, uoff, nit, probe, live, tag, sink), vph);
}
template <int N, class U, class Live, class Sink>
__device__ __forceinline__ bool ll_poll8(Sync& sy, int& vph, __amdgpu_buffer_rsrc_t r, int base, U uoff, int nit,
                                         int probe, Live live, uint32_t tag, Sink sink) {
  const unsigned limit = __builtin_amdgcn_readfirstlane(sy.spin);
  return wg_all(sy, ll_poll8_w<N>(limit, r, base, uoff, nit, probe, live, tag, sink), vph);
}

}  // namespace ll
