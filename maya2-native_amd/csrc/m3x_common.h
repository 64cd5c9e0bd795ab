// Shared device helpers for the m3x kernels (gfx950 / CDNA4, wave64).
//
// Everything here is compiled with -ffp-contract=off: a float expression means exactly the IEEE operations
// written, so the kernels that must be bit-exact against the CPU restatement (add+RMSNorm, q/k-norm+RoPE,
// the samplers) can spell their rounding order out. Fused multiply-adds are written as fmaf() where wanted.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define M3X_API extern "C" __attribute__((visibility("default")))

// Status codes returned by every entry point (0 = launched).
enum {
  M3X_OK = 0,
  M3X_EINVAL = -1,      // bad shape, stride, size or alignment
  M3X_ENULL = -2,       // a required pointer is null
  M3X_EWORKSPACE = -3,  // workspace too small
  M3X_ELAUNCH = -4,     // hipGetLastError() reported a launch failure
  M3X_EUNSUPPORTED = -5 // a shape/dtype combination no kernel here implements
};

enum { M3X_BF16 = 0, M3X_F16 = 1, M3X_F32 = 2 };

#define M3X_CHECK_LAUNCH()                                  \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return M3X_ELAUNCH; \
  } while (0)

// ------------------------------------------------------------------ 16-bit float storage
// Storage is uint16_t for both bf16 and fp16; the conversions below are the only way values enter or
// leave fp32, so both the kernels and the C oracle round identically (round-to-nearest-even).
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// gfx950's v_cvt_pk_bf16_f32 (two values per instruction, round-to-nearest-even): identical to the oracle's
// integer rounding for every non-NaN input; a NaN stays a NaN (its payload bits may differ).
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Element-type traits: DT = M3X_BF16 or M3X_F16 (16-bit storage); M3X_F32 below.
template <int DT> struct E;
template <> struct E<M3X_BF16> {
  static __device__ __forceinline__ float to_f(uint16_t v) { return bf2f(v); }
  static __device__ __forceinline__ uint16_t from_f(float f) { return f2bf(f); }
};
template <> struct E<M3X_F16> {
  static __device__ __forceinline__ float to_f(uint16_t v) { return h2f(v); }
  static __device__ __forceinline__ uint16_t from_f(float f) { return f2h(f); }
};

// fp32 storage (the fp32 compute paths): conversions are the identity, so every rnd<M3X_F32> is a no-op and a
// kernel instantiated for it computes the same fp32 expression without intermediate roundings.
template <> struct E<M3X_F32> {
  static __device__ __forceinline__ float to_f(float v) { return v; }
  static __device__ __forceinline__ float from_f(float f) { return f; }
};

// round a float through the storage type
template <int DT> __device__ __forceinline__ float rnd(float f) { return E<DT>::to_f(E<DT>::from_f(f)); }

// storage element of DT: uint16_t bit patterns for bf16 / fp16, float for fp32
template <int DT> struct Store { using T = uint16_t; };
template <> struct Store<M3X_F32> { using T = float; };
template <int DT> using Elt = typename Store<DT>::T;

// ------------------------------------------------------------------ 16-byte vectors
struct __align__(16) u16x8 { uint16_t v[8]; };
__device__ __forceinline__ u16x8 ld16(const uint16_t* p) {
  uint4 r = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(u16x8, r);
}
// Streaming read (non-temporal hint): for data read once per pass, such as the KV cache. A read-only stream
// with the hint runs at ~7.0 TB/s on MI355X against ~6.3 TB/s with plain loads.
__device__ __forceinline__ u16x8 ld16_nt(const uint16_t* p) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t r = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return __builtin_bit_cast(u16x8, r);
}
__device__ __forceinline__ void st16(uint16_t* p, const u16x8& x) {
  *reinterpret_cast<uint4*>(p) = __builtin_bit_cast(uint4, x);
}

// Eight consecutive elements of storage type DT: one 16-byte vector for 16-bit types, two for fp32. Kernels that
// move rows in groups of 8 elements use V8 / ldv / stv and so serve every dtype with one body; for 16-bit types
// they are exactly u16x8 / ld16 / st16.
struct __align__(16) f32x8 { float v[8]; };
template <int DT> struct V8T { using T = u16x8; };
template <> struct V8T<M3X_F32> { using T = f32x8; };
template <int DT> using V8 = typename V8T<DT>::T;
template <int DT> __device__ __forceinline__ V8<DT> ldv(const Elt<DT>* p) {
  if constexpr (DT == M3X_F32) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0];
    const uint4 b = reinterpret_cast<const uint4*>(p)[1];
    f32x8 r;
    r.v[0] = __uint_as_float(a.x), r.v[1] = __uint_as_float(a.y), r.v[2] = __uint_as_float(a.z);
    r.v[3] = __uint_as_float(a.w), r.v[4] = __uint_as_float(b.x), r.v[5] = __uint_as_float(b.y);
    r.v[6] = __uint_as_float(b.z), r.v[7] = __uint_as_float(b.w);
    return r;
  } else {
    return ld16(p);
  }
}
template <int DT> __device__ __forceinline__ void stv(Elt<DT>* p, const V8<DT>& x) {
  if constexpr (DT == M3X_F32) {
    reinterpret_cast<uint4*>(p)[0] = make_uint4(__float_as_uint(x.v[0]), __float_as_uint(x.v[1]),
                                                __float_as_uint(x.v[2]), __float_as_uint(x.v[3]));
    reinterpret_cast<uint4*>(p)[1] = make_uint4(__float_as_uint(x.v[4]), __float_as_uint(x.v[5]),
                                                __float_as_uint(x.v[6]), __float_as_uint(x.v[7]));
  } else {
    st16(p, x);
  }
}
template <int DT> __device__ __forceinline__ V8<DT> zero_v8() {
  V8<DT> z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z.v[e] = 0;
  return z;
}

// silu(g) = g / (1 + e^-g) of the 16-bit SwiGLU epilogues, whose result is rounded to bf16 / fp16 next: the hardware
// exp2 (v_exp_f32 of g * log2 e) and reciprocal (v_rcp_f32), each within about an ulp of fp32, instead of the
// library expf and the IEEE quotient (~30 instructions per element). g -> -inf gives -0, g -> +inf gives g.
__device__ __forceinline__ float silu16(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * g));
}

// ------------------------------------------------------------------ exp for the samplers
// Cody-Waite argument reduction (W. J. Cody and W. Waite, "Software Manual for the Elementary Functions",
// 1980): x = n*ln2 + r with ln2 split into a 16-bit-exact high part and a low part, |r| <= ln2/2, then a
// degree-7 Taylor polynomial for e^r by Horner's rule with fused multiply-adds, scaled by 2^n.
// Only called with x <= 0 (a logit minus the row maximum); x < -87 returns 0 so the result is never a
// subnormal (the weight of such a candidate is below 2^-125 of the top one). The C oracle carries the same
// function; both compile with contraction off, so they agree bit for bit.
__device__ __forceinline__ float m3x_expf(float x) {
  if (x < -87.0f) return 0.0f;
  const float L2E = 1.44269504088896341f;
  const float LN2_HI = 0.693145751953125f;         // 0x3f317200: 15 significant bits, n*LN2_HI exact for |n| < 512
  const float LN2_LO = 1.42860682030941723212e-6f; // ln2 - LN2_HI
  float n = rintf(x * L2E);
  float r = fmaf(-n, LN2_HI, x);
  r = fmaf(-n, LN2_LO, r);
  float p = 1.98412698412698413e-4f;  // 1/7!
  p = fmaf(p, r, 1.38888888888888889e-3f);  // 1/6!
  p = fmaf(p, r, 8.33333333333333333e-3f);  // 1/5!
  p = fmaf(p, r, 4.16666666666666667e-2f);  // 1/4!
  p = fmaf(p, r, 1.66666666666666667e-1f);  // 1/3!
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

// ------------------------------------------------------------------ wave reductions (wave64)
__device__ __forceinline__ float wave_sum_xor(float v, int width) {
  for (int s = width >> 1; s > 0; s >>= 1) v = v + __shfl_xor(v, s, 64);
  return v;
}
__device__ __forceinline__ float wave_max_xor(float v, int width) {
  for (int s = width >> 1; s > 0; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
  return v;
}

// Lane-group reductions without the LDS crossbar. Within a row of 16 lanes, DPP moves (quad_perm [1,0,3,2] and
// [2,3,0,1], then the half-row and row mirrors; once lanes of a quad hold equal values, a mirror pairs each lane
// with a lane of the partner quad or half). Across rows, gfx950's v_permlane16_swap / v_permlane32_swap applied
// to (v, v) return the two halves of each swapped pair, so their sum is v[i] + v[i ^ 16] (resp. ^ 32) in every
// lane, in the same order in both lanes of the pair.
template <int CTRL> __device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// DPP controls: row_shl:n (lane i reads lane i + n of its row of 16), row_ror:n (lane i reads lane (i + n) % 16),
// row_newbcast:n (every lane of a row reads lane n of the row)
constexpr int DPP_ROW_SHL(int n) { return 0x100 + n; }
constexpr int DPP_ROW_ROR(int n) { return 0x120 + n; }
constexpr int DPP_ROW_NEWBCAST(int n) { return 0x150 + n; }
// Fold-in-half within aligned groups of W lanes (W <= 64, a power of two): after it, the first lane of each group
// holds sum_g p[g] combined as p[g] + p[g + s] for s = W/2, ..., 1 (permlane swaps for s = 32, 16; DPP row
// shifts below). The other lanes hold partial or undefined values.
template <int W> __device__ __forceinline__ float fold_half_sum(float p) {
  if constexpr (W == 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(p), __float_as_uint(p), false, false);
    p = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (W >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(p), false, false);
    p = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (W >= 16) p = p + dppf<DPP_ROW_SHL(8)>(p);
  if constexpr (W >= 8) p = p + dppf<DPP_ROW_SHL(4)>(p);
  if constexpr (W >= 4) p = p + dppf<DPP_ROW_SHL(2)>(p);
  if constexpr (W >= 2) p = p + dppf<DPP_ROW_SHL(1)>(p);
  return p;
}
// every lane gets the sum (max) over its aligned group of W lanes, W in {8, 16}
template <int W> __device__ __forceinline__ float group_sum(float v) {
  static_assert(W == 8 || W == 16, "group width");
  v = v + dppf<0xB1>(v);
  v = v + dppf<0x4E>(v);
  v = v + dppf<0x141>(v);
  if constexpr (W == 16) v = v + dppf<0x140>(v);
  return v;
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// sum (max) over the lanes that share lane % W, W in {8, 16}: rows of W lanes combined
template <int W> __device__ __forceinline__ float across_sum(float v) {
  if constexpr (W == 8) v = v + dppf<0x128>(v);  // row_ror:8 pairs lane i with i ^ 8 within its row
  return xor32_sum(xor16_sum(v));
}
template <int W> __device__ __forceinline__ float across_max(float v) {
  if constexpr (W == 8) v = fmaxf(v, dppf<0x128>(v));
  return xor32_max(xor16_max(v));
}

// ------------------------------------------------------------------ MFMA (gfx950)
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// v_mfma_f32_16x16x32_{bf16,f16}: A is 16x32, B is 32x16, D is 16x16 fp32. An MFMA writes its result whatever
// the EXEC mask holds, so every condition around one must be wave-uniform as the compiler sees it (derive wave
// indices with readfirstlane): a condition it takes as divergent becomes an EXEC-masked block that the MFMA
// ignores.
// Lane l holds A[l%16][8*(l/16)+e] and B[8*(l/16)+e][l%16] for e = 0..7, and D[4*(l/16)+r][l%16] for r = 0..3.
template <int DT> __device__ __forceinline__ f32x4_t mfma16x16x32(const u16x8& a, const u16x8& b, f32x4_t c);
template <> __device__ __forceinline__ f32x4_t mfma16x16x32<M3X_BF16>(const u16x8& a, const u16x8& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4_t mfma16x16x32<M3X_F16>(const u16x8& a, const u16x8& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                0, 0, 0);
}

// fp32 operands in the same fragment layout (lane l holds A[l%16][8*(l/16)+e] and B[8*(l/16)+e][l%16], e = 0..7):
// eight v_mfma_f32_16x16x4_f32, instruction e taking element e of each lane, whose k index l/16 then stands for
// k = 8*(l/16)+e of the 32. Together they add the same 32 products into D (same D layout as above), in fp32.
__device__ __forceinline__ f32x4_t mfma16x16x32_f32(const f32x8& a, const f32x8& b, f32x4_t c) {
#pragma unroll
  for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[e], b.v[e], c, 0, 0, 0);
  return c;
}

// one 32-deep k step of the fragment layout for any storage type
template <int DT> __device__ __forceinline__ f32x4_t mfma_k32(const V8<DT>& a, const V8<DT>& b, f32x4_t c) {
  if constexpr (DT == M3X_F32) return mfma16x16x32_f32(a, b, c);
  else return mfma16x16x32<DT>(a, b, c);
}

static inline int m3x_ceil_div(long a, long b) { return (int)((a + b - 1) / b); }
static inline bool m3x_aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }
