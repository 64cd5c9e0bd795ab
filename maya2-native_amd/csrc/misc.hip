// Small index kernels of the frame step: per-row positions, lengths update, row gathers/scatters, the frame's
// code ring and per-slot counters. All integer work, exact by construction.
#include "m3x_common.h"

// pos[r] = lengths[slots[r]] + offset[r]   (serve/fast_backbone.py:178-179; offset null = 0)
__global__ void positions_kernel(const int64_t* __restrict__ lengths, const int64_t* __restrict__ slots,
                                 const int64_t* __restrict__ offset, int32_t* __restrict__ pos, int R) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  pos[r] = (int32_t)(lengths[slots[r]] + (offset ? offset[r] : 0));
}

M3X_API int m3x_positions(const int64_t* lengths, const int64_t* slots, const int64_t* offset, int32_t* pos, int R,
                          void* stream) {
  if (R < 0) return M3X_EINVAL;
  if (R == 0) return M3X_OK;
  if (!lengths || !slots || !pos) return M3X_ENULL;
  hipLaunchKernelGGL(positions_kernel, dim3(m3x_ceil_div(R, 256)), dim3(256), 0, (hipStream_t)stream, lengths, slots,
                     offset, pos, R);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// lengths[slots[r]] += real[r] for every row (duplicates accumulate, like index_add_; serve/fast_backbone.py:233).
// The rows of an inline prefill are one slot over consecutive rows: each wave sums every run of equal slots among
// its lanes and adds it once, from the run's first lane, so a 256-row prefill costs 4 atomics on its slot instead
// of 256 serialised ones. Duplicates that are not adjacent still meet in the atomic.
__global__ void lengths_add_kernel(int64_t* lengths, const int64_t* __restrict__ slots,
                                   const int64_t* __restrict__ real, int R) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const bool live = r < R;
  const long long s = live ? slots[r] : -1;
  const long long v = live ? real[r] : 0;
  const long long prev = __shfl_up(s, 1, 64);  // every lane takes part (a lane masked off reads as 0)
  const bool head = lane == 0 || prev != s;
  const unsigned long long heads = __ballot(head);
  long long incl = v;  // inclusive prefix sum over the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const long long t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  const unsigned long long later = lane == 63 ? 0ull : heads & (~0ull << (lane + 1));
  const int end = later ? __ffsll(later) - 1 : 64;  // the next run's first lane
  const long long upto = __shfl(incl, end - 1, 64);
  const long long run = upto - (incl - v);
  if (live && head && run) atomicAdd((unsigned long long*)&lengths[s], (unsigned long long)run);
}

M3X_API int m3x_lengths_add(int64_t* lengths, const int64_t* slots, const int64_t* real, int R, void* stream) {
  if (R < 0) return M3X_EINVAL;
  if (R == 0) return M3X_OK;
  if (!lengths || !slots || !real) return M3X_ENULL;
  hipLaunchKernelGGL(lengths_add_kernel, dim3(m3x_ceil_div(R, 256)), dim3(256), 0, (hipStream_t)stream, lengths, slots,
                     real, R);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// dst[dst_idx[r] or r][:] = src[src_idx[r] + src_off or r][:], rows of n 16-bit elements (n % 8 == 0).
// Indices are int64 (idx_i32 = 0) or int32 (idx_i32 = 1) with element stride ld_idx; src indices are clamped to
// [0, src_rows) so an out-of-range code cannot read outside the table (the reference raises on the host instead,
// tts/model/audio_io.py:30-32; the host surfaces validate before the step).
// Used for: prefix rows = embed[level][code] (serve/fast_depth.py:135,196), x = feedback[slots], feedback[slots] = y.
__global__ void copy_rows_kernel(const uint16_t* __restrict__ src, long ld_src, const void* src_idx, long src_off,
                                 long src_rows, uint16_t* __restrict__ dst, long ld_dst, const int64_t* dst_idx,
                                 int rows, int nvec, int idx_i32, long ld_idx) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * nvec) return;
  const int r = (int)(i / nvec), v = (int)(i % nvec);
  long sr = r;
  if (src_idx) {
    sr = (idx_i32 ? (long)((const int32_t*)src_idx)[(long)r * ld_idx] : ((const int64_t*)src_idx)[(long)r * ld_idx]) +
         src_off;
    sr = sr < 0 ? 0 : (sr >= src_rows ? src_rows - 1 : sr);
  }
  const long dr = dst_idx ? dst_idx[r] : r;
  st16(dst + dr * ld_dst + 8 * v, ld16(src + sr * ld_src + 8 * v));
}

M3X_API int m3x_copy_rows(const void* src, long ld_src, const void* src_idx, long src_off, long src_rows, void* dst,
                          long ld_dst, const int64_t* dst_idx, int rows, int n, int idx_i32, long ld_idx,
                          void* stream) {
  if (rows < 0 || n <= 0 || (n & 7) || (ld_src & 7) || (ld_dst & 7)) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!src || !dst) return M3X_ENULL;
  if (src_idx && src_rows <= 0) return M3X_EINVAL;
  if (!m3x_aligned16(src) || !m3x_aligned16(dst)) return M3X_EINVAL;
  const long total = (long)rows * (n / 8);
  hipLaunchKernelGGL(copy_rows_kernel, dim3(m3x_ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)src, ld_src, src_idx, src_off, src_rows, (uint16_t*)dst, ld_dst, dst_idx, rows,
                     n / 8, idx_i32, ld_idx);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// Frame code ring: ring[(*head) % depth][b][0..nq) = codes[b][0..nq) for b < B, then *head += 1.
// One workgroup, so the head update is ordered after every copy of this launch.
__global__ __launch_bounds__(1024) void code_ring_kernel(const int32_t* __restrict__ codes, long ld_codes,
                                                         int32_t* __restrict__ ring, int32_t* head, int depth,
                                                         int seats, int nq, int B) {
  // each thread's codes of a batch are all requested before the first store (clamped index, masked store), so a
  // 224 x 32 frame is one round trip rather than one per element
  constexpr int U = 8;
  const int total = B * nq;
  const int nt = blockDim.x;
  const int h = *head;
  for (int base = 0; base < total; base += nt * U) {
    int32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = min(base + (int)threadIdx.x + nt * u, total - 1);
      v[u] = codes[(long)(i / nq) * ld_codes + i % nq];
    }
    const int slotr = ((h % depth) + depth) % depth;
    int32_t* dst = ring + (long)slotr * seats * nq;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + (int)threadIdx.x + nt * u;
      if (i < total) dst[(long)(i / nq) * nq + i % nq] = v[u];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) *head = h + 1;
}

M3X_API int m3x_code_ring_write(const int32_t* codes, long ld_codes, int32_t* ring, int32_t* head, int depth,
                                int seats, int nq, int B, void* stream) {
  if (B < 0 || depth <= 0 || nq <= 0 || B > seats || ld_codes < nq) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!codes || !ring || !head) return M3X_ENULL;
  hipLaunchKernelGGL(code_ring_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, codes, ld_codes, ring, head, depth,
                     seats, nq, B);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ctr[slots[b]] += 1 (serve/fast_depth.py:199, row_ctr.index_add_)
__global__ void ctr_add_kernel(int32_t* ctr, const int64_t* __restrict__ slots, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) atomicAdd(&ctr[slots[b]], 1);
}

M3X_API int m3x_ctr_add(int32_t* ctr, const int64_t* slots, int B, void* stream) {
  if (B < 0) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!ctr || !slots) return M3X_ENULL;
  hipLaunchKernelGGL(ctr_add_kernel, dim3(m3x_ceil_div(B, 256)), dim3(256), 0, (hipStream_t)stream, ctr, slots, B);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Loop guard (maya3/guards.py:80-107 loop_detect_batch; engine tick maya3/engine.py:594-617), on the device so the
// check needs no host copy of the code history.
//
// hist_push: the history row of slot slots[b] (hist_len codes, oldest first, -1 = empty) shifts left by one and
// takes codes[b * ld_codes] as its newest entry (maya3/engine.py:585-586), and frames[slots[b]] (if given) counts the
// frame. One wave per seat; every lane reads its entries before any lane writes. Rows repeated within one call
// (the padding rows of a graph bucket, all on the dummy slot) race: that slot's row is scratch.
__global__ __launch_bounds__(64) void hist_push_kernel(int32_t* hist, long ld_hist, int64_t* frames,
                                                       const int64_t* __restrict__ slots,
                                                       const int64_t* __restrict__ codes, long ld_codes, int hist_len) {
  const int b = blockIdx.x;
  const long s = slots[b];
  int32_t* row = hist + s * ld_hist;
  const int l = threadIdx.x;
  if (frames && l == 0) frames[s] = frames[s] + 1;
  int32_t v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = l + 64 * e;
    v[e] = i + 1 < hist_len ? row[i + 1] : (i + 1 == hist_len ? (int32_t)codes[(long)b * ld_codes] : 0);
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = l + 64 * e;
    if (i < hist_len) row[i] = v[e];
  }
}

M3X_API int m3x_hist_push(int32_t* hist, long ld_hist, int64_t* frames, const int64_t* slots, const int64_t* codes,
                          long ld_codes, int B, int hist_len, void* stream) {
  if (B < 0 || hist_len <= 0 || hist_len > 256 || ld_hist < hist_len || ld_codes < 1) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!hist || !slots || !codes) return M3X_ENULL;
  hipLaunchKernelGGL(hist_push_kernel, dim3(B), dim3(64), 0, (hipStream_t)stream, hist, ld_hist, frames, slots, codes,
                     ld_codes, hist_len);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// loop_guard: row slots[r] of W (hist_len codes, newest last) with n[slots[r]] frames (row r and n[r] when slots is
// NULL) ->
//   out[r] = 0 (no loop), -1 (stall: the last `stall` codes all equal the first of them, n >= max(12, stall)) or p
//   (period: with win = the last period_win codes, the fraction of i < period_win - p with win[i + p] == win[i] is
//   >= period_thr, for the smallest p in pmin..pmax; needs n >= max(12, stall, period_win)). The fraction is the
//   reference's float64 mean, count / (period_win - p). One wave per row.
__global__ __launch_bounds__(64) void loop_guard_kernel(const int32_t* __restrict__ W, long ld_w,
                                                        const int64_t* __restrict__ slots,
                                                        const int64_t* __restrict__ n, int32_t* __restrict__ out,
                                                        int hist_len, int stall, int period_win, double period_thr,
                                                        int pmin, int pmax) {
  const int r = blockIdx.x;
  const int l = threadIdx.x;
  const long src = slots ? slots[r] : (long)r;
  const int32_t* row = W + src * ld_w;
  const long frames = n[src];
  const int st0 = hist_len - stall;
  const int32_t first = row[st0];
  const bool same = l >= stall || row[st0 + l] == first;
  const bool is_stall = __ballot(!same) == 0ull;
  const int w0 = hist_len - period_win;
  const int32_t wl = l < period_win ? row[w0 + l] : 0;
  int hit = 0;
  for (int p = pmin; p <= pmax && hit == 0; ++p) {
    const int m = period_win - p;
    const int32_t wp = l + p < period_win ? row[w0 + l + p] : 0;
    const int count = __popcll(__ballot(l < m && wp == wl));
    if ((double)count / (double)m >= period_thr) hit = p;
  }
  if (l == 0) {
    const long need = stall > 12 ? stall : 12;
    const long need_p = period_win > need ? period_win : need;
    int code = 0;
    if (frames >= need) {
      if (is_stall) code = -1;
      else if (frames >= need_p && hit) code = hit;
    }
    out[r] = code;
  }
}

M3X_API int m3x_loop_guard(const int32_t* W, long ld_w, const int64_t* slots, const int64_t* n, int32_t* out,
                           int rows, int hist_len, int stall, int period_win, double period_thr, int pmin, int pmax,
                           void* stream) {
  if (rows < 0 || hist_len <= 0 || ld_w < hist_len) return M3X_EINVAL;
  if (stall < 1 || stall > 64 || stall > hist_len || period_win < 2 || period_win > 64 || period_win > hist_len)
    return M3X_EINVAL;
  if (pmin < 1 || pmax < pmin || pmax >= period_win) return M3X_EINVAL;
  if (rows == 0) return M3X_OK;
  if (!W || !n || !out) return M3X_ENULL;
  hipLaunchKernelGGL(loop_guard_kernel, dim3(rows), dim3(64), 0, (hipStream_t)stream, W, ld_w, slots, n, out,
                     hist_len, stall, period_win, period_thr, pmin, pmax);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Tick readout (maya3/engine.py:558-563): one int64 row per seat for a single pinned host copy,
//   [stop, cb0, (loop code), (nq codes, two int32 per int64), (frame int16 PCM samples, four per int64)]
// with pcm16 = int16(rint(clamp(pcm, -1, 1) * 32767)) (torch's round is half to even, as rintf). Optional parts are
// left out when their pointer is NULL. One workgroup per seat.
__global__ __launch_bounds__(256) void tick_pack_kernel(const int64_t* __restrict__ stop,
                                                        const int64_t* __restrict__ cb0,
                                                        const int32_t* __restrict__ loop,
                                                        const int32_t* __restrict__ codes, long ld_codes, int nq,
                                                        const float* __restrict__ pcm, long ld_pcm, int frame,
                                                        int64_t* __restrict__ out, long ld_out) {
  const int b = blockIdx.x;
  int64_t* row = out + (long)b * ld_out;
  int col = 2;
  if (threadIdx.x == 0) {
    row[0] = stop[b];
    row[1] = cb0[b];
  }
  if (loop) {
    if (threadIdx.x == 0) row[col] = loop[b];
    col += 1;
  }
  if (codes) {
    for (int i = threadIdx.x; 2 * i < nq; i += blockDim.x) {
      const uint32_t lo = (uint32_t)codes[(long)b * ld_codes + 2 * i];
      const uint32_t hi = 2 * i + 1 < nq ? (uint32_t)codes[(long)b * ld_codes + 2 * i + 1] : 0u;
      row[col + i] = (int64_t)(((uint64_t)hi << 32) | lo);
    }
    col += (nq + 1) / 2;
  }
  if (pcm) {
    const float* p = pcm + (long)b * ld_pcm;
    for (int i = threadIdx.x; 4 * i < frame; i += blockDim.x) {
      uint64_t v = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (4 * i + e < frame) {
          const float x = fminf(fmaxf(p[4 * i + e], -1.0f), 1.0f) * 32767.0f;
          v |= (uint64_t)(uint16_t)(int16_t)rintf(x) << (16 * e);
        }
      }
      row[col + i] = (int64_t)v;
    }
  }
}

M3X_API int m3x_tick_pack_width(int with_loop, int nq, int frame) {
  if (nq < 0 || frame < 0) return -1;
  return 2 + (with_loop ? 1 : 0) + (nq + 1) / 2 + (frame + 3) / 4;
}

M3X_API int m3x_tick_pack(const int64_t* stop, const int64_t* cb0, const int32_t* loop, const int32_t* codes,
                          long ld_codes, int nq, const float* pcm, long ld_pcm, int frame, int64_t* out, long ld_out,
                          int B, void* stream) {
  if (B < 0 || (codes && (nq <= 0 || ld_codes < nq)) || (pcm && (frame <= 0 || ld_pcm < frame))) return M3X_EINVAL;
  if (B == 0) return M3X_OK;
  if (!stop || !cb0 || !out) return M3X_ENULL;
  if (ld_out < m3x_tick_pack_width(loop != nullptr, codes ? nq : 0, pcm ? frame : 0)) return M3X_EINVAL;
  hipLaunchKernelGGL(tick_pack_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, stop, cb0, loop, codes, ld_codes,
                     codes ? nq : 0, pcm, ld_pcm, pcm ? frame : 0, out, ld_out);
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// dst[r][c] = convert(src[r][c]) between bf16, fp16 and fp32 (round to nearest even). The frame step hands the
// backbone's bf16 hidden state to a depth that computes in another dtype (maya3/engine.py:192-199 builds the depth
// in fp16 by default) and takes the result back.
template <int SDT, int DDT>
__device__ __forceinline__ void cast_one(const void* src, void* dst, long si, long di) {
  float v;
  if constexpr (SDT == M3X_F32) v = ((const float*)src)[si];
  else v = E<SDT>::to_f(((const uint16_t*)src)[si]);
  if constexpr (DDT == M3X_F32) ((float*)dst)[di] = v;
  else ((uint16_t*)dst)[di] = E<DDT>::from_f(v);
}

template <int SDT, int DDT>
__global__ void cast_rows_kernel(const void* __restrict__ src, long ld_src, void* __restrict__ dst, long ld_dst,
                                 int rows, int n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * n) return;
  const long r = i / n, c = i % n;
  cast_one<SDT, DDT>(src, dst, r * ld_src + c, r * ld_dst + c);
}

M3X_API int m3x_cast_rows(const void* src, long ld_src, int src_dtype, void* dst, long ld_dst, int dst_dtype,
                          int rows, int n, void* stream) {
  if (rows < 0 || n <= 0 || ld_src < n || ld_dst < n) return M3X_EINVAL;
  if (src_dtype < 0 || src_dtype > 2 || dst_dtype < 0 || dst_dtype > 2) return M3X_EUNSUPPORTED;
  if (rows == 0) return M3X_OK;
  if (!src || !dst) return M3X_ENULL;
  const dim3 grid(m3x_ceil_div((long)rows * n, 256));
  hipStream_t st = (hipStream_t)stream;
#define M3X_CAST(S, D)                                                                                  \
  if (src_dtype == S && dst_dtype == D)                                                                 \
    hipLaunchKernelGGL((cast_rows_kernel<S, D>), grid, dim3(256), 0, st, src, ld_src, dst, ld_dst, rows, n);
  M3X_CAST(M3X_BF16, M3X_BF16) M3X_CAST(M3X_BF16, M3X_F16) M3X_CAST(M3X_BF16, M3X_F32)
  M3X_CAST(M3X_F16, M3X_BF16) M3X_CAST(M3X_F16, M3X_F16) M3X_CAST(M3X_F16, M3X_F32)
  M3X_CAST(M3X_F32, M3X_BF16) M3X_CAST(M3X_F32, M3X_F16) M3X_CAST(M3X_F32, M3X_F32)
#undef M3X_CAST
  M3X_CHECK_LAUNCH();
  return M3X_OK;
}

// The library's version, so a host binding can check it loaded the build it expects.
M3X_API int m3x_version(void) { return 16; }
