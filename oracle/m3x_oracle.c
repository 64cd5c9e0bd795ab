/* CPU oracle for the bit-exact parts of the m3x frame step.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may load this as
 * the reference they compare with. The product path (maya2-native_amd/m3x) never links or calls it.
 *
 * Each function restates the reference's arithmetic with the rounding points and the summation order the HIP
 * kernels commit to, written the plain way (full sorts, sequential loops), so that agreement is a check of the
 * kernels' indexing and parallel decomposition. Build: make -C oracle (gcc, -ffp-contract=off, SSE float).
 *
 * Pinning (what checks each function beyond the kernels): tests/test_oracle_bitexact.py
 *   o_bf16_round      vs torch's float->bfloat16 conversion (round-to-nearest-even), all bf16 patterns
 *   o_expf            vs math.exp: <= 2 ulp over [-87, 0], exact at 0, and e^(-ln2 k) = 2^-k
 *   o_add_rms         vs HF Qwen3RMSNorm / torch on random rows (<= 1 bf16 ulp) and a constant row (closed form)
 *   o_qk_norm_rope    vs the HF restatement of serve/fast_backbone.py's reference test (rel < 1e-2) and vs
 *                     position 0 (RoPE is the identity) and cos/sin pairs (rotation preserves each pair's norm)
 *   o_topk_sample     vs the exact top-k softmax (total variation over uniform draws), k=1 / u=0 -> argmax,
 *                     ties kept (x >= kth)
 *   o_cb0_sample      vs a torch restatement of maya3/engine.py:652-694 with the Gumbel race replaced by the
 *                     same inverse CDF (stop codes, renormalisation, penalty, bias); its top-p cut vs the
 *                     engine's softmax/sort/cumsum mask (:669-672) on distinct logits
 *   o_philox4x32_10   vs the Random123 known-answer vectors
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- bf16 */
static float bf2f(uint16_t b) {
  uint32_t u = ((uint32_t)b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float rbf(float f) { return bf2f(f2bf(f)); }

uint16_t o_bf16_round(float f) { return f2bf(f); }

void o_bf16_round_array(const float* x, uint16_t* y, long n) {
  for (long i = 0; i < n; ++i) y[i] = f2bf(x[i]);
}

/* ---------------------------------------------------------------- exp (Cody-Waite + degree-7 Taylor) */
float o_expf(float x) {
  if (x < -87.0f) return 0.0f;
  const float L2E = 1.44269504088896341f;
  const float LN2_HI = 0.693145751953125f;
  const float LN2_LO = 1.42860682030941723212e-6f;
  float n = rintf(x * L2E);
  float r = fmaf(-n, LN2_HI, x);
  r = fmaf(-n, LN2_LO, r);
  float p = 1.98412698412698413e-4f;
  p = fmaf(p, r, 1.38888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

void o_expf_array(const float* x, float* y, long n) {
  for (long i = 0; i < n; ++i) y[i] = o_expf(x[i]);
}

/* ---------------------------------------------------------------- reduction order R(N)
 * N/8 groups of 8 contiguous elements; each group's squares summed left to right; the N/8 partials folded in
 * half: p[g] += p[g + s] for s = N/16 .. 1.  */
static float tree_fold(float* p, int ng) {
  for (int s = ng / 2; s > 0; s >>= 1)
    for (int g = 0; g < s; ++g) p[g] = p[g] + p[g + s];
  return p[0];
}
static float sumsq_R(const float* x, int n) {
  float p[512];
  const int ng = n / 8;
  for (int g = 0; g < ng; ++g) {
    float s = x[8 * g] * x[8 * g];
    for (int e = 1; e < 8; ++e) s = s + x[8 * g + e] * x[8 * g + e];
    p[g] = s;
  }
  return tree_fold(p, ng);
}

/* serve/fast_backbone.py:95-104 (_add_rms); a == NULL: RMSNorm of h (HF Qwen3RMSNorm, :190) */
void o_add_rms(const uint16_t* h, const uint16_t* a, uint16_t* ho, uint16_t* y, const uint16_t* w, float eps,
               int rows, int n) {
  float x[4096];
  for (int r = 0; r < rows; ++r) {
    for (int i = 0; i < n; ++i) {
      float v = bf2f(h[(long)r * n + i]);
      if (a) v = rbf(v + bf2f(a[(long)r * n + i]));
      x[i] = v;
      if (ho) ho[(long)r * n + i] = f2bf(v);
    }
    const float ss = sumsq_R(x, n);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; ++i) y[(long)r * n + i] = f2bf(rbf(x[i] * inv) * bf2f(w[i]));
  }
}

/* serve/fast_backbone.py:61-92 (_qk_norm_rope_cache), rounding points :77-81.
 * qkv [rows, (H + 2KV) * D]; qout [rows, H, D]; kout [rows, KV, D] (the value placed at k_cache[slot, kh, pos]). */
void o_qk_norm_rope(const uint16_t* qkv, int rows, int H, int KV, int D, const int32_t* pos, const uint16_t* cosb,
                    const uint16_t* sinb, const uint16_t* wq, const uint16_t* wk, float eps, uint16_t* qout,
                    uint16_t* kout) {
  float x[256], yv[256];
  const int half = D / 2;
  for (int r = 0; r < rows; ++r) {
    const int ps = pos[r];
    for (int j = 0; j < H + KV; ++j) {
      const uint16_t* src = qkv + (long)r * (H + 2 * KV) * D + (long)j * D;
      const uint16_t* w = j < H ? wq : wk;
      for (int i = 0; i < D; ++i) x[i] = bf2f(src[i]);
      const float ss = sumsq_R(x, D);
      const float inv = 1.0f / sqrtf(ss / (float)D + eps);
      for (int i = 0; i < D; ++i) yv[i] = rbf(rbf(x[i] * inv) * bf2f(w[i]));
      uint16_t* dst = j < H ? qout + ((long)r * H + j) * D : kout + ((long)r * KV + (j - H)) * D;
      for (int i = 0; i < D; ++i) {
        const float c = bf2f(cosb[(long)ps * D + i]), s = bf2f(sinb[(long)ps * D + i]);
        const float a1 = yv[i] * c;
        if (i < half) {
          const float a2 = yv[i + half] * s;
          dst[i] = f2bf(a1 - a2);
        } else {
          const float a2 = yv[i - half] * s;
          dst[i] = f2bf(a1 + a2);
        }
      }
    }
  }
}

/* ---------------------------------------------------------------- samplers */
static uint32_t ordkey(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
typedef struct {
  uint32_t key;
  int idx;
  float x;
} Cand;
static int cand_cmp(const void* pa, const void* pb) {
  const Cand *a = (const Cand*)pa, *b = (const Cand*)pb;
  if (a->key != b->key) return a->key > b->key ? -1 : 1;
  return a->idx < b->idx ? -1 : (a->idx > b->idx ? 1 : 0);
}

/* sort x descending (index ascending on equal keys), return the number kept (x >= k-th largest) */
static int topk_order(const float* x, int V, int k, Cand* c) {
  for (int i = 0; i < V; ++i) {
    c[i].key = ordkey(x[i]);
    c[i].idx = i;
    c[i].x = x[i];
  }
  qsort(c, V, sizeof(Cand), cand_cmp);
  if (k > V) k = V;
  if (k < 1) k = 1;
  const float kth = c[k - 1].x;
  int n = 0;
  while (n < V && c[n].x >= kth) ++n;
  return n;
}

/* inverse CDF over c[0..n) skipping index `skip`; -1 if the weights sum to zero */
static int pick(const Cand* c, const float* w, int n, float u, int skip) {
  float S = 0.f;
  int last = -1;
  for (int j = 0; j < n; ++j) {
    if (c[j].idx == skip) continue;
    S = S + w[j];
    last = j;
  }
  if (last < 0 || !(S > 0.f)) return -1;
  const float t = u * S;
  float acc = 0.f;
  for (int j = 0; j < n; ++j) {
    if (c[j].idx == skip) continue;
    acc = acc + w[j];
    if (acc > t) return c[j].idx;
  }
  return c[last].idx;
}

/* depth sampler on a transformed row x (fp32): serve/fast_depth_kernels.py:48-79 contract with caller uniform */
int o_topk_sample(const float* x, int V, int k, float u, int greedy) {
  Cand* c = (Cand*)malloc(sizeof(Cand) * V);
  float* w = (float*)malloc(sizeof(float) * V);
  const int n = topk_order(x, V, k, c);
  int code = c[0].idx;
  if (!greedy) {
    for (int j = 0; j < n; ++j) w[j] = o_expf(c[j].x - c[0].x);
    const int p = pick(c, w, n, u, -1);
    if (p >= 0) code = p;
  }
  free(c);
  free(w);
  return code;
}

/* many draws from one transformed row (distribution tests): out[i] = sample for u[i] */
void o_topk_sample_many(const float* x, int V, int k, const float* u, int n_draws, int32_t* out) {
  Cand* c = (Cand*)malloc(sizeof(Cand) * V);
  float* w = (float*)malloc(sizeof(float) * V);
  const int n = topk_order(x, V, k, c);
  for (int j = 0; j < n; ++j) w[j] = o_expf(c[j].x - c[0].x);
  for (int i = 0; i < n_draws; ++i) {
    const int p = pick(c, w, n, u[i], -1);
    out[i] = p >= 0 ? p : c[0].idx;
  }
  free(c);
  free(w);
}

/* depth sampler from raw 16-bit logits: x = float(logit) * inv_temp (is_f16 selects fp16 storage) */
static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else {
      exp = 127 - 15 + 1;
      while (!(man & 0x400u)) {
        man <<= 1;
        --exp;
      }
      man &= 0x3ffu;
      u = sign | (exp << 23) | (man << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}
void o_topk_sample_rows(const uint16_t* logits, int B, int V, int is_f16, float inv_temp, int k, const float* u,
                        int greedy, int32_t* out) {
  float* x = (float*)malloc(sizeof(float) * V);
  for (int b = 0; b < B; ++b) {
    for (int i = 0; i < V; ++i) {
      const uint16_t v = logits[(long)b * V + i];
      x[i] = (is_f16 ? f16_to_f32(v) : bf2f(v)) * inv_temp;
    }
    out[b] = o_topk_sample(x, V, k, greedy ? 0.f : u[b], greedy);
  }
  free(x);
}

/* Top-p cut of a top-k kept set in sorted order (maya3/engine.py:669-672: drop a candidate when the probability
 * mass sorted before it exceeds top_p). Position j stays while run_(j-1) / S <= top_p, with run the sequential
 * fp32 running sum of the weights in order and S their total in the same order. Returns the kept length (>= 1). */
static int top_p_keep(const float* w, int n, float top_p) {
  float S = 0.f;
  for (int j = 0; j < n; ++j) S = S + w[j];
  float run = 0.f;
  for (int j = 0; j + 1 < n; ++j) {
    run = run + w[j];
    if (run / S > top_p) return j + 1;
  }
  return n;
}

/* cb0 controlled stop + sampling for one seat (maya3/engine.py:652-694), caller uniform in place of the
 * exponential race. State arrays are this seat's (scalars passed by pointer; hist of length hist_w).
 * top_p < 1 cuts the top-k set (top_p_keep) before the stop statistics and the draw.
 * Returns cb0; *stop gets the stop code. aeos < 0: no AEOS class (no stop logic, no exclusion). */
int o_cb0_sample(const uint16_t* logits, int V, int aeos, float temp, int k, float top_p, float bias, float rep,
                 int64_t* hist, int hist_w, int64_t* frames, int64_t min_frames, float* hazard, int32_t* ctr,
                 float u, int64_t* stop) {
  float* x = (float*)malloc(sizeof(float) * V);
  Cand* c = (Cand*)malloc(sizeof(Cand) * V);
  float* w = (float*)malloc(sizeof(float) * V);
  for (int i = 0; i < V; ++i) {
    float v = bf2f(logits[i]) / temp;
    if (i == aeos) v = v + bias;
    if (hist && i != aeos && rep != 0.f) {
      int seen = 0;
      for (int j = 0; j < hist_w; ++j) seen |= hist[j] == (int64_t)i;
      if (seen) v = v - rep;
    }
    x[i] = v;
  }
  if (k < 1) k = 1;
  if (k > V) k = V;
  int n = topk_order(x, V, k, c);
  for (int j = 0; j < n; ++j) w[j] = o_expf(c[j].x - c[0].x);
  if (top_p < 1.0f) n = top_p_keep(w, n, top_p);
  int cb0;
  *stop = 0;
  if (aeos >= 0) {
    float S = 0.f, wa = 0.f;
    for (int j = 0; j < n; ++j) {
      S = S + w[j];
      if (c[j].idx == aeos) wa = w[j];
    }
    const float pa = wa / S;
    const int arg = c[0].idx;
    if (frames && hazard) {
      const int can = *frames >= min_frames;
      const float hz0 = *hazard;
      const float hz = can ? 1.0f - (1.0f - hz0) * (1.0f - pa) : hz0;
      if (can && arg == aeos) *stop = 2;
      else if (can && pa >= 0.35f) *stop = 3;
      else if (can && hz >= 0.6f) *stop = 4;
      *hazard = hz;
      *frames = *frames + 1;
    }
    const int p = pick(c, w, n, u, aeos);
    cb0 = p < 0 ? 0 : p;
  } else {
    const int p = pick(c, w, n, u, -1);
    cb0 = p < 0 ? c[0].idx : p;
  }
  if (ctr) *ctr = *ctr + 1;
  if (hist && hist_w > 0) {
    for (int j = 0; j + 1 < hist_w; ++j) hist[j] = hist[j + 1];
    hist[hist_w - 1] = cb0;
  }
  free(x);
  free(c);
  free(w);
  return cb0;
}

/* ---------------------------------------------------------------- Philox4x32-10 (Salmon et al., SC11) */
void o_philox4x32_10(const uint32_t* ctr, const uint32_t* key, uint32_t* out) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t lo0 = (uint32_t)p0, hi0 = (uint32_t)(p0 >> 32), lo1 = (uint32_t)p1, hi1 = (uint32_t)(p1 >> 32);
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

float o_philox_uniform(uint32_t seed, uint32_t ctr, uint32_t level) {
  const uint32_t c[4] = {ctr, level, 0u, 0u}, k[2] = {seed, 0u};
  uint32_t o[4];
  o_philox4x32_10(c, k, o);
  return (float)(o[0] >> 8) * 5.9604644775390625e-8f;
}
