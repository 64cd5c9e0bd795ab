/* m3x: MI355X (gfx950) kernels of the Maya3 per-frame decode step, as a C ABI.
 *
 * Conventions (every entry point):
 *   - pointers are device pointers (from any HIP allocator); sizes/strides are in ELEMENTS;
 *   - 16-bit tensors are bf16 (dtype M3X_BF16 = 0) or fp16 (M3X_F16 = 1) stored as raw 16-bit words;
 *   - `stream` is a hipStream_t (NULL = the default stream); launches are stream-ordered, never synchronise and
 *     never allocate, so every call can be captured into a hipGraph; scratch memory comes in as `workspace`;
 *   - the return value is 0 (M3X_OK) when the kernels were launched, else a negative status:
 *       -1 M3X_EINVAL bad shape/stride/alignment, -2 M3X_ENULL missing pointer, -3 M3X_EWORKSPACE workspace too
 *       small, -4 M3X_ELAUNCH launch failed, -5 M3X_EUNSUPPORTED shape/dtype not implemented.
 * Reference citations are to MayaResearch/maya2-native.
 */
#ifndef M3X_H
#define M3X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { M3X_OK = 0, M3X_EINVAL = -1, M3X_ENULL = -2, M3X_EWORKSPACE = -3, M3X_ELAUNCH = -4, M3X_EUNSUPPORTED = -5 };
enum { M3X_BF16 = 0, M3X_F16 = 1, M3X_F32 = 2 };
enum { M3X_NORM_LAYER = 0, M3X_NORM_RMS = 1 };
enum { M3X_ACT_NONE = -1, M3X_ACT_SWIGLU = 0, M3X_ACT_GELU = 1 };

int m3x_version(void);

/* ---- backbone step (serve/fast_backbone.py StaticBackbone._forward, fuse_rope path :176-234) ---------------- */

/* pos[r] = lengths[slots[r]] + offset[r] (offset may be NULL).
 * Replaces `pos=self.lengths[slots]; pos=pos+offset` (serve/fast_backbone.py:178-179). */
int m3x_positions(const int64_t* lengths, const int64_t* slots, const int64_t* offset, int32_t* pos, int R,
                  void* stream);

/* lengths[slots[r]] += real[r] (duplicates accumulate).
 * Replaces `self.lengths.index_add_(0,slots,real)` (serve/fast_backbone.py:233). */
int m3x_lengths_add(int64_t* lengths, const int64_t* slots, const int64_t* real, int R, void* stream);

/* h_out = bf16(h + a); y = bf16(bf16(h_out * 1/sqrt(mean(h_out^2) + eps)) * w); a == NULL: y = RMSNorm(h).
 * n in {512, 1024, 2048}; h_out may alias h. Fixed fp32 reduction order (bit-exact vs the oracle).
 * Replaces `_add_rms` + `_add_norm` (serve/fast_backbone.py:95-104,236-240) and the HF input RMSNorm (:190). */
int m3x_add_rms(const void* h, long s_h, const void* a, long s_a, void* h_out, long s_ho, void* y, long s_y,
                const void* w, float eps, int rows, int n, void* stream);

/* Per-head q/k RMSNorm + RoPE (rotate_half) of qkv rows [q heads | k heads | v heads]; q heads -> q_out
 * [rows, heads, D]; k heads -> k_cache[slots[r], kh, pos[r], :]; v heads copied to v_cache at the same place.
 * head_dim in {64, 128}; cos/sin are [cap, head_dim] tables in bf16.
 * Replaces `_qk_norm_rope_cache` (serve/fast_backbone.py:61-92, launch :195-197). */
int m3x_qk_norm_rope_cache(const void* qkv, long s_qkv, void* q_out, long s_qo_b, long s_qo_h, void* k_cache,
                           void* v_cache, long sk_s, long sk_h, long sk_t, const int64_t* slots, const int32_t* pos,
                           const void* cos, const void* sin, long s_cos, const void* wq, const void* wk, float eps,
                           int rows, int heads, int kv_heads, int head_dim, int cap, void* stream);

/* Bytes of workspace m3x_decode_attn needs for (rows, kv_heads, max_ctx, chunk). */
size_t m3x_decode_attn_workspace(int rows, int kv_heads, int max_ctx, int chunk);

/* GQA decode attention in place over the static cache: out[r, h, :] = softmax(q[r,h]·K[slot,h/G,0..pos]^T * scale)
 * · V[...]; heads/kv_heads in {1, 2}; head_dim 128; chunk = keys per split (multiple of 128); max_ctx >= pos+1
 * for every row; cap % 32 == 0.
 * items (nullable) lists the step's work for one launch of 2 workgroups per CU: an item is split s (keys
 * [s * chunk, (s + 1) * chunk)) of m rows of one slot (1 <= m <= 16: a decode row, or up to 16 rows of an inline
 * prefill, one or two blocks of 16 / G rows), code 2048 * first_row + 32 * s + m; every split of every row in exactly
 * one item; rows < 2^20.
 * The items are dealt into bins = m3x_decode_attn_item_bins(...) bins, and items = [bins, start[0], ...,
 * start[bins], codes of bin 0, codes of bin 1, ...] (int32). An item's rows share one pass over the slot's keys,
 * each row causal up to its own pos; every row gets the same bits as without items. With items, out must be
 * 16-byte aligned with so_b, so_h % 8 == 0.
 * Replaces `_decode_attn` + `StaticBackbone._launch` (serve/fast_backbone.py:31-58,242-247), including the inline
 * prefill rows of `step_mixed` (:326-333). */
int m3x_decode_attn(const void* q, long sq_b, long sq_h, const void* k_cache, const void* v_cache, long sk_s,
                    long sk_h, long sk_t, int cap, void* out, long so_b, long so_h, const int64_t* slots,
                    const int32_t* pos, const int32_t* items, float scale, int rows, int heads, int kv_heads,
                    int head_dim, int max_ctx, int chunk, void* workspace, size_t ws_bytes, void* stream);

/* Bins of m3x_decode_attn's item launch for (rows, kv_heads, max_ctx, chunk): one workgroup per bin per kv head
 * and split, 2 workgroups per CU (512 over the kv heads). */
int m3x_decode_attn_item_bins(int rows, int kv_heads, int max_ctx, int chunk);

/* Host function (no GPU work): the item list of m3x_decode_attn for rows laid out as nruns runs, runs[3 i ..] =
 * (first row, rows, first position): a decode row is a run of one row, an inline prefill of T tokens a run of T rows
 * at consecutive positions of one slot. Each run is cut into blocks of up to 16 / (heads / kv_heads) rows and each
 * block's keys into splits of `chunk`; an item is one split of one block, costing its keys + 64. The items are dealt
 * into `bins` bins longest processing time first (stable on equal costs), each to the least loaded bin (lowest index
 * on equal loads). Writes [bins, start[0..bins], codes bin by bin] into out (capacity out_cap int32) and returns the
 * count, or a negative status. Replaces the host-side staging of `step_mixed`'s inline prefill rows
 * (serve/fast_backbone.py:326-333). */
long m3x_decode_attn_items(const int32_t* runs, int nruns, int heads, int kv_heads, int bins, int chunk, int32_t* out,
                           long out_cap);

/* m3x_decode_attn without a workspace argument, allocating nothing. No counterpart in the reference: it is for
 * callers that cannot allocate (code under graph capture, tight serving loops, harnesses that forbid allocation).
 * The split partials live in a file-scope device array of M3X_DECODE_ATTN_NOALLOC_SCRATCH bytes that each GPU holds
 * until the process ends; its address is taken on a device's first call (hipGetSymbolAddress, with the device
 * current). Returns M3X_EWORKSPACE when m3x_decode_attn_workspace(rows, kv_heads, max_ctx, chunk) exceeds that size
 * (nothing is launched). Calls that overlap on one GPU share the array and race. Results are m3x_decode_attn's. */
#define M3X_DECODE_ATTN_NOALLOC_SCRATCH (4u << 20)
int m3x_decode_attn_noalloc(const void* q, long sq_b, long sq_h, const void* k_cache, const void* v_cache, long sk_s,
                            long sk_h, long sk_t, int cap, void* out, long so_b, long so_h, const int64_t* slots,
                            const int32_t* pos, const int32_t* items, float scale, int rows, int heads, int kv_heads,
                            int head_dim, int max_ctx, int chunk, void* stream);

/* Elements of the packed form of an [N, K] weight (N rounded up to a multiple of 16, times K); -1 if K % 32. */
long m3x_packed_weight_elems(int N, int K);

/* Packs w[N, K] (row stride ldw; bf16, fp16 or fp32 per dtype) into MFMA fragment order for m3x_linear /
 * m3x_linear_act: the 16 x 32 fragment (row tile t, k step s) sits at element (t * K/32 + s) * 512, lane l's 8
 * values at + 8 l holding w[16 t + l % 16][32 s + 8 (l / 16) + e]; rows past N are zero. Done once per weight at
 * load time. Replaces nothing at run time: the reference multiplies nn.Linear weights in place (F.linear). */
int m3x_pack_weight(const void* w, long ldw, int N, int K, void* out, int dtype, void* stream);

/* y[M,N] = x[M,K] · w[N,K]^T with w packed by m3x_pack_weight; bf16/fp16 in and out with fp32 accumulation
 * (MFMA 16x16x32), or fp32 throughout (dtype M3X_F32: MFMA 16x16x4 f32, the fp32 depth and codec paths);
 * K % 32 == 0. Deterministic (K slices are summed in a fixed order inside the workgroup), one launch, no workspace.
 * Replaces `F.linear` / `nn.Linear` on the path: q|k|v, o, down (serve/fast_backbone.py:193,200,202),
 * cb0 head (tts/model/backbone.py:135-136), depth trunk and heads (serve/fast_depth.py:104,122,125,185-191). */
int m3x_linear(const void* x, long ldx, const void* w_packed, void* y, long ldy, int M, int N, int K, int dtype,
               void* stream);

/* Projection with a fused gated epilogue, weights packed by m3x_pack_weight. kind M3X_ACT_SWIGLU:
 * y[:, :I] = dt(dt(silu(dt(x·wg^T))) * dt(x·wu^T)) with wg, wu [I, K]; kind M3X_ACT_GELU: y[:, :I] = gelu(dt(x·wg^T)).
 * Replaces `gu=F.linear(y2,wgu); g,u=gu.chunk(2,-1); F.silu(g)*u` (serve/fast_backbone.py:201-202) and
 * `F.gelu(block.f1(y2))` (serve/fast_depth.py:123,186). */
int m3x_linear_act(const void* x, long ldx, const void* wg_packed, const void* wu_packed, void* y, long ldy, int M,
                   int I, int K, int kind, int dtype, void* stream);

/* Projection that joins the residual stream: h_out[m, :] = dt(h[m, :] + dt(x[m, :] . w^T)), then, when c is not
 * NULL, h_out[m, :] = dt(h_out[m, :] + c[(m / tc) * ldc + :]) (a per-seat constant such as the depth trunk's
 * speaker term). The same launch writes part[m * (N / 16) + j] (float2) for every 16-column tile j of the stored
 * row: (sum, sum of squares) for norm_kind M3X_NORM_RMS, (sum, sum of squared deviations from the tile mean) for
 * M3X_NORM_LAYER, which m3x_linear_normed turns into the norm that follows. bf16/fp16; K % 32 == 0, N % 16 == 0;
 * h_out may equal h. Replaces `F.linear(...)` followed by the add of `_add_rms` (serve/fast_backbone.py:95-104,
 * 200,202,236-240) and of `add_ln` (serve/fast_depth_kernels.py:14-45; serve/fast_depth.py:122,125,185,191). */
int m3x_linear_resid(const void* x, long ldx, const void* w_packed, const void* h, long ldh, const void* c, long ldc,
                     int tc, void* h_out, long ld_out, void* part, int M, int N, int K, int norm_kind, int dtype,
                     void* stream);

/* Projection of normed rows: y = act(norm(x) . W^T) for x [M, K = 1024] whose rows m3x_linear_resid wrote with
 * their tile statistics `part`, norm RMSNorm (weight nw) or LayerNorm (nw, nb; eps for both). The norm is folded:
 * the weights are packed from Wf = dt(W * nw) (per input column), and the product of the raw rows is scaled per row,
 * RMSNorm inv_rms * (x . Wf^T), LayerNorm rstd * (x . Wf^T) - rstd * mean * u + v with the fp32 column vectors
 * u[n] = sum_k Wf[n, k], v[n] = sum_k nb[k] W[n, k] (NULL for RMSNorm; 2N entries, gate then up, for SwiGLU). act as
 * m3x_linear_act (M3X_ACT_SWIGLU with wg/wu, M3X_ACT_GELU with wg) or M3X_ACT_NONE (plain, wu NULL). Against the
 * reference's order the one rounding to the storage type moves from the normed activation to the folded weight.
 * Replaces the norm of `_add_rms` / `add_ln` and the projection it feeds: q|k|v and gate|up
 * (serve/fast_backbone.py:186,193,199-202), the depth trunk's q|k|v, f1 / gate|up and the codebook head after the
 * final norm (serve/fast_depth.py:104,122-125,165-191). */
int m3x_linear_normed(const void* x, long ldx, const void* part, const float* u, const float* v, float eps,
                      int norm_kind, const void* wg_packed, const void* wu_packed, void* y, long ldy, int M, int N,
                      int K, int act, int dtype, void* stream);

/* The q|k|v projection followed by m3x_qk_norm_rope_cache on its bf16 output, head_dim 128: x . W^T with W
 * [(heads + 2 kv_heads) * 128, K] packed, or, when part is given (K = 1024), m3x_linear_normed's RMSNorm-folded
 * product of rows whose tile statistics are part (eps_in the input norm's epsilon, W packed from the folded
 * weight). When the row count's plan gives each workgroup whole heads (193..256 rows and above 512 at N = 4096,
 * K = 1024) the norm, RoPE and cache writes run in the projection's epilogue and qkv is not written; otherwise the
 * two launches run in turn through qkv [M, ld_qkv]. The outputs are the same bits either way.
 * Replaces `F.linear(x, wqkv)` + `_qk_norm_rope_cache` (serve/fast_backbone.py:193-197, 61-92). */
int m3x_linear_qk_rope(const void* x, long ldx, const void* part, float eps_in, const void* w_packed, void* qkv,
                       long ld_qkv, void* q_out, long s_qo_b, long s_qo_h, void* k_cache, void* v_cache, long sk_s,
                       long sk_h, long sk_t, const int64_t* slots, const int32_t* pos, const void* cos, const void* sin,
                       long s_cos, const void* wq, const void* wk, float eps, int M, int K, int heads, int kv_heads,
                       int head_dim, int cap, void* stream);

/* out[r, :I] = act(in[r, :]): M3X_ACT_SWIGLU: bf16(silu(g)) * u with in = [g | u] (2*I wide);
 * M3X_ACT_GELU: gelu(in[r, :I]) (erf form), for callers that already hold the projection output.
 * Replaces `F.silu(g_)*u_` (serve/fast_backbone.py:201-202) and `F.gelu` (serve/fast_depth.py:123,186). */
int m3x_act(const void* in, long ld_in, void* out, long ld_out, int rows, int I, int kind, int dtype, void* stream);

/* ---- depth frame step (serve/fast_depth.py FastDepth._compute/_compute_fused :84-203) ----------------------- */

/* Row r = (b, t) = (r / T, r % T): x_out = dt(x + a) [then dt(x_out + c[b])]; y = norm(x_out) with LayerNorm
 * (w, b) or RMSNorm (w). x and a are read at base + b*s?b + t*s?t; x_out and y are contiguous [rows, n]; c rows
 * have stride s_c (0 broadcasts); a, c, x_out may be NULL; n in {512, 1024, 2048}.
 * Replaces `_add_ln`/`add_ln` (serve/fast_depth_kernels.py:14-45) and the first-layer `n1` (serve/fast_depth.py:164). */
int m3x_add_norm(const void* x, long sxb, long sxt, const void* a, long sab, long sat, const void* c, long s_c,
                 void* x_out, void* y, const void* w, const void* b, float eps, int rows, int T, int n, int kind,
                 int dtype, void* stream);

/* out[r] = dt(x[r] + bias[r * ld_bias]) (ld_bias = 0 broadcasts one row); n % 8 == 0.
 * Replaces `d.in_proj(h) + self.level0` (serve/fast_depth.py:150). */
int m3x_add_rows(const void* x, long ld_x, const void* bias, long ld_bias, void* out, long ld_out, int rows, int n,
                 int dtype, void* stream);

/* Depth self-attention over one frame's positions: qkv rows (b, t) at positions p0+t, read at
 * qkv + b*sqb + t*sqt ([q|k|v] x heads x head_dim); write_kv stores their K/V into the scratch kd/vd
 * [B, heads, np, head_dim]; queries t >= tq0 attend keys 0..p0+t; output row (b, t-tq0) at out + b*sob + tq*sot.
 * np <= 64, head_dim in {64, 128}.
 * Replaces the trunk's `F.scaled_dot_product_attention` + within-group KV (serve/fast_depth.py:102-121,165-183). */
int m3x_depth_attn(const void* qkv, long sqb, long sqt, void* kd, void* vd, void* out, long sob, long sot, int B,
                   int T, int p0, int tq0, int heads, int head_dim, int np, float scale, int write_kv, int dtype,
                   void* stream);

/* Top-k sampler with caller uniforms (x = logit * inv_temp; inverse CDF over the kept set, order x desc / index
 * asc; greedy = argmax); V <= 4096; writes int32 or int64 codes to out[b * ld_out].
 * Replaces `_topk_sample`/`topk_sample` (serve/fast_depth_kernels.py:48-79) and the unfused sampler
 * (serve/fast_depth.py:125-132). */
int m3x_topk_sample(const void* logits, long ld_l, int V, const float* u, long ld_u, float inv_temp, int top_k,
                    int greedy, void* out, long ld_out, int out_i64, int B, int dtype, void* stream);

/* m3x_topk_sample, then the next codebook's input from each drawn code: prefix[b*ld_prefix + j] =
 * table[code*ld_table + j] (j < n, n = 1024 or 2048, codes clamped to [0, table_rows)); with y given, also
 * x_out[b*n + j] = that row and y[b*n + j] = its LayerNorm (kind 0: w, bias) or RMSNorm (kind 1: w), the
 * arithmetic of m3x_add_norm with no addend. Replaces, per codebook, the sampler + the prefix-row gather
 * (serve/fast_depth.py:137-138) + the next level's input norm (serve/fast_depth.py:164). */
int m3x_topk_sample_embed(const void* logits, long ld_l, int V, const float* u, long ld_u, float inv_temp, int top_k,
                          int greedy, void* out, long ld_out, int out_i64, int B, const void* table, long ld_table,
                          long table_rows, void* prefix, long ld_prefix, void* x_out, void* y, const void* w,
                          const void* b, float eps, int kind, int n, int dtype, void* stream);

/* cb0 controlled stop + sampling per seat (per-slot state indexed by slots[b]); any per-slot pointer may be NULL.
 * Replaces `Engine._cb0` (maya3/engine.py:652-694) with caller uniforms in place of `row_exponential`
 * (serve/fast_depth_kernels.py:82-98). topp_t[s] (or top_p when topp_t is NULL) below 1 applies the top-p cut
 * of :669-672 to the top-k set. hist_w (the repetition-penalty window, 12 frames by default in the engine) is at
 * most 256 (M3X_EINVAL above). */
int m3x_cb0_sample(const void* logits, long ld_l, int V, int aeos, const int64_t* slots, const float* u, long ld_u,
                   const float* temp_t, float temp, const int64_t* topk_t, int top_k, const float* topp_t,
                   float top_p, const float* aeos_bias,
                   const float* rep_t, int64_t* hist_t, int hist_w, int64_t* frames_t, const int64_t* min_t,
                   float* hazard_t, int32_t* ctr_t, int64_t* cb0_out, int32_t* cb0_i32, long ld_cb0_i32,
                   int64_t* stop_out, int B, void* stream);

/* u[b, j] = Philox4x32-10 uniform for counter (ctrs[s], level0 + j, 0, 0), key (seeds[s], 0), s = slots[b].
 * Replaces the per-request Philox streams keyed by (seed, frame counter, level)
 * (serve/fast_depth_kernels.py:63,90; maya3/engine.py:436-437). */
int m3x_philox_uniforms(const int32_t* seeds, const int32_t* ctrs, const int64_t* slots, float* out, long ld_out,
                        int level0, int nlevels, int B, void* stream);

/* out[b, c] = -log(max(u, 1e-12)) with u the Philox uniform of counter (ctrs[b], level, c, 0), key (seeds[b], 0),
 * for c < V (per-row seeds/counters, already gathered by the caller).
 * Replaces `_row_exponential`/`row_exponential` (serve/fast_depth_kernels.py:82-98). */
int m3x_philox_exponential(const int32_t* seeds, const int32_t* ctrs, float* out, long ld_out, int level, int V, int B,
                           void* stream);

/* One raw Philox4x32-10 block (for known-answer tests); all pointers on the device. */
int m3x_philox_block(const uint32_t* counter, const uint32_t* key, uint32_t* out, void* stream);

/* ctr[slots[b]] += 1. Replaces `self.row_ctr.index_add_(...)` (serve/fast_depth.py:199). */
int m3x_ctr_add(int32_t* ctr, const int64_t* slots, int B, void* stream);

/* Feedback embedding: y[b] = RMSNorm(dt(dt(sum_l table[codes[b,l] + n_codes*l]) / scale)) (fp32 sum, one final
 * rounding); n in {1024, 2048}.
 * Replaces `audio_in.table(codes+offsets)` + `audio_in.norm(e.sum(1)/scale)` (serve/fast_depth.py:200-203,
 * tts/model/audio_io.py:27-35). */
int m3x_feedback(const void* table, const int32_t* codes, long s_codes, void* out, long s_out, const void* w, float eps,
                 float scale, int B, int n, int n_q, int n_codes, int dtype, void* stream);

/* Row copy with optional gather (src_idx[r]+src_off, clamped to [0, src_rows)) and scatter (dst_idx[r]) of n
 * 16-bit elements per row (n % 8 == 0); indices int64 or int32 (idx_i32) with stride ld_idx.
 * Replaces `F.embedding(code, self.embed[level])` (serve/fast_depth.py:135,196) and the engine's
 * `self.feedback[idx]` gather / `self.feedback[idx] = fb` scatter (maya3/engine.py:542,556). */
int m3x_copy_rows(const void* src, long ld_src, const void* src_idx, long src_off, long src_rows, void* dst,
                  long ld_dst, const int64_t* dst_idx, int rows, int n, int idx_i32, long ld_idx, void* stream);

/* dst[r, :n] = src[r, :n] converted between M3X_BF16, M3X_F16 and M3X_F32 (round to nearest even).
 * Replaces the dtype casts around the depth when it runs in another dtype than the backbone: the engine builds
 * FastDepth in `depth_dtype` (fp16 by default, maya3/engine.py:53,192-199) and feeds it the bf16 hidden state. */
int m3x_cast_rows(const void* src, long ld_src, int src_dtype, void* dst, long ld_dst, int dst_dtype, int rows, int n,
                  void* stream);

/* ring[(*head) % depth, b, :] = codes[b, :nq] for b < B, then *head += 1 (int32 [depth, seats, nq] ring).
 * Replaces the per-tick code readout (serve/fast_depth.py:137,257; maya3/engine.py:559-563) with a device ring. */
int m3x_code_ring_write(const int32_t* codes, long ld_codes, int32_t* ring, int32_t* head, int depth, int seats, int nq,
                        int B, void* stream);

/* ---- loop guard (maya3/guards.py:80-107 loop_detect_batch; engine tick maya3/engine.py:585-617) ------------ */

/* The code history of slot slots[b] (hist row of hist_len <= 256 int32 codes, oldest first, -1 = empty) shifts
 * left by one and takes codes[b * ld_codes] as its newest entry; frames[slots[b]] += 1 when frames is not NULL.
 * A slot repeated within one call (a graph bucket's padding rows on the dummy slot) gets an undefined row.
 * Replaces the host-side `s.hist[:-1] = s.hist[1:]; s.hist[-1] = cb0` and `frames += 1` (maya3/engine.py:579,
 * 585-586). */
int m3x_hist_push(int32_t* hist, long ld_hist, int64_t* frames, const int64_t* slots, const int64_t* codes,
                  long ld_codes, int B, int hist_len, void* stream);

/* out[r] = 0 (no loop), -1 (stall) or p (period) for history row slots[r] of W (newest last) with n[slots[r]]
 * frames (row r and n[r] when slots is NULL), with the
 * rules of loop_detect_batch: stall = the last `stall` codes all equal, given n >= max(12, stall); period = the
 * smallest p in [pmin, pmax] whose match fraction over the last period_win codes (count / (period_win - p), in
 * float64) is >= period_thr, given n >= max(12, stall, period_win). Limits: 1 <= stall <= 64, 2 <= period_win <= 64,
 * both <= hist_len; 1 <= pmin <= pmax < period_win.
 * Replaces `loop_detect_batch` (maya3/guards.py:80-107), which the engine runs on the host after the tick's copy. */
int m3x_loop_guard(const int32_t* W, long ld_w, const int64_t* slots, const int64_t* n, int32_t* out, int rows,
                   int hist_len, int stall, int period_win, double period_thr, int pmin, int pmax, void* stream);

/* ---- tick readout (maya3/engine.py:558-563) ---------------------------------------------------------------- */

/* int64 words per seat of m3x_tick_pack's row: 2 + with_loop + ceil(nq / 2) + ceil(frame / 4). */
int m3x_tick_pack_width(int with_loop, int nq, int frame);

/* Row b of out (ld_out int64 words): [stop[b], cb0[b], loop[b] (if loop), the nq codes of codes row b two int32 per
 * word, low first (if codes), frame PCM samples of pcm row b as int16(rint(clamp(x, -1, 1) * 32767)) four per word,
 * lowest first (if pcm)], for one pinned host copy per tick.
 * Replaces `pcm16 = (pcm.clamp(-1, 1) * 32767).round().to(torch.int16); packed = torch.cat([code, cb0, pcm16...])`
 * (maya3/engine.py:558-560). */
int m3x_tick_pack(const int64_t* stop, const int64_t* cb0, const int32_t* loop, const int32_t* codes, long ld_codes,
                  int nq, const float* pcm, long ld_pcm, int frame, int64_t* out, long ld_out, int B, void* stream);

/* ---- Mimi one-frame decode (serve/fast_codec.py StaticMimi :32-277) ------------------------------------------
 * Activations are time-major [seat * T + t, channels], 16-bit with fp32 arithmetic; `slots` names each seat's
 * state row (padding seats may all name the dummy row, whose contents are scratch). Stateful kernels take a
 * `chunk` of rows per workgroup that is at least the state's depth. */

/* out[b] = [table_0[codes[b,0]] | dt(sum_{q>=1} table_q[codes[b,q]])] from tables [nq, n_codes, dim]; codes outside
 * [0, n_codes) are clamped. With one GEMM by [W_semantic | W_acoustic] it replaces `_quantizer`/`_rvq`
 * (serve/fast_codec.py:134-149). */
int m3x_rvq_decode(const int64_t* codes, long ld_codes, const void* tables, void* out, long ld_out, int B, int nq,
                   int n_codes, int dim, int dtype, void* stream);

/* Depthwise transposed conv (kernel k <= 2 s, stride s, no bias) of one frame per seat: out [B * s, C] = the
 * frame's outputs plus the slot's tail; tail [slot, (k - s) * C] (frames x channels) becomes the new overlap.
 * Replaces `_layer(self.m.upsample, ...)` (serve/fast_codec.py:112-130,188). */
int m3x_dwconvt(const void* x, long ld_x, const void* w, void* tail, long ld_tail, const int64_t* slots, void* out,
                int B, int C, int k, int s, int dtype, void* stream);

/* GEMM rows of a causal conv: cols[b*T + t, j*C + c] = joined[t + j*dil][c], joined = the slot's (k-1)*dil stored
 * frames then ELU(x) (use_elu) or x; the state becomes joined's last (k-1)*dil frames. cols = NULL only advances
 * the state.
 * Replaces the MimiConv1d branch of `_layer` (serve/fast_codec.py:104-111) with the ELU in front of it. */
int m3x_conv_gather(const void* x, long ld_x, void* state, long ld_state, const int64_t* slots, void* cols,
                    long ld_cols, int B, int T, int C, int k, int dil, int use_elu, int chunk, int dtype,
                    void* stream);

/* out = act(res + scale * (g + bias)) per row ([rows, C], C % 8 == 0; bias, scale, res optional; act = ELU when
 * use_elu). Replaces the conv bias add, `shortcut + x` (serve/fast_codec.py:127-130) with the next ELU, and
 * `h + layer_scale(a)` (:181-182). */
int m3x_rows_op(const void* g, long ld_g, const void* bias, const void* scale, const void* res, long ld_res,
                void* out, long ld_out, int rows, int C, int use_elu, int dtype, void* stream);

/* h = dt(h + scale * a) (m3x_rows_op's arithmetic), then y = LayerNorm(h) (w, b, eps; fp32 statistics) over rows of
 * n = 512. Replaces `h = h + layer.self_attn_layer_scale(a)` / `h + layer.mlp_layer_scale(...)` followed by the
 * next `post_attention_layernorm` / `input_layernorm` (serve/fast_codec.py:172,181-182). */
int m3x_resid_ln(void* h, long ld_h, const void* a, long ld_a, const void* scale, const void* w, const void* b,
                 void* y, long ld_y, float eps, int rows, int n, int dtype, void* stream);

/* y = act(res + (dt(x . w^T) + bias)) for N in {16, 32, 64, 128} output channels, w packed by m3x_pack_weight,
 * K % 32 == 0; bias and res optional; act = ELU when use_elu. The product of m3x_linear followed by the arithmetic
 * of m3x_rows_op in one launch. Replaces a SEANet MimiConv1d's `module.conv(x)` with its bias, the resnet
 * `shortcut + x` and the next ELU (serve/fast_codec.py:104-111,127-130) when the conv has at most 128 outputs.
 * With C > 0 the product's rows are m3x_conv_gather's (K = k * C; x [M, C], M = B * T; the slot's history
 * `state`, the ELU in front when pre_elu) read in place of a gathered copy; the caller then advances the history
 * with m3x_conv_gather(cols = NULL). C = 0: x is the [M, K] product input itself. */
int m3x_conv_gemm(const void* x, long ldx, const void* w_packed, const void* bias, const void* res, long ld_res,
                  void* y, long ldy, int M, int N, int K, int use_elu, const void* state, long ld_state,
                  const int64_t* slots, int T, int C, int dil, int pre_elu, int dtype, void* stream);

/* Overlap-add of a transposed conv (kernel k, stride s, s < k <= 2 s) from its GEMM columns cols[b*Tin + t,
 * j*C + c]: out [B * Tin * s, C] with the slot's tail added to the first k - s frames and bias; the new tail is the
 * overflow without bias. Replaces the MimiConvTranspose1d branch of `_layer` (serve/fast_codec.py:112-126). */
int m3x_convt_overlap(const void* cols, long ld_cols, void* tail, long ld_tail, const int64_t* slots,
                      const void* bias, void* out, long ld_out, int B, int Tin, int C, int k, int s, int chunk,
                      int dtype, void* stream);

/* Sliding-window attention of T <= 2 new tokens per seat at positions tokens[slot] + t over the slot's ring
 * (kring/vring [slots, ring, H, 64] post-RoPE, key_pos [slots, ring]); RoPE angle pos * inv_freq[i] (fp32),
 * cos/sin times rope_scale; ring <= 256, ring >= window + T - 1. Replaces the ring writes, mask, RoPE and SDPA of
 * `_transformer` (serve/fast_codec.py:157-180). */
int m3x_ring_attn(const void* qkv, long ld_qkv, void* kring, void* vring, int64_t* key_pos, const int64_t* tokens,
                  const int64_t* slots, const float* inv_freq, float rope_scale, void* out, long ld_out, int B, int T,
                  int H, int head_dim, int ring, int window, int dtype, void* stream);

/* tokens[slot] += T for each seat whose slot is not `dummy` (those slots distinct, one seat each), then
 * tokens[dummy] = 0.
 * Replaces `self.tokens.index_copy_(0, slots, start + count); self.tokens[self.dummy].zero_()` (:183-184). */
int m3x_advance_tokens(int64_t* tokens, const int64_t* slots, int B, int T, int dummy, void* stream);

/* Last conv (C -> 1 channel, kernel k, causal; C % 8 == 0, k * C <= 4096) to fp32 PCM [B, T] with fp32 weights
 * w[j*C + c] and the slot's k - 1 stored input frames; chunk (>= k - 1) is the samples per workgroup of the
 * general path (C <= 64 and k <= 9 take a fixed 128). Replaces the final MimiConv1d of `_forward` (serve/fast_codec.py:189-191). */
int m3x_final_conv(const void* x, long ld_x, void* state, long ld_state, const int64_t* slots, const float* w,
                   float bias, float* pcm, long ld_pcm, int B, int T, int C, int k, int chunk, int dtype,
                   void* stream);

/* ---- the depth frame over a run of continuing levels as one persistent kernel (serve/fast_depth.py:143-203) -- */

/* Arguments of m3x_depth_run: levels L0 .. L1-1, each continuing the weight group of level L0 - 1 (one position
 * per seat per level, T = 1), for B <= 16 seats. Trunk geometry: width 1024, H heads of hd in {128 (SwiGLU, act
 * M3X_ACT_SWIGLU, F 2816), 64 (GELU, act M3X_ACT_GELU, F 3072)}, `layers` <= 4 layers, codebooks of 2048 codes.
 * Weights are packed (m3x_pack_weight): per layer q|k|v [3*1024, 1024], o [1024, 1024], gate (or f1) [F, 1024],
 * up [F, 1024] (SwiGLU only), down [1024, F]; heads[L-1] [2048, 1024] for each level L of the run. Norms: kind
 * M3X_NORM_RMS (weights) with SwiGLU, M3X_NORM_LAYER (weights and biases) with GELU (other pairings:
 * M3X_EUNSUPPORTED), per-layer eps, and the final norm.
 * State: prefix[b * ld_prefix + p * 1024 ...] holds position L0's input row; the sampled code of level L goes to
 * codes[b * ld_codes + L] and, for L < 31, the next prefix row embed[L][code] to prefix position L + 1. kd/vd
 * [B][H][32][hd] per layer hold the group's K/V at positions < L0. u[b * ld_u + L - 1] is the uniform of level L.
 * xchg: m3x_depth_run_xchg_bytes() of device memory, zeroed before the first run and then left to the kernel;
 * sync: 4 int32, zeroed before the first run (the kernel keeps an epoch in [0], a counter in [1] and sets [2]
 * to 1 if a step's input never arrived, in which case the run's outputs are void; the word stays set until the
 * caller clears it). nwg must equal 256, and the device must hold all 256 workgroups at once (its CUs times the
 * kernel's workgroups per CU; else M3X_EUNSUPPORTED), since every workgroup waits on others. logits_out
 * (nullable): [31][B][2048] copy of the head outputs. prof (nullable): [256][2048] real-time counter stamps of
 * every workgroup's steps (profiling). probe: a poll of more 16-byte chunks per thread than this first waits on one
 * chunk per thread (fewer: every chunk each round). spin_limit: polling rounds before a wait gives up (0: 2^19;
 * a test passes a small one to make the waits give up while every workgroup still exits). */
typedef struct M3xDepthRun {
  int B, L0, L1, layers, H, hd, F, V, act, norm_kind, dtype, nwg;
  float inv_temp;
  int top_k, greedy;
  float eps1[4], eps2[4], eps_f;
  const void* n1w[4];
  const void* n1b[4];
  const void* n2w[4];
  const void* n2b[4];
  const void* fw;
  const void* fb;
  const void* wqkv[4];
  const void* wo[4];
  const void* wg[4];
  const void* wu[4];
  const void* wd[4];
  const void* heads[31];
  const void* embed;
  const void* cross;
  long ld_cross;
  void* prefix;
  long ld_prefix;
  int32_t* codes;
  long ld_codes;
  const float* u;
  long ld_u;
  const void* kd[4];
  const void* vd[4];
  long kv_sb, kv_sh;
  uint64_t* xchg;
  int32_t* sync;
  void* logits_out;
  uint64_t* prof;
  int probe;
  unsigned spin_limit;
} M3xDepthRun;

/* Bytes of the exchange area and of M3xDepthRun (a binding checks its layout against the latter). */
size_t m3x_depth_run_xchg_bytes(void);
size_t m3x_depth_run_args_bytes(void);

/* Launch the run described by *args (read on the host during the call; the kernel gets a copy).
 * Replaces the per-level loop of `_compute_fused` for continuing levels (serve/fast_depth.py:150-155 attention
 * over the within-group K/V, :179-190 the layers, :191-198 head, sampling and next prefix). */
int m3x_depth_run(const M3xDepthRun* args, void* stream);

/* After a run, in stream order: when the run's error word (sync[2]) is set, codes[b][L0 .. L1-1] = -1 for b < B.
 * A failed run's codes are void; every consumer of codes clamps them, and the host readouts raise on the sentinel.
 * The reference turns a GPU-side failure into an exception that fails the engine (maya3/engine.py:375-385). */
int m3x_depth_run_void(const int32_t* sync, int32_t* codes, long ld_codes, int B, int L0, int L1, void* stream);

/* ---- the one-row backbone decode as one persistent kernel (serve/fast_backbone.py:176-234) ------------------ */

/* Per layer: the packed weights as StaticBackbone packs them (q|k|v [4096, 1024] plain at layer 0 and with the input
 * RMSNorm weight folded in after it, o [1024, 2048], gate and up [3072, 1024] with the post-attention RMSNorm
 * weight folded in, down [1024, 3072]), the q/k norm weights [128] and the layer's caches [slots][8][cap][128]. */
typedef struct M3xBackboneLayer {
  const void* wqkv;
  const void* wo;
  const void* wg;
  const void* wu;
  const void* wd;
  const void* wq;
  const void* wk;
  void* kc;
  void* vc;
} M3xBackboneLayer;

/* Arguments of m3x_backbone_run: one decode row of the Qwen3-0.6B-shaped backbone (hidden 1024, 16 q / 8 kv heads
 * of 128, SwiGLU 3072, bf16) through `layers` layers. layer: a DEVICE array of M3xBackboneLayer. x [1024] is the
 * row's input; the last layer's residual goes to h_out [1024] (the caller's final norm reads it). slots[0] and
 * pos[0] (device) give the row's slot and position (0 <= pos < cap <= 4096); its key and value are written at pos
 * of every layer's caches (strides sk_s, sk_h, sk_t in elements), RoPE from cos/sin [cap][128] (row stride s_cos),
 * w_in0 the layer-0 input RMSNorm weight, eps the RMSNorm epsilon (also of the q/k norms), scale = 128^-0.5.
 * xchg: m3x_backbone_run_xchg_bytes() of device memory zeroed once; sync: 4 int32 zeroed once ([0] epoch, [1] a
 * counter, [2] set to 1 if a step's input never arrived within spin_limit polling rounds (0: 2^19), in which case
 * h_out is not written). nwg must equal 256 and the device must hold all of them at once (else M3X_EUNSUPPORTED).
 * probe: as M3xDepthRun's. prof (nullable): [256][512] real-time counter stamps of every workgroup's steps.
 * w_fin: the final RMSNorm weight [1024]; y_out [1024] receives the final norm of h_out (the add+norm kernels'
 * arithmetic). At the run's end lengths[slots[0]] += real[0] (int64), whether or not the run failed. */
typedef struct M3xBackboneRun {
  const M3xBackboneLayer* layer;
  int layers, cap, nwg, probe;
  unsigned spin_limit;
  float eps, scale;
  const void* x;
  void* h_out;
  const int64_t* slots;
  const int32_t* pos;
  const void* cos;
  const void* sin;
  long s_cos;
  const void* w_in0;
  long sk_s, sk_h, sk_t;
  uint64_t* xchg;
  int32_t* sync;
  uint64_t* prof;
  const void* w_fin;
  void* y_out;
  int64_t* lengths;
  const int64_t* real;
} M3xBackboneRun;

/* Bytes of the exchange area, of M3xBackboneRun and of M3xBackboneLayer (a binding checks its layouts). */
size_t m3x_backbone_run_xchg_bytes(void);
size_t m3x_backbone_run_args_bytes(void);
size_t m3x_backbone_run_layer_bytes(void);

/* Launch the run (args read on the host during the call). Replaces, for a one-row step, the layer loop of
 * `StaticBackbone._forward` (serve/fast_backbone.py:187-203: q|k|v, `_qk_norm_rope_cache`, `_decode_attn`, o, the
 * add+norms, gate|up, SwiGLU, down), its final norm (:229-232) and the length update (:233). */
int m3x_backbone_run(const M3xBackboneRun* args, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* M3X_H */
