/* libkoptim: C ABI of the MI355X (gfx950) decode-path kernels.
 *
 * Every entry point:
 *   - takes device pointers, plain integer sizes/strides (in elements) and an
 *     opaque hipStream_t (void*); no framework types cross this boundary;
 *   - enqueues its kernels on `stream`, allocates nothing, never synchronises
 *     (safe to record into a hipGraph);
 *   - returns 0 on success, a positive hipError_t if a launch failed, or a
 *     negative code if an argument was rejected on the host before launching:
 *       KO_EINVAL (-22) invalid pointer/size/alignment,
 *       KO_ERANGE (-34) a buffer too small for the requested shape,
 *       KO_ENOTSUP (-95) a shape the library does not serve (e.g. head_dim != 128).
 * bf16 tensors are passed as void* to their raw 16-bit storage.
 */
#ifndef KOPTIM_H
#define KOPTIM_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---- split-K GQA decode attention --------------------------------------
 * Replaces engine/kernels/fused.py:138-185 (_decode_attn_kernel) as launched by
 * DecodeAttention.__call__ (fused.py:221-230).
 * q        [B*T, nq*head_dim] bf16, row (b*T + t), nq = 4*nkv.
 * k_cache, v_cache: one layer [B, nkv, cap, head_dim] bf16, batch/head strides
 *          given, sequence stride head_dim, inner stride 1.
 * kv_lens  [B] int32 on the device; valid keys of sequence b are
 *          kv_lens[b] + len_offset (the reference passes pos with T: offset T).
 *          Query t sits at position valid-T+t and sees keys < valid-T+t+1.
 * unit     keys per work unit (multiple of 16); max_units*unit >= cap. Each unit
 *          leaves one fp32 partial slot per query row.
 * grid_waves  number of wavefronts launched (they take the units in rounds; with
 *          T == 1, 2-64 sequences and more than one round, the full units first and
 *          the part-filled last units by decreasing size, forward and backward over
 *          the workgroups in alternate rounds). With
 *          T == 1 a unit is split over the wavefronts of one workgroup: 4 when
 *          unit % 64 == 0, else 2 when unit % 32 == 0, else 1, so grid_waves
 *          should be a multiple of that count.
 * o_part   [B*T*nq*max_units*head_dim] fp32 scratch, ml [B*T*nq*max_units*2] fp32.
 * T in 1..8 (T > 4 runs as two launches of 2-4 query tokens), head_dim 128. */
int ko_decode_attn_partial(const void* q, const void* k_cache, const void* v_cache,
                           const int* kv_lens, int len_offset, int cap,
                           long long cache_b_stride, long long cache_h_stride, int B, int T,
                           int nkv, int head_dim, int unit, int max_units, int grid_waves,
                           float scale, float* o_part, float* ml, void* stream);

/* Log-sum-exp merge of the partials into out [B*T, nq*head_dim] bf16.
 * Replaces engine/kernels/fused.py:188-201 (_decode_combine_kernel), launched at
 * fused.py:231-234. */
int ko_decode_attn_combine(const float* o_part, const float* ml, const int* kv_lens,
                           int len_offset, int cap, int B, int T, int nq, int head_dim,
                           int unit, int max_units, void* out, void* stream);

/* The whole of DecodeAttention.__call__ (fused.py:221-234). With counters == NULL:
 * ko_decode_attn_partial followed by ko_decode_attn_combine, the reference's
 * two launches. With counters ([B*nkv] int32, zero before the first call;
 * every call leaves them zero) it is one launch per group of up to 4 query
 * tokens: the last work unit of each (sequence, KV head) merges that pair's
 * partials. The partials and the arrival count travel through device-coherent
 * (agent-scope) stores, loads and atomics; no fence or L2 write-back. */
int ko_decode_attn(const void* q, const void* k_cache, const void* v_cache, const int* kv_lens,
                   int len_offset, int cap, long long cache_b_stride, long long cache_h_stride,
                   int B, int T, int nkv, int head_dim, int unit, int max_units, int grid_waves,
                   float scale, float* o_part, float* ml, int* counters, void* out,
                   void* stream);

/* ko_decode_attn in its two-launch form (partials, then the log-sum-exp
 * combine) with no caller scratch and no allocation: the fp32 partials live in
 * a fixed 16 MiB device array of the library (one per GPU, held until the
 * process ends; its address is looked up on the first call on each device,
 * which may itself be made under graph capture). No counterpart in the reference: for callers that cannot allocate (code
 * under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Rejects with KO_ERANGE, before launching anything, a call whose
 * partials exceed the array: B*T*nq*max_units*(head_dim + 2) floats (plus up
 * to 63 of alignment) must fit in 4,194,304, e.g. B = 16 with 8192-key caches
 * and 4096-key units, or B = 1 with up to 1000 units. Every call on a GPU uses
 * that GPU's one array: calls that overlap on one GPU (other streams, other
 * threads) race and must be ordered by the caller. Other arguments as for
 * ko_decode_attn. */
int ko_decode_attn_noalloc(const void* q, const void* k_cache, const void* v_cache,
                           const int* kv_lens, int len_offset, int cap, long long cache_b_stride,
                           long long cache_h_stride, int B, int T, int nkv, int head_dim, int unit,
                           int max_units, int grid_waves, float scale, void* out, void* stream);

/* DecodeAttention.__call__ for T = 2..8 query tokens per sequence (the verify
 * step, engine/engine.py:409-411 with fused.py:221-234), computed as B*T rows of
 * the one-token kernel: row b*T + t attends keys 0 .. pos[b] + t of sequence b
 * (causal within the block, as ko_decode_attn with T tokens), and the last work
 * unit of each (row, KV head) merges that row's partials (counters [B*T*nkv]
 * int32, zero before the first call, left zero). o_part / ml are sized for
 * B*T rows. Same results as ko_decode_attn to fp32 rounding; one launch. */
int ko_decode_attn_token_rows(const void* q, const void* k_cache, const void* v_cache,
                              const int* pos, int cap, long long cache_b_stride,
                              long long cache_h_stride, int B, int T, int nkv, int head_dim,
                              int unit, int max_units, int grid_waves, float scale,
                              float* o_part, float* ml, int* counters, void* out, void* stream);

/* One decode step of attention straight from the bf16 QKV projection
 * qkv [B, (nq+2nkv)*head_dim] (T = 1): per-head q/k RMSNorm (gains q_w, k_w,
 * eps) and RoPE (cos/sin [max_pos, head_dim] bf16) at position pos[b], append
 * of k and v to cache slot pos[b], attention over keys 0..pos[b], and the
 * combine into out [B, nq*head_dim] (a second launch, or the fused last-unit
 * merge when counters != NULL, as for ko_decode_attn). Replaces the pair
 * qk_norm_rope (engine/kernels/fused.py:54-106) + DecodeAttention.__call__
 * (fused.py:221-234) as the reference's decode step calls them
 * (engine/engine.py:328-330). Positions must lie in [0, min(cap, max_pos)).
 * rope (optional, [B][2][head_dim] bf16, 16-byte aligned): the cos and sin rows
 * at pos[b] as ko_rope_rows writes them; the kernel then reads them instead of
 * the table rows behind the position, and for B == 1 (with a unit per
 * workgroup) issues its first loads before it reads the position.
 * units_per_seq = 0: units of `unit` keys. units_per_seq = U > 0 (counters
 * given, B <= 64, unit % 64 == 0): each sequence's pos[b] + 1 keys are cut
 * into at most U units of equal size, rounded up to a multiple of 64 and at
 * least `unit` keys, from its length at this step (max_units * unit >= cap
 * still sizes the partials). */
int ko_decode_attn_qkv(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                       const void* sin, int max_pos, const int* pos, void* k_cache,
                       void* v_cache, int cap, long long cache_b_stride,
                       long long cache_h_stride, int B, int nkv, int head_dim, int unit,
                       int max_units, int grid_waves, float eps, float scale, float* o_part,
                       float* ml, int* counters, void* out, const void* rope,
                       int units_per_seq, void* stream);

/* ko_decode_attn_qkv (with counters) and the o projection with its residual add
 * in ONE launch, for B <= 2 and unit % 64 == 0 (4 wavefronts per unit) and an
 * o-projection input width nq*head_dim <= 4096: out [B, nq*head_dim] receives
 * the merged attention output as before, and h [B, H] <- bf16(h + bf16(out @
 * w_o^T)) (w_o [H, nq*head_dim] bf16), the RESID GEMV of engine/engine.py:330-331
 * (kernels/gemv.py EPI_RESID), bit-identical to the separate launches. Extra
 * workgroups own 8 columns of the projection each; they load their weights while
 * the attention runs, and each wavefront reads the slice of the merged output
 * of a (sequence, KV head) pair once that pair's done flag is raised.
 * sync: ko_decode_attn_qkv_oproj_sync_ints() int32, 8-byte aligned, zero before
 * the first call; it carries a launch epoch from call to call (zeroing it again
 * between calls is allowed). err [1] int32 is set to 1 if a wait gave up
 * (never expected; the results of such a call are invalid) and stays set until
 * the caller clears it. spin_max: polls of a done flag before a wait gives up
 * (< 0: the library's bound, 2^21 polls of ~1 us; 0: give up at once, for tests
 * of that path). delay_ns: how long the projection workgroups hold their weight
 * loads so the attention's first loads go ahead of them (0: no delay). rope: as
 * for ko_decode_attn_qkv. Replaces engine.py:328-332 (attention, o projection
 * and its residual add); no single reference function. */
int ko_decode_attn_qkv_oproj(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                             const void* sin, int max_pos, const int* pos, void* k_cache,
                             void* v_cache, int cap, long long cache_b_stride,
                             long long cache_h_stride, int B, int nkv, int head_dim, int unit,
                             int max_units, int grid_waves, float eps, float scale,
                             float* o_part, float* ml, int* counters, void* out,
                             const void* w_o, void* h, int H, int* sync, int* err,
                             int delay_ns, int spin_max, const void* rope, void* stream);

/* int32 elements of ko_decode_attn_qkv_oproj's sync array (a size, not a status). */
long long ko_decode_attn_qkv_oproj_sync_ints(void);

/* out[b] = (cos[p], sin[p]), p = clamp(pos[b], 0, rows - 1): each sequence's
 * RoPE rows at its new position for the rope argument above (the rows that
 * qk_norm_rope, engine/kernels/fused.py:71-87, reads). cos/sin [rows, d] bf16,
 * out [B][2][d]; d % 8 == 0; 16-byte aligned. No reference counterpart: the
 * reference reads the rows inside qk_norm_rope. */
int ko_rope_rows(const int* pos, const void* cos, const void* sin, int rows, int d, int B,
                 void* out, void* stream);

/* ---- residual add + RMSNorm ---------------------------------------------
 * Replaces engine/kernels/fused.py:16-36 (_add_rms_norm_kernel) as launched by
 * add_rms_norm (fused.py:39-46). res [rows, n] bf16 (updated in place to
 * bf16(res + delta) when delta != NULL), weight [n], out [rows, n];
 * out = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))). n % 8 == 0, n <= 8192. */
int ko_add_rms_norm(void* res, const void* delta, const void* weight, void* out, int rows, int n,
                    float eps, void* stream);

/* ---- per-head q/k RMSNorm + RoPE + KV-cache append ----------------------
 * Replaces engine/kernels/fused.py:54-96 (_qk_norm_rope_kernel) as launched by
 * qk_norm_rope (fused.py:99-106). qkv [M, (nq+2nkv)*d] bf16, M = B*T; row m is
 * sequence m/T at position pos[m/T] + m%T. Writes q_out [M, nq*d], and k
 * (normed + roped) / v (raw) into one cache layer [B, nkv, cap, d] at that
 * position. cos/sin [rows, d] bf16 tables. Positions outside [0, max_pos)
 * (max_pos = min(cap, table rows)) are skipped. d == 128. */
int ko_qk_norm_rope(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                    const void* sin, const int* pos, void* q_out, void* k_cache, void* v_cache,
                    int M, int T, long long cache_b_stride, long long cache_h_stride, float eps,
                    int nq, int nkv, int d, int max_pos, void* stream);

/* Same from the fp32 QKV accumulator acc [B, (nq+2nkv)*d] (T = 1): rounds it to
 * bf16 first, re-zeroes it, and zeroes zero_buf[0..n_zero).
 * Replaces engine/kernels/gemv.py:219-268 (_qk_norm_rope_acc_kernel) as launched
 * by qk_norm_rope_acc (gemv.py:271-277). */
int ko_qk_norm_rope_acc(float* acc, const void* q_w, const void* k_w, const void* cos,
                        const void* sin, const int* pos, void* q_out, void* k_cache,
                        void* v_cache, float* zero_buf, int n_zero, int B,
                        long long cache_b_stride, long long cache_h_stride, float eps, int nq,
                        int nkv, int d, int max_pos, void* stream);

/* ---- SwiGLU ---------------------------------------------------------------
 * Replaces engine/kernels/fused.py:112-120 (_silu_mul_kernel) as launched by
 * silu_mul (fused.py:123-127): gu [M, 2I] (gate | up) bf16 ->
 * out [M, I] = bf16(bf16(silu(gate)) * up). I % 8 == 0. */
int ko_silu_mul(const void* gu, void* out, int M, int I, void* stream);

/* ---- embedding gather + sum of squares ------------------------------------
 * Replaces engine/kernels/gemv.py:201-211 (_embed_ss_kernel) as launched by
 * embed_ss (gemv.py:214-216): h[m] = emb[ids[m]] ([V, H] bf16, ids int64),
 * ss[m] = sum(h[m]^2) fp32 (ss may be NULL). Ids outside [0, V) gather zeros. */
int ko_embed_ss(const long long* ids, const void* emb, void* h, float* ss, int M, int H, int V,
                void* stream);

/* ---- fused skinny GEMM ------------------------------------------------------
 * Replaces engine/kernels/gemv.py:30-106 (_gemv_kernel) as launched by
 * Gemv.__call__ (gemv.py:140-150): y[M, N] = x[M, K] @ W[N, K]^T, bf16 in,
 * fp32 accumulate, every weight read once for all M rows.
 * norm != 0: x <- bf16(nw * bf16(x * rsqrt(ss/K + eps))); ss == NULL computes
 *            the row sums of squares from x.
 * epi 0 F32    y fp32 [M, N] (stored; atomically added if accumulate != 0)
 *     1 BF16   y bf16 [M, N]
 *     2 RESID  h [M, N] bf16 <- bf16(h + bf16(acc)); ss_out[m] += sum(h^2) if given
 *     3 SWIGLU w [2N, K] (gate | up); y bf16 = bf16(bf16(silu(bf16 g)) * bf16 u)
 *     4 ARGMAX ids[m] (int64) = argmax_n bf16(acc) with lowest index on ties
 *              (torch.argmax at engine/engine.py:291, fused into the LM head);
 *              bf16 logits stored in y when y != NULL; pos_inc[m] += 1 when
 *              pos_inc != NULL (the step's position advance, engine.py:292);
 *              next_h[m] = next_emb[ids[m]] ([N, K] table) when both are given
 *              (the next step's embedding gather, gemv.py:201-211);
 *              part: fp32 scratch of part_len >= ko_gemv_argmax_scratch(...).
 * layout 0: each 256-thread workgroup owns `rows` (4 or 8; 16 when M <= 2)
 *           columns; any M.
 * layout 1: each wavefront owns `rows` (1, 2, 4) columns, `waves` (2, 4)
 *           wavefronts per workgroup; M <= 4 per launch slice.
 * layout 2: MFMA 16-column tiles, M <= 16 per launch slice (rows padded with
 *           zeros), K in {2560, 4096, 9728} (SWIGLU: 2560, 4096); a persistent
 *           grid of at most 256 * `rows` (1, 2 or 4) workgroups, the fewest
 *           that keep the most tiles per workgroup at its minimum (384 tiles:
 *           192 workgroups of 2). `waves` 0, or 2 for two row tiles: M <= 32
 *           per launch slice, each weight load feeding both tiles (K in
 *           {2560, 4096}, SWIGLU 2560; a last slice of <= 16 rows runs on one
 *           tile). w must be in the tiled
 *           layout written by ko_gemv_tile (for SWIGLU: the gate rows tiled,
 *           then the up rows tiled, each padded to a multiple of 16 rows).
 * layout 3: layout 2's tiles and weight copy with the K range of a tile cut
 *           into `rows` slices (K = 128 * S * rows, S in {20, 19, 8, 4}), one
 *           4-wavefront workgroup per (tile, slice); the last slice of a tile
 *           to arrive adds the slices' fp32 partial tiles in slice order
 *           (deterministic) and runs the epilogue. No ARGMAX; NORM only with
 *           S = 20 and, for rows > 1, ss given. For rows > 1, part is its
 *           scratch (part_len >= ko_gemv_argmax_scratch(N, 3, rows, 0)): zero
 *           before the first call, left zero by every call (the tiles' arrival
 *           counters); calls that share it must not overlap.
 * layout 4: layout 2's tiles and weight copy with each tile cut into 16 K
 *           chunks of S steps (K = 512 * S, S in {19, 8, 5}); the chunks of all
 *           tiles are dealt out in order, one per wavefront, `rows` = 10 per
 *           workgroup, so every workgroup streams the same bytes; the last of
 *           a tile's workgroups adds their fp32 partial tiles in workgroup
 *           order (deterministic) and runs the epilogue. F32, BF16 or RESID, no
 *           NORM. `waves` 0, or 2 / 4 for two / four row tiles (M <= 32 / 64
 *           per launch slice, x of every tile loaded per K step with the
 *           weights; a slice runs on the fewest tiles that hold it). part is its
 *           scratch (part_len >= ko_gemv_argmax_scratch(N, 4, 10, waves)), with
 *           the rules of layout 3's.
 * K % 8 == 0. M larger than a slice is processed in several launches. */
int ko_gemv(const void* x, const void* w, void* y, const void* nw, const float* ss, void* h,
            float* ss_out, long long* ids, int* pos_inc, const void* next_emb, void* next_h,
            float* part, long long part_len, int M, int N, int K, int epi, int norm,
            int accumulate, int layout, int rows, int waves, float eps, void* stream);

/* The decode step's tail in one call: the LM head GEMV with the greedy argmax
 * (ko_gemv with epi 4, ARGMAX, and a NORM prologue when nw != NULL), followed
 * by the step's bookkeeping. Replaces engine/engine.py:290-292 (the LM head
 * GEMV, torch.argmax into ids, pos += 1) together with the per-token
 * device-to-host copy of ids into pinned memory (engine.py:437,516).
 * logits (bf16 [M, N]) may be NULL; ids [M] int64; pos [M] int32 is advanced.
 * next_emb/next_h: the next step's embedding gather, as for ko_gemv.
 * rope (optional, [M][2][head_dim] bf16, 16-byte aligned): receives the cos and
 * sin rows of cos/sin [max_pos, head_dim] at the advanced position (clamped to
 * [0, max_pos)), the rows ko_decode_attn_qkv(_oproj) take as `rope` in the
 * next step (what ko_rope_rows writes).
 * ring (optional, [ring_rows, M] int64 in pinned host memory): row
 * ring_ctr[m] (int32 on the device, in [0, ring_rows)) receives ids[m] with a
 * system-scope store and ring_ctr[m] advances by one, wrapping to 0; a host
 * that waits for the stream then reads the ids without a copy. err (optional,
 * with the ring; int32 on the device): while *err is nonzero (the err flag of
 * ko_decode_attn_qkv_oproj, set when a wait of that launch gave up and kept
 * until the caller clears it) the ring receives -2 in place of the ids, so a
 * host reading the ring sees the failure at the step where it happened.
 * Layouts, scratch (part) and the other arguments as for ko_gemv. */
int ko_lm_head_argmax(const void* x, const void* w, const void* nw, const float* ss, void* logits,
                      long long* ids, int* pos, const void* next_emb, void* next_h,
                      const void* cos, const void* sin, int max_pos, int head_dim, void* rope,
                      long long* ring, int ring_rows, int* ring_ctr, const int* err,
                      float* part, long long part_len, int M, int N, int K, int layout, int rows,
                      int waves, float eps, void* stream);

/* Number of fp32 scratch elements ko_gemv needs for N columns with this launch
 * configuration: the ARGMAX partials (epi 4) of layouts 0-2, or layout 3's
 * (rows > 1) and layout 4's slots and counters. A size, not a status; -1 for
 * bad arguments.
 * Helper of ko_gemv, no reference counterpart. */
long long ko_gemv_argmax_scratch(int N, int layout, int rows, int waves);

/* Replaces torch.argmax(logits, dim=-1, out=vout) of the speculative verify
 * step (engine/engine.py:413-415): ids[m] = argmax_n x[m, n] over bf16 logits
 * [M, N] with row stride ld elements (ld % 8 == 0, x 16-byte aligned), lowest
 * index on ties. One workgroup per row; no memset, so it can be captured in a
 * graph. */
int ko_argmax_rows(const void* x, long long ld, int M, int N, long long* ids, void* stream);

/* Re-lays a row-major bf16 weight w [rows, K] into the tiled layout of ko_gemv
 * layout 2: wt holds ceil(rows/16)*16*K elements; for row tile t and k step s
 * (32 columns) the 1 KiB block at element ((t * K/32 + s) * 64 + l) * 8 holds,
 * for l = 0..63, row 16 t + l % 16, columns 32 s + 8 (l / 16) .. + 7 (zeros past
 * the last row). K % 32 == 0. A one-time transform at weight load; no reference
 * counterpart (the reference's Triton GEMV reads its row-major weights). */
int ko_gemv_tile(const void* w, void* wt, int rows, int K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KOPTIM_H */
