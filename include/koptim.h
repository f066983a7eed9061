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
 *       KO_ENOTSUP (-95) a shape this build does not serve (e.g. head_dim != 128).
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
 * unit     keys per work unit (multiple of 16); max_units*unit >= cap.
 * grid_waves  number of wavefronts launched (they stride over the units).
 * o_part   [B*T*nq*max_units*head_dim] fp32 scratch, ml [B*T*nq*max_units*2] fp32.
 * T in 1..4, head_dim 128. */
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

/* Both passes: the whole of DecodeAttention.__call__ (fused.py:221-234). */
int ko_decode_attn(const void* q, const void* k_cache, const void* v_cache, const int* kv_lens,
                   int len_offset, int cap, long long cache_b_stride, long long cache_h_stride,
                   int B, int T, int nkv, int head_dim, int unit, int max_units, int grid_waves,
                   float scale, float* o_part, float* ml, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KOPTIM_H */
