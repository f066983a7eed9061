// Row kernels around the decode GEMVs, for gfx950.
//
// Each kernel restates the cast chain of the reference kernel it replaces
// (all arithmetic fp32, bf16 rounds exactly where the reference rounds):
//   ko_add_rms_norm      engine/kernels/fused.py:16-46
//   ko_qk_norm_rope      engine/kernels/fused.py:54-106  (bf16 qkv, T tokens/sequence)
//   ko_qk_norm_rope_acc  engine/kernels/gemv.py:219-277  (fp32 QKV accumulator, T=1)
//   ko_silu_mul          engine/kernels/fused.py:112-127
//   ko_embed_ss          engine/kernels/gemv.py:201-216
#include "ko_common.h"

using namespace ko;

namespace {

constexpr int NT = 256;

__device__ __forceinline__ float block_sum(float v, float* red) {
  // red: NT/64 floats of shared memory
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

// ---- residual add + RMSNorm: one workgroup per row -------------------------
// Up to 4 16-byte chunks per thread (n <= 8192).
__global__ __launch_bounds__(NT) void add_rms_norm_kernel(uint16_t* __restrict__ res,
                                                          const uint16_t* __restrict__ delta,
                                                          const uint16_t* __restrict__ wt,
                                                          uint16_t* __restrict__ out, int n,
                                                          float eps) {
  __shared__ float red[NT / 64];
  const long long row = blockIdx.x;
  const int nc = n >> 3;
  uint16_t* rp = res + row * n;
  const uint16_t* dp = delta ? delta + row * n : nullptr;
  uint16_t* op = out + row * n;
  float xs[4][8];
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + i * NT;
    if (c < nc) {
      uint4 xv = ldg16(rp + 8 * c);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
      float x[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = bf16lo(xw[e]);
        x[2 * e + 1] = bf16hi(xw[e]);
      }
      if (dp) {
        uint4 dv = ldg16(dp + 8 * c);
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // hidden = residual + hidden, rounded to bf16 (fused.py:27-30)
          x[2 * e] = round_bf16(x[2 * e] + bf16lo(dw[e]));
          x[2 * e + 1] = round_bf16(x[2 * e + 1] + bf16hi(dw[e]));
          o[e] = pack_bf16x2(x[2 * e], x[2 * e + 1]);
        }
        *reinterpret_cast<uint4*>(rp + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xs[i][e] = x[e];
        sq += x[e] * x[e];
      }
    }
  }
  const float var = block_sum(sq, red) / (float)n;
  const float rstd = rsqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + i * NT;
    if (c < nc) {
      uint4 wv = ldg16(wt + 8 * c);
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // bf16(w * bf16(x * rstd)) (fused.py:33-35)
        const float y0 = bf16lo(ww[e]) * round_bf16(xs[i][2 * e] * rstd);
        const float y1 = bf16hi(ww[e]) * round_bf16(xs[i][2 * e + 1] * rstd);
        o[e] = pack_bf16x2(y0, y1);
      }
      *reinterpret_cast<uint4*>(op + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// ---- per-head RMSNorm + RoPE + KV append: one wavefront per (row, head) -----
// Lane l owns head-dim elements 2l, 2l+1; its rotate_half partner is lane l^32.
template <bool ACC>
__global__ __launch_bounds__(NT) void qk_norm_rope_kernel(
    const void* __restrict__ src, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, const uint16_t* __restrict__ cosb,
    const uint16_t* __restrict__ sinb, const int* __restrict__ pos,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ kcache, uint16_t* __restrict__ vcache,
    float* __restrict__ zero_buf, int n_zero, int M, int T, long long cb, long long ch,
    float eps, int nq, int nkv, int max_pos) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
  const int nh = nq + 2 * nkv;
  if (ACC && zero_buf && blockIdx.x == 0) {
    for (int i = threadIdx.x; i < n_zero; i += NT) zero_buf[i] = 0.f;
  }
  if (item >= M * nh) return;
  const int m = item / nh;
  const int h = item - m * nh;
  const int b = m / T;
  const long long p = (long long)pos[b] + (m - b * T);
  // A position outside the cache / RoPE table is skipped rather than read or
  // written out of bounds (the accumulator is still consumed and re-zeroed).
  const bool in_range = p >= 0 && p < max_pos;
  const long long rowbase = (long long)m * nh * D + (long long)h * D;
  float x0, x1;
  uint32_t xbits;
  if (ACC) {
    // round the fp32 projection to bf16 (gemv.py:240-241), then re-zero it (gemv.py:242)
    float2* ap = reinterpret_cast<float2*>(const_cast<void*>(src)) + (rowbase >> 1) + lane;
    const float2 a = *ap;
    x0 = round_bf16(a.x);
    x1 = round_bf16(a.y);
    xbits = pack_bf16x2(x0, x1);
    *ap = make_float2(0.f, 0.f);
  } else {
    xbits = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(src) + rowbase)[lane];
    x0 = bf16lo(xbits);
    x1 = bf16hi(xbits);
  }
  if (!in_range) return;
  if (h >= nq + nkv) {  // V head: copy into the cache slot (fused.py:93-96)
    const int vh = h - nq - nkv;
    reinterpret_cast<uint32_t*>(vcache + b * cb + vh * ch + p * D)[lane] = xbits;
    return;
  }
  const uint16_t* w = h < nq ? qw : kw;
  const uint32_t wbits = reinterpret_cast<const uint32_t*>(w)[lane];
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = rsqrtf(ss / (float)D + eps);
  // xn = bf16(w * bf16(x * rstd)) (fused.py:80-81)
  const float n0 = round_bf16(bf16lo(wbits) * round_bf16(x0 * rstd));
  const float n1 = round_bf16(bf16hi(wbits) * round_bf16(x1 * rstd));
  float r0 = __shfl_xor(n0, 32, 64);
  float r1 = __shfl_xor(n1, 32, 64);
  if (lane < 32) {  // rotate_half: first half takes -x[d+64]
    r0 = -r0;
    r1 = -r1;
  }
  const uint32_t cbits = reinterpret_cast<const uint32_t*>(cosb + p * D)[lane];
  const uint32_t sbits = reinterpret_cast<const uint32_t*>(sinb + p * D)[lane];
  // y = bf16(bf16(xn*cos) + bf16(rot*sin)) (fused.py:85-87)
  const float y0 = round_bf16(n0 * bf16lo(cbits)) + round_bf16(r0 * bf16lo(sbits));
  const float y1 = round_bf16(n1 * bf16hi(cbits)) + round_bf16(r1 * bf16hi(sbits));
  const uint32_t ybits = pack_bf16x2(y0, y1);
  if (h < nq) {
    reinterpret_cast<uint32_t*>(q_out + (long long)m * nq * D + (long long)h * D)[lane] = ybits;
  } else {
    const int kh = h - nq;
    reinterpret_cast<uint32_t*>(kcache + b * cb + kh * ch + p * D)[lane] = ybits;
  }
}

// ---- SwiGLU: out = bf16(bf16(silu(g)) * u), gu = [M, 2I] -------------------
__device__ __forceinline__ float silu_bf16(float g) {
  return round_bf16(g / (1.0f + expf(-g)));
}

__global__ __launch_bounds__(NT) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                      uint16_t* __restrict__ out, int M, int I) {
  const int ic = I >> 3;
  const long long idx = (long long)blockIdx.x * NT + threadIdx.x;
  if (idx >= (long long)M * ic) return;
  const long long m = idx / ic;
  const int c = (int)(idx - m * ic);
  const uint4 gv = ldg16(gu + m * 2 * I + 8 * c);
  const uint4 uv = ldg16(gu + m * 2 * I + I + 8 * c);
  const uint32_t g[4] = {gv.x, gv.y, gv.z, gv.w};
  const uint32_t u[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(silu_bf16(bf16lo(g[e])) * bf16lo(u[e]),
                       silu_bf16(bf16hi(g[e])) * bf16hi(u[e]));
  *reinterpret_cast<uint4*>(out + m * I + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
}

// ---- embedding gather + sum of squares: one workgroup per row --------------
__global__ __launch_bounds__(NT) void embed_ss_kernel(const long long* __restrict__ ids,
                                                      const uint16_t* __restrict__ emb,
                                                      uint16_t* __restrict__ h,
                                                      float* __restrict__ ss, int H, int V) {
  __shared__ float red[NT / 64];
  const long long m = blockIdx.x;
  const long long tok = ids[m];
  const bool valid = tok >= 0 && tok < V;  // an out-of-vocabulary id gathers zeros
  const int hc = H >> 3;
  float sq = 0.f;
  for (int c = threadIdx.x; c < hc; c += NT) {
    const uint4 v = valid ? ldg16(emb + tok * H + 8 * c) : make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4*>(h + m * H + 8 * c) = v;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = bf16lo(w[e]), b2 = bf16hi(w[e]);
      sq += a * a + b2 * b2;
    }
  }
  const float s = block_sum(sq, red);
  if (threadIdx.x == 0 && ss) ss[m] = s;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The decode attention's RoPE rows: out[b] = (cos[p], sin[p]) with
// p = clamp(pos[b], 0, rows - 1), the rows qk_norm_rope reads for the new
// token (fused.py:71-87). One workgroup per sequence, 16-byte copies.
__global__ __launch_bounds__(64) void rope_rows_kernel(const int* __restrict__ pos,
                                                      const uint16_t* __restrict__ cosb,
                                                      const uint16_t* __restrict__ sinb, int rows,
                                                      int d, uint16_t* __restrict__ out) {
  const int b = blockIdx.x;
  const int p = min(max(pos[b], 0), rows - 1);
  const int chunks = d / 8;  // per row
  for (int i = threadIdx.x; i < 2 * chunks; i += blockDim.x) {
    const uint16_t* src = (i < chunks ? cosb : sinb) + (long long)p * d + 8 * (i % chunks);
    *reinterpret_cast<uint4*>(out + (long long)b * 2 * d + 8 * i) = ldg16(src);
  }
}

}  // namespace

extern "C" {

int ko_rope_rows(const int* pos, const void* cos, const void* sin, int rows, int d, int B,
                 void* out, void* stream) {
  if (!pos || !cos || !sin || !out || rows < 1 || B < 1 || d < 8 || (d & 7)) return KO_EINVAL;
  if (((uintptr_t)cos | (uintptr_t)sin | (uintptr_t)out) & 15) return KO_EINVAL;
  hipLaunchKernelGGL(rope_rows_kernel, dim3(B), dim3(64), 0, static_cast<hipStream_t>(stream), pos,
                     static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), rows,
                     d, static_cast<uint16_t*>(out));
  return KO_LAUNCH_STATUS();
}

int ko_add_rms_norm(void* res, const void* delta, const void* weight, void* out, int rows, int n,
                    float eps, void* stream) {
  if (!res || !weight || !out || rows < 1 || n < 8 || (n & 7) || n > 8 * 4 * NT)
    return n > 8 * 4 * NT ? KO_ENOTSUP : KO_EINVAL;
  if (!al16(res) || !al16(out) || !al16(weight) || (delta && !al16(delta))) return KO_EINVAL;
  hipLaunchKernelGGL(add_rms_norm_kernel, dim3(rows), dim3(NT), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t*>(res),
                     static_cast<const uint16_t*>(delta), static_cast<const uint16_t*>(weight),
                     static_cast<uint16_t*>(out), n, eps);
  return KO_LAUNCH_STATUS();
}

static int launch_qk(bool acc, const void* src, const void* q_w, const void* k_w, const void* cos,
                     const void* sin, const int* pos, void* q_out, void* k_cache, void* v_cache,
                     float* zero_buf, int n_zero, int M, int T, long long cb, long long ch,
                     float eps, int nq, int nkv, int d, int max_pos, void* stream) {
  if (!src || !q_w || !k_w || !cos || !sin || !pos || !q_out || !k_cache || !v_cache)
    return KO_EINVAL;
  if (d != 128) return KO_ENOTSUP;
  if (M < 1 || T < 1 || M % T || nq < 1 || nkv < 1 || cb < 0 || ch < 0 || (cb & 1) || (ch & 1) ||
      max_pos < 1)
    return KO_EINVAL;
  const int items = M * (nq + 2 * nkv);
  const int per = NT / 64;
  hipLaunchKernelGGL(acc ? qk_norm_rope_kernel<true> : qk_norm_rope_kernel<false>,
                     dim3((items + per - 1) / per), dim3(NT), 0, static_cast<hipStream_t>(stream),
                     src, static_cast<const uint16_t*>(q_w), static_cast<const uint16_t*>(k_w),
                     static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), pos,
                     static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), zero_buf, n_zero, M, T, cb, ch, eps, nq,
                     nkv, max_pos);
  return KO_LAUNCH_STATUS();
}

int ko_qk_norm_rope(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                    const void* sin, const int* pos, void* q_out, void* k_cache, void* v_cache,
                    int M, int T, long long cache_b_stride, long long cache_h_stride, float eps,
                    int nq, int nkv, int d, int max_pos, void* stream) {
  return launch_qk(false, qkv, q_w, k_w, cos, sin, pos, q_out, k_cache, v_cache, nullptr, 0, M,
                   T, cache_b_stride, cache_h_stride, eps, nq, nkv, d, max_pos, stream);
}

int ko_qk_norm_rope_acc(float* acc, const void* q_w, const void* k_w, const void* cos,
                        const void* sin, const int* pos, void* q_out, void* k_cache,
                        void* v_cache, float* zero_buf, int n_zero, int B,
                        long long cache_b_stride, long long cache_h_stride, float eps, int nq,
                        int nkv, int d, int max_pos, void* stream) {
  if (n_zero < 0 || (n_zero > 0 && !zero_buf)) return KO_EINVAL;
  return launch_qk(true, acc, q_w, k_w, cos, sin, pos, q_out, k_cache, v_cache, zero_buf, n_zero,
                   B, 1, cache_b_stride, cache_h_stride, eps, nq, nkv, d, max_pos, stream);
}

int ko_silu_mul(const void* gu, void* out, int M, int I, void* stream) {
  if (!gu || !out || M < 1 || I < 8 || (I & 7) || !al16(gu) || !al16(out)) return KO_EINVAL;
  const long long work = (long long)M * (I >> 3);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((work + NT - 1) / NT)), dim3(NT), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gu),
                     static_cast<uint16_t*>(out), M, I);
  return KO_LAUNCH_STATUS();
}

int ko_embed_ss(const long long* ids, const void* emb, void* h, float* ss, int M, int H, int V,
                void* stream) {
  if (!ids || !emb || !h || M < 1 || H < 8 || (H & 7) || V < 1 || !al16(emb) || !al16(h))
    return KO_EINVAL;
  hipLaunchKernelGGL(embed_ss_kernel, dim3(M), dim3(NT), 0, static_cast<hipStream_t>(stream), ids,
                     static_cast<const uint16_t*>(emb), static_cast<uint16_t*>(h), ss, H, V);
  return KO_LAUNCH_STATUS();
}

}  // extern "C"
