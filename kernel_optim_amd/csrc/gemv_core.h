// GEMV building blocks shared by gemv.hip and the fused attention + o
// projection kernel: arguments, prologue/epilogue math (the semantics of
// engine/kernels/gemv.py:7-18, 77-106) and the 1-2-row workgroup body.
#pragma once

#include "ko_common.h"

namespace ko {

constexpr int GEMV_NT = 256;
enum { EPI_F32 = 0, EPI_BF16 = 1, EPI_RESID = 2, EPI_SWIGLU = 3, EPI_ARGMAX = 4 };

struct GemvArgs {
  const uint16_t* x;
  const uint16_t* w;
  void* y;
  const uint16_t* nw;
  const float* ss;
  uint16_t* h;
  float* ss_out;
  float2* part;  // ARGMAX: [M][nparts] (value, index bits)
  int nparts;
  int mrows, N, K;
  float eps;
  int accumulate;
};

__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float c) {
  c = dot2_bf16(a.x, b.x, c);
  c = dot2_bf16(a.y, b.y, c);
  c = dot2_bf16(a.z, b.z, c);
  c = dot2_bf16(a.w, b.w, c);
  return c;
}

// bf16(nw * bf16(x * rstd)) on packed pairs (gemv.py:77-79).
__device__ __forceinline__ uint32_t norm2(uint32_t x, uint32_t w, float rstd) {
  const uint32_t t = pack_bf16x2(bf16lo(x) * rstd, bf16hi(x) * rstd);  // bf16(x * rstd)
  return pack_bf16x2(bf16lo(w) * bf16lo(t), bf16hi(w) * bf16hi(t));
}
__device__ __forceinline__ uint4 norm8(const uint4& x, const uint4& w, float rstd) {
  return make_uint4(norm2(x.x, w.x, rstd), norm2(x.y, w.y, rstd), norm2(x.z, w.z, rstd),
                    norm2(x.w, w.w, rstd));
}
__device__ __forceinline__ float sq8(const uint4& v) {
  const uint32_t e[4] = {v.x, v.y, v.z, v.w};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = bf16lo(e[i]), b = bf16hi(e[i]);
    s += a * a + b * b;
  }
  return s;
}

// RESID: the residual element (m, n) as raw bf16, loaded ahead of the work
// that produces its sum so the epilogue does not wait a memory round trip for
// it. Rows past mrows and columns past N read a valid element (unused).
__device__ __forceinline__ uint16_t resid_load(const GemvArgs& a, int m, int n) {
  const int mm = m < a.mrows ? m : 0, nn = n < a.N ? n : a.N - 1;
  return a.h[(long long)mm * a.N + nn];
}

// Epilogue for one finished output element (m, n) with full sums (tot, tot2).
// Returns the bf16-rounded new residual squared (RESID) or 0. RESID takes the
// residual from `hres` (resid_load) when given, else loads it here.
template <int EPI>
__device__ __forceinline__ float epilogue(const GemvArgs& a, int m, int n, float tot, float tot2,
                                          const uint16_t* hres = nullptr) {
  const long long o = (long long)m * a.N + n;
  if constexpr (EPI == EPI_F32) {
    float* y = static_cast<float*>(a.y);
    if (a.accumulate) atomicAdd(y + o, tot);
    else y[o] = tot;
  } else if constexpr (EPI == EPI_BF16) {
    static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(tot);
  } else if constexpr (EPI == EPI_SWIGLU) {
    const float g = round_bf16(tot), u = round_bf16(tot2);
    const float s = round_bf16(g / (1.0f + expf(-g)));
    static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(s * u);
  } else if constexpr (EPI == EPI_RESID) {
    const float hn = round_bf16(bf16_to_f32(hres ? *hres : a.h[o]) + round_bf16(tot));
    a.h[o] = f32_to_bf16(hn);
    return hn * hn;
  } else {  // ARGMAX: logits only; the selection is done by the caller
    if (a.y) static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(tot);
  }
  return 0.f;
}

// layout 0 for 1-4 rows of x: the same mapping with the load order arranged
// for the memory system. x (and the NORM gain) are loaded first and kept in
// registers (normalised once), then every weight chunk of the workgroup is
// issued; loads return in issue order, so a dot product never waits behind a
// later load. Chunk indices past K are clamped to a valid chunk whose x is
// zeroed, which keeps the loads unconditional and the wait counts exact.
// CPT = chunks of 8 per thread (K <= 2048 * CPT). wg: this workgroup's column
// group.
template <int M, int R, bool NORM, int EPI, int CPT>
__device__ __forceinline__ void gemv_row_body(const GemvArgs& a, int wg) {
  constexpr int NW = EPI == EPI_SWIGLU ? 2 * R : R;
  __shared__ float red[16][M * NW];
  __shared__ float s_sq[GEMV_NT / 64][M];
  __shared__ float s_h2[M * R];
  __shared__ float2 s_best[M * R];

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int n0 = wg * R;
  const int N = a.N, K = a.K, KC = K >> 3, mr = a.mrows;

  uint4 xr[M][CPT];
  uint4 nwr[NORM ? CPT : 1];
  auto load_x = [&]() {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = min(t + GEMV_NT * j, KC - 1);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        xr[m][j] = ldg16(a.x + (long long)(m < mr ? m : 0) * K + 8 * c);
      }
      if constexpr (NORM) nwr[j] = ldg16(a.nw + 8 * c);
    }
  };
  static_assert(M * R <= GEMV_NT, "one epilogue element per thread");
  // RESID: this thread's residual element, issued before the weights
  uint16_t hpre = 0;
  if constexpr (EPI == EPI_RESID) {
    const int ti = t < M * R ? t : 0;
    hpre = resid_load(a, ti / R, n0 + ti % R);
  }
  load_x();
  uint4 w[CPT][NW];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = min(t + GEMV_NT * j, KC - 1);
#pragma unroll
    for (int r = 0; r < NW; ++r) {
      const int n = r < R ? min(n0 + r, N - 1) : N + min(n0 + r - R, N - 1);
      w[j][r] = ldg16_stream(a.w + (long long)n * K + 8 * c);
    }
  }
  const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < CPT; ++j)
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (t + GEMV_NT * j >= KC || m >= mr) xr[m][j] = zero;

  if constexpr (NORM) {
    float rstd[M];
    if (a.ss) {
#pragma unroll
      for (int m = 0; m < M; ++m) rstd[m] = m < mr ? rsqrtf(a.ss[m] / (float)K + a.eps) : 0.f;
    } else {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float sq = 0.f;
#pragma unroll
        for (int j = 0; j < CPT; ++j) sq += sq8(xr[m][j]);
        sq = wave_sum(sq);
        if (lane == 0) s_sq[wv][m] = sq;
      }
      __syncthreads();
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < GEMV_NT / 64; ++i) tot += s_sq[i][m];
        rstd[m] = rsqrtf(tot / (float)K + a.eps);
      }
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int m = 0; m < M; ++m) xr[m][j] = norm8(xr[m][j], nwr[j], rstd[m]);
  }

  float acc[M][NW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NW; ++r) acc[m][r] = 0.f;
#pragma unroll
  for (int j = 0; j < CPT; ++j)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < NW; ++r) acc[m][r] = dot8(xr[m][j], w[j][r], acc[m][r]);

#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NW; ++r) {
      const float v = row_sum16(acc[m][r]);
      if ((lane & 15) == 0) red[wv * 4 + (lane >> 4)][m * NW + r] = v;
    }
  __syncthreads();

  for (int idx = t; idx < M * R; idx += GEMV_NT) {
    const int m = idx / R, r = idx - (idx / R) * R, n = n0 + r;
    float tot = 0.f, tot2 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      tot += red[i][m * NW + r];
      if constexpr (EPI == EPI_SWIGLU) tot2 += red[i][m * NW + R + r];
    }
    const bool ok = m < mr && n < N;
    float h2 = 0.f;
    if (ok) h2 = epilogue<EPI>(a, m, n, tot, tot2, &hpre);  // idx == t: M * R <= GEMV_NT
    if constexpr (EPI == EPI_RESID) s_h2[idx] = h2;
    if constexpr (EPI == EPI_ARGMAX)
      s_best[idx] = make_float2(ok ? round_bf16(tot) : -INFINITY,
                                __int_as_float(ok ? n : 0x7fffffff));
  }
  if constexpr (EPI == EPI_RESID) {
    if (a.ss_out) {
      __syncthreads();
      if (t < M && t < mr) {
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) sum += s_h2[t * R + r];
        atomicAdd(a.ss_out + t, sum);
      }
    }
  }
  if constexpr (EPI == EPI_ARGMAX) {
    __syncthreads();
    if (t < M && t < mr) {
      float2 best = s_best[t * R];
      for (int r = 1; r < R; ++r) {
        const float2 c = s_best[t * R + r];
        if (c.x > best.x) best = c;  // columns ascend with r: ties keep the lower index
      }
      a.part[(long long)t * a.nparts + wg] = best;
    }
  }
}


}  // namespace ko
