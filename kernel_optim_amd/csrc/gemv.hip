// Fused skinny GEMM ("GEMV") for the decode step on gfx950:
//   y[M, N] = x[M, K] @ W[N, K]^T, M <= 16 rows per launch, each weight read once.
//
// Replaces engine/kernels/gemv.py:30-150 (_gemv_kernel, Gemv.__call__) with the
// same prologue/epilogue semantics (gemv.py:7-18, 86-106):
//   NORM   : x <- bf16(nw * bf16(x * rstd)), rstd = rsqrt(ss/K + eps). ss is the
//            caller's per-row sum of squares, or (ss == NULL) it is computed here
//            from x, which every workgroup reads anyway.
//   F32    : y fp32 (stored, or atomically added when accumulate=1)
//   BF16   : y = bf16(acc)
//   RESID  : h <- bf16(h + bf16(acc)); ss_out[m] += sum_n h_new^2 (when given)
//   SWIGLU : W is [2N, K] = gate | up; y = bf16(bf16(silu(bf16 g)) * bf16 u)
//   ARGMAX : BF16 logits (stored when y != NULL) and ids[m] = argmax_n bf16(acc),
//            lowest index on ties (torch.argmax, engine.py:291), reduced across
//            workgroups by the last one to finish.
//
// Mapping: a 256-thread workgroup owns R output columns (2R weight rows for
// SWIGLU) over the full K. Thread t reads the 16-byte chunks t, t+256, ... of
// each row (coalesced 4 KiB per row per step), two steps in flight, and keeps
// M x R fp32 partial dots (v_dot2c_f32_bf16); partials are reduced with DPP
// row sums and 1 KiB of LDS. HBM traffic is the weights once; x comes from L2.
#include "ko_common.h"

using namespace ko;

namespace {

constexpr int NT = 256;
enum { EPI_F32 = 0, EPI_BF16 = 1, EPI_RESID = 2, EPI_SWIGLU = 3, EPI_ARGMAX = 4 };

struct GemvArgs {
  const uint16_t* x;
  const uint16_t* w;
  void* y;
  const uint16_t* nw;
  const float* ss;
  uint16_t* h;
  float* ss_out;
  long long* ids;
  float2* part;
  int* counter;
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

// bf16(nw * bf16(x * rstd)) on 8 packed elements (gemv.py:77-79).
__device__ __forceinline__ uint32_t norm2(uint32_t x, uint32_t w, float rstd) {
  const float a = bf16lo(w) * round_bf16(bf16lo(x) * rstd);
  const float b = bf16hi(w) * round_bf16(bf16hi(x) * rstd);
  return pack_bf16x2(a, b);
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

template <int M, int R, bool NORM, int EPI>
__global__ __launch_bounds__(NT) void gemv_kernel(GemvArgs a) {
  constexpr int NW = EPI == EPI_SWIGLU ? 2 * R : R;
  __shared__ float red[16][M * NW];
  __shared__ float s_rstd[M];
  __shared__ float s_h2[M * R];
  __shared__ float2 s_best[M * R];
  __shared__ int s_last;

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int n0 = blockIdx.x * R;
  const int N = a.N, K = a.K, KC = K >> 3, mr = a.mrows;

  const uint16_t* wp[NW];
#pragma unroll
  for (int r = 0; r < NW; ++r) {
    const int n = r < R ? min(n0 + r, N - 1) : N + min(n0 + r - R, N - 1);
    wp[r] = a.w + (long long)n * K;
  }

  // Weights of the first step do not depend on the prologue: issue them now.
  uint4 wa[NW], wb[NW];
  const bool has0 = t < KC;
  if (has0) {
#pragma unroll
    for (int r = 0; r < NW; ++r) wa[r] = ldg16_stream(wp[r] + 8 * t);
  }

  float rstd[M];
  if constexpr (NORM) {
    if (a.ss) {
#pragma unroll
      for (int m = 0; m < M; ++m) rstd[m] = m < mr ? rsqrtf(a.ss[m] / (float)K + a.eps) : 0.f;
    } else {
      float sq[M];
#pragma unroll
      for (int m = 0; m < M; ++m) sq[m] = 0.f;
      for (int c = t; c < KC; c += NT) {
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (m < mr) sq[m] += sq8(ldg16(a.x + (long long)m * K + 8 * c));
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float v = row_sum16(sq[m]);
        if ((lane & 15) == 0) red[wv * 4 + (lane >> 4)][m] = v;
      }
      __syncthreads();
      if (t < M) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += red[i][t];
        s_rstd[t] = rsqrtf(s / (float)K + a.eps);
      }
      __syncthreads();
#pragma unroll
      for (int m = 0; m < M; ++m) rstd[m] = s_rstd[m];
    }
  }

  float acc[M][NW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NW; ++r) acc[m][r] = 0.f;

  auto compute = [&](int c, const uint4* wr) {
    uint4 nwv;
    if constexpr (NORM) nwv = ldg16(a.nw + 8 * c);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (m < mr) {
        uint4 xv = ldg16(a.x + (long long)m * K + 8 * c);
        if constexpr (NORM) xv = norm8(xv, nwv, rstd[m]);
#pragma unroll
        for (int r = 0; r < NW; ++r) acc[m][r] = dot8(xv, wr[r], acc[m][r]);
      }
    }
  };

  if (has0) {
    for (int c = t; c < KC; c += 2 * NT) {
      const int c1 = c + NT;
      if (c1 < KC) {
#pragma unroll
        for (int r = 0; r < NW; ++r) wb[r] = ldg16_stream(wp[r] + 8 * c1);
      }
      compute(c, wa);
      if (c1 >= KC) break;
      const int c2 = c1 + NT;
      if (c2 < KC) {
#pragma unroll
        for (int r = 0; r < NW; ++r) wa[r] = ldg16_stream(wp[r] + 8 * c2);
      }
      compute(c1, wb);
    }
  }

  // ---- reduce the partial dots over the 256 threads ----
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NW; ++r) {
      const float v = row_sum16(acc[m][r]);
      if ((lane & 15) == 0) red[wv * 4 + (lane >> 4)][m * NW + r] = v;
    }
  __syncthreads();

  for (int idx = t; idx < M * R; idx += NT) {
    const int m = idx / R, r = idx - (idx / R) * R, n = n0 + r;
    float tot = 0.f, tot2 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      tot += red[i][m * NW + r];
      if constexpr (EPI == EPI_SWIGLU) tot2 += red[i][m * NW + R + r];
    }
    const bool ok = m < mr && n < N;
    const long long o = (long long)m * N + n;
    if constexpr (EPI == EPI_F32) {
      if (ok) {
        float* y = static_cast<float*>(a.y);
        if (a.accumulate) atomicAdd(y + o, tot);
        else y[o] = tot;
      }
    } else if constexpr (EPI == EPI_BF16) {
      if (ok) static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(tot);
    } else if constexpr (EPI == EPI_SWIGLU) {
      if (ok) {
        const float g = round_bf16(tot), u = round_bf16(tot2);
        const float s = round_bf16(g / (1.0f + expf(-g)));
        static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(s * u);
      }
    } else if constexpr (EPI == EPI_RESID) {
      float hn2 = 0.f;
      if (ok) {
        const float hn = round_bf16(bf16_to_f32(a.h[o]) + round_bf16(tot));
        a.h[o] = f32_to_bf16(hn);
        hn2 = hn * hn;
      }
      s_h2[idx] = hn2;
    } else {  // EPI_ARGMAX
      const float v = round_bf16(tot);
      if (ok && a.y) static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(tot);
      s_best[idx] = make_float2(ok ? v : -INFINITY, __int_as_float(ok ? n : 0x7fffffff));
    }
  }

  if constexpr (EPI == EPI_RESID) {
    if (a.ss_out) {
      __syncthreads();
      if (t < M && t < mr) {
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) s += s_h2[t * R + r];
        atomicAdd(a.ss_out + t, s);
      }
    }
  }

  if constexpr (EPI == EPI_ARGMAX) {
    __syncthreads();
    const int nwg = gridDim.x;
    if (t == 0) {
      for (int m = 0; m < mr; ++m) {
        float2 best = s_best[m * R];
        for (int r = 1; r < R; ++r) {
          const float2 c = s_best[m * R + r];
          if (c.x > best.x) best = c;  // columns ascend with r: ties keep the lower index
        }
        a.part[(long long)m * nwg + blockIdx.x] = best;
      }
      __threadfence();
      const int prev = atomicAdd(a.counter, 1);
      s_last = prev == nwg - 1;
    }
    __syncthreads();
    if (s_last) {
      __threadfence();
      for (int m = 0; m < mr; ++m) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int i = t; i < nwg; i += NT) {
          const float2 c = a.part[(long long)m * nwg + i];
          const int ci = __float_as_int(c.y);
          if (c.x > bv || (c.x == bv && ci < bi)) {
            bv = c.x;
            bi = ci;
          }
        }
        // workgroup argmax with lowest-index tie break
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          const float ov = __shfl_xor(bv, off, 64);
          const int oi = __shfl_xor(bi, off, 64);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (lane == 0) s_best[wv] = make_float2(bv, __int_as_float(bi));
        __syncthreads();
        if (t == 0) {
          float2 best = s_best[0];
          for (int i = 1; i < NT / 64; ++i) {
            const float2 c = s_best[i];
            if (c.x > best.x || (c.x == best.x && __float_as_int(c.y) < __float_as_int(best.y)))
              best = c;
          }
          a.ids[m] = __float_as_int(best.y);
        }
        __syncthreads();
      }
      if (t == 0) *a.counter = 0;  // ready for the next launch (graph replays)
    }
  }
}

template <int M, int R>
int launch_m(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  const dim3 grid((a.N + R - 1) / R), block(NT);
#define KO_G(NORMV, EPIV) hipLaunchKernelGGL((gemv_kernel<M, R, NORMV, EPIV>), grid, block, 0, s, a)
  switch (epi) {
    case EPI_F32: if (norm) KO_G(true, EPI_F32); else KO_G(false, EPI_F32); break;
    case EPI_BF16: if (norm) KO_G(true, EPI_BF16); else KO_G(false, EPI_BF16); break;
    case EPI_RESID: if (norm) KO_G(true, EPI_RESID); else KO_G(false, EPI_RESID); break;
    case EPI_SWIGLU: if (norm) KO_G(true, EPI_SWIGLU); else KO_G(false, EPI_SWIGLU); break;
    default: if (norm) KO_G(true, EPI_ARGMAX); else KO_G(false, EPI_ARGMAX); break;
  }
#undef KO_G
  return KO_LAUNCH_STATUS();
}

template <int R>
int launch_r(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  if (a.mrows <= 1) return launch_m<1, R>(a, epi, norm, s);
  if (a.mrows <= 2) return launch_m<2, R>(a, epi, norm, s);
  if (a.mrows <= 4) return launch_m<4, R>(a, epi, norm, s);
  if (a.mrows <= 8) return launch_m<8, R>(a, epi, norm, s);
  return launch_m<16, R>(a, epi, norm, s);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

int ko_gemv(const void* x, const void* w, void* y, const void* nw, const float* ss, void* h,
            float* ss_out, long long* ids, float* part, int* counter, int M, int N, int K,
            int epi, int norm, int accumulate, int rows_per_wg, float eps, void* stream) {
  if (!x || !w || M < 1 || N < 1 || K < 8 || (K & 7)) return KO_EINVAL;
  if (epi < EPI_F32 || epi > EPI_ARGMAX) return KO_EINVAL;
  if (!al16(x) || !al16(w)) return KO_EINVAL;
  if (norm && (!nw || !al16(nw))) return KO_EINVAL;
  if ((epi == EPI_F32 || epi == EPI_BF16 || epi == EPI_SWIGLU) && !y) return KO_EINVAL;
  if (epi == EPI_RESID && !h) return KO_EINVAL;
  if (epi == EPI_ARGMAX && (!ids || !part || !counter)) return KO_EINVAL;
  if (rows_per_wg != 4 && rows_per_wg != 8) return KO_ENOTSUP;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Slices of at most 16 rows per launch.
  for (int m0 = 0; m0 < M; m0 += 16) {
    GemvArgs a;
    const int mr = M - m0 < 16 ? M - m0 : 16;
    a.x = static_cast<const uint16_t*>(x) + (long long)m0 * K;
    a.w = static_cast<const uint16_t*>(w);
    a.y = nullptr;
    if (y) {
      const size_t esz = epi == EPI_F32 ? 4 : 2;
      a.y = static_cast<char*>(y) + (size_t)m0 * N * esz;
    }
    a.nw = static_cast<const uint16_t*>(nw);
    a.ss = ss ? ss + m0 : nullptr;
    a.h = h ? static_cast<uint16_t*>(h) + (long long)m0 * N : nullptr;
    a.ss_out = ss_out ? ss_out + m0 : nullptr;
    a.ids = ids ? ids + m0 : nullptr;
    a.part = reinterpret_cast<float2*>(part);
    a.counter = counter;
    a.mrows = mr;
    a.N = N;
    a.K = K;
    a.eps = eps;
    a.accumulate = accumulate;
    const int st = rows_per_wg == 4 ? launch_r<4>(a, epi, norm != 0, s)
                                    : launch_r<8>(a, epi, norm != 0, s);
    if (st) return st;
  }
  return KO_OK;
}

// Scratch floats needed by EPI_ARGMAX for N columns with rows_per_wg rows per
// workgroup: 2 per (row, workgroup) for at most 16 rows per launch.
long long ko_gemv_argmax_scratch(int N, int rows_per_wg) {
  if (N < 1 || rows_per_wg < 1) return -1;
  return 2LL * 16 * ((N + rows_per_wg - 1) / rows_per_wg);
}

}  // extern "C"
