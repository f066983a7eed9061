// Fused skinny GEMM, VALU layout 0 (a 256-thread workgroup per group of output
// columns, v_dot2c_f32_bf16 dot products); the semantics are those of
// gemv.hip's entry points (engine/kernels/gemv.py:30-106).
#include "gemv_launch.h"

using namespace ko;

namespace {

constexpr int NT = GEMV_NT;

// ---------------------------------------------------------------------------
// layout 0: 256-thread workgroup per R output columns
// ---------------------------------------------------------------------------
template <int M, int R, bool NORM, int EPI>
__global__ __launch_bounds__(NT) void gemv_block_kernel(GemvArgs a) {
  constexpr int NW = EPI == EPI_SWIGLU ? 2 * R : R;
  __shared__ float red[16][M * NW];
  __shared__ float s_rstd[M];
  __shared__ float s_h2[M * R];
  __shared__ float2 s_best[M * R];

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
    float h2 = 0.f;
    if (ok) h2 = epilogue<EPI>(a, m, n, tot, tot2);
    if constexpr (EPI == EPI_RESID) s_h2[idx] = h2;
    if constexpr (EPI == EPI_ARGMAX)
      s_best[idx] = make_float2(ok ? round_bf16(tot) : -INFINITY,
                                __int_as_float(ok ? n : 0x7fffffff));
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
    if (t < M && t < mr) {
      float2 best = s_best[t * R];
      for (int r = 1; r < R; ++r) {
        const float2 c = s_best[t * R + r];
        if (c.x > best.x) best = c;  // columns ascend with r: ties keep the lower index
      }
      a.part[(long long)t * a.nparts + blockIdx.x] = best;
    }
  }
}

template <int M, int R, bool NORM, int EPI, int CPT>
__global__ __launch_bounds__(NT) void gemv_row_kernel(GemvArgs a) {
  gemv_row_body<M, R, NORM, EPI, CPT>(a, blockIdx.x);
}

template <int M, int R, int CPT>
int launch_row(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  const dim3 grid((a.N + R - 1) / R), block(NT);
#define KO_G(NORMV, EPIV) \
  hipLaunchKernelGGL((gemv_row_kernel<M, R, NORMV, EPIV, CPT>), grid, block, 0, s, a)
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

template <int M, int R>
int launch_block(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  // 1-4 rows with K <= 10240: the register-resident row kernel
  if constexpr (M <= 4 && R <= 8) {
    const int KC = a.K >> 3;
    if (KC <= 2 * NT) return launch_row<M, R, 2>(a, epi, norm, s);
    if constexpr (M <= 2 || R <= 4)
      if (KC <= 5 * NT && !(epi == EPI_SWIGLU && R > 4))
        return launch_row<M, R, 5>(a, epi, norm, s);
  }
  const dim3 grid((a.N + R - 1) / R), block(NT);
#define KO_G(NORMV, EPIV) \
  hipLaunchKernelGGL((gemv_block_kernel<M, R, NORMV, EPIV>), grid, block, 0, s, a)
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
int launch_block_r(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  if (a.mrows <= 1) return launch_block<1, R>(a, epi, norm, s);
  if (a.mrows <= 2) return launch_block<2, R>(a, epi, norm, s);
  if (a.mrows <= 4) return launch_block<4, R>(a, epi, norm, s);
  if (a.mrows <= 8) return launch_block<8, R>(a, epi, norm, s);
  return launch_block<16, R>(a, epi, norm, s);
}

// 16 columns per workgroup (fewer ARGMAX partials for the finalize) for 1-2 rows.
int launch_block_r16(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  if (a.mrows <= 1) return launch_block<1, 16>(a, epi, norm, s);
  if (a.mrows <= 2) return launch_block<2, 16>(a, epi, norm, s);
  return KO_ENOTSUP;
}

}  // namespace

namespace ko {

int launch_layout0(const GemvArgs& a, int epi, bool norm, int rows, hipStream_t s) {
  return rows == 4   ? launch_block_r<4>(a, epi, norm, s)
         : rows == 8 ? launch_block_r<8>(a, epi, norm, s)
                     : launch_block_r16(a, epi, norm, s);
}

}  // namespace ko
