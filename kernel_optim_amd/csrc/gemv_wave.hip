// Fused skinny GEMM, VALU layout 1 (a wavefront per group of output columns,
// the normalised x shared through LDS); the semantics are those of gemv.hip's
// entry points (engine/kernels/gemv.py:30-106).
#include "gemv_launch.h"

using namespace ko;

namespace {

constexpr int NT = GEMV_NT;

// ---------------------------------------------------------------------------
// layout 1: one wavefront per RW output columns, WPB wavefronts per workgroup
// ---------------------------------------------------------------------------

template <int M, int RW, int WPB, bool NORM, int EPI>
__global__ __launch_bounds__(64 * WPB) void gemv_wave_kernel(GemvArgs a) {
  constexpr int NW = EPI == EPI_SWIGLU ? 2 * RW : RW;
  constexpr int UNR = 4;  // chunks per lane in flight per row
  __shared__ __align__(16) uint16_t s_x[NORM ? LDS_X_BYTES / 2 : 8];
  __shared__ float s_red[WPB][M];

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int N = a.N, K = a.K, KC = K >> 3, mr = a.mrows;
  const int unit = blockIdx.x * WPB + wv;   // this wave's row group
  const int n0 = unit * RW;

  const uint16_t* wp[NW];
#pragma unroll
  for (int r = 0; r < NW; ++r) {
    const int n = r < RW ? min(n0 + r, N - 1) : N + min(n0 + r - RW, N - 1);
    wp[r] = a.w + (long long)n * K;
  }

  // First weight chunks do not depend on the prologue.
  uint4 wcur[UNR][NW];
#pragma unroll
  for (int u = 0; u < UNR; ++u) {
    const int c = lane + 64 * u;
    if (c < KC) {
#pragma unroll
      for (int r = 0; r < NW; ++r) wcur[u][r] = ldg16_stream(wp[r] + 8 * c);
    }
  }

  const uint16_t* xsrc = a.x;
  if constexpr (NORM) {
    // rstd per row, then the normalised x into LDS, shared by the WPB waves.
    float rstd[M];
    if (a.ss) {
#pragma unroll
      for (int m = 0; m < M; ++m) rstd[m] = m < mr ? rsqrtf(a.ss[m] / (float)K + a.eps) : 0.f;
    } else {
      float sq[M];
#pragma unroll
      for (int m = 0; m < M; ++m) sq[m] = 0.f;
      for (int c = threadIdx.x; c < KC; c += 64 * WPB) {
#pragma unroll
        for (int m = 0; m < M; ++m)
          if (m < mr) sq[m] += sq8(ldg16(a.x + (long long)m * K + 8 * c));
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float v = wave_sum(sq[m]);
        if (lane == 0) s_red[wv][m] = v;
      }
      __syncthreads();
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < WPB; ++i) s += s_red[i][m];
        rstd[m] = rsqrtf(s / (float)K + a.eps);
      }
    }
    for (int c = threadIdx.x; c < KC; c += 64 * WPB) {
      const uint4 nwv = ldg16(a.nw + 8 * c);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint4 xv = m < mr ? ldg16(a.x + (long long)m * K + 8 * c) : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(s_x + (long long)m * K + 8 * c) = norm8(xv, nwv, rstd[m]);
      }
    }
    __syncthreads();
  }

  if (n0 >= N) return;  // a trailing wave with no rows (after the shared prologue)

  float acc[M][NW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NW; ++r) acc[m][r] = 0.f;

  for (int cb = 0; cb < KC; cb += 64 * UNR) {
    uint4 wnext[UNR][NW];
    const bool more = cb + 64 * UNR < KC;
    if (more) {
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int c = cb + 64 * UNR + lane + 64 * u;
        if (c < KC) {
#pragma unroll
          for (int r = 0; r < NW; ++r) wnext[u][r] = ldg16_stream(wp[r] + 8 * c);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = cb + lane + 64 * u;
      if (c < KC) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
          if (m < mr) {
            uint4 xv;
            if constexpr (NORM) xv = *reinterpret_cast<const uint4*>(s_x + (long long)m * K + 8 * c);
            else xv = ldg16(xsrc + (long long)m * K + 8 * c);
#pragma unroll
            for (int r = 0; r < NW; ++r) acc[m][r] = dot8(xv, wcur[u][r], acc[m][r]);
          }
        }
      }
    }
    if (!more) break;
#pragma unroll
    for (int u = 0; u < UNR; ++u)
#pragma unroll
      for (int r = 0; r < NW; ++r) wcur[u][r] = wnext[u][r];
  }

  // Reduce each (m, r) partial over the 64 lanes; every lane ends with the sums.
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NW; ++r) acc[m][r] = wave_sum(acc[m][r]);

  // Each output element is finished by one lane (lane (m*RW + r) % 64).
  float h2[M];
  float2 best[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    h2[m] = 0.f;
    best[m] = make_float2(-INFINITY, __int_as_float(0x7fffffff));
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = n0 + r;
      const bool ok = m < mr && n < N;
      if (ok && lane == ((m * RW + r) & 63))
        h2[m] += epilogue<EPI>(a, m, n, acc[m][r], EPI == EPI_SWIGLU ? acc[m][NW - RW + r] : 0.f);
      if constexpr (EPI == EPI_ARGMAX) {
        const float v = round_bf16(acc[m][r]);
        if (ok && v > best[m].x) best[m] = make_float2(v, __int_as_float(n));  // ties keep lower n
      }
    }
  if constexpr (EPI == EPI_RESID) {
    if (a.ss_out) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float s = wave_sum(h2[m]);
        if (m < mr && lane == 0) atomicAdd(a.ss_out + m, s);
      }
    }
  }
  if constexpr (EPI == EPI_ARGMAX) {
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < M; ++m)
        if (m < mr) a.part[(long long)m * a.nparts + unit] = best[m];
    }
  }
}

template <int M, int RW, int WPB>
int launch_wave(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  const int units = (a.N + RW - 1) / RW;
  const dim3 grid((units + WPB - 1) / WPB), block(64 * WPB);
#define KO_W(NORMV, EPIV) \
  hipLaunchKernelGGL((gemv_wave_kernel<M, RW, WPB, NORMV, EPIV>), grid, block, 0, s, a)
  switch (epi) {
    case EPI_F32: if (norm) KO_W(true, EPI_F32); else KO_W(false, EPI_F32); break;
    case EPI_BF16: if (norm) KO_W(true, EPI_BF16); else KO_W(false, EPI_BF16); break;
    case EPI_RESID: if (norm) KO_W(true, EPI_RESID); else KO_W(false, EPI_RESID); break;
    case EPI_SWIGLU: if (norm) KO_W(true, EPI_SWIGLU); else KO_W(false, EPI_SWIGLU); break;
    default: if (norm) KO_W(true, EPI_ARGMAX); else KO_W(false, EPI_ARGMAX); break;
  }
#undef KO_W
  return KO_LAUNCH_STATUS();
}

template <int RW, int WPB>
int launch_wave_m(const GemvArgs& a, int epi, bool norm, hipStream_t s) {
  if (a.mrows <= 1) return launch_wave<1, RW, WPB>(a, epi, norm, s);
  if (a.mrows <= 2) return launch_wave<2, RW, WPB>(a, epi, norm, s);
  return launch_wave<4, RW, WPB>(a, epi, norm, s);
}

int launch_wave_cfg(const GemvArgs& a, int epi, bool norm, int rw, int wpb, hipStream_t s) {
  if (rw == 1 && wpb == 2) return launch_wave_m<1, 2>(a, epi, norm, s);
  if (rw == 1 && wpb == 4) return launch_wave_m<1, 4>(a, epi, norm, s);
  if (rw == 2 && wpb == 2) return launch_wave_m<2, 2>(a, epi, norm, s);
  if (rw == 2 && wpb == 4) return launch_wave_m<2, 4>(a, epi, norm, s);
  if (rw == 4 && wpb == 2) return launch_wave_m<4, 2>(a, epi, norm, s);
  if (rw == 4 && wpb == 4) return launch_wave_m<4, 4>(a, epi, norm, s);
  return KO_ENOTSUP;
}

}  // namespace

namespace ko {

int launch_layout1(const GemvArgs& a, int epi, bool norm, int rw, int wpb, hipStream_t s) {
  return launch_wave_cfg(a, epi, norm, rw, wpb, s);
}

}  // namespace ko
