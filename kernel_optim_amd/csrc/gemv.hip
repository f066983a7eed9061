// Fused skinny GEMM ("GEMV") for the decode step on gfx950:
//   y[M, N] = x[M, K] @ W[N, K]^T, each weight read once for all M rows.
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
//   ARGMAX : bf16 logits (stored when y != NULL) and ids[m] = argmax_n bf16(acc),
//            lowest index on ties (torch.argmax, engine.py:291). Each work unit
//            writes its best (value, index) to scratch; a one-workgroup-per-row
//            finalize kernel reduces them in index order (no cross-workgroup
//            atomics) and optionally advances the decode positions.
//
// Two mappings of rows to the machine (both stream each weight row with
// coalesced 16-byte loads and accumulate with v_dot2c_f32_bf16):
//   layout 0 "block": a 256-thread workgroup owns R (4, 8; 16 for M <= 2)
//            output columns over the full K; thread t reads chunks t, t+256, ...;
//            M <= 16.
//   layout 1 "wave" : a wavefront owns RW output columns over the full K (lane l
//            reads chunks l, l+64, ...); WPB wavefronts per workgroup share the
//            normalised x through LDS, so the NORM prologue runs once per
//            workgroup. Row counts are chosen so every CU gets the same number
//            of rows (e.g. N=2560 -> 10 rows per CU). M <= 4.
//   layout 2 "mfma" : for up to 16 rows of x the product is a real contraction:
//            v_mfma_f32_16x16x32_bf16 with A = the (zero-padded) 16 rows of x and
//            B = 16 weight rows, one MFMA per 1 KiB of weights. A workgroup of
//            4 or 8 wavefronts owns a 16-column tile (plus the matching up tile
//            for SWIGLU), each wavefront a slice of K; the partial tiles are
//            summed through LDS and the epilogue runs one thread per (m, n).
//            Workgroups are persistent over tiles and the weight loads of the
//            next tile are issued during the last steps of the current one.
//            Each wavefront keeps its K slice of x (normalised for NORM) in
//            registers for all its tiles, so only weights stream. K is 2560
//            (8 wavefronts x 10 steps), 4096 (8 x 16) or 9728 (8 x 38). The
//            weights come in the tiled layout of ko_gemv_tile, in which every
//            load instruction reads 1 KiB contiguous (the MFMA operand layout
//            read from row-major weights touches 16 rows x 64 B per instruction
//            and tops out near 5 TB/s on MI355X).
#include "gemv_core.h"

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
  gemv_row_body<M, R, NORM, EPI, CPT, false>(a, blockIdx.x, [] {});
}

// ---------------------------------------------------------------------------
// layout 1: one wavefront per RW output columns, WPB wavefronts per workgroup
// ---------------------------------------------------------------------------
constexpr int LDS_X_BYTES = 40960;  // normalised x staged for the workgroup (M*K*2)

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

// ---------------------------------------------------------------------------
// layout 2: MFMA tiles of 16 columns, x rows padded to 16
// ---------------------------------------------------------------------------
constexpr int MFMA_CUS = 256;  // MI355X compute units: persistent grid = 256 x rows

// Row-wise (16-lane) argmax of (value, index): lowest index on ties.
__device__ __forceinline__ void row_argmax16(float& v, int& i) {
#define KO_ARG_STEP(CTRL)                                                                  \
  {                                                                                        \
    const float ov = dpp_f<CTRL>(v);                                                       \
    const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xf, 0xf, false);               \
    if (ov > v || (ov == v && oi < i)) {                                                   \
      v = ov;                                                                              \
      i = oi;                                                                              \
    }                                                                                      \
  }
  KO_ARG_STEP(0x128)
  KO_ARG_STEP(0x124)
  KO_ARG_STEP(0x122)
  KO_ARG_STEP(0x121)
#undef KO_ARG_STEP
}

template <int V>
struct IntC {
  static constexpr int value = V;
};

template <int EPI, bool NORM, int S, int PD, int WPG>
__global__ __launch_bounds__(64 * WPG) void gemv_mfma_kernel(GemvArgs a, int ntiles) {
  static_assert(S % PD == 0, "the weight ring must tile the K steps");
  constexpr int NW = EPI == EPI_SWIGLU ? 2 : 1;
  __shared__ float s_c[WPG][NW][16][17];
  __shared__ float s_sq[WPG][16];

  const int t = threadIdx.x, wv = t >> 6, lane = t & 63, col = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, mr = a.mrows;
  const int G = gridDim.x;
  const int kw0 = wv * (32 * S) + 8 * g;  // this lane's first k (step s adds 32 s)
  const bool mok = col < mr;               // A row m = col exists

  // Ring of PD weight steps in flight. The weights are in the tiled layout
  // (ko_gemv_tile): the B operand of (tile, step) is one 1 KiB block with lane
  // l's 16 bytes at 16 l, and a wavefront's steps are consecutive blocks.
  const int T = (N + 15) / 16, KS = K / 32;
  const uint16_t* wlane = a.w + (long long)(wv * S) * 512 + 8 * lane;
  uint4 wb[PD][NW];
  auto issue = [&](int tile, int s, int slot) {
#pragma unroll
    for (int r = 0; r < NW; ++r)
      wb[slot][r] = ldg16_stream(wlane + ((long long)(r * T + tile) * KS + s) * 512);
  };
  // This wavefront's K slice of x (A operand, row m = col), kept in registers
  // for every tile; NORM normalises it once. x (and, where registers allow, the
  // NORM gain) is loaded first, then the first tile's weights: loads return in
  // issue order, so the prologue runs while the weights stream. The weights
  // stay issued there (the scheduler would otherwise sink the loads next to
  // their MFMAs to save registers).
  constexpr bool NW_EARLY = NORM && S <= 10;
  bf16x8 xa[S];
  {
    const uint16_t* xrow = a.x + (long long)(mok ? col : 0) * K + kw0;
    uint4 xr[S], nwv[NW_EARLY ? S : 1];
#pragma unroll
    for (int s = 0; s < S; ++s) xr[s] = mok ? ldg16(xrow + 32 * s) : make_uint4(0, 0, 0, 0);
    if constexpr (NW_EARLY) {
#pragma unroll
      for (int s = 0; s < S; ++s) nwv[s] = ldg16(a.nw + kw0 + 32 * s);
    }
    __builtin_amdgcn_sched_barrier(0);  // x and the gain stay ahead of the weights
#pragma unroll
    for (int s = 0; s < PD; ++s) issue(blockIdx.x, s, s);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
      float rstd;
      if (a.ss) {
        rstd = mok ? rsqrtf(a.ss[col] / (float)K + a.eps) : 0.f;
      } else {
        float sq = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) sq += sq8(xr[s]);
        sq = sum_xor32(sum_xor16(sq));  // the 4 lane groups of row m
        if (g == 0) s_sq[wv][col] = sq;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < WPG; ++w) tot += s_sq[w][col];
        rstd = rsqrtf(tot / (float)K + a.eps);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        uint4 w;
        if constexpr (NW_EARLY) w = nwv[s];
        else w = ldg16(a.nw + kw0 + 32 * s);
        xr[s] = norm8(xr[s], w, rstd);
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) xa[s] = __builtin_bit_cast(bf16x8, xr[s]);
  }

  float bv = -INFINITY;  // ARGMAX: running best of row t / 16 (threads with t % 16 == 0)
  int bi = 0x7fffffff;
  // The wavefronts' partial tiles summed through LDS, then the epilogue, one
  // thread per (m, n).
  auto finish = [&](int tile, const f32x4* c) {
    // C lane layout: column col, rows 4g + i.
#pragma unroll
    for (int r = 0; r < NW; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_c[wv][r][4 * g + i][col] = c[r][i];
    __syncthreads();
    if (t < 256) {
      const int m = t >> 4, j = t & 15, n = tile * 16 + j;
      float tot = 0.f, tot2 = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) {
        tot += s_c[w][0][m][j];
        if constexpr (NW == 2) tot2 += s_c[w][NW - 1][m][j];
      }
      const bool ok = m < mr && n < N;
      float h2 = 0.f;
      if (ok) h2 = epilogue<EPI>(a, m, n, tot, tot2);
      if constexpr (EPI == EPI_RESID) {
        if (a.ss_out) {
          h2 = row_sum16(h2);
          if (j == 0 && m < mr) atomicAdd(a.ss_out + m, h2);
        }
      }
      if constexpr (EPI == EPI_ARGMAX) {
        float v = ok ? round_bf16(tot) : -INFINITY;
        int vi = ok ? n : 0x7fffffff;
        row_argmax16(v, vi);
        if (v > bv || (v == bv && vi < bi)) {
          bv = v;
          bi = vi;
        }
      }
    }
    __syncthreads();  // s_c is rewritten by the next tile
  };
  // One tile. Each consumed slot is refilled with the step PD ahead: of this
  // tile, or with ISSUE of the next one. The workgroup's last tile runs without
  // ISSUE, so nothing is loaded past it. (Re-issuing a clamped tile there
  // instead cost ~4.5 us of the 16-row gate/up GEMV's ~25.)
  auto run = [&](auto issue_c, int tile, int next) {
    constexpr bool ISSUE = decltype(issue_c)::value != 0;
    f32x4 c[NW];
#pragma unroll
    for (int r = 0; r < NW; ++r) c[r] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int slot = s % PD;
#pragma unroll
      for (int r = 0; r < NW; ++r)
        c[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[s], __builtin_bit_cast(bf16x8, wb[slot][r]),
                                                       c[r], 0, 0, 0);
      if (s + PD < S) issue(tile, s + PD, slot);
      else if constexpr (ISSUE) issue(next, s + PD - S, slot);
    }
    finish(tile, c);
  };

  int tile = blockIdx.x;
  for (; tile + G < ntiles; tile += G) run(IntC<1>{}, tile, tile + G);
  if (tile < ntiles) run(IntC<0>{}, tile, tile);
  if constexpr (EPI == EPI_ARGMAX) {
    const int m = t >> 4;
    if (t < 256 && (t & 15) == 0 && m < mr)
      a.part[(long long)m * a.nparts + blockIdx.x] = make_float2(bv, __int_as_float(bi));
  }
}

// layout 3: the layout-2 weight tiles with the K range of a tile cut into
// slices, one 4-wavefront workgroup per (tile, slice), a grid of
// ntiles * slices workgroups (not persistent). Wavefront w of slice q takes the
// S consecutive 32-wide K steps starting at (4 q + w) S, so slices = K / (128 S).
// With one slice the workgroup runs the epilogue itself. With more, each writes
// its fp32 16 x 16 partial tile to its own slot with device-coherent stores and
// counts its arrival on the tile's counter; the last to arrive adds the slots
// in slice order (the result does not depend on the arrival order), re-arms
// the counter and runs the epilogue. NORM computes the row norms from the
// wavefronts' x slices, so it needs one slice (or ss given).
constexpr int KSW = 4;       // wavefronts per workgroup of layout 3
constexpr int KS_MAX = 32;   // slices per tile
template <int EPI, bool NORM, int S, int PD>
__global__ __launch_bounds__(64 * KSW) void gemv_mfma_ks_kernel(GemvArgs a, int* __restrict__ ctr,
                                                               float* __restrict__ slots) {
  static_assert(EPI != EPI_ARGMAX, "the split-K layout has no argmax epilogue");
  constexpr int NW = EPI == EPI_SWIGLU ? 2 : 1;
  __shared__ float s_c[KSW][NW][16][17];
  __shared__ float s_sq[KSW][16];
  __shared__ int s_prev;
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63, col = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, mr = a.mrows;
  const int nsl = K / (32 * S * KSW);
  const int tile = blockIdx.x / nsl, slice = blockIdx.x - tile * nsl;
  const int T = (N + 15) / 16, KS = K / 32;
  const int sb = (slice * KSW + wv) * S;  // this wavefront's first K step
  const int kw0 = sb * 32 + 8 * g;        // this lane's first k
  const bool mok = col < mr;

  const uint16_t* wlane = a.w + 8 * lane;
  uint4 wb[PD][NW];
  auto issue = [&](int s, int slot) {
#pragma unroll
    for (int r = 0; r < NW; ++r)
      wb[slot][r] = ldg16_stream(wlane + ((long long)(r * T + tile) * KS + sb + s) * 512);
  };

  // x (and the NORM gain) first: loads return in issue order, so the prologue
  // then runs while the weights stream instead of after them.
  bf16x8 xa[S];
  {
    const uint16_t* xrow = a.x + (long long)(mok ? col : 0) * K + kw0;
    uint4 xr[S], nwv[NORM ? S : 1];
#pragma unroll
    for (int s = 0; s < S; ++s) xr[s] = mok ? ldg16(xrow + 32 * s) : make_uint4(0, 0, 0, 0);
    if constexpr (NORM) {
#pragma unroll
      for (int s = 0; s < S; ++s) nwv[s] = ldg16(a.nw + kw0 + 32 * s);
    }
    __builtin_amdgcn_sched_barrier(0);  // x and the gain stay ahead of the weights
#pragma unroll
    for (int s = 0; s < PD; ++s) issue(s, s);
    // keep the whole ring issued here: the scheduler would otherwise sink the
    // weight loads next to their MFMAs to save registers, leaving ~3 in flight
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
      float rstd;
      if (a.ss) {
        rstd = mok ? rsqrtf(a.ss[col] / (float)K + a.eps) : 0.f;
      } else {  // one slice: the KSW wavefronts hold the whole row
        float sq = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) sq += sq8(xr[s]);
        sq = sum_xor32(sum_xor16(sq));
        if (g == 0) s_sq[wv][col] = sq;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < KSW; ++w) tot += s_sq[w][col];
        rstd = rsqrtf(tot / (float)K + a.eps);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) xr[s] = norm8(xr[s], nwv[s], rstd);
    }
#pragma unroll
    for (int s = 0; s < S; ++s) xa[s] = __builtin_bit_cast(bf16x8, xr[s]);
  }

  f32x4 c[NW];
#pragma unroll
  for (int r = 0; r < NW; ++r) c[r] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int slot = s % PD;
#pragma unroll
    for (int r = 0; r < NW; ++r)
      c[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[s], __builtin_bit_cast(bf16x8, wb[slot][r]),
                                                     c[r], 0, 0, 0);
    if (s + PD < S) issue(s + PD, slot);
  }
  // C lane layout: column col, rows 4g + i.
#pragma unroll
  for (int r = 0; r < NW; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_c[wv][r][4 * g + i][col] = c[r][i];
  __syncthreads();
  const int m = t >> 4, j = t & 15, n = tile * 16 + j;
  float tot = 0.f, tot2 = 0.f;
#pragma unroll
  for (int w = 0; w < KSW; ++w) {
    tot += s_c[w][0][m][j];
    if constexpr (NW == 2) tot2 += s_c[w][NW - 1][m][j];
  }
  if (nsl > 1) {
    float* mine = slots + ((long long)(tile * nsl + slice) * NW) * 256 + t;
    __hip_atomic_store(mine, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (NW == 2) __hip_atomic_store(mine + 256, tot2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's slot stores are performed
    __syncthreads();
    if (t == 0) s_prev = __hip_atomic_fetch_add(ctr + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_prev != nsl - 1) return;
    const float* base = slots + (long long)tile * nsl * NW * 256 + t;
    float v[KS_MAX], v2[KS_MAX];
#pragma unroll
    for (int q = 0; q < KS_MAX; ++q) {
      v[q] = q < nsl ? __hip_atomic_load(base + q * NW * 256, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      if constexpr (NW == 2)
        v2[q] = q < nsl ? __hip_atomic_load(base + q * NW * 256 + 256, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    }
    tot = 0.f;
    tot2 = 0.f;
#pragma unroll
    for (int q = 0; q < KS_MAX; ++q) {
      if (q < nsl) {
        tot += v[q];
        if constexpr (NW == 2) tot2 += v2[q];
      }
    }
    if (t == 0) __hip_atomic_store(ctr + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const bool ok = m < mr && n < N;
  float h2 = 0.f;
  if (ok) h2 = epilogue<EPI>(a, m, n, tot, tot2);
  if constexpr (EPI == EPI_RESID) {
    if (a.ss_out) {
      h2 = row_sum16(h2);
      if (j == 0 && m < mr) atomicAdd(a.ss_out + m, h2);
    }
  }
}

// Weight layout of layout 2 ("tiled"): rows padded to a multiple of 16; for
// row tile t and k step s (32 columns) a 1 KiB block at ((t * K/32 + s) * 64 + l)
// * 8 elements holds, for lane l, row 16 t + l % 16, columns 32 s + 8 (l / 16)
// .. + 7 -- the v_mfma_f32_16x16x32_bf16 B-operand layout, so one 16-byte load
// per lane reads the block contiguously.
__global__ __launch_bounds__(256) void gemv_tile_kernel(const uint16_t* __restrict__ w,
                                                        uint16_t* __restrict__ wt, int rows,
                                                        int K, long long nchunks) {
  const int KS = K / 32;
  for (long long c = blockIdx.x * 256LL + threadIdx.x; c < nchunks; c += (long long)gridDim.x * 256) {
    const int l = (int)(c & 63);
    const long long blk = c >> 6;
    const int s = (int)(blk % KS);
    const long long t = blk / KS;
    const long long row = t * 16 + (l & 15);
    const int k = 32 * s + 8 * (l >> 4);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < rows) v = ldg16(w + row * K + k);
    *reinterpret_cast<uint4*>(wt + c * 8) = v;
  }
}

// One 1024-thread workgroup per row m: argmax over the work units' (value,
// index) pairs with the lowest index on ties. Optionally pos[m] += 1 (the decode step's position advance,
// engine.py:292) and h[m] = emb[ids[m]] (the next step's embedding gather,
// gemv.py:201-211, so the next step needs no gather launch).
constexpr int FT = 1024;
__device__ __forceinline__ void better(float v, int i, float& bv, int& bi) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}
__device__ __forceinline__ void better_xor16(float& v, int& i) {
  const unsigned vb = __builtin_bit_cast(unsigned, v);
  const auto pv = __builtin_amdgcn_permlane16_swap(vb, vb, false, false);
  const auto pi = __builtin_amdgcn_permlane16_swap((unsigned)i, (unsigned)i, false, false);
  // rows {0,0,2,2} and {1,1,3,3}: take the better of the two in every lane
  float a = __builtin_bit_cast(float, (unsigned)pv[0]), b = __builtin_bit_cast(float, (unsigned)pv[1]);
  int ia = (int)pi[0], ib = (int)pi[1];
  better(b, ib, a, ia);
  v = a;
  i = ia;
}
__device__ __forceinline__ void better_xor32(float& v, int& i) {
  const unsigned vb = __builtin_bit_cast(unsigned, v);
  const auto pv = __builtin_amdgcn_permlane32_swap(vb, vb, false, false);
  const auto pi = __builtin_amdgcn_permlane32_swap((unsigned)i, (unsigned)i, false, false);
  float a = __builtin_bit_cast(float, (unsigned)pv[0]), b = __builtin_bit_cast(float, (unsigned)pv[1]);
  int ia = (int)pi[0], ib = (int)pi[1];
  better(b, ib, a, ia);
  v = a;
  i = ia;
}

// All of a row's partial loads are issued before the first comparison (up to
// FL per thread, 24 x 1024 = 24576 work units in one round); the wave-level
// reductions use DPP and the gfx950 permlane swaps.
constexpr int FL = 24;
__global__ __launch_bounds__(FT) void argmax_finalize_kernel(
    const float2* __restrict__ part, int nparts, long long* __restrict__ ids,
    int* __restrict__ pos, const uint16_t* __restrict__ emb, uint16_t* __restrict__ h, int H,
    int V) {
  __shared__ float2 s_best[FT / 64];
  __shared__ int s_id;
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float2* pr = part + (long long)m * nparts;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i0 = t; i0 < nparts; i0 += FL * FT) {
    float2 c[FL];
#pragma unroll
    for (int j = 0; j < FL; ++j) {
      const int i = i0 + j * FT;
      c[j] = i < nparts ? pr[i] : make_float2(-INFINITY, __int_as_float(0x7fffffff));
    }
#pragma unroll
    for (int j = 0; j < FL; ++j) better(c[j].x, __float_as_int(c[j].y), bv, bi);
  }
  // within 16-lane rows (DPP row_ror), then across rows
#define KO_FIN_STEP(CTRL)                                                                   \
  {                                                                                         \
    const float ov = dpp_f<CTRL>(bv);                                                       \
    const int oi = __builtin_amdgcn_update_dpp(0, bi, CTRL, 0xf, 0xf, false);               \
    better(ov, oi, bv, bi);                                                                 \
  }
  KO_FIN_STEP(0x128)
  KO_FIN_STEP(0x124)
  KO_FIN_STEP(0x122)
  KO_FIN_STEP(0x121)
#undef KO_FIN_STEP
  better_xor16(bv, bi);
  better_xor32(bv, bi);
  if (lane == 0) s_best[wv] = make_float2(bv, __int_as_float(bi));
  __syncthreads();
  if (t == 0) {
    float2 b = s_best[0];
    float v = b.x;
    int i = __float_as_int(b.y);
    for (int w = 1; w < FT / 64; ++w) better(s_best[w].x, __float_as_int(s_best[w].y), v, i);
    ids[m] = i;
    if (pos) pos[m] += 1;
    s_id = i;
  }
  if (emb) {
    __syncthreads();
    const long long tok = s_id;
    if (tok >= 0 && tok < V) {
      for (int c = t; c < (H >> 3); c += FT)
        *reinterpret_cast<uint4*>(h + (long long)m * H + 8 * c) = ldg16(emb + tok * H + 8 * c);
    }
  }
}

// Greedy id of each row of bf16 logits [M, N] (row stride ld elements): one
// 1024-thread workgroup per row, lowest index on ties (torch.argmax over the
// verify step's logits, engine.py:413-415). Every thread reads 8 columns per
// 16-byte load, AL loads in flight before it compares; a scalar tail covers N
// not a multiple of 8.
constexpr int AL = 8;
__global__ __launch_bounds__(FT) void argmax_rows_kernel(const uint16_t* __restrict__ x,
                                                         long long ld, int N,
                                                         long long* __restrict__ ids) {
  __shared__ float2 s_best[FT / 64];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const uint16_t* row = x + (long long)m * ld;
  const int nc = N >> 3;  // whole 8-column chunks
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int c0 = t; c0 < nc; c0 += AL * FT) {
    uint4 u[AL];
#pragma unroll
    for (int j = 0; j < AL; ++j) {
      const int c = c0 + j * FT;
      u[j] = c < nc ? ldg16(row + 8 * c) : make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u,
                                                      0xff80ff80u);  // -inf
    }
#pragma unroll
    for (int j = 0; j < AL; ++j) {
      const int base = 8 * (c0 + j * FT);
      const uint32_t w[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        better(bf16lo(w[e]), base + 2 * e, bv, bi);
        better(bf16hi(w[e]), base + 2 * e + 1, bv, bi);
      }
    }
  }
  for (int c = 8 * nc + t; c < N; c += FT) better(bf16lo(row[c]), c, bv, bi);
#define KO_ROW_STEP(CTRL)                                                                   \
  {                                                                                         \
    const float ov = dpp_f<CTRL>(bv);                                                       \
    const int oi = __builtin_amdgcn_update_dpp(0, bi, CTRL, 0xf, 0xf, false);               \
    better(ov, oi, bv, bi);                                                                 \
  }
  KO_ROW_STEP(0x128)
  KO_ROW_STEP(0x124)
  KO_ROW_STEP(0x122)
  KO_ROW_STEP(0x121)
#undef KO_ROW_STEP
  better_xor16(bv, bi);
  better_xor32(bv, bi);
  if (lane == 0) s_best[wv] = make_float2(bv, __int_as_float(bi));
  __syncthreads();
  if (t == 0) {
    float v = s_best[0].x;
    int i = __float_as_int(s_best[0].y);
    for (int w = 1; w < FT / 64; ++w) better(s_best[w].x, __float_as_int(s_best[w].y), v, i);
    ids[m] = i;
  }
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

int mfma_grid(int N, int per_cu) {
  const int ntiles = (N + 15) / 16;
  const int g = MFMA_CUS * per_cu;
  return ntiles < g ? ntiles : g;
}

template <int S, int PD, int WPG>
int launch_mfma_s(const GemvArgs& a, int epi, bool norm, int grid, hipStream_t s) {
  const int ntiles = (a.N + 15) / 16;
#define KO_M(NORMV, EPIV)                                                             \
  hipLaunchKernelGGL((gemv_mfma_kernel<EPIV, NORMV, S, PD, WPG>), dim3(grid), dim3(64 * WPG), 0, \
                     s, a, ntiles)
  if (norm) {
    switch (epi) {
      case EPI_F32: KO_M(true, EPI_F32); break;
      case EPI_BF16: KO_M(true, EPI_BF16); break;
      case EPI_RESID: KO_M(true, EPI_RESID); break;
      case EPI_SWIGLU: KO_M(true, EPI_SWIGLU); break;
      default: KO_M(true, EPI_ARGMAX); break;
    }
  } else {
    switch (epi) {
      case EPI_F32: KO_M(false, EPI_F32); break;
      case EPI_BF16: KO_M(false, EPI_BF16); break;
      case EPI_RESID: KO_M(false, EPI_RESID); break;
      case EPI_SWIGLU: KO_M(false, EPI_SWIGLU); break;
      default: KO_M(false, EPI_ARGMAX); break;
    }
  }
#undef KO_M
  return KO_LAUNCH_STATUS();
}

// K = 32 * S * WPG: S steps of 32 per wavefront, WPG wavefronts splitting K.
// SWIGLU (two weight tiles) needs K <= 4096 to keep its registers.
bool mfma_supported(int K, int epi) {
  return K == 2560 || K == 4096 || (K == 9728 && epi != EPI_SWIGLU);
}

int launch_mfma(const GemvArgs& a, int epi, bool norm, int per_cu, hipStream_t s) {
  const int grid = mfma_grid(a.N, per_cu);
  switch (a.K) {
    case 2560: return launch_mfma_s<10, 10, 8>(a, epi, norm, grid, s);
    case 4096: return launch_mfma_s<16, 16, 8>(a, epi, norm, grid, s);
    default:
      if (epi == EPI_SWIGLU) return KO_ENOTSUP;
      return launch_mfma_s<38, 19, 8>(a, epi, norm, grid, s);
  }
}

// Steps per wavefront of layout 3 for K and a slice count (0: unsupported):
// S in {20, 19, 8, 4} with K = 128 * S * slices.
int ks_steps(int K, int slices) {
  if (slices < 1 || slices > KS_MAX || K % (128 * slices)) return 0;
  const int S = K / (128 * slices);
  return (S == 20 || S == 19 || S == 8 || S == 4) ? S : 0;
}

template <int S, int PD>
int launch_mfma_ks_s(const GemvArgs& a, int epi, bool norm, int slices, int* ctr, float* slots,
                     hipStream_t s) {
  const int grid = ((a.N + 15) / 16) * slices;
#define KO_K(NORMV, EPIV)                                                                  \
  hipLaunchKernelGGL((gemv_mfma_ks_kernel<EPIV, NORMV, S, PD>), dim3(grid), dim3(64 * KSW), 0, s, \
                     a, ctr, slots)
  if (norm) {
    if constexpr (S == 20) {
      switch (epi) {
        case EPI_F32: KO_K(true, EPI_F32); break;
        case EPI_BF16: KO_K(true, EPI_BF16); break;
        case EPI_RESID: KO_K(true, EPI_RESID); break;
        default: KO_K(true, EPI_SWIGLU); break;
      }
    } else {
      return KO_ENOTSUP;
    }
  } else {
    switch (epi) {
      case EPI_F32: KO_K(false, EPI_F32); break;
      case EPI_BF16: KO_K(false, EPI_BF16); break;
      case EPI_RESID: KO_K(false, EPI_RESID); break;
      default: KO_K(false, EPI_SWIGLU); break;
    }
  }
#undef KO_K
  return KO_LAUNCH_STATUS();
}

int launch_mfma_ks(const GemvArgs& a, int epi, bool norm, int slices, int* ctr, float* slots,
                   hipStream_t s) {
  // every weight step in flight at once, except SWIGLU's two tiles at 20 steps
  // (registers)
  switch (ks_steps(a.K, slices)) {
    case 20:
      if (epi == EPI_SWIGLU) return launch_mfma_ks_s<20, 10>(a, epi, norm, slices, ctr, slots, s);
      return launch_mfma_ks_s<20, 20>(a, epi, norm, slices, ctr, slots, s);
    case 19:
      if (epi == EPI_SWIGLU) return launch_mfma_ks_s<19, 10>(a, epi, norm, slices, ctr, slots, s);
      return launch_mfma_ks_s<19, 19>(a, epi, norm, slices, ctr, slots, s);
    case 8: return launch_mfma_ks_s<8, 8>(a, epi, norm, slices, ctr, slots, s);
    case 4: return launch_mfma_ks_s<4, 4>(a, epi, norm, slices, ctr, slots, s);
    default: return KO_ENOTSUP;
  }
}

// Layout 3 scratch (fp32 elements): the tiles' arrival counters (int32, zero
// before the first launch, left at zero by every launch), padded to 64, then
// two 16 x 16 fp32 slots (gate and up) per (tile, slice).
long long ks_scratch(int N, int slices) {
  const long long T = (N + 15) / 16;
  return ((T + 63) / 64) * 64 + T * slices * 2 * 256;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

long long parts_for(int N, int layout, int rows, int waves) {
  if (layout == 0) return (N + rows - 1) / rows;
  if (layout == 2) return mfma_grid(N, rows);
  if (layout != 1 || waves < 1) return 0;  // layout 3 has no ARGMAX partials
  const long long units = (N + rows - 1) / rows;
  return ((units + waves - 1) / waves) * waves;
}

}  // namespace

extern "C" {

int ko_gemv(const void* x, const void* w, void* y, const void* nw, const float* ss, void* h,
            float* ss_out, long long* ids, int* pos_inc, const void* next_emb, void* next_h,
            float* part, long long part_len, int M, int N, int K, int epi, int norm,
            int accumulate, int layout, int rows, int waves, float eps, void* stream) {
  if (!x || !w || M < 1 || N < 1 || K < 8 || (K & 7)) return KO_EINVAL;
  if (epi < EPI_F32 || epi > EPI_ARGMAX) return KO_EINVAL;
  if (!al16(x) || !al16(w)) return KO_EINVAL;
  if (norm && (!nw || !al16(nw))) return KO_EINVAL;
  if ((epi == EPI_F32 || epi == EPI_BF16 || epi == EPI_SWIGLU) && !y) return KO_EINVAL;
  if (epi == EPI_RESID && !h) return KO_EINVAL;
  if (layout == 0) {
    if (rows != 4 && rows != 8 && !(rows == 16 && M <= 2)) return KO_ENOTSUP;
  } else if (layout == 1) {
    if (waves != 2 && waves != 4) return KO_ENOTSUP;
    if (M > 4) return KO_ENOTSUP;
    if (norm && (long long)M * K * 2 > LDS_X_BYTES) return KO_ENOTSUP;
  } else if (layout == 2) {
    if (rows != 1 && rows != 2 && rows != 4) return KO_ENOTSUP;
    if (!mfma_supported(K, epi)) return KO_ENOTSUP;
  } else if (layout == 3) {
    if (epi == EPI_ARGMAX || !ks_steps(K, rows)) return KO_ENOTSUP;
    if (norm && rows > 1 && !ss) return KO_ENOTSUP;
    if (norm && ks_steps(K, rows) != 20) return KO_ENOTSUP;
    if (rows > 1 && (!part || !al16(part) || part_len < ks_scratch(N, rows))) return KO_ERANGE;
  } else {
    return KO_EINVAL;
  }
  const int mstep = layout == 1 ? 4 : 16;
  const long long nparts = parts_for(N, layout, rows, waves);
  if (epi == EPI_ARGMAX) {
    if (!ids || !part) return KO_EINVAL;
    if (part_len < 2LL * mstep * nparts) return KO_ERANGE;
    if ((next_emb == nullptr) != (next_h == nullptr)) return KO_EINVAL;
    if (next_emb && (!al16(next_emb) || !al16(next_h))) return KO_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int m0 = 0; m0 < M; m0 += mstep) {
    GemvArgs a;
    const int mr = M - m0 < mstep ? M - m0 : mstep;
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
    a.part = reinterpret_cast<float2*>(part);
    a.nparts = (int)nparts;
    a.mrows = mr;
    a.N = N;
    a.K = K;
    a.eps = eps;
    a.accumulate = accumulate;
    int st;
    if (layout == 0)
      st = rows == 4   ? launch_block_r<4>(a, epi, norm != 0, s)
           : rows == 8 ? launch_block_r<8>(a, epi, norm != 0, s)
                       : launch_block_r16(a, epi, norm != 0, s);
    else if (layout == 1)
      st = launch_wave_cfg(a, epi, norm != 0, rows, waves, s);
    else if (layout == 2)
      st = launch_mfma(a, epi, norm != 0, rows, s);
    else
      st = launch_mfma_ks(a, epi, norm != 0, rows, reinterpret_cast<int*>(part),
                          part + ((N + 15) / 16 + 63) / 64 * 64, s);
    if (st) return st;
    if (epi == EPI_ARGMAX) {
      hipLaunchKernelGGL(argmax_finalize_kernel, dim3(mr), dim3(FT), 0, s, a.part, a.nparts,
                         ids + m0, pos_inc ? pos_inc + m0 : nullptr,
                         static_cast<const uint16_t*>(next_emb),
                         next_h ? static_cast<uint16_t*>(next_h) + (long long)m0 * K : nullptr, K,
                         N);
      st = KO_LAUNCH_STATUS();
      if (st) return st;
    }
  }
  return KO_OK;
}

int ko_gemv_tile(const void* w, void* wt, int rows, int K, void* stream) {
  if (!w || !wt || rows < 1 || K < 32 || (K % 32)) return KO_EINVAL;
  if (!al16(w) || !al16(wt)) return KO_EINVAL;
  const long long nchunks = (long long)((rows + 15) / 16) * 16 * (K / 8);
  long long blocks = (nchunks + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(gemv_tile_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(wt), rows, K, nchunks);
  return KO_LAUNCH_STATUS();
}

int ko_argmax_rows(const void* x, long long ld, int M, int N, long long* ids, void* stream) {
  if (!x || !ids || M < 1 || N < 1 || ld < N || (ld & 7) || !al16(x)) return KO_EINVAL;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(M), dim3(FT), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), ld, N, ids);
  return KO_LAUNCH_STATUS();
}

// fp32 scratch elements ko_gemv needs for EPI 4 (ARGMAX) with this layout
// (a size, not a status; -1 for bad arguments).
long long ko_gemv_argmax_scratch(int N, int layout, int rows, int waves) {
  if (N < 1 || rows < 1 || (layout == 1 && waves < 1) || layout < 0 || layout > 3) return -1;
  if (layout == 3) return rows > 1 ? ks_scratch(N, rows) : 0;
  return 2LL * 16 * parts_for(N, layout, rows, waves);
}

}  // extern "C"
