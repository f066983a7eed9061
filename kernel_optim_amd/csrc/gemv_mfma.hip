// Fused skinny GEMM, MFMA layouts 2 and 3 (v_mfma_f32_16x16x32_bf16 on the
// tiled weight copy); the semantics are those of gemv.hip's entry points
// (engine/kernels/gemv.py:30-106).
#include "gemv_launch.h"

using namespace ko;

namespace {

// ---------------------------------------------------------------------------
// layout 2: MFMA tiles of 16 columns, x rows padded to 16
// ---------------------------------------------------------------------------

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

template <int EPI, bool NORM, int S, int PD, int WPG, int MT = 1>
__global__ __launch_bounds__(64 * WPG) void gemv_mfma_kernel(GemvArgs a, int ntiles) {
  static_assert(S % PD == 0, "the weight ring must tile the K steps");
  static_assert(MT == 1 || (MT == 2 && WPG * 64 >= 512), "16 or 32 rows of x");
  constexpr int NW = EPI == EPI_SWIGLU ? 2 : 1;
  constexpr bool HPRE = EPI == EPI_RESID && S <= 16;  // residual loaded ahead (registers)
  __shared__ float s_c[WPG][NW][16 * MT][17];
  __shared__ float s_sq[WPG][16 * MT];

  const int t = threadIdx.x, wv = t >> 6, lane = t & 63, col = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, mr = a.mrows;
  const int G = gridDim.x;
  const int kw0 = wv * (32 * S) + 8 * g;  // this lane's first k (step s adds 32 s)
  const bool mok = col < mr;               // A row m = col exists
  const bool mok2 = col + 16 < mr;         // MT = 2: the second row tile's row col + 16

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
  // their MFMAs to save registers). With NORM the compiler turns the masked x
  // loads into branches and waits for the second one before issuing the rest,
  // so the weights go out one memory round trip after x. Measured at 16 rows,
  // that order beats issuing everything at once (unmasked loads: qkv 10.5
  // against 10.3 us, gate/up 20.7 against 20.1) and an explicit wait for all
  // of x and the gain before the weights (10.4 / 20.7).
  constexpr bool NW_EARLY = NORM && S <= 10;
  bf16x8 xa[S];
  bf16x8 xa2[MT > 1 ? S : 1];  // MT = 2: rows 16..31 of x, the A operand of a second MFMA
  {
    const uint16_t* xrow = a.x + (long long)(mok ? col : 0) * K + kw0;
    uint4 xr[S], nwv[NW_EARLY ? S : 1], xr2[MT > 1 ? S : 1];
#pragma unroll
    for (int s = 0; s < S; ++s) xr[s] = mok ? ldg16(xrow + 32 * s) : make_uint4(0, 0, 0, 0);
    if constexpr (MT > 1) {
      const uint16_t* xrow2 = a.x + (long long)(mok2 ? col + 16 : 0) * K + kw0;
#pragma unroll
      for (int s = 0; s < S; ++s) xr2[s] = mok2 ? ldg16(xrow2 + 32 * s) : make_uint4(0, 0, 0, 0);
    }
    // the caller's row sums, loaded with x: a load issued after the weights
    // would make the norm wait for every weight step (loads return in order)
    float ssv = 0.f, ssv2 = 0.f;
    if constexpr (NORM) {
      if (a.ss) {
        ssv = a.ss[mok ? col : 0];
        if constexpr (MT > 1) ssv2 = a.ss[mok2 ? col + 16 : 0];
      }
    }
    if constexpr (NW_EARLY) {
#pragma unroll
      for (int s = 0; s < S; ++s) nwv[s] = ldg16(a.nw + kw0 + 32 * s);
    }
    __builtin_amdgcn_sched_barrier(0);  // x and the gain stay ahead of the weights
#pragma unroll
    for (int s = 0; s < PD; ++s) issue(blockIdx.x, s, s);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
      float rstd, rstd2 = 0.f;
      if (a.ss) {
        rstd = mok ? rsqrtf(ssv / (float)K + a.eps) : 0.f;
        if constexpr (MT > 1) rstd2 = mok2 ? rsqrtf(ssv2 / (float)K + a.eps) : 0.f;
      } else {
        float sq = 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) sq += sq8(xr[s]);
        sq = sum_xor32(sum_xor16(sq));  // the 4 lane groups of row m
        if (g == 0) s_sq[wv][col] = sq;
        if constexpr (MT > 1) {
          float sq2 = 0.f;
#pragma unroll
          for (int s = 0; s < S; ++s) sq2 += sq8(xr2[s]);
          sq2 = sum_xor32(sum_xor16(sq2));
          if (g == 0) s_sq[wv][16 + col] = sq2;
        }
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < WPG; ++w) tot += s_sq[w][col];
        rstd = rsqrtf(tot / (float)K + a.eps);
        if constexpr (MT > 1) {
          float tot2 = 0.f;
#pragma unroll
          for (int w = 0; w < WPG; ++w) tot2 += s_sq[w][16 + col];
          rstd2 = rsqrtf(tot2 / (float)K + a.eps);
        }
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        uint4 w;
        if constexpr (NW_EARLY) w = nwv[s];
        else w = ldg16(a.nw + kw0 + 32 * s);
        xr[s] = norm8(xr[s], w, rstd);
        if constexpr (MT > 1) xr2[s] = norm8(xr2[s], w, rstd2);
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) xa[s] = __builtin_bit_cast(bf16x8, xr[s]);
    if constexpr (MT > 1) {
#pragma unroll
      for (int s = 0; s < S; ++s) xa2[s] = __builtin_bit_cast(bf16x8, xr2[s]);
    }
  }

  float bv = -INFINITY;  // ARGMAX: running best of row t / 16 (threads with t % 16 == 0)
  int bi = 0x7fffffff;
  // The wavefronts' partial tiles summed through LDS, then the epilogue, one
  // thread per (m, n).
  auto finish = [&](int tile, const f32x4* c, const f32x4* c2, uint16_t hpre) {
    // C lane layout: column col, rows 4g + i (16 + 4g + i for the second row tile).
#pragma unroll
    for (int r = 0; r < NW; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) s_c[wv][r][4 * g + i][col] = c[r][i];
    if constexpr (MT > 1) {
#pragma unroll
      for (int r = 0; r < NW; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_c[wv][r][16 + 4 * g + i][col] = c2[r][i];
    }
    __syncthreads();
    if (t < 256 * MT) {
      const int m = t >> 4, j = t & 15, n = tile * 16 + j;
      float tot = 0.f, tot2 = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) {
        tot += s_c[w][0][m][j];
        if constexpr (NW == 2) tot2 += s_c[w][NW - 1][m][j];
      }
      const bool ok = m < mr && n < N;
      float h2 = 0.f;
      if (ok) h2 = epilogue<EPI>(a, m, n, tot, tot2, HPRE ? &hpre : nullptr);
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
    // RESID: the tile's residual element of this thread, issued behind the
    // tile's weights and ahead of the next tile's, so the epilogue finds it in
    // (not at 38 steps per wavefront, whose registers are full)
    uint16_t hpre = 0;
    if constexpr (HPRE) hpre = resid_load(a, (t >> 4) & (16 * MT - 1), tile * 16 + (t & 15));
    f32x4 c[NW], c2[MT > 1 ? NW : 1];
#pragma unroll
    for (int r = 0; r < NW; ++r) c[r] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (MT > 1) {
#pragma unroll
      for (int r = 0; r < NW; ++r) c2[r] = {0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int slot = s % PD;
#pragma unroll
      for (int r = 0; r < NW; ++r) {
        c[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[s], __builtin_bit_cast(bf16x8, wb[slot][r]),
                                                       c[r], 0, 0, 0);
        if constexpr (MT > 1)  // the same weights, rows 16..31: one weight pass for 32 rows
          c2[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa2[s], __builtin_bit_cast(bf16x8, wb[slot][r]),
                                                          c2[r], 0, 0, 0);
      }
      if (s + PD < S) issue(tile, s + PD, slot);
      else if constexpr (ISSUE) issue(next, s + PD - S, slot);
    }
    finish(tile, c, c2, hpre);
  };

  int tile = blockIdx.x;
  for (; tile + G < ntiles; tile += G) run(IntC<1>{}, tile, tile + G);
  if (tile < ntiles) run(IntC<0>{}, tile, tile);
  if constexpr (EPI == EPI_ARGMAX) {
    const int m = t >> 4;
    if (t < 256 * MT && (t & 15) == 0 && m < mr)
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

  uint16_t hpre = 0;
  // x (and the NORM gain) first: loads return in issue order, so the prologue
  // then runs while the weights stream instead of after them.
  bf16x8 xa[S];
  {
    const uint16_t* xrow = a.x + (long long)(mok ? col : 0) * K + kw0;
    uint4 xr[S], nwv[NORM ? S : 1];
#pragma unroll
    for (int s = 0; s < S; ++s) xr[s] = mok ? ldg16(xrow + 32 * s) : make_uint4(0, 0, 0, 0);
    float ssv = 0.f;  // the caller's row sums, loaded with x (as in layout 2)
    if constexpr (EPI == EPI_RESID)  // the residual, for the slice that merges
      hpre = resid_load(a, t >> 4, tile * 16 + (t & 15));
    if constexpr (NORM) {
      if (a.ss) ssv = a.ss[mok ? col : 0];
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
        rstd = mok ? rsqrtf(ssv / (float)K + a.eps) : 0.f;
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
  if (ok) h2 = epilogue<EPI>(a, m, n, tot, tot2, &hpre);
  if constexpr (EPI == EPI_RESID) {
    if (a.ss_out) {
      h2 = row_sum16(h2);
      if (j == 0 && m < mr) atomicAdd(a.ss_out + m, h2);
    }
  }
}

// layout 4: the layout-2 weight tiles cut into SK_CPT chunks of S K steps
// (K = 512 S), the T * SK_CPT chunks dealt out in order to workgroups of
// SK_W wavefronts, one chunk per wavefront ("stream-K"). Every CU then gets
// the same number of chunks, where layout 3's (tile, slice) workgroups leave
// some CUs one workgroup more than others (16 rows, down projection: 640
// workgroups of 4 wavefronts, and the time follows the CUs that hold 3). A
// workgroup's chunks span at most two tiles: its wavefronts' partial tiles are
// summed per tile through LDS (thread group 0 for the first tile, group 1 for
// the second), each sum goes to the tile's slot for this workgroup with
// device-coherent stores, and the workgroup counts itself on the tile's
// counter. The last of a tile's (2 or 3) workgroups adds the slots in
// workgroup order (the result does not depend on the arrival order), re-arms
// the counter and runs the epilogue.
// MT = 2: 32 rows of x, two MFMAs per weight load. x of both row tiles is
// loaded per K step with the weights (from L2: every tile reads all of x)
// instead of being held for the chunk (19 steps x 2 tiles would take 152
// VGPRs); rows past mrows load row 0 and are zeroed at the MFMA. Each merge
// thread handles rows m, m + 16, ... of its column. MT = 4: 64 rows the same way.
template <int EPI, int S, int PD, int MT = 1>
__global__ __launch_bounds__(64 * SK_W) void gemv_mfma_sk_kernel(GemvArgs a, int* __restrict__ ctr,
                                                                float* __restrict__ slots) {
  static_assert(EPI != EPI_ARGMAX && EPI != EPI_SWIGLU, "layout 4: F32, BF16 or RESID");
  static_assert(PD <= S, "the weight ring holds at most the chunk");
  static_assert(MT == 1 || MT == 2 || MT == 4, "16, 32 or 64 rows of x");
  __shared__ float s_c[SK_W][16 * MT][17];
  __shared__ int s_prev[2];
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63, col = lane & 15, g = lane >> 4;
  const int N = a.N, K = a.K, mr = a.mrows;
  const int T = (N + 15) / 16, KS = K / 32, nch = T * SK_CPT;
  const int c0 = blockIdx.x * SK_W;              // this workgroup's first chunk
  const int c = c0 + wv;                          // this wavefront's chunk
  const bool live = c < nch;
  const int cl = live ? c : nch - 1;              // past the end: a valid chunk, result unused
  const int tile = cl / SK_CPT;
  const int sb = (cl - tile * SK_CPT) * S;        // its first K step
  const int kw0 = sb * 32 + 8 * g;
  const bool mok = col < mr;

  const uint16_t* wlane = a.w + 8 * lane;
  const uint16_t* xrow = a.x + (long long)(mok ? col : 0) * K + kw0;
  // MT > 1: row col + 16 u of row tile u (row 0 when past mrows, then masked)
  const uint16_t* xrows[MT];
  uint32_t xmask[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    const bool ok = col + 16 * u < mr;
    xrows[u] = a.x + (long long)(ok ? col + 16 * u : 0) * K + kw0;
    xmask[u] = ok ? ~0u : 0u;
  }
  uint4 wb[PD];
  uint4 xb[MT > 1 ? PD : 1][MT];  // MT > 1: the step's x of every row tile
  auto issue = [&](int st, int slot) {
    if constexpr (MT > 1) {
#pragma unroll
      for (int u = 0; u < MT; ++u) xb[slot][u] = ldg16(xrows[u] + 32 * st);
    }
    wb[slot] = ldg16_stream(wlane + ((long long)tile * KS + sb + st) * 512);
  };
  // RESID: the residual elements this thread writes if its thread group's tile
  // (t0 + t / 256) is merged here, loaded with x
  uint16_t hpre[MT] = {};
  if constexpr (EPI == EPI_RESID) {
    const int tp = c0 / SK_CPT + (t >> 8);
#pragma unroll
    for (int u = 0; u < MT; ++u)
      hpre[u] = resid_load(a, 16 * u + ((t >> 4) & 15), (tp < T ? tp : T - 1) * 16 + (t & 15));
  }
  bf16x8 xa[MT == 1 ? S : 1];
  if constexpr (MT == 1) {
    uint4 xr[S];
#pragma unroll
    for (int st = 0; st < S; ++st) xr[st] = mok ? ldg16(xrow + 32 * st) : make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);  // x ahead of the weights
#pragma unroll
    for (int st = 0; st < PD; ++st) issue(st, st);
    __builtin_amdgcn_sched_barrier(0);  // the whole ring issued here
#pragma unroll
    for (int st = 0; st < S; ++st) xa[st] = __builtin_bit_cast(bf16x8, xr[st]);
  } else {
#pragma unroll
    for (int st = 0; st < PD; ++st) issue(st, st);
    __builtin_amdgcn_sched_barrier(0);  // the whole ring issued here
  }
  f32x4 acc[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) acc[u] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < S; ++st) {
    const int slot = st % PD;
    if constexpr (MT == 1) {
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[st], __builtin_bit_cast(bf16x8, wb[slot]),
                                                       acc[0], 0, 0, 0);
    } else {
      // zero the rows past mrows with masks (a select between the ring entry and
      // a zero vector would be turned into a select of addresses, in scratch)
#pragma unroll
      for (int u = 0; u < MT; ++u) {
        const uint4 v = xb[slot][u];
        const uint32_t k = xmask[u];
        const uint4 xv = make_uint4(v.x & k, v.y & k, v.z & k, v.w & k);
        acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xv),
                                                         __builtin_bit_cast(bf16x8, wb[slot]),
                                                         acc[u], 0, 0, 0);
      }
    }
    if (st + PD < S) issue(st + PD, slot);
  }
  // C lane layout: column col, rows 4g + i (16 u + 4g + i for row tile u).
#pragma unroll
  for (int u = 0; u < MT; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_c[wv][16 * u + 4 * g + i][col] = acc[u][i];
  __syncthreads();

  const int clast = (c0 + SK_W < nch ? c0 + SK_W : nch) - 1;
  const int t0 = c0 / SK_CPT, t1 = clast / SK_CPT;  // t1 - t0 <= 1 (SK_W < SK_CPT)
  const int gi = t >> 8;                            // thread group: tile t0 + gi
  const int tt = t0 + gi;
  const bool grp = gi <= t1 - t0;                   // uniform per wavefront
  const int r = t & 255, m = r >> 4, j = r & 15, n = tt * 16 + j;
  float tot[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) tot[u] = 0.f;
  int nwg = 1, sl = 0;
  if (grp) {
    const int v0 = (tt * SK_CPT > c0 ? tt * SK_CPT : c0) - c0;
    const int v1 = ((tt + 1) * SK_CPT < clast + 1 ? (tt + 1) * SK_CPT : clast + 1) - c0;
    for (int v = v0; v < v1; ++v)
#pragma unroll
      for (int u = 0; u < MT; ++u) tot[u] += s_c[v][16 * u + m][j];
    const int first = tt * SK_CPT / SK_W;
    nwg = (tt * SK_CPT + SK_CPT - 1) / SK_W - first + 1;
    sl = blockIdx.x - first;
    if (nwg > 1) {
#pragma unroll
      for (int u = 0; u < MT; ++u)
        __hip_atomic_store(slots + (((long long)tt * SK_SPT + sl) * MT + u) * 256 + r, tot[u],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's slot stores are performed
  __syncthreads();
  if (grp && r == 0 && nwg > 1)
    s_prev[gi] = __hip_atomic_fetch_add(ctr + tt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (!grp) return;
  if (nwg > 1) {
    if (s_prev[gi] != nwg - 1) return;
    const float* base = slots + (long long)tt * SK_SPT * MT * 256 + r;
    float v[SK_SPT][MT];
#pragma unroll
    for (int q = 0; q < SK_SPT; ++q)
#pragma unroll
      for (int u = 0; u < MT; ++u)
        v[q][u] = q < nwg ? __hip_atomic_load(base + (q * MT + u) * 256, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : 0.f;
#pragma unroll
    for (int u = 0; u < MT; ++u) {
      tot[u] = 0.f;
#pragma unroll
      for (int q = 0; q < SK_SPT; ++q)
        if (q < nwg) tot[u] += v[q][u];
    }
    if (r == 0) __hip_atomic_store(ctr + tt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    const int mm = 16 * u + m;
    const bool ok = mm < mr && n < N;
    float h2 = 0.f;
    if (ok) h2 = epilogue<EPI>(a, mm, n, tot[u], 0.f, &hpre[u]);
    if constexpr (EPI == EPI_RESID) {
      if (a.ss_out) {
        h2 = row_sum16(h2);
        if (j == 0 && mm < mr) atomicAdd(a.ss_out + mm, h2);
      }
    }
  }
}

// Two row tiles (MT = 2) are built only where launch_mfma sends them: SwiGLU with
// the short prefetch (PD < S, its doubled weights), every other epilogue with PD = S.
template <int EPI, int S, int PD, int MT>
constexpr bool mfma_built() {
  return MT == 1 || ((EPI == EPI_SWIGLU) == (PD < S));
}

template <int S, int PD, int WPG, int MT = 1>
int launch_mfma_s(const GemvArgs& a, int epi, bool norm, int grid, hipStream_t s) {
  const int ntiles = (a.N + 15) / 16;
#define KO_M(NORMV, EPIV)                                                              \
  if constexpr (mfma_built<EPIV, S, PD, MT>())                                         \
    hipLaunchKernelGGL((gemv_mfma_kernel<EPIV, NORMV, S, PD, WPG, MT>), dim3(grid),    \
                       dim3(64 * WPG), 0, s, a, ntiles);                               \
  else return KO_ENOTSUP
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


int launch_mfma(const GemvArgs& a, int epi, bool norm, int per_cu, int mt, hipStream_t s) {
  const int grid = mfma_grid(a.N, per_cu);
  if (mt == 2) {  // 32 rows per weight pass: x of both row tiles in registers (K <= 4096)
    switch (a.K) {
      case 2560:
        if (epi == EPI_SWIGLU) return launch_mfma_s<10, 5, 8, 2>(a, epi, norm, grid, s);
        return launch_mfma_s<10, 10, 8, 2>(a, epi, norm, grid, s);
      case 4096:
        if (epi == EPI_SWIGLU) return KO_ENOTSUP;
        return launch_mfma_s<16, 16, 8, 2>(a, epi, norm, grid, s);
      default: return KO_ENOTSUP;
    }
  }
  switch (a.K) {
    case 2560: return launch_mfma_s<10, 10, 8>(a, epi, norm, grid, s);
    case 4096: return launch_mfma_s<16, 16, 8>(a, epi, norm, grid, s);
    default:
      if (epi == EPI_SWIGLU) return KO_ENOTSUP;
      return launch_mfma_s<38, 19, 8>(a, epi, norm, grid, s);
  }
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


template <int S, int PD, int MT = 1>
int launch_mfma_sk_s(const GemvArgs& a, int epi, int* ctr, float* slots, hipStream_t s) {
  const dim3 grid(sk_grid(a.N));
#define KO_S(EPIV) \
  hipLaunchKernelGGL((gemv_mfma_sk_kernel<EPIV, S, PD, MT>), grid, dim3(64 * SK_W), 0, s, a, ctr, slots)
  switch (epi) {
    case EPI_F32: KO_S(EPI_F32); break;
    case EPI_BF16: KO_S(EPI_BF16); break;
    default: KO_S(EPI_RESID); break;
  }
#undef KO_S
  return KO_LAUNCH_STATUS();
}

int launch_mfma_sk(const GemvArgs& a, int epi, int mt, int* ctr, float* slots, hipStream_t s) {
  if (mt == 4) {  // 64 rows: x of four row tiles loaded per K step
    switch (sk_steps(a.K)) {
      case 19: return launch_mfma_sk_s<19, 6, 4>(a, epi, ctr, slots, s);
      case 8: return launch_mfma_sk_s<8, 6, 4>(a, epi, ctr, slots, s);
      case 5: return launch_mfma_sk_s<5, 5, 4>(a, epi, ctr, slots, s);
      default: return KO_ENOTSUP;
    }
  }
  if (mt == 2) {  // 32 rows: x of both row tiles loaded per K step
    switch (sk_steps(a.K)) {
      case 19: return launch_mfma_sk_s<19, 12, 2>(a, epi, ctr, slots, s);
      case 8: return launch_mfma_sk_s<8, 8, 2>(a, epi, ctr, slots, s);
      case 5: return launch_mfma_sk_s<5, 5, 2>(a, epi, ctr, slots, s);
      default: return KO_ENOTSUP;
    }
  }
  switch (sk_steps(a.K)) {
    case 19: return launch_mfma_sk_s<19, 10>(a, epi, ctr, slots, s);
    case 8: return launch_mfma_sk_s<8, 8>(a, epi, ctr, slots, s);
    case 5: return launch_mfma_sk_s<5, 5>(a, epi, ctr, slots, s);
    default: return KO_ENOTSUP;
  }
}


}  // namespace

namespace ko {

int launch_layout2(const GemvArgs& a, int epi, bool norm, int per_cu, int mt, hipStream_t s) {
  return launch_mfma(a, epi, norm, per_cu, mt, s);
}

int launch_layout3(const GemvArgs& a, int epi, bool norm, int slices, int* ctr, float* slots,
                   hipStream_t s) {
  return launch_mfma_ks(a, epi, norm, slices, ctr, slots, s);
}

int launch_layout4(const GemvArgs& a, int epi, int mt, int* ctr, float* slots, hipStream_t s) {
  return launch_mfma_sk(a, epi, mt, ctr, slots, s);
}

}  // namespace ko
