// Every decoder layer of one decode step (one query token, 1-2 sequences) in a
// single launch for gfx950.
//
// Replaces the per-layer loop of engine/engine.py:325-335 (add_rms_norm, the
// qkv / o / gate|up / down projections, qk_norm_rope, decode attention,
// silu_mul) for T = 1. Each layer is five stages of workgroups, in index order:
//   S0 qkv    : qkv <- W_qkv bf16(w_in * bf16(h * rstd))          (GEMV, NORM)
//   S1 attn   : q/k RMSNorm + RoPE, KV append, split-K attention, fused
//               combine -> attn                                    (attn1_body)
//   S2 o      : h <- bf16(h + bf16(W_o attn))                     (GEMV, RESID)
//   S3 gate|up: act <- bf16(silu(g) * u) of W_gu bf16(w_post * ...)(GEMV, SWIGLU)
//   S4 down   : h <- bf16(h + bf16(W_down act))                   (GEMV, RESID)
// with the same arithmetic and rounding as the separate launches. A stage's
// workgroups issue their weight (or cached key/value) loads first and then wait
// for the stage that produces their input (stage_sync.h), so the weights of
// the next stage stream while the current one finishes: the launch boundary,
// and the first-load latency behind it, that separate launches pay per stage
// is gone. Activations written and read inside the launch go through
// device-coherent stores and loads; the per-XCD L2 never serves them stale.
//
// Buffers: h [B, H] residual stream (in: the step's embeddings; out: the last
// layer's output), qkv [B, (nq+2nkv)*D], attn [B, nq*D], act [B, I] scratch
// activations; the attention's o_part/ml scratch as for ko_decode_attn_qkv;
// counters [L][B*nkv] and sync [L][5][STAGE_INTS] zero before the first launch
// (every launch leaves them zero); err set to 1 if a wait gave up.
#include "attn_core.h"
#include "stage_sync.h"

using namespace ko;

namespace {

// One row of the layer table (device memory): the layer's weights and cache.
struct LayerPtrs {
  const uint16_t* w_in;    // [H] input RMSNorm gain
  const uint16_t* qkv;     // [(nq+2nkv)*D, H]
  const uint16_t* q_norm;  // [D]
  const uint16_t* k_norm;  // [D]
  const uint16_t* o;       // [H, nq*D]
  const uint16_t* w_post;  // [H] post-attention RMSNorm gain
  const uint16_t* gu;      // [2I, H]: gate rows, then up rows
  const uint16_t* down;    // [H, I]
  uint16_t* kc;            // this layer's K cache [B, nkv, cap, D]
  uint16_t* vc;
};

constexpr int NSTAGE = 5;
enum { S_QKV = 0, S_ATTN, S_O, S_GU, S_DOWN };
// output columns per row group: qkv and o 8, gate|up and down 4 (their weight
// double buffers then fit the register budget the attention stage sets)
constexpr int R_QKV = 8, R_O = 8, R_GU = 4, R_DOWN = 4;
constexpr int CPT_H = 2;  // K = H, nq*D <= 2 * 2048
constexpr int CPT_I = 5;  // K = I <= 5 * 2048
constexpr int GMAX = 32;  // row groups per GEMV workgroup

struct LayersArgs {
  const LayerPtrs* layers;
  int L, per_layer;
  int nwg[NSTAGE];
  AttnArgs at;  // the layer's gains, cache and counters are filled in per workgroup
  uint16_t *h, *qkv, *attn, *act;
  int B, H, I, NQKV, QD;
  float eps;
  int* counters;
  int* sync;
  int* err;
  int o_delay_ticks;
};

// The attention stage's side of the hand-off: wait for S0 once per workgroup;
// the merge that completes the live pairs raises S1's flag and lowers S0's
// (every S1 workgroup that waited is past its wait by then).
struct ChainAttnHooks {
  static constexpr bool kWaitInput = true;
  static constexpr bool kNotify = true;
  int* prev;
  int* self;
  int* err;
  bool raise;
  __device__ void wait_input() const {
    if (threadIdx.x == 0) stage_wait(prev, blockIdx.x, err);
    __syncthreads();
  }
  __device__ void finish() const {
    if (raise) stage_flags(self, 1);
    stage_flags(prev, 0);
  }
  __device__ void merged(const AttnArgs&, int live) const {
    if (stage_arrive1(self, live)) finish();
  }
  __device__ void no_units() const {
    wait_input();
    if (threadIdx.x == 0) finish();
  }
};

// A GEMV stage's workgroup wg of nwg: row groups wg, wg + nwg, ... (G >= 2 of
// them), R output columns each, over the whole K, with the arithmetic and
// summation order of gemv_row_body (per-thread 8-element chunks t + 256 j,
// 16-lane row sums, then the 16 partials in order). Two
// groups' weights are in flight at any time (buffers A and B, refilled right
// after they are consumed), the first two before the wait for the input, so a
// workgroup streams continuously and pays its start-up, the wait and the final
// store acknowledgement once. x (and the NORM gain) are read once after the
// wait, with device-scope loads, and kept in registers; RESID's h entries of all
// the workgroup's groups are read then too (to LDS). Epilogue: one lane of
// wavefront 0 per output (sequence m, column r) sums that column's 16 partials;
// two quad-permute moves gather four columns' bf16 results into the lane that
// stores them with one device-coherent 8-byte store.
template <int M, int R, bool NORM, int EPI, int CPT, class WaitX>
__device__ __forceinline__ void gemv_loop(const GemvArgs& a, int wg, int nwg, WaitX&& wait_x) {
  constexpr int NW = EPI == EPI_SWIGLU ? 2 * R : R;
  constexpr int Q = R / 4;
  static_assert(R % 4 == 0 && M * R <= 64, "quads of outputs in wavefront 0");
  __shared__ float red[2][16][M * NW];
  __shared__ float s_sq[GEMV_NT / 64][M];
  __shared__ uint16_t s_h[EPI == EPI_RESID ? GMAX * M * R : 1];

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int N = a.N, K = a.K, KC = K >> 3, mr = a.mrows;
  const int ngroups = N / R;
  const int G = (ngroups - wg + nwg - 1) / nwg;  // this workgroup's groups (>= 2)

  auto issue = [&](int gi, uint4 (&w)[CPT][NW]) {
    const int n0 = (wg + gi * nwg) * R;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = min(t + GEMV_NT * j, KC - 1);
#pragma unroll
      for (int r = 0; r < NW; ++r) {
        const int n = r < R ? n0 + r : N + n0 + r - R;
        w[j][r] = ldg16_stream(a.w + (long long)n * K + 8 * c);
      }
    }
  };
  uint4 wa[CPT][NW], wb[CPT][NW];
  issue(0, wa);
  issue(1, wb);
  wait_x();

  uint4 xr[M][CPT];
  uint4 nwr[NORM ? CPT : 1];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = min(t + GEMV_NT * j, KC - 1);
#pragma unroll
    for (int m = 0; m < M; ++m) xr[m][j] = ldg16_coherent(a.x + (long long)(m < mr ? m : 0) * K + 8 * c);
    if constexpr (NORM) nwr[j] = ldg16(a.nw + 8 * c);
  }
  if constexpr (EPI == EPI_RESID) {  // h quads of every group: [gi][m][column]
    for (int i = t; i < G * M * Q; i += GEMV_NT) {
      const int gi = i / (M * Q), rem = i - gi * (M * Q), m = rem / Q, q = rem - m * Q;
      const uint2 hq = m < mr ? ldg8_coherent(a.h + (long long)m * N + (wg + gi * nwg) * R + 4 * q)
                              : make_uint2(0, 0);
      *reinterpret_cast<uint2*>(&s_h[(gi * M + m) * R + 4 * q]) = hq;
    }
  }
  const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < CPT; ++j)
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (t + GEMV_NT * j >= KC || m >= mr) xr[m][j] = zero;
  if constexpr (NORM) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float sq = 0.f;
#pragma unroll
      for (int j = 0; j < CPT; ++j) sq += sq8(xr[m][j]);
      sq = wave_sum(sq);
      if (lane == 0) s_sq[wv][m] = sq;
    }
    __syncthreads();
    float rstd[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float tot = 0.f;
#pragma unroll
      for (int i = 0; i < GEMV_NT / 64; ++i) tot += s_sq[i][m];
      rstd[m] = rsqrtf(tot / (float)K + a.eps);
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j)
#pragma unroll
      for (int m = 0; m < M; ++m) xr[m][j] = norm8(xr[m][j], nwr[j], rstd[m]);
  }

  // group gi from buffer w, through red[p]
  auto compute = [&](int gi, int p, const uint4 (&w)[CPT][NW]) {
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
        if ((lane & 15) == 0) red[p][wv * 4 + (lane >> 4)][m * NW + r] = v;
      }
    __syncthreads();  // also orders the s_h fills before their first reads
    if (t < M * R) {  // lane (m, r); quads of lanes hold 4 consecutive columns
      const int m = t / R, r = t - m * R;
      float tot = 0.f, tot2 = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        tot += red[p][k][m * NW + r];
        if constexpr (EPI == EPI_SWIGLU) tot2 += red[p][k][m * NW + R + r];
      }
      float v;
      if constexpr (EPI == EPI_BF16) {
        v = tot;
      } else if constexpr (EPI == EPI_SWIGLU) {
        const float gt = round_bf16(tot), u = round_bf16(tot2);
        v = round_bf16(gt / (1.0f + expf(-gt))) * u;
      } else {  // RESID: h <- bf16(h + bf16(y))
        v = bf16_to_f32(s_h[(gi * M + m) * R + r]) + round_bf16(tot);
      }
      const int b = f32_to_bf16(v);
      const int pair = b | (dpp_i<0xB1>(b) << 16);         // quad_perm(1,0,3,2): lanes 2j, 2j+1
      const int hi = dpp_i<0x4E>(pair);                      // quad_perm(2,3,0,1): the other pair
      if ((r & 3) == 0 && m < mr) {
        uint16_t* dst = EPI == EPI_RESID ? a.h : static_cast<uint16_t*>(a.y);
        stg8_coherent(dst + (long long)m * N + (wg + gi * nwg) * R + r,
                      make_uint2((uint32_t)pair, (uint32_t)hi));
      }
    }
  };
  // Buffers alternate; a refill is issued right after its buffer is consumed,
  // and only for a group that exists, at the end of the iteration so the
  // outstanding loads at every compute are the same on all paths.
  for (int gi = 0;; gi += 2) {
    compute(gi, 0, wa);
    if (gi + 2 >= G) {
      if (gi + 1 < G) compute(gi + 1, 1, wb);
      break;
    }
    issue(gi + 2, wa);
    compute(gi + 1, 1, wb);
    if (gi + 3 >= G) {
      compute(gi + 2, 0, wa);
      break;
    }
    issue(gi + 3, wb);
  }
}

// One GEMV stage workgroup: gemv_loop after an optional delay, waiting for
// `prev` (none for the launch's first stage); then its stores are performed
// and it arrives; the arrival that completes the stage raises its flag (unless
// nothing in the launch reads it) and lowers prev's.
template <int M, int R, bool NORM, int EPI, int CPT>
__device__ __forceinline__ void gemv_stage(const GemvArgs& g, int wg, int nwg, int* prev,
                                           int* self, bool raise, int* err, int delay_ticks) {
  if (delay_ticks > 0) {  // let the previous stage's latency-bound loads go first
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < (unsigned long long)delay_ticks) __builtin_amdgcn_s_sleep(4);
  }
  auto wait = [&] {
    if (prev) {
      if (threadIdx.x == 0) stage_wait(prev, wg, err);
      __syncthreads();
    }
  };
  gemv_loop<M, R, NORM, EPI, CPT>(g, wg, nwg, wait);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's output stores are performed
  __syncthreads();
  if (threadIdx.x == 0 && stage_arrive(self, wg, nwg)) {
    if (raise) stage_flags(self, 1);
    if (prev) stage_flags(prev, 0);
  }
}

template <int M>
__global__ __launch_bounds__(256) void decode_layers_kernel(LayersArgs a) {
  const int l = blockIdx.x / a.per_layer;
  int wg = blockIdx.x - l * a.per_layer;
  const LayerPtrs lw = a.layers[l];
  int* sy = a.sync + (long long)l * NSTAGE * STAGE_INTS;
  GemvArgs g = {};
  g.mrows = a.B;
  g.eps = a.eps;
  if (wg < a.nwg[S_QKV]) {
    g.x = a.h;
    g.w = lw.qkv;
    g.y = a.qkv;
    g.nw = lw.w_in;
    g.N = a.NQKV;
    g.K = a.H;
    int* prev = l > 0 ? sy - STAGE_INTS : nullptr;  // S4 of layer l - 1
    gemv_stage<M, R_QKV, true, EPI_BF16, CPT_H>(g, wg, a.nwg[S_QKV], prev, sy + S_QKV * STAGE_INTS,
                                                true, a.err, 0);
    return;
  }
  wg -= a.nwg[S_QKV];
  if (wg < a.nwg[S_ATTN]) {
    AttnArgs at = a.at;
    at.qw = lw.q_norm;
    at.kw = lw.k_norm;
    at.kc = lw.kc;
    at.vc = lw.vc;
    at.counters = a.counters + (long long)l * a.B * at.nkv;
    const ChainAttnHooks hk{sy + S_QKV * STAGE_INTS, sy + S_ATTN * STAGE_INTS, a.err, true};
    attn1_body<true, 4, true>(at, wg, a.nwg[S_ATTN], hk);
    return;
  }
  wg -= a.nwg[S_ATTN];
  if (wg < a.nwg[S_O]) {
    g.x = a.attn;
    g.w = lw.o;
    g.h = a.h;
    g.N = a.H;
    g.K = a.QD;
    gemv_stage<M, R_O, false, EPI_RESID, CPT_H>(g, wg, a.nwg[S_O], sy + S_ATTN * STAGE_INTS,
                                                sy + S_O * STAGE_INTS, true, a.err, a.o_delay_ticks);
    return;
  }
  wg -= a.nwg[S_O];
  if (wg < a.nwg[S_GU]) {
    g.x = a.h;
    g.w = lw.gu;
    g.y = a.act;
    g.nw = lw.w_post;
    g.N = a.I;
    g.K = a.H;
    gemv_stage<M, R_GU, true, EPI_SWIGLU, CPT_H>(g, wg, a.nwg[S_GU], sy + S_O * STAGE_INTS,
                                                 sy + S_GU * STAGE_INTS, true, a.err, 0);
    return;
  }
  wg -= a.nwg[S_GU];
  g.x = a.act;
  g.w = lw.down;
  g.h = a.h;
  g.N = a.H;
  g.K = a.I;
  gemv_stage<M, R_DOWN, false, EPI_RESID, CPT_I>(g, wg, a.nwg[S_DOWN], sy + S_GU * STAGE_INTS,
                                                  sy + S_DOWN * STAGE_INTS, l < a.L - 1, a.err, 0);
}

}  // namespace

extern "C" {

long long ko_decode_layers_sync_ints(int L) { return (long long)(L > 0 ? L : 0) * NSTAGE * STAGE_INTS; }

int ko_decode_layers(const void* layer_table, int L, void* h, void* qkv, void* attn, void* act,
                     int B, int H, int I, int nkv, int head_dim, const void* cos, const void* sin,
                     int max_pos, const int* pos, int cap, long long cache_b_stride,
                     long long cache_h_stride, int unit, int max_units, int grid_waves, float eps,
                     float scale, float* o_part, float* ml, int* counters, int* sync, int* err,
                     const int* gemv_wgs, int delay_ns, void* stream) {
  if (!layer_table || !h || !qkv || !attn || !act || !cos || !sin || !pos || !o_part || !ml ||
      !counters || !sync || !err)
    return KO_EINVAL;
  if (L < 1 || B < 1 || nkv < 1 || cap < 1 || max_pos < 1) return KO_EINVAL;
  if (head_dim != D) return KO_ENOTSUP;
  if (B > 2) return KO_ENOTSUP;
  if (unit < 16 || (unit & 15)) return KO_EINVAL;
  if (waves_per_unit(unit) != 4) return KO_ENOTSUP;
  if ((long long)max_units * unit < cap) return KO_ERANGE;
  if (grid_waves < 4 || (grid_waves & 3)) return KO_EINVAL;
  if ((cache_b_stride & 7) || (cache_h_stride & 7) || cache_b_stride < 0 || cache_h_stride < 0)
    return KO_EINVAL;
  const int QD = nkv * G * D, NQKV = (nkv * G + 2 * nkv) * D;
  if (H < 16 || H % 8 || I < 16 || I % 8) return KO_EINVAL;
  if (H > CPT_H * GEMV_NT * 8 || QD > CPT_H * GEMV_NT * 8 || I > CPT_I * GEMV_NT * 8)
    return KO_ENOTSUP;
  if (!aligned16(layer_table) || !aligned16(h) || !aligned16(qkv) || !aligned16(attn) ||
      !aligned16(act) || !aligned16(cos) || !aligned16(sin) || !aligned16(o_part))
    return KO_EINVAL;

  LayersArgs a = {};
  a.layers = static_cast<const LayerPtrs*>(layer_table);
  a.L = L;
  // workgroups per GEMV stage: 2 <= row groups per workgroup <= GMAX
  const int groups[4] = {NQKV / R_QKV, H / R_O, I / R_GU, H / R_DOWN};
  const int dflt[4] = {256, 160, 304, 160};
  const int stage_of[4] = {S_QKV, S_O, S_GU, S_DOWN};
  for (int i = 0; i < 4; ++i) {
    const int lo = (groups[i] + GMAX - 1) / GMAX, hi = groups[i] / 2;
    if (lo > hi) return KO_ENOTSUP;
    int n = gemv_wgs && gemv_wgs[i] > 0 ? gemv_wgs[i] : dflt[i];
    if (gemv_wgs && gemv_wgs[i] > 0 && (n < lo || n > hi)) return KO_ERANGE;
    a.nwg[stage_of[i]] = n < lo ? lo : n > hi ? hi : n;
  }
  a.nwg[S_ATTN] = grid_waves / 4;
  a.per_layer = 0;
  for (int s = 0; s < NSTAGE; ++s) a.per_layer += a.nwg[s];
  if ((long long)a.per_layer * L > 0x7fffffffLL) return KO_ERANGE;
  // kc / vc / gains / counters per layer come from the table inside the kernel
  a.at = base_args(nullptr, nullptr, pos, 1, cap, cache_b_stride, cache_h_stride, B, nkv, unit,
                   max_units, scale, o_part, ml);
  a.at.qkv = static_cast<const uint16_t*>(qkv);
  a.at.cosb = static_cast<const uint16_t*>(cos);
  a.at.sinb = static_cast<const uint16_t*>(sin);
  a.at.eps = eps;
  a.at.max_pos = max_pos;
  a.at.out = static_cast<uint16_t*>(attn);
  a.h = static_cast<uint16_t*>(h);
  a.qkv = static_cast<uint16_t*>(qkv);
  a.attn = static_cast<uint16_t*>(attn);
  a.act = static_cast<uint16_t*>(act);
  a.B = B;
  a.H = H;
  a.I = I;
  a.NQKV = NQKV;
  a.QD = QD;
  a.eps = eps;
  a.counters = counters;
  a.sync = sync;
  a.err = err;
  a.o_delay_ticks = delay_ns > 0 ? delay_ns / 10 : 0;  // s_memrealtime runs at 100 MHz
  const dim3 grid(a.per_layer * L), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 1)
    hipLaunchKernelGGL((decode_layers_kernel<1>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((decode_layers_kernel<2>), grid, block, 0, s, a);
  return KO_LAUNCH_STATUS();
}

}  // extern "C"
