// Decode attention, the o projection and the gate/up projection in one launch
// (one query token, 1-2 sequences): engine/engine.py:279-285 from the q/k norm
// + RoPE + KV append through the SwiGLU gate/up GEMV, i.e. qk_norm_rope_acc
// (engine/kernels/gemv.py:219-268), DecodeAttention (fused.py:204-234), the o
// GEMV with its residual add (gemv.py EPI_RESID) and the gate/up GEMV with its
// RMSNorm prologue and SwiGLU epilogue (gemv.py NORM + EPI_SWIGLU).
//
// Why one launch: at batch 1 the attention is a latency chain (q/k norm, a few
// 16-key steps, the partial merge) during which HBM is mostly idle, and the
// projections after it are weight streams that do not depend on it until their
// dot products. Workgroups are dispatched in index order:
//   [0, nattn)              attention units (attn1_body, fused merge)
//   [nattn, nattn + n_o)    o projection, 16 output columns each
//   [nattn + n_o, end)      gate/up projection, 16 output columns (16 gate and
//                           16 up weight rows) each
// A projection workgroup issues all its weight loads as soon as it is
// resident (after a short delay that lets the attention's loads go first),
// then waits for its input: the o projection for every (sequence, KV head)
// pair to be merged (the done flags of ko_decode_attn_qkv_oproj), the gate/up
// projection for every o-projection workgroup to have stored its residual
// columns (a second set of done flags). The gate/up workgroups that are
// resident during the attention hold their weights in registers while they
// wait; the rest are dispatched as earlier workgroups leave and stream as in
// a plain GEMV. Producers always have lower indices than their consumers, so
// every producer is resident or finished before a consumer can wait on it.
//
// Weight rows are row-major; a wavefront owns whole rows and each of its load
// instructions reads 1 KiB of one row (lane l: 16-byte chunks l, l + 64, ...),
// so its lanes also hold x's chunks l, l + 64, ... in registers and the NORM
// row sums need no cross-wave traffic.
#include "attn_core.h"

using namespace ko;

namespace {

constexpr int O_COLS = 16;   // o-projection columns per workgroup
// gate/up columns per workgroup (as many gate and up rows): 16 for one row of x,
// 8 for two (registers: the weights of the rows stay in flight during the wait)
template <int M>
constexpr int gu_cols() {
  return M == 1 ? 16 : 8;
}
// Second sync block (after the OPROJ_SYNC_INTS of the attention -> o hand-off):
// [0] o-projection groups done; then GU_FLAGS lines 128 bytes apart holding the
// gate/up input-ready flag, the count of that group's finished gate/up
// workgroups, and the count of that group's finished o-projection workgroups.
constexpr int GU_FLAG0 = 32, GU_FLAG_STRIDE = 32, GU_FLAGS = 32;
constexpr int MLP_SYNC_INTS = OPROJ_SYNC_INTS + GU_FLAG0 + GU_FLAG_STRIDE * GU_FLAGS;

struct MlpArgs {
  // o projection: x = the merged attention output [M, KO] (written in this
  // launch), w_o [H, KO], h [M, H] (residual, updated in place)
  const uint16_t* out;
  const uint16_t* w_o;
  uint16_t* h;
  int H;
  // gate/up: x = h [M, H] after the o projection, w_gu [2I, H] (gate | up),
  // w_post [H] (RMSNorm gain), act [M, I]
  const uint16_t* w_gu;
  const uint16_t* w_post;
  uint16_t* act;
  int I;
  float eps;
  int mrows;
  int* sync2;  // the second sync block
  int* err;
  int o_delay, gu_delay;  // s_memrealtime ticks (100 MHz)
};

__device__ __forceinline__ void delay_ticks(int ticks) {
  if (ticks > 0) {
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < (unsigned long long)ticks) __builtin_amdgcn_s_sleep(4);
  }
}

// Thread 0 polls a device-coherent flag (bounded: SPIN_MAX polls, then *err is
// set); returns true when the wait gave up. Every thread leaves after the poll.
__device__ __forceinline__ bool wait_flag(int* flag, int* err) {
  __shared__ int s_to;
  if (threadIdx.x == 0) {
    int it = 0, to = 0;
    while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
      __builtin_amdgcn_s_sleep(8);
      if (++it >= SPIN_MAX) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        to = 1;
        break;
      }
    }
    s_to = to;
  }
  __syncthreads();
  return s_to != 0;
}

// Arrival of one workgroup of a group of `in_grp` (thread 0): true for the last.
__device__ __forceinline__ bool arrive(int* ctr, int in_grp) {
  return __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == in_grp - 1;
}

// o projection, 16 columns of h per workgroup (K = 4096: 4 rows per wavefront,
// 8 chunks of each per lane), RESID epilogue h <- bf16(h + bf16(acc)) stored
// device-coherently for the gate/up workgroups of this launch.
template <int M>
__device__ void oproj_role(const AttnArgs& a, const MlpArgs& p, int wg, int nog) {
  constexpr int K = 4096, CPL = K / 512, RPW = O_COLS / 4;
  __shared__ float s_tot[M][O_COLS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = wg * O_COLS;
  delay_ticks(p.o_delay);
  uint4 w[RPW][CPL];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int n = min(n0 + wave * RPW + r, p.H - 1);
#pragma unroll
    for (int j = 0; j < CPL; ++j) w[r][j] = ldg16_stream(p.w_o + (long long)n * K + 8 * (lane + 64 * j));
  }
  // wait until every (sequence, KV head) pair has been merged
  const int grp = wg % OPROJ_FLAGS;
  int* flag = a.pairs_done + OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * grp;
  const bool timed_out = wait_flag(flag, p.err);
  uint4 x[M][CPL];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      x[m][j] = ldg16_coherent(p.out + (long long)(m < p.mrows ? m : 0) * K + 8 * (lane + 64 * j));
  float acc[M][RPW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) s = dot8(x[m][j], w[r][j], s);
      acc[m][r] = s;
    }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const float v = wave_sum(acc[m][r]);
      if (lane == 0) s_tot[m][wave * RPW + r] = v;
    }
  __syncthreads();
  if (t < M * O_COLS) {
    const int m = t / O_COLS, c = t - m * O_COLS, n = n0 + c;
    if (m < p.mrows && n < p.H) {
      uint16_t* hp = p.h + (long long)m * p.H + n;
      const float hn = round_bf16(bf16_to_f32(*hp) + round_bf16(s_tot[m][c]));
      __hip_atomic_store(hp, f32_to_bf16(hn), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's residual columns are performed
  __syncthreads();
  if (t == 0) {
    // the gate/up input is ready once every o-projection workgroup has arrived:
    // count in GU_FLAGS groups, then the groups; the last raises every flag
    const int g2 = wg % GU_FLAGS;
    int* line = p.sync2 + GU_FLAG0 + GU_FLAG_STRIDE * g2;
    const int in_g2 = (nog - g2 + GU_FLAGS - 1) / GU_FLAGS;
    if (arrive(line + 2, in_g2)) {
      __hip_atomic_store(line + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int groups = nog < GU_FLAGS ? nog : GU_FLAGS;
      if (arrive(p.sync2, groups)) {
        __hip_atomic_store(p.sync2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int f = 0; f < GU_FLAGS; ++f)
          __hip_atomic_store(p.sync2 + GU_FLAG0 + GU_FLAG_STRIDE * f, 1, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // re-arm the attention -> o hand-off (as attn_oproj_kernel): the last of a
    // flag group clears the flag and counts the group, the last group clears
    // the pair count; a workgroup whose wait gave up leaves it armed (*err set)
    if (!timed_out) {
      const int in_grp = (nog - grp + OPROJ_FLAGS - 1) / OPROJ_FLAGS;
      if (arrive(flag + 1, in_grp)) {
        __hip_atomic_store(flag, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(flag + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int groups = nog < OPROJ_FLAGS ? nog : OPROJ_FLAGS;
        if (arrive(a.pairs_done + 1, groups)) {
          __hip_atomic_store(a.pairs_done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(a.pairs_done + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
}

// gate/up projection, GU = gu_cols<M>() columns per workgroup (K = 2560:
// wavefronts 0-1 hold the GU gate rows, 2-3 the GU up rows, GU / 2 rows per
// wavefront, 5 chunks of each per lane), RMSNorm prologue on h (computed from
// the row, as gemv.py's NORM with the row's own sum of squares), SwiGLU
// epilogue into act.
template <int M>
__device__ void gateup_role(const MlpArgs& p, int wg, int nug) {
  constexpr int GU_COLS = gu_cols<M>();
  constexpr int K = 2560, CPL = K / 512, RPW = 2 * GU_COLS / 4;
  __shared__ float s_tot[M][2 * GU_COLS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = wg * GU_COLS;
  const int up = wave >= 2;  // waves 2-3: up rows
  const int cbase = n0 + (wave & 1) * RPW;
  delay_ticks(p.gu_delay);
  uint4 w[RPW][CPL];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int n = up * p.I + min(cbase + r, p.I - 1);
#pragma unroll
    for (int j = 0; j < CPL; ++j) w[r][j] = ldg16_stream(p.w_gu + (long long)n * K + 8 * (lane + 64 * j));
  }
  const int grp = wg % GU_FLAGS;
  int* line = p.sync2 + GU_FLAG0 + GU_FLAG_STRIDE * grp;
  const bool timed_out = wait_flag(line, p.err);
  uint4 x[M][CPL], nwc[CPL];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      x[m][j] = ldg16_coherent(p.h + (long long)(m < p.mrows ? m : 0) * K + 8 * (lane + 64 * j));
#pragma unroll
  for (int j = 0; j < CPL; ++j) nwc[j] = ldg16(p.w_post + 8 * (lane + 64 * j));
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) sq += sq8(x[m][j]);
    const float rstd = rsqrtf(wave_sum(sq) / (float)K + p.eps);
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[m][j] = norm8(x[m][j], nwc[j], rstd);
  }
  float acc[M][RPW];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) s = dot8(x[m][j], w[r][j], s);
      acc[m][r] = s;
    }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const float v = wave_sum(acc[m][r]);
      if (lane == 0) s_tot[m][wave * RPW + r] = v;  // [0, 16) gate, [16, 32) up
    }
  __syncthreads();
  if (t < M * GU_COLS) {
    const int m = t / GU_COLS, c = t - m * GU_COLS, n = n0 + c;
    if (m < p.mrows && n < p.I) {
      const float g = round_bf16(s_tot[m][c]), u = round_bf16(s_tot[m][GU_COLS + c]);
      const float s = round_bf16(g / (1.0f + expf(-g)));
      p.act[(long long)m * p.I + n] = f32_to_bf16(s * u);
    }
  }
  // re-arm: the last gate/up workgroup of a flag group clears the flag
  if (t == 0 && !timed_out) {
    const int in_grp = (nug - grp + GU_FLAGS - 1) / GU_FLAGS;
    if (arrive(line + 1, in_grp)) {
      __hip_atomic_store(line, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(line + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

struct MlpHooks {
  static constexpr bool kNotify = true;
  __device__ void merged(const AttnArgs& a, int live) const {
    const int prev =
        __hip_atomic_fetch_add(a.pairs_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == live - 1) {
      for (int f = 0; f < OPROJ_FLAGS; ++f)
        __hip_atomic_store(a.pairs_done + OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * f, 1,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __device__ void no_units() const {}  // the projection workgroups then time out (*err)
};

template <int M>
__global__ __launch_bounds__(256) void attn_o_gu_kernel(AttnArgs a, MlpArgs p, int nattn,
                                                        int nog) {
  const int wg = blockIdx.x;
  if (wg < nattn) {
    attn1_body<true, 4, true>(a, wg, nattn, MlpHooks{});
  } else if (wg < nattn + nog) {
    oproj_role<M>(a, p, wg - nattn, nog);
  } else {
    gateup_role<M>(p, wg - nattn - nog, gridDim.x - nattn - nog);
  }
}

}  // namespace

extern "C" {

long long ko_decode_attn_oproj_gateup_sync_ints(void) { return MLP_SYNC_INTS; }

int ko_decode_attn_oproj_gateup(const void* qkv, const void* q_w, const void* k_w,
                                const void* cos, const void* sin, int max_pos, const int* pos,
                                void* k_cache, void* v_cache, int cap, long long cache_b_stride,
                                long long cache_h_stride, int B, int nkv, int head_dim, int unit,
                                int max_units, int grid_waves, float eps, float scale,
                                float* o_part, float* ml, int* counters, void* out,
                                const void* w_o, void* h, int H, const void* w_gu,
                                const void* w_post, void* act, int I, int* sync, int* err,
                                int o_delay_ns, int gu_delay_ns, const void* rope, void* stream) {
  int st = check_common(k_cache, v_cache, pos, cap, cache_b_stride, cache_h_stride, B, 1, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (!qkv || !q_w || !k_w || !cos || !sin || !out || !counters || !w_o || !h || !w_gu ||
      !w_post || !act || !sync || !err || max_pos < 1 || grid_waves < 4)
    return KO_EINVAL;
  if (!aligned16(qkv) || !aligned16(q_w) || !aligned16(k_w) || !aligned16(cos) ||
      !aligned16(sin) || !aligned16(out) || !aligned16(w_o) || !aligned16(h) ||
      !aligned16(w_gu) || !aligned16(w_post) || !aligned16(act) || (rope && !aligned16(rope)))
    return KO_EINVAL;
  // the shapes the workgroup roles are built for: the o projection's input
  // width nq * head_dim = 4096 and the hidden size 2560 (Qwen3-4B)
  if (B > 2 || waves_per_unit(unit) != 4 || nkv * G * D != 4096 || H != 2560 || I < 1 ||
      (I & 7))
    return KO_ENOTSUP;
  AttnArgs a = base_args(k_cache, v_cache, pos, 1, cap, cache_b_stride, cache_h_stride, B, nkv,
                         unit, max_units, scale, o_part, ml);
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.qw = static_cast<const uint16_t*>(q_w);
  a.kw = static_cast<const uint16_t*>(k_w);
  a.cosb = static_cast<const uint16_t*>(cos);
  a.sinb = static_cast<const uint16_t*>(sin);
  a.eps = eps;
  a.max_pos = max_pos;
  a.counters = counters;
  a.out = static_cast<uint16_t*>(out);
  a.pairs_done = sync;
  a.rope = static_cast<const uint16_t*>(rope);
  MlpArgs p = {};
  p.out = static_cast<const uint16_t*>(out);
  p.w_o = static_cast<const uint16_t*>(w_o);
  p.h = static_cast<uint16_t*>(h);
  p.H = H;
  p.w_gu = static_cast<const uint16_t*>(w_gu);
  p.w_post = static_cast<const uint16_t*>(w_post);
  p.act = static_cast<uint16_t*>(act);
  p.I = I;
  p.eps = eps;
  p.mrows = B;
  p.sync2 = sync + OPROJ_SYNC_INTS;
  p.err = err;
  p.o_delay = o_delay_ns > 0 ? o_delay_ns / 10 : 0;  // s_memrealtime runs at 100 MHz
  p.gu_delay = gu_delay_ns > 0 ? gu_delay_ns / 10 : 0;
  const int nattn = grid_waves / 4;
  const int nog = (H + O_COLS - 1) / O_COLS;
  const int gcols = B == 1 ? gu_cols<1>() : gu_cols<2>();
  const int nug = (I + gcols - 1) / gcols;
  const dim3 grid(nattn + nog + nug), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 1)
    hipLaunchKernelGGL(attn_o_gu_kernel<1>, grid, block, 0, s, a, p, nattn, nog);
  else
    hipLaunchKernelGGL(attn_o_gu_kernel<2>, grid, block, 0, s, a, p, nattn, nog);
  return KO_LAUNCH_STATUS();
}

}  // extern "C"
