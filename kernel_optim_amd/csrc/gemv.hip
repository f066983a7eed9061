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
#include "gemv_launch.h"

using namespace ko;

namespace {

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
// index) pairs with the lowest index on ties. Optionally pos[m] += 1 (the decode
// step's position advance, engine.py:292) and h[m] = emb[ids[m]] (the next step's
// embedding gather, gemv.py:201-211, so the next step needs no gather launch),
// and the rest of the decode step's tail (StepTail): the RoPE rows of the new
// position for the next step's attention, and the id written straight into a
// ring in pinned host memory (no device-to-host copy per token), or -2 there
// when the step's attention + o projection launches report a failed wait.
constexpr int FT = 1024;

struct StepTail {
  // rope[m] = (cos[p], sin[p]) at the advanced position p = clamp(pos[m], 0, max_pos - 1)
  const uint16_t* cosb;
  const uint16_t* sinb;
  int max_pos, d;
  uint16_t* rope;
  // ring[slot * ring_ld + m] = ids[m] with slot = ring_ctr[m], then
  // ring_ctr[m] = (slot + 1) % ring_rows
  long long* ring;
  int ring_rows, ring_ld;
  int* ring_ctr;
  // with the ring: nonzero *err (a failed wait of ko_decode_attn_qkv_oproj,
  // left set until the host clears it) stores -2 in place of the id
  const int* err;
};
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
    int V, StepTail tail) {
  __shared__ float2 s_best[FT / 64];
  __shared__ int s_id, s_pos;
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float2* pr = part + (long long)m * nparts;
  int failed = 0;  // thread 0, issued ahead of the partials
  if (t == 0 && tail.ring && tail.err)
    failed = __hip_atomic_load(tail.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    int p = 0;
    if (pos) {
      p = pos[m] + 1;
      pos[m] = p;
    }
    s_id = i;
    s_pos = p;
    if (tail.ring) {
      // rows of the ring live in pinned host memory: a system-scope store
      const int c = tail.ring_ctr[m];
      const int slot = c >= 0 && c < tail.ring_rows ? c : 0;
      __hip_atomic_store(tail.ring + (long long)slot * tail.ring_ld + m,
                         failed ? -2LL : (long long)i, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
      tail.ring_ctr[m] = slot + 1 < tail.ring_rows ? slot + 1 : 0;
    }
  }
  if (emb || tail.rope) __syncthreads();
  if (emb) {
    const long long tok = s_id;
    if (tok >= 0 && tok < V) {
      for (int c = t; c < (H >> 3); c += FT)
        *reinterpret_cast<uint4*>(h + (long long)m * H + 8 * c) = ldg16(emb + tok * H + 8 * c);
    }
  }
  if (tail.rope) {
    const int p = min(max(s_pos, 0), tail.max_pos - 1);
    const int chunks = tail.d >> 3;
    for (int c = t; c < 2 * chunks; c += FT) {
      const uint16_t* src = (c < chunks ? tail.cosb : tail.sinb) + (long long)p * tail.d +
                            8 * (c < chunks ? c : c - chunks);
      *reinterpret_cast<uint4*>(tail.rope + (long long)m * 2 * tail.d + 8 * c) = ldg16(src);
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


bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

long long parts_for(int N, int layout, int rows, int waves) {
  if (layout == 0) return (N + rows - 1) / rows;
  if (layout == 2) return mfma_grid(N, rows);
  if (layout != 1 || waves < 1) return 0;  // layouts 3 and 4 have no ARGMAX partials
  const long long units = (N + rows - 1) / rows;
  return ((units + waves - 1) / waves) * waves;
}

int gemv_impl(const void* x, const void* w, void* y, const void* nw, const float* ss, void* h,
              float* ss_out, long long* ids, int* pos_inc, const void* next_emb, void* next_h,
              float* part, long long part_len, int M, int N, int K, int epi, int norm,
              int accumulate, int layout, int rows, int waves, float eps, const StepTail& tail,
              hipStream_t s) {
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
    if (waves != 0 && waves != 2) return KO_ENOTSUP;  // row tiles: 0 (one) or 2
    if (!mfma_supported(K, epi, waves == 2 ? 2 : 1)) return KO_ENOTSUP;
  } else if (layout == 3) {
    if (epi == EPI_ARGMAX || !ks_steps(K, rows)) return KO_ENOTSUP;
    if (norm && rows > 1 && !ss) return KO_ENOTSUP;
    if (norm && ks_steps(K, rows) != 20) return KO_ENOTSUP;
    if (rows > 1 && (!part || !al16(part) || part_len < ks_scratch(N, rows))) return KO_ERANGE;
  } else if (layout == 4) {
    if (norm || epi == EPI_ARGMAX || epi == EPI_SWIGLU || rows != SK_W || !sk_steps(K))
      return KO_ENOTSUP;
    if (waves != 0 && waves != 2 && waves != 4) return KO_ENOTSUP;  // row tiles: 0 (one), 2, 4
    if (!part || !al16(part) || part_len < sk_scratch(N, waves ? waves : 1)) return KO_ERANGE;
  } else {
    return KO_EINVAL;
  }
  const int mstep = mstep_for(layout, waves);
  const long long nparts = parts_for(N, layout, rows, waves);
  if (epi == EPI_ARGMAX) {
    if (!ids || !part) return KO_EINVAL;
    if (part_len < 2LL * mstep * nparts) return KO_ERANGE;
    if ((next_emb == nullptr) != (next_h == nullptr)) return KO_EINVAL;
    if (next_emb && (!al16(next_emb) || !al16(next_h))) return KO_EINVAL;
  }
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
      st = launch_layout0(a, epi, norm != 0, rows, s);
    else if (layout == 1)
      st = launch_layout1(a, epi, norm != 0, rows, waves, s);
    else if (layout == 2)
      st = launch_layout2(a, epi, norm != 0, rows, waves == 2 && mr > 16 ? 2 : 1, s);
    else if (layout == 3)
      st = launch_layout3(a, epi, norm != 0, rows, reinterpret_cast<int*>(part),
                          part + ((N + 15) / 16 + 63) / 64 * 64, s);
    else
      st = launch_layout4(a, epi, sk_tiles(waves, mr), reinterpret_cast<int*>(part),
                          part + ((N + 15) / 16 + 63) / 64 * 64, s);
    if (st) return st;
    if (epi == EPI_ARGMAX) {
      StepTail tl = tail;
      if (tl.rope) tl.rope += (long long)m0 * 2 * tl.d;
      if (tl.ring) {
        tl.ring += m0;
        tl.ring_ctr += m0;
      }
      hipLaunchKernelGGL(argmax_finalize_kernel, dim3(mr), dim3(FT), 0, s, a.part, a.nparts,
                         ids + m0, pos_inc ? pos_inc + m0 : nullptr,
                         static_cast<const uint16_t*>(next_emb),
                         next_h ? static_cast<uint16_t*>(next_h) + (long long)m0 * K : nullptr, K,
                         N, tl);
      st = KO_LAUNCH_STATUS();
      if (st) return st;
    }
  }
  return KO_OK;
}

}  // namespace

extern "C" {

int ko_gemv(const void* x, const void* w, void* y, const void* nw, const float* ss, void* h,
            float* ss_out, long long* ids, int* pos_inc, const void* next_emb, void* next_h,
            float* part, long long part_len, int M, int N, int K, int epi, int norm,
            int accumulate, int layout, int rows, int waves, float eps, void* stream) {
  const StepTail none = {};
  return gemv_impl(x, w, y, nw, ss, h, ss_out, ids, pos_inc, next_emb, next_h, part, part_len, M,
                   N, K, epi, norm, accumulate, layout, rows, waves, eps, none,
                   static_cast<hipStream_t>(stream));
}

int ko_lm_head_argmax(const void* x, const void* w, const void* nw, const float* ss, void* logits,
                      long long* ids, int* pos, const void* next_emb, void* next_h,
                      const void* cos, const void* sin, int max_pos, int head_dim, void* rope,
                      long long* ring, int ring_rows, int* ring_ctr, const int* err,
                      float* part, long long part_len, int M, int N, int K, int layout, int rows,
                      int waves, float eps, void* stream) {
  StepTail tail = {};
  if (rope) {
    if (!pos || !cos || !sin || max_pos < 1 || head_dim < 8 || (head_dim & 7)) return KO_EINVAL;
    if (!al16(cos) || !al16(sin) || !al16(rope)) return KO_EINVAL;
    tail.cosb = static_cast<const uint16_t*>(cos);
    tail.sinb = static_cast<const uint16_t*>(sin);
    tail.max_pos = max_pos;
    tail.d = head_dim;
    tail.rope = static_cast<uint16_t*>(rope);
  }
  if (ring) {
    if (!ring_ctr || ring_rows < 1) return KO_EINVAL;
    tail.ring = ring;
    tail.ring_rows = ring_rows;
    tail.ring_ld = M;
    tail.ring_ctr = ring_ctr;
    tail.err = err;
  }
  return gemv_impl(x, w, logits, nw, ss, nullptr, nullptr, ids, pos, next_emb, next_h, part,
                   part_len, M, N, K, EPI_ARGMAX, nw != nullptr, 0, layout, rows, waves, eps,
                   tail, static_cast<hipStream_t>(stream));
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
  if (N < 1 || rows < 1 || (layout == 1 && waves < 1) || layout < 0 || layout > 4) return -1;
  if (layout == 3) return rows > 1 ? ks_scratch(N, rows) : 0;
  if (layout == 4) return sk_scratch(N, waves == 2 || waves == 4 ? waves : 1);
  return 2LL * mstep_for(layout, waves) * parts_for(N, layout, rows, waves);
}

}  // extern "C"

