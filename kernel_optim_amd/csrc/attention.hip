// Split-K GQA decode attention for gfx950 (MI355X).
//
// Replaces engine/kernels/fused.py:138-234 (_decode_attn_kernel,
// _decode_combine_kernel, DecodeAttention.__call__). Semantics follow that
// code: T query tokens per sequence at positions kv_len-T .. kv_len-1, causal
// among themselves (query t sees keys < kv_len-T+t+1), softmax scale 1/sqrt(D),
// query head h reads KV head h/4, P rounded to bf16 before the PV product,
// fp32 partials (m, l, acc) merged by a log-sum-exp combine, rounded to bf16.
//
// Work decomposition (length-aware, graph-safe): a "unit" is (b, kv_head,
// c) covering keys [c*U, min((c+1)*U, kv_len_b)). Units are enumerated on the
// device from kv_len (read from device memory every launch), so sequences of
// different lengths get proportionally many units and the padded tail of the
// cache is never read. A fixed grid of wavefronts strides over the unit list.
//
// One wavefront per unit. Per 16-key step:
//   QK^T : 4 x v_mfma_f32_16x16x32_bf16. A = Q (16 rows = the 4 group heads
//          replicated 4x for T=1), B = K (16 key columns). Every lane ends with
//          the scores of one key for the 4 heads of its token.
//   softmax: online, with a wave-uniform running max per (token, head) that is
//          raised only when a score exceeds it by more than 2^8 (lazy
//          rescaling); exp2 with the log2(e) folded into the scale.
//   P    : rounded to bf16 and exchanged through 128*T bytes of LDS.
//   PV   : v_dot2c_f32_bf16 over key pairs; each lane owns 8 head-dim columns
//          of 4 keys per step, so V is read with fully coalesced 1 KiB loads.
//
// Variants (template flags):
//   QKV   : the unit builds its q itself from the bf16 QKV projection (per-head
//           RMSNorm + RoPE, engine/kernels/fused.py:71-87), and the unit that
//           owns the new key position also norms/ropes k, appends k and v to
//           the cache and uses them from registers (the work of
//           qk_norm_rope, fused.py:54-96, folded in; decode T = 1).
//   FUSED : the last unit of each (b, kv_head) to finish (per-pair arrival
//           counter) merges the pair's partials and writes the bf16 output,
//           so no second launch is needed; it re-arms the counter for the
//           next launch.
#include <type_traits>

#include "gemv_core.h"

using namespace ko;

namespace {

constexpr int D = 128;          // head dim
constexpr int G = 4;            // query heads per KV head
constexpr int WAVES = 4;        // wavefronts per workgroup
constexpr float TAU = 8.0f;     // lazy-rescale threshold, log2 units
constexpr float NEG_BIG = -1.0e30f;

constexpr int SPIN_MAX = 1 << 21;
// sync[] layout of ko_decode_attn_qkv_oproj: [0] merged-pair count, [1] projection
// workgroups past their wait, then OPROJ_FLAGS done-flag copies 128 bytes apart.
// Each flag line also carries, one int further on, the count of projection
// workgroups of that flag's group that have finished (re-arm bookkeeping).
constexpr int OPROJ_FLAG0 = 32, OPROJ_FLAG_STRIDE = 32, OPROJ_FLAGS = 32;
constexpr int OPROJ_SYNC_INTS = OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * OPROJ_FLAGS;

struct AttnArgs {
  const uint16_t* q;     // [B*T, nq*D] (unless QKV)
  const uint16_t* qkv;   // [B, (nq+2nkv)*D] (QKV)
  const uint16_t* qw;    // [D] q_norm gain (QKV)
  const uint16_t* kw;    // [D] k_norm gain (QKV)
  const uint16_t* cosb;  // [rows, D] (QKV)
  const uint16_t* sinb;
  float eps;
  int max_pos;           // rows of the RoPE tables (QKV)
  uint16_t* kc;
  uint16_t* vc;
  const int* lens;
  int len_off, cap;
  long long cb, ch;
  int B, nkv, unit, max_units;
  float scale_log2;
  float* o_part;
  float* ml;
  int* counters;         // [B*nkv] (FUSED)
  uint16_t* out;         // [B*T, nq*D] (FUSED)
  int* pairs_done;       // attention + o projection launch: merged (b, kv_head) pairs
};

__device__ __forceinline__ int nunits(int len, int unit) {
  return len > 0 ? (len + unit - 1) / unit : 0;
}
__device__ __forceinline__ int seq_len(const int* lens, int b, int off, int cap) {
  int l = lens[b] + off;
  return l < cap ? l : cap;
}

// Number of (b, c) pairs over the whole batch.
__device__ int count_pairs(const int* lens, int off, int cap, int B, int unit) {
  const int lane = lane_id();
  int tot = 0;
  for (int b0 = 0; b0 < B; b0 += 64) {
    const int b = b0 + lane;
    const int n = b < B ? nunits(seq_len(lens, b, off, cap), unit) : 0;
    tot += readlane(wave_incl_scan(n), 63);
  }
  return tot;
}

// Flattened pair index p -> (b, c).
__device__ void locate_pair(int p, const int* lens, int off, int cap, int B, int unit,
                            int& b_out, int& c_out) {
  const int lane = lane_id();
  int carry = 0;
  for (int b0 = 0; b0 < B; b0 += 64) {
    const int b = b0 + lane;
    const int n = b < B ? nunits(seq_len(lens, b, off, cap), unit) : 0;
    const int incl = wave_incl_scan(n) + carry;
    const int tot = readlane(incl, 63);
    if (p < tot) {
      const unsigned long long below = __ballot(incl <= p);
      const int k = uniform(__popcll(below));
      b_out = b0 + k;
      c_out = p - readlane(incl - n, k);
      return;
    }
    carry = tot;
  }
  b_out = -1;
  c_out = 0;
}

// Per-head RMSNorm + RoPE of one head held in the MFMA operand layout: lane
// (r, g) holds head-dim elements 32i+8g .. +7 for i = 0..3, and the four lanes
// r, r+16, r+32, r+48 together hold the whole head. The rotate_half partner of
// element d (d +- 64) is i +- 2 in the same lane.
__device__ __forceinline__ void norm_rope_head(const uint4 (&x)[4], const uint4 (&w)[4],
                                               const uint4 (&c)[4], const uint4 (&s)[4],
                                               float eps, uint4 (&y)[4]) {
  float xf[4][8], wf[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t xv[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
    const uint32_t wv[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xf[i][2 * e] = bf16lo(xv[e]);
      xf[i][2 * e + 1] = bf16hi(xv[e]);
      wf[i][2 * e] = bf16lo(wv[e]);
      wf[i][2 * e + 1] = bf16hi(wv[e]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += xf[i][e] * xf[i][e];
  ss = sum_xor32(sum_xor16(ss));
  const float rstd = rsqrtf(ss / (float)D + eps);
  float xn[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) xn[i][e] = round_bf16(wf[i][e] * round_bf16(xf[i][e] * rstd));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t cv[4] = {c[i].x, c[i].y, c[i].z, c[i].w};
    const uint32_t sv[4] = {s[i].x, s[i].y, s[i].z, s[i].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float yy[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = 2 * e + h;
        const float rot = i < 2 ? -xn[i + 2][k] : xn[i - 2][k];
        const float cf = h ? bf16hi(cv[e]) : bf16lo(cv[e]);
        const float sf = h ? bf16hi(sv[e]) : bf16lo(sv[e]);
        yy[h] = round_bf16(xn[i][k] * cf) + round_bf16(rot * sf);
      }
      o[e] = pack_bf16x2(yy[0], yy[1]);
    }
    y[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Log-sum-exp merge of the unit partials of row R (one wavefront; lane owns
// head-dim elements 2l, 2l+1), normalise, round to bf16. The row's unit count
// is n = nunits(kv_len); the loads of (m, l) and of the accumulators are issued
// for up to NB slots at a time (every slot in bounds) together with the length,
// so a merge of up to NB slots costs one memory round trip; slots >= n are
// masked. Pass n >= 0 when it is known already (then len_ptr is unused).
// 8-byte load; COHERENT reads at device scope (a relaxed agent-scope atomic
// load: global_load ... sc1), for data another workgroup of the same launch
// wrote with store_coherent.
template <bool COHERENT>
__device__ __forceinline__ float2 load2(const float* p) {
  if constexpr (COHERENT) {
    const unsigned long long u = __hip_atomic_load(
        reinterpret_cast<unsigned long long*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
        __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_bit_cast(float2, u);
  } else {
    return *reinterpret_cast<const float2*>(p);
  }
}
// 8-byte relaxed agent-scope atomic store (global_store ... sc1): written
// through to the device coherence point, so a device-scope load elsewhere sees
// it once this wave's s_waitcnt vmcnt(0) has passed.
__device__ __forceinline__ void store_coherent(float* p, float2 v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p),
                     __builtin_bit_cast(unsigned long long, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

template <int NB, bool COHERENT = false, bool COH_OUT = false>
__device__ void combine_row(const float* __restrict__ o_part, const float* __restrict__ ml,
                            long long R, int n, const int* len_ptr, int len_off, int cap,
                            int unit, int max_units, uint16_t* __restrict__ out) {
  const int lane = lane_id();
  const float* mlr = ml + 2 * R * max_units;
  const float* op = o_part + R * max_units * D + 2 * lane;
  float L = 0.f, o0 = 0.f, o1 = 0.f, M = NEG_BIG;
  static_assert(NB <= 64, "one (m, l) slot per lane");
  for (int c0 = 0; c0 < max_units; c0 += NB) {
    const int cn = min(NB, max_units - c0);
    const float2 mlc = lane < cn ? load2<COHERENT>(mlr + 2 * (c0 + lane)) : make_float2(NEG_BIG, 0.f);
    float2 a[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (j < cn) a[j] = load2<COHERENT>(op + (long long)(c0 + j) * D);
    if (n < 0) {
      int l = *len_ptr + len_off;
      n = nunits(l < cap ? l : cap, unit);
    }
    const int valid = min(cn, max(0, n - c0));
    if (valid <= 0) break;
    const float mc = lane < valid ? mlc.x : NEG_BIG;
    const float Mn = fmaxf(M, wave_max(mc));
    const float scale_old = __builtin_amdgcn_exp2f(M - Mn);
    const float w = lane < valid ? __builtin_amdgcn_exp2f(mc - Mn) : 0.f;
    L = L * scale_old + wave_sum(lane < valid ? w * mlc.y : 0.f);  // stale slots may hold NaN
    o0 *= scale_old;
    o1 *= scale_old;
    M = Mn;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < valid) {
        const float wj = readlane(w, j);
        o0 += wj * a[j].x;
        o1 += wj * a[j].y;
      }
    }
  }
  const float r0 = L > 0.f ? o0 / L : 0.f;
  const float r1 = L > 0.f ? o1 / L : 0.f;
  uint32_t* dst = reinterpret_cast<uint32_t*>(out + R * D) + lane;
  if constexpr (COH_OUT)  // read later in the same launch: a device-coherent store
    __hip_atomic_store(dst, pack_bf16x2(r0, r1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *dst = pack_bf16x2(r0, r1);
}

template <int T, bool QKV, bool FUSED>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  static_assert(!QKV || T == 1, "the QKV prologue serves one decode token per sequence");
  __shared__ __align__(16) uint16_t lds_p[WAVES][T][G][16];

  const int wpb = blockDim.x >> 6;   // wavefronts per workgroup (1..WAVES)
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;   // key slot of the QK lanes / column chunk of the PV lanes
  const int g = lane >> 4;   // MFMA k-group / PV key row
  const int nkv = a.nkv, nq = nkv * G, unit = a.unit, max_units = a.max_units;
  const int W = gridDim.x * wpb;
  uint16_t* myp = &lds_p[wave][0][0][0];

  // Up to 64 sequences: one load of the lengths and one prefix scan serve
  // every unit this wave processes (lane b holds sequence b's unit count and
  // inclusive prefix).
  const bool small_b = a.B <= 64;
  int my_n = 0, my_incl = 0, total;
  if (small_b) {
    my_n = lane < a.B ? nunits(seq_len(a.lens, lane, a.len_off, a.cap), unit) : 0;
    my_incl = wave_incl_scan(my_n);
    total = readlane(my_incl, 63) * nkv;
  } else {
    total = count_pairs(a.lens, a.len_off, a.cap, a.B, unit) * nkv;
  }

  for (int u = blockIdx.x * wpb + wave; u < total; u += W) {
    const int pidx = u / nkv;
    const int kvh = u - pidx * nkv;
    int b, c, kv_len;
    if (small_b) {
      b = uniform(__popcll(__ballot(my_incl <= pidx)));
      c = pidx - readlane(my_incl - my_n, b);
      kv_len = uniform(seq_len(a.lens, b, a.len_off, a.cap));
    } else {
      locate_pair(pidx, a.lens, a.len_off, a.cap, a.B, unit, b, c);
      b = uniform(b);
      c = uniform(c);
      if (b < 0) break;  // unreachable while lens[] is unchanged during the launch
      kv_len = uniform(seq_len(a.lens, b, a.len_off, a.cap));
    }
    const int k0 = c * unit;
    const int k1 = min(k0 + unit, kv_len);
    const uint16_t* kb = a.kc + (long long)b * a.cb + (long long)kvh * a.ch;
    const uint16_t* vb = a.vc + (long long)b * a.cb + (long long)kvh * a.ch;

    // ---- K/V loads of a 16-key step (clamped to the unit's last key) ----
    auto load_k = [&](int kk, uint4* kr) {
      const int key = min(kk + r, k1 - 1);
      const uint16_t* p = kb + (long long)key * D + 8 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[i] = ldg16_stream(p + 32 * i);
    };
    auto load_v = [&](int kk, uint4* vr) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int key = min(kk + g + 4 * s, k1 - 1);
        vr[s] = ldg16_stream(vb + (long long)key * D + 8 * r);
      }
    };
    uint4 ka[4], va[4], kb2[4], vb2[4];
    load_k(k0, ka);
    load_v(k0, va);

    // ---- Q as the MFMA A operand: row r -> (token (r/4)%T, head r%4); lane
    // group g supplies head-dim elements 32i+8g .. 32i+8g+7 for MFMA i ----
    bf16x8 qa[4];
    const int pnew = kv_len - 1;                     // QKV: position of the new key
    const bool has_new = QKV && k0 <= pnew && pnew < k1;
    uint4 knew[4], vnew;
    if constexpr (QKV) {
      const int nqkv = (nq + 2 * nkv) * D;
      const int pt = min(max(pnew, 0), a.max_pos - 1);
      const uint16_t* src = a.qkv + (long long)b * nqkv;
      uint4 xq[4], wq[4], cs[4], sn[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * i + 8 * g;
        xq[i] = ldg16(src + (kvh * G + (r & 3)) * D + d);
        wq[i] = ldg16(a.qw + d);
        cs[i] = ldg16(a.cosb + (long long)pt * D + d);
        sn[i] = ldg16(a.sinb + (long long)pt * D + d);
      }
      uint4 qn[4];
      norm_rope_head(xq, wq, cs, sn, a.eps, qn);
#pragma unroll
      for (int i = 0; i < 4; ++i) qa[i] = __builtin_bit_cast(bf16x8, qn[i]);
      if (has_new) {
        uint4 xk[4], wk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * i + 8 * g;
          xk[i] = ldg16(src + (nq + kvh) * D + d);
          wk[i] = ldg16(a.kw + d);
        }
        norm_rope_head(xk, wk, cs, sn, a.eps, knew);
        vnew = ldg16(src + (nq + nkv + kvh) * D + 8 * r);
        // KV append at slot pnew (fused.py:88-96): k by the r == 0 lanes,
        // v by the g == 0 lanes.
        uint16_t* kdst = a.kc + (long long)b * a.cb + (long long)kvh * a.ch + (long long)pnew * D;
        uint16_t* vdst = a.vc + (long long)b * a.cb + (long long)kvh * a.ch + (long long)pnew * D;
        if (r == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(kdst + 32 * i + 8 * g) = knew[i];
        }
        if (g == 0) *reinterpret_cast<uint4*>(vdst + 8 * r) = vnew;
      }
    } else {
      const int trow = (r >> 2) % T;
      const uint16_t* qrow =
          a.q + ((long long)(b * T + trow) * nq + kvh * G + (r & 3)) * D + 8 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) qa[i] = __builtin_bit_cast(bf16x8, ldg16(qrow + 32 * i));
    }

    const int tq = g % T;                           // token of this lane's score rows
    const int lim = min(k1, kv_len - T + tq + 1);   // exclusive causal key limit

    float mu[T][G];
    float acc[T][G][8];
    float lsum[G];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int j = 0; j < G; ++j) {
        mu[t][j] = NEG_BIG;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[t][j][e] = 0.f;
      }
#pragma unroll
    for (int j = 0; j < G; ++j) lsum[j] = 0.f;

    auto step = [&](int kk, const uint4* kr_in, const uint4* vr_in) {
      uint4 kr[4], vr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kr[i] = kr_in[i];
        vr[i] = vr_in[i];
      }
      if (has_new && kk <= pnew && pnew < kk + 16) {  // the new key: use registers
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (r == pnew - kk) kr[i] = knew[i];
          if (kk + g + 4 * i == pnew) vr[i] = vnew;
        }
      }
      f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i], __builtin_bit_cast(bf16x8, kr[i]),
                                                     sc, 0, 0, 0);
      const bool valid = (kk + r) < lim;
      float s[G], mrow[G];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        s[j] = valid ? sc[j] * a.scale_log2 : -INFINITY;
        float m = mu[0][j];
#pragma unroll
        for (int t = 1; t < T; ++t) m = (tq == t) ? mu[t][j] : m;
        mrow[j] = m;
      }
      bool need = false;
#pragma unroll
      for (int j = 0; j < G; ++j) need |= s[j] > mrow[j] + TAU;
      if (__ballot(need)) {
        float rm[G];
#pragma unroll
        for (int j = 0; j < G; ++j) rm[j] = row_max16(s[j]);
        float alpha[T][G];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int j = 0; j < G; ++j) {
            const float mn = fmaxf(mu[t][j], readlane(rm[j], 16 * t));
            alpha[t][j] = __builtin_amdgcn_exp2f(mu[t][j] - mn);
            mu[t][j] = mn;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[t][j][e] *= alpha[t][j];
          }
#pragma unroll
        for (int j = 0; j < G; ++j) {
          float al = alpha[0][j], m = mu[0][j];
#pragma unroll
          for (int t = 1; t < T; ++t) {
            al = (tq == t) ? alpha[t][j] : al;
            m = (tq == t) ? mu[t][j] : m;
          }
          lsum[j] *= al;
          mrow[j] = m;
        }
      }
      float pf[G];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        pf[j] = __builtin_amdgcn_exp2f(s[j] - mrow[j]);
        lsum[j] += pf[j];
      }
      // P (bf16) -> LDS, key order permuted so that a PV lane's 4 keys
      // (g, g+4, g+8, g+12) are contiguous.
      const int pos = (r & 3) * 4 + (r >> 2);
      if (T == 1) {
        const float v = g == 0 ? pf[0] : g == 1 ? pf[1] : g == 2 ? pf[2] : pf[3];
        myp[g * 16 + pos] = f32_to_bf16(v);
      } else if (g < T) {
#pragma unroll
        for (int j = 0; j < G; ++j) myp[(g * G + j) * 16 + pos] = f32_to_bf16(pf[j]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      uint2 pw[T][G];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int j = 0; j < G; ++j)
          pw[t][j] = *reinterpret_cast<const uint2*>(myp + (t * G + j) * 16 + 4 * g);
#pragma unroll
      for (int sp = 0; sp < 2; ++sp) {
        const uint32_t xs[4] = {vr[2 * sp].x, vr[2 * sp].y, vr[2 * sp].z, vr[2 * sp].w};
        const uint32_t ys[4] = {vr[2 * sp + 1].x, vr[2 * sp + 1].y, vr[2 * sp + 1].z,
                                vr[2 * sp + 1].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = (xs[e] & 0xffffu) | (ys[e] << 16);
          const uint32_t hi = (xs[e] >> 16) | (ys[e] & 0xffff0000u);
#pragma unroll
          for (int t = 0; t < T; ++t)
#pragma unroll
            for (int j = 0; j < G; ++j) {
              const uint32_t pword = sp ? pw[t][j].y : pw[t][j].x;
              acc[t][j][2 * e] = dot2_bf16(pword, lo, acc[t][j][2 * e]);
              acc[t][j][2 * e + 1] = dot2_bf16(pword, hi, acc[t][j][2 * e + 1]);
            }
        }
      }
      // The next step overwrites this wave's P slot; LDS ops of one wave
      // execute in order, so the reads above complete first.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
    };

    // Two-deep software pipeline over 16-key steps.
    for (int kk = k0; kk < k1; kk += 32) {
      load_k(kk + 16, kb2);
      load_v(kk + 16, vb2);
      step(kk, ka, va);
      if (kk + 16 >= k1) break;
      load_k(kk + 32, ka);
      load_v(kk + 32, va);
      step(kk + 16, kb2, vb2);
    }

    // ---- unit epilogue: reduce and write the fp32 partials ----
    float lrow[G];
#pragma unroll
    for (int j = 0; j < G; ++j) lrow[j] = row_sum16(lsum[j]);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int j = 0; j < G; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[t][j][e] = sum_xor32(sum_xor16(acc[t][j][e]));
        }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const long long R = (long long)(b * T + t) * nq + kvh * G + g;
      float* dst = a.o_part + (R * max_units + c) * D + 8 * r;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        if (g == j) {
          reinterpret_cast<float4*>(dst)[0] =
              make_float4(acc[t][j][0], acc[t][j][1], acc[t][j][2], acc[t][j][3]);
          reinterpret_cast<float4*>(dst)[1] =
              make_float4(acc[t][j][4], acc[t][j][5], acc[t][j][6], acc[t][j][7]);
        }
      }
    }
    if (g < T && r < G) {
      float m = mu[0][0], l = lrow[0];
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int j = 0; j < G; ++j) {
          m = (g == t && r == j) ? mu[t][j] : m;
          l = (r == j) ? lrow[j] : l;
        }
      const long long R = (long long)(b * T + g) * nq + kvh * G + r;
      reinterpret_cast<float2*>(a.ml)[R * max_units + c] = make_float2(m, l);
    }

    if constexpr (FUSED) {
      // Publish this unit's partials, count its arrival; the last arrival of
      // the (b, kv_head) pair merges the pair's partials.
      __threadfence();
      int prev = 0;
      int* ctr = a.counters + (long long)b * nkv + kvh;
      if (lane == 0) prev = atomicAdd(ctr, 1);
      prev = readlane(prev, 0);
      const int n = nunits(kv_len, unit);
      if (prev == n - 1) {
        __threadfence();
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int j = 0; j < G; ++j)
            combine_row<32>(a.o_part, a.ml, (long long)(b * T + t) * nq + kvh * G + j, n, nullptr, 0,
                        a.cap, unit, max_units, a.out);
        if (lane == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// RMSNorm + RoPE of one head held two elements per lane (lane l: elements 2l,
// 2l+1), the cast chain of fused.py:71-87: xn = bf16(w * bf16(x * rstd)),
// y = bf16(bf16(xn * cos) + bf16(rotate_half(xn) * sin)). rotate_half's partner
// of element d (d +- 64) sits 32 lanes away. Returns y packed as 2 bf16. Call
// with all 64 lanes active.
__device__ __forceinline__ uint32_t norm_rope2(uint32_t x, uint32_t w, uint32_t cw, uint32_t sw,
                                               float eps) {
  const float x0 = bf16lo(x), x1 = bf16hi(x);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = rsqrtf(ss / (float)D + eps);
  const float n0 = round_bf16(bf16lo(w) * round_bf16(x0 * rstd));
  const float n1 = round_bf16(bf16hi(w) * round_bf16(x1 * rstd));
  const uint32_t nb = pack_bf16x2(n0, n1);  // exact: n0, n1 are bf16 values
  const auto sw32 = __builtin_amdgcn_permlane32_swap(nb, nb, false, false);
  const bool lo_half = lane_id() < 32;
  const uint32_t pb = lo_half ? (uint32_t)sw32[1] : (uint32_t)sw32[0];
  const float r0 = lo_half ? -bf16lo(pb) : bf16lo(pb);
  const float r1 = lo_half ? -bf16hi(pb) : bf16hi(pb);
  const float y0 = round_bf16(n0 * bf16lo(cw)) + round_bf16(r0 * bf16lo(sw));
  const float y1 = round_bf16(n1 * bf16hi(cw)) + round_bf16(r1 * bf16hi(sw));
  return pack_bf16x2(y0, y1);
}

// One decode token per sequence (T = 1) with WM wavefronts per workgroup. A
// unit of `unit` keys of one (b, kv_head) pair is split into WM contiguous
// sub-ranges of sub = unit / WM keys, one per wavefront; the wavefronts'
// partials are merged through LDS, so a unit stores a single fp32 (m, l, acc)
// slot and the combine reads few slots. Per unit:
//   - every global load is issued before any wait (K/V of the first 16-key
//     step, the q inputs, the new k/v inputs), so they cost one round trip;
//   - QKV: the workgroup norms and ropes its 4 q heads once, G / WM heads per
//     wavefront at two elements per lane, and wavefront 0 of the unit that
//     holds the new key position also the new k (and appends k and v to the
//     cache); the heads go through LDS into the MFMA operand layout;
//   - the 16-key step is the T = 1 case of attn_kernel's: every 16-lane row of
//     the QK^T result holds the same 16 scores (the A rows are the 4 heads
//     replicated), so the running max stays wave-uniform without cross-row
//     traffic.
// wg / nwg: this workgroup's index among the nwg attention workgroups.
// OPROJ (with FUSED): the merged outputs are stored device-coherently and each
// merge bumps a.pairs_done, for the o-projection workgroups of the same launch.
template <bool QKV, int WM, bool FUSED, bool OPROJ = false>
__device__ __forceinline__ void attn1_body(const AttnArgs& a, int wg, int nwg) {
  static_assert(!OPROJ || FUSED, "the o projection consumes the merged output");
  __shared__ int lds_prev;
  __shared__ __align__(16) uint16_t lds_p[WM][G * 16];
  __shared__ __align__(16) float lds_acc[WM][4][G][D];  // [wave][key group g][head][col]
  __shared__ float lds_ml[WM][G][2];
  __shared__ __align__(16) uint32_t lds_q[G][D / 2];     // QKV: roped q heads (bf16 pairs)
  __shared__ __align__(16) uint32_t lds_k[D / 2];        // QKV: roped new key

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int nkv = a.nkv, nq = nkv * G, unit = a.unit, max_units = a.max_units;
  const int sub = unit / WM;
  uint16_t* myp = lds_p[wave];

  const bool small_b = a.B <= 64;
  int my_n = 0, my_incl = 0, total;
  if (small_b) {
    my_n = lane < a.B ? nunits(seq_len(a.lens, lane, a.len_off, a.cap), unit) : 0;
    my_incl = wave_incl_scan(my_n);
    total = readlane(my_incl, 63) * nkv;
  } else {
    total = count_pairs(a.lens, a.len_off, a.cap, a.B, unit) * nkv;
  }

  for (int u = wg; u < total; u += nwg) {
    const int pidx = u / nkv;
    const int kvh = u - pidx * nkv;
    int b, c, kv_len;
    if (small_b) {
      b = uniform(__popcll(__ballot(my_incl <= pidx)));
      c = pidx - readlane(my_incl - my_n, b);
      kv_len = uniform(seq_len(a.lens, b, a.len_off, a.cap));
    } else {
      locate_pair(pidx, a.lens, a.len_off, a.cap, a.B, unit, b, c);
      b = uniform(b);
      c = uniform(c);
      if (b < 0) break;  // unreachable while lens[] is unchanged during the launch
      kv_len = uniform(seq_len(a.lens, b, a.len_off, a.cap));
    }
    const int ku1 = min((c + 1) * unit, kv_len);
    const int k0 = c * unit + wave * sub;
    const int k1 = min(k0 + sub, ku1);
    const bool active = k0 < k1;  // the last unit of a sequence may leave waves idle
    const int pnew = kv_len - 1;
    const bool new_unit = QKV && pnew < ku1;  // this unit holds the new key position
    const bool has_new = new_unit && active && k0 <= pnew && pnew < k1;

    float mu[G], lsum[G], acc[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      mu[j] = NEG_BIG;
      lsum[j] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    }

    const uint16_t* kb = a.kc + (long long)b * a.cb + (long long)kvh * a.ch;
    const uint16_t* vb = a.vc + (long long)b * a.cb + (long long)kvh * a.ch;
    auto load_k = [&](int kk, uint4* kr) {
      const int key = min(kk + r, k1 - 1);
      const uint16_t* p = kb + (long long)key * D + 8 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[i] = ldg16_stream(p + 32 * i);
    };
    auto load_v = [&](int kk, uint4* vr) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int key = min(kk + g + 4 * s4, k1 - 1);
        vr[s4] = ldg16_stream(vb + (long long)key * D + 8 * r);
      }
    };
    uint4 ka[4], va[4], kb2[4], vb2[4];
    if (active) {
      load_k(k0, ka);
      load_v(k0, va);
    }

    bf16x8 qa[4];
    uint4 knew[4], vnew;
    if constexpr (QKV) {
      // q heads normed by each wavefront (wavefronts past the 4th norm none)
      constexpr int NH = G / WM > 0 ? G / WM : 1;
      const bool has_q = wave < G;
      const int nqkv = (nq + 2 * nkv) * D;
      const int pt = min(max(pnew, 0), a.max_pos - 1);
      const uint16_t* src = a.qkv + (long long)b * nqkv;
      const bool do_k = new_unit && wave == (WM > G ? G : 0);  // the new key: an idle wavefront if any
      uint32_t xh[NH], xk = 0, kwv = 0, vv = 0;
#pragma unroll
      for (int n = 0; n < NH; ++n)
        xh[n] = has_q ? reinterpret_cast<const uint32_t*>(src + (kvh * G + wave + n * WM) * D)[lane] : 0u;
      const uint32_t qwv = reinterpret_cast<const uint32_t*>(a.qw)[lane];
      const uint32_t cwv = reinterpret_cast<const uint32_t*>(a.cosb + (long long)pt * D)[lane];
      const uint32_t swv = reinterpret_cast<const uint32_t*>(a.sinb + (long long)pt * D)[lane];
      if (do_k) {
        xk = reinterpret_cast<const uint32_t*>(src + (nq + kvh) * D)[lane];
        kwv = reinterpret_cast<const uint32_t*>(a.kw)[lane];
        vv = reinterpret_cast<const uint32_t*>(src + (nq + nkv + kvh) * D)[lane];
      }
      if (has_new) vnew = ldg16(src + (nq + nkv + kvh) * D + 8 * r);
      asm volatile("" ::: "memory");  // keep every load above ahead of the first wait
      if (has_q) {
#pragma unroll
        for (int n = 0; n < NH; ++n) lds_q[wave + n * WM][lane] = norm_rope2(xh[n], qwv, cwv, swv, a.eps);
      }
      if (do_k) {
        // the new key: to LDS for the wavefront that owns it, and the KV
        // append at slot pnew (fused.py:88-96)
        const uint32_t kn = norm_rope2(xk, kwv, cwv, swv, a.eps);
        lds_k[lane] = kn;
        const long long slot = (long long)b * a.cb + (long long)kvh * a.ch + (long long)pnew * D;
        reinterpret_cast<uint32_t*>(a.kc + slot)[lane] = kn;
        reinterpret_cast<uint32_t*>(a.vc + slot)[lane] = vv;
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; ++i)
        qa[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&lds_q[r & 3][16 * i + 4 * g]));
      if (has_new) {
#pragma unroll
        for (int i = 0; i < 4; ++i) knew[i] = *reinterpret_cast<const uint4*>(&lds_k[16 * i + 4 * g]);
      }
    } else {
      const uint16_t* qrow = a.q + ((long long)b * nq + kvh * G + (r & 3)) * D + 8 * g;
      uint4 qv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = ldg16(qrow + 32 * i);
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < 4; ++i) qa[i] = __builtin_bit_cast(bf16x8, qv[i]);
    }

    if (active) {
      // kr / vr are consumed by this step, so the new key is patched in place.
      // FIRST (the wavefront's first step, with acc = l = 0 and no running max
      // yet) sets the max from the step's scores instead of rescaling.
      auto step = [&](int kk, uint4 (&kr)[4], uint4 (&vr)[4], auto first_tag) {
        constexpr bool FIRST = decltype(first_tag)::value;
        if (QKV && has_new && kk <= pnew && pnew < kk + 16) {  // the new key: from registers
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (r == pnew - kk) kr[i] = knew[i];
            // keys past pnew were clamped onto its (not yet written) slot:
            // give them the new value too, so P = 0 never meets stale data
            if (kk + g + 4 * i >= pnew) vr[i] = vnew;
          }
        }
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i], __builtin_bit_cast(bf16x8, kr[i]),
                                                       sc, 0, 0, 0);
        const bool valid = (kk + r) < k1;
        float sv[G];
#pragma unroll
        for (int j = 0; j < G; ++j) sv[j] = valid ? sc[j] * a.scale_log2 : -INFINITY;
        if constexpr (FIRST) {
          // key kk is valid, so every row max is finite
#pragma unroll
          for (int j = 0; j < G; ++j) mu[j] = row_max16(sv[j]);
        } else {
          bool need = false;
#pragma unroll
          for (int j = 0; j < G; ++j) need |= sv[j] > mu[j] + TAU;
          if (__ballot(need)) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
              const float mn = fmaxf(mu[j], row_max16(sv[j]));
              const float al = __builtin_amdgcn_exp2f(mu[j] - mn);
              mu[j] = mn;
              lsum[j] *= al;
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[j][e] *= al;
            }
          }
        }
        float pf[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
          pf[j] = __builtin_amdgcn_exp2f(sv[j] - mu[j]);
          lsum[j] = FIRST ? pf[j] : lsum[j] + pf[j];
        }
        const int pos = (r & 3) * 4 + (r >> 2);
        const float pv = g == 0 ? pf[0] : g == 1 ? pf[1] : g == 2 ? pf[2] : pf[3];
        myp[g * 16 + pos] = f32_to_bf16(pv);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint2 pw[G];
#pragma unroll
        for (int j = 0; j < G; ++j) pw[j] = *reinterpret_cast<const uint2*>(myp + j * 16 + 4 * g);
#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
          const uint32_t xs4[4] = {vr[2 * sp].x, vr[2 * sp].y, vr[2 * sp].z, vr[2 * sp].w};
          const uint32_t ys4[4] = {vr[2 * sp + 1].x, vr[2 * sp + 1].y, vr[2 * sp + 1].z,
                                   vr[2 * sp + 1].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // (x.lo16, y.lo16) and (x.hi16, y.hi16) with one v_perm_b32 each
            const uint32_t lo = __builtin_amdgcn_perm(ys4[e], xs4[e], 0x05040100u);
            const uint32_t hi = __builtin_amdgcn_perm(ys4[e], xs4[e], 0x07060302u);
#pragma unroll
            for (int j = 0; j < G; ++j) {
              const uint32_t pword = sp ? pw[j].y : pw[j].x;
              const bool zero = FIRST && sp == 0;  // the first products start the sums
              acc[j][2 * e] = dot2_bf16(pword, lo, zero ? 0.f : acc[j][2 * e]);
              acc[j][2 * e + 1] = dot2_bf16(pword, hi, zero ? 0.f : acc[j][2 * e + 1]);
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
      };

      using First = std::integral_constant<bool, true>;
      using Next = std::integral_constant<bool, false>;
      if (k1 - k0 <= 16) {
        step(k0, ka, va, First{});  // one step: no prefetch
      } else {
        // Two-deep software pipeline over 16-key steps (loads clamp to k1 - 1,
        // so they are unconditional and the wait counts stay exact).
        load_k(k0 + 16, kb2);
        load_v(k0 + 16, vb2);
        step(k0, ka, va, First{});
        for (int kk = k0; kk < k1; kk += 32) {
          if (kk + 16 >= k1) break;
          load_k(kk + 32, ka);
          load_v(kk + 32, va);
          step(kk + 16, kb2, vb2, Next{});
          if (kk + 32 >= k1) break;
          load_k(kk + 48, kb2);
          load_v(kk + 48, vb2);
          step(kk + 32, ka, va, Next{});
        }
      }
    }

    // ---- merge the WM wavefront partials of the unit through LDS ----
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float* dst = &lds_acc[wave][g][j][8 * r];
      reinterpret_cast<float4*>(dst)[0] = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
      reinterpret_cast<float4*>(dst)[1] = make_float4(acc[j][4], acc[j][5], acc[j][6], acc[j][7]);
    }
    float lrow[G];
#pragma unroll
    for (int j = 0; j < G; ++j) lrow[j] = row_sum16(lsum[j]);  // the 4 rows hold equal sums
    if (lane < G) {
      float m = mu[0], l = lrow[0];
#pragma unroll
      for (int j = 1; j < G; ++j) {
        m = lane == j ? mu[j] : m;
        l = lane == j ? lrow[j] : l;
      }
      lds_ml[wave][lane][0] = m;
      lds_ml[wave][lane][1] = l;
    }
    __syncthreads();
    {
      constexpr int V = G * D / (64 * WM);  // outputs per thread
      const int o0 = threadIdx.x * V;
      const int j = o0 / D, d0 = o0 - j * D;
      float Mx = NEG_BIG;
#pragma unroll
      for (int w = 0; w < WM; ++w) Mx = fmaxf(Mx, lds_ml[w][j][0]);
      float L = 0.f, o[V];
#pragma unroll
      for (int v = 0; v < V; ++v) o[v] = 0.f;
#pragma unroll
      for (int w = 0; w < WM; ++w) {
        const float sw = __builtin_amdgcn_exp2f(lds_ml[w][j][0] - Mx);
        L += sw * lds_ml[w][j][1];
        float t[V];
#pragma unroll
        for (int v = 0; v < V; ++v) t[v] = 0.f;
#pragma unroll
        for (int kg = 0; kg < 4; ++kg)
#pragma unroll
          for (int v = 0; v < V; ++v) t[v] += lds_acc[w][kg][j][d0 + v];
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] += sw * t[v];
      }
      const long long R = (long long)b * nq + kvh * G + j;
      float* dst = a.o_part + (R * max_units + c) * D + d0;
      if constexpr (FUSED) {
        if constexpr (V == 1) {
          __hip_atomic_store(dst, o[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
#pragma unroll
          for (int v = 0; v < V; v += 2) store_coherent(dst + v, make_float2(o[v], o[v + 1]));
        }
        if (d0 == 0) store_coherent(a.ml + 2 * (R * max_units + c), make_float2(Mx, L));
      } else {
        if constexpr (V == 1) {
          dst[0] = o[0];
        } else {
#pragma unroll
          for (int v = 0; v < V; v += 2)
            reinterpret_cast<float2*>(dst + v)[0] = make_float2(o[v], o[v + 1]);
        }
        if (d0 == 0) reinterpret_cast<float2*>(a.ml)[R * max_units + c] = make_float2(Mx, L);
      }
    }
    if constexpr (FUSED) {
      // Count the unit's arrival once every thread's partial stores are
      // performed at device scope; the last unit of the (b, kv_head) pair to
      // arrive merges the pair's partials with device-scope loads and re-arms
      // the counter for the next launch. Nothing waits on another workgroup.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      int* ctr = a.counters + (long long)b * nkv + kvh;
      if (threadIdx.x == 0)
        lds_prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      const int n = nunits(kv_len, unit);
      if (lds_prev == n - 1) {
        for (int j = wave; j < G; j += WM)
          combine_row<32, true, OPROJ>(a.o_part, a.ml, (long long)b * nq + kvh * G + j, n,
                                       nullptr, 0, a.cap, unit, max_units, a.out);
        if constexpr (OPROJ) {
          __builtin_amdgcn_s_waitcnt(0);  // this wave's merged row is performed
          __syncthreads();
        }
        [[maybe_unused]] const int live_pairs = __popcll(__ballot(my_n > 0)) * nkv;
        if (threadIdx.x == 0) {
          __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if constexpr (OPROJ) {
            // the pair that completes the count raises the done flag (one copy
            // per 128-byte line, so its waiters do not queue on one address)
            const int live = live_pairs;
            const int prev =
                __hip_atomic_fetch_add(a.pairs_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (prev == live - 1) {
              for (int f = 0; f < OPROJ_FLAGS; ++f)
                __hip_atomic_store(a.pairs_done + OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * f, 1,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
          }
        }
      }
    }
    __syncthreads();  // the next unit reuses the LDS
  }
}

template <bool QKV, int WM, bool FUSED>
__global__ __launch_bounds__(64 * WM) void attn1_kernel(AttnArgs a) {
  attn1_body<QKV, WM, FUSED>(a, blockIdx.x, gridDim.x);
}

// Decode attention and the o projection in one launch (one query token, 1-2
// sequences, 4 wavefronts per unit). Workgroups [0, nattn) run the attention
// units with the fused combine; the rest each own 8 output columns of the o
// projection: they issue all their weight loads, wait until every (b, kv_head)
// pair has been merged (a device-coherent counter), then read the merged
// attention output with device-scope loads and finish as the RESID GEMV
// (h <- bf16(h + bf16(W_o attn))). The o-projection weights thus stream while
// the attention's latency chain runs instead of after it. Workgroups are
// dispatched in index order, so every attention workgroup is resident before
// any o-projection workgroup waits; the wait is also bounded (SPIN_MAX polls,
// then *err is set and the workgroup goes on). The last o-projection workgroup
// through the wait re-arms both counters for the next launch.


template <bool QKV, int M>
__global__ __launch_bounds__(256) void attn_oproj_kernel(AttnArgs a, GemvArgs g, int nattn,
                                                         int delay_ticks, int* err) {
  if ((int)blockIdx.x < nattn) {
    attn1_body<QKV, 4, true, true>(a, blockIdx.x, nattn);
    return;
  }
  const int wg = blockIdx.x - nattn;
  const int nog = gridDim.x - nattn;
  // Let the attention's first (latency-critical) loads go ahead of this
  // workgroup's weight stream: a short wait on the real-time counter.
  if (delay_ticks > 0) {
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < (unsigned long long)delay_ticks) __builtin_amdgcn_s_sleep(4);
  }
  const int grp = wg % OPROJ_FLAGS;
  int* flag = a.pairs_done + OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * grp;
  auto wait_x = [&] {
    if (threadIdx.x == 0) {
      int it = 0;
      while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
        __builtin_amdgcn_s_sleep(8);
        if (++it >= SPIN_MAX) {
          __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
    }
    __syncthreads();
  };
  gemv_row_body<M, 8, false, EPI_RESID, 2, true>(g, wg, wait_x);
  // Re-arm for the next launch, off the critical path: the last workgroup of a
  // flag group clears that flag and counts the group; the last group clears the
  // pair count and the group count.
  if (threadIdx.x == 0) {
    const int in_grp = (nog - grp + OPROJ_FLAGS - 1) / OPROJ_FLAGS;  // workgroups of group grp
    if (__hip_atomic_fetch_add(flag + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        in_grp - 1) {
      __hip_atomic_store(flag, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(flag + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int groups = nog < OPROJ_FLAGS ? nog : OPROJ_FLAGS;
      if (__hip_atomic_fetch_add(a.pairs_done + 1, 1, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) == groups - 1) {
        __hip_atomic_store(a.pairs_done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.pairs_done + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Second pass when no counters are given: one wavefront per output row.
__global__ __launch_bounds__(256) void attn_combine_kernel(
    const float* __restrict__ o_part, const float* __restrict__ ml,
    const int* __restrict__ lens, int len_off, int cap, int T, int nq, int rows, int unit,
    int max_units, uint16_t* __restrict__ out) {
  const int R = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (R >= rows) return;
  const int b = R / (T * nq);
  combine_row<64>(o_part, ml, R, -1, lens + b, len_off, cap, unit, max_units, out);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(const void* kc, const void* vc, const int* lens, int cap, long long cb,
                 long long ch, int B, int T, int nkv, int head_dim, int unit, int max_units,
                 const float* o_part, const float* ml) {
  if (!kc || !vc || !lens || !o_part || !ml) return KO_EINVAL;
  if (head_dim != D) return KO_ENOTSUP;
  if (T < 1 || T > 4) return KO_ENOTSUP;
  if (B < 1 || nkv < 1 || cap < 1) return KO_EINVAL;
  if (unit < 16 || (unit & 15)) return KO_EINVAL;
  if ((long long)max_units * unit < cap) return KO_ERANGE;
  if (!aligned16(kc) || !aligned16(vc) || !aligned16(o_part)) return KO_EINVAL;
  if ((cb & 7) || (ch & 7) || cb < 0 || ch < 0) return KO_EINVAL;
  return KO_OK;
}

template <int T, bool QKV, bool FUSED>
int launch(const AttnArgs& a, int grid_waves, hipStream_t s) {
  // Small grids run one wavefront per workgroup so they spread over more CUs.
  const int wpb = grid_waves <= 1024 ? 1 : WAVES;
  const dim3 grid((grid_waves + wpb - 1) / wpb), block(64 * wpb);
  hipLaunchKernelGGL((attn_kernel<T, QKV, FUSED>), grid, block, 0, s, a);
  return KO_LAUNCH_STATUS();
}

// Wavefronts per workgroup of attn1_kernel for a unit size: 8 for long units
// (>= 1024 keys, at least 8 steps per wavefront), else the largest of 4, 2, 1
// that splits the unit into whole 16-key steps.
int waves_per_unit(int unit) {
  if (unit >= 1024 && unit % 128 == 0) return 8;
  return unit % 64 == 0 ? 4 : unit % 32 == 0 ? 2 : 1;
}

template <bool QKV, int WM, bool FUSED>
int launch1_wm(const AttnArgs& a, int grid_waves, hipStream_t s) {
  const dim3 grid((grid_waves + WM - 1) / WM), block(64 * WM);
  hipLaunchKernelGGL((attn1_kernel<QKV, WM, FUSED>), grid, block, 0, s, a);
  return KO_LAUNCH_STATUS();
}

template <bool QKV, bool FUSED>
int launch1(const AttnArgs& a, int grid_waves, hipStream_t s) {
  switch (waves_per_unit(a.unit)) {
    case 8: return launch1_wm<QKV, 8, FUSED>(a, grid_waves, s);
    case 4: return launch1_wm<QKV, 4, FUSED>(a, grid_waves, s);
    case 2: return launch1_wm<QKV, 2, FUSED>(a, grid_waves, s);
    default: return launch1_wm<QKV, 1, FUSED>(a, grid_waves, s);
  }
}

template <bool FUSED>
int launch_t(const AttnArgs& a, int T, int grid_waves, hipStream_t s) {
  switch (T) {
    case 1: return launch1<false, FUSED>(a, grid_waves, s);
    case 2: return launch<2, false, FUSED>(a, grid_waves, s);
    case 3: return launch<3, false, FUSED>(a, grid_waves, s);
    default: return launch<4, false, FUSED>(a, grid_waves, s);
  }
}

AttnArgs base_args(const void* k_cache, const void* v_cache, const int* lens, int len_offset,
                   int cap, long long cb, long long ch, int B, int nkv, int unit, int max_units,
                   float scale, float* o_part, float* ml) {
  AttnArgs a = {};
  a.kc = static_cast<uint16_t*>(const_cast<void*>(k_cache));
  a.vc = static_cast<uint16_t*>(const_cast<void*>(v_cache));
  a.lens = lens;
  a.len_off = len_offset;
  a.cap = cap;
  a.cb = cb;
  a.ch = ch;
  a.B = B;
  a.nkv = nkv;
  a.unit = unit;
  a.max_units = max_units;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.o_part = o_part;
  a.ml = ml;
  a.max_pos = 1;
  return a;
}

}  // namespace

extern "C" {

int ko_decode_attn_partial(const void* q, const void* k_cache, const void* v_cache,
                           const int* kv_lens, int len_offset, int cap,
                           long long cache_b_stride, long long cache_h_stride, int B, int T,
                           int nkv, int head_dim, int unit, int max_units, int grid_waves,
                           float scale, float* o_part, float* ml, void* stream) {
  int st = check_common(k_cache, v_cache, kv_lens, cap, cache_b_stride, cache_h_stride, B, T, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (!q || !aligned16(q) || grid_waves < 1) return KO_EINVAL;
  AttnArgs a = base_args(k_cache, v_cache, kv_lens, len_offset, cap, cache_b_stride,
                         cache_h_stride, B, nkv, unit, max_units, scale, o_part, ml);
  a.q = static_cast<const uint16_t*>(q);
  return launch_t<false>(a, T, grid_waves, static_cast<hipStream_t>(stream));
}

int ko_decode_attn_combine(const float* o_part, const float* ml, const int* kv_lens,
                           int len_offset, int cap, int B, int T, int nq, int head_dim, int unit,
                           int max_units, void* out, void* stream) {
  if (!o_part || !ml || !kv_lens || !out) return KO_EINVAL;
  if (head_dim != D) return KO_ENOTSUP;
  if (B < 1 || T < 1 || nq < 1 || unit < 1 || (long long)max_units * unit < cap) return KO_EINVAL;
  if (!aligned16(out)) return KO_EINVAL;
  const int rows = B * T * nq;
  const int wpb = rows <= 1024 ? 1 : WAVES;  // small merges: spread rows over more CUs
  hipLaunchKernelGGL(attn_combine_kernel, dim3((rows + wpb - 1) / wpb), dim3(64 * wpb), 0,
                     static_cast<hipStream_t>(stream), o_part, ml, kv_lens, len_offset, cap, T,
                     nq, rows, unit, max_units, static_cast<uint16_t*>(out));
  return KO_LAUNCH_STATUS();
}

int ko_decode_attn(const void* q, const void* k_cache, const void* v_cache, const int* kv_lens,
                   int len_offset, int cap, long long cache_b_stride, long long cache_h_stride,
                   int B, int T, int nkv, int head_dim, int unit, int max_units, int grid_waves,
                   float scale, float* o_part, float* ml, int* counters, void* out,
                   void* stream) {
  if (!counters) {
    int st = ko_decode_attn_partial(q, k_cache, v_cache, kv_lens, len_offset, cap,
                                    cache_b_stride, cache_h_stride, B, T, nkv, head_dim, unit,
                                    max_units, grid_waves, scale, o_part, ml, stream);
    if (st) return st;
    return ko_decode_attn_combine(o_part, ml, kv_lens, len_offset, cap, B, T, nkv * G, head_dim,
                                  unit, max_units, out, stream);
  }
  int st = check_common(k_cache, v_cache, kv_lens, cap, cache_b_stride, cache_h_stride, B, T, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (!q || !aligned16(q) || !out || !aligned16(out) || grid_waves < 1) return KO_EINVAL;
  AttnArgs a = base_args(k_cache, v_cache, kv_lens, len_offset, cap, cache_b_stride,
                         cache_h_stride, B, nkv, unit, max_units, scale, o_part, ml);
  a.q = static_cast<const uint16_t*>(q);
  a.counters = counters;
  a.out = static_cast<uint16_t*>(out);
  return launch_t<true>(a, T, grid_waves, static_cast<hipStream_t>(stream));
}

int ko_decode_attn_qkv(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                       const void* sin, int max_pos, const int* pos, void* k_cache,
                       void* v_cache, int cap, long long cache_b_stride,
                       long long cache_h_stride, int B, int nkv, int head_dim, int unit,
                       int max_units, int grid_waves, float eps, float scale, float* o_part,
                       float* ml, int* counters, void* out, void* stream) {
  int st = check_common(k_cache, v_cache, pos, cap, cache_b_stride, cache_h_stride, B, 1, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (!qkv || !q_w || !k_w || !cos || !sin || !out || max_pos < 1 || grid_waves < 1)
    return KO_EINVAL;
  if (!aligned16(qkv) || !aligned16(q_w) || !aligned16(k_w) || !aligned16(cos) ||
      !aligned16(sin) || !aligned16(out))
    return KO_EINVAL;
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (counters) return launch1<true, true>(a, grid_waves, s);
  st = launch1<true, false>(a, grid_waves, s);
  if (st) return st;
  return ko_decode_attn_combine(o_part, ml, pos, 1, cap, B, 1, nkv * G, head_dim, unit,
                                max_units, out, stream);
}

long long ko_decode_attn_qkv_oproj_sync_ints(void) { return OPROJ_SYNC_INTS; }

int ko_decode_attn_qkv_oproj(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                             const void* sin, int max_pos, const int* pos, void* k_cache,
                             void* v_cache, int cap, long long cache_b_stride,
                             long long cache_h_stride, int B, int nkv, int head_dim, int unit,
                             int max_units, int grid_waves, float eps, float scale,
                             float* o_part, float* ml, int* counters, void* out,
                             const void* w_o, void* h, int H, int* sync, int* err,
                             int delay_ns, void* stream) {
  int st = check_common(k_cache, v_cache, pos, cap, cache_b_stride, cache_h_stride, B, 1, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (!qkv || !q_w || !k_w || !cos || !sin || !out || !counters || !w_o || !h || !sync || !err ||
      max_pos < 1 || grid_waves < 4 || H < 8 || (H & 7))
    return KO_EINVAL;
  if (!aligned16(qkv) || !aligned16(q_w) || !aligned16(k_w) || !aligned16(cos) ||
      !aligned16(sin) || !aligned16(out) || !aligned16(w_o) || !aligned16(h))
    return KO_EINVAL;
  if (B > 2 || waves_per_unit(unit) != 4) return KO_ENOTSUP;
  const int K = nkv * G * D;  // o projection input width
  if (K > 2 * GEMV_NT * 8) return KO_ENOTSUP;
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
  GemvArgs g = {};
  g.x = static_cast<const uint16_t*>(out);
  g.w = static_cast<const uint16_t*>(w_o);
  g.h = static_cast<uint16_t*>(h);
  g.mrows = B;
  g.N = H;
  g.K = K;
  g.eps = eps;
  const int nattn = grid_waves / 4;
  const dim3 grid(nattn + (H + 7) / 8), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int ticks = delay_ns > 0 ? delay_ns / 10 : 0;  // s_memrealtime runs at 100 MHz
  if (B == 1)
    hipLaunchKernelGGL((attn_oproj_kernel<true, 1>), grid, block, 0, s, a, g, nattn, ticks, err);
  else
    hipLaunchKernelGGL((attn_oproj_kernel<true, 2>), grid, block, 0, s, a, g, nattn, ticks, err);
  return KO_LAUNCH_STATUS();
}

}  // extern "C"
