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
#include "attn_core.h"

#include <mutex>

using namespace ko;

// Scratch of ko_decode_attn_noalloc: the fp32 partials (o_part, then ml) of the
// two-launch form, in a fixed device array instead of caller or library
// allocations. Each GPU the library runs on holds its own copy, for the life of
// the process; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (noalloc_scratch below).
constexpr long long KO_NOALLOC_SCRATCH_FLOATS = (16LL << 20) / 4;  // 16 MiB
static __device__ __align__(256) float scratch[KO_NOALLOC_SCRATCH_FLOATS];

namespace {

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
  int my_n = 0, my_incl = 0, total, my_len = 0;
  if (small_b) {
    if (lane < a.B) {
      my_len = seq_len(a.lens, lane, a.len_off, a.cap);
      my_n = nunits(my_len, unit);
    }
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
      kv_len = readlane(my_len, b);  // lane b loaded it: no second round trip
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
          a.q + ((long long)(b * a.tstride + a.t0 + trow) * nq + kvh * G + (r & 3)) * D + 8 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) qa[i] = __builtin_bit_cast(bf16x8, ldg16(qrow + 32 * i));
    }

    const int tq = g % T;                           // token of this lane's score rows
    // exclusive causal key limit: token t0 + tq of the call's tstride tokens
    // sits at key position kv_len - tstride + t0 + tq
    const int lim = min(k1, kv_len - a.tstride + a.t0 + tq + 1);

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
    // With FUSED the partials are read back in this launch by another
    // workgroup: device-coherent stores (no L2 write-back needed).
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const long long R = (long long)(b * a.tstride + a.t0 + t) * nq + kvh * G + g;
      float* dst = a.o_part + (R * max_units + c) * D + 8 * r;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        if (g == j) {
          if constexpr (FUSED) {
#pragma unroll
            for (int e = 0; e < 8; e += 2)
              store_coherent(dst + e, make_float2(acc[t][j][e], acc[t][j][e + 1]));
          } else {
            reinterpret_cast<float4*>(dst)[0] =
                make_float4(acc[t][j][0], acc[t][j][1], acc[t][j][2], acc[t][j][3]);
            reinterpret_cast<float4*>(dst)[1] =
                make_float4(acc[t][j][4], acc[t][j][5], acc[t][j][6], acc[t][j][7]);
          }
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
      const long long R = (long long)(b * a.tstride + a.t0 + g) * nq + kvh * G + r;
      if constexpr (FUSED)
        store_coherent(a.ml + 2 * (R * max_units + c), make_float2(m, l));
      else
        reinterpret_cast<float2*>(a.ml)[R * max_units + c] = make_float2(m, l);
    }

    if constexpr (FUSED) {
      // Count the unit's arrival once this wavefront's partial stores are
      // performed at device scope; the last arrival of the (b, kv_head) pair
      // merges the pair's partials with device-scope loads.
      __builtin_amdgcn_s_waitcnt(0);
      int prev = 0;
      int* ctr = a.counters + (long long)b * nkv + kvh;
      if (lane == 0) prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      prev = readlane(prev, 0);
      const int n = nunits(kv_len, unit);
      if (prev == n - 1) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int j = 0; j < G; ++j)
            combine_row<32, true>(a.o_part, a.ml,
                                  (long long)(b * a.tstride + a.t0 + t) * nq + kvh * G + j, n,
                                  nullptr, 0, a.cap, unit, max_units, a.out);
        if (lane == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <bool QKV, int WM, bool FUSED>
__global__ __launch_bounds__(64 * WM) void attn1_kernel(AttnArgs a) {
  attn1_body<QKV, WM, FUSED>(a, blockIdx.x, gridDim.x);
}

// Decode attention and the o projection in one launch (one query token, 1-2
// sequences, 4 wavefronts per unit). Workgroups [0, nattn) run the attention
// units with the fused combine; the rest each own 8 output columns of the o
// projection: they issue all their weight loads while the attention's latency
// chain runs, then finish as the RESID GEMV (h <- bf16(h + bf16(W_o attn))),
// each wavefront reading a chunk of the merged attention output (device-scope
// loads) as soon as the done flags of the (sequence, KV head) pairs it covers
// are raised. Workgroups are dispatched in index order, so every attention
// workgroup is resident before any o-projection workgroup waits; the waits are
// also bounded (spin_max polls, then *err is set and the wavefront goes on).
// Synchronisation words: OPROJ_FLAG0 and what follows it.

// The 8-byte word of a workgroup's group: the launch epoch (high half) and the
// count of the group's workgroups that have been counted this launch (low half).
// A projection workgroup counts itself at its start (the epoch comes back with
// the add), an attention workgroup reads the epoch with a plain device-scope
// load at its start and counts itself at its end, so no atomic sits on the
// attention's path to its merge. The last workgroup of the group to be counted
// stores (epoch + 1, 0) for the next launch; by then every workgroup of the
// group has read the epoch.
struct OprojGroup {
  unsigned long long* word = nullptr;
  int in_grp = 0;
  __device__ void locate(int* sync, int blk, int nblk) {
    const int grp = blk % OPROJ_FLAGS;
    word = reinterpret_cast<unsigned long long*>(sync + OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * grp +
                                                 OPROJ_GROUP_WORD);
    in_grp = (nblk - grp + OPROJ_FLAGS - 1) / OPROJ_FLAGS;
  }
  // The epoch alone (the word's high half, 4 bytes: an 8-byte load whose dead
  // low half is reused at once makes the compiler wait for every load in flight).
  __device__ int peek_epoch() const {
    return __hip_atomic_load(reinterpret_cast<int*>(word) + 1, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  // Count this workgroup; returns the epoch.
  __device__ int count() const {
    const unsigned long long old =
        __hip_atomic_fetch_add(word, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int e = (int)(old >> 32);
    if ((unsigned)old == (unsigned)(in_grp - 1))
      __hip_atomic_store(word, (unsigned long long)(unsigned)(e + 1) << 32, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    return e;
  }
};

// The attention side: the merging workgroup of pair p raises copy f of p's done
// flag in line f for every f (one store per lane), so each group of waiters
// polls its own 128-byte line.
struct OprojHooks {
  static constexpr bool kNotify = true;
  int* sync;
  int blk, nblk;
  OprojGroup grp;  // thread 0
  int epoch = 0;   // thread 0
  __device__ void begin() {
    if (threadIdx.x == 0) {
      grp.locate(sync, blk, nblk);
      epoch = grp.peek_epoch();
    }
  }
  __device__ void merged(const AttnArgs&, int pair) const {  // wavefront 0
    const int flag = readlane(epoch, 0) + 1;
    const int l = lane_id();
    if (l < OPROJ_FLAGS)
      __hip_atomic_store(sync + OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * l + pair, flag,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __device__ void end() {
    if (threadIdx.x == 0) grp.count();
  }
  __device__ void no_units() const {}  // the projection workgroups then give up (*err)
};

// The o projection (M rows, 8 output columns per workgroup): gemv_row_body's
// RESID GEMV with R = 8 and two 8-element chunks of K per thread, c = t and
// c = t + 256. The workgroup issues its weight loads, then wavefront 0 polls the
// done flags of all M * nkv (sequence, KV head) pairs of its copy (one int per
// lane, one load per poll) until every one holds this launch's value; then the
// workgroup reads the merged attention output with device-scope loads. The sums
// run in gemv_row_body's order, so h is bit-identical to attention followed by
// the separate RESID GEMV.
template <int M>
__device__ void oproj_body(const GemvArgs& g, int wg, int nkv, int* sync, int* err,
                           int delay_ticks, int spin_max) {
  constexpr int R = 8, CPT = 2;
  __shared__ float red[16][M * R];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int n0 = wg * R;
  const int N = g.N, K = g.K, KC = K >> 3, mr = g.mrows;
  // Let the attention's first (latency-critical) loads go ahead of this
  // workgroup's weight stream: a short wait on the real-time counter.
  if (delay_ticks > 0) {
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < (unsigned long long)delay_ticks) __builtin_amdgcn_s_sleep(4);
  }
  uint16_t hpre;  // this thread's residual element, issued before the weights
  {
    const int ti = t < M * R ? t : 0;
    hpre = resid_load(g, ti / R, n0 + ti % R);
  }
  uint4 w[CPT][R];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = min(t + GEMV_NT * j, KC - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) w[j][r] = ldg16_stream(g.w + (long long)min(n0 + r, N - 1) * K + 8 * c);
  }
  if (wv == 0) {
    int e = 0;
    if (lane == 0) {
      OprojGroup grp;
      grp.locate(sync, blockIdx.x, gridDim.x);
      e = grp.count();
    }
    const int flag = readlane(e, 0) + 1;
    const int npairs = mr * nkv;  // <= OPROJ_MAX_PAIRS
    const int* fp = sync + OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * (blockIdx.x % OPROJ_FLAGS) +
                    (lane < npairs ? lane : 0);
    // One poll in flight with a short sleep between polls: more polls in flight
    // (four, a quarter round trip apart) measured slower, as they load the flag
    // lines and the merges' coherent traffic.
    bool ok = false;
    for (int it = 0; it < spin_max; ++it) {
      const int v = __hip_atomic_load(fp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__ballot(lane < npairs && v != flag) == 0) {
        ok = true;
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
    if (!ok && lane == 0) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const uint4 zero = make_uint4(0, 0, 0, 0);
  uint4 x[CPT][M];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int c = t + GEMV_NT * j;
#pragma unroll
    for (int m = 0; m < M; ++m)
      x[j][m] = c < KC && m < mr ? ldg16_coherent(g.x + (long long)m * K + 8 * c) : zero;
  }
  float acc[M][R];
#pragma unroll
  for (int j = 0; j < CPT; ++j)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = dot8(x[j][m], w[j][r], j == 0 ? 0.f : acc[m][r]);
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = row_sum16(acc[m][r]);
      if ((lane & 15) == 0) red[wv * 4 + (lane >> 4)][m * R + r] = v;
    }
  __syncthreads();
  if (t < M * R) {
    const int m = t / R, r = t - (t / R) * R, n = n0 + r;
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) tot += red[i][m * R + r];
    if (m < mr && n < N) epilogue<EPI_RESID>(g, m, n, tot, 0.f, &hpre);
  }
}

template <bool QKV, int M>
__global__ __launch_bounds__(256) void attn_oproj_kernel(AttnArgs a, GemvArgs g, int nattn,
                                                         int delay_ticks, int spin_max, int* err) {
  if ((int)blockIdx.x < nattn) {
    OprojHooks hooks;
    hooks.sync = a.pairs_done;
    hooks.blk = blockIdx.x;
    hooks.nblk = gridDim.x;
    attn1_body<QKV, 4, true>(a, blockIdx.x, nattn, hooks);
    return;
  }
  oproj_body<M>(g, blockIdx.x - nattn, a.nkv, a.pairs_done, err, delay_ticks, spin_max);
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

template <int T, bool QKV, bool FUSED>
int launch(const AttnArgs& a, int grid_waves, hipStream_t s) {
  // Small grids run one wavefront per workgroup so they spread over more CUs.
  const int wpb = grid_waves <= 1024 ? 1 : WAVES;
  const dim3 grid((grid_waves + wpb - 1) / wpb), block(64 * wpb);
  hipLaunchKernelGGL((attn_kernel<T, QKV, FUSED>), grid, block, 0, s, a);
  return KO_LAUNCH_STATUS();
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
    case 4: return launch1_wm<QKV, 4, FUSED>(a, grid_waves, s);
    case 2: return launch1_wm<QKV, 2, FUSED>(a, grid_waves, s);
    default: return launch1_wm<QKV, 1, FUSED>(a, grid_waves, s);
  }
}

template <bool FUSED>
int launch_tc(const AttnArgs& a, int tc, int grid_waves, hipStream_t s) {
  switch (tc) {
    case 2: return launch<2, false, FUSED>(a, grid_waves, s);
    case 3: return launch<3, false, FUSED>(a, grid_waves, s);
    default: return launch<4, false, FUSED>(a, grid_waves, s);
  }
}

// T query tokens per sequence: T = 1 is the decode kernel; T = 2..4 one
// launch of attn_kernel<T>; T = 5..8 two launches of 2-4 tokens each (5 =
// 3 + 2, 6 = 3 + 3, 7 = 4 + 3, 8 = 4 + 4). Every launch covers the whole key
// range of the call with the causal limit of its own tokens, so all have the
// same units per pair and the merge of a row sees the unit count of the call.
template <bool FUSED>
int launch_t(AttnArgs a, int T, int grid_waves, hipStream_t s) {
  if (T == 1) return launch1<false, FUSED>(a, grid_waves, s);
  a.tstride = T;
  const int n = (T + 3) / 4;
  for (int i = 0, t0 = 0; i < n; ++i) {
    const int tc = (T - t0 + (n - i) - 1) / (n - i);  // 2..4 tokens
    a.t0 = t0;
    const int st = launch_tc<FUSED>(a, tc, grid_waves, s);
    if (st) return st;
    t0 += tc;
  }
  return KO_OK;
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

int ko_decode_attn_token_rows(const void* q, const void* k_cache, const void* v_cache,
                              const int* pos, int cap, long long cache_b_stride,
                              long long cache_h_stride, int B, int T, int nkv, int head_dim,
                              int unit, int max_units, int grid_waves, float scale,
                              float* o_part, float* ml, int* counters, void* out, void* stream) {
  int st = check_common(k_cache, v_cache, pos, cap, cache_b_stride, cache_h_stride, B, T, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (T < 2 || !counters || !q || !aligned16(q) || !out || !aligned16(out) || grid_waves < 1)
    return KO_EINVAL;
  // row b * T + t: the one-token kernel over keys 0 .. pos[b] + t of sequence b
  AttnArgs a = base_args(k_cache, v_cache, pos, 1, cap, cache_b_stride, cache_h_stride, B * T,
                         nkv, unit, max_units, scale, o_part, ml);
  a.rep = T;
  a.q = static_cast<const uint16_t*>(q);
  a.counters = counters;
  a.out = static_cast<uint16_t*>(out);
  return launch1<false, true>(a, grid_waves, static_cast<hipStream_t>(stream));
}

int ko_decode_attn_qkv(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                       const void* sin, int max_pos, const int* pos, void* k_cache,
                       void* v_cache, int cap, long long cache_b_stride,
                       long long cache_h_stride, int B, int nkv, int head_dim, int unit,
                       int max_units, int grid_waves, float eps, float scale, float* o_part,
                       float* ml, int* counters, void* out, const void* rope, int units_per_seq,
                       void* stream) {
  int st = check_common(k_cache, v_cache, pos, cap, cache_b_stride, cache_h_stride, B, 1, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (!qkv || !q_w || !k_w || !cos || !sin || !out || max_pos < 1 || grid_waves < 1)
    return KO_EINVAL;
  if (units_per_seq < 0) return KO_EINVAL;
  // per-sequence units: one wavefront split (4 per unit), the fused merge, and
  // the small-batch unit enumeration
  if (units_per_seq > 0 && (!counters || B > 64 || unit % 64)) return KO_ENOTSUP;
  if (!aligned16(qkv) || !aligned16(q_w) || !aligned16(k_w) || !aligned16(cos) ||
      !aligned16(sin) || !aligned16(out) || (rope && !aligned16(rope)))
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
  a.rope = static_cast<const uint16_t*>(rope);
  a.usplit = units_per_seq;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (counters) return launch1<true, true>(a, grid_waves, s);
  st = launch1<true, false>(a, grid_waves, s);
  if (st) return st;
  return ko_decode_attn_combine(o_part, ml, pos, 1, cap, B, 1, nkv * G, head_dim, unit,
                                max_units, out, stream);
}

long long ko_decode_attn_qkv_oproj_sync_ints(void) { return OPROJ_SYNC_INTS; }

}  // extern "C"

namespace {

constexpr int KO_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[KO_MAX_DEVICES] = {};

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept; 0 on success.
int noalloc_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= KO_MAX_DEVICES) return KO_ENOTSUP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return KO_EINVAL;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return KO_OK;
}

}  // namespace

extern "C" {

int ko_decode_attn_noalloc(const void* q, const void* k_cache, const void* v_cache,
                           const int* kv_lens, int len_offset, int cap, long long cache_b_stride,
                           long long cache_h_stride, int B, int T, int nkv, int head_dim, int unit,
                           int max_units, int grid_waves, float scale, void* out, void* stream) {
  if (B < 1 || T < 1 || nkv < 1 || max_units < 1 || head_dim != D) return KO_EINVAL;
  const long long rows = (long long)B * T * nkv * G;
  const long long n_part = rows * max_units * D;
  const long long off_ml = (n_part + 63) / 64 * 64;  // ml starts 256-byte aligned
  if (off_ml + rows * max_units * 2 > KO_NOALLOC_SCRATCH_FLOATS) return KO_ERANGE;
  float* base = nullptr;
  int st = noalloc_scratch(&base);
  if (st) return st;
  return ko_decode_attn(q, k_cache, v_cache, kv_lens, len_offset, cap, cache_b_stride,
                        cache_h_stride, B, T, nkv, head_dim, unit, max_units, grid_waves, scale,
                        base, base + off_ml, nullptr, out, stream);
}

int ko_decode_attn_qkv_oproj(const void* qkv, const void* q_w, const void* k_w, const void* cos,
                             const void* sin, int max_pos, const int* pos, void* k_cache,
                             void* v_cache, int cap, long long cache_b_stride,
                             long long cache_h_stride, int B, int nkv, int head_dim, int unit,
                             int max_units, int grid_waves, float eps, float scale,
                             float* o_part, float* ml, int* counters, void* out,
                             const void* w_o, void* h, int H, int* sync, int* err,
                             int delay_ns, int spin_max, const void* rope, void* stream) {
  int st = check_common(k_cache, v_cache, pos, cap, cache_b_stride, cache_h_stride, B, 1, nkv,
                        head_dim, unit, max_units, o_part, ml);
  if (st) return st;
  if (!qkv || !q_w || !k_w || !cos || !sin || !out || !counters || !w_o || !h || !sync || !err ||
      max_pos < 1 || grid_waves < 4 || H < 8 || (H & 7))
    return KO_EINVAL;
  if (!aligned16(qkv) || !aligned16(q_w) || !aligned16(k_w) || !aligned16(cos) ||
      !aligned16(sin) || !aligned16(out) || !aligned16(w_o) || !aligned16(h) ||
      (rope && !aligned16(rope)) || (reinterpret_cast<uintptr_t>(sync) & 7u))
    return KO_EINVAL;
  if (B > 2 || waves_per_unit(unit) != 4) return KO_ENOTSUP;
  const int K = nkv * G * D;  // o projection input width
  if (K > 2 * GEMV_NT * 8 || B * nkv > OPROJ_MAX_PAIRS) return KO_ENOTSUP;
  if (spin_max < 0) spin_max = SPIN_MAX;
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
    hipLaunchKernelGGL((attn_oproj_kernel<true, 1>), grid, block, 0, s, a, g, nattn, ticks,
                       spin_max, err);
  else
    hipLaunchKernelGGL((attn_oproj_kernel<true, 2>), grid, block, 0, s, a, g, nattn, ticks,
                       spin_max, err);
  return KO_LAUNCH_STATUS();
}

}  // extern "C"
