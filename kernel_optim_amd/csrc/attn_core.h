// One-query-token split-K GQA decode attention body for gfx950, shared by the
// attention launches of attention.hip (alone, and with the o projection in the
// same launch): argument block, unit enumeration over ragged lengths, the
// log-sum-exp combine, and the per-workgroup unit loop. Semantics are those
// of engine/kernels/fused.py:138-234 with the per-head q/k RMSNorm + RoPE and
// KV append of fused.py:54-96 folded in (QKV).
#pragma once

#include <type_traits>

#include "gemv_core.h"

namespace ko {

constexpr int D = 128;          // head dim
constexpr int G = 4;            // query heads per KV head
constexpr int WAVES = 4;        // wavefronts per workgroup
constexpr float TAU = 8.0f;     // lazy-rescale threshold, log2 units
constexpr float NEG_BIG = -1.0e30f;

constexpr int SPIN_MAX = 1 << 21;
// sync[] of ko_decode_attn_qkv_oproj (all zero before the first launch): OPROJ_FLAGS
// lines of 128 bytes from int OPROJ_FLAG0 on, one per group of workgroups
// (workgroup w of the launch belongs to group w % OPROJ_FLAGS). Line f holds
//   - ints [0, OPROJ_MAX_PAIRS): copy f of the done flag of each (sequence, KV
//     head) pair p = b * nkv + kv_head, which the pair's merging workgroup sets
//     to E + 1 once the pair's merged output is performed;
//   - the 8-byte word at int OPROJ_GROUP_WORD: the group's launch epoch E (high
//     half) and the count of its workgroups counted so far (low half).
// Every workgroup reads E from its group word before it uses it and counts
// itself in the word once; the last one counted sets the word to (E + 1, 0).
// Each launch thus waits for flags equal to E + 1 where the launch before set
// E, so a flag left by an earlier launch never reads as set and no flag is
// ever cleared.
constexpr int OPROJ_FLAG0 = 32, OPROJ_FLAG_STRIDE = 32, OPROJ_FLAGS = 32;
constexpr int OPROJ_MAX_PAIRS = 16, OPROJ_GROUP_WORD = 16;
constexpr int OPROJ_SYNC_INTS = OPROJ_FLAG0 + OPROJ_FLAG_STRIDE * OPROJ_FLAGS;

constexpr int MAX_T = 8;  // query tokens per sequence of one attention call

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
  // One-token kernel, B <= 64, fused merge: cut each sequence's keys into at
  // most usplit units of equal size (a multiple of 64, at least `unit`) from
  // its current length, instead of fixed units of `unit` keys (0: fixed).
  int usplit;
  // Query tokens per sequence in the q / out / partial row layout (T of the
  // call), and the first token this launch serves: calls of more than 4
  // tokens run in launches of up to 4 (attn_kernel's tile holds 4 tokens x 4
  // heads).
  int tstride, t0;
  // Rows per sequence of the one-token kernel (1 normally): with rep > 1 row r
  // is query token r % rep of sequence r / rep, reads that sequence's cache and
  // sees lens[r / rep] + len_off + r % rep keys (the verify step's tokens run
  // as rows of their own; no QKV prologue, fused merge only).
  int rep;
  float scale_log2;
  float* o_part;
  float* ml;
  int* counters;         // [B*nkv] (FUSED)
  uint16_t* out;         // [B*T, nq*D] (FUSED)
  int* pairs_done;       // attention + o projection launch: merged (b, kv_head) pairs
  const uint16_t* rope;  // [B][2][D]: cos and sin rows at each sequence's new position
                         // (QKV; optional, else cosb / sinb at pos)
};

__device__ __forceinline__ int nunits(int len, int unit) {
  return len > 0 ? (len + unit - 1) / unit : 0;
}
// Keys per unit of a sequence of len keys: `unit`, or with usplit > 0 the
// length cut into usplit parts, rounded up to a multiple of 64, at least `unit`.
__device__ __forceinline__ int unit_for(int len, int unit, int usplit) {
  if (usplit <= 0 || len <= 0) return unit;
  const int u = ((len + usplit - 1) / usplit + 63) & ~63;
  return u > unit ? u : unit;
}
__device__ __forceinline__ int seq_len(const int* lens, int b, int off, int cap, int rep = 1) {
  int l;
  if (rep == 1) {
    l = lens[b] + off;
  } else {
    const int bc = b / rep;
    l = lens[bc] + off + (b - bc * rep);
  }
  return l < cap ? l : cap;
}

// Number of (b, c) pairs over the whole batch.
__device__ inline int count_pairs(const int* lens, int off, int cap, int B, int unit, int rep = 1) {
  const int lane = lane_id();
  int tot = 0;
  for (int b0 = 0; b0 < B; b0 += 64) {
    const int b = b0 + lane;
    const int n = b < B ? nunits(seq_len(lens, b, off, cap, rep), unit) : 0;
    tot += readlane(wave_incl_scan(n), 63);
  }
  return tot;
}

// Flattened pair index p -> (b, c).
__device__ inline void locate_pair(int p, const int* lens, int off, int cap, int B, int unit,
                            int& b_out, int& c_out, int rep = 1) {
  const int lane = lane_id();
  int carry = 0;
  for (int b0 = 0; b0 < B; b0 += 64) {
    const int b = b0 + lane;
    const int n = b < B ? nunits(seq_len(lens, b, off, cap, rep), unit) : 0;
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
    // slots to load: the valid ones when n is known, else every slot (n is
    // read from the lengths while the loads are in flight)
    const int cn = n >= 0 ? min(NB, max(0, n - c0)) : min(NB, max_units - c0);
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
//
// Hooks: what a launch that holds the consumer of the merged output adds
// (NoAttnHooks: nothing). kNotify (with FUSED): the merged output is read later
// in the same launch: it is stored device-coherently, and once a pair's merged
// rows are performed wavefront 0 calls merged(a, pair) with the pair's index
// b * nkv + kv_head. begin() runs once per workgroup after its first loads are
// issued, end() once after its last unit; no_units() runs on workgroup 0 when
// no sequence has a key (then nothing is merged).
struct NoAttnHooks {
  static constexpr bool kNotify = false;
  __device__ void begin() {}
  __device__ void merged(const AttnArgs&, int) const {}
  __device__ void end() {}
  __device__ void no_units() const {}
};

template <bool QKV, int WM, bool FUSED, class Hooks = NoAttnHooks>
__device__ __forceinline__ void attn1_body(const AttnArgs& a, int wg, int nwg,
                                           Hooks hooks = Hooks{}) {
  static_assert(!Hooks::kNotify || FUSED, "a consumer in the launch reads the merged output");
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

  // Per-unit inputs. One query token, one sequence, the RoPE rows given and at
  // most one unit per workgroup: this workgroup's unit u = wg is (c = wg / nkv,
  // kv head wg % nkv) whatever the length, so its q-side loads and its first
  // K/V step go out before the length is read (with the keys clamped to the
  // cache instead of the length; keys past the length are masked and patched
  // as with the length clamp, so the result is the same).
  constexpr int NH = G / WM > 0 ? G / WM : 1;  // q heads normed per wavefront
  constexpr int KW = WM > G ? G : 0;           // the wavefront that norms the new key
  const int nqkv = (nq + 2 * nkv) * D;
  uint4 ka[4], va[4];
  uint32_t xh[NH], qwv = 0, cwv = 0, swv = 0, xk = 0, kwv = 0, vv = 0;
  uint4 vnew = make_uint4(0, 0, 0, 0);
  const bool spec = QKV && a.B == 1 && a.rope != nullptr && a.usplit == 0 &&
                    nwg >= nkv * max_units;
  if (spec && wg < nkv * max_units) {
    const int c = wg / nkv, kvh = wg - c * nkv;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.qkv);
#pragma unroll
    for (int n = 0; n < NH; ++n) xh[n] = wave < G ? src[(kvh * G + wave + n * WM) * (D / 2) + lane] : 0u;
    qwv = reinterpret_cast<const uint32_t*>(a.qw)[lane];
    cwv = reinterpret_cast<const uint32_t*>(a.rope)[lane];
    swv = reinterpret_cast<const uint32_t*>(a.rope + D)[lane];
    if (wave == KW) {
      xk = src[(nq + kvh) * (D / 2) + lane];
      kwv = reinterpret_cast<const uint32_t*>(a.kw)[lane];
      vv = src[(nq + nkv + kvh) * (D / 2) + lane];
    }
    vnew = ldg16(a.qkv + (nq + nkv + kvh) * D + 8 * r);
    const int k0 = c * unit + wave * sub;
    if (k0 < a.cap) {
      const int klim = min(k0 + sub, a.cap) - 1;
      const uint16_t* kb = a.kc + (long long)kvh * a.ch;
      const uint16_t* vb = a.vc + (long long)kvh * a.ch;
      const uint16_t* p = kb + (long long)min(k0 + r, klim) * D + 8 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) ka[i] = ldg16_stream(p + 32 * i);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        va[s4] = ldg16_stream(vb + (long long)min(k0 + g + 4 * s4, klim) * D + 8 * r);
    }
  }
  hooks.begin();

  const bool small_b = a.B <= 64;
  int my_n = 0, my_incl = 0, total, len1 = 0, my_len = 0;  // lane b: sequence b (B <= 64)
  if (a.B == 1) {
    // one sequence: its length through a scalar load (the constant address
    // space), which waits on its own counter instead of queueing behind the
    // vector loads above
    const int len = *(const __attribute__((address_space(4))) int*)a.lens + a.len_off;
    len1 = len < a.cap ? len : a.cap;
    my_n = lane == 0 ? nunits(len1, unit_for(len1, unit, a.usplit)) : 0;
    my_incl = readlane(my_n, 0);
    total = my_incl * nkv;
  } else if (small_b) {
    if (lane < a.B) {
      my_len = seq_len(a.lens, lane, a.len_off, a.cap, a.rep);
      my_n = nunits(my_len, unit_for(my_len, unit, a.usplit));
    }
    my_incl = wave_incl_scan(my_n);
    total = readlane(my_incl, 63) * nkv;
  } else {
    total = count_pairs(a.lens, a.len_off, a.cap, a.B, unit, a.rep) * nkv;
  }
  if constexpr (Hooks::kNotify)
    if (total == 0 && wg == 0) hooks.no_units();

  // 2..64 sequences with fixed units: the units are dealt out largest first, the
  // full units (every sequence's first len / unit) and then the part-filled last
  // units in decreasing size (ties: lower sequence first), in a snake order over
  // the workgroups (forward on even rounds, backward on odd ones), so ragged
  // lengths leave every workgroup about the same number of keys (with one
  // round of units the order does not matter). Lane b holds sequence b's count
  // of full units and its last unit's rank.
  const bool balanced = small_b && a.B > 1 && a.usplit == 0 && total > nwg;
  int my_f = 0, my_fincl = 0, my_rank = 0, my_rem = 0, nfull = 0;
  if (balanced) {
    my_f = my_len / unit;
    my_rem = my_len - my_f * unit;
    my_fincl = wave_incl_scan(my_f);
    nfull = readlane(my_fincl, 63);
    for (int j = 0; j < a.B; ++j) {
      const int rj = readlane(my_rem, j);
      my_rank += rj > my_rem || (rj == my_rem && j < lane) ? 1 : 0;
    }
  }

  for (int k = 0;; ++k) {
    const int u = k * nwg + (balanced && (k & 1) ? nwg - 1 - wg : wg);
    if (u >= total) break;
    const bool pre = spec && u == wg;  // this unit's first loads are in flight already
    const int pidx = u / nkv;
    const int kvh = u - pidx * nkv;
    int b, c, kv_len;
    if (a.B == 1) {
      b = 0;
      c = pidx;
      kv_len = len1;
    } else if (balanced) {
      if (pidx < nfull) {
        b = uniform(__popcll(__ballot(my_fincl <= pidx)));
        c = pidx - readlane(my_fincl - my_f, b);
      } else {  // the part-filled unit of rank pidx - nfull
        b = uniform(__builtin_ctzll(__ballot(my_rem > 0 && my_rank == pidx - nfull)));
        c = readlane(my_f, b);
      }
      kv_len = readlane(my_len, b);
    } else if (small_b) {
      b = uniform(__popcll(__ballot(my_incl <= pidx)));
      c = pidx - readlane(my_incl - my_n, b);
      kv_len = readlane(my_len, b);  // lane b loaded it: no second round trip
    } else {
      locate_pair(pidx, a.lens, a.len_off, a.cap, a.B, unit, b, c, a.rep);
      b = uniform(b);
      c = uniform(c);
      if (b < 0) break;  // unreachable while lens[] is unchanged during the launch
      kv_len = uniform(seq_len(a.lens, b, a.len_off, a.cap, a.rep));
    }
    const int unit_b = unit_for(kv_len, unit, a.usplit);  // uniform: one sequence per unit
    const int sub_b = a.usplit > 0 ? unit_b / WM : sub;
    const int ku1 = min((c + 1) * unit_b, kv_len);
    const int k0 = c * unit_b + wave * sub_b;
    const int k1 = min(k0 + sub_b, ku1);
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

    const long long cb_off = (long long)(a.rep == 1 ? b : b / a.rep) * a.cb;  // its cache
    const uint16_t* kb = a.kc + cb_off + (long long)kvh * a.ch;
    const uint16_t* vb = a.vc + cb_off + (long long)kvh * a.ch;
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
    // The first step's K/V loads go out after the q-side loads: loads return
    // in issue order, so the q norm / RoPE then never waits for the K/V data.
    uint4 kb2[4], vb2[4];
    auto load_first_kv = [&] {
      if (active && !pre) {
        load_k(k0, ka);
        load_v(k0, va);
      }
    };

    bf16x8 qa[4];
    uint4 knew[4];
    if constexpr (QKV) {
      // q heads normed by each wavefront (wavefronts past the 4th norm none)
      const bool has_q = wave < G;
      const uint16_t* src = a.qkv + (long long)b * nqkv;
      const bool do_k = new_unit && wave == KW;  // the new key: an idle wavefront if any
      if (!pre) {
        // 2 bf16 of a head row per lane
        auto ld_in = [&](const uint16_t* row) -> uint32_t {
          return reinterpret_cast<const uint32_t*>(row)[lane];
        };
#pragma unroll
        for (int n = 0; n < NH; ++n) xh[n] = has_q ? ld_in(src + (kvh * G + wave + n * WM) * D) : 0u;
        qwv = reinterpret_cast<const uint32_t*>(a.qw)[lane];
        if (a.rope) {
          cwv = reinterpret_cast<const uint32_t*>(a.rope + (long long)b * 2 * D)[lane];
          swv = reinterpret_cast<const uint32_t*>(a.rope + (long long)b * 2 * D + D)[lane];
        } else {
          const int pt = min(max(pnew, 0), a.max_pos - 1);
          cwv = reinterpret_cast<const uint32_t*>(a.cosb + (long long)pt * D)[lane];
          swv = reinterpret_cast<const uint32_t*>(a.sinb + (long long)pt * D)[lane];
        }
        if (do_k) {
          xk = ld_in(src + (nq + kvh) * D);
          kwv = reinterpret_cast<const uint32_t*>(a.kw)[lane];
          vv = ld_in(src + (nq + nkv + kvh) * D);
        }
        if (has_new) vnew = ldg16(src + (nq + nkv + kvh) * D + 8 * r);
      }
      load_first_kv();
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
      load_first_kv();
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
      const int n = nunits(kv_len, unit_b);
      if (lds_prev == n - 1) {
        for (int j = wave; j < G; j += WM)
          combine_row<32, true, Hooks::kNotify>(a.o_part, a.ml, (long long)b * nq + kvh * G + j,
                                                n, nullptr, 0, a.cap, unit, max_units, a.out);
        if constexpr (Hooks::kNotify) {
          __builtin_amdgcn_s_waitcnt(0);  // this wave's merged row is performed
          __syncthreads();
          if (wave == 0) hooks.merged(a, b * nkv + kvh);
        }
        if (threadIdx.x == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();  // the next unit reuses the LDS
  }
  hooks.end();
}


// ---- host-side helpers of the attention launches ----
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int check_common(const void* kc, const void* vc, const int* lens, int cap, long long cb,
                 long long ch, int B, int T, int nkv, int head_dim, int unit, int max_units,
                 const float* o_part, const float* ml) {
  if (!kc || !vc || !lens || !o_part || !ml) return KO_EINVAL;
  if (head_dim != D) return KO_ENOTSUP;
  if (T < 1 || T > MAX_T) return KO_ENOTSUP;
  if (B < 1 || nkv < 1 || cap < 1) return KO_EINVAL;
  if (unit < 16 || (unit & 15)) return KO_EINVAL;
  if ((long long)max_units * unit < cap) return KO_ERANGE;
  if (!aligned16(kc) || !aligned16(vc) || !aligned16(o_part)) return KO_EINVAL;
  if ((cb & 7) || (ch & 7) || cb < 0 || ch < 0) return KO_EINVAL;
  return KO_OK;
}

// Wavefronts per workgroup of attn1_kernel for a unit size: the largest of 4,
// 2, 1 that splits the unit into whole 16-key steps. (8 wavefronts per long
// unit measured slower on MI355X: B16 x 8K partials 85.5 against 83.6 us.)

inline int waves_per_unit(int unit) {
  return unit % 64 == 0 ? 4 : unit % 32 == 0 ? 2 : 1;
}

inline AttnArgs base_args(const void* k_cache, const void* v_cache, const int* lens, int len_offset,
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
  a.tstride = 1;
  a.t0 = 0;
  a.rep = 1;
  return a;
}

}  // namespace ko
