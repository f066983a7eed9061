// Stage-to-stage hand-off between the workgroups of one launch.
//
// A launch that runs several dependent stages (each a set of workgroups with
// consecutive indices, every stage after the ones it reads from) lets a
// consumer workgroup start its own independent loads (weights, cached keys)
// before its input exists, then wait for the stage that produces the input.
//
// Per stage, a block of STAGE_INTS int32 in device memory, zero before the
// launch and left zero after it:
//   lines 0..31   arrival counters of 32 groups (workgroup index % 32),
//   line 32       count of complete groups,
//   lines 33..64  32 copies of the done flag (a waiter polls copy index % 32,
//                 so the polls of many workgroups spread over 32 addresses).
// Lines are 128 bytes apart. All accesses are relaxed agent-scope atomics
// (global_load / global_store / global_atomic ... sc1, performed at the device
// coherence point); a producer's data stores are device-coherent stores too,
// performed (s_waitcnt vmcnt(0)) before the producer arrives. Same-address
// atomics serialise at tens of ns each, hence the two-level count.
//
// Progress: a workgroup waits only for stages with lower workgroup indices, and
// each XCD dispatches its workgroups in index order, so the workgroups waited
// for are resident or finished. Each wait is also bounded: after SPIN polls, or
// as soon as another waiter has given up, it sets *err and returns (the launch
// then finishes with invalid results instead of hanging).
#pragma once

#include "ko_common.h"

namespace ko {

constexpr int ST_LINE = 32;  // int32 per 128-byte line
constexpr int ST_GROUPS = 32;
constexpr int ST_TOP = ST_GROUPS * ST_LINE;
constexpr int ST_FLAG0 = ST_TOP + ST_LINE;
constexpr int STAGE_INTS = ST_FLAG0 + ST_GROUPS * ST_LINE;
constexpr int ST_SPIN = 1 << 18;

__device__ __forceinline__ int st_load(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int st_add(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One thread. Arrival of workgroup idx of a stage of n workgroups (every idx in
// [0, n) arrives once, after its outputs are performed). Returns true for the
// arrival that completes the stage; the counters are left zero.
__device__ inline bool stage_arrive(int* st, int idx, int n) {
  const int grp = idx % ST_GROUPS;
  const int in_grp = (n - grp + ST_GROUPS - 1) / ST_GROUPS;  // idx in [0, n) with idx % 32 == grp
  int* gc = st + grp * ST_LINE;
  if (st_add(gc, 1) != in_grp - 1) return false;
  st_store(gc, 0);
  const int groups = n < ST_GROUPS ? n : ST_GROUPS;
  if (st_add(st + ST_TOP, 1) != groups - 1) return false;
  st_store(st + ST_TOP, 0);
  return true;
}

// One thread. Arrival counted on a single counter (stages with few arrivals
// whose indices are not 0..n-1). Returns true for the n-th arrival.
__device__ inline bool stage_arrive1(int* st, int n) {
  if (st_add(st + ST_TOP, 1) != n - 1) return false;
  st_store(st + ST_TOP, 0);
  return true;
}

// One thread: set / clear every copy of the done flag.
__device__ inline void stage_flags(int* st, int v) {
  for (int f = 0; f < ST_GROUPS; ++f) st_store(st + ST_FLAG0 + f * ST_LINE, v);
}

// One thread: wait for the done flag of stage st (copy idx % 32).
__device__ inline void stage_wait(const int* st, int idx, int* err) {
  const int* f = st + ST_FLAG0 + (idx % ST_GROUPS) * ST_LINE;
  for (int it = 0; st_load(f) == 0; ++it) {
    if ((it & 15) == 15 && st_load(err) != 0) return;  // another waiter gave up
    if (it >= ST_SPIN) {
      st_store(err, 1);
      return;
    }
    __builtin_amdgcn_s_sleep(8);
  }
}

}  // namespace ko
