// expert_cache_manage on gfx950: one policy step of one layer's cache in ONE wavefront.
//
// Behaviour follows kernels/expert_cache.hip:191-282 and tests/test_policy.py:83-132
// (the step is restated in oracle/policy.c); the structure is this file's own:
//
//  * Every global load the step needs (step counter, ids, slot_expert, slot_stamp, the
//    first 512 table entries) is issued up front, so the step costs one memory round trip
//    plus the stores. There are no workgroup barriers: all cross-lane traffic is DPP,
//    ballots, or LDS ordered by lgkmcnt waits.
//  * Slots live in registers, CS per lane (slot s = lane + 64*c). The LDS holds the routed
//    flags and the table (for E <= 4096) so that the remap can read the updated table
//    without another trip to memory.
//  * Misses are enumerated in ascending expert id with ballot + popcount prefixes.
//  * Victims are the nact smallest keys (stamp << 20 | slot) among the slots whose expert
//    is not routed this step, assigned in ascending key order to the misses in ascending
//    id order. Few inserts: repeated DPP wave-min (one 6-step DPP reduction per insert).
//    Many inserts: every evictable key is ranked against all keys broadcast from LDS.
//    Both give the same assignment (keys are unique, installing does not change any other
//    slot's key or evictability).
//  * A fused tail rewrites the caller's routing ids into slot ids against the updated table
//    (vllm_expert_cache/cache.py:108-110 semantics, negative ids wrapping).
#pragma once
#include <type_traits>

#include "wave.h"

namespace ec {

constexpr int kSlotBits = 20;
constexpr int kSlotMask = (1 << kSlotBits) - 1;
constexpr int kMaxSlots = 1024;
constexpr int kMaxInserts = 1024;
constexpr int kLdsExperts = 4096;   // flags + table fit in LDS up to this many experts
constexpr int kIdRegs = 4;          // ids held in registers: mk <= 256
constexpr int kTabRegs = 8;         // table entries prefetched per lane: E <= 512
constexpr long long kKeyMax = 0x7FFFFFFFFFFFFFFFll;

struct ManageArgs {
  const void* ids;
  int mk, E, S, max_distinct, max_inserts;
  int* table;
  int* map_cold;
  int* slot_expert;
  long long* slot_stamp;
  unsigned char* routed;
  long long* step;
  int* miss;
  int* n_miss;
  int policy, decay;
  void* out;  // remap output (dtype of ids), or null
};

// Experts above kLdsExperts (GLOBAL_E) keep their flags in the caller's `routed` buffer and
// read the table from memory; the LDS arrays for them shrink to one element.
template <bool GLOBAL_E>
struct ManageLds {
  unsigned char flag[GLOBAL_E ? 1 : kLdsExperts];
  unsigned char hit[kMaxSlots];    // slot refreshed by a routed expert this step
  unsigned char fresh[kMaxSlots];  // slot received an insert this step
  int tab[GLOBAL_E ? 1 : kLdsExperts];
  int se[kMaxSlots];               // slot -> expert, for the installs
  long long key[kMaxSlots + 2];    // rank path: key or INT64_MAX
  int vic[kMaxInserts];            // insert r -> victim slot
  int mis[kMaxInserts];            // insert r -> missing expert
};

template <int IDB>
__device__ __forceinline__ long long load_id(const void* p, int i) {
  if constexpr (IDB == 8)
    return reinterpret_cast<const long long*>(p)[i];
  else
    return (long long)reinterpret_cast<const int*>(p)[i];
}

template <int IDB>
__device__ __forceinline__ void store_id(void* p, int i, int v) {
  if constexpr (IDB == 8)
    reinterpret_cast<long long*>(p)[i] = (long long)v;
  else
    reinterpret_cast<int*>(p)[i] = v;
}

template <bool GLOBAL_E>
__device__ __forceinline__ void step_sync() {
  if constexpr (GLOBAL_E)
    mem_sync();
  else
    lds_sync();
}

__device__ __forceinline__ long long victim_key(long long stamp, int slot) {
  return (long long)(((unsigned long long)stamp << kSlotBits) | (unsigned long long)slot);
}

// Which victim search is cheaper: nact wave-min reductions (~CS + 40 instructions each)
// or one rank pass (S keys from LDS against CS keys per lane).
template <int CS>
__device__ __forceinline__ bool use_argmin(int nact, int S) {
  return nact * (CS + 40) <= S * CS + 256;
}

// One policy step. On return, the updated table is in L.tab (or in memory for GLOBAL_E)
// and idv holds ids[lane + 64k] (or -1 past mk).
template <int CS, bool GLOBAL_E, int IDB>
__device__ __forceinline__ void manage_step(const ManageArgs& a, ManageLds<GLOBAL_E>& L,
                                            long long (&idv)[kIdRegs]) {
  const int lane = __lane_id();
  const int E = a.E, S = a.S, mk = a.mk;

  // ---- every independent load, issued together ---------------------------------------
  // Addresses are clamped into range instead of predicated, so no load waits behind a
  // branch; lanes past the end substitute their sentinel after the loads return.
  const long long st = a.step[0] + 1;
  using IdT = typename std::conditional<IDB == 8, long long, int>::type;
  IdT raw[kIdRegs];
  if (mk > 0) {
#pragma unroll
    for (int k = 0; k < kIdRegs; ++k)
      raw[k] = reinterpret_cast<const IdT*>(a.ids)[min(lane + k * kWave, mk - 1)];
  }
  int se[CS];
  long long sp[CS];
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int s = min(lane + c * kWave, S - 1);
    se[c] = a.slot_expert[s];
    sp[c] = a.slot_stamp[s];
  }
  int tv[kTabRegs];
  if constexpr (!GLOBAL_E) {
#pragma unroll
    for (int u = 0; u < kTabRegs; ++u) tv[u] = a.table[min(lane + u * kWave, E - 1)];
  }
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k)
    idv[k] = (mk > 0 && lane + k * kWave < mk) ? (long long)raw[k] : -1;
#pragma unroll
  for (int c = 0; c < CS; ++c)
    if (lane + c * kWave >= S) se[c] = -1;

  unsigned char* flag;
  if constexpr (GLOBAL_E)
    flag = a.routed;
  else
    flag = L.flag;

  for (int e = lane; e < E; e += kWave) flag[e] = 0;
  for (int s = lane; s < S; s += kWave) {
    L.hit[s] = 0;
    L.fresh[s] = 0;
  }
  step_sync<GLOBAL_E>();

  // ---- routed flags (ids outside [0,E) are padding; int64 ids truncate like .to(int32))
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k) {
    const int e = (int)idv[k];
    if (e >= 0 && e < E) flag[e] = 1;
  }
  for (int i = lane + kIdRegs * kWave; i < mk; i += kWave) {
    const int e = (int)load_id<IDB>(a.ids, i);
    if (e >= 0 && e < E) flag[e] = 1;
  }
  if constexpr (!GLOBAL_E) {
#pragma unroll
    for (int u = 0; u < kTabRegs; ++u) {
      const int e = lane + u * kWave;
      if (e < E) L.tab[e] = tv[u];
    }
    for (int base = kTabRegs * kWave; base < E; base += kTabRegs * kWave) {
#pragma unroll
      for (int u = 0; u < kTabRegs; ++u) {
        const int e = base + lane + u * kWave;
        tv[u] = a.table[min(e, E - 1)];
      }
#pragma unroll
      for (int u = 0; u < kTabRegs; ++u) {
        const int e = base + lane + u * kWave;
        if (e < E) L.tab[e] = tv[u];
      }
    }
  }
  step_sync<GLOBAL_E>();

  // ---- distinct count; the caller's `routed` is left holding the flags ----------------
  int cnt = 0;
  for (int base = 0; base < E; base += kWave) {
    const int e = base + lane;
    const bool f = e < E && flag[e];
    if constexpr (!GLOBAL_E) {
      if (e < E) a.routed[e] = f ? 1 : 0;
    }
    cnt += __popcll(__ballot(f));
  }
  if (cnt > a.max_distinct) {  // wide step: read through, nothing else changes
    if (lane == 0) {
      a.step[0] = st;
      a.n_miss[0] = 0;
    }
    return;
  }

  // ---- hits mark their slot; misses enumerate in ascending expert id -----------------
  int total = 0;
  for (int base = 0; base < E; base += kWave) {
    const int e = base + lane;
    const bool f = e < E && flag[e];
    int t = -1;
    if (f) {
      if constexpr (GLOBAL_E)
        t = a.table[e];
      else
        t = L.tab[e];
    }
    if (f && t >= 0 && t < S) L.hit[t] = 1;
    const bool m = f && t < 0;
    const unsigned long long mask = __ballot(m);
    const int j = total + __popcll(mask & lanes_below());
    if (m && j < a.max_inserts) {
      L.mis[j] = e;
      a.miss[2 * j] = e;
    }
    total += __popcll(mask);
  }
  const int nins = min(total, a.max_inserts);
  lds_sync();

  const bool lru = a.policy == 0;
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int s = lane + c * kWave;
    if (s < S && L.hit[s]) sp[c] = lru ? st : (long long)((unsigned long long)sp[c] + 1ull);
  }
  if (nins == 0) {  // no inserts: refreshed stamps only, no ageing
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      const int s = lane + c * kWave;
      if (s < S && L.hit[s]) a.slot_stamp[s] = sp[c];
    }
    if (lane == 0) {
      a.step[0] = st;
      a.n_miss[0] = 0;
    }
    return;
  }

  // LFU ageing on inserting steps where st % decay == 0
  if (!lru && a.decay > 0 && (st % (long long)a.decay) == 0) {
#pragma unroll
    for (int c = 0; c < CS; ++c) sp[c] >>= 1;
  }

  // ---- keys of the evictable slots (expert not routed this step) ---------------------
  long long key[CS];
  bool ev[CS];
  int nev = 0;
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int s = lane + c * kWave;
    const int x = se[c];
    ev[c] = s < S && (x < 0 || x >= E || !flag[x]);
    key[c] = victim_key(sp[c], s);
    nev += __popcll(__ballot(ev[c]));
    if (s < S) L.se[s] = x;
  }
  const int nact = min(nins, nev);

  // ---- victims: the nact smallest keys, ascending ------------------------------------
  if (use_argmin<CS>(nact, S)) {
    for (int r = 0; r < nact; ++r) {
      long long m = kKeyMax;
#pragma unroll
      for (int c = 0; c < CS; ++c)
        if (ev[c] && key[c] < m) m = key[c];
      m = wave_min_i64(m);
      const int sl = (int)(m & kSlotMask);
#pragma unroll
      for (int c = 0; c < CS; ++c)
        if (lane + c * kWave == sl) ev[c] = false;
      if (lane == 0) L.vic[r] = sl;
    }
  } else {
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      const int s = lane + c * kWave;
      if (s < S) L.key[s] = ev[c] ? key[c] : kKeyMax;
    }
    if (lane == 0) L.key[S] = kKeyMax;  // pad to an even count for paired reads
    lds_sync();
    int rank[CS];
#pragma unroll
    for (int c = 0; c < CS; ++c) rank[c] = 0;
    const int S2 = (S + 1) & ~1;
    for (int j = 0; j < S2; j += 2) {
      const long long k0 = L.key[j], k1 = L.key[j + 1];
#pragma unroll
      for (int c = 0; c < CS; ++c) rank[c] += (k0 < key[c]) + (k1 < key[c]);
    }
#pragma unroll
    for (int c = 0; c < CS; ++c)
      if (ev[c] && rank[c] < nins) L.vic[rank[c]] = lane + c * kWave;
  }
  lds_sync();

  // ---- installs (distinct slots, distinct experts: independent, one per lane) ---------
  const long long fresh = lru ? st : 1;
  for (int r = lane; r < nact; r += kWave) {
    const int sl = L.vic[r];
    const int e = L.mis[r];
    const int old = L.se[sl];
    if (old >= 0 && old < E) {
      a.table[old] = -1;
      a.map_cold[old] = old;
      if constexpr (!GLOBAL_E) L.tab[old] = -1;
    }
    a.table[e] = sl;
    a.map_cold[e] = -1;
    a.miss[2 * r + 1] = sl;
    if constexpr (!GLOBAL_E) L.tab[e] = sl;
    L.fresh[sl] = 1;
    L.se[sl] = e;
  }
  step_sync<GLOBAL_E>();

#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int s = lane + c * kWave;
    if (s < S) {
      if (L.fresh[s]) {
        se[c] = L.se[s];
        sp[c] = fresh;
      }
      a.slot_expert[s] = se[c];
      a.slot_stamp[s] = sp[c];
    }
  }
  if (lane == 0) {
    a.step[0] = st;
    a.n_miss[0] = nact;
  }
}

// out[i] = table[ids[i]] against the updated table, negative ids wrapping.
template <bool GLOBAL_E, int IDB>
__device__ __forceinline__ void remap_tail(const ManageArgs& a, const ManageLds<GLOBAL_E>& L,
                                           const long long (&idv)[kIdRegs]) {
  const int lane = __lane_id();
  const int E = a.E, mk = a.mk;
  auto lookup = [&](long long v) -> int {
    if (v < 0) v += E;
    if (v < 0 || v >= E) return -1;
    if constexpr (GLOBAL_E)
      return a.table[v];
    else
      return L.tab[v];
  };
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k) {
    const int i = lane + k * kWave;
    if (i < mk) store_id<IDB>(a.out, i, lookup(idv[k]));
  }
  for (int i = lane + kIdRegs * kWave; i < mk; i += kWave)
    store_id<IDB>(a.out, i, lookup(load_id<IDB>(a.ids, i)));
}

template <int CS, bool GLOBAL_E, int IDB, bool REMAP>
__global__ __launch_bounds__(kWave) void manage_k(ManageArgs a) {
  __shared__ ManageLds<GLOBAL_E> L;
  long long idv[kIdRegs];
  manage_step<CS, GLOBAL_E, IDB>(a, L, idv);
  if constexpr (REMAP) {
    if constexpr (GLOBAL_E) mem_sync();
    else lds_sync();
    remap_tail<GLOBAL_E, IDB>(a, L, idv);
  }
}

// Standalone remap, any grid; one id per lane per iteration.
template <int IDB>
__global__ __launch_bounds__(256) void remap_k(const void* ids, int n, const int* table, int E,
                                               void* out) {
  const int stride = gridDim.x * blockDim.x;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    long long v = load_id<IDB>(ids, i);
    if (v < 0) v += E;
    store_id<IDB>(out, i, (v >= 0 && v < E) ? table[v] : -1);
  }
}

}  // namespace ec
