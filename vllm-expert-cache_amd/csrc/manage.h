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
//    Many inserts: a binary search on the key value finds the nact-th smallest key (each
//    probe one ballot count per register chunk); the victims at or below it are ranked
//    among themselves. Both give the same assignment (keys are unique, installing does not
//    change any other slot's key or evictability).
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
constexpr int kTabRegs = 8;         // most table entries held per lane: E <= 512
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
  alignas(16) unsigned char flag[GLOBAL_E ? 16 : kLdsExperts];  // cleared 16 bytes a lane
  alignas(16) unsigned char hit[kMaxSlots];  // slot refreshed by a routed expert this step
  int tab[GLOBAL_E ? 1 : kLdsExperts];
  alignas(16) long long key[kMaxSlots + 8];  // select path: victim keys, INT64_MAX padded
  int rank[kMaxSlots];             // select path: key order of each compacted victim
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

// Which victim search is cheaper: a wave-min reduction plus its install per insert
// (measured on gfx950: ~0.27 us per insert with one slot per lane, ~0.3-0.6 us with 2-8),
// or the threshold select, whose cost hardly depends on the insert count (~1.3 us with one
// slot per lane, ~2-3.6 us with 2-8). The crossovers are about 3 and 6 inserts.
template <int CS>
__device__ __forceinline__ bool use_argmin(int nact, int nev) {
  (void)nev;
  return nact <= (CS == 1 ? 3 : 6);
}

__device__ __forceinline__ long long uniform_i64(long long v) {
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned long long)v);
  const unsigned hi =
      (unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned long long)v >> 32));
  return (long long)(((unsigned long long)hi << 32) | lo);
}

// Table chunks of 64 experts a lane holds in registers for E experts: the launch picks the
// smallest of 1, 2, 4, 8 that covers E (8 also above 512 experts, which the general loops
// handle), so small expert counts do not carry code for 512.
constexpr int table_chunks(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : 8; }

// One policy step. On return, the updated table is in L.tab (or in memory for GLOBAL_E)
// and idv holds ids[lane + 64k] (or -1 past mk). TQ table chunks are held in registers.
//
// PF makes it the prefetch step for predicted ids: the step counter is neither read nor
// written, resident predicted experts keep their stamps, there is no ageing, and installs
// get stamp -1, which marks them pending. Victims are chosen exactly as in a real step (a
// pending slot's key is below every real key, so older unconfirmed predictions go first).
//
// A real step settles the pending slots it finds once it is served (past the read-through
// check): a slot whose expert is routed is confirmed and ends the step with the stamp a
// real install of this step gets (st under LRU, 1 under LFU; after any ageing); a slot
// whose expert is not routed is dropped -- the expert leaves the table and the slot is left
// empty at stamp 0, so a prefetch copy still in flight may stop short. The reference never
// holds a negative stamp, so on its states none of this runs.
template <int CS, bool GLOBAL_E, int IDB, int TQ, bool PF = false>
__device__ __forceinline__ void manage_step(const ManageArgs& a, ManageLds<GLOBAL_E>& L,
                                            long long (&idv)[kIdRegs]) {
  static_assert(!PF || IDB == 4, "prefetch takes int32 ids");
  const int lane = __lane_id();
  const int E = a.E, S = a.S, mk = a.mk;

  // ---- every independent load, issued together ---------------------------------------
  // Addresses are clamped into range instead of predicated, so no load waits behind a
  // branch; lanes past the end substitute their sentinel after the loads return. The step
  // counter is a vector load: a scalar load would count in lgkmcnt, and every LDS fence
  // below would stall on it.
  long long st_v = 0;
  if constexpr (!PF)
    st_v = __hip_atomic_load(a.step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // No branch around the id loads either (a branch join would make the compiler wait for
  // them before issuing the rest): with no ids, they read the 8-byte step counter (the
  // prefetch step: the first table entry) instead.
  using IdT = typename std::conditional<IDB == 8, long long, int>::type;
  const IdT* dummy = PF ? reinterpret_cast<const IdT*>(a.table)
                        : reinterpret_cast<const IdT*>(a.step);
  const IdT* ip = mk > 0 ? reinterpret_cast<const IdT*>(a.ids) : dummy;
  const int last_id = mk > 0 ? mk - 1 : 0;
  IdT raw[kIdRegs];
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k) raw[k] = ip[min(lane + k * kWave, last_id)];
  int se[CS];
  long long sp[CS];
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int s = min(lane + c * kWave, S - 1);
    se[c] = a.slot_expert[s];
    sp[c] = a.slot_stamp[s];
  }
  int tv[TQ];
  if constexpr (!GLOBAL_E) {
#pragma unroll
    for (int u = 0; u < TQ; ++u) tv[u] = a.table[min(lane + u * kWave, E - 1)];
  }
  unsigned char* flag;
  if constexpr (GLOBAL_E)
    flag = a.routed;
  else
    flag = L.flag;

  // clears: 16 bytes per lane per store (E <= 4096 and S <= 1024 stay inside the arrays)
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  if constexpr (GLOBAL_E) {
    for (int e = lane; e < E; e += kWave) flag[e] = 0;
  } else {
    for (int i = lane * 16; i < E; i += kWave * 16)
      *reinterpret_cast<u32x4*>(&L.flag[i]) = u32x4{0, 0, 0, 0};
  }
  for (int i = lane * 16; i < S; i += kWave * 16)
    *reinterpret_cast<u32x4*>(&L.hit[i]) = u32x4{0, 0, 0, 0};
  step_sync<GLOBAL_E>();

  // ---- routed flags (ids outside [0,E) are padding; int64 ids truncate like .to(int32))
  // The sentinels for lanes past mk / S are applied only now, after the first fence, so
  // that fence does not wait for the loads.
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k)
    idv[k] = (mk > 0 && lane + k * kWave < mk) ? (long long)raw[k] : -1;
#pragma unroll
  for (int c = 0; c < CS; ++c)
    if (lane + c * kWave >= S) se[c] = -1;
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
    // entries past E (below 512) are written too: nothing reads them
#pragma unroll
    for (int u = 0; u < TQ; ++u) L.tab[lane + u * kWave] = tv[u];
    for (int base = TQ * kWave; base < E; base += kTabRegs * kWave) {
      int tw[kTabRegs];
#pragma unroll
      for (int u = 0; u < kTabRegs; ++u) tw[u] = a.table[min(base + lane + u * kWave, E - 1)];
#pragma unroll
      for (int u = 0; u < kTabRegs; ++u) {
        const int e = base + lane + u * kWave;
        if (e < E) L.tab[e] = tw[u];
      }
    }
  }
  step_sync<GLOBAL_E>();

  // ---- distinct count (the caller's `routed` is left holding the flags), then hits mark
  // ---- their slot and misses enumerate in ascending expert id ------------------------
  int cnt = 0, total = 0;
  if (!GLOBAL_E && E <= TQ * kWave) {
    // the whole table is in registers: one batch of flag reads, no table re-read; chunks
    // past E are skipped on a uniform branch
    const int nchunk = (E + kWave - 1) / kWave;
    unsigned char fb[TQ];
    bool fl[TQ];
#pragma unroll
    for (int u = 0; u < TQ; ++u) fb[u] = flag[min(lane + u * kWave, E - 1)];
#pragma unroll
    for (int u = 0; u < TQ; ++u) fl[u] = (fb[u] != 0) & (lane + u * kWave < E);
#pragma unroll
    for (int u = 0; u < TQ; ++u) {
      if (u < nchunk) {
        // lanes past E store routed[E-1]'s own flag there: no store needs a branch
        a.routed[min(lane + u * kWave, E - 1)] = fb[u] != 0 ? 1 : 0;
        cnt += __popcll(__ballot(fl[u]));
      }
    }
    if (cnt > a.max_distinct) {  // wide step: read through, nothing else changes
      if (lane == 0) {
        if constexpr (!PF) a.step[0] = st_v + 1;
        a.n_miss[0] = 0;
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < TQ; ++u) {
      if (u < nchunk) {
        const int e = lane + u * kWave;
        const int t = tv[u];
        if (!PF && fl[u] && t >= 0 && t < S) L.hit[t] = 1;
        const bool m = fl[u] && t < 0;
        const unsigned long long mask = __ballot(m);
        const int j = total + __popcll(mask & lanes_below());
        if (m && j < a.max_inserts) L.mis[j] = e;
        total += __popcll(mask);
      }
    }
  } else {
    for (int base = 0; base < E; base += kWave) {
      const int e = base + lane;
      const bool f = e < E && flag[e];
      if constexpr (!GLOBAL_E) {
        if (e < E) a.routed[e] = f ? 1 : 0;
      }
      cnt += __popcll(__ballot(f));
    }
    if (cnt > a.max_distinct) {
      if (lane == 0) {
        if constexpr (!PF) a.step[0] = st_v + 1;
        a.n_miss[0] = 0;
      }
      return;
    }
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
      if (!PF && f && t >= 0 && t < S) L.hit[t] = 1;
      const bool m = f && t < 0;
      const unsigned long long mask = __ballot(m);
      const int j = total + __popcll(mask & lanes_below());
      if (m && j < a.max_inserts) L.mis[j] = e;
      total += __popcll(mask);
    }
  }
  const int nins = min(total, a.max_inserts);
  lds_sync();

  // ---- slot side: refreshed stamps, whether each slot's expert is routed, and pending
  // ---- prefetch installs confirmed or dropped -----------------------------------------
  const long long st = uniform_i64(st_v) + 1;
  const bool lru = a.policy == 0;
  const long long fresh = PF ? -1 : lru ? st : 1;
  bool fx[CS];
  // all flag reads first, with clamped indexes, so they are in flight together (a
  // short-circuit test would put each read behind its own branch and wait)
  unsigned char hv[CS], fv[CS];
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    hv[c] = L.hit[min(lane + c * kWave, S - 1)];
    fv[c] = flag[min(max(se[c], 0), E - 1)];
  }
  int sign = 0;  // the OR of the stamps' high words: negative iff a stamp is
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int x = se[c];
    fx[c] = (x >= 0) & (x < E) & (fv[c] != 0);
    sign |= (int)((unsigned long long)sp[c] >> 32);
  }
  const bool ageing = !PF && !lru && nins > 0 && a.decay > 0 && (st % (long long)a.decay) == 0;
  // Pending prefetch installs (negative stamps; none on the reference's states) are
  // settled first, behind one wave-uniform branch, one slot per lane and iteration through
  // LDS so the code stays small whatever the slots per lane. An unrouted one is dropped; a
  // routed one is handed to the hit refresh below at the stamp that makes it end the step
  // at an install's stamp: 0 (+1 = 1 under LFU; st under LRU), or 1 when this step ages
  // (+1, halved = 1).
  if (!PF && __ballot(sign < 0) != 0) {
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      const int s = lane + c * kWave;
      if (s < S) {
        L.key[s] = sp[c];
        L.rank[s] = se[c];
      }
    }
    lds_sync();
#pragma unroll 1
    for (int s = lane; s < S; s += kWave) {
      const int x = L.rank[s];
      if (L.key[s] < 0 && x >= 0 && x < E) {
        if (flag[x]) {
          L.key[s] = ageing ? 1 : 0;
          L.hit[s] = 1;
        } else {  // distinct slots hold distinct experts: no write conflicts
          a.table[x] = -1;
          a.map_cold[x] = x;
          if constexpr (!GLOBAL_E) L.tab[x] = -1;
          L.rank[s] = -1;
          L.key[s] = 0;
          if (nins == 0) {
            a.slot_expert[s] = -1;
            a.slot_stamp[s] = 0;
          }
        }
      }
    }
    lds_sync();
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      const int s = min(lane + c * kWave, S - 1);
      sp[c] = L.key[s];
      se[c] = lane + c * kWave < S ? L.rank[s] : -1;
      hv[c] = L.hit[s];
    }
  }
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int s = lane + c * kWave;
    const bool hit = !PF && (s < S) & (hv[c] != 0);
    if (hit) sp[c] = lru ? st : (long long)((unsigned long long)sp[c] + 1ull);
    if (nins == 0 && hit) a.slot_stamp[s] = sp[c];
  }
  if (nins == 0) {  // no inserts: refreshed stamps only, no ageing
    if (lane == 0) {
      if constexpr (!PF) a.step[0] = st;
      a.n_miss[0] = 0;
    }
    return;
  }

  // LFU ageing on inserting steps where st % decay == 0
  if (ageing) {
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
    ev[c] = s < S && !fx[c];
    key[c] = victim_key(sp[c], s);
    nev += __popcll(__ballot(ev[c]));
  }
  const int nact = min(nins, nev);

  if (use_argmin<CS>(nact, nev)) {
    // ---- few inserts: repeated wave-min, each insert installed as soon as it is found.
    // The victim's old expert comes from its owner lane's register, the insert r-th miss
    // from lane r's copy of the miss list.
    const int my_mis = L.mis[min(lane, nins - 1)];
    for (int r = 0; r < nact; ++r) {
      long long m = kKeyMax;
#pragma unroll
      for (int c = 0; c < CS; ++c)
        if (ev[c] && key[c] < m) m = key[c];
      m = wave_min_i64(m);
      const int sl = (int)(m & kSlotMask);
      const int csl = sl >> 6, lsl = sl & (kWave - 1);
      const int e = __builtin_amdgcn_readlane(my_mis, r);
      int old = -1;
#pragma unroll
      for (int c = 0; c < CS; ++c)
        if (c == csl) old = __builtin_amdgcn_readlane(se[c], lsl);
#pragma unroll
      for (int c = 0; c < CS; ++c)
        if (c == csl && lane == lsl) {
          ev[c] = false;
          se[c] = e;
          sp[c] = fresh;
        }
      if (lane == 0) {
        if (old >= 0 && old < E) {
          a.table[old] = -1;
          a.map_cold[old] = old;
          if constexpr (!GLOBAL_E) L.tab[old] = -1;
        }
        a.table[e] = sl;
        a.map_cold[e] = -1;
        a.miss[2 * r + 1] = sl;
        if constexpr (!GLOBAL_E) L.tab[e] = sl;
      }
    }
  } else {
    // ---- many inserts: threshold select. With h = key >> 20 (the stamp bits), sigma is
    // ---- the smallest h such that at least nact evictable keys have h <= sigma, found by
    // ---- binary search with one ballot count per register chunk per probe. Every
    // ---- evictable key below bucket sigma is a victim; the rest of the nact come from
    // ---- bucket sigma in slot order (= key order within a bucket). Each lane then installs
    // ---- its own victims from registers (distinct slots, distinct experts, disjoint table
    // ---- entries, so the installs need no ordering among themselves).
    long long kmin = kKeyMax, nmax = kKeyMax;  // smallest key, and ~largest key
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      if (ev[c] && key[c] < kmin) kmin = key[c];
      if (ev[c] && ~key[c] < nmax) nmax = ~key[c];
    }
    const long long hmin = wave_min_i64(kmin) >> kSlotBits;
    const long long hmax = (~wave_min_i64(nmax)) >> kSlotBits;
    long long sigma;
    if ((unsigned long long)(hmax - hmin) < (1ull << 31)) {
      // stamp spreads below 2^31: 32-bit compares on h - hmin (non-evictable: all ones)
      unsigned rel[CS];
#pragma unroll
      for (int c = 0; c < CS; ++c)
        rel[c] = ev[c] ? (unsigned)((key[c] >> kSlotBits) - hmin) : 0xFFFFFFFFu;
      unsigned lo = 0, hi = (unsigned)(hmax - hmin);
      while (lo < hi) {
        const unsigned mid = (lo + hi) >> 1;
        int n = 0;
#pragma unroll
        for (int c = 0; c < CS; ++c) n += __popcll(__ballot(rel[c] <= mid));
        if (n >= nact)
          hi = mid;
        else
          lo = mid + 1;
      }
      sigma = hmin + (long long)lo;
    } else {
      long long lo = hmin, hi = hmax;
      while (lo < hi) {
        const long long mid = lo + ((hi - lo) >> 1);
        int n = 0;
#pragma unroll
        for (int c = 0; c < CS; ++c) n += __popcll(__ballot(ev[c] && (key[c] >> kSlotBits) <= mid));
        if (n >= nact)
          hi = mid;
        else
          lo = mid + 1;
      }
      sigma = lo;
    }

    // victims: below bucket sigma, or in it among the first `need` by slot
    bool below[CS], inb[CS];
    int nbelow = 0;
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      const long long h = key[c] >> kSlotBits;
      below[c] = ev[c] && h < sigma;
      inb[c] = ev[c] && h == sigma;
      nbelow += __popcll(__ballot(below[c]));
    }
    const int need = nact - nbelow;
    int pos[CS];  // insert index of each victim, or -1
    int seen_b = 0, seen_in = 0;
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      const unsigned long long mb = __ballot(below[c]), mi = __ballot(inb[c]);
      const int rb = seen_b + __popcll(mb & lanes_below());
      const int ri = seen_in + __popcll(mi & lanes_below());
      pos[c] = inb[c] && ri < need ? nbelow + ri : -1;
      if (below[c]) {
        L.key[rb] = key[c];
        pos[c] = rb;  // compaction index until ranked
      }
      seen_b += __popcll(mb);
      seen_in += __popcll(mi);
    }
    if (nbelow > 0) {
      // victims below the bucket take inserts 0..nbelow-1 in key order: rank each among
      // them (every lane reads the same keys, an LDS broadcast, 8 per batch)
      const int n8 = (nbelow + 7) & ~7;
      if (lane < n8 - nbelow) L.key[nbelow + lane] = kKeyMax;
      lds_sync();
      typedef long long i64x2 __attribute__((ext_vector_type(2)));
      const i64x2* kp = reinterpret_cast<const i64x2*>(L.key);
      for (int j0 = 0; j0 < nbelow; j0 += kWave) {
        const int j = j0 + lane;
        const long long kj = L.key[min(j, n8 - 1)];
        int rank = 0;
        for (int i = 0; i < n8; i += 8) {
          const i64x2 k01 = kp[i / 2], k23 = kp[i / 2 + 1], k45 = kp[i / 2 + 2],
                      k67 = kp[i / 2 + 3];
          rank += (k01.x < kj) + (k01.y < kj) + (k23.x < kj) + (k23.y < kj) + (k45.x < kj) +
                  (k45.y < kj) + (k67.x < kj) + (k67.y < kj);
        }
        if (j < nbelow) L.rank[j] = rank;
      }
      lds_sync();
#pragma unroll
      for (int c = 0; c < CS; ++c)
        if (below[c]) pos[c] = L.rank[pos[c]];
    }

    // installs, each by the lane holding the victim slot
    int ne[CS];
#pragma unroll
    for (int c = 0; c < CS; ++c) ne[c] = L.mis[max(pos[c], 0)];
#pragma unroll
    for (int c = 0; c < CS; ++c) {
      if (pos[c] >= 0) {
        const int s = lane + c * kWave;
        const int old = se[c], e = ne[c];
        if (old >= 0 && old < E) {
          a.table[old] = -1;
          a.map_cold[old] = old;
          if constexpr (!GLOBAL_E) L.tab[old] = -1;
        }
        a.table[e] = s;
        a.map_cold[e] = -1;
        a.miss[2 * pos[c] + 1] = s;
        if constexpr (!GLOBAL_E) L.tab[e] = s;
        se[c] = e;
        sp[c] = fresh;
      }
    }
  }
  step_sync<GLOBAL_E>();

  // the caller's miss list gets every counted miss id (miss[2j], j < nins), also past nact
  for (int j = lane; j < nins; j += kWave) a.miss[2 * j] = L.mis[j];
#pragma unroll
  for (int c = 0; c < CS; ++c) {
    const int s = lane + c * kWave;
    if (s < S) {
      a.slot_expert[s] = se[c];
      a.slot_stamp[s] = sp[c];
    }
  }
  if (lane == 0) {
    if constexpr (!PF) a.step[0] = st;
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

// Makes every kernel argument live in SGPRs at this point, so the compiler issues all the
// argument loads together (one round trip) instead of sinking some into later branches.
__device__ __forceinline__ void args_in_sgprs(const ManageArgs& a) {
  asm volatile("" ::"s"(a.ids), "s"(a.table), "s"(a.map_cold), "s"(a.slot_expert),
               "s"(a.slot_stamp), "s"(a.routed), "s"(a.step), "s"(a.miss), "s"(a.n_miss),
               "s"(a.out), "s"(a.mk), "s"(a.E), "s"(a.S), "s"(a.max_distinct),
               "s"(a.max_inserts), "s"(a.policy), "s"(a.decay));
}

template <int CS, bool GLOBAL_E, int IDB, bool REMAP, int TQ>
__global__ __launch_bounds__(kWave) void manage_k(ManageArgs a) {
  __shared__ ManageLds<GLOBAL_E> L;
  args_in_sgprs(a);
  long long idv[kIdRegs];
  manage_step<CS, GLOBAL_E, IDB, TQ>(a, L, idv);
  if constexpr (REMAP) {
    if constexpr (GLOBAL_E) mem_sync();
    else lds_sync();
    remap_tail<GLOBAL_E, IDB>(a, L, idv);
  }
}

// The prefetch step (manage_step with PF) for int32 predicted ids.
template <int CS, bool GLOBAL_E, int TQ>
__global__ __launch_bounds__(kWave) void prefetch_k(ManageArgs a) {
  __shared__ ManageLds<GLOBAL_E> L;
  args_in_sgprs(a);
  long long idv[kIdRegs];
  manage_step<CS, GLOBAL_E, 4, TQ, true>(a, L, idv);
}

// Two workgroups, two layers: workgroup 0 runs layer a's policy step and remap (manage_k
// with REMAP), workgroup 1 the prefetch step of another layer p (prefetch_k). The host
// rejects states that share arrays, so the workgroups touch disjoint memory and need no
// ordering between them; the pair occupies one node of the stream instead of two.
template <int CS, bool GLOBAL_E, int IDB, int TQ>
__global__ __launch_bounds__(kWave) void manage_prefetch_k(ManageArgs a, ManageArgs p) {
  __shared__ ManageLds<GLOBAL_E> L;
  long long idv[kIdRegs];
  if (blockIdx.x == 0) {
    args_in_sgprs(a);
    manage_step<CS, GLOBAL_E, IDB, TQ>(a, L, idv);
    if constexpr (GLOBAL_E) mem_sync();
    else lds_sync();
    remap_tail<GLOBAL_E, IDB>(a, L, idv);
  } else {
    args_in_sgprs(p);
    manage_step<CS, GLOBAL_E, 4, TQ, true>(p, L, idv);
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
