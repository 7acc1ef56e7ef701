// expert_cache_fused on gfx950: the LRU policy step followed by both moe_align_block_size
// outputs, in one wavefront (kernels/expert_cache.hip:431-588 semantics).
//
// The policy half is manage_step with policy 0 and no decay (a hit and an install both stamp
// the current step). The align half buckets every routing id against the updated table --
// resident ids by slot ("hot"), the rest by expert id ("cold") -- pads each bucket to a
// multiple of the block size, scans, and places each id at its bucket offset plus its rank
// among the earlier ids of the same bucket, so the output is in token order within every
// bucket for every mk (the reference is token-ordered for mk <= 256 and unordered above).
#pragma once
#include "manage.h"

namespace ec {

constexpr int kMaxAlignExperts = 1024;

struct AlignArgs {
  int bs, L, NB;
  int* sorted_hot;
  int* eids_hot;
  int* npad_hot;
  int* sorted_cold;
  int* eids_cold;
  int* npad_cold;
};

struct AlignLds {
  int cur_h[kMaxSlots + 1];          // counts, then placement cursors, per slot bucket
  int cur_c[kMaxAlignExperts + 1];   // same per expert bucket
  int cum_h[kMaxSlots + 1];
  int cum_c[kMaxAlignExperts + 1];
};

// Combined bucket key of one routing id: slot s (hot), kMaxSlots + e (cold), -1 (skipped).
__device__ __forceinline__ int align_key(int e, int E, int S, const int* tab) {
  if (e < 0 || e >= E) return -1;
  const int s = tab[e];
  return ((unsigned)s < (unsigned)S) ? s : kMaxSlots + e;
}

// Exclusive scan of block-padded counts over nb buckets; each lane owns a contiguous run.
__device__ __forceinline__ void padded_scan(const int* cnt, int* cum, int nb, int bs) {
  const int lane = __lane_id();
  const int per = (nb + kWave - 1) / kWave;
  const int lo = min(lane * per, nb), hi = min(lo + per, nb);
  int local = 0;
  for (int b = lo; b < hi; ++b) local += ((cnt[b] + bs - 1) / bs) * bs;
  const int incl = wave_incl_scan(local);
  int run = incl - local;
  for (int b = lo; b < hi; ++b) {
    cum[b] = run;
    run += ((cnt[b] + bs - 1) / bs) * bs;
  }
  if (lane == kWave - 1) cum[nb] = incl;
}

__device__ __forceinline__ void fill_eids(const int* cum, int nb, int bs, int NB, int* eids) {
  for (int b = __lane_id(); b < nb; b += kWave)
    for (int q = cum[b] / bs; q < cum[b + 1] / bs && q < NB; ++q) eids[q] = b;
}

__device__ __forceinline__ void align_tail(const ManageArgs& a, const AlignArgs& g,
                                           const ManageLds<false>& L, AlignLds& A) {
  const int lane = __lane_id();
  const int E = a.E, S = a.S, mk = a.mk, bs = g.bs;
  const int* ids = reinterpret_cast<const int*>(a.ids);

  for (int i = lane; i < g.L; i += kWave) {
    g.sorted_hot[i] = mk;
    g.sorted_cold[i] = mk;
  }
  for (int i = lane; i < g.NB; i += kWave) {
    g.eids_hot[i] = -1;
    g.eids_cold[i] = -1;
  }
  for (int b = lane; b < S; b += kWave) A.cur_h[b] = 0;
  for (int b = lane; b < E; b += kWave) A.cur_c[b] = 0;
  lds_sync();

  for (int i = lane; i < mk; i += kWave) {
    const int k = align_key(ids[i], E, S, L.tab);
    if (k >= kMaxSlots)
      atomicAdd(&A.cur_c[k - kMaxSlots], 1);
    else if (k >= 0)
      atomicAdd(&A.cur_h[k], 1);
  }
  lds_sync();
  padded_scan(A.cur_h, A.cum_h, S, bs);
  padded_scan(A.cur_c, A.cum_c, E, bs);
  lds_sync();
  if (lane == 0) {
    g.npad_hot[0] = A.cum_h[S];
    g.npad_cold[0] = A.cum_c[E];
  }
  for (int b = lane; b < S; b += kWave) A.cur_h[b] = A.cum_h[b];
  for (int b = lane; b < E; b += kWave) A.cur_c[b] = A.cum_c[b];
  mem_sync();  // the defaults above are written before any real entry lands on them

  fill_eids(A.cum_h, S, bs, g.NB, g.eids_hot);
  fill_eids(A.cum_c, E, bs, g.NB, g.eids_cold);

  for (int base = 0; base < mk; base += kWave) {
    const int i = base + lane;
    const int k = i < mk ? align_key(ids[i], E, S, L.tab) : -1;
    int before = 0, after = 0;
    for (int jl = 0; jl < kWave; ++jl) {
      const int kj = wave_lane_value(k, jl);
      before += (kj == k && jl < lane);
      after += (kj == k && jl > lane);
    }
    int* cur = k >= kMaxSlots ? &A.cur_c[k - kMaxSlots] : &A.cur_h[k < 0 ? 0 : k];
    if (k >= 0) {
      const int pos = *cur + before;
      int* sorted = k >= kMaxSlots ? g.sorted_cold : g.sorted_hot;
      if (pos < g.L) sorted[pos] = i;
    }
    lds_sync();
    if (k >= 0 && after == 0) *cur += before + 1;
    lds_sync();
  }
}

template <int CS>
__global__ __launch_bounds__(kWave) void fused_k(ManageArgs a, AlignArgs g) {
  __shared__ ManageLds<false> L;
  __shared__ AlignLds A;
  args_in_sgprs(a);
  long long idv[kIdRegs];
  manage_step<CS, false, 4>(a, L, idv);
  lds_sync();
  align_tail(a, g, L, A);
}

}  // namespace ec
