// expert_cache_fused on gfx950: the LRU policy step followed by both moe_align_block_size
// outputs, in one wavefront (kernels/expert_cache.hip:431-588 semantics).
//
// The policy half is manage_step with policy 0 and no decay (a hit and an install both stamp
// the current step). The align half buckets every routing id against the updated table --
// resident ids by slot ("hot"), the rest by expert id ("cold") -- pads each bucket to a
// multiple of the block size, scans, and places each id at its bucket offset plus its rank
// among the earlier ids of the same bucket, so the output is in token order within every
// bucket for every mk (the reference is token-ordered for mk <= 256 and unordered above).
// Below each side's padded total the outputs are built in LDS (padding, block expert ids,
// then the placed ids) and copied out with coalesced stores; past it the defaults go
// straight to memory. No output position is written twice, so no fence is needed; outputs
// too large for LDS are filled with their defaults in memory first and fenced.
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

// Per side, the ids and block expert ids below the padded total are built in LDS and
// copied out once when they fit in kStage ints (decode and chunked-prefill shapes).
constexpr int kStage = 10240;

struct AlignLds {
  int cur_h[kMaxSlots + 1];          // counts, then placement cursors, per slot bucket
  int cur_c[kMaxAlignExperts + 1];   // same per expert bucket
  unsigned long long lanes[kMaxSlots + kMaxAlignExperts];  // per bucket key: lanes of a block
  alignas(16) int stage[2][kStage];  // per side: sorted, then expert ids from round4(n)
};

// Combined bucket key of one routing id: slot s (hot), kMaxSlots + e (cold), -1 (skipped).
__device__ __forceinline__ int align_key(int e, int E, int S, const int* tab) {
  if (e < 0 || e >= E) return -1;
  const int s = tab[e];
  return ((unsigned)s < (unsigned)S) ? s : kMaxSlots + e;
}

// x / bs for the wave-uniform block size: a shift for powers of two (vLLM's block sizes).
struct BlockDiv {
  int bs, shift;
  __device__ __forceinline__ explicit BlockDiv(int b)
      : bs(b), shift((b & (b - 1)) == 0 ? __builtin_ctz((unsigned)b) : -1) {}
  __device__ __forceinline__ int div(int x) const { return shift >= 0 ? x >> shift : x / bs; }
  __device__ __forceinline__ int pad(int x) const { return div(x + bs - 1) * bs; }
};

// Exclusive scan of block-padded counts, 64 buckets per chunk (bucket c*64 + lane in chunk
// c), kept in registers: ex[c] is the bucket's first position, pc[c] its padded count.
// Returns the padded total. NC chunks cover nb buckets; chunks past nb are skipped on a
// uniform branch. The count reads of every chunk are issued before the first scan.
template <int NC>
__device__ __forceinline__ int padded_scan(const int* cnt, int nb, BlockDiv d, int (&ex)[NC],
                                           int (&pc)[NC]) {
  const int lane = __lane_id();
  int raw[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) raw[c] = cnt[min(c * kWave + lane, nb - 1)];
  int run = 0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    pc[c] = c * kWave + lane < nb ? d.pad(raw[c]) : 0;
    ex[c] = run;
    if (c * kWave < nb) {
      const int incl = wave_incl_scan(pc[c]);
      ex[c] = run + incl - pc[c];
      run += __builtin_amdgcn_readlane(incl, kWave - 1);
    }
  }
  return run;
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// dst[from, to) = v over the wave; 16-byte stores when dst is 16-byte aligned.
__device__ __forceinline__ void fill_i32(int* dst, int from, int to, int v) {
  const int lane = __lane_id();
  if (from >= to) return;
  if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    const int a0 = min((from + 3) & ~3, to);
    const int a1 = a0 + ((to - a0) & ~3);
    if (from + lane < a0) dst[from + lane] = v;
    for (int p = a0 + 4 * lane; p < a1; p += 4 * kWave)
      *reinterpret_cast<i32x4*>(dst + p) = i32x4{v, v, v, v};
    if (a1 + lane < to) dst[a1 + lane] = v;
  } else {
    for (int p = from + lane; p < to; p += kWave) dst[p] = v;
  }
}

// dst[0, n) = src[0, n) from 16-byte aligned LDS; 16-byte stores when dst is aligned.
__device__ __forceinline__ void copy_out(int* dst, const int* src, int n) {
  const int lane = __lane_id();
  if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    const int n4 = n & ~3;
    for (int p = 4 * lane; p < n4; p += 4 * kWave)
      *reinterpret_cast<i32x4*>(dst + p) = *reinterpret_cast<const i32x4*>(src + p);
    if (n4 + lane < n) dst[n4 + lane] = src[n4 + lane];
  } else {
    for (int p = lane; p < n; p += kWave) dst[p] = src[p];
  }
}

// Expert id of every block of every non-empty bucket, from the scan held in registers.
template <int NC>
__device__ __forceinline__ void fill_eids(const int (&ex)[NC], const int (&pc)[NC], int nb,
                                          BlockDiv d, int NB, int* eids) {
  const int lane = __lane_id();
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int b = c * kWave + lane;
    if (b < nb) {
      const int q1 = min(d.div(ex[c] + pc[c]), NB);
      for (int q = d.div(ex[c]); q < q1; ++q) eids[q] = b;
    }
  }
}

// Places the ids of one block of 64 (lane -> id i, bucket key kk or -1) at their bucket's
// cursor plus their rank among the earlier ids of the same bucket in the block, so every
// bucket is in token order. The lanes sharing a bucket are found by an atomic OR of lane
// bits into the bucket's mask (order-free, so deterministic; every mask starts the block at
// zero); a lane's rank is the popcount of the mask below it. The bucket's last lane moves
// the cursor and clears the mask for the next block.
__device__ __forceinline__ void place_block(const AlignArgs& g, AlignLds& A, int kk, int i,
                                            int* sorted_hot, int* sorted_cold) {
  const int lane = __lane_id();
  if (kk >= 0) atomicOr(&A.lanes[kk], 1ull << lane);
  lds_sync();
  const int kc = kk < 0 ? 0 : kk;
  int* cur = kc >= kMaxSlots ? &A.cur_c[kc - kMaxSlots] : &A.cur_h[kc];
  const unsigned long long m = A.lanes[kc];
  const int c0 = *cur;
  if (kk >= 0) {
    const int pos = c0 + __popcll(m & lanes_below());
    int* sorted = kk >= kMaxSlots ? sorted_cold : sorted_hot;
    if (pos < g.L) sorted[pos] = i;
    if ((m >> lane) == 1ull) {
      *cur = c0 + __popcll(m);
      A.lanes[kc] = 0ull;
    }
  }
  lds_sync();
}

// Every id in token order: the first kIdRegs blocks from the keys held in registers, the
// rest from memory.
__device__ __forceinline__ void place_ids(const ManageArgs& a, const AlignArgs& g,
                                          const ManageLds<false>& L, AlignLds& A,
                                          const int (&key)[kIdRegs], int* sorted_hot,
                                          int* sorted_cold) {
  const int lane = __lane_id();
  const int mk = a.mk;
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k)
    if (k * kWave < mk) place_block(g, A, key[k], lane + k * kWave, sorted_hot, sorted_cold);
  const int* ids = reinterpret_cast<const int*>(a.ids);
  for (int base = kIdRegs * kWave; base < mk; base += kWave) {
    const int i = base + lane;
    const int kk = i < mk ? align_key(ids[i], a.E, a.S, L.tab) : -1;
    place_block(g, A, kk, i, sorted_hot, sorted_cold);
  }
}

template <int CS, int TQ>
__device__ __forceinline__ void align_tail(const ManageArgs& a, const AlignArgs& g,
                                           const ManageLds<false>& L, AlignLds& A,
                                           const long long (&idv)[kIdRegs]) {
  // chunks of 64 buckets per side: the slots per lane cover S; the table chunks cover E up
  // to 512, and 16 chunks cover the rest (E <= kMaxAlignExperts)
  constexpr int CC = TQ == kTabRegs ? kMaxAlignExperts / kWave : TQ;
  const int lane = __lane_id();
  const int E = a.E, S = a.S, mk = a.mk;
  const BlockDiv d(g.bs);
  const int* ids = reinterpret_cast<const int*>(a.ids);

  // bucket key of every id held in registers (the table lookups issued together)
  int key[kIdRegs];
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k)
    key[k] = lane + k * kWave < mk ? align_key((int)idv[k], E, S, L.tab) : -1;
  for (int b = lane; b < S; b += kWave) A.cur_h[b] = 0;
  for (int b = lane; b < E; b += kWave) A.cur_c[b] = 0;
  lds_sync();
  // counts per bucket; each used bucket's lane mask starts at zero for the placement
#pragma unroll
  for (int k = 0; k < kIdRegs; ++k) {
    const int kk = key[k];
    if (kk >= kMaxSlots)
      atomicAdd(&A.cur_c[kk - kMaxSlots], 1);
    else if (kk >= 0)
      atomicAdd(&A.cur_h[kk], 1);
    if (kk >= 0) A.lanes[kk] = 0ull;
  }
  for (int i = lane + kIdRegs * kWave; i < mk; i += kWave) {
    const int kk = align_key(ids[i], E, S, L.tab);
    if (kk >= kMaxSlots)
      atomicAdd(&A.cur_c[kk - kMaxSlots], 1);
    else if (kk >= 0)
      atomicAdd(&A.cur_h[kk], 1);
    if (kk >= 0) A.lanes[kk] = 0ull;
  }
  lds_sync();
  int exh[CS], pch[CS], exc[CC], pcc[CC];
  const int tot_h = padded_scan(A.cur_h, S, d, exh, pch);
  const int tot_c = padded_scan(A.cur_c, E, d, exc, pcc);
  if (lane == 0) {
    g.npad_hot[0] = tot_h;
    g.npad_cold[0] = tot_c;
  }
  // placement cursors start at each bucket's first position (the counts were read above)
#pragma unroll
  for (int c = 0; c < CS; ++c)
    if (c * kWave + lane < S) A.cur_h[c * kWave + lane] = exh[c];
#pragma unroll
  for (int c = 0; c < CC; ++c)
    if (c * kWave + lane < E) A.cur_c[c * kWave + lane] = exc[c];

  // Every position below a side's padded total is an id or its bucket's padding, every
  // block below it belongs to a bucket; past it the outputs hold mk and -1.
  const int nh = min(tot_h, g.L), nc = min(tot_c, g.L);
  const int qh = min(d.div(tot_h), g.NB), qc = min(d.div(tot_c), g.NB);
  const int oh = (nh + 3) & ~3, oc = (nc + 3) & ~3;
  if (oh + qh <= kStage && oc + qc <= kStage) {
    int* sh = A.stage[0];
    int* sc = A.stage[1];
    fill_i32(sh, 0, nh, mk);
    fill_i32(sc, 0, nc, mk);
    fill_eids(exh, pch, S, d, g.NB, sh + oh);
    fill_eids(exc, pcc, E, d, g.NB, sc + oc);
    fill_i32(g.sorted_hot, nh, g.L, mk);
    fill_i32(g.sorted_cold, nc, g.L, mk);
    fill_i32(g.eids_hot, qh, g.NB, -1);
    fill_i32(g.eids_cold, qc, g.NB, -1);
    lds_sync();
    place_ids(a, g, L, A, key, sh, sc);  // ends with an LDS sync
    copy_out(g.sorted_hot, sh, nh);
    copy_out(g.eids_hot, sh + oh, qh);
    copy_out(g.sorted_cold, sc, nc);
    copy_out(g.eids_cold, sc + oc, qc);
  } else {
    fill_i32(g.sorted_hot, 0, g.L, mk);
    fill_i32(g.eids_hot, 0, g.NB, -1);
    fill_i32(g.sorted_cold, 0, g.L, mk);
    fill_i32(g.eids_cold, 0, g.NB, -1);
    mem_sync();  // the defaults are written before any entry below lands on them
    fill_eids(exh, pch, S, d, g.NB, g.eids_hot);
    fill_eids(exc, pcc, E, d, g.NB, g.eids_cold);
    place_ids(a, g, L, A, key, g.sorted_hot, g.sorted_cold);
  }
}

template <int CS, int TQ>
__global__ __launch_bounds__(kWave) void fused_k(ManageArgs a, AlignArgs g) {
  __shared__ ManageLds<false> L;
  __shared__ AlignLds A;
  args_in_sgprs(a);
  long long idv[kIdRegs];
  manage_step<CS, false, 4, TQ>(a, L, idv);
  lds_sync();
  align_tail<CS, TQ>(a, g, L, A, idv);
}

}  // namespace ec
