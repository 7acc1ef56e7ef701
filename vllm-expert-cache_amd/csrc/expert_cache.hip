// libexpertcache.so: C-ABI entry points (declared in include/expert_cache.h).
//
// Argument checks run on the host before any HIP call and return -1, exactly where the
// reference's C-ABI does (kernels/expert_cache.hip:596-598, :616-618, :631-634); otherwise
// each entry point launches one kernel on the caller's stream and returns hipGetLastError().
// The library keeps no state and allocates nothing.
#include <hip/hip_runtime.h>

#include "../../include/expert_cache.h"
#include "align.h"
#include "gather.h"
#include "manage.h"

namespace ec {
namespace {

// [p, p + pn) and [q, q + qn) share a byte
bool ranges_meet(const void* p, long long pn, const void* q, long long qn) {
  const long long a = (long long)reinterpret_cast<uintptr_t>(p);
  const long long b = (long long)reinterpret_cast<uintptr_t>(q);
  return pn > 0 && qn > 0 && a < b + qn && b < a + pn;
}

bool manage_args_bad(int E, int S, int max_inserts, int policy) {
  if (E <= 0 || S <= 0 || S > kMaxSlots || S > kSlotMask) return true;
  if (max_inserts < 0 || max_inserts > kMaxInserts) return true;
  if (policy < 0 || policy > 1) return true;
  return false;
}

// Slots per lane (CS) by S, and table chunks held in registers (TQ) by E.
template <int IDB, bool REMAP, int TQ>
int launch_manage_tq(const ManageArgs& a, hipStream_t stream) {
  const dim3 grid(1), block(kWave);
  if (a.S <= 64) {
    hipLaunchKernelGGL((manage_k<1, false, IDB, REMAP, TQ>), grid, block, 0, stream, a);
  } else if (a.S <= 128) {
    hipLaunchKernelGGL((manage_k<2, false, IDB, REMAP, TQ>), grid, block, 0, stream, a);
  } else if (a.S <= 256) {
    hipLaunchKernelGGL((manage_k<4, false, IDB, REMAP, TQ>), grid, block, 0, stream, a);
  } else if (a.S <= 512) {
    hipLaunchKernelGGL((manage_k<8, false, IDB, REMAP, TQ>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((manage_k<16, false, IDB, REMAP, TQ>), grid, block, 0, stream, a);
  }
  return (int)hipGetLastError();
}

template <int IDB, bool REMAP>
int launch_manage(const ManageArgs& a, hipStream_t stream) {
  if (a.E > kLdsExperts) {
    hipLaunchKernelGGL((manage_k<16, true, IDB, REMAP, kTabRegs>), dim3(1), dim3(kWave), 0,
                       stream, a);
    return (int)hipGetLastError();
  }
  switch (table_chunks(a.E)) {
    case 1: return launch_manage_tq<IDB, REMAP, 1>(a, stream);
    case 2: return launch_manage_tq<IDB, REMAP, 2>(a, stream);
    case 4: return launch_manage_tq<IDB, REMAP, 4>(a, stream);
    default: return launch_manage_tq<IDB, REMAP, kTabRegs>(a, stream);
  }
}

template <int TQ>
int launch_prefetch_tq(const ManageArgs& a, hipStream_t stream) {
  const dim3 grid(1), block(kWave);
  if (a.S <= 64)
    hipLaunchKernelGGL((prefetch_k<1, false, TQ>), grid, block, 0, stream, a);
  else if (a.S <= 128)
    hipLaunchKernelGGL((prefetch_k<2, false, TQ>), grid, block, 0, stream, a);
  else if (a.S <= 256)
    hipLaunchKernelGGL((prefetch_k<4, false, TQ>), grid, block, 0, stream, a);
  else if (a.S <= 512)
    hipLaunchKernelGGL((prefetch_k<8, false, TQ>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((prefetch_k<16, false, TQ>), grid, block, 0, stream, a);
  return (int)hipGetLastError();
}

int launch_prefetch(const ManageArgs& a, hipStream_t stream) {
  if (a.E > kLdsExperts) {
    hipLaunchKernelGGL((prefetch_k<16, true, kTabRegs>), dim3(1), dim3(kWave), 0, stream, a);
    return (int)hipGetLastError();
  }
  switch (table_chunks(a.E)) {
    case 1: return launch_prefetch_tq<1>(a, stream);
    case 2: return launch_prefetch_tq<2>(a, stream);
    case 4: return launch_prefetch_tq<4>(a, stream);
    default: return launch_prefetch_tq<kTabRegs>(a, stream);
  }
}

// Both layers share E and S, so one variant serves the two workgroups.
template <int IDB, int TQ>
int launch_manage_prefetch_tq(const ManageArgs& a, const ManageArgs& p, hipStream_t stream) {
  const dim3 grid(2), block(kWave);
  if (a.S <= 64)
    hipLaunchKernelGGL((manage_prefetch_k<1, false, IDB, TQ>), grid, block, 0, stream, a, p);
  else if (a.S <= 128)
    hipLaunchKernelGGL((manage_prefetch_k<2, false, IDB, TQ>), grid, block, 0, stream, a, p);
  else if (a.S <= 256)
    hipLaunchKernelGGL((manage_prefetch_k<4, false, IDB, TQ>), grid, block, 0, stream, a, p);
  else if (a.S <= 512)
    hipLaunchKernelGGL((manage_prefetch_k<8, false, IDB, TQ>), grid, block, 0, stream, a, p);
  else
    hipLaunchKernelGGL((manage_prefetch_k<16, false, IDB, TQ>), grid, block, 0, stream, a, p);
  return (int)hipGetLastError();
}

template <int IDB>
int launch_manage_prefetch(const ManageArgs& a, const ManageArgs& p, hipStream_t stream) {
  if (a.E > kLdsExperts) {
    hipLaunchKernelGGL((manage_prefetch_k<16, true, IDB, kTabRegs>), dim3(2), dim3(kWave), 0,
                       stream, a, p);
    return (int)hipGetLastError();
  }
  switch (table_chunks(a.E)) {
    case 1: return launch_manage_prefetch_tq<IDB, 1>(a, p, stream);
    case 2: return launch_manage_prefetch_tq<IDB, 2>(a, p, stream);
    case 4: return launch_manage_prefetch_tq<IDB, 4>(a, p, stream);
    default: return launch_manage_prefetch_tq<IDB, kTabRegs>(a, p, stream);
  }
}

template <int TQ>
int launch_fused_tq(const ManageArgs& a, const AlignArgs& g, hipStream_t stream) {
  const dim3 grid(1), block(kWave);
  if (a.S <= 64)
    hipLaunchKernelGGL((fused_k<1, TQ>), grid, block, 0, stream, a, g);
  else if (a.S <= 128)
    hipLaunchKernelGGL((fused_k<2, TQ>), grid, block, 0, stream, a, g);
  else if (a.S <= 256)
    hipLaunchKernelGGL((fused_k<4, TQ>), grid, block, 0, stream, a, g);
  else if (a.S <= 512)
    hipLaunchKernelGGL((fused_k<8, TQ>), grid, block, 0, stream, a, g);
  else
    hipLaunchKernelGGL((fused_k<16, TQ>), grid, block, 0, stream, a, g);
  return (int)hipGetLastError();
}

int launch_fused(const ManageArgs& a, const AlignArgs& g, hipStream_t stream) {
  switch (table_chunks(a.E)) {
    case 1: return launch_fused_tq<1>(a, g, stream);
    case 2: return launch_fused_tq<2>(a, g, stream);
    case 4: return launch_fused_tq<4>(a, g, stream);
    default: return launch_fused_tq<kTabRegs>(a, g, stream);
  }
}

ManageArgs make_args(const void* ids, int mk, int E, int S, int max_distinct, int max_inserts,
                     int* table, int* map_cold, int* slot_expert, long long* slot_stamp,
                     unsigned char* routed, long long* step, int* miss, int* n_miss,
                     int policy, int decay, void* out) {
  ManageArgs a;
  a.ids = ids;
  a.mk = mk;
  a.E = E;
  a.S = S;
  a.max_distinct = max_distinct;
  a.max_inserts = max_inserts;
  a.table = table;
  a.map_cold = map_cold;
  a.slot_expert = slot_expert;
  a.slot_stamp = slot_stamp;
  a.routed = routed;
  a.step = step;
  a.miss = miss;
  a.n_miss = n_miss;
  a.policy = policy;
  a.decay = decay;
  a.out = out;
  return a;
}

}  // namespace
}  // namespace ec

using namespace ec;

extern "C" {

int expert_cache_manage(const int* topk_ids, int mk, int E, int S, int max_distinct,
                        int max_inserts, int* table, int* map_cold, int* slot_expert,
                        long long* slot_stamp, unsigned char* routed, long long* step,
                        int* miss, int* n_miss, int policy, int decay, hipStream_t stream) {
  if (manage_args_bad(E, S, max_inserts, policy)) return -1;
  const ManageArgs a = make_args(topk_ids, mk, E, S, max_distinct, max_inserts, table, map_cold,
                                 slot_expert, slot_stamp, routed, step, miss, n_miss, policy,
                                 decay, nullptr);
  return launch_manage<4, false>(a, stream);
}

int expert_cache_manage_remap(const void* ids, int id_bytes, int mk, int E, int S,
                              int max_distinct, int max_inserts, int* table, int* map_cold,
                              int* slot_expert, long long* slot_stamp, unsigned char* routed,
                              long long* step, int* miss, int* n_miss, int policy, int decay,
                              void* out, hipStream_t stream) {
  if (manage_args_bad(E, S, max_inserts, policy)) return -1;
  if (id_bytes != 4 && id_bytes != 8) return -1;
  if (mk > 0 && out == nullptr) return -1;
  const ManageArgs a = make_args(ids, mk, E, S, max_distinct, max_inserts, table, map_cold,
                                 slot_expert, slot_stamp, routed, step, miss, n_miss, policy,
                                 decay, out);
  return id_bytes == 8 ? launch_manage<8, true>(a, stream) : launch_manage<4, true>(a, stream);
}

int expert_cache_prefetch(const int* pred_ids, int mk, int E, int S, int max_inserts,
                          int* table, int* map_cold, int* slot_expert, long long* slot_stamp,
                          unsigned char* routed, int* miss, int* n_miss, hipStream_t stream) {
  if (manage_args_bad(E, S, max_inserts, 0) || mk < 0) return -1;
  // max_distinct = E: a prediction never reads through; no step counter is touched
  const ManageArgs a = make_args(pred_ids, mk, E, S, E, max_inserts, table, map_cold,
                                 slot_expert, slot_stamp, routed, nullptr, miss, n_miss, 0, 0,
                                 nullptr);
  return launch_prefetch(a, stream);
}

int expert_cache_manage_remap_prefetch(
    const void* ids, int id_bytes, int mk, int E, int S, int max_distinct, int max_inserts,
    int* table, int* map_cold, int* slot_expert, long long* slot_stamp, unsigned char* routed,
    long long* step, int* miss, int* n_miss, int policy, int decay, void* out,
    const int* pred_ids, int pk, int pf_max_inserts, int* pf_table, int* pf_map_cold,
    int* pf_slot_expert, long long* pf_slot_stamp, unsigned char* pf_routed, int* pf_miss,
    int* pf_n_miss, hipStream_t stream) {
  if (manage_args_bad(E, S, max_inserts, policy)) return -1;
  if (id_bytes != 4 && id_bytes != 8) return -1;
  if (mk > 0 && out == nullptr) return -1;
  if (manage_args_bad(E, S, pf_max_inserts, 0) || pk < 0) return -1;
  // the two workgroups run unordered: the layers must not share any array
  const long long e4 = 4LL * E, s4 = 4LL * S;
  if (ranges_meet(table, e4, pf_table, e4) || ranges_meet(map_cold, e4, pf_map_cold, e4) ||
      ranges_meet(slot_expert, s4, pf_slot_expert, s4) ||
      ranges_meet(slot_stamp, 2 * s4, pf_slot_stamp, 2 * s4) ||
      ranges_meet(routed, E, pf_routed, E) ||
      ranges_meet(miss, 8LL * max_inserts, pf_miss, 8LL * pf_max_inserts) ||
      ranges_meet(n_miss, 4, pf_n_miss, 4))
    return -1;
  const ManageArgs a = make_args(ids, mk, E, S, max_distinct, max_inserts, table, map_cold,
                                 slot_expert, slot_stamp, routed, step, miss, n_miss, policy,
                                 decay, out);
  const ManageArgs p = make_args(pred_ids, pk, E, S, E, pf_max_inserts, pf_table, pf_map_cold,
                                 pf_slot_expert, pf_slot_stamp, pf_routed, nullptr, pf_miss,
                                 pf_n_miss, 0, 0, nullptr);
  return id_bytes == 8 ? launch_manage_prefetch<8>(a, p, stream)
                       : launch_manage_prefetch<4>(a, p, stream);
}

int expert_cache_remap(const void* ids, int n, int id_bytes, const int* table, int E,
                       void* out, hipStream_t stream) {
  if (E <= 0 || n < 0 || (id_bytes != 4 && id_bytes != 8)) return -1;
  if (n == 0) return 0;
  const int blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  if (id_bytes == 8)
    hipLaunchKernelGGL((remap_k<8>), dim3(blocks), dim3(256), 0, stream, ids, n, table, E, out);
  else
    hipLaunchKernelGGL((remap_k<4>), dim3(blocks), dim3(256), 0, stream, ids, n, table, E, out);
  return (int)hipGetLastError();
}

int expert_cache_fused(const int* topk_ids, int mk, int E, int S, int max_distinct,
                       int max_inserts, int* table, int* map_cold, int* slot_expert,
                       long long* slot_stamp, unsigned char* routed, long long* step,
                       int* miss, int* n_miss, int bs, int L, int NB, int* sorted_hot,
                       int* eids_hot, int* npad_hot, int* sorted_cold, int* eids_cold,
                       int* npad_cold, hipStream_t stream) {
  if (E <= 0 || E > kMaxAlignExperts || S <= 0 || S > kMaxSlots || S > kSlotMask) return -1;
  if (bs <= 0 || L <= 0 || NB <= 0 || mk < 0) return -1;
  if (max_inserts < 0 || max_inserts > kMaxAlignExperts) return -1;
  const ManageArgs a = make_args(topk_ids, mk, E, S, max_distinct, max_inserts, table, map_cold,
                                 slot_expert, slot_stamp, routed, step, miss, n_miss, 0, 0,
                                 nullptr);
  AlignArgs g;
  g.bs = bs;
  g.L = L;
  g.NB = NB;
  g.sorted_hot = sorted_hot;
  g.eids_hot = eids_hot;
  g.npad_hot = npad_hot;
  g.sorted_cold = sorted_cold;
  g.eids_cold = eids_cold;
  g.npad_cold = npad_cold;
  return launch_fused(a, g, stream);
}

int expert_cache_gather(void* d0, const void* s0, long b0, void* d1, const void* s1, long b1,
                        void* d2, const void* s2, long b2, void* d3, const void* s3, long b3,
                        void* d4, const void* s4, long b4, void* d5, const void* s5, long b5,
                        const int* miss, const int* n_miss, int chunks, int lanes,
                        hipStream_t stream) {
  void* const dst[kGatherBufs] = {d0, d1, d2, d3, d4, d5};
  const void* const src[kGatherBufs] = {s0, s1, s2, s3, s4, s5};
  const long bytes[kGatherBufs] = {b0, b1, b2, b3, b4, b5};
  GatherArgs g;
  if (n_miss == nullptr || !gather_plan(dst, src, bytes, chunks, lanes, g)) return -1;
  hipLaunchKernelGGL((gather_k<kGatherUnroll, true, false, false>), dim3(chunks, lanes),
                     dim3(kGatherThreads), 0, stream, g, miss, n_miss, nullptr);
  return (int)hipGetLastError();
}

int expert_cache_gather_live(void* d0, const void* s0, long b0, void* d1, const void* s1,
                             long b1, void* d2, const void* s2, long b2, void* d3,
                             const void* s3, long b3, void* d4, const void* s4, long b4,
                             void* d5, const void* s5, long b5, const int* miss,
                             const int* n_miss, const int* slot_expert, int chunks, int lanes,
                             hipStream_t stream) {
  void* const dst[kGatherBufs] = {d0, d1, d2, d3, d4, d5};
  const void* const src[kGatherBufs] = {s0, s1, s2, s3, s4, s5};
  const long bytes[kGatherBufs] = {b0, b1, b2, b3, b4, b5};
  GatherArgs g;
  if (n_miss == nullptr || slot_expert == nullptr) return -1;
  if (!gather_plan(dst, src, bytes, chunks, lanes, g)) return -1;
  hipLaunchKernelGGL((gather_k<kGatherUnroll, true, false, true>), dim3(chunks, lanes),
                     dim3(kGatherThreads), 0, stream, g, miss, n_miss, slot_expert);
  return (int)hipGetLastError();
}

}  // extern "C"
