// bench_stamps.so: the decode chain's two kernels with clock stamps, for bench.py's
// in-chain timing (built by __graft_entry__.build(); not part of libexpertcache.so).
//
// Each stamped kernel runs the product kernel's device code unchanged between two reads of
// the GPU's constant-rate clock (s_memrealtime) -- the first as the kernel's first
// instruction, the second after its own stores have completed (s_waitcnt 0, and for the
// gather a workgroup barrier) -- and writes the pair with vector stores into a row of the
// caller's stamp buffer: row[0] = entry, row[1] = exit. So the bench can read, per launch in
// the decode graph, how long the kernel ran and how long the chain took to start it, with
// no event packets between the nodes and no profiler attached.
//
//   stamped_manage_remap  expert_cache_manage_remap (int32 ids, E <= 4096) + one row
//   stamped_gather        expert_cache_gather + one row per workgroup (chunks x lanes rows)
//   stamped_empty         an empty kernel + one row: the chain's floor
//   stamped_clock_khz     the nominal rate of the stamps' clock, as the device reports it
#include <hip/hip_runtime.h>

#include "vllm-expert-cache_amd/csrc/gather.h"
#include "vllm-expert-cache_amd/csrc/manage.h"

namespace {

using namespace ec;

__device__ __forceinline__ unsigned long long clock_now() {
  return __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ void put_row(unsigned long long* row, unsigned long long t0,
                                        unsigned long long t1) {
  typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u64x2*>(row) = u64x2{t0, t1};
}

// manage_k<CS, false, 4, true, TQ> with stamps
template <int CS, int TQ>
__global__ __launch_bounds__(kWave) void stamped_manage_k(ManageArgs a,
                                                          unsigned long long* row) {
  const unsigned long long t0 = clock_now();
  __shared__ ManageLds<false> L;
  args_in_sgprs(a);
  long long idv[kIdRegs];
  manage_step<CS, false, 4, TQ>(a, L, idv);
  lds_sync();
  remap_tail<false, 4>(a, L, idv);
  __builtin_amdgcn_s_waitcnt(0);
  const unsigned long long t1 = clock_now();
  if (__lane_id() == 0) put_row(row, t0, t1);
}

// gather_k<kGatherUnroll, true, false, false> with stamps, one row per workgroup
__global__ __launch_bounds__(kGatherThreads) void stamped_gather_k(
    GatherArgs g, const int* __restrict__ miss, const int* __restrict__ n_miss,
    unsigned long long* rows) {
  const unsigned long long t0 = clock_now();
  const long long wg = (long long)blockIdx.y * gridDim.x + blockIdx.x;
  gather_walk<kGatherUnroll, true, false, false>(g, miss, n_miss, nullptr, wg);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const unsigned long long t1 = clock_now();
  if (threadIdx.x == 0) put_row(rows + 2 * wg, t0, t1);
}

__global__ __launch_bounds__(kWave) void stamped_empty_k(unsigned long long* row) {
  const unsigned long long t0 = clock_now();
  if (__lane_id() == 0) put_row(row, t0, clock_now());
}

template <int TQ>
void launch_tq(const ManageArgs& a, unsigned long long* row, hipStream_t s) {
  if (a.S <= 64)
    hipLaunchKernelGGL((stamped_manage_k<1, TQ>), dim3(1), dim3(kWave), 0, s, a, row);
  else if (a.S <= 128)
    hipLaunchKernelGGL((stamped_manage_k<2, TQ>), dim3(1), dim3(kWave), 0, s, a, row);
  else if (a.S <= 256)
    hipLaunchKernelGGL((stamped_manage_k<4, TQ>), dim3(1), dim3(kWave), 0, s, a, row);
  else if (a.S <= 512)
    hipLaunchKernelGGL((stamped_manage_k<8, TQ>), dim3(1), dim3(kWave), 0, s, a, row);
  else
    hipLaunchKernelGGL((stamped_manage_k<16, TQ>), dim3(1), dim3(kWave), 0, s, a, row);
}

}  // namespace

extern "C" {

// expert_cache_manage_remap's arguments (int32 ids only, E <= 4096) plus the stamp row.
int stamped_manage_remap(const void* ids, int id_bytes, int mk, int E, int S, int max_distinct,
                         int max_inserts, int* table, int* map_cold, int* slot_expert,
                         long long* slot_stamp, unsigned char* routed, long long* step,
                         int* miss, int* n_miss, int policy, int decay, void* out,
                         unsigned long long* row, hipStream_t stream) {
  if (E <= 0 || E > kLdsExperts || S <= 0 || S > kMaxSlots || id_bytes != 4) return -1;
  if (max_inserts < 0 || max_inserts > kMaxInserts || policy < 0 || policy > 1) return -1;
  if ((mk > 0 && out == nullptr) || row == nullptr) return -1;
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
  switch (table_chunks(E)) {
    case 1: launch_tq<1>(a, row, stream); break;
    case 2: launch_tq<2>(a, row, stream); break;
    case 4: launch_tq<4>(a, row, stream); break;
    default: launch_tq<kTabRegs>(a, row, stream); break;
  }
  return (int)hipGetLastError();
}

// expert_cache_gather's arguments plus the stamp rows (one per workgroup: chunks x lanes).
int stamped_gather(void* d0, const void* s0, long b0, void* d1, const void* s1, long b1,
                   void* d2, const void* s2, long b2, void* d3, const void* s3, long b3,
                   void* d4, const void* s4, long b4, void* d5, const void* s5, long b5,
                   const int* miss, const int* n_miss, int chunks, int lanes,
                   unsigned long long* rows, hipStream_t stream) {
  void* const dst[kGatherBufs] = {d0, d1, d2, d3, d4, d5};
  const void* const src[kGatherBufs] = {s0, s1, s2, s3, s4, s5};
  const long bytes[kGatherBufs] = {b0, b1, b2, b3, b4, b5};
  GatherArgs g;
  if (n_miss == nullptr || rows == nullptr || !gather_plan(dst, src, bytes, chunks, lanes, g))
    return -1;
  hipLaunchKernelGGL(stamped_gather_k, dim3(chunks, lanes), dim3(kGatherThreads), 0, stream, g,
                     miss, n_miss, rows);
  return (int)hipGetLastError();
}

int stamped_empty(unsigned long long* row, hipStream_t stream) {
  if (row == nullptr) return -1;
  hipLaunchKernelGGL(stamped_empty_k, dim3(1), dim3(kWave), 0, stream, row);
  return (int)hipGetLastError();
}

// The device's nominal rate of the clock the stamps read, in kHz (-1 if not reported).
int stamped_clock_khz(int device) {
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeWallClockRate, device) != hipSuccess) return -1;
  return v;
}

}  // extern "C"
