// Wave64 primitives for gfx950 (CDNA4): DPP reductions/scans and LDS-only syncs.
//
// Every kernel in this library that uses them runs as ONE wavefront per workgroup, so a
// "barrier" is only an ordering point for LDS traffic between lanes of that wave: the
// compiler drops s_barrier for a 64-lane workgroup and the local-address-space fence
// waits for LDS operations (lgkmcnt) only, leaving global loads in flight across it.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ec {

constexpr int kWave = 64;

// Orders LDS accesses of the wave before/after this point.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders LDS and global accesses of the wave before/after this point, and waits until the
// wave's outstanding memory operations have completed.
__device__ __forceinline__ void mem_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
}

__device__ __forceinline__ unsigned long long lanes_below() {
  return (1ull << __lane_id()) - 1ull;
}

// One DPP step of a signed 64-bit min: lanes whose DPP source is outside the row pattern
// (or in a row the mask leaves out) combine with INT64_MAX, i.e. keep their value.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ long long dpp_min_step(long long v) {
  const int lo = (int)(unsigned long long)v;
  const int hi = (int)((unsigned long long)v >> 32);
  const int olo = __builtin_amdgcn_update_dpp((int)0xFFFFFFFF, lo, CTRL, ROWMASK, 0xF, false);
  const int ohi = __builtin_amdgcn_update_dpp(0x7FFFFFFF, hi, CTRL, ROWMASK, 0xF, false);
  const long long o = (long long)(((unsigned long long)(unsigned)ohi << 32) | (unsigned)olo);
  return o < v ? o : v;
}

// Minimum of `v` over all 64 lanes, returned to every lane (all lanes must be active).
// row_shr 1,2,4,8 leaves each row's minimum in its lane 15; row_bcast 15 and 31 fold the
// four rows into lane 63, which is read back as a wave-uniform value.
__device__ __forceinline__ long long wave_min_i64(long long v) {
  v = dpp_min_step<0x111, 0xF>(v);
  v = dpp_min_step<0x112, 0xF>(v);
  v = dpp_min_step<0x114, 0xF>(v);
  v = dpp_min_step<0x118, 0xF>(v);
  v = dpp_min_step<0x142, 0xA>(v);
  v = dpp_min_step<0x143, 0xC>(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned long long)v, 63);
  const unsigned hi =
      (unsigned)__builtin_amdgcn_readlane((int)((unsigned long long)v >> 32), 63);
  return (long long)(((unsigned long long)hi << 32) | lo);
}

template <int CTRL, int ROWMASK>
__device__ __forceinline__ int dpp_add_step(int v) {
  return v + __builtin_amdgcn_update_dpp(0, v, CTRL, ROWMASK, 0xF, false);
}

// Inclusive prefix sum over the 64 lanes in lane order (all lanes must be active).
__device__ __forceinline__ int wave_incl_scan(int v) {
  v = dpp_add_step<0x111, 0xF>(v);
  v = dpp_add_step<0x112, 0xF>(v);
  v = dpp_add_step<0x114, 0xF>(v);
  v = dpp_add_step<0x118, 0xF>(v);
  v = dpp_add_step<0x142, 0xA>(v);
  v = dpp_add_step<0x143, 0xC>(v);
  return v;
}

__device__ __forceinline__ int wave_lane_value(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

}  // namespace ec
