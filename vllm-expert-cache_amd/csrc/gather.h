// expert_cache_gather on gfx950: copy each missing expert's slabs from host-readable memory
// into its HBM slot (kernels/expert_cache.hip:284-314 semantics: for j < n_miss and every
// buffer b, dst_b[slot_j] <- src_b[expert_j]).
//
// The work is flattened instead of split by miss: one miss is `per_miss` tiles (each buffer
// cut into tiles of 256 lanes x U 16-byte vectors), and tile t of the whole step goes to
// workgroup t mod grid, so the grid's loads form one front that streams through the miss
// list in address order whatever n_miss is. What bounds the copy is the host link, and it
// is saturated by a modest amount of data in flight (grid x tile, ~256 KB); the grid is
// sized for that, not for the CU count. The grid shape is fixed at launch and the tile
// count is read from n_miss on the device, so the launch stays graph-capturable.
#pragma once
#include <hip/hip_runtime.h>

namespace ec {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGatherBufs = 6;
constexpr int kGatherThreads = 256;

struct GatherArgs {
  u32x4* dst[kGatherBufs];
  const u32x4* src[kGatherBufs];
  long long vec[kGatherBufs];            // 16-byte vectors per expert
  long long tile0[kGatherBufs + 1];      // first tile of buffer b within one miss
  int nbuf;                              // distinct buffers after de-duplication
};

template <int U, bool NT_LOAD, bool NT_STORE>
__global__ __launch_bounds__(kGatherThreads) void gather_k(GatherArgs g,
                                                           const int* __restrict__ miss,
                                                           const int* __restrict__ n_miss) {
  constexpr int kTile = kGatherThreads * U;
  const long long per_miss = g.tile0[g.nbuf];
  const long long total = (long long)n_miss[0] * per_miss;
  const long long nblk = (long long)gridDim.x * gridDim.y;
  for (long long t = (long long)blockIdx.y * gridDim.x + blockIdx.x; t < total; t += nblk) {
    const int j = (int)(t / per_miss);
    const long long r = t - (long long)j * per_miss;
    int b = 0;
    while (b + 1 < g.nbuf && r >= g.tile0[b + 1]) ++b;
    const int e = miss[2 * j];
    const int sl = miss[2 * j + 1];
    const long long V = g.vec[b];
    const long long off = (r - g.tile0[b]) * kTile;
    const int n = (int)min((long long)kTile, V - off);
    const u32x4* __restrict__ s = g.src[b] + (long long)e * V + off;
    u32x4* __restrict__ d = g.dst[b] + (long long)sl * V + off;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = threadIdx.x + u * kGatherThreads;
      if (i < n) {
        if constexpr (NT_LOAD)
          v[u] = __builtin_nontemporal_load(s + i);
        else
          v[u] = s[i];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = threadIdx.x + u * kGatherThreads;
      if (i < n) {
        if constexpr (NT_STORE)
          __builtin_nontemporal_store(v[u], d + i);
        else
          d[i] = v[u];
      }
    }
  }
}

}  // namespace ec
