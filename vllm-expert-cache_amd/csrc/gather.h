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
  long long per;                         // tiles per miss (tile0[nbuf])
  long long jstep, rstep;                // a workgroup's stride in (miss, tile): grid / per,
                                         // grid % per (computed by the host)
  int nbuf;                              // distinct buffers after de-duplication
};

// Position of one tile: miss j, buffer b, first vector `off`, vectors `n`, and the source and
// destination of that range.
struct GatherTile {
  const u32x4* src;
  u32x4* dst;
  int n;
};

// The buffer of tile r and its fields are picked with constant indexes only (a select
// chain), so every field is a kernel argument the wave loads once, up front.
template <int U>
__device__ __forceinline__ GatherTile gather_tile(const GatherArgs& g, int e, int sl,
                                                  long long r) {
  constexpr long long kTile = (long long)kGatherThreads * U;
  const u32x4* src = g.src[0];
  u32x4* dst = g.dst[0];
  long long V = g.vec[0], first = g.tile0[0];
#pragma unroll
  for (int i = 1; i < kGatherBufs; ++i) {
    if (i < g.nbuf && r >= g.tile0[i]) {
      src = g.src[i];
      dst = g.dst[i];
      V = g.vec[i];
      first = g.tile0[i];
    }
  }
  const long long off = (r - first) * kTile;
  GatherTile t;
  t.src = src + (long long)e * V + off;
  t.dst = dst + (long long)sl * V + off;
  t.n = (int)min(kTile, V - off);
  return t;
}

template <int U, bool NT_LOAD>
__device__ __forceinline__ void tile_load(const GatherTile& t, u32x4 (&v)[U]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = threadIdx.x + u * kGatherThreads;
    if (i < t.n) {
      if constexpr (NT_LOAD)
        v[u] = __builtin_nontemporal_load(t.src + i);
      else
        v[u] = t.src[i];
    }
  }
}

template <int U, bool NT_STORE>
__device__ __forceinline__ void tile_store(const GatherTile& t, const u32x4 (&v)[U]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = threadIdx.x + u * kGatherThreads;
    if (i < t.n) {
      if constexpr (NT_STORE)
        __builtin_nontemporal_store(v[u], t.dst + i);
      else
        t.dst[i] = v[u];
    }
  }
}

// Each workgroup walks tiles blockId, blockId + grid, ... of the step. The walk keeps its
// (miss, tile-in-miss) position incrementally (no division per tile), reloads the miss pair
// only when the walk moves to another miss, and issues the next tile's host loads before
// storing the current tile, so the scalar bookkeeping never sits between two tiles' loads.
//
// LIVE is the copy of a prefetch step's installs, which may overlap the real step that
// settles them: a dropped prediction's slot stops naming its expert. Before loading each
// tile after a miss's first, the workgroup compares slot_expert[slot] with the expert and
// stops loading that miss once they differ. The comparison uses a device-coherent load
// issued one tile ahead, so no tile load waits for it; the first tile of a miss is loaded
// without one. Tiles already loaded are still stored: a dropped slot is empty, or gets
// another expert whose own copy the caller orders after this kernel.
template <int U, bool NT_LOAD, bool NT_STORE, bool LIVE>
__device__ __forceinline__ void gather_walk(const GatherArgs& g, const int* __restrict__ miss,
                                            const int* __restrict__ n_miss,
                                            const int* slot_expert, long long t0) {
  const long long per = g.per;
  // The miss list is read only below n_miss, as kernels/expert_cache.hip:294-298 reads it:
  // a caller with no insert capacity (max_inserts = 0) may pass an empty list.
  const int nm = n_miss[0];
  if (nm <= 0 || per <= 0 || t0 >= (long long)nm * per) return;
  const long long jstep = g.jstep, rstep = g.rstep;
  // first tile: in miss 0 whenever a miss spans more tiles than the grid has workgroups
  int j = t0 < per ? 0 : (int)(t0 / per);
  long long r = t0 - (long long)j * per;
  int e = miss[2 * j], sl = miss[2 * j + 1];
  // slot_expert[sl] as last read, for the next tile of the same miss; every such read is
  // issued before the tile loads that follow it, so waiting for it never waits for them
  int seen = 0;
  if constexpr (LIVE)
    seen = __hip_atomic_load(slot_expert + sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  GatherTile cur = gather_tile<U>(g, e, sl, r);
  u32x4 v[U];
  tile_load<U, NT_LOAD>(cur, v);
  bool have = true;  // v holds tile `cur`, to be stored
  for (;;) {
    // advance to this workgroup's next tile
    int jn = j + (int)jstep;
    long long rn = r + rstep;
    if (rn >= per) {
      rn -= per;
      ++jn;
    }
    if (jn >= nm) break;
    bool live = true;
    if (jn != j) {
      e = miss[2 * jn];
      sl = miss[2 * jn + 1];
      if constexpr (LIVE)
        seen = __hip_atomic_load(slot_expert + sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if constexpr (LIVE) {
      live = seen == e;
      if (live)
        seen = __hip_atomic_load(slot_expert + sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    j = jn;
    r = rn;
    GatherTile next = cur;
    u32x4 w[U];
    if (live) {
      next = gather_tile<U>(g, e, sl, r);
      tile_load<U, NT_LOAD>(next, w);
    }
    if (have) tile_store<U, NT_STORE>(cur, v);
    have = live;
    if (live) {
      cur = next;
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = w[u];
    }
  }
  if (have) tile_store<U, NT_STORE>(cur, v);
}

template <int U, bool NT_LOAD, bool NT_STORE, bool LIVE>
__global__ __launch_bounds__(kGatherThreads) void gather_k(GatherArgs g,
                                                           const int* __restrict__ miss,
                                                           const int* __restrict__ n_miss,
                                                           const int* slot_expert) {
  gather_walk<U, NT_LOAD, NT_STORE, LIVE>(g, miss, n_miss, slot_expert,
                                          (long long)blockIdx.y * gridDim.x + blockIdx.x);
}

// Gather tile: 256 lanes x 2 vectors = 8 KB per workgroup iteration, loads non-temporal
// (host rows are streamed once), stores default so the fresh slot stays in cache for the
// GEMM that reads it next. Measured on MI355X over PCIe Gen5: the host link saturates at
// ~128-256 KB in flight (its bandwidth-delay product); far more in flight at once (every
// tile of an expert issued together) drops a 4.7 MB expert from ~54.5 to ~41 GB/s. So the
// caller's grid should be small (32 workgroups x 8 KB = 256 KB) and the tiles stream
// through the expert in order, each workgroup taking every grid-th tile. Fewer, wider
// workgroups with the same bytes in flight are slower (16 x 16 KB and 8 x 32 KB took 1.26x
// and 2.3x as long per decode step): one compute unit keeps only so many host reads in
// flight, so the reads must spread over many.
constexpr int kGatherUnroll = 2;

// The gather's launch arguments from the six (dst, src, bytes) triples: the checks of
// kernels/expert_cache.hip:631-634, then the buffers with a repeated (dst, src, bytes) -- the
// caller's padding of a short list -- dropped, since they would copy the same bytes to the
// same place, and each workgroup's stride through the step's (miss, tile) space.
inline bool gather_plan(void* const (&dst)[kGatherBufs], const void* const (&src)[kGatherBufs],
                        const long (&bytes)[kGatherBufs], int chunks, int lanes,
                        GatherArgs& g) {
  for (int i = 0; i < kGatherBufs; i++)
    if (bytes[i] <= 0 || bytes[i] % 16) return false;
  if (chunks <= 0 || lanes <= 0) return false;
  constexpr long long kTile = (long long)kGatherThreads * kGatherUnroll;
  g.nbuf = 0;
  g.tile0[0] = 0;
  for (int i = 0; i < kGatherBufs; i++) {
    bool dup = false;
    for (int k = 0; k < i; k++)
      dup = dup || (dst[k] == dst[i] && src[k] == src[i] && bytes[k] == bytes[i]);
    if (dup) continue;
    const int b = g.nbuf++;
    g.dst[b] = static_cast<u32x4*>(dst[i]);
    g.src[b] = static_cast<const u32x4*>(src[i]);
    g.vec[b] = bytes[i] / 16;
    g.tile0[b + 1] = g.tile0[b] + (g.vec[b] + kTile - 1) / kTile;
  }
  for (int b = g.nbuf; b < kGatherBufs; b++) {
    g.dst[b] = nullptr;
    g.src[b] = nullptr;
    g.vec[b] = 0;
    g.tile0[b + 1] = g.tile0[b];
  }
  g.per = g.tile0[g.nbuf];
  const long long nblk = (long long)chunks * lanes;
  g.jstep = g.per > 0 ? nblk / g.per : 0;
  g.rstep = g.per > 0 ? nblk % g.per : 0;
  return true;
}

}  // namespace ec
