/*
 * libexpertcache.so -- C-ABI of the per-MoE-layer expert cache, built for gfx950 (MI355X).
 *
 * Every pointer is caller-owned (device memory, or for gather sources host memory the
 * device can read); the library allocates nothing and keeps no state. Every call is
 * asynchronous on `stream`, reads no device value back to the host and allocates nothing,
 * so any sequence of calls can be captured into a HIP graph.
 *
 * Return value: 0 on success; -1 when an argument check fails (checked on the host before
 * any HIP call, so these paths need no GPU); otherwise the hipError_t of the launch.
 *
 * State of one layer's cache (what the caller allocates, vllm_expert_cache/cache.py:84-92):
 *   table       int32[E]    expert -> slot, or -1
 *   map_cold    int32[E]    expert -> itself when not resident, else -1
 *   slot_expert int32[S]    slot -> expert, or -1
 *   slot_stamp  int64[S]    slot priority: last step routed (LRU) or hit count (LFU)
 *   routed      uint8[E]    left holding this step's routed flags
 *   step        int64[1]    calls so far
 *   miss        int32[2*max_inserts]  (expert, slot) pairs of this step's inserts
 *   n_miss      int32[1]    number of pairs
 */
#ifndef EXPERT_CACHE_H
#define EXPERT_CACHE_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/*
 * One policy step: mark the experts routed this step, refresh the priority of the resident
 * ones, pick victims among the slots not needed this step (lowest (stamp, slot) first),
 * install the missing experts in ascending id order and write the miss list.
 * policy 0 = LRU, 1 = LFU (counts halve every `decay` steps on steps that insert).
 * Fails with -1 unless E > 0, 0 < S <= 1024, 0 <= max_inserts <= 1024, policy in {0, 1}.
 *
 * Replaces: kernels/expert_cache.hip:592-603 (same signature, same checks, same results);
 * bound by vllm_expert_cache/_lib.py:44-47.
 */
int expert_cache_manage(const int* topk_ids, int mk, int E, int S, int max_distinct,
                        int max_inserts, int* table, int* map_cold, int* slot_expert,
                        long long* slot_stamp, unsigned char* routed, long long* step,
                        int* miss, int* n_miss, int policy, int decay, hipStream_t stream);

/*
 * Copy every missing expert's slabs from host-readable memory into its slot: for
 * j < *n_miss and each of the six buffers, dst_b[slot_j] <- src_b[expert_j], b_b bytes per
 * expert. A buffer repeated with the same (dst, src, bytes) is copied once. `miss` is read
 * only for j < *n_miss, so a list with no capacity is accepted while *n_miss is 0.
 * The grid is chunks x lanes workgroups of 256 lanes; the work (miss, buffer, tile) is
 * spread over the whole grid whatever n_miss is.
 * Fails with -1 unless every b_b > 0 and b_b % 16 == 0, chunks > 0 and lanes > 0, and
 * when n_miss is null (every launch reads *n_miss on the device).
 *
 * Replaces: kernels/expert_cache.hip:626-643 (same signature and checks, plus the null
 * n_miss, which the reference's kernel would dereference);
 * bound by vllm_expert_cache/_lib.py:49-53.
 */
int expert_cache_gather(void* d0, const void* s0, long b0, void* d1, const void* s1, long b1,
                        void* d2, const void* s2, long b2, void* d3, const void* s3, long b3,
                        void* d4, const void* s4, long b4, void* d5, const void* s5, long b5,
                        const int* miss, const int* n_miss, int chunks, int lanes,
                        hipStream_t stream);

/*
 * expert_cache_gather for the miss list of a prefetch step (expert_cache_prefetch), which
 * may run while the real step that settles those installs runs on another stream: a tile of
 * pair (e, slot) is loaded only while slot_expert[slot] == e, so once the real step drops a
 * prediction its copy stops within a tile or two per workgroup. The comparison reads
 * slot_expert with device-coherent loads; the first tile of each pair is loaded without
 * one. Tiles already loaded are stored. Confirmed and still-pending predictions are copied
 * whole. The caller must order any later copy into these slots (the real step's gather)
 * after this call, as it must for any prefetch copy.
 * Fails with -1 where expert_cache_gather does, or when slot_expert is null.
 *
 * No counterpart in the reference's C-ABI (prefetch is README.md:392-394's next step).
 */
int expert_cache_gather_live(void* d0, const void* s0, long b0, void* d1, const void* s1,
                             long b1, void* d2, const void* s2, long b2, void* d3,
                             const void* s3, long b3, void* d4, const void* s4, long b4,
                             void* d5, const void* s5, long b5, const int* miss,
                             const int* n_miss, const int* slot_expert, int chunks, int lanes,
                             hipStream_t stream);

/*
 * The LRU policy step (hits and installs stamp the current step, no decay) followed by both
 * moe_align_block_size outputs built from the updated table: the resident side bucketed by
 * slot, the non-resident side bucketed by expert id; sentinel mk in sorted_*, -1 in unused
 * eids_* blocks, ids outside [0, E) skipped. Within a bucket, ids are in token order.
 * L and NB must be the lengths vLLM's wrapper allocates:
 *   L = mk < E ? min(mk*bs, mk + E*(bs-1)) : mk + E*(bs-1),  NB = ceil(L / bs).
 * Fails with -1 unless 0 < E <= 1024, 0 < S <= 1024, bs, L, NB > 0, mk >= 0,
 * 0 <= max_inserts <= 1024.
 *
 * Replaces: kernels/expert_cache.hip:605-624 (same signature and checks).
 */
int expert_cache_fused(const int* topk_ids, int mk, int E, int S, int max_distinct,
                       int max_inserts, int* table, int* map_cold, int* slot_expert,
                       long long* slot_stamp, unsigned char* routed, long long* step,
                       int* miss, int* n_miss, int bs, int L, int NB, int* sorted_hot,
                       int* eids_hot, int* npad_hot, int* sorted_cold, int* eids_cold,
                       int* npad_cold, hipStream_t stream);

/*
 * Routing ids from expert space to slot space: out[i] = table[ids[i]], a negative id
 * wrapping to table[E + id] as torch indexing does. `id_bytes` is 4 (int32 ids and out) or
 * 8 (int64 ids and out). An id outside [-E, E) (an index error in torch) gives -1.
 * Fails with -1 unless E > 0, n >= 0 and id_bytes is 4 or 8.
 *
 * Replaces: vllm_expert_cache/cache.py:108-110 (`table[ids.long()].to(ids.dtype)`, three
 * torch kernels); no counterpart in the reference's C-ABI.
 */
int expert_cache_remap(const void* ids, int n, int id_bytes, const int* table, int E,
                       void* out, hipStream_t stream);

/*
 * expert_cache_manage followed by expert_cache_remap of the same ids against the updated
 * table, in one launch. `ids` are int32 (id_bytes 4) or int64 (id_bytes 8); the policy sees
 * each id truncated to int32, as the reference's `topk_ids.to(torch.int32)` does, and `out`
 * receives the slot ids in the dtype of `ids`. Argument checks are those of
 * expert_cache_manage plus id_bytes in {4, 8} and out non-null when mk > 0.
 *
 * Replaces: vllm_expert_cache/cache.py:116-133 plus :163 (cast, manage, and the torch
 * remap); no counterpart in the reference's C-ABI.
 */
int expert_cache_manage_remap(const void* ids, int id_bytes, int mk, int E, int S,
                              int max_distinct, int max_inserts, int* table, int* map_cold,
                              int* slot_expert, long long* slot_stamp, unsigned char* routed,
                              long long* step, int* miss, int* n_miss, int policy, int decay,
                              void* out, hipStream_t stream);

/*
 * Prefetch step: bring the experts predicted for this layer's next step into slots ahead of
 * that step, so their copy can run (expert_cache_gather over this call's miss list, on any
 * stream) while other work proceeds. It installs like expert_cache_manage -- the predicted
 * experts that are not resident, in ascending id order, into the lowest (stamp, slot) keys
 * among the slots whose expert is not predicted, at most max_inserts of them, writing the
 * (expert, slot) pairs to miss and their count to n_miss -- but it does not advance any step
 * counter, leaves the stamps of resident predicted experts alone, never ages, and gives each
 * install stamp -1, marking it pending. The next served call of expert_cache_manage (or of
 * the manage_remap / fused entry points) settles every pending slot before counting hits:
 * one whose expert is routed is confirmed and ends that step with the stamp a real install
 * of the step gets (the step number under LRU, 1 under LFU, after any ageing); one whose
 * expert is not routed is dropped -- table[e] = -1, map_cold[e] = e, the slot empty at stamp
 * 0 -- so a wrong prediction leaves nothing resident behind. A right prediction leaves the
 * policy state after the next expert_cache_manage equal to what that call alone would give
 * (except on an LFU step that would have aged the counts). Pending keys sort below every
 * real key, so a further prefetch step evicts unconfirmed predictions first. The
 * reference's states never hold a negative stamp, so on them nothing here changes.
 * `routed` is left holding the predicted flags. pred_ids are int32; ids outside [0, E) are
 * ignored. Use a miss/n_miss pair of its own, not the one the real step's gather reads, and
 * copy with expert_cache_gather_live so that dropped predictions stop copying.
 * Fails with -1 unless E > 0, 0 < S <= 1024, 0 <= max_inserts <= 1024 and mk >= 0.
 *
 * No counterpart in the reference's C-ABI: README.md:392-394 names next-layer prefetch as
 * the path's next step without implementing it.
 */
int expert_cache_prefetch(const int* pred_ids, int mk, int E, int S, int max_inserts,
                          int* table, int* map_cold, int* slot_expert, long long* slot_stamp,
                          unsigned char* routed, int* miss, int* n_miss, hipStream_t stream);

/*
 * expert_cache_manage_remap on one layer's state and expert_cache_prefetch on another's, in
 * one launch of two workgroups: the results are exactly those of the two calls made
 * separately (in either order). A decode step that predicts the next layer's routing before
 * this layer's policy step puts one node on the stream for both instead of two. The pf_*
 * arguments are expert_cache_prefetch's, for the other layer; both layers have E experts
 * and S slots. Argument checks are those of the two calls, and it also fails with -1 when
 * the two layers' table, map_cold, slot_expert, slot_stamp, routed, miss (2 x max_inserts
 * ints against 2 x pf_max_inserts) or n_miss arrays overlap. No array of one layer may
 * overlap any array of the other, since the workgroups run unordered.
 *
 * No counterpart in the reference's C-ABI, like expert_cache_prefetch (README.md:392-394).
 */
int expert_cache_manage_remap_prefetch(
    const void* ids, int id_bytes, int mk, int E, int S, int max_distinct, int max_inserts,
    int* table, int* map_cold, int* slot_expert, long long* slot_stamp, unsigned char* routed,
    long long* step, int* miss, int* n_miss, int policy, int decay, void* out,
    const int* pred_ids, int pk, int pf_max_inserts, int* pf_table, int* pf_map_cold,
    int* pf_slot_expert, long long* pf_slot_stamp, unsigned char* pf_routed, int* pf_miss,
    int* pf_n_miss, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EXPERT_CACHE_H */
