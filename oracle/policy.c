/*
 * CPU oracle for the per-layer expert-cache path (manage, remap, gather, fused align).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links or calls this file. It is
 * used by tests/ and __graft_entry__.smoke() to check the GPU path's results against, and
 * by bench.py's cpu_baseline leg as the CPU policy that is timed beside the GPU path.
 *
 * It restates, in plain C, the algorithm of the reference's policy model and kernel:
 *
 *   manage (serial form)  tests/test_policy.py:83-132      (ref_step, numpy model: one argmin
 *                                                            per insert over the evictable set)
 *   manage (rank form)    kernels/expert_cache.hip:191-282 (expert_cache_manage_k) with
 *                         kernels/expert_cache.hip:104-189 (installVictim / pickVictims: the
 *                                                            nins smallest keys, by rank)
 *   remap                 vllm_expert_cache/cache.py:108-110 (table[ids.long()].to(ids.dtype),
 *                                                            negative ids wrap like torch)
 *   gather                kernels/expert_cache.hip:284-314 (byte copy of each miss's slabs)
 *   fused align           kernels/expert_cache.hip:431-588 (LRU manage + both
 *                                                            moe_align_block_size outputs)
 *   prefetch              README.md:392-394 names next-layer prefetch; its install-only
 *                         step is defined below and pinned against the manage rules
 *
 * Two independent victim rules (serial argmin, batched rank-select) are kept on purpose: the
 * reference argues they are the same answer (kernels/expert_cache.hip:83-97) and the tests
 * check that claim on every step of every trace.
 *
 * Where the reference would index out of bounds on a corrupt state (a slot_expert or table
 * entry outside [0,E) / [0,S)), this oracle and the HIP kernels ignore the entry instead.
 * No reachable state has such an entry.
 */
#define _POSIX_C_SOURCE 199309L
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define OR_SLOT_BITS 20
#define OR_SLOT_MASK ((1 << OR_SLOT_BITS) - 1)
#define OR_MAXS 1024
#define OR_MAXINS 1024
#define OR_MAXE_FUSED 1024

/* Argument checks of the C-ABI (kernels/expert_cache.hip:596-598). */
static int manage_args_bad(int E, int S, int max_inserts, int policy) {
  if (E <= 0 || S <= 0 || S > OR_MAXS || S > OR_SLOT_MASK) return 1;
  if (max_inserts < 0 || max_inserts > OR_MAXINS) return 1;
  if (policy < 0 || policy > 1) return 1;
  return 0;
}

/* Victim key: (stamp, slot) packed as the kernel packs it, stamp<<20 | slot
 * (kernels/expert_cache.hip:132-133). The shift is done unsigned so that the bits match the
 * kernel's signed shift without C undefined behaviour. */
static inline int64_t vkey(int64_t stamp, int slot) {
  return (int64_t)(((uint64_t)stamp << OR_SLOT_BITS) | (uint64_t)slot);
}

static inline int slot_evictable(const int32_t* slot_expert, const uint8_t* routed, int E,
                                 int i) {
  const int x = slot_expert[i];
  return x < 0 || x >= E || !routed[x];
}

/* Front half shared by both victim rules: steps 1-6 of one manage call.
 * Returns the number of inserts to attempt (nins), or -1 when the call stops early
 * (read-through or nothing to insert). `misses` receives the missing experts in ascending
 * id order (at most nins of them).
 *
 * Pending prefetch installs. A slot whose stamp is negative holds an expert that
 * oracle_prefetch installed and no real step has seen since (the reference never produces a
 * negative stamp, so on its states nothing below changes). Once the step is served (past the
 * read-through check), each such slot is settled before hits are counted:
 *   - its expert is routed: the prediction is confirmed, and the slot ends the step with the
 *     stamp a real install of this step gets (st under LRU, 1 under LFU; after any ageing),
 *     instead of a hit's refresh;
 *   - its expert is not routed: the prediction is dropped, as if it had never been copied
 *     (its copy may be cut short): table = -1 and map_cold = itself for the expert, the slot
 *     becomes empty with stamp 0 and is evictable like any other empty slot. */
static int manage_front(const int32_t* ids, int mk, int E, int S, int max_distinct,
                        int max_inserts, int32_t* table, int32_t* map_cold,
                        int32_t* slot_expert, int64_t* slot_stamp, uint8_t* routed,
                        int64_t* step, int32_t* miss, int32_t* n_miss, int policy, int decay,
                        int32_t* misses, int64_t* st_out) {
  /* step advances and n_miss clears on every call (kernels/expert_cache.hip:214-217) */
  step[0] += 1;
  n_miss[0] = 0;
  const int64_t st = step[0];
  *st_out = st;

  /* routed flags; ids outside [0,E) are padding (kernels/expert_cache.hip:218-225) */
  memset(routed, 0, (size_t)E);
  for (int i = 0; i < mk; i++) {
    const int e = ids[i];
    if (e >= 0 && e < E) routed[e] = 1;
  }
  int cnt = 0;
  for (int e = 0; e < E; e++) cnt += routed[e];
  if (cnt > max_distinct) return -1; /* read-through: nothing else changes (:228-232) */

  /* settle pending prefetch installs (see above) */
  const int64_t fresh = (policy == 0) ? st : 1;
  uint8_t confirmed[OR_MAXS];
  for (int i = 0; i < S; i++) {
    const int x = slot_expert[i];
    confirmed[i] = 0;
    if (slot_stamp[i] >= 0 || x < 0 || x >= E) continue;
    if (routed[x]) {
      confirmed[i] = 1;
    } else {
      table[x] = -1;
      map_cold[x] = x;
      slot_expert[i] = -1;
      slot_stamp[i] = 0;
    }
  }

  /* hits refresh, misses enumerate in ascending id (:234-246; test_policy.py:97-106) */
  int total = 0;
  for (int e = 0; e < E; e++) {
    if (!routed[e]) continue;
    const int s = table[e];
    if (s >= 0) {
      if (s < S && !confirmed[s])
        slot_stamp[s] = (policy == 0) ? st : (int64_t)((uint64_t)slot_stamp[s] + 1);
    } else {
      if (total < max_inserts) misses[total] = e;
      total++;
    }
  }
  const int nins = total < max_inserts ? total : max_inserts;
  for (int j = 0; j < nins; j++) miss[2 * j] = misses[j]; /* even if fewer install (:252-259) */

  /* LFU ageing: halve every stamp on inserting steps where st % decay == 0 (:261-267); no
   * decay on a step without inserts (:251) */
  if (nins > 0 && policy != 0 && decay > 0 && (st % (int64_t)decay) == 0)
    for (int i = 0; i < S; i++) slot_stamp[i] >>= 1;
  for (int i = 0; i < S; i++)
    if (confirmed[i]) slot_stamp[i] = fresh;
  return nins > 0 ? nins : -1;
}

/* installVictim (kernels/expert_cache.hip:104-121; test_policy.py:122-131) */
static void install(int r, int sl, int32_t e, int64_t fresh, int E, int32_t* table,
                    int32_t* map_cold, int32_t* slot_expert, int64_t* slot_stamp,
                    int32_t* miss) {
  const int old = slot_expert[sl];
  if (old >= 0 && old < E) {
    table[old] = -1;
    map_cold[old] = old;
  }
  slot_expert[sl] = e;
  slot_stamp[sl] = fresh;
  table[e] = sl;
  map_cold[e] = -1;
  miss[2 * r + 1] = sl;
}

/* Serial rule: argmin over the evictable slots, one insert at a time, by (stamp, slot)
 * compared as a pair, exactly as ref_step does (test_policy.py:117-131). */
int oracle_manage_serial(const int32_t* ids, int mk, int E, int S, int max_distinct,
                         int max_inserts, int32_t* table, int32_t* map_cold,
                         int32_t* slot_expert, int64_t* slot_stamp, uint8_t* routed,
                         int64_t* step, int32_t* miss, int32_t* n_miss, int policy,
                         int decay) {
  if (manage_args_bad(E, S, max_inserts, policy)) return -1;
  int32_t misses[OR_MAXINS];
  int64_t st;
  const int nins = manage_front(ids, mk, E, S, max_distinct, max_inserts, table, map_cold,
                                slot_expert, slot_stamp, routed, step, miss, n_miss, policy,
                                decay, misses, &st);
  if (nins < 0) return 0;
  const int64_t fresh = (policy == 0) ? st : 1;
  int nact = 0;
  for (int r = 0; r < nins; r++) {
    int best = -1;
    for (int i = 0; i < S; i++) {
      if (!slot_evictable(slot_expert, routed, E, i)) continue;
      if (best < 0 || slot_stamp[i] < slot_stamp[best] ||
          (slot_stamp[i] == slot_stamp[best] && i < best))
        best = i;
    }
    if (best < 0) break; /* nothing evictable left */
    install(r, best, misses[r], fresh, E, table, map_cold, slot_expert, slot_stamp, miss);
    nact++;
  }
  n_miss[0] = nact;
  return 0;
}

/* Rank rule: every evictable slot is ranked by its packed key against the set that was
 * evictable on entry; rank r < nins receives the r-th miss (kernels/expert_cache.hip:159-188). */
int oracle_manage_rank(const int32_t* ids, int mk, int E, int S, int max_distinct,
                       int max_inserts, int32_t* table, int32_t* map_cold,
                       int32_t* slot_expert, int64_t* slot_stamp, uint8_t* routed,
                       int64_t* step, int32_t* miss, int32_t* n_miss, int policy, int decay) {
  if (manage_args_bad(E, S, max_inserts, policy)) return -1;
  int32_t misses[OR_MAXINS];
  int64_t st;
  const int nins = manage_front(ids, mk, E, S, max_distinct, max_inserts, table, map_cold,
                                slot_expert, slot_stamp, routed, step, miss, n_miss, policy,
                                decay, misses, &st);
  if (nins < 0) return 0;
  const int64_t fresh = (policy == 0) ? st : 1;
  int64_t key[OR_MAXS];
  uint8_t ev[OR_MAXS];
  int vic[OR_MAXINS];
  int nev = 0;
  for (int i = 0; i < S; i++) {
    ev[i] = (uint8_t)slot_evictable(slot_expert, routed, E, i);
    key[i] = vkey(slot_stamp[i], i);
    nev += ev[i];
  }
  for (int i = 0; i < S; i++) {
    if (!ev[i]) continue;
    int rank = 0;
    for (int j = 0; j < S; j++) rank += (ev[j] && key[j] < key[i]);
    if (rank < nins) vic[rank] = i;
  }
  const int nact = nins < nev ? nins : nev;
  for (int r = 0; r < nact; r++)
    install(r, vic[r], misses[r], fresh, E, table, map_cold, slot_expert, slot_stamp, miss);
  n_miss[0] = nact;
  return 0;
}

/* ---------------------------------------------------------------------------------------
 * Prefetch: the install-only step that brings a layer's predicted experts in ahead of its
 * next real step (README.md:392-394 names the idea; the reference has no implementation, so
 * these rules are this library's own and are pinned by tests against the manage rules):
 *   - n_miss = 0; `routed` is left holding the predicted flags (ids outside [0,E) ignored);
 *   - the step counter does not move, resident predicted experts keep their stamps, no decay;
 *   - the predicted experts that are not resident, in ascending id order, are the misses;
 *     nins = min(misses, max_inserts), miss[2j] = misses[j] for j < nins;
 *   - victims are the nins smallest keys stamp<<20 | slot among the slots whose expert is not
 *     predicted, exactly as in manage; each install gets stamp -1, which marks it pending:
 *     the next served manage step confirms it if its expert is routed (the slot takes the
 *     stamp a real install of that step gets) and drops it otherwise (the slot is emptied),
 *     see manage_front. A pending slot's key is below every real key, so a later prefetch
 *     step evicts unconfirmed predictions first.
 * Consequence, checked by the tests: with the prediction equal to the next step's routed set,
 * prefetch followed by manage leaves the same state as manage alone, with the miss list
 * moved to the prefetch, whenever that manage step would not decay. A wrong prediction
 * leaves no expert behind: the step that drops it empties its slot.
 * `rule` 0 = serial argmin, 1 = rank.
 * ------------------------------------------------------------------------------------- */
int oracle_prefetch(const int32_t* ids, int mk, int E, int S, int max_inserts, int32_t* table,
                    int32_t* map_cold, int32_t* slot_expert, int64_t* slot_stamp,
                    uint8_t* routed, int32_t* miss, int32_t* n_miss, int rule) {
  if (manage_args_bad(E, S, max_inserts, 0) || mk < 0) return -1;
  n_miss[0] = 0;
  memset(routed, 0, (size_t)E);
  for (int i = 0; i < mk; i++) {
    const int e = ids[i];
    if (e >= 0 && e < E) routed[e] = 1;
  }
  int32_t misses[OR_MAXINS];
  int total = 0;
  for (int e = 0; e < E; e++) {
    if (!routed[e] || table[e] >= 0) continue;
    if (total < max_inserts) misses[total] = e;
    total++;
  }
  const int nins = total < max_inserts ? total : max_inserts;
  for (int j = 0; j < nins; j++) miss[2 * j] = misses[j];
  if (nins == 0) return 0;

  int nact = 0;
  if (rule == 0) {
    for (int r = 0; r < nins; r++) {
      int best = -1;
      for (int i = 0; i < S; i++) {
        if (!slot_evictable(slot_expert, routed, E, i)) continue;
        if (best < 0 || slot_stamp[i] < slot_stamp[best] ||
            (slot_stamp[i] == slot_stamp[best] && i < best))
          best = i;
      }
      if (best < 0) break;
      install(r, best, misses[r], -1, E, table, map_cold, slot_expert, slot_stamp, miss);
      nact++;
    }
  } else {
    int64_t key[OR_MAXS];
    uint8_t ev[OR_MAXS];
    int vic[OR_MAXINS];
    int nev = 0;
    for (int i = 0; i < S; i++) {
      ev[i] = (uint8_t)slot_evictable(slot_expert, routed, E, i);
      key[i] = vkey(slot_stamp[i], i);
      nev += ev[i];
    }
    for (int i = 0; i < S; i++) {
      if (!ev[i]) continue;
      int rank = 0;
      for (int j = 0; j < S; j++) rank += (ev[j] && key[j] < key[i]);
      if (rank < nins) vic[rank] = i;
    }
    nact = nins < nev ? nins : nev;
    for (int r = 0; r < nact; r++)
      install(r, vic[r], misses[r], -1, E, table, map_cold, slot_expert, slot_stamp, miss);
  }
  n_miss[0] = nact;
  return 0;
}

/* Remap (vllm_expert_cache/cache.py:108-110): out[i] = table[ids[i]], where a negative id
 * wraps to table[E + id] as torch advanced indexing does. torch raises on ids outside
 * [-E, E); the oracle writes -1 there, which is what the HIP remap writes. */
void oracle_remap_i32(const int32_t* ids, int n, const int32_t* table, int E, int32_t* out) {
  for (int i = 0; i < n; i++) {
    int64_t v = ids[i];
    if (v < 0) v += E;
    out[i] = (v >= 0 && v < E) ? table[v] : -1;
  }
}

void oracle_remap_i64(const int64_t* ids, int n, const int32_t* table, int E, int64_t* out) {
  for (int i = 0; i < n; i++) {
    int64_t v = ids[i];
    if (v < 0) v += E;
    out[i] = (v >= 0 && v < E) ? (int64_t)table[v] : -1;
  }
}

/* Gather (kernels/expert_cache.hip:284-314): for j < n_miss and every buffer b,
 * dst_b[slot_j] <- src_b[expert_j], `bytes[b]` bytes per expert. */
void oracle_gather(int nbuf, uint8_t* const* dst, const uint8_t* const* src,
                   const int64_t* bytes, const int32_t* miss, int n_miss) {
  for (int j = 0; j < n_miss; j++) {
    const int e = miss[2 * j], sl = miss[2 * j + 1];
    for (int b = 0; b < nbuf; b++)
      memcpy(dst[b] + (size_t)sl * (size_t)bytes[b], src[b] + (size_t)e * (size_t)bytes[b],
             (size_t)bytes[b]);
  }
}

/*
 * One layer over a whole routing trace, the way the plugin drives it
 * (vllm_expert_cache/cache.py:99-106, :112-133): a step whose mk exceeds S reads through and
 * does not call manage at all; otherwise manage runs with max_distinct = min(E, mk) and
 * max_inserts = S. `rule` 0 = serial, 1 = rank. Optional per-step records (NULL to skip):
 *   n_miss_hist[T]             inserts per step (-1 on a read-through step)
 *   miss_hist[T * 2S]          the miss buffer after each step
 *   state_hist[T * (2E+3S+2)]  int32 words: table | map_cold | slot_expert | slot_stamp (as
 *                              2 words each) | step (2 words), after each step
 * Returns 0, or -1 on bad arguments.
 */
int oracle_run_trace(const int32_t* ids, int T, int mk, int E, int S, int policy, int decay,
                     int rule, int32_t* table, int32_t* map_cold, int32_t* slot_expert,
                     int64_t* slot_stamp, uint8_t* routed, int64_t* step, int32_t* miss,
                     int32_t* n_miss, int32_t* n_miss_hist, int32_t* miss_hist,
                     int32_t* state_hist) {
  if (manage_args_bad(E, S, S, policy) || T < 0 || mk < 0) return -1;
  const int md = mk < E ? mk : E;
  const size_t words = (size_t)2 * E + 3 * (size_t)S + 2;
  for (int t = 0; t < T; t++) {
    const int32_t* row = ids + (size_t)t * (size_t)mk;
    int served = mk <= S;
    if (served) {
      if (rule == 0)
        oracle_manage_serial(row, mk, E, S, md, S, table, map_cold, slot_expert, slot_stamp,
                             routed, step, miss, n_miss, policy, decay);
      else
        oracle_manage_rank(row, mk, E, S, md, S, table, map_cold, slot_expert, slot_stamp,
                           routed, step, miss, n_miss, policy, decay);
    }
    if (n_miss_hist) n_miss_hist[t] = served ? n_miss[0] : -1;
    if (miss_hist) memcpy(miss_hist + (size_t)t * 2 * S, miss, sizeof(int32_t) * 2 * S);
    if (state_hist) {
      int32_t* w = state_hist + (size_t)t * words;
      memcpy(w, table, sizeof(int32_t) * E);
      memcpy(w + E, map_cold, sizeof(int32_t) * E);
      memcpy(w + 2 * E, slot_expert, sizeof(int32_t) * S);
      memcpy(w + 2 * E + S, slot_stamp, sizeof(int64_t) * S);
      memcpy(w + 2 * E + 3 * S, step, sizeof(int64_t));
    }
  }
  return 0;
}

/* Wall-clock seconds, for the CPU-baseline timing in bench.py. */
double oracle_now(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ---------------------------------------------------------------------------------------
 * Fused manage + moe_align_block_size (kernels/expert_cache.hip:431-588, C-ABI :610-624).
 *
 * The manage half is the LRU rule only: a hit sets stamp = st and an install sets stamp = st
 * (:481, :505), there is no decay, and the policy argument does not exist. After it, both
 * align outputs are built from the updated table:
 *   hot  side: ids whose expert is resident, bucketed by slot   (bucket b in [0,S))
 *   cold side: ids whose expert is not resident, bucketed by expert id (bucket b in [0,E))
 * Per side: cnt[b] ids per bucket, padded to a multiple of bs; cum[b] the exclusive scan of
 * the padded counts; npad = cum[nb]; eids[cum[b]/bs .. cum[b+1]/bs) = b, the rest of eids[NB]
 * is -1; sorted[0..L) = mk except sorted[cum[b] + k] = the k-th id (in index order) of
 * bucket b. Ids outside [0,E) are skipped on both sides. Ordering within a bucket is by
 * token index, which is what the reference produces for mk <= 256 (:555-575).
 * ------------------------------------------------------------------------------------- */
static void align_side(int mk, const int32_t* key, int nb, int bs, int L, int NB,
                       int32_t* sorted, int32_t* eids, int32_t* npad) {
  int64_t* cum = (int64_t*)calloc((size_t)nb + 1, sizeof(int64_t));
  int64_t* cur = (int64_t*)calloc((size_t)nb + 1, sizeof(int64_t));
  int64_t* cnt = (int64_t*)calloc((size_t)nb + 1, sizeof(int64_t));
  for (int i = 0; i < mk; i++)
    if (key[i] >= 0 && key[i] < nb) cnt[key[i]]++;
  for (int b = 0; b < nb; b++) cum[b + 1] = cum[b] + ((cnt[b] + bs - 1) / bs) * bs;
  npad[0] = (int32_t)cum[nb];
  for (int i = 0; i < L; i++) sorted[i] = mk;
  for (int i = 0; i < NB; i++) eids[i] = -1;
  for (int b = 0; b < nb; b++)
    for (int64_t i = cum[b]; i < cum[b + 1]; i += bs)
      if (i / bs < NB) eids[i / bs] = b;
  for (int b = 0; b < nb; b++) cur[b] = cum[b];
  for (int i = 0; i < mk; i++) {
    const int b = key[i];
    if (b < 0 || b >= nb) continue;
    if (cur[b] < L) sorted[cur[b]] = i;
    cur[b]++;
  }
  free(cum);
  free(cur);
  free(cnt);
}

int oracle_fused(const int32_t* ids, int mk, int E, int S, int max_distinct, int max_inserts,
                 int32_t* table, int32_t* map_cold, int32_t* slot_expert, int64_t* slot_stamp,
                 uint8_t* routed, int64_t* step, int32_t* miss, int32_t* n_miss, int bs,
                 int L, int NB, int32_t* sorted_hot, int32_t* eids_hot, int32_t* npad_hot,
                 int32_t* sorted_cold, int32_t* eids_cold, int32_t* npad_cold) {
  /* argument checks of kernels/expert_cache.hip:616-618 */
  if (E <= 0 || E > OR_MAXE_FUSED || S <= 0 || S > OR_MAXS || S > OR_SLOT_MASK) return -1;
  if (bs <= 0 || L <= 0 || NB <= 0 || mk < 0) return -1;
  if (max_inserts < 0 || max_inserts > OR_MAXE_FUSED) return -1;

  /* manage half: the rank rule with policy 0 and no decay */
  int32_t misses[OR_MAXE_FUSED];
  int64_t st;
  const int nins = manage_front(ids, mk, E, S, max_distinct, max_inserts, table, map_cold,
                                slot_expert, slot_stamp, routed, step, miss, n_miss, 0, 0,
                                misses, &st);
  if (nins > 0) {
    int64_t key[OR_MAXS];
    uint8_t ev[OR_MAXS];
    int vic[OR_MAXE_FUSED];
    int nev = 0;
    for (int i = 0; i < S; i++) {
      ev[i] = (uint8_t)slot_evictable(slot_expert, routed, E, i);
      key[i] = vkey(slot_stamp[i], i);
      nev += ev[i];
    }
    for (int i = 0; i < S; i++) {
      if (!ev[i]) continue;
      int rank = 0;
      for (int j = 0; j < S; j++) rank += (ev[j] && key[j] < key[i]);
      if (rank < nins) vic[rank] = i;
    }
    const int nact = nins < nev ? nins : nev;
    for (int r = 0; r < nact; r++)
      install(r, vic[r], misses[r], st, E, table, map_cold, slot_expert, slot_stamp, miss);
    n_miss[0] = nact;
  }

  /* align half from the updated table */
  int32_t* kh = (int32_t*)malloc(sizeof(int32_t) * (size_t)(mk > 0 ? mk : 1));
  int32_t* kc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(mk > 0 ? mk : 1));
  for (int i = 0; i < mk; i++) {
    const int e = ids[i];
    kh[i] = kc[i] = -1;
    if (e < 0 || e >= E) continue;
    const int s = table[e];
    if ((unsigned)s < (unsigned)S)
      kh[i] = s;
    else
      kc[i] = e;
  }
  align_side(mk, kh, S, bs, L, NB, sorted_hot, eids_hot, npad_hot);
  align_side(mk, kc, E, bs, L, NB, sorted_cold, eids_cold, npad_cold);
  free(kh);
  free(kc);
  return 0;
}

/*
 * oracle_fused over a whole routing trace ids[T * mk] of one layer, with max_distinct =
 * min(E, mk) and max_inserts = S, for the CPU-baseline timing in bench.py. The align
 * outputs hold the last step's. Returns 0, or the first failing step's return code.
 */
int oracle_fused_trace(const int32_t* ids, int T, int mk, int E, int S, int bs, int L, int NB,
                       int32_t* table, int32_t* map_cold, int32_t* slot_expert,
                       int64_t* slot_stamp, uint8_t* routed, int64_t* step, int32_t* miss,
                       int32_t* n_miss, int32_t* sorted_hot, int32_t* eids_hot,
                       int32_t* npad_hot, int32_t* sorted_cold, int32_t* eids_cold,
                       int32_t* npad_cold) {
  if (T < 0 || mk < 0) return -1;
  const int md = mk < E ? mk : E;
  for (int t = 0; t < T; t++) {
    const int rc = oracle_fused(ids + (size_t)t * (size_t)mk, mk, E, S, md, S, table, map_cold,
                                slot_expert, slot_stamp, routed, step, miss, n_miss, bs, L, NB,
                                sorted_hot, eids_hot, npad_hot, sorted_cold, eids_cold,
                                npad_cold);
    if (rc != 0) return rc;
  }
  return 0;
}
