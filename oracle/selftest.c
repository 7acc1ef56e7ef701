/*
 * Self-test of the CPU oracle (policy.c), built with AddressSanitizer and UndefinedBehavior-
 * Sanitizer by tests/test_oracle_sanitized.py (or `make -C oracle selftest`).
 *
 * TEST INFRASTRUCTURE ONLY, like policy.c. Random shapes -- E from 1 to 1100, S from 1 to
 * 1024 (also S > E), 0 to 700 ids with padding and out-of-range values, insert caps from
 * 0 to 1024, stamps spread to the limits of int64 -- drive:
 *   - the policy step under both victim rules, compared field by field after every step
 *     while no stamp reaches 2^43 (beyond it the key stamp << 20 | slot that the reference's
 *     kernel compares overflows, and the serial rule's (stamp, slot) pair order is a different
 *     order; the rank rule is the kernel's), with the state invariants checked always;
 *   - the prefetch step under both rules, likewise;
 *   - the fused step (block sizes 1 to 17) with its output lengths as vLLM allocates them;
 *   - remap of int32 and int64 ids.
 * Any out-of-bounds access or undefined operation stops the run with a sanitizer report;
 * a rule mismatch or broken invariant exits with status 1.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int oracle_manage_serial(const int32_t*, int, int, int, int, int, int32_t*, int32_t*, int32_t*,
                         int64_t*, uint8_t*, int64_t*, int32_t*, int32_t*, int, int);
int oracle_manage_rank(const int32_t*, int, int, int, int, int, int32_t*, int32_t*, int32_t*,
                       int64_t*, uint8_t*, int64_t*, int32_t*, int32_t*, int, int);
int oracle_prefetch(const int32_t*, int, int, int, int, int32_t*, int32_t*, int32_t*, int64_t*,
                    uint8_t*, int32_t*, int32_t*, int);
int oracle_fused(const int32_t*, int, int, int, int, int, int32_t*, int32_t*, int32_t*, int64_t*,
                 uint8_t*, int64_t*, int32_t*, int32_t*, int, int, int, int32_t*, int32_t*,
                 int32_t*, int32_t*, int32_t*, int32_t*);
void oracle_remap_i32(const int32_t*, int, const int32_t*, int, int32_t*);
void oracle_remap_i64(const int64_t*, int, const int32_t*, int, int64_t*);

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}
static int pick(const int* v, int n) { return v[next_u64() % (uint64_t)n]; }
static int range(int lo, int hi) { return lo + (int)(next_u64() % (uint64_t)(hi - lo)); }

typedef struct {
  int E, S, cap;
  int32_t *table, *map_cold, *slot_expert, *miss, *n_miss;
  int64_t *slot_stamp, *step;
  uint8_t* routed;
} St;

static void st_alloc(St* s, int E, int S, int cap) {
  s->E = E;
  s->S = S;
  s->cap = cap;
  s->table = malloc(sizeof(int32_t) * E);
  s->map_cold = malloc(sizeof(int32_t) * E);
  s->slot_expert = malloc(sizeof(int32_t) * S);
  s->slot_stamp = malloc(sizeof(int64_t) * S);
  s->routed = malloc((size_t)E);
  s->step = malloc(sizeof(int64_t));
  s->miss = malloc(sizeof(int32_t) * 2 * cap);
  s->n_miss = malloc(sizeof(int32_t));
}

static void st_free(St* s) {
  free(s->table);
  free(s->map_cold);
  free(s->slot_expert);
  free(s->slot_stamp);
  free(s->routed);
  free(s->step);
  free(s->miss);
  free(s->n_miss);
}

static void st_copy(St* d, const St* s) {
  memcpy(d->table, s->table, sizeof(int32_t) * s->E);
  memcpy(d->map_cold, s->map_cold, sizeof(int32_t) * s->E);
  memcpy(d->slot_expert, s->slot_expert, sizeof(int32_t) * s->S);
  memcpy(d->slot_stamp, s->slot_stamp, sizeof(int64_t) * s->S);
  memcpy(d->routed, s->routed, (size_t)s->E);
  memcpy(d->step, s->step, sizeof(int64_t));
  memcpy(d->miss, s->miss, sizeof(int32_t) * 2 * s->cap);
  memcpy(d->n_miss, s->n_miss, sizeof(int32_t));
}

static int st_equal(const St* a, const St* b) {
  return !memcmp(a->table, b->table, sizeof(int32_t) * a->E) &&
         !memcmp(a->map_cold, b->map_cold, sizeof(int32_t) * a->E) &&
         !memcmp(a->slot_expert, b->slot_expert, sizeof(int32_t) * a->S) &&
         !memcmp(a->slot_stamp, b->slot_stamp, sizeof(int64_t) * a->S) &&
         !memcmp(a->routed, b->routed, (size_t)a->E) && a->step[0] == b->step[0] &&
         !memcmp(a->miss, b->miss, sizeof(int32_t) * 2 * a->cap) && a->n_miss[0] == b->n_miss[0];
}

/* table and map_cold complementary, no expert in two slots, table[slot_expert[s]] == s */
static int invariants(const St* s) {
  int resident = 0;
  for (int e = 0; e < s->E; e++) {
    const int t = s->table[e];
    if (t >= 0) {
      if (s->map_cold[e] != -1 || t >= s->S || s->slot_expert[t] != e) return 0;
      resident++;
    } else if (s->map_cold[e] != e) {
      return 0;
    }
  }
  int live = 0;
  for (int i = 0; i < s->S; i++)
    if (s->slot_expert[i] >= 0) live++;
  return live == resident;
}

/* a random consistent warm state; returns whether every stamp is small (|stamp| < 2^43
 * after the run's growth, so no victim key overflows) */
static int warm(St* s) {
  for (int e = 0; e < s->E; e++) {
    s->table[e] = -1;
    s->map_cold[e] = e;
  }
  for (int i = 0; i < s->S; i++) s->slot_expert[i] = -1;
  const int nhot = range(0, (s->S < s->E ? s->S : s->E) + 1);
  for (int k = 0; k < nhot; k++) {
    int e, sl;
    do e = range(0, s->E); while (s->table[e] >= 0);
    do sl = range(0, s->S); while (s->slot_expert[sl] >= 0);
    s->table[e] = sl;
    s->map_cold[e] = -1;
    s->slot_expert[sl] = e;
  }
  const int kind = range(0, 3);
  for (int i = 0; i < s->S; i++) {
    const uint64_t r = next_u64();
    s->slot_stamp[i] = kind == 0 ? (int64_t)(r % 1000)
                       : kind == 1 ? (int64_t)(r >> 1)        /* up to 2^63 - 1 */
                                   : (int64_t)r;              /* any sign */
  }
  memset(s->routed, 0, (size_t)s->E);
  s->step[0] = (int64_t)(next_u64() % 100000);
  memset(s->miss, 0, sizeof(int32_t) * 2 * s->cap);
  s->n_miss[0] = 0;
  return kind == 0;
}

static int fail(const char* what, int c, int t) {
  fprintf(stderr, "selftest: %s differs (case %d step %d)\n", what, c, t);
  exit(1);
}

int main(int argc, char** argv) {
  const int cases = argc > 1 ? atoi(argv[1]) : 300;
  static const int Es[] = {1, 2, 7, 64, 128, 257, 512, 1000, 1024, 1100};
  static const int Ss[] = {1, 2, 3, 16, 63, 64, 65, 129, 300, 513, 1024};
  static const int mks[] = {0, 1, 8, 33, 64, 200, 257, 700};
  for (int c = 0; c < cases; c++) {
    const int E = pick(Es, 10), S = pick(Ss, 11), mk = pick(mks, 8);
    const int caps[] = {0, 1, 4, S, 1024};
    const int mi = pick(caps, 5), cap = mi > 1 ? mi : 1;
    const int policy = range(0, 2);
    static const int decays[] = {0, 1, 3, 64};
    const int decay = pick(decays, 4);
    St a, b;
    st_alloc(&a, E, S, cap);
    st_alloc(&b, E, S, cap);
    const int small = warm(&a);
    st_copy(&b, &a);
    int32_t* ids = malloc(sizeof(int32_t) * (mk > 0 ? mk : 1));
    for (int t = 0; t < 8; t++) {
      for (int i = 0; i < mk; i++) ids[i] = range(-3, E + 3);
      const int md = range(-1, E + 2);
      if (t % 3 == 2) { /* a prefetch step, both rules */
        if (oracle_prefetch(ids, mk, E, S, mi, a.table, a.map_cold, a.slot_expert, a.slot_stamp,
                            a.routed, a.miss, a.n_miss, 0) ||
            oracle_prefetch(ids, mk, E, S, mi, b.table, b.map_cold, b.slot_expert, b.slot_stamp,
                            b.routed, b.miss, b.n_miss, 1))
          return fail("prefetch return", c, t);
      } else {
        if (oracle_manage_serial(ids, mk, E, S, md, mi, a.table, a.map_cold, a.slot_expert,
                                 a.slot_stamp, a.routed, a.step, a.miss, a.n_miss, policy,
                                 decay) ||
            oracle_manage_rank(ids, mk, E, S, md, mi, b.table, b.map_cold, b.slot_expert,
                               b.slot_stamp, b.routed, b.step, b.miss, b.n_miss, policy, decay))
          return fail("manage return", c, t);
      }
      if (small && !st_equal(&a, &b)) return fail("serial vs rank state", c, t);
      if (!small) st_copy(&a, &b); /* continue both from the kernel's (rank) order */
      if (!invariants(&a)) return fail("invariants", c, t);
      /* remap of the same ids, int32 and int64 */
      int32_t* o32 = malloc(sizeof(int32_t) * (mk > 0 ? mk : 1));
      int64_t* i64 = malloc(sizeof(int64_t) * (mk > 0 ? mk : 1));
      int64_t* o64 = malloc(sizeof(int64_t) * (mk > 0 ? mk : 1));
      for (int i = 0; i < mk; i++) i64[i] = ids[i];
      oracle_remap_i32(ids, mk, a.table, E, o32);
      oracle_remap_i64(i64, mk, a.table, E, o64);
      for (int i = 0; i < mk; i++)
        if ((int64_t)o32[i] != o64[i]) return fail("remap i32 vs i64", c, t);
      free(o32);
      free(i64);
      free(o64);
    }
    /* fused, on a fresh cold state, when the shape is one it accepts */
    if (E <= 1024 && mi <= 1024) {
      const int bs = range(1, 18);
      const long Ll = mk < E ? (mk * bs < mk + E * (bs - 1) ? (long)mk * bs
                                                           : (long)mk + (long)E * (bs - 1))
                             : (long)mk + (long)E * (bs - 1);
      const int L = Ll > 0 ? (int)Ll : 1, NB = (L + bs - 1) / bs;
      St f;
      st_alloc(&f, E, S, S);
      warm(&f);
      int32_t *sh = malloc(sizeof(int32_t) * L), *eh = malloc(sizeof(int32_t) * NB);
      int32_t *sc = malloc(sizeof(int32_t) * L), *ec = malloc(sizeof(int32_t) * NB);
      int32_t nh, nc;
      for (int t = 0; t < 3; t++) {
        for (int i = 0; i < mk; i++) ids[i] = range(-3, E + 3);
        if (oracle_fused(ids, mk, E, S, mk < E ? mk : E, S, f.table, f.map_cold,
                         f.slot_expert, f.slot_stamp, f.routed, f.step, f.miss, f.n_miss, bs, L,
                         NB, sh, eh, &nh, sc, ec, &nc))
          return fail("fused return", c, t);
        if (!invariants(&f)) return fail("fused invariants", c, t);
        if (nh % bs || nc % bs) return fail("fused padding", c, t);
      }
      free(sh);
      free(eh);
      free(sc);
      free(ec);
      st_free(&f);
    }
    free(ids);
    st_free(&a);
    st_free(&b);
  }
  printf("selftest: %d cases passed\n", cases);
  return 0;
}
