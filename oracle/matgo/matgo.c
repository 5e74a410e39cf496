/*
 * The oracle: a plain-C restatement of the reference Shin Matgo engine
 * (include/cugo/ headers) and of the batch operations of the reference PyTorch extension
 * (python/csrc/torch50_ext.cu:53-363), as CPU loops over 248-byte rows.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library (oracle/libcugo_oracle.so, through oracle/ref.py);
 * the product (cugo_amd/) never does.  Each function cites the reference file:line it
 * restates; the restatement is pinned against the reference's own build
 * (oracle/_ref, where it compiles) and against the golden fixtures in tests/golden/.
 *
 * Row semantics (python/csrc/torch50_ext.cu):
 *   invalid env id      -> zero observation, done=1, status=-1 (:71-87, :108-118)
 *   out-of-range action -> 0xFFFF, i.e. kNotLegal (:96-99)
 *   clone/branch        -> byte copy of the parent, zero row for an invalid id (:271-314)
 * Padding bytes of every row written here are zero.
 */
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <string.h>

#include "canonical.h"

#define ROW 248

static Env load_row(const uint8_t* row) {
  Env e;
  memcpy(&e, row, sizeof e);
  return e;
}

static void store_row(const Env* e, uint8_t* row) {
  memcpy(row, e, sizeof *e);
  for (int k = 0; k < 10; ++k) memset(row + kPadRanges[k][0], 0, (size_t)(kPadRanges[k][1] - kPadRanges[k][0]));
}

static void write_observation(const Env* e, float* f, uint8_t* legal, uint8_t* player, uint8_t* done,
                              int16_t* status) { /* torch50_ext.cu:53-69 */
  const Packet p = make_packet(e);
  encode_packet(&p, f);
  for (int a = 0; a < ACTIONS; ++a) legal[a] = (uint8_t)tm_has(p.legal, (unsigned)a);
  *player = p.player;
  *done = e->done != 0;
  *status = (int16_t)p.status;
}

static void write_invalid_observation(float* f, uint8_t* legal, uint8_t* player, uint8_t* done,
                                      int16_t* status) {
  memset(f, 0, sizeof(float) * FEATURES);
  memset(legal, 0, ACTIONS);
  *player = 0;
  *done = 1;
  *status = -1;
}

static uint16_t clamp_action(int64_t raw) { /* torch50_ext.cu:96-99 */
  return raw >= 0 && raw < ACTIONS ? (uint16_t)raw : (uint16_t)INVALID_TORCH_ACTION;
}

static void write_step(const StepResult* r, float* reward, uint8_t* done, uint8_t* nagari,
                       int16_t* status, uint8_t* committed) { /* torch50_ext.cu:89-106 */
  *reward = (float)r->reward0;
  *done = r->done != 0;
  *nagari = r->nagari != 0;
  *status = (int16_t)r->status;
  *committed = r->committed != 0;
}

static void write_invalid_step(float* reward, uint8_t* done, uint8_t* nagari, int16_t* status,
                               uint8_t* committed) {
  *reward = 0.0f;
  *done = 1;
  *nagari = 0;
  *status = -1;
  *committed = 0;
}

static int valid_id(int64_t id, int64_t env_count) { return id >= 0 && id < env_count; }

/* ---- a small pthread pool: body(ctx, i) for i in [0, n) in chunks of 64 ---- */
typedef void (*body_fn)(void* ctx, int64_t i);
typedef struct { body_fn body; void* ctx; int64_t n; _Atomic int64_t next; } Pool;

static void* pool_worker(void* arg) {
  Pool* p = (Pool*)arg;
  for (;;) {
    const int64_t begin = atomic_fetch_add(&p->next, 64);
    if (begin >= p->n) return NULL;
    const int64_t end = begin + 64 < p->n ? begin + 64 : p->n;
    for (int64_t i = begin; i < end; ++i) p->body(p->ctx, i);
  }
}

static void parallel_for(int64_t n, int threads, body_fn body, void* ctx) {
  Pool p;
  p.body = body;
  p.ctx = ctx;
  p.n = n;
  atomic_init(&p.next, 0);
  if (threads <= 1 || n < 2) {
    for (int64_t i = 0; i < n; ++i) body(ctx, i);
    return;
  }
  if (threads > 64) threads = 64;
  pthread_t tid[64];
  int started = 0;
  for (int t = 0; t < threads; ++t)
    if (pthread_create(&tid[t], NULL, pool_worker, &p) == 0) ++started;
  if (started == 0) pool_worker(&p);
  for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
}

static uint64_t fnv(uint64_t h, const void* data, size_t n) {
  const uint8_t* p = (const uint8_t*)data;
  for (size_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

static uint64_t splitmix_first(uint64_t seed) {
  uint64_t s = seed;
  const uint64_t v = splitmix_next(&s);
  return v != 0 ? v : 1;
}

static uint64_t xorshift_next(uint64_t* x) {
  *x ^= *x << 13;
  *x ^= *x >> 7;
  *x ^= *x << 17;
  return *x;
}

/* ======================================================================== API */

int cugo_oracle_state_bytes(void) { return (int)sizeof(Env); }

/* Threads of the batch loops below (1 by default).  Rows are independent, so a threaded
 * loop gives the sequential loop's outputs; step_indexed with ids stays sequential, since
 * duplicate ids step the same row in order. */
static int g_threads = 1;

void cugo_oracle_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }

typedef struct { const int64_t* seeds; const int64_t* first; uint8_t* states; } CreateCtx;

static void create_one(void* ctx, int64_t i) {
  const CreateCtx* c = (const CreateCtx*)ctx;
  const Env e = make_env((uint64_t)c->seeds[i], (unsigned)(c->first[i] & 1));
  store_row(&e, c->states + i * ROW);
}

void cugo_oracle_create(const int64_t* seeds, const int64_t* first, int64_t n, uint8_t* states) {
  CreateCtx c = {seeds, first, states};
  parallel_for(n, g_threads, create_one, &c);
}

typedef struct {
  const uint8_t* states; const int64_t* ids; int64_t env_count;
  float* features; uint8_t* legal; uint8_t* player; uint8_t* done; int16_t* status;
} ObserveCtx;

static void observe_one(void* ctx, int64_t i) {
  const ObserveCtx* c = (const ObserveCtx*)ctx;
  const int64_t id = c->ids ? c->ids[i] : i;
  if (!valid_id(id, c->env_count)) {
    write_invalid_observation(c->features + i * FEATURES, c->legal + i * ACTIONS, c->player + i,
                              c->done + i, c->status + i);
    return;
  }
  const Env e = load_row(c->states + id * ROW);
  write_observation(&e, c->features + i * FEATURES, c->legal + i * ACTIONS, c->player + i,
                    c->done + i, c->status + i);
}

void cugo_oracle_observe_indexed(const uint8_t* states, const int64_t* ids, int64_t n, int64_t env_count,
                                 float* features, uint8_t* legal, uint8_t* player, uint8_t* done,
                                 int16_t* status) {
  ObserveCtx c = {states, ids, env_count, features, legal, player, done, status};
  parallel_for(n, g_threads, observe_one, &c);
}

typedef struct {
  uint8_t* states; const int64_t* ids; const int64_t* actions; int64_t env_count;
  float* reward; uint8_t* done; uint8_t* nagari; int16_t* status; uint8_t* committed;
  int64_t* events;
} StepCtx;

static void step_one(void* ctx, int64_t i) {
  const StepCtx* c = (const StepCtx*)ctx;
  const int64_t id = c->ids ? c->ids[i] : i;
  int64_t ev[EVENT_WORDS] = {0};
  if (!valid_id(id, c->env_count)) {
    write_invalid_step(c->reward + i, c->done + i, c->nagari + i, c->status + i, c->committed + i);
  } else {
    Env e = load_row(c->states + id * ROW);
    const StepResult r = torch_step_event(&e, clamp_action(c->actions[i]), ev);
    store_row(&e, c->states + id * ROW);
    write_step(&r, c->reward + i, c->done + i, c->nagari + i, c->status + i, c->committed + i);
  }
  if (c->events) memcpy(c->events + i * EVENT_WORDS, ev, sizeof ev);
}

void cugo_oracle_step_indexed(uint8_t* states, const int64_t* ids, const int64_t* actions, int64_t n,
                              int64_t env_count, float* reward, uint8_t* done, uint8_t* nagari,
                              int16_t* status, uint8_t* committed, int64_t* events) {
  StepCtx c = {states, ids, actions, env_count, reward, done, nagari, status, committed, events};
  parallel_for(n, ids ? 1 : g_threads, step_one, &c);
}

void cugo_oracle_start(const uint8_t* states, int64_t n, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    const Env e = load_row(states + i * ROW);
    pack_start(&e, out + i * START_WORDS);
  }
}

void cugo_oracle_clone_indexed(const uint8_t* states, const int64_t* ids, int64_t n, int64_t env_count,
                               uint8_t* children) {
  for (int64_t i = 0; i < n; ++i) {
    if (valid_id(ids[i], env_count)) memcpy(children + i * ROW, states + ids[i] * ROW, ROW);
    else memset(children + i * ROW, 0, ROW);
  }
}

void cugo_oracle_branch_indexed(const uint8_t* states, const int64_t* ids, const int64_t* actions,
                                int64_t n, int64_t env_count, uint8_t* children, float* reward,
                                uint8_t* done, uint8_t* nagari, int16_t* status, uint8_t* committed) {
  for (int64_t i = 0; i < n; ++i) {
    if (!valid_id(ids[i], env_count)) {
      memset(children + i * ROW, 0, ROW);
      write_invalid_step(reward + i, done + i, nagari + i, status + i, committed + i);
      continue;
    }
    Env e = load_row(states + ids[i] * ROW);
    const StepResult r = torch_step(&e, clamp_action(actions[i]));
    store_row(&e, children + i * ROW);
    write_step(&r, reward + i, done + i, nagari + i, status + i, committed + i);
  }
}

void cugo_oracle_hands_indexed(const uint8_t* states, const int64_t* ids, int64_t n, int64_t env_count,
                               int64_t* hands) { /* torch50_ext.cu:316-334 */
  for (int64_t i = 0; i < n; ++i) {
    if (!valid_id(ids[i], env_count)) { hands[2 * i] = hands[2 * i + 1] = 0; continue; }
    const Env e = load_row(states + ids[i] * ROW);
    hands[2 * i] = (int64_t)e.g.sp.game.turn.hand0;
    hands[2 * i + 1] = (int64_t)e.g.sp.game.turn.hand1;
  }
}

void cugo_oracle_stock_indexed(const uint8_t* states, const int64_t* ids, int64_t n, int64_t env_count,
                               int64_t* stock) { /* torch50_ext.cu:336-363: stops at a bonus card */
  for (int64_t i = 0; i < n; ++i) {
    uint64_t packed = ~0ull;
    if (valid_id(ids[i], env_count)) {
      const Env e = load_row(states + ids[i] * ROW);
      mask_t remaining = e.g.sp.game.turn.stock;
      uint64_t rng = e.g.sp.game.turn.rng;
      for (int k = 0; k < 8; ++k) {
        const card_t c = draw_stock_card(&remaining, &rng);
        if (!is_standard(c)) break;
        packed &= ~(0xffull << (8 * k));
        packed |= (uint64_t)c << (8 * k);
      }
    }
    stock[i] = (int64_t)packed;
  }
}

int64_t cugo_oracle_reward0(const uint8_t* row) {
  const Env e = load_row(row);
  return torch_reward0(&e);
}

/* Random-policy protocol: game i from seed base+i, first=i&1; each decision takes
 * legal[xorshift64() % count] over the ascending legal list, sampler state
 * SplitMix64(seed).next(); full observe + step_events per decision.  Per game: FNV-1a
 * digest of the record stream, decision count, exact final reward of player 0.
 * Record layout:
 *   [features f32 x720][mask u8 x179][player u8][done u8][status i16][action i64]
 *   [reward f32][done u8][nagari u8][status i16][committed u8][events i64 x9] */
enum { RECORD_BYTES = FEATURES * 4 + ACTIONS + 1 + 1 + 2 + 8 + 4 + 1 + 1 + 2 + 1 + EVENT_WORDS * 8 };

int cugo_oracle_record_bytes(void) { return RECORD_BYTES; }

typedef struct {
  uint64_t base_seed;
  uint64_t* digest;
  int32_t* steps;
  int64_t* final_reward;
  uint8_t* records;
  int64_t record_games;
  int32_t record_cap;
  _Atomic int64_t total;
} PlayCtx;

static void play_one(void* arg, int64_t i) {
  PlayCtx* c = (PlayCtx*)arg;
  const uint64_t seed = c->base_seed + (uint64_t)i;
  Env e = make_env(seed, (unsigned)(i & 1));
  uint64_t x = splitmix_first(seed);
  uint64_t h = 0xcbf29ce484222325ull;
  uint8_t rec[RECORD_BYTES];
  int32_t count = 0;
  while (e.done == 0 && count < 512) {
    float* f = (float*)(void*)rec;
    uint8_t* legal = rec + FEATURES * 4;
    uint8_t* o = legal + ACTIONS;
    int16_t ostatus;
    write_observation(&e, f, legal, o, o + 1, &ostatus);
    memcpy(o + 2, &ostatus, 2);
    uint16_t list[ACTIONS];
    int m = 0;
    for (int a = 0; a < ACTIONS; ++a)
      if (legal[a]) list[m++] = (uint16_t)a;
    const int64_t action = m ? (int64_t)list[xorshift_next(&x) % (unsigned)m] : -1;
    memcpy(o + 4, &action, 8);
    int64_t words[EVENT_WORDS];
    const StepResult s = torch_step_event(&e, clamp_action(action), words);
    uint8_t* q = o + 12;
    float reward;
    uint8_t sd, sn, sc;
    int16_t ss;
    write_step(&s, &reward, &sd, &sn, &ss, &sc);
    memcpy(q, &reward, 4);
    q[4] = sd;
    q[5] = sn;
    memcpy(q + 6, &ss, 2);
    q[8] = sc;
    memcpy(q + 9, words, sizeof words);
    if (c->digest) h = fnv(h, rec, RECORD_BYTES);
    if (c->records && i < c->record_games && count < c->record_cap)
      memcpy(c->records + ((size_t)i * (size_t)c->record_cap + (size_t)count) * RECORD_BYTES, rec, RECORD_BYTES);
    ++count;
    if (m == 0) break;
  }
  if (c->digest) c->digest[i] = h;
  if (c->steps) c->steps[i] = count;
  if (c->final_reward) c->final_reward[i] = torch_reward0(&e);
  atomic_fetch_add(&c->total, count);
}

int64_t cugo_oracle_play_random(uint64_t base_seed, int64_t n, int threads, uint64_t* digest, int32_t* steps,
                                int64_t* final_reward, uint8_t* records, int64_t record_games,
                                int32_t record_cap) {
  PlayCtx c;
  c.base_seed = base_seed;
  c.digest = digest;
  c.steps = steps;
  c.final_reward = final_reward;
  c.records = records;
  c.record_games = record_games;
  c.record_cap = record_cap;
  atomic_init(&c.total, 0);
  parallel_for(n, threads, play_one, &c);
  return atomic_load(&c.total);
}

/* Branch workload: child i = clone(roots[ids[i]]) stepped with actions[i], optionally
 * observed into a scratch row; returns a checksum so the work is not elided. */
typedef struct {
  const uint8_t* roots;
  const int64_t* ids;
  const int64_t* actions;
  int observe;
  _Atomic uint64_t sum;
} BranchCtx;

static void branch_one(void* arg, int64_t i) {
  BranchCtx* c = (BranchCtx*)arg;
  Env e = load_row(c->roots + c->ids[i] * ROW);
  const StepResult r = torch_step(&e, clamp_action(c->actions[i]));
  uint64_t local = (uint64_t)r.status + e.g.sp.game.turn.stock;
  if (c->observe) {
    float f[FEATURES];
    uint8_t legal[ACTIONS], player, done;
    int16_t status;
    write_observation(&e, f, legal, &player, &done, &status);
    uint32_t bits;
    memcpy(&bits, &f[453], 4);
    local += bits + legal[0] + player;
  }
  atomic_fetch_add(&c->sum, local);
}

uint64_t cugo_oracle_branch_work(const uint8_t* roots, const int64_t* ids, const int64_t* actions, int64_t n,
                                 int threads, int observe) {
  BranchCtx c;
  c.roots = roots;
  c.ids = ids;
  c.actions = actions;
  c.observe = observe;
  atomic_init(&c.sum, 0);
  parallel_for(n, threads, branch_one, &c);
  return atomic_load(&c.sum);
}

/* ---- rule-level entry points for the reference's known-answer tests ---- */

/* score_captured (hwatu.h:153-199) -> 10 bytes in ScoreBreakdown field order */
void cugo_oracle_score(uint64_t cards, int gukjin_as_pi, uint8_t* out) {
  const Score s = score_captured(cards, gukjin_as_pi);
  const uint8_t v[10] = {s.bright_count, s.animal_count, s.ribbon_count, s.pi_units, s.bright_points,
                         s.animal_points, s.ribbon_points, s.pi_points, s.flags, s.total};
  memcpy(out, v, 10);
}

/* go_adjusted_score50 (game50.h:136-147): points after go */
uint64_t cugo_oracle_go_points(uint8_t base, uint8_t go_count) { return go_adjusted_points(base, go_count); }

/* settle_terminal50 (settlement50.h:95-208) of a row: status, winner, final points, side */
void cugo_oracle_settle(const uint8_t* row, int64_t* out) {
  const Env e = load_row(row);
  const Settlement st = settle(&e.g);
  out[0] = st.status;
  out[1] = st.winner;
  out[2] = (int64_t)st.final_points;
  out[3] = st.side0;
}

/* rollout_canonical_torch50 (torch50.h:598-619) from seeds[i] / first[i] with at most
 * max_actions primary actions: five digest words a game (pack_canonical). */
typedef struct { const int64_t* seeds; const int64_t* first; int max_actions; int64_t* out; } CanonCtx;

static void canonical_one(void* arg, int64_t i) {
  const CanonCtx* c = (const CanonCtx*)arg;
  const CanonicalResult r = rollout_canonical_torch((uint64_t)c->seeds[i], (unsigned)(c->first[i] & 1),
                                                    (uint16_t)c->max_actions);
  pack_canonical(&r, c->out + 5 * i);
}

void cugo_oracle_rollout_canonical(const int64_t* seeds, const int64_t* first, int64_t n, int max_actions,
                                   int threads, int explicit_form, int64_t* out) {
  (void)explicit_form; /* the oracle restates the torch form only */
  CanonCtx c = {seeds, first, max_actions, out};
  parallel_for(n, threads, canonical_one, &c);
}

/* For the canonical driver's probes: over n games from seed base + i * 0x9E3779B97F4A7C15
 * (first = i & 1) played with the canonical action (random_policy = 0) or a uniform
 * random legal action (xorshift64 from SplitMix64(i), random_policy = 1), counts the
 * decision states outside a pending choice (out[0]) and those where canonical_action50's
 * probe status is not kOk (out[1]).  random_policy = 2 plays the canonical action but
 * probes a copy of each state whose stock is emptied (a planted failure for the tests). */
typedef struct { uint64_t base; int random_policy; _Atomic int64_t states, failures; } ProbeCtx;

static void probe_one(void* arg, int64_t i) {
  ProbeCtx* c = (ProbeCtx*)arg;
  Env e = make_env(c->base + (uint64_t)i * 0x9E3779B97F4A7C15ull, (unsigned)(i & 1));
  uint64_t x = splitmix_first((uint64_t)i);
  int64_t states = 0, failures = 0;
  while (!e.done && e.n_primary < 128) {
    if (!e.pending.active) {
      ++states;
      Terminal probed = e.g;
      if (c->random_policy == 2) probed.sp.game.turn.stock = 0; /* planted: nothing to draw */
      if (canonical_action(&probed).status != AS_OK) ++failures;
    }
    uint16_t a = INVALID_TORCH_ACTION;
    if (c->random_policy != 1) {
      a = canonical_torch_action(&e);
    } else {
      const Packet p = make_packet(&e);
      uint16_t list[ACTIONS];
      int count = 0;
      for (unsigned k = 0; k < ACTIONS; ++k)
        if (tm_has(p.legal, k)) list[count++] = (uint16_t)k;
      if (count) a = list[xorshift_next(&x) % (uint64_t)count];
    }
    if (a == INVALID_TORCH_ACTION || torch_step(&e, a).status != AS_OK) break;
  }
  atomic_fetch_add(&c->states, states);
  atomic_fetch_add(&c->failures, failures);
}

void cugo_oracle_canonical_probe_failures(uint64_t base, int64_t n, int random_policy, int threads,
                                          int64_t* out) {
  ProbeCtx c;
  c.base = base;
  c.random_policy = random_policy;
  atomic_init(&c.states, 0);
  atomic_init(&c.failures, 0);
  parallel_for(n, threads, probe_one, &c);
  out[0] = atomic_load(&c.states);
  out[1] = atomic_load(&c.failures);
}
