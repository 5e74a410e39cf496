/*
 * Oracle restatement (plain C), part 11: the torch contract - 179-way action mask,
 * 720-float observation, unified step, event and start records
 * (include/cugo/game/torch50.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_TORCH_H_
#define CUGO_ORACLE_TORCH_H_

#include <math.h>

#include "postchance.h"

enum { FEATURES = 720, ACTIONS = 179, CHOICE_BEGIN = 127, GUKJIN_BEGIN = 177, EVENT_WORDS = 9,
       START_WORDS = 8 };
#define INVALID_TORCH_ACTION 0xffffu

typedef struct {
  Observation obs;
  uint64_t legal[3];
  mask_t selected_pi;
  uint16_t primary_action;
  card_t revealed;
  uint8_t requested_pi, player, decision_kind, status;
} Packet;

static void tm_set(uint64_t* m, unsigned a) { /* torch50.h:142-149 */
  if (a >= ACTIONS) return;
  m[a >> 6] |= (uint64_t)1 << (a & 63u);
}
static int tm_has(const uint64_t* m, unsigned a) {
  if (a >= ACTIONS) return 0;
  return (int)((m[a >> 6] >> (a & 63u)) & 1u);
}

static int hands_exhausted(const Terminal* s) { /* rollout50.h:576-582 */
  return s->sp.game.turn.phase == PHASE_PLAY && s->sp.game.turn.hand0 == 0 &&
         s->sp.game.turn.hand1 == 0 && s->sp.credits0 == 0 && s->sp.credits1 == 0;
}

static int nagari_ready(const Env* e) { /* torch50.h:196-201 */
  return e->pending.active == 0 && !t_finished(&e->g) && !t_has_ct_choice(&e->g) &&
         !g_has_choice(&e->g.sp.game) && hands_exhausted(&e->g);
}

static void refresh_done(Env* e) { /* torch50.h:203-216 */
  if (t_finished(&e->g)) { e->done = 1; e->nagari = 0; return; }
  if (nagari_ready(e)) { e->done = 1; e->nagari = 1; return; }
  e->done = 0;
  e->nagari = 0;
}

static Env make_env(uint64_t seed, unsigned first) { /* torch50.h:218-236 */
  Env e;
  memset(&e, 0, sizeof e);
  e.g = make_terminal_state(deal_50(seed), first & 1u);
  e.status = AS_OK;
  refresh_done(&e);
  return e;
}

static Packet make_packet(const Env* e) { /* torch50.h:245-296 */
  Packet p;
  memset(&p, 0, sizeof p);
  if (e->pending.active) {
    Terminal staged;
    memset(&staged, 0, sizeof staged);
    const Probe pr = probe_postchance(&e->g, &e->pending, &staged);
    p.selected_pi = e->pending.selected_pi;
    p.primary_action = e->pending.primary_action;
    p.revealed = pr.revealed;
    p.requested_pi = pr.requested_pi;
    p.player = e->pending.actor;
    if (pr.status != AS_OK) {
      p.decision_kind = PC_NONE;
      p.status = pr.status;
      return p; /* zero observation, empty mask */
    }
    p.obs = pack_postchance_observation(&e->g, &staged, &e->pending, &pr);
    mask_t cards = pr.legal_cards & DECK_MASK;
    while (cards) tm_set(p.legal, CHOICE_BEGIN + pop_first(&cards));
    p.decision_kind = pr.decision;
    p.status = AS_OK;
    return p;
  }
  p.obs = pack_observation(&e->g);
  const PrimaryMask pm = legal_primary(&e->g);
  unsigned player = decision_player(&e->g);
  if (player > 1u) player = e->g.sp.game.turn.actor & 1u;
  const int gukjin = p.obs.decision_kind == DK_GUKJIN;
  if (!e->done) {
    if (gukjin) { tm_set(p.legal, GUKJIN_BEGIN); tm_set(p.legal, GUKJIN_BEGIN + 1u); }
    else { p.legal[0] = pm.lo; p.legal[1] = pm.hi; }
  }
  p.selected_pi = 0;
  p.primary_action = PA_INVALID;
  p.revealed = NO_CARD;
  p.requested_pi = 0;
  p.player = (uint8_t)player;
  p.decision_kind = e->done ? 0 : p.obs.decision_kind;
  p.status = AS_OK;
  return p;
}

static float unit(uint32_t value, uint32_t scale) { /* torch50.h:298-303 */
  if (scale == 0) return 0.0f;
  const float r = (float)value / (float)scale;
  return r > 1.0f ? 1.0f : r;
}

static void card_plane(float* f, int offset, mask_t cards) {
  for (int c = 0; c < DECK_CARDS; ++c) f[offset + c] = (cards >> c) & 1u ? 1.0f : 0.0f;
}
static void month_plane(float* f, int offset, uint16_t months) {
  for (int m = 0; m < MONTHS; ++m) f[offset + m] = (months >> m) & 1u ? 1.0f : 0.0f;
}

static void encode_packet(const Packet* p, float* f) { /* torch50.h:334-470 */
  for (int i = 0; i < FEATURES; ++i) f[i] = 0.0f;
  const Observation* o = &p->obs;
  const mask_t planes[6] = {o->own_hand, o->floor, o->own_cap, o->opp_cap, o->pending_public, o->unseen};
  for (int k = 0; k < 6; ++k) card_plane(f, k * DECK_CARDS, planes[k]);
  const uint16_t months[8] = {o->own_shaken, o->opp_shaken, o->ppuk, o->own_ppuk,
                              o->opp_ppuk, o->b2ppuk, o->b3ppuk, o->ct_months};
  for (int k = 0; k < 8; ++k) month_plane(f, 300 + k * MONTHS, months[k]);
  int choices = 0;
  for (int c = 0; c < DECK_CARDS; ++c) {
    const int legal = tm_has(p->legal, CHOICE_BEGIN + (unsigned)c);
    f[396 + c] = legal ? 1.0f : 0.0f;
    choices += legal;
  }
  if (p->decision_kind >= 1u && p->decision_kind <= 5u) f[446 + p->decision_kind] = 1.0f;
  f[446] = o->own_first ? 1.0f : 0.0f;
  f[452] = unit(o->opp_hand_count, 10);
  float* s = f + 453;
  s[0] = unit(o->turn, 32);
  s[1] = unit(o->stock_count, 30);
  s[2] = unit(o->own_go, 8);
  s[3] = unit(o->opp_go, 8);
  s[4] = unit(o->own_lgo, 64);
  s[5] = unit(o->opp_lgo, 64);
  s[6] = unit(o->own_base, 64);
  s[7] = unit(o->opp_base, 64);
  s[8] = unit(o->own_bombs, 4);
  s[9] = unit(o->opp_bombs, 4);
  s[10] = unit(o->own_cred, 4);
  s[11] = unit(o->opp_cred, 4);
  s[12] = unit(o->own_pcount, 3);
  s[13] = unit(o->opp_pcount, 3);
  s[14] = unit(o->own_streak <= 3u ? o->own_streak : 0u, 3);
  s[15] = unit(o->opp_streak <= 3u ? o->opp_streak : 0u, 3);
  s[16] = o->own_gdp ? 1.0f : 0.0f;
  s[17] = o->opp_gdp ? 1.0f : 0.0f;
  {
    const float bits = log2f(1.0f + (float)o->stop_points) / 12.0f;
    s[18] = bits > 1.0f ? 1.0f : bits;
  }
  s[19] = p->primary_action < PA_COUNT ? (float)(p->primary_action + 1u) / (float)PA_COUNT : 0.0f;
  s[20] = is_physical(p->revealed) ? (float)(p->revealed + 1u) / (float)DECK_CARDS : 0.0f;
  s[21] = unit(o->own_pi, 20);
  s[22] = unit((uint32_t)choices, 50);
  s[23] = unit((uint32_t)ccount(o->own_hand), 50);
  s[24] = unit((uint32_t)ccount(o->floor), 50);
  s[25] = unit((uint32_t)ccount(o->unseen), 50);
  for (int c = 0; c < STD_CARDS; ++c) f[496 + c] = (o->mission >> c) & 1u ? 1.0f : 0.0f;
  float* x = f + 544;
  x[0] = o->mtype == MISSION_EASY ? 1.0f : 0.0f;
  x[1] = o->mtype == MISSION_NORMAL ? 1.0f : 0.0f;
  x[2] = o->mtype == MISSION_HARD ? 1.0f : 0.0f;
  x[3] = o->mtype == MISSION_NO_CONDITION ? 1.0f : 0.0f;
  x[4] = o->mtype == MISSION_TRIPLE ? 1.0f : 0.0f;
  x[5] = unit(o->mmult, 4);
  x[6] = unit(o->own_mm, 8);
  x[7] = unit(o->opp_mm, 8);
  x[8] = p->decision_kind == DK_GUKJIN ? 1.0f : 0.0f;
  x[9] = o->own_locked ? 1.0f : 0.0f;
  x[10] = o->opp_locked ? 1.0f : 0.0f;
  x[11] = o->last_turn ? 1.0f : 0.0f;
  const float side = (float)o->own_side / 64.0f;
  x[12] = side > 1.0f ? 1.0f : side < -1.0f ? -1.0f : side;
  x[13] = unit(o->round, 8);
  x[14] = o->own_streak == PPUK_FIRST || o->own_streak == PPUK_SECOND ? 1.0f : 0.0f;
  x[15] = o->opp_streak == PPUK_FIRST || o->opp_streak == PPUK_SECOND ? 1.0f : 0.0f;
  month_plane(f, 479, o->neutral);
  float* t = f + 491;
  t[0] = unit(o->opp_pi, 20);
  t[1] = unit(o->own_bright, 5);
  t[2] = unit(o->opp_bright, 5);
  t[3] = unit(o->own_animal, 10);
  t[4] = unit(o->opp_animal, 10);
  f[710] = unit(o->own_ribbon, 10);
  f[711] = unit(o->opp_ribbon, 10);
  card_plane(f, 560, o->own_played);
  card_plane(f, 610, o->opp_played);
  card_plane(f, 660, o->opp_known);
}

static int64_t torch_reward0(const Env* e) { /* torch50.h:472-478 */
  if (!e->done) return 0;
  if (e->nagari) return nagari_reward(&e->g, 0);
  if (!t_finished(&e->g)) return 0;
  const Settlement st = settle(&e->g);
  return settlement_reward(&st, 0);
}

static void record_primary(Env* e, uint8_t kind) { /* torch50.h:480-489 */
  ++e->n_primary;
  if (kind == AK_PLAY_BONUS) ++e->n_bonus;
  if (kind == AK_SHAKE || kind == AK_BOMB || kind == AK_GRENADE || kind == AK_BOMB_CREDIT) ++e->n_special;
  if (kind == AK_GO) ++e->n_go;
}

typedef struct {
  uint8_t status;
  int64_t reward0;
  uint8_t done, nagari, committed;
} StepResult;

static StepResult torch_step(Env* e, uint16_t action) { /* torch50.h:491-540 */
  StepResult r = {AS_OK, 0, 0, 0, 0};
  if (e->done) {
    e->status = AS_GAME_FINISHED;
    r.status = e->status; r.reward0 = torch_reward0(e); r.done = e->done; r.nagari = e->nagari;
    return r;
  }
  const Packet p = make_packet(e);
  if (p.status != AS_OK) {
    e->status = p.status;
    r.status = e->status; r.done = e->done; r.nagari = e->nagari;
    return r;
  }
  if (!tm_has(p.legal, action)) {
    e->status = AS_NOT_LEGAL;
    r.status = e->status; r.done = e->done; r.nagari = e->nagari;
    return r;
  }
  PcStep step;
  if (e->pending.active) {
    const card_t card = (card_t)(action - CHOICE_BEGIN);
    if (p.decision_kind == PC_PI_CARD) ++e->n_pi; else ++e->n_resolve;
    ++e->n_choice;
    step = choose_postchance_card(&e->g, &e->pending, card);
  } else {
    step = start_postchance_action(&e->g, action, &e->pending);
  }
  if (step.status != AS_OK) {
    e->status = step.status;
    r.status = e->status; r.done = e->done; r.nagari = e->nagari;
    return r;
  }
  if (step.committed) {
    record_primary(e, e->pending.action.kind);
    r.committed = 1;
  }
  e->status = AS_OK;
  refresh_done(e);
  r.status = AS_OK;
  r.reward0 = torch_reward0(e);
  r.done = e->done;
  r.nagari = e->nagari;
  return r;
}

/* torch50.h:644-678: the committed action's table-wide difference */
static void make_event(const Env* before, const Env* after, int64_t* out) {
  const Turn* b = &before->g.sp.game.turn;
  const Turn* a = &after->g.sp.game.turn;
  const unsigned actor = after->pending.actor & 1u;
  const mask_t hb = actor == 0 ? b->hand0 : b->hand1, ha = actor == 0 ? a->hand0 : a->hand1;
  const mask_t rb = actor == 0 ? before->g.revealed0 : before->g.revealed1;
  const mask_t ra = actor == 0 ? after->g.revealed0 : after->g.revealed1;
  const mask_t played = hb & ~ha, drawn = ha & ~hb;
  out[0] = (int64_t)played;
  out[1] = (int64_t)drawn;
  out[2] = (int64_t)(b->stock & ~a->stock & ~drawn);
  out[3] = (int64_t)(a->captured0 & ~b->captured0);
  out[4] = (int64_t)(a->captured1 & ~b->captured1);
  out[5] = (int64_t)(b->captured0 & ~a->captured0);
  out[6] = (int64_t)(b->captured1 & ~a->captured1);
  out[7] = (int64_t)(ra & ~rb);
  out[8] = (int64_t)actor | ((int64_t)after->pending.action.kind << 8);
}

static StepResult torch_step_event(Env* e, uint16_t action, int64_t* event) { /* torch50.h:701-707 */
  const Env before = *e;
  const StepResult r = torch_step(e, action);
  if (r.committed) make_event(&before, e, event);
  else for (int k = 0; k < EVENT_WORDS; ++k) event[k] = 0;
  return r;
}

static void pack_start(const Env* e, int64_t* out) { /* torch50.h:684-698 */
  const Turn* t = &e->g.sp.game.turn;
  out[0] = (int64_t)t->hand0;
  out[1] = (int64_t)t->hand1;
  out[2] = (int64_t)t->floor;
  out[3] = (int64_t)t->captured0;
  out[4] = (int64_t)t->captured1;
  out[5] = (int64_t)t->mission;
  out[6] = (int64_t)t->neutral_ppuk;
  out[7] = (int64_t)e->g.mission_type | ((int64_t)e->g.mission_mult << 8) |
           ((int64_t)(t->actor & 1u) << 16) | ((int64_t)e->g.mm0 << 24) | ((int64_t)e->g.mm1 << 32);
}

#endif
