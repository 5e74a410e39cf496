/*
 * Oracle restatement (plain C), part 9: decision kind, the 127-bit primary mask and the
 * information-set observation (include/cugo/game/policy50.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_POLICY_H_
#define CUGO_ORACLE_POLICY_H_

#include "apply.h"

enum { PA_PLAY_BONUS = 48, PA_SHAKE = 50, PA_BOMB = 98, PA_GRENADE = 110, PA_BOMB_CREDIT = 122,
       PA_GO = 123, PA_STOP = 124, PA_CT_WIN = 125, PA_CT_CONTINUE = 126, PA_COUNT = 127,
       PA_GUKJIN_PI = 177, PA_GUKJIN_ANIMAL = 178, PA_INVALID = 0xffff };
enum { DK_NONE = 0, DK_PRIMARY = 1, DK_GO_STOP = 2, DK_CHONGTONG = 3, DK_GUKJIN = 7 };

typedef struct { uint64_t lo, hi; } PrimaryMask;

static void pm_set(PrimaryMask* m, unsigned a) {
  if (a >= PA_COUNT) return;
  if (a < 64u) m->lo |= (uint64_t)1 << a; else m->hi |= (uint64_t)1 << (a - 64u);
}
static int pm_has(PrimaryMask m, unsigned a) {
  if (a >= PA_COUNT) return 0;
  return a < 64u ? (int)((m.lo >> a) & 1u) : (int)((m.hi >> (a - 64u)) & 1u);
}

static uint8_t decision_kind(const Terminal* s) { /* policy50.h:151-160 */
  if (t_finished(s)) return DK_NONE;
  if (t_has_ct_choice(s)) return DK_CHONGTONG;
  if (g_has_gukjin(&s->sp.game)) return DK_GUKJIN;
  if (g_has_decision(&s->sp.game)) return DK_GO_STOP;
  if (s->sp.game.turn.phase == PHASE_PLAY) return DK_PRIMARY;
  return DK_NONE;
}

static uint8_t decision_player(const Terminal* s) { /* policy50.h:161-170 */
  if (t_finished(s)) return NO_PLAYER;
  if (t_has_ct_choice(s)) return s->ct_actor;
  if (g_has_gukjin(&s->sp.game)) return g_gukjin_actor(&s->sp.game);
  if (g_has_decision(&s->sp.game)) return s->sp.game.decision_actor;
  return s->sp.game.turn.actor;
}

static PrimaryMask legal_primary(const Terminal* s) { /* policy50.h:173-236 */
  PrimaryMask m = {0, 0};
  const uint8_t dk = decision_kind(s);
  if (dk == DK_CHONGTONG) { pm_set(&m, PA_CT_WIN); pm_set(&m, PA_CT_CONTINUE); return m; }
  if (dk == DK_GO_STOP) { pm_set(&m, PA_GO); pm_set(&m, PA_STOP); return m; }
  if (dk != DK_PRIMARY) return m;
  const Turn* t = &s->sp.game.turn;
  const unsigned actor = t->actor;
  const mask_t hand = active_hand(t);
  if (t->stock == 0) return m;
  const uint16_t forced = forced_special_months(&s->sp);
  mask_t std_cards = hand & STD_MASK;
  while (std_cards) {
    const card_t c = pop_first(&std_cards);
    if (forced & (uint16_t)(1u << cmonth(c))) continue;
    pm_set(&m, c);
  }
  if (hand & cbit(BONUS2)) pm_set(&m, PA_PLAY_BONUS);
  if (hand & cbit(BONUS3)) pm_set(&m, PA_PLAY_BONUS + 1u);
  const uint16_t shake = legal_shake_months(&s->sp);
  mask_t shake_cards = hand & STD_MASK;
  while (shake_cards) {
    const card_t c = pop_first(&shake_cards);
    if (shake & (uint16_t)(1u << cmonth(c))) pm_set(&m, PA_SHAKE + c);
  }
  const uint16_t bombs = legal_bomb_months(&s->sp), grenades = legal_grenade_months(&s->sp);
  for (unsigned month = 0; month < MONTHS; ++month) {
    const uint16_t b = (uint16_t)(1u << month);
    if (bombs & b) pm_set(&m, PA_BOMB + month);
    if (grenades & b) pm_set(&m, PA_GRENADE + month);
  }
  if (credits_of(&s->sp, actor)) pm_set(&m, PA_BOMB_CREDIT);
  return m;
}

static mask_t pending_public(const Turn* t) { /* policy50.h:339-346 */
  mask_t c = t->pending_bonus;
  if (is_standard(t->pending_played)) c |= cbit(t->pending_played);
  if (is_standard(t->pending_drawn)) c |= cbit(t->pending_drawn);
  return c;
}

static uint8_t first_player(const Turn* t) { return (uint8_t)((t->actor ^ t->turn_index) & 1u); }

static uint32_t stop_points(const Terminal* s) { /* policy50.h:354-365 */
  if (decision_kind(s) != DK_GO_STOP) return 0;
  Terminal stopped = *s;
  if (terminal_go_stop(&stopped, STOP) != GS_OK || !t_finished(&stopped)) return 0;
  const Settlement st = settle(&stopped);
  if (st.status != SETTLE_OK) return 0;
  return st.final_points > 0xffffffffull ? 0xffffffffu : (uint32_t)st.final_points;
}

/* PolicyObservation50 (policy50.h:49-120): only what the 720-feature encoder reads */
typedef struct {
  mask_t own_hand, floor, own_cap, opp_cap, pending_public, unseen;
  uint16_t own_shaken, opp_shaken, ppuk, own_ppuk, opp_ppuk, b2ppuk, b3ppuk, ct_months, turn;
  uint8_t decision_kind, stock_count, own_go, opp_go, own_lgo, opp_lgo, own_base, opp_base;
  uint8_t own_bombs, opp_bombs, own_cred, opp_cred, own_pcount, opp_pcount, own_streak, opp_streak;
  uint8_t own_gdp, opp_gdp;
  mask_t mission;
  int32_t own_side;
  uint8_t mtype, mmult, own_mm, opp_mm, own_locked, opp_locked, round, last_turn;
  uint16_t neutral;
  mask_t own_played, opp_played, opp_known;
  uint8_t own_first, opp_hand_count, own_pi, opp_pi, own_bright, opp_bright;
  uint8_t own_animal, opp_animal, own_ribbon, opp_ribbon;
  uint32_t stop_points;
} Observation;

static Observation pack_observation(const Terminal* s) { /* policy50.h:367-467 */
  Observation o;
  memset(&o, 0, sizeof o);
  const Turn* t = &s->sp.game.turn;
  unsigned player = decision_player(s);
  if (player > 1u) player = t->actor & 1u;
  const unsigned opp = player ^ 1u;
  o.own_hand = player == 0 ? t->hand0 : t->hand1;
  o.own_cap = captured_of(t, player);
  o.opp_cap = captured_of(t, opp);
  o.pending_public = pending_public(t);
  const mask_t known = o.own_hand | t->floor | o.own_cap | o.opp_cap | o.pending_public;
  const mask_t opp_revealed = player == 0 ? s->revealed1 : s->revealed0;
  o.opp_known = opp_revealed & DECK_MASK & ~known;
  o.unseen = DECK_MASK & ~known & ~o.opp_known;
  const mask_t own_held = player == 0 ? s->held0 : s->held1;
  const mask_t opp_held = player == 0 ? s->held1 : s->held0;
  const mask_t opp_hand = player == 0 ? t->hand1 : t->hand0;
  const uint16_t owner1 = (uint16_t)(t->owner1 & ALL_MONTH_BITS);
  const uint16_t owner0 = (uint16_t)(t->ppuk_months & (uint16_t)~owner1);
  const uint16_t sh0 = (uint16_t)(s->sp.shaken0 | s->sp.shaken4_0);
  const uint16_t sh1 = (uint16_t)(s->sp.shaken1 | s->sp.shaken4_1);
  const Score own = score_player(t, player), oth = score_player(t, opp);
  o.floor = t->floor;
  o.own_shaken = player == 0 ? sh0 : sh1;
  o.opp_shaken = player == 0 ? sh1 : sh0;
  o.ppuk = t->ppuk_months;
  o.own_ppuk = player == 0 ? owner0 : owner1;
  o.opp_ppuk = player == 0 ? owner1 : owner0;
  o.b2ppuk = t->bonus2_ppuk;
  o.b3ppuk = t->bonus3_ppuk;
  o.ct_months = s->ct_months;
  o.turn = t->turn_index;
  o.decision_kind = decision_kind(s);
  o.stock_count = (uint8_t)ccount(t->stock);
  o.own_go = go_count_of(&s->sp.game, player);
  o.opp_go = go_count_of(&s->sp.game, opp);
  o.own_lgo = last_go_of(&s->sp.game, player);
  o.opp_lgo = last_go_of(&s->sp.game, opp);
  o.own_base = own.total;
  o.opp_base = oth.total;
  o.own_bombs = bombs_of(&s->sp, player);
  o.opp_bombs = bombs_of(&s->sp, opp);
  o.own_cred = credits_of(&s->sp, player);
  o.opp_cred = credits_of(&s->sp, opp);
  o.own_pcount = player == 0 ? s->ppuk_count0 : s->ppuk_count1;
  o.opp_pcount = player == 0 ? s->ppuk_count1 : s->ppuk_count0;
  o.own_streak = player == 0 ? s->streak0 : s->streak1;
  o.opp_streak = player == 0 ? s->streak1 : s->streak0;
  o.own_gdp = (uint8_t)gukjin_role_pi(t, player);
  o.opp_gdp = (uint8_t)gukjin_role_pi(t, opp);
  o.mission = t->mission;
  o.own_side = player == 0 ? s->side0 : -s->side0;
  o.mtype = s->mission_type;
  o.mmult = s->mission_mult;
  o.own_mm = mission_multi_of(s, player);
  o.opp_mm = mission_multi_of(s, opp);
  o.own_locked = (uint8_t)gukjin_locked(t, player);
  o.opp_locked = (uint8_t)gukjin_locked(t, opp);
  o.round = round_mult(s);
  o.last_turn = (uint8_t)is_last_turn(t);
  o.neutral = t->neutral_ppuk;
  o.own_played = own_held & ~o.own_hand;
  o.opp_played = opp_held & ~opp_hand;
  o.own_first = (uint8_t)(first_player(t) == player);
  o.opp_hand_count = (uint8_t)ccount(opp_hand);
  o.own_pi = own.pi_units;
  o.opp_pi = oth.pi_units;
  o.own_bright = own.bright_count;
  o.opp_bright = oth.bright_count;
  o.own_animal = own.animal_count;
  o.opp_animal = oth.animal_count;
  o.own_ribbon = own.ribbon_count;
  o.opp_ribbon = oth.ribbon_count;
  o.stop_points = stop_points(s);
  return o;
}

#endif
