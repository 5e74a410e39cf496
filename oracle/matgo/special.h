/*
 * Oracle restatement (plain C), part 5: shake / bomb / grenade / bomb credit
 * (include/cugo/game/special50.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_SPECIAL_H_
#define CUGO_ORACLE_SPECIAL_H_

#include "game.h"

enum { SK_SHAKE = 0, SK_BOMB = 1, SK_GRENADE = 2, SK_BOMB_CREDIT = 3 };
enum { SP_OK = 0, SP_WRONG_PHASE, SP_INVALID_CARD, SP_INVALID_MONTH, SP_NOT_LEGAL, SP_STOCK_EMPTY,
       SP_RESOLVE_CHOICE_REQUIRED, SP_INVALID_RESOLVE_CHOICE, SP_PI_SELECTION_REQUIRED,
       SP_INVALID_PI_SELECTION };
enum { SE_SHAKE = 1, SE_BOMB = 2, SE_GRENADE = 4, SE_BOMB_CREDIT = 8, SE_SWEEP = 16 };

typedef struct {
  uint8_t status, events, actor, base, decision_opened, steal;
  card_t drawn;
  mask_t captured, stock_bonuses;
  PiResult pi;
} SpecialResult;

static uint16_t shaken_of(const Special* s, unsigned p) { return (p & 1u) == 0 ? s->shaken0 : s->shaken1; }
static uint16_t shaken4_of(const Special* s, unsigned p) { return (p & 1u) == 0 ? s->shaken4_0 : s->shaken4_1; }
static uint8_t bombs_of(const Special* s, unsigned p) { return (p & 1u) == 0 ? s->bombs0 : s->bombs1; }
static uint8_t credits_of(const Special* s, unsigned p) { return (p & 1u) == 0 ? s->credits0 : s->credits1; }
static mask_t month_of_mask(mask_t cards, unsigned m) { return m < MONTHS ? cards & month_cards(m) : 0; }

static int special_ready(const Special* s) { /* special50.h:65-68 */
  return !g_finished(&s->game) && !g_has_choice(&s->game) && s->game.turn.phase == PHASE_PLAY;
}

static uint16_t legal_special_months(const Special* s, int in_hand, int on_floor, int exclude_shaken) {
  /* special50.h:69-86 */
  if (!special_ready(s)) return 0;
  const Turn* t = &s->game.turn;
  const mask_t h = active_hand(t) & STD_MASK;
  const mask_t f = t->floor & STD_MASK;
  const uint16_t old = !exclude_shaken ? 0 : in_hand == 4 ? shaken4_of(s, t->actor) : shaken_of(s, t->actor);
  uint16_t out = 0;
  for (unsigned m = 0; m < MONTHS; ++m) {
    const uint16_t b = (uint16_t)(1u << m);
    if ((old & b) == 0 && ccount(month_of_mask(h, m)) == in_hand && ccount(month_of_mask(f, m)) == on_floor)
      out |= b;
  }
  return out;
}
static uint16_t legal_shake_months(const Special* s) {
  return (uint16_t)(legal_special_months(s, 3, 0, 1) | legal_special_months(s, 4, 0, 1));
}
static uint16_t legal_bomb_months(const Special* s) { return legal_special_months(s, 3, 1, 0); }
static uint16_t legal_grenade_months(const Special* s) { return legal_special_months(s, 2, 2, 0); }
static uint16_t forced_special_months(const Special* s) {
  return (uint16_t)(legal_bomb_months(s) | legal_grenade_months(s));
}
static uint8_t shake_count(const Special* s, unsigned p) {
  return (uint8_t)(ccount(shaken_of(s, p)) + ccount(shaken4_of(s, p)));
}
static uint64_t bomb_shake_multiplier(const Special* s, unsigned p) { /* special50.h:117-121 */
  uint8_t n = (uint8_t)(bombs_of(s, p) + shake_count(s, p));
  uint64_t x = 1;
  while (n--) x *= 2u;
  return x;
}

static SpecialResult special_error(uint8_t status) {
  SpecialResult r;
  memset(&r, 0, sizeof r);
  r.status = status;
  r.actor = NO_PLAYER;
  r.drawn = NO_CARD;
  return r;
}
static uint8_t pi_status_to_special(uint8_t s) {
  return s == PT_SELECTION_REQUIRED ? SP_PI_SELECTION_REQUIRED
       : s == PT_INVALID_SELECTION ? SP_INVALID_PI_SELECTION : SP_OK;
}

typedef struct { uint8_t status, events; card_t drawn; mask_t bonuses; Resolve resolve; } DrawOnly;

static DrawOnly draw_only_special(Turn* t, card_t choice) { /* special50.h:144-166 */
  DrawOnly d;
  memset(&d, 0, sizeof d);
  mask_t stock = t->stock;
  uint64_t rng = t->rng;
  const Flip f = draw_with_bonus_chain(&stock, &rng);
  if (!is_standard(f.card)) {
    d.status = SP_STOCK_EMPTY;
    d.drawn = NO_CARD;
    d.resolve = resolve_fail(RS_WRONG_PHASE);
    return d;
  }
  t->stock = stock;
  t->rng = rng;
  Resolve rr;
  memset(&rr, 0, sizeof rr);
  rr.last_turn = (uint8_t)is_last_turn(t);
  const uint8_t rs = resolve_against_floor(t, f.card, choice, &rr);
  d.drawn = f.card;
  d.bonuses = f.bonuses;
  if (rs != RS_OK) {
    d.status = rs == RS_CHOICE_REQUIRED ? SP_RESOLVE_CHOICE_REQUIRED : SP_INVALID_RESOLVE_CHOICE;
    d.resolve = resolve_fail(rs);
    return d;
  }
  if (f.bonuses) capture_cards(t, f.bonuses, &rr);
  if (t->floor == 0 && rr.captured) {
    rr.events |= EV_SWEEP;
    d.events |= SE_SWEEP;
  }
  rr.status = RS_OK;
  d.status = SP_OK;
  d.resolve = rr;
  return d;
}

static void finish_draw_only(Turn* t) { /* special50.h:167-170 */
  t->pending_played = NO_CARD;
  t->pending_drawn = NO_CARD;
  t->pending_bonus = 0;
  t->phase = PHASE_PLAY;
  t->actor ^= 1u;
  ++t->turn_index;
}

static uint8_t begin_regular_play_game(Game* g, card_t card) { /* game50.h:240-245 */
  if (g_finished(g) || g_has_choice(g)) return TS_WRONG_PHASE;
  return begin_regular_play(&g->turn, card);
}
static uint8_t draw_for_game(Game* g) { /* game50.h:247-252 */
  if (g_finished(g) || g_has_choice(g)) return TS_WRONG_PHASE;
  return draw_for_turn(&g->turn);
}

static SpecialResult begin_shake(Special* s, card_t card) { /* special50.h:171-188 */
  if (!special_ready(s)) return special_error(SP_WRONG_PHASE);
  if (!is_standard(card)) return special_error(SP_INVALID_CARD);
  const unsigned m = cmonth(card);
  const uint16_t b = (uint16_t)(1u << m);
  if ((legal_shake_months(s) & b) == 0 || (active_hand(&s->game.turn) & cbit(card)) == 0)
    return special_error(SP_NOT_LEGAL);
  Special n = *s;
  const int four = ccount(month_of_mask(active_hand(&s->game.turn), m)) == 4;
  uint16_t* shaken = four ? (n.game.turn.actor == 0 ? &n.shaken4_0 : &n.shaken4_1)
                          : (n.game.turn.actor == 0 ? &n.shaken0 : &n.shaken1);
  *shaken |= b;
  if (begin_regular_play_game(&n.game, card) != TS_OK) return special_error(SP_NOT_LEGAL);
  *s = n;
  SpecialResult r = special_error(SP_OK);
  r.events = SE_SHAKE;
  return r;
}

static SpecialResult capture_special(Special* s, unsigned month, int grenade, card_t choice, mask_t sel) {
  /* special50.h:189-231 */
  if (!special_ready(s)) return special_error(SP_WRONG_PHASE);
  if (month >= MONTHS) return special_error(SP_INVALID_MONTH);
  const uint16_t b = (uint16_t)(1u << month);
  const uint16_t legal = grenade ? legal_grenade_months(s) : legal_bomb_months(s);
  if ((legal & b) == 0) return special_error(SP_NOT_LEGAL);
  Special n = *s;
  Turn* t = &n.game.turn;
  const unsigned actor = t->actor;
  mask_t* hand = hand_of(t, actor);
  const mask_t hc = month_of_mask(*hand, month), fc = month_of_mask(t->floor & STD_MASK, month);
  const mask_t immediate = hc | fc;
  *hand &= ~hc;
  t->floor &= ~fc;
  if (actor == 0) {
    t->captured0 |= immediate;
    n.credits0 = (uint8_t)(n.credits0 + (grenade ? 1u : 2u));
    if (!grenade) ++n.bombs0;
  } else {
    t->captured1 |= immediate;
    n.credits1 = (uint8_t)(n.credits1 + (grenade ? 1u : 2u));
    if (!grenade) ++n.bombs1;
  }
  const DrawOnly d = draw_only_special(t, choice);
  if (d.status != SP_OK) return special_error(d.status);
  const uint8_t steal = (uint8_t)((is_last_turn(t) ? 0u : 1u) + steal_count(&d.resolve));
  finish_draw_only(t);
  const PiResult pt = apply_pi_steal_state(t, actor, steal, sel);
  if (pt.status != PT_OK) {
    SpecialResult r = special_error(pi_status_to_special(pt.status));
    r.pi = pt; r.steal = steal; r.drawn = d.drawn; r.stock_bonuses = d.bonuses;
    return r;
  }
  const uint8_t score = base_score(&n.game, actor);
  const int opened = finish_turn_game(&n.game, actor);
  *s = n;
  SpecialResult r;
  r.status = SP_OK;
  r.events = (uint8_t)((grenade ? SE_GRENADE : SE_BOMB) | d.events);
  r.actor = (uint8_t)actor;
  r.base = score;
  r.decision_opened = (uint8_t)opened;
  r.steal = steal;
  r.drawn = d.drawn;
  r.captured = immediate | d.resolve.captured;
  r.stock_bonuses = d.bonuses;
  r.pi = pt;
  return r;
}

static SpecialResult play_bomb_credit(Special* s, card_t choice, mask_t sel) { /* special50.h:242-265 */
  if (!special_ready(s)) return special_error(SP_WRONG_PHASE);
  const unsigned actor = s->game.turn.actor;
  if (!credits_of(s, actor)) return special_error(SP_NOT_LEGAL);
  Special n = *s;
  if (actor == 0) --n.credits0; else --n.credits1;
  const DrawOnly d = draw_only_special(&n.game.turn, choice);
  if (d.status != SP_OK) return special_error(d.status);
  const uint8_t steal = steal_count(&d.resolve);
  finish_draw_only(&n.game.turn);
  const PiResult pt = apply_pi_steal_state(&n.game.turn, actor, steal, sel);
  if (pt.status != PT_OK) {
    SpecialResult r = special_error(pi_status_to_special(pt.status));
    r.pi = pt; r.steal = steal; r.drawn = d.drawn; r.stock_bonuses = d.bonuses;
    return r;
  }
  const uint8_t score = base_score(&n.game, actor);
  const int opened = finish_turn_game(&n.game, actor);
  *s = n;
  SpecialResult r;
  r.status = SP_OK;
  r.events = (uint8_t)(SE_BOMB_CREDIT | d.events);
  r.actor = (uint8_t)actor;
  r.base = score;
  r.decision_opened = (uint8_t)opened;
  r.steal = steal;
  r.drawn = d.drawn;
  r.captured = d.resolve.captured;
  r.stock_bonuses = d.bonuses;
  r.pi = pt;
  return r;
}

static SpecialResult apply_special(Special* s, uint8_t kind, card_t card, uint8_t month, card_t drawn_match,
                                   mask_t sel) { /* special50.h:266-274 */
  switch (kind) {
    case SK_SHAKE: return begin_shake(s, card);
    case SK_BOMB: return capture_special(s, month, 0, drawn_match, sel);
    case SK_GRENADE: return capture_special(s, month, 1, drawn_match, sel);
    case SK_BOMB_CREDIT: return play_bomb_credit(s, drawn_match, sel);
    default: return special_error(SP_NOT_LEGAL);
  }
}

#endif
