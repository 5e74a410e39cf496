/*
 * Oracle restatement (plain C), part 2: turn mechanics (include/cugo/game/turn50.h).
 * TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_TURN_H_
#define CUGO_ORACLE_TURN_H_

#include "cards.h"

#define LAST_TURN_INDEX 18 /* turn50.h:27 */

typedef struct {
  uint8_t status, events, own_ppuk, opp_ppuk;
  mask_t captured;
  uint8_t last_turn;
} Resolve;

static uint16_t floor_triple_months(mask_t floor) { /* turn50.h:139-147 */
  uint16_t months = 0;
  for (unsigned m = 0; m < MONTHS; ++m)
    if (ccount(floor & month_cards(m)) == 3) months |= (uint16_t)(1u << m);
  return months;
}

/* turn50.h:150-167: floor bonuses to the first player, refill from the stock */
static void refill_initial_floor_bonuses(Deal* d, unsigned first) {
  const mask_t bonuses = d->floor & BONUS_MASK;
  d->floor &= ~bonuses;
  if ((first & 1u) == 0) d->captured0 |= bonuses; else d->captured1 |= bonuses;
  int missing = ccount(bonuses);
  if (missing == 0) return;
  uint64_t s = d->rng;
  while (missing > 0 && d->stock != 0) {
    const card_t c = draw_uniform_card(&d->stock, &s);
    if (is_bonus(c)) {
      if ((first & 1u) == 0) d->captured0 |= cbit(c); else d->captured1 |= cbit(c);
      continue;
    }
    d->floor |= cbit(c);
    --missing;
  }
  d->rng = s;
}

static Turn make_turn_state(Deal d, unsigned first) { /* turn50.h:169-192 */
  refill_initial_floor_bonuses(&d, first);
  Turn t;
  memset(&t, 0, sizeof t);
  t.hand0 = d.hand0; t.hand1 = d.hand1; t.floor = d.floor; t.stock = d.stock;
  t.captured0 = d.captured0; t.captured1 = d.captured1; t.rng = d.rng;
  t.actor = (uint8_t)(first & 1u);
  t.phase = PHASE_PLAY;
  t.pending_played = NO_CARD;
  t.pending_drawn = NO_CARD;
  t.neutral_ppuk = floor_triple_months(d.floor & STD_MASK);
  return t;
}

static int is_last_turn(const Turn* t) { return t->turn_index >= LAST_TURN_INDEX; }
static int auto_floor_choice(mask_t matches) { /* turn50.h:200-202 */
  return ccount(matches) == 2 && (matches & ~plain_pi_mask()) == 0;
}
static mask_t* hand_of(Turn* t, unsigned p) { return (p & 1u) == 0 ? &t->hand0 : &t->hand1; }
static mask_t* cap_ref(Turn* t, unsigned p) { return (p & 1u) == 0 ? &t->captured0 : &t->captured1; }
static mask_t active_hand(const Turn* t) { return t->actor == 0 ? t->hand0 : t->hand1; }
static mask_t floor_matches(const Turn* t, card_t c) {
  return (t->floor & STD_MASK) & month_cards(cmonth(c));
}
static mask_t ppuk_bonus_for_month(const Turn* t, uint16_t mb) {
  mask_t r = 0;
  if (t->bonus2_ppuk & mb) r |= cbit(BONUS2);
  if (t->bonus3_ppuk & mb) r |= cbit(BONUS3);
  return r;
}
static void clear_ppuk_bonus(Turn* t, uint16_t mb) {
  t->bonus2_ppuk &= (uint16_t)~mb;
  t->bonus3_ppuk &= (uint16_t)~mb;
}
static void attach_pending_bonuses(Turn* t, uint16_t mb) {
  if (t->pending_bonus & cbit(BONUS2)) t->bonus2_ppuk |= mb;
  if (t->pending_bonus & cbit(BONUS3)) t->bonus3_ppuk |= mb;
}

typedef struct { uint8_t status; card_t replacement; uint8_t steal; } TurnBonus;

static TurnBonus play_bonus_for_turn(Turn* t, card_t bonus) { /* turn50.h:245-276 */
  TurnBonus r = {TS_WRONG_PHASE, NO_CARD, 0};
  if (t->phase != PHASE_PLAY) return r;
  const BonusPlay b = play_hand_bonus(hand_of(t, t->actor), &t->stock, cap_ref(t, t->actor),
                                      &t->rng, bonus);
  switch (b.status) {
    case BP_OK:
      r.status = TS_OK;
      r.replacement = b.replacement;
      r.steal = is_last_turn(t) ? 0 : b.steal;
      return r;
    case BP_NOT_IN_HAND: r.status = TS_NOT_IN_HAND; return r;
    case BP_STOCK_EMPTY: r.status = TS_STOCK_EMPTY; return r;
    default: r.status = TS_INVALID_CARD; return r;
  }
}

static uint8_t begin_regular_play(Turn* t, card_t card) { /* turn50.h:278-295 */
  if (t->phase != PHASE_PLAY) return TS_WRONG_PHASE;
  if (!is_standard(card)) return TS_INVALID_CARD;
  mask_t* hand = hand_of(t, t->actor);
  if ((*hand & cbit(card)) == 0) return TS_NOT_IN_HAND;
  *hand &= ~cbit(card);
  t->pending_played = card;
  t->pending_drawn = NO_CARD;
  t->pending_bonus = 0;
  t->phase = PHASE_DRAW;
  return TS_OK;
}

static uint8_t draw_for_turn(Turn* t) { /* turn50.h:296-311 */
  if (t->phase != PHASE_DRAW) return TS_WRONG_PHASE;
  mask_t stock = t->stock;
  uint64_t rng = t->rng;
  const Flip f = draw_with_bonus_chain(&stock, &rng);
  if (!is_standard(f.card)) return TS_STOCK_EMPTY;
  t->stock = stock;
  t->rng = rng;
  t->pending_drawn = f.card;
  t->pending_bonus = f.bonuses;
  t->phase = PHASE_RESOLVE;
  return TS_OK;
}

static void record_ppuk_capture(Turn* t, card_t c, Resolve* r) { /* turn50.h:317-331 */
  const uint16_t mb = month_bit(c);
  if ((t->ppuk_months & mb) == 0) return;
  const unsigned owner = (t->owner1 & mb) ? 1u : 0u;
  if (owner == t->actor) ++r->own_ppuk; else ++r->opp_ppuk;
  t->ppuk_months &= (uint16_t)~mb;
  t->owner1 &= (uint16_t)~mb;
}

static void capture_cards(Turn* t, mask_t cards, Resolve* r) { /* turn50.h:332-341 */
  *cap_ref(t, t->actor) |= cards;
  r->captured |= cards;
}

static uint8_t resolve_against_floor(Turn* t, card_t card, card_t choice, Resolve* r) {
  /* turn50.h:342-383 */
  const mask_t matches = floor_matches(t, card);
  const int n = ccount(matches);
  if (n == 0) {
    t->floor |= cbit(card);
    return RS_OK;
  }
  mask_t take = 0;
  if (n == 1) {
    take = matches;
  } else if (n == 2) {
    if (auto_floor_choice(matches) && (choice == NO_CARD || (matches & cbit(choice)) == 0))
      choice = first_of(matches);
    if (choice == NO_CARD) return RS_CHOICE_REQUIRED;
    if (!is_standard(choice) || (matches & cbit(choice)) == 0) return RS_INVALID_CHOICE;
    take = cbit(choice);
  } else {
    take = matches;
    const uint16_t mb = month_bit(card);
    if (t->ppuk_months & mb) {
      take |= ppuk_bonus_for_month(t, mb);
      clear_ppuk_bonus(t, mb);
      record_ppuk_capture(t, card, r);
    } else if (t->neutral_ppuk & mb) {
      t->neutral_ppuk &= (uint16_t)~mb;
      ++r->opp_ppuk;
    }
  }
  t->floor &= ~take;
  capture_cards(t, take | cbit(card), r);
  return RS_OK;
}

static void finish_resolved_turn(Turn* t) { /* turn50.h:384-391 */
  t->pending_played = NO_CARD;
  t->pending_drawn = NO_CARD;
  t->pending_bonus = 0;
  t->phase = PHASE_PLAY;
  t->actor ^= 1u;
  ++t->turn_index;
}

static Resolve resolve_fail(uint8_t status) {
  Resolve r;
  memset(&r, 0, sizeof r);
  r.status = status;
  return r;
}

/* turn50.h:418-508: resolve the played and the flipped card on a copy, commit on success */
static Resolve resolve_turn(Turn* t, card_t played_choice, card_t drawn_choice) {
  Resolve r = resolve_fail(RS_WRONG_PHASE);
  if (t->phase != PHASE_RESOLVE) return r;
  Turn next = *t;
  const card_t played = next.pending_played, drawn = next.pending_drawn;
  const mask_t pm = floor_matches(&next, played);
  const int pmc = ccount(pm);
  const int same = cmonth(played) == cmonth(drawn);
  const int last = is_last_turn(&next);
  r.last_turn = (uint8_t)last;
  if (same && pmc == 1) {
    if (last) {
      uint8_t st = resolve_against_floor(&next, played, played_choice, &r);
      if (st != RS_OK) return resolve_fail(st);
      st = resolve_against_floor(&next, drawn, drawn_choice, &r);
      if (st != RS_OK) return resolve_fail(st);
      if (next.pending_bonus) capture_cards(&next, next.pending_bonus, &r);
    } else {
      next.floor |= cbit(played) | cbit(drawn) | next.pending_bonus;
      const uint16_t mb = month_bit(played);
      next.ppuk_months |= mb;
      if (next.actor == 0) next.owner1 &= (uint16_t)~mb; else next.owner1 |= mb;
      attach_pending_bonuses(&next, mb);
      r.events |= EV_PPUK;
    }
  } else if (same && pmc == 2) {
    next.floor &= ~pm;
    capture_cards(&next, pm | cbit(played) | cbit(drawn) | next.pending_bonus, &r);
    r.events |= EV_TTADAK;
  } else if (same && pmc == 0) {
    capture_cards(&next, cbit(played) | cbit(drawn) | next.pending_bonus, &r);
    if (!last) r.events |= EV_JJOK;
  } else {
    uint8_t st = resolve_against_floor(&next, played, played_choice, &r);
    if (st != RS_OK) return resolve_fail(st);
    st = resolve_against_floor(&next, drawn, drawn_choice, &r);
    if (st != RS_OK) return resolve_fail(st);
    if (next.pending_bonus) capture_cards(&next, next.pending_bonus, &r);
  }
  if (next.floor == 0 && r.captured != 0) r.events |= EV_SWEEP;
  finish_resolved_turn(&next);
  *t = next;
  r.status = RS_OK;
  return r;
}

#endif
