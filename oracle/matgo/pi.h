/*
 * Oracle restatement (plain C), part 3: automatic pi transfer
 * (include/cugo/game/pi_transfer.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_PI_H_
#define CUGO_ORACLE_PI_H_

#include "turn.h"

enum { PT_OK = 0, PT_SELECTION_REQUIRED = 1, PT_INVALID_SELECTION = 2 };

typedef struct {
  uint8_t status, requested, available, transferred, transferred_units;
  mask_t transferred_mask;
} PiResult;

static PiResult pi_result(uint8_t status, uint8_t requested, uint8_t available) {
  PiResult r;
  memset(&r, 0, sizeof r);
  r.status = status;
  r.requested = requested;
  r.available = available;
  return r;
}

static uint8_t steal_count(const Resolve* r) { /* pi_transfer.h:51-62 */
  if (r->status != RS_OK || r->last_turn) return 0;
  unsigned n = (unsigned)r->opp_ppuk + 2u * (unsigned)r->own_ppuk;
  if (r->events & EV_JJOK) ++n;
  if (r->events & EV_TTADAK) ++n;
  if (r->events & EV_SWEEP) ++n;
  n += (unsigned)ccount(r->captured & BONUS_MASK);
  return (uint8_t)n;
}

static uint8_t pi_card_value(card_t c) { /* pi_transfer.h:79-84 */
  if (c == BONUS3) return 3;
  if (c == BONUS2 || c == GUKJIN || (DOUBLE_PI_MASK & cbit(c))) return 2;
  return 1;
}

/* pi_transfer.h:90-111: lowest value first, non-mission before mission (or all
 * non-mission first when the victim owns every mission card), then card id. */
static mask_t steal_selection(mask_t candidates, mask_t mission, int owns_mission, uint8_t count) {
  mask_t chosen = 0;
  for (int key = 0; key < 6 && count != 0; ++key) {
    const int is_mission = owns_mission ? key >= 3 : (key & 1) != 0;
    const uint8_t value = (uint8_t)(owns_mission ? 1 + key % 3 : 1 + key / 2);
    mask_t pool = candidates & (is_mission ? mission : ~mission);
    while (pool != 0 && count != 0) {
      const card_t c = pop_first(&pool);
      if (pi_card_value(c) != value) continue;
      chosen |= cbit(c);
      --count;
    }
  }
  return chosen;
}

static PiResult apply_pi_steal(Turn* t, unsigned thief_player, uint8_t requested,
                               mask_t selection, int victim_gukjin_pi) {
  /* pi_transfer.h:125-210 */
  thief_player &= 1u;
  const unsigned victim_player = thief_player ^ 1u;
  mask_t* thief = cap_ref(t, thief_player);
  mask_t* victim = cap_ref(t, victim_player);
  const mask_t candidates = pi_card_mask(*victim, victim_gukjin_pi);
  const uint8_t available = (uint8_t)ccount(candidates);
  if (requested == 0) return pi_result(PT_OK, 0, available);
  if (available == 0) {
    decide_gukjin(t, victim_player, 0);
    return pi_result(PT_OK, requested, available);
  }
  if (available > requested && selection == 0) {
    const int owns = t->mission != 0 && (t->mission & ~*victim) == 0;
    selection = steal_selection(candidates, t->mission, owns, requested);
  }
  const uint8_t required = requested < available ? requested : available;
  mask_t transfer;
  if (available <= requested) {
    if (selection != 0 && selection != candidates)
      return pi_result(PT_INVALID_SELECTION, requested, available);
    transfer = candidates;
  } else {
    if (selection == 0) return pi_result(PT_SELECTION_REQUIRED, requested, available);
    if ((selection & ~candidates) != 0 || ccount(selection) != required)
      return pi_result(PT_INVALID_SELECTION, requested, available);
    transfer = selection;
  }
  *victim &= ~transfer;
  *thief |= transfer;
  if (transfer & cbit(GUKJIN)) /* pi_transfer.h:66-77: the double-pi role stays behind */
    t->owner1 &= (uint16_t)~(gukjin_pi_flag(thief_player) | gukjin_pi_flag(victim_player));
  if (available < requested) decide_gukjin(t, victim_player, 0);
  PiResult r = pi_result(PT_OK, requested, available);
  r.transferred = (uint8_t)ccount(transfer);
  r.transferred_units = pi_units(transfer, victim_gukjin_pi);
  r.transferred_mask = transfer;
  return r;
}

/* apply_pi_steal50 with the victim's persistent score options (pi_transfer.h:212-222) */
static PiResult apply_pi_steal_state(Turn* t, unsigned thief_player, uint8_t requested, mask_t selection) {
  return apply_pi_steal(t, thief_player, requested, selection, gukjin_as_pi(t, (thief_player & 1u) ^ 1u));
}

typedef struct { Resolve resolve; PiResult pi; } ResolvePi;

/* pi_transfer.h:232-254 with state options */
static ResolvePi resolve_turn_with_pi(Turn* t, card_t pc, card_t dc, mask_t pi_sel) {
  ResolvePi out;
  Turn next = *t;
  const unsigned thief = t->actor;
  out.resolve = resolve_turn(&next, pc, dc);
  if (out.resolve.status != RS_OK) {
    out.pi = pi_result(PT_OK, 0, 0);
    return out;
  }
  out.pi = apply_pi_steal_state(&next, thief, steal_count(&out.resolve), pi_sel);
  if (out.pi.status != PT_OK) return out;
  *t = next;
  return out;
}

typedef struct { TurnBonus play; PiResult pi; } BonusPi;

/* pi_transfer.h:270-291 with state options */
static BonusPi play_bonus_with_pi(Turn* t, card_t bonus, mask_t pi_sel) {
  BonusPi out;
  Turn next = *t;
  const unsigned thief = t->actor;
  out.play = play_bonus_for_turn(&next, bonus);
  if (out.play.status != TS_OK) {
    out.pi = pi_result(PT_OK, 0, 0);
    return out;
  }
  out.pi = apply_pi_steal_state(&next, thief, out.play.steal, pi_sel);
  if (out.pi.status != PT_OK) return out;
  *t = next;
  return out;
}

#endif
