/*
 * Oracle restatement (plain C), part 11: the deterministic canonical driver
 * (include/cugo/game/rollout50.h:138-179, 400-715 and torch50.h:542-619).
 * TEST INFRASTRUCTURE ONLY.
 *
 * The torch form of the driver turns the canonical Action50 into its primary action
 * index (policy50.h:238-271), which carries kind, card and month only: the resolve
 * choices and pi selection that canonicalize_* fill in are dropped.  What reaches the
 * result of each canonicalize_* probe is therefore its status, and that is what the
 * probes below compute.
 */
#ifndef CUGO_ORACLE_CANONICAL_H_
#define CUGO_ORACLE_CANONICAL_H_

#include "torch.h"

enum { END_TERMINAL = 0, END_NAGARI = 1, END_STALLED = 2, END_ACTION_ERROR = 3,
       END_MAX_ACTIONS = 4 }; /* rollout50.h:70-76 */

/* rollout50.h:138-154 */
static void canonical_choice_step(mask_t* floor, card_t card, card_t* choice) {
  const mask_t matches = *floor & month_cards(cmonth(card));
  const int count = ccount(matches);
  if (count == 0) {
    *floor |= cbit(card);
  } else if (count == 1) {
    *floor &= ~matches;
  } else if (count == 2) {
    *choice = first_of(matches);
    *floor &= ~cbit(*choice);
  } else {
    *floor &= ~matches;
  }
}

/* rollout50.h:156-179: floor choices (played, drawn) a canonical resolve takes */
static void canonical_resolve_choices(const Turn* t, card_t* played_choice, card_t* drawn_choice) {
  *played_choice = NO_CARD;
  *drawn_choice = NO_CARD;
  if (t->phase != PHASE_RESOLVE || !is_standard(t->pending_played) ||
      !is_standard(t->pending_drawn))
    return;
  const card_t played = t->pending_played, drawn = t->pending_drawn;
  mask_t floor = t->floor & STD_MASK;
  const int played_count = ccount(floor & month_cards(cmonth(played)));
  const int same_month = cmonth(played) == cmonth(drawn);
  if (same_month && played_count == 1 && !is_last_turn(t)) return;
  if (same_month && (played_count == 0 || played_count == 2)) return;
  canonical_choice_step(&floor, played, played_choice);
  canonical_choice_step(&floor, drawn, drawn_choice);
}

/* rollout50.h:400-428 (status only) */
static uint8_t canonicalize_regular(const Terminal* s, card_t card, uint8_t month, int shake) {
  Terminal temp = *s;
  if (shake) {
    const SpecialResult started = terminal_special(&temp, SK_SHAKE, card, month, NO_CARD, 0);
    const uint8_t st = map_special_status(started.status);
    if (st != AS_OK) return st;
  } else {
    const uint8_t st = map_turn_status(begin_regular_play_terminal(&temp, card));
    if (st != AS_OK) return st;
  }
  const uint8_t drawn = map_turn_status(draw_for_terminal(&temp));
  if (drawn != AS_OK) return drawn;
  card_t pc, dc;
  canonical_resolve_choices(&temp.sp.game.turn, &pc, &dc);
  Turn resolved = temp.sp.game.turn;
  const Resolve rr = resolve_turn(&resolved, pc, dc);
  return map_resolve_status(rr.status);
}

/* rollout50.h:430-447 (status only) */
static uint8_t canonicalize_bonus(const Terminal* s, card_t card) {
  Terminal temp = *s;
  const TerminalBonus probe = play_bonus_terminal(&temp, card, 0);
  if (probe.bonus.play.status != TS_OK) return map_turn_status(probe.bonus.play.status);
  if (probe.bonus.pi.status == PT_SELECTION_REQUIRED) return AS_OK;
  return map_pi_status(probe.bonus.pi.status);
}

/* rollout50.h:449-489 (status only): a resolve choice is searched over the standard
 * floor cards in id order */
static uint8_t canonicalize_special(const Terminal* s, uint8_t kind, uint8_t month) {
  Terminal temp = *s;
  SpecialResult r = terminal_special(&temp, kind, NO_CARD, month, NO_CARD, 0);
  if (r.status == SP_RESOLVE_CHOICE_REQUIRED) {
    mask_t candidates = s->sp.game.turn.floor & STD_MASK;
    int found = 0;
    while (candidates != 0) {
      const card_t candidate = pop_first(&candidates);
      Terminal cs = *s;
      const SpecialResult cr = terminal_special(&cs, kind, NO_CARD, month, candidate, 0);
      if (cr.status != SP_RESOLVE_CHOICE_REQUIRED && cr.status != SP_INVALID_RESOLVE_CHOICE) {
        r = cr;
        found = 1;
        break;
      }
    }
    if (!found) return AS_RESOLVE_CHOICE_REQUIRED;
  }
  if (r.status == SP_PI_SELECTION_REQUIRED) return AS_OK;
  return map_special_status(r.status);
}

static uint8_t first_month_of(uint16_t months) { /* rollout50.h:113-119 */
  for (uint8_t m = 0; m < MONTHS; ++m)
    if (months & (uint16_t)(1u << m)) return m;
  return 0xffu;
}

typedef struct { uint8_t status; uint16_t index; } CanonicalIndex;

/* canonical_action50 (rollout50.h:496-574) mapped by primary_action_index50
 * (policy50.h:238-271): ChongtongWin 125, GukjinPi 177, Go 123 / Stop 124, BombCredit
 * 122, PlayBonus 48 + (card == 49), Bomb 98 + month, Grenade 110 + month, Shake 50 + card,
 * PlayCard card. */
static CanonicalIndex canonical_action(const Terminal* s) {
  CanonicalIndex out = {AS_OK, INVALID_TORCH_ACTION};
  if (t_finished(s)) { out.status = AS_GAME_FINISHED; return out; }
  if (t_has_ct_choice(s)) { out.index = 125; return out; }
  if (g_has_gukjin(&s->sp.game)) { out.index = 177; return out; }
  if (g_has_decision(&s->sp.game)) {
    out.index = go_count_of(&s->sp.game, s->sp.game.decision_actor) == 0 ? 123 : 124;
    return out;
  }
  if (s->sp.game.turn.phase != PHASE_PLAY) { out.status = AS_WRONG_PHASE; return out; }
  const unsigned actor = s->sp.game.turn.actor;
  const mask_t hand = active_hand(&s->sp.game.turn);
  if (credits_of(&s->sp, actor) != 0) {
    out.status = canonicalize_special(s, SK_BOMB_CREDIT, 0xffu);
    out.index = 122;
    return out;
  }
  const mask_t bonuses = hand & BONUS_MASK;
  if (bonuses != 0) {
    const card_t card = first_of(bonuses);
    out.status = canonicalize_bonus(s, card);
    out.index = card == BONUS2 ? 48 : 49;
    return out;
  }
  const uint16_t bombs = legal_bomb_months(&s->sp);
  if (bombs != 0) {
    const uint8_t month = first_month_of(bombs);
    out.status = canonicalize_special(s, SK_BOMB, month);
    out.index = (uint16_t)(98 + month);
    return out;
  }
  const uint16_t grenades = legal_grenade_months(&s->sp);
  if (grenades != 0) {
    const uint8_t month = first_month_of(grenades);
    out.status = canonicalize_special(s, SK_GRENADE, month);
    out.index = (uint16_t)(110 + month);
    return out;
  }
  const uint16_t shakes = legal_shake_months(&s->sp);
  if (shakes != 0) {
    const uint8_t month = first_month_of(shakes);
    const card_t card = first_of(month_of_mask(hand & STD_MASK, month));
    out.status = canonicalize_regular(s, card, month, 1);
    out.index = is_standard(card) ? (uint16_t)(50 + card) : INVALID_TORCH_ACTION;
    return out;
  }
  const mask_t standard = hand & STD_MASK;
  if (standard != 0) {
    const card_t card = first_of(standard);
    out.status = canonicalize_regular(s, card, 0xffu, 0);
    out.index = card;
    return out;
  }
  out.status = AS_NOT_LEGAL;
  return out;
}

/* torch50.h:542-558 */
static uint16_t canonical_torch_action(const Env* e) {
  if (e->done) return INVALID_TORCH_ACTION;
  if (e->pending.active) {
    const Packet p = make_packet(e);
    if (p.status != AS_OK) return INVALID_TORCH_ACTION;
    for (uint16_t card = 0; card < DECK_CARDS; ++card)
      if (tm_has(p.legal, (unsigned)(127 + card))) return (uint16_t)(127 + card);
    return INVALID_TORCH_ACTION;
  }
  const CanonicalIndex c = canonical_action(&e->g);
  if (c.status != AS_OK) return INVALID_TORCH_ACTION;
  return c.index;
}

/* RolloutResult50 (rollout50.h:78-91) plus TorchRollout50's choice counters
 * (torch50.h:621-626) */
typedef struct {
  uint8_t end, action_status, terminal_reason, winner, next_round_multiplier;
  uint16_t actions, turns, bonus_actions, special_actions, go_actions;
  uint64_t final_points;
  int64_t reward0;
  uint16_t choice_actions, resolve_choices, pi_choices;
} CanonicalResult;

/* finish_terminal_rollout50 (rollout50.h:584-614) and finish_torch_rollout50
 * (torch50.h:560-596) */
static CanonicalResult finish_torch_rollout(const Env* e, uint8_t fallback_end) {
  CanonicalResult r;
  memset(&r, 0, sizeof r);
  r.actions = e->n_primary;
  r.turns = e->g.sp.game.turn.turn_index;
  r.bonus_actions = e->n_bonus;
  r.special_actions = e->n_special;
  r.go_actions = e->n_go;
  r.choice_actions = e->n_choice;
  r.resolve_choices = e->n_resolve;
  r.pi_choices = e->n_pi;
  r.terminal_reason = REASON_NONE;
  r.winner = NO_PLAYER;
  r.next_round_multiplier = 1;
  if (t_finished(&e->g)) {
    const Settlement st = settle(&e->g);
    r.terminal_reason = e->g.reason;
    if (st.status != SETTLE_OK) {
      r.end = END_ACTION_ERROR;
      r.action_status = AS_INVALID_ACTION;
      r.winner = e->g.winner;
      return r;
    }
    r.end = END_TERMINAL;
    r.action_status = AS_OK;
    r.winner = st.winner;
    r.final_points = st.final_points;
    r.reward0 = settlement_reward(&st, 0);
    return r;
  }
  if (e->nagari) {
    r.end = END_NAGARI;
    r.action_status = AS_OK;
    r.next_round_multiplier = 2;
    r.reward0 = nagari_reward(&e->g, 0);
    return r;
  }
  r.end = fallback_end;
  r.action_status = e->status;
  return r;
}

/* rollout_canonical_torch50 (torch50.h:598-619) */
static CanonicalResult rollout_canonical_torch(uint64_t seed, unsigned first, uint16_t max_actions) {
  Env e = make_env(seed, first);
  while (!e.done && e.n_primary < max_actions) {
    const uint16_t action = canonical_torch_action(&e);
    if (action == INVALID_TORCH_ACTION) {
      e.status = AS_INVALID_ACTION;
      return finish_torch_rollout(&e, END_STALLED);
    }
    const StepResult step = torch_step(&e, action);
    if (step.status != AS_OK) return finish_torch_rollout(&e, END_ACTION_ERROR);
  }
  return finish_torch_rollout(&e, e.done ? END_TERMINAL : END_MAX_ACTIONS);
}

/* The five digest words of one rollout (this repository's packing):
 *   0 final_points   1 reward0
 *   2 actions | turns << 16 | bonus_actions << 32 | special_actions << 48
 *   3 go_actions | end << 16 | action_status << 24 | terminal_reason << 32 | winner << 40
 *     | next_round_multiplier << 48
 *   4 choice_actions | resolve_choices << 16 | pi_choices << 32 */
static void pack_canonical(const CanonicalResult* r, int64_t* out) {
  out[0] = (int64_t)r->final_points;
  out[1] = r->reward0;
  out[2] = (int64_t)((uint64_t)r->actions | (uint64_t)r->turns << 16 |
                     (uint64_t)r->bonus_actions << 32 | (uint64_t)r->special_actions << 48);
  out[3] = (int64_t)((uint64_t)r->go_actions | (uint64_t)r->end << 16 |
                     (uint64_t)r->action_status << 24 | (uint64_t)r->terminal_reason << 32 |
                     (uint64_t)r->winner << 40 | (uint64_t)r->next_round_multiplier << 48);
  out[4] = (int64_t)((uint64_t)r->choice_actions | (uint64_t)r->resolve_choices << 16 |
                     (uint64_t)r->pi_choices << 32);
}

#endif
