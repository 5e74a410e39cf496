/*
 * Oracle restatement (plain C), part 10: staged floor/pi choices after a flip
 * (include/cugo/game/postchance50.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_POSTCHANCE_H_
#define CUGO_ORACLE_POSTCHANCE_H_

#include "policy.h"

enum { PC_NONE = 0, PC_RESOLVE_PLAYED = 4, PC_RESOLVE_DRAWN = 5, PC_PI_CARD = 6 };

typedef struct {
  uint8_t status, decision;
  mask_t legal_cards;
  card_t revealed;
  uint8_t requested_pi;
} Probe;

static Probe probe_result(uint8_t status, uint8_t decision, mask_t legal, card_t revealed, uint8_t req) {
  Probe p = {status, decision, legal, revealed, req};
  return p;
}

static uint8_t decode_primary_raw(const Terminal* s, unsigned index, Action* a) {
  /* postchance50.h:84-148 */
  if (index == PA_GUKJIN_PI || index == PA_GUKJIN_ANIMAL) {
    if (decision_kind(s) != DK_GUKJIN) {
      *a = make_action(AK_PLAY_CARD); /* kInvalidAction50 */
      return AS_NOT_LEGAL;
    }
    *a = make_action(index == PA_GUKJIN_PI ? AK_GUKJIN_PI : AK_GUKJIN_ANIMAL);
    return AS_OK;
  }
  if (!pm_has(legal_primary(s), index)) {
    *a = make_action(AK_PLAY_CARD);
    return AS_NOT_LEGAL;
  }
  if (index < PA_PLAY_BONUS) { *a = make_action(AK_PLAY_CARD); a->card = (card_t)index; }
  else if (index < PA_SHAKE) { *a = make_action(AK_PLAY_BONUS); a->card = index == PA_PLAY_BONUS ? BONUS2 : BONUS3; }
  else if (index < PA_BOMB) {
    *a = make_action(AK_SHAKE);
    a->card = (card_t)(index - PA_SHAKE);
    a->month = cmonth(a->card);
  } else if (index < PA_GRENADE) { *a = make_action(AK_BOMB); a->month = (uint8_t)(index - PA_BOMB); }
  else if (index < PA_BOMB_CREDIT) { *a = make_action(AK_GRENADE); a->month = (uint8_t)(index - PA_GRENADE); }
  else if (index == PA_BOMB_CREDIT) *a = make_action(AK_BOMB_CREDIT);
  else if (index == PA_GO) *a = make_action(AK_GO);
  else if (index == PA_STOP) *a = make_action(AK_STOP);
  else if (index == PA_CT_WIN) *a = make_action(AK_CT_WIN);
  else *a = make_action(AK_CT_CONTINUE);
  return AS_OK;
}

typedef struct { uint8_t status, decision; mask_t legal; Turn table; } ChoiceProbe;

static ChoiceProbe probe_resolve_choices(const Turn* t, card_t pc, card_t dc) { /* :150-206 */
  ChoiceProbe out;
  out.status = RS_OK;
  out.decision = PC_NONE;
  out.legal = 0;
  out.table = *t;
  if (t->phase != PHASE_RESOLVE) { out.status = RS_WRONG_PHASE; return out; }
  const card_t played = t->pending_played, drawn = t->pending_drawn;
  const int pmc = ccount(floor_matches(t, played));
  const int same = cmonth(played) == cmonth(drawn);
  const int last = is_last_turn(t);
  if (same && pmc == 1 && !last) return out;
  if (same && (pmc == 0 || pmc == 2)) return out;
  Turn next = *t;
  Resolve r;
  memset(&r, 0, sizeof r);
  mask_t candidates = floor_matches(&next, played);
  uint8_t st = resolve_against_floor(&next, played, pc, &r);
  if (st == RS_CHOICE_REQUIRED) {
    out.status = st; out.decision = PC_RESOLVE_PLAYED; out.legal = candidates;
    return out;
  }
  if (st != RS_OK) { out.status = st; return out; }
  next.pending_played = NO_CARD; /* the played card is no longer pending */
  const Turn table = next;
  candidates = floor_matches(&next, drawn);
  st = resolve_against_floor(&next, drawn, dc, &r);
  if (st == RS_CHOICE_REQUIRED) {
    out.status = st; out.decision = PC_RESOLVE_DRAWN; out.legal = candidates; out.table = table;
    return out;
  }
  if (st != RS_OK) { out.status = st; return out; }
  return out;
}

static mask_t postchance_pi_candidates(const Turn* t, unsigned actor) { /* :207-213 */
  const unsigned victim = (actor & 1u) ^ 1u;
  return pi_card_mask(captured_of(t, victim), gukjin_as_pi(t, victim));
}

static Probe probe_pi_choice(const Terminal* staged, const Pending* pd, card_t revealed, uint8_t requested) {
  /* postchance50.h:214-249 */
  const mask_t cand = postchance_pi_candidates(&staged->sp.game.turn, pd->actor);
  const uint8_t available = (uint8_t)ccount(cand);
  const uint8_t selected = (uint8_t)ccount(pd->selected_pi);
  if (pd->selected_pi & ~cand) return probe_result(AS_INVALID_PI_SELECTION, PC_NONE, 0, revealed, requested);
  if (requested == 0 || available <= requested || pd->selected_pi == 0) {
    if (pd->selected_pi != 0 && (requested == 0 || available <= requested))
      return probe_result(AS_INVALID_PI_SELECTION, PC_NONE, 0, revealed, requested);
    return probe_result(AS_OK, PC_NONE, 0, revealed, requested);
  }
  if (selected > requested) return probe_result(AS_INVALID_PI_SELECTION, PC_NONE, 0, revealed, requested);
  if (selected < requested) return probe_result(AS_OK, PC_PI_CARD, cand & ~pd->selected_pi, revealed, requested);
  return probe_result(AS_OK, PC_NONE, 0, revealed, requested);
}

static Probe probe_regular(const Terminal* s, const Pending* pd, Terminal* staged, int shake) {
  /* postchance50.h:250-286 */
  *staged = *s;
  uint8_t st;
  if (shake) st = map_special_status(begin_shake(&staged->sp, pd->action.card).status);
  else st = map_turn_status(begin_regular_play_terminal(staged, pd->action.card));
  if (st != AS_OK) return probe_result(st, PC_NONE, 0, NO_CARD, 0);
  st = map_turn_status(draw_for_terminal(staged));
  if (st != AS_OK) return probe_result(st, PC_NONE, 0, NO_CARD, 0);
  const card_t revealed = staged->sp.game.turn.pending_drawn;
  const ChoiceProbe ch = probe_resolve_choices(&staged->sp.game.turn, pd->action.played_match,
                                               pd->action.drawn_match);
  if (ch.status == RS_CHOICE_REQUIRED) {
    staged->sp.game.turn = ch.table;
    return probe_result(AS_OK, ch.decision, ch.legal, revealed, 0);
  }
  if (ch.status == RS_INVALID_CHOICE) return probe_result(AS_INVALID_RESOLVE_CHOICE, PC_NONE, 0, revealed, 0);
  if (ch.status != RS_OK) return probe_result(AS_NOT_LEGAL, PC_NONE, 0, revealed, 0);
  Turn resolved = staged->sp.game.turn;
  const Resolve rr = resolve_turn(&resolved, pd->action.played_match, pd->action.drawn_match);
  if (rr.status != RS_OK) return probe_result(map_resolve_status(rr.status), PC_NONE, 0, revealed, 0);
  staged->sp.game.turn = resolved;
  return probe_pi_choice(staged, pd, revealed, steal_count(&rr));
}

static Probe probe_bonus(const Terminal* s, const Pending* pd, Terminal* staged) { /* :287-298 */
  *staged = *s;
  const TurnBonus played = play_bonus_for_turn(&staged->sp.game.turn, pd->action.card);
  const uint8_t st = map_turn_status(played.status);
  if (st != AS_OK) return probe_result(st, PC_NONE, 0, NO_CARD, 0);
  return probe_pi_choice(staged, pd, played.replacement, played.steal);
}

static Probe probe_special(const Terminal* s, const Pending* pd, Terminal* staged) { /* :299-374 */
  *staged = *s;
  Special* sp = &staged->sp;
  Turn* t = &sp->game.turn;
  const unsigned actor = pd->actor;
  uint8_t base_steal = 0;
  if (pd->action.kind == AK_BOMB || pd->action.kind == AK_GRENADE) {
    const int grenade = pd->action.kind == AK_GRENADE;
    const unsigned month = pd->action.month;
    if (!special_ready(sp) || month >= MONTHS) return probe_result(AS_NOT_LEGAL, PC_NONE, 0, NO_CARD, 0);
    const uint16_t b = (uint16_t)(1u << month);
    const uint16_t legal = grenade ? legal_grenade_months(sp) : legal_bomb_months(sp);
    if ((legal & b) == 0) return probe_result(AS_NOT_LEGAL, PC_NONE, 0, NO_CARD, 0);
    mask_t* hand = hand_of(t, actor);
    mask_t* cap = cap_ref(t, actor);
    const mask_t hc = month_of_mask(*hand, month), fc = month_of_mask(t->floor & STD_MASK, month);
    *hand &= ~hc;
    t->floor &= ~fc;
    *cap |= hc | fc;
    if (actor == 0) {
      sp->credits0 = (uint8_t)(sp->credits0 + (grenade ? 1u : 2u));
      if (!grenade) ++sp->bombs0;
    } else {
      sp->credits1 = (uint8_t)(sp->credits1 + (grenade ? 1u : 2u));
      if (!grenade) ++sp->bombs1;
    }
    base_steal = is_last_turn(t) ? 0u : 1u;
  } else if (pd->action.kind == AK_BOMB_CREDIT) {
    if (!special_ready(sp) || credits_of(sp, actor) == 0) return probe_result(AS_NOT_LEGAL, PC_NONE, 0, NO_CARD, 0);
    if (actor == 0) --sp->credits0; else --sp->credits1;
  } else {
    return probe_result(AS_INVALID_ACTION, PC_NONE, 0, NO_CARD, 0);
  }
  const DrawOnly d = draw_only_special(t, pd->action.drawn_match);
  if (d.status == SP_RESOLVE_CHOICE_REQUIRED) {
    t->pending_drawn = d.drawn;
    t->pending_bonus = d.bonuses;
    return probe_result(AS_OK, PC_RESOLVE_DRAWN, floor_matches(t, d.drawn), d.drawn, 0);
  }
  if (d.status == SP_INVALID_RESOLVE_CHOICE) return probe_result(AS_INVALID_RESOLVE_CHOICE, PC_NONE, 0, d.drawn, 0);
  if (d.status != SP_OK) return probe_result(map_special_status(d.status), PC_NONE, 0, d.drawn, 0);
  const uint8_t requested = (uint8_t)(base_steal + steal_count(&d.resolve));
  finish_draw_only(t);
  return probe_pi_choice(staged, pd, d.drawn, requested);
}

static Probe probe_postchance(const Terminal* s, const Pending* pd, Terminal* staged) { /* :375-405 */
  if (!pd->active) {
    *staged = *s;
    return probe_result(AS_WRONG_PHASE, PC_NONE, 0, NO_CARD, 0);
  }
  switch (pd->action.kind) {
    case AK_PLAY_CARD: return probe_regular(s, pd, staged, 0);
    case AK_SHAKE: return probe_regular(s, pd, staged, 1);
    case AK_PLAY_BONUS: return probe_bonus(s, pd, staged);
    case AK_BOMB: case AK_GRENADE: case AK_BOMB_CREDIT: return probe_special(s, pd, staged);
    case AK_GO: case AK_STOP: case AK_CT_WIN: case AK_CT_CONTINUE: case AK_GUKJIN_PI: case AK_GUKJIN_ANIMAL:
      *staged = *s;
      return probe_result(AS_OK, PC_NONE, 0, NO_CARD, 0);
    default:
      *staged = *s;
      return probe_result(AS_INVALID_ACTION, PC_NONE, 0, NO_CARD, 0);
  }
}

static Observation pack_postchance_observation(const Terminal* original, const Terminal* staged,
                                               const Pending* pd, const Probe* pr) { /* :406-426 */
  Terminal view = *staged;
  view.sp.game.turn.actor = pd->actor;
  view.sp.game.turn.turn_index = original->sp.game.turn.turn_index;
  Observation o = pack_observation(&view);
  o.decision_kind = pr->decision;
  if (is_physical(pr->revealed)) {
    const mask_t b = cbit(pr->revealed);
    const mask_t known = o.own_hand | o.floor | o.own_cap | o.opp_cap | o.pending_public;
    if ((known & b) == 0) {
      o.pending_public |= b;
      o.unseen &= ~b;
    }
  }
  return o;
}

typedef struct { uint8_t status, committed; } PcStep;

static PcStep continue_postchance(Terminal* s, Pending* pd) { /* postchance50.h:447-474 */
  PcStep out = {AS_OK, 0};
  Terminal staged;
  memset(&staged, 0, sizeof staged);
  const Probe pr = probe_postchance(s, pd, &staged);
  if (pr.status != AS_OK) { out.status = pr.status; return out; }
  if (pr.decision != PC_NONE) return out;
  Action a = pd->action;
  if (pd->selected_pi != 0) a.pi_cards = pd->selected_pi;
  const ActionResult applied = apply_action(s, a);
  if (applied.status != AS_OK) { out.status = applied.status; return out; }
  pd->action = a;
  pd->active = 0;
  out.committed = 1;
  return out;
}

static PcStep start_postchance_action(Terminal* s, unsigned primary, Pending* pd) { /* :475-488 */
  Action a = make_action(AK_PLAY_CARD);
  const uint8_t st = decode_primary_raw(s, primary, &a);
  unsigned actor = decision_player(s);
  if (actor > 1u) actor = s->sp.game.turn.actor & 1u;
  memset(pd, 0, sizeof *pd);
  pd->action = a;
  pd->selected_pi = 0;
  pd->primary_action = (uint16_t)primary;
  pd->actor = (uint8_t)actor;
  pd->active = 0;
  if (st != AS_OK) { PcStep e = {st, 0}; return e; }
  pd->active = 1;
  return continue_postchance(s, pd);
}

static PcStep choose_postchance_card(Terminal* s, Pending* pd, card_t card) { /* :489-518 */
  Terminal staged;
  memset(&staged, 0, sizeof staged);
  const Probe pr = probe_postchance(s, pd, &staged);
  if (pr.status != AS_OK) { PcStep e = {pr.status, 0}; return e; }
  if (pr.decision == PC_NONE) return continue_postchance(s, pd);
  if (!is_physical(card) || (pr.legal_cards & cbit(card)) == 0) {
    PcStep e = {pr.decision == PC_PI_CARD ? AS_INVALID_PI_SELECTION : AS_INVALID_RESOLVE_CHOICE, 0};
    return e;
  }
  if (pr.decision == PC_RESOLVE_PLAYED) pd->action.played_match = card;
  else if (pr.decision == PC_RESOLVE_DRAWN) pd->action.drawn_match = card;
  else if (pr.decision == PC_PI_CARD) pd->selected_pi |= cbit(card);
  return continue_postchance(s, pd);
}

#endif
