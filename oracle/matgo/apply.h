/*
 * Oracle restatement (plain C), part 8: transactional action application
 * (include/cugo/game/rollout50.h:18-68, 187-399).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_APPLY_H_
#define CUGO_ORACLE_APPLY_H_

#include "settlement.h"

enum { AK_PLAY_CARD = 0, AK_PLAY_BONUS = 1, AK_SHAKE = 2, AK_BOMB = 3, AK_GRENADE = 4,
       AK_BOMB_CREDIT = 5, AK_GO = 6, AK_STOP = 7, AK_CT_WIN = 8, AK_CT_CONTINUE = 9,
       AK_GUKJIN_PI = 10, AK_GUKJIN_ANIMAL = 11 };
enum { AS_OK = 0, AS_WRONG_PHASE = 1, AS_INVALID_ACTION = 2, AS_NOT_LEGAL = 3, AS_STOCK_EMPTY = 4,
       AS_RESOLVE_CHOICE_REQUIRED = 5, AS_INVALID_RESOLVE_CHOICE = 6, AS_PI_SELECTION_REQUIRED = 7,
       AS_INVALID_PI_SELECTION = 8, AS_GAME_FINISHED = 9 };

typedef struct {
  uint8_t status, kind, actor, turn_completed, decision_opened, terminal_opened;
} ActionResult;

static Action make_action(uint8_t kind) { /* rollout50.h:108-111 */
  Action a;
  memset(&a, 0, sizeof a);
  a.kind = kind;
  a.card = NO_CARD;
  a.month = 0xffu;
  a.played_match = NO_CARD;
  a.drawn_match = NO_CARD;
  a.pi_cards = 0;
  return a;
}

static uint8_t map_turn_status(uint8_t s) { /* rollout50.h:170-175 */
  if (s == TS_OK) return AS_OK;
  if (s == TS_STOCK_EMPTY) return AS_STOCK_EMPTY;
  if (s == TS_WRONG_PHASE) return AS_WRONG_PHASE;
  return AS_NOT_LEGAL;
}
static uint8_t map_resolve_status(uint8_t s) { /* rollout50.h:176-186 */
  if (s == RS_OK) return AS_OK;
  if (s == RS_CHOICE_REQUIRED) return AS_RESOLVE_CHOICE_REQUIRED;
  if (s == RS_INVALID_CHOICE) return AS_INVALID_RESOLVE_CHOICE;
  if (s == RS_WRONG_PHASE) return AS_WRONG_PHASE;
  return AS_NOT_LEGAL;
}
static uint8_t map_pi_status(uint8_t s) { /* rollout50.h:187-192 */
  if (s == PT_OK) return AS_OK;
  if (s == PT_SELECTION_REQUIRED) return AS_PI_SELECTION_REQUIRED;
  return AS_INVALID_PI_SELECTION;
}
static uint8_t map_special_status(uint8_t s) { /* rollout50.h:193-210 */
  switch (s) {
    case SP_OK: return AS_OK;
    case SP_WRONG_PHASE: return AS_WRONG_PHASE;
    case SP_STOCK_EMPTY: return AS_STOCK_EMPTY;
    case SP_RESOLVE_CHOICE_REQUIRED: return AS_RESOLVE_CHOICE_REQUIRED;
    case SP_INVALID_RESOLVE_CHOICE: return AS_INVALID_RESOLVE_CHOICE;
    case SP_PI_SELECTION_REQUIRED: return AS_PI_SELECTION_REQUIRED;
    case SP_INVALID_PI_SELECTION: return AS_INVALID_PI_SELECTION;
    default: return AS_NOT_LEGAL;
  }
}

static ActionResult action_result(uint8_t status, uint8_t kind, uint8_t actor, uint8_t turn,
                                  uint8_t decision, uint8_t terminal) {
  ActionResult r = {status, kind, actor, turn, decision, terminal};
  return r;
}

/* Play card / shake tail: draw, resolve with pi transfer, commit (rollout50.h:300-345) */
static ActionResult finish_card_action(Terminal* s, Terminal* next, const Action* a, uint8_t actor) {
  uint8_t st = map_turn_status(draw_for_terminal(next));
  if (st != AS_OK) return action_result(st, a->kind, actor, 0, 0, 0);
  const TerminalResolve rs = resolve_terminal_turn(next, a->played_match, a->drawn_match, a->pi_cards);
  st = map_resolve_status(rs.game.turn.resolve.status);
  if (st == AS_OK) st = map_pi_status(rs.game.turn.pi.status);
  if (st != AS_OK) return action_result(st, a->kind, actor, 0, 0, 0);
  const uint8_t decision = (uint8_t)g_has_choice(&next->sp.game);
  const uint8_t terminal = (uint8_t)t_finished(next);
  *s = *next;
  return action_result(AS_OK, a->kind, actor, 1, decision, terminal);
}

static ActionResult apply_action_body(Terminal* s, Action a) { /* rollout50.h:231-385 */
  const uint8_t actor = s->sp.game.turn.actor;
  if (t_finished(s)) return action_result(AS_GAME_FINISHED, a.kind, actor, 0, 0, 0);
  Terminal next = *s;
  next.held0 |= next.sp.game.turn.hand0;
  next.held1 |= next.sp.game.turn.hand1;
  if (a.kind == AK_CT_WIN || a.kind == AK_CT_CONTINUE) {
    if (apply_chongtong_action(&next, a.kind == AK_CT_WIN ? CT_WIN : CT_CONTINUE) != TM_OK)
      return action_result(AS_NOT_LEGAL, a.kind, actor, 0, 0, 0);
    const uint8_t terminal = (uint8_t)t_finished(&next);
    *s = next;
    return action_result(AS_OK, a.kind, actor, 0, 0, terminal);
  }
  if (a.kind == AK_GO || a.kind == AK_STOP) {
    if (terminal_go_stop(&next, a.kind == AK_GO ? GO : STOP) != GS_OK)
      return action_result(AS_NOT_LEGAL, a.kind, actor, 0, 0, 0);
    const uint8_t terminal = (uint8_t)t_finished(&next);
    *s = next;
    return action_result(AS_OK, a.kind, actor, 0, 0, terminal);
  }
  if (a.kind == AK_GUKJIN_PI || a.kind == AK_GUKJIN_ANIMAL) {
    if (terminal_gukjin_decision(&next, a.kind == AK_GUKJIN_PI) != GS_OK)
      return action_result(AS_NOT_LEGAL, a.kind, actor, 0, 0, 0);
    const uint8_t decision = (uint8_t)g_has_choice(&next.sp.game);
    const uint8_t terminal = (uint8_t)t_finished(&next);
    *s = next;
    return action_result(AS_OK, a.kind, actor, 0, decision, terminal);
  }
  if (t_has_ct_choice(&next) || g_has_choice(&next.sp.game))
    return action_result(AS_WRONG_PHASE, a.kind, actor, 0, 0, 0);
  if (a.kind == AK_PLAY_BONUS) {
    const TerminalBonus r = play_bonus_terminal(&next, a.card, a.pi_cards);
    uint8_t st = map_turn_status(r.bonus.play.status);
    if (st == AS_OK) st = map_pi_status(r.bonus.pi.status);
    if (st != AS_OK) return action_result(st, a.kind, actor, 0, 0, 0);
    *s = next;
    return action_result(AS_OK, a.kind, actor, 0, 0, 0);
  }
  if (a.kind == AK_BOMB || a.kind == AK_GRENADE || a.kind == AK_BOMB_CREDIT) {
    const uint8_t kind = a.kind == AK_BOMB ? SK_BOMB : a.kind == AK_GRENADE ? SK_GRENADE : SK_BOMB_CREDIT;
    const SpecialResult r = terminal_special(&next, kind, a.card, a.month, a.drawn_match, a.pi_cards);
    const uint8_t st = map_special_status(r.status);
    if (st != AS_OK) return action_result(st, a.kind, actor, 0, 0, 0);
    const uint8_t decision = (uint8_t)g_has_choice(&next.sp.game);
    const uint8_t terminal = (uint8_t)t_finished(&next);
    *s = next;
    return action_result(AS_OK, a.kind, actor, 1, decision, terminal);
  }
  if (a.kind == AK_SHAKE) {
    if (is_standard(a.card)) { /* the shaken month's cards in hand become public */
      const mask_t shown = month_of_mask(active_hand(&next.sp.game.turn), cmonth(a.card));
      if (actor == 0) next.revealed0 |= shown; else next.revealed1 |= shown;
    }
    const SpecialResult started = terminal_special(&next, SK_SHAKE, a.card, a.month, NO_CARD, 0);
    const uint8_t st = map_special_status(started.status);
    if (st != AS_OK) return action_result(st, a.kind, actor, 0, 0, 0);
    return finish_card_action(s, &next, &a, actor);
  }
  if (a.kind == AK_PLAY_CARD) {
    /* a card of a bomb/grenade month is only playable as that bomb/grenade */
    if (is_standard(a.card) && (forced_special_months(&next.sp) & (uint16_t)(1u << cmonth(a.card))))
      return action_result(AS_NOT_LEGAL, a.kind, actor, 0, 0, 0);
    const uint8_t st = map_turn_status(begin_regular_play_terminal(&next, a.card));
    if (st != AS_OK) return action_result(st, a.kind, actor, 0, 0, 0);
    return finish_card_action(s, &next, &a, actor);
  }
  return action_result(AS_INVALID_ACTION, a.kind, actor, 0, 0, 0);
}

static ActionResult apply_action(Terminal* s, Action a) { /* rollout50.h:391-399 */
  const ActionResult r = apply_action_body(s, a);
  if (r.status == AS_OK) {
    s->held0 |= s->sp.game.turn.hand0;
    s->held1 |= s->sp.game.turn.hand1;
  }
  return r;
}

#endif
