/*
 * Oracle restatement (plain C), part 6: terminal reasons, missions, Chongtong, ppuk
 * chain and side payments (include/cugo/game/terminal50.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_TERMINAL_H_
#define CUGO_ORACLE_TERMINAL_H_

#include "special.h"

#define CHONGTONG_POINTS 10u
#define THREE_PPUK_POINTS 7u
#define EVENT_PAYMENT 7
enum { PPUK_NONE = 0, PPUK_FIRST = 1, PPUK_SECOND = 2, PPUK_THIRD = 3, PPUK_ONE = 4, PPUK_TWO = 5,
       PPUK_THREE = 6 };
enum { MISSION_NONE = 0, MISSION_EASY = 1, MISSION_NORMAL = 2, MISSION_HARD = 3,
       MISSION_NO_CONDITION = 4, MISSION_TRIPLE = 6 };
enum { REASON_NONE = 0, REASON_STOP = 1, REASON_INITIAL_CT = 2, REASON_FLOOR_CT = 3,
       REASON_BONUS_CT = 4, REASON_THREE_PPUK = 5 };
enum { CT_WIN = 0, CT_CONTINUE = 1 };
enum { TM_OK = 0, TM_FINISHED = 1, TM_CT_PENDING = 2, TM_NO_CT = 3, TM_INVALID = 4 };

static uint8_t round_mult(const Terminal* s) { return s->round_mult == 0 ? 1u : s->round_mult; }
static uint8_t mission_multi_of(const Terminal* s, unsigned p) { return (p & 1u) == 0 ? s->mm0 : s->mm1; }
static void add_side_payment(Terminal* s, unsigned receiver, int32_t base) { /* terminal50.h:113-117 */
  const int32_t amount = base * (int32_t)round_mult(s);
  s->side0 += (receiver & 1u) == 0 ? amount : -amount;
}

/* Hangame card numbers are 1-based (terminal50.h:118-125) */
static mask_t hg(int a, int b, int c) {
  mask_t m = cbit((card_t)(a - 1)) | cbit((card_t)(b - 1));
  if (c) m |= cbit((card_t)(c - 1));
  return m;
}

static mask_t mission_cards_for(uint8_t type, uint8_t index) { /* terminal50.h:129-159 */
  if (type == MISSION_EASY) {
    if (index == 10) return hg(9, 29, 0);
    return hg(4 * index + 1, 4 * index + 2, 0);
  }
  if (type == MISSION_NORMAL) return month_cards(index);
  if (type == MISSION_HARD || type == MISSION_TRIPLE) {
    const int tri = type == MISSION_TRIPLE;
    if (tri && index >= 4) ++index;
    switch (index) {
      case 0: return hg(22, 34, 38);
      case 1: return hg(2, 6, 10);
      case 2: return hg(14, 18, 26);
      case 3: return hg(5, 13, 30);
      case 4: return hg(33, 42, 48);
      case 5: return tri ? hg(5, 25, 46) : hg(21, 25, 37);
      case 6: return tri ? hg(21, 25, 37) : hg(1, 9, 29);
      case 7: return tri ? hg(1, 9, 29) : hg(1, 9, 41);
      case 8: return tri ? hg(1, 9, 41) : hg(1, 29, 41);
      case 9: return tri ? hg(1, 29, 41) : hg(9, 29, 41);
      case 10: return tri ? hg(9, 29, 41) : hg(5, 13, 46);
      case 11: return tri ? hg(5, 13, 46) : hg(5, 30, 46);
      case 12: return tri ? hg(5, 30, 46) : hg(13, 30, 46);
      case 13: return tri ? hg(13, 30, 46) : hg(5, 25, 46);
      default: return 0;
    }
  }
  return 0;
}

static void assign_mission(Terminal* s, uint64_t seed) { /* terminal50.h:164-183 */
  uint64_t rng = seed ^ 0x6d697373696f6e35ull;
  const uint32_t kind = uniform_bounded(&rng, 5u);
  const uint8_t multiplier = (uint8_t)(2u + uniform_bounded(&rng, 3u));
  uint8_t type = MISSION_EASY;
  uint32_t options = 11u;
  if (kind == 1u) { type = MISSION_NORMAL; options = 12u; }
  else if (kind == 2u) { type = MISSION_HARD; options = 14u; }
  else if (kind == 3u) { type = MISSION_NO_CONDITION; options = 0u; }
  else if (kind == 4u) { type = MISSION_TRIPLE; options = 13u; }
  const uint8_t index = options == 0u ? 0u : (uint8_t)uniform_bounded(&rng, options);
  s->mission_type = type;
  s->mission_mult = type == MISSION_TRIPLE ? 0u : multiplier;
  s->sp.game.turn.mission = mission_cards_for(type, index);
  if (type == MISSION_NO_CONDITION) { s->mm0 = multiplier; s->mm1 = multiplier; }
}

static void update_missions(Terminal* s, unsigned actor, mask_t acquired) { /* terminal50.h:186-197 */
  const Turn* t = &s->sp.game.turn;
  const mask_t mine = (actor & 1u) == 0 ? t->captured0 : t->captured1;
  uint8_t* multi = (actor & 1u) == 0 ? &s->mm0 : &s->mm1;
  if (s->mission_type == MISSION_TRIPLE) {
    *multi = (uint8_t)(1u << ccount(t->mission & mine));
    return;
  }
  if (t->mission == 0 || (acquired & t->mission) == 0) return;
  if ((t->mission & ~mine) == 0) *multi = s->mission_mult;
}

static uint16_t chongtong_months(mask_t cards) { /* terminal50.h:215-224 */
  cards &= STD_MASK;
  uint16_t r = 0;
  for (unsigned m = 0; m < MONTHS; ++m)
    if ((cards & month_cards(m)) == month_cards(m)) r |= (uint16_t)(1u << m);
  return r;
}

static int t_finished(const Terminal* s) { return s->reason != REASON_NONE; }
static int t_has_ct_choice(const Terminal* s) { return s->ct_actor <= 1u; }

static void mark_terminal(Terminal* s, unsigned winner, uint8_t reason, uint64_t points) {
  /* terminal50.h:264-275 */
  s->winner = (uint8_t)(winner & 1u);
  s->reason = reason;
  s->points = points;
  s->ct_actor = NO_PLAYER;
  s->ct_months = 0;
  s->sp.game.decision_actor = NO_PLAYER;
  s->sp.game.gukjin_decision = 0;
}

static Terminal make_terminal_state(Deal deal, unsigned first) { /* terminal50.h:277-315 */
  Terminal s;
  memset(&s, 0, sizeof s);
  s.sp.game.turn = make_turn_state(deal, first);
  s.sp.game.decision_actor = NO_PLAYER;
  s.sp.game.winner = NO_PLAYER;
  s.ct_actor = NO_PLAYER;
  s.winner = NO_PLAYER;
  s.reason = REASON_NONE;
  s.round_mult = 1;
  s.mission_type = MISSION_NONE;
  assign_mission(&s, deal.rng); /* the deal's stream state, before the floor refill */
  update_missions(&s, 0, 0);
  update_missions(&s, 1, 0);
  const Turn* t = &s.sp.game.turn;
  s.held0 = t->hand0;
  s.held1 = t->hand1;
  /* detect_initial_chongtong50 (terminal50.h:226-252) on the dealt hands and the
   * refilled floor */
  const uint16_t h0 = chongtong_months(deal.hand0), h1 = chongtong_months(deal.hand1);
  const uint16_t fl = chongtong_months(t->floor);
  const unsigned f = first & 1u;
  if (fl) mark_terminal(&s, f, REASON_FLOOR_CT, CHONGTONG_POINTS);
  else if (h0 && h1) mark_terminal(&s, f, REASON_INITIAL_CT, CHONGTONG_POINTS);
  else if (h0) mark_terminal(&s, 0, REASON_INITIAL_CT, CHONGTONG_POINTS);
  else if (h1) mark_terminal(&s, 1, REASON_INITIAL_CT, CHONGTONG_POINTS);
  return s;
}

static void sync_game_stop(Terminal* s) { /* terminal50.h:316-323 */
  if (s->reason != REASON_NONE || !g_finished(&s->sp.game)) return;
  const uint8_t w = s->sp.game.winner;
  s->winner = w;
  s->reason = REASON_STOP;
  s->points = go_adjusted_points(base_score(&s->sp.game, w), go_count_of(&s->sp.game, w)) *
              bomb_shake_multiplier(&s->sp, w);
}

static int record_completed_turn_ppuk(Terminal* s, unsigned actor, int made_ppuk) {
  /* terminal50.h:339-362 */
  if (t_finished(s) || !made_ppuk) return 0;
  actor &= 1u;
  uint8_t* count = actor == 0 ? &s->ppuk_count0 : &s->ppuk_count1;
  uint8_t* ppuk = actor == 0 ? &s->streak0 : &s->streak1;
  const uint16_t turn = s->sp.game.turn.turn_index;
  if (*count != 0xffu) ++*count;
  switch (*ppuk) {
    case PPUK_NONE: *ppuk = turn <= 1u ? PPUK_FIRST : PPUK_ONE; break;
    case PPUK_FIRST: *ppuk = turn <= 3u ? PPUK_SECOND : PPUK_TWO; break;
    case PPUK_SECOND: *ppuk = turn <= 5u ? PPUK_THIRD : PPUK_THREE; break;
    case PPUK_ONE: *ppuk = PPUK_TWO; break;
    case PPUK_TWO: *ppuk = PPUK_THREE; break;
    default: break;
  }
  if (*ppuk == PPUK_FIRST || *ppuk == PPUK_SECOND || *ppuk == PPUK_THIRD)
    add_side_payment(s, actor, EVENT_PAYMENT * (int32_t)*ppuk);
  if (*ppuk != PPUK_THIRD && *ppuk != PPUK_THREE) return 0;
  mark_terminal(s, actor, REASON_THREE_PPUK, THREE_PPUK_POINTS);
  return 1;
}

static int open_bonus_chongtong_choice(Terminal* s, unsigned actor, uint16_t formed) {
  /* terminal50.h:363-374 */
  if (t_finished(s) || t_has_ct_choice(s) || actor > 1u || formed == 0) return 0;
  s->ct_actor = (uint8_t)actor;
  s->ct_months = (uint16_t)(formed & ALL_MONTH_BITS);
  return s->ct_months != 0;
}

static uint8_t apply_chongtong_action(Terminal* s, unsigned action) { /* terminal50.h:375-392 */
  if (t_finished(s)) return TM_FINISHED;
  if (!t_has_ct_choice(s)) return TM_NO_CT;
  if (action > CT_CONTINUE) return TM_INVALID;
  const uint8_t actor = s->ct_actor;
  if (action == CT_WIN) {
    mark_terminal(s, actor, REASON_BONUS_CT, CHONGTONG_POINTS);
    return TM_OK;
  }
  s->ct_actor = NO_PLAYER;
  s->ct_months = 0;
  return TM_OK;
}

static uint8_t begin_regular_play_terminal(Terminal* s, card_t card) { /* terminal50.h:393-399 */
  if (t_finished(s) || t_has_ct_choice(s)) return TS_WRONG_PHASE;
  return begin_regular_play_game(&s->sp.game, card);
}
static uint8_t draw_for_terminal(Terminal* s) { /* terminal50.h:400-405 */
  if (t_finished(s) || t_has_ct_choice(s)) return TS_WRONG_PHASE;
  return draw_for_game(&s->sp.game);
}

typedef struct { BonusPi bonus; uint16_t formed; uint8_t choice_opened; } TerminalBonus;

static TerminalBonus play_bonus_terminal(Terminal* s, card_t bonus, mask_t sel) { /* :406-441 */
  TerminalBonus out;
  memset(&out, 0, sizeof out);
  if (t_finished(s) || t_has_ct_choice(s)) {
    out.bonus.play.status = TS_WRONG_PHASE;
    out.bonus.play.replacement = NO_CARD;
    out.bonus.pi = pi_result(PT_OK, 0, 0);
    return out;
  }
  Terminal next = *s;
  const unsigned actor = next.sp.game.turn.actor;
  const uint16_t before = chongtong_months(active_hand(&next.sp.game.turn));
  /* play_bonus_for_game50_with_pi_transfer (game50.h:254-263) */
  if (g_finished(&next.sp.game) || g_has_choice(&next.sp.game)) {
    out.bonus.play.status = TS_WRONG_PHASE;
    out.bonus.play.replacement = NO_CARD;
    out.bonus.pi = pi_result(PT_OK, 0, 0);
    return out;
  }
  out.bonus = play_bonus_with_pi(&next.sp.game.turn, bonus, sel);
  if (out.bonus.play.status != TS_OK || out.bonus.pi.status != PT_OK) return out;
  if (out.bonus.pi.transferred_mask) update_missions(&next, actor, out.bonus.pi.transferred_mask);
  const uint16_t after = chongtong_months(active_hand(&next.sp.game.turn));
  out.formed = (uint16_t)(after & (uint16_t)~before);
  out.choice_opened = (uint8_t)open_bonus_chongtong_choice(&next, actor, out.formed);
  *s = next;
  return out;
}

typedef struct { GameResolve game; uint8_t terminal_opened; } TerminalResolve;

static TerminalResolve resolve_terminal_turn(Terminal* s, card_t pc, card_t dc, mask_t sel) {
  /* terminal50.h:456-503 */
  TerminalResolve out;
  memset(&out, 0, sizeof out);
  if (t_finished(s) || t_has_ct_choice(s)) {
    out.game.turn.resolve = resolve_fail(RS_WRONG_PHASE);
    out.game.turn.pi = pi_result(PT_OK, 0, 0);
    out.game.completed_actor = NO_PLAYER;
    return out;
  }
  Terminal next = *s;
  const unsigned actor = next.sp.game.turn.actor;
  const mask_t before = captured_of(&next.sp.game.turn, actor);
  out.game = resolve_game_turn(&next.sp.game, pc, dc, sel);
  if (out.game.turn.resolve.status != RS_OK || out.game.turn.pi.status != PT_OK) return out;
  const uint8_t events = out.game.turn.resolve.events;
  if ((events & EV_TTADAK) && next.sp.game.turn.turn_index == 1u)
    add_side_payment(&next, actor, EVENT_PAYMENT);
  const mask_t after = captured_of(&next.sp.game.turn, actor);
  update_missions(&next, actor, after & ~before);
  const int terminal = record_completed_turn_ppuk(&next, actor, (events & EV_PPUK) != 0);
  sync_game_stop(&next);
  if (terminal) out.game.decision_opened = 0;
  out.terminal_opened = (uint8_t)terminal;
  *s = next;
  return out;
}

static SpecialResult terminal_special(Terminal* s, uint8_t kind, card_t card, uint8_t month,
                                      card_t drawn_match, mask_t sel) { /* terminal50.h:504-526 */
  if (t_finished(s) || t_has_ct_choice(s)) return special_error(SP_WRONG_PHASE);
  Terminal next = *s;
  const unsigned actor = next.sp.game.turn.actor;
  const mask_t before = captured_of(&next.sp.game.turn, actor);
  const SpecialResult r = apply_special(&next.sp, kind, card, month, drawn_match, sel);
  if (r.status != SP_OK) return r;
  if (kind != SK_SHAKE) {
    const mask_t after = captured_of(&next.sp.game.turn, actor);
    update_missions(&next, actor, after & ~before);
    sync_game_stop(&next);
  }
  *s = next;
  return r;
}

static uint8_t terminal_gukjin_decision(Terminal* s, int as_pi) { /* terminal50.h:527-538 */
  if (t_finished(s) || t_has_ct_choice(s)) return GS_FINISHED;
  Terminal next = *s;
  const uint8_t st = apply_gukjin_decision(&next.sp.game, as_pi);
  if (st != GS_OK) return st;
  sync_game_stop(&next);
  *s = next;
  return st;
}

static uint8_t terminal_go_stop(Terminal* s, unsigned action) { /* terminal50.h:539-550 */
  if (t_finished(s) || t_has_ct_choice(s)) return GS_FINISHED;
  Terminal next = *s;
  const uint8_t st = apply_go_stop(&next.sp.game, action);
  if (st != GS_OK) return st;
  sync_game_stop(&next);
  *s = next;
  return st;
}

#endif
