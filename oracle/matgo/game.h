/*
 * Oracle restatement (plain C), part 4: Go/Stop and the Gukjin prompt
 * (include/cugo/game/game50.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_GAME_H_
#define CUGO_ORACLE_GAME_H_

#include "pi.h"

#define DECISION_BASE_POINTS 7 /* game50.h:16 */
enum { GS_OK = 0, GS_NO_DECISION = 1, GS_FINISHED = 2, GS_INVALID = 3 };
enum { GO = 0, STOP = 1 };

static int g_has_decision(const Game* g) { return g->decision_actor <= 1u; }
static int g_has_gukjin(const Game* g) { return g->gukjin_decision != 0; }
static uint8_t g_gukjin_actor(const Game* g) {
  return g->gukjin_decision ? (uint8_t)(g->gukjin_decision - 1u) : NO_PLAYER;
}
static int g_has_choice(const Game* g) { return g_has_decision(g) || g_has_gukjin(g); }
static int g_finished(const Game* g) { return g->winner <= 1u; }
static uint8_t go_count_of(const Game* g, unsigned p) { return (p & 1u) == 0 ? g->go0 : g->go1; }
static uint8_t last_go_of(const Game* g, unsigned p) { return (p & 1u) == 0 ? g->last_go0 : g->last_go1; }
static uint8_t base_score(const Game* g, unsigned p) { return score_player(&g->turn, p).total; }

static uint64_t go_multiplier(uint8_t go_count) { /* game50.h:126-134 */
  uint64_t m = 1;
  for (unsigned go = 3; go <= go_count; ++go) {
    m *= 2u;
    if (go == 0xffu) break;
  }
  return m;
}
static uint64_t go_adjusted_points(uint8_t base, uint8_t go_count) { /* game50.h:136-147 */
  return ((uint64_t)base + (uint64_t)go_count) * go_multiplier(go_count);
}

static int maybe_open_go_stop(Game* g, unsigned actor) { /* game50.h:159-181 */
  if (actor > 1u || g_finished(g) || g_has_choice(g)) return 0;
  const uint8_t base = base_score(g, actor);
  const uint8_t gc = go_count_of(g, actor);
  const int eligible = gc == 0 ? base >= DECISION_BASE_POINTS : base > last_go_of(g, actor);
  if (!eligible) return 0;
  auto_decide_loser_gukjin(&g->turn, actor ^ 1u);
  if (g->turn.turn_index > LAST_TURN_INDEX) {
    g->winner = (uint8_t)actor;
    return 0;
  }
  g->decision_actor = (uint8_t)actor;
  return 1;
}

static int finish_turn_game(Game* g, unsigned actor) { /* game50.h:184-199 */
  if (actor > 1u || g_finished(g) || g_has_choice(g)) return 0;
  if (gukjin_prompt_due(&g->turn, actor, go_count_of(g, actor))) {
    g->gukjin_decision = (uint8_t)(actor + 1u);
    return 1;
  }
  return maybe_open_go_stop(g, actor);
}

static uint8_t apply_gukjin_decision(Game* g, int as_pi) { /* game50.h:201-210 */
  if (g_finished(g)) return GS_FINISHED;
  if (!g_has_gukjin(g)) return GS_NO_DECISION;
  const uint8_t actor = g_gukjin_actor(g);
  decide_gukjin(&g->turn, actor, as_pi);
  g->gukjin_decision = 0;
  maybe_open_go_stop(g, actor);
  return GS_OK;
}

static uint8_t apply_go_stop(Game* g, unsigned action) { /* game50.h:212-238 */
  if (g_finished(g)) return GS_FINISHED;
  if (!g_has_decision(g)) return GS_NO_DECISION;
  if (action > STOP) return GS_INVALID;
  const uint8_t actor = g->decision_actor;
  if (action == STOP) {
    auto_decide_loser_gukjin(&g->turn, actor ^ 1u);
    g->winner = actor;
    g->decision_actor = NO_PLAYER;
    return GS_OK;
  }
  const uint8_t base = base_score(g, actor);
  if (actor == 0) { ++g->go0; g->last_go0 = base; }
  else { ++g->go1; g->last_go1 = base; }
  g->decision_actor = NO_PLAYER;
  return GS_OK;
}

typedef struct {
  ResolvePi turn;
  uint8_t completed_actor, base, decision_opened;
} GameResolve;

static GameResolve resolve_game_turn(Game* g, card_t pc, card_t dc, mask_t pi_sel) {
  /* game50.h:271-305 */
  GameResolve out;
  memset(&out, 0, sizeof out);
  if (g_finished(g) || g_has_choice(g)) {
    out.turn.resolve = resolve_fail(RS_WRONG_PHASE);
    out.turn.pi = pi_result(PT_OK, 0, 0);
    out.completed_actor = NO_PLAYER;
    return out;
  }
  const uint8_t actor = g->turn.actor;
  Game next = *g;
  out.turn = resolve_turn_with_pi(&next.turn, pc, dc, pi_sel);
  out.completed_actor = actor;
  if (out.turn.resolve.status != RS_OK || out.turn.pi.status != PT_OK) return out;
  out.base = base_score(&next, actor);
  out.decision_opened = (uint8_t)finish_turn_game(&next, actor);
  *g = next;
  return out;
}

#endif
