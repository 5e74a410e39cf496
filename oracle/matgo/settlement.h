/*
 * Oracle restatement (plain C), part 7: settlement and rewards
 * (include/cugo/game/settlement50.h).  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_SETTLEMENT_H_
#define CUGO_ORACLE_SETTLEMENT_H_

#include "terminal.h"

enum { SETTLE_OK = 0, SETTLE_NOT_FINISHED = 1, SETTLE_INVALID_WINNER = 2 };

typedef struct {
  uint8_t status, reason, winner;
  uint64_t final_points;
  int64_t side0;
} Settlement;

static int fixed_special(uint8_t reason) { /* settlement50.h:88-94 */
  return reason == REASON_INITIAL_CT || reason == REASON_FLOOR_CT || reason == REASON_BONUS_CT ||
         reason == REASON_THREE_PPUK;
}

static Settlement settle(const Terminal* s) { /* settlement50.h:95-208 */
  Settlement r;
  r.status = SETTLE_NOT_FINISHED;
  r.reason = REASON_NONE;
  r.winner = NO_PLAYER;
  r.final_points = 0;
  r.side0 = 0;
  if (!t_finished(s)) return r;
  r.reason = s->reason;
  if (s->winner > 1u) { r.status = SETTLE_INVALID_WINNER; return r; }
  const unsigned winner = s->winner, loser = winner ^ 1u;
  const Turn* t = &s->sp.game.turn;
  const Score ws = score_player(t, winner), ls = score_player(t, loser);
  const uint8_t go_count = go_count_of(&s->sp.game, winner);
  const uint64_t round = round_mult(s);
  r.status = SETTLE_OK;
  r.winner = (uint8_t)winner;
  r.side0 = (int64_t)s->side0;
  if (fixed_special(s->reason)) {
    r.final_points = s->points * round;
    return r;
  }
  const uint64_t after_go = go_adjusted_points(ws.total, go_count);
  const uint64_t special_mult = bomb_shake_multiplier(&s->sp, winner);
  uint64_t bak = 1;
  if (ws.flags & SF_MEONGTTA) bak *= 2u;
  if (ws.pi_units >= 10u && ls.pi_units >= 1u && ls.pi_units <= 7u) bak *= 2u;  /* pi-bak */
  if (ws.bright_count >= 3u && ls.bright_count == 0u) bak *= 2u;               /* gwang-bak */
  if (go_count_of(&s->sp.game, loser) != 0u) bak *= 2u;                       /* dok-bak */
  uint64_t mission = mission_multi_of(s, winner);
  if (mission == 0u) mission = 1u;
  const int void_game = captured_of(t, loser) == 0;
  const uint64_t after_special = after_go * special_mult;
  r.final_points = void_game ? 0u : after_special * bak * mission * round;
  return r;
}

static int64_t settlement_reward(const Settlement* st, unsigned player) { /* settlement50.h:211-218 */
  if (st->status != SETTLE_OK || player > 1u) return 0;
  const int64_t pts = (int64_t)st->final_points;
  const int64_t side = player == 0 ? st->side0 : -st->side0;
  return (player == st->winner ? pts : -pts) + side;
}

static int64_t nagari_reward(const Terminal* s, unsigned player) { /* settlement50.h:220-225 */
  const int64_t side = s->side0;
  return player == 0 ? side : -side;
}

#endif
