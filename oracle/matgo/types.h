/*
 * Oracle restatement of the reference Shin Matgo engine in plain C: types.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle/matgo/matgo.c).  The structs mirror the
 * reference's trivially-copyable state so a 248-byte row is this struct's bytes:
 *   TurnState50          include/cugo/game/turn50.h:92-115        96 bytes
 *   GameState50          include/cugo/game/game50.h:38-48        104 bytes
 *   SpecialGameState50   include/cugo/game/special50.h:25-32     120 bytes
 *   TerminalGameState50  include/cugo/game/terminal50.h:74-102   192 bytes
 *   PostChancePending50  include/cugo/game/postchance50.h:22-28   32 bytes
 *   TorchEnv50           include/cugo/game/torch50.h:108-121     248 bytes
 */
#ifndef CUGO_ORACLE_TYPES_H_
#define CUGO_ORACLE_TYPES_H_

#include <stddef.h>
#include <stdint.h>
#include <string.h>

typedef uint8_t card_t;  /* month * 4 + slot; 48, 49 bonus; 0xff none (card.h:14-30) */
typedef uint64_t mask_t; /* one bit per card */

enum {
  MONTHS = 12,
  STD_CARDS = 48,
  DECK_CARDS = 50,
  BONUS2 = 48,
  BONUS3 = 49,
  NO_CARD = 0xff,
  NO_PLAYER = 0xff,
};

#define STD_MASK ((((mask_t)1) << STD_CARDS) - 1)
#define BONUS_MASK ((((mask_t)1) << BONUS2) | (((mask_t)1) << BONUS3))
#define DECK_MASK ((((mask_t)1) << DECK_CARDS) - 1)
#define ALL_MONTH_BITS ((uint16_t)0x0fff)

/* turn50.h:30-60 */
enum { PHASE_PLAY = 0, PHASE_DRAW = 1, PHASE_RESOLVE = 2 };
enum { TS_OK = 0, TS_WRONG_PHASE = 1, TS_INVALID_CARD = 2, TS_NOT_IN_HAND = 3, TS_STOCK_EMPTY = 4 };
enum { RS_OK = 0, RS_WRONG_PHASE = 1, RS_CHOICE_REQUIRED = 2, RS_INVALID_CHOICE = 3,
       RS_UNSUPPORTED_LAST = 4 };
enum { EV_PPUK = 1, EV_JJOK = 2, EV_TTADAK = 4, EV_SWEEP = 8 };

typedef struct {
  mask_t hand0, hand1, floor, stock, captured0, captured1;
  uint64_t rng;
  mask_t pending_bonus;
  uint16_t ppuk_months, owner1, bonus2_ppuk, bonus3_ppuk, turn_index;
  uint8_t actor, phase;
  card_t pending_played, pending_drawn;
  mask_t mission;
  uint16_t neutral_ppuk;
} Turn;

typedef struct {
  Turn turn;
  uint8_t go0, go1, last_go0, last_go1, decision_actor, winner, gukjin_decision;
} Game;

typedef struct {
  Game game;
  uint16_t shaken0, shaken1;
  uint8_t bombs0, bombs1, credits0, credits1;
  uint16_t shaken4_0, shaken4_1;
} Special;

typedef struct {
  Special sp;
  uint8_t ppuk_count0, ppuk_count1, streak0, streak1, ct_actor;
  uint16_t ct_months;
  uint8_t winner, reason;
  uint64_t points;
  int32_t side0;
  uint8_t round_mult, mission_type, mission_mult, mm0, mm1;
  mask_t held0, held1, revealed0, revealed1;
} Terminal;

typedef struct {
  uint8_t kind;
  card_t card;
  uint8_t month;
  card_t played_match, drawn_match;
  mask_t pi_cards;
} Action;

typedef struct {
  Action action;
  mask_t selected_pi;
  uint16_t primary_action;
  uint8_t actor, active;
} Pending;

typedef struct {
  Terminal g;
  Pending pending;
  uint16_t n_primary, n_choice, n_resolve, n_pi, n_bonus, n_special, n_go;
  uint8_t status, done, nagari;
} Env;

_Static_assert(sizeof(Turn) == 96, "TurnState50 size");
_Static_assert(offsetof(Turn, ppuk_months) == 64 && offsetof(Turn, turn_index) == 72 &&
                   offsetof(Turn, actor) == 74 && offsetof(Turn, mission) == 80 &&
                   offsetof(Turn, neutral_ppuk) == 88,
               "TurnState50 offsets");
_Static_assert(sizeof(Game) == 104 && offsetof(Game, go0) == 96, "GameState50");
_Static_assert(sizeof(Special) == 120 && offsetof(Special, shaken4_1) == 114, "SpecialGameState50");
_Static_assert(sizeof(Terminal) == 192 && offsetof(Terminal, ct_months) == 126 &&
                   offsetof(Terminal, points) == 136 && offsetof(Terminal, side0) == 144 &&
                   offsetof(Terminal, mm1) == 152 && offsetof(Terminal, held0) == 160,
               "TerminalGameState50");
_Static_assert(sizeof(Action) == 16 && offsetof(Action, pi_cards) == 8, "Action50");
_Static_assert(sizeof(Pending) == 32 && offsetof(Pending, active) == 27, "PostChancePending50");
_Static_assert(sizeof(Env) == 248 && offsetof(Env, pending) == 192 && offsetof(Env, n_primary) == 224 &&
                   offsetof(Env, status) == 238 && offsetof(Env, nagari) == 240,
               "TorchEnv50");

/* Byte ranges of a row that hold no field: written as zero. */
static const int kPadRanges[10][2] = {{78, 80},   {90, 96},   {103, 104}, {116, 120}, {125, 126},
                                      {130, 136}, {153, 160}, {197, 200}, {220, 224}, {241, 248}};

/* score breakdown (hwatu.h:111-122) */
typedef struct {
  uint8_t bright_count, animal_count, ribbon_count, pi_units;
  uint8_t bright_points, animal_points, ribbon_points, pi_points, flags, total;
} Score;

#endif
