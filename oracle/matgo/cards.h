/*
 * Oracle restatement (plain C), part 1: cards, RNG, scoring, deal, bonus cards and the
 * persistent Gukjin role.  TEST INFRASTRUCTURE ONLY.
 */
#ifndef CUGO_ORACLE_CARDS_H_
#define CUGO_ORACLE_CARDS_H_

#include "types.h"

/* ---- card.h:14-120 ---- */
static inline mask_t cbit(card_t c) { return ((mask_t)1) << c; }
static inline uint8_t cmonth(card_t c) { return (uint8_t)(c >> 2); }
static inline card_t mkcard(unsigned month, unsigned slot) { return (card_t)((month << 2) | slot); }
static inline mask_t month_cards(unsigned month) { return ((mask_t)0xf) << (month * 4u); }
static inline int is_standard(card_t c) { return c < STD_CARDS; }
static inline int is_bonus(card_t c) { return c == BONUS2 || c == BONUS3; }
static inline int is_physical(card_t c) { return c < DECK_CARDS; }
static inline int ccount(mask_t m) { return __builtin_popcountll(m); }
static inline card_t first_of(mask_t m) { return m ? (card_t)__builtin_ctzll(m) : NO_CARD; }
static inline card_t pop_first(mask_t* m) {
  const card_t c = first_of(*m);
  if (c != NO_CARD) *m &= *m - 1;
  return c;
}
/* card.h:97-120 (host branch): drop `rank` lowest bits, then the lowest remaining */
static card_t select_by_rank(mask_t m, uint32_t rank) {
  if (rank >= (uint32_t)ccount(m)) return NO_CARD;
  while (rank-- != 0u) m &= m - 1;
  return first_of(m);
}
static inline uint16_t month_bit(card_t c) { return (uint16_t)(1u << cmonth(c)); }

/* ---- rng.h:13-60 ---- */
static uint64_t splitmix_next(uint64_t* state) {
  uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static uint32_t uniform_bounded(uint64_t* state, uint32_t bound) {
  if (bound <= 1u) return 0u;
  for (;;) {
    const uint32_t x = (uint32_t)(splitmix_next(state) >> 32);
    const uint64_t product = (uint64_t)x * bound;
    const uint32_t low = (uint32_t)product;
    if (low < bound) {
      const uint32_t threshold = (0u - bound) % bound;
      if (low < threshold) continue;
    }
    return (uint32_t)(product >> 32);
  }
}

/* ---- hwatu.h:18-199 ---- */
#define C_(m, s) (((mask_t)1) << ((m) * 4 + (s)))
#define BRIGHT_MASK (C_(0, 0) | C_(2, 0) | C_(7, 0) | C_(10, 0) | C_(11, 0))
#define RAIN_BRIGHT 44 /* make_card(11, 0) */
#define ANIMAL_MASK \
  (C_(1, 0) | C_(3, 0) | C_(4, 0) | C_(5, 0) | C_(6, 0) | C_(7, 1) | C_(8, 0) | C_(9, 0) | C_(11, 1))
#define GUKJIN 32 /* make_card(8, 0) */
#define RIBBON_MASK                                                                        \
  (C_(0, 1) | C_(1, 1) | C_(2, 1) | C_(3, 1) | C_(4, 1) | C_(5, 1) | C_(6, 1) | C_(8, 1) | \
   C_(9, 1) | C_(11, 2))
#define DOUBLE_PI_MASK (C_(10, 1) | C_(11, 3))
#define GODORI_MASK (C_(1, 0) | C_(3, 0) | C_(7, 1))
#define HONGDAN_MASK (C_(0, 1) | C_(1, 1) | C_(2, 1))
#define CHODAN_MASK (C_(3, 1) | C_(4, 1) | C_(6, 1))
#define CHEONGDAN_MASK (C_(5, 1) | C_(8, 1) | C_(9, 1))

static mask_t plain_pi_mask(void) { /* slots 2, 3 of months 0..10 */
  mask_t m = 0;
  for (unsigned month = 0; month < 11; ++month) m |= C_(month, 2) | C_(month, 3);
  return m;
}

enum { SF_GODORI = 1, SF_HONGDAN = 2, SF_CHODAN = 4, SF_CHEONGDAN = 8, SF_MEONGTTA = 16 };

static mask_t pi_card_mask(mask_t cards, int gukjin_pi) { /* hwatu.h:133-140 */
  mask_t m = cards & (plain_pi_mask() | DOUBLE_PI_MASK | BONUS_MASK);
  if (gukjin_pi) m |= cards & cbit(GUKJIN);
  return m;
}

static uint8_t pi_units(mask_t cards, int gukjin_pi) { /* hwatu.h:141-151 */
  unsigned u = (unsigned)ccount(cards & plain_pi_mask());
  u += 2u * (unsigned)ccount(cards & DOUBLE_PI_MASK);
  if (cards & cbit(BONUS2)) u += 2u;
  if (cards & cbit(BONUS3)) u += 3u;
  if (gukjin_pi && (cards & cbit(GUKJIN))) u += 2u;
  return (uint8_t)u;
}

static int has_all(mask_t cards, mask_t subset) { return (cards & subset) == subset; }

static Score score_captured(mask_t cards, int gukjin_pi) { /* hwatu.h:153-199 */
  Score s;
  memset(&s, 0, sizeof s);
  s.bright_count = (uint8_t)ccount(cards & BRIGHT_MASK);
  mask_t animals = cards & ANIMAL_MASK;
  if (gukjin_pi) animals &= ~cbit(GUKJIN);
  s.animal_count = (uint8_t)ccount(animals);
  s.ribbon_count = (uint8_t)ccount(cards & RIBBON_MASK);
  s.pi_units = pi_units(cards, gukjin_pi);
  if (s.bright_count == 3) s.bright_points = (cards & cbit(RAIN_BRIGHT)) ? 2 : 3;
  else if (s.bright_count == 4) s.bright_points = 4;
  else if (s.bright_count == 5) s.bright_points = 15;
  s.animal_points = s.animal_count >= 5 ? (uint8_t)(s.animal_count - 4) : 0;
  if (has_all(animals, GODORI_MASK)) {
    s.flags |= SF_GODORI;
    s.animal_points = (uint8_t)(s.animal_points + 5u);
  }
  if (s.animal_count >= 7) s.flags |= SF_MEONGTTA;
  s.ribbon_points = s.ribbon_count >= 5 ? (uint8_t)(s.ribbon_count - 4) : 0;
  if (has_all(cards, HONGDAN_MASK)) { s.flags |= SF_HONGDAN; s.ribbon_points = (uint8_t)(s.ribbon_points + 3u); }
  if (has_all(cards, CHODAN_MASK)) { s.flags |= SF_CHODAN; s.ribbon_points = (uint8_t)(s.ribbon_points + 3u); }
  if (has_all(cards, CHEONGDAN_MASK)) { s.flags |= SF_CHEONGDAN; s.ribbon_points = (uint8_t)(s.ribbon_points + 3u); }
  s.pi_points = s.pi_units >= 10 ? (uint8_t)(s.pi_units - 9) : 0;
  s.total = (uint8_t)((unsigned)s.bright_points + s.animal_points + s.ribbon_points + s.pi_points);
  return s;
}

/* ---- deal.h:50-101 (no forced-draw hook: host replay only) ---- */
static card_t draw_uniform_card(mask_t* remaining, uint64_t* rng) {
  const uint32_t count = (uint32_t)ccount(*remaining);
  if (count == 0u) return NO_CARD;
  const uint32_t rank = uniform_bounded(rng, count);
  const card_t card = select_by_rank(*remaining, rank);
  *remaining &= ~cbit(card);
  return card;
}

static card_t draw_stock_card(mask_t* stock, uint64_t* rng_state) { /* deal.h:70-80 */
  if (*stock == 0) return NO_CARD;
  uint64_t s = *rng_state;
  const card_t card = draw_uniform_card(stock, &s);
  *rng_state = s;
  return card;
}

typedef struct {
  mask_t hand0, hand1, floor, stock, captured0, captured1;
  uint64_t rng;
} Deal;

static Deal deal_50(uint64_t seed) { /* deal.h:82-92 */
  Deal d;
  uint64_t s = seed;
  mask_t remaining = DECK_MASK;
  d.hand0 = d.hand1 = d.floor = 0;
  for (int i = 0; i < 10; ++i) d.hand0 |= cbit(draw_uniform_card(&remaining, &s));
  for (int i = 0; i < 10; ++i) d.hand1 |= cbit(draw_uniform_card(&remaining, &s));
  for (int i = 0; i < 8; ++i) d.floor |= cbit(draw_uniform_card(&remaining, &s));
  d.stock = remaining;
  d.captured0 = d.captured1 = 0;
  d.rng = s;
  return d;
}

/* ---- bonus.h:37-81 ---- */
enum { BP_OK = 0, BP_NOT_BONUS = 1, BP_NOT_IN_HAND = 2, BP_STOCK_EMPTY = 3 };
typedef struct { uint8_t status; card_t replacement; uint8_t steal; } BonusPlay;

static BonusPlay play_hand_bonus(mask_t* hand, mask_t* stock, mask_t* captured, uint64_t* rng,
                                 card_t bonus) {
  BonusPlay r = {BP_NOT_BONUS, NO_CARD, 0};
  if (!is_bonus(bonus)) return r;
  if ((*hand & cbit(bonus)) == 0) { r.status = BP_NOT_IN_HAND; return r; }
  if (*stock == 0) { r.status = BP_STOCK_EMPTY; return r; }
  mask_t next_stock = *stock;
  uint64_t next_rng = *rng;
  const card_t rep = draw_stock_card(&next_stock, &next_rng);
  if (!is_physical(rep)) { r.status = BP_STOCK_EMPTY; return r; }
  *hand = (*hand & ~cbit(bonus)) | cbit(rep);
  *captured |= cbit(bonus);
  *stock = next_stock;
  *rng = next_rng;
  r.status = BP_OK;
  r.replacement = rep;
  r.steal = 1;
  return r;
}

typedef struct { card_t card; mask_t bonuses; } Flip;

static Flip draw_with_bonus_chain(mask_t* stock, uint64_t* rng) { /* bonus.h:68-81 */
  Flip f = {NO_CARD, 0};
  while (*stock != 0) {
    const card_t c = draw_stock_card(stock, rng);
    if (is_bonus(c)) { f.bonuses |= cbit(c); continue; }
    f.card = c;
    return f;
  }
  return f;
}

/* ---- gukjin_state.h:19-173: role bits live in owner1 bits 12-15 ---- */
#define GUKJIN_PI0 ((uint16_t)(1u << 12))
#define GUKJIN_PI1 ((uint16_t)(1u << 13))
#define GUKJIN_LOCK0 ((uint16_t)(1u << 14))
#define GUKJIN_LOCK1 ((uint16_t)(1u << 15))

static mask_t captured_of(const Turn* t, unsigned player) {
  return (player & 1u) == 0 ? t->captured0 : t->captured1;
}
static uint16_t gukjin_pi_flag(unsigned player) { return (player & 1u) == 0 ? GUKJIN_PI0 : GUKJIN_PI1; }
static uint16_t gukjin_lock_flag(unsigned player) { return (player & 1u) == 0 ? GUKJIN_LOCK0 : GUKJIN_LOCK1; }
static int gukjin_role_pi(const Turn* t, unsigned player) { return (t->owner1 & gukjin_pi_flag(player)) != 0; }
/* persistent_score_options_for_player50: Gukjin counts as double pi when owned and flagged */
static int gukjin_as_pi(const Turn* t, unsigned player) {
  return (captured_of(t, player) & cbit(GUKJIN)) != 0 && gukjin_role_pi(t, player);
}
static Score score_player(const Turn* t, unsigned player) {
  return score_captured(captured_of(t, player), gukjin_as_pi(t, player));
}
static int gukjin_locked(const Turn* t, unsigned player) { return (t->owner1 & gukjin_lock_flag(player)) != 0; }
static int gukjin_undecided(const Turn* t, unsigned player) {
  return (captured_of(t, player) & cbit(GUKJIN)) != 0 && !gukjin_role_pi(t, player) &&
         !gukjin_locked(t, player);
}
static int decide_gukjin(Turn* t, unsigned player, int as_pi) { /* gukjin_state.h:117-123 */
  if (!gukjin_undecided(t, player)) return 0;
  t->owner1 |= gukjin_lock_flag(player);
  if (as_pi) t->owner1 |= gukjin_pi_flag(player);
  return 1;
}
static int gukjin_prompt_due(const Turn* t, unsigned player, unsigned go_count) { /* :127-136 */
  if (!gukjin_undecided(t, player)) return 0;
  const mask_t cap = captured_of(t, player);
  if (pi_units(cap, 0) < 8u) return 0;
  const unsigned converted = score_captured(cap, 1).total;
  return converted + go_count >= 7u;
}
static void auto_decide_loser_gukjin(Turn* t, unsigned loser) { /* :141-148 */
  const uint8_t pi = pi_units(captured_of(t, loser), gukjin_as_pi(t, loser));
  if (pi == 6u || pi == 7u) decide_gukjin(t, loser, 1);
  else if (pi == 0u) decide_gukjin(t, loser, 0);
}

#endif
