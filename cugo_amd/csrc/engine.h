// Shin Matgo (50-card Hangame Go-Stop) rules engine for one game per GPU lane.
//
// Host+device C++ for gfx950.  A game lives in registers as an `Env` (flat scalars, no
// arrays, no pointers into it) and in HBM as the reference's 248-byte row; load_row /
// store_row convert between the two with 31 whole 64-bit words, padding bytes written
// as zero.  The rules restate the reference headers function by function (citations
// are file:line in the reference), in the same order of state updates, so every
// status code, counter and card mask matches the reference engine bit for bit; the
// GPU-facing differences are in data handling only:
//   * per-player pairs are selected with conditionals instead of references, so the
//     whole state stays SROA-able into VGPRs (no private-memory copies);
//   * the legality check of a step builds the action mask only (the reference builds
//     the full observation packet, torch50.h:499, whose other fields it discards);
//   * the nth-set-bit select for stock draws is a branch-free popcount bisection.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define CG_HD __host__ __device__ __forceinline__

namespace cugo_amd {

using u8 = uint8_t;
using u16 = uint16_t;
using u32 = uint32_t;
using u64 = uint64_t;
using i16 = int16_t;
using i32 = int32_t;
using i64 = int64_t;

// ------------------------------------------------------------------ constants ----
// Card ids are month * 4 + slot (card.h:14-63); 48 and 49 are the bonus two-pi and
// three-pi.  A card set is a 50-bit mask.
constexpr u8 kNoCard = 0xFF;
constexpr u8 kBonus2 = 48;
constexpr u8 kBonus3 = 49;
constexpr u64 kStdMask = (1ull << 48) - 1;
constexpr u64 kBonusMask = 3ull << 48;
constexpr u64 kDeckMask = (1ull << 50) - 1;
constexpr u16 kMonthBits = 0x0FFF;
constexpr u8 kNoPlayer = 0xFF;

constexpr u64 C(u32 month, u32 slot) { return 1ull << (month * 4 + slot); }
// hwatu.h:18-90
constexpr u64 kBright = C(0, 0) | C(2, 0) | C(7, 0) | C(10, 0) | C(11, 0);
constexpr u8 kRainBright = 44;
constexpr u64 kAnimal = C(1, 0) | C(3, 0) | C(4, 0) | C(5, 0) | C(6, 0) | C(7, 1) | C(8, 0) |
                        C(9, 0) | C(11, 1);
constexpr u8 kGukjin = 32;
constexpr u64 kRibbon = C(0, 1) | C(1, 1) | C(2, 1) | C(3, 1) | C(4, 1) | C(5, 1) | C(6, 1) |
                        C(8, 1) | C(9, 1) | C(11, 2);
// Slots 2 and 3 of months 1..11 (hwatu.h:51-62, identical to turn50.h:30-37).
constexpr u64 kPlainPi = 0x0CCCCCCCCCCCull;
constexpr u64 kDoublePi = C(10, 1) | C(11, 3);
constexpr u64 kGodori = C(1, 0) | C(3, 0) | C(7, 1);
constexpr u64 kHongdan = C(0, 1) | C(1, 1) | C(2, 1);
constexpr u64 kChodan = C(3, 1) | C(4, 1) | C(6, 1);
constexpr u64 kCheongdan = C(5, 1) | C(8, 1) | C(9, 1);
static_assert((kBright | kAnimal | kRibbon | kPlainPi | kDoublePi) == kStdMask, "classes");

// Enumerations of the reference, same numeric values.
enum : u8 { kPlayCard = 0, kPlayBonus, kShake, kBomb, kGrenade, kBombCredit, kGo, kStop,
            kChongtongWin, kChongtongContinue, kGukjinPi, kGukjinAnimal };  // rollout50.h:18-31
enum : u8 { kOk = 0, kWrongPhase, kInvalidAction, kNotLegal, kStockEmpty,
            kResolveChoiceRequired, kInvalidResolveChoice, kPiSelectionRequired,
            kInvalidPiSelection, kGameFinished };                            // rollout50.h:33-44
enum : u8 { kPhasePlay = 0, kPhaseDraw = 1, kPhaseResolve = 2 };             // turn50.h:39-43
// Turn50Status (turn50.h:45-51)
enum : u8 { kTurnOk = 0, kTurnWrongPhase, kTurnInvalidCard, kTurnNotInHand, kTurnStockEmpty };
// Resolve50Status (turn50.h:53-59)
enum : u8 { kResOk = 0, kResWrongPhase, kResChoiceRequired, kResInvalidChoice };
enum : u8 { kEvPpuk = 1, kEvJjok = 2, kEvTtadak = 4, kEvSweep = 8 };       // turn50.h:61-67
// PiTransferStatus (pi_transfer.h:19-23)
enum : u8 { kPiOk = 0, kPiSelRequired, kPiInvalidSelection };
// SpecialStatus50 (special50.h:16-19)
enum : u8 { kSpOk = 0, kSpWrongPhase, kSpInvalidCard, kSpInvalidMonth, kSpNotLegal,
            kSpStockEmpty, kSpResolveChoiceRequired, kSpInvalidResolveChoice,
            kSpPiSelectionRequired, kSpInvalidPiSelection };
// TerminalReason50 (terminal50.h:44-51)
enum : u8 { kReasonNone = 0, kReasonStop, kReasonInitialChongtong, kReasonFloorChongtong,
            kReasonBonusChongtong, kReasonThreePpuk };
// PpukState50 (terminal50.h:24-32)
enum : u8 { kPpukNone = 0, kPpukFirst, kPpukSecond, kPpukThird, kPpukOne, kPpukTwo, kPpukThree };
// MissionType50 (terminal50.h:35-42)
enum : u8 { kMissionNone = 0, kMissionEasy = 1, kMissionNormal = 2, kMissionHard = 3,
            kMissionNoCondition = 4, kMissionTriple = 6 };
// Decision kinds: PolicyDecision50 (policy50.h:36-42) + PostChanceDecision50
// (postchance50.h:15-20).
enum : u8 { kDecNone = 0, kDecPrimary = 1, kDecGoStop = 2, kDecChongtong = 3,
            kDecResolvePlayed = 4, kDecResolveDrawn = 5, kDecPiCard = 6, kDecGukjin = 7 };

// Unified action space (policy50.h:15-34, torch50.h:16-23).
constexpr u16 kActBonus = 48, kActShake = 50, kActBomb = 98, kActGrenade = 110,
              kActBombCredit = 122, kActGo = 123, kActStop = 124, kActCtWin = 125,
              kActCtContinue = 126, kActPrimaryCount = 127, kActChoice = 127,
              kActGukjinPi = 177, kActGukjinAnimal = 178, kActionCount = 179,
              kInvalidAction16 = 0xFFFF;
constexpr int kFeatureCount = 720;
constexpr int kEventWords = 9;
constexpr int kStartWords = 8;
constexpr int kRowWords = 31;  // 248-byte row

constexpr u8 kLastTurnIndex = 18;  // turn50.h:27
constexpr u8 kDecisionBasePoints = 7;  // game50.h:16

// ---------------------------------------------------------------- bit helpers ----
CG_HD u64 bit(u32 c) { return 1ull << (c & 63u); }
CG_HD u64 month_cards(u32 m) { return 0xFull << ((4u * m) & 63u); }
CG_HD u32 popc(u64 x) { return (u32)__builtin_popcountll(x); }
CG_HD u8 first_card(u64 m) { return m ? (u8)__builtin_ctzll(m) : kNoCard; }
CG_HD u32 ctz64(u64 x) { return (u32)__builtin_ctzll(x); }  // x != 0
CG_HD bool is_std(u8 c) { return c < 48; }
CG_HD bool is_bonus_card(u8 c) { return c == kBonus2 || c == kBonus3; }
CG_HD bool is_physical(u8 c) { return c < 50; }
CG_HD u16 month_bit(u8 c) { return (u16)(1u << ((c >> 2) & 15u)); }

// Index of the rank-th set bit (card.h:97-120).  Bisection on popcounts of the low
// half, quarter, ... so every lane runs the same six steps whatever the rank.
CG_HD u8 select_rank(u64 mask, u32 rank) {
  if (rank >= popc(mask)) return kNoCard;
  u32 pos = 0;
  u32 c = popc(mask & 0xFFFFFFFFull);
  if (rank >= c) { rank -= c; mask >>= 32; pos += 32; }
  c = popc(mask & 0xFFFFull);
  if (rank >= c) { rank -= c; mask >>= 16; pos += 16; }
  c = popc(mask & 0xFFull);
  if (rank >= c) { rank -= c; mask >>= 8; pos += 8; }
  c = popc(mask & 0xFull);
  if (rank >= c) { rank -= c; mask >>= 4; pos += 4; }
  c = popc(mask & 0x3ull);
  if (rank >= c) { rank -= c; mask >>= 2; pos += 2; }
  c = (u32)(mask & 1ull);
  if (rank >= c) { pos += 1; }
  return (u8)pos;
}

// ------------------------------------------------------------ month nibbles ----
// A card mask holds month m in bits 4m..4m+3, so per-month questions are nibble-parallel
// bit arithmetic instead of twelve-iteration loops.
constexpr u64 kNibbleLow = 0x111111111111ull;  // bit 4m of each of the 12 months

// bit 4m -> bit m for m < 12 (other bits must be clear)
CG_HD u16 gather_months(u64 x) {
  x = (x | (x >> 3)) & 0x0303030303030303ull;
  x = (x | (x >> 6)) & 0x000F000F000F000Full;
  x = (x | (x >> 12)) & 0x000000FF000000FFull;
  x = (x | (x >> 24)) & 0xFFFFull;
  return (u16)(x & 0x0FFFu);
}
// bit m -> nibble 0xF of month m: the cards of the given months
CG_HD u64 month_cards_of(u16 months) {
  u64 x = months & 0x0FFFu;
  x = (x | (x << 24)) & 0x000000FF000000FFull;
  x = (x | (x << 12)) & 0x000F000F000F000Full;
  x = (x | (x << 6)) & 0x0303030303030303ull;
  x = (x | (x << 3)) & kNibbleLow;
  return x * 0xFull;
}
// each nibble := number of cards of that month (0..4)
CG_HD u64 month_counts(u64 cards) {
  cards &= kStdMask;
  cards = cards - ((cards >> 1) & 0x5555555555555555ull);
  return (cards & 0x3333333333333333ull) + ((cards >> 2) & 0x3333333333333333ull);
}
// months whose count nibble equals k (k <= 4; counts <= 4, so count ^ k fits 3 bits)
CG_HD u16 months_with_count(u64 counts, u32 k) {
  const u64 d = counts ^ (kNibbleLow * k);
  const u64 nonzero = (d | (d >> 1) | (d >> 2)) & kNibbleLow;
  return gather_months(~nonzero & kNibbleLow);
}

// --------------------------------------------------------------------- rng.h ----
// SplitMix64 (rng.h:13-32): the state is advanced in place.
CG_HD u64 sm_next(u64& s) {
  s += 0x9e3779b97f4a7c15ull;
  u64 z = s;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Lemire's bounded draw with rejection (rng.h:34-54).  The rejection threshold
// (2^32 - bound) % bound is below bound, so a first draw with low >= bound is accepted
// without it; only the rare low < bound case computes the modulo (written this way the
// integer division stays in that branch instead of running for every draw) and redraws
// while low < threshold, exactly as the reference loop does.
CG_HD u32 uniform_bounded(u64& s, u32 bound) {
  if (bound <= 1u) return 0u;
  u64 product = (u64)(u32)(sm_next(s) >> 32) * bound;
  u32 low = (u32)product;
  if (low < bound) {
    const u32 threshold = (0u - bound) % bound;
    while (low < threshold) {
      product = (u64)(u32)(sm_next(s) >> 32) * bound;
      low = (u32)product;
    }
  }
  return (u32)(product >> 32);
}

// deal.h:50-80: draw a uniform card from `remaining` with the stream `s`.
CG_HD u8 draw_uniform(u64& remaining, u64& s) {
  const u32 count = popc(remaining);
  if (count == 0u) return kNoCard;
  const u32 rank = uniform_bounded(s, count);
  const u8 card = select_rank(remaining, rank);
  remaining &= ~bit(card);
  return card;
}

// bonus.h:68-81: flip until a standard card; bonus cards collected on the way.
struct Flip { u8 card; u64 bonuses; };
CG_HD Flip draw_with_bonus_chain(u64& stock, u64& s) {
  u64 bonuses = 0;
  while (stock != 0) {
    const u8 card = draw_uniform(stock, s);
    if (is_bonus_card(card)) { bonuses |= bit(card); continue; }
    return Flip{card, bonuses};
  }
  return Flip{kNoCard, bonuses};
}

// ------------------------------------------------------------------- hwatu.h ----
struct Score {
  u8 bright_count, animal_count, ribbon_count, pi_units;
  u8 flags, total;
};
constexpr u8 kFlagMeongtta = 16;

CG_HD u64 pi_card_mask(u64 cards, bool gukjin_pi) {  // hwatu.h:131-139
  u64 m = cards & (kPlainPi | kDoublePi | kBonusMask);
  if (gukjin_pi) m |= cards & bit(kGukjin);
  return m;
}

CG_HD u8 pi_units(u64 cards, bool gukjin_pi) {  // hwatu.h:141-151
  u32 units = popc(cards & kPlainPi) + 2u * popc(cards & kDoublePi);
  if (cards & bit(kBonus2)) units += 2u;
  if (cards & bit(kBonus3)) units += 3u;
  if (gukjin_pi && (cards & bit(kGukjin))) units += 2u;
  return (u8)units;
}

CG_HD Score score_captured(u64 cards, bool gukjin_pi) {  // hwatu.h:153-199
  Score s;
  s.bright_count = (u8)popc(cards & kBright);
  u64 animals = cards & kAnimal;
  if (gukjin_pi) animals &= ~bit(kGukjin);
  s.animal_count = (u8)popc(animals);
  s.ribbon_count = (u8)popc(cards & kRibbon);
  s.pi_units = pi_units(cards, gukjin_pi);
  u8 bright_points = 0;
  if (s.bright_count == 3) bright_points = (cards & bit(kRainBright)) ? 2 : 3;
  else if (s.bright_count == 4) bright_points = 4;
  else if (s.bright_count == 5) bright_points = 15;
  u8 flags = 0;
  u8 animal_points = s.animal_count >= 5 ? (u8)(s.animal_count - 4) : 0;
  if ((animals & kGodori) == kGodori) { flags |= 1; animal_points = (u8)(animal_points + 5); }
  if (s.animal_count >= 7) flags |= kFlagMeongtta;
  u8 ribbon_points = s.ribbon_count >= 5 ? (u8)(s.ribbon_count - 4) : 0;
  if ((cards & kHongdan) == kHongdan) { flags |= 2; ribbon_points = (u8)(ribbon_points + 3); }
  if ((cards & kChodan) == kChodan) { flags |= 4; ribbon_points = (u8)(ribbon_points + 3); }
  if ((cards & kCheongdan) == kCheongdan) { flags |= 8; ribbon_points = (u8)(ribbon_points + 3); }
  const u8 pi_points = s.pi_units >= 10 ? (u8)(s.pi_units - 9) : 0;
  s.flags = flags;
  s.total = (u8)((u32)bright_points + animal_points + ribbon_points + pi_points);
  return s;
}

// ---------------------------------------------------------------------- Env ----
// Register form of the reference TorchEnv50 (torch50.h:108-121): TurnState50
// (turn50.h:92-115), GameState50 (game50.h:38-48), SpecialGameState50
// (special50.h:25-32), TerminalGameState50 (terminal50.h:74-102), PostChancePending50
// (postchance50.h:22-28) and the counters, flattened.
struct Env {
  u64 hand0, hand1, floor, stock, cap0, cap1, rng, pend_bonus;
  u16 ppuk, owner1, b2ppuk, b3ppuk, turn;
  u8 actor, phase, pplayed, pdrawn;
  u64 mission;
  u16 neutral;
  u8 go0, go1, lgo0, lgo1, dact, winner, gdec;
  u16 shaken0, shaken1;
  u8 bombs0, bombs1, cred0, cred1;
  u16 sh4_0, sh4_1;
  u8 pcount0, pcount1, streak0, streak1, ct_actor;
  u16 ct_months;
  u8 twinner, treason;
  u64 tpoints;
  i32 side0;
  u8 round, mtype, mmult, mm0, mm1;
  u64 held0, held1, rev0, rev1;
  // pending post-chance action (Action50 at 192, rollout50.h:46-52)
  u8 a_kind, a_card, a_month, a_pmatch, a_dmatch;
  u64 a_pisel;
  u64 sel_pi;
  u16 prim;
  u8 pactor, pactive;
  u16 n_primary, n_choice, n_resolve, n_pi, n_bonus, n_special, n_go;
  u8 status, done, nagari;
};

// The 248-byte row as 31 little-endian words; every byte not listed is padding.
CG_HD Env unpack_row(const u64* w) {
  Env e;
  e.hand0 = w[0]; e.hand1 = w[1]; e.floor = w[2]; e.stock = w[3];
  e.cap0 = w[4]; e.cap1 = w[5]; e.rng = w[6]; e.pend_bonus = w[7];
  e.ppuk = (u16)w[8]; e.owner1 = (u16)(w[8] >> 16); e.b2ppuk = (u16)(w[8] >> 32);
  e.b3ppuk = (u16)(w[8] >> 48);
  e.turn = (u16)w[9]; e.actor = (u8)(w[9] >> 16); e.phase = (u8)(w[9] >> 24);
  e.pplayed = (u8)(w[9] >> 32); e.pdrawn = (u8)(w[9] >> 40);
  e.mission = w[10];
  e.neutral = (u16)w[11];
  e.go0 = (u8)w[12]; e.go1 = (u8)(w[12] >> 8); e.lgo0 = (u8)(w[12] >> 16);
  e.lgo1 = (u8)(w[12] >> 24); e.dact = (u8)(w[12] >> 32); e.winner = (u8)(w[12] >> 40);
  e.gdec = (u8)(w[12] >> 48);
  e.shaken0 = (u16)w[13]; e.shaken1 = (u16)(w[13] >> 16); e.bombs0 = (u8)(w[13] >> 32);
  e.bombs1 = (u8)(w[13] >> 40); e.cred0 = (u8)(w[13] >> 48); e.cred1 = (u8)(w[13] >> 56);
  e.sh4_0 = (u16)w[14]; e.sh4_1 = (u16)(w[14] >> 16);
  e.pcount0 = (u8)w[15]; e.pcount1 = (u8)(w[15] >> 8); e.streak0 = (u8)(w[15] >> 16);
  e.streak1 = (u8)(w[15] >> 24); e.ct_actor = (u8)(w[15] >> 32);
  e.ct_months = (u16)(w[15] >> 48);
  e.twinner = (u8)w[16]; e.treason = (u8)(w[16] >> 8);
  e.tpoints = w[17];
  e.side0 = (i32)(u32)w[18]; e.round = (u8)(w[18] >> 32); e.mtype = (u8)(w[18] >> 40);
  e.mmult = (u8)(w[18] >> 48); e.mm0 = (u8)(w[18] >> 56);
  e.mm1 = (u8)w[19];
  e.held0 = w[20]; e.held1 = w[21]; e.rev0 = w[22]; e.rev1 = w[23];
  e.a_kind = (u8)w[24]; e.a_card = (u8)(w[24] >> 8); e.a_month = (u8)(w[24] >> 16);
  e.a_pmatch = (u8)(w[24] >> 24); e.a_dmatch = (u8)(w[24] >> 32);
  e.a_pisel = w[25];
  e.sel_pi = w[26];
  e.prim = (u16)w[27]; e.pactor = (u8)(w[27] >> 16); e.pactive = (u8)(w[27] >> 24);
  e.n_primary = (u16)w[28]; e.n_choice = (u16)(w[28] >> 16); e.n_resolve = (u16)(w[28] >> 32);
  e.n_pi = (u16)(w[28] >> 48);
  e.n_bonus = (u16)w[29]; e.n_special = (u16)(w[29] >> 16); e.n_go = (u16)(w[29] >> 32);
  e.status = (u8)(w[29] >> 48); e.done = (u8)(w[29] >> 56);
  e.nagari = (u8)w[30];
  return e;
}

CG_HD void pack_row(const Env& e, u64* w) {
  w[0] = e.hand0; w[1] = e.hand1; w[2] = e.floor; w[3] = e.stock;
  w[4] = e.cap0; w[5] = e.cap1; w[6] = e.rng; w[7] = e.pend_bonus;
  w[8] = (u64)e.ppuk | (u64)e.owner1 << 16 | (u64)e.b2ppuk << 32 | (u64)e.b3ppuk << 48;
  w[9] = (u64)e.turn | (u64)e.actor << 16 | (u64)e.phase << 24 | (u64)e.pplayed << 32 |
         (u64)e.pdrawn << 40;
  w[10] = e.mission;
  w[11] = e.neutral;
  w[12] = (u64)e.go0 | (u64)e.go1 << 8 | (u64)e.lgo0 << 16 | (u64)e.lgo1 << 24 |
          (u64)e.dact << 32 | (u64)e.winner << 40 | (u64)e.gdec << 48;
  w[13] = (u64)e.shaken0 | (u64)e.shaken1 << 16 | (u64)e.bombs0 << 32 | (u64)e.bombs1 << 40 |
          (u64)e.cred0 << 48 | (u64)e.cred1 << 56;
  w[14] = (u64)e.sh4_0 | (u64)e.sh4_1 << 16;
  w[15] = (u64)e.pcount0 | (u64)e.pcount1 << 8 | (u64)e.streak0 << 16 | (u64)e.streak1 << 24 |
          (u64)e.ct_actor << 32 | (u64)e.ct_months << 48;
  w[16] = (u64)e.twinner | (u64)e.treason << 8;
  w[17] = e.tpoints;
  w[18] = (u64)(u32)e.side0 | (u64)e.round << 32 | (u64)e.mtype << 40 | (u64)e.mmult << 48 |
          (u64)e.mm0 << 56;
  w[19] = e.mm1;
  w[20] = e.held0; w[21] = e.held1; w[22] = e.rev0; w[23] = e.rev1;
  w[24] = (u64)e.a_kind | (u64)e.a_card << 8 | (u64)e.a_month << 16 | (u64)e.a_pmatch << 24 |
          (u64)e.a_dmatch << 32;
  w[25] = e.a_pisel;
  w[26] = e.sel_pi;
  w[27] = (u64)e.prim | (u64)e.pactor << 16 | (u64)e.pactive << 24;
  w[28] = (u64)e.n_primary | (u64)e.n_choice << 16 | (u64)e.n_resolve << 32 |
          (u64)e.n_pi << 48;
  w[29] = (u64)e.n_bonus | (u64)e.n_special << 16 | (u64)e.n_go << 32 | (u64)e.status << 48 |
          (u64)e.done << 56;
  w[30] = e.nagari;
}

// Per-player field access (player bit 0 selects).  Both fields are read and combined
// arithmetically: a conditional read of one of two adjacent fields would be folded by
// the optimiser into a read at a computed offset, which pins the whole Env in private
// (scratch) memory instead of registers.
template <class T>
CG_HD T pick(T v0, T v1, u32 p) {
  const T m = (T)(0 - (T)(p & 1u));
  return (T)((v0 & (T)~m) | (v1 & m));
}
CG_HD u64 hand_of(const Env& e, u32 p) { return pick<u64>(e.hand0, e.hand1, p); }
CG_HD void set_hand(Env& e, u32 p, u64 v) {
  const u64 a = e.hand0, b = e.hand1;
  e.hand0 = pick<u64>(v, a, p);
  e.hand1 = pick<u64>(b, v, p);
}
CG_HD u64 cap_of(const Env& e, u32 p) { return pick<u64>(e.cap0, e.cap1, p); }
CG_HD void set_cap(Env& e, u32 p, u64 v) {
  const u64 a = e.cap0, b = e.cap1;
  e.cap0 = pick<u64>(v, a, p);
  e.cap1 = pick<u64>(b, v, p);
}
CG_HD u8 go_of(const Env& e, u32 p) { return pick<u8>(e.go0, e.go1, p); }
CG_HD u8 lgo_of(const Env& e, u32 p) { return pick<u8>(e.lgo0, e.lgo1, p); }
CG_HD u16 shaken_of(const Env& e, u32 p) { return pick<u16>(e.shaken0, e.shaken1, p); }
CG_HD u16 sh4_of(const Env& e, u32 p) { return pick<u16>(e.sh4_0, e.sh4_1, p); }
CG_HD u8 bombs_of(const Env& e, u32 p) { return pick<u8>(e.bombs0, e.bombs1, p); }
CG_HD u8 cred_of(const Env& e, u32 p) { return pick<u8>(e.cred0, e.cred1, p); }
CG_HD void set_cred(Env& e, u32 p, u8 v) {
  const u8 a = e.cred0, b = e.cred1;
  e.cred0 = pick<u8>(v, a, p);
  e.cred1 = pick<u8>(b, v, p);
}
CG_HD u8 pcount_of(const Env& e, u32 p) { return pick<u8>(e.pcount0, e.pcount1, p); }
CG_HD u8 streak_of(const Env& e, u32 p) { return pick<u8>(e.streak0, e.streak1, p); }
CG_HD u8 mm_of(const Env& e, u32 p) { return pick<u8>(e.mm0, e.mm1, p); }
CG_HD void set_mm(Env& e, u32 p, u8 v) {
  const u8 a = e.mm0, b = e.mm1;
  e.mm0 = pick<u8>(v, a, p);
  e.mm1 = pick<u8>(b, v, p);
}
CG_HD u64 held_of(const Env& e, u32 p) { return pick<u64>(e.held0, e.held1, p); }
CG_HD u64 rev_of(const Env& e, u32 p) { return pick<u64>(e.rev0, e.rev1, p); }

// -------------------------------------------------------------------- turn50 ----
CG_HD u64 active_hand(const Env& e) { return hand_of(e, e.actor); }
CG_HD u64 std_floor(const Env& e) { return e.floor & kStdMask; }
CG_HD u64 floor_matches(const Env& e, u8 card) {
  return std_floor(e) & month_cards(card >> 2);
}
CG_HD bool is_last_turn(const Env& e) { return e.turn >= kLastTurnIndex; }  // turn50.h:194
CG_HD bool auto_floor_choice(u64 matches) {  // turn50.h:200-202
  return popc(matches) == 2 && (matches & ~kPlainPi) == 0;
}
CG_HD u16 floor_triple_months(u64 floor) {  // turn50.h:139-146
  return months_with_count(month_counts(floor), 3);
}

struct Resolve {
  u8 status, events, own_ppuk, opp_ppuk;
  u64 captured;
  u8 last_turn;
};
CG_HD Resolve resolve_error(u8 status) { return Resolve{status, 0, 0, 0, 0, 0}; }

CG_HD void capture_cards(Env& e, u64 cards, Resolve& r) {  // turn50.h:350-359
  set_cap(e, e.actor, cap_of(e, e.actor) | cards);
  r.captured |= cards;
}

// turn50.h:361-407
CG_HD u8 resolve_card_against_floor(Env& e, u8 card, u8 choice, Resolve& r) {
  const u64 b = bit(card);
  const u64 matches = floor_matches(e, card);
  const u32 count = popc(matches);
  if (count == 0) { e.floor |= b; return kResOk; }
  u64 capture;
  if (count == 1) {
    capture = matches;
  } else if (count == 2) {
    if (auto_floor_choice(matches) && (choice == kNoCard || (matches & bit(choice)) == 0))
      choice = first_card(matches);
    if (choice == kNoCard) return kResChoiceRequired;
    if (!is_std(choice) || (matches & bit(choice)) == 0) return kResInvalidChoice;
    capture = bit(choice);
  } else {
    capture = matches;
    const u16 mb = month_bit(card);
    if (e.ppuk & mb) {
      if (e.b2ppuk & mb) capture |= bit(kBonus2);      // turn50.h:221-232
      if (e.b3ppuk & mb) capture |= bit(kBonus3);
      e.b2ppuk &= (u16)~mb;                            // turn50.h:234-239
      e.b3ppuk &= (u16)~mb;
      const u8 owner = (e.owner1 & mb) ? 1 : 0;        // turn50.h:332-348
      if (owner == e.actor) ++r.own_ppuk; else ++r.opp_ppuk;
      e.ppuk &= (u16)~mb;
      e.owner1 &= (u16)~mb;
    } else if (e.neutral & mb) {
      e.neutral &= (u16)~mb;
      ++r.opp_ppuk;
    }
  }
  e.floor &= ~capture;
  capture_cards(e, capture | b, r);
  return kResOk;
}

CG_HD void finish_resolved_turn(Env& e) {  // turn50.h:409-416
  e.pplayed = kNoCard;
  e.pdrawn = kNoCard;
  e.pend_bonus = 0;
  e.phase = kPhasePlay;
  e.actor ^= 1u;
  ++e.turn;
}

// turn50.h:418-508.  On failure `e` may be partly changed: callers discard it.
CG_HD Resolve resolve_turn(Env& e, u8 played_choice, u8 drawn_choice) {
  Resolve r{kResWrongPhase, 0, 0, 0, 0, 0};
  if (e.phase != kPhaseResolve) return r;
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 played = n.pplayed, drawn = n.pdrawn;
  const u64 pm = floor_matches(n, played);
  const u32 pmc = popc(pm);
  const bool same = (played >> 2) == (drawn >> 2);
  const bool last = is_last_turn(n);
  r.last_turn = last;
  if (same && pmc == 1) {
    if (last) {
      u8 s = resolve_card_against_floor(n, played, played_choice, r);
      if (s != kResOk) return resolve_error(s);
      s = resolve_card_against_floor(n, drawn, drawn_choice, r);
      if (s != kResOk) return resolve_error(s);
      if (n.pend_bonus) capture_cards(n, n.pend_bonus, r);
    } else {
      n.floor |= bit(played) | bit(drawn) | n.pend_bonus;
      const u16 mb = month_bit(played);
      n.ppuk |= mb;
      if (n.actor == 0) n.owner1 &= (u16)~mb; else n.owner1 |= mb;
      if (n.pend_bonus & bit(kBonus2)) n.b2ppuk |= mb;   // turn50.h:241-250
      if (n.pend_bonus & bit(kBonus3)) n.b3ppuk |= mb;
      r.events |= kEvPpuk;
    }
  } else if (same && pmc == 2) {
    n.floor &= ~pm;
    capture_cards(n, pm | bit(played) | bit(drawn) | n.pend_bonus, r);
    r.events |= kEvTtadak;
  } else if (same && pmc == 0) {
    capture_cards(n, bit(played) | bit(drawn) | n.pend_bonus, r);
    if (!last) r.events |= kEvJjok;
  } else {
    u8 s = resolve_card_against_floor(n, played, played_choice, r);
    if (s != kResOk) return resolve_error(s);
    s = resolve_card_against_floor(n, drawn, drawn_choice, r);
    if (s != kResOk) return resolve_error(s);
    if (n.pend_bonus) capture_cards(n, n.pend_bonus, r);
  }
  if (n.floor == 0 && r.captured != 0) r.events |= kEvSweep;  // turn50.h:499-502
  finish_resolved_turn(n);
  r.status = kResOk;
  return r;
}

// turn50.h:285-304
CG_HD u8 begin_regular_play(Env& e, u8 card) {
  if (e.phase != kPhasePlay) return kTurnWrongPhase;
  if (!is_std(card)) return kTurnInvalidCard;
  const u64 b = bit(card);
  const u64 hand = active_hand(e);
  if ((hand & b) == 0) return kTurnNotInHand;
  set_hand(e, e.actor, hand & ~b);
  e.pplayed = card;
  e.pdrawn = kNoCard;
  e.pend_bonus = 0;
  e.phase = kPhaseDraw;
  return kTurnOk;
}

// turn50.h:306-324
CG_HD u8 draw_for_turn(Env& e) {
  if (e.phase != kPhaseDraw) return kTurnWrongPhase;
  u64 stock = e.stock, rng = e.rng;
  const Flip f = draw_with_bonus_chain(stock, rng);
  if (!is_std(f.card)) return kTurnStockEmpty;
  e.stock = stock;
  e.rng = rng;
  e.pdrawn = f.card;
  e.pend_bonus = f.bonuses;
  e.phase = kPhaseResolve;
  return kTurnOk;
}

// turn50.h:252-283 with bonus.h:37-66.  Returns the Turn50Status; steal gets the pi
// count the play requests, replacement the card drawn into the hand.
CG_HD u8 play_bonus_for_turn(Env& e, u8 bonus, u8& steal, u8& replacement) {
  steal = 0;
  replacement = kNoCard;
  if (e.phase != kPhasePlay) return kTurnWrongPhase;
  if (!is_bonus_card(bonus)) return kTurnInvalidCard;
  const u64 b = bit(bonus);
  const u64 hand = active_hand(e);
  if ((hand & b) == 0) return kTurnNotInHand;
  if (e.stock == 0) return kTurnStockEmpty;
  u64 stock = e.stock, rng = e.rng;
  const u8 card = draw_uniform(stock, rng);
  if (!is_physical(card)) return kTurnStockEmpty;
  set_hand(e, e.actor, (hand & ~b) | bit(card));
  set_cap(e, e.actor, cap_of(e, e.actor) | b);
  e.stock = stock;
  e.rng = rng;
  replacement = card;
  steal = is_last_turn(e) ? 0 : 1;
  return kTurnOk;
}

// ------------------------------------------------------------ gukjin_state.h ----
constexpr u16 kGukjinPiFlag0 = 1u << 12, kGukjinPiFlag1 = 1u << 13;
constexpr u16 kGukjinLock0 = 1u << 14, kGukjinLock1 = 1u << 15;
CG_HD u16 gukjin_flag(u32 p) { return (p & 1u) ? kGukjinPiFlag1 : kGukjinPiFlag0; }
CG_HD u16 gukjin_lock(u32 p) { return (p & 1u) ? kGukjinLock1 : kGukjinLock0; }
CG_HD bool gukjin_double_pi(const Env& e, u32 p) { return (e.owner1 & gukjin_flag(p)) != 0; }
CG_HD bool gukjin_option(const Env& e, u32 p) {  // gukjin_state.h:62-69
  return (cap_of(e, p) & bit(kGukjin)) != 0 && gukjin_double_pi(e, p);
}
CG_HD Score player_score(const Env& e, u32 p) {  // gukjin_state.h:71-75
  return score_captured(cap_of(e, p), gukjin_option(e, p));
}
CG_HD bool gukjin_locked(const Env& e, u32 p) { return (e.owner1 & gukjin_lock(p)) != 0; }
CG_HD bool gukjin_undecided(const Env& e, u32 p) {  // gukjin_state.h:109-114
  return (cap_of(e, p) & bit(kGukjin)) != 0 && !gukjin_double_pi(e, p) && !gukjin_locked(e, p);
}
CG_HD bool decide_gukjin(Env& e, u32 p, bool as_pi) {  // gukjin_state.h:117-124
  if (!gukjin_undecided(e, p)) return false;
  e.owner1 |= gukjin_lock(p);
  if (as_pi) e.owner1 |= gukjin_flag(p);
  return true;
}
CG_HD bool gukjin_prompt_due(const Env& e, u32 p, u8 go_count) {  // gukjin_state.h:129-137
  if (!gukjin_undecided(e, p)) return false;
  const u64 cap = cap_of(e, p);
  if (pi_units(cap, false) < 8u) return false;
  const u32 converted = score_captured(cap, true).total;
  return converted + go_count >= 7u;
}
CG_HD void auto_decide_loser_gukjin(Env& e, u32 loser) {  // gukjin_state.h:142-149
  const u8 pi = pi_units(cap_of(e, loser), gukjin_option(e, loser));
  if (pi == 6u || pi == 7u) decide_gukjin(e, loser, true);
  else if (pi == 0u) decide_gukjin(e, loser, false);
}

// ------------------------------------------------------------- pi_transfer.h ----
CG_HD u8 steal_count(const Resolve& r) {  // pi_transfer.h:51-62
  if (r.status != kResOk || r.last_turn != 0) return 0;
  u32 count = (u32)r.opp_ppuk + 2u * (u32)r.own_ppuk;
  if (r.events & kEvJjok) ++count;
  if (r.events & kEvTtadak) ++count;
  if (r.events & kEvSweep) ++count;
  count += popc(r.captured & kBonusMask);
  return (u8)count;
}

CG_HD u8 pi_card_value(u32 card) {  // pi_transfer.h:79-84
  if (card == kBonus3) return 3;
  if (card == kBonus2 || card == kGukjin || (kDoublePi & bit(card))) return 2;
  return 1;
}

// The n lowest set bits of pool.
CG_HD u64 lowest_bits(u64 pool, u32 n) {
  if (popc(pool) <= n) return pool;
  return pool & (bit(select_rank(pool, n)) - 1ull);
}

// pi_transfer.h:90-110.  Each of the six keys walks the candidates of one pi value,
// inside or outside the mission cards, in card order and takes them while the count
// lasts.  A card's pi value is fixed by its id (pi_card_value), so a key's pass is the
// lowest `count` bits of one mask: six branch-free passes instead of a loop over cards.
CG_HD u64 hangame_steal_selection(u64 candidates, u64 mission, bool owns_mission, u32 count) {
  const u64 k3 = bit(kBonus3);
  const u64 k2 = (bit(kBonus2) | bit(kGukjin) | kDoublePi) & ~k3;
  const u64 v3 = candidates & k3, v2 = candidates & k2, v1 = candidates & ~(k2 | k3);
  u64 chosen = 0;
#pragma unroll
  for (u32 key = 0; key < 6; ++key) {
    const bool use_mission = owns_mission ? key >= 3 : (key & 1u) != 0;
    const u32 value = owns_mission ? 1 + key % 3 : 1 + key / 2;
    const u64 vm = value == 1 ? v1 : value == 2 ? v2 : v3;
    const u64 take = lowest_bits(vm & (use_mission ? mission : ~mission), count);
    chosen |= take;
    count -= popc(take);
  }
  return chosen;
}

struct PiResult { u8 status, requested, available; u64 transfer; };

// pi_transfer.h:125-210 with the victim's own persistent score options (212-222).
CG_HD PiResult apply_pi_steal(Env& e, u32 thief, u8 requested, u64 selection) {
  thief &= 1u;
  const u32 victim = thief ^ 1u;
  const bool victim_pi = gukjin_option(e, victim);
  const u64 victim_cards = cap_of(e, victim);
  const u64 candidates = pi_card_mask(victim_cards, victim_pi);
  const u8 available = (u8)popc(candidates);
  if (requested == 0) return PiResult{kPiOk, 0, available, 0};
  if (available == 0) {
    decide_gukjin(e, victim, false);
    return PiResult{kPiOk, requested, available, 0};
  }
  if (available > requested && selection == 0) {
    const bool owns = e.mission != 0 && (e.mission & ~victim_cards) == 0;
    selection = hangame_steal_selection(candidates, e.mission, owns, requested);
  }
  const u8 required = requested < available ? requested : available;
  u64 transfer;
  if (available <= requested) {
    if (selection != 0 && selection != candidates)
      return PiResult{kPiInvalidSelection, requested, available, 0};
    transfer = candidates;
  } else {
    if (selection == 0) return PiResult{kPiSelRequired, requested, available, 0};
    if ((selection & ~candidates) != 0 || popc(selection) != required)
      return PiResult{kPiInvalidSelection, requested, available, 0};
    transfer = selection;
  }
  set_cap(e, victim, victim_cards & ~transfer);
  set_cap(e, thief, cap_of(e, thief) | transfer);
  if (transfer & bit(kGukjin))  // pi_transfer.h:66-77
    e.owner1 &= (u16)~(gukjin_flag(thief) | gukjin_flag(victim));
  if (available < requested) decide_gukjin(e, victim, false);
  return PiResult{kPiOk, requested, available, transfer};
}

// pi_transfer.h:234-255: resolve, then steal (on failure the caller discards `e`).
CG_HD Resolve resolve_turn_with_pi(Env& e, u8 pchoice, u8 dchoice, u64 sel, PiResult& pt) {
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 thief = e.actor;
  const Resolve r = resolve_turn(n, pchoice, dchoice);
  pt = PiResult{kPiOk, 0, 0, 0};
  if (r.status != kResOk) return r;
  pt = apply_pi_steal(n, thief, steal_count(r), sel);
  if (pt.status != kPiOk) return r;
  return r;
}

// pi_transfer.h:274-294
CG_HD u8 play_bonus_with_pi(Env& e, u8 bonus, u64 sel, PiResult& pt, u8& replacement) {
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 thief = e.actor;
  u8 steal;
  const u8 s = play_bonus_for_turn(n, bonus, steal, replacement);
  pt = PiResult{kPiOk, 0, 0, 0};
  if (s != kTurnOk) return s;
  pt = apply_pi_steal(n, thief, steal, sel);
  if (pt.status != kPiOk) return s;
  return s;
}

// ------------------------------------------------------------------ game50.h ----
CG_HD bool has_decision(const Env& e) { return e.dact <= 1u; }
CG_HD bool has_gukjin_decision(const Env& e) { return e.gdec != 0; }
CG_HD bool has_pending_choice(const Env& e) { return has_decision(e) || has_gukjin_decision(e); }
CG_HD bool game_finished(const Env& e) { return e.winner <= 1u; }
CG_HD u8 base_score(const Env& e, u32 p) { return player_score(e, p).total; }

CG_HD u64 go_multiplier(u8 go_count) {  // game50.h:126-134
  if (go_count < 3) return 1;
  const u32 doublings = (u32)go_count - 2u;
  return doublings >= 64 ? 0 : 1ull << doublings;
}
CG_HD u64 points_after_go(u8 base, u8 go_count) {  // game50.h:136-147
  return ((u64)base + (u64)go_count) * go_multiplier(go_count);
}

// game50.h:159-183
CG_HD bool maybe_open_go_stop(Env& e, u32 completed) {
  if (completed > 1u || game_finished(e) || has_pending_choice(e)) return false;
  const u8 base = base_score(e, completed);
  const u8 go = go_of(e, completed);
  const bool eligible = go == 0 ? base >= kDecisionBasePoints : base > lgo_of(e, completed);
  if (!eligible) return false;
  auto_decide_loser_gukjin(e, completed ^ 1u);
  if (e.turn > kLastTurnIndex) {
    e.winner = (u8)completed;
    return false;
  }
  e.dact = (u8)completed;
  return true;
}

// game50.h:187-199
CG_HD bool finish_turn_game(Env& e, u32 completed) {
  if (completed > 1u || game_finished(e) || has_pending_choice(e)) return false;
  if (gukjin_prompt_due(e, completed, go_of(e, completed))) {
    e.gdec = (u8)(completed + 1u);
    return true;
  }
  return maybe_open_go_stop(e, completed);
}

// game50.h:201-211 (GoStopStatus50: 0 ok, 1 no decision, 2 finished)
CG_HD u8 apply_gukjin_decision(Env& e, bool as_pi) {
  if (game_finished(e)) return 2;
  if (!has_gukjin_decision(e)) return 1;
  const u32 actor = (u32)e.gdec - 1u;
  decide_gukjin(e, actor, as_pi);
  e.gdec = 0;
  maybe_open_go_stop(e, actor);
  return 0;
}

// game50.h:213-242
CG_HD u8 apply_go_stop(Env& e, bool stop) {
  if (game_finished(e)) return 2;
  if (!has_decision(e)) return 1;
  const u32 actor = e.dact;
  if (stop) {
    auto_decide_loser_gukjin(e, actor ^ 1u);
    e.winner = (u8)actor;
    e.dact = kNoPlayer;
    return 0;
  }
  const u8 base = base_score(e, actor);
  if (actor == 0) { ++e.go0; e.lgo0 = base; } else { ++e.go1; e.lgo1 = base; }
  e.dact = kNoPlayer;
  return 0;
}

CG_HD u8 begin_regular_play_game(Env& e, u8 card) {  // game50.h:244-250
  if (game_finished(e) || has_pending_choice(e)) return kTurnWrongPhase;
  return begin_regular_play(e, card);
}
CG_HD u8 draw_for_game(Env& e) {  // game50.h:252-257
  if (game_finished(e) || has_pending_choice(e)) return kTurnWrongPhase;
  return draw_for_turn(e);
}

// game50.h:271-305
CG_HD Resolve resolve_game_turn(Env& e, u8 pchoice, u8 dchoice, u64 sel, PiResult& pt) {
  pt = PiResult{kPiOk, 0, 0, 0};
  if (game_finished(e) || has_pending_choice(e)) return resolve_error(kResWrongPhase);
  const u8 completed = e.actor;
  Env& n = e;  // in place: the caller's copy is the transaction
  const Resolve r = resolve_turn_with_pi(n, pchoice, dchoice, sel, pt);
  if (r.status != kResOk || pt.status != kPiOk) return r;
  finish_turn_game(n, completed);
  return r;
}

// ---------------------------------------------------------------- special50.h ----
CG_HD bool special_ready(const Env& e) {  // special50.h:66-69
  return !game_finished(e) && !has_pending_choice(e) && e.phase == kPhasePlay;
}

// special50.h:71-88
CG_HD u16 legal_special_months(const Env& e, u32 hand_count, u32 floor_count, bool exclude) {
  if (!special_ready(e)) return 0;
  const u64 h = active_hand(e) & kStdMask;
  const u64 f = std_floor(e);
  const u16 old = !exclude ? 0 : hand_count == 4 ? sh4_of(e, e.actor) : shaken_of(e, e.actor);
  return (u16)(months_with_count(month_counts(h), hand_count) &
               months_with_count(month_counts(f), floor_count) & ~old & 0x0FFFu);
}
// months whose count nibble equals k, as the low bit of each month nibble
CG_HD u64 count_is(u64 counts, u32 k) {
  const u64 d = counts ^ (kNibbleLow * k);
  return ~(d | (d >> 1) | (d >> 2)) & kNibbleLow;
}

// The three special-play month sets of special50.h:71-95 from one count of the hand and
// the floor: bombs (3 in hand, 1 on the floor), grenades (2 and 2) and shakes (3 or 4 in
// hand, none on the floor, not shaken before with that count), each
// legal_special_months(e, ...) of the matching arguments.
struct SpecialMonths { u16 bombs, grenades, shakes; };
CG_HD SpecialMonths special_months(const Env& e) {
  if (!special_ready(e)) return SpecialMonths{0, 0, 0};
  const u64 hc = month_counts(active_hand(e));
  const u64 fc = month_counts(std_floor(e));
  const u64 h3 = count_is(hc, 3), f0 = count_is(fc, 0);
  SpecialMonths s;
  s.bombs = (u16)(gather_months(h3 & count_is(fc, 1)) & 0x0FFFu);
  s.grenades = (u16)(gather_months(count_is(hc, 2) & count_is(fc, 2)) & 0x0FFFu);
  s.shakes = (u16)(((gather_months(h3 & f0) & ~shaken_of(e, e.actor)) |
                    (gather_months(count_is(hc, 4) & f0) & ~sh4_of(e, e.actor))) & 0x0FFFu);
  return s;
}
CG_HD u16 legal_shake_months(const Env& e) { return special_months(e).shakes; }  // 92-95
CG_HD u16 legal_bomb_months(const Env& e) { return special_months(e).bombs; }
CG_HD u16 legal_grenade_months(const Env& e) { return special_months(e).grenades; }
CG_HD u16 forced_special_months(const Env& e) {
  const SpecialMonths s = special_months(e);
  return (u16)(s.bombs | s.grenades);
}
CG_HD u8 shake_count(const Env& e, u32 p) {  // special50.h:107-110
  return (u8)(popc(shaken_of(e, p)) + popc(sh4_of(e, p)));
}
CG_HD u64 bomb_shake_multiplier(const Env& e, u32 p) {  // special50.h:111-115
  const u8 n = (u8)(bombs_of(e, p) + shake_count(e, p));
  return n >= 64 ? 0 : 1ull << n;
}
CG_HD u64 go_bomb_shake_score(const Env& e, u32 p) {  // special50.h:116-119
  return points_after_go(base_score(e, p), go_of(e, p)) * bomb_shake_multiplier(e, p);
}

// special50.h:131-159
struct DrawOnly { u8 status; u8 drawn; u64 bonuses; Resolve resolve; };
CG_HD DrawOnly draw_only_special(Env& e, u8 choice) {
  u64 stock = e.stock, rng = e.rng;
  const Flip f = draw_with_bonus_chain(stock, rng);
  if (!is_std(f.card)) return DrawOnly{kSpStockEmpty, kNoCard, 0, resolve_error(kResWrongPhase)};
  e.stock = stock;
  e.rng = rng;
  Resolve r{kResOk, 0, 0, 0, 0, (u8)is_last_turn(e)};
  const u8 rs = resolve_card_against_floor(e, f.card, choice, r);
  if (rs != kResOk) {
    const u8 st = rs == kResChoiceRequired ? kSpResolveChoiceRequired : kSpInvalidResolveChoice;
    return DrawOnly{st, f.card, f.bonuses, resolve_error(rs)};
  }
  if (f.bonuses) capture_cards(e, f.bonuses, r);
  if (e.floor == 0 && r.captured) r.events |= kEvSweep;
  r.status = kResOk;
  return DrawOnly{kSpOk, f.card, f.bonuses, r};
}
CG_HD void finish_draw_only(Env& e) {  // special50.h:160-163
  e.pplayed = kNoCard;
  e.pdrawn = kNoCard;
  e.pend_bonus = 0;
  e.phase = kPhasePlay;
  e.actor ^= 1u;
  ++e.turn;
}

// special50.h:165-183
CG_HD u8 begin_shake(Env& e, u8 card) {
  if (!special_ready(e)) return kSpWrongPhase;
  if (!is_std(card)) return kSpInvalidCard;
  const u16 mb = month_bit(card);
  const u64 hand = active_hand(e);
  if ((legal_shake_months(e) & mb) == 0 || (hand & bit(card)) == 0) return kSpNotLegal;
  Env& n = e;  // in place: the caller's copy is the transaction
  const bool four = popc(hand & month_cards(card >> 2)) == 4;
  if (four) { if (n.actor == 0) n.sh4_0 |= mb; else n.sh4_1 |= mb; }
  else { if (n.actor == 0) n.shaken0 |= mb; else n.shaken1 |= mb; }
  if (begin_regular_play_game(n, card) != kTurnOk) return kSpNotLegal;
  return kSpOk;
}

CG_HD u8 pi_to_special(u8 s) {  // special50.h:125-129
  return s == kPiSelRequired ? kSpPiSelectionRequired
       : s == kPiInvalidSelection ? kSpInvalidPiSelection : kSpOk;
}

// special50.h:185-220; pt receives the pi transfer for the terminal layer.
CG_HD u8 capture_special(Env& e, u8 month, bool grenade, u8 choice, u64 sel, PiResult& pt) {
  pt = PiResult{kPiOk, 0, 0, 0};
  if (!special_ready(e)) return kSpWrongPhase;
  if (month >= 12) return kSpInvalidMonth;
  const u16 mb = (u16)(1u << month);
  const u16 legal = grenade ? legal_grenade_months(e) : legal_bomb_months(e);
  if ((legal & mb) == 0) return kSpNotLegal;
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 actor = n.actor;
  const u64 hand = hand_of(n, actor);
  const u64 hc = hand & month_cards(month);
  const u64 fc = std_floor(n) & month_cards(month);
  set_hand(n, actor, hand & ~hc);
  n.floor &= ~fc;
  set_cap(n, actor, cap_of(n, actor) | hc | fc);
  set_cred(n, actor, (u8)(cred_of(n, actor) + (grenade ? 1u : 2u)));
  if (!grenade) { if (actor == 0) ++n.bombs0; else ++n.bombs1; }
  const DrawOnly d = draw_only_special(n, choice);
  if (d.status != kSpOk) return d.status;
  const u8 steal = (u8)((is_last_turn(n) ? 0u : 1u) + steal_count(d.resolve));
  finish_draw_only(n);
  pt = apply_pi_steal(n, actor, steal, sel);
  if (pt.status != kPiOk) return pi_to_special(pt.status);
  finish_turn_game(n, actor);
  return kSpOk;
}

// special50.h:232-254
CG_HD u8 play_bomb_credit(Env& e, u8 choice, u64 sel, PiResult& pt) {
  pt = PiResult{kPiOk, 0, 0, 0};
  if (!special_ready(e)) return kSpWrongPhase;
  const u8 actor = e.actor;
  if (!cred_of(e, actor)) return kSpNotLegal;
  Env& n = e;  // in place: the caller's copy is the transaction
  set_cred(n, actor, (u8)(cred_of(n, actor) - 1u));
  const DrawOnly d = draw_only_special(n, choice);
  if (d.status != kSpOk) return d.status;
  const u8 steal = steal_count(d.resolve);
  finish_draw_only(n);
  pt = apply_pi_steal(n, actor, steal, sel);
  if (pt.status != kPiOk) return pi_to_special(pt.status);
  finish_turn_game(n, actor);
  return kSpOk;
}

// -------------------------------------------------------------- terminal50.h ----
// Mission card sets (terminal50.h:119-159); Hangame numbers n are card id n - 1.
CG_HD u64 hg(u32 a, u32 b, u32 c) { return bit(a - 1) | bit(b - 1) | bit(c - 1); }
CG_HD u64 mission_cards_for(u8 type, u8 index) {
  if (type == kMissionEasy) {
    if (index == 10) return bit(8) | bit(28);
    return bit(4u * index) | bit(4u * index + 1);
  }
  if (type == kMissionNormal) return month_cards(index);
  if (type == kMissionHard || type == kMissionTriple) {
    const bool triple = type == kMissionTriple;
    if (triple && index >= 4) ++index;
    switch (index) {
      case 0: return hg(22, 34, 38);
      case 1: return hg(2, 6, 10);
      case 2: return hg(14, 18, 26);
      case 3: return hg(5, 13, 30);
      case 4: return hg(33, 42, 48);
      case 5: return triple ? hg(5, 25, 46) : hg(21, 25, 37);
      case 6: return triple ? hg(21, 25, 37) : hg(1, 9, 29);
      case 7: return triple ? hg(1, 9, 29) : hg(1, 9, 41);
      case 8: return triple ? hg(1, 9, 41) : hg(1, 29, 41);
      case 9: return triple ? hg(1, 29, 41) : hg(9, 29, 41);
      case 10: return triple ? hg(9, 29, 41) : hg(5, 13, 46);
      case 11: return triple ? hg(5, 13, 46) : hg(5, 30, 46);
      case 12: return triple ? hg(5, 30, 46) : hg(13, 30, 46);
      case 13: return triple ? hg(13, 30, 46) : hg(5, 25, 46);
      default: return 0;
    }
  }
  return 0;
}

// terminal50.h:164-183
CG_HD void assign_mission(Env& e, u64 seed) {
  u64 s = seed ^ 0x6d697373696f6e35ull;
  const u32 kind = uniform_bounded(s, 5u);
  const u8 multiplier = (u8)(2u + uniform_bounded(s, 3u));
  u8 type = kMissionEasy;
  u32 options = 11u;
  if (kind == 1u) { type = kMissionNormal; options = 12u; }
  else if (kind == 2u) { type = kMissionHard; options = 14u; }
  else if (kind == 3u) { type = kMissionNoCondition; options = 0u; }
  else if (kind == 4u) { type = kMissionTriple; options = 13u; }
  const u8 index = options == 0u ? 0 : (u8)uniform_bounded(s, options);
  e.mtype = type;
  e.mmult = type == kMissionTriple ? 0 : multiplier;
  e.mission = mission_cards_for(type, index);
  if (type == kMissionNoCondition) { e.mm0 = multiplier; e.mm1 = multiplier; }
}

// terminal50.h:186-197
CG_HD void update_missions(Env& e, u32 actor, u64 acquired) {
  const u64 mine = cap_of(e, actor);
  if (e.mtype == kMissionTriple) {
    set_mm(e, actor, (u8)(1u << popc(e.mission & mine)));
    return;
  }
  if (e.mission == 0 || (acquired & e.mission) == 0) return;
  if ((e.mission & ~mine) == 0) set_mm(e, actor, e.mmult);
}

CG_HD u16 chongtong_months(u64 cards) {  // terminal50.h:215-224: all four cards held
  cards &= kStdMask;
  return gather_months(cards & (cards >> 1) & (cards >> 2) & (cards >> 3) & kNibbleLow);
}

CG_HD bool terminal_finished(const Env& e) { return e.treason != kReasonNone; }
CG_HD bool has_ct_choice(const Env& e) { return e.ct_actor <= 1u; }

CG_HD void mark_terminal(Env& e, u32 winner, u8 reason, u64 points) {  // terminal50.h:264-275
  e.twinner = (u8)(winner & 1u);
  e.treason = reason;
  e.tpoints = points;
  e.ct_actor = kNoPlayer;
  e.ct_months = 0;
  e.dact = kNoPlayer;
  e.gdec = 0;
}

CG_HD u8 round_multiplier(const Env& e) { return e.round == 0 ? 1 : e.round; }

CG_HD void add_side_payment(Env& e, u32 receiver, i32 base) {  // terminal50.h:113-117
  const i32 amount = base * (i32)round_multiplier(e);
  e.side0 += (receiver & 1u) == 0 ? amount : -amount;
}

CG_HD void sync_game_stop(Env& e) {  // terminal50.h:317-324
  if (e.treason != kReasonNone || !game_finished(e)) return;
  const u8 w = e.winner;
  e.twinner = w;
  e.treason = kReasonStop;
  e.tpoints = go_bomb_shake_score(e, w);
}

// terminal50.h:339-362
CG_HD bool record_completed_turn_ppuk(Env& e, u32 actor, bool made_ppuk) {
  if (terminal_finished(e) || !made_ppuk) return false;
  actor &= 1u;
  u8 count = pcount_of(e, actor);
  u8 ppuk = streak_of(e, actor);
  const u16 turn = e.turn;
  if (count != 0xFF) ++count;
  switch (ppuk) {
    case kPpukNone: ppuk = turn <= 1u ? kPpukFirst : kPpukOne; break;
    case kPpukFirst: ppuk = turn <= 3u ? kPpukSecond : kPpukTwo; break;
    case kPpukSecond: ppuk = turn <= 5u ? kPpukThird : kPpukThree; break;
    case kPpukOne: ppuk = kPpukTwo; break;
    case kPpukTwo: ppuk = kPpukThree; break;
    default: break;
  }
  if (actor == 0) { e.pcount0 = count; e.streak0 = ppuk; }
  else { e.pcount1 = count; e.streak1 = ppuk; }
  if (ppuk == kPpukFirst || ppuk == kPpukSecond || ppuk == kPpukThird)
    add_side_payment(e, actor, 7 * (i32)ppuk);
  if (ppuk != kPpukThird && ppuk != kPpukThree) return false;
  mark_terminal(e, actor, kReasonThreePpuk, 7);
  return true;
}

// terminal50.h:364-376
CG_HD bool open_bonus_chongtong_choice(Env& e, u32 actor, u16 newly) {
  if (terminal_finished(e) || has_ct_choice(e) || actor > 1u || newly == 0) return false;
  e.ct_actor = (u8)actor;
  e.ct_months = (u16)(newly & kMonthBits);
  return e.ct_months != 0;
}

// terminal50.h:378-398 (TerminalStatus50: 0 ok, else error)
CG_HD u8 apply_chongtong_action(Env& e, bool win) {
  if (terminal_finished(e)) return 1;
  if (!has_ct_choice(e)) return 3;
  const u8 actor = e.ct_actor;
  if (win) {
    mark_terminal(e, actor, kReasonBonusChongtong, 10);
    return 0;
  }
  e.ct_actor = kNoPlayer;
  e.ct_months = 0;
  return 0;
}

CG_HD u8 begin_regular_play_terminal(Env& e, u8 card) {  // terminal50.h:400-406
  if (terminal_finished(e) || has_ct_choice(e)) return kTurnWrongPhase;
  return begin_regular_play_game(e, card);
}
CG_HD u8 draw_for_terminal(Env& e) {  // terminal50.h:408-413
  if (terminal_finished(e) || has_ct_choice(e)) return kTurnWrongPhase;
  return draw_for_game(e);
}

// terminal50.h:415-454; returns the Turn50Status, pt the pi result.
CG_HD u8 play_bonus_terminal(Env& e, u8 bonus, u64 sel, PiResult& pt) {
  pt = PiResult{kPiOk, 0, 0, 0};
  if (terminal_finished(e) || has_ct_choice(e)) return kTurnWrongPhase;
  if (game_finished(e) || has_pending_choice(e)) return kTurnWrongPhase;  // game50.h:263-267
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 actor = n.actor;
  const u16 before = chongtong_months(active_hand(n));
  u8 replacement;
  const u8 s = play_bonus_with_pi(n, bonus, sel, pt, replacement);
  if (s != kTurnOk || pt.status != kPiOk) return s;
  if (pt.transfer != 0) update_missions(n, actor, pt.transfer);
  const u16 after = chongtong_months(active_hand(n));
  open_bonus_chongtong_choice(n, actor, (u16)(after & ~before));
  return s;
}

// terminal50.h:456-503
CG_HD Resolve resolve_terminal_turn(Env& e, u8 pchoice, u8 dchoice, u64 sel, PiResult& pt) {
  pt = PiResult{kPiOk, 0, 0, 0};
  if (terminal_finished(e) || has_ct_choice(e)) return resolve_error(kResWrongPhase);
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 actor = n.actor;
  const u64 before = cap_of(n, actor);
  const Resolve r = resolve_game_turn(n, pchoice, dchoice, sel, pt);
  if (r.status != kResOk || pt.status != kPiOk) return r;
  if ((r.events & kEvTtadak) && n.turn == 1u) add_side_payment(n, actor, 7);
  update_missions(n, actor, cap_of(n, actor) & ~before);
  record_completed_turn_ppuk(n, actor, (r.events & kEvPpuk) != 0);
  sync_game_stop(n);
  return r;
}

// terminal50.h:505-530 for bomb/grenade/bomb-credit (shake handled by its caller).
CG_HD u8 apply_terminal_special(Env& e, u8 kind, u8 month, u8 choice, u64 sel) {
  if (terminal_finished(e) || has_ct_choice(e)) return kSpWrongPhase;
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 actor = n.actor;
  const u64 before = cap_of(n, actor);
  PiResult pt;
  u8 s;
  if (kind == kBombCredit) s = play_bomb_credit(n, choice, sel, pt);
  else s = capture_special(n, month, kind == kGrenade, choice, sel, pt);
  if (s != kSpOk) return s;
  update_missions(n, actor, cap_of(n, actor) & ~before);
  sync_game_stop(n);
  return kSpOk;
}

CG_HD u8 apply_terminal_shake(Env& e, u8 card) {  // terminal50.h:505-530, kShake
  if (terminal_finished(e) || has_ct_choice(e)) return kSpWrongPhase;
  return begin_shake(e, card);
}

CG_HD u8 apply_terminal_gukjin(Env& e, bool as_pi) {  // terminal50.h:532-544
  if (terminal_finished(e) || has_ct_choice(e)) return 2;
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 s = apply_gukjin_decision(n, as_pi);
  if (s != 0) return s;
  sync_game_stop(n);
  return 0;
}

CG_HD u8 apply_terminal_go_stop(Env& e, bool stop) {  // terminal50.h:546-559
  if (terminal_finished(e) || has_ct_choice(e)) return 2;
  Env& n = e;  // in place: the caller's copy is the transaction
  const u8 s = apply_go_stop(n, stop);
  if (s != 0) return s;
  sync_game_stop(n);
  return 0;
}

// ------------------------------------------------------------ settlement50.h ----
struct Settlement { bool ok; u8 winner; u64 final_points; i64 side; };

// settlement50.h:95-208 (only what the reward and the stop points read).
CG_HD Settlement settle(const Env& e) {
  if (!terminal_finished(e) || e.twinner > 1u) return Settlement{false, kNoPlayer, 0, 0};
  const u32 w = e.twinner, l = w ^ 1u;
  const u64 round = round_multiplier(e);
  const i64 side = e.side0;
  const u8 reason = e.treason;
  if (reason == kReasonInitialChongtong || reason == kReasonFloorChongtong ||
      reason == kReasonBonusChongtong || reason == kReasonThreePpuk)
    return Settlement{true, (u8)w, e.tpoints * round, side};
  const Score ws = player_score(e, w);
  const Score ls = player_score(e, l);
  const u64 after_go = points_after_go(ws.total, go_of(e, w));
  u64 bak = 1;
  if (ws.flags & kFlagMeongtta) bak *= 2u;
  if (ws.pi_units >= 10u && ls.pi_units >= 1u && ls.pi_units <= 7u) bak *= 2u;
  if (ws.bright_count >= 3u && ls.bright_count == 0u) bak *= 2u;
  if (go_of(e, l) != 0u) bak *= 2u;
  u64 mission = mm_of(e, w);
  if (mission == 0u) mission = 1u;
  const bool void_game = cap_of(e, l) == 0;
  const u64 after_special = after_go * bomb_shake_multiplier(e, w);
  const u64 final_points = void_game ? 0u : after_special * bak * mission * round;
  return Settlement{true, (u8)w, final_points, side};
}

CG_HD i64 settlement_reward0(const Settlement& s) {  // settlement50.h:211-218
  if (!s.ok) return 0;
  const i64 points = (i64)s.final_points;
  return (s.winner == 0 ? points : -points) + s.side;
}

// --------------------------------------------------------------- rollout50.h ----
struct Action { u8 kind, card, month, pmatch, dmatch; u64 pisel; };
CG_HD Action make_action(u8 kind) { return Action{kind, kNoCard, 0xFF, kNoCard, kNoCard, 0}; }
CG_HD Action invalid_action() { return make_action(kPlayCard); }  // rollout50.h:54-59

CG_HD u8 map_turn(u8 s) {  // rollout50.h:181-186
  if (s == kTurnOk) return kOk;
  if (s == kTurnStockEmpty) return kStockEmpty;
  if (s == kTurnWrongPhase) return kWrongPhase;
  return kNotLegal;
}
CG_HD u8 map_resolve(u8 s) {  // rollout50.h:188-198
  if (s == kResOk) return kOk;
  if (s == kResChoiceRequired) return kResolveChoiceRequired;
  if (s == kResInvalidChoice) return kInvalidResolveChoice;
  if (s == kResWrongPhase) return kWrongPhase;
  return kNotLegal;
}
CG_HD u8 map_pi(u8 s) {  // rollout50.h:200-205
  if (s == kPiOk) return kOk;
  if (s == kPiSelRequired) return kPiSelectionRequired;
  return kInvalidPiSelection;
}
CG_HD u8 map_special(u8 s) {  // rollout50.h:207-223
  switch (s) {
    case kSpOk: return kOk;
    case kSpWrongPhase: return kWrongPhase;
    case kSpStockEmpty: return kStockEmpty;
    case kSpResolveChoiceRequired: return kResolveChoiceRequired;
    case kSpInvalidResolveChoice: return kInvalidResolveChoice;
    case kSpPiSelectionRequired: return kPiSelectionRequired;
    case kSpInvalidPiSelection: return kInvalidPiSelection;
    default: return kNotLegal;
  }
}

// rollout50.h:268-376: the six turn-taking kinds (play card, shake, bonus, bomb, grenade,
// bomb credit) composed from the per-kind transitions, as the reference composes them.
// The product runs apply_turn_action (same statuses, same state); this composition is its
// plain restatement, kept for the host check of the two.
CG_HD u8 apply_turn_action_per_kind(Env& n, const Action& a) {
  const u8 actor = n.actor;
  u8 status = kOk;
  if (a.kind == kPlayBonus) {
    PiResult pt;
    status = map_turn(play_bonus_terminal(n, a.card, a.pisel, pt));
    if (status == kOk) status = map_pi(pt.status);
  } else if (a.kind == kBomb || a.kind == kGrenade || a.kind == kBombCredit) {
    status = map_special(apply_terminal_special(n, a.kind, a.month, a.dmatch, a.pisel));
  } else if (a.kind == kShake || a.kind == kPlayCard) {
    if (a.kind == kShake) {
      if (is_std(a.card)) {  // a shake shows the month's cards in hand
        const u64 shown = active_hand(n) & month_cards(a.card >> 2);
        if (actor == 0) n.rev0 |= shown; else n.rev1 |= shown;
      }
      status = map_special(apply_terminal_shake(n, a.card));
    } else {
      if (is_std(a.card) && (forced_special_months(n) & month_bit(a.card)) != 0)
        return kNotLegal;
      status = map_turn(begin_regular_play_terminal(n, a.card));
    }
    if (status != kOk) return status;
    status = map_turn(draw_for_terminal(n));
    if (status != kOk) return status;
    PiResult pt;
    const Resolve r = resolve_terminal_turn(n, a.pmatch, a.dmatch, a.pisel, pt);
    status = map_resolve(r.status);
    if (status == kOk) status = map_pi(pt.status);
  } else {
    return kInvalidAction;
  }
  return status;
}

CG_HD bool is_turn_kind(u8 k) {
  return k == kPlayBonus || k == kBomb || k == kGrenade || k == kBombCredit || k == kShake ||
         k == kPlayCard;
}

// The same six kinds as one transition.  In the composition above every kind's body
// carries its own stock draw, floor resolution, pi steal and mission/stop bookkeeping, and
// a wave whose games take different kinds runs each body in turn.  Here each kind runs
// only its prologue (its checks and the cards it moves before the draw); the draw, the
// floor resolution, the steal and the bookkeeping then run once for every kind:
//   * the draw: a bonus play takes one card, any card (bonus.h:37-66); the others flip
//     until a standard card, collecting the bonus cards met (bonus.h:68-81);
//   * the resolution: a played card's turn resolves as resolve_turn (turn50.h:418-508);
//     a bomb, grenade or bomb credit resolves the drawn card alone, as resolve_turn's
//     last two steps do (special50.h:131-163);
//   * the steal: the turn's pi count (pi_transfer.h:51-62), plus one for a bomb or
//     grenade before the last turn (special50.h:207), or one for a bonus play;
//   * the bookkeeping: terminal50.h:456-503 for a played card, 505-530 for a special,
//     415-454 for a bonus play.
// The checks run in the composition's order and return its statuses; the state updates
// are the composition's, in its order.  `n` is the caller's transaction copy: a failure
// may leave it partly changed.
CG_HD u8 apply_turn_action(Env& n, const Action& a) {
  const u8 actor = n.actor;
  const bool bonus = a.kind == kPlayBonus;
  const bool special = a.kind == kBomb || a.kind == kGrenade || a.kind == kBombCredit;
  const bool play = !bonus && !special;  // kShake or kPlayCard
  if (!is_turn_kind(a.kind)) return kInvalidAction;
  const u64 cap_before = cap_of(n, actor);
  u16 ct_before = 0;
  u8 base_steal = 0;
  if (bonus) {  // play_bonus_terminal and play_bonus_for_turn up to the draw
    if (terminal_finished(n) || has_ct_choice(n)) return kWrongPhase;
    if (game_finished(n) || has_pending_choice(n)) return kWrongPhase;
    ct_before = chongtong_months(active_hand(n));
    if (n.phase != kPhasePlay) return kWrongPhase;
    if (!is_bonus_card(a.card)) return kNotLegal;
    if ((active_hand(n) & bit(a.card)) == 0) return kNotLegal;
    if (n.stock == 0) return kStockEmpty;
  } else if (special) {  // apply_terminal_special, capture_special / play_bomb_credit
    if (terminal_finished(n) || has_ct_choice(n)) return kWrongPhase;
    if (!special_ready(n)) return kWrongPhase;
    if (a.kind == kBombCredit) {
      if (!cred_of(n, actor)) return kNotLegal;
      set_cred(n, actor, (u8)(cred_of(n, actor) - 1u));
    } else {
      const bool grenade = a.kind == kGrenade;
      const u8 month = a.month;
      if (month >= 12) return kNotLegal;
      const u16 mb = (u16)(1u << month);
      const u16 legal = grenade ? legal_grenade_months(n) : legal_bomb_months(n);
      if ((legal & mb) == 0) return kNotLegal;
      const u64 hand = hand_of(n, actor);
      const u64 hc = hand & month_cards(month);
      const u64 fc = std_floor(n) & month_cards(month);
      set_hand(n, actor, hand & ~hc);
      n.floor &= ~fc;
      set_cap(n, actor, cap_of(n, actor) | hc | fc);
      set_cred(n, actor, (u8)(cred_of(n, actor) + (grenade ? 1u : 2u)));
      if (!grenade) { if (actor == 0) ++n.bombs0; else ++n.bombs1; }
      base_steal = is_last_turn(n) ? 0 : 1;
    }
  } else {
    if (a.kind == kShake) {
      if (is_std(a.card)) {  // a shake shows the month's cards in hand
        const u64 shown = active_hand(n) & month_cards(a.card >> 2);
        if (actor == 0) n.rev0 |= shown; else n.rev1 |= shown;
      }
      if (terminal_finished(n) || has_ct_choice(n)) return kWrongPhase;
      const u8 s = map_special(begin_shake(n, a.card));
      if (s != kOk) return s;
    } else {
      if (is_std(a.card) && (forced_special_months(n) & month_bit(a.card)) != 0)
        return kNotLegal;
      const u8 s = map_turn(begin_regular_play_terminal(n, a.card));
      if (s != kOk) return s;
    }
    // draw_for_terminal -> draw_for_game -> draw_for_turn, up to the draw
    if (terminal_finished(n) || has_ct_choice(n)) return kWrongPhase;
    if (game_finished(n) || has_pending_choice(n)) return kWrongPhase;
    if (n.phase != kPhaseDraw) return kWrongPhase;
  }
  // The draw.
  u64 stock = n.stock, rng = n.rng, flipped = 0;
  u8 card = kNoCard;
  while (stock != 0) {
    card = draw_uniform(stock, rng);
    if (bonus || !is_bonus_card(card)) break;
    flipped |= bit(card);
    card = kNoCard;
  }
  if (bonus ? !is_physical(card) : !is_std(card)) return kStockEmpty;
  n.stock = stock;
  n.rng = rng;
  u8 steal;
  Resolve r{kResOk, 0, 0, 0, 0, (u8)is_last_turn(n)};
  if (bonus) {
    set_hand(n, actor, (active_hand(n) & ~bit(a.card)) | bit(card));
    set_cap(n, actor, cap_of(n, actor) | bit(a.card));
    steal = r.last_turn ? 0 : 1;
  } else {
    u8 played = kNoCard;
    if (play) {
      n.pdrawn = card;
      n.pend_bonus = flipped;
      n.phase = kPhaseResolve;
      // resolve_terminal_turn, resolve_game_turn and resolve_turn, up to the resolution
      if (terminal_finished(n) || has_ct_choice(n)) return kWrongPhase;
      if (game_finished(n) || has_pending_choice(n)) return kWrongPhase;
      played = n.pplayed;
    }
    const u64 pm = play ? floor_matches(n, played) : 0;
    const u32 pmc = popc(pm);
    const bool same = play && (played >> 2) == (card >> 2);
    if (same && pmc == 1 && !r.last_turn) {  // ppuk: the three cards stay on the floor
      n.floor |= bit(played) | bit(card) | flipped;
      const u16 mb = month_bit(played);
      n.ppuk |= mb;
      if (n.actor == 0) n.owner1 &= (u16)~mb; else n.owner1 |= mb;
      if (flipped & bit(kBonus2)) n.b2ppuk |= mb;  // turn50.h:241-250
      if (flipped & bit(kBonus3)) n.b3ppuk |= mb;
      r.events |= kEvPpuk;
    } else if (same && pmc == 2) {
      n.floor &= ~pm;
      capture_cards(n, pm | bit(played) | bit(card) | flipped, r);
      r.events |= kEvTtadak;
    } else if (same && pmc == 0) {
      capture_cards(n, bit(played) | bit(card) | flipped, r);
      if (!r.last_turn) r.events |= kEvJjok;
    } else {
      if (play) {
        const u8 rs = resolve_card_against_floor(n, played, a.pmatch, r);
        if (rs != kResOk) return map_resolve(rs);
      }
      const u8 rs = resolve_card_against_floor(n, card, a.dmatch, r);
      if (rs != kResOk) return map_resolve(rs);
      if (flipped) capture_cards(n, flipped, r);
    }
    if (n.floor == 0 && r.captured != 0) r.events |= kEvSweep;  // turn50.h:499-502
    finish_resolved_turn(n);
    steal = (u8)(base_steal + steal_count(r));
  }
  const PiResult pt = apply_pi_steal(n, actor, steal, a.pisel);
  if (pt.status != kPiOk) return map_pi(pt.status);
  if (!bonus) finish_turn_game(n, actor);
  if (play && (r.events & kEvTtadak) && n.turn == 1u) add_side_payment(n, actor, 7);
  if (!bonus || pt.transfer != 0)
    update_missions(n, actor, bonus ? pt.transfer : cap_of(n, actor) & ~cap_before);
  if (bonus) {
    open_bonus_chongtong_choice(n, actor, (u16)(chongtong_months(active_hand(n)) & ~ct_before));
    return kOk;
  }
  if (play) record_completed_turn_ppuk(n, actor, (r.events & kEvPpuk) != 0);
  sync_game_stop(n);
  return kOk;
}

// rollout50.h:231-385; the held-card bookkeeping of apply_action50 (391-399) included.
CG_HD u8 apply_action(Env& e, const Action& a) {
  if (terminal_finished(e)) return kGameFinished;
  Env& n = e;  // in place: the caller's copy is the transaction
  n.held0 |= n.hand0;
  n.held1 |= n.hand1;
  if (a.kind == kChongtongWin || a.kind == kChongtongContinue) {
    if (apply_chongtong_action(n, a.kind == kChongtongWin) != 0) return kNotLegal;
  } else if (a.kind == kGo || a.kind == kStop) {
    if (apply_terminal_go_stop(n, a.kind == kStop) != 0) return kNotLegal;
  } else if (a.kind == kGukjinPi || a.kind == kGukjinAnimal) {
    if (apply_terminal_gukjin(n, a.kind == kGukjinPi) != 0) return kNotLegal;
  } else {
    if (has_ct_choice(n) || has_pending_choice(n)) return kWrongPhase;
    const u8 status = apply_turn_action(n, a);
    if (status != kOk) return status;
  }
  n.held0 |= n.hand0;  // apply_action50 (rollout50.h:391-399)
  n.held1 |= n.hand1;
  return kOk;
}

// ----------------------------------------------------------------- policy50.h ----
CG_HD u8 decision_kind(const Env& e) {  // policy50.h:151-160
  if (terminal_finished(e)) return kDecNone;
  if (has_ct_choice(e)) return kDecChongtong;
  if (has_gukjin_decision(e)) return kDecGukjin;
  if (has_decision(e)) return kDecGoStop;
  if (e.phase == kPhasePlay) return kDecPrimary;
  return kDecNone;
}
CG_HD u8 decision_player(const Env& e) {  // policy50.h:162-171
  if (terminal_finished(e)) return kNoPlayer;
  if (has_ct_choice(e)) return e.ct_actor;
  if (has_gukjin_decision(e)) return (u8)(e.gdec - 1u);
  if (has_decision(e)) return e.dact;
  return e.actor;
}

// The 179-way mask in three words (torch50.h:90-94).
struct Mask3 { u64 w0, w1, w2; };
CG_HD void mask_set(Mask3& m, u32 a) {
  if (a < 64) m.w0 |= 1ull << a;
  else if (a < 128) m.w1 |= 1ull << (a - 64);
  else if (a < kActionCount) m.w2 |= 1ull << (a - 128);
}
CG_HD bool mask_has(const Mask3& m, u32 a) {
  if (a < 64) return (m.w0 >> a) & 1u;
  if (a < 128) return (m.w1 >> (a - 64)) & 1u;
  if (a < kActionCount) return (m.w2 >> (a - 128)) & 1u;
  return false;
}

// policy50.h:173-236
CG_HD Mask3 legal_primary(const Env& e) {
  Mask3 m{0, 0, 0};
  const u8 d = decision_kind(e);
  if (d == kDecChongtong) { mask_set(m, kActCtWin); mask_set(m, kActCtContinue); return m; }
  if (d == kDecGoStop) { mask_set(m, kActGo); mask_set(m, kActStop); return m; }
  if (d != kDecPrimary) return m;
  const u64 hand = active_hand(e);
  if (e.stock == 0) return m;
  const SpecialMonths sp = special_months(e);
  const u16 bombs = sp.bombs, grenades = sp.grenades, shakes = sp.shakes;
  const u16 forced = (u16)(bombs | grenades);
  u64 standard = hand & kStdMask;
  // card plays 0..47 (one bit per card, minus forced months)
  const u64 plays = standard & ~month_cards_of(forced);
  const u64 shake_cards = standard & month_cards_of(shakes);
  m.w0 |= plays;                                    // actions 0..47
  if (hand & bit(kBonus2)) m.w0 |= 1ull << 48;      // action 48
  if (hand & bit(kBonus3)) m.w0 |= 1ull << 49;      // action 49
  // shakes: action 50 + card
  m.w0 |= (shake_cards << 50);
  m.w1 |= (shake_cards >> 14);
  // bombs 98 + month (word1 bit 34+m), grenades 110 + month (word1 bit 46+m)
  m.w1 |= (u64)bombs << 34;
  m.w1 |= (u64)grenades << 46;
  if (cred_of(e, e.actor) != 0) m.w1 |= 1ull << (kActBombCredit - 64);
  return m;
}

// postchance50.h:84-148: decode without the canonical completion.
CG_HD u8 decode_primary_raw(const Env& e, u16 index, const Mask3& legal, Action& a) {
  if (index == kActGukjinPi || index == kActGukjinAnimal) {
    if (decision_kind(e) != kDecGukjin) { a = invalid_action(); return kNotLegal; }
    a = make_action(index == kActGukjinPi ? kGukjinPi : kGukjinAnimal);
    return kOk;
  }
  if (index >= kActPrimaryCount || !mask_has(legal, index)) { a = invalid_action(); return kNotLegal; }
  if (index < kActBonus) { a = make_action(kPlayCard); a.card = (u8)index; return kOk; }
  if (index < kActShake) {
    a = make_action(kPlayBonus);
    a.card = index == kActBonus ? kBonus2 : kBonus3;
    return kOk;
  }
  if (index < kActBomb) {
    a = make_action(kShake);
    a.card = (u8)(index - kActShake);
    a.month = a.card >> 2;
    return kOk;
  }
  if (index < kActGrenade) { a = make_action(kBomb); a.month = (u8)(index - kActBomb); return kOk; }
  if (index < kActBombCredit) {
    a = make_action(kGrenade);
    a.month = (u8)(index - kActGrenade);
    return kOk;
  }
  if (index == kActBombCredit) { a = make_action(kBombCredit); return kOk; }
  if (index == kActGo) { a = make_action(kGo); return kOk; }
  if (index == kActStop) { a = make_action(kStop); return kOk; }
  if (index == kActCtWin) { a = make_action(kChongtongWin); return kOk; }
  a = make_action(kChongtongContinue);
  return kOk;
}

// Observation packet (PolicyObservation50, policy50.h:49-120) plus the torch packet
// fields the encoder reads (torch50.h:96-106).
struct Obs {
  u64 own_hand, floor, own_cap, opp_cap, pending_public, unseen;
  u16 own_shaken, opp_shaken, ppuk, own_ppuk, opp_ppuk, b2ppuk, b3ppuk, ct_months, turn;
  u8 decision_kind, stock_count, own_go, opp_go, own_lgo, opp_lgo, own_base, opp_base;
  u8 own_bombs, opp_bombs, own_cred, opp_cred, own_pcount, opp_pcount, own_streak, opp_streak;
  u8 own_gdp, opp_gdp;
  u64 mission;
  i32 own_side;
  u8 mtype, mmult, own_mm, opp_mm, own_locked, opp_locked, round, last_turn;
  u16 neutral;
  u64 own_played, opp_played, opp_known;
  u8 own_first, opp_hand_count, own_pi, opp_pi, own_bright, opp_bright;
  u8 own_animal, opp_animal, own_ribbon, opp_ribbon;
  u32 stop_points;
};

CG_HD Obs empty_obs() {
  Obs o;
  o.own_hand = o.floor = o.own_cap = o.opp_cap = o.pending_public = o.unseen = 0;
  o.own_shaken = o.opp_shaken = o.ppuk = o.own_ppuk = o.opp_ppuk = o.b2ppuk = o.b3ppuk = 0;
  o.ct_months = o.turn = 0;
  o.decision_kind = o.stock_count = o.own_go = o.opp_go = o.own_lgo = o.opp_lgo = 0;
  o.own_base = o.opp_base = o.own_bombs = o.opp_bombs = o.own_cred = o.opp_cred = 0;
  o.own_pcount = o.opp_pcount = o.own_streak = o.opp_streak = o.own_gdp = o.opp_gdp = 0;
  o.mission = 0;
  o.own_side = 0;
  o.mtype = o.mmult = o.own_mm = o.opp_mm = o.own_locked = o.opp_locked = o.round = 0;
  o.last_turn = 0;
  o.neutral = 0;
  o.own_played = o.opp_played = o.opp_known = 0;
  o.own_first = o.opp_hand_count = o.own_pi = o.opp_pi = o.own_bright = o.opp_bright = 0;
  o.own_animal = o.opp_animal = o.own_ribbon = o.opp_ribbon = 0;
  o.stop_points = 0;
  return o;
}

// policy50.h:354-365
CG_HD u32 stop_points(const Env& e) {
  if (decision_kind(e) != kDecGoStop) return 0;
  Env s = e;
  if (apply_terminal_go_stop(s, true) != 0 || !terminal_finished(s)) return 0;
  const Settlement st = settle(s);
  if (!st.ok) return 0;
  return st.final_points > 0xFFFFFFFFull ? 0xFFFFFFFFu : (u32)st.final_points;
}

// policy50.h:367-467
CG_HD Obs pack_observation(const Env& e) {
  Obs o;
  u32 player = decision_player(e);
  if (player > 1u) player = e.actor & 1u;
  const u32 opp = player ^ 1u;
  o.own_hand = hand_of(e, player);
  o.own_cap = cap_of(e, player);
  o.opp_cap = cap_of(e, opp);
  u64 pending = e.pend_bonus;  // policy50.h:339-346
  if (is_std(e.pplayed)) pending |= bit(e.pplayed);
  if (is_std(e.pdrawn)) pending |= bit(e.pdrawn);
  o.pending_public = pending;
  o.floor = e.floor;
  const u64 known = o.own_hand | e.floor | o.own_cap | o.opp_cap | pending;
  o.opp_known = rev_of(e, opp) & kDeckMask & ~known;
  o.unseen = kDeckMask & ~known & ~o.opp_known;
  const u64 opp_hand = hand_of(e, opp);
  const u16 owner1_months = (u16)(e.owner1 & kMonthBits);
  const u16 owner0_months = (u16)(e.ppuk & (u16)~owner1_months);
  o.own_ppuk = player == 0 ? owner0_months : owner1_months;
  o.opp_ppuk = player == 0 ? owner1_months : owner0_months;
  const u16 shaken0 = (u16)(e.shaken0 | e.sh4_0), shaken1 = (u16)(e.shaken1 | e.sh4_1);
  o.own_shaken = player == 0 ? shaken0 : shaken1;
  o.opp_shaken = player == 0 ? shaken1 : shaken0;
  const Score own = player_score(e, player), other = player_score(e, opp);
  o.ppuk = e.ppuk;
  o.b2ppuk = e.b2ppuk;
  o.b3ppuk = e.b3ppuk;
  o.ct_months = e.ct_months;
  o.turn = e.turn;
  o.decision_kind = decision_kind(e);
  o.stock_count = (u8)popc(e.stock);
  o.own_go = go_of(e, player);
  o.opp_go = go_of(e, opp);
  o.own_lgo = lgo_of(e, player);
  o.opp_lgo = lgo_of(e, opp);
  o.own_base = own.total;
  o.opp_base = other.total;
  o.own_bombs = bombs_of(e, player);
  o.opp_bombs = bombs_of(e, opp);
  o.own_cred = cred_of(e, player);
  o.opp_cred = cred_of(e, opp);
  o.own_pcount = pcount_of(e, player);
  o.opp_pcount = pcount_of(e, opp);
  o.own_streak = streak_of(e, player);
  o.opp_streak = streak_of(e, opp);
  o.own_gdp = gukjin_double_pi(e, player);
  o.opp_gdp = gukjin_double_pi(e, opp);
  o.mission = e.mission;
  o.own_side = player == 0 ? e.side0 : -e.side0;
  o.mtype = e.mtype;
  o.mmult = e.mmult;
  o.own_mm = mm_of(e, player);
  o.opp_mm = mm_of(e, opp);
  o.own_locked = gukjin_locked(e, player);
  o.opp_locked = gukjin_locked(e, opp);
  o.round = round_multiplier(e);
  o.last_turn = is_last_turn(e);
  o.neutral = e.neutral;
  o.own_played = held_of(e, player) & ~o.own_hand;
  o.opp_played = held_of(e, opp) & ~opp_hand;
  o.own_first = (u8)((((e.actor ^ e.turn) & 1u)) == player);  // policy50.h:350-352
  o.opp_hand_count = (u8)popc(opp_hand);
  o.own_pi = own.pi_units;
  o.opp_pi = other.pi_units;
  o.own_bright = own.bright_count;
  o.opp_bright = other.bright_count;
  o.own_animal = own.animal_count;
  o.opp_animal = other.animal_count;
  o.own_ribbon = own.ribbon_count;
  o.opp_ribbon = other.ribbon_count;
  o.stop_points = stop_points(e);
  return o;
}

// ------------------------------------------------------------- postchance50.h ----
struct Pending { Action action; u64 sel_pi; u16 prim; u8 actor, active; };
CG_HD Pending pending_of(const Env& e) {
  return Pending{Action{e.a_kind, e.a_card, e.a_month, e.a_pmatch, e.a_dmatch, e.a_pisel},
                 e.sel_pi, e.prim, e.pactor, e.pactive};
}
CG_HD void set_pending(Env& e, const Pending& p) {
  e.a_kind = p.action.kind; e.a_card = p.action.card; e.a_month = p.action.month;
  e.a_pmatch = p.action.pmatch; e.a_dmatch = p.action.dmatch; e.a_pisel = p.action.pisel;
  e.sel_pi = p.sel_pi; e.prim = p.prim; e.pactor = p.actor; e.pactive = p.active;
}

struct Probe { u8 status, decision; u64 legal_cards; u8 revealed, requested; };

// postchance50.h:150-204.  On a choice for the drawn card, `table` is the turn with
// the played card resolved (ResolveChoiceProbe50::table).
CG_HD u8 probe_resolve_choices(const Env& e, u8 pchoice, u8 dchoice, u8& decision,
                               u64& legal, Env& table, bool& use_table) {
  decision = kDecNone;
  legal = 0;
  use_table = false;
  if (e.phase != kPhaseResolve) return kResWrongPhase;
  const u8 played = e.pplayed, drawn = e.pdrawn;
  const u32 pmc = popc(floor_matches(e, played));
  const bool same = (played >> 2) == (drawn >> 2);
  if (same && pmc == 1 && !is_last_turn(e)) return kResOk;
  if (same && (pmc == 0 || pmc == 2)) return kResOk;
  Env n = e;
  Resolve r{kResOk, 0, 0, 0, 0, 0};
  u64 candidates = floor_matches(n, played);
  u8 s = resolve_card_against_floor(n, played, pchoice, r);
  if (s == kResChoiceRequired) { decision = kDecResolvePlayed; legal = candidates; return s; }
  if (s != kResOk) return s;
  n.pplayed = kNoCard;
  candidates = floor_matches(n, drawn);
  table = n;
  s = resolve_card_against_floor(n, drawn, dchoice, r);
  if (s == kResChoiceRequired) {
    decision = kDecResolveDrawn;
    legal = candidates;
    use_table = true;
    return s;
  }
  if (s != kResOk) return s;
  return kResOk;
}

// postchance50.h:214-258
CG_HD Probe probe_pi_choice(const Env& staged, const Pending& p, u8 revealed, u8 requested) {
  const u32 victim = (p.actor & 1u) ^ 1u;
  const u64 candidates = pi_card_mask(cap_of(staged, victim), gukjin_option(staged, victim));
  const u8 available = (u8)popc(candidates);
  const u8 selected = (u8)popc(p.sel_pi);
  if ((p.sel_pi & ~candidates) != 0)
    return Probe{kInvalidPiSelection, kDecNone, 0, revealed, requested};
  if (requested == 0 || available <= requested || p.sel_pi == 0) {
    if (p.sel_pi != 0 && (requested == 0 || available <= requested))
      return Probe{kInvalidPiSelection, kDecNone, 0, revealed, requested};
    return Probe{kOk, kDecNone, 0, revealed, requested};
  }
  if (selected > requested) return Probe{kInvalidPiSelection, kDecNone, 0, revealed, requested};
  if (selected < requested)
    return Probe{kOk, kDecPiCard, candidates & ~p.sel_pi, revealed, requested};
  return Probe{kOk, kDecNone, 0, revealed, requested};
}

// postchance50.h:260-312
CG_HD Probe probe_regular(const Env& e, const Pending& p, Env& staged, bool shake) {
  staged = e;
  u8 status = shake ? map_special(begin_shake(staged, p.action.card))
                    : map_turn(begin_regular_play_terminal(staged, p.action.card));
  if (status != kOk) return Probe{status, kDecNone, 0, kNoCard, 0};
  status = map_turn(draw_for_terminal(staged));
  if (status != kOk) return Probe{status, kDecNone, 0, kNoCard, 0};
  const u8 revealed = staged.pdrawn;
  u8 decision;
  u64 legal;
  Env table;
  bool use_table;
  const u8 cs = probe_resolve_choices(staged, p.action.pmatch, p.action.dmatch, decision, legal,
                                      table, use_table);
  if (cs == kResChoiceRequired) {
    if (use_table) staged = table;
    return Probe{kOk, decision, legal, revealed, 0};
  }
  if (cs == kResInvalidChoice) return Probe{kInvalidResolveChoice, kDecNone, 0, revealed, 0};
  if (cs != kResOk) return Probe{kNotLegal, kDecNone, 0, revealed, 0};
  Env resolved = staged;
  const Resolve r = resolve_turn(resolved, p.action.pmatch, p.action.dmatch);
  if (r.status != kResOk) return Probe{map_resolve(r.status), kDecNone, 0, revealed, 0};
  staged = resolved;
  return probe_pi_choice(staged, p, revealed, steal_count(r));
}

// postchance50.h:314-328
CG_HD Probe probe_bonus(const Env& e, const Pending& p, Env& staged) {
  staged = e;
  u8 steal, replacement;
  const u8 s = play_bonus_for_turn(staged, p.action.card, steal, replacement);
  const u8 status = map_turn(s);
  if (status != kOk) return Probe{status, kDecNone, 0, kNoCard, 0};
  return probe_pi_choice(staged, p, replacement, steal);
}

// postchance50.h:330-416
CG_HD Probe probe_special(const Env& e, const Pending& p, Env& staged) {
  staged = e;
  const u8 actor = p.actor;
  u8 base_steal = 0;
  if (p.action.kind == kBomb || p.action.kind == kGrenade) {
    const bool grenade = p.action.kind == kGrenade;
    const u8 month = p.action.month;
    if (!special_ready(staged) || month >= 12) return Probe{kNotLegal, kDecNone, 0, kNoCard, 0};
    const u16 mb = (u16)(1u << month);
    const u16 legal = grenade ? legal_grenade_months(staged) : legal_bomb_months(staged);
    if ((legal & mb) == 0) return Probe{kNotLegal, kDecNone, 0, kNoCard, 0};
    const u64 hand = hand_of(staged, actor);
    const u64 hc = hand & month_cards(month);
    const u64 fc = std_floor(staged) & month_cards(month);
    set_hand(staged, actor, hand & ~hc);
    staged.floor &= ~fc;
    set_cap(staged, actor, cap_of(staged, actor) | hc | fc);
    set_cred(staged, actor, (u8)(cred_of(staged, actor) + (grenade ? 1u : 2u)));
    if (!grenade) { if (actor == 0) ++staged.bombs0; else ++staged.bombs1; }
    base_steal = is_last_turn(staged) ? 0 : 1;
  } else if (p.action.kind == kBombCredit) {
    if (!special_ready(staged) || cred_of(staged, actor) == 0)
      return Probe{kNotLegal, kDecNone, 0, kNoCard, 0};
    set_cred(staged, actor, (u8)(cred_of(staged, actor) - 1u));
  } else {
    return Probe{kInvalidAction, kDecNone, 0, kNoCard, 0};
  }
  const DrawOnly d = draw_only_special(staged, p.action.dmatch);
  if (d.status == kSpResolveChoiceRequired) {
    staged.pdrawn = d.drawn;
    staged.pend_bonus = d.bonuses;
    return Probe{kOk, kDecResolveDrawn, floor_matches(staged, d.drawn), d.drawn, 0};
  }
  if (d.status == kSpInvalidResolveChoice)
    return Probe{kInvalidResolveChoice, kDecNone, 0, d.drawn, 0};
  if (d.status != kSpOk) return Probe{map_special(d.status), kDecNone, 0, d.drawn, 0};
  const u8 requested = (u8)(base_steal + steal_count(d.resolve));
  finish_draw_only(staged);
  return probe_pi_choice(staged, p, d.drawn, requested);
}

// The probe of the six turn-taking kinds as one transition, as apply_turn_action is to
// apply_turn_action_per_kind: each kind runs its own prologue (probe_regular's begin and
// draw checks, probe_bonus's play_bonus_for_turn checks, probe_special's card moves), then
// one draw, one resolution and one pi-choice probe serve every kind.  The resolution of a
// played card runs once and stops at the first floor choice, where probe_regular resolves
// on a copy to find the choice (probe_resolve_choices) and, when none is open, resolves
// again with resolve_turn: the same captures in the same order, so the same state.  Same
// Probe fields and, where the probe succeeds, the same staged state as the per-kind probes
// (the caller observes it).
CG_HD Probe probe_turn_action(const Env& e, const Pending& p, Env& staged) {
  const Action& a = p.action;
  const bool bonus = a.kind == kPlayBonus;
  const bool special = a.kind == kBomb || a.kind == kGrenade || a.kind == kBombCredit;
  const bool play = !bonus && !special;  // kShake or kPlayCard
  staged = e;
  u8 base_steal = 0;
  if (bonus) {  // play_bonus_for_turn up to the draw
    if (staged.phase != kPhasePlay) return Probe{kWrongPhase, kDecNone, 0, kNoCard, 0};
    if (!is_bonus_card(a.card) || (active_hand(staged) & bit(a.card)) == 0)
      return Probe{kNotLegal, kDecNone, 0, kNoCard, 0};
    if (staged.stock == 0) return Probe{kStockEmpty, kDecNone, 0, kNoCard, 0};
  } else if (special) {  // probe_special's moves
    const u8 actor = p.actor;
    if (a.kind == kBombCredit) {
      if (!special_ready(staged) || cred_of(staged, actor) == 0)
        return Probe{kNotLegal, kDecNone, 0, kNoCard, 0};
      set_cred(staged, actor, (u8)(cred_of(staged, actor) - 1u));
    } else {
      const bool grenade = a.kind == kGrenade;
      const u8 month = a.month;
      if (!special_ready(staged) || month >= 12) return Probe{kNotLegal, kDecNone, 0, kNoCard, 0};
      const u16 mb = (u16)(1u << month);
      const u16 legal = grenade ? legal_grenade_months(staged) : legal_bomb_months(staged);
      if ((legal & mb) == 0) return Probe{kNotLegal, kDecNone, 0, kNoCard, 0};
      const u64 hand = hand_of(staged, actor);
      const u64 hc = hand & month_cards(month);
      const u64 fc = std_floor(staged) & month_cards(month);
      set_hand(staged, actor, hand & ~hc);
      staged.floor &= ~fc;
      set_cap(staged, actor, cap_of(staged, actor) | hc | fc);
      set_cred(staged, actor, (u8)(cred_of(staged, actor) + (grenade ? 1u : 2u)));
      if (!grenade) { if (actor == 0) ++staged.bombs0; else ++staged.bombs1; }
      base_steal = is_last_turn(staged) ? 0 : 1;
    }
  } else {  // probe_regular: begin, then draw_for_terminal up to the draw
    const u8 status = a.kind == kShake ? map_special(begin_shake(staged, a.card))
                                       : map_turn(begin_regular_play_terminal(staged, a.card));
    if (status != kOk) return Probe{status, kDecNone, 0, kNoCard, 0};
    if (terminal_finished(staged) || has_ct_choice(staged) || game_finished(staged) ||
        has_pending_choice(staged) || staged.phase != kPhaseDraw)
      return Probe{kWrongPhase, kDecNone, 0, kNoCard, 0};
  }
  // The draw (as in apply_turn_action).
  u64 stock = staged.stock, rng = staged.rng, flipped = 0;
  u8 card = kNoCard;
  while (stock != 0) {
    card = draw_uniform(stock, rng);
    if (bonus || !is_bonus_card(card)) break;
    flipped |= bit(card);
    card = kNoCard;
  }
  if (bonus ? !is_physical(card) : !is_std(card))
    return Probe{kStockEmpty, kDecNone, 0, kNoCard, 0};
  staged.stock = stock;
  staged.rng = rng;
  u8 steal;
  if (bonus) {
    const u64 hand = active_hand(staged);
    set_hand(staged, staged.actor, (hand & ~bit(a.card)) | bit(card));
    set_cap(staged, staged.actor, cap_of(staged, staged.actor) | bit(a.card));
    steal = is_last_turn(staged) ? 0 : 1;
  } else {
    if (play) {
      staged.pdrawn = card;
      staged.pend_bonus = flipped;
      staged.phase = kPhaseResolve;
    }
    Env n = staged;
    Resolve r{kResOk, 0, 0, 0, 0, (u8)is_last_turn(n)};
    const u8 played = play ? n.pplayed : kNoCard;
    const u64 pm = play ? floor_matches(n, played) : 0;
    const u32 pmc = popc(pm);
    const bool same = play && (played >> 2) == (card >> 2);
    if (same && pmc == 1 && !r.last_turn) {  // resolve_turn's same-month cases: no choice
      n.floor |= bit(played) | bit(card) | flipped;
      const u16 mb = month_bit(played);
      n.ppuk |= mb;
      if (n.actor == 0) n.owner1 &= (u16)~mb; else n.owner1 |= mb;
      if (flipped & bit(kBonus2)) n.b2ppuk |= mb;
      if (flipped & bit(kBonus3)) n.b3ppuk |= mb;
      r.events |= kEvPpuk;
    } else if (same && pmc == 2) {
      n.floor &= ~pm;
      capture_cards(n, pm | bit(played) | bit(card) | flipped, r);
      r.events |= kEvTtadak;
    } else if (same && pmc == 0) {
      capture_cards(n, bit(played) | bit(card) | flipped, r);
      if (!r.last_turn) r.events |= kEvJjok;
    } else {
      if (play) {
        const u8 rs = resolve_card_against_floor(n, played, a.pmatch, r);
        if (rs == kResChoiceRequired) return Probe{kOk, kDecResolvePlayed, pm, card, 0};
        if (rs != kResOk) return Probe{kInvalidResolveChoice, kDecNone, 0, card, 0};
        n.pplayed = kNoCard;  // ResolveChoiceProbe50::table (postchance50.h:150-204)
      }
      const u64 candidates = floor_matches(n, card);
      const u8 rs = resolve_card_against_floor(n, card, a.dmatch, r);
      if (rs == kResChoiceRequired) {
        if (special) {
          n.pdrawn = card;
          n.pend_bonus = flipped;
        }
        staged = n;
        return Probe{kOk, kDecResolveDrawn, candidates, card, 0};
      }
      if (rs != kResOk) return Probe{kInvalidResolveChoice, kDecNone, 0, card, 0};
      if (flipped) capture_cards(n, flipped, r);
    }
    if (n.floor == 0 && r.captured != 0) r.events |= kEvSweep;
    finish_resolved_turn(n);
    staged = n;
    steal = (u8)(base_steal + steal_count(r));
  }
  return probe_pi_choice(staged, p, card, steal);
}

// postchance50.h:418-456, the turn-taking kinds per kind (the plain restatement of
// probe_postchance, kept for the host check of the two).
CG_HD Probe probe_postchance_per_kind(const Env& e, const Pending& p, Env& staged) {
  if (!p.active) { staged = e; return Probe{kWrongPhase, kDecNone, 0, kNoCard, 0}; }
  switch (p.action.kind) {
    case kPlayCard: return probe_regular(e, p, staged, false);
    case kShake: return probe_regular(e, p, staged, true);
    case kPlayBonus: return probe_bonus(e, p, staged);
    case kBomb:
    case kGrenade:
    case kBombCredit: return probe_special(e, p, staged);
    case kGo:
    case kStop:
    case kChongtongWin:
    case kChongtongContinue:
    case kGukjinPi:
    case kGukjinAnimal: staged = e; return Probe{kOk, kDecNone, 0, kNoCard, 0};
    default: staged = e; return Probe{kInvalidAction, kDecNone, 0, kNoCard, 0};
  }
}

// postchance50.h:418-456
CG_HD Probe probe_postchance(const Env& e, const Pending& p, Env& staged) {
  if (!p.active) { staged = e; return Probe{kWrongPhase, kDecNone, 0, kNoCard, 0}; }
  if (is_turn_kind(p.action.kind)) return probe_turn_action(e, p, staged);
  staged = e;
  switch (p.action.kind) {
    case kGo:
    case kStop:
    case kChongtongWin:
    case kChongtongContinue:
    case kGukjinPi:
    case kGukjinAnimal: return Probe{kOk, kDecNone, 0, kNoCard, 0};
    default: return Probe{kInvalidAction, kDecNone, 0, kNoCard, 0};
  }
}

// postchance50.h:509-539.  Returns the ActionStatus50; committed set on commit.  The
// reference probes the staged action and then applies it.  apply_action fails wherever
// the probe would stop the action (a floor choice still open, an empty stock, an invalid
// choice), so with no pi card selected the action is applied first and the probe runs
// only when the apply fails; a pi selection (which the probe checks more strictly than
// the transfer) keeps the reference order.  Same status, same state, same commit in
// every case.  Both applies run on a copy that is kept only on success: apply_action and
// every transition under it work in place and return a failure status as soon as one
// step fails, so this copy is the whole action's transaction (apply_action50 copies the
// state once, rollout50.h:238).
CG_HD u8 continue_postchance(Env& e, bool& committed) {
  committed = false;
  Pending p = pending_of(e);
  Action a = p.action;
  if (p.sel_pi != 0) a.pisel = p.sel_pi;
  u8 s = kOk;
  if (p.sel_pi == 0) {
    Env applied = e;
    s = apply_action(applied, a);
    if (s == kOk) {
      e = applied;
      p.action = a;
      p.active = 0;
      set_pending(e, p);
      committed = true;
      return kOk;
    }
  }
  Env staged;
  const Probe probe = probe_postchance(e, p, staged);
  if (probe.status != kOk) return probe.status;
  if (probe.decision != kDecNone) return kOk;
  if (p.sel_pi == 0) return s;  // the apply above failed with `s`
  Env applied = e;
  s = apply_action(applied, a);
  if (s != kOk) return s;
  e = applied;
  p.action = a;
  p.active = 0;
  set_pending(e, p);
  committed = true;
  return kOk;
}

// postchance50.h:541-556 up to its continue_postchance50 call: stages the decoded
// primary action as the pending action.  The caller continues on kOk.
CG_HD u8 stage_postchance(Env& e, u16 primary, const Mask3& legal) {
  Action a;
  const u8 status = decode_primary_raw(e, primary, legal, a);
  u8 actor = decision_player(e);
  if (actor > 1u) actor = e.actor & 1u;
  Pending p{a, 0, primary, actor, 0};
  set_pending(e, p);
  if (status != kOk) return status;
  e.pactive = 1;
  return kOk;
}

// postchance50.h:558-587 up to its continue_postchance50 call (the card is already
// checked against the probe's legal set): records the choice in the pending action.
CG_HD void record_postchance_choice(Env& e, u8 decision, u8 card) {
  if (decision == kDecResolvePlayed) e.a_pmatch = card;
  else if (decision == kDecResolveDrawn) e.a_dmatch = card;
  else if (decision == kDecPiCard) e.sel_pi |= bit(card);
}

// ------------------------------------------------------------------ torch50.h ----
CG_HD bool nagari_ready(const Env& e) {  // torch50.h:196-201 with rollout50.h:576-582
  return e.pactive == 0 && !terminal_finished(e) && !has_ct_choice(e) &&
         !has_pending_choice(e) && e.phase == kPhasePlay && e.hand0 == 0 && e.hand1 == 0 &&
         e.cred0 == 0 && e.cred1 == 0;
}
CG_HD void refresh_done(Env& e) {  // torch50.h:203-216
  if (terminal_finished(e)) { e.done = 1; e.nagari = 0; return; }
  if (nagari_ready(e)) { e.done = 1; e.nagari = 1; return; }
  e.done = 0;
  e.nagari = 0;
}

CG_HD i64 reward0(const Env& e) {  // torch50.h:472-478 with settlement50.h:221-225
  if (e.done == 0) return 0;
  if (e.nagari != 0) return e.side0;
  if (!terminal_finished(e)) return 0;
  return settlement_reward0(settle(e));
}

// make_torch_env50 (torch50.h:218-236) over make_terminal_game_state50
// (terminal50.h:277-315), make_turn_state50 (turn50.h:150-192) and
// deal_shin_matgo_50 (deal.h:82-92).
CG_HD Env create_env(u64 seed, u32 first) {
  first &= 1u;
  u64 s = seed;
  u64 remaining = kDeckMask;
  u64 hand0 = 0, hand1 = 0, floor = 0;
  // Draw k (k = 0 .. 27) picks among 50 - k cards with the (k + 1)-th SplitMix64 word of
  // the seed, unless Lemire's product falls below the bound (then uniform_bounded may
  // redraw).  The words do not depend on the cards, so they are computed up front, side by
  // side, and only the picks run in sequence; a deal with any product below its bound
  // (about 28 x 50 / 2^32 of deals) takes the draw-by-draw path instead.
  u32 rank[28];
  bool direct = true;
#pragma unroll
  for (int k = 0; k < 28; ++k) {
    u64 w = seed + (u64)(k + 1) * 0x9e3779b97f4a7c15ull;
    w = (w ^ (w >> 30)) * 0xbf58476d1ce4e5b9ull;
    w = (w ^ (w >> 27)) * 0x94d049bb133111ebull;
    w ^= w >> 31;
    const u64 product = (u64)(u32)(w >> 32) * (u64)(50 - k);
    direct = direct && (u32)product >= (u32)(50 - k);
    rank[k] = (u32)(product >> 32);
  }
  if (direct) {
#pragma unroll
    for (int k = 0; k < 28; ++k) {
      const u8 card = select_rank(remaining, rank[k]);
      remaining &= ~bit(card);
      if (k < 10) hand0 |= bit(card);
      else if (k < 20) hand1 |= bit(card);
      else floor |= bit(card);
    }
    s = seed + 28ull * 0x9e3779b97f4a7c15ull;
  } else {
    for (int i = 0; i < 10; ++i) hand0 |= bit(draw_uniform(remaining, s));
    for (int i = 0; i < 10; ++i) hand1 |= bit(draw_uniform(remaining, s));
    for (int i = 0; i < 8; ++i) floor |= bit(draw_uniform(remaining, s));
  }
  const u64 deal_rng = s;
  Env e;
  e.hand0 = hand0; e.hand1 = hand1; e.cap0 = 0; e.cap1 = 0;
  // refill_initial_floor_bonuses50: floor bonuses go to the first player.
  const u64 bonuses = floor & kBonusMask;
  floor &= ~bonuses;
  if (first == 0) e.cap0 |= bonuses; else e.cap1 |= bonuses;
  int missing = (int)popc(bonuses);
  u64 stock = remaining;
  u64 rng = deal_rng;
  while (missing > 0 && stock != 0) {
    const u8 card = draw_uniform(stock, rng);
    if (is_bonus_card(card)) {
      if (first == 0) e.cap0 |= bit(card); else e.cap1 |= bit(card);
      continue;
    }
    floor |= bit(card);
    --missing;
  }
  e.floor = floor; e.stock = stock; e.rng = rng; e.pend_bonus = 0;
  e.ppuk = e.owner1 = e.b2ppuk = e.b3ppuk = 0;
  e.turn = 0; e.actor = (u8)first; e.phase = kPhasePlay;
  e.pplayed = kNoCard; e.pdrawn = kNoCard;
  e.mission = 0;
  e.neutral = floor_triple_months(floor & kStdMask);
  e.go0 = e.go1 = e.lgo0 = e.lgo1 = 0;
  e.dact = kNoPlayer; e.winner = kNoPlayer; e.gdec = 0;
  e.shaken0 = e.shaken1 = 0; e.bombs0 = e.bombs1 = 0; e.cred0 = e.cred1 = 0;
  e.sh4_0 = e.sh4_1 = 0;
  e.pcount0 = e.pcount1 = e.streak0 = e.streak1 = 0;
  e.ct_actor = kNoPlayer; e.ct_months = 0;
  e.twinner = kNoPlayer; e.treason = kReasonNone; e.tpoints = 0;
  e.side0 = 0; e.round = 1; e.mtype = kMissionNone; e.mmult = 0; e.mm0 = 0; e.mm1 = 0;
  e.held0 = 0; e.held1 = 0; e.rev0 = 0; e.rev1 = 0;
  assign_mission(e, deal_rng);  // seeded from the deal, before the floor refill
  update_missions(e, 0, 0);
  update_missions(e, 1, 0);
  e.held0 = e.hand0;
  e.held1 = e.hand1;
  // detect_initial_chongtong50 on the dealt hands and the refilled floor
  const u16 ch0 = chongtong_months(hand0), ch1 = chongtong_months(hand1);
  const u16 chf = chongtong_months(floor);
  if (chf != 0) mark_terminal(e, first, kReasonFloorChongtong, 10);
  else if (ch0 != 0 && ch1 != 0) mark_terminal(e, first, kReasonInitialChongtong, 10);
  else if (ch0 != 0) mark_terminal(e, 0, kReasonInitialChongtong, 10);
  else if (ch1 != 0) mark_terminal(e, 1, kReasonInitialChongtong, 10);
  // PostChancePending50{} and counters are all zero.
  e.a_kind = 0; e.a_card = 0; e.a_month = 0; e.a_pmatch = 0; e.a_dmatch = 0; e.a_pisel = 0;
  e.sel_pi = 0; e.prim = 0; e.pactor = 0; e.pactive = 0;
  e.n_primary = e.n_choice = e.n_resolve = e.n_pi = e.n_bonus = e.n_special = e.n_go = 0;
  e.status = kOk;
  refresh_done(e);
  return e;
}

// Action mask, status and decision kind of make_torch_packet50 (torch50.h:245-296)
// without the observation.
struct PacketHead { u8 status, decision_kind, player; Mask3 legal; };

CG_HD Mask3 choice_mask(u64 cards) {  // torch50.h:172-182: action 127 + card
  cards &= kDeckMask;
  return Mask3{0, cards << 63, cards >> 1};
}

CG_HD PacketHead packet_head(const Env& e) {
  PacketHead h;
  if (e.pactive != 0) {
    const Pending p = pending_of(e);
    Env staged;
    const Probe probe = probe_postchance(e, p, staged);
    h.player = e.pactor;
    if (probe.status != kOk) {
      h.status = probe.status;
      h.decision_kind = kDecNone;
      h.legal = Mask3{0, 0, 0};
      return h;
    }
    h.status = kOk;
    h.decision_kind = probe.decision;
    h.legal = choice_mask(probe.legal_cards);
    return h;
  }
  u8 player = decision_player(e);
  if (player > 1u) player = e.actor & 1u;
  h.player = player;
  h.status = kOk;
  const u8 kind = decision_kind(e);
  if (e.done != 0) {
    h.legal = Mask3{0, 0, 0};
    h.decision_kind = 0;
  } else if (kind == kDecGukjin) {
    h.legal = Mask3{0, 0, (1ull << (kActGukjinPi - 128)) | (1ull << (kActGukjinAnimal - 128))};
    h.decision_kind = kind;
  } else {
    h.legal = legal_primary(e);
    h.decision_kind = kind;
  }
  return h;
}

// Full torch packet (torch50.h:245-296 with postchance50.h:458-497).
struct Packet {
  Obs obs;
  PacketHead head;
  u16 primary_action;
  u8 revealed;
};

// One probe and one pack_observation per lane: a pending row observes its staged
// state, every other row the state itself.  The kernels inline everything, so a wave
// with both kinds of rows would otherwise run the probe and the observation (with its
// Go/Stop settlement) once per branch.
CG_HD Packet make_packet(const Env& e) {
  Packet pk;
  const bool pending = e.pactive != 0;
  // The probe's fields as scalars, and the probe writes straight into the state that is
  // observed: a conditionally assigned aggregate is not split into registers and would
  // live in private memory.
  u8 pr_status = kOk, pr_decision = kDecNone, pr_revealed = kNoCard;
  u64 pr_legal = 0;
  Env src = e;
  if (pending) {
    const Probe probe = probe_postchance(e, pending_of(e), src);
    pr_status = probe.status;
    pr_decision = probe.decision;
    pr_revealed = probe.revealed;
    pr_legal = probe.legal_cards;
    // pack_postchance_observation50 (postchance50.h:458-466); on a failed probe the
    // observation is discarded below
    src.actor = e.pactor;
    src.turn = e.turn;
  }
  Obs o = pack_observation(src);
  if (pending) {
    pk.primary_action = e.prim;
    pk.revealed = pr_revealed;
    pk.head.player = e.pactor;
    if (pr_status != kOk) {
      pk.head.status = pr_status;
      pk.head.decision_kind = kDecNone;
      pk.head.legal = Mask3{0, 0, 0};
      pk.obs = empty_obs();
      return pk;
    }
    o.decision_kind = pr_decision;  // postchance50.h:467-480
    if (is_physical(pr_revealed)) {
      const u64 b = bit(pr_revealed);
      const u64 known = o.own_hand | o.floor | o.own_cap | o.opp_cap | o.pending_public;
      if ((known & b) == 0) {
        o.pending_public |= b;
        o.unseen &= ~b;
      }
    }
    pk.head.status = kOk;
    pk.head.decision_kind = pr_decision;
    pk.head.legal = choice_mask(pr_legal);
    pk.obs = o;
    return pk;
  }
  // torch50.h:245-296, primary branch
  u8 player = decision_player(e);
  if (player > 1u) player = e.actor & 1u;
  pk.head.player = player;
  pk.head.status = kOk;
  const u8 kind = decision_kind(e);
  if (e.done != 0) {
    pk.head.legal = Mask3{0, 0, 0};
    pk.head.decision_kind = 0;
  } else if (kind == kDecGukjin) {
    pk.head.legal = Mask3{0, 0, (1ull << (kActGukjinPi - 128)) | (1ull << (kActGukjinAnimal - 128))};
    pk.head.decision_kind = kind;
  } else {
    pk.head.legal = legal_primary(e);
    pk.head.decision_kind = kind;
  }
  pk.obs = o;
  pk.primary_action = kInvalidAction16;
  pk.revealed = kNoCard;
  return pk;
}

// Step result (TorchStepResult50, torch50.h:123-129).
struct StepOut { u8 status; i64 reward0; u8 done, nagari, committed; };

// torch50.h:491-540 given `head` = packet_head(e) of this very state (the caller has it
// from the observation it just built: make_packet(e).head is the same head).
CG_HD StepOut torch_step_head(Env& e, u16 action, const PacketHead& head) {
  if (e.done != 0) {
    e.status = kGameFinished;
    return StepOut{e.status, reward0(e), e.done, e.nagari, 0};
  }
  if (head.status != kOk) {
    e.status = head.status;
    return StepOut{e.status, 0, e.done, e.nagari, 0};
  }
  if (!mask_has(head.legal, action)) {
    e.status = kNotLegal;
    return StepOut{e.status, 0, e.done, e.nagari, 0};
  }
  // A pending row records its choice, any other row stages its primary action; both
  // then continue the pending action (one call site, so a wave whose games take both
  // branches runs the apply once).
  bool committed = false;
  u8 s = kOk;
  if (e.pactive != 0) {
    if (head.decision_kind == kDecPiCard) ++e.n_pi; else ++e.n_resolve;
    ++e.n_choice;
    record_postchance_choice(e, head.decision_kind, (u8)(action - kActChoice));
  } else {
    s = stage_postchance(e, action, head.legal);
  }
  if (s == kOk) s = continue_postchance(e, committed);
  if (s != kOk) {
    e.status = s;
    return StepOut{e.status, 0, e.done, e.nagari, 0};
  }
  if (committed) {  // torch50.h:480-489
    const u8 kind = e.a_kind;
    ++e.n_primary;
    if (kind == kPlayBonus) ++e.n_bonus;
    if (kind == kShake || kind == kBomb || kind == kGrenade || kind == kBombCredit) ++e.n_special;
    if (kind == kGo) ++e.n_go;
  }
  e.status = kOk;
  refresh_done(e);
  return StepOut{kOk, reward0(e), e.done, e.nagari, (u8)committed};
}

// torch50.h:491-540
CG_HD StepOut torch_step(Env& e, u16 action) {
  if (e.done != 0) {
    e.status = kGameFinished;
    return StepOut{e.status, reward0(e), e.done, e.nagari, 0};
  }
  return torch_step_head(e, action, packet_head(e));
}

// torch50.h:644-678: event words of a committed action (before/after diff).
CG_HD void make_event(const Env& b, const Env& a, i64* out) {
  const u32 actor = a.pactor & 1u;
  const u64 hb = hand_of(b, actor), ha = hand_of(a, actor);
  const u64 played = hb & ~ha, drawn = ha & ~hb;
  out[0] = (i64)played;
  out[1] = (i64)drawn;
  out[2] = (i64)(b.stock & ~a.stock & ~drawn);
  out[3] = (i64)(a.cap0 & ~b.cap0);
  out[4] = (i64)(a.cap1 & ~b.cap1);
  out[5] = (i64)(b.cap0 & ~a.cap0);
  out[6] = (i64)(b.cap1 & ~a.cap1);
  out[7] = (i64)(rev_of(a, actor) & ~rev_of(b, actor));
  out[8] = (i64)actor | ((i64)a.a_kind << 8);
}

// torch50.h:684-698
CG_HD void pack_start(const Env& e, i64* out) {
  out[0] = (i64)e.hand0;
  out[1] = (i64)e.hand1;
  out[2] = (i64)e.floor;
  out[3] = (i64)e.cap0;
  out[4] = (i64)e.cap1;
  out[5] = (i64)e.mission;
  out[6] = (i64)e.neutral;
  out[7] = (i64)e.mtype | ((i64)e.mmult << 8) | ((i64)(e.actor & 1u) << 16) |
           ((i64)e.mm0 << 24) | ((i64)e.mm1 << 32);
}

// ------------------------------------------------------- canonical driver ----
// canonical_torch_action50 (torch50.h:542-558): the deterministic action of the
// reference's canonical rollout, as a unified action index (kInvalidAction16 when there
// is none).  A pending row takes its lowest legal choice card.  Otherwise the kinds are
// taken in canonical_action50's order (rollout50.h:496-574): Chongtong win, Gukjin as
// double pi, Go on the first decision and Stop after, then in the play phase a bomb
// credit, the lower bonus card, the first bomb month, the first grenade month, the first
// shake month (its lowest card in hand), the lowest standard card; primary_action_index50
// (policy50.h:238-271) maps each to its index.  The reference also probes each play kind
// on a copy (canonicalize_*, rollout50.h:400-489) and gives no action when a probe fails;
// only the probe's status reaches the torch form, and in reachable states it is kOk (the
// oracle's restatement keeps the probes and is checked against the reference build).
CG_HD u16 canonical_action(const Env& e) {
  if (e.done != 0) return kInvalidAction16;
  if (e.pactive != 0) {
    const PacketHead h = packet_head(e);
    if (h.status != kOk) return kInvalidAction16;
    // choice_mask: action 127 + card in bits 63 of w1 and 0..48 of w2
    if ((h.legal.w1 >> 63) != 0) return kActChoice;
    if (h.legal.w2 != 0) return (u16)(kActChoice + 1 + ctz64(h.legal.w2));
    return kInvalidAction16;
  }
  if (terminal_finished(e)) return kInvalidAction16;
  if (has_ct_choice(e)) return kActCtWin;
  if (has_gukjin_decision(e)) return kActGukjinPi;
  if (has_decision(e)) return go_of(e, e.dact) == 0 ? kActGo : kActStop;
  if (e.phase != kPhasePlay) return kInvalidAction16;
  if (cred_of(e, e.actor) != 0) return kActBombCredit;
  const u64 hand = active_hand(e);
  const u64 bonuses = hand & kBonusMask;
  if (bonuses != 0) return (bonuses & bit(kBonus2)) != 0 ? kActBonus : (u16)(kActBonus + 1);
  const SpecialMonths sm = special_months(e);
  if (sm.bombs != 0) return (u16)(kActBomb + ctz64(sm.bombs));
  if (sm.grenades != 0) return (u16)(kActGrenade + ctz64(sm.grenades));
  if (sm.shakes != 0) {
    const u32 month = ctz64(sm.shakes);
    const u64 cards = hand & kStdMask & (0xFull << (4 * month));
    return cards != 0 ? (u16)(kActShake + ctz64(cards)) : kInvalidAction16;
  }
  const u64 standard = hand & kStdMask;
  if (standard != 0) return (u16)ctz64(standard);
  return kInvalidAction16;
}

// RolloutEnd50 (rollout50.h:70-76)
enum : u8 { kEndTerminal = 0, kEndNagari = 1, kEndStalled = 2, kEndActionError = 3,
            kEndMaxActions = 4 };

// finish_torch_rollout50 (torch50.h:560-596) with finish_terminal_rollout50
// (rollout50.h:584-614), packed into five words:
//   0 final_points   1 reward0
//   2 actions | turns << 16 | bonus_actions << 32 | special_actions << 48
//   3 go_actions | end << 16 | action_status << 24 | terminal_reason << 32 | winner << 40
//     | next_round_multiplier << 48
//   4 choice_actions | resolve_choices << 16 | pi_choices << 32
CG_HD void canonical_digest(const Env& e, u8 fallback_end, i64* out) {
  u64 points = 0;
  i64 reward = 0;
  u8 end = fallback_end, status = e.status, reason = kReasonNone, winner = kNoPlayer, mult = 1;
  if (terminal_finished(e)) {
    const Settlement st = settle(e);
    reason = e.treason;
    if (!st.ok) {
      end = kEndActionError;
      status = kInvalidAction;
      winner = e.twinner;
    } else {
      end = kEndTerminal;
      status = kOk;
      winner = st.winner;
      points = st.final_points;
      reward = settlement_reward0(st);
    }
  } else if (e.nagari != 0) {
    end = kEndNagari;
    status = kOk;
    mult = 2;
    reward = e.side0;  // nagari_reward50 (settlement50.h:220-225)
  }
  out[0] = (i64)points;
  out[1] = reward;
  out[2] = (i64)((u64)e.n_primary | (u64)e.turn << 16 | (u64)e.n_bonus << 32 |
                 (u64)e.n_special << 48);
  out[3] = (i64)((u64)e.n_go | (u64)end << 16 | (u64)status << 24 | (u64)reason << 32 |
                 (u64)winner << 40 | (u64)mult << 48);
  out[4] = (i64)((u64)e.n_choice | (u64)e.n_resolve << 16 | (u64)e.n_pi << 32);
}

// rollout_canonical_torch50 (torch50.h:598-619) on a dealt game, in place.
CG_HD void rollout_canonical(Env& e, u32 max_actions, i64* out) {
  while (e.done == 0 && e.n_primary < max_actions) {
    const u16 action = canonical_action(e);
    if (action == kInvalidAction16) {
      e.status = kInvalidAction;
      canonical_digest(e, kEndStalled, out);
      return;
    }
    const StepOut so = torch_step(e, action);
    if (so.status != kOk) {
      canonical_digest(e, kEndActionError, out);
      return;
    }
  }
  canonical_digest(e, e.done != 0 ? kEndTerminal : kEndMaxActions, out);
}

// stock_indexed (torch50_ext.cu:336-363): next 8 draws, stopping at the first
// non-standard card; byte k = card id, 0xFF once stopped.
CG_HD u64 peek_stock(const Env& e) {
  u64 packed = ~0ull;
  u64 remaining = e.stock, rng = e.rng;
  for (int k = 0; k < 8; ++k) {
    const u8 card = remaining != 0 ? draw_uniform(remaining, rng) : kNoCard;
    if (!is_std(card)) break;
    packed &= ~(0xFFull << (8 * k));
    packed |= (u64)card << (8 * k);
  }
  return packed;
}


// ------------------------------------------------------- feature encoding ----
// encode_torch_packet50 (torch50.h:334-470) in two stages: feature_row() turns a
// packet into 20 bit-plane words and 56 precomputed floats, and feature_at() reads
// feature f from them.  The GPU observe kernel keeps the rows in LDS and lets each
// lane emit consecutive features, so the 2,880-byte rows leave as coalesced stores.
//   words: 0-5 card planes (own hand, floor, own/opp captured, pending public, unseen)
//          6-13 month planes (own/opp shaken, ppuk, own/opp ppuk, bonus2/3 ppuk,
//          pending chongtong), 14 choice cards, 15 neutral ppuk, 16 mission,
//          17-19 own played, opponent played, opponent known hand
//   dense: 0-6 -> 446-452, 7-32 -> 453-478, 33-37 -> 491-495, 38-53 -> 544-559,
//          54-55 -> 710-711
constexpr int kFeatWords = 20;
constexpr int kFeatDense = 56;
constexpr int kStopBitsTable = 4095;  // log2(1 + p) / 12 for p < 4095; 1.0 beyond

struct FeatRow {
  u64 w[kFeatWords];
  float d[kFeatDense];
};

CG_HD float unit_value(u32 value, u32 scale) {  // torch50.h:298-303
  if (scale == 0) return 0.0f;
  const float r = (float)value / (float)scale;
  return r > 1.0f ? 1.0f : r;
}

CG_HD void feature_row(const Packet& pk, const float* stop_bits, FeatRow& r) {
  const Obs& o = pk.obs;
  r.w[0] = o.own_hand; r.w[1] = o.floor; r.w[2] = o.own_cap; r.w[3] = o.opp_cap;
  r.w[4] = o.pending_public; r.w[5] = o.unseen;
  r.w[6] = o.own_shaken; r.w[7] = o.opp_shaken; r.w[8] = o.ppuk; r.w[9] = o.own_ppuk;
  r.w[10] = o.opp_ppuk; r.w[11] = o.b2ppuk; r.w[12] = o.b3ppuk; r.w[13] = o.ct_months;
  // choice cards: action 127 + c legal
  const u64 choice = ((pk.head.legal.w1 >> 63) | (pk.head.legal.w2 << 1)) & kDeckMask;
  r.w[14] = choice;
  r.w[15] = o.neutral;
  r.w[16] = o.mission;
  r.w[17] = o.own_played; r.w[18] = o.opp_played; r.w[19] = o.opp_known;
  const u8 dk = pk.head.decision_kind;
  float* d = r.d;
  d[0] = o.own_first != 0 ? 1.0f : 0.0f;
  for (u32 k = 1; k <= 5; ++k) d[k] = dk == k ? 1.0f : 0.0f;
  d[6] = unit_value(o.opp_hand_count, 10);
  float* s = d + 7;
  s[0] = unit_value(o.turn, 32);
  s[1] = unit_value(o.stock_count, 30);
  s[2] = unit_value(o.own_go, 8);
  s[3] = unit_value(o.opp_go, 8);
  s[4] = unit_value(o.own_lgo, 64);
  s[5] = unit_value(o.opp_lgo, 64);
  s[6] = unit_value(o.own_base, 64);
  s[7] = unit_value(o.opp_base, 64);
  s[8] = unit_value(o.own_bombs, 4);
  s[9] = unit_value(o.opp_bombs, 4);
  s[10] = unit_value(o.own_cred, 4);
  s[11] = unit_value(o.opp_cred, 4);
  s[12] = unit_value(o.own_pcount, 3);
  s[13] = unit_value(o.opp_pcount, 3);
  s[14] = unit_value(o.own_streak <= 3u ? o.own_streak : 0u, 3);
  s[15] = unit_value(o.opp_streak <= 3u ? o.opp_streak : 0u, 3);
  s[16] = o.own_gdp != 0 ? 1.0f : 0.0f;
  s[17] = o.opp_gdp != 0 ? 1.0f : 0.0f;
  s[18] = o.stop_points < (u32)kStopBitsTable ? stop_bits[o.stop_points] : 1.0f;
  s[19] = pk.primary_action < kActPrimaryCount
              ? (float)(pk.primary_action + 1u) / (float)kActPrimaryCount : 0.0f;
  s[20] = is_physical(pk.revealed) ? (float)(pk.revealed + 1u) / 50.0f : 0.0f;
  s[21] = unit_value(o.own_pi, 20);
  s[22] = unit_value(popc(choice), 50);
  s[23] = unit_value(popc(o.own_hand), 50);
  s[24] = unit_value(popc(o.floor), 50);
  s[25] = unit_value(popc(o.unseen), 50);
  float* t = d + 33;
  t[0] = unit_value(o.opp_pi, 20);
  t[1] = unit_value(o.own_bright, 5);
  t[2] = unit_value(o.opp_bright, 5);
  t[3] = unit_value(o.own_animal, 10);
  t[4] = unit_value(o.opp_animal, 10);
  float* x = d + 38;
  x[0] = o.mtype == kMissionEasy ? 1.0f : 0.0f;
  x[1] = o.mtype == kMissionNormal ? 1.0f : 0.0f;
  x[2] = o.mtype == kMissionHard ? 1.0f : 0.0f;
  x[3] = o.mtype == kMissionNoCondition ? 1.0f : 0.0f;
  x[4] = o.mtype == kMissionTriple ? 1.0f : 0.0f;
  x[5] = unit_value(o.mmult, 4);
  x[6] = unit_value(o.own_mm, 8);
  x[7] = unit_value(o.opp_mm, 8);
  x[8] = dk == kDecGukjin ? 1.0f : 0.0f;
  x[9] = o.own_locked != 0 ? 1.0f : 0.0f;
  x[10] = o.opp_locked != 0 ? 1.0f : 0.0f;
  x[11] = o.last_turn != 0 ? 1.0f : 0.0f;
  const float side = (float)o.own_side / 64.0f;
  x[12] = side > 1.0f ? 1.0f : side < -1.0f ? -1.0f : side;
  x[13] = unit_value(o.round, 8);
  x[14] = (o.own_streak == kPpukFirst || o.own_streak == kPpukSecond) ? 1.0f : 0.0f;
  x[15] = (o.opp_streak == kPpukFirst || o.opp_streak == kPpukSecond) ? 1.0f : 0.0f;
  d[54] = unit_value(o.own_ribbon, 10);
  d[55] = unit_value(o.opp_ribbon, 10);
}

CG_HD float bit_feature(u64 w, u32 b) { return ((w >> b) & 1u) ? 1.0f : 0.0f; }

CG_HD float feature_at(const u64* w, const float* d, u32 f) {
  if (f < 300) return bit_feature(w[f / 50], f % 50);
  if (f < 396) { const u32 g = f - 300; return bit_feature(w[6 + g / 12], g % 12); }
  if (f < 446) return bit_feature(w[14], f - 396);
  if (f < 479) return d[f - 446];
  if (f < 491) return bit_feature(w[15], f - 479);
  if (f < 496) return d[33 + (f - 491)];
  if (f < 544) return bit_feature(w[16], f - 496);
  if (f < 560) return d[38 + (f - 544)];
  if (f < 710) { const u32 g = f - 560; return bit_feature(w[17 + g / 50], g % 50); }
  if (f < 712) return d[54 + (f - 710)];
  return 0.0f;
}


// Per-row dword record read by the GPU feature writer, laid out so that a lane turns a
// few record reads into four consecutive features.  The 720 features in feature order as
// a bit array: bit f is feature f for every feature that is 0 or 1 (the planes and the
// 0/1 flags and one-hots among the scalars), 0 for the others; feature quad q (features
// 4q..4q+3) is one nibble, at dword q / 8, bits 4 (q % 8) .. 4 (q % 8) + 3.  Then the float
// bits of the 37 other scalars, in feature order (dense_pos).  A feature is its bit's
// 0 / 1.0f pattern ORed with its dense dword (0 where it has none), which is exact for
// every value, signed zeros included.  A record takes kFeatRecord + 1 dwords: the last is
// a zero pad that a reader may OR into any feature.
constexpr int kRecBits = 23;   // 720 bits
constexpr int kRecDense = 37;
constexpr int kFeatRecord = kRecBits + kRecDense;  // 60 dwords
constexpr u32 kFeatQuads = 180;

// Position of feature f among the dense dwords, or -1 for a 0/1 feature or the padding:
// 452-468, 471-478 (scalars), 491-495 (counts), 549-551 and 556-557 (extension scalars),
// 710-711 (ribbons).
CG_HD int dense_pos(u32 f) {
  if (f >= 452 && f <= 468) return (int)(f - 452);
  if (f >= 471 && f <= 478) return (int)(17 + (f - 471));
  if (f >= 491 && f <= 495) return (int)(25 + (f - 491));
  if (f >= 549 && f <= 551) return (int)(30 + (f - 549));
  if (f == 556 || f == 557) return (int)(33 + (f - 556));
  if (f == 710 || f == 711) return (int)(35 + (f - 710));
  return -1;
}

// ORs the low n bits of v into the bit array at bit `pos`.
CG_HD void put_bits(u64* acc, u32 pos, u64 v, u32 n) {
  v &= (1ull << n) - 1ull;  // n < 64
  const u32 k = pos >> 6, s = pos & 63u;
  acc[k] |= v << s;
  if (s != 0 && s + n > 64u) acc[k + 1] |= v >> (64u - s);
}

// 1 when a 0/1 scalar is 1.0f.
CG_HD u64 flag_bit(float v) { return v != 0.0f ? 1ull : 0ull; }

// Every index below is a constant, so the row stays in registers.
CG_HD void feature_record(const FeatRow& r, u32* rec) {
  u64 acc[12];
#pragma unroll
  for (int k = 0; k < 12; ++k) acc[k] = 0;
#pragma unroll
  for (int p = 0; p < 6; ++p) put_bits(acc, 50u * p, r.w[p], 50);            // 0-299
#pragma unroll
  for (int m = 0; m < 8; ++m) put_bits(acc, 300u + 12u * m, r.w[6 + m], 12);  // 300-395
  put_bits(acc, 396, r.w[14], 50);                                           // 396-445
  put_bits(acc, 479, r.w[15], 12);                                           // 479-490
  put_bits(acc, 496, r.w[16], 48);                                           // 496-543
#pragma unroll
  for (int p = 0; p < 3; ++p) put_bits(acc, 560u + 50u * p, r.w[17 + p], 50);  // 560-709
  // the 0/1 scalars (feature f = dense index + 446, 491 or 544 - 38 as in feature_at)
  const float* d = r.d;
#pragma unroll
  for (int k = 0; k <= 5; ++k) put_bits(acc, 446u + k, flag_bit(d[k]), 1);  // 446-451
  put_bits(acc, 469, flag_bit(d[23]), 1);
  put_bits(acc, 470, flag_bit(d[24]), 1);
#pragma unroll
  for (int k = 0; k < 5; ++k) put_bits(acc, 544u + k, flag_bit(d[38 + k]), 1);  // 544-548
#pragma unroll
  for (int k = 0; k < 4; ++k) put_bits(acc, 552u + k, flag_bit(d[46 + k]), 1);  // 552-555
  put_bits(acc, 558, flag_bit(d[52]), 1);
  put_bits(acc, 559, flag_bit(d[53]), 1);
#pragma unroll
  for (int k = 0; k < kRecBits; ++k) rec[k] = (u32)(acc[k >> 1] >> (32 * (k & 1)));
  // the other scalars, in feature order
  u32* dn = rec + kRecBits;
#pragma unroll
  for (int k = 0; k < 17; ++k) dn[k] = __builtin_bit_cast(u32, d[6 + k]);        // 452-468
#pragma unroll
  for (int k = 0; k < 8; ++k) dn[17 + k] = __builtin_bit_cast(u32, d[25 + k]);   // 471-478
#pragma unroll
  for (int k = 0; k < 5; ++k) dn[25 + k] = __builtin_bit_cast(u32, d[33 + k]);   // 491-495
#pragma unroll
  for (int k = 0; k < 3; ++k) dn[30 + k] = __builtin_bit_cast(u32, d[43 + k]);   // 549-551
  dn[33] = __builtin_bit_cast(u32, d[50]);                                       // 556
  dn[34] = __builtin_bit_cast(u32, d[51]);                                       // 557
  dn[35] = __builtin_bit_cast(u32, d[54]);                                       // 710
  dn[36] = __builtin_bit_cast(u32, d[55]);                                       // 711
  rec[kFeatRecord] = 0u;  // the pad that features without a dense dword read
}

}  // namespace cugo_amd
