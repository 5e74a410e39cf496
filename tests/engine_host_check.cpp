// Host checks of engine helpers that replace a plainer formulation with bit arithmetic.
// Built and run by tests/test_cpu_engine_host.py (host code only; no GPU):
//  1. feature_record + the GPU writer's decode (nibble -> 0/1.0f patterns, OR the dense
//     dword or the zero pad) == feature_at for every one of the 720 features;
//  2. hangame_steal_selection (six mask passes) == the card-by-card loop of
//     pi_transfer.h:90-110;
//  3. special_months == legal_special_months (special50.h:71-95) for bombs, grenades and
//     shakes;
//  4. apply_turn_action (the six turn-taking kinds as one transition) == the per-kind
//     composition (rollout50.h:268-376) on states of random games: same status, and on
//     success the same row;
//  5. probe_postchance (the same kinds' post-chance probe as one transition) ==
//     probe_postchance_per_kind (postchance50.h:418-456) on the same states: same Probe
//     fields, and where the probe succeeds the same staged row;
//  6. create_env's deal (the draws' SplitMix64 words computed up front) == the draw-by-draw
//     deal (deal.h:82-92 with draw_uniform) on random seeds and on seeds where a draw's
//     Lemire product falls below its bound (found by search, so the fallback runs).
// Prints one line per check and exits non-zero on the first mismatch.
#include "engine.h"

#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

using namespace cugo_amd;

static u32 bits_of(float f) { u32 b; std::memcpy(&b, &f, 4); return b; }

static int check_records(std::mt19937_64& g) {
  const int binary[] = {0, 1, 2, 3, 4, 5, 23, 24, 38, 39, 40, 41, 42, 46, 47, 48, 49, 52, 53};
  for (int it = 0; it < 20000; ++it) {
    FeatRow r;
    for (int k = 0; k < kFeatWords; ++k) r.w[k] = g() & (it % 3 ? ~0ull : g());
    for (int k = 0; k < kFeatDense; ++k) {
      u32 b = (u32)g();
      if (it % 5 == 0) b = 0x80000000u;  // -0.0
      if (it % 7 == 0) b = 0x7fc00001u;  // a NaN payload
      std::memcpy(&r.d[k], &b, 4);
    }
    for (int k : binary) r.d[k] = (g() & 1) ? 1.0f : 0.0f;
    u32 rec[kFeatRecord + 1];
    std::memset(rec, 0xAB, sizeof rec);
    feature_record(r, rec);
    for (u32 q = 0; q < kFeatQuads; ++q) {
      const u32 nib = rec[q >> 3] >> (4 * (q & 7));
      for (u32 k = 0; k < 4; ++k) {
        const int pos = dense_pos(4 * q + k);
        const u32 got = ((0u - ((nib >> k) & 1u)) & 0x3f800000u) |
                        rec[kRecBits + (pos >= 0 ? pos : kRecDense)];
        const u32 want = bits_of(feature_at(r.w, r.d, 4 * q + k));
        if (got != want) {
          std::printf("record: feature %u got %08x want %08x\n", 4 * q + k, got, want);
          return 1;
        }
      }
    }
  }
  std::printf("records: 20000 rows, 720 features each, equal\n");
  return 0;
}

// pi_transfer.h:90-110 as written there: keys in order, cards in ascending order.
static u64 steal_loop(u64 candidates, u64 mission, bool owns_mission, u32 count) {
  u64 chosen = 0;
  for (u32 key = 0; key < 6 && count != 0; ++key) {
    const bool use_mission = owns_mission ? key >= 3 : (key & 1u) != 0;
    const u32 value = owns_mission ? 1 + key % 3 : 1 + key / 2;
    u64 pool = candidates & (use_mission ? mission : ~mission);
    while (pool != 0 && count != 0) {
      const u32 card = (u32)__builtin_ctzll(pool);
      pool &= pool - 1;
      if (pi_card_value(card) != value) continue;
      chosen |= bit(card);
      --count;
    }
  }
  return chosen;
}

static int check_steal(std::mt19937_64& g) {
  const u64 pis = kPlainPi | kDoublePi | kBonusMask | bit(kGukjin);
  for (int it = 0; it < 500000; ++it) {
    const u64 cand = (g() & g() & pis) | (it % 4 == 0 ? pis & g() : 0);
    const u64 mission = g() & g() & kDeckMask;
    const bool owns = g() & 1;
    const u32 count = (u32)(g() % 8);
    if (hangame_steal_selection(cand, mission, owns, count) != steal_loop(cand, mission, owns, count)) {
      std::printf("steal: candidates %llx mission %llx owns %d count %u\n",
                  (unsigned long long)cand, (unsigned long long)mission, owns, count);
      return 1;
    }
  }
  std::printf("steal selection: 500000 cases equal\n");
  return 0;
}

static int check_special_months(std::mt19937_64& g) {
  for (int it = 0; it < 500000; ++it) {
    Env e{};
    e.hand0 = g() & g() & kDeckMask;
    e.hand1 = g() & g() & kDeckMask;
    if (it % 3 == 0) e.hand0 |= g() & kDeckMask;
    e.floor = g() & g() & (it % 2 ? g() : ~0ull) & kDeckMask;
    e.actor = (u8)(g() & 1);
    e.shaken0 = (u16)g(); e.shaken1 = (u16)g(); e.sh4_0 = (u16)g(); e.sh4_1 = (u16)g();
    e.phase = it % 17 == 0 ? kPhaseResolve : kPhasePlay;
    e.winner = it % 19 == 0 ? 0 : kNoPlayer;
    e.dact = kNoPlayer;
    e.gdec = it % 23 == 0 ? 1 : 0;
    const SpecialMonths s = special_months(e);
    const u16 bombs = legal_special_months(e, 3, 1, false);
    const u16 grenades = legal_special_months(e, 2, 2, false);
    const u16 shakes =
        (u16)(legal_special_months(e, 3, 0, true) | legal_special_months(e, 4, 0, true));
    if (s.bombs != bombs || s.grenades != grenades || s.shakes != shakes) {
      std::printf("special months: %x/%x %x/%x %x/%x\n", s.bombs, bombs, s.grenades, grenades,
                  s.shakes, shakes);
      return 1;
    }
  }
  std::printf("special months: 500000 states equal\n");
  return 0;
}

// Any set bit of m, or kNoCard.
static u8 any_bit(u64 m, std::mt19937_64& g) {
  const u32 c = (u32)__builtin_popcountll(m);
  return c == 0 ? kNoCard : select_rank(m, (u32)(g() % c));
}

static int check_turn_actions(std::mt19937_64& g) {
  static const u8 kinds[] = {kPlayCard, kPlayCard, kPlayCard, kShake, kPlayBonus,
                             kBomb, kGrenade, kBombCredit};
  long cases = 0, ok = 0, probes = 0, probes_ok = 0, choices = 0;
  for (int game = 0; game < 3000; ++game) {
    Env e = create_env(g(), (u32)(g() & 1));
    for (int t = 0; t < 60 && !e.done; ++t) {
      // The two transitions on actions built from this state: mostly cards from the
      // actor's hand, months of its legal specials and floor cards of the card's month,
      // sometimes anything.
      for (int k = 0; k < 24; ++k) {
        Action a = make_action(kinds[g() % 8]);
        const u64 hand = active_hand(e);
        const bool wild = g() % 5 == 0;
        a.card = wild ? (u8)(g() % 52) : any_bit(hand, g);
        const SpecialMonths sm = special_months(e);
        const u16 months = a.kind == kBomb ? sm.bombs : a.kind == kGrenade ? sm.grenades
                                                                            : sm.shakes;
        a.month = wild || months == 0 ? (u8)(g() % 13) : (u8)__builtin_ctz(months);
        a.pmatch = g() % 3 ? kNoCard : any_bit(std_floor(e), g);
        a.dmatch = g() % 3 ? kNoCard : any_bit(std_floor(e), g);
        const u64 opp = pi_card_mask(cap_of(e, e.actor ^ 1u), false);
        a.pisel = g() % 4 ? 0 : opp & g();
        Env x = e, y = e;
        const u8 sx = apply_turn_action(x, a);
        const u8 sy = apply_turn_action_per_kind(y, a);
        u64 rx[kRowWords], ry[kRowWords];
        pack_row(x, rx);
        pack_row(y, ry);
        ++cases;
        if (sx != sy || (sx == kOk && std::memcmp(rx, ry, sizeof rx) != 0)) {
          std::printf("turn action: game %d turn %d kind %u card %u month %u: status %u vs %u\n",
                      game, t, a.kind, a.card, a.month, sx, sy);
          return 1;
        }
        ok += sx == kOk;
        // The post-chance probe of the same action staged as the pending one.
        Pending pd{a, 0, 0, (u8)(g() % 8 ? e.actor : g() & 1), 1};
        if (g() % 4 == 0) pd.sel_pi = opp & g();
        Env sa, sb;
        const Probe pa = probe_postchance(e, pd, sa);
        const Probe pb = probe_postchance_per_kind(e, pd, sb);
        u64 qa[kRowWords], qb[kRowWords];
        pack_row(sa, qa);
        pack_row(sb, qb);
        ++probes;
        if (pa.status != pb.status || pa.decision != pb.decision ||
            pa.legal_cards != pb.legal_cards || pa.revealed != pb.revealed ||
            pa.requested != pb.requested ||
            (pa.status == kOk && std::memcmp(qa, qb, sizeof qa) != 0)) {
          std::printf("probe: game %d turn %d kind %u card %u month %u: status %u/%u "
                      "decision %u/%u revealed %u/%u requested %u/%u\n", game, t, a.kind,
                      a.card, a.month, pa.status, pb.status, pa.decision, pb.decision,
                      pa.revealed, pb.revealed, pa.requested, pb.requested);
          return 1;
        }
        probes_ok += pa.status == kOk;
        choices += pa.decision != kDecNone;
      }
      // Advance the game with a uniform legal action.
      const PacketHead h = packet_head(e);
      const u64 w[3] = {h.legal.w0, h.legal.w1, h.legal.w2};
      const u32 c = (u32)(__builtin_popcountll(w[0]) + __builtin_popcountll(w[1]) +
                          __builtin_popcountll(w[2]));
      if (c == 0) break;
      u32 r = (u32)(g() % c);
      u16 act = 0;
      for (u32 i = 0; i < 3; ++i) {
        const u32 ci = (u32)__builtin_popcountll(w[i]);
        if (r < ci) { act = (u16)(64 * i + select_rank(w[i], r)); break; }
        r -= ci;
      }
      torch_step(e, act);
    }
  }
  std::printf("turn actions: %ld cases (%ld applied) equal\n", cases, ok);
  std::printf("post-chance probes: %ld cases (%ld ok, %ld open a choice) equal\n", probes,
              probes_ok, choices);
  return 0;
}

// deal.h:82-92 draw by draw: hands of 10, floor of 8, the stream left after them.
static void deal_by_draws(u64 seed, u64& h0, u64& h1, u64& fl, u64& rest, u64& rng) {
  u64 s = seed, remaining = kDeckMask;
  h0 = h1 = fl = 0;
  for (int i = 0; i < 10; ++i) h0 |= bit(draw_uniform(remaining, s));
  for (int i = 0; i < 10; ++i) h1 |= bit(draw_uniform(remaining, s));
  for (int i = 0; i < 8; ++i) fl |= bit(draw_uniform(remaining, s));
  rest = remaining;
  rng = s;
}

// Some draw of the deal of `seed` has Lemire's low word below its bound.
static bool low_draw(u64 seed) {
  u64 s = seed;
  for (u32 k = 0; k < 28; ++k) {
    const u64 product = (u64)(u32)(sm_next(s) >> 32) * (50u - k);
    if ((u32)product < 50u - k) return true;
  }
  return false;
}

static int check_deal(std::mt19937_64& g) {
  std::vector<u64> seeds;
  for (int i = 0; i < 200000; ++i) seeds.push_back(g());
  int found = 0;
  for (u64 seed = 0x9E3779B97F4A7C15ull; found < 4; seed += 0x2545F4914F6CDD1Dull)
    if (low_draw(seed)) { seeds.push_back(seed); ++found; }
  for (const u64 seed : seeds) {
    const Env e = create_env(seed, (u32)(seed & 1));
    u64 h0, h1, fl, rest, rng;
    deal_by_draws(seed, h0, h1, fl, rest, rng);
    // create_env moves floor bonus cards to the first player and refills the floor from
    // the stock: compare before that, through the cards and the stream it left.
    const u64 bonus = fl & kBonusMask;
    const u64 caps = e.cap0 | e.cap1;
    if (e.hand0 != h0 || e.hand1 != h1 || (bonus != 0 ? (caps & bonus) != bonus
                                                      : (e.floor != fl || e.stock != rest ||
                                                         e.rng != rng))) {
      std::printf("deal: seed %llx differs\n", (unsigned long long)seed);
      return 1;
    }
  }
  std::printf("deal: %zu seeds (%d with a draw in the rejection zone) equal\n", seeds.size(),
              found);
  return 0;
}

int main() {
  std::mt19937_64 g(20261201);
  if (check_records(g)) return 1;
  if (check_steal(g)) return 1;
  if (check_special_months(g)) return 1;
  if (check_turn_actions(g)) return 1;
  if (check_deal(g)) return 1;
  return 0;
}
