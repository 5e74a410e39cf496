// C-ABI harness over the reference's header-only Shin Matgo engine.
//
// TEST INFRASTRUCTURE ONLY.  This file is this repository's own code; it includes the
// reference headers (include/cugo/game/torch50.h) from the reference checkout at build
// time (oracle/Makefile) and exposes the batch operations of the reference extension
// (python/csrc/torch50_ext.cu:53-363) as plain CPU loops over 248-byte rows, so the
// tests and bench.py's cpu_baseline leg can run the reference engine itself.  Nothing in
// the product (cugo_amd/) links or loads this library.
//
// Row semantics follow python/csrc/torch50_ext.cu:
//   invalid env id      -> zero observation, done=1, status=-1 (:71-87, :108-118)
//   out-of-range action -> 0xFFFF, i.e. kNotLegal (:96-99)
//   clone/branch        -> byte copy of the parent, zero row for an invalid id (:271-314)
// Padding bytes of every row this harness writes are set to zero (the reference leaves
// them unspecified), so rows compare byte-for-byte with the HIP engine's rows.

#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#include <atomic>

#include "cugo/game/torch50.h"

namespace cg = cugo::game;
namespace core = cugo::core;

static_assert(sizeof(cg::TorchEnv50) == 248, "reference row size changed");

namespace {

constexpr int kF = cg::kTorch50FeatureCount;   // 720
constexpr int kA = cg::kTorch50ActionCount;    // 179
constexpr int kE = cg::kTorch50EventWords;     // 9
constexpr int kS = cg::kTorch50StartWords;     // 8

// Byte ranges of TorchEnv50 that hold no field (measured with offsetof).
constexpr int kPad[][2] = {{78, 80},   {90, 96},   {103, 104}, {116, 120}, {125, 126},
                           {130, 136}, {153, 160}, {197, 200}, {220, 224}, {241, 248}};

void zero_padding(std::uint8_t* row) {
  for (const auto& r : kPad) std::memset(row + r[0], 0, r[1] - r[0]);
}

cg::TorchEnv50 load(const std::uint8_t* row) {
  cg::TorchEnv50 env;
  std::memcpy(&env, row, sizeof env);
  return env;
}

void store(const cg::TorchEnv50& env, std::uint8_t* row) {
  std::memcpy(row, &env, sizeof env);
  zero_padding(row);
}

void write_observation(const cg::TorchEnv50& env, float* f, std::uint8_t* legal,
                       std::uint8_t* player, std::uint8_t* done, std::int16_t* status) {
  const cg::TorchPacket50 p = cg::make_torch_packet50(env);
  cg::encode_torch_packet50(p, f);
  for (int a = 0; a < kA; ++a)
    legal[a] = cg::has_torch_action50(p.legal_actions, static_cast<std::uint16_t>(a)) ? 1 : 0;
  *player = p.decision_player;
  *done = env.done != 0;
  *status = static_cast<std::int16_t>(p.status);
}

void write_invalid_observation(float* f, std::uint8_t* legal, std::uint8_t* player,
                               std::uint8_t* done, std::int16_t* status) {
  std::memset(f, 0, sizeof(float) * kF);
  std::memset(legal, 0, kA);
  *player = 0;
  *done = 1;
  *status = -1;
}

std::uint16_t clamp_action(std::int64_t raw) {
  return raw >= 0 && raw < kA ? static_cast<std::uint16_t>(raw) : cg::kInvalidTorch50Action;
}

void write_step(const cg::TorchStepResult50& r, float* reward, std::uint8_t* done,
                std::uint8_t* nagari, std::int16_t* status, std::uint8_t* committed) {
  *reward = static_cast<float>(r.reward0);
  *done = r.done != 0;
  *nagari = r.nagari != 0;
  *status = static_cast<std::int16_t>(r.status);
  *committed = r.primary_committed != 0;
}

void write_invalid_step(float* reward, std::uint8_t* done, std::uint8_t* nagari,
                        std::int16_t* status, std::uint8_t* committed) {
  *reward = 0.0f;
  *done = 1;
  *nagari = 0;
  *status = -1;
  *committed = 0;
}

bool valid(std::int64_t id, std::int64_t env_count) { return id >= 0 && id < env_count; }

// Runs body(i) for i in [0, n) over `threads` std::threads (contiguous chunks).
template <class F>
void parallel_for(std::int64_t n, int threads, F body) {
  if (threads <= 1 || n < 2) {
    for (std::int64_t i = 0; i < n; ++i) body(i);
    return;
  }
  std::atomic<std::int64_t> next{0};
  constexpr std::int64_t kChunk = 64;
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t) {
    pool.emplace_back([&] {
      for (;;) {
        const std::int64_t begin = next.fetch_add(kChunk);
        if (begin >= n) return;
        const std::int64_t end = begin + kChunk < n ? begin + kChunk : n;
        for (std::int64_t i = begin; i < end; ++i) body(i);
      }
    });
  }
  for (auto& th : pool) th.join();
}

// FNV-1a over bytes: the per-game digest of a random-policy record stream.
std::uint64_t fnv(std::uint64_t h, const void* data, std::size_t n) {
  const auto* p = static_cast<const std::uint8_t*>(data);
  for (std::size_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

std::uint64_t splitmix_first(std::uint64_t seed) {
  core::SplitMix64 s{seed};
  const std::uint64_t v = s.next_u64();
  return v != 0 ? v : 1;
}

std::uint64_t xorshift_next(std::uint64_t& x) {
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  return x;
}

}  // namespace

extern "C" {

int cugo_ref_state_bytes() { return static_cast<int>(sizeof(cg::TorchEnv50)); }

void cugo_ref_create(const std::int64_t* seeds, const std::int64_t* first, std::int64_t n,
                     std::uint8_t* states) {
  for (std::int64_t i = 0; i < n; ++i) {
    const cg::TorchEnv50 env = cg::make_torch_env50(static_cast<std::uint64_t>(seeds[i]),
                                                    static_cast<std::uint8_t>(first[i] & 1));
    store(env, states + i * 248);
  }
}

void cugo_ref_observe_indexed(const std::uint8_t* states, const std::int64_t* ids,
                              std::int64_t n, std::int64_t env_count, float* features,
                              std::uint8_t* legal, std::uint8_t* player, std::uint8_t* done,
                              std::int16_t* status) {
  for (std::int64_t i = 0; i < n; ++i) {
    const std::int64_t id = ids != nullptr ? ids[i] : i;
    if (!valid(id, env_count)) {
      write_invalid_observation(features + i * kF, legal + i * kA, player + i, done + i,
                                status + i);
      continue;
    }
    write_observation(load(states + id * 248), features + i * kF, legal + i * kA, player + i,
                      done + i, status + i);
  }
}

void cugo_ref_step_indexed(std::uint8_t* states, const std::int64_t* ids,
                           const std::int64_t* actions, std::int64_t n, std::int64_t env_count,
                           float* reward, std::uint8_t* done, std::uint8_t* nagari,
                           std::int16_t* status, std::uint8_t* committed, std::int64_t* events) {
  for (std::int64_t i = 0; i < n; ++i) {
    const std::int64_t id = ids != nullptr ? ids[i] : i;
    cg::TorchEvent50 ev{};
    if (!valid(id, env_count)) {
      write_invalid_step(reward + i, done + i, nagari + i, status + i, committed + i);
    } else {
      cg::TorchEnv50 env = load(states + id * 248);
      const cg::TorchStepResult50 r = cg::torch_step_event50(env, clamp_action(actions[i]), ev);
      store(env, states + id * 248);
      write_step(r, reward + i, done + i, nagari + i, status + i, committed + i);
    }
    if (events != nullptr) cg::pack_torch_event50(ev, events + i * kE);
  }
}

void cugo_ref_start(const std::uint8_t* states, std::int64_t n, std::int64_t* out) {
  for (std::int64_t i = 0; i < n; ++i) cg::pack_torch_start50(load(states + i * 248), out + i * kS);
}

void cugo_ref_clone_indexed(const std::uint8_t* states, const std::int64_t* ids, std::int64_t n,
                            std::int64_t env_count, std::uint8_t* children) {
  for (std::int64_t i = 0; i < n; ++i) {
    if (valid(ids[i], env_count)) std::memcpy(children + i * 248, states + ids[i] * 248, 248);
    else std::memset(children + i * 248, 0, 248);
  }
}

void cugo_ref_branch_indexed(const std::uint8_t* states, const std::int64_t* ids,
                             const std::int64_t* actions, std::int64_t n, std::int64_t env_count,
                             std::uint8_t* children, float* reward, std::uint8_t* done,
                             std::uint8_t* nagari, std::int16_t* status,
                             std::uint8_t* committed) {
  for (std::int64_t i = 0; i < n; ++i) {
    if (!valid(ids[i], env_count)) {
      std::memset(children + i * 248, 0, 248);
      write_invalid_step(reward + i, done + i, nagari + i, status + i, committed + i);
      continue;
    }
    cg::TorchEnv50 env = load(states + ids[i] * 248);
    const cg::TorchStepResult50 r = cg::torch_step50(env, clamp_action(actions[i]));
    store(env, children + i * 248);
    write_step(r, reward + i, done + i, nagari + i, status + i, committed + i);
  }
}

void cugo_ref_hands_indexed(const std::uint8_t* states, const std::int64_t* ids, std::int64_t n,
                            std::int64_t env_count, std::int64_t* hands) {
  for (std::int64_t i = 0; i < n; ++i) {
    if (!valid(ids[i], env_count)) {
      hands[2 * i] = hands[2 * i + 1] = 0;
      continue;
    }
    const cg::TorchEnv50 env = load(states + ids[i] * 248);
    hands[2 * i] = static_cast<std::int64_t>(env.game.special.game.turn.hand0);
    hands[2 * i + 1] = static_cast<std::int64_t>(env.game.special.game.turn.hand1);
  }
}

void cugo_ref_stock_indexed(const std::uint8_t* states, const std::int64_t* ids, std::int64_t n,
                            std::int64_t env_count, std::int64_t* stock) {
  for (std::int64_t i = 0; i < n; ++i) {
    std::uint64_t packed = ~0ull;
    if (valid(ids[i], env_count)) {
      const cg::TorchEnv50 env = load(states + ids[i] * 248);
      core::CardMask remaining = env.game.special.game.turn.stock;
      std::uint64_t rng = env.game.special.game.turn.rng_state;
      for (int k = 0; k < 8; ++k) {
        const core::CardId card = cg::draw_stock_card(remaining, rng);
        if (!core::is_standard_card(card)) break;
        packed &= ~(0xFFull << (8 * k));
        packed |= static_cast<std::uint64_t>(card) << (8 * k);
      }
    }
    stock[i] = static_cast<std::int64_t>(packed);
  }
}

// Exact int64 reward of player 0 for a row (torch50.h:472-478); 0 while not done.
std::int64_t cugo_ref_reward0(const std::uint8_t* row) { return cg::torch_reward0_50(load(row)); }

// Plays n random-policy games: game i is created from seed base+i with first=i&1, and
// each decision takes legal[xorshift64() % count] over the ascending legal list, the
// sampler state being SplitMix64(seed).next().  Every decision does the full observe
// (720 features + 179 mask) and step_events work.  Outputs per game: the FNV-1a digest
// of the record stream, the decision count and the exact final reward of player 0.
// If records != nullptr, the first `record_games` games also dump every step record:
//   [features f32 x720][mask u8 x179][player u8][done u8][status i16][action i64]
//   [reward f32][done u8][nagari u8][status i16][committed u8][events i64 x9]
// with at most `record_cap` steps per game.  Null output arrays are skipped (the
// timed CPU baseline passes none, so it does only the engine work).  Returns the total
// number of decisions.
constexpr int kRecordBytes = kF * 4 + kA + 1 + 1 + 2 + 8 + 4 + 1 + 1 + 2 + 1 + kE * 8;

int cugo_ref_record_bytes() { return kRecordBytes; }

std::int64_t cugo_ref_play_random(std::uint64_t base_seed, std::int64_t n, int threads,
                                  std::uint64_t* digest, std::int32_t* steps,
                                  std::int64_t* final_reward, std::uint8_t* records,
                                  std::int64_t record_games, std::int32_t record_cap) {
  std::atomic<std::int64_t> total{0};
  parallel_for(n, threads, [&](std::int64_t i) {
    const std::uint64_t seed = base_seed + static_cast<std::uint64_t>(i);
    cg::TorchEnv50 env = cg::make_torch_env50(seed, static_cast<std::uint8_t>(i & 1));
    std::uint64_t x = splitmix_first(seed);
    std::uint64_t h = 0xcbf29ce484222325ull;
    std::uint8_t rec[kRecordBytes];
    std::int32_t count = 0;
    while (env.done == 0 && count < 512) {
      std::uint8_t* r = rec;
      float* f = reinterpret_cast<float*>(r);
      std::uint8_t* legal = r + kF * 4;
      std::uint8_t* o = legal + kA;
      std::int16_t ostatus;
      write_observation(env, f, legal, o, o + 1, &ostatus);
      std::memcpy(o + 2, &ostatus, 2);
      std::uint16_t list[kA];
      int m = 0;
      for (int a = 0; a < kA; ++a)
        if (legal[a]) list[m++] = static_cast<std::uint16_t>(a);
      const std::int64_t action = m != 0 ? list[xorshift_next(x) % static_cast<unsigned>(m)] : -1;
      std::memcpy(o + 4, &action, 8);
      cg::TorchEvent50 ev{};
      const cg::TorchStepResult50 s = cg::torch_step_event50(env, clamp_action(action), ev);
      std::uint8_t* q = o + 12;
      float reward;
      std::uint8_t sd, sn, sc;
      std::int16_t ss;
      write_step(s, &reward, &sd, &sn, &ss, &sc);
      std::memcpy(q, &reward, 4);
      q[4] = sd;
      q[5] = sn;
      std::memcpy(q + 6, &ss, 2);
      q[8] = sc;
      std::int64_t words[kE];
      cg::pack_torch_event50(ev, words);
      std::memcpy(q + 9, words, sizeof words);
      if (digest != nullptr) h = fnv(h, rec, kRecordBytes);
      if (records != nullptr && i < record_games && count < record_cap)
        std::memcpy(records + (i * record_cap + count) * kRecordBytes, rec, kRecordBytes);
      ++count;
      if (m == 0) break;
    }
    if (digest != nullptr) digest[i] = h;
    if (steps != nullptr) steps[i] = count;
    if (final_reward != nullptr) final_reward[i] = cg::torch_reward0_50(env);
    total.fetch_add(count);
  });
  return total.load();
}

// Branch workload on the CPU: child i = clone(roots[ids[i]]) stepped with actions[i];
// when observe != 0 the child is also observed (features and mask written to a per-thread
// scratch, as the GPU writes them to HBM).  Returns a checksum of the children so the
// work cannot be optimised away.
std::uint64_t cugo_ref_branch_work(const std::uint8_t* roots, const std::int64_t* ids,
                                   const std::int64_t* actions, std::int64_t n, int threads,
                                   int observe) {
  std::atomic<std::uint64_t> sum{0};
  parallel_for(n, threads, [&](std::int64_t i) {
    cg::TorchEnv50 env = load(roots + ids[i] * 248);
    const cg::TorchStepResult50 r = cg::torch_step50(env, clamp_action(actions[i]));
    std::uint64_t local = static_cast<std::uint64_t>(r.status) + env.game.special.game.turn.stock;
    if (observe) {
      float f[kF];
      std::uint8_t legal[kA];
      std::uint8_t player, done;
      std::int16_t status;
      write_observation(env, f, legal, &player, &done, &status);
      std::uint32_t bits;
      std::memcpy(&bits, &f[453], 4);
      local += bits + legal[0] + player;
    }
    sum.fetch_add(local, std::memory_order_relaxed);
  });
  return sum.load();
}

// The reference's canonical rollouts (include/cugo/game/torch50.h:598-619, the torch
// form, and rollout50.h:616-703, the explicit form its GPU bench times) from
// seed[i] / first[i] with at most max_actions primary actions; five digest words a game
// (packing in oracle/matgo/canonical.h).  The explicit form has no choice counters: its
// word 4 is zero.
void pack_rollout(const cg::RolloutResult50& r, std::uint16_t choice, std::uint16_t resolve,
                  std::uint16_t pi, std::int64_t* out) {
  out[0] = static_cast<std::int64_t>(r.final_points);
  out[1] = r.reward0;
  out[2] = static_cast<std::int64_t>(
      std::uint64_t{r.actions} | std::uint64_t{r.turns} << 16 |
      std::uint64_t{r.bonus_actions} << 32 | std::uint64_t{r.special_actions} << 48);
  out[3] = static_cast<std::int64_t>(
      std::uint64_t{r.go_actions} | std::uint64_t{static_cast<std::uint8_t>(r.end)} << 16 |
      std::uint64_t{static_cast<std::uint8_t>(r.action_status)} << 24 |
      std::uint64_t{static_cast<std::uint8_t>(r.terminal_reason)} << 32 |
      std::uint64_t{r.winner} << 40 | std::uint64_t{r.next_round_multiplier} << 48);
  out[4] = static_cast<std::int64_t>(std::uint64_t{choice} | std::uint64_t{resolve} << 16 |
                                     std::uint64_t{pi} << 32);
}

void cugo_ref_rollout_canonical(const std::int64_t* seeds, const std::int64_t* first,
                                std::int64_t n, int max_actions, int threads, int explicit_form,
                                std::int64_t* out) {
  parallel_for(n, threads, [&](std::int64_t i) {
    const auto seed = static_cast<std::uint64_t>(seeds[i]);
    const auto f = static_cast<std::uint8_t>(first[i] & 1);
    const auto cap = static_cast<std::uint16_t>(max_actions);
    if (explicit_form) {
      pack_rollout(cg::rollout_canonical50(seed, f, cap), 0, 0, 0, out + 5 * i);
    } else {
      const cg::TorchRollout50 r = cg::rollout_canonical_torch50(seed, f, cap);
      pack_rollout(r.result, r.choice_actions, r.resolve_choices, r.pi_choices, out + 5 * i);
    }
  });
}

}  // extern "C"
