// PyTorch-ROCm extension `cugo_torch50_ext`: the reference module's operations
// (python/csrc/torch50_ext.cpp:36-72) over the C ABI of libcugo_hip.so.
//
// Each operation checks its tensors like the reference (torch50_ext.cu:26-51, same
// messages), allocates the outputs with torch::empty on the states' device, and calls
// the C ABI on the current HIP stream.  Nothing here synchronises, so the operations
// can be captured in HIP graphs.
#include <torch/extension.h>

// PyTorch-ROCm keeps torch's device type "cuda" for HIP devices; these are its native
// HIP guard and stream accessors for that device type.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "../../include/cugo_hip.h"

namespace {

void check_1d(const torch::Tensor& t, at::ScalarType dtype, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.dim() == 1, name, " must be one-dimensional");
  TORCH_CHECK(t.scalar_type() == dtype, name, " has the wrong dtype");
}

void check_states(const torch::Tensor& s) {
  TORCH_CHECK(s.is_cuda(), "states must be a CUDA tensor");
  TORCH_CHECK(s.is_contiguous(), "states must be contiguous");
  TORCH_CHECK(s.scalar_type() == at::kByte, "states must have dtype torch.uint8");
  TORCH_CHECK(s.dim() == 2, "states must have shape [N, STATE_BYTES]");
  TORCH_CHECK(s.size(1) == CUGO_STATE_BYTES, "states second dimension must equal STATE_BYTES");
  TORCH_CHECK(reinterpret_cast<std::uintptr_t>(s.data_ptr()) % 8 == 0,
              "states must be 8-byte aligned");
}

void check_same_device(const torch::Tensor& a, const torch::Tensor& b, const char* an,
                       const char* bn) {
  TORCH_CHECK(a.device() == b.device(), an, " and ", bn, " must be on the same CUDA device");
}

void check_call(int rc, const char* op) {
  TORCH_CHECK(rc == 0, "cugo_hip ", op, " failed with code ", rc);
}

hipStream_t stream() { return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(); }

using DeviceGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

torch::TensorOptions on(const torch::Tensor& t, at::ScalarType dtype) {
  return torch::TensorOptions().device(t.device()).dtype(dtype);
}

std::vector<torch::Tensor> observation_outputs(int64_t n, const torch::Tensor& like) {
  return {torch::empty({n, CUGO_FEATURE_COUNT}, on(like, at::kFloat)),
          torch::empty({n, CUGO_ACTION_COUNT}, on(like, at::kBool)),
          torch::empty({n}, on(like, at::kByte)), torch::empty({n}, on(like, at::kBool)),
          torch::empty({n}, on(like, at::kShort))};
}

// `out` if given (a contiguous tensor of `dtype` and `shape` on like's device: a caller's
// buffer the kernel writes into), else a new tensor.
torch::Tensor out_or_new(const c10::optional<torch::Tensor>& out, std::vector<int64_t> shape,
                         at::ScalarType dtype, const torch::Tensor& like, const char* name) {
  if (!out.has_value()) return torch::empty(shape, on(like, dtype));
  TORCH_CHECK(out->is_contiguous() && out->scalar_type() == dtype &&
                  out->sizes() == at::IntArrayRef(shape),
              name, " must be a contiguous ", c10::toString(dtype), " tensor of shape ", shape);
  check_same_device(like, *out, "input", name);
  return *out;
}

std::vector<torch::Tensor> step_outputs(int64_t n, const torch::Tensor& like) {
  return {torch::empty({n}, on(like, at::kFloat)), torch::empty({n}, on(like, at::kBool)),
          torch::empty({n}, on(like, at::kBool)), torch::empty({n}, on(like, at::kShort)),
          torch::empty({n}, on(like, at::kBool))};
}

uint8_t* u8p(const torch::Tensor& t) { return reinterpret_cast<uint8_t*>(t.data_ptr()); }

torch::Tensor create(torch::Tensor seeds, torch::Tensor first) {
  check_1d(seeds, at::kLong, "seeds");
  check_1d(first, at::kLong, "first_players");
  TORCH_CHECK(seeds.numel() == first.numel(),
              "seeds and first_players must have the same length");
  check_same_device(seeds, first, "seeds", "first_players");
  const DeviceGuard guard(seeds.device());
  const int64_t n = seeds.numel();
  auto states = torch::empty({n, CUGO_STATE_BYTES}, on(seeds, at::kByte));
  check_call(cugo_create(seeds.data_ptr<int64_t>(), first.data_ptr<int64_t>(), n, u8p(states),
                         stream()),
             "create");
  return states;
}

std::vector<torch::Tensor> observe(torch::Tensor states) {
  check_states(states);
  const DeviceGuard guard(states.device());
  const int64_t n = states.size(0);
  auto o = observation_outputs(n, states);
  check_call(cugo_observe(u8p(states), n, o[0].data_ptr<float>(), u8p(o[1]), u8p(o[2]),
                          u8p(o[3]), o[4].data_ptr<int16_t>(), stream()),
             "observe");
  return o;
}

// observe with the features written rounded to bfloat16 into `features` (a contiguous
// bf16 [N, 720] tensor, e.g. a row block of a rollout buffer): (features, legal, player,
// done, status), features equal to observe's rounded as torch rounds float32 to bfloat16;
// with a sampler, also observe_sample's draw (actions last).
std::vector<torch::Tensor> observe_bf16(torch::Tensor states, torch::Tensor features,
                                        c10::optional<torch::Tensor> sampler,
                                        c10::optional<torch::Tensor> legal) {
  check_states(states);
  const int64_t n = states.size(0);
  TORCH_CHECK(features.is_contiguous() && features.scalar_type() == at::kBFloat16 &&
                  features.dim() == 2 && features.size(0) == n &&
                  features.size(1) == CUGO_FEATURE_COUNT,
              "features must be a contiguous bfloat16 [N, 720] tensor");
  check_same_device(states, features, "states", "features");
  if (sampler.has_value()) {
    check_1d(*sampler, at::kLong, "sampler");
    TORCH_CHECK(sampler->numel() == n, "sampler must have one entry per state row");
    check_same_device(states, *sampler, "states", "sampler");
  }
  const DeviceGuard guard(states.device());
  std::vector<torch::Tensor> o{features,
                               out_or_new(legal, {n, CUGO_ACTION_COUNT}, at::kBool, states, "legal"),
                               torch::empty({n}, on(states, at::kByte)),
                               torch::empty({n}, on(states, at::kBool)),
                               torch::empty({n}, on(states, at::kShort))};
  if (sampler.has_value()) o.push_back(torch::empty({n}, on(states, at::kLong)));
  check_call(cugo_observe_bf16(
                 u8p(states), n, reinterpret_cast<uint16_t*>(features.data_ptr()), u8p(o[1]),
                 u8p(o[2]), u8p(o[3]), o[4].data_ptr<int16_t>(),
                 sampler.has_value() ? reinterpret_cast<uint64_t*>(sampler->data_ptr()) : nullptr,
                 sampler.has_value() ? o[5].data_ptr<int64_t>() : nullptr, stream()),
             "observe_bf16");
  return o;
}

// observe plus sample_uniform's draw in one launch: (features, legal, player, done,
// status, actions); sampler advances in place as sample_uniform advances it.
std::vector<torch::Tensor> observe_sample(torch::Tensor states, torch::Tensor sampler) {
  check_states(states);
  const int64_t n = states.size(0);
  check_1d(sampler, at::kLong, "sampler");
  TORCH_CHECK(sampler.numel() == n, "sampler must have one entry per state row");
  check_same_device(states, sampler, "states", "sampler");
  const DeviceGuard guard(states.device());
  auto o = observation_outputs(n, states);
  o.push_back(torch::empty({n}, on(states, at::kLong)));
  check_call(cugo_observe_sample(u8p(states), n, o[0].data_ptr<float>(), u8p(o[1]), u8p(o[2]),
                                 u8p(o[3]), o[4].data_ptr<int16_t>(),
                                 reinterpret_cast<uint64_t*>(sampler.data_ptr()),
                                 o[5].data_ptr<int64_t>(), stream()),
             "observe_sample");
  return o;
}

std::vector<torch::Tensor> observe_indexed(torch::Tensor states, torch::Tensor ids) {
  check_states(states);
  check_1d(ids, at::kLong, "env_ids");
  check_same_device(states, ids, "states", "env_ids");
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto o = observation_outputs(n, states);
  check_call(cugo_observe_indexed(u8p(states), states.size(0), ids.data_ptr<int64_t>(), n,
                                  o[0].data_ptr<float>(), u8p(o[1]), u8p(o[2]), u8p(o[3]),
                                  o[4].data_ptr<int16_t>(), stream()),
             "observe_indexed");
  return o;
}

std::vector<torch::Tensor> step(torch::Tensor states, torch::Tensor actions) {
  check_states(states);
  check_1d(actions, at::kLong, "actions");
  TORCH_CHECK(states.size(0) == actions.numel(),
              "states and actions must have the same batch size");
  check_same_device(states, actions, "states", "actions");
  const DeviceGuard guard(states.device());
  const int64_t n = states.size(0);
  auto o = step_outputs(n, states);
  check_call(cugo_step(u8p(states), actions.data_ptr<int64_t>(), n, o[0].data_ptr<float>(),
                       u8p(o[1]), u8p(o[2]), o[3].data_ptr<int16_t>(), u8p(o[4]), stream()),
             "step");
  return o;
}

void check_indexed_actions(const torch::Tensor& states, const torch::Tensor& ids,
                           const torch::Tensor& actions) {
  check_states(states);
  check_1d(ids, at::kLong, "env_ids");
  check_1d(actions, at::kLong, "actions");
  TORCH_CHECK(ids.numel() == actions.numel(), "env_ids and actions must have the same length");
  check_same_device(states, ids, "states", "env_ids");
  check_same_device(states, actions, "states", "actions");
}

std::vector<torch::Tensor> step_indexed(torch::Tensor states, torch::Tensor ids,
                                        torch::Tensor actions) {
  check_indexed_actions(states, ids, actions);
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto o = step_outputs(n, states);
  check_call(cugo_step_indexed(u8p(states), states.size(0), ids.data_ptr<int64_t>(),
                               actions.data_ptr<int64_t>(), n, o[0].data_ptr<float>(),
                               u8p(o[1]), u8p(o[2]), o[3].data_ptr<int16_t>(), u8p(o[4]),
                               stream()),
             "step_indexed");
  return o;
}

std::vector<torch::Tensor> step_events_indexed(torch::Tensor states, torch::Tensor ids,
                                               torch::Tensor actions) {
  check_indexed_actions(states, ids, actions);
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto o = step_outputs(n, states);
  auto events = torch::empty({n, CUGO_EVENT_WORDS}, on(states, at::kLong));
  check_call(cugo_step_events_indexed(u8p(states), states.size(0), ids.data_ptr<int64_t>(),
                                      actions.data_ptr<int64_t>(), n, o[0].data_ptr<float>(),
                                      u8p(o[1]), u8p(o[2]), o[3].data_ptr<int16_t>(), u8p(o[4]),
                                      events.data_ptr<int64_t>(), stream()),
             "step_events_indexed");
  o.push_back(events);
  return o;
}

torch::Tensor start(torch::Tensor states) {
  check_states(states);
  const DeviceGuard guard(states.device());
  const int64_t n = states.size(0);
  auto out = torch::empty({n, CUGO_START_WORDS}, on(states, at::kLong));
  check_call(cugo_start(u8p(states), n, out.data_ptr<int64_t>(), stream()), "start");
  return out;
}

torch::Tensor clone_indexed(torch::Tensor states, torch::Tensor ids) {
  check_states(states);
  check_1d(ids, at::kLong, "env_ids");
  check_same_device(states, ids, "states", "env_ids");
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto children = torch::empty({n, CUGO_STATE_BYTES}, on(states, at::kByte));
  check_call(cugo_clone_indexed(u8p(states), states.size(0), ids.data_ptr<int64_t>(), n,
                                u8p(children), stream()),
             "clone_indexed");
  return children;
}

std::vector<torch::Tensor> branch_indexed(torch::Tensor states, torch::Tensor ids,
                                          torch::Tensor actions) {
  check_indexed_actions(states, ids, actions);
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto children = torch::empty({n, CUGO_STATE_BYTES}, on(states, at::kByte));
  auto o = step_outputs(n, states);
  check_call(cugo_branch_indexed(u8p(states), states.size(0), ids.data_ptr<int64_t>(),
                                 actions.data_ptr<int64_t>(), n, u8p(children),
                                 o[0].data_ptr<float>(), u8p(o[1]), u8p(o[2]),
                                 o[3].data_ptr<int16_t>(), u8p(o[4]), stream()),
             "branch_indexed");
  return {children, o[0], o[1], o[2], o[3], o[4]};
}

torch::Tensor hands_indexed(torch::Tensor states, torch::Tensor ids) {
  check_states(states);
  check_1d(ids, at::kLong, "env_ids");
  check_same_device(states, ids, "states", "env_ids");
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto hands = torch::empty({n, 2}, on(states, at::kLong));
  check_call(cugo_hands_indexed(u8p(states), states.size(0), ids.data_ptr<int64_t>(), n,
                                hands.data_ptr<int64_t>(), stream()),
             "hands_indexed");
  return hands;
}

torch::Tensor stock_indexed(torch::Tensor states, torch::Tensor ids) {
  check_states(states);
  check_1d(ids, at::kLong, "env_ids");
  check_same_device(states, ids, "states", "env_ids");
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto stock = torch::empty({n}, on(states, at::kLong));
  check_call(cugo_stock_indexed(u8p(states), states.size(0), ids.data_ptr<int64_t>(), n,
                                stock.data_ptr<int64_t>(), stream()),
             "stock_indexed");
  return stock;
}

// Random-policy driver operations (not in the reference module; used by the
// throughput harness).  sampler: uint64 [N] (int64 tensor), generation: int32 [N],
// completed: int64 [1] counter, or None (generation then counts finished games).
unsigned long long* counter_ptr(const c10::optional<torch::Tensor>& completed,
                                const torch::Tensor& states) {
  if (!completed.has_value()) return nullptr;
  check_1d(*completed, at::kLong, "completed");
  TORCH_CHECK(completed->numel() >= 1, "completed must hold one counter");
  check_same_device(states, *completed, "states", "completed");
  return reinterpret_cast<unsigned long long*>(completed->data_ptr());
}

torch::Tensor sample_uniform(torch::Tensor legal, torch::Tensor sampler) {
  TORCH_CHECK(legal.is_cuda() && legal.is_contiguous() && legal.dim() == 2 &&
                  legal.size(1) == CUGO_ACTION_COUNT && legal.scalar_type() == at::kBool,
              "legal must be a contiguous CUDA bool [N, ACTION_COUNT] tensor");
  check_1d(sampler, at::kLong, "sampler");
  TORCH_CHECK(sampler.numel() == legal.size(0), "sampler and legal must have the same length");
  check_same_device(legal, sampler, "legal", "sampler");
  const DeviceGuard guard(legal.device());
  const int64_t n = legal.size(0);
  auto actions = torch::empty({n}, on(legal, at::kLong));
  check_call(cugo_sample_uniform(u8p(legal), n, reinterpret_cast<uint64_t*>(sampler.data_ptr()),
                                 actions.data_ptr<int64_t>(), stream()),
             "sample_uniform");
  return actions;
}

void reset_done(torch::Tensor states, torch::Tensor done, int64_t base_seed,
                torch::Tensor generation, torch::Tensor sampler,
                c10::optional<torch::Tensor> completed) {
  check_states(states);
  const int64_t n = states.size(0);
  check_1d(done, at::kBool, "done");
  check_1d(generation, at::kInt, "generation");
  check_1d(sampler, at::kLong, "sampler");
  TORCH_CHECK(done.numel() == n && generation.numel() == n && sampler.numel() == n,
              "done, generation and sampler must have one entry per state row");
  const DeviceGuard guard(states.device());
  check_call(cugo_reset_done(u8p(states), u8p(done), n, static_cast<uint64_t>(base_seed),
                             reinterpret_cast<uint32_t*>(generation.data_ptr()),
                             reinterpret_cast<uint64_t*>(sampler.data_ptr()),
                             counter_ptr(completed, states), stream()),
             "reset_done");
}

// Spare slots per row: spares holds S * n rows (S = 1, 2 or 4) and spare_gen S * n entries,
// slot-major (the C ABI's cugo_refill_spares layout).
int64_t spare_slots(const torch::Tensor& spares, const torch::Tensor& spare_gen, int64_t n) {
  const int64_t rows = spares.size(0);
  const int64_t s = n > 0 ? rows / n : 1;
  TORCH_CHECK(n > 0 ? rows == s * n && (s == 1 || s == 2 || s == 4) : rows == 0,
              "spares must hold 1, 2 or 4 rows per game row");
  TORCH_CHECK(spare_gen.numel() == rows, "spare_gen must have one entry per spare row");
  return s;
}

void refill_spares(torch::Tensor spares, torch::Tensor spare_gen, torch::Tensor generation,
                   int64_t base_seed, int64_t seed_stride) {
  check_states(spares);
  check_1d(spare_gen, at::kInt, "spare_gen");
  check_1d(generation, at::kInt, "generation");
  const int64_t n = generation.numel();
  const int64_t slots = spare_slots(spares, spare_gen, n);
  const DeviceGuard guard(spares.device());
  check_call(cugo_refill_spares(u8p(spares), reinterpret_cast<uint32_t*>(spare_gen.data_ptr()),
                                reinterpret_cast<const uint32_t*>(generation.data_ptr()), n,
                                static_cast<uint64_t>(base_seed),
                                seed_stride < 0 ? n : seed_stride, slots, stream()),
             "refill_spares");
}

void reset_done_spares(torch::Tensor states, torch::Tensor done, int64_t base_seed,
                       torch::Tensor generation, torch::Tensor sampler,
                       c10::optional<torch::Tensor> completed, torch::Tensor spares,
                       torch::Tensor spare_gen, int64_t seed_stride) {
  check_states(states);
  check_states(spares);
  const int64_t n = states.size(0);
  check_1d(done, at::kBool, "done");
  check_1d(generation, at::kInt, "generation");
  check_1d(sampler, at::kLong, "sampler");
  check_1d(spare_gen, at::kInt, "spare_gen");
  TORCH_CHECK(done.numel() == n && generation.numel() == n && sampler.numel() == n,
              "done, generation and sampler must have one entry per row");
  const int64_t slots = spare_slots(spares, spare_gen, n);
  const DeviceGuard guard(states.device());
  check_call(cugo_reset_done_spares(
                 u8p(states), u8p(done), n, static_cast<uint64_t>(base_seed),
                 seed_stride < 0 ? n : seed_stride,
                 reinterpret_cast<uint32_t*>(generation.data_ptr()),
                 reinterpret_cast<uint64_t*>(sampler.data_ptr()),
                 counter_ptr(completed, states), u8p(spares),
                 reinterpret_cast<const uint32_t*>(spare_gen.data_ptr()), slots, stream()),
             "reset_done_spares");
}

// branch_indexed then observe_indexed of the children in one launch: (children, reward,
// done, nagari, status, committed, features, legal, player, obs_done, obs_status).
std::vector<torch::Tensor> branch_observe_indexed(torch::Tensor states, torch::Tensor ids,
                                                  torch::Tensor actions) {
  check_indexed_actions(states, ids, actions);
  const DeviceGuard guard(states.device());
  const int64_t n = ids.numel();
  auto children = torch::empty({n, CUGO_STATE_BYTES}, on(states, at::kByte));
  auto st = step_outputs(n, states);
  auto ob = observation_outputs(n, states);
  check_call(cugo_branch_observe_indexed(
                 u8p(states), states.size(0), ids.data_ptr<int64_t>(),
                 actions.data_ptr<int64_t>(), n, u8p(children), st[0].data_ptr<float>(),
                 u8p(st[1]), u8p(st[2]), st[3].data_ptr<int16_t>(), u8p(st[4]),
                 ob[0].data_ptr<float>(), u8p(ob[1]), u8p(ob[2]), u8p(ob[3]),
                 ob[4].data_ptr<int16_t>(), stream()),
             "branch_observe_indexed");
  std::vector<torch::Tensor> out{children};
  out.insert(out.end(), st.begin(), st.end());
  out.insert(out.end(), ob.begin(), ob.end());
  return out;
}

// rollout_canonical(seeds, first_players, max_actions=128) -> int64 [N, 5] digest words of
// the canonical whole-game driver (torch50.h:598-619).
torch::Tensor rollout_canonical(torch::Tensor seeds, torch::Tensor first, int64_t max_actions) {
  check_1d(seeds, at::kLong, "seeds");
  check_1d(first, at::kLong, "first_players");
  TORCH_CHECK(seeds.numel() == first.numel(), "seeds and first_players must have the same length");
  check_same_device(seeds, first, "seeds", "first_players");
  TORCH_CHECK(max_actions >= 0 && max_actions <= 0xFFFF, "max_actions must lie in [0, 65535]");
  const DeviceGuard guard(seeds.device());
  const int64_t n = seeds.numel();
  auto out = torch::empty({n, 5}, on(seeds, at::kLong));
  check_call(cugo_rollout_canonical(seeds.data_ptr<int64_t>(), first.data_ptr<int64_t>(), n,
                                    max_actions, out.data_ptr<int64_t>(), stream()),
             "rollout_canonical");
  return out;
}

// `steps` x (observe_sample then step_reset_spares) in one launch, the last step's
// (features, legal, player, done, status, actions, reward, step done, nagari, step status,
// committed); with record=True every step's, each output [steps, n, ...].
std::vector<torch::Tensor> play_random(torch::Tensor states, torch::Tensor sampler,
                                       int64_t base_seed, torch::Tensor generation,
                                       torch::Tensor spares, torch::Tensor spare_gen,
                                       int64_t seed_stride, int64_t steps, bool record) {
  check_states(states);
  check_states(spares);
  TORCH_CHECK(steps >= 1 && steps <= (1 << 20), "steps must lie in [1, 2^20]");
  const int64_t n = states.size(0);
  check_1d(sampler, at::kLong, "sampler");
  check_1d(generation, at::kInt, "generation");
  check_1d(spare_gen, at::kInt, "spare_gen");
  TORCH_CHECK(sampler.numel() == n && generation.numel() == n,
              "sampler and generation must have one entry per row");
  const int64_t slots = spare_slots(spares, spare_gen, n);
  check_same_device(states, sampler, "states", "sampler");
  check_same_device(states, generation, "states", "generation");
  check_same_device(states, spares, "states", "spares");
  check_same_device(states, spare_gen, "states", "spare_gen");
  const DeviceGuard guard(states.device());
  // Recorded: `steps` blocks of step_rows rows (n rounded up to 4: a block's mask bytes
  // start 4-byte aligned), returned as [steps, n, ...] views.
  const int64_t step_rows = record ? (n + 3) / 4 * 4 : 0;
  const int64_t rows = record ? steps * step_rows : n;
  auto o = observation_outputs(rows, states);
  o.push_back(torch::empty({rows}, on(states, at::kLong)));
  auto st = step_outputs(rows, states);
  o.insert(o.end(), st.begin(), st.end());
  uint64_t* smp = reinterpret_cast<uint64_t*>(sampler.data_ptr());
  uint32_t* gen = reinterpret_cast<uint32_t*>(generation.data_ptr());
  const uint32_t* sg = reinterpret_cast<const uint32_t*>(spare_gen.data_ptr());
  const int64_t stride = seed_stride < 0 ? n : seed_stride;
  if (record) {
    check_call(cugo_play_random_record(
                   u8p(states), n, smp, o[0].data_ptr<float>(), u8p(o[1]), u8p(o[2]),
                   u8p(o[3]), o[4].data_ptr<int16_t>(), o[5].data_ptr<int64_t>(),
                   o[6].data_ptr<float>(), u8p(o[7]), u8p(o[8]), o[9].data_ptr<int16_t>(),
                   u8p(o[10]), static_cast<uint64_t>(base_seed), stride, gen, u8p(spares), sg,
                   slots, steps, step_rows, stream()),
               "play_random");
    for (auto& t : o) {
      std::vector<int64_t> shape{steps, step_rows};
      for (int64_t d = 1; d < t.dim(); ++d) shape.push_back(t.size(d));
      t = t.view(shape).narrow(1, 0, n);
    }
    return o;
  }
  check_call(cugo_play_random(u8p(states), n, smp, o[0].data_ptr<float>(), u8p(o[1]),
                              u8p(o[2]), u8p(o[3]), o[4].data_ptr<int16_t>(),
                              o[5].data_ptr<int64_t>(), o[6].data_ptr<float>(), u8p(o[7]),
                              u8p(o[8]), o[9].data_ptr<int16_t>(), u8p(o[10]),
                              static_cast<uint64_t>(base_seed), stride, gen, u8p(spares), sg,
                              slots, steps, stream()),
             "play_random");
  return o;
}

// step then reset_done_spares (completed=None) in one launch; returns the step outputs.
std::vector<torch::Tensor> step_reset_spares(torch::Tensor states, torch::Tensor actions,
                                             int64_t base_seed, torch::Tensor generation,
                                             torch::Tensor sampler, torch::Tensor spares,
                                             torch::Tensor spare_gen, int64_t seed_stride,
                                             c10::optional<torch::Tensor> reward,
                                             c10::optional<torch::Tensor> done) {
  check_states(states);
  check_states(spares);
  const int64_t n = states.size(0);
  check_1d(actions, at::kLong, "actions");
  check_1d(generation, at::kInt, "generation");
  check_1d(sampler, at::kLong, "sampler");
  check_1d(spare_gen, at::kInt, "spare_gen");
  TORCH_CHECK(actions.numel() == n && generation.numel() == n && sampler.numel() == n,
              "actions, generation and sampler must have one entry per row");
  const int64_t slots = spare_slots(spares, spare_gen, n);
  check_same_device(states, actions, "states", "actions");
  check_same_device(states, generation, "states", "generation");
  check_same_device(states, sampler, "states", "sampler");
  check_same_device(states, spares, "states", "spares");
  check_same_device(states, spare_gen, "states", "spare_gen");
  const DeviceGuard guard(states.device());
  auto o = step_outputs(n, states);
  if (reward.has_value()) o[0] = out_or_new(reward, {n}, at::kFloat, states, "reward");
  if (done.has_value()) o[1] = out_or_new(done, {n}, at::kBool, states, "done");
  check_call(cugo_step_reset_spares(
                 u8p(states), actions.data_ptr<int64_t>(), n, o[0].data_ptr<float>(), u8p(o[1]),
                 u8p(o[2]), o[3].data_ptr<int16_t>(), u8p(o[4]),
                 static_cast<uint64_t>(base_seed), seed_stride < 0 ? n : seed_stride,
                 reinterpret_cast<uint32_t*>(generation.data_ptr()),
                 reinterpret_cast<uint64_t*>(sampler.data_ptr()), u8p(spares),
                 reinterpret_cast<const uint32_t*>(spare_gen.data_ptr()), slots, stream()),
             "step_reset_spares");
  return o;
}

// step_reset_spares then observe (float32 features) or observe_bf16 (bfloat16) of the new
// states in one launch, the features written into `features` (a contiguous [N, 720]
// tensor, e.g. a row block of a rollout buffer); returns the step outputs then the
// observation's: (reward, done, nagari, status, committed, features, legal, player,
// obs_done, obs_status).  A stale spare is dealt into its slot before it is taken.
std::vector<torch::Tensor> step_observe_spares(torch::Tensor states, torch::Tensor actions,
                                               int64_t base_seed, torch::Tensor generation,
                                               torch::Tensor sampler, torch::Tensor spares,
                                               torch::Tensor spare_gen, torch::Tensor features,
                                               int64_t seed_stride,
                                               c10::optional<torch::Tensor> reward,
                                               c10::optional<torch::Tensor> done,
                                               c10::optional<torch::Tensor> legal) {
  check_states(states);
  check_states(spares);
  const int64_t n = states.size(0);
  check_1d(actions, at::kLong, "actions");
  check_1d(generation, at::kInt, "generation");
  check_1d(sampler, at::kLong, "sampler");
  check_1d(spare_gen, at::kInt, "spare_gen");
  TORCH_CHECK(actions.numel() == n && generation.numel() == n && sampler.numel() == n,
              "actions, generation and sampler must have one entry per row");
  const int64_t slots = spare_slots(spares, spare_gen, n);
  TORCH_CHECK(features.is_contiguous() && features.dim() == 2 && features.size(0) == n &&
                  features.size(1) == CUGO_FEATURE_COUNT &&
                  (features.scalar_type() == at::kBFloat16 ||
                   features.scalar_type() == at::kFloat),
              "features must be a contiguous float32 or bfloat16 [N, 720] tensor");
  check_same_device(states, actions, "states", "actions");
  check_same_device(states, generation, "states", "generation");
  check_same_device(states, sampler, "states", "sampler");
  check_same_device(states, spares, "states", "spares");
  check_same_device(states, spare_gen, "states", "spare_gen");
  check_same_device(states, features, "states", "features");
  const DeviceGuard guard(states.device());
  auto o = step_outputs(n, states);
  if (reward.has_value()) o[0] = out_or_new(reward, {n}, at::kFloat, states, "reward");
  if (done.has_value()) o[1] = out_or_new(done, {n}, at::kBool, states, "done");
  o.push_back(features);
  o.push_back(out_or_new(legal, {n, CUGO_ACTION_COUNT}, at::kBool, states, "legal"));
  o.push_back(torch::empty({n}, on(states, at::kByte)));
  o.push_back(torch::empty({n}, on(states, at::kBool)));
  o.push_back(torch::empty({n}, on(states, at::kShort)));
  const bool bf16 = features.scalar_type() == at::kBFloat16;
  check_call(cugo_step_observe_spares(
                 u8p(states), actions.data_ptr<int64_t>(), n, o[0].data_ptr<float>(), u8p(o[1]),
                 u8p(o[2]), o[3].data_ptr<int16_t>(), u8p(o[4]),
                 static_cast<uint64_t>(base_seed), seed_stride < 0 ? n : seed_stride,
                 reinterpret_cast<uint32_t*>(generation.data_ptr()),
                 reinterpret_cast<uint64_t*>(sampler.data_ptr()), u8p(spares),
                 reinterpret_cast<const uint32_t*>(spare_gen.data_ptr()), slots,
                 bf16 ? CUGO_DTYPE_BF16 : CUGO_DTYPE_F32, features.data_ptr(), u8p(o[6]),
                 u8p(o[7]), u8p(o[8]), o[9].data_ptr<int16_t>(), stream()),
             "step_observe_spares");
  return o;
}

// redeal(states, seat, keys, rng): in place (python/cugo_ppo50.py:122-148 given its draws).
void redeal(torch::Tensor states, torch::Tensor seat, torch::Tensor keys, torch::Tensor rng) {
  check_states(states);
  const int64_t n = states.size(0);
  check_1d(seat, at::kLong, "seat");
  check_1d(rng, at::kLong, "rng");
  TORCH_CHECK(keys.is_cuda() && keys.is_contiguous() && keys.scalar_type() == at::kFloat &&
                  keys.dim() == 2 && keys.size(0) == n && keys.size(1) == 50,
              "keys must be a contiguous CUDA float32 [n, 50] tensor");
  TORCH_CHECK(seat.numel() == n && rng.numel() == n, "seat and rng must have one entry per row");
  check_same_device(states, seat, "states", "seat");
  check_same_device(states, keys, "states", "keys");
  check_same_device(states, rng, "states", "rng");
  const DeviceGuard guard(states.device());
  check_call(cugo_redeal(u8p(states), seat.data_ptr<int64_t>(), keys.data_ptr<float>(),
                         rng.data_ptr<int64_t>(), n, stream()),
             "redeal");
}

// accept_worlds(features, legal, real_features, real_legal, missing, candidates, out) ->
// same bool [n]: one try of redeal_worlds (python/cugo_ppo50.py:151-172): candidate j is
// kept when its observation equals the real row missing[j] % R's, and then copied to
// row missing[j] of out, in place (cugo_accept_worlds).
torch::Tensor accept_worlds(torch::Tensor features, torch::Tensor legal, torch::Tensor real_features,
                            torch::Tensor real_legal, torch::Tensor missing, torch::Tensor candidates,
                            torch::Tensor out) {
  check_states(candidates);
  check_states(out);
  const int64_t n = candidates.size(0), rows = real_features.size(0);
  check_1d(missing, at::kLong, "missing");
  TORCH_CHECK(missing.numel() == n, "missing must have one entry per candidate");
  TORCH_CHECK(features.is_contiguous() && features.scalar_type() == at::kFloat &&
                  features.dim() == 2 && features.size(0) == n &&
                  features.size(1) == CUGO_FEATURE_COUNT &&
                  real_features.is_contiguous() && real_features.scalar_type() == at::kFloat &&
                  real_features.dim() == 2 && real_features.size(1) == CUGO_FEATURE_COUNT,
              "features and real_features must be contiguous float32 [*, FEATURE_COUNT] tensors");
  TORCH_CHECK(legal.is_contiguous() && legal.scalar_type() == at::kBool && legal.dim() == 2 &&
                  legal.size(0) == n && legal.size(1) == CUGO_ACTION_COUNT &&
                  real_legal.is_contiguous() && real_legal.scalar_type() == at::kBool &&
                  real_legal.dim() == 2 && real_legal.size(0) == rows &&
                  real_legal.size(1) == CUGO_ACTION_COUNT,
              "legal and real_legal must be contiguous bool [*, ACTION_COUNT] tensors");
  TORCH_CHECK(n == 0 || rows > 0, "the real rows must not be empty");
  for (const auto* t : {&features, &legal, &real_features, &real_legal, &missing, &out})
    check_same_device(candidates, *t, "candidates", "an input");
  const DeviceGuard guard(candidates.device());
  auto same = torch::empty({n}, on(candidates, at::kBool));
  check_call(cugo_accept_worlds(features.data_ptr<float>(), u8p(legal),
                                real_features.data_ptr<float>(), u8p(real_legal),
                                missing.data_ptr<int64_t>(), rows, n, u8p(candidates), u8p(out),
                                out.size(0), u8p(same), stream()),
             "accept_worlds");
  return same;
}

torch::Tensor seed_samplers(int64_t n, int64_t base_seed, torch::Tensor generation) {
  check_1d(generation, at::kInt, "generation");
  TORCH_CHECK(generation.numel() == n, "generation must have n entries");
  const DeviceGuard guard(generation.device());
  auto sampler = torch::empty({n}, on(generation, at::kLong));
  check_call(cugo_seed_samplers(n, static_cast<uint64_t>(base_seed),
                                reinterpret_cast<const uint32_t*>(generation.data_ptr()),
                                reinterpret_cast<uint64_t*>(sampler.data_ptr()), stream()),
             "seed_samplers");
  return sampler;
}

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat:
      return CUGO_DTYPE_F32;
    case at::kHalf:
      return CUGO_DTYPE_F16;
    case at::kBFloat16:
      return CUGO_DTYPE_BF16;
    default:
      TORCH_CHECK(false, "decode_attention supports float32, float16 and bfloat16, got ", t);
  }
}

// Checks shared by both decode entry points.
void check_decode(const torch::Tensor& q, const torch::Tensor& keys, const torch::Tensor& values,
                  const torch::Tensor& pos, const c10::optional<torch::Tensor>& rows) {
  TORCH_CHECK(q.is_cuda(), "q must be a CUDA tensor");
  TORCH_CHECK(q.dim() == 3, "q must have shape [n, heads, dh]");
  TORCH_CHECK(keys.dim() == 4 && values.sizes() == keys.sizes(),
              "keys and values must have the same shape [rows, heads, slots, dh]");
  TORCH_CHECK(keys.is_contiguous() && values.is_contiguous(), "keys and values must be contiguous");
  TORCH_CHECK(keys.scalar_type() == values.scalar_type(), "keys and values must have one dtype");
  TORCH_CHECK(keys.size(1) == q.size(1) && keys.size(3) == q.size(2),
              "q [n, heads, dh] does not match the cache's heads and dh");
  check_same_device(q, keys, "q", "keys");
  check_same_device(q, values, "q", "values");
  check_1d(pos, at::kLong, "pos");
  TORCH_CHECK(pos.numel() == q.size(0), "pos must have one entry per query");
  check_same_device(q, pos, "q", "pos");
  if (rows.has_value()) {
    check_1d(*rows, at::kLong, "rows");
    TORCH_CHECK(rows->numel() == q.size(0), "rows must have one entry per query");
    check_same_device(q, *rows, "q", "rows");
  }
}

// decode_attention(q, keys, values, pos, rows=None, order=None)
// (python/cugo_seq_attention50.py:43-62): q [n, heads, dh]; keys/values
// [rows, heads, slots, dh]; pos/rows int64 [n] -> [n, heads, dh] in q's dtype; `order`
// (int32 [n], a permutation of the queries, e.g. decode_order's) only changes which
// workgroups serve which queries.
// [n, heads, dh] rows read in place when each row's [heads, dh] block is contiguous (a
// column slice of a packed [n, 3 d] projection is); otherwise a contiguous copy.
torch::Tensor row_blocks(const torch::Tensor& t) {
  const bool in_place = t.stride(2) == 1 && t.stride(1) == t.size(2) &&
                        (t.size(0) <= 1 || t.stride(0) >= t.size(1) * t.size(2));
  return in_place ? t : t.contiguous();
}

int64_t block_stride(const torch::Tensor& t) {
  return t.size(0) <= 1 ? t.size(1) * t.size(2) : t.stride(0);
}

const int32_t* order_ptr(const c10::optional<torch::Tensor>& order, const torch::Tensor& q) {
  if (!order.has_value()) return nullptr;
  check_1d(*order, at::kInt, "order");
  TORCH_CHECK(order->numel() == q.size(0), "order must have one entry per query");
  check_same_device(q, *order, "q", "order");
  return order->data_ptr<int32_t>();
}

torch::Tensor decode_attention(torch::Tensor q, torch::Tensor keys, torch::Tensor values,
                               torch::Tensor pos, c10::optional<torch::Tensor> rows,
                               c10::optional<torch::Tensor> order) {
  check_decode(q, keys, values, pos, rows);
  const int32_t* ord = order_ptr(order, q);
  const DeviceGuard guard(q.device());
  q = row_blocks(q);
  auto out = torch::empty(q.sizes(), q.options());
  const int64_t dh = q.size(2);
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(dh)));
  check_call(cugo_decode_attention(dtype_code(q.scalar_type()), dtype_code(keys.scalar_type()),
                                   q.data_ptr(), block_stride(q), keys.data_ptr(),
                                   values.data_ptr(), pos.data_ptr<int64_t>(),
                                   rows.has_value() ? rows->data_ptr<int64_t>() : nullptr, ord,
                                   q.size(0), q.size(1), dh, keys.size(2), keys.size(0), scale,
                                   out.data_ptr(), stream()),
             "decode_attention");
  return out;
}

// kv_append(k_new, v_new, keys, values, pos, rows=None): the KV append of
// decode_attention_append without the attention (cugo_kv_append), in place.
void kv_append(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor keys,
               torch::Tensor values, torch::Tensor pos, c10::optional<torch::Tensor> rows) {
  check_decode(k_new, keys, values, pos, rows);
  TORCH_CHECK(v_new.sizes() == k_new.sizes(), "k_new and v_new must have one shape");
  TORCH_CHECK(k_new.scalar_type() == keys.scalar_type() && v_new.scalar_type() == keys.scalar_type(),
              "k_new and v_new must have the cache's dtype");
  check_same_device(k_new, v_new, "k_new", "v_new");
  const DeviceGuard guard(k_new.device());
  k_new = row_blocks(k_new);
  v_new = row_blocks(v_new);
  const int64_t elem = keys.element_size();
  if (block_stride(k_new) != block_stride(v_new) || (block_stride(k_new) * elem) % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(k_new.data_ptr()) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(v_new.data_ptr()) & 15u) != 0) {
    k_new = k_new.contiguous();
    v_new = v_new.contiguous();
  }
  check_call(cugo_kv_append(dtype_code(keys.scalar_type()), k_new.data_ptr(), v_new.data_ptr(),
                            block_stride(k_new), keys.data_ptr(), values.data_ptr(),
                            pos.data_ptr<int64_t>(),
                            rows.has_value() ? rows->data_ptr<int64_t>() : nullptr,
                            k_new.size(0), k_new.size(1), k_new.size(2), keys.size(2),
                            keys.size(0), stream()),
             "kv_append");
}

// decode_order(pos int64 [n], slots) -> int32 [n]: the queries longest first by
// min(pos, slots - 1) (cugo_decode_order), for decode_attention's `order`.
torch::Tensor decode_order(torch::Tensor pos, int64_t slots) {
  check_1d(pos, at::kLong, "pos");
  TORCH_CHECK(pos.is_cuda(), "pos must be a CUDA tensor");
  TORCH_CHECK(slots > 0, "slots must be positive");
  const DeviceGuard guard(pos.device());
  auto order = torch::empty({pos.numel()}, on(pos, at::kInt));
  check_call(cugo_decode_order(pos.data_ptr<int64_t>(), pos.numel(), slots,
                               order.data_ptr<int32_t>(), stream()),
             "decode_order");
  return order;
}

// decode_attention_append(q, k_new, v_new, keys, values, pos, rows=None, out=None,
// order=None): writes k_new and v_new ([n, heads, dh], cast to the cache dtype) to slot pos
// of each query's row, in place, then attends as decode_attention
// (python/cugo_seq50.py:313-320 in one launch), into `out` when given.
torch::Tensor decode_attention_append(torch::Tensor q, torch::Tensor k_new, torch::Tensor v_new,
                                      torch::Tensor keys, torch::Tensor values, torch::Tensor pos,
                                      c10::optional<torch::Tensor> rows,
                                      c10::optional<torch::Tensor> out_opt,
                                      c10::optional<torch::Tensor> order) {
  check_decode(q, keys, values, pos, rows);
  const int32_t* ord = order_ptr(order, q);
  TORCH_CHECK(k_new.sizes() == q.sizes() && v_new.sizes() == q.sizes(),
              "k_new and v_new must have q's shape [n, heads, dh]");
  check_same_device(q, k_new, "q", "k_new");
  check_same_device(q, v_new, "q", "v_new");
  const DeviceGuard guard(q.device());
  q = row_blocks(q);
  k_new = row_blocks(k_new.to(keys.scalar_type()));
  v_new = row_blocks(v_new.to(keys.scalar_type()));
  const int64_t elem = keys.element_size();
  if (block_stride(k_new) != block_stride(v_new) || (block_stride(k_new) * elem) % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(k_new.data_ptr()) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(v_new.data_ptr()) & 15u) != 0) {
    k_new = k_new.contiguous();
    v_new = v_new.contiguous();
  }
  torch::Tensor out;
  if (out_opt.has_value()) {
    out = *out_opt;
    TORCH_CHECK(out.is_contiguous() && out.sizes() == q.sizes() &&
                    out.scalar_type() == q.scalar_type(),
                "out must be a contiguous tensor of q's shape and dtype");
    check_same_device(q, out, "q", "out");
  } else {
    out = torch::empty(q.sizes(), q.options());
  }
  const int64_t dh = q.size(2);
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(dh)));
  check_call(cugo_decode_attention_append(
                 dtype_code(q.scalar_type()), dtype_code(keys.scalar_type()), q.data_ptr(),
                 block_stride(q), k_new.data_ptr(), v_new.data_ptr(), block_stride(k_new),
                 keys.data_ptr(), values.data_ptr(),
                 pos.data_ptr<int64_t>(), rows.has_value() ? rows->data_ptr<int64_t>() : nullptr,
                 ord, q.size(0), q.size(1), dh, keys.size(2), keys.size(0), scale, out.data_ptr(),
                 stream()),
             "decode_attention_append");
  return out;
}

}  // namespace

// ---------------------------------------------------------------- seq self-play ----
void check_token_weights(const torch::Tensor& weight_t, const torch::Tensor& bias,
                         const torch::Tensor& position, const torch::Tensor& token_type,
                         int64_t in_features, const torch::Tensor& like) {
  TORCH_CHECK(weight_t.is_cuda() && weight_t.is_contiguous() && weight_t.dim() == 2 &&
                  weight_t.size(0) == in_features,
              "weight_t must be a contiguous CUDA tensor [", in_features, ", d]");
  const int64_t d = weight_t.size(1);
  const auto t = weight_t.scalar_type();
  TORCH_CHECK(t == at::kBFloat16 || t == at::kFloat, "token weights must be bfloat16 or float32");
  TORCH_CHECK(bias.scalar_type() == t && position.scalar_type() == t &&
                  token_type.scalar_type() == t,
              "bias, position and token_type must have weight_t's dtype");
  TORCH_CHECK(bias.is_contiguous() && bias.numel() == d, "bias must be contiguous [d]");
  TORCH_CHECK(position.is_contiguous() && position.dim() == 2 && position.size(1) == d,
              "position must be contiguous [rows, d]");
  TORCH_CHECK(token_type.is_contiguous() && token_type.dim() == 2 && token_type.size(0) == 3 &&
                  token_type.size(1) == d,
              "token_type must be contiguous [3, d]");
  TORCH_CHECK(d == 64 || d == 128 || d == 256 || d == 512 || d == 1024,
              "d must be 64, 128, 256, 512 or 1024");
  check_same_device(like, weight_t, "words", "weight_t");
  check_same_device(like, bias, "words", "bias");
  check_same_device(like, position, "words", "position");
  check_same_device(like, token_type, "words", "token_type");
}

int token_dtype(const torch::Tensor& w) {
  return w.scalar_type() == at::kBFloat16 ? CUGO_DTYPE_BF16 : CUGO_DTYPE_F32;
}

// event_tokens(words [n, 9], seat [n], index [n], weight_t [414, d], bias, position,
// token_type, out=None) -> [n, d]: SeqNet.event_token (python/cugo_seq50.py:276-282),
// written into `out` (contiguous [n, d]) when given.
torch::Tensor event_tokens(torch::Tensor words, torch::Tensor seat, torch::Tensor index,
                           torch::Tensor weight_t, torch::Tensor bias, torch::Tensor position,
                           torch::Tensor token_type, c10::optional<torch::Tensor> out_opt,
                           c10::optional<torch::Tensor> ln_weight,
                           c10::optional<torch::Tensor> ln_bias, double eps,
                           c10::optional<torch::Tensor> ln_out) {
  TORCH_CHECK(words.is_cuda() && words.is_contiguous() && words.dim() == 2 &&
                  words.size(1) == CUGO_EVENT_WORDS && words.scalar_type() == at::kLong,
              "words must be a contiguous CUDA int64 [n, EVENT_WORDS] tensor");
  // seat names the rows; words and index may hold each event once for several seats
  const int64_t word_rows = words.size(0);
  check_1d(seat, at::kLong, "seat");
  check_1d(index, at::kLong, "index");
  const int64_t n = seat.numel();
  TORCH_CHECK(index.numel() == word_rows, "index must have one entry per event row");
  TORCH_CHECK(n == 0 || (word_rows > 0 && n % word_rows == 0),
              "the number of seats must be a multiple of the number of events");
  check_same_device(words, seat, "words", "seat");
  check_same_device(words, index, "words", "index");
  check_token_weights(weight_t, bias, position, token_type, 8 * 50 + 12 + 2, words);
  const DeviceGuard guard(words.device());
  auto out = out_or_new(out_opt, {n, weight_t.size(1)}, weight_t.scalar_type(), words, "out");
  // with ln_out: also the tokens' LayerNorm (the first layer's norm1) into ln_out
  TORCH_CHECK(ln_out.has_value() == (ln_weight.has_value() && ln_bias.has_value()),
              "ln_out goes with ln_weight and ln_bias");
  const int64_t d = weight_t.size(1);
  if (ln_out.has_value()) {
    for (const auto* t : {&*ln_weight, &*ln_bias})
      TORCH_CHECK(t->scalar_type() == weight_t.scalar_type() && t->is_contiguous() &&
                      t->numel() == d,
                  "ln_weight and ln_bias must be contiguous [d] tensors of the weights' dtype");
    TORCH_CHECK(ln_out->scalar_type() == weight_t.scalar_type() && ln_out->is_contiguous() &&
                    ln_out->dim() == 2 && ln_out->size(0) == n && ln_out->size(1) == d,
                "ln_out must be a contiguous [n, d] tensor of the weights' dtype");
    check_same_device(words, *ln_weight, "words", "ln_weight");
    check_same_device(words, *ln_bias, "words", "ln_bias");
    check_same_device(words, *ln_out, "words", "ln_out");
  }
  check_call(cugo_event_tokens(token_dtype(weight_t), words.data_ptr<int64_t>(), word_rows,
                               seat.data_ptr<int64_t>(), index.data_ptr<int64_t>(), n,
                               weight_t.data_ptr(), bias.data_ptr(), position.data_ptr(),
                               position.size(0), token_type.data_ptr(), d, out.data_ptr(),
                               ln_out.has_value() ? ln_weight->data_ptr() : nullptr,
                               ln_out.has_value() ? ln_bias->data_ptr() : nullptr,
                               static_cast<float>(eps),
                               ln_out.has_value() ? ln_out->data_ptr() : nullptr, stream()),
             "event_tokens");
  return out;
}

// start_tokens(start [n, 8], seat [n], weight_t [274, d], bias, position, token_type)
// -> [n, d]: SeqNet.start_token (python/cugo_seq50.py:271-274).
torch::Tensor start_tokens(torch::Tensor start, torch::Tensor seat, torch::Tensor weight_t,
                           torch::Tensor bias, torch::Tensor position,
                           torch::Tensor token_type) {
  TORCH_CHECK(start.is_cuda() && start.is_contiguous() && start.dim() == 2 &&
                  start.size(1) == CUGO_START_WORDS && start.scalar_type() == at::kLong,
              "start must be a contiguous CUDA int64 [n, START_WORDS] tensor");
  const int64_t n = start.size(0);
  check_1d(seat, at::kLong, "seat");
  TORCH_CHECK(seat.numel() == n, "seat must have n entries");
  check_same_device(start, seat, "start", "seat");
  check_token_weights(weight_t, bias, position, token_type, 5 * 50 + 12 + 8 + 4, start);
  const DeviceGuard guard(start.device());
  auto out = torch::empty({n, weight_t.size(1)}, on(start, weight_t.scalar_type()));
  check_call(cugo_start_tokens(token_dtype(weight_t), start.data_ptr<int64_t>(),
                               seat.data_ptr<int64_t>(), n, weight_t.data_ptr(),
                               bias.data_ptr(), position.data_ptr(), token_type.data_ptr(),
                               weight_t.size(1), out.data_ptr(), stream()),
             "start_tokens");
  return out;
}

// add_layernorm(x [n, d], y [n, d] or None, weight [d], bias [d], eps) -> (x + y, LN(x + y));
// with y None: (x, LN(x)).  The residual add and the next pre-norm of a
// TransformerEncoderLayer step (python/cugo_seq50.py:318-322) in one launch.
std::vector<torch::Tensor> add_layernorm(torch::Tensor x, c10::optional<torch::Tensor> y,
                                         torch::Tensor weight, torch::Tensor bias, double eps) {
  TORCH_CHECK(x.is_cuda() && x.is_contiguous() && x.dim() == 2,
              "x must be a contiguous CUDA [n, d] tensor");
  const auto t = x.scalar_type();
  TORCH_CHECK(t == at::kBFloat16 || t == at::kFloat, "add_layernorm supports bfloat16 and float32");
  const int64_t n = x.size(0), d = x.size(1);
  TORCH_CHECK(d == 64 || d == 128 || d == 256 || d == 512 || d == 1024,
              "d must be 64, 128, 256, 512 or 1024");
  TORCH_CHECK(weight.scalar_type() == t && bias.scalar_type() == t && weight.numel() == d &&
                  bias.numel() == d && weight.is_contiguous() && bias.is_contiguous(),
              "weight and bias must be contiguous [d] tensors of x's dtype");
  check_same_device(x, weight, "x", "weight");
  check_same_device(x, bias, "x", "bias");
  torch::Tensor yc;
  if (y.has_value()) {
    yc = y->contiguous();
    TORCH_CHECK(yc.sizes() == x.sizes() && yc.scalar_type() == t, "y must match x");
    check_same_device(x, yc, "x", "y");
  }
  const DeviceGuard guard(x.device());
  auto x_out = y.has_value() ? torch::empty_like(x) : x;
  auto ln = torch::empty_like(x);
  check_call(cugo_add_layernorm(t == at::kBFloat16 ? CUGO_DTYPE_BF16 : CUGO_DTYPE_F32,
                                x.data_ptr(), y.has_value() ? yc.data_ptr() : nullptr,
                                weight.data_ptr(), bias.data_ptr(), static_cast<float>(eps), n,
                                d, x_out.data_ptr(), ln.data_ptr(), stream()),
             "add_layernorm");
  return {x_out, ln};
}

// linear(x [m, k] bf16, w_packed, n, bias [n] bf16 or None, gelu, tile, residual [m, n] or
// None) -> y [m, n] bf16: nn.Linear (and with gelu=True the nn.GELU() after it; with a
// residual, residual + that) of the decoder step
// (python/cugo_seq50.py:291-322) in one launch.  w_packed is the layer's weight [n, k] as
// mlp_pack_weight(weight, roundup(n, 16), k) lays it out.  x may be a row-strided view
// (unit stride along k).
torch::Tensor linear(torch::Tensor x, torch::Tensor w_packed, int64_t n,
                     c10::optional<torch::Tensor> bias, bool gelu, int64_t tile,
                     c10::optional<torch::Tensor> residual, c10::optional<torch::Tensor> out) {
  TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.scalar_type() == at::kBFloat16 && x.stride(1) == 1,
              "x must be a CUDA bfloat16 [m, k] tensor with unit stride along k");
  const int64_t m = x.size(0), k = x.size(1);
  TORCH_CHECK(n > 0 && w_packed.scalar_type() == at::kBFloat16 && w_packed.is_contiguous() &&
                  w_packed.numel() == (n + 15) / 16 * 16 * k,
              "w_packed must be a contiguous bfloat16 tensor of roundup(n, 16) * k elements");
  check_same_device(x, w_packed, "x", "w_packed");
  if (bias.has_value()) {
    TORCH_CHECK(bias->scalar_type() == at::kBFloat16 && bias->is_contiguous() && bias->numel() == n,
                "bias must be a contiguous bfloat16 [n] tensor");
    check_same_device(x, *bias, "x", "bias");
  }
  int64_t ldr = 0;
  if (residual.has_value()) {
    TORCH_CHECK(residual->scalar_type() == at::kBFloat16 && residual->is_contiguous() &&
                    ((residual->dim() == 2 && residual->size(0) == m && residual->size(1) == n) ||
                     (residual->dim() == 1 && residual->size(0) == n)),
                "residual must be a contiguous bfloat16 [m, n] tensor or an [n] row for all");
    check_same_device(x, *residual, "x", "residual");
    ldr = residual->dim() == 2 ? n : 0;
  }
  const DeviceGuard guard(x.device());
  auto y = out_or_new(out, {m, n}, at::kBFloat16, x, "out");
  const int64_t ldx = m > 1 ? x.stride(0) : k;
  check_call(cugo_linear(gelu ? CUGO_LINEAR_GELU : CUGO_LINEAR_NONE, x.data_ptr(), ldx,
                         w_packed.data_ptr(), bias.has_value() ? bias->data_ptr() : nullptr,
                         residual.has_value() ? residual->data_ptr() : nullptr, ldr, m, n, k,
                         y.data_ptr(), n, static_cast<int>(tile), stream()),
             "linear");
  return y;
}

// linear_add_layernorm(x [m, k], w_packed, bias, res [m, 256], ln_weight, ln_bias, eps)
// -> (x_out, ln): linear then add_layernorm(res, y, ...) in one launch (the out_proj /
// linear2 of a pre-norm layer with the residual add and the next norm,
// python/cugo_seq50.py:316-322); all bf16.
std::vector<torch::Tensor> linear_add_layernorm(torch::Tensor x, torch::Tensor w_packed,
                                                c10::optional<torch::Tensor> bias,
                                                torch::Tensor res, torch::Tensor ln_weight,
                                                torch::Tensor ln_bias, double eps,
                                                int64_t tile, c10::optional<torch::Tensor> out,
                                                c10::optional<torch::Tensor> ln_out) {
  TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.scalar_type() == at::kBFloat16 && x.stride(1) == 1,
              "x must be a CUDA bfloat16 [m, k] tensor with unit stride along k");
  const int64_t m = x.size(0), k = x.size(1), n = 256;
  TORCH_CHECK(res.is_contiguous() && res.scalar_type() == at::kBFloat16 &&
                  ((res.dim() == 2 && res.size(0) == m && res.size(1) == n) ||
                   (res.dim() == 1 && res.size(0) == n)),
              "res must be a contiguous bfloat16 [m, 256] tensor or a [256] row for all");
  TORCH_CHECK(w_packed.scalar_type() == at::kBFloat16 && w_packed.is_contiguous() &&
                  w_packed.numel() == n * k,
              "w_packed must be the packed bfloat16 [256, k] weight");
  TORCH_CHECK(ln_weight.scalar_type() == at::kBFloat16 && ln_bias.scalar_type() == at::kBFloat16 &&
                  ln_weight.numel() == n && ln_bias.numel() == n && ln_weight.is_contiguous() &&
                  ln_bias.is_contiguous(),
              "ln_weight and ln_bias must be contiguous bfloat16 [256] tensors");
  check_same_device(x, w_packed, "x", "w_packed");
  check_same_device(x, res, "x", "res");
  check_same_device(x, ln_weight, "x", "ln_weight");
  check_same_device(x, ln_bias, "x", "ln_bias");
  if (bias.has_value()) {
    TORCH_CHECK(bias->scalar_type() == at::kBFloat16 && bias->is_contiguous() && bias->numel() == n,
                "bias must be a contiguous bfloat16 [256] tensor");
    check_same_device(x, *bias, "x", "bias");
  }
  const DeviceGuard guard(x.device());
  auto x_out = out_or_new(out, {m, n}, at::kBFloat16, x, "out");
  auto ln = out_or_new(ln_out, {m, n}, at::kBFloat16, x, "ln_out");
  const int64_t ldx = m > 1 ? x.stride(0) : k;
  check_call(cugo_linear_add_layernorm(x.data_ptr(), ldx, w_packed.data_ptr(),
                                       bias.has_value() ? bias->data_ptr() : nullptr, m, n, k,
                                       res.data_ptr(), res.dim() == 2 ? n : 0,
                                       ln_weight.data_ptr(), ln_bias.data_ptr(),
                                       static_cast<float>(eps), x_out.data_ptr(), ln.data_ptr(),
                                       static_cast<int>(tile), stream()),
             "linear_add_layernorm");
  return {x_out, ln};
}

// query_input(features f32 [n, 720], legal bool [n, 179], columns int32 [width] or None,
// q_in [n, q_stride] bf16/f32): SeqNet._query's input rows, zero-padded (cugo_query_input).
void query_input(torch::Tensor features, torch::Tensor legal, c10::optional<torch::Tensor> columns,
                 torch::Tensor q_in) {
  TORCH_CHECK(features.is_cuda() && features.is_contiguous() && features.dim() == 2 &&
                  features.size(1) == CUGO_FEATURE_COUNT && features.scalar_type() == at::kFloat,
              "features must be a contiguous CUDA float32 [n, 720] tensor");
  const int64_t n = features.size(0);
  TORCH_CHECK(legal.is_contiguous() && legal.dim() == 2 && legal.size(0) == n &&
                  legal.size(1) == CUGO_ACTION_COUNT && legal.scalar_type() == at::kBool,
              "legal must be a contiguous bool [n, 179] tensor");
  int64_t width = CUGO_FEATURE_COUNT;
  const int32_t* cols = nullptr;
  if (columns.has_value()) {
    TORCH_CHECK(columns->is_contiguous() && columns->dim() == 1 &&
                    columns->scalar_type() == at::kInt && columns->numel() >= 1 &&
                    columns->numel() <= CUGO_FEATURE_COUNT,
                "columns must be a contiguous int32 vector of at most 720 feature columns");
    check_same_device(features, *columns, "features", "columns");
    width = columns->numel();
    cols = columns->data_ptr<int32_t>();
  }
  TORCH_CHECK(q_in.is_contiguous() && q_in.dim() == 2 && q_in.size(0) == n &&
                  q_in.size(1) >= width + CUGO_ACTION_COUNT &&
                  (q_in.scalar_type() == at::kBFloat16 || q_in.scalar_type() == at::kFloat),
              "q_in must be a contiguous bfloat16 or float32 [n, >= width + 179] tensor");
  check_same_device(features, legal, "features", "legal");
  check_same_device(features, q_in, "features", "q_in");
  const DeviceGuard guard(features.device());
  check_call(cugo_query_input(q_in.scalar_type() == at::kBFloat16 ? CUGO_DTYPE_BF16 : CUGO_DTYPE_F32,
                              features.data_ptr<float>(), u8p(legal), cols, width, n,
                              q_in.data_ptr(), q_in.size(1), stream()),
             "query_input");
}

// out_proj's part of out_proj_ffn: the packed [256, 256] weight, its bias and norm2.
struct OutProj {
  const torch::Tensor* wo_packed;
  const torch::Tensor* bo;
  const torch::Tensor* ln2_weight;
  const torch::Tensor* ln2_bias;
  double eps2;
};

// The feed-forward half (cugo_ffn), or with `op` out_proj + add + norm2 before it
// (cugo_out_proj_ffn, h then being the attention output).
static std::vector<torch::Tensor> ffn_impl(torch::Tensor h, torch::Tensor x,
                                           torch::Tensor w1_packed, torch::Tensor b1,
                                           torch::Tensor w2_packed, torch::Tensor b2,
                                           c10::optional<torch::Tensor> ln_weight,
                                           c10::optional<torch::Tensor> ln_bias, double eps,
                                           int64_t rows, c10::optional<torch::Tensor> out,
                                           const OutProj* op) {
  const char* hname = op != nullptr ? "att" : "h";
  TORCH_CHECK(h.is_cuda() && h.dim() == 2 && h.size(1) == 256 && h.scalar_type() == at::kBFloat16 &&
                  h.stride(1) == 1,
              hname, " must be a CUDA bfloat16 [m, 256] tensor with unit stride along its columns");
  const int64_t m = h.size(0);
  TORCH_CHECK(x.is_contiguous() && x.dim() == 2 && x.size(0) == m && x.size(1) == 256 &&
                  x.scalar_type() == at::kBFloat16,
              "x must be a contiguous bfloat16 [m, 256] tensor");
  TORCH_CHECK(w1_packed.scalar_type() == at::kBFloat16 && w1_packed.is_contiguous() &&
                  w1_packed.numel() == 1024 * 256 && w2_packed.scalar_type() == at::kBFloat16 &&
                  w2_packed.is_contiguous() && w2_packed.numel() == 256 * 1024,
              "w1_packed and w2_packed must be the packed bfloat16 [1024, 256] and [256, 1024] "
              "weights");
  TORCH_CHECK(b1.scalar_type() == at::kBFloat16 && b1.is_contiguous() && b1.numel() == 1024 &&
                  b2.scalar_type() == at::kBFloat16 && b2.is_contiguous() && b2.numel() == 256,
              "b1 and b2 must be contiguous bfloat16 [1024] and [256] tensors");
  TORCH_CHECK(ln_weight.has_value() == ln_bias.has_value(), "ln_weight and ln_bias go together");
  for (const auto* t : {&x, &w1_packed, &b1, &w2_packed, &b2}) check_same_device(h, *t, hname, "an input");
  if (ln_weight.has_value()) {
    TORCH_CHECK(ln_weight->scalar_type() == at::kBFloat16 && ln_bias->scalar_type() == at::kBFloat16 &&
                    ln_weight->numel() == 256 && ln_bias->numel() == 256 &&
                    ln_weight->is_contiguous() && ln_bias->is_contiguous(),
                "ln_weight and ln_bias must be contiguous bfloat16 [256] tensors");
    check_same_device(h, *ln_weight, hname, "ln_weight");
    check_same_device(h, *ln_bias, hname, "ln_bias");
  }
  if (op != nullptr) {
    TORCH_CHECK(op->wo_packed->scalar_type() == at::kBFloat16 && op->wo_packed->is_contiguous() &&
                    op->wo_packed->numel() == 256 * 256,
                "wo_packed must be the packed bfloat16 [256, 256] weight");
    for (const auto* t : {op->bo, op->ln2_weight, op->ln2_bias})
      TORCH_CHECK(t->scalar_type() == at::kBFloat16 && t->is_contiguous() && t->numel() == 256,
                  "bo, ln2_weight and ln2_bias must be contiguous bfloat16 [256] tensors");
    for (const auto* t : {op->wo_packed, op->bo, op->ln2_weight, op->ln2_bias})
      check_same_device(h, *t, hname, "an input");
  }
  const DeviceGuard guard(h.device());
  auto x_out = out_or_new(out, {m, 256}, at::kBFloat16, h, "out");
  auto ln = ln_weight.has_value() ? torch::empty({m, 256}, on(h, at::kBFloat16))
                                  : torch::empty({0}, on(h, at::kBFloat16));
  const int64_t ldh = m > 1 ? h.stride(0) : 256;
  void* lw = ln_weight.has_value() ? ln_weight->data_ptr() : nullptr;
  void* lb = ln_bias.has_value() ? ln_bias->data_ptr() : nullptr;
  void* lnp = ln_weight.has_value() ? ln.data_ptr() : nullptr;
  if (op == nullptr)
    check_call(cugo_ffn(h.data_ptr(), ldh, x.data_ptr(), w1_packed.data_ptr(), b1.data_ptr(),
                        w2_packed.data_ptr(), b2.data_ptr(), lw, lb, static_cast<float>(eps), m,
                        x_out.data_ptr(), lnp, static_cast<int>(rows), stream()),
               "ffn");
  else
    check_call(cugo_out_proj_ffn(h.data_ptr(), ldh, x.data_ptr(), op->wo_packed->data_ptr(),
                                 op->bo->data_ptr(), op->ln2_weight->data_ptr(),
                                 op->ln2_bias->data_ptr(), static_cast<float>(op->eps2),
                                 w1_packed.data_ptr(), b1.data_ptr(), w2_packed.data_ptr(),
                                 b2.data_ptr(), lw, lb, static_cast<float>(eps), m,
                                 x_out.data_ptr(), lnp, static_cast<int>(rows), stream()),
               "out_proj_ffn");
  return {x_out, ln};
}

// ffn(h [m, 256], x [m, 256], w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, eps, rows,
// out) -> (x_out, ln): the feed-forward half of a pre-norm layer with the residual add and
// the next norm (python/cugo_seq50.py:319-322) in one launch (cugo_ffn); without
// ln_weight, ln is an empty tensor and x_out = x + linear2(GELU(linear1(h))).  `out`, if
// given, receives x_out (it may be x).
std::vector<torch::Tensor> ffn(torch::Tensor h, torch::Tensor x, torch::Tensor w1_packed,
                               torch::Tensor b1, torch::Tensor w2_packed, torch::Tensor b2,
                               c10::optional<torch::Tensor> ln_weight,
                               c10::optional<torch::Tensor> ln_bias, double eps, int64_t rows,
                               c10::optional<torch::Tensor> out) {
  return ffn_impl(h, x, w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, eps, rows, out,
                  nullptr);
}

// out_proj_ffn(att [m, 256], x [m, 256], wo_packed, bo, ln2_weight, ln2_bias, eps2,
// w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, eps, rows, out) -> (x_out, ln): the
// layer after its attention (python/cugo_seq50.py:317-322) in one launch
// (cugo_out_proj_ffn): x1 = x + out_proj(att), h = norm2(x1), x_out = x1 +
// linear2(GELU(linear1(h))), ln = the next norm of x_out (empty without ln_weight).
std::vector<torch::Tensor> out_proj_ffn(torch::Tensor att, torch::Tensor x,
                                        torch::Tensor wo_packed, torch::Tensor bo,
                                        torch::Tensor ln2_weight, torch::Tensor ln2_bias,
                                        double eps2, torch::Tensor w1_packed, torch::Tensor b1,
                                        torch::Tensor w2_packed, torch::Tensor b2,
                                        c10::optional<torch::Tensor> ln_weight,
                                        c10::optional<torch::Tensor> ln_bias, double eps,
                                        int64_t rows, c10::optional<torch::Tensor> out) {
  const OutProj op{&wo_packed, &bo, &ln2_weight, &ln2_bias, eps2};
  return ffn_impl(att, x, w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, eps, rows, out, &op);
}

// paired_select(active, status, done, any_legal, player, a_seat, act_a, act_b, bad,
// any_active, playing=None) -> actions int64 [n]; paired_update(active, step_status,
// new_done, reward0, nagari, final_reward0, final_nagari, bad, any_active, steps,
// playing=None): the bookkeeping of a resident paired-evaluation step (cugo_paired_select
// / cugo_paired_update); `playing` (int32 [1]) ends a step at 1 while a game is active.
namespace {
void check_n(const torch::Tensor& t, int64_t n, at::ScalarType dt, const char* name) {
  TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.numel() == n && t.scalar_type() == dt,
              name, " must be a contiguous CUDA ", c10::toString(dt), " tensor of ", n,
              " elements");
}
}  // namespace

int32_t* playing_ptr(const c10::optional<torch::Tensor>& playing, const torch::Tensor& like) {
  if (!playing.has_value()) return nullptr;
  check_n(*playing, 1, at::kInt, "playing");
  check_same_device(like, *playing, "active", "playing");
  return playing->data_ptr<int32_t>();
}

torch::Tensor paired_select(torch::Tensor active, torch::Tensor status, torch::Tensor done,
                            torch::Tensor any_legal, torch::Tensor player, torch::Tensor a_seat,
                            torch::Tensor act_a, torch::Tensor act_b, torch::Tensor bad,
                            torch::Tensor any_active, c10::optional<torch::Tensor> playing) {
  const int64_t n = active.numel();
  check_n(active, n, at::kBool, "active");
  check_n(status, n, at::kShort, "status");
  check_n(done, n, at::kBool, "done");
  check_n(any_legal, n, at::kBool, "any_legal");
  check_n(player, n, at::kByte, "player");
  check_n(a_seat, n, at::kLong, "a_seat");
  check_n(act_a, n, at::kLong, "act_a");
  check_n(act_b, n, at::kLong, "act_b");
  check_n(bad, 3, at::kLong, "bad");
  check_n(any_active, 1, at::kInt, "any_active");
  for (const auto* t : {&status, &done, &any_legal, &player, &a_seat, &act_a, &act_b, &bad,
                        &any_active})
    check_same_device(active, *t, "active", "an input");
  const DeviceGuard guard(active.device());
  auto actions = torch::empty({n}, on(active, at::kLong));
  check_call(cugo_paired_select(u8p(active), status.data_ptr<int16_t>(), u8p(done), u8p(any_legal),
                                u8p(player), a_seat.data_ptr<int64_t>(), act_a.data_ptr<int64_t>(),
                                act_b.data_ptr<int64_t>(), n, actions.data_ptr<int64_t>(),
                                bad.data_ptr<int64_t>(), any_active.data_ptr<int32_t>(),
                                playing_ptr(playing, active), stream()),
             "paired_select");
  return actions;
}

void paired_update(torch::Tensor active, torch::Tensor step_status, torch::Tensor new_done,
                   torch::Tensor reward0, torch::Tensor nagari, torch::Tensor final_reward0,
                   torch::Tensor final_nagari, torch::Tensor bad, torch::Tensor any_active,
                   torch::Tensor steps, c10::optional<torch::Tensor> playing) {
  const int64_t n = active.numel();
  check_n(active, n, at::kBool, "active");
  check_n(step_status, n, at::kShort, "step_status");
  check_n(new_done, n, at::kBool, "new_done");
  check_n(reward0, n, at::kFloat, "reward0");
  check_n(nagari, n, at::kBool, "nagari");
  check_n(final_reward0, n, at::kFloat, "final_reward0");
  check_n(final_nagari, n, at::kBool, "final_nagari");
  check_n(bad, 3, at::kLong, "bad");
  check_n(any_active, 1, at::kInt, "any_active");
  check_n(steps, 1, at::kLong, "steps");
  for (const auto* t : {&step_status, &new_done, &reward0, &nagari, &final_reward0,
                        &final_nagari, &bad, &any_active, &steps})
    check_same_device(active, *t, "active", "an input");
  const DeviceGuard guard(active.device());
  check_call(cugo_paired_update(u8p(active), step_status.data_ptr<int16_t>(), u8p(new_done),
                                reward0.data_ptr<float>(), u8p(nagari), n,
                                final_reward0.data_ptr<float>(), u8p(final_nagari),
                                bad.data_ptr<int64_t>(), any_active.data_ptr<int32_t>(),
                                steps.data_ptr<int64_t>(), playing_ptr(playing, active),
                                stream()),
             "paired_update");
}

// store_probe(out uint8, rows, row_bytes, steps, distinct): the calibration launch
// cugo_store_probe (play_random's observation-row stores without the game) into `out`.
void store_probe(torch::Tensor out, int64_t rows, int64_t row_bytes, int64_t steps,
                 bool distinct) {
  TORCH_CHECK(out.is_cuda() && out.is_contiguous() && out.scalar_type() == at::kByte,
              "out must be a contiguous CUDA uint8 tensor");
  TORCH_CHECK(rows >= 0 && rows % 64 == 0 && row_bytes > 0 && row_bytes % 16 == 0 &&
                  steps >= 0,
              "rows must be a multiple of 64 and row_bytes a multiple of 16");
  TORCH_CHECK(out.numel() >= rows * row_bytes * (distinct ? steps : 1),
              "out is smaller than the rows the probe writes");
  TORCH_CHECK(reinterpret_cast<uintptr_t>(out.data_ptr()) % 16 == 0, "out must be 16-byte aligned");
  const DeviceGuard guard(out.device());
  check_call(cugo_store_probe(out.data_ptr(), rows, row_bytes, steps, distinct ? 1 : 0,
                              stream()),
             "store_probe");
}

// paired_events(active, step_status, committed, new_done, count, length_a, event_pos_a,
// query_pos_a, length_b, event_pos_b, query_pos_b): the event bookkeeping of a paired
// evaluation of sequence policies (cugo_paired_events): a kept event's slot (or -1) into
// event_pos_*, the next query's slot (or -1) into query_pos_*, and the counts and cache
// paired_movers(player uint8 [n], seat int64 [n], query_pos int64 [n]): query_pos = -1
// where the mover is not in `seat` (cugo_paired_movers).
void paired_movers(torch::Tensor player, torch::Tensor seat, torch::Tensor query_pos) {
  check_1d(player, at::kByte, "player");
  check_1d(seat, at::kLong, "seat");
  check_1d(query_pos, at::kLong, "query_pos");
  const int64_t n = player.numel();
  TORCH_CHECK(seat.numel() == n && query_pos.numel() == n,
              "player, seat and query_pos must have one entry per game");
  check_same_device(player, seat, "player", "seat");
  check_same_device(player, query_pos, "player", "query_pos");
  const DeviceGuard guard(player.device());
  check_call(cugo_paired_movers(player.data_ptr<uint8_t>(), seat.data_ptr<int64_t>(), n,
                                query_pos.data_ptr<int64_t>(), stream()),
             "paired_movers");
}

// lengths advanced.
void paired_events(torch::Tensor active, torch::Tensor step_status, torch::Tensor committed,
                   torch::Tensor new_done, torch::Tensor count, torch::Tensor length_a,
                   torch::Tensor event_pos_a, torch::Tensor query_pos_a,
                   c10::optional<torch::Tensor> length_b, c10::optional<torch::Tensor> event_pos_b,
                   c10::optional<torch::Tensor> query_pos_b) {
  const int64_t n = active.numel();
  check_n(active, n, at::kBool, "active");
  check_n(step_status, n, at::kShort, "step_status");
  check_n(committed, n, at::kBool, "committed");
  check_n(new_done, n, at::kBool, "new_done");
  check_n(count, n, at::kLong, "count");
  check_n(length_a, n, at::kLong, "length_a");
  check_n(event_pos_a, n, at::kLong, "event_pos_a");
  check_n(query_pos_a, n, at::kLong, "query_pos_a");
  for (const auto* t : {&step_status, &committed, &new_done, &count, &length_a, &event_pos_a,
                        &query_pos_a})
    check_same_device(active, *t, "active", "an input");
  TORCH_CHECK(length_b.has_value() == event_pos_b.has_value() &&
                  length_b.has_value() == query_pos_b.has_value(),
              "length_b, event_pos_b and query_pos_b go together");
  int64_t* lb = nullptr;
  int64_t* pb = nullptr;
  int64_t* qb = nullptr;
  if (length_b.has_value()) {
    check_n(*length_b, n, at::kLong, "length_b");
    check_n(*event_pos_b, n, at::kLong, "event_pos_b");
    check_n(*query_pos_b, n, at::kLong, "query_pos_b");
    check_same_device(active, *length_b, "active", "length_b");
    check_same_device(active, *event_pos_b, "active", "event_pos_b");
    check_same_device(active, *query_pos_b, "active", "query_pos_b");
    lb = length_b->data_ptr<int64_t>();
    pb = event_pos_b->data_ptr<int64_t>();
    qb = query_pos_b->data_ptr<int64_t>();
  }
  const DeviceGuard guard(active.device());
  check_call(cugo_paired_events(u8p(active), step_status.data_ptr<int16_t>(), u8p(committed),
                                u8p(new_done), n, count.data_ptr<int64_t>(),
                                length_a.data_ptr<int64_t>(), event_pos_a.data_ptr<int64_t>(),
                                query_pos_a.data_ptr<int64_t>(), lb, pb, qb, stream()),
             "paired_events");
}

// masked_argmax(logits [n, A] f32/bf16, legal bool [n, A]) -> int64 [n]: the greedy
// action of python/cugo_eval50.py:125-127 (argmax of logits.float() masked with -1e30).
torch::Tensor masked_argmax(torch::Tensor logits, torch::Tensor legal) {
  TORCH_CHECK(logits.is_cuda() && logits.is_contiguous() && logits.dim() == 2 &&
                  (logits.scalar_type() == at::kFloat || logits.scalar_type() == at::kBFloat16),
              "logits must be a contiguous CUDA float32 or bfloat16 [n, A] tensor");
  TORCH_CHECK(legal.is_contiguous() && legal.sizes() == logits.sizes() &&
                  legal.scalar_type() == at::kBool,
              "legal must be a contiguous bool tensor shaped like logits");
  check_same_device(logits, legal, "logits", "legal");
  const DeviceGuard guard(logits.device());
  auto actions = torch::empty({logits.size(0)}, on(logits, at::kLong));
  check_call(cugo_gumbel_sample(logits.scalar_type() == at::kFloat ? CUGO_DTYPE_F32 : CUGO_DTYPE_BF16,
                                logits.data_ptr(), u8p(legal), nullptr, logits.size(0),
                                logits.size(1), actions.data_ptr<int64_t>(), nullptr, stream()),
             "masked_argmax");
  return actions;
}

// gumbel_sample(logits f32 [n, A], legal bool [n, A], uniforms f32 [n, A]) -> (actions
// int64 [n], logp f32 [n]): the sampling of WaveCollector._step
// (python/cugo_seq_selfplay50.py:125-130) with the uniforms supplied.
std::vector<torch::Tensor> gumbel_sample(torch::Tensor logits, torch::Tensor legal,
                                         torch::Tensor uniforms,
                                         c10::optional<torch::Tensor> actions_out,
                                         c10::optional<torch::Tensor> logp_out) {
  TORCH_CHECK(logits.is_cuda() && logits.is_contiguous() && logits.dim() == 2 &&
                  (logits.scalar_type() == at::kFloat || logits.scalar_type() == at::kBFloat16),
              "logits must be a contiguous CUDA float32 or bfloat16 [n, A] tensor");
  TORCH_CHECK(legal.is_contiguous() && legal.sizes() == logits.sizes() &&
                  legal.scalar_type() == at::kBool,
              "legal must be a contiguous bool tensor shaped like logits");
  TORCH_CHECK(uniforms.is_contiguous() && uniforms.sizes() == logits.sizes() &&
                  uniforms.scalar_type() == at::kFloat,
              "uniforms must be a contiguous float32 tensor shaped like logits");
  check_same_device(logits, legal, "logits", "legal");
  check_same_device(logits, uniforms, "logits", "uniforms");
  const DeviceGuard guard(logits.device());
  const int64_t n = logits.size(0);
  auto actions = out_or_new(actions_out, {n}, at::kLong, logits, "actions");
  auto logp = out_or_new(logp_out, {n}, at::kFloat, logits, "logp");
  check_call(cugo_gumbel_sample(logits.scalar_type() == at::kFloat ? CUGO_DTYPE_F32 : CUGO_DTYPE_BF16,
                                logits.data_ptr(), u8p(legal), uniforms.data_ptr<float>(),
                                n, logits.size(1), actions.data_ptr<int64_t>(),
                                logp.data_ptr<float>(), stream()),
             "gumbel_sample");
  return {actions, logp};
}

// gumbel_sample_philox(logits f32 or bf16 [n, A], legal bool [n, A], seed, epoch int64 [1]
// (device), offset) -> (actions int64 [n], logp f32 [n]): gumbel_sample with uniforms drawn
// in the kernel from Philox4x32-10 (cugo_gumbel_sample_philox); uniforms_out, if given,
// receives them.
std::vector<torch::Tensor> gumbel_sample_philox(torch::Tensor logits, torch::Tensor legal,
                                                int64_t seed, torch::Tensor epoch,
                                                int64_t offset,
                                                c10::optional<torch::Tensor> actions_out,
                                                c10::optional<torch::Tensor> logp_out,
                                                c10::optional<torch::Tensor> uniforms_out) {
  TORCH_CHECK(logits.is_cuda() && logits.is_contiguous() && logits.dim() == 2 &&
                  (logits.scalar_type() == at::kFloat || logits.scalar_type() == at::kBFloat16),
              "logits must be a contiguous CUDA float32 or bfloat16 [n, A] tensor");
  TORCH_CHECK(legal.is_contiguous() && legal.sizes() == logits.sizes() &&
                  legal.scalar_type() == at::kBool,
              "legal must be a contiguous bool tensor shaped like logits");
  TORCH_CHECK(logits.size(1) <= 192, "at most 192 actions");
  TORCH_CHECK(epoch.numel() == 1 && epoch.scalar_type() == at::kLong,
              "epoch must be a one-element int64 tensor");
  TORCH_CHECK(offset >= 0 && offset <= 0xFFFFFFFFll, "offset must fit 32 bits");
  check_same_device(logits, legal, "logits", "legal");
  check_same_device(logits, epoch, "logits", "epoch");
  const DeviceGuard guard(logits.device());
  const int64_t n = logits.size(0);
  auto actions = out_or_new(actions_out, {n}, at::kLong, logits, "actions");
  auto logp = out_or_new(logp_out, {n}, at::kFloat, logits, "logp");
  float* u = nullptr;
  if (uniforms_out.has_value()) {
    TORCH_CHECK(uniforms_out->is_contiguous() && uniforms_out->sizes() == logits.sizes() &&
                    uniforms_out->scalar_type() == at::kFloat,
                "uniforms_out must be a contiguous float32 tensor shaped like logits");
    check_same_device(logits, *uniforms_out, "logits", "uniforms_out");
    u = uniforms_out->data_ptr<float>();
  }
  check_call(cugo_gumbel_sample_philox(
                 logits.scalar_type() == at::kFloat ? CUGO_DTYPE_F32 : CUGO_DTYPE_BF16,
                 logits.data_ptr(), u8p(legal), static_cast<uint64_t>(seed),
                 reinterpret_cast<const uint64_t*>(epoch.data_ptr()), (uint32_t)offset, n,
                 logits.size(1), actions.data_ptr<int64_t>(), logp.data_ptr<float>(), u,
                 stream()),
             "gumbel_sample_philox");
  return {actions, logp};
}

// mlp_pack_weight(w bf16 [rows, cols], rows_pad, cols_pad) -> packed bf16 [rows_pad *
// cols_pad]: w in the order the actor kernel reads its MFMA operands
// (cugo_mlp_pack_weight).
torch::Tensor mlp_pack_weight(torch::Tensor w, int64_t rows_pad, int64_t cols_pad) {
  TORCH_CHECK(w.is_cuda() && w.is_contiguous() && w.dim() == 2 &&
                  w.scalar_type() == at::kBFloat16,
              "w must be a contiguous CUDA bfloat16 [rows, cols] tensor");
  TORCH_CHECK(w.size(0) <= rows_pad && w.size(1) <= cols_pad && rows_pad % 16 == 0 &&
                  cols_pad % 32 == 0,
              "rows_pad (a multiple of 16) and cols_pad (of 32) must cover w");
  const DeviceGuard guard(w.device());
  auto packed = torch::empty({rows_pad * cols_pad}, on(w, at::kBFloat16));
  check_call(cugo_mlp_pack_weight(w.data_ptr(), w.size(0), w.size(1), rows_pad, cols_pad,
                                  packed.data_ptr(), stream()),
             "mlp_pack_weight");
  return packed;
}

// mlp_actor_forward(x [n, F] f32 or bf16, x_copy bf16 [n, F] or None, packed weights and
// bf16 vectors, actions, eps) -> (logits bf16 [n, actions], value f32 [n]): the residual
// MLP actor's forward pass in one launch (cugo_mlp_actor_forward).  ln_w / ln_b hold the
// blocks' LayerNorms then the final one; w_in, w1, w2 and w_head come from
// mlp_pack_weight (w_head: the logits weight with the value weight as its last row).
std::vector<torch::Tensor> mlp_actor_forward(
    torch::Tensor x, c10::optional<torch::Tensor> x_copy, torch::Tensor w_in,
    torch::Tensor b_in, std::vector<torch::Tensor> ln_w, std::vector<torch::Tensor> ln_b,
    std::vector<torch::Tensor> w1, std::vector<torch::Tensor> b1, std::vector<torch::Tensor> w2,
    std::vector<torch::Tensor> b2, torch::Tensor w_head, torch::Tensor b_head, int64_t actions,
    double eps, c10::optional<torch::Tensor> value_out) {
  TORCH_CHECK(x.is_cuda() && x.is_contiguous() && x.dim() == 2 &&
                  (x.scalar_type() == at::kFloat || x.scalar_type() == at::kBFloat16),
              "x must be a contiguous CUDA float32 or bfloat16 [n, F] tensor");
  const int64_t n = x.size(0), f = x.size(1);
  const int64_t blocks = static_cast<int64_t>(w1.size());
  TORCH_CHECK(blocks <= CUGO_MLP_MAX_BLOCKS, "at most ", CUGO_MLP_MAX_BLOCKS, " blocks");
  TORCH_CHECK(b1.size() == w1.size() && w2.size() == w1.size() && b2.size() == w1.size() &&
                  ln_w.size() == w1.size() + 1 && ln_b.size() == w1.size() + 1,
              "one fc1, fc2 and LayerNorm per block and a final LayerNorm");
  const int64_t d = b_in.dim() == 1 ? b_in.size(0) : -1;
  auto check_w = [&](const torch::Tensor& t, std::vector<int64_t> shape, const char* name) {
    TORCH_CHECK(t.is_cuda() && t.is_contiguous() && t.scalar_type() == at::kBFloat16 &&
                    t.sizes() == at::IntArrayRef(shape),
                name, " must be a contiguous CUDA bfloat16 tensor of shape ", shape);
    check_same_device(x, t, "x", name);
  };
  check_w(w_in, {d * CUGO_MLP_MAX_FEATURES}, "w_in (packed)");
  check_w(b_in, {d}, "b_in");
  for (int64_t b = 0; b <= blocks; ++b) {
    check_w(ln_w[b], {d}, "ln_w");
    check_w(ln_b[b], {d}, "ln_b");
  }
  for (int64_t b = 0; b < blocks; ++b) {
    check_w(w1[b], {d * d}, "w1 (packed)");
    check_w(b1[b], {d}, "b1");
    check_w(w2[b], {d * d}, "w2 (packed)");
    check_w(b2[b], {d}, "b2");
  }
  check_w(w_head, {CUGO_MLP_HEAD_ROWS * d}, "w_head (packed)");
  check_w(b_head, {actions + 1}, "b_head");
  if (x_copy.has_value()) {
    TORCH_CHECK(x_copy->is_contiguous() && x_copy->scalar_type() == at::kBFloat16 &&
                    x_copy->sizes() == x.sizes(),
                "x_copy must be a contiguous bfloat16 tensor shaped like x");
    check_same_device(x, *x_copy, "x", "x_copy");
  }
  CugoMlpWeights w{};
  w.hidden = static_cast<int>(d);
  w.blocks = static_cast<int>(blocks);
  w.features = static_cast<int>(f);
  w.actions = static_cast<int>(actions);
  w.eps = static_cast<float>(eps);
  w.w_in = w_in.data_ptr();
  w.b_in = b_in.data_ptr();
  for (int64_t b = 0; b <= blocks; ++b) {
    w.ln_w[b] = ln_w[b].data_ptr();
    w.ln_b[b] = ln_b[b].data_ptr();
  }
  for (int64_t b = 0; b < blocks; ++b) {
    w.w1[b] = w1[b].data_ptr();
    w.b1[b] = b1[b].data_ptr();
    w.w2[b] = w2[b].data_ptr();
    w.b2[b] = b2[b].data_ptr();
  }
  w.w_head = w_head.data_ptr();
  w.b_head = b_head.data_ptr();
  const DeviceGuard guard(x.device());
  auto logits = torch::empty({n, actions}, on(x, at::kBFloat16));
  auto value = out_or_new(value_out, {n}, at::kFloat, x, "value");
  const int rc = cugo_mlp_actor_forward(
      x.scalar_type() == at::kFloat ? CUGO_DTYPE_F32 : CUGO_DTYPE_BF16, x.data_ptr(),
      x_copy.has_value() ? x_copy->data_ptr() : nullptr, n, &w, logits.data_ptr(),
      value.data_ptr<float>(), stream());
  TORCH_CHECK(rc != -3, "mlp_actor_forward: unsupported shape (hidden 512, at most ",
              CUGO_MLP_MAX_BLOCKS, " blocks, features a multiple of 8 up to ",
              CUGO_MLP_MAX_FEATURES, ", at most ", CUGO_MLP_HEAD_ROWS - 1, " actions)");
  check_call(rc, "mlp_actor_forward");
  return {logits, value};
}

// The tensors of one self-play wave, held for the wave's life, and the step's two
// bookkeeping launches (cugo_selfplay_prepare / _advance).
class SelfPlayState {
 public:
  SelfPlayState(int64_t w, int64_t max_steps, torch::Tensor step_index, torch::Tensor count,
                torch::Tensor events, torch::Tensor cache_length, torch::Tensor final_reward0,
                torch::Tensor final_nagari, torch::Tensor finished, torch::Tensor bad,
                torch::Tensor rec_features, torch::Tensor rec_legal, torch::Tensor rec_logp,
                torch::Tensor rec_actions, torch::Tensor rec_opp_hand, torch::Tensor rec_stock,
                torch::Tensor rec_stop_points, torch::Tensor rec_seat, torch::Tensor rec_count,
                torch::Tensor rec_valid, c10::optional<torch::Tensor> columns,
                int64_t pool_games, torch::Tensor learner_seat,
                c10::optional<torch::Tensor> opp_cache_length)
      : keep_{step_index, count, events, cache_length, final_reward0, final_nagari, finished,
              bad, rec_features, rec_legal, rec_logp, rec_actions, rec_opp_hand, rec_stock,
              rec_stop_points, rec_seat, rec_count, rec_valid, learner_seat} {
    TORCH_CHECK(w >= 0 && max_steps >= 0, "w and max_steps must be non-negative");
    TORCH_CHECK(pool_games >= 0 && pool_games <= w, "pool_games must be in [0, w]");
    int64_t width = CUGO_FEATURE_COUNT;
    const int32_t* cols = nullptr;
    if (columns.has_value()) {
      const auto c = *columns;
      TORCH_CHECK(c.is_cuda() && c.is_contiguous() && c.scalar_type() == at::kInt &&
                      c.dim() == 1 && c.numel() >= 1 && c.numel() <= CUGO_FEATURE_COUNT,
                  "columns must be a contiguous CUDA int32 [width] tensor");
      const auto host = c.cpu();
      const int32_t* v = host.data_ptr<int32_t>();
      for (int64_t j = 0; j < host.numel(); ++j)
        TORCH_CHECK(v[j] >= 0 && v[j] < CUGO_FEATURE_COUNT, "a feature column is out of range");
      width = c.numel();
      cols = c.data_ptr<int32_t>();
      keep_.push_back(c);
    }
    int64_t* opp_len = nullptr;
    if (pool_games > 0) {
      TORCH_CHECK(opp_cache_length.has_value(), "a pool needs the opponent's cache lengths");
      const auto o = *opp_cache_length;
      TORCH_CHECK(o.is_cuda() && o.is_contiguous() && o.scalar_type() == at::kLong &&
                      o.numel() >= pool_games,
                  "the opponent's cache lengths must be int64 with one entry per pool game");
      opp_len = o.data_ptr<int64_t>();
      keep_.push_back(o);
    }
    const auto dev = count.device();
    for (const auto& t : keep_)
      TORCH_CHECK(t.is_cuda() && t.device() == dev && t.is_contiguous(),
                  "self-play tensors must be contiguous and on one CUDA device");
    auto want = [](const torch::Tensor& t, at::ScalarType type, std::vector<int64_t> shape,
                   const char* name) {
      TORCH_CHECK(t.scalar_type() == type && t.sizes().vec() == shape, name,
                  " has the wrong dtype or shape");
    };
    const int64_t s = max_steps;
    want(step_index, at::kLong, {2}, "step_index");
    want(count, at::kLong, {w}, "count");
    want(events, at::kLong, {w, 48, CUGO_EVENT_WORDS}, "events");
    want(cache_length, at::kLong, {2 * w}, "cache length");
    want(final_reward0, at::kFloat, {w}, "final_reward0");
    want(final_nagari, at::kBool, {w}, "final_nagari");
    want(finished, at::kBool, {w}, "finished");
    TORCH_CHECK(bad.scalar_type() == at::kLong && bad.numel() == 1, "bad must be one int64");
    want(rec_features, at::kBFloat16, {s, w, width}, "rec_features");
    want(learner_seat, at::kLong, {w}, "learner_seat");
    want(rec_legal, at::kBool, {s, w, CUGO_ACTION_COUNT}, "rec_legal");
    want(rec_logp, at::kFloat, {s, w}, "rec_logp");
    want(rec_valid, at::kBool, {s, w}, "rec_valid");
    for (const auto* t : {&rec_actions, &rec_opp_hand, &rec_stock, &rec_stop_points, &rec_seat,
                          &rec_count})
      want(*t, at::kLong, {s, w}, "a recorded int64 field");
    auto l = [](const torch::Tensor& t) { return t.data_ptr<int64_t>(); };
    c_ = CugoSelfPlayWave{w,
                          max_steps,
                          width,
                          cols,
                          pool_games,
                          learner_seat.data_ptr<int64_t>(),
                          opp_len,
                          l(step_index),
                          l(count),
                          l(events),
                          l(cache_length),
                          final_reward0.data_ptr<float>(),
                          u8p(final_nagari),
                          u8p(finished),
                          reinterpret_cast<unsigned long long*>(bad.data_ptr()),
                          reinterpret_cast<uint16_t*>(rec_features.data_ptr()),
                          u8p(rec_legal),
                          rec_logp.data_ptr<float>(),
                          l(rec_actions),
                          l(rec_opp_hand),
                          l(rec_stock),
                          l(rec_stop_points),
                          l(rec_seat),
                          l(rec_count),
                          u8p(rec_valid)};
  }

  // -> (q_in [w, q_stride or width + 179] of q_dtype, query_rows int64 [w], query_pos int64
  // [w] = the cache length of each query row); with q_stride > 0 the columns past
  // width + 179 are zeros (a padded query input)
  std::vector<torch::Tensor> prepare(torch::Tensor states, torch::Tensor features,
                                     torch::Tensor legal, torch::Tensor player,
                                     torch::Tensor done, torch::Tensor status,
                                     c10::optional<torch::Tensor> stock,
                                     at::ScalarType q_dtype, int64_t q_stride) {
    const int64_t w = c_.w;
    check_states(states);
    TORCH_CHECK(states.size(0) == w, "states must hold the wave's w rows");
    TORCH_CHECK(features.is_contiguous() && features.scalar_type() == at::kFloat &&
                    features.sizes() == torch::IntArrayRef({w, CUGO_FEATURE_COUNT}),
                "features must be float32 [w, FEATURE_COUNT]");
    TORCH_CHECK(legal.is_contiguous() && legal.scalar_type() == at::kBool &&
                    legal.sizes() == torch::IntArrayRef({w, CUGO_ACTION_COUNT}),
                "legal must be bool [w, ACTION_COUNT]");
    TORCH_CHECK(player.numel() == w && done.numel() == w && status.numel() == w &&
                    player.scalar_type() == at::kByte && done.scalar_type() == at::kBool &&
                    status.scalar_type() == at::kShort,
                "player/done/status must be observe's [w] outputs");
    TORCH_CHECK(!stock.has_value() ||
                    (stock->numel() == w && stock->scalar_type() == at::kLong &&
                     stock->is_contiguous() && stock->device() == keep_[0].device()),
                "stock must be stock_indexed's [w] output");
    TORCH_CHECK(q_dtype == at::kBFloat16 || q_dtype == at::kFloat,
                "the query dtype must be bfloat16 or float32");
    for (const auto* t : {&states, &features, &legal, &player, &done, &status})
      TORCH_CHECK(t->device() == keep_[0].device(), "inputs must be on the wave's device");
    const DeviceGuard guard(states.device());
    TORCH_CHECK(q_stride == 0 || q_stride >= c_.width + CUGO_ACTION_COUNT,
                "q_stride must be 0 or at least width + ACTION_COUNT");
    c_.q_stride = q_stride;
    auto q_in = torch::empty({w, q_stride > 0 ? q_stride : c_.width + CUGO_ACTION_COUNT},
                             on(states, q_dtype));
    auto rows = torch::empty({w}, on(states, at::kLong));
    auto pos = torch::empty({w}, on(states, at::kLong));
    c_.query_pos = pos.data_ptr<int64_t>();
    check_call(cugo_selfplay_prepare(&c_, q_dtype == at::kBFloat16 ? CUGO_DTYPE_BF16 : CUGO_DTYPE_F32,
                                     u8p(states), features.data_ptr<float>(), u8p(legal),
                                     u8p(player), u8p(done), status.data_ptr<int16_t>(),
                                     stock.has_value() ? stock->data_ptr<int64_t>() : nullptr,
                                     q_in.data_ptr(),
                                     rows.data_ptr<int64_t>(), stream()),
               "selfplay_prepare");
    return {q_in, rows, pos};
  }

  // The counter every advance raises by one (the Philox noise epoch of the next step).
  void set_noise_epoch(torch::Tensor epoch) {
    TORCH_CHECK(epoch.numel() == 1 && epoch.scalar_type() == at::kLong && epoch.is_cuda() &&
                    epoch.device() == keep_[0].device(),
                "epoch must be a one-element int64 tensor on the wave's device");
    keep_.push_back(epoch);
    c_.noise_epoch = reinterpret_cast<uint64_t*>(epoch.data_ptr());
  }

  // The flag every prepare clears and every advance sets while a game is still played.
  void set_playing(torch::Tensor playing) {
    TORCH_CHECK(playing.numel() == 1 && playing.scalar_type() == at::kInt && playing.is_cuda() &&
                    playing.device() == keep_[0].device(),
                "playing must be a one-element int32 tensor on the wave's device");
    keep_.push_back(playing);
    c_.playing = playing.data_ptr<int32_t>();
  }

  // Where every advance writes each cache row's length before the step's events count.
  void set_event_pos(torch::Tensor event_pos) {
    TORCH_CHECK(event_pos.numel() == 2 * c_.w && event_pos.scalar_type() == at::kLong &&
                    event_pos.is_contiguous() && event_pos.device() == keep_[0].device(),
                "event_pos must be a contiguous int64 [2 w] tensor on the wave's device");
    keep_.push_back(event_pos);
    c_.event_pos = event_pos.data_ptr<int64_t>();
  }

  void advance(torch::Tensor done, torch::Tensor reward0, torch::Tensor new_done,
               torch::Tensor nagari, torch::Tensor step_status, torch::Tensor committed,
               torch::Tensor events, torch::Tensor actions, torch::Tensor logp) {
    const int64_t w = c_.w;
    TORCH_CHECK(done.numel() == w && reward0.numel() == w && new_done.numel() == w &&
                    nagari.numel() == w && step_status.numel() == w && committed.numel() == w &&
                    actions.numel() == w && logp.numel() == w,
                "step outputs must have one entry per game");
    TORCH_CHECK(done.scalar_type() == at::kBool && reward0.scalar_type() == at::kFloat &&
                    new_done.scalar_type() == at::kBool && nagari.scalar_type() == at::kBool &&
                    step_status.scalar_type() == at::kShort &&
                    committed.scalar_type() == at::kBool && actions.scalar_type() == at::kLong &&
                    logp.scalar_type() == at::kFloat,
                "step outputs have the wrong dtypes");
    TORCH_CHECK(events.is_contiguous() && events.scalar_type() == at::kLong &&
                    events.sizes() == torch::IntArrayRef({w, CUGO_EVENT_WORDS}),
                "events must be int64 [w, EVENT_WORDS]");
    for (const auto* t : {&done, &reward0, &new_done, &nagari, &step_status, &committed,
                          &actions, &logp})
      TORCH_CHECK(t->is_contiguous() && t->device() == keep_[0].device(),
                  "step outputs must be contiguous on the wave's device");
    const DeviceGuard guard(done.device());
    check_call(cugo_selfplay_advance(&c_, u8p(done), reward0.data_ptr<float>(), u8p(new_done),
                                     u8p(nagari), step_status.data_ptr<int16_t>(),
                                     u8p(committed), events.data_ptr<int64_t>(),
                                     actions.data_ptr<int64_t>(), logp.data_ptr<float>(),
                                     stream()),
               "selfplay_advance");
  }

 private:
  std::vector<torch::Tensor> keep_;
  CugoSelfPlayWave c_{};
};

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Cugo Shin Matgo batch environment on gfx950 (HIP)";
  m.def("create", &create, "Create a GPU-resident batch of 248-byte game rows");
  m.def("observe", &observe, "Encode features and legal masks on the current stream");
  m.def("observe_indexed", &observe_indexed, "Encode only selected rows");
  m.def("step", &step, "Apply unified actions to every row in place");
  m.def("step_indexed", &step_indexed, "Apply unified actions to selected rows in place");
  m.def("clone_indexed", &clone_indexed, "Clone selected rows");
  m.def("branch_indexed", &branch_indexed, "Clone selected rows and step the clones");
  m.def("hands_indexed", &hands_indexed, "[N, 2] int64 hand masks of both players");
  m.def("stock_indexed", &stock_indexed, "[N] int64: the next 8 stock draws, one per byte");
  m.def("step_events_indexed", &step_events_indexed,
        "step_indexed plus [N, EVENT_WORDS] int64 event records");
  m.def("start", &start, "[N, START_WORDS] int64 opening records");
  m.def("sample_uniform", &sample_uniform, "Uniform legal action per row (xorshift64)");
  m.def("observe_sample", &observe_sample,
        "observe plus sample_uniform's draw: (features, legal, player, done, status, actions)");
  m.def("reset_done", &reset_done, "Re-create finished rows with their next seed",
        pybind11::arg("states"), pybind11::arg("done"), pybind11::arg("base_seed"),
        pybind11::arg("generation"), pybind11::arg("sampler"),
        pybind11::arg("completed") = pybind11::none());
  m.def("seed_samplers", &seed_samplers, "Per-row sampler state from the row seeds");
  m.def("redeal", &redeal, "Redeal the observer's opponent hand and the stock, in place");
  m.def("refill_spares", &refill_spares, "Pre-deal the next game of rows with a stale spare",
        pybind11::arg("spares"), pybind11::arg("spare_gen"), pybind11::arg("generation"),
        pybind11::arg("base_seed"), pybind11::arg("seed_stride") = -1);
  m.def("reset_done_spares", &reset_done_spares,
        "reset_done, taking each finished row's next game from its pre-dealt spare",
        pybind11::arg("states"), pybind11::arg("done"), pybind11::arg("base_seed"),
        pybind11::arg("generation"), pybind11::arg("sampler"), pybind11::arg("completed"),
        pybind11::arg("spares"), pybind11::arg("spare_gen"), pybind11::arg("seed_stride") = -1);
  m.def("branch_observe_indexed", &branch_observe_indexed,
        "branch_indexed then observe_indexed of the children, in one launch");
  m.def("play_random", &play_random,
        "steps x (observe_sample then step_reset_spares) in one launch; last step's outputs",
        pybind11::arg("states"), pybind11::arg("sampler"), pybind11::arg("base_seed"),
        pybind11::arg("generation"), pybind11::arg("spares"), pybind11::arg("spare_gen"),
        pybind11::arg("seed_stride") = -1, pybind11::arg("steps") = 1,
        pybind11::arg("record") = false);
  m.def("rollout_canonical", &rollout_canonical,
        "Canonical whole-game rollouts (rollout_canonical_torch50): [N, 5] digest words",
        pybind11::arg("seeds"), pybind11::arg("first_players"),
        pybind11::arg("max_actions") = 128);
  m.def("step_reset_spares", &step_reset_spares,
        "step, then reset_done_spares of the finished rows, in one launch",
        pybind11::arg("states"), pybind11::arg("actions"), pybind11::arg("base_seed"),
        pybind11::arg("generation"), pybind11::arg("sampler"), pybind11::arg("spares"),
        pybind11::arg("spare_gen"), pybind11::arg("seed_stride") = -1,
        pybind11::arg("reward") = pybind11::none(), pybind11::arg("done") = pybind11::none());
  m.def("step_observe_spares", &step_observe_spares,
        "step_reset_spares, then observe (float32 or bfloat16 features, into `features`) of the "
        "new states, in one launch",
        pybind11::arg("states"), pybind11::arg("actions"), pybind11::arg("base_seed"),
        pybind11::arg("generation"), pybind11::arg("sampler"), pybind11::arg("spares"),
        pybind11::arg("spare_gen"), pybind11::arg("features"), pybind11::arg("seed_stride") = -1,
        pybind11::arg("reward") = pybind11::none(), pybind11::arg("done") = pybind11::none(),
        pybind11::arg("legal") = pybind11::none());
  m.def("gumbel_sample_philox", &gumbel_sample_philox,
        "gumbel_sample with uniforms drawn in the kernel from Philox4x32-10",
        pybind11::arg("logits"), pybind11::arg("legal"), pybind11::arg("seed"),
        pybind11::arg("epoch"), pybind11::arg("offset"), pybind11::arg("actions") = pybind11::none(),
        pybind11::arg("logp") = pybind11::none(), pybind11::arg("uniforms_out") = pybind11::none());
  m.def("event_tokens", &event_tokens, "SeqNet.event_token: event_in(encode_events) + position + type",
        pybind11::arg("words"), pybind11::arg("seat"), pybind11::arg("index"),
        pybind11::arg("weight_t"), pybind11::arg("bias"), pybind11::arg("position"),
        pybind11::arg("token_type"), pybind11::arg("out") = pybind11::none(),
        pybind11::arg("ln_weight") = pybind11::none(), pybind11::arg("ln_bias") = pybind11::none(),
        pybind11::arg("eps") = 1e-5, pybind11::arg("ln_out") = pybind11::none());
  m.def("start_tokens", &start_tokens, "SeqNet.start_token: start_in(encode_start) + position + type");
  m.def("add_layernorm", &add_layernorm, "x + y and LayerNorm(x + y) in one launch",
        pybind11::arg("x"), pybind11::arg("y"), pybind11::arg("weight"), pybind11::arg("bias"),
        pybind11::arg("eps"));
  m.def("linear", &linear, "bf16 x weight^T + bias, optionally followed by GELU, in one launch",
        pybind11::arg("x"), pybind11::arg("w_packed"), pybind11::arg("n"),
        pybind11::arg("bias") = pybind11::none(), pybind11::arg("gelu") = false,
        pybind11::arg("tile") = 0, pybind11::arg("residual") = pybind11::none(),
        pybind11::arg("out") = pybind11::none());
  m.def("linear_add_layernorm", &linear_add_layernorm,
        "linear, then the residual add and LayerNorm of add_layernorm, in one launch",
        pybind11::arg("x"), pybind11::arg("w_packed"), pybind11::arg("bias"), pybind11::arg("res"),
        pybind11::arg("ln_weight"), pybind11::arg("ln_bias"), pybind11::arg("eps"),
        pybind11::arg("tile") = 0, pybind11::arg("out") = pybind11::none(),
        pybind11::arg("ln_out") = pybind11::none());
  pybind11::class_<SelfPlayState>(m, "SelfPlayState",
                                   "A self-play wave's tensors and its step bookkeeping")
      .def(pybind11::init<int64_t, int64_t, torch::Tensor, torch::Tensor, torch::Tensor,
                          torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor,
                          torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor,
                          torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor,
                          torch::Tensor, torch::Tensor, torch::Tensor,
                          c10::optional<torch::Tensor>, int64_t, torch::Tensor,
                          c10::optional<torch::Tensor>>())
      .def("prepare", &SelfPlayState::prepare, pybind11::arg("states"), pybind11::arg("features"),
           pybind11::arg("legal"), pybind11::arg("player"), pybind11::arg("done"),
           pybind11::arg("status"), pybind11::arg("stock"), pybind11::arg("q_dtype"),
           pybind11::arg("q_stride") = 0)
      .def("advance", &SelfPlayState::advance)
      .def("set_noise_epoch", &SelfPlayState::set_noise_epoch)
      .def("set_event_pos", &SelfPlayState::set_event_pos)
      .def("set_playing", &SelfPlayState::set_playing);
  m.def("query_input", &query_input, "SeqNet._query's input rows, zero-padded, into q_in",
        pybind11::arg("features"), pybind11::arg("legal"), pybind11::arg("columns"),
        pybind11::arg("q_in"));
  m.def("ffn", &ffn,
        "linear1 + GELU + linear2 + residual add (+ the next LayerNorm) in one launch",
        pybind11::arg("h"), pybind11::arg("x"), pybind11::arg("w1_packed"), pybind11::arg("b1"),
        pybind11::arg("w2_packed"), pybind11::arg("b2"),
        pybind11::arg("ln_weight") = pybind11::none(), pybind11::arg("ln_bias") = pybind11::none(),
        pybind11::arg("eps") = 1e-5, pybind11::arg("rows") = 0,
        pybind11::arg("out") = pybind11::none());
  m.def("out_proj_ffn", &out_proj_ffn,
        "out_proj + residual add + norm2, then ffn, in one launch",
        pybind11::arg("att"), pybind11::arg("x"), pybind11::arg("wo_packed"), pybind11::arg("bo"),
        pybind11::arg("ln2_weight"), pybind11::arg("ln2_bias"), pybind11::arg("eps2"),
        pybind11::arg("w1_packed"), pybind11::arg("b1"), pybind11::arg("w2_packed"),
        pybind11::arg("b2"), pybind11::arg("ln_weight") = pybind11::none(),
        pybind11::arg("ln_bias") = pybind11::none(), pybind11::arg("eps") = 1e-5,
        pybind11::arg("rows") = 0, pybind11::arg("out") = pybind11::none());
  m.def("paired_select", &paired_select,
        "paired evaluation: observe checks and each game's action from its mover's model",
        pybind11::arg("active"), pybind11::arg("status"), pybind11::arg("done"),
        pybind11::arg("any_legal"), pybind11::arg("player"), pybind11::arg("a_seat"),
        pybind11::arg("act_a"), pybind11::arg("act_b"), pybind11::arg("bad"),
        pybind11::arg("any_active"), pybind11::arg("playing") = pybind11::none());
  m.def("paired_update", &paired_update,
        "paired evaluation: step checks, final rewards and the active mask after a step",
        pybind11::arg("active"), pybind11::arg("step_status"), pybind11::arg("new_done"),
        pybind11::arg("reward0"), pybind11::arg("nagari"), pybind11::arg("final_reward0"),
        pybind11::arg("final_nagari"), pybind11::arg("bad"), pybind11::arg("any_active"),
        pybind11::arg("steps"), pybind11::arg("playing") = pybind11::none());
  m.def("store_probe", &store_probe,
        "calibration: play_random's observation-row store pattern without the game",
        pybind11::arg("out"), pybind11::arg("rows"), pybind11::arg("row_bytes"),
        pybind11::arg("steps"), pybind11::arg("distinct"));
  m.def("paired_movers", &paired_movers,
        "query_pos = -1 for the games whose mover is not in the policy's seat",
        pybind11::arg("player"), pybind11::arg("seat"), pybind11::arg("query_pos"));
  m.def("paired_events", &paired_events,
        "paired evaluation of sequence policies: event and query slots, counts, cache lengths",
        pybind11::arg("active"), pybind11::arg("step_status"), pybind11::arg("committed"),
        pybind11::arg("new_done"), pybind11::arg("count"), pybind11::arg("length_a"),
        pybind11::arg("event_pos_a"), pybind11::arg("query_pos_a"),
        pybind11::arg("length_b") = pybind11::none(),
        pybind11::arg("event_pos_b") = pybind11::none(),
        pybind11::arg("query_pos_b") = pybind11::none());
  m.def("masked_argmax", &masked_argmax, "Greedy action: argmax of the legal logits");
  m.def("mlp_pack_weight", &mlp_pack_weight,
        "bf16 matrix in the actor kernel's MFMA operand order", pybind11::arg("w"),
        pybind11::arg("rows_pad"), pybind11::arg("cols_pad"));
  m.def("mlp_actor_forward", &mlp_actor_forward,
        "residual MLP actor forward in one launch -> (logits bf16, value f32)",
        pybind11::arg("x"), pybind11::arg("x_copy"), pybind11::arg("w_in"),
        pybind11::arg("b_in"), pybind11::arg("ln_w"), pybind11::arg("ln_b"),
        pybind11::arg("w1"), pybind11::arg("b1"), pybind11::arg("w2"), pybind11::arg("b2"),
        pybind11::arg("w_head"), pybind11::arg("b_head"), pybind11::arg("actions"),
        pybind11::arg("eps"), pybind11::arg("value") = pybind11::none());
  m.def("observe_bf16", &observe_bf16,
        "observe (and observe_sample's draw, given a sampler) with bfloat16 features written "
        "into a given tensor",
        pybind11::arg("states"), pybind11::arg("features"),
        pybind11::arg("sampler") = pybind11::none(), pybind11::arg("legal") = pybind11::none());
  m.def("gumbel_sample", &gumbel_sample, "Masked Gumbel-max action and its log-softmax probability",
        pybind11::arg("logits"), pybind11::arg("legal"), pybind11::arg("uniforms"),
        pybind11::arg("actions") = pybind11::none(), pybind11::arg("logp") = pybind11::none());
  m.def("decode_attention", &decode_attention, "Single-query attention over a KV cache",
        pybind11::arg("q"), pybind11::arg("keys"), pybind11::arg("values"), pybind11::arg("pos"),
        pybind11::arg("rows") = pybind11::none(), pybind11::arg("order") = pybind11::none());
  m.def("decode_attention_append", &decode_attention_append,
        "Write the new key/value at slot pos, then single-query attention",
        pybind11::arg("q"), pybind11::arg("k_new"), pybind11::arg("v_new"),
        pybind11::arg("keys"), pybind11::arg("values"), pybind11::arg("pos"),
        pybind11::arg("rows") = pybind11::none(), pybind11::arg("out") = pybind11::none(),
        pybind11::arg("order") = pybind11::none());
  m.def("kv_append", &kv_append,
        "the KV append of decode_attention_append without the attention, in place",
        pybind11::arg("k_new"), pybind11::arg("v_new"), pybind11::arg("keys"),
        pybind11::arg("values"), pybind11::arg("pos"), pybind11::arg("rows") = pybind11::none());
  m.def("accept_worlds", &accept_worlds,
        "redeal_worlds' acceptance test and copy of one try, in one launch");
  m.def("decode_order", &decode_order,
        "The queries longest first (int32 permutation) for the decode calls' `order`",
        pybind11::arg("pos"), pybind11::arg("slots"));
  m.attr("FEATURE_COUNT") = pybind11::int_(CUGO_FEATURE_COUNT);
  m.attr("ACTION_COUNT") = pybind11::int_(CUGO_ACTION_COUNT);
  m.attr("PRIMARY_ACTION_COUNT") = pybind11::int_(CUGO_PRIMARY_ACTION_COUNT);
  m.attr("CHOICE_ACTION_BEGIN") = pybind11::int_(CUGO_CHOICE_ACTION_BEGIN);
  m.attr("EVENT_WORDS") = pybind11::int_(CUGO_EVENT_WORDS);
  m.attr("START_WORDS") = pybind11::int_(CUGO_START_WORDS);
  m.attr("STATE_BYTES") = pybind11::int_(CUGO_STATE_BYTES);
  m.attr("STATUS_OK") = pybind11::int_(CUGO_STATUS_OK);
}
