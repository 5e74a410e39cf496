/*
 * cugo_hip.h - C ABI of the gfx950 Shin Matgo batch engine (libcugo_hip.so).
 *
 * One entry point per operation of the reference PyTorch extension
 * (python/csrc/torch50_ext.cpp:36-59, host wrappers python/csrc/torch50_ext.cu:406-686).
 * The C ABI takes plain device pointers, element counts and a hipStream_t; it allocates
 * nothing and never synchronises, so every call is an asynchronous launch on `stream`
 * and is safe inside HIP graph capture.  Shape/dtype/device checks stay with the
 * caller (the PyTorch extension raises the reference's RuntimeErrors,
 * torch50_ext.cu:26-51); per-row problems go to the `status` outputs exactly as in
 * the reference (-1 for an env id outside [0, env_count), ActionStatus50 0..9 otherwise,
 * include/cugo/game/rollout50.h:33-44).
 *
 * Layout contract (identical to the reference TorchEnv50, torch50.h:108-121):
 *   states   uint8 [n, CUGO_STATE_BYTES] rows, 8-byte aligned, row i = game i
 *   features float [n, CUGO_FEATURE_COUNT]      legal    uint8 (0/1) [n, CUGO_ACTION_COUNT]
 *   events   int64 [n, CUGO_EVENT_WORDS]         start    int64 [n, CUGO_START_WORDS]
 *   bool outputs are one byte 0/1 (torch.bool).
 * Padding bytes of every row the library writes are zero.
 *
 * Return value: 0 (hipSuccess) or the hipError_t of the launch; a negative value for
 * an invalid argument (negative count, null pointer with a non-zero count).
 */
#ifndef CUGO_HIP_H_
#define CUGO_HIP_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CUGO_FEATURE_COUNT 720        /* torch50.h:55 */
#define CUGO_ACTION_COUNT 179         /* torch50.h:22 */
#define CUGO_PRIMARY_ACTION_COUNT 127 /* torch50.h:16 */
#define CUGO_CHOICE_ACTION_BEGIN 127  /* torch50.h:17 */
#define CUGO_EVENT_WORDS 9            /* torch50.h:628 */
#define CUGO_START_WORDS 8            /* torch50.h:629 */
#define CUGO_STATE_BYTES 248          /* sizeof(TorchEnv50) */
#define CUGO_STATUS_OK 0              /* ActionStatus50::kOk */
#define CUGO_INVALID_INDEX_STATUS (-1) /* torch50_ext.cu:24 */

/* Library/ABI version (major << 16 | minor). */
int cugo_version(void);

/* create(seeds, first_players) -> states (torch50_ext.cu:131-141, 406-427). */
int cugo_create(const int64_t* seeds, const int64_t* first_players, int64_t n,
                uint8_t* states, hipStream_t stream);

/* observe(states) (torch50_ext.cu:143-158, 429-446). */
int cugo_observe(const uint8_t* states, int64_t n, float* features, uint8_t* legal,
                 uint8_t* player, uint8_t* done, int16_t* status, hipStream_t stream);

/* observe_indexed(states, env_ids) (torch50_ext.cu:160-184, 448-472). */
int cugo_observe_indexed(const uint8_t* states, int64_t env_count, const int64_t* env_ids,
                         int64_t n, float* features, uint8_t* legal, uint8_t* player,
                         uint8_t* done, int16_t* status, hipStream_t stream);

/* step(states, actions), in place (torch50_ext.cu:186-200, 474-497). */
int cugo_step(uint8_t* states, const int64_t* actions, int64_t n, float* reward,
              uint8_t* done, uint8_t* nagari, int16_t* status, uint8_t* committed,
              hipStream_t stream);

/* step_indexed(states, env_ids, actions), in place (torch50_ext.cu:202-225, 499-528). */
int cugo_step_indexed(uint8_t* states, int64_t env_count, const int64_t* env_ids,
                      const int64_t* actions, int64_t n, float* reward, uint8_t* done,
                      uint8_t* nagari, int16_t* status, uint8_t* committed,
                      hipStream_t stream);

/* step_events_indexed(states, env_ids, actions) (torch50_ext.cu:227-262, 554-588). */
int cugo_step_events_indexed(uint8_t* states, int64_t env_count, const int64_t* env_ids,
                             const int64_t* actions, int64_t n, float* reward, uint8_t* done,
                             uint8_t* nagari, int16_t* status, uint8_t* committed,
                             int64_t* events, hipStream_t stream);

/* start(states) (torch50_ext.cu:264-269, 590-605). */
int cugo_start(const uint8_t* states, int64_t n, int64_t* out, hipStream_t stream);

/* clone_indexed(states, env_ids) -> children (torch50_ext.cu:271-286, 607-629). */
int cugo_clone_indexed(const uint8_t* states, int64_t env_count, const int64_t* env_ids,
                       int64_t n, uint8_t* children, hipStream_t stream);

/* branch_indexed(states, env_ids, actions) -> children + step outputs; parents are
 * read only (torch50_ext.cu:288-314, 631-662). */
int cugo_branch_indexed(const uint8_t* states, int64_t env_count, const int64_t* env_ids,
                        const int64_t* actions, int64_t n, uint8_t* children, float* reward,
                        uint8_t* done, uint8_t* nagari, int16_t* status, uint8_t* committed,
                        hipStream_t stream);

/* hands_indexed(states, env_ids) -> int64 [n, 2] (torch50_ext.cu:316-334, 664-686). */
int cugo_hands_indexed(const uint8_t* states, int64_t env_count, const int64_t* env_ids,
                       int64_t n, int64_t* hands, hipStream_t stream);

/* stock_indexed(states, env_ids) -> int64 [n] (torch50_ext.cu:336-363, 530-552). */
int cugo_stock_indexed(const uint8_t* states, int64_t env_count, const int64_t* env_ids,
                       int64_t n, int64_t* stock, hipStream_t stream);

/*
 * Random-policy driver pieces (no counterpart in the reference extension; the
 * reference's own smoke harness samples in Python, python/torch50_smoke.py:33-36).
 *   cugo_sample_uniform: action[i] = legal list of row i [xorshift64(sampler[i]) % count],
 *     -1 when the row has no legal action; sampler words advance in place.
 *   cugo_reset_done: every row with done[i] != 0 is re-created from
 *     seed = base_seed + i + batch * (++generation[i]) with first = i & 1, and its
 *     sampler re-seeded from the same seed; completed[0] += number of rows reset
 *     (completed may be NULL: generation[] already counts each row's finished games,
 *     and one same-address atomic per 64 rows costs more than the rest of the kernel).
 *   cugo_observe_sample: cugo_observe plus cugo_sample_uniform's draw for every row,
 *     taken from the legal mask while the kernel holds it (one launch, the mask is not
 *     read back); outputs are those of the two calls.
 */
int cugo_sample_uniform(const uint8_t* legal, int64_t n, uint64_t* sampler, int64_t* actions,
                        hipStream_t stream);
/* cugo_observe_bf16: cugo_observe with the features rounded to bfloat16 (uint16 bits
 * [n, CUGO_FEATURE_COUNT], round to nearest even, as torch converts float32), for callers
 * that keep bf16 observations (the PPO rollout's buffer); with sampler and actions (both
 * or neither NULL) also cugo_observe_sample's draw.  No reference counterpart. */
int cugo_observe_bf16(const uint8_t* states, int64_t n, uint16_t* features, uint8_t* legal,
                      uint8_t* player, uint8_t* done, int16_t* status, uint64_t* sampler,
                      int64_t* actions, hipStream_t stream);
int cugo_observe_sample(const uint8_t* states, int64_t n, float* features, uint8_t* legal,
                        uint8_t* player, uint8_t* done, int16_t* status, uint64_t* sampler,
                        int64_t* actions, hipStream_t stream);
int cugo_reset_done(uint8_t* states, const uint8_t* done, int64_t n, uint64_t base_seed,
                    uint32_t* generation, uint64_t* sampler, unsigned long long* completed,
                    hipStream_t stream);
/* Pre-dealt next games for cugo_reset_done_spares: each row i holds spares for its next
 * S = spare_slots games (1, 2 or 4).  Game g of row i (seed = base_seed + i +
 * seed_stride * g, first = i & 1) is pre-dealt in spare row (g & (S - 1)) * n + i, valid
 * when spare_gen of that row equals g.  For g = generation[i] + 1 .. generation[i] + S,
 * every stale one is dealt and its spare_gen set.  spares: uint8 [S * n,
 * CUGO_STATE_BYTES]; spare_gen: uint32 [S * n], start it at 0.  seed_stride = n gives
 * cugo_reset_done's seeds; a slice of a larger batch starting at an even row r0 passes
 * base_seed + r0 and the whole batch's size.  More slots serve rows that finish several
 * games between refills without dealing inline. */
int cugo_refill_spares(uint8_t* spares, uint32_t* spare_gen, const uint32_t* generation,
                       int64_t n, uint64_t base_seed, int64_t seed_stride, int64_t spare_slots,
                       hipStream_t stream);
/* Same effect as cugo_reset_done with seed = base_seed + i + seed_stride * generation[i],
 * except that a finished row copies its next game from its pre-dealt spare (the
 * cugo_refill_spares layout with the same spare_slots) when one is there, and deals it
 * inline otherwise. */
int cugo_reset_done_spares(uint8_t* states, const uint8_t* done, int64_t n, uint64_t base_seed,
                           int64_t seed_stride, uint32_t* generation, uint64_t* sampler,
                           unsigned long long* completed, const uint8_t* spares,
                           const uint32_t* spare_gen, int64_t spare_slots, hipStream_t stream);
/* cugo_branch_indexed followed by cugo_observe_indexed of the children (ids 0..n-1), in
 * one launch (the reference's callers do both, python/cugo_ppo50.py:96-98): children and
 * the step outputs as cugo_branch_indexed, then the children's observation as
 * cugo_observe (features/legal/player/obs_done/obs_status); the children are not read
 * back. */
int cugo_branch_observe_indexed(const uint8_t* states, int64_t env_count, const int64_t* ids,
                                const int64_t* actions, int64_t n, uint8_t* children,
                                float* reward, uint8_t* done, uint8_t* nagari, int16_t* status,
                                uint8_t* committed, float* features, uint8_t* legal,
                                uint8_t* player, uint8_t* obs_done, int16_t* obs_status,
                                hipStream_t stream);
/* `steps` (1 .. 2^20) random-policy self-play steps in one launch, each
 * cugo_observe_sample followed by cugo_step_reset_spares on its actions, with the effect
 * of `steps` calls of one step each: the outputs (observation, actions, then the step's
 * outputs) are the last step's, and every step's observation is written.  The games stay
 * on chip between steps, and one step's observation stores overlap the step and the next
 * observation.  The reference's loop calls observe, samples and steps once per step
 * (python/torch50_smoke.py); steps = 1 is that loop's step in one launch.  A finished row
 * whose next game's spare is stale gets that game dealt into the spare's slot (spare_gen is
 * left as it was) and takes it from there. */
int cugo_play_random(uint8_t* states, int64_t n, uint64_t* sampler, float* features,
                     uint8_t* legal, uint8_t* player, uint8_t* obs_done, int16_t* obs_status,
                     int64_t* actions, float* reward, uint8_t* done, uint8_t* nagari,
                     int16_t* status, uint8_t* committed, uint64_t base_seed,
                     int64_t seed_stride, uint32_t* generation, uint8_t* spares,
                     const uint32_t* spare_gen, int64_t spare_slots, int64_t steps,
                     hipStream_t stream);
/* cugo_play_random (the same kernel) keeping every step's outputs: step s (0 .. steps - 1)
 * writes rows s * step_rows .. s * step_rows + n - 1 of each output, so the outputs hold
 * `steps` blocks of step_rows rows (features [steps * step_rows, 720], and so on), and
 * the states, generation and sampler end as cugo_play_random leaves them.  step_rows must
 * be at least n and a multiple of 4; rows n .. step_rows - 1 of a block are not written.
 * A test and diagnostics form of the random-policy loop (no counterpart in the reference,
 * whose loop keeps each step's outputs by calling observe and step once per step,
 * python/torch50_smoke.py:22-50). */
int cugo_play_random_record(uint8_t* states, int64_t n, uint64_t* sampler, float* features,
                            uint8_t* legal, uint8_t* player, uint8_t* obs_done,
                            int16_t* obs_status, int64_t* actions, float* reward,
                            uint8_t* done, uint8_t* nagari, int16_t* status,
                            uint8_t* committed, uint64_t base_seed, int64_t seed_stride,
                            uint32_t* generation, uint8_t* spares, const uint32_t* spare_gen,
                            int64_t spare_slots, int64_t steps, int64_t step_rows,
                            hipStream_t stream);
/* cugo_step followed by cugo_reset_done_spares(states, done, n, base_seed, seed_stride,
 * generation, sampler, NULL, spares, spare_gen, spare_slots) in one launch: the outputs are the
 * step's (done[i] = 1 for the game that just finished), and each finished row already
 * holds its next game when the call returns. */
int cugo_step_reset_spares(uint8_t* states, const int64_t* actions, int64_t n, float* reward,
                           uint8_t* done, uint8_t* nagari, int16_t* status, uint8_t* committed,
                           uint64_t base_seed, int64_t seed_stride, uint32_t* generation,
                           uint64_t* sampler, const uint8_t* spares, const uint32_t* spare_gen,
                           int64_t spare_slots, hipStream_t stream);
/* cugo_step_observe_spares: cugo_step_reset_spares followed by cugo_observe (features_dtype
 * CUGO_DTYPE_F32, float [n, CUGO_FEATURE_COUNT]) or cugo_observe_bf16 (CUGO_DTYPE_BF16,
 * uint16 bits) of the new states, in one launch, with the outputs of both calls.  A
 * finished row whose spare is stale gets its next game dealt into the spare's slot first
 * (so spares is written; spare_gen is not).  No reference counterpart: the PPO rollout's
 * engine between two actor passes (python/cugo_ppo50.py:321-450 steps, then observes). */
int cugo_step_observe_spares(uint8_t* states, const int64_t* actions, int64_t n, float* reward,
                             uint8_t* done, uint8_t* nagari, int16_t* status,
                             uint8_t* committed, uint64_t base_seed, int64_t seed_stride,
                             uint32_t* generation, uint64_t* sampler, uint8_t* spares,
                             const uint32_t* spare_gen, int64_t spare_slots, int features_dtype,
                             void* features, uint8_t* legal, uint8_t* player,
                             uint8_t* obs_done, int16_t* obs_status, hipStream_t stream);
/* redeal (python/cugo_ppo50.py:122-148, `_redeal`) in place on rows [n, CUGO_STATE_BYTES]
 * for observer seat[i], given the reference's random draws: keys f32 [n, 50]
 * (torch.rand(n, 50)) rank the unknown cards (the opponent's cards not shown by a shake,
 * and the stock); the opponent's new free cards are the `count` unknown cards with the
 * smallest keys, ties to the lower card id; the rest is the stock; held follows the new
 * hand; the RNG word becomes rng[i] (torch.randint(-2**62, 2**62, (n,))). */
int cugo_redeal(uint8_t* states, const int64_t* seat, const float* keys, const int64_t* rng,
                int64_t n, hipStream_t stream);
/* redeal_worlds' acceptance test and copy (python/cugo_ppo50.py:151-172, one try): the
 * candidate rows [n, CUGO_STATE_BYTES] (redealt copies of rows missing[j] % rows) with
 * their observations features f32 [n, CUGO_FEATURE_COUNT] and legal [n, CUGO_ACTION_COUNT];
 * same[j] = 1 when candidate j's features and legal mask equal the real deal's
 * (real_features / real_legal row missing[j] % rows, value for value as torch's ==), and
 * then its row is copied to row missing[j] of out [out_rows, CUGO_STATE_BYTES]; a
 * missing[j] outside [0, out_rows) is never written (same[j] = 0).  No reference
 * counterpart as one call (the reference's torch ops compare, gather and copy). */
int cugo_accept_worlds(const float* features, const uint8_t* legal, const float* real_features,
                       const uint8_t* real_legal, const int64_t* missing, int64_t rows,
                       int64_t n, const uint8_t* candidates, uint8_t* out, int64_t out_rows,
                       uint8_t* same, hipStream_t stream);
/* sampler[i] = SplitMix64(base_seed + i + batch * generation[i]).next(), never 0. */
int cugo_seed_samplers(int64_t n, uint64_t base_seed, const uint32_t* generation,
                       uint64_t* sampler, hipStream_t stream);

/* The reference's canonical rollout driver (rollout_canonical_torch50, torch50.h:598-619,
 * over canonical_torch_action50, torch50.h:542-558, and canonical_action50,
 * rollout50.h:496-574; the digest of rollout_digest50, rollout50.h:706-719, plus
 * TorchRollout50's choice counters): game i is dealt from seeds[i] / first_players[i]
 * and played with the deterministic canonical action until it ends or has taken
 * max_actions (0 .. 65535) primary actions.  digest int64 [n, 5]:
 *   0 final_points   1 reward0 (seat 0)
 *   2 actions | turns << 16 | bonus_actions << 32 | special_actions << 48
 *   3 go_actions | end << 16 | action_status << 24 | terminal_reason << 32 | winner << 40
 *     | next_round_multiplier << 48    (end: RolloutEnd50, rollout50.h:70-76)
 *   4 choice_actions | resolve_choices << 16 | pi_choices << 32
 * The reference runs it on the CPU (torch50_test.cpp:160-191) and times its explicit
 * form on the GPU (tests/cuda_rollout50_bench.cu:22-33), whose digest words 0-3 equal
 * these. */
int cugo_rollout_canonical(const int64_t* seeds, const int64_t* first_players, int64_t n,
                           int64_t max_actions, int64_t* digest, hipStream_t stream);

/* Allocation-free random-policy play.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It computes exactly what cugo_refill_spares (2 slots,
 * on fresh spares) followed by cugo_play_random(..., steps) computes on the same states,
 * sampler and generation, with the spares taken from a static device array the library
 * holds on each device (31.5 MiB, allocated with the code object) instead of a caller's
 * workspace.  It calls no allocator.  n may be at most CUGO_NOALLOC_MAX_ROWS; a larger n
 * returns CUGO_ERROR_SCRATCH_LIMIT and launches nothing.  `stream` must belong to the
 * current device.  Every call on one device shares that array (each call first marks
 * all its spares stale, so earlier calls do not change the results): calls that overlap
 * on one device, on different streams or from different threads, race. */
#define CUGO_NOALLOC_MAX_ROWS 65536
#define CUGO_ERROR_SCRATCH_LIMIT (-27)
int cugo_play_random_noalloc(uint8_t* states, int64_t n, uint64_t* sampler, float* features,
                             uint8_t* legal, uint8_t* player, uint8_t* obs_done,
                             int16_t* obs_status, int64_t* actions, float* reward,
                             uint8_t* done, uint8_t* nagari, int16_t* status,
                             uint8_t* committed, uint64_t base_seed, int64_t seed_stride,
                             uint32_t* generation, int64_t steps, hipStream_t stream);

/*
 * Single-query decode attention over a per-row KV cache
 * (python/cugo_seq_attention50.py:43-62, the Triton `_decode_kernel` at :21-40 and its
 * two-matmul fallback at :58-62):
 *
 *   out[i, h, :] = sum_t softmax_t(scale * q[i,h,:] . keys[r,h,t,:]) values[r,h,t,:]
 *   with r = rows[i] (rows == NULL: r = i) and t = 0 .. min(pos[i], slots - 1).
 *
 *   q             [n, heads, dh] of q_dtype: q[i, h, :] at q + i * q_stride + h * dh
 *                 (q_stride >= heads * dh elements; a column slice of a packed
 *                 in-projection output is read in place)
 *   out           [n, heads, dh] of q_dtype, contiguous
 *   keys, values  [cache_rows, heads, slots, dh] of kv_dtype, contiguous, 16-byte aligned
 *   pos, rows     int64 [n]
 *   order         int32 [n] or NULL: the order in which the launch takes the queries (a
 *                 permutation of 0 .. n - 1, e.g. cugo_decode_order's); it changes no
 *                 result, only which queries the last workgroups serve (an entry outside
 *                 [0, n) is skipped: its query is not computed)
 * Softmax and accumulation are fp32; out is rounded to q_dtype.  dh is 16, 32, 64 or 128
 * (dh * element size >= 16 bytes).  A query whose pos is negative, or whose row is outside
 * [0, cache_rows), gets a NaN output (the reference's softmax over no slot is NaN) and
 * reads no cache memory.  Returns -1 for a bad count or null pointer, -2 for an
 * unsupported dtype, -3 for an unsupported dh, -4 for a misaligned cache pointer.
 */
#define CUGO_DTYPE_F32 0
#define CUGO_DTYPE_F16 1
#define CUGO_DTYPE_BF16 2

int cugo_decode_attention(int q_dtype, int kv_dtype, const void* q, int64_t q_stride,
                          const void* keys, const void* values, const int64_t* pos,
                          const int64_t* rows, const int32_t* order, int64_t n, int64_t heads,
                          int64_t dh, int64_t slots, int64_t cache_rows, float scale, void* out,
                          hipStream_t stream);

/*
 * The reference caller's KV append fused with the decode (python/cugo_seq50.py:313-320:
 * index_put_ of the new key/value at slot pos[i] of row rows[i], then decode_attention):
 * k_new/v_new [n, heads, dh] of kv_dtype (16-byte aligned; row i at i * new_stride
 * elements, new_stride * element size a multiple of 16) are written to slot
 * min(pos[i], slots - 1) of each query's row, and the query attends slots 0..pos as
 * above, taking the new slot from registers.  Two queries naming the same row write the
 * same slot (as index_put_ with repeated indices, the value that lands is either one).
 */
int cugo_decode_attention_append(int q_dtype, int kv_dtype, const void* q, int64_t q_stride,
                                 const void* k_new, const void* v_new, int64_t new_stride,
                                 void* keys, void* values, const int64_t* pos,
                                 const int64_t* rows, const int32_t* order, int64_t n,
                                 int64_t heads, int64_t dh, int64_t slots, int64_t cache_rows,
                                 float scale, void* out, hipStream_t stream);

/*
 * The KV append of cugo_decode_attention_append without the attention, for tokens whose
 * attention output nothing reads (the event tokens at a sequence policy's last layer:
 * the reference discards their outputs, cugo_seq_selfplay50.py:156): k_new / v_new
 * [n, heads, dh] of kv_dtype (row i at i * new_stride elements, 16-byte aligned) to slot
 * min(pos[i], slots - 1) of row rows[i] (rows NULL: row i) of keys / values, as
 * index_put_ does (cugo_seq50.py:317-318); pos < 0 or a row outside [0, cache_rows)
 * writes nothing.  Same return codes as cugo_decode_attention_append.
 */
int cugo_kv_append(int kv_dtype, const void* k_new, const void* v_new, int64_t new_stride,
                   void* keys, void* values, const int64_t* pos, const int64_t* rows,
                   int64_t n, int64_t heads, int64_t dh, int64_t slots, int64_t cache_rows,
                   hipStream_t stream);

/*
 * The order for cugo_decode_attention / _append that takes ragged rows longest first: order (int32
 * [n]) receives a permutation of 0 .. n - 1 sorted by min(pos, slots - 1), longest first
 * (negative pos last), in bins of 2^s lengths where slots >> s < 4,096 (s = 0 below 4,096
 * slots).  The dispatcher starts workgroups in index order as others finish, so the long
 * rows start first and the short ones fill in at the end of the launch.  A row's place
 * within its bin may differ between calls; no decode result depends on it.  One
 * workgroup; computed once, it serves every layer of a step and, while lengths grow
 * together, the following steps.  Returns -1 for n outside [0, 2^31), slots <= 0 or a
 * null pointer.  No reference counterpart (the reference's Triton grid takes the rows in
 * index order, cugo_seq_attention50.py:43-56).
 */
int cugo_decode_order(const int64_t* pos, int64_t n, int64_t slots, int32_t* order,
                      hipStream_t stream);

/*
 * Event-sequence policy self-play (python/cugo_seq50.py, python/cugo_seq_selfplay50.py).
 * dtype: CUGO_DTYPE_BF16 or CUGO_DTYPE_F32 for every weight and the output; d in
 * {64, 128, 256, 512, 1024}.  weight_t is the Linear weight transposed ([in, d],
 * contiguous), bias [d], position [position_rows, d], token_type [3, d].
 *
 * Row pointers (weights, bias, position, token_type, x, y, outputs) must be aligned to
 * (d / 64) elements (a torch allocation is); -4 otherwise.
 *
 * cugo_event_tokens: out[r] = SeqNet.event_token(words[j], seat[r], index[j]) with
 *   j = r % word_rows (cugo_seq50.py:276-282 with encode_events :91-110): event_in applied
 *   to the 414-wide observer-relative token of the 9-word event, + position[1 + min(index,
 *   47)] + token_type[1], with the reference's bf16 roundings (after the Linear, after
 *   each add).  words int64 [word_rows, 9] and index int64 [word_rows] (word_rows divides
 *   n: the self-play step passes each event once for both seats), seat int64 [n],
 *   weight_t [414, d], out [n, d].  With ln non-NULL, also ln[r] = LayerNorm(out[r]) *
 *   ln_weight + ln_bias ([d] each; the first encoder layer's norm1, cugo_seq50.py:318),
 *   the bits cugo_add_layernorm gives on out (ln NULL: ln_weight and ln_bias unused).
 */
int cugo_event_tokens(int dtype, const int64_t* words, int64_t word_rows, const int64_t* seat,
                      const int64_t* index, int64_t n, const void* weight_t, const void* bias,
                      const void* position, int64_t position_rows, const void* token_type,
                      int64_t d, void* out, const void* ln_weight, const void* ln_bias,
                      float eps, void* ln, hipStream_t stream);
/* cugo_start_tokens: out[i] = SeqNet.start_token(start[i], seat[i]) (cugo_seq50.py:271-274
 * with encode_start :113-128): start_in of the 274-wide opening token + position[0] +
 * token_type[0].  start int64 [n, 8], seat int64 [n], weight_t [274, d], out [n, d]. */
int cugo_start_tokens(int dtype, const int64_t* start, const int64_t* seat, int64_t n,
                      const void* weight_t, const void* bias, const void* position,
                      const void* token_type, int64_t d, void* out, hipStream_t stream);
/* cugo_add_layernorm: the residual step of a pre-norm transformer layer
 * (nn.TransformerEncoderLayer, norm_first; python/cugo_seq50.py:318-322):
 * x_out = x + y (rounded to dtype; y == NULL leaves x_out unwritten and normalises x),
 * ln = LayerNorm(x_out) * weight + bias with fp32 row statistics, rounded to dtype.
 * x, y, x_out, ln [n, d]; weight, bias [d]; x_out may alias x. */
int cugo_add_layernorm(int dtype, const void* x, const void* y, const void* weight,
                       const void* bias, float eps, int64_t n, int64_t d, void* x_out, void* ln,
                       hipStream_t stream);
/* cugo_linear: the nn.Linear layers of SeqNet.cached_step (cugo_seq50.py:291-322: the
 * packed in-projection, out_proj, linear1 followed by the layer's GELU, linear2), bf16:
 * y = act(x w^T + bias), each element rounded to bf16 after the bias and, with
 * CUGO_LINEAR_GELU, GELU(v) = v / 2 (1 + erf(v / sqrt 2)) of that value rounded again.
 * x [m, k] with row stride ldx; w [n, k] (nn.Linear's layout) given as w_packed, its
 * cugo_mlp_pack_weight form with rows_pad = roundup(n, 16) and cols_pad = k; bias [n] or
 * NULL; y [m, n] with row stride ldy; residual NULL or [m, n] with row stride ldr (0: one
 * [n] row for every row), added to each output after its rounding and rounded again (the
 * last layer's x + linear2(u), cugo_seq50.py:322; the query token's + token_type[2],
 * :166-180); y may alias residual; fp32 accumulation.  Requires k in {64, 128, 256,
 * 512, 1024}, ldx % 8 == 0, ldy >= n, x and w_packed 16-byte aligned, y and bias 8-byte
 * aligned, and with a residual n % 4 == 0 and ldy % 4 == 0 (any n without one: the
 * head's 179 logits).  tile: 0 chooses the workgroup tile from the shape; 1-7 force
 * 32 x 128, 64 x 128 (8 wavefronts), 64 x 128, 128 x 128 (8), 64 x 64, 128 x 128 or
 * 32 x 256 (rows x columns; -7 where the X panel, rows x k, passes the LDS).  Returns -3
 * for an unsupported shape,
 * -4 for misaligned pointers, -5 for sizes beyond 32-bit byte offsets. */
#define CUGO_LINEAR_NONE 0
#define CUGO_LINEAR_GELU 1
int cugo_linear(int act, const void* x, int64_t ldx, const void* w_packed, const void* bias,
                const void* residual, int64_t ldr, int64_t m, int64_t n, int64_t k, void* y,
                int64_t ldy, int tile, hipStream_t stream);
/* cugo_linear_add_layernorm: cugo_linear (no activation) followed by cugo_add_layernorm of
 * its output onto res, in one launch: the out_proj / linear2 of a pre-norm encoder layer
 * with the residual add and the next LayerNorm (cugo_seq50.py:316-322).  y = bf16(x w^T +
 * bias); x_out = bf16(res + y); ln = LayerNorm(x_out) * ln_weight + ln_bias, with the
 * statistics and roundings of cugo_add_layernorm.  n must be 256; res [m, 256] with row
 * stride ldr (256 for contiguous rows; 0: one [256] row added to every row, the query
 * token's + token_type[2], cugo_seq50.py:166-180, normalised by the first layer's norm1);
 * x_out, ln contiguous [m, 256] (x_out may alias res); other requirements as
 * cugo_linear.  tile: 0 by shape; 1 for 32-row tiles on 4 wavefronts, 2 on 8, 3 for
 * 16-row tiles on 4, 4 for 64-row tiles on 8. */
int cugo_linear_add_layernorm(const void* x, int64_t ldx, const void* w_packed,
                              const void* bias, int64_t m, int64_t n, int64_t k, const void* res,
                              int64_t ldr, const void* ln_weight, const void* ln_bias, float eps,
                              void* x_out, void* ln, int tile, hipStream_t stream);
/* cugo_ffn: the feed-forward half of a pre-norm encoder layer of SeqNet.cached_step
 * (cugo_seq50.py:319-322) with the norm after it, in one launch, for d_model 256 and a
 * 1,024-wide hidden layer: u = GELU(h w1^T + b1) (each rounded to bf16 as cugo_linear
 * with CUGO_LINEAR_GELU), y = bf16(u w2^T + b2), x_out = bf16(x + y), and with ln_weight
 * ln = LayerNorm(x_out) * ln_weight + ln_bias (the next layer's norm1 or the final norm,
 * as cugo_linear_add_layernorm).  The same bits as cugo_linear (GELU) followed by
 * cugo_linear_add_layernorm (or by cugo_linear with the residual, when ln_weight and
 * ln_bias are NULL); the hidden layer never leaves the chip.  h [m, 256] with row stride
 * ldh (16-byte aligned); x, x_out, ln contiguous [m, 256] (x_out may alias x); w1_packed
 * the [1,024, 256] linear1 weight and w2_packed the [256, 1,024] linear2 weight in
 * cugo_mlp_pack_weight form (rows_pad = rows, cols_pad = cols); b1 [1,024], b2 [256],
 * ln_weight / ln_bias [256]; all bf16.  rows: rows a workgroup (16, 32, 48 or 64; 0 chooses by
 * m).  No reference counterpart as one call. */
int cugo_ffn(const void* h, int64_t ldh, const void* x, const void* w1_packed, const void* b1,
             const void* w2_packed, const void* b2, const void* ln_weight, const void* ln_bias,
             float eps, int64_t m, void* x_out, void* ln, int rows, hipStream_t stream);
/* cugo_out_proj_ffn: the rest of a pre-norm encoder layer of SeqNet.cached_step after the
 * attention (cugo_seq50.py:317-322) in one launch: x1 = bf16(x + bf16(att wo^T + bo)),
 * h = LayerNorm(x1) * ln2_weight + ln2_bias (norm2, eps2), then cugo_ffn of (h, x1): the
 * same bits as cugo_linear_add_layernorm (out_proj + add + norm2) followed by cugo_ffn,
 * with neither x1 nor h leaving the chip.  att [m, 256] with row stride ld_att (16-byte
 * aligned), wo_packed the [256, 256] out_proj weight in cugo_mlp_pack_weight form, bo,
 * ln2_weight, ln2_bias [256] bf16; the rest as cugo_ffn (x_out may alias x).  No reference
 * counterpart as one call. */
int cugo_out_proj_ffn(const void* att, int64_t ld_att, const void* x, const void* wo_packed,
                      const void* bo, const void* ln2_weight, const void* ln2_bias, float eps2,
                      const void* w1_packed, const void* b1, const void* w2_packed,
                      const void* b2, const void* ln_weight, const void* ln_bias, float eps,
                      int64_t m, void* x_out, void* ln, int rows, hipStream_t stream);
/* cugo_gumbel_sample: the sampling of WaveCollector._step (cugo_seq_selfplay50.py:125-130)
 * given the uniforms torch.rand_like drew: masked = legal ? logits : -1e30;
 * actions[i] = argmax_a(masked - log(-log(clamp(u, 1e-20, 1)))) (first index on ties);
 * logp[i] = log_softmax(masked)[actions[i]].  logits [n, A] of logits_dtype (F32 or BF16,
 * which converts exactly), uniforms f32 [n, A], legal bool [n, A].  uniforms == NULL
 * gives the greedy masked argmax of cugo_eval50.py:125-127 (no noise); logp == NULL skips
 * the log-probability. */
int cugo_gumbel_sample(int logits_dtype, const void* logits, const uint8_t* legal,
                       const float* uniforms, int64_t n, int64_t actions_count, int64_t* actions,
                       float* logp, hipStream_t stream);

/* cugo_gumbel_sample_philox: cugo_gumbel_sample with its uniforms drawn in the kernel
 * from Philox4x32-10 (Salmon et al., SC 2011) instead of read from memory: for row r and
 * action a, word (a / 16) % 4 of the generator at counter (r mod 2^32, (a % 16) + 64 (a / 64)
 * + 256 (r / 2^32), offset, *epoch mod 2^32) under the key (seed mod 2^32, seed / 2^32), as
 * (word >> 8) * 2^-24.  epoch is device memory (read at run time, so a captured graph can
 * advance it between replays); offset tells apart the calls of one epoch (e.g. the step
 * of a rollout).  actions_count <= 192.  uniforms_out, if not NULL, receives the uniforms
 * f32 [n, A].  No reference counterpart: the PPO rollout's sampler, whose uniforms the
 * reference draws with torch (python/cugo_ppo50.py:321-450). */
int cugo_gumbel_sample_philox(int logits_dtype, const void* logits, const uint8_t* legal,
                              uint64_t seed, const uint64_t* epoch, uint32_t offset, int64_t n,
                              int64_t actions_count, int64_t* actions, float* logp,
                              float* uniforms_out, hipStream_t stream);

/* The weights of a residual MLP actor (bf16 device pointers): h = x W_in^T + b_in; per
 * block h += W2 relu(W1 LN_b(h) + b1) + b2; z = LN_blocks(h); [logits, value] = z W_head^T
 * + b_head.  The matrices are packed by cugo_mlp_pack_weight (Linear weights [out, in]):
 * w_in [hidden, features] padded to [hidden, CUGO_MLP_MAX_FEATURES]; w1, w2 [hidden,
 * hidden]; w_head = the logits weight [actions, hidden] with the value weight [1, hidden]
 * as row `actions`, padded to [CUGO_MLP_HEAD_ROWS, hidden].  b_head [actions + 1]: the
 * logits biases, then the value bias. */
#define CUGO_MLP_MAX_BLOCKS 4
#define CUGO_MLP_MAX_FEATURES 768
#define CUGO_MLP_HEAD_ROWS 256
typedef struct CugoMlpWeights {
  int hidden;   /* must be 512 */
  int blocks;   /* 0 .. CUGO_MLP_MAX_BLOCKS */
  int features; /* multiple of 8, at most CUGO_MLP_MAX_FEATURES */
  int actions;  /* logits; actions + 1 <= CUGO_MLP_HEAD_ROWS */
  float eps;    /* LayerNorm epsilon */
  const void* w_in;
  const void* b_in;
  const void* ln_w[CUGO_MLP_MAX_BLOCKS + 1]; /* block LayerNorms, then the final one */
  const void* ln_b[CUGO_MLP_MAX_BLOCKS + 1];
  const void* w1[CUGO_MLP_MAX_BLOCKS];
  const void* b1[CUGO_MLP_MAX_BLOCKS];
  const void* w2[CUGO_MLP_MAX_BLOCKS];
  const void* b2[CUGO_MLP_MAX_BLOCKS];
  const void* w_head;
  const void* b_head;
} CugoMlpWeights;

/* cugo_mlp_pack_weight: a bf16 matrix w [rows, cols] (row major) in the order the actor
 * kernel reads its MFMA B operands: packed[((t * S + s) * 64 + 16 q + r) * 8 + i] =
 * w[16 t + r][32 s + 8 q + i] with S = cols_pad / 32, zero outside [rows, cols).
 * rows_pad a multiple of 16, cols_pad of 32; packed holds rows_pad * cols_pad values.
 * Run once per weight update. */
int cugo_mlp_pack_weight(const void* w, int64_t rows, int64_t cols, int64_t rows_pad,
                         int64_t cols_pad, void* packed, hipStream_t stream);

/* cugo_mlp_actor_forward: the PPO rollout actor's forward pass in one launch (no reference
 * counterpart: the reference's collector, python/cugo_ppo50.py:321-450, runs its actor as
 * torch layers).  x [n, features] of x_dtype (F32 or BF16); x_copy, if not NULL, receives
 * x rounded to bf16 [n, features]; logits bf16 [n, actions]; value f32 [n].  bf16
 * operands, fp32 accumulation, the residual stream kept in fp32 between blocks.  Returns
 * -3 for an unsupported shape. */
int cugo_mlp_actor_forward(int x_dtype, const void* x, void* x_copy, int64_t n,
                           const CugoMlpWeights* weights, void* logits, float* value,
                           hipStream_t stream);

/* The tensors of one self-play wave (WaveCollector, cugo_seq_selfplay50.py:45-76), w games,
 * max_steps recorded steps; every pointer is device memory. */
typedef struct CugoSelfPlayWave {
  int64_t w, max_steps;
  int64_t width;                  /* recorded / query feature columns: 720, or the
                                     events-mode context columns */
  const int32_t* columns;         /* [width] feature columns kept, NULL = all 720 */
  int64_t pool_games;             /* games 0 .. pool_games-1 face the frozen opponent */
  const int64_t* learner_seat;    /* [w]: the learner's seat (read for pool games) */
  int64_t* opp_cache_length;      /* [max(1, pool_games)]: the opponent's cache lengths
                                     (NULL without a pool) */
  int64_t* step_index;            /* [2]: [0] the step being recorded (prepare copies [1]
                                     into it), [1] the next one (advance writes [0] + 1);
                                     both 0 at a wave's start */
  int64_t* count;                 /* [w]: events committed so far */
  int64_t* events;                /* [w, 48, 9]: event log */
  int64_t* cache_length;          /* [2 w]: KV-cache lengths, row = seat * w + game */
  float* final_reward0;           /* [w] */
  uint8_t* final_nagari;          /* [w] bool */
  uint8_t* finished;              /* [w] bool */
  unsigned long long* bad;        /* [1] int64: bad observe/step results */
  uint16_t* rec_features;         /* [max_steps, w, width] bf16 */
  uint8_t* rec_legal;             /* [max_steps, w, 179] bool */
  float* rec_logp;                /* [max_steps, w] */
  int64_t* rec_actions;           /* [max_steps, w], and likewise: */
  int64_t* rec_opp_hand;
  int64_t* rec_stock;
  int64_t* rec_stop_points;
  int64_t* rec_seat;
  int64_t* rec_count;
  uint8_t* rec_valid;             /* [max_steps, w] bool */
  int64_t q_stride;               /* elements between q_in rows, >= width + 179 (the
                                     columns past width + 179 are written as zeros); 0 means
                                     width + 179 */
  uint64_t* noise_epoch;          /* [1] or NULL: advanced by one by every
                                     cugo_selfplay_advance (the epoch of the step's Philox
                                     noise, cugo_gumbel_sample_philox) */
  int64_t* query_pos;             /* [w] or NULL: cugo_selfplay_prepare writes
                                     cache_length[query_rows[i]], the query's cache slot,
                                     or -1 for a game that is over (the decode skips it) */
  int64_t* event_pos;             /* [2 w] or NULL: cugo_selfplay_advance writes each cache
                                     row's length before the step's events are counted (the
                                     slots the step's event tokens go to), or -1 where the
                                     step's event is not kept (no committed action, or a
                                     game already over: the decode skips the row) */
  int32_t* playing;               /* [1] or NULL: cugo_selfplay_prepare clears it and
                                     cugo_selfplay_advance sets it to 1 when a game is still
                                     being played after the step (the host's stop test,
                                     without a reduction launch) */
} CugoSelfPlayWave;

/* cugo_selfplay_prepare: the step's work between observe and the policy
 * (cugo_seq_selfplay50.py:110-140): bad += active & (status != OK or no legal action);
 * q_in [w, width + 179] of q_dtype (row stride q_stride, zero padded) = (the kept feature
 * columns, legal as 0/1), the policy's query input; records of step step_index (skipped outside [0, max_steps)): the
 * kept features as bf16, legal, opponent hand (hands word 1 - player of the state row),
 * stock, stop points (round(exp2(12 f[471]) - 1), cugo_contract50.py:40-42), seat, count,
 * valid = active and the learner moves (a pool game's mover may be the opponent);
 * query_rows [w] = (player & 1) * w + game.  states [w, 248] (row = game), features
 * f32 [w, 720], legal bool [w, 179], player/done [w], status i16 [w] (observe outputs),
 * stock int64 [w] (stock_indexed before the step), or NULL: the same words taken from the
 * state rows here (no stock_indexed launch). */
int cugo_selfplay_prepare(const CugoSelfPlayWave* wave, int q_dtype, const uint8_t* states,
                          const float* features, const uint8_t* legal, const uint8_t* player,
                          const uint8_t* done, const int16_t* status, const int64_t* stock,
                          void* q_in, int64_t* query_rows, hipStream_t stream);
/* cugo_store_probe: a calibration launch with no counterpart in the reference: the store
 * pattern of play_random's observation rows without the game (each 64-lane wave owns 64
 * consecutive rows of row_bytes and writes them 4 rows at a time as 1 KiB float4 stores),
 * `steps` times, into rows [s * rows, (s + 1) * rows) at step s when `distinct`, else over
 * rows [0, rows) every step.  out holds rows * row_bytes bytes (times steps when
 * distinct), 16-byte aligned; rows a multiple of 64, row_bytes a multiple of 16. */
int cugo_store_probe(void* out, int64_t rows, int64_t row_bytes, int64_t steps, int distinct,
                     hipStream_t stream);

/* cugo_query_input: the query token's input row of SeqNet._query (cugo_seq50.py:166-180)
 * for callers outside the self-play step: q_in[i] = [features[i][columns] (or all 720),
 * legal[i] as 0/1] in q_dtype (CUGO_DTYPE_BF16 rounded to nearest even, or CUGO_DTYPE_F32),
 * zero-padded to q_stride >= width + 179 columns.  features f32 [n, 720], legal bool
 * [n, 179], columns int32 [width] or NULL (width 720); a column index outside [0, 720)
 * writes NaN.  No reference counterpart as one call (the reference concatenates with torch
 * ops). */
int cugo_query_input(int q_dtype, const float* features, const uint8_t* legal,
                     const int32_t* columns, int64_t width, int64_t n, void* q_in,
                     int64_t q_stride, hipStream_t stream);

/* Paired evaluation on resident games (evaluate_paired, cugo_eval50.py:137-361, with
 * finished games masked instead of dropped; no counterpart in the reference, whose loop
 * does this with torch ops).  cugo_paired_select, after observe: bad[0] += active &
 * status != OK, bad[1] += active & status == OK & (done | !any_legal), *any_active = 1 if
 * any game is active, actions[i] = player[i] == a_seat[i] ? act_a[i] : act_b[i];
 * *playing = 0 when playing is not NULL.
 * cugo_paired_update, after the engine step: *steps += 1 and *any_active = 0 if it was set;
 * bad[2] += active & step_status != OK; games that end now (active, OK, new_done) keep
 * reward0 and nagari in final_reward0 / final_nagari; active &= OK & !new_done; *playing =
 * 1 when a game is still active (the host's stop test without a reduction launch).  bool
 * arrays are one byte; bad int64 [3]. */
int cugo_paired_select(const uint8_t* active, const int16_t* status, const uint8_t* done,
                       const uint8_t* any_legal, const uint8_t* player, const int64_t* a_seat,
                       const int64_t* act_a, const int64_t* act_b, int64_t n, int64_t* actions,
                       int64_t* bad, int32_t* any_active, int32_t* playing,
                       hipStream_t stream);
int cugo_paired_update(uint8_t* active, const int16_t* step_status, const uint8_t* new_done,
                       const float* reward0, const uint8_t* nagari, int64_t n,
                       float* final_reward0, uint8_t* final_nagari, int64_t* bad,
                       int32_t* any_active, int64_t* steps, int32_t* playing,
                       hipStream_t stream);
/* cugo_paired_movers: query_pos[i] = -1 for every game whose mover (player[i], the
 * observation's) is not in seat[i], the seat a sequence policy plays: that policy's pass
 * then skips those games' queries, as the reference feeds each model only its movers
 * (cugo_eval50.py:130-135). */
int cugo_paired_movers(const uint8_t* player, const int64_t* seat, int64_t n,
                       int64_t* query_pos, hipStream_t stream);

/* cugo_paired_events: the event log of a paired evaluation of sequence policies, which the
 * reference keeps in a History (History.record, cugo_seq50.py:62-67, called at
 * cugo_eval50.py:258-263; no counterpart as one call), as each policy's KV-cache lengths.
 * After the engine step (step_events_indexed) and the event tokens, before
 * cugo_paired_update.  A game's event is kept when the game is active, its step status is
 * OK and its action committed: event_pos_a[i] = length_a[i] (the slot its token takes at
 * the next step's pass), then count[i] and length_a[i] advance by one; an event not kept
 * gets event_pos_a[i] = -1 (its row of the pass is skipped).  query_pos_a[i] is the slot of
 * the next step's query: the new length_a[i] for a game that is active, OK and not
 * finished by this step, else -1 (skipped).  The same for policy b, whose three arrays are
 * all NULL when one policy keeps a cache.  int64 arrays of n entries; bool arrays one
 * byte. */
int cugo_paired_events(const uint8_t* active, const int16_t* step_status,
                       const uint8_t* committed, const uint8_t* new_done, int64_t n,
                       int64_t* count, int64_t* length_a, int64_t* event_pos_a,
                       int64_t* query_pos_a, int64_t* length_b, int64_t* event_pos_b,
                       int64_t* query_pos_b, hipStream_t stream);

/* cugo_selfplay_advance: the step's work after the engine step (cugo_seq_selfplay50.py:
 * 146-163): bad += active & (step status != OK); games that finished now keep reward0 and
 * the nagari flag and are marked finished; a committed event goes to slot min(count, 47)
 * of the log and advances both seats' cache lengths and the count; actions and logp are
 * recorded at step step_index; a pool game's committed event also advances the opponent's
 * cache length.  done = observe's done before the step; the others are
 * step_events_indexed's outputs.  Call after the event tokens were appended. */
int cugo_selfplay_advance(const CugoSelfPlayWave* wave, const uint8_t* done,
                          const float* reward0, const uint8_t* new_done, const uint8_t* nagari,
                          const int16_t* step_status, const uint8_t* committed,
                          const int64_t* events, const int64_t* actions, const float* logp,
                          hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CUGO_HIP_H_ */
