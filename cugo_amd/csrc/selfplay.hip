// Token embeddings, the residual add + LayerNorm of the decoder layers and action
// sampling of the event-sequence policy's self-play step, for gfx950.
//
// Reference: python/cugo_seq50.py (encode_events :91-110, encode_start :113-128,
// SeqNet.start_token :271-274, SeqNet.event_token :276-282) and the sampling lines of
// WaveCollector._step (python/cugo_seq_selfplay50.py:125-130).
//
// An event or opening token is a 0/1 vector (card planes, a one-hot kind or mission
// type) plus a few small scalars, and the first thing the policy does with it is a
// Linear layer.  Instead of materialising the [n, 414] or [n, 274] token and running a
// GEMM, each row sums the weight columns of its set bits (weights stored transposed,
// one contiguous d-element row per input feature, so a column read is coalesced), then
// adds the bias, the position row and the token-type row with the same roundings as
// the reference's bf16 ops:
//   r1 = round(bias + sum_j token_j * W[:, j])      (nn.Linear, fp32 accumulation)
//   r2 = round(r1 + position[p])                     (bf16 add)
//   out = round(r2 + token_type[t])                  (bf16 add)
// One 64-lane wavefront per row; the row's words are wave-uniform, so the walk over its
// set bits is scalar, and lane l owns the d / 64 consecutive output columns from
// l d / 64 (one wide load per weight row).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <initializer_list>

#include "../../include/cugo_hip.h"
#include "engine.h"

namespace cugo_amd {
namespace tokens {

typedef int64_t i64;
typedef uint64_t u64;

constexpr u64 kCardMask = (1ull << 50) - 1ull;
constexpr int kEventIn = 8 * 50 + 12 + 2;      // EVENT_IN, cugo_seq50.py:40
constexpr int kStartIn = 5 * 50 + 12 + 8 + 4;  // START_IN, cugo_seq50.py:41
constexpr int kKinds = 12;                     // KINDS, cugo_seq50.py:38
constexpr int kMaxEvents = 48;                 // MAX_EVENTS, cugo_seq50.py:37
constexpr int kRowsPerBlock = 4;

struct BF16 {
  using storage = uint16_t;
  __device__ static float to_float(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
  // Round to nearest even; NaN stays a quiet NaN (the conversion torch uses).
  __device__ static uint16_t from_float(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  __device__ static float round(float f) { return to_float(from_float(f)); }
  // 4 consecutive values (p 8-byte aligned)
  __device__ static void store4(uint16_t* p, float4 x) {
    *reinterpret_cast<uint2*>(p) =
        make_uint2((uint32_t)from_float(x.x) | ((uint32_t)from_float(x.y) << 16),
                   (uint32_t)from_float(x.z) | ((uint32_t)from_float(x.w) << 16));
  }
};

struct F32 {
  using storage = float;
  __device__ static float to_float(float x) { return x; }
  __device__ static float from_float(float f) { return f; }
  __device__ static float round(float f) { return f; }
  __device__ static void store4(float* p, float4 x) { *reinterpret_cast<float4*>(p) = x; }
};

__device__ inline int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// K consecutive elements as one (K * element size)-byte access: every row of d = 64 K
// elements starts 64 K-element aligned, and lane l owns columns l K .. l K + K - 1.
template <class S, int K>
struct alignas(sizeof(S) * K) Vec {
  S v[K];
};

template <class T, int K>
__device__ inline void load_row(const typename T::storage* p, float (&f)[K]) {
  const auto vec = *reinterpret_cast<const Vec<typename T::storage, K>*>(p);
#pragma unroll
  for (int k = 0; k < K; ++k) f[k] = T::to_float(vec.v[k]);
}

template <class T, int K>
__device__ inline void store_row(typename T::storage* p, const float (&f)[K]) {
  Vec<typename T::storage, K> vec;
#pragma unroll
  for (int k = 0; k < K; ++k) vec.v[k] = T::from_float(f[k]);
  *reinterpret_cast<Vec<typename T::storage, K>*>(p) = vec;
}

// acc[k] += W[row j] at this lane's columns, for every set bit j of `bits` (offset `base`).
template <class T, int K>
__device__ inline void add_bits(float (&acc)[K], u64 bits, int base,
                                const typename T::storage* wt, int d, int lane) {
  while (bits != 0) {
    const int j = base + __builtin_ctzll(bits);
    bits &= bits - 1ull;
    float w[K];
    load_row<T, K>(wt + (i64)j * d + lane * K, w);
#pragma unroll
    for (int k = 0; k < K; ++k) acc[k] += w[k];
  }
}

template <class T, int K>
__device__ inline void add_scaled(float (&acc)[K], float x, int j,
                                  const typename T::storage* wt, int d, int lane) {
  float w[K];
  load_row<T, K>(wt + (i64)j * d + lane * K, w);
#pragma unroll
  for (int k = 0; k < K; ++k) acc[k] += x * w[k];
}

// ln[lane's columns] = LayerNorm(v) * w + b of one row held K values a lane over a
// wavefront: fp32 mean and variance (two passes, xor-shuffle sums), rounded to the dtype
// (nn.LayerNorm on the dtype's values; add_layernorm_kernel below and the token kernels'
// fused norm share it, so they give the same bits).
template <class T, int K>
__device__ inline void row_norm(const float (&v)[K], const typename T::storage* w,
                                const typename T::storage* b, float eps, int d, int lane,
                                typename T::storage* ln) {
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) sum += v[k];
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  const float mean = sum / (float)d;
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float c = v[k] - mean;
    sq += c * c;
  }
  for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
  const float rstd = 1.0f / sqrtf(sq / (float)d + eps);
  float wv[K], bv[K], o[K];
  load_row<T, K>(w + lane * K, wv);
  load_row<T, K>(b + lane * K, bv);
#pragma unroll
  for (int k = 0; k < K; ++k) o[k] = (v[k] - mean) * rstd * wv[k] + bv[k];
  store_row<T, K>(ln + lane * K, o);
}

// The token's last two adds and its store; with `norm`, also LayerNorm of the stored
// token into norm.out (the first layer's norm1, as add_layernorm would compute it).
template <class T>
struct TokenNorm {
  const typename T::storage* w;
  const typename T::storage* b;
  float eps;
  typename T::storage* out;  // NULL: no norm
};

template <class T, int K>
__device__ inline void finish(float (&acc)[K], const typename T::storage* position,
                              const typename T::storage* token_type,
                              typename T::storage* out, int d, int lane,
                              const TokenNorm<T>& norm = TokenNorm<T>{}, i64 row = 0) {
  float p[K], t[K], o[K];
  load_row<T, K>(position + lane * K, p);
  load_row<T, K>(token_type + lane * K, t);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float r1 = T::round(acc[k]);
    const float r2 = T::round(r1 + p[k]);
    o[k] = r2 + t[k];
  }
  store_row<T, K>(out + lane * K, o);
  if (norm.out != nullptr) {
    float v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = T::round(o[k]);  // the stored token's values
    row_norm<T, K>(v, norm.w, norm.b, norm.eps, d, lane, norm.out + row * d);
  }
}

// SeqNet.event_token(words, seat, index) (cugo_seq50.py:276-282) with encode_events
// (:91-110) on one event per row: slots played, own drawn (hidden unless the observer
// is the actor), flipped, my/opponent gain, my/opponent loss (seat 0 reads players 0/1
// as my/opponent, seat 1 the other way round), shown; then one-hot kind (clamped to 11),
// the "me" bit and the opponent's hidden draw count; position row 1 + min(index, 47).
template <class T, int K>
__global__ __launch_bounds__(64 * kRowsPerBlock) void event_tokens_kernel(
    const i64* words, i64 word_rows, const i64* seat, const i64* index, i64 n,
    const typename T::storage* wt, const typename T::storage* bias,
    const typename T::storage* position, i64 position_rows,
    const typename T::storage* token_type, int d, typename T::storage* out,
    TokenNorm<T> norm) {
  const int lane = threadIdx.x & 63;
  const i64 r = (i64)blockIdx.x * kRowsPerBlock + uniform(threadIdx.x >> 6);
  if (r >= n) return;
  const i64 wr = r % word_rows;  // one event read for every seat that observes it
  const i64* ev = words + wr * 9;
  const u64 header = (u64)ev[8];
  const i64 s = seat[r];
  const bool me = (i64)(header & 0xFFu) == s;
  const bool first = s == 0;
  const int kind = (int)((header >> 8) & 0xFFu);
  float acc[K];
  load_row<T, K>(bias + lane * K, acc);
  const u64 w3 = (u64)ev[3], w4 = (u64)ev[4], w5 = (u64)ev[5], w6 = (u64)ev[6];
  add_bits<T>(acc, (u64)ev[0] & kCardMask, 0, wt, d, lane);
  if (me) add_bits<T>(acc, (u64)ev[1] & kCardMask, 50, wt, d, lane);
  add_bits<T>(acc, (u64)ev[2] & kCardMask, 100, wt, d, lane);
  add_bits<T>(acc, (first ? w3 : w4) & kCardMask, 150, wt, d, lane);
  add_bits<T>(acc, (first ? w4 : w3) & kCardMask, 200, wt, d, lane);
  add_bits<T>(acc, (first ? w5 : w6) & kCardMask, 250, wt, d, lane);
  add_bits<T>(acc, (first ? w6 : w5) & kCardMask, 300, wt, d, lane);
  add_bits<T>(acc, (u64)ev[7] & kCardMask, 350, wt, d, lane);
  add_bits<T>(acc, 1ull, 400 + (kind < kKinds - 1 ? kind : kKinds - 1), wt, d, lane);
  if (me) {
    add_bits<T>(acc, 1ull, 412, wt, d, lane);
  } else {
    const int drawn = __builtin_popcountll((u64)ev[1] & kCardMask);
    if (drawn != 0) add_scaled<T>(acc, (float)drawn, 413, wt, d, lane);
  }
  i64 p = index[wr];
  p = 1 + (p < kMaxEvents - 1 ? p : kMaxEvents - 1);
  if (p < 0) p = 0;
  if (p >= position_rows) p = position_rows - 1;
  finish<T>(acc, position + p * d, token_type + d, out + r * d, d, lane, norm, r);
}

// SeqNet.start_token(start, seat) (cugo_seq50.py:271-274) with encode_start (:113-128):
// planes of the observer's hand, the floor, own and opponent captures and the mission
// cards, the 12 neutral-month bits, one-hot mission type (clamped to 7), then four
// scalars (multiplier / 4, observer moves first, own and opponent mission months / 8),
// rounded to the token dtype as the reference's `.to(dtype)` does; position row 0.
template <class T, int K>
__global__ __launch_bounds__(64 * kRowsPerBlock) void start_tokens_kernel(
    const i64* start, const i64* seat, i64 n, const typename T::storage* wt,
    const typename T::storage* bias, const typename T::storage* position,
    const typename T::storage* token_type, int d, typename T::storage* out) {
  const int lane = threadIdx.x & 63;
  const i64 r = (i64)blockIdx.x * kRowsPerBlock + uniform(threadIdx.x >> 6);
  if (r >= n) return;
  const i64* st = start + r * 8;
  const i64 s = seat[r];
  const bool first = s == 0;
  const u64 header = (u64)st[7];
  float acc[K];
  load_row<T, K>(bias + lane * K, acc);
  const u64 s0 = (u64)st[0], s1 = (u64)st[1], s3 = (u64)st[3], s4 = (u64)st[4];
  add_bits<T>(acc, (first ? s0 : s1) & kCardMask, 0, wt, d, lane);
  add_bits<T>(acc, (u64)st[2] & kCardMask, 50, wt, d, lane);
  add_bits<T>(acc, (first ? s3 : s4) & kCardMask, 100, wt, d, lane);
  add_bits<T>(acc, (first ? s4 : s3) & kCardMask, 150, wt, d, lane);
  add_bits<T>(acc, (u64)st[5] & kCardMask, 200, wt, d, lane);
  add_bits<T>(acc, (u64)st[6] & 0xFFFull, 250, wt, d, lane);
  const int mtype = (int)(header & 0xFFu);
  add_bits<T>(acc, 1ull, 262 + (mtype < 7 ? mtype : 7), wt, d, lane);
  const float m0 = (float)((header >> 24) & 0xFFu) / 8.0f;
  const float m1 = (float)((header >> 32) & 0xFFu) / 8.0f;
  const float scalars[4] = {(float)((header >> 8) & 0xFFu) / 4.0f,
                            (i64)((header >> 16) & 1u) == s ? 1.0f : 0.0f,
                            first ? m0 : m1, first ? m1 : m0};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float x = T::round(scalars[q]);
    if (x != 0.0f) add_scaled<T>(acc, x, 270 + q, wt, d, lane);
  }
  finish<T>(acc, position, token_type, out + r * d, d, lane);
}

// WaveCollector._step's sampling (cugo_seq_selfplay50.py:125-130) for one row per
// wavefront: masked = legal ? logit : -1e30; action = argmax(masked - log(-log(clamp(u,
// 1e-20, 1)))) with the first index on ties (torch.argmax); logp = log_softmax(masked)
// at the action, computed as (masked[a] - max) - log(sum exp(masked - max)).
// Logits of type T (bf16 logits convert to fp32 exactly, as the reference's `.float()`).
// u == nullptr: no noise, the greedy masked argmax (cugo_eval50.py:125-127).
// Only legal actions need the two logarithms and the exponential: for u < 1 the noise
// lies in [-3.9, 16.7], and -1e30 plus it rounds to -1e30 in fp32 (the spacing there is
// 2^76), so an illegal action's noisy value is -1e30 (+inf when u = 1, where
// -log(-log(1)) = +inf); and its exp(-1e30 - max) is 0 whenever some action is legal.
// A row with no legal action sums exp(0) over every action, as the reference does.
template <class T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void gumbel_kernel(
    const typename T::storage* logits, const uint8_t* legal, const float* u, i64 n,
    int actions_count, i64* actions, float* logp) {
  const int lane = threadIdx.x & 63;
  const i64 r = (i64)blockIdx.x * kRowsPerBlock + uniform(threadIdx.x >> 6);
  if (r >= n) return;
  const typename T::storage* lr = logits + r * actions_count;
  const uint8_t* gr = legal + r * actions_count;
  const float* ur = u != nullptr ? u + r * actions_count : nullptr;
  float best = -INFINITY, top = -INFINITY;
  int best_a = actions_count;  // above every real index
  bool any = false;
  for (int a = lane; a < actions_count; a += 64) {
    const bool ok = gr[a] != 0;
    any |= ok;
    const float m = ok ? T::to_float(lr[a]) : -1.0e30f;
    float v = m;
    if (ur != nullptr) {
      const float uc = fminf(fmaxf(ur[a], 1.0e-20f), 1.0f);
      if (ok) v = m + -logf(-logf(uc));
      else if (uc >= 1.0f) v = INFINITY;
    }
    if (v > best) { best = v; best_a = a; }
    top = fmaxf(top, m);
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off);
    const int oa = __shfl_xor(best_a, off);
    if (ob > best || (ob == best && oa < best_a)) { best = ob; best_a = oa; }
    top = fmaxf(top, __shfl_xor(top, off));
  }
  any = __ballot(any) != 0;
  float sum = 0.0f;
  if (logp != nullptr) {
    for (int a = lane; a < actions_count; a += 64) {
      const bool ok = gr[a] != 0;
      if (ok) sum += expf(T::to_float(lr[a]) - top);
      else if (!any) sum += 1.0f;  // exp(-1e30 - (-1e30))
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  }
  if (lane == 0) {
    const int a = best_a < actions_count ? best_a : 0;
    const float m = gr[a] ? T::to_float(lr[a]) : -1.0e30f;
    actions[r] = a;
    if (logp != nullptr) logp[r] = (m - top) - logf(sum);
  }
}

// Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as 1,
// 2, 3", SC 2011): ten rounds, each mapping the counter (c0, c1, c2, c3) under the key
// (k0, k1) to (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)), the key
// bumped by the Weyl constants between rounds.
struct Philox4 {
  uint32_t x[4];
};
__device__ inline Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                        uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = M0 * c0, hi0 = __umulhi(M0, c0);
    const uint32_t lo1 = M1 * c2, hi1 = __umulhi(M1, c2);
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += W0;
    k1 += W1;
  }
  return {{c0, c1, c2, c3}};
}

// The uniforms of cugo_gumbel_sample_philox: for row r and action a, word (a / 16) % 4 of
// Philox4x32-10 at counter (r mod 2^32, (a % 16) + 64 (a / 64) + 256 (r / 2^32), offset,
// *epoch mod 2^32) under the key (seed mod 2^32, seed / 2^32), as (word >> 8) * 2^-24, in
// [0, 1).  A lane of gumbel_rows_kernel holds actions j + 16 k (k < 12): three counters.
struct PhiloxNoise {
  uint32_t k0, k1, offset;
  const uint64_t* epoch;
  float* u_out;  // if not NULL, the uniforms drawn, [n, A] (for tests)
};

// The same sampling with 16 lanes per row and four rows per wavefront, for rows of at
// most kGumbelLanes * kGumbelPer actions: lane j of a row takes actions j, j + 16, ...,
// issues all of its loads before any arithmetic, and keeps its masked logits in
// registers for the softmax sum, so a row costs one round of memory latency.  Ties and
// the reductions follow gumbel_kernel (the largest value, the first index among equal
// ones); only the order of the fp32 softmax sum differs.  kNoise: 0 no noise (greedy),
// 1 the uniforms u [n, A], 2 uniforms drawn here from Philox (PhiloxNoise).
constexpr int kGumbelLanes = 16;
constexpr int kGumbelPer = 12;  // up to 192 actions
static_assert(kGumbelPer == 12, "a Philox lane draws three blocks of four uniforms");

template <class T, int kNoise>
__global__ __launch_bounds__(256) void gumbel_rows_kernel(
    const typename T::storage* logits, const uint8_t* legal, const float* u, i64 n,
    int actions_count, i64* actions, float* logp, PhiloxNoise px) {
  const int j = threadIdx.x & (kGumbelLanes - 1);
  const i64 r = (i64)blockIdx.x * (256 / kGumbelLanes) + (threadIdx.x / kGumbelLanes);
  const bool row_ok = r < n;
  // Every load is unconditional, at an index clamped into the arrays (a lane past the
  // last row or action reads an element that exists and ignores it), so all of a lane's
  // loads are in flight together instead of each waiting on the legal byte before it.
  const i64 rr = row_ok ? r : n - 1;
  const typename T::storage* lr = logits + rr * actions_count;
  const uint8_t* gr = legal + rr * actions_count;
  const float* ur = kNoise == 1 ? u + rr * actions_count : nullptr;
  uint8_t gb[kGumbelPer];
  typename T::storage lv[kGumbelPer];
  float uv[kGumbelPer];
#pragma unroll
  for (int k = 0; k < kGumbelPer; ++k) {
    const int a = j + kGumbelLanes * k;
    const int ac = a < actions_count ? a : actions_count - 1;
    gb[k] = gr[ac];
    lv[k] = lr[ac];
    uv[k] = kNoise == 1 ? ur[ac] : 0.0f;
  }
  if constexpr (kNoise == 2) {
    const uint32_t epoch = (uint32_t)*px.epoch;
    const uint32_t row_hi = (uint32_t)((uint64_t)rr >> 32) << 8;
#pragma unroll
    for (int g = 0; g < kGumbelPer / 4; ++g) {
      const Philox4 w = philox4x32_10((uint32_t)rr, (uint32_t)(j + 64 * g) + row_hi, px.offset,
                                      epoch, px.k0, px.k1);
#pragma unroll
      for (int q = 0; q < 4; ++q) uv[4 * g + q] = (float)(w.x[q] >> 8) * 0x1.0p-24f;
    }
    if (px.u_out != nullptr && row_ok) {
#pragma unroll
      for (int k = 0; k < kGumbelPer; ++k) {
        const int a = j + kGumbelLanes * k;
        if (a < actions_count) px.u_out[r * actions_count + a] = uv[k];
      }
    }
  }
  bool ok[kGumbelPer];
  float m[kGumbelPer], uc[kGumbelPer];
#pragma unroll
  for (int k = 0; k < kGumbelPer; ++k) {
    const int a = j + kGumbelLanes * k;
    const bool in = row_ok && a < actions_count;
    ok[k] = in && gb[k] != 0;
    m[k] = ok[k] ? T::to_float(lv[k]) : -1.0e30f;
    uc[k] = fminf(fmaxf(uv[k], 1.0e-20f), 1.0f);
  }
  float best = -INFINITY, best_m = -1.0e30f, top = -INFINITY;
  int best_a = 1 << 30;  // above every real index
  bool any = false;
#pragma unroll
  for (int k = 0; k < kGumbelPer; ++k) {
    const int a = j + kGumbelLanes * k;
    if (!row_ok || a >= actions_count) continue;
    any |= ok[k];
    float v = m[k];
    if (kNoise != 0) {
      if (ok[k]) v = m[k] + -logf(-logf(uc[k]));
      else if (uc[k] >= 1.0f) v = INFINITY;
    }
    if (v > best) { best = v; best_a = a; best_m = m[k]; }
    top = fmaxf(top, m[k]);
  }
  for (int off = kGumbelLanes / 2; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off);
    const int oa = __shfl_xor(best_a, off);
    const float om = __shfl_xor(best_m, off);
    if (ob > best || (ob == best && oa < best_a)) { best = ob; best_a = oa; best_m = om; }
    top = fmaxf(top, __shfl_xor(top, off));
    const int other = __shfl_xor((int)any, off);  // every lane takes part in the shuffle
    any = any || other != 0;
  }
  float sum = 0.0f;
  if (logp != nullptr) {
#pragma unroll
    for (int k = 0; k < kGumbelPer; ++k) {
      const int a = j + kGumbelLanes * k;
      if (!row_ok || a >= actions_count) continue;
      if (ok[k]) sum += expf(m[k] - top);
      else if (!any) sum += 1.0f;  // exp(-1e30 - (-1e30))
    }
    for (int off = kGumbelLanes / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  }
  if (j == 0 && row_ok) {
    const bool found = best_a < actions_count;
    actions[r] = found ? best_a : 0;
    const float mv = found ? best_m : m[0];  // lane 0 holds action 0
    if (logp != nullptr) logp[r] = (mv - top) - logf(sum);
  }
}

// ------------------------------------------------------------ step bookkeeping ----
// WaveCollector._step (cugo_seq_selfplay50.py:108-163, no opponent pool) around the
// policy: what it does with torch ops between observe and the query, and after the engine
// step, as two kernels.

constexpr int kFeatures = 720;
constexpr int kActions = 179;
constexpr int kStopPointsColumn = 471;  // cugo_contract50.py:31
constexpr int kRowWords = 31;           // 248-byte state row

// Before the policy (:110-140): bad += active & (status != OK | no legal action); the
// query input row [bf16(features), legal as 0/1] of the policy dtype; the records of step
// step_index (features as bf16, legal, opponent hand = hands word 1 - player of the row,
// stock, stop points = round(exp2(12 f[471]) - 1) (cugo_contract50.py:40-42), seat,
// count, valid = active); and the mover's cache row (player & 1) * w + game.
// One wavefront per game.
template <class T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void prepare_kernel(
    CugoSelfPlayWave wave, const u64* states, const float* features, const uint8_t* legal,
    const uint8_t* player, const uint8_t* done, const int16_t* status, const i64* stock,
    typename T::storage* q_in, i64* query_rows) {
  const int lane = threadIdx.x & 63;
  const i64 i = (i64)blockIdx.x * kRowsPerBlock + uniform(threadIdx.x >> 6);
  const i64 w = wave.w;
  if (i >= w) return;
  if (i == 0 && lane == 0 && wave.playing != nullptr) wave.playing[0] = 0;  // advance sets it
  // this step's index: the one advance left in step_index[1], kept in step_index[0] for
  // advance (no thread here reads [0], none in advance writes it)
  const i64 step = wave.step_index[1];
  if (i == 0 && lane == 0) wave.step_index[0] = step;
  const bool record = step >= 0 && step < wave.max_steps;
  const i64 rec = step * w + i;
  const float* f = features + i * kFeatures;
  const int width = (int)wave.width;
  const int q_stride = wave.q_stride > 0 ? (int)wave.q_stride : width + kActions;
  typename T::storage* q = q_in + i * q_stride;
  for (int j = width + kActions + lane; j < q_stride; j += 64) q[j] = T::from_float(0.0f);
  const bool by4 = wave.columns == nullptr && wave.q_stride > 0 && wave.q_stride % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(q_in) | reinterpret_cast<uintptr_t>(features)) &
                    15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(wave.rec_features) & 7u) == 0;
  if (by4) {
    // every column in order, 4-element aligned rows: a lane converts 4 features at a time
    // (one 16-byte load, 8- or 16-byte stores; width = 720 is a multiple of 4)
    const float4* f4 = reinterpret_cast<const float4*>(f);
    for (int j = lane; j < kFeatures / 4; j += 64) {
      const float4 x = f4[j];
      T::store4(q + 4 * j, x);
      if (record) BF16::store4(wave.rec_features + rec * width + 4 * j, x);
    }
  } else {
    for (int j = lane; j < width; j += 64) {
      const float x = f[wave.columns != nullptr ? wave.columns[j] : j];
      q[j] = T::from_float(x);
      if (record) wave.rec_features[rec * width + j] = BF16::from_float(x);
    }
  }
  const uint8_t* g = legal + i * kActions;
  bool any = false;
  for (int j = lane; j < kActions; j += 64) {
    const uint8_t b = g[j] != 0;
    any |= b;
    q[width + j] = T::from_float(b ? 1.0f : 0.0f);
    if (record) wave.rec_legal[rec * kActions + j] = b;
  }
  any = __ballot(any) != 0;
  if (lane != 0) return;
  const bool active = done[i] == 0;
  if (active && (status[i] != 0 || !any)) atomicAdd(wave.bad, 1ull);
  const i64 p = (i64)player[i];
  query_rows[i] = (p & 1) * w + i;
  // a finished game's query attends nothing (its row is skipped: no cache read or write,
  // a NaN output that nothing uses)
  if (wave.query_pos != nullptr) wave.query_pos[i] = active ? wave.cache_length[(p & 1) * w + i] : -1;
  if (!record) return;
  wave.rec_seat[rec] = p;
  wave.rec_count[rec] = wave.count[i];
  wave.rec_opp_hand[rec] = (i64)states[i * kRowWords + (1 - p)];
  if (stock != nullptr) {
    wave.rec_stock[rec] = stock[i];
  } else {  // stock_indexed's value, from the row in hand (kernels.hip stock_kernel)
    Env e;
    e.stock = states[i * kRowWords + 3];
    e.rng = states[i * kRowWords + 6];
    wave.rec_stock[rec] = (i64)peek_stock(e);
  }
  wave.rec_stop_points[rec] = (i64)rintf(exp2f(12.0f * f[kStopPointsColumn]) - 1.0f);
  // a pool game's decision belongs to the learner only when the learner's seat moves
  wave.rec_valid[rec] = active && (i >= wave.pool_games || p == wave.learner_seat[i]);
}

// cugo_query_input: [features (the kept columns), legal as 0/1] in the policy dtype,
// zero-padded to q_stride columns (SeqNet._query's input, cugo_seq50.py:166-180).  One
// wavefront per row; a column index outside [0, 720) gives NaN (no read outside the row).
template <class T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void query_input_kernel(
    const float* features, const uint8_t* legal, const int32_t* columns, int width,
    int q_stride, i64 n, typename T::storage* q_in) {
  const int lane = threadIdx.x & 63;
  const i64 i = (i64)blockIdx.x * kRowsPerBlock + uniform(threadIdx.x >> 6);
  if (i >= n) return;
  const float* f = features + i * kFeatures;
  typename T::storage* q = q_in + i * q_stride;
  for (int j = lane; j < width; j += 64) {
    const int c = columns != nullptr ? columns[j] : j;  // a column outside the features: NaN
    q[j] = T::from_float(c >= 0 && c < kFeatures ? f[c] : __builtin_nanf(""));
  }
  const uint8_t* g = legal + i * kActions;
  for (int j = lane; j < kActions; j += 64) q[width + j] = T::from_float(g[j] != 0 ? 1.0f : 0.0f);
  for (int j = width + kActions + lane; j < q_stride; j += 64) q[j] = T::from_float(0.0f);
}

// After the engine step (:146-163): bad += active & (step status != OK); a game that
// finished now keeps its reward and nagari flag and is marked finished; a committed
// action's event goes to slot min(count, 47) of the log, and both seats' cache lengths
// and the count advance; the step's action and log-probability are recorded.  One thread
// per game; call after the event tokens were appended (they use the old count).
__global__ __launch_bounds__(256) void advance_kernel(
    CugoSelfPlayWave wave, const uint8_t* done, const float* reward0, const uint8_t* new_done,
    const uint8_t* nagari, const int16_t* step_status, const uint8_t* committed,
    const i64* events, const i64* actions, const float* logp) {
  const i64 w = wave.w;
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0 && wave.noise_epoch != nullptr) wave.noise_epoch[0] += 1;  // read by no one here
  const bool in = i < w;
  const bool active = in && done[i] == 0;
  const u64 bad = __ballot(active && step_status[i] != 0);
  if ((threadIdx.x & 63) == 0 && bad != 0)
    atomicAdd(wave.bad, (unsigned long long)__popcll(bad));
  // a game still being played after this step: the wave goes on (prepare cleared the flag)
  const u64 playing = __ballot(active && new_done[i] == 0);
  if ((threadIdx.x & 63) == 0 && playing != 0 && wave.playing != nullptr) wave.playing[0] = 1;
  if (!in) return;
  if (active && new_done[i]) {
    wave.final_reward0[i] = reward0[i];
    if (nagari[i]) wave.final_nagari[i] = 1;
    wave.finished[i] = 1;
  }
  // The slots of this step's event tokens; an event that is not kept (no committed action,
  // or a game already over) goes nowhere: its row of the next pass is skipped.
  const bool keep = active && committed[i];
  if (wave.event_pos != nullptr) {
    wave.event_pos[i] = keep ? wave.cache_length[i] : -1;
    wave.event_pos[w + i] = keep ? wave.cache_length[w + i] : -1;
  }
  const i64 c = wave.count[i];
  if (keep) {
    const i64 slot = c < kMaxEvents - 1 ? c : kMaxEvents - 1;
    i64* log = wave.events + (i * kMaxEvents + slot) * 9;
    for (int k = 0; k < 9; ++k) log[k] = events[i * 9 + k];
    wave.cache_length[i] += 1;
    wave.cache_length[w + i] += 1;
    if (i < wave.pool_games) wave.opp_cache_length[i] += 1;
    wave.count[i] = c + 1;
  }
  const i64 step = wave.step_index[0];
  if (i == 0) wave.step_index[1] = step + 1;  // the next step's (no thread here reads [1])
  if (step >= 0 && step < wave.max_steps) {
    wave.rec_actions[step * w + i] = actions[i];
    wave.rec_logp[step * w + i] = logp[i];
  }
}

// Paired evaluation on resident games (cugo_eval50.py:137-361 without dropping finished
// games): the bookkeeping of a step around the models and the engine step.  Before the
// step: the observe checks of the active games, the decision-step count, and each game's
// action from the model whose seat moves.  After it: the step check, the final reward and
// nagari flag of games that end now, and the active mask.
__global__ __launch_bounds__(256) void paired_select_kernel(
    const uint8_t* active, const int16_t* status, const uint8_t* done,
    const uint8_t* any_legal, const uint8_t* player, const i64* a_seat, const i64* act_a,
    const i64* act_b, i64 n, i64* actions, i64* bad, int* any_active, int* playing) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0 && playing != nullptr) *playing = 0;  // paired_update sets it
  const bool in = i < n;
  const bool act = in && active[i] != 0;
  const bool fine = in && status[i] == 0;
  const u64 obs_bad = __ballot(act && !fine);
  const u64 legal_bad = __ballot(act && fine && (done[i] != 0 || any_legal[i] == 0));
  const u64 live = __ballot(act);
  if ((threadIdx.x & 63) == 0) {
    if (obs_bad != 0) atomicAdd(reinterpret_cast<unsigned long long*>(bad), (unsigned long long)__popcll(obs_bad));
    if (legal_bad != 0)
      atomicAdd(reinterpret_cast<unsigned long long*>(bad + 1), (unsigned long long)__popcll(legal_bad));
    if (live != 0) *any_active = 1;
  }
  if (in) actions[i] = (i64)player[i] == a_seat[i] ? act_a[i] : act_b[i];
}

__global__ __launch_bounds__(256) void paired_update_kernel(
    uint8_t* active, const int16_t* step_status, const uint8_t* new_done, const float* reward0,
    const uint8_t* nagari, i64 n, float* final_reward0, uint8_t* final_nagari, i64* bad,
    int* any_active, i64* steps, int* playing) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0 && *any_active != 0) {  // one decision step more; the flag is read by no one else
    *steps += 1;
    *any_active = 0;
  }
  const bool in = i < n;
  const bool act = in && active[i] != 0;
  const bool ok = in && step_status[i] == 0;
  const u64 step_bad = __ballot(act && !ok);
  if ((threadIdx.x & 63) == 0 && step_bad != 0)
    atomicAdd(reinterpret_cast<unsigned long long*>(bad + 2), (unsigned long long)__popcll(step_bad));
  // a game still active after the update: the evaluation goes on (paired_select cleared it)
  const u64 left = __ballot(act && ok && new_done[i] == 0);
  if ((threadIdx.x & 63) == 0 && left != 0 && playing != nullptr) *playing = 1;
  if (!act) return;
  if (ok && new_done[i] != 0) {
    final_reward0[i] = reward0[i];
    if (nagari[i] != 0) final_nagari[i] = 1;
  }
  active[i] = ok && new_done[i] == 0;
}

// A paired evaluation's policy answers only for the games whose mover sits in its seat
// (cugo_eval50.py:130-135 feeds each model its movers): the query of every other game is
// skipped by the step's decode (query_pos = -1: no cache read or write, NaN logits that
// nothing reads).  After the observation, before the policy's pass.  One thread per game.
__global__ __launch_bounds__(256) void paired_movers_kernel(const uint8_t* player,
                                                            const i64* seat, i64 n,
                                                            i64* query_pos) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n && (i64)player[i] != seat[i]) query_pos[i] = -1;
}

// The event log of a paired evaluation of sequence policies (History.record,
// cugo_seq50.py:62-67, called at cugo_eval50.py:258-263), kept as each policy's cache
// length: after the engine step and the event tokens (which read the old count), before
// paired_update clears the active flags.  A game's event is kept when the game was active,
// its step is OK and its action committed: its token goes to slot length_m[i] of policy
// m's cache row i at the next step's pass (event_pos_m), and count[i] and every length_m[i]
// advance; any other event's row is skipped at that pass (event_pos_m = -1).  The next
// step's query of a game still playing (active, OK, not finished now) goes to slot
// length_m[i] (query_pos_m); a finished game's query row is skipped (-1).  One thread per
// game.
__global__ __launch_bounds__(256) void paired_events_kernel(
    const uint8_t* active, const int16_t* step_status, const uint8_t* committed,
    const uint8_t* new_done, i64 n, i64* count, i64* length_a, i64* event_pos_a,
    i64* query_pos_a, i64* length_b, i64* event_pos_b, i64* query_pos_b) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const bool live = active[i] != 0 && step_status[i] == 0;
  const bool keep = live && committed[i] != 0;
  const bool next = live && new_done[i] == 0;
  const i64 la = length_a[i];
  event_pos_a[i] = keep ? la : -1;
  query_pos_a[i] = next ? la + (keep ? 1 : 0) : -1;
  if (keep) length_a[i] = la + 1;
  if (length_b != nullptr) {
    const i64 lb = length_b[i];
    event_pos_b[i] = keep ? lb : -1;
    query_pos_b[i] = next ? lb + (keep ? 1 : 0) : -1;
    if (keep) length_b[i] = lb + 1;
  }
  if (keep) count[i] += 1;
}

// Pre-norm transformer residual step (nn.TransformerEncoderLayer with norm_first,
// python/cugo_seq50.py:318-322): x_out = x + y rounded to the dtype (y == nullptr: x_out is
// not written and x is normalised as is), then ln = LayerNorm(x_out) with fp32 mean and
// variance over the row, rounded to the dtype.  One wavefront per row, K = d / 64
// consecutive columns per lane.
template <class T, int K>
__global__ __launch_bounds__(64 * kRowsPerBlock) void add_layernorm_kernel(
    const typename T::storage* x, const typename T::storage* y, const typename T::storage* w,
    const typename T::storage* b, float eps, i64 n, int d, typename T::storage* x_out,
    typename T::storage* ln) {
  const int lane = threadIdx.x & 63;
  const i64 r = (i64)blockIdx.x * kRowsPerBlock + uniform(threadIdx.x >> 6);
  if (r >= n) return;
  const i64 at = r * d + lane * K;
  float v[K];
  load_row<T, K>(x + at, v);
  if (y != nullptr) {
    float u[K];
    load_row<T, K>(y + at, u);
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = T::round(v[k] + u[k]);
    store_row<T, K>(x_out + at, v);
  }
  row_norm<T, K>(v, w, b, eps, d, lane, ln + r * d);
}

template <class T>
int launch_add_layernorm(const void* x, const void* y, const void* w, const void* b, float eps,
                         i64 n, int d, void* x_out, void* ln, hipStream_t stream) {
  using S = typename T::storage;
  const unsigned grid = (unsigned)((n + kRowsPerBlock - 1) / kRowsPerBlock);
#define CUGO_LN_CASE(KK)                                                                    \
  case KK:                                                                                  \
    add_layernorm_kernel<T, KK><<<grid, 64 * kRowsPerBlock, 0, stream>>>(                   \
        (const S*)x, (const S*)y, (const S*)w, (const S*)b, eps, n, d, (S*)x_out, (S*)ln);  \
    break;
  switch (d / 64) {
    CUGO_LN_CASE(1)
    CUGO_LN_CASE(2)
    CUGO_LN_CASE(4)
    CUGO_LN_CASE(8)
    CUGO_LN_CASE(16)
    default:
      return -3;
  }
#undef CUGO_LN_CASE
  return (int)hipGetLastError();
}

template <class T>
int launch_event(const i64* words, i64 word_rows, const i64* seat, const i64* index, i64 n,
                 const void* wt,
                 const void* bias, const void* position, i64 position_rows,
                 const void* token_type, int d, void* out, const void* ln_w, const void* ln_b,
                 float eps, void* ln, hipStream_t stream) {
  using S = typename T::storage;
  const unsigned grid = (unsigned)((n + kRowsPerBlock - 1) / kRowsPerBlock);
  const TokenNorm<T> norm{(const S*)ln_w, (const S*)ln_b, eps, (S*)ln};
#define CUGO_EVENT_CASE(KK)                                                                 \
  case KK:                                                                                  \
    event_tokens_kernel<T, KK><<<grid, 64 * kRowsPerBlock, 0, stream>>>(                    \
        words, word_rows, seat, index, n, (const S*)wt, (const S*)bias, (const S*)position, \
        position_rows, (const S*)token_type, d, (S*)out, norm);                             \
    break;
  switch (d / 64) {
    CUGO_EVENT_CASE(1)
    CUGO_EVENT_CASE(2)
    CUGO_EVENT_CASE(4)
    CUGO_EVENT_CASE(8)
    CUGO_EVENT_CASE(16)
    default:
      return -3;
  }
#undef CUGO_EVENT_CASE
  return (int)hipGetLastError();
}

template <class T>
int launch_start(const i64* start, const i64* seat, i64 n, const void* wt, const void* bias,
                 const void* position, const void* token_type, int d, void* out,
                 hipStream_t stream) {
  using S = typename T::storage;
  const unsigned grid = (unsigned)((n + kRowsPerBlock - 1) / kRowsPerBlock);
#define CUGO_START_CASE(KK)                                                                 \
  case KK:                                                                                  \
    start_tokens_kernel<T, KK><<<grid, 64 * kRowsPerBlock, 0, stream>>>(                    \
        start, seat, n, (const S*)wt, (const S*)bias, (const S*)position,                   \
        (const S*)token_type, d, (S*)out);                                                  \
    break;
  switch (d / 64) {
    CUGO_START_CASE(1)
    CUGO_START_CASE(2)
    CUGO_START_CASE(4)
    CUGO_START_CASE(8)
    CUGO_START_CASE(16)
    default:
      return -3;
  }
#undef CUGO_START_CASE
  return (int)hipGetLastError();
}

bool valid_width(int64_t d) {
  return d == 64 || d == 128 || d == 256 || d == 512 || d == 1024;
}

// Every row pointer must allow the (d / 64)-element accesses of load_row / store_row.
bool aligned_rows(int dtype, int64_t d, std::initializer_list<const void*> ptrs) {
  const uintptr_t bytes = (uintptr_t)(d / 64) * (dtype == CUGO_DTYPE_F32 ? 4u : 2u);
  for (const void* p : ptrs)
    if (p != nullptr && (reinterpret_cast<uintptr_t>(p) % bytes) != 0) return false;
  return true;
}

}  // namespace tokens
}  // namespace cugo_amd

using namespace cugo_amd::tokens;

extern "C" {

int cugo_event_tokens(int dtype, const int64_t* words, int64_t word_rows, const int64_t* seat,
                      const int64_t* index, int64_t n, const void* weight_t, const void* bias,
                      const void* position, int64_t position_rows, const void* token_type,
                      int64_t d, void* out, const void* ln_weight, const void* ln_bias,
                      float eps, void* ln, hipStream_t stream) {
  if (n < 0 || position_rows < 1 || (n > 0 && (word_rows < 1 || n % word_rows != 0)) ||
      (n > 0 && (!words || !seat || !index || !weight_t || !bias || !position ||
                 !token_type || !out)) ||
      (ln != nullptr && (!ln_weight || !ln_bias)))
    return -1;
  if (!valid_width(d)) return -3;
  if (!aligned_rows(dtype, d, {weight_t, bias, position, token_type, out, ln_weight, ln_bias, ln}))
    return -4;
  if (n == 0) return 0;
  if (dtype == CUGO_DTYPE_BF16)
    return launch_event<BF16>(words, word_rows, seat, index, n, weight_t, bias, position,
                              position_rows, token_type, (int)d, out, ln_weight, ln_bias, eps,
                              ln, stream);
  if (dtype == CUGO_DTYPE_F32)
    return launch_event<F32>(words, word_rows, seat, index, n, weight_t, bias, position,
                             position_rows, token_type, (int)d, out, ln_weight, ln_bias, eps, ln,
                             stream);
  return -2;
}

int cugo_start_tokens(int dtype, const int64_t* start, const int64_t* seat, int64_t n,
                      const void* weight_t, const void* bias, const void* position,
                      const void* token_type, int64_t d, void* out, hipStream_t stream) {
  if (n < 0 ||
      (n > 0 && (!start || !seat || !weight_t || !bias || !position || !token_type || !out)))
    return -1;
  if (!valid_width(d)) return -3;
  if (!aligned_rows(dtype, d, {weight_t, bias, position, token_type, out})) return -4;
  if (n == 0) return 0;
  if (dtype == CUGO_DTYPE_BF16)
    return launch_start<BF16>(start, seat, n, weight_t, bias, position, token_type, (int)d,
                              out, stream);
  if (dtype == CUGO_DTYPE_F32)
    return launch_start<F32>(start, seat, n, weight_t, bias, position, token_type, (int)d,
                             out, stream);
  return -2;
}

int cugo_add_layernorm(int dtype, const void* x, const void* y, const void* weight,
                       const void* bias, float eps, int64_t n, int64_t d, void* x_out, void* ln,
                       hipStream_t stream) {
  if (n < 0 || (n > 0 && (!x || !weight || !bias || !ln || (y && !x_out)))) return -1;
  if (!valid_width(d)) return -3;
  if (!aligned_rows(dtype, d, {x, y, weight, bias, x_out, ln})) return -4;
  if (n == 0) return 0;
  if (dtype == CUGO_DTYPE_BF16)
    return launch_add_layernorm<BF16>(x, y, weight, bias, eps, n, (int)d, x_out, ln, stream);
  if (dtype == CUGO_DTYPE_F32)
    return launch_add_layernorm<F32>(x, y, weight, bias, eps, n, (int)d, x_out, ln, stream);
  return -2;
}

int cugo_gumbel_sample(int logits_dtype, const void* logits, const uint8_t* legal,
                       const float* uniforms, int64_t n, int64_t actions_count, int64_t* actions,
                       float* logp, hipStream_t stream) {
  if (n < 0 || actions_count < 1 || actions_count > (1 << 20) ||
      (n > 0 && (!logits || !legal || !actions)))
    return -1;
  if (n == 0) return 0;
  if (logits_dtype != CUGO_DTYPE_F32 && logits_dtype != CUGO_DTYPE_BF16) return -2;
  const bool f32 = logits_dtype == CUGO_DTYPE_F32;
  if (actions_count <= kGumbelLanes * kGumbelPer) {
    const unsigned grid = (unsigned)((n + 256 / kGumbelLanes - 1) / (256 / kGumbelLanes));
#define CUGO_GUMBEL_ROWS(TT, NOISE, PTR)                                                   \
  gumbel_rows_kernel<TT, NOISE><<<grid, 256, 0, stream>>>(                                  \
      (PTR)logits, legal, uniforms, n, (int)actions_count, actions, logp, PhiloxNoise{})
    if (f32 && uniforms) CUGO_GUMBEL_ROWS(F32, 1, const float*);
    else if (f32) CUGO_GUMBEL_ROWS(F32, 0, const float*);
    else if (uniforms) CUGO_GUMBEL_ROWS(BF16, 1, const uint16_t*);
    else CUGO_GUMBEL_ROWS(BF16, 0, const uint16_t*);
#undef CUGO_GUMBEL_ROWS
    return (int)hipGetLastError();
  }
  const unsigned grid = (unsigned)((n + kRowsPerBlock - 1) / kRowsPerBlock);
  if (f32)
    gumbel_kernel<F32><<<grid, 64 * kRowsPerBlock, 0, stream>>>(
        (const float*)logits, legal, uniforms, n, (int)actions_count, actions, logp);
  else
    gumbel_kernel<BF16><<<grid, 64 * kRowsPerBlock, 0, stream>>>(
        (const uint16_t*)logits, legal, uniforms, n, (int)actions_count, actions, logp);
  return (int)hipGetLastError();
}

int cugo_gumbel_sample_philox(int logits_dtype, const void* logits, const uint8_t* legal,
                              uint64_t seed, const uint64_t* epoch, uint32_t offset, int64_t n,
                              int64_t actions_count, int64_t* actions, float* logp,
                              float* uniforms_out, hipStream_t stream) {
  if (n < 0 || actions_count < 1 || actions_count > kGumbelLanes * kGumbelPer ||
      (n > 0 && (!logits || !legal || !actions || !epoch)))
    return -1;
  if (n == 0) return 0;
  if (logits_dtype != CUGO_DTYPE_F32 && logits_dtype != CUGO_DTYPE_BF16) return -2;
  const PhiloxNoise px{(uint32_t)seed, (uint32_t)(seed >> 32), offset, epoch, uniforms_out};
  const unsigned grid = (unsigned)((n + 256 / kGumbelLanes - 1) / (256 / kGumbelLanes));
  if (logits_dtype == CUGO_DTYPE_F32)
    gumbel_rows_kernel<F32, 2><<<grid, 256, 0, stream>>>(
        (const float*)logits, legal, nullptr, n, (int)actions_count, actions, logp, px);
  else
    gumbel_rows_kernel<BF16, 2><<<grid, 256, 0, stream>>>(
        (const uint16_t*)logits, legal, nullptr, n, (int)actions_count, actions, logp, px);
  return (int)hipGetLastError();
}

int cugo_selfplay_prepare(const CugoSelfPlayWave* wave, int q_dtype, const uint8_t* states,
                          const float* features, const uint8_t* legal, const uint8_t* player,
                          const uint8_t* done, const int16_t* status, const int64_t* stock,
                          void* q_in, int64_t* query_rows, hipStream_t stream) {
  if (!wave || wave->w < 0 || wave->max_steps < 0 || wave->width < 1 ||
      wave->width > kFeatures || (wave->columns == nullptr && wave->width != kFeatures) ||
      wave->pool_games < 0 || wave->pool_games > wave->w ||
      (wave->pool_games > 0 && !wave->learner_seat) ||
      (wave->q_stride != 0 && wave->q_stride < wave->width + kActions))
    return -1;
  const int64_t w = wave->w;
  if (w > 0 && (!states || !features || !legal || !player || !done || !status ||
                !q_in || !query_rows || !wave->step_index || !wave->count || !wave->bad ||
                !wave->rec_features || !wave->rec_legal || !wave->rec_opp_hand ||
                !wave->rec_stock || !wave->rec_stop_points || !wave->rec_seat ||
                !wave->rec_count || !wave->rec_valid))
    return -1;
  if (w == 0) return 0;
  const unsigned grid = (unsigned)((w + kRowsPerBlock - 1) / kRowsPerBlock);
  if (q_dtype == CUGO_DTYPE_BF16)
    prepare_kernel<BF16><<<grid, 64 * kRowsPerBlock, 0, stream>>>(
        *wave, reinterpret_cast<const u64*>(states), features, legal, player, done, status,
        stock, (uint16_t*)q_in, query_rows);
  else if (q_dtype == CUGO_DTYPE_F32)
    prepare_kernel<F32><<<grid, 64 * kRowsPerBlock, 0, stream>>>(
        *wave, reinterpret_cast<const u64*>(states), features, legal, player, done, status,
        stock, (float*)q_in, query_rows);
  else
    return -2;
  return (int)hipGetLastError();
}

int cugo_query_input(int q_dtype, const float* features, const uint8_t* legal,
                     const int32_t* columns, int64_t width, int64_t n, void* q_in,
                     int64_t q_stride, hipStream_t stream) {
  if (n < 0 || width < 1 || width > kFeatures || (columns == nullptr && width != kFeatures) ||
      q_stride < width + kActions || q_stride > (1 << 16) ||
      (n > 0 && (!features || !legal || !q_in)))
    return -1;
  if (n == 0) return 0;
  const unsigned grid = (unsigned)((n + kRowsPerBlock - 1) / kRowsPerBlock);
  if (q_dtype == CUGO_DTYPE_BF16)
    query_input_kernel<BF16><<<grid, 64 * kRowsPerBlock, 0, stream>>>(
        features, legal, columns, (int)width, (int)q_stride, n, (uint16_t*)q_in);
  else if (q_dtype == CUGO_DTYPE_F32)
    query_input_kernel<F32><<<grid, 64 * kRowsPerBlock, 0, stream>>>(
        features, legal, columns, (int)width, (int)q_stride, n, (float*)q_in);
  else
    return -2;
  return (int)hipGetLastError();
}

int cugo_paired_select(const uint8_t* active, const int16_t* status, const uint8_t* done,
                       const uint8_t* any_legal, const uint8_t* player, const int64_t* a_seat,
                       const int64_t* act_a, const int64_t* act_b, int64_t n, int64_t* actions,
                       int64_t* bad, int32_t* any_active, int32_t* playing,
                       hipStream_t stream) {
  if (n < 0 || (n > 0 && (!active || !status || !done || !any_legal || !player || !a_seat ||
                          !act_a || !act_b || !actions || !bad || !any_active)))
    return -1;
  if (n == 0) return 0;
  paired_select_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
      active, status, done, any_legal, player, a_seat, act_a, act_b, n, actions, bad,
      any_active, playing);
  return (int)hipGetLastError();
}

int cugo_paired_update(uint8_t* active, const int16_t* step_status, const uint8_t* new_done,
                       const float* reward0, const uint8_t* nagari, int64_t n,
                       float* final_reward0, uint8_t* final_nagari, int64_t* bad,
                       int32_t* any_active, int64_t* steps, int32_t* playing,
                       hipStream_t stream) {
  if (n < 0 || !bad || !any_active || !steps ||
      (n > 0 && (!active || !step_status || !new_done || !reward0 || !nagari || !final_reward0 ||
                 !final_nagari)))
    return -1;
  paired_update_kernel<<<(unsigned)((n + 255) / 256 > 0 ? (n + 255) / 256 : 1), 256, 0, stream>>>(
      active, step_status, new_done, reward0, nagari, n, final_reward0, final_nagari, bad,
      any_active, steps, playing);
  return (int)hipGetLastError();
}

int cugo_paired_movers(const uint8_t* player, const int64_t* seat, int64_t n,
                       int64_t* query_pos, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!player || !seat || !query_pos))) return -1;
  if (n == 0) return 0;
  paired_movers_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(player, seat, n,
                                                                        query_pos);
  return (int)hipGetLastError();
}

int cugo_paired_events(const uint8_t* active, const int16_t* step_status,
                       const uint8_t* committed, const uint8_t* new_done, int64_t n,
                       int64_t* count, int64_t* length_a, int64_t* event_pos_a,
                       int64_t* query_pos_a, int64_t* length_b, int64_t* event_pos_b,
                       int64_t* query_pos_b, hipStream_t stream) {
  const bool has_b = length_b != nullptr;
  if (n < 0 || (n > 0 && (!active || !step_status || !committed || !new_done || !count ||
                          !length_a || !event_pos_a || !query_pos_a)) ||
      (event_pos_b != nullptr) != has_b || (query_pos_b != nullptr) != has_b)
    return -1;
  if (n == 0) return 0;
  paired_events_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
      active, step_status, committed, new_done, n, count, length_a, event_pos_a, query_pos_a,
      length_b, event_pos_b, query_pos_b);
  return (int)hipGetLastError();
}

int cugo_selfplay_advance(const CugoSelfPlayWave* wave, const uint8_t* done,
                          const float* reward0, const uint8_t* new_done, const uint8_t* nagari,
                          const int16_t* step_status, const uint8_t* committed,
                          const int64_t* events, const int64_t* actions, const float* logp,
                          hipStream_t stream) {
  if (!wave || wave->w < 0 || wave->max_steps < 0 || wave->pool_games < 0 ||
      wave->pool_games > wave->w || (wave->pool_games > 0 && !wave->opp_cache_length))
    return -1;
  const int64_t w = wave->w;
  if (w > 0 && (!done || !reward0 || !new_done || !nagari || !step_status || !committed ||
                !events || !actions || !logp || !wave->step_index || !wave->count ||
                !wave->events || !wave->cache_length || !wave->final_reward0 ||
                !wave->final_nagari || !wave->finished || !wave->bad || !wave->rec_actions ||
                !wave->rec_logp))
    return -1;
  if (w == 0) return 0;
  advance_kernel<<<(unsigned)((w + 255) / 256), 256, 0, stream>>>(
      *wave, done, reward0, new_done, nagari, step_status, committed, events, actions, logp);
  return (int)hipGetLastError();
}

}  // extern "C"
