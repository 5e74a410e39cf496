// Single-query decode attention over a per-row KV cache, for gfx950.
//
// Reference: python/cugo_seq_attention50.py:21-62 (`decode_attention`: Triton kernel with
// a two-matmul fallback) and its caller python/cugo_seq50.py:291-322 (`cached_step`: the
// new key/value is written to slot `length[row]` with index_put_, then the query attends
// slots 0..pos of its row).
//
//   out[i, h, :] = sum_t softmax_t(q[i,h,:] . K[r,h,t,:] * scale) V[r,h,t,:],
//   r = rows[i], t = 0 .. min(pos[i], slots - 1)
//
// The work is a memory stream: every (query, head) reads (pos + 1) key and value rows
// of dh elements once, and does ~2 flops per byte.  Layout of the work:
//   * a 64-lane wavefront serves G consecutive heads of one query (64 / G lanes each):
//     up to 8, so the wavefront count drops by G and each wavefront keeps its heads'
//     loads in flight together (pick_group); a
//     256-thread workgroup holds four wavefronts, which for heads % (4 G) == 0 share the
//     query and so the sequence length;
//   * a slot row of dh elements is split into 16-byte parts; L = dh*elem/16 lanes hold
//     one slot and a head's lanes cover S = 64/(G L) consecutive slots per load
//     instruction (1 KiB of contiguous cache per instruction at G = 1);
//   * U = 8 such loads of K and of V are issued before any math (16 KiB in flight per
//     wave), the last partial chunk as one masked set of U loads; then scores are
//     reduced over the L lanes of a slot;
//   * softmax is online (running max / sum per lane group, base-2 exponentials with
//     log2(e) folded into the scale) and the S lane groups merge their partial
//     (max, sum, accumulator) triples with a log-sum-exp butterfly at the end.
// CUGO_DECODE_FORCE_GROUP (a compile-time define) pins G for tuning builds.
// Arithmetic is fp32 throughout, output rounded to the query's dtype (as the Triton
// kernel does, cugo_seq_attention50.py:31-40).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/cugo_hip.h"

namespace cugo_amd {
namespace decode {

struct BF16 {
  using storage = uint16_t;
  __device__ static float to_float(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
  // Round to nearest even; NaN stays a quiet NaN (the conversion torch uses).
  __device__ static uint16_t from_float(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  // 16 bytes -> 8 floats.
  __device__ static void unpack(const uint4& r, float* f) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

struct F16 {
  using storage = _Float16;
  __device__ static float to_float(_Float16 x) { return (float)x; }
  __device__ static _Float16 from_float(float f) { return (_Float16)f; }
  __device__ static void unpack(const uint4& r, float* f) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
      f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
  }
};

struct F32 {
  using storage = float;
  __device__ static float to_float(float x) { return x; }
  __device__ static float from_float(float f) { return f; }
  __device__ static void unpack(const uint4& r, float* f) {
    f[0] = __uint_as_float(r.x);
    f[1] = __uint_as_float(r.y);
    f[2] = __uint_as_float(r.z);
    f[3] = __uint_as_float(r.w);
  }
};

constexpr float kNegInf = -__builtin_inff();
constexpr int kWaves = 4;   // wavefronts per workgroup
constexpr int kUnroll = 8;  // loads of K (and of V) in flight per lane

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// exp2(a - b) for a running maximum `a` that may still be -inf (empty so far).
__device__ inline float rescale(float a, float b) { return a == kNegInf ? 0.f : exp2_fast(a - b); }

template <int L>
__device__ inline float reduce_lanes(float s) {
#pragma unroll
  for (int off = 1; off < L; off <<= 1) s += __shfl_xor(s, off, 64);
  return s;
}

// G (query, head) pairs per wavefront, consecutive heads of one query: W = 64 / G lanes
// per head.  G = 1 streams long rows (16 slots of dh = 32 bf16 per load per head); a larger
// G serves short rows (a 50-slot cache) with fewer wavefronts, each issuing the loads of
// all its heads at once.
template <class QT, class KT, int DH, bool APPEND, int G, int U = kUnroll>
__global__ __launch_bounds__(64 * kWaves) void decode_kernel(
    const typename QT::storage* __restrict__ q, typename KT::storage* __restrict__ keys,
    typename KT::storage* __restrict__ values, const typename KT::storage* __restrict__ k_new,
    const typename KT::storage* __restrict__ v_new, const int64_t* __restrict__ pos_in,
    const int64_t* __restrict__ rows, typename QT::storage* __restrict__ out, int64_t groups,
    int heads, int64_t slots, int64_t cache_rows, float scale_log2, int64_t q_stride,
    int64_t new_stride) {
  using KS = typename KT::storage;
  constexpr int E = 16 / (int)sizeof(KS);  // elements per 16-byte part
  constexpr int L = DH / E;                // lanes per slot
  constexpr int W = 64 / G;                // lanes per head
  constexpr int S = W / L;                 // slots per wavefront load, per head
  static_assert(DH % E == 0 && L >= 1 && L <= 64 && (L & (L - 1)) == 0, "unsupported dh");
  static_assert(G >= 1 && (G & (G - 1)) == 0 && W % L == 0 && S >= 1, "unsupported grouping");

  const int lane = threadIdx.x & 63;
  const int64_t group = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (group >= groups) return;  // uniform over the wavefront
  const int64_t pair0 = group * G;
  const int64_t query = pair0 / heads;
  const int64_t pair = pair0 + lane / W;
  const int head = (int)(pair - query * heads);
  const int sub = lane % L;         // which 16-byte part of a slot row
  const int srow = (lane % W) / L;  // which slot of a load
  const int64_t row = rows ? rows[query] : query;
  int64_t pos = pos_in[query];
  typename QT::storage* o = out + pair * DH + sub * E;

  if (row < 0 || row >= cache_rows || pos < 0) {
    // No slot to attend (the reference's softmax over an all -inf row is NaN) or a row
    // outside the cache: the output is NaN and nothing is read or written.
    if (srow == 0) {
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = QT::from_float(__builtin_nanf(""));
    }
    return;
  }
  if (pos >= slots) pos = slots - 1;

  const size_t base = ((size_t)row * heads + head) * (size_t)slots * DH + sub * E;
  const KS* kb = keys + base;
  const KS* vb = values + base;

  float qv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) qv[e] = QT::to_float(q[query * q_stride + head * DH + sub * E + e]);

  float m = kNegInf, l = 0.f, acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;

  int64_t limit = pos + 1;  // cache slots read: [0, limit)
  if constexpr (APPEND) {
    // The new key/value goes to slot `pos` (cugo_seq50.py:317-318) and is attended from
    // registers; the cache loop reads slots [0, pos).
    limit = pos;
    const int64_t at = query * new_stride + head * DH + sub * E;
    const uint4 kn = *reinterpret_cast<const uint4*>(k_new + at);
    const uint4 vn = *reinterpret_cast<const uint4*>(v_new + at);
    if (srow == 0) {
      *reinterpret_cast<uint4*>(keys + base + (size_t)pos * DH) = kn;
      *reinterpret_cast<uint4*>(values + base + (size_t)pos * DH) = vn;
    }
    float kf[E], vf[E];
    KT::unpack(kn, kf);
    KT::unpack(vn, vf);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) s = __builtin_fmaf(qv[e], kf[e], s);
    s = reduce_lanes<L>(s) * scale_log2;
    if (srow == 0) {
      m = s;
      l = 1.f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = vf[e];
    }
  }

  int64_t c = 0;
  // Full chunks: U loads of S slots each, every slot valid.
  for (; c + (int64_t)S * U <= limit; c += (int64_t)S * U) {
    uint4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t off = (size_t)(c + u * S + srow) * DH;
      kr[u] = *reinterpret_cast<const uint4*>(kb + off);
      vr[u] = *reinterpret_cast<const uint4*>(vb + off);
    }
    float s[U];
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kf[E];
      KT::unpack(kr[u], kf);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) d = __builtin_fmaf(qv[e], kf[e], d);
      s[u] = reduce_lanes<L>(d) * scale_log2;
      mx = fmaxf(mx, s[u]);
    }
    const float mn = fmaxf(m, mx);
    const float alpha = rescale(m, mn);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float p = exp2_fast(s[u] - mn);
      l += p;
      float vf[E];
      KT::unpack(vr[u], vf);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = __builtin_fmaf(p, vf[e], acc[e]);
    }
    m = mn;
  }
  // Tail: one masked chunk of U loads (slots >= limit skipped), so a short row costs one
  // round trip to memory rather than one per S slots.
  if (c < limit) {
    uint4 kr[U], vr[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t slot = c + u * S + srow;
      valid[u] = slot < limit;  // uniform over a slot's L lanes
      kr[u] = make_uint4(0, 0, 0, 0);
      vr[u] = make_uint4(0, 0, 0, 0);
      if (valid[u]) {
        kr[u] = *reinterpret_cast<const uint4*>(kb + (size_t)slot * DH);
        vr[u] = *reinterpret_cast<const uint4*>(vb + (size_t)slot * DH);
      }
    }
    float s[U];
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kf[E];
      KT::unpack(kr[u], kf);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) d = __builtin_fmaf(qv[e], kf[e], d);
      // every lane takes part in the shuffles, valid or not
      const float r = reduce_lanes<L>(d) * scale_log2;
      s[u] = valid[u] ? r : kNegInf;
      mx = fmaxf(mx, s[u]);
    }
    const float mn = fmaxf(m, mx);
    const float alpha = rescale(m, mn);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float p = valid[u] ? exp2_fast(s[u] - mn) : 0.f;
      l += p;
      float vf[E];
      KT::unpack(vr[u], vf);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = __builtin_fmaf(p, vf[e], acc[e]);
    }
    m = mn;
  }

  // Merge the S slot groups of each head (lanes with the same `sub`): log-sum-exp
  // butterfly inside the head's W lanes.
#pragma unroll
  for (int off = L; off < W; off <<= 1) {
    const float mo = __shfl_xor(m, off, 64);
    const float lo = __shfl_xor(l, off, 64);
    const float mn = fmaxf(m, mo);
    const float a = rescale(m, mn);
    const float b = rescale(mo, mn);
    l = l * a + lo * b;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float ao = __shfl_xor(acc[e], off, 64);
      acc[e] = acc[e] * a + ao * b;
    }
    m = mn;
  }
  if (srow == 0) {
    const float inv = 1.f / l;
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = QT::from_float(acc[e] * inv);
  }
}

template <class QT, class KT, int DH, bool APPEND, int G>
int launch_group(const void* q, void* keys, void* values, const void* k_new, const void* v_new,
                 const int64_t* pos, const int64_t* rows, void* out, int64_t n, int64_t heads,
                 int64_t slots, int64_t cache_rows, float scale, int64_t q_stride,
                 int64_t new_stride, hipStream_t stream) {
  using QS = typename QT::storage;
  using KS = typename KT::storage;
  const int64_t groups = n * heads / G;
  const int64_t blocks = (groups + kWaves - 1) / kWaves;
  const float scale_log2 = scale * 1.4426950408889634f;  // softmax in base 2
  hipLaunchKernelGGL((decode_kernel<QT, KT, DH, APPEND, G>), dim3((unsigned)blocks),
                     dim3(64 * kWaves), 0, stream, static_cast<const QS*>(q),
                     static_cast<KS*>(keys), static_cast<KS*>(values),
                     static_cast<const KS*>(k_new), static_cast<const KS*>(v_new), pos, rows,
                     static_cast<QS*>(out), groups, (int)heads, slots, cache_rows, scale_log2,
                     q_stride, new_stride);
  return (int)hipGetLastError();
}

// Heads per wavefront.  Measured on MI355X (4,096 queries x 8 heads, dh 32 bf16): rows of
// up to ~50 slots run 2-2.5x faster with 8 heads per wavefront than with one (fewer
// wavefronts, each with all its loads in flight), and on a 320-slot cache 8 beats 2 both
// for one game's rows (mean 20 slots: 18.5 against 23.5 us) and for full rows (mean 297:
// 219 against 223 us).  So: up to 8, whatever the capacity (a grouping must divide
// `heads` and fit G * L <= 64 lanes).
template <int L>
int pick_group(int64_t heads, int64_t slots) {
#ifdef CUGO_DECODE_FORCE_GROUP
  if (heads % CUGO_DECODE_FORCE_GROUP == 0 && CUGO_DECODE_FORCE_GROUP * L <= 64)
    return CUGO_DECODE_FORCE_GROUP;
#endif
  (void)slots;  // the row lengths, not the capacity, decide, and they are not known here
  const int want = 8;
  int best = 1;
  for (int g = 2; g <= want; g <<= 1)
    if (heads % g == 0 && g * L <= 64) best = g;
  return best;
}

template <class QT, class KT, int DH, bool APPEND>
int launch(const void* q, void* keys, void* values, const void* k_new, const void* v_new,
           const int64_t* pos, const int64_t* rows, void* out, int64_t n, int64_t heads,
           int64_t slots, int64_t cache_rows, float scale, int64_t q_stride, int64_t new_stride,
           hipStream_t stream) {
  constexpr int L = DH / (16 / (int)sizeof(typename KT::storage));
  switch (pick_group<L>(heads, slots)) {
#define CUGO_GROUP(GG)                                                                        \
  case GG:                                                                                    \
    if constexpr (GG * L <= 64)                                                               \
      return launch_group<QT, KT, DH, APPEND, GG>(q, keys, values, k_new, v_new, pos, rows,   \
                                                  out, n, heads, slots, cache_rows, scale,    \
                                                  q_stride, new_stride, stream);              \
    return -3;
    CUGO_GROUP(2)
    CUGO_GROUP(4)
    CUGO_GROUP(8)
#undef CUGO_GROUP
    default:
      return launch_group<QT, KT, DH, APPEND, 1>(q, keys, values, k_new, v_new, pos, rows, out,
                                                 n, heads, slots, cache_rows, scale, q_stride,
                                                 new_stride, stream);
  }
}

template <class QT, class KT, bool APPEND>
int by_dh(int64_t dh, const void* q, void* keys, void* values, const void* k_new,
          const void* v_new, const int64_t* pos, const int64_t* rows, void* out, int64_t n,
          int64_t heads, int64_t slots, int64_t cache_rows, float scale, int64_t q_stride,
          int64_t new_stride, hipStream_t stream) {
  switch (dh) {
#define CUGO_DH(D)                                                                       \
  case D:                                                                                \
    if constexpr (16 / sizeof(typename KT::storage) <= D)                                \
      return launch<QT, KT, D, APPEND>(q, keys, values, k_new, v_new, pos, rows, out, n, \
                                       heads, slots, cache_rows, scale, q_stride,        \
                                       new_stride, stream);                              \
    return -3;
    CUGO_DH(16)
    CUGO_DH(32)
    CUGO_DH(64)
    CUGO_DH(128)
#undef CUGO_DH
    default:
      return -3;
  }
}

template <bool APPEND>
int dispatch(int q_dtype, int kv_dtype, int64_t dh, const void* q, void* keys, void* values,
             const void* k_new, const void* v_new, const int64_t* pos, const int64_t* rows,
             void* out, int64_t n, int64_t heads, int64_t slots, int64_t cache_rows,
             float scale, int64_t q_stride, int64_t new_stride, hipStream_t stream) {
#define CUGO_KV(QTYPE)                                                                      \
  switch (kv_dtype) {                                                                       \
    case CUGO_DTYPE_BF16:                                                                   \
      return by_dh<QTYPE, BF16, APPEND>(dh, q, keys, values, k_new, v_new, pos, rows, out, \
                                        n, heads, slots, cache_rows, scale, q_stride,      \
                                        new_stride, stream);                               \
    case CUGO_DTYPE_F16:                                                                    \
      return by_dh<QTYPE, F16, APPEND>(dh, q, keys, values, k_new, v_new, pos, rows, out,  \
                                       n, heads, slots, cache_rows, scale, q_stride,       \
                                       new_stride, stream);                                \
    case CUGO_DTYPE_F32:                                                                    \
      return by_dh<QTYPE, F32, APPEND>(dh, q, keys, values, k_new, v_new, pos, rows, out,  \
                                       n, heads, slots, cache_rows, scale, q_stride,       \
                                       new_stride, stream);                                \
    default:                                                                                \
      return -2;                                                                            \
  }
  switch (q_dtype) {
    case CUGO_DTYPE_BF16:
      CUGO_KV(BF16)
    case CUGO_DTYPE_F16:
      CUGO_KV(F16)
    case CUGO_DTYPE_F32:
      CUGO_KV(F32)
    default:
      return -2;
  }
#undef CUGO_KV
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_args(const void* q, const void* keys, const void* values, const int64_t* pos,
               const void* out, int64_t n, int64_t heads, int64_t dh, int64_t slots,
               int64_t cache_rows) {
  if (n < 0 || heads <= 0 || dh <= 0 || slots <= 0 || cache_rows < 0) return -1;
  if (n > 0 && (!q || !keys || !values || !pos || !out)) return -1;
  if (!aligned16(keys) || !aligned16(values)) return -4;
  return 0;
}

}  // namespace decode
}  // namespace cugo_amd

extern "C" {

int cugo_decode_attention(int q_dtype, int kv_dtype, const void* q, int64_t q_stride,
                          const void* keys, const void* values, const int64_t* pos,
                          const int64_t* rows, int64_t n, int64_t heads, int64_t dh,
                          int64_t slots, int64_t cache_rows, float scale, void* out,
                          hipStream_t stream) {
  using namespace cugo_amd::decode;
  const int bad = check_args(q, keys, values, pos, out, n, heads, dh, slots, cache_rows);
  if (bad) return bad;
  if (q_stride < heads * dh) return -1;
  if (n == 0) return 0;
  return dispatch<false>(q_dtype, kv_dtype, dh, q, const_cast<void*>(keys),
                         const_cast<void*>(values), nullptr, nullptr, pos, rows, out, n, heads,
                         slots, cache_rows, scale, q_stride, 0, stream);
}

int cugo_decode_attention_append(int q_dtype, int kv_dtype, const void* q, int64_t q_stride,
                                 const void* k_new, const void* v_new, int64_t new_stride,
                                 void* keys, void* values, const int64_t* pos,
                                 const int64_t* rows, int64_t n, int64_t heads, int64_t dh,
                                 int64_t slots, int64_t cache_rows, float scale, void* out,
                                 hipStream_t stream) {
  using namespace cugo_amd::decode;
  const int bad = check_args(q, keys, values, pos, out, n, heads, dh, slots, cache_rows);
  if (bad) return bad;
  if (n > 0 && (!k_new || !v_new)) return -1;
  if (q_stride < heads * dh || new_stride < heads * dh) return -1;
  const int64_t kv_size = kv_dtype == CUGO_DTYPE_F32 ? 4 : 2;
  if (!aligned16(k_new) || !aligned16(v_new) || (new_stride * kv_size) % 16 != 0) return -4;
  if (n == 0) return 0;
  return dispatch<true>(q_dtype, kv_dtype, dh, q, keys, values, k_new, v_new, pos, rows, out,
                        n, heads, slots, cache_rows, scale, q_stride, new_stride, stream);
}

}  // extern "C"
