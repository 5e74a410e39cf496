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
//     loads in flight together (pick_group);
//   * P wavefronts serve one such group, each taking every P-th chunk of the row's slots,
//     and merge their partial softmaxes through LDS (pick: split_rows): P = 1 on short
//     caches, 2 on long ones, so that long ragged rows do not end a launch alone;
//     a 256-thread workgroup holds four wavefronts (4 / P groups);
//   * a slot row of dh elements is split into 16-byte parts; L = dh*elem/16 lanes hold
//     one slot and a head's lanes cover S = 64/(G L) consecutive slots per load
//     instruction (1 KiB of contiguous cache per instruction at G = 1);
//   * U = 8 such loads of K and of V are issued before any math (16 KiB in flight per
//     wave), the last partial chunk as one masked set of U loads; then scores are
//     reduced over the L lanes of a slot;
//   * softmax is online (running max / sum per lane group, base-2 exponentials with
//     log2(e) folded into the scale) and the S lane groups merge their partial
//     (max, sum, accumulator) triples with a log-sum-exp butterfly at the end; then
//     the P parts' triples merge the same way.
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

// A cache load: non-temporal on the long caches (kStream: P > 1), whose launches stream
// through more cache than the last-level cache holds, and whose plain loads would evict
// what the layer's linear launches keep there.  Measured on the [4, 4,096, 8, 320, 32]
// cache, ms a 4-layer step plain / non-temporal: rows to a uniform target in [1, 320]
// 0.751 / 0.667, rows filled to ~308 slots 1.162 / 1.050, one game a row (~20 slots)
// 0.270 / 0.246 (plain loads on rows of at most 64 slots only: 0.271).  The decode launch
// alone on one layer's cache, us: 141 / 125, 244 / 222, and one game a row 18.9 / 23.5,
// the last-level cache keeping those rows (95 MB) from launch to launch; over the 4
// layers' caches in turn, as the step reads them, one game a row takes 25.6 with plain
// loads on its short rows and 24.2 non-temporal.  Short caches keep plain loads: the
// self-play step's query launch re-reads, from the last-level cache, the rows its event
// launch has just read.
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
template <bool kStream, class T>
__device__ inline uint4 load_slot(const T* p) {
  if constexpr (kStream) {
    const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}

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

// Online softmax state of one lane: running maximum (base 2), sum and accumulator.
template <int E>
struct Partial {
  float m, l, acc[E];
};

// Folds `U` loaded key/value rows (scores already scaled, -inf where masked) into `st`.
template <class KT, int E, int L, int U>
__device__ inline void fold_chunk(Partial<E>& st, const float (&qv)[E], const uint4 (&kr)[U],
                                  const uint4 (&vr)[U], const bool (&valid)[U],
                                  float scale_log2) {
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
  const float mn = fmaxf(st.m, mx);
  const float alpha = rescale(st.m, mn);
  st.l *= alpha;
#pragma unroll
  for (int e = 0; e < E; ++e) st.acc[e] *= alpha;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float p = valid[u] ? exp2_fast(s[u] - mn) : 0.f;
    st.l += p;
    float vf[E];
    KT::unpack(vr[u], vf);
#pragma unroll
    for (int e = 0; e < E; ++e) st.acc[e] = __builtin_fmaf(p, vf[e], st.acc[e]);
  }
  st.m = mn;
}

// a <- a merged with (mo, lo, ao): the log-sum-exp combination of two partial softmaxes.
template <int E>
__device__ inline void merge(Partial<E>& a, float mo, float lo, const float (&ao)[E]) {
  const float mn = fmaxf(a.m, mo);
  const float x = rescale(a.m, mn);
  const float y = rescale(mo, mn);
  a.l = a.l * x + lo * y;
#pragma unroll
  for (int e = 0; e < E; ++e) a.acc[e] = a.acc[e] * x + ao[e] * y;
  a.m = mn;
}

// G (query, head) pairs per group, consecutive heads of one query: W = 64 / G lanes per
// head.  G = 1 streams long rows (16 slots of dh = 32 bf16 per load per head); a larger G
// serves short rows with fewer wavefronts, each issuing the loads of all its heads at once.
// P wavefronts of a workgroup serve one group: wavefront p takes the slot chunks p, p + P,
// p + 2P, ... of the group's row, and the P partial softmaxes merge through LDS.  With P = 1
// a wavefront's work is its row's length, so on ragged rows the longest rows end the launch
// with few loads in flight; with P > 1 a row's chunks spread over P wavefronts and a launch
// holds P times as many, which the dispatcher starts as others finish.
// `order`, when given, is a permutation of the queries: the g-th group of the launch serves
// query order[g / (heads / G)] instead of g / (heads / G).  Which workgroup serves a query
// changes nothing in its result (the same wavefronts in the same roles); the dispatcher
// starts workgroups in index order as others finish, so queries ordered longest first
// (cugo_decode_order) end a ragged launch with short work.
template <class QT, class KT, int DH, bool APPEND, int G, int P, int U = kUnroll>
__global__ __launch_bounds__(64 * kWaves) void decode_kernel(
    const typename QT::storage* __restrict__ q, typename KT::storage* __restrict__ keys,
    typename KT::storage* __restrict__ values, const typename KT::storage* __restrict__ k_new,
    const typename KT::storage* __restrict__ v_new, const int64_t* __restrict__ pos_in,
    const int64_t* __restrict__ rows, const int32_t* __restrict__ order,
    typename QT::storage* __restrict__ out, int64_t groups, int heads, int64_t slots,
    int64_t cache_rows, float scale_log2, int64_t q_stride, int64_t new_stride) {
  using KS = typename KT::storage;
  constexpr int E = 16 / (int)sizeof(KS);  // elements per 16-byte part
  constexpr int L = DH / E;                // lanes per slot
  constexpr int W = 64 / G;                // lanes per head
  constexpr int S = W / L;                 // slots per wavefront load, per head
  constexpr int CH = S * U;                // slots per chunk (U loads)
  static_assert(DH % E == 0 && L >= 1 && L <= 64 && (L & (L - 1)) == 0, "unsupported dh");
  static_assert(G >= 1 && (G & (G - 1)) == 0 && W % L == 0 && S >= 1, "unsupported grouping");
  static_assert(P >= 1 && kWaves % P == 0, "parts must divide the workgroup's wavefronts");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int part = wave % P;
  const int64_t group = (int64_t)blockIdx.x * (kWaves / P) + wave / P;
  const int sub = lane % L;         // which 16-byte part of a slot row
  const int srow = (lane % W) / L;  // which slot of a load
  // Every wavefront runs to the end of the kernel (P > 1 merges after a barrier); `live`
  // says whether this group attends, `nan_out` whether it writes NaN instead.
  bool live = false, nan_out = false;
  Partial<E> st;
  st.m = kNegInf;
  st.l = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) st.acc[e] = 0.f;
  int64_t pair = 0;
  // uniform over the wavefront (and over the group's P wavefronts)
  const int64_t slot_q = group * G / heads;  // the query's place in the launch
  const int64_t n = groups * G / heads;
  const int64_t query = order != nullptr && group < groups ? (int64_t)order[slot_q] : slot_q;
  if (group < groups && query >= 0 && query < n) {  // an order entry outside [0, n): no work
    const int head = (int)(group * G - slot_q * heads) + lane / W;
    pair = query * heads + head;
    const int64_t row = rows ? rows[query] : query;
    int64_t pos = pos_in[query];
    if (row < 0 || row >= cache_rows || pos < 0) {
      // No slot to attend (the reference's softmax over an all -inf row is NaN) or a row
      // outside the cache: the output is NaN and nothing is read or written.
      nan_out = true;
    } else {
      live = true;
      if (pos >= slots) pos = slots - 1;
    }
    // A part whose first chunk lies past the row's cached slots (and that does not append)
    // has nothing to attend: it only takes part in the merge, with an empty state.
    const int64_t cached = APPEND ? pos : pos + 1;
    if (live && ((int64_t)part * CH < cached || (APPEND && part == 0))) {
      const size_t base = ((size_t)row * heads + head) * (size_t)slots * DH + sub * E;
      const KS* kb = keys + base;
      const KS* vb = values + base;
      float qv[E];
#pragma unroll
      for (int e = 0; e < E; ++e)
        qv[e] = QT::to_float(q[query * q_stride + head * DH + sub * E + e]);

      const int64_t limit = cached;  // cache slots read: [0, limit)
      if constexpr (APPEND) {
        // The new key/value goes to slot `pos` (cugo_seq50.py:317-318) and is attended from
        // registers by part 0; the cache loop reads slots [0, pos).
        if (part == 0) {
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
            st.m = s;
            st.l = 1.f;
#pragma unroll
            for (int e = 0; e < E; ++e) st.acc[e] = vf[e];
          }
        }
      }

      int64_t c = (int64_t)part * CH;
      // Full chunks: U loads of S slots each, every slot valid.
      for (; c + CH <= limit; c += (int64_t)P * CH) {
        uint4 kr[U], vr[U];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const size_t off = (size_t)(c + u * S + srow) * DH;
          kr[u] = load_slot<(P > 1)>(kb + off);
          vr[u] = load_slot<(P > 1)>(vb + off);
          valid[u] = true;
        }
        fold_chunk<KT, E, L, U>(st, qv, kr, vr, valid, scale_log2);
      }
      // The row's last, partial chunk (at most one, on one part): one masked set of U
      // loads (slots >= limit skipped), so a short row costs one round trip to memory
      // rather than one per S slots.
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
            kr[u] = load_slot<(P > 1)>(kb + (size_t)slot * DH);
            vr[u] = load_slot<(P > 1)>(vb + (size_t)slot * DH);
          }
        }
        fold_chunk<KT, E, L, U>(st, qv, kr, vr, valid, scale_log2);
      }

      // Merge the S slot groups of each head (lanes with the same `sub`): log-sum-exp
      // butterfly inside the head's W lanes.
#pragma unroll
      for (int off = L; off < W; off <<= 1) {
        const float mo = __shfl_xor(st.m, off, 64);
        const float lo = __shfl_xor(st.l, off, 64);
        float ao[E];
#pragma unroll
        for (int e = 0; e < E; ++e) ao[e] = __shfl_xor(st.acc[e], off, 64);
        merge<E>(st, mo, lo, ao);
      }
    }
  }
  if constexpr (P > 1) {
    // Lanes with srow == 0 hold their head's state for one 16-byte part; parts 1..P-1
    // hand theirs to part 0 through LDS.
    __shared__ float shared_state[kWaves][G * L][E + 2];
    const int slot_idx = (lane / W) * L + sub;
    if (live && part != 0 && srow == 0) {
      float* d = shared_state[wave][slot_idx];
      d[0] = st.m;
      d[1] = st.l;
#pragma unroll
      for (int e = 0; e < E; ++e) d[2 + e] = st.acc[e];
    }
    __syncthreads();
    if (live && part == 0 && srow == 0) {
#pragma unroll
      for (int p = 1; p < P; ++p) {
        const float* d = shared_state[wave + p][slot_idx];
        float ao[E];
#pragma unroll
        for (int e = 0; e < E; ++e) ao[e] = d[2 + e];
        merge<E>(st, d[0], d[1], ao);
      }
    }
  }
  if (part == 0 && srow == 0 && (live || nan_out)) {
    typename QT::storage* o = out + pair * DH + sub * E;
    if (nan_out) {
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = QT::from_float(__builtin_nanf(""));
    } else {
      const float inv = 1.f / st.l;
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] = QT::from_float(st.acc[e] * inv);
    }
  }
}

template <class QT, class KT, int DH, bool APPEND, int G, int P>
int launch_group(const void* q, void* keys, void* values, const void* k_new, const void* v_new,
                 const int64_t* pos, const int64_t* rows, const int32_t* order, void* out,
                 int64_t n, int64_t heads, int64_t slots, int64_t cache_rows, float scale,
                 int64_t q_stride, int64_t new_stride, hipStream_t stream) {
  using QS = typename QT::storage;
  using KS = typename KT::storage;
  const int64_t groups = n * heads / G;
  constexpr int kGroupsPerBlock = kWaves / P;
  const int64_t blocks = (groups + kGroupsPerBlock - 1) / kGroupsPerBlock;
  const float scale_log2 = scale * 1.4426950408889634f;  // softmax in base 2
  hipLaunchKernelGGL((decode_kernel<QT, KT, DH, APPEND, G, P>), dim3((unsigned)blocks),
                     dim3(64 * kWaves), 0, stream, static_cast<const QS*>(q),
                     static_cast<KS*>(keys), static_cast<KS*>(values),
                     static_cast<const KS*>(k_new), static_cast<const KS*>(v_new), pos, rows,
                     order, static_cast<QS*>(out), groups, (int)heads, slots, cache_rows,
                     scale_log2, q_stride, new_stride);
  return (int)hipGetLastError();
}

// Wavefronts per group: P = 2 for caches longer than 64 slots, whose rows may be long and
// ragged, 1 otherwise.  Measured on MI355X at 4,096 queries x 8 heads on a 320-slot cache
// (rows from seeded games; ms per launch for P = 1 / 2 / 4): rows up to a uniform target in
// [1, 320] 0.156 / 0.150 / 0.143, rows filled to ~308 slots 0.241 / 0.233 / 0.232, one
// game a row (~20 slots) 0.0185 / 0.0178 / 0.0212.  Four parts quadruple the wavefronts,
// which short rows pay for in dispatch rounds; two parts are faster on all three.  On the
// self-play policy's 50-slot cache (events then queries of 4,096 games, rows of 0-40
// slots) two parts took the whole decision step from 0.483 to 0.516 ms: one there.
// CUGO_DECODE_FORCE_PARTS (a compile-time define) pins P for tuning builds.
inline bool split_rows(int64_t slots) { return slots > 64; }

template <class QT, class KT, int DH, bool APPEND, int G>
int launch_parts(const void* q, void* keys, void* values, const void* k_new, const void* v_new,
                 const int64_t* pos, const int64_t* rows, const int32_t* order, void* out,
                 int64_t n, int64_t heads, int64_t slots, int64_t cache_rows, float scale,
                 int64_t q_stride, int64_t new_stride, hipStream_t stream) {
#ifdef CUGO_DECODE_FORCE_PARTS
  (void)split_rows;
  return launch_group<QT, KT, DH, APPEND, G, CUGO_DECODE_FORCE_PARTS>(
      q, keys, values, k_new, v_new, pos, rows, order, out, n, heads, slots, cache_rows, scale,
      q_stride, new_stride, stream);
#else
  if (split_rows(slots))
    return launch_group<QT, KT, DH, APPEND, G, 2>(q, keys, values, k_new, v_new, pos, rows,
                                                  order, out, n, heads, slots, cache_rows, scale,
                                                  q_stride, new_stride, stream);
  return launch_group<QT, KT, DH, APPEND, G, 1>(q, keys, values, k_new, v_new, pos, rows, order,
                                                out, n, heads, slots, cache_rows, scale, q_stride,
                                                new_stride, stream);
#endif
}

// Heads per wavefront.  Measured on MI355X (4,096 queries x 8 heads, dh 32 bf16): rows of
// up to ~50 slots run 2-2.5x faster with 8 heads per wavefront than with one (fewer
// wavefronts, each with all its loads in flight), and on a 320-slot cache 8 beats 2 both
// for one game's rows (mean 20 slots: 18.5 against 23.5 us) and for full rows (mean 297:
// 219 against 223 us), and 4 loses to 8 on every set (one game a row 0.42 of HBM against
// 0.49, full rows 0.73 against 0.75, the self-play step 0.459 against 0.428 ms).  So: up
// to 8, whatever the capacity (a grouping must divide `heads` and fit G * L <= 64 lanes).
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
           const int64_t* pos, const int64_t* rows, const int32_t* order, void* out, int64_t n,
           int64_t heads, int64_t slots, int64_t cache_rows, float scale, int64_t q_stride,
           int64_t new_stride, hipStream_t stream) {
  constexpr int L = DH / (16 / (int)sizeof(typename KT::storage));
  switch (pick_group<L>(heads, slots)) {
#define CUGO_GROUP(GG)                                                                        \
  case GG:                                                                                    \
    if constexpr (GG * L <= 64)                                                               \
      return launch_parts<QT, KT, DH, APPEND, GG>(q, keys, values, k_new, v_new, pos, rows,   \
                                                  order, out, n, heads, slots, cache_rows,    \
                                                  scale, q_stride, new_stride, stream);       \
    return -3;
    CUGO_GROUP(2)
    CUGO_GROUP(4)
    CUGO_GROUP(8)
#undef CUGO_GROUP
    default:
      return launch_parts<QT, KT, DH, APPEND, 1>(q, keys, values, k_new, v_new, pos, rows,
                                                 order, out, n, heads, slots, cache_rows, scale,
                                                 q_stride, new_stride, stream);
  }
}

template <class QT, class KT, bool APPEND>
int by_dh(int64_t dh, const void* q, void* keys, void* values, const void* k_new,
          const void* v_new, const int64_t* pos, const int64_t* rows, const int32_t* order,
          void* out, int64_t n, int64_t heads, int64_t slots, int64_t cache_rows, float scale,
          int64_t q_stride, int64_t new_stride, hipStream_t stream) {
  switch (dh) {
#define CUGO_DH(D)                                                                       \
  case D:                                                                                \
    if constexpr (16 / sizeof(typename KT::storage) <= D)                                \
      return launch<QT, KT, D, APPEND>(q, keys, values, k_new, v_new, pos, rows, order, \
                                       out, n, heads, slots, cache_rows, scale,          \
                                       q_stride, new_stride, stream);                    \
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
             const int32_t* order, void* out, int64_t n, int64_t heads, int64_t slots,
             int64_t cache_rows, float scale, int64_t q_stride, int64_t new_stride,
             hipStream_t stream) {
#define CUGO_KV(QTYPE)                                                                        \
  switch (kv_dtype) {                                                                         \
    case CUGO_DTYPE_BF16:                                                                     \
      return by_dh<QTYPE, BF16, APPEND>(dh, q, keys, values, k_new, v_new, pos, rows, order,  \
                                        out, n, heads, slots, cache_rows, scale, q_stride,    \
                                        new_stride, stream);                                  \
    case CUGO_DTYPE_F16:                                                                      \
      return by_dh<QTYPE, F16, APPEND>(dh, q, keys, values, k_new, v_new, pos, rows, order,   \
                                       out, n, heads, slots, cache_rows, scale, q_stride,     \
                                       new_stride, stream);                                   \
    case CUGO_DTYPE_F32:                                                                      \
      return by_dh<QTYPE, F32, APPEND>(dh, q, keys, values, k_new, v_new, pos, rows, order,   \
                                       out, n, heads, slots, cache_rows, scale, q_stride,     \
                                       new_stride, stream);                                   \
    default:                                                                                  \
      return -2;                                                                              \
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

// The KV append alone (cugo_seq50.py:317-318, the index_put_ of a token's new key and
// value), for tokens whose attention output nothing reads: one thread per 16-byte part of
// a (token, head) row, keys[rows[i], h, min(pos[i], slots - 1)] = k_new[i, h] and likewise
// for values; a token with pos < 0 or a row outside the cache writes nothing.
template <class KT, int DH>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const typename KT::storage* __restrict__ k_new, const typename KT::storage* __restrict__ v_new,
    int64_t new_stride, typename KT::storage* __restrict__ keys,
    typename KT::storage* __restrict__ values, const int64_t* __restrict__ pos_in,
    const int64_t* __restrict__ rows, int64_t n, int heads, int64_t slots, int64_t cache_rows) {
  constexpr int E = 16 / (int)sizeof(typename KT::storage);
  constexpr int kParts = DH / E;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * heads * kParts) return;
  const int64_t i = t / (heads * kParts);
  const int rest = (int)(t - i * heads * kParts);
  const int head = rest / kParts, part = rest % kParts;
  int64_t pos = pos_in[i];
  const int64_t row = rows ? rows[i] : i;
  if (pos < 0 || row < 0 || row >= cache_rows) return;
  if (pos >= slots) pos = slots - 1;
  const int64_t src = i * new_stride + head * DH + part * E;
  const size_t dst = (((size_t)row * heads + head) * (size_t)slots + pos) * DH + part * E;
  *reinterpret_cast<uint4*>(keys + dst) = *reinterpret_cast<const uint4*>(k_new + src);
  *reinterpret_cast<uint4*>(values + dst) = *reinterpret_cast<const uint4*>(v_new + src);
}

template <class KT>
int kv_append_by_dh(int64_t dh, const void* k_new, const void* v_new, int64_t new_stride,
                    void* keys, void* values, const int64_t* pos, const int64_t* rows,
                    int64_t n, int64_t heads, int64_t slots, int64_t cache_rows,
                    hipStream_t stream) {
  using KS = typename KT::storage;
  const int64_t parts = dh * (int64_t)sizeof(KS) / 16;
  const unsigned blocks = (unsigned)((n * heads * parts + 255) / 256);
  switch (dh) {
#define CUGO_APPEND_DH(D)                                                                    \
  case D:                                                                                    \
    if constexpr (16 / sizeof(KS) <= D) {                                                    \
      hipLaunchKernelGGL((kv_append_kernel<KT, D>), dim3(blocks), dim3(256), 0, stream,     \
                         static_cast<const KS*>(k_new), static_cast<const KS*>(v_new),       \
                         new_stride, static_cast<KS*>(keys), static_cast<KS*>(values), pos,  \
                         rows, n, (int)heads, slots, cache_rows);                            \
      return (int)hipGetLastError();                                                         \
    }                                                                                        \
    return -3;
    CUGO_APPEND_DH(16)
    CUGO_APPEND_DH(32)
    CUGO_APPEND_DH(64)
    CUGO_APPEND_DH(128)
#undef CUGO_APPEND_DH
    default:
      return -3;
  }
}

// cugo_decode_order: the queries longest first (by min(pos, slots - 1); a negative pos
// last), binned by length: bin b holds the rows with slots - 1 - clamp(pos) in
// [b << shift, (b + 1) << shift).  One workgroup: a histogram of the bins in LDS, an
// exclusive scan over it, then every query takes the next place of its bin.  Places within
// a bin go in the order the LDS atomics return them, which may differ between calls; the
// decode's results do not depend on the order.
constexpr int kOrderThreads = 1024;
constexpr int kOrderBins = 4096;

__global__ __launch_bounds__(kOrderThreads) void order_kernel(const int64_t* __restrict__ pos,
                                                              int64_t n, int64_t slots, int shift,
                                                              int32_t* __restrict__ order) {
  __shared__ int next[kOrderBins];  // the bins' counts, then their next free place
  __shared__ int partial[kOrderThreads];
  const int tid = threadIdx.x;
  for (int b = tid; b < kOrderBins; b += kOrderThreads) next[b] = 0;
  __syncthreads();
  auto bin_of = [&](int64_t i) {
    int64_t p = pos[i];
    p = p < 0 ? -1 : (p >= slots ? slots - 1 : p);
    return (int)((slots - 1 - p) >> shift);  // < kOrderBins by the choice of shift
  };
  for (int64_t i = tid; i < n; i += kOrderThreads) atomicAdd(&next[bin_of(i)], 1);
  __syncthreads();
  constexpr int kPer = kOrderBins / kOrderThreads;  // consecutive bins a thread scans
  int count[kPer];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    count[k] = next[tid * kPer + k];
    sum += count[k];
  }
  partial[tid] = sum;
  __syncthreads();
  for (int off = 1; off < kOrderThreads; off <<= 1) {  // inclusive scan of the sums
    const int v = tid >= off ? partial[tid - off] : 0;
    __syncthreads();
    partial[tid] += v;
    __syncthreads();
  }
  int start = partial[tid] - sum;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    next[tid * kPer + k] = start;
    start += count[k];
  }
  __syncthreads();
  for (int64_t i = tid; i < n; i += kOrderThreads)
    order[atomicAdd(&next[bin_of(i)], 1)] = (int32_t)i;
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
                          const int64_t* rows, const int32_t* order, int64_t n, int64_t heads,
                          int64_t dh, int64_t slots, int64_t cache_rows, float scale, void* out,
                          hipStream_t stream) {
  using namespace cugo_amd::decode;
  const int bad = check_args(q, keys, values, pos, out, n, heads, dh, slots, cache_rows);
  if (bad) return bad;
  if (q_stride < heads * dh) return -1;
  if (n == 0) return 0;
  return dispatch<false>(q_dtype, kv_dtype, dh, q, const_cast<void*>(keys),
                         const_cast<void*>(values), nullptr, nullptr, pos, rows, order, out, n,
                         heads, slots, cache_rows, scale, q_stride, 0, stream);
}

int cugo_decode_attention_append(int q_dtype, int kv_dtype, const void* q, int64_t q_stride,
                                 const void* k_new, const void* v_new, int64_t new_stride,
                                 void* keys, void* values, const int64_t* pos,
                                 const int64_t* rows, const int32_t* order, int64_t n,
                                 int64_t heads, int64_t dh, int64_t slots, int64_t cache_rows,
                                 float scale, void* out, hipStream_t stream) {
  using namespace cugo_amd::decode;
  const int bad = check_args(q, keys, values, pos, out, n, heads, dh, slots, cache_rows);
  if (bad) return bad;
  if (n > 0 && (!k_new || !v_new)) return -1;
  if (q_stride < heads * dh || new_stride < heads * dh) return -1;
  const int64_t kv_size = kv_dtype == CUGO_DTYPE_F32 ? 4 : 2;
  if (!aligned16(k_new) || !aligned16(v_new) || (new_stride * kv_size) % 16 != 0) return -4;
  if (n == 0) return 0;
  return dispatch<true>(q_dtype, kv_dtype, dh, q, keys, values, k_new, v_new, pos, rows, order,
                        out, n, heads, slots, cache_rows, scale, q_stride, new_stride, stream);
}

int cugo_kv_append(int kv_dtype, const void* k_new, const void* v_new, int64_t new_stride,
                   void* keys, void* values, const int64_t* pos, const int64_t* rows,
                   int64_t n, int64_t heads, int64_t dh, int64_t slots, int64_t cache_rows,
                   hipStream_t stream) {
  using namespace cugo_amd::decode;
  if (n < 0 || heads <= 0 || dh <= 0 || slots <= 0 || cache_rows < 0 || new_stride < heads * dh)
    return -1;
  if (n > 0 && (!k_new || !v_new || !keys || !values || !pos)) return -1;
  const int64_t kv_size = kv_dtype == CUGO_DTYPE_F32 ? 4 : 2;
  if (!aligned16(keys) || !aligned16(values) || !aligned16(k_new) || !aligned16(v_new) ||
      (new_stride * kv_size) % 16 != 0)
    return -4;
  if (n == 0) return 0;
  switch (kv_dtype) {
    case CUGO_DTYPE_BF16:
      return kv_append_by_dh<BF16>(dh, k_new, v_new, new_stride, keys, values, pos, rows, n,
                                   heads, slots, cache_rows, stream);
    case CUGO_DTYPE_F16:
      return kv_append_by_dh<F16>(dh, k_new, v_new, new_stride, keys, values, pos, rows, n,
                                  heads, slots, cache_rows, stream);
    case CUGO_DTYPE_F32:
      return kv_append_by_dh<F32>(dh, k_new, v_new, new_stride, keys, values, pos, rows, n,
                                  heads, slots, cache_rows, stream);
    default:
      return -2;
  }
}

int cugo_decode_order(const int64_t* pos, int64_t n, int64_t slots, int32_t* order,
                      hipStream_t stream) {
  using namespace cugo_amd::decode;
  if (n < 0 || n > INT32_MAX || slots <= 0 || (n > 0 && (!pos || !order))) return -1;
  if (n == 0) return 0;
  int shift = 0;  // bins of 2^shift consecutive lengths, at most kOrderBins of them
  while ((slots >> shift) >= kOrderBins) ++shift;
  hipLaunchKernelGGL(order_kernel, dim3(1), dim3(kOrderThreads), 0, stream, pos, n, slots, shift,
                     order);
  return (int)hipGetLastError();
}

}  // extern "C"
