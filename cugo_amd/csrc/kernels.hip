// gfx950 kernels and the C ABI of libcugo_hip.so (declared in include/cugo_hip.h).
//
// Every row kernel works on tiles of 64 games with one 64-lane wavefront per
// workgroup.  The tile's 248-byte rows move between HBM and LDS with coalesced 8-byte
// accesses (consecutive lanes touch consecutive words, also for gathered rows, whose
// 31 words are contiguous), and each lane then runs one game in registers.  The
// observation is the widest output (2,880 + 179 bytes per row): lanes first build a
// compact per-row feature record in LDS, then the wavefront writes the feature rows as
// consecutive float4 stores and the legal-mask rows as consecutive 32-bit words, so
// every output byte is written once, in order.
#include <hip/hip_runtime.h>

#include <mutex>

#include "engine.h"
#include "../../include/cugo_hip.h"

namespace cugo_amd {

constexpr int kTile = 64;
constexpr int kTileWords = kTile * kRowWords;  // 1,984

// log2f(1 + p) / 12 clamped to 1 for p < 4095 (torch50.h:405-408), generated at build
// time with the host C library's log2f, so the values are the reference engine's own.
__constant__ float c_stop_bits[kStopBitsTable] = {
#include "stop_bits.inc"
};

__device__ inline i64 tile_base() { return (i64)blockIdx.x * kTile; }

__device__ inline int tile_count(i64 base, i64 n) {
  const i64 left = n - base;
  return left < kTile ? (int)left : kTile;
}

__device__ inline bool valid_id(i64 id, i64 env_count) { return id >= 0 && id < env_count; }

// Loads the tile's rows into LDS with kThreads threads; src row r is `ids[r]` (gathered,
// zero row when the id is invalid) or base + r (contiguous) when ids_lds is null.  Each
// thread first loads all of its words into registers, at indices clamped into the rows
// that exist, and only then writes LDS: loads guarded by a branch, or a store of each
// load before the next, would each wait out a full memory round trip.
template <int kThreads = kTile, int kMaxRows = kTile>
__device__ inline void stage_in(u64* lds, const u64* states, const i64* ids_lds, i64 base,
                                int count, i64 env_count) {
  constexpr int kPer = (kMaxRows * kRowWords + kThreads - 1) / kThreads;
  constexpr int kBatch = kPer < 16 ? kPer : 16;  // words in flight per thread
  const int words = count * kRowWords;  // count >= 1 in every launched tile
  const bool gather = ids_lds != nullptr;
  if (gather && env_count <= 0) {  // no row to read: every id is invalid
    for (int j = threadIdx.x; j < words; j += kThreads) lds[j] = 0ull;
    return;
  }
  const u64* src = states + base * kRowWords;
#pragma unroll
  for (int p0 = 0; p0 < kPer; p0 += kBatch) {
    u64 v[kBatch];
    bool ok[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int j0 = threadIdx.x + (p0 + q) * kThreads;
      const int j = j0 < words ? j0 : words - 1;
      if (!gather) {
        ok[q] = true;
        v[q] = src[j];
      } else {
        const int r = j / kRowWords;
        const int k = j - r * kRowWords;
        const i64 id = ids_lds[r];
        ok[q] = valid_id(id, env_count);
        v[q] = states[(ok[q] ? id : 0) * kRowWords + k];
      }
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int j = threadIdx.x + (p0 + q) * kThreads;
      if (p0 + q < kPer && j < words) lds[j] = ok[q] ? v[q] : 0ull;
    }
  }
}

// Stores the tile's rows from LDS with kThreads threads: to dst rows base + r
// (contiguous) or, when ids_lds is given, to rows ids[r] with a valid id (scatter, in
// place).  All of a thread's LDS reads come before its stores.
template <int kThreads = kTile, int kMaxRows = kTile>
__device__ inline void stage_out(const u64* lds, u64* dst, const i64* ids_lds, i64 base,
                                 int count, i64 env_count) {
  constexpr int kPer = (kMaxRows * kRowWords + kThreads - 1) / kThreads;
  const int words = count * kRowWords;
  u64 v[kPer];
#pragma unroll
  for (int p = 0; p < kPer; ++p) {
    const int j = threadIdx.x + p * kThreads;
    v[p] = lds[j < words ? j : words - 1];
  }
  if (ids_lds == nullptr) {
    u64* out = dst + base * kRowWords;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int j = threadIdx.x + p * kThreads;
      if (j < words) out[j] = v[p];
    }
  } else {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int j = threadIdx.x + p * kThreads;
      if (j >= words) continue;
      const int r = j / kRowWords;
      const int k = j - r * kRowWords;
      const i64 id = ids_lds[r];
      if (valid_id(id, env_count)) dst[id * kRowWords + k] = v[p];
    }
  }
}

__device__ inline u16 clamp_action(i64 raw) {  // torch50_ext.cu:96-99
  return raw >= 0 && raw < kActionCount ? (u16)raw : kInvalidAction16;
}

// ------------------------------------------------------------------- create ----
__global__ __launch_bounds__(kTile) void create_kernel(const i64* seeds, const i64* first,
                                                       i64 n, u64* states) {
  __shared__ u64 rows[kTileWords];
  const i64 base = tile_base();
  const int count = tile_count(base, n);
  const int lane = threadIdx.x;
  if (lane < count) {
    const Env e = create_env((u64)seeds[base + lane], (u32)(first[base + lane] & 1));
    pack_row(e, rows + lane * kRowWords);
  }
  __syncthreads();
  stage_out(rows, states, nullptr, base, count, 0);
}

// ------------------------------------------------------------------ observe ----
// LDS of one observe tile: the staged rows are dead once every lane has unpacked its
// row, so the per-row feature records and masks reuse the same bytes.
constexpr int kRecStride = kFeatRecord + 1;  // + the zero pad; odd: no bank conflicts
template <int kRows>
struct RecordBufferOf {  // one step's observation of a tile of kRows games, before it is stored
  u32 rec[kRows][kRecStride];
  u64 legal[kRows][3];
};
using RecordBuffer = RecordBufferOf<kTile>;
template <int kRows>
struct ObserveTileOf {
  union {
    u64 rows[kRows * kRowWords];
    RecordBufferOf<kRows> out;
  };
};
using ObserveTile = ObserveTileOf<kTile>;

// Four consecutive mask bits -> four bytes 0/1 (little-endian).
__device__ inline u32 spread4(u32 x) {
  return (x & 1u) | ((x & 2u) << 7) | ((x & 4u) << 14) | ((x & 8u) << 21);
}

// The tile's observation from its LDS records, stored by every wave that calls this.  A
// wave claims work items from the tile's LDS counter `next` (zeroed before the records
// were written) until none is left: items 0 .. count - 1 are feature rows (lane owns the
// float4 columns q = lane, lane + 64, lane + 128 < 180 of the row, so a store instruction
// covers 1 KiB; a column is one nibble of the record's bit array, ORed with the record's
// dense dwords for the 12 columns that hold other scalars), then 64-dword chunks of the
// legal mask bytes, then their unaligned tail.  A wave that arrives late (one that also
// stepped the games) takes what is left, so no wave idles while another stores alone.
// The claiming lane is the wave's first active lane, and every pass raises the counter,
// so every wave leaves the loop.  A claim is kClaim items: a claim of kClaim feature rows
// issues all its LDS reads before its 3 x kClaim stores, so more rows a claim keep more
// stores in flight per wave, at the cost of 20 VGPRs a row.
// bf16 bits of a finite float's bits, rounded to nearest even (torch's float -> bfloat16).
__device__ inline u32 bf16_bits(u32 f) { return (f + 0x7fffu + ((f >> 16) & 1u)) >> 16; }

// Four features (float bits) of a row's float4 column `quad` (index row * kQuads + quad),
// as float32 or, with kBf16, rounded to bfloat16.  Plain stores: non-temporal ones
// measured slower (play_random 1.013 -> 1.305 ms a 32-step launch, observe at 65,536 rows
// 42.9 -> 53.5 us), the last-level cache taking the store bursts in.
template <bool kBf16>
__device__ inline void store_quad(void* features, i64 index, const uint4& v) {
  if constexpr (kBf16) {
    uint2 p;
    p.x = bf16_bits(v.x) | (bf16_bits(v.y) << 16);
    p.y = bf16_bits(v.z) | (bf16_bits(v.w) << 16);
    reinterpret_cast<uint2*>(features)[index] = p;
  } else {
    reinterpret_cast<uint4*>(features)[index] = v;
  }
}

template <int kClaim, bool kBf16 = false, int kRows = kTile>
__device__ inline void store_observation(const RecordBufferOf<kRows>& t, i64 base, int count,
                                         void* features, u8* legal, int* next) {
  const int lane = threadIdx.x & (kTile - 1);
  constexpr int kQuads = kFeatureCount / 4;  // 180
  // Each of the lane's columns 1 and 2: its features' dense dwords, or the record's zero
  // pad dword (column 0, quads 0..63, holds no dense feature; lanes past quad 179 read the
  // pad too).
  int dpos[3][4];
  for (int c = 1; c < 3; ++c)
    for (int k = 0; k < 4; ++k) {
      const int q = lane + kTile * c;
      const int pos = q < kQuads ? dense_pos((u32)(4 * q + k)) : -1;
      dpos[c][k] = kRecBits + (pos >= 0 ? pos : kRecDense);
    }
  const i64 fbase = base * kQuads;  // the tile's first float4 column
  // Legal mask: count x 179 bytes from a 4-byte aligned base (64 * 179 % 4 == 0); word
  // w holds tile bytes 4w..4w+3, i.e. actions a..a+3 of row r unless it straddles rows.
  u8* lout = legal + base * kActionCount;
  const int bytes = count * kActionCount;
  const int full = bytes / 4;
  const int chunks = (full + kTile - 1) / kTile;
  const int items = count + chunks + (bytes > 4 * full ? 1 : 0);
  const int leader = __ffsll((long long)__ballot(1)) - 1;
  for (;;) {
    int claim = 0;
    if (lane == leader) claim = atomicAdd(next, kClaim);
    const int item0 = __builtin_amdgcn_readfirstlane(claim);
    if (item0 >= items) break;
    if (item0 + kClaim - 1 < count) {
      // kClaim feature rows: every LDS read of the rows first (column 2's lanes past quad
      // 179 read in-range dwords and store nothing), then the 3 x kClaim float4 stores.
      u32 nib[kClaim][3], dv[kClaim][3][4];
#pragma unroll
      for (int j = 0; j < kClaim; ++j) {
        const u32* rec = t.rec[item0 + j];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const int q = lane + kTile * c;
          nib[j][c] = rec[q >> 3] >> (4 * (q & 7));
          if (c > 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) dv[j][c][k] = rec[dpos[c][k]];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kClaim; ++j) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const int q = lane + kTile * c;
          uint4 v;  // 0 or 1.0f per bit
          v.x = (0u - (nib[j][c] & 1u)) & 0x3f800000u;
          v.y = (0u - ((nib[j][c] >> 1) & 1u)) & 0x3f800000u;
          v.z = (0u - ((nib[j][c] >> 2) & 1u)) & 0x3f800000u;
          v.w = (0u - ((nib[j][c] >> 3) & 1u)) & 0x3f800000u;
          if (c > 0) {
            v.x |= dv[j][c][0];
            v.y |= dv[j][c][1];
            v.z |= dv[j][c][2];
            v.w |= dv[j][c][3];
          }
          if (q < kQuads) store_quad<kBf16>(features, fbase + (item0 + j) * kQuads + q, v);
        }
      }
      continue;
    }
    for (int item = item0; item < item0 + kClaim && item < items; ++item) {
    if (item < count) {
      const int r = item;
      const u32* rec = t.rec[r];
      for (int c = 0; c < 3; ++c) {
        const int q = lane + kTile * c;
        if (q < kQuads) {
          const u32 nib = rec[q >> 3] >> (4 * (q & 7));
          uint4 v;  // 0 or 1.0f per bit
          v.x = (0u - (nib & 1u)) & 0x3f800000u;
          v.y = (0u - ((nib >> 1) & 1u)) & 0x3f800000u;
          v.z = (0u - ((nib >> 2) & 1u)) & 0x3f800000u;
          v.w = (0u - ((nib >> 3) & 1u)) & 0x3f800000u;
          if (c > 0) {  // unconditional reads: lanes without a dense feature read the pad
            v.x |= rec[dpos[c][0]];
            v.y |= rec[dpos[c][1]];
            v.z |= rec[dpos[c][2]];
            v.w |= rec[dpos[c][3]];
          }
          store_quad<kBf16>(features, fbase + r * kQuads + q, v);
        }
      }
    } else if (item < count + chunks) {
      const int w = (item - count) * kTile + lane;
      if (w < full) {
        const int b0 = w * 4;
        const int r = b0 / kActionCount;
        const int a = b0 - r * kActionCount;
        u32 packed;
        if (a + 3 < kActionCount) {
          const u64* m = t.legal[r];
          const int lo = a >> 6, sh = a & 63;
          u64 bits = m[lo] >> sh;
          if (sh > 60) bits |= m[lo + 1] << (64 - sh);
          packed = spread4((u32)(bits & 0xFu));
        } else {
          packed = 0;
          for (int b = 0; b < 4; ++b) {
            const int at = b0 + b;
            const int rr = at / kActionCount;
            const int aa = at - rr * kActionCount;
            packed |= (u32)((t.legal[rr][aa >> 6] >> (aa & 63)) & 1u) << (8 * b);
          }
        }
        reinterpret_cast<u32*>(lout)[w] = packed;
      }
    } else {
      const int at = 4 * full + lane;
      if (at < bytes) {
        const int r = at / kActionCount;
        const int a = at - r * kActionCount;
        lout[at] = (u8)((t.legal[r][a >> 6] >> (a & 63)) & 1u);
      }
    }
    }
  }
}

// One tile of 64 games per 192-thread workgroup: wave 0 runs the 64 games (one per
// lane) and writes their records; then all three waves share the 64 x 3,059 output
// bytes, so a wave whose games took long to compute does not store its rows alone.
// Three waves, because the kernel's ~160 VGPRs allow three waves per SIMD: four
// workgroups per CU then hold all 1,024 tiles of a 65,536-row batch at once.
constexpr int kObsThreads = 192;

// ------------------------------------------------------- random-policy draw ----
__device__ inline u64 xorshift64(u64& x) {
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  return x;
}

__device__ inline u64 sampler_seed(u64 seed) {
  u64 s = seed;
  const u64 v = sm_next(s);
  return v != 0 ? v : 1ull;
}

// Uniform draw over the set bits of a 179-bit action mask (actions 0..63 in m0, 64..127
// in m1, 128..178 in m2): one xorshift64 step of the sampler word x, then the
// (value % count)-th set bit.  -1, with x untouched, when no bit is set.
__device__ inline i64 draw_legal(u64 m0, u64 m1, u64 m2, u64& x) {
  const u32 c0 = popc(m0), c1 = popc(m1);
  const u32 total = c0 + c1 + popc(m2);
  if (total == 0) return -1;
  const u32 pick = (u32)(xorshift64(x) % total);
  if (pick < c0) return select_rank(m0, pick);
  if (pick < c0 + c1) return 64 + select_rank(m1, pick - c0);
  return 128 + select_rank(m2, pick - c0 - c1);
}

// kSample: also draw each row's random-policy action from its legal mask while the mask
// is in registers (draw_legal with sampler[i], into actions[i]), as sample_kernel would
// from the stored mask.
// kBf16: the features are written rounded to bfloat16 (uint16 [n, 720]), as torch's
// conversion of the float32 features rounds them.
// kRows games a tile (at most 64): see obs_rows().
template <bool kIndexed, bool kSample = false, bool kBf16 = false, int kRows = kTile>
__global__ __launch_bounds__(kObsThreads) void observe_kernel(const u64* states, i64 env_count,
                                                              const i64* ids, i64 n,
                                                              void* features, u8* legal,
                                                              u8* player, u8* done,
                                                              i16* status, u64* sampler = nullptr,
                                                              i64* actions = nullptr) {
  static_assert(kRows >= 1 && kRows <= kTile, "a tile is at most one wavefront of games");
  __shared__ ObserveTileOf<kRows> t;
  __shared__ i64 tile_ids[kRows];
  __shared__ int next_item;  // store_observation's work counter
  const i64 base = (i64)blockIdx.x * kRows;
  const int count = n - base < kRows ? (int)(n - base) : kRows;
  const int tid = threadIdx.x;
  const int lane = tid & (kTile - 1);
  const int wave = tid / kTile;
  if (kIndexed && tid < count) tile_ids[tid] = ids[base + tid];
  if (tid == 0) next_item = 0;
  __syncthreads();
  stage_in<kObsThreads, kRows>(t.rows, states, kIndexed ? tile_ids : nullptr, base, count,
                               env_count);  // all threads
  __syncthreads();
  const bool active = wave == 0 && lane < count;
  const bool ok = active && (!kIndexed || valid_id(tile_ids[lane], env_count));
  Env e;
  if (ok) e = unpack_row(t.rows + lane * kRowWords);
  __syncthreads();  // rows are dead from here on; their bytes become the records
  if (active) {
    const i64 i = base + lane;
    u32* rec = t.out.rec[lane];
    if (ok) {
      const Packet pk = make_packet(e);
      FeatRow fr;
      feature_row(pk, c_stop_bits, fr);
      feature_record(fr, rec);
      t.out.legal[lane][0] = pk.head.legal.w0;
      t.out.legal[lane][1] = pk.head.legal.w1;
      t.out.legal[lane][2] = pk.head.legal.w2;
      player[i] = pk.head.player;
      done[i] = e.done != 0;
      status[i] = (i16)pk.head.status;
      if (kSample) {
        u64 x = sampler[i];
        const i64 a = draw_legal(pk.head.legal.w0, pk.head.legal.w1, pk.head.legal.w2, x);
        if (a >= 0) sampler[i] = x;
        actions[i] = a;
      }
    } else {  // invalid id (torch50_ext.cu:71-87): an all-zero row
      for (int k = 0; k <= kFeatRecord; ++k) rec[k] = 0u;
      t.out.legal[lane][0] = t.out.legal[lane][1] = t.out.legal[lane][2] = 0;
      player[i] = 0;
      done[i] = 1;
      status[i] = CUGO_INVALID_INDEX_STATUS;
      if (kSample) actions[i] = -1;
    }
  }
  __syncthreads();
  store_observation<2, kBf16, kRows>(t.out, base, count, features, legal, &next_item);
}

// --------------------------------------------------------------------- step ----
// Auto-reset of finished rows inside the step (kMode 3): the next game of row i is
// seed = base_seed + i + stride * (++generation[i]), copied from its pre-dealt spare when
// one is there and dealt inline otherwise; sampler[i] is re-seeded from it.  Spares come in
// S = slot_mask + 1 slots of `rows` rows (S = 1, 2 or 4): generation g of row i is pre-dealt
// in spare row (g & slot_mask) * rows + i, valid when spare_gen of that row equals g.
// play_kernel deals a stale spare's game into its slot before taking it; the step
// kernels only read the spares.
struct AutoReset {
  u64 base_seed, stride;
  u32* generation;
  u64* sampler;
  u64* spares;
  const u32* spare_gen;
  i64 rows;
  u32 slot_mask;
};
__device__ inline i64 spare_row(const AutoReset& ar, i64 i, u32 gen) {
  return (i64)(gen & ar.slot_mask) * ar.rows + i;
}

// kMode: 0 = step (contiguous, in place), 1 = step_indexed (gather/scatter in place),
// 3 = step with the auto-reset above (contiguous, in place); branch_indexed has its own
// kernel below.
// kThreads = 128: two waves per tile of 64 games, both stage the rows in and out and
// wave 0 runs the games (one per lane).  At ~250 VGPRs two waves fit per SIMD, so this
// is the shape while every tile of the grid is resident at once (up to four per CU);
// a larger grid queues tiles, and then one wave per tile (kThreads = 64) keeps twice as
// many games computing per CU.
template <int kMode, bool kEvents, int kStepThreads, int kRows = kTile>
__global__ __launch_bounds__(kStepThreads) void step_kernel(u64* states, i64 env_count, const i64* ids,
                                                     const i64* actions, i64 n,
                                                     float* reward, u8* done, u8* nagari,
                                                     i16* status, u8* committed, i64* events,
                                                     AutoReset ar) {
  static_assert(kRows >= 1 && kRows <= kTile, "a tile is at most one wavefront of games");
  __shared__ u64 rows[kRows * kRowWords];
  __shared__ i64 tile_ids[kRows];
  __shared__ i64 ev[kRows * kEventWords];
  __shared__ int spare_rows[kRows];  // kMode 3: tile rows whose next game is a spare
  __shared__ i64 spare_src[kRows];   // kMode 3: their spare rows
  __shared__ int spare_count;
  const i64 base = (i64)blockIdx.x * kRows;
  const int count = n - base < kRows ? (int)(n - base) : kRows;
  const int lane = threadIdx.x;
  constexpr bool kIndexed = kMode == 1;
  if (kIndexed && lane < count) tile_ids[lane] = ids[base + lane];
  __syncthreads();
  stage_in<kStepThreads, kRows>(rows, states, kIndexed ? tile_ids : nullptr, base, count, env_count);
  __syncthreads();
  bool take_spare = false;
  u32 gen0 = 0, spare0 = 0;  // kMode 3: issued before the step so their latency hides
  i64 src = 0;                // kMode 3: the spare row of generation gen0 + 1
  if (kMode == 3 && lane < count) {
    gen0 = ar.generation[base + lane];
    src = spare_row(ar, base + lane, gen0 + 1u);
    spare0 = ar.spare_gen[src];
  }
  if (lane < count) {
    const i64 i = base + lane;
    const bool ok = !kIndexed || valid_id(tile_ids[lane], env_count);
    u64* row = rows + lane * kRowWords;
    i64* evr = ev + lane * kEventWords;
    if (ok) {
      Env e = unpack_row(row);
      const StepOut so = torch_step(e, clamp_action(actions[i]));
      if (kEvents) {
        if (so.committed) {
          // make_torch_event50 against the untouched row still in LDS
          Env before;
          before.hand0 = row[0]; before.hand1 = row[1]; before.stock = row[3];
          before.cap0 = row[4]; before.cap1 = row[5]; before.rev0 = row[22];
          before.rev1 = row[23];
          make_event(before, e, evr);
        } else {
          for (int k = 0; k < kEventWords; ++k) evr[k] = 0;
        }
      }
      pack_row(e, row);
      reward[i] = (float)so.reward0;
      done[i] = so.done;
      nagari[i] = so.nagari;
      status[i] = (i16)so.status;
      committed[i] = so.committed;
      if (kMode == 3 && so.done) {
        const u32 gen = gen0 + 1u;
        ar.generation[i] = gen;
        const u64 seed = ar.base_seed + (u64)i + ar.stride * gen;
        ar.sampler[i] = sampler_seed(seed);
        take_spare = spare0 == gen;
        if (!take_spare) pack_row(create_env(seed, (u32)(i & 1)), row);
      }
    } else {  // torch50_ext.cu:108-118
      if (kEvents) for (int k = 0; k < kEventWords; ++k) evr[k] = 0;
      reward[i] = 0.0f;
      done[i] = 1;
      nagari[i] = 0;
      status[i] = CUGO_INVALID_INDEX_STATUS;
      committed[i] = 0;
    }
  }
  if (kMode == 3) {
    // Compact the spare-taking rows so that every lane's spare load is independent:
    // a tile with f such rows moves 31 f words in ceil(31 f / threads) passes.
    const u64 ballot = __ballot(take_spare);
    if (take_spare) {
      const int at = (int)__popcll(ballot & ((1ull << lane) - 1ull));
      spare_rows[at] = lane;
      spare_src[at] = src;
    }
    if (lane == 0) spare_count = (int)__popcll(ballot);
    __syncthreads();
    const int words = spare_count * kRowWords;
    for (int j = lane; j < words; j += kStepThreads) {
      const int c = j / kRowWords;
      const int k = j - c * kRowWords;
      rows[spare_rows[c] * kRowWords + k] = ar.spares[spare_src[c] * kRowWords + k];
    }
  }
  __syncthreads();
  stage_out<kStepThreads, kRows>(rows, states, kIndexed ? tile_ids : nullptr, base, count, env_count);
  if (kEvents) {
    i64* eout = events + base * kEventWords;
    for (int j = lane; j < count * kEventWords; j += kStepThreads) eout[j] = ev[j];
  }
}

// ------------------------------------------------------------------ branch ----
// branch_indexed (torch50_ext.cu:288-314): each lane reads its parent row straight from
// global memory (branching children of one root read the same row, so a wave's loads are
// broadcasts from L2), steps it in registers, and the wave's 64 child rows go out through
// LDS as one contiguous block.  The transition holds ~200 VGPRs, which allows two waves
// per SIMD; capping registers for three or four waves spills 144 / 356 bytes a lane and
// measured 1.35x / 2.7x slower on 1,048,576 children, and staging the parents through LDS
// as well, as the other step kernels do, measured 1.13x slower.
// kRows children a wavefront: at 1,048,576 children (16,384 wavefronts, many rounds) 64
// took 0.103 ms, 48 0.126 and 32 0.153: fewer children a wavefront run fewer divergent
// rule paths each, but the launch issues more wavefronts of the same length.
// Waves whose 64 children share one parent (C3's layout) were also given a path that
// reads the parent with scalar loads and builds its legality head once in scalar
// registers: VALU instructions fell from 2,095 to 1,978 a wave (the head is that
// small a part of the step), SALU rose from 634 to 871, VGPRs stayed at 198, and the
// launch took the same time (0.100-0.102 ms against 0.099-0.105), so it was dropped.
// Tiles of 256 children grouped by action in LDS before the step (a counting sort, so a
// wavefront's lanes share one or two actions' rule paths) took 0.110 ms: dropped too.
template <int kRows>
__global__ __launch_bounds__(kTile) void branch_kernel(const u64* parents, i64 env_count,
                                                       const i64* ids, const i64* actions,
                                                       i64 n, u64* children, float* reward,
                                                       u8* done, u8* nagari, i16* status,
                                                       u8* committed) {
  __shared__ u64 tile[kRows * kRowWords];
  const int lane = threadIdx.x;
  const i64 base = (i64)blockIdx.x * kRows;
  const i64 i = base + lane;
  const int count = n - base < kRows ? (int)(n - base) : kRows;
  if (lane < kRows && i < n) {
    const i64 id = ids[i];
    u64 row[kRowWords];
    if (valid_id(id, env_count)) {
      const u64* src = parents + id * kRowWords;
#pragma unroll
      for (int k = 0; k < kRowWords; ++k) row[k] = src[k];
      Env e = unpack_row(row);
      const StepOut so = torch_step(e, clamp_action(actions[i]));
      pack_row(e, row);
      reward[i] = (float)so.reward0;
      done[i] = so.done;
      nagari[i] = so.nagari;
      status[i] = (i16)so.status;
      committed[i] = so.committed;
    } else {  // torch50_ext.cu:108-118: a zero child
#pragma unroll
      for (int k = 0; k < kRowWords; ++k) row[k] = 0;
      reward[i] = 0.0f;
      done[i] = 1;
      nagari[i] = 0;
      status[i] = CUGO_INVALID_INDEX_STATUS;
      committed[i] = 0;
    }
#pragma unroll
    for (int k = 0; k < kRowWords; ++k) tile[lane * kRowWords + k] = row[k];
  }
  // The tile's child rows leave as one contiguous block: stored from registers, a store
  // instruction wrote 8 bytes into each of 64 rows 248 bytes apart, and the L1's queue of
  // partial-line writes stalled the wave most of the time.
  __syncthreads();
  u64* out = children + base * kRowWords;
  const int words = count * kRowWords;
#pragma unroll
  for (int j = 0; j < (kRows * kRowWords + kTile - 1) / kTile; ++j) {
    const int w = j * kTile + lane;
    if (w < words) out[w] = tile[w];
  }
}

// ------------------------------------------------------------ random play ----
// `steps` random-policy self-play steps in one launch, each the work of
// observe_kernel<false, true> (the observation and the uniform legal draw) followed by
// step_kernel<3> (the step and the auto-reset of finished rows), with the last step's
// outputs.  Two waves per tile of 64 games; wave 0 keeps the games in registers for the
// whole launch.  Step s's observation records go to LDS buffer s % 2: while wave 1 stores
// step s - 1's observation from the other buffer, wave 0 steps the games, deals the
// finished ones their next game, builds step s's records and draws its actions, then
// takes over the stores that are left.  So the HBM-bound stores run beside the integer
// work of both the step and the next observation, and the rows are read and written
// once per launch.  Two waves per SIMD (the register budget is pinned to 256 VGPRs, with
// no private memory: the code object's private segment is 0 bytes): four tiles per CU
// (34 KiB of LDS each), every tile of a 65,536-row batch resident at once.
constexpr int kPlayThreads = 128;
constexpr int64_t kMaxPlaySteps = 1 << 20;

// The game of `seed` dealt into the 31-word row `dst`.
__device__ __attribute__((noinline)) void deal_into(u64 seed, u32 first, u64* dst) {
  pack_row(create_env(seed, first), dst);
}
constexpr int kPlayClaim = 4;  // rows a store claim (the observe kernels' third wave needs 2)

// step_rows = 0: every step's outputs overwrite the same n rows (the loop keeps only the
// last step's); step_rows >= n, a multiple of 4: step s writes rows s * step_rows + i of
// outputs with `steps` blocks of step_rows rows, so every step's observation is kept.
__global__ __launch_bounds__(kPlayThreads) __attribute__((amdgpu_waves_per_eu(2)))
void play_kernel(
    u64* states, i64 n, u64* sampler, float* features, u8* legal, u8* player, u8* obs_done,
    i16* obs_status, i64* actions, float* reward, u8* done, u8* nagari, i16* status,
    u8* committed, AutoReset ar, int steps, i64 step_rows) {
  __shared__ ObserveTile t;    // the rows, then the records of even steps, then the rows
  __shared__ RecordBuffer t1;  // the records of odd steps
  __shared__ int next_item[2];  // store_observation's work counters, by step parity
  const i64 base = tile_base();
  const int count = tile_count(base, n);
  const int tid = threadIdx.x;
  const int lane = tid & (kTile - 1);
  const int wave = tid / kTile;
  const i64 i = base + lane;
  if (tid < 2) next_item[tid] = 0;
  // A plain loop: the rows are read once per launch, and the batched form of stage_in
  // measured 3-4 % slower here (this kernel's loop runs at its full register budget).
  {
    const u64* src = states + base * kRowWords;
    for (int j = tid; j < count * kRowWords; j += kPlayThreads) t.rows[j] = src[j];
  }
  const bool active = wave == 0 && lane < count;
  u32 gen = 0;
  u32 have = 0;  // bit k: the spare of generation gen + 1 + k is pre-dealt
  u64 xc = 0;    // the committed sampler state
  if (active) {  // issued early so their latency hides
    gen = ar.generation[i];
    for (u32 k = 0; k <= ar.slot_mask; ++k)
      if (ar.spare_gen[spare_row(ar, i, gen + 1u + k)] == gen + 1u + k) have |= 1u << k;
    xc = sampler[i];
  }
  __syncthreads();
  Env e;  // the game this lane plays (its next game once it finishes)
  if (active) e = unpack_row(t.rows + lane * kRowWords);
  __syncthreads();  // rows are dead from here on; their bytes become even steps' records
  i64 a = -1;
  u64 xt = 0;  // the sampler state after the draw (committed with the step)
  PacketHead head{};
  // Iteration s steps the games for step s - 1 (s > 0), observes step s into buffer s % 2
  // (s < steps) and stores step s - 1's observation (s > 0).
  for (int s = 0; s <= steps; ++s) {
    RecordBuffer& cur = (s & 1) ? t1 : t.out;
    if (active) {
      if (s > 0) {
        // The observation reads one copy of the game and the step another: building the
        // packet from the very Env that is then stepped leaves an engine temporary in
        // private memory.
        Env g = e;
        const StepOut so = torch_step_head(g, clamp_action(a), head);
        const i64 at = i + (i64)(s - 1) * step_rows;  // step s - 1's output row
        reward[at] = (float)so.reward0;
        done[at] = so.done;
        nagari[at] = so.nagari;
        status[at] = (i16)so.status;
        committed[at] = so.committed;
        if (so.done) {  // the next game: this generation's spare, or dealt here if stale
          ++gen;
          const u64 seed = ar.base_seed + (u64)i + ar.stride * gen;
          xc = sampler_seed(seed);
          // A stale spare gets its game dealt into its own slot first (out of line: the
          // deal inlined here doubles the loop's register pressure for a rare path).
          const i64 row = spare_row(ar, i, gen);
          if ((have & 1u) == 0) deal_into(seed, (u32)(i & 1), ar.spares + row * kRowWords);
          g = unpack_row(ar.spares + row * kRowWords);
          have >>= 1;
        } else if (a >= 0) {
          xc = xt;
        }
        e = g;
      }
      if (s < steps) {
        const Env seen = e;
        const Packet pk = make_packet(seen);
        FeatRow fr;
        feature_row(pk, c_stop_bits, fr);
        feature_record(fr, cur.rec[lane]);
        cur.legal[lane][0] = pk.head.legal.w0;
        cur.legal[lane][1] = pk.head.legal.w1;
        cur.legal[lane][2] = pk.head.legal.w2;
        const i64 at = i + (i64)s * step_rows;  // step s's output row
        player[at] = pk.head.player;
        obs_done[at] = seen.done != 0;
        obs_status[at] = (i16)pk.head.status;
        xt = xc;
        a = draw_legal(pk.head.legal.w0, pk.head.legal.w1, pk.head.legal.w2, xt);
        actions[at] = a;
        head = pk.head;
      }
    }
    if (s > 0) {  // step s - 1's observation, from the other buffer
      const i64 rows_before = (i64)(s - 1) * step_rows;
      store_observation<kPlayClaim>((s & 1) ? t.out : t1, base, count,
                                    features + rows_before * kFeatureCount,
                                    legal + rows_before * kActionCount,
                                    &next_item[(s - 1) & 1]);
    }
    if (tid == 0) next_item[s & 1] = 0;  // for iteration s + 1 (its last use has ended)
    __syncthreads();
  }
  if (active) {
    pack_row(e, t.rows + lane * kRowWords);
    ar.generation[i] = gen;
    sampler[i] = xc;
  }
  __syncthreads();
  {
    u64* out = states + base * kRowWords;
    for (int j = tid; j < count * kRowWords; j += kPlayThreads) out[j] = t.rows[j];
  }
}

// ------------------------------------------------------------ step + observe ----
// step_kernel<3> (step with the caller's actions, then the auto-reset of finished rows)
// followed by observe_kernel of the new states, in one launch: the PPO rollout's engine
// between two actor passes.  Two waves per tile of kRows games: both stage the rows in;
// wave 0 steps its games, deals the finished ones their next game (the pre-dealt spare,
// dealt into its slot first if stale, as play_kernel does), builds the new states'
// observation records in LDS and packs the rows; then both waves store the observation
// and the rows.  The rows are read and written once, where the two launches read them
// twice and wrote them once more.
constexpr int kStepObserveRows = 32;  // games a tile (see cugo_step_observe_spares)

template <bool kBf16, int kRows, int kThreads>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void step_observe_kernel(u64* states, i64 n, const i64* actions, float* reward, u8* done,
                         u8* nagari, i16* status, u8* committed, AutoReset ar, void* features,
                         u8* legal, u8* player, u8* obs_done, i16* obs_status) {
  static_assert(kRows >= 1 && kRows <= kTile, "a tile is at most one wavefront of games");
  __shared__ u64 rows[kRows * kRowWords];     // the rows in, the new rows out
  __shared__ RecordBufferOf<kRows> rb;        // the new states' observation records
  __shared__ int next_item;                   // store_observation's work counter
  const i64 base = (i64)blockIdx.x * kRows;
  const int count = n - base < kRows ? (int)(n - base) : kRows;
  const int tid = threadIdx.x;
  const int lane = tid & (kTile - 1);
  const int wave = tid / kTile;
  const i64 i = base + lane;
  if (tid == 0) next_item = 0;
  stage_in<kThreads, kRows>(rows, states, nullptr, base, count, n);
  __syncthreads();
  if (wave == 0 && lane < count) {
    u32 gen = ar.generation[i];
    const i64 srow = spare_row(ar, i, gen + 1u);
    const u32 sgen = ar.spare_gen[srow];  // issued before the step so its latency hides
    u64* row = rows + lane * kRowWords;
    Env e = unpack_row(row);
    const StepOut so = torch_step(e, clamp_action(actions[i]));
    reward[i] = (float)so.reward0;
    done[i] = so.done;
    nagari[i] = so.nagari;
    status[i] = (i16)so.status;
    committed[i] = so.committed;
    if (so.done) {  // the next game: its spare, dealt into the slot first if stale
      ++gen;
      ar.generation[i] = gen;
      const u64 seed = ar.base_seed + (u64)i + ar.stride * gen;
      ar.sampler[i] = sampler_seed(seed);
      if (sgen != gen) deal_into(seed, (u32)(i & 1), ar.spares + srow * kRowWords);
      e = unpack_row(ar.spares + srow * kRowWords);
    }
    const Packet pk = make_packet(e);
    FeatRow fr;
    feature_row(pk, c_stop_bits, fr);
    feature_record(fr, rb.rec[lane]);
    rb.legal[lane][0] = pk.head.legal.w0;
    rb.legal[lane][1] = pk.head.legal.w1;
    rb.legal[lane][2] = pk.head.legal.w2;
    player[i] = pk.head.player;
    obs_done[i] = e.done != 0;
    obs_status[i] = (i16)pk.head.status;
    pack_row(e, row);
  }
  __syncthreads();
  store_observation<kPlayClaim, kBf16, kRows>(rb, base, count, features, legal, &next_item);
  stage_out<kThreads, kRows>(rows, states, nullptr, base, count, n);
}

// ---------------------------------------------------------- branch + observe ----
// branch_indexed then observe_indexed of the children (the reference's callers do exactly
// this, python/cugo_ppo50.py:96-98), in one launch with the same outputs.  Two waves per
// tile of 64 children: wave 0 gathers the parents, steps the clones and builds the
// children's observation records in LDS; then wave 1 stores the observations while wave 0
// writes the child rows from registers (each lane its own row), so the children are never
// read back, and joins the stores after.
__global__ __launch_bounds__(kPlayThreads) void branch_observe_kernel(
    const u64* parents, i64 env_count, const i64* ids, const i64* actions, i64 n,
    u64* children, float* reward, u8* done, u8* nagari, i16* status, u8* committed,
    float* features, u8* legal, u8* player, u8* obs_done, i16* obs_status) {
  __shared__ ObserveTile t;
  __shared__ i64 tile_ids[kTile];
  __shared__ int next_item;  // store_observation's work counter
  const i64 base = tile_base();
  const int count = tile_count(base, n);
  const int tid = threadIdx.x;
  const int lane = tid & (kTile - 1);
  const int wave = tid / kTile;
  if (tid < count) tile_ids[tid] = ids[base + tid];
  if (tid == 0) next_item = 0;
  __syncthreads();
  // A plain gather loop: the batched form of stage_in measured 3.5 % slower here.
  for (int j = tid; j < count * kRowWords; j += kPlayThreads) {
    const int r = j / kRowWords;
    const i64 id = tile_ids[r];
    t.rows[j] = valid_id(id, env_count) ? parents[id * kRowWords + (j - r * kRowWords)] : 0ull;
  }
  __syncthreads();
  const bool active = wave == 0 && lane < count;
  // The clone is unpacked and stepped in one block before the rows are overwritten: an
  // Env unpacked before a barrier and stepped after it leaves an engine temporary in
  // private memory.
  Env e;  // the parent (a zero row for an invalid id), then the child
  const i64 i = base + lane;
  if (active) {
    e = unpack_row(t.rows + lane * kRowWords);
    if (valid_id(tile_ids[lane], env_count)) {
      const StepOut so = torch_step(e, clamp_action(actions[i]));
      reward[i] = (float)so.reward0;
      done[i] = so.done;
      nagari[i] = so.nagari;
      status[i] = (i16)so.status;
      committed[i] = so.committed;
    } else {  // torch50_ext.cu:108-118: a zero child, whose observation follows
      reward[i] = 0.0f;
      done[i] = 1;
      nagari[i] = 0;
      status[i] = CUGO_INVALID_INDEX_STATUS;
      committed[i] = 0;
    }
  }
  __syncthreads();  // rows are dead from here on; their bytes become the records
  if (active) {
    const Env seen = e;  // observed from a copy (see play_kernel)
    const Packet pk = make_packet(seen);
    FeatRow fr;
    feature_row(pk, c_stop_bits, fr);
    feature_record(fr, t.out.rec[lane]);
    t.out.legal[lane][0] = pk.head.legal.w0;
    t.out.legal[lane][1] = pk.head.legal.w1;
    t.out.legal[lane][2] = pk.head.legal.w2;
    player[i] = pk.head.player;
    obs_done[i] = seen.done != 0;
    obs_status[i] = (i16)pk.head.status;
  }
  __syncthreads();
  if (wave == 0) {
    if (lane < count) {
      u64 row[kRowWords];
      pack_row(e, row);
      u64* out = children + i * kRowWords;
#pragma unroll
      for (int k = 0; k < kRowWords; ++k) out[k] = row[k];
    }
  }
  // (Staging these rows through LDS as branch_kernel does measured 5 % slower here: wave
  // 0 joins the observation's stores later.)
  store_observation<2>(t.out, base, count, features, legal, &next_item);  // wave 0 after its rows
}

// ----------------------------------------------------------- calibration ----
// play_kernel's observation-row stores without the game, to measure what the memory
// system gives that store pattern: each 64-lane wave owns 64 consecutive rows of
// `row_f4` float4s and writes them 4 rows at a time, a row as float4 stores of 1 KiB
// (lane l writes float4 l + 64 k of the row), `steps` times; step s writes rows
// [s * rows, (s + 1) * rows) when `distinct`, else rows [0, rows) again.
__global__ __launch_bounds__(256) void store_probe_kernel(float4* out, i64 rows, int row_f4,
                                                          int steps, int distinct) {
  const int lane = threadIdx.x & 63;
  const i64 wave = ((i64)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  if (wave * 64 >= rows) return;
  const float4 v = make_float4(1.0f, 0.0f, 1.0f, 0.0f);
  for (int s = 0; s < steps; ++s) {
    float4* step = out + (distinct ? (i64)s * rows * row_f4 : 0);
    for (int r0 = 0; r0 < 64; r0 += 4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float4* row = step + (wave * 64 + r0 + q) * row_f4;
        for (int c = lane; c < row_f4; c += 64) row[c] = v;
      }
    }
  }
}

// -------------------------------------------------------------------- small ----
__global__ __launch_bounds__(256) void start_kernel(const u64* states, i64 n, i64* out) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const u64* w = states + i * kRowWords;
  Env e;
  e.hand0 = w[0]; e.hand1 = w[1]; e.floor = w[2]; e.cap0 = w[4]; e.cap1 = w[5];
  e.mission = w[10]; e.neutral = (u16)w[11]; e.actor = (u8)(w[9] >> 16);
  e.mtype = (u8)(w[18] >> 40); e.mmult = (u8)(w[18] >> 48); e.mm0 = (u8)(w[18] >> 56);
  e.mm1 = (u8)w[19];
  i64 o[kStartWords];
  pack_start(e, o);
  for (int k = 0; k < kStartWords; ++k) out[i * kStartWords + k] = o[k];
}

// One 8-byte word per lane: word j of the output is word j % 31 of row j / 31.
__global__ __launch_bounds__(256) void clone_kernel(const u64* states, i64 env_count,
                                                    const i64* ids, i64 n, u64* children) {
  const i64 words = n * kRowWords;
  for (i64 j = (i64)blockIdx.x * blockDim.x + threadIdx.x; j < words;
       j += (i64)gridDim.x * blockDim.x) {
    const i64 r = j / kRowWords;
    const i64 k = j - r * kRowWords;
    const i64 id = ids[r];
    children[j] = valid_id(id, env_count) ? states[id * kRowWords + k] : 0ull;
  }
}

__global__ __launch_bounds__(256) void hands_kernel(const u64* states, i64 env_count,
                                                    const i64* ids, i64 n, i64* hands) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const i64 id = ids[i];
  const bool ok = valid_id(id, env_count);
  hands[2 * i] = ok ? (i64)states[id * kRowWords + 0] : 0;
  hands[2 * i + 1] = ok ? (i64)states[id * kRowWords + 1] : 0;
}

__global__ __launch_bounds__(256) void stock_kernel(const u64* states, i64 env_count,
                                                    const i64* ids, i64 n, i64* stock) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const i64 id = ids[i];
  u64 packed = ~0ull;
  if (valid_id(id, env_count)) {
    Env e;
    e.stock = states[id * kRowWords + 3];
    e.rng = states[id * kRowWords + 6];
    packed = peek_stock(e);
  }
  stock[i] = (i64)packed;
}

// ------------------------------------------------------- random-policy driver ----
// Tile of 64 mask rows staged in LDS (coalesced dwords); lane r turns its row's 179
// bytes into three 64-bit words and picks the rank-th set bit.  A dword of four 0/1
// bytes becomes a nibble with one multiply: d * 0x00204081 = d + d<<7 + d<<14 + d<<21
// puts byte k's bit at position 21 + k with no other term landing in bits 21..24.
constexpr int kMaskWords = kTile * kActionCount / 4;  // 2,864

__device__ inline u32 nibble_of_bytes(u32 d) { return ((d * 0x00204081u) >> 21) & 0xFu; }

__global__ __launch_bounds__(kTile) void sample_kernel(const u8* legal, i64 n, u64* sampler,
                                                       i64* actions) {
  __shared__ u32 masks[kMaskWords + 2];  // +2: a row's last dword read may pass the tile
  const i64 base = tile_base();
  const int count = tile_count(base, n);
  const int lane = threadIdx.x;
  const u8* src = legal + base * kActionCount;
  const int bytes = count * kActionCount;
  const int full = bytes / 4;
  for (int w = lane; w < full; w += kTile) masks[w] = reinterpret_cast<const u32*>(src)[w];
  if (lane < 2) masks[kMaskWords + lane] = 0u;
  if (full * 4 < bytes && lane == 0) {  // partial last dword (only in a partial tile)
    u32 d = 0;
    for (int at = full * 4; at < bytes; ++at) d |= (u32)src[at] << (8 * (at - full * 4));
    masks[full] = d;
  }
  __syncthreads();
  if (lane >= count) return;
  const int b0 = lane * kActionCount;
  const int k0 = b0 >> 2;
  const int off = b0 & 3;  // the row starts at byte `off` of dword k0
  u64 w[3] = {0, 0, 0};    // bit 4j + i = byte i of dword k0 + j
#pragma unroll
  for (int j = 0; j < 46; ++j)
    w[j >> 4] |= (u64)nibble_of_bytes(masks[k0 + j]) << ((j & 15) * 4);
  // drop the `off` leading bits, keep 179
  const u64 m0 = (w[0] >> off) | (off ? w[1] << (64 - off) : 0ull);
  const u64 m1 = (w[1] >> off) | (off ? w[2] << (64 - off) : 0ull);
  const u64 m2 = (w[2] >> off) & ((1ull << (kActionCount - 128)) - 1ull);
  const i64 i = base + lane;
  u64 x = sampler[i];
  const i64 a = draw_legal(m0, m1, m2, x);
  if (a >= 0) sampler[i] = x;
  actions[i] = a;
}

__global__ __launch_bounds__(kTile) void reset_kernel(u64* states, const u8* done, i64 n,
                                                      u64 base_seed, u32* generation,
                                                      u64* sampler,
                                                      unsigned long long* completed) {
  __shared__ u64 rows[kTileWords];
  __shared__ int flags[kTile];
  const i64 base = tile_base();
  const int count = tile_count(base, n);
  const int lane = threadIdx.x;
  const bool reset = lane < count && done[base + lane] != 0;
  flags[lane] = reset;
  if (reset) {
    const i64 i = base + lane;
    const u32 gen = generation[i] + 1u;
    generation[i] = gen;
    const u64 seed = base_seed + (u64)i + (u64)n * gen;
    const Env e = create_env(seed, (u32)(i & 1));
    pack_row(e, rows + lane * kRowWords);
    sampler[i] = sampler_seed(seed);
  }
  const u64 ballot = __ballot(reset);
  if (completed != nullptr && lane == 0 && ballot != 0)
    atomicAdd(completed, (unsigned long long)__popcll(ballot));
  __syncthreads();
  u64* out = states + base * kRowWords;
  for (int j = lane; j < count * kRowWords; j += kTile)
    if (flags[j / kRowWords]) out[j] = rows[j];
}

// Pre-deals the next S games of each row where their spares are stale: generation
// g = generation[i] + k (k = 1 .. S) of row i goes to spare row (g & (S - 1)) * n + i, with
// spare_gen of that row = g.  Block b serves k = 1 + b / tiles, so the S deals of a row run
// side by side rather than one after another.
__global__ __launch_bounds__(kTile) void refill_kernel(u64* spares, u32* spare_gen,
                                                       const u32* generation, i64 n,
                                                       u64 base_seed, u64 stride,
                                                       u32 slot_mask, i64 tiles_per_slot) {
  __shared__ u64 rows[kTileWords];
  __shared__ int flags[kTile];
  __shared__ i64 dst_row[kTile];
  const u32 k = 1u + (u32)(blockIdx.x / tiles_per_slot);
  const i64 base = (i64)(blockIdx.x % tiles_per_slot) * kTile;
  const int count = tile_count(base, n);
  const int lane = threadIdx.x;
  const i64 i = base + lane;
  const u32 g = lane < count ? generation[i] + k : 0u;
  const i64 dst = (i64)(g & slot_mask) * n + i;
  const bool stale = lane < count && spare_gen[dst] != g;
  flags[lane] = stale;
  dst_row[lane] = dst;
  if (stale) {
    const u64 seed = base_seed + (u64)i + stride * g;
    pack_row(create_env(seed, (u32)(i & 1)), rows + lane * kRowWords);
    spare_gen[dst] = g;
  }
  __syncthreads();
  for (int j = lane; j < count * kRowWords; j += kTile) {
    const int r = j / kRowWords;
    if (flags[r]) spares[dst_row[r] * kRowWords + (j - r * kRowWords)] = rows[j];
  }
}

// reset_kernel's result, taking a finished row's next game from its pre-dealt spare
// (dealt inline only when the spare is stale).
__global__ __launch_bounds__(kTile) void reset_spare_kernel(u64* states, const u8* done, i64 n,
                                                            u64 base_seed, u64 stride,
                                                            u32* generation,
                                                            u64* sampler,
                                                            unsigned long long* completed,
                                                            const u64* spares,
                                                            const u32* spare_gen,
                                                            u32 slot_mask) {
  __shared__ u64 rows[kTileWords];
  __shared__ int flags[kTile];
  __shared__ i64 src_row[kTile];
  const i64 base = tile_base();
  const int count = tile_count(base, n);
  const int lane = threadIdx.x;
  const i64 i = base + lane;
  const bool reset = lane < count && done[i] != 0;
  u32 gen = 0;
  bool from_spare = false;
  if (reset) {
    gen = generation[i] + 1u;
    generation[i] = gen;
    const i64 src = (i64)(gen & slot_mask) * n + i;
    src_row[lane] = src;
    from_spare = spare_gen[src] == gen;
    sampler[i] = sampler_seed(base_seed + (u64)i + stride * gen);
  }
  // 1: copy the spare row, 2: the row dealt inline into LDS
  flags[lane] = reset ? (from_spare ? 1 : 2) : 0;
  if (reset && !from_spare)
    pack_row(create_env(base_seed + (u64)i + stride * gen, (u32)(i & 1)), rows + lane * kRowWords);
  const u64 ballot = __ballot(reset);
  if (completed != nullptr && lane == 0 && ballot != 0)
    atomicAdd(completed, (unsigned long long)__popcll(ballot));
  __syncthreads();
  // Consecutive lanes move consecutive words of the tile's flagged rows: independent,
  // coalesced loads, spare rows straight from HBM to HBM.
  u64* out = states + base * kRowWords;
  for (int j = lane; j < count * kRowWords; j += kTile) {
    const int r = j / kRowWords;
    const int f = flags[r];
    if (f == 1) out[j] = spares[src_row[r] * kRowWords + (j - r * kRowWords)];
    else if (f == 2) out[j] = rows[j];
  }
}

// ---------------------------------------------------------------- redeal ----
// _redeal (python/cugo_ppo50.py:122-148) on rows in place, given its random draws: the
// observer's opponent gets a new unrevealed hand from the cards the observer cannot see
// (the opponent's free cards and the stock), the rest becomes the stock, held follows the
// new hand and the row's RNG word is replaced.  keys [n, 50] are the uniforms the
// reference draws with torch.rand; the new free cards are the `count` unknown cards with
// the smallest keys (ties to the lower card id: the reference's argsort leaves tie order
// open).  One wavefront per row, lane j = card j.
constexpr int kWordHand0 = 0, kWordHand1 = 1, kWordStock = 3, kWordRng = 6;
constexpr int kWordHeld0 = 20, kWordHeld1 = 21, kWordRev0 = 22, kWordRev1 = 23;

__global__ __launch_bounds__(256) void redeal_kernel(u64* states, const i64* seat,
                                                     const float* keys, const i64* rng, i64 n) {
  const int lane = threadIdx.x & 63;
  const i64 r = (i64)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= n) return;
  u64* w = states + r * kRowWords;
  const bool s0 = seat[r] == 0;
  const u64 hand = s0 ? w[kWordHand1] : w[kWordHand0];
  const u64 fixed = hand & (s0 ? w[kWordRev1] : w[kWordRev0]);  // shown by a shake
  const u64 held = s0 ? w[kWordHeld1] : w[kWordHeld0];
  const u64 free_cards = hand & ~fixed;
  const u64 unknown = free_cards | w[kWordStock];
  const u32 count = popc(free_cards);
  const bool mine = lane < 50 && ((unknown >> lane) & 1ull);
  const float key = mine ? keys[r * 50 + lane] : 2.0f;
  u32 rank = 0;
  for (int k = 0; k < 50; ++k) {
    const float other = __shfl(key, k);
    rank += (other < key || (other == key && k < lane)) ? 1u : 0u;
  }
  const u64 new_free = __ballot(mine && rank < count);
  if (lane != 0) return;
  const u64 new_hand = fixed | new_free;
  const u64 new_held = (held & ~hand) | new_hand;
  w[kWordStock] = unknown & ~new_free;
  w[s0 ? kWordHand1 : kWordHand0] = new_hand;
  w[s0 ? kWordHeld1 : kWordHeld0] = new_held;
  w[kWordRng] = (u64)rng[r];
}

// redeal_worlds' acceptance test and copy (python/cugo_ppo50.py:151-172): candidate j, a
// redealt copy of row missing[j] % rows, is kept when its observer's features and legal
// mask equal the real deal's value for value (torch's ==, then all over the row); a kept
// candidate's row goes to row missing[j] of out (rows of out outside [0, out_rows) are
// never written: such a candidate is reported as not kept).  One wavefront per candidate.
__global__ __launch_bounds__(256) void accept_worlds_kernel(
    const float* f, const u8* l, const float* f_real, const u8* l_real, const i64* missing,
    i64 rows, i64 n, const u64* cand, u64* out, i64 out_rows, u8* same) {
  const int lane = threadIdx.x & 63;
  const i64 j = (i64)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (j >= n) return;
  const i64 dst = missing[j];
  const bool in = dst >= 0 && dst < out_rows;
  const i64 r = in ? dst % rows : 0;
  bool eq = in;
  for (int k = lane; k < kFeatureCount; k += 64)
    eq = eq && f[j * kFeatureCount + k] == f_real[r * kFeatureCount + k];
  for (int k = lane; k < kActionCount; k += 64)
    eq = eq && l[j * kActionCount + k] == l_real[r * kActionCount + k];
  const bool all = __ballot(!eq) == 0;  // every lane of the row agrees
  if (lane == 0) same[j] = all ? 1 : 0;
  if (all && lane < kRowWords) out[dst * kRowWords + lane] = cand[j * kRowWords + lane];
}

// ------------------------------------------------------- canonical rollout ----
// rollout_canonical_torch50 (torch50.h:598-619): each lane deals game i from seeds[i] /
// first[i] and plays it to the end with the canonical action in registers, then writes
// its five digest words; a tile's 64 x 5 words leave through LDS as one contiguous block.
// The whole game is integer work with 56 bytes of HBM traffic, so the kernel is bound by
// instruction issue; one wave per workgroup lets a wave whose games end early retire.
constexpr int kCanonicalWords = 5;

__global__ __launch_bounds__(kTile) void canonical_kernel(const i64* seeds, const i64* first,
                                                          i64 n, u32 max_actions, i64* out) {
  __shared__ i64 digest[kTile * kCanonicalWords];
  const i64 base = tile_base();
  const int count = tile_count(base, n);
  const int lane = threadIdx.x;
  if (lane < count) {
    Env e = create_env((u64)seeds[base + lane], (u32)(first[base + lane] & 1));
    rollout_canonical(e, max_actions, digest + lane * kCanonicalWords);
  }
  __syncthreads();
  i64* dst = out + base * kCanonicalWords;
  for (int j = lane; j < count * kCanonicalWords; j += kTile) dst[j] = digest[j];
}

__global__ __launch_bounds__(256) void seed_kernel(i64 n, u64 base_seed, const u32* generation,
                                                   u64* sampler) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const u64 gen = generation != nullptr ? generation[i] : 0u;
  sampler[i] = sampler_seed(base_seed + (u64)i + (u64)n * gen);
}

// ------------------------------------------------------ allocation-free play ----
// The spares of cugo_play_random_noalloc: kNoAllocSlots pre-dealt games for each of up to
// CUGO_NOALLOC_MAX_ROWS rows (slot-major, 31 words a row), then their spare_gen words
// (uint32, two a word).  Allocated with the code object on each device the library runs
// on and held until the process ends (31.5 MiB).  Host code never passes `scratch` itself
// to a kernel: it passes the device address that hipGetSymbolAddress returns for it.
constexpr int kNoAllocSlots = 2;
constexpr i64 kNoAllocSpareWords = (i64)kNoAllocSlots * CUGO_NOALLOC_MAX_ROWS * kRowWords;
constexpr i64 kNoAllocGenWords = (i64)kNoAllocSlots * CUGO_NOALLOC_MAX_ROWS / 2;
static __device__ __align__(256) u64 scratch[kNoAllocSpareWords + kNoAllocGenWords];

__global__ __launch_bounds__(256) void clear_u32_kernel(u32* words, i64 n) {
  const i64 i = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) words[i] = 0u;
}

}  // namespace cugo_amd

// ===================================================================== C ABI ====
using namespace cugo_amd;

namespace {
inline unsigned tiles(int64_t n) { return (unsigned)((n + kTile - 1) / kTile); }
// Spare slots per row: 1, 2 or 4 (a power of two: a generation's slot is a mask of it).
inline bool valid_slots(int64_t s) { return s == 1 || s == 2 || s == 4; }

// Compute units of the current device (cached per device).
inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// step_kernel launch: two waves per tile while all tiles fit at once (four per CU).
// Games a tile of the observe and step kernels, by batch.  A wavefront runs the union of
// its games' rule paths, so at small batches (every tile resident, most SIMDs without a
// computing wavefront) smaller tiles finish sooner; at large ones the wavefronts of
// 64 games issue fewer instructions in all.  Measured on MI355X (us a launch for 64 / 32 /
// 16 games a tile, graphs of 20 launches on mid-game rows):
//   observe            n = 4,096: 20.6 / 15.7 / 12.4    16,384: 22.8 / 18.8 / 16.5
//                      32,768: 28.5 / 24.9 / 31.5       65,536: 41.5 / 46.5 / 50.2
//   step_events_indexed 2,048: 19.3 / 18.7 / 14.5       8,192: 20.0 / 18.9 / 19.9
//                      32,768: 24.5 / 21.5 / 22.6       65,536: 26.6 / 47.8 / 41.0
inline int obs_rows(int64_t n) { return n <= 16384 ? 16 : n <= 32768 ? 32 : kTile; }
inline int step_rows(int64_t n) { return n <= 4096 ? 16 : n <= 32768 ? 32 : kTile; }

template <bool kIndexed, bool kSample, bool kBf16, class... Args>
inline void launch_observe(int64_t n, hipStream_t stream, Args... args) {
  switch (obs_rows(n)) {
    case 16:
      observe_kernel<kIndexed, kSample, kBf16, 16>
          <<<(unsigned)((n + 15) / 16), kObsThreads, 0, stream>>>(args...);
      break;
    case 32:
      observe_kernel<kIndexed, kSample, kBf16, 32>
          <<<(unsigned)((n + 31) / 32), kObsThreads, 0, stream>>>(args...);
      break;
    default:
      observe_kernel<kIndexed, kSample, kBf16, kTile><<<tiles(n), kObsThreads, 0, stream>>>(args...);
  }
}

template <int kMode, bool kEvents, class... Args>
inline void launch_step(int64_t n, hipStream_t stream, Args... args) {
  const int rows = step_rows(n);
  if (rows == 16) {
    step_kernel<kMode, kEvents, 64, 16><<<(unsigned)((n + 15) / 16), 64, 0, stream>>>(args...);
  } else if (rows == 32) {
    step_kernel<kMode, kEvents, 128, 32><<<(unsigned)((n + 31) / 32), 128, 0, stream>>>(args...);
  } else if ((int64_t)tiles(n) <= 4 * (int64_t)device_cus()) {
    step_kernel<kMode, kEvents, 128><<<tiles(n), 128, 0, stream>>>(args...);
  } else {
    step_kernel<kMode, kEvents, 64><<<tiles(n), 64, 0, stream>>>(args...);
  }
}
inline unsigned blocks256(int64_t n) { return (unsigned)((n + 255) / 256); }
inline int launched() { return (int)hipGetLastError(); }
constexpr int kBadArgument = -22;
}  // namespace

extern "C" {

int cugo_version(void) { return (1 << 16) | 0; }

int cugo_create(const int64_t* seeds, const int64_t* first, int64_t n, uint8_t* states,
                hipStream_t stream) {
  if (n < 0 || (n > 0 && (!seeds || !first || !states))) return kBadArgument;
  if (n == 0) return 0;
  create_kernel<<<tiles(n), kTile, 0, stream>>>(seeds, first, n,
                                                reinterpret_cast<u64*>(states));
  return launched();
}

int cugo_observe(const uint8_t* states, int64_t n, float* features, uint8_t* legal,
                 uint8_t* player, uint8_t* done, int16_t* status, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!states || !features || !legal || !player || !done || !status)))
    return kBadArgument;
  if (n == 0) return 0;
  launch_observe<false, false, false>(n, stream, reinterpret_cast<const u64*>(states), n,
                                      (const i64*)nullptr, n, (void*)features, legal, player,
                                      done, status, (u64*)nullptr, (i64*)nullptr);
  return launched();
}

int cugo_observe_bf16(const uint8_t* states, int64_t n, uint16_t* features, uint8_t* legal,
                      uint8_t* player, uint8_t* done, int16_t* status, uint64_t* sampler,
                      int64_t* actions, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!states || !features || !legal || !player || !done || !status)) ||
      (sampler == nullptr) != (actions == nullptr))
    return kBadArgument;
  if (n == 0) return 0;
  if (sampler != nullptr)
    launch_observe<false, true, true>(n, stream, reinterpret_cast<const u64*>(states), n,
                                      (const i64*)nullptr, n, (void*)features, legal, player,
                                      done, status, reinterpret_cast<u64*>(sampler), actions);
  else
    launch_observe<false, false, true>(n, stream, reinterpret_cast<const u64*>(states), n,
                                       (const i64*)nullptr, n, (void*)features, legal, player,
                                       done, status, (u64*)nullptr, (i64*)nullptr);
  return launched();
}

int cugo_observe_sample(const uint8_t* states, int64_t n, float* features, uint8_t* legal,
                        uint8_t* player, uint8_t* done, int16_t* status, uint64_t* sampler,
                        int64_t* actions, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!states || !features || !legal || !player || !done || !status ||
                          !sampler || !actions)))
    return kBadArgument;
  if (n == 0) return 0;
  launch_observe<false, true, false>(n, stream, reinterpret_cast<const u64*>(states), n,
                                     (const i64*)nullptr, n, (void*)features, legal, player,
                                     done, status, reinterpret_cast<u64*>(sampler), actions);
  return launched();
}

int cugo_observe_indexed(const uint8_t* states, int64_t env_count, const int64_t* ids,
                         int64_t n, float* features, uint8_t* legal, uint8_t* player,
                         uint8_t* done, int16_t* status, hipStream_t stream) {
  if (n < 0 || env_count < 0 ||
      (n > 0 && (!ids || !features || !legal || !player || !done || !status)))
    return kBadArgument;
  if (n == 0) return 0;
  launch_observe<true, false, false>(n, stream, reinterpret_cast<const u64*>(states), env_count,
                                     ids, n, (void*)features, legal, player, done, status,
                                     (u64*)nullptr, (i64*)nullptr);
  return launched();
}

int cugo_step(uint8_t* states, const int64_t* actions, int64_t n, float* reward, uint8_t* done,
              uint8_t* nagari, int16_t* status, uint8_t* committed, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!states || !actions || !reward || !done || !nagari || !status ||
                          !committed)))
    return kBadArgument;
  if (n == 0) return 0;
  launch_step<0, false>(n, stream, 
      reinterpret_cast<u64*>(states), n, nullptr, actions, n, reward, done, nagari,
      status, committed, nullptr, AutoReset{});
  return launched();
}

}  // extern "C"

namespace {
// play_random and its recording form: step_rows = 0 keeps only the last step's outputs.
int play_random(uint8_t* states, int64_t n, uint64_t* sampler, float* features,
                uint8_t* legal, uint8_t* player, uint8_t* obs_done, int16_t* obs_status,
                int64_t* actions, float* reward, uint8_t* done, uint8_t* nagari,
                int16_t* status, uint8_t* committed, uint64_t base_seed, int64_t seed_stride,
                uint32_t* generation, uint8_t* spares, const uint32_t* spare_gen,
                int64_t spare_slots, int64_t steps, int64_t step_rows, hipStream_t stream) {
  if (n < 0 || seed_stride < 0 || steps < 1 || steps > kMaxPlaySteps ||
      !valid_slots(spare_slots) ||
      (n > 0 && (!states || !sampler || !features || !legal || !player || !obs_done ||
                 !obs_status || !actions || !reward || !done || !nagari || !status ||
                 !committed || !generation || !spares || !spare_gen)))
    return kBadArgument;
  if (n == 0) return 0;
  const AutoReset ar{base_seed, (u64)seed_stride, generation, reinterpret_cast<u64*>(sampler),
                     reinterpret_cast<u64*>(spares), spare_gen, n, (u32)(spare_slots - 1)};
  play_kernel<<<tiles(n), kPlayThreads, 0, stream>>>(
      reinterpret_cast<u64*>(states), n, reinterpret_cast<u64*>(sampler), features, legal,
      player, obs_done, obs_status, actions, reward, done, nagari, status, committed, ar,
      (int)steps, step_rows);
  return launched();
}
}  // namespace

extern "C" {

int cugo_play_random(uint8_t* states, int64_t n, uint64_t* sampler, float* features,
                     uint8_t* legal, uint8_t* player, uint8_t* obs_done, int16_t* obs_status,
                     int64_t* actions, float* reward, uint8_t* done, uint8_t* nagari,
                     int16_t* status, uint8_t* committed, uint64_t base_seed,
                     int64_t seed_stride, uint32_t* generation, uint8_t* spares,
                     const uint32_t* spare_gen, int64_t spare_slots, int64_t steps,
                     hipStream_t stream) {
  return play_random(states, n, sampler, features, legal, player, obs_done, obs_status,
                     actions, reward, done, nagari, status, committed, base_seed, seed_stride,
                     generation, spares, spare_gen, spare_slots, steps, 0, stream);
}

int cugo_play_random_record(uint8_t* states, int64_t n, uint64_t* sampler, float* features,
                            uint8_t* legal, uint8_t* player, uint8_t* obs_done,
                            int16_t* obs_status, int64_t* actions, float* reward,
                            uint8_t* done, uint8_t* nagari, int16_t* status,
                            uint8_t* committed, uint64_t base_seed, int64_t seed_stride,
                            uint32_t* generation, uint8_t* spares, const uint32_t* spare_gen,
                            int64_t spare_slots, int64_t steps, int64_t step_rows,
                            hipStream_t stream) {
  // Step s's legal-mask block starts at byte s * step_rows * 179, which the kernel's
  // 32-bit mask stores need 4-byte aligned.
  if (step_rows < n || step_rows % 4 != 0) return kBadArgument;
  return play_random(states, n, sampler, features, legal, player, obs_done, obs_status,
                     actions, reward, done, nagari, status, committed, base_seed, seed_stride,
                     generation, spares, spare_gen, spare_slots, steps, step_rows, stream);
}

int cugo_branch_observe_indexed(const uint8_t* states, int64_t env_count, const int64_t* ids,
                                const int64_t* actions, int64_t n, uint8_t* children,
                                float* reward, uint8_t* done, uint8_t* nagari, int16_t* status,
                                uint8_t* committed, float* features, uint8_t* legal,
                                uint8_t* player, uint8_t* obs_done, int16_t* obs_status,
                                hipStream_t stream) {
  if (n < 0 || env_count < 0 ||
      (n > 0 && (!ids || !actions || !children || !reward || !done || !nagari || !status ||
                 !committed || !features || !legal || !player || !obs_done || !obs_status)))
    return kBadArgument;
  if (n == 0) return 0;
  branch_observe_kernel<<<tiles(n), kPlayThreads, 0, stream>>>(
      reinterpret_cast<const u64*>(states), env_count, ids, actions, n,
      reinterpret_cast<u64*>(children), reward, done, nagari, status, committed, features,
      legal, player, obs_done, obs_status);
  return launched();
}

int cugo_step_reset_spares(uint8_t* states, const int64_t* actions, int64_t n, float* reward,
                           uint8_t* done, uint8_t* nagari, int16_t* status, uint8_t* committed,
                           uint64_t base_seed, int64_t seed_stride, uint32_t* generation,
                           uint64_t* sampler, const uint8_t* spares, const uint32_t* spare_gen,
                           int64_t spare_slots, hipStream_t stream) {
  if (n < 0 || seed_stride < 0 || !valid_slots(spare_slots) ||
      (n > 0 && (!states || !actions || !reward || !done || !nagari || !status || !committed ||
                 !generation || !sampler || !spares || !spare_gen)))
    return kBadArgument;
  if (n == 0) return 0;
  // step_kernel<3> only reads the spares
  const AutoReset ar{base_seed, (u64)seed_stride, generation, reinterpret_cast<u64*>(sampler),
                     const_cast<u64*>(reinterpret_cast<const u64*>(spares)), spare_gen, n,
                     (u32)(spare_slots - 1)};
  launch_step<3, false>(n, stream, reinterpret_cast<u64*>(states), n, nullptr, actions, n,
                        reward, done, nagari, status, committed, nullptr, ar);
  return launched();
}

int cugo_step_observe_spares(uint8_t* states, const int64_t* actions, int64_t n, float* reward,
                             uint8_t* done, uint8_t* nagari, int16_t* status,
                             uint8_t* committed, uint64_t base_seed, int64_t seed_stride,
                             uint32_t* generation, uint64_t* sampler, uint8_t* spares,
                             const uint32_t* spare_gen, int64_t spare_slots, int features_dtype,
                             void* features, uint8_t* legal, uint8_t* player,
                             uint8_t* obs_done, int16_t* obs_status, hipStream_t stream) {
  if (n < 0 || seed_stride < 0 || !valid_slots(spare_slots) ||
      (features_dtype != CUGO_DTYPE_F32 && features_dtype != CUGO_DTYPE_BF16) ||
      (n > 0 && (!states || !actions || !reward || !done || !nagari || !status || !committed ||
                 !generation || !sampler || !spares || !spare_gen || !features || !legal ||
                 !player || !obs_done || !obs_status)))
    return kBadArgument;
  if (n == 0) return 0;
  const AutoReset ar{base_seed, (u64)seed_stride, generation, reinterpret_cast<u64*>(sampler),
                     reinterpret_cast<u64*>(spares), spare_gen, n, (u32)(spare_slots - 1)};
  // Games a tile: measured on MI355X at 32,768 rows (the PPO rollout's batch), us a launch
  // for (games, threads): (64, 128) 54.0, (32, 128) 44.2, (32, 64) 50.3, (24, 64) 50.1,
  // (16, 64) 45.5, (16, 128) 71.9.  A wavefront runs the union of its games' rule paths, so
  // fewer games a wavefront execute fewer divergent branches, while more wavefronts than
  // the ~210 VGPRs let a SIMD hold (two) cost a second round.
  constexpr int kRows = kStepObserveRows, kThreads = kPlayThreads;
  if (features_dtype == CUGO_DTYPE_BF16)
    step_observe_kernel<true, kRows, kThreads><<<(unsigned)((n + kRows - 1) / kRows), kThreads,
                                                0, stream>>>(
        reinterpret_cast<u64*>(states), n, actions, reward, done, nagari, status, committed, ar,
        features, legal, player, obs_done, obs_status);
  else
    step_observe_kernel<false, kRows, kThreads><<<(unsigned)((n + kRows - 1) / kRows), kThreads,
                                                 0, stream>>>(
        reinterpret_cast<u64*>(states), n, actions, reward, done, nagari, status, committed, ar,
        features, legal, player, obs_done, obs_status);
  return launched();
}

int cugo_step_indexed(uint8_t* states, int64_t env_count, const int64_t* ids,
                      const int64_t* actions, int64_t n, float* reward, uint8_t* done,
                      uint8_t* nagari, int16_t* status, uint8_t* committed,
                      hipStream_t stream) {
  if (n < 0 || env_count < 0 ||
      (n > 0 && (!ids || !actions || !reward || !done || !nagari || !status || !committed)))
    return kBadArgument;
  if (n == 0) return 0;
  launch_step<1, false>(n, stream, 
      reinterpret_cast<u64*>(states), env_count, ids, actions, n, reward, done,
      nagari, status, committed, nullptr, AutoReset{});
  return launched();
}

int cugo_step_events_indexed(uint8_t* states, int64_t env_count, const int64_t* ids,
                             const int64_t* actions, int64_t n, float* reward, uint8_t* done,
                             uint8_t* nagari, int16_t* status, uint8_t* committed,
                             int64_t* events, hipStream_t stream) {
  if (n < 0 || env_count < 0 ||
      (n > 0 && (!ids || !actions || !reward || !done || !nagari || !status || !committed ||
                 !events)))
    return kBadArgument;
  if (n == 0) return 0;
  launch_step<1, true>(n, stream, 
      reinterpret_cast<u64*>(states), env_count, ids, actions, n, reward, done,
      nagari, status, committed, events, AutoReset{});
  return launched();
}

int cugo_start(const uint8_t* states, int64_t n, int64_t* out, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!states || !out))) return kBadArgument;
  if (n == 0) return 0;
  start_kernel<<<blocks256(n), 256, 0, stream>>>(reinterpret_cast<const u64*>(states), n, out);
  return launched();
}

int cugo_store_probe(void* out, int64_t rows, int64_t row_bytes, int64_t steps, int distinct,
                     hipStream_t stream) {
  if (rows < 0 || rows % 64 != 0 || row_bytes <= 0 || row_bytes % 16 != 0 ||
      row_bytes > (1 << 20) || steps < 0 || steps > (1 << 16) || (rows > 0 && !out))
    return kBadArgument;
  if (rows == 0 || steps == 0) return 0;
  const int64_t waves = rows / 64;
  store_probe_kernel<<<(unsigned)((waves + 3) / 4), 256, 0, stream>>>(
      reinterpret_cast<float4*>(out), rows, (int)(row_bytes / 16), (int)steps, distinct != 0);
  return launched();
}

int cugo_clone_indexed(const uint8_t* states, int64_t env_count, const int64_t* ids, int64_t n,
                       uint8_t* children, hipStream_t stream) {
  if (n < 0 || env_count < 0 || (n > 0 && (!ids || !children))) return kBadArgument;
  if (n == 0) return 0;
  const int64_t words = n * kRowWords;
  int64_t grid = (words + 255) / 256;
  if (grid > 65536) grid = 65536;
  clone_kernel<<<(unsigned)grid, 256, 0, stream>>>(reinterpret_cast<const u64*>(states),
                                                   env_count, ids, n,
                                                   reinterpret_cast<u64*>(children));
  return launched();
}

int cugo_branch_indexed(const uint8_t* states, int64_t env_count, const int64_t* ids,
                        const int64_t* actions, int64_t n, uint8_t* children, float* reward,
                        uint8_t* done, uint8_t* nagari, int16_t* status, uint8_t* committed,
                        hipStream_t stream) {
  if (n < 0 || env_count < 0 ||
      (n > 0 && (!ids || !actions || !children || !reward || !done || !nagari || !status ||
                 !committed)))
    return kBadArgument;
  if (n == 0) return 0;
  branch_kernel<kTile><<<tiles(n), kTile, 0, stream>>>(reinterpret_cast<const u64*>(states),
                                                env_count, ids, actions, n,
                                                reinterpret_cast<u64*>(children), reward,
                                                done, nagari, status, committed);
  return launched();
}

int cugo_hands_indexed(const uint8_t* states, int64_t env_count, const int64_t* ids, int64_t n,
                       int64_t* hands, hipStream_t stream) {
  if (n < 0 || env_count < 0 || (n > 0 && (!ids || !hands))) return kBadArgument;
  if (n == 0) return 0;
  hands_kernel<<<blocks256(n), 256, 0, stream>>>(reinterpret_cast<const u64*>(states),
                                                 env_count, ids, n, hands);
  return launched();
}

int cugo_stock_indexed(const uint8_t* states, int64_t env_count, const int64_t* ids, int64_t n,
                       int64_t* stock, hipStream_t stream) {
  if (n < 0 || env_count < 0 || (n > 0 && (!ids || !stock))) return kBadArgument;
  if (n == 0) return 0;
  stock_kernel<<<blocks256(n), 256, 0, stream>>>(reinterpret_cast<const u64*>(states),
                                                 env_count, ids, n, stock);
  return launched();
}

int cugo_sample_uniform(const uint8_t* legal, int64_t n, uint64_t* sampler, int64_t* actions,
                        hipStream_t stream) {
  if (n < 0 || (n > 0 && (!legal || !sampler || !actions))) return kBadArgument;
  if (n == 0) return 0;
  sample_kernel<<<tiles(n), kTile, 0, stream>>>(legal, n, sampler, actions);
  return launched();
}

int cugo_reset_done(uint8_t* states, const uint8_t* done, int64_t n, uint64_t base_seed,
                    uint32_t* generation, uint64_t* sampler, unsigned long long* completed,
                    hipStream_t stream) {
  if (n < 0 || (n > 0 && (!states || !done || !generation || !sampler))) return kBadArgument;
  if (n == 0) return 0;
  reset_kernel<<<tiles(n), kTile, 0, stream>>>(reinterpret_cast<u64*>(states), done, n,
                                               base_seed, generation, sampler, completed);
  return launched();
}

int cugo_refill_spares(uint8_t* spares, uint32_t* spare_gen, const uint32_t* generation,
                       int64_t n, uint64_t base_seed, int64_t seed_stride, int64_t spare_slots,
                       hipStream_t stream) {
  if (n < 0 || seed_stride < 0 || !valid_slots(spare_slots) ||
      (n > 0 && (!spares || !spare_gen || !generation)))
    return kBadArgument;
  if (n == 0) return 0;
  const i64 per_slot = tiles(n);
  refill_kernel<<<(unsigned)(per_slot * spare_slots), kTile, 0, stream>>>(
      reinterpret_cast<u64*>(spares), spare_gen, generation, n, base_seed, (u64)seed_stride,
      (u32)(spare_slots - 1), per_slot);
  return launched();
}

int cugo_reset_done_spares(uint8_t* states, const uint8_t* done, int64_t n, uint64_t base_seed,
                           int64_t seed_stride, uint32_t* generation, uint64_t* sampler,
                           unsigned long long* completed, const uint8_t* spares,
                           const uint32_t* spare_gen, int64_t spare_slots, hipStream_t stream) {
  if (n < 0 || seed_stride < 0 || !valid_slots(spare_slots) ||
      (n > 0 && (!states || !done || !generation || !sampler || !spares || !spare_gen)))
    return kBadArgument;
  if (n == 0) return 0;
  reset_spare_kernel<<<tiles(n), kTile, 0, stream>>>(
      reinterpret_cast<u64*>(states), done, n, base_seed, (u64)seed_stride, generation, sampler,
      completed, reinterpret_cast<const u64*>(spares), spare_gen, (u32)(spare_slots - 1));
  return launched();
}

int cugo_redeal(uint8_t* states, const int64_t* seat, const float* keys, const int64_t* rng,
                int64_t n, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!states || !seat || !keys || !rng))) return kBadArgument;
  if (n == 0) return 0;
  redeal_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(reinterpret_cast<u64*>(states), seat,
                                                            keys, rng, n);
  return launched();
}

int cugo_accept_worlds(const float* features, const uint8_t* legal, const float* real_features,
                       const uint8_t* real_legal, const int64_t* missing, int64_t rows,
                       int64_t n, const uint8_t* candidates, uint8_t* out, int64_t out_rows,
                       uint8_t* same, hipStream_t stream) {
  if (n < 0 || (n > 0 && (rows < 1 || !features || !legal || !real_features || !real_legal ||
                          !missing || !candidates || !out || !same)))
    return kBadArgument;
  if (n == 0) return 0;
  accept_worlds_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(
      features, legal, real_features, real_legal, missing, rows, n,
      reinterpret_cast<const u64*>(candidates), reinterpret_cast<u64*>(out), out_rows, same);
  return launched();
}

int cugo_seed_samplers(int64_t n, uint64_t base_seed, const uint32_t* generation,
                       uint64_t* sampler, hipStream_t stream) {
  if (n < 0 || (n > 0 && !sampler)) return kBadArgument;
  if (n == 0) return 0;
  seed_kernel<<<blocks256(n), 256, 0, stream>>>(n, base_seed, generation, sampler);
  return launched();
}

// ---------------------------------------------------- allocation-free play ----
}  // extern "C"

namespace {
// The device address of `scratch` on each device, looked up on the first
// cugo_play_random_noalloc call with that device current.
std::mutex g_scratch_lock;
u64* g_scratch[64] = {};

int scratch_on_current_device(u64** out) {
  int dev = 0;
  const hipError_t got = hipGetDevice(&dev);
  if (got != hipSuccess) return (int)got;
  if (dev < 0 || dev >= 64) return kBadArgument;
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(cugo_amd::scratch));
    if (rc != hipSuccess) return (int)rc;
    if (ptr == nullptr) return (int)hipErrorInvalidSymbol;
    g_scratch[dev] = static_cast<u64*>(ptr);
  }
  *out = g_scratch[dev];
  return 0;
}
}  // namespace

extern "C" {

int cugo_play_random_noalloc(uint8_t* states, int64_t n, uint64_t* sampler, float* features,
                             uint8_t* legal, uint8_t* player, uint8_t* obs_done,
                             int16_t* obs_status, int64_t* actions, float* reward,
                             uint8_t* done, uint8_t* nagari, int16_t* status,
                             uint8_t* committed, uint64_t base_seed, int64_t seed_stride,
                             uint32_t* generation, int64_t steps, hipStream_t stream) {
  if (n > CUGO_NOALLOC_MAX_ROWS) return CUGO_ERROR_SCRATCH_LIMIT;
  if (n < 0 || seed_stride < 0 || steps < 1 || steps > kMaxPlaySteps ||
      (n > 0 && (!states || !sampler || !features || !legal || !player || !obs_done ||
                 !obs_status || !actions || !reward || !done || !nagari || !status ||
                 !committed || !generation)))
    return kBadArgument;
  if (n == 0) return 0;
  u64* base = nullptr;
  const int rc = scratch_on_current_device(&base);
  if (rc != 0) return rc;
  u64* spares = base;
  u32* spare_gen = reinterpret_cast<u32*>(base + kNoAllocSpareWords);
  // The previous call's spares belong to other games: mark every slot stale (a fill
  // kernel, so the sequence can be captured into a graph), then deal them all.
  const i64 slot_rows = (i64)kNoAllocSlots * n;
  clear_u32_kernel<<<blocks256(slot_rows), 256, 0, stream>>>(spare_gen, slot_rows);
  const i64 per_slot = tiles(n);
  refill_kernel<<<(unsigned)(per_slot * kNoAllocSlots), kTile, 0, stream>>>(
      spares, spare_gen, generation, n, base_seed, (u64)seed_stride,
      (u32)(kNoAllocSlots - 1), per_slot);
  const int queued = launched();
  if (queued != 0) return queued;
  return play_random(states, n, sampler, features, legal, player, obs_done, obs_status,
                     actions, reward, done, nagari, status, committed, base_seed, seed_stride,
                     generation, reinterpret_cast<uint8_t*>(spares), spare_gen, kNoAllocSlots,
                     steps, 0, stream);
}

int cugo_rollout_canonical(const int64_t* seeds, const int64_t* first_players, int64_t n,
                           int64_t max_actions, int64_t* digest, hipStream_t stream) {
  if (n < 0 || max_actions < 0 || max_actions > 0xFFFF ||
      (n > 0 && (!seeds || !first_players || !digest)))
    return kBadArgument;
  if (n == 0) return 0;
  canonical_kernel<<<tiles(n), kTile, 0, stream>>>(seeds, first_players, n, (u32)max_actions,
                                                   digest);
  return launched();
}

}  // extern "C"
