// Fused forward pass of the residual MLP actor on MFMA, for gfx950.
//
// The actor (cugo_amd/rollout.py ResidualMlpActor, the PPO rollout's policy):
//   h = x W_in^T + b_in
//   for each block:  h = h + W2 relu(W1 LN(h) + b1) + b2       (LN with its own affine)
//   z = LN(h);  logits = z W_l^T + b_l;  value = z w_v + b_v
// With one GEMM per layer through a library, every layer reads and writes a [B, 512]
// activation tensor in HBM and each residual add + LayerNorm is another pass over two of
// them.  Here a workgroup owns 128 rows for the whole network: the residual stream h stays
// in the wavefronts' MFMA accumulators (fp32), each layer's bf16 input sits in LDS, and
// only the weights stream in from L2.
//
// Why 128 rows: every workgroup reads all 4.07 MB of weights once, so the weight bytes a
// CU pulls through its L1 per FLOP fall as the rows of a tile grow.  With 64-row tiles the
// L1's fill rate (about 17 bytes a cycle per CU, its miss queue full a third of the time)
// bounded the kernel with the MFMA pipe a quarter busy.
//
// Layout of the work (512 threads, 8 wavefronts, two per SIMD, one workgroup per CU; 256
// registers a lane, the accumulators in AGPRs):
//   * wavefront w owns columns [64 w, 64 w + 64) of h for all 128 rows: 8 x 4 tiles of
//     16 x 16 (128 accumulator registers), v_mfma_f32_16x16x32_bf16 over K in steps of 32
//     (lane l holds A[l % 16][8 (l / 16) + 0..7], B[8 (l / 16) + 0..7][l % 16] and
//     D[4 (l / 16) + 0..3][l % 16]);
//   * LDS holds Z, the 128 x 512 bf16 input of the current layer (128 KiB), and U, one
//     128-column chunk of relu(fc1) (32 KiB): fc1 and fc2 run chunk by chunk, fc1's chunk
//     on a 2 x 4 grid of wavefronts (64 rows x 32 columns each) into U, then h += U W2's
//     matching K slice.  Z and U store 16-byte group g of row r at g ^ (r & 7), so the 16
//     rows of an A fragment read 8 different bank slots without padding (160 KiB in all);
//   * the input x passes through Z in two column slices ([0, 512) and [512, 768));
//   * B fragments come from weights packed once in fragment order (cugo_mlp_pack_weight):
//     the 64 lanes' 8 values of one (16-row tile, K step) are 1 KiB of contiguous memory,
//     so one load instruction is a contiguous 1 KiB read; they sit in a ring of registers
//     a few K steps ahead of the MFMAs, and the next step's A fragments are read from LDS
//     while the current step's MFMAs issue;
//   * LayerNorm: per-row sum and sum of squares over a wavefront's 64 columns by
//     shuffles, across the 8 wavefronts through LDS (over U, which is free then);
//   * the head (up to 255 logits + the value) is one 256-wide layer, 32 columns a
//     wavefront.
// Why not four wavefronts of 128 columns each: h alone would then fill the 256
// accumulator registers a lane can address, and the compiler gives every MFMA of a kernel
// the same accumulator file, so fc1's accumulators would have nowhere to go.
// Arithmetic: bf16 operands, fp32 accumulation; h is kept in fp32 between blocks (the
// layer-by-layer path rounds it to bf16), LN statistics in fp32.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/cugo_hip.h"

namespace cugo_amd {
namespace mlp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 512;                  // hidden width
constexpr int kM = 128;                  // rows per workgroup
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMT = kM / 16;             // row tiles
constexpr int kNT = kD / (16 * kWaves);  // column tiles of h per wavefront
constexpr int kK = 32;                   // K per MFMA
constexpr int kFrag = 64 * 8;            // elements of one packed B fragment
constexpr int kSteps = kD / kK;          // K steps of a 512-wide layer
constexpr int kChunk = 128;              // fc1 columns per chunk
constexpr int kChunks = kD / kChunk;
constexpr int kZGroups = kD / 8;         // 16-byte groups in a row of Z
constexpr int kHeadN = CUGO_MLP_HEAD_ROWS;  // logits + value, padded
constexpr int kHeadNT = kHeadN / (16 * kWaves);
constexpr int kMaxIn = CUGO_MLP_MAX_FEATURES;
constexpr int kMaxBlocks = CUGO_MLP_MAX_BLOCKS;
constexpr int kInSteps = kMaxIn / kK;    // K steps of the input layer (zero-padded)
constexpr int kInSlice2 = kInSteps - kSteps;  // K steps of the input's second slice
// K steps of weights in flight ahead of the MFMAs: the ring costs (depth + 1) x NT x 4
// registers.
constexpr int kDepthWide = 2;    // the 4-tile GEMMs (h's columns, the head)
constexpr int kDepthNarrow = 3;  // fc1's 2-tile chunk GEMM
// fc1's grid of wavefronts over a 128 x 128 chunk
constexpr int kGridRows = 2;
constexpr int kGridCols = kWaves / kGridRows;
constexpr int kU_MT = kMT / kGridRows;                // 4 row tiles
constexpr int kU_NT = kChunk / (16 * kGridCols);      // 2 column tiles
static_assert(kMaxIn % kK == 0 && kInSlice2 > 0 && kInSlice2 <= kSteps, "input slices");
static_assert(kHeadN % (16 * kWaves) == 0 && kChunk % (16 * 2) == 0, "whole tiles");
static_assert((kM * kD + kM * kChunk) * 2 <= 160 * 1024, "Z and U fit the LDS");
static_assert((kWaves + 1) * kM * 2 * 4 <= kM * kChunk * 2, "the LayerNorm sums fit in U");

struct Weights {
  const __bf16* w_in;  // packed, kD x kMaxIn
  const __bf16* b_in;
  const __bf16* ln_w[kMaxBlocks + 1];
  const __bf16* ln_b[kMaxBlocks + 1];
  const __bf16* w1[kMaxBlocks];  // packed, kD x kD
  const __bf16* b1[kMaxBlocks];
  const __bf16* w2[kMaxBlocks];
  const __bf16* b2[kMaxBlocks];
  const __bf16* w_head;  // packed, kHeadN x kD
  const __bf16* b_head;  // actions + 1
  int blocks, features, actions;
  float eps;
};

// Element offset of (row r, column k) in an LDS activation tile of kM rows: K step by K
// step ([k / 32][r][32]), so one MFMA A fragment (16 rows, one K step) is 1 KiB and the
// next row tile 1 KiB further; within a row's 64 bytes, 16-byte group g sits at
// g ^ ((r >> 1) & 3), so the 16 rows of a fragment read at one group cover every bank.
__device__ inline int swz(int r, int k) {
  return ((k >> 5) * kM + r) * 32 + (((((k >> 3) & 3) ^ ((r >> 1) & 3))) << 3) + (k & 7);
}

// Where the accumulator layout lands in a swz() tile: element (r0 + 16 mt + 4 q4 + i,
// c0 + 16 t + l16), r0 a multiple of 8 and c0 of 32, is at
//   base[2 (t & 1) + (i >> 1)] + (c0 / 32 + t / 2) * 32 kM + 32 r0 + 512 mt + 32 i,
// base[c] = 128 q4 + (l16 & 7) + 8 (((2 (q4 & 1)) | (l16 >> 3)) ^ c): four lane bases and
// static offsets, so a layer's stores hold four address registers.
struct StoreBases {
  int base[4];
  __device__ StoreBases(int q4, int l16) {
    const int xl = (2 * (q4 & 1)) | (l16 >> 3);
#pragma unroll
    for (int c = 0; c < 4; ++c) base[c] = 128 * q4 + (l16 & 7) + ((xl ^ c) << 3);
  }
  __device__ int at(int r0, int c0, int mt, int t, int i) const {
    return base[(2 * (t & 1)) | (i >> 1)] + (c0 / 32 + t / 2) * 32 * kM + 32 * r0 + 512 * mt +
           32 * i;
  }
};

// A GEMM's B operand: a matrix packed in fragment order with steps_total K steps a tile
// (fragment (tile, step) at (tile * steps_total + step) * kFrag, lane l's 8 values at l * 8),
// from n tile tile0 and K step kbase on.  It is read through a buffer resource: the lane's
// byte offset is one register for every load and the rest of the offset is a scalar, so
// the loads hold no 64-bit address registers.
struct BSrc {
  __amdgpu_buffer_rsrc_t rsrc;
  int b0, ts;  // bytes: the first fragment, the distance between n tiles
  __device__ BSrc(__amdgpu_buffer_rsrc_t r, int steps_total, int tile0, int kbase)
      : rsrc(r), b0((tile0 * steps_total + kbase) * kFrag * 2), ts(steps_total * kFrag * 2) {
    // Opaque where the GEMM starts: otherwise the scalar offsets of every load of the
    // unrolled chunk loop are hoisted out of the blocks loop together, and they spill.
    asm volatile("" : "+s"(b0));
  }
  __device__ bf16x8 at(int t, int s, int lane_off) const {
    return __builtin_bit_cast(
        bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane_off, b0 + t * ts + s * kFrag * 2, 0));
  }
};

// The first DEPTH K steps of a GEMM's B fragments, into its ring: issued ahead of the
// GEMM (before a barrier or an LDS phase), so their latency is not the GEMM's first wait.
template <int NT, int NSTEPS, int DEPTH>
__device__ inline void ring_fill(bf16x8 (&b)[DEPTH + 1][NT], const BSrc& src, int lane) {
#pragma unroll
  for (int j = 0; j < DEPTH; ++j)
    if (j < NSTEPS) {
#pragma unroll
      for (int t = 0; t < NT; ++t) b[j][t] = src.at(t, j, lane * 16);
    }
}

// acc[mt][t] += A[rows a_row0 + 16 mt .., K steps 0 .. NSTEPS) x B[K steps .., n tile t],
// with the ring b filled by ring_fill.  A is an LDS tile laid out by swz(); its fragments
// are one lane base plus static offsets.
template <int MT, int NT, int NSTEPS, int DEPTH, int ABUF>
__device__ inline void gemm_run(f32x4 (&acc)[MT][NT], bf16x8 (&b)[DEPTH + 1][NT],
                                const BSrc& src, const __bf16* A, int a_row0, int lane,
                                int l16, int q4) {
  constexpr int R = DEPTH + 1;
  const int lane_off = lane * 16;
  // swz(a_row0 + 16 mt + l16, 32 s + 8 q4) = a_lane + s * 32 kM + mt * 512.  K steps from 8
  // on are past a DS read's 16-bit byte offset, so they get a second base, kept opaque:
  // otherwise the compiler makes one address register per (step, row tile) and shares them
  // between GEMMs, and they spill.
  const int a_lane = (a_row0 + l16) * 32 + ((q4 ^ ((l16 >> 1) & 3)) << 3);
  int a_hi = a_lane + 8 * 32 * kM;
  asm volatile("" : "+v"(a_hi));
  auto a_at = [&](int mt, int s) {
    const int at = s < 8 ? a_lane + s * 32 * kM : a_hi + (s - 8) * 32 * kM;
    return *reinterpret_cast<const bf16x8*>(A + at + mt * 512);
  };
  // ABUF = 2: the next step's A fragments are read while this step's MFMAs issue.  ABUF = 1:
  // the same in half steps (half the row tiles' fragments at a time), for the same
  // registers as one step's fragments.
  constexpr int AH = ABUF == 2 ? MT : MT / 2;  // fragments a stage holds
  static_assert(ABUF == 2 || MT % 2 == 0, "half steps need an even row tile count");
  bf16x8 a[2][AH];
#pragma unroll
  for (int m = 0; m < AH; ++m) a[0][m] = a_at(m, 0);
  constexpr int kStages = ABUF == 2 ? 1 : 2;  // stages a step
#pragma unroll
  for (int s = 0; s < NSTEPS; ++s) {
    if (s + DEPTH < NSTEPS) {
#pragma unroll
      for (int t = 0; t < NT; ++t) b[(s + DEPTH) % R][t] = src.at(t, s + DEPTH, lane_off);
    }
#pragma unroll
    for (int h = 0; h < kStages; ++h) {
      const int stage = s * kStages + h;
      const int next = stage + 1;  // the stage whose fragments load now
      if (next < NSTEPS * kStages) {
        const int ns = next / kStages, nh = next % kStages;
#pragma unroll
        for (int m = 0; m < AH; ++m) a[next & 1][m] = a_at(nh * AH + m, ns);
      }
#pragma unroll
      for (int m = 0; m < AH; ++m)
#pragma unroll
        for (int t = 0; t < NT; ++t)
          acc[h * AH + m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              a[stage & 1][m], b[s % R][t], acc[h * AH + m][t], 0, 0, 0);
    }
    // Keep the ring: without a fence the scheduler hoists every K step's loads to the top
    // of the unrolled loop, and their registers spill.
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ring_fill + gemm_run.
template <int MT, int NT, int NSTEPS, int DEPTH, int ABUF>
__device__ inline void gemm(f32x4 (&acc)[MT][NT], const BSrc& src, const __bf16* A, int a_row0,
                            int lane, int l16, int q4) {
  bf16x8 b[DEPTH + 1][NT];
  ring_fill<NT, NSTEPS, DEPTH>(b, src, lane);
  gemm_run<MT, NT, NSTEPS, DEPTH, ABUF>(acc, b, src, A, a_row0, lane, l16, q4);
}

// acc[..][t][i] = bias[n0 + 16 t + l16] (every row).
template <int MT, int NT>
__device__ inline void set_bias(f32x4 (&acc)[MT][NT], const __bf16* bias, int n0, int l16) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float v = (float)bias[n0 + 16 * t + l16];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt][t] = f32x4{v, v, v, v};
  }
}

// Sum over the 16 lanes of a DPP row (lanes 16 k .. 16 k + 15), left in every one of them:
// xor 1 and xor 2 within quads, then the half-row and row mirrors.
template <int kCtrl>
__device__ inline float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl,
                                                            0xf, 0xf, true));
}
// v[j] = its sum over the 16 lanes of a DPP row (lanes 16 k .. 16 k + 15), left in every
// one of them: xor 1 and xor 2 within quads, then the half-row and row mirrors.
template <int N>
__device__ inline void row16_sums(float (&v)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] += dpp_mov<0xb1>(v[j]);   // quad_perm [1, 0, 3, 2]
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] += dpp_mov<0x4e>(v[j]);   // quad_perm [2, 3, 0, 1]
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] += dpp_mov<0x141>(v[j]);  // row_half_mirror
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] += dpp_mov<0x140>(v[j]);  // row_mirror
}

// Z[r][n] = bf16(LN(h)[r][n] * gamma[n] + beta[n]) for the wavefront's columns; every
// wavefront calls it.  Per-row partial sums (sum, sum of squares over a wavefront's
// columns) go to `red` (over U); after a barrier, thread r < kM turns row r's into
// (rstd, -mean * rstd) once; after a second barrier every lane reads its rows' pair and
// normalises with two FMAs a value.
__device__ inline void layer_norm(const f32x4 (&h)[kMT][kNT], const __bf16* gamma,
                                  const __bf16* beta, float eps, __bf16* Z, float* red,
                                  int wave, int l16, int q4, int tid) {
  float* stats = red + kWaves * kM * 2;  // [kM][2]
  // per (row tile, row) partial sums, half the row tiles at a time; their DPP reductions
  // run stage by stage, so consecutive DPP reads never depend on the instruction just
  // before them
  constexpr int kHalf = kMT / 2;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    float a[kHalf * 4], b[kHalf * 4];
#pragma unroll
    for (int m = 0; m < kHalf; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = 0.f, y = 0.f;
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
          const float v = h[half * kHalf + m][t][i];
          x += v;
          y = __builtin_fmaf(v, v, y);
        }
        a[m * 4 + i] = x;
        b[m * 4 + i] = y;
      }
    // the 16 lanes with the same q4 hold the same rows
    row16_sums<kHalf * 4>(a);
    row16_sums<kHalf * 4>(b);
    if (l16 == 0) {
#pragma unroll
      for (int m = 0; m < kHalf; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * (half * kHalf + m) + 4 * q4 + i;
          *reinterpret_cast<float2*>(red + (wave * kM + r) * 2) =
              make_float2(a[m * 4 + i], b[m * 4 + i]);
        }
    }
  }
  __syncthreads();
  if (tid < kM) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float2 p = *reinterpret_cast<const float2*>(red + (w * kM + tid) * 2);
      a += p.x;
      b += p.y;
    }
    const float mean = a * (1.f / kD);
    const float var = fmaxf(b * (1.f / kD) - mean * mean, 0.f);
    const float rstd = __builtin_amdgcn_rsqf(var + eps);  // hardware reciprocal square root
    *reinterpret_cast<float2*>(stats + tid * 2) = make_float2(rstd, -mean * rstd);
  }
  __syncthreads();
  const int n0 = wave * (16 * kNT);
  const StoreBases sb(q4, l16);
  float g[kNT], be[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    g[t] = (float)gamma[n0 + 16 * t + l16];
    be[t] = (float)beta[n0 + 16 * t + l16];
  }
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 st = *reinterpret_cast<const float2*>(stats + (16 * mt + 4 * q4 + i) * 2);
#pragma unroll
      for (int t = 0; t < kNT; ++t)
        Z[sb.at(0, n0, mt, t, i)] = (__bf16)__builtin_fmaf(
            __builtin_fmaf(h[mt][t][i], st.x, st.y), g[t], be[t]);
    }
}

template <class TIn>
struct Input;
template <>
struct Input<float> {
  // eight elements as bf16 (round to nearest even, as torch's conversion)
  __device__ static uint4 load8(const float* p) {
    const float4 v0 = *reinterpret_cast<const float4*>(p);
    const float4 v1 = *reinterpret_cast<const float4*>(p + 4);
    auto two = [](float lo, float hi) {
      return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
    };
    return make_uint4(two(v0.x, v0.y), two(v0.z, v0.w), two(v1.x, v1.y), two(v1.z, v1.w));
  }
};
template <>
struct Input<__bf16> {
  __device__ static uint4 load8(const __bf16* p) { return *reinterpret_cast<const uint4*>(p); }
};

// Columns [c0, c0 + 8 GROUPS) of the tile's rows of x -> Z's groups 0 .. GROUPS (bf16;
// zero past the features and past the last row), and their bf16 copy to x_copy.  Loads at
// clamped indices are issued eight at a time before any is used.
template <class TIn, int GROUPS>
__device__ inline void load_input(const TIn* __restrict__ x, __bf16* __restrict__ x_copy,
                                  int64_t n, int F, int64_t row0, int c0, __bf16* Z, int tid) {
  constexpr int kTotal = kM * GROUPS;
  static_assert(kTotal % (kThreads * 8) == 0, "whole batches");
#pragma unroll 1
  for (int j0 = 0; j0 < kTotal; j0 += kThreads * 8) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u * kThreads + tid;
      const int r = j / GROUPS;
      const int col = c0 + 8 * (j - r * GROUPS);
      const int64_t g = row0 + r < n ? row0 + r : n - 1;
      v[u] = Input<TIn>::load8(x + g * F + (col < F ? col : F - 8));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u * kThreads + tid;
      const int r = j / GROUPS;
      const int col = c0 + 8 * (j - r * GROUPS);
      const bool valid = row0 + r < n && col < F;
      const uint4 val = valid ? v[u] : make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4*>(Z + swz(r, col - c0)) = val;
      if (x_copy != nullptr && valid)
        *reinterpret_cast<uint4*>(x_copy + (row0 + r) * F + col) = val;
    }
  }
}

template <class TIn>
__global__ __launch_bounds__(kThreads) void actor_kernel(const TIn* __restrict__ x,
                                                            __bf16* __restrict__ x_copy,
                                                            int64_t n, Weights w,
                                                            __bf16* __restrict__ logits,
                                                            float* __restrict__ value) {
  __shared__ __attribute__((aligned(16))) __bf16 smem[kM * kD + kM * kChunk];
  __bf16* Z = smem;
  __bf16* U = smem + kM * kD;
  float* red = reinterpret_cast<float*>(U);  // LayerNorm sums, while U is free

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * kM;
  const int F = w.features;
  const int n0 = wave * (16 * kNT);  // this wavefront's first column of h
  const int tile0 = n0 / 16;
  // fc1's grid: rows [64 wr, 64 wr + 64), chunk columns [32 wc, 32 wc + 32)
  const int wr = wave / kGridCols, wc = wave % kGridCols;
  const StoreBases sb(q4, l16);

  auto rsrc = [](const __bf16* p, int rows, int cols) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(p), (short)0, rows * cols * 2,
                                             0x00020000);
  };

  // ---- input layer, x in two column slices through Z
  f32x4 h[kMT][kNT];
  set_bias<kMT, kNT>(h, w.b_in, n0, l16);
  const auto w_in = rsrc(w.w_in, kD, kMaxIn);
  load_input<TIn, kZGroups>(x, x_copy, n, F, row0, 0, Z, tid);
  __syncthreads();
  gemm<kMT, kNT, kSteps, kDepthWide, 1>(h, BSrc(w_in, kInSteps, tile0, 0), Z, 0, lane, l16, q4);
  __syncthreads();  // Z read
  load_input<TIn, kInSlice2 * kK / 8>(x, x_copy, n, F, row0, kD, Z, tid);
  __syncthreads();
  gemm<kMT, kNT, kInSlice2, kDepthWide, 1>(h, BSrc(w_in, kInSteps, tile0, kSteps), Z, 0, lane,
                                           l16, q4);

  const int ucol = 16 * kU_NT * wc;  // this wavefront's columns within a chunk
  const int urow = 16 * kU_MT * wr;
  for (int b = 0; b < w.blocks; ++b) {
    const auto w1 = rsrc(w.w1[b], kD, kD);
    const auto w2 = rsrc(w.w2[b], kD, kD);
    // z = LN(h) -> Z.  The barriers inside come after every wavefront's last read of the
    // previous layer's input (Z) and of U, so both can be overwritten after them.
    layer_norm(h, w.ln_w[b], w.ln_b[b], w.eps, Z, red, wave, l16, q4, tid);
    __syncthreads();  // Z complete
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      f32x4 u[kU_MT][kU_NT];
      set_bias<kU_MT, kU_NT>(u, w.b1[b], kChunk * c + ucol, l16);
      gemm<kU_MT, kU_NT, kSteps, kDepthNarrow, 2>(u, BSrc(w1, kSteps, (kChunk * c + ucol) / 16, 0),
                                                   Z, urow, lane, l16, q4);
#pragma unroll
      for (int mt = 0; mt < kU_MT; ++mt)
#pragma unroll
        for (int t = 0; t < kU_NT; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            U[sb.at(urow, ucol, mt, t, i)] = (__bf16)fmaxf(u[mt][t][i], 0.f);
      __syncthreads();  // U complete
      gemm<kMT, kNT, kChunk / kK, kDepthWide, 1>(h, BSrc(w2, kSteps, tile0, c * (kChunk / kK)), U,
                                                 0, lane, l16, q4);
      __syncthreads();  // U read
    }
    const __bf16* b2 = w.b2[b];
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const float v = (float)b2[n0 + 16 * t + l16];
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) h[mt][t] += f32x4{v, v, v, v};
    }
  }

  // ---- head: columns [0, A) logits, A the value, the rest padding (zero weights)
  const int A = w.actions;
  const int hn0 = wave * (16 * kHeadNT);
  layer_norm(h, w.ln_w[w.blocks], w.ln_b[w.blocks], w.eps, Z, red, wave, l16, q4, tid);
  __syncthreads();  // Z complete
  f32x4 o[kMT][kHeadNT];
#pragma unroll
  for (int t = 0; t < kHeadNT; ++t) {
    const int col = hn0 + 16 * t + l16;
    const float v = col <= A ? (float)w.b_head[col] : 0.f;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) o[mt][t] = f32x4{v, v, v, v};
  }
  gemm<kMT, kHeadNT, kSteps, kDepthNarrow, 1>(o, BSrc(rsrc(w.w_head, kHeadN, kD), kSteps, hn0 / 16, 0),
                                              Z, 0, lane, l16, q4);
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = row0 + 16 * mt + 4 * q4 + i;
      if (r >= n) continue;
#pragma unroll
      for (int t = 0; t < kHeadNT; ++t) {
        const int col = hn0 + 16 * t + l16;
        if (col < A)
          logits[r * A + col] = (__bf16)o[mt][t][i];
        else if (col == A)
          value[r] = o[mt][t][i];
      }
    }
}

// packed[((tile * steps + step) * 64 + (q * 16 + r)) * 8 + i] = w[16 tile + r][32 step +
// 8 q + i], zero outside [rows, cols): one thread per packed element.
__global__ void pack_kernel(const __bf16* __restrict__ w, int64_t rows, int64_t cols,
                            int64_t rows_pad, int64_t cols_pad, __bf16* __restrict__ packed) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = rows_pad * cols_pad;
  if (j >= total) return;
  const int64_t steps = cols_pad / kK;
  const int i = (int)(j & 7);
  const int l = (int)((j >> 3) & 63);
  const int64_t frag = j >> 9;
  const int64_t step = frag % steps;
  const int64_t tile = frag / steps;
  const int64_t rr = tile * 16 + (l & 15);
  const int64_t cc = step * kK + 8 * (l >> 4) + i;
  packed[j] = (rr < rows && cc < cols) ? w[rr * cols + cc] : (__bf16)0.f;
}

}  // namespace mlp
}  // namespace cugo_amd

extern "C" int cugo_mlp_pack_weight(const void* w, int64_t rows, int64_t cols,
                                    int64_t rows_pad, int64_t cols_pad, void* packed,
                                    hipStream_t stream) {
  using namespace cugo_amd::mlp;
  if (rows < 0 || cols < 0 || rows > rows_pad || cols > cols_pad || rows_pad % 16 != 0 ||
      cols_pad % kK != 0)
    return -1;
  const int64_t total = rows_pad * cols_pad;
  if (total == 0) return 0;
  if (packed == nullptr || (w == nullptr && rows * cols > 0)) return -1;
  const unsigned blocks = (unsigned)((total + 255) / 256);
  hipLaunchKernelGGL(pack_kernel, dim3(blocks), dim3(256), 0, stream,
                     static_cast<const __bf16*>(w), rows, cols, rows_pad, cols_pad,
                     static_cast<__bf16*>(packed));
  return (int)hipGetLastError();
}

extern "C" int cugo_mlp_actor_forward(int x_dtype, const void* x, void* x_copy, int64_t n,
                                      const CugoMlpWeights* weights, void* logits,
                                      float* value, hipStream_t stream) {
  using namespace cugo_amd::mlp;
  if (weights == nullptr || n < 0) return -1;
  const CugoMlpWeights& src = *weights;
  if (src.hidden != kD || src.blocks < 0 || src.blocks > kMaxBlocks || src.features <= 0 ||
      src.features > kMaxIn || src.features % 8 != 0 || src.actions <= 0 ||
      src.actions + 1 > kHeadN)
    return -3;
  if (n == 0) return 0;
  if (x == nullptr || logits == nullptr || value == nullptr) return -1;
  Weights w{};
  w.w_in = static_cast<const __bf16*>(src.w_in);
  w.b_in = static_cast<const __bf16*>(src.b_in);
  for (int b = 0; b <= src.blocks; ++b) {
    w.ln_w[b] = static_cast<const __bf16*>(src.ln_w[b]);
    w.ln_b[b] = static_cast<const __bf16*>(src.ln_b[b]);
  }
  for (int b = 0; b < src.blocks; ++b) {
    w.w1[b] = static_cast<const __bf16*>(src.w1[b]);
    w.b1[b] = static_cast<const __bf16*>(src.b1[b]);
    w.w2[b] = static_cast<const __bf16*>(src.w2[b]);
    w.b2[b] = static_cast<const __bf16*>(src.b2[b]);
  }
  w.w_head = static_cast<const __bf16*>(src.w_head);
  w.b_head = static_cast<const __bf16*>(src.b_head);
  w.blocks = src.blocks;
  w.features = src.features;
  w.actions = src.actions;
  w.eps = src.eps;
  const unsigned grid = (unsigned)((n + kM - 1) / kM);
  auto* xc = static_cast<__bf16*>(x_copy);
  auto* lg = static_cast<__bf16*>(logits);
  switch (x_dtype) {
    case CUGO_DTYPE_F32:
      hipLaunchKernelGGL(actor_kernel<float>, dim3(grid), dim3(kThreads), 0, stream,
                         static_cast<const float*>(x), xc, n, w, lg, value);
      break;
    case CUGO_DTYPE_BF16:
      hipLaunchKernelGGL(actor_kernel<__bf16>, dim3(grid), dim3(kThreads), 0, stream,
                         static_cast<const __bf16*>(x), xc, n, w, lg, value);
      break;
    default:
      return -2;
  }
  return (int)hipGetLastError();
}
