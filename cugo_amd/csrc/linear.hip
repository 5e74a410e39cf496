// bf16 linear layers on MFMA for gfx950: Y = act(X W^T + b), optionally with GELU.
//
// The sequence policy's decoder step (cugo_amd/seq_decode.py, the reference's
// SeqNet.cached_step, python/cugo_seq50.py:291-322) runs its nn.Linear layers over one
// token a row: 4,096 query rows and 8,192 event rows a self-play step, K = 256 (1,024 for
// linear2), N = 256-1,024.  At these sizes a library GEMM reaches a fraction of HBM
// bandwidth on its operand bytes, and the feed-forward's GELU is one more pass over the
// widest activation (N = 1,024).  This kernel is sized for them.
//
// What bounds it is the vector memory path of a CU, not the MFMA pipe: a load instruction
// costs the texture addresser a cycle for every cache line each 16-lane quarter of the
// wavefront touches.  An MFMA operand fragment read straight from a row-major matrix puts
// 16 rows (16 lines, 16 bytes of each) in every quarter-wave: 16 bytes a cycle.  So:
//   * W is packed once in fragment order (cugo_mlp_pack_weight: 64 lanes x 16 bytes of one
//     fragment are 1 KiB of contiguous memory), and each wavefront loads its fragments
//     straight into a register ring D K steps ahead of the MFMAs;
//   * the workgroup's X panel (BM rows x all of K, at most 128 KiB) is copied into LDS
//     once with row-contiguous loads (a quarter-wave reads 256 contiguous bytes), in
//     K-step-major order with the 16-byte groups of a row XOR-swizzled, so one fragment
//     (16 rows x 64 bytes) is a conflict-free 1 KiB read; one barrier, then the
//     wavefronts read their X fragments from LDS;
//   * a workgroup is a WR x WC grid of wavefronts, each owning 16 TM rows x 16 TN columns
//     of the tile (BM = 16 TM WR, BN = 16 TN WC): wavefronts of one grid column load the
//     same W fragments, the second from L1;
//   * v_mfma_f32_16x16x32_bf16 with W as the A operand and X as the B operand, i.e. the
//     product is formed transposed: lane l then holds Y[16 mt + l % 16][16 nt + 4 (l / 16)
//     + 0..3], four adjacent columns;
//   * the epilogue adds the bias, rounds to bf16 (what the library layer stores), and for
//     GELU evaluates x / 2 (1 + erf(x / sqrt 2)) in fp32 on that bf16 value and rounds
//     again, the two steps nn.Linear + nn.GELU() take in bf16; the tile then goes through
//     the LDS (over the dead X panel) so that it leaves in 16-byte row pieces, whole lines
//     a quarter-wave (stored from the accumulator layout, a quarter-wave would write 8
//     bytes into each of 16 rows).
// Workgroup ids are remapped so that consecutive tiles run on one XCD (the dispatcher
// deals workgroups to the 8 XCDs in turn), keeping a row panel's reads in one L2.
//
// Arithmetic: bf16 operands, fp32 accumulation in K order; partial rows and columns are
// clamped on load and masked on store.
#include <hip/hip_runtime.h>

#include <atomic>

#include <stdint.h>

#include "../../include/cugo_hip.h"

namespace cugo_amd {
namespace linear {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kK = 32;  // K per MFMA
constexpr int kFragBytes = 64 * 16;

struct Args {
  const __bf16* x;
  const __bf16* w;     // packed: fragment (tile, step) at (tile * KS + step) * 1 KiB
  const __bf16* bias;  // [n] or NULL
  __bf16* y;           // with kAddNorm: x_out = res + (x W^T + b)
  int m, n, ldx, ldy;
  int col_blocks;  // workgroups along n
  int wtiles;      // 16-row tiles of the packed W
  // the residual (row stride ldr, 0: one row for all), added to the output after its
  // rounding (NULL: none); kAddNorm's too, its rows of n = BN elements
  const __bf16* res;
  int ldr;
  const __bf16* ln_w;
  const __bf16* ln_b;
  __bf16* ln;
  float eps;
};

// Epilogues beyond CUGO_LINEAR_NONE / CUGO_LINEAR_GELU: the residual add and the
// LayerNorm after it (a pre-norm layer's out_proj or linear2 followed by the next norm).
constexpr int kAddNorm = 2;

// Eight bf16 sums, each rounded from fp32 as torch adds bf16 tensors.
__device__ inline uint4 add_bf16(uint4 a, uint4 b) {
  const bf16x8 x = __builtin_bit_cast(bf16x8, a), y = __builtin_bit_cast(bf16x8, b);
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (__bf16)((float)x[i] + (float)y[i]);
  return __builtin_bit_cast(uint4, z);
}

__device__ inline float gelu(float v) {
  return v * 0.5f * (1.0f + erff(v * 0.70710678118654752440f));
}

// Element offset of (row r, column k) in the LDS X panel of BM rows: K step major
// ([k / 32][r][32]), the 16-byte group g of a row's 64 bytes at g ^ ((r >> 1) & 3).
template <int BM>
__device__ inline int xs_at(int r, int k) {
  return ((k >> 5) * BM + r) * 32 + ((((k >> 3) & 3) ^ ((r >> 1) & 3)) << 3) + (k & 7);
}

template <int TM, int TN, int WR, int WC, int D, int KS, int ACT>
__global__ __launch_bounds__(64 * WR * WC) void linear_kernel(Args a) {
  constexpr int kT = 64 * WR * WC;         // threads
  constexpr int BM = 16 * TM * WR;         // rows of the workgroup's tile
  constexpr int BN = 16 * TN * WC;         // columns
  constexpr int R = D + 1;                 // ring slots
  constexpr int kGroups = BM * KS * 4;     // 16-byte groups of the X panel
  constexpr int kBatch = 8;                // loads in flight a thread while staging
  constexpr int kOutStride = BN + 16;      // elements a row of the staged output tile
  constexpr int kXsElems = BM * KS * kK;
  constexpr int kLds = kXsElems > BM * kOutStride ? kXsElems : BM * kOutStride;
  static_assert(kLds * 2 <= 160 * 1024, "the tile fits the LDS");
  __shared__ __attribute__((aligned(16))) __bf16 xs[kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave / WC, wc = wave % WC;
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  const int rb = bid / a.col_blocks;
  const int m0 = rb * BM;
  const int nb0 = (bid - rb * a.col_blocks) * BN;  // the workgroup's first column
  const int n0 = nb0 + wc * 16 * TN;               // this wavefront's
  const int r0 = wr * 16 * TM;                     // this wavefront's first row in the tile
  const int l16 = lane & 15, q4 = lane >> 4;

  // W's first D K steps, issued before the X panel's copy so both are in flight.
  const auto wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(a.w), (short)0,
                                                     a.wtiles * KS * kFragBytes, 0x00020000);
  int wt[TN];  // byte offset of fragment (tile, 0); tiles past the end read the last one
#pragma unroll
  for (int t = 0; t < TN; ++t) wt[t] = min(n0 / 16 + t, a.wtiles - 1) * KS * kFragBytes;
  bf16x8 wb[R][TN];
  auto load_w = [&](int s, int slot) {
#pragma unroll
    for (int t = 0; t < TN; ++t)
      wb[slot][t] = __builtin_bit_cast(
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(wrs, lane * 16, wt[t] + s * kFragBytes, 0));
  };
#pragma unroll
  for (int j = 0; j < D; ++j)
    if (j < KS) load_w(j, j);

  // kAddNorm: the residual rows this wavefront normalises (row wave + WR WC j of the
  // tile), loaded now so their latency hides behind the GEMM.
  constexpr int kNormRows = ACT == kAddNorm ? BM / (WR * WC) : 1;
  bf16x4 res_v[kNormRows];
  if constexpr (ACT == kAddNorm) {
#pragma unroll
    for (int j = 0; j < kNormRows; ++j) {
      const int row = min(m0 + wave + WR * WC * j, a.m - 1);
      res_v[j] = *reinterpret_cast<const bf16x4*>(a.res + (int64_t)row * a.ldr + lane * 4);
    }
  }

  // The X panel: thread tid copies 16-byte groups tid, tid + kT, ... (row-major order,
  // so a quarter-wave reads 256 contiguous bytes of one row).
  const auto xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__bf16*>(a.x), (short)0, ((a.m - 1) * a.ldx + KS * kK) * 2, 0x00020000);
#pragma unroll
  for (int b0 = 0; b0 < kGroups; b0 += kT * kBatch) {
    uint4 v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int gi = b0 + j * kT + tid;
      if (gi < kGroups) {
        const int r = gi / (KS * 4), c = gi % (KS * 4);
        const int row = min(m0 + r, a.m - 1);
        v[j] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (row * a.ldx + 8 * c) * 2, 0, 0));
      }
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int gi = b0 + j * kT + tid;
      if (gi < kGroups) {
        const int r = gi / (KS * 4), c = gi % (KS * 4);
        *reinterpret_cast<uint4*>(xs + xs_at<BM>(r, 8 * c)) = v[j];
      }
    }
  }
  __syncthreads();

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The K loop is unrolled whole (KS is a template argument): with a run-time trip count
  // the compiler cannot count the loads in flight across the loop's branches and waits
  // for all of them before every step's MFMAs.
  // X fragments are double-buffered: step s + 1's are read from LDS before step s's MFMAs
  // issue, so the MFMAs do not wait on the LDS every step.
  const int x_lane = xs_at<BM>(r0 + l16, 8 * q4);
  auto load_x = [&](bf16x8 (&xa)[TM], int s) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      xa[i] = *reinterpret_cast<const bf16x8*>(xs + x_lane + (s * BM + 16 * i) * 32);
  };
  bf16x8 xa[2][TM];
  load_x(xa[0], 0);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (s + D < KS) load_w(s + D, (s + D) % R);
    if (s + 1 < KS) load_x(xa[(s + 1) & 1], s + 1);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int t = 0; t < TN; ++t)
        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb[s % R][t], xa[s & 1][i],
                                                            acc[i][t], 0, 0, 0);
    // Keep the ring: without a fence the scheduler hoists later K steps' loads.
    __builtin_amdgcn_sched_barrier(0);
  }

  // Epilogue: bias, bf16, GELU, into the LDS as a row-major BM x BN tile (the X panel is
  // dead once every wavefront is past the barrier), then out in 16-byte row pieces: a
  // quarter-wave writes whole lines instead of 16 rows' 8 bytes each.
  float bias[TN][4];
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int col = n0 + 16 * t + 4 * q4;
#pragma unroll
    for (int c = 0; c < 4; ++c) bias[t][c] = 0.f;
    if (a.bias != nullptr && col + 4 <= a.n) {
      const bf16x4 bv = *reinterpret_cast<const bf16x4*>(a.bias + col);
#pragma unroll
      for (int c = 0; c < 4; ++c) bias[t][c] = (float)bv[c];
    } else if (a.bias != nullptr) {  // the last columns of an n that is not a multiple of 4
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (col + c < a.n) bias[t][c] = (float)a.bias[col + c];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      bf16x4 out;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const __bf16 v = (__bf16)(acc[i][t][c] + bias[t][c]);
        out[c] = ACT == CUGO_LINEAR_GELU ? (__bf16)gelu((float)v) : v;
      }
      const int r = r0 + 16 * i + l16, c = wc * 16 * TN + 16 * t + 4 * q4;
      *reinterpret_cast<bf16x4*>(xs + r * kOutStride + c) = out;
    }
  __syncthreads();
  if constexpr (ACT == kAddNorm) {
    // One wavefront a row, 4 elements a lane, in the order and arithmetic of
    // add_layernorm_kernel (selfplay.hip): x_out = bf16(res + y); two-pass fp32 mean and
    // variance by lane sums and xor shuffles; ln = bf16((v - mean) rstd w + b).
    static_assert(BN == 256, "a workgroup holds whole 256-wide rows");
    constexpr int KE = BN / 64;
    static_assert(BM % (WR * WC) == 0, "whole rows a wavefront");
    const bf16x4 wv4 = *reinterpret_cast<const bf16x4*>(a.ln_w + lane * KE);
    const bf16x4 bv4 = *reinterpret_cast<const bf16x4*>(a.ln_b + lane * KE);
#pragma unroll
    for (int j = 0; j < kNormRows; ++j) {
      const int r = wave + WR * WC * j;
      const int row = m0 + r;
      if (row >= a.m) break;
      const bf16x4 yv = *reinterpret_cast<const bf16x4*>(xs + r * kOutStride + lane * KE);
      const int64_t at = (int64_t)row * a.ldy + lane * KE;
      const bf16x4 xv = res_v[j];
      float v[KE];
      bf16x4 xo;
#pragma unroll
      for (int k = 0; k < KE; ++k) {
        xo[k] = (__bf16)((float)xv[k] + (float)yv[k]);
        v[k] = (float)xo[k];
      }
      *reinterpret_cast<bf16x4*>(a.y + at) = xo;
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < KE; ++k) sum += v[k];
      for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
      const float mean = sum / (float)BN;
      float sq = 0.0f;
#pragma unroll
      for (int k = 0; k < KE; ++k) {
        const float c = v[k] - mean;
        sq += c * c;
      }
      for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
      const float rstd = 1.0f / sqrtf(sq / (float)BN + a.eps);
      bf16x4 o;
#pragma unroll
      for (int k = 0; k < KE; ++k)
        o[k] = (__bf16)((v[k] - mean) * rstd * (float)wv4[k] + (float)bv4[k]);
      *reinterpret_cast<bf16x4*>(a.ln + at) = o;
    }
    return;
  }
  constexpr int kPieces = BM * BN / 8;  // 16-byte pieces of the tile
  const bool wide = (a.ldy & 7) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 &&
                    (a.res == nullptr ||
                     ((a.ldr & 7) == 0 && (reinterpret_cast<uintptr_t>(a.res) & 15) == 0));
  // n or ldy not a multiple of 4 (e.g. 179 logits a row): element stores, no residual
  const bool narrow = ((a.n | a.ldy) & 3) != 0;
#pragma unroll
  for (int p0 = 0; p0 < kPieces; p0 += kT) {
    const int p = p0 + tid;
    if (p < kPieces) {
      const int r = p / (BN / 8), c = (p % (BN / 8)) * 8;
      const int row = m0 + r, col = nb0 + c;
      if (row < a.m && col < a.n) {
        uint4 v = *reinterpret_cast<const uint4*>(xs + r * kOutStride + c);
        __bf16* dst = a.y + (int64_t)row * a.ldy + col;
        const __bf16* rsrc = a.res + (int64_t)row * a.ldr + col;
        if (wide && col + 8 <= a.n) {
          if (a.res != nullptr) v = add_bf16(v, *reinterpret_cast<const uint4*>(rsrc));
          *reinterpret_cast<uint4*>(dst) = v;
        } else if (narrow) {
          const bf16x8 e8 = __builtin_bit_cast(bf16x8, v);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (col + e < a.n) dst[e] = e8[e];
        } else {
          if (a.res != nullptr) {
            const uint2 lo = *reinterpret_cast<const uint2*>(rsrc);
            const uint2 hi = col + 8 <= a.n ? *reinterpret_cast<const uint2*>(rsrc + 4)
                                            : uint2{0u, 0u};
            v = add_bf16(v, uint4{lo.x, lo.y, hi.x, hi.y});
          }
          *reinterpret_cast<uint2*>(dst) = uint2{v.x, v.y};
          if (col + 8 <= a.n) *reinterpret_cast<uint2*>(dst + 4) = uint2{v.z, v.w};
        }
      }
    }
  }
}

template <int TM, int TN, int WR, int WC, int D, int KS>
int launch_ks(const Args& a, int act, hipStream_t stream) {
  constexpr int BM = 16 * TM * WR;
  if constexpr (BM * KS * kK * 2 > 160 * 1024) {
    return -7;  // the X panel does not fit the LDS at this depth
  } else if constexpr (16 * TN * WC != 256) {
    if (act == kAddNorm) return -3;
    const unsigned grid = (unsigned)(((a.m + BM - 1) / BM) * a.col_blocks);
    if (act == CUGO_LINEAR_GELU)
      linear_kernel<TM, TN, WR, WC, D, KS, CUGO_LINEAR_GELU>
          <<<grid, 64 * WR * WC, 0, stream>>>(a);
    else
      linear_kernel<TM, TN, WR, WC, D, KS, CUGO_LINEAR_NONE>
          <<<grid, 64 * WR * WC, 0, stream>>>(a);
    return (int)hipGetLastError();
  } else {
    const unsigned grid = (unsigned)(((a.m + BM - 1) / BM) * a.col_blocks);
    if (act == CUGO_LINEAR_GELU)
      linear_kernel<TM, TN, WR, WC, D, KS, CUGO_LINEAR_GELU>
          <<<grid, 64 * WR * WC, 0, stream>>>(a);
    else if (act == kAddNorm)
      linear_kernel<TM, TN, WR, WC, D, KS, kAddNorm><<<grid, 64 * WR * WC, 0, stream>>>(a);
    else
      linear_kernel<TM, TN, WR, WC, D, KS, CUGO_LINEAR_NONE>
          <<<grid, 64 * WR * WC, 0, stream>>>(a);
    return (int)hipGetLastError();
  }
}

template <int TM, int TN, int WR, int WC, int D>
int launch(const Args& base, int k, int act, hipStream_t stream) {
  Args a = base;
  a.col_blocks = (a.n + 16 * TN * WC - 1) / (16 * TN * WC);
  switch (k / kK) {
    case 2: return launch_ks<TM, TN, WR, WC, D, 2>(a, act, stream);
    case 4: return launch_ks<TM, TN, WR, WC, D, 4>(a, act, stream);
    case 8: return launch_ks<TM, TN, WR, WC, D, 8>(a, act, stream);
    case 16: return launch_ks<TM, TN, WR, WC, D, 16>(a, act, stream);
    case 32: return launch_ks<TM, TN, WR, WC, D, 32>(a, act, stream);
    default: return -3;
  }
}

// ---------------------------------------------------------------- feed-forward ----
// The feed-forward half of a pre-norm encoder layer in one launch (cugo_seq50.py:319-322:
// x + linear2(GELU(linear1(h))), h = norm2(x), then the next layer's norm1 or the final
// norm), for d = 256 and a 1,024-wide hidden layer.  The two-launch form writes the
// [m, 1,024] GELU output to HBM and reads it back; here a workgroup owns 16 MT rows for
// the whole block and the hidden layer never leaves the CU:
//   * h's rows (256 columns) are copied into LDS once (the X panel layout of
//     linear_kernel); the hidden layer runs in four 256-column chunks: each of the 8
//     wavefronts computes 32 columns of the chunk for all rows (linear1, W1 as the MFMA A
//     operand, K = 256), adds the bias, rounds, applies GELU and rounds again, and writes
//     them to a chunk buffer in LDS (two buffers, so one barrier a chunk); then each
//     wavefront adds the chunk's K slice of linear2 into its 32 output columns for all
//     rows (accumulators in registers across the chunks, K order 0 .. 1,023 as the
//     one-launch linear2 runs it); a chunk's GELU runs a 4-column group a K step beside
//     the MFMAs of the next chunk's linear1 (the last chunk's beside the third linear2
//     slice), which took 12,288 rows from 26.6 to 24.9 us;
//   * the epilogue is linear_kernel's: bias, bf16, the residual add, the LayerNorm (or
//     the plain residual), through LDS row-major;
//   * with kOut (cugo_out_proj_ffn) the layer's out_proj runs first, on the attention
//     output's rows in the panel, with linear_kernel's kAddNorm epilogue (x1 = x +
//     out_proj, kept in registers as the feed-forward's residual; h = norm2(x1) written
//     over the panel), so neither x1 nor h leaves the CU.
// Every rounding and every fp32 sum is in the order of linear (GELU) + linear_add_layernorm
// (or linear with the residual), and with kOut of linear_add_layernorm before them, so the
// outputs are the same bits.
// What bounds it: each workgroup streams all 1 MiB of W1 and W2 (and W_o's 128 KiB)
// through its CU's L1 (the FLOPs a weight byte buys are the tile's rows), ~20 bytes a
// cycle a CU when every CU reads the same weights at once; the GELU's erff is ~5 us of
// VALU at 12,288 rows (the launch without it: 20.5 against 26.1 us).  A GELU table in LDS
// (gelu() of the 4,736 bf16 inputs without a closed form, built by each workgroup, then
// looked up; the same bits on every finite input) made the launch slower: 39.6 against
// 31.9 us at 12,288 rows.
// Weights: linear_kernel's packed fragments, W1 [1,024, 256] (8 K steps a 16-row tile)
// and W2 [256, 1,024] (32 K steps a tile), read through buffer loads a few K steps ahead
// of the MFMAs.
namespace ffn {

constexpr int kD = 256;       // model width
constexpr int kF = 1024;      // hidden width
constexpr int kC = 256;       // hidden columns a chunk
constexpr int kChunks = kF / kC;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kS1 = kD / kK;  // K steps of linear1 (8)
constexpr int kSc = kC / kK;  // K steps of linear2 a chunk (8)
constexpr int kS2 = kF / kK;  // K steps of linear2 (32)
// The phases of ffn_kernel's loop: which weight (linear2's: true), which chunk, which
// chunk's GELU runs beside it (-1: none), and whether a barrier follows it.
constexpr int kPhases = 2 * kChunks;
__host__ __device__ constexpr bool phase_w2(int p) { return p == 2 || p == 4 || p >= 6; }
__host__ __device__ constexpr int phase_chunk(int p) {
  return p == 0 ? 0 : p == 1 ? 1 : p == 2 ? 0 : p == 3 ? 2 : p == 4 ? 1 : p == 5 ? 3 : p == 6 ? 2 : 3;
}
__host__ __device__ constexpr int phase_gelu(int p) {
  return p == 1 ? 0 : p == 3 ? 1 : p == 5 ? 2 : p == 6 ? 3 : -1;
}
__host__ __device__ constexpr bool phase_barrier(int p) {
  return p == 1 || p == 3 || p == 5 || p == 6;
}
static_assert(kChunks == 4 && kS1 == kSc, "the phase table is written for four chunks");

struct Args {
  const __bf16* h;  // [m, 256], row stride ldh (with wo: the attention output)
  const __bf16* x;  // residual [m, 256], contiguous
  // With wo (kOut): h is computed here, x1 = x + bf16(h_in W_o^T + b_o), h = LN2(x1), and
  // x1 is the feed-forward's residual (out_proj + add + norm2, linear_add_layernorm).
  const __bf16* wo;
  const __bf16* bo;
  const __bf16* ln2_w;
  const __bf16* ln2_b;
  float eps2;
  const __bf16* w1;
  const __bf16* b1;
  const __bf16* w2;
  const __bf16* b2;
  const __bf16* ln_w;  // NULL: x_out = x + y only
  const __bf16* ln_b;
  float eps;
  __bf16* x_out;  // [m, 256] contiguous (may alias x)
  __bf16* ln;     // [m, 256] contiguous, with ln_w
  int m, ldh;
};

template <int MT, int kDepth, bool kOut>
__global__ __launch_bounds__(kThreads) void ffn_kernel(Args a) {
  constexpr int kR = kDepth + 1;  // ring slots: K steps of weights in flight ahead of MFMAs
  constexpr int BM = 16 * MT;
  constexpr int kPanel = BM * kD;            // elements of h's panel, and of a chunk buffer
  constexpr int kOutStride = kD + 16;        // elements a row of the staged output
  static_assert(BM * kOutStride <= 2 * kPanel, "the staged output fits two panels");
  static_assert(3 * kPanel * 2 <= 160 * 1024, "the panel and two chunks fit the LDS");
  __shared__ __attribute__((aligned(16))) __bf16 smem[3 * kPanel];
  __bf16* hs = smem;               // h's rows (xs_at layout, BM rows, K = 256)
  __bf16* us = smem + kPanel;      // chunk buffers 0 and 1 (xs_at layout, K = 256)
  __bf16* staged = smem;           // the output tile, after the last chunk (hs + us[0])

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, q4 = lane >> 4;
  const int m0 = blockIdx.x * BM;
  const int c0 = wave * 32;  // this wavefront's columns: of each chunk, and of the output

  const auto w1r = __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(a.w1), (short)0,
                                                     (kF / 16) * kS1 * kFragBytes, 0x00020000);
  const auto w2r = __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(a.w2), (short)0,
                                                     (kD / 16) * kS2 * kFragBytes, 0x00020000);
  // W1 fragment (chunk c, tile t, step s): hidden columns 256 c + 32 wave + 16 t;
  // W2 fragment (tile t, step s): output columns 32 wave + 16 t, K step s of 32.
  auto w1_at = [&](int c, int t, int s) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
        w1r, lane * 16, ((16 * c + 2 * wave + t) * kS1 + s) * kFragBytes, 0));
  };
  auto w2_at = [&](int t, int s) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
        w2r, lane * 16, ((2 * wave + t) * kS2 + s) * kFragBytes, 0));
  };
  // W_o fragment (tile t, step s): out_proj's output columns 32 wave + 16 t
  const auto wor = __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(a.wo), (short)0,
                                                     kOut ? (kD / 16) * kS1 * kFragBytes : 0,
                                                     0x00020000);
  auto wo_at = [&](int t, int s) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
        wor, lane * 16, ((2 * wave + t) * kS1 + s) * kFragBytes, 0));
  };
  constexpr int kPre = kOut ? kS1 : 0;  // ring steps of out_proj, before the phases

  // One ring for the weights, in the order they are used (out_proj's 8 K steps first
  // with kOut, then the phases below, 8 K steps each): step g of that sequence sits in
  // slot g % kR.
  bf16x8 ring[kR][2];
  auto w_at = [&](int g, int t) {
    if (kOut && g < kPre) return wo_at(t, g);
    const int p = (g - kPre) / kS1, s = (g - kPre) % kS1, c = phase_chunk(p);
    return phase_w2(p) ? w2_at(t, kSc * c + s) : w1_at(c, t, s);
  };
#pragma unroll
  for (int j = 0; j < kDepth; ++j)
#pragma unroll
    for (int t = 0; t < 2; ++t) ring[j][t] = w_at(j, t);

  constexpr int kNormRows = BM / kWaves;  // rows a wavefront finishes in the epilogue
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  // the residual rows this wavefront finishes (row wave + 8 j, columns 4 lane + 0..3):
  // with kOut, x's rows now (x1 replaces them after out_proj), else x's at the epilogue
  bf16x4_t res_v[kNormRows];
  if constexpr (kOut) {
#pragma unroll
    for (int j = 0; j < kNormRows; ++j) {
      const int row = min(m0 + wave + kWaves * j, a.m - 1);
      res_v[j] = *reinterpret_cast<const bf16x4_t*>(a.x + (int64_t)row * kD + lane * 4);
    }
  }

  // h's panel: thread tid copies 16-byte groups tid, tid + kThreads, ... (row-major).
  {
    constexpr int kGroups = BM * kD / 8;
    const auto hr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__bf16*>(a.h), (short)0, ((a.m - 1) * a.ldh + kD) * 2, 0x00020000);
    constexpr int kBatch = 8;
#pragma unroll
    for (int b0 = 0; b0 < kGroups; b0 += kThreads * kBatch) {
      uint4 v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int gi = b0 + j * kThreads + tid;
        if (gi < kGroups) {
          const int r = gi / (kD / 8), c = gi % (kD / 8);
          const int row = min(m0 + r, a.m - 1);
          v[j] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(hr, (row * a.ldh + 8 * c) * 2, 0, 0));
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int gi = b0 + j * kThreads + tid;
        if (gi < kGroups) {
          const int r = gi / (kD / 8), c = gi % (kD / 8);
          *reinterpret_cast<uint4*>(hs + xs_at<BM>(r, 8 * c)) = v[j];
        }
      }
    }
  }
  __syncthreads();

  const int x_lane = xs_at<BM>(l16, 8 * q4);  // B fragments: row tile i, K step s at
                                              // x_lane + (s * BM + 16 i) * 32
  f32x4 y[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) y[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 xa[2][MT];

  if constexpr (kOut) {
    // ---- out_proj into y over the attention rows in hs (linear_kernel's K order), then
    // linear_kernel's kAddNorm epilogue: bias, bf16, staged row-major over the chunk
    // buffers, x1 = bf16(x + y) per row (kept in res_v), h = LN2(x1) into hs
#pragma unroll
    for (int i = 0; i < MT; ++i)
      xa[0][i] = *reinterpret_cast<const bf16x8*>(hs + x_lane + 16 * i * 32);
#pragma unroll
    for (int s = 0; s < kS1; ++s) {
#pragma unroll
      for (int t = 0; t < 2; ++t) ring[(s + kDepth) % kR][t] = w_at(s + kDepth, t);
      if (s + 1 < kS1) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
          xa[(s + 1) & 1][i] =
              *reinterpret_cast<const bf16x8*>(hs + x_lane + ((s + 1) * BM + 16 * i) * 32);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          y[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ring[s % kR][t], xa[s & 1][i],
                                                            y[i][t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    float bov[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const bf16x4_t bv = *reinterpret_cast<const bf16x4_t*>(a.bo + c0 + 16 * t + 4 * q4);
#pragma unroll
      for (int e = 0; e < 4; ++e) bov[t][e] = (float)bv[e];
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        bf16x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (__bf16)(y[i][t][e] + bov[t][e]);
        *reinterpret_cast<bf16x4_t*>(us + (16 * i + l16) * kOutStride + c0 + 16 * t + 4 * q4) =
            o;
        y[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    __syncthreads();  // the tile is staged; every wavefront is past its reads of hs
    const bf16x4_t wv4 = *reinterpret_cast<const bf16x4_t*>(a.ln2_w + lane * 4);
    const bf16x4_t bv4 = *reinterpret_cast<const bf16x4_t*>(a.ln2_b + lane * 4);
#pragma unroll
    for (int j = 0; j < kNormRows; ++j) {  // every row of the tile: A phases read them all
      const int r = wave + kWaves * j;
      const bf16x4_t yv = *reinterpret_cast<const bf16x4_t*>(us + r * kOutStride + lane * 4);
      float v[4];
      bf16x4_t x1;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        x1[k] = (__bf16)((float)res_v[j][k] + (float)yv[k]);
        v[k] = (float)x1[k];
      }
      res_v[j] = x1;
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) sum += v[k];
      for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
      const float mean = sum / (float)kD;
      float sq = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float d = v[k] - mean;
        sq += d * d;
      }
      for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
      const float rstd = 1.0f / sqrtf(sq / (float)kD + a.eps2);
      bf16x4_t o;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        o[k] = (__bf16)((v[k] - mean) * rstd * (float)wv4[k] + (float)bv4[k]);
      *reinterpret_cast<bf16x4_t*>(hs + xs_at<BM>(r, 4 * lane)) = o;
    }
    __syncthreads();  // h's panel is complete; the staged tile is dead
  }

  // Phases of 8 K steps: A(c) = linear1 of chunk c into u[c & 1], B(c) = linear2's K
  // slice of chunk c into y, G(c) = chunk c's bias + GELU into chunk buffer c & 1, in the
  // order A0 | A1 G0 | bar | B0 | A2 G1 | bar | B1 | A3 G2 | bar | B2 G3 | bar | B3:
  // each GELU runs on VALU beside another phase's MFMAs, and every chunk buffer is written
  // only after the barrier that follows the last read of its previous contents.
  f32x4 u[2][MT][2];
#pragma unroll
  for (int p = 0; p < kPhases; ++p) {
    const bool w2 = phase_w2(p);
    const int c = phase_chunk(p);
    const int gc = phase_gelu(p);  // the chunk whose GELU runs in this phase, or -1
    const __bf16* src = w2 ? us + (c & 1) * kPanel : hs;  // the B operands' panel
    bf16x4_t b1v[2];  // linear1's bias at this lane's columns of chunk gc
    if (gc >= 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
        b1v[t] = *reinterpret_cast<const bf16x4_t*>(a.b1 + kC * gc + c0 + 16 * t + 4 * q4);
    }
    if (!w2) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t) u[c & 1][i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
      xa[0][i] = *reinterpret_cast<const bf16x8*>(src + x_lane + 16 * i * 32);
#pragma unroll
    for (int s = 0; s < kS1; ++s) {
      const int g = kPre + kS1 * p + s;
      if (g + kDepth < kPre + kS1 * kPhases) {
#pragma unroll
        for (int t = 0; t < 2; ++t) ring[(g + kDepth) % kR][t] = w_at(g + kDepth, t);
      }
      if (s + 1 < kS1) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
          xa[(s + 1) & 1][i] =
              *reinterpret_cast<const bf16x8*>(src + x_lane + ((s + 1) * BM + 16 * i) * 32);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (w2)
            y[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ring[g % kR][t], xa[s & 1][i],
                                                              y[i][t], 0, 0, 0);
          else
            u[c & 1][i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                ring[g % kR][t], xa[s & 1][i], u[c & 1][i][t], 0, 0, 0);
        }
      // one 4-column group of G(gc) a step: bias, bf16, GELU, bf16 (linear_kernel's GELU
      // epilogue); lane l holds hidden columns c0 + 16 t + 4 q4 + 0..3 of row 16 i + l16
      if (gc >= 0 && s < 2 * MT) {
        const int i = s / 2, t = s % 2;
        bf16x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const __bf16 v = (__bf16)(u[gc & 1][i][t][e] + (float)b1v[t][e]);
          o[e] = (__bf16)gelu((float)v);
        }
        *reinterpret_cast<bf16x4_t*>(us + (gc & 1) * kPanel +
                                     xs_at<BM>(16 * i + l16, c0 + 16 * t + 4 * q4)) = o;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (phase_barrier(p)) __syncthreads();
  }

  // ---- epilogue: bias, bf16, staged row-major over h's panel and chunk buffer 0 (both
  // dead: every wavefront passed the last chunk's barrier after its last read of them)
  float b2v[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const bf16x4_t bv = *reinterpret_cast<const bf16x4_t*>(a.b2 + c0 + 16 * t + 4 * q4);
#pragma unroll
    for (int e = 0; e < 4; ++e) b2v[t][e] = (float)bv[e];
  }
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      bf16x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (__bf16)(y[i][t][e] + b2v[t][e]);
      *reinterpret_cast<bf16x4_t*>(staged + (16 * i + l16) * kOutStride + c0 + 16 * t +
                                   4 * q4) = o;
    }
  if constexpr (!kOut) {
#pragma unroll
    for (int j = 0; j < kNormRows; ++j) {
      const int row = min(m0 + wave + kWaves * j, a.m - 1);
      res_v[j] = *reinterpret_cast<const bf16x4_t*>(a.x + (int64_t)row * kD + lane * 4);
    }
  }
  __syncthreads();
  // one wavefront a row, 4 elements a lane: x_out = bf16(res + y); with ln_w, the
  // LayerNorm of linear_kernel's kAddNorm epilogue
  constexpr int KE = kD / 64;
  const bool norm = a.ln_w != nullptr;
  bf16x4_t wv4, bv4;
  if (norm) {
    wv4 = *reinterpret_cast<const bf16x4_t*>(a.ln_w + lane * KE);
    bv4 = *reinterpret_cast<const bf16x4_t*>(a.ln_b + lane * KE);
  }
#pragma unroll
  for (int j = 0; j < kNormRows; ++j) {
    const int r = wave + kWaves * j;
    const int row = m0 + r;
    if (row >= a.m) break;
    const bf16x4_t yv = *reinterpret_cast<const bf16x4_t*>(staged + r * kOutStride + lane * KE);
    const int64_t at = (int64_t)row * kD + lane * KE;
    const bf16x4_t xv = res_v[j];
    float v[KE];
    bf16x4_t xo;
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      xo[k] = (__bf16)((float)xv[k] + (float)yv[k]);
      v[k] = (float)xo[k];
    }
    *reinterpret_cast<bf16x4_t*>(a.x_out + at) = xo;
    if (!norm) continue;
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < KE; ++k) sum += v[k];
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    const float mean = sum / (float)kD;
    float sq = 0.0f;
#pragma unroll
    for (int k = 0; k < KE; ++k) {
      const float d = v[k] - mean;
      sq += d * d;
    }
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
    const float rstd = 1.0f / sqrtf(sq / (float)kD + a.eps);
    bf16x4_t o;
#pragma unroll
    for (int k = 0; k < KE; ++k)
      o[k] = (__bf16)((v[k] - mean) * rstd * (float)wv4[k] + (float)bv4[k]);
    *reinterpret_cast<bf16x4_t*>(a.ln + at) = o;
  }
}

}  // namespace ffn

}  // namespace linear
}  // namespace cugo_amd

using namespace cugo_amd::linear;

extern "C" {

int cugo_linear(int act, const void* x, int64_t ldx, const void* w_packed, const void* bias,
                const void* residual, int64_t ldr, int64_t m, int64_t n, int64_t k, void* y,
                int64_t ldy, int tile, hipStream_t stream) {
  if (m < 0 || n < 1 || k < 1 || (m > 0 && (!x || !w_packed || !y))) return -1;
  if (act != CUGO_LINEAR_NONE && act != CUGO_LINEAR_GELU) return -2;
  const bool k_ok = k == 64 || k == 128 || k == 256 || k == 512 || k == 1024;
  if (!k_ok || ldx < k || ldx % 8 != 0 || ldy < n ||
      (residual != nullptr && (n % 4 != 0 || ldy % 4 != 0 || (ldr != 0 && (ldr < n || ldr % 4 != 0)))))
    return -3;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_packed)) % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(bias) |
       reinterpret_cast<uintptr_t>(residual)) % 8 != 0)
    return -4;
  // Buffer offsets are 32-bit byte offsets.
  if (m * ldx >= (int64_t(1) << 30) || (n + 15) * k >= (int64_t(1) << 30)) return -5;
  if (m == 0) return 0;
  Args a{};
  a.x = static_cast<const __bf16*>(x);
  a.w = static_cast<const __bf16*>(w_packed);
  a.bias = static_cast<const __bf16*>(bias);
  a.res = static_cast<const __bf16*>(residual);
  a.ldr = (int)ldr;
  a.y = static_cast<__bf16*>(y);
  a.m = (int)m;
  a.n = (int)n;
  a.ldx = (int)ldx;
  a.ldy = (int)ldy;
  a.wtiles = (int)((n + 15) / 16);
  if (tile == 0) {  // by the decoder step's shapes: 64-row tiles once 32-row ones pass
    // ~4 a CU, 128-row tiles past ~8 (in_proj, us by tile 1 / 2 / 4: 4,096 x 768 x 256
    // 5.7 / 6.4 / 6.2; 12,288 rows 12.6 / 12.6 / 12.0; 16,384 rows 16.5 / 15.6 / 13.2)
    const int64_t blocks32 = ((m + 31) / 32) * ((n + 127) / 128);
    tile = blocks32 > 2048 && k <= 512 ? 4 : blocks32 > 1024 ? 2 : 1;
  }
  switch (tile) {
    case 1: return launch<2, 2, 1, 4, 3>(a, (int)k, act, stream);  // 32 rows x 128 columns
    case 2: return launch<2, 2, 2, 4, 3>(a, (int)k, act, stream);  // 64 x 128, 8 wavefronts
    case 3: return launch<2, 4, 2, 2, 2>(a, (int)k, act, stream);  // 64 x 128
    case 4: return launch<4, 2, 2, 4, 2>(a, (int)k, act, stream);  // 128 x 128, 8 wavefronts
    case 5: return launch<2, 2, 2, 2, 3>(a, (int)k, act, stream);  // 64 x 64
    case 6: return launch<4, 4, 2, 2, 2>(a, (int)k, act, stream);  // 128 x 128, 4 waves
    case 7: return launch<2, 4, 1, 4, 2>(a, (int)k, act, stream);  // 32 x 256
    default: return -6;
  }
}

int cugo_linear_add_layernorm(const void* x, int64_t ldx, const void* w_packed,
                              const void* bias, int64_t m, int64_t n, int64_t k, const void* res,
                              int64_t ldr, const void* ln_weight, const void* ln_bias, float eps,
                              void* x_out, void* ln, int tile, hipStream_t stream) {
  if (m < 0 || (m > 0 && (!x || !w_packed || !res || !ln_weight || !ln_bias || !x_out || !ln)))
    return -1;
  const bool k_ok = k == 64 || k == 128 || k == 256 || k == 512 || k == 1024;
  if (!k_ok || n != 256 || ldx < k || ldx % 8 != 0 || (ldr != 0 && (ldr < n || ldr % 4 != 0)))
    return -3;
  const uintptr_t p16 = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_packed);
  const uintptr_t p8 = reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(res) |
                       reinterpret_cast<uintptr_t>(ln_weight) |
                       reinterpret_cast<uintptr_t>(ln_bias) | reinterpret_cast<uintptr_t>(x_out) |
                       reinterpret_cast<uintptr_t>(ln);
  if (p16 % 16 != 0 || p8 % 8 != 0) return -4;
  if (m * ldx >= (int64_t(1) << 30) || (n + 15) * k >= (int64_t(1) << 30)) return -5;
  if (m == 0) return 0;
  Args a{};
  a.x = static_cast<const __bf16*>(x);
  a.w = static_cast<const __bf16*>(w_packed);
  a.bias = static_cast<const __bf16*>(bias);
  a.y = static_cast<__bf16*>(x_out);
  a.m = (int)m;
  a.n = (int)n;
  a.ldx = (int)ldx;
  a.ldy = (int)n;
  a.wtiles = (int)((n + 15) / 16);
  a.res = static_cast<const __bf16*>(res);
  a.ldr = (int)ldr;
  a.ln_w = static_cast<const __bf16*>(ln_weight);
  a.ln_b = static_cast<const __bf16*>(ln_bias);
  a.ln = static_cast<__bf16*>(ln);
  a.eps = eps;
  // By shape: 64-row tiles for the deep (k = 1,024) layer of 8,192 rows or more (W's bytes
  // a row halve: 17.8 against 19.1 us at 12,288 rows), 32-row tiles otherwise.
  if (tile == 0) tile = k > 512 && m >= 8192 ? 4 : 2;
  switch (tile) {
    case 1: return launch<2, 4, 1, 4, 2>(a, (int)k, kAddNorm, stream);  // 32 x 256, 4 waves
    case 2: return launch<2, 2, 1, 8, 3>(a, (int)k, kAddNorm, stream);  // 32 x 256, 8 waves
    case 3: return launch<1, 4, 1, 4, 2>(a, (int)k, kAddNorm, stream);  // 16 x 256, 4 waves
    case 4: return launch<4, 2, 1, 8, 2>(a, (int)k, kAddNorm, stream);  // 64 x 256, 8 waves
    default: return -6;
  }
}


// The launch shared by cugo_ffn and cugo_out_proj_ffn: rows a workgroup (0: by m) and
// the kernel with or without the out_proj prologue.
static int ffn_launch(const ffn::Args& a, int rows, bool out, hipStream_t stream) {
  const int64_t m = a.m;
  if (rows == 0) {
    // Rows a workgroup: every workgroup streams all 1 MiB of weights through its CU's
    // L1 (1.125 MiB with out_proj), which bounds the kernel, so the tile that leaves each
    // CU the fewest rows (rounds of one workgroup a CU x rows), the larger on a tie (fewer
    // workgroups streaming the weights).  Measured with out_proj (us, 16 / 32 / 48 / 64
    // rows): 4,096 rows 19.7 / 24.7 / 33.2 / -; 8,192: 30.6 / 27.5 / 33.8 / -; 12,288:
    // 42.9 / 48.8 / 36.0 / 43.4; 16,384: - / 53.4 / 65.8 / 45.7; without it, 12,288: 39.5 /
    // 34.0 / 31.1 / 36.6.
    // the device's CU count, asked once a device (every caller stores the same answer)
    static std::atomic<int> cus_of[64];
    int cus = 256;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
      cus = cus_of[dev].load(std::memory_order_relaxed);
      if (cus == 0) {
        int n = 0;
        cus = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) ==
                          hipSuccess && n > 0 ? n : 256;
        cus_of[dev].store(cus, std::memory_order_relaxed);
      }
    }
    int64_t best = -1;
    for (int r : {16, 32, 48, 64}) {
      const int64_t load = ((m + r - 1) / r + cus - 1) / cus * r;
      if (best < 0 || load <= best) {
        best = load;
        rows = r;
      }
    }
  }
  // K steps of weights in flight: 3 -> 5 took 12,288 rows from 33.2 to 31.9 us (48-row
  // tiles), 7 no further
  const auto grid = [&](int r) { return (unsigned)((m + r - 1) / r); };
#define CUGO_FFN_LAUNCH(MT, R)                                                            \
  if (out)                                                                                \
    ffn::ffn_kernel<MT, 5, true><<<grid(R), ffn::kThreads, 0, stream>>>(a);               \
  else                                                                                    \
    ffn::ffn_kernel<MT, 5, false><<<grid(R), ffn::kThreads, 0, stream>>>(a);              \
  break;
  switch (rows) {
    case 16: CUGO_FFN_LAUNCH(1, 16)
    case 32: CUGO_FFN_LAUNCH(2, 32)
    case 48: CUGO_FFN_LAUNCH(3, 48)
    case 64: CUGO_FFN_LAUNCH(4, 64)
    default: return -6;
  }
#undef CUGO_FFN_LAUNCH
  return (int)hipGetLastError();
}

// Argument checks of the feed-forward half, shared by both entry points.
static int ffn_check(const void* h, int64_t ldh, const void* x, const void* w1_packed,
                     const void* b1, const void* w2_packed, const void* b2, const void* ln_weight,
                     const void* ln_bias, int64_t m, const void* x_out, const void* ln) {
  if (m < 0 || (m > 0 && (!h || !x || !w1_packed || !b1 || !w2_packed || !b2 || !x_out)) ||
      (ln_weight == nullptr) != (ln_bias == nullptr) || (m > 0 && ln_weight != nullptr && !ln))
    return -1;
  if (ldh < 256 || ldh % 8 != 0) return -3;
  const uintptr_t p16 = reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(w1_packed) |
                        reinterpret_cast<uintptr_t>(w2_packed);
  const uintptr_t p8 = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(b1) |
                       reinterpret_cast<uintptr_t>(b2) | reinterpret_cast<uintptr_t>(x_out) |
                       reinterpret_cast<uintptr_t>(ln_weight) |
                       reinterpret_cast<uintptr_t>(ln_bias) | reinterpret_cast<uintptr_t>(ln);
  if (p16 % 16 != 0 || p8 % 8 != 0) return -4;
  if (m * ldh >= (int64_t(1) << 30)) return -5;
  return 0;
}

static ffn::Args ffn_args(const void* h, int64_t ldh, const void* x, const void* w1_packed,
                          const void* b1, const void* w2_packed, const void* b2,
                          const void* ln_weight, const void* ln_bias, float eps, int64_t m,
                          void* x_out, void* ln) {
  ffn::Args a{};
  a.h = static_cast<const __bf16*>(h);
  a.x = static_cast<const __bf16*>(x);
  a.w1 = static_cast<const __bf16*>(w1_packed);
  a.b1 = static_cast<const __bf16*>(b1);
  a.w2 = static_cast<const __bf16*>(w2_packed);
  a.b2 = static_cast<const __bf16*>(b2);
  a.ln_w = static_cast<const __bf16*>(ln_weight);
  a.ln_b = static_cast<const __bf16*>(ln_bias);
  a.eps = eps;
  a.x_out = static_cast<__bf16*>(x_out);
  a.ln = static_cast<__bf16*>(ln);
  a.m = (int)m;
  a.ldh = (int)ldh;
  return a;
}

int cugo_ffn(const void* h, int64_t ldh, const void* x, const void* w1_packed, const void* b1,
             const void* w2_packed, const void* b2, const void* ln_weight, const void* ln_bias,
             float eps, int64_t m, void* x_out, void* ln, int rows, hipStream_t stream) {
  const int rc = ffn_check(h, ldh, x, w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, m,
                           x_out, ln);
  if (rc != 0 || m == 0) return rc;
  return ffn_launch(
      ffn_args(h, ldh, x, w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, eps, m, x_out, ln),
      rows, false, stream);
}

int cugo_out_proj_ffn(const void* att, int64_t ld_att, const void* x, const void* wo_packed,
                      const void* bo, const void* ln2_weight, const void* ln2_bias, float eps2,
                      const void* w1_packed, const void* b1, const void* w2_packed,
                      const void* b2, const void* ln_weight, const void* ln_bias, float eps,
                      int64_t m, void* x_out, void* ln, int rows, hipStream_t stream) {
  int rc = ffn_check(att, ld_att, x, w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, m, x_out,
                     ln);
  if (rc != 0) return rc;
  if (m > 0 && (!wo_packed || !bo || !ln2_weight || !ln2_bias)) return -1;
  if ((reinterpret_cast<uintptr_t>(wo_packed) % 16) != 0 ||
      ((reinterpret_cast<uintptr_t>(bo) | reinterpret_cast<uintptr_t>(ln2_weight) |
        reinterpret_cast<uintptr_t>(ln2_bias)) % 8) != 0)
    return -4;
  if (m == 0) return 0;
  ffn::Args a =
      ffn_args(att, ld_att, x, w1_packed, b1, w2_packed, b2, ln_weight, ln_bias, eps, m, x_out, ln);
  a.wo = static_cast<const __bf16*>(wo_packed);
  a.bo = static_cast<const __bf16*>(bo);
  a.ln2_w = static_cast<const __bf16*>(ln2_weight);
  a.ln2_b = static_cast<const __bf16*>(ln2_bias);
  a.eps2 = eps2;
  return ffn_launch(a, rows, true, stream);
}

}  // extern "C"
