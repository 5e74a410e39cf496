// Fused forward pass of the residual MLP actor on MFMA, for gfx950.
//
// The actor (cugo_amd/rollout.py ResidualMlpActor, the PPO rollout's policy):
//   h = x W_in^T + b_in
//   for each block:  h = h + W2 relu(W1 LN(h) + b1) + b2       (LN with its own affine)
//   z = LN(h);  logits = z W_l^T + b_l;  value = z w_v + b_v
// With one GEMM per layer through a library, every layer reads and writes a [B, 512]
// activation tensor in HBM and each residual add + LayerNorm is another pass over two of
// them.  Here a workgroup owns 64 rows for the whole network: the residual stream h stays
// in the wavefronts' MFMA accumulators (fp32), each layer's bf16 input (x, LN(h) or
// relu(...)) sits in LDS, and only the weights stream in from L2.
//
// Layout of the work (512 threads, 8 wavefronts, two per SIMD, one workgroup per CU):
//   * wavefront w computes output columns [64 w, 64 w + 64) of every 512-wide layer for
//     all 64 rows: 4 x 4 tiles of 16 x 16, v_mfma_f32_16x16x32_bf16 over K in steps of 32
//     (lane l holds A[l % 16][8 (l / 16) + 0..7], B[8 (l / 16) + 0..7][l % 16] and
//     D[4 (l / 16) + 0..3][l % 16]);
//   * A fragments are 16-byte LDS reads of the row-major bf16 activation (row stride 520
//     elements, so the 16 rows of a fragment start on different banks);
//   * B fragments come from weights packed once in fragment order (cugo_mlp_pack_weight):
//     the 64 lanes' 8 values of one (16-row tile, K step) are 1 KiB of contiguous memory,
//     so one load instruction is a contiguous 1 KiB read.  Read straight from the Linear
//     weight [out, in], the 16 lanes of a quarter-wave would touch 16 rows, 16 cache
//     lines per quarter-wave: the L1's tag lookups, not the MFMAs, bounded that form
//     (0.29 ms for 32,768 rows);
//   * the B fragments sit in a ring of registers kDepth K steps ahead of the MFMAs (the K
//     loop is unrolled, so the ring is indexed statically);
//   * LayerNorm: per-row sum and sum of squares over a wavefront's 64 columns by
//     shuffles, across the 8 wavefronts through LDS;
//   * the head (up to 255 logits + the value) is one 256-wide layer, 32 columns a
//     wavefront.
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
constexpr int kM = 64;                   // rows per workgroup
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMT = kM / 16;             // row tiles
constexpr int kNT = kD / (16 * kWaves);  // column tiles per wavefront
constexpr int kK = 32;                   // K per MFMA
constexpr int kFrag = 64 * 8;            // elements of one packed B fragment
constexpr int kZS = kD + 8;              // LDS row stride (elements) of the activations
constexpr int kHeadN = CUGO_MLP_HEAD_ROWS;  // logits + value, padded
constexpr int kHeadNT = kHeadN / (16 * kWaves);
constexpr int kMaxIn = CUGO_MLP_MAX_FEATURES;
constexpr int kMaxBlocks = CUGO_MLP_MAX_BLOCKS;
constexpr int kInSteps = kMaxIn / kK;    // K steps of the input layer (zero-padded)
// K steps of weights in flight ahead of the MFMAs (CUGO_MLP_DEPTH pins it for tuning
// builds).
#ifdef CUGO_MLP_DEPTH
constexpr int kDepth = CUGO_MLP_DEPTH;
#else
constexpr int kDepth = 4;
#endif
constexpr int kActBytes = kM * kZS * 2;                  // one activation buffer
constexpr int kSmemBytes = 2 * kActBytes;                // Z and U (x overlays both)
static_assert(kM * (kMaxIn + 8) * 2 <= kSmemBytes, "the input tile must fit in Z and U");
static_assert(kMaxIn % kK == 0 && kHeadN % (16 * kWaves) == 0, "whole tiles");

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

// acc[mt][t] += A[16 mt .., 0..32 STEPS) x B[.., 16 (tile0 + t) ..], A a row-major bf16
// LDS tile, B packed in fragment order: fragment (n tile, K step) at (tile * STEPS +
// step) * kFrag, lane l's 8 values at l * 8.  The K steps run from step `rot` round to
// `rot` - 1: workgroups that start together read the same weights, and a different
// starting step per workgroup spreads their reads over the matrix.
template <int NT, int STEPS>
__device__ inline void gemm(f32x4 (&acc)[kMT][NT], const __bf16* A, int a_stride,
                            const __bf16* packed, int tile0, int lane, int l16, int q4,
                            int rot) {
  constexpr int R = kDepth + 1;
  rot %= STEPS;
  const __bf16* base = packed + (size_t)tile0 * STEPS * kFrag + lane * 8;
  const __bf16* a_base = A + l16 * a_stride + 8 * q4;
  auto step_of = [rot](int s) {  // uniform over the workgroup
    int sk = s + rot;
    return sk - (sk >= STEPS ? STEPS : 0);
  };
  bf16x8 b[R][NT];
#pragma unroll
  for (int j = 0; j < kDepth; ++j)
    if (j < STEPS) {
      const int sk = step_of(j);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        b[j][t] = *reinterpret_cast<const bf16x8*>(base + (size_t)(t * STEPS + sk) * kFrag);
    }
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    if (s + kDepth < STEPS) {
      const int sk = step_of(s + kDepth);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        b[(s + kDepth) % R][t] =
            *reinterpret_cast<const bf16x8*>(base + (size_t)(t * STEPS + sk) * kFrag);
    }
    const int k = step_of(s) * kK;
    bf16x8 a[kMT];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
      a[mt] = *reinterpret_cast<const bf16x8*>(a_base + 16 * mt * a_stride + k);
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        acc[mt][t] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], b[s % R][t], acc[mt][t], 0, 0, 0);
  }
}

// acc[..][t][i] = bias[n0 + 16 t + l16] (every row).
template <int NT>
__device__ inline void set_bias(f32x4 (&acc)[kMT][NT], const __bf16* bias, int n0, int l16) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float v = (float)bias[n0 + 16 * t + l16];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) acc[mt][t] = f32x4{v, v, v, v};
  }
}

// Z[r][n] = bf16(LN(h)[r][n] * gamma[n] + beta[n]) for the wavefront's columns; every
// wavefront calls it (one barrier inside: the per-row partial sums cross wavefronts in
// `red`).
__device__ inline void layer_norm(const f32x4 (&h)[kMT][kNT], const __bf16* gamma,
                                  const __bf16* beta, float eps, __bf16* Z, float* red,
                                  int wave, int l16, int q4) {
  float s[kMT][4], ss[kMT][4];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        const float v = h[mt][t][i];
        a += v;
        b = __builtin_fmaf(v, v, b);
      }
      s[mt][i] = a;
      ss[mt][i] = b;
    }
  // the 16 lanes with the same q4 hold the same rows
#pragma unroll
  for (int off = 1; off < 16; off <<= 1)
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[mt][i] += __shfl_xor(s[mt][i], off, 64);
        ss[mt][i] += __shfl_xor(ss[mt][i], off, 64);
      }
  if (l16 == 0) {
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * mt + 4 * q4 + i;
        red[(wave * kM + r) * 2] = s[mt][i];
        red[(wave * kM + r) * 2 + 1] = ss[mt][i];
      }
  }
  __syncthreads();
  float g[kNT], be[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int n = wave * (16 * kNT) + 16 * t + l16;
    g[t] = (float)gamma[n];
    be[t] = (float)beta[n];
  }
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * mt + 4 * q4 + i;
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        a += red[(w * kM + r) * 2];
        b += red[(w * kM + r) * 2 + 1];
      }
      const float mean = a * (1.f / kD);
      const float var = fmaxf(b * (1.f / kD) - mean * mean, 0.f);
      const float rstd = 1.f / sqrtf(var + eps);
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        const int n = wave * (16 * kNT) + 16 * t + l16;
        Z[r * kZS + n] = (__bf16)((h[mt][t][i] - mean) * rstd * g[t] + be[t]);
      }
    }
}

template <class TIn>
struct Input;
template <>
struct Input<float> {
  // four elements as bf16
  __device__ static uint2 load4(const float* p) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    uint2 r;
    r.x = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v.x) |
          ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v.y) << 16);
    r.y = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v.z) |
          ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v.w) << 16);
    return r;
  }
};
template <>
struct Input<__bf16> {
  __device__ static uint2 load4(const __bf16* p) { return *reinterpret_cast<const uint2*>(p); }
};

template <class TIn>
__global__ __launch_bounds__(kThreads, 1) void actor_kernel(const TIn* __restrict__ x,
                                                            __bf16* __restrict__ x_copy,
                                                            int64_t n, Weights w,
                                                            __bf16* __restrict__ logits,
                                                            float* __restrict__ value) {
  __shared__ __attribute__((aligned(16))) __bf16 smem[kSmemBytes / 2];
  __shared__ float red[kWaves * kM * 2];
  __bf16* Z = smem;
  __bf16* U = smem + kActBytes / 2;
  __bf16* X = smem;  // the input tile, before the first LayerNorm

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * kM;
  const int F = w.features;
  constexpr int xs = kMaxIn + 8;  // LDS row stride of the input tile

  // ---- input tile -> LDS (bf16, zero columns up to kMaxIn), and its bf16 copy to x_copy
  {
    const int quads = F / 4;
    const int total = kM * quads;
    for (int j0 = 0; j0 < total; j0 += kThreads * 8) {
      uint2 v[8];
      int r[8], c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u * kThreads + tid;
        const int jj = j < total ? j : total - 1;
        r[u] = jj / quads;
        c[u] = jj - r[u] * quads;
        const int64_t g = row0 + r[u] < n ? row0 + r[u] : n - 1;
        v[u] = Input<TIn>::load4(x + g * F + 4 * c[u]);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u * kThreads + tid;
        if (j >= total) continue;
        const bool valid = row0 + r[u] < n;
        const uint2 val = valid ? v[u] : make_uint2(0u, 0u);
        *reinterpret_cast<uint2*>(X + r[u] * xs + 4 * c[u]) = val;
        if (x_copy != nullptr && valid)
          *reinterpret_cast<uint2*>(x_copy + (row0 + r[u]) * F + 4 * c[u]) = val;
      }
    }
    const int pad = kMaxIn - F;
    if (pad > 0)
      for (int j = tid; j < kM * pad; j += kThreads)
        X[(j / pad) * xs + F + j % pad] = (__bf16)0.f;
  }
  __syncthreads();

  const int n0 = wave * (16 * kNT);  // this wavefront's first column of a 512-wide layer
  const int tile0 = n0 / 16;
  const int rot = (int)(blockIdx.x % 64u);  // first K step of this workgroup's GEMMs
  f32x4 h[kMT][kNT];
  set_bias<kNT>(h, w.b_in, n0, l16);
  gemm<kNT, kInSteps>(h, X, xs, w.w_in, tile0, lane, l16, q4, rot);

  for (int b = 0; b < w.blocks; ++b) {
    // z = LN(h) -> Z.  The barrier inside comes after every wavefront's last read of the
    // previous layer's input (X or Z), so Z can be overwritten after it.
    layer_norm(h, w.ln_w[b], w.ln_b[b], w.eps, Z, red, wave, l16, q4);
    __syncthreads();  // Z complete
    // fc1 in two halves of the wavefront's columns, so that its accumulators, h and the
    // weight ring fit the 256 registers two wavefronts per SIMD allow.  relu(u) -> U (last
    // read by the previous block's second layer, before the barrier above).
    constexpr int kHalf = kNT / 2;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int c0 = n0 + 16 * kHalf * half;
      f32x4 u[kMT][kHalf];
      set_bias<kHalf>(u, w.b1[b], c0, l16);
      gemm<kHalf, kD / kK>(u, Z, kZS, w.w1[b], c0 / 16, lane, l16, q4, rot);
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int t = 0; t < kHalf; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            U[(16 * mt + 4 * q4 + i) * kZS + c0 + 16 * t + l16] =
                (__bf16)fmaxf(u[mt][t][i], 0.f);
    }
    __syncthreads();  // U complete
    {
      const __bf16* b2 = w.b2[b];
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        const float v = (float)b2[n0 + 16 * t + l16];
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt) h[mt][t] += f32x4{v, v, v, v};
      }
      gemm<kNT, kD / kK>(h, U, kZS, w.w2[b], tile0, lane, l16, q4, rot);
    }
  }

  layer_norm(h, w.ln_w[w.blocks], w.ln_b[w.blocks], w.eps, Z, red, wave, l16, q4);
  __syncthreads();  // Z complete

  // ---- head: columns [0, A) logits, A the value, the rest padding (zero weights)
  const int A = w.actions;
  const int hn0 = wave * (16 * kHeadNT);
  f32x4 o[kMT][kHeadNT];
#pragma unroll
  for (int t = 0; t < kHeadNT; ++t) {
    const int col = hn0 + 16 * t + l16;
    const float v = col <= A ? (float)w.b_head[col] : 0.f;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) o[mt][t] = f32x4{v, v, v, v};
  }
  gemm<kHeadNT, kD / kK>(o, Z, kZS, w.w_head, hn0 / 16, lane, l16, q4, rot);
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
