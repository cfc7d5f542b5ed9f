// Radial MLP of the conv-TP weights on fp32 matrix cores (v_mfma_f32_16x16x4f32).
//
// Semantics: the reference's radial network (`blocks.py:234-241`,
// `radial.py` RadialMLP): w = silu(silu(silu(ef W0) W1) W2) W3, with the
// e3nn-normalised weights folded into W0..W3 at load time, no biases.
// Shapes: ef [E][nb], W0 [nb][64], W1, W2 [64][64], W3 [64][W] (W = 128 * slots).
//
// The work is split so every launch has thousands of waves:
//   k_mlp_hidden     W0..W2 staged in LDS, 16-edge groups per wave: h3 [E][64]
//   k_mlp_out        w = h3 @ W3, block tile 64 edges x W/2 columns
//   k_mlp_gh3        dL/dh3 = gw @ W3^T, 32 edges per block, K split over 4 waves, deep prefetch
//   k_mlp_hidden_bwd same grouping: recompute the pre-activations, back to dL/def
//
// Fragment layout of the 16x16x4 instruction (checked on gfx950): lane l holds
// A[l%16][k] and B[k][l%16] with k = l/16; accumulator element i of lane l is
// D[4*(l/16) + i][l%16].  The contraction index may be permuted as long as A
// and B agree, so for a 16-wide k chunk lane group g = l/16 takes
// k = 16c + 4g + s at step s: A and B values then come as one float4 per lane
// whenever the operand is stored with k contiguous.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "common.h"

namespace mace {
namespace {

typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4v mfma16(float a, float b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// sigmoid from the hardware exp2 / reciprocal (about 2 ulp); saturates cleanly:
// exp overflow gives rcp(inf) = 0
__device__ __forceinline__ float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }
__device__ __forceinline__ float dsilu(float x) {
  const float s = sigmoid(x);
  return s * (1.f + x * (1.f - s));
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float comp(const float4& v, int s) {
  return s == 0 ? v.x : s == 1 ? v.y : s == 2 ? v.z : v.w;
}

// Orders this wave's LDS accesses before and after the call (the tile is
// private to the wave, so no block barrier is needed).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int H = RADIAL_H;  // hidden width (64)
constexpr int XP = H + 4;    // padded LDS row
constexpr int RT = 16;       // edges per wave in the hidden-layer kernels

constexpr int WP = H + 1;  // LDS row stride of the staged weights (conflict-free both ways)

// The three small weight matrices of one radial MLP, staged once per block.
struct MlpW {
  float w0[NBESSEL_MAX][WP];
  float w1[H][WP];
  float w2[H][WP];
};

__device__ __forceinline__ void stage_weights(MlpW& sw, int nb, const float* __restrict__ W0,
                                              const float* __restrict__ W1, const float* __restrict__ W2) {
  for (int i = threadIdx.x; i < nb * H; i += blockDim.x) sw.w0[i / H][i % H] = W0[i];
  for (int i = threadIdx.x; i < H * H; i += blockDim.x) {
    sw.w1[i / H][i % H] = W1[i];
    sw.w2[i / H][i % H] = W2[i];
  }
  __syncthreads();
}

// One wave: out(16 x 64) = A(16 x K) @ B(K x 64), A in a wave-private LDS tile
// (row stride XP); B[k][n] = Wl[k][n], or Wl[n][k] when TR (the transposed
// product of the backward pass), Wl staged in LDS with row stride WP.
template <bool TR>
__device__ __forceinline__ void wave_gemm_lds(const float (*A)[XP], int K, const float (*Wl)[WP], f4v* acc) {
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f4v{0.f, 0.f, 0.f, 0.f};
  if (K % 16 != 0) {  // radial-basis input (K = num_bessel): plain k-steps, zero padded
    for (int k0 = 0; k0 < K; k0 += 4) {
      const int k = k0 + g;
      const float a = (k < K) ? A[r][k] : 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float b = (k < K) ? (TR ? Wl[16 * t + r][k] : Wl[k][16 * t + r]) : 0.f;
        acc[t] = mfma16(a, b, acc[t]);
      }
    }
    return;
  }
  for (int c = 0; c < K; c += 16) {
    const float4 a4 = ld4(&A[r][c + 4 * g]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = c + 4 * g + s;
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = mfma16(comp(a4, s), TR ? Wl[16 * t + r][k] : Wl[k][16 * t + r], acc[t]);
    }
  }
}

// accumulator tiles (optionally through silu) -> wave-private LDS tile
// (activations rounded to fp16 values under the float16 feature policy)
__device__ __forceinline__ void store_tile(float (*X)[XP], const f4v* acc, bool act, bool half = false) {
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) X[4 * g + i][16 * t + r] = act ? qh(silu(acc[t][i]), half) : acc[t][i];
}

// Rows e0..e0+15 of ef into the wave's tile, then the three hidden layers;
// leaves the pre-activations a1..a3 in accumulator layout.
__device__ __forceinline__ void hidden_fwd(float (*X)[XP], const MlpW& sw, int64_t E, int64_t e0, int nb,
                                           const float* __restrict__ ef, f4v* a1, f4v* a2, f4v* a3, bool half) {
  const int l = threadIdx.x & 63;
  for (int i = l; i < RT * nb; i += 64) {
    const int e = i / nb, k = i % nb;
    X[e][k] = (e0 + e < E) ? ef[(e0 + e) * nb + k] : 0.f;
  }
  wave_sync();
  wave_gemm_lds<false>(X, nb, sw.w0, a1);
  wave_sync();
  store_tile(X, a1, true, half);
  wave_sync();
  wave_gemm_lds<false>(X, H, sw.w1, a2);
  wave_sync();
  store_tile(X, a2, true, half);
  wave_sync();
  wave_gemm_lds<false>(X, H, sw.w2, a3);
  wave_sync();
}

// Waves walk 16-edge groups (grid-stride) after the block has staged W0..W2.
// Output h3 by MODE: H3_F32 float [E][64]; H3_F16 (float16 feature policy)
// _Float16 [E][64]; H3_SPLIT (operand of the split-fp16 product) _Float16
// [E][2][64]: row e scaled by a power of two that maps its largest magnitude into
// [2^14, 2^15), then hi = fp16(v) in [e][0] and lo = fp16(v - hi) in [e][1];
// h3inv[e] = the inverse scale.
constexpr int H3_F32 = 0, H3_F16 = 1, H3_SPLIT = 2;

template <int MODE>
__global__ void __launch_bounds__(256) k_mlp_hidden(int64_t E, int nb, const float* __restrict__ ef,
                                                    const float* __restrict__ W0, const float* __restrict__ W1,
                                                    const float* __restrict__ W2, void* __restrict__ h3v,
                                                    float* __restrict__ h3inv) {
  __shared__ MlpW sw;
  __shared__ __align__(16) float sX[4][RT][XP];
  stage_weights(sw, nb, W0, W1, W2);
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t ngroups = (E + RT - 1) / RT;
  for (int64_t gi = (int64_t)blockIdx.x * 4 + wv; gi < ngroups; gi += (int64_t)gridDim.x * 4) {
    const int64_t e0 = gi * RT;
    f4v a1[4], a2[4], a3[4];
    hidden_fwd(sX[wv], sw, E, e0, nb, ef, a1, a2, a3, MODE == H3_F16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t e = e0 + 4 * g + i;  // row 4g + i lies in lanes 16g .. 16g + 15, columns 16t + r
      if constexpr (MODE == H3_SPLIT) {
        float v[4], m = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          v[t] = silu(a3[t][i]);
          m = fmaxf(m, fabsf(v[t]));
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        const int ex = m > 0.f ? ilogbf(m) : 0;
        const float sc = ldexpf(1.f, 14 - ex);
        if (e < E) {
          _Float16* dst = static_cast<_Float16*>(h3v) + e * 2 * H;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float x = v[t] * sc;
            const _Float16 hi = (_Float16)x;
            dst[16 * t + r] = hi;
            dst[H + 16 * t + r] = (_Float16)(x - (float)hi);
          }
          if (r == 0) h3inv[e] = ldexpf(1.f, ex - 14);
        }
      } else {
        using HT = typename std::conditional<MODE == H3_F16, _Float16, float>::type;
        if (e < E)
#pragma unroll
          for (int t = 0; t < 4; ++t) static_cast<HT*>(h3v)[e * H + 16 * t + r] = (HT)silu(a3[t][i]);
      }
    }
  }
}

// w[E][W] = h3[E][64] @ W3, W3 given transposed (W3T [W][64], k contiguous).
// Block = 64 edges x W/2 columns; wave q takes W/8 columns (a multiple of 16;
// the last step is half wide when it is not a multiple of 32) in steps of 32 with the 64 x 64 A fragments held in registers and the B
// values of the next step loaded during the current one.  Each step's 64 x 32
// result goes through a wave-private LDS tile so that it is written as whole
// 128-byte row segments.  (Plain stores: the TP kernel that reads w next finds
// it in the last-level cache.)
__global__ void __launch_bounds__(256) k_mlp_out(int64_t E, int W, const float* __restrict__ h3,
                                                 const float* __restrict__ W3T, float* __restrict__ w) {
  __shared__ __align__(16) float sO[4][64][36];
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 64;
  const int per = W / 8;
  const int cb = blockIdx.y * (W / 2) + wv * per, ce = cb + per;
  float4 a[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t row = min(row0 + 16 * t + r, E - 1);  // rows past the end are computed, not stored
#pragma unroll
    for (int c = 0; c < 4; ++c) a[t][c] = ld4(h3 + row * H + 16 * c + 4 * g);
  }
  float4 b[2][4], bn[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int c = 0; c < 4; ++c) b[u][c] = ld4(W3T + (int64_t)min(cb + 16 * u + r, W - 1) * H + 16 * c + 4 * g);
  float(*O)[36] = sO[wv];
  for (int c0 = cb; c0 < ce; c0 += 32) {
    if (c0 + 32 < ce) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          bn[u][c] = ld4(W3T + (int64_t)min(c0 + 32 + 16 * u + r, W - 1) * H + 16 * c + 4 * g);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the multiplies
    f4v o[4][2];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) o[t][u] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int u = 0; u < 2; ++u) o[t][u] = mfma16(comp(a[t][c], s), comp(b[u][c], s), o[t][u]);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) O[16 * t + 4 * g + i][16 * u + r] = o[t][u][i];
    wave_sync();
#pragma unroll
    for (int q = 0; q < 8; ++q) {  // lane l: row l/8 + 8q, columns 4 (l%8) .. + 3
      const int rr = (l >> 3) + 8 * q;
      const int64_t row = row0 + rr;
      if (row < E && c0 + 4 * (l & 7) < ce) {
        *reinterpret_cast<float4*>(&w[row * W + c0 + 4 * (l & 7)]) = ld4(&O[rr][4 * (l & 7)]);
      }
    }
    wave_sync();
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) b[u][c] = bn[u][c];
  }
}

// Float16 feature policy: w[E][W] (fp16) = h3[E][64] (fp16) @ W3 (fp16, given
// transposed W3T [W][64]) on v_mfma_f32_16x16x32_f16 with fp32 accumulation;
// lane l holds A[l%16][8(l/16) .. +7] and B[8(l/16) .. +7][l%16] of a 32-wide
// k chunk (checked on gfx950), D as in the fp32 instruction.  Tiling as in
// k_mlp_out; each 64 x 32 result is staged in LDS as fp16 and written as 64-byte
// row segments.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4v mfma16h(h8 a, h8 b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__global__ void __launch_bounds__(256) k_mlp_out_h(int64_t E, int W, const _Float16* __restrict__ h3,
                                                   const _Float16* __restrict__ W3T, _Float16* __restrict__ w) {
  __shared__ __align__(16) _Float16 sO[4][64][40];
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 64;
  const int per = W / 8;
  const int cb = blockIdx.y * (W / 2) + wv * per, ce = cb + per;
  h8 a[4][2];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t row = min(row0 + 16 * t + r, E - 1);  // rows past the end are computed, not stored
#pragma unroll
    for (int c = 0; c < 2; ++c) a[t][c] = *reinterpret_cast<const h8*>(h3 + row * H + 32 * c + 8 * g);
  }
  h8 b[2][2], bn[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int c = 0; c < 2; ++c)
      b[u][c] = *reinterpret_cast<const h8*>(W3T + (int64_t)min(cb + 16 * u + r, W - 1) * H + 32 * c + 8 * g);
  _Float16(*O)[40] = sO[wv];
  for (int c0 = cb; c0 < ce; c0 += 32) {
    if (c0 + 32 < ce) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          bn[u][c] = *reinterpret_cast<const h8*>(W3T + (int64_t)min(c0 + 32 + 16 * u + r, W - 1) * H + 32 * c +
                                                  8 * g);
    }
    __builtin_amdgcn_sched_barrier(0);
    f4v o[4][2];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) o[t][u] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) o[t][u] = mfma16h(a[t][c], b[u][c], o[t][u]);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) O[16 * t + 4 * g + i][16 * u + r] = (_Float16)o[t][u][i];
    wave_sync();
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // lane l: row l/4 + 16q, columns 8 (l%4) .. + 7
      const int rr = (l >> 2) + 16 * q;
      const int64_t row = row0 + rr;
      if (row < E && c0 + 8 * (l & 3) < ce)
        *reinterpret_cast<h8*>(&w[row * W + c0 + 8 * (l & 3)]) = *reinterpret_cast<const h8*>(&O[rr][8 * (l & 3)]);
    }
    wave_sync();
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int c = 0; c < 2; ++c) b[u][c] = bn[u][c];
  }
}

// Float32 policy on fp16 matrix cores: w[E][W] (fp32) = h3 @ W3 with both
// operands split into fp16 pairs, a = a_hi + a_lo (h3 per-row scaled, see
// k_mlp_hidden; W3 scaled by one power of two, cscale = its inverse), and
//   a b ~ a_hi b_hi + a_hi b_lo + a_lo b_hi
// on v_mfma_f32_16x16x32_f16 with fp32 accumulation (the dropped a_lo b_lo and
// the split residuals are about 2^-22 of |a b|).  W3Tx = [hi | lo] planes of W3^T
// [W][64].  Tiling, prefetch and the LDS-staged 128-byte row stores as in
// k_mlp_out; the row scales are applied when the tile is staged.
__global__ void __launch_bounds__(256) k_mlp_out_x(int64_t E, int W, const _Float16* __restrict__ h3x,
                                                   const float* __restrict__ h3inv,
                                                   const _Float16* __restrict__ W3Tx, float cscale,
                                                   float* __restrict__ w) {
  __shared__ __align__(16) float sO[4][64][36];
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 64;
  const int per = W / 8;
  const int cb = blockIdx.y * (W / 2) + wv * per, ce = cb + per;
  h8 ah[4][2], al[4][2];
  float rs[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t row = min(row0 + 16 * t + r, E - 1);  // rows past the end are computed, not stored
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      ah[t][c] = *reinterpret_cast<const h8*>(h3x + row * 2 * H + 32 * c + 8 * g);
      al[t][c] = *reinterpret_cast<const h8*>(h3x + row * 2 * H + H + 32 * c + 8 * g);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) rs[t][i] = h3inv[min(row0 + 16 * t + 4 * g + i, E - 1)] * cscale;
  }
  const _Float16* W3lo = W3Tx + (int64_t)W * H;
  h8 bh[2][2], bl[2][2], bnh[2][2], bnl[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int64_t o = (int64_t)min(cb + 16 * u + r, W - 1) * H + 32 * c + 8 * g;
      bh[u][c] = *reinterpret_cast<const h8*>(W3Tx + o);
      bl[u][c] = *reinterpret_cast<const h8*>(W3lo + o);
    }
  float(*O)[36] = sO[wv];
  for (int c0 = cb; c0 < ce; c0 += 32) {
    if (c0 + 32 < ce) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int64_t o = (int64_t)min(c0 + 32 + 16 * u + r, W - 1) * H + 32 * c + 8 * g;
          bnh[u][c] = *reinterpret_cast<const h8*>(W3Tx + o);
          bnl[u][c] = *reinterpret_cast<const h8*>(W3lo + o);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the multiplies
    f4v o[4][2];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) o[t][u] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          o[t][u] = mfma16h(ah[t][c], bl[u][c], o[t][u]);
          o[t][u] = mfma16h(al[t][c], bh[u][c], o[t][u]);
          o[t][u] = mfma16h(ah[t][c], bh[u][c], o[t][u]);
        }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) O[16 * t + 4 * g + i][16 * u + r] = o[t][u][i] * rs[t][i];
    wave_sync();
#pragma unroll
    for (int q = 0; q < 8; ++q) {  // lane l: row l/8 + 8q, columns 4 (l%8) .. + 3
      const int rr = (l >> 3) + 8 * q;
      const int64_t row = row0 + rr;
      if (row < E && c0 + 4 * (l & 7) < ce)
        *reinterpret_cast<float4*>(&w[row * W + c0 + 4 * (l & 7)]) = ld4(&O[rr][4 * (l & 7)]);
    }
    wave_sync();
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        bh[u][c] = bnh[u][c];
        bl[u][c] = bnl[u][c];
      }
  }
}

// gh3[E][64] = gw[E][W] @ W3^T with W3 [64][W] (k contiguous).  Block = 32
// edges; wave q takes the k range [q W/4, (q+1) W/4) in 16-wide chunks.  The
// gw rows (the HBM stream) are loaded GH_PF chunks ahead through a register
// ring, the W3 values one chunk ahead; the four partial tiles are summed in
// LDS in a fixed order.
constexpr int GH_PF = 4;

__global__ void __launch_bounds__(256) k_mlp_gh3(int64_t E, int W, const float* __restrict__ gw,
                                                 const float* __restrict__ W3, float* __restrict__ gh3) {
  __shared__ f4v sP[4][8][64];
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 32;
  const int kq = W / 4, kb = wv * kq, nch = kq / 16;
  const float* ar[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t row = min(row0 + 16 * t + r, E - 1);  // rows past the end are computed, not stored
    ar[t] = gw + row * (int64_t)W + kb + 4 * g;
  }
  const float* br = W3 + (int64_t)r * W + kb + 4 * g;
  float4 ring[GH_PF][2], b[4], bn[4];
#pragma unroll
  for (int p = 0; p < GH_PF; ++p)
#pragma unroll
    for (int t = 0; t < 2; ++t) ring[p][t] = ld4(ar[t] + 16 * min(p, nch - 1));
#pragma unroll
  for (int u = 0; u < 4; ++u) b[u] = ld4(br + (int64_t)16 * u * W);
  f4v acc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = f4v{0.f, 0.f, 0.f, 0.f};
  for (int ch = 0; ch < nch; ch += GH_PF) {
#pragma unroll
    for (int p = 0; p < GH_PF; ++p) {
      const int cc = ch + p;
      if (cc < nch) {
        const int nbk = min(cc + 1, nch - 1), na = min(cc + GH_PF, nch - 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) bn[u] = ld4(br + (int64_t)16 * u * W + 16 * nbk);
        const float4 cur[2] = {ring[p][0], ring[p][1]};
#pragma unroll
        for (int t = 0; t < 2; ++t) ring[p][t] = ld4(ar[t] + 16 * na);
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the multiplies
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[t][u] = mfma16(comp(cur[t], s), comp(b[u], s), acc[t][u]);
#pragma unroll
        for (int u = 0; u < 4; ++u) b[u] = bn[u];
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) sP[wv][t][l] = acc[t >> 2][t & 3];
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = 2 * wv + h, rt = t >> 2, ct = t & 3;
    const f4v s = ((sP[0][t][l] + sP[1][t][l]) + sP[2][t][l]) + sP[3][t][l];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + 16 * rt + 4 * g + i;
      if (row < E) gh3[row * H + 16 * ct + r] = s[i];
    }
  }
}

// Float16 feature policy: gh3 = gw @ W3^T with gw fp16 [E][W] scaled per (edge,
// channel half) -- gw[e][slot*128 + u] * gscale[e][u / 64] is the gradient -- and
// W3 fp16 [64][W]; v_mfma_f32_16x16x32_f16 with fp32 accumulation.  A 32-wide k
// chunk lies in one channel half, so the products of the two halves accumulate
// separately and are combined with their row scales before the fixed-order
// cross-wave sum.  Block = 32 edges, K split over the 4 waves, gw chunks loaded
// GH_PF ahead.
__global__ void __launch_bounds__(256) k_mlp_gh3_h(int64_t E, int W, const _Float16* __restrict__ gw,
                                                   const float* __restrict__ gscale,
                                                   const _Float16* __restrict__ W3h, float* __restrict__ gh3) {
  __shared__ f4v sP[4][8][64];
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * 32;
  const int kq = W / 4, kb = wv * kq, nch = kq / 32;
  const _Float16* ar[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t row = min(row0 + 16 * t + r, E - 1);  // rows past the end are computed, not stored
    ar[t] = gw + row * (int64_t)W + kb + 8 * g;
  }
  const _Float16* br = W3h + (int64_t)r * W + kb + 8 * g;
  h8 ring[GH_PF][2], b[4], bn[4];
#pragma unroll
  for (int p = 0; p < GH_PF; ++p)
#pragma unroll
    for (int t = 0; t < 2; ++t) ring[p][t] = *reinterpret_cast<const h8*>(ar[t] + 32 * min(p, nch - 1));
#pragma unroll
  for (int u = 0; u < 4; ++u) b[u] = *reinterpret_cast<const h8*>(br + (int64_t)16 * u * W);
  f4v acc[2][2][4];  // [channel half][row tile][column tile]
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[hh][t][u] = f4v{0.f, 0.f, 0.f, 0.f};
  for (int ch = 0; ch < nch; ch += GH_PF) {
#pragma unroll
    for (int p = 0; p < GH_PF; ++p) {
      const int cc = ch + p;
      if (cc < nch) {
        const int nbk = min(cc + 1, nch - 1), na = min(cc + GH_PF, nch - 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) bn[u] = *reinterpret_cast<const h8*>(br + (int64_t)16 * u * W + 32 * nbk);
        const h8 cur[2] = {ring[p][0], ring[p][1]};
#pragma unroll
        for (int t = 0; t < 2; ++t) ring[p][t] = *reinterpret_cast<const h8*>(ar[t] + 32 * na);
        __builtin_amdgcn_sched_barrier(0);
        if ((kb + 32 * cc) & 64) {  // second channel half of a slot
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[1][t][u] = mfma16h(cur[t], b[u], acc[1][t][u]);
        } else {
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[0][t][u] = mfma16h(cur[t], b[u], acc[0][t][u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) b[u] = bn[u];
      }
    }
  }
  // combine the halves with their row scales (rows 4g + i of each row tile)
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = min(row0 + 16 * t + 4 * g + i, E - 1);
      const float s0 = gscale[2 * row], s1 = gscale[2 * row + 1];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[0][t][u][i] = acc[0][t][u][i] * s0 + acc[1][t][u][i] * s1;
    }
#pragma unroll
  for (int t = 0; t < 8; ++t) sP[wv][t][l] = acc[0][t >> 2][t & 3];
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = 2 * wv + h, rt = t >> 2, ct = t & 3;
    const f4v sm = ((sP[0][t][l] + sP[1][t][l]) + sP[2][t][l]) + sP[3][t][l];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + 16 * rt + 4 * g + i;
      if (row < E) gh3[row * H + 16 * ct + r] = sm[i];
    }
  }
}

// Float32 policy on fp16 matrix cores: gh3 = gw @ W3^T from the fp32 gradient gw
// [E][W].  Each wave runs the whole K loop for 16 edges in 32-wide chunks; the
// block stages each chunk of W3x = [hi | lo] planes of W3 [64][W] (scaled by
// 1 / cscale) in LDS, double-buffered.  Operand roles are swapped (A = W3 rows
// j, B = gw^T with the edges as columns), so lane (g, r) owns edge r's eight k
// values of the chunk and the output column of that edge: it scales them by the
// power of two that maps the chunk's largest |gw| of the edge (reduced over the
// four lanes of the edge) into [2^14, 2^15), splits them into fp16 hi + lo and
// folds the inverse scale into its accumulators after the chunk's three products
//   W3_hi x gw_lo + W3_lo x gw_hi + W3_hi x gw_hi
// (about 2^-22 relative per product).  gw loaded GX_PF chunks ahead.
constexpr int GX_PF = 2;

__global__ void __launch_bounds__(256) k_mlp_gh3_x(int64_t E, int W, const float* __restrict__ gw,
                                                   const _Float16* __restrict__ W3x, float cscale,
                                                   float* __restrict__ gh3) {
  __shared__ __align__(16) _Float16 sB[2][2][H][32];  // [buffer][hi, lo][j][k of the chunk]
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wv) * 16, lo_b = (int64_t)H * W;
  const int nch = W / 32;
  const float* ar = gw + min(row0 + r, E - 1) * (int64_t)W + 8 * g;  // rows past the end: computed, not stored
  const int bj = threadIdx.x >> 2, bk = 8 * (threadIdx.x & 3);      // staging: one 8-wide k piece of row bj
  const _Float16* bsrc = W3x + (int64_t)bj * W + bk;
  float4 ring[GX_PF][2];
#pragma unroll
  for (int p = 0; p < GX_PF; ++p) {
    const float* q = ar + 32 * min(p, nch - 1);
    ring[p][0] = ld4(q);
    ring[p][1] = ld4(q + 4);
  }
  h8 st0 = *reinterpret_cast<const h8*>(bsrc), st1 = *reinterpret_cast<const h8*>(bsrc + lo_b);
  *reinterpret_cast<h8*>(&sB[0][0][bj][bk]) = st0;
  *reinterpret_cast<h8*>(&sB[0][1][bj][bk]) = st1;
  __syncthreads();
  f4v acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) acc[u] = f4v{0.f, 0.f, 0.f, 0.f};
  for (int ch = 0; ch < nch; ch += GX_PF) {
#pragma unroll
    for (int p = 0; p < GX_PF; ++p) {
      const int cc = ch + p;
      if (cc < nch) {  // uniform over the block
        const int buf = cc & 1;
        if (cc + 1 < nch) {
          st0 = *reinterpret_cast<const h8*>(bsrc + 32 * (cc + 1));
          st1 = *reinterpret_cast<const h8*>(bsrc + lo_b + 32 * (cc + 1));
        }
        const float4 c0 = ring[p][0], c1 = ring[p][1];
        {
          const float* q = ar + 32 * min(cc + GX_PF, nch - 1);
          ring[p][0] = ld4(q);
          ring[p][1] = ld4(q + 4);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the arithmetic
        const float v[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        float m = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(v[q]));
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        // floor(log2 m) from the exponent field; zero / subnormal chunks take -100 (finite scales)
        const int ex = max((int)((__float_as_uint(m) >> 23) & 0xff) - 127, -100);
        const float sc = __uint_as_float((unsigned)(127 + 14 - ex) << 23);
        const float inv = __uint_as_float((unsigned)(127 - 14 + ex) << 23);
        h8 xh, xl;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float x = v[q] * sc;
          const _Float16 hi = (_Float16)x;
          xh[q] = hi;
          xl[q] = (_Float16)(x - (float)hi);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const h8 wh = *reinterpret_cast<const h8*>(&sB[buf][0][16 * u + r][8 * g]);
          const h8 wl = *reinterpret_cast<const h8*>(&sB[buf][1][16 * u + r][8 * g]);
          f4v d = mfma16h(wl, xh, f4v{0.f, 0.f, 0.f, 0.f});
          d = mfma16h(wh, xl, d);
          d = mfma16h(wh, xh, d);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] = fmaf(d[i], inv, acc[u][i]);
        }
        if (cc + 1 < nch) {
          *reinterpret_cast<h8*>(&sB[buf ^ 1][0][bj][bk]) = st0;
          *reinterpret_cast<h8*>(&sB[buf ^ 1][1][bj][bk]) = st1;
        }
        __syncthreads();
      }
    }
  }
  const int64_t row = row0 + r;  // lane (g, r) holds gh3[row][16u + 4g + i]
  if (row < E)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      *reinterpret_cast<float4*>(gh3 + row * H + 16 * u + 4 * g) =
          float4{acc[u][0] * cscale, acc[u][1] * cscale, acc[u][2] * cscale, acc[u][3] * cscale};
}

// dL/def from dL/dh3: recompute a1..a3, then
//   g_a3 = g_h3 * silu'(a3), g_a2 = (g_a3 W2^T) * silu'(a2),
//   g_a1 = (g_a2 W1^T) * silu'(a1), g_ef = g_a1 W0^T
// (the transposed products read the staged W0..W2 transposed).
__global__ void __launch_bounds__(256) k_mlp_hidden_bwd(int64_t E, int nb, const float* __restrict__ ef,
                                                        const float* __restrict__ W0, const float* __restrict__ W1,
                                                        const float* __restrict__ W2, const float* __restrict__ gh3,
                                                        float* __restrict__ gef, int accumulate, int half) {
  __shared__ MlpW sw;
  __shared__ __align__(16) float sX[4][RT][XP];
  stage_weights(sw, nb, W0, W1, W2);
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  float(*X)[XP] = sX[wv];
  const int64_t ngroups = (E + RT - 1) / RT;
  for (int64_t gi = (int64_t)blockIdx.x * 4 + wv; gi < ngroups; gi += (int64_t)gridDim.x * 4) {
    const int64_t e0 = gi * RT;
    f4v a1[4], a2[4], a3[4], t[4];
    hidden_fwd(X, sw, E, e0, nb, ef, a1, a2, a3, half);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t e = e0 + 4 * g + i;
#pragma unroll
      for (int q = 0; q < 4; ++q) t[q][i] = (e < E) ? gh3[e * H + 16 * q + r] * dsilu(a3[q][i]) : 0.f;
    }
    store_tile(X, t, false);
    wave_sync();
    wave_gemm_lds<true>(X, H, sw.w2, t);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) t[q][i] *= dsilu(a2[q][i]);
    wave_sync();
    store_tile(X, t, false);
    wave_sync();
    wave_gemm_lds<true>(X, H, sw.w1, t);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) t[q][i] *= dsilu(a1[q][i]);
    wave_sync();
    store_tile(X, t, false);
    wave_sync();
    // g_ef (16 x nb) = g_a1 (16 x 64) @ W0^T: one column tile, columns >= nb padded
    f4v o = f4v{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < H; c += 16) {
      const float4 a4 = ld4(&X[r][c + 4 * g]);
#pragma unroll
      for (int s = 0; s < 4; ++s) o = mfma16(comp(a4, s), (r < nb) ? sw.w0[r][c + 4 * g + s] : 0.f, o);
    }
    if (r < nb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t e = e0 + 4 * g + i;
        if (e < E) {
          float* dst = gef + e * nb + r;
          *dst = accumulate ? *dst + o[i] : o[i];
        }
      }
    }
    wave_sync();
  }
}

inline unsigned nblk(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

}  // namespace

// grid of the hidden-layer kernels: enough blocks to fill the device, each
// staging the weights once and walking several 64-edge groups
inline unsigned hidden_grid(int64_t E) { return (unsigned)std::min<int64_t>((E + 63) / 64, 512); }

void launch_mlp_hidden(hipStream_t st, int64_t E, int nb, const float* ef, const float* W0, const float* W1,
                       const float* W2, void* h3, float* h3inv, int mode) {
  if (E <= 0) return;
  const dim3 grid(hidden_grid(E)), blk(256);
  if (mode == H3_SPLIT)
    hipLaunchKernelGGL(k_mlp_hidden<H3_SPLIT>, grid, blk, 0, st, E, nb, ef, W0, W1, W2, h3, h3inv);
  else if (mode == H3_F16)
    hipLaunchKernelGGL(k_mlp_hidden<H3_F16>, grid, blk, 0, st, E, nb, ef, W0, W1, W2, h3, h3inv);
  else
    hipLaunchKernelGGL(k_mlp_hidden<H3_F32>, grid, blk, 0, st, E, nb, ef, W0, W1, W2, h3, h3inv);
}

void launch_mlp_out(hipStream_t st, int64_t E, int W, const void* h3, const void* W3T, void* w, int half) {
  if (E <= 0) return;
  if (half)
    hipLaunchKernelGGL(k_mlp_out_h, dim3(nblk(E, 64), 2), dim3(256), 0, st, E, W, static_cast<const _Float16*>(h3),
                       static_cast<const _Float16*>(W3T), static_cast<_Float16*>(w));
  else
    hipLaunchKernelGGL(k_mlp_out, dim3(nblk(E, 64), 2), dim3(256), 0, st, E, W, static_cast<const float*>(h3),
                       static_cast<const float*>(W3T), static_cast<float*>(w));
}

void launch_mlp_out_x(hipStream_t st, int64_t E, int W, const void* h3x, const float* h3inv, const void* W3Tx,
                      float cscale, float* w) {
  if (E <= 0) return;
  hipLaunchKernelGGL(k_mlp_out_x, dim3(nblk(E, 64), 2), dim3(256), 0, st, E, W, static_cast<const _Float16*>(h3x),
                     h3inv, static_cast<const _Float16*>(W3Tx), cscale, w);
}

void launch_mlp_gh3(hipStream_t st, int64_t E, int W, const float* gw, const float* W3, float* gh3) {
  if (E <= 0) return;
  hipLaunchKernelGGL(k_mlp_gh3, dim3(nblk(E, 32)), dim3(256), 0, st, E, W, gw, W3, gh3);
}

void launch_mlp_gh3_x(hipStream_t st, int64_t E, int W, const float* gw, const void* W3x, float cscale,
                      float* gh3) {
  if (E <= 0) return;
  hipLaunchKernelGGL(k_mlp_gh3_x, dim3(nblk(E, 64)), dim3(256), 0, st, E, W, gw,
                     static_cast<const _Float16*>(W3x), cscale, gh3);
}

void launch_mlp_gh3_h(hipStream_t st, int64_t E, int W, const void* gw, const float* gscale, const void* W3h,
                      float* gh3) {
  if (E <= 0) return;
  hipLaunchKernelGGL(k_mlp_gh3_h, dim3(nblk(E, 32)), dim3(256), 0, st, E, W, static_cast<const _Float16*>(gw),
                     gscale, static_cast<const _Float16*>(W3h), gh3);
}

void launch_mlp_hidden_bwd(hipStream_t st, int64_t E, int nb, const float* ef, const float* W0, const float* W1,
                           const float* W2, const float* gh3, float* gef, int accumulate, int half) {
  if (E <= 0) return;
  hipLaunchKernelGGL(k_mlp_hidden_bwd, dim3(hidden_grid(E)), dim3(256), 0, st, E, nb, ef, W0, W1, W2, gh3, gef,
                     accumulate, half);
}

}  // namespace mace
