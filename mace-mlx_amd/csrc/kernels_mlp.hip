// Radial MLP of the conv-TP weights on fp32 matrix cores (v_mfma_f32_16x16x4f32).
//
// Semantics: the reference's radial network (`blocks.py:234-241`,
// `radial.py` RadialMLP): w = silu(silu(silu(ef W0) W1) W2) W3, with the
// e3nn-normalised weights folded into W0..W3 at load time, no biases.
// Shapes: ef [E][nb], W0 [nb][64], W1, W2 [64][64], W3 [64][W] (W = 128 * slots).
//
// The work is split so every launch has thousands of waves:
//   k_mlp_hidden     16 edges per wave, activations in registers, permuted W0..W2 tiles in LDS: h3
//   k_mlp_out        w = h3 @ W3, block tile 64 edges x W/2 columns (k_mlp_out_h: fp16 policy;
//                    k_mlp_out_x: float32 policy on fp16 matrix cores with split operands)
//   k_mlp_gh3        dL/dh3 = gw @ W3^T (k_mlp_gh3_h: fp16 policy; k_mlp_gh3_x: split operands)
//   k_mlp_hidden_bwd as k_mlp_hidden, from the saved silu' values back to dL/def
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

// ---------------------------------------------------------------------------
// Hidden layers, activations held in registers.
//
// Each wave takes 16 edges.  Products run with swapped roles, Y^T = W^T X^T:
// A = weight rows (output feature n = 16 t' + r), B = X^T with the 16 edges as
// columns, so lane (g, r) supplies edge r's inputs and receives, for output
// tile t', D[4g + i][r] = Y[edge r][n = 16 t' + 4g + i].  After a layer each lane
// therefore holds 16 of its edge's 64 features, n in {16 t + 4 g + i}, kept as
// v[4 t + i].  The next layer contracts over those registers directly: at k
// step s = 4 t + i lane group g supplies k = pi(s, g) = 16 t + 4 g + i (the
// steps cover every k once), and the weight tiles are staged in LDS permuted to
// the same order, one float4 (the four output tiles t') per lane and step.  The
// first layer contracts over the Bessel features with pi(s, g) = 4 s + g.
// ---------------------------------------------------------------------------
constexpr int NB4 = NBESSEL_MAX / 4;

__device__ __forceinline__ int kperm(int s, int g) { return 16 * (s >> 2) + 4 * g + (s & 3); }

// forward weight tiles: w0[s][g][r] = W0[4s + g][16 t' + r] (zero past nb),
// w1/w2[s][g][r] = W[kperm(s, g)][16 t' + r], t' = float4 component
struct MlpFwdW {
  float4 w0[NB4][4][16];
  float4 w1[16][4][16];
  float4 w2[16][4][16];
};
// transposed tiles of the backward pass: wTq[s][g][r] = W[16 t' + r][kperm(s, g)];
// w0T[t][g][r] = W0[r][16 t + 4 g + i] (component i; zero for r >= nb)
struct MlpBwdW {
  float4 w1T[16][4][16];
  float4 w2T[16][4][16];
  float4 w0T[4][4][16];
};

__device__ void stage_fwd(MlpFwdW& sw, int nb, const float* __restrict__ W0, const float* __restrict__ W1,
                          const float* __restrict__ W2) {
  float* w0 = &sw.w0[0][0][0].x;
  for (int i = threadIdx.x; i < NB4 * 4 * 16 * 4; i += blockDim.x) {
    const int tp = i & 3, r = (i >> 2) & 15, g = (i >> 6) & 3, st = i >> 8, k = 4 * st + g;
    w0[i] = k < nb ? W0[k * H + 16 * tp + r] : 0.f;
  }
  float* w1 = &sw.w1[0][0][0].x;
  float* w2 = &sw.w2[0][0][0].x;
  for (int i = threadIdx.x; i < 16 * 4 * 16 * 4; i += blockDim.x) {
    const int tp = i & 3, r = (i >> 2) & 15, g = (i >> 6) & 3, st = i >> 8, k = kperm(st, g);
    w1[i] = W1[k * H + 16 * tp + r];
    w2[i] = W2[k * H + 16 * tp + r];
  }
}

__device__ void stage_bwd(MlpBwdW& sw, int nb, const float* __restrict__ W0, const float* __restrict__ W1,
                          const float* __restrict__ W2) {
  float* w1 = &sw.w1T[0][0][0].x;
  float* w2 = &sw.w2T[0][0][0].x;
  for (int i = threadIdx.x; i < 16 * 4 * 16 * 4; i += blockDim.x) {
    const int tp = i & 3, r = (i >> 2) & 15, g = (i >> 6) & 3, st = i >> 8, n = kperm(st, g);
    w1[i] = W1[(16 * tp + r) * H + n];
    w2[i] = W2[(16 * tp + r) * H + n];
  }
  float* w0 = &sw.w0T[0][0][0].x;
  for (int i = threadIdx.x; i < 4 * 4 * 16 * 4; i += blockDim.x) {
    const int ii = i & 3, r = (i >> 2) & 15, g = (i >> 6) & 3, t = i >> 8;
    w0[i] = r < nb ? W0[r * H + 16 * t + 4 * g + ii] : 0.f;
  }
}

// builds the tile images once per model (one block); the kernels then stage them
// with coalesced float4 copies
__global__ void __launch_bounds__(256) k_mlp_permute(int nb, const float* __restrict__ W0,
                                                     const float* __restrict__ W1, const float* __restrict__ W2,
                                                     MlpFwdW* __restrict__ fw, MlpBwdW* __restrict__ bw) {
  stage_fwd(*fw, nb, W0, W1, W2);
  stage_bwd(*bw, nb, W0, W1, W2);
}

template <typename T>
__device__ __forceinline__ void stage_copy(T& dst, const T* __restrict__ src) {
  constexpr int N4 = sizeof(T) / 16;
  float4* d = reinterpret_cast<float4*>(&dst);
  const float4* q = reinterpret_cast<const float4*>(src);
  for (int i = threadIdx.x; i < N4; i += blockDim.x) d[i] = q[i];
}

// one 64-wide layer: acc[t'] = sum over the 16 k steps of W-tile (t') x v[s]; lane: the
// lane index (the LayerNorm kernels pass one the compiler cannot see as loop-invariant)
__device__ __forceinline__ void layer64(const float4 (*w)[4][16], const float* v, f4v* acc,
                                        int lane = threadIdx.x & 63) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const float4 wv = w[st][g][r];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = mfma16(comp(wv, t), v[st], acc[t]);
  }
}

// silu' of one layer's pre-activations (lane layout) into a saved row: d[16t + i] (d = row + 4g)
__device__ __forceinline__ void store_ds(float* d, const f4v* a) {
#pragma unroll
  for (int t = 0; t < 4; ++t)
    *reinterpret_cast<float4*>(d + 16 * t) = float4{dsilu(a[t][0]), dsilu(a[t][1]), dsilu(a[t][2]), dsilu(a[t][3])};
}

// The three hidden layers for edges e0 .. e0+15 (lane's edge e0 + r): leaves the
// pre-activations a3 (a[t][i] = feature 16t + 4g + i); activations between
// layers rounded by mode rnd (RND_*, the feature policy).  dsp (null or
// the lane's position in row ds[e][0][.]) receives silu' of a1..a3.
__device__ __forceinline__ void hidden_fwd(const MlpFwdW& sw, int64_t E, int64_t e0, int nb,
                                           const float* __restrict__ ef, f4v* a3, int rnd, float* dsp) {
  f4v a1[4], a2[4];
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t e = e0 + r;
#pragma unroll
  for (int t = 0; t < 4; ++t) a1[t] = f4v{0.f, 0.f, 0.f, 0.f};
  const int nst = (nb + 3) >> 2;
  for (int st = 0; st < nst; ++st) {
    const int k = 4 * st + g;
    const float x = (e < E && k < nb) ? ef[e * nb + k] : 0.f;
    const float4 wv = sw.w0[st][g][r];
#pragma unroll
    for (int t = 0; t < 4; ++t) a1[t] = mfma16(comp(wv, t), x, a1[t]);
  }
  float v[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) v[q] = qh(silu(a1[q >> 2][q & 3]), rnd);
  if (dsp) store_ds(dsp, a1);
  layer64(sw.w1, v, a2);
#pragma unroll
  for (int q = 0; q < 16; ++q) v[q] = qh(silu(a2[q >> 2][q & 3]), rnd);
  if (dsp) store_ds(dsp + H, a2);
  layer64(sw.w2, v, a3);
  if (dsp) store_ds(dsp + 2 * H, a3);
}

// 16-edge groups per wave (grid-stride) after the block has staged the weights.
// Output h3 by MODE: H3_F32 float [E][64]; H3_F16 (float16 feature policy)
// _Float16 [E][64]; H3_BF16 (bfloat16 policy) float [E][64] holding bf16 values; H3_SPLIT (operand of the split-fp16 product) _Float16
// [E][2][64]: row e scaled by a power of two that maps its largest magnitude into
// [2^14, 2^15), then hi = fp16(v) in [e][0] and lo = fp16(v - hi) in [e][1];
// h3inv[e] = the inverse scale.

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// ds (optional): silu'(a1), silu'(a2), silu'(a3) as ds[e][layer][64] for the backward pass.
template <int MODE>
__global__ void __launch_bounds__(256) k_mlp_hidden(int64_t E, int nb, const float* __restrict__ ef,
                                                    const MlpFwdW* __restrict__ tiles, void* __restrict__ h3v,
                                                    float* __restrict__ h3inv, float* __restrict__ ds) {
  __shared__ MlpFwdW sw;
  stage_copy(sw, tiles);
  __syncthreads();
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t ngroups = (E + 15) / 16;
  for (int64_t gi = (int64_t)blockIdx.x * 4 + wv; gi < ngroups; gi += (int64_t)gridDim.x * 4) {
    const int64_t e0 = gi * 16, e = e0 + r;
    f4v a3[4];
    constexpr int rnd = MODE == H3_F16 ? RND_F16 : MODE == H3_BF16 ? RND_BF16 : RND_NONE;
    hidden_fwd(sw, E, e0, nb, ef, a3, rnd, (ds && e < E) ? ds + e * 3 * H + 4 * g : nullptr);
    float v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = silu(a3[q >> 2][q & 3]);
    if constexpr (MODE == H3_BF16)
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = round_bf16(v[q]);
    if constexpr (MODE == H3_SPLIT) {
      float m = 0.f;
#pragma unroll
      for (int q = 0; q < 16; ++q) m = fmaxf(m, fabsf(v[q]));
      m = max4_rows(m);  // the four lanes of edge r
      // floor(log2 m) from the exponent field; zero / subnormal rows take -100 (finite scales)
      const int ex = max((int)((__float_as_uint(m) >> 23) & 0xff) - 127, -100);
      const float sc = __uint_as_float((unsigned)(127 + 14 - ex) << 23);
      if (e < E) {
        _Float16* dst = static_cast<_Float16*>(h3v) + e * 2 * H;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          h4 hi, lo;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x = v[4 * t + i] * sc;
            hi[i] = (_Float16)x;
            lo[i] = (_Float16)(x - (float)hi[i]);
          }
          *reinterpret_cast<h4*>(dst + 16 * t + 4 * g) = hi;
          *reinterpret_cast<h4*>(dst + H + 16 * t + 4 * g) = lo;
        }
        if (g == 0) h3inv[e] = __uint_as_float((unsigned)(127 - 14 + ex) << 23);
      }
    } else if constexpr (MODE == H3_F16) {
      if (e < E)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          *reinterpret_cast<h4*>(static_cast<_Float16*>(h3v) + e * H + 16 * t + 4 * g) =
              h4{(_Float16)v[4 * t], (_Float16)v[4 * t + 1], (_Float16)v[4 * t + 2], (_Float16)v[4 * t + 3]};
    } else {
      if (e < E)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          *reinterpret_cast<float4*>(static_cast<float*>(h3v) + e * H + 16 * t + 4 * g) =
              float4{v[4 * t], v[4 * t + 1], v[4 * t + 2], v[4 * t + 3]};
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
// bias (optional, [W]) and rs (optional, [E]): w = (h3 W3 + bias) rs[row] (the mh-1 block's output
// layer with its bias and, under apply_cutoff = false, the edge's envelope)
__global__ void __launch_bounds__(256) k_mlp_out(int64_t E, int W, const float* __restrict__ h3,
                                                 const float* __restrict__ W3T, float* __restrict__ w,
                                                 const float* __restrict__ bias, const float* __restrict__ rs,
                                                 int rnd) {
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
        float4 o = ld4(&O[rr][4 * (l & 7)]);
        if (bias) {
          const float4 bb = ld4(bias + c0 + 4 * (l & 7));
          o = float4{o.x + bb.x, o.y + bb.y, o.z + bb.z, o.w + bb.w};
        }
        if (rs) {
          const float f = rs[row];
          o = float4{o.x * f, o.y * f, o.z * f, o.w * f};
        }
        if (rnd) o = float4{qh(o.x, rnd), qh(o.y, rnd), qh(o.z, rnd), qh(o.w, rnd)};
        *reinterpret_cast<float4*>(&w[row * W + c0 + 4 * (l & 7)]) = o;
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
// k_mlp_out (stores nontemporal: the TP kernel streams w back with nontemporal loads);
// the row scales are applied when the tile is staged.  bias ([W]) and cut ([E]), each
// optional, make it w = (h3 W3 + bias) cut[e] (the mh-1 output layer).
__global__ void __launch_bounds__(256) k_mlp_out_x(int64_t E, int W, const _Float16* __restrict__ h3x,
                                                   const float* __restrict__ h3inv,
                                                   const _Float16* __restrict__ W3Tx, float cscale,
                                                   float* __restrict__ w, const float* __restrict__ bias,
                                                   const float* __restrict__ cut) {
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
      if (row < E && c0 + 4 * (l & 7) < ce) {
        f4v o = *reinterpret_cast<const f4v*>(&O[rr][4 * (l & 7)]);
        if (bias) o += *reinterpret_cast<const f4v*>(bias + c0 + 4 * (l & 7));
        if (cut) o *= cut[row];
        __builtin_nontemporal_store(o, reinterpret_cast<f4v*>(&w[row * W + c0 + 4 * (l & 7)]));
      }
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

// b3 (optional, [W]): also gwb[row] = sum_c gw[row][c] b3[c] (the mh-1 output layer's bias), summed
// per lane, over the lane's four k groups and over the four waves in a fixed order
__global__ void __launch_bounds__(256) k_mlp_gh3(int64_t E, int W, const float* __restrict__ gw,
                                                 const float* __restrict__ W3, float* __restrict__ gh3,
                                                 const float* __restrict__ b3, float* __restrict__ gwb) {
  __shared__ f4v sP[4][8][64];
  __shared__ float sB[4][2][16];
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
  float pb[2] = {0.f, 0.f};  // this lane's share of gw . b3 for its two rows
  for (int ch = 0; ch < nch; ch += GH_PF) {
#pragma unroll
    for (int p = 0; p < GH_PF; ++p) {
      const int cc = ch + p;
      if (cc < nch) {
        const int nbk = min(cc + 1, nch - 1), na = min(cc + GH_PF, nch - 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) bn[u] = ld4(br + (int64_t)16 * u * W + 16 * nbk);
        const float4 cur[2] = {ring[p][0], ring[p][1]};
        if (b3) {
          const float4 bb = ld4(b3 + kb + 16 * cc + 4 * g);
#pragma unroll
          for (int t = 0; t < 2; ++t)
            pb[t] = fmaf(cur[t].w, bb.w, fmaf(cur[t].z, bb.z, fmaf(cur[t].y, bb.y, fmaf(cur[t].x, bb.x, pb[t]))));
        }
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
  if (b3) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float q = sum4_rows(pb[t]);  // the four k groups of row 16 t + r
      if (g == 0) sB[wv][t][r] = q;
    }
  }
  __syncthreads();
  if (b3 && wv == 0 && l < 32) {
    const int t = l >> 4;
    const int64_t row = row0 + 16 * t + r;
    if (row < E) gwb[row] = ((sB[0][t][r] + sB[1][t][r]) + sB[2][t][r]) + sB[3][t][r];
  }
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
// [E][W].  Each wave runs the whole K loop for 16 edges in 64-wide stages; the
// block stages each stage of W3x = [hi | lo] planes of W3 [64][W] (scaled by
// 1 / cscale) in LDS, double-buffered (rows padded to 72 halves: conflict-free
// 16-byte reads).  Operand roles are swapped (A = W3 rows j, B = gw^T with the
// edges as columns), so lane (g, r) owns edge r's sixteen k values of the stage
// (two 32-wide MFMA chunks) and the output column of that edge: it scales them by
// the power of two that maps the stage's largest |gw| of the edge (reduced over
// the four lanes of the edge) into [2^14, 2^15), splits them into fp16 hi + lo and
// folds the inverse scale into its accumulators after the stage's products
//   W3_hi x gw_lo + W3_lo x gw_hi + W3_hi x gw_hi
// (about 2^-22 relative per product).  gw loaded two stages ahead.  b3 (optional,
// [W]): also gwb[e] = gw[e] . b3 in fp32, per lane, then over the edge's four lanes.
constexpr int GX_KS = 64;       // k per stage (one scale, one barrier)
constexpr int GX_RS = GX_KS + 8;

__global__ void __launch_bounds__(256) k_mlp_gh3_x(int64_t E, int W, const float* __restrict__ gw,
                                                   const _Float16* __restrict__ W3x, float cscale,
                                                   float* __restrict__ gh3, const float* __restrict__ b3,
                                                   float* __restrict__ gwb) {
  __shared__ __align__(16) _Float16 sB[2][2][H][GX_RS];  // [buffer][hi, lo][j][k of the stage]
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wv) * 16, lo_b = (int64_t)H * W;
  const int nst = W / GX_KS;
  const float* ar = gw + min(row0 + r, E - 1) * (int64_t)W + 8 * g;  // rows past the end: computed, not stored
  const int bj = threadIdx.x >> 2, bk = 8 * (threadIdx.x & 3);      // staging: row bj, k bk and bk + 32
  const _Float16* bsrc = W3x + (int64_t)bj * W + bk;
  float4 ring[2][2][2];  // [stage slot][32-wide chunk][two float4]
  auto load_x = [&](int st, float4 (*dst)[2]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float* p = ar + GX_KS * st + 32 * q;
      dst[q][0] = ld4(p);
      dst[q][1] = ld4(p + 4);
    }
  };
  h8 stw[2][2];  // [chunk][hi, lo]
  auto load_w = [&](int st) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const _Float16* p = bsrc + GX_KS * st + 32 * q;
      stw[q][0] = *reinterpret_cast<const h8*>(p);
      stw[q][1] = *reinterpret_cast<const h8*>(p + lo_b);
    }
  };
  auto store_w = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      *reinterpret_cast<h8*>(&sB[buf][0][bj][32 * q + bk]) = stw[q][0];
      *reinterpret_cast<h8*>(&sB[buf][1][bj][32 * q + bk]) = stw[q][1];
    }
  };
  load_x(0, ring[0]);
  load_x(min(1, nst - 1), ring[1]);
  load_w(0);
  store_w(0);
  __syncthreads();
  f4v acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) acc[u] = f4v{0.f, 0.f, 0.f, 0.f};
  float pb = 0.f;  // this lane's share of gw . b3
  for (int s0 = 0; s0 < nst; s0 += 2) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int st = s0 + p;
      if (st < nst) {  // uniform over the block
        const int buf = st & 1;
        if (st + 1 < nst) load_w(st + 1);
        float4 cur[2][2];
#pragma unroll
        for (int q = 0; q < 2; ++q) cur[q][0] = ring[p][q][0], cur[q][1] = ring[p][q][1];
        load_x(min(st + 2, nst - 1), ring[p]);
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the arithmetic
        if (b3) {
#pragma unroll
          for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float4 bb = ld4(b3 + GX_KS * st + 32 * q + 8 * g + 4 * h), x = cur[q][h];
              pb = fmaf(x.w, bb.w, fmaf(x.z, bb.z, fmaf(x.y, bb.y, fmaf(x.x, bb.x, pb))));
            }
        }
        float m = 0.f;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            m = fmaxf(m, fmaxf(fmaxf(fabsf(cur[q][h].x), fabsf(cur[q][h].y)),
                               fmaxf(fabsf(cur[q][h].z), fabsf(cur[q][h].w))));
        m = max4_rows(m);  // the four lanes of edge r
        // floor(log2 m) from the exponent field; zero / subnormal stages take -100 (finite scales)
        const int ex = max((int)((__float_as_uint(m) >> 23) & 0xff) - 127, -100);
        const float sc = __uint_as_float((unsigned)(127 + 14 - ex) << 23);
        const float inv = __uint_as_float((unsigned)(127 - 14 + ex) << 23);
        f4v d[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) d[u] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float v[8] = {cur[q][0].x, cur[q][0].y, cur[q][0].z, cur[q][0].w,
                              cur[q][1].x, cur[q][1].y, cur[q][1].z, cur[q][1].w};
          h8 xh, xl;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float x = v[j] * sc;
            const _Float16 hi = (_Float16)x;
            xh[j] = hi;
            xl[j] = (_Float16)(x - (float)hi);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const h8 wh = *reinterpret_cast<const h8*>(&sB[buf][0][16 * u + r][32 * q + 8 * g]);
            const h8 wl = *reinterpret_cast<const h8*>(&sB[buf][1][16 * u + r][32 * q + 8 * g]);
            d[u] = mfma16h(wl, xh, d[u]);
            d[u] = mfma16h(wh, xl, d[u]);
            d[u] = mfma16h(wh, xh, d[u]);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] = fmaf(d[u][i], inv, acc[u][i]);
        if (st + 1 < nst) store_w(buf ^ 1);
        __syncthreads();
      }
    }
  }
  const int64_t row = row0 + r;  // lane (g, r) holds gh3[row][16u + 4g + i]
  if (b3) {
    pb = sum4_rows(pb);
    if (g == 0 && row < E) gwb[row] = pb;
  }
  if (row < E)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      *reinterpret_cast<float4*>(gh3 + row * H + 16 * u + 4 * g) =
          float4{acc[u][0] * cscale, acc[u][1] * cscale, acc[u][2] * cscale, acc[u][3] * cscale};
}

// dL/def from dL/dh3 for 16 edges per wave, with silu'(a1..a3) saved by the
// forward kernel (ds[e][layer][64]):
//   g_a3 = g_h3 * silu'(a3), g_a2 = (g_a3 W2^T) * silu'(a2),
//   g_a1 = (g_a2 W1^T) * silu'(a1), g_ef = g_a1 W0^T
// in the register layout of the forward pass (the transposed products read the
// staged transposed tiles; g_ef comes out as D[k = 4g + i][edge r], k < nb).
__device__ __forceinline__ void ld_row16(const float* p, int g, float* v) {  // features 16t + 4g + i
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float4 x = ld4(p + 16 * t + 4 * g);
    v[4 * t] = x.x, v[4 * t + 1] = x.y, v[4 * t + 2] = x.z, v[4 * t + 3] = x.w;
  }
}

__global__ void __launch_bounds__(256) k_mlp_hidden_bwd(int64_t E, int nb, const MlpBwdW* __restrict__ tiles,
                                                        const float* __restrict__ ds, const float* __restrict__ gh3,
                                                        float* __restrict__ gef, int accumulate) {
  __shared__ MlpBwdW sw;
  stage_copy(sw, tiles);
  __syncthreads();
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t ngroups = (E + 15) / 16;
  for (int64_t gi = (int64_t)blockIdx.x * 4 + wv; gi < ngroups; gi += (int64_t)gridDim.x * 4) {
    const int64_t e0 = gi * 16, e = e0 + r, ec = e < E ? e : E - 1;  // rows past the end: computed, not stored
    const float* d = ds + ec * 3 * H;
    float v[16], dv[16];
    f4v acc[4];
    ld_row16(gh3 + ec * H, g, v);
    ld_row16(d + 2 * H, g, dv);
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] *= dv[q];
    ld_row16(d + H, g, dv);
    layer64(sw.w2T, v, acc);
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = acc[q >> 2][q & 3] * dv[q];
    ld_row16(d, g, dv);
    layer64(sw.w1T, v, acc);
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = acc[q >> 2][q & 3] * dv[q];
    f4v o = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float4 wq = sw.w0T[t][g][r];
#pragma unroll
      for (int i = 0; i < 4; ++i) o = mfma16(comp(wq, i), v[4 * t + i], o);
    }
    if (e < E) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = 4 * g + i;
        if (k < nb) {
          float* dst = gef + e * nb + k;
          *dst = accumulate ? *dst + o[i] : o[i];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Hidden layers on fp16 matrix cores with split operands (float32 policy).
//
// Same register layout as the fp32 kernels (lane (g, r) holds edge r's features
// n = 16t + 4g + i as v[4t + i]); v_mfma_f32_16x16x32_f16 takes eight k per lane,
// so a 64-wide layer is two chunks c, lane group g supplying in chunk c the eight
// values of tiles t = 2c, 2c + 1:
//   slot (c, g, j) <-> k = kperm2(c, g, j) = 16 (2c + j/4) + 4g + j%4.
// Activations are scaled per edge and layer (largest magnitude of the edge's 64
// values into [2^14, 2^15), reduced over its four lanes) and split into fp16
// hi + lo; weights are split once per model with one power-of-two scale per
// matrix; three products per pair, fp32 accumulation (about 2^-22 relative per
// product).  The first layer contracts over the Bessel features, slot (g, j) <->
// k = 8g + j (zero past nb).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int kperm2(int c, int g, int j) { return 16 * (2 * c + (j >> 2)) + 4 * g + (j & 3); }

// split tile images, [.. ][hi, lo][lane] (lane = 16 g + r)
// NP planes: 2 (hi, lo) as built; 1 (hi) staged under a half-precision policy, whose rounded
// weights have zero lo planes (half the LDS, so more blocks per CU)
template <int NP>
struct MlpFwdXT {
  h8 w0[4][NP][64];     // [t'] A[n = 16t' + r][8g + j] = W0[8g + j][n]
  h8 w1[2][4][NP][64];  // [c][t'] A[n = 16t' + r][slot] = W1[kperm2(c, g, j)][n]
  h8 w2[2][4][NP][64];
};
template <int NP>
struct MlpBwdXT {
  h8 w2T[2][4][NP][64];  // [c][t'] A[k = 16t' + r][slot] = W2[k][kperm2(c, g, j)]
  h8 w1T[2][4][NP][64];
  h8 w0T[2][NP][64];     // [c] A[k = r][slot] = W0[r][kperm2(c, g, j)] (zero for r >= nb)
};
using MlpFwdX = MlpFwdXT<2>;
using MlpBwdX = MlpBwdXT<2>;

// stage the hi planes of a two-plane image (every member's innermost dimensions are [2][64])
template <class D, class S>
__device__ __forceinline__ void stage_hi(D& dst, const S* __restrict__ src) {
  static_assert(2 * sizeof(D) == sizeof(S), "a one-plane image of a two-plane one");
  constexpr int N = (int)(sizeof(D) / sizeof(h8));
  const h8* q = reinterpret_cast<const h8*>(src);
  h8* d = reinterpret_cast<h8*>(&dst);
  for (int i = threadIdx.x; i < N; i += blockDim.x) d[i] = q[(i >> 6) * 128 + (i & 63)];
}
// the image as a kernel keeps it in LDS: both planes, or the hi planes (NP = 1)
template <int NP, class D, class S>
__device__ __forceinline__ void stage_planes(D& dst, const S* __restrict__ src) {
  if constexpr (NP == 2)
    stage_copy(dst, src);
  else
    stage_hi(dst, src);
}

__device__ __forceinline__ void split_pair(float x, _Float16& hi, _Float16& lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}
// element j of the pair of vectors (hi, lo)
__device__ __forceinline__ void split_into(float x, h8& hi, h8& lo, int j) {
  const _Float16 a = (_Float16)x;
  hi[j] = a;
  lo[j] = (_Float16)(x - (float)a);
}

__global__ void __launch_bounds__(256) k_mlp_permute_x(int nb, const float* __restrict__ W0,
                                                       const float* __restrict__ W1, const float* __restrict__ W2,
                                                       float s0, float s1, float s2, MlpFwdX* __restrict__ fw,
                                                       MlpBwdX* __restrict__ bw) {
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4, q = threadIdx.x >> 6;  // q: one of 4 tiles
  for (int c = 0; c < 2; ++c) {
    h8 a[2][2], b[2][2];  // [forward W1, W2 | backward W2T, W1T][hi, lo]
    for (int j = 0; j < 8; ++j) {
      const int k = kperm2(c, g, j), n = 16 * q + r;
      split_into(W1[k * H + n] * s1, a[0][0], a[0][1], j);
      split_into(W2[k * H + n] * s2, a[1][0], a[1][1], j);
      split_into(W2[n * H + k] * s2, b[0][0], b[0][1], j);
      split_into(W1[n * H + k] * s1, b[1][0], b[1][1], j);
    }
    for (int pl = 0; pl < 2; ++pl) {
      fw->w1[c][q][pl][l] = a[0][pl];
      fw->w2[c][q][pl][l] = a[1][pl];
      bw->w2T[c][q][pl][l] = b[0][pl];
      bw->w1T[c][q][pl][l] = b[1][pl];
    }
    if (q == 0) {
      h8 t[2];
      for (int j = 0; j < 8; ++j) split_into(r < nb ? W0[r * H + kperm2(c, g, j)] * s0 : 0.f, t[0], t[1], j);
      bw->w0T[c][0][l] = t[0];
      bw->w0T[c][1][l] = t[1];
    }
  }
  h8 t[2];
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * g + j;
    split_into(k < nb ? W0[k * H + 16 * q + r] * s0 : 0.f, t[0], t[1], j);
  }
  fw->w0[q][0][l] = t[0];
  fw->w0[q][1][l] = t[1];
}

// per-edge scale of a lane's values: returns the scale, sets *inv = its inverse
template <int NV>
__device__ __forceinline__ float edge_scale(const float* v, float* inv) {
  float m = 0.f;
#pragma unroll
  for (int q = 0; q < NV; ++q) m = fmaxf(m, fabsf(v[q]));
  m = max4_rows(m);  // the four lanes of edge r
  // floor(log2 m) from the exponent field; zero / subnormal edges take -100 (finite scales)
  const int ex = max((int)((__float_as_uint(m) >> 23) & 0xff) - 127, -100);
  *inv = __uint_as_float((unsigned)(127 - 14 + ex) << 23);
  return __uint_as_float((unsigned)(127 + 14 - ex) << 23);
}

// The lane index, with OPQ through an empty asm statement: weight-fragment reads indexed by it
// stay inside the edge-group loops.  Hoisted out of the loop, the six layers' fragments of the
// recomputing VJP hold ~300 VGPRs and leave one wave per SIMD (measured: 29 -> 26 us per
// launch un-hoisted); the forward's three layers are faster hoisted (97 -> 240 VGPRs).
template <bool OPQ>
__device__ __forceinline__ int lane_opaque() {
  int l = threadIdx.x & 63;
  if constexpr (OPQ) asm volatile("" : "+v"(l));
  return l;
}

// one 64-wide layer from the lane's 16 values v (all four output tiles t'):
// acc[t'] = (A_t' x v) with A = tile image w[c][t'][hi, lo][lane], times winv.  ALO / XLO: the
// weights' / the inputs' lo planes may be nonzero; under a half-precision feature policy the
// rounded weights and activations have zero lo planes (an fp16 value, or a bf16 value, times a
// power of two is one fp16 value), so those products add exact zeros and are skipped
template <bool OPQ, bool ALO = true, bool XLO = true, int NP = 2>
__device__ __forceinline__ void layer64x(const h8 (*w)[4][NP][64], const float* v, float winv, f4v* acc) {
  static_assert(NP == 2 || !ALO, "the weights' lo planes are staged");
  const int l = lane_opaque<OPQ>();
  float inv;
  const float sc = edge_scale<16>(v, &inv);
  inv *= winv;
  f4v d[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) d[t] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    h8 xh, xl;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      _Float16 hi, lo;
      split_pair(v[4 * (2 * c + (j >> 2)) + (j & 3)] * sc, hi, lo);
      xh[j] = hi;
      xl[j] = lo;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const h8 wh = w[c][t][0][l];
      if constexpr (ALO) d[t] = mfma16h(w[c][t][NP - 1][l], xh, d[t]);
      if constexpr (XLO) d[t] = mfma16h(wh, xl, d[t]);
      d[t] = mfma16h(wh, xh, d[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = d[t] * inv;
}

// forward of the split kernels: first layer over the Bessel features, then two 64-wide
// layers, the activations between them rounded by mode RND (the feature policy); dsp as in
// hidden_fwd; leaves a1, a2, a3 (the VJP recomputes them this way, with the same
// instructions, instead of reading saved derivatives)
template <bool OPQ, int RND, int NP>
__device__ __forceinline__ void hidden_fwd_x(const MlpFwdXT<NP>& sw, const float* winv, int64_t E, int64_t e0, int nb,
                                             const float* __restrict__ ef, f4v* a1, f4v* a2, f4v* a3, float* dsp) {
  // half-precision policies: weights, features and activations are rounded values (zero lo
  // planes), so one product per operand pair
  constexpr bool FULL = RND == RND_NONE;
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t e = e0 + r;
  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * g + j;
    x[j] = (e < E && k < nb) ? ef[e * nb + k] : 0.f;
  }
  {
    float inv;
    const float sc = edge_scale<8>(x, &inv);
    inv *= winv[0];
    h8 xh, xl;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      _Float16 hi, lo;
      split_pair(x[j] * sc, hi, lo);
      xh[j] = hi;
      xl[j] = lo;
    }
    const int lo = lane_opaque<OPQ>();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const h8 wh = sw.w0[t][0][lo];
      f4v d = f4v{0.f, 0.f, 0.f, 0.f};
      if constexpr (FULL) {
        d = mfma16h(sw.w0[t][NP - 1][lo], xh, d);
        d = mfma16h(wh, xl, d);
      }
      d = mfma16h(wh, xh, d);
      a1[t] = d * inv;
    }
  }
  float v[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) v[q] = qh(silu(a1[q >> 2][q & 3]), RND);
  if (dsp) store_ds(dsp, a1);
  layer64x<OPQ, FULL, FULL, NP>(sw.w1, v, winv[1], a2);
#pragma unroll
  for (int q = 0; q < 16; ++q) v[q] = qh(silu(a2[q >> 2][q & 3]), RND);
  if (dsp) store_ds(dsp + H, a2);
  layer64x<OPQ, FULL, FULL, NP>(sw.w2, v, winv[2], a3);
  if (dsp) store_ds(dsp + 2 * H, a3);
}

struct MlpWinv {
  float w[3];
};

// waves per block of the split hidden-layer kernels (forward; recomputing VJP; measured: six-wave
// VJP blocks, three waves per SIMD, are slower than four-wave ones, 27.6 vs 25.9 us)
constexpr int kHidFwdWaves = 4;
constexpr int kHidBwdWaves = 4;

// h3 as split pairs [E][2][64] + h3inv (H3_SPLIT layout) and silu' saved in ds; under a
// half-precision feature policy (RND) the activations are rounded first (h3's lo plane is then 0)
template <int RND>
__global__ void __launch_bounds__(64 * kHidFwdWaves) k_mlp_hidden_x(int64_t E, int nb, const float* __restrict__ ef,
                                                      const MlpFwdX* __restrict__ tiles, MlpWinv wi,
                                                      _Float16* __restrict__ h3x, float* __restrict__ h3inv,
                                                      float* __restrict__ ds, int store_lo) {
  constexpr int NP = RND == RND_NONE ? 2 : 1;
  // a rounded h3's lo plane is zero: written only for readers of both planes
  const bool lo_out = RND == RND_NONE || store_lo;
  __shared__ MlpFwdXT<NP> sw;
  stage_planes<NP>(sw, tiles);
  __syncthreads();
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t ngroups = (E + 15) / 16;
  for (int64_t gi = (int64_t)blockIdx.x * kHidFwdWaves + wv; gi < ngroups; gi += (int64_t)gridDim.x * kHidFwdWaves) {
    const int64_t e0 = gi * 16, e = e0 + r;
    f4v a1[4], a2[4], a3[4];
    hidden_fwd_x<false, RND, NP>(sw, wi.w, E, e0, nb, ef, a1, a2, a3, (ds && e < E) ? ds + e * 3 * H + 4 * g : nullptr);
    float v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = qh(silu(a3[q >> 2][q & 3]), RND);
    float inv;
    const float sc = edge_scale<16>(v, &inv);
    if (e < E) {
      _Float16* dst = h3x + e * 2 * H;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        h4 hi, lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          _Float16 a, b;
          split_pair(v[4 * t + i] * sc, a, b);
          hi[i] = a;
          lo[i] = b;
        }
        *reinterpret_cast<h4*>(dst + 16 * t + 4 * g) = hi;
        if (lo_out) *reinterpret_cast<h4*>(dst + H + 16 * t + 4 * g) = lo;
      }
      if (g == 0) h3inv[e] = inv;
    }
  }
}

// gh3: np partials [np][E][64] (stride pstride floats), added in order.  RECOMP:
// silu'(a1..a3) from the forward layers recomputed from ef (tiles ftiles, rounding mode
// RND as the forward) instead of read from ds.
template <bool RECOMP, int NW, int RND>
__global__ void __launch_bounds__(64 * NW) k_mlp_hidden_bwd_x(int64_t E, int nb, const MlpFwdX* __restrict__ ftiles,
                                                          const MlpBwdX* __restrict__ tiles, MlpWinv wi,
                                                          const float* __restrict__ ef, const float* __restrict__ ds,
                                                          const float* __restrict__ gh3, int np, int64_t pstride,
                                                          float* __restrict__ gef, int accumulate) {
  constexpr int NP = RND == RND_NONE ? 2 : 1;
  __shared__ MlpBwdXT<NP> sw;
  __shared__ __align__(16) char swf_raw[RECOMP ? sizeof(MlpFwdXT<NP>) : 16];
  MlpFwdXT<NP>& swf = *reinterpret_cast<MlpFwdXT<NP>*>(swf_raw);
  stage_planes<NP>(sw, tiles);
  if constexpr (RECOMP) stage_planes<NP>(swf, ftiles);
  __syncthreads();
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t ngroups = (E + 15) / 16;
  for (int64_t gi = (int64_t)blockIdx.x * NW + wv; gi < ngroups; gi += (int64_t)gridDim.x * NW) {
    const int64_t e0 = gi * 16, e = e0 + r, ec = e < E ? e : E - 1;  // rows past the end: computed, not stored
    float v[16], dv[16];
    f4v acc[4];
    f4v a1[4], a2[4], a3[4];  // RECOMP: the pre-activations, rebuilt
    if constexpr (RECOMP) hidden_fwd_x<true, RND, NP>(swf, wi.w, E, e0, nb, ef, a1, a2, a3, nullptr);
    // silu' of layer k's pre-activations in the lane's layout (feature 16t + 4g + i -> [4t + i])
    auto dsl = [&](int k, float* out) {
      if constexpr (RECOMP) {
        const f4v* a = k == 0 ? a1 : k == 1 ? a2 : a3;
#pragma unroll
        for (int q = 0; q < 16; ++q) out[q] = dsilu(a[q >> 2][q & 3]);
      } else {
        ld_row16(ds + ec * 3 * H + k * H, g, out);
      }
    };
    ld_row16(gh3 + ec * H, g, v);
    for (int pp = 1; pp < np; ++pp) {
      ld_row16(gh3 + pp * pstride + ec * H, g, dv);
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] += dv[q];
    }
    dsl(2, dv);
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] *= dv[q];
    dsl(1, dv);
    // the gradients are float32 (lo planes nonzero); the weights' lo planes are zero under a
    // half-precision policy
    constexpr bool WLO = RND == RND_NONE;
    layer64x<RECOMP, WLO, true, NP>(sw.w2T, v, wi.w[2], acc);
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = acc[q >> 2][q & 3] * dv[q];
    dsl(0, dv);
    layer64x<RECOMP, WLO, true, NP>(sw.w1T, v, wi.w[1], acc);
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = acc[q >> 2][q & 3] * dv[q];
    // g_ef = g_a1 W0^T: one output tile (rows k < nb)
    float inv;
    const float sc = edge_scale<16>(v, &inv);
    inv *= wi.w[0];
    f4v o = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      h8 xh, xl;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        _Float16 hi, lo;
        split_pair(v[4 * (2 * c + (j >> 2)) + (j & 3)] * sc, hi, lo);
        xh[j] = hi;
        xl[j] = lo;
      }
      const int lo = lane_opaque<RECOMP>();
      const h8 wh = sw.w0T[c][0][lo];
      if constexpr (WLO) o = mfma16h(sw.w0T[c][NP - 1][lo], xh, o);
      o = mfma16h(wh, xl, o);
      o = mfma16h(wh, xh, o);
    }
    if (e < E) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = 4 * g + i;
        if (k < nb) {
          float* dst = gef + e * nb + k;
          *dst = accumulate ? *dst + o[i] * inv : o[i] * inv;
        }
      }
    }
  }
}

inline unsigned nblk(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }


// ---------------------------------------------------------------------------
// mh-1 non-linear interaction block: LayerNorm radial MLP and density MLP
// (blocks.py:735-807, radial.py:344-357) on fp32 matrix cores, 16 edges per
// wave in the register layout of the hidden-layer kernels above (lane (g, r)
// holds edge r's features n = 16t + 4g + i as v[4t + i]).
//   z1 = W0e^T ef + ts[species(sender)] + tt[species(receiver)]   (tt holds b1)
//   a_k = silu(LN(z_k) s_k + c_k),  z_{k+1} = W_k^T a_k + bias_k,  h3 = a_3
// A LayerNorm's statistics over an edge's 64 features: 16 values in each of its
// four lanes, summed locally, then over the lanes (sum4_rows); two passes (mean,
// then the centred second moment), eps 1e-5 (MLX's default).
// Density: zd = Wd0e^T ef + dts + dtt, ad = silu(LN(zd) sd + cd), x = wd1 . ad + bd1,
// dens = tanh(x^2) cut.
// ---------------------------------------------------------------------------
struct LnSmall {  // the small per-layer vectors, staged in LDS
  float ln[3][2][64];
  float bias[2][64];
  float dln[2][64];
  float dw1[68];
};

__device__ __forceinline__ void stage_small(LnSmall& S, const LnMlpParams& P) {
  for (int i = threadIdx.x; i < 384; i += blockDim.x) (&S.ln[0][0][0])[i] = P.ln[i];
  for (int i = threadIdx.x; i < 128; i += blockDim.x) {
    (&S.bias[0][0])[i] = P.bias[i];
    (&S.dln[0][0])[i] = P.dln[i];
  }
  for (int i = threadIdx.x; i < 65; i += blockDim.x) S.dw1[i] = P.dw1[i];
}

// the lane's 16 features of a per-species table row
__device__ __forceinline__ void add_row16(const float* __restrict__ row, int g, float* z) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float4 x = ld4(row + 16 * t + 4 * g);
    z[4 * t] += x.x, z[4 * t + 1] += x.y, z[4 * t + 2] += x.z, z[4 * t + 3] += x.w;
  }
}

// LayerNorm of an edge's features z (the lane's 16): xh = (z - mean) * rstd
__device__ __forceinline__ float ln_stats(const float* z, float* xh) {
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) s += z[q];
  const float mu = sum4_rows(s) * (1.f / 64.f);
  float v = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const float d = z[q] - mu;
    v = fmaf(d, d, v);
  }
  const float rstd = 1.f / sqrtf(sum4_rows(v) * (1.f / 64.f) + 1e-5f);
#pragma unroll
  for (int q = 0; q < 16; ++q) xh[q] = (z[q] - mu) * rstd;
  return rstd;
}

__device__ __forceinline__ int fidx(int q, int g) { return 16 * (q >> 2) + 4 * g + (q & 3); }

// the first layer's ef part: acc[t'] = W0^T ef for the lane's edge (w0 tile image)
__device__ __forceinline__ void first_layer(const float4 (*w0)[4][16], const float* __restrict__ ef, int64_t ec,
                                            int nb, f4v* acc, int lane) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f4v{0.f, 0.f, 0.f, 0.f};
  const int nst = (nb + 3) >> 2;
  for (int st = 0; st < nst; ++st) {
    const int k = 4 * st + g;
    const float x = k < nb ? ef[ec * nb + k] : 0.f;
    const float4 wv = w0[st][g][r];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = mfma16(comp(wv, t), x, acc[t]);
  }
}

// forward of one edge group, keeping what the VJP needs: xh[k] (normalised z of layer k),
// rstd[k], h3 = a_3; density: xhd, rstdd, x
struct LnFwdState {
  float xh[3][16];
  float rstd[3];
  float h3[16];
  float xhd[16];
  float rstdd, x;
};

// the two 64-wide hidden layers as split-fp16 tile images (the layout of MlpFwdX.w1 / w2, and of
// MlpBwdX.w2T / w1T for the VJP), one power-of-two scale per matrix (LnMlpParams.winv)
struct LnHidX {
  h8 a[2][2][4][2][64];  // [layer 1, 2 | VJP: layer 2^T, 1^T][c][t'][hi, lo][lane]
};

// SPLIT: the hidden layers on fp16 matrix cores with split operands (hx), else fp32 matrix cores
// (sw.w1 / w2); the first layer (K = num_bessel) stays on fp32 matrix cores either way
template <bool SPLIT>
__device__ __forceinline__ void ln_mlp_fwd(const float4 (*w0)[4][16], const MlpFwdW& sw, const LnHidX& hx,
                                           const float4 (*dw0)[4][16], const LnSmall& S,
                                           const LnMlpParams& P, const float* __restrict__ ef, int64_t ec, int nb,
                                           int zs, int zr, LnFwdState& F, int lane) {
  const int g = lane >> 4;
  f4v acc[4];
  float z[16], v[16];
  first_layer(w0, ef, ec, nb, acc, lane);
#pragma unroll
  for (int q = 0; q < 16; ++q) z[q] = acc[q >> 2][q & 3];
  add_row16(P.ts + (int64_t)zs * H, g, z);
  add_row16(P.tt + (int64_t)zr * H, g, z);
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    F.rstd[k] = ln_stats(z, F.xh[k]);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int n = fidx(q, g);
      v[q] = silu(fmaf(F.xh[k][q], S.ln[k][0][n], S.ln[k][1][n]));
    }
    if (k < 2) {
      if constexpr (SPLIT)
        layer64x<true>(hx.a[k], v, P.winv[k + 1], acc);  // layer k + 1's weights W_{k+1}
      else
        layer64(k == 0 ? sw.w1 : sw.w2, v, acc, lane);
#pragma unroll
      for (int q = 0; q < 16; ++q) z[q] = acc[q >> 2][q & 3] + S.bias[k][fidx(q, g)];
    }
  }
#pragma unroll
  for (int q = 0; q < 16; ++q) F.h3[q] = v[q];
  // density MLP
  first_layer(dw0, ef, ec, nb, acc, lane);
#pragma unroll
  for (int q = 0; q < 16; ++q) z[q] = acc[q >> 2][q & 3];
  add_row16(P.dts + (int64_t)zs * H, g, z);
  add_row16(P.dtt + (int64_t)zr * H, g, z);
  F.rstdd = ln_stats(z, F.xhd);
  float xs = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int n = fidx(q, g);
    xs = fmaf(silu(fmaf(F.xhd[q], S.dln[0][n], S.dln[1][n])), S.dw1[n], xs);
  }
  F.x = sum4_rows(xs) + S.dw1[64];
}

// hidden layers of the split path: layers 1, 2 of an MlpFwdX image (tx, forward) or layers 2^T,
// 1^T of an MlpBwdX image (VJP) into LDS
__device__ __forceinline__ void stage_hid(h8 (*dst)[2][4][2][64], const h8 (*l0)[4][2][64], const h8 (*l1)[4][2][64]) {
  constexpr int N = 2 * 4 * 2 * 64;
  for (int i = threadIdx.x; i < N; i += blockDim.x) {
    (&dst[0][0][0][0][0])[i] = (&l0[0][0][0][0])[i];
    (&dst[1][0][0][0][0])[i] = (&l1[0][0][0][0])[i];
  }
}

template <bool SPLIT>
__global__ void __launch_bounds__(256) k_rmlp_ln_fwd(int64_t E, int nb, const float* __restrict__ ef,
                                                     const float* __restrict__ cut, const int* __restrict__ sender,
                                                     const int* __restrict__ receiver,
                                                     const int* __restrict__ species, const MlpFwdW* __restrict__ tiles,
                                                     const MlpFwdX* __restrict__ tiles_x,
                                                     const MlpFwdW* __restrict__ dtiles, LnMlpParams P,
                                                     void* __restrict__ h3, float* __restrict__ h3inv,
                                                     float* __restrict__ dens, int half) {
  // SPLIT stages the first layer (fp32) and the split hidden images; else the fp32 tile image
  __shared__ __align__(16) char sw_raw[SPLIT ? 16 : sizeof(MlpFwdW)];
  __shared__ __align__(16) char hx_raw[SPLIT ? sizeof(LnHidX) : 16];
  __shared__ float4 sw0[SPLIT ? NB4 : 1][4][16];
  __shared__ float4 sdw0[NB4][4][16];
  __shared__ LnSmall S;
  MlpFwdW& sw = *reinterpret_cast<MlpFwdW*>(sw_raw);
  LnHidX& hx = *reinterpret_cast<LnHidX*>(hx_raw);
  if constexpr (SPLIT) {
    for (int i = threadIdx.x; i < NB4 * 4 * 16; i += blockDim.x) (&sw0[0][0][0])[i] = (&tiles->w0[0][0][0])[i];
    stage_hid(hx.a, tiles_x->w1, tiles_x->w2);
  } else {
    stage_copy(sw, tiles);
  }
  const float4 (*w0)[4][16] = SPLIT ? sw0 : sw.w0;
  for (int i = threadIdx.x; i < NB4 * 4 * 16; i += blockDim.x) (&sdw0[0][0][0])[i] = (&dtiles->w0[0][0][0])[i];
  stage_small(S, P);
  __syncthreads();
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t ngroups = (E + 15) / 16;
  for (int64_t gi = (int64_t)blockIdx.x * 4 + wv; gi < ngroups; gi += (int64_t)gridDim.x * 4) {
    const int64_t e = gi * 16 + r, ec = e < E ? e : E - 1;  // rows past the end: computed, not stored
    const int zs = species[sender[ec]], zr = species[receiver[ec]];
    // the lane index as a value the compiler cannot hoist: the LDS reads of weights and
    // LayerNorm vectors indexed by it stay inside the loop (hoisted, they hold ~400 registers)
    const int lo = lane_opaque<true>();
    LnFwdState F;
    ln_mlp_fwd<SPLIT>(w0, sw, hx, sdw0, S, P, ef, ec, nb, zs, zr, F, lo);
    // the stored activation under a half-precision policy (its split lo plane is then zero)
#pragma unroll
    for (int q = 0; q < 16; ++q) F.h3[q] = qh(F.h3[q], half);
    if (h3inv) {  // split pairs [E][2][64] with the row scale's inverse, as k_mlp_hidden_x writes them
      float inv;
      const float sc = edge_scale<16>(F.h3, &inv);
      if (e < E) {
        _Float16* dst = static_cast<_Float16*>(h3) + e * 2 * H;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          h4 hi, lo;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            _Float16 a, b;
            split_pair(F.h3[4 * t + i] * sc, a, b);
            hi[i] = a;
            lo[i] = b;
          }
          *reinterpret_cast<h4*>(dst + 16 * t + 4 * g) = hi;
          *reinterpret_cast<h4*>(dst + H + 16 * t + 4 * g) = lo;
        }
        if (g == 0) h3inv[e] = inv;
      }
    } else if (e < E) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        *reinterpret_cast<float4*>(static_cast<float*>(h3) + e * H + 16 * t + 4 * g) =
            float4{F.h3[4 * t], F.h3[4 * t + 1], F.h3[4 * t + 2], F.h3[4 * t + 3]};
    }
    if (e < E && g == 0) dens[e] = qh(tanhf(F.x * F.x) * (cut ? cut[e] : 1.f), half);
  }
}

// LayerNorm + SiLU VJP of one layer: dz from dL/da (g), in place
__device__ __forceinline__ void ln_silu_bwd(float* gv, const float* xh, float rstd, const float* sc, const float* sh,
                                            int g) {
  float dxh[16], s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int n = fidx(q, g);
    const float y = fmaf(xh[q], sc[n], sh[n]);
    dxh[q] = gv[q] * dsilu(y) * sc[n];
    s1 += dxh[q];
    s2 = fmaf(dxh[q], xh[q], s2);
  }
  s1 = sum4_rows(s1) * (1.f / 64.f);
  s2 = sum4_rows(s2) * (1.f / 64.f);
#pragma unroll
  for (int q = 0; q < 16; ++q) gv[q] = rstd * (dxh[q] - s1 - xh[q] * s2);
}

// gef contributions of a first layer: o[i] = sum_n W0[k = 4g + i][n] dz[n] (w0T tile image)
__device__ __forceinline__ void first_layer_T(const float4 (*w0T)[4][16], const float* dz, f4v& o, int lane) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float4 wq = w0T[t][g][r];
#pragma unroll
    for (int i = 0; i < 4; ++i) o = mfma16(comp(wq, i), dz[4 * t + i], o);
  }
}

// waves per block of the LayerNorm VJP: its staged weights (85 KB) fit once per CU, so two
// waves per SIMD come from one eight-wave block
constexpr int kLnBwdWaves = 8;

template <bool SPLIT>
__global__ void __launch_bounds__(64 * kLnBwdWaves) k_rmlp_ln_bwd(int64_t E, int nb, const float* __restrict__ ef,
                                                     const float* __restrict__ cut, const int* __restrict__ sender,
                                                     const int* __restrict__ receiver,
                                                     const int* __restrict__ species, const MlpFwdW* __restrict__ tiles,
                                                     const MlpBwdW* __restrict__ btiles,
                                                     const MlpFwdX* __restrict__ tiles_x,
                                                     const MlpBwdX* __restrict__ btiles_x,
                                                     const MlpFwdW* __restrict__ dtiles,
                                                     const MlpBwdW* __restrict__ dbtiles, LnMlpParams P,
                                                     const float* __restrict__ G, const float* __restrict__ gwb,
                                                     int np, const float* __restrict__ drho,
                                                     float* __restrict__ gef, float* __restrict__ gcut,
                                                     int accumulate) {
  // SPLIT: the first layers (fp32) and the split images of the hidden layers (forward and
  // transposed); else the fp32 tile images
  __shared__ __align__(16) char sw_raw[SPLIT ? 16 : sizeof(MlpFwdW)];
  __shared__ __align__(16) char sb_raw[SPLIT ? 16 : sizeof(MlpBwdW)];
  __shared__ __align__(16) char hx_raw[SPLIT ? sizeof(LnHidX) : 16];
  __shared__ __align__(16) char hb_raw[SPLIT ? sizeof(LnHidX) : 16];
  __shared__ float4 sw0[SPLIT ? NB4 : 1][4][16];
  __shared__ float4 sw0T[SPLIT ? 4 : 1][4][16];
  __shared__ float4 sdw0[NB4][4][16];
  __shared__ float4 sdw0T[4][4][16];
  __shared__ LnSmall S;
  MlpFwdW& sw = *reinterpret_cast<MlpFwdW*>(sw_raw);
  MlpBwdW& sb = *reinterpret_cast<MlpBwdW*>(sb_raw);
  LnHidX& hx = *reinterpret_cast<LnHidX*>(hx_raw);
  LnHidX& hb = *reinterpret_cast<LnHidX*>(hb_raw);
  if constexpr (SPLIT) {
    for (int i = threadIdx.x; i < NB4 * 4 * 16; i += blockDim.x) (&sw0[0][0][0])[i] = (&tiles->w0[0][0][0])[i];
    for (int i = threadIdx.x; i < 4 * 4 * 16; i += blockDim.x) (&sw0T[0][0][0])[i] = (&btiles->w0T[0][0][0])[i];
    stage_hid(hx.a, tiles_x->w1, tiles_x->w2);
    stage_hid(hb.a, btiles_x->w2T, btiles_x->w1T);
  } else {
    stage_copy(sw, tiles);
    stage_copy(sb, btiles);
  }
  const float4 (*w0)[4][16] = SPLIT ? sw0 : sw.w0;
  const float4 (*w0T)[4][16] = SPLIT ? sw0T : sb.w0T;
  for (int i = threadIdx.x; i < NB4 * 4 * 16; i += blockDim.x) (&sdw0[0][0][0])[i] = (&dtiles->w0[0][0][0])[i];
  for (int i = threadIdx.x; i < 4 * 4 * 16; i += blockDim.x) (&sdw0T[0][0][0])[i] = (&dbtiles->w0T[0][0][0])[i];
  stage_small(S, P);
  __syncthreads();
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int64_t ngroups = (E + 15) / 16;
  for (int64_t gi = (int64_t)blockIdx.x * kLnBwdWaves + wv; gi < ngroups; gi += (int64_t)gridDim.x * kLnBwdWaves) {
    const int64_t e = gi * 16 + r, ec = e < E ? e : E - 1;
    const int rcv = receiver[ec];
    const int zs = species[sender[ec]], zr = species[rcv];
    const int lo = lane_opaque<true>(), go = lo >> 4;  // as in k_rmlp_ln_fwd
    LnFwdState F;
    ln_mlp_fwd<SPLIT>(w0, sw, hx, sdw0, S, P, ef, ec, nb, zs, zr, F, lo);
    const float ce = cut ? cut[ec] : 1.f;
    float gv[16], gb = gwb[ec];
    ld_row16(G + ec * H, g, gv);
    for (int k = 1; k < np; ++k) {  // partials added in order
      float t[16];
      ld_row16(G + (k * E + ec) * H, g, t);
#pragma unroll
      for (int q = 0; q < 16; ++q) gv[q] += t[q];
      gb += gwb[k * E + ec];
    }
    // w = cut (h3 W3 + b3): dL/dcut = h3 . G + gw . b3, dL/dh3 = cut G
    float hg = 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) hg = fmaf(F.h3[q], gv[q], hg);
    float gc = sum4_rows(hg) + gb;
#pragma unroll
    for (int q = 0; q < 16; ++q) gv[q] *= ce;
    f4v acc[4];
#pragma unroll
    for (int k = 2; k >= 0; --k) {
      ln_silu_bwd(gv, F.xh[k], F.rstd[k], S.ln[k][0], S.ln[k][1], go);
      if (k > 0) {
        if constexpr (SPLIT)
          layer64x<true>(hb.a[2 - k], gv, P.winv[k], acc);  // layer k's transpose: image 2 - k
        else
          layer64(k == 2 ? sb.w2T : sb.w1T, gv, acc, lo);
#pragma unroll
        for (int q = 0; q < 16; ++q) gv[q] = acc[q >> 2][q & 3];
      }
    }
    f4v o = f4v{0.f, 0.f, 0.f, 0.f};
    first_layer_T(w0T, gv, o, lo);
    // density: dens = tanh(x^2) cut, rho[receiver] = sum of dens
    const float th = tanhf(F.x * F.x);
    const float gd = drho[rcv];
    gc = fmaf(gd, th, gc);
    const float gx = gd * ce * (1.f - th * th) * 2.f * F.x;
#pragma unroll
    for (int q = 0; q < 16; ++q) gv[q] = gx * S.dw1[fidx(q, go)];
    ln_silu_bwd(gv, F.xhd, F.rstdd, S.dln[0], S.dln[1], go);
    first_layer_T(sdw0T, gv, o, lo);
    if (e < E) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = 4 * g + i;
        if (k < nb) {
          float* dst = gef + e * nb + k;
          *dst = accumulate ? *dst + o[i] : o[i];
        }
      }
      if (gcut && g == 0) gcut[e] = accumulate ? gcut[e] + gc : gc;
    }
  }
}
}  // namespace

// grid of the hidden-layer kernels: enough blocks to fill the device, each
// staging the weights once and walking several 64-edge groups
// persistent grids, each wave walking 16-edge groups: two blocks per CU for the forward (three
// fit under the half policies; measured slower: 0.345 -> 0.352 ms per launch on HEA32000)
inline unsigned hidden_grid(int64_t E) {
  return (unsigned)std::min<int64_t>((E + 16 * kHidFwdWaves - 1) / (16 * kHidFwdWaves), 512);
}
// the recomputing VJP stages both tile images (76 KB; 38 KB under the half policies, hi planes
// only): as many blocks as fit at once, two per CU, or three under the half policies
inline unsigned hidden_bwd_grid(int64_t E, int rnd) {
  return (unsigned)std::min<int64_t>((E + 16 * kHidBwdWaves - 1) / (16 * kHidBwdWaves), rnd == RND_NONE ? 512 : 768);
}

size_t mlp_tile_bytes() { return sizeof(MlpFwdW) + sizeof(MlpBwdW); }
size_t mlp_tile_x_bytes() { return sizeof(MlpFwdX) + sizeof(MlpBwdX); }

void launch_mlp_permute_x(hipStream_t st, int nb, const float* W0, const float* W1, const float* W2,
                          const float* scale3, void* tiles) {
  MlpFwdX* fw = static_cast<MlpFwdX*>(tiles);
  MlpBwdX* bw = reinterpret_cast<MlpBwdX*>(static_cast<char*>(tiles) + sizeof(MlpFwdX));
  MACE_LAUNCH(k_mlp_permute_x, dim3(1), dim3(256), 0, st, nb, W0, W1, W2, scale3[0], scale3[1], scale3[2],
                     fw, bw);
}

void launch_mlp_hidden_x(hipStream_t st, int64_t E, int nb, const float* ef, const void* tiles,
                         const float* winv3, void* h3x, float* h3inv, float* ds, int rnd, int store_lo) {
  if (E <= 0) return;
  MlpWinv wi{{winv3[0], winv3[1], winv3[2]}};
#define MACE_HX(R)                                                                                 \
  MACE_LAUNCH(k_mlp_hidden_x<R>, dim3(hidden_grid(E)), dim3(64 * kHidFwdWaves), 0, st, E, nb, ef, \
              static_cast<const MlpFwdX*>(tiles), wi, static_cast<_Float16*>(h3x), h3inv, ds, store_lo)
  if (rnd == RND_F16)
    MACE_HX(RND_F16);
  else if (rnd == RND_BF16)
    MACE_HX(RND_BF16);
  else
    MACE_HX(RND_NONE);
#undef MACE_HX
}

void launch_mlp_hidden_bwd_x(hipStream_t st, int64_t E, int nb, const void* tiles, const float* winv3,
                             const float* ef, const float* ds, const float* gh3, int np, float* gef, int accumulate,
                             int rnd) {
  if (E <= 0) return;
  MlpWinv wi{{winv3[0], winv3[1], winv3[2]}};
  const MlpFwdX* fw = static_cast<const MlpFwdX*>(tiles);
  const MlpBwdX* bw = reinterpret_cast<const MlpBwdX*>(static_cast<const char*>(tiles) + sizeof(MlpFwdX));
  if (ds) {
    MACE_LAUNCH((k_mlp_hidden_bwd_x<false, 4, RND_NONE>), dim3(hidden_grid(E)), dim3(256), 0, st, E, nb, fw, bw, wi,
                ef, ds, gh3, np, E * H, gef, accumulate);
    return;
  }
#define MACE_HBX(R)                                                                                              \
  MACE_LAUNCH((k_mlp_hidden_bwd_x<true, kHidBwdWaves, R>), dim3(hidden_bwd_grid(E, R)), dim3(64 * kHidBwdWaves), 0, \
              st, E, nb, fw, bw, wi, ef, ds, gh3, np, E * H, gef, accumulate)
  if (rnd == RND_F16)
    MACE_HBX(RND_F16);
  else if (rnd == RND_BF16)
    MACE_HBX(RND_BF16);
  else
    MACE_HBX(RND_NONE);
#undef MACE_HBX
}

void launch_mlp_permute(hipStream_t st, int nb, const float* W0, const float* W1, const float* W2, void* tiles) {
  MlpFwdW* fw = static_cast<MlpFwdW*>(tiles);
  MlpBwdW* bw = reinterpret_cast<MlpBwdW*>(static_cast<char*>(tiles) + sizeof(MlpFwdW));
  MACE_LAUNCH(k_mlp_permute, dim3(1), dim3(256), 0, st, nb, W0, W1, W2, fw, bw);
}

void launch_mlp_hidden(hipStream_t st, int64_t E, int nb, const float* ef, const void* tiles, void* h3,
                       float* h3inv, float* ds, int mode) {
  if (E <= 0) return;
  const dim3 grid(hidden_grid(E)), blk(256);
  const MlpFwdW* fw = static_cast<const MlpFwdW*>(tiles);
  if (mode == H3_SPLIT)
    MACE_LAUNCH(k_mlp_hidden<H3_SPLIT>, grid, blk, 0, st, E, nb, ef, fw, h3, h3inv, ds);
  else if (mode == H3_F16)
    MACE_LAUNCH(k_mlp_hidden<H3_F16>, grid, blk, 0, st, E, nb, ef, fw, h3, h3inv, ds);
  else if (mode == H3_BF16)
    MACE_LAUNCH(k_mlp_hidden<H3_BF16>, grid, blk, 0, st, E, nb, ef, fw, h3, h3inv, ds);
  else
    MACE_LAUNCH(k_mlp_hidden<H3_F32>, grid, blk, 0, st, E, nb, ef, fw, h3, h3inv, ds);
}

void launch_mlp_out(hipStream_t st, int64_t E, int W, const void* h3, const void* W3T, void* w, int rnd,
                    const float* bias, const float* rs) {
  if (E <= 0) return;
  if (rnd == RND_F16)
    MACE_LAUNCH(k_mlp_out_h, dim3(nblk(E, 64), 2), dim3(256), 0, st, E, W, static_cast<const _Float16*>(h3),
                       static_cast<const _Float16*>(W3T), static_cast<_Float16*>(w));
  else
    MACE_LAUNCH(k_mlp_out, dim3(nblk(E, 64), 2), dim3(256), 0, st, E, W, static_cast<const float*>(h3),
                       static_cast<const float*>(W3T), static_cast<float*>(w), bias, rs, rnd);
}

void launch_mlp_out_x(hipStream_t st, int64_t E, int W, const void* h3x, const float* h3inv, const void* W3Tx,
                      float cscale, float* w, const float* bias, const float* rs) {
  if (E <= 0) return;
  MACE_LAUNCH(k_mlp_out_x, dim3(nblk(E, 64), 2), dim3(256), 0, st, E, W, static_cast<const _Float16*>(h3x),
                     h3inv, static_cast<const _Float16*>(W3Tx), cscale, w, bias, rs);
}

void launch_mlp_gh3(hipStream_t st, int64_t E, int W, const float* gw, const float* W3, float* gh3,
                    const float* b3, float* gwb) {
  if (E <= 0) return;
  MACE_LAUNCH(k_mlp_gh3, dim3(nblk(E, 32)), dim3(256), 0, st, E, W, gw, W3, gh3, b3, gwb);
}

void launch_mlp_gh3_x(hipStream_t st, int64_t E, int W, const float* gw, const void* W3x, float cscale,
                      float* gh3, const float* b3, float* gwb) {
  if (E <= 0) return;
  MACE_LAUNCH(k_mlp_gh3_x, dim3(nblk(E, 64)), dim3(256), 0, st, E, W, gw,
                     static_cast<const _Float16*>(W3x), cscale, gh3, b3, gwb);
}

void launch_mlp_gh3_h(hipStream_t st, int64_t E, int W, const void* gw, const float* gscale, const void* W3h,
                      float* gh3) {
  if (E <= 0) return;
  MACE_LAUNCH(k_mlp_gh3_h, dim3(nblk(E, 32)), dim3(256), 0, st, E, W, static_cast<const _Float16*>(gw),
                     gscale, static_cast<const _Float16*>(W3h), gh3);
}

void launch_mlp_hidden_bwd(hipStream_t st, int64_t E, int nb, const void* tiles, const float* ds, const float* gh3,
                           float* gef, int accumulate) {
  if (E <= 0) return;
  const MlpBwdW* bw = reinterpret_cast<const MlpBwdW*>(static_cast<const char*>(tiles) + sizeof(MlpFwdW));
  MACE_LAUNCH(k_mlp_hidden_bwd, dim3(hidden_grid(E)), dim3(256), 0, st, E, nb, bw, ds, gh3, gef, accumulate);
}

size_t mlp_tile_fwd_bytes() { return sizeof(MlpFwdW); }
size_t mlp_tile_x_fwd_bytes() { return sizeof(MlpFwdX); }

void launch_rmlp_ln_fwd(hipStream_t st, int64_t E, int nb, const float* ef, const float* cut, const int* sender,
                        const int* receiver, const int* species, const void* tiles, const void* tiles_x,
                        const void* dtiles, const LnMlpParams& P, void* h3, float* h3inv, float* dens, int half) {
  if (E <= 0) return;
  // one 16-edge group per wave up to three blocks per CU (44 / 46 KB of LDS each)
  const unsigned grid = (unsigned)std::min<int64_t>((E + 63) / 64, 768);
  const MlpFwdX* tx = static_cast<const MlpFwdX*>(tiles_x);
#define MACE_LNF(SP)                                                                                            \
  MACE_LAUNCH(k_rmlp_ln_fwd<SP>, dim3(grid), dim3(256), 0, st, E, nb, ef, cut, sender, receiver, species,        \
              static_cast<const MlpFwdW*>(tiles), tx, static_cast<const MlpFwdW*>(dtiles), P, h3, h3inv, dens, half)
  if (tx)
    MACE_LNF(true);
  else
    MACE_LNF(false);
#undef MACE_LNF
}

void launch_rmlp_ln_bwd(hipStream_t st, int64_t E, int nb, const float* ef, const float* cut, const int* sender,
                        const int* receiver, const int* species, const void* tiles, const void* btiles,
                        const void* tiles_x, const void* btiles_x, const void* dtiles, const void* dbtiles,
                        const LnMlpParams& P, const float* G, const float* gwb, int np, const float* drho, float* gef,
                        float* gcut, int accumulate) {
  if (E <= 0) return;
  const unsigned grid = (unsigned)std::min<int64_t>((E + 16 * kLnBwdWaves - 1) / (16 * kLnBwdWaves), 256);
  const MlpFwdX* tx = static_cast<const MlpFwdX*>(tiles_x);
  const MlpBwdX* bx = static_cast<const MlpBwdX*>(btiles_x);
#define MACE_LNB(SP)                                                                                             \
  MACE_LAUNCH(k_rmlp_ln_bwd<SP>, dim3(grid), dim3(64 * kLnBwdWaves), 0, st, E, nb, ef, cut, sender, receiver,   \
              species, static_cast<const MlpFwdW*>(tiles), static_cast<const MlpBwdW*>(btiles), tx, bx,          \
              static_cast<const MlpFwdW*>(dtiles), static_cast<const MlpBwdW*>(dbtiles), P, G, gwb, np, drho, gef, \
              gcut, accumulate)
  if (tx)
    MACE_LNB(true);
  else
    MACE_LNB(false);
#undef MACE_LNB
}

}  // namespace mace
