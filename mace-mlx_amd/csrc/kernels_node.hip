// Node-parallel kernels: grouped products on matrix cores (irrep-wise linears, the
// per-species skip connections over species-sorted rows), node embedding, symmetric
// contraction (+VJP), readouts, energy assembly and the deterministic force / virial
// reductions.
#include <hip/hip_runtime.h>

#include "common.h"

namespace mace {
namespace {

// ---------------------------------------------------------------------------
// grouped GEMM on fp32 matrix cores (v_mfma_f32_16x16x4f32; lane l holds
// A[l%16][k], B[k][l%16], D[4(l/16)+i][l%16]; within a 16-wide k chunk lane
// group g = l/16 takes k = 16c + 4g + s at step s, so A and B^T rows give one
// float4 per lane and chunk).
//
// A block is 4 waves; each wave computes a 16 x (16 CT) output tile (CT = 1:
// block = 16 rows x 64 columns; CT = 4: block = 32 rows x 128 columns).  The K dimension (operand 1, then operand 2) is consumed in batches
// of KB 16-wide chunks whose loads are all in flight together; with DB the
// next batch is loaded while the current one is multiplied.  Small groups
// (few row tiles) use CT = 1 for parallelism, large ones CT = 4 so that each
// A fragment feeds four column tiles.
// ---------------------------------------------------------------------------
typedef float f4v __attribute__((ext_vector_type(4)));

struct GemmChunkSrc {
  const float* xrow1;  // row n, block m of operand 1
  const float* xrow2;
  const float* wt1;    // B^T row of the first output column of operand 1
  const float* wt2;
  int K1, K2, stride1, stride2;
};

template <int CT>
__device__ __forceinline__ void gemm_load_chunk(const GemmChunkSrc& S, int ci, int g, float4& a, float4* b) {
  int k = ci * 16;
  const bool first = k < S.K1;
  if (!first) k -= S.K1;
  const float* xr = first ? S.xrow1 : S.xrow2;
  const int st = first ? S.stride1 : S.stride2, K = first ? S.K1 : S.K2;
  const float* wr = first ? S.wt1 : S.wt2;
  a = *reinterpret_cast<const float4*>(xr + (k / NC) * st + (k % NC) + 4 * g);
#pragma unroll
  for (int t = 0; t < CT; ++t) b[t] = *reinterpret_cast<const float4*>(wr + (int64_t)16 * t * K + k + 4 * g);
}

template <int CT, int KB, bool DB>
__global__ void __launch_bounds__(256) k_gemm_group(GemmGroup G) {
  int q = 0;
  while (q + 1 < G.n && (int)blockIdx.x >= G.p[q + 1].tile_begin) ++q;
  const GemmProb& P = G.p[q];
  const int t = blockIdx.x - P.tile_begin;
  constexpr int WROWS = CT == 4 ? 2 : 1, WCOLS = 4 / WROWS;  // waves per block along rows / columns
  const int tm = t / P.tiles_n, tn = t % P.tiles_n;
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int rt = tm * WROWS + wv / WCOLS;  // this wave's 16-row tile
  const int col0 = tn * (WCOLS * 16 * CT) + (wv % WCOLS) * 16 * CT;
  const int row = rt * 16 + r;
  const bool live = row < P.rows;
  const int nl = live ? row / P.d : 0, m = live ? row - nl * P.d : 0;  // dead rows read row 0, store nothing
  const int n = P.rowmap ? P.rowmap[nl] : nl;
  GemmChunkSrc S;
  S.xrow1 = P.X1 + (int64_t)n * P.ldx1 + P.in_base1 + m * NC;
  S.xrow2 = P.K2 > 0 ? P.X2 + (int64_t)n * P.ldx2 + P.in_base2 + m * NC : S.xrow1;
  S.wt1 = P.WT1 + (int64_t)(col0 + r) * P.K1;
  S.wt2 = P.K2 > 0 ? P.WT2 + (int64_t)(col0 + r) * P.K2 : S.wt1;
  S.K1 = P.K1;
  S.K2 = P.K2;
  S.stride1 = P.in_stride1;
  S.stride2 = P.in_stride2;
  const int nch = (P.K1 + P.K2) / 16;
  f4v acc[CT];
#pragma unroll
  for (int u = 0; u < CT; ++u) acc[u] = f4v{0.f, 0.f, 0.f, 0.f};
  float4 a[KB], b[KB][CT], an[DB ? KB : 1], bn[DB ? KB : 1][CT];
  if (DB) {
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (j < nch) gemm_load_chunk<CT>(S, j, g, a[j], b[j]);
  }
  for (int c0 = 0; c0 < nch; c0 += KB) {
    if (DB) {
#pragma unroll
      for (int j = 0; j < KB; ++j)
        if (c0 + KB + j < nch) gemm_load_chunk<CT>(S, c0 + KB + j, g, an[DB ? j : 0], bn[DB ? j : 0]);
    } else {
#pragma unroll
      for (int j = 0; j < KB; ++j)
        if (c0 + j < nch) gemm_load_chunk<CT>(S, c0 + j, g, a[j], b[j]);
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads of the batch issued before the multiplies
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (c0 + j < nch) {
        const float av[4] = {a[j].x, a[j].y, a[j].z, a[j].w};
#pragma unroll
        for (int u = 0; u < CT; ++u) {
          const float bv[4] = {b[j][u].x, b[j][u].y, b[j][u].z, b[j][u].w};
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s2], bv[s2], acc[u], 0, 0, 0);
        }
      }
    }
    if (DB) {
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        a[j] = an[DB ? j : 0];
#pragma unroll
        for (int u = 0; u < CT; ++u) b[j][u] = bn[DB ? j : 0][u];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < CT; ++u) {
    const int col = col0 + 16 * u + r;
    const float bias = P.bias ? P.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ro = rt * 16 + 4 * g + i;
      if (ro >= P.rows) continue;
      const int nlo = ro / P.d, mo = ro - nlo * P.d;
      const int no = P.rowmap ? P.rowmap[nlo] : nlo;
      float* y = P.Y + (int64_t)no * P.ldy + P.out_base + (col / NC) * P.out_stride + mo * NC + (col % NC);
      const float v = acc[u][i] * (P.rowscale ? P.rowscale[no] : 1.f) + bias;
      *y = qh(P.accumulate ? *y + v : v, G.round_half);
    }
  }
}

// Float32 policy on fp16 matrix cores: the grouped products of k_gemm_group with
// both operands split into fp16 pairs (a = a_hi + a_lo, three products per pair,
// fp32 accumulation; about 2^-22 relative per product).  Roles are swapped: A =
// weight rows (output columns), B = X^T with a tile's 16 rows as columns, so lane
// (g, r) owns row r's eight k values of a 32-wide chunk and the accumulators of
// that row: it scales the values by the power of two that maps their chunk's
// largest magnitude (reduced over the row's four lanes) into [2^14, 2^15), splits
// them and folds the inverse scale (times the weights' own, winv) into the
// accumulators after the chunk.  Weights come as [hi | lo] planes WX [Cout][K]
// scaled by 1 / winv.  Block = 64 rows x 64 output columns (wave = one 16-row
// tile x the 64 columns); the block stages each chunk of its 64 weight rows in
// LDS, double-buffered, and the X chunks are loaded two ahead.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4v mfma16h(h8 a, h8 b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

struct GemmXSrc {
  const float* xr[2];     // row n, component m of operands 1 and 2
  const _Float16* w[2];   // hi plane row of the staging thread's column
  int K1, stride[2], K[2];
  float winv[2];
};

// this lane's eight X values of chunk ci (k = 32 ci + 8 g ...)
__device__ __forceinline__ void gx_load_x(const GemmXSrc& S, int ci, int g, float4& x0, float4& x1) {
  int k = 32 * ci;
  const int o = k < S.K1 ? 0 : 1;
  if (o) k -= S.K1;
  const float* p = S.xr[o] + (k / NC) * S.stride[o] + (k % NC) + 8 * g;
  x0 = *reinterpret_cast<const float4*>(p);
  x1 = *reinterpret_cast<const float4*>(p + 4);
}

// CW: 16-column tiles per wave (4: blocks of 64 columns; 8: of 128, so that a row block's X is read
// by half as many blocks when every problem's output width is a multiple of 128)
template <int CW>
__global__ void __launch_bounds__(256) k_gemm_group_x(GemmGroup G) {
  constexpr int BC = 16 * CW;                          // output columns per block
  constexpr int SPT = 256 / BC, SEG = 32 / SPT, NH = SEG / 8;  // staging: threads per column, k each, h8 each
  __shared__ __align__(16) _Float16 sW[2][2][BC][40];  // [buffer][hi, lo][column][k of the chunk + pad]
  int q = 0;
  while (q + 1 < G.n && (int)blockIdx.x >= G.p[q + 1].tile_begin) ++q;
  const GemmProb& P = G.p[q];
  const int t = blockIdx.x - P.tile_begin;
  const int tm = t / P.tiles_n, tn = t % P.tiles_n;
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int rt = tm * 4 + wv;
  const int row = rt * 16 + r;
  const bool live = row < P.rows;
  const int nl = live ? row / P.d : 0, m = live ? row - nl * P.d : 0;  // dead rows read row 0, store nothing
  const int n = P.rowmap ? P.rowmap[nl] : nl;
  GemmXSrc S;
  S.K1 = P.K1;
  S.K[0] = P.K1;
  S.K[1] = P.K2;
  S.stride[0] = P.in_stride1;
  S.stride[1] = P.in_stride2;
  S.xr[0] = P.X1 + (int64_t)n * P.ldx1 + P.in_base1 + m * NC;
  S.xr[1] = P.K2 > 0 ? P.X2 + (int64_t)n * P.ldx2 + P.in_base2 + m * NC : S.xr[0];
  S.winv[0] = P.winv1;
  S.winv[1] = P.winv2;
  // staging: thread -> column tn * BC + tid / SPT, SEG k at SEG (tid % SPT), both planes
  const int scol = threadIdx.x / SPT, kq = SEG * (threadIdx.x % SPT);
  S.w[0] = P.WX1 + (int64_t)(tn * BC + scol) * P.K1;
  S.w[1] = P.K2 > 0 ? P.WX2 + (int64_t)(tn * BC + scol) * P.K2 : S.w[0];
  const int64_t plane[2] = {(int64_t)P.Cout * P.K1, (int64_t)P.Cout * P.K2};
  const int nch = (P.K1 + P.K2) / 32;
  float4 ring[2][2];
  gx_load_x(S, 0, g, ring[0][0], ring[0][1]);
  gx_load_x(S, min(1, nch - 1), g, ring[1][0], ring[1][1]);
  auto load_w = [&](int ci, h8 (*w)[NH]) {  // this thread's SEG values of chunk ci, hi and lo
    int k = 32 * ci;
    const int o = k < S.K1 ? 0 : 1;
    if (o) k -= S.K1;
#pragma unroll
    for (int i = 0; i < NH; ++i) {
      w[0][i] = *reinterpret_cast<const h8*>(S.w[o] + k + kq + 8 * i);
      w[1][i] = *reinterpret_cast<const h8*>(S.w[o] + plane[o] + k + kq + 8 * i);
    }
  };
  auto stage_w = [&](int buf, h8 (*w)[NH]) {
#pragma unroll
    for (int pl = 0; pl < 2; ++pl)
#pragma unroll
      for (int i = 0; i < NH; ++i) *reinterpret_cast<h8*>(&sW[buf][pl][scol][kq + 8 * i]) = w[pl][i];
  };
  h8 ws[2][NH];
  load_w(0, ws);
  stage_w(0, ws);
  __syncthreads();
  f4v acc[CW];
#pragma unroll
  for (int u = 0; u < CW; ++u) acc[u] = f4v{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nch; c0 += 2) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int cc = c0 + p;
      if (cc < nch) {  // uniform over the block
        const int buf = cc & 1;
        if (cc + 1 < nch) load_w(cc + 1, ws);
        const float4 c0v = ring[p][0], c1v = ring[p][1];
        gx_load_x(S, min(cc + 2, nch - 1), g, ring[p][0], ring[p][1]);
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the arithmetic
        const float v[8] = {c0v.x, c0v.y, c0v.z, c0v.w, c1v.x, c1v.y, c1v.z, c1v.w};
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
        mx = max4_rows(mx);  // the four lanes of row r
        // floor(log2 mx) from the exponent field; zero / subnormal chunks take -100 (finite scales)
        const int ex = max((int)((__float_as_uint(mx) >> 23) & 0xff) - 127, -100);
        const float sc = __uint_as_float((unsigned)(127 + 14 - ex) << 23);
        const float inv = __uint_as_float((unsigned)(127 - 14 + ex) << 23) * S.winv[32 * cc < S.K1 ? 0 : 1];
        h8 xh, xl;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = v[j] * sc;
          const _Float16 hi = (_Float16)x;
          xh[j] = hi;
          xl[j] = (_Float16)(x - (float)hi);
        }
#pragma unroll
        for (int u = 0; u < CW; ++u) {
          const int col = 16 * u + r;
          const h8 wh = *reinterpret_cast<const h8*>(&sW[buf][0][col][8 * g]);
          const h8 wl = *reinterpret_cast<const h8*>(&sW[buf][1][col][8 * g]);
          f4v d = mfma16h(wl, xh, f4v{0.f, 0.f, 0.f, 0.f});
          d = mfma16h(wh, xl, d);
          d = mfma16h(wh, xh, d);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[u][i] = fmaf(d[i], inv, acc[u][i]);
        }
        if (cc + 1 < nch) stage_w(buf ^ 1, ws);
        __syncthreads();
      }
    }
  }
  if (!live) return;
  const float rs = P.rowscale ? P.rowscale[n] : 1.f;
#pragma unroll
  for (int u = 0; u < CW; ++u) {
    const int col = tn * BC + 16 * u + 4 * g;  // four consecutive output columns
    float* y = P.Y + (int64_t)n * P.ldy + P.out_base + (col / NC) * P.out_stride + m * NC + (col % NC);
    float4 v = float4{acc[u][0] * rs, acc[u][1] * rs, acc[u][2] * rs, acc[u][3] * rs};
    if (P.bias) {
      const float4 b = *reinterpret_cast<const float4*>(P.bias + col);
      v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
    }
    if (P.accumulate) {
      const float4 o = *reinterpret_cast<const float4*>(y);
      v.x += o.x, v.y += o.y, v.z += o.z, v.w += o.w;
    }
    if (G.round_half) v = float4{qh(v.x, G.round_half), qh(v.y, G.round_half), qh(v.z, G.round_half), qh(v.w, G.round_half)};
    *reinterpret_cast<float4*>(y) = v;
  }
}

// first-layer node features h0[n] = embedding of the species and, with a table, the first
// linear_up output up0[z] (a function of the species only, built once per model)
__global__ void k_embed(int N, const int* __restrict__ species, const float* __restrict__ emb, int ld,
                        float* __restrict__ h, int half, const float* __restrict__ up_tab, float* __restrict__ h_up) {
  const int n = blockIdx.x, u = threadIdx.x, z = species[n];
  h[(int64_t)n * ld + u] = qh(emb[z * NC + u], half);
  if (up_tab) h_up[(int64_t)n * ld + u] = qh(up_tab[z * NC + u], half);
}

// ---------------------------------------------------------------------------
// symmetric contraction: thread = (node, channel); generated polynomials
// ---------------------------------------------------------------------------
struct ScW {
  const float* w[3];
};

template <int LOUT, int CORR>
struct ScPoly;
#define MACE_SC(L, C)                                                                              \
  template <>                                                                                      \
  struct ScPoly<L, C> {                                                                            \
    static constexpr int KT = SC_L##L##_C##C##_KT;                                                 \
    __device__ static void fwd(const float* f, const float* w, float* o) { sc_l##L##_c##C##_fwd(f, w, o); } \
    __device__ static void vjp(const float* f, const float* w, const float* go, float* g) {       \
      sc_l##L##_c##C##_vjp(f, w, go, g);                                                           \
    }                                                                                              \
  };
MACE_SC(0, 1) MACE_SC(0, 2) MACE_SC(0, 3)
MACE_SC(1, 1) MACE_SC(1, 2) MACE_SC(1, 3)
MACE_SC(2, 1) MACE_SC(2, 2) MACE_SC(2, 3)
#undef MACE_SC

template <int LOUT, int CORR>
__device__ __forceinline__ void sc_block_fwd(const float* f, const float* __restrict__ Wl, int z, int c,
                                             float* __restrict__ Bn, int half) {
  using P = ScPoly<LOUT, CORR>;
  float w[P::KT];
  const float* wz = Wl + (int64_t)z * P::KT * NC + c;
#pragma unroll
  for (int k = 0; k < P::KT; ++k) w[k] = wz[k * NC];
  float o[2 * LOUT + 1];
  P::fwd(f, w, o);
#pragma unroll
  for (int m = 0; m < 2 * LOUT + 1; ++m) Bn[NC * (LOUT * LOUT + m) + c] = qh(o[m], half);
}

template <int LOUT, int CORR>
__device__ __forceinline__ void sc_block_vjp(const float* f, const float* __restrict__ Wl, int z, int c,
                                             const float* __restrict__ gBn, float* g) {
  using P = ScPoly<LOUT, CORR>;
  float w[P::KT];
  const float* wz = Wl + (int64_t)z * P::KT * NC + c;
#pragma unroll
  for (int k = 0; k < P::KT; ++k) w[k] = wz[k * NC];
  float go[2 * LOUT + 1];
#pragma unroll
  for (int m = 0; m < 2 * LOUT + 1; ++m) go[m] = gBn[NC * (LOUT * LOUT + m) + c];
  float gl[16];
  P::vjp(f, w, go, gl);
#pragma unroll
  for (int i = 0; i < 16; ++i) g[i] += gl[i];
}

// Block (n, b) evaluates output block b (0e, 1o, 2e) of node n; NOUT, the layer's number of
// output blocks, is a template parameter so an instantiation holds only the polynomials it can
// run.  Correlation 3: 0e alone takes 59 VGPRs (eight waves per SIMD), 0e / 1o 255 (two),
// 0e / 1o / 2e 381 (one), against 456 for one thread running every block in turn.
template <int CORR, int NOUT>
__global__ void __launch_bounds__(NC) __attribute__((amdgpu_waves_per_eu(NOUT < 3 ? 2 : 1))) k_sc_fwd(int N, const float* __restrict__ A, int ldA,
                                               const int* __restrict__ species, ScW W, float* __restrict__ B,
                                               int ldB, int half) {
  const int n = blockIdx.x, c = threadIdx.x, b = blockIdx.y;
  float f[16];
  const float* An = A + (int64_t)n * ldA + c;
#pragma unroll
  for (int i = 0; i < 16; ++i) f[i] = An[i * NC];
  const int z = species[n];
  float* Bn = B + (int64_t)n * ldB;
  if constexpr (NOUT == 1) {
    sc_block_fwd<0, CORR>(f, W.w[0], z, c, Bn, half);
  } else if constexpr (NOUT == 2) {
    if (b == 0)
      sc_block_fwd<0, CORR>(f, W.w[0], z, c, Bn, half);
    else
      sc_block_fwd<1, CORR>(f, W.w[1], z, c, Bn, half);
  } else {
    if (b == 0)
      sc_block_fwd<0, CORR>(f, W.w[0], z, c, Bn, half);
    else if (b == 1)
      sc_block_fwd<1, CORR>(f, W.w[1], z, c, Bn, half);
    else
      sc_block_fwd<2, CORR>(f, W.w[2], z, c, Bn, half);
  }
}

// NOUT: output blocks of the layer (a template parameter: a layer with the 0e block only runs
// an instantiation without the larger polynomials' registers)
template <int CORR, int NOUT>
__global__ void __launch_bounds__(NC) k_sc_bwd(int N, const float* __restrict__ A, int ldA,
                                               const int* __restrict__ species, ScW W, const float* __restrict__ gB,
                                               int ldB, float* __restrict__ gA) {
  const int n = blockIdx.x, c = threadIdx.x;
  float f[16], g[16];
  const float* An = A + (int64_t)n * ldA + c;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    f[i] = An[i * NC];
    g[i] = 0.f;
  }
  const int z = species[n];
  const float* gBn = gB + (int64_t)n * ldB;
  sc_block_vjp<0, CORR>(f, W.w[0], z, c, gBn, g);
  if constexpr (NOUT > 1) sc_block_vjp<1, CORR>(f, W.w[1], z, c, gBn, g);
  if constexpr (NOUT > 2) sc_block_vjp<2, CORR>(f, W.w[2], z, c, gBn, g);
  float* gAn = gA + (int64_t)n * ldA + c;
#pragma unroll
  for (int i = 0; i < 16; ++i) gAn[i * NC] = g[i];
}

// ---------------------------------------------------------------------------
// wave reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// ---------------------------------------------------------------------------
// energy assembly and reductions (fixed order: deterministic)
// ---------------------------------------------------------------------------
// Readouts, node energies and the first backward gradient in one pass, one
// wavefront per atom (layers 0 .. L-2: linear readouts of h_{l+1}; layer L-1: the
// MLP readout 128 -> 16 -> silu -> 1, `blocks.py:540-608`):
//   node_e[n] = E0[z] + sum of the atom's pair-repulsion edge energies + readouts,
//   gh[n][u] = dE/dh_L[n][u] = sum_j W1[u][j] W2[j] silu'(y_j)
// (dE/dnode_e = 1, so the readout's VJP needs nothing from later kernels).  Lane l
// computes hidden unit j = l / 4 over the channel quarter (NC / 4) (l % 4) .. + NC / 4 - 1;
// a channel sum of the linear readouts and of the gradient takes lane l's channels
// l, l + 64, ... (NSLICE of them), the highest first.
struct ReadoutArgs {
  const float* h[4];   // h_{l+1}, 0e block at the row start
  const float* ro[4];  // linear readout weights (layers < L-1)
  int ldh[4];
  int L;
  const float* W1;     // last layer: [NC][16]
  const float* W2;     // [16]
  float* gh;           // dE/dh_L, row stride ldgh
  int ldgh;
};

__global__ void __launch_bounds__(256) k_energy_readout(int N, const int* __restrict__ species,
                                                        const float* __restrict__ e0,
                                                        const int* __restrict__ rowptr,
                                                        const float* __restrict__ zbl_e, ReadoutArgs A,
                                                        float* __restrict__ node_e, double* __restrict__ part,
                                                        int half) {
  __shared__ double red[4];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + w;
  double acc = 0.0;
  if (n < N) {  // wave-uniform
    float z = 0.f;
    if (zbl_e)
      for (int e = rowptr[n] + l; e < rowptr[n + 1]; e += 64) z += zbl_e[e];
    float v = e0[species[n]] + wave_sum(z);
    for (int k = 0; k + 1 < A.L; ++k) {  // linear readouts
      const float* hn = A.h[k] + (int64_t)n * A.ldh[k];
      float t = hn[l + 64 * (NSLICE - 1)] * A.ro[k][l + 64 * (NSLICE - 1)];
#pragma unroll
      for (int q = NSLICE - 2; q >= 0; --q) t = fmaf(hn[l + 64 * q], A.ro[k][l + 64 * q], t);
      const float a = wave_sum(t);
      v += qh(a, half);
    }
    {  // MLP readout of the last layer and its gradient
      const float* hn = A.h[A.L - 1] + (int64_t)n * A.ldh[A.L - 1];
      const int j = l >> 2, q = l & 3;
      float y = 0.f;
#pragma unroll 8
      for (int u = (NC / 4) * q; u < (NC / 4) * (q + 1); ++u) y = fmaf(hn[u], A.W1[u * 16 + j], y);
      y += __shfl_xor(y, 1);
      y += __shfl_xor(y, 2);
      y = qh(y, half);
      const float sg = 1.f / (1.f + expf(-y));
      float a = (q == 0) ? qh(y * sg, half) * A.W2[j] : 0.f;
#pragma unroll
      for (int off = 4; off < 64; off <<= 1) a += __shfl_xor(a, off);
      v += qh(a, half);
      const float cj = A.W2[j] * sg * (1.f + y * (1.f - sg));  // on the four lanes of unit j
      float gq[NSLICE];
#pragma unroll
      for (int q2 = 0; q2 < NSLICE; ++q2) gq[q2] = 0.f;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const float c = __shfl(cj, 4 * jj);
#pragma unroll
        for (int q2 = 0; q2 < NSLICE; ++q2) gq[q2] = fmaf(A.W1[(l + 64 * q2) * 16 + jj], c, gq[q2]);
      }
      float* gn = A.gh + (int64_t)n * A.ldgh;
#pragma unroll
      for (int q2 = 0; q2 < NSLICE; ++q2) gn[l + 64 * q2] = gq[q2];
    }
    if (l == 0) node_e[n] = v;
    acc = (double)v;
  }
  if (l == 0) red[w] = acc;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// fixed-order sum of block partials (deterministic); one block
__global__ void __launch_bounds__(256) k_sum_partials(const double* __restrict__ part, int nblk,
                                                      double* __restrict__ out) {
  double a = 0.0;
  for (int b = threadIdx.x; b < nblk; b += 256) a += part[b];
  const double t = block_sum_fixed(a);
  if (threadIdx.x == 0) *out = t;
}


__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// one wavefront per atom: F_a = -(sum over edges received by a - sum over edges sent by a) of dE/dv
// vir_zero (may be null): receives nine zeros (no virial requested, or no edges)
__global__ void __launch_bounds__(256) k_forces(int N, const int* __restrict__ rowptr, const int* __restrict__ rowptr_s,
                                                const int* __restrict__ perm_s, const float* __restrict__ gv,
                                                double* __restrict__ F, double* __restrict__ vir_zero,
                                                const double* __restrict__ e_part, int e_nblk,
                                                double* __restrict__ energy) {
  if (blockIdx.x == 0) {
    // the total energy: k_energy_readout's block partials in k_sum_partials' fixed order (a
    // launch of its own on the step's critical path otherwise; nothing before needs the sum)
    double s = 0.0;
    for (int b = threadIdx.x; b < e_nblk; b += 256) s += e_part[b];
    s = block_sum_fixed(s);
    if (threadIdx.x == 0) *energy = s;
    if (vir_zero && threadIdx.x < 9) vir_zero[threadIdx.x] = 0.0;
  }
  const int a = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (a >= N) return;  // whole wavefront exits together
  double fx = 0.0, fy = 0.0, fz = 0.0;
  for (int e = rowptr[a] + l; e < rowptr[a + 1]; e += 64) {
    fx -= gv[3 * e];
    fy -= gv[3 * e + 1];
    fz -= gv[3 * e + 2];
  }
  for (int k = rowptr_s[a] + l; k < rowptr_s[a + 1]; k += 64) {
    const int e = perm_s[k];
    fx += gv[3 * e];
    fy += gv[3 * e + 1];
    fz += gv[3 * e + 2];
  }
  fx = wave_sum_d(fx);
  fy = wave_sum_d(fy);
  fz = wave_sum_d(fz);
  if (l == 0) {
    F[3 * a] = fx;
    F[3 * a + 1] = fy;
    F[3 * a + 2] = fz;
  }
}

// writes zeros to vir[0..8] (no atoms)
__global__ void __launch_bounds__(64) k_zeros(double* __restrict__ vir) {
  if (threadIdx.x < 9) vir[threadIdx.x] = 0.0;
}

// G[a][b] = sum_e v_e[a] g_e[b]: the per-block partials of k_edge_bwd summed in block order
// (thread t adds partials t, t + 256, ..., then a fixed-order tree: deterministic); writes the
// symmetrised virial dE/d(eps_sym) = (G + G^T) / 2 (calculators.py:536-561).
__global__ void __launch_bounds__(256) k_virial_reduce(const double* __restrict__ part, int nblk,
                                                       double* __restrict__ vir) {
  double G[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    double a = 0.0;
    for (int b = threadIdx.x; b < nblk; b += 256) a += part[9 * b + k];
    G[k] = block_sum_fixed(a);
  }
  if (threadIdx.x < 9) {
    const int r = threadIdx.x / 3, c = threadIdx.x % 3;
    vir[threadIdx.x] = 0.5 * (G[3 * r + c] + G[3 * c + r]);
  }
}

// A batch of structures (graph_sum, utils.py:35-44): block g sums the node energies of
// structure g's atoms [gptr[g], gptr[g+1]) in a fixed order -- the same float node energies
// the total is summed from.
__global__ void __launch_bounds__(256) k_graph_energy(const int* __restrict__ gptr, const float* __restrict__ node_e,
                                                      double* __restrict__ eg) {
  const int g = blockIdx.x;
  double a = 0.0;
  for (int i = gptr[g] + threadIdx.x; i < gptr[g + 1]; i += 256) a += (double)node_e[i];
  const double t = block_sum_fixed(a);
  if (threadIdx.x == 0) eg[g] = t;
}

// Per-structure virial: structure g's edges are the receiver-CSR range of its atoms; the same
// products v_e[a] g_e[b] as k_edge_bwd's partials, summed in a fixed order and symmetrised.
__global__ void __launch_bounds__(256) k_graph_virial(const int* __restrict__ gptr, const int* __restrict__ rowptr,
                                                      const EdgeGeom* __restrict__ geom, const float* __restrict__ gv,
                                                      double* __restrict__ vir) {
  const int g = blockIdx.x;
  const int e0 = rowptr[gptr[g]], e1 = rowptr[gptr[g + 1]];
  double G[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) G[k] = 0.0;
  for (int e = e0 + threadIdx.x; e < e1; e += 256) {
    const EdgeGeom q = geom[e];
    const double v[3] = {q.x, q.y, q.z};
    const double d[3] = {gv[3 * e], gv[3 * e + 1], gv[3 * e + 2]};
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) G[3 * a + b] += v[a] * d[b];
  }
#pragma unroll
  for (int k = 0; k < 9; ++k) G[k] = block_sum_fixed(G[k]);
  if (threadIdx.x < 9) {
    const int r = threadIdx.x / 3, c = threadIdx.x % 3;
    vir[9 * g + threadIdx.x] = 0.5 * (G[3 * r + c] + G[3 * c + r]);
  }
}

// ---------------------------------------------------------------------------
// mh-1 non-linear interaction block, node side (blocks.py:735-807).  Q = linear_1(M) / (beta
// rho + alpha) and R = linear_res(up) in the gate-input layout [scalars C | gates of the
// l = 1, 2, 3 blocks, C each | 1o 3C | 2e 5C | 3o 7C] (component-major blocks; R covers the
// prefix of nres columns its input blocks reach); the gate (gate.py:19-164) writes the
// interaction irreps [0e C | 1o 3C | 2e 5C | 3o 7C].
// ---------------------------------------------------------------------------
constexpr float kSiluNorm = 1.6791768074035645f;     // normalize2mom(silu)
constexpr float kSigmoidNorm = 1.8467055569904827f;  // normalize2mom(sigmoid)

__device__ __forceinline__ float sigm(float x) { return 1.f / (1.f + expf(-x)); }

// rinv[n] = 1 / (beta rho_n + alpha), rho_n = sum of the receiver's edge densities (fixed order)
__global__ void __launch_bounds__(256) k_mh1_rho(int N, const int* __restrict__ rowptr, const float* __restrict__ dens,
                                                 float alpha, float beta, float* __restrict__ rinv) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (n >= N) return;
  float acc = 0.f;
  for (int e = rowptr[n] + l; e < rowptr[n + 1]; e += 64) acc += dens[e];
  acc = wave_sum(acc);
  if (l == 0) rinv[n] = 1.f / fmaf(beta, acc, alpha);
}

__device__ __forceinline__ float gate_in(const float* __restrict__ q, const float* __restrict__ rr, int nres, int j) {
  return j < nres ? q[j] + rr[j] : q[j];
}

// one thread per (node, channel): gout = gate(Q + R)
__global__ void __launch_bounds__(NC) k_mh1_gate(int N, const float* __restrict__ Q, const float* __restrict__ R,
                                                 int nres, float* __restrict__ gout, int half) {
  const int n = blockIdx.x, u = threadIdx.x;
  const float* q = Q + (int64_t)n * kGateInDim;
  const float* rr = R + (int64_t)n * nres;
  float* o = gout + (int64_t)n * 16 * NC;
  const float s = gate_in(q, rr, nres, u);
  o[u] = qh(kSiluNorm * s * sigm(s), half);
#pragma unroll
  for (int l = 1; l <= 3; ++l) {
    const float gt = kSigmoidNorm * sigm(gate_in(q, rr, nres, l * NC + u));
    const int qb = 4 * NC + NC * (l * l - 1), ob = NC * l * l;
    for (int m = 0; m < 2 * l + 1; ++m) o[ob + m * NC + u] = qh(gt * gate_in(q, rr, nres, qb + m * NC + u), half);
  }
}

// VJP: gP = dL/d(Q + R) from gG = dL/dgout, and dL/drho[n] = -beta rinv[n] sum_j gP[n][j] Q[n][j]
// (Q = linear_1(M) rinv): thread u holds columns j = u + k C (k = 0 .. 18), the block sums its
// waves' partial sums in wave order
__global__ void __launch_bounds__(NC) k_mh1_gate_bwd(int N, const float* __restrict__ Q, const float* __restrict__ R,
                                                     int nres, const float* __restrict__ gG, float* __restrict__ gP,
                                                     const float* __restrict__ rinv, float beta,
                                                     float* __restrict__ drho) {
  __shared__ float part[NC / 64];
  const int n = blockIdx.x, u = threadIdx.x;
  const float* q = Q + (int64_t)n * kGateInDim;
  const float* rr = R + (int64_t)n * nres;
  const float* go = gG + (int64_t)n * 16 * NC;
  float* gp = gP + (int64_t)n * kGateInDim;
  const float s = gate_in(q, rr, nres, u);
  const float sg = sigm(s);
  const float g0 = go[u] * kSiluNorm * sg * (1.f + s * (1.f - sg));
  gp[u] = g0;
  float pd = g0 * q[u];
#pragma unroll
  for (int l = 1; l <= 3; ++l) {
    const float gs = sigm(gate_in(q, rr, nres, l * NC + u));
    const int qb = 4 * NC + NC * (l * l - 1), ob = NC * l * l;
    float dgt = 0.f;
    for (int m = 0; m < 2 * l + 1; ++m) {
      const float gm = go[ob + m * NC + u];
      dgt = fmaf(gm, gate_in(q, rr, nres, qb + m * NC + u), dgt);
      const float gv = kSigmoidNorm * gs * gm;
      gp[qb + m * NC + u] = gv;
      pd = fmaf(gv, q[qb + m * NC + u], pd);
    }
    const float gl = dgt * kSigmoidNorm * gs * (1.f - gs);
    gp[l * NC + u] = gl;
    pd = fmaf(gl, q[l * NC + u], pd);
  }
  pd = wave_sum(pd);
  if ((u & 63) == 0) part[u >> 6] = pd;
  __syncthreads();
  if (u == 0) {
    float t = part[0];
#pragma unroll
    for (int w = 1; w < NC / 64; ++w) t += part[w];
    drho[n] = -beta * rinv[n] * t;
  }
}

}  // namespace

static inline unsigned cdiv(int64_t a, int b) { return (unsigned)((a + b - 1) / b); }

void launch_graph_energy(hipStream_t st, int G, const int* gptr, const float* node_e, double* eg) {
  if (G <= 0) return;
  MACE_LAUNCH(k_graph_energy, dim3(G), dim3(256), 0, st, gptr, node_e, eg);
}

void launch_graph_virial(hipStream_t st, int G, const int* gptr, const int* rowptr, const EdgeGeom* geom,
                         const float* gv, double* vir) {
  if (G <= 0) return;
  MACE_LAUNCH(k_graph_virial, dim3(G), dim3(256), 0, st, gptr, rowptr, geom, gv, vir);
}

void launch_embed(hipStream_t st, int N, const int* species, const float* emb, int ld, float* h, int half,
                  const float* up_tab, float* h_up) {
  if (N <= 0) return;
  MACE_LAUNCH(k_embed, dim3(N), dim3(NC), 0, st, N, species, emb, ld, h, half, up_tab, h_up);
}

void launch_sc_fwd(hipStream_t st, int N, int nout, int corr, const float* A, int ldA, const int* species,
                   const float* const* Wsc, float* B, int ldB, int half) {
  if (N <= 0) return;
  ScW w{{Wsc[0], nout > 1 ? Wsc[1] : nullptr, nout > 2 ? Wsc[2] : nullptr}};
  const dim3 grid((unsigned)N, (unsigned)nout);
#define MACE_SCF(C)                                                                                   \
  if (nout == 1)                                                                                      \
    MACE_LAUNCH((k_sc_fwd<C, 1>), grid, dim3(NC), 0, st, N, A, ldA, species, w, B, ldB, half);        \
  else if (nout == 2)                                                                                 \
    MACE_LAUNCH((k_sc_fwd<C, 2>), grid, dim3(NC), 0, st, N, A, ldA, species, w, B, ldB, half);        \
  else                                                                                                \
    MACE_LAUNCH((k_sc_fwd<C, 3>), grid, dim3(NC), 0, st, N, A, ldA, species, w, B, ldB, half);
  switch (corr) {
    case 1: MACE_SCF(1) break;
    case 2: MACE_SCF(2) break;
    case 3: MACE_SCF(3) break;
  }
#undef MACE_SCF
}

void launch_sc_bwd(hipStream_t st, int N, int nout, int corr, const float* A, int ldA, const int* species,
                   const float* const* Wsc, const float* gB, int ldB, float* gA) {
  if (N <= 0) return;
  ScW w{{Wsc[0], nout > 1 ? Wsc[1] : nullptr, nout > 2 ? Wsc[2] : nullptr}};
#define MACE_SCB(C)                                                                                   \
  if (nout == 1)                                                                                      \
    MACE_LAUNCH((k_sc_bwd<C, 1>), dim3(N), dim3(NC), 0, st, N, A, ldA, species, w, gB, ldB, gA);      \
  else if (nout == 2)                                                                                 \
    MACE_LAUNCH((k_sc_bwd<C, 2>), dim3(N), dim3(NC), 0, st, N, A, ldA, species, w, gB, ldB, gA);      \
  else                                                                                                \
    MACE_LAUNCH((k_sc_bwd<C, 3>), dim3(N), dim3(NC), 0, st, N, A, ldA, species, w, gB, ldB, gA);
  switch (corr) {  // nout is 1..3: checked at model load
    case 1: MACE_SCB(1) break;
    case 2: MACE_SCB(2) break;
    case 3: MACE_SCB(3) break;
  }
#undef MACE_SCB
}

void launch_virial_reduce(hipStream_t st, const double* part, int nblk, double* vir) {
  MACE_LAUNCH(k_virial_reduce, dim3(1), dim3(256), 0, st, part, nblk, vir);
}

void launch_energy_readout(hipStream_t st, int N, const int* species, const float* e0, const int* rowptr,
                           const float* zbl_e, int L, const float* const* h, const int* ldh, const float* const* ro,
                           const float* W1, const float* W2, float* gh, int ldgh, float* node_e, double* part,
                           int half) {
  ReadoutArgs A{};
  A.L = L;
  for (int k = 0; k < L && k < 4; ++k) {
    A.h[k] = h[k];
    A.ldh[k] = ldh[k];
    A.ro[k] = ro[k];
  }
  A.W1 = W1;
  A.W2 = W2;
  A.gh = gh;
  A.ldgh = ldgh;
  const int nblk = (int)cdiv(N, 4);
  if (nblk > 0)
    MACE_LAUNCH(k_energy_readout, dim3(nblk), dim3(256), 0, st, N, species, e0, rowptr, zbl_e, A, node_e,
                       part, half);
}

void launch_forces(hipStream_t st, int N, const int* rowptr, const int* rowptr_s, const int* perm_s,
                   const float* gv, double* forces, double* vir_zero, const double* e_part, double* energy) {
  const int e_nblk = (int)cdiv(N, 4);  // k_energy_readout's grid
  if (N <= 0) {
    MACE_LAUNCH(k_sum_partials, dim3(1), dim3(256), 0, st, e_part, 0, energy);
    if (vir_zero) MACE_LAUNCH(k_zeros, dim3(1), dim3(64), 0, st, vir_zero);
    return;
  }
  MACE_LAUNCH(k_forces, dim3(cdiv(N, 4)), dim3(256), 0, st, N, rowptr, rowptr_s, perm_s, gv, forces,
                     vir_zero, e_part, e_nblk, energy);
}

void launch_gemm_group(hipStream_t st, GemmGroup& g) {
  if (g.split) {  // 64 rows x 64 (or 128) columns per block
    // 128 columns when every output width allows it and the launch still has blocks for every CU
    // several times over (each row block's X is then read by half as many blocks)
    int64_t wide_tiles = 0;
    bool c128 = true;
    for (int q = 0; q < g.n; ++q) {
      c128 = c128 && g.p[q].Cout % 128 == 0;
      wide_tiles += cdiv(g.p[q].rows, 64) * (g.p[q].Cout / 128);
    }
    const int bc = c128 && wide_tiles >= 2048 ? 128 : 64;
    int tiles = 0;
    for (int q = 0; q < g.n; ++q) {
      GemmProb& P = g.p[q];
      P.tiles_n = P.Cout / bc;
      P.tile_begin = tiles;
      tiles += (int)cdiv(P.rows, 64) * P.tiles_n;
    }
    g.total_tiles = tiles;
    if (tiles <= 0) return;
    if (bc == 128)
      MACE_LAUNCH(k_gemm_group_x<8>, dim3(tiles), dim3(256), 0, st, g);
    else
      MACE_LAUNCH(k_gemm_group_x<4>, dim3(tiles), dim3(256), 0, st, g);
    return;
  }
  int row_tiles = 0;
  bool c128 = true;  // every problem's output width a multiple of 128 (not so at 192 channels)
  for (int q = 0; q < g.n; ++q) {
    row_tiles += (int)cdiv(g.p[q].rows, 16) * (g.p[q].Cout / 64);
    c128 = c128 && g.p[q].Cout % 128 == 0;
  }
  const bool wide = c128 && row_tiles >= 1024;  // enough blocks even with four column tiles per wave
  const int rows_per_block = wide ? 32 : 16, cols_per_block = wide ? 128 : 64;  // Cout: a multiple of 64
  int tiles = 0;
  for (int q = 0; q < g.n; ++q) {
    GemmProb& P = g.p[q];
    P.tiles_n = P.Cout / cols_per_block;
    P.tile_begin = tiles;
    tiles += (int)cdiv(P.rows, rows_per_block) * P.tiles_n;
  }
  g.total_tiles = tiles;
  if (tiles <= 0) return;
  if (wide)
    MACE_LAUNCH((k_gemm_group<4, 2, false>), dim3(tiles), dim3(256), 0, st, g);
  else
    MACE_LAUNCH((k_gemm_group<1, 8, true>), dim3(tiles), dim3(256), 0, st, g);
}


void launch_mh1_rho(hipStream_t st, int N, const int* rowptr, const float* dens, float alpha, float beta,
                    float* rinv) {
  if (N <= 0) return;
  MACE_LAUNCH(k_mh1_rho, dim3((N + 3) / 4), dim3(256), 0, st, N, rowptr, dens, alpha, beta, rinv);
}

void launch_mh1_gate(hipStream_t st, int N, const float* Q, const float* R, int nres, float* gout, int half) {
  if (N <= 0) return;
  MACE_LAUNCH(k_mh1_gate, dim3(N), dim3(NC), 0, st, N, Q, R, nres, gout, half);
}

void launch_mh1_gate_bwd(hipStream_t st, int N, const float* Q, const float* R, int nres, const float* gG,
                         float* gP, const float* rinv, float beta, float* drho) {
  if (N <= 0) return;
  MACE_LAUNCH(k_mh1_gate_bwd, dim3(N), dim3(NC), 0, st, N, Q, R, nres, gG, gP, rinv, beta, drho);
}

}  // namespace mace
