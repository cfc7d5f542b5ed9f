// Internal declarations shared by the kernel translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gen/tables.h"

namespace mace {

// Channel multiplicity of every irrep block.  The launchers check it at model
// load time; all kernels are compiled for this width (MACE_NC: 128, or 256 for the
// wide library; a multiple of 64, the channel slice of the tensor-product kernels).
#ifndef MACE_NC
#define MACE_NC 128
#endif
constexpr int NC = MACE_NC;
static_assert(NC % 64 == 0, "channel count must be a multiple of 64");
constexpr int NSLICE = NC / 64;  // 64-channel slices (one wave's lanes) of a channel block
constexpr int NBESSEL_MAX = 16;
constexpr int RADIAL_H = 64;   // radial-MLP hidden width compiled in

// Host-side count of the kernel dispatches this library has issued on the calling
// thread; the per-site profiler uses it to name every dispatch of a step.
extern thread_local int64_t g_dispatches;
#define MACE_LAUNCH(...)                \
  do {                                  \
    ++::mace::g_dispatches;             \
    hipLaunchKernelGGL(__VA_ARGS__);    \
  } while (0)

// fixed-order tree sum over a 256-thread block (result in every thread)
__device__ inline double block_sum_fixed(double a) {
  __shared__ double red[256];
  red[threadIdx.x] = a;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  const double t = red[0];
  __syncthreads();
  return t;
}

// Node feature layout (all internal node tensors): blocks in irreps order,
// inside a block the element (channel u, component m) sits at m * NC + u.
__host__ __device__ constexpr int block_off(int l) { return NC * l * l; }  // blocks 0..l-1 dense

// Per-edge TP table entry q (row-major i*K + c) of the shared (3-block) layout: the sum over
// x in [m1s(q), m1s(q+1)) of Y[m1j(x)] * m1v(x) (M1, l1 = 1), likewise m2* for M2 (l1 = 2)
__device__ constexpr int m1s(int q) { return TP3_M1_START[q]; }
__device__ constexpr int m1j(int x) { return TP3_M1_J[x]; }
__device__ constexpr float m1v(int x) { return TP3_M1_V[x]; }
__device__ constexpr int m2s(int q) { return TP3_M2_START[q]; }
__device__ constexpr int m2j(int x) { return TP3_M2_J[x]; }
__device__ constexpr float m2v(int x) { return TP3_M2_V[x]; }

struct EdgeGeom {        // per-edge record written by the front end
  float x, y, z, r;
};

// ----------------------------------------------------------------------------
// launchers (kernels_*.hip)
// ----------------------------------------------------------------------------

// edge front end: vectors, SH, radial features, ZBL edge energies
struct FrontParams {
  double cell[9];
  float r_max;
  float bessel_pref;     // sqrt(2 / r_max)
  int nbessel;
  int pcut;
  int has_zbl;
  int zbl_p;
  float zbl_a_exp;
  float zbl_a_pref;
  float zbl_scale;
  int feature_half;      // rounding mode of the stored SH and radial features (RND_*)
  int agnesi;            // Agnesi distance transform of r before the Bessel basis
  float ag_q, ag_p, ag_a;
  int apply_cutoff;      // 0: the envelope is not applied to ef; it goes to cut[e] (mh-1)
};

// Rounding of the stored activations of the feature path: RND_F16 (float16 feature
// policy) to the nearest fp16 value, RND_BF16 (bfloat16 policy) to the nearest bf16
// value (ties to even: the upper 16 bits of the fp32 pattern after adding 0x7fff plus
// the lowest kept bit; infinities stay infinite; a NaN, which the addition could carry
// into the sign or exponent, becomes the quiet NaN of its upper bits instead), RND_NONE
// leaves x
constexpr int RND_NONE = 0, RND_F16 = 1, RND_BF16 = 2;
__host__ __device__ __forceinline__ float round_bf16(float x) {
  unsigned u = __builtin_bit_cast(unsigned, x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __builtin_bit_cast(float, (u | 0x00400000u) & 0xffff0000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __builtin_bit_cast(float, u & 0xffff0000u);
}
__device__ __forceinline__ float qh(float x, int mode) {
  return mode == RND_F16 ? (float)(_Float16)x : mode == RND_BF16 ? round_bf16(x) : x;
}

// max over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the lanes holding one
// edge's k values in the 16x16 fragments), with the gfx950 permlane swaps: after
// swapping x's upper half with its own lower half, the two results hold each
// lane's value and its partner's (likewise for odd / even 16-lane rows)
__device__ __forceinline__ float max4_rows(float m) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  m = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// sum of x over the four lanes {l, l ^ 16, l ^ 32, l ^ 48} (the same value, in the same
// order of additions, on all four)
__device__ __forceinline__ float sum4_rows(float m) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  m = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ag_cov: covalent radius per species for the Agnesi transform (unused without it)
// cut (used when p.apply_cutoff == 0): the envelope of every edge, cut[e]
void launch_edge_fwd(hipStream_t st, int64_t E, const double* pos, const int* sender,
                     const int* receiver, const int* shifts, const int* species,
                     const float* bessel_w, const float* zbl_z, const float* zbl_cov,
                     const float* ag_cov, const FrontParams& p, const double* gcell, const int* gid,
                     EdgeGeom* geom, float* Y, float* ef, float* zbl_e, float* Mt, int mts, int nent,
                     float* cut);
// gcut (used when p.apply_cutoff == 0): dL/dcut[e]
void launch_edge_bwd(hipStream_t st, int64_t E, const int* sender, const int* receiver, const int* species,
                     const float* bessel_w, const float* zbl_z, const float* zbl_cov, const float* ag_cov,
                     const FrontParams& p, const EdgeGeom* geom, const float* gY, int gyp, const float* gef, float* gv,
                     double* vir_part, const float* gcut);
// symmetrised virial from the per-block partials of launch_edge_bwd
void launch_virial_reduce(hipStream_t st, const double* part, int nblk, double* vir);
// a batch of G structures with atoms [gptr[g], gptr[g+1]): per-structure energies and virials
void launch_graph_energy(hipStream_t st, int G, const int* gptr, const float* node_e, double* eg);
void launch_graph_virial(hipStream_t st, int G, const int* gptr, const int* rowptr, const EdgeGeom* geom,
                         const float* gv, double* vir);
// density normalisation (blocks.py:372-380): rinv[n] = 1 / (1 + sum_{e -> n} tanh((ef_e . wd)^2))
void launch_density_fwd(hipStream_t st, int N, const int* rowptr, const float* ef, int nb,
                        const float* wd, float* rinv);
// grho[n] = -rinv[n] * sum_j gA[n][j] A[n][j]  (A: the normalised message, dint values per node)
void launch_density_node_bwd(hipStream_t st, int N, int dint, const float* gA, const float* A,
                             const float* rinv, float* grho);
// gef[e] += grho[recv(e)] * d tanh((ef_e . wd)^2) / d ef_e
void launch_density_edge_bwd(hipStream_t st, int64_t E, const int* receiver, const float* ef, int nb,
                             const float* wd, const float* grho, float* gef);

// radial MLP, ef (E x nb) -> w (E x W); weights [in][out] row-major, W3T = W3 transposed [W][64].
// h3 [E][64] = silu(silu(silu(ef W0) W1) W2); w = h3 W3.  W0..W2 enter as tile images built once
// per model by launch_mlp_permute (mlp_tile_bytes() bytes).  mode 0: fp32 h3; 1 (float16 feature
// policy): hidden activations rounded to fp16, h3 fp16; 2: h3 as scaled fp16 hi/lo pairs [E][2][64]
// with inverse row scales h3inv[E] (operand of launch_mlp_out_x); 3 (bfloat16 policy): hidden
// activations and the fp32 h3 rounded to bf16 values.  ds (may be null): silu' of the
// three pre-activations, ds[E][3][64], for launch_mlp_hidden_bwd.
constexpr int H3_F32 = 0, H3_F16 = 1, H3_SPLIT = 2, H3_BF16 = 3;  // launch_mlp_hidden modes
size_t mlp_tile_bytes();
void launch_mlp_permute(hipStream_t st, int nb, const float* W0, const float* W1, const float* W2, void* tiles);
void launch_mlp_hidden(hipStream_t st, int64_t E, int nb, const float* ef, const void* tiles, void* h3,
                       float* h3inv, float* ds, int mode);
// float32 policy on fp16 matrix cores (split operands): tile images of W0..W2 split with the
// power-of-two scales scale3 (inverse winv3), h3 written as in mode 2
size_t mlp_tile_x_bytes();
void launch_mlp_permute_x(hipStream_t st, int nb, const float* W0, const float* W1, const float* W2,
                          const float* scale3, void* tiles);
// rnd: rounding mode of the activations (RND_*; the split of a rounded h3 has a zero lo plane,
// which is not written when store_lo is 0: for readers of the hi plane only)
void launch_mlp_hidden_x(hipStream_t st, int64_t E, int nb, const float* ef, const void* tiles,
                         const float* winv3, void* h3x, float* h3inv, float* ds, int rnd, int store_lo = 1);
// gh3: np partials of dL/dh3 ([np][E][64]), added in order; ds null: silu' of the
// hidden pre-activations recomputed from ef with the forward's rounding mode rnd (the forward
// then need not save them)
void launch_mlp_hidden_bwd_x(hipStream_t st, int64_t E, int nb, const void* tiles, const float* winv3,
                             const float* ef, const float* ds, const float* gh3, int np, float* gef,
                             int accumulate, int rnd);
// rnd RND_F16: h3, W3T and w fp16 arrays (fp32 accumulation); else fp32, with bias ([W], may be
// null) and rs ([E], may be null): w = (h3 W3 + bias) rs[e], rounded by rnd (RND_NONE / RND_BF16)
void launch_mlp_out(hipStream_t st, int64_t E, int W, const void* h3, const void* W3T, void* w,
                    int rnd, const float* bias, const float* rs);
// float32 policy on fp16 matrix cores: w (fp32) from the split h3 of mode 2 and W3Tx = [hi | lo]
// fp16 planes of W3^T [W][64] scaled by 1 / cscale; bias ([W]) and rs ([E]) as launch_mlp_out
void launch_mlp_out_x(hipStream_t st, int64_t E, int W, const void* h3x, const float* h3inv,
                      const void* W3Tx, float cscale, float* w, const float* bias, const float* rs);
// VJP: gh3 = gw W3^T, then gef (+)= dL/def through the hidden layers (saved silu' values);
// with b3 ([W]) also gwb[e] = gw[e] . b3
void launch_mlp_gh3(hipStream_t st, int64_t E, int W, const float* gw, const float* W3, float* gh3,
                    const float* b3, float* gwb);

// mh-1 non-linear interaction block (blocks.py:611-807).  LayerNorm radial MLP (radial.py:344-357)
// over [ef | source species embedding | target species embedding]: the species parts of the
// first Linear are per-species tables ts / tt ([n_el][64], tt with the bias); tiles: the
// launch_mlp_permute image of (ef part of layer 1 [nb][64], layer 2 [64][64], layer 3 [64][64]);
// dtiles: the same for the density MLP's first layer (only its first matrix is used).
struct LnMlpParams {
  const float* ts;    // [n_el][64]
  const float* tt;    // [n_el][64]
  const float* ln;    // [3][2][64]: LayerNorm scale, shift after layers 1..3
  const float* bias;  // [2][64]: biases of layers 2, 3
  const float* dts;   // [n_el][64] density MLP
  const float* dtt;   // [n_el][64] (+ bias)
  const float* dln;   // [2][64]
  const float* dw1;   // [65]: output weights, then the output bias
  float winv[3];      // inverse power-of-two scales of the split images of W0, W1, W2
};
// h3 = silu(LN(...)) of the third layer, fp32 [E][64] with h3inv null, else split pairs
// [E][2][64] with inverse row scales h3inv[E] (as launch_mlp_hidden mode 2);
// dens[e] = tanh(x^2) cut[e] (cut may be null: 1); both rounded by mode half (RND_*, the feature
// policy) before they are stored
// tiles_x (null: the hidden layers on fp32 matrix cores): the split images of W0..W2 as
// launch_mlp_permute_x writes them, for the hidden layers on fp16 matrix cores (split operands)
void launch_rmlp_ln_fwd(hipStream_t st, int64_t E, int nb, const float* ef, const float* cut,
                        const int* sender, const int* receiver, const int* species, const void* tiles,
                        const void* tiles_x, const void* dtiles, const LnMlpParams& P, void* h3, float* h3inv,
                        float* dens, int half);
// VJP from G = gw W3^T (np partials [np][E][64], added in order), gwb = gw . b3 (np partials
// [np][E]) and drho ([N], dL/d(sum of the receiver's edge densities)): gef (+)= dL/def ([E][nb])
// and, with cut, gcut (+)= dL/dcut ([E]); btiles / dbtiles: the transposed images
// (launch_mlp_permute's second half)
void launch_rmlp_ln_bwd(hipStream_t st, int64_t E, int nb, const float* ef, const float* cut,
                        const int* sender, const int* receiver, const int* species, const void* tiles,
                        const void* btiles, const void* tiles_x, const void* btiles_x, const void* dtiles,
                        const void* dbtiles, const LnMlpParams& P, const float* G, const float* gwb, int np,
                        const float* drho, float* gef, float* gcut, int accumulate);
size_t mlp_tile_fwd_bytes();  // offset of the transposed image inside an mlp_tile_bytes() block
size_t mlp_tile_x_fwd_bytes();  // ... inside an mlp_tile_x_bytes() block
// node side of the mh-1 block.  Q [N][kGateInDim] = linear_1(M) / (beta rho + alpha), R [N][nres]
// = linear_res(linear_up(h)) over the leading nres columns of the gate input layout
// [scalars C | gates C x 3 | 1o 3C | 2e 5C | 3o 7C]; gout [N][16 C] = gate(Q + R)
constexpr int kGateInDim = 19 * NC;
void launch_mh1_rho(hipStream_t st, int N, const int* rowptr, const float* dens, float alpha, float beta,
                    float* rinv);
void launch_mh1_gate(hipStream_t st, int N, const float* Q, const float* R, int nres, float* gout, int half);
// also drho[n] = dL/drho_n = -beta rinv[n] sum_j gP[n][j] Q[n][j]
void launch_mh1_gate_bwd(hipStream_t st, int N, const float* Q, const float* R, int nres, const float* gG,
                         float* gP, const float* rinv, float beta, float* drho);

// float16 feature policy: gw fp16 with per-(edge, channel half) scales, W3 fp16 [64][W]
void launch_mlp_gh3_h(hipStream_t st, int64_t E, int W, const void* gw, const float* gscale, const void* W3h,
                      float* gh3);
// float32 policy on fp16 matrix cores: gw fp32 [E][W] (split per edge and 32-wide k chunk in the
// kernel), W3x = [hi | lo] fp16 planes of W3 [64][W] scaled by 1 / cscale; b3 and gwb as
// launch_mlp_gh3
void launch_mlp_gh3_x(hipStream_t st, int64_t E, int W, const float* gw, const void* W3x, float cscale,
                      float* gh3, const float* b3, float* gwb);
void launch_mlp_hidden_bwd(hipStream_t st, int64_t E, int nb, const void* tiles, const float* ds,
                           const float* gh3, float* gef, int accumulate);

// per-edge x2-first tables Mt[e] (row stride mts) for the l1 >= 1 TP paths
int tp_table_entries(int max_lin);
// conv TP fused with the receiver-CSR scatter; half is the rounding mode of M (RND_*); w is
// _Float16 under RND_F16 (float16 feature policy), else float
void launch_tp_fwd(hipStream_t st, int lin, int N, const int* rowptr, const int* sender,
                   const float* Y, const float* Mt, int mts, const void* w, const float* up, float* M,
                   int half);
// TP VJP, receiver-centric; gY is [E][2][16] (per channel half).  With gxe != null the
// per-edge input gradient is also stored, row pos_s[e] of gxe ([E][LIN^2 * NC], sender order).
// half == RND_F16 (float16 policy): w and gw are fp16, gw [E][W] scaled per (edge, channel half)
// by 1 / gscale[e][half]; else w and gw are float [E][W]
void launch_tp_bwd_recv(hipStream_t st, int lin, int N, const int* rowptr, const int* sender,
                        const float* Y, const float* Mt, int mts, const void* w, const float* up,
                        const float* gM, void* gw, float* gscale, float* gY, int accumulate_gY,
                        const int* pos_s, float* gxe, int half);
// gup[a] = sum of the sender-ordered gxe rows of node a
// Radial-MLP output layer fused into the TP forward (split products, lin = 1..3): w is
// built per 16-edge tile from the split h3 planes (h3x, h3inv) and the split W3^T planes
// (W3Tx, scale wscale), M is written as by launch_tp_fwd and w ([E][W]) for the VJP; w and
// M rounded by rnd (RND_*, the feature policy), w stored as 16-bit fp16 / bf16 patterns under
// RND_F16 / RND_BF16 (exact: the values are already rounded).
// b3 (non-linear interaction block, float32 policy; null otherwise): w = (W3^T h3 + b3) cut
// (cut [E], may be null: 1)
void launch_tpx_fwd(hipStream_t st, int lin, int N, int64_t E, const int* rowptr, const int* sender, const float* Y,
                    const float* Mt, int mts, const void* h3x, const float* h3inv, const void* W3Tx, int W,
                    float wscale, const float* up, float* M, float* w, int rnd, const float* b3, const float* cut,
                    int store_w = 1);
// TP VJP with the radial-MLP output layer's backward product fused in (split products,
// lin = 1..3): reads w ([E][W], written by
// launch_tpx_fwd), writes the dL/dh3 partials gh3p ([P][E][64], P = 2 x input
// degrees of the layer), dL/dY partials into gY[e][p][16] (gyp partials per
// edge; written, or added when accumulate_gY) and, with gxe, the per-edge dL/dx
// rows as launch_tp_bwd_recv does (as fp16 values when wfmt is RND_F16).  wfmt: the storage
// format of w (the forward's rnd).  b3
// (non-linear interaction block, float32 policy; null otherwise): also the partials
// gwbp[p][e] = sum over partial p's columns k of dL/dw[e][k] b3[k] ([P][E]).
void launch_tpx_bwd(hipStream_t st, int lin, int N, int64_t E, const int* rowptr, const int* sender, const float* Y,
                    const float* Mt, int mts, const float* w, const void* W3x, int W, float wscale, const float* up,
                    const float* gM, const int* pos_s, float* gxe, float* gY, int gyp, int accumulate_gY,
                    float* gh3p, int wfmt, const float* b3, float* gwbp, const void* h3x = nullptr,
                    const float* h3inv = nullptr, const void* W3Tx = nullptr, int rebuild_w = 0);
// rebuild_w: w is not read but made again from h3x / h3inv / W3Tx (the forward's operands), which
// the forward then need not store (launch_tpx_fwd store_w = 0); allowed where
// tpx_rebuilds_w(lin, wfmt, b3 != null): a half-precision policy (one product per tile), one or
// two input blocks, the standard interaction block
bool tpx_rebuilds_w(int lin, int wfmt, bool nonlinear);
// p[0 .. n) = 0 (a kernel, not a memset: safe inside captured graphs)
void launch_fill_zero(hipStream_t st, float* p, int64_t n);
// gx16: the rows hold fp16 values (launch_tpx_bwd under the float16 policy), else floats;
// accumulate: gup += the sums (else gup = the sums)
void launch_tp_gather_gx(hipStream_t st, int lin, int N, const int* rowptr_s, const float* gxe,
                         float* gup, int gx16, int accumulate);

// Grouped fp32-MFMA GEMM over node rows: up to GEMM_MAX problems in one launch.
// Each problem: Y[row, c] (+)= sum_k X1[row, k] WT1[c][k] + sum_k X2[row, k] WT2[c][k] + bias[c]
// with rows (node n, component m): X[n, in_base + (k/NC) in_stride + m NC + k%NC], Y likewise
// with out_base / out_stride.  With rowmap, problem row i d + m addresses node rowmap[i] (the
// atoms of one species, for per-species weights).
constexpr int GEMM_MAX = 16;
struct GemmProb {
  int d, rows, K1, K2, Cout;
  const float* X1;
  int ldx1, in_base1, in_stride1;
  const float* WT1;  // B^T of operand 1: [Cout][K1]
  const float* X2;
  int ldx2, in_base2, in_stride2;
  const float* WT2;  // B^T of operand 2: [Cout][K2]
  float* Y;
  int ldy, out_base, out_stride;
  const float* bias;
  const float* rowscale;  // optional per-node factor on the product (before bias / accumulate)
  const int* rowmap;      // optional: node of each problem row block (rows = d x its length)
  int accumulate;
  int tiles_n, tile_begin;
  // split products (GemmGroup::split): [hi | lo] fp16 planes of WT1 / WT2 scaled by 1 / winv
  const _Float16* WX1;
  const _Float16* WX2;
  float winv1, winv2;
};
struct GemmGroup {
  GemmProb p[GEMM_MAX];
  int n;
  int total_tiles;
  int round_half;  // rounding mode of the outputs (RND_*)
  int split;       // float32 policy on fp16 matrix cores (split operands, WX1 / WX2 set)
};
// passed by value as a kernel argument: keep it within the 4 KiB kernel-argument budget
static_assert(sizeof(GemmGroup) <= 4096, "GemmGroup exceeds 4 KiB of kernel arguments");
void launch_gemm_group(hipStream_t st, GemmGroup& g);

// h0 = embedding per species; with up_tab, also h_up = up_tab[species] (first linear_up, which
// depends on the species only)
void launch_embed(hipStream_t st, int N, const int* species, const float* emb, int ld, float* h, int half,
                  const float* up_tab, float* h_up);

// symmetric contraction (all output blocks of one product layer)
void launch_sc_fwd(hipStream_t st, int N, int nout, int corr, const float* A, int ldA,
                   const int* species, const float* const* Wsc, float* B, int ldB, int half);
void launch_sc_bwd(hipStream_t st, int N, int nout, int corr, const float* A, int ldA,
                   const int* species, const float* const* Wsc, const float* gB, int ldB,
                   float* gA);


// readouts of every layer (linear for l < L-1 on h[l], MLP W1 [128][16], W2 [16] for the last),
// node energies, their total and dE/dh_L (gh, row stride ldgh) in one pass
void launch_energy_readout(hipStream_t st, int N, const int* species, const float* e0, const int* rowptr,
                           const float* zbl_e, int L, const float* const* h, const int* ldh, const float* const* ro,
                           const float* W1, const float* W2, float* gh, int ldgh, float* node_e, double* part,
                           int half);
// vir_zero (may be null) receives nine zeros
// also writes the total energy from the readout's block partials (fixed order)
void launch_forces(hipStream_t st, int N, const int* rowptr, const int* rowptr_s, const int* perm_s,
                   const float* gv, double* forces, double* vir_zero, const double* e_part, double* energy);

// neighbour list
struct NLParams {
  double cell[9];       // effective cell (rows)
  double inv[9];        // inverse of the effective cell
  double origin[3];
  int periodic[3];
  int nbin[3];
  int range[3];
  double cutoff2;
};
// atoms [i0, i0 + n): one structure, its bins numbered from bin_off; iota[i] = i for the sort;
// pos_build: a copy of the positions (the reference of the skin criterion)
void launch_nl_bin(hipStream_t st, int i0, int n, const double* pos, const NLParams& p, int bin_off,
                   double* wpos, int* img, int* bin, int* iota, double* pos_build);
// *flag = 1 if some atom's squared displacement from pos_build exceeds thr2 (flag not cleared)
void launch_max_disp(hipStream_t st, int n, const double* pos, const double* pos_build, double thr2, int* flag);
// start[b] (b = 0 .. nbins) = first position of key b in the sorted keys[0 .. n); with wpos, also
// wpos_s / img_s = the positions / images of atoms[0 .. n) (the atoms in key order)
// One structure of at most kNlSmall atoms: binning, the stable sort by bin and the bins' first
// positions in one block (the outputs of launch_nl_bin + a sort + launch_key_starts)
constexpr int kNlSmall = 1024;
void launch_nl_prep_small(hipStream_t st, int n, const double* pos, const NLParams& p, int nbins, int key_bits,
                          double* wpos, int* img, int* bin, double* pos_build, int* bin_sorted, int* atoms,
                          int* bin_start, double* wpos_s, int* img_s);
// exclusive prefix sum of n <= 2 kNlSmall ints in one block
void launch_exclusive_sum_small(hipStream_t st, int n, const int* in, int* out);
void launch_key_starts(hipStream_t st, int n, const int* keys, int nbins, int* start, const int* atoms = nullptr,
                       const double* wpos = nullptr, const int* img = nullptr, double* wpos_s = nullptr,
                       int* img_s = nullptr);
// counts[j] for the structure's atoms and cpre[j][k] (row stride cstride) = the number of j's
// edges before its k-th neighbour cell, k = 0 .. ncell; hits[j] (hcap int pairs per atom): j's
// first hcap edges as (candidate slot, cell index); also sets *tail = 0 and *missing = 0
void launch_nl_count(hipStream_t st, int i0, int n, const NLParams& p, int bin_off, const double* wpos,
                     const double* wpos_s, const int* bin, const int* bin_start, const int* bin_atoms, int cstride,
                     int* cpre, int* hits, int hcap, int* counts, int* tail, int* missing);
// the edges of the structure's rows, and perm_s = pos_s = the reverse of every edge (the
// sender-side CSR of the symmetric list; an edge without a reverse maps to itself and is counted
// in *missing); rows of no more than hcap edges are written from the count pass's hits
void launch_nl_fill(hipStream_t st, int i0, int n, const NLParams& p, int bin_off, const double* wpos,
                    const double* wpos_s, const int* img, const int* img_s, const int* bin, const int* bin_start,
                    const int* bin_atoms, const int* rowptr, int cstride, const int* cpre, const int* hits, int hcap,
                    int* sender, int* receiver, int* shifts, int* perm_s, int* pos_s, int* missing);
void launch_fill_iota(hipStream_t st, int n, int* out);
void launch_count_keys(hipStream_t st, int64_t E, const int* keys, int* counts);

}  // namespace mace
