// Channelwise CG edge tensor product fused with the receiver-CSR segmented sum,
// and its VJPs.
//
// Semantics: the reference's uvu conv TP (`tensor_product.py:833-1043`) with
// per-edge weights w[e, slot*C + u], followed by scatter_sum onto receivers
// (`utils.py:20-32`, `blocks.py:273-274`):
//   M[n, slot, k, u] = sum_{e: recv(e) = n} w[e, slot, u] *
//                      sum_{i, j} x[send(e), l1, i, u] Y[e, l2, j] C_slot[i, j, k] pw_slot
// Layouts (internal): x = up[n][NC*(l1^2 + i) + u]; M[n][NC*acc(slot, k) + u];
// w[e][slot*NC + u]; Y[e][16].
//
// Per-edge x2-first tables Mt[e] = [M1(3 x K1) | M2(5 x K2)] with
// M_l1[i][col] = sum_j Y_j C[i, j, k] pw are built once per step by
// the edge front end, k_edge_fwd (they depend only on Y), and shared by every layer.
//
// TP kernels: one workgroup per node, NG groups of NC threads (thread = channel
// u, so a node's 128 channels are two wave64s per group).  Group g takes a
// contiguous share of the node's edges.  Edge indices, senders and the Y / Mt
// rows are wave-uniform, so they are read through scalar loads; the next
// edge's weights and inputs are loaded while the current one is computed.
// There is no barrier inside the edge loop; the NG partial results are
// combined once at the end in a fixed order (deterministic, no atomics).
//
// dL/dY of an edge is a sum over the 128 channels: each wave reduces its 64
// lanes' 16 partials with a recursive-halving shuffle (17 exchanges) and
// stores them in gY[e][slice][16] (slice = which 64 channels); the edge backward
// adds the two halves.
#include <hip/hip_runtime.h>

#include <stdexcept>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "common.h"

namespace mace {
namespace {

template <int LIN>
struct TPT;

#define MACE_TP_TRAITS(N)                                                          \
  template <>                                                                      \
  struct TPT<N> {                                                                  \
    static constexpr int NSLOT = TP##N##_NSLOT, NACC = TP##N##_NACC;               \
    static constexpr int K1 = TP##N##_K1, K2 = TP##N##_K2;                         \
    __host__ __device__ static constexpr int l1(int s) { return TP##N##_L1[s]; }   \
    __host__ __device__ static constexpr int l2(int s) { return TP##N##_L2[s]; }   \
    __host__ __device__ static constexpr int l3(int s) { return TP##N##_L3[s]; }   \
    __host__ __device__ static constexpr int acc(int s) { return TP##N##_ACC[s]; } \
    __host__ __device__ static constexpr int col(int s) { return TP##N##_COL[s]; } \
  };
MACE_TP_TRAITS(1)
MACE_TP_TRAITS(2)
MACE_TP_TRAITS(3)
#undef MACE_TP_TRAITS

constexpr int MT_M2 = TP3_M1_NE;  // offset of the l1 = 2 table inside an Mt row

// The CG terms of each M1 (l1 = 1) / M2 (l1 = 2) table entry q (M[q] = sum over terms of
// Y[j] v), padded to two with (j, v) = (0, 0): tables a lane indexes with its own entry number.
template <int NE>
struct MTerms {
  int j[NE][2];
  float v[NE][2];
};
template <int NE>
constexpr int max_terms(const int (&start)[NE + 1]) {
  int m = 0;
  for (int q = 0; q < NE; ++q) m = start[q + 1] - start[q] > m ? start[q + 1] - start[q] : m;
  return m;
}
static_assert(max_terms<TP3_M1_NE>(TP3_M1_START) <= 2, "M1 entries with more than two CG terms");
static_assert(max_terms<TP3_M2_NE>(TP3_M2_START) <= 2, "M2 entries with more than two CG terms");
template <int NE, int NT>
constexpr MTerms<NE> make_terms(const int (&start)[NE + 1], const int (&js)[NT], const float (&vs)[NT]) {
  MTerms<NE> t{};
  for (int q = 0; q < NE; ++q)
    for (int x = start[q]; x < start[q + 1]; ++x) {
      t.j[q][x - start[q]] = js[x];
      t.v[q][x - start[q]] = vs[x];
    }
  return t;
}
__constant__ const MTerms<TP3_M1_NE> kM1Terms = make_terms<TP3_M1_NE>(TP3_M1_START, TP3_M1_J, TP3_M1_V);
__constant__ const MTerms<TP3_M2_NE> kM2Terms = make_terms<TP3_M2_NE>(TP3_M2_START, TP3_M2_J, TP3_M2_V);

static_assert(TP2_K1 == TP3_K1, "shared M1 layout");

// Inputs of one edge for one channel, loaded ahead of use.
template <int LIN>
struct EdgeIn {
  float w[TPT<LIN>::NSLOT];
  float x0, x1[3], x2[5];
};

template <int LIN>
__device__ __forceinline__ void load_x(const float* __restrict__ xs, float& x0, float* x1, float* x2) {
  x0 = xs[0];
  if constexpr (LIN >= 2) {
#pragma unroll
    for (int i = 0; i < 3; ++i) x1[i] = xs[NC * (1 + i)];
  }
  if constexpr (LIN >= 3) {
#pragma unroll
    for (int i = 0; i < 5; ++i) x2[i] = xs[NC * (4 + i)];
  }
}

// Per-edge weights.  In the VJP they are a read-once stream written long
// before (NT: nontemporal loads, which keep them from evicting the gathered
// node rows and the edge tables from L2); the forward pass reads them right
// after the radial MLP wrote them and uses plain loads, which can hit in the
// last-level cache.
// WT = float, or _Float16 under the float16 feature policy.
template <int LIN, bool NT, typename WT>
__device__ __forceinline__ void load_w(const WT* __restrict__ we, float* wv) {
#pragma unroll
  for (int s = 0; s < TPT<LIN>::NSLOT; ++s)
    wv[s] = (float)(NT ? __builtin_nontemporal_load(we + s * NC) : we[s * NC]);
}

// Forward contribution of one edge to this channel's accumulators.  GRP >= 0
// restricts the sum to the slots whose input block is l1 = GRP.
template <int LIN, int GRP = -1>
__device__ __forceinline__ void tp_edge_fwd(float* acc, const EdgeIn<LIN>& in, const float* __restrict__ Ye,
                                            const float* __restrict__ Me, const float* M2) {
  using T = TPT<LIN>;
#pragma unroll
  for (int s = 0; s < T::NSLOT; ++s) {
    if (GRP >= 0 && T::l1(s) != GRP) continue;
    const float ww = in.w[s];
    const int a0 = T::acc(s), d = 2 * T::l3(s) + 1;
    if (T::l1(s) == 0) {
      const float xw = in.x0 * ww;
#pragma unroll
      for (int m = 0; m < d; ++m) acc[a0 + m] = fmaf(xw, Ye[T::l2(s) * T::l2(s) + m], acc[a0 + m]);
    } else if (T::l1(s) == 1) {
      const int c0 = T::col(s);
#pragma unroll
      for (int k = 0; k < d; ++k) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) t = fmaf(in.x1[i], Me[i * T::K1 + c0 + k], t);
        acc[a0 + k] = fmaf(ww, t, acc[a0 + k]);
      }
    } else {
      const int c0 = T::col(s);
#pragma unroll
      for (int k = 0; k < d; ++k) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 5; ++i) t = fmaf(in.x2[i], M2[i * T::K2 + c0 + k], t);
        acc[a0 + k] = fmaf(ww, t, acc[a0 + k]);
      }
    }
    // three input blocks: keep each slot's LDS table reads next to their use
    // (hoisting all 155 of them would cost as many registers)
    if constexpr (LIN == 3) __builtin_amdgcn_sched_barrier(0);
  }
}

// Group of NC threads this thread belongs to.  NC is a multiple of the wave
// size, so the value is wave-uniform; readfirstlane tells the compiler, which
// then keeps edge indices in scalar registers and reads the per-edge Y / Mt
// rows with scalar loads.
__device__ __forceinline__ int group_id() {
  static_assert(NC % 64 == 0, "a group spans whole waves");
  return __builtin_amdgcn_readfirstlane(threadIdx.x / NC);
}

// With three input blocks an edge's tables hold 72 + 155 values, more than the
// scalar registers take; the l1 = 2 part is then staged per wave in LDS
// (double-buffered, the next edge's part loaded into registers while the
// current edge is computed) and read back as broadcast LDS loads.
constexpr int M2N = TP3_M2_NE, M2PAD = 160;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct M2Stage {
  float r[3];
  __device__ __forceinline__ void load(const float* __restrict__ row, int lane) {
#pragma unroll
    for (int j = 0; j < 3; ++j) r[j] = (lane + 64 * j < M2N) ? row[lane + 64 * j] : 0.f;
  }
  __device__ __forceinline__ void store(float* buf, int lane) const {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (lane + 64 * j < M2N) buf[lane + 64 * j] = r[j];
  }
};

// share [gb, ge) of a node's edge range [beg, end) taken by group g of NG
template <int NG>
__device__ __forceinline__ void group_range(int beg, int end, int g, int& gb, int& ge) {
  const int per = (end - beg + NG - 1) / NG;
  gb = min(end, beg + g * per);
  ge = min(end, gb + per);
}

// Fixed-order combine of per-group register vectors v[NV] into group 0.
template <int NV, int NG>
__device__ __forceinline__ void combine_groups(float* v, int g, int u, float (*sRed)[NC]) {
#pragma unroll 1
  for (int q = NG - 1; q >= 1; --q) {
    __syncthreads();
    if (g == q)
#pragma unroll
      for (int a = 0; a < NV; ++a) sRed[a][u] = v[a];
    __syncthreads();
    if (g == q - 1)
#pragma unroll
      for (int a = 0; a < NV; ++a) v[a] += sRed[a][u];
  }
}

template <int LIN, int NG, typename WT>
__global__ void __launch_bounds__(NC* NG) k_tp_fwd(int N, const int* __restrict__ rowptr,
                                                   const int* __restrict__ sender, const float* __restrict__ Y,
                                                   const float* __restrict__ Mt, int mts,
                                                   const WT* __restrict__ w, const float* __restrict__ up,
                                                   float* __restrict__ M, int half) {
  using T = TPT<LIN>;
  constexpr int DIN = NC * LIN * LIN, DMID = NC * T::NACC, WN = NC * T::NSLOT;
  const int n = blockIdx.x, g = group_id(), u = threadIdx.x % NC;
  float acc[T::NACC];
#pragma unroll
  for (int a = 0; a < T::NACC; ++a) acc[a] = 0.f;
  constexpr bool STAGE = LIN == 3;
  __shared__ float sM2[STAGE ? NSLICE * NG * 2 * M2PAD : 1];  // [wave][buffer][M2PAD]
  const int lane = threadIdx.x & 63;
  float* m2buf = sM2 + (STAGE ? (threadIdx.x >> 6) * 2 * M2PAD : 0);
  int gb, ge;
  group_range<NG>(rowptr[n], rowptr[n + 1], g, gb, ge);
  if (gb < ge) {
    EdgeIn<LIN> cur, nxt;
    M2Stage stg;
    load_w<LIN, true, WT>(w + (int64_t)gb * WN + u, cur.w);
    load_x<LIN>(up + (int64_t)sender[gb] * DIN + u, cur.x0, cur.x1, cur.x2);
    if constexpr (STAGE) {
      stg.load(Mt + (int64_t)gb * mts + MT_M2, lane);
      stg.store(m2buf, lane);
      wave_sync();
    }
    int buf = 0;
#pragma unroll 1
    for (int e = gb; e < ge; ++e) {
      if (e + 1 < ge) {
        load_w<LIN, true, WT>(w + (int64_t)(e + 1) * WN + u, nxt.w);
        load_x<LIN>(up + (int64_t)sender[e + 1] * DIN + u, nxt.x0, nxt.x1, nxt.x2);
        if constexpr (STAGE) stg.load(Mt + (int64_t)(e + 1) * mts + MT_M2, lane);
      }
      const float* Me = Mt + (int64_t)e * mts;
      tp_edge_fwd<LIN>(acc, cur, Y + (int64_t)e * 16, Me, STAGE ? m2buf + buf * M2PAD : Me + MT_M2);
      if constexpr (STAGE) {
        if (e + 1 < ge) {
          wave_sync();
          stg.store(m2buf + (buf ^ 1) * M2PAD, lane);
          wave_sync();
          buf ^= 1;
        }
      }
      cur = nxt;
    }
  }
  if constexpr (NG > 1) {
    __shared__ float sRed[T::NACC][NC];
    combine_groups<T::NACC, NG>(acc, g, u, sRed);
  }
  if (g == 0) {
    float* Mn = M + (int64_t)n * DMID + u;
#pragma unroll
    for (int a = 0; a < T::NACC; ++a) Mn[a * NC] = qh(acc[a], half);
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Sum over the 64 lanes of a wave of v[16]: lane l returns the total of
// component (l >> 2) & 15.  Recursive halving, all in VALU: each exchange step
// halves the components a lane keeps (the 32- and 16-lane exchanges with the
// permlane swaps of gfx950, the 8- and 4-lane ones with DPP), then two
// butterflies inside each quad finish the sum.
__device__ __forceinline__ float wave_sum16(const float* v) {
  const int lane = __lane_id();
  float a[8], b[4], c[2];
#pragma unroll
  for (int k = 0; k < 8; ++k) {  // lanes 0-31 keep component k, lanes 32-63 component k + 8
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 8]), false, false);
    a[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // rows 0 and 2 keep a[k], rows 1 and 3 a[k + 4]
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[k]), __float_as_uint(a[k + 4]), false, false);
    b[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  {
    const bool hi = lane & 8;  // partner lane ^ 8: rotation of the 16-lane row by 8
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float send = hi ? b[k] : b[k + 2], keep = hi ? b[k + 2] : b[k];
      c[k] = keep + dpp_f<0x128>(send);  // row_ror:8
    }
  }
  const bool hi = lane & 4;  // partner lane ^ 4: lane - 4 for the upper four of each eight, lane + 4 below
  const float send = hi ? c[0] : c[1], keep = hi ? c[1] : c[0];
  // both shifts run on the whole wave (a DPP read from a lane outside a divergent
  // branch would see 0), then each lane picks its partner's
  const float from_below = dpp_f<0x114>(send), from_above = dpp_f<0x104>(send);  // row_shr:4 / row_shl:4
  float d = keep + (hi ? from_below : from_above);
  d += dpp_f<0x4e>(d);  // quad_perm [2, 3, 0, 1]: lane ^ 2
  d += dpp_f<0xb1>(d);  // quad_perm [1, 0, 3, 2]: lane ^ 1
  return d;
}

// dL/dw of one edge and channel (all slots) into row gwe (stride NC).  GWT =
// float, or _Float16 under the float16 feature policy: each wave then scales
// its 64 channels x slots by a power of two that maps their largest magnitude
// into [2^14, 2^15) (so small gradients keep fp16 precision) and stores the
// inverse in gscale[e][slice].
template <int NSLOT, typename GWT>
__device__ __forceinline__ void store_gw(const float* gws, GWT* __restrict__ gwe, float* __restrict__ gscale,
                                         int64_t e, int u) {
  if constexpr (sizeof(GWT) == 4) {
#pragma unroll
    for (int s = 0; s < NSLOT; ++s) __builtin_nontemporal_store(gws[s], gwe + s * NC);
  } else {
    float m = 0.f;
#pragma unroll
    for (int s = 0; s < NSLOT; ++s) m = fmaxf(m, fabsf(gws[s]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    const int ex = m > 0.f ? ilogbf(m) : 0;
    const float sc = ldexpf(1.f, 14 - ex);
#pragma unroll
    for (int s = 0; s < NSLOT; ++s) gwe[s * NC] = (GWT)(gws[s] * sc);
    if ((u & 63) == 0) gscale[e * NSLICE + (u >> 6)] = ldexpf(1.f, ex - 14);
  }
}

// Store this wave's reduced dL/dY of edge e into gY[e][slice][16].
__device__ __forceinline__ void store_gY(const float* gYu, int64_t e, int u, float* __restrict__ gY, int accumulate) {
  const float s = wave_sum16(gYu);
  const int lane = __lane_id();
  if ((lane & 3) == 0) {
    float* dst = gY + e * 16 * NSLICE + (u >> 6) * 16 + (lane >> 2);
    *dst = accumulate ? *dst + s : s;
  }
}

// Per-edge VJP of one channel: given g = dL/dM[recv] (this channel), writes
// dL/dw, accumulates the input gradient (if GX) and this channel's dL/dY.
// bit j of CG1_MASK[i]: the l1 = 1 table row i (entries i*K1 .. i*K1 + 23) has a CG term in
// Y component j (a compile-time table, so the tests below fold away)
constexpr unsigned cg1_mask_row(int i) {
  unsigned m = 0;
  for (int q = i * TP3_K1; q < (i + 1) * TP3_K1; ++q)
    for (int x = TP3_M1_START[q]; x < TP3_M1_START[q + 1]; ++x) m |= 1u << TP3_M1_J[x];
  return m;
}
constexpr unsigned CG1_MASK[3] = {cg1_mask_row(0), cg1_mask_row(1), cg1_mask_row(2)};

template <int LIN, bool GX, int GRP = -1>
__device__ __forceinline__ void tp_edge_vjp(const float* g, const EdgeIn<LIN>& in, float* gw_out,
                                            const float* __restrict__ Ye, const float* __restrict__ Me,
                                            const float* M2, float& gx0, float* gx1, float* gx2, float* gYu) {
  using T = TPT<LIN>;
  // l1 = 1 slots: dL/dY_j = sum_i x1[i] u1[i][j] with u1[i][j] = sum_(s,k) w g C1[i, j, col(s) + k]
  // (the x1 factor taken out of the CG sums: one product per (i, j) pair, not one per term)
  constexpr bool L1SLOTS = LIN >= 2 && (GRP == -1 || GRP == 1);
  float u1[3][16];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) u1[i][j] = 0.f;
#pragma unroll
  for (int s = 0; s < T::NSLOT; ++s) {
    if (GRP >= 0 && T::l1(s) != GRP) continue;  // only the slots of input block l1 = GRP
    const float ww = in.w[s];
    const int a0 = T::acc(s), d = 2 * T::l3(s) + 1, l2 = T::l2(s);
    float gws = 0.f;
    if (T::l1(s) == 0) {
      float t = 0.f;
      const float xw = in.x0 * ww;
#pragma unroll
      for (int m = 0; m < d; ++m) {
        t = fmaf(g[a0 + m], Ye[l2 * l2 + m], t);
        gYu[l2 * l2 + m] = fmaf(xw, g[a0 + m], gYu[l2 * l2 + m]);
      }
      gws = in.x0 * t;
      if (GX) gx0 = fmaf(ww, t, gx0);
    } else if (T::l1(s) == 1) {
      const int c0 = T::col(s);
#pragma unroll
      for (int k = 0; k < d; ++k) {
        const float wg = ww * g[a0 + k];
        float mk = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const int q = i * T::K1 + c0 + k;
          const float mq = Me[q];
          mk = fmaf(in.x1[i], mq, mk);
          if (GX) gx1[i] = fmaf(wg, mq, gx1[i]);
#pragma unroll
          for (int x = m1s(q); x < m1s(q + 1); ++x) u1[i][m1j(x)] = fmaf(wg, m1v(x), u1[i][m1j(x)]);
        }
        gws = fmaf(g[a0 + k], mk, gws);
      }
    } else {
      const int c0 = T::col(s);
#pragma unroll
      for (int k = 0; k < d; ++k) {
        const float wg = ww * g[a0 + k];
        float mk = 0.f;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
          const int q = i * T::K2 + c0 + k;
          const float mq = M2[q];
          mk = fmaf(in.x2[i], mq, mk);
          if (GX) gx2[i] = fmaf(wg, mq, gx2[i]);
          const float cq = wg * in.x2[i];
#pragma unroll
          for (int x = m2s(q); x < m2s(q + 1); ++x) gYu[m2j(x)] = fmaf(cq, m2v(x), gYu[m2j(x)]);
        }
        gws = fmaf(g[a0 + k], mk, gws);
      }
    }
    gw_out[s] = gws;
    if constexpr (LIN == 3) __builtin_amdgcn_sched_barrier(0);  // as in tp_edge_fwd
  }
  if constexpr (L1SLOTS) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if ((CG1_MASK[i] >> j) & 1u) gYu[j] = fmaf(in.x1[i], u1[i][j], gYu[j]);
  }
}

// Receiver-centric VJP.  Node n's block walks its incoming edges with dL/dM[n]
// held in registers.  With GX the per-edge input gradient
//   gxe[pos_s[e]][l1^2 + i][u] = dL/dx[send(e), l1, i, u] restricted to edge e
// is stored in sender order (pos_s = inverse of the sender permutation), so
// k_tp_gather_gx sums each node's rows as one contiguous segment.  Without GX
// (first interaction: constant embedding input) only dL/dw and dL/dY are made.
template <int LIN, int NG, bool GX, typename WT>
__global__ void __launch_bounds__(NC* NG) k_tp_bwd_recv(int N, const int* __restrict__ rowptr,
                                                        const int* __restrict__ sender, const float* __restrict__ Y,
                                                        const float* __restrict__ Mt, int mts,
                                                        const WT* __restrict__ w, const float* __restrict__ up,
                                                        const float* __restrict__ gM, WT* __restrict__ gw,
                                                        float* __restrict__ gscale,
                                                        float* __restrict__ gY, int accumulate_gY,
                                                        const int* __restrict__ pos_s, float* __restrict__ gxe) {
  using T = TPT<LIN>;
  constexpr int DIN = NC * LIN * LIN, DMID = NC * T::NACC, WN = NC * T::NSLOT;
  const int n = blockIdx.x, g = group_id(), u = threadIdx.x % NC;
  int gb, ge;
  group_range<NG>(rowptr[n], rowptr[n + 1], g, gb, ge);
  if (gb >= ge) return;
  float gm[T::NACC];
  const float* gMn = gM + (int64_t)n * DMID + u;
#pragma unroll
  for (int a = 0; a < T::NACC; ++a) gm[a] = gMn[a * NC];
  constexpr bool STAGE = LIN == 3;
  __shared__ float sM2[STAGE ? NSLICE * NG * 2 * M2PAD : 1];  // [wave][buffer][M2PAD]
  const int lane = threadIdx.x & 63;
  float* m2buf = sM2 + (STAGE ? (threadIdx.x >> 6) * 2 * M2PAD : 0);
  EdgeIn<LIN> cur, nxt;
  M2Stage stg;
  load_w<LIN, true, WT>(w + (int64_t)gb * WN + u, cur.w);
  load_x<LIN>(up + (int64_t)sender[gb] * DIN + u, cur.x0, cur.x1, cur.x2);
  if constexpr (STAGE) {
    stg.load(Mt + (int64_t)gb * mts + MT_M2, lane);
    stg.store(m2buf, lane);
    wave_sync();
  }
  int buf = 0;
#pragma unroll 1
  for (int e = gb; e < ge; ++e) {
    if (e + 1 < ge) {
      load_w<LIN, true, WT>(w + (int64_t)(e + 1) * WN + u, nxt.w);
      load_x<LIN>(up + (int64_t)sender[e + 1] * DIN + u, nxt.x0, nxt.x1, nxt.x2);
      if constexpr (STAGE) stg.load(Mt + (int64_t)(e + 1) * mts + MT_M2, lane);
    }
    float gYu[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) gYu[j] = 0.f;
    float gx0 = 0.f, gx1[3] = {0.f, 0.f, 0.f}, gx2[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
    const float* Me = Mt + (int64_t)e * mts;
    float gws[T::NSLOT];
    tp_edge_vjp<LIN, GX>(gm, cur, gws, Y + (int64_t)e * 16, Me, STAGE ? m2buf + buf * M2PAD : Me + MT_M2, gx0,
                         gx1, gx2, gYu);
    store_gw<T::NSLOT>(gws, gw + (int64_t)e * WN + u, gscale, e, u);
    if constexpr (GX) {
      float* dst = gxe + (int64_t)pos_s[e] * DIN + u;
      dst[0] = gx0;
      if constexpr (LIN >= 2) {
#pragma unroll
        for (int i = 0; i < 3; ++i) dst[NC * (1 + i)] = gx1[i];
      }
      if constexpr (LIN >= 3) {
#pragma unroll
        for (int i = 0; i < 5; ++i) dst[NC * (4 + i)] = gx2[i];
      }
    }
    store_gY(gYu, e, u, gY, accumulate_gY);
    if constexpr (STAGE) {
      if (e + 1 < ge) {
        wave_sync();
        stg.store(m2buf + (buf ^ 1) * M2PAD, lane);
        wave_sync();
        buf ^= 1;
      }
    }
    cur = nxt;
  }
}

// gup[a][:] (= or +=, accumulate) the sum over the edges sent by a (a contiguous segment of the
// sender-ordered gxe rows, din entries each, summed in order into four interleaved partial sums,
// fp32).  GT: the rows' element type (fp16 under the float16 policy's fused VJP).  A wave per
// (atom, chunk of 64 VEC columns): lane l sums columns VEC (64 chunk + l) .. + VEC - 1 of the
// atom's rows with 16-byte loads (a whole 1 KB fp16 row per wave load), eight rows in flight.
template <typename GT>
__global__ void __launch_bounds__(256) k_tp_gather_gx(int N, int din, int nchunk, const int* __restrict__ rowptr_s,
                                                      const GT* __restrict__ gxe, float* __restrict__ gup,
                                                      int accumulate) {
  constexpr int VEC = 16 / sizeof(GT);
  typedef GT gv __attribute__((ext_vector_type(VEC)));
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int a = unit / nchunk, col = VEC * (64 * (unit % nchunk) + (threadIdx.x & 63));
  if (a >= N || col >= din) return;  // din is a multiple of 64: a lane's VEC columns are all in or all out
  const int beg = rowptr_s[a], end = rowptr_s[a + 1];
  const GT* src = gxe + col;
  auto row = [&](int k) { return *reinterpret_cast<const gv*>(src + (int64_t)k * din); };
  float s[4][VEC];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int v = 0; v < VEC; ++v) s[q][v] = 0.f;
  auto add = [&](int q, const gv& x) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) s[q][v] += (float)x[v];
  };
  int k = beg;
  for (; k + 7 < end; k += 8) {
    gv x[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) x[b] = row(k + b);
#pragma unroll
    for (int b = 0; b < 8; ++b) add(b & 3, x[b]);
  }
  for (; k + 3 < end; k += 4) {
    gv x[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) x[b] = row(k + b);
#pragma unroll
    for (int b = 0; b < 4; ++b) add(b, x[b]);
  }
  for (; k < end; ++k) add(0, row(k));
  float4* o = reinterpret_cast<float4*>(gup + (int64_t)a * din + col);
#pragma unroll
  for (int h = 0; h < VEC / 4; ++h) {
    float4 t;
    t.x = (s[0][4 * h] + s[1][4 * h]) + (s[2][4 * h] + s[3][4 * h]);
    t.y = (s[0][4 * h + 1] + s[1][4 * h + 1]) + (s[2][4 * h + 1] + s[3][4 * h + 1]);
    t.z = (s[0][4 * h + 2] + s[1][4 * h + 2]) + (s[2][4 * h + 2] + s[3][4 * h + 2]);
    t.w = (s[0][4 * h + 3] + s[1][4 * h + 3]) + (s[2][4 * h + 3] + s[3][4 * h + 3]);
    if (accumulate) {
      const float4 p = o[h];
      t.x += p.x, t.y += p.y, t.z += p.z, t.w += p.w;
    }
    o[h] = t;
  }
}

// ---------------------------------------------------------------------------
// Radial-MLP output layer fused into the TP forward (float32 policy).
//
// The per-edge weights w[e, slot, u] = wscale * h3inv[e] * sum_q h3[e, q] W3[q, slot NC + u]
// are made per 16-edge tile on the fp16 matrix cores with split operands
// (h3 as hi / lo planes scaled per edge, W3 as hi / lo planes scaled per matrix:
// lo.hi + hi.lo + hi.hi, the terms and order of k_mlp_out_x) straight into LDS,
// consumed there by the TP, and written out once for the VJP.
//
// Block = XW waves; wave k owns receiver XW * blockIdx.x + k and walks its
// edges two per step (small systems: spr waves per receiver, each walking a
// contiguous chunk of its edges; the chunks' sums are added in order at the
// end), lane = channel c0 + u of the block's 64-channel slice
// (blockIdx.y).  blockIdx.z selects the slots handled: those whose input block
// is one l1 (highest l1 first), so the groups read and write disjoint data.
// Tile column r = 2k + b holds edge b of wave k's current pair.  The W3 rows of
// the block's (slots, slice) stay in registers as MFMA A fragments (roles
// swapped: D[column 4g + i][edge r], so each lane writes four consecutive
// columns of one edge); wave k holds column tiles k, k + XW, ...  The tile is
// double-buffered, one barrier per step.
// ---------------------------------------------------------------------------
typedef float f4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f4v mfma16h(h8 a, h8 b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The per-edge weights w the fused forward keeps for its VJP: float, or under a half-precision
// feature policy the 16-bit pattern of the value it already holds (fp16, or the upper half of
// the fp32 pattern for bf16), exact either way: half the bytes of the largest per-edge stream.
template <int RND>
__device__ __forceinline__ void store_w(float* w, int64_t o, float x) {
  if constexpr (RND == RND_NONE) {
    __builtin_nontemporal_store(x, w + o);
  } else {
    const unsigned short h = RND == RND_F16 ? __builtin_bit_cast(unsigned short, (_Float16)x)
                                            : (unsigned short)(__float_as_uint(x) >> 16);
    __builtin_nontemporal_store(h, reinterpret_cast<unsigned short*>(w) + o);
  }
}
template <int RND>
__device__ __forceinline__ float load_w_nt(const float* w, int64_t o) {
  if constexpr (RND == RND_NONE) {
    return __builtin_nontemporal_load(w + o);
  } else {
    const unsigned short h = __builtin_nontemporal_load(reinterpret_cast<const unsigned short*>(w) + o);
    return RND == RND_F16 ? (float)__builtin_bit_cast(_Float16, h) : __uint_as_float((unsigned)h << 16);
  }
}

// The 16-bit pattern of a weight already rounded under a half-precision policy, and back
template <int RND>
__device__ __forceinline__ unsigned short w16_bits(float x) {
  return RND == RND_F16 ? __builtin_bit_cast(unsigned short, (_Float16)x) : (unsigned short)(__float_as_uint(x) >> 16);
}
template <int RND>
__device__ __forceinline__ float w16_value(unsigned short h) {
  return RND == RND_F16 ? (float)__builtin_bit_cast(_Float16, h) : __uint_as_float((unsigned)h << 16);
}

// Raw buffer views (stride 0): the hardware range check drops a store, and returns zero for a
// load, whose byte offset is at or past the view's size.  Padding lanes and past-the-end edges
// take an offset past every view (or a view of size 0), so the fused kernels' stores need no
// branch and no dummy target: every path issues the same memory operations (the compiler's
// wait counts stay exact) and no wave writes memory that another wave writes.
constexpr unsigned BUF_OOB = 0x80000000u;  // views are smaller than 2 GiB
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_view(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buf_store(float v, __amdgpu_buffer_rsrc_t r, unsigned off) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, 0);
}
__device__ __forceinline__ void buf_store4(float4 v, __amdgpu_buffer_rsrc_t r, unsigned off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), r,
                                         (int)off, 0, 0);
}
__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
// store_w through a view of one edge's row (element index o; aux 2 = nontemporal)
template <int RND>
__device__ __forceinline__ void store_w_buf(__amdgpu_buffer_rsrc_t r, unsigned o, float x) {
  if constexpr (RND == RND_NONE) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, (int)(4 * o), 0, 2);
  } else {
    const unsigned short h = RND == RND_F16 ? __builtin_bit_cast(unsigned short, (_Float16)x)
                                            : (unsigned short)(__float_as_uint(x) >> 16);
    __builtin_amdgcn_raw_buffer_store_b16(h, r, (int)(2 * o), 0, 2);
  }
}

constexpr int XW = 8;          // waves per fused block (receivers in flight)
// edges per wave and step in the fused forward (a step's tile: XW * EPW edges).  4 halves the
// steps and made the forward 2-4% faster, but the VJP that later reads the weights it wrote
// ran 5% slower (same code; only the order in which w reached memory differed): net loss
constexpr int EPW = 2;
constexpr int XH = RADIAL_H;   // radial hidden width (the contraction of the output layer)
static_assert(XH == 64, "two 32-wide k steps");

// the slots of one input block l1
template <int LIN, int L1>
struct GrpT {
  using T = TPT<LIN>;
  __host__ __device__ static constexpr int count() {
    int n = 0;
    for (int s = 0; s < T::NSLOT; ++s) n += T::l1(s) == L1 ? 1 : 0;
    return n;
  }
  static constexpr int G = count();
  // accumulator components of the group's slots
  __host__ __device__ static constexpr int acc_count() {
    int n = 0;
    for (int s = 0; s < T::NSLOT; ++s) n += T::l1(s) == L1 ? 2 * T::l3(s) + 1 : 0;
    return n;
  }
  // position of slot s among the group's slots
  __host__ __device__ static constexpr int local(int s) {
    int k = 0;
    for (int q = 0; q < s; ++q) k += T::l1(q) == L1 ? 1 : 0;
    return k;
  }
  // slot of group position si (compile-time si)
  __host__ __device__ static constexpr int slot_of(int si) {
    for (int s = 0; s < T::NSLOT; ++s)
      if (T::l1(s) == L1 && local(s) == si) return s;
    return 0;
  }
  // slot of group position si (run-time si: a select chain over the slots)
  __device__ static int slot(int si) {
    int res = 0;
#pragma unroll
    for (int s = 0; s < T::NSLOT; ++s)
      if (T::l1(s) == L1 && local(s) == si) res = s;
    return res;
  }
};

// largest group (LDS size of the fused kernels)
template <int LIN>
constexpr int gmax() {
  return LIN == 1   ? GrpT<1, 0>::G
         : LIN == 2 ? std::max(GrpT<2, 0>::G, GrpT<2, 1>::G)
                    : std::max({GrpT<3, 0>::G, GrpT<3, 1>::G, GrpT<3, 2>::G});
}
// entries of the per-edge table row an l1 group reads (Y itself for l1 = 0, M1 / M2 else),
// and that count rounded up to four (the row stride in LDS)
constexpr int tpx_tab(int l1) { return l1 == 0 ? 16 : l1 == 1 ? TP3_M1_NE : TP3_M2_NE; }
constexpr int tpx_tab_pad(int l1) { return (tpx_tab(l1) + 3) & ~3; }
// steps per w tile of the fused forward: two (one barrier per two steps) where the doubled LDS
// tile still leaves the block's occupancy unchanged (one input block runs two blocks per CU)
constexpr int tpx_fwd_steps(int lin) { return lin == 1 ? 1 : 2; }

// scalar parameters of the fused forward (pointers are passed separately, as
// __restrict__ kernel arguments: uniform loads through them then use the
// scalar cache)
struct TpxDims {
  int N, W, mts;
  int64_t E;
  float wscale;
  // non-linear interaction block (NL): w = (W3^T h3 + b3) cut, b3 [W], cut [E] (null: 1)
  const float* b3;
  const float* cut;
  // log2 of the waves per receiver (spr = 1, 2, 4 or 8; XW / spr receivers per block): a
  // receiver's edges split into spr contiguous chunks, one per wave, their message sums added
  // in chunk order at the end
  int sprl;
  // 0: w is not stored (the VJP rebuilds it from h3 and W3)
  int store_w;
};

#define MACE_TPX_FWD_PTRS                                                                                   \
  const int *__restrict__ rowptr, const int *__restrict__ sender, const float *__restrict__ Y,              \
      const float *__restrict__ Mt, const _Float16 *__restrict__ h3x, const float *__restrict__ h3inv,     \
      const _Float16 *__restrict__ W3Tx, const float *__restrict__ up, float *__restrict__ M,               \
      float *__restrict__ w
#define MACE_TPX_FWD_ARGS rowptr, sender, Y, Mt, h3x, h3inv, W3Tx, up, M, w
// h3x: [E][hi 64 | lo 64]; h3inv: [E]; W3Tx: [W][64] hi plane, then lo plane;
// w: [E][W] for the VJP

template <int LIN, int L1, int RND, bool NL>
__device__ __forceinline__ void tpx_fwd(const TpxDims& a, MACE_TPX_FWD_PTRS, float* sw, float* stab, _Float16* hbuf,
                                        float* hiv, float* hcv) {
  using T = TPT<LIN>;
  using GR = GrpT<LIN, L1>;
  constexpr int G = GR::G, CT = 4 * G, NCTW = (CT + XW - 1) / XW, RS = 64 * G + 4;
  constexpr int DIN = NC * LIN * LIN, DMID = NC * T::NACC, NX = 2 * L1 + 1;
  // steps per w tile (one barrier each), tile columns (edges) per tile, 16-column MFMA tiles
  constexpr int TPS = tpx_fwd_steps(LIN), TC = XW * EPW * TPS, NTC = TC / 16;
  // wave index through readfirstlane: receiver, edge indices and senders are then
  // wave-uniform scalars (scalar loads, no vector-memory waits on the prefetches)
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4, u = l;
  const int c0 = 64 * blockIdx.y, nb0 = (XW >> a.sprl) * blockIdx.x;  // XW / spr receivers per block
  // wave k: receiver nb0 + k / spr, chunk k % spr of its edges -> [wb, we)
  auto wave_range = [&](int k, int& wn, int& wb, int& we) {
    wn = nb0 + (k >> a.sprl);
    const int c = k & ((1 << a.sprl) - 1);
    const int rb = rowptr[min(wn, a.N)], re = wn < a.N ? rowptr[wn + 1] : rb;
    const int cnt = re - rb, csz = (cnt + (1 << a.sprl) - 1) >> a.sprl;
    wb = rb + min(cnt, c * csz);
    we = rb + min(cnt, (c + 1) * csz);
  };
  int n, beg, end;
  wave_range(wv, n, beg, end);
  int ns;
  {
    int nq, qb, qe;
    wave_range(l & (XW - 1), nq, qb, qe);  // lanes 0..7: the block's waves
    ns = (qe - qb + EPW - 1) / EPW;
  }
#pragma unroll
  for (int off = 1; off < XW; off <<= 1) ns = max(ns, __shfl_xor(ns, off));
  const int nsteps = __builtin_amdgcn_readfirstlane(ns);

  // Under a half-precision policy (RND) W3 and h3 hold rounded values: their lo planes are zero,
  // so a w tile is the one product hi.hi (the same sums: the skipped products add exact zeros)
  constexpr bool FULL = RND == RND_NONE;
  // half policies, two or three input blocks: the w tiles hold 16-bit patterns and only h3's hi
  // planes are staged (half the LDS: two blocks per CU)
  constexpr bool HT = !FULL && LIN >= 2;
  h8 wa[NCTW][2][FULL ? 2 : 1];  // [tile][k step][hi, lo]
#pragma unroll
  for (int m = 0; m < NCTW; ++m) {
    const int ct = wv + XW * m;
    if (CT % XW == 0 || ct < CT) {
      const int gc = 16 * ct + r;
      const int64_t col = (int64_t)GR::slot(gc >> 6) * NC + c0 + (gc & 63);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        wa[m][c][0] = *reinterpret_cast<const h8*>(W3Tx + col * XH + 32 * c + 8 * g);
        if constexpr (FULL) wa[m][c][FULL ? 1 : 0] = *reinterpret_cast<const h8*>(W3Tx + ((int64_t)a.W + col) * XH + 32 * c + 8 * g);
      }
    }
  }
  // NL: b3 of this lane's result rows (channels 16 ct + 4 g + i of the group's columns)
  float bw[NL ? NCTW : 1][4];
  if constexpr (NL) {
#pragma unroll
    for (int m = 0; m < NCTW; ++m) {
      const int ct = wv + XW * m;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gc = min(16 * ct + 4 * g + i, 64 * G - 1);  // rows of absent tiles: not used
        bw[m][i] = a.b3[GR::slot(gc >> 6) * NC + c0 + (gc & 63)];
      }
    }
  }
  const auto cutv = buf_view(a.cut, a.cut ? 4u * (unsigned)a.E : 0u);
  // Every vector-memory operation below is unconditional (indices clamped, stores
  // of past-the-end edges dropped by a buffer view of size 0), so the number in
  // flight is the same on every path and the compiler's wait counts stay exact: a
  // step waits only for what it consumes, never for the prefetches behind it.
  //
  // Two ring slots (the step loop is unrolled by two, so a slot is a set of
  // registers): slot j & 1 holds step j's inputs, and step j refills it for step
  // j + 2 once its edges are done; sender indices (scalar loads) are fetched a
  // step before the rows they address.
  const int64_t elast = a.E - 1;  // E >= 1 whenever a step runs
  constexpr int TS = tpx_tab(L1), TSP = tpx_tab_pad(L1), TH = (TS + 63) / 64;
  // entries of a table row a lane loads: l1 = 0, the Y row itself; l1 = 1, 2, Y component
  // l & 15, from which the M1 / M2 row is built in LDS
  constexpr int TL = L1 >= 1 ? 1 : TH;
  static_assert(TS <= 192 && L1 <= 2, "table rows of up to 192 entries");
  // this wave's table rows (Y for l1 = 0 slots, M1 for l1 = 1, M2 for l1 = 2), then its Y rows
  float* tb = stab + wv * EPW * TSP;
  float* yb = stab + XW * EPW * TSP + wv * EPW * 16;
  // l1 >= 1: the CG terms (at most two) of the table entries q = l + 64 h this lane builds
  int mj[TH][2];
  float mv[TH][2];
#pragma unroll
  for (int h = 0; h < TH; ++h) {
    const int q = min(l + 64 * h, TS - 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      mj[h][t] = L1 == 1 ? kM1Terms.j[q][t] : L1 == 2 ? kM2Terms.j[q][t] : 0;
      mv[h][t] = L1 == 1 ? kM1Terms.v[q][t] : L1 == 2 ? kM2Terms.v[q][t] : 0.f;
    }
  }
  // The TC h3 rows of a step's tile (hi and lo planes) are fetched once per block,
  // TC / 2 bytes per thread, and staged in LDS (double-buffered, written before the
  // barrier of the step before their use); each wave then reads its B fragments
  // from there.  Thread t fetches tile column hr, plane hpl, fp16 entries
  // HQ hq .. HQ hq + HQ - 1.
  static_assert(XW == 8 && (TC == 16 || TC == 32), "the h3 tile is fetched by 512 threads");
  constexpr int TPR = 512 / TC, HQ = 128 / TPR;  // threads per tile row; fp16 entries per thread
  typedef unsigned hv __attribute__((ext_vector_type(HQ / 2)));
  const int hr = threadIdx.x / TPR, hpl = (threadIdx.x % TPR) / (TPR / 2), hq = threadIdx.x % (TPR / 2);
  // tile column hr: step TPS t + hr / 16 of the tile, edge hr % EPW of wave (hr % 16) / EPW
  const int hs = hr / 16;
  int hb0;
  {
    int hn, hend;
    wave_range((hr % 16) / EPW, hn, hb0, hend);
  }
  struct HSlot {
    hv h;        // this thread's share of a tile's h3 rows
    float hinv;  // inverse scale of its row
    float cut;   // NL: its cutoff factor
  };
  HSlot H;
  struct Slot {
    float x[EPW][NX];   // sender rows of the wave's edges
    float t[EPW][TL];   // their table rows (this lane's entries; l1 = 1: Y components)
    int snd[EPW];       // sender indices
  };
  Slot s0, s1;
  auto load_snd = [&](int j, Slot& S) {
#pragma unroll
    for (int b = 0; b < EPW; ++b) S.snd[b] = sender[min<int64_t>(beg + EPW * j + b, elast)];
  };
  auto load_h = [&](int t) {  // tile t's share
    // columns past a receiver's end: not stored
    const int64_t row = min<int64_t>(hb0 + EPW * (TPS * t + hs) + hr % EPW, elast);
    // (half policies: the lo-plane threads fetch the hi row beside them, same cache lines)
    H.h = *reinterpret_cast<const hv*>(h3x + row * 2 * XH + (FULL ? hpl : 0) * XH + HQ * hq);
    H.hinv = h3inv[row];
    if constexpr (NL) H.cut = buf_load(cutv, 4u * (unsigned)row);  // 0 without a cut array
  };
  auto store_h = [&](int t) {  // H holds tile t's share (half policies: hi planes only)
    if (!HT || hpl == 0)
      *reinterpret_cast<hv*>(hbuf + (((t & 1) * (HT ? 1 : 2) + hpl) * TC + hr) * 72 + HQ * hq) = H.h;
    if (hpl == 0 && hq == 0) {
      hiv[(t & 1) * TC + hr] = H.hinv;
      if constexpr (NL) hcv[(t & 1) * TC + hr] = a.cut ? H.cut : 1.f;
    }
  };
  auto load_slot = [&](int j, Slot& S) {  // S.snd already holds step j's indices
#pragma unroll
    for (int b = 0; b < EPW; ++b) {
      const float* xs = up + (int64_t)S.snd[b] * DIN + NC * L1 * L1 + c0 + u;
#pragma unroll
      for (int i = 0; i < NX; ++i) S.x[b][i] = xs[NC * i];
      const int64_t e = min<int64_t>(beg + EPW * j + b, elast);
      if constexpr (L1 >= 1) {
        S.t[b][0] = Y[e * 16 + (l & 15)];
      } else {
#pragma unroll
        for (int h = 0; h < TH; ++h) S.t[b][h] = Y[e * 16 + min(l + 64 * h, TS - 1)];
      }
    }
  };
  float acc[T::NACC];
#pragma unroll
  for (int q = 0; q < T::NACC; ++q) acc[q] = 0.f;
  // w tile t (the columns of steps TPS t .. TPS t + TPS - 1): this wave's column tiles of
  // W3^T h3, from the h3 rows staged in hbuf t & 1, into LDS buffer t & 1
  auto products = [&](int t) {
    float* tile = sw + (t & 1) * TC * RS;
    unsigned short* tile16 = reinterpret_cast<unsigned short*>(sw) + (t & 1) * TC * RS;
#pragma unroll
    for (int t2 = 0; t2 < NTC; ++t2) {
      h8 bx[2][2];  // B fragments of tile column 16 t2 + r: [k step][hi, lo]
      const int col = 16 * t2 + r;
      const _Float16* hrow = hbuf + ((t & 1) * (HT ? 1 : 2) * TC + col) * 72 + 8 * g;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        bx[c][0] = *reinterpret_cast<const h8*>(hrow + 32 * c);
        if constexpr (FULL) bx[c][1] = *reinterpret_cast<const h8*>(hrow + TC * 72 + 32 * c);
      }
      f4v d[NCTW];
#pragma unroll
      for (int m = 0; m < NCTW; ++m) d[m] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int p = FULL ? 0 : 2; p < 3; ++p)
#pragma unroll
          for (int m = 0; m < NCTW; ++m)
            if (CT % XW == 0 || wv + XW * m < CT)  // every wave's tiles exist when XW divides CT
              d[m] = mfma16h(wa[m][c][p == 2 ? 0 : (p ^ 1) & (FULL ? 1 : 0)],
                             bx[c][p == 1 ? 1 : 0], d[m]);  // lo.hi, hi.lo, hi.hi
      const float bsc = hiv[(t & 1) * TC + col] * a.wscale;
      if constexpr (NL) {
        const float cc = hcv[(t & 1) * TC + col];
#pragma unroll
        for (int m = 0; m < NCTW; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i) d[m][i] = fmaf(d[m][i], bsc, bw[m][i]) * cc;
      } else {
#pragma unroll
        for (int m = 0; m < NCTW; ++m) d[m] *= bsc;
      }
#pragma unroll
      for (int m = 0; m < NCTW; ++m) {
        const int ct = wv + XW * m;
        if (CT % XW == 0 || ct < CT) {
          if constexpr (!HT) {
            *reinterpret_cast<float4*>(tile + col * RS + 16 * ct + 4 * g) =
                float4{qh(d[m][0], RND), qh(d[m][1], RND), qh(d[m][2], RND), qh(d[m][3], RND)};
          } else {  // the rounded values as 16-bit patterns
            typedef unsigned short us4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<us4*>(tile16 + col * RS + 16 * ct + 4 * g) =
                us4{w16_bits<RND>(qh(d[m][0], RND)), w16_bits<RND>(qh(d[m][1], RND)),
                    w16_bits<RND>(qh(d[m][2], RND)), w16_bits<RND>(qh(d[m][3], RND))};
          }
        }
      }
    }
  };
  // tile t: its products, the next tile's h3 rows staged (their last readers, products(t - 1),
  // are past the previous barrier) and the one after fetched, then the barrier that publishes it
  auto tile_begin = [&](int t) {
    products(t);
    store_h(t + 1);
    load_h(t + 2);
    __syncthreads();
  };
  // the channel-wise TP of the wave's edges of step j (w tile j / TPS) and the w stores
  auto edges = [&](int j, Slot& S, Slot& Snext) {
    // half policies: 16-bit patterns, TC RS of them per tile
    const float* tile = sw + ((j / TPS) & 1) * TC * RS;
    const unsigned short* tile16 = reinterpret_cast<const unsigned short*>(sw) + ((j / TPS) & 1) * TC * RS;
    if constexpr (L1 >= 1) {  // M1 / M2 rows from the Y rows: the terms and order of k_edge_fwd
#pragma unroll
      for (int b = 0; b < EPW; ++b)
        if (l < 16) yb[16 * b + l] = S.t[b][0];
      wave_sync();
#pragma unroll
      for (int b = 0; b < EPW; ++b)
#pragma unroll
        for (int h = 0; h < TH; ++h)
          if (l + 64 * h < TS)
            tb[b * TSP + l + 64 * h] =
                fmaf(yb[16 * b + mj[h][1]], mv[h][1], fmaf(yb[16 * b + mj[h][0]], mv[h][0], 0.f));
    } else {
#pragma unroll
      for (int b = 0; b < EPW; ++b)
#pragma unroll
        for (int h = 0; h < TH; ++h)
          if (l + 64 * h < TS) tb[b * TSP + l + 64 * h] = S.t[b][h];
    }
    wave_sync();
    load_snd(j + 3, Snext);  // Snext's step j + 1 rows are already in flight
#pragma unroll
    for (int b = 0; b < EPW; ++b) {
      const int e = beg + EPW * j + b;
      const bool valid = e < end;
      float wv_s[T::NSLOT];
      const int ro = (16 * (j % TPS) + EPW * wv + b) * RS + u;
      const float* trow = tile + ro;
      const unsigned short* trow16 = tile16 + ro;
#pragma unroll
      for (int s = 0; s < T::NSLOT; ++s)
        if (T::l1(s) == L1) wv_s[s] = HT ? w16_value<RND>(trow16[64 * GR::local(s)]) : trow[64 * GR::local(s)];
      if (valid) {
        EdgeIn<LIN> in;
        in.x0 = 0.f;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
          if constexpr (L1 == 0) in.x0 = S.x[b][i];
          if constexpr (L1 == 1) in.x1[i] = S.x[b][i];
          if constexpr (L1 == 2) in.x2[i] = S.x[b][i];
        }
#pragma unroll
        for (int s = 0; s < T::NSLOT; ++s)
          if (T::l1(s) == L1) in.w[s] = wv_s[s];
        const float* trow_t = tb + b * TSP;  // Y (l1 = 0), M1 (l1 = 1) or M2 (l1 = 2)
        tp_edge_fwd<LIN, L1>(acc, in, trow_t, trow_t, trow_t);
      }
      if (a.store_w) {
        constexpr unsigned WB = RND == RND_NONE ? 4 : 2;  // bytes per stored weight
        const auto wr = buf_view(reinterpret_cast<char*>(w) + (int64_t)min<int64_t>(e, elast) * a.W * WB,
                                 valid ? (unsigned)a.W * WB : 0u);
#pragma unroll
        for (int s = 0; s < T::NSLOT; ++s)
          if (T::l1(s) == L1) store_w_buf<RND>(wr, (unsigned)(c0 + u + s * NC), wv_s[s]);
      }
    }
    wave_sync();  // table row reads done before the next step's store
    load_slot(j + 2, S);  // S.snd was refilled with step j + 2's indices during step j - 1
  };
  const int nsteps2 = (nsteps + 1) & ~1;  // even: both ring slots every trip (TPS divides it)
  if (nsteps2 > 0) {
    load_snd(0, s0);
    load_snd(1, s1);
    load_h(0);
    load_slot(0, s0);
    load_slot(1, s1);
    load_snd(2, s0);
    store_h(0);
    load_h(1);
    __syncthreads();  // nsteps2 is uniform over the block
  }
#pragma unroll 1
  for (int j = 0; j < nsteps2; j += 2) {
    tile_begin(j / TPS);
    edges(j, s0, s1);
    if constexpr (TPS == 1) tile_begin(j + 1);
    edges(j + 1, s1, s0);
  }
  if (a.sprl > 0) {  // uniform: the chunks' sums through LDS (the w tile buffer), in chunk order
    constexpr int GA = GR::acc_count();
    static_assert((XW - 1) * GA * 64 <= (HT ? 1 : 2) * TC * RS, "chunk partials fit the w tile buffer");
    __syncthreads();  // every wave is done with the tiles
    const int c = wv & ((1 << a.sprl) - 1);
    if (c > 0) {
      float* part = sw + ((wv - 1) * GA) * 64 + u;
      int q = 0;
#pragma unroll
      for (int s = 0; s < T::NSLOT; ++s)
        if (T::l1(s) == L1)
#pragma unroll
          for (int m = 0; m < 2 * T::l3(s) + 1; ++m) part[64 * q++] = acc[T::acc(s) + m];
    }
    __syncthreads();
    if (c == 0)
      for (int k = 1; k < (1 << a.sprl); ++k) {
        const float* part = sw + ((wv + k - 1) * GA) * 64 + u;
        int q = 0;
#pragma unroll
        for (int s = 0; s < T::NSLOT; ++s)
          if (T::l1(s) == L1)
#pragma unroll
            for (int m = 0; m < 2 * T::l3(s) + 1; ++m) acc[T::acc(s) + m] += part[64 * q++];
      }
  }
  if (n < a.N && (wv & ((1 << a.sprl) - 1)) == 0) {
    float* Mn = M + (int64_t)n * DMID + c0 + u;
#pragma unroll
    for (int s = 0; s < T::NSLOT; ++s)
      if (T::l1(s) == L1)
#pragma unroll
        for (int m = 0; m < 2 * T::l3(s) + 1; ++m) Mn[NC * (T::acc(s) + m)] = qh(acc[T::acc(s) + m], RND);
  }
}

// RND: rounding mode of w and M under a half-precision feature policy (the split operands
// of rounded h3 and weights have zero lo planes, so w is the float32 product, then rounded)
template <int LIN, int RND, bool NL>
// two input blocks under a half policy, standard interaction block: 64 KB of LDS and at most 128
// VGPRs (a few spilled), two blocks per CU (the non-linear block's epilogue would spill more)
__global__ void __launch_bounds__(64 * XW, RND != RND_NONE && LIN == 2 && !NL ? 4 : 2) k_tpx_fwd(TpxDims a, MACE_TPX_FWD_PTRS) {
  constexpr int TC = XW * EPW * tpx_fwd_steps(LIN);
  constexpr int NPL = RND == RND_NONE || LIN == 1 ? 2 : 1;  // 1: 16-bit w tiles, h3 hi planes only
  __shared__ __align__(16) float sw[NPL * TC * (64 * gmax<LIN>() + 4)];  // [tile][column][RS]
  __shared__ __align__(16) float stab[XW * EPW * (tpx_tab_pad(LIN - 1) + 16)];  // table rows + Y rows
  __shared__ __align__(16) _Float16 hbuf[2 * NPL * TC * 72];  // [tile][hi, lo][tile column][64 + pad]
  __shared__ float hiv[2 * TC];
  __shared__ float hcv[NL ? 2 * TC : 1];  // NL: the tile columns' cutoff factors
  if constexpr (LIN == 1) {
    tpx_fwd<1, 0, RND, NL>(a, MACE_TPX_FWD_ARGS, sw, stab, hbuf, hiv, hcv);
  } else if constexpr (LIN == 2) {
    if (blockIdx.z == 0)
      tpx_fwd<2, 1, RND, NL>(a, MACE_TPX_FWD_ARGS, sw, stab, hbuf, hiv, hcv);
    else
      tpx_fwd<2, 0, RND, NL>(a, MACE_TPX_FWD_ARGS, sw, stab, hbuf, hiv, hcv);
  } else {
    if (blockIdx.z == 0)
      tpx_fwd<3, 2, RND, NL>(a, MACE_TPX_FWD_ARGS, sw, stab, hbuf, hiv, hcv);
    else if (blockIdx.z == 1)
      tpx_fwd<3, 1, RND, NL>(a, MACE_TPX_FWD_ARGS, sw, stab, hbuf, hiv, hcv);
    else
      tpx_fwd<3, 0, RND, NL>(a, MACE_TPX_FWD_ARGS, sw, stab, hbuf, hiv, hcv);
  }
}

// ---------------------------------------------------------------------------
// TP VJP with the radial-MLP output layer's backward product fused in.
//
// Same decomposition as the fused forward (wave = receiver, 64-channel slice,
// one input degree l1 per block).  A step runs the per-edge VJP of the wave's
// two edges (dL/dw, dL/dx, dL/dY), stores dL/dw into the block's 16-edge LDS
// tile, and after the barrier multiplies the tile by the block's W3 rows on
// the fp16 matrix cores:
//   gh3p[p][e][q] = wscale * sum_{slot in group, u in slice} dL/dw[e, slot, u] W3[q, slot NC + u]
// with split operands (W3 as hi / lo planes scaled per matrix; dL/dw split
// once, by the wave that made it, after scaling the edge's largest magnitude
// over the block's columns into [2^14, 2^15): its hi / lo planes and inverse
// scale go to LDS; lo.hi + hi.lo + hi.hi).  p = NSLICE blockIdx.z + blockIdx.y indexes
// the (group, slice) partials; the hidden-layer VJP adds them in order.
// Roles are swapped (D[q][edge]); wave k takes q tile k & 3 and half k >> 2 of
// the group's k steps, holding those W3 fragments in registers; the two halves
// of a q tile meet through LDS one step later (no second barrier).
// dL/dY partials go to gY[e][p][16] and dL/dx rows to gxe[pos_s[e]] (this
// group's components, this slice's channels; fp16 values under the float16
// policy, which halves the largest per-edge stream the VJP writes).  As in the forward, every load
// is unconditional (clamped indices); stores of padding edges are skipped.
// ---------------------------------------------------------------------------
// l1 = 1 slots of a receiver-centric VJP, refactored around what stays fixed while a
// wave walks one receiver's edges: g = dL/dM[recv] (per channel) and the CG tables B
// (CG x path weight, Me[i][col] = sum_j Y_j B[j, i, col]).  With the per-receiver table
//   R[s][i][j] = sum_(k in s) g[col_s + k] B[j, i, col_s + k]        (vjp_l1_table)
// the per-edge VJP is one bilinear form in (x1 w, Y):
//   h[i][s]   = sum_(k in s) g[col_s + k] Me[i][col_s + k] = sum_j Y_j R[s][i][j]
//   dL/dw[s]  = sum_i x1[i] h[i][s],  dL/dx1[i] += sum_s w[s] h[i][s]
//   dL/dY_j  += sum_(s, i) x1[i] w[s] R[s][i][j]
// two products per nonzero (s, i, j) instead of the per-edge CG sums over (i, k, terms)
// of tp_edge_vjp, and no per-edge M1 table.  R is held in registers (its zero pattern is
// compile-time).
// bit j: row i of the M1 table has a CG term in Y component j in one of the columns
// [col, col + d) (one slot); folded to a constant where the arguments are
__device__ constexpr unsigned rmask(int col, int d, int i) {
  unsigned m = 0;
  for (int k = 0; k < d; ++k) {
    const int q = i * TP3_K1 + col + k;
    for (int x = m1s(q); x < m1s(q + 1); ++x) m |= 1u << m1j(x);
  }
  return m;
}

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>): loop indices that are
// constants by construction (a register array indexed by them never needs memory, whatever
// the unroller decides for a long loop)
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

template <int LIN>
__device__ __forceinline__ void vjp_l1_table(const float* g, float (*R)[3][16]) {
  using T = TPT<LIN>;
  using GR = GrpT<LIN, 1>;
  static_for<GR::G>([&](auto lsc) {
    constexpr int ls = decltype(lsc)::value, s = GR::slot_of(ls);
    constexpr int a0 = T::acc(s), d = 2 * T::l3(s) + 1, c0 = T::col(s);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
      for (int j = 0; j < 16; ++j) R[ls][i][j] = 0.f;
#pragma unroll
      for (int k = 0; k < d; ++k) {
        const int q = i * T::K1 + c0 + k;
#pragma unroll
        for (int x = m1s(q); x < m1s(q + 1); ++x) R[ls][i][m1j(x)] = fmaf(g[a0 + k], m1v(x), R[ls][i][m1j(x)]);
      }
    }
  });
}

template <int LIN, bool GX>
__device__ __forceinline__ void tp_edge_vjp_l1(const float (*R)[3][16], const EdgeIn<LIN>& in, float* gw_out,
                                               const float* Ye, float* gx1, float* gYu) {
  using T = TPT<LIN>;
  using GR = GrpT<LIN, 1>;
  static_for<GR::G>([&](auto lsc) {
    constexpr int ls = decltype(lsc)::value, s = GR::slot_of(ls);
    constexpr int d = 2 * T::l3(s) + 1, c0 = T::col(s);
    const float ww = in.w[s];
    float gws = 0.f;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const unsigned mask = rmask(c0, d, i);
      float h = 0.f;  // sum_k g[col_s + k] Me[i][col_s + k] = sum_j Y_j R[s][i][j]
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if ((mask >> j) & 1u) h = fmaf(Ye[j], R[ls][i][j], h);
      gws = fmaf(in.x1[i], h, gws);
      if (GX) gx1[i] = fmaf(ww, h, gx1[i]);
      const float z = in.x1[i] * ww;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if ((mask >> j) & 1u) gYu[j] = fmaf(z, R[ls][i][j], gYu[j]);
    }
    gw_out[s] = gws;
  });
}

// Largest value of a nonnegative x over the wave (DPP row scan, then the two
// row broadcasts; lane 63 ends with the total), as a wave-uniform value.  The
// scan runs on the bit patterns, whose unsigned order is that of nonnegative
// floats: unsigned max needs no NaN canonicalisation and fuses with the DPP
// move (lanes without a source read 0, the identity).
template <int CTRL>
__device__ __forceinline__ unsigned dpp_u(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, true);
}
__device__ __forceinline__ float wave_max_nonneg(float x) {
  unsigned m = __float_as_uint(x);
  m = max(m, dpp_u<0x111>(m));  // row_shr:1
  m = max(m, dpp_u<0x112>(m));  // row_shr:2
  m = max(m, dpp_u<0x114>(m));  // row_shr:4
  m = max(m, dpp_u<0x118>(m));  // row_shr:8
  m = max(m, dpp_u<0x142>(m));  // row_bcast:15
  m = max(m, dpp_u<0x143>(m));  // row_bcast:31
  return __uint_as_float((unsigned)__builtin_amdgcn_readlane((int)m, 63));
}
// Sum of x over the wave, in lane 63 (the same DPP scan: row prefix sums, then the two row
// broadcasts; lanes without a source add 0).  Fixed order, so the result is deterministic.
__device__ __forceinline__ float wave_sum_lane63(float x) {
  x += dpp_f<0x111>(x);  // row_shr:1
  x += dpp_f<0x112>(x);  // row_shr:2
  x += dpp_f<0x114>(x);  // row_shr:4
  x += dpp_f<0x118>(x);  // row_shr:8
  x += dpp_f<0x142>(x);  // row_bcast:15
  x += dpp_f<0x143>(x);  // row_bcast:31
  return x;
}

struct TpxBwdDims {
  int N, W, mts;
  int64_t E;
  float wscale;
  int accumulate_gY;
  int gyp;  // partials per edge in gY
  // non-linear interaction block (NL): gwbp[p][e] = sum over partial p's columns k of
  // dL/dw[e][k] b3[k] (b3 [W], gwbp [P][E])
  const float* b3;
  float* gwbp;
  // log2 of the waves per receiver (spr = 1, 2, 4 or 8; XW / spr receivers per block): a
  // receiver's edges split into spr contiguous chunks, one per wave, so that a small system's
  // few receivers fill the chip (the VJP of an edge depends on its receiver's dL/dM only:
  // nothing to combine)
  int sprl;
};

#define MACE_TPX_BWD_PTRS                                                                                   \
  const int *__restrict__ rowptr, const int *__restrict__ sender, const float *__restrict__ Y,              \
      const float *__restrict__ Mt, const float *__restrict__ w, const _Float16 *__restrict__ W3x,           \
      const float *__restrict__ up, const float *__restrict__ gM, const int *__restrict__ pos_s,            \
      float *__restrict__ gxe, float *__restrict__ gY, float *__restrict__ gh3p,                            \
      const _Float16 *__restrict__ h3x, const float *__restrict__ h3inv, const _Float16 *__restrict__ W3Tx
#define MACE_TPX_BWD_ARGS rowptr, sender, Y, Mt, w, W3x, up, gM, pos_s, gxe, gY, gh3p, h3x, h3inv, W3Tx
// W3x: [64][W] hi plane, then lo plane; gh3p: [P][E][64]; with RW, h3x / h3inv / W3Tx as the
// forward reads them (w is then not read)

template <int LIN, int L1, bool GX, int WF, bool NL, bool RW>
__device__ __forceinline__ void tpx_bwd(const TpxBwdDims& a, MACE_TPX_BWD_PTRS, _Float16* sg, float* sinv,
                                        float* sy, float* sp, float* sm2, _Float16* hbuf, float* hiv) {
  using T = TPT<LIN>;
  using GR = GrpT<LIN, L1>;
  constexpr int G = GR::G, RS = 64 * G + 8;  // fp16 row stride: 16-byte reads of 8 lanes hit distinct banks
  constexpr int DIN = NC * LIN * LIN, DMID = NC * T::NACC, NX = 2 * L1 + 1;
  static_assert(L1 <= 2, "input blocks l1 = 0, 1, 2");
  // l1 = 2: the CG terms (at most two) of the M2 entries q = l + 64 h this lane builds from the
  // step's Y rows (into sm2: this wave's two rows)
  constexpr int M2H = L1 == 2 ? (TP3_M2_NE + 63) / 64 : 1, M2S = tpx_tab_pad(2);
  int m2j_[M2H][2];
  float m2v_[M2H][2];
#pragma unroll
  for (int h = 0; h < M2H; ++h) {
    const int q = min((int)(threadIdx.x & 63) + 64 * h, TP3_M2_NE - 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      m2j_[h][t] = L1 == 2 ? kM2Terms.j[q][t] : 0;
      m2v_[h][t] = L1 == 2 ? kM2Terms.v[q][t] : 0.f;
    }
  }
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4, u = l;
  const int rpb = XW >> a.sprl;  // receivers per block
  const int c0 = 64 * blockIdx.y, nb0 = rpb * blockIdx.x, p = NSLICE * blockIdx.z + blockIdx.y;
  // wave k: receiver nb0 + k / spr, chunk k % spr of its edges -> [wb, we)
  auto wave_range = [&](int k, int& wn, int& wb, int& we) {
    wn = nb0 + (k >> a.sprl);
    const int c = k & ((1 << a.sprl) - 1);
    const int rb = rowptr[min(wn, a.N)], re = wn < a.N ? rowptr[wn + 1] : rb;
    const int cnt = re - rb, csz = (cnt + (1 << a.sprl) - 1) >> a.sprl;
    wb = rb + min(cnt, c * csz);
    we = rb + min(cnt, (c + 1) * csz);
  };
  int n, beg, end;
  wave_range(wv, n, beg, end);
  int nr, cb, ce;
  wave_range(r >> 1, nr, cb, ce);  // the wave whose edges are tile columns r
  int ns = (ce - cb + 1) >> 1;
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) ns = max(ns, __shfl_xor(ns, off));
  const int nsteps = __builtin_amdgcn_readfirstlane(ns);
  const int64_t elast = a.E - 1;
  // the block's edges [eb0, eb1) (its receivers' rows): a view of their dL/dh3 partial rows p
  const int eb0 = rowptr[min(nb0, a.N)], eb1 = rowptr[min(nb0 + rpb, a.N)];
  const auto gh3v = buf_view(gh3p + ((int64_t)p * a.E + eb0) * XH, 4u * XH * (unsigned)(eb1 - eb0));
  // NL: the block's entries of gw . b3 partial p, and b3 of this lane's channel in the group slots
  const auto gwbv = buf_view(NL ? a.gwbp + (int64_t)p * a.E + eb0 : nullptr, NL ? 4u * (unsigned)(eb1 - eb0) : 0u);
  float b3c[NL ? T::NSLOT : 1];
  if constexpr (NL) {
#pragma unroll
    for (int s = 0; s < T::NSLOT; ++s)
      if (T::l1(s) == L1) b3c[s] = a.b3[s * NC + c0 + u];
  }

  // W3 rows q = 16 qt + r, group k steps kh G .. kh G + G - 1 (32 columns each).  Under a
  // half-precision policy (WF) W3 holds rounded values: its lo plane is zero and the product
  // lo.hi is skipped (it adds exact zeros); dL/dw is carried as one fp16 value (scaled per edge),
  // as the reference's half-precision gradients are, so hi.hi is the only product.  The float32
  // policy splits both operands: lo.hi + hi.lo + hi.hi
  constexpr bool WLO = WF == RND_NONE;
  const int qt = wv & 3, kh = wv >> 2;
  h8 wa[G][WLO ? 2 : 1];
#pragma unroll
  for (int ks = 0; ks < G; ++ks) {
    const int kk = kh * G + ks;
    const int64_t o = (int64_t)(16 * qt + r) * a.W + GR::slot(kk >> 1) * NC + c0 + 32 * (kk & 1) + 8 * g;
    wa[ks][0] = *reinterpret_cast<const h8*>(W3x + o);
    if constexpr (WLO) wa[ks][WLO ? 1 : 0] = *reinterpret_cast<const h8*>(W3x + (int64_t)XH * a.W + o);
  }
  // RW (half-precision policies, one or two input blocks, standard interactions): w is not
  // read back but rebuilt per pair of steps, 32 edges, from their h3 rows and W3^T with the
  // forward's operands, products and epilogue (the values the forward used, bit for bit), into
  // the lo-plane half of the pair's sg buffer (the dL/dw tile has one plane under these
  // policies).  The tile of pair t + 1 is made during pair t (published by the barrier that ends
  // it) from h3 rows staged in LDS during pair t - 1 and fetched during pair t - 2.
  static_assert(!RW || (!WLO && LIN <= 2 && !NL), "w is rebuilt under the half policies only");
  constexpr int CT = 4 * G, NCTW = (CT + XW - 1) / XW;  // 16-column tiles of the group, per wave
  h8 wt[RW ? NCTW : 1][2];  // W3^T fragments: [column tile][k step]
  // h3 staging: threads 0 .. 255 (the lower half) fetch eight fp16 each of tile column hr
  // (pair-relative)
  const int hr = (threadIdx.x >> 3) & 31, hq = threadIdx.x & 7;
  int hb0 = 0;
  h8 hreg;
  float hinvr = 0.f;
  if constexpr (RW) {
#pragma unroll
    for (int m = 0; m < NCTW; ++m) {
      const int ct = wv + XW * m;
      if (CT % XW == 0 || ct < CT) {
        const int gc = 16 * ct + r;
        const int64_t col = (int64_t)GR::slot(gc >> 6) * NC + c0 + (gc & 63);
#pragma unroll
        for (int c = 0; c < 2; ++c) wt[m][c] = *reinterpret_cast<const h8*>(W3Tx + col * XH + 32 * c + 8 * g);
      }
    }
    int hn, hend;
    wave_range((hr % 16) >> 1, hn, hb0, hend);  // tile column hr: edge hr & 1 of wave (hr % 16) / 2
  }
  // pair t's h3 rows: tile column hr is step 2 t + hr / 16 of its wave
  auto load_h = [&](int t) {
    const int64_t row = min<int64_t>(hb0 + 2 * (2 * t + hr / 16) + (hr & 1), elast);
    hreg = *reinterpret_cast<const h8*>(h3x + row * 2 * XH + 8 * hq);  // the hi plane
    hinvr = h3inv[row];
  };
  auto store_h = [&](int t) {
    if (threadIdx.x < 256) {
      *reinterpret_cast<h8*>(hbuf + ((t & 1) * 32 + hr) * 72 + 8 * hq) = hreg;
      if (hq == 0) hiv[(t & 1) * 32 + hr] = hinvr;
    }
  };
  // w tile t: this wave's column tiles of W3^T h3 for the pair's two 16-edge halves (the
  // forward's hi.hi products over two k steps, scale, rounding), as 16-bit patterns, in three
  // stages that the step loop spreads over a pair of steps (each stage's latency hidden behind
  // an edge step): the B fragments and scales from LDS, the products, the epilogue and store
  struct WtStage {
    h8 bx[2][2];      // [half][k step]
    f4v d[2][NCTW];   // [half][column tile]
    float bsc[2];
  };
  WtStage wsg;
  auto wt_read = [&](int t) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int col = 16 * h + r;
      const _Float16* hrow = hbuf + ((t & 1) * 32 + col) * 72 + 8 * g;
#pragma unroll
      for (int c = 0; c < 2; ++c) wsg.bx[h][c] = *reinterpret_cast<const h8*>(hrow + 32 * c);
      wsg.bsc[h] = hiv[(t & 1) * 32 + col] * a.wscale;
    }
  };
  auto wt_mma = [&]() {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int m = 0; m < NCTW; ++m) wsg.d[h][m] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int m = 0; m < NCTW; ++m)
          if (CT % XW == 0 || wv + XW * m < CT) wsg.d[h][m] = mfma16h(wt[m][c], wsg.bx[h][c], wsg.d[h][m]);
    }
  };
  auto wt_store = [&](int t) {
    _Float16* wb = sg + ((t & 1) * 2 + 1) * 32 * RS;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int col = 16 * h + r;
#pragma unroll
      for (int m = 0; m < NCTW; ++m) {
        const int ct = wv + XW * m;
        if (CT % XW == 0 || ct < CT) {
          const f4v d = wsg.d[h][m] * wsg.bsc[h];
          typedef unsigned short us4 __attribute__((ext_vector_type(4)));
          const us4 v = {w16_bits<WF>(qh(d[0], WF)), w16_bits<WF>(qh(d[1], WF)), w16_bits<WF>(qh(d[2], WF)),
                         w16_bits<WF>(qh(d[3], WF))};
          *reinterpret_cast<us4*>(wb + col * RS + 16 * ct + 4 * g) = v;
        }
      }
    }
  };
  // dL/dM of this wave's receiver (group slots, slice channels); for l1 = 1 only through
  // its CG contraction R (tp_edge_vjp_l1)
  float gm[T::NACC];
  {
    const float* gMn = gM + (int64_t)min(n, a.N - 1) * DMID + c0 + u;
#pragma unroll
    for (int s = 0; s < T::NSLOT; ++s)
      if (T::l1(s) == L1)
#pragma unroll
        for (int m = 0; m < 2 * T::l3(s) + 1; ++m) gm[T::acc(s) + m] = gMn[NC * (T::acc(s) + m)];
  }
  float R1[L1 == 1 ? G : 1][3][16];
  if constexpr (L1 == 1) vjp_l1_table<LIN>(gm, R1);
  // A step's inputs: weights, sender rows, Y components, pos_s and the dL/dY partials already
  // held (accumulate_gY) of its two edges, loaded a step ahead (indices and pos_s a step earlier
  // still).  Two sets: the step loop is unrolled by two, so a step reads one set and fills the
  // other, with no copies between them.
  struct StepIn {
    float w[2][T::NSLOT], x[2][NX], y[2], gy[2];
    int ps[2];
  };
  StepIn in0, in1;
  int snd[2], psn[2];  // indices / pos_s of step j + 2
  // gY[e][p][16] entry of lane l (lanes 4k hold component k after the wave sum): a view of
  // edge e's partials that only those lanes of an edge that exists address
  const unsigned gyo = (l & 3) == 0 ? 4u * (16 * p + (l >> 2)) : BUF_OOB;
  auto gy_view = [&](int e, bool on) {
    return buf_view(gY + min<int64_t>(e, elast) * a.gyp * 16, on ? 64u * a.gyp : 0u);
  };
  auto load_idx = [&](int j) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t e = min<int64_t>(beg + 2 * j + b, elast);
      snd[b] = sender[e];
      if (GX) psn[b] = pos_s[e];
    }
  };
  auto load_in = [&](int j, StepIn& S) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t e = min<int64_t>(beg + 2 * j + b, elast);
      const int64_t wo = e * a.W + c0 + u;
      if constexpr (!RW) {
#pragma unroll
        for (int s = 0; s < T::NSLOT; ++s)
          if (T::l1(s) == L1) S.w[b][s] = load_w_nt<WF>(w, wo + s * NC);
      }
      const float* xs = up + (int64_t)snd[b] * DIN + NC * L1 * L1 + c0 + u;
#pragma unroll
      for (int i = 0; i < NX; ++i) S.x[b][i] = xs[NC * i];
      S.y[b] = Y[e * 16 + (l & 15)];  // lane l holds component l & 15 (stored to LDS at the step)
      if (GX) S.ps[b] = psn[b];
      const int ej = beg + 2 * j + b;
      S.gy[b] = buf_load(gy_view(ej, a.accumulate_gY && ej < end), gyo);
    }
  };
  // The dL/dw tile of a pair of steps t (steps 2t, 2t + 1: sub-tile h = step & 1, 16 edge
  // columns each) is multiplied by W3 during the next pair's first step, after the barrier
  // that ends pair t: one barrier per two steps, and the two waves that share a SIMD (wave k
  // and k + 4: halves kh = 0, 1 of the k steps) run their products at opposite ends of that
  // step, so one wave's matrix-core work overlaps the other's VALU work.
  f4v prev[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};  // lower half: its share of pair t - 1
  // dL/dh3 of the pair before t: add the upper half's share (written to LDS during the
  // previous pair) and store (lower half only)
  auto flush = [&](int t, bool lower) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f4v o = *reinterpret_cast<const f4v*>(sp + ((((t - 1) & 1) * 2 + h) * 4 + qt) * 256 + 4 * l);
      const int e = cb + 2 * (2 * (t - 1) + h) + (r & 1);
      const bool valid = lower && t > 0 && e < ce;
      buf_store4(float4{(prev[h][0] + o[0]) * a.wscale, (prev[h][1] + o[1]) * a.wscale,
                        (prev[h][2] + o[2]) * a.wscale, (prev[h][3] + o[3]) * a.wscale},
                 gh3v, valid ? 4u * (XH * (unsigned)(e - eb0) + 16 * qt + 4 * g) : BUF_OOB);
    }
  };
  float* ys = sy + wv * 32;  // this wave's two Y rows (LDS; read back as broadcasts)
  auto edges = [&](int j, const StepIn& S, StepIn& Snext) {
    // [pair buffer][hi, lo][32 edge columns][RS]; this step's sub-tile
    _Float16* tile = sg + ((j >> 1) & 1) * 2 * 32 * RS + (j & 1) * 16 * RS;
    float* tinv = sinv + ((j >> 1) & 1) * 32 + (j & 1) * 16;
    if (l < 32) ys[l] = l < 16 ? S.y[0] : S.y[1];  // constant indices: S stays in registers
    wave_sync();
    float* m2w = sm2 + wv * 2 * M2S;  // l1 = 2: this wave's two M2 rows
    if constexpr (L1 == 2) {  // the terms and order of k_edge_fwd
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int h = 0; h < M2H; ++h)
          if (l + 64 * h < TP3_M2_NE)
            m2w[b * M2S + l + 64 * h] =
                fmaf(ys[16 * b + m2j_[h][1]], m2v_[h][1], fmaf(ys[16 * b + m2j_[h][0]], m2v_[h][0], 0.f));
      wave_sync();
    }
    load_in(j + 1, Snext);
    load_idx(j + 2);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int e = beg + 2 * j + b;
      const bool valid = e < end;
      float gYu[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) gYu[q] = 0.f;
      float gx0 = 0.f, gx1[3] = {0.f, 0.f, 0.f}, gx2[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
      float gws[T::NSLOT];
#pragma unroll
      for (int s = 0; s < T::NSLOT; ++s) gws[s] = 0.f;
      // a past-the-end edge computes on the clamped edge's inputs and its results are dropped
      // (no branch); three input blocks keep the branch, whose shorter live ranges fit in registers
      if (LIN < 3 || valid) {
        EdgeIn<LIN> in;
        in.x0 = 0.f;
#pragma unroll
        for (int i = 0; i < NX; ++i) {
          if constexpr (L1 == 0) in.x0 = S.x[b][i];
          if constexpr (L1 == 1) in.x1[i] = S.x[b][i];
          if constexpr (L1 == 2) in.x2[i] = S.x[b][i];
        }
        if constexpr (RW) {  // this edge's row of the rebuilt tile (column 16 (j & 1) + 2 wv + b)
          const unsigned short* wrow = reinterpret_cast<const unsigned short*>(
              sg + (((j >> 1) & 1) * 2 + 1) * 32 * RS + (16 * (j & 1) + 2 * wv + b) * RS + u);
#pragma unroll
          for (int s = 0; s < T::NSLOT; ++s)
            if (T::l1(s) == L1) in.w[s] = w16_value<WF>(wrow[64 * GR::local(s)]);
        } else {
#pragma unroll
          for (int s = 0; s < T::NSLOT; ++s)
            if (T::l1(s) == L1) in.w[s] = S.w[b][s];
        }
        const float* yrow = ys + 16 * b;
        if constexpr (L1 == 1)
          tp_edge_vjp_l1<LIN, GX>(R1, in, gws, yrow, gx1, gYu);
        else
          tp_edge_vjp<LIN, GX, L1>(gm, in, gws, yrow, yrow, m2w + b * M2S, gx0, gx1, gx2, gYu);
      }
      {  // split dL/dw for the matrix cores: one scale per edge (over the block's columns)
        float m = 0.f;
#pragma unroll
        for (int s = 0; s < T::NSLOT; ++s)
          if (T::l1(s) == L1) m = fmaxf(m, fabsf(gws[s]));
        m = wave_max_nonneg(m);
        // floor(log2 m) from the exponent field; zero / subnormal edges take -100 (finite scales)
        const int ex = max((int)((__float_as_uint(m) >> 23) & 0xff) - 127, -100);
        const float sc = __uint_as_float((unsigned)(127 + 14 - ex) << 23);
        _Float16* trow = tile + (2 * wv + b) * RS + u;
#pragma unroll
        for (int s = 0; s < T::NSLOT; ++s)
          if (T::l1(s) == L1) {
            const float x = gws[s] * sc;
            const _Float16 hi = (_Float16)x;
            trow[64 * GR::local(s)] = hi;
            if constexpr (WLO) trow[32 * RS + 64 * GR::local(s)] = (_Float16)(x - (float)hi);
          }
        if (l == 0) tinv[2 * wv + b] = __uint_as_float((unsigned)(127 - 14 + ex) << 23);
      }
      if constexpr (NL) {  // gw . b3 over this block's columns, stored by lane 63
        float pb = 0.f;
#pragma unroll
        for (int s = 0; s < T::NSLOT; ++s)
          if (T::l1(s) == L1) pb = fmaf(gws[s], b3c[s], pb);
        pb = wave_sum_lane63(pb);
        buf_store(pb, gwbv, l == 63 && valid ? 4u * (unsigned)(e - eb0) : BUF_OOB);
      }
      if constexpr (GX && WF == RND_F16) {  // float16 policy: the rows as fp16 values
        const auto gxv = buf_view(reinterpret_cast<_Float16*>(gxe) + (int64_t)S.ps[b] * DIN, valid ? 2u * DIN : 0u);
#pragma unroll
        for (int i = 0; i < NX; ++i) {
          const float v = L1 == 0 ? gx0 : L1 == 1 ? gx1[i] : gx2[i];
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (_Float16)v), gxv,
                                                (int)(2u * (NC * (L1 * L1 + i) + c0 + u)), 0, 0);
        }
      } else if constexpr (GX) {
        const auto gxv = buf_view(gxe + (int64_t)S.ps[b] * DIN, valid ? 4u * DIN : 0u);
#pragma unroll
        for (int i = 0; i < NX; ++i)
          buf_store(L1 == 0 ? gx0 : L1 == 1 ? gx1[i] : gx2[i], gxv, 4u * (NC * (L1 * L1 + i) + c0 + u));
      }
      const float ysum = wave_sum16(gYu);
      buf_store(a.accumulate_gY ? S.gy[b] + ysum : ysum, gy_view(e, valid), gyo);
    }
  };
  // dL/dh3 of pair t (half kh of the k steps; the two sub-tiles' products interleaved); the
  // lower half then flushes pair t - 1, the upper half leaves its share in LDS.  HALF: 0 lower,
  // 1 upper, 2 either (kh at run time: the lower half's LDS writes go to slots nobody reads)
  auto products = [&](int t, auto half) {
    constexpr int HALF = decltype(half)::value;
    const _Float16* pt = sg + (t & 1) * 2 * 32 * RS;
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < G; ++ks)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const _Float16* src = pt + (16 * h + r) * RS + 32 * (kh * G + ks) + 8 * g;
        const h8 xh = *reinterpret_cast<const h8*>(src);
        if constexpr (WLO) {
          const h8 xl = *reinterpret_cast<const h8*>(src + 32 * RS);
          acc[h] = mfma16h(wa[ks][WLO ? 1 : 0], xh, acc[h]);
          acc[h] = mfma16h(wa[ks][0], xl, acc[h]);
        }
        acc[h] = mfma16h(wa[ks][0], xh, acc[h]);
      }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float inv = sinv[(t & 1) * 32 + 16 * h + r];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[h][i] *= inv;
    }
    if constexpr (HALF != 1) flush(t, HALF == 0 || kh == 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if constexpr (HALF != 0)
        *reinterpret_cast<f4v*>(sp + ((HALF == 1 || kh ? (t & 1) * 2 + h : 4 + h) * 4 + qt) * 256 + 4 * l) = acc[h];
      if constexpr (HALF != 1) prev[h] = acc[h];
    }
  };
  const int nsteps2 = (nsteps + 1) & ~1;
  // the step loop of one half (kh uniform per wave: the barriers of both loops pair up)
  auto run = [&](auto half) {
    constexpr int HALF = decltype(half)::value;
    // RW, during pair t: the lower half (waves 0 .. 3) stages the h3 rows of pair t + 2 and
    // fetches those of pair t + 3; every wave makes its share of pair t + 1's w tile (fragments
    // read at the start, products between the two steps, stored at the end)
    auto rw_begin = [&](int t) {
      if constexpr (RW && HALF == 0) {
        store_h(t + 2);
        load_h(t + 3);
      }
      if constexpr (RW) wt_read(t + 1);
    };
    auto rw_mid = [&]() {
      if constexpr (RW) wt_mma();
    };
    auto rw_end = [&](int t) {
      if constexpr (RW) wt_store(t + 1);
    };
    rw_begin(0);
    edges(0, in0, in1);
    wave_sync();  // this step's Y- and M2-row reads are done before the next step's stores
    rw_mid();
    edges(1, in1, in0);
    rw_end(0);
    __syncthreads();
#pragma unroll 1
    for (int j = 2; j < nsteps2; j += 2) {  // nsteps2 is even
      rw_begin(j >> 1);
      if constexpr (HALF == 0) products((j >> 1) - 1, half);
      edges(j, in0, in1);
      if constexpr (HALF == 1) products((j >> 1) - 1, half);
      wave_sync();
      rw_mid();
      edges(j + 1, in1, in0);
      rw_end(j >> 1);
      __syncthreads();  // also: the Y- and M2-row reads are done before the next step's stores
    }
    products((nsteps2 >> 1) - 1, half);
    __syncthreads();
    if constexpr (HALF == 0) flush(nsteps2 >> 1, true);
  };
  // three input blocks: both halves run their products right after the barrier that ends each
  // pair (the staggered order's longer live ranges spill registers there)
  auto run_unstaggered = [&]() {
#pragma unroll 1
    for (int j = 0; j < nsteps2; j += 2) {
      edges(j, in0, in1);
      wave_sync();
      edges(j + 1, in1, in0);
      __syncthreads();
      products(j >> 1, std::integral_constant<int, 2>{});
    }
    __syncthreads();
    flush(nsteps2 >> 1, kh == 0);
  };
  if (nsteps2 == 0) return;  // uniform over the block: no receiver of it has edges
  // some receiver of the block has edges, so E >= 1 and the clamped indices are valid
  if constexpr (RW) {  // the first w tile, and the h3 rows of the second staged (lower half)
    if (kh == 0) {
      load_h(0);
      store_h(0);
      load_h(1);
      store_h(1);
      load_h(2);
    }
    __syncthreads();
    wt_read(0);
    wt_mma();
    wt_store(0);
    __syncthreads();
  }
  load_idx(0);
  load_in(0, in0);
  load_idx(1);
  if constexpr (LIN == 3)
    run_unstaggered();
  else if (kh == 0)
    run(std::integral_constant<int, 0>{});
  else
    run(std::integral_constant<int, 1>{});
}

// WF: storage format of w (RND_*, as the forward that wrote it); RW: w rebuilt instead of read
template <int LIN, bool GX, int WF, bool NL, bool RW>
__global__ void __launch_bounds__(64 * XW, 2) k_tpx_bwd(TpxBwdDims a, MACE_TPX_BWD_PTRS) {
  __shared__ __align__(16) _Float16 sg[2 * 2 * 32 * (64 * gmax<LIN>() + 8)];  // [pair][hi, lo][edge][RS]
  __shared__ float sinv[2 * 32];
  __shared__ __align__(16) float sy[XW * 32];      // [wave][edge][16]: the step's Y rows
  // [two pairs + the lower half's slots][sub-tile][q tile][lane][4]
  __shared__ __align__(16) float sp[6 * 4 * 256];
  __shared__ __align__(16) float sm2[LIN == 3 ? XW * 2 * tpx_tab_pad(2) : 4];  // [wave][edge][M2 row]
  __shared__ __align__(16) _Float16 hbuf[RW ? 2 * 32 * 72 : 8];  // RW: [pair buffer][edge][h3 row + pad]
  __shared__ float hiv[RW ? 64 : 1];                              // RW: their inverse scales
  if constexpr (LIN == 1) {
    tpx_bwd<1, 0, GX, WF, NL, RW>(a, MACE_TPX_BWD_ARGS, sg, sinv, sy, sp, sm2, hbuf, hiv);
  } else if constexpr (LIN == 2) {
    if (blockIdx.z == 0)
      tpx_bwd<2, 1, GX, WF, NL, RW>(a, MACE_TPX_BWD_ARGS, sg, sinv, sy, sp, sm2, hbuf, hiv);
    else
      tpx_bwd<2, 0, GX, WF, NL, RW>(a, MACE_TPX_BWD_ARGS, sg, sinv, sy, sp, sm2, hbuf, hiv);
  } else {
    if (blockIdx.z == 0)
      tpx_bwd<3, 2, GX, WF, NL, false>(a, MACE_TPX_BWD_ARGS, sg, sinv, sy, sp, sm2, hbuf, hiv);
    else if (blockIdx.z == 1)
      tpx_bwd<3, 1, GX, WF, NL, false>(a, MACE_TPX_BWD_ARGS, sg, sinv, sy, sp, sm2, hbuf, hiv);
    else
      tpx_bwd<3, 0, GX, WF, NL, false>(a, MACE_TPX_BWD_ARGS, sg, sinv, sy, sp, sm2, hbuf, hiv);
  }
}

__global__ void __launch_bounds__(256) k_fill_zero(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.f;
}

// groups per node for each number of input blocks
constexpr int ng_for(int lin) { return lin == 1 ? 2 : 2; }

template <int LIN, typename WT>
void launch_fwd(hipStream_t st, int N, const int* rowptr, const int* sender, const float* Y, const float* Mt, int mts,
                const void* w, const float* up, float* M, int half) {
  constexpr int NG = ng_for(LIN);
  MACE_LAUNCH((k_tp_fwd<LIN, NG, WT>), dim3(N), dim3(NC * NG), 0, st, N, rowptr, sender, Y, Mt, mts,
                     static_cast<const WT*>(w), up, M, half);
}

template <int LIN, bool GX, typename WT>
void launch_recv(hipStream_t st, int N, const int* rowptr, const int* sender, const float* Y, const float* Mt,
                 int mts, const void* w, const float* up, const float* gM, void* gw, float* gscale, float* gY,
                 int accumulate_gY, const int* pos_s, float* gxe) {
  constexpr int NG = ng_for(LIN);
  MACE_LAUNCH((k_tp_bwd_recv<LIN, NG, GX, WT>), dim3(N), dim3(NC * NG), 0, st, N, rowptr, sender, Y, Mt,
                     mts, static_cast<const WT*>(w), up, gM, static_cast<WT*>(gw), gscale, gY, accumulate_gY,
                     pos_s, gxe);
}

}  // namespace

int tp_table_entries(int max_lin) { return max_lin >= 3 ? TP3_M1_NE + TP3_M2_NE : max_lin == 2 ? TP3_M1_NE : 0; }


void launch_tp_fwd(hipStream_t st, int lin, int N, const int* rowptr, const int* sender, const float* Y,
                   const float* Mt, int mts, const void* w, const float* up, float* M, int half) {
  if (N <= 0) return;
#define MACE_FWD(L)                                                        \
  half == RND_F16 ? launch_fwd<L, _Float16>(st, N, rowptr, sender, Y, Mt, mts, w, up, M, half) \
                  : launch_fwd<L, float>(st, N, rowptr, sender, Y, Mt, mts, w, up, M, half)
  switch (lin) {
    case 1: MACE_FWD(1); break;
    case 2: MACE_FWD(2); break;
    case 3: MACE_FWD(3); break;
  }
#undef MACE_FWD
}

void launch_tp_bwd_recv(hipStream_t st, int lin, int N, const int* rowptr, const int* sender, const float* Y,
                        const float* Mt, int mts, const void* w, const float* up, const float* gM, void* gw,
                        float* gscale, float* gY, int accumulate_gY, const int* pos_s, float* gxe, int half) {
  if (N <= 0) return;
#define MACE_RECV(L, G)                                                                                          \
  half == RND_F16 ? launch_recv<L, G, _Float16>(st, N, rowptr, sender, Y, Mt, mts, w, up, gM, gw, gscale, gY, accumulate_gY, \
                                     pos_s, gxe)                                                                 \
       : launch_recv<L, G, float>(st, N, rowptr, sender, Y, Mt, mts, w, up, gM, gw, gscale, gY, accumulate_gY,   \
                                  pos_s, gxe)
  const bool gx = gxe != nullptr;
  switch (lin) {
    case 1: gx ? MACE_RECV(1, true) : MACE_RECV(1, false); break;
    case 2: gx ? MACE_RECV(2, true) : MACE_RECV(2, false); break;
    case 3: gx ? MACE_RECV(3, true) : MACE_RECV(3, false); break;
  }
#undef MACE_RECV
}

// the fused TP kernels split a receiver's edges over several waves below this many blocks per
// layer (256 CUs; Si1000's layer 0 has 250 blocks of one receiver per wave and stays so)
constexpr int kTpxMinBlocks = 240;
// log2 of the waves per receiver of a fused TP launch over N receivers: the fewest (1 to XW) that
// give kTpxMinBlocks blocks
int tpx_split_log2(int N, int lin) {
  int l = 0;
  while ((1 << l) < XW && (int64_t)((N + (XW >> l) - 1) / (XW >> l)) * NSLICE * lin < kTpxMinBlocks) ++l;
  return l;
}

void launch_tpx_fwd(hipStream_t st, int lin, int N, int64_t E, const int* rowptr, const int* sender, const float* Y,
                    const float* Mt, int mts, const void* h3x, const float* h3inv, const void* W3Tx, int W,
                    float wscale, const float* up, float* M, float* w, int rnd, const float* b3, const float* cut,
                    int store_w) {
  if (N <= 0) return;
  // waves per receiver: enough blocks for the CUs (small systems), one otherwise
  const int sprl = tpx_split_log2(N, lin);
  const TpxDims a{N, W, mts, E, wscale, b3, cut, sprl, store_w};
  // y: channel slice; z: input block l1
  const dim3 grid((unsigned)((N + (XW >> sprl) - 1) / (XW >> sprl)), NSLICE, (unsigned)lin);
  const _Float16* hx = static_cast<const _Float16*>(h3x);
  const _Float16* wt = static_cast<const _Float16*>(W3Tx);
#define MACE_TPXF(L, R, NLV) \
  MACE_LAUNCH((k_tpx_fwd<L, R, NLV>), grid, dim3(64 * XW), 0, st, a, rowptr, sender, Y, Mt, hx, h3inv, wt, up, M, w)
  // NL: the non-linear block's bias / envelope epilogue (b3 given)
#define MACE_TPXF_RN(L, NLV)     \
  if (rnd == RND_F16)            \
    MACE_TPXF(L, RND_F16, NLV);  \
  else if (rnd == RND_BF16)      \
    MACE_TPXF(L, RND_BF16, NLV); \
  else                           \
    MACE_TPXF(L, RND_NONE, NLV);
#define MACE_TPXF_R(L)          \
  if (b3) {                     \
    MACE_TPXF_RN(L, true)       \
  } else {                      \
    MACE_TPXF_RN(L, false)      \
  }
  if (lin == 1) {
    MACE_TPXF_R(1)
  } else if (lin == 2) {
    MACE_TPXF_R(2)
  } else {
    MACE_TPXF_R(3)
  }
#undef MACE_TPXF_R
#undef MACE_TPXF_RN
#undef MACE_TPXF
}


void launch_tpx_bwd(hipStream_t st, int lin, int N, int64_t E, const int* rowptr, const int* sender, const float* Y,
                    const float* Mt, int mts, const float* w, const void* W3x, int W, float wscale, const float* up,
                    const float* gM, const int* pos_s, float* gxe, float* gY, int gyp, int accumulate_gY,
                    float* gh3p, int wfmt, const float* b3, float* gwbp, const void* h3x, const float* h3inv,
                    const void* W3Tx, int rebuild_w) {
  if (N <= 0 || E <= 0) return;  // no edges: no dL/dw, dL/dY, dL/dx rows to write
  if (rebuild_w && !tpx_rebuilds_w(lin, wfmt, b3 != nullptr))
    throw std::invalid_argument("launch_tpx_bwd: w is rebuilt only under a half-precision policy, one or two "
                                "input blocks and the standard interaction block");
  // waves per receiver: enough blocks for the CUs (small systems), one otherwise
  const int sprl = tpx_split_log2(N, lin);
  const TpxBwdDims a{N, W, mts, E, wscale, accumulate_gY, gyp, b3, gwbp, sprl};
  const dim3 grid((unsigned)((N + (XW >> sprl) - 1) / (XW >> sprl)), NSLICE, (unsigned)lin);
  const _Float16* wx = static_cast<const _Float16*>(W3x);
  const _Float16* hx = static_cast<const _Float16*>(h3x);
  const _Float16* wtx = static_cast<const _Float16*>(W3Tx);
#define MACE_TPXB_RW(L, GXV, WF, NLV, RWV)                                                                       \
  MACE_LAUNCH((k_tpx_bwd<L, GXV, WF, NLV, RWV>), grid, dim3(64 * XW), 0, st, a, rowptr, sender, Y, Mt, w, wx, up, \
              gM, pos_s, gxe, gY, gh3p, hx, h3inv, wtx)
  // RW: only where tpx_rebuilds_w allows it (instantiated for those template arguments only)
#define MACE_TPXB(L, GXV, WF, NLV)                                          \
  do {                                                                      \
    if constexpr (WF != RND_NONE && !NLV && L <= 2) {                       \
      if (rebuild_w)                                                        \
        MACE_TPXB_RW(L, GXV, WF, NLV, true);                                \
      else                                                                  \
        MACE_TPXB_RW(L, GXV, WF, NLV, false);                               \
    } else {                                                                \
      MACE_TPXB_RW(L, GXV, WF, NLV, false);                                 \
    }                                                                       \
  } while (0)
  // NL: the non-linear block's gw . b3 partials (b3 given)
#define MACE_TPXB_WN(L, GXV, NLV)       \
  if (wfmt == RND_F16)                  \
    MACE_TPXB(L, GXV, RND_F16, NLV);    \
  else if (wfmt == RND_BF16)            \
    MACE_TPXB(L, GXV, RND_BF16, NLV);   \
  else                                  \
    MACE_TPXB(L, GXV, RND_NONE, NLV);
#define MACE_TPXB_WF(L, GXV)         \
  if (b3) {                          \
    MACE_TPXB_WN(L, GXV, true)       \
  } else {                           \
    MACE_TPXB_WN(L, GXV, false)      \
  }
  const bool gx = gxe != nullptr;
  if (lin == 1) {
    if (gx) { MACE_TPXB_WF(1, true) } else { MACE_TPXB_WF(1, false) }
  } else if (lin == 2) {
    if (gx) { MACE_TPXB_WF(2, true) } else { MACE_TPXB_WF(2, false) }
  } else {
    if (gx) { MACE_TPXB_WF(3, true) } else { MACE_TPXB_WF(3, false) }
  }
#undef MACE_TPXB_WF
#undef MACE_TPXB_WN
#undef MACE_TPXB
#undef MACE_TPXB_RW
}

bool tpx_rebuilds_w(int lin, int wfmt, bool nonlinear) { return wfmt != RND_NONE && lin <= 2 && !nonlinear; }

void launch_fill_zero(hipStream_t st, float* p, int64_t n) {
  if (n <= 0) return;
  MACE_LAUNCH(k_fill_zero, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 1024)), dim3(256), 0, st, p, n);
}

void launch_tp_gather_gx(hipStream_t st, int lin, int N, const int* rowptr_s, const float* gxe, float* gup,
                         int gx16, int accumulate) {
  if (N <= 0) return;
  const int din = NC * lin * lin;  // a multiple of 64
  auto go = [&](auto tag, const auto* src) {
    using GT = decltype(tag);
    const int nchunk = (din + 64 * (16 / (int)sizeof(GT)) - 1) / (64 * (16 / (int)sizeof(GT)));
    const int64_t units = (int64_t)N * nchunk;
    MACE_LAUNCH(k_tp_gather_gx<GT>, dim3((unsigned)((units + 3) / 4)), dim3(256), 0, st, N, din, nchunk, rowptr_s,
                src, gup, accumulate);
  };
  if (gx16)
    go(_Float16{}, reinterpret_cast<const _Float16*>(gxe));
  else
    go(float{}, gxe);
}

}  // namespace mace
