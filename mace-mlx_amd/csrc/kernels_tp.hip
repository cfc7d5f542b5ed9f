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
// One workgroup of NC threads (thread = channel u) owns one node.  Edges are
// processed in batches of EB: their SH rows are staged in LDS and turned into
// the x2-first tables M_l1[i][col] = sum_j Y_j C[i, j, k] pw (shared by all
// channels), then every thread accumulates its channel's outputs in registers.
// The segmented sum is the register accumulation itself: no atomics, results
// are deterministic.
#include <hip/hip_runtime.h>

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
    static constexpr int M1_NE = TP##N##_M1_NE, M2_NE = TP##N##_M2_NE;             \
    __host__ __device__ static constexpr int l1(int s) { return TP##N##_L1[s]; }   \
    __host__ __device__ static constexpr int l2(int s) { return TP##N##_L2[s]; }   \
    __host__ __device__ static constexpr int l3(int s) { return TP##N##_L3[s]; }   \
    __host__ __device__ static constexpr int acc(int s) { return TP##N##_ACC[s]; } \
    __host__ __device__ static constexpr int col(int s) { return TP##N##_COL[s]; } \
    __device__ static constexpr int m1s(int q) { return TP##N##_M1_START[q]; }    \
    __device__ static constexpr int m1j(int x) { return TP##N##_M1_J[x]; }        \
    __device__ static constexpr float m1v(int x) { return TP##N##_M1_V[x]; }      \
    __device__ static constexpr int m2s(int q) { return TP##N##_M2_START[q]; }    \
    __device__ static constexpr int m2j(int x) { return TP##N##_M2_J[x]; }        \
    __device__ static constexpr float m2v(int x) { return TP##N##_M2_V[x]; }      \
  };
MACE_TP_TRAITS(1)
MACE_TP_TRAITS(2)
MACE_TP_TRAITS(3)
#undef MACE_TP_TRAITS

constexpr int EB_F = 8;  // edges per LDS batch, forward
constexpr int EB_B = 4;  // edges per LDS batch, backward (gY transpose buffer)

template <int LIN>
struct Smem {
  using T = TPT<LIN>;
  static constexpr int M1W = T::M1_NE > 0 ? T::M1_NE : 1;
  static constexpr int M2W = T::M2_NE > 0 ? T::M2_NE : 1;
};

// Stage Y rows of a batch and build the x2-first tables.
template <int LIN, int EB>
__device__ __forceinline__ void stage_batch(int nb, const int* eid, const float* __restrict__ Y,
                                            float (*sY)[16], float (*sM1)[Smem<LIN>::M1W],
                                            float (*sM2)[Smem<LIN>::M2W]) {
  using T = TPT<LIN>;
  const int u = threadIdx.x;
  for (int t = u; t < nb * 16; t += NC) sY[t >> 4][t & 15] = Y[(int64_t)eid[t >> 4] * 16 + (t & 15)];
  __syncthreads();
  if constexpr (T::M1_NE > 0) {
    for (int t = u; t < nb * T::M1_NE; t += NC) {
      const int b = t / T::M1_NE, q = t % T::M1_NE;
      float a = 0.f;
      for (int x = T::m1s(q); x < T::m1s(q + 1); ++x) a = fmaf(sY[b][T::m1j(x)], T::m1v(x), a);
      sM1[b][q] = a;
    }
  }
  if constexpr (T::M2_NE > 0) {
    for (int t = u; t < nb * T::M2_NE; t += NC) {
      const int b = t / T::M2_NE, q = t % T::M2_NE;
      float a = 0.f;
      for (int x = T::m2s(q); x < T::m2s(q + 1); ++x) a = fmaf(sY[b][T::m2j(x)], T::m2v(x), a);
      sM2[b][q] = a;
    }
  }
  __syncthreads();
}

template <int LIN>
__device__ __forceinline__ void load_x(const float* __restrict__ xs, int u, float& x0, float* x1, float* x2) {
  x0 = xs[u];
  if constexpr (LIN >= 2) {
#pragma unroll
    for (int i = 0; i < 3; ++i) x1[i] = xs[NC * (1 + i) + u];
  }
  if constexpr (LIN >= 3) {
#pragma unroll
    for (int i = 0; i < 5; ++i) x2[i] = xs[NC * (4 + i) + u];
  }
}

template <int LIN>
__global__ void __launch_bounds__(NC) k_tp_fwd(int N, const int* __restrict__ rowptr,
                                               const int* __restrict__ sender, const float* __restrict__ Y,
                                               const float* __restrict__ w, const float* __restrict__ up,
                                               float* __restrict__ M) {
  using T = TPT<LIN>;
  constexpr int DIN = NC * LIN * LIN, DMID = NC * T::NACC, WN = NC * T::NSLOT;
  __shared__ float sY[EB_F][16];
  __shared__ float sM1[EB_F][Smem<LIN>::M1W];
  __shared__ float sM2[EB_F][Smem<LIN>::M2W];
  __shared__ int sE[EB_F], sS[EB_F];
  const int n = blockIdx.x, u = threadIdx.x;
  float acc[T::NACC];
#pragma unroll
  for (int a = 0; a < T::NACC; ++a) acc[a] = 0.f;
  const int beg = rowptr[n], end = rowptr[n + 1];
  for (int e0 = beg; e0 < end; e0 += EB_F) {
    const int nb = min(EB_F, end - e0);
    __syncthreads();
    if (u < nb) {
      sE[u] = e0 + u;
      sS[u] = sender[e0 + u];
    }
    __syncthreads();
    stage_batch<LIN, EB_F>(nb, sE, Y, sY, sM1, sM2);
    for (int b = 0; b < nb; ++b) {
      const int64_t e = sE[b];
      float x0, x1[3], x2[5];
      load_x<LIN>(up + (int64_t)sS[b] * DIN, u, x0, x1, x2);
      const float* we = w + e * WN + u;
#pragma unroll
      for (int s = 0; s < T::NSLOT; ++s) {
        const float ww = we[s * NC];
        constexpr int dummy = 0;
        (void)dummy;
        const int a0 = T::acc(s), d = 2 * T::l3(s) + 1;
        if (T::l1(s) == 0) {
          const float xw = x0 * ww;
#pragma unroll
          for (int m = 0; m < d; ++m) acc[a0 + m] = fmaf(xw, sY[b][T::l2(s) * T::l2(s) + m], acc[a0 + m]);
        } else if (T::l1(s) == 1) {
          const int c0 = T::col(s);
#pragma unroll
          for (int k = 0; k < d; ++k) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < 3; ++i) t = fmaf(x1[i], sM1[b][i * T::K1 + c0 + k], t);
            acc[a0 + k] = fmaf(ww, t, acc[a0 + k]);
          }
        } else {
          const int c0 = T::col(s);
#pragma unroll
          for (int k = 0; k < d; ++k) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < 5; ++i) t = fmaf(x2[i], sM2[b][i * T::K2 + c0 + k], t);
            acc[a0 + k] = fmaf(ww, t, acc[a0 + k]);
          }
        }
      }
    }
  }
  float* Mn = M + (int64_t)n * DMID + u;
#pragma unroll
  for (int a = 0; a < T::NACC; ++a) Mn[a * NC] = acc[a];
}

// Per-edge VJP of one thread's channel: given g = dL/dM[recv] (this channel),
// accumulates the input gradient (if GX), writes dL/dw and adds this channel's
// share of dL/dY into gYu.
template <int LIN, bool GX>
__device__ __forceinline__ void tp_edge_vjp(const float* g, const float* __restrict__ we, float* __restrict__ gwe,
                                            float x0, const float* x1, const float* x2, const float* sYb,
                                            const float* sM1b, const float* sM2b, float& gx0, float* gx1,
                                            float* gx2, float* gYu) {
  using T = TPT<LIN>;
#pragma unroll
  for (int s = 0; s < T::NSLOT; ++s) {
    const float ww = we[s * NC];
    const int a0 = T::acc(s), d = 2 * T::l3(s) + 1, l2 = T::l2(s);
    float gws = 0.f;
    if (T::l1(s) == 0) {
      float t = 0.f;
#pragma unroll
      for (int m = 0; m < d; ++m) {
        t = fmaf(g[a0 + m], sYb[l2 * l2 + m], t);
        gYu[l2 * l2 + m] = fmaf(x0 * ww, g[a0 + m], gYu[l2 * l2 + m]);
      }
      gws = x0 * t;
      if (GX) gx0 = fmaf(ww, t, gx0);
    } else if (T::l1(s) == 1) {
      const int c0 = T::col(s);
#pragma unroll
      for (int k = 0; k < d; ++k) {
        float mk = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const int q = i * T::K1 + c0 + k;
          mk = fmaf(x1[i], sM1b[q], mk);
          if (GX) gx1[i] = fmaf(ww * g[a0 + k], sM1b[q], gx1[i]);
          const float c = ww * x1[i] * g[a0 + k];
#pragma unroll
          for (int x = T::m1s(q); x < T::m1s(q + 1); ++x) gYu[T::m1j(x)] = fmaf(c, T::m1v(x), gYu[T::m1j(x)]);
        }
        gws = fmaf(g[a0 + k], mk, gws);
      }
    } else {
      const int c0 = T::col(s);
#pragma unroll
      for (int k = 0; k < d; ++k) {
        float mk = 0.f;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
          const int q = i * T::K2 + c0 + k;
          mk = fmaf(x2[i], sM2b[q], mk);
          if (GX) gx2[i] = fmaf(ww * g[a0 + k], sM2b[q], gx2[i]);
          const float c = ww * x2[i] * g[a0 + k];
#pragma unroll
          for (int x = T::m2s(q); x < T::m2s(q + 1); ++x) gYu[T::m2j(x)] = fmaf(c, T::m2v(x), gYu[T::m2j(x)]);
        }
        gws = fmaf(g[a0 + k], mk, gws);
      }
    }
    gwe[s * NC] = gws;
  }
}

// Block reduction of the per-channel dL/dY partials of a batch: sR[b*16 + j][u].
__device__ __forceinline__ void reduce_gY(int nb, const int* eid, float (*sR)[NC + 1], float* __restrict__ gY,
                                          int accumulate) {
  const int u = threadIdx.x;
  const int q = u >> 1, h = u & 1;  // row q = b*16 + j (EB_B*16 = 64 rows), half h
  float a = 0.f;
#pragma unroll 8
  for (int c = 0; c < NC / 2; ++c) a += sR[q][h * (NC / 2) + c];
  a += __shfl_xor(a, 1);
  const int b = q >> 4, j = q & 15;
  if (h == 0 && b < nb) {
    float* dst = gY + (int64_t)eid[b] * 16 + j;
    *dst = accumulate ? *dst + a : a;
  }
}

template <int LIN>
__global__ void __launch_bounds__(NC) k_tp_bwd_recv(int N, const int* __restrict__ rowptr,
                                                    const int* __restrict__ sender, const float* __restrict__ Y,
                                                    const float* __restrict__ w, const float* __restrict__ up,
                                                    const float* __restrict__ gM, float* __restrict__ gw,
                                                    float* __restrict__ gY, int accumulate_gY) {
  using T = TPT<LIN>;
  constexpr int DIN = NC * LIN * LIN, DMID = NC * T::NACC, WN = NC * T::NSLOT;
  static_assert(EB_B * 16 == NC / 2, "gY reduction maps 2 threads per row");
  __shared__ float sY[EB_B][16];
  __shared__ float sM1[EB_B][Smem<LIN>::M1W];
  __shared__ float sM2[EB_B][Smem<LIN>::M2W];
  __shared__ float sR[EB_B * 16][NC + 1];
  __shared__ int sE[EB_B], sS[EB_B];
  const int n = blockIdx.x, u = threadIdx.x;
  float g[T::NACC];
  const float* gMn = gM + (int64_t)n * DMID + u;
#pragma unroll
  for (int a = 0; a < T::NACC; ++a) g[a] = gMn[a * NC];
  const int beg = rowptr[n], end = rowptr[n + 1];
  for (int e0 = beg; e0 < end; e0 += EB_B) {
    const int nb = min(EB_B, end - e0);
    __syncthreads();
    if (u < nb) {
      sE[u] = e0 + u;
      sS[u] = sender[e0 + u];
    }
    __syncthreads();
    stage_batch<LIN, EB_B>(nb, sE, Y, sY, sM1, sM2);
    for (int b = 0; b < EB_B; ++b) {
      float gYu[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) gYu[j] = 0.f;
      if (b < nb) {
        const int64_t e = sE[b];
        float x0, x1[3], x2[5], gx0 = 0.f, gx1[3], gx2[5];
        load_x<LIN>(up + (int64_t)sS[b] * DIN, u, x0, x1, x2);
        tp_edge_vjp<LIN, false>(g, w + e * WN + u, gw + e * WN + u, x0, x1, x2, sY[b], sM1[b], sM2[b], gx0,
                                gx1, gx2, gYu);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) sR[b * 16 + j][u] = gYu[j];
    }
    __syncthreads();
    reduce_gY(nb, sE, sR, gY, accumulate_gY);
  }
}

template <int LIN>
__global__ void __launch_bounds__(NC) k_tp_bwd_send(int N, const int* __restrict__ rowptr_s,
                                                    const int* __restrict__ perm_s,
                                                    const int* __restrict__ receiver, const float* __restrict__ Y,
                                                    const float* __restrict__ w, const float* __restrict__ up,
                                                    const float* __restrict__ gM, float* __restrict__ gw,
                                                    float* __restrict__ gY, float* __restrict__ gup,
                                                    int accumulate_gY) {
  using T = TPT<LIN>;
  constexpr int DIN = NC * LIN * LIN, DMID = NC * T::NACC, WN = NC * T::NSLOT;
  __shared__ float sY[EB_B][16];
  __shared__ float sM1[EB_B][Smem<LIN>::M1W];
  __shared__ float sM2[EB_B][Smem<LIN>::M2W];
  __shared__ float sR[EB_B * 16][NC + 1];
  __shared__ int sE[EB_B], sRv[EB_B];
  const int a = blockIdx.x, u = threadIdx.x;
  float x0, x1[3], x2[5];
  load_x<LIN>(up + (int64_t)a * DIN, u, x0, x1, x2);
  float gx0 = 0.f, gx1[3] = {0.f, 0.f, 0.f}, gx2[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
  const int beg = rowptr_s[a], end = rowptr_s[a + 1];
  for (int k0 = beg; k0 < end; k0 += EB_B) {
    const int nb = min(EB_B, end - k0);
    __syncthreads();
    if (u < nb) {
      const int e = perm_s[k0 + u];
      sE[u] = e;
      sRv[u] = receiver[e];
    }
    __syncthreads();
    stage_batch<LIN, EB_B>(nb, sE, Y, sY, sM1, sM2);
    for (int b = 0; b < EB_B; ++b) {
      float gYu[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) gYu[j] = 0.f;
      if (b < nb) {
        const int64_t e = sE[b];
        float g[T::NACC];
        const float* gMr = gM + (int64_t)sRv[b] * DMID + u;
#pragma unroll
        for (int q = 0; q < T::NACC; ++q) g[q] = gMr[q * NC];
        tp_edge_vjp<LIN, true>(g, w + e * WN + u, gw + e * WN + u, x0, x1, x2, sY[b], sM1[b], sM2[b], gx0, gx1,
                               gx2, gYu);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) sR[b * 16 + j][u] = gYu[j];
    }
    __syncthreads();
    reduce_gY(nb, sE, sR, gY, accumulate_gY);
  }
  float* go = gup + (int64_t)a * DIN + u;
  go[0] = gx0;
  if constexpr (LIN >= 2) {
#pragma unroll
    for (int i = 0; i < 3; ++i) go[NC * (1 + i)] = gx1[i];
  }
  if constexpr (LIN >= 3) {
#pragma unroll
    for (int i = 0; i < 5; ++i) go[NC * (4 + i)] = gx2[i];
  }
}

}  // namespace

void launch_tp_fwd(hipStream_t st, int lin, int N, const int* rowptr, const int* sender, const float* Y,
                   const float* w, const float* up, float* M) {
  if (N <= 0) return;
  switch (lin) {
    case 1: hipLaunchKernelGGL(k_tp_fwd<1>, dim3(N), dim3(NC), 0, st, N, rowptr, sender, Y, w, up, M); break;
    case 2: hipLaunchKernelGGL(k_tp_fwd<2>, dim3(N), dim3(NC), 0, st, N, rowptr, sender, Y, w, up, M); break;
    case 3: hipLaunchKernelGGL(k_tp_fwd<3>, dim3(N), dim3(NC), 0, st, N, rowptr, sender, Y, w, up, M); break;
  }
}

void launch_tp_bwd_recv(hipStream_t st, int lin, int N, const int* rowptr, const int* sender, const float* Y,
                        const float* w, const float* up, const float* gM, float* gw, float* gY,
                        int accumulate_gY) {
  if (N <= 0) return;
  switch (lin) {
    case 1:
      hipLaunchKernelGGL(k_tp_bwd_recv<1>, dim3(N), dim3(NC), 0, st, N, rowptr, sender, Y, w, up, gM, gw, gY,
                         accumulate_gY);
      break;
    case 2:
      hipLaunchKernelGGL(k_tp_bwd_recv<2>, dim3(N), dim3(NC), 0, st, N, rowptr, sender, Y, w, up, gM, gw, gY,
                         accumulate_gY);
      break;
    case 3:
      hipLaunchKernelGGL(k_tp_bwd_recv<3>, dim3(N), dim3(NC), 0, st, N, rowptr, sender, Y, w, up, gM, gw, gY,
                         accumulate_gY);
      break;
  }
}

void launch_tp_bwd_send(hipStream_t st, int lin, int N, const int* rowptr_s, const int* perm_s,
                        const int* receiver, const float* Y, const float* w, const float* up, const float* gM,
                        float* gw, float* gY, float* gup, int accumulate_gY) {
  if (N <= 0) return;
  switch (lin) {
    case 1:
      hipLaunchKernelGGL(k_tp_bwd_send<1>, dim3(N), dim3(NC), 0, st, N, rowptr_s, perm_s, receiver, Y, w, up, gM,
                         gw, gY, gup, accumulate_gY);
      break;
    case 2:
      hipLaunchKernelGGL(k_tp_bwd_send<2>, dim3(N), dim3(NC), 0, st, N, rowptr_s, perm_s, receiver, Y, w, up, gM,
                         gw, gY, gup, accumulate_gY);
      break;
    case 3:
      hipLaunchKernelGGL(k_tp_bwd_send<3>, dim3(N), dim3(NC), 0, st, N, rowptr_s, perm_s, receiver, Y, w, up, gM,
                         gw, gY, gup, accumulate_gY);
      break;
  }
}

}  // namespace mace
