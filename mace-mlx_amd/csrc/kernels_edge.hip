// Edge-parallel kernels: front end (geometry, spherical harmonics, radial basis,
// ZBL), its VJP, the radial MLP forward/backward, and the device neighbour list.
#include <hip/hip_runtime.h>

#include <climits>
#include <hipcub/hipcub.hpp>
#include <stdexcept>

#include "common.h"

namespace mace {

namespace {

constexpr float SQRT3 = 1.7320508075688772f;

__device__ __forceinline__ float poly_env(float u, int p, float* denv) {
  // envelope(u) = 1 - c1 u^p + c2 u^(p+1) - c3 u^(p+2) for u < 1, else 0
  // (radial.py:18-34); also returns d envelope / du.
  if (!(u < 1.0f)) {
    *denv = 0.f;
    return 0.f;
  }
  const float pf = (float)p;
  const float c1 = (pf + 1.f) * (pf + 2.f) * 0.5f, c2 = pf * (pf + 2.f), c3 = pf * (pf + 1.f) * 0.5f;
  float up1 = 1.f;  // u^(p-1)
  for (int i = 0; i < p - 1; ++i) up1 *= u;
  const float up = up1 * u;
  *denv = -c1 * pf * up1 + c2 * (pf + 1.f) * up - c3 * (pf + 2.f) * up * u;
  return 1.f - c1 * up + c2 * up * u - c3 * up * u * u;
}

__device__ __forceinline__ void sh16(float ux, float uy, float uz, float* Y) {
  Y[0] = 1.f;
  Y[1] = SQRT3 * ux;
  Y[2] = SQRT3 * uy;
  Y[3] = SQRT3 * uz;
#pragma unroll
  for (int k = 4; k < 16; ++k) Y[k] = 0.f;
#pragma unroll
  for (int t = 0; t < SH2_NT; ++t) Y[4 + SH2_K[t]] += SH2_V[t] * Y[1 + SH2_I[t]] * Y[1 + SH2_J[t]];
#pragma unroll
  for (int t = 0; t < SH3_NT; ++t) Y[9 + SH3_K[t]] += SH3_V[t] * Y[4 + SH3_I[t]] * Y[1 + SH3_J[t]];
}

__device__ __forceinline__ void edge_vec(const double* __restrict__ pos, const int* __restrict__ sh,
                                         const double* cell, int s, int r, int64_t e, float& x,
                                         float& y, float& z) {
  const double S0 = sh[3 * e], S1 = sh[3 * e + 1], S2 = sh[3 * e + 2];
  x = (float)(pos[3 * r] - pos[3 * s] + S0 * cell[0] + S1 * cell[3] + S2 * cell[6]);
  y = (float)(pos[3 * r + 1] - pos[3 * s + 1] + S0 * cell[1] + S1 * cell[4] + S2 * cell[7]);
  z = (float)(pos[3 * r + 2] - pos[3 * s + 2] + S0 * cell[2] + S1 * cell[5] + S2 * cell[8]);
}

__device__ __forceinline__ float zbl_phi(float x, float* dphi) {
  const float e0 = expf(-3.2f * x), e1 = expf(-0.9423f * x), e2 = expf(-0.4028f * x),
              e3 = expf(-0.2016f * x);
  *dphi = -3.2f * 0.1818f * e0 - 0.9423f * 0.5099f * e1 - 0.4028f * 0.2802f * e2 -
          0.2016f * 0.02817f * e3;
  return 0.1818f * e0 + 0.5099f * e1 + 0.2802f * e2 + 0.02817f * e3;
}

// Agnesi transform (radial.py:231-262): t = 1 / (1 + a x^q / (1 + x^(q-p))),
// x = r / r0; returns t and dt/dr.
__device__ __forceinline__ float agnesi_t(float r, float r0, const FrontParams& p, float* dtdr) {
  const float x = fmaxf(r / r0, 1e-12f);
  const float xq = powf(x, p.ag_q), xqp = powf(x, p.ag_q - p.ag_p);
  const float den = 1.f + xqp;
  const float t = 1.f / (1.f + p.ag_a * xq / den);
  const float dfdx = p.ag_a * (p.ag_q * xq * den - (p.ag_q - p.ag_p) * xq * xqp) / (x * den * den);
  *dtdr = -t * t * dfdx / r0;
  return t;
}

// Also writes the per-edge TP tables Mt[e] = [M1 (3 x K1) | M2 (5 x K2)] (NENT = 72 or 227
// entries, row stride mts, a multiple of 16) from the edge's stored Y, four entries per store.
template <int NENT>
__global__ void __launch_bounds__(256) k_edge_fwd(
    int64_t E, const double* __restrict__ pos, const int* __restrict__ sender,
    const int* __restrict__ receiver, const int* __restrict__ shifts, const int* __restrict__ species,
    const float* __restrict__ bessel_w, const float* __restrict__ zbl_z,
    const float* __restrict__ zbl_cov, const float* __restrict__ ag_cov, FrontParams p,
    const double* __restrict__ gcell, const int* __restrict__ gid, EdgeGeom* __restrict__ geom,
    float* __restrict__ Y, float* __restrict__ ef, float* __restrict__ zbl_e, float* __restrict__ Mt, int mts,
    float* __restrict__ cut) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int s = sender[e], r = receiver[e];
  float x, y, z;
  // a batch of structures: the receiver's structure's cell (gcell [G][9], gid per atom)
  edge_vec(pos, shifts, gcell ? gcell + 9 * gid[r] : p.cell, s, r, e, x, y, z);
  const float rr = sqrtf(fmaxf(x * x + y * y + z * z, 1e-24f));
  geom[e] = EdgeGeom{x, y, z, rr};
  const float inv = 1.f / rr;
  float Yl[16];
  sh16(x * inv, y * inv, z * inv, Yl);
  float4* Y4 = reinterpret_cast<float4*>(Y + 16 * e);
#pragma unroll
  for (int j = 0; j < 16; ++j) Yl[j] = qh(Yl[j], p.feature_half);  // the stored values
#pragma unroll
  for (int q = 0; q < 4; ++q) Y4[q] = make_float4(Yl[4 * q], Yl[4 * q + 1], Yl[4 * q + 2], Yl[4 * q + 3]);
  if constexpr (NENT > 0) {
    float4* T4 = reinterpret_cast<float4*>(Mt + e * mts);
    auto entry = [&](int q) {
      float a = 0.f;
      if (q < TP3_M1_NE) {
#pragma unroll
        for (int x = m1s(q); x < m1s(q + 1); ++x) a = fmaf(Yl[m1j(x)], m1v(x), a);
      } else if (q < NENT) {
#pragma unroll
        for (int x = m2s(q - TP3_M1_NE); x < m2s(q - TP3_M1_NE + 1); ++x) a = fmaf(Yl[m2j(x)], m2v(x), a);
      }
      return a;
    };
#pragma unroll
    for (int q = 0; q < NENT; q += 4) T4[q / 4] = make_float4(entry(q), entry(q + 1), entry(q + 2), entry(q + 3));
  }
  float denv;
  const float env = poly_env(rr / p.r_max, p.pcut, &denv);
  float rb = rr;  // argument of the Bessel basis
  if (p.agnesi) {
    float dtdr;
    rb = agnesi_t(rr, 0.5f * (ag_cov[species[s]] + ag_cov[species[r]]), p, &dtdr);
  }
  // apply_cutoff = 0 (radial.py:316-318): the basis alone; the envelope goes to cut
  const float envb = p.apply_cutoff ? env : 1.f;
  if (!p.apply_cutoff) cut[e] = env;
  for (int n = 0; n < p.nbessel; ++n) {
    const float w = bessel_w[n];
    const float b = (rb == 0.f) ? p.bessel_pref * w : p.bessel_pref * sinf(w * rb) / rb;
    ef[(int64_t)p.nbessel * e + n] = qh(b * envb, p.feature_half);
  }
  if (p.has_zbl) {
    const int zs = species[s], zr = species[r];
    const float Zu = zbl_z[zs], Zv = zbl_z[zr];
    const float a = p.zbl_a_pref * 0.529f / (powf(Zu, p.zbl_a_exp) + powf(Zv, p.zbl_a_exp));
    float dphi;
    const float phi = zbl_phi(rr / a, &dphi);
    const float rmax = zbl_cov[zs] + zbl_cov[zr];
    float dz;
    const float envz = poly_env(rr / rmax, p.zbl_p, &dz);
    zbl_e[e] = p.zbl_scale * 0.5f * (14.3996f * Zu * Zv) / rr * phi * envz;
  }
}

__global__ void __launch_bounds__(256) k_edge_bwd(
    int64_t E, const int* __restrict__ sender, const int* __restrict__ receiver,
    const int* __restrict__ species, const float* __restrict__ bessel_w,
    const float* __restrict__ zbl_z, const float* __restrict__ zbl_cov, const float* __restrict__ ag_cov,
    FrontParams p, const EdgeGeom* __restrict__ geom, const float* __restrict__ gY, int gyp,
    const float* __restrict__ gef, float* __restrict__ gv, double* __restrict__ vir_part,
    const float* __restrict__ gcut) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  double vir[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) vir[k] = 0.0;
  if (e < E) {
    const EdgeGeom g = geom[e];
    const float rr = g.r;
    const float inv = 1.f / rr;
    const float ux = g.x * inv, uy = g.y * inv, uz = g.z * inv;
    float Yl[16];
    sh16(ux, uy, uz, Yl);
    float G[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) G[k] = gY[16 * gyp * e + k];
    for (int q = 1; q < gyp; ++q)  // the TP VJP's partials (channel slices / slot groups), in order
#pragma unroll
      for (int k = 0; k < 16; ++k) G[k] += gY[16 * (gyp * e + q) + k];
    // reverse through the recursion (l = 3, then l = 2)
#pragma unroll
    for (int t = 0; t < SH3_NT; ++t) {
      const float gk = G[9 + SH3_K[t]] * SH3_V[t];
      G[4 + SH3_I[t]] += gk * Yl[1 + SH3_J[t]];
      G[1 + SH3_J[t]] += gk * Yl[4 + SH3_I[t]];
    }
#pragma unroll
    for (int t = 0; t < SH2_NT; ++t) {
      const float gk = G[4 + SH2_K[t]] * SH2_V[t];
      G[1 + SH2_I[t]] += gk * Yl[1 + SH2_J[t]];
      G[1 + SH2_J[t]] += gk * Yl[1 + SH2_I[t]];
    }
    const float gux = SQRT3 * G[1], guy = SQRT3 * G[2], guz = SQRT3 * G[3];
    const float dot = gux * ux + guy * uy + guz * uz;
    float gx = (gux - dot * ux) * inv, gy = (guy - dot * uy) * inv, gz = (guz - dot * uz) * inv;
    // radial part
    float denv;
    const float env = poly_env(rr / p.r_max, p.pcut, &denv);
    float rb = rr, drb = 1.f;  // Bessel argument and its derivative in r
    if (p.agnesi) rb = agnesi_t(rr, 0.5f * (ag_cov[species[sender[e]]] + ag_cov[species[receiver[e]]]), p, &drb);
    // with a separate cutoff the features are the basis alone and dL/dcut enters here
    float gr = p.apply_cutoff ? 0.f : gcut[e] * denv / p.r_max;
    const float envb = p.apply_cutoff ? env : 1.f, denvb = p.apply_cutoff ? denv : 0.f;
    for (int n = 0; n < p.nbessel; ++n) {
      const float w = bessel_w[n];
      float b, db;
      if (rb == 0.f) {
        b = p.bessel_pref * w;
        db = 0.f;
      } else {
        float sn, cs;
        sincosf(w * rb, &sn, &cs);
        b = p.bessel_pref * sn / rb;
        db = p.bessel_pref * (w * cs * rb - sn) / (rb * rb);
      }
      gr += gef[(int64_t)p.nbessel * e + n] * (db * drb * envb + b * denvb / p.r_max);
    }
    if (p.has_zbl) {
      const int zs = species[sender[e]], zr = species[receiver[e]];
      const float Zu = zbl_z[zs], Zv = zbl_z[zr];
      const float a = p.zbl_a_pref * 0.529f / (powf(Zu, p.zbl_a_exp) + powf(Zv, p.zbl_a_exp));
      float dphi;
      const float phi = zbl_phi(rr / a, &dphi);
      const float rmax = zbl_cov[zs] + zbl_cov[zr];
      float dz;
      const float envz = poly_env(rr / rmax, p.zbl_p, &dz);
      const float K = p.zbl_scale * 0.5f * 14.3996f * Zu * Zv;
      gr += K * ((dphi / a) / rr * envz - phi / (rr * rr) * envz + phi / rr * dz / rmax);
    }
    gx += gr * ux;
    gy += gr * uy;
    gz += gr * uz;
    gv[3 * e] = gx;
    gv[3 * e + 1] = gy;
    gv[3 * e + 2] = gz;
    const float v[3] = {g.x, g.y, g.z}, gg[3] = {gx, gy, gz};
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) vir[3 * a + b] = (double)v[a] * (double)gg[b];
  }
  if (vir_part == nullptr) return;
  __shared__ double red[9][256];
#pragma unroll
  for (int k = 0; k < 9; ++k) red[k][threadIdx.x] = vir[k];
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off)
#pragma unroll
      for (int k = 0; k < 9; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x < 9) vir_part[9 * blockIdx.x + threadIdx.x] = red[threadIdx.x][0];
}

// ---------------------------------------------------------------------------
// density normalisation (blocks.py:282-490): one wave per node, fixed-order sums
// ---------------------------------------------------------------------------
__device__ __forceinline__ float edge_density_arg(const float* __restrict__ ef, int nb, const float* __restrict__ wd,
                                                  int64_t e) {
  float s = 0.f;
  for (int k = 0; k < nb; ++k) s = fmaf(ef[e * nb + k], wd[k], s);
  return s;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__global__ void __launch_bounds__(256) k_density_fwd(int N, const int* __restrict__ rowptr,
                                                     const float* __restrict__ ef, int nb,
                                                     const float* __restrict__ wd, float* __restrict__ rinv) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (n >= N) return;
  float acc = 0.f;
  for (int e = rowptr[n] + l; e < rowptr[n + 1]; e += 64) {
    const float s = edge_density_arg(ef, nb, wd, e);
    acc += tanhf(s * s);
  }
  acc = wave_sum_f(acc);
  if (l == 0) rinv[n] = 1.f / (1.f + acc);
}

__global__ void __launch_bounds__(256) k_density_node_bwd(int N, int dint, const float* __restrict__ gA,
                                                          const float* __restrict__ A, const float* __restrict__ rinv,
                                                          float* __restrict__ grho) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (n >= N) return;
  const float* g = gA + (int64_t)n * dint;
  const float* a = A + (int64_t)n * dint;
  float acc = 0.f;
  for (int j = l; j < dint; j += 64) acc = fmaf(g[j], a[j], acc);
  acc = wave_sum_f(acc);
  if (l == 0) grho[n] = -rinv[n] * acc;
}

__global__ void __launch_bounds__(256) k_density_edge_bwd(int64_t E, const int* __restrict__ receiver,
                                                          const float* __restrict__ ef, int nb,
                                                          const float* __restrict__ wd, const float* __restrict__ grho,
                                                          float* __restrict__ gef) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const float s = edge_density_arg(ef, nb, wd, e);
  const float d = tanhf(s * s);
  const float c = grho[receiver[e]] * (1.f - d * d) * 2.f * s;
  for (int k = 0; k < nb; ++k) gef[e * nb + k] += c * wd[k];
}

// ---------------------------------------------------------------------------
// neighbour list
// ---------------------------------------------------------------------------

__device__ __forceinline__ int floordiv(int a, int b) {
  int q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

// Atoms [i0, i0 + n) form one structure (a batch is a union of structures, each in its own
// cell); its bins are numbered from bin_off so that all structures share one sorted bin array.
// iota[i] = i: the values of the sort by bin; pos_build: the positions of this build (the
// reference of the skin criterion).
// Atom i's wrapped position w (cell coordinates) and image, and its bin (returned)
__device__ __forceinline__ int nl_bin_atom(int i, const double* __restrict__ pos, const NLParams& p, int bin_off,
                                           double* __restrict__ pos_build, double* wpos_i, int* img_i) {
  for (int k = 0; k < 3; ++k) pos_build[3 * i + k] = pos[3 * i + k];
  const double d0 = pos[3 * i] - p.origin[0], d1 = pos[3 * i + 1] - p.origin[1],
               d2 = pos[3 * i + 2] - p.origin[2];
  double f[3], w[3];
  int b[3];
  for (int k = 0; k < 3; ++k) {
    f[k] = d0 * p.inv[0 * 3 + k] + d1 * p.inv[1 * 3 + k] + d2 * p.inv[2 * 3 + k];
    int n = 0;
    if (p.periodic[k]) {
      n = (int)floor(f[k]);
      w[k] = f[k] - (double)n;
      if (w[k] >= 1.0) {  // rounding guard
        w[k] -= 1.0;
        n += 1;
      }
    } else {
      w[k] = f[k];
    }
    img_i[k] = n;
    int bk = (int)floor(w[k] * p.nbin[k]);
    bk = bk < 0 ? 0 : (bk >= p.nbin[k] ? p.nbin[k] - 1 : bk);
    b[k] = bk;
  }
  for (int k = 0; k < 3; ++k)
    wpos_i[k] = w[0] * p.cell[0 * 3 + k] + w[1] * p.cell[1 * 3 + k] + w[2] * p.cell[2 * 3 + k];
  return bin_off + (b[0] * p.nbin[1] + b[1]) * p.nbin[2] + b[2];
}

__global__ void k_nl_bin(int i0, int n, const double* __restrict__ pos, NLParams p, int bin_off,
                         double* __restrict__ wpos, int* __restrict__ img, int* __restrict__ bin,
                         int* __restrict__ iota, double* __restrict__ pos_build) {
  if ((int)(blockIdx.x * blockDim.x + threadIdx.x) >= n) return;
  const int i = i0 + blockIdx.x * blockDim.x + threadIdx.x;
  iota[i] = i;
  double w[3];
  int im[3];
  bin[i] = nl_bin_atom(i, pos, p, bin_off, pos_build, w, im);
  for (int k = 0; k < 3; ++k) wpos[3 * i + k] = w[k], img[3 * i + k] = im[k];
}

// One structure of at most kNlSmall atoms in one block, in place of k_nl_bin + the device-wide
// sort by bin + k_key_starts (ten launches for a few microseconds of work each): thread t bins
// atom t, a block radix sort (stable: the atoms of a bin stay in index order) orders the
// atoms by bin, and each bin's first position is a binary search over the sorted bins.
// Padding entries take the key nbins, past every bin.
__global__ void __launch_bounds__(kNlSmall) k_nl_prep_small(int n, const double* __restrict__ pos, NLParams p,
                                                            int nbins, int key_bits, double* __restrict__ wpos,
                                                            int* __restrict__ img, int* __restrict__ bin,
                                                            double* __restrict__ pos_build,
                                                            int* __restrict__ bin_sorted, int* __restrict__ atoms,
                                                            int* __restrict__ bin_start, double* __restrict__ wpos_s,
                                                            int* __restrict__ img_s) {
  using Sort = hipcub::BlockRadixSort<int, kNlSmall, 1, int>;
  __shared__ typename Sort::TempStorage tmp;
  __shared__ int sk[kNlSmall];
  __shared__ double sw[kNlSmall][3];
  __shared__ int si[kNlSmall][3];
  const int t = threadIdx.x;
  int key[1] = {nbins}, val[1] = {t};
  if (t < n) {
    double w[3];
    int im[3];
    key[0] = nl_bin_atom(t, pos, p, 0, pos_build, w, im);
    bin[t] = key[0];
    for (int k = 0; k < 3; ++k) {
      wpos[3 * t + k] = w[k], img[3 * t + k] = im[k];
      sw[t][k] = w[k], si[t][k] = im[k];
    }
  }
  __syncthreads();  // sw / si complete before any thread reads them below
  Sort(tmp).Sort(key, val, 0, key_bits);
  sk[t] = key[0];
  if (t < n) {
    const int a = val[0];
    bin_sorted[t] = key[0];
    atoms[t] = a;
    for (int k = 0; k < 3; ++k) wpos_s[3 * t + k] = sw[a][k], img_s[3 * t + k] = si[a][k];
  }
  __syncthreads();
  for (int b = t; b <= nbins; b += kNlSmall) {
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sk[mid] < b) lo = mid + 1; else hi = mid;
    }
    bin_start[b] = lo;
  }
}

// out[i] = in[0] + .. + in[i - 1] for i < n <= 2 kNlSmall, in one block
__global__ void __launch_bounds__(kNlSmall) k_exclusive_sum_small(int n, const int* __restrict__ in,
                                                                  int* __restrict__ out) {
  using Scan = hipcub::BlockScan<int, kNlSmall>;
  __shared__ typename Scan::TempStorage tmp;
  int v[2];
  for (int q = 0; q < 2; ++q) {
    const int i = 2 * threadIdx.x + q;
    v[q] = i < n ? in[i] : 0;
  }
  Scan(tmp).ExclusiveSum(v, v);
  for (int q = 0; q < 2; ++q) {
    const int i = 2 * threadIdx.x + q;
    if (i < n) out[i] = v[q];
  }
}

// One wave per receiver atom j.  Its neighbour cells, in a fixed order (o0 outer, o2 inner),
// are taken 64 at a time: lane k looks up cell k's image shift T and atom range, a wave
// prefix sum lays the cells' atoms out as one candidate range, and the lanes test those
// candidates 64 at a time (a lane finds its candidate's cell by a binary search over the
// prefix sums in LDS).  Hits are counted with a ballot, and in the fill pass each hit lane
// writes at the running count plus its rank among the hit lanes, so the edge order (cell
// order, then position in the cell) is deterministic and identical in both passes.
struct NLWaveScratch {
  int end[64];    // inclusive prefix sums of the chunk's cell sizes
  int start[64];  // first entry of each cell in bin_atoms
  int T[64][3];   // image shift of each cell
};

// wpos_s / img_s: the wrapped positions and images in bin order (entry s of bin_atoms), so that a
// candidate's position is read at its slot, in parallel with its atom index.
//
// Reverse edges without a search.  A receiver's cells are visited in a fixed order k = 0 ..
// ncell - 1 of their offsets o in [-r, r]^3, and negating the offset maps k to ncell - 1 - k.
// If receiver j finds atom i through cell k (image T), then i finds j through cell
// ncell - 1 - k (image -T, the bin of j), among the atoms of j's bin in slot order, and with the
// same distance bit for bit.  The count pass therefore stores, per receiver and cell, the number
// of edges of its row before that cell (cpre, row stride cstride >= ncell + 1), and the fill
// pass places the reverse of each edge it writes at rowptr[i] + cpre[i][ncell - 1 - k] + the
// number of atoms of j's bin before j that i also reaches through that cell (usually none or
// one: bins are half a cutoff wide).  perm_s = pos_s = that position (the reverse map is an
// involution).  A position outside that cell's range means the list is not symmetric: the edge
// maps to itself and is counted in *missing.
// What the fill pass writes for one edge e = (i -> j) of row j at position o: sender, receiver,
// shift, and the position of its reverse (perm_s = pos_s).  slot: i's slot in bin order; k and
// T: the cell of the receiver's visit that holds that image of i.
struct NLFillCtx {
  int j, jb0, jslot, ncell, cstride;
  double xj, yj, zj;
};
__device__ __forceinline__ void nl_emit(const NLParams& p, const NLFillCtx& f, int o, int i, int slot, int k,
                                        const int* Tc, const double* __restrict__ wpos_s,
                                        const int* __restrict__ img, const int* __restrict__ img_s,
                                        const int* __restrict__ bin_atoms, const int* __restrict__ rowptr,
                                        const int* __restrict__ cpre, int* __restrict__ sender,
                                        int* __restrict__ receiver, int* __restrict__ shifts,
                                        int* __restrict__ perm_s, int* __restrict__ pos_s,
                                        int* __restrict__ missing) {
  const int j = f.j;
  sender[o] = i;
  receiver[o] = j;
  // D = x_j - x_i + S.cell with x = wpos + img.cell  =>  S = -T - img_j + img_i
  shifts[3 * o + 0] = -Tc[0] - img[3 * j + 0] + img_s[3 * slot + 0];
  shifts[3 * o + 1] = -Tc[1] - img[3 * j + 1] + img_s[3 * slot + 1];
  shifts[3 * o + 2] = -Tc[2] - img[3 * j + 2] + img_s[3 * slot + 2];
  // the reverse (j -> i, -S): row i, cell kr, after the atoms of j's bin before j that i
  // reaches through it (i's visit: receiver i, candidate a, image -Tc, same expression)
  const int kr = f.ncell - 1 - k;
  const int R0 = -Tc[0], R1 = -Tc[1], R2 = -Tc[2];
  const double rx = R0 * p.cell[0] + R1 * p.cell[3] + R2 * p.cell[6];
  const double ry = R0 * p.cell[1] + R1 * p.cell[4] + R2 * p.cell[7];
  const double rz = R0 * p.cell[2] + R1 * p.cell[5] + R2 * p.cell[8];
  const double xi = wpos_s[3 * slot], yi = wpos_s[3 * slot + 1], zi = wpos_s[3 * slot + 2];
  int rank = 0;
  for (int s2 = f.jb0; s2 < f.jslot; ++s2) {
    if (bin_atoms[s2] == i && R0 == 0 && R1 == 0 && R2 == 0) continue;
    const double dx = (xi - wpos_s[3 * s2]) - rx, dy = (yi - wpos_s[3 * s2 + 1]) - ry,
                 dz = (zi - wpos_s[3 * s2 + 2]) - rz;
    rank += dx * dx + dy * dy + dz * dz < p.cutoff2 ? 1 : 0;
  }
  const int* ci = cpre + (int64_t)i * f.cstride + kr;
  const int ri = rowptr[i];
  int rv = ri + ci[0] + rank;
  if (rv >= ri + ci[1]) {
    atomicAdd(missing, 1);
    rv = o;
  }
  perm_s[o] = rv;
  pos_s[o] = rv;
}

// The receiver j's bin coordinates (b0, b1, b2 within its structure's bins) and the image shift
// of its candidate cell k (offset o in [-r, r]^3, k = o0 outer, o2 inner); false when the cell
// lies outside a non-periodic direction
__device__ __forceinline__ bool nl_cell(const NLParams& p, int b0, int b1, int b2, int k, int* T, int* c) {
  const int n1 = 2 * p.range[1] + 1, n2 = 2 * p.range[2] + 1;
  const int o[3] = {k / (n1 * n2) - p.range[0], (k / n2) % n1 - p.range[1], k % n2 - p.range[2]};
  const int bb[3] = {b0, b1, b2};
  bool ok = true;
  for (int d = 0; d < 3; ++d) {
    c[d] = bb[d] + o[d];
    T[d] = 0;
    if (p.periodic[d]) {
      T[d] = floordiv(c[d], p.nbin[d]);
      c[d] -= T[d] * p.nbin[d];
    } else if (c[d] < 0 || c[d] >= p.nbin[d]) {
      ok = false;
    }
  }
  return ok;
}

// The count pass also records each hit of receiver j, in row order, as (slot, cell index) in
// hits[j][0 .. hcap): the fill pass then writes the rows from those lists without testing any
// distance again (a receiver with more than hcap hits is visited again in full).
template <bool FILL>
__device__ __forceinline__ int nl_visit(int j, const NLParams& p, int bin_off, const double* __restrict__ wpos,
                                        const double* __restrict__ wpos_s, const int* __restrict__ img,
                                        const int* __restrict__ img_s, const int* __restrict__ bin,
                                        const int* __restrict__ bin_start, const int* __restrict__ bin_atoms,
                                        const int* __restrict__ rowptr, int cstride, int* __restrict__ cpre,
                                        int2* __restrict__ hits, int hcap, int* __restrict__ sender,
                                        int* __restrict__ receiver, int* __restrict__ shifts,
                                        int* __restrict__ perm_s, int* __restrict__ pos_s,
                                        int* __restrict__ missing, NLWaveScratch& sc) {
  const int lane = __lane_id();
  const int bj = bin[j] - bin_off;
  const int b2 = bj % p.nbin[2], b1 = (bj / p.nbin[2]) % p.nbin[1], b0 = bj / (p.nbin[2] * p.nbin[1]);
  const double xj = wpos[3 * j], yj = wpos[3 * j + 1], zj = wpos[3 * j + 2];
  const int ncell = (2 * p.range[0] + 1) * (2 * p.range[1] + 1) * (2 * p.range[2] + 1);
  // fill pass: the slots of j's own bin before j (wave-uniform: every lane scans the same few)
  NLFillCtx f{j, 0, 0, ncell, cstride, xj, yj, zj};
  int out0 = 0;
  if constexpr (FILL) {
    out0 = rowptr[j];
    f.jb0 = bin_start[bin[j]];
    const int jb1 = bin_start[bin[j] + 1];
    for (f.jslot = f.jb0; f.jslot < jb1 && bin_atoms[f.jslot] != j;) ++f.jslot;  // j is in its bin
  }
  int cnt = 0;
  for (int k0 = 0; k0 < ncell; k0 += 64) {
    // lane k: cell k0 + k (size 0 when past the end or outside a non-periodic direction)
    int size = 0, first = 0, T[3] = {0, 0, 0};
    const int k = k0 + lane;
    if (k < ncell) {
      int c[3];
      if (nl_cell(p, b0, b1, b2, k, T, c)) {
        const int cb = bin_off + (c[0] * p.nbin[1] + c[1]) * p.nbin[2] + c[2];
        first = bin_start[cb];
        size = bin_start[cb + 1] - first;
      }
    }
    int incl = size;  // inclusive prefix sum over the lanes
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off);
      if (lane >= off) incl += v;
    }
    sc.end[lane] = incl;
    sc.start[lane] = first;
    sc.T[lane][0] = T[0], sc.T[lane][1] = T[1], sc.T[lane][2] = T[2];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    const int total = __shfl(incl, 63);
    const int cnt0 = cnt;
    int ccnt = 0;  // count pass: hits in this lane's cell
    for (int t0 = 0; t0 < total; t0 += 64) {
      const int t = t0 + lane;
      bool hit = false;
      int i = 0, lo = 0, slot = 0, Tc[3] = {0, 0, 0};
      if (t < total) {
        int hi = 63;  // first cell whose inclusive end exceeds t
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (sc.end[mid] > t) hi = mid;
          else lo = mid + 1;
        }
        const int before = lo > 0 ? sc.end[lo - 1] : 0;
        slot = sc.start[lo] + (t - before);
        i = bin_atoms[slot];
        const double xi = wpos_s[3 * slot], yi = wpos_s[3 * slot + 1], zi = wpos_s[3 * slot + 2];
        Tc[0] = sc.T[lo][0], Tc[1] = sc.T[lo][1], Tc[2] = sc.T[lo][2];
        if (!(i == j && Tc[0] == 0 && Tc[1] == 0 && Tc[2] == 0)) {
          const double tx = Tc[0] * p.cell[0] + Tc[1] * p.cell[3] + Tc[2] * p.cell[6];
          const double ty = Tc[0] * p.cell[1] + Tc[1] * p.cell[4] + Tc[2] * p.cell[7];
          const double tz = Tc[0] * p.cell[2] + Tc[1] * p.cell[5] + Tc[2] * p.cell[8];
          // image of atom i at wpos_i + T.cell; D = (x_j - x_i) - T.cell, rounded so that the
          // reverse pair (i, j, -T) gets exactly -D: the list is symmetric bit for bit
          const double dx = (xj - xi) - tx, dy = (yj - yi) - ty, dz = (zj - zi) - tz;
          hit = dx * dx + dy * dy + dz * dz < p.cutoff2;
        }
      }
      const unsigned long long m = __ballot(hit);
      const int rank = cnt + __popcll(m & ((1ull << lane) - 1ull));  // the hit's place in the row
      if constexpr (!FILL) {  // this lane's cell covers candidates [incl - size, incl)
        const int a = max(incl - size - t0, 0), b = min(incl - t0, 64);
        if (b > a) {
          const unsigned long long hm = b == 64 ? ~0ull : (1ull << b) - 1ull;
          ccnt += __popcll(m & hm & ~((1ull << a) - 1ull));
        }
        if (hit && rank < hcap) hits[(int64_t)j * hcap + rank] = make_int2(slot, k0 + lo);
      }
      if (FILL && hit)
        nl_emit(p, f, out0 + rank, i, slot, k0 + lo, Tc, wpos_s, img, img_s, bin_atoms, rowptr, cpre, sender,
                receiver, shifts, perm_s, pos_s, missing);
      cnt += __popcll(m);
    }
    if constexpr (!FILL) {  // cpre[j][k0 + lane] = edges of the row before this cell
      int ex = ccnt;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(ex, off);
        if (lane >= off) ex += v;
      }
      if (k < ncell) cpre[(int64_t)j * cstride + k] = cnt0 + ex - ccnt;
    }
    // the scratch is rewritten by the next chunk only after every lane is done with it
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  if (!FILL && lane == 0) cpre[(int64_t)j * cstride + ncell] = cnt;
  return cnt;
}

// four receiver atoms per 256-thread block, one wave each
// also clears *tail (the count slot past the last atom, so that the exclusive scan ends on the
// total) and *missing (the reverse-edge check's counter)
__global__ void __launch_bounds__(256) k_nl_count(int i0, int n, NLParams p, int bin_off,
                                                  const double* __restrict__ wpos, const double* __restrict__ wpos_s,
                                                  const int* __restrict__ bin, const int* __restrict__ bin_start,
                                                  const int* __restrict__ bin_atoms, int cstride,
                                                  int* __restrict__ cpre, int2* __restrict__ hits, int hcap,
                                                  int* __restrict__ counts, int* __restrict__ tail,
                                                  int* __restrict__ missing) {
  __shared__ NLWaveScratch sc[4];
  if (blockIdx.x == 0 && threadIdx.x == 0) *tail = 0, *missing = 0;
  if ((int)(blockIdx.x * 4 + (threadIdx.x >> 6)) >= n) return;
  const int j = i0 + blockIdx.x * 4 + (threadIdx.x >> 6);
  const int c = nl_visit<false>(j, p, bin_off, wpos, wpos_s, nullptr, nullptr, bin, bin_start, bin_atoms, nullptr,
                                cstride, cpre, hits, hcap, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                sc[threadIdx.x >> 6]);
  if (__lane_id() == 0) counts[j] = c;
}

// A receiver whose hits the count pass recorded (no more than hcap) writes its row from them:
// lane t takes hits t, t + 64, ... (slot and cell index; the cell's image shift follows from the
// index); others are visited again in full.
__global__ void __launch_bounds__(256) k_nl_fill(int i0, int n, NLParams p, int bin_off,
                                                 const double* __restrict__ wpos, const double* __restrict__ wpos_s,
                                                 const int* __restrict__ img, const int* __restrict__ img_s,
                                                 const int* __restrict__ bin, const int* __restrict__ bin_start,
                                                 const int* __restrict__ bin_atoms, const int* __restrict__ rowptr,
                                                 int cstride, const int* __restrict__ cpre,
                                                 const int2* __restrict__ hits, int hcap, int* __restrict__ sender,
                                                 int* __restrict__ receiver, int* __restrict__ shifts,
                                                 int* __restrict__ perm_s, int* __restrict__ pos_s,
                                                 int* __restrict__ missing) {
  __shared__ NLWaveScratch sc[4];
  if ((int)(blockIdx.x * 4 + (threadIdx.x >> 6)) >= n) return;
  const int j = i0 + blockIdx.x * 4 + (threadIdx.x >> 6);
  const int out0 = rowptr[j], cnt = rowptr[j + 1] - out0;
  if (cnt > hcap) {
    nl_visit<true>(j, p, bin_off, wpos, wpos_s, img, img_s, bin, bin_start, bin_atoms, rowptr, cstride,
                   const_cast<int*>(cpre), nullptr, 0, sender, receiver, shifts, perm_s, pos_s, missing,
                   sc[threadIdx.x >> 6]);
    return;
  }
  const int bj = bin[j] - bin_off;
  const int b2 = bj % p.nbin[2], b1 = (bj / p.nbin[2]) % p.nbin[1], b0 = bj / (p.nbin[2] * p.nbin[1]);
  NLFillCtx f{j, bin_start[bin[j]], 0, (2 * p.range[0] + 1) * (2 * p.range[1] + 1) * (2 * p.range[2] + 1),
              cstride, wpos[3 * j], wpos[3 * j + 1], wpos[3 * j + 2]};
  const int jb1 = bin_start[bin[j] + 1];
  for (f.jslot = f.jb0; f.jslot < jb1 && bin_atoms[f.jslot] != j;) ++f.jslot;  // j is in its bin
  const int2* hj = hits + (int64_t)j * hcap;
  for (int t = __lane_id(); t < cnt; t += 64) {
    const int2 h = hj[t];
    int T[3], c[3];
    nl_cell(p, b0, b1, b2, h.y, T, c);
    nl_emit(p, f, out0 + t, bin_atoms[h.x], h.x, h.y, T, wpos_s, img, img_s, bin_atoms, rowptr, cpre, sender,
            receiver, shifts, perm_s, pos_s, missing);
  }
}

// *flag = 1 when some atom moved by more than sqrt(thr2) since pos_build (every writer stores
// the same value, so the order does not matter)
__global__ void k_max_disp(int n, const double* __restrict__ pos, const double* __restrict__ pos_build,
                           double thr2, int* __restrict__ flag) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  double d2 = 0.0;
  for (int k = 0; k < 3; ++k) {
    const double d = pos[3 * i + k] - pos_build[3 * i + k];
    d2 += d * d;
  }
  if (d2 > thr2) *flag = 1;
}

// start[b] = first position of key b in the sorted keys[0 .. n) (b = 0 .. nbins): the CSR of a
// sorted key array by binary search, with no counts to clear or scan
// The neighbour-list build also gathers the wrapped positions and images in bin order (slot r
// of the sorted atoms), when wpos is given.
__global__ void k_key_starts(int n, const int* __restrict__ keys, int nbins, int* __restrict__ start,
                             const int* __restrict__ atoms, const double* __restrict__ wpos,
                             const int* __restrict__ img, double* __restrict__ wpos_s, int* __restrict__ img_s) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (wpos && b < n) {
    const int a = atoms[b];
    for (int k = 0; k < 3; ++k) wpos_s[3 * b + k] = wpos[3 * a + k], img_s[3 * b + k] = img[3 * a + k];
  }
  if (b > nbins) return;
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (keys[mid] < b) lo = mid + 1; else hi = mid;
  }
  start[b] = lo;
}

__global__ void k_iota(int n, int* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = i;
}

__global__ void k_count_keys(int64_t E, const int* __restrict__ keys, int* __restrict__ counts) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < E) atomicAdd(&counts[keys[e]], 1);  // integer counts: order-independent
}

}  // namespace

static inline unsigned nblk(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

void launch_edge_fwd(hipStream_t st, int64_t E, const double* pos, const int* sender, const int* receiver,
                     const int* shifts, const int* species, const float* bessel_w, const float* zbl_z,
                     const float* zbl_cov, const float* ag_cov, const FrontParams& p, const double* gcell,
                     const int* gid, EdgeGeom* geom, float* Y, float* ef, float* zbl_e, float* Mt, int mts,
                     int nent, float* cut) {
  if (E <= 0) return;
#define MACE_EDGE_FWD(NE)                                                                                      \
  MACE_LAUNCH(k_edge_fwd<NE>, dim3(nblk(E, 256)), dim3(256), 0, st, E, pos, sender, receiver, shifts, \
                     species, bessel_w, zbl_z, zbl_cov, ag_cov, p, gcell, gid, geom, Y, ef, zbl_e, Mt, mts, cut)
  if (nent == 0) MACE_EDGE_FWD(0);
  else if (nent == TP3_M1_NE) MACE_EDGE_FWD(TP3_M1_NE);
  else MACE_EDGE_FWD(TP3_M1_NE + TP3_M2_NE);
#undef MACE_EDGE_FWD
}

void launch_edge_bwd(hipStream_t st, int64_t E, const int* sender, const int* receiver, const int* species,
                     const float* bessel_w, const float* zbl_z, const float* zbl_cov, const float* ag_cov,
                     const FrontParams& p, const EdgeGeom* geom, const float* gY, int gyp, const float* gef,
                     float* gv, double* vir_part, const float* gcut) {
  if (E <= 0) return;
  MACE_LAUNCH(k_edge_bwd, dim3(nblk(E, 256)), dim3(256), 0, st, E, sender, receiver, species,
                     bessel_w, zbl_z, zbl_cov, ag_cov, p, geom, gY, gyp, gef, gv, vir_part, gcut);
}

void launch_density_fwd(hipStream_t st, int N, const int* rowptr, const float* ef, int nb, const float* wd,
                        float* rinv) {
  if (N <= 0) return;
  MACE_LAUNCH(k_density_fwd, dim3(nblk(N, 4)), dim3(256), 0, st, N, rowptr, ef, nb, wd, rinv);
}

void launch_density_node_bwd(hipStream_t st, int N, int dint, const float* gA, const float* A, const float* rinv,
                             float* grho) {
  if (N <= 0) return;
  MACE_LAUNCH(k_density_node_bwd, dim3(nblk(N, 4)), dim3(256), 0, st, N, dint, gA, A, rinv, grho);
}

void launch_density_edge_bwd(hipStream_t st, int64_t E, const int* receiver, const float* ef, int nb,
                             const float* wd, const float* grho, float* gef) {
  if (E <= 0) return;
  MACE_LAUNCH(k_density_edge_bwd, dim3(nblk(E, 256)), dim3(256), 0, st, E, receiver, ef, nb, wd, grho, gef);
}

void launch_nl_bin(hipStream_t st, int i0, int n, const double* pos, const NLParams& p, int bin_off, double* wpos,
                   int* img, int* bin, int* iota, double* pos_build) {
  if (n <= 0) return;
  MACE_LAUNCH(k_nl_bin, dim3(nblk(n, 256)), dim3(256), 0, st, i0, n, pos, p, bin_off, wpos, img, bin, iota,
              pos_build);
}

void launch_nl_prep_small(hipStream_t st, int n, const double* pos, const NLParams& p, int nbins, int key_bits,
                          double* wpos, int* img, int* bin, double* pos_build, int* bin_sorted, int* atoms,
                          int* bin_start, double* wpos_s, int* img_s) {
  if (n <= 0 || n > kNlSmall) throw std::invalid_argument("launch_nl_prep_small: 1 .. kNlSmall atoms");
  MACE_LAUNCH(k_nl_prep_small, dim3(1), dim3(kNlSmall), 0, st, n, pos, p, nbins, key_bits, wpos, img, bin, pos_build,
              bin_sorted, atoms, bin_start, wpos_s, img_s);
}

void launch_exclusive_sum_small(hipStream_t st, int n, const int* in, int* out) {
  if (n <= 0) return;
  if (n > 2 * kNlSmall) throw std::invalid_argument("launch_exclusive_sum_small: at most 2 kNlSmall entries");
  MACE_LAUNCH(k_exclusive_sum_small, dim3(1), dim3(kNlSmall), 0, st, n, in, out);
}

void launch_max_disp(hipStream_t st, int n, const double* pos, const double* pos_build, double thr2, int* flag) {
  if (n <= 0) return;
  MACE_LAUNCH(k_max_disp, dim3(nblk(n, 256)), dim3(256), 0, st, n, pos, pos_build, thr2, flag);
}

void launch_key_starts(hipStream_t st, int n, const int* keys, int nbins, int* start, const int* atoms,
                       const double* wpos, const int* img, double* wpos_s, int* img_s) {
  const int64_t m = std::max<int64_t>((int64_t)nbins + 1, wpos ? n : 0);
  MACE_LAUNCH(k_key_starts, dim3(nblk(m, 256)), dim3(256), 0, st, n, keys, nbins, start, atoms, wpos, img, wpos_s,
              img_s);
}

void launch_nl_count(hipStream_t st, int i0, int n, const NLParams& p, int bin_off, const double* wpos,
                     const double* wpos_s, const int* bin, const int* bin_start, const int* bin_atoms, int cstride,
                     int* cpre, int* hits, int hcap, int* counts, int* tail, int* missing) {
  if (n <= 0) return;
  MACE_LAUNCH(k_nl_count, dim3(nblk(n, 4)), dim3(256), 0, st, i0, n, p, bin_off, wpos, wpos_s, bin, bin_start,
                     bin_atoms, cstride, cpre, reinterpret_cast<int2*>(hits), hcap, counts, tail, missing);
}

void launch_nl_fill(hipStream_t st, int i0, int n, const NLParams& p, int bin_off, const double* wpos,
                    const double* wpos_s, const int* img, const int* img_s, const int* bin, const int* bin_start,
                    const int* bin_atoms, const int* rowptr, int cstride, const int* cpre, const int* hits, int hcap,
                    int* sender, int* receiver, int* shifts, int* perm_s, int* pos_s, int* missing) {
  if (n <= 0) return;
  MACE_LAUNCH(k_nl_fill, dim3(nblk(n, 4)), dim3(256), 0, st, i0, n, p, bin_off, wpos, wpos_s, img, img_s, bin,
                     bin_start, bin_atoms, rowptr, cstride, cpre, reinterpret_cast<const int2*>(hits), hcap, sender,
                     receiver, shifts, perm_s, pos_s, missing);
}

void launch_fill_iota(hipStream_t st, int n, int* out) {
  if (n <= 0) return;
  MACE_LAUNCH(k_iota, dim3(nblk(n, 256)), dim3(256), 0, st, n, out);
}

void launch_count_keys(hipStream_t st, int64_t E, const int* keys, int* counts) {
  if (E <= 0) return;
  MACE_LAUNCH(k_count_keys, dim3(nblk(E, 256)), dim3(256), 0, st, E, keys, counts);
}


}  // namespace mace
