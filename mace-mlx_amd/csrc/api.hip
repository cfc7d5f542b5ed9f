// C ABI of the engine (include/mace_hip.h): context, model upload, topology,
// device neighbour list with skin cache, and the energy / forces / virial step.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mace_hip.h"
#include "common.h"

using namespace mace;

thread_local int64_t mace::g_dispatches = 0;

// Scratch of mace_step_device_noalloc: the per-block energy partials of the readout
// (ceil(N / 4) + 1 doubles) followed by the per-block virial partials of the edge VJP
// (9 ceil(E / 256) doubles).  One copy per device, held until the process ends.  Host
// code never uses the name: its device address, looked up once per device with
// hipGetSymbolAddress, is kept in g_scratch_ptr.
constexpr size_t kScratchDoubles = size_t(1) << 18;  // 2 MiB
static __device__ __align__(256) double scratch[kScratchDoubles];

namespace {

struct Err {
  int code;
};

#define HIPCHK(expr)                                                                          \
  do {                                                                                        \
    hipError_t _e = (expr);                                                                   \
    if (_e != hipSuccess) fail(MACE_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

template <class T>
struct DBuf {
  T* p = nullptr;
  size_t n = 0;
  void ensure(size_t count);
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
};

std::string g_fail_msg;

std::mutex g_scratch_mu;
std::vector<double*> g_scratch_ptr;  // per device ordinal: address of `scratch` there

// partials of dL/dY and dL/dh3 per edge: the receiver VJP writes one per
// channel half; the fused TP VJP one per (input degree, 64-channel slice)
constexpr int kGyMax = 3 * NSLICE;  // dL/dY / dL/dh3 partials per edge, at most
inline int tpx_parts(int lin) { return NSLICE * lin; }  // (channel slice, input block) partials
[[noreturn]] void fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_fail_msg = buf;
  throw Err{code};
}

template <class T>
void DBuf<T>::ensure(size_t count) {
  if (count <= n && p) return;
  release();
  size_t c = std::max<size_t>(count, 1);
  HIPCHK(hipMalloc((void**)&p, c * sizeof(T)));
  n = c;
}

int n_tp_slots(int lin) { return lin == 1 ? TP1_NSLOT : lin == 2 ? TP2_NSLOT : TP3_NSLOT; }
int n_tp_acc(int lin) { return lin == 1 ? TP1_NACC : lin == 2 ? TP2_NACC : TP3_NACC; }
const int* tp_l3(int lin) { return lin == 1 ? TP1_L3 : lin == 2 ? TP2_L3 : TP3_L3; }
const int* tp_accoff(int lin) { return lin == 1 ? TP1_ACC : lin == 2 ? TP2_ACC : TP3_ACC; }
int sc_kt(int lout, int corr) {
  static const int kt[3][3] = {{SC_L0_C1_KT, SC_L0_C2_KT, SC_L0_C3_KT},
                               {SC_L1_C1_KT, SC_L1_C2_KT, SC_L1_C3_KT},
                               {SC_L2_C1_KT, SC_L2_C2_KT, SC_L2_C3_KT}};
  return kt[lout][corr - 1];
}

struct Layer {
  int lin = 1, lhid = 1, corr = 3;
  int din = 0, dhid = 0, dmid = 0, dint = 0, wn = 0;
  DBuf<float> up[3], upT[3], skip[3], skipT[3], mlp[4], mlpT[4], lin_[4], linT[4], sc[3], plin[3], plinT[3];
  DBuf<float> ro, ro1, ro2;
  DBuf<_Float16> mlpT3h, mlp3h;  // fp16 copies of W3^T and W3 (float16 feature policy)
  DBuf<_Float16> mlpT3x, mlp3x;  // [hi | lo] fp16 planes of W3^T and W3 scaled by 1 / w3inv (float32 policy)
  DBuf<unsigned char> mlp_tiles;    // permuted W0..W2 tile images of the hidden-layer kernels
  DBuf<unsigned char> mlp_tiles_x;  // the same, split into fp16 pairs (float32 policy)
  float mlp_winv[3] = {1.f, 1.f, 1.f};
  float w3inv = 1.f;
  bool resid = true;       // residual block (skip from the input); else the skip acts on the message
  DBuf<float> mskip[4], mskipT[4], dens;
  int nskip = 0;
  // per-step activations (TP weights: w, or wh under the float16 feature policy)
  DBuf<float> h_up, A, w;
  DBuf<float> A2, rinv;  // message after its skip FCTP (non-residual block); 1 / (1 + density)
  DBuf<float> ds;        // silu' of the radial MLP's pre-activations, [E][3][64]
  DBuf<_Float16> wh;
  // h3 and its inverse scales kept for this layer's VJP, which rebuilds w from them (a later
  // layer overwrites the shared buffers)
  DBuf<float> h3own, h3invown;
  const void* wptr(bool half) const { return half ? static_cast<const void*>(wh.p) : static_cast<const void*>(w.p); }
  // mh-1 non-linear interaction block (blocks.py:611-807).  The conv TP acts on linear_up's
  // output (ledge blocks, dedge floats per node); lin / din stay the layer input's.
  bool nonlin = false;
  int ledge = 0, dedge = 0;
  int nres = 0;                  // columns of linear_res's output (a prefix of the gate input)
  float alpha = 1.f, beta = 0.f;
  DBuf<float> b3;                // radial-MLP output bias [W]
  DBuf<float> rmlp_ts, rmlp_tt, rmlp_ln, rmlp_bias, dmlp_ts, dmlp_tt, dmlp_ln, dmlp_w1;
  DBuf<unsigned char> dmlp_tiles;  // tile images of the density MLP's first layer (ef part)
  DBuf<float> res_[4], resT[4], lin2[4], lin2T[4];
  DBuf<float> Q, R, Gt;          // per step: linear_1 / (beta rho + alpha), linear_res, gate output
  LnMlpParams lnp() const {
    return LnMlpParams{rmlp_ts.p, rmlp_tt.p, rmlp_ln.p, rmlp_bias.p, dmlp_ts.p, dmlp_tt.p, dmlp_ln.p, dmlp_w1.p,
                       {mlp_winv[0], mlp_winv[1], mlp_winv[2]}};
  }
  int tl() const { return nonlin ? ledge : lin; }  // input blocks of the conv TP
  int dtp() const { return nonlin ? dedge : din; }
};

}  // namespace

struct mace_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  // model
  bool model_ready = false;
  mace_model_dims dims{};
  std::map<std::string, std::vector<float>> host_tensors;
  std::vector<Layer> layers;
  int max_lin = 1;
  int mts = 0;  // row stride of the per-edge TP tables Mt (0: no layer has l1 >= 1 inputs)
  DBuf<float> e0, bessel_w, zbl_z, zbl_cov, ag_cov, embed;
  DBuf<float> up0_tab;  // first linear_up per species [n_el][C]
  DBuf<float> gA2, grho;  // backward scratch of the message skip / density normalisation
  // mh-1: per-edge envelope and its gradient (apply_cutoff = 0), edge densities, gw . b3,
  // dL/d(gate input), all-zero species (element-agnostic product)
  DBuf<float> cutv, gcut, mh_dens, gwb, gP;
  DBuf<int> zero_species;
  DBuf<int> nl_missing;       // edges of the last list build without a reverse edge (device count)
  int* nl_missing_h = nullptr;  // pinned host copy, read after the next synchronisation
  int* e_pinned = nullptr;      // the list build's edge count, read back through pinned memory
  DBuf<double> nl_pos_d;        // positions at the last list build (device skin criterion)
  DBuf<int> skin_flag;
  int* skin_pinned = nullptr;
  bool nl_check_pending = false;  // a list build whose reverse-edge count is not yet read
  bool srow_shared = false;       // sender CSR row pointers = rowptr (symmetric device-built list)
  // system
  int N = 0;
  std::vector<int> species_h;
  double cell[9] = {0};
  uint8_t pbc[3] = {0, 0, 0};
  double skin = 0.5;
  bool system_ready = false;
  // a batch of G structures (G = 1 for mace_set_system): atoms [gptr[g], gptr[g+1]), each with
  // its own cell and pbc; cell / pbc above hold structure 0
  int G = 1;
  std::vector<int> gptr_h{0, 0};
  std::vector<double> gcell_h = std::vector<double>(9, 0.0);
  std::vector<uint8_t> gpbc_h = std::vector<uint8_t>(3, 0);
  DBuf<int> gptr, gid;
  DBuf<double> gcell, eg, gvir;  // per-structure cells, energies, virials
  DBuf<int> species;
  // atoms sorted by species (stable): sp_perm[sp_off[z] .. sp_off[z] + sp_cnt[z]) = the atoms of
  // species z, the row maps of the per-species products
  DBuf<int> sp_perm;
  std::vector<int> sp_cnt, sp_off;
  DBuf<double> pos;
  double* pos_pinned = nullptr;
  size_t pos_pinned_n = 0;
  // neighbour list state
  bool nl_valid = false, edges_manual = false;
  std::vector<double> nl_pos;  // positions at the last rebuild
  int64_t E = 0;
  DBuf<int> sender, receiver, shifts, rowptr, rowptr_s, perm_s, pos_s;
  DBuf<int> nl_img, nl_bin, nl_bin_sorted, nl_atoms, nl_iota, nl_counts, nl_bin_count, nl_bin_start;
  DBuf<double> nl_wpos, nl_wpos_s;
  DBuf<int> nl_img_s, nl_cpre, nl_hits;
  // hits recorded per receiver by the count pass (rows up to this long are written from them):
  // 1.5 x the last build's mean row, at least 128 and at most 1024
  int nl_hcap = 128;
  DBuf<int> e_tmp_i, e_tmp_j, e_tmp_s, e_perm, e_keys;
  DBuf<unsigned char> cub_tmp;
  // per-step edge buffers
  DBuf<EdgeGeom> geom;
  DBuf<float> Y, Mt, ef, zbl_e, gY, gef, gv, gw, gxe, h3;
  DBuf<float> gh3p;  // fused TP VJP: dL/dh3 partials [P][E][64]
  DBuf<_Float16> h3h, gwh;  // radial-MLP hidden output, dL/dw under the float16 feature policy
  DBuf<float> gscale;       // per-(edge, channel half) scale of gwh
  DBuf<float> h3inv;        // per-edge inverse scale of h3 as split fp16 pairs
  DBuf<double> vir_part;
  // node buffers
  std::vector<DBuf<float>> h;  // h[0..L]
  DBuf<float> M, B, gB, gA, gM, gh0, gh1, gup, node_e;
  DBuf<double> out;  // [energy, vir9, forces 3N]
  DBuf<double> e_part;  // per-block energy partials
  double* out_pinned = nullptr;
  float* ne_pinned = nullptr;
  size_t out_pinned_n = 0;
  hipEvent_t ev[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
  double timings[4] = {0, 0, 0, 0};
  bool last_nl = false;
  bool embed_valid = false;  // h0 / first h_up written for the current species and buffers
  // captured step graphs (forward, backward) and what they were captured for
  struct StepGraph {
    hipGraphExec_t exec = nullptr;
    const void* a = nullptr;
    const void* b = nullptr;
    int flag = 0;
  };
  bool use_graphs = true;
  bool split_products = true;  // float32 policy: matrix products on fp16 matrix cores (split operands)
  bool fused_tp = true;        // with split products: radial-MLP output layer fused into the TP kernels
  bool rebuild_w = true;       // half-precision policies: the fused VJP rebuilds w instead of reading it
  struct SplitW {
    DBuf<_Float16> x;  // [hi | lo] planes of the weights scaled by 1 / winv
    float winv = 1.f;
  };
  std::map<const float*, SplitW> wsplit;  // split copies of the grouped-GEMM weights, by device pointer
  StepGraph g_fwd, g_bwd;
  hipStream_t cap_stream = nullptr;  // step graphs are captured here (nothing runs on it)
  // per-launch-site profiling
  bool profiling = false;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_used = 0;
  struct Pending {
    std::string name;
    size_t e0, e1;
  };
  std::vector<Pending> pending;
  std::map<std::string, std::pair<double, int64_t>> prof_acc;
  std::vector<std::string> launch_log;  // site of every dispatch of the last profiled step
  double* scratch = nullptr;            // this device's `scratch` (mace_step_device_noalloc)
};

namespace {

int guard(mace_ctx* ctx, const std::function<void()>& fn) {
  try {
    fn();
    return MACE_OK;
  } catch (const Err& e) {
    if (ctx) ctx->err = g_fail_msg;
    return e.code;
  } catch (const std::exception& e) {
    if (ctx) ctx->err = e.what();
    return MACE_ERR_INVALID;
  }
}

void set_device(mace_ctx* c) { HIPCHK(hipSetDevice(c->device)); }

// Device address of `scratch` on `device` (current), looked up on the first call per device.
double* scratch_on(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= device) g_scratch_ptr.resize(device + 1, nullptr);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) fail(MACE_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[device] = static_cast<double*>(p);
  }
  return g_scratch_ptr[device];
}

size_t prof_event(mace_ctx* c) {
  if (c->ev_used == c->ev_pool.size()) {
    hipEvent_t e;
    HIPCHK(hipEventCreate(&e));
    c->ev_pool.push_back(e);
  }
  return c->ev_used++;
}

// Brackets one kernel launch with HIP events on the context stream when
// profiling is enabled (no-op otherwise).
struct Site {
  mace_ctx* c;
  std::string name;
  size_t e0 = 0;
  int64_t d0 = 0;
  Site(mace_ctx* ctx, std::string nm) : c(ctx), name(std::move(nm)) {
    if (!c->profiling) return;
    e0 = prof_event(c);
    HIPCHK(hipEventRecord(c->ev_pool[e0], c->stream));
    d0 = g_dispatches;
  }
  ~Site() noexcept(false) {
    if (!c->profiling) return;
    const size_t e1 = prof_event(c);
    HIPCHK(hipEventRecord(c->ev_pool[e1], c->stream));
    c->pending.push_back({name, e0, e1});
    for (int64_t k = d0; k < g_dispatches; ++k) c->launch_log.push_back(name);
  }
};

void prof_harvest(mace_ctx* c) {
  if (c->pending.empty()) {
    c->ev_used = 0;
    return;
  }
  HIPCHK(hipStreamSynchronize(c->stream));
  for (auto& p : c->pending) {
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, c->ev_pool[p.e0], c->ev_pool[p.e1]));
    auto& a = c->prof_acc[p.name];
    a.first += ms;
    a.second += 1;
  }
  c->pending.clear();
  c->ev_used = 0;
}

std::string lname(const char* base, size_t l) { return std::string(base) + ".L" + std::to_string(l); }

const std::vector<float>& tensor(mace_ctx* c, const std::string& name, size_t count) {
  auto it = c->host_tensors.find(name);
  if (it == c->host_tensors.end()) fail(MACE_ERR_INVALID, "model tensor '%s' missing", name.c_str());
  if (it->second.size() != count)
    fail(MACE_ERR_INVALID, "model tensor '%s' has %zu values, expected %zu", name.c_str(), it->second.size(), count);
  return it->second;
}

void upload(mace_ctx* c, DBuf<float>& dst, const std::vector<float>& v) {
  dst.ensure(v.size());
  HIPCHK(hipMemcpy(dst.p, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
}

void upload_half(mace_ctx* c, DBuf<_Float16>& dst, const std::vector<float>& v) {
  std::vector<_Float16> h(v.size());
  for (size_t i = 0; i < v.size(); ++i) h[i] = (_Float16)v[i];
  dst.ensure(h.size());
  HIPCHK(hipMemcpy(dst.p, h.data(), h.size() * sizeof(_Float16), hipMemcpyHostToDevice));
}

// v * scale as consecutive fp16 planes [hi | lo], hi = fp16(x), lo = fp16(x - hi)
void upload_split(mace_ctx* c, DBuf<_Float16>& dst, const std::vector<float>& v, float scale) {
  std::vector<_Float16> h(2 * v.size());
  for (size_t i = 0; i < v.size(); ++i) {
    const float x = v[i] * scale;
    const _Float16 hi = (_Float16)x;
    h[i] = hi;
    h[v.size() + i] = (_Float16)(x - (float)hi);
  }
  dst.ensure(h.size());
  HIPCHK(hipMemcpy(dst.p, h.data(), h.size() * sizeof(_Float16), hipMemcpyHostToDevice));
}

// split copy of `count` device floats at p (largest magnitude scaled into [2^14, 2^15))
void make_split(mace_ctx* c, const float* p, size_t count) {
  if (!p || count == 0 || c->wsplit.count(p)) return;
  std::vector<float> h(count);
  HIPCHK(hipMemcpy(h.data(), p, count * sizeof(float), hipMemcpyDeviceToHost));
  float m = 0.f;
  for (float x : h) m = std::max(m, std::fabs(x));
  const int ex = m > 0.f ? std::ilogb(m) : 0;
  auto& sw = c->wsplit[p];
  sw.winv = std::ldexp(1.f, ex - 14);
  upload_split(c, sw.x, h, std::ldexp(1.f, 14 - ex));
}

// The atoms sorted by species (stable) for the model's element count: row maps of the
// per-species products (species_h holds valid indices)
void set_species_order(mace_ctx* c) {
  const int n = (int)c->species_h.size(), nel = c->dims.num_elements;
  c->sp_cnt.assign(nel, 0);
  c->sp_off.assign(nel + 1, 0);
  for (int i = 0; i < n; ++i) ++c->sp_cnt[c->species_h[i]];
  for (int z = 0; z < nel; ++z) c->sp_off[z + 1] = c->sp_off[z] + c->sp_cnt[z];
  std::vector<int> perm(std::max(n, 1), 0), fill(c->sp_off.begin(), c->sp_off.end() - 1);
  for (int i = 0; i < n; ++i) perm[fill[c->species_h[i]]++] = i;
  c->sp_perm.ensure(perm.size());
  HIPCHK(hipMemcpy(c->sp_perm.p, perm.data(), perm.size() * sizeof(int), hipMemcpyHostToDevice));
}

std::vector<float> transpose(const std::vector<float>& a, int rows, int cols, int batch = 1) {
  std::vector<float> t(a.size());
  for (int b = 0; b < batch; ++b)
    for (int i = 0; i < rows; ++i)
      for (int j = 0; j < cols; ++j)
        t[(size_t)b * rows * cols + (size_t)j * rows + i] = a[(size_t)b * rows * cols + (size_t)i * cols + j];
  return t;
}

// split operands of the radial output matrix w3 [64][W]: largest magnitude scaled into [2^14, 2^15)
void upload_w3_split(mace_ctx* c, Layer& L, const std::vector<float>& w3) {
  float m = 0.f;
  for (float x : w3) m = std::max(m, std::fabs(x));
  const int ex = m > 0.f ? std::ilogb(m) : 0;
  L.w3inv = std::ldexp(1.f, ex - 14);
  upload_split(c, L.mlpT3x, transpose(w3, RADIAL_H, L.wn), std::ldexp(1.f, 14 - ex));
  upload_split(c, L.mlp3x, w3, std::ldexp(1.f, 14 - ex));
}

void invalidate_graphs(mace_ctx* c);
void invalidate_node_state(mace_ctx* c);

void free_layers(mace_ctx* c) {
  for (auto& L : c->layers) {
    for (auto* arr : {L.up, L.upT, L.skip, L.skipT, L.sc, L.plin, L.plinT})
      for (int i = 0; i < 3; ++i) arr[i].release();
    for (int i = 0; i < 4; ++i) L.mlp[i].release(), L.mlpT[i].release(), L.lin_[i].release(), L.linT[i].release();
    L.ro.release(), L.ro1.release(), L.ro2.release(), L.h_up.release(), L.A.release(), L.w.release(),
        L.wh.release(), L.mlpT3h.release(), L.mlp3h.release(), L.A2.release(), L.rinv.release(),
        L.dens.release(), L.mlpT3x.release(), L.mlp3x.release(), L.mlp_tiles.release(), L.ds.release(),
        L.mlp_tiles_x.release(), L.b3.release(), L.rmlp_ts.release(), L.rmlp_tt.release(), L.rmlp_ln.release(),
        L.rmlp_bias.release(), L.dmlp_ts.release(), L.dmlp_tt.release(), L.dmlp_ln.release(), L.dmlp_w1.release(),
        L.dmlp_tiles.release(), L.Q.release(), L.R.release(), L.Gt.release(), L.h3own.release(),
        L.h3invown.release();
    for (int i = 0; i < 4; ++i) L.mskip[i].release(), L.mskipT[i].release();
    for (int i = 0; i < 4; ++i) L.res_[i].release(), L.resT[i].release(), L.lin2[i].release(), L.lin2T[i].release();
  }
  c->layers.clear();
  for (auto& kv : c->wsplit) kv.second.x.release();
  c->wsplit.clear();
}

// symmetric contraction, product linear and readout of layer l (both interaction kinds)
void build_product_readout(mace_ctx* c, Layer& L, int l) {
  const auto& d = c->dims;
  const int C = NC;
  const int nel = d.agnostic_product ? 1 : d.num_elements;  // blocks.py:510-533
  const std::string p = "L" + std::to_string(l) + ".";
  for (int b = 0; b < L.lhid; ++b) {
    upload(c, L.sc[b], tensor(c, p + "sc." + std::to_string(b), (size_t)nel * sc_kt(b, L.corr) * C));
    const auto& w = tensor(c, p + "plin." + std::to_string(b), (size_t)C * C);
    upload(c, L.plin[b], w);
    upload(c, L.plinT[b], transpose(w, C, C));
  }
  if (l < d.num_layers - 1) {
    upload(c, L.ro, tensor(c, p + "ro", C));
  } else {
    if (L.lhid != 1) fail(MACE_ERR_UNSUPPORTED, "last layer must be scalar");
    upload(c, L.ro1, tensor(c, p + "ro1", (size_t)C * 16));
    upload(c, L.ro2, tensor(c, p + "ro2", 16));
  }
}

// mh-1 non-linear interaction block (blocks.py:611-733): tensors L<l>.up.<b> (input block b ->
// edge block b), skip.<b> (plain linear, [C][C]), rmlp.{w0 [nb][64], w1, w2 [64][64] ([in][out]),
// ts, tt [n_el][64], ln [3][2][64], bias [2][64], b3 [W]}, mlp.3 [64][W], dmlp.{w0 [nb][64],
// ts, tt [n_el][64], ln [2][64], w1 [65]}, ab [2] (alpha, beta), res.<lo> [C][C or 4C],
// lin.<lo> [slots x C][C or 4C], lin2.<lo> [C][C]
void build_layer_nonlin(mace_ctx* c, Layer& L, int l) {
  const auto& d = c->dims;
  const int C = NC, nel = d.num_elements, nb = d.num_bessel;
  const std::string p = "L" + std::to_string(l) + ".";
  L.nonlin = true;
  L.ledge = d.layer_edge_blocks[l];
  if (L.ledge < 1 || L.ledge > 3) fail(MACE_ERR_UNSUPPORTED, "layer %d edge irreps blocks %d", l, L.ledge);
  if (l == 0 && L.ledge != 1) fail(MACE_ERR_UNSUPPORTED, "first layer edge irreps must be scalar");
  L.dedge = C * L.ledge * L.ledge;
  L.dmid = C * n_tp_acc(L.ledge);
  L.wn = C * n_tp_slots(L.ledge);
  L.nres = 4 * C + C * (L.ledge * L.ledge - 1);
  L.resid = true;
  for (int b = 0; b < std::min(L.lin, L.ledge); ++b) {
    const auto& w = tensor(c, p + "up." + std::to_string(b), (size_t)C * C);
    upload(c, L.up[b], w);
    upload(c, L.upT[b], transpose(w, C, C));
  }
  L.nskip = std::min(L.lin, L.lhid);
  for (int b = 0; b < L.nskip; ++b) {
    const auto& w = tensor(c, p + "skip." + std::to_string(b), (size_t)C * C);
    upload(c, L.skip[b], w);
    upload(c, L.skipT[b], transpose(w, C, C));
  }
  {  // LayerNorm radial MLP and density MLP
    const auto& w0 = tensor(c, p + "rmlp.w0", (size_t)nb * RADIAL_H);
    const auto& w1 = tensor(c, p + "rmlp.w1", (size_t)RADIAL_H * RADIAL_H);
    const auto& w2 = tensor(c, p + "rmlp.w2", (size_t)RADIAL_H * RADIAL_H);
    DBuf<float> t0, t1, t2;
    upload(c, t0, w0), upload(c, t1, w1), upload(c, t2, w2);
    L.mlp_tiles.ensure(mlp_tile_bytes());
    launch_mlp_permute(c->stream, nb, t0.p, t1.p, t2.p, L.mlp_tiles.p);
    {  // split images for the hidden layers on fp16 matrix cores, one power-of-two scale per matrix
      float sc[3];
      const std::vector<float>* ws[3] = {&w0, &w1, &w2};
      for (int k = 0; k < 3; ++k) {
        float m = 0.f;
        for (float x : *ws[k]) m = std::max(m, std::fabs(x));
        const int ex = m > 0.f ? std::ilogb(m) : 0;
        sc[k] = std::ldexp(1.f, 14 - ex);
        L.mlp_winv[k] = std::ldexp(1.f, ex - 14);
      }
      L.mlp_tiles_x.ensure(mlp_tile_x_bytes());
      launch_mlp_permute_x(c->stream, nb, t0.p, t1.p, t2.p, sc, L.mlp_tiles_x.p);
    }
    DBuf<float> d0;
    upload(c, d0, tensor(c, p + "dmlp.w0", (size_t)nb * RADIAL_H));
    L.dmlp_tiles.ensure(mlp_tile_bytes());
    launch_mlp_permute(c->stream, nb, d0.p, t1.p, t2.p, L.dmlp_tiles.p);  // only the first matrix is used
    HIPCHK(hipGetLastError());
    HIPCHK(hipStreamSynchronize(c->stream));
    t0.release(), t1.release(), t2.release(), d0.release();
    upload(c, L.rmlp_ts, tensor(c, p + "rmlp.ts", (size_t)nel * RADIAL_H));
    upload(c, L.rmlp_tt, tensor(c, p + "rmlp.tt", (size_t)nel * RADIAL_H));
    upload(c, L.rmlp_ln, tensor(c, p + "rmlp.ln", (size_t)6 * RADIAL_H));
    upload(c, L.rmlp_bias, tensor(c, p + "rmlp.bias", (size_t)2 * RADIAL_H));
    upload(c, L.b3, tensor(c, p + "rmlp.b3", (size_t)L.wn));
    const auto& w3 = tensor(c, p + "mlp.3", (size_t)RADIAL_H * L.wn);
    upload(c, L.mlp[3], w3);
    upload(c, L.mlpT[3], transpose(w3, RADIAL_H, L.wn));
    upload_w3_split(c, L, w3);
    upload(c, L.dmlp_ts, tensor(c, p + "dmlp.ts", (size_t)nel * RADIAL_H));
    upload(c, L.dmlp_tt, tensor(c, p + "dmlp.tt", (size_t)nel * RADIAL_H));
    upload(c, L.dmlp_ln, tensor(c, p + "dmlp.ln", (size_t)2 * RADIAL_H));
    upload(c, L.dmlp_w1, tensor(c, p + "dmlp.w1", (size_t)RADIAL_H + 1));
    const auto& ab = tensor(c, p + "ab", 2);
    L.alpha = ab[0];
    L.beta = ab[1];
  }
  const int* l3 = tp_l3(L.ledge);
  for (int lo = 0; lo < 4; ++lo) {
    const int cout = lo == 0 ? 4 * C : C;
    int ns = 0;
    for (int s = 0; s < n_tp_slots(L.ledge); ++s) ns += (l3[s] == lo);
    const auto& w = tensor(c, p + "lin." + std::to_string(lo), (size_t)ns * C * cout);
    upload(c, L.lin_[lo], w);
    upload(c, L.linT[lo], transpose(w, ns * C, cout));
    if (lo < L.ledge) {
      const auto& r = tensor(c, p + "res." + std::to_string(lo), (size_t)C * cout);
      upload(c, L.res_[lo], r);
      upload(c, L.resT[lo], transpose(r, C, cout));
    }
    const auto& w2 = tensor(c, p + "lin2." + std::to_string(lo), (size_t)C * C);
    upload(c, L.lin2[lo], w2);
    upload(c, L.lin2T[lo], transpose(w2, C, C));
  }
  build_product_readout(c, L, l);
}

void build_model(mace_ctx* c) {
  invalidate_node_state(c);
  const auto& d = c->dims;
  const int C = NC;
  if (d.num_channels != NC) fail(MACE_ERR_UNSUPPORTED, "num_channels=%d (compiled for %d)", d.num_channels, NC);
  if (d.max_ell != 3) fail(MACE_ERR_UNSUPPORTED, "max_ell=%d (compiled for 3)", d.max_ell);
  if (d.radial_hidden != RADIAL_H || d.radial_depth != 3)
    fail(MACE_ERR_UNSUPPORTED, "radial MLP %dx%d (compiled for 3 hidden layers of %d)", d.radial_depth,
         d.radial_hidden, RADIAL_H);
  if (d.num_bessel < 1 || d.num_bessel > NBESSEL_MAX) fail(MACE_ERR_UNSUPPORTED, "num_bessel=%d", d.num_bessel);
  if (d.num_layers < 1 || d.num_layers > 4) fail(MACE_ERR_UNSUPPORTED, "num_layers=%d", d.num_layers);
  if (d.num_elements < 1) fail(MACE_ERR_INVALID, "num_elements=%d", d.num_elements);
  if (d.feature_half < RND_NONE || d.feature_half > RND_BF16)
    fail(MACE_ERR_INVALID, "feature_half=%d (0 float32, 1 float16, 2 bfloat16)", d.feature_half);
  const int nel = d.num_elements, nb = d.num_bessel;
  upload(c, c->e0, tensor(c, "e0", nel));
  upload(c, c->bessel_w, tensor(c, "bessel_w", nb));
  upload(c, c->embed, tensor(c, "embed", (size_t)nel * C));
  {  // first linear_up as a per-species table: up0[z] = h0[z] W (fp64 sums; rounded values under
     // the half-precision feature policies, as the product would give)
    const auto& emb = tensor(c, "embed", (size_t)nel * C);
    const auto& w = tensor(c, "L0.up.0", (size_t)C * C);
    auto rnd = [&](float x) {
      return d.feature_half == RND_F16 ? (float)(_Float16)x : d.feature_half == RND_BF16 ? round_bf16(x) : x;
    };
    std::vector<float> tab((size_t)nel * C);
    for (int z = 0; z < nel; ++z)
      for (int col = 0; col < C; ++col) {
        double a = 0.0;
        for (int k = 0; k < C; ++k) a += (double)rnd(emb[(size_t)z * C + k]) * w[(size_t)k * C + col];
        tab[(size_t)z * C + col] = rnd((float)a);
      }
    upload(c, c->up0_tab, tab);
  }
  if (d.has_zbl) {
    upload(c, c->zbl_z, tensor(c, "zbl_z", nel));
    upload(c, c->zbl_cov, tensor(c, "zbl_cov", nel));
  }
  if (d.agnesi) upload(c, c->ag_cov, tensor(c, "agnesi_cov", nel));
  free_layers(c);
  c->layers.resize(d.num_layers);
  for (int l = 0; l < d.num_layers; ++l) {
    Layer& L = c->layers[l];
    L.lin = d.layer_in_blocks[l];
    L.lhid = d.layer_hid_blocks[l];
    L.corr = d.correlation[l];
    if (L.lin < 1 || L.lin > 3 || L.lhid < 1 || L.lhid > 3)
      fail(MACE_ERR_UNSUPPORTED, "layer %d irreps blocks in=%d hid=%d", l, L.lin, L.lhid);
    if (L.corr < 1 || L.corr > 3) fail(MACE_ERR_UNSUPPORTED, "correlation %d", L.corr);
    if (l == 0 && L.lin != 1) fail(MACE_ERR_UNSUPPORTED, "first layer input must be scalar");
    if (l > 0 && L.lin != d.layer_hid_blocks[l - 1]) fail(MACE_ERR_INVALID, "layer %d input mismatch", l);
    L.din = C * L.lin * L.lin;
    L.dhid = C * L.lhid * L.lhid;
    L.dint = C * 16;
    L.dmid = C * n_tp_acc(L.lin);
    L.wn = C * n_tp_slots(L.lin);
    if (d.nonlinear) {
      build_layer_nonlin(c, L, l);
      continue;
    }
    if (d.separate_cutoff) fail(MACE_ERR_UNSUPPORTED, "a separate cutoff outside the non-linear interaction block");
    const std::string p = "L" + std::to_string(l) + ".";
    for (int b = 0; b < L.lin; ++b) {
      const auto& w = tensor(c, p + "up." + std::to_string(b), (size_t)C * C);
      upload(c, L.up[b], w);
      upload(c, L.upT[b], transpose(w, C, C));
    }
    L.resid = !(l == 0 && d.first_nonresidual);
    L.nskip = L.resid ? std::min(L.lin, L.lhid) : 0;
    for (int b = 0; b < L.nskip; ++b) {
      const auto& w = tensor(c, p + "skip." + std::to_string(b), (size_t)nel * C * C);
      upload(c, L.skip[b], w);
      upload(c, L.skipT[b], transpose(w, C, C, nel));
    }
    if (!L.resid)
      for (int lo = 0; lo < 4; ++lo) {
        const auto& w = tensor(c, p + "mskip." + std::to_string(lo), (size_t)nel * C * C);
        upload(c, L.mskip[lo], w);
        upload(c, L.mskipT[lo], transpose(w, C, C, nel));
      }
    if (d.density_norm) upload(c, L.dens, tensor(c, p + "dens", nb));
    {
      const int rows[4] = {nb, RADIAL_H, RADIAL_H, RADIAL_H};
      const int cols[4] = {RADIAL_H, RADIAL_H, RADIAL_H, L.wn};
      for (int k = 0; k < 4; ++k) {
        const auto& w = tensor(c, p + "mlp." + std::to_string(k), (size_t)rows[k] * cols[k]);
        upload(c, L.mlp[k], w);
        upload(c, L.mlpT[k], transpose(w, rows[k], cols[k]));
        if (k == 3 && d.feature_half == RND_F16) {
          upload_half(c, L.mlpT3h, transpose(w, rows[k], cols[k]));
          upload_half(c, L.mlp3h, w);
        }
        if (k == 3) upload_w3_split(c, L, w);
      }
      L.mlp_tiles.ensure(mlp_tile_bytes());
      launch_mlp_permute(c->stream, nb, L.mlp[0].p, L.mlp[1].p, L.mlp[2].p, L.mlp_tiles.p);
      {  // split images, one power-of-two scale per matrix (lo planes 0 for rounded weights)
        float sc[3];
        for (int k = 0; k < 3; ++k) {
          float m = 0.f;
          for (float x : tensor(c, p + "mlp." + std::to_string(k), (size_t)rows[k] * cols[k])) m = std::max(m, std::fabs(x));
          const int ex = m > 0.f ? std::ilogb(m) : 0;
          sc[k] = std::ldexp(1.f, 14 - ex);
          L.mlp_winv[k] = std::ldexp(1.f, ex - 14);
        }
        L.mlp_tiles_x.ensure(mlp_tile_x_bytes());
        launch_mlp_permute_x(c->stream, nb, L.mlp[0].p, L.mlp[1].p, L.mlp[2].p, sc, L.mlp_tiles_x.p);
      }
      HIPCHK(hipGetLastError());
      HIPCHK(hipStreamSynchronize(c->stream));
    }
    const int* l3 = tp_l3(L.lin);
    for (int lo = 0; lo < 4; ++lo) {
      int ns = 0;
      for (int s = 0; s < n_tp_slots(L.lin); ++s) ns += (l3[s] == lo);
      const auto& w = tensor(c, p + "lin." + std::to_string(lo), (size_t)ns * C * C);
      upload(c, L.lin_[lo], w);
      upload(c, L.linT[lo], transpose(w, ns * C, C));
    }
    build_product_readout(c, L, l);
  }
  {  // split copies of every weight matrix the grouped products use
    const size_t CC = (size_t)C * C;
    for (Layer& L : c->layers) {
      for (int b = 0; b < L.lin; ++b) make_split(c, L.up[b].p, CC), make_split(c, L.upT[b].p, CC);
      for (int b = 0; b < L.lhid; ++b) make_split(c, L.plin[b].p, CC), make_split(c, L.plinT[b].p, CC);
      // per-species weights (skip connection, message skip): one split copy per element's slice
      const int nsl = L.nonlin ? 1 : c->dims.num_elements;
      for (int z = 0; z < nsl; ++z) {
        for (int b = 0; b < L.nskip; ++b) make_split(c, L.skip[b].p + z * CC, CC), make_split(c, L.skipT[b].p + z * CC, CC);
        if (!L.resid)
          for (int lo = 0; lo < 4; ++lo) make_split(c, L.mskip[lo].p + z * CC, CC), make_split(c, L.mskipT[lo].p + z * CC, CC);
      }
      const int* l3 = tp_l3(L.tl());
      for (int lo = 0; lo < 4; ++lo) {
        size_t ns = 0;
        for (int q = 0; q < n_tp_slots(L.tl()); ++q) ns += (l3[q] == lo);
        const size_t cw = (L.nonlin && lo == 0) ? 4 : 1;  // the mh-1 scalar outputs: 4 C columns
        make_split(c, L.lin_[lo].p, ns * CC * cw), make_split(c, L.linT[lo].p, ns * CC * cw);
        if (L.nonlin) {
          if (lo < L.ledge) make_split(c, L.res_[lo].p, CC * cw), make_split(c, L.resT[lo].p, CC * cw);
          make_split(c, L.lin2[lo].p, CC), make_split(c, L.lin2T[lo].p, CC);
        }
      }
    }
  }
  c->max_lin = 1;
  for (const Layer& L : c->layers) c->max_lin = std::max(c->max_lin, L.tl());
  c->mts = (tp_table_entries(c->max_lin) + 15) / 16 * 16;
  c->host_tensors.clear();
  c->model_ready = true;
}

// ---------------------------------------------------------------------------
// buffers
// ---------------------------------------------------------------------------
void ensure_node_buffers(mace_ctx* c) {
  invalidate_node_state(c);
  const int N = std::max(c->N, 1);
  const int L = (int)c->layers.size();
  c->h.resize(L + 1);
  // work-array row widths: the widest use over the layers (M / dL/dM: dmid; B / dL/dB: dhid;
  // dL/dA: dint; dL/dh: din and dhid; dL/d(up): the conv TP input)
  int wmid = 0, whid = 0, wint = NC * 16, win = 0, wtp = 0;
  for (int l = 0; l < L; ++l) {
    Layer& ly = c->layers[l];
    c->h[l].ensure((size_t)N * ly.din);
    ly.h_up.ensure((size_t)N * ly.dtp());
    ly.A.ensure((size_t)N * ly.dint);
    if (!ly.resid) ly.A2.ensure((size_t)N * ly.dint);
    if (c->dims.density_norm || ly.nonlin) ly.rinv.ensure(N);
    if (ly.nonlin) {
      ly.Q.ensure((size_t)N * kGateInDim);
      ly.R.ensure((size_t)N * ly.nres);
      ly.Gt.ensure((size_t)N * ly.dint);
      c->gP.ensure((size_t)N * kGateInDim);
    }
    wmid = std::max(wmid, ly.dmid);
    whid = std::max(whid, ly.dhid);
    wint = std::max(wint, ly.dint);
    win = std::max(win, ly.din);
    wtp = std::max(wtp, ly.dtp());
  }
  if (c->dims.agnostic_product && c->zero_species.n < (size_t)N) {
    c->zero_species.ensure(N);
    HIPCHK(hipMemset(c->zero_species.p, 0, (size_t)N * sizeof(int)));
  }
  c->h[L].ensure((size_t)N * c->layers[L - 1].dhid);
  c->M.ensure((size_t)N * wmid);
  c->gM.ensure((size_t)N * wmid);
  c->B.ensure((size_t)N * whid);
  c->gB.ensure((size_t)N * whid);
  c->gA.ensure((size_t)N * wint);
  c->gA2.ensure((size_t)N * wint);
  c->gh0.ensure((size_t)N * std::max(win, whid));
  c->gh1.ensure((size_t)N * std::max(win, whid));
  c->gup.ensure((size_t)N * std::max(win, wtp));
  c->grho.ensure(N);
  c->node_e.ensure(N);
  c->e_part.ensure((N + 3) / 4 + 1);

  c->out.ensure(10 + 3 * (size_t)N);
  c->pos.ensure(3 * (size_t)N);
  if (c->out_pinned_n < (size_t)N) {
    if (c->out_pinned) (void)hipHostFree(c->out_pinned);
    if (c->ne_pinned) (void)hipHostFree(c->ne_pinned);
    if (c->pos_pinned) (void)hipHostFree(c->pos_pinned);
    HIPCHK(hipHostMalloc((void**)&c->out_pinned, (10 + 3 * (size_t)N) * sizeof(double), hipHostMallocDefault));
    HIPCHK(hipHostMalloc((void**)&c->ne_pinned, (size_t)N * sizeof(float), hipHostMallocDefault));
    HIPCHK(hipHostMalloc((void**)&c->pos_pinned, 3 * (size_t)N * sizeof(double), hipHostMallocDefault));
    c->out_pinned_n = N;
  }
}

// Which kernels a step runs (from the model and the two switches).  fused: the radial-MLP
// output layer inside the TP kernels (split products), under every feature policy (the
// rounding modes are template parameters of the fused forward; under a half-precision policy the
// non-linear interaction block runs on this path only, check_step_path); split: the radial MLP's
// hidden layers on split-fp16
// products (fused path, or the float32 policy); h16: the float16 policy's separate path with
// fp16 h3 / w / dL/dw arrays.  Neither split nor h16: fp32 products, silu' saved (ds).
struct StepPath {
  bool fused, split, h16;
};
StepPath step_path(const mace_ctx* c) {
  StepPath p;
  p.fused = c->split_products && c->fused_tp;
  p.split = p.fused || (c->dims.feature_half == RND_NONE && c->split_products);
  p.h16 = !p.split && c->dims.feature_half == RND_F16;
  return p;
}

// The fused VJP of layer L rebuilds w from h3 (half-precision policies, one or two input blocks,
// standard interaction block), so its forward does not store w
bool layer_rw(const mace_ctx* c, const Layer& L) {
  return c->rebuild_w && step_path(c).fused && !L.nonlin && tpx_rebuilds_w(L.lin, c->dims.feature_half, false);
}
// layer l's h3 / h3inv: its own buffers when its VJP reads them and a later layer would overwrite
// the shared ones
bool own_h3(const mace_ctx* c, size_t l) { return l + 1 < c->layers.size() && layer_rw(c, c->layers[l]); }
float* h3_of(mace_ctx* c, size_t l) { return own_h3(c, l) ? c->layers[l].h3own.p : c->h3.p; }
float* h3inv_of(mace_ctx* c, size_t l) { return own_h3(c, l) ? c->layers[l].h3invown.p : c->h3inv.p; }

void ensure_edge_buffers(mace_ctx* c, int64_t E) {
  invalidate_graphs(c);
  const size_t e = (size_t)std::max<int64_t>(E, 1);
  int maxw = 0;
  const StepPath path = step_path(c);
  const bool half = path.h16;  // fp16 w / h3 / gw storage
  for (auto& ly : c->layers) {
    if (half)
      ly.wh.ensure(e * ly.wn);
    else
      ly.w.ensure(e * ly.wn);
    maxw = std::max(maxw, ly.wn);
    if (!path.split) ly.ds.ensure(e * 3 * RADIAL_H);
  }
  if (half) c->h3h.ensure(e * RADIAL_H);
  size_t maxdin = 0;  // per-edge input gradients of the layers after the first
  for (size_t l = 1; l < c->layers.size(); ++l) maxdin = std::max(maxdin, (size_t)c->layers[l].dtp());
  if (!c->layers.empty() && c->layers[0].nonlin) {
    c->mh_dens.ensure(e);
    c->gwb.ensure(e * kGyMax);  // gw . b3, one partial per fused-VJP block column
    if (c->dims.separate_cutoff) c->cutv.ensure(e), c->gcut.ensure(e);
  }
  if (maxdin > 0) c->gxe.ensure(e * maxdin);
  c->geom.ensure(e);
  c->Y.ensure(e * 16);
  c->ef.ensure(e * c->dims.num_bessel);
  c->zbl_e.ensure(e);
  c->gY.ensure(e * 16 * kGyMax);
  c->gh3p.ensure(e * RADIAL_H * kGyMax);
  c->gef.ensure(e * c->dims.num_bessel);
  c->h3.ensure(e * RADIAL_H);
  c->gv.ensure(e * 3);
  if (!path.fused) {  // the separate passes' per-edge CG tables and dL/dw (the fused kernels keep both on chip)
    if (c->mts > 0) c->Mt.ensure(e * c->mts);
    if (half)
      c->gwh.ensure(e * maxw);
    else
      c->gw.ensure(e * maxw);
    c->gscale.ensure(e * NSLICE);
  }
  c->h3inv.ensure(e);
  for (size_t l = 0; l < c->layers.size(); ++l)
    if (own_h3(c, l)) c->layers[l].h3own.ensure(e * RADIAL_H), c->layers[l].h3invown.ensure(e);
  c->vir_part.ensure(9 * ((e + 255) / 256));

}

void ensure_edge_index(mace_ctx* c, int64_t E) {
  const size_t e = (size_t)std::max<int64_t>(E, 1);
  c->sender.ensure(e);
  c->receiver.ensure(e);
  c->shifts.ensure(3 * e);
  c->perm_s.ensure(e);
  c->pos_s.ensure(e);
  c->e_keys.ensure(e);
  c->e_perm.ensure(e);
  c->nl_iota.ensure(std::max<size_t>(e, (size_t)c->N + 1));
  c->e_tmp_i.ensure(e);
  c->e_tmp_j.ensure(e);
  c->e_tmp_s.ensure(3 * e);
}

int bits_for(int64_t maxval) {
  int b = 1;
  while (b < 31 && ((int64_t)1 << b) <= maxval) ++b;
  return b;
}

void cub_sort_pairs(mace_ctx* c, const int* kin, int* kout, const int* vin, int* vout, int64_t n, int64_t maxkey) {
  if (n <= 0) return;
  size_t bytes = 0;
  HIPCHK(hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, kin, kout, vin, vout, (int)n, 0, bits_for(maxkey),
                                            c->stream));
  c->cub_tmp.ensure(bytes);
  HIPCHK(hipcub::DeviceRadixSort::SortPairs(c->cub_tmp.p, bytes, kin, kout, vin, vout, (int)n, 0, bits_for(maxkey),
                                            c->stream));
}

void cub_exclusive_sum(mace_ctx* c, const int* in, int* out, int64_t n) {
  size_t bytes = 0;
  HIPCHK(hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, in, out, (int)n, c->stream));
  c->cub_tmp.ensure(bytes);
  HIPCHK(hipcub::DeviceScan::ExclusiveSum(c->cub_tmp.p, bytes, in, out, (int)n, c->stream));
}

// CSR rowptr from (unsorted) keys: counts + exclusive scan over n+1 entries
void build_rowptr(mace_ctx* c, const int* keys, int64_t E, int n, int* rowptr) {
  c->nl_counts.ensure((size_t)n + 1);
  HIPCHK(hipMemsetAsync(c->nl_counts.p, 0, ((size_t)n + 1) * sizeof(int), c->stream));
  launch_count_keys(c->stream, E, keys, c->nl_counts.p);
  cub_exclusive_sum(c, c->nl_counts.p, rowptr, (int64_t)n + 1);
}

__global__ void k_invert_perm(int64_t E, const int* __restrict__ perm, int* __restrict__ pos) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k < E) pos[perm[k]] = (int)k;
}

// sender-side CSR: perm_s = edge ids stably sorted by sender, pos_s its inverse
void build_sender_csr(mace_ctx* c) {
  const int64_t E = c->E;
  c->rowptr_s.ensure((size_t)c->N + 1);
  if (E > 0) {
    launch_fill_iota(c->stream, (int)E, c->nl_iota.p);
    cub_sort_pairs(c, c->sender.p, c->e_keys.p, c->nl_iota.p, c->perm_s.p, E, c->N);
    MACE_LAUNCH(k_invert_perm, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, c->stream, E, c->perm_s.p,
                       c->pos_s.p);
  }
  build_rowptr(c, c->sender.p, E, c->N, c->rowptr_s.p);
  c->srow_shared = false;
}

double plane_spacing(const double* cell, int k) {
  const double* a = cell + 3 * ((k + 1) % 3);
  const double* b = cell + 3 * ((k + 2) % 3);
  const double cx = a[1] * b[2] - a[2] * b[1], cy = a[2] * b[0] - a[0] * b[2], cz = a[0] * b[1] - a[1] * b[0];
  const double vol = std::fabs(cell[0] * (cell[4] * cell[8] - cell[5] * cell[7]) -
                               cell[1] * (cell[3] * cell[8] - cell[5] * cell[6]) +
                               cell[2] * (cell[3] * cell[7] - cell[4] * cell[6]));
  return vol / std::sqrt(cx * cx + cy * cy + cz * cz);
}

bool invert3(const double* m, double* inv) {
  const double det = m[0] * (m[4] * m[8] - m[5] * m[7]) - m[1] * (m[3] * m[8] - m[5] * m[6]) +
                     m[2] * (m[3] * m[7] - m[4] * m[6]);
  if (std::fabs(det) < 1e-300) return false;
  inv[0] = (m[4] * m[8] - m[5] * m[7]) / det;
  inv[1] = (m[2] * m[7] - m[1] * m[8]) / det;
  inv[2] = (m[1] * m[5] - m[2] * m[4]) / det;
  inv[3] = (m[5] * m[6] - m[3] * m[8]) / det;
  inv[4] = (m[0] * m[8] - m[2] * m[6]) / det;
  inv[5] = (m[2] * m[3] - m[0] * m[5]) / det;
  inv[6] = (m[3] * m[7] - m[4] * m[6]) / det;
  inv[7] = (m[1] * m[6] - m[0] * m[7]) / det;
  inv[8] = (m[0] * m[4] - m[1] * m[3]) / det;
  return true;
}

// Effective cell for the binning: periodic rows are the cell rows; each
// non-periodic row is replaced by a vector orthogonal to the periodic rows that
// spans the atoms' extent plus a margin (positions along it are never wrapped).
NLParams nl_params(const double* cell_in, const uint8_t* pbc, const double* pos, int N, double cutoff) {
  NLParams p{};
  double cell[9];
  std::memcpy(cell, cell_in, sizeof cell);
  int nper = 0;
  for (int k = 0; k < 3; ++k) nper += pbc[k] ? 1 : 0;
  double origin[3] = {0, 0, 0};
  if (nper < 3) {
    // orthonormal directions for the non-periodic axes
    double dirs[3][3];
    std::vector<int> per, non;
    for (int k = 0; k < 3; ++k) (pbc[k] ? per : non).push_back(k);
    if (per.size() == 2) {
      const double* a = cell + 3 * per[0];
      const double* b = cell + 3 * per[1];
      double n[3] = {a[1] * b[2] - a[2] * b[1], a[2] * b[0] - a[0] * b[2], a[0] * b[1] - a[1] * b[0]};
      const double nn = std::sqrt(n[0] * n[0] + n[1] * n[1] + n[2] * n[2]);
      if (nn < 1e-12) fail(MACE_ERR_INVALID, "degenerate periodic cell vectors");
      for (int q = 0; q < 3; ++q) dirs[non[0]][q] = n[q] / nn;
    } else if (per.size() == 1) {
      const double* a = cell + 3 * per[0];
      const double na = std::sqrt(a[0] * a[0] + a[1] * a[1] + a[2] * a[2]);
      if (na < 1e-12) fail(MACE_ERR_INVALID, "degenerate periodic cell vector");
      double e1[3] = {a[0] / na, a[1] / na, a[2] / na};
      double t[3] = {1, 0, 0};
      if (std::fabs(e1[0]) > 0.9) t[0] = 0, t[1] = 1;
      double u[3] = {e1[1] * t[2] - e1[2] * t[1], e1[2] * t[0] - e1[0] * t[2], e1[0] * t[1] - e1[1] * t[0]};
      const double nu = std::sqrt(u[0] * u[0] + u[1] * u[1] + u[2] * u[2]);
      for (int q = 0; q < 3; ++q) u[q] /= nu;
      double v[3] = {e1[1] * u[2] - e1[2] * u[1], e1[2] * u[0] - e1[0] * u[2], e1[0] * u[1] - e1[1] * u[0]};
      for (int q = 0; q < 3; ++q) dirs[non[0]][q] = u[q], dirs[non[1]][q] = v[q];
    } else {
      for (int k = 0; k < 3; ++k)
        for (int q = 0; q < 3; ++q) dirs[k][q] = (k == q) ? 1.0 : 0.0;
    }
    for (int k : non) {
      double lo = 1e300, hi = -1e300;
      for (int i = 0; i < N; ++i) {
        const double s = pos[3 * i] * dirs[k][0] + pos[3 * i + 1] * dirs[k][1] + pos[3 * i + 2] * dirs[k][2];
        lo = std::min(lo, s);
        hi = std::max(hi, s);
      }
      if (N == 0) lo = hi = 0;
      const double len = (hi - lo) + 2.0 * cutoff + 1.0;
      for (int q = 0; q < 3; ++q) {
        cell[3 * k + q] = dirs[k][q] * len;
        origin[q] += dirs[k][q] * (lo - cutoff - 0.5);
      }
    }
  }
  std::memcpy(p.cell, cell, sizeof cell);
  if (!invert3(cell, p.inv)) fail(MACE_ERR_INVALID, "cell is singular for a periodic direction");
  for (int k = 0; k < 3; ++k) {
    p.origin[k] = origin[k];
    p.periodic[k] = pbc[k] ? 1 : 0;
    // bins half a cutoff wide: a receiver's candidates are the atoms of (2r + 1)^3 = 125 bins
    // (r = 2) instead of 27 cutoff-wide bins, i.e. about 0.58 of the volume
    const double d = plane_spacing(cell, k);
    int nbin = (int)std::floor(2.0 * d / cutoff);
    nbin = std::max(1, std::min(nbin, 256));
    p.nbin[k] = nbin;
    p.range[k] = (int)std::ceil(cutoff * nbin / d + 1e-9);
    if (!p.periodic[k]) p.range[k] = std::min(p.range[k], nbin);
  }
  // the fill pass packs a cell index and the cell count into 16 bits each
  if ((int64_t)(2 * p.range[0] + 1) * (2 * p.range[1] + 1) * (2 * p.range[2] + 1) >= 32768)
    fail(MACE_ERR_INVALID, "cell too small for the cutoff (more than 32767 neighbour cells per atom)");
  p.cutoff2 = cutoff * cutoff;
  return p;
}

// One cell list per structure of the batch (each in its own cell, atoms [gptr[g], gptr[g+1])),
// bins numbered consecutively across structures so that one sort and one scan serve all.
void build_nl(mace_ctx* c, const double* pos_host) {
  invalidate_graphs(c);
  const int N = c->N;
  const int G = c->G;
  const double cutoff = c->dims.r_max + std::max(c->skin, 0.0);
  std::vector<NLParams> ps(G);
  std::vector<int> bin_off(G + 1, 0);
  for (int g = 0; g < G; ++g) {
    const int i0 = c->gptr_h[g], n = c->gptr_h[g + 1] - i0;
    ps[g] = nl_params(c->gcell_h.data() + 9 * g, c->gpbc_h.data() + 3 * g, pos_host + 3 * (size_t)i0, n, cutoff);
    const int64_t nb = (int64_t)ps[g].nbin[0] * ps[g].nbin[1] * ps[g].nbin[2];
    if (bin_off[g] + nb > INT32_MAX / 2) fail(MACE_ERR_INVALID, "too many neighbour-list bins");
    bin_off[g + 1] = bin_off[g] + (int)nb;
  }
  const int nbins = bin_off[G];
  // per receiver and neighbour cell, the edges of its row before that cell (count pass; the
  // fill pass places each reverse edge with it): row stride = the largest cell count + 1
  int cstride = 1;
  for (int g = 0; g < G; ++g)
    cstride = std::max(cstride, (2 * ps[g].range[0] + 1) * (2 * ps[g].range[1] + 1) * (2 * ps[g].range[2] + 1) + 1);
  c->nl_wpos.ensure(3 * (size_t)N);
  c->nl_pos_d.ensure(3 * (size_t)N);
  c->nl_img.ensure(3 * (size_t)N);
  c->nl_bin.ensure(N);
  c->nl_bin_sorted.ensure(N);
  c->nl_atoms.ensure(N);
  c->nl_iota.ensure((size_t)N + 1);
  c->nl_bin_start.ensure((size_t)nbins + 1);
  c->rowptr.ensure((size_t)N + 1);
  c->nl_wpos_s.ensure(3 * (size_t)N);
  c->nl_img_s.ensure(3 * (size_t)N);
  if (G == 1 && N > 0 && N <= kNlSmall) {
    // one structure of up to kNlSmall atoms: binning, sort and bin starts in one block
    launch_nl_prep_small(c->stream, N, c->pos.p, ps[0], nbins, bits_for(nbins), c->nl_wpos.p, c->nl_img.p,
                         c->nl_bin.p, c->nl_pos_d.p, c->nl_bin_sorted.p, c->nl_atoms.p, c->nl_bin_start.p,
                         c->nl_wpos_s.p, c->nl_img_s.p);
  } else {
    for (int g = 0; g < G; ++g)
      launch_nl_bin(c->stream, c->gptr_h[g], c->gptr_h[g + 1] - c->gptr_h[g], c->pos.p, ps[g], bin_off[g],
                    c->nl_wpos.p, c->nl_img.p, c->nl_bin.p, c->nl_iota.p, c->nl_pos_d.p);
    // atoms sorted by bin (stable: within a bin by index), then each bin's first position
    cub_sort_pairs(c, c->nl_bin.p, c->nl_bin_sorted.p, c->nl_iota.p, c->nl_atoms.p, N, nbins);
    launch_key_starts(c->stream, N, c->nl_bin_sorted.p, nbins, c->nl_bin_start.p, c->nl_atoms.p, c->nl_wpos.p,
                      c->nl_img.p, c->nl_wpos_s.p, c->nl_img_s.p);
  }
  c->nl_counts.ensure((size_t)N + 1);
  c->nl_missing.ensure(1);
  c->nl_cpre.ensure(std::max<size_t>((size_t)N * cstride, 1));
  const int hcap = c->nl_hcap;
  c->nl_hits.ensure(std::max<size_t>(2 * (size_t)N * hcap, 2));
  if (N == 0) {  // no count pass to clear the scan's last slot and the reverse-edge counter
    HIPCHK(hipMemsetAsync(c->nl_counts.p, 0, sizeof(int), c->stream));
    HIPCHK(hipMemsetAsync(c->nl_missing.p, 0, sizeof(int), c->stream));
  }
  for (int g = 0; g < G; ++g)
    launch_nl_count(c->stream, c->gptr_h[g], c->gptr_h[g + 1] - c->gptr_h[g], ps[g], bin_off[g], c->nl_wpos.p,
                    c->nl_wpos_s.p, c->nl_bin.p, c->nl_bin_start.p, c->nl_atoms.p, cstride, c->nl_cpre.p,
                    c->nl_hits.p, hcap, c->nl_counts.p, c->nl_counts.p + N, c->nl_missing.p);
  if (N + 1 <= 2 * kNlSmall)
    launch_exclusive_sum_small(c->stream, N + 1, c->nl_counts.p, c->rowptr.p);
  else
    cub_exclusive_sum(c, c->nl_counts.p, c->rowptr.p, (int64_t)N + 1);
  // the edge count sizes the per-edge arrays and the launches: read back (pinned memory: a copy
  // into pageable memory costs more than this whole wait)
  if (!c->e_pinned) HIPCHK(hipHostMalloc((void**)&c->e_pinned, sizeof(int), hipHostMallocDefault));
  // The copy lands after the scan (stream order): poll the pinned word, which returns sooner
  // than a blocking synchronisation (the GPU idles until the fill is launched); synchronise
  // instead if it has not landed within 0.2 s
  volatile int* ep = c->e_pinned;
  *ep = -1;
  HIPCHK(hipMemcpyAsync(c->e_pinned, c->rowptr.p + N, sizeof(int), hipMemcpyDeviceToHost, c->stream));
  const auto t0 = std::chrono::steady_clock::now();
  while (*ep < 0)
    if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(200)) {
      HIPCHK(hipStreamSynchronize(c->stream));
      break;
    }
  c->E = *ep;
  ensure_edge_index(c, c->E);
  // the fill pass also writes the sender-side CSR of the (symmetric) list without a sort: its
  // row pointers are rowptr's (srow), perm_s = pos_s = the reverse of each edge; the count of
  // edges without a reverse is read at the next synchronisation (check_nl_missing)
  for (int g = 0; g < G; ++g)
    launch_nl_fill(c->stream, c->gptr_h[g], c->gptr_h[g + 1] - c->gptr_h[g], ps[g], bin_off[g], c->nl_wpos.p,
                   c->nl_wpos_s.p, c->nl_img.p, c->nl_img_s.p, c->nl_bin.p, c->nl_bin_start.p, c->nl_atoms.p,
                   c->rowptr.p, cstride, c->nl_cpre.p, c->nl_hits.p, hcap, c->sender.p, c->receiver.p,
                   c->shifts.p, c->perm_s.p, c->pos_s.p, c->nl_missing.p);
  if (N > 0) c->nl_hcap = (int)std::min<int64_t>(1024, std::max<int64_t>(128, (3 * c->E / N) / 2 + 1));
  c->srow_shared = true;
  c->nl_check_pending = true;
  ensure_edge_buffers(c, c->E);
  // positions at this build, for the host-side skin check of mace_step (unknown when the build
  // took device positions of a fully periodic system: the next mace_step then rebuilds)
  if (pos_host)
    c->nl_pos.assign(pos_host, pos_host + 3 * (size_t)N);
  else
    c->nl_pos.clear();
  c->nl_valid = true;
}

// Reverse-edge count of the last list build into pinned memory (queued before a
// synchronisation, when a build has not been checked yet)
void queue_nl_missing(mace_ctx* c) {
  if (!c->nl_check_pending) return;
  if (!c->nl_missing_h) HIPCHK(hipHostMalloc((void**)&c->nl_missing_h, sizeof(int), hipHostMallocDefault));
  HIPCHK(hipMemcpyAsync(c->nl_missing_h, c->nl_missing.p, sizeof(int), hipMemcpyDeviceToHost, c->stream));
}

// after that synchronisation: a list build whose edges lacked reverses is an internal error
void check_nl_missing(mace_ctx* c) {
  if (!c->nl_check_pending) return;
  c->nl_check_pending = false;
  if (*c->nl_missing_h > 0) {
    const int m = *c->nl_missing_h;
    c->nl_valid = false;
    fail(MACE_ERR_STATE, "neighbour list not symmetric: %d edges without a reverse", m);
  }
}

// The skin criterion of mace_step (calculators.py:266-283) for device-resident positions: the
// largest displacement since the last list build, reduced on the device and read back.
bool skin_exceeded_on_device(mace_ctx* c, const double* d_positions) {
  const int N = c->N;
  if (c->skin <= 0 || c->nl_pos_d.n < 3 * (size_t)N) return true;
  if (N == 0) return false;
  c->skin_flag.ensure(1);
  if (!c->skin_pinned) HIPCHK(hipHostMalloc((void**)&c->skin_pinned, sizeof(int), hipHostMallocDefault));
  HIPCHK(hipMemsetAsync(c->skin_flag.p, 0, sizeof(int), c->stream));
  launch_max_disp(c->stream, N, d_positions, c->nl_pos_d.p, 0.25 * c->skin * c->skin, c->skin_flag.p);
  HIPCHK(hipMemcpyAsync(c->skin_pinned, c->skin_flag.p, sizeof(int), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(hipStreamSynchronize(c->stream));
  return *c->skin_pinned != 0;
}

// row pointers of the sender-side CSR
const int* srow(const mace_ctx* c) { return c->srow_shared ? c->rowptr.p : c->rowptr_s.p; }

__global__ void k_gather_edges(int64_t E, const int* perm, const int* si, const int* ri, const int* ss, int* so,
                               int* ro, int* sso) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int q = perm[e];
  so[e] = si[q];
  ro[e] = ri[q];
  sso[3 * e] = ss[3 * q];
  sso[3 * e + 1] = ss[3 * q + 1];
  sso[3 * e + 2] = ss[3 * q + 2];
}

// ---------------------------------------------------------------------------
// the step
// ---------------------------------------------------------------------------
GemmProb gprob(int N, int d, int K1, int Cout, const float* X1, int ldx1, int base1, int stride1, const float* WT1,
                float* Y, int ldy, int obase, int ostride) {
  GemmProb P{};
  P.d = d;
  P.rows = N * d;
  P.K1 = K1;
  P.K2 = 0;
  P.Cout = Cout;
  P.X1 = X1;
  P.ldx1 = ldx1;
  P.in_base1 = base1;
  P.in_stride1 = stride1;
  P.WT1 = WT1;
  P.Y = Y;
  P.ldy = ldy;
  P.out_base = obase;
  P.out_stride = ostride;
  return P;
}

// grouped products: on fp16 matrix cores with split operands when enabled and every weight
// matrix has its split copy, else on fp32 matrix cores (either way rounded by g.round_half)
void run_gemm(mace_ctx* c, hipStream_t st, GemmGroup& g) {
  g.split = 0;
  if (c->split_products) {
    bool ok = true;
    for (int q = 0; q < g.n && ok; ++q) {
      GemmProb& P = g.p[q];
      auto a = c->wsplit.find(P.WT1);
      auto b = P.K2 > 0 ? c->wsplit.find(P.WT2) : a;
      ok = a != c->wsplit.end() && b != c->wsplit.end() && P.Cout % 64 == 0 && P.K1 % 32 == 0 && P.K2 % 32 == 0;
      if (!ok) break;
      P.WX1 = a->second.x.p;
      P.winv1 = a->second.winv;
      P.WX2 = b->second.x.p;
      P.winv2 = b->second.winv;
    }
    g.split = ok ? 1 : 0;
  }
  launch_gemm_group(st, g);
}

void slot_range(const Layer& L, int lo, int* first, int* cnt) {
  const int* l3 = tp_l3(L.tl());
  *first = -1;
  *cnt = 0;
  for (int q = 0; q < n_tp_slots(L.tl()); ++q)
    if (l3[q] == lo) {
      if (*first < 0) *first = q;
      ++*cnt;
    }
}

FrontParams front_params(mace_ctx* c) {
  FrontParams p{};
  std::memcpy(p.cell, c->cell, sizeof p.cell);
  p.r_max = (float)c->dims.r_max;
  p.bessel_pref = (float)std::sqrt(2.0 / c->dims.r_max);
  p.nbessel = c->dims.num_bessel;
  p.pcut = c->dims.num_poly_cutoff;
  p.has_zbl = c->dims.has_zbl;
  p.zbl_p = c->dims.zbl_p;
  p.zbl_a_exp = (float)c->dims.zbl_a_exp;
  p.zbl_a_pref = (float)c->dims.zbl_a_prefactor;
  p.zbl_scale = (float)c->dims.zbl_scale;
  p.feature_half = c->dims.feature_half;
  p.agnesi = c->dims.agnesi != 0;
  p.ag_q = (float)c->dims.agnesi_q;
  p.ag_p = (float)c->dims.agnesi_p;
  p.ag_a = (float)c->dims.agnesi_a;
  p.apply_cutoff = !c->dims.separate_cutoff;
  return p;
}

// A list of grouped products in launches of at most GEMM_MAX problems each.
void run_gemm_list(mace_ctx* c, hipStream_t st, const std::vector<GemmProb>& probs, int round_half) {
  for (size_t q0 = 0; q0 < probs.size(); q0 += GEMM_MAX) {
    GemmGroup g{};
    g.round_half = round_half;
    for (size_t q = q0; q < probs.size() && q < q0 + GEMM_MAX; ++q) g.p[g.n++] = probs[q];
    run_gemm(c, st, g);
  }
}

// Products with per-species weights (one-hot node attributes: the skip connection's and the
// message skip's FCTPs, blocks.py:171-176, 225-230): P once per species present, over that
// species' atoms (row map into the species-sorted atom order), operand `which` (1 or 2) taking
// element z's [C][C] slice of W.  One element: P with W itself, over every atom.
void add_species_probs(mace_ctx* c, const GemmProb& P, int which, const float* W, std::vector<GemmProb>& out) {
  if (c->dims.num_elements == 1) {
    GemmProb Q = P;
    (which == 1 ? Q.WT1 : Q.WT2) = W;
    out.push_back(Q);
    return;
  }
  const size_t CC = (size_t)NC * NC;
  for (int z = 0; z < c->dims.num_elements; ++z) {
    if (c->sp_cnt[z] == 0) continue;
    GemmProb Q = P;
    Q.rows = c->sp_cnt[z] * P.d;
    Q.rowmap = c->sp_perm.p + c->sp_off[z];
    (which == 1 ? Q.WT1 : Q.WT2) = W + z * CC;
    out.push_back(Q);
  }
}

// operand 2 of P = the skip connection's input block b (x W_skip[species])
void set_skip_operand(GemmProb& P, const float* X, int ldx, int b) {
  P.K2 = NC;
  P.X2 = X;
  P.ldx2 = ldx;
  P.in_base2 = NC * b * b;
  P.in_stride2 = 0;
}

// Message skip FCTP of a non-residual block (blocks.py:171-176): per interaction block lo,
// out[n][lo] = in[n][lo] W_lo[species(n)]; WT = the transposed per-element weights [n_el][C][C]
// (pw and CG folded): mskipT for the forward, mskip for its VJP.
void run_msg_skip(mace_ctx* c, Layer& L, const float* in, float* out, const DBuf<float>* WT, int half) {
  std::vector<GemmProb> probs;
  for (int lo = 0; lo < 4; ++lo)
    add_species_probs(c, gprob(c->N, 2 * lo + 1, NC, NC, in, L.dint, NC * lo * lo, 0, nullptr, out, L.dint,
                               NC * lo * lo, 0),
                      1, WT[lo].p, probs);
  run_gemm_list(c, c->stream, probs, half);
}

// Discard captured step graphs (launch arguments or buffers changed).
void invalidate_graphs(mace_ctx* c) {
  for (auto* g : {&c->g_fwd, &c->g_bwd}) {
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    *g = mace_ctx::StepGraph{};
  }
}

// ... and the species features (model, species or node buffers changed; an edge-list
// change leaves them valid)
void invalidate_node_state(mace_ctx* c) {
  invalidate_graphs(c);
  c->embed_valid = false;
}

// First-layer node features h0 and the first linear_up output: functions of the species
// only (the embedding is stop_gradient'ed, model.py:382), so they are written once per
// system / model / buffer set, before the step, not by every step.
// Product paths a step can take for the loaded model, checked before anything is launched or
// captured: non-linear interaction blocks under a half-precision policy run on the fused
// split-product path only (the comparison paths keep float32 buffers)
void check_step_path(const mace_ctx* c) {
  if (c->dims.nonlinear && c->dims.feature_half && !step_path(c).fused)
    fail(MACE_ERR_UNSUPPORTED, "non-linear interaction blocks under a half-precision policy run on the fused "
                               "split-product path only (split products and the fused TP on)");
  // the comparison paths' separate radial output kernels are laid out for two channel slices
  if (NC != 128 && !step_path(c).fused)
    fail(MACE_ERR_UNSUPPORTED, "the %d-channel engine runs the fused split-product path only", NC);
}

void ensure_embed(mace_ctx* c) {
  if (c->embed_valid) return;
  Site s(c, "embed");
  launch_embed(c->stream, c->N, c->species.p, c->embed.p, c->layers[0].din, c->h[0].p, c->dims.feature_half,
               c->up0_tab.p, c->layers[0].h_up.p);
  c->embed_valid = true;
}

bool graphs_active(const mace_ctx* c) { return c->use_graphs && !c->profiling; }

// Capture body() (a sequence of launches on c->stream) into g for the binding (a, b, flag),
// without running it: c->stream is the capture stream meanwhile, so this can happen while the
// engine stream still executes earlier work.
template <class F>
void capture_graph(mace_ctx* c, mace_ctx::StepGraph& g, const void* a, const void* b, int flag, F&& body) {
  if (g.exec) (void)hipGraphExecDestroy(g.exec);
  g = mace_ctx::StepGraph{};
  struct Swap {  // the engine stream is back in place on every exit
    mace_ctx* c;
    hipStream_t run;
    ~Swap() { c->stream = run; }
  } swap{c, c->stream};
  c->stream = c->cap_stream;
  hipGraph_t graph = nullptr;
  HIPCHK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  try {
    body();
  } catch (...) {
    (void)hipStreamEndCapture(c->stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    throw;
  }
  HIPCHK(hipStreamEndCapture(c->stream, &graph));
  const hipError_t e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) {
    g.exec = nullptr;
    fail(MACE_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  }
  g.a = a;
  g.b = b;
  g.flag = flag;
}

// Run body() through the graph captured for the binding (a, b, flag), capturing it first if
// needed; eager when graphs are off or per-launch profiling is on.
template <class F>
void run_captured(mace_ctx* c, mace_ctx::StepGraph& g, const void* a, const void* b, int flag, F&& body) {
  if (!graphs_active(c)) {
    body();
    return;
  }
  if (!g.exec || g.a != a || g.b != b || g.flag != flag) capture_graph(c, g, a, b, flag, body);
  HIPCHK(hipGraphLaunch(g.exec, c->stream));
}

// the species index array the symmetric contraction reads: all zeros for the element-agnostic
// product (blocks.py:510-533)
const int* sc_species(mace_ctx* c) { return c->dims.agnostic_product ? c->zero_species.p : c->species.p; }

// column offset of output degree lo in the gate-input layout [scalars | 3 gate blocks | 1o | 2e | 3o]
inline int gate_in_base(int lo) { return lo == 0 ? 0 : 4 * NC + NC * (lo * lo - 1); }

// mh-1 non-linear interaction block and its product, h -> hn (blocks.py:735-807, 493-537)
void forward_nonlin(mace_ctx* c, int l, const float* h, float* hn) {
  hipStream_t st = c->stream;
  Layer& L = c->layers[l];
  const int N = c->N;
  const int64_t E = c->E;
  const int nb = c->dims.num_bessel;
  const float* cut = c->dims.separate_cutoff ? c->cutv.p : nullptr;
  const bool split = c->split_products;  // h3 W3 on fp16 matrix cores (split operands)
  const bool fused = step_path(c).fused;   // ... inside the TP kernels
  // rounding mode of the stored activations (float16 / bfloat16 feature policies): the default
  // fused path carries it; the comparison paths (separate radial output pass, fp32 matrix cores)
  // keep their float32 buffers and run under the float32 policy only
  const int half = c->dims.feature_half;  // check_step_path: half implies split && fused here
  {  // LayerNorm radial MLP (last hidden activation) and the edge densities
    Site s(c, lname("mlp_ln", l));
    launch_rmlp_ln_fwd(st, E, nb, c->ef.p, cut, c->sender.p, c->receiver.p, c->species.p, L.mlp_tiles.p,
                       split ? L.mlp_tiles_x.p : nullptr, L.dmlp_tiles.p, L.lnp(), c->h3.p,
                       split ? c->h3inv.p : nullptr, c->mh_dens.p, half);
  }
  if (!fused) {  // w = (h3 W3 + b3) cut
    Site s(c, lname("mlp_out", l));
    if (split)
      launch_mlp_out_x(st, E, L.wn, c->h3.p, c->h3inv.p, L.mlpT3x.p, L.w3inv, L.w.p, L.b3.p, cut);
    else
      launch_mlp_out(st, E, L.wn, c->h3.p, L.mlpT[3].p, L.w.p, 0, L.b3.p, cut);
  }
  if (l > 0) {  // the first layer's comes from the species table (launch_embed)
    Site s(c, lname("linear_up", l));
    if (L.ledge > L.lin) launch_fill_zero(st, L.h_up.p, (int64_t)N * L.dedge);  // edge blocks without input
    GemmGroup g{};
    for (int b = 0; b < std::min(L.lin, L.ledge); ++b)
      g.p[g.n++] = gprob(N, 2 * b + 1, NC, NC, h, L.din, NC * b * b, 0, L.upT[b].p, L.h_up.p, L.dedge, NC * b * b, 0);
    g.round_half = half;
    run_gemm(c, st, g);
  }
  {
    Site s(c, lname("tp_fwd", l));
    if (fused)  // w = (h3 W3 + b3) cut formed per edge tile, and stored for the VJP
      launch_tpx_fwd(st, L.ledge, N, E, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, c->h3.p, c->h3inv.p,
                     L.mlpT3x.p, L.wn, L.w3inv, L.h_up.p, c->M.p, L.w.p, half, L.b3.p, cut);
    else
      launch_tp_fwd(st, L.ledge, N, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, L.w.p, L.h_up.p, c->M.p, 0);
  }
  {  // rinv = 1 / (beta rho + alpha)
    Site s(c, lname("density", l));
    launch_mh1_rho(st, N, c->rowptr.p, c->mh_dens.p, L.alpha, L.beta, L.rinv.p);
  }
  {  // Q = linear_1(M) / (beta rho + alpha), and in the same launch R = linear_res(up)
    Site s(c, lname("linear_msg", l));
    const int* ao = tp_accoff(L.ledge);
    GemmGroup g{};
    for (int lo = 0; lo < L.ledge; ++lo) {
      const int d = 2 * lo + 1;
      g.p[g.n++] = gprob(N, d, NC, lo == 0 ? 4 * NC : NC, L.h_up.p, L.dedge, NC * lo * lo, 0, L.resT[lo].p, L.R.p,
                         L.nres, gate_in_base(lo), NC * d);
    }
    for (int lo = 0; lo < 4; ++lo) {
      int first, cnt;
      slot_range(L, lo, &first, &cnt);
      const int d = 2 * lo + 1;
      g.p[g.n++] = gprob(N, d, cnt * NC, lo == 0 ? 4 * NC : NC, c->M.p, L.dmid, NC * ao[first], NC * d,
                         L.linT[lo].p, L.Q.p, kGateInDim, gate_in_base(lo), NC * d);
      g.p[g.n - 1].rowscale = L.rinv.p;
    }
    g.round_half = half;
    run_gemm(c, st, g);
  }
  {
    Site s(c, lname("gate", l));
    launch_mh1_gate(st, N, L.Q.p, L.R.p, L.nres, L.Gt.p, half);
  }
  {
    Site s(c, lname("linear_2", l));
    GemmGroup g{};
    for (int lo = 0; lo < 4; ++lo)
      g.p[g.n++] = gprob(N, 2 * lo + 1, NC, NC, L.Gt.p, L.dint, NC * lo * lo, 0, L.lin2T[lo].p, L.A.p, L.dint,
                         NC * lo * lo, 0);
    g.round_half = half;
    run_gemm(c, st, g);
  }
  const float* scw[3] = {L.sc[0].p, L.sc[1].p, L.sc[2].p};
  {
    Site s(c, lname("sc_fwd", l));
    launch_sc_fwd(st, N, L.lhid, L.corr, L.A.p, L.dint, sc_species(c), scw, c->B.p, L.dhid, half);
  }
  {  // h' = PLin(B) + Skip(h) (plain linear skip)
    Site s(c, lname("linear_prod", l));
    GemmGroup g{};
    for (int b = 0; b < L.lhid; ++b) {
      GemmProb P = gprob(N, 2 * b + 1, NC, NC, c->B.p, L.dhid, NC * b * b, 0, L.plinT[b].p, hn, L.dhid, NC * b * b, 0);
      if (b < L.nskip) {
        P.K2 = NC;
        P.X2 = h;
        P.ldx2 = L.din;
        P.in_base2 = NC * b * b;
        P.in_stride2 = 0;
        P.WT2 = L.skipT[b].p;
      }
      g.p[g.n++] = P;
    }
    g.round_half = half;
    run_gemm(c, st, g);
  }
}

// VJP of forward_nonlin: from gh = dE/dh_{l+1}; for l > 0 writes gh_next = dE/dh_l (with the
// previous layer's linear readout as the 0e bias)
void backward_nonlin(mace_ctx* c, int l, const float* gh, float* gh_next, int first_edge_grad, int gyp) {
  hipStream_t st = c->stream;
  Layer& Ly = c->layers[l];
  const int N = c->N;
  const int64_t E = c->E;
  const int nb = c->dims.num_bessel;
  const float* cut = c->dims.separate_cutoff ? c->cutv.p : nullptr;
  {  // gB = PLin^T gh
    Site s(c, lname("linear_prod_bwd", l));
    GemmGroup g{};
    for (int b = 0; b < Ly.lhid; ++b)
      g.p[g.n++] = gprob(N, 2 * b + 1, NC, NC, gh, Ly.dhid, NC * b * b, 0, Ly.plin[b].p, c->gB.p, Ly.dhid, NC * b * b, 0);
    run_gemm(c, st, g);
  }
  const float* scw[3] = {Ly.sc[0].p, Ly.sc[1].p, Ly.sc[2].p};
  {
    Site s(c, lname("sc_bwd", l));
    launch_sc_bwd(st, N, Ly.lhid, Ly.corr, Ly.A.p, Ly.dint, sc_species(c), scw, c->gB.p, Ly.dhid, c->gA.p);
  }
  {  // dL/dgate-output = Lin2^T gA
    Site s(c, lname("linear_2_bwd", l));
    GemmGroup g{};
    for (int lo = 0; lo < 4; ++lo)
      g.p[g.n++] = gprob(N, 2 * lo + 1, NC, NC, c->gA.p, Ly.dint, NC * lo * lo, 0, Ly.lin2[lo].p, c->gA2.p, Ly.dint,
                         NC * lo * lo, 0);
    run_gemm(c, st, g);
  }
  {  // gP = dL/d(Q + R) and dL/drho
    Site s(c, lname("gate_bwd", l));
    launch_mh1_gate_bwd(st, N, Ly.Q.p, Ly.R.p, Ly.nres, c->gA2.p, c->gP.p, Ly.rinv.p, Ly.beta, c->grho.p);
  }
  {  // gM = Lin1^T gP / (beta rho + alpha), and for l > 0 in the same launch gup = Res^T gP (the
     // gather of the TP's dL/dx rows adds to it)
    Site s(c, lname("linear_msg_bwd", l));
    const int* ao = tp_accoff(Ly.ledge);
    GemmGroup g{};
    for (int lo = 0; l > 0 && lo < Ly.ledge; ++lo) {
      const int d = 2 * lo + 1;
      g.p[g.n++] = gprob(N, d, lo == 0 ? 4 * NC : NC, NC, c->gP.p, kGateInDim, gate_in_base(lo), NC * d,
                         Ly.res_[lo].p, c->gup.p, Ly.dedge, NC * lo * lo, 0);
    }
    for (int lo = 0; lo < 4; ++lo) {
      int first, cnt;
      slot_range(Ly, lo, &first, &cnt);
      const int d = 2 * lo + 1;
      g.p[g.n++] = gprob(N, d, lo == 0 ? 4 * NC : NC, cnt * NC, c->gP.p, kGateInDim, gate_in_base(lo), NC * d,
                         Ly.lin_[lo].p, c->gM.p, Ly.dmid, NC * ao[first], NC * d);
      g.p[g.n - 1].rowscale = Ly.rinv.p;
    }
    run_gemm(c, st, g);
  }
  const bool fused = step_path(c).fused;
  if (fused) {  // dL/dw stays on chip: G = gw W3^T and gw . b3 as per-block-column partials
    Site s(c, lname("tp_bwd", l));
    int acc_gy = first_edge_grad;
    if (!acc_gy && tpx_parts(Ly.ledge) < gyp) {  // partials this layer does not write start at zero
      launch_fill_zero(st, c->gY.p, E * 16 * gyp);
      acc_gy = 1;
    }
    launch_tpx_bwd(st, Ly.ledge, N, E, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, Ly.w.p, Ly.mlp3x.p, Ly.wn,
                   Ly.w3inv, Ly.h_up.p, c->gM.p, c->pos_s.p, l > 0 ? c->gxe.p : nullptr, c->gY.p, gyp, acc_gy,
                   c->gh3p.p, c->dims.feature_half, Ly.b3.p, c->gwb.p);  // w as the forward stored it
  } else {
    Site s(c, lname("tp_bwd", l));
    launch_tp_bwd_recv(st, Ly.ledge, N, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, Ly.w.p, Ly.h_up.p,
                       c->gM.p, c->gw.p, c->gscale.p, c->gY.p, first_edge_grad, c->pos_s.p,
                       l > 0 ? c->gxe.p : nullptr, 0);
  }
  if (l > 0) {
    Site s(c, lname("tp_gather", l));
    launch_tp_gather_gx(st, Ly.ledge, N, srow(c), c->gxe.p, c->gup.p, fused && c->dims.feature_half == RND_F16,
                        1);
  }
  if (!fused) {  // G = gw W3^T (into h3), gwb = gw . b3
    Site s(c, lname("mlp_gh3", l));
    if (c->split_products)
      launch_mlp_gh3_x(st, E, Ly.wn, c->gw.p, Ly.mlp3x.p, Ly.w3inv, c->h3.p, Ly.b3.p, c->gwb.p);
    else
      launch_mlp_gh3(st, E, Ly.wn, c->gw.p, Ly.mlp[3].p, c->h3.p, Ly.b3.p, c->gwb.p);
  }
  {
    Site s(c, lname("mlp_ln_bwd", l));
    const size_t fb = mlp_tile_fwd_bytes(), fbx = mlp_tile_x_fwd_bytes();
    const bool sx = c->split_products;  // the hidden layers on split-fp16 products, as the forward
    launch_rmlp_ln_bwd(st, E, nb, c->ef.p, cut, c->sender.p, c->receiver.p, c->species.p, Ly.mlp_tiles.p,
                       Ly.mlp_tiles.p + fb, sx ? Ly.mlp_tiles_x.p : nullptr, sx ? Ly.mlp_tiles_x.p + fbx : nullptr,
                       Ly.dmlp_tiles.p, Ly.dmlp_tiles.p + fb, Ly.lnp(),
                       fused ? c->gh3p.p : c->h3.p, c->gwb.p, fused ? tpx_parts(Ly.ledge) : 1, c->grho.p, c->gef.p,
                       cut ? c->gcut.p : nullptr, first_edge_grad);
  }
  if (l == 0) return;
  {  // dE/dh_l = Up^T gup + Skip^T gh + readout_{l-1}' (bias on the 0e block)
    Site s(c, lname("linear_up_bwd", l));
    if (Ly.lin > std::max(Ly.ledge, Ly.nskip)) launch_fill_zero(st, gh_next, (int64_t)N * Ly.din);
    GemmGroup g{};
    for (int b = 0; b < Ly.lin; ++b) {
      GemmProb P{};
      if (b < Ly.ledge) {
        P = gprob(N, 2 * b + 1, NC, NC, c->gup.p, Ly.dedge, NC * b * b, 0, Ly.up[b].p, gh_next, Ly.din, NC * b * b, 0);
        if (b < Ly.nskip) {
          P.K2 = NC;
          P.X2 = gh;
          P.ldx2 = Ly.dhid;
          P.in_base2 = NC * b * b;
          P.in_stride2 = 0;
          P.WT2 = Ly.skip[b].p;
        }
      } else if (b < Ly.nskip) {
        P = gprob(N, 2 * b + 1, NC, NC, gh, Ly.dhid, NC * b * b, 0, Ly.skip[b].p, gh_next, Ly.din, NC * b * b, 0);
      } else {
        continue;
      }
      if (b == 0) P.bias = c->layers[l - 1].ro.p;
      g.p[g.n++] = P;
    }
    run_gemm(c, st, g);
  }
}

void forward(mace_ctx* c, const double* pos, double* out, double* e_part) {
  if (c->profiling) c->launch_log.clear();  // a step starts here
  hipStream_t st = c->stream;
  const int N = c->N;
  const int64_t E = c->E;
  const int nb = c->dims.num_bessel;
  const int half = c->dims.feature_half;  // rounding mode of the stored activations (RND_*)
  const StepPath path = step_path(c);
  const bool h16 = path.h16, split = path.split, fused = path.fused;
  FrontParams fp = front_params(c);
  {
    Site s(c, "edge_fwd");
    launch_edge_fwd(st, E, pos, c->sender.p, c->receiver.p, c->shifts.p, c->species.p, c->bessel_w.p, c->zbl_z.p,
                    c->zbl_cov.p, c->ag_cov.p, fp, c->G > 1 ? c->gcell.p : nullptr, c->gid.p, c->geom.p, c->Y.p,
                    c->ef.p, c->zbl_e.p, c->Mt.p, c->mts,
                    // the fused TP kernels build their tables on chip from Y
                    (c->mts > 0 && !fused) ? tp_table_entries(c->max_lin) : 0, c->cutv.p);
  }
  for (size_t l = 0; l < c->layers.size(); ++l) {
    Layer& L = c->layers[l];
    const float* h = c->h[l].p;
    float* hn = c->h[l + 1].p;
    if (L.nonlin) {
      forward_nonlin(c, (int)l, h, hn);
      continue;
    }
    {
      Site s(c, lname("mlp_hidden", l));
      // split: h3 holds E x 2 x 64 fp16 (the same bytes as E x 64 floats)
      if (split)
        // no silu' saved: the VJP recomputes the hidden layers from ef
        // the fused kernels read h3's hi plane only (its lo plane is zero under a half policy)
        launch_mlp_hidden_x(st, E, nb, c->ef.p, L.mlp_tiles_x.p, L.mlp_winv, h3_of(c, l), h3inv_of(c, l), nullptr,
                            half, !(fused && half != RND_NONE));
      else
        launch_mlp_hidden(st, E, nb, c->ef.p, L.mlp_tiles.p,
                          h16 ? static_cast<void*>(c->h3h.p) : static_cast<void*>(c->h3.p), c->h3inv.p, L.ds.p,
                          h16 ? H3_F16 : half == RND_BF16 ? H3_BF16 : H3_F32);
    }
    if (!fused) {
      Site s(c, lname("mlp_out", l));
      if (h16)
        launch_mlp_out(st, E, L.wn, c->h3h.p, L.mlpT3h.p, L.wh.p, RND_F16, nullptr, nullptr);
      else if (split)
        launch_mlp_out_x(st, E, L.wn, c->h3.p, c->h3inv.p, L.mlpT3x.p, L.w3inv, L.w.p, nullptr, nullptr);
      else
        launch_mlp_out(st, E, L.wn, c->h3.p, L.mlpT[3].p, L.w.p, half, nullptr, nullptr);
    }
    if (l > 0) {  // the first layer's comes from the species table (launch_embed)
      Site s(c, lname("linear_up", l));
      GemmGroup g{};
      g.round_half = half;
      for (int b = 0; b < L.lin; ++b)
        g.p[g.n++] = gprob(N, 2 * b + 1, NC, NC, h, L.din, NC * b * b, 0, L.upT[b].p, L.h_up.p, L.din, NC * b * b, 0);
      run_gemm(c, st, g);
    }
    {
      Site s(c, lname("tp_fwd", l));
      if (fused)
        launch_tpx_fwd(st, L.lin, N, E, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, h3_of(c, l),
                       h3inv_of(c, l), L.mlpT3x.p, L.wn, L.w3inv, L.h_up.p, c->M.p, L.w.p, half, nullptr, nullptr,
                       !layer_rw(c, L));
      else
        launch_tp_fwd(st, L.lin, N, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, L.wptr(h16), L.h_up.p,
                      c->M.p, half);
    }
    const int* ao = tp_accoff(L.lin);
    if (c->dims.density_norm) {
      Site s(c, lname("density", l));
      launch_density_fwd(st, N, c->rowptr.p, c->ef.p, nb, L.dens.p, L.rinv.p);
    }
    {
      Site s(c, lname("linear_msg", l));
      GemmGroup g{};
      g.round_half = half;
      for (int lo = 0; lo < 4; ++lo) {
        int first, cnt;
        slot_range(L, lo, &first, &cnt);
        const int d = 2 * lo + 1;
        g.p[g.n++] = gprob(N, d, cnt * NC, NC, c->M.p, L.dmid, NC * ao[first], NC * d, L.linT[lo].p, L.A.p, L.dint,
                           NC * lo * lo, 0);
        if (c->dims.density_norm) g.p[g.n - 1].rowscale = L.rinv.p;
      }
      run_gemm(c, st, g);
    }
    if (!L.resid) {  // non-residual block: species-dependent skip FCTP on the message
      Site s(c, lname("message_skip", l));
      run_msg_skip(c, L, L.A.p, L.A2.p, L.mskipT, half);
    }
    const float* sc_in = L.resid ? L.A.p : L.A2.p;
    const float* scw[3] = {L.sc[0].p, L.sc[1].p, L.sc[2].p};
    {
      Site s(c, lname("sc_fwd", l));
      launch_sc_fwd(st, N, L.lhid, L.corr, sc_in, L.dint, sc_species(c), scw, c->B.p, L.dhid, half);
    }
    {
      // h' = PLin(B) + Skip(h): one two-operand GEMM per hidden block (and species present)
      Site s(c, lname("linear_prod", l));
      std::vector<GemmProb> probs;
      for (int b = 0; b < L.lhid; ++b) {
        GemmProb P = gprob(N, 2 * b + 1, NC, NC, c->B.p, L.dhid, NC * b * b, 0, L.plinT[b].p, hn, L.dhid, NC * b * b, 0);
        if (b < L.nskip) {
          set_skip_operand(P, h, L.din, b);
          add_species_probs(c, P, 2, L.skipT[b].p, probs);
        } else {
          probs.push_back(P);
        }
      }
      run_gemm_list(c, st, probs, half);
    }
  }
  // readouts, node energies and dE/dh_L (the backward's starting gradient) in one pass
  const int L = (int)c->layers.size();
  const float* hs[4] = {nullptr, nullptr, nullptr, nullptr};
  const float* ros[4] = {nullptr, nullptr, nullptr, nullptr};
  int lds[4] = {0, 0, 0, 0};
  for (int l = 0; l < L; ++l) {
    hs[l] = c->h[l + 1].p;
    lds[l] = c->layers[l].dhid;
    ros[l] = c->layers[l].ro.p;
  }
  Site s(c, "energy_readout");
  launch_energy_readout(st, N, c->species.p, c->e0.p, c->rowptr.p, c->dims.has_zbl ? c->zbl_e.p : nullptr, L, hs,
                        lds, ros, c->layers[L - 1].ro1.p, c->layers[L - 1].ro2.p, c->gh0.p, c->layers[L - 1].dhid,
                        c->node_e.p, e_part, half);
  if (c->G > 1) {
    Site s2(c, "graph_energy");
    launch_graph_energy(st, c->G, c->gptr.p, c->node_e.p, c->eg.p);
  }
}

void backward(mace_ctx* c, bool stress, double* out, const double* e_part, double* vir_part) {
  hipStream_t st = c->stream;
  const int N = c->N;
  const int64_t E = c->E;
  const int nb = c->dims.num_bessel;
  const int L = (int)c->layers.size();
  const int half = c->dims.feature_half;
  const StepPath path = step_path(c);
  const bool h16 = path.h16, split = path.split, fused = path.fused;
  int gyp = NSLICE;  // dL/dY partials per edge
  if (fused)
    for (const Layer& Ly : c->layers) gyp = std::max(gyp, tpx_parts(Ly.tl()));
  // dE/dh_L from the nonlinear readout: written by the forward's energy_readout pass
  float* gh = c->gh0.p;
  float* gh_next = c->gh1.p;
  for (int l = L - 1; l >= 0; --l) {
    Layer& Ly = c->layers[l];
    if (Ly.nonlin) {
      backward_nonlin(c, l, gh, gh_next, (l == L - 1) ? 0 : 1, gyp);
      if (l > 0) std::swap(gh, gh_next);
      continue;
    }
    {  // gB = PLin^T gh
      Site s(c, lname("linear_prod_bwd", l));
      GemmGroup g{};
      for (int b = 0; b < Ly.lhid; ++b)
        g.p[g.n++] =
            gprob(N, 2 * b + 1, NC, NC, gh, Ly.dhid, NC * b * b, 0, Ly.plin[b].p, c->gB.p, Ly.dhid, NC * b * b, 0);
      run_gemm(c, st, g);
    }
    const float* scw[3] = {Ly.sc[0].p, Ly.sc[1].p, Ly.sc[2].p};
    {
      Site s(c, lname("sc_bwd", l));
      launch_sc_bwd(st, N, Ly.lhid, Ly.corr, Ly.resid ? Ly.A.p : Ly.A2.p, Ly.dint, sc_species(c), scw, c->gB.p,
                    Ly.dhid, c->gA.p);
    }
    // gradient of the (normalised) message linear's output
    const float* gmsg = c->gA.p;
    if (!Ly.resid) {
      Site s(c, lname("message_skip_bwd", l));
      run_msg_skip(c, Ly, c->gA.p, c->gA2.p, Ly.mskip, 0);
      gmsg = c->gA2.p;
    }
    if (c->dims.density_norm) {
      Site s(c, lname("density_bwd", l));
      launch_density_node_bwd(st, N, Ly.dint, gmsg, Ly.A.p, Ly.rinv.p, c->grho.p);
    }
    const int* ao = tp_accoff(Ly.lin);
    {
      Site s(c, lname("linear_msg_bwd", l));
      GemmGroup g{};
      for (int lo = 0; lo < 4; ++lo) {
        int first, cnt;
        slot_range(Ly, lo, &first, &cnt);
        const int d = 2 * lo + 1;
        g.p[g.n++] = gprob(N, d, NC, cnt * NC, gmsg, Ly.dint, NC * lo * lo, 0, Ly.lin_[lo].p, c->gM.p, Ly.dmid,
                           NC * ao[first], NC * d);
        if (c->dims.density_norm) g.p[g.n - 1].rowscale = Ly.rinv.p;
      }
      run_gemm(c, st, g);
    }
    const int first_edge_grad = (l == L - 1) ? 0 : 1;  // gY / gef: write on the first layer visited
    if (fused) {
      // dL/dw stays on chip: the radial-MLP output layer's VJP (dL/dh3 partials) is fused in
      Site s(c, lname("tp_bwd", l));
      int acc_gy = first_edge_grad;
      if (!acc_gy && tpx_parts(Ly.lin) < gyp) {  // partials this layer does not write start at zero
        launch_fill_zero(st, c->gY.p, E * 16 * gyp);
        acc_gy = 1;
      }
      launch_tpx_bwd(st, Ly.lin, N, E, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, Ly.w.p, Ly.mlp3x.p, Ly.wn,
                     Ly.w3inv, Ly.h_up.p, c->gM.p, c->pos_s.p, l > 0 ? c->gxe.p : nullptr, c->gY.p, gyp, acc_gy,
                     c->gh3p.p, half, nullptr, nullptr, h3_of(c, l), h3inv_of(c, l), Ly.mlpT3x.p,
                     layer_rw(c, Ly));
    } else {
      // layers after the first also need dL/dx: per-edge rows in sender order, then a segmented sum
      Site s(c, lname("tp_bwd", l));
      launch_tp_bwd_recv(st, Ly.lin, N, c->rowptr.p, c->sender.p, c->Y.p, c->Mt.p, c->mts, Ly.wptr(h16),
                         Ly.h_up.p, c->gM.p, h16 ? static_cast<void*>(c->gwh.p) : static_cast<void*>(c->gw.p),
                         c->gscale.p, c->gY.p, first_edge_grad, c->pos_s.p, l > 0 ? c->gxe.p : nullptr, half);
    }
    if (l > 0) {
      Site s(c, lname("tp_gather", l));
      launch_tp_gather_gx(st, Ly.lin, N, srow(c), c->gxe.p, c->gup.p, fused && half == RND_F16, 0);
    }
    if (!fused) {
      Site s(c, lname("mlp_gh3", l));
      if (h16)
        launch_mlp_gh3_h(st, E, Ly.wn, c->gwh.p, c->gscale.p, Ly.mlp3h.p, c->h3.p);
      else if (split)
        launch_mlp_gh3_x(st, E, Ly.wn, c->gw.p, Ly.mlp3x.p, Ly.w3inv, c->h3.p, nullptr, nullptr);
      else
        launch_mlp_gh3(st, E, Ly.wn, c->gw.p, Ly.mlp[3].p, c->h3.p, nullptr, nullptr);
    }
    {
      Site s(c, lname("mlp_hidden_bwd", l));
      if (split)
        launch_mlp_hidden_bwd_x(st, E, nb, Ly.mlp_tiles_x.p, Ly.mlp_winv, c->ef.p, nullptr, fused ? c->gh3p.p : c->h3.p,
                                fused ? tpx_parts(Ly.lin) : 1, c->gef.p, first_edge_grad, half);
      else
        launch_mlp_hidden_bwd(st, E, nb, Ly.mlp_tiles.p, Ly.ds.p, c->h3.p, c->gef.p, first_edge_grad);
    }
    if (c->dims.density_norm) {  // edge densities' share of dL/def (after gef has been written)
      Site s(c, lname("density_edge_bwd", l));
      launch_density_edge_bwd(st, E, c->receiver.p, c->ef.p, nb, Ly.dens.p, c->grho.p, c->gef.p);
    }
    if (l > 0) {
      // dE/dh_l = Up^T gup + Skip^T gh + readout_{l-1}'
      {
        // dE/dh_l = Up^T gup + Skip^T gh (per species present) + readout_{l-1}' (bias on the 0e block)
        Site s(c, lname("linear_up_bwd", l));
        std::vector<GemmProb> probs;
        for (int b = 0; b < Ly.lin; ++b) {
          GemmProb P =
              gprob(N, 2 * b + 1, NC, NC, c->gup.p, Ly.din, NC * b * b, 0, Ly.up[b].p, gh_next, Ly.din, NC * b * b, 0);
          if (b == 0) P.bias = c->layers[l - 1].ro.p;
          if (b < Ly.nskip) {
            set_skip_operand(P, gh, Ly.dhid, b);
            add_species_probs(c, P, 2, Ly.skip[b].p, probs);
          } else {
            probs.push_back(P);
          }
        }
        run_gemm_list(c, st, probs, 0);
      }
      std::swap(gh, gh_next);
    }
  }
  FrontParams fp = front_params(c);
  {
    Site s(c, "edge_bwd");
    launch_edge_bwd(st, E, c->sender.p, c->receiver.p, c->species.p, c->bessel_w.p, c->zbl_z.p, c->zbl_cov.p,
                    c->ag_cov.p, fp,
                    c->geom.p, c->gY.p, gyp, c->gef.p, c->gv.p, stress ? vir_part : nullptr, c->gcut.p);
  }
  {
    Site s(c, "forces");
    launch_forces(st, N, c->rowptr.p, srow(c), c->perm_s.p, c->gv.p, out + 10,
                  (stress && E > 0) ? nullptr : out + 1, e_part, out);
  }
  if (stress && E > 0) {
    Site s(c, "virial");
    launch_virial_reduce(st, vir_part, (int)((E + 255) / 256), out + 1);
  }
  if (stress && c->G > 1) {
    Site s(c, "graph_virial");
    launch_graph_virial(st, c->G, c->gptr.p, c->rowptr.p, c->geom.p, c->gv.p, c->gvir.p);
  }
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

int mace_create(int32_t device, mace_ctx** out) {
  if (!out) return MACE_ERR_INVALID;
  *out = nullptr;
  mace_ctx* c = new mace_ctx();
  c->device = device;
  int rc = guard(c, [&] {
    int n = 0;
    HIPCHK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) fail(MACE_ERR_INVALID, "device %d out of range (%d devices)", device, n);
    set_device(c);
    c->scratch = scratch_on(device);
    // A blocking stream: its work is ordered with the null stream's (PyTorch's default
    // stream, and the synchronous copies of this library), so positions written there
    // before mace_step_device are seen by the step without an explicit wait.
    HIPCHK(hipStreamCreateWithFlags(&c->stream, hipStreamDefault));
    HIPCHK(hipStreamCreateWithFlags(&c->cap_stream, hipStreamNonBlocking));
    for (auto& e : c->ev) HIPCHK(hipEventCreate(&e));
  });
  if (rc != MACE_OK) {
    g_fail_msg = c->err;
    delete c;
    return rc;
  }
  *out = c;
  return MACE_OK;
}

static void free_all(mace_ctx* c) {
  invalidate_node_state(c);
  free_layers(c);
  for (auto& b : c->h) b.release();
  c->h3h.release();
  c->gwh.release();
  c->gscale.release();
  c->h3inv.release();
  for (auto* b : {&c->gptr, &c->gid}) b->release();
  for (auto* b : {&c->gcell, &c->eg, &c->gvir}) b->release();
  for (auto* b : {&c->e0, &c->bessel_w, &c->zbl_z, &c->zbl_cov, &c->ag_cov, &c->gA2, &c->grho, &c->embed, &c->up0_tab, &c->Y, &c->Mt, &c->ef, &c->zbl_e, &c->gY, &c->gef,
                  &c->gv, &c->gw, &c->gxe, &c->h3, &c->gh3p, &c->M, &c->B, &c->gB, &c->gA, &c->gM, &c->gh0, &c->gh1, &c->gup,
                  &c->node_e, &c->cutv, &c->gcut, &c->mh_dens, &c->gwb, &c->gP})
    b->release();
  c->zero_species.release();
  for (auto* b : {&c->species, &c->sp_perm, &c->sender, &c->receiver, &c->shifts, &c->rowptr, &c->rowptr_s, &c->perm_s, &c->pos_s,
                  &c->nl_img, &c->nl_img_s, &c->nl_cpre, &c->nl_hits, &c->nl_bin, &c->nl_bin_sorted, &c->nl_atoms, &c->nl_iota, &c->nl_counts,
                  &c->nl_bin_count, &c->nl_bin_start, &c->e_tmp_i, &c->e_tmp_j, &c->e_tmp_s, &c->e_perm,
                  &c->e_keys})
    b->release();
  c->pos.release();
  c->nl_wpos.release();
  c->nl_wpos_s.release();
  c->vir_part.release();
  c->out.release();
  c->e_part.release();
  c->geom.release();
  c->cub_tmp.release();
  if (c->out_pinned) (void)hipHostFree(c->out_pinned);
  if (c->ne_pinned) (void)hipHostFree(c->ne_pinned);
  if (c->pos_pinned) (void)hipHostFree(c->pos_pinned);
  if (c->nl_missing_h) (void)hipHostFree(c->nl_missing_h);
  if (c->e_pinned) (void)hipHostFree(c->e_pinned);
  if (c->skin_pinned) (void)hipHostFree(c->skin_pinned);
  c->e_pinned = nullptr;
  c->skin_pinned = nullptr;
  c->nl_pos_d.release();
  c->skin_flag.release();
  c->out_pinned = nullptr;
  c->ne_pinned = nullptr;
  c->pos_pinned = nullptr;
  c->nl_missing_h = nullptr;
  c->nl_missing.release();
  c->nl_check_pending = false;
}

void mace_destroy(mace_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  free_all(c);
  for (auto& e : c->ev)
    if (e) (void)hipEventDestroy(e);
  for (auto& e : c->ev_pool) (void)hipEventDestroy(e);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  if (c->cap_stream) (void)hipStreamDestroy(c->cap_stream);
  delete c;
}

const char* mace_last_error(const mace_ctx* c) { return c ? c->err.c_str() : g_fail_msg.c_str(); }

int mace_model_begin(mace_ctx* c, const mace_model_dims* dims) {
  if (!c || !dims) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    HIPCHK(hipStreamSynchronize(c->stream));  // queued steps still read the old model
    c->dims = *dims;
    c->host_tensors.clear();
    c->model_ready = false;
  });
}

int mace_model_set_tensor(mace_ctx* c, const char* name, const float* data, int64_t count) {
  if (!c || !name || (count > 0 && !data) || count < 0) return MACE_ERR_INVALID;
  return guard(c, [&] { c->host_tensors[name] = std::vector<float>(data, data + count); });
}

int mace_model_end(mace_ctx* c) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    HIPCHK(hipStreamSynchronize(c->stream));
    build_model(c);
    // the cached edges were built for the previous model's r_max + skin
    if (!c->edges_manual) c->nl_valid = false;
    if (c->system_ready) {
      // the system's species must be elements of the new model (else mace_set_system again)
      for (int z : c->species_h)
        if (z >= c->dims.num_elements) c->system_ready = false;
    }
    if (c->system_ready) {
      set_species_order(c);
      ensure_node_buffers(c);
      ensure_edge_buffers(c, c->E);  // per-layer edge buffers of the new model
    }
  });
}

namespace {

// G structures, n_atoms[g] atoms each, concatenated; cells9 [G][9], pbc3 [G][3].
void set_batch(mace_ctx* c, int32_t G, const int32_t* n_atoms, const int32_t* species, const double* cells9,
               const uint8_t* pbc3, double skin) {
  if (!c->model_ready) fail(MACE_ERR_STATE, "model not loaded");
  if (G < 1 || !n_atoms || !cells9 || !pbc3) fail(MACE_ERR_INVALID, "bad system arguments");
  std::vector<int> gp(G + 1, 0);
  for (int g = 0; g < G; ++g) {
    if (n_atoms[g] < 0) fail(MACE_ERR_INVALID, "structure %d: negative atom count", g);
    if ((int64_t)gp[g] + n_atoms[g] > INT32_MAX / 4) fail(MACE_ERR_INVALID, "too many atoms");
    gp[g + 1] = gp[g] + n_atoms[g];
  }
  const int n = gp[G];
  if (n > 0 && !species) fail(MACE_ERR_INVALID, "species is NULL");
  set_device(c);
  // steps queued by mace_step_device may still read the arrays rewritten below
  HIPCHK(hipStreamSynchronize(c->stream));
  for (int i = 0; i < n; ++i)
    if (species[i] < 0 || species[i] >= c->dims.num_elements)
      fail(MACE_ERR_SPECIES, "atom %d: species index %d outside [0, %d)", i, species[i], c->dims.num_elements);
  bool topo_changed = (n != c->N) || !c->system_ready || G != c->G || gp != c->gptr_h;
  if (!topo_changed) {
    for (int k = 0; k < 3 * G; ++k) topo_changed |= ((pbc3[k] != 0) != (c->gpbc_h[k] != 0));
    for (int k = 0; k < 9 * G; ++k) topo_changed |= std::fabs(cells9[k] - c->gcell_h[k]) > 1e-10;
  }
  topo_changed |= (skin != c->skin);
  c->N = n;
  c->skin = skin;
  c->G = G;
  c->gptr_h = gp;
  c->gcell_h.assign(cells9, cells9 + 9 * (size_t)G);
  c->gpbc_h.resize(3 * (size_t)G);
  for (int k = 0; k < 3 * G; ++k) c->gpbc_h[k] = pbc3[k] ? 1 : 0;
  std::memcpy(c->cell, cells9, sizeof c->cell);
  for (int k = 0; k < 3; ++k) c->pbc[k] = c->gpbc_h[k];
  // per-structure device arrays (read only when G > 1)
  std::vector<int> gid(std::max(n, 1), 0);
  for (int g = 0; g < G; ++g)
    for (int i = gp[g]; i < gp[g + 1]; ++i) gid[i] = g;
  const void* before[5] = {c->gptr.p, c->gid.p, c->gcell.p, c->eg.p, c->gvir.p};
  c->gptr.ensure(G + 1);
  c->gid.ensure(std::max(n, 1));
  c->gcell.ensure(9 * (size_t)G);
  c->eg.ensure(G);
  c->gvir.ensure(9 * (size_t)G);
  const void* after[5] = {c->gptr.p, c->gid.p, c->gcell.p, c->eg.p, c->gvir.p};
  if (std::memcmp(before, after, sizeof before) != 0) invalidate_graphs(c);  // captured steps hold pointers
  HIPCHK(hipMemcpy(c->gptr.p, gp.data(), (G + 1) * sizeof(int), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->gid.p, gid.data(), gid.size() * sizeof(int), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->gcell.p, cells9, 9 * (size_t)G * sizeof(double), hipMemcpyHostToDevice));
  HIPCHK(hipMemset(c->gvir.p, 0, 9 * (size_t)G * sizeof(double)));
  ensure_node_buffers(c);
  {
    c->species.ensure(std::max(n, 1));
    if (n > 0) HIPCHK(hipMemcpy(c->species.p, species, (size_t)n * sizeof(int), hipMemcpyHostToDevice));
    c->species_h.assign(species, species + n);
    set_species_order(c);
    if (topo_changed || c->edges_manual) {  // a manual edge list lasts until the next set_system
      c->nl_valid = false;
      c->edges_manual = false;
    }
    c->system_ready = true;
  }
}

}  // namespace

int mace_set_system(mace_ctx* c, int32_t n, const int32_t* species, const double* cell9, const uint8_t* pbc3,
                    double skin) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    if (n < 0 || (n > 0 && !species) || !cell9 || !pbc3) fail(MACE_ERR_INVALID, "bad system arguments");
    set_batch(c, 1, &n, species, cell9, pbc3, skin);
  });
}

int mace_set_batch(mace_ctx* c, int32_t n_structures, const int32_t* n_atoms, const int32_t* species,
                   const double* cells9, const uint8_t* pbc3, double skin) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] { set_batch(c, n_structures, n_atoms, species, cells9, pbc3, skin); });
}

int mace_set_edges(mace_ctx* c, int64_t E, const int32_t* sender, const int32_t* receiver, const int32_t* shifts3) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    if (!c->system_ready) fail(MACE_ERR_STATE, "system not set");
    if (E < 0 || (E > 0 && (!sender || !receiver || !shifts3))) fail(MACE_ERR_INVALID, "bad edge arrays");
    if (E > INT32_MAX / 4) fail(MACE_ERR_INVALID, "too many edges");
    for (int64_t e = 0; e < E; ++e)
      if (sender[e] < 0 || sender[e] >= c->N || receiver[e] < 0 || receiver[e] >= c->N)
        fail(MACE_ERR_INVALID, "edge %lld references atom outside [0, %d)", (long long)e, c->N);
    set_device(c);
    HIPCHK(hipStreamSynchronize(c->stream));
    c->E = E;
    ensure_edge_index(c, E);
    if (E > 0) {
      HIPCHK(hipMemcpy(c->e_tmp_i.p, sender, E * sizeof(int), hipMemcpyHostToDevice));
      HIPCHK(hipMemcpy(c->e_tmp_j.p, receiver, E * sizeof(int), hipMemcpyHostToDevice));
      HIPCHK(hipMemcpy(c->e_tmp_s.p, shifts3, 3 * E * sizeof(int), hipMemcpyHostToDevice));
      launch_fill_iota(c->stream, (int)E, c->nl_iota.p);
      cub_sort_pairs(c, c->e_tmp_j.p, c->e_keys.p, c->nl_iota.p, c->e_perm.p, E, c->N);
      MACE_LAUNCH(k_gather_edges, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, c->stream, E, c->e_perm.p,
                         c->e_tmp_i.p, c->e_tmp_j.p, c->e_tmp_s.p, c->sender.p, c->receiver.p, c->shifts.p);
    }
    c->rowptr.ensure((size_t)c->N + 1);
    build_rowptr(c, c->receiver.p, E, c->N, c->rowptr.p);
    build_sender_csr(c);
    ensure_edge_buffers(c, E);
    HIPCHK(hipStreamSynchronize(c->stream));
    c->nl_valid = true;
    c->edges_manual = true;
  });
}

int mace_get_edges(mace_ctx* c, int64_t cap, int32_t* sender, int32_t* receiver, int32_t* shifts3, int64_t* n_edges) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    if (!c->nl_valid) fail(MACE_ERR_STATE, "no edge list (call mace_step first)");
    if (n_edges) *n_edges = c->E;
    if (!sender && !receiver && !shifts3) return;
    if (cap < c->E) fail(MACE_ERR_INVALID, "capacity %lld < %lld edges", (long long)cap, (long long)c->E);
    set_device(c);
    HIPCHK(hipStreamSynchronize(c->stream));
    if (c->E > 0) {
      if (sender) HIPCHK(hipMemcpy(sender, c->sender.p, c->E * sizeof(int), hipMemcpyDeviceToHost));
      if (receiver) HIPCHK(hipMemcpy(receiver, c->receiver.p, c->E * sizeof(int), hipMemcpyDeviceToHost));
      if (shifts3) HIPCHK(hipMemcpy(shifts3, c->shifts.p, 3 * c->E * sizeof(int), hipMemcpyDeviceToHost));
    }
  });
}

int mace_step(mace_ctx* c, const double* positions, uint32_t flags, double* energy, double* node_energy,
              double* forces, double* virial9) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    if (!c->system_ready) fail(MACE_ERR_STATE, "system not set");
    if (c->N > 0 && !positions) fail(MACE_ERR_INVALID, "positions is NULL");
    if (!energy) fail(MACE_ERR_INVALID, "energy is NULL");
    set_device(c);
    check_step_path(c);
    const int N = c->N;
    const bool stress = (flags & MACE_STEP_STRESS) != 0;
    hipStream_t st = c->stream;
    HIPCHK(hipEventRecord(c->ev[0], st));
    std::memcpy(c->pos_pinned, positions, 3 * (size_t)N * sizeof(double));
    if (N > 0) HIPCHK(hipMemcpyAsync(c->pos.p, c->pos_pinned, 3 * (size_t)N * sizeof(double), hipMemcpyHostToDevice, st));
    // neighbour-list cache check (calculators.py:266-283)
    bool rebuild = !c->nl_valid || (flags & MACE_STEP_FORCE_NL);
    if (!rebuild && !c->edges_manual) {
      if (c->skin <= 0 || c->nl_pos.size() != 3 * (size_t)N) {
        rebuild = true;
      } else {
        double maxd2 = 0;
        for (int i = 0; i < N; ++i) {
          double d2 = 0;
          for (int k = 0; k < 3; ++k) {
            const double d = positions[3 * i + k] - c->nl_pos[3 * i + k];
            d2 += d * d;
          }
          maxd2 = std::max(maxd2, d2);
        }
        rebuild = std::sqrt(maxd2) > c->skin / 2;
      }
    }
    if (c->edges_manual && (flags & MACE_STEP_FORCE_NL)) c->edges_manual = false;
    c->last_nl = rebuild && !c->edges_manual;
    if (c->last_nl) build_nl(c, positions);
    HIPCHK(hipEventRecord(c->ev[1], st));
    ensure_embed(c);
    // a step on a freshly built list runs eagerly; the graphs for the next steps are captured
    // below, while the GPU executes it
    const bool ahead = c->last_nl && graphs_active(c);
    auto fwd = [&] { forward(c, c->pos.p, c->out.p, c->e_part.p); };
    auto bwd = [&] { backward(c, stress, c->out.p, c->e_part.p, c->vir_part.p); };
    if (ahead) fwd(); else run_captured(c, c->g_fwd, c->pos.p, c->out.p, 0, fwd);
    HIPCHK(hipEventRecord(c->ev[2], st));
    if (ahead) bwd(); else run_captured(c, c->g_bwd, c->out.p, nullptr, stress, bwd);
    HIPCHK(hipEventRecord(c->ev[3], st));
    HIPCHK(hipMemcpyAsync(c->out_pinned, c->out.p, (10 + 3 * (size_t)N) * sizeof(double), hipMemcpyDeviceToHost, st));
    if (node_energy && N > 0)
      HIPCHK(hipMemcpyAsync(c->ne_pinned, c->node_e.p, (size_t)N * sizeof(float), hipMemcpyDeviceToHost, st));
    HIPCHK(hipEventRecord(c->ev[4], st));
    queue_nl_missing(c);
    if (ahead) {
      capture_graph(c, c->g_fwd, c->pos.p, c->out.p, 0, fwd);
      capture_graph(c, c->g_bwd, c->out.p, nullptr, stress, bwd);
    }
    HIPCHK(hipStreamSynchronize(st));
    HIPCHK(hipGetLastError());
    check_nl_missing(c);
    *energy = c->out_pinned[0];
    if (virial9 && stress) std::memcpy(virial9, c->out_pinned + 1, 9 * sizeof(double));
    if (forces) std::memcpy(forces, c->out_pinned + 10, 3 * (size_t)N * sizeof(double));
    if (node_energy)
      for (int i = 0; i < N; ++i) node_energy[i] = (double)c->ne_pinned[i];
    float ms[4];
    HIPCHK(hipEventElapsedTime(&ms[0], c->ev[0], c->ev[4]));
    HIPCHK(hipEventElapsedTime(&ms[1], c->ev[0], c->ev[1]));
    HIPCHK(hipEventElapsedTime(&ms[2], c->ev[1], c->ev[2]));
    HIPCHK(hipEventElapsedTime(&ms[3], c->ev[2], c->ev[3]));
    for (int k = 0; k < 4; ++k) c->timings[k] = ms[k];
    if (!c->last_nl) c->timings[1] = 0.0;
    prof_harvest(c);
  });
}

int mace_step_batch(mace_ctx* c, const double* positions, uint32_t flags, double* energies, double* node_energy,
                    double* forces, double* virials9) {
  if (!c) return MACE_ERR_INVALID;
  if (!energies) {
    c->err = "energies is NULL";
    return MACE_ERR_INVALID;
  }
  const bool stress = (flags & MACE_STEP_STRESS) != 0;
  double e = 0.0, vir[9] = {0};
  const int rc = mace_step(c, positions, flags, &e, node_energy, forces, stress ? vir : nullptr);
  if (rc != MACE_OK) return rc;
  return guard(c, [&] {
    const int G = c->G;
    if (G == 1) {
      energies[0] = e;
      if (virials9) std::memcpy(virials9, vir, sizeof vir);
      return;
    }
    set_device(c);
    HIPCHK(hipMemcpy(energies, c->eg.p, G * sizeof(double), hipMemcpyDeviceToHost));
    if (virials9) {
      if (stress) HIPCHK(hipMemcpy(virials9, c->gvir.p, 9 * (size_t)G * sizeof(double), hipMemcpyDeviceToHost));
      else std::fill(virials9, virials9 + 9 * (size_t)G, 0.0);
    }
  });
}

int mace_step_device(mace_ctx* c, const double* d_positions, uint32_t flags, double* d_out) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    if (!c->system_ready) fail(MACE_ERR_STATE, "system not set");
    if ((c->N > 0 && !d_positions) || !d_out) fail(MACE_ERR_INVALID, "NULL device pointer");
    set_device(c);
    check_step_path(c);
    const int N = c->N;
    hipStream_t st = c->stream;
    bool rebuilt = false;
    bool rebuild = (flags & MACE_STEP_FORCE_NL) || !c->nl_valid;
    if (!rebuild && (flags & MACE_STEP_SKIN_CHECK) && !c->edges_manual) rebuild = skin_exceeded_on_device(c, d_positions);
    if (rebuild) {
      if (N > 0)
        HIPCHK(hipMemcpyAsync(c->pos.p, d_positions, 3 * (size_t)N * sizeof(double), hipMemcpyDeviceToDevice, st));
      // host positions only for the extents of non-periodic directions
      bool periodic = true;
      for (uint8_t f : c->gpbc_h) periodic = periodic && f;
      std::vector<double> host;
      if (!periodic) {
        host.resize(3 * (size_t)N);
        if (N > 0)
          HIPCHK(hipMemcpyAsync(host.data(), d_positions, host.size() * sizeof(double), hipMemcpyDeviceToHost, st));
        HIPCHK(hipStreamSynchronize(st));
      }
      c->edges_manual = false;
      build_nl(c, periodic ? nullptr : host.data());
      rebuilt = true;
    }
    const bool stress = (flags & MACE_STEP_STRESS) != 0;
    ensure_embed(c);
    auto fwd = [&] { forward(c, d_positions, d_out, c->e_part.p); };
    auto bwd = [&] { backward(c, stress, d_out, c->e_part.p, c->vir_part.p); };
    if (rebuilt && graphs_active(c)) {
      // eagerly on the fresh list (the build discarded the graphs).  The graphs are captured by
      // the next step that replays them: this call returns without waiting, so that capture
      // overlaps the GPU's work on this step, and a run of rebuilding steps captures none
      fwd();
      bwd();
    } else {
      run_captured(c, c->g_fwd, d_positions, d_out, 0, fwd);
      run_captured(c, c->g_bwd, d_out, nullptr, stress, bwd);
    }
  });
}

int mace_step_device_noalloc(mace_ctx* c, const double* d_positions, uint32_t flags, double* d_out) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    if (!c->system_ready) fail(MACE_ERR_STATE, "system not set");
    if ((c->N > 0 && !d_positions) || !d_out) fail(MACE_ERR_INVALID, "NULL device pointer");
    if (flags & MACE_STEP_FORCE_NL)
      fail(MACE_ERR_INVALID, "mace_step_device_noalloc never rebuilds the neighbour list (MACE_STEP_FORCE_NL)");
    if (!c->nl_valid)
      fail(MACE_ERR_STATE, "no neighbour list: build it with mace_step or mace_step_device first");
    if (c->profiling) fail(MACE_ERR_STATE, "per-launch profiling is on (it creates events): switch it off");
    if (!c->scratch) fail(MACE_ERR_STATE, "scratch address not set up for this context's device");
    const int64_t E = c->E;
    const size_t e_n = (size_t)((c->N + 3) / 4) + 1;
    const size_t v_n = 9 * (size_t)((E + 255) / 256);
    if (e_n + v_n > kScratchDoubles)
      fail(MACE_ERR_INVALID,
           "system too large for mace_step_device_noalloc: %d atoms and %lld edges need %zu scratch doubles, "
           "the maximum is %zu (use mace_step_device)",
           c->N, (long long)E, e_n + v_n, kScratchDoubles);
    set_device(c);
    check_step_path(c);
    const bool stress = (flags & MACE_STEP_STRESS) != 0;
    double* e_part = c->scratch;      // every block writes its own slot: nothing to clear
    double* vir_part = c->scratch + e_n;
    ensure_embed(c);
    forward(c, d_positions, d_out, e_part);
    backward(c, stress, d_out, e_part, vir_part);
  });
}

int mace_set_graphs(mace_ctx* c, int32_t enable) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    c->use_graphs = enable != 0;
    if (!c->use_graphs) invalidate_graphs(c);
  });
}

int mace_set_split_products(mace_ctx* c, int32_t enable) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    c->split_products = enable != 0;
    invalidate_graphs(c);
    if (c->model_ready && c->E > 0) ensure_edge_buffers(c, c->E);  // the arrays of the path now taken
  });
}

int mace_set_rebuild_w(mace_ctx* c, int32_t enable) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    HIPCHK(hipStreamSynchronize(c->stream));  // queued steps still read the stored w
    c->rebuild_w = enable != 0;
    invalidate_graphs(c);
    if (c->model_ready && c->E > 0) ensure_edge_buffers(c, c->E);
  });
}

int mace_set_fused_tp(mace_ctx* c, int32_t enable) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    c->fused_tp = enable != 0;
    invalidate_graphs(c);
    if (c->model_ready && c->E > 0) ensure_edge_buffers(c, c->E);
  });
}

int mace_sync(mace_ctx* c) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    queue_nl_missing(c);
    HIPCHK(hipStreamSynchronize(c->stream));
    HIPCHK(hipGetLastError());
    check_nl_missing(c);
    prof_harvest(c);
  });
}

int mace_set_profiling(mace_ctx* c, int32_t enable) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    prof_harvest(c);
    c->profiling = enable != 0;
    c->prof_acc.clear();
  });
}

int mace_get_kernel_times(mace_ctx* c, char* names, int64_t names_len, double* total_ms, int64_t* counts,
                          int32_t capacity, int32_t* n_sites) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    set_device(c);
    prof_harvest(c);
    if (n_sites) *n_sites = (int32_t)c->prof_acc.size();
    if (!names) return;
    std::string all;
    int32_t i = 0;
    for (auto& kv : c->prof_acc) {
      if (i >= capacity) break;
      all += kv.first + "\n";
      if (total_ms) total_ms[i] = kv.second.first;
      if (counts) counts[i] = kv.second.second;
      ++i;
    }
    if ((int64_t)all.size() + 1 > names_len) fail(MACE_ERR_INVALID, "names buffer too small (%zu)", all.size() + 1);
    std::memcpy(names, all.c_str(), all.size() + 1);
    c->prof_acc.clear();
  });
}

int mace_get_launch_order(mace_ctx* c, char* names, int64_t names_len, int32_t* n_dispatches) {
  if (!c) return MACE_ERR_INVALID;
  return guard(c, [&] {
    if (n_dispatches) *n_dispatches = (int32_t)c->launch_log.size();
    if (!names) return;
    std::string all;
    for (auto& s : c->launch_log) all += s + "\n";
    if ((int64_t)all.size() + 1 > names_len) fail(MACE_ERR_INVALID, "names buffer too small (%zu)", all.size() + 1);
    std::memcpy(names, all.c_str(), all.size() + 1);
  });
}

int mace_get_timings(const mace_ctx* c, double* out, int32_t n) {
  if (!c || !out) return MACE_ERR_INVALID;
  const int m = std::min<int32_t>(n, 4);
  for (int k = 0; k < m; ++k) out[k] = c->timings[k];
  return m;
}

}  // extern "C"
