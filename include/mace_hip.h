/*
 * mace_hip.h -- C ABI of the MI355X MACE energy / forces / stress engine.
 *
 * The library replaces the reference's per-step compiled function
 *   step(pos, node_attrs, edge_index, shifts, cell, batch) -> ((E, node_energy), dE/dpos)
 * of `mace_mlx/calculators.py:424-476` and its stress variant
 * `calculators.py:482-563`, plus the matscipy neighbour list with skin caching of
 * `calculators.py:44-55,266-310`.  The Python host (`mace_mlx_amd.calculators`)
 * keeps the reference's ASE-facing API (`mace_mp`, `mace_off`, `MACECalculator`)
 * and drives these entry points through ctypes.
 *
 * Conventions
 *   - Every entry point returns MACE_OK (0) or a negative MACE_ERR_* code; the
 *     message of the last failure is available from mace_last_error().  No C++
 *     exception crosses the boundary.
 *   - The caller owns every host array; the context owns all device memory and
 *     one HIP stream.  A context is not re-entrant (one thread at a time);
 *     several contexts may share a device.
 *   - Ordering: the context's stream is a blocking stream, so its work is ordered
 *     with the null stream (PyTorch's default stream): device arrays written there
 *     before mace_step_device are read after the writes land, and null-stream work
 *     queued after mace_step_device waits for the step.  Work on any other stream
 *     must be synchronised by the caller first.  mace_model_begin / _end,
 *     mace_set_system / _batch and mace_set_edges wait for the context's queued
 *     steps before they replace what those steps read.
 *   - Edges follow the reference: edge_index = [sender i; receiver j], shift S,
 *     edge vector D = x_j - x_i + S @ cell (`utils.py:47-84`).
 */
#ifndef MACE_HIP_H
#define MACE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MACE_OK 0
#define MACE_ERR_INVALID (-1)     /* bad argument / inconsistent sizes   -> ValueError */
#define MACE_ERR_HIP (-2)         /* HIP runtime failure                 -> RuntimeError */
#define MACE_ERR_UNSUPPORTED (-3) /* model topology not implemented      -> NotImplementedError */
#define MACE_ERR_STATE (-4)       /* call order (model / system missing) -> RuntimeError */
#define MACE_ERR_SPECIES (-5)     /* species index outside the model     -> ValueError */

/* mace_step flags */
#define MACE_STEP_FORCES 1u        /* compute forces (always on in practice)               */
#define MACE_STEP_STRESS 2u        /* also compute the virial dE/d(eps) (calculators.py:526) */
#define MACE_STEP_FORCE_NL 4u      /* rebuild the neighbour list regardless of the skin     */
#define MACE_STEP_SKIN_CHECK 8u    /* mace_step_device: apply the skin criterion on the
                                      device (calculators.py:266-283)                     */

typedef struct mace_ctx mace_ctx;

/* Model dimensions; every array passed to mace_model_set_tensor is checked
 * against the sizes these imply. */
typedef struct mace_model_dims {
  int32_t num_elements;      /* one-hot width (len(z_table))                    */
  int32_t num_channels;      /* multiplicity of every irrep block (128)         */
  int32_t max_ell;           /* spherical-harmonic degree (3)                   */
  int32_t num_bessel;        /* radial basis size (8)                           */
  int32_t num_poly_cutoff;   /* polynomial envelope order p (5)                 */
  int32_t num_layers;        /* interaction layers (2)                          */
  int32_t radial_hidden;     /* width of the radial MLP hidden layers (64)      */
  int32_t radial_depth;      /* number of hidden layers of the radial MLP (3)   */
  int32_t layer_in_blocks[4];  /* input irreps of layer l: blocks 0e,1o,2e[:n]  */
  int32_t layer_hid_blocks[4]; /* hidden (output) irreps of layer l             */
  int32_t correlation[4];
  int32_t has_zbl;
  int32_t zbl_p;
  double r_max;
  double zbl_a_exp;
  double zbl_a_prefactor;
  double zbl_scale;          /* ScaleShiftMACE scale applied to the pair term  */
  int32_t feature_half;      /* 1: float16 feature policy (model.py:1-15, 592-661): weights
                                rounded to fp16 on the host except E0 / Bessel frequencies,
                                SH and radial features and every stored activation of the
                                feature path rounded to fp16, TP weights held in fp16,
                                accumulation in fp32; 2: bfloat16 policy (model.py:592-596,
                                705-711): the same rounding points with bf16 values (round
                                to nearest even), held in fp32 arrays; 0: float32 throughout */
  int32_t density_norm;      /* 1: density-normalised interactions (blocks.py:282-490):
                                tensor L<l>.dens, message linear / (1 + sum tanh((ef.w)^2)) */
  int32_t first_nonresidual; /* 1: first interaction without residual skip; its skip FCTP
                                acts on the message (blocks.py:68-176): tensors L0.mskip.<l> */
  int32_t agnesi;            /* 1: Agnesi distance transform before the Bessel basis
                                (radial.py:207-262): tensor agnesi_cov (radius per element) */
  double agnesi_q;
  double agnesi_p;
  double agnesi_a;
  int32_t nonlinear;         /* 1: mh-1 non-linear interaction blocks (blocks.py:611-807):
                                LayerNorm radial / density MLPs over [ef | source | target
                                species embedding], message linear_1 / (beta rho + alpha) +
                                linear_res, gate, linear_2; plain-linear skip (tensors
                                L<l>.rmlp.*, L<l>.dmlp.*, L<l>.ab, L<l>.res.<l>, L<l>.lin2.<l>) */
  int32_t separate_cutoff;   /* 1: apply_cutoff = False (radial.py:316-318): the polynomial
                                envelope multiplies the TP weights and the edge densities
                                instead of the radial basis; only with nonlinear = 1          */
  int32_t agnostic_product;  /* 1: one set of symmetric-contraction weights for every element
                                (blocks.py:510-533): tensors L<l>.sc.<b> hold one element        */
  int32_t layer_edge_blocks[4]; /* nonlinear: blocks 0e,1o,2e[:n] of linear_up's output (edge
                                irreps, model.py:192-211); 0 otherwise                          */
} mace_model_dims;

/* Context lifetime.  device = HIP device ordinal. */
int mace_create(int32_t device, mace_ctx** out);
void mace_destroy(mace_ctx* ctx);
const char* mace_last_error(const mace_ctx* ctx);

/* Model upload.  Tensor names and layouts are produced by
 * mace_mlx_amd.device_model from the reference's config.json + weights.npz
 * (`model.py:664-720`); see that module for the list. */
int mace_model_begin(mace_ctx* ctx, const mace_model_dims* dims);
int mace_model_set_tensor(mace_ctx* ctx, const char* name, const float* data, int64_t count);
int mace_model_end(mace_ctx* ctx);

/* System topology: atom count, species index per atom (0..num_elements-1),
 * cell (row-major 3x3, rows = lattice vectors) and pbc flags.  Changing the
 * cell or pbc beyond 1e-10 invalidates the neighbour list
 * (`calculators.py:266-283`).  skin <= 0 rebuilds every step.  The species
 * array is also sorted here (per-species row maps of the element-dependent skip
 * products), so a new assignment at the same atom count goes through this call. */
int mace_set_system(mace_ctx* ctx, int32_t n_atoms, const int32_t* species,
                    const double* cell9, const uint8_t* pbc3, double skin);

/* One energy + forces (+ virial) evaluation at `positions` (n_atoms x 3, Angstrom).
 *   energy       : total energy (eV)
 *   node_energy  : n_atoms per-atom energies, may be NULL
 *   forces       : n_atoms x 3, -dE/dpos, may be NULL
 *   virial9      : dE/d(eps_sym) (3x3, row-major; stress = virial / |det cell|),
 *                  only with MACE_STEP_STRESS, may be NULL
 * Synchronous.  Rebuilds the neighbour list on the device when the skin
 * criterion of `calculators.py:266-283` fails. */
int mace_step(mace_ctx* ctx, const double* positions, uint32_t flags, double* energy,
              double* node_energy, double* forces, double* virial9);

/* A batch of independent structures evaluated in one step: the reference model's
 * batched call (`model.py:440-484`: positions of all structures, `batch` = structure
 * index per atom, energies summed per structure by `graph_sum`, `utils.py:35-44`).
 * Structure g has n_atoms[g] atoms (consecutive in species / positions / forces),
 * its own cell (cells9 + 9 g) and pbc (pbc3 + 3 g); no edge joins two structures.
 * mace_set_system is the one-structure case.  mace_step_batch returns
 *   energies   : n_structures energies (eV)
 *   virials9   : n_structures x 9, per-structure dE/d(eps_sym) with MACE_STEP_STRESS
 *                (zeros without), may be NULL
 * and node_energy / forces over all atoms as mace_step; the total energy and virial
 * of the batch are what mace_step / mace_step_device report for it. */
int mace_set_batch(mace_ctx* ctx, int32_t n_structures, const int32_t* n_atoms,
                   const int32_t* species, const double* cells9, const uint8_t* pbc3, double skin);
int mace_step_batch(mace_ctx* ctx, const double* positions, uint32_t flags, double* energies,
                    double* node_energy, double* forces, double* virials9);

/* Test hooks.  mace_set_edges installs an explicit edge list (bypassing the
 * neighbour list until the next mace_set_system); mace_get_edges copies the
 * current list (receiver-sorted) out.  *n_edges returns the count; arrays may be
 * NULL to query the count only. */
int mace_set_edges(mace_ctx* ctx, int64_t n_edges, const int32_t* sender,
                   const int32_t* receiver, const int32_t* shifts3);
int mace_get_edges(mace_ctx* ctx, int64_t capacity, int32_t* sender, int32_t* receiver,
                   int32_t* shifts3, int64_t* n_edges);

/* Device-resident variant of mace_step for callers that keep positions and
 * results in HBM (MD integrators on the GPU, benchmarks).  d_positions: device
 * array n_atoms x 3 (double); d_out: device array of 10 + 3 n_atoms doubles that
 * receives [energy, virial (3x3, symmetrised, zero without MACE_STEP_STRESS),
 * forces (n_atoms x 3)].  Work is queued on the context's stream and the call
 * returns without synchronising (mace_sync waits).  The neighbour list is used
 * as cached: the caller guarantees no atom moved more than skin/2 since the last
 * rebuild, or passes MACE_STEP_FORCE_NL (which rebuilds, synchronously), or passes
 * MACE_STEP_SKIN_CHECK: the largest displacement since the last rebuild is then reduced
 * on the device and read back (one synchronisation per step), and the list is rebuilt
 * when it exceeds skin/2 (skin <= 0: every step), the criterion of mace_step.
 * No host-side counterpart in the reference (its step always round-trips
 * through host arrays, calculators.py:455-476). */
int mace_step_device(mace_ctx* ctx, const double* d_positions, uint32_t flags, double* d_out);
int mace_sync(mace_ctx* ctx);

/* mace_step_device for callers that cannot allocate device memory: code that captures
 * the step into its own HIP graph, tight serving / MD loops, harnesses that forbid
 * allocation.  No counterpart in the reference.  Same arguments and results as
 * mace_step_device; the call allocates and frees nothing (no hipMalloc / hipFree, no
 * event creation, no graph capture of its own: the step's kernels are launched one by one
 * on the context's stream, so a caller may capture them).  The per-block energy and
 * virial partials come from a fixed per-device array of 2 MiB inside the library
 * ((ceil(n_atoms / 4) + 1) + 9 ceil(n_edges / 256) doubles must fit 262144: about 7
 * million edges), which every call on that device shares and which keeps the last
 * call's contents; calls that overlap on one device (several contexts, several streams)
 * race on it.  Everything else uses the context's buffers, sized by mace_set_system /
 * mace_set_batch and the last neighbour-list build, so the neighbour list must exist
 * (built by mace_step or mace_step_device) and is never rebuilt here: the caller keeps
 * every atom within skin/2 of where it was built.  Errors: MACE_ERR_STATE without a
 * neighbour list or with profiling on; MACE_ERR_INVALID for MACE_STEP_FORCE_NL or a
 * system beyond the array's size. */
int mace_step_device_noalloc(mace_ctx* ctx, const double* d_positions, uint32_t flags, double* d_out);

/* Per-launch-site device timing (HIP events around every kernel launch of the
 * step, on the context's stream).  Enabling adds two event records per launch.
 * mace_get_kernel_times synchronises, then reports for each site its name
 * ('\n'-separated in names), accumulated milliseconds and launch count, and
 * resets the accumulators.  *n_sites receives the number of sites. */
int mace_set_profiling(mace_ctx* ctx, int32_t enable);
int mace_get_kernel_times(mace_ctx* ctx, char* names, int64_t names_len, double* total_ms,
                          int64_t* counts, int32_t capacity, int32_t* n_sites);

/* The launch site of every kernel dispatch of the last step run with profiling
 * enabled, in dispatch order ('\n'-separated; a site that dispatches k kernels is
 * listed k times).  *n_dispatches receives the count; names may be NULL to query
 * it only.  Used to map a profiler's per-dispatch records (rocprofv3 kernel trace,
 * counters) to launch sites.  No counterpart in the reference. */
int mace_get_launch_order(mace_ctx* ctx, char* names, int64_t names_len, int32_t* n_dispatches);

/* Step replay through HIP graphs (default on).  The forward and the backward
 * launches of a step are captured once per (positions, output, stress) binding
 * and neighbour-list / buffer state, then replayed with one hipGraphLaunch
 * each; any rebuild or reallocation discards them.  Profiling mode always runs
 * eagerly.  Results are identical either way (the kernels are deterministic).
 * No counterpart in the reference (its analogue is mx.compile,
 * calculators.py:424-453). */
int mace_set_graphs(mace_ctx* ctx, int32_t enable);

/* Float32 policy: matrix products on fp16 matrix cores with both operands split
 * into fp16 pairs, a = a_hi + a_lo (power-of-two scales per row and 32-wide k
 * chunk, or per weight matrix), three products per pair and fp32 accumulation:
 * about 2^-21 relative error per product, within the float32 tolerances (default
 * on).  Covers the radial MLP's output layer (w = h3 W3 and its transpose in the
 * backward pass) and the node linears (up / message / product / skip, both
 * passes).  0 selects fp32 matrix cores throughout.  Ignored under the float16
 * feature policy.  No counterpart in the reference (its matmuls run in the model
 * dtype, model.py:592-661). */
int mace_set_split_products(mace_ctx* ctx, int32_t enable);

/* With split products on (float32 feature policy): build the radial MLP's
 * per-edge tensor-product weights inside the tensor-product kernels, tile by
 * tile, instead of materialising them in a separate pass first (enable != 0,
 * the default).  The arithmetic is the same split product; only the order of
 * the work changes.  Off selects the separate passes (kept for comparison).
 * No counterpart in the reference (the same evaluation as
 * blocks.py:253-274). */
int mace_set_fused_tp(mace_ctx* ctx, int32_t enable);

/* Float16 and bfloat16 feature policies, standard interaction blocks with one
 * or two input-degree blocks: the tensor-product VJP rebuilds the per-edge
 * weights w from the radial MLP's last hidden layer (kept by the forward) on
 * matrix cores instead of reading w back from memory, and the forward then
 * does not store w (enable != 0, the default).  The rebuilt values are the
 * same 16-bit numbers the forward used, so results do not change.  No
 * counterpart in the reference (the same evaluation as blocks.py:253-274). */
int mace_set_rebuild_w(mace_ctx* ctx, int32_t enable);

/* Timing of the last mace_step (device milliseconds, HIP events on the
 * context's stream): [0] whole step, [1] neighbour list (0 if cached),
 * [2] forward, [3] backward.  Returns the number of values written. */
int mace_get_timings(const mace_ctx* ctx, double* out, int32_t n);

#ifdef __cplusplus
}
#endif
#endif /* MACE_HIP_H */
