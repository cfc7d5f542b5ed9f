"""CPU parity oracle -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker / CPU baseline.
The product path (``mace_mlx_amd``) never imports it and has no CPU fallback:
without the HIP library it raises.

Contents
--------
``model``      PyTorch-CPU (float64 / float32) restatement of the reference MACE
               energy model; forces and stress come from torch autograd, i.e.
               independently of the hand-written GPU VJPs.
``neighbors``  float64 brute-force periodic neighbour enumeration (i, j, S).

Pinning (what checks each part against something other than itself):

* coupling constants (3j, D, U) -- golden vectors written from the reference's
  own `clebsch_gordan.py` (tests/golden/cg_fixtures.npz) plus 3j invariants;
* spherical harmonics -- closed forms for l <= 2, component norm 2l+1,
  equivariance under the reference's Wigner-D;
* Bessel / cutoff -- closed-form values and boundary behaviour;
* ZBL -- at the universal screening parameters, an isolated pair's energy equals
  the published ZBL universal potential (Ziegler, Biersack & Littmark 1985,
  five-digit coefficients, CODATA constants) within the reference's four-digit
  rounding, and planted coefficient / exponent swaps fail by more than 1 %;
* radial MLP -- the model file's layers load strictly into a torch
  ``nn.Sequential(Linear(bias=False), SiLU, ...)`` with the same output;
* density normalisation -- on a lattice where every edge has the same features,
  the block equals the plain block with avg_num_neighbors = 1 + k tanh(c^2);
* neighbour list -- edge counts recorded by the reference (2944 for Si64,
  46000 for Si1000, `docs/prototypes/profile_results.json`), shell counts, and
  the (i, j, S) <-> (j, i, -S) pairing;
* whole model -- finite-difference forces and stress, translation / rotation /
  permutation invariance, sum of forces = 0, stress symmetry, the stress-path
  forces equal the energy-path forces, single-atom and far-pair cases;
* symmetric contraction -- the row-compressed main step equals the dense einsum
  definition (`symmetric_contraction.py:95-121`) on random tensors;
* architecture bookkeeping -- the layer-1 conv-TP instruction table the reference
  records (`docs/prototypes/teamA_convtp_batch.md:18-29`), the EquivariantLinear
  known answer of the reference's own test (`tests/test_linear.py:194-226`), and
  the unit second moment every Linear / FCTP / conv-TP output must have;
* mh-1 block -- LayerNorm and the LayerNorm MLP against torch's own modules, the
  gate against its closed form and equivariance, e3nn's normalize2mom constants
  recomputed the way e3nn computes them, FD forces / stress, and the reductions
  beta = 0 (density off) and agnostic product = copied per-element weights.

Every function of ``model`` and ``neighbors`` has a check above.  Parity
unpinned outside them: the MLX-executed values of the reference itself (MLX is
not installable here), MLX's RNG / initialisers (weights are exchanged as
files), and ASE's covalent-radius table (a published table is vendored instead).
"""
