"""Pins the architecture bookkeeping (instruction lists, slot order, path weights)
against answers the reference itself holds, and the normalisations against the
second-moment property they are defined by.

* The layer-1 conv-TP instruction table of the medium architecture recorded in the
  reference (`docs/prototypes/teamA_convtp_batch.md:18-29`: i_in1, i_in2, i_out,
  (d1, d2, do), path weights 1 / 1.7321 / 2.2361 / 2.6458), its derived sizes
  (weight_numel 1280, K0 = 16, K1 = 24, OUTDIM = 5120:
  `docs/prototypes/team_metal_proto_mul21.py:4-15`, `teamA_convtp_batch.md:31-33`),
  checked for all three generators: the oracle's restatement, the product's
  `model_io.conv_tp_instructions` and the kernel-table generator `gen_tables`.
* The EquivariantLinear known answer of the reference's own test
  (`tests/test_linear.py:194-226`): `2x0e + 3x0e -> 1x0e` has two instructions with
  path weight 1/sqrt(5) and y = pw (x0 . w0 + x1 . w1).
* Component normalisation: with unit-variance inputs, component-normalised spherical
  harmonics and N(0, 1) weights every output component of a Linear, an FCTP and a
  conv TP has unit second moment (that is what the path weights are chosen for,
  `linear.py:46-74`, `tensor_product.py:1080-1098`, `utils.py:143-154`).  A dropped
  or misplaced path-weight factor moves some slot's moment by a factor 3/5/7 or
  its inverse and fails.
"""

import math

import numpy as np
import pytest
import torch

import gen_tables
from mace_mlx_amd import model_io
from mace_mlx_amd.irreps import Irreps
from oracle import model as om

# teamA_convtp_batch.md:18-29 -- (i_in1, i_in2, i_out, (d1, d2, do), path_weight)
REF_TABLE = [
    (0, 0, 0, (1, 1, 1), 1.0000),
    (1, 1, 1, (3, 3, 1), 1.0000),
    (0, 1, 2, (1, 3, 3), 1.7321),
    (1, 0, 3, (3, 1, 3), 1.7321),
    (1, 2, 4, (3, 5, 3), 1.7321),
    (0, 2, 5, (1, 5, 5), 2.2361),
    (1, 1, 6, (3, 3, 5), 2.2361),
    (1, 3, 7, (3, 7, 5), 2.2361),
    (0, 3, 8, (1, 7, 7), 2.6458),
    (1, 2, 9, (3, 5, 7), 2.6458),
]

IN1 = Irreps("128x0e+128x1o")
SH = Irreps("0e+1o+2e+3o")
TARGET = Irreps("128x0e+128x1o+128x2e+128x3o")


def _check_table(mid, inst):
    assert len(inst) == len(REF_TABLE)
    for (i1, i2, io, pw), (ri1, ri2, rio, dims, rpw) in zip(inst, REF_TABLE):
        assert (i1, i2, io) == (ri1, ri2, rio)
        assert (IN1[i1].ir.dim, SH[i2].ir.dim, mid[io].ir.dim) == dims
        assert abs(pw - rpw) < 5e-5
    # uvu with one weight per (instruction, channel): weight_numel = n_instr * 128
    assert sum(IN1[i1].mul * SH[i2].mul for i1, i2, _, _ in inst) == 1280
    assert mid.dim == 5120
    # scalar group (l1 = 0) output components K0 and l1 = 1 group K1
    assert sum(mid[io].ir.dim for i1, _, io, _ in inst if i1 == 0) == 16
    assert sum(mid[io].ir.dim for i1, _, io, _ in inst if i1 == 1) == 24
    assert sum(SH[i2].ir.dim * mid[io].ir.dim for i1, i2, io, _ in inst if i1 == 1) == 106


def test_convtp_table_oracle():
    mid, inst = om.conv_tp_instructions(IN1, SH, TARGET)
    _check_table(mid, inst)
    tp = om.ConvTP(IN1, SH, TARGET)
    assert tp.weight_numel == 1280


def test_convtp_table_product():
    mid, inst = model_io.conv_tp_instructions(IN1, SH, TARGET)
    _check_table(mid, inst)


def test_convtp_table_kernel_generator():
    slots = gen_tables.tp_layout(2)
    assert len(slots) == len(REF_TABLE)
    for slot, (i1, i2, io, dims, pw) in zip(slots, REF_TABLE):
        l1, l2, l3 = slot
        # blocks 0e, 1o of the input and 0e, 1o, 2e, 3o of the SH: index = degree
        assert (l1, l2) == (i1, i2)
        assert (2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1) == dims
        assert abs(gen_tables.tp_path_weight(slot) - pw) < 5e-5
    assert 128 * sum(2 * s[2] + 1 for s in slots) == 5120
    # the one-block layout (layer 0) is the l1 = 0 rows of the same table, in order
    assert gen_tables.tp_layout(1) == [s for s in slots if s[0] == 0]


def test_convtp_large_has_17_instructions():
    """Large layer 1 (`utils.py:118-124` with sources 0e / 1o / 2e): 4 + 6 + 7."""
    big = Irreps("128x0e+128x1o+128x2e")
    for gen in (om.conv_tp_instructions, model_io.conv_tp_instructions):
        mid, inst = gen(big, SH, TARGET)
        assert [sum(1 for t in inst if t[0] == b) for b in range(3)] == [4, 6, 7]
        assert 128 * len(inst) == 2176 and mid.dim == 9088
    slots = gen_tables.tp_layout(3)
    mid, inst = model_io.conv_tp_instructions(big, SH, TARGET)
    assert [(big[i1].ir.l, SH[i2].ir.l, mid[io].ir.l) for i1, i2, io, _ in inst] == slots


def test_linear_known_answer():
    """`tests/test_linear.py:194-226` of the reference."""
    ii, io = Irreps("2x0e+3x0e"), Irreps("1x0e")
    inst = model_io.linear_instructions(ii, io)
    assert [(a, b) for a, b, *_ in inst] == [(0, 0), (1, 0)]
    for t in inst:
        assert abs(t[-1] - 1.0 / math.sqrt(5.0)) < 1e-12
    rng = np.random.default_rng(0)
    w0, w1 = rng.normal(size=(2, 1)), rng.normal(size=(3, 1))
    lin = om.Linear(ii, io, [torch.tensor(w0), torch.tensor(w1)])
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0, 5.0]], dtype=torch.float64)
    y = lin(x).numpy()
    pw = 1.0 / math.sqrt(5.0)
    want = pw * (np.array([1.0, 2.0]) @ w0) + pw * (np.array([3.0, 4.0, 5.0]) @ w1)
    np.testing.assert_allclose(y[0], want, atol=1e-12)


# ---------------------------------------------------------------------------
# second moments
# ---------------------------------------------------------------------------

def _unit_sh(n, lmax, seed):
    v = torch.as_tensor(np.random.default_rng(seed).normal(size=(n, 3)))
    return om.spherical_harmonics(v, lmax)


def _moments(y, irreps):
    """Mean square per output block (averaged over samples, channels, components).
    Shared weight matrices make each block's moment a chi-square over its K x M
    weights; the multiplicities below keep that spread near 2-3 %."""
    out = []
    for b, off in zip(irreps, irreps.offsets):
        out.append(float((y[:, off:off + b.dim] ** 2).mean()))
    return np.array(out)


@pytest.mark.parametrize("spec_in,spec_out", [
    ("48x0e+32x0e+40x1o+24x1o+64x2e", "64x0e+48x1o+56x2e"),
    ("128x0e+128x1o", "128x0e+128x1o"),
])
def test_linear_unit_second_moment(spec_in, spec_out):
    ii, io = Irreps(spec_in), Irreps(spec_out)
    g = torch.Generator().manual_seed(1)
    ws = [torch.randn(a[2], a[3], generator=g, dtype=torch.float64)
          for a in model_io.linear_instructions(ii, io)]
    lin = om.Linear(ii, io, ws)
    x = torch.randn(4000, ii.dim, generator=g, dtype=torch.float64)
    m = _moments(lin(x), io)
    np.testing.assert_allclose(m, 1.0, rtol=0.06)


def test_fctp_unit_second_moment():
    """FCTP (uvw) with a generic second input: every output block has unit moment."""
    i1, n2 = Irreps("40x0e+32x1o+24x2e"), 5
    io = Irreps("48x0e+40x1o+32x2e")
    inst = model_io.fctp_instructions(i1, Irreps(f"{n2}x0e"), io)
    g = torch.Generator().manual_seed(2)
    ws = [torch.randn(i1[i].mul, n2, io[k].mul, generator=g, dtype=torch.float64)
          for i, _, k, _ in inst]
    fc = om.SkipFCTP(i1, n2, io, ws)
    x1 = torch.randn(6000, i1.dim, generator=g, dtype=torch.float64)
    x2 = torch.randn(6000, n2, generator=g, dtype=torch.float64)
    m = _moments(fc(x1, x2), io)
    np.testing.assert_allclose(m, 1.0, rtol=0.06)


@pytest.mark.parametrize("spec_in", ["32x0e", "32x0e+32x1o", "32x0e+32x1o+32x2e"])
def test_convtp_unit_second_moment(spec_in):
    """uvu conv TP: x ~ N(0,1), Y component-normalised over random directions,
    w ~ N(0,1) -> every output slot has unit second moment."""
    i1 = Irreps(spec_in)
    tgt = Irreps("32x0e+32x1o+32x2e+32x3o")
    tp = om.ConvTP(i1, SH, tgt)
    n = 6000
    g = torch.Generator().manual_seed(3)
    x1 = torch.randn(n, i1.dim, generator=g, dtype=torch.float64)
    Y = _unit_sh(n, 3, 4)
    w = torch.randn(n, tp.weight_numel, generator=g, dtype=torch.float64)
    m = _moments(tp(x1, Y, w), tp.mid)
    np.testing.assert_allclose(m, 1.0, rtol=0.07)
