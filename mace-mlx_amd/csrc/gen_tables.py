"""Build step: emit ``gen/tables.h`` for the HIP library from the host constants.

Everything in the generated header is a function of the irreps algebra only
(SH degree lmax = 3, hidden blocks l = 0..2 with parity (-1)^l), not of any model
weights, so the kernels can index registers with compile-time constants:

* SH recursion couplings (`spherical_harmonics.py:31-40`) as sparse term lists;
* conv-TP layouts for LIN = 1, 2, 3 input blocks (`utils.py:87-156` slot order)
  and the path-weighted CG terms of every l1 >= 1 instruction, grouped by output
  column for the x2-first contraction M[i, col] = sum_j Y_j C[i, j, k] pw;
* symmetric-contraction polynomials (`symmetric_contraction.py:124-595`) for
  coupling irreps 0e+1o+2e+3o, outputs 0e / 1o / 2e, correlation 1..3: the U
  tensors symmetrised over the feature monomial f_a f_b f_c and emitted as
  straight-line forward and VJP device functions.

Usage: python gen_tables.py <out_dir>
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from mace_mlx_amd.cg import sh_coupling, u_matrix, wigner_3j  # noqa: E402

LMAX_SH = 3
SH_DIM = (LMAX_SH + 1) ** 2


def f32(x: float) -> str:
    s = repr(float(np.float32(x)))
    if "e" not in s and "." not in s:
        s += ".0"
    return s + "f"


def tp_layout(lin: int):
    """Slots of the conv TP for input blocks l1 = 0..lin-1 (parity (-1)^l1)."""
    created = []
    for l1 in range(lin):
        for l2 in range(LMAX_SH + 1):
            for l3 in range(abs(l1 - l2), l1 + l2 + 1):
                if l3 <= LMAX_SH and (l1 + l2 + l3) % 2 == 0:
                    created.append((l1, l2, l3))
    order = sorted(range(len(created)), key=lambda k: created[k][2])  # stable
    return [created[k] for k in order]


def tp_path_weight(slot) -> float:
    """Path weight of one uvu instruction, `utils.py:143-154`: sqrt(dim_out / alpha)
    with alpha the summed multiplicity of the SH block, which is 1 for every slot
    here (each instruction owns its output slot)."""
    return math.sqrt(2 * slot[2] + 1)


def emit_sh(out):
    out.append("// SH recursion Y_l[k] += Y_{l-1}[i] * Y_1[j] * v  (e3nn basis)")
    for l in (2, 3):
        C = sh_coupling(l)
        terms = [(i, j, k, C[i, j, k]) for i in range(C.shape[0]) for j in range(3)
                 for k in range(C.shape[2]) if abs(C[i, j, k]) > 1e-12]
        out.append(f"constexpr int SH{l}_NT = {len(terms)};")
        out.append(f"constexpr int SH{l}_I[] = {{{', '.join(str(t[0]) for t in terms)}}};")
        out.append(f"constexpr int SH{l}_J[] = {{{', '.join(str(t[1]) for t in terms)}}};")
        out.append(f"constexpr int SH{l}_K[] = {{{', '.join(str(t[2]) for t in terms)}}};")
        out.append(f"constexpr float SH{l}_V[] = {{{', '.join(f32(t[3]) for t in terms)}}};")


def emit_tp(out, lin: int):
    """Emit the layout and M tables of one TP variant; returns {l1: (K, starts, js, vs)}."""
    slots = tp_layout(lin)
    ns = len(slots)
    d = [2 * s[2] + 1 for s in slots]
    acc_off = np.concatenate([[0], np.cumsum(d)]).tolist()
    P = f"TP{lin}"
    out.append(f"// ---- conv TP layout, {lin} input block(s) ----")
    out.append(f"constexpr int {P}_NSLOT = {ns};")
    out.append(f"constexpr int {P}_NACC = {acc_off[-1]};")
    out.append(f"constexpr int {P}_L1[] = {{{', '.join(str(s[0]) for s in slots)}}};")
    out.append(f"constexpr int {P}_L2[] = {{{', '.join(str(s[1]) for s in slots)}}};")
    out.append(f"constexpr int {P}_L3[] = {{{', '.join(str(s[2]) for s in slots)}}};")
    out.append(f"constexpr int {P}_ACC[] = {{{', '.join(str(a) for a in acc_off)}}};")
    # M-table columns per source degree l1 >= 1
    col = {}
    kcount = {}
    for sidx, (l1, l2, l3) in enumerate(slots):
        if l1 == 0:
            continue
        col[sidx] = kcount.get(l1, 0)
        kcount[l1] = kcount.get(l1, 0) + 2 * l3 + 1
    out.append(f"constexpr int {P}_COL[] = {{{', '.join(str(col.get(s, -1)) for s in range(ns))}}};")
    tables = {}
    for l1 in range(1, 3):
        K = kcount.get(l1, 0)
        out.append(f"constexpr int {P}_K{l1} = {K};")
        # entries (i, c) in row-major order i*K + c, each with SH terms (j, val)
        starts, js, vs = [0], [], []
        for i in range(2 * l1 + 1):
            for c in range(K):
                # find slot / k for column c
                for sidx, (a, l2, l3) in enumerate(slots):
                    if a == l1 and col[sidx] <= c < col[sidx] + 2 * l3 + 1:
                        k = c - col[sidx]
                        pw = tp_path_weight(slots[sidx])
                        C = wigner_3j(l1, l2, l3)
                        for j in range(2 * l2 + 1):
                            v = C[i, j, k] * pw
                            if abs(v) > 1e-12:
                                js.append(l2 * l2 + j)
                                vs.append(v)
                        break
                starts.append(len(js))
        if K == 0:
            starts, js, vs = [0], [0], [0.0]
        out.append(f"constexpr int {P}_M{l1}_NE = {(2 * l1 + 1) * K};")
        out.append(f"constexpr int {P}_M{l1}_START[] = {{{', '.join(map(str, starts))}}};")
        out.append(f"constexpr int {P}_M{l1}_J[] = {{{', '.join(map(str, js))}}};")
        out.append(f"constexpr float {P}_M{l1}_V[] = {{{', '.join(f32(v) for v in vs)}}};")
        tables[l1] = (K, starts, js, vs)
    return tables


def sc_poly(lout: int, corr: int):
    """Symmetrised polynomial terms: list over nu of dict {(p, mono, k): coef}."""
    ir = {0: "0e", 1: "1o", 2: "2e"}[lout]
    koff = 0
    terms = []
    ks = []
    for nu in range(corr, 0, -1):
        U = u_matrix("0e+1o+2e+3o", ir, nu)
        if lout == 0:
            U = U[None]
        K = U.shape[-1]
        nz = np.argwhere(np.abs(U) > 1e-12)
        acc = {}
        for t in nz:
            p, k = int(t[0]), int(t[-1])
            mono = tuple(sorted(int(x) for x in t[1:-1]))
            acc[(p, mono, koff + k)] = acc.get((p, mono, koff + k), 0.0) + float(U[tuple(t)])
        terms.extend((key, v) for key, v in acc.items() if abs(v) > 1e-12)
        ks.append(K)
        koff += K
    return terms, ks


def emit_sc(out, lout: int, corr: int):
    terms, ks = sc_poly(lout, corr)
    P = 2 * lout + 1
    KT = sum(ks)
    name = f"sc_l{lout}_c{corr}"
    out.append(f"// symmetric contraction, output l={lout}, correlation {corr}: "
               f"{len(terms)} terms, weights per channel = {KT} ({'+'.join(map(str, ks))})")
    out.append(f"constexpr int SC_L{lout}_C{corr}_KT = {KT};")
    monos = sorted({m for (p, m, k), _ in terms}, key=lambda m: (len(m), m))
    mid = {m: n for n, m in enumerate(monos)}
    by_mono = {}
    for (p, m, k), v in terms:
        by_mono.setdefault(m, []).append((p, k, v))

    def mono_expr(m):
        return "*".join(f"f[{i}]" for i in m)

    # forward
    out.append(f"__device__ __forceinline__ void {name}_fwd(const float* __restrict__ f, "
               f"const float* __restrict__ w, float* __restrict__ o) {{")
    for p in range(P):
        out.append(f"  float o{p} = 0.f;")
    for m in monos:
        out.append(f"  {{ const float t = {mono_expr(m)};")
        per_p = {}
        for p, k, v in by_mono[m]:
            per_p.setdefault(p, []).append((k, v))
        for p, lst in sorted(per_p.items()):
            s = " + ".join(f"{f32(v)}*w[{k}]" for k, v in lst)
            out.append(f"    o{p} = fmaf(t, {s}, o{p});")
        out.append("  }")
    for p in range(P):
        out.append(f"  o[{p}] = o{p};")
    out.append("}")
    # VJP w.r.t. f: g[i] = sum_p go[p] sum_{m,k} coef w[k] d mono / d f_i
    out.append(f"__device__ __forceinline__ void {name}_vjp(const float* __restrict__ f, "
               f"const float* __restrict__ w, const float* __restrict__ go, float* __restrict__ g) {{")
    for i in range(16):
        out.append(f"  float g{i} = 0.f;")
    for m in monos:
        per_p = {}
        for p, k, v in by_mono[m]:
            per_p.setdefault(p, []).append((k, v))
        s = " + ".join(f"go[{p}]*(" + " + ".join(f"{f32(v)}*w[{k}]" for k, v in lst) + ")"
                       for p, lst in sorted(per_p.items()))
        out.append(f"  {{ const float a = {s};")
        for pos in range(len(m)):
            rest = [m[q] for q in range(len(m)) if q != pos]
            fac = "*".join(f"f[{i}]" for i in rest) if rest else "1.f"
            out.append(f"    g{m[pos]} = fmaf(a, {fac}, g{m[pos]});")
        out.append("  }")
    for i in range(16):
        out.append(f"  g[{i}] = g{i};")
    out.append("}")


def main(out_dir: str) -> None:
    od = Path(out_dir)
    od.mkdir(parents=True, exist_ok=True)
    out = ["// Generated by gen_tables.py -- do not edit.", "#pragma once", ""]
    out.append(f"constexpr int SH_DIM = {SH_DIM};")
    emit_sh(out)
    tabs = {lin: emit_tp(out, lin) for lin in (1, 2, 3)}
    # The per-edge M tables are built once (TP3 layout) and shared by every layer,
    # so the l1 = 1 columns must coincide for 2 and 3 input blocks.
    if tabs[2][1] != tabs[3][1]:
        raise RuntimeError("M1 tables differ between 2 and 3 input blocks")
    for lout in (0, 1, 2):
        for corr in (1, 2, 3):
            emit_sc(out, lout, corr)
    text = "\n".join(out) + "\n"
    target = od / "tables.h"
    if not target.exists() or target.read_text() != text:
        target.write_text(text)
    print(f"wrote {target} ({len(out)} lines)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else str(HERE / "gen"))
