"""O(3) irrep bookkeeping for the host-side constant builders.

Feature layout convention (the same one the reference uses, `irreps.py:100-329`
and `linear.py:434-439`): a flat feature row is the concatenation of blocks
``mul x (l, p)``; inside a block the element ``(u, m)`` sits at ``u * (2l+1) + m``
("mul-major").  Nothing here touches device memory: the classes are only used to
derive offsets, instruction lists and normalisation constants that the HIP
library receives as plain integer/float tables.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from typing import Iterable, Iterator, List, Sequence, Tuple, Union

_IRREP_RE = re.compile(r"^\s*(\d+)\s*([eoy])\s*$")


@dataclass(frozen=True, order=False)
class Irrep:
    """A single irrep ``(l, p)``; ``p`` is +1 (``e``) or -1 (``o``)."""

    l: int
    p: int

    def __post_init__(self):
        if not isinstance(self.l, int) or self.l < 0:
            raise ValueError(f"l must be a non-negative int, got {self.l!r}")
        if self.p not in (1, -1):
            raise ValueError(f"p must be +1 or -1, got {self.p!r}")

    @staticmethod
    def parse(spec: Union[str, "Irrep", Tuple[int, int]]) -> "Irrep":
        if isinstance(spec, Irrep):
            return spec
        if isinstance(spec, tuple):
            return Irrep(int(spec[0]), int(spec[1]))
        m = _IRREP_RE.match(spec)
        if m is None:
            raise ValueError(f"Cannot parse irrep string: {spec!r}")
        l = int(m.group(1))
        c = m.group(2)
        p = 1 if c == "e" else -1 if c == "o" else (-1) ** l
        return Irrep(l, p)

    @property
    def dim(self) -> int:
        return 2 * self.l + 1

    def sort_key(self) -> Tuple[int, int]:
        # Ordering used by Irreps.sort in the reference (irreps.py:196-205):
        # by l, then by p with odd (-1) before even (+1).
        return (self.l, self.p)

    def couple(self, other: "Irrep") -> List["Irrep"]:
        """All irreps in self (x) other: |l1-l2| <= l <= l1+l2, p = p1*p2."""
        p = self.p * other.p
        return [Irrep(l, p) for l in range(abs(self.l - other.l), self.l + other.l + 1)]

    def __str__(self) -> str:
        return f"{self.l}{'e' if self.p == 1 else 'o'}"

    __repr__ = __str__


@dataclass(frozen=True)
class MulIrrep:
    mul: int
    ir: Irrep

    @property
    def dim(self) -> int:
        return self.mul * self.ir.dim

    def __iter__(self):  # allow ``mul, ir = block``
        yield self.mul
        yield self.ir


class Irreps:
    """Ordered direct sum of ``mul x irrep`` blocks (e3nn string format)."""

    def __init__(self, spec: Union[str, "Irreps", Sequence, None] = None):
        if spec is None:
            self.blocks: Tuple[MulIrrep, ...] = ()
        elif isinstance(spec, Irreps):
            self.blocks = spec.blocks
        elif isinstance(spec, str):
            self.blocks = tuple(self._parse(spec))
        else:
            out = []
            for item in spec:
                if isinstance(item, MulIrrep):
                    out.append(item)
                elif isinstance(item, Irrep):
                    out.append(MulIrrep(1, item))
                elif isinstance(item, str):
                    out.extend(self._parse(item))
                else:
                    mul, ir = item
                    out.append(MulIrrep(int(mul), Irrep.parse(ir)))
            self.blocks = tuple(out)

    @staticmethod
    def _parse(s: str) -> Iterator[MulIrrep]:
        for part in s.split("+"):
            part = part.strip()
            if not part:
                continue
            if "x" in part:
                mul, ir = part.split("x", 1)
                yield MulIrrep(int(mul), Irrep.parse(ir))
            else:
                yield MulIrrep(1, Irrep.parse(part))

    @staticmethod
    def spherical_harmonics(lmax: int) -> "Irreps":
        return Irreps([(1, Irrep(l, (-1) ** l)) for l in range(lmax + 1)])

    # --- sizes and offsets -------------------------------------------------
    @property
    def dim(self) -> int:
        return sum(b.dim for b in self.blocks)

    @property
    def offsets(self) -> List[int]:
        out, off = [], 0
        for b in self.blocks:
            out.append(off)
            off += b.dim
        return out

    @property
    def lmax(self) -> int:
        return max(b.ir.l for b in self.blocks)

    def count(self, ir: Union[str, Irrep]) -> int:
        ir = Irrep.parse(ir)
        return sum(b.mul for b in self.blocks if b.ir == ir)

    def sorted_with_perm(self) -> Tuple["Irreps", Tuple[int, ...], Tuple[int, ...]]:
        """Stable sort by (l, p).  Returns (sorted, p, inv) with
        ``sorted.blocks[k] == self.blocks[p[k]]`` and ``inv[p[k]] == k``."""
        order = sorted(range(len(self.blocks)), key=lambda i: self.blocks[i].ir.sort_key())
        inv = [0] * len(order)
        for k, i in enumerate(order):
            inv[i] = k
        return Irreps([self.blocks[i] for i in order]), tuple(order), tuple(inv)

    def simplify(self) -> "Irreps":
        """Adjacent blocks of the same irrep merged (e3nn ``Irreps.simplify``); the flat
        feature layout is unchanged, since each block is mul-major."""
        out: List[MulIrrep] = []
        for b in self.blocks:
            if out and out[-1].ir == b.ir:
                out[-1] = MulIrrep(out[-1].mul + b.mul, b.ir)
            elif b.mul > 0:
                out.append(b)
        return Irreps(out)

    def __iter__(self):
        return iter(self.blocks)

    def __len__(self) -> int:
        return len(self.blocks)

    def __getitem__(self, i) -> MulIrrep:
        return self.blocks[i]

    def __contains__(self, ir) -> bool:
        ir = Irrep.parse(ir)
        return any(b.ir == ir for b in self.blocks)

    def __eq__(self, other) -> bool:
        if isinstance(other, str):
            other = Irreps(other)
        return isinstance(other, Irreps) and self.blocks == other.blocks

    def __hash__(self) -> int:
        return hash(self.blocks)

    def __add__(self, other) -> "Irreps":
        return Irreps(list(self.blocks) + list(Irreps(other).blocks))

    def __str__(self) -> str:
        return " + ".join(f"{b.mul}x{b.ir}" if b.mul != 1 else f"{b.ir}" for b in self.blocks)

    __repr__ = __str__


def scalar_part(irreps: Irreps) -> Irreps:
    return Irreps([b for b in irreps if b.ir.l == 0])


def iter_blocks(irreps: Irreps) -> Iterable[Tuple[int, int, Irrep, int]]:
    """Yield (index, offset, irrep, mul) for each block."""
    for i, (b, off) in enumerate(zip(irreps.blocks, irreps.offsets)):
        yield i, off, b.ir, b.mul
