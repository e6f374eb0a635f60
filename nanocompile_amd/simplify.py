"""Integer index arithmetic of loop IR: affine forms, value ranges, and removable divisions.

A schedule that re-lays an operand (``pack``) writes each read as
``(flat / cols / block) * cols * block + (flat % cols) * block + ...``; once the
loop ranges are known most of those divisions are provably exact or provably
within one period, and disappear. This is the job the reference's
simplify.py does for its schedules (simplify.py:127-139, 172-186); this
module does it its own way:

* an index is read as an affine form, ``sum(coeff * atom) + const``, where an
  atom is a loop variable, a symbol, or any sub-expression that is not
  affine (a product of two variables, a division that cannot be removed);
* each loop variable ranges over ``[0, extent - 1]``; a symbol over
  ``[0, inf)``; an atom's range follows from its parts;
* ``a / c`` and ``a % c`` for a constant ``c > 0`` split ``a`` into the terms
  with coefficients divisible by ``c`` and the rest ``r``; when ``r`` is
  provably in ``[0, c)`` the division is those terms' coefficients over ``c``
  and the remainder is ``r``.

Only integer index expressions are touched; float arithmetic never is.
"""

from __future__ import annotations

from nanocompile_amd import lir

I64 = lir.DType("i64")
INF = float("inf")


def kind(x) -> str:
    return type(x).__name__


def _key(x) -> str:
    return repr(x)


class Affine:
    """``const + sum(coeff * atom)``, atoms keyed by their repr."""

    __slots__ = ("const", "terms", "atoms")

    def __init__(self, const: int = 0, terms=None, atoms=None) -> None:
        self.const = const
        self.terms: dict[str, int] = dict(terms or {})
        self.atoms: dict[str, object] = dict(atoms or {})

    def plus(self, other: "Affine", sign: int = 1) -> "Affine":
        out = Affine(self.const + sign * other.const, self.terms, self.atoms)
        for k, c in other.terms.items():
            out.terms[k] = out.terms.get(k, 0) + sign * c
            out.atoms[k] = other.atoms[k]
            if out.terms[k] == 0:
                del out.terms[k]
        return out

    def scaled(self, c: int) -> "Affine":
        if c == 0:
            return Affine()
        return Affine(self.const * c, {k: v * c for k, v in self.terms.items()}, self.atoms)


def _is_int(x) -> bool:
    return getattr(x, "dtype", I64).is_int if hasattr(getattr(x, "dtype", None), "is_int") else True


def affine(x) -> Affine:
    k = kind(x)
    if k == "Const" and isinstance(x.value, int):
        return Affine(int(x.value))
    if k == "Binary" and x.dtype.is_int and x.op in ("add", "sub"):
        return affine(x.a).plus(affine(x.b), 1 if x.op == "add" else -1)
    if k == "Binary" and x.dtype.is_int and x.op == "mul":
        a, b = affine(x.a), affine(x.b)
        if not a.terms:
            return b.scaled(a.const)
        if not b.terms:
            return a.scaled(b.const)
    if k == "Cast" and x.dtype.is_int and kind(x.a) in ("Var", "Sym"):
        return affine(x.a)
    return Affine(0, {_key(x): 1}, {_key(x): x})


def coefficient(index, var: str):
    """The coefficient of loop variable ``var`` in ``index`` if it appears only linearly, else None."""
    a = affine(index)
    total = 0
    for k, c in a.terms.items():
        atom = a.atoms[k]
        if kind(atom) == "Var" and atom.name == var:
            total += c
        elif _mentions(atom, var):
            return None
    return total


def _mentions(x, var: str) -> bool:
    from nanocompile_amd.gpu_schedule import uses_var
    return uses_var(x, var)


def value_range(x, ranges: dict[str, tuple]) -> tuple:
    """[lo, hi] of an integer expression (either may be +-inf when unknown)."""
    k = kind(x)
    if k == "Const":
        v = x.value
        return (v, v) if isinstance(v, int) else (-INF, INF)
    if k == "Var":
        return ranges.get(x.name, (-INF, INF))
    if k == "Sym":
        return (0, INF)
    if k == "Cast" and x.dtype.is_int and kind(x.a) in ("Var", "Sym", "Binary", "Const"):
        return value_range(x.a, ranges) if getattr(x.a, "dtype", I64).is_int else (-INF, INF)
    if k == "Binary" and x.dtype.is_int:
        a, b = value_range(x.a, ranges), value_range(x.b, ranges)
        if x.op == "add":
            return (a[0] + b[0], a[1] + b[1])
        if x.op == "sub":
            return (a[0] - b[1], a[1] - b[0])
        if x.op == "mul":
            products = [_mul(p, q) for p in a for q in b]
            return (min(products), max(products))
        if x.op in ("idiv", "mod") and b[0] == b[1] and isinstance(b[0], int) and b[0] > 0 and a[0] >= 0:
            c = b[0]
            if x.op == "idiv":
                return (a[0] // c, a[1] // c if a[1] != INF else INF)
            return (0, min(c - 1, a[1]))
    return (-INF, INF)


def _mul(p, q):
    if p == 0 or q == 0:
        return 0
    return p * q


def _const(v: int):
    return lir.Const(int(v), I64)


def _build(a: Affine):
    """An expression for an affine form (terms in a fixed order, then the constant)."""
    out = None
    for key in sorted(a.terms):
        c, atom = a.terms[key], a.atoms[key]
        term = atom if c == 1 else lir.Binary("mul", atom, _const(c), I64)
        out = term if out is None else lir.Binary("add", out, term, I64)
    if out is None:
        return _const(a.const)
    if a.const:
        out = lir.Binary("add", out, _const(a.const), I64)
    return out


def expression(a: Affine):
    """An integer expression with the value of the affine form ``a``."""
    return _build(a)


def _range_of_affine(a: Affine, ranges) -> tuple:
    lo = hi = a.const
    for key, c in a.terms.items():
        r = value_range(a.atoms[key], ranges)
        ends = (_mul(c, r[0]), _mul(c, r[1]))
        lo, hi = lo + min(ends), hi + max(ends)
    return lo, hi


def simplify(x, ranges: dict[str, tuple]):
    """``x`` with provable integer divisions and remainders removed (recursively)."""
    k = kind(x)
    if k == "Load":
        return lir.Load(x.param, simplify(x.index, ranges), x.dtype)
    if k == "Local":
        return lir.Local(x.name, simplify(x.index, ranges), x.dtype)
    if k == "Unary":
        return lir.Unary(x.op, simplify(x.a, ranges), x.dtype)
    if k == "Cast":
        return lir.Cast(simplify(x.a, ranges), x.dtype)
    if k == "Select":
        return lir.Select(simplify(x.cond, ranges), simplify(x.a, ranges), simplify(x.b, ranges), x.dtype)
    if k == "Fma":
        return lir.Fma(simplify(x.a, ranges), simplify(x.b, ranges), simplify(x.c, ranges), x.dtype)
    if k == "Dp4":
        return lir.Dp4(simplify(x.a, ranges), simplify(x.b, ranges), x.dtype)
    if k != "Binary":
        return x
    a, b = simplify(x.a, ranges), simplify(x.b, ranges)
    x = lir.Binary(x.op, a, b, x.dtype)
    if not x.dtype.is_int or x.op not in ("idiv", "mod"):
        return x
    if not (kind(b) == "Const" and isinstance(b.value, int) and b.value > 0):
        return x
    c = int(b.value)
    if c == 1:
        return _const(0) if x.op == "mod" else a
    form = affine(a)
    whole = Affine(form.const - form.const % c)
    rest = Affine(form.const % c)
    for key, coeff in form.terms.items():
        part = Affine(0, {key: coeff}, {key: form.atoms[key]})
        if coeff % c == 0:
            whole = whole.plus(part)
        else:
            rest = rest.plus(part)
    lo, hi = _range_of_affine(rest, ranges)
    if lo >= 0 and hi < c:
        if x.op == "mod":
            return _build(rest)
        quotient = Affine(whole.const // c, {key: v // c for key, v in whole.terms.items()}, whole.atoms)
        return _build(quotient)
    return x


def simplify_body(stmts, ranges: dict[str, tuple] | None = None) -> tuple:
    """Every index in ``stmts`` simplified with the ranges of the loops around it."""
    ranges = dict(ranges or {})
    out = []
    for s in stmts:
        k = kind(s)
        if k == "Loop":
            extent = simplify(s.extent, ranges)
            lo_hi = value_range(extent, ranges)
            inner = dict(ranges)
            inner[s.var] = (0, lo_hi[1] - 1 if lo_hi[1] != INF else INF)
            out.append(lir.Loop(s.var, extent, simplify_body(s.body, inner), s.kind))
        elif k == "Block":
            out.append(lir.Block(simplify_body(s.body, ranges)))
        elif k == "Store":
            out.append(lir.Store(s.param, simplify(s.index, ranges), simplify(s.value, ranges)))
        elif k == "Let":
            out.append(lir.Let(s.var, simplify(s.value, ranges)))
        elif k == "Assign":
            out.append(lir.Assign(s.var, simplify(s.value, ranges)))
        elif k == "Fail":
            out.append(lir.Fail(simplify(s.cond, ranges), s.code))
        elif k == "ArrayStore":
            out.append(lir.ArrayStore(s.name, simplify(s.index, ranges), simplify(s.value, ranges)))
        else:
            out.append(s)
    return tuple(out)
