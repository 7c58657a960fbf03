"""VNNLIB reader: a property file -> ``VNNSpec`` (the unsafe region in DNF).

Reads both forms VNN-COMP uses:
  - version 1: ``(declare-const X_3 Real)``, variables ``X_i`` / ``Y_i``;
  - version 2: ``(declare-network N (declare-input X float32 [1, 1, 1, 5])
    (declare-output Y float32 [1, 5]))``, variables ``X[0,0,0,3]``, flat
    index row-major over the declared shape.
Assertions are conjoined; ``and`` / ``or`` nest and are expanded to DNF.
Atoms are ``(<= a b)``, ``(>= a b)``, ``(< a b)``, ``(> a b)`` over linear
terms (numbers, variables, ``+``, ``-``, ``*`` by a number).

Each DNF clause becomes one disjunct, mapped the way the reference maps its
parsed properties onto its spec types (vnnlib_loader.py:806-948):
  - a bound on one input variable narrows that clause's input box;
  - ``c Y_i + k <= 0`` is ``Y_i <= -k/c`` (c > 0) or ``Y_i >= -k/c``
    (c < 0): a threshold Constraint;
  - ``c (Y_a - Y_b) <= 0`` (no constant) is PairwiseConstraint(pred=a,
    comp=b): unsafe when Y_b >= Y_a;
  - strictness is dropped (closing the unsafe region is sound);
  - anything else raises NotImplementedError.
The global box is the union of the clause boxes (missing bounds 0); the
clauses carry their own box only when the boxes differ between clauses.
"""
import re

import numpy as np

from .spec import Conjunct, Constraint, PairwiseConstraint, VNNSpec


def _tokens(text):
    text = re.sub(r';[^\n]*', ' ', text)
    out = []
    i, n = 0, len(text)
    while i < n:
        c = text[i]
        if c.isspace():
            i += 1
        elif c in '()':
            out.append(c)
            i += 1
        else:
            j = i
            depth = 0
            while j < n and (depth > 0 or not (text[j].isspace() or text[j] in '()')):
                if text[j] == '[':
                    depth += 1
                elif text[j] == ']':
                    depth -= 1
                j += 1
            out.append(text[i:j])
            i = j
    return out


def _sexprs(tokens):
    stack, cur = [], []
    for t in tokens:
        if t == '(':
            stack.append(cur)
            cur = []
        elif t == ')':
            if not stack:
                raise ValueError('vnnlib: unbalanced )')
            done, cur = cur, stack.pop()
            cur.append(done)
        else:
            cur.append(t)
    if stack:
        raise ValueError('vnnlib: unbalanced (')
    return cur


def _shape(tok):
    inner = tok.replace(' ', '').strip('[]')
    return [int(x) for x in inner.split(',') if x]


class _Vars:
    def __init__(self):
        self.kind = {}    # declared tensor name -> 'X' | 'Y'
        self.shape = {}
        self.n = {'X': 0, 'Y': 0}

    def declare(self, name, kind, shape):
        self.kind[name] = kind
        self.shape[name] = shape
        self.n[kind] = max(self.n[kind], int(np.prod(shape)) if shape else 1)

    def resolve(self, tok):
        """'X_3' / 'X[0,0,0,3]' -> ('X', 3); None if not a variable."""
        m = re.fullmatch(r'([A-Za-z_][A-Za-z0-9_]*)\[([0-9, ]+)\]', tok)
        if m:
            name = m.group(1)
            if name not in self.kind:
                raise ValueError(f'vnnlib: undeclared tensor {name!r}')
            idx = [int(x) for x in m.group(2).replace(' ', '').split(',')]
            shp = self.shape[name]
            if len(idx) != len(shp) or any(not 0 <= i < s for i, s in zip(idx, shp)):
                raise ValueError(f'vnnlib: index {tok!r} outside shape {shp}')
            return self.kind[name], int(np.ravel_multi_index(idx, shp))
        m = re.fullmatch(r'([XY])_([0-9]+)', tok)
        if m:
            i = int(m.group(2))
            self.n[m.group(1)] = max(self.n[m.group(1)], i + 1)
            return m.group(1), i
        return None


def _linear(e, vs):
    """Term -> ({(kind, i): coeff}, constant)."""
    if isinstance(e, str):
        v = vs.resolve(e)
        if v is not None:
            return {v: 1.0}, 0.0
        return {}, float(e)
    op, args = e[0], [_linear(a, vs) for a in e[1:]]
    if op == '+' or (op == '-' and len(args) > 1):
        coef, k = dict(args[0][0]), args[0][1]
        sg = 1.0 if op == '+' else -1.0
        for c2, k2 in args[1:]:
            for v, c in c2.items():
                coef[v] = coef.get(v, 0.0) + sg * c
            k += sg * k2
        return coef, k
    if op == '-':
        return {v: -c for v, c in args[0][0].items()}, -args[0][1]
    if op == '*':
        k, coef, kvar = 1.0, None, 0.0
        for c2, k2 in args:
            if c2:
                if coef is not None:
                    raise NotImplementedError('vnnlib: nonlinear term')
                coef, kvar = c2, k2
            else:
                k *= k2
        if coef is None:
            return {}, k
        return {v: c * k for v, c in coef.items()}, kvar * k
    raise NotImplementedError(f'vnnlib: unsupported term operator {op!r}')


def _dnf(e, vs):
    """Formula -> list of clauses, each a list of atoms (coeffs, const)
    meaning sum coeff v + const <= 0."""
    if isinstance(e, str) or not e:
        raise ValueError(f'vnnlib: not a formula: {e!r}')
    op = e[0]
    if op == 'and':
        out = [[]]
        for a in e[1:]:
            out = [c + d for c in out for d in _dnf(a, vs)]
        return out
    if op == 'or':
        return [c for a in e[1:] for c in _dnf(a, vs)]
    if op in ('<=', '<', '>=', '>'):
        if len(e) != 3:
            raise NotImplementedError('vnnlib: chained comparison')
        (cl, kl), (cr, kr) = _linear(e[1], vs), _linear(e[2], vs)
        sg = 1.0 if op in ('<=', '<') else -1.0  # lhs - rhs <= 0, or rhs - lhs <= 0
        coef = dict((v, sg * c) for v, c in cl.items())
        for v, c in cr.items():
            coef[v] = coef.get(v, 0.0) - sg * c
        coef = {v: c for v, c in coef.items() if c != 0.0}
        return [[(coef, sg * (kl - kr))]]
    raise NotImplementedError(f'vnnlib: unsupported connective {op!r}')


def _zero(v):
    return 0.0 if v == 0.0 else float(v)


def _clause(atoms):
    box, ycons = {}, []
    for coef, k in atoms:
        kinds = {v[0] for v in coef}
        if kinds == {'X'} and len(coef) == 1:
            (_, i), c = next(iter(coef.items()))
            bound = _zero(-k / c)
            lo, hi = box.get(i, (None, None))
            if c > 0:
                hi = bound if hi is None else min(hi, bound)
            else:
                lo = bound if lo is None else max(lo, bound)
            box[i] = (lo, hi)
        elif kinds == {'Y'} and len(coef) == 1:
            (_, i), c = next(iter(coef.items()))
            ycons.append(Constraint(i, '<=' if c > 0 else '>=', _zero(-k / c)))
        elif kinds == {'Y'} and len(coef) == 2 and k == 0.0:
            (va, ca), (vb, cb) = sorted(coef.items(), key=lambda t: t[0][1])
            if ca * cb < 0 and abs(abs(ca) - abs(cb)) <= 1e-9 * max(abs(ca), abs(cb)):
                pred, comp = (va[1], vb[1]) if ca > 0 else (vb[1], va[1])
                ycons.append(PairwiseConstraint(pred=pred, comp=comp))
            else:
                raise NotImplementedError(f'vnnlib: output constraint {coef} not pairwise')
        else:
            raise NotImplementedError(f'vnnlib: constraint {coef} + {k} <= 0 not supported')
    return box, ycons


def parse_vnnlib(text, dtype=np.float32):
    """VNNSpec of a VNNLIB property (see the module docstring)."""
    vs = _Vars()
    asserts = []
    for s in _sexprs(_tokens(text)):
        if not isinstance(s, list) or not s:
            raise ValueError(f'vnnlib: unexpected top-level token {s!r}')
        if s[0] == 'declare-const':
            vs.resolve(s[1])
        elif s[0] == 'declare-network':
            for item in s[2:]:
                if item[0] in ('declare-input', 'declare-output'):
                    vs.declare(item[1], 'X' if item[0] == 'declare-input' else 'Y',
                               _shape(item[3]) if len(item) > 3 else [])
        elif s[0] == 'assert':
            asserts.append(s[1])
        elif s[0] in ('vnnlib-version', 'set-logic', 'check-sat', 'get-model'):
            continue
        else:
            raise NotImplementedError(f'vnnlib: unsupported statement {s[0]!r}')
    clauses = [[]]
    for a in asserts:
        clauses = [c + d for c in clauses for d in _dnf(a, vs)]
    parsed = [_clause(c) for c in clauses]
    n_in = vs.n['X']
    union = {}
    for box, _ in parsed:
        for i, (lo, hi) in box.items():
            ulo, uhi = union.get(i, (None, None))
            if lo is not None:
                ulo = lo if ulo is None else min(ulo, lo)
            if hi is not None:
                uhi = hi if uhi is None else max(uhi, hi)
            union[i] = (ulo, uhi)
    x_lo = np.array([union.get(i, (0, 0))[0] or 0 for i in range(n_in)], dtype=dtype)
    x_hi = np.array([union.get(i, (0, 0))[1] or 0 for i in range(n_in)], dtype=dtype)
    keys = {tuple(sorted(b.items())) for b, _ in parsed}
    per_box = len(parsed) > 1 and len(keys) > 1
    disj = []
    for box, ycons in parsed:
        if not ycons:
            raise ValueError('vnnlib: a disjunct has no output constraint')
        if per_box:
            lo = np.array([box.get(i, (None, None))[0] if box.get(i, (None, None))[0] is not None
                           else x_lo[i] for i in range(n_in)], dtype=dtype)
            hi = np.array([box.get(i, (None, None))[1] if box.get(i, (None, None))[1] is not None
                           else x_hi[i] for i in range(n_in)], dtype=dtype)
            disj.append(Conjunct(ycons, input_lo=lo, input_hi=hi))
        else:
            disj.append(Conjunct(ycons))
    return VNNSpec(x_lo, x_hi, disj)


def load_vnnlib(path, dtype=np.float32):
    with open(path) as f:
        return parse_vnnlib(f.read(), dtype)
