"""Output specifications in disjunctive normal form.

Mirrors the reference's spec types (spec.py:13-263): the unsafe region is an
OR of conjuncts, each an AND of output constraints.  The bound engine only
consumes ``VNNSpec.as_linear_queries`` (spec.py:218-249): one linear query
``w . y + b`` per constraint, proven safe when its minimum is > 0.
"""
from dataclasses import dataclass, field

import numpy as np


@dataclass
class Constraint:
    """Threshold constraint ``Y[index] op value`` with op in {'>=', '<='}."""
    index: int
    op: str
    value: float
    strict: bool = False


@dataclass
class PairwiseConstraint:
    """Unsafe when ``Y[comp] >= Y[pred]``."""
    pred: int
    comp: int
    strict: bool = False


@dataclass
class Conjunct:
    constraints: list
    input_lo: 'np.ndarray | None' = None
    input_hi: 'np.ndarray | None' = None


@dataclass
class VNNSpec:
    x_lo: 'np.ndarray'
    x_hi: 'np.ndarray'
    disjuncts: list = field(default_factory=list)

    def __post_init__(self):
        self.x_lo = np.asarray(self.x_lo, dtype=np.float64)
        self.x_hi = np.asarray(self.x_hi, dtype=np.float64)

    def as_linear_queries(self, n_output):
        """List of (disjunct index, w (n_output,) float64, bias).

        Pairwise (pred, comp): w = e_pred - e_comp, b = 0.
        ``Y[i] >= v``: w = -e_i, b = v.  ``Y[i] <= v``: w = e_i, b = -v.
        (spec.py:218-249)
        """
        out = []
        for di, conj in enumerate(self.disjuncts):
            for c in conj.constraints:
                w = np.zeros(n_output, dtype=np.float64)
                if isinstance(c, PairwiseConstraint):
                    w[c.pred] = 1.0
                    w[c.comp] = -1.0
                    out.append((di, w, 0.0))
                elif c.op == '>=':
                    w[c.index] = -1.0
                    out.append((di, w, float(c.value)))
                elif c.op == '<=':
                    w[c.index] = 1.0
                    out.append((di, w, -float(c.value)))
                else:
                    raise ValueError(f'unknown constraint op {c.op!r}')
        return out


def dedup_queries(queries):
    """Deduplicate identical (w, b) halfspaces across disjuncts.

    Returns (unique [(w float64 array, b)], disj_q_idx {disjunct: [positions]})
    keyed on (w bytes, round(b, 12)) in first-seen order
    (verify_graph.py:12647-12682).
    """
    key_pos = {}
    uniq = []
    disj_q_idx = {}
    for di, w, b in queries:
        w = np.asarray(w, dtype=np.float64).reshape(-1)
        key = (w.tobytes(), round(float(b), 12))
        pos = key_pos.get(key)
        if pos is None:
            pos = len(uniq)
            key_pos[key] = pos
            uniq.append((w, float(b)))
        disj_q_idx.setdefault(di, []).append(pos)
    return uniq, disj_q_idx
