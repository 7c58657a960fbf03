"""Shared helpers for the test suite (not collected)."""
import numpy as np
import torch

from vibecheck_amd import workloads as wk
from vibecheck_amd.spec import dedup_queries


def tiny_mlp(widths, seed, dtype=torch.float64, bias_std=0.1, device='cpu'):
    Ws, bs = wk.mlp_params(widths, seed=seed, bias_std=bias_std)
    return wk.mlp_gg(Ws, bs, device=device, dtype=dtype)


def tiny_cnn(seed=0, dtype=torch.float64, device='cpu'):
    """Conv(2->3, 3x3, p1) - relu - Conv(3->2, 3x3, s2) - relu - flatten -
    fc 18->4 - relu - fc 4->2 on 2x6x6 inputs."""
    return wk.cnn_gg([(3, 3, 1, 1), (2, 3, 2, 0)], [4, 2], (2, 6, 6),
                     seed=seed, device=device, dtype=dtype)


def sample_box(xl, xh, n, seed=0):
    """n uniform points per box: (B, n, d)."""
    g = torch.Generator().manual_seed(seed)
    t = torch.rand(xl.shape[0], n, xl.shape[1], generator=g, dtype=xl.dtype)
    return xl.unsqueeze(1) + t * (xh - xl).unsqueeze(1)


def spec_for(n_out, one_disjunct=True, dtype=torch.float64):
    """spec_ew / disj_q_idx for rows y0 - yi (i = 1..n_out-1)."""
    spec = wk.pairwise_spec(n_out, [0.0], [0.0], one_disjunct)
    uq, dq = dedup_queries(spec.as_linear_queries(n_out))
    spec_ew = {i: (torch.tensor(w, dtype=dtype), b) for i, (w, b) in enumerate(uq)}
    return spec_ew, dq


def to_dev(gg, device, dtype=torch.float32):
    """Copy of a gg dict with tensors moved to device/dtype."""
    ops = []
    for op in gg['ops']:
        o = {}
        for k, v in op.items():
            if k.startswith('_'):
                continue
            o[k] = v.to(device=device, dtype=dtype) if torch.is_tensor(v) else v
        ops.append(o)
    out = dict(gg)
    out['ops'] = ops
    return out


def rel_err_ok(a, b, rtol=1e-5, atol=1e-6):
    """Boolean mask of entries within |a-b| <= atol + rtol*|b|."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return (a - b).abs() <= atol + rtol * b.abs()


def clip_tolerance(A, acc, xl, xh, rtol=1e-5, atol=1e-6):
    """Per (row, dimension) tolerance of a clipped box coordinate: the clip
    threshold (-b_q - sum_{j != i} A_qj x_j) / A_qi carries the rounding of
    its numerator, atol + rtol (|b_q| + sum_j |A_qj| max(|xl_j|, |xh_j|)),
    divided by |A_qi|; the largest over the halfspaces that can cut
    dimension i (|A_qi| > 1e-12), capped by the box width, plus the plain
    tolerance of the coordinate.  A (R, Q, n), acc (R, Q), xl, xh (R, n):
    the rows' halfspaces and unclipped boxes."""
    A, acc, xl, xh = (t.detach().double().cpu() for t in (A, acc, xl, xh))
    xm = torch.maximum(xl.abs(), xh.abs())
    scale = acc.abs() + (A.abs() * xm.unsqueeze(1)).sum(-1)
    cut = A.abs() > 1e-12
    per = torch.where(cut, (atol + rtol * scale).unsqueeze(-1) / A.abs().clamp(min=1e-30),
                      torch.zeros_like(A))
    return torch.minimum(per.amax(1), xh - xl) + atol + rtol * xm
