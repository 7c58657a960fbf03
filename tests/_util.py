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


def nd_mlp_gg(seed=0, dtype=torch.float64, device='cpu', out_nd=True):
    """An fc in the N-D batched MatMul form (ONNX MatMul on a (3, 7) input,
    W (16, 7): output (3, 16)), relu, flatten, fc 48 -> 6, relu, fc 6 -> 3.
    ``out_nd`` False drops the first fc's out_shape_nd."""
    g = torch.Generator().manual_seed(seed)
    W0 = torch.randn(16, 7, generator=g, dtype=torch.float64) * (2 / 7) ** 0.5
    b0 = torch.randn(16, generator=g, dtype=torch.float64) * 0.1
    W1 = torch.randn(6, 48, generator=g, dtype=torch.float64) * (2 / 48) ** 0.5
    b1 = torch.randn(6, generator=g, dtype=torch.float64) * 0.1
    W2 = torch.randn(3, 6, generator=g, dtype=torch.float64) * (2 / 6) ** 0.5
    b2 = torch.randn(3, generator=g, dtype=torch.float64) * 0.1
    cv = dict(device=device, dtype=dtype)
    fc0 = {'name': 'fc0', 'type': 'fc', 'inputs': ['input'], 'W': W0.to(**cv),
           'bias': b0.to(**cv), 'in_shapes_nd': [(3, 7)]}
    if out_nd:
        fc0['out_shape_nd'] = (3, 16)
    ops = [fc0,
           {'name': 'relu0', 'type': 'relu', 'inputs': ['fc0'], 'layer_idx': 0},
           {'name': 'flat', 'type': 'reshape', 'inputs': ['relu0']},
           {'name': 'fc1', 'type': 'fc', 'inputs': ['flat'], 'W': W1.to(**cv),
            'bias': b1.to(**cv)},
           {'name': 'relu1', 'type': 'relu', 'inputs': ['fc1'], 'layer_idx': 1},
           {'name': 'fc2', 'type': 'fc', 'inputs': ['relu1'], 'W': W2.to(**cv),
            'bias': b2.to(**cv)}]
    return {'ops': ops, 'relu_names': ['relu0', 'relu1'], 'fork_points': set(),
            'n_relu': 2, 'input_name': 'input', 'input_n': 21, 'input_shape': (1, 3, 7)}


def nd_as_block_diag(gg):
    """The same net with the N-D fc written as a plain fc of the
    block-diagonal kron(I_3, W0) and bias repeated 3 times."""
    import copy
    out = copy.copy(gg)
    ops = [dict(op) for op in gg['ops']]
    W0, b0 = ops[0]['W'], ops[0]['bias']
    ops[0] = {'name': 'fc0', 'type': 'fc', 'inputs': ['input'],
              'W': torch.block_diag(W0, W0, W0), 'bias': b0.repeat(3)}
    out['ops'] = ops
    return out
