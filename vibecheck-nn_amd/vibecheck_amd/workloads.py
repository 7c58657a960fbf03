"""Seeded synthetic networks, input domains and specs for the five workloads.

Every generator draws from its own CPU ``torch.Generator`` so the same seed
gives the same tensors on any host; callers move results to the device.

Networks are returned as ``gg`` dicts with the schema that
``ComputeGraph.gpu_graph`` produces in the reference
(network.py:1707-2910; fc ops at network.py:2001-2007, relu ops at
network.py:2010-2018, conv ops at network.py:1748-1781).

Weights: Kaiming-normal, std = sqrt(2 / fan_in), fan_in = C_in*kH*kW for
conv.  ACAS-shape biases are N(0, 0.01) read as std 0.01; the other nets use
zero biases.
"""
import math

import numpy as np

import torch

from .spec import Conjunct, PairwiseConstraint, VNNSpec

INPUT_NAME = 'X'


def _gen(seed):
    g = torch.Generator(device='cpu')
    g.manual_seed(int(seed))
    return g


def _kaiming(shape, fan_in, g):
    return torch.randn(*shape, generator=g, dtype=torch.float64) * math.sqrt(
        2.0 / fan_in)


def _fc_op(name, inp, W, b, device, dtype):
    return {'name': name, 'type': 'fc', 'inputs': [inp],
            'W': W.to(device=device, dtype=dtype).contiguous(),
            'bias': b.to(device=device, dtype=dtype).contiguous()}


def _finish(ops, n_in, input_shape):
    refs = {}
    for op in ops:
        for i in op['inputs']:
            refs[i] = refs.get(i, 0) + 1
    relu_names = [op['name'] for op in ops if op['type'] == 'relu']
    return {'ops': ops, 'relu_names': relu_names,
            'fork_points': {n for n, c in refs.items() if c > 1},
            'n_relu': len(relu_names), 'input_name': INPUT_NAME,
            'input_n': n_in, 'input_shape': input_shape}


def mlp_gg(weights, biases, device='cpu', dtype=torch.float32):
    """``gg`` for fc -> relu -> ... -> fc from lists of (n_out, n_in) W and b."""
    ops = []
    prev = INPUT_NAME
    for i, (W, b) in enumerate(zip(weights, biases)):
        ops.append(_fc_op(f'fc{i}', prev, W, b, device, dtype))
        prev = f'fc{i}'
        if i < len(weights) - 1:
            ops.append({'name': f'relu{i}', 'type': 'relu', 'inputs': [prev],
                        'layer_idx': i})
            prev = f'relu{i}'
    n_in = int(weights[0].shape[1])
    return _finish(ops, n_in, (1, n_in))


def residual_mlp_gg(n_in, width, n_out, seed=0, device='cpu', dtype=torch.float32,
                    n_blocks=2):
    """A residual ReLU MLP in the op form the reference's ONNX reader emits
    (network.py:1925-2150): input normalisation as sub (mean) then mul
    (1 / std) constants, fc0 -> relu, then ``n_blocks`` blocks
    y = relu(fc_b(relu(fc_a(x))) + x) whose skip is an 'add' with
    is_merge (x is a fork point), a constant 'add' offset and a scalar
    'mul' by -1 before the head's last fc, which ends in a constant 'add'.
    Kaiming-normal weights, biases N(0, 0.1^2), seeded."""
    g = _gen(seed)

    def fc(name, inp, n_o, n_i):
        W = torch.randn(n_o, n_i, generator=g, dtype=torch.float64) * (2.0 / n_i) ** 0.5
        b = torch.randn(n_o, generator=g, dtype=torch.float64) * 0.1
        return _fc_op(name, inp, W.float(), b.float(), device, dtype)

    mean = (torch.rand(n_in, generator=g, dtype=torch.float64) - 0.5).numpy()
    std = (0.5 + torch.rand(n_in, generator=g, dtype=torch.float64)).numpy()
    ops = [{'name': 'norm_sub', 'type': 'sub', 'inputs': [INPUT_NAME], 'bias': mean},
           {'name': 'norm_mul', 'type': 'mul', 'inputs': ['norm_sub'], 'scale': 1.0 / std},
           fc('fc0', 'norm_mul', width, n_in),
           {'name': 'relu0', 'type': 'relu', 'inputs': ['fc0'], 'layer_idx': 0}]
    prev, L = 'relu0', 1
    for k in range(n_blocks):
        ops.append(fc(f'b{k}_fa', prev, width, width))
        ops.append({'name': f'b{k}_ra', 'type': 'relu', 'inputs': [f'b{k}_fa'],
                    'layer_idx': L})
        ops.append(fc(f'b{k}_fb', f'b{k}_ra', width, width))
        ops.append({'name': f'b{k}_add', 'type': 'add', 'inputs': [f'b{k}_fb', prev],
                    'is_merge': True, 'bias': None})
        ops.append({'name': f'b{k}_rb', 'type': 'relu', 'inputs': [f'b{k}_add'],
                    'layer_idx': L + 1})
        prev, L = f'b{k}_rb', L + 2
    off = (torch.rand(width, generator=g, dtype=torch.float64) * 0.2 - 0.1).numpy()
    ops.append({'name': 'head_off', 'type': 'add', 'inputs': [prev], 'is_merge': False,
                'bias': off})
    ops.append({'name': 'head_neg', 'type': 'mul', 'inputs': ['head_off'],
                'scale': np.array([-1.0])})
    ops.append(fc('head', 'head_neg', n_out, width))
    ops.append({'name': 'out', 'type': 'add', 'inputs': ['head'], 'is_merge': False,
                'bias': (torch.rand(n_out, generator=g, dtype=torch.float64) - 0.5).numpy()})
    return _finish(ops, n_in, (1, n_in))


def mlp_params(widths, seed=0, bias_std=0.0):
    """Kaiming-normal fc stack for ``widths`` = [n_in, h1, ..., n_out]."""
    g = _gen(seed)
    Ws, bs = [], []
    for n_in, n_out in zip(widths[:-1], widths[1:]):
        Ws.append(_kaiming((n_out, n_in), n_in, g))
        if bias_std > 0:
            bs.append(torch.randn(n_out, generator=g,
                                  dtype=torch.float64) * bias_std)
        else:
            bs.append(torch.zeros(n_out, dtype=torch.float64))
    return Ws, bs


def conv_out_hw(h, w, k, s, p):
    return (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1


def cnn_gg(conv_specs, fc_widths, in_shape, seed=0, device='cpu',
           dtype=torch.float32):
    """Conv/ReLU stack, flatten, then fc/ReLU stack (zero biases).

    ``conv_specs`` = [(C_out, k, stride, pad), ...]; ``fc_widths`` lists the
    fc output widths.  Conv ops carry the same fields the reference's
    ``gpu_graph`` writes, including ``output_padding`` computed so that a
    transposed conv reproduces ``in_shape`` (network.py:1761-1764).
    """
    g = _gen(seed)
    ops = []
    prev = INPUT_NAME
    C, H, W_ = in_shape
    li = 0
    for ci, (C_out, k, s, p) in enumerate(conv_specs):
        kern = _kaiming((C_out, C, k, k), C * k * k, g)
        Ho, Wo = conv_out_hw(H, W_, k, s, p)
        oph = H - ((Ho - 1) * s - 2 * p + k)
        opw = W_ - ((Wo - 1) * s - 2 * p + k)
        ops.append({'name': f'conv{ci}', 'type': 'conv', 'inputs': [prev],
                    'kernel': kern.to(device=device, dtype=dtype).contiguous(),
                    'bias': torch.zeros(C_out, dtype=dtype, device=device),
                    'in_shape': (C, H, W_), 'out_shape': (C_out, Ho, Wo),
                    'stride': (s, s), 'padding': (p, p),
                    'output_padding': (oph, opw),
                    'n_out': C_out * Ho * Wo})
        prev = f'conv{ci}'
        ops.append({'name': f'relu{li}', 'type': 'relu', 'inputs': [prev],
                    'layer_idx': li})
        prev = f'relu{li}'
        li += 1
        C, H, W_ = C_out, Ho, Wo
    ops.append({'name': 'flatten', 'type': 'reshape', 'inputs': [prev]})
    prev = 'flatten'
    n = C * H * W_
    for fi, n_out in enumerate(fc_widths):
        Wm = _kaiming((n_out, n), n, g)
        ops.append(_fc_op(f'fc{fi}', prev, Wm, torch.zeros(n_out,
                                                            dtype=torch.float64),
                          device, dtype))
        prev = f'fc{fi}'
        if fi < len(fc_widths) - 1:
            ops.append({'name': f'relu{li}', 'type': 'relu', 'inputs': [prev],
                        'layer_idx': li})
            prev = f'relu{li}'
            li += 1
        n = n_out
    n_in = in_shape[0] * in_shape[1] * in_shape[2]
    return _finish(ops, n_in, (1,) + tuple(in_shape))


# --------------------------------------------------------------------------
# The five workloads
# --------------------------------------------------------------------------

ACAS_WIDTHS = [5, 50, 50, 50, 50, 50, 50, 5]


def acas_gg(seed=0, device='cpu', dtype=torch.float32):
    """5 -> [50]x6 -> 5 ReLU MLP, Kaiming-normal W, N(0, 0.01) biases."""
    Ws, bs = mlp_params(ACAS_WIDTHS, seed=seed, bias_std=0.01)
    return mlp_gg(Ws, bs, device, dtype)


def acas_boxes(B, seed=1, device='cpu', dtype=torch.float32):
    """Centres U[-1, 1]^5, per-dim half-widths U[0.005, 0.05]."""
    g = _gen(seed)
    c = torch.rand(B, 5, generator=g, dtype=torch.float64) * 2 - 1
    r = 0.005 + torch.rand(B, 5, generator=g, dtype=torch.float64) * 0.045
    xl = (c - r).to(device=device, dtype=dtype)
    xh = (c + r).to(device=device, dtype=dtype)
    return xl, xh


def pairwise_spec(n_out, x_lo, x_hi, one_disjunct):
    """Rows y0 - yi (i = 1..n_out-1).

    ``one_disjunct``: all rows in one conjunct (closed iff ANY row's lb > 0);
    otherwise one single-row disjunct per row (closed iff ALL lb > 0).
    """
    cons = [PairwiseConstraint(0, i) for i in range(1, n_out)]
    if one_disjunct:
        disj = [Conjunct(cons)]
    else:
        disj = [Conjunct([c]) for c in cons]
    return VNNSpec(x_lo, x_hi, disj)


def acas_spec(x_lo=None, x_hi=None):
    if x_lo is None:
        x_lo, x_hi = [-1.0] * 5, [1.0] * 5
    return pairwise_spec(5, x_lo, x_hi, one_disjunct=True)


MNIST_MLP_WIDTHS = [784, 1024, 1024, 1024, 1024, 10]


def mnist_mlp_gg(seed=0, device='cpu', dtype=torch.float32):
    Ws, bs = mlp_params(MNIST_MLP_WIDTHS, seed=seed)
    return mlp_gg(Ws, bs, device, dtype)


def linf_boxes(B, n, eps, seed=1, device='cpu', dtype=torch.float32):
    """Centres U[0,1]^n, box [c - eps, c + eps] clipped to [0, 1]."""
    g = _gen(seed)
    c = torch.rand(B, n, generator=g, dtype=torch.float64)
    xl = (c - eps).clamp(0.0, 1.0).to(device=device, dtype=dtype)
    xh = (c + eps).clamp(0.0, 1.0).to(device=device, dtype=dtype)
    return xl, xh


def mnist_mlp_boxes(B=512, seed=1, device='cpu', dtype=torch.float32):
    return linf_boxes(B, 784, 0.02, seed, device, dtype)


CNN_CONVS = [(32, 3, 1, 1), (64, 4, 2, 1), (64, 4, 2, 1)]
CNN_FC = [512, 10]
CNN_IN = (3, 32, 32)


def cifar_cnn_gg(seed=0, device='cpu', dtype=torch.float32):
    return cnn_gg(CNN_CONVS, CNN_FC, CNN_IN, seed=seed, device=device,
                  dtype=dtype)


def cifar_cnn_boxes(B=64, seed=1, device='cpu', dtype=torch.float32):
    return linf_boxes(B, 3 * 32 * 32, 2.0 / 255.0, seed, device, dtype)


DEEP_MLP_WIDTHS = [784, 256, 256, 256, 256, 256, 256, 10]


def deep_mlp_gg(seed=0, device='cpu', dtype=torch.float32):
    Ws, bs = mlp_params(DEEP_MLP_WIDTHS, seed=seed)
    return mlp_gg(Ws, bs, device, dtype)


def relu_split_domains(root_unstable, n_domains=8192, n_splits=8, seed=2):
    """Per-subdomain ReLU split sets for the ReLU-split workload.

    ``root_unstable`` is a list of (layer_idx, neuron) pairs unstable at the
    root.  Each subdomain draws ``n_splits`` distinct pairs without
    replacement and a side per pair (0 = OFF: z <= 0, 1 = ON: z >= 0).
    Returns (layer (D, S) int64, neuron (D, S) int64, side (D, S) int64).
    """
    g = _gen(seed)
    cand = torch.tensor(root_unstable, dtype=torch.int64)
    m = cand.shape[0]
    if m < n_splits:
        raise ValueError(f'only {m} root-unstable neurons, need {n_splits}')
    keys = torch.rand(n_domains, m, generator=g)
    pick = keys.argsort(dim=1)[:, :n_splits]
    side = (torch.rand(n_domains, n_splits, generator=g) < 0.5).to(torch.int64)
    chosen = cand[pick]
    return chosen[..., 0].contiguous(), chosen[..., 1].contiguous(), side


def relu_clamps_from_splits(layer, neuron, side, widths, device='cpu',
                            dtype=torch.float32):
    """Expand split lists into the reference's ``relu_clamps`` dict.

    ``relu_clamps[L] = (cl, ch)`` with -inf/+inf where unclamped, ch = 0 for
    an OFF split and cl = 0 for an ON split (verify_milp.py:2739-2752).
    """
    D = layer.shape[0]
    clamps = {}
    for L, n_L in enumerate(widths):
        cl = torch.full((D, n_L), -float('inf'), dtype=dtype)
        ch = torch.full((D, n_L), float('inf'), dtype=dtype)
        sel = layer == L
        if sel.any():
            rows = torch.arange(D).unsqueeze(1).expand_as(layer)[sel]
            cols = neuron[sel]
            sd = side[sel]
            off = sd == 0
            ch[rows[off], cols[off]] = 0.0
            cl[rows[~off], cols[~off]] = 0.0
            clamps[L] = (cl.to(device), ch.to(device))
    return clamps
