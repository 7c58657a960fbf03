"""On-disk formats: the ONNX reader and the VNNLIB reader (CPU).

Known answers come from the reference's bundled example
(examples/ACASXU_run2a_2_2_batch_2000.onnx with prop_1 / prop_2, copied as
fixtures under tests/golden/acasxu/): its README prints the violating input
of prop_2 and the network's output there, which the loaded network must
reproduce; the properties' boxes and constraints are read off the files.
Synthetic models written by a small protobuf encoder here pin the ops the
example does not use (Gemm with transB/alpha/beta, Conv with stride and
padding, input scaling) against a plain numpy forward pass."""
import os
import struct

import numpy as np
import pytest
import torch

from oracle import ref_bound as rb
from vibecheck_amd import onnx_net, vnnlib
from vibecheck_amd.spec import Constraint, PairwiseConstraint

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'acasxu')
NET = os.path.join(GOLD, 'ACASXU_run2a_2_2_batch_2000.onnx')

# README.md:59-71 of the reference: prop_2's satisfying assignment
WITNESS_X = [0.6208617091178894, -0.01862180233001709, -0.024315983057022095,
             0.47021740674972534, -0.46439468860626221]
WITNESS_Y = [0.023801768198609352, -0.021306384354829788, 0.023232858628034592,
             -0.016359567642211914, 0.023021360859274864]


def test_acasxu_network_structure():
    gg = onnx_net.load_onnx(NET)
    kinds = [op['type'] for op in gg['ops']]
    assert kinds == ['fc', 'relu'] * 6 + ['fc']
    assert [tuple(op['W'].shape) for op in gg['ops'] if op['type'] == 'fc'] == \
        [(50, 5)] + [(50, 50)] * 5 + [(5, 50)]
    assert gg['input_n'] == 5 and gg['n_relu'] == 6
    assert [op['layer_idx'] for op in gg['ops'] if op['type'] == 'relu'] == list(range(6))


@pytest.mark.parametrize('dtype,tol', [(torch.float64, 1e-8), (torch.float32, 2e-8)])
def test_acasxu_witness_known_answer(dtype, tol):
    """The reference's printed output at prop_2's witness (fp32 values
    printed to 17 digits)."""
    gg = onnx_net.load_onnx(NET, dtype=dtype)
    y, _ = rb.point_forward(torch.tensor([WITNESS_X], dtype=dtype), gg)
    err = (y.double()[0] - torch.tensor(WITNESS_Y, dtype=torch.float64)).abs().max()
    assert float(err) < tol, float(err)
    # prop_2's unsafe region: COC (output 0) is maximal there
    assert int(y[0].argmax()) == 0


def test_acasxu_properties():
    box_lo = np.array([0.6, -0.5, -0.5, 0.45, -0.5], dtype=np.float32)
    box_hi = np.array([0.679857769, 0.5, 0.5, 0.5, -0.45], dtype=np.float32)
    p1 = vnnlib.load_vnnlib(os.path.join(GOLD, 'prop_1.vnnlib'))
    assert np.array_equal(p1.x_lo, box_lo.astype(np.float64))
    assert np.array_equal(p1.x_hi, box_hi.astype(np.float64))
    assert len(p1.disjuncts) == 1
    assert p1.disjuncts[0].constraints == [Constraint(0, '>=', 3.991125645861615)]
    (di, w, b), = p1.as_linear_queries(5)
    assert di == 0 and list(w) == [-1, 0, 0, 0, 0] and b == 3.991125645861615
    p2 = vnnlib.load_vnnlib(os.path.join(GOLD, 'prop_2.vnnlib'))
    assert np.array_equal(p2.x_lo, p1.x_lo) and np.array_equal(p2.x_hi, p1.x_hi)
    assert p2.disjuncts[0].constraints == [PairwiseConstraint(pred=i, comp=0)
                                           for i in range(1, 5)]
    qs = p2.as_linear_queries(5)
    assert [list(w) for _, w, _ in qs] == [[-1, 1, 0, 0, 0], [-1, 0, 1, 0, 0],
                                           [-1, 0, 0, 1, 0], [-1, 0, 0, 0, 1]]
    # the witness lies in the box and in the unsafe region of every query
    x = np.array(WITNESS_X)
    assert np.all(x >= p2.x_lo) and np.all(x <= p2.x_hi)
    assert all(float(w @ np.array(WITNESS_Y)) + b <= 0 for _, w, b in qs)


def test_vnnlib_forms_and_dnf():
    text = """
    ; version-1 form, two output disjuncts with their own input boxes
    (declare-const X_0 Real)
    (declare-const X_1 Real)
    (declare-const Y_0 Real)
    (declare-const Y_1 Real)
    (declare-const Y_2 Real)
    (assert (or
        (and (>= X_0 -1) (<= X_0 0) (>= X_1 0.5) (<= X_1 (+ 0.25 0.5)) (>= Y_1 Y_0))
        (and (>= X_0 0) (<= X_0 1) (>= X_1 0.5) (<= X_1 0.75)
             (<= (* 2 Y_2) 3) (> Y_0 Y_2))))
    """
    sp = vnnlib.parse_vnnlib(text)
    assert list(sp.x_lo) == [-1.0, 0.5] and list(sp.x_hi) == [1.0, 0.75]
    d0, d1 = sp.disjuncts
    assert d0.constraints == [PairwiseConstraint(pred=0, comp=1)]
    assert list(d0.input_lo) == [-1.0, 0.5] and list(d0.input_hi) == [0.0, 0.75]
    assert d1.constraints == [Constraint(2, '<=', 1.5), PairwiseConstraint(pred=2, comp=0)]
    assert list(d1.input_lo) == [0.0, 0.5] and list(d1.input_hi) == [1.0, 0.75]
    # conjoined asserts distribute over an output OR; one shared box
    text2 = """
    (declare-network N (declare-input X float32 [1, 2]) (declare-output Y float32 [1, 3]))
    (assert (<= X[0,0] 1)) (assert (>= X[0,0] 0)) (assert (<= X[0,1] 2)) (assert (>= X[0,1] 1))
    (assert (or (and (>= Y[0,0] 4)) (and (<= Y[0,2] Y[0,1]))))
    """
    sp2 = vnnlib.parse_vnnlib(text2)
    assert [d.constraints for d in sp2.disjuncts] == [[Constraint(0, '>=', 4.0)],
                                                      [PairwiseConstraint(pred=2, comp=1)]]
    assert all(d.input_lo is None for d in sp2.disjuncts)
    with pytest.raises(NotImplementedError):
        vnnlib.parse_vnnlib('(declare-const X_0 Real)(declare-const Y_0 Real)'
                            '(assert (<= X_0 1))(assert (<= (* Y_0 Y_0) 1))')
    with pytest.raises(NotImplementedError):
        vnnlib.parse_vnnlib('(declare-const X_0 Real)(declare-const Y_0 Real)'
                            '(declare-const Y_1 Real)(assert (<= X_0 1))'
                            '(assert (<= Y_0 (* 2 Y_1)))')


# ------------------------------------------------------- a protobuf writer
def _v(n):
    out = bytearray()
    n &= (1 << 64) - 1
    while True:
        b = n & 0x7F
        n >>= 7
        if n:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _f(num, payload):
    if isinstance(payload, int):
        return _v(num << 3) + _v(payload)
    if isinstance(payload, float):
        return _v((num << 3) | 5) + struct.pack('<f', payload)
    if isinstance(payload, str):
        payload = payload.encode()
    return _v((num << 3) | 2) + _v(len(payload)) + payload


def _tensor(name, arr):
    arr = np.asarray(arr, dtype=np.float32)
    return b''.join(_f(1, int(d)) for d in arr.shape) + _f(2, 1) + _f(8, name) + \
        _f(9, arr.tobytes())


def _node(op, ins, outs, **attrs):
    b = b''.join(_f(1, i) for i in ins) + b''.join(_f(2, o) for o in outs) + _f(4, op)
    for k, v in attrs.items():
        if isinstance(v, list):
            a = _f(1, k) + b''.join(_f(8, int(x)) for x in v) + _f(20, 7)
        elif isinstance(v, float):
            a = _f(1, k) + _f(2, v) + _f(20, 1)
        else:
            a = _f(1, k) + _f(3, int(v)) + _f(20, 2)
        b += _f(5, a)
    return b


def _value_info(name, shape):
    dims = b''.join(_f(1, _f(1, int(d))) for d in shape)
    return _f(1, name) + _f(2, _f(1, _f(1, 1) + _f(2, dims)))


def _model(nodes, inits, in_shape):
    g = b''.join(_f(1, n) for n in nodes) + _f(2, 'g') + \
        b''.join(_f(5, _tensor(k, v)) for k, v in inits.items()) + \
        _f(11, _value_info('input', in_shape)) + _f(12, _value_info('out', [1]))
    return _f(1, 8) + _f(8, _f(2, 13)) + _f(7, g)


def _np_conv(x, K, b, s, p):
    C, H, W = x.shape
    Co, _, kh, kw = K.shape
    xp = np.pad(x, ((0, 0), (p, p), (p, p)))
    Ho, Wo = (H + 2 * p - kh) // s + 1, (W + 2 * p - kw) // s + 1
    out = np.zeros((Co, Ho, Wo))
    for yo in range(Ho):
        for xo in range(Wo):
            patch = xp[:, yo * s:yo * s + kh, xo * s:xo * s + kw]
            out[:, yo, xo] = (K * patch[None]).sum((1, 2, 3)) + b
    return out


@pytest.mark.parametrize('norm,pad', [('sub_div', 0), ('mul', 1)])
def test_onnx_synthetic_gemm_conv_and_input_scaling(norm, pad):
    rng = np.random.default_rng(5 + pad)
    K = rng.standard_normal((3, 2, 3, 3)).astype(np.float32)
    kb = rng.standard_normal(3).astype(np.float32)
    mean = rng.standard_normal((1, 2, 1, 1)).astype(np.float32)
    std = (rng.random((1, 2, 1, 1)) + 0.5).astype(np.float32)
    Ho = (5 + 2 * pad - 3) // 2 + 1
    G = rng.standard_normal((4, 3 * Ho * Ho)).astype(np.float32)    # Gemm B, transB
    gc = rng.standard_normal(4).astype(np.float32)
    W2 = rng.standard_normal((4, 2)).astype(np.float32)    # MatMul weight
    b2 = rng.standard_normal(2).astype(np.float32)
    if norm == 'sub_div':
        pre = [_node('Sub', ['input', 'mean'], ['t0']), _node('Div', ['t0', 'std'], ['t1'])]
    else:
        pre = [_node('Identity', ['input'], ['t0']), _node('Mul', ['t0', 'std'], ['t1'])]
    nodes = pre + [
        _node('Conv', ['t1', 'K', 'kb'], ['t2'], strides=[2, 2], pads=[pad] * 4,
              kernel_shape=[3, 3]),
        _node('Relu', ['t2'], ['t3']), _node('Flatten', ['t3'], ['t4'], axis=1),
        _node('Gemm', ['t4', 'G', 'gc'], ['t5'], transB=1, alpha=0.5, beta=2.0),
        _node('Relu', ['t5'], ['t6']), _node('MatMul', ['t6', 'W2'], ['t7']),
        _node('Add', ['t7', 'b2'], ['out'])]
    data = _model(nodes, dict(mean=mean, std=std, K=K, kb=kb, G=G, gc=gc, W2=W2, b2=b2),
                  [1, 2, 5, 5])
    gg = onnx_net.onnx_to_gg(data, dtype=torch.float64)
    assert [op['type'] for op in gg['ops']] == ['conv', 'relu', 'reshape', 'fc', 'relu', 'fc']
    x = rng.random((1, 2, 5, 5))
    xn = (x - mean) / std if norm == 'sub_div' else x * std
    h = np.maximum(_np_conv(xn[0], K.astype(np.float64), kb, 2, pad), 0)
    h = np.maximum(0.5 * h.reshape(-1) @ G.T.astype(np.float64) + 2.0 * gc, 0)
    ref = h @ W2 + b2
    got, _ = rb.point_forward(torch.tensor(x.reshape(1, -1)), gg)
    assert np.allclose(got.numpy()[0], ref, rtol=1e-9, atol=1e-9)


def test_onnx_refuses_what_it_cannot_represent():
    with pytest.raises(NotImplementedError):
        onnx_net.onnx_to_gg(_model([_node('Sigmoid', ['input'], ['out'])], {}, [1, 3]))
    K = np.ones((1, 1, 3, 3), dtype=np.float32)
    nodes = [_node('Sub', ['input', 'm'], ['t0']),
             _node('Conv', ['t0', 'K'], ['out'], pads=[1, 1, 1, 1], kernel_shape=[3, 3])]
    with pytest.raises(NotImplementedError):
        onnx_net.onnx_to_gg(_model(nodes, dict(m=np.full((1, 1, 1, 1), 0.5), K=K),
                                   [1, 1, 4, 4]))


def test_onnx_synthetic_residual_and_affine_ops():
    """A residual MLP written as ONNX: Gemm -> Relu (r1) -> Gemm -> Add with
    r1 (a merge of two computed tensors) -> Relu -> Mul by a constant ->
    Sub a constant -> (const - x) -> Div by a constant -> MatMul.  The
    reader emits the reference's op forms (merge add; mul, sub, mul(-1) +
    add, mul(1/c)); the oracle's point forward of the gg equals numpy's."""
    rng = np.random.default_rng(11)
    W1 = rng.standard_normal((6, 4)).astype(np.float32)   # Gemm B, transB
    c1 = rng.standard_normal(6).astype(np.float32)
    W2 = rng.standard_normal((6, 6)).astype(np.float32)
    c2 = rng.standard_normal(6).astype(np.float32)
    sc = (rng.random(6) + 0.5).astype(np.float32)
    sh = rng.standard_normal(6).astype(np.float32)
    k0 = rng.standard_normal(6).astype(np.float32)
    dv = (rng.random(6) + 1.0).astype(np.float32)
    W3 = rng.standard_normal((6, 3)).astype(np.float32)   # MatMul weight
    nodes = [_node('Gemm', ['input', 'W1', 'c1'], ['t1'], transB=1),
             _node('Relu', ['t1'], ['r1']),
             _node('Gemm', ['r1', 'W2', 'c2'], ['t2'], transB=1),
             _node('Add', ['t2', 'r1'], ['t3']),
             _node('Relu', ['t3'], ['r2']),
             _node('Mul', ['r2', 'sc'], ['t4']),
             _node('Sub', ['t4', 'sh'], ['t5']),
             _node('Sub', ['k0', 't5'], ['t6']),
             _node('Div', ['t6', 'dv'], ['t7']),
             _node('MatMul', ['t7', 'W3'], ['out'])]
    data = _model(nodes, dict(W1=W1, c1=c1, W2=W2, c2=c2, sc=sc, sh=sh, k0=k0, dv=dv, W3=W3),
                  [1, 4])
    gg = onnx_net.onnx_to_gg(data, dtype=torch.float64)
    types = [(op['type'], op.get('is_merge')) for op in gg['ops']]
    assert types == [('fc', None), ('relu', None), ('fc', None), ('add', True),
                     ('relu', None), ('mul', None), ('sub', None), ('mul', None),
                     ('add', False), ('mul', None), ('fc', None)]
    assert gg['ops'][1]['name'] in gg['fork_points']
    x = rng.random((5, 4))
    f = lambda a: a.astype(np.float64)
    r1 = np.maximum(x @ f(W1).T + f(c1), 0)
    r2 = np.maximum(r1 @ f(W2).T + f(c2) + r1, 0)
    t7 = (f(k0) - (r2 * f(sc) - f(sh))) / f(dv)
    ref = t7 @ f(W3)
    got, _ = rb.point_forward(torch.tensor(x), gg)
    assert np.allclose(got.numpy(), ref, rtol=1e-9, atol=1e-9)


def test_onnx_constant_with_a_batch_axis():
    """A per-channel constant exported with a leading batch axis, (1, C, 1,
    1), against a computed (C, H, W) tensor is read as the channel vector
    (the exporter's batch axis dropped); one that does not broadcast is
    refused with NotImplementedError, not a numpy ValueError."""
    rng = np.random.default_rng(3)
    K = rng.standard_normal((3, 2, 3, 3)).astype(np.float32)
    cb = rng.standard_normal((1, 3, 1, 1)).astype(np.float32)
    G = rng.standard_normal((2, 3 * 9)).astype(np.float32)

    def model(c):
        nodes = [_node('Conv', ['input', 'K'], ['t1'], pads=[1, 1, 1, 1], kernel_shape=[3, 3]),
                 _node('Add', ['t1', 'cb'], ['t2']), _node('Relu', ['t2'], ['t3']),
                 _node('Flatten', ['t3'], ['t4'], axis=1),
                 _node('Gemm', ['t4', 'G'], ['out'], transB=1)]
        return _model(nodes, dict(K=K, cb=c, G=G), [1, 2, 3, 3])

    gg = onnx_net.onnx_to_gg(model(cb), dtype=torch.float64)
    x = rng.random((1, 2, 3, 3))
    h = np.maximum(_np_conv(x[0], K.astype(np.float64), np.zeros(3), 1, 1)
                   + cb[0].astype(np.float64), 0)
    ref = h.reshape(-1) @ G.T.astype(np.float64)
    got, _ = rb.point_forward(torch.tensor(x.reshape(1, -1)), gg)
    assert np.allclose(got.numpy()[0], ref, rtol=1e-9, atol=1e-9)
    with pytest.raises(NotImplementedError):
        onnx_net.onnx_to_gg(model(np.ones((1, 4, 1, 1), dtype=np.float32)))
