"""Minimal ONNX reader: an .onnx file -> the bound engine's ``gg`` dict.

The ``onnx`` package is not needed: the file is decoded straight from the
protobuf wire format of onnx.proto (varints, 32/64-bit words and
length-delimited fields).  Only the messages and fields the engine's
networks use are read:

  ModelProto.graph (7); GraphProto.node (1), .initializer (5), .input (11),
  .output (12); NodeProto.input (1), .output (2), .op_type (4),
  .attribute (5); AttributeProto.name (1), .f (2), .i (3), .t (5),
  .floats (7), .ints (8); TensorProto.dims (1), .data_type (2),
  .float_data (4), .int64_data (7), .name (8), .raw_data (9),
  .double_data (10); ValueInfoProto.name (1), .type (2) -> tensor_type (1)
  -> shape (2) -> dim (1) -> dim_value (1).

Supported graphs are the feed-forward Linear/Conv/ReLU networks the engine
bounds (the reference builds its ``gg`` from the same ops in
network.py:1707-2910): MatMul or Gemm with a constant weight (+ Add of a
constant bias) -> fc; Relu -> relu; Conv (group 1, dilation 1, symmetric
pads) -> conv; Flatten / Reshape -> reshape; Identity and Dropout pass
through.  An elementwise Sub / Add / Mul / Div of a constant on the network
input (input normalisation) is folded into the first fc or conv: an
all-zero offset or unit scale is dropped exactly, anything else changes
that layer's weights and bias (computed in float64, then rounded once).  A
conv takes per-channel transforms only, and no offset when it pads.
Elsewhere in the graph an Add of two computed tensors becomes a residual
merge ('add' with is_merge), and an Add / Sub / Mul / Div of a computed
tensor and a constant becomes an 'add' / 'sub' / 'mul' op with the
constant spelled out over the tensor's values (const - x as a negation
then an add; x / c as a mul by 1 / c), the op forms of the reference's
reader (network.py:1925-1946, 2020-2053, 2100-2150).
Any other op raises NotImplementedError, as the reference does for ops it
cannot bound.
"""
import struct

import numpy as np
import torch

INPUT_NAME = 'X'

# ONNX TensorProto.DataType codes this reader decodes
_FLOAT, _INT64, _DOUBLE, _INT32 = 1, 7, 11, 6


# ---------------------------------------------------------------- protobuf
def _varint(buf, i):
    v = shift = 0
    while True:
        c = buf[i]
        i += 1
        v |= (c & 0x7F) << shift
        shift += 7
        if c < 0x80:
            return v, i


def _fields(buf):
    """Decode one message: list of (field number, wire type, value)."""
    out = []
    i, n = 0, len(buf)
    while i < n:
        key, i = _varint(buf, i)
        f, wt = key >> 3, key & 7
        if wt == 0:
            v, i = _varint(buf, i)
        elif wt == 1:
            v, i = buf[i:i + 8], i + 8
        elif wt == 5:
            v, i = buf[i:i + 4], i + 4
        elif wt == 2:
            ln, i = _varint(buf, i)
            v, i = buf[i:i + ln], i + ln
        else:
            raise ValueError(f'onnx: unsupported protobuf wire type {wt}')
        out.append((f, wt, v))
    return out


def _ints(entries):
    """Repeated int64 field, packed (wire type 2) or not."""
    vals = []
    for wt, v in entries:
        if wt == 0:
            vals.append(v)
        else:
            j = 0
            while j < len(v):
                x, j = _varint(v, j)
                vals.append(x)
    # two's complement for negative int64
    return [x - (1 << 64) if x >= (1 << 63) else x for x in vals]


def _group(fields):
    d = {}
    for f, wt, v in fields:
        d.setdefault(f, []).append((wt, v))
    return d


def _str(entries):
    return bytes(entries[0][1]).decode('utf-8') if entries else ''


def _tensor(buf):
    t = _group(_fields(buf))
    dims = _ints(t.get(1, []))
    dt = t[2][0][1] if 2 in t else _FLOAT
    name = _str(t.get(8, []))
    if 9 in t:
        raw = bytes(t[9][0][1])
        np_dt = {_FLOAT: '<f4', _DOUBLE: '<f8', _INT64: '<i8', _INT32: '<i4'}.get(dt)
        if np_dt is None:
            raise NotImplementedError(f'onnx: tensor {name!r} has data type {dt}')
        arr = np.frombuffer(raw, dtype=np_dt).copy()
    elif dt == _FLOAT:
        vals = []
        for wt, v in t.get(4, []):
            b = bytes(v)
            if wt == 2:
                vals.extend(struct.unpack(f'<{len(b) // 4}f', b))
            else:
                vals.extend(struct.unpack('<f', b))
        arr = np.array(vals, dtype=np.float32)
    elif dt == _DOUBLE:
        vals = []
        for wt, v in t.get(10, []):
            b = bytes(v)
            vals.extend(struct.unpack(f'<{len(b) // 8}d', b))
        arr = np.array(vals, dtype=np.float64)
    elif dt in (_INT64, _INT32):
        arr = np.array(_ints(t.get(7, []) if dt == _INT64 else t.get(5, [])), dtype=np.int64)
    else:
        raise NotImplementedError(f'onnx: tensor {name!r} has data type {dt}')
    return name, arr.reshape(dims) if dims else arr.reshape(())


def _attrs(entries):
    out = {}
    for _, v in entries:
        a = _group(_fields(v))
        name = _str(a.get(1, []))
        if 2 in a:
            out[name] = struct.unpack('<f', bytes(a[2][0][1]))[0]
        elif 3 in a:
            out[name] = _ints(a[3])[0]
        elif 5 in a:
            out[name] = _tensor(a[5][0][1])[1]
        elif 8 in a:
            out[name] = _ints(a[8])
        elif 7 in a:
            b = b''.join(bytes(v2) for _, v2 in a[7])
            out[name] = list(struct.unpack(f'<{len(b) // 4}f', b))
        elif 4 in a:
            out[name] = bytes(a[4][0][1]).decode('utf-8', 'replace')
    return out


def _value_shape(buf):
    v = _group(_fields(buf))
    name = _str(v.get(1, []))
    shape = []
    if 2 in v:
        tp = _group(_fields(v[2][0][1]))
        if 1 in tp:
            tt = _group(_fields(tp[1][0][1]))
            if 2 in tt:
                for _, d in _group(_fields(tt[2][0][1])).get(1, []):
                    dd = _group(_fields(d))
                    shape.append(_ints(dd[1])[0] if 1 in dd else 1)
    return name, shape


def read_model(data):
    """Parse ONNX bytes: (nodes [(op, inputs, outputs, attrs)], initializers
    {name: ndarray}, graph inputs [(name, shape)], graph outputs [name])."""
    m = _group(_fields(data))
    if 7 not in m:
        raise ValueError('onnx: no graph in model')
    g = _group(_fields(m[7][0][1]))
    inits = dict(_tensor(v) for _, v in g.get(5, []))
    nodes = []
    for _, v in g.get(1, []):
        nd = _group(_fields(v))
        nodes.append((_str(nd.get(4, [])),
                      [bytes(x).decode() for _, x in nd.get(1, [])],
                      [bytes(x).decode() for _, x in nd.get(2, [])],
                      _attrs(nd.get(5, []))))
    inputs = [_value_shape(v) for _, v in g.get(11, [])]
    inputs = [(n, s) for n, s in inputs if n not in inits]
    outputs = [_value_shape(v)[0] for _, v in g.get(12, [])]
    return nodes, inits, inputs, outputs


# ---------------------------------------------------------------- gg build
def _broadcast_const(c, shape):
    """An elementwise constant spelled out over a tensor of ``shape`` (the
    batch dim excluded), flattened.  Leading size-1 axes beyond the
    tensor's rank are the exporter's batch axis, e.g. (1, C, 1, 1) against
    (C, H, W), and are dropped first; any other shape that numpy does not
    broadcast raises NotImplementedError."""
    c = np.asarray(c, dtype=np.float64)
    while c.ndim > len(shape) and c.shape[0] == 1:
        c = c[0]
    try:
        return np.ascontiguousarray(np.broadcast_to(c, tuple(shape))).reshape(-1)
    except ValueError:
        raise NotImplementedError(f'onnx: constant of shape {c.shape} against a tensor '
                                  f'of shape {tuple(shape)}') from None


class _InputAffine:
    """The network input after elementwise constant ops: s * x + o."""

    def __init__(self, shape):
        self.shape = list(shape)
        n = int(np.prod(self.shape))
        self.s = np.ones(n)
        self.o = np.zeros(n)

    def apply(self, op, c):
        c = _broadcast_const(c, self.shape)
        if op == 'Sub':
            self.o = self.o - c
        elif op == 'Add':
            self.o = self.o + c
        elif op == 'Mul':
            self.s, self.o = self.s * c, self.o * c
        elif op == 'Div':
            self.s, self.o = self.s / c, self.o / c

    @property
    def identity(self):
        return bool(np.all(self.s == 1.0) and np.all(self.o == 0.0))


def onnx_to_gg(data, device='cpu', dtype=torch.float32):
    """Build the ``gg`` dict (the schema of the reference's gpu_graph, as
    produced by vibecheck_amd.workloads) from ONNX bytes."""
    nodes, inits, inputs, _ = read_model(data)
    if len(inputs) != 1:
        raise NotImplementedError(f'onnx: {len(inputs)} graph inputs (one supported)')
    in_name, in_shape = inputs[0]
    dims = [d for d in in_shape]
    n_in = int(np.prod(dims)) if dims else 0
    # value of every tensor name: ('const', ndarray) | ('in', _InputAffine)
    # | ('op', gg op name, shape) | ('fc', gg op index, shape) (bias pending)
    val = {k: ('const', v) for k, v in inits.items()}
    val[in_name] = ('in', _InputAffine(dims if dims else [1]))
    ops = []
    n_relu = 0

    def src(v):
        if v[0] == 'in':
            if not v[1].identity:
                raise NotImplementedError('onnx: input transform feeds a non-affine op')
            return INPUT_NAME, v[1].shape
        return v[1] if v[0] == 'op' else ops[v[1]]['name'], v[2]

    def add_op(op):
        op['name'] = f"{op['type']}{len(ops)}"
        ops.append(op)
        return op['name']

    for op_type, ins, outs, at in nodes:
        xs = [val.get(i) for i in ins]
        if op_type == 'Constant':
            val[outs[0]] = ('const', np.asarray(at['value']))
        elif op_type in ('Identity', 'Dropout'):
            val[outs[0]] = xs[0]
        elif op_type in ('Sub', 'Add', 'Mul', 'Div') and xs[0] and xs[0][0] == 'in' \
                and xs[1] and xs[1][0] == 'const':
            xs[0][1].apply(op_type, xs[1][1])
            val[outs[0]] = xs[0]
        elif op_type == 'Add' and xs[0] and xs[0][0] == 'fc' and xs[1] and xs[1][0] == 'const':
            op = ops[xs[0][1]]
            b = np.asarray(xs[1][1], dtype=np.float64).reshape(-1)
            op['_b64'] = op['_b64'] + np.broadcast_to(b, op['_b64'].shape)
            val[outs[0]] = xs[0]
        elif op_type in ('MatMul', 'Gemm'):
            a = xs[0]
            if not (xs[1] and xs[1][0] == 'const'):
                raise NotImplementedError(f'onnx: {op_type} with a non-constant weight')
            Wm = np.asarray(xs[1][1], dtype=np.float64)
            bias = np.zeros(Wm.shape[-1] if op_type == 'MatMul' else 0)
            if op_type == 'Gemm':
                if at.get('transA', 0):
                    raise NotImplementedError('onnx: Gemm with transA')
                if at.get('transB', 0):
                    Wm = Wm.T
                Wm = Wm * float(at.get('alpha', 1.0))
                bias = np.zeros(Wm.shape[1])
                if len(xs) > 2 and xs[2] is not None:
                    if xs[2][0] != 'const':
                        raise NotImplementedError('onnx: Gemm with a non-constant C')
                    bias = float(at.get('beta', 1.0)) * np.broadcast_to(
                        np.asarray(xs[2][1], dtype=np.float64).reshape(-1), (Wm.shape[1],))
            W = Wm.T.copy()  # (n_out, n_in)
            if a[0] == 'in':
                aff = a[1]
                bias = bias + W @ aff.o
                W = W * aff.s[None, :]
                inp = INPUT_NAME
            else:
                inp = src(a)[0]
            i = len(ops)
            add_op({'type': 'fc', 'inputs': [inp], '_W64': W, '_b64': np.array(bias, dtype=np.float64)})
            val[outs[0]] = ('fc', i, [W.shape[0]])
        elif op_type == 'Relu':
            name, shape = src(xs[0])
            r = add_op({'type': 'relu', 'inputs': [name], 'layer_idx': n_relu})
            n_relu += 1
            val[outs[0]] = ('op', r, shape)
        elif op_type in ('Flatten', 'Reshape'):
            a = xs[0]
            if a[0] == 'in':
                val[outs[0]] = a
                continue
            name, shape = src(a)
            r = add_op({'type': 'reshape', 'inputs': [name]})
            val[outs[0]] = ('op', r, [int(np.prod(shape))])
        elif op_type == 'Conv':
            a = xs[0]
            if not (xs[1] and xs[1][0] == 'const'):
                raise NotImplementedError('onnx: Conv with a non-constant kernel')
            K = np.asarray(xs[1][1], dtype=np.float64)
            C_out, C_in, kh, kw = K.shape
            if at.get('group', 1) != 1 or any(d != 1 for d in at.get('dilations', [1, 1])):
                raise NotImplementedError('onnx: grouped or dilated Conv')
            pads = at.get('pads', [0, 0, 0, 0])
            if pads[0] != pads[2] or pads[1] != pads[3]:
                raise NotImplementedError('onnx: asymmetric Conv padding')
            st = at.get('strides', [1, 1])
            b = (np.asarray(xs[2][1], dtype=np.float64).reshape(-1)
                 if len(xs) > 2 and xs[2] is not None else np.zeros(C_out))
            if a[0] == 'in':
                shape = a[1].shape[-3:]
                if not a[1].identity:
                    s = a[1].s.reshape(shape)
                    o = a[1].o.reshape(shape)
                    if not (np.all(s == s[:, :1, :1]) and np.all(o == o[:, :1, :1])):
                        raise NotImplementedError('onnx: per-pixel input transform before Conv')
                    if np.any(o != 0.0) and (pads[0] or pads[1]):
                        # the zero padding of the shifted input is not a
                        # zero of the raw input: no per-channel bias matches
                        raise NotImplementedError('onnx: input offset before a padded Conv')
                    b = b + (K * o[None, :, 0, 0, None, None]).sum((1, 2, 3))
                    K = K * s[None, :, 0, 0, None, None]
                inp = INPUT_NAME
            else:
                inp, shape = src(a)
            C, H, W_ = [int(d) for d in shape[-3:]]
            Ho = (H + 2 * pads[0] - kh) // st[0] + 1
            Wo = (W_ + 2 * pads[1] - kw) // st[1] + 1
            oph = H - ((Ho - 1) * st[0] - 2 * pads[0] + kh)
            opw = W_ - ((Wo - 1) * st[1] - 2 * pads[1] + kw)
            r = add_op({'type': 'conv', 'inputs': [inp], '_K64': K, '_b64': b,
                        'in_shape': (C, H, W_), 'out_shape': (C_out, Ho, Wo),
                        'stride': (st[0], st[1]), 'padding': (pads[0], pads[1]),
                        'output_padding': (oph, opw), 'n_out': C_out * Ho * Wo})
            val[outs[0]] = ('op', r, [C_out, Ho, Wo])
        elif op_type == 'Add' and xs[0] and xs[1] and xs[0][0] != 'const' \
                and xs[1][0] != 'const':
            # two live inputs: a residual merge (network.py:2020-2053)
            (na, sa), (nb, sb_) = src(xs[0]), src(xs[1])
            if int(np.prod(sa)) != int(np.prod(sb_)):
                raise NotImplementedError('onnx: Add of differently shaped tensors')
            r = add_op({'type': 'add', 'inputs': [na, nb], 'is_merge': True, 'bias': None})
            val[outs[0]] = ('op', r, sa)
        elif op_type in ('Add', 'Sub', 'Mul', 'Div') and xs[0] and xs[1] \
                and (xs[0][0] == 'const') != (xs[1][0] == 'const'):
            # a computed tensor and a constant (network.py:1925-1946,
            # 2100-2150): the constant spelled out over the tensor's values
            live_first = xs[1][0] == 'const'
            name, shape = src(xs[0] if live_first else xs[1])
            c = np.asarray((xs[1] if live_first else xs[0])[1], dtype=np.float64)
            flat = _broadcast_const(c, shape) if c.size != 1 else c.reshape(-1)
            if op_type == 'Add':
                r = add_op({'type': 'add', 'inputs': [name], 'is_merge': False, 'bias': flat})
            elif op_type == 'Sub' and live_first:
                r = add_op({'type': 'sub', 'inputs': [name], 'bias': flat})
            elif op_type == 'Sub':
                # const - x: negate, then add the constant
                m = add_op({'type': 'mul', 'inputs': [name], 'scale': np.array([-1.0])})
                r = add_op({'type': 'add', 'inputs': [m], 'is_merge': False, 'bias': flat})
            elif op_type == 'Mul':
                r = add_op({'type': 'mul', 'inputs': [name], 'scale': flat})
            elif live_first:
                r = add_op({'type': 'mul', 'inputs': [name], 'scale': 1.0 / flat})
            else:
                raise NotImplementedError('onnx: Div of a constant by a tensor')
            val[outs[0]] = ('op', r, shape)
        else:
            raise NotImplementedError(f'onnx: unsupported op {op_type!r}')

    for op in ops:
        if op['type'] == 'fc':
            op['W'] = torch.as_tensor(op.pop('_W64')).to(device=device, dtype=dtype).contiguous()
            op['bias'] = torch.as_tensor(op.pop('_b64')).to(device=device, dtype=dtype).contiguous()
        elif op['type'] == 'conv':
            op['kernel'] = torch.as_tensor(op.pop('_K64')).to(device=device,
                                                              dtype=dtype).contiguous()
            op['bias'] = torch.as_tensor(op.pop('_b64')).to(device=device, dtype=dtype).contiguous()
    refs = {}
    for op in ops:
        for i in op['inputs']:
            refs[i] = refs.get(i, 0) + 1
    relu_names = [op['name'] for op in ops if op['type'] == 'relu']
    return {'ops': ops, 'relu_names': relu_names,
            'fork_points': {n for n, c in refs.items() if c > 1},
            'n_relu': len(relu_names), 'input_name': INPUT_NAME,
            'input_n': n_in, 'input_shape': tuple(dims) if dims else (1, n_in)}


def load_onnx(path, device='cpu', dtype=torch.float32):
    """``gg`` of the network in an .onnx file (see onnx_to_gg)."""
    with open(path, 'rb') as f:
        return onnx_to_gg(f.read(), device=device, dtype=dtype)
