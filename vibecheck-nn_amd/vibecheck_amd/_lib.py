"""ctypes binding of libvibecheck_amd.so (the C ABI in include/vibecheck_amd.h).

The library is the only compute path: if it is missing, or a tensor is not
on the GPU, calls raise instead of falling back to anything else.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, 'libvibecheck_amd.so')

VC_OK, VC_ERR_ARG, VC_ERR_OOM, VC_ERR_UNSUPPORTED, VC_ERR_LAUNCH = 0, 1, 2, 3, 4
VC_ZONO_WIDE_COLS = 512     # generator columns of vc_mlp_tiled_zono_wide
VC_ALPHA_CHUNK = 4          # iterations per launch of vc_mlp_tiled_alpha_run

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_D = ctypes.c_double

# name -> argtypes (restype int unless listed in _RESTYPE)
SIGNATURES = {
    'vc_abi_version': [],
    'vc_make_slopes': [_P, _P, _L, _P, _P, _P, _P, _P, _P, _P],
    'vc_ibp_fc': [_P, _P, _L, _I, _P, _P, _I, _P, _P, _P],
    'vc_ibp_conv': [_P, _P, _L, _I, _I, _I, _P, _P, _I, _I, _I, _I, _I, _I,
                    _I, _I, _I, _P, _P, _P],
    'vc_ibp_relu': [_P, _P, _L, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    'vc_zono_input': [_P, _P, _L, _I, _P, _I, _P, _P, _P],
    'vc_affine_ew': [_P, _L, _I, _L, _P, _I, _I, _P, _P],
    'vc_interval_mul': [_P, _P, _L, _I, _P, _I, _P, _P, _P],
    'vc_add_ew': [_P, _P, _L, _P, _P],
    'vc_zono_merge': [_P, _I, _P, _I, _I, _L, _P, _P],
    'vc_rows_bias_dot': [_P, _L, _I, _I, _I, _P, _I, _F, _P, _P],
    'vc_zono_fc': [_P, _P, _L, _I, _I, _P, _P, _I, _P, _P, _P],
    'vc_zono_conv': [_P, _P, _L, _I, _I, _I, _I, _P, _P, _I, _I, _I, _I, _I,
                     _I, _I, _I, _I, _P, _P, _P],
    'vc_zono_relu_bounds': [_P, _P, _L, _I, _I, _P, _P, _P, _P, _P],
    'vc_zono_relu_apply': [_P, _P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P],
    'vc_backward_fc': [_P, _L, _I, _I, _P, _P, _P, _I, _P, _P, _P, _I, _P,
                       _P, _P, _I, _P],
    'vc_backward_fc_grouped': [_P, _L, _I, _I, _P, _P, _P, _P, _L, _P, _P, _I, _P, _P, _P,
                               _I, _P],
    'vc_group_clamp': [_P, _L, _L, _P, _P, _P],
    'vc_backward_relu': [_P, _L, _I, _I, _P, _P, _P, _I, _P, _P, _P, _P],
    'vc_relax_slopes': [_P, _P, _P, _L, _P, _P, _P, _P],
    'vc_alpha_grad_step_slopes': [_P, _P, _L, _I, _I, _P, _P, _P, _I, _P, _P,
                                  _I, _P, _P],
    'vc_backward_conv': [_P, _L, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                         _I, _I, _I, _P, _P, _P],
    'vc_conv_t_pack_floats': [_I, _I, _I, _I, _I, _I],
    'vc_backward_relu_conv_ok': [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I],
    'vc_backward_relu_conv': [_P, _L, _L, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                              _I, _I, _I, _I, _I, _I, _P, _P, _P],
    'vc_conv_t_pack': [_P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P],
    'vc_backward_conv_packed': [_P, _L, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                                _I, _I, _I, _P, _P, _P],
    'vc_concretize': [_P, _P, _P, _P, _L, _I, _I, _I, _P, _P],
    'vc_crown_intersect': [_P, _P, _I, _L, _I, _P, _P, _P],
    'vc_unstable_union': [_P, _P, _L, _I, _P, _P],
    'vc_alpha_init': [_P, _P, _L, _P, _P],
    'vc_alpha_grad_step': [_P, _P, _L, _I, _I, _P, _P, _P, _I, _P, _P, _I,
                           _P, _P],
    'vc_alpha_grad_reduce': [_P, _P, _I, _L, _I, _I, _P, _P, _P, _P, _P],
    'vc_alpha_grad_input': [_P, _P, _P, _L, _I, _I, _P, _P, _I, _P, _P],
    'vc_adam_step': [_P, _P, _P, _P, _L, _D, _D, _D, _D, _D, _F, _F, _P],
    'vc_beta_adam_step': [_P, _P, _P, _P, _P, _L, _D, _D, _D, _D, _D, _P, _P],
    'vc_split_beta_sign': [_P, _P, _L, _P, _P],
    'vc_split_clamps': [_P, _P, _P, _L, _I, _L, _I, _P, _P, _P, _P],
    'vc_best_update': [_P, _P, _L, _I, _P, _P],
    'vc_box_shrunk': [_P, _P, _P, _P, _L, _P, _P],
    'vc_closure': [_P, _L, _I, _P, _P, _I, _P, _P],
    'vc_clip_box': [_P, _P, _P, _P, _L, _I, _I, _P, _P, _I, _P, _P, _P, _P],
    'vc_branch_topk': [_P, _P, _P, _P, _L, _I, _I, _I, _F, _F, _I, _P, _P, _P],
    'vc_split_multi_plan': [_P, _P, _P, _L, _I, _I, _P, _P, _P],
    'vc_split_multi': [_P, _P, _P, _P, _L, _I, _I, _P, _P, _P],
    'vc_alpha_band_keys': [_P, _L, _I, _P, _P, _I, _P, _F, _P, _P, _P],
    'vc_rank_select_desc': [_P, _P, _L, _L, _P, _P],
    'vc_alpha_grad_step_rows': [_P, _P, _L, _I, _I, _P, _P, _P, _I, _P, _P, _I, _P, _P, _P],
    'vc_alpha_grad_rows': [_P, _P, _I, _L, _I, _I, _P, _P, _P, _P],
    'vc_bound_tighten': [_P, _P, _P, _L, _I, _P],
    'vc_best_sum': [_P, _P, _L, _I, _P, _P],
    'vc_best_rows_with_A': [_P, _P, _P, _P, _L, _I, _I, _I, _P],
    'vc_compact_workspace': [_L],
    'vc_compact': [_P, _L, _I, _P, _P, _P, _L, _P],
    'vc_scatter_max_rows': [_P, _P, _P, _L, _I, _P],
    'vc_gather_rows': [_P, _P, _L, _I, _P, _P],
    'vc_scatter_rows': [_P, _P, _L, _I, _P, _P],
    'vc_mlp_frag_floats': [_P, _I, _I],
    'vc_mlp_pack': [_P, _P, _I, _I, _P, _P],
    'vc_mlp_zono_bounds': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P],
    'vc_mlp_crown': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                     _I, _P, _P, _P, _P, _P, _P],
    'vc_mlp_alpha_iter': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _I,
                          _P, _P, _P, _D, _D, _D, _D, _D, _P],
    'vc_mlp_tiled_floats': [_P, _I],
    'vc_mlp_tiled_pack': [_P, _P, _P, _I, _P, _P],
    'vc_mlp_tiled_crown': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I,
                           _I, _P, _P, _P, _P, _P, _P, _P, _P],
    'vc_mlp_tiled_alpha_iter': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                                _P, _P, _P, _D, _D, _D, _D, _D, _I, _P, _P],
    'vc_mlp_tiled_alpha_run': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _I,
                               _P, _P, _P, _P, _D, _D, _D, _D, _D, _I, _D, _P, _P, _P],
    'vc_mlp_tiled_crown_mode': [_L],
    'vc_mlp_crown_rows_workspace': [_P, _I, _L],
    'vc_mlp_crown_rows': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                          _P, _P, _P, _P, _P, _P, _P, _L, _P],
    'vc_mlp_tiled_crown_noalloc': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                   _P, _P, _P, _P, _P, _P],
    'vc_unstable_union_layers': [_P, _P, _P, _I, _L, _P, _P],
    'vc_union_compact': [_P, _P, _I, _P, _P, _P],
    'vc_gather_rows_multi': [_P, _P, _P, _I, _P, _L, _P],
    'vc_alpha_control': [_P, _P, _L, _I, _D, _P, _P, _P],
    'vc_mlp_tiled_zono_bounds': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P],
    'vc_mlp_zono_wide': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P],
    'vc_mlp_tiled_zono_wide': [_P, _I, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P],
    'vc_mlp_bab_round_workspace': [_P, _I, _L, _I],
    'vc_mlp_bab_round_lookahead_workspace': [_P, _I, _L, _I, _L],
    'vc_mlp_bab_round_handoff_offsets': [_P, _I, _L, _I, _P],
    'vc_mlp_bab_round': [_P, _I, _P, _P, _I, _P, _P, _P, _P, _I, _L, _P, _P, _I, _D, _D, _D,
                         _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                         _P, _P, _L, _P, _P, _L, _L, _P, _P, _P, _P, _P, _P],
    'vc_widest_axis': [_P, _P, _L, _I, _P, _P, _P],
    'vc_bisect': [_P, _P, _P, _P, _L, _I, _P, _P, _P, _P, _P],
}
_RESTYPE = {'vc_compact_workspace': ctypes.c_int64,
            'vc_conv_t_pack_floats': ctypes.c_int64,
            'vc_mlp_crown_rows_workspace': ctypes.c_int64,
            'vc_mlp_bab_round_workspace': ctypes.c_int64,
            'vc_mlp_bab_round_lookahead_workspace': ctypes.c_int64,
            'vc_mlp_frag_floats': ctypes.c_int64,
            'vc_mlp_tiled_floats': ctypes.c_int64}


def host_array(ctype, values):
    """ctypes array of host values; returns (array, address) -- keep the
    array alive for the duration of the call."""
    arr = (ctype * max(1, len(values)))(*values)
    return arr, ctypes.addressof(arr)

_lib = None


class HipLibraryMissing(ImportError):
    pass


def load():
    """Load (once) and return the ctypes library handle."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipLibraryMissing(
            f'{LIB_PATH} is not built; run __graft_entry__.build() or '
            f'make -C vibecheck-nn_amd/csrc')
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    _lib = lib
    return lib


def check(rc, name):
    if rc == VC_OK:
        return
    msg = f'{name} failed with status {rc}'
    if rc == VC_ERR_OOM:
        raise torch.cuda.OutOfMemoryError(msg)
    if rc == VC_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == VC_ERR_ARG:
        raise ValueError(msg)
    raise RuntimeError(msg)


def mlp_crown_flops(dims, n, B, cnt, do_crown, Q):
    """Algorithmic flops of one vc_mlp_crown launch: every seeded row of
    layer L (2 cnt[L] rows) goes through fc_{L-1} .. fc_0 backward, every
    spec row through fc_{n-1} .. fc_0; a row through fc_l costs
    2 d[l] d[l+1]."""
    step = [2.0 * dims[l] * dims[l + 1] for l in range(n)]
    per_dom = 0.0
    if do_crown:
        for L in range(n):
            per_dom += 2 * cnt[L] * sum(step[:L])
    per_dom += Q * sum(step)
    return per_dom * B


def _flops_mlp_crown(a):
    n = a[1]
    dims = list((ctypes.c_int32 * (n + 1)).from_address(a[0]))
    cnt = list((ctypes.c_int32 * n).from_address(a[12])) if a[13] else [0] * n
    return mlp_crown_flops(dims, n, a[4], cnt, a[13], a[14])


def seed_flops(dims, seeded):
    """Algorithmic flops of the seeded rows of vc_mlp_tiled_crown launches,
    from the per-layer seeded-neuron totals of its seed_rows output (each
    seeded neuron is two rows through fc_{L-1} .. fc_0)."""
    step = [2.0 * dims[l] * dims[l + 1] for l in range(len(dims) - 1)]
    return sum(2.0 * int(seeded[L]) * sum(step[:L]) for L in range(len(dims) - 1))


def _flops_tiled_spec(a):
    # Spec rows only: the seeded rows depend on each domain's bounds when
    # per_domain is set, so they are counted by the kernel (seed_flops).
    n = a[1]
    dims = list((ctypes.c_int32 * (n + 1)).from_address(a[0]))
    return mlp_crown_flops(dims, n, a[4], [0] * n, 0, a[15])


# Algorithmic work per launch, from the call's arguments (used by the
# optional per-entry-point timing below).
_FLOPS = {
    # 2 * M * n_out * n_in
    'vc_backward_fc': lambda a: 2.0 * a[1] * a[3] * a[11],
    'vc_mlp_crown': _flops_mlp_crown,
    'vc_mlp_tiled_crown': _flops_tiled_spec,
    'vc_mlp_crown_rows': _flops_tiled_spec,
}

_timing = None
_timing_when = {}
# Event pairs of earlier timing sessions, reused: creating a HIP event costs
# tens of microseconds of host time, which inside a timed region is time
# the GPU can spend idle.
_EV_FREE = []


def timing_begin(names, when=None):
    """Record HIP events around every call of the named entry points (on the
    current stream, which is the launch stream).  ``when``: {name:
    predicate(batch)}; a launch timed through timing_events on a batch the
    predicate rejects is not recorded."""
    global _timing, _timing_when
    _timing = {n: [] for n in names}
    _timing_when = dict(when or {})


def timing_end():
    """Stop recording; returns {name: {'launches', 'seconds', 'flops',
    'per_launch': [(seconds, flops, args), ...]}}."""
    global _timing
    rec, _timing = _timing, None
    torch.cuda.synchronize()
    out = {}
    for n, lst in (rec or {}).items():
        per = [(s.elapsed_time(e) / 1e3, f, a) for s, e, f, a, _ in lst]
        _EV_FREE.extend(pool for _, _, _, _, pool in lst)
        out[n] = {'launches': len(per), 'seconds': sum(p[0] for p in per),
                  'flops': sum(p[1] for p in per), 'per_launch': per}
    return out


def _event_pair():
    if _EV_FREE:
        return _EV_FREE.pop()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()  # creates the events; their user records them again
    e.record()
    return s, e


def timing_events(name, batch=None):
    """A recorded (start, end) event pair for a launch of `name` made inside
    another entry point, when `name` is being timed on this batch (else
    None)."""
    if _timing is None or name not in _timing:
        return None
    w = _timing_when.get(name)
    if w is not None and batch is not None and not w(batch):
        return None
    return _event_pair()


def timing_add(name, events, flops, args, pool=None):
    """File a launch timed with timing_events.  ``pool``: the event pair
    that goes back to the pool, when the span's (start, end) borrows an
    event of another record (default: the span's own pair)."""
    _timing[name].append((events[0], events[1], flops, args,
                          pool if pool is not None else tuple(events)))


def call(name, *args):
    lib = load()
    if _timing is not None and name in _timing:
        s, e = _event_pair()
        s.record()
        rc = getattr(lib, name)(*args)
        e.record()
        _timing[name].append((s, e, _FLOPS.get(name, lambda a: 0.0)(args), args, (s, e)))
        check(rc, name)
        return
    check(getattr(lib, name)(*args), name)


def ptr(t):
    """Device pointer of a contiguous GPU tensor (or None)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError('vibecheck_amd: tensor is not on the GPU '
                           '(the HIP library is the only compute path)')
    if not t.is_contiguous():
        raise ValueError('vibecheck_amd: tensor must be contiguous')
    return t.data_ptr()


def f32(t):
    """Contiguous fp32 GPU view of t (raises for other dtypes)."""
    if t is None:
        return None
    if t.dtype != torch.float32:
        raise NotImplementedError(
            f'vibecheck_amd computes in fp32 only, got {t.dtype}')
    if not t.is_cuda:
        raise RuntimeError('vibecheck_amd: tensor is not on the GPU '
                           '(the HIP library is the only compute path)')
    return t.contiguous()


def stream():
    """The current HIP stream of the current device (raw handle)."""
    return torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())
