"""vc_mlp_tiled_crown_noalloc (the CROWN bound with its scratch in a static
device array) against the allocating path it replaces
(vc_unstable_union_layers + vc_union_compact + vc_mlp_tiled_crown with
caller buffers): bit-identical bounds, spec bound, A and acc, on two calls
in a row, the second on a smaller batch (the array keeps the first call's
contents), through both CROWN kernels (one wavefront per domain above
4 x CUs domains, domains shared by a workgroup below)."""
import ctypes

import pytest
import torch

from vibecheck_amd import mlp_fused as mf
from vibecheck_amd import verify_zono_bnb as vz
from vibecheck_amd import workloads as wk
from vibecheck_amd._lib import call, host_array, ptr, stream

import _util

pytestmark = pytest.mark.gpu
F32 = torch.float32


def _noalloc(plan, xl, xh, sb, do_crown, per_domain, S, acc0):
    B = xl.shape[0]
    dev = xl.device
    Q = S.shape[0]
    lo_in = [sb[L][0].contiguous() for L in range(plan.n)]
    hi_in = [sb[L][1].contiguous() for L in range(plan.n)]
    lo_out = [torch.full_like(t, float('nan')) for t in lo_in]
    hi_out = [torch.full_like(t, float('nan')) for t in hi_in]
    lb = torch.full((B, Q), float('nan'), device=dev)
    A = torch.full((B, Q, plan.dims[0]), float('nan'), device=dev)
    acc = torch.full((B, Q), float('nan'), device=dev)
    keep = [host_array(ctypes.c_void_p, [ptr(t) for t in ts])
            for ts in (lo_in, hi_in, lo_out, hi_out)]
    call('vc_mlp_tiled_crown_noalloc', plan.dims_p, plan.n, ptr(plan.tfrag),
         ptr(plan.bias_cat), B, ptr(xl), ptr(xh), *[k[1] for k in keep],
         1 if do_crown else 0, 1 if per_domain else 0, Q, ptr(S), ptr(acc0), ptr(lb), ptr(A),
         ptr(acc), stream())
    tight = {L: (lo_out[L], hi_out[L]) for L in range(plan.n)} if do_crown else None
    return tight, lb, A, acc


@pytest.mark.parametrize('per_domain', [0, 1])
def test_crown_noalloc_matches_allocating_path(gpu, per_domain):
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    gg = wk.acas_gg(device=gpu, dtype=F32)
    plan = mf.plan_for(gg, gpu)
    assert plan is not None and plan.tfrag is not None
    se_c, _ = _util.spec_for(5, dtype=F32)
    se = {k: (w.to(gpu), b) for k, (w, b) in se_c.items()}
    Wq, bq = vz._spec_rows(se, gpu)
    S, acc0 = mf.fold_spec(plan, Wq, bq)
    for call_no, (B, seed) in enumerate(((4 * n_cu + 3000, 1), (max(64, 2 * n_cu + 5), 2))):
        print(f'call {call_no}: B={B} per_domain={per_domain}', flush=True)
        xl, xh = wk.acas_boxes(B, seed=seed, device=gpu, dtype=F32)
        c, r = (xl + xh) / 2, (xh - xl) / 2
        xl, xh = (c - 3 * r).contiguous(), (c + 3 * r).contiguous()
        sb = vz._zono_sb(gg, xl, xh, gpu, F32)
        want = mf.crown(plan, xl, xh, sb, True, spec=(Wq, bq), want_linear=True,
                        per_domain=bool(per_domain))
        got = _noalloc(plan, xl, xh, sb, True, per_domain, S, acc0)
        torch.cuda.synchronize()
        for L in range(plan.n):
            assert torch.equal(got[0][L][0], want[0][L][0]), (call_no, L, 'lo')
            assert torch.equal(got[0][L][1], want[0][L][1]), (call_no, L, 'hi')
        for k, what in ((1, 'lb'), (2, 'A'), (3, 'acc')):
            assert torch.equal(got[k], want[k]), (call_no, what)
        # the spec bound alone (no union in the scratch)
        want0 = mf.crown(plan, xl, xh, sb, False, spec=(Wq, bq), want_linear=True)
        got0 = _noalloc(plan, xl, xh, sb, False, per_domain, S, acc0)
        torch.cuda.synchronize()
        for k, what in ((1, 'lb'), (2, 'A'), (3, 'acc')):
            assert torch.equal(got0[k], want0[k]), (call_no, 'spec only', what)


def test_crown_noalloc_refuses_nets_beyond_its_scratch(gpu):
    """Both refusals come before any pointer is read or kernel launched:
    17 ReLU layers exceed the layer limit (16); 16 layers of 65 neurons
    (1,040 union entries) exceed the 1,024 (16 x 64) the array holds."""
    from vibecheck_amd import _lib
    for widths in ([64] * 17, [65] * 16):
        dims = host_array(ctypes.c_int32, [5] + widths)
        rc = _lib.load().vc_mlp_tiled_crown_noalloc(
            dims[1], len(widths), None, None, 1, None, None, None, None, None, None, 1, 0, 4,
            None, None, None, None, None, None)
        assert rc == _lib.VC_ERR_UNSUPPORTED, widths
