"""The small-channel transposed convolution as a GEMM and a fold
(k_conv_t_fold, behind vc_backward_conv for C_in <= 4, C_in kh kw <= 32,
C_out <= 64) and its fused form with the relu relaxation before it
(vc_backward_relu_conv), against torch's conv_transpose2d in fp64 on the
same fp32 inputs and against the separate relu and conv calls
(verify_zono_bnb.py:4409-4453, 4568-4593)."""
import pytest
import torch
import torch.nn.functional as F

from vibecheck_amd import verify_zono_bnb as vz
from vibecheck_amd import workloads as wk
from vibecheck_amd._lib import call, load, ptr

import _util
from test_gpu_parity import assert_interval, cpu

pytestmark = pytest.mark.gpu

# (C_in, H, W, C_out, k, stride, pad): the CIFAR CNN's first layer, an
# MNIST-style stride-2 layer, odd sizes (widths not a multiple of 4, C_out
# not a multiple of 4), C_out at the limit of 64, a 300-wide image (one
# source row per band), kernel equal to the stride, stride 3 with
# C_in kh kw = 32, a 1x1 source image, padding at or above the stride.
FOLD_GEOMS = [(3, 32, 32, 32, 3, 1, 1), (1, 28, 28, 16, 4, 2, 1), (2, 9, 11, 5, 3, 2, 1),
              (3, 8, 8, 64, 3, 1, 1), (1, 12, 300, 4, 3, 1, 1), (4, 10, 12, 8, 2, 2, 0),
              (2, 7, 9, 3, 4, 3, 2), (1, 5, 5, 2, 5, 1, 0), (1, 6, 7, 3, 3, 2, 2),
              (2, 9, 9, 4, 4, 2, 3)]


def _geom(geom):
    C_in, H, W, C_out, k, s, p = geom
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    return C_in, H, W, C_out, k, s, p, Ho, Wo


def _conv_t64(ew, K, s, p, H, W, Ho, Wo, k):
    oph, opw = H - ((Ho - 1) * s - 2 * p + k), W - ((Wo - 1) * s - 2 * p + k)
    return F.conv_transpose2d(ew, K, stride=s, padding=p, output_padding=(oph, opw))


def _backward_conv(dew, M, dK, db, geom, out, acc):
    C_in, H, W, C_out, k, s, p, Ho, Wo = _geom(geom)
    st = torch.cuda.current_stream().cuda_stream
    call('vc_backward_conv', ptr(dew), M, ptr(dK), ptr(db), C_out, Ho, Wo, C_in, H, W, k, k, s,
         s, p, p, ptr(out), ptr(acc), st)


@pytest.mark.parametrize('geom', FOLD_GEOMS)
def test_fold_against_fp64(gpu, geom):
    C_in, H, W, C_out, k, s, p, Ho, Wo = _geom(geom)
    assert load().vc_backward_relu_conv_ok(C_out, Ho, Wo, C_in, H, W, k, k, s, s, p, p) == 1
    g = torch.Generator().manual_seed(sum(geom))
    K = torch.randn(C_out, C_in, k, k, generator=g) / (C_in * k * k) ** 0.5
    bias = torch.randn(C_out, generator=g) * 0.1
    M = 7
    ew = torch.randn(M, C_out, Ho, Wo, generator=g)
    acc0 = torch.randn(M, generator=g)
    dK, db, dew = K.to(gpu), bias.to(gpu), ew.to(gpu)
    out = torch.full((M, C_in * H * W), float('nan'), device=gpu)
    acc = acc0.to(gpu)
    _backward_conv(dew, M, dK, db, geom, out, acc)
    K64 = K.double()
    ref = _conv_t64(ew.double(), K64, s, p, H, W, Ho, Wo, k).reshape(M, -1)
    sc = _conv_t64(ew.double().abs(), K64.abs(), s, p, H, W, Ho, Wo, k).reshape(M, -1)
    aref = acc0.double() + (ew.double() * bias.double().view(1, -1, 1, 1)).sum((1, 2, 3))
    asc = acc0.double().abs() + (ew.double().abs() * bias.double().abs().view(1, -1, 1, 1)).sum(
        (1, 2, 3))
    torch.cuda.synchronize()
    err = (cpu(out).double() - ref).abs()
    assert bool((err <= 1e-6 + 1e-5 * sc).all()), (geom, float(err.max()))
    aerr = (cpu(acc).double() - aref).abs()
    assert bool((aerr <= 1e-6 + 1e-5 * asc).all()), (geom, float(aerr.max()))
    # without a bias the accumulator is not touched (and may be absent)
    out2 = torch.empty_like(out)
    st = torch.cuda.current_stream().cuda_stream
    call('vc_backward_conv', ptr(dew), M, ptr(dK), None, C_out, Ho, Wo, C_in, H, W, k, k, s, s,
         p, p, ptr(out2), None, st)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)


def test_fold_rows_independent_of_batch(gpu):
    """Many more images than workgroups (each workgroup loops over images
    in an XCD-grouped order): every row equals the same row computed in a
    launch of its own, bit for bit, outputs and accumulators."""
    geom = FOLD_GEOMS[0]
    C_in, H, W, C_out, k, s, p, Ho, Wo = _geom(geom)
    g = torch.Generator(device=gpu).manual_seed(11)
    M = 5003
    dK = torch.randn(C_out, C_in, k, k, device=gpu, generator=g) * 0.2
    db = torch.randn(C_out, device=gpu, generator=g) * 0.1
    dew = torch.randn(M, C_out * Ho * Wo, device=gpu, generator=g)
    acc0 = torch.randn(M, device=gpu, generator=g)
    out = torch.empty(M, C_in * H * W, device=gpu)
    acc = acc0.clone()
    _backward_conv(dew, M, dK, db, geom, out, acc)
    for m0 in (0, 1234, 2500, M - 3):
        o1 = torch.empty(3, C_in * H * W, device=gpu)
        a1 = acc0[m0:m0 + 3].clone()
        _backward_conv(dew[m0:m0 + 3].contiguous(), 3, dK, db, geom, o1, a1)
        torch.cuda.synchronize()
        assert torch.equal(o1, out[m0:m0 + 3]) and torch.equal(a1, acc[m0:m0 + 3]), m0


def _relu_bounds(B, n, g, gpu):
    lo = torch.randn(B, n, device=gpu, generator=g)
    hi = lo + torch.rand(B, n, device=gpu, generator=g) * 2
    # exact zeros and ties at the slope's 0.5 threshold
    lo[:, :7] = 0.0
    hi[:, 7:11] = 0.0
    lo[:, 11:13], hi[:, 11:13] = -1.0, 1.0
    return lo, hi


@pytest.mark.parametrize('geom', [FOLD_GEOMS[0], FOLD_GEOMS[1], FOLD_GEOMS[2]])
@pytest.mark.parametrize('shared', [True, False])
@pytest.mark.parametrize('form', ['plain', 'alpha', 'beta'])
def test_relu_conv_fused_matches_separate(gpu, geom, shared, form):
    """vc_backward_relu_conv against vc_backward_relu then vc_backward_conv
    on the expanded rows: ew_out bit-identical, acc equal up to the order
    of its fp64 sums (one fp32 rounding step at most)."""
    _fused_vs_separate(gpu, geom, shared, form, 6, 5)


@pytest.mark.parametrize('B,R', [(10, 37), (64, 300)])
def test_relu_conv_fused_ragged_tiles(gpu, B, R):
    """Shared rows over more domains and rows than one image tile (8
    domains x about an XCD's workgroups), the last tiles ragged in both."""
    _fused_vs_separate(gpu, FOLD_GEOMS[0], True, 'plain', B, R)


def _fused_vs_separate(gpu, geom, shared, form, B, R):
    C_in, H, W, C_out, k, s, p, Ho, Wo = _geom(geom)
    n = C_out * Ho * Wo
    g = torch.Generator(device=gpu).manual_seed(sum(geom) + 7 * shared + B + R +
                                                  {'plain': 0, 'alpha': 1, 'beta': 2}[form])
    M = B * R
    dK = torch.randn(C_out, C_in, k, k, device=gpu, generator=g) * 0.3
    db = torch.randn(C_out, device=gpu, generator=g) * 0.1
    lo, hi = _relu_bounds(B, n, g, gpu)
    alpha = torch.rand(B, n, device=gpu, generator=g) if form == 'alpha' else None
    beta = torch.randn(B, n, device=gpu, generator=g) * 0.1 if form == 'beta' else None
    x = torch.randn(R if shared else M, n, device=gpu, generator=g)
    x[:, ::5] = 0.0
    acc0 = torch.randn(M, device=gpu, generator=g)
    st = torch.cuda.current_stream().cuda_stream
    # separate: expand, relu, conv
    xe = x.unsqueeze(0).expand(B, R, n).reshape(M, n).contiguous() if shared else x
    e = torch.empty(M, n, device=gpu)
    acc_ref = acc0.clone()
    call('vc_backward_relu', ptr(xe), M, R, n, ptr(lo), ptr(hi), ptr(alpha), 0, ptr(beta), ptr(e),
         ptr(acc_ref), st)
    out_ref = torch.empty(M, C_in * H * W, device=gpu)
    _backward_conv(e, M, dK, db, geom, out_ref, acc_ref)
    # fused
    ls, us, ut = (torch.empty(B, n, device=gpu) for _ in range(3))
    call('vc_relax_slopes', ptr(lo), ptr(hi), ptr(alpha), B * n, ptr(ls), ptr(us), ptr(ut), st)
    out = torch.full((M, C_in * H * W), float('nan'), device=gpu)
    acc = acc0.clone()
    call('vc_backward_relu_conv', ptr(x), M, R, 1 if shared else 0, ptr(ls), ptr(us), ptr(ut),
         ptr(beta), ptr(dK), ptr(db), C_out, Ho, Wo, C_in, H, W, k, k, s, s, p, p, ptr(out),
         ptr(acc), st)
    torch.cuda.synchronize()
    assert torch.equal(out, out_ref), (geom, shared, form)
    # one fp32 rounding after each of the two fp64 sums: a few ulps of the
    # magnitudes summed
    dom = torch.arange(M, device=gpu) // R
    s_relu = (xe.clamp(max=0).double() * ut[dom].double()).abs().sum(1)
    bias_el = db.repeat_interleave(Ho * Wo).double()
    s_bias = (e.double() * bias_el).abs().sum(1)
    tol = 4 * torch.finfo(torch.float32).eps * (acc0.double().abs() + s_relu + s_bias)
    d = (acc.double() - acc_ref.double()).abs()
    assert bool((d <= tol).all()), (geom, shared, form, float(d.max()))


def test_relu_conv_rejects_outside_geometry(gpu):
    """A geometry beyond the fused kernel's limits is refused with
    VC_ERR_UNSUPPORTED before any launch (the caller takes the separate
    calls)."""
    lib = load()
    assert lib.vc_backward_relu_conv_ok(32, 16, 16, 32, 32, 32, 4, 4, 2, 2, 1, 1) == 0  # C_in 32
    assert lib.vc_backward_relu_conv_ok(65, 8, 8, 3, 8, 8, 3, 3, 1, 1, 1, 1) == 0  # C_out 65
    assert lib.vc_backward_relu_conv_ok(8, 8, 8, 4, 8, 8, 3, 3, 1, 1, 1, 1) == 0  # C_in kh kw 36
    assert lib.vc_backward_relu_conv_ok(8, 8, 8, 3, 9, 8, 3, 3, 1, 1, 1, 1) == 0  # bad geometry
    x = torch.zeros(4, 32 * 16 * 16, device=gpu)
    z = torch.zeros(4, 32 * 16 * 16, device=gpu)
    K = torch.zeros(32, 32, 4, 4, device=gpu)
    out = torch.zeros(4, 32 * 32 * 32, device=gpu)
    acc = torch.zeros(4, device=gpu)
    rc = lib.vc_backward_relu_conv(ptr(x), 4, 4, 0, ptr(z), ptr(z), ptr(z), None, ptr(K), None,
                                   32, 16, 16, 32, 32, 32, 4, 4, 2, 2, 1, 1, ptr(out), ptr(acc),
                                   torch.cuda.current_stream().cuda_stream)
    assert rc != 0


def test_cnn_crown_fused_relu_conv_matches_unfused(gpu):
    """The CNN's CROWN intermediate bounds with the relu fused into the
    first layer's conv backward against the separate relu and conv calls
    (the oracle comparisons of the CNN run the fused form)."""
    gg_c = wk.cifar_cnn_gg(dtype=torch.float32)
    gg_g = _util.to_dev(gg_c, gpu)
    xl, xh = wk.cifar_cnn_boxes(3)
    dxl, dxh = xl.to(gpu), xh.to(gpu)
    ibp = vz._ibp_forward_graph_batched(dxl, dxh, gg_g, gpu, torch.float32)
    got = {}
    try:
        for fused in (True, False):
            vz.FUSED_RELU_CONV = fused
            got[fused] = vz._crown_intermediate_batched(gg_g, dxl, dxh, gpu, torch.float32,
                                                        sb=ibp)
    finally:
        vz.FUSED_RELU_CONV = True
    for L in got[True]:
        assert_interval(got[True][L], got[False][L], f'fused vs separate L{L}')
