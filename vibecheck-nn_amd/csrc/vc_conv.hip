// Convolution layers of the bound engine (NCHW, zero padding):
//   - interval forward: conv2d(mid, K) + bias -/+ conv2d(rad, |K|)
//     (verify_zono_bnb.py:1098-1107)
//   - zonotope forward on generator columns (verify_zono_bnb.py:3400-3425)
//   - CROWN backward: acc += ew . bias[channel], ew <- conv_transpose2d(ew)
//     (verify_zono_bnb.py:4568-4593)
// Direct forms: one thread per output element.
#include "vc_common.h"

namespace {

constexpr int NT = 256;

struct ConvGeom {
  int C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo;
};

__global__ void k_ibp_conv(const float* l, const float* h, int64_t B, ConvGeom g,
                           const float* K, const float* bias, float* lo, float* hi) {
  const int64_t n_out = (int64_t)g.C_out * g.Ho * g.Wo;
  const int64_t total = B * n_out;
  const int64_t n_in = (int64_t)g.C_in * g.H * g.W;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / n_out;
    const int o = (int)(i % n_out);
    const int co = o / (g.Ho * g.Wo);
    const int yo = (o / g.Wo) % g.Ho;
    const int xo = o % g.Wo;
    KSum sm, sr;
    const float* lb = l + b * n_in;
    const float* hb = h + b * n_in;
    for (int ci = 0; ci < g.C_in; ++ci)
      for (int ky = 0; ky < g.kh; ++ky) {
        const int yi = yo * g.sh - g.ph + ky;
        if (yi < 0 || yi >= g.H) continue;
        for (int kx = 0; kx < g.kw; ++kx) {
          const int xi = xo * g.sw - g.pw + kx;
          if (xi < 0 || xi >= g.W) continue;
          const int64_t e = ((int64_t)ci * g.H + yi) * g.W + xi;
          const float lv = lb[e], hv = hb[e];
          const float kv = K[((co * g.C_in + ci) * g.kh + ky) * g.kw + kx];
          sm.add(kv * ((lv + hv) / 2.f));
          sr.add(fabsf(kv) * ((hv - lv) / 2.f));
        }
      }
    const float mv = sm.value(), rv = sr.value();
    const float mc = bias ? mv + bias[co] : mv;
    lo[i] = mc - rv;
    hi[i] = mc + rv;
  }
}

// Zonotope generators: G (B, n_in, K) -> G_out (B, n_out, K), each
// generator column k of domain b convolved (no bias).
__global__ void k_zono_conv_gen(const float* G, int64_t B, int Kg, ConvGeom g, const float* K,
                                float* Go) {
  const int64_t n_out = (int64_t)g.C_out * g.Ho * g.Wo;
  const int64_t n_in = (int64_t)g.C_in * g.H * g.W;
  const int64_t total = B * n_out * Kg;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int k = (int)(i % Kg);
    const int64_t bo = i / Kg;
    const int64_t b = bo / n_out;
    const int o = (int)(bo % n_out);
    const int co = o / (g.Ho * g.Wo);
    const int yo = (o / g.Wo) % g.Ho;
    const int xo = o % g.Wo;
    KSum s;
    for (int ci = 0; ci < g.C_in; ++ci)
      for (int ky = 0; ky < g.kh; ++ky) {
        const int yi = yo * g.sh - g.ph + ky;
        if (yi < 0 || yi >= g.H) continue;
        for (int kx = 0; kx < g.kw; ++kx) {
          const int xi = xo * g.sw - g.pw + kx;
          if (xi < 0 || xi >= g.W) continue;
          const int64_t e = ((int64_t)ci * g.H + yi) * g.W + xi;
          s.add(K[((co * g.C_in + ci) * g.kh + ky) * g.kw + kx] * G[(b * n_in + e) * Kg + k]);
        }
      }
    Go[i] = s.value();
  }
}

__global__ void k_conv_center(const float* c, int64_t B, ConvGeom g, const float* K,
                              const float* bias, float* co_out) {
  const int64_t n_out = (int64_t)g.C_out * g.Ho * g.Wo;
  const int64_t n_in = (int64_t)g.C_in * g.H * g.W;
  const int64_t total = B * n_out;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / n_out;
    const int o = (int)(i % n_out);
    const int co = o / (g.Ho * g.Wo);
    const int yo = (o / g.Wo) % g.Ho;
    const int xo = o % g.Wo;
    KSum s;
    for (int ci = 0; ci < g.C_in; ++ci)
      for (int ky = 0; ky < g.kh; ++ky) {
        const int yi = yo * g.sh - g.ph + ky;
        if (yi < 0 || yi >= g.H) continue;
        for (int kx = 0; kx < g.kw; ++kx) {
          const int xi = xo * g.sw - g.pw + kx;
          if (xi < 0 || xi >= g.W) continue;
          s.add(K[((co * g.C_in + ci) * g.kh + ky) * g.kw + kx] *
                c[b * n_in + ((int64_t)ci * g.H + yi) * g.W + xi]);
        }
      }
    const float sv = s.value();
    co_out[i] = bias ? sv + bias[co] : sv;
  }
}

// Transposed conv: out[m, ci, yi, xi] = sum over (co, ky, kx) with
// yi = yo*sh - ph + ky, xi = xo*sw - pw + kx of ew[m, co, yo, xo] K[co, ci, ky, kx].
__global__ void k_conv_transpose(const float* ew, int64_t M, ConvGeom g, const float* K,
                                 float* out) {
  const int64_t n_out = (int64_t)g.C_out * g.Ho * g.Wo;
  const int64_t n_in = (int64_t)g.C_in * g.H * g.W;
  const int64_t total = M * n_in;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / n_in;
    const int e = (int)(i % n_in);
    const int ci = e / (g.H * g.W);
    const int yi = (e / g.W) % g.H;
    const int xi = e % g.W;
    KSum s;
    const float* em = ew + m * n_out;
    for (int ky = 0; ky < g.kh; ++ky) {
      const int ty = yi + g.ph - ky;
      if (ty < 0 || ty % g.sh) continue;
      const int yo = ty / g.sh;
      if (yo >= g.Ho) continue;
      for (int kx = 0; kx < g.kw; ++kx) {
        const int tx = xi + g.pw - kx;
        if (tx < 0 || tx % g.sw) continue;
        const int xo = tx / g.sw;
        if (xo >= g.Wo) continue;
        for (int co = 0; co < g.C_out; ++co)
          s.add(em[((int64_t)co * g.Ho + yo) * g.Wo + xo] *
                K[((co * g.C_in + ci) * g.kh + ky) * g.kw + kx]);
      }
    }
    out[i] = s.value();
  }
}

// acc[m] += sum_{co, p} ew[m, co, p] * bias[co]; one wave per row.
__global__ void k_conv_bias_dot(const float* ew, int64_t M, int C_out, int sp,
                                const float* bias, float* acc) {
  const int lane = threadIdx.x & 63;
  for (int64_t m = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6; m < M;
       m += ((int64_t)gridDim.x * blockDim.x) >> 6) {
    const int64_t n = (int64_t)C_out * sp;
    KSum ks;
    for (int64_t j = lane; j < n; j += 64) ks.add(ew[m * n + j] * bias[j / sp]);
    const float s = wave_sum_comp(ks);
    if (lane == 0) acc[m] += s;
  }
}

int check_geom(const ConvGeom& g) {
  if (g.C_in <= 0 || g.H <= 0 || g.W <= 0 || g.C_out <= 0 || g.kh <= 0 || g.kw <= 0 ||
      g.sh <= 0 || g.sw <= 0 || g.ph < 0 || g.pw < 0)
    return VC_ERR_ARG;
  if (g.Ho != (g.H + 2 * g.ph - g.kh) / g.sh + 1) return VC_ERR_ARG;
  if (g.Wo != (g.W + 2 * g.pw - g.kw) / g.sw + 1) return VC_ERR_ARG;
  if (g.Ho <= 0 || g.Wo <= 0) return VC_ERR_ARG;
  return VC_OK;
}

}  // namespace

extern "C" int vc_ibp_conv(const float* l, const float* h, int64_t B, int C_in, int H, int W,
                           const float* kernel, const float* bias, int C_out, int kh, int kw,
                           int sh, int sw, int ph, int pw, int H_out, int W_out, float* lo,
                           float* hi, vc_stream_t stream) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK || !l || !h || !kernel || !lo || !hi || B < 0) return VC_ERR_ARG;
  const int64_t total = B * (int64_t)C_out * H_out * W_out;
  if (total == 0) return VC_OK;
  hipLaunchKernelGGL(k_ibp_conv, dim3(vc_blocks(total, NT)), dim3(NT), 0, (hipStream_t)stream,
                     l, h, B, g, kernel, bias, lo, hi);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_zono_conv(const float* c, const float* G, int64_t B, int Kg, int C_in, int H,
                            int W, const float* kernel, const float* bias, int C_out, int kh,
                            int kw, int sh, int sw, int ph, int pw, int H_out, int W_out,
                            float* c_out, float* G_out, vc_stream_t stream) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK || !c || !kernel || !c_out || B < 0 || Kg < 0) return VC_ERR_ARG;
  if (Kg > 0 && (!G || !G_out)) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const int64_t total = B * (int64_t)C_out * H_out * W_out;
  if (total == 0) return VC_OK;
  hipLaunchKernelGGL(k_conv_center, dim3(vc_blocks(total, NT)), dim3(NT), 0, st, c, B, g,
                     kernel, bias, c_out);
  if (Kg > 0)
    hipLaunchKernelGGL(k_zono_conv_gen, dim3(vc_blocks(total * Kg, NT)), dim3(NT), 0, st, G,
                       B, Kg, g, kernel, G_out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_backward_conv(const float* ew_in, int64_t M, const float* kernel,
                                const float* bias, int C_out, int H_out, int W_out, int C_in,
                                int H, int W, int kh, int kw, int sh, int sw, int ph, int pw,
                                float* ew_out, float* acc, vc_stream_t stream) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK || !ew_in || !kernel || !ew_out || M < 0) return VC_ERR_ARG;
  if (bias && !acc) return VC_ERR_ARG;
  if (M == 0) return VC_OK;
  hipStream_t st = (hipStream_t)stream;
  if (bias)
    hipLaunchKernelGGL(k_conv_bias_dot, dim3(vc_blocks(M * 64, NT)), dim3(NT), 0, st, ew_in, M,
                       C_out, H_out * W_out, bias, acc);
  const int64_t total = M * (int64_t)C_in * H * W;
  hipLaunchKernelGGL(k_conv_transpose, dim3(vc_blocks(total, NT)), dim3(NT), 0, st, ew_in, M,
                     g, kernel, ew_out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}
