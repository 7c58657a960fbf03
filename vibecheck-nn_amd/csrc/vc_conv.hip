// Convolution layers of the bound engine (NCHW, zero padding) as implicit
// GEMMs on the MFMA core (vc_gemm_core.h): rows are output channels,
// columns are (image, output pixel[, generator column]), K runs over
// (input channel, kernel tap), and the B loader gathers the input pixels
// of a column (zero outside the image), so no im2col copy exists.
//   - interval forward: conv2d(mid, K) + bias -/+ conv2d(rad, |K|)
//     (verify_zono_bnb.py:1098-1107), both products in one launch;
//   - zonotope forward: conv2d(c, K) + bias and every generator column
//     convolved without bias (verify_zono_bnb.py:3400-3425);
//   - CROWN backward: acc += ew . bias[channel] and ew <- conv_transpose2d
//     (verify_zono_bnb.py:4568-4593).  The transposed convolution is split
//     by output parity (y mod sh, x mod sw) into sh * sw correlations, one
//     per batch index of the launch: output pixel (yy, xx) of class
//     (py, px) is y = sh yy + py, and only the taps ky = ky0 + sh ty with
//     ky0 = (py + ph) mod sh reach it, from source row yy + cy - ty with
//     cy = (py + ph - ky0) / sh (the same along x), so no zero tap is
//     multiplied.
#include "vc_gemm_core.h"
#include "vc_mlp_common.h"

namespace {

using namespace vcg;

struct ConvGeom {
  int C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo;
};

// Parity class bz of a transposed convolution along one dimension.
struct TapClass {
  int k0, c;  // first tap, source offset
};
__device__ __forceinline__ TapClass tap_class(int parity, int pad, int s) {
  const int k0 = (parity + pad) % s;
  return TapClass{k0, (parity + pad - k0) / s};
}

// ------------------------------------------------------------ B: gather
// Column n = (img * npix + pix) * nk + g, pix = py * Wg + px.  Element
// (k, n) = src[img * s_img + g + c * s_c + y * s_y + x * s_x] with
// c = k / T, t = k % T, ty = t / Tx, tx = t % Tx, y = py * psy + oy + dsg ty,
// x = px * psx + ox + dsg tx, zero outside [0, Hs) x [0, Ws).  TR: the
// offsets (oy, ox) are those of the transposed-convolution parity class bz
// (dsg = -1), else (-ph, -pw) (dsg = +1).  NS = 2 gathers two sources
// (interval lo, hi) into (mid, rad).
// ROWQ: every quad of columns is four consecutive pixels of one row (the
// host checked the grid width and pixel count are multiples of 4, nk = 1),
// so only the row path is compiled.
template <int NS, bool TR, bool ROWQ = false>
struct LoadGather {
  static constexpr bool kTrans = false;
  const float *src, *src2;
  int64_t s_img, s_c;
  int s_y, s_x, Hs, Ws;
  int nk, T, Tx, psy, psx, ph, pw, sh, sw, Wg;
  int64_t per_img;  // npix * nk
  FastDiv f_img, f_nk, f_wg, f_T, f_Tx;
  struct Col {
    int64_t off;
    int yb, xb, mode, n;
  };
  struct Raw {
    float x[NS][4];
  };
  __device__ void origin(int64_t bz, int& oy, int& ox) const {
    if (TR) {
      oy = tap_class((int)bz / sw, ph, sh).c;
      ox = tap_class((int)bz % sw, pw, sw).c;
    } else {
      oy = -ph;
      ox = -pw;
    }
  }
  __device__ void place(int n, int oy, int ox, int64_t& off, int& yb, int& xb, int& g,
                        int& px) const {
    const int img = (int)f_img.div((uint32_t)n);
    const int r = n - (int)(img * per_img);
    const int pix = (int)f_nk.div((uint32_t)r);
    g = r - pix * nk;
    const int py = (int)f_wg.div((uint32_t)pix);
    px = pix - py * Wg;
    off = img * s_img + g;
    yb = py * psy + oy;
    xb = px * psx + ox;
  }
  __device__ Col col(int64_t bz, int n) const {
    int oy, ox, g, px;
    Col c;
    origin(bz, oy, ox);
    place(n, oy, ox, c.off, c.yb, c.xb, g, px);
    c.n = n;
    // 0: the quad's columns are consecutive pixels of one row (step psx);
    // 1: consecutive generator columns of one pixel; 2: anything else
    c.mode = (nk == 1 && px + 3 < Wg) ? 0 : ((nk > 1 && g + 3 < nk) ? 1 : 2);
    c.mode |= (int)bz << 2;
    return c;
  }
  __device__ float at(const float* base, int y, int x) const {
    return ((unsigned)y < (unsigned)Hs && (unsigned)x < (unsigned)Ws) ? base[y * s_y + x * s_x]
                                                                      : 0.f;
  }
  template <bool VEC>
  __device__ void fetch(const Col& cl, int k, int cnt, Raw& r) const {
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) r.x[s][j] = 0.f;
    if (cnt == 0) return;
    const int c = (int)f_T.div((uint32_t)k);
    const int t = k - c * T;
    const int ty = (int)f_Tx.div((uint32_t)t);
    const int tx = t - ty * Tx;
    const int dy = TR ? -ty : ty, dx = TR ? -tx : tx;
    const int mode = ROWQ ? 0 : (cl.mode & 3);
    if (mode == 2) {
      int oy, ox;
      origin(cl.mode >> 2, oy, ox);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j < cnt) {
          int64_t off;
          int yb, xb, g, px;
          place(cl.n + j, oy, ox, off, yb, xb, g, px);
          r.x[0][j] = at(src + off + c * s_c, yb + dy, xb + dx);
          if (NS == 2) r.x[NS - 1][j] = at(src2 + off + c * s_c, yb + dy, xb + dx);
        }
      }
      return;
    }
    const int y = cl.yb + dy;
    const float* b1 = src + cl.off + c * s_c;
    const float* b2 = NS == 2 ? src2 + cl.off + c * s_c : nullptr;
    if (TR && NS == 1 && mode == 0 && cnt == 4) {
      // the transposed conv's rows are contiguous (unit pixel steps): a
      // quad inside the image is four consecutive floats, one 16-byte load
      // when aligned, else four loads without bounds checks
      const int x0 = cl.xb + dx;
      if ((unsigned)y < (unsigned)Hs && x0 >= 0 && x0 + 3 < Ws) {
        const float* p = b1 + y * s_y + x0;
        if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
          const float4 v = *reinterpret_cast<const float4*>(p);
          r.x[0][0] = v.x, r.x[0][1] = v.y, r.x[0][2] = v.z, r.x[0][3] = v.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) r.x[0][j] = p[j];
        }
        return;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < cnt) {
        const int x = cl.xb + dx + (mode == 0 ? psx * j : 0);
        const int gj = mode == 1 ? j : 0;
        r.x[0][j] = at(b1 + gj, y, x);
        if (NS == 2) r.x[NS - 1][j] = at(b2 + gj, y, x);
      }
    }
  }
  __device__ static void finish(const Raw& r, float (*v)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (NS == 2) {
        v[0][j] = (r.x[0][j] + r.x[NS - 1][j]) / 2.f;
        v[NS - 1][j] = (r.x[NS - 1][j] - r.x[0][j]) / 2.f;
      } else {
        v[0][j] = r.x[0][j];
      }
    }
  }
};

// ------------------------------------------------------------ A: weights
// Forward: A = K viewed (C_out, C_in kh kw), rows co; with NA = 2 the
// second operand is |K| (the interval radius product).
template <int NA>
struct LoadKernel {
  static constexpr int kBK = 32;
  static constexpr bool kSmallM = true;
  const float* K;
  int ld;
  struct Row {
    int64_t o;
  };
  struct Raw {
    float x[4];
  };
  __device__ Row row(int64_t, int64_t m, bool) const { return Row{m * ld}; }
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    ld4<false>(K + rw.o + k, n, x.x);
  }
  template <bool VEC>
  __device__ void finish(const Row&, int, int, const Raw& x, float (*v)[4], KSum&, bool) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[0][j] = x.x[j];
      if (NA == 2) v[NA - 1][j] = fabsf(x.x[j]);
    }
  }
};

// Transposed, parity class bz: A[ci][(co, ty, tx)] = K[co][ci][ky0 + sh ty]
// [kx0 + sw tx], zero for taps past the kernel (classes with fewer taps).
struct LoadKernelT {
  static constexpr int kBK = 32;
  static constexpr bool kSmallM = true;
  const float* K;
  int C_in, kh, kw, sh, sw, ph, pw, T, Tx, Ty;
  FastDiv f_T, f_Tx;
  struct Row {
    int ci, ky0, kx0;
  };
  struct Raw {
    float x[4];
  };
  __device__ Row row(int64_t bz, int64_t m, bool) const {
    return Row{(int)m, tap_class((int)bz / sw, ph, sh).k0, tap_class((int)bz % sw, pw, sw).k0};
  }
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    int co = (int)f_T.div((uint32_t)k);
    const int t = k - co * T;
    int ty = (int)f_Tx.div((uint32_t)t);
    int tx = t - ty * Tx;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = 0.f;
      const int ky = rw.ky0 + sh * ty, kx = rw.kx0 + sw * tx;
      if (j < n && ky < kh && kx < kw) v = K[(((int64_t)co * C_in + rw.ci) * kh + ky) * kw + kx];
      x.x[j] = v;
      if (++tx == Tx) {
        tx = 0;
        if (++ty == Ty) {
          ty = 0;
          ++co;
        }
      }
    }
  }
  template <bool VEC>
  __device__ void finish(const Row&, int, int, const Raw& x, float (*v)[4], KSum&, bool) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[0][j] = x.x[j];
  }
};

// Pre-packed transposed taps (vc_conv_t_pack): class bz's A rows at
// A + bz * cs, row ci at ci * ld, so the loader does no tap arithmetic.
// The same values in the same k order as LoadKernelT, the same K-tiles.
struct LoadPackedT {
  static constexpr int kBK = 32;
  static constexpr bool kSmallM = true;
  const float* A;
  int64_t cs;  // floats per parity class
  int ld;      // floats per row (Kd rounded up to 4)
  struct Row {
    int64_t o;
  };
  struct Raw {
    float x[4];
  };
  __device__ Row row(int64_t bz, int64_t m, bool) const { return Row{bz * cs + m * ld}; }
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    // rows are 16-byte aligned (ld a multiple of 4, A from the allocator)
    ld4<true>(A + rw.o + k, n, x.x);
  }
  template <bool VEC>
  __device__ void finish(const Row&, int, int, const Raw& x, float (*v)[4], KSum&, bool) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[0][j] = x.x[j];
  }
};

// A[bz][ci][(co, ty, tx)] = K[co][ci][ky0 + sh ty][kx0 + sw tx] for every
// parity class bz (LoadKernelT's values), zero past the kernel and in the
// row padding.
__global__ void k_conv_t_pack(const float* __restrict__ K, ConvGeom g, int Ty, int Tx, int ld,
                              float* __restrict__ out) {
  const int classes = g.sh * g.sw;
  const int64_t total = (int64_t)classes * g.C_in * ld;
  const int Kd = g.C_out * Ty * Tx;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int k = (int)(t % ld);
    const int64_t rest = t / ld;
    const int ci = (int)(rest % g.C_in);
    const int bz = (int)(rest / g.C_in);
    float v = 0.f;
    if (k < Kd) {
      const int co = k / (Ty * Tx), tt = k % (Ty * Tx);
      const int ty = tt / Tx, tx = tt % Tx;
      const int ky = tap_class(bz / g.sw, g.ph, g.sh).k0 + g.sh * ty;
      const int kx = tap_class(bz % g.sw, g.pw, g.sw).k0 + g.sw * tx;
      if (ky < g.kh && kx < g.kw) v = K[(((int64_t)co * g.C_in + ci) * g.kh + ky) * g.kw + kx];
    }
    out[t] = v;
  }
}

// ------------------------------------------------------------ epilogues
// Forward outputs: column n = img * per_img + r -> out[img * o_img + m * o_c + r]
// (r = pix * nk + g).  NA = 2: interval (lo, hi) = mid + bias -/+ rad.
template <int NA>
struct EpConv {
  const float* bias;
  float *out, *out2;
  int64_t per_img, o_img, o_c;
  FastDiv f_img;
  __device__ void operator()(int64_t, int64_t m, int n, const float* c) const {
    const int img = (int)f_img.div((uint32_t)n);
    const int64_t r = n - img * per_img;
    const int64_t o = img * o_img + m * o_c + r;
    const float mc = bias ? c[0] + bias[m] : c[0];
    if (NA == 2) {
      out[o] = mc - c[NA - 1];
      out2[o] = mc + c[NA - 1];
    } else {
      out[o] = mc;
    }
  }
};

// Transposed outputs of parity class bz: column n = (img, yy, xx) on the
// class grid (Hc, Wc) -> out[img][ci = m][sh yy + py][sw xx + px], inside H x W.
struct EpConvT {
  float* out;
  int H, W, Wc, sh, sw;
  int64_t per_img, o_img;
  FastDiv f_img, f_wc;
  __device__ void operator()(int64_t bz, int64_t m, int n, const float* c) const {
    const int img = (int)f_img.div((uint32_t)n);
    const int pix = n - (int)(img * per_img);
    const int yy = (int)f_wc.div((uint32_t)pix);
    const int xx = pix - yy * Wc;
    const int y = sh * yy + (int)bz / sw, x = sw * xx + (int)bz % sw;
    if (y < H && x < W) out[img * o_img + (m * H + y) * (int64_t)W + x] = c[0];
  }
};

// Transposed convolution onto few channels (C_in <= 4, the network's
// input layer): an MFMA tile would hold C_in of its 64 rows, so one thread
// takes one output pixel of one row and all CI channels.  The kernel taps
// sit in LDS as doubles; products and sums are fp64 FMAs, rounded once.
// Neighbouring threads read neighbouring source pixels.
constexpr int kSmallC = 4;
constexpr int kSmallCLds = 48 * 1024;  // bytes of LDS for the taps

template <int CI>
__global__ __launch_bounds__(NT) void k_conv_t_smallc(const float* ew, int64_t M, ConvGeom g,
                                                      const float* K, float* out) {
  extern __shared__ double wd[];  // [C_out][kh][kw][CI]
  const int taps = g.C_out * g.kh * g.kw;
  for (int i = threadIdx.x; i < taps * CI; i += NT) {
    const int ci = i % CI, r = i / CI;
    const int kx = r % g.kw, ky = (r / g.kw) % g.kh, co = r / (g.kw * g.kh);
    wd[i] = (double)K[((co * g.C_in + ci) * g.kh + ky) * g.kw + kx];
  }
  __syncthreads();
  const int64_t hw = (int64_t)g.H * g.W, total = M * hw;
  const int64_t so = (int64_t)g.Ho * g.Wo;
  for (int64_t i = blockIdx.x * (int64_t)NT + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * NT) {
    const int64_t m = i / hw;
    const int p = (int)(i - m * hw);
    const int y = p / g.W, x = p - (p / g.W) * g.W;
    double acc[CI];
#pragma unroll
    for (int c = 0; c < CI; ++c) acc[c] = 0.0;
    const float* em = ew + m * g.C_out * so;
    for (int ky = 0; ky < g.kh; ++ky) {
      const int ty = y + g.ph - ky;
      if (ty < 0 || ty % g.sh) continue;
      const int oy = ty / g.sh;
      if (oy >= g.Ho) continue;
      for (int kx = 0; kx < g.kw; ++kx) {
        const int tx = x + g.pw - kx;
        if (tx < 0 || tx % g.sw) continue;
        const int ox = tx / g.sw;
        if (ox >= g.Wo) continue;
        const float* e = em + oy * g.Wo + ox;
        const double* w = wd + (ky * g.kw + kx) * CI;
        const int wstep = g.kh * g.kw * CI;
        int co = 0;
        for (; co + 8 <= g.C_out; co += 8) {  // eight loads in flight
          float v8[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v8[u] = e[(co + u) * so];
#pragma unroll
          for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int c = 0; c < CI; ++c)
              acc[c] = __builtin_fma((double)v8[u], w[(co + u) * wstep + c], acc[c]);
        }
        for (; co < g.C_out; ++co) {
          const double v = (double)e[co * so];
#pragma unroll
          for (int c = 0; c < CI; ++c) acc[c] = __builtin_fma(v, w[co * wstep + c], acc[c]);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CI; ++c) out[(m * g.C_in + c) * hw + p] = (float)acc[c];
  }
}

// Transposed convolution onto few values per tap set (C_in kh kw <= 32, the
// network's input layer) as a GEMM and a fold (the conv branch of the
// backward, verify_zono_bnb.py:4568-4593, and in the fused form the relu
// branch before it, :4409-4453).  Per image, first
//   Y[(ci, ky, kx), q] = sum_co K[co, ci, ky, kx] e[co, q]
// over the source pixels q on the MFMA (M = C_in kh kw in MT tiles of 16
// rows, K = C_out, N = source pixels), then
//   out[ci, y, x] = sum of Y[(ci, ky, kx), (qy, qx)] over the taps with
//   sh qy = y + ph - ky and sw qx = x + pw - kx inside the source image,
// the tap sum in fp64, rounded once (each Y value is an fp32 MFMA sum over
// C_out <= 64 products).  Each source value is loaded once, so the conv
// bias dot (acc += e . bias[co], as k_conv_bias_dot) and, in the fused
// form, the ReLU relaxation that produces e from the rows x above the
// ReLU (e = pos(x) lo_s + neg(x) up_s [+ beta], acc += neg(x) up_t, the
// arithmetic of the relu backward) ride on that load.
// A workgroup takes one image at a time: source rows in bands of BS whose
// Y go to an LDS ring of RS >= BS + (kh - 1) / sh rows; after each band the
// output rows whose taps all lie in the ring are folded and stored.  A
// wave's 64 source pixels per pass are c0 + 4 r + j (lane column r of
// N-tile j), so a lane's four consecutive pixels are one 16-byte load.
constexpr int kFoldNT = 256;
constexpr int kFoldMaxMF = 32;
constexpr int kFoldMaxCout = 64;
constexpr int kFoldMaxLds = 64 * 1024;

struct FoldArgs {
  const float* ew;  // R rows (shared) or M rows of C_out Ho Wo
  int64_t M, R, B;  // rows out, rows per domain, domains (M / R)
  int shared;
  const float *ls, *us, *ut, *beta;  // (B, C_out Ho Wo) slopes and beta, or null
  const float* K;                    // (C_out, C_in, kh, kw)
  const float* bias;                 // (C_out) or null
  float* out;                        // (M, C_in H W)
  float* acc;                        // (M)
  int C_out, Ho, Wo, C_in, H, W, kh, kw, sh, sw, ph, pw;
  int MF, nks, BS, RS;
  int hl, hr;  // zero columns left and right of each Y ring row
  int DB, SB;  // image tile (shared rows): domains x rows
  int ndb;     // tiles along the domains
  int64_t total;  // image slots (M, or whole tiles)
  FastDiv f_W, f_Wo, f_RS, f_sh, f_sw, f_R, f_DB, f_ndb, f_tile;
};

__device__ __forceinline__ float neg_of(float a) { return a > 0.f ? 0.f : a; }

// One K-step's operands of a lane: its quad of source values (channel
// co = 4 ks + gq, pixels pq .. pq + 3) and, fused, their slopes and beta.
// The bases are uniform over the workgroup, the offsets 32-bit.
struct FoldLd {
  float x[4], l[4], u[4], t[4], b[4];
};

struct FoldSrc {
  const float *x, *l, *u, *t, *b;  // the image's row and its domain's slopes (b may be null)
};

// FULL: every lane of the wave in range (a uniform fact of the chunk and the
// channel count): no masks, no zero fills.  RL: 0 plain, 1 relu, 2 relu +
// beta.
template <int RL, bool VEC, bool FULL>
__device__ __forceinline__ void fold_load(const FoldSrc& sp, int C_out, int HoWo, int pq,
                                          int p_hi, int ks, int gq, FoldLd& d) {
  const int co = 4 * ks + gq;
  const uint32_t off = (uint32_t)(co * HoWo + pq);
  if (!FULL) {
#pragma unroll
    for (int j = 0; j < 4; ++j) d.x[j] = d.l[j] = d.u[j] = d.t[j] = d.b[j] = 0.f;
    if (co >= C_out) return;
  }
  if (VEC) {
    if (!FULL && pq >= p_hi) return;  // p_hi and pq are multiples of 4: the whole quad
    const float4 v = *reinterpret_cast<const float4*>(sp.x + off);
    d.x[0] = v.x, d.x[1] = v.y, d.x[2] = v.z, d.x[3] = v.w;
    if (RL > 0) {
      const float4 lv = *reinterpret_cast<const float4*>(sp.l + off);
      const float4 uv = *reinterpret_cast<const float4*>(sp.u + off);
      const float4 tv = *reinterpret_cast<const float4*>(sp.t + off);
      d.l[0] = lv.x, d.l[1] = lv.y, d.l[2] = lv.z, d.l[3] = lv.w;
      d.u[0] = uv.x, d.u[1] = uv.y, d.u[2] = uv.z, d.u[3] = uv.w;
      d.t[0] = tv.x, d.t[1] = tv.y, d.t[2] = tv.z, d.t[3] = tv.w;
    }
    if (RL == 2) {
      const float4 bv = *reinterpret_cast<const float4*>(sp.b + off);
      d.b[0] = bv.x, d.b[1] = bv.y, d.b[2] = bv.z, d.b[3] = bv.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (pq + j < p_hi) {
        d.x[j] = sp.x[off + j];
        if (RL > 0) {
          d.l[j] = sp.l[off + j];
          d.u[j] = sp.u[off + j];
          d.t[j] = sp.t[off + j];
        }
        if (RL == 2) d.b[j] = sp.b[off + j];
      }
  }
}

// The K-step: relax (fused form), the bias dot, MT x 4 MFMAs.  Elements
// outside the image or channel range hold zeros and add nothing.
template <int MT, int RL>
__device__ __forceinline__ void fold_use(const float* As, const float* Bsh, bool has_bias,
                                         int lane, int ks, int gq, FoldLd& d, v4f (*yt)[4],
                                         double& p_relu, double& p_bias) {
  if (RL > 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // pos(x) lo_s + neg(x) up_s with one of the two parts zero: the
      // nonzero product itself (the same value; a zero may differ in sign)
      const float x = d.x[j];
      float e = x * (x < 0.f ? d.u[j] : d.l[j]);
      if (RL == 2) e = e + d.b[j];
      p_relu += (double)(neg_of(x) * d.t[j]);
      d.x[j] = e;
    }
  }
  if (has_bias) {
    const float bc = Bsh[4 * ks + gq];  // zero past C_out
#pragma unroll
    for (int j = 0; j < 4; ++j) p_bias += (double)(d.x[j] * bc);
  }
  float af[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) af[mt] = As[(ks * MT + mt) * 64 + lane];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) yt[mt][j] = mfma16x16x4(af[mt], d.x[j], yt[mt][j]);
}

// The Y ring: for each m, RS rows of Wp = hl + Wo + hr columns (source
// column qx at hl + qx, hl = Tx - 1 zero columns on the left, hr on the
// right: every column a fold reads exists) and one zero row (slot RS), the
// target of every tap outside the kernel or the source rows.  Zeroed once;
// Y stores write only the interior.
template <int MT, int RL, bool VEC>
__global__ __launch_bounds__(kFoldNT) void k_conv_t_fold(FoldArgs a) {
  constexpr bool RELU = RL > 0;
  extern __shared__ __align__(16) float lds[];
  __shared__ double red[2][kFoldNT / 64];
  float* As = lds;                    // [nks][MT][64]: lane l's A value of K-step ks, tile mt
  float* Bsh = As + a.nks * MT * 64;  // [4 nks]: the bias, zero past C_out
  float* Yr = Bsh + a.nks * 4;        // [MF][RS + 1][Wp]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int gq = lane >> 4, r = lane & 15;
  const int HoWo = a.Ho * a.Wo;
  const int64_t n_e = (int64_t)a.C_out * HoWo;
  const int64_t n_o = (int64_t)a.C_in * a.H * a.W;
  const int Wp = a.hl + a.Wo + a.hr;
  const int ringsz = (a.RS + 1) * Wp;
  const int kk = a.kh * a.kw;
  const int Ty = (a.kh + a.sh - 1) / a.sh, Tx = (a.kw + a.sw - 1) / a.sw;
  // A[m][co] = K[co][ci][ky][kx] with m = (ci kh + ky) kw + kx, i.e. K[co MF + m]
  for (int i = tid; i < a.nks * MT * 64; i += kFoldNT) {
    const int l = i & 63, mt = (i >> 6) % MT, ks = (i >> 6) / MT;
    const int co = 4 * ks + (l >> 4), m = 16 * mt + (l & 15);
    As[i] = (co < a.C_out && m < a.MF) ? a.K[(int64_t)co * a.MF + m] : 0.f;
  }
  for (int i = tid; i < a.nks * 4; i += kFoldNT) Bsh[i] = (a.bias && i < a.C_out) ? a.bias[i] : 0.f;
  for (int i = tid; i < a.MF * ringsz; i += kFoldNT) Yr[i] = 0.f;
  __syncthreads();
  // Shared source rows: the images run in tiles of DB domains x SB rows,
  // about the images in flight on one XCD, so that its L2 serves both the
  // DB domains' slopes and the SB rows to the whole tile (ragged tiles skip
  // their missing images).  Per-domain rows run in row order.
  // (image counts below 2^31: 32-bit index arithmetic)
  for (int64_t t = blockIdx.x; t < a.total; t += gridDim.x) {
    const uint32_t w = (uint32_t)xcd_tile(t, a.total);
    int64_t m, src;
    if (a.shared) {
      const uint32_t tl = a.f_tile.div(w), in = w - tl * a.DB * a.SB;
      const uint32_t sb = a.f_ndb.div(tl), ib = a.f_DB.div(in);
      const uint32_t b = (tl - sb * a.ndb) * a.DB + (in - ib * a.DB), s = sb * a.SB + ib;
      if (b >= (uint32_t)a.B || s >= (uint32_t)a.R) continue;
      m = (int64_t)b * a.R + s;
      src = s;
    } else {
      m = w;
      src = w;
    }
    FoldSrc sp;
    sp.x = a.ew + src * n_e;
    if (RELU) {
      const int64_t so = (int64_t)a.f_R.div((uint32_t)m) * n_e;
      sp.l = a.ls + so;
      sp.u = a.us + so;
      sp.t = a.ut + so;
      sp.b = a.beta ? a.beta + so : nullptr;
    } else {
      sp.l = sp.u = sp.t = sp.b = nullptr;
    }
    float* orow = a.out + m * n_o;
    double p_relu = 0.0, p_bias = 0.0;
    int yo = 0;
    for (int q0 = 0; q0 < a.Ho; q0 += a.BS) {
      const int qe = min(a.Ho, q0 + a.BS);
      const int p_hi = qe * a.Wo;
      for (int c0 = q0 * a.Wo + 64 * wv; c0 < p_hi; c0 += kFoldNT) {
        const int pq = c0 + 4 * r;
        v4f yt[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < 4; ++j) yt[mt][j] = v4f{0.f, 0.f, 0.f, 0.f};
        if (VEC && c0 + 63 < p_hi && (a.C_out & 3) == 0) {
          // the next K-step's loads in flight during this one's arithmetic
          // (the last step reloads itself: always in range)
          FoldLd cur;
          fold_load<RL, VEC, true>(sp, a.C_out, HoWo, pq, p_hi, 0, gq, cur);
          for (int ks = 0; ks < a.nks; ++ks) {
            FoldLd nxt;
            fold_load<RL, VEC, true>(sp, a.C_out, HoWo, pq, p_hi, min(ks + 1, a.nks - 1), gq, nxt);
            fold_use<MT, RL>(As, Bsh, a.bias != nullptr, lane, ks, gq, cur, yt, p_relu, p_bias);
            cur = nxt;
          }
        } else {
          for (int ks = 0; ks < a.nks; ++ks) {
            FoldLd d;
            fold_load<RL, VEC, false>(sp, a.C_out, HoWo, pq, p_hi, ks, gq, d);
            fold_use<MT, RL>(As, Bsh, a.bias != nullptr, lane, ks, gq, d, yt, p_relu, p_bias);
          }
        }
        // lane (gq, r) holds Y[16 mt + 4 gq + e][pq + j] in yt[mt][j][e]; with
        // Wo a multiple of 4 (VEC) the quad lies in one source row
        const int qyq = (int)a.f_Wo.div((uint32_t)pq);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int p = pq + j;
          if (p < p_hi) {
            const int qy = VEC ? qyq : (int)a.f_Wo.div((uint32_t)p), qx = p - qy * a.Wo;
            const int slot = qy - (int)a.f_RS.div((uint32_t)qy) * a.RS;
            float* yp = Yr + slot * Wp + a.hl + qx;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int mm = 16 * mt + 4 * gq + e;
                if (mm < a.MF) yp[mm * ringsz] = yt[mt][j][e];
              }
          }
        }
      }
      __syncthreads();
      // output rows y < sh qe - ph take taps from source rows < qe only
      int ye = qe == a.Ho ? a.H : min(a.H, a.sh * qe - a.ph);
      if (ye < yo) ye = yo;
      const int cnt = (ye - yo) * a.W;
      for (int i = tid; i < cnt; i += kFoldNT) {
        const int dy = (int)a.f_W.div((uint32_t)i), x = i - dy * a.W, y = yo + dy;
        const int ty0 = y + a.ph, tx0 = x + a.pw;
        const int qy0 = (int)a.f_sh.div((uint32_t)ty0), ky0 = ty0 - qy0 * a.sh;
        const int qx0 = (int)a.f_sw.div((uint32_t)tx0), kx0 = tx0 - qx0 * a.sw;
        double sum[kSmallC];
#pragma unroll
        for (int c = 0; c < kSmallC; ++c) sum[c] = 0.0;
        for (int ty = 0; ty < Ty; ++ty) {
          const int ky = ky0 + a.sh * ty, qy = qy0 - ty;
          const bool vy = ky < a.kh && qy >= 0 && qy < a.Ho;
          const int row = vy ? (qy - (int)a.f_RS.div((uint32_t)qy) * a.RS) : a.RS;
          const int kyc = vy ? ky : 0;
          for (int tx = 0; tx < Tx; ++tx) {
            const int kx = kx0 + a.sw * tx;
            const bool v = vy && kx < a.kw;
            const int off = (kyc * a.kw + (v ? kx : 0)) * ringsz + (v ? row : a.RS) * Wp + a.hl +
                            qx0 - tx;
#pragma unroll
            for (int c = 0; c < kSmallC; ++c)
              if (c < a.C_in) sum[c] += (double)Yr[c * kk * ringsz + off];
          }
        }
        float* op = orow + (int64_t)y * a.W + x;
#pragma unroll
        for (int c = 0; c < kSmallC; ++c)
          if (c < a.C_in) op[(int64_t)c * a.H * a.W] = (float)sum[c];
      }
      yo = ye;
      __syncthreads();
    }
    if (RELU || a.bias) {
      // the relu's intercepts, then the bias dot, each rounded into acc as
      // the two separate steps round them
      p_relu = wave_sum_f64(p_relu);
      p_bias = wave_sum_f64(p_bias);
      if (lane == 0) {
        red[0][wv] = p_relu;
        red[1][wv] = p_bias;
      }
      __syncthreads();
      if (tid == 0) {
        float v = a.acc[m];
        if (RELU) v = (float)((double)v + ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])));
        if (a.bias) v = (float)((double)v + ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])));
        a.acc[m] = v;
      }
    }
  }
}

// acc[m] += sum_{co, p} ew[m, co, p] * bias[co].  One workgroup per row
// (rows of a conv layer are tens of thousands of values long); products in
// fp32 as the reference's (ew * bias_flat) forms them, summed in fp64,
// reduced over the workgroup in a fixed order.
template <bool VEC>
__global__ __launch_bounds__(NT) void k_conv_bias_dot(const float* ew, int64_t M, int C_out,
                                                      int sp, FastDiv f_sp, const float* bias,
                                                      float* acc) {
  __shared__ double red[NT / 64];
  const int64_t n = (int64_t)C_out * sp;
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    const float* row = ew + m * n;
    double p = 0.0;
    if (VEC) {
      for (int64_t q = threadIdx.x; 4 * q < n; q += NT) {
        const float4 v = reinterpret_cast<const float4*>(row)[q];
        const uint32_t j = (uint32_t)(4 * q);
        p += (double)(v.x * bias[f_sp.div(j)]);
        p += (double)(v.y * bias[f_sp.div(j + 1)]);
        p += (double)(v.z * bias[f_sp.div(j + 2)]);
        p += (double)(v.w * bias[f_sp.div(j + 3)]);
      }
    } else {
      for (int64_t j = threadIdx.x; j < n; j += NT)
        p += (double)(row[j] * bias[f_sp.div((uint32_t)j)]);
    }
    p = wave_sum_f64(p);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = p;
    __syncthreads();
    if (threadIdx.x == 0)
      acc[m] = (float)((double)acc[m] + ((red[0] + red[1]) + (red[2] + red[3])));
    __syncthreads();
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

// Columns and K of one implicit GEMM must fit the core's int indices (and
// the 31-bit range of FastDiv).
constexpr int64_t kMaxDim = (int64_t(1) << 31) - 1;

// The gather of a forward convolution over images of (C_in, H, W) laid out
// with the given strides; nk generator columns per pixel.
template <int NS>
LoadGather<NS, false> forward_gather(const ConvGeom& g, const float* src, const float* src2,
                                     int64_t s_img, int64_t s_c, int s_y, int s_x, int nk) {
  LoadGather<NS, false> b{};
  b.src = src;
  b.src2 = src2;
  b.s_img = s_img;
  b.s_c = s_c;
  b.s_y = s_y;
  b.s_x = s_x;
  b.Hs = g.H;
  b.Ws = g.W;
  b.nk = nk;
  b.T = g.kh * g.kw;
  b.Tx = g.kw;
  b.psy = g.sh;
  b.psx = g.sw;
  b.ph = g.ph;
  b.pw = g.pw;
  b.sh = g.sh;
  b.sw = g.sw;
  b.Wg = g.Wo;
  b.per_img = (int64_t)g.Ho * g.Wo * nk;
  b.f_img = FastDiv::make((uint32_t)b.per_img);
  b.f_nk = FastDiv::make((uint32_t)nk);
  b.f_wg = FastDiv::make((uint32_t)g.Wo);
  b.f_T = FastDiv::make((uint32_t)b.T);
  b.f_Tx = FastDiv::make((uint32_t)b.Tx);
  return b;
}

}  // namespace

extern "C" int vc_ibp_conv(const float* l, const float* h, int64_t B, int C_in, int H, int W,
                           const float* kernel, const float* bias, int C_out, int kh, int kw,
                           int sh, int sw, int ph, int pw, int H_out, int W_out, float* lo,
                           float* hi, vc_stream_t stream) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK || !l || !h || !kernel || !lo || !hi || B < 0) return VC_ERR_ARG;
  const int64_t npix = (int64_t)H_out * W_out, N = B * npix, Kd = (int64_t)C_in * kh * kw;
  if (N == 0) return VC_OK;
  if (N > kMaxDim || Kd > kMaxDim) return VC_ERR_UNSUPPORTED;
  const int64_t n_in = (int64_t)C_in * H * W;
  auto gb = forward_gather<2>(g, l, h, n_in, (int64_t)H * W, W, 1, 1);
  EpConv<2> ep{bias, lo, hi, npix, (int64_t)C_out * npix, npix, FastDiv::make((uint32_t)npix)};
  return launch_gemm<2, false>(1, C_out, (int)N, (int)Kd, LoadKernel<2>{kernel, (int)Kd}, gb, ep,
                               nullptr, false, (hipStream_t)stream);
}

extern "C" int vc_zono_conv(const float* c, const float* G, int64_t B, int Kg, int C_in, int H,
                            int W, const float* kernel, const float* bias, int C_out, int kh,
                            int kw, int sh, int sw, int ph, int pw, int H_out, int W_out,
                            float* c_out, float* G_out, vc_stream_t stream) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK || !c || !kernel || !c_out || B < 0 || Kg < 0) return VC_ERR_ARG;
  if (Kg > 0 && (!G || !G_out)) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const int64_t npix = (int64_t)H_out * W_out, Kd = (int64_t)C_in * kh * kw;
  const int64_t n_in = (int64_t)C_in * H * W, n_out = (int64_t)C_out * npix;
  if (B == 0) return VC_OK;
  if (B * npix * (Kg > 0 ? Kg : 1) > kMaxDim || Kd > kMaxDim) return VC_ERR_UNSUPPORTED;
  {
    auto gb = forward_gather<1>(g, c, nullptr, n_in, (int64_t)H * W, W, 1, 1);
    EpConv<1> ep{bias, c_out, nullptr, npix, n_out, npix, FastDiv::make((uint32_t)npix)};
    const int rc = launch_gemm<1, false>(1, C_out, (int)(B * npix), (int)Kd,
                                         LoadKernel<1>{kernel, (int)Kd}, gb, ep, nullptr, false, st);
    if (rc != VC_OK) return rc;
  }
  if (Kg == 0) return VC_OK;
  // generator columns: element (b, ci, y, x, k) at ((b n_in + (ci H + y) W + x) Kg + k
  auto gb = forward_gather<1>(g, G, nullptr, n_in * Kg, (int64_t)H * W * Kg, W * Kg, Kg, Kg);
  const int64_t per = npix * Kg;
  EpConv<1> ep{nullptr, G_out, nullptr, per, n_out * Kg, per, FastDiv::make((uint32_t)per)};
  return launch_gemm<1, false>(1, C_out, (int)(B * per), (int)Kd, LoadKernel<1>{kernel, (int)Kd},
                               gb, ep, nullptr, false, st);
}

namespace {

// Band and ring sizes of k_conv_t_fold for a geometry, or false when the
// geometry is outside its limits.  Bands of about 256 source pixels (one
// pass of the four waves), halved until the LDS fits.
struct FoldPlan {
  int MT, nks, BS, RS, hl, hr;
  size_t lds;
};

bool fold_plan(int C_out, int Ho, int Wo, int C_in, int W, int kh, int kw, int sh, int sw,
               int pw, FoldPlan& f) {
  const int64_t MF = (int64_t)C_in * kh * kw;
  if (MF > kFoldMaxMF || C_out > kFoldMaxCout || C_in > kSmallC) return false;
  f.MT = MF > 16 ? 2 : 1;
  f.nks = (C_out + 3) / 4;
  f.hl = (kw + sw - 1) / sw - 1;
  f.hr = (W - 1 + pw) / sw - (Wo - 1);
  if (f.hr < 0) f.hr = 0;
  f.BS = Wo >= 256 ? 1 : 256 / Wo;
  if (f.BS > Ho) f.BS = Ho;
  for (;;) {
    f.RS = f.BS + (kh - 1) / sh;
    f.lds = ((size_t)f.nks * (f.MT * 64 + 4) +
             (size_t)MF * (f.RS + 1) * (f.hl + Wo + f.hr)) * sizeof(float);
    if (f.lds <= (size_t)kFoldMaxLds) return true;
    if (f.BS == 1) return false;
    f.BS /= 2;
  }
}

template <int MT, int RL>
void launch_fold_vec(const FoldArgs& a, bool vec, dim3 grid, size_t lds, hipStream_t st) {
  if (vec)
    hipLaunchKernelGGL((k_conv_t_fold<MT, RL, true>), grid, dim3(kFoldNT), lds, st, a);
  else
    hipLaunchKernelGGL((k_conv_t_fold<MT, RL, false>), grid, dim3(kFoldNT), lds, st, a);
}

template <int MT>
void launch_fold_rl(const FoldArgs& a, bool vec, dim3 grid, size_t lds, hipStream_t st) {
  if (!a.ls)
    launch_fold_vec<MT, 0>(a, vec, grid, lds, st);
  else if (!a.beta)
    launch_fold_vec<MT, 1>(a, vec, grid, lds, st);
  else
    launch_fold_vec<MT, 2>(a, vec, grid, lds, st);
}

// One image per workgroup at a time, as many workgroups as fit the CUs
// (a multiple of 8, so each keeps its XCD across images).
int launch_fold(FoldArgs a, const FoldPlan& f, hipStream_t st) {
  a.MF = a.C_in * a.kh * a.kw;
  a.nks = f.nks;
  a.BS = f.BS;
  a.RS = f.RS;
  a.hl = f.hl;
  a.hr = f.hr;
  a.f_W = FastDiv::make((uint32_t)a.W);
  a.f_Wo = FastDiv::make((uint32_t)a.Wo);
  a.f_RS = FastDiv::make((uint32_t)a.RS);
  a.f_sh = FastDiv::make((uint32_t)a.sh);
  a.f_sw = FastDiv::make((uint32_t)a.sw);
  const bool relu = a.ls != nullptr;
  bool vec = a.Wo % 4 == 0 && aligned16(a.ew);
  if (relu) vec = vec && aligned16(a.ls) && aligned16(a.us) && aligned16(a.ut) &&
                  (!a.beta || aligned16(a.beta));
  int per_cu = (int)((160 * 1024) / (f.lds + 2 * (kFoldNT / 64) * sizeof(double)));
  if (per_cu > 8) per_cu = 8;
  if (per_cu < 1) per_cu = 1;
  int64_t grid = (int64_t)vcm::cu_count() * per_cu;
  grid -= grid % 8;
  // a tile is about one XCD's images in flight
  const int64_t flight = grid / 8 > 1 ? grid / 8 : 1;
  a.DB = (int)(a.B < 8 ? a.B : 8);
  a.SB = (int)((flight + a.DB - 1) / a.DB);
  if (a.SB > a.R) a.SB = (int)a.R;
  a.ndb = (int)((a.B + a.DB - 1) / a.DB);
  a.total = a.shared ? (int64_t)a.ndb * ((a.R + a.SB - 1) / a.SB) * a.DB * a.SB : a.M;
  if (a.total >= (int64_t(1) << 31)) return VC_ERR_UNSUPPORTED;
  a.f_R = FastDiv::make((uint32_t)a.R);
  a.f_DB = FastDiv::make((uint32_t)a.DB);
  a.f_ndb = FastDiv::make((uint32_t)a.ndb);
  a.f_tile = FastDiv::make((uint32_t)(a.DB * a.SB));
  if (grid > a.M) grid = a.M;
  const dim3 g((unsigned)grid);
  if (f.MT == 1)
    launch_fold_rl<1>(a, vec, g, f.lds, st);
  else
    launch_fold_rl<2>(a, vec, g, f.lds, st);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

// Row length of the packed transposed taps: C_out Ty Tx rounded up to 4.
int conv_t_ld(int C_out, int kh, int kw, int sh, int sw) {
  const int Ty = (kh + sh - 1) / sh, Tx = (kw + sw - 1) / sw;
  return (C_out * Ty * Tx + 3) & ~3;
}

int backward_conv(const float* ew_in, int64_t M, const float* kernel, const float* packed,
                  const float* bias, int C_out, int H_out, int W_out, int C_in, int H, int W,
                  int kh, int kw, int sh, int sw, int ph, int pw, float* ew_out, float* acc,
                  vc_stream_t stream) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK || !ew_in || !kernel || !ew_out || M < 0) return VC_ERR_ARG;
  if (bias && !acc) return VC_ERR_ARG;
  if (M == 0) return VC_OK;
  hipStream_t st = (hipStream_t)stream;
  const int Hc = (H + sh - 1) / sh, Wc = (W + sw - 1) / sw;
  const int Ty = (kh + sh - 1) / sh, Tx = (kw + sw - 1) / sw;
  const int64_t npix = (int64_t)Hc * Wc, N = M * npix, Kd = (int64_t)C_out * Ty * Tx;
  if (N > kMaxDim || Kd > kMaxDim) return VC_ERR_UNSUPPORTED;
  FoldPlan fp;
  if (M < (int64_t(1) << 31) && fold_plan(C_out, H_out, W_out, C_in, W, kh, kw, sh, sw, pw, fp)) {
    FoldArgs a{};
    a.ew = ew_in;
    a.M = M;
    a.R = 1;
    a.B = M;
    a.shared = 0;
    a.K = kernel;
    a.bias = bias;
    a.out = ew_out;
    a.acc = acc;
    a.C_out = C_out, a.Ho = H_out, a.Wo = W_out, a.C_in = C_in, a.H = H, a.W = W;
    a.kh = kh, a.kw = kw, a.sh = sh, a.sw = sw, a.ph = ph, a.pw = pw;
    return launch_fold(a, fp, st);
  }
  if (bias) {
    const int sp = H_out * W_out;
    const bool v = ((int64_t)C_out * sp) % 4 == 0 && aligned16(ew_in);
    const dim3 grid((unsigned)(M < kMaxGrid ? M : kMaxGrid));
    if (v)
      hipLaunchKernelGGL(k_conv_bias_dot<true>, grid, dim3(NT), 0, st, ew_in, M, C_out, sp,
                         FastDiv::make((uint32_t)sp), bias, acc);
    else
      hipLaunchKernelGGL(k_conv_bias_dot<false>, grid, dim3(NT), 0, st, ew_in, M, C_out, sp,
                         FastDiv::make((uint32_t)sp), bias, acc);
  }
  VC_LAUNCH_CHECK();
  const size_t lds = (size_t)C_out * kh * kw * C_in * sizeof(double);
  if (C_in <= kSmallC && lds <= (size_t)kSmallCLds) {
    const int64_t total = M * H * W;
    const dim3 grid((unsigned)((total + NT - 1) / NT < kMaxGrid ? (total + NT - 1) / NT : kMaxGrid));
    switch (C_in) {
      case 1: hipLaunchKernelGGL(k_conv_t_smallc<1>, grid, dim3(NT), lds, st, ew_in, M, g, kernel, ew_out); break;
      case 2: hipLaunchKernelGGL(k_conv_t_smallc<2>, grid, dim3(NT), lds, st, ew_in, M, g, kernel, ew_out); break;
      case 3: hipLaunchKernelGGL(k_conv_t_smallc<3>, grid, dim3(NT), lds, st, ew_in, M, g, kernel, ew_out); break;
      default: hipLaunchKernelGGL(k_conv_t_smallc<4>, grid, dim3(NT), lds, st, ew_in, M, g, kernel, ew_out); break;
    }
    VC_LAUNCH_CHECK();
    return VC_OK;
  }
  auto run = [&](auto gb) {
    gb.src = ew_in;
    gb.src2 = nullptr;
    gb.s_img = (int64_t)C_out * H_out * W_out;
    gb.s_c = (int64_t)H_out * W_out;
    gb.s_y = W_out;
    gb.s_x = 1;
    gb.Hs = H_out;
    gb.Ws = W_out;
    gb.nk = 1;
    gb.T = Ty * Tx;
    gb.Tx = Tx;
    gb.psy = 1;
    gb.psx = 1;
    gb.ph = ph;
    gb.pw = pw;
    gb.sh = sh;
    gb.sw = sw;
    gb.Wg = Wc;
    gb.per_img = npix;
    gb.f_img = FastDiv::make((uint32_t)npix);
    gb.f_nk = FastDiv::make(1);
    gb.f_wg = FastDiv::make((uint32_t)Wc);
    gb.f_T = FastDiv::make((uint32_t)gb.T);
    gb.f_Tx = FastDiv::make((uint32_t)Tx);
    EpConvT ep{ew_out, H, W, Wc, sh, sw, npix, (int64_t)C_in * H * W,
               FastDiv::make((uint32_t)npix), FastDiv::make((uint32_t)Wc)};
    if (packed && aligned16(packed)) {
      const int ld = conv_t_ld(C_out, kh, kw, sh, sw);
      LoadPackedT la{packed, (int64_t)C_in * ld, ld};
      return launch_gemm<1, false>((int64_t)sh * sw, C_in, (int)N, (int)Kd, la, gb, ep, nullptr,
                                   false, st);
    }
    LoadKernelT la{kernel, C_in, kh, kw, sh, sw, ph, pw, Ty * Tx, Tx, Ty,
                   FastDiv::make((uint32_t)(Ty * Tx)), FastDiv::make((uint32_t)Tx)};
    return launch_gemm<1, false>((int64_t)sh * sw, C_in, (int)N, (int)Kd, la, gb, ep, nullptr,
                                 false, st);
  };
  // quads of 4 columns start at multiples of 4; with the class grid's width
  // and pixel count multiples of 4 each lies in one source row
  if (Wc % 4 == 0 && npix % 4 == 0) return run(LoadGather<1, true, true>{});
  return run(LoadGather<1, true, false>{});
}

}  // namespace

extern "C" int vc_backward_conv(const float* ew_in, int64_t M, const float* kernel,
                                const float* bias, int C_out, int H_out, int W_out, int C_in,
                                int H, int W, int kh, int kw, int sh, int sw, int ph, int pw,
                                float* ew_out, float* acc, vc_stream_t stream) {
  return backward_conv(ew_in, M, kernel, nullptr, bias, C_out, H_out, W_out, C_in, H, W, kh, kw,
                       sh, sw, ph, pw, ew_out, acc, stream);
}

extern "C" int64_t vc_conv_t_pack_floats(int C_out, int C_in, int kh, int kw, int sh, int sw) {
  if (C_out <= 0 || C_in <= 0 || kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0) return -VC_ERR_ARG;
  return (int64_t)sh * sw * C_in * conv_t_ld(C_out, kh, kw, sh, sw);
}

extern "C" int vc_conv_t_pack(const float* kernel, int C_out, int C_in, int kh, int kw, int sh,
                              int sw, int ph, int pw, float* out, vc_stream_t stream) {
  if (!kernel || !out || C_out <= 0 || C_in <= 0 || kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 ||
      ph < 0 || pw < 0)
    return VC_ERR_ARG;
  ConvGeom g{C_in, 1, 1, C_out, kh, kw, sh, sw, ph, pw, 1, 1};
  const int Ty = (kh + sh - 1) / sh, Tx = (kw + sw - 1) / sw;
  const int ld = conv_t_ld(C_out, kh, kw, sh, sw);
  const int64_t total = (int64_t)sh * sw * C_in * ld;
  hipLaunchKernelGGL(k_conv_t_pack, dim3(vc_blocks(total, NT)), dim3(NT), 0, (hipStream_t)stream,
                     kernel, g, Ty, Tx, ld, out);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_backward_conv_packed(const float* ew_in, int64_t M, const float* kernel,
                                       const float* packed, const float* bias, int C_out,
                                       int H_out, int W_out, int C_in, int H, int W, int kh,
                                       int kw, int sh, int sw, int ph, int pw, float* ew_out,
                                       float* acc, vc_stream_t stream) {
  if (!packed) return VC_ERR_ARG;
  return backward_conv(ew_in, M, kernel, packed, bias, C_out, H_out, W_out, C_in, H, W, kh, kw,
                       sh, sw, ph, pw, ew_out, acc, stream);
}

extern "C" int vc_backward_relu_conv_ok(int C_out, int H_out, int W_out, int C_in, int H, int W,
                                        int kh, int kw, int sh, int sw, int ph, int pw) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK) return 0;
  FoldPlan fp;
  return fold_plan(C_out, H_out, W_out, C_in, W, kh, kw, sh, sw, pw, fp) ? 1 : 0;
}

extern "C" int vc_backward_relu_conv(const float* ew_in, int64_t M, int64_t R, int ew_shared,
                                     const float* lo_s, const float* up_s, const float* up_t,
                                     const float* beta, const float* kernel, const float* bias,
                                     int C_out, int H_out, int W_out, int C_in, int H, int W,
                                     int kh, int kw, int sh, int sw, int ph, int pw,
                                     float* ew_out, float* acc, vc_stream_t stream) {
  ConvGeom g{C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, H_out, W_out};
  if (check_geom(g) != VC_OK || !ew_in || !kernel || !ew_out || !acc || !lo_s || !up_s ||
      !up_t || M < 0 || R <= 0 || M % R)
    return VC_ERR_ARG;
  FoldPlan fp;
  if (!fold_plan(C_out, H_out, W_out, C_in, W, kh, kw, sh, sw, pw, fp)) return VC_ERR_UNSUPPORTED;
  if ((int64_t)C_out * H_out * W_out > kMaxDim) return VC_ERR_UNSUPPORTED;
  if (M == 0) return VC_OK;
  FoldArgs a{};
  a.ew = ew_in;
  a.M = M;
  a.R = R;
  a.B = M / R;
  a.shared = ew_shared ? 1 : 0;
  a.ls = lo_s;
  a.us = up_s;
  a.ut = up_t;
  a.beta = beta;
  a.K = kernel;
  a.bias = bias;
  a.out = ew_out;
  a.acc = acc;
  a.C_out = C_out, a.Ho = H_out, a.Wo = W_out, a.C_in = C_in, a.H = H, a.W = W;
  a.kh = kh, a.kw = kw, a.sh = sh, a.sw = sw, a.ph = ph, a.pw = pw;
  return launch_fold(a, fp, (hipStream_t)stream);
}
