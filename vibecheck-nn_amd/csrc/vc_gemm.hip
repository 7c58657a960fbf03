// fp32 MFMA GEMMs of the fc layers: the interval forward, the zonotope
// forward, the CROWN backward step (fused, or two-phase through relax_out),
// and the alpha gradient sweep.  The GEMM core is vc_gemm_core.h; the
// plain products (no arithmetic in the operand loads, no epilogue) run
// rocBLAS's sgemm.
#include <rocblas/rocblas.h>

#include "vc_gemm_core.h"
#include "vc_relax.h"

namespace {

using namespace vcg;

// rocBLAS handles, one per device and host thread (the stream is handle
// state, so threads on their own streams never share one), created on
// first use and kept for the life of the process.
constexpr int kMaxDevices = 64;
thread_local rocblas_handle t_blas[kMaxDevices] = {};

int blas_handle(rocblas_handle& out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return VC_ERR_LAUNCH;
  if (!t_blas[dev]) {
    rocblas_handle h = nullptr;
    if (rocblas_create_handle(&h) != rocblas_status_success) return VC_ERR_LAUNCH;
    t_blas[dev] = h;
  }
  out = t_blas[dev];
  return VC_OK;
}

// C (M x N) = A (M x K) B (K x N), row-major fp32, on `st`: rocBLAS's
// column-major sgemm computes C^T = B^T A^T from the same memory.  M is
// taken in slices whose element counts stay within its 32-bit sizes.
int plain_gemm(const float* A, int64_t M, int K, const float* B, int N, float* C,
               hipStream_t st) {
  if (M == 0) return VC_OK;
  rocblas_handle h = nullptr;
  const int rc = blas_handle(h);
  if (rc != VC_OK) return rc;
  if (rocblas_set_stream(h, st) != rocblas_status_success) return VC_ERR_LAUNCH;
  const float one = 1.f, zero = 0.f;
  const int64_t step = std::max<int64_t>(1, ((int64_t)1 << 30) / std::max(K, N));
  for (int64_t m0 = 0; m0 < M; m0 += step) {
    const int mm = (int)std::min<int64_t>(step, M - m0);
    if (rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none, N, mm, K, &one, B, N,
                      A + m0 * K, K, &zero, C + m0 * N, N) != rocblas_status_success)
      return VC_ERR_LAUNCH;
  }
  return VC_OK;
}

// C[b] (M x N) = A (M x K) B[b] (K x N) for b < nb, row-major fp32, A shared
// (rocBLAS's strided-batched sgemm: C[b]^T = B[b]^T A^T), in slices of the
// batch that keep its 32-bit sizes in range.
int plain_gemm_shared_a(const float* A, int M, int K, const float* B, int64_t nb, int N,
                        float* C, hipStream_t st) {
  if (nb == 0) return VC_OK;
  rocblas_handle h = nullptr;
  const int rc = blas_handle(h);
  if (rc != VC_OK) return rc;
  if (rocblas_set_stream(h, st) != rocblas_status_success) return VC_ERR_LAUNCH;
  const float one = 1.f, zero = 0.f;
  const int64_t sb = (int64_t)K * N, sc = (int64_t)M * N;
  const int64_t step = std::max<int64_t>(1, std::min<int64_t>(((int64_t)1 << 30) / std::max(sb, sc),
                                                              0x7fffffff));
  for (int64_t b0 = 0; b0 < nb; b0 += step) {
    const int cnt = (int)std::min<int64_t>(step, nb - b0);
    if (rocblas_sgemm_strided_batched(h, rocblas_operation_none, rocblas_operation_none, N, M, K,
                                      &one, B + b0 * sb, N, sb, A, K, 0, &zero, C + b0 * sc, N,
                                      sc, cnt) != rocblas_status_success)
      return VC_ERR_LAUNCH;
  }
  return VC_OK;
}

// vc_backward_fc runs its two-phase form (relaxed rows through relax_out)
// from this row width up; narrower rows keep the fused prologue.
constexpr int kTwoPhaseMinWidth = 64;

// ------------------------------------------------------------- A loaders
struct LoadMidRad {  // A = (mid, rad) of an interval row-block
  static constexpr int kBK = 32;
  const float *l, *h;
  int ld;
  struct Row {
    int64_t o;
  };
  struct Raw {
    float l[4], h[4];
  };
  __device__ Row row(int64_t, int64_t m, bool) const { return Row{m * ld}; }
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    ld4<VEC>(l + rw.o + k, n, x.l);
    ld4<VEC>(h + rw.o + k, n, x.h);
  }
  template <bool VEC>
  __device__ void finish(const Row&, int, int, const Raw& x, float (*v)[4], KSum&, bool) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[0][j] = (x.l[j] + x.h[j]) / 2.f;
      v[1][j] = (x.h[j] - x.l[j]) / 2.f;
    }
  }
};

// The group of domain d, read in range: an index outside [0, n_groups)
// reads group 0 (vc_group_clamp reports such indices to the caller).
__device__ __forceinline__ int64_t safe_group(const int64_t* group, int64_t n_groups, int64_t d) {
  const int64_t g = group[d];
  return (uint64_t)g < (uint64_t)n_groups ? g : 0;
}

// CROWN backward: relaxation of ew rows at a relu, then the fc product.
// Per element: ep = max(x, 0), en = min(x, 0); e = ep * lo_s + en * up_s
// (+ beta); row part en * up_t (+ e * bias[k]); lo_s from the alpha
// override when given (active -> 1, unstable -> alpha, dead -> 0).
struct LoadRelaxRow {
  static constexpr int kBK = 16;  // 32 measured slower at every shape (more live registers)
  const float* ew;
  int ld;  // n_out
  int R;
  const float *lo, *hi, *alpha, *beta, *bias;
  int alpha_per_row;
  float* relax_out;
  int ew_bcast;  // rows shared by all domains: row m reads ew[m % R]
  const int64_t* alpha_group = nullptr;  // per-row alpha of domain d's group: (G, R, ld)
  int64_t n_groups = 0;                   // G: an index outside [0, G) reads group 0
  struct Row {
    int64_t xo, dom, mo, ao;  // offsets of the ew row, the domain's neurons, row m, alpha
    bool ro;                  // this tile writes relax_out
  };
  struct Raw {
    float x[4], lo[4], hi[4], a[4], b[4];
  };
  __device__ Row row(int64_t, int64_t m, bool first) const {
    const int64_t d = m / R;
    const int64_t ao = alpha_group ? (safe_group(alpha_group, n_groups, d) * R + (m - d * R)) * ld
                                   : (alpha_per_row ? m * ld : d * ld);
    return Row{(ew_bcast ? m - d * R : m) * ld, d * ld, m * ld, ao,
               first && relax_out != nullptr};
  }
  // alpha and beta travel with the prefetched tile, so their latency hides
  // behind the previous tile's MFMAs like the rows'
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    ld4<VEC>(ew + rw.xo + k, n, x.x);
    if (lo) {
      ld4<VEC>(lo + rw.dom + k, n, x.lo);
      ld4<VEC>(hi + rw.dom + k, n, x.hi);
      if (alpha) ld4<VEC>(alpha + rw.ao + k, n, x.a);
      if (beta) ld4<VEC>(beta + rw.dom + k, n, x.b);
    }
  }
  template <bool VEC>
  __device__ void finish(const Row& rw, int k, int n, const Raw& x, float (*v)[4], KSum& part,
                         bool rows) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float e = x.x[j], p = 0.f;
      if (j < n) {
        if (lo) {
          Relax s = relax(x.lo[j], x.hi[j]);
          float ls = s.lo_s;
          if (alpha) ls = s.active ? 1.f : (s.unstable ? x.a[j] : 0.f);
          const float ep = fmaxf(e, 0.f), en = fminf(e, 0.f);
          e = ep * ls + en * s.up_s;
          if (beta) e = e + x.b[j];
          p = en * s.up_t;
        }
        if (bias) p += e * bias[k + j];
        if (rw.ro) relax_out[rw.mo + k + j] = e;
        if (rows) part.add(p);
      }
      v[0][j] = e;
    }
  }
};

// alpha gradient sweep with precomputed slopes (ls with the alpha override).
struct LoadGradSlopes {
  static constexpr int kBK = 32;
  const float *gE, *P;
  int ld, R;
  const float *ls, *us, *ut;
  int p_bcast;
  struct Row {
    int64_t mo, po, dom;
  };
  struct Raw {
    float ge[4], pv[4];
  };
  __device__ Row row(int64_t, int64_t m, bool) const {
    const int64_t d = m / R;
    return Row{m * ld, (p_bcast ? m - d * R : m) * ld, d * ld};
  }
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    ld4<VEC>(gE + rw.mo + k, n, x.ge);
    ld4<VEC>(P + rw.po + k, n, x.pv);
  }
  template <bool VEC>
  __device__ void finish(const Row& rw, int k, int n, const Raw& x, float (*v)[4], KSum&,
                         bool) const {
    float sl[4], su[4], st[4];
    ld4<VEC>(ls + rw.dom + k, n, sl);
    ld4<VEC>(us + rw.dom + k, n, su);
    ld4<VEC>(ut + rw.dom + k, n, st);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float gp = 0.f;
      if (j < n) {
        const bool mp = x.pv[j] >= 0.f, mn = x.pv[j] <= 0.f;
        const float f = (mp ? sl[j] : 0.f) + (mn ? su[j] : 0.f);
        gp = x.ge[j] * f;
        if (mn) gp += st[j];
      }
      v[0][j] = gp;
    }
  }
};

// alpha gradient sweep: gP = gE * (mpos ls + mneg up_s) + mneg up_t.
struct LoadGradRelax {
  static constexpr int kBK = 16;
  const float *gE, *P;
  int ld, R;
  const float *lo, *hi, *alpha;
  int p_bcast;    // P shared by all domains: row m reads P[m % R]
  int alpha_row;  // alpha (M, ld), one per row (per-query alpha), else (B, ld)
  float* galpha_rows = nullptr;  // d lb / d alpha per row (M, ld), written by column tile 0
  struct Row {
    int64_t mo, po, dom;
    bool go;  // this tile writes galpha_rows
  };
  struct Raw {
    float ge[4], pv[4], lo[4], hi[4], a[4];
  };
  __device__ Row row(int64_t, int64_t m, bool first) const {
    const int64_t d = m / R;
    return Row{m * ld, (p_bcast ? m - d * R : m) * ld, d * ld, first && galpha_rows != nullptr};
  }
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    ld4<VEC>(gE + rw.mo + k, n, x.ge);
    ld4<VEC>(P + rw.po + k, n, x.pv);
    ld4<VEC>(lo + rw.dom + k, n, x.lo);
    ld4<VEC>(hi + rw.dom + k, n, x.hi);
    if (alpha) ld4<VEC>(alpha + (alpha_row ? rw.mo : rw.dom) + k, n, x.a);
  }
  template <bool VEC>
  __device__ void finish(const Row& rw, int k, int n, const Raw& x, float (*v)[4], KSum&,
                         bool) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float gp = 0.f;
      if (j < n) {
        Relax s = relax(x.lo[j], x.hi[j]);
        float ls = s.lo_s;
        if (alpha) ls = s.active ? 1.f : (s.unstable ? x.a[j] : 0.f);
        if (rw.go) galpha_rows[rw.mo + k + j] = s.unstable ? x.ge[j] * fmaxf(x.pv[j], 0.f) : 0.f;
        const bool mp = x.pv[j] >= 0.f, mn = x.pv[j] <= 0.f;
        const float f = (mp ? ls : 0.f) + (mn ? s.up_s : 0.f);
        gp = x.ge[j] * f;
        if (mn) gp += s.up_t;
      }
      v[0][j] = gp;
    }
  }
};

struct LoadGradInput {  // gA = xl [A >= 0] + xh [A <= 0]
  static constexpr int kBK = 32;
  const float *A, *xl, *xh;
  int ld, R;
  struct Row {
    int64_t mo, dom;
  };
  struct Raw {
    float a[4], l[4], h[4];
  };
  __device__ Row row(int64_t, int64_t m, bool) const { return Row{m * ld, (m / R) * ld}; }
  template <bool VEC>
  __device__ void fetch(const Row& rw, int k, int n, Raw& x) const {
    ld4<VEC>(A + rw.mo + k, n, x.a);
    ld4<VEC>(xl + rw.dom + k, n, x.l);
    ld4<VEC>(xh + rw.dom + k, n, x.h);
  }
  template <bool VEC>
  __device__ void finish(const Row&, int, int n, const Raw& x, float (*v)[4], KSum&,
                         bool) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float gv = 0.f;
      if (j < n) {
        if (x.a[j] >= 0.f) gv += x.l[j];
        if (x.a[j] <= 0.f) gv += x.h[j];
      }
      v[0][j] = gv;
    }
  }
};

// ------------------------------------------------------------- B loaders
struct LoadWtAbs {  // B[k][n] = (W[n][k], |W[n][k]|), W (n_out, ld)
  static constexpr bool kTrans = true;
  const float* W;
  int ld;
  struct Col {
    int64_t o;
  };
  struct Raw {
    float x[4];
  };
  __device__ Col col(int64_t, int n) const { return Col{(int64_t)n * ld}; }
  template <bool VEC>
  __device__ void fetch(const Col& c, int k, int cnt, Raw& r) const {
    float* o = r.x;
    ld4<VEC>(W + c.o + k, cnt, o);
  }
  __device__ static void finish(const Raw& r, float (*v)[4]) {
    const float* x = r.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[0][j] = x[j];
      v[1][j] = fabsf(x[j]);
    }
  }
};

// ------------------------------------------------------------- epilogues
struct EpIbp {
  const float* bias;
  float *lo, *hi;
  int ld;
  __device__ void operator()(int64_t, int64_t m, int n, const float* c) const {
    const float mc = bias ? c[0] + bias[n] : c[0];
    lo[m * ld + n] = mc - c[1];
    hi[m * ld + n] = mc + c[1];
  }
};

// Phase 1 of the two-phase backward step (vc_backward_fc with relax_out):
// the relaxed rows e = pos(ew) ls + neg(ew) up_s [+ beta] into out, and
// acc[m] += sum_k (neg(ew) up_t + e bias[k]) in fp64.  A workgroup takes
// RR consecutive rows and streams their columns in float4 quads (the four
// waves read neighbouring addresses); when the rows belong to one domain
// the relaxation of each neuron is computed once for all of them.  HBM
// bound: 8 bytes per element plus the per-domain bounds.
constexpr int RR = 4;

template <bool VEC>
__global__ __launch_bounds__(NT) void k_relax_rows(const float* ew, int64_t M, int R, int n,
                                                   const float* lo, const float* hi,
                                                   const float* alpha, int alpha_per_row,
                                                   const int64_t* alpha_group, int64_t n_groups,
                                                   const float* beta, const float* bias,
                                                   int ew_bcast, float* out, float* acc) {
  __shared__ double red[NT / 64][RR];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nq = (n + 3) >> 2;
  for (int64_t m0 = (int64_t)blockIdx.x * RR; m0 < M; m0 += (int64_t)gridDim.x * RR) {
    int64_t mr[RR], dr[RR], xr[RR];
#pragma unroll
    for (int k = 0; k < RR; ++k) {
      mr[k] = m0 + k < M ? m0 + k : M - 1;  // past the end: recompute the last row, no store
      dr[k] = mr[k] / R;
      xr[k] = ew_bcast ? mr[k] - dr[k] * R : mr[k];
    }
    const bool shared = dr[0] == dr[RR - 1] && !(alpha && (alpha_per_row || alpha_group));
    double p[RR];
#pragma unroll
    for (int k = 0; k < RR; ++k) p[k] = 0.0;
    for (int i = threadIdx.x; i < nq; i += NT) {
      const int c = 4 * i;
      const int cnt = n - c < 4 ? n - c : 4;
      float x[RR][4], e[RR][4], bi[4];
#pragma unroll
      for (int k = 0; k < RR; ++k) ld4<VEC>(ew + xr[k] * n + c, cnt, x[k]);
      if (bias) ld4<VEC>(bias + c, cnt, bi);
#pragma unroll
      for (int k = 0; k < RR; ++k) {
        if (k > 0 && shared) break;
        float l4[4], h4[4], a4[4], b4[4];
        ld4<VEC>(lo + dr[k] * n + c, cnt, l4);
        ld4<VEC>(hi + dr[k] * n + c, cnt, h4);
        if (alpha) {
          const int64_t ar = alpha_group
                                 ? safe_group(alpha_group, n_groups, dr[k]) * R + (mr[k] - dr[k] * R)
                                 : (alpha_per_row ? mr[k] : dr[k]);
          ld4<VEC>(alpha + ar * n + c, cnt, a4);
        }
        if (beta) ld4<VEC>(beta + dr[k] * n + c, cnt, b4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (j >= cnt) break;
          const Relax r = relax(l4[j], h4[j]);
          const float ls = alpha ? (r.active ? 1.f : (r.unstable ? a4[j] : 0.f)) : r.lo_s;
#pragma unroll
          for (int q = 0; q < RR; ++q) {
            if (!(shared ? true : q == k)) continue;
            const float ep = fmaxf(x[q][j], 0.f), en = fminf(x[q][j], 0.f);
            float v = ep * ls + en * r.up_s;
            if (beta) v = v + b4[j];
            float pp = en * r.up_t;
            if (bias) pp += v * bi[j];
            p[q] += (double)pp;
            e[q][j] = v;
          }
        }
      }
#pragma unroll
      for (int k = 0; k < RR; ++k) {
        if (m0 + k >= M) break;
        float* o = out + mr[k] * n + c;
        if (VEC && cnt == 4) {
          *reinterpret_cast<float4*>(o) = make_float4(e[k][0], e[k][1], e[k][2], e[k][3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (j < cnt) o[j] = e[k][j];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < RR; ++k) {
      const double t = wave_sum_f64(p[k]);
      if (lane == 0) red[wv][k] = t;
    }
    __syncthreads();
    if (threadIdx.x < RR && m0 + threadIdx.x < M) {
      const int k = threadIdx.x;
      const double t = (red[0][k] + red[1][k]) + (red[2][k] + red[3][k]);
      acc[m0 + k] = (float)((double)acc[m0 + k] + t);
    }
    __syncthreads();
  }
}

// lo_s (alpha override: active 1, unstable alpha, dead 0), up_s, up_t of
// every (domain, neuron), the relax() arithmetic.
__global__ void k_relax_slopes(const float* lo, const float* hi, const float* alpha, int64_t n,
                               float* ls, float* us, float* ut) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const Relax s = relax(lo[i], hi[i]);
    float l = s.lo_s;
    if (alpha) l = s.active ? 1.f : (s.unstable ? alpha[i] : 0.f);
    ls[i] = l;
    us[i] = s.up_s;
    ut[i] = s.up_t;
  }
}

}  // namespace

extern "C" int vc_ibp_fc(const float* l, const float* h, int64_t B, int n_in,
                         const float* W, const float* bias, int n_out, float* lo,
                         float* hi, vc_stream_t stream) {
  if (!l || !h || !W || !lo || !hi || n_in <= 0 || n_out <= 0 || B < 0) return VC_ERR_ARG;
  const bool vec = vec_ok({l, h, W}, {n_in});
  return launch_gemm<2, false>(1, B, n_out, n_in, LoadMidRad{l, h, n_in}, LoadWtAbs{W, n_in},
                               EpIbp{bias, lo, hi, n_out}, nullptr, vec, (hipStream_t)stream);
}

extern "C" int vc_zono_fc(const float* c, const float* G, int64_t B, int n_in, int K,
                          const float* W, const float* bias, int n_out, float* c_out,
                          float* G_out, vc_stream_t stream) {
  if (!c || !W || !c_out || n_in <= 0 || n_out <= 0 || B < 0 || K < 0) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_gemm<1, false>(1, B, n_out, n_in, LoadRow{c, n_in}, LoadWt{W, n_in},
                                 EpStoreBias{bias, c_out, n_out}, nullptr,
                                 vec_ok({c, W}, {n_in}), st);
  if (rc != VC_OK || K == 0 || B == 0) return rc;
  if (!G || !G_out) return VC_ERR_ARG;
  // G_out[b] (n_out x K) = W (n_out x n_in) G[b] (n_in x K): a plain
  // batched product with W shared
  return plain_gemm_shared_a(W, n_out, n_in, G, B, K, G_out, st);
}

// Phase 1 for narrow rows (n <= 64): one 16-lane row of the wavefront per
// backward row, a quad of 4 columns per lane, RN rows per workgroup pass;
// the row's constant term is summed over its 16 lanes in fp64.  Same
// arithmetic per element as k_relax_rows, whose quads-per-thread mapping
// leaves 3/4 of a workgroup idle at 64 columns.  Below 64 columns the
// fused form is faster (the relaxed rows' round trip through HBM costs more
// than the loads' arithmetic), so the two-phase step starts at 64.
constexpr int RN = NT / 16;
constexpr int kNarrowMaxWidth = 64;

template <bool VEC>
__global__ __launch_bounds__(NT) void k_relax_rows_narrow(const float* ew, int64_t M, int R,
                                                          int n, const float* lo, const float* hi,
                                                          const float* alpha, int alpha_per_row,
                                                          const int64_t* alpha_group,
                                                          int64_t n_groups,
                                                          const float* beta, const float* bias,
                                                          int ew_bcast, float* out, float* acc) {
  const int c = 4 * (threadIdx.x & 15);
  const int cnt = n - c < 4 ? n - c : 4;  // <= 0: the lane holds no column
  for (int64_t m0 = (int64_t)blockIdx.x * RN; m0 < M; m0 += (int64_t)gridDim.x * RN) {
    const int64_t mm = m0 + (threadIdx.x >> 4);
    const int64_t m = mm < M ? mm : M - 1;  // past the end: recompute the last row, no store
    const int64_t d = m / R;
    const int64_t xr = ew_bcast ? m - d * R : m;
    double p = 0.0;
    if (cnt > 0) {
      float x[4], l4[4], h4[4], a4[4], b4[4], bi[4], e[4];
      ld4<VEC>(ew + xr * n + c, cnt, x);
      ld4<VEC>(lo + d * n + c, cnt, l4);
      ld4<VEC>(hi + d * n + c, cnt, h4);
      if (alpha) {
        const int64_t ar = alpha_group ? safe_group(alpha_group, n_groups, d) * R + (m - d * R)
                                       : (alpha_per_row ? m : d);
        ld4<VEC>(alpha + ar * n + c, cnt, a4);
      }
      if (beta) ld4<VEC>(beta + d * n + c, cnt, b4);
      if (bias) ld4<VEC>(bias + c, cnt, bi);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        e[j] = 0.f;
        if (j >= cnt) continue;
        const Relax r = relax(l4[j], h4[j]);
        const float ls = alpha ? (r.active ? 1.f : (r.unstable ? a4[j] : 0.f)) : r.lo_s;
        const float ep = fmaxf(x[j], 0.f), en = fminf(x[j], 0.f);
        float v = ep * ls + en * r.up_s;
        if (beta) v = v + b4[j];
        float pp = en * r.up_t;
        if (bias) pp += v * bi[j];
        p += (double)pp;
        e[j] = v;
      }
      if (mm < M) {
        float* o = out + mm * n + c;
        if (VEC && cnt == 4) {
          *reinterpret_cast<float4*>(o) = make_float4(e[0], e[1], e[2], e[3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (j < cnt) o[j] = e[j];
        }
      }
    }
    p = row_sum16(p);
    if ((threadIdx.x & 15) == 0 && mm < M) acc[mm] = (float)((double)acc[mm] + p);
  }
}

namespace {

int backward_fc(const float* ew_in, int64_t M, int R, int n_out, const float* relu_lo,
                const float* relu_hi, const float* alpha, int alpha_per_row,
                const int64_t* alpha_group, int64_t n_groups, const float* beta, const float* W,
                const float* bias, int n_in, float* ew_out, float* acc, float* relax_out,
                int ew_bcast, vc_stream_t stream) {
  if (!ew_in || !W || !ew_out || R <= 0 || n_out <= 0 || n_in <= 0 || M < 0) return VC_ERR_ARG;
  if ((relu_lo == nullptr) != (relu_hi == nullptr)) return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  if ((relu_lo || bias) && !acc) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (M == 0) return VC_OK;
  if (relu_lo && relax_out && n_out >= kTwoPhaseMinWidth) {
    // Two phases: the relaxed rows go through HBM once (phase 1, into
    // relax_out, which the contract fills anyway), and the product runs as
    // a plain GEMM whose prologue holds no per-element arithmetic.
    const bool v1 = vec_ok({ew_in, relu_lo, relu_hi, alpha, beta, bias, relax_out}, {n_out});
    if (n_out <= kNarrowMaxWidth) {
      const int64_t grid = (M + RN - 1) / RN < kMaxGrid ? (M + RN - 1) / RN : kMaxGrid;
      if (v1)
        hipLaunchKernelGGL(k_relax_rows_narrow<true>, dim3((unsigned)grid), dim3(NT), 0, st,
                           ew_in, M, R, n_out, relu_lo, relu_hi, alpha, alpha_per_row, alpha_group, n_groups,
                           beta, bias, ew_bcast, relax_out, acc);
      else
        hipLaunchKernelGGL(k_relax_rows_narrow<false>, dim3((unsigned)grid), dim3(NT), 0, st,
                           ew_in, M, R, n_out, relu_lo, relu_hi, alpha, alpha_per_row, alpha_group, n_groups,
                           beta, bias, ew_bcast, relax_out, acc);
      VC_LAUNCH_CHECK();
      return plain_gemm(relax_out, M, n_out, W, n_in, ew_out, st);
    }
    const int64_t grid = (M + RR - 1) / RR < kMaxGrid ? (M + RR - 1) / RR : kMaxGrid;
    if (v1)
      hipLaunchKernelGGL(k_relax_rows<true>, dim3((unsigned)grid), dim3(NT), 0, st, ew_in, M, R,
                         n_out, relu_lo, relu_hi, alpha, alpha_per_row, alpha_group, n_groups, beta, bias,
                         ew_bcast, relax_out, acc);
    else
      hipLaunchKernelGGL(k_relax_rows<false>, dim3((unsigned)grid), dim3(NT), 0, st, ew_in, M, R,
                         n_out, relu_lo, relu_hi, alpha, alpha_per_row, alpha_group, n_groups, beta, bias,
                         ew_bcast, relax_out, acc);
    VC_LAUNCH_CHECK();
    return plain_gemm(relax_out, M, n_out, W, n_in, ew_out, st);
  }
  if (!relu_lo && !bias && !relax_out && !ew_bcast)
    return plain_gemm(ew_in, M, n_out, W, n_in, ew_out, st);
  LoadRelaxRow la{ew_in, n_out, R, relu_lo, relu_hi, alpha, beta, bias, alpha_per_row, relax_out,
                  ew_bcast, alpha_group, n_groups};
  const bool vec = vec_ok({ew_in, relu_lo, relu_hi, alpha, beta, W}, {n_out, n_in});
  return launch_gemm<1, true>(1, M, n_in, n_out, la, LoadW{W, n_in},
                              EpStoreBias{nullptr, ew_out, n_in}, acc, vec, st);
}

}  // namespace

extern "C" int vc_backward_fc(const float* ew_in, int64_t M, int R, int n_out,
                              const float* relu_lo, const float* relu_hi,
                              const float* alpha, int alpha_per_row, const float* beta,
                              const float* W, const float* bias, int n_in, float* ew_out,
                              float* acc, float* relax_out, int ew_bcast,
                              vc_stream_t stream) {
  return backward_fc(ew_in, M, R, n_out, relu_lo, relu_hi, alpha, alpha_per_row, nullptr, 0, beta,
                     W, bias, n_in, ew_out, acc, relax_out, ew_bcast, stream);
}

extern "C" int vc_backward_fc_grouped(const float* ew_in, int64_t M, int R, int n_out,
                                      const float* relu_lo, const float* relu_hi,
                                      const float* alpha_groups, const int64_t* group,
                                      int64_t n_groups, const float* W, const float* bias,
                                      int n_in, float* ew_out, float* acc, float* relax_out,
                                      int ew_bcast, vc_stream_t stream) {
  if (!relu_lo || !alpha_groups || !group || n_groups < 1) return VC_ERR_ARG;
  return backward_fc(ew_in, M, R, n_out, relu_lo, relu_hi, alpha_groups, 0, group, n_groups,
                     nullptr, W, bias, n_in, ew_out, acc, relax_out, ew_bcast, stream);
}

extern "C" int vc_alpha_grad_step(const float* gE, const float* P, int64_t M, int R, int n,
                                  const float* relu_lo, const float* relu_hi,
                                  const float* alpha, int p_bcast,
                                  const float* W_next, const float* bias_next, int n_next,
                                  float* g_out, vc_stream_t stream) {
  if (!gE || !P || !relu_lo || !relu_hi || !g_out || R <= 0 || n <= 0 || M < 0) return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  if (!W_next) return VC_ERR_UNSUPPORTED;
  LoadGradRelax la{gE, P, n, R, relu_lo, relu_hi, alpha, p_bcast, 0};
  const bool vec = vec_ok({gE, P, relu_lo, relu_hi, alpha, W_next}, {n});
  return launch_gemm<1, false>(1, M, n_next, n, la, LoadWt{W_next, n},
                               EpStoreBias{bias_next, g_out, n_next}, nullptr, vec,
                               (hipStream_t)stream);
}

extern "C" int vc_alpha_grad_step_rows(const float* gE, const float* P, int64_t M, int R, int n,
                                       const float* relu_lo, const float* relu_hi,
                                       const float* alpha_rows, int p_bcast,
                                       const float* W_next, const float* bias_next, int n_next,
                                       float* g_out, float* galpha_rows,
                                       vc_stream_t stream) {
  if (!gE || !P || !relu_lo || !relu_hi || !alpha_rows || !g_out || R <= 0 || n <= 0 || M < 0)
    return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  if (!W_next) return VC_ERR_UNSUPPORTED;
  LoadGradRelax la{gE, P, n, R, relu_lo, relu_hi, alpha_rows, p_bcast, 1, galpha_rows};
  const bool vec = vec_ok({gE, P, relu_lo, relu_hi, alpha_rows, W_next}, {n});
  return launch_gemm<1, false>(1, M, n_next, n, la, LoadWt{W_next, n},
                               EpStoreBias{bias_next, g_out, n_next}, nullptr, vec,
                               (hipStream_t)stream);
}

extern "C" int vc_alpha_grad_input(const float* A, const float* xl, const float* xh,
                                   int64_t M, int R, int n_in, const float* W0,
                                   const float* bias0, int n1, float* g_out,
                                   vc_stream_t stream) {
  if (!A || !xl || !xh || !W0 || !g_out || R <= 0 || n_in <= 0 || n1 <= 0) return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  const bool vec = vec_ok({A, xl, xh, W0}, {n_in});
  return launch_gemm<1, false>(1, M, n1, n_in, LoadGradInput{A, xl, xh, n_in, R},
                               LoadWt{W0, n_in}, EpStoreBias{bias0, g_out, n1}, nullptr, vec,
                               (hipStream_t)stream);
}

extern "C" int vc_relax_slopes(const float* relu_lo, const float* relu_hi, const float* alpha,
                               int64_t n, float* lo_s, float* up_s, float* up_t,
                               vc_stream_t stream) {
  if (n < 0 || (n > 0 && (!relu_lo || !relu_hi || !lo_s || !up_s || !up_t))) return VC_ERR_ARG;
  if (n == 0) return VC_OK;
  hipLaunchKernelGGL(k_relax_slopes, dim3(vc_blocks(n, NT)), dim3(NT), 0, (hipStream_t)stream,
                     relu_lo, relu_hi, alpha, n, lo_s, up_s, up_t);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

extern "C" int vc_alpha_grad_step_slopes(const float* gE, const float* P, int64_t M, int R,
                                         int n, const float* lo_s, const float* up_s,
                                         const float* up_t, int p_bcast, const float* W_next,
                                         const float* bias_next, int n_next, float* g_out,
                                         vc_stream_t stream) {
  if (!gE || !P || !lo_s || !up_s || !up_t || !g_out || R <= 0 || n <= 0 || M < 0)
    return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  if (!W_next) return VC_ERR_UNSUPPORTED;
  LoadGradSlopes la{gE, P, n, R, lo_s, up_s, up_t, p_bcast};
  const bool vec = vec_ok({gE, P, lo_s, up_s, up_t, W_next}, {n});
  return launch_gemm<1, false>(1, M, n_next, n, la, LoadWt{W_next, n},
                               EpStoreBias{bias_next, g_out, n_next}, nullptr, vec,
                               (hipStream_t)stream);
}
