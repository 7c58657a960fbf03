// Generic fp32 MFMA GEMM with fused prologues/epilogues.
//
// C[m, n] = sum_k A[m, k] * B[k, n] on a 64x64 workgroup tile, BK = 16,
// 256 threads = 4 waves in a 2x2 arrangement, each wave owning a 32x32
// sub-tile of 2x2 blocks of v_mfma_f32_16x16x4_f32.  A and B tiles are
// staged through LDS; the A loader is a functor, so the ReLU relaxation of
// the CROWN backward (pos/neg split, slope select, acc += neg . up_t and
// acc += e . bias) runs in registers while the tile is loaded.
#include "vc_common.h"
#include "vc_relax.h"

namespace {

constexpr int BM = 64, BN = 64, BK = 16;
constexpr int LDA_S = BM + 16;  // padded LDS row stride (bank spread)
constexpr int LDB_S = BN + 16;
constexpr int NT = 256;

// ---------------------------------------------------------------- core
// NA: number of A operands (1, or 2 for the dual IBP product).
// TRANS_B: B is given as Bt[n][k] (k contiguous) instead of B[k][n].
// ACC_ROWS: the loader returns a per-element row contribution summed into
//   acc[m] by the blockIdx.y == 0 column of tiles.
template <int NA, bool TRANS_B, bool ACC_ROWS, class LA, class LB, class EP>
__global__ __launch_bounds__(NT) void gemm_kernel(int64_t M, int N, int K,
                                                   int tiles_n, LA la, LB lb,
                                                   EP ep, float* acc_rows) {
  __shared__ float As[NA][BK][LDA_S];
  __shared__ float Bs[NA][BK][LDB_S];
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int wm = w >> 1, wn = w & 1;
  const int64_t bz = blockIdx.x / tiles_n;
  const int bx = blockIdx.x % tiles_n;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int n0 = bx * BN;

  // Running sums with TwoSum compensation: each BK-deep K-tile is reduced
  // by MFMA into a fresh accumulator and then folded into (acc, cmp), so
  // the rounding error no longer grows with K (the fp32 sums are at least
  // as accurate as a blocked CPU BLAS).
  v4f acc[NA][2][2], cmp[NA][2][2];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[a][i][j] = v4f{0.f, 0.f, 0.f, 0.f};
        cmp[a][i][j] = v4f{0.f, 0.f, 0.f, 0.f};
      }

  KSum rowpart[4];
  const bool do_rows = ACC_ROWS && (bx == 0) && acc_rows != nullptr;

  for (int k0 = 0; k0 < K; k0 += BK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + NT * i;
      const int mm = idx >> 4, kk = idx & 15;
      const int64_t m = m0 + mm;
      const int k = k0 + kk;
      float v[NA];
      float part = 0.f;
      if (m < M && k < K) {
        la(bz, m, k, v, part);
      } else {
#pragma unroll
        for (int a = 0; a < NA; ++a) v[a] = 0.f;
      }
      if (do_rows) rowpart[i].add(part);
#pragma unroll
      for (int a = 0; a < NA; ++a) As[a][kk][mm] = v[a];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = tid + NT * i;
      int kk, nn;
      if (TRANS_B) {
        nn = idx >> 4;
        kk = idx & 15;
      } else {
        kk = idx >> 6;
        nn = idx & 63;
      }
      const int k = k0 + kk, n = n0 + nn;
      float v[NA];
      if (k < K && n < N) {
        lb(bz, k, n, v);
      } else {
#pragma unroll
        for (int a = 0; a < NA; ++a) v[a] = 0.f;
      }
#pragma unroll
      for (int a = 0; a < NA; ++a) Bs[a][kk][nn] = v[a];
    }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      v4f t[2][2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) t[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < BK / 4; ++ks) {
        float af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) af[i] = As[a][ks * 4 + g][wm * 32 + i * 16 + r];
#pragma unroll
        for (int j = 0; j < 2; ++j) bf[j] = Bs[a][ks * 4 + g][wn * 32 + j * 16 + r];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) t[i][j] = mfma16x16x4(af[i], bf[j], t[i][j]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float s = acc[a][i][j][e], c = cmp[a][i][j][e];
            two_sum_acc(s, c, t[i][j][e]);
            acc[a][i][j][e] = s;
            cmp[a][i][j][e] = c;
          }
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[a][i][j] += cmp[a][i][j];

  if (do_rows) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float p = rowpart[i].value();
      p += __shfl_xor(p, 8, 16);
      p += __shfl_xor(p, 4, 16);
      p += __shfl_xor(p, 2, 16);
      p += __shfl_xor(p, 1, 16);
      const int64_t m = m0 + ((tid + NT * i) >> 4);
      if ((tid & 15) == 0 && m < M) acc_rows[m] += p;
    }
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm * 32 + i * 16 + 4 * g + e;
        const int n = n0 + wn * 32 + j * 16 + r;
        if (m < M && n < N) {
          float c[NA];
#pragma unroll
          for (int a = 0; a < NA; ++a) c[a] = acc[a][i][j][e];
          ep(bz, m, n, c);
        }
      }
}

template <int NA, bool TRANS_B, bool ACC_ROWS, class LA, class LB, class EP>
int launch_gemm(int64_t batch, int64_t M, int N, int K, LA la, LB lb, EP ep,
                float* acc_rows, hipStream_t st) {
  if (M <= 0 || N <= 0 || batch <= 0) return VC_OK;
  const int tiles_n = (N + BN - 1) / BN;
  const int64_t tiles_m = (M + BM - 1) / BM;
  if (tiles_m > 2147483647LL || batch * tiles_n > 2147483647LL) return VC_ERR_ARG;
  dim3 grid((unsigned)(batch * tiles_n), (unsigned)tiles_m);
  hipLaunchKernelGGL((gemm_kernel<NA, TRANS_B, ACC_ROWS, LA, LB, EP>), grid,
                     dim3(NT), 0, st, M, N, K, tiles_n, la, lb, ep, acc_rows);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

// ------------------------------------------------------------- functors
struct LoadMidRad {  // A = (mid, rad) of an interval row-block
  const float *l, *h;
  int ld;
  __device__ void operator()(int64_t, int64_t m, int k, float* v, float&) const {
    const float lo = l[m * ld + k], hi = h[m * ld + k];
    v[0] = (lo + hi) / 2.f;
    v[1] = (hi - lo) / 2.f;
  }
};
struct LoadWtAbs {  // B[k][n] = (W[n][k], |W[n][k]|)
  const float* W;
  int ld;
  __device__ void operator()(int64_t, int k, int n, float* v) const {
    const float w = W[(int64_t)n * ld + k];
    v[0] = w;
    v[1] = fabsf(w);
  }
};
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

struct LoadRow {  // A[m][k] plain
  const float* A;
  int ld;
  __device__ void operator()(int64_t, int64_t m, int k, float* v, float&) const {
    v[0] = A[m * ld + k];
  }
};
struct LoadWt {  // B[k][n] = W[n][k]
  const float* W;
  int ld;
  __device__ void operator()(int64_t, int k, int n, float* v) const {
    v[0] = W[(int64_t)n * ld + k];
  }
};
struct LoadW {  // B[k][n] = W[k][n]
  const float* W;
  int ld;
  __device__ void operator()(int64_t, int k, int n, float* v) const {
    v[0] = W[(int64_t)k * ld + n];
  }
};
struct EpStoreBias {
  const float* bias;
  float* out;
  int ld;
  __device__ void operator()(int64_t, int64_t m, int n, const float* c) const {
    out[m * ld + n] = bias ? c[0] + bias[n] : c[0];
  }
};

// Zonotope generators: A = W (shared), B = G[b] (n_in x K), out G_out[b].
struct LoadWshared {
  const float* W;
  int ld;
  __device__ void operator()(int64_t, int64_t m, int k, float* v, float&) const {
    v[0] = W[m * ld + k];
  }
};
struct LoadGen {
  const float* G;
  int64_t stride_b;
  int ld;
  __device__ void operator()(int64_t bz, int k, int n, float* v) const {
    v[0] = G[bz * stride_b + (int64_t)k * ld + n];
  }
};
struct EpGen {
  float* G;
  int64_t stride_b;
  int ld;
  __device__ void operator()(int64_t bz, int64_t m, int n, const float* c) const {
    G[bz * stride_b + m * ld + n] = c[0];
  }
};

// CROWN backward: relaxation of ew rows at a relu, then the fc product.
struct LoadRelaxRow {
  const float* ew;
  int ld;  // n_out
  int R;
  const float *lo, *hi, *alpha, *beta, *bias;
  int alpha_per_row;
  float* relax_out;
  int ew_bcast;  // rows shared by all domains: row m reads ew[m % R]
  __device__ void operator()(int64_t, int64_t m, int k, float* v, float& part) const {
    const float x = ew[(ew_bcast ? m % R : m) * ld + k];
    float e = x, p = 0.f;
    if (lo) {
      const int64_t d = m / R;
      const int64_t bi = d * ld + k;
      Relax s = relax(lo[bi], hi[bi]);
      float ls = s.lo_s;
      if (alpha) {
        const float a = alpha_per_row ? alpha[m * ld + k] : alpha[bi];
        ls = s.active ? 1.f : (s.unstable ? a : 0.f);
      }
      const float ep = fmaxf(x, 0.f), en = fminf(x, 0.f);
      e = ep * ls + en * s.up_s;
      if (beta) e = e + beta[bi];
      p = en * s.up_t;
    }
    if (bias) p += e * bias[k];
    if (relax_out) relax_out[m * ld + k] = e;
    v[0] = e;
    part = p;
  }
};

// alpha gradient sweep: gP = gE * (mpos ls + mneg up_s) + mneg up_t.
struct LoadGradRelax {
  const float *gE, *P;
  int ld, R;
  const float *lo, *hi, *alpha;
  int p_bcast;  // P shared by all domains: row m reads P[m % R]
  __device__ void operator()(int64_t, int64_t m, int k, float* v, float&) const {
    const int64_t bi = (m / R) * ld + k;
    const float ge = gE[m * ld + k], pv = P[(p_bcast ? m % R : m) * ld + k];
    Relax s = relax(lo[bi], hi[bi]);
    float ls = s.lo_s;
    if (alpha) ls = s.active ? 1.f : (s.unstable ? alpha[bi] : 0.f);
    const bool mp = pv >= 0.f, mn = pv <= 0.f;
    float f = (mp ? ls : 0.f) + (mn ? s.up_s : 0.f);
    float gp = ge * f;
    if (mn) gp += s.up_t;
    v[0] = gp;
  }
};
struct LoadGradInput {  // gA = xl [A >= 0] + xh [A <= 0]
  const float *A, *xl, *xh;
  int ld, R;
  __device__ void operator()(int64_t, int64_t m, int k, float* v, float&) const {
    const float a = A[m * ld + k];
    const int64_t bi = (m / R) * ld + k;
    float gv = 0.f;
    if (a >= 0.f) gv += xl[bi];
    if (a <= 0.f) gv += xh[bi];
    v[0] = gv;
  }
};

}  // namespace

extern "C" int vc_ibp_fc(const float* l, const float* h, int64_t B, int n_in,
                         const float* W, const float* bias, int n_out, float* lo,
                         float* hi, vc_stream_t stream) {
  if (!l || !h || !W || !lo || !hi || n_in <= 0 || n_out <= 0 || B < 0) return VC_ERR_ARG;
  return launch_gemm<2, true, false>(1, B, n_out, n_in, LoadMidRad{l, h, n_in},
                                     LoadWtAbs{W, n_in}, EpIbp{bias, lo, hi, n_out},
                                     nullptr, (hipStream_t)stream);
}

extern "C" int vc_zono_fc(const float* c, const float* G, int64_t B, int n_in, int K,
                          const float* W, const float* bias, int n_out, float* c_out,
                          float* G_out, vc_stream_t stream) {
  if (!c || !W || !c_out || n_in <= 0 || n_out <= 0 || B < 0 || K < 0) return VC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_gemm<1, true, false>(1, B, n_out, n_in, LoadRow{c, n_in}, LoadWt{W, n_in},
                                       EpStoreBias{bias, c_out, n_out}, nullptr, st);
  if (rc != VC_OK || K == 0 || B == 0) return rc;
  if (!G || !G_out) return VC_ERR_ARG;
  return launch_gemm<1, false, false>(B, n_out, K, n_in, LoadWshared{W, n_in},
                                      LoadGen{G, (int64_t)n_in * K, K},
                                      EpGen{G_out, (int64_t)n_out * K, K}, nullptr, st);
}

extern "C" int vc_backward_fc(const float* ew_in, int64_t M, int R, int n_out,
                              const float* relu_lo, const float* relu_hi,
                              const float* alpha, int alpha_per_row, const float* beta,
                              const float* W, const float* bias, int n_in, float* ew_out,
                              float* acc, float* relax_out, int ew_bcast,
                              vc_stream_t stream) {
  if (!ew_in || !W || !ew_out || R <= 0 || n_out <= 0 || n_in <= 0 || M < 0) return VC_ERR_ARG;
  if ((relu_lo == nullptr) != (relu_hi == nullptr)) return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  if ((relu_lo || bias) && !acc) return VC_ERR_ARG;
  LoadRelaxRow la{ew_in, n_out, R, relu_lo, relu_hi, alpha, beta, bias, alpha_per_row, relax_out,
                  ew_bcast};
  return launch_gemm<1, false, true>(1, M, n_in, n_out, la, LoadW{W, n_in},
                                     EpStoreBias{nullptr, ew_out, n_in}, acc,
                                     (hipStream_t)stream);
}

extern "C" int vc_alpha_grad_step(const float* gE, const float* P, int64_t M, int R, int n,
                                  const float* relu_lo, const float* relu_hi,
                                  const float* alpha, int p_bcast,
                                  const float* W_next, const float* bias_next, int n_next,
                                  float* g_out, vc_stream_t stream) {
  if (!gE || !P || !relu_lo || !relu_hi || !g_out || R <= 0 || n <= 0 || M < 0) return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  if (!W_next) return VC_ERR_UNSUPPORTED;
  LoadGradRelax la{gE, P, n, R, relu_lo, relu_hi, alpha, p_bcast};
  return launch_gemm<1, true, false>(1, M, n_next, n, la, LoadWt{W_next, n},
                                     EpStoreBias{bias_next, g_out, n_next}, nullptr,
                                     (hipStream_t)stream);
}

extern "C" int vc_alpha_grad_input(const float* A, const float* xl, const float* xh,
                                   int64_t M, int R, int n_in, const float* W0,
                                   const float* bias0, int n1, float* g_out,
                                   vc_stream_t stream) {
  if (!A || !xl || !xh || !W0 || !g_out || R <= 0 || n_in <= 0 || n1 <= 0) return VC_ERR_ARG;
  if (M % R != 0) return VC_ERR_ARG;
  return launch_gemm<1, true, false>(1, M, n1, n_in, LoadGradInput{A, xl, xh, n_in, R},
                                     LoadWt{W0, n_in}, EpStoreBias{bias0, g_out, n1},
                                     nullptr, (hipStream_t)stream);
}
