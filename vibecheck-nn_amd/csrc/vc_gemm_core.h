// Core of the library's fp32 MFMA GEMMs (fc layers in vc_gemm.hip, the
// implicit-GEMM convolutions in vc_conv.hip).
//
// C[m, n] = sum_k A[m, k] * B[k, n] on 64x64 workgroup tiles: 256 threads
// (4 waves, 2 x 2), each wave a 32x32 sub-tile of 2 x 2 blocks of
// v_mfma_f32_16x16x4_f32.  The operands come from loader functors, so the
// ReLU relaxation of a CROWN backward row or the pixel gather of a
// convolution runs in registers while a tile is loaded.
//
// K runs in BK-deep tiles through two LDS buffers: the global loads of tile
// t+1 are issued into registers before the MFMAs of tile t, and the
// loader's arithmetic and the LDS store of tile t+1 follow them, so one
// barrier per tile.  Operands arrive as quads of 4 consecutive elements
// along their contiguous dimension (one 16-byte load when the host found
// every stride and base aligned).  Per-row and per-column index math is
// done once per tile, not per element.
//
// Each K-tile is reduced by MFMA into a fresh fp32 accumulator and folded
// into an fp64 running sum (two VALU ops per element), so the rounding
// error does not grow with K: the BK-term tile partials are summed exactly
// enough to round once at the end (the fp32 sums are at least as accurate
// as a blocked CPU BLAS).
//
// Tiles are dealt so that the workgroups of one XCD (blocks b with the same
// b mod 8) take consecutive tiles: the column tiles of one row block share
// that XCD's L2 for the A rows.
#pragma once
#include <initializer_list>
#include <type_traits>

#include "vc_common.h"

namespace vcg {

constexpr int NT = 256;
constexpr int PAD = 16;  // LDS row padding: MFMA fragment reads hit distinct banks

// LDS row of element kk (0 .. BK-1) of a K-tile.  Quads deliver 4
// consecutive k; element j of quad q is stored at row (BK/4) j + q, so the
// quads of a row block land in different banks.  A and B use the same map;
// the order of k inside a tile does not change the product.
template <int BK>
__device__ __forceinline__ int krow(int kk) { return (BK / 4) * (kk & 3) + (kk >> 2); }

// p[0 .. n-1] into o[0..3] (n <= 4), zeros past n; one 16-byte load when
// VEC and n == 4 (VEC: the host checked 16-byte alignment of every quad).
template <bool VEC>
__device__ __forceinline__ void ld4(const float* p, int n, float* o) {
  if (VEC && n == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
    o[3] = v.w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o[j] = 0.f;
      if (j < n) o[j] = p[j];
    }
  }
}

__device__ __forceinline__ int clamp4(int64_t v) { return v <= 0 ? 0 : (v >= 4 ? 4 : (int)v); }

// Workgroup b of n (1-D grid) -> tile index: the blocks that run on one
// XCD (same b mod 8) get one contiguous range of tiles.
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t n) {
  const int64_t q = n >> 3, rem = n & 7;
  const int64_t x = b & 7, i = b >> 3;
  return x * q + (x < rem ? x : rem) + i;
}

// Unsigned division by a runtime constant d >= 1 for n < 2^31, as one
// multiply-high, an add and a shift (the round-up method of Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994):
// l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, q = (mulhi(n, m) + n) >> l.
struct FastDiv {
  uint32_t d, m, l;
  static FastDiv make(uint32_t d) {
    uint32_t l = 0;
    while ((1u << l) < d) ++l;
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1;
    return FastDiv{d, (uint32_t)m, l};
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#ifdef __HIP_DEVICE_COMPILE__
    const uint32_t t = __umulhi(n, m);
#else
    const uint32_t t = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
    return (t + n) >> l;
  }
};

// ---------------------------------------------------------------- core
// NA: number of A/B operand pairs (1, or 2 for the dual IBP product).
// ACC_ROWS: the A loader also returns a per-element row contribution,
//   summed into acc_rows[m] by the first column tile of each row block.
// LA (A loader): Row row(bz, m, first_col_tile); Raw; fetch<VEC>(row, k, n, raw);
//   finish(row, k, n, raw, v[NA][4], KSum&) for the quad A[m][k .. k+n-1].
// LB (B loader): kTrans (quads along k of Bt[n][k], else along n of B[k][n]);
//   Col col(bz, n) per quad (n: its column, or its first column when the
//   quad runs along n), computed once per tile; fetch<VEC>(col, k, cnt,
//   raw[4]) for the quad starting at row k with cnt valid elements (zeros
//   past cnt); Raw; finish(raw, v[NA][4]).
// EP (epilogue): operator()(bz, m, n, c[NA]).
template <int NA, bool ACC_ROWS, int FM, int FN, int BK, bool VEC, class LA, class LB, class EP>
__global__ __launch_bounds__(NT) void gemm_kernel(int64_t M, int N, int K, int tiles_n,
                                                   int64_t tiles_m, int64_t n_tiles, LA la,
                                                   LB lb, EP ep, float* acc_rows) {
  constexpr int BM = 32 * FM, BN = 32 * FN;
  constexpr int SA = BM + PAD, SB = BN + PAD;
  constexpr int QR = BK / 4;     // quads per row of a K-tile
  constexpr int RP = NT / QR;    // rows covered by one pass of the workgroup
  // 32-row tiles with 16-deep K-tiles: one pass covers 64 rows, so only the
  // threads of the first 32 load A (AH)
  constexpr bool AH = BM < RP;
  constexpr int QA = AH ? 1 : BM / RP;  // A quads per thread per K-tile
  constexpr int QB = BN / RP;           // B quads per thread per K-tile
  static_assert((AH ? RP == 2 * BM : QA * RP == BM) && QB * RP == BN, "tile / thread mismatch");
  constexpr bool TB = LB::kTrans;
  __shared__ __align__(16) float As[2][NA][BK][SA];
  __shared__ __align__(16) float Bs[2][NA][BK][SB];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int wm = w >> 1, wn = w & 1;
  const int q4 = tid % QR;  // quad slot along k (A, and B when transposed)
  const int r4 = tid / QR;  // row (A) or column (transposed B) of the quad

  for (int64_t blk = blockIdx.x; blk < n_tiles; blk += gridDim.x) {
    int64_t t = xcd_tile(blk, n_tiles);
    const int tn = (int)(t % tiles_n);
    t /= tiles_n;
    const int64_t tm = t % tiles_m;
    const int64_t bz = t / tiles_m;
    const int64_t m0 = tm * BM;
    const int n0 = tn * BN;
    const bool do_rows = ACC_ROWS && tn == 0 && acc_rows != nullptr;

    typename LA::Row arow[QA];
    bool aok[QA];
    const bool a_in = !AH || r4 < BM;
#pragma unroll
    for (int p = 0; p < QA; ++p) {
      const int64_t m = m0 + r4 + RP * p;
      aok[p] = a_in && m < M;
      arow[p] = la.row(bz, aok[p] ? m : m0, tn == 0);
    }

    double acc[NA][FM][FN][4];
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[a][i][j][e] = 0.0;
    KSum rowpart[QA];

    typename LB::Col bcol[QB];
#pragma unroll
    for (int p = 0; p < QB; ++p) {
      const int n = TB ? n0 + r4 + RP * p : n0 + 4 * ((tid + NT * p) % (BN / 4));
      bcol[p] = lb.col(bz, n < N ? n : n0);
    }

    typename LA::Raw araw[QA];
    int acnt[QA];
    typename LB::Raw braw[QB];

    auto fetch = [&](int k0) {
#pragma unroll
      for (int p = 0; p < QA; ++p) {
        const int k = k0 + 4 * q4;
        acnt[p] = aok[p] ? clamp4((int64_t)K - k) : 0;
        la.template fetch<VEC>(arow[p], k, acnt[p], araw[p]);
      }
#pragma unroll
      for (int p = 0; p < QB; ++p) {
        int k, cnt;
        if (TB) {
          k = k0 + 4 * q4;
          cnt = n0 + r4 + RP * p < N ? clamp4((int64_t)K - k) : 0;
        } else {
          const int qi = tid + NT * p;
          k = k0 + qi / (BN / 4);
          cnt = k < K ? clamp4((int64_t)N - (n0 + 4 * (qi % (BN / 4)))) : 0;
        }
        lb.template fetch<VEC>(bcol[p], k, cnt, braw[p]);
      }
    };

    auto store = [&](int k0, int buf) {
      if (a_in) {
#pragma unroll
        for (int p = 0; p < QA; ++p) {
          float v[NA][4];
          la.template finish<VEC>(arow[p], k0 + 4 * q4, acnt[p], araw[p], v, rowpart[p],
                                  do_rows);
          const int mm = r4 + RP * p;
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int j = 0; j < 4; ++j) As[buf][a][QR * j + q4][mm] = v[a][j];
        }
      }
#pragma unroll
      for (int p = 0; p < QB; ++p) {
        float v[NA][4];
        LB::finish(braw[p], v);
        if (TB) {
          const int nn = r4 + RP * p;
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int j = 0; j < 4; ++j) Bs[buf][a][QR * j + q4][nn] = v[a][j];
        } else {
          const int qi = tid + NT * p;
          const int kk = qi / (BN / 4), nn = 4 * (qi % (BN / 4));
#pragma unroll
          for (int a = 0; a < NA; ++a)
            *reinterpret_cast<float4*>(&Bs[buf][a][krow<BK>(kk)][nn]) =
                make_float4(v[a][0], v[a][1], v[a][2], v[a][3]);
        }
      }
    };

    fetch(0);
    store(0, 0);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < K; k0 += BK) {
      const bool more = k0 + BK < K;
      if (more) fetch(k0 + BK);
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        v4f tt[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) tt[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < BK / 4; ++ks) {
          float af[FM], bf[FN];
#pragma unroll
          for (int i = 0; i < FM; ++i) af[i] = As[buf][a][4 * ks + g][wm * 16 * FM + 16 * i + r];
#pragma unroll
          for (int j = 0; j < FN; ++j) bf[j] = Bs[buf][a][4 * ks + g][wn * 16 * FN + 16 * j + r];
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) tt[i][j] = mfma16x16x4(af[i], bf[j], tt[i][j]);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[a][i][j][e] += (double)tt[i][j][e];
      }
      if (more) store(k0 + BK, buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }

    if (do_rows) {
#pragma unroll
      for (int p = 0; p < QA; ++p) {
        float v = rowpart[p].value();
#pragma unroll
        for (int o = 1; o < QR; o <<= 1) v += __shfl_xor(v, o, 64);
        if (q4 == 0 && aok[p]) acc_rows[m0 + r4 + RP * p] += v;
      }
    }

#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t m = m0 + wm * 16 * FM + i * 16 + 4 * g + e;
          const int n = n0 + wn * 16 * FN + j * 16 + r;
          if (m < M && n < N) {
            float c[NA];
#pragma unroll
            for (int a = 0; a < NA; ++a) c[a] = (float)acc[a][i][j][e];
            ep(bz, m, n, c);
          }
        }
  }
}

constexpr int64_t kMaxGrid = 1 << 20;  // workgroups; tiles beyond loop (a multiple of 8)

constexpr int64_t kFewTiles = 512;  // two 64x64 tiles per CU (2048 measured: mixed, mostly slower)

// Loaders opt into 32-row tiles for M <= 32 with a static kSmallM = true.
template <class T, class = void>
struct small_m_ok : std::false_type {};
template <class T>
struct small_m_ok<T, std::void_t<decltype(T::kSmallM)>> : std::bool_constant<T::kSmallM> {};

template <int NA, bool ACC_ROWS, int FM, class LA, class LB, class EP>
int launch_fm(int64_t batch, int64_t M, int N, int K, LA la, LB lb, EP ep, float* acc_rows,
              bool vec, hipStream_t st) {
  constexpr int FN = 2, BM = 32 * FM, BN = 32 * FN, BK = LA::kBK;
  const int tiles_n = (N + BN - 1) / BN;
  const int64_t tiles_m = (M + BM - 1) / BM;
  const int64_t n_tiles = batch * tiles_m * tiles_n;
  const int64_t grid = n_tiles < kMaxGrid ? n_tiles : kMaxGrid;
  if (vec)
    hipLaunchKernelGGL((gemm_kernel<NA, ACC_ROWS, FM, FN, BK, true, LA, LB, EP>),
                       dim3((unsigned)grid), dim3(NT), 0, st, M, N, K, tiles_n, tiles_m, n_tiles,
                       la, lb, ep, acc_rows);
  else
    hipLaunchKernelGGL((gemm_kernel<NA, ACC_ROWS, FM, FN, BK, false, LA, LB, EP>),
                       dim3((unsigned)grid), dim3(NT), 0, st, M, N, K, tiles_n, tiles_m, n_tiles,
                       la, lb, ep, acc_rows);
  VC_LAUNCH_CHECK();
  return VC_OK;
}

// One tile shape, 64x64 (FM = FN = 2), for every GEMM: measured on MI355X
// against 128x64 and 128x128 at the workload shapes (1024-wide fc backward,
// 256-wide spec backward, 784->256 interval fc, 1024x1024 zonotope
// generators), the small tile wins everywhere, because it keeps 3-4 waves
// per SIMD to cover the global-load latency.  Loaders that declare kSmallM
// (the convolutions, whose row count is a channel count) get 32x64 tiles
// when M <= 32.  The K-tile depth comes from the A loader: 32 for plain
// loads (fewer barriers, the fold every 32 k), 16 when the loader's
// per-element arithmetic holds more registers.
template <int NA, bool ACC_ROWS, class LA, class LB, class EP>
int launch_gemm(int64_t batch, int64_t M, int N, int K, LA la, LB lb, EP ep, float* acc_rows,
                bool vec, hipStream_t st) {
  if (M <= 0 || N <= 0 || batch <= 0) return VC_OK;
  if constexpr (small_m_ok<LA>::value) {
    if (M <= 32) return launch_fm<NA, ACC_ROWS, 1>(batch, M, N, K, la, lb, ep, acc_rows, vec, st);
  }
  // fewer 64-row tiles than kFewTiles: 32-row tiles double the workgroups
  // of a launch that would leave CUs without a second workgroup
  if (batch * ((M + 63) / 64) * ((N + 63) / 64) < kFewTiles)
    return launch_fm<NA, ACC_ROWS, 1>(batch, M, N, K, la, lb, ep, acc_rows, vec, st);
  return launch_fm<NA, ACC_ROWS, 2>(batch, M, N, K, la, lb, ep, acc_rows, vec, st);
}

// every pointer 16-byte aligned and every stride a multiple of 4 floats
inline bool vec_ok(std::initializer_list<const void*> ptrs,
                          std::initializer_list<int64_t> strides) {
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return false;
  for (int64_t s : strides)
    if (s % 4) return false;
  return true;
}


// ------------------------------------------------------------ shared loaders
struct LoadRow {  // A[m][k] plain (row-major, ld)
  static constexpr int kBK = 32;
  const float* A;
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
    ld4<VEC>(A + rw.o + k, n, x.x);
  }
  template <bool VEC>
  __device__ void finish(const Row&, int, int, const Raw& x, float (*v)[4], KSum&, bool) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[0][j] = x.x[j];
  }
};

struct LoadW {  // B[k][n] = W[k][n]
  static constexpr bool kTrans = false;
  const float* W;
  int ld;
  struct Col {
    int n;
  };
  struct Raw {
    float x[4];
  };
  __device__ Col col(int64_t, int n) const { return Col{n}; }
  template <bool VEC>
  __device__ void fetch(const Col& c, int k, int cnt, Raw& r) const {
    float* o = r.x;
    ld4<VEC>(W + (int64_t)k * ld + c.n, cnt, o);
  }
  __device__ static void finish(const Raw& r, float (*v)[4]) {
    const float* x = r.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[0][j] = x[j];
  }
};

struct LoadWt {  // B[k][n] = W[n][k]
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
    for (int j = 0; j < 4; ++j) v[0][j] = x[j];
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

}  // namespace vcg
