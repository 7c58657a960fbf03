// One input-split BaB round on the narrow-MLP kernels, orchestrated on the
// host in C++ (verify_graph.py:12855-13382 as restated by bab_step in
// vibecheck_amd/verify_graph.py): zonotope bounds, CROWN intermediate bounds
// with the spec bound and its input linearization, closure, alpha-CROWN on
// the open leaves, closure again, one halfspace clip, widest-axis
// bisection.  Every step is one of the library's entry points on the
// caller's stream; the three counts the round needs on the host (open,
// unclosed, feasible + split) are read with a stream synchronisation each,
// with no interpreter between a count and the launches that use it.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "vc_common.h"
#include "vc_mlp_common.h"

namespace {

using vcm::MAXL;

// Bump allocation of the round's buffers from the caller's workspace (or,
// with base == nullptr, the size of that layout).
struct Carve {
  char* base;
  size_t used;
  template <class T>
  T* take(int64_t n) {
    const size_t bytes = ((size_t)std::max<int64_t>(n, 1) * sizeof(T) + 255) & ~(size_t)255;
    T* r = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += bytes;
    return r;
  }
};

// The bound phase's buffers for B boxes.
struct BoundBufs {
  float *sb_lo[MAXL], *sb_hi[MAXL];  // zonotope bounds (B, d_L)
  float *t_lo[MAXL], *t_hi[MAXL];    // CROWN bounds (B, d_L)
  uint8_t* ovf;                      // zonotope overflow flags (B)
  int64_t* idx;                      // overflow / open-leaf list (B)
  int64_t* cnt;                      // counts [4]
  int32_t* uidx;                     // union lists (sum d)
  int32_t* umeta;                    // union counts and offsets (2 n)
  unsigned long long* umask;         // union as bit masks [MAXL]
  int32_t* queue;                    // work counters [2]
  void* rws;                         // layer-synchronous CROWN workspace (large B)
  int64_t rws_bytes;
};

// The clip and split phases' buffers for B leaves.
struct TailBufs {
  int64_t *idx, *idx2, *cnt;  // compaction outputs (B) and counts [4]
  void* cws;                  // compaction workspace
  int64_t cws_bytes;
  float *u_xl, *u_xh, *u_A, *u_acc, *c_xl, *c_xh;
  int64_t* ax_u;
  uint8_t *usable, *split;
};

struct RoundBufs {
  BoundBufs b;
  TailBufs t;  // shares the bound phase's list and counts
  // alpha on the open leaves (sized for B)
  float *a_lo[MAXL], *a_hi[MAXL];
  float *a_xl, *a_xh, *a_state, *a_lb, *a_best, *a_ctl;
};

// The next round's bound phase as a round with lookahead hands it over,
// for its B kept children in the order of the next batch: the spec bound,
// its input linearization and the zonotope bounds alpha starts from, and
// the counters that round starts from (cnt[3], its open-leaf count, zero).
struct Handoff {
  float *lb, *A, *acc;
  float *sb_lo[MAXL], *sb_hi[MAXL];
  int64_t* cnt;  // [4]
};

// The lookahead's buffers: the handoff (reserved for cap rows, laid out for
// the kept count), the clip and split of the CROWN-open leaves of a B-box
// round, their children (at most cap) with the bound phase's outputs, and
// the compactions to what alpha leaves open.  The children's BoundBufs
// follow at bound_off, carved for their actual count.
struct LookBufs {
  Handoff h;
  uint8_t* closed_c;  // the CROWN closure (B)
  int64_t* unc;       // the CROWN-unclosed leaves (B)
  uint8_t* feas;      // (B)
  TailBufs t;
  float *cxl, *cxh;   // children, the high halves first (cap, n_in)
  float *b_lb, *b_A, *b_acc;
  // closed-after-alpha flags of the unclosed leaves, of the feasible ones
  // (B) and of the children (cap); the kept positions of each
  uint8_t *fu, *ff, *drop;
  int64_t *ku, *kf, *kidx;
  int64_t* fidx;      // the kept feasible leaves' rows of the clipped boxes (B)
  void* kws;
  int64_t kws_bytes;
  size_t bound_off;
};

void carve_bound(Carve& c, BoundBufs& b, const int32_t* dims, int n, int64_t B) {
  // batches above 4 x CUs take the layer-synchronous CROWN, which needs no
  // buffers for the CROWN bounds
  b.rws_bytes = vc_mlp_tiled_crown_mode(B) == 0 ? vc_mlp_crown_rows_workspace(dims, n, B) : 0;
  if (b.rws_bytes < 0) b.rws_bytes = 0;
  int sumd = 0;
  for (int l = 0; l < n; ++l) {
    const int d = dims[l + 1];
    sumd += d;
    b.sb_lo[l] = c.take<float>(B * d);
    b.sb_hi[l] = c.take<float>(B * d);
    b.t_lo[l] = b.rws_bytes > 0 ? nullptr : c.take<float>(B * d);
    b.t_hi[l] = b.rws_bytes > 0 ? nullptr : c.take<float>(B * d);
  }
  b.ovf = c.take<uint8_t>(B);
  b.idx = c.take<int64_t>(B);
  b.cnt = c.take<int64_t>(4);
  b.uidx = c.take<int32_t>(sumd);
  b.umeta = c.take<int32_t>(2 * n);
  b.umask = c.take<unsigned long long>(MAXL);
  b.queue = c.take<int32_t>(2);
  b.rws = b.rws_bytes > 0 ? c.take<char>(b.rws_bytes) : nullptr;
}

// idx and cnt come from the caller (the round's own share the bound
// phase's).
void carve_tail(Carve& c, TailBufs& t, int n_in, int Q, int64_t B) {
  t.idx2 = c.take<int64_t>(B);
  t.cws_bytes = vc_compact_workspace(B);
  t.cws = c.take<char>(t.cws_bytes);
  t.u_xl = c.take<float>(B * n_in);
  t.u_xh = c.take<float>(B * n_in);
  t.u_A = c.take<float>(B * Q * n_in);
  t.u_acc = c.take<float>(B * Q);
  t.c_xl = c.take<float>(B * n_in);
  t.c_xh = c.take<float>(B * n_in);
  t.ax_u = c.take<int64_t>(B);
  t.usable = c.take<uint8_t>(B);
  t.split = c.take<uint8_t>(B);
}

void carve(Carve& c, RoundBufs& r, const int32_t* dims, int n, int64_t B, int Q) {
  const int n_in = dims[0];
  carve_bound(c, r.b, dims, n, B);
  int sumd = 0;
  for (int l = 0; l < n; ++l) {
    const int d = dims[l + 1];
    sumd += d;
    r.a_lo[l] = c.take<float>(B * d);
    r.a_hi[l] = c.take<float>(B * d);
  }
  r.t.idx = r.b.idx;
  r.t.cnt = r.b.cnt;
  carve_tail(c, r.t, n_in, Q, B);
  r.a_xl = c.take<float>(B * n_in);
  r.a_xh = c.take<float>(B * n_in);
  r.a_state = c.take<float>(3 * (int64_t)sumd * B);
  r.a_lb = c.take<float>((int64_t)VC_ALPHA_CHUNK * B * Q);
  r.a_best = c.take<float>(B * Q);
  r.a_ctl = c.take<float>(4);
}

void carve_handoff(Carve& c, Handoff& h, const int32_t* dims, int n, int64_t B, int Q) {
  const int n_in = dims[0];
  h.lb = c.take<float>(B * Q);
  h.A = c.take<float>(B * Q * n_in);
  h.acc = c.take<float>(B * Q);
  for (int l = 0; l < n; ++l) {
    h.sb_lo[l] = c.take<float>(B * dims[l + 1]);
    h.sb_hi[l] = c.take<float>(B * dims[l + 1]);
  }
  h.cnt = c.take<int64_t>(4);
}

void carve_look(Carve& c, LookBufs& L, const int32_t* dims, int n, int64_t B, int Q,
                int64_t cap) {
  const int n_in = dims[0];
  carve_handoff(c, L.h, dims, n, cap, Q);
  L.closed_c = c.take<uint8_t>(B);
  L.unc = c.take<int64_t>(B);
  L.feas = c.take<uint8_t>(B);
  L.t.idx = c.take<int64_t>(B);
  L.t.cnt = c.take<int64_t>(4);
  carve_tail(c, L.t, n_in, Q, B);
  L.cxl = c.take<float>(cap * n_in);
  L.cxh = c.take<float>(cap * n_in);
  L.b_lb = c.take<float>(cap * Q);
  L.b_A = c.take<float>(cap * Q * n_in);
  L.b_acc = c.take<float>(cap * Q);
  L.fu = c.take<uint8_t>(B);
  L.ff = c.take<uint8_t>(B);
  L.drop = c.take<uint8_t>(cap);
  L.ku = c.take<int64_t>(B);
  L.kf = c.take<int64_t>(B);
  L.kidx = c.take<int64_t>(cap);
  L.fidx = c.take<int64_t>(B);
  L.kws_bytes = vc_compact_workspace(cap);
  L.kws = c.take<char>(L.kws_bytes);
  L.bound_off = c.used;
}

}  // namespace

extern "C" int64_t vc_mlp_bab_round_workspace(const int32_t* dims, int n_relu, int64_t B,
                                              int Q) {
  if (!dims || n_relu < 1 || n_relu > MAXL || B < 0 || Q < 1) return -VC_ERR_ARG;
  Carve c{nullptr, 0};
  RoundBufs r;
  carve(c, r, dims, n_relu, B, Q);
  return (int64_t)c.used;
}

extern "C" int64_t vc_mlp_bab_round_lookahead_workspace(const int32_t* dims, int n_relu,
                                                        int64_t B, int Q, int64_t cap) {
  if (!dims || n_relu < 1 || n_relu > MAXL || B < 0 || Q < 1 || cap < 0) return -VC_ERR_ARG;
  Carve c{nullptr, 0};
  LookBufs L;
  carve_look(c, L, dims, n_relu, B, Q, cap);
  // the children's bound phase, in either CROWN form their count may take
  const size_t at = c.used;
  BoundBufs bb;
  carve_bound(c, bb, dims, n_relu, cap);
  const size_t big = c.used;
  c.used = at;
  carve_bound(c, bb, dims, n_relu, std::min<int64_t>(cap, (int64_t)vcm::cu_count() * 4));
  return (int64_t)std::max(big, c.used);
}

extern "C" int vc_mlp_bab_round_handoff_offsets(const int32_t* dims, int n_relu, int64_t B,
                                                int Q, int64_t* off) {
  if (!dims || !off || n_relu < 1 || n_relu > MAXL || B < 0 || Q < 1) return VC_ERR_ARG;
  Carve c{reinterpret_cast<char*>(256), 0};  // any aligned base: offsets only
  Handoff h;
  carve_handoff(c, h, dims, n_relu, B, Q);
  off[0] = reinterpret_cast<char*>(h.lb) - reinterpret_cast<char*>(256);
  off[1] = reinterpret_cast<char*>(h.A) - reinterpret_cast<char*>(256);
  off[2] = reinterpret_cast<char*>(h.acc) - reinterpret_cast<char*>(256);
  return VC_OK;
}

namespace {

// alpha's evaluated-iteration count (ctl[2]) as a device count.
__global__ void k_ctl_count(const float* __restrict__ ctl, int64_t* out) {
  if (threadIdx.x == 0) *out = (int64_t)ctl[2];
}

// Device counts to pinned host words, stored by the GPU (system scope);
// with ctl, word k is the alpha loop's evaluated iterations (ctl[2]).
__global__ void k_counts_to_host(const int64_t* __restrict__ dev, int k, int64_t* host,
                                 const float* __restrict__ ctl) {
  if (threadIdx.x < k)
    __hip_atomic_store(host + threadIdx.x, dev[threadIdx.x], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
  if (ctl && threadIdx.x == k)
    __hip_atomic_store(host + k, (int64_t)ctl[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// k counts from the device once every launch before them has run.  With
// pinned host words the GPU stores them there and the host polls (no copy,
// no wake-up latency); the poll is bounded, then the stream is synchronised
// and the counts are read from device memory.
// With ctl, one more count follows the k: the alpha loop's evaluated
// iterations (host[k]; dev[k] is then scratch for the fallback).
// post_counts enqueues the store, wait_counts reads (the host can enqueue
// other streams' work in between); read_counts does both.
int post_counts(const int64_t* dev, int k, int64_t* pinned, hipStream_t st,
                const float* ctl = nullptr) {
  if (!pinned) return VC_OK;
  const int kk = ctl ? k + 1 : k;
  volatile int64_t* pw = pinned;
  for (int i = 0; i < kk; ++i) pw[i] = -1;
  hipLaunchKernelGGL(k_counts_to_host, dim3(1), dim3(64), 0, st, dev, k, pinned, ctl);
  return hipGetLastError() == hipSuccess ? VC_OK : VC_ERR_LAUNCH;
}

int wait_counts(const int64_t* dev, int k, int64_t* host, int64_t* pinned, hipStream_t st,
                const float* ctl = nullptr) {
  const int kk = ctl ? k + 1 : k;
  if (pinned) {
    volatile int64_t* pw = pinned;
    for (long spin = 0; spin < (1l << 26); ++spin) {
      bool ready = true;
      for (int i = 0; i < kk; ++i) ready = ready && pw[i] >= 0;
      if (ready) {
        for (int i = 0; i < kk; ++i) host[i] = pw[i];
        return VC_OK;
      }
    }
  }
  if (ctl) {
    hipLaunchKernelGGL(k_ctl_count, dim3(1), dim3(64), 0, st, ctl, const_cast<int64_t*>(dev) + k);
    if (hipGetLastError() != hipSuccess) return VC_ERR_LAUNCH;
  }
  if (hipMemcpyAsync(host, dev, sizeof(int64_t) * kk, hipMemcpyDeviceToHost, st) != hipSuccess)
    return VC_ERR_LAUNCH;
  return hipStreamSynchronize(st) == hipSuccess ? VC_OK : VC_ERR_LAUNCH;
}

int read_counts(const int64_t* dev, int k, int64_t* host, int64_t* pinned, hipStream_t st,
                const float* ctl = nullptr) {
  const int rc = post_counts(dev, k, pinned, st, ctl);
  return rc != VC_OK ? rc : wait_counts(dev, k, host, pinned, st, ctl);
}

// Clip shrink accounting of the phase timer: w[0] += sum of max(xh - xl, 0)
// over the n values before the clip, w[1] += the same after it.  Double
// atomics per wavefront (any order: a profiling ratio, not a bound).
__global__ void k_clip_widths(const float* __restrict__ xl, const float* __restrict__ xh,
                              const float* __restrict__ cl, const float* __restrict__ ch,
                              int64_t n, double* w) {
  double a = 0.0, b = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    a += (double)fmaxf(xh[i] - xl[i], 0.0f);
    b += (double)fmaxf(ch[i] - cl[i], 0.0f);
  }
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_down(a, o, 64);
    b += __shfl_down(b, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(w, a);
    atomicAdd(w + 1, b);
  }
}

// vc_gather_rows_multi in launches of at most 32 arrays.
int gather(const float* const* in, float* const* out, const int32_t* cols, int n_arrays,
           const int64_t* idx, int64_t n_rows, vc_stream_t stream) {
  for (int a0 = 0; a0 < n_arrays; a0 += 32) {
    const int k = std::min(32, n_arrays - a0);
    const int rc = vc_gather_rows_multi(in + a0, out + a0, cols + a0, k, idx, n_rows, stream);
    if (rc != VC_OK) return rc;
  }
  return VC_OK;
}

}  // namespace

#define VC_TRY(x)                 \
  do {                            \
    const int rc_ = (x);          \
    if (rc_ != VC_OK) return rc_; \
  } while (0)

namespace {

// The round's phases, in the order the phase timer's events close them.
enum RoundPhase { PH_BOUND = 0, PH_ALPHA = 1, PH_CLIP = 2, PH_SPLIT = 3 };

// Records phase event k (0: round start; 1..4: end of bound, alpha, clip,
// split) when the caller asked for them.
int mark(void* const* phase_ev, int k, hipStream_t st) {
  if (!phase_ev) return VC_OK;
  return hipEventRecord((hipEvent_t)phase_ev[k], st) == hipSuccess ? VC_OK : VC_ERR_LAUNCH;
}

// Which of a lookahead's leaves and children alpha closed: over the
// CROWN-unclosed leaves unc (n_u), fu[i] = closed[unc[i]]; over their
// feasible ones (positions fpos in unc, n_f), ff[i] = closed[unc[fpos[i]]];
// over the children of the split ones (positions spos, n_s; the high halves
// first, then the low ones, each in split order), drop[i] =
// closed[unc[spos[i mod n_s]]].
__global__ void k_look_flags(const uint8_t* __restrict__ closed, const int64_t* __restrict__ unc,
                             int64_t n_u, const int64_t* __restrict__ fpos, int64_t n_f,
                             const int64_t* __restrict__ spos, int64_t n_s,
                             uint8_t* __restrict__ fu, uint8_t* __restrict__ ff,
                             uint8_t* __restrict__ drop) {
  const int64_t tot = n_u + n_f + 2 * n_s;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < tot;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (i < n_u) {
      fu[i] = closed[unc[i]] ? 1 : 0;
    } else if (i < n_u + n_f) {
      const int64_t j = i - n_u;
      ff[j] = closed[unc[fpos[j]]] ? 1 : 0;
    } else {
      const int64_t j = i - n_u - n_f;
      drop[j] = closed[unc[spos[j < n_s ? j : j - n_s]]] ? 1 : 0;
    }
  }
}

// The round's unclosed list and feasible flags, and the clipped-box rows of
// its feasible leaves, from a lookahead's: unclosed[i] = unc[ku[i]],
// feasible[i] = feas[ku[i]] (i < n_unc); fidx[i] = fpos[kf[i]] (i < n_f).
__global__ void k_look_take(const int64_t* __restrict__ unc, const uint8_t* __restrict__ feas,
                            const int64_t* __restrict__ ku, int64_t n_unc,
                            const int64_t* __restrict__ fpos, const int64_t* __restrict__ kf,
                            int64_t n_f, int64_t* __restrict__ unclosed,
                            uint8_t* __restrict__ feasible, int64_t* __restrict__ fidx) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_unc + n_f;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (i < n_unc) {
      unclosed[i] = unc[ku[i]];
      feasible[i] = feas[ku[i]];
    } else {
      fidx[i - n_unc] = fpos[kf[i - n_unc]];
    }
  }
}

// The bound phase: zonotope, union of the unstable neurons, CROWN + spec.
// The zonotope passes leave the union of the unstable sets (same bounds,
// no second pass over them), and for the rows form its per-domain seed
// masks in its workspace; the one-wavefront pass lists its overflowing
// domains itself.  The round reads only the spec bound of the CROWN pass
// (alpha restarts from the zonotope bounds): the rows form writes no CROWN
// bounds.
int bound_phase(const int32_t* dims, int n, const float* frag, const float* bias_cat, int64_t B,
                const float* xl, const float* xh, BoundBufs& b, int Q, const float* spec_rows,
                const float* spec_acc, float* lb, float* A, float* acc, uint64_t* seed_rows,
                void* crown_ev0, void* crown_ev1, hipStream_t st) {
  if (b.rws) {
    VC_TRY(vcm::zono_bounds_masked(dims, n, frag, bias_cat, B, xl, xh, b.sb_lo, b.sb_hi, b.ovf,
                                   b.queue + 1, b.rws, b.idx, b.cnt, b.cnt + 3, st));
    VC_TRY(vcm::zono_wide_masked(dims, n, frag, bias_cat, B, xl, xh, b.sb_lo, b.sb_hi, b.ovf,
                                 b.idx, b.cnt, b.rws, st));
  } else {
    VC_TRY(vcm::zono_bounds_listed(dims, n, frag, bias_cat, B, xl, xh, b.sb_lo, b.sb_hi, b.ovf,
                                   b.queue + 1, b.idx, b.cnt, b.umask, b.cnt + 3, st));
    VC_TRY(vcm::zono_wide_union(dims, n, frag, bias_cat, B, xl, xh, b.sb_lo, b.sb_hi, b.ovf,
                                b.idx, b.cnt, b.umask, st));
    VC_TRY(vcm::union_lists(dims, n, b.umask, b.uidx, b.umeta, st));
  }
  if (crown_ev0 && hipEventRecord((hipEvent_t)crown_ev0, st) != hipSuccess) return VC_ERR_LAUNCH;
  if (b.rws)
    VC_TRY(vcm::crown_rows_premasked(dims, n, frag, bias_cat, B, xl, xh, b.sb_lo, b.sb_hi, Q,
                                     spec_rows, spec_acc, lb, A, acc, seed_rows, b.rws,
                                     b.rws_bytes, st));
  else
    VC_TRY(vc_mlp_tiled_crown(dims, n, frag, bias_cat, B, xl, xh, b.sb_lo, b.sb_hi, b.t_lo,
                              b.t_hi, b.uidx, b.umeta, 1, 1, Q, spec_rows, spec_acc, lb, A, acc,
                              seed_rows, b.queue, (vc_stream_t)st));
  if (crown_ev1 && hipEventRecord((hipEvent_t)crown_ev1, st) != hipSuccess) return VC_ERR_LAUNCH;
  return VC_OK;
}

// Where the clip and split phases write: the unclosed list, the feasible
// flags, the feasible rows and the children (low_xl / low_xh null: right
// after the nu high children, in high_xl / high_xh).
struct TailOut {
  int64_t* unclosed;
  uint8_t* feasible;
  float *xl_split, *xh_split;
  int64_t* ax;
  float *low_xl, *low_xh, *high_xl, *high_xh;
  float* low_at(float* low, float* high, int64_t nu, int n_in) const {
    return low ? low : high + nu * (int64_t)n_in;
  }
};

// The clip and split phases on the leaves `closed` leaves open: the
// unclosed compaction (its count read with alpha's evaluated iterations
// when a_ctl is given), the gather, clip, widest axis, the feasible and
// split compaction, the feasible rows' gather and the bisection.
int tail_phases(const int32_t* dims, int Q, const int32_t* d_ptr, const int32_t* q_idx,
                int n_disj, int64_t B, const float* xl, const float* xh, const float* A,
                const float* acc, const uint8_t* closed, const TailBufs& t, const TailOut& o,
                const float* a_ctl, double* clip_widths, void* const* phase_ev,
                int64_t* pinned, hipStream_t st, int& phase, int64_t& n_unc, int64_t& n_eval,
                int64_t& nf, int64_t& nu) {
  const int n_in = dims[0];
  const vc_stream_t stream = (vc_stream_t)st;
  phase = PH_CLIP;
  VC_TRY(vc_compact(closed, B, 1, o.unclosed, t.cnt, t.cws, t.cws_bytes, stream));
  if (a_ctl) {
    int64_t two[2];
    VC_TRY(read_counts(t.cnt, 1, two, pinned, st, a_ctl));
    n_unc = two[0];
    n_eval = two[1];
  } else {
    VC_TRY(read_counts(t.cnt, 1, &n_unc, pinned, st));
  }
  nf = nu = 0;
  if (n_unc > 0) {
    float* gout[4] = {t.u_xl, t.u_xh, t.u_A, t.u_acc};
    const float* gin[4] = {xl, xh, A, acc};
    const int32_t gcols[4] = {n_in, n_in, Q * n_in, Q};
    VC_TRY(gather(gin, gout, gcols, 4, o.unclosed, n_unc, stream));
    VC_TRY(vc_clip_box(t.u_xl, t.u_xh, t.u_A, t.u_acc, n_unc, Q, n_in, d_ptr, q_idx, n_disj,
                       t.c_xl, t.c_xh, o.feasible, stream));
    if (clip_widths) {
      const int64_t nv = n_unc * n_in;
      const int blocks = (int)std::min<int64_t>((nv + 255) / 256, 1024);
      hipLaunchKernelGGL(k_clip_widths, dim3(blocks), dim3(256), 0, st, t.u_xl, t.u_xh, t.c_xl,
                         t.c_xh, nv, clip_widths);
      if (hipGetLastError() != hipSuccess) return VC_ERR_LAUNCH;
    }
    VC_TRY(vc_widest_axis(t.c_xl, t.c_xh, n_unc, n_in, t.ax_u, t.usable, stream));
    // the feasible leaves, and the feasible ones with a usable split axis
    VC_TRY(vcm::compact_feasible_split(o.feasible, t.usable, n_unc, t.idx, t.cnt, t.idx2,
                                       t.cnt + 1, t.split, t.cws, t.cws_bytes, st));
    int64_t two[2];
    VC_TRY(read_counts(t.cnt, 2, two, pinned, st));
    nf = two[0];
    nu = two[1];
    if (nf > 0) {
      // the int64 axes travel as float pairs through the row gather (bit copy)
      const float* fin[3] = {t.c_xl, t.c_xh, reinterpret_cast<const float*>(t.ax_u)};
      float* fout[3] = {o.xl_split, o.xh_split, reinterpret_cast<float*>(o.ax)};
      const int32_t fcols[3] = {n_in, n_in, 2};
      VC_TRY(gather(fin, fout, fcols, 3, t.idx, nf, stream));
    }
  }
  VC_TRY(mark(phase_ev, 3, st));
  phase = PH_SPLIT;
  if (nu > 0)
    VC_TRY(vc_bisect(t.c_xl, t.c_xh, t.ax_u, t.idx2, nu, n_in,
                     o.low_at(o.low_xl, o.high_xl, nu, n_in),
                     o.low_at(o.low_xh, o.high_xh, nu, n_in), o.high_xl, o.high_xh, stream));
  VC_TRY(mark(phase_ev, 4, st));
  return VC_OK;
}

// Fork / join events of the lookahead, destroyed with the call (a pending
// event's resources go when it completes).  Once forked, every way out of
// the call joins: `stream` waits for the aux stream's work, so that nothing
// the caller frees or reuses after the call is still in use there.
struct EventPair {
  hipEvent_t e[2] = {nullptr, nullptr};
  hipStream_t st = nullptr, ast = nullptr;  // set while forked
  int join() {
    if (!ast) return VC_OK;
    const bool ok = hipEventRecord(e[1], ast) == hipSuccess &&
                    hipStreamWaitEvent(st, e[1], 0) == hipSuccess;
    ast = nullptr;
    return ok ? VC_OK : VC_ERR_LAUNCH;
  }
  ~EventPair() {
    (void)join();
    for (hipEvent_t x : e)
      if (x) (void)hipEventDestroy(x);
  }
  int make() {
    for (hipEvent_t& x : e)
      if (hipEventCreateWithFlags(&x, hipEventDisableTiming) != hipSuccess) return VC_ERR_LAUNCH;
    return VC_OK;
  }
};

int bab_round(const int32_t* dims, int n_relu, const float* frag, const float* bias_cat, int Q,
              const float* spec_rows, const float* spec_acc, const int32_t* d_ptr,
              const int32_t* q_idx, int n_disj, int64_t B, const float* xl, const float* xh,
              int alpha_iters, double alpha_lr, double alpha_lr_decay, double alpha_early_stop,
              float* lb, float* A, float* acc, uint8_t* closed, int64_t* unclosed,
              uint8_t* feasible, float* xl_split, float* xh_split, int64_t* ax, float* low_xl,
              float* low_xh, float* high_xl, float* high_xh, uint64_t* seed_rows,
              void* crown_ev0, void* crown_ev1, void* const* phase_ev, double* clip_widths,
              void* work, int64_t work_bytes, const void* pre, void* la_work,
              int64_t la_bytes, int64_t la_cap, vc_stream_t aux_stream, int32_t* stop_host,
              int64_t* pinned, int64_t* counts, int& phase, vc_stream_t stream) {
  phase = PH_BOUND;
  if (!dims || !frag || !bias_cat || !spec_rows || !spec_acc || !d_ptr || !q_idx || !xl ||
      !xh || !lb || !A || !acc || !closed || !unclosed || !feasible || !xl_split ||
      !xh_split || !ax || !high_xl || !high_xh || !work || !counts)
    return VC_ERR_ARG;
  // the low children in their own arrays, or both after the high ones
  if ((low_xl == nullptr) != (low_xh == nullptr)) return VC_ERR_ARG;
  if (n_relu < 1 || n_relu > MAXL || B < 0 || Q < 1 || n_disj < 0 || la_cap < 0)
    return VC_ERR_ARG;
  // la_work with aux_stream: the overlapped lookahead; without: the next
  // round's bound phase after the split, on `stream` (the low children
  // must follow the high ones, so that they are the next batch as it is)
  const bool tail = la_work && !aux_stream;
  if (tail && low_xl) return VC_ERR_ARG;
  const int64_t need = vc_mlp_bab_round_workspace(dims, n_relu, B, Q);
  if (need < 0) return (int)-need;
  if (work_bytes < need) return VC_ERR_OOM;
  if (la_work) {
    const int64_t la_need = vc_mlp_bab_round_lookahead_workspace(dims, n_relu, B, Q, la_cap);
    if (la_need < 0) return (int)-la_need;
    if (la_bytes < la_need) return VC_ERR_OOM;
  }
  const int n = n_relu, n_in = dims[0];
  int sumd = 0;
  for (int l = 1; l <= n; ++l) sumd += dims[l];
  // the wide zonotope pass must hold every generator the net can have
  int max_cols = 1;
  for (int l = 0; l < n; ++l) max_cols += dims[l];
  if (max_cols > VC_ZONO_WIDE_COLS) return VC_ERR_UNSUPPORTED;
  for (int k = 0; k < 7; ++k) counts[k] = 0;
  counts[6] = -1;
  hipStream_t st = (hipStream_t)stream;
  VC_TRY(mark(phase_ev, 0, st));
  if (B == 0) {
    for (int k = 1; k <= 4; ++k) VC_TRY(mark(phase_ev, k, st));
    return VC_OK;
  }
  Carve c{reinterpret_cast<char*>(work), 0};
  RoundBufs r;
  carve(c, r, dims, n, B, Q);

  // ---- bound phase, or the one a previous round's lookahead handed over
  // (its spec bound, A and acc read in place when the caller points lb, A
  // and acc there: vc_mlp_bab_round_handoff_offsets)
  if (pre) {
    Carve hc{reinterpret_cast<char*>(const_cast<void*>(pre)), 0};
    Handoff h;
    carve_handoff(hc, h, dims, n, B, Q);
    if ((lb != h.lb &&
         hipMemcpyAsync(lb, h.lb, sizeof(float) * B * Q, hipMemcpyDeviceToDevice, st) !=
             hipSuccess) ||
        (A != h.A && hipMemcpyAsync(A, h.A, sizeof(float) * B * Q * n_in,
                                    hipMemcpyDeviceToDevice, st) != hipSuccess) ||
        (acc != h.acc &&
         hipMemcpyAsync(acc, h.acc, sizeof(float) * B * Q, hipMemcpyDeviceToDevice, st) !=
             hipSuccess))
      return VC_ERR_LAUNCH;
    for (int l = 0; l < n; ++l) {
      r.b.sb_lo[l] = h.sb_lo[l];
      r.b.sb_hi[l] = h.sb_hi[l];
    }
    r.b.cnt = r.t.cnt = h.cnt;
  } else {
    VC_TRY(bound_phase(dims, n, frag, bias_cat, B, xl, xh, r.b, Q, spec_rows, spec_acc, lb, A,
                       acc, seed_rows, crown_ev0, crown_ev1, st));
  }
  // with alpha, the closure also lists the open leaves (their order is
  // immaterial: each leaf's alpha is its own, and their bounds go back by
  // index), counted in cnt[3], which the zonotope pass's init (or the
  // handoff's clear) zeroed
  if (alpha_iters > 0)
    VC_TRY(vcm::closure_open(lb, B, Q, d_ptr, q_idx, n_disj, closed, r.b.idx, r.b.cnt + 3, st));
  else
    VC_TRY(vc_closure(lb, B, Q, d_ptr, q_idx, n_disj, closed, stream));
  VC_TRY(mark(phase_ev, 1, st));

  // ---- alpha-CROWN on the open leaves, from their zonotope bounds
  phase = PH_ALPHA;
  int64_t n_open = 0, n_eval = 0;
  if (alpha_iters > 0) VC_TRY(read_counts(r.b.cnt + 3, 1, &n_open, pinned, st));
  // With a lookahead (and no phase events or clip widths asked for), this
  // stream clips and splits the leaves the CROWN bound leaves open while
  // alpha and the raise of its rows run on the aux stream, every chunk
  // enqueued at once (its kernels skip the iterations after a stop) and
  // on at most 3/4 of the compute units; then this stream bounds all the
  // children.  After alpha, the round's own outputs are the lookahead's
  // restricted to the leaves alpha leaves open (each leaf's clip and split
  // are its own, and every compaction keeps the order), and the next
  // round's bound phase is the children's restricted to theirs.
  const bool look = la_work && !tail && n_open > 0 && !phase_ev && !clip_widths;
  hipStream_t ast = look ? (hipStream_t)aux_stream : st;
  EventPair ev;
  LookBufs L;
  if (look) {
    Carve lc{reinterpret_cast<char*>(la_work), 0};
    carve_look(lc, L, dims, n, B, Q, la_cap);
    // the CROWN closure, before alpha raises rows of `closed`
    if (hipMemcpyAsync(L.closed_c, closed, B, hipMemcpyDeviceToDevice, st) != hipSuccess)
      return VC_ERR_LAUNCH;
    VC_TRY(ev.make());
    if (hipEventRecord(ev.e[0], st) != hipSuccess ||
        hipStreamWaitEvent(ast, ev.e[0], 0) != hipSuccess)
      return VC_ERR_LAUNCH;
    ev.st = st;
    ev.ast = ast;
    // the CROWN-open leaves in order (n_open of them), their clip, widest
    // axis and the feasible and split compactions; the counts posted
    VC_TRY(vc_compact(L.closed_c, B, 1, L.unc, L.t.cnt, L.t.cws, L.t.cws_bytes, stream));
    float* gout[4] = {L.t.u_xl, L.t.u_xh, L.t.u_A, L.t.u_acc};
    const float* gin[4] = {xl, xh, A, acc};
    const int32_t gcols[4] = {n_in, n_in, Q * n_in, Q};
    VC_TRY(gather(gin, gout, gcols, 4, L.unc, n_open, stream));
    VC_TRY(vc_clip_box(L.t.u_xl, L.t.u_xh, L.t.u_A, L.t.u_acc, n_open, Q, n_in, d_ptr, q_idx,
                       n_disj, L.t.c_xl, L.t.c_xh, L.feas, stream));
    VC_TRY(vc_widest_axis(L.t.c_xl, L.t.c_xh, n_open, n_in, L.t.ax_u, L.t.usable, stream));
    VC_TRY(vcm::compact_feasible_split(L.feas, L.t.usable, n_open, L.t.idx, L.t.cnt, L.t.idx2,
                                       L.t.cnt + 1, L.t.split, L.t.cws, L.t.cws_bytes, st));
    VC_TRY(post_counts(L.t.cnt, 2, pinned, st));
  }
  if (n_open > 0) {
    const float* gin[2 * MAXL + 2];
    float* gout[2 * MAXL + 2];
    int32_t gcols[2 * MAXL + 2];
    for (int l = 0; l < n; ++l) {
      gin[2 * l] = r.b.sb_lo[l];
      gin[2 * l + 1] = r.b.sb_hi[l];
      gout[2 * l] = r.a_lo[l];
      gout[2 * l + 1] = r.a_hi[l];
      gcols[2 * l] = gcols[2 * l + 1] = dims[l + 1];
    }
    gin[2 * n] = xl;
    gin[2 * n + 1] = xh;
    gout[2 * n] = r.a_xl;
    gout[2 * n + 1] = r.a_xh;
    gcols[2 * n] = gcols[2 * n + 1] = n_in;
    VC_TRY(gather(gin, gout, gcols, 2 * n + 2, r.b.idx, n_open, (vc_stream_t)ast));
    float *alpha[MAXL], *m1[MAXL], *m2[MAXL];
    int64_t off = 0;
    for (int l = 0; l < n; ++l) {
      const int64_t sz = n_open * dims[l + 1];
      alpha[l] = r.a_state + off;
      m1[l] = r.a_state + (int64_t)sumd * n_open + off;
      m2[l] = r.a_state + 2 * (int64_t)sumd * n_open + off;
      off += sz;
    }
    int32_t* sh = look ? nullptr : stop_host;
    if (sh) {
      reinterpret_cast<volatile int32_t*>(sh)[0] = 0;
      reinterpret_cast<volatile int32_t*>(sh)[1] = 0;
    }
    VC_TRY(vcm::alpha_run(dims, n, frag, bias_cat, n_open, r.a_xl, r.a_xh, r.a_lo, r.a_hi, alpha,
                          m1, m2, Q, spec_rows, spec_acc, r.a_lb, r.a_best, 0.9, 0.999, 1e-8,
                          alpha_lr, alpha_lr_decay, alpha_iters, alpha_early_stop, r.a_ctl, sh,
                          look ? std::max(1, 3 * vcm::cu_count() / 4) : 0, (vc_stream_t)ast));
    // the open leaves are distinct rows (a compaction's output)
    VC_TRY(vcm::scatter_max_close(lb, r.b.idx, r.a_best, n_open, Q, d_ptr, q_idx, n_disj, closed,
                                  ast));
  }

  if (look) {
    phase = PH_CLIP;
    int64_t two[2];
    VC_TRY(wait_counts(L.t.cnt, 2, two, pinned, st));
    const int64_t nf_l = two[0], nu_l = two[1];
    const int64_t bn = 2 * nu_l;
    bool fits = bn <= la_cap;
    BoundBufs bb;
    if (fits) {
      Carve bc{reinterpret_cast<char*>(la_work), L.bound_off};
      carve_bound(bc, bb, dims, n, bn);
      fits = (int64_t)bc.used <= la_bytes;
    }
    if (fits && nu_l > 0) {
      // the children, the high halves first, and their bound phase
      VC_TRY(vc_bisect(L.t.c_xl, L.t.c_xh, L.t.ax_u, L.t.idx2, nu_l, n_in, L.cxl + nu_l * n_in,
                       L.cxh + nu_l * n_in, L.cxl, L.cxh, stream));
      VC_TRY(bound_phase(dims, n, frag, bias_cat, bn, L.cxl, L.cxh, bb, Q, spec_rows, spec_acc,
                         L.b_lb, L.b_A, L.b_acc, nullptr, nullptr, nullptr, st));
    }
    // join: what follows reads alpha's closure
    VC_TRY(ev.join());
    if (fits) {
      const int64_t tot = n_open + nf_l + 2 * nu_l;
      hipLaunchKernelGGL(k_look_flags, dim3((unsigned)std::min<int64_t>((tot + 255) / 256, 1024)),
                         dim3(256), 0, st, closed, L.unc, n_open, L.t.idx, nf_l, L.t.idx2, nu_l,
                         L.fu, L.ff, L.drop);
      if (hipGetLastError() != hipSuccess) return VC_ERR_LAUNCH;
      if (hipMemsetAsync(r.t.cnt, 0, sizeof(int64_t) * 3, st) != hipSuccess)
        return VC_ERR_LAUNCH;
      VC_TRY(vc_compact(L.fu, n_open, 1, L.ku, r.t.cnt, L.t.cws, L.t.cws_bytes, stream));
      if (nf_l > 0)
        VC_TRY(vc_compact(L.ff, nf_l, 1, L.kf, r.t.cnt + 1, L.t.cws, L.t.cws_bytes, stream));
      if (nu_l > 0)
        VC_TRY(vc_compact(L.drop, bn, 1, L.kidx, r.t.cnt + 2, L.kws, L.kws_bytes, stream));
      int64_t four[4];
      VC_TRY(read_counts(r.t.cnt, 3, four, pinned, st, r.a_ctl));
      const int64_t n_unc = four[0], nf = four[1], n_keep = four[2];
      n_eval = four[3];
      // the kept children are twice the split leaves alpha leaves open
      if (n_keep % 2 != 0 || n_keep > bn || nf > nf_l || n_unc > n_open) return VC_ERR_LAUNCH;
      const int64_t nu = n_keep / 2;
      if (n_unc + nf > 0) {
        hipLaunchKernelGGL(k_look_take,
                           dim3((unsigned)std::min<int64_t>((n_unc + nf + 255) / 256, 1024)),
                           dim3(256), 0, st, L.unc, L.feas, L.ku, n_unc, L.t.idx, L.kf, nf,
                           unclosed, feasible, L.fidx);
        if (hipGetLastError() != hipSuccess) return VC_ERR_LAUNCH;
      }
      if (nf > 0) {
        // the int64 axes travel as float pairs through the row gather (bit copy)
        const float* fin[3] = {L.t.c_xl, L.t.c_xh, reinterpret_cast<const float*>(L.t.ax_u)};
        float* fout[3] = {xl_split, xh_split, reinterpret_cast<float*>(ax)};
        const int32_t fcols[3] = {n_in, n_in, 2};
        VC_TRY(gather(fin, fout, fcols, 3, L.fidx, nf, stream));
      }
      if (nu > 0) {
        // high children are the kept ones of the first half, low ones of the
        // second (both in one gather when the low ones follow the high ones)
        const float* cin[2] = {L.cxl, L.cxh};
        float* hout[2] = {high_xl, high_xh};
        const int32_t ccols[2] = {n_in, n_in};
        if (low_xl) {
          float* lout[2] = {low_xl, low_xh};
          VC_TRY(gather(cin, hout, ccols, 2, L.kidx, nu, stream));
          VC_TRY(gather(cin, lout, ccols, 2, L.kidx + nu, nu, stream));
        } else {
          VC_TRY(gather(cin, hout, ccols, 2, L.kidx, n_keep, stream));
        }
        // the next round's bound phase
        Carve hc{reinterpret_cast<char*>(la_work), 0};
        Handoff h;
        carve_handoff(hc, h, dims, n, n_keep, Q);
        const float* hin[3 + 2 * MAXL] = {L.b_lb, L.b_A, L.b_acc};
        float* hto[3 + 2 * MAXL] = {h.lb, h.A, h.acc};
        int32_t hcols[3 + 2 * MAXL] = {Q, Q * n_in, Q};
        for (int l = 0; l < n; ++l) {
          hin[3 + 2 * l] = bb.sb_lo[l];
          hin[4 + 2 * l] = bb.sb_hi[l];
          hto[3 + 2 * l] = h.sb_lo[l];
          hto[4 + 2 * l] = h.sb_hi[l];
          hcols[3 + 2 * l] = hcols[4 + 2 * l] = dims[l + 1];
        }
        VC_TRY(gather(hin, hto, hcols, 3 + 2 * n, L.kidx, n_keep, stream));
        if (hipMemsetAsync(h.cnt, 0, sizeof(int64_t) * 4, st) != hipSuccess)
          return VC_ERR_LAUNCH;
      }
      counts[0] = n_open;
      counts[1] = n_eval;
      counts[2] = n_unc;
      counts[3] = nf;
      counts[4] = nu;
      counts[5] = nf - nu;
      counts[6] = n_keep;
      return VC_OK;
    }
    // more children than the lookahead holds: the round's own clip and
    // split, in order
  }
  VC_TRY(mark(phase_ev, 2, st));

  // ---- clip, widest axis and bisection of the unclosed leaves
  TailOut o{unclosed, feasible, xl_split, xh_split, ax, low_xl, low_xh, high_xl, high_xh};
  int64_t n_unc = 0, nf = 0, nu = 0;
  VC_TRY(tail_phases(dims, Q, d_ptr, q_idx, n_disj, B, xl, xh, A, acc, closed, r.t, o,
                     n_open > 0 ? r.a_ctl : nullptr, clip_widths, phase_ev, pinned, st, phase,
                     n_unc, n_eval, nf, nu));
  counts[0] = n_open;
  counts[1] = n_eval;
  counts[2] = n_unc;
  counts[3] = nf;
  counts[4] = nu;
  counts[5] = nf - nu;
  // ---- the next round's bound phase on the children (high then low, one
  // block), its outputs where the next call's `pre` takes them: the GPU
  // runs it while the host returns from this call and makes the next one
  if (tail && nu > 0 && 2 * nu <= la_cap && !phase_ev && !clip_widths) {
    const int64_t bn = 2 * nu;
    Carve hc{reinterpret_cast<char*>(la_work), 0};
    Handoff h;
    carve_handoff(hc, h, dims, n, bn, Q);
    Carve cc{nullptr, 0};
    Handoff hcap;
    carve_handoff(cc, hcap, dims, n, la_cap, Q);
    Carve bc{reinterpret_cast<char*>(la_work), cc.used};
    BoundBufs bb;
    carve_bound(bc, bb, dims, n, bn);
    if ((int64_t)bc.used > la_bytes) return VC_ERR_OOM;
    for (int l = 0; l < n; ++l) {
      bb.sb_lo[l] = h.sb_lo[l];
      bb.sb_hi[l] = h.sb_hi[l];
    }
    bb.cnt = h.cnt;  // the zonotope pass's init clears cnt[3] for the next round
    VC_TRY(bound_phase(dims, n, frag, bias_cat, bn, high_xl, high_xh, bb, Q, spec_rows,
                       spec_acc, h.lb, h.A, h.acc, nullptr, nullptr, nullptr, st));
    counts[6] = bn;
  }
  return VC_OK;
}

}  // namespace

extern "C" int vc_mlp_bab_round(const int32_t* dims, int n_relu, const float* frag,
                                const float* bias_cat, int Q, const float* spec_rows,
                                const float* spec_acc, const int32_t* d_ptr,
                                const int32_t* q_idx, int n_disj, int64_t B, const float* xl,
                                const float* xh, int alpha_iters, double alpha_lr,
                                double alpha_lr_decay, double alpha_early_stop, float* lb,
                                float* A, float* acc, uint8_t* closed, int64_t* unclosed,
                                uint8_t* feasible, float* xl_split, float* xh_split, int64_t* ax,
                                float* low_xl, float* low_xh, float* high_xl, float* high_xh,
                                uint64_t* seed_rows, void* crown_ev0, void* crown_ev1,
                                void* const* phase_ev, double* clip_widths, void* work,
                                int64_t work_bytes, const void* pre, void* la_work,
                                int64_t la_bytes, int64_t la_cap, vc_stream_t aux_stream,
                                int32_t* stop_host, int64_t* pinned, int64_t* counts,
                                int32_t* fail_phase, vc_stream_t stream) {
  int phase = PH_BOUND;
  const int rc = bab_round(dims, n_relu, frag, bias_cat, Q, spec_rows, spec_acc, d_ptr, q_idx,
                           n_disj, B, xl, xh, alpha_iters, alpha_lr, alpha_lr_decay,
                           alpha_early_stop, lb, A, acc, closed, unclosed, feasible, xl_split,
                           xh_split, ax, low_xl, low_xh, high_xl, high_xh, seed_rows,
                           crown_ev0, crown_ev1, phase_ev, clip_widths, work, work_bytes, pre,
                           la_work, la_bytes, la_cap, aux_stream, stop_host, pinned, counts,
                           phase, stream);
  if (fail_phase) *fail_phase = rc == VC_OK ? -1 : phase;
  return rc;
}
