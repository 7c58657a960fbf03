/*
 * vibecheck_amd -- C ABI of the MI355X (gfx950) batched linear-bound-
 * propagation library.
 *
 * Conventions
 *   - All tensors are fp32 (flags uint8, indices int32/int64), device
 *     pointers, row-major, contiguous.  "B" is the number of domains
 *     (boxes); "R" is the number of backward rows per domain (spec queries
 *     Q, or 2k seeded rows); a backward row m belongs to domain m / R.
 *   - Every call is asynchronous on the given HIP stream (hipStream_t passed
 *     as void*) and returns a status code (VC_OK on success).  Scratch comes
 *     from caller workspaces; the only device memory the library allocates
 *     is rocBLAS's own, when the first plain fp32 product (vc_backward_fc's
 *     second phase, vc_zono_fc's generator product) on a device and host
 *     thread creates its handle, kept for the life of the process.
 *   - Each entry point names the reference function it replaces
 *     (src/vibecheck/<file>:<line>).
 */
#ifndef VIBECHECK_AMD_H
#define VIBECHECK_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VC_OK 0
#define VC_ERR_ARG 1         /* bad shape / null pointer / size limit */
#define VC_ERR_OOM 2         /* workspace too small */
#define VC_ERR_UNSUPPORTED 3 /* op or layout not supported */
#define VC_ERR_LAUNCH 4      /* HIP launch / runtime error */

/* Generator columns (centre included) that vc_mlp_tiled_zono_wide holds
 * per domain; a net whose 1 + d[0] + d[1] + ... + d[n-1] stays within it
 * never leaves a domain to a layer-wise fallback. */
#define VC_ZONO_WIDE_COLS 512

/* Iterations vc_mlp_tiled_alpha_run may run in one launch. */
#define VC_ALPHA_CHUNK 4

typedef void *vc_stream_t;

/* Library version, for the host to check the ABI it loaded. */
int vc_abi_version(void);

/* ---- ReLU relaxation ------------------------------------------------- */

/* CROWN adaptive slopes, elementwise over n values.
 * Replaces _make_slopes (verify_zono_bnb.py:503-522). */
int vc_make_slopes(const float *lo, const float *hi, int64_t n, float *lo_s,
                   float *up_s, float *up_t, uint8_t *active, uint8_t *dead,
                   uint8_t *unstable, vc_stream_t stream);

/* ---- IBP forward ----------------------------------------------------- */

/* fc layer of the interval forward: mid/rad through W and |W|.
 * l, h (B, n_in); W (n_out, n_in); bias (n_out) or NULL; lo, hi (B, n_out).
 * Replaces the fc branch of _ibp_forward_graph_batched
 * (verify_zono_bnb.py:1108-1113). */
int vc_ibp_fc(const float *l, const float *h, int64_t B, int n_in,
              const float *W, const float *bias, int n_out, float *lo,
              float *hi, vc_stream_t stream);

/* conv layer of the interval forward (NCHW, square stride/pad pairs).
 * kernel (C_out, C_in, kh, kw); bias (C_out) or NULL.
 * Replaces the conv branch of _ibp_forward_graph_batched
 * (verify_zono_bnb.py:1098-1107). */
int vc_ibp_conv(const float *l, const float *h, int64_t B, int C_in, int H,
                int W, const float *kernel, const float *bias, int C_out,
                int kh, int kw, int sh, int sw, int ph, int pw, int H_out,
                int W_out, float *lo, float *hi, vc_stream_t stream);

/* relu of the interval forward: intersect root bounds (n, nullable) and
 * split clamps (B, n, nullable), repair hi = max(hi, lo), write the
 * pre-activation bounds sb_lo/sb_hi (B, n) and, when post_lo/post_hi are
 * non-NULL, the clamp(min=0) outputs.  l/h NULL (both) means an unbounded
 * input interval; the root bounds are then required and the result is the
 * root broadcast to B domains intersected with the clamps.
 * Replaces the relu branch of _ibp_forward_graph_batched
 * (verify_zono_bnb.py:1114-1129) and, with l/h NULL, the clamped layers of
 * the no-reforward domain bounds (verify_milp.py:2706-2717). */
int vc_ibp_relu(const float *l, const float *h, int64_t B, int n,
                const float *root_lo, const float *root_hi, const float *cl,
                const float *ch, float *sb_lo, float *sb_hi, float *post_lo,
                float *post_hi, vc_stream_t stream);

/* ---- Zonotope forward ------------------------------------------------ */

/* Input zonotope: c = (xl+xh)/2 (B, n); G (B, n, K) with one column per
 * input dim listed in var_idx (K entries), G[b, var_idx[k], k] = radius.
 * Replaces verify_zono_bnb.py:3093-3110. */
int vc_zono_input(const float *xl, const float *xh, int64_t B, int n,
                  const int32_t *var_idx, int K, float *c, float *G,
                  vc_stream_t stream);

/* fc layer: c_out = c W^T + bias (B, n_out); G_out[b] = W G[b]
 * (B, n_out, K), a plain batched product (rocBLAS's strided-batched
 * sgemm).  Replaces verify_zono_bnb.py:3169-3173. */
int vc_zono_fc(const float *c, const float *G, int64_t B, int n_in, int K,
               const float *W, const float *bias, int n_out, float *c_out,
               float *G_out, vc_stream_t stream);

/* conv layer: c_out = conv2d(c, kernel) + bias; each generator column of
 * G (B, n_in, Kg) convolved without bias into G_out (B, n_out, Kg).
 * Replaces verify_zono_bnb.py:3400-3425. */
int vc_zono_conv(const float *c, const float *G, int64_t B, int Kg, int C_in,
                 int H, int W, const float *kernel, const float *bias,
                 int C_out, int kh, int kw, int sh, int sw, int ph, int pw,
                 int H_out, int W_out, float *c_out, float *G_out,
                 vc_stream_t stream);

/* relu stage 1: lo/hi = c -/+ sum_k |G| (B, n), and per-domain unstable
 * counts cnt (B) plus unstable ranks rank (B, n) (exclusive count of
 * unstable neurons before j in domain b).
 * Replaces verify_zono_bnb.py:3175-3199. */
int vc_zono_relu_bounds(const float *c, const float *G, int64_t B, int n,
                        int K, float *lo, float *hi, int32_t *rank,
                        int32_t *cnt, vc_stream_t stream);

/* relu stage 2: c_out = lam c + mu; G_out (B, n, K + K_new) = [lam G | new]
 * with new[b, j, rank[b, j]] = mu for unstable j.
 * Replaces verify_zono_bnb.py:3185-3210. */
int vc_zono_relu_apply(const float *c, const float *G, const float *lo,
                       const float *hi, const int32_t *rank, int64_t B, int n,
                       int K, int K_new, float *c_out, float *G_out,
                       vc_stream_t stream);

/* ---- add / sub / mul ops (constant and residual merge) --------------- */

/* out = x + v (mode 0), x - v (mode 1) or x * v (mode 2), elementwise over
 * x of outer x n x inner floats; element i of the n is (t / inner) % n and
 * its constant v[i] (nv == n) or v[0] (nv == 1).  inner = 1 for (B, n)
 * rows, K for (B, n, K) generators.  Replaces the constant add and sub of
 * the interval forward (verify_zono_bnb.py:1136-1143), the zonotope's add
 * and sub of the centre (3235-3265) and mul of centre and generators
 * (3501-3536), and the backward's mul, ew * scale (4686-4712). */
int vc_affine_ew(const float *x, int64_t outer, int n, int64_t inner,
                 const float *v, int nv, int mode, float *out,
                 vc_stream_t stream);

/* Interval times a constant (B, n): lo = min(s l, s h), hi = max(s l, s h)
 * with torch.minimum / torch.maximum's NaN and tie rules; s scalar
 * (ns == 1) or per element (ns == n).  Replaces the mul branch of
 * _ibp_forward_graph_batched (verify_zono_bnb.py:1144-1148). */
int vc_interval_mul(const float *l, const float *h, int64_t B, int n,
                    const float *s, int ns, float *lo, float *hi,
                    vc_stream_t stream);

/* out = a + b over total floats: a residual merge's interval bounds and
 * zonotope centre (verify_zono_bnb.py:1133-1135, 3213-3234), and the sum
 * of backward rows arriving at a fork point from two consumers
 * (ew_at[inp] + ew, verify_zono_bnb.py:4462-4469). */
int vc_add_ew(const float *a, const float *b, int64_t total, float *out,
              vc_stream_t stream);

/* Generators of a residual merge, rows = B * n: Gout (rows, Ka + Kb -
 * shared) = [Ga[:, :shared] + Gb[:, :shared] | Ga[:, shared:] |
 * Gb[:, shared:]]; `shared` is the generator count at the branches' fork
 * point (_find_shared_gens_count).  Replaces verify_zono_bnb.py:3213-3234. */
int vc_zono_merge(const float *Ga, int Ka, const float *Gb, int Kb, int shared,
                  int64_t rows, float *Gout, vc_stream_t stream);

/* acc[m] += sign * sum_i ew[row, i] v[i] over M rows of n (row = m, or
 * m % R when shared: rows common to every domain), the products in fp32
 * summed in fp64: the constant add's (sign 1) and sub's (sign -1)
 * contribution to the backward's constant term.  Replaces
 * verify_zono_bnb.py:4469-4504 and 4506-4518. */
int vc_rows_bias_dot(const float *ew, int64_t M, int R, int n, int shared,
                     const float *v, int nv, float sign, float *acc,
                     vc_stream_t stream);

/* ---- CROWN backward -------------------------------------------------- */

/* One backward step through [relu ->] fc, fused.
 *   ew_in  (M, n_out), M = B * R rows; row m belongs to domain m / R.
 *   If relu_lo/relu_hi (B, n_out) are non-NULL the rows are first relaxed
 *   with the CROWN slopes of those pre-activation bounds:
 *       e = pos(ew) * ls + neg(ew) * up_s [+ beta],  acc += neg(ew) . up_t
 *   with ls = active + unstable * alpha when alpha is non-NULL (alpha is
 *   (B, n_out), or (M, n_out) when alpha_per_row != 0), else the adaptive
 *   lower slope; beta (B, n_out) is optional.  Then
 *       acc += e . bias (bias nullable),  ew_out (M, n_in) = e W,
 *   with W (n_out, n_in).  When relax_out is non-NULL the relaxed rows e
 *   are also written there (M, n_out); with a relu and n_out >= 64 the step
 *   then runs in two phases (the relaxation streams e into relax_out, and
 *   rocBLAS's fp32 sgemm reads it back), which is faster than relaxing
 *   inside the GEMM's loads, so callers that can spare the buffer should
 *   pass it.  Without a relu, bias, relax_out or shared rows the product
 *   is that sgemm alone.
 *   With ew_bcast != 0, ew_in is (R, n_out) and shared by every domain
 *   (row m reads row m % R).
 * Replaces the fc and relu branches of _spec_backward_graph_batched
 * (verify_zono_bnb.py:4379-4453). */
int vc_backward_fc(const float *ew_in, int64_t M, int R, int n_out,
                   const float *relu_lo, const float *relu_hi,
                   const float *alpha, int alpha_per_row, const float *beta,
                   const float *W, const float *bias, int n_in, float *ew_out,
                   float *acc, float *relax_out, int ew_bcast,
                   vc_stream_t stream);

/* vc_backward_fc with the per-row alpha of a group: alpha_groups (G, R,
 * n_out) holds one alpha per (group, row, neuron) and domain d reads the
 * rows of group group[d] (B int64; n_groups = G).  An index outside
 * [0, G) reads group 0 instead of memory past the buffer; callers that do
 * not build the indices themselves pass them through vc_group_clamp first,
 * which reports such indices.  No beta.  The hybrid replay's frozen layer
 * alphas, shared by every leaf of a group, bound without a per-leaf copy:
 * replaces the alpha_b = a.expand(B, -1, -1) of verify_hybrid_acasxu.py:
 * 286-287 with the backward of verify_zono_bnb.py:4409-4453 that reads it. */
int vc_backward_fc_grouped(const float *ew_in, int64_t M, int R, int n_out,
                           const float *relu_lo, const float *relu_hi,
                           const float *alpha_groups, const int64_t *group,
                           int64_t n_groups, const float *W, const float *bias, int n_in,
                           float *ew_out, float *acc, float *relax_out, int ew_bcast,
                           vc_stream_t stream);

/* Group indices made safe to read by: out[b] = group[b] when it lies in
 * [0, n_groups), else 0, and *bad = 1 if any did not (the caller zeroes
 * *bad beforehand and reads it at its next synchronisation).  The hybrid
 * replay's check of the leaves' group indices (verify_hybrid_acasxu.py:
 * 286-287 indexes the group alphas by them). */
int vc_group_clamp(const int64_t *group, int64_t B, int64_t n_groups, int64_t *out,
                   int32_t *bad, vc_stream_t stream);

/* Slopes of a relu layer for the backward, elementwise over n (= B * n_L)
 * pre-activation bounds: lo_s = active + unstable * alpha when alpha (same
 * layout) is non-NULL, else the adaptive lower slope; up_s, up_t as in
 * _make_slopes (verify_zono_bnb.py:503-522, with the alpha override of
 * verify_zono_bnb.py:4422-4433).  Feeds vc_alpha_grad_step_slopes, which
 * then does no per-element division. */
int vc_relax_slopes(const float *relu_lo, const float *relu_hi,
                    const float *alpha, int64_t n, float *lo_s, float *up_s,
                    float *up_t, vc_stream_t stream);

/* relu backward step alone (for a relu that is not fed by an fc):
 * ew_out (M, n) = relaxed rows, acc += neg(ew) . up_t.  Same arguments as
 * the relu part of vc_backward_fc.  Replaces verify_zono_bnb.py:4409-4453. */
int vc_backward_relu(const float *ew_in, int64_t M, int R, int n,
                     const float *relu_lo, const float *relu_hi,
                     const float *alpha, int alpha_per_row, const float *beta,
                     float *ew_out, float *acc, vc_stream_t stream);

/* conv backward: acc += sum ew * bias[channel]; ew_out = conv_transpose2d
 * of ew (M, C_out*H_out*W_out) to (M, C_in*H*W).
 * Replaces verify_zono_bnb.py:4568-4593. */
int vc_backward_conv(const float *ew_in, int64_t M, const float *kernel,
                     const float *bias, int C_out, int H_out, int W_out,
                     int C_in, int H, int W, int kh, int kw, int sh, int sw,
                     int ph, int pw, float *ew_out, float *acc,
                     vc_stream_t stream);

/* The taps of the transposed convolution packed once per kernel for
 * vc_backward_conv_packed: for each of the sh * sw output-parity classes,
 * C_in rows of C_out * ceil(kh / sh) * ceil(kw / sw) taps (zero past the
 * kernel), rows padded to a multiple of 4 floats; vc_conv_t_pack_floats
 * gives the size.  The reference has no counterpart (it calls
 * conv_transpose2d, verify_zono_bnb.py:4568-4593): the packing is this
 * build's weight cache, like the reference's cached op tensors
 * (verify_zono_bnb.py:4482-4486). */
int64_t vc_conv_t_pack_floats(int C_out, int C_in, int kh, int kw, int sh, int sw);
int vc_conv_t_pack(const float *kernel, int C_out, int C_in, int kh, int kw, int sh,
                   int sw, int ph, int pw, float *out, vc_stream_t stream);

/* vc_backward_conv reading the packed taps (16-byte aligned, from
 * vc_conv_t_pack of the same kernel and geometry) instead of deriving each
 * tap from the kernel in every K-tile: the same values in the same order,
 * so the same results bit for bit.  kernel is still read when C_in <= 4
 * (that form takes no packing).  Replaces verify_zono_bnb.py:4568-4593. */
int vc_backward_conv_packed(const float *ew_in, int64_t M, const float *kernel,
                            const float *packed, const float *bias, int C_out, int H_out,
                            int W_out, int C_in, int H, int W, int kh, int kw, int sh, int sw,
                            int ph, int pw, float *ew_out, float *acc, vc_stream_t stream);

/* The relu backward step fused into the following conv backward, for
 * convolutions onto few values per tap set (C_in <= 4, C_in kh kw <= 32,
 * C_out <= 64: the network's input layer; vc_backward_relu_conv_ok says
 * whether a geometry qualifies, else VC_ERR_UNSUPPORTED and the caller
 * takes vc_backward_relu + vc_backward_conv).  Row m = d * R + s of the
 * M = B * R rows out is relaxed with domain d's slopes (lo_s, up_s, up_t
 * from vc_relax_slopes, (B, C_out * H_out * W_out); beta the same shape or
 * NULL) from input row s (ew_shared: ew_in holds the R rows every domain
 * shares) or m, then transposed-convolved:
 *   e = pos(x) lo_s + neg(x) up_s [+ beta];  acc[m] += neg(x) . up_t;
 *   acc[m] += e . bias[channel];  ew_out[m] = conv_transpose2d(e).
 * The same arithmetic as the two separate calls: ew_out is bit-identical,
 * and acc differs from theirs only by the order of its fp64 sums.
 * Replaces verify_zono_bnb.py:4409-4453 followed by 4568-4593. */
int vc_backward_relu_conv_ok(int C_out, int H_out, int W_out, int C_in, int H, int W,
                             int kh, int kw, int sh, int sw, int ph, int pw);
int vc_backward_relu_conv(const float *ew_in, int64_t M, int64_t R, int ew_shared,
                          const float *lo_s, const float *up_s, const float *up_t,
                          const float *beta, const float *kernel, const float *bias,
                          int C_out, int H_out, int W_out, int C_in, int H, int W,
                          int kh, int kw, int sh, int sw, int ph, int pw,
                          float *ew_out, float *acc, vc_stream_t stream);

/* Concretization over the input boxes:
 *   lb[m] = acc[m] + sum_i pos(A[m,i]) xl[b,i] + neg(A[m,i]) xh[b,i].
 * A (M, n_in), acc/lb (M), xl/xh (B, n_in), M = B * R.  With a_bcast != 0,
 * A is (R, n_in) and shared by every domain.
 * Replaces verify_zono_bnb.py:5117-5134. */
int vc_concretize(const float *A, const float *acc, const float *xl,
                  const float *xh, int64_t M, int R, int n_in, int a_bcast,
                  float *lb, vc_stream_t stream);

/* CROWN intermediate-bound intersection for one seeded chunk:
 *   lo[b, idx[t]] = max(lo, sl[b, t]); hi = max(min(hi, -sl[b, k+t]), lo')
 * sl (B, 2k) from a backward seeded with [+I_k; -I_k]; lo/hi (B, n) in place.
 * Replaces verify_zono_bnb.py:4140-4145. */
int vc_crown_intersect(const float *sl, const int32_t *idx, int k, int64_t B,
                       int n, float *lo, float *hi, vc_stream_t stream);

/* Union over domains of unstable neurons: flag[j] = any_b lo<0<hi.
 * Replaces verify_zono_bnb.py:4123. */
int vc_unstable_union(const float *lo, const float *hi, int64_t B, int n,
                      uint8_t *flag, vc_stream_t stream);

/* ---- alpha-CROWN ----------------------------------------------------- */

/* alpha initialisation alpha = (up_s > 0.5) * unstable over n neurons.
 * Replaces verify_zono_bnb.py:5169-5173. */
int vc_alpha_init(const float *lo, const float *hi, int64_t n, float *alpha,
                  vc_stream_t stream);

/* Gradient sweep step through one relu of the alpha backward, fused with
 * the next fc's transposed product (forward direction):
 *   gP (M, n) = gE * (mpos * ls + mneg * up_s) + mneg * up_t, where P is
 *   the stored pre-relaxation rows ((M, n), or (R, n) shared by all domains
 *   when p_bcast != 0), mpos = P >= 0, mneg = P <= 0 (torch's clamp
 *   subgradient at 0), ls = active + unstable * alpha (alpha (B, n) or NULL
 *   for the adaptive slope);  g_out (M, n_next) = gP W_next^T + bias_next,
 *   W_next (n_next, n), bias_next nullable.
 * With vc_alpha_grad_reduce and vc_alpha_grad_input this is the autograd
 * of _spec_backward_graph_batched w.r.t. alpha (verify_zono_bnb.py:5261). */
int vc_alpha_grad_step(const float *gE, const float *P, int64_t M, int R, int n,
                       const float *relu_lo, const float *relu_hi,
                       const float *alpha, int p_bcast, const float *W_next,
                       const float *bias_next, int n_next, float *g_out,
                       vc_stream_t stream);

/* vc_alpha_grad_step with the relaxation given as slopes (B, n) from
 * vc_relax_slopes (lo_s carries the alpha override).  Bit-identical to
 * vc_alpha_grad_step on the bounds and alpha the slopes came from. */
int vc_alpha_grad_step_slopes(const float *gE, const float *P, int64_t M,
                              int R, int n, const float *lo_s,
                              const float *up_s, const float *up_t,
                              int p_bcast, const float *W_next,
                              const float *bias_next, int n_next,
                              float *g_out, vc_stream_t stream);

/* vc_alpha_grad_step with one alpha per backward row (the per-query alpha
 * of the hybrid freeze / replay verifier, verify_hybrid_acasxu.py:164-318):
 * alpha_rows (M, n), row m's lower slope active + unstable * alpha_rows[m].
 * galpha_rows (M, n), if not NULL, also receives d lb / d alpha_rows (what
 * vc_alpha_grad_rows computes), from the same loads. */
int vc_alpha_grad_step_rows(const float *gE, const float *P, int64_t M, int R,
                            int n, const float *relu_lo, const float *relu_hi,
                            const float *alpha_rows, int p_bcast,
                            const float *W_next, const float *bias_next,
                            int n_next, float *g_out, float *galpha_rows,
                            vc_stream_t stream);

/* d lb / d alpha with one alpha per row: galpha (M, n)[m, j] = gE[m, j] *
 * pos(P[m, j]) where neuron j of row m's domain (m / R) is unstable, else 0
 * (P (M, n), or (R, n) shared when p_bcast).  The per-row form of
 * vc_alpha_grad_reduce (the autograd of the per-query alpha backward). */
int vc_alpha_grad_rows(const float *gE, const float *P, int p_bcast, int64_t M,
                       int R, int n, const float *relu_lo, const float *relu_hi,
                       float *galpha, vc_stream_t stream);

/* d lb / d alpha for one layer: galpha[b, j] = sum over the R rows of b of
 * gE[m, j] * pos(P[m, j]), zero where the neuron is not unstable;
 * gbeta[b, j] (nullable) = sum over rows of gE[m, j] (d lb / d beta).
 * P as in vc_alpha_grad_step. */
int vc_alpha_grad_reduce(const float *gE, const float *P, int p_bcast,
                         int64_t B, int R, int n, const float *relu_lo,
                         const float *relu_hi, float *galpha, float *gbeta,
                         vc_stream_t stream);

/* Input-side gradient of the concretization and the first fc:
 * g (M, n_in) = xl * (A >= 0) + xh * (A <= 0) (torch's clamp subgradient),
 * g_out (M, n1) = g W0^T + bias0 with W0 (n1, n_in), bias0 (n1) nullable. */
int vc_alpha_grad_input(const float *A, const float *xl, const float *xh,
                        int64_t M, int R, int n_in, const float *W0,
                        const float *bias0, int n1, float *g_out,
                        vc_stream_t stream);

/* Adam step on n parameters with torch.optim.Adam's update order and
 * rounding (betas b1, b2, eps as the Python floats torch holds; the weights
 * 1 - b are formed in double and rounded to fp32), minimising -lb: the
 * gradient is -lb_grad; m = fma(1-b1, g - m, m), v = fma((1-b2) g, g, v b2),
 * p += (-step_size * m) / (sqrt(v) / bc2_sqrt + eps), then the projection
 * clamp to [lo_clamp, hi_clamp].  step_size = lr / (1 - b1^step) and
 * bc2_sqrt = sqrt(1 - b2^step) (step 1-based) are host-computed doubles. */
int vc_adam_step(float *param, const float *lb_grad, float *exp_avg,
                 float *exp_avg_sq, int64_t n, double b1, double b2, double eps,
                 double step_size, double bc2_sqrt, float lo_clamp,
                 float hi_clamp, vc_stream_t stream);

/* ReLU-split beta, one Adam step on n parameters: the backward sees the
 * signed beta (beta * sign), lb_grad_signed is d lb / d signed (the gbeta of
 * vc_alpha_grad_reduce), so the parameter gradient is sign * lb_grad_signed.
 * torch.optim.Adam update order on -lb as vc_adam_step, then beta clamped
 * to >= 0 and beta_signed = beta * sign written for the next evaluation.
 * Replaces the beta half of the Adam loop of verify_milp.py:2785-2807
 * (rsb = beta * sign at :2791, opt.step() and beta.clamp_(min=0)). */
int vc_beta_adam_step(float *beta, const float *sign,
                      const float *lb_grad_signed, float *exp_avg,
                      float *exp_avg_sq, int64_t n, double b1, double b2,
                      double eps, double step_size, double bc2_sqrt,
                      float *beta_signed, vc_stream_t stream);

/* sign (n) of each split neuron from dense clamps cl/ch (n): -1 where
 * cl == 0 (ON), else +1 where ch == 0 (OFF), else 0.
 * Replaces verify_milp.py:2777-2784. */
int vc_split_beta_sign(const float *cl, const float *ch, int64_t n,
                       float *sign, vc_stream_t stream);

/* Dense clamps of relu layer L for D domains from per-domain split lists
 * layer/neuron/side (D, S) int64 (layer -1 marks an unused slot; side 0 =
 * OFF: z <= 0, side 1 = ON: z >= 0): cl/ch (D, n) get -inf/+inf except 0
 * at the split neurons, and sign (nullable) as vc_split_beta_sign.
 * Replaces the per-domain clamp-building loop of verify_milp.py:2738-2752. */
int vc_split_clamps(const int64_t *layer, const int64_t *neuron,
                    const int64_t *side, int64_t D, int S, int64_t L, int n,
                    float *cl, float *ch, float *sign, vc_stream_t stream);

/* best = max(best, lb) elementwise (first call: copy when init != 0), and
 * out[0] = max over best, out[1] = 1.0 if all best > 0 else 0.0.
 * Replaces verify_zono_bnb.py:5252-5259. */
int vc_best_update(float *best, const float *lb, int64_t n, int init,
                   float *out2, vc_stream_t stream);

/* The bookkeeping of alpha-CROWN iteration `it` (0-based) without a host
 * round trip: best = lb (it == 0) or max(best, lb), then the loop control
 * of the reference -- stop when every best bound is > 0, or (it > 0) when
 * the global max of best rose by less than eps since the previous
 * iteration.  ctl (4 floats, start {-inf, 0, 0, 0}) = {previous max,
 * stopped, evaluated iterations, this max}; once stopped, later calls do
 * nothing, and vc_mlp_tiled_alpha_iter given ctl skips its work.
 * stop_host (nullable, pinned host memory): set to 1 when the loop stops,
 * a hint for the host thread that enqueues the iterations.
 * Replaces verify_zono_bnb.py:5252-5287 (best, the two breaks, prev_max). */
int vc_alpha_control(float *best, const float *lb, int64_t n, int it,
                     double eps, float *ctl, int32_t *stop_host, vc_stream_t stream);

/* ---- Whole-network kernels for narrow fc/ReLU chains ------------------- */
/* dims (host array, n_relu + 1 entries): dims[0] = inputs, dims[l + 1] =
 * width of ReLU layer l (the output of fc_l); every width <= 64,
 * 1 <= n_relu <= 16.  The final fc (to the network outputs) is not part of
 * these kernels; the caller folds it into the spec rows.  Weight fragments
 * are packed once per network; bias_cat concatenates the biases of
 * fc_0 .. fc_{n_relu-1}.  Per-layer tensors are passed as host arrays of
 * n_relu device pointers.  Return VC_ERR_UNSUPPORTED for shapes outside
 * these limits (the caller then uses the layer-wise entry points). */

/* Number of floats of the packed fragments (negative status on error). */
int64_t vc_mlp_frag_floats(const int32_t *dims, int n_relu, int forward);

/* Pack fc_0 .. fc_{n_relu-1} (W[l]: dims[l+1] x dims[l], device) into MFMA
 * A-operand fragments: forward (zonotope, A = W) or backward (CROWN, A = W^T). */
int vc_mlp_pack(const float *const *W, const int32_t *dims, int n_relu,
                int forward, float *frag, vc_stream_t stream);

/* Zonotope pre-activation bounds of every ReLU layer, one wavefront per
 * domain with the generator matrix in registers (per-domain generator
 * count: up to 128 columns including the centre, then a second pass with
 * one 4-wave workgroup and up to 512 columns per domain over the domains
 * that did not fit).  lo_out/hi_out[l]
 * (B, dims[l+1]).  overflow[b] = 1 when domain b needs more generator
 * columns; its bounds are then incomplete and must be recomputed with the
 * layer-wise entry points.
 * Replaces the ReLU bounds of _forward_zonotope_graph_batched
 * (verify_zono_bnb.py:3079-3211). */
int vc_mlp_zono_bounds(const int32_t *dims, int n_relu, const float *frag_fwd,
                       const float *bias_cat, int64_t B, const float *xl,
                       const float *xh, float *const *lo_out,
                       float *const *hi_out, int32_t *overflow,
                       vc_stream_t stream);

/* The second pass of vc_mlp_zono_bounds alone: the domains with
 * overflow[b] != 0 get one 4-wave workgroup and up to 512 generator
 * columns; overflow[b] is rewritten (1 = still does not fit).
 * Replaces the ReLU bounds of _forward_zonotope_graph_batched
 * (verify_zono_bnb.py:3079-3211) for those domains. */
int vc_mlp_zono_wide(const int32_t *dims, int n_relu, const float *frag_fwd,
                     const float *bias_cat, int64_t B, const float *xl,
                     const float *xh, float *const *lo_out, float *const *hi_out,
                     int32_t *overflow, vc_stream_t stream);

/* The first pass of vc_mlp_zono_bounds with the tile shape fixed at
 * compile time (frag from vc_mlp_tiled_pack): one wavefront per domain, up
 * to 128 generator columns including the centre; overflow[b] = 1 (a byte
 * flag, as vc_compact reads) for the domains that need more (to be
 * finished by vc_mlp_tiled_zono_wide).  queue: as for vc_mlp_tiled_crown
 * (domains differ in cost by their generator counts).
 * Replaces the ReLU bounds of _forward_zonotope_graph_batched
 * (verify_zono_bnb.py:3079-3211). */
int vc_mlp_tiled_zono_bounds(const int32_t *dims, int n_relu, const float *frag,
                             const float *bias_cat, int64_t B, const float *xl,
                             const float *xh, float *const *lo_out,
                             float *const *hi_out, uint8_t *overflow, int32_t *queue,
                             vc_stream_t stream);

/* vc_mlp_zono_wide with the tile shape fixed at compile time (frag from
 * vc_mlp_tiled_pack): the *n_list domains list[0 .. *n_list) (device
 * memory, as vc_compact writes them from the overflow flags), dealt
 * round-robin over the workgroups, one 4-wave workgroup per domain with up
 * to 512 generator columns spread over the waves; overflow[list[k]]
 * rewritten (1 = still does not fit).  The count is read on the device, so
 * the call needs no host synchronisation.
 * Replaces the ReLU bounds of _forward_zonotope_graph_batched
 * (verify_zono_bnb.py:3079-3211) for those domains. */
int vc_mlp_tiled_zono_wide(const int32_t *dims, int n_relu, const float *frag,
                           const float *bias_cat, int64_t B, const float *xl,
                           const float *xh, float *const *lo_out,
                           float *const *hi_out, uint8_t *overflow,
                           const int64_t *list, const int64_t *n_list,
                           vc_stream_t stream);

/* CROWN intermediate bounds and the spec backward, whole network per
 * wavefront.  With do_crown != 0, layer L is tightened by seeding
 * [+I; -I] at its pre-activation for the idx_cnt[L] neurons listed in
 * idx_all (concatenated per layer), intersecting with lo_in/hi_in and
 * writing lo_out/hi_out[L] (B, dims[L+1]); with do_crown == 0 the bounds
 * lo_in/hi_in are used as given.  With Q > 0 (Q <= 32) the spec rows
 * spec_rows (Q, dims[n_relu]) and their constants spec_acc (Q) -- the spec
 * already folded through the final fc -- are propagated to the input:
 * lb_out (B, Q), and when non-NULL A_out (B, Q, dims[0]), acc_out (B, Q).
 * Replaces _crown_intermediate_batched (verify_zono_bnb.py:4077-4147) and
 * _spec_backward_graph_batched with return_input_linear
 * (verify_zono_bnb.py:4270-4453, 5117-5134). */
int vc_mlp_crown(const int32_t *dims, int n_relu, const float *frag_bwd,
                 const float *bias_cat, int64_t B, const float *xl,
                 const float *xh, const float *const *lo_in,
                 const float *const *hi_in, float *const *lo_out,
                 float *const *hi_out, const int32_t *idx_all,
                 const int32_t *idx_cnt, int do_crown, int Q,
                 const float *spec_rows, const float *spec_acc, float *lb_out,
                 float *A_out, float *acc_out, vc_stream_t stream);

/* Floats of the fragment buffer of vc_mlp_tiled_crown for this network, or
 * minus a status when no shape-specialised kernel holds it (every hidden
 * fc then needs K-steps and M-tiles beyond the largest instantiation).
 * Part of the replacement of _crown_intermediate_batched
 * (verify_zono_bnb.py:4077-4147). */
int64_t vc_mlp_tiled_floats(const int32_t *dims, int n_relu);

/* Pack fc_0 .. fc_{n_relu-1} (W[l] (dims[l+1], dims[l]), bias[l]
 * (dims[l+1])) into the vc_mlp_tiled_crown layout: each fc's transposed
 * weights plus its bias as one extra row of the MFMA A operand, hidden
 * layers as [K-step][lane][M-tile]. */
int vc_mlp_tiled_pack(const float *const *W, const float *const *bias,
                      const int32_t *dims, int n_relu, float *frag,
                      vc_stream_t stream);

/* Which kernel vc_mlp_tiled_crown runs for B domains on the current
 * device: 0 = one wavefront per domain (large batches), 1 = several
 * wavefronts per domain, up to 4 domains per workgroup (B <= 4 x compute
 * units).  Both compute the same rows with the same arithmetic.  No
 * counterpart in the reference (a dispatch rule of this library). */
int vc_mlp_tiled_crown_mode(int64_t B);

/* vc_mlp_crown with the tile shape fixed at compile time (same results;
 * frag from vc_mlp_tiled_pack, Q <= 64): no MFMA under a runtime condition,
 * the fc bias carried by the MFMA, the per-row constants accumulated in
 * fp64.  The seeded neuron lists stay on the device: idx_meta (device,
 * 2 * n_relu int32) holds the per-layer counts, then their offsets into
 * idx_all, as written by vc_union_compact.  per_domain != 0 seeds, in each
 * domain, only the listed neurons with lo < 0 and hi > -1e-7 there: the
 * spec bound, A, acc and every relaxation are those of seeding the whole
 * list (the other neurons have slopes their tightening cannot change);
 * lo_out/hi_out of the unseeded neurons keep lo_in/hi_in.  seed_rows
 * (device, n_relu uint64, nullable) accumulates the seeded neurons per
 * layer over all domains (the work done, for the roofline).  queue
 * (device int32, nullable): a counter the call resets and then uses to hand
 * the domains to wavefronts as they finish (domains differ in cost by
 * their seed counts); calls that may overlap in time need distinct
 * counters.  Batches with vc_mlp_tiled_crown_mode(B) == 1 spread each
 * domain's row tiles over several wavefronts (identical results).
 * Replaces _crown_intermediate_batched (verify_zono_bnb.py:4077-4147) and
 * _spec_backward_graph_batched with return_input_linear
 * (verify_zono_bnb.py:4270-4453, 5117-5134). */
int vc_mlp_tiled_crown(const int32_t *dims, int n_relu, const float *frag,
                       const float *bias_cat, int64_t B, const float *xl,
                       const float *xh, const float *const *lo_in,
                       const float *const *hi_in, float *const *lo_out,
                       float *const *hi_out, const int32_t *idx_all,
                       const int32_t *idx_meta, int do_crown, int per_domain,
                       int Q, const float *spec_rows, const float *spec_acc,
                       float *lb_out, float *A_out, float *acc_out,
                       uint64_t *seed_rows, int32_t *queue, vc_stream_t stream);

/* vc_mlp_tiled_crown with the work laid out by layer (same arguments and
 * results, bit for bit; seed_rows as there; queue not needed): the seeded
 * rows of one layer of every domain are packed into full 16-row MFMA tiles
 * and the spec rows of 16 / Q domains share a tile, where
 * vc_mlp_tiled_crown gives every domain tiles of its own.  Each row reads
 * its domain's slopes of the layers below from a slope buffer in `work`
 * (vc_mlp_crown_rows_workspace(dims, n_relu, B) bytes: masks, row offsets,
 * row lists and bounds of one layer, and the slopes of every layer, 512 B
 * per domain and layer).  lo_out/hi_out: nullable (both or neither).
 * idx_all/idx_meta: the union lists of vc_union_compact, or null: then the
 * union of the neurons unstable in some domain (lo < 0 < hi) is formed here,
 * in the same pass over the bounds that builds the per-domain seed masks
 * (the same union, so the same results).  B < 2^24; the workspace size is
 * -VC_ERR_UNSUPPORTED past it, and callers then take vc_mlp_tiled_crown.  Replaces
 * _crown_intermediate_batched + the spec backward (verify_zono_bnb.py:
 * 4077-4147, 4270-4453, 5117-5134) for narrow MLPs. */
int64_t vc_mlp_crown_rows_workspace(const int32_t *dims, int n_relu, int64_t B);
int vc_mlp_crown_rows(const int32_t *dims, int n_relu, const float *frag,
                      const float *bias_cat, int64_t B, const float *xl,
                      const float *xh, const float *const *lo_in,
                      const float *const *hi_in, float *const *lo_out,
                      float *const *hi_out, const int32_t *idx_all,
                      const int32_t *idx_meta, int do_crown, int per_domain,
                      int Q, const float *spec_rows, const float *spec_acc,
                      float *lb_out, float *A_out, float *acc_out,
                      uint64_t *seed_rows, void *work, int64_t work_bytes,
                      vc_stream_t stream);

/* No counterpart in the reference: vc_mlp_tiled_crown for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  Same arguments, kernels and
 * results as vc_unstable_union_layers + vc_union_compact +
 * vc_mlp_tiled_crown (seed_rows off), but the union flags, its index lists
 * and the domain queue's counter live in a static 8 KiB device array, one
 * per GPU, held until the process ends; the call allocates nothing.  The
 * caller passes the inputs and outputs only.  Limit: the ReLU widths may
 * sum to at most 1024 (VC_ERR_UNSUPPORTED beyond).  Calls that overlap on
 * one GPU (two host threads, or two streams) share the array and race:
 * serialise them.  Any batch size B.  The GPU is the one running `stream`
 * (the current device for the null stream). */
int vc_mlp_tiled_crown_noalloc(const int32_t *dims, int n_relu,
                               const float *frag, const float *bias_cat,
                               int64_t B, const float *xl, const float *xh,
                               const float *const *lo_in,
                               const float *const *hi_in,
                               float *const *lo_out, float *const *hi_out,
                               int do_crown, int per_domain, int Q,
                               const float *spec_rows, const float *spec_acc,
                               float *lb_out, float *A_out, float *acc_out,
                               vc_stream_t stream);

/* The neurons unstable in any domain, per layer, for the CROWN seeding of
 * _crown_intermediate_batched (verify_zono_bnb.py:4123): flags (sum of
 * widths, uint8) = 1 where some domain has lo < 0 < hi, for n_layers
 * layers lo[L]/hi[L] (B, widths[L]) in one launch (flags cleared first). */
int vc_unstable_union_layers(const float *const *lo, const float *const *hi,
                             const int32_t *widths, int n_layers, int64_t B,
                             uint8_t *flags, vc_stream_t stream);

/* Compact the flags of vc_unstable_union_layers (n_layers <= 16): idx
 * (device, sum of widths int32) lists layer L's flagged neurons in
 * increasing order from offset off[L]; meta (device, 2 n_layers int32) =
 * {cnt[0..n_layers), off[0..n_layers)}.  Part of verify_zono_bnb.py:4123. */
int vc_union_compact(const uint8_t *flags, const int32_t *widths, int n_layers,
                     int32_t *idx, int32_t *meta, vc_stream_t stream);

/* One batched alpha-CROWN Adam iteration, whole network per wavefront
 * (n_relu <= 7, 1 <= Q <= 16): evaluates lb_out (B, Q) with lower slopes
 * active + unstable * alpha on the bounds lo/hi, computes d(sum lb)/d alpha
 * analytically (torch's clamp subgradients) and applies torch.optim.Adam on
 * -sum lb (betas b1, b2, eps; step_size = lr / (1 - b1^step), bc2_sqrt =
 * sqrt(1 - b2^step)) followed by the clamp to [0, 1].  alpha, exp_avg,
 * exp_avg_sq: per-layer (B, dims[l+1]) device arrays, updated in place.
 * Replaces one iteration of _run_alpha_crown_inputsplit_batched
 * (verify_zono_bnb.py:5248-5266). */
int vc_mlp_alpha_iter(const int32_t *dims, int n_relu, const float *frag_bwd,
                      const float *bias_cat, int64_t B, const float *xl,
                      const float *xh, const float *const *lo,
                      const float *const *hi, float *const *alpha,
                      float *const *exp_avg, float *const *exp_avg_sq, int Q,
                      const float *spec_rows, const float *spec_acc,
                      float *lb_out, double b1, double b2, double eps,
                      double step_size, double bc2_sqrt, vc_stream_t stream);

/* vc_mlp_alpha_iter with the tile shape fixed at compile time (same
 * arguments and results; frag from vc_mlp_tiled_pack; n_relu <= 16 as the
 * LDS allows, 1 <= Q <= 16): the pre-relaxation rows kept in LDS, the fc
 * biases carried by the MFMA in both directions.  init != 0 (the first
 * iteration): alpha starts at (up_s > 0.5) * unstable and the Adam state at
 * zero, whatever the arrays hold.  ctl (nullable): the loop state of
 * vc_alpha_control; the call does nothing once it says stopped.  grad
 * (nullable; else per-layer (B, dims[l+1]) device arrays): the iteration's
 * d(sum_q lb_q)/d alpha, the gradient its Adam step took with the opposite
 * sign (torch minimises -sum lb), 0 off the unstable set.
 * Replaces one iteration of _run_alpha_crown_inputsplit_batched
 * (verify_zono_bnb.py:5248-5266). */
int vc_mlp_tiled_alpha_iter(const int32_t *dims, int n_relu, const float *frag,
                            const float *bias_cat, int64_t B, const float *xl,
                            const float *xh, const float *const *lo,
                            const float *const *hi, float *const *alpha,
                            float *const *exp_avg, float *const *exp_avg_sq,
                            float *const *grad, int Q, const float *spec_rows,
                            const float *spec_acc, float *lb_out, double b1,
                            double b2, double eps, double step_size,
                            double bc2_sqrt, int init, const float *ctl,
                            vc_stream_t stream);

/* The whole loop of _run_alpha_crown_inputsplit_batched
 * (verify_zono_bnb.py:5239-5287) in one call: n_iters >= 1 iterations of
 * vc_mlp_tiled_alpha_iter, each followed by vc_alpha_control, launched
 * back to back with the loop control on the device.  Batches of at most
 * 4 x compute units run up to VC_ALPHA_CHUNK iterations per launch on
 * their LDS state; the control then takes those iterations in order and
 * discards the ones after a stop (the result is that of stopping there).
 * lb_out: scratch of VC_ALPHA_CHUNK x B x Q floats.  ctl (4 floats) is set
 * here and ends as vc_alpha_control leaves it (ctl[2] = evaluated
 * iterations); best (B, Q) = the best bound per spec row.  Torch Adam's
 * schedule: step size lr_t / (1 - b1^t), bias correction (1 - b2^t)^0.5,
 * lr_{t+1} = lr_t * lr_decay.  stop_host (nullable; two int32 words of
 * pinned host memory, zero on entry): the control sets word 0 when the
 * loop stops and stores in word 1 how many iterations it has taken; the
 * host keeps one chunk of iterations enqueued beyond the controls it has
 * seen (a bounded wait) and skips the chunks after a stop, which would do
 * nothing. */
int vc_mlp_tiled_alpha_run(const int32_t *dims, int n_relu, const float *frag,
                           const float *bias_cat, int64_t B, const float *xl,
                           const float *xh, const float *const *lo,
                           const float *const *hi, float *const *alpha,
                           float *const *exp_avg, float *const *exp_avg_sq, int Q,
                           const float *spec_rows, const float *spec_acc,
                           float *lb_out, float *best, double b1, double b2,
                           double eps, double lr, double lr_decay, int n_iters,
                           double early_stop_eps, float *ctl, int32_t *stop_host,
                           vc_stream_t stream);

/* ---- Input-split BaB step ---------------------------------------------- */

/* Closure: closed[b] = AND over disjuncts d of (OR over q in d of
 * lb[b, q] > 0); disjunct d owns q_idx[d_ptr[d] .. d_ptr[d+1]).
 * Replaces verify_graph.py:12899-12908. */
int vc_closure(const float *lb, int64_t B, int Q, const int32_t *d_ptr,
               const int32_t *q_idx, int n_disj, uint8_t *closed,
               vc_stream_t stream);

/* Halfspace box clip of {x in [xl, xh] : A_q x + b_q <= 0 for q in D} per
 * disjunct D, and the bounding box of the union over feasible disjuncts
 * (single disjunct: plain clip).  A (B, Q, n), b (B, Q); Q <= 64 and at
 * most 64 queries per disjunct (VC_ERR_UNSUPPORTED beyond 64 queries).
 * Replaces _clip_box_by_halfspaces_batched (verify_graph.py:12363-12426)
 * and the multi-disjunct union (verify_graph.py:13040-13074). */
int vc_clip_box(const float *xl, const float *xh, const float *A,
                const float *b, int64_t B, int Q, int n, const int32_t *d_ptr,
                const int32_t *q_idx, int n_disj, float *xl_out,
                float *xh_out, uint8_t *feasible, vc_stream_t stream);

/* flag[0] = 1 if the new boxes are tighter anywhere than the old ones
 * (xl_new > xl_old or xh_new < xh_old over the n entries), else 0: the stop
 * test of the clip loop, `((xl_new > xl_c) | (xh_new < xh_c)).any()`
 * (verify_graph.py:13036-13081, stop test at 13078). */
int vc_box_shrunk(const float *xl_old, const float *xh_old,
                  const float *xl_new, const float *xh_new, int64_t n,
                  int32_t *flag, vc_stream_t stream);

/* Ascending stream compaction: idx_out[0..count) = positions of non-zero
 * flags (of zero flags when select_zero != 0); count_out[0] = count.
 * workspace >= vc_compact_workspace(n) bytes.
 * Replaces torch.nonzero on the closure / feasibility / usable masks
 * (verify_graph.py:12986, 13115, 13372). */
int64_t vc_compact_workspace(int64_t n);
int vc_compact(const uint8_t *flags, int64_t n, int select_zero,
               int64_t *idx_out, int64_t *count_out, void *workspace,
               int64_t ws_bytes, vc_stream_t stream);

/* Max-merge of row blocks: rows[idx[r], :] = max(rows[idx[r], :], src[r, :])
 * over rows of q floats.  Replaces the alpha-CROWN merge
 * spec_lbs_b[close_idx] = max(old, new) (verify_graph.py:12966-12967). */
int vc_scatter_max_rows(float *rows, const int64_t *idx, const float *src,
                        int64_t n_rows, int q, vc_stream_t stream);

/* Row gather: out[r] = in[idx[r]] for rows of `cols` floats. */
int vc_gather_rows(const float *in, const int64_t *idx, int64_t n_rows,
                   int cols, float *out, vc_stream_t stream);

/* vc_gather_rows for n_arrays (<= 32) arrays in one launch: out[a] (n_rows,
 * cols[a]) = in[a][idx] with the same row list. */
int vc_gather_rows_multi(const float *const *in, float *const *out,
                         const int32_t *cols, int n_arrays, const int64_t *idx,
                         int64_t n_rows, vc_stream_t stream);

/* Row scatter: out[idx[r]] = in[r] for rows of `cols` floats. */
int vc_scatter_rows(const float *in, const int64_t *idx, int64_t n_rows,
                    int cols, float *out, vc_stream_t stream);

/* Widest-dimension selection: ax[b] = first argmax_i (xh - xl)[b, i];
 * usable[b] = (xh - xl)[b, ax] > 1e-12.
 * Replaces verify_graph.py:13291 and 13366-13369. */
int vc_widest_axis(const float *xl, const float *xh, int64_t B, int n,
                   int64_t *ax, uint8_t *usable, vc_stream_t stream);

/* Bisection of the usable leaves listed in u_idx (n_u entries): children
 * low = (xl, xh with ax = mid) and high = (xl with ax = mid, xh),
 * mid = (lo + hi) * 0.5.  Outputs are (n_u, n) each.
 * Replaces verify_graph.py:13370-13382. */
int vc_bisect(const float *xl, const float *xh, const int64_t *ax,
              const int64_t *u_idx, int64_t n_u, int n, float *low_xl,
              float *low_xh, float *high_xl, float *high_xh,
              vc_stream_t stream);

/* Split-dimension selection: the K (1..8, <= n) best input dimensions of
 * each of B leaves, best first, into dims (B, K).  Scores in the
 * reference's fp32 operation order (verify_graph.py:13271-13285):
 *   mode 0: widest, w_i = xh_i - xl_i;
 *   mode 1: SB sum, w_i * sum_q |A[b, q, i]| (q ascending);
 *   mode 2: SB margin, max_q (max(|A[b, q, i]|, thr) * w_i / 2 + lb[b, q] * mw).
 * A (B, Q, n) is the leaves' input linearization, lb (B, Q) their spec lower
 * bounds (mode 2 only).  Ties go to the lower index (torch.argmax's first
 * maximum for K = 1; for K > 1 the order of a stable descending sort, which
 * is torch.topk's wherever the scores differ).  usable (B, nullable): the
 * first chosen dimension is wider than 1e-12 (the bisection's test).
 * Replaces the score and argmax / topk of verify_graph.py:13244-13291,
 * 13348-13351. */
int vc_branch_topk(const float *xl, const float *xh, const float *A,
                   const float *lb, int64_t B, int Q, int n, int mode,
                   float thr, float mw, int K, int64_t *dims,
                   uint8_t *usable, vc_stream_t stream);

/* Plan of the 2^K-way split (verify_graph.py:13392-13420): per leaf the
 * usable dimensions among its K split dimensions dims (B, K) (width >
 * 1e-12), children 2^K_u (0 when none is usable).  offsets (B + 1): the
 * exclusive prefix sum of the child counts, offsets[B] the total;
 * n_degenerate: leaves with no usable dimension.  One workgroup. */
int vc_split_multi_plan(const float *xl, const float *xh, const int64_t *dims,
                        int64_t B, int n, int K, int64_t *offsets,
                        int64_t *n_degenerate, vc_stream_t stream);

/* The children of that plan into out_xl / out_xh (offsets[B], n): leaf b's
 * child combo (0 .. 2^K_u - 1) at row offsets[b] + combo, bit k of combo
 * taking the high half (lower end = midpoint (lo + hi) / 2) of the k-th
 * usable dimension, else the low half.  Replaces the per-leaf loop of
 * verify_graph.py:13392-13420. */
int vc_split_multi(const float *xl, const float *xh, const int64_t *dims,
                   const int64_t *offsets, int64_t B, int n, int K,
                   float *out_xl, float *out_xh, vc_stream_t stream);

/* Boundary band of the alpha-CROWN leaves (verify_graph.py:12938-12946):
 * keys (B) = min over disjuncts of the max over the disjunct's queries of
 * lb (B, Q) (disjunct table as vc_closure); cand (B) = not closed and key >
 * neg_eps (the reference's -alpha_eps, as fp32). */
int vc_alpha_band_keys(const float *lb, int64_t B, int Q, const int32_t *d_ptr,
                       const int32_t *q_idx, int n_disj, const uint8_t *closed,
                       float neg_eps, float *keys, uint8_t *cand,
                       vc_stream_t stream);

/* The k_max best of C candidates (leaves idx, ascending) by key,
 * descending, ties in leaf order (a stable sort; the reference's argsort
 * leaves their order open): out[0 .. min(C, k_max) - 1].  Replaces the
 * argsort and truncation of verify_graph.py:12947-12950. */
int vc_rank_select_desc(const float *keys, const int64_t *idx, int64_t C,
                        int64_t k_max, int64_t *out, vc_stream_t stream);

/* Layer tightening of the hybrid freeze / replay (verify_hybrid_acasxu.py:
 * 231-235, 279-283): with sl (B, 2n) the lower bounds of the seeded rows
 * [+I; -I], lo = max(lo, sl[:, :n]), hi = min(hi, -sl[:, n:]),
 * lo = min(lo, hi), in place on lo, hi (B, n). */
int vc_bound_tighten(float *lo, float *hi, const float *sl, int64_t B, int n,
                     vc_stream_t stream);

/* best = max(best, lb) over n values (a copy when init != 0), and
 * out[0] = the sum of best in fp64 (the early-stop quantity of the freeze's
 * Adam loops, verify_hybrid_acasxu.py:212-225, 262-272).  One workgroup. */
int vc_best_sum(float *best, const float *lb, int64_t n, int init, double *out,
                vc_stream_t stream);

/* Replay's running best (verify_hybrid_acasxu.py:302-311): per leaf b,
 * imp = lb[b] > best[b] (every entry when init != 0), best[b] = where(imp,
 * lb[b], best[b]); when any entry improved, best_A[b] = A[b] (Q x n_in). */
int vc_best_rows_with_A(float *best, const float *lb, float *best_A,
                        const float *A, int64_t B, int Q, int n_in, int init,
                        vc_stream_t stream);

/* One input-split BaB round on the narrow-MLP kernels (the bound,
 * alpha, clip and split phases of verify_graph.py:12855-13382, with
 * crown intermediate bounds, the clip on and alpha-CROWN on every open leaf),
 * orchestrated in host C++: every step is one of the entry points above on
 * `stream`; the three counts the round needs (open, unclosed, feasible +
 * split) are read on the host (see `pinned`).  frag, bias_cat: from
 * vc_mlp_tiled_pack; spec_rows/spec_acc: the Q spec rows folded through the
 * last fc; d_ptr/q_idx/n_disj: the disjunct table of vc_closure.  Outputs,
 * device, sized for B rows: lb (B, Q), A (B, Q, n_in), acc (B, Q), closed
 * (B), unclosed (the first counts[2] entries), feasible (per unclosed row),
 * xl_split/xh_split/ax (the first counts[3] rows), low/high children (the
 * first counts[4] rows).  low_xl and low_xh both null: the low children
 * follow the high ones in high_xl / high_xh (rows counts[4] .. 2 counts[4];
 * each then holds 2 B rows), so the next batch in a LIFO worklist's pop
 * order (high, then low) is one contiguous block instead of a
 * concatenation.  counts (host int64[7]) = {open leaves, alpha
 * iterations evaluated, unclosed, feasible, split, degenerate, handed-over
 * children (-1: no lookahead)}.  work:
 * vc_mlp_bab_round_workspace(dims, n_relu, B, Q) bytes of device memory;
 * stop_host: as for vc_mlp_tiled_alpha_run.  seed_rows (nullable): as for
 * vc_mlp_tiled_crown; crown_ev0/crown_ev1 (nullable hipEvent_t): recorded
 * on `stream` around the vc_mlp_tiled_crown call (its timing).  phase_ev
 * (nullable, 5 hipEvent_t): recorded on `stream` at the round's start and
 * at the end of its bound (zonotope, CROWN, closure), alpha (with the
 * closure of the raised rows), clip (unclosed compaction, clip, widest
 * axis, feasible compaction and gather) and split (bisection) phases: the
 * driver's per-phase profile without a synchronisation per phase
 * (verify_graph.py:12814-12833, 12984-12985, 13227-13228, 13430-13433).
 * clip_widths (nullable, device double[2], zeroed by the caller):
 * += the sums of max(xh - xl, 0) over the unclosed leaves before and after
 * the clip (the profile's shrink ratio, verify_graph.py:13108-13113).
 * pinned (nullable, pinned host memory, >= 2 int64): the GPU stores each
 * count there and the host polls it (bounded, then a stream
 * synchronisation) instead of a device-to-host copy and a
 * synchronisation.  fail_phase (nullable host int32): -1 on success, else
 * the phase whose step returned the error (0 bound, 1 alpha, 2 clip,
 * 3 split): the driver halves the batch only on the bound phase's errors
 * (verify_graph.py:12853-12897), and alpha's keep the CROWN bound
 * (:12962-12969).  VC_ERR_UNSUPPORTED when the net can have more zonotope
 * generators than VC_ZONO_WIDE_COLS.  Replaces one iteration of
 * _input_split_batched_inner's loop body (verify_graph.py:12855-13382),
 * as bab_step restates it.
 *
 * Lookahead (la_work non-null, with aux_stream: another stream of the same
 * device at the default priority).  When alpha runs, it and the raise of
 * its rows go to aux_stream with every chunk enqueued at once (stop_host is
 * not used), while `stream` clips and splits the leaves the CROWN bound
 * leaves open and runs the bound phase on all their children (the high
 * halves first, then the low ones: the order in which a LIFO worklist pops
 * the two pushes).  After alpha, the children of the leaves it closed are
 * dropped, and the bound phase of the others -- the next batch, in its
 * order -- is left at the start of la_work for the next round's `pre`;
 * counts[6] is their number (2 counts[4]).  Each box's bounds depend on that
 * box alone, and alpha only closes leaves, so the round and the next one
 * give the results they give without it.  la_work:
 * vc_mlp_bab_round_lookahead_workspace(dims, n_relu, B, Q, la_cap) bytes;
 * more than la_cap children (or a bound workspace beyond la_bytes) skip
 * the lookahead (counts[6] = -1).  pre (nullable): the la_work of the
 * previous round's call, whose counts[6] is this call's B, with xl/xh that
 * round's high then low children: the round takes its bound phase from there
 * (crown_ev0/crown_ev1 and seed_rows are then not used).  la_work must stay
 * untouched until the next round's call has returned.
 *
 * Tail bound (la_work non-null, aux_stream null, low_xl and low_xh null):
 * no overlap; after the split, `stream` runs the bound phase on the
 * 2 counts[4] children (high then low, the next batch as it is) and leaves
 * it in la_work for the next call's `pre` (counts[6] = 2 counts[4]; -1
 * above la_cap, or with phase_ev or clip_widths).  The GPU then works while
 * the host returns from this call and makes the next one.  la_bytes as for
 * the lookahead. */
int64_t vc_mlp_bab_round_workspace(const int32_t *dims, int n_relu, int64_t B,
                                   int Q);
int64_t vc_mlp_bab_round_lookahead_workspace(const int32_t *dims, int n_relu,
                                             int64_t B, int Q, int64_t la_cap);

/* Byte offsets (off[0..2]) in la_work of the handed-over spec bound (B, Q),
 * A (B, Q, n_in) and acc (B, Q) of B children.  A call given that la_work
 * as `pre` with its lb, A and acc at those addresses reads and updates
 * them in place instead of copying them (any other outputs are filled
 * with copies).  Has no counterpart in the reference: the layout of the
 * handoff between two native rounds. */
int vc_mlp_bab_round_handoff_offsets(const int32_t *dims, int n_relu, int64_t B,
                                     int Q, int64_t *off);
int vc_mlp_bab_round(const int32_t *dims, int n_relu, const float *frag,
                     const float *bias_cat, int Q, const float *spec_rows,
                     const float *spec_acc, const int32_t *d_ptr,
                     const int32_t *q_idx, int n_disj, int64_t B,
                     const float *xl, const float *xh, int alpha_iters,
                     double alpha_lr, double alpha_lr_decay,
                     double alpha_early_stop, float *lb, float *A, float *acc,
                     uint8_t *closed, int64_t *unclosed, uint8_t *feasible,
                     float *xl_split, float *xh_split, int64_t *ax,
                     float *low_xl, float *low_xh, float *high_xl,
                     float *high_xh, uint64_t *seed_rows, void *crown_ev0,
                     void *crown_ev1, void *const *phase_ev, double *clip_widths,
                     void *work, int64_t work_bytes, const void *pre,
                     void *la_work, int64_t la_bytes, int64_t la_cap,
                     vc_stream_t aux_stream, int32_t *stop_host,
                     int64_t *pinned, int64_t *counts, int32_t *fail_phase,
                     vc_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VIBECHECK_AMD_H */
