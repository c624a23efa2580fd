/*
 * rqf_scan.h -- C ABI of the MI355X (gfx950) complex linear-recurrence scan
 * library (librqf_hip.so).
 *
 * Each entry point replaces one host->device launch of the reference's
 * Triton kernels (Sequel-Institute/prospective-rqf, rqf_models/ops/).  The
 * citations name the launch site being replaced.
 *
 * Conventions
 *   - All pointers are device pointers into caller-owned memory.  The library
 *     never allocates device memory.  Where scratch is needed, a *_workspace()
 *     query returns its size and the caller passes the buffer in.
 *   - Complex tensors are complex64 stored interleaved (re, im) as float
 *     pairs.  Every tensor is dense and C-contiguous in the layout named.
 *   - "FBT" layout: element (f, b, t) at (f*B + b)*T + t (channel-outermost).
 *     "BTF" layout: element (b, t, f) at (b*T + t)*F + f.
 *   - Launches are asynchronous on `stream` (a hipStream_t; NULL is the null
 *     stream).  No function synchronises the host.
 *   - Return value: RQF_OK (0) on success; a negative RQF_ERR_* for a bad
 *     argument; a positive hipError_t when a launch fails.
 *   - Size limit: a dispatch counts its work-items in 32 bits, and a larger
 *     grid would run truncated with no launch error.  A call whose scan grid
 *     needs more than 2^32 - 1 work-items returns RQF_ERR_ARG before launching
 *     anything.  For example, the (B,T,F) scans take B * ceil(F / 16) <=
 *     8388607 blocks of 512 threads (F <= 134217712 at B = 1).  The FBT and
 *     selective forwards take up to 8388607 rows (F * B, rounded up per XCD
 *     chunk of the batch).  Reductions over filters or channels stride, so
 *     they take any size.
 *   - Row length: the selective scans take T < 2^30 steps (RQF_ERR_ARG
 *     otherwise); the time-invariant and multi-oscillator scans take any T.
 *   - Results are deterministic: coefficient gradients are reduced from
 *     per-row partial sums in a fixed order (no floating-point atomics).
 *   - Calls are reentrant.  No mutable global state exists, except for the
 *     one no-allocation entry point (rqf_fbt_recompute_bwd_noalloc), whose
 *     static per-GPU scratch calls on one GPU share.
 */
#ifndef RQF_SCAN_H
#define RQF_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *rqf_stream_t; /* hipStream_t */

enum {
  RQF_OK = 0,
  RQF_ERR_ARG = -1,       /* null pointer, bad shape or chunk, or an oversized grid */
  RQF_ERR_WORKSPACE = -2, /* workspace missing or too small */
  RQF_ERR_ALIGN = -3,     /* a tensor is not 8-byte aligned */
  RQF_ERR_SCRATCH = -4    /* problem exceeds the static scratch of a no-allocation entry */
};

/* Bytes of the static device scratch of rqf_fbt_recompute_bwd_noalloc (per GPU). */
#define RQF_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)

/* Library version string and the offload target it was built for. */
const char *rqf_version(void);
/* Human-readable message for a return code of this library. */
const char *rqf_error_string(int code);

/* ------------------------------------------------------------------------ *
 * Time-invariant scans in the reference's (batch, time, filters) API.       *
 *   x[t] = C1*x[t-1] + C2*u[t]                           (plain)            *
 *   x[t] = C1*x[t-1] + tap0*u[t] + tap1*u[t-1]           (prospective)      *
 * c1, c2, tap0, tap1: (F,) complex.  u, out, states, grads: BTF complex.    *
 * grad_c1 / grad_c2 / grad_tap0 / grad_tap1: (F,) complex, overwritten.     *
 * ------------------------------------------------------------------------ */

size_t rqf_btf_scan_workspace(int64_t B, int64_t T, int64_t F);

/* Replaces `_chunked_scan_kernel[grid](...)`
 * (rqf_models/ops/chunked_scan_kernel.py:238-247) including its two permute
 * copies (:231, :249): works on (B,T,F) directly. */
int rqf_chunked_scan_fwd(const float *c1, const float *c2, const float *u, float *out,
                         int64_t B, int64_t T, int64_t F, void *workspace,
                         size_t workspace_bytes, rqf_stream_t stream);

/* Replaces `_chunked_scan_backward_kernel[grid](...)`
 * (rqf_models/ops/chunked_scan_kernel.py:286-299): grad_u = conj(C2) g,
 * grad_C1 = sum conj(x[t-1]) g, grad_C2 = sum conj(u) g, where x is the
 * forward's output.  grad_C1 is evaluated with the order of summation
 * exchanged, from u, so `states` (the saved output the reference passes) is
 * accepted but not read and may be NULL. */
int rqf_chunked_scan_bwd(const float *c1, const float *c2, const float *u,
                         const float *states, const float *grad_out, float *grad_u,
                         float *grad_c1, float *grad_c2, int64_t B, int64_t T, int64_t F,
                         void *workspace, size_t workspace_bytes, rqf_stream_t stream);

/* Replaces `_chunked_prospective_kernel[grid](...)`
 * (rqf_models/ops/chunked_scan_kernel.py:459-469). */
int rqf_chunked_prospective_fwd(const float *c1, const float *tap0, const float *tap1,
                                const float *x, float *out, int64_t B, int64_t T, int64_t F,
                                void *workspace, size_t workspace_bytes,
                                rqf_stream_t stream);

/* Replaces `_ChunkedProspectiveScanFunction.backward`
 * (rqf_models/ops/chunked_scan_kernel.py:491-503): the chunked adjoint plus
 * its PyTorch finisher, fused: grad_x = conj(tap0) g[t] + conj(tap1) g[t+1].
 * As in rqf_chunked_scan_bwd, `states` is accepted but not read (may be NULL). */
int rqf_chunked_prospective_bwd(const float *c1, const float *tap0, const float *tap1,
                                const float *x, const float *states, const float *grad_out,
                                float *grad_x, float *grad_c1, float *grad_tap0,
                                float *grad_tap1, int64_t B, int64_t T, int64_t F,
                                void *workspace, size_t workspace_bytes,
                                rqf_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Multi-oscillator scans with C-weight reduction, and the |y| readout       *
 * (BTF layout).  N >= 1 oscillators per filter f, index f*N + n:          *
 *   x_n[t] = C1_n*x_n[t-1] + C2_n*u[t]                                      *
 *   y[t]   = sum_n cw_n*x_n[t]          (cw NULL: y = x_0, requires N = 1)  *
 * c1, c2, cw: (F*N,) complex (cw is the reference's real (F*N, 2) view).    *
 * u: (B,T,F) complex, or real when u_real != 0.                            *
 * ------------------------------------------------------------------------ */

/* Workspace bytes of rqf_multi_osc_fwd (backward = 0) or _bwd (backward = 1);
 * 0 for a shape they reject (N < 1 or N > 2^20, B*ceil(F/16) past 4194303
 * blocks of up to 1024 threads, F*N past 2^31 - 1).  The forward needs none unless N > 4 with out_abs.  Up to
 * 65536 filters the forward addresses each pass of up to 2048 steps through
 * one 32-bit buffer range; wider rows run it with 64-bit addresses. */
size_t rqf_multi_osc_workspace(int64_t B, int64_t T, int64_t F, int64_t N, int32_t backward);

/* Replaces `_sequential_scan_multi_osc_kernel[grid](...)` with EPILOGUE 0 / 1
 * (rqf_models/ops/triton_scan_kernel.py:1991-2015 and its abs and real-input
 * twins, :2019-2087, :2688-2760), and, with cw NULL and N = 1, the fused |y|
 * scan of `sequential_scan_abs` (rqf_models/ops/scan.py:381-432).
 * out: (B,T,F) complex, or real |y| when out_abs != 0. */
int rqf_multi_osc_fwd(const float *c1, const float *c2, const float *cw, const float *u,
                      int32_t u_real, float *out, int32_t out_abs, int64_t B, int64_t T,
                      int64_t F, int64_t N, void *workspace, size_t workspace_bytes,
                      rqf_stream_t stream);

/* Replaces `_sequential_scan_multi_osc_backward_kernel[grid](...)` and its
 * real-input twin (rqf_models/ops/triton_scan_kernel.py:2370-2404, :2880):
 *   d_n[t] = conj(C1_n) d_n[t+1] + conj(cw_n) grad_out[t]
 *   grad_u = sum_n conj(C2_n) d_n (real part for real u),
 *   grad_c1_n = sum d_n[t] conj(x_n[t-1]), grad_c2_n = sum d_n conj(u),
 *   grad_cw_n = sum grad_out conj(x_n)   (each (F*N,) complex, overwritten).
 * Any of grad_u / grad_c1 / grad_c2 / grad_cw may be NULL (not computed). */
int rqf_multi_osc_bwd(const float *c1, const float *c2, const float *cw, const float *u,
                      int32_t u_real, const float *grad_out, float *grad_u, float *grad_c1,
                      float *grad_c2, float *grad_cw, int64_t B, int64_t T, int64_t F,
                      int64_t N, void *workspace, size_t workspace_bytes,
                      rqf_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Two-tap prospective scans in channel-outermost FBT layout.               *
 *   raw[t] = C1*raw[t-1] + tap0*z[t] + tap1*z[t-1]                          *
 *   act    = relu(Re raw) + i relu(Im raw)                                  *
 * ------------------------------------------------------------------------ */

/* Rows x NC entry states kept by the recompute variant (NC for a given T). */
int64_t rqf_fbt_carry_chunks(int64_t T);
size_t rqf_fbt_workspace(int64_t F, int64_t B, int64_t T);

/* Replaces `_fbt_prospective_kernel[grid](...)`
 * (rqf_models/ops/fbt_scan_kernel.py:269-282).  act may be NULL. */
int rqf_fbt_prospective_fwd(const float *c1, const float *tap0, const float *tap1,
                            const float *z, float *raw, float *act, int64_t F, int64_t B,
                            int64_t T, rqf_stream_t stream);

/* Replaces `_fbt_prospective_backward_kernel[grid](...)`
 * (rqf_models/ops/fbt_scan_kernel.py:307-324).  With fuse_act the cotangent is
 * on the split-ReLU output (mask from raw > 0). */
int rqf_fbt_prospective_bwd(const float *c1, const float *tap0, const float *tap1,
                            const float *z, const float *raw, const float *grad_out,
                            int32_t fuse_act, float *grad_z, float *grad_c1,
                            float *grad_tap0, float *grad_tap1, int64_t F, int64_t B,
                            int64_t T, void *workspace, size_t workspace_bytes,
                            rqf_stream_t stream);

/* Replaces `_fbt_recompute_forward_kernel[grid](...)`
 * (rqf_models/ops/fbt_scan_kernel.py:618-631).  Writes the split-ReLU output
 * and carry: (F*B, rqf_fbt_carry_chunks(T)) complex entry states. */
int rqf_fbt_recompute_fwd(const float *c1, const float *tap0, const float *tap1,
                          const float *z, float *act, float *carry, int64_t F, int64_t B,
                          int64_t T, rqf_stream_t stream);

/* rqf_fbt_recompute_fwd with the encoder's residual connection fused into the
 * output store: act = split-ReLU(raw) + skip, skip (F,B,T) complex (the
 * layer input).  Replaces the block call plus the separate skip add of
 * `PureRQFEncoder._forward_fbt_stack` (rqf_models/backbones/rqf/pure.py:
 * 530-534).  The carries are the scan's own states, so
 * rqf_fbt_recompute_bwd applies unchanged (the skip's gradient is the
 * identity). */
int rqf_fbt_recompute_skip_fwd(const float *c1, const float *tap0, const float *tap1,
                               const float *z, const float *skip, float *act, float *carry,
                               int64_t F, int64_t B, int64_t T, rqf_stream_t stream);

/* Layer 0 on a real input of one feature per step (the raw waveform): the
 * recompute scan with its drive formed on the fly, z[f,b,t] = wz[f] x[b,t],
 * from x real (B, T) and wz complex (F,), instead of read from a
 * materialised (F,B,T) drive.  Replaces the stacked real GEMM plus
 * `_fbt_recompute_planar_forward_kernel` of `_Layer0RealScan.forward`
 * (rqf_models/ops/fbt_scan_kernel.py:692-761, 939-972) for D = 1.  Same
 * outputs as rqf_fbt_recompute_fwd on z = wz x. */
int rqf_fbt_layer0_fwd(const float *c1, const float *tap0, const float *tap1, const float *wz,
                       const float *x, float *act, float *carry, int64_t F, int64_t B, int64_t T,
                       rqf_stream_t stream);

/* The backward of rqf_fbt_layer0_fwd: replays the scan from the carries with
 * the drive formed from x, and writes grad_z (F,B,T) complex and the
 * coefficient gradients, as rqf_fbt_recompute_bwd on z = wz x.  Replaces
 * `_fbt_recompute_planar_backward_kernel` (fbt_scan_kernel.py:764-896);
 * grad_z feeds rqf_layer0_grads.  Workspace: rqf_fbt_workspace(F, B, T). */
int rqf_fbt_layer0_bwd(const float *c1, const float *tap0, const float *tap1, const float *wz,
                       const float *x, const float *carry, const float *grad_out, float *grad_z,
                       float *grad_c1, float *grad_tap0, float *grad_tap1, int64_t F, int64_t B,
                       int64_t T, void *workspace, size_t workspace_bytes, rqf_stream_t stream);

/* Replaces `_fbt_recompute_backward_kernel[grid](...)`
 * (rqf_models/ops/fbt_scan_kernel.py:653-669). */
int rqf_fbt_recompute_bwd(const float *c1, const float *tap0, const float *tap1,
                          const float *z, const float *carry, const float *grad_out,
                          float *grad_z, float *grad_c1, float *grad_tap0, float *grad_tap1,
                          int64_t F, int64_t B, int64_t T, void *workspace,
                          size_t workspace_bytes, rqf_stream_t stream);

/* rqf_fbt_recompute_bwd without a workspace argument and without allocating.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The per-row partial sums live in a static device
 * array of RQF_NOALLOC_SCRATCH_BYTES per GPU (4 MiB: F*B <= 87381 rows), held
 * until the process ends; larger problems return RQF_ERR_SCRATCH before any
 * launch.  The first call on a device looks the array's address up (once per
 * device).  All calls on one GPU share that array: calls that overlap on one
 * GPU (concurrent streams or threads) race and must be serialised by the
 * caller.  Results equal rqf_fbt_recompute_bwd's bit for bit. */
int rqf_fbt_recompute_bwd_noalloc(const float *c1, const float *tap0, const float *tap1,
                                  const float *z, const float *carry, const float *grad_out,
                                  float *grad_z, float *grad_c1, float *grad_tap0,
                                  float *grad_tap1, int64_t F, int64_t B, int64_t T,
                                  rqf_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Selective fused scan (FBT layout).                                        *
 * ------------------------------------------------------------------------ */

/* Mirrors `SelectiveScanInputs` (rqf_models/ops/selective_scan.py:10-23)
 * with its options tuple unpacked in the order of
 * rqf_models/backbones/rqf/selective.py:249-262. */
typedef struct rqf_selective_inputs {
  int64_t F, B, T; /* channels, batch, time */
  int64_t G;       /* rows of warp_logits (0 without a frequency warp) */
  const float *gamma_logits; /* (F,B,T) f32, or NULL without gamma control */
  const float *warp_logits;  /* (G,B,T) f32, or NULL */
  const float *write_logits; /* (F,B,T) f32, or NULL */
  const float *bias, *theta, *minimum, *span, *step, *horizon, *theta_minimum,
      *theta_maximum;        /* (F,) f32 */
  const int64_t *groups;     /* (F,) warp group of each channel, each in [0, G), or NULL.
                              * Out-of-range entries are clamped into [0, G) on the device
                              * (no out-of-bounds access; the results are then those of the
                              * clamped groups): validate on the host. */
  int32_t has_gamma, has_warp, has_write, log_shift;
  float gamma_scale, warp_scale;
  int32_t prospective, gamma_horizon, write_sigmoid;
  float write_max, write_bias;
  int32_t bound_warp;
  /* Optional (F,) order in which the forward visits the channels, a
   * permutation of 0..F-1 that keeps each warp group's channels adjacent
   * (e.g. a stable argsort of `groups`), so a group's warp-logit rows are
   * shared in L2 while its channels stream.  NULL visits 0..F-1.  No
   * reference counterpart: it only changes the schedule, not the results. */
  const int32_t *order;
} rqf_selective_inputs;

/* Replaces `_forward[(f*b,)](...)` in `selective_forward`
 * (rqf_models/ops/selective_scan_kernel.py:497-513).
 * z: (F,B,T) complex drive.  raw / act: (F,B,T) complex or NULL (not both).
 * entries: (F*B, ceil(T/chunk)) complex, the state entering each chunk.
 * chunk: positive power of two. */
int rqf_selective_fwd(const rqf_selective_inputs *in, const float *z, int64_t chunk,
                      float *raw, float *act, float *entries, rqf_stream_t stream);

/* rqf_selective_fwd with the encoder's residual connection fused into the
 * output stores: raw = state + skip and act = split-ReLU(state) + skip, skip
 * (F,B,T) complex (the layer input).  Replaces the block call plus the two
 * skip adds `source = raw + h`, `h = out + h` of
 * `PureRQFEncoder._forward_selective_stack`
 * (rqf_models/backbones/rqf/pure.py:486-496).  entries hold the scan's own
 * states, so rqf_selective_bwd applies unchanged (the skip's gradient is the
 * identity). */
int rqf_selective_skip_fwd(const rqf_selective_inputs *in, const float *z, int64_t chunk,
                           const float *skip, float *raw, float *act, float *entries,
                           rqf_stream_t stream);

size_t rqf_selective_bwd_workspace(const rqf_selective_inputs *in, int64_t chunk);

/* Replaces `_backward[(f*b,)](...)`, `_group_reduce[...]` and the fp64 partial
 * sum of `selective_backward` (rqf_models/ops/selective_scan_kernel.py:530-560).
 * gy (cotangent of raw) and gx (of act) are (F,B,T) complex or NULL.
 * dz, dzw: (F,B,T) complex; pass dzw == dz unless truncated.
 * dg, dw: (F,B,T) f32 (NULL when the head is absent); dd: (G,B,T) f32.
 * dbias, dtheta: (F,) f32. */
int rqf_selective_bwd(const rqf_selective_inputs *in, const float *z, const float *entries,
                      int64_t chunk, const float *gy, const float *gx, int32_t activate,
                      int32_t truncated, float *dz, float *dzw, float *dg, float *dd,
                      float *dw, float *dbias, float *dtheta, void *workspace,
                      size_t workspace_bytes, rqf_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Projection GEMM of a selective layer on MFMA, fp32:                       *
 *   C (M x N) = A (M x K) . B (K x N).                                      *
 * It has no single reference counterpart. With the drive and selector       *
 * weights stacked in A it replaces two reference GEMMs and the copy         *
 * between them:                                                             *
 *   - z = weight @ x (rqf_models/ops/selective_scan.py:117-118);            *
 *   - the logits (weights @ v).split(sizes) over                            *
 *     v = cat(x.real, x.imag) (rqf_models/backbones/rqf/selective.py:205-217). *
 * With their adjoints stacked it computes dx = weight.mH @ dz               *
 * (selective_scan.py:144) plus the selector's weights.T @ grad              *
 * (selective.py:96) in one pass.                                            *
 *   weights: (k_pad, m_pad) fp32, k-major (m contiguous), zero padded;      *
 *            k_pad a multiple of 16, m_pad a multiple of 128.               *
 *   B: b_cplx_rows complex64 rows of n (complex row d is K rows 2d, 2d+1:   *
 *      real and imaginary part), then b_real_rows fp32 rows of n.           *
 *   C: out_cplx_rows complex64 rows (rows 2f, 2f+1 of C), then              *
 *      out_real_rows fp32 rows of n.                                        *
 *   The real rows may take a bias and a ReLU (a Linear + ReLU layer on the  *
 *   stacked [Re; Im] of complex features: the per-timestep readout,         *
 *   train.py:74-136).                                                       *
 * Returns RQF_ERR_ARG when 2*b_cplx_rows + b_real_rows > k_pad or           *
 * 2*out_cplx_rows + out_real_rows > m_pad.                                  *
 * ------------------------------------------------------------------------ */
typedef struct rqf_proj_gemm_args {
  const float *weights;
  int64_t k_pad, m_pad;
  const float *b_cplx;
  int64_t b_cplx_rows;
  const float *b_real;
  int64_t b_real_rows;
  int64_t n;
  float *out_cplx;
  int64_t out_cplx_rows;
  float *out_real;
  int64_t out_real_rows;
  const float *out_real_bias; /* out_real_rows biases added to the real rows, or NULL */
  int64_t out_real_relu;      /* nonzero: max(0, .) on the real rows after the bias */
} rqf_proj_gemm_args;

int rqf_proj_gemm(const rqf_proj_gemm_args *args, rqf_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Gradients of the real-input layer 0's projection z = (Wr + i Wi) h, for  *
 * a narrow input, from grad_z (complex64, F x n) in one pass:              *
 *   grad_h (D x n)          = Re(W^H grad_z) = Wr^T Re(gz) + Wi^T Im(gz)    *
 *   grad_w_stacked (2F x D) = [Re gz; Im gz] h^T                            *
 * with w_stacked the real (2F x D) [Wr; Wi] and h the real (D x n) input.   *
 * Replaces the backward GEMMs of _Layer0RealScan                            *
 * (rqf_models/ops/fbt_scan_kernel.py:993-996).  Either output may be NULL.  *
 * grad_h needs 1 <= D <= 16, grad_w_stacked 1 <= D <= 2 and a workspace of  *
 * rqf_layer0_grads_workspace(F, D, n) bytes (its per-wavefront partials,    *
 * reduced in a fixed order in fp64); wider inputs get RQF_ERR_ARG (use     *
 * rqf_proj_gemm and a library GEMM).  Deterministic.                        *
 * ------------------------------------------------------------------------ */
size_t rqf_layer0_grads_workspace(int64_t F, int64_t D, int64_t n);
int rqf_layer0_grads(const float *w_stacked, const float *grad_z, const float *h, float *grad_h,
                     float *grad_w_stacked, int64_t F, int64_t D, int64_t n, void *workspace,
                     size_t workspace_bytes, rqf_stream_t stream);

/* ------------------------------------------------------------------------ *
 * Self-test of the wave-level scan primitives (no reference counterpart):   *
 * in: 64 lanes x 4 complex (P, s) affine maps; out: inclusive prefix (fwd)  *
 * and suffix (rev) compositions.                                            *
 * ------------------------------------------------------------------------ */
int rqf_selftest_wave_scan(const float *in, float *out_fwd, float *out_rev,
                           rqf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RQF_SCAN_H */
