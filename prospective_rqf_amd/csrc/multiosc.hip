// multiosc.hip -- multi-oscillator time-invariant scans with C-weight
// reduction, and the fused |y| readout, in the (batch, time, filters) API.
//
//   x_n[t] = C1_n x_n[t-1] + C2_n u[t]        n = 0..N-1 oscillators of filter f
//   y[t]   = sum_n cw_n x_n[t]                (no cw: y = x_0, N = 1)
//   out    = y  or  |y|
//
// The reference's fused multi-oscillator family
// (rqf_models/ops/triton_scan_kernel.py:1826-2019 forward, :2089-2279
// backward, :2688-3071 real-input variants) and its single-oscillator |y|
// readout (scan.py:381-432) compute these with one program per (batch,
// filter) walking all T steps serially.
//
// Here a task is (batch, time segment, filter) with the filter fastest, so a
// wavefront reads 64 consecutive inputs per step.  A task keeps the filter's
// NP oscillators (N padded to a power of two; padded oscillators have zero
// coefficients) in registers over its segment.  Segments are joined by a
// carry pass per (batch, oscillator, filter) over the segments (three-phase
// scan).
//
// The scanned state is w_n = x_n / C2_n, i.e. w_n[t] = C1_n w_n[t-1] + u[t],
// with C2_n applied at the output: y = sum_n (cw_n C2_n) w_n.  No division
// happens; C2 = 0 is fine.
//
// Backward.  The adjoint e_n[t] = conj(C1_n) e_n[t+1] + grad_out[t] runs as a
// reverse three-phase scan (local pass, carry, final pass); grad_u is
// sum_n conj(cw_n C2_n) e_n.  The reference's coefficient sums pair the
// adjoint at t with the state at t-1, which a reverse sweep does not have.
// Exchanging the order of summation pairs them with u instead
// (mosc_coef_stage2_kernel): against e_n for grad_C2 and grad_cw, and against
// f_n, the derivative of e_n's recurrence with respect to conj(C1_n), for
// grad_C1.  f_n is itself a reverse recurrence, f_n[t] = conj(C1_n) f_n[t+1] +
// e_n[t+1], carried between segments with e_n.  So the final pass reads
// grad_out and u once and produces grad_u and all three sums, with no forward
// state, no checkpoints and no per-step state tensor (the reference keeps
// every state in a (B*F, T, N) scratch tensor).
//
// Coefficient gradients are reduced deterministically: per-task fp32 partial
// sums over at most kMoscMaxSeg steps, then an ordered fp64 reduction per
// oscillator.
#include "rqf_device.h"
#include "rqf_scan.h"

#include <algorithm>

using namespace rqf;

namespace {

constexpr int kMoscMaxOsc = 8;     // oscillators per filter (N <= 8)
// Steps per segment, at most.  Config 6 fwd+bwd: 74.2 Gelem/s at 256 (about 4
// wavefronts per SIMD), 76.7 at 128, 72.3 at 64 (longer carry chains, more
// segment states).
#ifndef RQF_MOSC_MAX_SEG
#define RQF_MOSC_MAX_SEG 128
#endif
constexpr int kMoscMaxSeg = RQF_MOSC_MAX_SEG;
constexpr int kMoscMinSeg = 16;    // steps per segment, at least (when T allows)
constexpr int64_t kMoscLanes = 65536;  // target number of tasks
// Steps per streamed chunk (see stream_steps).  Config 6 (B=32 T=16000 F=128,
// N=4) fwd+bwd on one MI355X: 70.1 Gelem/s with one load in flight per wave,
// 71.6 with 8-step chunks, 71.0 with 16, 69.8 with 32 for the local passes
// (the final passes' 16-step chunks reach 153 VGPRs).
#ifndef RQF_MOSC_STREAM
#define RQF_MOSC_STREAM 8
#endif
#ifndef RQF_MOSC_STREAM_FINAL
#define RQF_MOSC_STREAM_FINAL 8
#endif
constexpr int kStream = RQF_MOSC_STREAM;
constexpr int kStreamFinal = RQF_MOSC_STREAM_FINAL;

__device__ __forceinline__ c32 ldc(const float* p, int64_t i) { return mk(p[2 * i], p[2 * i + 1]); }
__device__ __forceinline__ void stc(float* p, int64_t i, c32 v) {
  p[2 * i] = v.r;
  p[2 * i + 1] = v.i;
}

struct MoscShape {
  int64_t B, T, F, S, L, tasks;
  int N;
};

template <bool REAL>
__device__ __forceinline__ c32 load_u(const float* __restrict__ u, int64_t e) {
  return REAL ? mk(u[e], 0.0f) : ldc(u, e);
}

// Coefficients of the filter's oscillators (index f*N + n; zero when n >= N).
template <int NP>
__device__ __forceinline__ void load_osc(const float* __restrict__ p, int64_t f, int N,
                                         c32 (&v)[NP]) {
#pragma unroll
  for (int n = 0; n < NP; ++n) v[n] = n < N ? ldc(p, f * N + n) : mk(0.0f, 0.0f);
}

struct Task {
  int64_t b, s, f, tb, te;
};
__device__ __forceinline__ Task task_of(const MoscShape& sh, int64_t task) {
  Task k;
  k.f = task % sh.F;
  const int64_t bs = task / sh.F;
  k.s = bs % sh.S;
  k.b = bs / sh.S;
  k.tb = k.s * sh.L;
  k.te = min(sh.T, k.tb + sh.L);
  return k;
}
// Segment states: (b, s, n, f) with f fastest.
__device__ __forceinline__ int64_t seg_idx(const MoscShape& sh, int64_t b, int64_t s, int n,
                                           int64_t f, int NP) {
  return ((b * sh.S + s) * NP + n) * sh.F + f;
}

// One step of the scanned state w_n[t] = C1_n w_n[t-1] + u[t].
template <bool REAL>
__device__ __forceinline__ c32 step_w(c32 a, c32 w, c32 ut) {
  return REAL ? cmadr(a, w, ut.r) : cmad(a, w, ut);
}

// Phase 1 of the forward: each segment's end states from a zero entry.
template <int NP, bool REAL>
__global__ __launch_bounds__(256) void mosc_fwd_local_kernel(const float* __restrict__ c1,
                                                             const float* __restrict__ u,
                                                             float* __restrict__ seg,
                                                             MoscShape sh) {
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], w[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
#pragma unroll
  for (int n = 0; n < NP; ++n) w[n] = mk(0.0f, 0.0f);
  const int64_t base = k.b * sh.T * sh.F + k.f;
  c32 ub[kStream];
  stream_steps<kStream, true>(
      k.tb, k.te, [&](int j, int64_t t) { ub[j] = load_u<REAL>(u, base + t * sh.F); },
      [&](int j, int64_t) {
#pragma unroll
        for (int n = 0; n < NP; ++n) w[n] = step_w<REAL>(a[n], w[n], ub[j]);
      });
#pragma unroll
  for (int n = 0; n < NP; ++n) stc(seg, seg_idx(sh, k.b, k.s, n, k.f, NP), w[n]);
}

// Phase 2: exclusive fold over the segments, in place, per (b, n, f).
//   forward: w_in[s+1] = C1^L w_in[s] + w_end[s]                    (w_in[0] = 0)
//   adjoint: the pair (e, f) entering segment s from its end,
//            e_out[s-1] = P e_out[s] + e_start[s]
//            f_out[s-1] = P f_out[s] + len(s) P' e_out[s] + f_start[s]   (TAN)
//            with P = conj(C1)^len(s), P' = conj(C1)^(len(s)-1), and zero
//            at s = S-1.
// len(s) steps of zero input take (e, f) to (P e, P f + len P' e), by
// induction on the adjoint step (see mosc_bwd_final_kernel).
template <int NP, bool ADJ, bool TAN>
__global__ __launch_bounds__(256) void mosc_carry_kernel(const float* __restrict__ c1,
                                                         float* __restrict__ seg,
                                                         float* __restrict__ segf,
                                                         MoscShape sh) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= sh.B * NP * sh.F) return;
  const int64_t f = id % sh.F, bn = id / sh.F;
  const int n = (int)(bn % NP);
  const int64_t b = bn / NP;
  const c32 a = n < sh.N ? ldc(c1, f * sh.N + n) : mk(0.0f, 0.0f);
  // Powers and the fold in fp64: a float32 power is off by ~L ulp, a bias that
  // every hop of a long-memory channel would repeat.
  // The segments' values are loaded kStream at a time (stream_steps); each
  // is overwritten only after it has been read.
  c64d e = mkd(0.0, 0.0);
  if (!ADJ) {
    const c64d aL = dpow(widen(a), sh.L);
    c32 vb[kStream];
    stream_steps<kStream, true>(
        0, sh.S, [&](int j, int64_t s) { vb[j] = ldc(seg, seg_idx(sh, b, s, n, f, NP)); },
        [&](int j, int64_t s) {
          stc(seg, seg_idx(sh, b, s, n, f, NP), narrow(e));
          e = dmad(aL, e, widen(vb[j]));
        });
  } else {
    const c64d ac = dconj(widen(a));
    const int64_t lenLast = sh.T - (sh.S - 1) * sh.L;
    const c64d p1 = sh.L > 1 ? dpow(ac, sh.L - 1) : mkd(1.0, 0.0);
    const c64d p1Last = lenLast > 1 ? dpow(ac, lenLast - 1) : mkd(1.0, 0.0);
    const c64d p = dmul(p1, ac), pLast = dmul(p1Last, ac);
    const c64d q = mkd(p1.r * (double)sh.L, p1.i * (double)sh.L);
    const c64d qLast = mkd(p1Last.r * (double)lenLast, p1Last.i * (double)lenLast);
    c64d ef = mkd(0.0, 0.0);
    c32 vb[kStream], vfb[kStream];
    stream_steps<kStream, false>(
        0, sh.S,
        [&](int j, int64_t s) {
          const int64_t i = seg_idx(sh, b, s, n, f, NP);
          vb[j] = ldc(seg, i);
          if (TAN) vfb[j] = ldc(segf, i);
        },
        [&](int j, int64_t s) {
          const bool last = s == sh.S - 1;
          const int64_t i = seg_idx(sh, b, s, n, f, NP);
          stc(seg, i, narrow(e));
          if (TAN) {
            stc(segf, i, narrow(ef));
            ef = dmad(last ? pLast : p, ef, dmad(last ? qLast : q, e, widen(vfb[j])));
          }
          e = dmad(last ? pLast : p, e, widen(vb[j]));
        });
  }
}

// Output weights of the scanned state: y = sum_n (cw_n C2_n) w_n, or C2_0 w_0
// without C-weights.
template <int NP, bool CW>
__device__ __forceinline__ void load_out_weights(const float* __restrict__ c2,
                                                 const float* __restrict__ cw, int64_t f, int N,
                                                 c32 (&h)[NP]) {
  load_osc<NP>(c2, f, N, h);
  if (CW) {
    c32 w[NP];
    load_osc<NP>(cw, f, N, w);
#pragma unroll
    for (int n = 0; n < NP; ++n) h[n] = cmul(w[n], h[n]);
  }
}

// Phase 3 of the forward: rescan each segment from its entry state and write
// y = sum_n cw_n C2_n w_n (CW) or C2_0 w_0, as complex or as |y| (ABS).
template <int NP, bool REAL, bool CW, bool ABS>
__global__ __launch_bounds__(256) void mosc_fwd_final_kernel(
    const float* __restrict__ c1, const float* __restrict__ c2, const float* __restrict__ cw,
    const float* __restrict__ u, const float* __restrict__ seg, float* __restrict__ out,
    MoscShape sh) {
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], h[NP], w[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
  load_out_weights<NP, CW>(c2, cw, k.f, sh.N, h);
#pragma unroll
  for (int n = 0; n < NP; ++n) w[n] = ldc(seg, seg_idx(sh, k.b, k.s, n, k.f, NP));
  const int64_t base = k.b * sh.T * sh.F + k.f;
  c32 ub[kStreamFinal];
  stream_steps<kStreamFinal, true>(
      k.tb, k.te, [&](int j, int64_t t) { ub[j] = load_u<REAL>(u, base + t * sh.F); },
      [&](int j, int64_t t) {
        c32 y = mk(0.0f, 0.0f);
#pragma unroll
        for (int n = 0; n < NP; ++n) {
          w[n] = step_w<REAL>(a[n], w[n], ub[j]);
          if (CW || n == 0) y = cmad(h[n], w[n], y);
        }
        const int64_t e = base + t * sh.F;
        if (ABS)
          out[e] = sqrtf(fmaf(y.r, y.r, y.i * y.i));
        else
          stc(out, e, y);
      });
}

// One reverse step of the adjoint pair (see mosc_bwd_final_kernel).
template <bool TAN>
__device__ __forceinline__ void step_adj(c32 a, c32& e, c32& f, c32 gt) {
  if (TAN) f = cjmad(a, f, e);
  e = cjmad(a, e, gt);
}

// Phase 1 of the backward: each segment's adjoint pair at its first step from
// a zero pair after its last step.
template <int NP, bool TAN>
__global__ __launch_bounds__(256) void mosc_bwd_local_kernel(const float* __restrict__ c1,
                                                             const float* __restrict__ gy,
                                                             float* __restrict__ segb,
                                                             float* __restrict__ segf,
                                                             MoscShape sh) {
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], d[NP], f[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
#pragma unroll
  for (int n = 0; n < NP; ++n) d[n] = f[n] = mk(0.0f, 0.0f);
  const int64_t base = k.b * sh.T * sh.F + k.f;
  c32 gb[kStream];
  stream_steps<kStream, false>(
      k.tb, k.te, [&](int j, int64_t t) { gb[j] = ldc(gy, base + t * sh.F); },
      [&](int j, int64_t) {
#pragma unroll
        for (int n = 0; n < NP; ++n) step_adj<TAN>(a[n], d[n], f[n], gb[j]);
      });
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    const int64_t i = seg_idx(sh, k.b, k.s, n, k.f, NP);
    stc(segb, i, d[n]);
    if (TAN) stc(segf, i, f[n]);
  }
}

// Phase 3 of the backward, from each segment's exit pair, for t descending:
//   f_n[t]    = conj(C1_n) f_n[t+1] + e_n[t+1]                  (TAN)
//   e_n[t]    = conj(C1_n) e_n[t+1] + gy[t]
//   grad_u[t] = sum_n conj(cw_n C2_n) e_n[t]   (GU; real u: its real part)
//   Q_n += e_n[t] conj(u[t]),  R_n += f_n[t] conj(u[t])         (TAN)
// e_n is the reference's adjoint d_n without its conj(cw_n) factor, and
// f_n[t] = sum_{s>t} conj(C1_n)^(s-1-t) e_n[s], the derivative of e_n's
// recurrence with respect to conj(C1_n).  Partial sums go to
// part[(n*4 + j)*tasks + task] (j: Re Q, Im Q, Re R, Im R).
template <int NP, bool REAL, bool TAN, bool GU>
__global__ __launch_bounds__(256) void mosc_bwd_final_kernel(
    const float* __restrict__ c1, const float* __restrict__ c2, const float* __restrict__ cw,
    const float* __restrict__ u, const float* __restrict__ gy, const float* __restrict__ segb,
    const float* __restrict__ segf, float* __restrict__ gu, float* __restrict__ part,
    MoscShape sh) {
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], h[NP], d[NP], f[NP], q[NP], r[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
  if (GU) load_out_weights<NP, true>(c2, cw, k.f, sh.N, h);
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    const int64_t i = seg_idx(sh, k.b, k.s, n, k.f, NP);
    d[n] = ldc(segb, i);
    f[n] = TAN ? ldc(segf, i) : mk(0.0f, 0.0f);
    q[n] = r[n] = mk(0.0f, 0.0f);
  }
  const int64_t base = k.b * sh.T * sh.F + k.f;
  c32 gb[kStreamFinal], ub[kStreamFinal];
  stream_steps<kStreamFinal, false>(
      k.tb, k.te,
      [&](int j, int64_t t) {
        gb[j] = ldc(gy, base + t * sh.F);
        if (TAN) ub[j] = load_u<REAL>(u, base + t * sh.F);
      },
      [&](int j, int64_t t) {
        c32 g = mk(0.0f, 0.0f);
#pragma unroll
        for (int n = 0; n < NP; ++n) {
          step_adj<TAN>(a[n], d[n], f[n], gb[j]);
          if (GU) g = cjmad(h[n], d[n], g);
          if (TAN) {
            if (REAL) {
              q[n] = csmad(ub[j].r, d[n], q[n]);
              r[n] = csmad(ub[j].r, f[n], r[n]);
            } else {
              q[n] = cjmad(ub[j], d[n], q[n]);
              r[n] = cjmad(ub[j], f[n], r[n]);
            }
          }
        }
        if (GU) {
          const int64_t e = base + t * sh.F;
          if (REAL)
            gu[e] = g.r;
          else
            stc(gu, e, g);
        }
      });
  if (TAN) {
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      float* p = part + (int64_t)n * 4 * sh.tasks + task;
      p[0] = q[n].r;
      p[sh.tasks] = q[n].i;
      p[2 * sh.tasks] = r[n].r;
      p[3 * sh.tasks] = r[n].i;
    }
  }
}

// Coefficient-gradient reduction, stage 1: partial sums over a run of task
// rows m in [m0, m1) (m = b*S + s), in fp64, in m order.  Thread i covers
// (nj, f) = (i / F, i % F) of the 4*NP*F sums, so a wavefront reads
// consecutive f of one row; the loads of 16 rows issue together.
__global__ __launch_bounds__(256) void mosc_coef_stage1_kernel(const float* __restrict__ part,
                                                               MoscShape sh, int NP, int64_t run,
                                                               double* __restrict__ s1) {
  const int64_t n_sums = (int64_t)4 * NP * sh.F;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_sums) return;
  const int64_t c = blockIdx.y;
  const int64_t nj = i / sh.F, f = i - nj * sh.F;
  const int64_t M = sh.B * sh.S;
  const int64_t m0 = c * run, m1 = min(M, m0 + run);
  const float* p = part + nj * sh.tasks + f;
  double acc = 0.0;
  for (int64_t m = m0; m < m1; m += 16) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = m + k < m1 ? p[(m + k) * sh.F] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 16; ++k) acc += v[k];
  }
  s1[c * n_sums + i] = acc;
}

// Stage 2: grad_C1, grad_C2, grad_cw of oscillator n of filter f (one
// wavefront per f*N + n) from the stage-1 sums of Q and R (lane l adds chunks
// l, l+64, ..., then a fixed-shape wave sum), then
//   grad_C1 = conj(cw C2) R,   grad_C2 = conj(cw) Q,   grad_cw = conj(C2) Q.
// These are the reference's sums, with x_n = C2_n w_n and d_n = conj(cw_n) e_n
// and the order of summation exchanged (u[r] enters w_n[t] with C1^(t-r)):
//   sum_t d_n[t] conj(u[t])     = conj(cw_n) sum_t e_n[t] conj(u[t])
//   sum_t gy[t] conj(x_n[t])    = conj(C2_n) sum_r conj(u[r]) sum_{t>=r} conj(C1)^(t-r) gy[t]
//                               = conj(C2_n) sum_r e_n[r] conj(u[r])
//   sum_t d_n[t] conj(x_n[t-1]) = conj(cw_n C2_n) sum_r conj(u[r]) sum_{t>r} conj(C1)^(t-1-r) e_n[t]
//                               = conj(cw_n C2_n) sum_r f_n[r] conj(u[r]).
__global__ __launch_bounds__(kWave) void mosc_coef_stage2_kernel(
    const double* __restrict__ s1, int64_t chunks, const float* __restrict__ c2,
    const float* __restrict__ cw, MoscShape sh, int NP, float* __restrict__ gc1,
    float* __restrict__ gc2, float* __restrict__ gcw) {
  const int64_t fn = blockIdx.x;  // f*N + n: one wavefront each
  const int64_t f = fn / sh.N;
  const int n = (int)(fn - f * sh.N);
  const int lane = threadIdx.x;
  const int64_t n_sums = (int64_t)4 * NP * sh.F;
  double s[4] = {0, 0, 0, 0};
  for (int64_t c = lane; c < chunks; c += kWave) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] += s1[c * n_sums + ((int64_t)n * 4 + j) * sh.F + f];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) s[j] = wave_sum(s[j]);
  if (lane == 0) {
    const c64d q = mkd(s[0], s[1]), r = mkd(s[2], s[3]);
    const c64d g2 = dconj(widen(ldc(c2, fn))), gw = dconj(widen(ldc(cw, fn)));
    if (gc1) stc(gc1, fn, narrow(dmul(dmul(gw, g2), r)));
    if (gc2) stc(gc2, fn, narrow(dmul(gw, q)));
    if (gcw) stc(gcw, fn, narrow(dmul(g2, q)));
  }
}

inline size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }
inline bool aligned8(const void* p) { return p == nullptr || ((uintptr_t)p & 7) == 0; }
inline bool aligned4(const void* p) { return p == nullptr || ((uintptr_t)p & 3) == 0; }

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RQF_OK : (int)err;
}

int pad_osc(int N) {
  int np = 1;
  while (np < N) np <<= 1;
  return np;
}

MoscShape mosc_shape(int64_t B, int64_t T, int64_t F, int N) {
  MoscShape sh;
  sh.B = B;
  sh.T = T;
  sh.F = F;
  sh.N = N;
  const int64_t lanes = std::max<int64_t>(B * F, 1);
  int64_t S = (kMoscLanes + lanes - 1) / lanes;
  S = std::min<int64_t>(S, std::max<int64_t>(T / kMoscMinSeg, 1));
  S = std::max<int64_t>(S, (T + kMoscMaxSeg - 1) / kMoscMaxSeg);
  S = std::max<int64_t>(S, 1);
  sh.L = T > 0 ? (T + S - 1) / S : 1;
  sh.S = T > 0 ? (T + sh.L - 1) / sh.L : 1;
  sh.tasks = B * sh.S * F;
  return sh;
}

// Segment states of one kind: (b, s, n, f) complex.
size_t mosc_states(const MoscShape& sh) {
  return round256((size_t)(sh.B * sh.S * pad_osc(sh.N) * sh.F) * 8);
}

// Workspace: forward, the w entries; backward, the adjoint pair's entries and
// the per-task partial sums.
struct MoscWs {
  size_t seg, segf, part, s1, total;
};
// Rows of task partials per stage-1 chunk of the coefficient reduction, and
// the number of chunks.
constexpr int64_t kCoefRun = 16;
int64_t coef_run(const MoscShape&) { return kCoefRun; }
int64_t coef_chunks(const MoscShape& sh) {
  return std::max<int64_t>((sh.B * sh.S + coef_run(sh) - 1) / coef_run(sh), 1);
}
MoscWs mosc_ws(const MoscShape& sh, bool backward) {
  const size_t states = mosc_states(sh);
  MoscWs w;
  w.seg = 0;
  if (!backward) {
    w.segf = w.part = w.s1 = w.total = states;
    return w;
  }
  w.segf = states;
  w.part = 2 * states;
  w.s1 = w.part + round256((size_t)sh.tasks * pad_osc(sh.N) * 4 * 4);
  w.total = w.s1 + round256((size_t)coef_chunks(sh) * 4 * pad_osc(sh.N) * sh.F * 8);
  return w;
}

template <class Fn>
int with_np(int N, Fn&& fn) {
  switch (pad_osc(N)) {
    case 1: fn(std::integral_constant<int, 1>{}); return RQF_OK;
    case 2: fn(std::integral_constant<int, 2>{}); return RQF_OK;
    case 4: fn(std::integral_constant<int, 4>{}); return RQF_OK;
    case 8: fn(std::integral_constant<int, 8>{}); return RQF_OK;
    default: return RQF_ERR_ARG;
  }
}

bool bad_shape(int64_t B, int64_t T, int64_t F, int64_t N) {
  return B < 0 || T < 0 || F < 0 || N < 1 || N > kMoscMaxOsc;
}

// Phases 1-3 of the backward, for the gradients requested (tan: the
// coefficient sums; gu: grad_u).
template <int NP, bool REAL, bool TAN, bool GU>
void launch_bwd(const float* c1, const float* c2, const float* cw, const float* u,
                const float* gy, float* segb, float* segf, float* gu, float* part,
                const MoscShape& sh, hipStream_t s) {
  const dim3 block(256), grid((unsigned)((sh.tasks + 255) / 256));
  const dim3 cgrid((unsigned)((sh.B * NP * sh.F + 255) / 256));
  hipLaunchKernelGGL((mosc_bwd_local_kernel<NP, TAN>), grid, block, 0, s, c1, gy, segb, segf, sh);
  hipLaunchKernelGGL((mosc_carry_kernel<NP, true, TAN>), cgrid, block, 0, s, c1, segb, segf, sh);
  hipLaunchKernelGGL((mosc_bwd_final_kernel<NP, REAL, TAN, GU>), grid, block, 0, s, c1, c2, cw,
                     u, gy, segb, segf, gu, part, sh);
}

}  // namespace

// ------------------------------- C ABI ------------------------------------

extern "C" size_t rqf_multi_osc_workspace(int64_t B, int64_t T, int64_t F, int64_t N,
                                          int32_t backward) {
  if (bad_shape(B, T, F, N)) return 0;
  return mosc_ws(mosc_shape(B, T, F, (int)N), backward != 0).total;
}

extern "C" int rqf_multi_osc_fwd(const float* c1, const float* c2, const float* cw,
                                 const float* u, int32_t u_real, float* out, int32_t out_abs,
                                 int64_t B, int64_t T, int64_t F, int64_t N, void* workspace,
                                 size_t workspace_bytes, rqf_stream_t stream) {
  if (bad_shape(B, T, F, N) || (!cw && N != 1)) return RQF_ERR_ARG;
  if (B * T * F == 0) return RQF_OK;
  if (!c1 || !c2 || !u || !out) return RQF_ERR_ARG;
  if (!aligned8(c1) || !aligned8(c2) || !aligned8(cw) || !(u_real ? aligned4(u) : aligned8(u)) ||
      !(out_abs ? aligned4(out) : aligned8(out)))
    return RQF_ERR_ALIGN;
  const MoscShape sh = mosc_shape(B, T, F, (int)N);
  const MoscWs w = mosc_ws(sh, false);
  if (!workspace || workspace_bytes < w.total) return RQF_ERR_WORKSPACE;
  float* seg = (float*)((char*)workspace + w.seg);
  hipStream_t s = (hipStream_t)stream;
  const dim3 block(256), grid((unsigned)((sh.tasks + 255) / 256));
  const int64_t carriers = B * pad_osc((int)N) * F;
  const dim3 cgrid((unsigned)((carriers + 255) / 256));
  const int rc = with_np((int)N, [&](auto npc) {
    constexpr int NP = decltype(npc)::value;
    if (u_real)
      hipLaunchKernelGGL((mosc_fwd_local_kernel<NP, true>), grid, block, 0, s, c1, u, seg, sh);
    else
      hipLaunchKernelGGL((mosc_fwd_local_kernel<NP, false>), grid, block, 0, s, c1, u, seg, sh);
    hipLaunchKernelGGL((mosc_carry_kernel<NP, false, false>), cgrid, block, 0, s, c1, seg,
                       nullptr, sh);
    const bool has_cw = cw != nullptr;
    if (u_real) {
      if (has_cw && out_abs)
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, true, true, true>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
      else if (has_cw)
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, true, true, false>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
      else if (out_abs)
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, true, false, true>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
      else
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, true, false, false>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
    } else {
      if (has_cw && out_abs)
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, false, true, true>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
      else if (has_cw)
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, false, true, false>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
      else if (out_abs)
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, false, false, true>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
      else
        hipLaunchKernelGGL((mosc_fwd_final_kernel<NP, false, false, false>), grid, block, 0, s, c1, c2, cw, u, seg, out, sh);
    }
  });
  return rc ? rc : launch_status();
}

extern "C" int rqf_multi_osc_bwd(const float* c1, const float* c2, const float* cw,
                                 const float* u, int32_t u_real, const float* grad_out,
                                 float* grad_u, float* grad_c1, float* grad_c2, float* grad_cw,
                                 int64_t B, int64_t T, int64_t F, int64_t N, void* workspace,
                                 size_t workspace_bytes, rqf_stream_t stream) {
  if (bad_shape(B, T, F, N) || !cw) return RQF_ERR_ARG;
  if (F == 0) return RQF_OK;
  if (!c1 || !c2) return RQF_ERR_ARG;
  if (B * T > 0 && (!u || !grad_out)) return RQF_ERR_ARG;
  if (!aligned8(c1) || !aligned8(c2) || !aligned8(cw) || !aligned8(grad_out) ||
      !(u_real ? aligned4(u) && aligned4(grad_u) : aligned8(u) && aligned8(grad_u)) ||
      !aligned8(grad_c1) || !aligned8(grad_c2) || !aligned8(grad_cw))
    return RQF_ERR_ALIGN;
  const MoscShape sh = mosc_shape(B, T, F, (int)N);
  const MoscWs w = mosc_ws(sh, true);
  if (w.total && (!workspace || workspace_bytes < w.total)) return RQF_ERR_WORKSPACE;
  char* ws = (char*)workspace;
  float* segb = (float*)(ws + w.seg);
  float* segf = (float*)(ws + w.segf);
  float* part = (float*)(ws + w.part);
  const bool coefs = grad_c1 || grad_c2 || grad_cw;
  hipStream_t s = (hipStream_t)stream;
  const int rc = with_np((int)N, [&](auto npc) {
    constexpr int NP = decltype(npc)::value;
    if (B * T == 0 || (!coefs && !grad_u)) return;
    if (u_real) {
      if (coefs && grad_u)
        launch_bwd<NP, true, true, true>(c1, c2, cw, u, grad_out, segb, segf, grad_u, part, sh, s);
      else if (coefs)
        launch_bwd<NP, true, true, false>(c1, c2, cw, u, grad_out, segb, segf, grad_u, part, sh, s);
      else
        launch_bwd<NP, true, false, true>(c1, c2, cw, u, grad_out, segb, segf, grad_u, part, sh, s);
    } else {
      if (coefs && grad_u)
        launch_bwd<NP, false, true, true>(c1, c2, cw, u, grad_out, segb, segf, grad_u, part, sh, s);
      else if (coefs)
        launch_bwd<NP, false, true, false>(c1, c2, cw, u, grad_out, segb, segf, grad_u, part, sh, s);
      else
        launch_bwd<NP, false, false, true>(c1, c2, cw, u, grad_out, segb, segf, grad_u, part, sh, s);
    }
  });
  if (rc) return rc;
  if (coefs) {
    MoscShape rs = sh;
    if (B * T == 0) {
      rs.B = 0;  // no partial rows: the reduction writes zeros
      rs.S = 0;
    }
    const int NP = pad_osc((int)N);
    const int64_t chunks = coef_chunks(sh), n_sums = (int64_t)4 * NP * F;
    double* s1 = (double*)(ws + w.s1);
    hipLaunchKernelGGL(mosc_coef_stage1_kernel,
                       dim3((unsigned)((n_sums + 255) / 256), (unsigned)chunks), dim3(256), 0, s,
                       part, rs, NP, coef_run(sh), s1);
    hipLaunchKernelGGL(mosc_coef_stage2_kernel, dim3((unsigned)(F * N)), dim3(kWave), 0, s, s1,
                       chunks, c2, cw, rs, NP, grad_c1, grad_c2, grad_cw);
  }
  return launch_status();
}
