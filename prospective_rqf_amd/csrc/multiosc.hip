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
// scan).  The backward runs the adjoint the same way.  For the coefficient
// gradients, which pair the adjoint at t with the state at t-1, it writes
// checkpoints of the forward state every LC steps during a forward sweep of
// the segment, then walks the segment's LC-step chunks backwards, recomputing
// each chunk's states into registers from its checkpoint.  No division by C1
// and no per-step state tensor are needed.
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
constexpr int kMoscMaxSeg = 256;   // steps per segment, at most
constexpr int kMoscMinSeg = 16;    // steps per segment, at least (when T allows)
constexpr int64_t kMoscLanes = 65536;  // target number of tasks
// Backward register chunk: kMoscChunk / NP steps (at least 2) of all NP
// oscillator states are recomputed into registers per checkpoint.  Config 6
// (N = 4) backward: 1.34 ms with 8, 1.49 with 16, 1.34 with 32 (206 VGPRs
// against 110).
#ifndef RQF_MOSC_CHUNK
#define RQF_MOSC_CHUNK 8
#endif
constexpr int kMoscChunk = RQF_MOSC_CHUNK;

__device__ __forceinline__ c32 ldc(const float* p, int64_t i) { return mk(p[2 * i], p[2 * i + 1]); }
__device__ __forceinline__ void stc(float* p, int64_t i, c32 v) {
  p[2 * i] = v.r;
  p[2 * i + 1] = v.i;
}

struct MoscShape {
  int64_t B, T, F, S, L, tasks;
  int N, LC, NCH;
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

// Phase 1 of the forward: each segment's end states from a zero entry.
template <int NP, bool REAL>
__global__ __launch_bounds__(256) void mosc_fwd_local_kernel(const float* __restrict__ c1,
                                                             const float* __restrict__ c2,
                                                             const float* __restrict__ u,
                                                             float* __restrict__ seg,
                                                             MoscShape sh) {
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], g[NP], x[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
  load_osc<NP>(c2, k.f, sh.N, g);
#pragma unroll
  for (int n = 0; n < NP; ++n) x[n] = mk(0.0f, 0.0f);
  const int64_t base = k.b * sh.T * sh.F + k.f;
#pragma unroll 8
  for (int64_t t = k.tb; t < k.te; ++t) {
    const c32 ut = load_u<REAL>(u, base + t * sh.F);
#pragma unroll
    for (int n = 0; n < NP; ++n) x[n] = cmad(a[n], x[n], cmul(g[n], ut));
  }
#pragma unroll
  for (int n = 0; n < NP; ++n) stc(seg, seg_idx(sh, k.b, k.s, n, k.f, NP), x[n]);
}

// Phase 2: exclusive fold over the segments, in place, per (b, n, f).
//   forward: entry[s+1] = C1^L entry[s] + end[s]                (entry[0] = 0)
//   adjoint: exit[s-1] = conj(C1)^len(s) exit[s] + start[s]     (exit[S-1] = 0)
// where exit[s] is the adjoint entering segment s from its end.
template <int NP, bool ADJ>
__global__ __launch_bounds__(256) void mosc_carry_kernel(const float* __restrict__ c1,
                                                         float* __restrict__ seg, MoscShape sh) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= sh.B * NP * sh.F) return;
  const int64_t f = id % sh.F, bn = id / sh.F;
  const int n = (int)(bn % NP);
  const int64_t b = bn / NP;
  const c32 a = n < sh.N ? ldc(c1, f * sh.N + n) : mk(0.0f, 0.0f);
  // Powers and the fold in fp64: a float32 power is off by ~L ulp, a bias that
  // every hop of a long-memory channel would repeat.
  c64d e = mkd(0.0, 0.0);
  if (!ADJ) {
    const c64d aL = dpow(widen(a), sh.L);
    for (int64_t s = 0; s < sh.S; ++s) {
      const int64_t i = seg_idx(sh, b, s, n, f, NP);
      const c32 v = ldc(seg, i);
      stc(seg, i, narrow(e));
      e = dmad(aL, e, widen(v));
    }
  } else {
    const c64d ac = dconj(widen(a));
    const c64d acL = dpow(ac, sh.L);
    const c64d acLast = dpow(ac, sh.T - (sh.S - 1) * sh.L);
    for (int64_t s = sh.S - 1; s >= 0; --s) {
      const int64_t i = seg_idx(sh, b, s, n, f, NP);
      const c32 v = ldc(seg, i);
      stc(seg, i, narrow(e));
      e = dmad(s == sh.S - 1 ? acLast : acL, e, widen(v));
    }
  }
}

// Phase 3 of the forward: rescan each segment from its entry state and write
// y = sum_n cw_n x_n (CW) or x_0, as complex or as |y| (ABS).
template <int NP, bool REAL, bool CW, bool ABS>
__global__ __launch_bounds__(256) void mosc_fwd_final_kernel(
    const float* __restrict__ c1, const float* __restrict__ c2, const float* __restrict__ cw,
    const float* __restrict__ u, const float* __restrict__ seg, float* __restrict__ out,
    MoscShape sh) {
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], g[NP], w[NP], x[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
  load_osc<NP>(c2, k.f, sh.N, g);
  if (CW) load_osc<NP>(cw, k.f, sh.N, w);
#pragma unroll
  for (int n = 0; n < NP; ++n) x[n] = ldc(seg, seg_idx(sh, k.b, k.s, n, k.f, NP));
  const int64_t base = k.b * sh.T * sh.F + k.f;
#pragma unroll 8
  for (int64_t t = k.tb; t < k.te; ++t) {
    const int64_t e = base + t * sh.F;
    const c32 ut = load_u<REAL>(u, e);
    c32 y = mk(0.0f, 0.0f);
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      x[n] = cmad(a[n], x[n], cmul(g[n], ut));
      y = CW ? cmad(w[n], x[n], y) : (n == 0 ? x[0] : y);
    }
    if (ABS)
      out[e] = sqrtf(fmaf(y.r, y.r, y.i * y.i));
    else
      stc(out, e, y);
  }
}

// Phase 1 of the backward: each segment's adjoint at its first step from a
// zero adjoint after its last step; the scan input is conj(cw_n) gy[t].
template <int NP>
__global__ __launch_bounds__(256) void mosc_bwd_local_kernel(const float* __restrict__ c1,
                                                             const float* __restrict__ cw,
                                                             const float* __restrict__ gy,
                                                             float* __restrict__ segb,
                                                             MoscShape sh) {
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], w[NP], d[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
  load_osc<NP>(cw, k.f, sh.N, w);
#pragma unroll
  for (int n = 0; n < NP; ++n) d[n] = mk(0.0f, 0.0f);
  const int64_t base = k.b * sh.T * sh.F + k.f;
#pragma unroll 8
  for (int64_t t = k.te - 1; t >= k.tb; --t) {
    const c32 gt = ldc(gy, base + t * sh.F);
#pragma unroll
    for (int n = 0; n < NP; ++n) d[n] = cjmad(a[n], d[n], cjmul(w[n], gt));
  }
#pragma unroll
  for (int n = 0; n < NP; ++n) stc(segb, seg_idx(sh, k.b, k.s, n, k.f, NP), d[n]);
}

// Phase 3 of the backward.  Per task: forward sweep writing a checkpoint of
// the states every LC steps; then the chunks in reverse, each recomputing its
// LC states into registers and running the adjoint over them:
//   d_n[t]     = conj(C1_n) d_n[t+1] + conj(cw_n) gy[t]
//   grad_u[t]  = sum_n conj(C2_n) d_n[t]          (real u: its real part)
//   grad_C1_n += d_n[t] conj(x_n[t-1]),  grad_C2_n += d_n[t] conj(u[t]),
//   grad_cw_n += gy[t] conj(x_n[t])
// Partial sums per task go to part[(n*6 + j)*tasks + task].
template <int NP, bool REAL>
__global__ __launch_bounds__(256) void mosc_bwd_final_kernel(
    const float* __restrict__ c1, const float* __restrict__ c2, const float* __restrict__ cw,
    const float* __restrict__ u, const float* __restrict__ gy, const float* __restrict__ seg,
    const float* __restrict__ segb, float* __restrict__ ckpt, float* __restrict__ gu,
    float* __restrict__ part, MoscShape sh) {
  constexpr int LC = kMoscChunk / NP > 2 ? kMoscChunk / NP : 2;
  const int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (task >= sh.tasks) return;
  const Task k = task_of(sh, task);
  c32 a[NP], g[NP], w[NP], x[NP], d[NP];
  load_osc<NP>(c1, k.f, sh.N, a);
  load_osc<NP>(c2, k.f, sh.N, g);
  load_osc<NP>(cw, k.f, sh.N, w);
  const int64_t base = k.b * sh.T * sh.F + k.f;
  // Forward sweep: checkpoint the state entering every chunk.
#pragma unroll
  for (int n = 0; n < NP; ++n) x[n] = ldc(seg, seg_idx(sh, k.b, k.s, n, k.f, NP));
  const int nch = (int)((k.te - k.tb + LC - 1) / LC);
  for (int c = 0; c < nch; ++c) {
#pragma unroll
    for (int n = 0; n < NP; ++n) stc(ckpt, ((int64_t)c * NP + n) * sh.tasks + task, x[n]);
    if (c + 1 == nch) break;
    const int64_t t0 = k.tb + (int64_t)c * LC;
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      const c32 ut = load_u<REAL>(u, base + (t0 + j) * sh.F);
#pragma unroll
      for (int n = 0; n < NP; ++n) x[n] = cmad(a[n], x[n], cmul(g[n], ut));
    }
  }
  // Reverse over the chunks.
#pragma unroll
  for (int n = 0; n < NP; ++n) d[n] = ldc(segb, seg_idx(sh, k.b, k.s, n, k.f, NP));
  float acc[NP][6];
#pragma unroll
  for (int n = 0; n < NP; ++n)
#pragma unroll
    for (int j = 0; j < 6; ++j) acc[n][j] = 0.0f;
  for (int c = nch - 1; c >= 0; --c) {
    const int64_t t0 = k.tb + (int64_t)c * LC;
    const int cnt = (int)min<int64_t>(LC, k.te - t0);
    c32 x0[NP], xs[LC][NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) x0[n] = ldc(ckpt, ((int64_t)c * NP + n) * sh.tasks + task);
#pragma unroll
    for (int j = 0; j < LC; ++j) {
      const c32 ut = j < cnt ? load_u<REAL>(u, base + (t0 + j) * sh.F) : mk(0.0f, 0.0f);
#pragma unroll
      for (int n = 0; n < NP; ++n)
        xs[j][n] = cmad(a[n], j ? xs[j - 1][n] : x0[n], cmul(g[n], ut));
    }
#pragma unroll
    for (int j = LC - 1; j >= 0; --j) {
      if (j >= cnt) continue;
      const int64_t e = base + (t0 + j) * sh.F;
      const c32 gt = ldc(gy, e);
      const c32 ut = load_u<REAL>(u, e);  // re-read: cache-resident from the chunk's replay
      c32 gsum = mk(0.0f, 0.0f);
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        d[n] = cjmad(a[n], d[n], cjmul(w[n], gt));
        gsum = cjmad(g[n], d[n], gsum);
        const c32 xp = j ? xs[j - 1][n] : x0[n];
        const c32 s1 = cjmul(xp, d[n]);     // d conj(x[t-1])
        const c32 s2 = cjmul(ut, d[n]);     // d conj(u[t])
        const c32 s3 = cjmul(xs[j][n], gt); // gy conj(x[t])
        acc[n][0] += s1.r;
        acc[n][1] += s1.i;
        acc[n][2] += s2.r;
        acc[n][3] += s2.i;
        acc[n][4] += s3.r;
        acc[n][5] += s3.i;
      }
      if (gu) {
        if (REAL)
          gu[e] = gsum.r;
        else
          stc(gu, e, gsum);
      }
    }
  }
#pragma unroll
  for (int n = 0; n < NP; ++n)
#pragma unroll
    for (int j = 0; j < 6; ++j) part[((int64_t)n * 6 + j) * sh.tasks + task] = acc[n][j];
}

// grad_C1, grad_C2, grad_cw of oscillator n of filter f: one wavefront per
// (f, n < N) sums the B*S task partials in a fixed order in fp64.
__global__ __launch_bounds__(64) void mosc_coef_reduce_kernel(const float* __restrict__ part,
                                                              MoscShape sh, int NP,
                                                              float* __restrict__ gc1,
                                                              float* __restrict__ gc2,
                                                              float* __restrict__ gcw) {
  const int64_t fn = blockIdx.x;  // f*N + n
  const int64_t f = fn / sh.N;
  const int n = (int)(fn - f * sh.N);
  const int lane = threadIdx.x;
  const int64_t M = sh.B * sh.S;
  double s[6] = {0, 0, 0, 0, 0, 0};
  for (int64_t m = lane; m < M; m += kWave) {
#pragma unroll
    for (int j = 0; j < 6; ++j) s[j] += part[((int64_t)n * 6 + j) * sh.tasks + m * sh.F + f];
  }
#pragma unroll
  for (int j = 0; j < 6; ++j) s[j] = wave_sum(s[j]);
  if (lane == 0) {
    if (gc1) {
      gc1[2 * fn] = (float)s[0];
      gc1[2 * fn + 1] = (float)s[1];
    }
    if (gc2) {
      gc2[2 * fn] = (float)s[2];
      gc2[2 * fn + 1] = (float)s[3];
    }
    if (gcw) {
      gcw[2 * fn] = (float)s[4];
      gcw[2 * fn + 1] = (float)s[5];
    }
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
  const int NP = pad_osc(N);
  sh.LC = kMoscChunk / NP > 2 ? kMoscChunk / NP : 2;
  const int64_t lanes = std::max<int64_t>(B * F, 1);
  int64_t S = (kMoscLanes + lanes - 1) / lanes;
  S = std::min<int64_t>(S, std::max<int64_t>(T / kMoscMinSeg, 1));
  S = std::max<int64_t>(S, (T + kMoscMaxSeg - 1) / kMoscMaxSeg);
  S = std::max<int64_t>(S, 1);
  sh.L = T > 0 ? (T + S - 1) / S : 1;
  sh.S = T > 0 ? (T + sh.L - 1) / sh.L : 1;
  sh.tasks = B * sh.S * F;
  sh.NCH = (int)((sh.L + sh.LC - 1) / sh.LC);
  return sh;
}

struct MoscWs {
  size_t seg, segb, ckpt, part, total;
};
MoscWs mosc_ws(const MoscShape& sh, bool backward) {
  const int NP = pad_osc(sh.N);
  const size_t states = (size_t)(sh.B * sh.S * NP * sh.F) * 8;
  MoscWs w;
  size_t off = 0;
  w.seg = off;
  off += round256(states);
  w.segb = off;
  if (backward) off += round256(states);
  w.ckpt = off;
  if (backward) off += round256((size_t)sh.tasks * sh.NCH * NP * 8);
  w.part = off;
  if (backward) off += round256((size_t)sh.tasks * NP * 6 * 4);
  w.total = off;
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
      hipLaunchKernelGGL((mosc_fwd_local_kernel<NP, true>), grid, block, 0, s, c1, c2, u, seg, sh);
    else
      hipLaunchKernelGGL((mosc_fwd_local_kernel<NP, false>), grid, block, 0, s, c1, c2, u, seg, sh);
    hipLaunchKernelGGL((mosc_carry_kernel<NP, false>), cgrid, block, 0, s, c1, seg, sh);
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
  float* seg = (float*)(ws + w.seg);
  float* segb = (float*)(ws + w.segb);
  float* ckpt = (float*)(ws + w.ckpt);
  float* part = (float*)(ws + w.part);
  hipStream_t s = (hipStream_t)stream;
  const dim3 block(256), grid((unsigned)((sh.tasks + 255) / 256));
  const int64_t carriers = B * pad_osc((int)N) * F;
  const dim3 cgrid((unsigned)((carriers + 255) / 256));
  const bool work = B * T > 0;
  const int rc = with_np((int)N, [&](auto npc) {
    constexpr int NP = decltype(npc)::value;
    if (!work) return;
    if (u_real)
      hipLaunchKernelGGL((mosc_fwd_local_kernel<NP, true>), grid, block, 0, s, c1, c2, u, seg, sh);
    else
      hipLaunchKernelGGL((mosc_fwd_local_kernel<NP, false>), grid, block, 0, s, c1, c2, u, seg, sh);
    hipLaunchKernelGGL((mosc_carry_kernel<NP, false>), cgrid, block, 0, s, c1, seg, sh);
    hipLaunchKernelGGL((mosc_bwd_local_kernel<NP>), grid, block, 0, s, c1, cw, grad_out, segb, sh);
    hipLaunchKernelGGL((mosc_carry_kernel<NP, true>), cgrid, block, 0, s, c1, segb, sh);
    if (u_real)
      hipLaunchKernelGGL((mosc_bwd_final_kernel<NP, true>), grid, block, 0, s, c1, c2, cw, u,
                         grad_out, seg, segb, ckpt, grad_u, part, sh);
    else
      hipLaunchKernelGGL((mosc_bwd_final_kernel<NP, false>), grid, block, 0, s, c1, c2, cw, u,
                         grad_out, seg, segb, ckpt, grad_u, part, sh);
  });
  if (rc) return rc;
  MoscShape rs = sh;
  if (!work) {
    rs.B = 0;  // no partial rows: the reduction writes zeros
    rs.S = 0;
  }
  if (grad_c1 || grad_c2 || grad_cw)
    hipLaunchKernelGGL(mosc_coef_reduce_kernel, dim3((unsigned)(F * N)), dim3(kWave), 0, s,
                       part, rs, pad_osc((int)N), grad_c1, grad_c2, grad_cw);
  return launch_status();
}
