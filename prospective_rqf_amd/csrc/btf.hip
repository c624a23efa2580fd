// btf.hip -- single-pass time-invariant scans in the reference's
// (batch, time, filters) layout for gfx950.
//
//   y[t] = c1*y[t-1] + k0*x[t] + k1*x[t-1]      (k1 = 0: the plain C2 scan)
//
// and their adjoint (chunked_scan_kernel.py:60-209, :374-526).
//
// A block owns FC consecutive filters of one batch element and walks the whole
// sequence in passes of NSEG segments of LS steps.  Thread i takes filter
// f0 + i % FC and segment i / FC of the pass, so for each step a wavefront
// touches 64/FC runs of FC consecutive complex values (FC*8 bytes each).  A
// thread loads its segment's inputs once into registers (the next pass's are
// loaded while the current one computes), scans them from a zero state,
// publishes the segment's end state in LDS, and after one barrier folds the
// end states of the pass's earlier segments onto the block's carry, in fp64
// with the exact power c1^LS, to get its entry state.  It then replays the
// segment from the registers and writes the outputs.  The carry past the
// pass's last segment moves to the next pass.  So every input is read once
// and every output written once, and no carry crosses a block: on gfx950 a
// release/acquire between blocks writes back and invalidates the L2.
//
// The adjoint runs the same way in reverse time, carrying the pair (g, h):
// g the adjoint of the state and h its derivative with respect to conj(c1),
// from which grad_c1 follows without the forward states (see
// btf_bwd_kernel).  Coefficient gradients are per-(batch, filter) fp64 partial
// sums, reduced over the batch in a fixed order: deterministic.
#include "rqf_device.h"
#include "rqf_scan.h"

#include <algorithm>

using namespace rqf;

namespace {

// Filters per block (FC * 8-byte runs), threads per block and steps per
// segment of each direction.  Config 2's workload in (B,T,F) layout, measured
// (forward / backward ms): FC 16, 512 threads, 16 steps: 0.241 / 0.361; 32
// steps: 0.216 / 0.879 (the backward then spills); 8 steps: 0.266 / 0.379;
// FC 8: 0.344 / 0.549 (64-byte runs); FC 32: 0.313 / 0.457 (128 blocks);
// 256 threads: 0.257 / 0.370; 1024 threads: 0.238 / 1.19 (spills).
#ifndef RQF_BTF_FC
#define RQF_BTF_FC 16
#endif
#ifndef RQF_BTF_LS_FWD
#define RQF_BTF_LS_FWD 32
#endif
#ifndef RQF_BTF_LS_BWD
#define RQF_BTF_LS_BWD 16
#endif
#ifndef RQF_BTF_THREADS
#define RQF_BTF_THREADS 512
#endif
constexpr int kFC = RQF_BTF_FC;
constexpr int kThreads = RQF_BTF_THREADS;
constexpr int kNSeg = kThreads / kFC;  // segments per pass
constexpr int kWaves = kThreads / kWave;
static_assert(kThreads % kWave == 0 && kWave % kFC == 0, "whole segments per wavefront");

__device__ __forceinline__ c32 ldc(const float* p, int64_t i) {
  const float2 v = *reinterpret_cast<const float2*>(p + 2 * i);
  return mk(v.x, v.y);
}

struct Lane {
  int fl, sg;     // filter lane and segment of the thread
  int64_t f;      // filter
  int64_t b;      // batch element
  bool fv;        // f < F
  int64_t base;   // element (b, 0, f)
};

__device__ __forceinline__ Lane lane_of(int64_t T, int64_t F) {
  Lane l;
  l.fl = (int)threadIdx.x % kFC;
  l.sg = (int)threadIdx.x / kFC;
  const int64_t nfc = (F + kFC - 1) / kFC;
  // The filter groups of one batch element share the cache lines of its
  // (B,T,F) rows: keep them on one XCD.
  const int64_t blk = xcd_contiguous(blockIdx.x, gridDim.x);
  l.b = blk / nfc;
  l.f = (blk % nfc) * kFC + l.fl;
  l.fv = l.f < F;
  l.base = l.b * T * F + (l.fv ? l.f : 0);
  return l;
}

// The thread's segment [tb, tb + LS) of a stream in (B,T,F) layout; zero
// outside [0, T) and for filters past F.
template <int LS>
__device__ __forceinline__ void load_seg(const float* __restrict__ p, const Lane& l, int64_t tb,
                                         int64_t T, int64_t F, c32 (&v)[LS]) {
#pragma unroll
  for (int j = 0; j < LS; ++j) {
    const int64_t t = tb + j;
    v[j] = (l.fv && t < T) ? ldc(p, l.base + t * F) : mk(0.0f, 0.0f);
  }
}

// A pass that lies wholly inside [0, T) is addressed from a wave-uniform
// base per step (scalar arithmetic) plus the lane's fixed offset: one 64-bit
// add per element and no test, where load_seg multiplies and tests each one.
// Config 2's workload on (B,T,F) tensors: the backward's pass loop 1350 ->
// 1112 VALU instructions per lane, forward / backward 0.2222 / 0.3623 ->
// 0.2210 / 0.3595 ms (rotated runs on one box).
//
// Byte offset of step pt of the lane's batch element.  The offset, not the
// pointer, goes through readfirstlane: a pointer rebuilt from integers loses
// its address space and its stores become flat ones.
__device__ __forceinline__ int64_t pass_off(const Lane& l, int64_t pt, int64_t T, int64_t F) {
  return (int64_t)uniform64((uint64_t)((l.b * T + pt) * F * 8));
}
// The lane's byte offset from its pass's base: its segment's first step and
// its filter (filter 0 for a lane past F, whose values are never stored).
__device__ __forceinline__ uint64_t seg_off(const Lane& l, int LS, int64_t F) {
  return (uint64_t)(((int64_t)l.sg * LS * F + (l.fv ? l.f : 0)) * 8);
}
// A whole segment: base pb of the pass, lane offset lo, stp bytes per step.
template <int LS>
__device__ __forceinline__ void load_seg_w(const char* pb, uint64_t lo, uint64_t stp,
                                           c32 (&v)[LS]) {
#pragma unroll
  for (int j = 0; j < LS; ++j) {
    const float2 x = *reinterpret_cast<const float2*>((pb + (uint64_t)j * stp) + lo);
    v[j] = mk(x.x, x.y);
  }
}
__device__ __forceinline__ void st_w(char* pb, uint64_t lo, uint64_t stp, int j, c32 v) {
  *reinterpret_cast<float2*>((pb + (uint64_t)j * stp) + lo) = make_float2(v.r, v.i);
}

__device__ __forceinline__ c32 load_at(const float* __restrict__ p, const Lane& l, int64_t t,
                                       int64_t T, int64_t F) {
  return (l.fv && t >= 0 && t < T) ? ldc(p, l.base + t * F) : mk(0.0f, 0.0f);
}

__device__ __forceinline__ double2 d2(c64d v) { return make_double2(v.r, v.i); }
__device__ __forceinline__ c64d cd(double2 v) { return mkd(v.x, v.y); }

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <bool PROSP, int kLS = RQF_BTF_LS_FWD>
__global__ __launch_bounds__(kThreads) void btf_fwd_kernel(const float* __restrict__ c1,
                                                          const float* __restrict__ k0p,
                                                          const float* __restrict__ k1p,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ out, int64_t T,
                                                          int64_t F) {
  constexpr int kPass = kNSeg * kLS;  // steps per pass
  __shared__ double2 s_tot[2][kWaves][kFC];  // each wavefront's segments, composed
  __shared__ double2 s_carry[2][kFC];
  const Lane l = lane_of(T, F);
  const int lane = lane_id(), w = wave_id(), q = lane / kFC;
  const c32 a = l.fv ? ldc(c1, l.f) : mk(0.0f, 0.0f);
  const c32 k0 = l.fv ? ldc(k0p, l.f) : mk(0.0f, 0.0f);
  const c32 k1 = (PROSP && l.fv) ? ldc(k1p, l.f) : mk(0.0f, 0.0f);
  // a^LS (one segment), a^(q LS) and a^(G LS) (one wavefront's segments)
  const c64d aL = dpow(widen(a), kLS);
  const c64d aLq = dpow(aL, q), aLG = dpow(aL, kWave / kFC);
  if (l.sg == 0) s_carry[0][l.fl] = make_double2(0.0, 0.0);
  const uint64_t lo = seg_off(l, kLS, F);
  const uint64_t stp = uniform64((uint64_t)F * 8);
  const char* const xb = reinterpret_cast<const char*>(x);
  c32 xv[kLS], xn[kLS];
  load_seg(x, l, (int64_t)l.sg * kLS, T, F, xv);
  int p = 0;
  for (int64_t pt = 0; pt < T; pt += kPass) {
    const int64_t tb = pt + (int64_t)l.sg * kLS;
    if (pt + 2 * kPass <= T)
      load_seg_w<kLS>(xb + pass_off(l, pt + kPass, T, F), lo, stp, xn);
    else if (pt + kPass < T)
      load_seg(x, l, tb + kPass, T, F, xn);
    const c32 xm1 = PROSP ? load_at(x, l, tb - 1, T, F) : mk(0.0f, 0.0f);
    // The segment from a zero state.
    c32 y = mk(0.0f, 0.0f), xp = xm1;
#pragma unroll
    for (int j = 0; j < kLS; ++j) {
      const c32 d = PROSP ? cmad(k1, xp, cmul(k0, xv[j])) : cmul(k0, xv[j]);
      y = cmad(a, y, d);
      xp = xv[j];
    }
    // Entry state, in fp64: the wavefront's earlier segments (cross-lane),
    // then the block's carry and the earlier wavefronts (LDS).
    c64d incl;
    const c64d ex = wave_seg_prefix<kFC>(widen(y), aL, lane, incl);
    if (q == kWave / kFC - 1) s_tot[p][w][l.fl] = d2(incl);
    __syncthreads();
    c64d cw = cd(s_carry[p][l.fl]);
    for (int v = 0; v < w; ++v) cw = dmad(aLG, cw, cd(s_tot[p][v][l.fl]));
    const c64d e = dmad(aLq, cw, ex);
    if (w == kWaves - 1 && q == kWave / kFC - 1) s_carry[p ^ 1][l.fl] = d2(dmad(aLG, cw, incl));
    // Replay from the entry state.
    c32 ys = narrow(e);
    xp = xm1;
    const bool whole = pt + kPass <= T;
    char* const ob = reinterpret_cast<char*>(out) + pass_off(l, pt, T, F);
#pragma unroll
    for (int j = 0; j < kLS; ++j) {
      const c32 d = PROSP ? cmad(k1, xp, cmul(k0, xv[j])) : cmul(k0, xv[j]);
      ys = cmad(a, ys, d);
      xp = xv[j];
      if (l.fv && (whole || tb + j < T)) st_w(ob, lo, stp, j, ys);
    }
#pragma unroll
    for (int j = 0; j < kLS; ++j) xv[j] = xn[j];
    p ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Backward.  For t descending:
//   g[t] = conj(c1) g[t+1] + gy[t]              (the adjoint of the drive)
//   h[t] = conj(c1) h[t+1] + g[t+1]
//   grad_x[t] = conj(k0) g[t] + conj(k1) g[t+1]
//   sums: conj(d[t]) h[t] (grad_c1), conj(x[t]) g[t] (k0), conj(x[t-1]) g[t] (k1)
// with the drive d[t] = k0 x[t] + k1 x[t-1].  The reference's grad_c1 is
// sum_t g[t] conj(y[t-1]) over the saved states y; exchanging the order of
// summation (y[t-1] = sum_{r<t} c1^(t-1-r) d[r]) gives sum_r conj(d[r]) h[r],
// since h[r] = sum_{t>r} conj(c1)^(t-1-r) g[t].  So the pass reads gy and x
// only, not the saved states.  LS steps take the pair entering a segment
// (at its end) to (P g + G, P h + LS P' g + H) at its start, P = conj(c1)^LS,
// P' = conj(c1)^(LS-1), (G, H) the segment's own pair from a zero entry.  A
// segment past T has zero cotangents, so every segment is a full one.
// ---------------------------------------------------------------------------
struct Pair {
  double2 g, h;
};

template <bool PROSP, int kLS = RQF_BTF_LS_BWD>
__global__ __launch_bounds__(kThreads) void btf_bwd_kernel(
    const float* __restrict__ c1, const float* __restrict__ k0p, const float* __restrict__ k1p,
    const float* __restrict__ x, const float* __restrict__ gy, float* __restrict__ gx,
    double* __restrict__ partial, int64_t T, int64_t F) {
  constexpr int kPass = kNSeg * kLS;  // steps per pass
  __shared__ Pair s_tot[2][kWaves][kFC];  // each wavefront's segments, composed
  __shared__ Pair s_carry[2][kFC];
  __shared__ double s_red[kWaves][kFC][6];
  const Lane l = lane_of(T, F);
  const int lane = lane_id(), w = wave_id(), q = lane / kFC;
  constexpr int G = kWave / kFC;
  const c32 a = l.fv ? ldc(c1, l.f) : mk(0.0f, 0.0f);
  const c32 ac = conjg(a);
  const c32 k0 = l.fv ? ldc(k0p, l.f) : mk(0.0f, 0.0f);
  const c32 k1 = (PROSP && l.fv) ? ldc(k1p, l.f) : mk(0.0f, 0.0f);
  // Pair map of one segment and of one wavefront's G segments.
  const c64d p1 = kLS > 1 ? dconj(dpow(widen(a), kLS - 1)) : mkd(1.0, 0.0);
  PairMap one;
  one.P = dmul(p1, widen(ac));
  one.c = mkd(p1.r * (double)kLS, p1.i * (double)kLS);
  PairMap wmap = one;
  for (int k = 1; k < G; k <<= 1) wmap = pair_map_mul(wmap, wmap);
  if (l.sg == 0) s_carry[0][l.fl] = Pair{make_double2(0.0, 0.0), make_double2(0.0, 0.0)};
  const int64_t npass = (T + kPass - 1) / kPass;
  const uint64_t lo = seg_off(l, kLS, F);
  const uint64_t stp = uniform64((uint64_t)F * 8);
  const char* const gyb = reinterpret_cast<const char*>(gy);
  const char* const xb = reinterpret_cast<const char*>(x);
  c32 gv[kLS], xv[kLS], gn[kLS], xn[kLS];
  int64_t pt = (npass - 1) * kPass;
  load_seg(gy, l, pt + (int64_t)l.sg * kLS, T, F, gv);
  load_seg(x, l, pt + (int64_t)l.sg * kLS, T, F, xv);
  double s1r = 0, s1i = 0, s0r = 0, s0i = 0, s2r = 0, s2i = 0;
  int p = 0;
  for (; pt >= 0; pt -= kPass) {
    const int64_t tb = pt + (int64_t)l.sg * kLS;
    if (pt > 0) {
      // Every pass before the last lies wholly inside [0, T).
      const int64_t po = pass_off(l, pt - kPass, T, F);
      load_seg_w<kLS>(gyb + po, lo, stp, gn);
      load_seg_w<kLS>(xb + po, lo, stp, xn);
    }
    const c32 xm1 = load_at(x, l, tb - 1, T, F);
    // The segment's pair at its first step from a zero pair after it.
    c32 g = mk(0.0f, 0.0f), h = mk(0.0f, 0.0f);
#pragma unroll
    for (int j = kLS - 1; j >= 0; --j) {
      h = cmad(ac, h, g);
      g = cmad(ac, g, gv[j]);
    }
    // Pair entering the segment, in fp64: the wavefront's later segments
    // (cross-lane), then the block's carry and the later wavefronts (LDS).
    c64d xg, xh, ig, ih;
    PairMap after;
    wave_seg_suffix<kFC>(widen(g), widen(h), one, lane, xg, xh, ig, ih, after);
    if (q == 0) s_tot[p][w][l.fl] = Pair{d2(ig), d2(ih)};
    __syncthreads();
    const Pair cr = s_carry[p][l.fl];
    c64d cg = cd(cr.g), ch = cd(cr.h);
    for (int v = kWaves - 1; v > w; --v) {
      const Pair t = s_tot[p][v][l.fl];
      pair_apply(wmap, cd(t.g), cd(t.h), cg, ch);
    }
    c64d eg = cg, eh = ch;
    pair_apply(after, xg, xh, eg, eh);
    if (w == 0 && q == 0) {
      pair_apply(wmap, ig, ih, cg, ch);
      s_carry[p ^ 1][l.fl] = Pair{d2(cg), d2(ch)};
    }
    // Replay: grad_x and the coefficient sums.
    c32 gnext = narrow(eg), hnext = narrow(eh);
    const bool whole = pt + kPass <= T;
    char* const gxb = reinterpret_cast<char*>(gx) + pass_off(l, pt, T, F);
    float a1r = 0, a1i = 0, a0r = 0, a0i = 0, a2r = 0, a2i = 0;
#pragma unroll
    for (int j = kLS - 1; j >= 0; --j) {
      const c32 hh = cmad(ac, hnext, gnext);
      const c32 gg = cmad(ac, gnext, gv[j]);
      const c32 xp = j ? xv[j - 1] : xm1;
      if (l.fv && (whole || tb + j < T))
        st_w(gxb, lo, stp, j, PROSP ? cjmad(k1, gnext, cjmul(k0, gg)) : cjmul(k0, gg));
      const c32 d = PROSP ? cmad(k1, xp, cmul(k0, xv[j])) : cmul(k0, xv[j]);
      const c32 t1 = cjmul(d, hh), t0 = cjmul(xv[j], gg);
      a1r += t1.r;
      a1i += t1.i;
      a0r += t0.r;
      a0i += t0.i;
      if (PROSP) {
        const c32 t2 = cjmul(xp, gg);
        a2r += t2.r;
        a2i += t2.i;
      }
      gnext = gg;
      hnext = hh;
    }
    s1r += a1r;
    s1i += a1i;
    s0r += a0r;
    s0i += a0i;
    s2r += a2r;
    s2i += a2i;
#pragma unroll
    for (int j = 0; j < kLS; ++j) {
      gv[j] = gn[j];
      xv[j] = xn[j];
    }
    p ^= 1;
  }
  // Per-filter sums over the block's segments, in a fixed order: the
  // wavefront's segments by shuffles, then the wavefronts in LDS.
  double s[6] = {s1r, s1i, s0r, s0i, s2r, s2i};
#pragma unroll
  for (int j = 0; j < 6; ++j)
    for (int off = kWave / 2; off >= kFC; off >>= 1) s[j] += __shfl_down(s[j], off);
  if (lane < kFC) {
#pragma unroll
    for (int j = 0; j < 6; ++j) s_red[w][lane][j] = s[j];
  }
  __syncthreads();
  if (threadIdx.x < kFC && l.fv) {
    double acc[6] = {0, 0, 0, 0, 0, 0};
    for (int v = 0; v < kWaves; ++v)
#pragma unroll
      for (int j = 0; j < 6; ++j) acc[j] += s_red[v][threadIdx.x][j];
    double* o = partial + 6 * (l.b * F + l.f);
#pragma unroll
    for (int j = 0; j < 6; ++j) o[j] = acc[j];
  }
}

// grad[f] = sum over b of partial[6*(b*F + f) + j] in fp64: one wavefront per
// filter (block f, f + gridDim.x, ...), lane l sums b = l, l + 64, ... in
// order, then a fixed-shape wave reduction.
__global__ __launch_bounds__(kWave) void btf_coef_reduce_kernel(const double* __restrict__ partial,
                                                                int64_t B, int64_t F,
                                                                float* __restrict__ gc1,
                                                                float* __restrict__ gk0,
                                                                float* __restrict__ gk1) {
  const int lane = threadIdx.x;
  for (int64_t f = blockIdx.x; f < F; f += gridDim.x) {
    double s[6] = {0, 0, 0, 0, 0, 0};
    for (int64_t b = lane; b < B; b += kWave) {
      const double* p = partial + 6 * (b * F + f);
#pragma unroll
      for (int j = 0; j < 6; ++j) s[j] += p[j];
    }
#pragma unroll
    for (int j = 0; j < 6; ++j) s[j] = wave_sum(s[j]);
    if (lane == 0) {
      gc1[2 * f] = (float)s[0];
      gc1[2 * f + 1] = (float)s[1];
      gk0[2 * f] = (float)s[2];
      gk0[2 * f + 1] = (float)s[3];
      if (gk1) {
        gk1[2 * f] = (float)s[4];
        gk1[2 * f + 1] = (float)s[5];
      }
    }
  }
}

inline bool aligned8(const void* p) { return p == nullptr || ((uintptr_t)p & 7) == 0; }
inline size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RQF_OK : (int)err;
}

int64_t btf_blocks(int64_t B, int64_t F) { return B * ((F + kFC - 1) / kFC); }
dim3 btf_grid(int64_t B, int64_t F) { return dim3((unsigned)btf_blocks(B, F)); }

// The backward's per-(batch, filter) partial sums; the forward needs none.
size_t btf_ws(int64_t B, int64_t T, int64_t F) {
  (void)T;
  return round256(sizeof(double) * 6 * (size_t)std::max<int64_t>(B * F, 1));
}

int btf_fwd(const float* c1, const float* k0, const float* k1, const float* x, float* out,
            int64_t B, int64_t T, int64_t F, void* ws, size_t ws_bytes, hipStream_t s) {
  (void)ws;
  (void)ws_bytes;
  if (B < 0 || T < 0 || F < 0) return RQF_ERR_ARG;
  if (B * T * F == 0) return RQF_OK;
  if (!c1 || !k0 || !x || !out) return RQF_ERR_ARG;
  if (!grid_fits(btf_blocks(B, F), kThreads)) return RQF_ERR_ARG;
  if (!aligned8(x) || !aligned8(out)) return RQF_ERR_ALIGN;
  if (k1)
    hipLaunchKernelGGL(btf_fwd_kernel<true>, btf_grid(B, F), dim3(kThreads), 0, s, c1, k0, k1, x,
                       out, T, F);
  else
    hipLaunchKernelGGL(btf_fwd_kernel<false>, btf_grid(B, F), dim3(kThreads), 0, s, c1, k0, k1,
                       x, out, T, F);
  return launch_status();
}

int btf_bwd(const float* c1, const float* k0, const float* k1, const float* x,
            const float* states, const float* gout, float* gx, float* gc1, float* gk0,
            float* gk1, int64_t B, int64_t T, int64_t F, void* ws, size_t ws_bytes,
            hipStream_t s) {
  if (B < 0 || T < 0 || F < 0) return RQF_ERR_ARG;
  if (F == 0) return RQF_OK;
  if (!c1 || !k0 || !gc1 || !gk0 || (k1 && !gk1)) return RQF_ERR_ARG;
  (void)states;  // grad_c1 comes from x (see btf_bwd_kernel)
  if (B * T > 0 && (!x || !gout || !gx)) return RQF_ERR_ARG;
  if (B * T > 0 && !grid_fits(btf_blocks(B, F), kThreads)) return RQF_ERR_ARG;
  if (!aligned8(x) || !aligned8(states) || !aligned8(gout) || !aligned8(gx)) return RQF_ERR_ALIGN;
  const size_t need = btf_ws(B, T, F);
  if (!ws || ws_bytes < need) return RQF_ERR_WORKSPACE;
  double* partial = (double*)ws;
  if (B * T > 0) {
    if (k1)
      hipLaunchKernelGGL(btf_bwd_kernel<true>, btf_grid(B, F), dim3(kThreads), 0, s, c1, k0, k1, x,
                         gout, gx, partial, T, F);
    else
      hipLaunchKernelGGL(btf_bwd_kernel<false>, btf_grid(B, F), dim3(kThreads), 0, s, c1, k0, k1,
                         x, gout, gx, partial, T, F);
  }
  hipLaunchKernelGGL(btf_coef_reduce_kernel, dim3(stride_blocks(F)), dim3(kWave), 0, s, partial,
                     B * T > 0 ? B : (int64_t)0, F, gc1, gk0, gk1);
  return launch_status();
}

}  // namespace

// ------------------------------- C ABI ------------------------------------

extern "C" size_t rqf_btf_scan_workspace(int64_t B, int64_t T, int64_t F) {
  if (B < 0 || T < 0 || F < 0) return 0;
  return btf_ws(B, T, F);
}

extern "C" int rqf_chunked_scan_fwd(const float* c1, const float* c2, const float* u, float* out,
                                    int64_t B, int64_t T, int64_t F, void* ws, size_t ws_bytes,
                                    rqf_stream_t stream) {
  return btf_fwd(c1, c2, nullptr, u, out, B, T, F, ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int rqf_chunked_scan_bwd(const float* c1, const float* c2, const float* u,
                                    const float* states, const float* grad_out, float* grad_u,
                                    float* grad_c1, float* grad_c2, int64_t B, int64_t T,
                                    int64_t F, void* ws, size_t ws_bytes, rqf_stream_t stream) {
  return btf_bwd(c1, c2, nullptr, u, states, grad_out, grad_u, grad_c1, grad_c2, nullptr, B, T, F,
                 ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int rqf_chunked_prospective_fwd(const float* c1, const float* tap0, const float* tap1,
                                           const float* x, float* out, int64_t B, int64_t T,
                                           int64_t F, void* ws, size_t ws_bytes,
                                           rqf_stream_t stream) {
  if (!tap1) return RQF_ERR_ARG;
  return btf_fwd(c1, tap0, tap1, x, out, B, T, F, ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int rqf_chunked_prospective_bwd(const float* c1, const float* tap0, const float* tap1,
                                           const float* x, const float* states,
                                           const float* grad_out, float* grad_x, float* grad_c1,
                                           float* grad_tap0, float* grad_tap1, int64_t B,
                                           int64_t T, int64_t F, void* ws, size_t ws_bytes,
                                           rqf_stream_t stream) {
  if (!tap1 || !grad_tap1) return RQF_ERR_ARG;
  return btf_bwd(c1, tap0, tap1, x, states, grad_out, grad_x, grad_c1, grad_tap0, grad_tap1, B, T,
                 F, ws, ws_bytes, (hipStream_t)stream);
}
