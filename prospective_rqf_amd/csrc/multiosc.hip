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
// Here, as in btf.hip, a block owns 16 consecutive filters of one batch
// element and walks the sequence in passes of 4 segments of LS steps per
// wavefront; a thread takes one (filter, segment) of each pass with the
// filter's oscillators (N padded to a power of two NP <= 4, padded ones with
// zero coefficients) in registers.  It loads its segment's inputs once (the
// next pass's while the current one computes), scans them from a zero state
// per oscillator, and gets its entry states from the segments before it: the
// wavefront's earlier segments by cross-lane moves (fp32, at most 3 hops,
// exactly rounded maps), the earlier wavefronts' and the block's carry
// through LDS.  The thread then replays the segment and writes the output.
//   * Forward: each thread folds the earlier wavefronts' totals itself (fp32);
//     one thread per (filter, oscillator) extends the carry in fp64.  Blocks
//     of 16 wavefronts where the registers allow (real input), else 8.
//   * Backward: after the barrier one wavefront, one lane per (oscillator,
//     filter), walks the block's wavefronts from the carry in fp64, records
//     the pair entering each in LDS and extends the carry; after a second
//     barrier each thread applies one map to its entry.  That keeps the
//     serial part of the fold off every other wavefront.
// Filter groups of one batch element run on one XCD (xcd_contiguous): with
// real input a group reads half of each 128-byte line of a (B,T,F) row.
// Inputs are read once, outputs written once, and no carry crosses a block.
// More than 4 oscillators run in chunks of 4, each adding its share to the
// output (or to grad_u).
//
// The scanned state is w_n = x_n / C2_n, i.e. w_n[t] = C1_n w_n[t-1] + u[t],
// with C2_n applied at the output: y = sum_n (cw_n C2_n) w_n.  No division
// happens; C2 = 0 is fine.
//
// Backward.  The adjoint e_n[t] = conj(C1_n) e_n[t+1] + grad_out[t] runs the
// same way in reverse time; grad_u is sum_n conj(cw_n C2_n) e_n.  The
// reference's coefficient sums pair the adjoint at t with the state at t-1,
// which a reverse sweep does not have.  Exchanging the order of summation
// pairs them with u instead (mosc_coef_kernel): against e_n for grad_C2 and
// grad_cw, and against f_n, the derivative of e_n's recurrence with respect to
// conj(C1_n), for grad_C1.  f_n is itself a reverse recurrence, f_n[t] =
// conj(C1_n) f_n[t+1] + e_n[t+1], carried between segments with e_n.  So the
// pass reads grad_out and u once and produces grad_u and all three sums, with
// no forward state and no per-step state tensor (the reference keeps every
// state in a (B*F, T, N) scratch tensor).
//
// Coefficient gradients are reduced deterministically: per-(batch, filter,
// oscillator) fp64 partial sums, then an ordered reduction over the batch.
#include "rqf_device.h"
#include "rqf_scan.h"

#include <algorithm>
#include <cstdint>

using namespace rqf;

namespace {

constexpr int kMaxChunk = 4;  // oscillators per kernel launch
constexpr int kFC = 16;       // filters per block
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kNSeg = kThreads / kFC;  // segments per pass
constexpr int kG = kWave / kFC;        // segments per wavefront

// Steps per segment, by padded oscillator count (registers: the segment's
// inputs and the next pass's are held per thread).
template <int NP>
struct Seg {
  static constexpr int fwd = NP <= 2 ? 32 : 16;
  static constexpr int bwd = NP == 1 ? 16 : 8;
};

__device__ __forceinline__ c32 ldc(const float* p, int64_t i) {
  const float2 v = *reinterpret_cast<const float2*>(p + 2 * i);
  return mk(v.x, v.y);
}
__device__ __forceinline__ void stc(float* p, int64_t i, c32 v) {
  *reinterpret_cast<float2*>(p + 2 * i) = make_float2(v.r, v.i);
}
__device__ __forceinline__ double2 d2(c64d v) { return make_double2(v.r, v.i); }
__device__ __forceinline__ c64d cd(double2 v) { return mkd(v.x, v.y); }

struct Lane {
  int fl, sg, lane, w, q;
  int64_t f, b;
  bool fv;
  int64_t base;  // element (b, 0, f)
};

__device__ __forceinline__ Lane lane_of(int64_t T, int64_t F) {
  Lane l;
  l.fl = (int)threadIdx.x % kFC;
  l.sg = (int)threadIdx.x / kFC;
  l.lane = lane_id();
  l.w = wave_id();
  l.q = l.lane / kFC;
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

// Global memory goes through buffer descriptors (wave-uniform, in scalar
// registers).  A Pass names steps [pt, min(T, pt + pass)) of the block's
// batch element in one tensor; the descriptor of step j of every segment
// starts j rows further and is j rows shorter, so all steps of a segment use
// the lane's one byte offset: that of its segment's first step and its
// filter, or kBufOut for a filter past F.  Steps past T and filters past F
// then read zero and drop their stores with no test and no per-element
// address arithmetic (the host keeps pass * F * 8 below 2^31).
struct Pass {
  const char* base;
  int n;          // valid steps from base
  uint32_t step;  // bytes per time step
  // (a signed max, not a saturating subtraction of bytes: that has no scalar
  // instruction, and a descriptor in vector registers costs a loop per access)
  __device__ __forceinline__ brsrc at(int j) const {
    return buf_rsrc(base + (uint32_t)j * step, (uint32_t)std::max(n - j, 0) * step);
  }
};
__device__ __forceinline__ uint32_t lane_off(const Lane& l, int LS, int64_t F, int esz) {
  return l.fv ? (uint32_t)(((int64_t)l.sg * LS * F + l.f) * esz) : kBufOut;
}
__device__ __forceinline__ Pass pass_of(const float* p, const Lane& l, int64_t pt, int64_t pass,
                                        int64_t T, int64_t F, int esz) {
  // Everything here is wave-uniform; readfirstlane pins it to scalar
  // registers, which the descriptors need (a 64-bit compare or select the
  // compiler does in vector registers would otherwise leave them there).
  const uint64_t base =
      reinterpret_cast<uint64_t>(p) + (uint64_t)((l.b * T + std::min(pt, T)) * F * esz);
  Pass s;
  s.base = reinterpret_cast<const char*>(
      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32)) << 32) |
      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base));
  s.n = __builtin_amdgcn_readfirstlane((int)(pt < T ? std::min(T, pt + pass) - pt : 0));
  s.step = (uint32_t)__builtin_amdgcn_readfirstlane((int)(F * esz));
  return s;
}

// Inputs of the thread's segment (lane offset lo in pass s); zero past T and
// for filters past F.
template <int LS, bool REAL>
__device__ __forceinline__ void load_seg(const Pass& s, uint32_t lo, c32 (&v)[LS]) {
#pragma unroll
  for (int j = 0; j < LS; ++j)
    v[j] = REAL ? mk(buf_ldf(s.at(j), lo), 0.0f) : buf_ldc(s.at(j), lo);
}

// The backward goes through global addresses: descriptors measured slower
// there (0.47 -> 0.49 ms at config 6: three streams of 8-step segments, a
// descriptor per step and stream).  A pass that lies wholly inside [0, T)
// (every pass but the last) is addressed from a wave-uniform base per step
// (scalar arithmetic) plus the lane's fixed offset, one 64-bit add per
// element and no test; the per-element multiply, the range test and its
// exec mask of load_seg_g dropped the pass loop from 1326 to 1176 VALU
// instructions per lane at config 6 (backward 0.479 -> 0.468 ms).
//
// Byte offset of step pt of the lane's batch element in a (B,T,F) stream.
// The offset, not the pointer, goes through readfirstlane: a pointer rebuilt
// from integers loses its address space and its stores become flat ones.
__device__ __forceinline__ int64_t pass_off(const Lane& l, int64_t pt, int64_t T, int64_t F,
                                            int esz) {
  return (int64_t)uniform64((uint64_t)((l.b * T + pt) * F * esz));
}
// The lane's byte offset from its pass's base: its segment's first step and
// its filter (filter 0 for a lane past F, whose values are never stored).
__device__ __forceinline__ uint64_t seg_off(const Lane& l, int LS, int64_t F, int esz) {
  return (uint64_t)(((int64_t)l.sg * LS * F + (l.fv ? l.f : 0)) * esz);
}
// A whole segment: base pb of the pass, lane offset lo, stp bytes per step.
template <int LS, bool REAL>
__device__ __forceinline__ void load_seg_w(const char* pb, uint64_t lo, uint64_t stp,
                                           c32 (&v)[LS]) {
#pragma unroll
  for (int j = 0; j < LS; ++j) {
    const char* q = (pb + (uint64_t)j * stp) + lo;
    if (REAL) {
      v[j] = mk(*reinterpret_cast<const float*>(q), 0.0f);
    } else {
      const float2 x = *reinterpret_cast<const float2*>(q);
      v[j] = mk(x.x, x.y);
    }
  }
}
// Any segment, with a test per element (the last pass, which may pass T).
template <int LS, bool REAL>
__device__ __forceinline__ void load_seg_g(const float* __restrict__ p, const Lane& l, int64_t tb,
                                           int64_t T, int64_t F, c32 (&v)[LS]) {
#pragma unroll
  for (int j = 0; j < LS; ++j) {
    const int64_t t = tb + j;
    const bool in = l.fv && t < T;
    if (REAL)
      v[j] = mk(in ? p[l.base + t * F] : 0.0f, 0.0f);
    else
      v[j] = in ? ldc(p, l.base + t * F) : mk(0.0f, 0.0f);
  }
}

// Coefficients of oscillators n0 .. n0+NP-1 of the lane's filter (index
// f*N + n; zero past N).
template <int NP>
__device__ __forceinline__ void load_osc(const float* __restrict__ p, const Lane& l, int N, int n0,
                                         c32 (&v)[NP]) {
#pragma unroll
  for (int n = 0; n < NP; ++n)
    v[n] = (l.fv && n0 + n < N) ? ldc(p, l.f * N + n0 + n) : mk(0.0f, 0.0f);
}

// Output weights of the scanned state: y = sum_n (cw_n C2_n) w_n, or C2_0 w_0
// without C-weights.
template <int NP, bool CW>
__device__ __forceinline__ void load_out_weights(const float* __restrict__ c2,
                                                 const float* __restrict__ cw, const Lane& l,
                                                 int N, int n0, c32 (&h)[NP]) {
  load_osc<NP>(c2, l, N, n0, h);
  if (CW) {
    c32 w[NP];
    load_osc<NP>(cw, l, N, n0, w);
#pragma unroll
    for (int n = 0; n < NP; ++n) h[n] = cmul(w[n], h[n]);
  }
}

__device__ __forceinline__ c32 shfl_up_c(c32 v, int d) {
  return mk(__shfl_up(v.r, d), __shfl_up(v.i, d));
}
__device__ __forceinline__ c32 shfl_down_c(c32 v, int d) {
  return mk(__shfl_down(v.r, d), __shfl_down(v.i, d));
}

// Powers of one filter's oscillator coefficient a over spans of segments of
// LS steps, computed once per block in fp64 and rounded: m1 = a^LS (one
// segment), m2 = m1^2, mG = m1^G (one wavefront's segments), mq[q] = m1^q,
// and mB = m1^(G*W) (one pass of W wavefronts), kept in fp64 for the carry
// chain.
struct FwdMaps {
  c32 m1, m2, mG, mq[kG];
  double2 mB;
};
template <int LS, int W>
__device__ __forceinline__ FwdMaps fwd_maps(c32 a) {
  FwdMaps k;
  const c64d m1 = dpow(widen(a), LS);
  k.m1 = narrow(m1);
  k.m2 = narrow(dmul(m1, m1));
#pragma unroll
  for (int q = 0; q < kG; ++q) k.mq[q] = narrow(dpow(m1, q));
  const c64d mG = dpow(m1, kG);
  k.mG = narrow(mG);
  k.mB = d2(dpow(mG, W));
  return k;
}

// ---------------------------------------------------------------------------
// Forward.  yin (optional, complex (B,T,F)) is added to this chunk's y: the
// earlier chunks' share.  yout receives y (complex) or |y| (ABS).  A block
// has W wavefronts: 16 (4 per SIMD) where the registers allow it, to hide
// more memory latency per CU, else 8.  G64: 64-bit global addresses with a
// test per element instead of the buffer descriptors, for rows too wide for
// one 32-bit range per pass (F > kDescFilters).
// ---------------------------------------------------------------------------
template <int NP, bool REAL, bool CW, bool ABS, int W, bool G64>
__global__ __launch_bounds__(W* kWave) void mosc_fwd_kernel(
    const float* __restrict__ c1, const float* __restrict__ c2, const float* __restrict__ cw,
    const float* __restrict__ u, const float* yin, float* yout, int64_t T, int64_t F, int N,
    int n0) {
  constexpr int LS = Seg<NP>::fwd;
  constexpr int kPass = W * kG * LS;
  __shared__ c32 s_tot[2][W][NP][kFC];
  __shared__ double2 s_carry[2][NP][kFC];
  __shared__ FwdMaps s_k[NP][kFC];
  const Lane l = lane_of(T, F);
  c32 a[NP], hw[NP];
  load_osc<NP>(c1, l, N, n0, a);
  load_out_weights<NP, CW>(c2, cw, l, N, n0, hw);
  if (l.sg == 0) {
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      s_carry[0][n][l.fl] = make_double2(0.0, 0.0);
      s_k[n][l.fl] = fwd_maps<LS, W>(a[n]);
    }
  }
  __syncthreads();
  constexpr int kUs = REAL ? 4 : 8;
  const uint32_t lo_u = lane_off(l, LS, F, kUs), lo_c = lane_off(l, LS, F, 8),
                 lo_a = lane_off(l, LS, F, 4);
  c32 uv[LS], un[LS];
  auto load_pass = [&](int64_t pt, c32(&v)[LS]) {
    if constexpr (G64)
      load_seg_g<LS, REAL>(u, l, pt + (int64_t)l.sg * LS, T, F, v);
    else
      load_seg<LS, REAL>(pass_of(u, l, pt, kPass, T, F, kUs), lo_u, v);
  };
  load_pass(0, uv);
  int p = 0;
  for (int64_t pt = 0; pt < T; pt += kPass) {
    if (pt + kPass < T) load_pass(pt + kPass, un);
    // Each oscillator's segment from a zero state.
    c32 w[NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) w[n] = mk(0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < LS; ++j)
#pragma unroll
      for (int n = 0; n < NP; ++n) w[n] = REAL ? cmadr(a[n], w[n], uv[j].r) : cmad(a[n], w[n], uv[j]);
    // Entry states: the wavefront's earlier segments (cross-lane), then the
    // block's carry and the earlier wavefronts (LDS).  Within a pass at most
    // 10 segment hops are folded, in fp32 with exactly rounded powers; the
    // carry from pass to pass, a chain of T / pass hops, is kept in fp64.
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const FwdMaps& k = s_k[n][l.fl];
      c32 incl = w[n];
      c32 prev = shfl_up_c(incl, kFC);
      if (l.q >= 1) incl = cmad(k.m1, prev, incl);
      prev = shfl_up_c(incl, 2 * kFC);
      if (l.q >= 2) incl = cmad(k.m2, prev, incl);
      if (l.q == kG - 1) s_tot[p][l.w][n][l.fl] = incl;
      const c32 ex = shfl_up_c(incl, kFC);
      w[n] = l.q >= 1 ? ex : mk(0.0f, 0.0f);
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const FwdMaps& k = s_k[n][l.fl];
      const c64d carry = cd(s_carry[p][n][l.fl]);
      c32 cw_ = narrow(carry);
      for (int v = 0; v < l.w; ++v) cw_ = cmad(k.mG, cw_, s_tot[p][v][n][l.fl]);
      if (l.w == W - 1 && l.q == kG - 1) {
        c32 z = mk(0.0f, 0.0f);
        for (int v = 0; v < W; ++v) z = cmad(k.mG, z, s_tot[p][v][n][l.fl]);
        s_carry[p ^ 1][n][l.fl] = d2(dmad(cd(k.mB), carry, widen(z)));
      }
      w[n] = cmad(k.mq[l.q], cw_, w[n]);
    }
    // Replay and write.
    const Pass sy = pass_of(yout, l, pt, kPass, T, F, ABS ? 4 : 8);
    const Pass si = pass_of(yin ? yin : yout, l, pt, kPass, T, F, 8);
    const int64_t tb = pt + (int64_t)l.sg * LS;
#pragma unroll
    for (int j = 0; j < LS; ++j) {
      c32 y = mk(0.0f, 0.0f);
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        w[n] = REAL ? cmadr(a[n], w[n], uv[j].r) : cmad(a[n], w[n], uv[j]);
        if (CW || n == 0) y = cmad(hw[n], w[n], y);
      }
      if constexpr (G64) {
        const bool in = l.fv && tb + j < T;
        const int64_t e = l.base + (tb + j) * F;
        if (yin && in) y = cadd(y, ldc(yin, e));
        if (in) {
          if (ABS)
            yout[e] = sqrtf(fmaf(y.r, y.r, y.i * y.i));
          else
            stc(yout, e, y);
        }
      } else {
        if (yin) y = cadd(y, buf_ldc(si.at(j), lo_c));
        if (ABS)
          buf_stf(sy.at(j), lo_a, sqrtf(fmaf(y.r, y.r, y.i * y.i)));
        else
          buf_stc(sy.at(j), lo_c, y);
      }
    }
#pragma unroll
    for (int j = 0; j < LS; ++j) uv[j] = un[j];
    p ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Backward, from each segment's exit pair, for t descending:
//   f_n[t]    = conj(C1_n) f_n[t+1] + e_n[t+1]                  (TAN)
//   e_n[t]    = conj(C1_n) e_n[t+1] + gy[t]
//   grad_u[t] = sum_n conj(cw_n C2_n) e_n[t]   (GU; real u: its real part)
//   Q_n += e_n[t] conj(u[t]),  R_n += f_n[t] conj(u[t])         (TAN)
// e_n is the reference's adjoint d_n without its conj(cw_n) factor, and
// f_n[t] = sum_{s>t} conj(C1_n)^(s-1-t) e_n[s], the derivative of e_n's
// recurrence with respect to conj(C1_n).  LS steps of zero input take the
// pair (e, f) to (P e, P f + LS P' e), P = conj(C1)^LS, P' = conj(C1)^(LS-1)
// (the PairMap of rqf_device.h).  gin (optional) is added to grad_u: the
// earlier oscillator chunks' share.  Partial sums go to
// part[((b*F + f)*N + n)*4 + j] (j: Re Q, Im Q, Re R, Im R).
// ---------------------------------------------------------------------------
struct Pair {
  double2 g, h;
};
struct Pair32 {
  c32 g, h;
};
// A pair map in fp32 (see PairMap).
struct PairMap32 {
  c32 P, c;
};
__device__ __forceinline__ PairMap32 narrow_map(PairMap m) { return {narrow(m.P), narrow(m.c)}; }
// (g, h) entering a span with map m and own pair (G, H) -> the span's start pair.
__device__ __forceinline__ void pair_apply32(PairMap32 m, c32 G, c32 H, c32& g, c32& h) {
  const c32 ng = cmad(m.P, g, G);
  h = cmad(m.P, h, cmad(m.c, g, H));
  g = ng;
}

// Pair map of one segment of LS steps: P = conj(a)^LS, c = LS conj(a)^(LS-1).
template <int LS>
__device__ __forceinline__ PairMap one_segment(c32 a) {
  const c64d p1 = LS > 1 ? dconj(dpow(widen(a), LS - 1)) : mkd(1.0, 0.0);
  PairMap m;
  m.P = dmul(p1, dconj(widen(a)));
  m.c = mkd(p1.r * (double)LS, p1.i * (double)LS);
  return m;
}

// One filter's pair maps over spans of segments, computed once per block in
// fp64 and rounded: one and two segments, the G-1-q segments after segment q
// of a wavefront, and one wavefront's G segments (also kept in fp64 for the
// carry chain).
struct BwdMaps {
  PairMap32 one, two, after[kG];
  Pair wave;  // (P, c) of one wavefront's segments, fp64
};
template <int LS>
__device__ __forceinline__ BwdMaps bwd_maps(c32 a) {
  BwdMaps k;
  const PairMap one = one_segment<LS>(a);
  const PairMap two = pair_map_mul(one, one);
  PairMap wave = one;
  for (int i = 1; i < kG; ++i) wave = pair_map_mul(wave, one);
  k.one = narrow_map(one);
  k.two = narrow_map(two);
  k.wave = Pair{d2(wave.P), d2(wave.c)};
  PairMap acc;
  acc.P = mkd(1.0, 0.0);
  acc.c = mkd(0.0, 0.0);
  for (int q = kG - 1; q >= 0; --q) {  // after[q]: the G-1-q segments after q
    k.after[q] = narrow_map(acc);
    acc = pair_map_mul(acc, one);
  }
  return k;
}

template <int NP, bool REAL, bool TAN, bool GU>
__global__ __launch_bounds__(kThreads) void mosc_bwd_kernel(
    const float* __restrict__ c1, const float* __restrict__ c2, const float* __restrict__ cw,
    const float* __restrict__ u, const float* __restrict__ gy, const float* gin, float* gu,
    double* __restrict__ part, int64_t T, int64_t F, int N, int n0) {
  constexpr int LS = Seg<NP>::bwd;
  constexpr int kPass = kNSeg * LS;
  // Per pass: each wavefront's pair from a zero entry (s_tot), the pair
  // entering each wavefront (s_ent) and the block's carry (fp64).
  __shared__ Pair32 s_tot[kWaves][NP][kFC];
  __shared__ Pair32 s_ent[kWaves][NP][kFC];
  __shared__ Pair s_carry[NP][kFC];
  __shared__ BwdMaps s_k[NP][kFC];
  __shared__ double s_red[TAN ? kWaves * kFC * 4 * NP : 1];
  const Lane l = lane_of(T, F);
  c32 a[NP], hw[NP];
  load_osc<NP>(c1, l, N, n0, a);
  if (GU) load_out_weights<NP, true>(c2, cw, l, N, n0, hw);
  if (l.sg == 0) {
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      s_carry[n][l.fl] = Pair{make_double2(0.0, 0.0), make_double2(0.0, 0.0)};
      s_k[n][l.fl] = bwd_maps<LS>(a[n]);
    }
  }
  __syncthreads();
  // Q and R partial sums of the lane's segments, accumulated straight from
  // every step (fp32 within the lane, fp64 across lanes and batches).
  float qr[NP][4];
#pragma unroll
  for (int n = 0; n < NP; ++n) qr[n][0] = qr[n][1] = qr[n][2] = qr[n][3] = 0.0f;
  const int64_t npass = (T + kPass - 1) / kPass;
  constexpr int kUs = REAL ? 4 : 8;  // bytes per element of u and grad_u
  const uint64_t lo8 = seg_off(l, LS, F, 8), lou = seg_off(l, LS, F, kUs);
  const uint64_t stp8 = uniform64((uint64_t)F * 8);
  const uint64_t stpu = uniform64((uint64_t)F * kUs);
  const char* const gyb = reinterpret_cast<const char*>(gy);
  const char* const ub = reinterpret_cast<const char*>(u);
  c32 gv[LS], gn[LS], uv[TAN ? LS : 1], un[TAN ? LS : 1];
  int64_t pt = (npass - 1) * kPass;
  load_seg_g<LS, false>(gy, l, pt + (int64_t)l.sg * LS, T, F, gv);
  if constexpr (TAN) load_seg_g<LS, REAL>(u, l, pt + (int64_t)l.sg * LS, T, F, uv);
  for (; pt >= 0; pt -= kPass) {
    const int64_t tb = pt + (int64_t)l.sg * LS;
    if (pt > 0) {
      // Every pass before the last lies wholly inside [0, T).
      load_seg_w<LS, false>(gyb + pass_off(l, pt - kPass, T, F, 8), lo8, stp8, gn);
      if constexpr (TAN)
        load_seg_w<LS, REAL>(ub + pass_off(l, pt - kPass, T, F, kUs), lou, stpu, un);
    }
    // Each oscillator's pair at the segment's first step from a zero pair.
    c32 e[NP], f[NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) e[n] = f[n] = mk(0.0f, 0.0f);
#pragma unroll
    for (int j = LS - 1; j >= 0; --j)
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        if (TAN) f[n] = cjmad(a[n], f[n], e[n]);
        e[n] = cjmad(a[n], e[n], gv[j]);
      }
    // Entry pairs.  The wavefront's later segments come by cross-lane moves
    // (at most 3 hops, fp32 with exactly rounded maps).  Then one wavefront
    // walks the block's wavefronts from the carry, latest first, one lane per
    // (oscillator, filter): it records the pair entering each wavefront and
    // carries the chain on, in fp64, to the next (earlier) pass.
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const BwdMaps& k = s_k[n][l.fl];
      c32 ig = e[n], ih = f[n];
      c32 ng = shfl_down_c(ig, kFC), nh = shfl_down_c(ih, kFC);
      if (l.q + 1 < kG) pair_apply32(k.one, ig, ih, ng, nh), ig = ng, ih = nh;
      ng = shfl_down_c(ig, 2 * kFC);
      nh = shfl_down_c(ih, 2 * kFC);
      if (l.q + 2 < kG) pair_apply32(k.two, ig, ih, ng, nh), ig = ng, ih = nh;
      if (l.q == 0) s_tot[l.w][n][l.fl] = Pair32{ig, ih};
      const c32 xg = shfl_down_c(ig, kFC), xh = shfl_down_c(ih, kFC);
      e[n] = l.q + 1 < kG ? xg : mk(0.0f, 0.0f);
      f[n] = l.q + 1 < kG ? xh : mk(0.0f, 0.0f);
    }
    __syncthreads();
    if (l.w == 0 && l.lane < NP * kFC) {
      const int n = l.lane / kFC, fl = l.lane % kFC;
      const Pair wm = s_k[n][fl].wave;
      PairMap pm;
      pm.P = cd(wm.g);
      pm.c = cd(wm.h);
      const Pair cr = s_carry[n][fl];
      c64d g = cd(cr.g), h = cd(cr.h);
#pragma unroll 1
      for (int v = kWaves - 1; v >= 0; --v) {
        s_ent[v][n][fl] = Pair32{narrow(g), narrow(h)};
        const Pair32 t = s_tot[v][n][fl];
        pair_apply(pm, widen(t.g), widen(t.h), g, h);
      }
      s_carry[n][fl] = Pair{d2(g), d2(h)};
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const Pair32 en = s_ent[l.w][n][l.fl];
      c32 cg = en.g, ch = en.h;
      pair_apply32(s_k[n][l.fl].after[l.q], e[n], f[n], cg, ch);
      e[n] = cg;
      f[n] = ch;
    }
    // Replay: grad_u and the coefficient sums.
    c32 go[GU ? LS : 1];
#pragma unroll
    for (int j = LS - 1; j >= 0; --j) {
      c32 g = mk(0.0f, 0.0f);
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        if (TAN) f[n] = cjmad(a[n], f[n], e[n]);
        e[n] = cjmad(a[n], e[n], gv[j]);
        if (GU) g = cjmad(hw[n], e[n], g);
        if constexpr (TAN) {
          // Q += e conj(u), R += f conj(u), as fused multiply-adds.
          const c32 uj = uv[j];
          qr[n][0] = fmaf(uj.r, e[n].r, qr[n][0]);
          qr[n][1] = fmaf(uj.r, e[n].i, qr[n][1]);
          qr[n][2] = fmaf(uj.r, f[n].r, qr[n][2]);
          qr[n][3] = fmaf(uj.r, f[n].i, qr[n][3]);
          if (!REAL) {
            qr[n][0] = fmaf(uj.i, e[n].i, qr[n][0]);
            qr[n][1] = fmaf(-uj.i, e[n].r, qr[n][1]);
            qr[n][2] = fmaf(uj.i, f[n].i, qr[n][2]);
            qr[n][3] = fmaf(-uj.i, f[n].r, qr[n][3]);
          }
        }
      }
      if constexpr (GU) go[j] = g;
    }
    if constexpr (GU) {
      // grad_u of the segment, after its steps (no stores inside the chain);
      // only the last pass can pass T.
      const bool whole = pt + kPass <= T;
      const int64_t po = pass_off(l, pt, T, F, kUs);
      char* const gb = reinterpret_cast<char*>(gu) + po;
      const char* const ib = gin ? reinterpret_cast<const char*>(gin) + po : nullptr;
#pragma unroll
      for (int j = 0; j < LS; ++j) {
        if (l.fv && (whole || tb + j < T)) {
          const uint64_t o = (uint64_t)j * stpu + lou;
          if (REAL) {
            *reinterpret_cast<float*>(gb + o) =
                go[j].r + (ib ? *reinterpret_cast<const float*>(ib + o) : 0.0f);
          } else {
            c32 v = go[j];
            if (ib) {
              const float2 x = *reinterpret_cast<const float2*>(ib + o);
              v = cadd(v, mk(x.x, x.y));
            }
            *reinterpret_cast<float2*>(gb + o) = make_float2(v.r, v.i);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < LS; ++j) {
      gv[j] = gn[j];
      if constexpr (TAN) uv[j] = un[j];
    }
  }
  if (!TAN) return;
  // Per (filter, oscillator) sums over the block's segments, in a fixed order:
  // the wavefront's segments by shuffles, then the wavefronts in LDS.
#pragma unroll
  for (int n = 0; n < NP; ++n)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      double v = (double)qr[n][k];
      for (int off = kWave / 2; off >= kFC; off >>= 1) v += __shfl_down(v, off);
      if (l.lane < kFC) s_red[((l.w * kFC) + l.lane) * 4 * NP + 4 * n + k] = v;
    }
  __syncthreads();
  if (threadIdx.x < kFC && l.fv) {
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      if (n0 + n >= N) break;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        double acc = 0.0;
        for (int v = 0; v < kWaves; ++v) acc += s_red[((v * kFC) + threadIdx.x) * 4 * NP + 4 * n + k];
        part[((l.b * F + l.f) * N + n0 + n) * 4 + k] = acc;
      }
    }
  }
}

// grad_C1, grad_C2, grad_cw of oscillator n of filter f (one wavefront per
// f*N + n) from the partial sums of Q and R (lane l adds b = l, l + 64, ...,
// then a fixed-shape wave sum), then
//   grad_C1 = conj(cw C2) R,   grad_C2 = conj(cw) Q,   grad_cw = conj(C2) Q.
// These are the reference's sums, with x_n = C2_n w_n and d_n = conj(cw_n) e_n
// and the order of summation exchanged (u[r] enters w_n[t] with C1^(t-r)):
//   sum_t d_n[t] conj(u[t])     = conj(cw_n) sum_t e_n[t] conj(u[t])
//   sum_t gy[t] conj(x_n[t])    = conj(C2_n) sum_r conj(u[r]) sum_{t>=r} conj(C1)^(t-r) gy[t]
//                               = conj(C2_n) sum_r e_n[r] conj(u[r])
//   sum_t d_n[t] conj(x_n[t-1]) = conj(cw_n C2_n) sum_r conj(u[r]) sum_{t>r} conj(C1)^(t-1-r) e_n[t]
//                               = conj(cw_n C2_n) sum_r f_n[r] conj(u[r]).
__global__ __launch_bounds__(kWave) void mosc_coef_kernel(const double* __restrict__ part,
                                                          int64_t B, int64_t F, int N,
                                                          const float* __restrict__ c2,
                                                          const float* __restrict__ cw,
                                                          float* __restrict__ gc1,
                                                          float* __restrict__ gc2,
                                                          float* __restrict__ gcw) {
  const int lane = threadIdx.x;
  for (int64_t fn = blockIdx.x; fn < F * N; fn += gridDim.x) {  // fn = f*N + n
    double s[4] = {0, 0, 0, 0};
    for (int64_t b = lane; b < B; b += kWave) {
      const double* p = part + (b * F * N + fn) * 4;
#pragma unroll
      for (int k = 0; k < 4; ++k) s[k] += p[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) s[k] = wave_sum(s[k]);
    if (lane == 0) {
      const c64d q = mkd(s[0], s[1]), r = mkd(s[2], s[3]);
      const c64d g2 = dconj(widen(ldc(c2, fn))), gw = dconj(widen(ldc(cw, fn)));
      if (gc1) stc(gc1, fn, narrow(dmul(dmul(gw, g2), r)));
      if (gc2) stc(gc2, fn, narrow(dmul(gw, q)));
      if (gcw) stc(gcw, fn, narrow(dmul(g2, q)));
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
  while (np < N && np < kMaxChunk) np <<= 1;
  return np;
}

dim3 mosc_grid(int64_t B, int64_t F) { return dim3((unsigned)(B * ((F + kFC - 1) / kFC))); }

// F <= kDescFilters keeps every pass's descriptor (at most 2048 steps of F
// complex elements) below 2^31 bytes; wider rows run the forward with 64-bit
// addresses (the backward always does).  The scan grids bound the rest: B
// blocks per 16 filters, of up to kMaxBlockThreads work-items each, within
// one dispatch's 32-bit work-item count (grid_fits).  The coefficient
// reduction strides over the (filter, oscillator) pairs, so it takes any F*N
// below 2^31.
constexpr int64_t kDescFilters = 65536;
constexpr int kMaxBlockThreads = 16 * kWave;
static_assert(kThreads <= kMaxBlockThreads, "the backward's blocks within the grid bound");
bool bad_shape(int64_t B, int64_t T, int64_t F, int64_t N) {
  if (B < 0 || T < 0 || F < 0 || N < 1 || N > (int64_t)1 << 20) return true;
  return !grid_fits(B * ((F + kFC - 1) / kFC), kMaxBlockThreads) || F * N > INT32_MAX;
}

// Workspace: forward, a complex (B,T,F) partial when a |y| output needs more
// than one chunk of oscillators; backward, the per-(batch, filter, oscillator)
// partial sums.
size_t mosc_ws(int64_t B, int64_t T, int64_t F, int64_t N, bool backward) {
  if (backward) return round256(sizeof(double) * 4 * (size_t)std::max<int64_t>(B * F * N, 1));
  return N > kMaxChunk ? round256(sizeof(float) * 2 * (size_t)(B * T * F)) : 0;
}

template <class Fn>
void with_np(int np, Fn&& fn) {
  switch (np) {
    case 1: fn(std::integral_constant<int, 1>{}); return;
    case 2: fn(std::integral_constant<int, 2>{}); return;
    default: fn(std::integral_constant<int, 4>{}); return;
  }
}

template <int NP, bool REAL, bool G64>
void launch_fwd(const float* c1, const float* c2, const float* cw, const float* u,
                const float* yin, float* yout, bool abs_out, int64_t B, int64_t T, int64_t F,
                int N, int n0, hipStream_t s) {
  // 16 wavefronts per block where the kernel fits in 128 VGPRs (real input;
  // without C-weights, which only one oscillator has, at most two), 12 where
  // it fits in 168 (complex input, 4 oscillators: 0.271 -> 0.250 ms at
  // config 6), else 8.
  constexpr int W = REAL ? 16 : (NP == 4 ? 12 : 8), W1 = REAL && NP <= 2 ? 16 : 8;
  static_assert(W * kWave <= kMaxBlockThreads && W1 * kWave <= kMaxBlockThreads, "grid bound");
  const dim3 grid = mosc_grid(B, F), block(W * kWave), block1(W1 * kWave);
  if (cw && abs_out) {
    hipLaunchKernelGGL((mosc_fwd_kernel<NP, REAL, true, true, W, G64>), grid, block, 0, s, c1, c2, cw, u, yin, yout, T, F, N, n0);
  } else if (cw) {
    hipLaunchKernelGGL((mosc_fwd_kernel<NP, REAL, true, false, W, G64>), grid, block, 0, s, c1, c2, cw, u, yin, yout, T, F, N, n0);
  } else if constexpr (NP == 1) {  // without C-weights N is 1 (checked by the caller)
    if (abs_out)
      hipLaunchKernelGGL((mosc_fwd_kernel<NP, REAL, false, true, W1, G64>), grid, block1, 0, s, c1, c2, cw, u, yin, yout, T, F, N, n0);
    else
      hipLaunchKernelGGL((mosc_fwd_kernel<NP, REAL, false, false, W1, G64>), grid, block1, 0, s, c1, c2, cw, u, yin, yout, T, F, N, n0);
  }
}

template <int NP, bool REAL>
void launch_bwd(const float* c1, const float* c2, const float* cw, const float* u,
                const float* gy, const float* gin, float* gu, double* part, bool tan, bool gu_on,
                int64_t B, int64_t T, int64_t F, int N, int n0, hipStream_t s) {
  const dim3 grid = mosc_grid(B, F), block(kThreads);
  if (tan && gu_on)
    hipLaunchKernelGGL((mosc_bwd_kernel<NP, REAL, true, true>), grid, block, 0, s, c1, c2, cw, u, gy, gin, gu, part, T, F, N, n0);
  else if (tan)
    hipLaunchKernelGGL((mosc_bwd_kernel<NP, REAL, true, false>), grid, block, 0, s, c1, c2, cw, u, gy, gin, gu, part, T, F, N, n0);
  else
    hipLaunchKernelGGL((mosc_bwd_kernel<NP, REAL, false, true>), grid, block, 0, s, c1, c2, cw, u, gy, gin, gu, part, T, F, N, n0);
}

}  // namespace

// ------------------------------- C ABI ------------------------------------

extern "C" size_t rqf_multi_osc_workspace(int64_t B, int64_t T, int64_t F, int64_t N,
                                          int32_t backward) {
  if (bad_shape(B, T, F, N)) return 0;
  return mosc_ws(B, T, F, N, backward != 0);
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
  const size_t need = mosc_ws(B, T, F, N, false);
  if (need && (!workspace || workspace_bytes < need)) return RQF_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int chunks = (int)((N + kMaxChunk - 1) / kMaxChunk);
  // Complex partial of y between chunks: the output itself, or the workspace
  // when the output is |y|.
  float* ypart = out_abs ? (float*)workspace : out;
  for (int c = 0; c < chunks; ++c) {
    const int n0 = c * kMaxChunk;
    const int np = pad_osc((int)std::min<int64_t>(N - n0, kMaxChunk));
    const bool last = c + 1 == chunks;
    const float* yin = c > 0 ? ypart : nullptr;
    float* yout = last ? out : ypart;
    const bool abs_here = last && out_abs;
    with_np(np, [&](auto npc) {
      constexpr int NP = decltype(npc)::value;
      if (F > kDescFilters) {
        if (u_real)
          launch_fwd<NP, true, true>(c1, c2, cw, u, yin, yout, abs_here, B, T, F, (int)N, n0, s);
        else
          launch_fwd<NP, false, true>(c1, c2, cw, u, yin, yout, abs_here, B, T, F, (int)N, n0, s);
      } else if (u_real) {
        launch_fwd<NP, true, false>(c1, c2, cw, u, yin, yout, abs_here, B, T, F, (int)N, n0, s);
      } else {
        launch_fwd<NP, false, false>(c1, c2, cw, u, yin, yout, abs_here, B, T, F, (int)N, n0, s);
      }
    });
  }
  return launch_status();
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
  const size_t need = mosc_ws(B, T, F, N, true);
  if (!workspace || workspace_bytes < need) return RQF_ERR_WORKSPACE;
  double* part = (double*)workspace;
  const bool coefs = grad_c1 || grad_c2 || grad_cw;
  hipStream_t s = (hipStream_t)stream;
  if (B * T > 0 && (coefs || grad_u)) {
    const int chunks = (int)((N + kMaxChunk - 1) / kMaxChunk);
    for (int c = 0; c < chunks; ++c) {
      const int n0 = c * kMaxChunk;
      const int np = pad_osc((int)std::min<int64_t>(N - n0, kMaxChunk));
      const float* gin = c > 0 ? grad_u : nullptr;
      with_np(np, [&](auto npc) {
        constexpr int NP = decltype(npc)::value;
        if (u_real)
          launch_bwd<NP, true>(c1, c2, cw, u, grad_out, gin, grad_u, part, coefs, grad_u != nullptr,
                               B, T, F, (int)N, n0, s);
        else
          launch_bwd<NP, false>(c1, c2, cw, u, grad_out, gin, grad_u, part, coefs,
                                grad_u != nullptr, B, T, F, (int)N, n0, s);
      });
    }
  }
  if (coefs)
    hipLaunchKernelGGL(mosc_coef_kernel, dim3(stride_blocks(F * N)), dim3(kWave), 0, s, part,
                       B * T > 0 ? B : (int64_t)0, F, (int)N, c2, cw, grad_c1, grad_c2, grad_cw);
  return launch_status();
}
