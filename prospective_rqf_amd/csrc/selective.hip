// selective.hip -- fused selective complex scan for gfx950.
//
// Forward  y[t] = A[t] y[t-1] + gate[t] (bp[t] z[t] + bn[t] z[t-1]),  y[-1] = 0
// with A, bp, bn, gate computed per element from the controller logits
// (gamma / warp / write heads) and the per-channel parameters, the ZOH
// discretisation and the prospective two-tap input
// (rqf_models/ops/selective_scan_kernel.py:16-101, docs/selective_rqf.md:84-104).
// The coefficients never touch HBM: only z, the logits, the outputs and the
// per-chunk entry states cross the kernel boundary.
//
// Work decomposition: one wavefront owns one (channel, batch) row and walks
// it in tiles of 64*K consecutive steps.  Lane l holds steps [l*K, l*K+K) of
// the tile, so every global access is a contiguous 64*K*elem-byte stretch
// (float4 loads when T % 4 == 0).  A tile is scanned as
//   1. per-lane serial composition of its K affine maps,
//   2. DPP wave scan of the 64 lane maps (tile entry state folded into lane 0),
//   3. per-lane serial replay from the lane's entry state,
// and the tile's exit state is carried to the next tile in a register.
//
// The backward walks the tiles in reverse: it replays the forward from the
// stored entry state (for the ReLU mask and y[t-1]), runs the adjoint
//   d[t] = e[t] + conj(A[t+1]) d[t+1]
// with the same three-step structure in suffix order, and forms every
// gradient in registers (the reference's _backward, selective_scan_kernel.py:250-462).
#include "rqf_device.h"
#include "rqf_scan.h"

using namespace rqf;

namespace {

constexpr int kSelK = 4;                     // steps per lane per tile
constexpr int kSelTile = kWave * kSelK;      // steps per tile
constexpr int kSelWaves = 4;                 // wavefronts per block

// Wave-uniform per-channel parameters.
struct Chan {
  float bias, theta, lo, span, eta, horizon, thlo, thhi;
  int64_t warp_base;  // element offset of this row's warp logits
};

__device__ __forceinline__ Chan load_chan(const rqf_selective_inputs& p, int64_t f, int64_t b) {
  Chan c;
  c.bias = p.bias[f];
  c.theta = p.theta[f];
  c.lo = p.minimum[f];
  c.span = p.span[f];
  c.eta = p.step[f];
  c.horizon = p.horizon[f];
  c.thlo = p.theta_minimum[f];
  c.thhi = p.theta_maximum[f];
  c.warp_base = p.has_warp ? (p.groups[f] * p.B + b) * p.T : 0;
  return c;
}

// Controller + ZOH + prospective taps for one element
// (rqf_models/ops/selective_scan_kernel.py:16-101).
struct Coef {
  c32 A, phi, bp, bn;  // bp, bn: taps before the write gate
  float gamma, theta, gate, sig, warp, inv_den, ratio;
};

__device__ __forceinline__ void coef(const rqf_selective_inputs& p, const Chan& c, float gv,
                                     float dv, float wv, Coef& e) {
  float gamma = c.bias, sig = 0.0f;
  if (p.has_gamma) {
    if (p.log_shift) {
      sig = ftanh(gv);
      gamma = fexp(fmaf(p.gamma_scale, sig, c.bias));
    } else {
      sig = fsigmoid(c.bias + gv);
      gamma = fmaf(c.span, sig, c.lo);
    }
  }
  float theta = c.theta, warp = 0.0f;
  if (p.has_warp) {
    warp = ftanh(dv);
    theta *= fexp(p.warp_scale * warp);
    if (p.bound_warp) theta = fminf(fmaxf(theta, c.thlo), c.thhi);
  }
  float gate = 1.0f;
  if (p.has_write) gate = p.write_sigmoid ? p.write_max * fsigmoid(wv + p.write_bias) : 1.0f + wv;
  zoh(-gamma * c.eta, (1.0f - gamma) * theta * c.eta, e.A, e.phi, e.inv_den);
  e.bp = cscale(gamma * c.eta, e.phi);
  e.bn = mk(0.0f, 0.0f);
  e.ratio = 0.0f;
  if (p.prospective) {
    e.ratio = p.gamma_horizon ? frcp(gamma) : c.horizon;
    const c32 ex = cscale(e.ratio * gamma, e.A);
    e.bp = cadd(e.bp, ex);
    e.bn = mk(-ex.r, -ex.i);
  }
  e.gamma = gamma;
  e.theta = theta;
  e.gate = gate;
  e.sig = sig;
  e.warp = warp;
}

// ---------------------------------------------------------------------------
// Tile loads / stores.  VEC: T % 4 == 0 and 16-byte aligned bases, so each
// lane's K = 4 steps are either all inside [0, T) or all outside.
// ---------------------------------------------------------------------------
template <bool VEC>
__device__ __forceinline__ void load_c4(const float* __restrict__ row, int64_t tb, int64_t T,
                                        c32 (&v)[kSelK]) {
  if (VEC) {
    if (tb < T) {
      const float4 a = *reinterpret_cast<const float4*>(row + 2 * tb);
      const float4 b = *reinterpret_cast<const float4*>(row + 2 * tb + 4);
      v[0] = mk(a.x, a.y);
      v[1] = mk(a.z, a.w);
      v[2] = mk(b.x, b.y);
      v[3] = mk(b.z, b.w);
    } else {
#pragma unroll
      for (int k = 0; k < kSelK; ++k) v[k] = mk(0.0f, 0.0f);
    }
  } else {
#pragma unroll
    for (int k = 0; k < kSelK; ++k)
      v[k] = (tb + k < T) ? mk(row[2 * (tb + k)], row[2 * (tb + k) + 1]) : mk(0.0f, 0.0f);
  }
}

template <bool VEC>
__device__ __forceinline__ void load_f4(const float* __restrict__ row, int64_t tb, int64_t T,
                                        float (&v)[kSelK]) {
  if (VEC) {
    if (tb < T) {
      const float4 a = *reinterpret_cast<const float4*>(row + tb);
      v[0] = a.x;
      v[1] = a.y;
      v[2] = a.z;
      v[3] = a.w;
    } else {
#pragma unroll
      for (int k = 0; k < kSelK; ++k) v[k] = 0.0f;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kSelK; ++k) v[k] = (tb + k < T) ? row[tb + k] : 0.0f;
  }
}

template <bool VEC>
__device__ __forceinline__ void store_c4(float* __restrict__ row, int64_t tb, int64_t T,
                                         const c32 (&v)[kSelK]) {
  if (VEC) {
    if (tb < T) {
      *reinterpret_cast<float4*>(row + 2 * tb) = make_float4(v[0].r, v[0].i, v[1].r, v[1].i);
      *reinterpret_cast<float4*>(row + 2 * tb + 4) = make_float4(v[2].r, v[2].i, v[3].r, v[3].i);
    }
  } else {
#pragma unroll
    for (int k = 0; k < kSelK; ++k)
      if (tb + k < T) {
        row[2 * (tb + k)] = v[k].r;
        row[2 * (tb + k) + 1] = v[k].i;
      }
  }
}

template <bool VEC>
__device__ __forceinline__ void store_f4(float* __restrict__ row, int64_t tb, int64_t T,
                                         const float (&v)[kSelK]) {
  if (VEC) {
    if (tb < T) *reinterpret_cast<float4*>(row + tb) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int k = 0; k < kSelK; ++k)
      if (tb + k < T) row[tb + k] = v[k];
  }
}

__device__ __forceinline__ c32 relu2(c32 v) { return mk(fmaxf(v.r, 0.0f), fmaxf(v.i, 0.0f)); }

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(kSelWaves* kWave) void selective_fwd_kernel(
    const rqf_selective_inputs p, const float* __restrict__ z, float* __restrict__ raw,
    float* __restrict__ act, float* __restrict__ entries, int64_t chunk, int64_t nc) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * kSelWaves + (threadIdx.x >> 6);
  const int64_t T = p.T;
  if (row >= p.F * p.B) return;  // whole wavefronts exit together
  const int64_t f = row / p.B, b = row - f * p.B;
  const Chan c = load_chan(p, f, b);
  const float* zr = z + 2 * row * T;
  const float* gr = p.has_gamma ? p.gamma_logits + row * T : nullptr;
  const float* wr = p.has_write ? p.write_logits + row * T : nullptr;
  const float* dr = p.has_warp ? p.warp_logits + c.warp_base : nullptr;
  float* rawr = raw ? raw + 2 * row * T : nullptr;
  float* actr = act ? act + 2 * row * T : nullptr;
  float* ent = entries + 2 * row * nc;
  if (lane == 0) {
    ent[0] = 0.0f;
    ent[1] = 0.0f;
  }
  c32 y = mk(0.0f, 0.0f), zlast = mk(0.0f, 0.0f);
  for (int64_t t0 = 0; t0 < T; t0 += kSelTile) {
    const int64_t tb = t0 + lane * kSelK;
    c32 zv[kSelK];
    float gv[kSelK], wv[kSelK], dv[kSelK];
    load_c4<VEC>(zr, tb, T, zv);
    if (gr) load_f4<VEC>(gr, tb, T, gv);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) gv[k] = 0.0f;
    if (wr) load_f4<VEC>(wr, tb, T, wv);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) wv[k] = 0.0f;
    if (dr) load_f4<VEC>(dr, tb, T, dv);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) dv[k] = 0.0f;
    const c32 zp0 = shift_up(zv[kSelK - 1], zlast, lane);

    c32 A[kSelK], u[kSelK];
#pragma unroll
    for (int k = 0; k < kSelK; ++k) {
      Coef e;
      coef(p, c, gv[k], dv[k], wv[k], e);
      c32 drive = cmul(e.bp, zv[k]);
      if (p.prospective) drive = cmad(e.bn, k ? zv[k - 1] : zp0, drive);
      const bool in = tb + k < T;
      A[k] = in ? e.A : mk(1.0f, 0.0f);
      u[k] = in ? cscale(e.gate, drive) : mk(0.0f, 0.0f);
    }
    // 1. lane-local composition
    c32 P = A[0], s = u[0];
#pragma unroll
    for (int k = 1; k < kSelK; ++k) {
      s = cmad(A[k], s, u[k]);
      P = cmul(A[k], P);
    }
    if (lane == 0) s = cmad(P, y, s);
    // 2. wave scan: s becomes the state after the lane's last step
    wave_scan_fwd(P, s);
    // 3. replay from the lane's entry state
    c32 yk = shift_up(s, y, lane);
    c32 out[kSelK];
#pragma unroll
    for (int k = 0; k < kSelK; ++k) {
      yk = cmad(A[k], yk, u[k]);
      out[k] = yk;
      const int64_t t = tb + k;
      if (t + 1 < T && ((t + 1) & (chunk - 1)) == 0) {
        const int64_t j = (t + 1) / chunk;
        ent[2 * j] = yk.r;
        ent[2 * j + 1] = yk.i;
      }
    }
    if (rawr) store_c4<VEC>(rawr, tb, T, out);
    if (actr) {
#pragma unroll
      for (int k = 0; k < kSelK; ++k) out[k] = relu2(out[k]);
      store_c4<VEC>(actr, tb, T, out);
    }
    y = readlane(s, kWave - 1);
    zlast = readlane(zv[kSelK - 1], kWave - 1);
  }
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
struct BwdOut {
  float* dz;   // x-path drive gradient (only written when truncated)
  float* dzw;  // W-path drive gradient (== dz when not truncated)
  float* dg;
  float* ddc;  // per-channel warp gradient (F,B,T) scratch
  float* dw;
  double* partial;  // (2, F*B): sum over t of d/dbias and d/dtheta per row
};

template <bool VEC>
__global__ __launch_bounds__(kSelWaves* kWave) void selective_bwd_kernel(
    const rqf_selective_inputs p, const float* __restrict__ z,
    const float* __restrict__ entries, int64_t chunk, int64_t nc,
    const float* __restrict__ gy, const float* __restrict__ gx, int truncated, BwdOut o) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * kSelWaves + (threadIdx.x >> 6);
  const int64_t T = p.T, R = p.F * p.B;
  if (row >= R) return;
  const int64_t f = row / p.B, b = row - f * p.B;
  const Chan c = load_chan(p, f, b);
  const float* zr = z + 2 * row * T;
  const float* gr = p.has_gamma ? p.gamma_logits + row * T : nullptr;
  const float* wr = p.has_write ? p.write_logits + row * T : nullptr;
  const float* dr = p.has_warp ? p.warp_logits + c.warp_base : nullptr;
  const float* gyr = gy ? gy + 2 * row * T : nullptr;
  const float* gxr = gx ? gx + 2 * row * T : nullptr;
  const float* ent = entries + 2 * row * nc;
  float* dzr = o.dz + 2 * row * T;
  float* dzwr = o.dzw + 2 * row * T;
  float* dgr = o.dg ? o.dg + row * T : nullptr;
  float* dwr = o.dw ? o.dw + row * T : nullptr;
  float* ddr = o.ddc ? o.ddc + row * T : nullptr;

  c32 dcarry = mk(0.0f, 0.0f);   // adjoint (or, truncated, cotangent) at the next tile's first step
  c32 Afirst = mk(0.0f, 0.0f);   // A at the next tile's first step (0 past the end)
  c32 nfirst = mk(0.0f, 0.0f);   // gated lag tap at the next tile's first step
  double sum_bias = 0.0, sum_theta = 0.0;
  const int64_t ntiles = (T + kSelTile - 1) / kSelTile;

  for (int64_t tile = ntiles - 1; tile >= 0; --tile) {
    const int64_t t0 = tile * kSelTile;
    const int64_t tb = t0 + lane * kSelK;
    c32 zv[kSelK], ey[kSelK], ex[kSelK];
    float gv[kSelK], wv[kSelK], dv[kSelK];
    load_c4<VEC>(zr, tb, T, zv);
    if (gr) load_f4<VEC>(gr, tb, T, gv);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) gv[k] = 0.0f;
    if (wr) load_f4<VEC>(wr, tb, T, wv);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) wv[k] = 0.0f;
    if (dr) load_f4<VEC>(dr, tb, T, dv);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) dv[k] = 0.0f;
    if (gyr) load_c4<VEC>(gyr, tb, T, ey);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) ey[k] = mk(0.0f, 0.0f);
    if (gxr) load_c4<VEC>(gxr, tb, T, ex);
    else
#pragma unroll
      for (int k = 0; k < kSelK; ++k) ex[k] = mk(0.0f, 0.0f);
    // z[t0-1] (uniform address) feeds lane 0's lag tap.
    const c32 zprev_tile = t0 > 0 ? mk(zr[2 * (t0 - 1)], zr[2 * (t0 - 1) + 1]) : mk(0.0f, 0.0f);
    const c32 zp0 = shift_up(zv[kSelK - 1], zprev_tile, lane);

    Coef e[kSelK];
    c32 A[kSelK], u[kSelK];
#pragma unroll
    for (int k = 0; k < kSelK; ++k) {
      coef(p, c, gv[k], dv[k], wv[k], e[k]);
      c32 drive = cmul(e[k].bp, zv[k]);
      if (p.prospective) drive = cmad(e[k].bn, k ? zv[k - 1] : zp0, drive);
      const bool in = tb + k < T;
      A[k] = in ? e[k].A : mk(1.0f, 0.0f);
      u[k] = in ? cscale(e[k].gate, drive) : mk(0.0f, 0.0f);
    }
    // Forward replay from the tile's entry state.
    const c32 y0 = mk(ent[2 * (t0 / chunk)], ent[2 * (t0 / chunk) + 1]);
    c32 P = A[0], s = u[0];
#pragma unroll
    for (int k = 1; k < kSelK; ++k) {
      s = cmad(A[k], s, u[k]);
      P = cmul(A[k], P);
    }
    if (lane == 0) s = cmad(P, y0, s);
    wave_scan_fwd(P, s);
    c32 yk = shift_up(s, y0, lane);
    c32 yprev[kSelK], ecot[kSelK];
#pragma unroll
    for (int k = 0; k < kSelK; ++k) {
      yprev[k] = yk;
      yk = cmad(A[k], yk, u[k]);
      // raw-output cotangent, plus the split-ReLU cotangent where raw > 0
      ecot[k] = mk(ey[k].r + (yk.r > 0.0f ? ex[k].r : 0.0f), ey[k].i + (yk.i > 0.0f ? ex[k].i : 0.0f));
    }
    // Neighbour coefficients A[t+1], gated n[t+1] (0 past the end).
    c32 An[kSelK], nn[kSelK];
#pragma unroll
    for (int k = 0; k < kSelK; ++k) {
      const bool in = tb + k < T;
      A[k] = in ? A[k] : mk(0.0f, 0.0f);
      u[k] = in ? cscale(e[k].gate, e[k].bn) : mk(0.0f, 0.0f);  // reuse: gated lag tap
    }
#pragma unroll
    for (int k = 0; k < kSelK - 1; ++k) {
      An[k] = A[k + 1];
      nn[k] = u[k + 1];
    }
    An[kSelK - 1] = shift_down(A[0], Afirst, lane);
    nn[kSelK - 1] = shift_down(u[0], nfirst, lane);
    Afirst = readlane(A[0], 0);
    nfirst = readlane(u[0], 0);

    // Adjoint d[t] = e[t] + conj(A[t+1]) d[t+1]  (truncated: d = e).
    c32 dnext;
    if (truncated) {
      dnext = shift_down(ecot[0], dcarry, lane);
      dcarry = readlane(ecot[0], 0);
    } else {
      c32 Q = mk(1.0f, 0.0f), r = mk(0.0f, 0.0f);
#pragma unroll
      for (int k = kSelK - 1; k >= 0; --k) {
        r = cjmad(An[k], r, ecot[k]);
        Q = cjmul(An[k], Q);
      }
      if (lane == kWave - 1) r = cmad(Q, dcarry, r);
      wave_scan_rev(Q, r, lane);
      dnext = shift_down(r, dcarry, lane);
      dcarry = readlane(r, 0);
    }

    c32 gz[kSelK], gzw[kSelK];
    float gg[kSelK], gw[kSelK], gd[kSelK];
    float tile_bias = 0.0f, tile_theta = 0.0f;
#pragma unroll
    for (int k = kSelK - 1; k >= 0; --k) {
      const Coef& q = e[k];
      const c32 d = truncated ? ecot[k] : cjmad(An[k], dnext, ecot[k]);
      const c32 cur = cjmul(cscale(q.gate, q.bp), d);
      gz[k] = cur;
      gzw[k] = cjmad(nn[k], dnext, cur);
      dnext = d;
      // Gradients of the gated taps and of A.
      const c32 zp = k ? zv[k - 1] : zp0;
      const c32 dp = cjmul(zv[k], d);
      const c32 dn = cjmul(zp, d);
      c32 dA = cjmul(yprev[k], d);
      const float dgate = q.bp.r * dp.r + q.bp.i * dp.i + q.bn.r * dn.r + q.bn.i * dn.i;
      const c32 dbp = cscale(q.gate, dp), dbn = cscale(q.gate, dn);
      float dgamma = 0.0f;
      if (p.prospective) {
        const c32 qd = csub(dbp, dbn);
        if (!p.gamma_horizon) dgamma = q.ratio * (qd.r * q.A.r + qd.i * q.A.i);
        dA = cadd(dA, cscale(q.ratio * q.gamma, qd));
      }
      // phi'(a) = (A - phi)/a, or its series for |a|^2 < 1/64 (cubic below 1e-8);
      // selective_scan_kernel.py:119-148.
      const float ar = -q.gamma * c.eta, ai = (1.0f - q.gamma) * q.theta * c.eta;
      const float den = fmaf(ar, ar, ai * ai);
      c32 fp;
      const c32 a = mk(ar, ai);
      if (den < 0.015625f) {
        if (den < 1.0e-8f) {
          fp = cmad(a, cmad(a, mk(1.0f / 8.0f, 0.0f), mk(1.0f / 3.0f, 0.0f)), mk(0.5f, 0.0f));
        } else {
          c32 sr = mk(1.0f / 45360.0f, 0.0f);
          sr = cmad(a, sr, mk(1.0f / 5760.0f, 0.0f));
          sr = cmad(a, sr, mk(1.0f / 840.0f, 0.0f));
          sr = cmad(a, sr, mk(1.0f / 144.0f, 0.0f));
          sr = cmad(a, sr, mk(1.0f / 30.0f, 0.0f));
          sr = cmad(a, sr, mk(1.0f / 8.0f, 0.0f));
          sr = cmad(a, sr, mk(1.0f / 3.0f, 0.0f));
          fp = cmad(a, sr, mk(0.5f, 0.0f));
        }
      } else {
        const c32 x = csub(q.A, q.phi);
        fp = cscale(q.inv_den, cmul(x, conjg(a)));
      }
      const float gh = q.gamma * c.eta;
      // da = conj(A) dA + gamma*eta*conj(phi') dbp
      const c32 da = cadd(cjmul(q.A, dA), cscale(gh, cjmul(fp, dbp)));
      dgamma += c.eta * (q.phi.r * dbp.r + q.phi.i * dbp.i - da.r - q.theta * da.i);
      float dth = c.eta * (1.0f - q.gamma) * da.i;
      const bool in = tb + k < T;
      // controller chain rules (selective_scan_kernel.py:441-460)
      float dbias;
      if (p.has_gamma) {
        if (p.log_shift) {
          dbias = dgamma * q.gamma;
          gg[k] = dbias * p.gamma_scale * (1.0f - q.sig * q.sig);
        } else {
          dbias = dgamma * c.span * q.sig * (1.0f - q.sig);
          gg[k] = dbias;
        }
      } else {
        dbias = dgamma;
        gg[k] = 0.0f;
      }
      if (p.has_warp) {
        const float scale = fexp(p.warp_scale * q.warp);
        if (p.bound_warp) {
          const float unclamped = c.theta * scale;
          // torch.clamp passes the gradient at both exact edges
          if (!(unclamped >= c.thlo && unclamped <= c.thhi)) dth = 0.0f;
        }
        gd[k] = dth * q.theta * p.warp_scale * (1.0f - q.warp * q.warp);
        dth *= scale;
      } else {
        gd[k] = 0.0f;
      }
      gw[k] = p.write_sigmoid ? dgate * q.gate * (1.0f - q.gate / p.write_max) : dgate;
      tile_bias += in ? dbias : 0.0f;
      tile_theta += in ? dth : 0.0f;
    }
    sum_bias += (double)tile_bias;
    sum_theta += (double)tile_theta;
    store_c4<VEC>(dzwr, tb, T, gzw);
    if (truncated) store_c4<VEC>(dzr, tb, T, gz);
    if (dgr) store_f4<VEC>(dgr, tb, T, gg);
    if (dwr) store_f4<VEC>(dwr, tb, T, gw);
    if (ddr) store_f4<VEC>(ddr, tb, T, gd);
  }
  sum_bias = wave_sum(sum_bias);
  sum_theta = wave_sum(sum_theta);
  if (lane == 0) {
    o.partial[row] = sum_bias;
    o.partial[R + row] = sum_theta;
  }
}

// dd[g, i] = sum over channels f of group g (ascending f) of ddc[f, i], i over B*T.
__global__ __launch_bounds__(256) void group_reduce_kernel(const float* __restrict__ ddc,
                                                           const int64_t* __restrict__ groups,
                                                           float* __restrict__ dd, int64_t F,
                                                           int64_t G, int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  for (int64_t g = 0; g < G; ++g) {
    float acc = 0.0f;
    for (int64_t f = 0; f < F; ++f)
      if (groups[f] == g) acc += ddc[f * N + i];
    dd[g * N + i] = acc;
  }
}

// dbias[f] = sum_b partial[f*B + b] (fp64, ascending b); same for dtheta.
__global__ __launch_bounds__(256) void partial_reduce_kernel(const double* __restrict__ partial,
                                                             float* __restrict__ dbias,
                                                             float* __restrict__ dtheta,
                                                             int64_t F, int64_t B) {
  const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= F) return;
  double sb = 0.0, st = 0.0;
  for (int64_t b = 0; b < B; ++b) {
    sb += partial[f * B + b];
    st += partial[F * B + f * B + b];
  }
  dbias[f] = (float)sb;
  dtheta[f] = (float)st;
}

// Zero-fill of n 32-bit words (graph-capture safe, unlike a memset node).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

void zero_words(void* p, int64_t nwords, hipStream_t s) {
  if (nwords > 0)
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0, s,
                       (uint32_t*)p, nwords);
}

__global__ void wave_scan_selftest_kernel(const float* in, float* out_fwd, float* out_rev) {
  const int lane = lane_id();
  c32 P = mk(in[4 * lane], in[4 * lane + 1]), s = mk(in[4 * lane + 2], in[4 * lane + 3]);
  c32 Q = P, r = s;
  wave_scan_fwd(P, s);
  wave_scan_rev(Q, r, lane);
  out_fwd[4 * lane] = P.r;
  out_fwd[4 * lane + 1] = P.i;
  out_fwd[4 * lane + 2] = s.r;
  out_fwd[4 * lane + 3] = s.i;
  out_rev[4 * lane] = Q.r;
  out_rev[4 * lane + 1] = Q.i;
  out_rev[4 * lane + 2] = r.r;
  out_rev[4 * lane + 3] = r.i;
}

inline bool aligned16(const void* ptr) { return ptr == nullptr || ((uintptr_t)ptr & 15) == 0; }
inline bool aligned8(const void* ptr) { return ptr == nullptr || ((uintptr_t)ptr & 7) == 0; }
inline size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }
inline bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RQF_OK : (int)err;
}

int check_inputs(const rqf_selective_inputs* in) {
  if (!in || in->F < 0 || in->B < 0 || in->T < 0) return RQF_ERR_ARG;
  if (!in->bias || !in->theta || !in->minimum || !in->span || !in->step || !in->horizon ||
      !in->theta_minimum || !in->theta_maximum)
    return RQF_ERR_ARG;
  if (in->has_gamma && !in->gamma_logits) return RQF_ERR_ARG;
  if (in->has_write && !in->write_logits) return RQF_ERR_ARG;
  if (in->has_warp && (!in->warp_logits || !in->groups || in->G < 1)) return RQF_ERR_ARG;
  return RQF_OK;
}

bool vec_ok(const rqf_selective_inputs* in, std::initializer_list<const void*> ptrs) {
  if (in->T % 4) return false;
  if (!aligned16(in->gamma_logits) || !aligned16(in->warp_logits) || !aligned16(in->write_logits))
    return false;
  for (const void* q : ptrs)
    if (!aligned16(q)) return false;
  return true;
}

}  // namespace

extern "C" int rqf_selective_fwd(const rqf_selective_inputs* in, const float* z, int64_t chunk,
                                 float* raw, float* act, float* entries, rqf_stream_t stream) {
  if (!in || in->F < 0 || in->B < 0 || in->T < 0 || !pow2(chunk)) return RQF_ERR_ARG;
  const int64_t R = in->F * in->B;
  if (R == 0 || in->T == 0) return RQF_OK;
  int st = check_inputs(in);
  if (st) return st;
  if (!z || !entries || (!raw && !act)) return RQF_ERR_ARG;
  if (!aligned8(z) || !aligned8(raw) || !aligned8(act) || !aligned8(entries)) return RQF_ERR_ALIGN;
  const int64_t nc = (in->T + chunk - 1) / chunk;
  const dim3 grid((unsigned)((R + kSelWaves - 1) / kSelWaves)), block(kSelWaves * kWave);
  hipStream_t s = (hipStream_t)stream;
  if (vec_ok(in, {z, raw, act}))
    hipLaunchKernelGGL(selective_fwd_kernel<true>, grid, block, 0, s, *in, z, raw, act, entries,
                       chunk, nc);
  else
    hipLaunchKernelGGL(selective_fwd_kernel<false>, grid, block, 0, s, *in, z, raw, act, entries,
                       chunk, nc);
  return launch_status();
}

namespace {
struct SelWs {
  size_t partial, tile_entries, ddc, total;
};
SelWs sel_ws_layout(const rqf_selective_inputs* in, int64_t chunk) {
  SelWs w;
  const int64_t R = in->F * in->B;
  w.partial = 0;
  size_t off = round256(sizeof(double) * 2 * (size_t)R);
  w.tile_entries = off;
  if (chunk > kSelTile) off += round256(sizeof(float) * 2 * (size_t)R * ((in->T + kSelTile - 1) / kSelTile + 1));
  w.ddc = off;
  if (in->has_warp) off += round256(sizeof(float) * (size_t)R * (size_t)in->T);
  w.total = off;
  return w;
}
}  // namespace

extern "C" size_t rqf_selective_bwd_workspace(const rqf_selective_inputs* in, int64_t chunk) {
  if (!in) return 0;
  return sel_ws_layout(in, chunk).total;
}

extern "C" int rqf_selective_bwd(const rqf_selective_inputs* in, const float* z,
                                 const float* entries, int64_t chunk, const float* gy,
                                 const float* gx, int32_t activate, int32_t truncated, float* dz,
                                 float* dzw, float* dg, float* dd, float* dw, float* dbias,
                                 float* dtheta, void* workspace, size_t workspace_bytes,
                                 rqf_stream_t stream) {
  (void)activate;  // the split-ReLU cotangent is gx; its mask is recomputed from raw
  if (!in || in->F < 0 || in->B < 0 || in->T < 0 || !pow2(chunk)) return RQF_ERR_ARG;
  const bool nonempty = in->F * in->B * in->T > 0;
  if (in->F > 0 && (!dbias || !dtheta)) return RQF_ERR_ARG;
  if (nonempty) {
    int st = check_inputs(in);
    if (st) return st;
    if (!z || !entries || !dz || !dzw) return RQF_ERR_ARG;
    if (truncated && dz == dzw) return RQF_ERR_ARG;
    if ((in->has_gamma && !dg) || (in->has_write && !dw) || (in->has_warp && !dd))
      return RQF_ERR_ARG;
  }
  const SelWs w = sel_ws_layout(in, chunk);
  if (workspace_bytes < w.total || (w.total && !workspace)) return RQF_ERR_WORKSPACE;
  if (!aligned8(z) || !aligned8(gy) || !aligned8(gx) || !aligned8(dz) || !aligned8(dzw))
    return RQF_ERR_ALIGN;
  const int64_t R = in->F * in->B, T = in->T;
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  double* partial = (double*)(ws + w.partial);
  if (R > 0 && T > 0) {
    const dim3 grid((unsigned)((R + kSelWaves - 1) / kSelWaves)), block(kSelWaves * kWave);
    const float* ent = entries;
    int64_t ent_chunk = chunk, nc = (T + chunk - 1) / chunk;
    const bool vec = vec_ok(in, {z, gy, gx, dz, dzw, dg, dw});
    if (chunk > kSelTile) {
      // Entry states every tile: replay the forward once with chunk = tile.
      float* te = (float*)(ws + w.tile_entries);
      ent_chunk = kSelTile;
      nc = (T + kSelTile - 1) / kSelTile;
      if (vec)
        hipLaunchKernelGGL(selective_fwd_kernel<true>, grid, block, 0, s, *in, z, nullptr,
                           nullptr, te, ent_chunk, nc);
      else
        hipLaunchKernelGGL(selective_fwd_kernel<false>, grid, block, 0, s, *in, z, nullptr,
                           nullptr, te, ent_chunk, nc);
      ent = te;
    }
    BwdOut o;
    o.dz = dz;
    o.dzw = dzw;
    o.dg = in->has_gamma ? dg : nullptr;
    o.dw = in->has_write ? dw : nullptr;
    o.ddc = in->has_warp ? (float*)(ws + w.ddc) : nullptr;
    o.partial = partial;
    if (vec)
      hipLaunchKernelGGL(selective_bwd_kernel<true>, grid, block, 0, s, *in, z, ent, ent_chunk,
                         nc, gy, gx, (int)truncated, o);
    else
      hipLaunchKernelGGL(selective_bwd_kernel<false>, grid, block, 0, s, *in, z, ent, ent_chunk,
                         nc, gy, gx, (int)truncated, o);
    if (in->has_warp) {
      const int64_t N = in->B * T;
      hipLaunchKernelGGL(group_reduce_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, s,
                         o.ddc, in->groups, dd, in->F, in->G, N);
    }
  } else {
    zero_words(partial, 4 * R, s);
    if (in->has_warp && dd) zero_words(dd, in->G * in->B * T, s);
  }
  if (in->F > 0)
    hipLaunchKernelGGL(partial_reduce_kernel, dim3((unsigned)((in->F + 255) / 256)), dim3(256), 0,
                       s, partial, dbias, dtheta, in->F, in->B);
  return launch_status();
}

extern "C" int rqf_selftest_wave_scan(const float* in, float* out_fwd, float* out_rev,
                                      rqf_stream_t stream) {
  if (!in || !out_fwd || !out_rev) return RQF_ERR_ARG;
  hipLaunchKernelGGL(wave_scan_selftest_kernel, dim3(1), dim3(kWave), 0, (hipStream_t)stream, in,
                     out_fwd, out_rev);
  return launch_status();
}
