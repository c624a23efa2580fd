// timeinv.hip -- time-invariant two-tap scans for gfx950.
//
//   y[t] = c1*y[t-1] + k0*x[t] + k1*x[t-1]      (k1 = 0: plain C2 scan)
//
// Two families:
//
// FBT (channel-outermost, rows contiguous in time): tiles of 64*K steps, lane
// l holding K consecutive steps.  Tile = lane-serial composition -> DPP wave
// scan -> lane-serial replay, as in the selective kernels.  The forward runs
// row blocks (8 wavefronts per row, K = 8); the backward runs one row per
// wavefront (K = 4), or row blocks on 2 KB-aligned rows.  The backward runs
// the adjoint g[t] = e[t] + conj(c1) g[t+1] the same way in suffix order and
// keeps raw[t-1] and g[t+1] in registers, so it needs none of the
// reference's divisions by c1 (fbt_scan_kernel.py:157-160, 518-521).
//
// The same scans in the reference's (batch, time, filters) layout are in
// btf.hip.
//
// Coefficient gradients are reduced deterministically: per-task partial sums
// in fp64, then an ordered reduction per channel.
#include "rqf_device.h"
#include "rqf_scan.h"

#include <atomic>
#include <mutex>

using namespace rqf;

// Scratch of rqf_fbt_recompute_bwd_noalloc: the per-row fp64 partial sums of
// the coefficient gradients (6 doubles per (channel, batch) row), in a static
// device array instead of a caller workspace.  Every GPU the library runs on
// holds its own copy until the process ends.
static __device__ __align__(256) unsigned char scratch[RQF_NOALLOC_SCRATCH_BYTES];

namespace {

// Steps per lane of the one-row-per-wavefront kernels.  4 (a 32-byte stretch
// per lane, 2 KB per wavefront load) streams faster than 8 (64 bytes per
// lane) on gfx950: wider per-lane stretches make each load instruction's
// footprint sparser.  (The row-block kernels move full tiles through LDS, one
// contiguous 1 KB per instruction, and use K = 8.)
#ifndef RQF_TI_K
#define RQF_TI_K 4
#endif

constexpr int kTiK = RQF_TI_K;
constexpr int kTiTile = kWave * kTiK;
constexpr int kTiWaves = 4;

__device__ __forceinline__ c32 ldc(const float* p, int64_t i) { return mk(p[2 * i], p[2 * i + 1]); }
__device__ __forceinline__ void stc(float* p, int64_t i, c32 v) {
  p[2 * i] = v.r;
  p[2 * i + 1] = v.i;
}
__device__ __forceinline__ c32 relu2(c32 v) { return mk(fmaxf(v.r, 0.0f), fmaxf(v.i, 0.0f)); }
__device__ __forceinline__ c32 mask_by(c32 g, c32 raw) {
  return mk(raw.r > 0.0f ? g.r : 0.0f, raw.i > 0.0f ? g.i : 0.0f);
}

// A complex row advanced to step t0 (wave-uniform), its 64-bit offset pinned
// to scalar registers: the LDS-transposed tile I/O then addresses each lane
// from a scalar base plus a 32-bit offset, for rows of any length (a 32-bit
// step offset would overflow past 2^30 steps).
template <class P>
__device__ __forceinline__ P* at_step(P* row, int64_t t0) {
  return row + (int64_t)uniform64((uint64_t)(2 * t0));
}

// VEC: T even and 16-byte aligned rows: a lane's K steps are all in or all out
// of range when T % K == 0; otherwise the tail uses guarded scalar access.
template <bool VEC>
__device__ __forceinline__ void load8(const float* __restrict__ row, int64_t tb, int64_t T,
                                      c32 (&v)[kTiK]) {
  if (VEC && tb + kTiK <= T) {
#pragma unroll
    for (int j = 0; j < kTiK / 2; ++j) {
      const float4 a = *reinterpret_cast<const float4*>(row + 2 * tb + 4 * j);
      v[2 * j] = mk(a.x, a.y);
      v[2 * j + 1] = mk(a.z, a.w);
    }
  } else {
#pragma unroll
    for (int k = 0; k < kTiK; ++k) v[k] = (tb + k < T) ? ldc(row, tb + k) : mk(0.0f, 0.0f);
  }
}
template <bool VEC>
__device__ __forceinline__ void store8(float* __restrict__ row, int64_t tb, int64_t T,
                                       const c32 (&v)[kTiK]) {
  if (VEC && tb + kTiK <= T) {
#pragma unroll
    for (int j = 0; j < kTiK / 2; ++j)
      *reinterpret_cast<float4*>(row + 2 * tb + 4 * j) =
          make_float4(v[2 * j].r, v[2 * j].i, v[2 * j + 1].r, v[2 * j + 1].i);
  } else {
#pragma unroll
    for (int k = 0; k < kTiK; ++k)
      if (tb + k < T) stc(row, tb + k, v[k]);
  }
}

// ---------------------------------------------------------------------------
// The drive z of a row: read from a complex (F*B, T) array, or (L0: layer 0
// on a real input of one feature) formed on the fly as z[f,b,t] = wz[f]
// x[b,t] from the real (B, T) input and the filter's complex weight.  In the
// L0 form every row of one batch element reads the same x row, which stays
// in L2, so the drive costs no HBM traffic of its own.
// ---------------------------------------------------------------------------
struct Drive {
  const float* z;   // complex (F*B, T) (not L0)
  const float* x;   // real (B, T): set for L0, null otherwise
  const float* wz;  // complex (F,) (L0)
};

struct RowDrive {
  const float* zr;  // the row's z
  const float* xr;  // the row's x (L0)
  c32 wz;           // the row's weight (L0)
};

template <bool L0>
__device__ __forceinline__ RowDrive row_drive(const float* z, const float* x, const float* wz,
                                              int64_t row, int64_t f, int64_t B, int64_t T) {
  RowDrive r;
  r.zr = L0 ? nullptr : z + 2 * row * T;
  r.xr = L0 ? x + (row % B) * T : nullptr;
  r.wz = L0 ? ldc(wz, f) : mk(0.0f, 0.0f);
  return r;
}

// z at step t (0 outside [0, T)).
template <bool L0>
__device__ __forceinline__ c32 drive_at(const RowDrive& r, int64_t t, int64_t T) {
  if (t < 0 || t >= T) return mk(0.0f, 0.0f);
  return L0 ? cscale(r.xr[t], r.wz) : ldc(r.zr, t);
}

// z at the lane's K steps [tb, tb + K).  FULL: the whole tile is in range and
// rows are 16-byte aligned (L0: T % 4 == 0 and x aligned; otherwise the
// complex row is aligned and, with LDS, moved through the wavefront's slice).
template <int K, bool L0, bool LDS>
__device__ __forceinline__ void drive_tile(const RowDrive& r, int64_t t0, int64_t tb, int64_t T,
                                           int lane, bool full, float4* io, c32 (&v)[K]) {
  if (L0) {
    if (full) {
      static_assert(K % 4 == 0, "whole float4s of x per lane");
#pragma unroll
      for (int j = 0; j < K / 4; ++j) {
        const float4 q = *reinterpret_cast<const float4*>(r.xr + tb + 4 * j);
        v[4 * j] = cscale(q.x, r.wz);
        v[4 * j + 1] = cscale(q.y, r.wz);
        v[4 * j + 2] = cscale(q.z, r.wz);
        v[4 * j + 3] = cscale(q.w, r.wz);
      }
    } else {
#pragma unroll
      for (int k = 0; k < K; ++k) v[k] = tb + k < T ? cscale(r.xr[tb + k], r.wz) : mk(0.0f, 0.0f);
    }
  } else if (full && LDS) {
    load_c_lds<K>(at_step(r.zr, t0), 0, lane, io, v);
  } else if (full) {
#pragma unroll
    for (int j = 0; j < K / 2; ++j) {
      const float4 q = *reinterpret_cast<const float4*>(r.zr + 2 * tb + 4 * j);
      v[2 * j] = mk(q.x, q.y);
      v[2 * j + 1] = mk(q.z, q.w);
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = (tb + k < T) ? ldc(r.zr, tb + k) : mk(0.0f, 0.0f);
  }
}

// ---------------------------------------------------------------------------
// FBT forward, row-block form: a block of kTfWaves wavefronts owns one row and
// walks it in super-tiles of kTfWaves tiles of kTfTile steps (kTfK per lane),
// wavefront w taking tile w of each, so that concurrent wavefronts stream
// adjacent stretches of the same rows.  Each wavefront scans its tile from a
// zero entry and publishes the tile's map (P, s) in LDS; after one barrier it
// composes the maps of the tiles before it onto the block's carry and replays
// from there.  Full tiles move through a wavefront-private LDS slice (one
// contiguous 1 KB per global instruction).  Entry carries stay at the
// backward's kTiTile granularity.
// ---------------------------------------------------------------------------
#ifndef RQF_TI_FWD_K
#define RQF_TI_FWD_K 8
#endif
#ifndef RQF_TI_FWD_RB_WAVES
#define RQF_TI_FWD_RB_WAVES 8
#endif
constexpr int kTfK = RQF_TI_FWD_K, kTfTile = kWave * kTfK, kTfWaves = RQF_TI_FWD_RB_WAVES;
static_assert(kTfTile % kTiTile == 0, "forward tiles hold whole carry tiles");

// skip (nullable, FBT like z): added to the act output (a residual connection
// around the layer); raw and the carries stay the scan's own states.
template <bool VEC, bool L0 = false>
__global__ __launch_bounds__(kTfWaves* kWave) void fbt_fwd_rb_kernel(
    const float* __restrict__ c1, const float* __restrict__ tap0, const float* __restrict__ tap1,
    const float* __restrict__ z, const float* __restrict__ x, const float* __restrict__ wz,
    const float* __restrict__ skip, float* __restrict__ raw,
    float* __restrict__ act, float* __restrict__ carry, int64_t F, int64_t B, int64_t T,
    int64_t nc) {
  constexpr int K = kTfK, W = kTfWaves;
  __shared__ float4 s_io[W][kTfTile / 2];
  __shared__ float2 s_map[2][W];  // offset of each wavefront's tile map (its power is ptile)
  const int lane = lane_id();
  const int w = wave_id();
  float4* io = &s_io[w][0];
  const int64_t row = blockIdx.x;
  const int64_t f = row / B;
  const c32 a = ldc(c1, f), k0 = ldc(tap0, f), k1 = ldc(tap1, f);
  const c64d A = dpow(widen(a), K);
  const ScanPow pw = scan_pow_fwd(A, lane);
  const c32 pex = narrow(dpow(A, lane));          // power of the lanes before this one
  const c32 ptile = uniform(narrow(dpow(A, kWave)));  // a tile's map
  const RowDrive rd = row_drive<L0>(z, x, wz, row, f, B, T);
  float* rawr = raw ? raw + 2 * row * T : nullptr;
  float* actr = act ? act + 2 * row * T : nullptr;
  const float* skr = skip ? skip + 2 * row * T : nullptr;
  c32 y = mk(0.0f, 0.0f);  // the row's state entering the super-tile
  int parity = 0;
  for (int64_t st0 = 0; st0 < T; st0 += (int64_t)W * kTfTile) {
    const int64_t t0 = st0 + (int64_t)w * kTfTile;
    const bool has = t0 < T;
    const bool full = VEC && t0 + kTfTile <= T;
    const int64_t tb = t0 + lane * K;
    c32 u[K];
    c32 s = mk(0.0f, 0.0f);
    if (has) {
      c32 zv[K];
      drive_tile<K, L0, true>(rd, t0, tb, T, lane, full, io, zv);
      const c32 zlast = drive_at<L0>(rd, t0 - 1, T);
      const c32 zp0 = shift_up(zv[K - 1], zlast, lane);
#pragma unroll
      for (int k = 0; k < K; ++k) u[k] = cmad(k1, k ? zv[k - 1] : zp0, cmul(k0, zv[k]));
#pragma unroll
      for (int k = 0; k < K; ++k) s = cmad(a, s, u[k]);
      wave_scan_fwd_pow(s, pw);  // inclusive prefix offsets of the tile, zero entry
      if (lane == kWave - 1) s_map[parity][w] = make_float2(s.r, s.i);
    }
    __syncthreads();
    c32 ye = y, yr = y;
    for (int v = 0; v < W && st0 + (int64_t)v * kTfTile < T; ++v) {
      if (v == w) ye = yr;
      const float2 m = s_map[parity][v];
      yr = cmad(ptile, yr, mk(m.x, m.y));
    }
    if (has) {
      const c32 sex = shift_up(s, mk(0.0f, 0.0f), lane);
      c32 yk = cmad(pex, ye, sex);
      c32 out[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        yk = cmad(a, yk, u[k]);
        out[k] = yk;
      }
      if (carry) {
        // Carry tiles of kTiTile steps: the state entering each one.
        const int64_t c0 = t0 / kTiTile;
        if (lane == 0) stc(carry, row * nc + c0, ye);
        constexpr int kLanesPerCarry = kTiTile / K;
        if (lane % kLanesPerCarry == kLanesPerCarry - 1 && lane != kWave - 1) {
          const int64_t ci = c0 + (lane + 1) / kLanesPerCarry;
          if (ci * kTiTile < T) stc(carry, row * nc + ci, out[K - 1]);
        }
      }
      if (rawr) {
        if (full) {
          store_c_lds<K>(at_step(rawr, t0), 0, lane, io, out);
        } else {
#pragma unroll
          for (int k = 0; k < K; ++k)
            if (tb + k < T) stc(rawr, tb + k, out[k]);
        }
      }
      if (actr) {
#pragma unroll
        for (int k = 0; k < K; ++k) out[k] = relu2(out[k]);
        if (skr) {
          c32 sk[K];
          if (full) {
            load_c_lds<K>(at_step(skr, t0), 0, lane, io, sk);
          } else {
#pragma unroll
            for (int k = 0; k < K; ++k) sk[k] = (tb + k < T) ? ldc(skr, tb + k) : mk(0.0f, 0.0f);
          }
#pragma unroll
          for (int k = 0; k < K; ++k) out[k] = cadd(out[k], sk[k]);
        }
        if (full) {
          store_c_lds<K>(at_step(actr, t0), 0, lane, io, out);
        } else {
#pragma unroll
          for (int k = 0; k < K; ++k)
            if (tb + k < T) stc(actr, tb + k, out[k]);
        }
      }
    }
    y = yr;
    parity ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Row-block backward.  A block of kRbWaves wavefronts owns one row and walks
// it in super-tiles of kRbWaves consecutive tiles of kTbTile steps (kTbK per
// lane), wavefront w taking tile w of each, so concurrent wavefronts stream
// adjacent stretches of the same rows; full tiles move through a
// wavefront-private LDS slice (one contiguous 1 KB per global instruction).
// When the row stride is a multiple of 2 KB (T a multiple of kTiTile) the
// one-row-per-wavefront form's concurrent streams sit at aliased offsets and
// lose 3-4%; there this form is faster (config 5 backward: 0.353 ms one row
// per wavefront, 0.341 with 4 waves x 256-step tiles, 0.330 with 4 waves x
// 512-step tiles through LDS, 0.390 with 8 waves x 512 steps through LDS).  On
// unaligned rows the per-row form stays ahead (config 2: 0.353 against 0.359)
// and is kept.  The forward states of a tile come from its stored entry
// (REPLAY) or from raw, so only the adjoint needs the block scan: each
// wavefront scans its tile from a zero carry and publishes the tile's suffix
// map (Q, r) in LDS; after one barrier every wavefront composes the maps of
// the tiles after it onto the block's adjoint carry.  Map slots are
// double-buffered, so one barrier per super-tile suffices.
// ---------------------------------------------------------------------------
#ifndef RQF_TI_RB_WAVES
#define RQF_TI_RB_WAVES 4
#endif
#ifndef RQF_TI_BWD_K
#define RQF_TI_BWD_K 8
#endif
constexpr int kTbK = RQF_TI_BWD_K, kTbTile = kWave * kTbK;
static_assert(kTbTile % kTiTile == 0, "backward tiles start on carry tiles");
constexpr int kRbWaves = RQF_TI_RB_WAVES;

// Super-tiles are walked from the end; wavefront w takes tile w of each.
// Complex tile of K steps per lane: full tiles through the wavefront's LDS
// slice, partial tiles element by element.
template <int K>
__device__ __forceinline__ void ld_tile(const float* __restrict__ row, int64_t t0, int64_t tb,
                                        int64_t T, int lane, bool full, float4* io, c32 (&v)[K]) {
  if (full) {
    load_c_lds<K>(at_step(row, t0), 0, lane, io, v);
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = (tb + k < T) ? ldc(row, tb + k) : mk(0.0f, 0.0f);
  }
}
template <int K>
__device__ __forceinline__ void st_tile(float* __restrict__ row, int64_t t0, int64_t tb, int64_t T,
                                        int lane, bool full, float4* io, const c32 (&v)[K]) {
  if (full) {
    store_c_lds<K>(at_step(row, t0), 0, lane, io, v);
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (tb + k < T) stc(row, tb + k, v[k]);
  }
}

// Super-tiles are walked from the end; wavefront w takes tile w of each.
template <bool VEC, bool REPLAY, bool L0 = false>
__global__ __launch_bounds__(kRbWaves* kWave) void fbt_bwd_rb_kernel(
    const float* __restrict__ c1, const float* __restrict__ tap0, const float* __restrict__ tap1,
    const float* __restrict__ z, const float* __restrict__ x, const float* __restrict__ wz,
    const float* __restrict__ raw, const float* __restrict__ carry,
    const float* __restrict__ gout, int mask, float* __restrict__ gz,
    double* __restrict__ partial, int64_t F, int64_t B, int64_t T, int64_t nc) {
  constexpr int K = kTbK, TILE = kTbTile, W = kRbWaves;
  __shared__ float2 s_map[2][W];  // offset of each wavefront's tile suffix map (power ptile)
  __shared__ double s_part[W][6];
  __shared__ float4 s_io[W][TILE / 2];
  const int lane = lane_id();
  const int w = wave_id();
  float4* io = &s_io[w][0];
  const int64_t row = blockIdx.x;
  const int64_t f = row / B;
  const c32 a = ldc(c1, f), k0 = ldc(tap0, f), k1 = ldc(tap1, f);
  const c32 ac = conjg(a);
  const c64d A = dpow(widen(a), K), Ac = dconj(A);
  const ScanPow pf = scan_pow_fwd(A, lane);  // the replay's forward scan; in-row adjoint powers
  const RevPow pr = scan_pow_rev(A, lane);
  const c32 psfx = narrow(dpow(Ac, kWave - lane));     // this lane and the ones after it
  const c32 ptile = uniform(narrow(dpow(Ac, kWave)));  // a whole tile
  const RowDrive rd = row_drive<L0>(z, x, wz, row, f, B, T);
  const float* rr = REPLAY ? nullptr : raw + 2 * row * T;
  const float* gr = gout + 2 * row * T;
  float* gzr = gz + 2 * row * T;
  c32 gcarry = mk(0.0f, 0.0f);  // adjoint entering the super-tile from later times
  double s1r = 0, s1i = 0, s0r = 0, s0i = 0, s2r = 0, s2i = 0;
  const int64_t ntiles = (T + TILE - 1) / TILE;
  const int64_t nsuper = (ntiles + W - 1) / W;
  int parity = 0;
  for (int64_t sti = nsuper - 1; sti >= 0; --sti) {
    const int64_t tile = sti * W + w;
    const int64_t t0 = tile * TILE;
    const bool has = t0 < T;
    const bool full = VEC && t0 + TILE <= T;
    const int64_t tb = t0 + lane * K;
    const int cnt = (int)min<int64_t>(max<int64_t>(T - tb, 0), K);
    c32 zv[K], yv[K], ev[K];
    c32 zp0 = mk(0.0f, 0.0f), yp0 = mk(0.0f, 0.0f);
    c32 r = mk(0.0f, 0.0f);
    if (has) {
      drive_tile<K, L0, true>(rd, t0, tb, T, lane, full, io, zv);
      ld_tile<K>(gr, t0, tb, T, lane, full, io, ev);
      const c32 zprev_tile = drive_at<L0>(rd, t0 - 1, T);
      zp0 = shift_up(zv[K - 1], zprev_tile, lane);
      if (REPLAY) {
        c32 u[K];
#pragma unroll
        for (int k = 0; k < K; ++k) u[k] = cmad(k1, k ? zv[k - 1] : zp0, cmul(k0, zv[k]));
        const c32 y0 = ldc(carry, row * nc + t0 / kTiTile);  // carries every kTiTile steps
        c32 s = mk(0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < K; ++k) s = cmad(a, s, u[k]);
        if (lane == 0) s = cmad(pf.p[0], y0, s);
        wave_scan_fwd_pow(s, pf);
        c32 yk = shift_up(s, y0, lane);
        yp0 = yk;
#pragma unroll
        for (int k = 0; k < K; ++k) {
          yk = cmad(a, yk, u[k]);
          yv[k] = yk;
        }
      } else {
        ld_tile<K>(rr, t0, tb, T, lane, full, io, yv);
        const c32 rprev_tile = t0 > 0 ? ldc(rr, t0 - 1) : mk(0.0f, 0.0f);
        yp0 = shift_up(yv[K - 1], rprev_tile, lane);
      }
      if (mask) {
#pragma unroll
        for (int k = 0; k < K; ++k) ev[k] = mask_by(ev[k], yv[k]);
      }
      // Suffix composition of g -> e + conj(a) g over the lane's steps (zero
      // cotangent past the end of the row).
#pragma unroll
      for (int k = K - 1; k >= 0; --k) r = cmad(ac, r, ev[k]);
      wave_scan_rev_pow(r, pf, pr, lane);  // inclusive suffix over lanes, zero carry
    }
    // Tiles past the end publish a zero offset; they only occur in the first
    // super-tile walked, whose carry is zero, so the tile power applies alike.
    if (lane == 0) s_map[parity][w] = make_float2(r.r, r.i);
    __syncthreads();
    c32 gin = gcarry;  // adjoint entering this tile from its end
    for (int v = W - 1; v > w; --v) {
      const float2 m = s_map[parity][v];
      gin = cmad(ptile, gin, mk(m.x, m.y));
    }
    c32 gn = gin;  // the next (earlier) super-tile's carry
    for (int v = w; v >= 0; --v) {
      const float2 m = s_map[parity][v];
      gn = cmad(ptile, gn, mk(m.x, m.y));
    }
    if (has) {
      c32 gnext = shift_down(cmad(psfx, gin, r), gin, lane);
      c32 go[K];
      float a1r = 0, a1i = 0, a0r = 0, a0i = 0, a2r = 0, a2i = 0;
#pragma unroll
      for (int k = K - 1; k >= 0; --k) {
        const c32 g = cmad(ac, gnext, ev[k]);
        go[k] = cjmad(k1, gnext, cjmul(k0, g));
        const c32 yp = k ? yv[k - 1] : yp0;
        const c32 zp = k ? zv[k - 1] : zp0;
        const c32 t1 = cjmul(yp, g), t0c = cjmul(zv[k], g), t2 = cjmul(zp, g);
        const bool in = k < cnt;
        a1r += in ? t1.r : 0.0f;
        a1i += in ? t1.i : 0.0f;
        a0r += in ? t0c.r : 0.0f;
        a0i += in ? t0c.i : 0.0f;
        a2r += in ? t2.r : 0.0f;
        a2i += in ? t2.i : 0.0f;
        gnext = g;
      }
      st_tile<K>(gzr, t0, tb, T, lane, full, io, go);
      s1r += a1r;
      s1i += a1i;
      s0r += a0r;
      s0i += a0i;
      s2r += a2r;
      s2i += a2i;
    }
    gcarry = gn;
    parity ^= 1;
  }
  // Per-wavefront sums, then the wavefronts in a fixed order.
  const double sums[6] = {wave_sum(s1r), wave_sum(s1i), wave_sum(s0r),
                          wave_sum(s0i), wave_sum(s2r), wave_sum(s2i)};
  if (lane == 0)
    for (int j = 0; j < 6; ++j) s_part[w][j] = sums[j];
  __syncthreads();
  if (threadIdx.x < 6) {
    double t = 0.0;
    for (int v = 0; v < W; ++v) t += s_part[v][threadIdx.x];
    partial[6 * row + threadIdx.x] = t;
  }
}

// ---------------------------------------------------------------------------
// FBT backward.  REPLAY: raw recomputed from the per-tile carry; otherwise raw
// is read.  MASK: cotangent is on the split-ReLU output.
// partial: per row, 6 doubles (gc1.re, gc1.im, gk0.re, gk0.im, gk1.re, gk1.im).
// ---------------------------------------------------------------------------
template <bool VEC, bool REPLAY, bool L0 = false>
__global__ __launch_bounds__(kTiWaves* kWave) void fbt_bwd_kernel(
    const float* __restrict__ c1, const float* __restrict__ tap0, const float* __restrict__ tap1,
    const float* __restrict__ z, const float* __restrict__ x, const float* __restrict__ wz,
    const float* __restrict__ raw, const float* __restrict__ carry,
    const float* __restrict__ gout, int mask, float* __restrict__ gz,
    double* __restrict__ partial, int64_t F, int64_t B, int64_t T, int64_t nc) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * kTiWaves + wave_id();
  if (row >= F * B) return;
  const int64_t f = row / B;
  const c32 a = ldc(c1, f), k0 = ldc(tap0, f), k1 = ldc(tap1, f);
  const c32 ac = conjg(a);
  const c64d A = dpow(widen(a), kTiK);
  const ScanPow pf = scan_pow_fwd(A, lane);  // the replay's forward scan; in-row adjoint powers
  const RevPow pr = scan_pow_rev(A, lane);
  const RowDrive rd = row_drive<L0>(z, x, wz, row, f, B, T);
  const float* rr = REPLAY ? nullptr : raw + 2 * row * T;
  const float* gr = gout + 2 * row * T;
  float* gzr = gz + 2 * row * T;
  c32 gcarry = mk(0.0f, 0.0f);
  double s1r = 0, s1i = 0, s0r = 0, s0i = 0, s2r = 0, s2i = 0;
  const int64_t ntiles = (T + kTiTile - 1) / kTiTile;
  // The lane's kTiK drive values from step tb (per-lane range check, as load8).
  auto load_z = [&](int64_t tb, c32(&v)[kTiK]) {
    drive_tile<kTiK, L0, false>(rd, 0, tb, T, lane, VEC && tb + kTiK <= T, nullptr, v);
  };
  // The previous tile's (in walk order: next) drive and cotangent are loaded
  // before this tile's scans (software pipeline).
  c32 znext[kTiK], enext[kTiK];
  load_z((ntiles - 1) * kTiTile + lane * kTiK, znext);
  load8<VEC>(gr, (ntiles - 1) * kTiTile + lane * kTiK, T, enext);
  for (int64_t tile = ntiles - 1; tile >= 0; --tile) {
    const int64_t t0 = tile * kTiTile;
    const int64_t tb = t0 + lane * kTiK;
    const int cnt = (int)min<int64_t>(max<int64_t>(T - tb, 0), kTiK);
    c32 zv[kTiK], yv[kTiK], ev[kTiK];
#pragma unroll
    for (int k = 0; k < kTiK; ++k) {
      zv[k] = znext[k];
      ev[k] = enext[k];
    }
    if (tile > 0) {
      load_z(tb - kTiTile, znext);
      load8<VEC>(gr, tb - kTiTile, T, enext);
    }
    const c32 zprev_tile = drive_at<L0>(rd, t0 - 1, T);
    const c32 zp0 = shift_up(zv[kTiK - 1], zprev_tile, lane);
    c32 yp0;
    if (REPLAY) {
      c32 u[kTiK];
#pragma unroll
      for (int k = 0; k < kTiK; ++k) u[k] = cmad(k1, k ? zv[k - 1] : zp0, cmul(k0, zv[k]));
      const c32 y0 = ldc(carry, row * nc + tile);
      c32 s = mk(0.0f, 0.0f);
#pragma unroll
      for (int k = 0; k < kTiK; ++k) s = cmad(a, s, u[k]);
      if (lane == 0) s = cmad(pf.p[0], y0, s);
      wave_scan_fwd_pow(s, pf);
      c32 yk = shift_up(s, y0, lane);
      yp0 = yk;
#pragma unroll
      for (int k = 0; k < kTiK; ++k) {
        yk = cmad(a, yk, u[k]);
        yv[k] = yk;
      }
    } else {
      load8<VEC>(rr, tb, T, yv);
      const c32 rprev_tile = t0 > 0 ? ldc(rr, t0 - 1) : mk(0.0f, 0.0f);
      yp0 = shift_up(yv[kTiK - 1], rprev_tile, lane);
    }
    if (mask) {
#pragma unroll
      for (int k = 0; k < kTiK; ++k) ev[k] = mask_by(ev[k], yv[k]);
    }
    // Suffix composition of g -> e + conj(a) g over the lane's steps (zero
    // cotangent past the end of the row).
    c32 r = mk(0.0f, 0.0f);
#pragma unroll
    for (int k = kTiK - 1; k >= 0; --k) r = cmad(ac, r, ev[k]);
    if (lane == kWave - 1) r = cjmad(pf.p[0], gcarry, r);
    wave_scan_rev_pow(r, pf, pr, lane);
    c32 gnext = shift_down(r, gcarry, lane);
    gcarry = readlane(r, 0);
    c32 go[kTiK];
    float a1r = 0, a1i = 0, a0r = 0, a0i = 0, a2r = 0, a2i = 0;
#pragma unroll
    for (int k = kTiK - 1; k >= 0; --k) {
      const c32 g = cmad(ac, gnext, ev[k]);
      go[k] = cjmad(k1, gnext, cjmul(k0, g));
      const c32 yp = k ? yv[k - 1] : yp0;
      const c32 zp = k ? zv[k - 1] : zp0;
      const c32 t1 = cjmul(yp, g), t0c = cjmul(zv[k], g), t2 = cjmul(zp, g);
      const bool in = k < cnt;
      a1r += in ? t1.r : 0.0f;
      a1i += in ? t1.i : 0.0f;
      a0r += in ? t0c.r : 0.0f;
      a0i += in ? t0c.i : 0.0f;
      a2r += in ? t2.r : 0.0f;
      a2i += in ? t2.i : 0.0f;
      gnext = g;
    }
    store8<VEC>(gzr, tb, T, go);
    s1r += a1r;
    s1i += a1i;
    s0r += a0r;
    s0i += a0i;
    s2r += a2r;
    s2i += a2i;
  }
  s1r = wave_sum(s1r);
  s1i = wave_sum(s1i);
  s0r = wave_sum(s0r);
  s0i = wave_sum(s0i);
  s2r = wave_sum(s2r);
  s2i = wave_sum(s2i);
  if (lane == 0) {
    double* o = partial + 6 * row;
    o[0] = s1r;
    o[1] = s1i;
    o[2] = s0r;
    o[3] = s0i;
    o[4] = s2r;
    o[5] = s2i;
  }
}

// grad[f] = sum over m of partial[6*(f*stride_f + m*stride_m) + j] in fp64:
// one wavefront per channel, lane l sums m = l, l+64, ... in order, then a
// fixed-shape wave reduction (deterministic).  FBT layout: stride_f = M,
// stride_m = 1.
__global__ __launch_bounds__(kWave) void coef_reduce_kernel(const double* __restrict__ partial,
                                                            int64_t F, int64_t M, int64_t stride_f,
                                                            int64_t stride_m,
                                                            float* __restrict__ gc1,
                                                            float* __restrict__ gk0,
                                                            float* __restrict__ gk1) {
  const int lane = threadIdx.x;
  for (int64_t f = blockIdx.x; f < F; f += gridDim.x) {
    double s[6] = {0, 0, 0, 0, 0, 0};
    for (int64_t m = lane; m < M; m += kWave) {
      const double* p = partial + 6 * (f * stride_f + m * stride_m);
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

inline bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; }
inline bool aligned8(const void* p) { return p == nullptr || ((uintptr_t)p & 7) == 0; }
inline bool aligned4(const void* p) { return p == nullptr || ((uintptr_t)p & 3) == 0; }
inline size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RQF_OK : (int)err;
}

// z may also come as the layer-0 drive (drv.x set: z = wz[f] x[b, t]).
int fbt_fwd(const float* c1, const float* t0, const float* t1, Drive drv, const float* skip,
            float* raw, float* act, float* carry, int64_t F, int64_t B, int64_t T,
            hipStream_t s) {
  if (F < 0 || B < 0 || T < 0) return RQF_ERR_ARG;
  const int64_t R = F * B;
  if (R == 0 || T == 0) return RQF_OK;
  const bool l0 = drv.x != nullptr;
  if (!c1 || !t0 || !t1 || (l0 ? !drv.wz : !drv.z) || (!raw && !act))
    return RQF_ERR_ARG;
  if (!aligned8(drv.z) || !aligned8(drv.wz) || !aligned4(drv.x) || !aligned8(skip) ||
      !aligned8(raw) || !aligned8(act) || !aligned8(carry))
    return RQF_ERR_ALIGN;
  if (skip && !act) return RQF_ERR_ARG;
  if (!grid_fits(R, kTfWaves * kWave)) return RQF_ERR_ARG;
  const int64_t nc = (T + kTiTile - 1) / kTiTile;
  const bool vec = T % 2 == 0 && (l0 ? T % 4 == 0 && aligned16(drv.x) : aligned16(drv.z)) &&
                   aligned16(skip) && aligned16(raw) && aligned16(act);
  {
    const dim3 grid((unsigned)R), block(kTfWaves * kWave);
    if (l0 && vec)
      hipLaunchKernelGGL((fbt_fwd_rb_kernel<true, true>), grid, block, 0, s, c1, t0, t1, drv.z, drv.x, drv.wz,
                         skip, raw, act, carry, F, B, T, nc);
    else if (l0)
      hipLaunchKernelGGL((fbt_fwd_rb_kernel<false, true>), grid, block, 0, s, c1, t0, t1, drv.z, drv.x, drv.wz,
                         skip, raw, act, carry, F, B, T, nc);
    else if (vec)
      hipLaunchKernelGGL((fbt_fwd_rb_kernel<true, false>), grid, block, 0, s, c1, t0, t1, drv.z, drv.x, drv.wz,
                         skip, raw, act, carry, F, B, T, nc);
    else
      hipLaunchKernelGGL((fbt_fwd_rb_kernel<false, false>), grid, block, 0, s, c1, t0, t1, drv.z, drv.x, drv.wz,
                         skip, raw, act, carry, F, B, T, nc);
  }
  return launch_status();
}

size_t fbt_ws(int64_t F, int64_t B) { return round256(sizeof(double) * 6 * (size_t)(F * B)); }

template <bool L0>
void launch_fbt_bwd_kernels(bool rowblock, bool vec, const float* c1, const float* t0,
                            const float* t1, Drive drv, const float* raw, const float* carry,
                            const float* gout, int mask, float* gz, double* partial, int64_t F,
                            int64_t B, int64_t T, int64_t nc, hipStream_t s) {
  const int64_t R = F * B;
  const dim3 grid = rowblock ? dim3((unsigned)R) : dim3((unsigned)((R + kTiWaves - 1) / kTiWaves));
  const dim3 block = rowblock ? dim3(kRbWaves * kWave) : dim3(kTiWaves * kWave);
#define RQF_FBT_BWD(KERNEL, V, REPLAY)                                                         \
  hipLaunchKernelGGL((KERNEL<V, REPLAY, L0>), grid, block, 0, s, c1, t0, t1, drv.z, drv.x,      \
                     drv.wz, raw, carry, gout, mask, gz, partial, F, B, T, nc)
  // The layer-0 drive comes only with the recompute form (carries, no raw).
  if (rowblock) {
    if (carry) {
      if (vec) RQF_FBT_BWD(fbt_bwd_rb_kernel, true, true);
      else RQF_FBT_BWD(fbt_bwd_rb_kernel, false, true);
    } else if constexpr (!L0) {
      if (vec) RQF_FBT_BWD(fbt_bwd_rb_kernel, true, false);
      else RQF_FBT_BWD(fbt_bwd_rb_kernel, false, false);
    }
  } else if (carry) {
    if (vec) RQF_FBT_BWD(fbt_bwd_kernel, true, true);
    else RQF_FBT_BWD(fbt_bwd_kernel, false, true);
  } else if constexpr (!L0) {
    if (vec) RQF_FBT_BWD(fbt_bwd_kernel, true, false);
    else RQF_FBT_BWD(fbt_bwd_kernel, false, false);
  }
#undef RQF_FBT_BWD
}

// z may also come as the layer-0 drive (drv.x set: z = wz[f] x[b, t]).
int fbt_bwd(const float* c1, const float* t0, const float* t1, Drive drv, const float* raw,
            const float* carry, const float* gout, int mask, float* gz, float* gc1, float* gt0,
            float* gt1, int64_t F, int64_t B, int64_t T, void* ws, size_t ws_bytes,
            hipStream_t s) {
  if (F < 0 || B < 0 || T < 0) return RQF_ERR_ARG;
  if (F == 0) return RQF_OK;
  if (!gc1 || !gt0 || !gt1) return RQF_ERR_ARG;
  const bool l0 = drv.x != nullptr;
  if (B * T > 0 && (!c1 || !t0 || !t1 || (l0 ? !drv.wz : !drv.z) || !gout || !gz ||
                    (!raw && !carry)))
    return RQF_ERR_ARG;
  if (!aligned8(drv.z) || !aligned8(drv.wz) || !aligned4(drv.x) || !aligned8(raw) ||
      !aligned8(gout) || !aligned8(gz))
    return RQF_ERR_ALIGN;
  const int64_t R = F * B;
  // the row-block backward on 2 KB-aligned rows, the per-row one otherwise
  const bool rowblock = T % kTiTile == 0;
  if (R > 0 && T > 0 &&
      !(rowblock ? grid_fits(R, kRbWaves * kWave)
                 : grid_fits((R + kTiWaves - 1) / kTiWaves, kTiWaves * kWave)))
    return RQF_ERR_ARG;
  const size_t need = fbt_ws(F, B);
  if (need && (!ws || ws_bytes < need)) return RQF_ERR_WORKSPACE;
  double* partial = (double*)ws;
  if (R > 0 && T > 0) {
    const int64_t nc = (T + kTiTile - 1) / kTiTile;
    const bool vec = T % 2 == 0 && (l0 ? T % 4 == 0 && aligned16(drv.x) : aligned16(drv.z)) &&
                     aligned16(raw) && aligned16(gout) && aligned16(gz);
    if (l0)
      launch_fbt_bwd_kernels<true>(rowblock, vec, c1, t0, t1, drv, raw, carry, gout, mask, gz,
                                   partial, F, B, T, nc, s);
    else
      launch_fbt_bwd_kernels<false>(rowblock, vec, c1, t0, t1, drv, raw, carry, gout, mask, gz,
                                    partial, F, B, T, nc, s);
    hipLaunchKernelGGL(coef_reduce_kernel, dim3(stride_blocks(F)), dim3(kWave), 0, s,
                       partial, F, B, B, (int64_t)1, gc1, gt0, gt1);
  } else {
    hipLaunchKernelGGL(coef_reduce_kernel, dim3(stride_blocks(F)), dim3(kWave), 0, s,
                       partial, F, (int64_t)0, B, (int64_t)1, gc1, gt0, gt1);
  }
  return launch_status();
}

// Device address of `scratch` on the device that runs `stream`.  The host
// name of the array is only a stand-in for it, so the address is looked up
// once per device with hipGetSymbolAddress (that device current) and kept.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return RQF_ERR_ARG;
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      int cur = -1;
      if ((e = hipGetDevice(&cur)) != hipSuccess) return (int)e;
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      const hipError_t back = cur != dev ? hipSetDevice(cur) : hipSuccess;
      if (e != hipSuccess) return (int)e;
      if (back != hipSuccess) return (int)back;
      if (!ptr) return RQF_ERR_SCRATCH;
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return RQF_OK;
}

}  // namespace

// ------------------------------- C ABI ------------------------------------

extern "C" int64_t rqf_fbt_carry_chunks(int64_t T) { return T > 0 ? (T + kTiTile - 1) / kTiTile : 0; }

extern "C" size_t rqf_fbt_workspace(int64_t F, int64_t B, int64_t T) {
  (void)T;
  return fbt_ws(F, B);
}

extern "C" int rqf_fbt_prospective_fwd(const float* c1, const float* tap0, const float* tap1,
                                       const float* z, float* raw, float* act, int64_t F,
                                       int64_t B, int64_t T, rqf_stream_t stream) {
  if (!raw && F * B * T > 0) return RQF_ERR_ARG;
  return fbt_fwd(c1, tap0, tap1, Drive{z, nullptr, nullptr}, nullptr, raw, act, nullptr, F, B, T, (hipStream_t)stream);
}

extern "C" int rqf_fbt_prospective_bwd(const float* c1, const float* tap0, const float* tap1,
                                       const float* z, const float* raw, const float* grad_out,
                                       int32_t fuse_act, float* grad_z, float* grad_c1,
                                       float* grad_tap0, float* grad_tap1, int64_t F, int64_t B,
                                       int64_t T, void* ws, size_t ws_bytes, rqf_stream_t stream) {
  if (!raw && F * B * T > 0) return RQF_ERR_ARG;
  return fbt_bwd(c1, tap0, tap1, Drive{z, nullptr, nullptr}, raw, nullptr, grad_out, fuse_act, grad_z, grad_c1, grad_tap0,
                 grad_tap1, F, B, T, ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int rqf_fbt_recompute_fwd(const float* c1, const float* tap0, const float* tap1,
                                     const float* z, float* act, float* carry, int64_t F,
                                     int64_t B, int64_t T, rqf_stream_t stream) {
  if ((!act || !carry) && F * B * T > 0) return RQF_ERR_ARG;
  return fbt_fwd(c1, tap0, tap1, Drive{z, nullptr, nullptr}, nullptr, nullptr, act, carry, F, B, T, (hipStream_t)stream);
}

extern "C" int rqf_fbt_recompute_skip_fwd(const float* c1, const float* tap0, const float* tap1,
                                          const float* z, const float* skip, float* act,
                                          float* carry, int64_t F, int64_t B, int64_t T,
                                          rqf_stream_t stream) {
  if ((!act || !carry || !skip) && F * B * T > 0) return RQF_ERR_ARG;
  return fbt_fwd(c1, tap0, tap1, Drive{z, nullptr, nullptr}, skip, nullptr, act, carry, F, B, T, (hipStream_t)stream);
}

extern "C" int rqf_fbt_recompute_bwd(const float* c1, const float* tap0, const float* tap1,
                                     const float* z, const float* carry, const float* grad_out,
                                     float* grad_z, float* grad_c1, float* grad_tap0,
                                     float* grad_tap1, int64_t F, int64_t B, int64_t T, void* ws,
                                     size_t ws_bytes, rqf_stream_t stream) {
  if (!carry && F * B * T > 0) return RQF_ERR_ARG;
  return fbt_bwd(c1, tap0, tap1, Drive{z, nullptr, nullptr}, nullptr, carry, grad_out, 1, grad_z, grad_c1, grad_tap0,
                 grad_tap1, F, B, T, ws, ws_bytes, (hipStream_t)stream);
}

extern "C" int rqf_fbt_recompute_bwd_noalloc(const float* c1, const float* tap0,
                                             const float* tap1, const float* z,
                                             const float* carry, const float* grad_out,
                                             float* grad_z, float* grad_c1, float* grad_tap0,
                                             float* grad_tap1, int64_t F, int64_t B, int64_t T,
                                             rqf_stream_t stream) {
  if (F < 0 || B < 0 || T < 0) return RQF_ERR_ARG;
  // Size check first, before any pointer is looked at or any HIP call made.
  constexpr int64_t kMaxRows = (int64_t)(RQF_NOALLOC_SCRATCH_BYTES / (6 * sizeof(double)));
  if (B > 0 && F > kMaxRows / B) return RQF_ERR_SCRATCH;
  if (F == 0) return RQF_OK;
  if (!carry && F * B * T > 0) return RQF_ERR_ARG;
  const size_t need = fbt_ws(F, B);
  void* ws = nullptr;
  if (need) {
    const int st = scratch_address((hipStream_t)stream, &ws);
    if (st) return st;
  }
  // Every row's partial slot is written before the ordered reduction reads
  // it (same stream), so nothing is cleared.
  return fbt_bwd(c1, tap0, tap1, Drive{z, nullptr, nullptr}, nullptr, carry, grad_out, 1, grad_z, grad_c1, grad_tap0,
                 grad_tap1, F, B, T, ws, RQF_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream);
}

extern "C" const char* rqf_version(void) { return "rqf_hip 0.1.0 (gfx950)"; }

extern "C" const char* rqf_error_string(int code) {
  switch (code) {
    case RQF_OK:
      return "ok";
    case RQF_ERR_ARG:
      return "invalid argument (null pointer, shape, chunk, or a grid past one dispatch's "
             "2^32 - 1 work-items)";
    case RQF_ERR_WORKSPACE:
      return "workspace missing or too small";
    case RQF_ERR_ALIGN:
      return "tensor not 8-byte aligned";
    case RQF_ERR_SCRATCH:
      return "problem larger than the static scratch of a no-allocation entry point";
    default:
      return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

extern "C" int rqf_fbt_layer0_fwd(const float* c1, const float* tap0, const float* tap1,
                                  const float* wz, const float* x, float* act, float* carry,
                                  int64_t F, int64_t B, int64_t T, rqf_stream_t stream) {
  if (!x && F * B * T > 0) return RQF_ERR_ARG;
  return fbt_fwd(c1, tap0, tap1, Drive{nullptr, x, wz}, nullptr, nullptr, act, carry, F, B, T,
                 (hipStream_t)stream);
}

extern "C" int rqf_fbt_layer0_bwd(const float* c1, const float* tap0, const float* tap1,
                                  const float* wz, const float* x, const float* carry,
                                  const float* grad_out, float* grad_z, float* grad_c1,
                                  float* grad_tap0, float* grad_tap1, int64_t F, int64_t B,
                                  int64_t T, void* workspace, size_t workspace_bytes,
                                  rqf_stream_t stream) {
  if (!x && F * B * T > 0) return RQF_ERR_ARG;
  return fbt_bwd(c1, tap0, tap1, Drive{nullptr, x, wz}, nullptr, carry, grad_out, 1, grad_z,
                 grad_c1, grad_tap0, grad_tap1, F, B, T, workspace, workspace_bytes,
                 (hipStream_t)stream);
}
