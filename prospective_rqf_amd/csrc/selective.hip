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
// Tiles: rows are walked in tiles of 64*K steps, one wavefront per tile.
// Lane l holds steps [l*K, l*K+K) of a tile, so each global access is one
// contiguous stretch (float4 when T % 4 == 0).  A tile is scanned as
//   1. per-lane serial composition of its K affine maps,
//   2. DPP wave scan of the 64 lane maps,
//   3. per-lane serial replay from the lane's entry state.
// Full tiles run without per-step range masks; only the last (partial) tile
// has them.
//
// Forward: a block owns one (channel, batch) row and walks it in super-tiles
// of consecutive tiles, one per wavefront; the tiles' maps meet in LDS behind
// one barrier per super-tile.  Blocks are dealt to the 8 XCDs in contiguous
// ranges and visit the channels of a warp group together, so concurrently
// streamed rows stay adjacent and the group's warp-logit rows stay in L2.
//
// Backward: the tiles are walked in reverse.  Each tile replays its forward
// from the stored entry state (ReLU mask and y[t-1]), runs the adjoint
//   d[t] = e[t] + conj(A[t+1]) d[t+1]
// with the same three-step structure in suffix order, and forms every
// gradient in registers (the reference's _backward,
// selective_scan_kernel.py:250-462).  A block serves the channels of one warp
// group for one batch element (or a run of them, the split form), stages the
// group's warp values in LDS and sums the group's warp-logit gradient in LDS
// in a fixed order; per-channel parameter gradients are per-row fp64 partial
// sums reduced in a fixed order.  No floating-point atomics: results are
// deterministic.
#include "rqf_device.h"
#include "rqf_scan.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <type_traits>

using namespace rqf;

#ifndef RQF_SEL_FWD_K
#define RQF_SEL_FWD_K 8
#endif
#ifndef RQF_SEL_BWD_K
#define RQF_SEL_BWD_K 4
#endif
// Minimum waves per SIMD the backward is compiled for: 3 caps it at 168
// VGPRs (it needs ~176 unconstrained, without spilling at 168).
#ifndef RQF_BWD_WAVES_PER_EU
#define RQF_BWD_WAVES_PER_EU 3
#endif

namespace {

constexpr int kFwdK = RQF_SEL_FWD_K;  // steps per lane per tile, forward
constexpr int kBwdK = RQF_SEL_BWD_K;  // steps per lane per tile, backward
constexpr int kXcds = kXcdCount;      // MI355X: 8 XCDs, blocks dealt round-robin

// XCD x runs a contiguous range of logical blocks.
__device__ __forceinline__ int64_t xcd_remap(int64_t P, int64_t n) { return xcd_contiguous(P, n); }

// Option specialisation.  Like the reference's constexpr kernel flags
// (selective_scan_kernel.py:35-46), the structural options can be compile-time
// constants: a kernel instantiated with O >= 0 takes its switches from the
// bits of O and every option branch folds away, so one tile is one basic
// block the scheduler can interleave.  O = kOptRuntime reads them from the
// inputs.  Bits that cannot matter are cleared (normalise_options) so that
// equivalent option sets share one instantiation.
enum : int {
  kOptGamma = 1,
  kOptLogShift = 2,
  kOptWarp = 4,
  kOptBound = 8,
  kOptWrite = 16,
  kOptWriteSigmoid = 32,
  kOptProspective = 64,
  kOptGammaHorizon = 128,
  kOptRuntime = -1,
};

__host__ __device__ constexpr int normalise_options(int o) {
  return (o & kOptGamma ? o : o & ~kOptLogShift) & (o & kOptWarp ? ~0 : ~kOptBound) &
         (o & kOptWrite ? ~0 : ~kOptWriteSigmoid) & (o & kOptProspective ? ~0 : ~kOptGammaHorizon);
}

template <int O>
__device__ __forceinline__ rqf_selective_inputs with_options(rqf_selective_inputs p) {
  if constexpr (O >= 0) {
    p.has_gamma = (O & kOptGamma) != 0;
    p.log_shift = (O & kOptLogShift) != 0;
    p.has_warp = (O & kOptWarp) != 0;
    p.bound_warp = (O & kOptBound) != 0;
    p.has_write = (O & kOptWrite) != 0;
    p.write_sigmoid = (O & kOptWriteSigmoid) != 0;
    p.prospective = (O & kOptProspective) != 0;
    p.gamma_horizon = (O & kOptGammaHorizon) != 0;
  }
  return p;
}

// Compiled option sets (normalised).  Anything else runs the kOptRuntime kernels.
//  - sigmoid gamma + grouped/global warp with band bound + sigmoid write + prospective
//    (the selective-copying cell, experiment/selective_copying.yaml)
//  - sigmoid gamma + prospective; sigmoid gamma alone (pure_rqf_selective.yaml)
//  - the same three without the band bound / with a gamma-mode horizon are left
//    to the run-time kernels.
constexpr int kOptSets[] = {
    kOptGamma | kOptWarp | kOptBound | kOptWrite | kOptWriteSigmoid | kOptProspective,
    kOptGamma | kOptProspective,
    kOptGamma,
};

// Wave-uniform per-channel parameters and option reciprocals.
struct Chan {
  float bias, theta, lo, span, inv_span, eta, horizon, thlo, thhi, inv_theta;
  float inv_write_max, inv_gamma_scale;
  float thlo_m;  // min(thlo, thhi): the band clamp's median bound
};

// Warp group of channel f, a row of warp_logits.  The documented precondition
// is 0 <= groups[f] < G (the Python layer rejects anything else before a
// launch); the clamp keeps a C-ABI caller that breaks it inside warp_logits
// and the team tables.
__host__ __device__ __forceinline__ int clamp_group(int64_t g, int64_t G) {
  return (int)(g < 0 ? 0 : (g >= G ? G - 1 : g));
}
__device__ __forceinline__ int64_t group_of(const rqf_selective_inputs& p, int64_t f) {
  return clamp_group(p.groups[f], p.G);
}

__device__ __forceinline__ Chan load_chan(const rqf_selective_inputs& p, int64_t f) {
  Chan c;
  c.bias = p.bias[f];
  c.theta = p.theta[f];
  c.lo = p.minimum[f];
  c.span = p.span[f];
  c.inv_span = 1.0f / c.span;
  c.eta = p.step[f];
  c.horizon = p.horizon[f];
  c.thlo = p.theta_minimum[f];
  c.thhi = p.theta_maximum[f];
  c.thlo_m = fminf(c.thlo, c.thhi);
  c.inv_theta = 1.0f / c.theta;
  c.inv_write_max = 1.0f / p.write_max;
  c.inv_gamma_scale = 1.0f / p.gamma_scale;
  return c;
}

// Controller links (rqf_models/ops/selective_scan_kernel.py:16-72).
struct Ctl {
  float gamma, theta_u, gate;  // theta_u: warped theta before the band clamp
  float wt;                    // tanh(warp logit), 0 without a warp head
};

// With the warp head's wt = tanh(warp logit) and ws = exp(warp_scale * wt) given.
__device__ __forceinline__ Ctl controller_w(const rqf_selective_inputs& p, const Chan& c, float gv,
                                            float wt, float ws, float wv) {
  Ctl o;
  o.gamma = c.bias;
  if (p.has_gamma) {
    if (p.log_shift)
      o.gamma = fexp(fmaf(p.gamma_scale, ftanh(gv), c.bias));
    else
      o.gamma = fmaf(c.span, fsigmoid(c.bias + gv), c.lo);
  }
  o.wt = p.has_warp ? wt : 0.0f;
  o.theta_u = p.has_warp ? c.theta * ws : c.theta;
  o.gate = 1.0f;
  if (p.has_write) o.gate = p.write_sigmoid ? p.write_max * fsigmoid(wv + p.write_bias) : 1.0f + wv;
  return o;
}

__device__ __forceinline__ float warp_tanh(const rqf_selective_inputs& p, float dv) {
  return p.has_warp ? ftanh(dv) : 0.0f;
}
__device__ __forceinline__ float warp_factor(const rqf_selective_inputs& p, float wt) {
  return p.has_warp ? fexp(p.warp_scale * wt) : 1.0f;
}

__device__ __forceinline__ Ctl controller(const rqf_selective_inputs& p, const Chan& c, float gv,
                                          float dv, float wv) {
  const float wt = warp_tanh(p, dv);
  return controller_w(p, c, gv, wt, warp_factor(p, wt), wv);
}

// The band clamp applies to the warped frequency only (selective_scan_kernel.py:59-64).
// As one v_med3_f32: med3(th, min(lo, hi), hi) = min(max(th, lo), hi) for
// every non-NaN th, inverted bounds included (both give hi).  fminf/fmaxf of a
// loaded bound would also quiet it for NaN semantics on every step.
__device__ __forceinline__ float clamp_theta(const rqf_selective_inputs& p, const Chan& c, float th) {
  return p.has_warp && p.bound_warp ? __builtin_amdgcn_fmed3f(th, c.thlo_m, c.thhi) : th;
}

// ratio * gamma of the prospective tap: 1 in gamma-horizon mode (ratio = 1/gamma).
__device__ __forceinline__ float ratio_gamma(const rqf_selective_inputs& p, const Chan& c,
                                             float gamma) {
  return p.gamma_horizon ? 1.0f : c.horizon * gamma;
}

// A and the gated drive u = gate*(bp z + bn zp) of one step, with
// bp z + bn zp = gamma*eta*phi*z + ratio*gamma*A*(z - zp).
__device__ __forceinline__ void step_coef(const rqf_selective_inputs& p, const Chan& c,
                                          const Ctl& q, c32 zk, c32 zp, c32& A, c32& phi,
                                          c32& u, float& inv_den, float& ai, float& den) {
  const float ar = -q.gamma * c.eta;
  ai = (1.0f - q.gamma) * clamp_theta(p, c, q.theta_u) * c.eta;
  den = fmaf(ar, ar, ai * ai);
  zoh(ar, ai, A, phi, inv_den);
  c32 drive = cscale(q.gamma * c.eta, cmul(phi, zk));
  if (p.prospective) drive = cmad(cscale(ratio_gamma(p, c, q.gamma), A), csub(zk, zp), drive);
  u = cscale(q.gate, drive);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// ---------------------------------------------------------------------------
// Tile loads / stores with 32-bit in-row offsets.  VEC: T % 4 == 0 and
// 16-byte aligned rows; then a float4 group is entirely inside or outside
// [0, T).  TAIL: the tile may extend past T (range checks on).
// ---------------------------------------------------------------------------
template <int K, bool VEC, bool TAIL>
__device__ __forceinline__ void load_c(const float* __restrict__ row, int tb, int T, c32 (&v)[K]) {
  if (VEC) {
#pragma unroll
    for (int j = 0; j < K / 2; ++j) {
      if (!TAIL || tb + 2 * j < T) {
        const float4 a = ld4(row + 2 * tb + 4 * j);
        v[2 * j] = mk(a.x, a.y);
        v[2 * j + 1] = mk(a.z, a.w);
      } else {
        v[2 * j] = mk(0.0f, 0.0f);
        v[2 * j + 1] = mk(0.0f, 0.0f);
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k)
      v[k] = (tb + k < T) ? mk(row[2 * (tb + k)], row[2 * (tb + k) + 1]) : mk(0.0f, 0.0f);
  }
}

template <int K, bool VEC, bool TAIL>
__device__ __forceinline__ void load_f(const float* __restrict__ row, int tb, int T, float (&v)[K]) {
  if (VEC) {
#pragma unroll
    for (int j = 0; j < K / 4; ++j) {
      if (!TAIL || tb + 4 * j < T) {
        const float4 a = ld4(row + tb + 4 * j);
        v[4 * j] = a.x;
        v[4 * j + 1] = a.y;
        v[4 * j + 2] = a.z;
        v[4 * j + 3] = a.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[4 * j + q] = 0.0f;
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = (tb + k < T) ? row[tb + k] : 0.0f;
  }
}

template <int K, bool VEC, bool TAIL>
__device__ __forceinline__ void store_c(float* __restrict__ row, int tb, int T, const c32 (&v)[K]) {
  if (VEC) {
#pragma unroll
    for (int j = 0; j < K / 2; ++j)
      if (!TAIL || tb + 2 * j < T)
        st4(row + 2 * tb + 4 * j, make_float4(v[2 * j].r, v[2 * j].i, v[2 * j + 1].r, v[2 * j + 1].i));
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (tb + k < T) {
        row[2 * (tb + k)] = v[k].r;
        row[2 * (tb + k) + 1] = v[k].i;
      }
  }
}

template <int K, bool VEC, bool TAIL>
__device__ __forceinline__ void store_f(float* __restrict__ row, int tb, int T, const float (&v)[K]) {
  if (VEC) {
#pragma unroll
    for (int j = 0; j < K / 4; ++j)
      if (!TAIL || tb + 4 * j < T)
        st4(row + tb + 4 * j, make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]));
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (tb + k < T) row[tb + k] = v[k];
  }
}


template <int K>
__device__ __forceinline__ void zero(float (&v)[K]) {
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = 0.0f;
}
__device__ __forceinline__ c32 relu2(c32 v) { return mk(fmaxf(v.r, 0.0f), fmaxf(v.i, 0.0f)); }

// Row coordinates of logical row L (batch-major order).
// Logical row order: the batch is cut into kXcds chunks of bc = ceil(B/8)
// elements, chunk c = XCD c's share (with the XCD-contiguous block remap).
// Inside a chunk rows go channel-major, batch-minor: the bc rows of one
// channel are adjacent in memory, so the rows a chunk streams concurrently
// cover few address ranges, and all channels of a batch element stay on one
// XCD.  Channels are visited in the optional `order` permutation, which keeps
// a warp group's channels adjacent, so the group's warp-logit rows stay in the
// XCD's L2 while its channels stream.  Logical rows past B are idle.
struct RowId {
  int64_t f, b, row;
  bool valid;
};
__device__ __forceinline__ int64_t batch_chunk(const rqf_selective_inputs& p) {
  return (p.B + kXcds - 1) / kXcds;
}
__device__ __forceinline__ RowId row_id(const rqf_selective_inputs& p, int64_t L) {
  RowId r;
  const int64_t bc = batch_chunk(p), per = p.F * bc;
  const int64_t c = L / per, rem = L - c * per;
  const int64_t pos = rem / bc;  // channel position in the visiting order
  r.b = c * bc + (rem - pos * bc);
  // group-contiguous channel order (clamped like the group indices)
  r.f = p.order ? (int64_t)min(max(p.order[pos], 0), (int)p.F - 1) : pos;
  r.valid = c < kXcds && r.b < p.B;
  r.row = r.f * p.B + r.b;
  return r;
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
struct FwdRow {
  const float* zr;
  const float* gr;
  const float* wr;
  const float* dr;
  float* rawr;
  float* actr;
  const float* skr;  // residual added to both outputs (the layer input), or nullptr
  float* ent;
  float4* io;  // this wavefront's LDS slice for transposed complex I/O (or nullptr)
  int T, chunk;
  c32 y, zlast;
};

// Inputs of one forward tile (per lane).
template <int K>
struct FwdIn {
  c32 zv[K];
  float gv[K], wv[K], dv[K];
};

// The heads' presence is taken from the options (compile-time constants of a
// compiled option set), not from the row pointers: a pointer plus an offset
// is not provably non-null, and a run-time test keeps a mask alive per head.
template <int K, bool VEC, bool TAIL>
__device__ __forceinline__ void fwd_load(const rqf_selective_inputs& p, const FwdRow& r, int t0,
                                         int lane, FwdIn<K>& in) {
  const int T = r.T;
  const int tb = t0 + lane * K;
  if (VEC && !TAIL)
    load_c_lds<K>(r.zr, t0, lane, r.io, in.zv);
  else
    load_c<K, VEC, TAIL>(r.zr, tb, T, in.zv);
  if (p.has_gamma) load_f<K, VEC, TAIL>(r.gr, tb, T, in.gv); else zero(in.gv);
  if (p.has_write) load_f<K, VEC, TAIL>(r.wr, tb, T, in.wv); else zero(in.wv);
  if (p.has_warp) load_f<K, VEC, TAIL>(r.dr, tb, T, in.dv); else zero(in.dv);
}

// Per-step coefficients of one tile: A (decay) and u (drive) of each of the
// lane's K steps.  zlast_tile: z[t0 - 1] (0 at t0 = 0).
template <int K, bool TAIL>
__device__ __forceinline__ void fwd_steps(const rqf_selective_inputs& p, const Chan& c, int T,
                                          int t0, int lane, const FwdIn<K>& in, c32 zlast_tile,
                                          c32 (&A)[K], c32 (&u)[K]) {
  const int tb = t0 + lane * K;
  const c32 zp0 = shift_up(in.zv[K - 1], zlast_tile, lane);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const Ctl q = controller(p, c, in.gv[k], in.dv[k], in.wv[k]);
    c32 phi;
    float inv_den, ai, den;
    step_coef(p, c, q, in.zv[k], k ? in.zv[k - 1] : zp0, A[k], phi, u[k], inv_den, ai, den);
    if (TAIL && tb + k >= T) {
      A[k] = mk(1.0f, 0.0f);
      u[k] = mk(0.0f, 0.0f);
    }
  }
}

// Chunk entry states and the raw / act outputs of one tile.
template <int K, bool VEC, bool TAIL>
__device__ __forceinline__ void fwd_emit(const FwdRow& r, int t0, int lane, c32 (&out)[K]) {
  const int T = r.T;
  const int tb = t0 + lane * K;
  // Entry states: the state after step t with (t+1) % chunk == 0 enters chunk (t+1)/chunk.
  if (r.chunk >= K) {
    const int t1 = tb + K;
    if (t1 < T && (t1 & (r.chunk - 1)) == 0) {
      r.ent[2 * (t1 / r.chunk)] = out[K - 1].r;
      r.ent[2 * (t1 / r.chunk) + 1] = out[K - 1].i;
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int t1 = tb + k + 1;
      if (t1 < T && (t1 & (r.chunk - 1)) == 0) {
        r.ent[2 * (t1 / r.chunk)] = out[k].r;
        r.ent[2 * (t1 / r.chunk) + 1] = out[k].i;
      }
    }
  }
  constexpr bool lds_io = VEC && !TAIL;
  c32 sk[K];
  if (r.skr) {
    if (lds_io)
      load_c_lds<K>(r.skr, t0, lane, r.io, sk);
    else
      load_c<K, VEC, TAIL>(r.skr, tb, T, sk);
  }
  if (r.rawr) {
    c32 o[K];
#pragma unroll
    for (int k = 0; k < K; ++k) o[k] = r.skr ? cadd(out[k], sk[k]) : out[k];
    if (lds_io)
      store_c_lds<K>(r.rawr, t0, lane, r.io, o);
    else
      store_c<K, VEC, TAIL>(r.rawr, tb, T, o);
  }
  if (r.actr) {
#pragma unroll
    for (int k = 0; k < K; ++k) out[k] = r.skr ? cadd(relu2(out[k]), sk[k]) : relu2(out[k]);
    if (lds_io)
      store_c_lds<K>(r.actr, t0, lane, r.io, out);
    else
      store_c<K, VEC, TAIL>(r.actr, tb, T, out);
  }
}

// Forward, row-block form: a block of kFwdRbWaves wavefronts owns one row and
// walks it in super-tiles of kFwdRbWaves consecutive tiles, wavefront w
// taking tile w of each, so that concurrent wavefronts stream adjacent
// stretches of the same rows (8 waves x 512 steps = 32 KB of each complex
// stream per super-tile).  Each wavefront scans its tile from a zero entry
// and publishes the tile's affine map (P, s) in LDS; after one barrier it
// composes the maps of the tiles before it onto the block's carry and
// replays its steps from there.  Map slots are double-buffered, so one
// barrier per super-tile suffices.  Config 3 forward, measured: 1.746 ms one
// row per wavefront (K = 4); row blocks of 2 / 4 / 8 / 16 waves: 1.765 /
// 1.729 / 1.688 / - (K = 4), 8 waves with K = 8: 1.644, 16 waves with K = 8:
// 1.753, 4 waves with K = 16: 1.701; without the LDS transpose 1.837.
// Calls that write one complex output, raw or act (24 B per element instead
// of 32), run blocks of kFwdRbWavesRaw = 4 wavefronts: their arithmetic
// weighs more against their streams, and twice as many independent blocks
// per CU overlap one block's barrier and replay with another's loads.
// Config 4 (T = 4096, K = 8), measured on one box: raw-only layer 1 0.352 ->
// 0.320 ms with 4 waves; raw+act layer 0 0.403 ms with 8 against 0.425 with
// 4, config 3 1.668 against 1.718; config 3's act-only contract 1.314 ->
// 1.282 ms with 4.
#ifndef RQF_FWD_RB_WAVES
#define RQF_FWD_RB_WAVES 8
#endif
#ifndef RQF_FWD_RB_WAVES_RAW
#define RQF_FWD_RB_WAVES_RAW 4
#endif
constexpr int kFwdRbWaves = RQF_FWD_RB_WAVES;
constexpr int kFwdRbWavesRaw = RQF_FWD_RB_WAVES_RAW;

template <int O, bool VEC, int W>
__global__ __launch_bounds__(W* kWave)
    void selective_fwd_rb_kernel(
    const rqf_selective_inputs pin, const float* __restrict__ z, const float* __restrict__ skip,
    float* __restrict__ raw, float* __restrict__ act, float* __restrict__ entries, int chunk,
    int nc) {
  constexpr int K = kFwdK, TILE = kWave * K;
  const rqf_selective_inputs p = with_options<O>(pin);
  __shared__ float4 s_io[W][TILE / 2];
  __shared__ float4 s_map[2][W];
  const int lane = lane_id();
  const int w = wave_id();
  const RowId id = row_id(p, xcd_remap(blockIdx.x, gridDim.x));
  if (!id.valid) return;  // the whole block
  const Chan c = load_chan(p, id.f);
  FwdRow r;
  r.T = (int)p.T;
  r.chunk = chunk;
  const int T = r.T;
  const int64_t base = id.row * T;
  r.zr = z + 2 * base;
  r.gr = p.has_gamma ? p.gamma_logits + base : nullptr;
  r.wr = p.has_write ? p.write_logits + base : nullptr;
  r.dr = p.has_warp ? p.warp_logits + (group_of(p, id.f) * p.B + id.b) * T : nullptr;
  r.rawr = raw ? raw + 2 * base : nullptr;
  r.actr = act ? act + 2 * base : nullptr;
  r.skr = skip ? skip + 2 * base : nullptr;
  r.ent = entries + 2 * id.row * nc;
  r.io = &s_io[w][0];
  if (w == 0 && lane == 0) {
    r.ent[0] = 0.0f;
    r.ent[1] = 0.0f;
  }
  const int full = VEC ? T / TILE : 0;
  c32 y = mk(0.0f, 0.0f);  // the row's state entering the super-tile
  int parity = 0;
  for (int st0 = 0; st0 < T; st0 += W * TILE) {
    const int t0 = st0 + w * TILE;
    const bool has = t0 < T;
    c32 A[K], u[K];
    c32 P = mk(1.0f, 0.0f), s = mk(0.0f, 0.0f);
    if (has) {
      const c32 zlast = t0 > 0 ? mk(r.zr[2 * (t0 - 1)], r.zr[2 * (t0 - 1) + 1]) : mk(0.0f, 0.0f);
      FwdIn<K> in;
      if (t0 / TILE < full) {
        fwd_load<K, VEC, false>(p, r, t0, lane, in);
        fwd_steps<K, false>(p, c, T, t0, lane, in, zlast, A, u);
      } else {
        fwd_load<K, VEC, true>(p, r, t0, lane, in);
        fwd_steps<K, true>(p, c, T, t0, lane, in, zlast, A, u);
      }
      P = A[0];
      s = u[0];
#pragma unroll
      for (int k = 1; k < K; ++k) {
        s = cmad(A[k], s, u[k]);
        P = cmul(A[k], P);
      }
      wave_scan_fwd(P, s);  // inclusive prefix maps of the tile, zero entry
      if (lane == kWave - 1) s_map[parity][w] = make_float4(P.r, P.i, s.r, s.i);
    }
    __syncthreads();
    // Entry of this tile and the carry past the super-tile.
    c32 ye = y, yr = y;
    for (int v = 0; v < W && st0 + v * TILE < T; ++v) {
      if (v == w) ye = yr;
      const float4 m = s_map[parity][v];
      yr = cmad(mk(m.x, m.y), yr, mk(m.z, m.w));
    }
    if (has) {
      const c32 pex = shift_up(P, mk(1.0f, 0.0f), lane);
      const c32 sex = shift_up(s, mk(0.0f, 0.0f), lane);
      c32 yk = cmad(pex, ye, sex);
      c32 out[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        yk = cmad(A[k], yk, u[k]);
        out[k] = yk;
      }
      if (t0 / TILE < full)
        fwd_emit<K, VEC, false>(r, t0, lane, out);
      else
        fwd_emit<K, VEC, true>(r, t0, lane, out);
    }
    y = yr;
    parity ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
struct BwdOut {
  float* dz;        // x-path drive gradient (only written when truncated)
  float* dzw;       // W-path drive gradient (== dz when not truncated)
  float* dg;
  float* dw;
  float* dd_part;   // (S, B, T) warp-logit gradient summed over each split (team kernel)
  float* dd;        // (G, B, T) warp-logit gradient (team kernel, groups with one split)
  double* partial;  // (2, F*B): per row sums of d/dbias and d/dtheta
};

struct BwdRow {
  const float* zr;
  const float* gr;
  const float* wr;
  const float* gyr;
  const float* gxr;
  const float* ent;
  float* dzr;
  float* dzwr;
  float* dgr;
  float* dwr;
  float4* sdd;    // this wavefront's slot of the team's LDS warp-gradient tile (or null)
  const float* swg;  // team LDS stage of the tile: warp_scale*(1 - tanh(warp logit)^2)
  const float* sws;  // and exp(warp_scale * tanh(warp logit)) per step
  int T, chunk, truncated;
  c32 dcarry;  // adjoint (truncated: cotangent) at the next tile's first step
  c32 Afirst;  // A at the next tile's first step (0 past the end)
  float cfirst;  // gate*ratio*gamma at the next tile's first step
  double sum_bias, sum_theta;
};

// Cotangent set of a backward call.  Calls under full BPTT with float4 rows
// and a compiled option set are compiled with it fixed (gy only, gx only or
// both), so a tile carries no register, load, mask or select for an absent
// cotangent, no run-time test of the truncation flag or of the heads'
// pointers.  Measured with rotated runs on one box: config 4's raw-only
// layer 1 backward 0.608 -> 0.590-0.594 ms; with both cotangents (config 3,
// config 4's layer 0) 2.698 -> 2.676 and 0.691 -> 0.686 ms, once the
// cotangent loads are kept below the tile's coefficient math (a scheduling
// barrier; hoisted above it they raised the register pressure and the
// fixed form ran 0.7% slower than the run-time one).  kCtRuntime reads
// everything from the call.
enum : int { kCtRuntime = 0, kCtGy = 1, kCtGx = 2, kCtGyGx = 3 };
template <int CT>
struct Cot {
  static constexpr bool fixed = CT != kCtRuntime;
  static constexpr bool gy = CT == kCtGy || CT == kCtGyGx;
  static constexpr bool gx = CT == kCtGx || CT == kCtGyGx;
};
// Truncated backward (TBPTT(1))?  Never for a fixed cotangent set.
template <int CT>
__device__ __forceinline__ bool truncated_of(int truncated) {
  return Cot<CT>::fixed ? false : truncated != 0;
}

// Staged warp values of the lane's K steps (from LDS): the frequency factor
// exp(warp_scale * tanh) and the tanh derivative factor warp_scale*(1 - tanh^2).
template <int K>
__device__ __forceinline__ void lds_warp_factor(const BwdRow& r, int lane, float (&ws)[K]) {
  static_assert(K % 4 == 0, "whole float4s of staged warp values per lane");
#pragma unroll
  for (int j = 0; j < K / 4; ++j) {
    const float4 b = reinterpret_cast<const float4*>(r.sws)[lane * (K / 4) + j];
    ws[4 * j] = b.x, ws[4 * j + 1] = b.y, ws[4 * j + 2] = b.z, ws[4 * j + 3] = b.w;
  }
}
template <int K>
__device__ __forceinline__ void lds_warp(const BwdRow& r, int lane, float (&wg)[K], float (&ws)[K]) {
  lds_warp_factor<K>(r, lane, ws);
#pragma unroll
  for (int j = 0; j < K / 4; ++j) {
    const float4 a = reinterpret_cast<const float4*>(r.swg)[lane * (K / 4) + j];
    wg[4 * j] = a.x, wg[4 * j + 1] = a.y, wg[4 * j + 2] = a.z, wg[4 * j + 3] = a.w;
  }
}
// The staged values of one step: exp(warp_scale * wt), warp_scale*(1 - wt^2).
__device__ __forceinline__ void warp_stage(const rqf_selective_inputs& p, float dv, float& ws,
                                           float& wg) {
  const float wt = warp_tanh(p, dv);
  ws = warp_factor(p, wt);
  wg = p.warp_scale * fmaf(-wt, wt, 1.0f);
}

// Per-step values of one backward tile, kept from its replay phase for its
// gradient phase.
template <int K>
struct BwdTile {
  static_assert(K >= 2, "a lane holds its first step and the product M of the rest");
  c32 A[K], phi[K];  // decay and ZOH phi of every step (A = 0 past the end)
  c32 yprev[K], ecot[K];  // forward state before the step; cotangent on raw
  c32 M;  // product of A over the lane's steps after its first (full tiles)
  // ivd = 1/|a|^2, aim = Im a, dsq = |a|^2 of the ZOH exponent a, reused by the VJP
  float gam[K], gate[K], ivd[K], aim[K], dsq[K];
  c32 zp0;   // z of the step before the lane's first
  float c0;  // lag-tap weight gate*ratio*gamma of the lane's first step
};

// Replay phase of a backward tile: the coefficients of every step, the
// forward replay from the tile's entry state and the cotangent e on raw.
// The warp values of the tile come from the block's LDS stage (r.swg, r.sws).
// zv: the tile's drive; zprev_tile: z[t0 - 1] (0 at t0 = 0).
template <int K, bool VEC, bool TAIL, int CT>
__device__ __forceinline__ void bwd_tile_replay(const rqf_selective_inputs& p, const Chan& c,
                                                const BwdRow& r, int t0, int lane,
                                                const c32 (&zv)[K], c32 zprev_tile,
                                                BwdTile<K>& s) {
  const int T = r.T;
  const int tb = t0 + lane * K;
  float gv[K], wv[K];
  // A fixed cotangent set takes the heads' presence from the options, like
  // the forward (the run-time form keeps its pointer tests).
  if (Cot<CT>::fixed ? p.has_gamma : r.gr != nullptr)
    load_f<K, VEC, TAIL>(r.gr, tb, T, gv);
  else
    zero(gv);
  if (Cot<CT>::fixed ? p.has_write : r.wr != nullptr)
    load_f<K, VEC, TAIL>(r.wr, tb, T, wv);
  else
    zero(wv);
  s.zp0 = shift_up(zv[K - 1], zprev_tile, lane);

  // Coefficients; kept per step: A, phi, gamma and gate.
  c32 u[K];
  float sws[K];
  lds_warp_factor<K>(r, lane, sws);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const Ctl q = controller_w(p, c, gv[k], 0.0f, sws[k], wv[k]);
    step_coef(p, c, q, zv[k], k ? zv[k - 1] : s.zp0, s.A[k], s.phi[k], u[k], s.ivd[k],
              s.aim[k], s.dsq[k]);
    s.gam[k] = q.gamma;
    s.gate[k] = q.gate;
    if (TAIL && tb + k >= T) u[k] = mk(0.0f, 0.0f);
  }
  // Forward states y[t-1] of every step, and the cotangent e[t] on raw: the
  // raw output plus the split-ReLU cotangent where raw > 0.
  c32 ey[K], ex[K];
  // Keep the cotangent loads below the coefficient math: hoisted above it
  // they raise the register pressure across the tile's busiest stretch.
  if (Cot<CT>::fixed) __builtin_amdgcn_sched_barrier(0);
  if (Cot<CT>::fixed ? Cot<CT>::gy : r.gyr != nullptr) {
    load_c<K, VEC, TAIL>(r.gyr, tb, T, ey);
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) ey[k] = mk(0.0f, 0.0f);
  }
  if (Cot<CT>::fixed ? Cot<CT>::gx : r.gxr != nullptr) {
    load_c<K, VEC, TAIL>(r.gxr, tb, T, ex);
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) ex[k] = mk(0.0f, 0.0f);
  }
  {
    // Replay the forward from the tile's entry state.  The lane's map is
    // P = A[0] * M with M the product over its later steps, which the adjoint's
    // map reuses.
    const c32 y0 = mk(r.ent[2 * (t0 / r.chunk)], r.ent[2 * (t0 / r.chunk) + 1]);
    c32 Am[K];
#pragma unroll
    for (int k = 0; k < K; ++k) Am[k] = (TAIL && tb + k >= T) ? mk(1.0f, 0.0f) : s.A[k];
    c32 sy = u[0];
    s.M = Am[1];
#pragma unroll
    for (int k = 1; k < K; ++k) {
      sy = cmad(Am[k], sy, u[k]);
      if (k > 1) s.M = cmul(Am[k], s.M);
    }
    c32 P = cmul(s.M, Am[0]);
    if (lane == 0) sy = cmad(P, y0, sy);
    wave_scan_fwd(P, sy);
    c32 yk = shift_up(sy, y0, lane);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      s.yprev[k] = yk;
      yk = cmad(Am[k], yk, u[k]);
      if constexpr (Cot<CT>::gy && !Cot<CT>::gx)
        s.ecot[k] = ey[k];
      else if constexpr (Cot<CT>::gx && !Cot<CT>::gy)
        s.ecot[k] = mk(yk.r > 0.0f ? ex[k].r : 0.0f, yk.i > 0.0f ? ex[k].i : 0.0f);
      else
        s.ecot[k] = mk(ey[k].r + (yk.r > 0.0f ? ex[k].r : 0.0f),
                       ey[k].i + (yk.i > 0.0f ? ex[k].i : 0.0f));
    }
  }
  if (TAIL) {
    // Past-the-end steps have A = 0 and no lag tap for the adjoint.
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (tb + k >= T) {
        s.A[k] = mk(0.0f, 0.0f);
        s.gate[k] = 0.0f;
      }
  }
  // Lag-tap weight cn = gate*ratio*gamma (gated n = -cn*A) of the lane's first step.
  s.c0 = p.prospective ? s.gate[0] * ratio_gamma(p, c, s.gam[0]) : 0.0f;
}

// The lane's adjoint map d_first = rr + Q d_next over its K steps, where
// d_next is the adjoint at the step after the lane's last and A_lane_next
// the decay of that step: the suffix composition of d[t] = e[t] + conj(A[t+1]) d[t+1].
// On full tiles Q = conj(M A_lane_next) from the replay's product M; on the
// last (TAIL) tile the replay's A past the row's end differs (1, not 0).
template <int K, bool TAIL>
__device__ __forceinline__ void bwd_lane_adjoint(const BwdTile<K>& s, c32 A_lane_next, c32& Q,
                                                 c32& rr) {
  Q = mk(1.0f, 0.0f);
  rr = mk(0.0f, 0.0f);
#pragma unroll
  for (int k = K - 1; k >= 0; --k) {
    const c32 An = k + 1 < K ? s.A[k + 1] : A_lane_next;
    rr = cjmad(An, rr, s.ecot[k]);
    if (TAIL) Q = cjmul(An, Q);
  }
  if (!TAIL) Q = conjg(cmul(s.M, A_lane_next));
}

// Gradient phase of a backward tile, given the adjoint dnext at the step
// after the lane's last (the cotangent there when truncated), the decay
// A_lane_next and the lag-tap weight cn_lane_next of that step.  gd_out
// (optional) receives the lane's warp-logit gradients.
template <int K, bool VEC, bool TAIL, int CT>
__device__ __forceinline__ void bwd_tile_grads(const rqf_selective_inputs& p, const Chan& c,
                                               BwdRow& r, int t0, int lane, const c32 (&zv)[K],
                                               const BwdTile<K>& s, c32 dnext, c32 A_lane_next,
                                               float cn_lane_next, float* gd_out = nullptr) {
  const int T = r.T;
  const int tb = t0 + lane * K;
  float swg[K], sws[K];
  // Re-read the staged warp values here rather than keep them live across
  // the scans (the compiler barrier stops it from reusing the first read).
  __asm__ volatile("" ::: "memory");
  lds_warp<K>(r, lane, swg, sws);
  c32 gz[K], gzw[K];
  float gg[K], gw[K], gd[K];
  float tile_bias = 0.0f, tile_theta = 0.0f;
#pragma unroll
  for (int k = K - 1; k >= 0; --k) {
    const c32 An = k + 1 < K ? s.A[k + 1] : A_lane_next;
    float cn;
    if (k + 1 < K)
      cn = p.prospective ? s.gate[k + 1] * ratio_gamma(p, c, s.gam[k + 1]) : 0.0f;
    else
      cn = cn_lane_next;
    const c32 d = truncated_of<CT>(r.truncated) ? s.ecot[k] : cjmad(An, dnext, s.ecot[k]);
    const float gamma = s.gam[k], gt = s.gate[k];
    const float rg = p.prospective ? ratio_gamma(p, c, gamma) : 0.0f;
    const float gh = gamma * c.eta;
    // Step map: y = A y_prev + gt*(gh*phi*z + rg*A*(z - zp)); the un-gated taps
    // are bp = gh*phi + rg*A on z and bn = -rg*A on zp.
    // x-path input gradient conj(gt*bp) d, and the W-path one adds the next
    // step's lag tap conj(n[t+1]) d[t+1] with n[t+1] = -cn*s.A[t+1].
    const c32 gphi = cscale(gt * gh, s.phi[k]);
    const c32 gbp = p.prospective ? csmad(gt * rg, s.A[k], gphi) : gphi;
    const c32 cur = cjmul(gbp, d);
    gz[k] = cur;
    gzw[k] = p.prospective ? cjmad(cscale(-cn, An), dnext, cur) : cur;
    dnext = d;
    // cz = conj(z) d; for the prospective tap cw = conj(z - zp) d.
    const c32 cz = cjmul(zv[k], d);
    const float pz = cdot(s.phi[k], cz);  // Re(conj(phi z) d)
    float dgate = gh * pz;              // dL/dgate = Re(conj(drive) d)
    float dgamma = gt * c.eta * pz;     // through gh = gamma*eta
    c32 dA = cjmul(s.yprev[k], d);      // dL/dA = conj(y_prev + gt*rg*(z - zp)) d
    if (p.prospective) {
      const c32 zp = k ? zv[k - 1] : s.zp0;
      const c32 cw = cjmul(csub(zv[k], zp), d);
      const float aw = cdot(s.A[k], cw);  // Re(conj(A (z - zp)) d)
      dgate = fmaf(rg, aw, dgate);
      if (!p.gamma_horizon) dgamma = fmaf(gt * c.horizon, aw, dgamma);  // through rg
      dA = csmad(gt * rg, cw, dA);
    }
    // phi'(a) = sum_m (m+1) a^m / (m+2)!  (the reference's series,
    // selective_scan_kernel.py:119-148), here to degree 4 for |a| < 1/32
    // (truncation < 1e-10 relative) and (A - phi)/a above, where the
    // cancellation in A - phi costs at most ~1e-5 relative.
    const float th_u = p.has_warp ? c.theta * sws[k] : c.theta;
    const float theta = clamp_theta(p, c, th_u);
    const c32 a = mk(-gh, s.aim[k]);
    c32 fp;
    if (s.dsq[k] < 9.765625e-4f) {
      c32 sr = cmadrr(a, 1.0f / 144.0f, 1.0f / 30.0f);
      sr = cmadr(a, sr, 1.0f / 8.0f);
      sr = cmadr(a, sr, 1.0f / 3.0f);
      fp = cmadr(a, sr, 0.5f);
    } else {
      // 1/|a|^2 as the ZOH formed it
      fp = cscale(s.ivd[k], cmul(csub(s.A[k], s.phi[k]), conjg(a)));
    }
    // da = conj(A) dA + conj(phi') dphi with dphi = gt*gh*cz; then through
    // a = (-gamma*eta, (1 - gamma)*theta*eta).  (Folding the two terms through
    // the step map into conj(y + gt*gh*(phi' - phi)*z) d saves four operations
    // but cancels when A -> 0: y and gt*gh*phi*z are then nearly equal.)
    const c32 da = cjmad(fp, cscale(gt * gh, cz), cjmul(s.A[k], dA));
    dgamma -= c.eta * fmaf(theta, da.i, da.r);
    float dth = c.eta * (1.0f - gamma) * da.i;
    // controller chain rules (selective_scan_kernel.py:441-460)
    float dbias;
    if (p.has_gamma) {
      if (p.log_shift) {
        dbias = dgamma * gamma;
        // tanh of the gamma logit, from gamma = exp(bias + scale*tanh)
        const float sg =
            (__builtin_amdgcn_logf(gamma) * 0.6931471805599453f - c.bias) * c.inv_gamma_scale;
        gg[k] = dbias * p.gamma_scale * (1.0f - sg * sg);
      } else {
        const float sg = (gamma - c.lo) * c.inv_span;
        dbias = dgamma * c.span * sg * (1.0f - sg);
        gg[k] = dbias;
      }
    } else {
      dbias = dgamma;
      gg[k] = 0.0f;
    }
    if (p.has_warp) {
      // exp(scale*w) = d theta_u / d theta
      const float ws = sws[k];
      // d exp(scale*tanh(w))/dw = exp(scale*tanh(w)) * scale*(1 - tanh(w)^2)
      const float wg = swg[k];
      // torch.clamp passes the gradient at both exact edges
      if (p.bound_warp && !(th_u >= c.thlo && th_u <= c.thhi)) dth = 0.0f;
      gd[k] = dth * theta * wg;
      dth *= ws;
    } else {
      gd[k] = 0.0f;
    }
    gw[k] = p.write_sigmoid ? dgate * gt * (1.0f - gt * c.inv_write_max) : dgate;
    if (TAIL && tb + k >= T) {
      dbias = 0.0f;
      dth = 0.0f;
    }
    tile_bias += dbias;
    tile_theta += dth;
  }
  r.sum_bias += (double)tile_bias;
  r.sum_theta += (double)tile_theta;
  store_c<K, VEC, TAIL>(r.dzwr, tb, T, gzw);
  if (truncated_of<CT>(r.truncated)) store_c<K, VEC, TAIL>(r.dzr, tb, T, gz);
  if (Cot<CT>::fixed ? p.has_gamma : r.dgr != nullptr) store_f<K, VEC, TAIL>(r.dgr, tb, T, gg);
  if (Cot<CT>::fixed ? p.has_write : r.dwr != nullptr) store_f<K, VEC, TAIL>(r.dwr, tb, T, gw);
  if (r.sdd) {
    static_assert(K % 4 == 0, "whole float4s of warp gradient per lane");
#pragma unroll
    for (int j = 0; j < K / 4; ++j)
      r.sdd[lane * (K / 4) + j] =
          make_float4(gd[4 * j], gd[4 * j + 1], gd[4 * j + 2], gd[4 * j + 3]);
  }
  if (gd_out) {
#pragma unroll
    for (int k = 0; k < K; ++k) gd_out[k] = gd[k];
  }
}

// One backward tile of a row walked by one wavefront: the tile's exit adjoint
// state (r.dcarry) and the next tile's first decay and lag-tap weight
// (r.Afirst, r.cfirst) come in through r and go out for the tile before it.
template <int K, bool VEC, bool TAIL, int CT>
__device__ __forceinline__ void bwd_tile(const rqf_selective_inputs& p, const Chan& c, BwdRow& r,
                                         int t0, int lane, const c32 (&zv)[K], c32 zprev_tile) {
  BwdTile<K> s;
  bwd_tile_replay<K, VEC, TAIL, CT>(p, c, r, t0, lane, zv, zprev_tile, s);
  const c32 A_lane_next = shift_down(s.A[0], r.Afirst, lane);
  const float cn_lane_next = shift_down(s.c0, r.cfirst, lane);
  r.Afirst = readlane(s.A[0], 0);
  r.cfirst = readlane(s.c0, 0);

  // Adjoint d[t] = e[t] + conj(A[t+1]) d[t+1]  (truncated: d = e).
  c32 dnext;
  if (truncated_of<CT>(r.truncated)) {
    dnext = shift_down(s.ecot[0], r.dcarry, lane);
    r.dcarry = readlane(s.ecot[0], 0);
  } else {
    c32 Q, rr;
    bwd_lane_adjoint<K, TAIL>(s, A_lane_next, Q, rr);
    if (lane == kWave - 1) rr = cmad(Q, r.dcarry, rr);
    wave_scan_rev(Q, rr, lane);
    dnext = shift_down(rr, r.dcarry, lane);
    r.dcarry = readlane(rr, 0);
  }

  bwd_tile_grads<K, VEC, TAIL, CT>(p, c, r, t0, lane, zv, s, dnext, A_lane_next, cn_lane_next);
}

// ---------------------------------------------------------------------------
// Backward, team form: a block of kTeam wavefronts owns a split, up to
// kMaxSplitTeams consecutive teams of one warp group, for one batch element.
// A team is up to kTeam channels of the group, one per wavefront.  The block
// walks the row backwards in segments of kSegTiles tiles: it stages the
// segment's warp tanh and frequency factor in LDS once, then runs each team
// of the split over the segment in turn, carrying every channel's adjoint
// state across segments in LDS.  Per tile the team sums its warp-logit
// gradient in LDS (fixed order over channels, one barrier per tile with
// double-buffered LDS) and adds it to the segment's group sum, also in LDS
// and in fixed team order.  A group served by one split writes its gradient
// row directly; otherwise each split writes a partial row and a small pass
// sums the splits of the group in order.
// ---------------------------------------------------------------------------
#ifndef RQF_TEAM_WAVES
#define RQF_TEAM_WAVES 4
#endif
constexpr int kTeam = RQF_TEAM_WAVES;
#ifndef RQF_BWD_SEG_TILES
#define RQF_BWD_SEG_TILES 8
#endif
constexpr int kSegTiles = RQF_BWD_SEG_TILES;
constexpr int kMaxSplitTeams = 16;
// Teams per split are sized so that the grid holds at least
// kSplitBlocksPerCu blocks per CU; the environment variable
// RQF_BWD_SPLIT_TEAMS=<n> fixes it instead (tests and tuning).  Longer splits
// cut the partial-row traffic but leave fewer, longer blocks: at config 3
// (8 teams per group and batch element, 3 resident blocks per CU) 2 teams per
// split measured best (2.77 ms against 2.79 for 1, 2.84 for 3, 3.06 for 4
// and 2.91 for 8).
constexpr int kCus = 256;  // MI355X
constexpr int kSplitBlocksPerCu = 8;

// Team table built on the device (no host round trip).  Channels are ordered
// by (warp group, channel index); a team is up to kTeam consecutive channels
// of one group.  Without a warp head all channels form one group.
struct Teams {
  const int* order;   // (F,) channels sorted by group
  const int* first;   // (S,) index into order of the team's first channel
  const int* count;   // (S,) channels in the team
  const int* group;   // (S,) warp group of the team
  const int* nteams;  // (1,) number of teams in use
  const int* sfirst;  // (S,) first team of each split
  const int* sn;      // (S,) teams in each split
  const int* gsplit;  // (G+1,) first split of each group
  const int* nsplits; // (1,) number of splits in use
  const int* gteam;   // (G+1,) first team of each group
  int slots;          // S: upper bound on the number of teams (and splits)
};

// Group-sorted channel order and team table, built on the device from the
// group indices (int64, as the reference's warp_groups buffer); a team is up
// to `tsize` consecutive channels of one group.  Groups,
// per-group counts and offsets are staged in LDS (F <= kBuildLds and
// G <= kBuildGroups, else a slower pass over global memory).
constexpr int kBuildLds = 4096;
constexpr int kBuildGroups = 1024;
// The team table without LDS staging (F > kBuildLds or G > kBuildGroups).
__device__ void team_build_global(const int64_t* __restrict__ groups, int F, int G, int tsize,
                                  int* order, int* first, int* count, int* group, int* gteam,
                                  int* nteams, int* gcount, int* moff) {
  const int tid = threadIdx.x, nt = blockDim.x;
  auto grp = [&](int f) { return groups ? clamp_group(groups[f], G) : 0; };
  for (int g = tid; g < G; g += nt) {
    int n = 0;
    for (int f = 0; f < F; ++f) n += grp(f) == g;
    gcount[g] = n;
  }
  __syncthreads();
  if (tid == 0) {
    int off = 0, toff = 0;
    for (int g = 0; g < G; ++g) {
      moff[g] = off;
      gteam[g] = toff;
      off += gcount[g];
      toff += (gcount[g] + tsize - 1) / tsize;
    }
    gteam[G] = toff;
    *nteams = toff;
  }
  __syncthreads();
  for (int f = tid; f < F; f += nt) {
    const int g = grp(f);
    int rank = 0;
    for (int q = 0; q < f; ++q) rank += grp(q) == g;
    order[moff[g] + rank] = f;
  }
  for (int g = tid; g < G; g += nt) {
    const int n = gcount[g], ntm = (n + tsize - 1) / tsize;
    for (int t = 0; t < ntm; ++t) {
      const int id = gteam[g] + t;
      first[id] = moff[g] + t * tsize;
      count[id] = min(tsize, n - t * tsize);
      group[id] = g;
    }
  }
}

__global__ __launch_bounds__(256) void team_build_kernel(const int64_t* __restrict__ groups,
                                                         int F, int G, int Q, int tsize, int* order,
                                                         int* first, int* count, int* group,
                                                         int* gteam, int* nteams, int* gcount,
                                                         int* moff, int* sfirst, int* sn,
                                                         int* gsplit, int* nsplits) {
  __shared__ int4 sg4[kBuildLds / 4];
  __shared__ int s_count[kBuildGroups], s_moff[kBuildGroups], s_gteam[kBuildGroups + 1];
  __shared__ int s_gsplit[kBuildGroups + 1];
  int* sg = reinterpret_cast<int*>(sg4);
  const int tid = threadIdx.x, nt = blockDim.x;
  if (F <= kBuildLds && G <= kBuildGroups) {
    // Everything after the one read of `groups` stays in LDS; the global
    // tables are written once and never read back here.
    const int F4 = (F + 3) & ~3;
    for (int f = tid; f < F4; f += nt) sg[f] = f < F ? (groups ? clamp_group(groups[f], G) : 0) : -1;
    for (int g = tid; g < G; g += nt) s_count[g] = 0;
    __syncthreads();
    for (int f = tid; f < F; f += nt) atomicAdd(&s_count[sg[f]], 1);
    __syncthreads();
    if (tid == 0) {
      int off = 0, toff = 0, soff = 0;
      for (int g = 0; g < G; ++g) {
        const int ntm = (s_count[g] + tsize - 1) / tsize;
        s_moff[g] = off;
        s_gteam[g] = toff;
        s_gsplit[g] = soff;
        off += s_count[g];
        toff += ntm;
        soff += (ntm + Q - 1) / Q;  // splits: runs of up to Q consecutive teams
      }
      s_gteam[G] = toff;
      s_gsplit[G] = soff;
      *nteams = toff;
      *nsplits = soff;
    }
    __syncthreads();
    // Stable rank of channel f within its group: earlier channels of the same
    // group, counted four at a time from LDS.
    for (int f = tid; f < F; f += nt) {
      const int g = sg[f];
      int rank = 0;
      const int q4 = f >> 2;
      for (int j = 0; j < q4; ++j) {
        const int4 v = sg4[j];
        rank += (v.x == g) + (v.y == g) + (v.z == g) + (v.w == g);
      }
      for (int q = q4 << 2; q < f; ++q) rank += sg[q] == g;
      order[s_moff[g] + rank] = f;
    }
    for (int g = tid; g <= G; g += nt) {
      gteam[g] = s_gteam[g];
      gsplit[g] = s_gsplit[g];
    }
    for (int g = tid; g < G; g += nt) {
      const int n = s_count[g], ntm = (n + tsize - 1) / tsize;
      gcount[g] = n;
      moff[g] = s_moff[g];
      for (int t = 0; t < ntm; ++t) {
        const int id = s_gteam[g] + t;
        first[id] = s_moff[g] + t * tsize;
        count[id] = min(tsize, n - t * tsize);
        group[id] = g;
      }
      for (int j = 0; j * Q < ntm; ++j) {
        sfirst[s_gsplit[g] + j] = s_gteam[g] + j * Q;
        sn[s_gsplit[g] + j] = min(Q, ntm - j * Q);
      }
    }
    return;
  }
  team_build_global(groups, F, G, tsize, order, first, count, group, gteam, nteams, gcount,
                    moff);
  // Splits: runs of up to Q consecutive teams of one group.
  __syncthreads();
  if (tid == 0) {
    int off = 0;
    for (int g = 0; g < G; ++g) {
      gsplit[g] = off;
      off += (gteam[g + 1] - gteam[g] + Q - 1) / Q;
    }
    gsplit[G] = off;
    *nsplits = off;
  }
  __syncthreads();
  for (int g = tid; g < G; g += nt) {
    const int t0 = gteam[g], ntm = gteam[g + 1] - t0;
    for (int j = 0; j * Q < ntm; ++j) {
      sfirst[gsplit[g] + j] = t0 + j * Q;
      sn[gsplit[g] + j] = min(Q, ntm - j * Q);
    }
  }
}

template <int O, bool VEC, int CT>
__global__ __launch_bounds__(kTeam* kWave)
    __attribute__((amdgpu_waves_per_eu(RQF_BWD_WAVES_PER_EU))) void selective_bwd_team_kernel(
        const rqf_selective_inputs pin, const float* __restrict__ z,
        const float* __restrict__ entries, int chunk, int nc, const float* __restrict__ gy,
        const float* __restrict__ gx, int truncated, Teams tm, BwdOut o) {
  const rqf_selective_inputs p = with_options<O>(pin);
  constexpr int K = kBwdK, TILE = kWave * K, NT = kTeam * kWave, SEG = kSegTiles * TILE;
  static_assert(TILE % NT == 0 || NT % TILE == 0, "team staging and reduction: whole tiles");
  constexpr int PER = TILE >= NT ? TILE / NT : 1;  // tile elements per thread (reduction)
  constexpr int kChans = kMaxSplitTeams * kTeam;
  __shared__ float4 s_dd[2][kTeam][TILE / 4];
  __shared__ float4 s_wg[SEG / 4], s_ws[SEG / 4];  // staged scale*(1 - tanh^2), exp(scale*tanh)
  __shared__ float s_seg[SEG];                     // the segment's group gradient so far
  __shared__ float4 s_carry[kChans];               // (dcarry, Afirst) of each channel
  __shared__ float s_cfirst[kChans];
  __shared__ double s_sum[kChans][2];              // dbias, dtheta sums of finished segments
  const int lane = lane_id();
  const int w = wave_id();
  // Logical block -> (batch chunk, split slot, batch element), XCD-contiguous chunks.
  const int64_t bc = batch_chunk(p);
  const int64_t L = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t per = (int64_t)tm.slots * bc;
  const int64_t ci = L / per, rem = L - ci * per;
  const int slot = (int)(rem / bc);
  const int64_t b = ci * bc + (rem - (int64_t)slot * bc);
  if (ci >= kXcds || b >= p.B || slot >= *tm.nsplits) return;  // block-uniform
  const int team0 = tm.sfirst[slot], nteam = tm.sn[slot];
  const int g = tm.group[team0];
  const int T = (int)p.T;
  const bool warp = p.has_warp;
  // The group's warp-logit gradient row, or this split's partial row.
  float* ddrow = nullptr;
  if (warp)
    ddrow = tm.gsplit[g + 1] - tm.gsplit[g] == 1 ? o.dd + ((int64_t)g * p.B + b) * T
                                                 : o.dd_part + ((int64_t)slot * p.B + b) * T;
  const float* dwr = warp ? p.warp_logits + ((int64_t)g * p.B + b) * T : nullptr;
  const int ntiles = (T + TILE - 1) / TILE;
  const int full = VEC ? T / TILE : 0;
  const int seg_tiles = warp ? kSegTiles : ntiles;  // no warp: one segment
  const int nseg = (ntiles + seg_tiles - 1) / seg_tiles;
  float* swg = reinterpret_cast<float*>(&s_wg[0]);
  float* sws = reinterpret_cast<float*>(&s_ws[0]);

  BwdRow r;
  r.T = T;
  r.chunk = chunk;
  r.truncated = truncated;
  r.sdd = nullptr;
  r.swg = swg;
  r.sws = sws;
  Chan c;
  int64_t row = 0;
  bool active = false;
  int members = 0;
  int parity = 0;
  for (int sg = nseg - 1; sg >= 0; --sg) {
    const int tile_lo = sg * seg_tiles, tile_hi = min(ntiles, tile_lo + seg_tiles);
    const int s0 = tile_lo * TILE;
    if (warp) {
      // Stage the segment's warp values for all teams of the split.  The
      // previous segment's last tile barrier ordered its reads before this.
      const int n = (tile_hi - tile_lo) * TILE;
      for (int i = (int)threadIdx.x; i < n; i += NT) {
        const int t = s0 + i;
        warp_stage(p, t < T ? dwr[t] : 0.0f, sws[i], swg[i]);
      }
      __syncthreads();
    }
    for (int qi = 0; qi < nteam; ++qi) {
      const int ch = qi * kTeam + w;
      if (nteam > 1 || sg == nseg - 1) {
        // Switch this wavefront to channel w of team qi.
        const int team = team0 + qi;
        members = tm.count[team];
        active = w < members;
        const int64_t f = tm.order[tm.first[team] + (active ? w : 0)];
        row = f * p.B + b;
        c = load_chan(p, f);
        const int64_t base = row * T;
        r.zr = z + 2 * base;
        r.gr = p.has_gamma ? p.gamma_logits + base : nullptr;
        r.wr = p.has_write ? p.write_logits + base : nullptr;
        r.gyr = gy ? gy + 2 * base : nullptr;
        r.gxr = gx ? gx + 2 * base : nullptr;
        r.ent = entries + 2 * row * nc;
        r.dzr = o.dz + 2 * base;
        r.dzwr = o.dzw + 2 * base;
        r.dgr = o.dg ? o.dg + base : nullptr;
        r.dwr = o.dw ? o.dw + base : nullptr;
        r.sum_bias = 0.0;
        r.sum_theta = 0.0;
        if (sg == nseg - 1) {
          r.dcarry = mk(0.0f, 0.0f);
          r.Afirst = mk(0.0f, 0.0f);
          r.cfirst = 0.0f;
        } else {
          const float4 cs = s_carry[ch];
          r.dcarry = readlane(mk(cs.x, cs.y), 0);
          r.Afirst = readlane(mk(cs.z, cs.w), 0);
          r.cfirst = readlane(s_cfirst[ch], 0);
        }
      }
      for (int tile = tile_hi - 1; tile >= tile_lo; --tile) {
        const int t0 = tile * TILE;
        if (warp) {
          r.swg = swg + (t0 - s0);
          r.sws = sws + (t0 - s0);
          r.sdd = &s_dd[parity][w][0];
        }
        if (active) {
          const c32 zprev_tile =
              t0 > 0 ? mk(r.zr[2 * (t0 - 1)], r.zr[2 * (t0 - 1) + 1]) : mk(0.0f, 0.0f);
          c32 zv[K];
          if (tile >= full) {
            load_c<K, VEC, true>(r.zr, t0 + lane * K, T, zv);
            bwd_tile<K, VEC, true, CT>(p, c, r, t0, lane, zv, zprev_tile);
          } else {
            load_c<K, VEC, false>(r.zr, t0 + lane * K, T, zv);
            bwd_tile<K, VEC, false, CT>(p, c, r, t0, lane, zv, zprev_tile);
          }
        }
        if (warp) {
          __syncthreads();
          // Thread i owns step i of every tile: the team's sum (fixed channel
          // order) joins the segment's group sum (fixed team order).
          const float* sd = reinterpret_cast<const float*>(&s_dd[parity][0][0]);
#pragma unroll
          for (int q = 0; q < PER; ++q) {
            const int i = q * NT + (int)threadIdx.x;
            if (NT > TILE && i >= TILE) break;
            float acc = 0.0f;
            for (int m = 0; m < members; ++m) acc += sd[m * TILE + i];
            const int j = t0 - s0 + i, t = t0 + i;
            if (qi > 0) acc = s_seg[j] + acc;
            if (qi + 1 < nteam)
              s_seg[j] = acc;
            else if (t < T)
              ddrow[t] = acc;
          }
        }
        parity ^= 1;
      }
      if (nteam > 1 && active) {
        // Park the channel's state until the next segment.
        const double sb = wave_sum(r.sum_bias);
        const double st = wave_sum(r.sum_theta);
        if (lane == 0) {
          const double pb = sg == nseg - 1 ? 0.0 : s_sum[ch][0];
          const double pt = sg == nseg - 1 ? 0.0 : s_sum[ch][1];
          if (sg > 0) {
            s_carry[ch] = make_float4(r.dcarry.r, r.dcarry.i, r.Afirst.r, r.Afirst.i);
            s_cfirst[ch] = r.cfirst;
            s_sum[ch][0] = pb + sb;
            s_sum[ch][1] = pt + st;
          } else {
            o.partial[row] = pb + sb;
            o.partial[p.F * p.B + row] = pt + st;
          }
        }
      }
    }
  }
  if (nteam == 1 && active) {
    const double sb = wave_sum(r.sum_bias);
    const double st = wave_sum(r.sum_theta);
    if (lane == 0) {
      o.partial[row] = sb;
      o.partial[p.F * p.B + row] = st;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward, group form: one block per (warp group, batch element) runs every
// team of the group, so the group's warp-logit gradient is complete inside
// the block: no split partial rows and no closing pass over them.  The block
// lists its group's channels itself from `groups` (no team table, no launch
// before it).  The block
// is TC x TW = 12 wavefronts, TC channel slots (one team of TC channels) times
// TW time slots (6 x 2, 4 x 3 or 3 x 4), and walks the rows backwards in super-tiles of TW consecutive
// tiles, time slot w taking tile w of each, so that concurrent
// wavefronts stream adjacent stretches of every row.  A wavefront replays its
// tile's forward from the stored entry state (entries are kept per tile),
// scans the tile's adjoint from a zero state and publishes the tile's map
//     D = R + Q conj(A') D'
// with D the adjoint at the tile's first step and A', D' the decay and the
// adjoint at the first step of the tile after it.  The channel's wavefronts
// then meet (a barrier of the channel's TW wavefronts only, on an LDS
// counter) and each composes the maps of the tiles after its own onto the
// channel's carry and forms its gradients.  The group's warp-logit gradient is
// summed in a fixed order, team after team and channel after channel: a
// wavefront waits on an LDS counter until the channel before it has added its
// tile, then adds its own straight from registers.  There is no block-wide
// barrier per super-tile, so the channels drift apart and their memory waits
// overlap each other's arithmetic, as independent blocks would.  (With two
// block barriers per super-tile the 12 wavefronts moved in lockstep: 2.84
// against 2.78 ms for the split form at config 3.)  Warp values are staged
// per segment of kGrpSegTiles tiles for all teams, behind block barriers; each
// channel's carry and fp64 sums are parked in LDS between segments.  Three
// shapes: 6 x 2, 4 x 3 and 3 x 4 (teams of 6, 4 or 3), chosen by the places
// they leave idle at the row length and group size (group_team_size).
//
// Every wait is bounded: one that runs out sets a flag that ends every other
// wait of the block at once. After its last barrier the block then writes
// NaN over every output it owns: its channels' dz / dzw, dg and dw rows, its
// dd row, and its dbias / dtheta partials. A broken dependency therefore
// shows as NaN gradients, not as a hang or as finite values composed from
// maps that never arrived.  The waits only point to earlier channels of the
// same super-tile or to the channel's own wavefronts at the same super-tile,
// so none of them is circular.
// ---------------------------------------------------------------------------
constexpr int kGrpWaves = 12;      // channel slots x time slots
// Segments of 24 tiles (6144 steps): config 3 rows restage 3 times instead of
// 6, config 4 rows (16 tiles) never.  Measured on one box, alternating builds:
// config 3 backward 2.687-2.694 -> 2.670-2.671 ms, config 4 layer 1
// 0.623-0.625 -> 0.606 ms; 36 tiles measured the same as 24 with 40% more LDS.
#ifndef RQF_GRP_SEG_TILES
#define RQF_GRP_SEG_TILES 24
#endif
constexpr int kGrpSegTiles = RQF_GRP_SEG_TILES;  // tiles per staged segment
constexpr int kGrpMaxChans = 256;  // channels of one group whose state LDS parks
constexpr int kGrpSpins = 1 << 20;  // bound on one wait (tens of ms)

// Wait until the LDS counter reaches `target`; false if the wait ran out or
// another wait of the block did.
__device__ __forceinline__ bool lds_await(int* counter, int target, int* abort) {
  for (int n = 0; n < kGrpSpins; ++n) {
    if (__hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target)
      return true;
    if (__hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  __hip_atomic_store(abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return false;
}
// Count one more arrival after the wavefront's earlier LDS writes (all lanes
// take part in the fence; lane 0 counts).
__device__ __forceinline__ void lds_release_add(int* counter, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if (lane == 0) __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int O, bool VEC, int TC, int CT>
__global__ __launch_bounds__(kGrpWaves* kWave)
    __attribute__((amdgpu_waves_per_eu(RQF_BWD_WAVES_PER_EU))) void selective_bwd_grp_kernel(
        const rqf_selective_inputs pin, const float* __restrict__ z,
        const float* __restrict__ entries, int chunk, int nc, const float* __restrict__ gy,
        const float* __restrict__ gx, int truncated, BwdOut o, int abort0) {
  const rqf_selective_inputs p = with_options<O>(pin);
  const bool trunc = truncated_of<CT>(truncated);
  constexpr int kGrpTC = TC, kGrpTW = kGrpWaves / TC, kGrpSegSt = kGrpSegTiles / kGrpTW;
  static_assert(kGrpTC * kGrpTW == kGrpWaves && kGrpSegSt * kGrpTW == kGrpSegTiles,
                "slot shape");
  constexpr int K = kBwdK, TILE = kWave * K, NT = kGrpWaves * kWave, ST = kGrpTW * TILE;
  constexpr int SEG = kGrpSegSt * ST;
  // channel places: whole teams of TC covering up to kGrpMaxChans channels
  constexpr int kChans = (kGrpMaxChans + TC - 1) / TC * TC;
  static_assert(K % 4 == 0, "whole float4s of warp gradient per lane");
  __shared__ float4 s_wg[SEG / 4], s_ws[SEG / 4];  // staged scale*(1 - tanh^2), exp(scale*tanh)
  __shared__ float4 s_seg[SEG / 4];                // the segment's group gradient so far
  __shared__ float4 s_map[2][kGrpTC][kGrpTW][2];   // (R, Q), (A at the first step, cn, -)
  __shared__ int s_arrive[kGrpTC];                 // channel barrier arrivals
  __shared__ int s_added[kGrpSegSt][kGrpTW];       // group-sum contributions so far
  __shared__ int s_abort;
  __shared__ float4 s_park[kChans];                // (D, A) carry of each channel
  __shared__ float s_pcf[kChans];                  // lag-tap weight of the carry
  __shared__ double s_sum[kChans][kGrpTW][2];      // dbias, dtheta sums per time slot
  __shared__ int s_order[kChans];                  // the group's channels, ascending
  __shared__ int s_wcnt[kGrpWaves];
  const int lane = lane_id();
  const int w = wave_id();
  // A channel's time slots are consecutive wavefronts, which the SIMDs take
  // round-robin: each SIMD holds wavefronts of different channels.
  const int cs = w / kGrpTW, tw = w % kGrpTW;
  const int64_t L = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t g = L / p.B, b = L - g * p.B;
  if (g >= p.G) return;  // block-uniform
  // The group's channels in ascending order, straight from `groups` (one
  // channel per thread: F <= kGrpMaxChans < NT): a ballot per wavefront
  // places each after the earlier wavefronts' members.  Teams are runs of TC
  // consecutive members, the last one partial.
  int ng = 0;
  {
    const int f = (int)threadIdx.x;
    const bool mine = f < p.F && group_of(p, f) == g;
    const unsigned long long m = __ballot(mine);
    if (lane == 0) s_wcnt[w] = __popcll(m);
    __syncthreads();
    int off = 0;
    for (int v = 0; v < kGrpWaves; ++v) {
      off += v < w ? s_wcnt[v] : 0;
      ng += s_wcnt[v];
    }
    if (mine) s_order[off + __popcll(m & ((1ull << lane) - 1ull))] = f;
    __syncthreads();
  }
  const int nteam = (ng + TC - 1) / TC;
  const int T = (int)p.T;
  float* ddrow = o.dd + (g * p.B + b) * T;
  if (nteam == 0) {
    // a group without channels has a zero warp-logit gradient
    for (int t = (int)threadIdx.x; t < T; t += NT) ddrow[t] = 0.0f;
    return;
  }
  const float* dwr = p.warp_logits + (g * p.B + b) * T;
  const int ntiles = (T + TILE - 1) / TILE;
  const int full = VEC ? T / TILE : 0;
  const int nst = (ntiles + kGrpTW - 1) / kGrpTW;
  const int nseg = (nst + kGrpSegSt - 1) / kGrpSegSt;
  float* swg = reinterpret_cast<float*>(&s_wg[0]);
  float* sws = reinterpret_cast<float*>(&s_ws[0]);
  float* sseg = reinterpret_cast<float*>(&s_seg[0]);
  if (threadIdx.x < kGrpTC) s_arrive[threadIdx.x] = 0;
  // abort0 (a host test switch, read once) starts the block as if a wait had
  // run out: every wait then gives up unless its count is already there.
  if (threadIdx.x == 0) s_abort = abort0 != 0;

  BwdRow r;
  r.T = T;
  r.chunk = chunk;
  r.truncated = truncated;
  r.sdd = nullptr;
  r.swg = swg;
  r.sws = sws;
  r.dcarry = mk(0.0f, 0.0f);
  r.Afirst = mk(0.0f, 0.0f);
  r.cfirst = 0.0f;
  Chan c;
  int gen = 0;  // channel barriers passed (the same count in every slot of a channel)
  // The channel's carry: adjoint, decay and lag-tap weight at the first step
  // after the super-tile being walked.
  c32 Dc = mk(0.0f, 0.0f), Ac = mk(0.0f, 0.0f);
  float cc = 0.0f;
  for (int sg = nseg - 1; sg >= 0; --sg) {
    const int st_lo = sg * kGrpSegSt, st_hi = min(nst, st_lo + kGrpSegSt);
    const int s0 = st_lo * ST;
    {
      // Stage the segment's warp values for all teams.  Every wavefront has
      // left the previous segment (the barrier) before they are replaced.
      __syncthreads();
      const int n = (st_hi - st_lo) * ST;
      for (int i = (int)threadIdx.x; i < n; i += NT) {
        const int t = s0 + i;
        warp_stage(p, t < T ? dwr[t] : 0.0f, sws[i], swg[i]);
      }
      if (threadIdx.x < kGrpSegSt * kGrpTW) (&s_added[0][0])[threadIdx.x] = 0;
      __syncthreads();
    }
    for (int qi = 0; qi < nteam; ++qi) {
      const int ch = qi * kGrpTC + cs;
      if (ch >= ng) continue;  // the whole channel slot sits this (last) team out
      const int64_t f = s_order[ch];
      const int64_t row = f * p.B + b;
      c = load_chan(p, f);
      const int64_t base = row * T;
      r.zr = z + 2 * base;
      r.gr = p.has_gamma ? p.gamma_logits + base : nullptr;
      r.wr = p.has_write ? p.write_logits + base : nullptr;
      r.gyr = gy ? gy + 2 * base : nullptr;
      r.gxr = gx ? gx + 2 * base : nullptr;
      r.ent = entries + 2 * row * nc;
      r.dzr = o.dz + 2 * base;
      r.dzwr = o.dzw + 2 * base;
      r.dgr = o.dg ? o.dg + base : nullptr;
      r.dwr = o.dw ? o.dw + base : nullptr;
      r.sum_bias = 0.0;
      r.sum_theta = 0.0;
      if (sg == nseg - 1) {
        Dc = mk(0.0f, 0.0f);
        Ac = mk(0.0f, 0.0f);
        cc = 0.0f;
      } else {
        const float4 v = s_park[ch];
        Dc = mk(v.x, v.y);
        Ac = mk(v.z, v.w);
        cc = s_pcf[ch];
      }
      // this channel's place in the group sum's order, and the last place
      const int place = ch;
      const int last = ng - 1;
      for (int st = st_hi - 1; st >= st_lo; --st) {
        const int tile = st * kGrpTW + tw;
        const int t0 = tile * TILE;
        const bool valid = tile < ntiles;
        const int buf = gen & 1;
        r.swg = swg + (t0 - s0);
        r.sws = sws + (t0 - s0);
        BwdTile<K> s;
        c32 zv[K];
        c32 Q = mk(1.0f, 0.0f), rr = mk(0.0f, 0.0f);
        if (valid) {
          const c32 zprev_tile =
              t0 > 0 ? mk(r.zr[2 * (t0 - 1)], r.zr[2 * (t0 - 1) + 1]) : mk(0.0f, 0.0f);
          if (tile >= full) {
            load_c<K, VEC, true>(r.zr, t0 + lane * K, T, zv);
            bwd_tile_replay<K, VEC, true, CT>(p, c, r, t0, lane, zv, zprev_tile, s);
          } else {
            load_c<K, VEC, false>(r.zr, t0 + lane * K, T, zv);
            bwd_tile_replay<K, VEC, false, CT>(p, c, r, t0, lane, zv, zprev_tile, s);
          }
          if (!trunc) {
            // Lane 63's step after its last is the next tile's first: its
            // decay stays out of the tile's own map (1 here) and comes in with D'.
            const c32 A_ln = shift_down(s.A[0], mk(1.0f, 0.0f), lane);
            if (tile >= full)
              bwd_lane_adjoint<K, true>(s, A_ln, Q, rr);
            else
              bwd_lane_adjoint<K, false>(s, A_ln, Q, rr);
            wave_scan_rev(Q, rr, lane);
          }
          if (lane == 0) {
            s_map[buf][cs][tw][0] = trunc ? make_float4(s.ecot[0].r, s.ecot[0].i, 0.0f, 0.0f)
                                              : make_float4(rr.r, rr.i, Q.r, Q.i);
            s_map[buf][cs][tw][1] = make_float4(s.A[0].r, s.A[0].i, s.c0, 0.0f);
          }
        } else if (lane == 0) {
          // a tile past the row's end: zero adjoint, decay and lag tap
          s_map[buf][cs][tw][0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          s_map[buf][cs][tw][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        // Channel barrier: the channel's maps of this super-tile are in.
        ++gen;
        lds_release_add(&s_arrive[cs], lane);
        lds_await(&s_arrive[cs], kGrpTW * gen, &s_abort);
        // Compose the maps of the super-tile's tiles, latest first, onto the
        // carry: (Dn, An, cn) at the first step after tile tw, and the carry
        // for the super-tile before this one.
        c32 Dn = Dc, An = Ac, D1 = Dc, A1 = Ac;
        float cn = cc, c1 = cc;
#pragma unroll
        for (int j = kGrpTW - 1; j >= 0; --j) {
          if (j == tw) {
            D1 = Dn;
            A1 = An;
            c1 = cn;
          }
          const float4 m0 = s_map[buf][cs][j][0], m1 = s_map[buf][cs][j][1];
          Dn = trunc ? mk(m0.x, m0.y) : cmad(mk(m0.z, m0.w), cjmul(An, Dn), mk(m0.x, m0.y));
          An = mk(m1.x, m1.y);
          cn = m1.z;
        }
        Dc = Dn;
        Ac = An;
        cc = cn;
        float gd[K];
#pragma unroll
        for (int k = 0; k < K; ++k) gd[k] = 0.0f;
        if (valid) {
          const c32 A_lane_next = shift_down(s.A[0], A1, lane);
          const float cn_lane_next = shift_down(s.c0, c1, lane);
          c32 dnext;
          if (trunc) {
            dnext = shift_down(s.ecot[0], D1, lane);
          } else {
            // the lane's adjoint at its first step, then the next lane's
            const c32 dfirst = cmad(Q, cjmul(A1, D1), rr);
            dnext = shift_down(dfirst, D1, lane);
          }
          if (tile >= full)
            bwd_tile_grads<K, VEC, true, CT>(p, c, r, t0, lane, zv, s, dnext, A_lane_next,
                                               cn_lane_next, gd);
          else
            bwd_tile_grads<K, VEC, false, CT>(p, c, r, t0, lane, zv, s, dnext, A_lane_next,
                                                cn_lane_next, gd);
        }
        // The group sum of this tile's steps, in the fixed (team, channel)
        // order: wait for the channel before, add, pass on.
        int* added = &s_added[st - st_lo][tw];
        lds_await(added, place, &s_abort);
        const int j0 = t0 - s0 + lane * K, tb = t0 + lane * K;
        float4 acc = make_float4(gd[0], gd[1], gd[2], gd[3]);
        if (place > 0) {
          const float4 prev = reinterpret_cast<const float4*>(sseg + j0)[0];
          acc = make_float4(prev.x + acc.x, prev.y + acc.y, prev.z + acc.z, prev.w + acc.w);
        }
        if (place < last) {
          reinterpret_cast<float4*>(sseg + j0)[0] = acc;
        } else if (VEC && tb + K <= T) {
          *reinterpret_cast<float4*>(ddrow + tb) = acc;
        } else {
          const float a4[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (tb + k < T) ddrow[tb + k] = a4[k];
        }
        lds_release_add(added, lane);
      }
      // Park the channel's carry (every time slot holds the same one) and add
      // this wavefront's sums to its slot.
      if (sg > 0 && tw == 0 && lane == 0) {
        s_park[ch] = make_float4(Dc.r, Dc.i, Ac.r, Ac.i);
        s_pcf[ch] = cc;
      }
      const double sb = wave_sum(r.sum_bias);
      const double sth = wave_sum(r.sum_theta);
      if (lane == 0) {
        s_sum[ch][tw][0] = (sg == nseg - 1 ? 0.0 : s_sum[ch][tw][0]) + sb;
        s_sum[ch][tw][1] = (sg == nseg - 1 ? 0.0 : s_sum[ch][tw][1]) + sth;
      }
    }
  }
  __syncthreads();
  if (s_abort) {
    // A wait ran out (block-uniform after the barrier): carries and group sums
    // may have been composed from maps that had not arrived, so every output
    // row this block owns is overwritten with NaN, not left finite and wrong.
    const float nan = __builtin_nanf("");
    for (int i = 0; i < ng; ++i) {
      const int64_t base = ((int64_t)s_order[i] * p.B + b) * T;
      for (int t = (int)threadIdx.x; t < 2 * T; t += NT) {
        o.dzw[2 * base + t] = nan;
        if (truncated) o.dz[2 * base + t] = nan;
      }
      for (int t = (int)threadIdx.x; t < T; t += NT) {
        if (o.dg) o.dg[base + t] = nan;
        if (o.dw) o.dw[base + t] = nan;
      }
    }
    for (int t = (int)threadIdx.x; t < T; t += NT) ddrow[t] = nan;
  }
  // Per-row fp64 partials of dbias and dtheta: the time slots in fixed order.
  for (int i = (int)threadIdx.x; i < ng; i += NT) {
    {
      const int64_t row = (int64_t)s_order[i] * p.B + b;
      double sb = 0.0, sth = 0.0;
#pragma unroll
      for (int j = 0; j < kGrpTW; ++j) {
        sb += s_sum[i][j][0];
        sth += s_sum[i][j][1];
      }
      if (s_abort) sb = sth = __builtin_nan("");  // a wait ran out: flag the results
      o.partial[row] = sb;
      o.partial[p.F * p.B + row] = sth;
    }
  }
}

// dd[g, b, t] = sum over the splits of group g (fixed order) of dd_part[split, b, t],
// for groups not served by exactly one split (those wrote dd directly).
// VEC: N % 4 == 0 and 16-byte aligned dd; thread i sums one float4.
template <bool VEC>
__device__ __forceinline__ void team_reduce_at(int64_t i, const float* __restrict__ dd_part,
                                               const int* __restrict__ gsplit,
                                               float* __restrict__ dd, int64_t G, int64_t N) {
  if (VEC) {
    const int64_t n4 = N / 4;
    if (i >= G * n4) return;
    const int64_t g = i / n4, n = (i - g * n4) * 4;
    if (gsplit[g + 1] - gsplit[g] == 1) return;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s = gsplit[g]; s < gsplit[g + 1]; ++s) {
      const float4 v = ld4(dd_part + (int64_t)s * N + n);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    st4(dd + g * N + n, acc);
  } else {
    if (i >= G * N) return;
    const int64_t g = i / N, n = i - g * N;
    if (gsplit[g + 1] - gsplit[g] == 1) return;
    float acc = 0.0f;
    for (int s = gsplit[g]; s < gsplit[g + 1]; ++s) acc += dd_part[(int64_t)s * N + n];
    dd[i] = acc;
  }
}


// dbias[f] = sum_b partial[f*B + b] in fp64, same for dtheta: one wavefront
// per channel, lane l sums b = l, l+64, ... in order, then a fixed-shape wave
// reduction (deterministic).
__device__ __forceinline__ void partial_reduce_at(int64_t f, int lane,
                                                  const double* __restrict__ partial,
                                                  float* __restrict__ dbias,
                                                  float* __restrict__ dtheta, int64_t F,
                                                  int64_t B) {
  double sb = 0.0, st = 0.0;
  for (int64_t b = lane; b < B; b += kWave) {
    sb += partial[f * B + b];
    st += partial[F * B + f * B + b];
  }
  sb = wave_sum(sb);
  st = wave_sum(st);
  if (lane == 0) {
    dbias[f] = (float)sb;
    dtheta[f] = (float)st;
  }
}

// The backward's closing pass, one launch: blocks [0, dd_blocks) sum the
// split partial rows of the warp-logit gradient (dd_part may be null, then
// dd_blocks is 0), the blocks after them reduce dbias and dtheta, one
// wavefront per channel.
constexpr int kFinishThreads = 256;
template <bool VEC>
__global__ __launch_bounds__(kFinishThreads) void bwd_finish_kernel(
    const float* __restrict__ dd_part, const int* __restrict__ gsplit, float* __restrict__ dd,
    int64_t G, int64_t N, int64_t dd_blocks, const double* __restrict__ partial,
    float* __restrict__ dbias, float* __restrict__ dtheta, int64_t F, int64_t B) {
  if ((int64_t)blockIdx.x < dd_blocks) {
    team_reduce_at<VEC>((int64_t)blockIdx.x * kFinishThreads + threadIdx.x, dd_part, gsplit, dd,
                        G, N);
    return;
  }
  const int64_t f = ((int64_t)blockIdx.x - dd_blocks) * (kFinishThreads / kWave) + wave_id();
  if (f < F) partial_reduce_at(f, lane_id(), partial, dbias, dtheta, F, B);
}

// Blocks of the finishing pass: the dd items (float4s with `vec`), then one
// wavefront per channel.
int64_t finish_dd_blocks(int64_t G, int64_t N, bool with_dd, bool vec) {
  const int64_t items = with_dd ? (vec ? G * (N / 4) : G * N) : 0;
  return (items + kFinishThreads - 1) / kFinishThreads;
}
int64_t finish_pr_blocks(int64_t F) {
  return (F + kFinishThreads / kWave - 1) / (kFinishThreads / kWave);
}

void launch_finish(const float* dd_part, const int* gsplit, float* dd, int64_t G, int64_t N,
                   const double* partial, float* dbias, float* dtheta, int64_t F, int64_t B,
                   hipStream_t s) {
  const bool vec = dd_part && N % 4 == 0 && ((uintptr_t)dd & 15) == 0;
  const int64_t dd_blocks = finish_dd_blocks(G, N, dd_part != nullptr, vec);
  const int64_t pr_blocks = finish_pr_blocks(F);
  const dim3 grid((unsigned)(dd_blocks + pr_blocks)), block(kFinishThreads);
  if (dd_blocks + pr_blocks == 0) return;
  if (vec)
    hipLaunchKernelGGL(bwd_finish_kernel<true>, grid, block, 0, s, dd_part, gsplit, dd, G, N,
                       dd_blocks, partial, dbias, dtheta, F, B);
  else
    hipLaunchKernelGGL(bwd_finish_kernel<false>, grid, block, 0, s, dd_part, gsplit, dd, G, N,
                       dd_blocks, partial, dbias, dtheta, F, B);
}

// Zero-fill of n 32-bit words (graph-capture safe, unlike a memset node),
// grid-stride over at most stride_blocks blocks.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

void zero_words(void* p, int64_t nwords, hipStream_t s) {
  if (nwords > 0)
    hipLaunchKernelGGL(zero_words_kernel, dim3(stride_blocks((nwords + 255) / 256)), dim3(256), 0,
                       s, (uint32_t*)p, nwords);
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
// Chunk as a kernel int: anything >= 2^30 behaves like 2^30 since T < 2^30.
inline int chunk_int(int64_t chunk) { return (int)(chunk > (1 << 30) ? (1 << 30) : chunk); }

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RQF_OK : (int)err;
}

int check_inputs(const rqf_selective_inputs* in) {
  if (!in || in->F < 0 || in->B < 0 || in->T < 0) return RQF_ERR_ARG;
  if (in->T >= ((int64_t)1 << 30)) return RQF_ERR_ARG;  // in-row offsets are 32-bit
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

int options_of(const rqf_selective_inputs* in) {
  const int o = (in->has_gamma ? kOptGamma : 0) | (in->log_shift ? kOptLogShift : 0) |
                (in->has_warp ? kOptWarp : 0) | (in->bound_warp ? kOptBound : 0) |
                (in->has_write ? kOptWrite : 0) | (in->write_sigmoid ? kOptWriteSigmoid : 0) |
                (in->prospective ? kOptProspective : 0) |
                (in->gamma_horizon ? kOptGammaHorizon : 0);
  return normalise_options(o);
}

// Calls fn(std::integral_constant<int, O>) with O the compiled option set equal
// to `opts`, or kOptRuntime when none is.
template <class Fn>
void with_option_set(int opts, Fn&& fn) {
  static_assert(sizeof(kOptSets) / sizeof(kOptSets[0]) == 3, "one case per compiled set");
  switch (opts) {
    case kOptSets[0]: fn(std::integral_constant<int, kOptSets[0]>{}); return;
    case kOptSets[1]: fn(std::integral_constant<int, kOptSets[1]>{}); return;
    case kOptSets[2]: fn(std::integral_constant<int, kOptSets[2]>{}); return;
    default: fn(std::integral_constant<int, kOptRuntime>{}); return;
  }
}

// Cotangent set a backward call is compiled for: fixed under full BPTT with
// float4 rows and a compiled option set, else run time.
int cotangent_set(int opts, bool vec, const float* gy, const float* gx, bool truncated) {
  if (truncated || !vec || opts == kOptRuntime || (!gy && !gx)) return kCtRuntime;
  return gy && gx ? kCtGyGx : (gy ? kCtGy : kCtGx);
}

// Calls fn(std::integral_constant<int, CT>) with CT the compiled cotangent set.
template <class Fn>
void with_cotangent_set(int ct, Fn&& fn) {
  switch (ct) {
    case kCtGy: fn(std::integral_constant<int, kCtGy>{}); return;
    case kCtGyGx: fn(std::integral_constant<int, kCtGyGx>{}); return;
    case kCtGx: fn(std::integral_constant<int, kCtGx>{}); return;
    default: fn(std::integral_constant<int, kCtRuntime>{}); return;
  }
}

// RQF_GRP_FORCE_TIMEOUT=1 starts every block of the group-form backward in
// the state a wait that ran out leaves (tests of that path): the waits give up
// at once and every output the blocks own is written as NaN, without
// hanging.  The flag is read once per block, so the wait loops keep
// their constant bound and no register.
int grp_force_timeout() {
  const char* e = std::getenv("RQF_GRP_FORCE_TIMEOUT");
  return e && !std::strcmp(e, "1") ? 1 : 0;
}

// Forward block size: kFwdRbWavesRaw wavefronts for calls that stream z, the
// logits and one complex output (raw or act); kFwdRbWaves when both outputs
// or a skip tensor add streams.  The act-only contract at config 3's shape,
// rotated runs on one box: 1.314 -> 1.282 ms with the narrow blocks.
// RQF_FWD_WAVES=narrow|wide forces one (tests and tuning).
bool fwd_narrow_blocks(bool extra_streams) {
  if (const char* e = std::getenv("RQF_FWD_WAVES")) {
    if (!std::strcmp(e, "narrow")) return true;
    if (!std::strcmp(e, "wide")) return false;
  }
  return !extra_streams;
}

// Logical rows of the forward's grid: the batch in kXcds chunks of
// ceil(B / kXcds) elements, times F channels (row_id).
int64_t fwd_blocks(const rqf_selective_inputs* in) {
  return kXcds * in->F * ((in->B + kXcds - 1) / kXcds);
}
constexpr int kFwdMaxThreads = std::max(kFwdRbWaves, kFwdRbWavesRaw) * kWave;

void launch_fwd(const rqf_selective_inputs* in, const float* z, const float* skip, float* raw,
                float* act, float* entries, int chunk, int nc, bool vec, hipStream_t s) {
  const dim3 grid((unsigned)fwd_blocks(in));
  const bool narrow = fwd_narrow_blocks((raw != nullptr && act != nullptr) || skip != nullptr);
  const dim3 block((narrow ? kFwdRbWavesRaw : kFwdRbWaves) * kWave);
  with_option_set(options_of(in), [&](auto oc) {
    constexpr int O = decltype(oc)::value;
    if (narrow) {
      if (vec)
        hipLaunchKernelGGL((selective_fwd_rb_kernel<O, true, kFwdRbWavesRaw>), grid, block, 0, s,
                           *in, z, skip, raw, act, entries, chunk, nc);
      else
        hipLaunchKernelGGL((selective_fwd_rb_kernel<O, false, kFwdRbWavesRaw>), grid, block, 0,
                           s, *in, z, skip, raw, act, entries, chunk, nc);
    } else {
      if (vec)
        hipLaunchKernelGGL((selective_fwd_rb_kernel<O, true, kFwdRbWaves>), grid, block, 0, s,
                           *in, z, skip, raw, act, entries, chunk, nc);
      else
        hipLaunchKernelGGL((selective_fwd_rb_kernel<O, false, kFwdRbWaves>), grid, block, 0, s,
                           *in, z, skip, raw, act, entries, chunk, nc);
    }
  });
}

constexpr int kBwdTile = kWave * kBwdK;

// Entry states of every backward tile for a call whose chunk is longer than
// one tile.  The forward kept the state entering each chunk.  One wavefront
// per (row, chunk) starts from it and replays the chunk's tiles except the
// last, whose exit is the next chunk's entry.  It records the state entering
// each tile.  A tile is the coefficients of its steps, the lanes' composed
// maps and one wave scan; its exit is the scan's total applied to the carry.
// Against a full forward, a chunk of c tiles reads and computes c - 1 of them
// and writes no outputs, and its wavefronts run every (row, chunk) at once.
// Every replayed tile ends before T (its exit enters a tile that exists), so
// no tile is ragged.
constexpr int kRebuildWaves = 4;
template <int O, bool VEC>
__global__ __launch_bounds__(kRebuildWaves* kWave) void selective_rebuild_kernel(
    const rqf_selective_inputs pin, const float* __restrict__ z,
    const float* __restrict__ entries, int chunk, int nc, float* __restrict__ tile_entries,
    int nt, int64_t tasks) {
  constexpr int K = kBwdK, TILE = kBwdTile;
  const rqf_selective_inputs p = with_options<O>(pin);
  __shared__ float4 s_io[kRebuildWaves][TILE / 2];
  const int lane = lane_id();
  const int64_t task = (int64_t)blockIdx.x * kRebuildWaves + wave_id();
  if (task >= tasks) return;  // wave-uniform
  const int64_t row = task / nc;
  const int ci = (int)(task - row * nc);
  const int64_t f = row / p.B, b = row - f * p.B;
  const Chan c = load_chan(p, f);
  FwdRow r{};  // inputs only: no outputs, skip or entries are written through it
  r.T = (int)p.T;
  const int T = r.T;
  const int64_t base = row * T;
  r.zr = z + 2 * base;
  r.gr = p.has_gamma ? p.gamma_logits + base : nullptr;
  r.wr = p.has_write ? p.write_logits + base : nullptr;
  r.dr = p.has_warp ? p.warp_logits + (group_of(p, f) * p.B + b) * T : nullptr;
  r.io = &s_io[wave_id()][0];
  const int per = chunk / TILE;  // tiles per chunk
  const int tile0 = ci * per;
  c32 y = mk(entries[2 * (row * nc + ci)], entries[2 * (row * nc + ci) + 1]);
  float* te = tile_entries + 2 * row * nt;
  if (lane == 0) {
    te[2 * tile0] = y.r;
    te[2 * tile0 + 1] = y.i;
  }
  for (int j = 0; j + 1 < per && tile0 + j + 1 < nt; ++j) {
    const int t0 = (tile0 + j) * TILE;
    const c32 zlast = t0 > 0 ? mk(r.zr[2 * (t0 - 1)], r.zr[2 * (t0 - 1) + 1]) : mk(0.0f, 0.0f);
    FwdIn<K> in;
    c32 A[K], u[K];
    fwd_load<K, VEC, false>(p, r, t0, lane, in);
    fwd_steps<K, false>(p, c, T, t0, lane, in, zlast, A, u);
    c32 P = A[0], s = u[0];
#pragma unroll
    for (int k = 1; k < K; ++k) {
      s = cmad(A[k], s, u[k]);
      P = cmul(A[k], P);
    }
    wave_scan_fwd(P, s);  // lane 63: the whole tile's map
    y = cmad(readlane(P, kWave - 1), y, readlane(s, kWave - 1));
    if (lane == 0) {
      te[2 * (tile0 + j + 1)] = y.r;
      te[2 * (tile0 + j + 1) + 1] = y.i;
    }
  }
}

int64_t rebuild_tasks(const rqf_selective_inputs* in, int nc) { return in->F * in->B * nc; }
int64_t rebuild_blocks(const rqf_selective_inputs* in, int nc) {
  return (rebuild_tasks(in, nc) + kRebuildWaves - 1) / kRebuildWaves;
}

void launch_rebuild(const rqf_selective_inputs* in, const float* z, const float* entries,
                    int chunk, int nc, float* tile_entries, int nt, bool vec, hipStream_t s) {
  const dim3 grid((unsigned)rebuild_blocks(in, nc)), block(kRebuildWaves * kWave);
  const int64_t tasks = rebuild_tasks(in, nc);
  with_option_set(options_of(in), [&](auto oc) {
    constexpr int O = decltype(oc)::value;
    if (vec)
      hipLaunchKernelGGL((selective_rebuild_kernel<O, true>), grid, block, 0, s, *in, z, entries,
                         chunk, nc, tile_entries, nt, tasks);
    else
      hipLaunchKernelGGL((selective_rebuild_kernel<O, false>), grid, block, 0, s, *in, z, entries,
                         chunk, nc, tile_entries, nt, tasks);
  });
}

}  // namespace

namespace {
int selective_fwd(const rqf_selective_inputs* in, const float* z, int64_t chunk, const float* skip,
                  float* raw, float* act, float* entries, rqf_stream_t stream) {
  if (!in || in->F < 0 || in->B < 0 || in->T < 0 || !pow2(chunk)) return RQF_ERR_ARG;
  const int64_t R = in->F * in->B;
  if (R == 0 || in->T == 0) return RQF_OK;
  int st = check_inputs(in);
  if (st) return st;
  if (!z || !entries || (!raw && !act)) return RQF_ERR_ARG;
  if (!grid_fits(fwd_blocks(in), kFwdMaxThreads)) return RQF_ERR_ARG;
  if (!aligned8(z) || !aligned8(skip) || !aligned8(raw) || !aligned8(act) || !aligned8(entries))
    return RQF_ERR_ALIGN;
  const int nc = (int)((in->T + chunk - 1) / chunk);
  launch_fwd(in, z, skip, raw, act, entries, chunk_int(chunk), nc,
             vec_ok(in, {z, skip, raw, act}), (hipStream_t)stream);
  return launch_status();
}
}  // namespace

extern "C" int rqf_selective_fwd(const rqf_selective_inputs* in, const float* z, int64_t chunk,
                                 float* raw, float* act, float* entries, rqf_stream_t stream) {
  return selective_fwd(in, z, chunk, nullptr, raw, act, entries, stream);
}

extern "C" int rqf_selective_skip_fwd(const rqf_selective_inputs* in, const float* z,
                                      int64_t chunk, const float* skip, float* raw, float* act,
                                      float* entries, rqf_stream_t stream) {
  if (!skip && in && in->F * in->B * in->T > 0) return RQF_ERR_ARG;
  return selective_fwd(in, z, chunk, skip, raw, act, entries, stream);
}

namespace {
// Teams per split of the backward (see the team kernel).
int split_teams(const rqf_selective_inputs* in) {
  if (!in->has_warp) return 1;
  if (const char* e = std::getenv("RQF_BWD_SPLIT_TEAMS")) {
    const int q = std::atoi(e);
    if (q > 0) return std::min(q, kMaxSplitTeams);
  }
  // Balanced groups assumed: at least kSplitBlocksPerCu blocks per CU.
  const int64_t teams = (in->F + kTeam - 1) / kTeam;
  const int64_t q = teams * in->B / (kSplitBlocksPerCu * kCus);
  return (int)std::max<int64_t>(1, std::min<int64_t>(kMaxSplitTeams, q));
}

// Channel slots of the group form's blocks (6 x 2, 4 x 3 or 3 x 4
// wavefronts): the shape that leaves the fewest (time slot, channel slot)
// places idle, with the group size taken as F / G (balanced groups); on a tie
// the one with more channel slots, whose tiles compose fewer maps.  At config
// 4's layer 0 (16 tiles, 64 channels per group: 3 x 4 and 6 x 2 both leave 2
// of 66 channel places idle) 6 x 2 measured 0.690 against 0.725 ms; at config
// 3 (63 tiles, 32 channels) 4 x 3 leaves none idle and measured 2.73 against
// 2.78 ms for 6 x 2.  (2 x 6 spills registers: 0.745 ms at config 4.)
// RQF_BWD_GRP_TEAM=3|4|6 picks one for tests and tuning.
int group_team_size(const rqf_selective_inputs* in) {
  if (const char* e = std::getenv("RQF_BWD_GRP_TEAM")) {
    if (!std::strcmp(e, "3")) return 3;
    if (!std::strcmp(e, "4")) return 4;
    if (!std::strcmp(e, "6")) return 6;
  }
  const int64_t ntiles = (in->T + kBwdTile - 1) / kBwdTile;
  const int64_t n = std::max<int64_t>(1, in->F / std::max<int64_t>(1, in->G));
  int64_t best_idle = -1;
  int best = 4;
  if (ntiles == 0) return best;  // no tiles (T = 0): any shape, and no places to divide by
  for (int tc : {6, 4, 3}) {
    const int64_t tw = kGrpWaves / tc;
    const int64_t places = (ntiles + tw - 1) / tw * tw * ((n + tc - 1) / tc * tc);
    // idle places per 10^4, so that the two shapes compare exactly
    const int64_t idle = (places - ntiles * n) * 10000 / places;
    if (best_idle < 0 || idle < best_idle) {
      best_idle = idle;
      best = tc;
    }
  }
  return best;
}

// The group form of the backward needs the warp head and no group with more
// channels than its LDS parks (F <= kGrpMaxChans).  It runs by default when
// the (group, batch element) blocks give every CU one and its chosen shape
// leaves at most 1/32 of the places idle, on the memory-heavier contract
// (with the activation's cotangent gx: 48 B per element) or in the 6 x 2
// shape.  Without gx (40 B per element) the tiles' arithmetic dominates, and
// composing 3 or 4 tiles' maps costs more than the form's overlap gains.
// Measured against the split form (ms): config 3's shape, 4 x 3, with gx
// 2.70-2.75 against 2.75-2.79, without gx 2.58 against 2.52-2.55; config 4's
// layer 0 (gx) 0.686-0.690 in 6 x 2 against 0.738-0.743; its layer 1 (no gx)
// 0.651-0.653 in 6 x 2 against 0.667, and 0.695-0.702 in 3 x 4 against
// 0.647-0.649 (another box).  The environment variable RQF_BWD_FORM=group|split
// picks a form for tests and tuning; setting RQF_BWD_SPLIT_TEAMS picks the
// split form.
bool use_group_form(const rqf_selective_inputs* in, bool with_gx) {
  if (!in->has_warp || in->F > kGrpMaxChans) return false;
  if (std::getenv("RQF_BWD_SPLIT_TEAMS")) return false;
  if (const char* e = std::getenv("RQF_BWD_FORM")) {
    if (!std::strcmp(e, "group")) return true;
    if (!std::strcmp(e, "split")) return false;
  }
  const int tc = group_team_size(in), tw = kGrpWaves / tc;
  const int64_t ntiles = (in->T + kBwdTile - 1) / kBwdTile;
  const int64_t n = std::max<int64_t>(1, in->F / std::max<int64_t>(1, in->G));
  const int64_t places = (ntiles + tw - 1) / tw * tw * ((n + tc - 1) / tc * tc);
  return (with_gx || tc == 6) && in->G * in->B >= kCus && places > 0 &&
         (places - ntiles * n) * 32 <= places;
}

struct SelWs {
  size_t partial, tile_entries, teams, dd, total;
  int slots, split_slots, Q, G, tsize;
  bool group_form;
};
SelWs sel_ws_layout(const rqf_selective_inputs* in, int64_t chunk, bool group_form) {
  SelWs w;
  const int64_t R = in->F * in->B;
  w.G = in->has_warp ? (int)in->G : 1;
  w.group_form = group_form;
  w.tsize = w.group_form ? group_team_size(in) : kTeam;
  const int teams = (int)((in->F + w.tsize - 1) / w.tsize);
  w.slots = w.G + teams;  // teams of all groups <= ceil(F/tsize) + G
  w.Q = split_teams(in);
  w.split_slots = std::min(w.slots, (teams + w.G) / w.Q + w.G);
  w.partial = 0;
  size_t off = round256(sizeof(double) * 2 * (size_t)R);
  w.tile_entries = off;
  if (chunk > kBwdTile)
    off += round256(sizeof(float) * 2 * (size_t)R * ((in->T + kBwdTile - 1) / kBwdTile + 1));
  w.teams = off;
  if (!w.group_form)  // the group form builds its channel lists in LDS
    off += round256(sizeof(int) * (size_t)(in->F + 5 * w.slots + 4 * w.G + 4));
  w.dd = off;
  if (in->has_warp && !w.group_form)
    off += round256(sizeof(float) * (size_t)w.split_slots * in->B * in->T);
  w.total = off;
  return w;
}

// Every grid a non-empty backward launches, within one dispatch's work-item
// count: the tile-entry rebuild (chunk > one tile), the group form's (group,
// batch element) blocks or the split form's team blocks, and the finishing
// pass (the split form's dd items, one wavefront per channel).
bool bwd_grids_fit(const rqf_selective_inputs* in, const SelWs& w, int64_t chunk) {
  const int nc = (int)((in->T + chunk - 1) / chunk);
  if (chunk > kBwdTile && !grid_fits(rebuild_blocks(in, nc), kRebuildWaves * kWave))
    return false;
  const int64_t pr = finish_pr_blocks(in->F);
  if (w.group_form)
    return grid_fits(in->G * in->B, kGrpWaves * kWave) && grid_fits(pr, kFinishThreads);
  const int64_t bc = (in->B + kXcds - 1) / kXcds;
  const int64_t dd = finish_dd_blocks(in->G, in->B * in->T, in->has_warp, false);
  return grid_fits(kXcds * w.split_slots * bc, kTeam * kWave) &&
         grid_fits(dd + pr, kFinishThreads);
}
}  // namespace

extern "C" size_t rqf_selective_bwd_workspace(const rqf_selective_inputs* in, int64_t chunk) {
  if (!in || in->F < 0 || in->B < 0 || in->T < 0) return 0;
  // enough for either form of the backward (the form depends on gx)
  return std::max(sel_ws_layout(in, chunk, false).total,
                  use_group_form(in, true) ? sel_ws_layout(in, chunk, true).total : size_t(0));
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
  const SelWs w = sel_ws_layout(in, chunk, use_group_form(in, gx != nullptr));
  if (nonempty ? !bwd_grids_fit(in, w, chunk)
               : !grid_fits(finish_pr_blocks(in->F), kFinishThreads))
    return RQF_ERR_ARG;
  if (workspace_bytes < w.total || (w.total && !workspace)) return RQF_ERR_WORKSPACE;
  if (!aligned8(z) || !aligned8(gy) || !aligned8(gx) || !aligned8(dz) || !aligned8(dzw))
    return RQF_ERR_ALIGN;
  const int64_t R = in->F * in->B, T = in->T;
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  double* partial = (double*)(ws + w.partial);
  if (nonempty) {
    const bool vec = vec_ok(in, {z, gy, gx, dz, dzw, dg, dw, dd});
    const float* ent = entries;
    int ent_chunk = chunk_int(chunk), nc = (int)((T + chunk - 1) / chunk);
    if (chunk > kBwdTile) {
      // Entry states at every backward tile, replayed from the chunk entries.
      float* te = (float*)(ws + w.tile_entries);
      const int nt = (int)((T + kBwdTile - 1) / kBwdTile);
      launch_rebuild(in, z, entries, ent_chunk, nc, te, nt, vec_ok(in, {z}), s);
      ent = te;
      ent_chunk = kBwdTile;
      nc = nt;
    }
    BwdOut o;
    o.dz = dz;
    o.dzw = dzw;
    o.dg = in->has_gamma ? dg : nullptr;
    o.dw = in->has_write ? dw : nullptr;
    o.dd_part = nullptr;
    o.partial = partial;
    o.dd = in->has_warp ? dd : nullptr;
    // The group form finds its group's channels itself: no team table.
    if (w.group_form) {
      const dim3 grid((unsigned)(in->G * in->B)), block(kGrpWaves * kWave);
      const int abort0 = grp_force_timeout();
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, s, *in, z, ent, ent_chunk, nc, gy, gx,
                           (int)truncated, o, abort0);
      };
      const int opts = options_of(in);
      with_option_set(opts, [&](auto oc) {
        constexpr int O = decltype(oc)::value;
        if constexpr (O != kOptRuntime && !(O & kOptWarp)) {
          return;  // not reached: the group form needs the warp head
        } else {
          with_cotangent_set(cotangent_set(O, vec, gy, gx, truncated), [&](auto cc) {
            constexpr int CT = decltype(cc)::value;
            if constexpr (CT != kCtRuntime) {
              // fixed sets: float4 rows under a compiled option set only
              if constexpr (O != kOptRuntime) {
                if (w.tsize == 3)
                  go(selective_bwd_grp_kernel<O, true, 3, CT>);
                else if (w.tsize == 6)
                  go(selective_bwd_grp_kernel<O, true, 6, CT>);
                else
                  go(selective_bwd_grp_kernel<O, true, 4, CT>);
              }
            } else if (w.tsize == 3) {
              vec ? go(selective_bwd_grp_kernel<O, true, 3, CT>)
                  : go(selective_bwd_grp_kernel<O, false, 3, CT>);
            } else if (w.tsize == 6) {
              vec ? go(selective_bwd_grp_kernel<O, true, 6, CT>)
                  : go(selective_bwd_grp_kernel<O, false, 6, CT>);
            } else {
              vec ? go(selective_bwd_grp_kernel<O, true, 4, CT>)
                  : go(selective_bwd_grp_kernel<O, false, 4, CT>);
            }
          });
        }
      });
      launch_finish(nullptr, nullptr, nullptr, 0, 0, partial, dbias, dtheta, in->F, in->B, s);
      return launch_status();
    }
    int* order = (int*)(ws + w.teams);
    int* first = order + in->F;
    int* count = first + w.slots;
    int* group = count + w.slots;
    int* gteam = group + w.slots;
    int* nteams = gteam + (w.G + 1);
    int* gcount = nteams + 1;
    int* moff = gcount + w.G;
    int* sfirst = moff + w.G;
    int* sn = sfirst + w.slots;
    int* gsplit = sn + w.slots;
    int* nsplits = gsplit + (w.G + 1);
    hipLaunchKernelGGL(team_build_kernel, dim3(1), dim3(256), 0, s,
                       in->has_warp ? in->groups : (const int64_t*)nullptr, (int)in->F, w.G, w.Q,
                       w.tsize, order, first, count, group, gteam, nteams, gcount, moff, sfirst, sn,
                       gsplit, nsplits);
    Teams tm;
    tm.order = order;
    tm.first = first;
    tm.count = count;
    tm.group = group;
    tm.nteams = nteams;
    tm.sfirst = sfirst;
    tm.sn = sn;
    tm.gsplit = gsplit;
    tm.nsplits = nsplits;
    tm.gteam = gteam;
    tm.slots = w.split_slots;
    o.dd_part = in->has_warp ? (float*)(ws + w.dd) : nullptr;
    const int64_t bc = (in->B + kXcds - 1) / kXcds;
    const dim3 grid((unsigned)(kXcds * w.split_slots * bc)), block(kTeam * kWave);
    with_option_set(options_of(in), [&](auto oc) {
      constexpr int O = decltype(oc)::value;
      with_cotangent_set(cotangent_set(O, vec, gy, gx, truncated), [&](auto cc) {
        constexpr int CT = decltype(cc)::value;
        if constexpr (CT != kCtRuntime) {
          if constexpr (O != kOptRuntime)
            hipLaunchKernelGGL((selective_bwd_team_kernel<O, true, CT>), grid, block, 0, s, *in,
                               z, ent, ent_chunk, nc, gy, gx, (int)truncated, tm, o);
        } else if (vec) {
          hipLaunchKernelGGL((selective_bwd_team_kernel<O, true, CT>), grid, block, 0, s, *in, z,
                             ent, ent_chunk, nc, gy, gx, (int)truncated, tm, o);
        } else {
          hipLaunchKernelGGL((selective_bwd_team_kernel<O, false, CT>), grid, block, 0, s, *in, z,
                             ent, ent_chunk, nc, gy, gx, (int)truncated, tm, o);
        }
      });
    });
    launch_finish(o.dd_part, gsplit, dd, in->G, in->B * T, partial, dbias, dtheta, in->F, in->B,
                  s);
  } else {
    zero_words(partial, 4 * R, s);
    if (in->has_warp && dd) zero_words(dd, in->G * in->B * T, s);
    launch_finish(nullptr, nullptr, nullptr, 0, 0, partial, dbias, dtheta, in->F, in->B, s);
  }
  return launch_status();
}

extern "C" int rqf_selftest_wave_scan(const float* in, float* out_fwd, float* out_rev,
                                      rqf_stream_t stream) {
  if (!in || !out_fwd || !out_rev) return RQF_ERR_ARG;
  hipLaunchKernelGGL(wave_scan_selftest_kernel, dim3(1), dim3(kWave), 0, (hipStream_t)stream, in,
                     out_fwd, out_rev);
  return launch_status();
}
