// rqf_device.h -- device-side building blocks shared by the scan kernels.
//
// * c32: complex fp32 value held as two VGPRs (interleaved in memory).
// * Wave-level inclusive scans of first-order affine maps over the 64 lanes of
//   a CDNA wavefront.  Forward (prefix) scans use DPP row_shr + row_bcast;
//   reverse (suffix) scans use DPP row_shl inside a 16-lane row and two
//   ds_bpermute steps across rows.
// * Elementwise math for the fused ZOH discretisation: exp via v_exp_f32,
//   reciprocal via v_rcp_f32, and polynomial sin/cos/expm1 whose relative
//   accuracy near zero is what the a -> 0 limits of the recurrence need.
//
// All wave-level helpers must be called with all 64 lanes active.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rqf {

constexpr int kWave = 64;

struct c32 {
  float r, i;
};

__device__ __forceinline__ c32 mk(float r, float i) {
  c32 v;
  v.r = r;
  v.i = i;
  return v;
}
__device__ __forceinline__ c32 cadd(c32 a, c32 b) { return mk(a.r + b.r, a.i + b.i); }
__device__ __forceinline__ c32 csub(c32 a, c32 b) { return mk(a.r - b.r, a.i - b.i); }
__device__ __forceinline__ c32 cscale(float s, c32 a) { return mk(s * a.r, s * a.i); }
// a*b
__device__ __forceinline__ c32 cmul(c32 a, c32 b) {
  return mk(fmaf(a.r, b.r, -a.i * b.i), fmaf(a.r, b.i, a.i * b.r));
}
// a*b + c
__device__ __forceinline__ c32 cmad(c32 a, c32 b, c32 c) {
  return mk(fmaf(a.r, b.r, fmaf(-a.i, b.i, c.r)), fmaf(a.r, b.i, fmaf(a.i, b.r, c.i)));
}
// conj(a)*b
__device__ __forceinline__ c32 cjmul(c32 a, c32 b) {
  return mk(fmaf(a.r, b.r, a.i * b.i), fmaf(a.r, b.i, -a.i * b.r));
}
// conj(a)*b + c
__device__ __forceinline__ c32 cjmad(c32 a, c32 b, c32 c) {
  return mk(fmaf(a.r, b.r, fmaf(a.i, b.i, c.r)), fmaf(a.r, b.i, fmaf(-a.i, b.r, c.i)));
}
__device__ __forceinline__ c32 conjg(c32 a) { return mk(a.r, -a.i); }
// s*a + c for real s (two FMAs; a complex product with a zero imaginary part
// would keep its multiplications by zero under IEEE rules)
__device__ __forceinline__ c32 csmad(float s, c32 a, c32 c) {
  return mk(fmaf(s, a.r, c.r), fmaf(s, a.i, c.i));
}
// a*b + c for real c
__device__ __forceinline__ c32 cmadr(c32 a, c32 b, float c) {
  return mk(fmaf(a.r, b.r, fmaf(-a.i, b.i, c)), fmaf(a.r, b.i, a.i * b.r));
}
// a*s + c for real s and c (first step of a Horner scheme with real coefficients)
__device__ __forceinline__ c32 cmadrr(c32 a, float s, float c) { return mk(fmaf(a.r, s, c), a.i * s); }
// Re(conj(a) b)
__device__ __forceinline__ float cdot(c32 a, c32 b) { return fmaf(a.r, b.r, a.i * b.i); }

// ---------------------------------------------------------------------------
// Complex fp64, for the few per-channel quantities whose float32 rounding
// would compound: powers a^n of the transition coefficient and the carry
// chains that apply them.  Binary powering squares its running factor, which
// doubles that factor's relative error at each step, so a^n evaluated in
// float32 is off by ~n ulp -- one systematic error per channel that every
// carry hop then repeats.  With |a| near 1 (trained filters reach
// |a| = 0.9996, a memory of ~2800 steps) a hop chain covers many hops and the
// coefficient gradients, sums of products of long-memory states, pick the
// bias up coherently.  In fp64 the power is exact to float32 precision once
// rounded.
// ---------------------------------------------------------------------------
struct c64d {
  double r, i;
};
__device__ __forceinline__ c64d mkd(double r, double i) {
  c64d v;
  v.r = r;
  v.i = i;
  return v;
}
__device__ __forceinline__ c64d widen(c32 a) { return mkd(a.r, a.i); }
__device__ __forceinline__ c32 narrow(c64d a) { return mk((float)a.r, (float)a.i); }
__device__ __forceinline__ c64d dconj(c64d a) { return mkd(a.r, -a.i); }
__device__ __forceinline__ c64d dmul(c64d a, c64d b) {
  return mkd(fma(a.r, b.r, -a.i * b.i), fma(a.r, b.i, a.i * b.r));
}
// a*b + c
__device__ __forceinline__ c64d dmad(c64d a, c64d b, c64d c) {
  return mkd(fma(a.r, b.r, fma(-a.i, b.i, c.r)), fma(a.r, b.i, fma(a.i, b.r, c.i)));
}
// a^n, n >= 0, by binary powering in fp64.
__device__ __forceinline__ c64d dpow(c64d a, int64_t n) {
  c64d r = mkd(1.0, 0.0);
  while (n > 0) {
    if (n & 1) r = dmul(r, a);
    a = dmul(a, a);
    n >>= 1;
  }
  return r;
}

// Index of this wavefront within its block, as a wave-uniform (scalar) value:
// the compiler cannot prove threadIdx.x >> 6 uniform, and everything derived
// from a divergent value (row pointers, per-channel parameters) would occupy
// vector registers.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// MI355X deals the blocks of a launch round-robin over its 8 XCDs (block P
// runs on XCD P % 8), and each XCD has its own L2.  Map P to a logical block
// id so that every XCD runs one contiguous range of the n logical blocks:
// neighbouring logical blocks, which usually share cache lines, then share an
// L2.  A bijection on [0, n) for any n.
constexpr int kXcdCount = 8;
__device__ __forceinline__ int64_t xcd_contiguous(int64_t P, int64_t n) {
  const int64_t x = P % kXcdCount, j = P / kXcdCount, q = n / kXcdCount, r = n % kXcdCount;
  return x * q + (x < r ? x : r) + j;
}

// A dispatch packet holds the grid size in work-items as a 32-bit value per
// dimension: a launch of `blocks` x `threads` past 2^32 - 1 work-items would
// run a truncated grid, with no error from the launch.  Entry points check
// each of their grids with this before launching anything.
__host__ __device__ constexpr bool grid_fits(int64_t blocks, int64_t threads) {
  return blocks >= 0 && threads > 0 && blocks <= (int64_t)0xFFFFFFFF / threads;
}
// Blocks of a grid-stride launch over n items, one per block: at most
// kStrideBlocks, so that it always fits.
constexpr int64_t kStrideBlocks = (int64_t)1 << 20;
__host__ __device__ constexpr unsigned stride_blocks(int64_t n) {
  return (unsigned)(n < 1 ? 1 : (n < kStrideBlocks ? n : kStrideBlocks));
}

// ---------------------------------------------------------------------------
// Raw buffer access: CDNA buffer instructions through a resource descriptor
// (base, size in bytes).  A load at a byte offset at or past the size returns
// zero and a store there is dropped, by the hardware's range check.  A
// streamed (B,T,F) pass takes its bounds (steps past the end of the sequence,
// filters past F) from the descriptor instead of a compare, a branch and a
// 64-bit address per element.  Offsets are 32-bit, passed whole as the vector
// offset; the scalar offset operand is always 0.
// ---------------------------------------------------------------------------
using brsrc = __amdgpu_buffer_rsrc_t;
constexpr int kBufWord3 = 0x00020000;       // descriptor word 3 on gfx9 (32-bit data format)
constexpr uint32_t kBufOut = 0x80000000u;  // a lane offset past every resource made here
__device__ __forceinline__ brsrc buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufWord3);
}
__device__ __forceinline__ float buf_ldf(brsrc r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ void buf_stf(brsrc r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)off, 0, 0);
}
// The 64-bit forms move a complex value as one <2 x float>: with the two
// 32-bit halves taken out of the loaded vector one by one, this compiler
// narrowed the load to its first dword and returned (re, re).
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32v2 __attribute__((vector_size(8)));
__device__ __forceinline__ c32 buf_ldc(brsrc r, uint32_t off) {
  const f32x2 v = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
  return mk(v.x, v.y);
}
__device__ __forceinline__ void buf_stc(brsrc r, uint32_t off, c32 v) {
  f32x2 w;
  w.x = v.r;
  w.y = v.i;
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32v2, w), r, (int)off, 0, 0);
}

// ---------------------------------------------------------------------------
// Cross-lane primitives
// ---------------------------------------------------------------------------

// DPP move of `src` from the lane selected by CTRL; lanes whose source lane is
// out of range (or whose row is masked off) receive `fill`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float src, float fill) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(src),
                                                    CTRL, ROW_MASK, 0xf, false));
}

// DPP move with zero fill: a lane whose source lane is out of its row
// receives 0 (bound_ctrl); every row and bank is written, so no fill value
// has to be staged in the destination first.
template <int CTRL>
__device__ __forceinline__ float dpp0(float src) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(src), CTRL, 0xf, 0xf, true));
}

// GFX9 DPP controls.  wave_shl:1 / wave_shr:1 move a value one lane across
// the whole 64-lane wavefront (GFX9 only).
constexpr int kRowShl1 = 0x101, kRowShl2 = 0x102, kRowShl4 = 0x104, kRowShl8 = 0x108;
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kWaveShl1 = 0x130, kWaveShr1 = 0x138;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

__device__ __forceinline__ float bperm(float v, int src_lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}
__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ c32 readlane(c32 v, int lane) {
  return mk(readlane(v.r, lane), readlane(v.i, lane));
}
__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Value of `v` held by lane-1 (lane 0 receives `fill`): one DPP wave shift
// per float, the lane without a source keeping `fill`.  (`lane` is unused.)
__device__ __forceinline__ float shift_up(float v, float fill, int) {
  return dpp<kWaveShr1>(v, fill);
}
__device__ __forceinline__ c32 shift_up(c32 v, c32 fill, int lane) {
  return mk(shift_up(v.r, fill.r, lane), shift_up(v.i, fill.i, lane));
}
// Value of `v` held by lane+1 (lane 63 receives `fill`).
__device__ __forceinline__ float shift_down(float v, float fill, int) {
  return dpp<kWaveShl1>(v, fill);
}
__device__ __forceinline__ c32 shift_down(c32 v, c32 fill, int lane) {
  return mk(shift_down(v.r, fill.r, lane), shift_down(v.i, fill.i, lane));
}

// One Hillis-Steele step of the prefix scan of affine maps x -> P x + s.
// The map received from an earlier lane is applied first.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ void fwd_step(c32& P, c32& s) {
  // Identity (P, s) = (1, 0) for lanes without a source: the zero parts via
  // bound_ctrl where every row takes part, staged fills where rows are masked.
  constexpr bool all_rows = ROW_MASK == 0xf;
  const c32 lp = mk(dpp<CTRL, ROW_MASK>(P.r, 1.0f),
                    all_rows ? dpp0<CTRL>(P.i) : dpp<CTRL, ROW_MASK>(P.i, 0.0f));
  const c32 ls = mk(all_rows ? dpp0<CTRL>(s.r) : dpp<CTRL, ROW_MASK>(s.r, 0.0f),
                    all_rows ? dpp0<CTRL>(s.i) : dpp<CTRL, ROW_MASK>(s.i, 0.0f));
  s = cmad(ls, P, s);
  P = cmul(lp, P);
}

// Inclusive prefix scan over lanes: lane i ends with the composition of the
// maps of lanes 0..i (lane 0's applied first).
__device__ __forceinline__ void wave_scan_fwd(c32& P, c32& s) {
  fwd_step<kRowShr1>(P, s);
  fwd_step<kRowShr2>(P, s);
  fwd_step<kRowShr4>(P, s);
  fwd_step<kRowShr8>(P, s);
  fwd_step<kRowBcast15, 0xa>(P, s);
  fwd_step<kRowBcast31, 0xc>(P, s);
}

// One step of the suffix scan of maps d -> Q d + r, where the map received
// from a later lane is applied first (it is closer to the end of time).
template <int CTRL>
__device__ __forceinline__ void rev_step(c32& Q, c32& r) {
  const c32 lq = mk(dpp<CTRL>(Q.r, 1.0f), dpp0<CTRL>(Q.i));
  const c32 lr = mk(dpp0<CTRL>(r.r), dpp0<CTRL>(r.i));
  r = cmad(Q, lr, r);
  Q = cmul(Q, lq);
}
__device__ __forceinline__ void rev_cross(c32& Q, c32& r, int src, bool valid) {
  c32 lq = mk(bperm(Q.r, src), bperm(Q.i, src));
  c32 lr = mk(bperm(r.r, src), bperm(r.i, src));
  if (!valid) {
    lq = mk(1.0f, 0.0f);
    lr = mk(0.0f, 0.0f);
  }
  r = cmad(Q, lr, r);
  Q = cmul(Q, lq);
}

// Inclusive suffix scan over lanes: lane i ends with the composition of the
// maps of lanes i..63 (lane 63's applied first).
__device__ __forceinline__ void wave_scan_rev(c32& Q, c32& r, int lane) {
  rev_step<kRowShl1>(Q, r);
  rev_step<kRowShl2>(Q, r);
  rev_step<kRowShl4>(Q, r);
  rev_step<kRowShl8>(Q, r);
  // Each lane now covers the rest of its 16-lane row; add whole rows after it.
  const int row = lane >> 4;
  rev_cross(Q, r, ((row + 1) & 3) << 4, row < 3);
  rev_cross(Q, r, ((row + 2) & 3) << 4, row < 2);
}

// ---------------------------------------------------------------------------
// Scans of a time-invariant recurrence.  Every lane applies the same map power
// A = a^K (K steps per lane; steps past the end of the row run with zero input,
// which changes nothing any valid step reads), so the map covering lanes i..j
// is A^(j-i+1) and the scans only propagate the offsets: at each step a lane
// adds its partner's offset times A^(lanes it already covers).  Those powers
// come from ScanPow, each rounded once from fp64, instead of the products of
// products the general scans form (a squaring doubles its factor's relative
// error, so A^64 composed in float32 is off by ~64 ulp of A -- a per-channel
// bias that every tile hop repeats).  Two DPP moves and one complex product per
// step fewer than the general scans.
// ---------------------------------------------------------------------------
struct ScanPow {
  c32 p[4];      // A^(2^j), j = 0..3: the in-row steps (wave-uniform)
  c32 row, row2; // per lane: the powers of the two cross-row steps
};
// Cross-row powers of the adjoint's suffix scan, whose map power is conj(A);
// its in-row powers are the conjugates of ScanPow::p.
struct RevPow {
  c32 row, row2;
};
// A wave-uniform value, marked as such.  (The compiler drops the readfirstlane
// when it already knows the value uniform and keeps the value in a VGPR; an
// inline-asm v_readfirstlane_b32 into an SGPR was measured to give wrong
// results here, so the builtin is kept.)
__device__ __forceinline__ float uniform(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ c32 uniform(c32 v) { return mk(uniform(v.r), uniform(v.i)); }
// A wave-uniform 64-bit value pinned to scalar registers.  Pass byte offsets
// through it, not pointers: a pointer rebuilt from integers loses its
// address space, and its stores become flat ones.
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32)) << 32) |
         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
}

// Powers for wave_scan_fwd_pow: lane i covers lanes 16*(i/16)..i before the
// first cross-row step and 32*(i/32)..i before the second.
__device__ __forceinline__ ScanPow scan_pow_fwd(c64d A, int lane) {
  ScanPow s;
  c64d q = A;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s.p[j] = uniform(narrow(q));
    q = dmul(q, q);
  }
  s.row = narrow(dpow(A, (lane & 15) + 1));
  s.row2 = narrow(dpow(A, (lane & 31) + 1));
  return s;
}
// Cross-row powers for wave_scan_rev_pow (A as for scan_pow_fwd): lane i covers
// lanes i..16*(i/16)+15 before the first cross-row step and i..16*(i/16)+31
// before the second.
__device__ __forceinline__ RevPow scan_pow_rev(c64d A, int lane) {
  const c64d Ac = dconj(A);
  RevPow s;
  s.row = narrow(dpow(Ac, 16 - (lane & 15)));
  s.row2 = narrow(dpow(Ac, 32 - (lane & 15)));
  return s;
}

// In-row step: the power is wave-uniform, so the partner multiplies its own
// offset by it and the DPP move folds into the add.  CONJ: the power is conj(p).
template <int CTRL, bool CONJ = false>
__device__ __forceinline__ void step_upow(c32& s, c32 p) {
  const c32 t = CONJ ? cjmul(p, s) : cmul(s, p);
  s = mk(s.r + dpp0<CTRL>(t.r), s.i + dpp0<CTRL>(t.i));
}
// Cross-row step: the power depends on the receiving lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void fwd_step_lpow(c32& s, c32 p) {
  const c32 ls = mk(dpp<CTRL, ROW_MASK>(s.r, 0.0f), dpp<CTRL, ROW_MASK>(s.i, 0.0f));
  s = cmad(ls, p, s);
}
// Inclusive prefix scan of the offsets: lane i ends with the offset of the
// composition of lanes 0..i (its power is A^(i+1)).
__device__ __forceinline__ void wave_scan_fwd_pow(c32& s, const ScanPow& pw) {
  step_upow<kRowShr1>(s, pw.p[0]);
  step_upow<kRowShr2>(s, pw.p[1]);
  step_upow<kRowShr4>(s, pw.p[2]);
  step_upow<kRowShr8>(s, pw.p[3]);
  fwd_step_lpow<kRowBcast15, 0xa>(s, pw.row);
  fwd_step_lpow<kRowBcast31, 0xc>(s, pw.row2);
}

// Inclusive suffix scan of the offsets of maps with power conj(A): lane i ends
// with the offset of the composition of lanes i..63 (its power is conj(A)^(64-i)).
__device__ __forceinline__ void wave_scan_rev_pow(c32& r, const ScanPow& pw, const RevPow& rv,
                                                  int lane) {
  step_upow<kRowShl1, true>(r, pw.p[0]);
  step_upow<kRowShl2, true>(r, pw.p[1]);
  step_upow<kRowShl4, true>(r, pw.p[2]);
  step_upow<kRowShl8, true>(r, pw.p[3]);
  const int row = lane >> 4;
  c32 lr = mk(bperm(r.r, ((row + 1) & 3) << 4), bperm(r.i, ((row + 1) & 3) << 4));
  if (row >= 3) lr = mk(0.0f, 0.0f);
  r = cmad(rv.row, lr, r);
  lr = mk(bperm(r.r, ((row + 2) & 3) << 4), bperm(r.i, ((row + 2) & 3) << 4));
  if (row >= 2) lr = mk(0.0f, 0.0f);
  r = cmad(rv.row2, lr, r);
}

// Complex tile I/O through a wavefront-private LDS slice (full tiles, VEC).
// Each global load/store instruction moves one contiguous 1 KB (lane l moves
// float4 j*64 + l); the lanes then exchange through LDS so that each holds its
// K consecutive steps.  A direct lane-contiguous access would make every
// instruction touch 2 KB at half density, which streams measurably slower.
// The slot swizzle spreads both LDS access patterns over the banks: a
// b128 access is served 8 lanes (128 B) at a time, and XOR-ing bits 3.. of
// the float4 index into its low log2(Q) bits gives those 8 lanes distinct
// 16-byte bank groups when they read Q consecutive float4s each (measured:
// K = 8 forward, 5.7e7 conflict cycles unswizzled in the low bits, 8.1e6 with).
template <int Q>
__device__ __forceinline__ int io_slot(int q) { return q ^ ((q >> 3) & (Q - 1)); }

template <int K>
__device__ __forceinline__ void load_c_lds(const float* __restrict__ row, int t0, int lane,
                                           float4* lds, c32 (&v)[K]) {
  constexpr int Q = K / 2;  // float4s per lane
#pragma unroll
  for (int j = 0; j < Q; ++j) lds[io_slot<Q>(j * kWave + lane)] = *reinterpret_cast<const float4*>(row + 2 * t0 + 4 * (j * kWave + lane));
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    const float4 a = lds[io_slot<Q>(lane * Q + j)];
    v[2 * j] = mk(a.x, a.y);
    v[2 * j + 1] = mk(a.z, a.w);
  }
  __builtin_amdgcn_wave_barrier();
}

template <int K>
__device__ __forceinline__ void store_c_lds(float* __restrict__ row, int t0, int lane, float4* lds,
                                            const c32 (&v)[K]) {
  constexpr int Q = K / 2;
#pragma unroll
  for (int j = 0; j < Q; ++j)
    lds[io_slot<Q>(lane * Q + j)] = make_float4(v[2 * j].r, v[2 * j].i, v[2 * j + 1].r, v[2 * j + 1].i);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < Q; ++j) *reinterpret_cast<float4*>(row + 2 * t0 + 4 * (j * kWave + lane)) = lds[io_slot<Q>(j * kWave + lane)];
  __builtin_amdgcn_wave_barrier();
}

// Walks a task's steps t = tb..te-1 (FWD) or te-1..tb in chunks of CH:
// load(j, t) fills chunk slot j for step t, step(j, t) consumes it.  All the
// loads of a chunk issue before any of its steps computes.  Left to itself the
// scheduler sinks each load next to its use (load, wait, compute, next load),
// which keeps one load in flight per wave and runs the pass at memory latency
// rather than bandwidth.  The last, partial chunk loads every slot too (slots
// past the segment re-read its last step, so every address stays inside it)
// and computes only its valid steps: stepping the tail one load at a time
// would cost a full memory latency per step.
template <int CH, bool FWD, class Load, class Step>
__device__ __forceinline__ void stream_steps(int64_t tb, int64_t te, Load&& load, Step&& step) {
  int64_t t = FWD ? tb : te - 1;
  const int64_t full = (te - tb) / CH;
  for (int64_t c = 0; c < full; ++c) {
#pragma unroll
    for (int j = 0; j < CH; ++j) load(j, FWD ? t + j : t - j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < CH; ++j) step(j, FWD ? t + j : t - j);
    t += FWD ? CH : -CH;
  }
  const int rem = (int)(te - tb - full * CH);
  if (rem == 0) return;
#pragma unroll
  for (int j = 0; j < CH; ++j) load(j, FWD ? min(t + j, te - 1) : max(t - j, tb));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < CH; ++j)
    if (j < rem) step(j, FWD ? t + j : t - j);
}

// ---------------------------------------------------------------------------
// Segment scans of the single-pass (batch, time, filters) kernels.  A block
// pass splits time into consecutive segments of LS steps; a wavefront holds
// G = 64 / FC of them, FC lanes (filters) each, lane l in segment l / FC.
// Each lane knows its segment's result from a zero entry; these helpers
// combine the results of the wavefront's segments in fp64 (Hillis-Steele over
// the G segments, by cross-lane moves of FC lanes), for time-invariant maps
// whose multiplier over one segment, m = a^LS (or conj(a)^LS), is the same
// for every segment of a lane's filter.
// ---------------------------------------------------------------------------
__device__ __forceinline__ c64d shfl_up_d(c64d v, int d) {
  return mkd(__shfl_up(v.r, d), __shfl_up(v.i, d));
}
__device__ __forceinline__ c64d shfl_down_d(c64d v, int d) {
  return mkd(__shfl_down(v.r, d), __shfl_down(v.i, d));
}

// Forward maps y -> m y + s.  Returns the exclusive prefix over the
// wavefront's segments before this lane's, E_q = sum_{j<q} m^(q-1-j) s_j
// (zero for q = 0), and sets `incl` to the inclusive one.
template <int FC>
__device__ __forceinline__ c64d wave_seg_prefix(c64d s, c64d m, int lane, c64d& incl) {
  constexpr int G = kWave / FC;
  incl = s;
  c64d pw = m;  // m^k
#pragma unroll
  for (int k = 1; k < G; k <<= 1) {
    const c64d prev = shfl_up_d(incl, k * FC);
    if (lane >= k * FC) incl = dmad(pw, prev, incl);
    pw = dmul(pw, pw);
  }
  const c64d ex = shfl_up_d(incl, FC);
  return lane >= FC ? ex : mkd(0.0, 0.0);
}

// Adjoint pair maps over a span of n segments (nL = n*LS steps), applied to the
// pair (g, h) entering at the span's end:
//   (g, h) -> (P_n g + G, P_n h + c_n g + H),
//   P_n = conj(a)^nL,  c_n = nL conj(a)^(nL-1),
// with (G, H) the span's own pair from a zero entry.  Composing the span of a
// segment with the span of n segments after it: G' = P_n G_after ... see
// wave_seg_suffix.
struct PairMap {
  c64d P, c;  // P_n, c_n
};
__device__ __forceinline__ PairMap pair_map_mul(PairMap x, PairMap y) {
  // span of x followed (in reverse time: preceded) by span of y
  PairMap r;
  r.P = dmul(x.P, y.P);
  r.c = dmad(x.P, y.c, dmul(x.c, y.P));
  return r;
}
// (g, h) entering at the end of a span with map `mp` and own pair (G, H):
// the pair at the span's start.
__device__ __forceinline__ void pair_apply(const PairMap& mp, c64d G, c64d H, c64d& g, c64d& h) {
  const c64d ng = dmad(mp.P, g, G);
  h = dmad(mp.P, h, dmad(mp.c, g, H));
  g = ng;
}

// Suffix over the wavefront's segments of the adjoint pair maps: returns in
// (eg, eh) the pair that the segments after this lane's produce from a zero
// pair at the wavefront's end, and in (ig, ih) the same including this lane's
// segment.  `one` is the map of one segment.  `span_after` returns the map of
// the segments after this lane's (q + 1 .. G - 1).
template <int FC>
__device__ __forceinline__ void wave_seg_suffix(c64d G0, c64d H0, PairMap one, int lane, c64d& eg,
                                                c64d& eh, c64d& ig, c64d& ih, PairMap& span_after) {
  constexpr int G = kWave / FC;
  const int q = lane / FC;
  ig = G0;
  ih = H0;
  PairMap pw = one;  // map of k segments
#pragma unroll
  for (int k = 1; k < G; k <<= 1) {
    // the composed pair of segments q+k .. (from lanes k*FC above)
    const c64d ng = shfl_down_d(ig, k * FC), nh = shfl_down_d(ih, k * FC);
    if (q + k < G) {
      // this lane's span (k segments) applied after the span that follows it
      c64d g = ng, h = nh;
      pair_apply(pw, ig, ih, g, h);
      ig = g;
      ih = h;
    }
    pw = pair_map_mul(pw, pw);
  }
  eg = shfl_down_d(ig, FC);
  eh = shfl_down_d(ih, FC);
  if (q + 1 >= G) eg = eh = mkd(0.0, 0.0);
  // map of G - 1 - q segments, by binary powering of `one`
  PairMap acc;
  acc.P = mkd(1.0, 0.0);
  acc.c = mkd(0.0, 0.0);
  PairMap base = one;
  for (int n = G - 1 - q; n > 0; n >>= 1) {
    if (n & 1) acc = pair_map_mul(acc, base);
    base = pair_map_mul(base, base);
  }
  span_after = acc;
}

// Sum of a double over the wave (result valid in every lane).
__device__ __forceinline__ double wave_sum(double v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// ---------------------------------------------------------------------------
// Elementwise math
// ---------------------------------------------------------------------------

__device__ __forceinline__ float fexp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fsigmoid(float x) { return frcp(1.0f + fexp(-x)); }
// tanh(x) = 1 - 2/(e^{2x} + 1); saturates to +-1 without overflow trouble.
__device__ __forceinline__ float ftanh(float x) {
  return fmaf(-2.0f, frcp(fexp(2.0f * x) + 1.0f), 1.0f);
}

// expm1(x) given e = exp(x): for |x| < 0.5 the degree-7 polynomial
// x + x^2 * r(x), r fitted (weighted least squares, Lawson iteration) to
// (expm1(x) - x)/x^2 on [-0.5, 0.5]: max relative error 3.1e-9 in fp64;
// otherwise e - 1 (no cancellation for |x| >= 0.5).
__device__ __forceinline__ float fexpm1(float x, float e) {
  if (fabsf(x) < 0.5f) {
    float r = fmaf(x, 1.9990473167705037e-04f, 1.3997542041360440e-03f);
    r = fmaf(x, r, 8.3330821525987070e-03f);
    r = fmaf(x, r, 4.1665312400424060e-02f);
    r = fmaf(x, r, 1.6666667932516960e-01f);
    r = fmaf(x, r, 5.0000004193574390e-01f);
    return fmaf(x * x, r, x);
  }
  return e - 1.0f;
}

// For an angle x: sin(x), and vers(x) = 1 - cos(x) = 2 sin^2(x/2).  The
// argument is reduced to r = x - 2*pi*q, |r| <= pi (Cody-Waite, two-part
// 2*pi); h = r/2 in [-pi/2, pi/2] goes through fitted polynomials
//   sin(h) = h * P(h^2)       degree 9, max relative error 4.3e-9
//   cos(h) = 1 + h^2 Q(h^2)   degree 10, max absolute error 2.4e-10
// (weighted least squares, Lawson iteration, on [0, (pi/2)^2]); then
//   sin x = 2 sin(h) cos(h),  1 - cos x = 2 sin^2(h).
__device__ __forceinline__ void fsin_vers(float x, float& s, float& vers) {
  const float q = rintf(x * 0.15915494309189535f);
  float r = fmaf(-q, 6.28318548202514648f, x);  // 2*pi rounded to fp32
  r = fmaf(-q, -1.7484556000744487e-07f, r);    // 2*pi - fp32(2*pi)
  const float h = 0.5f * r;
  const float u = h * h;
  float sp = fmaf(u, 2.6052247914144940e-06f, -1.9809075229821477e-04f);
  sp = fmaf(u, sp, 8.3330510624972130e-03f);
  sp = fmaf(u, sp, -1.6666657991867140e-01f);
  sp = fmaf(u, sp, 9.9999999573276810e-01f);
  const float sh = h * sp;
  float cp = fmaf(u, -2.6077094002825570e-07f, 2.4761885527010584e-05f);
  cp = fmaf(u, cp, -1.3888403492119570e-03f);
  cp = fmaf(u, cp, 4.1666640726599230e-02f);
  cp = fmaf(u, cp, -4.9999999549513570e-01f);
  const float ch = fmaf(u, cp, 1.0f);
  s = 2.0f * sh * ch;
  vers = 2.0f * sh * sh;
}

// Zero-order-hold pieces for a = ar + i ai:
//   A   = exp(a)
//   phi = (exp(a) - 1)/a, with the cubic series 1 + a/2 + a^2/6 + a^3/24 when
//         |a|^2 < 1e-8 (the reference's threshold, selective_scan.py:49-54)
// inv_den returns 1/|a|^2 (0 on the series branch) for reuse by the VJP.
__device__ __forceinline__ void zoh(float ar, float ai, c32& A, c32& phi, float& inv_den) {
  const float e = fexp(ar);
  float sn, vers;
  fsin_vers(ai, sn, vers);
  A = mk(e * (1.0f - vers), e * sn);
  const float den = fmaf(ar, ar, ai * ai);
  if (den < 1.0e-8f) {
    // 1 + a*(1/2 + a*(1/6 + a/24))
    c32 a = mk(ar, ai);
    c32 t = cmadrr(a, 1.0f / 24.0f, 1.0f / 6.0f);
    t = cmadr(a, t, 0.5f);
    phi = cmadr(a, t, 1.0f);
    inv_den = 0.0f;
  } else {
    // Re(e^a - 1) = expm1(ar) cos(ai) - (1 - cos ai) = expm1(ar)*(1 - vers) - vers:
    // both terms stay small near a = 0, so there is no cancellation.
    const float em1 = fexpm1(ar, e);
    const float er = fmaf(em1, 1.0f - vers, -vers);
    const float ei = e * sn;
    inv_den = frcp(den);
    phi = mk(fmaf(er, ar, ei * ai) * inv_den, fmaf(ei, ar, -er * ai) * inv_den);
  }
}

}  // namespace rqf
