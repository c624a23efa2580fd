// proj.hip -- the selective layer's projection GEMMs on MFMA (fp32).
//
// C (M x N) = A (M x K) . B (K x N), in fp32 with fp32 accumulation
// (v_mfma_f32_32x32x2_f32), where
//   * A is a small weight matrix packed on the host as (k_pad, m_pad), k-major
//     with m contiguous, zero padded to the tile sizes;
//   * B is gathered from a complex (rows, N) array -- complex row d gives K rows
//     2d (real part) and 2d+1 (imaginary part) -- followed by a real (rows, N)
//     array, so the interleaved complex input needs no [Re; Im] copy;
//   * C is scattered to a complex (rows, N) array -- rows 2f and 2f+1 are the
//     real and imaginary parts of complex row f -- followed by a real (rows, N)
//     array.
// With the drive and selector weights stacked in A, one pass over the layer
// input gives both z = W x and the logits Ws [Re x; Im x]
// (rqf_models/ops/selective_scan.py:117-118, rqf_models/backbones/rqf/
// selective.py:205-217); with their adjoints stacked, one pass over dz and the
// logit gradients gives dx (selective_scan.py:144, selective.py:96).
//
// Tiles: a 256-thread block computes a 128 x 128 tile of C in four 64 x 64
// wavefront tiles of 2 x 2 MFMA 32 x 32 blocks, walking K in stages of 16
// through double-buffered LDS (one barrier per stage).  Blocks are numbered so
// that the M tiles of one N tile run on one XCD and share its L2 copy of B.
//
// Measured at H = 256, B*T = 1.02M: 98 TFLOP/s forward, 96 for dx, 62% of the
// fp32 MFMA peak.  The library GEMMs it replaces run at 105-135 TFLOP/s, so
// despite saving the [Re; Im] copy and the add passes it is 5-8% slower than
// them.  Variants measured and dropped (forward, TFLOP/s):
// - wavefront tiles 2x4, 4x2, 4x4 (occupancy 1): 68-78;
// - all of a stage's fragments read before its MFMAs (occupancy 2): 82;
// - loads two stages ahead: 90;
// - tiles row-major with a stage's K values contiguous, so one ds_read_b128
//   brings four k-steps (two LDS waits per stage): 91.
#include "rqf_device.h"
#include "rqf_scan.h"

using namespace rqf;

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

// Wavefront tile: RQF_PROJ_TM x RQF_PROJ_TN blocks of 32 x 32; the block is
// 2 x 2 wavefronts.
#ifndef RQF_PROJ_TM
#define RQF_PROJ_TM 2
#endif
#ifndef RQF_PROJ_TN
#define RQF_PROJ_TN 2
#endif
constexpr int kTM = RQF_PROJ_TM, kTN = RQF_PROJ_TN;
// Occupancy (waves per SIMD) the register allocator is held to; 0 = no hint
// (which leaves this kernel at 2 waves: 64 accumulator AGPRs + 112 VGPRs; held
// to 3 it keeps the accumulators in VGPRs, 125 in all).
#ifndef RQF_PROJ_WAVES
#define RQF_PROJ_WAVES 3
#endif
constexpr int kPM = 64 * kTM, kPN = 64 * kTN, kPK = 16, kPThreads = 256;
// The host pads the weights' M to a multiple of 128 whatever the tile.
constexpr int kPMPad = 128;
static_assert(kPM % kPMPad == 0 || kPMPad % kPM == 0, "M tiles cover the padded weights");

// Blocks are dealt round-robin over the XCDs; give each XCD a contiguous range
// of tile ids.
__device__ __forceinline__ int64_t proj_xcd_order(int64_t P, int64_t n) { return xcd_contiguous(P, n); }

// Real B row j (0-based after the complex rows), or null past the last row.
__device__ __forceinline__ const float* real_row(const rqf_proj_gemm_args& g, int64_t j) {
  return j < g.b_real_rows ? g.b_real + j * g.n : nullptr;
}

// Two consecutive columns n, n+1 of B rows k (x, y) and k+1 (z, w); zero past
// the ends.  VEC: N is even, so n < N implies n + 1 < N and the complex pair
// is one aligned float4.
template <bool VEC>
__device__ __forceinline__ float4 load_b_pair(const rqf_proj_gemm_args& g, int64_t k, int64_t n) {
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (n >= g.n) return v;
  const int64_t kc = 2 * g.b_cplx_rows;
  if (k < kc) {
    const float* p = g.b_cplx + 2 * ((k >> 1) * g.n + n);
    if (VEC) {
      const float4 q = *reinterpret_cast<const float4*>(p);  // re n, im n, re n+1, im n+1
      v = make_float4(q.x, q.z, q.y, q.w);
    } else {
      v.x = p[0];
      v.z = p[1];
      if (n + 1 < g.n) {
        v.y = p[2];
        v.w = p[3];
      }
    }
    return v;
  }
  const float* r0 = real_row(g, k - kc);
  const float* r1 = real_row(g, k + 1 - kc);
  if (VEC) {
    if (r0) {
      const float2 q = *reinterpret_cast<const float2*>(r0 + n);
      v.x = q.x;
      v.y = q.y;
    }
    if (r1) {
      const float2 q = *reinterpret_cast<const float2*>(r1 + n);
      v.z = q.x;
      v.w = q.y;
    }
  } else {
    const bool n1 = n + 1 < g.n;
    if (r0) {
      v.x = r0[n];
      if (n1) v.y = r0[n + 1];
    }
    if (r1) {
      v.z = r1[n];
      if (n1) v.w = r1[n + 1];
    }
  }
  return v;
}

// FAST: N even (and at least 2), 16-byte aligned complex rows, 8-byte aligned
// real rows, and 2 * b_cplx_rows a multiple of the K stage.
template <bool VEC, bool FAST>
__global__ __launch_bounds__(kPThreads)
#if RQF_PROJ_WAVES
__attribute__((amdgpu_waves_per_eu(RQF_PROJ_WAVES)))
#endif
void proj_gemm_kernel(const rqf_proj_gemm_args g,
                                                              int64_t m_tiles, int64_t tiles) {
  __shared__ float s_a[2][kPK][kPM];
  __shared__ float s_b[2][kPK][kPN];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid >> 6;
  const int64_t id = proj_xcd_order(blockIdx.x, tiles);
  const int64_t m0 = (id % m_tiles) * kPM, n0 = (id / m_tiles) * kPN;
  const int wm = (w & 1) * (kPM / 2), wn = (w >> 1) * (kPN / 2);
  // Staging: an A stage is 16 rows of kPM/4 float4s; a B stage is 8 row pairs of
  // kPN/2 column pairs.
  constexpr int kA4 = kPM / 4, kB2 = kPN / 2;
  constexpr int kRa = kPK * kA4 / kPThreads, kRb = (kPK / 2) * kB2 / kPThreads;
  struct Slot {
    float4 a[kRa], b[kRb];
  };
  // Per-thread B offsets of the fast path (column clamped to N - 2).
  int64_t b_off[kRb], b_col[kRb];
  int b_pair[kRb];
#pragma unroll
  for (int r = 0; r < kRb; ++r) {
    const int idx = tid + r * kPThreads;
    const int64_t n = n0 + 2 * (idx % kB2);
    b_pair[r] = idx / kB2;
    b_col[r] = n < g.n - 2 ? n : g.n - 2;
    b_off[r] = b_pair[r] * g.n + b_col[r];
  }
  // Rows of the padded weights past m_pad: the last M tile of a 256-row tile
  // over 128-padded weights reads nothing there.
  auto fetch = [&](int64_t kt, Slot& sl) {
    float4 (&ra)[kRa] = sl.a;
    float4 (&rb)[kRb] = sl.b;
#pragma unroll
    for (int r = 0; r < kRa; ++r) {
      const int idx = tid + r * kPThreads;
      const int64_t krow = kt * kPK + idx / kA4, mcol = m0 + 4 * (idx % kA4);
      if (kPM <= kPMPad || mcol < g.m_pad)
        ra[r] = *reinterpret_cast<const float4*>(g.weights + krow * g.m_pad + mcol);
      else
        ra[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const int64_t k0 = kt * kPK, kc = 2 * g.b_cplx_rows;
    if (FAST) {
      // Every stage is all complex or all real rows (2 * b_cplx_rows is a multiple
      // of the stage).  Rows past the end and columns past N are clamped to the
      // last ones: the padded weights are zero there, and columns past N are
      // never stored, so the values read only need to be finite.
      if (k0 < kc) {
#pragma unroll
        for (int r = 0; r < kRb; ++r) {
          const float4 q = *reinterpret_cast<const float4*>(
              g.b_cplx + 2 * ((k0 >> 1) * g.n + b_off[r]));
          rb[r] = make_float4(q.x, q.z, q.y, q.w);
        }
      } else if (g.b_real_rows > 0) {
#pragma unroll
        for (int r = 0; r < kRb; ++r) {
          const int64_t j = k0 - kc + 2 * b_pair[r];
          const int64_t last = g.b_real_rows - 1;
          const float* base = g.b_real + b_col[r];
          const float2 a = *reinterpret_cast<const float2*>(base + (j < last ? j : last) * g.n);
          const float2 b =
              *reinterpret_cast<const float2*>(base + (j + 1 < last ? j + 1 : last) * g.n);
          rb[r] = make_float4(a.x, a.y, b.x, b.y);
        }
      } else {
#pragma unroll
        for (int r = 0; r < kRb; ++r) rb[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    } else {
#pragma unroll
      for (int r = 0; r < kRb; ++r) {
        const int idx = tid + r * kPThreads;
        rb[r] = load_b_pair<VEC>(g, k0 + 2 * (idx / kB2), n0 + 2 * (idx % kB2));
      }
    }
  };
  auto stage = [&](int buf, const Slot& sl) {
    const float4 (&ra)[kRa] = sl.a;
    const float4 (&rb)[kRb] = sl.b;
#pragma unroll
    for (int r = 0; r < kRa; ++r) {
      const int idx = tid + r * kPThreads;
      *reinterpret_cast<float4*>(&s_a[buf][idx / kA4][4 * (idx % kA4)]) = ra[r];
    }
#pragma unroll
    for (int r = 0; r < kRb; ++r) {
      const int idx = tid + r * kPThreads;
      const int p = idx / kB2, q = idx % kB2;
      *reinterpret_cast<float2*>(&s_b[buf][2 * p][2 * q]) = make_float2(rb[r].x, rb[r].y);
      *reinterpret_cast<float2*>(&s_b[buf][2 * p + 1][2 * q]) = make_float2(rb[r].z, rb[r].w);
    }
  };
  v16f acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  // A wavefront whose rows all lie past the output rows computes nothing (the
  // stacked forward has 2F + 2F + G rows, 1032 at H = 256, padded to 1152); it
  // still loads and waits at the barriers with its block.
  const int64_t mtot = 2 * g.out_cplx_rows + g.out_real_rows;
  const bool live = m0 + wm < mtot;

  const int64_t ktiles = g.k_pad / kPK;
  // While stage kt is computed from one LDS buffer, the next stage's global
  // loads are in flight into registers and go to the other buffer after it.
  Slot sl;
  fetch(0, sl);
  stage(0, sl);
  __syncthreads();
  const int kr = lane >> 5, col = lane & 31;
  // The operand fragments of k-step kk + 1 are read from LDS while the MFMAs of
  // step kk run (two fragment slots).
  auto frags = [&](int buf, int kk, float (&af)[kTM], float (&bf)[kTN]) {
#pragma unroll
    for (int i = 0; i < kTM; ++i) af[i] = s_a[buf][2 * kk + kr][wm + 32 * i + col];
#pragma unroll
    for (int j = 0; j < kTN; ++j) bf[j] = s_b[buf][2 * kk + kr][wn + 32 * j + col];
  };
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int buf = (int)(kt & 1);
    if (kt + 1 < ktiles) fetch(kt + 1, sl);
    if (live) {
      float af[2][kTM], bf[2][kTN];
      frags(buf, 0, af[0], bf[0]);
#pragma unroll
      for (int kk = 0; kk < kPK / 2; ++kk) {
        if (kk + 1 < kPK / 2) frags(buf, kk + 1, af[(kk + 1) & 1], bf[(kk + 1) & 1]);
#pragma unroll
        for (int i = 0; i < kTM; ++i)
#pragma unroll
          for (int j = 0; j < kTN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[kk & 1][i], bf[kk & 1][j],
                                                             acc[i][j], 0, 0, 0);
      }
    }
    if (kt + 1 < ktiles) stage(buf ^ 1, sl);
    __syncthreads();
  }

  // Lane l holds C[8*(v/4) + 4*(l/32) + v%4][l%32] of each 32 x 32 block.
  const int64_t mc = 2 * g.out_cplx_rows;
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int64_t n = n0 + wn + 32 * j + col;
      if (n >= g.n) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm + 32 * i + 8 * (v >> 2) + 4 * kr + (v & 3);
        if (m < mc) {
          if ((v & 1) == 0)  // rows m (even) and m + 1: one complex value
            *reinterpret_cast<float2*>(g.out_cplx + 2 * ((m >> 1) * g.n + n)) =
                make_float2(acc[i][j][v], acc[i][j][v + 1]);
        } else if (m < mtot) {
          float o = acc[i][j][v];
          if (g.out_real_bias) o += g.out_real_bias[m - mc];
          if (g.out_real_relu) o = fmaxf(o, 0.0f);
          g.out_real[(m - mc) * g.n + n] = o;
        }
      }
    }
}

inline bool aligned(const void* p, uintptr_t a) { return p == nullptr || ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

extern "C" int rqf_proj_gemm(const rqf_proj_gemm_args* args, rqf_stream_t stream) {
  if (!args) return RQF_ERR_ARG;
  const rqf_proj_gemm_args& g = *args;
  if (g.n < 0 || g.k_pad < 0 || g.m_pad < 0 || g.b_cplx_rows < 0 || g.out_cplx_rows < 0 ||
      g.out_real_rows < 0)
    return RQF_ERR_ARG;
  if (g.b_real_rows < 0 || (g.b_real_rows > 0 && !g.b_real)) return RQF_ERR_ARG;
  const int64_t k = 2 * g.b_cplx_rows + g.b_real_rows, m = 2 * g.out_cplx_rows + g.out_real_rows;
  if (g.k_pad % kPK || g.m_pad % kPMPad || k > g.k_pad || m > g.m_pad) return RQF_ERR_ARG;
  if (g.n == 0 || m == 0) return RQF_OK;
  if (!g.weights || (g.b_cplx_rows && !g.b_cplx) || (g.out_cplx_rows && !g.out_cplx) ||
      (g.out_real_rows && !g.out_real))
    return RQF_ERR_ARG;
  if (!aligned(g.weights, 16) || !aligned(g.b_cplx, 8) || !aligned(g.out_cplx, 8) ||
      !aligned(g.out_real, 4))
    return RQF_ERR_ALIGN;
  const bool vec = g.n % 2 == 0 && aligned(g.b_cplx, 16) && aligned(g.b_real, 8);
  const int64_t m_tiles = (g.m_pad + kPM - 1) / kPM, n_tiles = (g.n + kPN - 1) / kPN;
  const int64_t tiles = m_tiles * n_tiles;
  if (!grid_fits(tiles, kPThreads)) return RQF_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const bool fast = vec && g.n >= 2 && (2 * g.b_cplx_rows) % kPK == 0;
  if (fast)
    hipLaunchKernelGGL((proj_gemm_kernel<true, true>), dim3((unsigned)tiles), dim3(kPThreads), 0,
                       s, g, m_tiles, tiles);
  else if (vec)
    hipLaunchKernelGGL((proj_gemm_kernel<true, false>), dim3((unsigned)tiles), dim3(kPThreads),
                       0, s, g, m_tiles, tiles);
  else
    hipLaunchKernelGGL((proj_gemm_kernel<false, false>), dim3((unsigned)tiles), dim3(kPThreads),
                       0, s, g, m_tiles, tiles);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RQF_OK : (int)err;
}

// ---------------------------------------------------------------------------
// Gradients of the real-input layer 0's projection z = (Wr + i Wi) h for a
// narrow input (rqf_models/ops/fbt_scan_kernel.py:993-996):
//   grad_h (D, n)        = Re(W^H gz) = Wr^T Re(gz) + Wi^T Im(gz)
//   grad_w_stacked (2F, D) = [Re gz; Im gz] h^T.
// With D output rows the MFMA GEMM above would spend most of its 128-row
// tiles on padding, and the weight gradient is a reduction over all n
// columns; this pass reads gz once.  A thread owns kL0Cols adjacent columns
// and walks the F filters, with the weights read as wave-uniform scalars:
// it accumulates grad_h for its columns, and (D <= kL0MaxDW) its share of
// each filter's weight gradient, which a wavefront sum per filter turns
// into one partial per (wavefront, filter); layer0_wpart_reduce_kernel adds
// the partials in a fixed order in fp64.
// ---------------------------------------------------------------------------
namespace {
constexpr int kL0Threads = 256;
constexpr int kL0Cols = 4;    // columns per thread (two float4 loads of gz per filter)
constexpr int kL0MaxD = 16;   // widest input for grad_h
constexpr int kL0MaxDW = 2;   // widest input whose grad_w rides the same pass

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// VEC: n % 4 == 0 and gz 16-byte aligned, so a thread's columns all exist.
template <int DM, bool GH, bool GW, bool VEC>
__global__ __launch_bounds__(kL0Threads) void layer0_grads_kernel(
    const float* __restrict__ w, const float* __restrict__ gz, const float* __restrict__ h,
    float* __restrict__ gh, float* __restrict__ wpart, int64_t F, int D, int64_t n) {
  const int64_t j0 = ((int64_t)blockIdx.x * kL0Threads + threadIdx.x) * kL0Cols;
  const float* __restrict__ wr = w;          // (F, D): Re W
  const float* __restrict__ wi = w + F * D;  // (F, D): Im W
  float acc[kL0Cols][DM];
  float hv[GW ? kL0Cols : 1][DM];
#pragma unroll
  for (int c = 0; c < kL0Cols; ++c)
#pragma unroll
    for (int d = 0; d < DM; ++d) {
      acc[c][d] = 0.0f;
      if (GW) hv[c][d] = (d < D && j0 + c < n) ? h[d * n + j0 + c] : 0.0f;
    }
  const int wv = (int)(threadIdx.x / kWave);
  float* __restrict__ wp = GW ? wpart + ((int64_t)blockIdx.x * (kL0Threads / kWave) + wv) * F * D * 2
                              : nullptr;
  const bool in_cols = j0 < n;
  for (int64_t f = 0; f < F; ++f) {
    const float* row = gz + 2 * (f * n + j0);
    float g[2 * kL0Cols];
    if (VEC) {
      // n % 4 == 0, so a thread with j0 < n owns all kL0Cols columns and one
      // past the end owns none: it reads the filter's first columns instead
      // (in bounds) and contributes zeros, so the wavefront sums below stay
      // uniform across the wavefront.  A select, not a branch: loads under an
      // exec mask made config 2's layer-0 backward 10% slower (0.422 -> 0.463
      // ms; 0.425 with the select).
      const float* src = in_cols ? row : gz + 2 * f * n;
#pragma unroll
      for (int q = 0; q < kL0Cols / 2; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(src + 4 * q);
        g[4 * q] = in_cols ? v.x : 0.0f, g[4 * q + 1] = in_cols ? v.y : 0.0f;
        g[4 * q + 2] = in_cols ? v.z : 0.0f, g[4 * q + 3] = in_cols ? v.w : 0.0f;
      }
    } else {
#pragma unroll
      for (int c = 0; c < kL0Cols; ++c) {
        const bool in = j0 + c < n;
        g[2 * c] = in ? row[2 * c] : 0.0f;
        g[2 * c + 1] = in ? row[2 * c + 1] : 0.0f;
      }
    }
#pragma unroll
    for (int d = 0; d < DM; ++d) {
      if (d >= D) continue;
      if (GH) {
        const float r = wr[f * D + d], i = wi[f * D + d];
#pragma unroll
        for (int c = 0; c < kL0Cols; ++c)
          acc[c][d] = fmaf(r, g[2 * c], fmaf(i, g[2 * c + 1], acc[c][d]));
      }
      if (GW) {
        float sr = 0.0f, si = 0.0f;
#pragma unroll
        for (int c = 0; c < kL0Cols; ++c) {
          sr = fmaf(g[2 * c], hv[c][d], sr);
          si = fmaf(g[2 * c + 1], hv[c][d], si);
        }
        sr = wave_sum_f(sr);
        si = wave_sum_f(si);
        if (lane_id() == 0) {
          wp[(f * D + d) * 2] = sr;
          wp[(f * D + d) * 2 + 1] = si;
        }
      }
    }
  }
  if (GH) {
#pragma unroll
    for (int d = 0; d < DM; ++d)
      if (d < D)
#pragma unroll
        for (int c = 0; c < kL0Cols; ++c)
          if (j0 + c < n) gh[d * n + j0 + c] = acc[c][d];
  }
}

// grad_w_stacked[f][d] = sum over the P partials (fixed order, fp64) of the
// real parts, grad_w_stacked[F + f][d] of the imaginary parts; one wavefront
// per (f, d) (block fd, fd + gridDim.x, ...), lane l adding partials l,
// l + 64, ...
__global__ __launch_bounds__(kWave) void layer0_wpart_reduce_kernel(const float* __restrict__ wpart,
                                                                    int64_t P, int64_t F, int D,
                                                                    float* __restrict__ gw) {
  const int lane = threadIdx.x;
  for (int64_t fd = blockIdx.x; fd < F * D; fd += gridDim.x) {  // fd = f * D + d
    double sr = 0.0, si = 0.0;
    for (int64_t p = lane; p < P; p += kWave) {
      sr += wpart[(p * F * D + fd) * 2];
      si += wpart[(p * F * D + fd) * 2 + 1];
    }
    sr = wave_sum(sr);
    si = wave_sum(si);
    if (lane == 0) {
      const int64_t f = fd / D, d = fd % D;
      gw[f * D + d] = (float)sr;
      gw[(F + f) * D + d] = (float)si;
    }
  }
}

int64_t layer0_blocks(int64_t n) {
  return (n + (int64_t)kL0Threads * kL0Cols - 1) / ((int64_t)kL0Threads * kL0Cols);
}

template <int DM, bool GH, bool GW>
void launch_layer0(const float* w, const float* gz, const float* h, float* gh, float* wpart,
                   int64_t F, int D, int64_t n, bool vec, hipStream_t s) {
  const dim3 grid((unsigned)layer0_blocks(n)), block(kL0Threads);
  if (vec)
    hipLaunchKernelGGL((layer0_grads_kernel<DM, GH, GW, true>), grid, block, 0, s, w, gz, h, gh,
                       wpart, F, D, n);
  else
    hipLaunchKernelGGL((layer0_grads_kernel<DM, GH, GW, false>), grid, block, 0, s, w, gz, h,
                       gh, wpart, F, D, n);
}

template <int DM>
void launch_layer0_d(const float* w, const float* gz, const float* h, float* gh, float* wpart,
                     int64_t F, int D, int64_t n, bool vec, hipStream_t s) {
  if (gh && wpart) {
    if constexpr (DM <= kL0MaxDW) launch_layer0<DM, true, true>(w, gz, h, gh, wpart, F, D, n, vec, s);
  } else if (gh) {
    launch_layer0<DM, true, false>(w, gz, h, gh, wpart, F, D, n, vec, s);
  } else if constexpr (DM <= kL0MaxDW) {
    launch_layer0<DM, false, true>(w, gz, h, gh, wpart, F, D, n, vec, s);
  }
}
}  // namespace

extern "C" size_t rqf_layer0_grads_workspace(int64_t F, int64_t D, int64_t n) {
  if (F < 0 || D < 1 || D > kL0MaxDW || n < 0) return 0;
  const size_t bytes = sizeof(float) * 2 * (size_t)layer0_blocks(n) * (kL0Threads / kWave) *
                       (size_t)F * (size_t)D;
  return (bytes + 255) & ~(size_t)255;
}

extern "C" int rqf_layer0_grads(const float* w_stacked, const float* grad_z, const float* h,
                                float* grad_h, float* grad_w_stacked, int64_t F, int64_t D,
                                int64_t n, void* workspace, size_t workspace_bytes,
                                rqf_stream_t stream) {
  if (F < 0 || D < 1 || n < 0) return RQF_ERR_ARG;
  if ((grad_h && D > kL0MaxD) || (grad_w_stacked && D > kL0MaxDW)) return RQF_ERR_ARG;
  if (!grad_h && !grad_w_stacked) return RQF_OK;
  hipStream_t s = (hipStream_t)stream;
  // Empty sizes need no special case: with F = 0 the filter loop is empty and
  // grad_h is written as zeros; with n = 0 there are no partials and the
  // reduction writes zeros.
  if ((F > 0 && n > 0 && !grad_z) || (F > 0 && grad_h && !w_stacked) ||
      (n > 0 && grad_w_stacked && !h))
    return RQF_ERR_ARG;
  if (!aligned(w_stacked, 4) || !aligned(grad_z, 8) || !aligned(h, 4) || !aligned(grad_h, 4) ||
      !aligned(grad_w_stacked, 4))
    return RQF_ERR_ALIGN;
  if (!grid_fits(layer0_blocks(n), kL0Threads) || F * D > 0x7fffffff) return RQF_ERR_ARG;
  float* wpart = nullptr;
  if (grad_w_stacked) {
    const size_t need = rqf_layer0_grads_workspace(F, D, n);
    if (need && (!workspace || workspace_bytes < need)) return RQF_ERR_WORKSPACE;
    wpart = (float*)workspace;
  }
  const bool vec = n % kL0Cols == 0 && aligned(grad_z, 16);
  const int d = (int)D;
  if (n == 0)
    ;  // no columns: only the weight-gradient reduction (zeros) runs
  else if (d <= 1)
    launch_layer0_d<1>(w_stacked, grad_z, h, grad_h, wpart, F, d, n, vec, s);
  else if (d <= 2)
    launch_layer0_d<2>(w_stacked, grad_z, h, grad_h, wpart, F, d, n, vec, s);
  else if (d <= 4)
    launch_layer0_d<4>(w_stacked, grad_z, h, grad_h, wpart, F, d, n, vec, s);
  else if (d <= 8)
    launch_layer0_d<8>(w_stacked, grad_z, h, grad_h, wpart, F, d, n, vec, s);
  else
    launch_layer0_d<16>(w_stacked, grad_z, h, grad_h, wpart, F, d, n, vec, s);
  if (grad_w_stacked && F > 0) {
    const int64_t P = layer0_blocks(n) * (kL0Threads / kWave);
    hipLaunchKernelGGL(layer0_wpart_reduce_kernel, dim3(stride_blocks(F * D)), dim3(kWave), 0, s,
                       wpart, P, F, d, grad_w_stacked);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? RQF_OK : (int)err;
}
