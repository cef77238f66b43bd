// Raw-case preprocessing on the device: nonzero crop bounds, crop + transpose + per-channel
// normalisation, and the spline resampling of image data to the plans' spacing.
//
// Replaces the host steps of preprocess_raw_case (src/nnunet_mlx/data/preprocessing.py:63-163):
// the crop bounds of crop_to_nonzero (:166-214; no mask, as CT normalisation uses none),
// the CTNormalization branch of _normalize_channel (:274-285), and the data resize of
// resample_probabilities_or_data for spline plans (src/nnunet_mlx/data/resampling.py:87-172,
// 268-306, 379-442, 476-501), which the reference delegates to scikit-image's
// resize(order, mode="edge", anti_aliasing=False): scipy.ndimage.zoom in grid mode with
// edge extension, then a clip to the input's [min, max].
//
// Spline arithmetic (float64 throughout, no contraction):
//   * pad every resized axis by 12 voxels with edge replication (SciPy pads this way before
//     building coefficients for edge extension);
//   * order 3: per axis in turn, per line: multiply by the gain (1 - z)(1 - 1/z), causal
//     initialisation for edge extension c0' = (c0 + z^n c[n-1] + sum_{i=1}^{n-1} z^i (c[i] +
//     z^n c[n-1-i])) * z / (1 - z^2n) + c0 (terms past i = 48, below float64 resolution,
//     omitted), causal recursion c[i] += z c[i-1], anticausal initialisation
//     c[n-1] *= z / (z - 1), anticausal recursion c[i] = z (c[i+1] - c[i]), pole
//     z = sqrt(3) - 2;
//   * evaluation one axis at a time: output index o samples the padded coordinate
//     cc = (o + 0.5) * n_in / n_out - 0.5 + 12 with the cardinal cubic B-spline weights of
//     t = cc - floor(cc) at floor(cc) - 1 .. floor(cc) + 2 (order 1: 1 - t, t at floor(cc),
//     floor(cc) + 1), summed from 0 in tap order;
//   * whole volume: cast to float32, clip to the channel's input [min, max]; separate axis:
//     the other two axes resized per plane (float64, clipped to the plane's [min, max]),
//     then the separate axis by half-pixel nearest indices floor(old/new (o + 0.5) - 0.5 +
//     0.5) clamped, cast to float32 once.
// Roofline: HBM — the edge copy writes, each prefilter axis reads and writes twice (causal,
// anticausal) and each interpolation pass reads and writes its float64 array once; the
// crop/normalise pass reads and writes 4 B per kept voxel.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>

#include "nnx_internal.h"

namespace nnx {
namespace {

constexpr int kSplinePad = 12;
constexpr int kMinmaxParts = 16;  // blocks per plane of the min/max reduction

// ---- nonzero bounds -------------------------------------------------------------------

__global__ void bbox_init_kernel(int* bbox) {
  if (threadIdx.x < 3) {
    bbox[2 * threadIdx.x] = INT_MAX;
    bbox[2 * threadIdx.x + 1] = -1;
  }
}

// bbox[2a] / bbox[2a + 1] = smallest / largest index along axis a of a voxel where any
// channel is nonzero.  One wave per (x, y) row at a time, its lanes along z (coalesced);
// block minima and maxima reach memory by one vector atomic each.
__global__ __launch_bounds__(256) void bbox_kernel(const float* __restrict__ x, int C, int64_t X,
                                                   int64_t Y, int64_t Z, int* bbox) {
  __shared__ int red[6][4];
  int lo[3] = {INT_MAX, INT_MAX, INT_MAX}, hi[3] = {-1, -1, -1};
  const int64_t n = X * Y * Z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t r = blockIdx.x * (int64_t)4 + wave; r < X * Y; r += waves) {
    const float* row = x + r * Z;
    int zlo = INT_MAX, zhi = -1;
    for (int64_t z = lane; z < Z; z += 64) {
      bool nz = false;
      for (int c = 0; c < C; ++c) nz |= row[(int64_t)c * n + z] != 0.f;
      if (nz) {
        zlo = min(zlo, (int)z);
        zhi = max(zhi, (int)z);
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      zlo = min(zlo, __shfl_xor(zlo, o));
      zhi = max(zhi, __shfl_xor(zhi, o));
    }
    if (zhi >= 0) {
      const int rx = (int)(r / Y), ry = (int)(r % Y);
      lo[0] = min(lo[0], rx);
      hi[0] = max(hi[0], rx);
      lo[1] = min(lo[1], ry);
      hi[1] = max(hi[1], ry);
      lo[2] = min(lo[2], zlo);
      hi[2] = max(hi[2], zhi);
    }
  }
  if (lane == 0)
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      red[2 * a][wave] = lo[a];
      red[2 * a + 1][wave] = hi[a];
    }
  __syncthreads();
  if (threadIdx.x < 6) {
    const int k = threadIdx.x;
    int v = red[k][0];
    for (int w = 1; w < 4; ++w) v = (k & 1) ? max(v, red[k][w]) : min(v, red[k][w]);
    if (k & 1) {
      if (v >= 0) atomicMax(&bbox[k], v);
    } else if (v != INT_MAX) {
      atomicMin(&bbox[k], v);
    }
  }
}

// ---- crop + transpose + normalise -------------------------------------------------------

constexpr int kMaxNormChannels = 16;

struct ChannelNorms {
  int scheme[kMaxNormChannels];  // NNX_NORM_*
  float mean[kMaxNormChannels], std[kMaxNormChannels];  // std already max(std, 1e-8)
  float lower[kMaxNormChannels], upper[kMaxNormChannels];
};

// ---- filled nonzero mask ----------------------------------------------------------------
// Cells of the crop box (E0, E1, E2) of the raw volume: 2 = some channel nonzero, 1 =
// background reached from the box border through background (6-connected), 0 = background
// not reached yet.  After the sweeps converge the filled mask is cell != 1.

__global__ __launch_bounds__(256) void mask_init_kernel(const float* __restrict__ x, int C,
                                                        int64_t X, int64_t Y, int64_t Z,
                                                        int64_t b0, int64_t b1, int64_t b2,
                                                        int64_t E0, int64_t E1, int64_t E2,
                                                        uint8_t* __restrict__ cell) {
  const int64_t n = X * Y * Z, total = E0 * E1 * E2;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i2 = e % E2, i1 = (e / E2) % E1, i0 = e / (E1 * E2);
    const int64_t src = ((b0 + i0) * Y + (b1 + i1)) * Z + (b2 + i2);
    bool nz = false;
    for (int c = 0; c < C; ++c) nz |= x[(int64_t)c * n + src] != 0.f;
    const bool border = i0 == 0 || i1 == 0 || i2 == 0 || i0 == E0 - 1 || i1 == E1 - 1 ||
                        i2 == E2 - 1;
    cell[e] = nz ? 2 : (border ? 1 : 0);
  }
}

// Propagate "reached" along every line of `axis` in both directions (one thread per line;
// for axes 0 and 1 neighbouring threads hold neighbouring lines).  *changed = 1 when a
// cell changed.
__global__ __launch_bounds__(256) void mask_sweep_kernel(uint8_t* __restrict__ cell, int64_t E0,
                                                         int64_t E1, int64_t E2, int axis,
                                                         int* __restrict__ changed) {
  const int64_t dims[3] = {E0, E1, E2};
  const int64_t strides[3] = {E1 * E2, E2, 1};
  const int64_t len = dims[axis], stride = strides[axis];
  const int64_t lines = E0 * E1 * E2 / len;
  const int64_t line = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (line >= lines) return;
  int64_t base;
  if (axis == 2) base = line * E2;
  else if (axis == 1) base = (line / E2) * E1 * E2 + line % E2;
  else base = line;
  bool any = false, carry = false;
  for (int64_t i = 0; i < len; ++i) {
    uint8_t& v = cell[base + i * stride];
    if (v == 2) carry = false;
    else if (v == 1) carry = true;
    else if (carry) { v = 1; any = true; }
  }
  carry = false;
  for (int64_t i = len - 1; i >= 0; --i) {
    uint8_t& v = cell[base + i * stride];
    if (v == 2) carry = false;
    else if (v == 1) carry = true;
    else if (carry) { v = 1; any = true; }
  }
  if (any) *changed = 1;
}

__global__ void flag_clear_kernel(int* flag) { *flag = 0; }

__global__ __launch_bounds__(256) void mask_finish_kernel(uint8_t* __restrict__ cell, int64_t n) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x)
    cell[e] = cell[e] != 1;
}

// ---- channel extrema over the crop box ----------------------------------------------------

__global__ __launch_bounds__(256) void box_minmax_partial_kernel(
    const float* __restrict__ xc, int64_t Y, int64_t Z, int64_t b0, int64_t b1, int64_t b2,
    int64_t E0, int64_t E1, int64_t E2, float2* __restrict__ partial) {
  __shared__ float smin[4], smax[4];
  const int64_t total = E0 * E1 * E2;
  float lo = INFINITY, hi = -INFINITY;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i2 = e % E2, i1 = (e / E2) % E1, i0 = e / (E1 * E2);
    const float v = xc[((b0 + i0) * Y + (b1 + i1)) * Z + (b2 + i2)];
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    smin[wave] = lo;
    smax[wave] = hi;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    partial[blockIdx.x] = make_float2(fminf(fminf(smin[0], smin[1]), fminf(smin[2], smin[3])),
                                      fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3])));
}

__global__ __launch_bounds__(64) void box_minmax_final_kernel(const float2* __restrict__ partial,
                                                             int parts, float* __restrict__ out) {
  float lo = INFINITY, hi = -INFINITY;
  for (int i = threadIdx.x; i < parts; i += 64) {
    lo = fminf(lo, partial[i].x);
    hi = fmaxf(hi, partial[i].y);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  if (threadIdx.x == 0) {
    out[0] = lo;
    out[1] = hi;
  }
}

// ---- z-score statistics -----------------------------------------------------------------
// Per block: float64 sums over the crop box of channel c (mask cells only when `mask`),
// pass 0: (sum x, count), pass 1: (sum (x - mean32)^2, count) with mean32 = stats[2c].

constexpr int kStatBlocks = 1024;

__global__ __launch_bounds__(256) void zscore_partial_kernel(
    const float* __restrict__ xc, int64_t Y, int64_t Z, int64_t b0, int64_t b1, int64_t b2,
    int64_t E0, int64_t E1, int64_t E2, const uint8_t* __restrict__ mask, int pass,
    const float* __restrict__ stats, double2* __restrict__ partial) {
  __shared__ double ssum[4], scnt[4];
  const int64_t total = E0 * E1 * E2;
  const double mean = pass ? (double)stats[0] : 0.0;
  double acc = 0.0, cnt = 0.0;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    if (mask && !mask[e]) continue;
    const int64_t i2 = e % E2, i1 = (e / E2) % E1, i0 = e / (E1 * E2);
    const double v = (double)xc[((b0 + i0) * Y + (b1 + i1)) * Z + (b2 + i2)];
    acc += pass ? (v - mean) * (v - mean) : v;
    cnt += 1.0;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    acc += __shfl_xor(acc, o);
    cnt += __shfl_xor(cnt, o);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    ssum[wave] = acc;
    scnt[wave] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    partial[blockIdx.x] = make_double2(ssum[0] + ssum[1] + ssum[2] + ssum[3],
                                       scnt[0] + scnt[1] + scnt[2] + scnt[3]);
}

// stats[0] = float(sum / n) (pass 0) or stats[1] = float(sqrt(sum / n)) (pass 1); a fixed
// summation order over the partials, so the result is deterministic
__global__ __launch_bounds__(64) void zscore_final_kernel(const double2* __restrict__ partial,
                                                         int parts, int pass,
                                                         float* __restrict__ stats) {
  double acc = 0.0, cnt = 0.0;
  for (int i = threadIdx.x; i < parts; i += 64) {
    acc += partial[i].x;
    cnt += partial[i].y;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    acc += __shfl_xor(acc, o);
    cnt += __shfl_xor(cnt, o);
  }
  if (threadIdx.x == 0) {
    const double m = cnt > 0 ? acc / cnt : NAN;
    if (pass == 0) stats[0] = (float)m;
    else stats[1] = (float)sqrt(m);
  }
}

// out[c][o0][o1][o2] = norm_c(x[c][r0][r1][r2]) with r[t_k] = s_k + o_k: out axis k is input
// axis t_k, cropped to start s_k.  NNX_NORM_ZSCORE_MASKED normalises only where the filled
// mask (raw-order box starting at (m0, m1, m2), extents (*, ME1, ME2)) is set.
__global__ __launch_bounds__(256) void crop_normalize_kernel(
    const float* __restrict__ x, int C, int64_t X, int64_t Y, int64_t Z, int t0, int t1, int t2,
    int64_t s0, int64_t s1, int64_t s2, int64_t O0, int64_t O1, int64_t O2, ChannelNorms norms,
    const uint8_t* __restrict__ mask, int64_t m0, int64_t m1, int64_t m2, int64_t ME1,
    int64_t ME2, float* __restrict__ out) {
  const int64_t per = O0 * O1 * O2;
  const int64_t total = per * C;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(e / per);
    const int64_t p = e - c * per;
    const int64_t o2 = p % O2, o1 = (p / O2) % O1, o0 = p / (O1 * O2);
    const int64_t a0 = s0 + o0, a1 = s1 + o1, a2 = s2 + o2;
    const int64_t r0 = t0 == 0 ? a0 : t1 == 0 ? a1 : a2;
    const int64_t r1 = t0 == 1 ? a0 : t1 == 1 ? a1 : a2;
    const int64_t r2 = t0 == 2 ? a0 : t1 == 2 ? a1 : a2;
    float v = x[(int64_t)c * X * Y * Z + (r0 * Y + r1) * Z + r2];
    const int scheme = norms.scheme[c];
    if (scheme == NNX_NORM_CT) {
      v = fminf(fmaxf(v, norms.lower[c]), norms.upper[c]);
      v = __fdiv_rn(__fsub_rn(v, norms.mean[c]), norms.std[c]);
    } else if (scheme == NNX_NORM_ZSCORE ||
               (scheme == NNX_NORM_ZSCORE_MASKED &&
                mask[((r0 - m0) * ME1 + (r1 - m1)) * ME2 + (r2 - m2)])) {
      v = __fdiv_rn(__fsub_rn(v, norms.mean[c]), norms.std[c]);
    }
    out[e] = v;
  }
}

// ---- spline resampling -----------------------------------------------------------------

// out (P0, P1, P2) float64 = in (n0, n1, n2) float32 edge-extended by p_a on each side of
// axis a.
__global__ __launch_bounds__(256) void pad_edge_kernel(const float* __restrict__ in, int64_t n0,
                                                       int64_t n1, int64_t n2, int p0, int p1,
                                                       int p2, double* __restrict__ out) {
  const int64_t P0 = n0 + 2 * p0, P1 = n1 + 2 * p1, P2 = n2 + 2 * p2;
  const int64_t total = P0 * P1 * P2;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i2 = e % P2, i1 = (e / P2) % P1, i0 = e / (P1 * P2);
    const int64_t j0 = min(max(i0 - p0, (int64_t)0), n0 - 1);
    const int64_t j1 = min(max(i1 - p1, (int64_t)0), n1 - 1);
    const int64_t j2 = min(max(i2 - p2, (int64_t)0), n2 - 1);
    out[e] = (double)in[(j0 * n1 + j1) * n2 + j2];
  }
}

// The initial sums of the causal recursion run over the first and last kInitTaps
// elements only: |z|^48 ~ 3.5e-28, so later terms lie below float64 resolution.
constexpr int kInitTaps = 48;

// Cubic B-spline coefficients along `axis` (0 or 1) of a (P0, P1, P2) float64 array, in
// place; one thread per line, neighbouring threads on neighbouring lines (coalesced).  The
// gain is applied as each element is first read: c'[0] from the initial sum, then
// c[i] = gain c[i] + z c[i-1], c[n-1] *= z / (z - 1), c[i] = z (c[i+1] - c[i]).
__global__ __launch_bounds__(256) void prefilter_strided_kernel(double* __restrict__ c,
                                                                int64_t P0, int64_t P1,
                                                                int64_t P2, int axis, double z,
                                                                double z_n, double gain) {
  const int64_t dims[3] = {P0, P1, P2};
  const int64_t strides[3] = {P1 * P2, P2, 1};
  const int64_t n = dims[axis], s = strides[axis];
  const int a1 = axis == 0 ? 1 : 0, a2 = axis == 2 ? 1 : 2;
  const int64_t lines = dims[a1] * dims[a2];
  const int64_t l = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (l >= lines || n < 2) return;
  double* line = c + (l / dims[a2]) * strides[a1] + (l % dims[a2]) * strides[a2];
  const int64_t K = n - 1 < kInitTaps ? n - 1 : kInitTaps;
  const double c0 = line[0] * gain;
  double acc = c0 + z_n * (line[(n - 1) * s] * gain);
  double z_i = z;
  for (int64_t i = 1; i <= K; ++i) {
    acc = acc + z_i * (line[i * s] * gain + z_n * (line[(n - 1 - i) * s] * gain));
    z_i = z_i * z;
  }
  double prev = acc * (z / (1.0 - z_n * z_n)) + c0;
  line[0] = prev;
  for (int64_t i = 1; i < n; ++i) {
    prev = line[i * s] * gain + z * prev;
    line[i * s] = prev;
  }
  double next = prev * (z / (z - 1.0));
  line[(n - 1) * s] = next;
  for (int64_t i = n - 2; i >= 0; --i) {
    next = z * (next - line[i * s]);
    line[i * s] = next;
  }
}

// The same coefficients along the contiguous axis: lines are rows of n elements.  A block
// takes 256 consecutive rows (one per thread) and moves them through LDS in chunks of
// kTileW elements, so every global access reads or writes 128-byte row segments.
constexpr int kTileW = 16;

__global__ __launch_bounds__(256) void prefilter_contig_kernel(double* __restrict__ c,
                                                               int64_t lines, int64_t n,
                                                               double z, double z_n,
                                                               double gain) {
  __shared__ double tile[256][kTileW + 1];
  __shared__ double zp[kInitTaps + 1];
  const int t = threadIdx.x;
  const int64_t l0 = blockIdx.x * (int64_t)256;
  if (t == 0) {
    zp[0] = 1.0;
    for (int i = 1; i <= kInitTaps; ++i) zp[i] = zp[i - 1] * z;
  }
  auto load = [&](int64_t k0) {
    for (int p = 0; p < 256 / (256 / kTileW); ++p) {
      const int j = p * (256 / kTileW) + t / kTileW, q = t % kTileW;
      const int64_t i = k0 + q, line = l0 + j;
      tile[j][q] = (line < lines && i < n) ? c[line * n + i] : 0.0;
    }
  };
  auto store = [&](int64_t k0) {
    for (int p = 0; p < 256 / (256 / kTileW); ++p) {
      const int j = p * (256 / kTileW) + t / kTileW, q = t % kTileW;
      const int64_t i = k0 + q, line = l0 + j;
      if (line < lines && i < n) c[line * n + i] = tile[j][q];
    }
  };
  if (n < 2) return;
  const int64_t K = n - 1 < kInitTaps ? n - 1 : kInitTaps;
  // initial sum: head elements 1..K and tail elements n-1-K..n-2 (as distances 1..K)
  double c0 = 0.0, cn = 0.0, head = 0.0, tail = 0.0;
  for (int64_t k0 = 0; k0 <= K; k0 += kTileW) {
    __syncthreads();
    load(k0);
    __syncthreads();
    for (int q = 0; q < kTileW; ++q) {
      const int64_t i = k0 + q;
      if (i == 0) c0 = tile[t][q] * gain;
      else if (i <= K) head = head + zp[i] * (tile[t][q] * gain);
    }
  }
  for (int64_t k0 = (n - 1 - K) / kTileW * kTileW; k0 < n; k0 += kTileW) {
    __syncthreads();
    load(k0);
    __syncthreads();
    for (int q = 0; q < kTileW; ++q) {
      const int64_t i = k0 + q;
      if (i == n - 1) cn = tile[t][q] * gain;
      else if (i >= n - 1 - K && i < n - 1) tail = tail + zp[n - 1 - i] * (tile[t][q] * gain);
    }
  }
  const double acc = (c0 + z_n * cn) + head + z_n * tail;
  double prev = acc * (z / (1.0 - z_n * z_n)) + c0;
  for (int64_t k0 = 0; k0 < n; k0 += kTileW) {
    __syncthreads();
    load(k0);
    __syncthreads();
    for (int q = 0; q < kTileW; ++q) {
      const int64_t i = k0 + q;
      if (i >= n) break;
      if (i > 0) prev = tile[t][q] * gain + z * prev;
      tile[t][q] = prev;
    }
    __syncthreads();
    store(k0);
  }
  double next = prev * (z / (z - 1.0));
  for (int64_t k0 = (n - 1) / kTileW * kTileW; k0 >= 0; k0 -= kTileW) {
    __syncthreads();
    load(k0);
    __syncthreads();
    for (int q = kTileW - 1; q >= 0; --q) {
      const int64_t i = k0 + q;
      if (i >= n) continue;
      if (i < n - 1) next = z * (next - tile[t][q]);
      tile[t][q] = next;
    }
    __syncthreads();
    store(k0);
  }
}

// One interpolation pass along `axis`: in (I0, I1, I2) -> out with that axis n_out long.
// The axis holds n_in source samples padded by `pad` on each side.
template <int ORDER>
__global__ __launch_bounds__(256) void interp_axis_kernel(const double* __restrict__ in,
                                                          int64_t I0, int64_t I1, int64_t I2,
                                                          int axis, int64_t n_out, double ratio,
                                                          int pad, double* __restrict__ out) {
  int64_t dims[3] = {I0, I1, I2};
  const int64_t in_stride = axis == 0 ? I1 * I2 : axis == 1 ? I2 : 1;
  dims[axis] = n_out;
  const int64_t total = dims[0] * dims[1] * dims[2];
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t q2 = e % dims[2], q1 = (e / dims[2]) % dims[1], q0 = e / (dims[1] * dims[2]);
    const int64_t o = axis == 0 ? q0 : axis == 1 ? q1 : q2;
    // source element of tap 0 with the axis coordinate set to 0
    const int64_t row = axis == 0 ? q1 * I2 + q2 : axis == 1 ? q0 * I1 * I2 + q2
                                                             : (q0 * I1 + q1) * I2;
    const double cc = ((double)o + 0.5) * ratio - 0.5 + (double)pad;
    const double f = floor(cc);
    const double t = cc - f;
    double sum = 0.0;
    if constexpr (ORDER == 3) {
      const double u = 1.0 - t;
      const double w[4] = {u * u * u / 6.0, 2.0 / 3.0 - t * t + t * t * t / 2.0,
                           2.0 / 3.0 - u * u + u * u * u / 2.0, t * t * t / 6.0};
      const int64_t start = (int64_t)f - 1;
#pragma unroll
      for (int k = 0; k < 4; ++k) sum = sum + in[row + (start + k) * in_stride] * w[k];
    } else {
      const int64_t start = (int64_t)f;
      sum = sum + in[row + start * in_stride] * (1.0 - t);
      sum = sum + in[row + (start + 1) * in_stride] * t;
    }
    out[e] = sum;
  }
}

// part[k * parts + j] = (min, max) over part j of plane k along `axis` of a (n0, n1, n2)
// float32 channel; grid (planes, parts).
__global__ __launch_bounds__(256) void plane_minmax_kernel(const float* __restrict__ in,
                                                           int64_t n0, int64_t n1, int64_t n2,
                                                           int axis, float2* __restrict__ part) {
  __shared__ float smin[4], smax[4];
  const int64_t k = blockIdx.x;
  const int parts = gridDim.y, j = blockIdx.y;
  const int64_t dims[3] = {n0, n1, n2};
  const int a1 = axis == 0 ? 1 : 0, a2 = axis == 2 ? 1 : 2;
  const int64_t strides[3] = {n1 * n2, n2, 1};
  const int64_t m = dims[a1] * dims[a2];
  float lo = INFINITY, hi = -INFINITY;
  for (int64_t i = j * (int64_t)blockDim.x + threadIdx.x; i < m; i += (int64_t)parts * blockDim.x) {
    const float v = in[k * strides[axis] + (i / dims[a2]) * strides[a1] + (i % dims[a2]) * strides[a2]];
    lo = fminf(lo, v);
    hi = fmaxf(hi, v);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    smin[wave] = lo;
    smax[wave] = hi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) {
      lo = fminf(lo, smin[w]);
      hi = fmaxf(hi, smax[w]);
    }
    part[k * parts + j] = make_float2(lo, hi);
  }
}

// mm[k] = (min, max) over part[k * parts .. k * parts + parts), one thread per plane
__global__ __launch_bounds__(256) void plane_parts_kernel(const float2* __restrict__ part,
                                                          int64_t planes, int parts,
                                                          float2* __restrict__ mm) {
  const int64_t k = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (k >= planes) return;
  float lo = INFINITY, hi = -INFINITY;
  for (int j = 0; j < parts; ++j) {
    lo = fminf(lo, part[k * parts + j].x);
    hi = fmaxf(hi, part[k * parts + j].y);
  }
  mm[k] = make_float2(lo, hi);
}

// mm[n] = (min, max) over mm[0 .. n)
__global__ __launch_bounds__(64) void reduce_minmax_kernel(float2* mm, int64_t n) {
  float lo = INFINITY, hi = -INFINITY;
  for (int64_t i = threadIdx.x; i < n; i += 64) {
    lo = fminf(lo, mm[i].x);
    hi = fmaxf(hi, mm[i].y);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
  }
  if (threadIdx.x == 0) mm[n] = make_float2(lo, hi);
}

// One rounding of a float64 result: to float32, or to float16 (nearest even) when HALF,
// returned as float32.
template <bool HALF>
__device__ inline float round_result(double v) {
  if constexpr (HALF) return (float)(_Float16)v;  // correctly rounded (integer sequence)
  else return (float)v;
}

// whole-volume resize: out = clip(round(v), min, max); the bounds are values of the input,
// so clipping before or after the monotone rounding gives the same result
template <bool HALF>
__global__ __launch_bounds__(256) void cast_clip_kernel(const double* __restrict__ in, int64_t n,
                                                        const float2* __restrict__ mm,
                                                        float* __restrict__ out) {
  const float2 b = *mm;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x)
    out[e] = fminf(fmaxf(round_result<HALF>(in[e]), b.x), b.y);
}

// separate axis: out[.. o ..] = round(clip_k(inter[.. k ..])), k = nearest source plane of o
template <bool HALF>
__global__ __launch_bounds__(256) void plane_clip_nearest_kernel(
    const double* __restrict__ inter, int64_t d0, int64_t d1, int64_t d2, int axis,
    int64_t n_new, double ratio, const float2* __restrict__ mm, float* __restrict__ out) {
  int64_t dims[3] = {d0, d1, d2};
  const int64_t n_old = dims[axis];
  const int64_t in_stride = axis == 0 ? d1 * d2 : axis == 1 ? d2 : 1;
  dims[axis] = n_new;
  const int64_t total = dims[0] * dims[1] * dims[2];
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t q2 = e % dims[2], q1 = (e / dims[2]) % dims[1], q0 = e / (dims[1] * dims[2]);
    const int64_t o = axis == 0 ? q0 : axis == 1 ? q1 : q2;
    const int64_t row = axis == 0 ? q1 * d2 + q2 : axis == 1 ? q0 * d1 * d2 + q2
                                                             : (q0 * d1 + q1) * d2;
    const double coord = ratio * ((double)o + 0.5) - 0.5;
    int64_t k = (int64_t)floor(coord + 0.5);
    k = min(max(k, (int64_t)0), n_old - 1);
    const float2 b = mm[k];
    const double v = fmin(fmax(inter[row + k * in_stride], (double)b.x), (double)b.y);
    out[e] = round_result<HALF>(v);
  }
}

int blocks_for(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), 1 << 20)); }

struct SplinePlan {
  int64_t n[3], N[3];
  int pad[3];
  int axes[3], naxes;  // resized axes, in order
  int64_t a_elems, b_elems, mm_elems;
};

SplinePlan spline_plan(const int64_t* size, const int64_t* new_size, int separate_axis) {
  SplinePlan p{};
  p.naxes = 0;
  for (int a = 0; a < 3; ++a) {
    p.n[a] = size[a];
    p.N[a] = new_size[a];
    const bool resized = a != separate_axis;
    p.pad[a] = resized ? kSplinePad : 0;
    if (resized) p.axes[p.naxes++] = a;
  }
  // ping-pong: A holds the padded copy, B the first pass, A the second, B the third
  int64_t d[3] = {p.n[0] + 2 * p.pad[0], p.n[1] + 2 * p.pad[1], p.n[2] + 2 * p.pad[2]};
  int64_t sizes[4];
  sizes[0] = d[0] * d[1] * d[2];
  for (int k = 0; k < p.naxes; ++k) {
    d[p.axes[k]] = p.N[p.axes[k]];
    sizes[k + 1] = d[0] * d[1] * d[2];
  }
  p.a_elems = p.b_elems = 0;
  for (int k = 0; k <= p.naxes; ++k) {
    int64_t& slot = (k % 2 == 0) ? p.a_elems : p.b_elems;
    slot = std::max(slot, sizes[k]);
  }
  // per-plane (min, max) + the whole-volume entry, then the per-part partials
  const int64_t planes = separate_axis >= 0 ? p.n[separate_axis] : p.n[0];
  p.mm_elems = planes + 1 + planes * kMinmaxParts;
  return p;
}

}  // namespace

void nonzero_bbox(const float* x, int channels, const int64_t* size, int* bbox, hipStream_t st) {
  require(x && bbox && size, "bounding-box pointers must not be null");
  require(channels >= 1 && size[0] >= 1 && size[1] >= 1 && size[2] >= 1, "invalid volume shape");
  const int64_t n = size[0] * size[1] * size[2];
  require(size[0] < INT_MAX && size[1] < INT_MAX && size[2] < INT_MAX, "volume axis too long");
  ProfScope prof("preprocess_bbox", 0.0, 4.0 * (double)n * channels, st);
  hipLaunchKernelGGL(bbox_init_kernel, dim3(1), dim3(64), 0, st, bbox);
  hipLaunchKernelGGL(bbox_kernel,
                     dim3((unsigned)std::min<int64_t>(ceil_div(size[0] * size[1], 4), 8192)),
                     dim3(256), 0, st, x, channels, size[0], size[1], size[2], bbox);
  launch_check("nonzero_bbox");
}

int nonzero_mask_filled(const float* x, int channels, const int64_t* size, const int64_t* start,
                        const int64_t* extent, uint8_t* mask, void* work, hipStream_t st) {
  require(x && size && start && extent && mask && work, "mask pointers must not be null");
  require(channels >= 1, "mask needs at least one channel");
  for (int a = 0; a < 3; ++a)
    require(extent[a] >= 1 && start[a] >= 0 && start[a] <= size[a] &&
                extent[a] <= size[a] - start[a],
            "mask box outside the volume");
  const int64_t total = extent[0] * extent[1] * extent[2];
  int* flag = static_cast<int*>(work);
  ProfScope prof("preprocess_fill_holes", 0.0, 4.0 * (double)total * channels, st);
  hipLaunchKernelGGL(mask_init_kernel, dim3(blocks_for(total)), dim3(256), 0, st, x, channels,
                     size[0], size[1], size[2], start[0], start[1], start[2], extent[0],
                     extent[1], extent[2], mask);
  // every round with a change reaches at least one more cell, so at most `total` rounds
  int rounds = 0;
  for (int64_t r = 0; r <= total; ++r) {
    hipLaunchKernelGGL(flag_clear_kernel, dim3(1), dim3(1), 0, st, flag);
    for (int axis = 2; axis >= 0; --axis) {
      const int64_t lines = total / extent[axis];
      hipLaunchKernelGGL(mask_sweep_kernel, dim3((unsigned)ceil_div(lines, 256)), dim3(256), 0,
                         st, mask, extent[0], extent[1], extent[2], axis, flag);
    }
    int changed = 0;
    hip_check(hipMemcpyAsync(&changed, flag, sizeof(int), hipMemcpyDeviceToHost, st),
              "mask flag copy");
    hip_check(hipStreamSynchronize(st), "mask flag sync");
    ++rounds;
    if (!changed) break;
  }
  hipLaunchKernelGGL(mask_finish_kernel, dim3(blocks_for(total)), dim3(256), 0, st, mask, total);
  launch_check("nonzero_mask_filled");
  return rounds;
}

size_t zscore_stats_workspace() { return kStatBlocks * sizeof(double2); }

void zscore_stats(const float* x, int channels, const int64_t* size, int channel,
                  const int64_t* start, const int64_t* extent, const uint8_t* mask, float* stats,
                  void* work, hipStream_t st) {
  require(x && size && start && extent && stats && work, "z-score pointers must not be null");
  require(channel >= 0 && channel < channels, "z-score channel out of range");
  for (int a = 0; a < 3; ++a)
    require(extent[a] >= 1 && start[a] >= 0 && start[a] <= size[a] &&
                extent[a] <= size[a] - start[a],
            "z-score box outside the volume");
  const int64_t total = extent[0] * extent[1] * extent[2];
  const float* xc = x + (int64_t)channel * size[0] * size[1] * size[2];
  double2* partial = static_cast<double2*>(work);
  const int blocks = (int)std::min<int64_t>(kStatBlocks, ceil_div(total, 256));
  ProfScope prof("preprocess_zscore_stats", 0.0, 8.0 * (double)total, st);
  for (int pass = 0; pass < 2; ++pass) {
    hipLaunchKernelGGL(zscore_partial_kernel, dim3(blocks), dim3(256), 0, st, xc, size[1],
                       size[2], start[0], start[1], start[2], extent[0], extent[1], extent[2],
                       mask, pass, stats, partial);
    hipLaunchKernelGGL(zscore_final_kernel, dim3(1), dim3(64), 0, st, partial, blocks, pass,
                       stats);
  }
  launch_check("zscore_stats");
}

void box_minmax(const float* x, int channels, const int64_t* size, int channel,
                const int64_t* start, const int64_t* extent, float* minmax, void* work,
                hipStream_t st) {
  require(x && size && start && extent && minmax && work, "extrema pointers must not be null");
  require(channel >= 0 && channel < channels, "extrema channel out of range");
  for (int a = 0; a < 3; ++a)
    require(extent[a] >= 1 && start[a] >= 0 && start[a] <= size[a] &&
                extent[a] <= size[a] - start[a],
            "extrema box outside the volume");
  const int64_t total = extent[0] * extent[1] * extent[2];
  const float* xc = x + (int64_t)channel * size[0] * size[1] * size[2];
  float2* partial = static_cast<float2*>(work);  // zscore_stats_workspace() bytes suffice
  const int blocks = (int)std::min<int64_t>(kStatBlocks, ceil_div(total, 256));
  ProfScope prof("preprocess_minmax", 0.0, 4.0 * (double)total, st);
  hipLaunchKernelGGL(box_minmax_partial_kernel, dim3(blocks), dim3(256), 0, st, xc, size[1],
                     size[2], start[0], start[1], start[2], extent[0], extent[1], extent[2],
                     partial);
  hipLaunchKernelGGL(box_minmax_final_kernel, dim3(1), dim3(64), 0, st, partial, blocks, minmax);
  launch_check("box_minmax");
}

void crop_normalize(const float* x, int channels, const int64_t* size, const int* transpose,
                    const int64_t* start, const int64_t* out_size, const int* schemes,
                    const float* norm, float* out, hipStream_t st) {
  crop_normalize_masked(x, channels, size, transpose, start, out_size, schemes, norm, nullptr,
                        nullptr, nullptr, out, st);
}

void crop_normalize_masked(const float* x, int channels, const int64_t* size,
                           const int* transpose, const int64_t* start, const int64_t* out_size,
                           const int* schemes, const float* norm, const uint8_t* mask,
                           const int64_t* mask_start, const int64_t* mask_extent, float* out,
                           hipStream_t st) {
  require(x && out && size && transpose && start && out_size && schemes,
          "crop/normalise pointers must not be null");
  require(channels >= 1 && channels <= kMaxNormChannels,
          "device normalisation supports 1..16 channels");
  bool seen[3] = {false, false, false};
  for (int k = 0; k < 3; ++k) {
    require(transpose[k] >= 0 && transpose[k] < 3 && !seen[transpose[k]],
            "transpose must be a permutation of the three spatial axes");
    seen[transpose[k]] = true;
  }
  for (int k = 0; k < 3; ++k) {
    const int64_t n = size[transpose[k]];
    require(out_size[k] >= 1 && start[k] >= 0 && start[k] <= n &&
                out_size[k] <= n - start[k],
            "crop window outside the volume");
  }
  ChannelNorms cn{};
  bool masked = false;
  for (int c = 0; c < channels; ++c) {
    require(schemes[c] >= NNX_NORM_NONE && schemes[c] <= NNX_NORM_ZSCORE_MASKED,
            "device normalisation supports NoNormalization, CTNormalization and "
            "ZScoreNormalization");
    cn.scheme[c] = schemes[c];
    if (schemes[c] == NNX_NORM_ZSCORE || schemes[c] == NNX_NORM_ZSCORE_MASKED) {
      require(norm != nullptr, "z-score normalisation needs its statistics");
      const float* p = norm + 4 * c;
      require(std::isfinite(p[0]) && std::isfinite(p[1]) && p[1] >= 0.f,
              "z-score statistics must be finite with a non-negative std");
      cn.mean[c] = p[0];
      cn.std[c] = std::max(p[1], 1e-8f);
      masked |= schemes[c] == NNX_NORM_ZSCORE_MASKED;
    }
    if (schemes[c] == NNX_NORM_CT) {
      require(norm != nullptr, "CT normalisation needs its statistics");
      const float* p = norm + 4 * c;
      require(std::isfinite(p[0]) && std::isfinite(p[1]) && p[1] > 0.f && std::isfinite(p[2]) &&
                  std::isfinite(p[3]) && p[2] <= p[3],
              "CT statistics must be finite, std positive and the percentiles ordered");
      cn.mean[c] = p[0];
      cn.std[c] = std::max(p[1], 1e-8f);
      cn.lower[c] = p[2];
      cn.upper[c] = p[3];
    }
  }
  int64_t ms[3] = {0, 0, 0}, me[3] = {1, 1, 1};
  if (masked) {
    require(mask && mask_start && mask_extent, "masked z-score normalisation needs the mask");
    // every cropped voxel (raw axis transpose[k] from start[k]) must lie in the mask box
    for (int k = 0; k < 3; ++k) {
      const int a = transpose[k];
      require(mask_extent[a] >= 1 && start[k] >= mask_start[a] &&
                  start[k] + out_size[k] <= mask_start[a] + mask_extent[a],
              "crop window outside the mask box");
    }
    for (int a = 0; a < 3; ++a) {
      ms[a] = mask_start[a];
      me[a] = mask_extent[a];
    }
  }
  const int64_t total = out_size[0] * out_size[1] * out_size[2] * channels;
  ProfScope prof("preprocess_crop_normalize", 0.0, 8.0 * (double)total, st);
  hipLaunchKernelGGL(crop_normalize_kernel, dim3(blocks_for(total)), dim3(256), 0, st, x,
                     channels, size[0], size[1], size[2], transpose[0], transpose[1], transpose[2],
                     start[0], start[1], start[2], out_size[0], out_size[1], out_size[2], cn,
                     masked ? mask : nullptr, ms[0], ms[1], ms[2], me[1], me[2], out);
  launch_check("crop_normalize");
}

size_t resample_spline_workspace(const int64_t* size, const int64_t* new_size, int separate_axis) {
  const SplinePlan p = spline_plan(size, new_size, separate_axis);
  return (size_t)(p.a_elems + p.b_elems) * sizeof(double) + (size_t)p.mm_elems * sizeof(float2) +
         256;
}

void resample_spline(const float* x, int channels, const int64_t* size, const int64_t* new_size,
                     int order, int separate_axis, int order_z, void* work, size_t work_bytes,
                     float* out, hipStream_t st, bool round_half) {
  require(x && out && size && new_size, "resampling pointers must not be null");
  require(channels >= 1, "resampling needs at least one channel");
  for (int a = 0; a < 3; ++a)
    require(size[a] >= 1 && new_size[a] >= 1, "resampling shapes must be positive");
  require(order == 1 || order == 3, "device spline resampling supports orders 1 and 3");
  require(separate_axis >= -1 && separate_axis < 3, "separate axis must be -1, 0, 1 or 2");
  require(separate_axis < 0 || order_z == 0,
          "device separate-axis resampling supports order_z 0 (nearest)");
  const SplinePlan p = spline_plan(size, new_size, separate_axis);
  require(work && work_bytes >= resample_spline_workspace(size, new_size, separate_axis),
          "resampling workspace too small");
  double* A = static_cast<double*>(work);
  double* B = A + p.a_elems;
  float2* mm = reinterpret_cast<float2*>(B + p.b_elems);
  const int64_t in_vox = size[0] * size[1] * size[2];
  const int64_t out_vox = new_size[0] * new_size[1] * new_size[2];
  const double z = std::sqrt(3.0) - 2.0;
  const double gain = (1.0 - z) * (1.0 - 1.0 / z);
  const int mm_axis = separate_axis >= 0 ? separate_axis : 0;
  for (int c = 0; c < channels; ++c) {
    const float* xc = x + (int64_t)c * in_vox;
    const int64_t planes = size[mm_axis];
    float2* part = mm + planes + 1;
    {
      ProfScope prof("spline_minmax", 0.0, 4.0 * (double)in_vox, st);
      hipLaunchKernelGGL(plane_minmax_kernel, dim3((unsigned)planes, kMinmaxParts), dim3(256), 0,
                         st, xc, size[0], size[1], size[2], mm_axis, part);
      hipLaunchKernelGGL(plane_parts_kernel, dim3((unsigned)ceil_div(planes, 256)), dim3(256), 0,
                         st, part, planes, kMinmaxParts, mm);
      if (separate_axis < 0)
        hipLaunchKernelGGL(reduce_minmax_kernel, dim3(1), dim3(64), 0, st, mm, size[0]);
    }
    int64_t d[3] = {size[0] + 2 * p.pad[0], size[1] + 2 * p.pad[1], size[2] + 2 * p.pad[2]};
    {
      const int64_t padded = d[0] * d[1] * d[2];
      ProfScope prof("spline_pad", 0.0, 4.0 * (double)in_vox + 8.0 * (double)padded, st);
      hipLaunchKernelGGL(pad_edge_kernel, dim3(blocks_for(padded)), dim3(256), 0, st, xc, size[0],
                         size[1], size[2], p.pad[0], p.pad[1], p.pad[2], A);
    }
    if (order == 3) {
      for (int k = 0; k < p.naxes; ++k) {
        const int a = p.axes[k];
        const int64_t lines = d[0] * d[1] * d[2] / d[a];
        const double z_n = std::pow(z, (double)d[a]);
        // causal and anticausal sweeps: each reads and writes the array once
        ProfScope prof("spline_prefilter", 0.0, 32.0 * (double)(d[0] * d[1] * d[2]), st);
        if (a == 2)
          hipLaunchKernelGGL(prefilter_contig_kernel, dim3((unsigned)ceil_div(lines, 256)),
                             dim3(256), 0, st, A, lines, d[2], z, z_n, gain);
        else
          hipLaunchKernelGGL(prefilter_strided_kernel, dim3((unsigned)ceil_div(lines, 256)),
                             dim3(256), 0, st, A, d[0], d[1], d[2], a, z, z_n, gain);
      }
    }
    double* src = A;
    double* dst = B;
    for (int k = 0; k < p.naxes; ++k) {
      const int a = p.axes[k];
      int64_t od[3] = {d[0], d[1], d[2]};
      od[a] = new_size[a];
      const double ratio = (double)size[a] / (double)new_size[a];
      const int64_t total = od[0] * od[1] * od[2];
      ProfScope prof("spline_interp", 0.0, 8.0 * (double)(d[0] * d[1] * d[2] + total), st);
      if (order == 3)
        hipLaunchKernelGGL(interp_axis_kernel<3>, dim3(blocks_for(total)), dim3(256), 0, st, src,
                           d[0], d[1], d[2], a, new_size[a], ratio, p.pad[a], dst);
      else
        hipLaunchKernelGGL(interp_axis_kernel<1>, dim3(blocks_for(total)), dim3(256), 0, st, src,
                           d[0], d[1], d[2], a, new_size[a], ratio, p.pad[a], dst);
      d[a] = new_size[a];
      std::swap(src, dst);
    }
    float* oc = out + (int64_t)c * out_vox;
    ProfScope prof("spline_finish", 0.0, 8.0 * (double)(d[0] * d[1] * d[2]) + 4.0 * (double)out_vox,
                   st);
    if (separate_axis < 0) {
      auto kernel = round_half ? cast_clip_kernel<true> : cast_clip_kernel<false>;
      hipLaunchKernelGGL(kernel, dim3(blocks_for(out_vox)), dim3(256), 0, st, src, out_vox,
                         mm + size[0], oc);
    } else {
      const int a = separate_axis;
      auto kernel = round_half ? plane_clip_nearest_kernel<true> : plane_clip_nearest_kernel<false>;
      hipLaunchKernelGGL(kernel, dim3(blocks_for(out_vox)), dim3(256), 0, st, src, d[0], d[1],
                         d[2], a, new_size[a], (double)size[a] / (double)new_size[a], mm, oc);
    }
  }
  launch_check("resample_spline");
}

}  // namespace nnx
