// Fused class-logit restoration: half-pixel trilinear resampling (edge-clamped) of
// channels-last logits to the original grid, in float64, and the first-maximum argmax.
//
// Replaces the reference's fused Metal restoration
// (src/nnunet_mlx/kernels/metal_restore.py:69-137 kernel, :401-427 launch, :464-489 axis
// metadata).  The reference emulates float64 with double-single arithmetic because the
// host resampler it must agree with interpolates in float64; gfx950 has native float64,
// so every coordinate, weight, product and sum here is an IEEE float64 operation in the
// same order as the oracle's numpy restatement (no contraction: -ffp-contract=off).
//
// One thread per output voxel (grid-stride).  Per axis: c = (i + 0.5) * (S / T) - 0.5
// clipped to [0, S - 1], lower = floor(c), upper = min(lower + 1, S - 1), weights
// 1 - (c - lower) and c - lower.  Per class: the eight corners in the order
// 000, 001, 010, 011, 100, 101, 110, 111 (z, y, x bits), each term ((v * w_z) * w_y) * w_x,
// summed left to right from 0; the sum rounded to float32 (or to float16, nearest even,
// for float16 logits) is compared with strict ">" so ties keep the earliest class.
// Roofline: HBM — reads the source logits (8 corners per voxel, reused through the
// caches) and writes 2 bytes per output voxel; float64 VALU work ~(24 + 32 K) operations
// per output voxel.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "nnx_internal.h"

namespace nnx {
namespace {

struct AxisCoord {
  int lo, hi;
  double wlo, whi;
};

__device__ __forceinline__ AxisCoord axis_coord(int i, double ratio, int source) {
  double c = ((double)i + 0.5) * ratio - 0.5;
  c = fmin(fmax(c, 0.0), (double)(source - 1));
  AxisCoord a;
  a.lo = (int)floor(c);
  a.hi = a.lo + 1 < source ? a.lo + 1 : source - 1;
  a.whi = c - (double)a.lo;
  a.wlo = 1.0 - a.whi;
  return a;
}

template <bool HALF>
__device__ __forceinline__ double load_logit(const void* logits, int64_t i) {
  if constexpr (HALF)
    return (double)static_cast<const _Float16*>(logits)[i];
  else
    return (double)static_cast<const float*>(logits)[i];
}

template <bool HALF>
__global__ __launch_bounds__(256) void restore_argmax_kernel(const void* __restrict__ logits,
                                                             int classes, int sz, int sy, int sx,
                                                             int tz, int ty, int tx, double rz,
                                                             double ry, double rx,
                                                             uint16_t* __restrict__ labels) {
  const int64_t total = (int64_t)tz * ty * tx;
  const int64_t plane = (int64_t)sy * sx;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int x = (int)(e % tx);
    const int64_t rest = e / tx;
    const int y = (int)(rest % ty);
    const int z = (int)(rest / ty);
    const AxisCoord cz = axis_coord(z, rz, sz);
    const AxisCoord cy = axis_coord(y, ry, sy);
    const AxisCoord cx = axis_coord(x, rx, sx);
    const int zs[2] = {cz.lo, cz.hi}, ys[2] = {cy.lo, cy.hi}, xs[2] = {cx.lo, cx.hi};
    const double wz[2] = {cz.wlo, cz.whi}, wy[2] = {cy.wlo, cy.whi}, wx[2] = {cx.wlo, cx.whi};
    int64_t base[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
      base[c] = ((int64_t)zs[c >> 2] * plane + (int64_t)ys[(c >> 1) & 1] * sx + xs[c & 1]) * classes;
    float best = -INFINITY;
    int label = 0;
    for (int k = 0; k < classes; ++k) {
      double sum = 0.0;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const double v = load_logit<HALF>(logits, base[c] + k);
        sum = sum + ((v * wz[c >> 2]) * wy[(c >> 1) & 1]) * wx[c & 1];
      }
      const float value = HALF ? (float)(_Float16)sum : (float)sum;
      if (value > best) {
        best = value;
        label = k;
      }
    }
    labels[e] = (uint16_t)label;
  }
}

}  // namespace

void restore_labels(const void* logits, bool half, int classes, const int* src, const int* dst,
                    uint16_t* labels, hipStream_t st) {
  require(logits && labels && src && dst, "restoration pointers must not be null");
  require(classes >= 1 && classes <= 65536, "restoration supports 1..65536 classes");
  for (int i = 0; i < 3; ++i)
    require(src[i] >= 1 && dst[i] >= 1, "restoration shapes must be positive");
  const int64_t total = (int64_t)dst[0] * dst[1] * dst[2];
  const double rz = (double)src[0] / dst[0], ry = (double)src[1] / dst[1],
               rx = (double)src[2] / dst[2];
  const int64_t in_bytes = (int64_t)src[0] * src[1] * src[2] * classes * (half ? 2 : 4);
  ProfScope prof("restore_argmax", 0.0, (double)in_bytes + 2.0 * (double)total, st);
  const int blocks = (int)std::min<int64_t>(ceil_div(total, 256), 1 << 20);
  if (half)
    hipLaunchKernelGGL(restore_argmax_kernel<true>, dim3(blocks), dim3(256), 0, st, logits,
                       classes, src[0], src[1], src[2], dst[0], dst[1], dst[2], rz, ry, rx,
                       labels);
  else
    hipLaunchKernelGGL(restore_argmax_kernel<false>, dim3(blocks), dim3(256), 0, st, logits,
                       classes, src[0], src[1], src[2], dst[0], dst[1], dst[2], rz, ry, rx,
                       labels);
  launch_check("restore_labels");
}

}  // namespace nnx
