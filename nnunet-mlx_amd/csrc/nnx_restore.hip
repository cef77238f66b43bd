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

#include <algorithm>
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

// out[v] = class c of channels-last logits (n voxels, `classes` per voxel) as float32
template <bool HALF>
__global__ __launch_bounds__(256) void extract_class_kernel(const void* __restrict__ logits,
                                                            int classes, int c, int64_t n,
                                                            float* __restrict__ out) {
  for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < n;
       v += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = v * classes + c;
    if constexpr (HALF) out[v] = __half2float(static_cast<const __half*>(logits)[i]);
    else out[v] = static_cast<const float*>(logits)[i];
  }
}

// running first-maximum argmax: class 0 initialises, later classes win only when strictly
// greater (ties keep the earliest class)
__global__ __launch_bounds__(256) void argmax_update_kernel(const float* __restrict__ value,
                                                            int64_t n, int c,
                                                            float* __restrict__ best,
                                                            uint16_t* __restrict__ labels) {
  for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < n;
       v += (int64_t)gridDim.x * blockDim.x) {
    const float x = value[v];
    if (c == 0) {
      best[v] = x;
      labels[v] = 0;
    } else if (x > best[v]) {
      best[v] = x;
      labels[v] = (uint16_t)c;
    }
  }
}

int grid_for(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), 1 << 20)); }

int64_t align256(int64_t bytes) { return ceil_div(bytes, 256) * 256; }

}  // namespace

size_t restore_labels_spline_workspace(const int* src, const int* dst, int separate_axis) {
  const int64_t s[3] = {src[0], src[1], src[2]}, d[3] = {dst[0], dst[1], dst[2]};
  const int64_t n_src = s[0] * s[1] * s[2], n_dst = d[0] * d[1] * d[2];
  return (size_t)(align256(4 * n_src) + 2 * align256(4 * n_dst)) +
         resample_spline_workspace(s, d, separate_axis);
}

void restore_labels_spline(const void* logits, bool half, int classes, const int* src,
                           const int* dst, int order, int separate_axis, void* work,
                           size_t work_bytes, uint16_t* labels, hipStream_t st) {
  require(logits && labels && src && dst && work, "restoration pointers must not be null");
  require(classes >= 1 && classes <= 65536, "restoration supports 1..65536 classes");
  for (int i = 0; i < 3; ++i)
    require(src[i] >= 1 && dst[i] >= 1, "restoration shapes must be positive");
  require(separate_axis >= -1 && separate_axis < 3, "separate axis must be -1, 0, 1 or 2");
  require(work_bytes >= restore_labels_spline_workspace(src, dst, separate_axis),
          "restoration workspace too small");
  const int64_t s[3] = {src[0], src[1], src[2]}, d[3] = {dst[0], dst[1], dst[2]};
  const int64_t n_src = s[0] * s[1] * s[2], n_dst = d[0] * d[1] * d[2];
  char* base = static_cast<char*>(work);
  float* channel = reinterpret_cast<float*>(base);
  float* value = reinterpret_cast<float*>(base + align256(4 * n_src));
  float* best = reinterpret_cast<float*>(base + align256(4 * n_src) + align256(4 * n_dst));
  void* spline_work = base + align256(4 * n_src) + 2 * align256(4 * n_dst);
  const size_t spline_bytes = work_bytes - (size_t)(align256(4 * n_src) + 2 * align256(4 * n_dst));
  for (int c = 0; c < classes; ++c) {
    {
      ProfScope prof("restore_extract", 0.0, (half ? 2.0 : 4.0) * classes * n_src + 4.0 * n_src, st);
      if (half)
        hipLaunchKernelGGL(extract_class_kernel<true>, dim3(grid_for(n_src)), dim3(256), 0, st,
                           logits, classes, c, n_src, channel);
      else
        hipLaunchKernelGGL(extract_class_kernel<false>, dim3(grid_for(n_src)), dim3(256), 0, st,
                           logits, classes, c, n_src, channel);
    }
    resample_spline(channel, 1, s, d, order, separate_axis, 0, spline_work, spline_bytes, value,
                    st, half);
    ProfScope prof("restore_argmax_update", 0.0, 4.0 * n_dst + (c ? 8.0 : 6.0) * n_dst, st);
    hipLaunchKernelGGL(argmax_update_kernel, dim3(grid_for(n_dst)), dim3(256), 0, st, value,
                       n_dst, c, best, labels);
  }
  launch_check("restore_labels_spline");
}

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
