// Torch-grid resampling (nnU-Net's resample_torch_fornnunet: torch interpolate with
// align_corners=False) of float32 or float16 volumes, one pass over three spatial axes
// with arbitrary element strides, so that channels-first images and channels-last logits
// are read and written in place.  A separate-axis resampling is two passes (the planes
// across the axis, then the axis), composed by the caller.
//
// Per axis (source size S, target size T, float32 scale = S / T):
//   scaled  = scale * float32(i + 0.5)     (i alone for mode "nearest"), float32;
//   nearest = min(int(scaled), S - 1)                               (nearest modes);
//   linear: c = max(scaled - 0.5, 0) in float32, lower = min(int(c), S - 1),
//           upper = min(lower + 1, S - 1), f = c - floor(c), weights (1 - f, f) exact in
//           float64.
// A linear output is the sum over the eight corners (axis 0 the high bit) of
// ((v * w0) * w1) * w2 in float64, in corner order, rounded once to float32 (the value
// the reference computes with compensated float32 pairs).  Coordinates use separate
// multiply and add (the library compiles with -ffp-contract=off).
//
// One kernel, torch_grid_kernel: a thread per output voxel at a time (axis 2 across the
// lanes) loops over the channels and writes every (channel, voxel) element, or, for the
// restoration, resamples every class and keeps the first maximum, writing uint16 labels and
// no float intermediate.
#include <algorithm>
#include <cmath>
#include <vector>

#include "nnx_internal.h"

namespace nnx {
namespace {

struct AxisGrid {
  int S, T;
  float scale;
};

struct TorchGridArgs {
  const void* in;
  float* out;              // resize: output elements
  uint16_t* labels;        // argmax: contiguous T0 x T1 x T2 labels
  int C;
  AxisGrid ax[3];
  int64_t in_stride[4];    // channel, axis 0, 1, 2 (elements)
  int64_t out_stride[4];
};

// Per-axis interpolation of one output index: source offsets (elements) of the lower and
// upper taps and their float64 weights (linear), or of the nearest tap.
struct AxisTap {
  int64_t lo, hi;
  double wlo, whi;
};

template <int MODE>
__device__ __forceinline__ AxisTap axis_tap(const AxisGrid& g, int i, int64_t stride) {
  const float shifted = (float)i + (MODE == 1 ? 0.f : 0.5f);
  const float scaled = __fmul_rn(g.scale, shifted);
  AxisTap t;
  if (MODE != 0) {
    t.lo = t.hi = (int64_t)min((int)scaled, g.S - 1) * stride;
    t.wlo = 1.0;
    t.whi = 0.0;
  } else {
    const float coordinate = fmaxf(__fsub_rn(scaled, 0.5f), 0.f);
    const int lo = min((int)coordinate, g.S - 1);
    const int hi = min(lo + 1, g.S - 1);
    const double f = (double)__fsub_rn(coordinate, floorf(coordinate));
    t.lo = (int64_t)lo * stride;
    t.hi = (int64_t)hi * stride;
    t.wlo = 1.0 - f;
    t.whi = f;
  }
  return t;
}

template <bool HALF>
__device__ __forceinline__ double load_value(const void* p, int64_t i) {
  if constexpr (HALF)
    return (double)(float)static_cast<const _Float16*>(p)[i];
  else
    return (double)static_cast<const float*>(p)[i];
}

// the float32 value of one output element of channel base `src`
template <int MODE, bool HALF>
__device__ __forceinline__ float sample(const void* in, int64_t src, const AxisTap (&t)[3]) {
  if (MODE != 0) return (float)load_value<HALF>(in, src + t[0].lo + t[1].lo + t[2].lo);
  double sum = 0.0;
#pragma unroll
  for (int corner = 0; corner < 8; ++corner) {
    const int s0 = (corner >> 2) & 1, s1 = (corner >> 1) & 1, s2 = corner & 1;
    const double v = load_value<HALF>(
        in, src + (s0 ? t[0].hi : t[0].lo) + (s1 ? t[1].hi : t[1].lo) + (s2 ? t[2].hi : t[2].lo));
    double term = __dmul_rn(v, s0 ? t[0].whi : t[0].wlo);
    term = __dmul_rn(term, s1 ? t[1].whi : t[1].wlo);
    term = __dmul_rn(term, s2 ? t[2].whi : t[2].wlo);
    sum = __dadd_rn(sum, term);
  }
  return (float)sum;
}

// Workgroup = kLanes positions along axis 2 x kRows rows of axis 1 (grid x over runs of
// axis 2); rows and planes past the grid loop by its stride.  A linear launch has a
// workgroup per 256 positions of every row (one voxel a thread: its eight-tap loads need
// many waves in flight); a nearest one has 64 x 4 workgroups, about 16 per CU, looping over
// rows (one load a voxel, so workgroup launches would dominate).  A thread computes its
// voxel's taps once and loops over the channels: every channel of a resize (neighbouring
// lanes write neighbouring axis-2 positions of one channel), or every class of an argmax
// (strict `>`: the first maximum wins ties).
template <int MODE>
struct GridShape {
  static constexpr int kLanes = MODE == 0 ? 256 : 64, kRows = MODE == 0 ? 1 : 4;
};

template <int MODE, bool HALF, bool ARGMAX>
__global__ __launch_bounds__(256) void torch_grid_kernel(TorchGridArgs a) {
  constexpr int kLanes = GridShape<MODE>::kLanes, kRows = GridShape<MODE>::kRows;
  const int i2 = blockIdx.x * kLanes + threadIdx.x;
  if (i2 >= a.ax[2].T) return;
  AxisTap t[3];
  t[2] = axis_tap<MODE>(a.ax[2], i2, a.in_stride[3]);
  for (int i0 = blockIdx.z; i0 < a.ax[0].T; i0 += gridDim.z) {
    t[0] = axis_tap<MODE>(a.ax[0], i0, a.in_stride[1]);
    for (int i1 = blockIdx.y * kRows + threadIdx.y; i1 < a.ax[1].T; i1 += gridDim.y * kRows) {
      t[1] = axis_tap<MODE>(a.ax[1], i1, a.in_stride[2]);
      if constexpr (ARGMAX) {
        float best = sample<MODE, HALF>(a.in, 0, t);
        int label = 0;
        for (int k = 1; k < a.C; ++k) {
          const float value = sample<MODE, HALF>(a.in, (int64_t)k * a.in_stride[0], t);
          if (value > best) {
            best = value;
            label = k;
          }
        }
        a.labels[((int64_t)i0 * a.ax[1].T + i1) * a.ax[2].T + i2] = (uint16_t)label;
      } else {
        float* dst = a.out + i0 * a.out_stride[1] + i1 * a.out_stride[2] + i2 * a.out_stride[3];
        for (int c = 0; c < a.C; ++c)
          dst[c * a.out_stride[0]] = sample<MODE, HALF>(a.in, (int64_t)c * a.in_stride[0], t);
      }
    }
  }
}

TorchGridArgs make_args(const void* in, int channels, const int* in_size,
                        const int64_t* in_strides, const int* out_size, int mode, bool argmax) {
  require(in && in_size && out_size && in_strides, "Torch-grid resampling pointers must not be null");
  require(channels >= 1 && (!argmax || channels <= 65536),
          argmax ? "Torch-grid restoration needs 1..65536 classes"
                 : "Torch-grid resampling needs at least one channel");
  require(mode >= 0 && mode <= 2,
          "Torch-grid mode must be 0 (linear), 1 (nearest) or 2 (nearest-exact)");
  TorchGridArgs a{};
  a.in = in;
  a.C = channels;
  int64_t voxels = 1;
  for (int d = 0; d < 3; ++d) {
    require(in_size[d] >= 1 && out_size[d] >= 1, "Torch-grid sizes must be positive");
    a.ax[d].S = in_size[d];
    a.ax[d].T = out_size[d];
    a.ax[d].scale = (float)((double)in_size[d] / (double)out_size[d]);
    voxels *= out_size[d];
  }
  for (int d = 0; d < 4; ++d) {
    require(in_strides[d] >= 0, "Torch-grid strides must be non-negative");
    a.in_stride[d] = in_strides[d];
  }
  const int64_t n = argmax ? voxels : voxels * channels;
  require(n < ((int64_t)1 << 31), "Torch-grid output exceeds 2^31 elements");
  return a;
}

template <bool ARGMAX, int MODE, bool HALF>
void launch_mode(const TorchGridArgs& a, hipStream_t st) {
  constexpr int kLanes = GridShape<MODE>::kLanes, kRows = GridShape<MODE>::kRows;
  const int64_t runs = ceil_div(a.ax[2].T, kLanes);
  const int64_t planes = std::min(a.ax[0].T, 65535);
  const int64_t row_groups = ceil_div(a.ax[1].T, kRows);
  const int64_t per_plane =
      MODE == 0 ? row_groups
                : std::max<int64_t>(1, std::min(row_groups, ceil_div(4096, planes * runs)));
  const dim3 grid((unsigned)runs, (unsigned)std::min<int64_t>(per_plane, 65535), (unsigned)planes);
  hipLaunchKernelGGL((torch_grid_kernel<MODE, HALF, ARGMAX>), grid, dim3(kLanes, kRows), 0, st, a);
}

template <bool ARGMAX>
void launch(const TorchGridArgs& a, bool half, int mode, hipStream_t st) {
  if (mode == 0)
    half ? launch_mode<ARGMAX, 0, true>(a, st) : launch_mode<ARGMAX, 0, false>(a, st);
  else if (mode == 1)
    half ? launch_mode<ARGMAX, 1, true>(a, st) : launch_mode<ARGMAX, 1, false>(a, st);
  else
    half ? launch_mode<ARGMAX, 2, true>(a, st) : launch_mode<ARGMAX, 2, false>(a, st);
}

// Source voxels the grid reads: per axis the distinct indices its taps touch (every index
// for a linear upsample, a subset for downsampling and the nearest modes), computed with
// the kernel's float32 coordinate arithmetic.
double touched_source_voxels(const TorchGridArgs& a, int mode) {
  double voxels = 1.0;
  for (int d = 0; d < 3; ++d) {
    const int S = a.ax[d].S, T = a.ax[d].T;
    std::vector<char> hit(S, 0);
    for (int i = 0; i < T; ++i) {
      const float scaled = a.ax[d].scale * ((float)i + (mode == 1 ? 0.f : 0.5f));
      if (mode != 0) {
        hit[std::min((int)scaled, S - 1)] = 1;
      } else {
        const float coordinate = std::max(scaled - 0.5f, 0.f);
        const int lo = std::min((int)coordinate, S - 1);
        hit[lo] = 1;
        if (coordinate != std::floor(coordinate)) hit[std::min(lo + 1, S - 1)] = 1;
      }
    }
    int count = 0;
    for (char h : hit) count += h;
    voxels *= count;
  }
  return voxels;
}

}  // namespace

void torch_resize(const void* in, bool half, int channels, const int* in_size,
                  const int64_t* in_strides, float* out, const int* out_size,
                  const int64_t* out_strides, int mode, hipStream_t st) {
  TorchGridArgs a = make_args(in, channels, in_size, in_strides, out_size, mode, false);
  require(out && out_strides, "Torch-grid resampling pointers must not be null");
  for (int d = 0; d < 4; ++d) {
    require(out_strides[d] >= 0, "Torch-grid strides must be non-negative");
    a.out_stride[d] = out_strides[d];
  }
  a.out = out;
  // algorithmic bytes: every source element a tap touches read once, every output
  // element written once
  const double src_elems = (double)channels * touched_source_voxels(a, mode);
  const double out_elems = (double)channels * out_size[0] * out_size[1] * out_size[2];
  ProfScope prof(half ? "torch_resize_f16" : "torch_resize", 0.0,
                 (half ? 2.0 : 4.0) * src_elems + 4.0 * out_elems, st);
  launch<false>(a, half, mode, st);
  launch_check("torch_resize");
}

void torch_resize_argmax(const void* in, bool half, int classes, const int* in_size,
                         const int64_t* in_strides, const int* out_size, int mode,
                         uint16_t* labels, hipStream_t st) {
  TorchGridArgs a = make_args(in, classes, in_size, in_strides, out_size, mode, true);
  require(labels != nullptr, "Torch-grid restoration pointers must not be null");
  a.labels = labels;
  const double src_elems = (double)classes * touched_source_voxels(a, mode);
  const double voxels = (double)out_size[0] * out_size[1] * out_size[2];
  ProfScope prof(half ? "torch_argmax_f16" : "torch_argmax", 0.0,
                 (half ? 2.0 : 4.0) * src_elems + 2.0 * voxels, st);
  launch<true>(a, half, mode, st);
  launch_check("torch_resize_argmax");
}

}  // namespace nnx
