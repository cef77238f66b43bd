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
// Two kernels: torch_resize_kernel writes every (channel, voxel) element (one thread per
// element, output axis 2 fastest, so neighbouring lanes read neighbouring source voxels);
// torch_argmax_kernel resamples every class of one output voxel and keeps the first
// maximum (the restoration's argmax), writing uint16 labels and no float intermediate.
#include "nnx_internal.h"

namespace nnx {
namespace {

struct AxisGrid {
  int S, T;
  float scale;
};

struct TorchGridArgs {
  const void* in;
  float* out;              // torch_resize_kernel
  uint16_t* labels;        // torch_argmax_kernel (contiguous T0 x T1 x T2)
  int C;
  AxisGrid ax[3];
  int64_t in_stride[4];    // channel, axis 0, 1, 2 (elements)
  int64_t out_stride[4];
  unsigned T12, T012;      // T1 * T2, T0 * T1 * T2
  unsigned n;              // elements (resize) or voxels (argmax) to write, < 2^31
};

struct Stencil {
  int64_t off[2][3];       // source offsets (elements) of lower/upper (linear) per axis
  double w[2][3];          // weights of lower/upper per axis
  int64_t nearest;         // source offset of the nearest sample (nearest modes)
};

template <bool HALF>
__device__ __forceinline__ double load_value(const void* p, int64_t i) {
  if constexpr (HALF)
    return (double)(float)static_cast<const _Float16*>(p)[i];
  else
    return (double)static_cast<const float*>(p)[i];
}

template <int MODE>
__device__ __forceinline__ Stencil stencil(const TorchGridArgs& a, const unsigned (&pos)[3]) {
  Stencil s;
  s.nearest = 0;
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const float shifted = (float)pos[d] + (MODE == 1 ? 0.f : 0.5f);
    const float scaled = __fmul_rn(a.ax[d].scale, shifted);
    const int64_t stride = a.in_stride[1 + d];
    if (MODE != 0) {
      s.nearest += (int64_t)min((int)scaled, a.ax[d].S - 1) * stride;
    } else {
      const float coordinate = fmaxf(__fsub_rn(scaled, 0.5f), 0.f);
      const int lo = min((int)coordinate, a.ax[d].S - 1);
      const int hi = min(lo + 1, a.ax[d].S - 1);
      const double f = (double)__fsub_rn(coordinate, floorf(coordinate));
      s.off[0][d] = (int64_t)lo * stride;
      s.off[1][d] = (int64_t)hi * stride;
      s.w[0][d] = 1.0 - f;
      s.w[1][d] = f;
    }
  }
  return s;
}

// the float32 value of one output element of channel base `src`
template <int MODE, bool HALF>
__device__ __forceinline__ float sample(const void* in, int64_t src, const Stencil& s) {
  if (MODE != 0) return (float)load_value<HALF>(in, src + s.nearest);
  double sum = 0.0;
#pragma unroll
  for (int corner = 0; corner < 8; ++corner) {
    const int s0 = (corner >> 2) & 1, s1 = (corner >> 1) & 1, s2 = corner & 1;
    const double v = load_value<HALF>(in, src + s.off[s0][0] + s.off[s1][1] + s.off[s2][2]);
    double term = __dmul_rn(v, s.w[s0][0]);
    term = __dmul_rn(term, s.w[s1][1]);
    term = __dmul_rn(term, s.w[s2][2]);
    sum = __dadd_rn(sum, term);
  }
  return (float)sum;
}

__device__ __forceinline__ void position(const TorchGridArgs& a, unsigned r, unsigned (&pos)[3]) {
  const unsigned T2 = (unsigned)a.ax[2].T;
  pos[0] = r / a.T12;
  const unsigned rest = r - pos[0] * a.T12;
  pos[1] = rest / T2;
  pos[2] = rest - pos[1] * T2;
}

template <int MODE, bool HALF>
__global__ __launch_bounds__(256) void torch_resize_kernel(TorchGridArgs a) {
  for (unsigned e = blockIdx.x * blockDim.x + threadIdx.x; e < a.n; e += gridDim.x * blockDim.x) {
    const unsigned c = e / a.T012;
    unsigned pos[3];
    position(a, e - c * a.T012, pos);
    const Stencil s = stencil<MODE>(a, pos);
    const float value = sample<MODE, HALF>(a.in, (int64_t)c * a.in_stride[0], s);
    a.out[(int64_t)c * a.out_stride[0] + pos[0] * a.out_stride[1] + pos[1] * a.out_stride[2] +
          pos[2] * a.out_stride[3]] = value;
  }
}

template <int MODE, bool HALF>
__global__ __launch_bounds__(256) void torch_argmax_kernel(TorchGridArgs a) {
  for (unsigned e = blockIdx.x * blockDim.x + threadIdx.x; e < a.n; e += gridDim.x * blockDim.x) {
    unsigned pos[3];
    position(a, e, pos);
    const Stencil s = stencil<MODE>(a, pos);
    float best = sample<MODE, HALF>(a.in, 0, s);
    int label = 0;
    for (int k = 1; k < a.C; ++k) {
      const float value = sample<MODE, HALF>(a.in, (int64_t)k * a.in_stride[0], s);
      if (value > best) {  // first maximum wins ties
        best = value;
        label = k;
      }
    }
    a.labels[e] = (uint16_t)label;
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
  a.T12 = (unsigned)((int64_t)out_size[1] * out_size[2]);
  a.T012 = (unsigned)voxels;
  a.n = (unsigned)n;
  return a;
}

unsigned grid_of(unsigned n) { return (unsigned)std::min<int64_t>(ceil_div(n, 256), 1 << 16); }

template <bool ARGMAX, int MODE, bool HALF>
void launch_mode(const TorchGridArgs& a, hipStream_t st) {
  if constexpr (ARGMAX)
    hipLaunchKernelGGL((torch_argmax_kernel<MODE, HALF>), dim3(grid_of(a.n)), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((torch_resize_kernel<MODE, HALF>), dim3(grid_of(a.n)), dim3(256), 0, st, a);
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
  // algorithmic bytes: every source element read once, every output element written once
  const double src_elems = (double)channels * in_size[0] * in_size[1] * in_size[2];
  ProfScope prof(half ? "torch_resize_f16" : "torch_resize", 0.0,
                 (half ? 2.0 : 4.0) * src_elems + 4.0 * (double)a.n, st);
  launch<false>(a, half, mode, st);
  launch_check("torch_resize");
}

void torch_resize_argmax(const void* in, bool half, int classes, const int* in_size,
                         const int64_t* in_strides, const int* out_size, int mode,
                         uint16_t* labels, hipStream_t st) {
  TorchGridArgs a = make_args(in, classes, in_size, in_strides, out_size, mode, true);
  require(labels != nullptr, "Torch-grid restoration pointers must not be null");
  a.labels = labels;
  const double src_elems = (double)classes * in_size[0] * in_size[1] * in_size[2];
  ProfScope prof(half ? "torch_argmax_f16" : "torch_argmax", 0.0,
                 (half ? 2.0 : 4.0) * src_elems + 2.0 * (double)a.n, st);
  launch<true>(a, half, mode, st);
  launch_check("torch_resize_argmax");
}

}  // namespace nnx
