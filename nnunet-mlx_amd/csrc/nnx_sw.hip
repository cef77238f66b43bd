// GPU-resident sliding-window kernels.  All arithmetic is float32 (or IEEE half where
// the nnU-Net fp16 accumulation mode asks for it) with explicitly separate multiply and
// add, so the per-voxel results equal the reference's numpy/MLX sequence bit for bit
// given identical network outputs:
//   mirror average  p = ((view0 + view1') + view2') + ... ; p = p / nviews
//   float32 mode    acc = acc + p*g            norm = norm + g
//   fp16 mode       acc = f16(f32(acc) + p*f32(g))   norm = f16(norm + g)
//   finalize        q = f32(acc) / f32(norm) -> accumulation dtype; folds summed in that
//                   dtype; average = dtype(f32(total) / f32(nfolds)); argmax with the
//                   earliest channel winning ties, 65535 for non-finite scores.
#include "nnx_internal.h"

namespace nnx {
namespace {

struct Flips {
  int f[8];
};

__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

// Workgroups of one or more patch rows (y along threadIdx.y, z = blockIdx.y), threads along
// the row: every view's flipped source row is uniform over a row's threads, only x flips per
// lane.  Reads the source voxel of each channel (zero outside the volume) and writes the
// channels-last row of every view.  A thread takes a run of V consecutive (x, channel)
// elements of the row; with V = 4 (row length a multiple of 4 floats and a 16-byte aligned
// output: checked by the host) each view takes one 16-byte store.
template <int V>
__global__ __launch_bounds__(512) void gather_flip_kernel(
    const float* __restrict__ vol, int C, int64_t Z, int64_t Y, int64_t X, int pz, int py, int px,
    int oz, int oy, int ox, int PZ, int PY, int PX, Flips flips, int nviews,
    float* __restrict__ out) {
  typedef float run_t __attribute__((ext_vector_type(V)));
  const int y = blockIdx.x * blockDim.y + threadIdx.y, z = blockIdx.y;
  if (y >= PY) return;
  const int64_t pvox = (int64_t)PZ * PY * PX;
  const int64_t zyx = Z * Y * X;
  const int64_t prow = ((int64_t)z * PY + y) * PX;
  const int n = PX * C;
  for (int e0 = V * threadIdx.x; e0 < n; e0 += V * blockDim.x) {
    // every view's values first (loads in flight together), then the stores
    run_t val[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
#pragma unroll
      for (int i = 0; i < V; ++i) val[v][i] = 0.f;
      if (v < nviews) {
        const int f = flips.f[v];
        const int64_t gz = (int64_t)oz + ((f & 1) ? PZ - 1 - z : z) - pz;
        const int64_t gy = (int64_t)oy + ((f & 2) ? PY - 1 - y : y) - py;
        if (gz >= 0 && gz < Z && gy >= 0 && gy < Y) {
          const float* src = vol + (gz * Y + gy) * X;
#pragma unroll
          for (int i = 0; i < V; ++i) {
            const int e = e0 + i, x = e / C, c = e - x * C;
            const int64_t gx = (int64_t)ox + ((f & 4) ? PX - 1 - x : x) - px;
            if (gx >= 0 && gx < X) val[v][i] = src[(int64_t)c * zyx + gx];
          }
        }
      }
    }
#pragma unroll
    for (int v = 0; v < 8; ++v)
      if (v < nviews) *reinterpret_cast<run_t*>(out + ((int64_t)v * pvox + prow) * C + e0) = val[v];
  }
}

// Workgroups of one or more patch rows (y along threadIdx.y, z = blockIdx.y), threads along
// the row's (x, class) pairs: each view's flipped source row is uniform over a row's
// threads, consecutive lanes read
// consecutive floats of the prediction rows and update consecutive accumulator elements
// (whole cache lines); the class-0 lane of a voxel updates its normaliser.
template <bool kHalf>
__global__ __launch_bounds__(512) void accumulate_kernel(
    const float* __restrict__ pred, int nviews, Flips flips, int K, int PZ, int PY, int PX,
    const void* __restrict__ gaussian, int oz, int oy, int ox, int64_t QY, int64_t QX,
    void* __restrict__ acc, void* __restrict__ norm) {
  const int y = blockIdx.x * blockDim.y + threadIdx.y, z = blockIdx.y;
  if (y >= PY) return;
  const int64_t pvox = (int64_t)PZ * PY * PX;
  const int64_t prow = ((int64_t)z * PY + y) * PX;
  const int64_t qrow = (((int64_t)oz + z) * QY + (oy + y)) * QX + ox;
  const float count = (float)nviews;
  const int n = PX * K;
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const int x = e / K;
    const int k = e - x * K;
    // every view's value first (loads in flight together), then the sum in view order
    float t[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      t[v] = 0.f;
      if (v < nviews) {
        const int f = flips.f[v];
        const int64_t srow =
            ((int64_t)((f & 1) ? PZ - 1 - z : z) * PY + ((f & 2) ? PY - 1 - y : y)) * PX;
        const int sx = (f & 4) ? PX - 1 - x : x;
        t[v] = pred[((int64_t)v * pvox + srow + sx) * K + k];
      }
    }
    // the Gaussian weight and the accumulator's (and normaliser's) old values are requested
    // with the predictions, so the read-modify-write waits for one round of loads
    const int64_t dst = qrow + x;
    float g, a_old, n_old = 0.f;
    if constexpr (kHalf) {
      g = __half2float(reinterpret_cast<const __half*>(gaussian)[prow + x]);
      a_old = __half2float(reinterpret_cast<const __half*>(acc)[dst * K + k]);
      if (k == 0) n_old = __half2float(reinterpret_cast<const __half*>(norm)[dst]);
    } else {
      g = reinterpret_cast<const float*>(gaussian)[prow + x];
      a_old = reinterpret_cast<const float*>(acc)[dst * K + k];
      if (k == 0) n_old = reinterpret_cast<const float*>(norm)[dst];
    }
    float s = t[0];
#pragma unroll
    for (int v = 1; v < 8; ++v)
      if (v < nviews) s = add_rn(s, t[v]);
    if (nviews > 1) s = __fdiv_rn(s, count);
    const float w = mul_rn(s, g);
    if constexpr (kHalf) {
      reinterpret_cast<__half*>(acc)[dst * K + k] = __float2half_rn(add_rn(a_old, w));
      if (k == 0) reinterpret_cast<__half*>(norm)[dst] = __float2half_rn(add_rn(n_old, g));
    } else {
      reinterpret_cast<float*>(acc)[dst * K + k] = add_rn(a_old, w);
      if (k == 0) reinterpret_cast<float*>(norm)[dst] = add_rn(n_old, g);
    }
  }
}

template <bool kHalf>
__global__ __launch_bounds__(256) void fold_add_kernel(const void* __restrict__ acc,
                                                       const void* __restrict__ norm, int K,
                                                       int64_t QY, int64_t QX, int cz, int cy,
                                                       int cx, int64_t CZ, int64_t CY,
                                                       int64_t CX, int first,
                                                       void* __restrict__ total) {
  const int64_t n = CZ * CY * CX;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t x = i % CX;
    const int64_t y = (i / CX) % CY;
    const int64_t z = i / (CX * CY);
    const int64_t src = ((cz + z) * QY + (cy + y)) * QX + (cx + x);
    float den;
    if constexpr (kHalf)
      den = __half2float(reinterpret_cast<const __half*>(norm)[src]);
    else
      den = reinterpret_cast<const float*>(norm)[src];
    for (int k = 0; k < K; ++k) {
      float num;
      if constexpr (kHalf)
        num = __half2float(reinterpret_cast<const __half*>(acc)[src * K + k]);
      else
        num = reinterpret_cast<const float*>(acc)[src * K + k];
      const float q = __fdiv_rn(num, den);
      if constexpr (kHalf) {
        __half* t = reinterpret_cast<__half*>(total) + i * K + k;
        const __half qh = __float2half_rn(q);
        *t = first ? qh : __float2half_rn(add_rn(__half2float(*t), __half2float(qh)));
      } else {
        float* t = reinterpret_cast<float*>(total) + i * K + k;
        *t = first ? q : add_rn(*t, q);
      }
    }
  }
}

template <bool kHalf>
__global__ __launch_bounds__(256) void fold_finalize_kernel(const void* __restrict__ total, int K,
                                                            int64_t n, int nfolds,
                                                            void* __restrict__ logits,
                                                            uint16_t* __restrict__ labels,
                                                            unsigned int* invalid_count) {
  __shared__ unsigned int block_invalid;
  if (threadIdx.x == 0) block_invalid = 0;
  __syncthreads();
  unsigned int local_invalid = 0;
  const float fn = (float)nfolds;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float best = -INFINITY;
    unsigned int winner = 0xffffffffu;
    bool invalid = false;
    for (int k = 0; k < K; ++k) {
      float v;
      if constexpr (kHalf) {
        __half h = reinterpret_cast<const __half*>(total)[i * K + k];
        if (nfolds > 1) h = __float2half_rn(__fdiv_rn(__half2float(h), fn));
        if (logits) reinterpret_cast<__half*>(logits)[i * K + k] = h;
        v = __half2float(h);
      } else {
        v = reinterpret_cast<const float*>(total)[i * K + k];
        if (nfolds > 1) v = __fdiv_rn(v, fn);
        if (logits) reinterpret_cast<float*>(logits)[i * K + k] = v;
      }
      invalid |= !isfinite(v);
      if (v > best) {
        best = v;
        winner = (unsigned int)k;
      }
    }
    if (labels) labels[i] = invalid ? (uint16_t)65535 : (uint16_t)winner;
    local_invalid += invalid ? 1u : 0u;
  }
  if (local_invalid) atomicAdd(&block_invalid, local_invalid);
  __syncthreads();
  if (threadIdx.x == 0 && block_invalid && invalid_count) atomicAdd(invalid_count, block_invalid);
}

// Threads along a row: the row's elements rounded up to whole multiples of `unit` (a wave,
// or half a wave where two short rows share one), at most `cap`; and rows a workgroup
// (along y): up to 512 threads in all, so that short rows do not make a workgroup per row.
unsigned row_threads(int64_t n, int64_t cap = 512, int64_t unit = 64) {
  return (unsigned)std::min<int64_t>(cap, std::max<int64_t>(unit, ceil_div(n, unit) * unit));
}
unsigned rows_per_group(unsigned lanes) { return std::max(1u, std::min(16u, 512u / lanes)); }
constexpr int64_t kAccLanes = 128;  // accumulate: lanes along a row

unsigned grid_for(int64_t n) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), 65536)); }

Flips make_flips(const int* flips, int nviews) {
  require(nviews >= 1 && nviews <= 8, "between 1 and 8 mirrored views are supported");
  Flips f{};
  for (int v = 0; v < nviews; ++v) {
    require(flips[v] >= 0 && flips[v] < 8, "view flip masks must be in [0, 8)");
    f.f[v] = flips[v];
  }
  return f;
}

}  // namespace

void sw_gather_flip(const float* vol, int channels, const int64_t* size, const int* pad_before,
                    const int* offset, const int* patch, const int* flips, int nviews,
                    float* out, hipStream_t st) {
  require(vol && out, "gather pointers must not be null");
  require(channels >= 1, "gather needs at least one channel");
  const Flips f = make_flips(flips, nviews);
  require(patch[1] <= 65535 && patch[0] <= 65535, "patch rows exceed the launch grid");
  const double pvox = (double)patch[0] * patch[1] * patch[2];
  ProfScope prof("sw_gather_flip", 0.0, 4.0 * pvox * channels * (1 + nviews), st);
  // runs of 4 floats where every view's row starts 16-byte aligned, else single floats
  const int64_t row = (int64_t)patch[2] * channels;
  const bool vec = row % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
  const unsigned lanes = row_threads(ceil_div(row, vec ? 4 : 1), 128, 32);
  const unsigned rows = rows_per_group(lanes);
  const dim3 grid((unsigned)ceil_div(patch[1], rows), patch[0]), block(lanes, rows);
  if (vec)
    hipLaunchKernelGGL(gather_flip_kernel<4>, grid, block, 0, st, vol, channels, size[0], size[1],
                       size[2], pad_before[0], pad_before[1], pad_before[2], offset[0], offset[1],
                       offset[2], patch[0], patch[1], patch[2], f, nviews, out);
  else
    hipLaunchKernelGGL(gather_flip_kernel<1>, grid, block, 0, st, vol, channels, size[0], size[1],
                       size[2], pad_before[0], pad_before[1], pad_before[2], offset[0], offset[1],
                       offset[2], patch[0], patch[1], patch[2], f, nviews, out);
  launch_check("sw_gather_flip");
}

void sw_accumulate(const float* pred, int nviews, const int* flips, int k, const int* patch,
                   const void* gaussian, const int* offset, const int64_t* padded, int accum,
                   void* acc, void* norm, hipStream_t st) {
  require(pred && gaussian && acc && norm, "accumulate pointers must not be null");
  require(k >= 1, "accumulate needs at least one class");
  for (int i = 0; i < 3; ++i)
    require(offset[i] >= 0 && (int64_t)offset[i] + patch[i] <= padded[i],
            "tile outside the padded volume");
  const Flips f = make_flips(flips, nviews);
  const int64_t n = (int64_t)patch[0] * patch[1] * patch[2];
  require(patch[1] <= 65535 && patch[0] <= 65535, "patch rows exceed the launch grid");
  const double esz = accum == NNX_ACCUM_NNUNET_F16 ? 2.0 : 4.0;
  ProfScope prof("sw_accumulate", 0.0,
                 (double)n * (nviews * k * 4.0 + 2.0 * k * esz + 2.0 * esz + esz), st);
  // at most 128 lanes a row (longer rows loop), several rows a workgroup
  const unsigned lanes = row_threads((int64_t)patch[2] * k, kAccLanes), rows = rows_per_group(lanes);
  const dim3 grid((unsigned)ceil_div(patch[1], rows), patch[0]), block(lanes, rows);
  if (accum == NNX_ACCUM_NNUNET_F16)
    hipLaunchKernelGGL(accumulate_kernel<true>, grid, block, 0, st, pred, nviews,
                       f, k, patch[0], patch[1], patch[2], gaussian, offset[0], offset[1],
                       offset[2], padded[1], padded[2], acc, norm);
  else
    hipLaunchKernelGGL(accumulate_kernel<false>, grid, block, 0, st, pred, nviews,
                       f, k, patch[0], patch[1], patch[2], gaussian, offset[0], offset[1],
                       offset[2], padded[1], padded[2], acc, norm);
  launch_check("sw_accumulate");
}

void sw_fold_add(const void* acc, const void* norm, int k, const int64_t* padded,
                 const int* crop_lo, const int64_t* crop_size, int accum, bool first,
                 void* total, hipStream_t st) {
  require(acc && norm && total, "fold pointers must not be null");
  for (int i = 0; i < 3; ++i)
    require(crop_lo[i] >= 0 && crop_size[i] >= 0 && crop_lo[i] <= padded[i] &&
                crop_size[i] <= padded[i] - crop_lo[i],
            "crop outside the volume");
  const int64_t n = crop_size[0] * crop_size[1] * crop_size[2];
  const double esz = accum == NNX_ACCUM_NNUNET_F16 ? 2.0 : 4.0;
  ProfScope prof("sw_fold_add", 0.0, (double)n * (k * esz + esz + k * esz * (first ? 1 : 2)), st);
  if (accum == NNX_ACCUM_NNUNET_F16)
    hipLaunchKernelGGL(fold_add_kernel<true>, dim3(grid_for(n)), dim3(256), 0, st, acc, norm, k,
                       padded[1], padded[2], crop_lo[0], crop_lo[1], crop_lo[2], crop_size[0],
                       crop_size[1], crop_size[2], first ? 1 : 0, total);
  else
    hipLaunchKernelGGL(fold_add_kernel<false>, dim3(grid_for(n)), dim3(256), 0, st, acc, norm, k,
                       padded[1], padded[2], crop_lo[0], crop_lo[1], crop_lo[2], crop_size[0],
                       crop_size[1], crop_size[2], first ? 1 : 0, total);
  launch_check("sw_fold_add");
}

void sw_fold_finalize(const void* total, int k, int64_t voxels, int nfolds, int accum,
                      void* logits, uint16_t* labels, unsigned int* invalid, hipStream_t st) {
  require(total != nullptr, "fold total must not be null");
  require(k >= 1 && k <= 65535, "label reduction supports 1..65535 classes");
  require(nfolds >= 1, "at least one fold");
  if (invalid) fill_zero(invalid, sizeof(unsigned int), st);
  if (voxels <= 0) return;
  const double esz = accum == NNX_ACCUM_NNUNET_F16 ? 2.0 : 4.0;
  ProfScope prof("sw_fold_finalize", 0.0,
                 (double)voxels * (k * esz + (labels ? 2.0 : 0.0) + (logits ? k * esz : 0.0)), st);
  if (accum == NNX_ACCUM_NNUNET_F16)
    hipLaunchKernelGGL(fold_finalize_kernel<true>, dim3(grid_for(voxels)), dim3(256), 0, st, total,
                       k, voxels, nfolds, logits, labels, invalid);
  else
    hipLaunchKernelGGL(fold_finalize_kernel<false>, dim3(grid_for(voxels)), dim3(256), 0, st,
                       total, k, voxels, nfolds, logits, labels, invalid);
  launch_check("sw_fold_finalize");
}

}  // namespace nnx
